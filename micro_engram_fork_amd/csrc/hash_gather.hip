// Stages 1 and 2 of the Engram lookup path on gfx950: n-gram hashing and the multi-table row
// gather, fused into one kernel.
//
// Reference behaviour (micro_engram/module.py):
//   hash_ids   183-205  ids -> canon[clamp(ids)] -> causal n-gram window with raw pad_id where
//                       the token is before the sequence start or before the document start
//                       (position < i) -> sum_i tok_i * mults[k][i] -> % (2^31-1) % rows_k
//   hash_prev  207-226  the same from a [n, width] matrix of predecessors (-1 = missing)
//   lookup     146-154  per-table embedding rows, concatenated along the feature dim (233)
//
// Kernel layout. One 256-thread workgroup owns `tpb` consecutive tokens (tpb * n_tables <= 256,
// so every (token, table) pair has a thread):
//   phase 0  each (token, table) thread loads its table's constants (multipliers, order, fastmod
//            magic, base address) into registers, before and independent of the token loads;
//   phase 1  each (token, slot) thread loads one n-gram token, applies clamp + canon and the
//            pad rules, and leaves the value in LDS (tok[token][slot]);
//   phase 2  each (token, table) thread hashes its n-gram, writes the int64 row id (coalesced
//            along tokens, [n_tables, n] layout) and leaves the row's address in LDS;
//   phase 3  the workgroup copies the tokens' memory vectors: the output of the block is one
//            contiguous run of bytes, so thread c moves 16-byte chunk c (dwordx4 load from the
//            table row, dwordx4 store into mem). Eight lanes cover one 128-byte bf16 row, a
//            wavefront writes 1 KiB of consecutive output per instruction, and all of a
//            thread's chunks (up to kUnroll) are in flight before its first store.
// The kernel is a chain of dependent memory round trips (token ids -> canon entry -> table
// row -> store), and all workgroups of a launch are resident at once, so the chain's latency
// is paid once per launch and is the part of the time that is not bandwidth: the constants
// load off the chain, a null canon (identity map) takes one round trip out of it, and the
// row copy keeps every load of a thread in flight together. The output is written with
// non-temporal stores: it is consumed by the next kernel, and streaming it past the caches
// leaves them to the table rows (hot n-grams repeat) instead of dirty lines to write back.
// The row ids staged in LDS are what lets the copy run at full width: each output chunk is
// one lane's register, so the concatenated vector needs no further LDS round trip.
#include "me_common.h"

namespace me {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 8;

enum Mode : int { kModeSeq = 0, kModePrev = 1, kModeIdx = 2 };

struct TableMeta {
    uint64_t base[ME_MAX_TABLES];   // device address of table k (gather only)
    uint64_t magic[ME_MAX_TABLES];  // fastmod constant for rows32
    int64_t rows[ME_MAX_TABLES];    // rows of table k
    uint32_t rows32[ME_MAX_TABLES]; // rows if < 2^31 - 1, else 0 (the hash is already < rows)
    int32_t order[ME_MAX_TABLES];
};

struct LookupArgs {
    // token ids: [n] as batch x seq (kModeSeq) or [n, width] rows row_stride apart (kModePrev)
    const void *ids;
    int ids_i64;
    int64_t n;
    int64_t seq_len;
    int64_t row_stride;
    const void *pos;
    int pos_i64;
    int64_t pos_bstride;
    const int64_t *canon;  // nullable: identity map over [0, vocab)
    int64_t vocab;
    const int64_t *mults;
    int max_order;
    int64_t pad_id;
    // given row ids (kModeIdx)
    const int64_t *idx_in;
    int64_t idx_stride;
    // outputs
    int64_t *idx_out;  // nullable
    uint8_t *mem;      // nullable: hash only
    int n_tables;
    int tpb;
    int tpb_shift;
    int row_bytes;
    int cpr;        // chunks per table row
    int cpr_shift;  // log2(cpr) if cpr is a power of two, else -1
    TableMeta meta;
};

__device__ __forceinline__ int64_t load_id(const void *p, int is64, int64_t i) {
    return is64 ? static_cast<const int64_t *>(p)[i]
                : static_cast<int64_t>(static_cast<const int32_t *>(p)[i]);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int VEC>
struct Chunk;
template <>
struct Chunk<16> {
    using T = u32x4_t;
};
template <>
struct Chunk<4> {
    using T = uint32_t;
};
template <>
struct Chunk<2> {
    using T = uint16_t;
};

// GATHER = false: hash only (no memory vectors), its own instantiation without phase 3.
// PACED: at most two of a thread's row loads in flight, for launches of 8 tokens per workgroup
// (six chunks per thread) that are one round of resident workgroups. Measured on MI355X: the
// 8192-token prefill gather 12.4-12.5 us paced against 12.7-13.0 with all six in flight (every
// workgroup's requests queue at once, and fewer random-row requests queued together are served
// faster); launches of several rounds (65,536 tokens: 79.7 against 74 us) and those of 1-4
// tokens per workgroup (0.1-0.25 us) are faster unpaced.
template <int MODE, int VEC, bool GATHER, bool PACED = false>
__global__ __launch_bounds__(kBlock) void lookup_kernel(const LookupArgs a) {
    using V = typename Chunk<VEC>::T;
    __shared__ int64_t s_tok[64 * ME_MAX_ORDER];  // [tpb][max_order] hashed token values
    __shared__ uint64_t s_src[kBlock];  // [tpb * n_tables] source row address, token-major

    const int tid = threadIdx.x;
    const int nt = a.n_tables;
    const int mo = a.max_order;
    const int64_t g0 = static_cast<int64_t>(blockIdx.x) * a.tpb;
    const int ntok = static_cast<int>(min(static_cast<int64_t>(a.tpb), a.n - g0));

    // ---- phase 0: this thread's (token, table) pair and its table constants, in registers;
    // token index fastest so the [n_tables, n] row-id writes coalesce
    const int wi = tid & (a.tpb - 1);
    const int wk = tid >> a.tpb_shift;
    const bool worker = tid < a.tpb * nt && wi < ntok;
    uint64_t mult[ME_MAX_ORDER];
    int order = 0;
    uint64_t magic = 0, base = 0;
    uint32_t rows32 = 0;
    int64_t rows = 0, given = 0;
    if (worker) {
        base = a.meta.base[wk];
        if (MODE == kModeIdx) {
            rows = a.meta.rows[wk];
            given = a.idx_in[wk * a.idx_stride + g0 + wi];
        } else {
            order = a.meta.order[wk];
            magic = a.meta.magic[wk];
            rows32 = a.meta.rows32[wk];
#pragma unroll
            for (int s = 0; s < ME_MAX_ORDER; ++s)
                mult[s] = s < mo ? static_cast<uint64_t>(a.mults[wk * mo + s]) : 0ull;
        }
    }

    // ---- phase 1: n-gram token values. The id load is issued from a clamped address before
    // the window and document checks resolve, so its latency overlaps them.
    if (MODE == kModeSeq) {
        const uint32_t seq_len = static_cast<uint32_t>(a.seq_len);
        for (int e = tid; e < ntok * mo; e += kBlock) {
            const int i = e / mo, s = e - i * mo;
            const int64_t g = g0 + i;
            const int64_t id_raw = load_id(a.ids, a.ids_i64, g - s >= 0 ? g - s : 0);
            const uint32_t b = static_cast<uint32_t>(g) / seq_len;
            const uint32_t t = static_cast<uint32_t>(g) - b * seq_len;
            bool ok = static_cast<int>(t) >= s;
            if (ok && s > 0 && a.pos != nullptr)
                ok = load_id(a.pos, a.pos_i64, static_cast<int64_t>(b) * a.pos_bstride + t) >= s;
            int64_t v = a.pad_id;
            if (ok) {
                const int64_t id = id_raw < 0 ? 0 : (id_raw >= a.vocab ? a.vocab - 1 : id_raw);
                v = a.canon != nullptr ? a.canon[id] : id;
            }
            s_tok[i * ME_MAX_ORDER + s] = v;
        }
    } else if (MODE == kModePrev) {
        for (int e = tid; e < ntok * mo; e += kBlock) {
            const int i = e / mo, s = e - i * mo;
            int64_t id = load_id(a.ids, a.ids_i64, (g0 + i) * a.row_stride + s);
            int64_t v = a.pad_id;
            if (id >= 0) {
                id = id >= a.vocab ? a.vocab - 1 : id;
                v = a.canon != nullptr ? a.canon[id] : id;
            }
            s_tok[i * ME_MAX_ORDER + s] = v;
        }
    }
    if (MODE != kModeIdx) __syncthreads();

    // ---- phase 2: hash (or check the given row id), publish the source row address
    if (worker) {
        int64_t r;
        bool valid = true;
        if (MODE == kModeIdx) {
            r = given;
            valid = r >= 0 && r < rows;
        } else {
            uint64_t x = 0;
#pragma unroll
            for (int s = 0; s < ME_MAX_ORDER; ++s)
                if (s < order) x += static_cast<uint64_t>(s_tok[wi * ME_MAX_ORDER + s]) * mult[s];
            uint32_t h = floor_mod_prime(x);
            if (rows32 != 0) h = fastmod_u32(h, magic, rows32);
            r = h;
            if (a.idx_out != nullptr) a.idx_out[wk * a.n + g0 + wi] = r;
        }
        if (GATHER)
            s_src[wi * nt + wk] = valid ? base + static_cast<uint64_t>(r) * a.row_bytes : 0ull;
    }
    if (!GATHER) return;
    __syncthreads();

    // ---- phase 3: copy the block's memory vectors, chunk c of the block's output run. A
    // thread's chunks are walked in an order rotated by the block index, so that at any moment
    // the workgroups write different 4 KiB pieces of their runs instead of all writing the
    // same piece (runs are equal-sized and adjacent).
    // Three straight passes per batch of kUnroll chunks: every source address (LDS reads, one
    // wait), then every load, then every store, so all of a thread's loads are in flight at once.
    const int total = ntok * nt * a.cpr;
    uint8_t *dst = a.mem + static_cast<uint64_t>(g0) * nt * a.row_bytes;
    for (int c0 = tid; c0 < total; c0 += kBlock * kUnroll) {
        const int steps = min(kUnroll, (total - (c0 - tid) + kBlock - 1) / kBlock);
        const int rot = static_cast<int>(blockIdx.x % static_cast<unsigned>(steps));
        int chunk[kUnroll];
        uint64_t src[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int ur = u < steps ? (u + rot < steps ? u + rot : u + rot - steps) : u;
            const int c = c0 + ur * kBlock;
            chunk[u] = c;
            src[u] = 0;
            if (c < total) {
                const int p = a.cpr_shift >= 0 ? (c >> a.cpr_shift) : (c / a.cpr);
                const int off = c - p * a.cpr;
                const uint64_t row = s_src[p];
                src[u] = row != 0 ? row + static_cast<uint64_t>(off) * VEC : 0;
            }
        }
        V v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            v[u] = V{};
            if (src[u] != 0) v[u] = *as_global_addr<const V>(src[u]);
            if (PACED && u % 2 == 1 && u + 1 < kUnroll) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (chunk[u] < total)
                __builtin_nontemporal_store(
                    v[u], as_global(reinterpret_cast<V *>(dst + static_cast<uint64_t>(chunk[u]) * VEC)));
        }
    }
}

int log2_exact(int64_t v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int s = 0;
    while ((int64_t{1} << s) < v) ++s;
    return s;
}

// Validates the table set and fills the per-table metadata.
int fill_meta(LookupArgs &a, int32_t n_tables, const int32_t *table_orders,
              const int64_t *table_rows, int32_t max_order, bool need_orders) {
    ME_CHECK_ARG(n_tables >= 1 && n_tables <= ME_MAX_TABLES,
                 "n_tables must be in [1, %d], got %d", ME_MAX_TABLES, n_tables);
    ME_CHECK_ARG(table_rows != nullptr, "table_rows is null");
    if (need_orders) {
        ME_CHECK_ARG(max_order >= 1 && max_order <= ME_MAX_ORDER,
                     "max_order must be in [1, %d], got %d", ME_MAX_ORDER, max_order);
        ME_CHECK_ARG(table_orders != nullptr, "table_orders is null");
    }
    a.n_tables = n_tables;
    a.max_order = max_order;
    for (int k = 0; k < n_tables; ++k) {
        ME_CHECK_ARG(table_rows[k] >= 1, "table %d has %lld rows", k, (long long)table_rows[k]);
        a.meta.rows[k] = table_rows[k];
        const bool small = table_rows[k] < static_cast<int64_t>(kPrime);
        a.meta.rows32[k] = small ? static_cast<uint32_t>(table_rows[k]) : 0u;
        a.meta.magic[k] = small ? fastmod_magic(static_cast<uint32_t>(table_rows[k])) : 0ull;
        if (need_orders) {
            ME_CHECK_ARG(table_orders[k] >= 1 && table_orders[k] <= max_order,
                         "table %d has order %d outside [1, max_order=%d]", k, table_orders[k],
                         max_order);
            a.meta.order[k] = table_orders[k];
        }
    }
    int tpb = 1;
    while (tpb * 2 * n_tables <= kBlock && tpb * 2 <= 64) tpb *= 2;
    a.tpb = tpb;
    a.tpb_shift = log2_exact(tpb);
    return ME_OK;
}

int fill_gather(LookupArgs &a, const void *const *tables, int32_t dim, int dtype, void *mem,
                int *vec) {
    ME_CHECK_ARG(tables != nullptr, "tables is null");
    ME_CHECK_ARG(mem != nullptr || a.n == 0, "mem is null");
    ME_CHECK_ARG(dtype == ME_BF16 || dtype == ME_F32, "table dtype must be ME_BF16 or ME_F32");
    ME_CHECK_ARG(dim >= 1, "dim must be positive, got %d", dim);
    const int64_t row_bytes = static_cast<int64_t>(dim) * dtype_size(dtype);
    ME_CHECK_ARG(row_bytes <= (1 << 20), "dim %d too large", dim);
    for (int k = 0; k < a.n_tables; ++k) {
        ME_CHECK_ARG(tables[k] != nullptr, "table %d is null", k);
        a.meta.base[k] = reinterpret_cast<uint64_t>(tables[k]);
    }
    // Widest chunk every row start (table base, row stride, output offset) is aligned to.
    uint64_t align_or = static_cast<uint64_t>(row_bytes) | reinterpret_cast<uint64_t>(mem);
    for (int k = 0; k < a.n_tables; ++k) align_or |= a.meta.base[k];
    *vec = (align_or % 16 == 0) ? 16 : (align_or % 4 == 0) ? 4 : 2;
    a.mem = static_cast<uint8_t *>(mem);
    a.row_bytes = static_cast<int>(row_bytes);
    a.cpr = static_cast<int>(row_bytes / *vec);
    a.cpr_shift = log2_exact(a.cpr);
    ME_CHECK_ARG(static_cast<int64_t>(a.tpb) * a.n_tables * a.cpr < (int64_t{1} << 30),
                 "row too large for one workgroup");
    return ME_OK;
}

// Workgroups a launch keeps when its tokens allow: fewer tokens per workgroup for small batches
// (a 256-token decode step, the 2048-token fp32 case) so that every CU gets work.
constexpr int64_t kMinBlocks = 512;
// Largest launch that takes the paced copy (one round: every workgroup resident at once).
constexpr unsigned kPacedMaxBlocks = 2048;

template <int MODE>
int launch(const LookupArgs &a0, int vec, hipStream_t stream, const char *what) {
    if (a0.n == 0) return ME_OK;
    LookupArgs a = a0;
    while (a.tpb > 1 && ceil_div(a.n, static_cast<int64_t>(a.tpb)) < kMinBlocks) a.tpb >>= 1;
    a.tpb_shift = log2_exact(a.tpb);
    const dim3 grid(static_cast<unsigned>(ceil_div(a.n, a.tpb)));
    if (a.mem == nullptr) {
        hipLaunchKernelGGL((lookup_kernel<MODE, 16, false>), grid, dim3(kBlock), 0, stream, a);
        return check_launch(what);
    }
    if (vec == 16 && a.tpb >= 8 && grid.x <= kPacedMaxBlocks) {
        hipLaunchKernelGGL((lookup_kernel<MODE, 16, true, true>), grid, dim3(kBlock), 0, stream, a);
        return check_launch(what);
    }
    switch (vec) {
        case 16: hipLaunchKernelGGL((lookup_kernel<MODE, 16, true>), grid, dim3(kBlock), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((lookup_kernel<MODE, 4, true>), grid, dim3(kBlock), 0, stream, a); break;
        default: hipLaunchKernelGGL((lookup_kernel<MODE, 2, true>), grid, dim3(kBlock), 0, stream, a); break;
    }
    return check_launch(what);
}

int common_hash_args(LookupArgs &a, const int64_t *canon, int64_t vocab, const int64_t *mults,
                     int64_t pad_id) {
    ME_CHECK_ARG(mults != nullptr, "mults must not be null");
    ME_CHECK_ARG(vocab >= 1, "vocab must be positive");
    a.canon = canon;
    a.vocab = vocab;
    a.mults = mults;
    a.pad_id = pad_id;
    return ME_OK;
}

int seq_args(LookupArgs &a, const void *input_ids, int ids_dtype, int64_t batch, int64_t seq_len,
             const void *position_ids, int pos_dtype, int64_t pos_batch_stride) {
    ME_CHECK_ARG(ids_dtype == ME_I32 || ids_dtype == ME_I64, "ids dtype must be ME_I32/ME_I64");
    ME_CHECK_ARG(batch >= 0 && seq_len >= 0, "negative shape");
    ME_CHECK_ARG(input_ids != nullptr || batch * seq_len == 0, "input_ids is null");
    ME_CHECK_ARG(batch * seq_len < (int64_t{1} << 31), "too many tokens for one call");
    if (position_ids != nullptr) {
        ME_CHECK_ARG(pos_dtype == ME_I32 || pos_dtype == ME_I64,
                     "position dtype must be ME_I32/ME_I64");
        ME_CHECK_ARG(pos_batch_stride >= 0, "negative position batch stride");
    }
    a.ids = input_ids;
    a.ids_i64 = ids_dtype == ME_I64;
    a.n = batch * seq_len;
    a.seq_len = seq_len > 0 ? seq_len : 1;
    a.pos = position_ids;
    a.pos_i64 = pos_dtype == ME_I64;
    a.pos_bstride = pos_batch_stride;
    return ME_OK;
}

int prev_args(LookupArgs &a, const void *ids, int ids_dtype, int64_t n, int64_t width,
              int64_t row_stride) {
    ME_CHECK_ARG(ids_dtype == ME_I32 || ids_dtype == ME_I64, "ids dtype must be ME_I32/ME_I64");
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "bad token count %lld", (long long)n);
    ME_CHECK_ARG(ids != nullptr || n == 0, "ids is null");
    ME_CHECK_ARG(width >= a.max_order, "ids has %lld columns, the engram needs max_order=%d",
                 (long long)width, a.max_order);
    ME_CHECK_ARG(row_stride >= width, "row_stride %lld < width %lld", (long long)row_stride,
                 (long long)width);
    a.ids = ids;
    a.ids_i64 = ids_dtype == ME_I64;
    a.n = n;
    a.row_stride = row_stride;
    return ME_OK;
}

}  // namespace
}  // namespace me

using namespace me;

#define ME_TRY(expr)                 \
    do {                             \
        const int _st = (expr);      \
        if (_st != ME_OK) return _st; \
    } while (0)

extern "C" int me_hash_ngrams(const void *input_ids, int ids_dtype, int64_t batch, int64_t seq_len,
                              const void *position_ids, int pos_dtype, int64_t pos_batch_stride,
                              const int64_t *canon, int64_t vocab, const int64_t *mults,
                              int32_t max_order, int32_t n_tables, const int32_t *table_orders,
                              const int64_t *table_rows, int64_t pad_id, int64_t *idx_out,
                              void *stream) {
    LookupArgs a{};
    ME_TRY(fill_meta(a, n_tables, table_orders, table_rows, max_order, true));
    ME_TRY(seq_args(a, input_ids, ids_dtype, batch, seq_len, position_ids, pos_dtype,
                    pos_batch_stride));
    ME_TRY(common_hash_args(a, canon, vocab, mults, pad_id));
    ME_CHECK_ARG(idx_out != nullptr || a.n == 0, "idx_out is null");
    a.idx_out = idx_out;
    return launch<kModeSeq>(a, 16, as_stream(stream), "me_hash_ngrams");
}

extern "C" int me_hash_prev(const void *ids, int ids_dtype, int64_t n, int64_t width,
                            int64_t row_stride, const int64_t *canon, int64_t vocab,
                            const int64_t *mults, int32_t max_order, int32_t n_tables,
                            const int32_t *table_orders, const int64_t *table_rows, int64_t pad_id,
                            int64_t *idx_out, void *stream) {
    LookupArgs a{};
    ME_TRY(fill_meta(a, n_tables, table_orders, table_rows, max_order, true));
    ME_TRY(prev_args(a, ids, ids_dtype, n, width, row_stride));
    ME_TRY(common_hash_args(a, canon, vocab, mults, pad_id));
    ME_CHECK_ARG(idx_out != nullptr || a.n == 0, "idx_out is null");
    a.idx_out = idx_out;
    return launch<kModePrev>(a, 16, as_stream(stream), "me_hash_prev");
}

extern "C" int me_gather(const int64_t *idx, int64_t idx_table_stride, int64_t n, int32_t n_tables,
                         const void *const *tables, const int64_t *table_rows, int32_t dim,
                         int dtype, void *mem, void *stream) {
    LookupArgs a{};
    ME_TRY(fill_meta(a, n_tables, nullptr, table_rows, 1, false));
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "bad token count %lld", (long long)n);
    ME_CHECK_ARG(idx != nullptr || n == 0, "idx is null");
    ME_CHECK_ARG(idx_table_stride >= n, "idx_table_stride %lld < n %lld",
                 (long long)idx_table_stride, (long long)n);
    a.idx_in = idx;
    a.idx_stride = idx_table_stride;
    a.n = n;
    int vec = 16;
    ME_TRY(fill_gather(a, tables, dim, dtype, mem, &vec));
    return launch<kModeIdx>(a, vec, as_stream(stream), "me_gather");
}

extern "C" int me_hash_gather(const void *input_ids, int ids_dtype, int64_t batch, int64_t seq_len,
                              const void *position_ids, int pos_dtype, int64_t pos_batch_stride,
                              const int64_t *canon, int64_t vocab, const int64_t *mults,
                              int32_t max_order, int32_t n_tables, const int32_t *table_orders,
                              const int64_t *table_rows, int64_t pad_id, const void *const *tables,
                              int32_t dim, int dtype, void *mem, int64_t *idx_out, void *stream) {
    LookupArgs a{};
    ME_TRY(fill_meta(a, n_tables, table_orders, table_rows, max_order, true));
    ME_TRY(seq_args(a, input_ids, ids_dtype, batch, seq_len, position_ids, pos_dtype,
                    pos_batch_stride));
    ME_TRY(common_hash_args(a, canon, vocab, mults, pad_id));
    int vec = 16;
    ME_TRY(fill_gather(a, tables, dim, dtype, mem, &vec));
    a.idx_out = idx_out;
    return launch<kModeSeq>(a, vec, as_stream(stream), "me_hash_gather");
}

extern "C" int me_hash_prev_gather(const void *ids, int ids_dtype, int64_t n, int64_t width,
                                   int64_t row_stride, const int64_t *canon, int64_t vocab,
                                   const int64_t *mults, int32_t max_order, int32_t n_tables,
                                   const int32_t *table_orders, const int64_t *table_rows,
                                   int64_t pad_id, const void *const *tables, int32_t dim, int dtype,
                                   void *mem, int64_t *idx_out, void *stream) {
    LookupArgs a{};
    ME_TRY(fill_meta(a, n_tables, table_orders, table_rows, max_order, true));
    ME_TRY(prev_args(a, ids, ids_dtype, n, width, row_stride));
    ME_TRY(common_hash_args(a, canon, vocab, mults, pad_id));
    int vec = 16;
    ME_TRY(fill_gather(a, tables, dim, dtype, mem, &vec));
    a.idx_out = idx_out;
    return launch<kModePrev>(a, vec, as_stream(stream), "me_hash_prev_gather");
}
