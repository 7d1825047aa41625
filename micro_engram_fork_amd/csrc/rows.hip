// Stage 4 of the Engram lookup path on gfx950, the training side: touched-row dedup with
// coalesced gradient sums, the global gradient norm for clipping, and the lazy / row-wise Adam
// update of the touched rows with stochastic rounding to bf16.
//
// Reference:
//   dedup      micro_engram/rows.py:81 (torch.unique(return_inverse)), 117-118 and 144-146
//              (zeros().index_add_(0, inv, g)): unique keys ascending, the inverse index, and the
//              fp32 sum of each key's gradient rows in the order the rows appear
//   sumsq      rows.py:214-220 (the squared norm RowTables.clip scales against)
//   adam       micro_engram/optim.py:65-133, the sparse-gradient branch (88-97), per-row second
//              moment (112-114) and write-back with stochastic_bf16 (33-44, 120-132)
//
// Dedup = a stable LSD radix sort of (key, position) pairs, 8 key bits per pass: per-block digit
// histograms, one scan over [digit][block], then a scatter that ranks equal digits inside each
// wave with 8 ballots (lower lane = earlier element), so every pass keeps the positions of equal
// keys in increasing order. Segment heads of the sorted keys then give the unique keys, the
// inverse, and per-segment ranges; one thread per (segment, 4 columns) sums the gradient rows of
// its segment in ascending position order starting from +0.0 -- the order, and so the rounding,
// of CPU index_add_.
#include "me_common.h"

#include <cmath>

namespace me {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 8;                        // elements per thread per tile
constexpr int kTile = kThreads * kItems;         // 2048 elements per sort block
constexpr int kBins = 256;                       // 8-bit digits

__device__ __forceinline__ uint64_t lanes_below(int lane) { return (1ull << lane) - 1ull; }

// ---- radix sort -----------------------------------------------------------------------------
// hist[digit * stride + tile]: row `digit` holds that digit's count in every tile; rows are
// padded to a multiple of 4 tiles (zeros) so a row reads as 16-byte words.
__global__ __launch_bounds__(kThreads) void rs_hist(const uint64_t *keys, int64_t n, int shift,
                                                    uint32_t *hist, int nblocks, int stride) {
    __shared__ uint32_t s[kBins];
    const int tid = threadIdx.x;
    s[tid] = 0;
    __syncthreads();
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int64_t idx = base + i * kThreads + tid;
        if (idx < n) atomicAdd(&s[(keys[idx] >> shift) & (kBins - 1)], 1u);
    }
    __syncthreads();
    hist[static_cast<int64_t>(tid) * stride + blockIdx.x] = s[tid];
    if (blockIdx.x == 0)
        for (int b = nblocks; b < stride; ++b) hist[static_cast<int64_t>(tid) * stride + b] = 0u;
}

// Exclusive prefix sum of v[0..total) in place, one workgroup. If total_out is given, the sum
// of all entries is written there too.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    return x;
}

// Scatter of one tile. Its output base for digit d = (all keys with a smaller digit) + (keys
// with digit d in earlier tiles): thread d reads row d of the histogram as 16-byte words,
// summing the earlier tiles and all tiles, and a scan of the 256 totals across the workgroup
// orders the digits. Every tile derives its bases itself, so a pass is two launches.
__global__ __launch_bounds__(kThreads) void rs_scatter(const uint64_t *keys_in, const uint32_t *pos_in,
                                                       uint64_t *keys_out, uint32_t *pos_out,
                                                       int64_t n, int shift, const uint32_t *hist,
                                                       int stride) {
    __shared__ uint32_t s_base[kBins];
    __shared__ uint32_t s_wcnt[kThreads / 64][kBins];
    __shared__ uint32_t s_wtot[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {
        static_assert(kThreads == kBins, "one thread per digit");
        const uint4 *row = reinterpret_cast<const uint4 *>(hist + static_cast<int64_t>(tid) * stride);
        const int words = stride / 4, me = static_cast<int>(blockIdx.x);
        uint32_t mine = 0, tot = 0;
        for (int q0 = 0; q0 < words; q0 += 8) {
            uint4 x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) x[u] = q0 + u < words ? row[q0 + u] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int t0 = (q0 + u) * 4;
                const uint32_t c[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    tot += c[e];
                    if (t0 + e < me) mine += c[e];
                }
            }
        }
        const uint32_t incl = wave_inclusive_scan(tot, lane);
        if (lane == 63) s_wtot[wave] = incl;
        __syncthreads();
        uint32_t before = 0;
        for (int w = 0; w < wave; ++w) before += s_wtot[w];
        s_base[tid] = before + incl - tot + mine;
    }
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kTile;
    for (int i = 0; i < kItems; ++i) {
        const int64_t idx = base + i * kThreads + tid;
        const bool valid = idx < n;
        const uint64_t key = valid ? keys_in[idx] : 0ull;
        const uint32_t pos = valid ? (pos_in != nullptr ? pos_in[idx] : static_cast<uint32_t>(idx)) : 0u;
        const int digit = static_cast<int>((key >> shift) & (kBins - 1));
#pragma unroll
        for (int q = 0; q < kBins / 64; ++q) s_wcnt[wave][lane * (kBins / 64) + q] = 0u;
        // lanes of this wave holding the same digit
        uint64_t same = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool set = (digit >> bit) & 1;
            const uint64_t b = __ballot(set);
            same &= set ? b : ~b;
        }
        const int rank = __popcll(same & lanes_below(lane));
        __syncthreads();  // counts cleared (and the previous chunk's base update is done)
        if (valid && rank == 0) s_wcnt[wave][digit] = static_cast<uint32_t>(__popcll(same));
        __syncthreads();
        if (valid) {
            uint32_t off = s_base[digit] + static_cast<uint32_t>(rank);
            for (int w = 0; w < wave; ++w) off += s_wcnt[w][digit];
            keys_out[off] = key;
            pos_out[off] = pos;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) add += s_wcnt[w][tid];
        s_base[tid] += add;
        __syncthreads();  // the next chunk clears s_wcnt and reads s_base
    }
}

// ---- segments of the sorted keys -------------------------------------------------------------
// Tile layout for the segment pass: thread t owns elements [t * kItems, (t + 1) * kItems) of
// its block's tile, so a block-level exclusive scan of per-thread head counts numbers the heads.
__device__ __forceinline__ bool is_head(const uint64_t *k, int64_t i) {
    return i == 0 || k[i] != k[i - 1];
}

__global__ __launch_bounds__(kThreads) void seg_count(const uint64_t *skeys, int64_t n,
                                                      uint32_t *block_heads) {
    __shared__ uint32_t s[kThreads];
    const int tid = threadIdx.x;
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kTile + static_cast<int64_t>(tid) * kItems;
    uint32_t c = 0;
    for (int i = 0; i < kItems; ++i)
        if (b + i < n && is_head(skeys, b + i)) ++c;
    s[tid] = c;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (tid < off) s[tid] += s[tid + off];
        __syncthreads();
    }
    if (tid == 0) block_heads[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(kThreads) void seg_write(const uint64_t *skeys, const uint32_t *spos,
                                                      int64_t n, const uint32_t *block_heads,
                                                      int nblocks, int64_t *uniq, int64_t *inv,
                                                      uint32_t *seg_start, uint32_t *seg_pos,
                                                      int64_t *count) {
    __shared__ uint32_t s[kThreads];
    __shared__ uint32_t s_before[kThreads / 64], s_all[kThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {   // heads in the tiles before this one (and in all tiles, for the count)
        uint32_t before = 0, all = 0;
        for (int b = tid; b < nblocks; b += kThreads) {
            const uint32_t c = block_heads[b];
            all += c;
            if (b < static_cast<int>(blockIdx.x)) before += c;
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            before += __shfl_xor(before, off, 64);
            all += __shfl_xor(all, off, 64);
        }
        if (lane == 0) {
            s_before[wave] = before;
            s_all[wave] = all;
        }
    }
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kTile + static_cast<int64_t>(tid) * kItems;
    uint32_t c = 0;
    for (int i = 0; i < kItems; ++i)
        if (b + i < n && is_head(skeys, b + i)) ++c;
    s[tid] = c;
    __syncthreads();
    for (int off = 1; off < kThreads; off <<= 1) {
        const uint32_t t = tid >= off ? s[tid - off] : 0u;
        __syncthreads();
        s[tid] += t;
        __syncthreads();
    }
    uint32_t tile_base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        tile_base += s_before[w];
        total += s_all[w];
    }
    if (blockIdx.x == 0 && tid == 0) *count = total;
    // heads before this thread's first element, over the whole array
    uint32_t heads = tile_base + s[tid] - c;
    for (int i = 0; i < kItems; ++i) {
        const int64_t idx = b + i;
        if (idx >= n) break;
        if (is_head(skeys, idx)) {
            uniq[heads] = static_cast<int64_t>(skeys[idx]);
            seg_start[heads] = static_cast<uint32_t>(idx);
            seg_pos[heads] = spos[idx];  // the segment's first row, one load less for the sums
            ++heads;
        }
        inv[spos[idx]] = static_cast<int64_t>(heads) - 1;
        if (idx == n - 1) seg_start[heads] = static_cast<uint32_t>(n);
    }
}

__global__ void write_zero_count(int64_t *count) { *count = 0; }

// One thread per (segment, run of kCols columns): the segment's gradient rows summed in sorted
// (= original) order, starting from +0.0 like zeros().index_add_(). The segment's bounds, its
// first row and the segment count are independent loads; rows after the first are fetched four
// at a time and added in order.
__device__ __forceinline__ void load_cols(const float *p, float (&x)[4]) {
    const float4 v = *reinterpret_cast<const float4 *>(p);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
}
__device__ __forceinline__ void load_cols(const uint16_t *p, float (&x)[4]) {
    const uint2 v = *reinterpret_cast<const uint2 *>(p);
    x[0] = bf16_bits_to_float(static_cast<uint16_t>(v.x));
    x[1] = bf16_bits_to_float(static_cast<uint16_t>(v.x >> 16));
    x[2] = bf16_bits_to_float(static_cast<uint16_t>(v.y));
    x[3] = bf16_bits_to_float(static_cast<uint16_t>(v.y >> 16));
}
__device__ __forceinline__ void load_cols(const float *p, float (&x)[1]) { x[0] = *p; }
__device__ __forceinline__ void load_cols(const uint16_t *p, float (&x)[1]) {
    x[0] = bf16_bits_to_float(*p);
}

template <typename G, int kCols>
__global__ __launch_bounds__(kThreads) void seg_sum(const G *grads, uint32_t dim, const uint32_t *spos,
                                                    const uint32_t *seg_start, const uint32_t *seg_pos,
                                                    const int64_t *count, uint32_t max_segs,
                                                    float *gsum) {
    const uint32_t runs = dim / kCols;
    const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t seg = t / runs;
    if (seg >= max_segs) return;
    const uint32_t c0 = (t - seg * runs) * kCols;
    const uint32_t lo = seg_start[seg], hi = seg_start[seg + 1], first = seg_pos[seg];
    if (static_cast<int64_t>(seg) >= *count) return;
    float acc[kCols], x[kCols];
    load_cols(grads + static_cast<uint64_t>(first) * dim + c0, x);
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[c] = 0.f + x[c];
    uint32_t i = lo + 1;
    for (; i + 4 <= hi; i += 4) {
        uint32_t q[4];
        float y[4][kCols];
#pragma unroll
        for (int u = 0; u < 4; ++u) q[u] = spos[i + u];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_cols(grads + static_cast<uint64_t>(q[u]) * dim + c0, y[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int c = 0; c < kCols; ++c) acc[c] = acc[c] + y[u][c];
    }
    for (; i < hi; ++i) {
        load_cols(grads + static_cast<uint64_t>(spos[i]) * dim + c0, x);
#pragma unroll
        for (int c = 0; c < kCols; ++c) acc[c] = acc[c] + x[c];
    }
    float *out = gsum + static_cast<uint64_t>(seg) * dim + c0;
    if constexpr (kCols == 4)
        *reinterpret_cast<float4 *>(out) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    else
        out[0] = acc[0];
}

// ---- squared norm ---------------------------------------------------------------------------
constexpr int kSumBlocks = 256;

// Partial sums of x^2: block b sums elements b, b + kSumBlocks*kThreads, ... (grid-stride);
// then one workgroup adds the kSumBlocks partials in order. The order is fixed, so the result
// is deterministic.
__global__ __launch_bounds__(kThreads) void sumsq_partial(const float *x, int64_t n, float *partial) {
    __shared__ float s[kThreads];
    const int tid = threadIdx.x;
    float acc = 0.f;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + tid; i < n;
         i += static_cast<int64_t>(kSumBlocks) * kThreads)
        acc += x[i] * x[i];
    s[tid] = acc;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
        if (tid < off) s[tid] += s[tid + off];
        __syncthreads();
    }
    if (tid == 0) partial[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(kSumBlocks) void sumsq_final(const float *partial, float *out, int accumulate) {
    __shared__ float s[kSumBlocks];
    const int tid = threadIdx.x;
    s[tid] = partial[tid];
    __syncthreads();
    for (int off = kSumBlocks / 2; off > 0; off >>= 1) {
        if (tid < off) s[tid] += s[tid + off];
        __syncthreads();
    }
    if (tid == 0) *out = accumulate ? *out + s[0] : s[0];
}

// ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) ----------------------------------------
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
    constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
    constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(kM0, c.x), lo0 = kM0 * c.x;
        const uint32_t hi1 = __umulhi(kM1, c.z), lo1 = kM1 * c.z;
        c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
        k.x += kW0;
        k.y += kW1;
    }
    return c;
}

// 16 bits of rounding noise for element (row, col) of array `which` (0: weights, 1: first
// moment, 2: per-value second moment) of table `table` at step `step`.
__device__ __forceinline__ uint32_t sr_noise(uint64_t seed, uint32_t step, uint32_t table,
                                             uint64_t row, uint32_t col, uint32_t which) {
    const uint4 ctr = make_uint4(static_cast<uint32_t>(row), static_cast<uint32_t>(row >> 32), step,
                                 (table << 16) | (which << 14) | (col >> 3));
    const uint4 w = philox4x32_10(ctr, make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
    const uint32_t sel = (col >> 1) & 3;
    const uint32_t word = sel == 0 ? w.x : sel == 1 ? w.y : sel == 2 ? w.z : w.w;
    return (word >> (16 * (col & 1))) & 0xffffu;
}

// fp32 -> bf16 bits, stochastic: noise added below the kept 16 bits, then truncated; inf and NaN
// convert as usual (optim.py:39-44).
__device__ __forceinline__ uint16_t stochastic_bf16_bits(float x, uint32_t noise) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u) return float_to_bf16_bits_rne(x);
    return static_cast<uint16_t>((u + noise) >> 16);
}

// ---- lazy / row-wise Adam on touched rows ------------------------------------------------------
struct AdamTable {
    uint8_t *param;        // [rows, dim] of the parameter dtype
    uint8_t *exp_avg;      // like param
    uint8_t *exp_avg_sq;   // row-wise: [rows] fp32; per value: like param
    const int64_t *rows;   // [n] unique row ids
    const float *grads;    // [n, dim] fp32
    int64_t n;
    int64_t first;         // first global row slot of this table in the launch
    float neg_lr_bc1;      // -lr / (1 - beta1^step)
    float sqrt_bc2;        // sqrt(1 - beta2^step)
    uint32_t step;
    uint32_t stream_id;    // RNG stream of this table
};

constexpr int kAdamTables = 32;  // tables per launch (kernel arguments stay under 4 KiB)

struct AdamArgs {
    AdamTable t[kAdamTables];
    int n_tables;
    int64_t total;
    int dim;
    int param_bf16;
    int rowwise;
    int sq_bf16;           // per-value second moment stored as bf16
    int sr;
    int lazy;              // skip rows whose gradient is all zero
    uint64_t seed;
    float decay;           // 1 - lr * weight_decay (1: no decay)
    int has_decay;
    float beta1, one_minus_beta1, beta2, one_minus_beta2, eps;
    const float *sumsq;    // nullable: clip the gradients to max_norm against this squared norm
    float max_norm;
};

__device__ __forceinline__ float load_elem(const uint8_t *base, int bf16, int64_t i) {
    return bf16 ? bf16_bits_to_float(reinterpret_cast<const uint16_t *>(base)[i])
                : reinterpret_cast<const float *>(base)[i];
}

__device__ __forceinline__ void store_elem(uint8_t *base, int bf16, int64_t i, float v, int sr,
                                           uint32_t noise) {
    if (bf16)
        reinterpret_cast<uint16_t *>(base)[i] = sr ? stochastic_bf16_bits(v, noise) : float_to_bf16_bits_rne(v);
    else
        reinterpret_cast<float *>(base)[i] = v;
}

// One wave per touched row; lane c holds columns c, c + 64, ... of the row.
__global__ __launch_bounds__(kThreads) void adam_rows(const AdamArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (slot >= a.total) return;
    int k = 0;
    while (k + 1 < a.n_tables && a.t[k + 1].first <= slot) ++k;
    const AdamTable &t = a.t[k];
    const int64_t i = slot - t.first;
    const int64_t row = *as_global(t.rows + i);
    const int D = a.dim;
    const float *g_row = t.grads + i * D;
    float coef = 1.f;  // gradient clipping (rows.py:224-231): min(max_norm / (norm + 1e-6), 1)
    if (a.sumsq != nullptr) coef = fminf(a.max_norm / (sqrtf(*a.sumsq) + 1e-6f), 1.0f);

    // lazy: a row whose gradient is all zero is skipped entirely (optim.py:92-95)
    bool any = false;
    float gsq = 0.f;
    for (int c = lane; c < D; c += 64) {
        float g = g_row[c];
        if (a.sumsq != nullptr) g *= coef;
        any |= g != 0.f;
        gsq += g * g;
    }
    if (a.lazy && __ballot(any) == 0ull) return;
    if (a.rowwise) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) gsq += __shfl_xor(gsq, off, 64);
    }

    const int64_t prow = row * D;
    float v_row = 0.f, denom_row = 0.f;
    if (a.rowwise) {
        const float v = *as_global(reinterpret_cast<const float *>(t.exp_avg_sq) + row);
        v_row = fmaf(gsq / static_cast<float>(D), a.one_minus_beta2, v * a.beta2);
        denom_row = sqrtf(v_row) / t.sqrt_bc2 + a.eps;
    }
    for (int c = lane; c < D; c += 64) {
        float g = g_row[c];
        if (a.sumsq != nullptr) g *= coef;
        float p = load_elem(t.param, a.param_bf16, prow + c);
        float m = load_elem(t.exp_avg, a.param_bf16, prow + c);
        if (a.has_decay) p = p * a.decay;
        m = fmaf(g, a.one_minus_beta1, m * a.beta1);
        float denom;
        if (a.rowwise) {
            denom = denom_row;
        } else {
            float v = load_elem(t.exp_avg_sq, a.sq_bf16, prow + c);
            v = v * a.beta2 + a.one_minus_beta2 * g * g;
            denom = sqrtf(v) / t.sqrt_bc2 + a.eps;
            const uint32_t nv = a.sr && a.sq_bf16 ? sr_noise(a.seed, t.step, t.stream_id, row, c, 2) : 0u;
            store_elem(t.exp_avg_sq, a.sq_bf16, prow + c, v, a.sr, nv);
        }
        p = p + (t.neg_lr_bc1 * m) / denom;
        const bool rnd = a.sr && a.param_bf16;
        store_elem(t.param, a.param_bf16, prow + c, p, a.sr,
                   rnd ? sr_noise(a.seed, t.step, t.stream_id, row, c, 0) : 0u);
        store_elem(t.exp_avg, a.param_bf16, prow + c, m, a.sr,
                   rnd ? sr_noise(a.seed, t.step, t.stream_id, row, c, 1) : 0u);
    }
    if (a.rowwise && lane == 0) *as_global(reinterpret_cast<float *>(t.exp_avg_sq) + row) = v_row;
}

// Four consecutive columns c0..c0+3 (c0 % 4 == 0) share one Philox call: the same noise
// sr_noise gives each of them (word (col >> 1) & 3, half col & 1 of the call for col >> 3).
__device__ __forceinline__ void sr_noise4(uint64_t seed, uint32_t step, uint32_t table,
                                          uint64_t row, uint32_t c0, uint32_t which,
                                          uint32_t (&nz)[4]) {
    const uint4 ctr = make_uint4(static_cast<uint32_t>(row), static_cast<uint32_t>(row >> 32), step,
                                 (table << 16) | (which << 14) | (c0 >> 3));
    const uint4 w = philox4x32_10(ctr, make_uint2(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)));
    const bool low = ((c0 >> 1) & 3) == 0;
    const uint32_t wa = low ? w.x : w.z, wb = low ? w.y : w.w;
    nz[0] = wa & 0xffffu;
    nz[1] = wa >> 16;
    nz[2] = wb & 0xffffu;
    nz[3] = wb >> 16;
}

__device__ __forceinline__ void load4(const uint8_t *base, int bf16, int64_t e0, float (&x)[4]) {
    if (bf16) {
        const u32x2_v v = *as_global(reinterpret_cast<const u32x2_v *>(base + e0 * 2));
        x[0] = bf16_bits_to_float(static_cast<uint16_t>(v.x));
        x[1] = bf16_bits_to_float(static_cast<uint16_t>(v.x >> 16));
        x[2] = bf16_bits_to_float(static_cast<uint16_t>(v.y));
        x[3] = bf16_bits_to_float(static_cast<uint16_t>(v.y >> 16));
    } else {
        const f32x4_v v = *as_global(reinterpret_cast<const f32x4_v *>(base + e0 * 4));
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    }
}

__device__ __forceinline__ void store4(uint8_t *base, int bf16, int64_t e0, const float (&x)[4],
                                       int sr, const uint32_t (&nz)[4]) {
    if (bf16) {
        uint32_t h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            h[e] = sr ? stochastic_bf16_bits(x[e], nz[e]) : float_to_bf16_bits_rne(x[e]);
        *as_global(reinterpret_cast<u32x2_v *>(base + e0 * 2)) = u32x2_v{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
        *as_global(reinterpret_cast<f32x4_v *>(base + e0 * 4)) = f32x4_v{x[0], x[1], x[2], x[3]};
    }
}

// LPR lanes per touched row, four columns per lane (dim = 4 * LPR), 64 / LPR rows per wave:
// the same update as adam_rows with vector loads, one Philox call per lane per rounded array,
// and the launch's table list staged in LDS (rows of one wave may belong to different tables).
template <int LPR>
__global__ __launch_bounds__(kThreads) void adam_rows_vec(const AdamArgs a) {
    constexpr int kRowsPerWave = 64 / LPR;
    constexpr int kRowsPerBlock = kRowsPerWave * (kThreads / 64);
    constexpr int D = 4 * LPR;
    __shared__ AdamTable s_t[kAdamTables];
    const int tid = threadIdx.x;
    {
        static_assert(sizeof(AdamTable) % 8 == 0, "table record copied as 8-byte words");
        const uint64_t *src = reinterpret_cast<const uint64_t *>(a.t);
        uint64_t *dst = reinterpret_cast<uint64_t *>(s_t);
        const int words = a.n_tables * static_cast<int>(sizeof(AdamTable) / 8);
        for (int w = tid; w < words; w += kThreads) dst[w] = src[w];
    }
    __syncthreads();
    const int lane = tid & 63;
    const int sub = lane & (LPR - 1);
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (tid >> 6) * kRowsPerWave +
                         lane / LPR;
    if (slot >= a.total) return;  // whole rows: the lanes of one row share the slot
    int lo = 0, hi = a.n_tables - 1;  // last table whose first slot is <= slot
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_t[mid].first <= slot) lo = mid; else hi = mid - 1;
    }
    const AdamTable &t = s_t[lo];
    const int c0 = 4 * sub;
    const int64_t i = slot - t.first;
    const int64_t row = *as_global(t.rows + i);
    float g[4];
    load4(reinterpret_cast<const uint8_t *>(t.grads), 0, i * D + c0, g);
    float coef = 1.f;  // gradient clipping (rows.py:224-231): min(max_norm / (norm + 1e-6), 1)
    if (a.sumsq != nullptr) coef = fminf(a.max_norm / (sqrtf(*a.sumsq) + 1e-6f), 1.0f);
    bool any = false;
    float gsq = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (a.sumsq != nullptr) g[e] *= coef;
        any |= g[e] != 0.f;
        gsq += g[e] * g[e];
    }
    // lazy: a row whose gradient is all zero is skipped entirely (optim.py:92-95)
    const uint64_t mask = __ballot(any);
    const uint64_t row_bits = LPR == 64 ? mask : (mask >> ((lane / LPR) * LPR)) & ((1ull << (LPR & 63)) - 1);
    if (a.lazy && row_bits == 0ull) return;
    if (a.rowwise) {
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) gsq += __shfl_xor(gsq, off, 64);
    }
    const int64_t e0 = row * D + c0;
    float p[4], m[4], v[4];
    load4(t.param, a.param_bf16, e0, p);
    load4(t.exp_avg, a.param_bf16, e0, m);
    float v_row = 0.f, denom_row = 0.f;
    if (a.rowwise) {
        const float v0 = *as_global(reinterpret_cast<const float *>(t.exp_avg_sq) + row);
        v_row = fmaf(gsq / static_cast<float>(D), a.one_minus_beta2, v0 * a.beta2);
        denom_row = sqrtf(v_row) / t.sqrt_bc2 + a.eps;
    } else {
        load4(t.exp_avg_sq, a.sq_bf16, e0, v);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (a.has_decay) p[e] = p[e] * a.decay;
        m[e] = fmaf(g[e], a.one_minus_beta1, m[e] * a.beta1);
        float denom = denom_row;
        if (!a.rowwise) {
            v[e] = v[e] * a.beta2 + a.one_minus_beta2 * g[e] * g[e];
            denom = sqrtf(v[e]) / t.sqrt_bc2 + a.eps;
        }
        p[e] = p[e] + (t.neg_lr_bc1 * m[e]) / denom;
    }
    uint32_t nz[4] = {0u, 0u, 0u, 0u};
    if (!a.rowwise) {
        if (a.sr && a.sq_bf16) sr_noise4(a.seed, t.step, t.stream_id, row, c0, 2, nz);
        store4(t.exp_avg_sq, a.sq_bf16, e0, v, a.sr, nz);
    }
    const bool rnd = a.sr && a.param_bf16;
    if (rnd) sr_noise4(a.seed, t.step, t.stream_id, row, c0, 0, nz);
    store4(t.param, a.param_bf16, e0, p, a.sr, nz);
    if (rnd) sr_noise4(a.seed, t.step, t.stream_id, row, c0, 1, nz);
    store4(t.exp_avg, a.param_bf16, e0, m, a.sr, nz);
    if (a.rowwise && sub == 0) *as_global(reinterpret_cast<float *>(t.exp_avg_sq) + row) = v_row;
}

// Standalone stochastic rounding of n fp32 values; element i uses the noise of (row i / 4096,
// column i % 4096) of stream `stream_id` at step `step`, array 0.
__global__ __launch_bounds__(kThreads) void sr_convert(const float *x, int64_t n, uint16_t *out,
                                                       uint64_t seed, uint32_t step, uint32_t stream_id) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const uint64_t row = static_cast<uint64_t>(i) >> 12;
    const uint32_t col = static_cast<uint32_t>(i & 4095);
    out[i] = stochastic_bf16_bits(x[i], sr_noise(seed, step, stream_id, row, col, 0));
}

int sort_bits(int64_t key_bound) {
    int bits = 1;
    while (bits < 63 && (int64_t{1} << bits) < key_bound) ++bits;
    return bits;
}

struct DedupLayout {
    int nblocks, hist_stride;
    size_t keys_b, pos_a, pos_b, hist, heads, seg_start, seg_pos, total;
};

DedupLayout dedup_layout(int64_t n) {
    DedupLayout l{};
    l.nblocks = static_cast<int>(ceil_div(n, kTile));
    auto up = [](size_t x) { return (x + 255) & ~size_t{255}; };
    size_t off = 0;
    l.keys_b = off; off += up(static_cast<size_t>(n) * 8 * 2);  // two key buffers
    l.pos_a = off; off += up(static_cast<size_t>(n) * 4);
    l.pos_b = off; off += up(static_cast<size_t>(n) * 4);
    l.hist_stride = (l.nblocks + 3) & ~3;
    l.hist = off; off += up(static_cast<size_t>(kBins) * l.hist_stride * 4);
    l.heads = off; off += up(static_cast<size_t>(l.nblocks + 1) * 4);
    l.seg_start = off; off += up(static_cast<size_t>(n + 1) * 4);
    l.seg_pos = off; off += up(static_cast<size_t>(n) * 4);
    l.total = off;
    return l;
}

}  // namespace
}  // namespace me

using namespace me;

extern "C" int me_dedup_workspace_size(int64_t n, size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    *bytes = dedup_layout(n).total;
    return ME_OK;
}

extern "C" int me_dedup(const int64_t *keys, int64_t n, int64_t key_bound, const void *grads,
                        int grad_dtype, int32_t dim, int64_t *uniq, int64_t *inv, float *gsum,
                        int64_t *count, void *workspace, size_t workspace_size, void *stream) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "n out of range");
    ME_CHECK_ARG(key_bound >= 1, "key_bound must be positive");
    ME_CHECK_ARG(count != nullptr, "count is null");
    ME_CHECK_ARG(grads == nullptr || grad_dtype == ME_F32 || grad_dtype == ME_BF16,
                 "grad dtype must be fp32 or bf16");
    ME_CHECK_ARG(grads == nullptr || dim >= 1, "dim must be positive");
    hipStream_t s = as_stream(stream);
    if (n == 0) {
        hipLaunchKernelGGL(write_zero_count, dim3(1), dim3(1), 0, s, count);
        return check_launch("me_dedup");
    }
    ME_CHECK_ARG(keys && uniq && inv, "null tensor pointer");
    ME_CHECK_ARG(grads == nullptr || gsum != nullptr, "gsum is null");
    const DedupLayout l = dedup_layout(n);
    if (workspace == nullptr || workspace_size < l.total) {
        set_error("me_dedup: workspace of %zu bytes needed, got %zu", l.total, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    uint64_t *kb[2] = {reinterpret_cast<uint64_t *>(ws + l.keys_b),
                       reinterpret_cast<uint64_t *>(ws + l.keys_b) + n};
    uint32_t *pb[2] = {reinterpret_cast<uint32_t *>(ws + l.pos_a),
                       reinterpret_cast<uint32_t *>(ws + l.pos_b)};
    uint32_t *hist = reinterpret_cast<uint32_t *>(ws + l.hist);
    uint32_t *heads = reinterpret_cast<uint32_t *>(ws + l.heads);
    uint32_t *seg_start = reinterpret_cast<uint32_t *>(ws + l.seg_start);
    uint32_t *seg_pos = reinterpret_cast<uint32_t *>(ws + l.seg_pos);

    const int passes = (sort_bits(key_bound) + 7) / 8;
    const uint64_t *kin = reinterpret_cast<const uint64_t *>(keys);
    const uint32_t *pin = nullptr;
    const dim3 grid(static_cast<unsigned>(l.nblocks)), block(kThreads);
    int cur = 0;
    for (int p = 0; p < passes; ++p) {
        const int shift = 8 * p;
        hipLaunchKernelGGL(rs_hist, grid, block, 0, s, kin, n, shift, hist, l.nblocks, l.hist_stride);
        hipLaunchKernelGGL(rs_scatter, grid, block, 0, s, kin, pin, kb[cur], pb[cur], n, shift, hist,
                           l.hist_stride);
        kin = kb[cur];
        pin = pb[cur];
        cur ^= 1;
    }
    int st = check_launch("me_dedup (sort)");
    if (st != ME_OK) return st;
    hipLaunchKernelGGL(seg_count, grid, block, 0, s, kin, n, heads);
    hipLaunchKernelGGL(seg_write, grid, block, 0, s, kin, pin, n, heads, l.nblocks, uniq, inv,
                       seg_start, seg_pos, count);
    st = check_launch("me_dedup (segments)");
    if (st != ME_OK || grads == nullptr) return st;
    // four columns per thread when every row start is aligned for the vector loads and stores
    const size_t gsz = grad_dtype == ME_F32 ? 4 : 2;
    const bool vec = dim % 4 == 0 && reinterpret_cast<uintptr_t>(grads) % (4 * gsz) == 0 &&
                     reinterpret_cast<uintptr_t>(gsum) % 16 == 0;
    const int64_t threads = n * (vec ? dim / 4 : dim);
    ME_CHECK_ARG(threads < (int64_t{1} << 31), "n * dim = %lld too large for one call",
                 (long long)(n * dim));
    const dim3 sgrid(static_cast<unsigned>(ceil_div(threads, kThreads)));
    const uint32_t d = static_cast<uint32_t>(dim), ns = static_cast<uint32_t>(n);
    if (grad_dtype == ME_F32) {
        const float *g = static_cast<const float *>(grads);
        if (vec)
            hipLaunchKernelGGL((seg_sum<float, 4>), sgrid, block, 0, s, g, d, pin, seg_start, seg_pos,
                               count, ns, gsum);
        else
            hipLaunchKernelGGL((seg_sum<float, 1>), sgrid, block, 0, s, g, d, pin, seg_start, seg_pos,
                               count, ns, gsum);
    } else {
        const uint16_t *g = static_cast<const uint16_t *>(grads);
        if (vec)
            hipLaunchKernelGGL((seg_sum<uint16_t, 4>), sgrid, block, 0, s, g, d, pin, seg_start,
                               seg_pos, count, ns, gsum);
        else
            hipLaunchKernelGGL((seg_sum<uint16_t, 1>), sgrid, block, 0, s, g, d, pin, seg_start,
                               seg_pos, count, ns, gsum);
    }
    return check_launch("me_dedup (sums)");
}

extern "C" int me_sumsq(const float *x, int64_t n, float *out, int accumulate, void *workspace,
                        size_t workspace_size, void *stream) {
    ME_CHECK_ARG(out != nullptr, "out is null");
    ME_CHECK_ARG(n >= 0, "negative n");
    ME_CHECK_ARG(x != nullptr || n == 0, "x is null");
    if (workspace == nullptr || workspace_size < kSumBlocks * sizeof(float)) {
        set_error("me_sumsq: workspace of %zu bytes needed, got %zu", kSumBlocks * sizeof(float),
                  workspace_size);
        return ME_ERR_WORKSPACE;
    }
    float *partial = static_cast<float *>(workspace);
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(sumsq_partial, dim3(kSumBlocks), dim3(kThreads), 0, s, x, n, partial);
    hipLaunchKernelGGL(sumsq_final, dim3(1), dim3(kSumBlocks), 0, s, partial, out, accumulate);
    return check_launch("me_sumsq");
}

extern "C" int me_sparse_adam(int32_t n_tables, void *const *params, void *const *exp_avgs,
                              void *const *exp_avg_sqs, const int64_t *const *rows,
                              const float *const *grads, const int64_t *n_rows,
                              const int64_t *steps, const int32_t *stream_ids, int32_t dim,
                              int param_dtype, int rowwise, int sq_dtype, int lazy, double lr,
                              double beta1, double beta2, double eps, double weight_decay,
                              int stochastic_rounding, uint64_t seed, const float *grad_sumsq,
                              double max_norm, void *stream) {
    ME_CHECK_ARG(n_tables >= 1 && n_tables <= 65536, "n_tables must be in [1, 65536]");
    ME_CHECK_ARG(params && exp_avgs && exp_avg_sqs && rows && grads && n_rows && steps && stream_ids,
                 "null argument array");
    ME_CHECK_ARG(param_dtype == ME_BF16 || param_dtype == ME_F32, "param dtype must be bf16/fp32");
    ME_CHECK_ARG(dim >= 1, "dim must be positive");
    ME_CHECK_ARG(rowwise || sq_dtype == ME_BF16 || sq_dtype == ME_F32, "bad second-moment dtype");
    AdamArgs a{};
    a.dim = dim;
    a.param_bf16 = param_dtype == ME_BF16;
    a.rowwise = rowwise != 0;
    a.sq_bf16 = !rowwise && sq_dtype == ME_BF16;
    a.sr = stochastic_rounding != 0;
    a.lazy = lazy != 0;
    a.seed = seed;
    a.has_decay = weight_decay != 0.0;
    a.decay = static_cast<float>(1.0 - lr * weight_decay);
    a.beta1 = static_cast<float>(beta1);
    a.one_minus_beta1 = static_cast<float>(1.0 - beta1);
    a.beta2 = static_cast<float>(beta2);
    a.one_minus_beta2 = static_cast<float>(1.0 - beta2);
    a.eps = static_cast<float>(eps);
    a.sumsq = grad_sumsq;
    a.max_norm = static_cast<float>(max_norm);
    for (int k = 0; k < n_tables; ++k) {
        ME_CHECK_ARG(n_rows[k] >= 0, "table %d: negative row count", k);
        ME_CHECK_ARG(steps[k] >= 1, "table %d: step must be >= 1", k);
        ME_CHECK_ARG(n_rows[k] == 0 || (params[k] && exp_avgs[k] && exp_avg_sqs[k] && rows[k] && grads[k]),
                     "table %d: null tensor pointer", k);
        ME_CHECK_ARG(stream_ids[k] >= 0 && stream_ids[k] < 65536, "table %d: stream id out of range", k);
    }
    for (int k0 = 0; k0 < n_tables; k0 += kAdamTables) {
        const int nk = min(kAdamTables, n_tables - k0);
        int64_t total = 0;
        for (int q = 0; q < nk; ++q) {
            const int k = k0 + q;
            AdamTable &t = a.t[q];
            t.param = static_cast<uint8_t *>(params[k]);
            t.exp_avg = static_cast<uint8_t *>(exp_avgs[k]);
            t.exp_avg_sq = static_cast<uint8_t *>(exp_avg_sqs[k]);
            t.rows = rows[k];
            t.grads = grads[k];
            t.n = n_rows[k];
            t.first = total;
            const double step = static_cast<double>(steps[k]);
            const double bc1 = 1.0 - std::pow(beta1, step), bc2 = 1.0 - std::pow(beta2, step);
            t.neg_lr_bc1 = static_cast<float>(-lr / bc1);
            t.sqrt_bc2 = static_cast<float>(std::sqrt(bc2));
            t.step = static_cast<uint32_t>(steps[k]);
            t.stream_id = static_cast<uint32_t>(stream_ids[k]);
            total += n_rows[k];
        }
        a.n_tables = nk;
        a.total = total;
        if (total == 0) continue;
        // vector path: dim = 4 * lanes-per-row with lanes-per-row a power of two <= 64, and every
        // row start aligned for 4-element loads
        const int lpr = dim % 4 == 0 ? dim / 4 : 0;
        bool vec = lpr >= 1 && lpr <= 64 && (lpr & (lpr - 1)) == 0;
        const uintptr_t pal = a.param_bf16 ? 8 : 16, val = a.rowwise ? 4 : (a.sq_bf16 ? 8 : 16);
        for (int q = 0; q < nk && vec; ++q) {
            const AdamTable &t = a.t[q];
            vec = reinterpret_cast<uintptr_t>(t.param) % pal == 0 &&
                  reinterpret_cast<uintptr_t>(t.exp_avg) % pal == 0 &&
                  reinterpret_cast<uintptr_t>(t.exp_avg_sq) % val == 0 &&
                  reinterpret_cast<uintptr_t>(t.grads) % 16 == 0;
        }
        hipStream_t s = as_stream(stream);
        if (vec) {
            const int64_t per_block = (64 / lpr) * (kThreads / 64);
            const dim3 grid(static_cast<unsigned>(ceil_div(total, per_block)));
            switch (lpr) {
                case 1: hipLaunchKernelGGL(adam_rows_vec<1>, grid, dim3(kThreads), 0, s, a); break;
                case 2: hipLaunchKernelGGL(adam_rows_vec<2>, grid, dim3(kThreads), 0, s, a); break;
                case 4: hipLaunchKernelGGL(adam_rows_vec<4>, grid, dim3(kThreads), 0, s, a); break;
                case 8: hipLaunchKernelGGL(adam_rows_vec<8>, grid, dim3(kThreads), 0, s, a); break;
                case 16: hipLaunchKernelGGL(adam_rows_vec<16>, grid, dim3(kThreads), 0, s, a); break;
                case 32: hipLaunchKernelGGL(adam_rows_vec<32>, grid, dim3(kThreads), 0, s, a); break;
                default: hipLaunchKernelGGL(adam_rows_vec<64>, grid, dim3(kThreads), 0, s, a); break;
            }
        } else {
            const dim3 grid(static_cast<unsigned>(ceil_div(total, kThreads / 64)));
            hipLaunchKernelGGL(adam_rows, grid, dim3(kThreads), 0, s, a);
        }
        const int st = check_launch("me_sparse_adam");
        if (st != ME_OK) return st;
    }
    return ME_OK;
}

extern "C" int me_stochastic_bf16(const float *x, int64_t n, uint16_t *out, uint64_t seed,
                                  uint32_t step, uint32_t stream_id, void *stream) {
    ME_CHECK_ARG(n >= 0, "negative n");
    ME_CHECK_ARG((x != nullptr && out != nullptr) || n == 0, "null tensor pointer");
    ME_CHECK_ARG(stream_id < 65536, "stream id out of range");
    if (n == 0) return ME_OK;
    hipLaunchKernelGGL(sr_convert, dim3(static_cast<unsigned>(ceil_div(n, kThreads))), dim3(kThreads), 0,
                       as_stream(stream), x, n, out, seed, step, stream_id);
    return check_launch("me_stochastic_bf16");
}
