// Stage 3 for few tokens on gfx950: the key and value projections of the memory vectors,
//   kv[n][j]     = round_T(sum_m mem[n][m] W_K[j][m])        j < d
//   kv[n][d + j] = round_T(sum_m mem[n][m] W_V[j][m])        j < d
// the two nn.Linear calls of MicroEngram.inject (micro_engram/module.py:245, 254), for batches
// too small for the fused gate kernel's 256 x 224 tiles to fill the part (a serving decode step:
// 256 tokens against 10,752 output columns of K = 1536). me_gate_rows then does the gate and
// the residual add from kv.
//
// At this size the GEMM is bound by moving operands into the CUs: the weights (33 MB at the
// Gemma-scale shape) are read once per token tile, the memory vectors once per column tile.
// Measured on MI355X, loads that ask each 128-byte line for half of it (what an MFMA fragment
// loaded straight into registers is: 16 rows x 64 bytes) move the same bytes 1.5x slower than
// loads of whole lines. So operands go through LDS as in the fused gate kernel: a workgroup owns
// a TM-token x TN-column output tile, its K loop streams 128-byte k-slabs (one line of each of
// the TM + TN rows) into a ring of LDS slots with buffer_load ... lds (8 whole rows per
// instruction, no register staging), and its four waves, 2 x 2 over the tile, read their MFMA
// fragments back with ds_read_b128. Rows are XOR-swizzled by (row >> 1) & 7 over their eight
// 16-byte chunks, so a fragment read of 16 consecutive rows covers all LDS banks. R - 1 slabs are
// in flight while one is consumed; one barrier per slab. The tile is then staged in LDS (rounded
// to T) and written as 16-byte row segments.
//
// Output columns are laid out virtually as [K block | V block], each block padded to a multiple
// of 16 columns, so a 16-column MFMA block and an 8-row load read one weight matrix. Rows past the
// token count, padding columns and k past mem_dim read as zeros (per-lane offsets past the
// buffer); nothing outside the real output is stored.
//
// bf16: v_mfma_f32_16x16x32_bf16, a slab is 2 k-steps of 32. fp32: v_mfma_f32_16x16x4f32, a slab
// is 2 k-steps of 16: each lane reads 4 consecutive values and the four MFMAs of the step take
// component i of every lane (the sum runs over the same k in a permuted order in both operands).
#include "me_common.h"

namespace me {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int int32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kSlab = 128;        // bytes of k per row per slab (a cache line)
constexpr int kXcds = 8;
constexpr uint32_t kBufferConfig = 0x00020000u;  // raw buffer descriptor word 3 (gfx9 family)
constexpr int kLdsBytes = 160 * 1024;

struct ProjArgs {
    const uint8_t *mem;   // [n, m] of T
    const uint8_t *wk;    // [d, m] of T
    const uint8_t *wv;    // [d, m] of T
    uint8_t *kv;          // [n, 2d] of T
    int64_t n, d, m;
    int64_t d_pad;        // d rounded up to 16: the V block starts at virtual column d_pad
    uint32_t mem_bytes, w_bytes, row_bytes;
    int slabs;            // ceil(row_bytes / 128)
    int tiles_tok, tiles_total, per_xcd;
};

__device__ __forceinline__ int32x4 rsrc_of(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    int32x4 r;
    r.x = static_cast<int>(static_cast<uint32_t>(a));
    r.y = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xffffu);  // stride 0
    r.z = static_cast<int>(bytes);
    r.w = static_cast<int>(kBufferConfig);
    return r;
}

// 64 lanes x 16 bytes from the buffer (lane's byte voffset; at or past the range: zeros) into
// LDS at lds_base + 16 * lane. Counted by vmcnt, which the caller waits for explicitly.
__device__ __forceinline__ void dma16(const int32x4 &rsrc, uint32_t lds_base, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voffset), "s"(rsrc)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)p));
}

template <typename T>
struct Mma;
template <>
struct Mma<uint16_t> {  // a 16-byte fragment is one k-step of 32
    __device__ __forceinline__ static void run(floatx4 &acc, const u32x4_v &a, const u32x4_v &b) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    }
};
template <>
struct Mma<float> {  // a 16-byte fragment is four k values of each lane group: four MFMAs
    __device__ __forceinline__ static void run(floatx4 &acc, const u32x4_v &a, const u32x4_v &b) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[i]), __uint_as_float(b[i]), acc,
                                                       0, 0, 0);
    }
};

// T: element type; BA x BB 16-row blocks per wave (tokens x columns); waves 2 x 2; R ring slots.
template <typename T, int BA, int BB, int R>
__global__ __launch_bounds__(kThreads) void proj_kernel(const ProjArgs a) {
    constexpr int kEs = sizeof(T);
    constexpr int TM = 2 * 16 * BA;               // tokens per tile
    constexpr int TN = 2 * 16 * BB;               // columns per tile
    constexpr int kRows = TM + TN;                // rows per slab: A (tokens) then B (columns)
    constexpr int kSlot = kRows * kSlab;          // bytes per ring slot
    constexpr int kDma = kRows / 8;               // 8-row loads per slab
    static_assert(kDma % 4 == 0, "each wave issues the same number of loads");
    constexpr int kDmaWave = kDma / 4;
    static_assert(R >= 3 && R * kSlot <= kLdsBytes, "ring must fit in LDS");
    static_assert((R - 2) * kDmaWave <= 63, "vmcnt counts up to 63");
    constexpr int kStagePitch = TN * kEs + 16;    // epilogue staging row: TN values + pad
    static_assert(TM * kStagePitch <= R * kSlot, "epilogue staging must fit in the ring");
    __shared__ __attribute__((aligned(16))) uint8_t ring[R * kSlot];

    const int b = blockIdx.x;  // XCD x takes tiles [x per_xcd, (x+1) per_xcd), token tiles fastest
    const int tile = (b % kXcds) * a.per_xcd + b / kXcds;
    if (tile >= a.tiles_total) return;
    const int tok_tile = tile % a.tiles_tok;
    const int col_tile = tile / a.tiles_tok;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wa = wave & 1, wb = wave >> 1;      // the wave's quarter of the tile
    const int64_t tok0 = static_cast<int64_t>(tok_tile) * TM;
    const int64_t col0 = static_cast<int64_t>(col_tile) * TN;

    const int32x4 rm = rsrc_of(a.mem, a.mem_bytes);
    const int32x4 rk = rsrc_of(a.wk, a.w_bytes);
    const int32x4 rv = rsrc_of(a.wv, a.w_bytes);

    // Load i of this wave fills slab rows 8 (4 i + wave) + [0, 8): lane l takes row + l / 8 at
    // physical chunk l % 8, i.e. logical chunk (l % 8) ^ ((row >> 1) & 7). A lane's row offset
    // and chunk are fixed for the whole K loop; per slab the k offset is added, and a chunk past
    // the row (k tail), a token past n or a padding column reads past its buffer (zeros).
    uint32_t roff[kDmaWave], chk[kDmaWave], lim[kDmaWave];
    int src[kDmaWave];  // 0: mem, 1: W_K, 2: W_V (uniform per load)
#pragma unroll
    for (int i = 0; i < kDmaWave; ++i) {
        const int g8 = 8 * (4 * i + wave);         // first slab row of the load (uniform)
        const int row = g8 + (lane >> 3);
        chk[i] = static_cast<uint32_t>((lane & 7) ^ ((row >> 1) & 7)) * 16u;
        if (g8 < TM) {
            src[i] = 0;
            lim[i] = a.mem_bytes;
            const int64_t r = tok0 + row;
            roff[i] = r < a.n ? static_cast<uint32_t>(r) * a.row_bytes : a.mem_bytes;
        } else {
            const int64_t vc0 = col0 + (g8 - TM);  // virtual column of the load's 8 rows
            src[i] = vc0 < a.d_pad ? 1 : 2;
            lim[i] = a.w_bytes;
            const int64_t jr = (vc0 < a.d_pad ? vc0 : vc0 - a.d_pad) + (lane >> 3);
            roff[i] = (jr < a.d && vc0 < 2 * a.d_pad) ? static_cast<uint32_t>(jr) * a.row_bytes : a.w_bytes;
        }
    }
    const uint32_t ring_lds = lds_addr(ring);
    auto issue = [&](int sl) {
        const uint32_t slot = ring_lds + static_cast<uint32_t>(sl % R) * kSlot;
        const uint32_t kb = static_cast<uint32_t>(sl) * kSlab;
#pragma unroll
        for (int i = 0; i < kDmaWave; ++i) {
            const uint32_t dst = __builtin_amdgcn_readfirstlane(slot + static_cast<uint32_t>(4 * i + wave) * 1024u);
            const bool in = roff[i] < lim[i] && chk[i] + kb < a.row_bytes;
            const uint32_t vo = in ? roff[i] + chk[i] + kb : lim[i];
            dma16(src[i] == 0 ? rm : (src[i] == 1 ? rk : rv), dst, vo);
        }
    };

    floatx4 acc[BA][BB];
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int j = 0; j < BB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // fragment reads: k-step ks of the slab in `slot`; lane l reads row (l & 15) of a 16-row block
    // at logical chunk 4 ks + (l >> 4)
    const int fr = lane & 15;
    const int fq = lane >> 4;
    auto frag = [&](const uint8_t *slot, int row, int ks) {
        const int c = ((4 * ks + fq) ^ ((row >> 1) & 7)) << 4;
        return *reinterpret_cast<const u32x4_v *>(slot + row * kSlab + c);
    };

    const int slabs = a.slabs;
#pragma unroll
    for (int sl = 0; sl < R - 1; ++sl)
        if (sl < slabs) issue(sl);
    for (int sl = 0; sl < slabs; ++sl) {
        // slab sl landed for this wave (later slabs may fly), then for every wave
        if (sl + R - 2 < slabs)
            wait_vmcnt<(R - 2) * kDmaWave>();
        else
            wait_vmcnt<0>();
        __syncthreads();
        // the slot of slab sl - 1 is free: every wave read it before this barrier
        if (sl + R - 1 < slabs) issue(sl + R - 1);
        const uint8_t *slot = ring + (sl % R) * kSlot;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            u32x4_v fa[BA], fb[BB];
#pragma unroll
            for (int i = 0; i < BA; ++i) fa[i] = frag(slot, wa * 16 * BA + 16 * i + fr, ks);
#pragma unroll
            for (int j = 0; j < BB; ++j) fb[j] = frag(slot, TM + wb * 16 * BB + 16 * j + fr, ks);
#pragma unroll
            for (int i = 0; i < BA; ++i)
#pragma unroll
                for (int j = 0; j < BB; ++j) Mma<T>::run(acc[i][j], fa[i], fb[j]);
        }
    }
    __syncthreads();  // every wave is done with the ring (and no load is in flight): stage there

    // acc[i][j] lane l: token 16 i + 4 (l >> 4) + r and column 16 j + (l & 15) of the wave's
    // quarter; staged rounded to T as [TM][TN]
#pragma unroll
    for (int i = 0; i < BA; ++i)
#pragma unroll
        for (int j = 0; j < BB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = wa * 16 * BA + 16 * i + 4 * fq + r;
                const int col = wb * 16 * BB + 16 * j + fr;
                uint8_t *p = ring + row * kStagePitch + col * kEs;
                if constexpr (kEs == 2)
                    *reinterpret_cast<uint16_t *>(p) = float_to_bf16_bits_rne(acc[i][j][r]);
                else
                    *reinterpret_cast<float *>(p) = acc[i][j][r];
            }
    __syncthreads();
    // 16-byte row segments: TM rows x (TN * kEs / 16) segments
    constexpr int kSegs = TN * kEs / 16;
    constexpr int kPerSeg = 16 / kEs;
    const int64_t stride = 2 * a.d;
    for (int it = threadIdx.x; it < TM * kSegs; it += kThreads) {
        const int row = it / kSegs;
        const int seg = it % kSegs;
        const int64_t tok = tok0 + row;
        const int64_t vc = col0 + seg * kPerSeg;  // virtual column: K block, then V block
        const int64_t jr = vc < a.d_pad ? vc : vc - a.d_pad;
        if (tok >= a.n || jr >= a.d || vc >= 2 * a.d_pad) continue;
        const int64_t oc = vc < a.d_pad ? jr : a.d + jr;
        const u32x4_v v = *reinterpret_cast<const u32x4_v *>(ring + row * kStagePitch + seg * 16);
        *as_global(reinterpret_cast<u32x4_v *>(a.kv + (tok * stride + oc) * kEs)) = v;
    }
}

template <typename T, int BA, int BB, int R>
int launch(ProjArgs a, hipStream_t s) {
    constexpr int TM = 32 * BA, TN = 32 * BB;
    a.tiles_tok = static_cast<int>(ceil_div(a.n, TM));
    const int tiles_col = static_cast<int>(ceil_div(2 * a.d_pad, TN));
    a.tiles_total = a.tiles_tok * tiles_col;
    a.per_xcd = static_cast<int>(ceil_div(a.tiles_total, kXcds));
    hipLaunchKernelGGL((proj_kernel<T, BA, BB, R>), dim3(static_cast<unsigned>(a.per_xcd * kXcds)),
                       dim3(kThreads), 0, s, a);
    return check_launch("me_kv_proj");
}

}  // namespace
}  // namespace me

using namespace me;

extern "C" int me_kv_proj(const void *mem, int64_t n, int64_t mem_dim, const void *w_key,
                          const void *w_value, int64_t model_dim, int dtype, void *kv,
                          void *stream) {
    ME_CHECK_ARG(dtype == ME_BF16 || dtype == ME_F32, "dtype must be bf16 or fp32");
    ME_CHECK_ARG(n >= 0 && mem_dim >= 1 && model_dim >= 1, "bad shape");
    if (n == 0) return ME_OK;
    ME_CHECK_ARG(mem && w_key && w_value && kv, "null tensor pointer");
    const int64_t es = static_cast<int64_t>(dtype_size(dtype));
    ME_CHECK_ARG(model_dim % 8 == 0, "model_dim must be a multiple of 8");
    ME_CHECK_ARG((mem_dim * es) % 16 == 0, "mem_dim * element size must be a multiple of 16 bytes");
    ME_CHECK_ARG(n * mem_dim * es < (int64_t{1} << 31) && model_dim * mem_dim * es < (int64_t{1} << 31),
                 "mem and each weight must be under 2 GiB");
    ME_CHECK_ARG(n < (int64_t{1} << 24), "too many tokens for the few-token projection");
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    ME_CHECK_ARG(al16(mem) && al16(w_key) && al16(w_value) && al16(kv), "tensors must be 16-byte aligned");
    ProjArgs a{};
    a.mem = static_cast<const uint8_t *>(mem);
    a.wk = static_cast<const uint8_t *>(w_key);
    a.wv = static_cast<const uint8_t *>(w_value);
    a.kv = static_cast<uint8_t *>(kv);
    a.n = n;
    a.d = model_dim;
    a.m = mem_dim;
    a.d_pad = (model_dim + 15) / 16 * 16;
    a.row_bytes = static_cast<uint32_t>(mem_dim * es);
    a.slabs = static_cast<int>(ceil_div(a.row_bytes, kSlab));
    a.mem_bytes = static_cast<uint32_t>(n * mem_dim * es);
    a.w_bytes = static_cast<uint32_t>(model_dim * mem_dim * es);
    hipStream_t s = as_stream(stream);
    // Tiles (measured on MI355X at model dim 5376, mem dim 1536, bf16): small batches are
    // bound by how many bytes each CU keeps in flight from L2, so they take tiles whose ring
    // leaves room for two workgroups per CU (four slots of 128-byte slabs) -- up to 64 tokens
    // 32 x 96 (10.8 us against 12.8 us with one 64 x 96 workgroup per CU), up to 256 tokens
    // 64 x 96 (a 256-token decode step's projection: 15.8-16.0 us against 17.8 us with 128 x 96
    // and a five-slot ring; 128 x 64, 64 x 128 and 32 x 96 there: 17-20 us) -- and larger batches
    // the 128 x 192 tile, which moves the fewest bytes per MFMA (512 tokens 26.8 us, 1024 tokens
    // 50 us). fp32 (model dim 1024, mem dim 1024): small tiles fill the CUs and two workgroups
    // share one -- up to 768 tokens 32 x 64 (256 tokens 16.7 us against 72.5 with 128 x 128),
    // up to 1024 32 x 128 (40.9 us), above 64 x 128 with a three-slot ring (2048 tokens 72.3 us
    // against 74.8, 8192 tokens 276 against 295).
    if (dtype == ME_BF16) {
        if (n <= 64) return launch<uint16_t, 1, 3, 4>(a, s);
        if (n <= 256) return launch<uint16_t, 2, 3, 4>(a, s);
        return launch<uint16_t, 4, 6, 4>(a, s);
    }
    if (n <= 768) return launch<float, 1, 2, 5>(a, s);
    if (n <= 1024) return launch<float, 1, 4, 4>(a, s);
    return launch<float, 2, 4, 3>(a, s);
}
