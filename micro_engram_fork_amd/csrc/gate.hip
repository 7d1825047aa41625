// Stage 3 of the Engram lookup path on gfx950: the key/value projection of the memory vector
// and the scalar / scalar_sqrt gate, fused into the residual add.
//
// Reference (micro_engram/module.py:228-261), per token n with hidden x (d wide) and memory
// vector e (M wide):
//   K = round_T(W_K e)                       nn.Linear in the engram dtype T (fp32 accumulate)
//   h = rms_norm(x) * q_scale, k = rms_norm(K) * k_scale      (scales only for scalar_sqrt)
//   s = sum(h * k) / sqrt(d); scalar_sqrt: s = sign(s) * sqrt(max(|s|, 1e-6))
//   alpha = sigmoid(s); out = x + round_H(alpha * round_T(W_V e) * keep)
//
// Since h . k = rsqrt(mean x^2 + eps) * rsqrt(mean K^2 + eps) * sum_j x_j qs_j ks_j K_j, the
// gate needs three per-token sums over the model dim. Two launches:
//   key pass    C = W_K[j-tile] x mem[n-tile]^T on MFMA; the epilogue rounds K to T, stages it
//               in LDS and reduces sum K^2, sum x qs ks K and sum x^2 over the tile's columns
//               into a per-(column tile, token) partial (workspace). K never reaches HBM.
//   value pass  alpha per token from the partials (summed in column-tile order, so the result
//               is deterministic), the same GEMM with W_V, and the epilogue writes
//               x + round_H(alpha * round_T(V)) with coalesced 16-byte rows.
//
// GEMM tiling: a 256-thread workgroup owns a 256 (model dims j) x 256 (tokens n) output tile;
// its four waves each hold 128 x 128 as 4 x 4 tiles of v_mfma_f32_32x32x16_bf16 (fp32 engrams:
// v_mfma_f32_32x32x2f32). Both operands are K-contiguous in HBM (W is [d, M], mem is [N, M]).
// The K loop streams 128-byte k-slabs (one cache line of every one of the 256 A rows and 256
// B rows) through five 32 KiB LDS units: slab s's A rows go to unit 2s % 5 and its B rows to
// unit (2s + 1) % 5, so two slabs' worth of loads are in flight while one is consumed.
// buffer_load ... lds moves each 16-byte chunk straight from memory into LDS (no VGPR
// staging); one instruction fills 8 whole 128-byte rows, so every L2 request is a full line
// (64-byte slabs asked for each line twice, and the L1 address path, not the L2, set the
// pace). Out-of-range rows or K read as zeros through the buffer's range check. Within a row
// the eight 16-byte chunks are XOR-swizzled by ((row >> 1) & 7), so the 16 lanes a
// ds_read_b128 serves per cycle (16 consecutive rows at one logical chunk) cover all 64 LDS
// banks. A slab is four 16-wide k-steps and one workgroup barrier, placed in the last k-step:
// every fragment read of the slab is done by then, so the loads refilling its units and the
// reads of the next slab's first fragments run under that k-step's MFMAs.
// Epilogues: each wave stages its 128 x 128 tile of round_T(C) in LDS, then walks token rows
// with 16 lanes x 16 bytes per row, so every hidden load and output store is a coalesced
// 256-byte row segment. The key pass reduces its three sums per row across the 16 lanes with
// DPP row shifts and combines the two column waves in LDS. Workgroup ids are remapped so the
// 32 CUs of one XCD work on a compact group of tiles (8 token tiles x 4 column tiles) and share
// their operands in that XCD's L2. bf16 forward passes run the same scheme on 256 x 224 tiles
// of 16x16x32 MFMAs (gate224_kernel: whole rounds of tiles on the Gemma-scale shape).
#include "me_common.h"

#include <mutex>
#include <type_traits>

namespace me {
namespace {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int int32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kTile = 256;                         // output tile edge (j and n)
constexpr int kSlab = 128;                         // bytes of K per row per slab (a cache line)
constexpr int kUnit = kTile * kSlab;               // 32 KiB: one operand of one slab
constexpr int kUnits = 5;
constexpr int kRingBytes = kUnits * kUnit;         // 160 KiB
constexpr int kDmaPerOperand = kUnit / (kThreads * 16);  // 16-byte loads per thread: 8
constexpr int kStagePitch = 256 + 8;               // epilogue staging row: 256 B + pad
constexpr int kWaveStage = 128 * kStagePitch;      // one wave's staged 128-row tile
constexpr int kGroupTiles = 8;                     // token tiles per XCD group
constexpr int kXcds = 8;
constexpr uint32_t kBufferConfig = 0x00020000u;    // raw buffer descriptor word 3 (gfx9 family)
constexpr int kStoreNT = 2;                        // buffer store cache policy bit: non-temporal
static_assert(4 * kWaveStage + 2 * kTile * 3 * 4 <= kRingBytes, "epilogue must fit in the ring");

// Forward passes (key, value) and the backward's two passes over the same GEMM tiles.
enum Phase : int { kKey = 0, kValue = 1, kGradValue = 2, kGradKey = 3 };

struct GateArgs {
    const uint8_t *hidden;  // [n, d] of H
    const uint8_t *mem;     // [n, m] of T
    const uint8_t *w;       // [d, m] of T (W_K in the key pass, W_V in the value pass)
    const void *q_delta;    // [d] scale - 1 (nullable: scalar gate)
    const void *k_delta;
    const uint8_t *keep;    // [n] (nullable)
    uint8_t *out;           // [n, d] of H
    float *alpha_out;       // [n] (nullable)
    float *partials;        // [n_jt][n][3] per-column-tile sums (sum K^2, sum x qs ks K, sum x^2)
    float *alpha_eff;       // [n] gate of each token, 0 where keep is false
    int64_t n, d, m;
    uint32_t mem_bytes, w_bytes;  // buffer ranges (reads past them return zeros)
    uint32_t hidden_bytes, scale_bytes;  // ranges of the prefetched epilogue operands
    float *row_stats_out;   // forward, nullable: [n][4] sum x^2, sum K^2, sum x qs ks K, alpha
    // backward
    const uint8_t *grad_out;   // [n, d] of H: gradient of the output
    const float *row_stats;    // [n][4] the forward's row_stats_out
    uint8_t *grad_hidden;      // [n, d] of H
    uint8_t *grad_proj;        // [n, d] of T: dV (value side) or dK (key side)
    float *grad_partials;      // [n_jt][n] per-column-tile sums of g . V
    float *tok_coef;           // [n][3] per-token coefficients of the key side (a, c2, c3)
    float *col_partials;       // [n_nt][d] per-token-tile column sums of a x K
    int scale_bf16;
    int sqrt_mode;
    int n_jt, n_nt, total_tiles, per_xcd;
    float inv_d, inv_sqrt_d;
};

// ---- element access helpers -----------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float to_f(T v);
template <>
__device__ __forceinline__ float to_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f<uint16_t>(uint16_t v) { return bf16_bits_to_float(v); }

template <typename T>
__device__ __forceinline__ T from_f(float v);
template <>
__device__ __forceinline__ float from_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f<uint16_t>(float v) { return float_to_bf16_bits_rne(v); }

// Rounding of a value to storage type T, kept as float.
template <typename T>
__device__ __forceinline__ float round_t(float v) { return to_f<T>(from_f<T>(v)); }

// Two floats rounded to bf16 (nearest, ties to even) in one word, `lo` in the low half: one
// v_cvt_pk_bf16_f32 for the pair.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_v __attribute__((ext_vector_type(3)));
typedef float float2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// E consecutive elements of X (E * sizeof(X) a multiple of 8 bytes, 8-byte aligned) as floats.
template <typename X, int E>
__device__ __forceinline__ void load_run(const uint8_t *p, float (&v)[E]) {
    constexpr int kWords = E * sizeof(X) / 4;
    uint32_t w[kWords];
#pragma unroll
    for (int q = 0; q < kWords; q += 2) {
        const uint2 u = reinterpret_cast<const uint2 *>(p)[q / 2];
        w[q] = u.x;
        w[q + 1] = u.y;
    }
    const X *x = reinterpret_cast<const X *>(w);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = to_f<X>(x[e]);
}

// ---- memory -> LDS without registers ---------------------------------------------------------
__device__ __forceinline__ int32x4 buffer_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    int32x4 r;
    r.x = static_cast<int>(static_cast<uint32_t>(a));
    r.y = static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xffffu);  // stride 0
    r.z = static_cast<int>(bytes);
    r.w = static_cast<int>(kBufferConfig);
    return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)p));
}

// One wave moves 64 x 16 bytes: lane l's chunk at byte `voffset` of the buffer lands at LDS
// address lds_base + 16 * l. A voffset at or past the buffer's range reads zeros. The load is
// counted by vmcnt; the caller waits for it explicitly (the compiler does not see it).
__device__ __forceinline__ void dma16(const int32x4 &rsrc, uint32_t lds_base, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voffset), "s"(rsrc)
                 : "memory");
}

// The same with a uniform byte offset soffset added to every lane's voffset (the buffer's range
// check looks at voffset, so an out-of-range voffset still reads zeros).
__device__ __forceinline__ void dma16_so(const int32x4 &rsrc, uint32_t lds_base, uint32_t voffset,
                                         uint32_t soffset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voffset), "s"(rsrc), "s"(soffset)
                 : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// ---- MFMA k-steps ----------------------------------------------------------------------------
// A slab's A rows sit in LDS unit ua and its B rows in unit ub, [256 rows][128 B] swizzled; a
// slab is four 16-wide (bf16) k-steps. The wave's A rows are wj*128 + [0,128), its B rows
// wn*128 + [0,128). For k-step ks, lane l reads row (l & 31) of each 32-row subtile at logical
// chunk 2*ks + (l >> 5): lanes 0-31 carry one half of the step's k values and lanes 32-63 the
// other, identically for A and B, which is all the dot product needs.
template <typename T>
struct Frag;
template <>
struct Frag<uint16_t> {
    bf16x8 a[4], b[4];
};
template <>
struct Frag<float> {
    float4 a[4], b[4];
};

// Part p of a fragment: A subtile p (p < 4) or B subtile p - 4.
template <typename T>
__device__ __forceinline__ void load_frag_part(const uint8_t *ua, const uint8_t *ub, int ks, int wj,
                                               int wn, int lane, Frag<T> &f, int p) {
    const int r = lane & 31;
    const int c = ((2 * ks + (lane >> 5)) ^ ((r >> 1) & 7)) << 4;
    using V = decltype(f.a[0]);
    using VV = typename std::remove_reference<V>::type;
    if (p < 4)
        f.a[p] = *reinterpret_cast<const VV *>(ua + (wj * 128 + p * 32 + r) * kSlab + c);
    else
        f.b[p - 4] = *reinterpret_cast<const VV *>(ub + (wn * 128 + (p - 4) * 32 + r) * kSlab + c);
}

// The product of A subtile x and B subtile y for one k-step.
__device__ __forceinline__ void mfma_xy(const Frag<uint16_t> &f, floatx16 (&acc)[4][4], int x, int y) {
    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[x], f.b[y], acc[x][y], 0, 0, 0);
}
__device__ __forceinline__ void mfma_xy(const Frag<float> &f, floatx16 (&acc)[4][4], int x, int y) {
    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[x].x, f.b[y].x, acc[x][y], 0, 0, 0);
    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[x].y, f.b[y].y, acc[x][y], 0, 0, 0);
    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[x].z, f.b[y].z, acc[x][y], 0, 0, 0);
    acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[x].w, f.b[y].w, acc[x][y], 0, 0, 0);
}

// Element e of an accumulator tile, read out of its accumulation register in program order.
// The staging after the K loop reads one subtile at a time this way: left to itself the
// compiler copies all 256 accumulators into VGPRs at the loop exit, which leaves no room for
// anything else live there (the prefetched epilogue operands).
__device__ __forceinline__ float acc_read(const floatx16 &t, int e) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(t[e]));
    return v;
}

// Sum over the 16 lanes of a DPP row (lanes 16i .. 16i+15), exact in lane 16i + 15: an inclusive
// scan by row shifts of 1, 2, 4 and 8 (out-of-row sources read as 0).
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xf, 0xf, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xf, 0xf, true));
    return v;
}

__device__ __forceinline__ float gate_alpha(float sx2, float sk2, float sck, const GateArgs &a) {
    constexpr float kEps = 1.1920928955078125e-07f;  // torch.finfo(float32).eps: rms_norm default
    const float rh = 1.0f / sqrtf(sx2 * a.inv_d + kEps);
    const float rk = 1.0f / sqrtf(sk2 * a.inv_d + kEps);
    float s = rh * rk * sck * a.inv_sqrt_d;
    if (a.sqrt_mode) {
        const float sg = s > 0.f ? 1.f : (s < 0.f ? -1.f : 0.f);
        s = sg * sqrtf(fmaxf(fabsf(s), 1e-6f));
    }
    return 1.0f / (1.0f + expf(-s));
}

template <typename T, typename H, int PHASE>
__global__ __launch_bounds__(kThreads, 1) void gate_kernel(const GateArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[kRingBytes];

    // ---- tile of this workgroup: XCD-compact groups of 8 token tiles x all column tiles
    const int bid = blockIdx.x;
    const int logical = (bid % kXcds) * a.per_xcd + bid / kXcds;
    if (logical >= a.total_tiles) return;
    const int group_size = kGroupTiles * a.n_jt;
    const int group = logical / group_size;
    const int in_group = logical - group * group_size;
    const int first_nt = group * kGroupTiles;
    const int group_nts = min(kGroupTiles, a.n_nt - first_nt);
    const int nt = first_nt + in_group % group_nts;
    const int jt = in_group / group_nts;
    const int64_t j0 = static_cast<int64_t>(jt) * kTile;
    const int64_t n0 = static_cast<int64_t>(nt) * kTile;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wj = wave >> 1, wn = wave & 1;

    // the value pass reads its tokens' gates now; they are parked in LDS after the K loop
    float alpha_reg = 0.f;
    if (PHASE == kValue && n0 + tid < a.n) alpha_reg = a.alpha_eff[n0 + tid];
    // the backward's value side: the gate of the token with keep folded in; key side: the
    // token's coefficients (zero past the last token, so those rows add nothing)
    float coef_reg[3] = {0.f, 0.f, 0.f};
    if (PHASE == kGradValue && n0 + tid < a.n) {
        alpha_reg = a.row_stats[(n0 + tid) * 4 + 3];
        if (a.keep != nullptr && a.keep[n0 + tid] == 0) alpha_reg = 0.f;
    }
    if (PHASE == kGradKey && n0 + tid < a.n) {
#pragma unroll
        for (int c = 0; c < 3; ++c) coef_reg[c] = a.tok_coef[(n0 + tid) * 3 + c];
    }

    // ---- epilogue row walk geometry: 16 lanes x 16 bytes per token row, lane l16 owning
    // kLaneCols columns, rows rsub, rsub + 4, ... of the wave's 128
    constexpr int kPasses = sizeof(T) == 2 ? 1 : 2;
    constexpr int kPassCols = 128 / kPasses;     // columns staged per pass
    constexpr int kLaneCols = 16 / sizeof(T);    // columns per lane in the row walk (8 / 4)
    constexpr int kRowWords = kLaneCols * sizeof(H) / 4;  // hidden words per lane per row
    constexpr int kBatch = kRowWords <= 4 ? 32 : 16;      // rows whose hidden loads are in flight
    const int l16 = lane & 15, rsub = lane >> 4;
    const int64_t ntok0 = n0 + wn * 128;          // first token of the wave

    // ---- K loop over 128-byte slabs: A_s (W rows) in unit 2s % 5, B_s (mem rows) in (2s+1) % 5
    const uint32_t row_bytes = static_cast<uint32_t>(a.m * sizeof(T));
    const int slabs = static_cast<int>(ceil_div(row_bytes, kSlab));
    const int32x4 rsrc_w = buffer_rsrc(a.w, a.w_bytes);
    const int32x4 rsrc_m = buffer_rsrc(a.mem, a.mem_bytes);
    // load i of a wave fills rows 8 (8 wave + i) + [0, 8): lane l writes row + l / 8 at physical
    // chunk l % 8, which holds the row's logical chunk (l % 8) ^ ((row >> 1) & 7)
    uint32_t offw[kDmaPerOperand], offm[kDmaPerOperand], chunk[kDmaPerOperand];
    bool okw[kDmaPerOperand], okm[kDmaPerOperand];
#pragma unroll
    for (int i = 0; i < kDmaPerOperand; ++i) {
        const int row = (wave * kDmaPerOperand + i) * 8 + (lane >> 3);
        chunk[i] = static_cast<uint32_t>((lane & 7) ^ ((row >> 1) & 7)) * 16u;
        okw[i] = j0 + row < a.d;
        okm[i] = n0 + row < a.n;
        offw[i] = okw[i] ? static_cast<uint32_t>(j0 + row) * row_bytes + chunk[i] : 0u;
        offm[i] = okm[i] ? static_cast<uint32_t>(n0 + row) * row_bytes + chunk[i] : 0u;
    }
    const uint32_t ring_lds = lds_addr(ring);
    // load i of operand op (0: A, 1: B) of slab sl
    auto issue = [&](int sl, int op, int i) {
        const uint32_t kb = static_cast<uint32_t>(sl) * kSlab;
        const bool kin = kb + chunk[i] < row_bytes;
        const uint32_t dst = ring_lds + static_cast<uint32_t>((2 * sl + op) % kUnits) * kUnit +
                             static_cast<uint32_t>(wave * kDmaPerOperand + i) * 1024u;
        if (op == 0)
            dma16(rsrc_w, __builtin_amdgcn_readfirstlane(dst), okw[i] && kin ? offw[i] + kb : a.w_bytes);
        else
            dma16(rsrc_m, __builtin_amdgcn_readfirstlane(dst), okm[i] && kin ? offm[i] + kb : a.mem_bytes);
    };
    auto unit_a = [&](int sl) { return ring + ((2 * sl) % kUnits) * kUnit; };
    auto unit_b = [&](int sl) { return ring + ((2 * sl + 1) % kUnits) * kUnit; };
    floatx16 acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.f;

    // Slab s issues A_{s+2} under its k-step 0 (into B_{s-1}'s unit, free since the previous
    // barrier) and B_{s+2} after its barrier (into A_s's unit). Slabs past the end are issued
    // with out-of-range offsets, which write zeros into units nobody reads, so the number of
    // loads issued after any awaited one is fixed and every wait is a constant.
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int op = 0; op < 2; ++op)
#pragma unroll
            for (int i = 0; i < kDmaPerOperand; ++i) issue(sl, op, i);
    wait_vmcnt<2 * kDmaPerOperand>();  // A_0, B_0 landed (A_1, B_1 may fly)
    __syncthreads();
    Frag<T> f0, f1;
#pragma unroll
    for (int p = 0; p < 8; ++p) load_frag_part<T>(unit_a(0), unit_b(0), 0, wj, wn, lane, f0, p);
    // Every non-MFMA instruction of a slab is issued between MFMAs, where it costs the matrix
    // pipe nothing: k-steps 0-2 carry the reads of the next k-step's fragments (k-step 0 also
    // the loads of A_{s+2}); k-step 3 issues four MFMAs, waits for slab s+1 (A_{s+2} may still
    // fly), passes the barrier (every wave is done reading slab s), then carries the loads of
    // B_{s+2} and the reads of slab s+1's first fragments (the parts its first MFMAs need
    // come first). sched_barrier pins this order.
    constexpr int kFragOrder[8] = {0, 4, 5, 6, 7, 1, 2, 3};  // a0, b0..b3, a1..a3
    auto slab = [&](int sl, auto wait, auto dma) {
        const uint8_t *ua = unit_a(sl), *ub = unit_b(sl);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            mfma_xy(f0, acc, i >> 2, i & 3);
            __builtin_amdgcn_sched_barrier(0);
            if (decltype(dma)::value && i < kDmaPerOperand) {
                issue(sl + 2, 0, i);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (i & 1) {
                load_frag_part<T>(ua, ub, 1, wj, wn, lane, f1, kFragOrder[i >> 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            mfma_xy(f1, acc, i >> 2, i & 3);
            __builtin_amdgcn_sched_barrier(0);
            if (i & 1) {
                load_frag_part<T>(ua, ub, 2, wj, wn, lane, f0, kFragOrder[i >> 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            mfma_xy(f0, acc, i >> 2, i & 3);
            __builtin_amdgcn_sched_barrier(0);
            if (i & 1) {
                load_frag_part<T>(ua, ub, 3, wj, wn, lane, f1, kFragOrder[i >> 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mfma_xy(f1, acc, i >> 2, i & 3);
            __builtin_amdgcn_sched_barrier(0);
        }
        // slab s+1 landed: A_{s+2} may still fly
        if constexpr (decltype(wait)::value == 1) wait_vmcnt<kDmaPerOperand>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *na = unit_a(sl + 1), *nb = unit_b(sl + 1);
#pragma unroll
        for (int i = 4; i < 16; ++i) {
            mfma_xy(f1, acc, i >> 2, i & 3);
            __builtin_amdgcn_sched_barrier(0);
            const int q = i - 4;
            if (decltype(dma)::value && q < kDmaPerOperand) {
                issue(sl + 2, 1, q);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (q < 8) {  // past the last slab these read a stale unit; they are not used
                load_frag_part<T>(na, nb, 0, wj, wn, lane, f0, kFragOrder[q]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    using WaitSlab = std::integral_constant<int, 1>;
    using Dma = std::true_type;
    for (int sl = 0; sl < slabs; ++sl) slab(sl, WaitSlab{}, Dma{});
    wait_vmcnt<0>();  // the trailing out-of-range loads still write the ring
    __syncthreads();  // the ring is free for the epilogue

    // ---- epilogue: each wave stages round_T of its 128 x 128 tile as [token][column] rows
    // (pitch kStagePitch), then walks its token rows with 16 lanes x 16 bytes per row. fp32
    // tiles go in two column halves of 64.
    uint8_t *stage = ring + wave * kWaveStage;
    float *s_aux = reinterpret_cast<float *>(ring + 4 * kWaveStage);  // [2][256][3] or [256]
    const int r = lane & 31, half = lane >> 5;

    // s_aux: key [2 wj][256 tokens][3] sums; value [256] gates; grad value [256] gates then
    // [2 wj][256] sums of g . V; grad key [256][3] coefficients then [2 wn][256 columns]
    if (PHASE == kValue) {
        s_aux[tid] = alpha_reg;
    } else if (PHASE == kKey) {
        for (int e = tid; e < 2 * kTile * 3; e += kThreads) s_aux[e] = 0.f;
    } else if (PHASE == kGradValue) {
        s_aux[tid] = alpha_reg;
        s_aux[kTile + tid] = 0.f;
        s_aux[2 * kTile + tid] = 0.f;
    } else {
#pragma unroll
        for (int c = 0; c < 3; ++c) s_aux[tid * 3 + c] = coef_reg[c];
        s_aux[3 * kTile + tid] = 0.f;
        s_aux[4 * kTile + tid] = 0.f;
    }

    for (int pass = 0; pass < kPasses; ++pass) {
        // stage: acc[x][y][4g + e] is token 32y + r, column 32x + 8g + 4*half + e
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            if (kPasses == 2 && (x >> 1) != pass) continue;
#pragma unroll
            for (int y = 0; y < 4; ++y)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = (x % (4 / kPasses)) * 32 + 8 * g + 4 * half;
                    uint32_t w[sizeof(T)];
                    T *tv = reinterpret_cast<T *>(w);
#pragma unroll
                    for (int e = 0; e < 4; ++e) tv[e] = from_f<T>(acc_read(acc[x][y], 4 * g + e));
                    uint8_t *p = stage + (y * 32 + r) * kStagePitch + col * sizeof(T);
                    reinterpret_cast<uint2 *>(p)[0] = make_uint2(w[0], w[1]);
                    if constexpr (sizeof(T) == 4) reinterpret_cast<uint2 *>(p)[1] = make_uint2(w[2], w[3]);
                    if (g == 3) __builtin_amdgcn_sched_barrier(0);
                }
        }
        __syncthreads();  // staging (and s_aux) visible

        const int64_t jl = j0 + wj * 128 + pass * kPassCols + l16 * kLaneCols;  // lane's first column
        const bool jok = jl < a.d;  // d is a multiple of 8: a lane's columns are all in or all out
        float wcol[kLaneCols];  // q_scale * k_scale of the lane's columns (key pass)
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) wcol[e] = 1.f;
        constexpr bool kScaled = PHASE == kKey || PHASE == kGradKey;
        if (kScaled && jok && a.q_delta != nullptr) {
            float qv[kLaneCols], kv[kLaneCols];
            if (a.scale_bf16) {
                load_run<uint16_t, kLaneCols>(static_cast<const uint8_t *>(a.q_delta) + jl * 2, qv);
                load_run<uint16_t, kLaneCols>(static_cast<const uint8_t *>(a.k_delta) + jl * 2, kv);
            } else {
                load_run<float, kLaneCols>(static_cast<const uint8_t *>(a.q_delta) + jl * 4, qv);
                load_run<float, kLaneCols>(static_cast<const uint8_t *>(a.k_delta) + jl * 4, kv);
            }
#pragma unroll
            for (int e = 0; e < kLaneCols; ++e) wcol[e] = (1.f + qv[e]) * (1.f + kv[e]);
        }
        // rows of hidden (forward, key side of the backward) or of the output gradient (value
        // side); the key side of the backward reads both, in half-size batches
        constexpr int kRowBatch = PHASE == kGradKey ? kBatch / 2 : kBatch;
        float colp[kLaneCols];  // grad key: sums of a x K over the lane's rows
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) colp[e] = 0.f;
        const uint8_t *src0 = PHASE == kGradValue ? a.grad_out : a.hidden;
        for (int b0 = 0; b0 < 32; b0 += kRowBatch) {
            uint32_t xr[kRowBatch][kRowWords];
            uint32_t gr[PHASE == kGradKey ? kRowBatch : 1][kRowWords];
#pragma unroll
            for (int u = 0; u < kRowBatch; ++u) {
                const int row = (b0 + u) * 4 + rsub;
                const int64_t n = ntok0 + row;
                if (jok && n < a.n) {
                    const int64_t off = (n * a.d + jl) * static_cast<int64_t>(sizeof(H));
#pragma unroll
                    for (int q = 0; q < kRowWords; q += 2) {
                        const uint2 v = reinterpret_cast<const uint2 *>(src0 + off)[q / 2];
                        xr[u][q] = v.x;
                        xr[u][q + 1] = v.y;
                    }
                    if constexpr (PHASE == kGradKey) {
#pragma unroll
                        for (int q = 0; q < kRowWords; q += 2) {
                            const uint2 v = reinterpret_cast<const uint2 *>(a.grad_out + off)[q / 2];
                            gr[u][q] = v.x;
                            gr[u][q + 1] = v.y;
                        }
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < kRowWords; ++q) xr[u][q] = 0u;
                    if constexpr (PHASE == kGradKey) {
#pragma unroll
                        for (int q = 0; q < kRowWords; ++q) gr[u][q] = 0u;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < kRowBatch; ++u) {
                const int row = (b0 + u) * 4 + rsub;
                const int64_t n = ntok0 + row;
                const uint8_t *sp = stage + row * kStagePitch + (l16 * kLaneCols) * sizeof(T);
                uint32_t cw[4];
                const uint2 c0 = reinterpret_cast<const uint2 *>(sp)[0];
                const uint2 c1 = reinterpret_cast<const uint2 *>(sp)[1];
                cw[0] = c0.x; cw[1] = c0.y; cw[2] = c1.x; cw[3] = c1.y;
                const T *cv = reinterpret_cast<const T *>(cw);
                const H *xv = reinterpret_cast<const H *>(xr[u]);
                if (PHASE == kKey) {
                    float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
#pragma unroll
                    for (int e = 0; e < kLaneCols; ++e) {
                        const float kv = to_f<T>(cv[e]);
                        const float x = to_f<H>(xv[e]);
                        sk2 += kv * kv;
                        sck += x * wcol[e] * kv;
                        sx2 += x * x;
                    }
                    sk2 = row16_sum(sk2);
                    sck = row16_sum(sck);
                    sx2 = row16_sum(sx2);
                    if (l16 == 15) {
                        float *p = s_aux + (wj * kTile + wn * 128 + row) * 3;
                        p[0] += sk2;
                        p[1] += sck;
                        p[2] += sx2;
                    }
                } else if (PHASE == kValue) {
                    if (jok && n < a.n) {
                        const float alpha = s_aux[wn * 128 + row];
                        uint32_t ow[kRowWords];
                        H *ov = reinterpret_cast<H *>(ow);
#pragma unroll
                        for (int e = 0; e < kLaneCols; ++e)
                            ov[e] = from_f<H>(to_f<H>(xv[e]) + round_t<H>(alpha * to_f<T>(cv[e])));
                        // non-temporal: the output is not read again by this kernel, and written
                        // through it leaves no dirty lines for the next kernel's traffic to evict
                        uint8_t *p = a.out + (n * a.d + jl) * static_cast<int64_t>(sizeof(H));
#pragma unroll
                        for (int q = 0; q < kRowWords; q += 2)
                            __builtin_nontemporal_store(u32x2_t{ow[q], ow[q + 1]},
                                                        reinterpret_cast<u32x2_t *>(p) + q / 2);
                    }
                } else if (PHASE == kGradValue) {
                    // d alpha gets sum_j g_j V_j (keep is applied per token later); dV = alpha g,
                    // rounded to the engram dtype as the cast after the projection rounds it
                    const float alpha = s_aux[wn * 128 + row];
                    float gv = 0.f;
                    uint32_t dw[4];
                    T *dv = reinterpret_cast<T *>(dw);
#pragma unroll
                    for (int e = 0; e < kLaneCols; ++e) {
                        const float g = to_f<H>(xv[e]);
                        gv += g * to_f<T>(cv[e]);
                        dv[e] = from_f<T>(alpha * g);
                    }
                    gv = row16_sum(gv);
                    if (l16 == 15) s_aux[kTile + wj * kTile + wn * 128 + row] += gv;
                    if (jok && n < a.n) {
                        uint8_t *p = a.grad_proj + (n * a.d + jl) * static_cast<int64_t>(sizeof(T));
                        *reinterpret_cast<uint4 *>(p) = make_uint4(dw[0], dw[1], dw[2], dw[3]);
                    }
                } else {  // kGradKey
                    // with the token's coefficients (ca, c2, c3) and w = q_scale k_scale:
                    //   d hidden = g + round(ca w K - c2 x), dK = ca w x - c3 K, scales: ca x K
                    const float *cf = s_aux + (wn * 128 + row) * 3;
                    const float ca = cf[0], c2 = cf[1], c3 = cf[2];
                    const H *gv = reinterpret_cast<const H *>(gr[u]);
                    uint32_t hw[kRowWords], kw[4];
                    H *hv = reinterpret_cast<H *>(hw);
                    T *kv = reinterpret_cast<T *>(kw);
#pragma unroll
                    for (int e = 0; e < kLaneCols; ++e) {
                        const float K = to_f<T>(cv[e]);
                        const float x = to_f<H>(xv[e]);
                        const float dx = ca * wcol[e] * K - c2 * x;
                        hv[e] = from_f<H>(to_f<H>(gv[e]) + round_t<H>(dx));
                        kv[e] = from_f<T>(ca * wcol[e] * x - c3 * K);
                        colp[e] += ca * x * K;
                    }
                    if (jok && n < a.n) {
                        const int64_t off = n * a.d + jl;
                        uint8_t *ph = a.grad_hidden + off * static_cast<int64_t>(sizeof(H));
#pragma unroll
                        for (int q = 0; q < kRowWords; q += 2)
                            reinterpret_cast<uint2 *>(ph)[q / 2] = make_uint2(hw[q], hw[q + 1]);
                        uint8_t *pk = a.grad_proj + off * static_cast<int64_t>(sizeof(T));
                        *reinterpret_cast<uint4 *>(pk) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
                    }
                }
            }
        }
        if constexpr (PHASE == kGradKey) {
            // column sums over the wave's 128 tokens: the four row groups of a column block are
            // lanes l16, l16 + 16, l16 + 32, l16 + 48
#pragma unroll
            for (int e = 0; e < kLaneCols; ++e) {
                colp[e] += __shfl_xor(colp[e], 16, 64);
                colp[e] += __shfl_xor(colp[e], 32, 64);
            }
            if (rsub == 0) {
                const int c0 = wj * 128 + pass * kPassCols + l16 * kLaneCols;
#pragma unroll
                for (int e = 0; e < kLaneCols; ++e) s_aux[(3 + wn) * kTile + c0 + e] = colp[e];
            }
        }
        __syncthreads();  // the staging area is reused by the next pass; s_aux is complete
    }

    if (PHASE == kKey) {
        const int64_t n = n0 + tid;
        if (n < a.n) {
            const float *p0 = s_aux + tid * 3;
            const float *p1 = s_aux + (kTile + tid) * 3;
            float *o = a.partials + (static_cast<int64_t>(jt) * a.n + n) * 3;
            o[0] = p0[0] + p1[0];
            o[1] = p0[1] + p1[1];
            o[2] = p0[2] + p1[2];
        }
    } else if (PHASE == kGradValue) {
        const int64_t n = n0 + tid;
        if (n < a.n)
            a.grad_partials[static_cast<int64_t>(jt) * a.n + n] =
                s_aux[kTile + tid] + s_aux[2 * kTile + tid];
    } else if (PHASE == kGradKey) {
        const int64_t j = j0 + tid;
        if (j < a.d)
            a.col_partials[static_cast<int64_t>(nt) * a.d + j] =
                s_aux[3 * kTile + tid] + s_aux[4 * kTile + tid];
    }
}

// ---- 224-column tiles: bf16 forward passes on 16x16x32 MFMAs ------------------------------------
// The forward passes for bf16 engrams and bf16 hidden states (under 2 GiB) run on 256 (tokens) x
// 224 (columns) tiles; gate_kernel serves every other case. On the Gemma-scale shape (d 5376 =
// 24 x 224, 8192 tokens) that is 768 tiles, three full rounds of 256 CUs, where 256 x 256 tiles
// make 672 and leave 96 CUs idle in the third round. Each wave owns 128 tokens x 112 columns as
// 7 x 8 tiles of v_mfma_f32_16x16x32_bf16 (224 accumulators); a slab is two 32-wide k-steps. A
// slab's 224 W rows take 7 row loads per wave, its 256 mem rows 8. The ring, the swizzle, the
// load/barrier order and the epilogue follow gate_kernel. Under the last three slabs the
// workgroup also loads the first of each lane's 32 hidden rows into registers (16 with the key
// pass's scale deltas; 8 with the key pass's partial sums of the value pass's tokens, from which
// the value pass computes its gates after the K loop), so their latency and the HBM burst of
// every CU reaching its epilogue at once overlap the MFMAs; the other rows are loaded as the K
// loop ends.
constexpr int kTJ = 224;                // output columns per tile
constexpr int kWJ = kTJ / 2;            // columns per wave (112)
constexpr int kSubJ = kWJ / 16;         // 16-row A subtiles per wave (7)
constexpr int kSubN = 128 / 16;         // 16-row B subtiles per wave (8)
constexpr int kDmaA = kTJ / (8 * 4);    // A row loads per wave per slab (7)
constexpr int kDmaB = kTile / (8 * 4);  // B row loads per wave per slab (8)
constexpr int kParts = kSubJ + kSubN;   // fragment parts per k-step (15)
constexpr int kPitch16 = kWJ * 2 + 8;   // staged token row: 224 B + pad
constexpr int kWaveStage16 = 128 * kPitch16;
static_assert(4 * kWaveStage16 + 2 * kTile * 3 * 4 <= kRingBytes, "epilogue must fit in the ring");
static_assert(kTJ * kSlab <= kUnit, "a slab's W rows fit a ring unit");

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct Frag16 {
    bf16x8 a[kSubJ], b[kSubN];
};

__device__ __forceinline__ float acc_read4(const floatx4 &t, int e) {
    float v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(t[e]));
    return v;
}

// Part p of a k-step's fragments (A subtile p for p < 7, else B subtile p - 7): lane l reads row
// (l & 15) of the subtile at logical chunk 4 ks + (l >> 4) (8 of the k-step's 32 k values; the
// same lanes carry the same k values for A and B).
__device__ __forceinline__ void load_part16(const uint8_t *ua, const uint8_t *ub, int ks, int wj, int wn,
                                            int lane, Frag16 &f, int p) {
    const int r = lane & 15;
    if (p < kSubJ) {
        const int row = wj * kWJ + p * 16 + r;
        const int c = ((4 * ks + (lane >> 4)) ^ ((row >> 1) & 7)) << 4;
        f.a[p] = *reinterpret_cast<const bf16x8 *>(ua + row * kSlab + c);
    } else {
        const int row = wn * 128 + (p - kSubJ) * 16 + r;
        const int c = ((4 * ks + (lane >> 4)) ^ ((row >> 1) & 7)) << 4;
        f.b[p - kSubJ] = *reinterpret_cast<const bf16x8 *>(ub + row * kSlab + c);
    }
}

template <int PHASE>
__global__ __launch_bounds__(kThreads, 1) void gate224_kernel(const GateArgs a) {
    using T = uint16_t;
    using H = uint16_t;
    __shared__ __attribute__((aligned(16))) uint8_t ring[kRingBytes];

    // ---- tile of this workgroup: XCD-compact groups of 8 token tiles x all column tiles
    const int bid = blockIdx.x;
    const int logical = (bid % kXcds) * a.per_xcd + bid / kXcds;
    if (logical >= a.total_tiles) return;
    const int group_size = kGroupTiles * a.n_jt;
    const int group = logical / group_size;
    const int in_group = logical - group * group_size;
    const int first_nt = group * kGroupTiles;
    const int group_nts = min(kGroupTiles, a.n_nt - first_nt);
    const int nt = first_nt + in_group % group_nts;
    const int jt = in_group / group_nts;
    const int64_t j0 = static_cast<int64_t>(jt) * kTJ;
    const int64_t n0 = static_cast<int64_t>(nt) * kTile;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wj = wave >> 1, wn = wave & 1;


    // ---- epilogue row walk geometry: 14 of 16 lanes x 16 bytes per token row (the wave's 112
    // columns), lane l16 owning 8 columns, rows rsub, rsub + 4, ... of the wave's 128 tokens
    constexpr int kLaneCols = 8;
    const int l16 = lane & 15, rsub = lane >> 4;
    const int64_t ntok0 = n0 + wn * 128;
    const int64_t jl = j0 + wj * kWJ + l16 * kLaneCols;  // lane's first column
    const bool jok = l16 < kWJ / kLaneCols && jl < a.d;  // d is a multiple of 8
    // hidden rows 0..kPfRows-1 are loaded under the last slabs, the rest at the epilogue start;
    // with them the key pass loads its scale deltas and the value pass the key pass's partial
    // sums of token n0 + tid (kPartLoads column tiles, always that many loads so that the slab
    // waits count a fixed number; the ones past n_jt read zeros and are not summed)
    // The backward's passes (kGradValue: V and the output gradient g; kGradKey: K, hidden and g)
    // load nothing under their slabs; their per-token values (the gate with keep folded in, or
    // the three coefficients) are read before the K loop and used after it.
    constexpr int kPfRows = PHASE == kKey ? 16 : (PHASE == kValue ? 8 : 0);
    constexpr int kPartLoads = 24;
    constexpr int kPfLoads = PHASE == kKey ? kPfRows + 4 : (PHASE == kValue ? kPfRows + kPartLoads : 0);
    const int64_t n_tok = n0 + tid;
    const bool parts_late = PHASE == kValue && a.n_jt <= kPartLoads;
    float alpha_reg = 0.f;
    float coef_reg[3] = {0.f, 0.f, 0.f};
    // the gate of token n_tok, summed in column tile order exactly as gate_alpha_kernel sums
    // them (the tiles of column tile 0 also write the gates and row stats the caller asked for)
    auto set_alpha = [&](float sk2, float sck, float sx2) {
        float alpha = gate_alpha(sx2, sk2, sck, a);
        if (jt == 0) {
            if (a.alpha_out != nullptr) a.alpha_out[n_tok] = alpha;
            if (a.row_stats_out != nullptr) {
                float *st = a.row_stats_out + n_tok * 4;
                st[0] = sx2;
                st[1] = sk2;
                st[2] = sck;
                st[3] = alpha;
            }
        }
        if (a.keep != nullptr && a.keep[n_tok] == 0) alpha = 0.f;
        alpha_reg = alpha;
    };
    u32x3_v part[PHASE == kValue ? kPartLoads : 1];
    u32x4_v xpre[32];
    u32x4_v spre[PHASE == kKey || PHASE == kGradKey ? 4 : 1];
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.hidden), 0, static_cast<int>(a.hidden_bytes), kBufferConfig);
    // byte offset of the lane's 16 bytes in its row u (token ntok0 + 4u + rsub) of hidden and of
    // the output (same layout): the lane's first row plus u row strides, or the range end (reads
    // zeros, stores nothing) for a row past n or a lane past d; hidden is under 2 GiB
    const int rows_left = jok ? static_cast<int>(max(min(a.n - (ntok0 + rsub), static_cast<int64_t>(kTile)),
                                                     static_cast<int64_t>(0)))
                              : 0;
    const uint32_t xoff0 = jok ? static_cast<uint32_t>(((ntok0 + rsub) * a.d + jl) * 2) : 0u;
    const uint32_t xstride = static_cast<uint32_t>(a.d * 8);  // four rows
    auto row_off = [&](int u) { return 4 * u < rows_left ? xoff0 + static_cast<uint32_t>(u) * xstride : a.hidden_bytes; };
    const __amdgpu_buffer_rsrc_t ro =
        __builtin_amdgcn_make_buffer_rsrc(a.out, 0, static_cast<int>(a.hidden_bytes), kBufferConfig);
    auto load_rows = [&](int u0, int u1) {
#pragma unroll
        for (int u = u0; u < u1; ++u)
            xpre[u] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rh, row_off(u), 0, 0));
    };
    // the scale deltas of the lane's 8 columns (key pass, grad-key pass)
    auto load_scales = [&]() {
        const int esz = a.scale_bf16 ? 2 : 4;
        const uint32_t off = jok ? static_cast<uint32_t>(jl * esz) : a.scale_bytes;
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void *>(a.q_delta), 0, static_cast<int>(a.scale_bytes), kBufferConfig);
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void *>(a.k_delta), 0, static_cast<int>(a.scale_bytes), kBufferConfig);
        spre[0] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
        spre[1] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rq, off + 16, 0, 0));
        spre[2] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
        spre[3] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rk, off + 16, 0, 0));
    };
    auto prefetch = [&]() {
        if constexpr (PHASE == kKey) {
            load_rows(0, kPfRows);
            load_scales();
        } else if constexpr (PHASE == kValue) {
            load_rows(0, kPfRows);
            // the partials are [n_jt][n][3] floats (n * d < 2^30 here, so under 2^31 bytes)
            const uint32_t pbytes = static_cast<uint32_t>(a.n_jt * a.n * 12);
            const __amdgpu_buffer_rsrc_t rp =
                __builtin_amdgcn_make_buffer_rsrc(a.partials, 0, static_cast<int>(pbytes), kBufferConfig);
            const uint32_t pv = parts_late && n_tok < a.n ? static_cast<uint32_t>(n_tok * 12) : pbytes;
#pragma unroll
            for (int t = 0; t < kPartLoads; ++t)
                part[t] = __builtin_amdgcn_raw_buffer_load_b96(rp, t < a.n_jt ? pv : pbytes,
                                                               static_cast<uint32_t>(t * a.n * 12), 0);
        }
    };

    // ---- K loop over 128-byte slabs: A_s (W rows) in unit 2s % 5, B_s (mem rows) in (2s+1) % 5
    const uint32_t row_bytes = static_cast<uint32_t>(a.m * sizeof(T));
    const int slabs = static_cast<int>(ceil_div(row_bytes, kSlab));
    const int32x4 rsrc_w = buffer_rsrc(a.w, a.w_bytes);
    const int32x4 rsrc_m = buffer_rsrc(a.mem, a.mem_bytes);
    // A load i of a wave fills rows 8 (7 wave + i) + [0, 8), B load i rows 8 (8 wave + i) + [0, 8):
    // lane l writes row + l / 8 at physical chunk l % 8 (logical chunk (l % 8) ^ ((row >> 1) & 7)).
    // A lane's byte offset of each load is fixed for the whole K loop (out-of-range rows: the
    // buffer size, which reads zeros); the slab's offset goes in the scalar offset, and the LDS
    // destination is computed on scalars, so a load costs a few scalar instructions between two
    // 16-cycle MFMAs. Every slab issued is a whole one (row_bytes % 128 == 0, at least 3 slabs,
    // so the peeled tail issues none past the end).
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(wave));
    uint32_t offw[kDmaA], offm[kDmaB];
#pragma unroll
    for (int i = 0; i < kDmaA; ++i) {
        const int row = (wave * kDmaA + i) * 8 + (lane >> 3);
        const uint32_t ch = static_cast<uint32_t>((lane & 7) ^ ((row >> 1) & 7)) * 16u;
        offw[i] = j0 + row < a.d ? static_cast<uint32_t>(j0 + row) * row_bytes + ch : a.w_bytes;
    }
#pragma unroll
    for (int i = 0; i < kDmaB; ++i) {
        const int row = (wave * kDmaB + i) * 8 + (lane >> 3);
        const uint32_t ch = static_cast<uint32_t>((lane & 7) ^ ((row >> 1) & 7)) * 16u;
        offm[i] = n0 + row < a.n ? static_cast<uint32_t>(n0 + row) * row_bytes + ch : a.mem_bytes;
    }
    const uint32_t ring_lds = lds_addr(ring);
    // LDS destination of a load: the wave's first row in the unit, made opaque on a scalar register
    // per load so that the compiler adds the load's 1 KiB step there (left alone it keeps fifteen
    // hoisted destinations in vector registers and moves each back to a scalar: two vector
    // instructions and a wait state per load)
    const uint32_t wa0 = __builtin_amdgcn_readfirstlane(ring_lds + wave_s * (kDmaA * 1024u));
    const uint32_t wb0 = __builtin_amdgcn_readfirstlane(ring_lds + wave_s * (kDmaB * 1024u));
    auto issue_a = [&](int sl, int i) {
        uint32_t dst = wa0 + static_cast<uint32_t>((2 * sl) % kUnits) * kUnit;
        asm volatile("" : "+s"(dst));
        dma16_so(rsrc_w, dst + static_cast<uint32_t>(i) * 1024u, offw[i], static_cast<uint32_t>(sl) * kSlab);
    };
    auto issue_b = [&](int sl, int i) {
        uint32_t dst = wb0 + static_cast<uint32_t>((2 * sl + 1) % kUnits) * kUnit;
        asm volatile("" : "+s"(dst));
        dma16_so(rsrc_m, dst + static_cast<uint32_t>(i) * 1024u, offm[i], static_cast<uint32_t>(sl) * kSlab);
    };
    auto unit_a = [&](int sl) { return ring + ((2 * sl) % kUnits) * kUnit; };
    auto unit_b = [&](int sl) { return ring + ((2 * sl + 1) % kUnits) * kUnit; };
    floatx4 acc[kSubJ][kSubN];
#pragma unroll
    for (int x = 0; x < kSubJ; ++x)
#pragma unroll
        for (int y = 0; y < kSubN; ++y)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[x][y][e] = 0.f;

#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
#pragma unroll
        for (int i = 0; i < kDmaA; ++i) issue_a(sl, i);
#pragma unroll
        for (int i = 0; i < kDmaB; ++i) issue_b(sl, i);
    }
    // the backward's per-token values, loaded while the first slabs land (issued after their
    // row loads, so the first slab wait does not wait for them)
    if (PHASE == kGradValue && n_tok < a.n) {
        alpha_reg = a.row_stats[n_tok * 4 + 3];
        if (a.keep != nullptr && a.keep[n_tok] == 0) alpha_reg = 0.f;
    }
    if (PHASE == kGradKey && n_tok < a.n) {
#pragma unroll
        for (int c = 0; c < 3; ++c) coef_reg[c] = a.tok_coef[n_tok * 3 + c];
    }
    // value pass, more than kPartLoads column tiles: the gate of token n0 + tid from the key
    // pass's partial sums while the first slabs land (otherwise the sums are loaded with the
    // epilogue prefetch and the gate is computed after the K loop)
    if (PHASE == kValue && !parts_late && n_tok < a.n) {
        float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
#pragma unroll 8
        for (int t = 0; t < a.n_jt; ++t) {
            const float *p = a.partials + (static_cast<int64_t>(t) * a.n + n_tok) * 3;
            sk2 += p[0];
            sck += p[1];
            sx2 += p[2];
        }
        set_alpha(sk2, sck, sx2);
    }
    wait_vmcnt<kDmaA + kDmaB>();  // A_0, B_0 landed (A_1, B_1 may fly; loads issued after them only
                                  // make this wait longer)
    __syncthreads();
    Frag16 f0, f1;
    // fragment parts in the order the next k-step's MFMAs use them: a0, b0..b7, a1..a6
    auto part_of = [](int q) { return q == 0 ? 0 : (q <= kSubN ? kSubJ + q - 1 : q - kSubN); };
#pragma unroll
    for (int q = 0; q < kParts; ++q) load_part16(unit_a(0), unit_b(0), 0, wj, wn, lane, f0, part_of(q));

    constexpr int kMfma = kSubJ * kSubN;  // 56 per k-step
    const int pf_at = max(slabs - 3, 0);
    static_assert(kPfLoads + kDmaA + kDmaB <= 63, "vmcnt counts up to 63");
    // Slab s: k-step 0 issues A_{s+2} (into B_{s-1}'s unit, free since the previous barrier) and
    // reads k-step 1's fragments; k-step 1 waits for slab s+1 after its first kPre MFMAs, passes
    // the barrier, then issues B_{s+2} (into A_s's unit) and reads slab s+1's first fragments.
    // The row loads go one per kSpreadA (kSpreadB) MFMAs: the four waves leave the barrier
    // together, and back-to-back loads from all of them queue up behind each other and hold
    // the MFMAs between them (measured: 281 -> 273 us for the two passes on the Gemma-scale shape).
    constexpr int kSpreadA = 7, kSpreadB = 4;
    auto slab = [&](int sl, auto wait, auto dma) {
        const uint8_t *ua = unit_a(sl), *ub = unit_b(sl);
#pragma unroll
        for (int i = 0; i < kMfma; ++i) {
            acc[i / kSubN][i % kSubN] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                f0.a[i / kSubN], f0.b[i % kSubN], acc[i / kSubN][i % kSubN], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (decltype(dma)::value && i % kSpreadA == 0 && i / kSpreadA < kDmaA) {
                issue_a(sl + 2, i / kSpreadA);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (i % 3 == 2 && i / 3 < kParts) {
                load_part16(ua, ub, 1, wj, wn, lane, f1, part_of(i / 3));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // MFMAs of k-step 1 before the wait and the barrier (on the Gemma-scale shape 12 and 16
        // took 3 and 6 us longer for the two passes: the barrier waits less for the slowest wave)
        constexpr int kPre = 20;
        // every fragment read of the next k-step has an MFMA slot: k-step 0 reads after every
        // third MFMA, k-step 1 after every second one past the barrier (B loads first)
        static_assert(3 * kParts <= kMfma && kPre + 2 * kParts <= kMfma &&
                          kSpreadA * (kDmaA - 1) < kMfma && kSpreadB * (kDmaB - 1) < kMfma - kPre,
                      "fragment reads and loads fit the k-steps' MFMAs");
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
            acc[i / kSubN][i % kSubN] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                f1.a[i / kSubN], f1.b[i % kSubN], acc[i / kSubN][i % kSubN], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        // slab s+1 landed: A_{s+2} (or, in the slab after the prefetch, the prefetch) may still
        // fly; past the last slab there is nothing to wait for
        if constexpr (decltype(wait)::value == 1) wait_vmcnt<kDmaA>();
        if constexpr (decltype(wait)::value == 2) wait_vmcnt<kPfLoads>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *na = unit_a(sl + 1), *nb = unit_b(sl + 1);
#pragma unroll
        for (int i = kPre; i < kMfma; ++i) {
            acc[i / kSubN][i % kSubN] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                f1.a[i / kSubN], f1.b[i % kSubN], acc[i / kSubN][i % kSubN], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            const int q = i - kPre;
            if (decltype(dma)::value && q % kSpreadB == 0 && q / kSpreadB < kDmaB) {
                issue_b(sl + 2, q / kSpreadB);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (q % 2 == 1 && q / 2 < kParts) {  // past the last slab these read a stale unit; unused
                load_part16(na, nb, 0, wj, wn, lane, f0, part_of(q / 2));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    using WaitSlab = std::integral_constant<int, 1>;
    using WaitPrefetch = std::integral_constant<int, 2>;
    using NoWait = std::integral_constant<int, 0>;
    using Dma = std::true_type;
    using NoDma = std::false_type;
    for (int sl = 0; sl < pf_at; ++sl) slab(sl, WaitSlab{}, Dma{});
    slab(pf_at, WaitSlab{}, Dma{});
    prefetch();
    if (pf_at + 1 < slabs) slab(pf_at + 1, WaitPrefetch{}, NoDma{});
    for (int sl = pf_at + 2; sl < slabs; ++sl) slab(sl, NoWait{}, NoDma{});
    wait_vmcnt<0>();  // the trailing out-of-range loads still write the ring
    __syncthreads();  // the ring is free for the epilogue
    // operands of the backward's epilogues: the output gradient g (read) and the gradients
    // written, all [n, d] bf16 like hidden (same byte offsets)
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.grad_out), 0, static_cast<int>(a.hidden_bytes), kBufferConfig);
    const __amdgpu_buffer_rsrc_t rgp =
        __builtin_amdgcn_make_buffer_rsrc(a.grad_proj, 0, static_cast<int>(a.hidden_bytes), kBufferConfig);
    const __amdgpu_buffer_rsrc_t rgh =
        __builtin_amdgcn_make_buffer_rsrc(a.grad_hidden, 0, static_cast<int>(a.hidden_bytes), kBufferConfig);
    if constexpr (PHASE == kKey || PHASE == kValue) {
        load_rows(kPfRows, 32);
    } else if constexpr (PHASE == kGradValue) {
#pragma unroll
        for (int u = 0; u < 32; ++u)
            xpre[u] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rg, row_off(u), 0, 0));
    } else {
        if (a.q_delta != nullptr) load_scales();
    }
    if (parts_late && n_tok < a.n) {
        float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
#pragma unroll
        for (int t = 0; t < kPartLoads; ++t)
            if (t < a.n_jt) {
                sk2 += __uint_as_float(part[t][0]);
                sck += __uint_as_float(part[t][1]);
                sx2 += __uint_as_float(part[t][2]);
            }
        set_alpha(sk2, sck, sx2);
    }

    // ---- epilogue: each wave stages round_T of its 128 x 112 tile as [token][column] rows
    uint8_t *stage = ring + wave * kWaveStage16;
    // s_aux: key [2 wj][256 tokens][3] sums; value [256] gates; grad value [256] gates, then
    // [2 wj][256] sums of g . V; grad key [256][3] coefficients, then [2 wn][224 columns]
    float *s_aux = reinterpret_cast<float *>(ring + 4 * kWaveStage16);
    if (PHASE == kValue || PHASE == kGradValue) {
        s_aux[tid] = alpha_reg;
    } else if (PHASE == kKey) {
        for (int e = tid; e < 2 * kTile * 3; e += kThreads) s_aux[e] = 0.f;
    } else {
#pragma unroll
        for (int c = 0; c < 3; ++c) s_aux[tid * 3 + c] = coef_reg[c];
    }
    // acc[x][y][e] is column 16x + 4 (lane >> 4) + e of token 16y + (lane & 15)
    {
        const int tr = lane & 15, cq = lane >> 4;
#pragma unroll
        for (int x = 0; x < kSubJ; ++x)
#pragma unroll
            for (int y = 0; y < kSubN; ++y) {
                uint32_t w[2];
                T *tv = reinterpret_cast<T *>(w);
#pragma unroll
                for (int e = 0; e < 4; ++e) tv[e] = from_f<T>(acc_read4(acc[x][y], e));
                *reinterpret_cast<uint2 *>(stage + (16 * y + tr) * kPitch16 + (16 * x + 4 * cq) * 2) =
                    make_uint2(w[0], w[1]);
                if (y == kSubN - 1) __builtin_amdgcn_sched_barrier(0);
            }
    }
    __syncthreads();  // staging (and s_aux) visible

    float wcol[kLaneCols];  // q_scale * k_scale of the lane's columns (key and grad-key passes)
#pragma unroll
    for (int e = 0; e < kLaneCols; ++e) wcol[e] = 1.f;
    if ((PHASE == kKey || PHASE == kGradKey) && jok && a.q_delta != nullptr) {
        const uint32_t *qw = reinterpret_cast<const uint32_t *>(&spre[0]);
        const uint32_t *kw = reinterpret_cast<const uint32_t *>(&spre[2]);
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) {
            float qv, kv;
            if (a.scale_bf16) {
                qv = bf16_bits_to_float(static_cast<uint16_t>(qw[e / 2] >> (16 * (e & 1))));
                kv = bf16_bits_to_float(static_cast<uint16_t>(kw[e / 2] >> (16 * (e & 1))));
            } else {
                qv = __uint_as_float(qw[e]);
                kv = __uint_as_float(kw[e]);
            }
            wcol[e] = (1.f + qv) * (1.f + kv);
        }
    }
    // the staged row of the lane's 8 columns; lanes 14 and 15 of a row hold no columns: in the
    // value pass they read the pad and the next row (or the gates past the last row; all inside
    // the ring) and store nothing, elsewhere they take zeros so that row sums ignore them
    auto staged = [&](int row, uint32_t (&cw)[4]) {
        cw[0] = cw[1] = cw[2] = cw[3] = 0u;
        if (PHASE == kValue || l16 < kWJ / kLaneCols) {
            const uint8_t *sp = stage + row * kPitch16 + l16 * 16;
            const uint2 c0 = reinterpret_cast<const uint2 *>(sp)[0];
            const uint2 c1 = reinterpret_cast<const uint2 *>(sp)[1];
            cw[0] = c0.x; cw[1] = c0.y; cw[2] = c1.x; cw[3] = c1.y;
        }
    };
    if constexpr (PHASE != kGradKey) {
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            const int row = u * 4 + rsub;
            uint32_t cw[4];
            staged(row, cw);
            const T *cv = reinterpret_cast<const T *>(cw);
            const u32x4_v xq = xpre[u];
            uint32_t xw[4] = {xq[0], xq[1], xq[2], xq[3]};
            const H *xv = reinterpret_cast<const H *>(xw);
            if constexpr (PHASE == kKey) {
                float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
#pragma unroll
                for (int e = 0; e < kLaneCols; ++e) {
                    const float kv = to_f<T>(cv[e]);
                    const float x = to_f<H>(xv[e]);
                    sk2 += kv * kv;
                    sck += x * wcol[e] * kv;
                    sx2 += x * x;
                }
                sk2 = row16_sum(sk2);
                sck = row16_sum(sck);
                sx2 = row16_sum(sx2);
                if (l16 == 15) {
                    float *p = s_aux + (wj * kTile + wn * 128 + row) * 3;
                    p[0] = sk2;
                    p[1] = sck;
                    p[2] = sx2;
                }
            } else if constexpr (PHASE == kValue) {
                // x + round(alpha * V), V already rounded, two columns per conversion; a row past
                // n or a lane past d stores nothing (its offset is the range end)
                const float alpha = s_aux[wn * 128 + row];
                u32x4_v o;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t av = pack_bf16(alpha * bf16_lo(cw[h]), alpha * bf16_hi(cw[h]));
                    o[h] = pack_bf16(bf16_lo(xw[h]) + bf16_lo(av), bf16_hi(xw[h]) + bf16_hi(av));
                }
                __builtin_amdgcn_raw_buffer_store_b128(o, ro, row_off(u), 0, kStoreNT);
            } else {
                // grad value: d alpha gets sum_j g_j V_j (keep is applied per token later);
                // dV = alpha g, rounded to the engram dtype as the cast after the projection
                // rounds it (xw holds g here)
                const float alpha = s_aux[wn * 128 + row];
                float gv = 0.f;
                u32x4_v dv;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float g0 = bf16_lo(xw[h]), g1 = bf16_hi(xw[h]);
                    gv += g0 * bf16_lo(cw[h]);
                    gv += g1 * bf16_hi(cw[h]);
                    dv[h] = pack_bf16(alpha * g0, alpha * g1);
                }
                gv = row16_sum(gv);
                if (l16 == 15) s_aux[kTile + wj * kTile + wn * 128 + row] = gv;
                __builtin_amdgcn_raw_buffer_store_b128(dv, rgp, row_off(u), 0, kStoreNT);
            }
        }
    } else {
        // grad key, with the token's coefficients (ca, c2, c3) and w = q_scale k_scale:
        //   d hidden = g + round(ca w K - c2 x), dK = ca w x - c3 K, scales: sum of ca x K;
        // hidden and g rows are loaded eight rows at a time
        float colp[kLaneCols];
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) colp[e] = 0.f;
        constexpr int kGkBatch = 8;
        for (int b0 = 0; b0 < 32; b0 += kGkBatch) {
            u32x4_v xb[kGkBatch], gb[kGkBatch];
#pragma unroll
            for (int v = 0; v < kGkBatch; ++v) {
                xb[v] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rh, row_off(b0 + v), 0, 0));
                gb[v] = __builtin_bit_cast(u32x4_v, __builtin_amdgcn_raw_buffer_load_b128(rg, row_off(b0 + v), 0, 0));
            }
#pragma unroll
            for (int v = 0; v < kGkBatch; ++v) {
                const int u = b0 + v;
                const int row = u * 4 + rsub;
                uint32_t cw[4];
                staged(row, cw);
                const float *cf = s_aux + (wn * 128 + row) * 3;
                const float ca = cf[0], c2 = cf[1], c3 = cf[2];
                u32x4_v hv, kv;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    float K[2] = {bf16_lo(cw[h]), bf16_hi(cw[h])};
                    float x[2] = {bf16_lo(xb[v][h]), bf16_hi(xb[v][h])};
                    float g[2] = {bf16_lo(gb[v][h]), bf16_hi(gb[v][h])};
                    float dh[2], dk[2];
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const float w = wcol[2 * h + q];
                        const float dx = ca * w * K[q] - c2 * x[q];
                        dh[q] = g[q] + round_t<H>(dx);
                        dk[q] = ca * w * x[q] - c3 * K[q];
                        colp[2 * h + q] += ca * x[q] * K[q];
                    }
                    hv[h] = pack_bf16(dh[0], dh[1]);
                    kv[h] = pack_bf16(dk[0], dk[1]);
                }
                __builtin_amdgcn_raw_buffer_store_b128(hv, rgh, row_off(u), 0, kStoreNT);
                __builtin_amdgcn_raw_buffer_store_b128(kv, rgp, row_off(u), 0, kStoreNT);
            }
        }
        // column sums over the wave's 128 tokens: the four row groups of a column are lanes
        // l16, l16 + 16, l16 + 32, l16 + 48
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) {
            colp[e] += __shfl_xor(colp[e], 16, 64);
            colp[e] += __shfl_xor(colp[e], 32, 64);
        }
        if (rsub == 0 && l16 < kWJ / kLaneCols) {
            float *pc = s_aux + 3 * kTile + wn * kTJ + wj * kWJ + l16 * kLaneCols;
#pragma unroll
            for (int e = 0; e < kLaneCols; ++e) pc[e] = colp[e];
        }
    }
    if constexpr (PHASE == kKey) {
        __syncthreads();  // s_aux complete
        const int64_t n = n0 + tid;
        if (n < a.n) {
            const float *p0 = s_aux + tid * 3;
            const float *p1 = s_aux + (kTile + tid) * 3;
            float *o = a.partials + (static_cast<int64_t>(jt) * a.n + n) * 3;
            o[0] = p0[0] + p1[0];
            o[1] = p0[1] + p1[1];
            o[2] = p0[2] + p1[2];
        }
    } else if constexpr (PHASE == kGradValue) {
        __syncthreads();  // s_aux complete
        const int64_t n = n0 + tid;
        if (n < a.n)
            a.grad_partials[static_cast<int64_t>(jt) * a.n + n] = s_aux[kTile + tid] + s_aux[2 * kTile + tid];
    } else if constexpr (PHASE == kGradKey) {
        __syncthreads();  // s_aux complete
        const int64_t j = j0 + tid;
        if (tid < kTJ && j < a.d)
            a.col_partials[static_cast<int64_t>(nt) * a.d + j] =
                s_aux[3 * kTile + tid] + s_aux[3 * kTile + kTJ + tid];
    }
}

// Gate of every token from the key pass's partial sums, summed in column-tile order (so the
// result does not depend on scheduling); keep = false zeroes the gate.
__global__ __launch_bounds__(kThreads) void gate_alpha_kernel(const GateArgs a) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (n >= a.n) return;
    float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
#pragma unroll 8
    for (int t = 0; t < a.n_jt; ++t) {
        const float *p = a.partials + (static_cast<int64_t>(t) * a.n + n) * 3;
        sk2 += p[0];
        sck += p[1];
        sx2 += p[2];
    }
    float alpha = gate_alpha(sx2, sk2, sck, a);
    if (a.alpha_out != nullptr) a.alpha_out[n] = alpha;
    if (a.row_stats_out != nullptr) {
        float *st = a.row_stats_out + n * 4;
        st[0] = sx2;
        st[1] = sk2;
        st[2] = sck;
        st[3] = alpha;
    }
    if (a.keep != nullptr && a.keep[n] == 0) alpha = 0.f;
    a.alpha_eff[n] = alpha;
}

// Backward, per token, between its value side and its key side (module.py:240-251 under
// autograd). With r_h = rsqrt(mean x^2 + eps), r_k = rsqrt(mean K^2 + eps), s0 = r_h r_k sck /
// sqrt(d) (sck = sum x qs ks K) and alpha = sigmoid(s):
//   d alpha = keep * sum_j g_j V_j;  ds = d alpha * alpha (1 - alpha)
//   scalar_sqrt: s = sign(s0) sqrt(max(|s0|, 1e-6)) -> ds0 = ds / (2 sqrt|s0|) where |s0| >= 1e-6
//   (clamp_min passes the gradient at and above the bound), else 0; scalar gate: ds0 = ds
// and the rms-norm backward of h = x r_h qs and k = K r_k ks reduces to three coefficients
//   a = ds0 r_h r_k / sqrt(d), c2 = a r_h^2 sck / d, c3 = a r_k^2 sck / d
// with dx_j = a qs_j ks_j K_j - c2 x_j and dK_j = a qs_j ks_j x_j - c3 K_j (the sums the rms
// norm's backward needs, sum du u and sum dv v, are both r_h r_k ds0 sck / sqrt(d)).
__global__ __launch_bounds__(kThreads) void gate_grad_token_kernel(const GateArgs a) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (n >= a.n) return;
    constexpr float kEps = 1.1920928955078125e-07f;
    const float *st = a.row_stats + n * 4;
    const float sx2 = st[0], sk2 = st[1], sck = st[2], alpha = st[3];
    float dalpha = 0.f;
#pragma unroll 8
    for (int t = 0; t < a.n_jt; ++t) dalpha += a.grad_partials[static_cast<int64_t>(t) * a.n + n];
    if (a.keep != nullptr && a.keep[n] == 0) dalpha = 0.f;
    const float ds = dalpha * alpha * (1.f - alpha);
    const float rh = 1.0f / sqrtf(sx2 * a.inv_d + kEps);
    const float rk = 1.0f / sqrtf(sk2 * a.inv_d + kEps);
    const float s0 = rh * rk * sck * a.inv_sqrt_d;
    float ds0 = ds;
    if (a.sqrt_mode) ds0 = fabsf(s0) >= 1e-6f ? ds / (2.f * sqrtf(fabsf(s0))) : 0.f;
    const float ca = ds0 * rh * rk * a.inv_sqrt_d;
    float *cf = a.tok_coef + n * 3;
    cf[0] = ca;
    cf[1] = ca * rh * rh * sck * a.inv_d;
    cf[2] = ca * rk * rk * sck * a.inv_d;
}

// Backward of the scale deltas: P_j = sum over tokens of a x_j K_j (per token tile, then here),
// d q_scale_j = k_scale_j P_j and d k_scale_j = q_scale_j P_j (scale = 1 + delta).
__global__ __launch_bounds__(kThreads) void gate_grad_scale_kernel(const GateArgs a, float *grad_q,
                                                                   float *grad_k) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= a.d) return;
    float pj = 0.f;
    for (int t = 0; t < a.n_nt; ++t) pj += a.col_partials[static_cast<int64_t>(t) * a.d + j];
    float q, k;
    if (a.scale_bf16) {
        q = bf16_bits_to_float(static_cast<const uint16_t *>(a.q_delta)[j]);
        k = bf16_bits_to_float(static_cast<const uint16_t *>(a.k_delta)[j]);
    } else {
        q = static_cast<const float *>(a.q_delta)[j];
        k = static_cast<const float *>(a.k_delta)[j];
    }
    grad_q[j] = (1.f + k) * pj;
    grad_k[j] = (1.f + q) * pj;
}

// [n_jt][n][3] partial sums for the narrower (224-column) tiles, which also hold the 256-column
// tiles' ([ceil(d / 224) >= ceil(d / 256)]), then [n] gates
size_t workspace_bytes(int64_t n, int64_t d) {
    return (static_cast<size_t>(ceil_div(d, kTJ)) * 3 + 1) * static_cast<size_t>(n) * sizeof(float);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Backward workspace: [n_jt][n] value-side partials, [n][3] token coefficients, [n_nt][d]
// column partials (floats, each region 256-byte aligned).
struct GradLayout {
    size_t partials, coef, cols, total;
};

GradLayout grad_layout(int64_t n, int64_t d) {
    auto up = [](size_t x) { return (x + 255) & ~size_t{255}; };
    GradLayout l{};
    size_t off = 0;
    l.partials = off;  // per column tile: 224-column tiles make the most of them
    off += up(static_cast<size_t>(ceil_div(d, kTJ)) * static_cast<size_t>(n) * 4);
    l.coef = off;
    off += up(static_cast<size_t>(n) * 3 * 4);
    l.cols = off;
    off += up(static_cast<size_t>(ceil_div(n, kTile)) * static_cast<size_t>(d) * 4);
    l.total = off;
    return l;
}

// Shape, dtype and alignment checks shared by the forward and the backward; fills the
// arguments common to both.
int gate_common(GateArgs &a, const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                const void *mem, int64_t mem_dim, const void *w_key, const void *w_value, int dtype,
                const void *q_scale_delta, const void *k_scale_delta, int scale_dtype, int gate_mode,
                const uint8_t *keep) {
    ME_CHECK_ARG(hidden_dtype == ME_BF16 || hidden_dtype == ME_F32, "hidden dtype must be bf16/fp32");
    ME_CHECK_ARG(dtype == ME_BF16 || dtype == ME_F32, "engram dtype must be bf16/fp32");
    ME_CHECK_ARG(gate_mode == ME_GATE_SCALAR || gate_mode == ME_GATE_SCALAR_SQRT,
                 "gate_mode must be ME_GATE_SCALAR or ME_GATE_SCALAR_SQRT");
    ME_CHECK_ARG(n >= 0 && model_dim >= 1 && mem_dim >= 1, "bad shape");
    ME_CHECK_ARG(n < (int64_t{1} << 31) && model_dim < (int64_t{1} << 24) && mem_dim < (int64_t{1} << 24),
                 "shape too large");
    ME_CHECK_ARG(hidden && mem && w_key && w_value, "null tensor pointer");
    const size_t esz = dtype_size(dtype);
    ME_CHECK_ARG((mem_dim * esz) % 16 == 0, "mem_dim * element size must be a multiple of 16 bytes");
    ME_CHECK_ARG(model_dim % 8 == 0, "model_dim must be a multiple of 8");
    ME_CHECK_ARG(n * mem_dim * static_cast<int64_t>(esz) < (int64_t{1} << 31) &&
                     model_dim * mem_dim * static_cast<int64_t>(esz) < (int64_t{1} << 31),
                 "mem and the projection weights must each be under 2 GiB");
    ME_CHECK_ARG(aligned16(hidden) && aligned16(mem) && aligned16(w_key) && aligned16(w_value),
                 "tensors must be 16-byte aligned");
    if (gate_mode == ME_GATE_SCALAR_SQRT) {
        ME_CHECK_ARG(q_scale_delta && k_scale_delta, "scalar_sqrt needs q/k scale deltas");
        ME_CHECK_ARG(scale_dtype == ME_BF16 || scale_dtype == ME_F32, "scale dtype must be bf16/fp32");
        ME_CHECK_ARG(aligned16(q_scale_delta) && aligned16(k_scale_delta),
                     "scale tensors must be 16-byte aligned");
    }
    a.hidden = static_cast<const uint8_t *>(hidden);
    a.mem = static_cast<const uint8_t *>(mem);
    a.q_delta = gate_mode == ME_GATE_SCALAR_SQRT ? q_scale_delta : nullptr;
    a.k_delta = gate_mode == ME_GATE_SCALAR_SQRT ? k_scale_delta : nullptr;
    a.scale_bf16 = scale_dtype == ME_BF16;
    a.sqrt_mode = gate_mode == ME_GATE_SCALAR_SQRT;
    a.keep = keep;
    a.n = n;
    a.d = model_dim;
    a.m = mem_dim;
    a.mem_bytes = static_cast<uint32_t>(n * mem_dim * esz);
    a.w_bytes = static_cast<uint32_t>(model_dim * mem_dim * esz);
    a.scale_bytes = gate_mode == ME_GATE_SCALAR_SQRT
                        ? static_cast<uint32_t>(model_dim * (scale_dtype == ME_BF16 ? 2 : 4))
                        : 0u;
    a.n_jt = static_cast<int>(ceil_div(model_dim, kTile));
    a.n_nt = static_cast<int>(ceil_div(n, kTile));
    a.total_tiles = a.n_jt * a.n_nt;
    a.per_xcd = static_cast<int>(ceil_div(a.total_tiles, kXcds));
    a.inv_d = 1.0f / static_cast<float>(model_dim);
    a.inv_sqrt_d = static_cast<float>(1.0 / std::sqrt(static_cast<double>(model_dim)));
    return ME_OK;
}

}  // namespace
}  // namespace me

using namespace me;

extern "C" int me_gate_workspace_size(int64_t n, int64_t model_dim, size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    ME_CHECK_ARG(n >= 0 && model_dim >= 1, "bad shape n=%lld d=%lld", (long long)n,
                 (long long)model_dim);
    *bytes = workspace_bytes(n, model_dim);
    return ME_OK;
}

extern "C" int me_gate_residual(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                                const void *mem, int64_t mem_dim, const void *w_key,
                                const void *w_value, int dtype, const void *q_scale_delta,
                                const void *k_scale_delta, int scale_dtype, int gate_mode,
                                const uint8_t *keep, void *out, float *alpha_out,
                                float *row_stats, void *workspace, size_t workspace_size,
                                void *stream) {
    GateArgs a{};
    if (n == 0) return ME_OK;
    const int st = gate_common(a, hidden, hidden_dtype, n, model_dim, mem, mem_dim, w_key, w_value,
                               dtype, q_scale_delta, k_scale_delta, scale_dtype, gate_mode, keep);
    if (st != ME_OK) return st;
    ME_CHECK_ARG(out != nullptr && aligned16(out), "out must be a 16-byte aligned tensor");
    const size_t need = workspace_bytes(n, model_dim);
    if (workspace == nullptr || workspace_size < need) {
        set_error("me_gate_residual: workspace of %zu bytes needed, got %zu", need, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    a.out = static_cast<uint8_t *>(out);
    a.alpha_out = alpha_out;
    a.row_stats_out = row_stats;
    a.partials = static_cast<float *>(workspace);
    a.alpha_eff = a.partials + ceil_div(model_dim, kTJ) * 3 * n;
    const int64_t hidden_bytes = n * model_dim * static_cast<int64_t>(dtype_size(hidden_dtype));
    // the prefetching kernels address hidden with 32-bit buffer offsets
    const bool prefetch = dtype == ME_BF16 && hidden_dtype == ME_BF16 &&
                          hidden_bytes < (int64_t{1} << 31);
    a.hidden_bytes = prefetch ? static_cast<uint32_t>(hidden_bytes) : 0u;

    hipStream_t s = as_stream(stream);
    // the key pass reads W_K, the value pass W_V; both launches share the args
    GateArgs ak = a, av = a;
    ak.w = static_cast<const uint8_t *>(w_key);
    av.w = static_cast<const uint8_t *>(w_value);
    const dim3 grid(static_cast<unsigned>(a.per_xcd * kXcds));
#define ME_GATE_LAUNCH(T, H)                                                                     \
    do {                                                                                         \
        hipLaunchKernelGGL((gate_kernel<T, H, kKey>), grid, dim3(kThreads), 0, s, ak);          \
        int st_ = check_launch("me_gate_residual (key pass)");                                  \
        if (st_ != ME_OK) return st_;                                                            \
        hipLaunchKernelGGL(gate_alpha_kernel, dim3(static_cast<unsigned>(ceil_div(n, kThreads))), \
                           dim3(kThreads), 0, s, ak);                                            \
        st_ = check_launch("me_gate_residual (gate)");                                           \
        if (st_ != ME_OK) return st_;                                                            \
        hipLaunchKernelGGL((gate_kernel<T, H, kValue>), grid, dim3(kThreads), 0, s, av);        \
        return check_launch("me_gate_residual (value pass)");                                   \
    } while (0)
    if (dtype == ME_BF16) {
        if (hidden_dtype == ME_BF16 && prefetch && (mem_dim * 2) % kSlab == 0 && mem_dim * 2 >= 3 * kSlab) {
            // 256 x 224 tiles (16x16x32 MFMAs): whole slabs, at least three
            ak.n_jt = av.n_jt = static_cast<int>(ceil_div(model_dim, kTJ));
            ak.total_tiles = av.total_tiles = ak.n_jt * ak.n_nt;
            ak.per_xcd = av.per_xcd = static_cast<int>(ceil_div(ak.total_tiles, kXcds));
            const dim3 grid16(static_cast<unsigned>(ak.per_xcd * kXcds));
            hipLaunchKernelGGL(gate224_kernel<kKey>, grid16, dim3(kThreads), 0, s, ak);
            const int st_ = check_launch("me_gate_residual (key pass)");
            if (st_ != ME_OK) return st_;
            // the value pass computes each token's gate itself (no gate_alpha_kernel launch)
            hipLaunchKernelGGL(gate224_kernel<kValue>, grid16, dim3(kThreads), 0, s, av);
            return check_launch("me_gate_residual (value pass)");
        }
        if (hidden_dtype == ME_BF16) {
            ME_GATE_LAUNCH(uint16_t, uint16_t);
        }
        ME_GATE_LAUNCH(uint16_t, float);
    }
    if (hidden_dtype == ME_BF16) ME_GATE_LAUNCH(float, uint16_t);
    ME_GATE_LAUNCH(float, float);
#undef ME_GATE_LAUNCH
}

// ---- the allocation-free gate -----------------------------------------------------------------
// me_gate_residual_noalloc runs me_gate_residual with its workspace (the per-(column tile, token)
// partial sums and the per-token gates, fully written before they are read, so nothing needs
// clearing) in this file-scope device array instead of caller memory. Every GPU the library
// runs on holds its own copy until the process ends; its address on a device comes from
// hipGetSymbolAddress, asked once per device with that device current. Calls that overlap on
// one GPU share the array and race.
constexpr size_t kScratchBytes = size_t{4} << 20;  // 4 MiB: 14,364 tokens at model dim 5376
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace me {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_on[kMaxDevices] = {};

// The device address of `scratch` on the current device.
int scratch_on_current_device(void **ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("me_gate_residual_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
        return ME_ERR_HIP;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("me_gate_residual_noalloc: device %d beyond the %d this library tracks", dev, kMaxDevices);
        return ME_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_on[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("me_gate_residual_noalloc: no address for the scratch array on device %d: %s", dev,
                      hipGetErrorString(e));
            return ME_ERR_HIP;
        }
        g_scratch_on[dev] = p;
    }
    *ptr = g_scratch_on[dev];
    return ME_OK;
}
}  // namespace
}  // namespace me

extern "C" int me_gate_residual_noalloc(const void *hidden, int hidden_dtype, int64_t n,
                                        int64_t model_dim, const void *mem, int64_t mem_dim,
                                        const void *w_key, const void *w_value, int dtype,
                                        const void *q_scale_delta, const void *k_scale_delta,
                                        int scale_dtype, int gate_mode, const uint8_t *keep,
                                        void *out, float *alpha_out, float *row_stats,
                                        void *stream) {
    ME_CHECK_ARG(n >= 0 && model_dim >= 1, "bad shape n=%lld d=%lld", (long long)n, (long long)model_dim);
    if (n == 0) return ME_OK;
    const size_t need = workspace_bytes(n, model_dim);
    if (need > kScratchBytes) {
        set_error("me_gate_residual_noalloc: %lld tokens of model dim %lld need %zu bytes of scratch; the "
                  "static scratch holds %zu (at most %lld tokens at this model dim): use me_gate_residual "
                  "with a workspace",
                  (long long)n, (long long)model_dim, need, kScratchBytes,
                  (long long)(kScratchBytes / workspace_bytes(1, model_dim)));
        return ME_ERR_INVALID;
    }
    void *ws = nullptr;
    const int st = scratch_on_current_device(&ws);
    if (st != ME_OK) return st;
    return me_gate_residual(hidden, hidden_dtype, n, model_dim, mem, mem_dim, w_key, w_value, dtype,
                            q_scale_delta, k_scale_delta, scale_dtype, gate_mode, keep, out, alpha_out,
                            row_stats, ws, kScratchBytes, stream);
}

extern "C" int me_gate_backward_workspace_size(int64_t n, int64_t model_dim, size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    ME_CHECK_ARG(n >= 0 && model_dim >= 1, "bad shape n=%lld d=%lld", (long long)n,
                 (long long)model_dim);
    *bytes = grad_layout(n, model_dim).total;
    return ME_OK;
}

// Zeroes two fp32 vectors of n values (the scale gradients of an empty batch).
__global__ __launch_bounds__(256) void zero_two_f32_kernel(float *a, float *b, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        a[i] = 0.0f;
        b[i] = 0.0f;
    }
}

extern "C" int me_gate_backward(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                                const void *mem, int64_t mem_dim, const void *w_key,
                                const void *w_value, int dtype, const void *q_scale_delta,
                                const void *k_scale_delta, int scale_dtype, int gate_mode,
                                const uint8_t *keep, const void *grad_out, const float *row_stats,
                                void *grad_hidden, void *grad_key, void *grad_value,
                                float *grad_q_scale, float *grad_k_scale, void *workspace,
                                size_t workspace_size, void *stream) {
    GateArgs a{};
    if (n == 0) {
        // no tokens: the scale gradients are zero
        if (gate_mode == ME_GATE_SCALAR_SQRT && grad_q_scale != nullptr && grad_k_scale != nullptr) {
            // a fill kernel, not hipMemsetAsync: a captured backward then records no memset node
            ME_CHECK_ARG(model_dim >= 1 && model_dim < (int64_t{1} << 30), "bad model_dim");
            const unsigned blocks = static_cast<unsigned>(ceil_div(model_dim, 256));
            hipLaunchKernelGGL(zero_two_f32_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                               grad_q_scale, grad_k_scale, model_dim);
            return check_launch("me_gate_backward (zero scale gradients)");
        }
        return ME_OK;
    }
    const int st = gate_common(a, hidden, hidden_dtype, n, model_dim, mem, mem_dim, w_key, w_value,
                               dtype, q_scale_delta, k_scale_delta, scale_dtype, gate_mode, keep);
    if (st != ME_OK) return st;
    ME_CHECK_ARG(grad_out && row_stats && grad_hidden && grad_key && grad_value,
                 "null gradient pointer");
    ME_CHECK_ARG(aligned16(grad_out) && aligned16(grad_hidden) && aligned16(grad_key) &&
                     aligned16(grad_value),
                 "gradient tensors must be 16-byte aligned");
    if (gate_mode == ME_GATE_SCALAR_SQRT)
        ME_CHECK_ARG(grad_q_scale && grad_k_scale, "scalar_sqrt needs the scale gradient outputs");
    const GradLayout l = grad_layout(n, model_dim);
    if (workspace == nullptr || workspace_size < l.total) {
        set_error("me_gate_backward: workspace of %zu bytes needed, got %zu", l.total, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    a.grad_out = static_cast<const uint8_t *>(grad_out);
    a.row_stats = row_stats;
    a.grad_hidden = static_cast<uint8_t *>(grad_hidden);
    a.grad_partials = reinterpret_cast<float *>(ws + l.partials);
    a.tok_coef = reinterpret_cast<float *>(ws + l.coef);
    a.col_partials = reinterpret_cast<float *>(ws + l.cols);

    hipStream_t s = as_stream(stream);
    // value side (W_V, writes dV and the per-token sums of g . V), the per-token coefficients,
    // key side (W_K, writes d hidden and dK), then the scale gradients
    const int64_t hidden_bytes = n * model_dim * static_cast<int64_t>(dtype_size(hidden_dtype));
    if (dtype == ME_BF16 && hidden_dtype == ME_BF16 && hidden_bytes < (int64_t{1} << 31) &&
        (mem_dim * 2) % kSlab == 0 && mem_dim * 2 >= 3 * kSlab) {
        // bf16: the forward's 256 x 224 tiles (16x16x32 MFMAs, whole slabs, at least three)
        a.hidden_bytes = static_cast<uint32_t>(hidden_bytes);
        a.n_jt = static_cast<int>(ceil_div(model_dim, kTJ));
        a.total_tiles = a.n_jt * a.n_nt;
        a.per_xcd = static_cast<int>(ceil_div(a.total_tiles, kXcds));
        GateArgs av = a, ak = a;
        av.w = static_cast<const uint8_t *>(w_value);
        av.grad_proj = static_cast<uint8_t *>(grad_value);
        ak.w = static_cast<const uint8_t *>(w_key);
        ak.grad_proj = static_cast<uint8_t *>(grad_key);
        const dim3 grid16(static_cast<unsigned>(a.per_xcd * kXcds));
        hipLaunchKernelGGL(gate224_kernel<kGradValue>, grid16, dim3(kThreads), 0, s, av);
        int st_ = check_launch("me_gate_backward (value side)");
        if (st_ != ME_OK) return st_;
        hipLaunchKernelGGL(gate_grad_token_kernel, dim3(static_cast<unsigned>(ceil_div(n, kThreads))),
                           dim3(kThreads), 0, s, a);
        st_ = check_launch("me_gate_backward (token coefficients)");
        if (st_ != ME_OK) return st_;
        hipLaunchKernelGGL(gate224_kernel<kGradKey>, grid16, dim3(kThreads), 0, s, ak);
        st_ = check_launch("me_gate_backward (key side)");
        if (st_ != ME_OK) return st_;
        if (gate_mode != ME_GATE_SCALAR_SQRT) return ME_OK;
        hipLaunchKernelGGL(gate_grad_scale_kernel,
                           dim3(static_cast<unsigned>(ceil_div(model_dim, kThreads))), dim3(kThreads), 0, s,
                           a, grad_q_scale, grad_k_scale);
        return check_launch("me_gate_backward (scale gradients)");
    }
    GateArgs av = a, ak = a;
    av.w = static_cast<const uint8_t *>(w_value);
    av.grad_proj = static_cast<uint8_t *>(grad_value);
    ak.w = static_cast<const uint8_t *>(w_key);
    ak.grad_proj = static_cast<uint8_t *>(grad_key);
    const dim3 grid(static_cast<unsigned>(a.per_xcd * kXcds));
    const dim3 tok_grid(static_cast<unsigned>(ceil_div(n, kThreads)));
#define ME_GATE_GRAD_LAUNCH(T, H)                                                                \
    do {                                                                                         \
        hipLaunchKernelGGL((gate_kernel<T, H, kGradValue>), grid, dim3(kThreads), 0, s, av);    \
        int st_ = check_launch("me_gate_backward (value side)");                                \
        if (st_ != ME_OK) return st_;                                                            \
        hipLaunchKernelGGL(gate_grad_token_kernel, tok_grid, dim3(kThreads), 0, s, a);           \
        st_ = check_launch("me_gate_backward (token coefficients)");                             \
        if (st_ != ME_OK) return st_;                                                            \
        hipLaunchKernelGGL((gate_kernel<T, H, kGradKey>), grid, dim3(kThreads), 0, s, ak);      \
        st_ = check_launch("me_gate_backward (key side)");                                       \
        if (st_ != ME_OK) return st_;                                                            \
    } while (0)
    if (dtype == ME_BF16) {
        if (hidden_dtype == ME_BF16)
            ME_GATE_GRAD_LAUNCH(uint16_t, uint16_t);
        else
            ME_GATE_GRAD_LAUNCH(uint16_t, float);
    } else {
        if (hidden_dtype == ME_BF16)
            ME_GATE_GRAD_LAUNCH(float, uint16_t);
        else
            ME_GATE_GRAD_LAUNCH(float, float);
    }
#undef ME_GATE_GRAD_LAUNCH
    if (gate_mode != ME_GATE_SCALAR_SQRT) return ME_OK;
    hipLaunchKernelGGL(gate_grad_scale_kernel,
                       dim3(static_cast<unsigned>(ceil_div(model_dim, kThreads))), dim3(kThreads), 0, s,
                       a, grad_q_scale, grad_k_scale);
    return check_launch("me_gate_backward (scale gradients)");
}
