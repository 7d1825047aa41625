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
// v_mfma_f32_32x32x2f32). Both operands are K-contiguous in HBM (W is [d, M], mem is [N, M]),
// so each k-step is one 16-byte load per lane for A and for B. The K loop moves 128 bytes of K
// per row per step through a double-buffered LDS tile (2 x 64 KiB) whose 16-byte chunks are
// XOR-swizzled by (row & 7): a wave's ds_read_b128 of 32 rows at one k then hits distinct
// banks in every 8-lane group. Workgroup ids are remapped so the 32 CUs of one XCD work on a
// compact group of tiles (8 token tiles x 4 column tiles) and share their operands in that
// XCD's L2.
#include "me_common.h"

namespace me {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kTile = 256;         // output tile edge (j and n)
constexpr int kRowBytes = 128;     // bytes of K per row per k-step
constexpr int kOperandBytes = kTile * kRowBytes;            // 32 KiB
constexpr int kStagePitch = 512 + 16;                       // epilogue row: 512 B + pad
constexpr int kStageBytes = kTile * kStagePitch;            // 132 KiB
constexpr int kLoopBytes = 4 * kOperandBytes;               // 2 buffers x (A + B) = 128 KiB
constexpr int kSmemBytes = kStageBytes > kLoopBytes ? kStageBytes : kLoopBytes;
constexpr int kGroupTiles = 8;     // token tiles per XCD group
constexpr int kXcds = 8;

enum Phase : int { kKey = 0, kValue = 1 };

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

__device__ __forceinline__ float load_scale(const void *p, int is_bf16, int64_t j) {
    return is_bf16 ? bf16_bits_to_float(static_cast<const uint16_t *>(p)[j])
                   : static_cast<const float *>(p)[j];
}

// Loads/stores E consecutive elements of type X as floats (E * sizeof(X) is 8, 16 or 32 bytes).
template <typename X, int E>
__device__ __forceinline__ void load_row(const uint8_t *p, float (&v)[E]) {
    constexpr int kBytes = E * sizeof(X);
    static_assert(kBytes % 8 == 0, "row chunk must be a multiple of 8 bytes");
    uint32_t w[kBytes / 4];
#pragma unroll
    for (int q = 0; q < kBytes / 16; ++q) {
        const uint4 u = reinterpret_cast<const uint4 *>(p)[q];
        w[4 * q] = u.x; w[4 * q + 1] = u.y; w[4 * q + 2] = u.z; w[4 * q + 3] = u.w;
    }
    if (kBytes % 16 == 8) {
        const uint2 u = reinterpret_cast<const uint2 *>(p)[kBytes / 8 - 1];
        w[kBytes / 4 - 2] = u.x; w[kBytes / 4 - 1] = u.y;
    }
    const X *x = reinterpret_cast<const X *>(w);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = to_f<X>(x[e]);
}

template <typename X, int E>
__device__ __forceinline__ void store_row(uint8_t *p, const float (&v)[E]) {
    constexpr int kBytes = E * sizeof(X);
    uint32_t w[kBytes / 4];
    X *x = reinterpret_cast<X *>(w);
#pragma unroll
    for (int e = 0; e < E; ++e) x[e] = from_f<X>(v[e]);
#pragma unroll
    for (int q = 0; q < kBytes / 16; ++q)
        reinterpret_cast<uint4 *>(p)[q] = make_uint4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    if (kBytes % 16 == 8)
        reinterpret_cast<uint2 *>(p)[kBytes / 8 - 1] = make_uint2(w[kBytes / 4 - 2], w[kBytes / 4 - 1]);
}

// Raw bytes of E elements of X, loaded now and unpacked later (keeps a batch of global loads
// in flight without converting them to floats first).
template <typename X, int E>
struct RawRow {
    static constexpr int kWords = E * sizeof(X) / 4;
    uint32_t w[kWords];
};

template <typename X, int E>
__device__ __forceinline__ void load_raw(const uint8_t *p, RawRow<X, E> &r) {
    constexpr int kBytes = E * sizeof(X);
#pragma unroll
    for (int q = 0; q < kBytes / 16; ++q) {
        const uint4 u = reinterpret_cast<const uint4 *>(p)[q];
        r.w[4 * q] = u.x; r.w[4 * q + 1] = u.y; r.w[4 * q + 2] = u.z; r.w[4 * q + 3] = u.w;
    }
    if (kBytes % 16 == 8) {
        const uint2 u = reinterpret_cast<const uint2 *>(p)[kBytes / 8 - 1];
        r.w[kBytes / 4 - 2] = u.x; r.w[kBytes / 4 - 1] = u.y;
    }
}

template <typename X, int E>
__device__ __forceinline__ void unpack(const RawRow<X, E> &r, float (&v)[E]) {
    const X *x = reinterpret_cast<const X *>(r.w);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = to_f<X>(x[e]);
}

// ---- MFMA step over one 128-byte k-slab ---------------------------------------------------
// As/Bs: swizzled [256 rows][128 B] tiles. The wave's A rows are wj*128 + [0,128), its B rows
// wn*128 + [0,128). Lane l reads row (l & 31) of each 32-row subtile at 16-byte chunk
// c = 2*ks + (l >> 5), so lanes 0-31 carry one half of the step's k values and lanes 32-63 the
// other; A and B use the same assignment, which is all the dot product needs.
template <typename T>
__device__ __forceinline__ void mfma_slab(const uint8_t *As, const uint8_t *Bs, int wj, int wn,
                                          int lane, floatx16 (&acc)[4][4]);

template <>
__device__ __forceinline__ void mfma_slab<uint16_t>(const uint8_t *As, const uint8_t *Bs, int wj,
                                                    int wn, int lane, floatx16 (&acc)[4][4]) {
    const int r = lane & 31, swz = lane & 7;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int c = ((2 * ks + (lane >> 5)) ^ swz) << 4;
        bf16x8 af[4], bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            af[s] = *reinterpret_cast<const bf16x8 *>(As + (wj * 128 + s * 32 + r) * kRowBytes + c);
            bf[s] = *reinterpret_cast<const bf16x8 *>(Bs + (wn * 128 + s * 32 + r) * kRowBytes + c);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
}

template <>
__device__ __forceinline__ void mfma_slab<float>(const uint8_t *As, const uint8_t *Bs, int wj,
                                                 int wn, int lane, floatx16 (&acc)[4][4]) {
    const int r = lane & 31, swz = lane & 7;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int c = ((2 * ks + (lane >> 5)) ^ swz) << 4;
        float4 af[4], bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            af[s] = *reinterpret_cast<const float4 *>(As + (wj * 128 + s * 32 + r) * kRowBytes + c);
            bf[s] = *reinterpret_cast<const float4 *>(Bs + (wn * 128 + s * 32 + r) * kRowBytes + c);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].x, bf[b].x, acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].y, bf[b].y, acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].z, bf[b].z, acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a].w, bf[b].w, acc[a][b], 0, 0, 0);
            }
    }
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
    __shared__ __attribute__((aligned(16))) uint8_t smem[kSmemBytes];
    __shared__ float s_alpha[kTile];
    __shared__ float s_part[kTile][3];

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

    // the value pass reads the tile's gates now and parks them in LDS after the K loop
    float alpha_reg = 0.f;
    if (PHASE == kValue) {
        if (n0 + tid < a.n) alpha_reg = a.alpha_eff[n0 + tid];
    } else {
        s_part[tid][0] = 0.f;
        s_part[tid][1] = 0.f;
        s_part[tid][2] = 0.f;
    }

    // ---- GEMM: acc[a][b] = W[j-subtile a] x mem[n-subtile b]^T over the full K
    floatx16 acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[x][y][e] = 0.f;

    constexpr int kElems = kRowBytes / sizeof(T);  // k values per row per step
    const int64_t row_bytes = a.m * static_cast<int64_t>(sizeof(T));
    const int ksteps = static_cast<int>(ceil_div(a.m, kElems));
    uint4 ra[8], rb[8];

    auto gload = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = tid + kThreads * i;
            const int row = q >> 3, c = q & 7;
            const int64_t kb = static_cast<int64_t>(kt) * kRowBytes + c * 16;  // byte offset in K
            const bool kin = kb < row_bytes;
            ra[i] = (kin && j0 + row < a.d)
                        ? *reinterpret_cast<const uint4 *>(a.w + (j0 + row) * row_bytes + kb)
                        : make_uint4(0, 0, 0, 0);
            rb[i] = (kin && n0 + row < a.n)
                        ? *reinterpret_cast<const uint4 *>(a.mem + (n0 + row) * row_bytes + kb)
                        : make_uint4(0, 0, 0, 0);
        }
    };
    auto sstore = [&](int buf) {
        uint8_t *As = smem + buf * 2 * kOperandBytes;
        uint8_t *Bs = As + kOperandBytes;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = tid + kThreads * i;
            const int row = q >> 3, c = q & 7;
            const int off = row * kRowBytes + ((c ^ (row & 7)) << 4);
            *reinterpret_cast<uint4 *>(As + off) = ra[i];
            *reinterpret_cast<uint4 *>(Bs + off) = rb[i];
        }
    };

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < ksteps; ++kt) {
        if (kt + 1 < ksteps) gload(kt + 1);
        const uint8_t *As = smem + (kt & 1) * 2 * kOperandBytes;
        mfma_slab<T>(As, As + kOperandBytes, wj, wn, lane, acc);
        if (kt + 1 < ksteps) sstore((kt + 1) & 1);
        __syncthreads();
    }

    if (PHASE == kValue) s_alpha[tid] = alpha_reg;  // read after the staging barrier

    // ---- epilogue: stage round_T(C) as [token][column] rows in LDS, then walk token rows
    constexpr int kPasses = sizeof(T) == 2 ? 1 : 2;     // fp32 tiles are staged in two halves
    constexpr int kPassCols = kTile / kPasses;          // columns per pass
    constexpr int kLaneCols = kPassCols / 32;           // columns per lane (8 bf16 / 4 fp32)
    const int half = lane >> 5, sub = lane & 31;

    for (int pass = 0; pass < kPasses; ++pass) {
        if (kPasses == 1 || wj == pass) {
#pragma unroll
            for (int x = 0; x < 4; ++x)
#pragma unroll
                for (int y = 0; y < 4; ++y) {
                    const int nl = wn * 128 + y * 32 + sub;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        // rows 8g + 4*half + [0,4) of the 32x32 MFMA output are 4 consecutive j
                        const int jl = (kPasses == 1 ? wj * 128 : 0) + x * 32 + 8 * g + 4 * half;
                        float v[4] = {acc[x][y][4 * g], acc[x][y][4 * g + 1], acc[x][y][4 * g + 2],
                                      acc[x][y][4 * g + 3]};
                        store_row<T, 4>(smem + nl * kStagePitch + jl * sizeof(T), v);
                    }
                }
        }
        __syncthreads();

        // walk token rows: a half-wave (32 lanes x kLaneCols columns) per row, 8 rows per
        // step across the workgroup; the hidden loads of a whole batch of rows are issued
        // before any of them is used
        constexpr int kIters = kTile / 8;
        constexpr int kHBytes = kLaneCols * sizeof(H);
        constexpr int kBatch = kHBytes <= 16 ? kIters : kIters / 2;
        const int jl = sub * kLaneCols;
        const int64_t j = j0 + pass * kPassCols + jl;
        const bool jlive = j < a.d;
        float w[kLaneCols];  // q_scale * k_scale of the lane's columns (key pass)
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) {
            w[e] = 1.f;
            if (PHASE == kKey && jlive && a.q_delta != nullptr)
                w[e] = (1.f + load_scale(a.q_delta, a.scale_bf16, j + e)) *
                       (1.f + load_scale(a.k_delta, a.scale_bf16, j + e));
        }
        for (int b0 = 0; b0 < kIters; b0 += kBatch) {
            RawRow<H, kLaneCols> raw[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int64_t n = n0 + (b0 + u) * 8 + wave * 2 + half;
                if (jlive && n < a.n) {
                    load_raw<H, kLaneCols>(a.hidden + (n * a.d + j) * sizeof(H), raw[u]);
                } else {
#pragma unroll
                    for (int q = 0; q < RawRow<H, kLaneCols>::kWords; ++q) raw[u].w[q] = 0u;
                }
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int nl = (b0 + u) * 8 + wave * 2 + half;
                const int64_t n = n0 + nl;
                const bool live = jlive && n < a.n;
                float c[kLaneCols], x[kLaneCols];
                load_row<T, kLaneCols>(smem + nl * kStagePitch + jl * sizeof(T), c);
                unpack<H, kLaneCols>(raw[u], x);
                if (PHASE == kKey) {
                    float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
#pragma unroll
                    for (int e = 0; e < kLaneCols; ++e) {
                        sk2 += c[e] * c[e];
                        sck += x[e] * w[e] * c[e];
                        sx2 += x[e] * x[e];
                    }
#pragma unroll
                    for (int off = 16; off >= 1; off >>= 1) {
                        sk2 += __shfl_xor(sk2, off, 32);
                        sck += __shfl_xor(sck, off, 32);
                        sx2 += __shfl_xor(sx2, off, 32);
                    }
                    if (sub == 0) {
                        s_part[nl][0] += sk2;
                        s_part[nl][1] += sck;
                        s_part[nl][2] += sx2;
                    }
                } else if (live) {
                    const float alpha = s_alpha[nl];
                    float o[kLaneCols];
#pragma unroll
                    for (int e = 0; e < kLaneCols; ++e) o[e] = x[e] + round_t<H>(alpha * c[e]);
                    store_row<H, kLaneCols>(a.out + (n * a.d + j) * sizeof(H), o);
                }
            }
        }
        __syncthreads();
    }

    if (PHASE == kKey) {
        const int64_t n = n0 + tid;
        if (n < a.n) {
            float *p = a.partials + (static_cast<int64_t>(jt) * a.n + n) * 3;
            p[0] = s_part[tid][0];
            p[1] = s_part[tid][1];
            p[2] = s_part[tid][2];
        }
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
    if (a.keep != nullptr && a.keep[n] == 0) alpha = 0.f;
    a.alpha_eff[n] = alpha;
}

size_t workspace_bytes(int64_t n, int64_t d) {
    return (static_cast<size_t>(ceil_div(d, kTile)) * 3 + 1) * static_cast<size_t>(n) * sizeof(float);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

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
                                const uint8_t *keep, void *out, float *alpha_out, void *workspace,
                                size_t workspace_size, void *stream) {
    ME_CHECK_ARG(hidden_dtype == ME_BF16 || hidden_dtype == ME_F32, "hidden dtype must be bf16/fp32");
    ME_CHECK_ARG(dtype == ME_BF16 || dtype == ME_F32, "engram dtype must be bf16/fp32");
    ME_CHECK_ARG(gate_mode == ME_GATE_SCALAR || gate_mode == ME_GATE_SCALAR_SQRT,
                 "gate_mode must be ME_GATE_SCALAR or ME_GATE_SCALAR_SQRT");
    ME_CHECK_ARG(n >= 0 && model_dim >= 1 && mem_dim >= 1, "bad shape");
    ME_CHECK_ARG(n < (int64_t{1} << 31) && model_dim < (int64_t{1} << 24) && mem_dim < (int64_t{1} << 24),
                 "shape too large");
    if (n == 0) return ME_OK;
    ME_CHECK_ARG(hidden && mem && w_key && w_value && out, "null tensor pointer");
    const size_t esz = dtype_size(dtype), hsz = dtype_size(hidden_dtype);
    ME_CHECK_ARG((mem_dim * esz) % 16 == 0, "mem_dim * element size must be a multiple of 16 bytes");
    ME_CHECK_ARG(model_dim % 8 == 0, "model_dim must be a multiple of 8");
    ME_CHECK_ARG(aligned16(hidden) && aligned16(mem) && aligned16(w_key) && aligned16(w_value) &&
                     aligned16(out),
                 "tensors must be 16-byte aligned");
    (void)hsz;
    if (gate_mode == ME_GATE_SCALAR_SQRT) {
        ME_CHECK_ARG(q_scale_delta && k_scale_delta, "scalar_sqrt needs q/k scale deltas");
        ME_CHECK_ARG(scale_dtype == ME_BF16 || scale_dtype == ME_F32, "scale dtype must be bf16/fp32");
    }
    const size_t need = workspace_bytes(n, model_dim);
    if (workspace == nullptr || workspace_size < need) {
        set_error("me_gate_residual: workspace of %zu bytes needed, got %zu", need, workspace_size);
        return ME_ERR_WORKSPACE;
    }

    GateArgs a{};
    a.hidden = static_cast<const uint8_t *>(hidden);
    a.mem = static_cast<const uint8_t *>(mem);
    a.q_delta = gate_mode == ME_GATE_SCALAR_SQRT ? q_scale_delta : nullptr;
    a.k_delta = gate_mode == ME_GATE_SCALAR_SQRT ? k_scale_delta : nullptr;
    a.scale_bf16 = scale_dtype == ME_BF16;
    a.sqrt_mode = gate_mode == ME_GATE_SCALAR_SQRT;
    a.keep = keep;
    a.out = static_cast<uint8_t *>(out);
    a.alpha_out = alpha_out;
    a.partials = static_cast<float *>(workspace);
    a.alpha_eff = a.partials + ceil_div(model_dim, kTile) * 3 * n;
    a.n = n;
    a.d = model_dim;
    a.m = mem_dim;
    a.n_jt = static_cast<int>(ceil_div(model_dim, kTile));
    a.n_nt = static_cast<int>(ceil_div(n, kTile));
    a.total_tiles = a.n_jt * a.n_nt;
    a.per_xcd = static_cast<int>(ceil_div(a.total_tiles, kXcds));
    a.inv_d = 1.0f / static_cast<float>(model_dim);
    a.inv_sqrt_d = static_cast<float>(1.0 / std::sqrt(static_cast<double>(model_dim)));

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
        if (hidden_dtype == ME_BF16) ME_GATE_LAUNCH(uint16_t, uint16_t);
        ME_GATE_LAUNCH(uint16_t, float);
    }
    if (hidden_dtype == ME_BF16) ME_GATE_LAUNCH(float, uint16_t);
    ME_GATE_LAUNCH(float, float);
#undef ME_GATE_LAUNCH
}
