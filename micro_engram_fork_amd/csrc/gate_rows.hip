// Stage 3 for few tokens on gfx950: the scalar / scalar_sqrt gate and the residual add from key
// and value projections that are already computed.
//
// Reference (micro_engram/module.py:239-261), per token with hidden x (d wide), K = round_T(W_K
// e) and V = round_T(W_V e):
//   h = rms_norm(x) * q_scale, k = rms_norm(K) * k_scale        (scales only for scalar_sqrt)
//   s = sum(h * k) / sqrt(d); scalar_sqrt: s = sign(s) * sqrt(max(|s|, 1e-6))
//   alpha = sigmoid(s); out = x + round_H(alpha * V * keep)
//
// The fused two-pass kernel (gate.hip) computes K and V tile by tile on 256-token MFMA tiles:
// below about a thousand tokens it has fewer tiles than the part has CUs, and one tile's K loop
// sets its time. For such batches the projections run in the few-token GEMM (me_kv_proj,
// proj.hip) and this kernel does the rest in one pass over the rows: one 256-thread workgroup
// per token (a decode batch of 256 tokens fills the part's 256 CUs), 8 columns per thread per
// step with 16-byte loads of hidden, K and V issued together (V and hidden stay in registers
// for the output, so the row's only memory round trip is before the reduction), the three sums
// sum K^2, sum x (1 + dq) (1 + dk) K and sum x^2 reduced across the workgroup, the gate, then
// x + round_H(alpha V) written with 16-byte stores.
//
// Any width: rows whose model dim, row stride or addresses do not allow 16-byte accesses take the
// same kernel with one column per lane and step (scalar loads and stores), so an engram of any
// model dim and memory width runs (its projections then come from a library GEMM, the nn.Linear
// of module.py:245, 254, since the MFMA kernels need whole 16-byte rows).
//
// The backward of this stage from the same K and V rows (the autograd of module.py:239-261, what
// me_gate_backward computes on MFMA tiles for the shapes those take): per token, from the
// forward's row statistics (sum x^2, sum K^2, sck = sum x qs ks K, alpha),
//   dV = round_T(alpha keep g);  d alpha = keep sum g V;  ds = d alpha alpha (1 - alpha)
//   ds0 = ds / (2 sqrt|s0|) where |s0| >= 1e-6, else 0 (scalar_sqrt); ds0 = ds (scalar)
//   a = ds0 r_h r_k / sqrt(d), c2 = a r_h^2 sck / d, c3 = a r_k^2 sck / d
//   d hidden = g + round_H(a w K - c2 x), dK = round_T(a w x - c3 K)   (w = qs ks)
// one workgroup per token; then d q_scale_j = ks_j P_j and d k_scale_j = qs_j P_j with
// P_j = sum over tokens of a x_j K_j, per 256-token block and then over the blocks in order.
#include "me_common.h"

#include <cmath>
#include <initializer_list>

namespace me {
namespace {

constexpr int kThreads = 256;  // one token per workgroup
constexpr int kKeep = 3;      // steps kept in registers: rows up to 3 * 256 * LC columns
constexpr int kScaleBlock = 256;  // tokens per partial of the scale gradients

struct RowArgs {
    const uint8_t *hidden;  // [n, d] of H
    const uint8_t *k;       // [n, *] of T, row stride kv_stride elements
    const uint8_t *v;       // [n, *] of T, row stride kv_stride elements
    const uint8_t *q_delta; // [d] scale - 1 (nullable: scalar gate)
    const uint8_t *k_delta;
    const uint8_t *keep;    // [n] (nullable)
    uint8_t *out;           // [n, d] of H
    float *alpha_out;       // [n] (nullable)
    float *row_stats;       // [n, 4] (nullable): sum x^2, sum K^2, sum x qs ks K, alpha
    int64_t n, d, kv_stride;
    int scale_bf16, sqrt_mode;
    float inv_d, inv_sqrt_d;
    // backward
    const uint8_t *grad_out;  // [n, d] of H
    const float *stats_in;    // [n, 4] the forward's row statistics
    uint8_t *grad_hidden;     // [n, d] of H
    uint8_t *grad_k;          // [n, d] of T
    uint8_t *grad_v;          // [n, d] of T
    float *coef;              // [n] the token's a (workspace)
    float *col_part;          // [ceil(n / kScaleBlock)][d] (workspace)
};

// LC consecutive elements of X as floats: 16-byte accesses for LC = 8, single elements for 1.
template <typename X, int LC>
__device__ __forceinline__ void loadn(const uint8_t *p, float (&v)[LC]) {
    if constexpr (LC == 1) {
        if constexpr (sizeof(X) == 2) v[0] = bf16_bits_to_float(*as_global(reinterpret_cast<const uint16_t *>(p)));
        else v[0] = *as_global(reinterpret_cast<const float *>(p));
    } else if constexpr (sizeof(X) == 2) {
        const u32x4_v w = *as_global(reinterpret_cast<const u32x4_v *>(p));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf16_bits_to_float(static_cast<uint16_t>(w[e]));
            v[2 * e + 1] = bf16_bits_to_float(static_cast<uint16_t>(w[e] >> 16));
        }
    } else {
        const f32x4_v a = *as_global(reinterpret_cast<const f32x4_v *>(p));
        const f32x4_v b = *as_global(reinterpret_cast<const f32x4_v *>(p + 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = a[e];
            v[4 + e] = b[e];
        }
    }
}

// Stores LC values rounded to X (round to nearest even for bf16).
template <typename X, int LC>
__device__ __forceinline__ void storen(uint8_t *p, const float (&v)[LC]) {
    if constexpr (LC == 1) {
        if constexpr (sizeof(X) == 2) *as_global(reinterpret_cast<uint16_t *>(p)) = float_to_bf16_bits_rne(v[0]);
        else *as_global(reinterpret_cast<float *>(p)) = v[0];
    } else if constexpr (sizeof(X) == 2) {
        u32x4_v w;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = static_cast<uint32_t>(float_to_bf16_bits_rne(v[2 * e])) |
                   (static_cast<uint32_t>(float_to_bf16_bits_rne(v[2 * e + 1])) << 16);
        *as_global(reinterpret_cast<u32x4_v *>(p)) = w;
    } else {
        *as_global(reinterpret_cast<f32x4_v *>(p)) = f32x4_v{v[0], v[1], v[2], v[3]};
        *as_global(reinterpret_cast<f32x4_v *>(p + 16)) = f32x4_v{v[4], v[5], v[6], v[7]};
    }
}

// w = (1 + q delta)(1 + k delta) of LC columns from j (1 without scales).
template <int LC>
__device__ __forceinline__ void scale_products(const RowArgs &a, int64_t j, float (&w)[LC]) {
    if (a.q_delta != nullptr) {
        float qd[LC], kd[LC];
        if (a.scale_bf16) {
            loadn<uint16_t, LC>(a.q_delta + j * 2, qd);
            loadn<uint16_t, LC>(a.k_delta + j * 2, kd);
        } else {
            loadn<float, LC>(a.q_delta + j * 4, qd);
            loadn<float, LC>(a.k_delta + j * 4, kd);
        }
#pragma unroll
        for (int e = 0; e < LC; ++e) w[e] = (1.f + qd[e]) * (1.f + kd[e]);
    } else {
#pragma unroll
        for (int e = 0; e < LC; ++e) w[e] = 1.f;
    }
}

template <typename X>
__device__ __forceinline__ float round_to(float v) {
    if constexpr (sizeof(X) == 2) return round_to_bf16(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

// Sums of a block's threads, in wave order, the same in every thread.
template <int N>
__device__ __forceinline__ void block_sums(float (&v)[N], float (*s_part)[4]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = wave_sum(v[i]);
    if (lane == 0)
#pragma unroll
        for (int i = 0; i < N; ++i) s_part[wave][i] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        v[i] = 0.f;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) v[i] += s_part[w][i];
    }
}

template <typename H, typename T, int kLaneCols>
__global__ __launch_bounds__(kThreads) void gate_rows_kernel(const RowArgs a) {
    constexpr float kEps = 1.1920928955078125e-07f;  // torch.finfo(float32).eps: rms_norm default
    __shared__ float s_part[kThreads / 64][3];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t n = blockIdx.x;
    const uint8_t *x = a.hidden + n * a.d * static_cast<int64_t>(sizeof(H));
    const uint8_t *kr = a.k + n * a.kv_stride * static_cast<int64_t>(sizeof(T));
    const uint8_t *vr = a.v + n * a.kv_stride * static_cast<int64_t>(sizeof(T));
    float sk2 = 0.f, sck = 0.f, sx2 = 0.f;
    // the row's hidden and V values of the first kKeep steps stay in registers for the output
    float xk[kKeep][kLaneCols], vk[kKeep][kLaneCols];
    int it = 0;
    for (int64_t j = static_cast<int64_t>(tid) * kLaneCols; j < a.d; j += kThreads * kLaneCols, ++it) {
        float xv[kLaneCols], kv[kLaneCols], w[kLaneCols];
        loadn<H, kLaneCols>(x + j * sizeof(H), xv);
        loadn<T, kLaneCols>(kr + j * sizeof(T), kv);
#pragma unroll
        for (int q = 0; q < kKeep; ++q)
            if (q == it) {
#pragma unroll
                for (int e = 0; e < kLaneCols; ++e) xk[q][e] = xv[e];
                loadn<T, kLaneCols>(vr + j * sizeof(T), vk[q]);
            }
        scale_products<kLaneCols>(a, j, w);
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) {
            sk2 += kv[e] * kv[e];
            sck += xv[e] * w[e] * kv[e];
            sx2 += xv[e] * xv[e];
        }
    }
    sk2 = wave_sum(sk2);
    sck = wave_sum(sck);
    sx2 = wave_sum(sx2);
    if (lane == 0) {
        s_part[wave][0] = sk2;
        s_part[wave][1] = sck;
        s_part[wave][2] = sx2;
    }
    __syncthreads();
    sk2 = sck = sx2 = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {  // in wave order: the same sums in every thread
        sk2 += s_part[w][0];
        sck += s_part[w][1];
        sx2 += s_part[w][2];
    }
    const float rh = 1.0f / sqrtf(sx2 * a.inv_d + kEps);
    const float rk = 1.0f / sqrtf(sk2 * a.inv_d + kEps);
    float s = rh * rk * sck * a.inv_sqrt_d;
    if (a.sqrt_mode) {
        const float sg = s > 0.f ? 1.f : (s < 0.f ? -1.f : 0.f);
        s = sg * sqrtf(fmaxf(fabsf(s), 1e-6f));
    }
    float alpha = 1.0f / (1.0f + expf(-s));
    if (tid == 0) {
        if (a.alpha_out != nullptr) a.alpha_out[n] = alpha;
        if (a.row_stats != nullptr) {
            float *st = a.row_stats + n * 4;
            st[0] = sx2;
            st[1] = sk2;
            st[2] = sck;
            st[3] = alpha;
        }
    }
    if (a.keep != nullptr && a.keep[n] == 0) alpha = 0.f;
    uint8_t *o = a.out + n * a.d * static_cast<int64_t>(sizeof(H));
    it = 0;
    for (int64_t j = static_cast<int64_t>(tid) * kLaneCols; j < a.d; j += kThreads * kLaneCols, ++it) {
        float xv[kLaneCols], vv[kLaneCols], ov[kLaneCols];
        if (it < kKeep) {
#pragma unroll
            for (int q = 0; q < kKeep; ++q)
                if (q == it)
#pragma unroll
                    for (int e = 0; e < kLaneCols; ++e) {
                        xv[e] = xk[q][e];
                        vv[e] = vk[q][e];
                    }
        } else {  // rows wider than kKeep steps: the rest is read again
            loadn<H, kLaneCols>(x + j * sizeof(H), xv);
            loadn<T, kLaneCols>(vr + j * sizeof(T), vv);
        }
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) ov[e] = xv[e] + round_to<H>(alpha * vv[e]);
        storen<H, kLaneCols>(o + j * sizeof(H), ov);
    }
}

// Backward per token (see the file comment): dV and the row sum of g V, the token's
// coefficients, then d hidden and dK; the token's a goes to the workspace for the scale
// gradients.
template <typename H, typename T, int kLaneCols>
__global__ __launch_bounds__(kThreads) void gate_rows_grad_kernel(const RowArgs a) {
    constexpr float kEps = 1.1920928955078125e-07f;
    __shared__ float s_part[kThreads / 64][4];
    const int tid = threadIdx.x;
    const int64_t n = blockIdx.x;
    const int64_t hrow = n * a.d, krow = n * a.kv_stride;
    const uint8_t *x = a.hidden + hrow * static_cast<int64_t>(sizeof(H));
    const uint8_t *g = a.grad_out + hrow * static_cast<int64_t>(sizeof(H));
    const uint8_t *kr = a.k + krow * static_cast<int64_t>(sizeof(T));
    const uint8_t *vr = a.v + krow * static_cast<int64_t>(sizeof(T));
    const float *st = a.stats_in + n * 4;
    const float sx2 = st[0], sk2 = st[1], sck = st[2], alpha = st[3];
    const bool kept = a.keep == nullptr || a.keep[n] != 0;
    const float alpha_eff = kept ? alpha : 0.f;
    // dV = round_T(alpha keep g) and sum g V
    float gv[1] = {0.f};
    for (int64_t j = static_cast<int64_t>(tid) * kLaneCols; j < a.d; j += kThreads * kLaneCols) {
        float gg[kLaneCols], vv[kLaneCols], dv[kLaneCols];
        loadn<H, kLaneCols>(g + j * sizeof(H), gg);
        loadn<T, kLaneCols>(vr + j * sizeof(T), vv);
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) {
            gv[0] += gg[e] * vv[e];
            dv[e] = alpha_eff * gg[e];
        }
        storen<T, kLaneCols>(a.grad_v + (n * a.d + j) * static_cast<int64_t>(sizeof(T)), dv);
    }
    block_sums<1>(gv, s_part);
    const float dalpha = kept ? gv[0] : 0.f;
    const float ds = dalpha * alpha * (1.f - alpha);
    const float rh = 1.0f / sqrtf(sx2 * a.inv_d + kEps);
    const float rk = 1.0f / sqrtf(sk2 * a.inv_d + kEps);
    const float s0 = rh * rk * sck * a.inv_sqrt_d;
    float ds0 = ds;
    if (a.sqrt_mode) ds0 = fabsf(s0) >= 1e-6f ? ds / (2.f * sqrtf(fabsf(s0))) : 0.f;
    const float ca = ds0 * rh * rk * a.inv_sqrt_d;
    const float c2 = ca * rh * rh * sck * a.inv_d;
    const float c3 = ca * rk * rk * sck * a.inv_d;
    if (tid == 0) a.coef[n] = ca;
    for (int64_t j = static_cast<int64_t>(tid) * kLaneCols; j < a.d; j += kThreads * kLaneCols) {
        float xv[kLaneCols], kv[kLaneCols], gg[kLaneCols], w[kLaneCols], dx[kLaneCols], dk[kLaneCols];
        loadn<H, kLaneCols>(x + j * sizeof(H), xv);
        loadn<T, kLaneCols>(kr + j * sizeof(T), kv);
        loadn<H, kLaneCols>(g + j * sizeof(H), gg);
        scale_products<kLaneCols>(a, j, w);
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) {
            dx[e] = gg[e] + round_to<H>(ca * w[e] * kv[e] - c2 * xv[e]);
            dk[e] = ca * w[e] * xv[e] - c3 * kv[e];
        }
        storen<H, kLaneCols>(a.grad_hidden + (hrow + j) * static_cast<int64_t>(sizeof(H)), dx);
        storen<T, kLaneCols>(a.grad_k + (n * a.d + j) * static_cast<int64_t>(sizeof(T)), dk);
    }
}

// Scale gradients, first level: column j of token block b, sum over the block's tokens (in
// order) of a x_j K_j; one thread per column, consecutive threads on consecutive columns.
template <typename H, typename T>
__global__ __launch_bounds__(kThreads) void gate_rows_scale_part_kernel(const RowArgs a) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t b = blockIdx.y;
    if (j >= a.d) return;
    const int64_t n0 = b * kScaleBlock, n1 = min(n0 + kScaleBlock, a.n);
    float p = 0.f;
    for (int64_t n = n0; n < n1; ++n) {
        float xv[1], kv[1];
        loadn<H, 1>(a.hidden + (n * a.d + j) * static_cast<int64_t>(sizeof(H)), xv);
        loadn<T, 1>(a.k + (n * a.kv_stride + j) * static_cast<int64_t>(sizeof(T)), kv);
        p += a.coef[n] * xv[0] * kv[0];
    }
    a.col_part[b * a.d + j] = p;
}

// Second level: the blocks' partials in order, times the other scale.
__global__ __launch_bounds__(kThreads) void gate_rows_scale_kernel(const RowArgs a, int64_t blocks,
                                                                   float *grad_q, float *grad_k) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (j >= a.d) return;
    float p = 0.f;
    for (int64_t b = 0; b < blocks; ++b) p += a.col_part[b * a.d + j];
    float q, k;
    if (a.scale_bf16) {
        q = bf16_bits_to_float(reinterpret_cast<const uint16_t *>(a.q_delta)[j]);
        k = bf16_bits_to_float(reinterpret_cast<const uint16_t *>(a.k_delta)[j]);
    } else {
        q = reinterpret_cast<const float *>(a.q_delta)[j];
        k = reinterpret_cast<const float *>(a.k_delta)[j];
    }
    grad_q[j] = (1.f + k) * p;
    grad_k[j] = (1.f + q) * p;
}

bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace me

using namespace me;

namespace me {
namespace {

// The argument checks and fields shared by the forward and the backward of the row kernels.
int rows_common(RowArgs &a, const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                const void *k_proj, const void *v_proj, int64_t kv_stride, int dtype,
                const void *q_scale_delta, const void *k_scale_delta, int scale_dtype, int gate_mode,
                const uint8_t *keep) {
    ME_CHECK_ARG(n >= 0 && n < (int64_t{1} << 31), "bad token count %lld", (long long)n);
    ME_CHECK_ARG(model_dim >= 1, "model_dim must be positive, got %lld", (long long)model_dim);
    ME_CHECK_ARG(hidden_dtype == ME_BF16 || hidden_dtype == ME_F32, "hidden dtype must be bf16 or fp32");
    ME_CHECK_ARG(dtype == ME_BF16 || dtype == ME_F32, "projection dtype must be bf16 or fp32");
    ME_CHECK_ARG(gate_mode == ME_GATE_SCALAR || gate_mode == ME_GATE_SCALAR_SQRT, "unknown gate mode %d",
                 gate_mode);
    ME_CHECK_ARG(kv_stride >= model_dim, "kv_stride %lld < model_dim %lld", (long long)kv_stride,
                 (long long)model_dim);
    a.hidden = static_cast<const uint8_t *>(hidden);
    a.k = static_cast<const uint8_t *>(k_proj);
    a.v = static_cast<const uint8_t *>(v_proj);
    a.keep = keep;
    a.n = n;
    a.d = model_dim;
    a.kv_stride = kv_stride;
    a.sqrt_mode = gate_mode == ME_GATE_SCALAR_SQRT;
    if (a.sqrt_mode) {
        ME_CHECK_ARG(q_scale_delta && k_scale_delta, "scalar_sqrt needs both scale deltas");
        ME_CHECK_ARG(scale_dtype == ME_BF16 || scale_dtype == ME_F32, "scale dtype must be bf16 or fp32");
        a.q_delta = static_cast<const uint8_t *>(q_scale_delta);
        a.k_delta = static_cast<const uint8_t *>(k_scale_delta);
        a.scale_bf16 = scale_dtype == ME_BF16;
    }
    a.inv_d = 1.0f / static_cast<float>(model_dim);
    a.inv_sqrt_d = static_cast<float>(1.0 / std::sqrt(static_cast<double>(model_dim)));
    return ME_OK;
}

// 16-byte accesses of 8 columns when every row start allows them, else one column per step.
bool wide_rows(const RowArgs &a, std::initializer_list<const void *> ptrs) {
    if (a.d % 8 != 0 || a.kv_stride % 8 != 0) return false;
    for (const void *p : ptrs)
        if (p != nullptr && !aligned16(p)) return false;
    return true;
}

#define ME_ROWS_DISPATCH(KERNEL, LC, grid, s, a)                                                     \
    do {                                                                                            \
        if (hidden_dtype == ME_BF16) {                                                              \
            if (dtype == ME_BF16) hipLaunchKernelGGL((KERNEL<uint16_t, uint16_t, LC>), grid, dim3(kThreads), 0, s, a); \
            else hipLaunchKernelGGL((KERNEL<uint16_t, float, LC>), grid, dim3(kThreads), 0, s, a); \
        } else {                                                                                    \
            if (dtype == ME_BF16) hipLaunchKernelGGL((KERNEL<float, uint16_t, LC>), grid, dim3(kThreads), 0, s, a); \
            else hipLaunchKernelGGL((KERNEL<float, float, LC>), grid, dim3(kThreads), 0, s, a);    \
        }                                                                                           \
    } while (0)

size_t rows_grad_workspace(int64_t n, int64_t d) {
    const size_t coef = (static_cast<size_t>(n) * 4 + 255) & ~size_t{255};
    return coef + static_cast<size_t>(ceil_div(n, kScaleBlock)) * static_cast<size_t>(d) * 4;
}

}  // namespace
}  // namespace me

extern "C" int me_gate_rows(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                            const void *k_proj, const void *v_proj, int64_t kv_stride, int dtype,
                            const void *q_scale_delta, const void *k_scale_delta, int scale_dtype,
                            int gate_mode, const uint8_t *keep, void *out, float *alpha_out,
                            float *row_stats, void *stream) {
    RowArgs a{};
    const int st = rows_common(a, hidden, hidden_dtype, n, model_dim, k_proj, v_proj, kv_stride, dtype,
                               q_scale_delta, k_scale_delta, scale_dtype, gate_mode, keep);
    if (st != ME_OK) return st;
    if (n == 0) return ME_OK;
    ME_CHECK_ARG(hidden && k_proj && v_proj && out, "null tensor pointer");
    a.out = static_cast<uint8_t *>(out);
    a.alpha_out = alpha_out;
    a.row_stats = row_stats;
    const dim3 grid(static_cast<unsigned>(n));
    hipStream_t s = as_stream(stream);
    if (wide_rows(a, {hidden, k_proj, v_proj, out, a.q_delta, a.k_delta}))
        ME_ROWS_DISPATCH(gate_rows_kernel, 8, grid, s, a);
    else
        ME_ROWS_DISPATCH(gate_rows_kernel, 1, grid, s, a);
    return check_launch("me_gate_rows");
}

extern "C" int me_gate_rows_backward_workspace_size(int64_t n, int64_t model_dim, size_t *bytes) {
    ME_CHECK_ARG(bytes != nullptr, "bytes is null");
    ME_CHECK_ARG(n >= 0 && model_dim >= 1, "bad shape n=%lld d=%lld", (long long)n, (long long)model_dim);
    *bytes = rows_grad_workspace(n, model_dim);
    return ME_OK;
}

extern "C" int me_gate_rows_backward(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                                     const void *k_proj, const void *v_proj, int64_t kv_stride, int dtype,
                                     const void *q_scale_delta, const void *k_scale_delta, int scale_dtype,
                                     int gate_mode, const uint8_t *keep, const void *grad_out,
                                     const float *row_stats, void *grad_hidden, void *grad_key,
                                     void *grad_value, float *grad_q_scale, float *grad_k_scale,
                                     void *workspace, size_t workspace_size, void *stream) {
    RowArgs a{};
    const int st = rows_common(a, hidden, hidden_dtype, n, model_dim, k_proj, v_proj, kv_stride, dtype,
                               q_scale_delta, k_scale_delta, scale_dtype, gate_mode, keep);
    if (st != ME_OK) return st;
    hipStream_t s = as_stream(stream);
    if (n == 0) {  // no tokens: zero scale gradients (a fill kernel: nothing for a captured graph to memset)
        if (a.sqrt_mode && grad_q_scale && grad_k_scale) {
            hipLaunchKernelGGL(gate_rows_scale_kernel, dim3(static_cast<unsigned>(ceil_div(model_dim, kThreads))),
                               dim3(kThreads), 0, s, a, int64_t{0}, grad_q_scale, grad_k_scale);
            return check_launch("me_gate_rows_backward (zero scale gradients)");
        }
        return ME_OK;
    }
    ME_CHECK_ARG(hidden && k_proj && v_proj && grad_out && row_stats && grad_hidden && grad_key && grad_value,
                 "null tensor pointer");
    if (a.sqrt_mode) ME_CHECK_ARG(grad_q_scale && grad_k_scale, "scalar_sqrt needs the scale gradient outputs");
    const size_t need = rows_grad_workspace(n, model_dim);
    if (workspace == nullptr || workspace_size < need) {
        set_error("me_gate_rows_backward: workspace of %zu bytes needed, got %zu", need, workspace_size);
        return ME_ERR_WORKSPACE;
    }
    a.grad_out = static_cast<const uint8_t *>(grad_out);
    a.stats_in = row_stats;
    a.grad_hidden = static_cast<uint8_t *>(grad_hidden);
    a.grad_k = static_cast<uint8_t *>(grad_key);
    a.grad_v = static_cast<uint8_t *>(grad_value);
    a.coef = static_cast<float *>(workspace);
    a.col_part = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) +
                                           ((static_cast<size_t>(n) * 4 + 255) & ~size_t{255}));
    const dim3 grid(static_cast<unsigned>(n));
    if (wide_rows(a, {hidden, k_proj, v_proj, grad_out, grad_hidden, grad_key, grad_value, a.q_delta, a.k_delta}))
        ME_ROWS_DISPATCH(gate_rows_grad_kernel, 8, grid, s, a);
    else
        ME_ROWS_DISPATCH(gate_rows_grad_kernel, 1, grid, s, a);
    int st_ = check_launch("me_gate_rows_backward (rows)");
    if (st_ != ME_OK || !a.sqrt_mode) return st_;
    const int64_t blocks = ceil_div(n, kScaleBlock);
    const dim3 pgrid(static_cast<unsigned>(ceil_div(model_dim, kThreads)), static_cast<unsigned>(blocks));
    if (hidden_dtype == ME_BF16) {
        if (dtype == ME_BF16) hipLaunchKernelGGL((gate_rows_scale_part_kernel<uint16_t, uint16_t>), pgrid, dim3(kThreads), 0, s, a);
        else hipLaunchKernelGGL((gate_rows_scale_part_kernel<uint16_t, float>), pgrid, dim3(kThreads), 0, s, a);
    } else {
        if (dtype == ME_BF16) hipLaunchKernelGGL((gate_rows_scale_part_kernel<float, uint16_t>), pgrid, dim3(kThreads), 0, s, a);
        else hipLaunchKernelGGL((gate_rows_scale_part_kernel<float, float>), pgrid, dim3(kThreads), 0, s, a);
    }
    st_ = check_launch("me_gate_rows_backward (scale partials)");
    if (st_ != ME_OK) return st_;
    hipLaunchKernelGGL(gate_rows_scale_kernel, dim3(static_cast<unsigned>(ceil_div(model_dim, kThreads))),
                       dim3(kThreads), 0, s, a, blocks, grad_q_scale, grad_k_scale);
    return check_launch("me_gate_rows_backward (scale gradients)");
}
