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
#include "me_common.h"

#include <cmath>

namespace me {
namespace {

constexpr int kThreads = 256;  // one token per workgroup
constexpr int kLaneCols = 8;
constexpr int kKeep = 3;      // steps kept in registers: rows up to 3 * 2048 columns

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
};

template <typename X>
__device__ __forceinline__ void load8(const uint8_t *p, float (&v)[kLaneCols]);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint8_t *p, float (&v)[kLaneCols]) {
    const u32x4_v w = *as_global(reinterpret_cast<const u32x4_v *>(p));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf16_bits_to_float(static_cast<uint16_t>(w[e]));
        v[2 * e + 1] = bf16_bits_to_float(static_cast<uint16_t>(w[e] >> 16));
    }
}
template <>
__device__ __forceinline__ void load8<float>(const uint8_t *p, float (&v)[kLaneCols]) {
    const f32x4_v a = *as_global(reinterpret_cast<const f32x4_v *>(p));
    const f32x4_v b = *as_global(reinterpret_cast<const f32x4_v *>(p + 16));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = b[e];
    }
}

template <typename X>
__device__ __forceinline__ void store8(uint8_t *p, const float (&v)[kLaneCols]);
template <>
__device__ __forceinline__ void store8<uint16_t>(uint8_t *p, const float (&v)[kLaneCols]) {
    u32x4_v w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        w[e] = static_cast<uint32_t>(float_to_bf16_bits_rne(v[2 * e])) |
               (static_cast<uint32_t>(float_to_bf16_bits_rne(v[2 * e + 1])) << 16);
    *as_global(reinterpret_cast<u32x4_v *>(p)) = w;
}
template <>
__device__ __forceinline__ void store8<float>(uint8_t *p, const float (&v)[kLaneCols]) {
    *as_global(reinterpret_cast<f32x4_v *>(p)) = f32x4_v{v[0], v[1], v[2], v[3]};
    *as_global(reinterpret_cast<f32x4_v *>(p + 16)) = f32x4_v{v[4], v[5], v[6], v[7]};
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

template <typename H, typename T>
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
        load8<H>(x + j * sizeof(H), xv);
        load8<T>(kr + j * sizeof(T), kv);
#pragma unroll
        for (int q = 0; q < kKeep; ++q)
            if (q == it) {
#pragma unroll
                for (int e = 0; e < kLaneCols; ++e) xk[q][e] = xv[e];
                load8<T>(vr + j * sizeof(T), vk[q]);
            }
        if (a.q_delta != nullptr) {
            float qd[kLaneCols], kd[kLaneCols];
            if (a.scale_bf16) {
                load8<uint16_t>(a.q_delta + j * 2, qd);
                load8<uint16_t>(a.k_delta + j * 2, kd);
            } else {
                load8<float>(a.q_delta + j * 4, qd);
                load8<float>(a.k_delta + j * 4, kd);
            }
#pragma unroll
            for (int e = 0; e < kLaneCols; ++e) w[e] = (1.f + qd[e]) * (1.f + kd[e]);
        } else {
#pragma unroll
            for (int e = 0; e < kLaneCols; ++e) w[e] = 1.f;
        }
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
            load8<H>(x + j * sizeof(H), xv);
            load8<T>(vr + j * sizeof(T), vv);
        }
#pragma unroll
        for (int e = 0; e < kLaneCols; ++e) ov[e] = xv[e] + round_to<H>(alpha * vv[e]);
        store8<H>(o + j * sizeof(H), ov);
    }
}

bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace
}  // namespace me

using namespace me;

extern "C" int me_gate_rows(const void *hidden, int hidden_dtype, int64_t n, int64_t model_dim,
                            const void *k_proj, const void *v_proj, int64_t kv_stride, int dtype,
                            const void *q_scale_delta, const void *k_scale_delta, int scale_dtype,
                            int gate_mode, const uint8_t *keep, void *out, float *alpha_out,
                            float *row_stats, void *stream) {
    ME_CHECK_ARG(n >= 0, "negative token count");
    ME_CHECK_ARG(model_dim >= 8 && model_dim % 8 == 0, "model_dim must be a positive multiple of 8, got %lld",
                 (long long)model_dim);
    ME_CHECK_ARG(hidden_dtype == ME_BF16 || hidden_dtype == ME_F32, "hidden dtype must be bf16 or fp32");
    ME_CHECK_ARG(dtype == ME_BF16 || dtype == ME_F32, "projection dtype must be bf16 or fp32");
    ME_CHECK_ARG(gate_mode == ME_GATE_SCALAR || gate_mode == ME_GATE_SCALAR_SQRT, "unknown gate mode %d",
                 gate_mode);
    ME_CHECK_ARG(kv_stride >= model_dim && kv_stride % 8 == 0, "kv_stride %lld must be a multiple of 8, >= model_dim",
                 (long long)kv_stride);
    if (n == 0) return ME_OK;
    ME_CHECK_ARG(hidden && k_proj && v_proj && out, "null tensor pointer");
    ME_CHECK_ARG(aligned16(hidden) && aligned16(k_proj) && aligned16(v_proj) && aligned16(out),
                 "hidden, the projections and out must be 16-byte aligned");
    RowArgs a{};
    a.hidden = static_cast<const uint8_t *>(hidden);
    a.k = static_cast<const uint8_t *>(k_proj);
    a.v = static_cast<const uint8_t *>(v_proj);
    a.keep = keep;
    a.out = static_cast<uint8_t *>(out);
    a.alpha_out = alpha_out;
    a.row_stats = row_stats;
    a.n = n;
    a.d = model_dim;
    a.kv_stride = kv_stride;
    a.sqrt_mode = gate_mode == ME_GATE_SCALAR_SQRT;
    if (a.sqrt_mode) {
        ME_CHECK_ARG(q_scale_delta && k_scale_delta, "scalar_sqrt needs both scale deltas");
        ME_CHECK_ARG(scale_dtype == ME_BF16 || scale_dtype == ME_F32, "scale dtype must be bf16 or fp32");
        ME_CHECK_ARG(aligned16(q_scale_delta) && aligned16(k_scale_delta), "scale deltas must be 16-byte aligned");
        a.q_delta = static_cast<const uint8_t *>(q_scale_delta);
        a.k_delta = static_cast<const uint8_t *>(k_scale_delta);
        a.scale_bf16 = scale_dtype == ME_BF16;
    }
    a.inv_d = 1.0f / static_cast<float>(model_dim);
    a.inv_sqrt_d = static_cast<float>(1.0 / std::sqrt(static_cast<double>(model_dim)));
    ME_CHECK_ARG(n < (int64_t{1} << 31), "too many tokens for one call");
    const dim3 grid(static_cast<unsigned>(n));
    hipStream_t s = as_stream(stream);
    if (hidden_dtype == ME_BF16) {
        if (dtype == ME_BF16)
            hipLaunchKernelGGL((gate_rows_kernel<uint16_t, uint16_t>), grid, dim3(kThreads), 0, s, a);
        else
            hipLaunchKernelGGL((gate_rows_kernel<uint16_t, float>), grid, dim3(kThreads), 0, s, a);
    } else {
        if (dtype == ME_BF16)
            hipLaunchKernelGGL((gate_rows_kernel<float, uint16_t>), grid, dim3(kThreads), 0, s, a);
        else
            hipLaunchKernelGGL((gate_rows_kernel<float, float>), grid, dim3(kThreads), 0, s, a);
    }
    return check_launch("me_gate_rows");
}
