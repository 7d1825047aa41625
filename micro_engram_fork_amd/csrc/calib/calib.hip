// Calibration kernels for bench.py: what the part delivers for the gather's bytes with nothing
// of the engram path in front. Not part of the engram path; the library they build into
// (libmicro_engram_calib.so) is loaded by the benchmark only.
//
//   me_calib_copy_nt      dst = src in 16-byte chunks, `unroll` chunks per thread (all loads
//                         issued before the stores), non-temporal loads and stores: a plain
//                         sequential copy of the gather's output size.
//   me_calib_random_rows  out[t][k] = table_k[row(t, k)] for n_tok tokens and n_tables tables of
//                         64-element rows, with row(t, k) a 32-bit integer mix of (t * n_tables
//                         + k, salt) modulo the table's rows: the gather's access shape (random
//                         128-byte row reads, the concatenated rows written in token order) with
//                         the row ids coming from arithmetic, so no dependent load precedes the
//                         row reads.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(256) void copy_nt_kernel(const u32x4 *__restrict__ src,
                                                      u32x4 *__restrict__ dst, int64_t n16) {
    const int64_t b0 = static_cast<int64_t>(blockIdx.x) * 256 * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t i = b0 + static_cast<int64_t>(u) * 256;
        if (i < n16) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t i = b0 + static_cast<int64_t>(u) * 256;
        if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
    }
}

struct Tables {
    uint64_t base[64];
    uint32_t rows[64];
};

template <int U>
__global__ __launch_bounds__(256) void random_rows_kernel(const Tables t, int n_tables,
                                                          u32x4 *__restrict__ out, int64_t n16,
                                                          uint32_t salt) {
    // 16-byte chunk c of the output: row pair p = c / 8 (token p / n_tables, table p % n_tables)
    const int64_t b0 = static_cast<int64_t>(blockIdx.x) * 256 * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = b0 + static_cast<int64_t>(u) * 256;
        if (c < n16) {
            const uint32_t p = static_cast<uint32_t>(c >> 3);
            const uint32_t k = p % static_cast<uint32_t>(n_tables);
            uint32_t h = p * 2654435761u + salt;
            h ^= h >> 15;
            h *= 2246822519u;
            h ^= h >> 13;
            const uint32_t row = h % t.rows[k];
            v[u] = *(reinterpret_cast<const u32x4 *>(t.base[k] + static_cast<uint64_t>(row) * 128) +
                     (c & 7));
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = b0 + static_cast<int64_t>(u) * 256;
        if (c < n16) __builtin_nontemporal_store(v[u], out + c);
    }
}

}  // namespace

// bytes: multiple of 16; unroll: 3 or 12 (the best shapes measured on MI355X for 25 MB).
extern "C" int me_calib_copy_nt(const void *src, void *dst, int64_t bytes, int unroll,
                                void *stream) {
    if (bytes <= 0 || bytes % 16 != 0 || src == nullptr || dst == nullptr) return -1;
    const int64_t n16 = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (unroll == 3) {
        hipLaunchKernelGGL(copy_nt_kernel<3>, dim3((n16 + 767) / 768), dim3(256), 0, s,
                           static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), n16);
    } else if (unroll == 12) {
        hipLaunchKernelGGL(copy_nt_kernel<12>, dim3((n16 + 3071) / 3072), dim3(256), 0, s,
                           static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), n16);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// tables: n_tables device addresses of [rows, 64] bf16 tables (128-byte rows, 16-byte aligned);
// out: n_tok * n_tables * 128 bytes.
extern "C" int me_calib_random_rows(const void *const *tables, const int64_t *rows, int n_tables,
                                    void *out, int64_t n_tok, uint32_t salt, void *stream) {
    if (n_tables < 1 || n_tables > 64 || n_tok < 1 || out == nullptr) return -1;
    Tables t{};
    for (int k = 0; k < n_tables; ++k) {
        if (tables[k] == nullptr || rows[k] < 1 || rows[k] >= (int64_t{1} << 32)) return -1;
        t.base[k] = reinterpret_cast<uint64_t>(tables[k]);
        t.rows[k] = static_cast<uint32_t>(rows[k]);
    }
    const int64_t n16 = n_tok * n_tables * 8;
    hipLaunchKernelGGL(random_rows_kernel<2>, dim3((n16 + 511) / 512), dim3(256), 0,
                       static_cast<hipStream_t>(stream), t, n_tables, static_cast<u32x4 *>(out),
                       n16, salt);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
