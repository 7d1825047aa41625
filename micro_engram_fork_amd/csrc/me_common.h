// Shared pieces of the gfx950 kernels: error reporting, element types, bf16 rounding and
// the exact integer arithmetic of the n-gram hash.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "micro_engram.h"

namespace me {

// ---------------------------------------------------------------------------------------------
// Errors: every entry point returns a status code and leaves a message for me_last_error().
void set_error(const char *fmt, ...);

inline int fail(int code, const char *msg) {
    set_error("%s", msg);
    return code;
}

#define ME_CHECK_ARG(cond, ...)            \
    do {                                   \
        if (!(cond)) {                     \
            ::me::set_error(__VA_ARGS__);  \
            return ME_ERR_INVALID;         \
        }                                  \
    } while (0)

// Checks the launch just enqueued; returns ME_ERR_HIP with the runtime's message on failure.
int check_launch(const char *what);

inline size_t dtype_size(int dt) {
    switch (dt) {
        case ME_I32: return 4;
        case ME_I64: return 8;
        case ME_F32: return 4;
        case ME_BF16: return 2;
        case ME_U8: return 1;
        default: return 0;
    }
}

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32. bf16 is the upper half of an fp32; fp32 -> bf16 rounds to nearest, ties to
// even (what torch's .to(torch.bfloat16) does), NaN stays NaN. gfx950 converts in hardware
// (v_cvt_pk_bf16_f32, two values per instruction).
__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t float_to_bf16_bits_rne(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Value of an fp32 after a round trip through bf16 (the rounding a bf16 tensor applies).
__device__ __forceinline__ float round_to_bf16(float f) {
    return bf16_bits_to_float(float_to_bf16_bits_rne(f));
}

// ---------------------------------------------------------------------------------------------
// Hash arithmetic, exact for every int64 input.
//
// The reference sums token * mult in int64 (wrapping), then takes Python-style floor modulo
// by P = 2^31 - 1 and by the table's row count (torch's integer `%`). P is a Mersenne prime,
// so u mod P folds as (u & P) + (u >> 31) (2^31 == 1 mod P). The row count modulo uses
// Lemire, Kaser & Kurz, "Faster Remainder by Direct Computation" (2019): with
// M = floor((2^64 - 1) / d) + 1, a mod d = hi64((M * a mod 2^64) * d) for 32-bit a and d.
constexpr uint64_t kPrime = 2147483647ull;  // 2^31 - 1

__host__ __device__ __forceinline__ uint64_t mersenne_mod(uint64_t u) {  // u < 2^64
    uint64_t r = (u & kPrime) + (u >> 31);   // < 2^31 + 2^33
    r = (r & kPrime) + (r >> 31);            // < 2^31 + 8
    return r >= kPrime ? r - kPrime : r;
}

// floor modulo of a wrapped int64 sum by P: result in [0, P).
__host__ __device__ __forceinline__ uint32_t floor_mod_prime(uint64_t x_bits) {
    const int64_t x = static_cast<int64_t>(x_bits);
    if (x >= 0) return static_cast<uint32_t>(mersenne_mod(static_cast<uint64_t>(x)));
    // x < 0: x mod P = P - 1 - ((-x - 1) mod P); -x - 1 = ~x never overflows.
    return static_cast<uint32_t>(kPrime - 1 - mersenne_mod(~x_bits));
}

// Lemire constant for divisor d (1 <= d < 2^32). d == 1 gives 0, which yields remainder 0.
inline uint64_t fastmod_magic(uint32_t d) { return UINT64_MAX / d + 1; }

__device__ __forceinline__ uint32_t fastmod_u32(uint32_t a, uint64_t magic, uint32_t d) {
    const uint64_t low = magic * static_cast<uint64_t>(a);
    return static_cast<uint32_t>(__umul64hi(low, static_cast<uint64_t>(d)));
}

// ---------------------------------------------------------------------------------------------
// Global-memory view of a device address. A pointer the compiler cannot trace back to a kernel
// argument (one rebuilt from an integer, or read out of LDS) is generic, and accesses through
// it compile to flat_load / flat_store, which count on lgkmcnt as well as vmcnt: every later
// wait for an LDS read then also waits for them, which serialises a thread's loads. Through
// an address-space-1 pointer they compile to global_load / global_store, counted by vmcnt alone.
template <typename T>
using gmem_ptr = __attribute__((address_space(1))) T *;

// Clang vector types for loads and stores through such pointers (HIP's uint2 / float4 are
// class types, which cannot be copied out of another address space).
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ gmem_ptr<T> as_global(T *p) {
    return (gmem_ptr<T>)(p);
}

template <typename T>
__device__ __forceinline__ gmem_ptr<T> as_global_addr(uint64_t addr) {
    return (gmem_ptr<T>)(reinterpret_cast<T *>(addr));
}

// ---------------------------------------------------------------------------------------------
// Launch helpers.
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace me
