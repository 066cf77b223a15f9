// nkv_common.h -- shared types and helpers for the gfx950 NanoKV kernels.
//
// Written for CDNA4 (gfx950) only: wave64, bf16 MFMA
// (v_mfma_f32_32x32x16_bf16), hardware bf16 conversion (v_cvt_pk_bf16_f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/nanokv.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace nkv {

// ---------------------------------------------------------------- errors
// The last error message is thread-local; entry points return a negative
// NKV_ERR_* code and leave the text here (see nkv_last_error).
void set_error(const std::string& msg);
void clear_error();

#define NKV_REQUIRE(cond, code, msg)                                     \
    do {                                                                 \
        if (!(cond)) {                                                   \
            ::nkv::set_error(std::string(__func__) + ": " + (msg));      \
            return (code);                                               \
        }                                                                \
    } while (0)

#define NKV_HIP_CHECK(expr)                                                      \
    do {                                                                         \
        hipError_t _e = (expr);                                                  \
        if (_e != hipSuccess) {                                                  \
            ::nkv::set_error(std::string(__func__) + ": " #expr " failed: " +    \
                             hipGetErrorString(_e));                             \
            return NKV_ERR_HIP;                                                  \
        }                                                                        \
    } while (0)

// Launch-error check after <<<>>>: reports configuration errors without
// synchronising the stream.
#define NKV_LAUNCH_CHECK() NKV_HIP_CHECK(hipGetLastError())

// ---------------------------------------------------------------- numbers
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}

// fp16 bits -> fp32 (exact; subnormals handled by the hardware conversion).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    __bf16 h = (__bf16)f;  // v_cvt_pk_bf16_f32: round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ float bf16_round(float f) {
    return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

__device__ __forceinline__ float scale_bits_to_f32(uint16_t b, int scale_dtype) {
    return scale_dtype == NKV_DTYPE_FP16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace nkv
