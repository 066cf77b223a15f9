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
typedef double f64x2 __attribute__((ext_vector_type(2)));

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

// fp64 -> fp32 (round to nearest even), kept as an fp32 value: a later bf16
// rounding of it is the second of two roundings, as in the reference's
// fp64 -> fp32 -> bf16.  (Without the barrier the compiler may fold the two
// truncations into one fp64 -> bf16 rounding, which differs at double-
// rounding ties.)
__device__ __forceinline__ float f64_to_f32(double x) {
    float f = (float)x;
    __asm__("" : "+v"(f));
    return f;
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

// A load from device (global) memory through a pointer whose address space
// the compiler cannot infer (one read from a table in memory or from LDS).
// Such loads are otherwise flat, and flat loads also count against lgkmcnt:
// every wait for an LDS read would then wait for them as well.
#define NKV_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
    return *(const NKV_GLOBAL T*)p;
}

// ---------------------------------------------------------------- MFMA / LDS helpers
__device__ __forceinline__ int read_id(const void* ids, int id_bytes, int64_t i) {
    if (id_bytes == 1) return ldg(reinterpret_cast<const uint8_t*>(ids) + i);
    if (id_bytes == 2) return ldg(reinterpret_cast<const uint16_t*>(ids) + i);
    return ldg(reinterpret_cast<const int32_t*>(ids) + i);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

#define NKV_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// one 16-byte-per-lane global -> LDS DMA (the 64 lanes fill 1 KB at l); a
// function of its own so that kernel templates name no target builtin in
// their bodies (the host pass then instantiates them for every width)
__device__ __forceinline__ void dma16(const void* g, void* l) {
    __builtin_amdgcn_global_load_lds(g, NKV_LDS(l), 16, 0, 0);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits [3:0] and [15:14]; the
// other counters at their maxima, i.e. not waited on)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0) and s_barrier, with the compiler keeping memory
// accesses on their side of it (in-flight DMAs are not waited for)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ bf16x8 lds_b128(const uint16_t* p) {
    return *reinterpret_cast<const bf16x8*>(p);
}

// Two 8-byte LDS reads forming one bf16x8 operand: p[0..3] and p[8..11].
__device__ __forceinline__ bf16x8 lds_2x64(const uint16_t* p) {
    u32x2 a = *reinterpret_cast<const u32x2*>(p);
    u32x2 b = *reinterpret_cast<const u32x2*>(p + 8);
    u32x4 v = {a[0], a[1], b[0], b[1]};
    return as_bf16x8(v);
}

// v_mfma_f32_32x32x16_bf16.  Lane l supplies row l % 32 of A and column
// l % 32 of B with k = 8 * (l / 32) + [0, 8); accumulator element i of lane l
// is (row 8*(i/4) + 4*(l/32) + i%4, column l % 32).
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// max / sum of x over lanes l and l ^ 32 (v_permlane32_swap exchanges the
// two half-waves of two copies of x; the pair holds both values in either
// order, so the result is symmetric).
__device__ __forceinline__ float halfwave_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float halfwave_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Eight INT4 codes of one dword (byte j: code 2j low nibble, 2j+1 high
// nibble, stored as code + 7) times their group scale s, as the bf16x8 MFMA
// operand in k order.  (nibble - 7) * s = fma(nibble, s, -7 s): both products
// are exact in fp32 (<= 15 significant bits), so the fma returns the exact
// value and the bf16 conversion rounds it once, as the reference does.
// unpack8 in pieces: split() prepares the two masked words of w (opaque, so
// that v_cvt_f32_ubyte{0..3} converts each byte in one instruction), and
// pair(b) is operand dword b (codes 2b and 2b+1).
struct Unpack8 {
    uint32_t ev, od;
    __device__ __forceinline__ void split(uint32_t w) {
        ev = w & 0x0f0f0f0fu;
        od = (w >> 4) & 0x0f0f0f0fu;
        asm("" : "+v"(ev));
        asm("" : "+v"(od));
    }
    __device__ __forceinline__ uint32_t pair(int b, float s, float ns7) const {
        return pack_bf16x2(fmaf((float)((ev >> (8 * b)) & 0xffu), s, ns7),
                           fmaf((float)((od >> (8 * b)) & 0xffu), s, ns7));
    }
};

__device__ __forceinline__ bf16x8 unpack8(uint32_t w, float s, float ns7) {
    uint32_t ev = w & 0x0f0f0f0fu;         // codes 0, 2, 4, 6 (byte lanes)
    uint32_t od = (w >> 4) & 0x0f0f0f0fu;  // codes 1, 3, 5, 7
    // opaque: otherwise the known 4-bit range turns each byte conversion
    // into a bit-field extract plus a conversion, where v_cvt_f32_ubyte{0..3}
    // converts byte b of the masked word in one instruction
    asm("" : "+v"(ev));
    asm("" : "+v"(od));
    u32x4 o;
#pragma unroll
    for (int b = 0; b < 4; ++b)
        o[b] = pack_bf16x2(fmaf((float)((ev >> (8 * b)) & 0xffu), s, ns7),
                           fmaf((float)((od >> (8 * b)) & 0xffu), s, ns7));
    return as_bf16x8(o);
}

}  // namespace nkv
