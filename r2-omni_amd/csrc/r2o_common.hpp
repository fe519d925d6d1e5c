// Shared device helpers for the gfx950 SSPA kernels: element conversions, wave reductions,
// MFMA wrappers and bit utilities.  Written for CDNA4 wave64 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "r2o_sspa.h"

#define R2O_WAVE 64

typedef _Float16 r2o_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 r2o_bf16x8 __attribute__((ext_vector_type(8)));
typedef float r2o_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t r2o_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t r2o_u2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------- global-memory loads
// Pointers read from device-side descriptor tables are generic; loading through them would
// emit flat loads, which also count against lgkmcnt and so make every LDS wait drain the
// outstanding HBM prefetches.  Cast to the global address space before dereferencing.
#define R2O_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T r2o_ldg(const T* p) {
    return *(const R2O_GLOBAL T*)p;
}

// ------------------------------------------------------------------ element conversions
__device__ __forceinline__ float r2o_bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ float r2o_f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Round-to-nearest-even float -> bfloat16 bits (finite inputs; NaN stays NaN).
__device__ __forceinline__ uint32_t r2o_f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u) return (u >> 16) | ((u & 0xffffu) ? 0x40u : 0u);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Round-to-nearest-even float -> fp16 bits.
__device__ __forceinline__ uint32_t r2o_f32_to_f16(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

__device__ __forceinline__ float r2o_load_elem(const uint16_t* p, int64_t i, int dtype) {
    uint32_t b = p[i];
    return dtype == 0 ? r2o_bf16_to_f32(b) : r2o_f16_to_f32(b);
}

__device__ __forceinline__ float r2o_round_dtype(float x, int dtype) {
    return dtype == 0 ? r2o_bf16_to_f32(r2o_f32_to_bf16(x)) : r2o_f16_to_f32(r2o_f32_to_f16(x));
}

// ------------------------------------------------------------------------ wave reductions
__device__ __forceinline__ float r2o_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, R2O_WAVE));
    return v;
}

// ------------------------------------------------------------------------- bit utilities
// v_perm_b32: selects bytes from the 8-byte value {hi, lo} (lo = bytes 0..3).
__device__ __forceinline__ uint32_t r2o_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// ------------------------------------------------------------------------- MFMA wrappers
// 16x16x32 MFMA, gfx950.  Operand layout (per wave, lane l, l16 = l % 16, g = l / 16):
//   A: row m = l16, k = 8g .. 8g+7 ; B: column n = l16, k = 8g .. 8g+7
//   C/D: column n = l16, rows 4g .. 4g+3
__device__ __forceinline__ r2o_f4 r2o_mfma_f16(r2o_u4 a, r2o_u4 b, r2o_f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(r2o_half8, a),
                                                  __builtin_bit_cast(r2o_half8, b), c, 0, 0, 0);
}

__device__ __forceinline__ r2o_f4 r2o_mfma_bf16(r2o_u4 a, r2o_u4 b, r2o_f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(r2o_bf16x8, a),
                                                   __builtin_bit_cast(r2o_bf16x8, b), c, 0, 0, 0);
}

// Packed-half helpers (two fp16 in one dword).
typedef _Float16 r2o_h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t r2o_h2_sub(uint32_t a, uint32_t b) {
    r2o_h2 r = __builtin_bit_cast(r2o_h2, a) - __builtin_bit_cast(r2o_h2, b);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t r2o_h2_mul(uint32_t a, uint32_t b) {
    r2o_h2 r = __builtin_bit_cast(r2o_h2, a) * __builtin_bit_cast(r2o_h2, b);
    return __builtin_bit_cast(uint32_t, r);
}
// Two floats -> packed fp16 pair (round to nearest even).
__device__ __forceinline__ uint32_t r2o_pack_h2(float lo, float hi) {
    r2o_h2 r = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, r);
}
// Two floats -> packed bf16 pair (round to nearest even).
__device__ __forceinline__ uint32_t r2o_pack_bf2(float lo, float hi) {
    return r2o_f32_to_bf16(lo) | (r2o_f32_to_bf16(hi) << 16);
}

// Orthonormal 128-point FWHT of a row held by one wave: lane t holds x[t] in y0 and x[t + 64]
// in y1.  Stride 64 is a butterfly inside the lane, strides 32 .. 1 are lane-xor butterflies.
__device__ __forceinline__ void r2o_fwht128_pair(float& y0, float& y1, int t) {
    const float s0 = y0 + y1, s1 = y0 - y1;
    y0 = s0;
    y1 = s1;
#pragma unroll
    for (int stride = 1; stride < 64; stride <<= 1) {
        const float o0 = __shfl_xor(y0, stride, R2O_WAVE), o1 = __shfl_xor(y1, stride, R2O_WAVE);
        const bool upper = (t & stride) != 0;
        y0 = upper ? o0 - y0 : y0 + o0;
        y1 = upper ? o1 - y1 : y1 + o1;
    }
    y0 *= 0.08838834764831845f;
    y1 *= 0.08838834764831845f;
}

#define R2O_CHECK_LAUNCH()                                      \
    do {                                                        \
        if (hipGetLastError() != hipSuccess) return R2O_ELAUNCH; \
    } while (0)
