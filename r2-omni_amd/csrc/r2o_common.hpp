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

// a / b for 0 <= a < 2^22 and 1 <= b < 2^22 (head counts, head indices): the truncated product
// with the reciprocal estimate is within one of the quotient (relative error below 2^-22), and one
// remainder step each way corrects it; a few instructions in place of the integer division sequence.
__device__ __forceinline__ int r2o_div_small(int a, int b) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    const int r = a - q * b;
    q += (r >= b) - (r < 0);
    return q;
}

// ------------------------------------------------------------------ element conversions
__device__ __forceinline__ float r2o_bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ float r2o_f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// The float -> 16-bit roundings below round x itself, as the reference's float32 torch ops followed
// by a cast do: the empty asm makes x opaque, so the compiler cannot fold the operation that produced
// it into the conversion (it turns fp16(a * b) into one v_fma_mixlo_f16, a single rounding, even
// with contraction off).  r2o_pack_h2 / r2o_pack_bf2 (MFMA operands, no bit-exact contract) keep
// that freedom.

// Round-to-nearest-even float -> bfloat16 bits: gfx950's v_cvt_pk_bf16_f32 (NaN stays NaN).
__device__ __forceinline__ uint32_t r2o_f32_to_bf16(float x) {
    asm("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// Round-to-nearest-even float -> fp16 bits.
__device__ __forceinline__ uint32_t r2o_f32_to_f16(float x) {
    asm("" : "+v"(x));
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
// Two floats -> packed bf16 pair (round to nearest even), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t r2o_pack_bf2(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
}

// Cross-lane exchanges through the VALU, in place of the LDS-unit permute behind __shfl_xor:
// DPP within rows of 16 lanes, gfx950's v_permlane16_swap / v_permlane32_swap across rows.
template <int CTRL>
__device__ __forceinline__ float r2o_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// The value of lane (lane ^ M), M = 1, 2, 4 or 8.
template <int M>
__device__ __forceinline__ float r2o_lane_xor(float x) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8, "in-row exchange");
    if constexpr (M == 1) return r2o_dpp<0xB1>(x);  // quad_perm [1,0,3,2]
    else if constexpr (M == 2) return r2o_dpp<0x4E>(x);  // quad_perm [2,3,0,1]
    else if constexpr (M == 4) return r2o_dpp<0x1B>(r2o_dpp<0x141>(x));  // half-row mirror, then quad reverse
    else return r2o_dpp<0x128>(x);  // row_ror:8
}

// x swapped with itself across the M = 16 or 32 boundary: lanes below it get (first, second) =
// (x, x of lane ^ M), lanes above it (x of lane ^ M, x).
template <int M>
__device__ __forceinline__ void r2o_row_swap(float x, float& first, float& second) {
    static_assert(M == 16 || M == 32, "cross-row exchange");
    const uint32_t u = __float_as_uint(x);
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        first = __uint_as_float(r[0]);
        second = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        first = __uint_as_float(r[0]);
        second = __uint_as_float(r[1]);
    }
}

// x + (x of lane ^ M), the same value in both lanes of a pair, for M = 16 or 32.
template <int M>
__device__ __forceinline__ float r2o_sum_lane_pair(float x) {
    float a, b;
    r2o_row_swap<M>(x, a, b);
    return a + b;
}

// One butterfly stage of the FWHT over lanes: lane t without bit M keeps y + y', with it y' - y,
// where y' is lane t ^ M's value.
template <int M>
__device__ __forceinline__ void r2o_fwht_stage(float& y0, float& y1, int t) {
    const bool upper = (t & M) != 0;
    if constexpr (M < 16) {
        const float o0 = r2o_lane_xor<M>(y0), o1 = r2o_lane_xor<M>(y1);
        y0 = upper ? o0 - y0 : y0 + o0;
        y1 = upper ? o1 - y1 : y1 + o1;
    } else {
        float a0, b0, a1, b1;
        r2o_row_swap<M>(y0, a0, b0);
        r2o_row_swap<M>(y1, a1, b1);
        y0 = upper ? a0 - b0 : a0 + b0;
        y1 = upper ? a1 - b1 : a1 + b1;
    }
}

// Orthonormal 128-point FWHT of a row held by one full wave: lane t holds x[t] in y0 and x[t + 64]
// in y1.  Strides 1 .. 32 are lane-xor butterflies, stride 64 is a butterfly inside the lane, in
// the stage order of triton_fwht_128 (triton_qwen_mrope.py:23-32: stride 1 first, 64 last), so
// every fp32 sum is formed from the same operands in the same order.
__device__ __forceinline__ void r2o_fwht128_pair(float& y0, float& y1, int t) {
    r2o_fwht_stage<1>(y0, y1, t);
    r2o_fwht_stage<2>(y0, y1, t);
    r2o_fwht_stage<4>(y0, y1, t);
    r2o_fwht_stage<8>(y0, y1, t);
    r2o_fwht_stage<16>(y0, y1, t);
    r2o_fwht_stage<32>(y0, y1, t);
    const float s0 = y0 + y1, s1 = y0 - y1;
    y0 = s0 * 0.08838834764831845f;
    y1 = s1 * 0.08838834764831845f;
}

#define R2O_CHECK_LAUNCH()                                      \
    do {                                                        \
        if (hipGetLastError() != hipSuccess) return R2O_ELAUNCH; \
    } while (0)
