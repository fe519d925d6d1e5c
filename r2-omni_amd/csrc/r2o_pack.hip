// Quantise/pack, gather, Recent-FP append/shift and FWHT kernels for gfx950.
//
// Bit-exactness with the reference's torch CPU quantisers (compact_int4_key.py:83-110,
// quantization.py:19-50, int2_reference.py:96-151): IEEE fp32 division (__fdiv_rn), round half
// to even (__builtin_rintf -> v_rndne_f32), no contraction (the file is built with
// -ffp-contract=off), fp32 step quantisation with fp16-RNE storage of the step.
#include "r2o_common.hpp"

namespace {

constexpr float kEps = 1.0e-6f;

// ----------------------------------------------------------------------------- INT4 keys
// grid (superblocks to write, hkv), block 64: thread t owns channels 2t, 2t+1 (byte t).
__global__ __launch_bounds__(64) void pack_int4_k_kernel(
    const uint16_t* __restrict__ src, int dtype, int64_t src_tokens, const int64_t* __restrict__ index,
    int64_t n, int64_t tail, int64_t dst_start, uint8_t* packed, uint16_t* scale, uint8_t* zero,
    uint32_t* operands, int64_t capacity, int64_t superblocks, int sb) {
    __shared__ uint16_t s_half[128];
    __shared__ uint8_t s_zero[128];
    const int t = threadIdx.x;
    const int64_t h = blockIdx.y;
    const int64_t total = tail + n;
    const int64_t first = (int64_t)blockIdx.x * sb;  // relative to dst_start
    const int64_t count = min((int64_t)sb, total - first);
    if (count <= 0) return;
    const int64_t block_row = dst_start / sb + blockIdx.x;
    uint8_t* prow = packed + (h * capacity + dst_start + first) * 64 + t;
    uint16_t* srow = scale + (h * superblocks + block_row) * 128 + 2 * t;
    uint8_t* zrow = zero + (h * superblocks + block_row) * 128 + 2 * t;
    // old metadata of the tail superblock (only block 0 can hold tail positions)
    const float os0 = r2o_f16_to_f32(srow[0]), os1 = r2o_f16_to_f32(srow[1]);
    const float oz0 = (float)zrow[0], oz1 = (float)zrow[1];
    auto value = [&](int64_t j, float& x0, float& x1) {
        const int64_t pos = first + j;
        if (pos < tail) {  // dequantise-then-round the partial tail (compact_int4_key.py:215-216)
            const uint32_t b = prow[j * 64];
            x0 = r2o_round_dtype(((float)(b & 15u) - oz0) * os0, dtype);
            x1 = r2o_round_dtype(((float)(b >> 4) - oz1) * os1, dtype);
        } else {
            const int64_t i = pos - tail;
            const int64_t row = index ? index[i] : i;
            const uint32_t pair = *reinterpret_cast<const uint32_t*>(src + (h * src_tokens + row) * 128 + 2 * t);
            x0 = dtype == 0 ? r2o_bf16_to_f32(pair & 0xffffu) : r2o_f16_to_f32(pair & 0xffffu);
            x1 = dtype == 0 ? r2o_bf16_to_f32(pair >> 16) : r2o_f16_to_f32(pair >> 16);
        }
    };
    float mn0 = 0.f, mn1 = 0.f, mx0 = 0.f, mx1 = 0.f;  // min(min x, 0), max(max x, 0)
    for (int64_t j = 0; j < count; ++j) {
        float x0, x1;
        value(j, x0, x1);
        mn0 = fminf(mn0, x0); mx0 = fmaxf(mx0, x0);
        mn1 = fminf(mn1, x1); mx1 = fmaxf(mx1, x1);
    }
    const float st0 = fmaxf(__fdiv_rn(mx0 - mn0, 15.0f), kEps);
    const float st1 = fmaxf(__fdiv_rn(mx1 - mn1, 15.0f), kEps);
    const float zp0 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(-mn0, st0)), 0.f), 15.f);
    const float zp1 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(-mn1, st1)), 0.f), 15.f);
    for (int64_t j = 0; j < count; ++j) {
        float x0, x1;
        value(j, x0, x1);  // reads the old tail code before this thread overwrites it
        const float c0 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(x0, st0) + zp0), 0.f), 15.f);
        const float c1 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(x1, st1) + zp1), 0.f), 15.f);
        prow[j * 64] = (uint8_t)((uint32_t)c0 | ((uint32_t)c1 << 4));
    }
    const uint16_t h0 = (uint16_t)r2o_f32_to_f16(st0), h1 = (uint16_t)r2o_f32_to_f16(st1);
    srow[0] = h0;
    srow[1] = h1;
    zrow[0] = (uint8_t)zp0;
    zrow[1] = (uint8_t)zp1;
    if (operands) {  // QK MFMA operands of this superblock (layout in r2o_sspa.h)
        s_half[2 * t] = h0;
        s_half[2 * t + 1] = h1;
        s_zero[2 * t] = (uint8_t)zp0;
        s_zero[2 * t + 1] = (uint8_t)zp1;
        __syncthreads();
        const int g = t >> 4, j = (t >> 2) & 3, u = t & 3;
        const int c = 32 * g + 8 * j + u;
        uint32_t* orow = operands + (h * superblocks + block_row) * 128 + g * 32 + 4 * j + u;
        if (u & 1) {  // channel pair read in place 4 bits up: code enters as 1024 + 16 c
            orow[0] = r2o_f32_to_f16(r2o_f16_to_f32(s_half[c]) * 0.0625f) |
                      (r2o_f32_to_f16(r2o_f16_to_f32(s_half[c + 4]) * 0.0625f) << 16);
            orow[16] = (0xE400u | ((uint32_t)s_zero[c] << 4)) | ((0xE400u | ((uint32_t)s_zero[c + 4] << 4)) << 16);
        } else {
            orow[0] = (uint32_t)s_half[c] | ((uint32_t)s_half[c + 4] << 16);
            orow[16] = (0xE400u | s_zero[c]) | ((0xE400u | (uint32_t)s_zero[c + 4]) << 16);
        }
    }
}

// Whole superblocks (no tail to requantise), staged through LDS in chunks of 32 token rows by
// global->LDS DMA (four 256-byte rows per instruction, every DMA of a chunk issued before any is
// waited for; token rows from the gather index, broadcast by lane).  One pass over the chunks for
// the range and one for the codes (a 32-token superblock keeps its only chunk in LDS between the
// two; a larger one reads its chunks again, from L2).  The code rows leave through LDS as 16-byte
// stores.  10 KB of LDS for every superblock size.  Same arithmetic per element as
// pack_int4_k_kernel.
template <int SB>
__global__ __launch_bounds__(64) void pack_int4_k_full_kernel(
    const uint16_t* __restrict__ src, int dtype, int64_t src_tokens, const int64_t* __restrict__ index,
    int64_t n, int64_t dst_start, uint8_t* packed, uint16_t* scale, uint8_t* zero, uint32_t* operands,
    int64_t capacity, int64_t superblocks) {
    __shared__ uint16_t s_half[128];
    __shared__ uint8_t s_zero[128];
    __shared__ __align__(16) uint32_t s_raw[32 * 64];
    __shared__ __align__(16) uint8_t s_codes[32 * 64];
    const int t = threadIdx.x;
    const int64_t h = blockIdx.y;
    const int64_t first = (int64_t)blockIdx.x * SB;
    const int count = (int)min((int64_t)SB, n - first);
    const int64_t block_row = dst_start / SB + blockIdx.x;
    int row_lo = 0, row_hi = 0;  // source rows of tokens first + t and first + 64 + t
    if (t < count) row_lo = (int)(index ? index[first + t] : first + t);
    if (SB > 64 && t + 64 < count) row_hi = (int)(index ? index[first + 64 + t] : first + 64 + t);
    const int last = count > 64 ? __builtin_amdgcn_readlane(row_hi, count - 65)
                                : __builtin_amdgcn_readlane(row_lo, count - 1);
    // lane t moves 16-byte chunk t % 16 of token 32 c + 4 k + t / 16 (rows past the end re-read
    // the last token, whose LDS copy is never used)
    const uint16_t* hsrc = src + h * src_tokens * 128 + 8 * (t & 15);
    auto load_chunk = [&](int c) {
        int rows[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // every row first, then every DMA
            const int tk = 32 * c + 4 * k + (t >> 4);
            const int row = tk < 64 ? __shfl(row_lo, tk & 63, R2O_WAVE) : __shfl(row_hi, tk & 63, R2O_WAVE);
            rows[k] = tk < count ? row : last;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (32 * c + 4 * k < count)
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void*)(hsrc + (int64_t)rows[k] * 128),
                    (__attribute__((address_space(3))) void*)(s_raw + 4 * k * 64), 16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the chunk has landed
        __builtin_amdgcn_wave_barrier();
    };
    const int chunks = (count + 31) / 32;
    float mn0 = 0.f, mn1 = 0.f, mx0 = 0.f, mx1 = 0.f;  // min(min x, 0), max(max x, 0)
    for (int c = 0; c < chunks; ++c) {
        if (c > 0) __builtin_amdgcn_wave_barrier();  // every lane is done reading the previous chunk
        load_chunk(c);
        for (int j = 0; j < min(32, count - 32 * c); ++j) {
            const uint32_t raw = s_raw[j * 64 + t];
            const float x0 = dtype == 0 ? r2o_bf16_to_f32(raw & 0xffffu) : r2o_f16_to_f32(raw & 0xffffu);
            const float x1 = dtype == 0 ? r2o_bf16_to_f32(raw >> 16) : r2o_f16_to_f32(raw >> 16);
            mn0 = fminf(mn0, x0); mx0 = fmaxf(mx0, x0);
            mn1 = fminf(mn1, x1); mx1 = fmaxf(mx1, x1);
        }
    }
    const float st0 = fmaxf(__fdiv_rn(mx0 - mn0, 15.0f), kEps);
    const float st1 = fmaxf(__fdiv_rn(mx1 - mn1, 15.0f), kEps);
    const float zp0 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(-mn0, st0)), 0.f), 15.f);
    const float zp1 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(-mn1, st1)), 0.f), 15.f);
    uint8_t* pbase = packed + (h * capacity + dst_start + first) * 64;
    for (int c = 0; c < chunks; ++c) {
        if (chunks > 1) {
            __builtin_amdgcn_wave_barrier();
            load_chunk(c);
        }
        const int nj = min(32, count - 32 * c);
        for (int j = 0; j < nj; ++j) {
            const uint32_t raw = s_raw[j * 64 + t];
            const float x0 = dtype == 0 ? r2o_bf16_to_f32(raw & 0xffffu) : r2o_f16_to_f32(raw & 0xffffu);
            const float x1 = dtype == 0 ? r2o_bf16_to_f32(raw >> 16) : r2o_f16_to_f32(raw >> 16);
            const float c0 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(x0, st0) + zp0), 0.f), 15.f);
            const float c1 = fminf(fmaxf(__builtin_rintf(__fdiv_rn(x1, st1) + zp1), 0.f), 15.f);
            s_codes[j * 64 + t] = (uint8_t)((uint32_t)c0 | ((uint32_t)c1 << 4));
        }
        __builtin_amdgcn_wave_barrier();
        for (int k = t; k < nj * 4; k += 64)
            *reinterpret_cast<uint4*>(pbase + (32 * c) * 64 + k * 16) = *reinterpret_cast<const uint4*>(s_codes + k * 16);
        __builtin_amdgcn_wave_barrier();
    }
    const uint16_t h0 = (uint16_t)r2o_f32_to_f16(st0), h1 = (uint16_t)r2o_f32_to_f16(st1);
    s_half[2 * t] = h0;
    s_half[2 * t + 1] = h1;
    s_zero[2 * t] = (uint8_t)zp0;
    s_zero[2 * t + 1] = (uint8_t)zp1;
    __syncthreads();
    uint16_t* srow = scale + (h * superblocks + block_row) * 128 + 2 * t;
    uint8_t* zrow = zero + (h * superblocks + block_row) * 128 + 2 * t;
    srow[0] = h0;
    srow[1] = h1;
    zrow[0] = (uint8_t)zp0;
    zrow[1] = (uint8_t)zp1;
    if (operands) {  // QK MFMA operands of this superblock (layout in r2o_sspa.h)
        const int g = t >> 4, j = (t >> 2) & 3, u = t & 3;
        const int c = 32 * g + 8 * j + u;
        uint32_t* orow = operands + (h * superblocks + block_row) * 128 + g * 32 + 4 * j + u;
        if (u & 1) {  // channel pair read in place 4 bits up: code enters as 1024 + 16 c
            orow[0] = r2o_f32_to_f16(r2o_f16_to_f32(s_half[c]) * 0.0625f) |
                      (r2o_f32_to_f16(r2o_f16_to_f32(s_half[c + 4]) * 0.0625f) << 16);
            orow[16] = (0xE400u | ((uint32_t)s_zero[c] << 4)) | ((0xE400u | ((uint32_t)s_zero[c + 4] << 4)) << 16);
        } else {
            orow[0] = (uint32_t)s_half[c] | ((uint32_t)s_half[c + 4] << 16);
            orow[16] = (0xE400u | s_zero[c]) | ((0xE400u | (uint32_t)s_zero[c + 4]) << 16);
        }
    }
}

// ----------------------------------------------------------------------------- INT2 keys
// OScaR per-channel affine INT2 over superblocks (int2_reference.py:159-214, clip ratio 1):
// block min/max without 0, scale = range / 3, inv = (1 / range) * 3 (torch's ``3.0 / t``),
// zero = rne(-min * inv), offset = -zero * scale; constant channels keep scale 0 and offset = min.
// grid (superblocks to write, hkv), block 64: threads 0..31 quantise channels 4t..4t+3 (byte t
// of the 32-byte row); then all 64 write the QK MFMA operand pairs of the superblock.
__global__ __launch_bounds__(64) void pack_int2_k_kernel(
    const uint16_t* __restrict__ src, int dtype, int64_t src_tokens, const int64_t* __restrict__ index,
    int64_t n, int64_t tail, int64_t dst_start, uint8_t* packed, uint16_t* scale, uint16_t* offset,
    uint32_t* operands, int64_t capacity, int64_t superblocks, int sb) {
    __shared__ uint16_t s_half[128];
    __shared__ uint16_t s_off[128];
    const int t = threadIdx.x;
    const int64_t h = blockIdx.y;
    const int64_t total = tail + n;
    const int64_t first = (int64_t)blockIdx.x * sb;  // relative to dst_start
    const int64_t count = min((int64_t)sb, total - first);
    if (count <= 0) return;
    const int64_t block_row = dst_start / sb + blockIdx.x;
    if (t < 32) {
        uint8_t* prow = packed + (h * capacity + dst_start + first) * 32 + t;
        uint16_t* srow = scale + (h * superblocks + block_row) * 128 + 4 * t;
        uint16_t* orow = offset + (h * superblocks + block_row) * 128 + 4 * t;
        // old metadata of the tail superblock (only block 0 can hold tail positions)
        float os[4], oo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            os[i] = r2o_f16_to_f32(srow[i]);
            oo[i] = r2o_f16_to_f32(orow[i]);
        }
        auto value = [&](int64_t j, float (&x)[4]) {
            const int64_t pos = first + j;
            if (pos < tail) {  // dequantise-then-round the partial tail (compact_int2_key.py:114-121)
                const uint32_t b = prow[j * 32];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    x[i] = r2o_round_dtype(__fadd_rn(__fmul_rn((float)((b >> (2 * i)) & 3u), os[i]), oo[i]), dtype);
            } else {
                const int64_t i0 = pos - tail;
                const int64_t row = index ? index[i0] : i0;
                const uint2 q = *reinterpret_cast<const uint2*>(src + (h * src_tokens + row) * 128 + 4 * t);
                const uint32_t w[4] = {q.x & 0xffffu, q.x >> 16, q.y & 0xffffu, q.y >> 16};
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = dtype == 0 ? r2o_bf16_to_f32(w[i]) : r2o_f16_to_f32(w[i]);
            }
        };
        float mn[4], mx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mn[i] = INFINITY;
            mx[i] = -INFINITY;
        }
        for (int64_t j = 0; j < count; ++j) {
            float x[4];
            value(j, x);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mn[i] = fminf(mn[i], x[i]);
                mx[i] = fmaxf(mx[i], x[i]);
            }
        }
        float sc[4], inv[4], zp[4], off[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float rng = __fsub_rn(mx[i], mn[i]);
            const bool nonconst = rng > 0.f;
            sc[i] = nonconst ? __fdiv_rn(rng, 3.0f) : 0.f;
            inv[i] = nonconst ? __fmul_rn(__fdiv_rn(1.0f, fmaxf(rng, 1e-30f)), 3.0f) : 0.f;
            zp[i] = nonconst ? __builtin_rintf(__fmul_rn(-mn[i], inv[i])) : 0.f;
            off[i] = nonconst ? __fmul_rn(-zp[i], sc[i]) : mn[i];
        }
        for (int64_t j = 0; j < count; ++j) {
            float x[4];
            value(j, x);  // reads the old tail code before this thread overwrites it
            uint32_t byte = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float c = fminf(fmaxf(__builtin_rintf(__fadd_rn(__fmul_rn(x[i], inv[i]), zp[i])), 0.f), 3.f);
                byte |= (uint32_t)c << (2 * i);
            }
            prow[j * 32] = (uint8_t)byte;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t hs = (uint16_t)r2o_f32_to_f16(sc[i]), ho = (uint16_t)r2o_f32_to_f16(off[i]);
            srow[i] = hs;
            orow[i] = ho;
            s_half[4 * t + i] = hs;
            s_off[4 * t + i] = ho;
        }
    }
    if (operands) {  // QK MFMA operands of this superblock (layout in r2o_sspa.h)
        __syncthreads();
        const int g = t >> 4, j = (t >> 2) & 3, u = t & 3;
        const int c = 32 * g + 16 * (j >> 1) + 4 * (j & 1) + u;  // pair (c, c + 8)
        const float k = u == 0 ? 1.f : (u == 1 ? 0.25f : (u == 2 ? 0.0625f : 0.015625f));  // crumb u enters x 4^u
        uint32_t* orow = operands + (h * superblocks + block_row) * 128 + g * 32 + 4 * j + u;
        orow[0] = r2o_f32_to_f16(r2o_f16_to_f32(s_half[c]) * k) | (r2o_f32_to_f16(r2o_f16_to_f32(s_half[c + 8]) * k) << 16);
        orow[16] = (uint32_t)s_off[c] | ((uint32_t)s_off[c + 8] << 16);
    }
}

// ---------------------------------------------------------------------------- INT4 values
// One wave per token row (thread t owns channels 2t, 2t+1); each wave of a 256-thread block takes
// kVRows consecutive rows and issues all their loads first.  grid (ceil(n / (4 kVRows)), hkv).
constexpr int kVRows = 8;

__global__ __launch_bounds__(256) void pack_int4_v_kernel(
    const uint16_t* __restrict__ src, int dtype, int64_t src_tokens, const int64_t* __restrict__ index,
    int64_t n, int64_t dst_start, uint8_t* packed, float* scale, int64_t capacity) {
    const int t = threadIdx.x & 63;
    const int64_t h = blockIdx.y;
    const int64_t i0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kVRows;
    // every load first: the rows' indices (clamped to the last row, branch-free), then the rows
    int64_t rows[kVRows];
#pragma unroll
    for (int r = 0; r < kVRows; ++r) {
        const int64_t i = min(i0 + r, n - 1);
        rows[r] = index ? index[i] : i;
    }
    uint32_t pair[kVRows];
#pragma unroll
    for (int r = 0; r < kVRows; ++r)
        pair[r] = *reinterpret_cast<const uint32_t*>(src + (h * src_tokens + rows[r]) * 128 + 2 * t);
#pragma unroll
    for (int r = 0; r < kVRows; ++r) {
        const int64_t i = i0 + r;
        if (i >= n) break;
        const float x0 = dtype == 0 ? r2o_bf16_to_f32(pair[r] & 0xffffu) : r2o_f16_to_f32(pair[r] & 0xffffu);
        const float x1 = dtype == 0 ? r2o_bf16_to_f32(pair[r] >> 16) : r2o_f16_to_f32(pair[r] >> 16);
        const float amax = r2o_wave_max(fmaxf(fabsf(x0), fabsf(x1)));
        const float s = fmaxf(__fdiv_rn(amax, 7.0f), kEps);
        const int q0 = (int)fminf(fmaxf(__builtin_rintf(__fdiv_rn(x0, s)), -7.f), 7.f);
        const int q1 = (int)fminf(fmaxf(__builtin_rintf(__fdiv_rn(x1, s)), -7.f), 7.f);
        const int64_t dst = h * capacity + dst_start + i;
        packed[dst * 64 + t] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
        if (t == 0) scale[dst] = s;
    }
}

// ---------------------------------------------------------------------------- INT2 values
// One wave per token row as for INT4 values (thread t owns channels 2t, 2t+1; a group of G
// channels is G/2 consecutive threads), kVRows rows per wave with all loads issued first.
__device__ __forceinline__ void int2_value_row(uint32_t pair, int t, int dtype, int group, int64_t dst,
                                               uint8_t* packed, uint16_t* scale, uint8_t* zero) {
    const float x0 = dtype == 0 ? r2o_bf16_to_f32(pair & 0xffffu) : r2o_f16_to_f32(pair & 0xffffu);
    const float x1 = dtype == 0 ? r2o_bf16_to_f32(pair >> 16) : r2o_f16_to_f32(pair >> 16);
    float mn = fminf(x0, x1), mx = fmaxf(x0, x1);
    for (int o = 1; o < group / 2; o <<= 1) {
        mn = fminf(mn, __shfl_xor(mn, o, R2O_WAVE));
        mx = fmaxf(mx, __shfl_xor(mx, o, R2O_WAVE));
    }
    mn = fminf(mn, 0.f);
    mx = fmaxf(mx, 0.f);
    const float s = fmaxf(__fdiv_rn(mx - mn, 3.0f), kEps);
    const float z = fminf(fmaxf(__builtin_rintf(__fdiv_rn(-mn, s)), 0.f), 3.f);
    const uint32_t c0 = (uint32_t)fminf(fmaxf(__builtin_rintf(__fdiv_rn(x0, s) + z), 0.f), 3.f);
    const uint32_t c1 = (uint32_t)fminf(fmaxf(__builtin_rintf(__fdiv_rn(x1, s) + z), 0.f), 3.f);
    const uint32_t mine = c0 | (c1 << 2);
    const uint32_t next = (uint32_t)__shfl_down((int)mine, 1, R2O_WAVE);
    if ((t & 1) == 0) packed[dst * 32 + t / 2] = (uint8_t)(mine | (next << 4));
    const int groups = 128 / group;
    if (t % (group / 2) == 0) {
        const int gi = t / (group / 2);
        scale[dst * groups + gi] = (uint16_t)r2o_f32_to_f16(s);
        zero[dst * groups + gi] = (uint8_t)z;
    }
}

__global__ __launch_bounds__(256) void pack_int2_v_kernel(
    const uint16_t* __restrict__ src, int dtype, int64_t src_tokens, const int64_t* __restrict__ index,
    int64_t n, int64_t dst_start, int group, uint8_t* packed, uint16_t* scale, uint8_t* zero, int64_t capacity) {
    const int t = threadIdx.x & 63;
    const int64_t h = blockIdx.y;
    const int64_t i0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kVRows;
    // every load first: the rows' indices (clamped to the last row, branch-free), then the rows
    int64_t rows[kVRows];
#pragma unroll
    for (int r = 0; r < kVRows; ++r) {
        const int64_t i = min(i0 + r, n - 1);
        rows[r] = index ? index[i] : i;
    }
    uint32_t pair[kVRows];
#pragma unroll
    for (int r = 0; r < kVRows; ++r)
        pair[r] = *reinterpret_cast<const uint32_t*>(src + (h * src_tokens + rows[r]) * 128 + 2 * t);
#pragma unroll
    for (int r = 0; r < kVRows; ++r) {
        const int64_t i = i0 + r;
        if (i >= n) break;
        int2_value_row(pair[r], t, dtype, group, h * capacity + dst_start + i, packed, scale, zero);
    }
}

// ---------------------------------------------------------------------------- gather rows
// 64 rows per 256-thread block: thread t moves 16-byte chunk t % 16 of rows t / 16 + 16 k, all
// loads first.  grid (ceil(n / 64), hkv).
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint16_t* __restrict__ src, int64_t src_tokens,
                                                          const int64_t* __restrict__ index, int64_t n,
                                                          uint16_t* dst, int64_t dst_stride) {
    const int64_t h = blockIdx.y;
    const int c = threadIdx.x & 15;
    const int64_t i0 = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 4);
    int64_t rows[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // indices first (clamped to the last row, branch-free), then the rows
        const int64_t i = min(i0 + 16 * k, n - 1);
        rows[k] = index ? index[i] : i;
    }
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = *reinterpret_cast<const uint4*>(src + (h * src_tokens + rows[k]) * 128 + 8 * c);
#pragma unroll
    for (int k = 0; k < 4; ++k)  // keeps the four loads together (not sunk into the guarded stores)
        asm volatile("" ::"v"(v[k].x), "v"(v[k].y), "v"(v[k].z), "v"(v[k].w));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = i0 + 16 * k;
        if (i < n) *reinterpret_cast<uint4*>(dst + (h * dst_stride + i) * 128 + 8 * c) = v[k];
    }
}

// ------------------------------------------------------------------------ Recent-FP ring
__global__ __launch_bounds__(256) void recent_append_kernel(
    uint16_t* rk, uint16_t* rv, int64_t hkv, int64_t capacity, const uint16_t* __restrict__ nk,
    const uint16_t* __restrict__ nv, int64_t pos, int64_t gidx, int64_t lpos, int32_t* length,
    int64_t* gbuf, int64_t* lbuf, int64_t* page_lengths, int64_t page_size) {
    for (int64_t e = threadIdx.x; e < hkv * 128; e += blockDim.x) {
        const int64_t h = e / 128, d = e % 128;
        rk[(h * capacity + pos) * 128 + d] = nk[e];
        rv[(h * capacity + pos) * 128 + d] = nv[e];
    }
    if (threadIdx.x == 0) {
        gbuf[pos] = gidx;
        lbuf[pos] = lpos;
        *length = (int32_t)(pos + 1);
        page_lengths[pos / page_size] = pos % page_size + 1;
    }
}

// Single block: moves slots [flush, active) down by `flush` in rounds of at most `flush` rows
// so that no round reads a slot another round writes.
__global__ __launch_bounds__(256) void recent_shift_kernel(
    uint16_t* rk, uint16_t* rv, int64_t hkv, int64_t capacity, int64_t flush, int64_t active,
    int64_t* gbuf, int64_t* lbuf, int32_t* length, int64_t* page_lengths, int64_t page_size) {
    const int64_t remaining = active - flush;
    for (int64_t base = 0; base < remaining; base += flush) {
        const int64_t rows = min(flush, remaining - base);
        for (int64_t e = threadIdx.x; e < hkv * rows * 128; e += blockDim.x) {
            const int64_t h = e / (rows * 128), r = (e / 128) % rows, d = e % 128;
            const int64_t dst = (h * capacity + base + r) * 128 + d;
            const int64_t srcp = (h * capacity + base + r + flush) * 128 + d;
            rk[dst] = rk[srcp];
            rv[dst] = rv[srcp];
        }
        for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
            gbuf[base + r] = gbuf[base + r + flush];
            lbuf[base + r] = lbuf[base + r + flush];
        }
        __syncthreads();
    }
    const int64_t new_active = remaining > 0 ? remaining : 0;
    for (int64_t p = threadIdx.x; p < capacity / page_size; p += blockDim.x) {
        const int64_t v = new_active - p * page_size;
        page_lengths[p] = v < 0 ? 0 : (v > page_size ? page_size : v);
    }
    if (threadIdx.x == 0) *length = (int32_t)new_active;
}

// ---------------------------------------------------------------------------------- FWHT
// One 128-thread block per row; butterflies in the reference's stage order (stride 1 .. 64),
// then the fp32 normalisation 0.08838834764831845.
__global__ __launch_bounds__(128) void fwht128_kernel(const uint16_t* __restrict__ src, uint16_t* dst, int dtype) {
    __shared__ float buf[128];
    const int64_t row = blockIdx.x;
    const int d = threadIdx.x;
    buf[d] = r2o_load_elem(src, row * 128 + d, dtype);
    __syncthreads();
    for (int stride = 1; stride < 128; stride <<= 1) {
        const int pos = d & (stride - 1);
        const int base = (d / stride) * stride * 2;  // only the first 64 threads are used
        float a = 0.f, b = 0.f;
        if (d < 64) {
            const int blk = d / stride;
            const int i0 = blk * 2 * stride + pos;
            a = buf[i0];
            b = buf[i0 + stride];
        }
        __syncthreads();
        if (d < 64) {
            const int blk = d / stride;
            const int i0 = blk * 2 * stride + pos;
            buf[i0] = a + b;
            buf[i0 + stride] = a - b;
        }
        (void)base;
        __syncthreads();
    }
    const float y = buf[d] * 0.08838834764831845f;
    dst[row * 128 + d] = (uint16_t)(dtype == 0 ? r2o_f32_to_bf16(y) : r2o_f32_to_f16(y));
}

}  // namespace

extern "C" {

int r2o_pack_int4_k(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens, const int64_t* index,
                    int64_t n, int64_t tail, int64_t dst_start, uint8_t* packed, uint16_t* scale, uint8_t* zero,
                    uint32_t* operands, int64_t capacity, int64_t superblocks, int64_t superblock, void* stream) {
    if (!(superblock == 32 || superblock == 64 || superblock == 128) || (dtype != 0 && dtype != 1)) return R2O_EINVAL;
    if (hkv <= 0 || n < 0 || tail < 0 || tail >= superblock || dst_start < 0 || dst_start % superblock) return R2O_EINVAL;
    if (dst_start + tail + n > capacity || capacity % superblock || superblocks * superblock != capacity) return R2O_EINVAL;
    if (n > 0 && (!src || src_tokens <= 0)) return R2O_EINVAL;
    const int64_t total = tail + n;
    if (total == 0) return R2O_OK;
    const int64_t blocks = (total + superblock - 1) / superblock;
    if (tail == 0 && src_tokens <= 0x7fffffff) {  // whole superblocks: the register-resident packer
        const dim3 grid((unsigned)blocks, (unsigned)hkv);
        if (superblock == 32)
            hipLaunchKernelGGL(pack_int4_k_full_kernel<32>, grid, dim3(64), 0, (hipStream_t)stream, src, (int)dtype,
                               src_tokens, index, n, dst_start, packed, scale, zero, operands, capacity, superblocks);
        else if (superblock == 64)
            hipLaunchKernelGGL(pack_int4_k_full_kernel<64>, grid, dim3(64), 0, (hipStream_t)stream, src, (int)dtype,
                               src_tokens, index, n, dst_start, packed, scale, zero, operands, capacity, superblocks);
        else
            hipLaunchKernelGGL(pack_int4_k_full_kernel<128>, grid, dim3(64), 0, (hipStream_t)stream, src, (int)dtype,
                               src_tokens, index, n, dst_start, packed, scale, zero, operands, capacity, superblocks);
    } else {
        hipLaunchKernelGGL(pack_int4_k_kernel, dim3((unsigned)blocks, (unsigned)hkv), dim3(64), 0, (hipStream_t)stream,
                           src, (int)dtype, src_tokens, index, n, tail, dst_start, packed, scale, zero, operands,
                           capacity, superblocks, (int)superblock);
    }
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_pack_int2_k(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens, const int64_t* index,
                    int64_t n, int64_t tail, int64_t dst_start, uint8_t* packed, uint16_t* scale, uint16_t* offset,
                    uint32_t* operands, int64_t capacity, int64_t superblocks, int64_t superblock, void* stream) {
    if (!(superblock == 32 || superblock == 64 || superblock == 128) || (dtype != 0 && dtype != 1)) return R2O_EINVAL;
    if (hkv <= 0 || n < 0 || tail < 0 || tail >= superblock || dst_start < 0 || dst_start % superblock) return R2O_EINVAL;
    if (dst_start + tail + n > capacity || capacity % superblock || superblocks * superblock != capacity) return R2O_EINVAL;
    if (n > 0 && (!src || src_tokens <= 0)) return R2O_EINVAL;
    const int64_t total = tail + n;
    if (total == 0) return R2O_OK;
    const int64_t blocks = (total + superblock - 1) / superblock;
    hipLaunchKernelGGL(pack_int2_k_kernel, dim3((unsigned)blocks, (unsigned)hkv), dim3(64), 0, (hipStream_t)stream,
                       src, (int)dtype, src_tokens, index, n, tail, dst_start, packed, scale, offset, operands,
                       capacity, superblocks, (int)superblock);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_pack_int4_v(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens, const int64_t* index,
                    int64_t n, int64_t dst_start, uint8_t* packed, float* scale, int64_t capacity, void* stream) {
    if ((dtype != 0 && dtype != 1) || hkv <= 0 || n < 0 || dst_start < 0 || dst_start + n > capacity) return R2O_EINVAL;
    if (n == 0) return R2O_OK;
    if (!src || src_tokens <= 0 || n > 0x7fffffff || (!index && n > src_tokens)) return R2O_EINVAL;
    hipLaunchKernelGGL(pack_int4_v_kernel, dim3((unsigned)((n + 4 * kVRows - 1) / (4 * kVRows)), (unsigned)hkv), dim3(256),
                       0, (hipStream_t)stream, src, (int)dtype, src_tokens, index, n, dst_start, packed, scale, capacity);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_pack_int2_v(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens, const int64_t* index,
                    int64_t n, int64_t dst_start, int64_t group, uint8_t* packed, uint16_t* scale, uint8_t* zero,
                    int64_t capacity, void* stream) {
    if ((dtype != 0 && dtype != 1) || !(group == 32 || group == 64 || group == 128)) return R2O_EINVAL;
    if (hkv <= 0 || n < 0 || dst_start < 0 || dst_start + n > capacity) return R2O_EINVAL;
    if (n == 0) return R2O_OK;
    if (!src || src_tokens <= 0 || n > 0x7fffffff || (!index && n > src_tokens)) return R2O_EINVAL;
    hipLaunchKernelGGL(pack_int2_v_kernel, dim3((unsigned)((n + 4 * kVRows - 1) / (4 * kVRows)), (unsigned)hkv), dim3(256),
                       0, (hipStream_t)stream, src, (int)dtype, src_tokens, index, n, dst_start, (int)group, packed, scale,
                       zero, capacity);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_gather_rows(const uint16_t* src, int64_t hkv, int64_t src_tokens, const int64_t* index, int64_t n,
                    uint16_t* dst, int64_t dst_stride, void* stream) {
    if (hkv <= 0 || n < 0 || n > dst_stride || n > 0x7fffffff) return R2O_EINVAL;
    if (n == 0) return R2O_OK;
    if (!src || !dst) return R2O_EINVAL;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)hkv), dim3(256), 0,
                       (hipStream_t)stream, src, src_tokens, index, n, dst, dst_stride);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_recent_append(uint16_t* recent_k, uint16_t* recent_v, int64_t hkv, int64_t capacity, const uint16_t* new_k,
                      const uint16_t* new_v, int64_t position, int64_t global_index, int64_t logical_position,
                      int32_t* length, int64_t* global_buf, int64_t* logical_buf, int64_t* page_lengths,
                      int64_t page_size, void* stream) {
    if (hkv <= 0 || position < 0 || position >= capacity || page_size <= 0 || capacity % page_size) return R2O_EINVAL;
    if (!recent_k || !recent_v || !new_k || !new_v || !length || !global_buf || !logical_buf || !page_lengths)
        return R2O_EINVAL;
    hipLaunchKernelGGL(recent_append_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, recent_k, recent_v, hkv,
                       capacity, new_k, new_v, position, global_index, logical_position, length, global_buf,
                       logical_buf, page_lengths, page_size);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_recent_shift(uint16_t* recent_k, uint16_t* recent_v, int64_t hkv, int64_t capacity, int64_t flush,
                     int64_t active, int64_t* global_buf, int64_t* logical_buf, int32_t* length,
                     int64_t* page_lengths, int64_t page_size, void* stream) {
    if (hkv <= 0 || flush <= 0 || active < flush || active > capacity || page_size <= 0 || capacity % page_size)
        return R2O_EINVAL;
    hipLaunchKernelGGL(recent_shift_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, recent_k, recent_v, hkv,
                       capacity, flush, active, global_buf, logical_buf, length, page_lengths, page_size);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_fwht128(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t dtype, void* stream) {
    if (rows < 0 || rows > 0x7fffffff || (dtype != 0 && dtype != 1)) return R2O_EINVAL;
    if (rows == 0) return R2O_OK;
    hipLaunchKernelGGL(fwht128_kernel, dim3((unsigned)rows), dim3(128), 0, (hipStream_t)stream, src, dst, (int)dtype);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

const char* r2o_build_target(void) { return "gfx950"; }

}  // extern "C"
