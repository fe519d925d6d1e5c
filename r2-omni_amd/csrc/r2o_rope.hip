// Decode-step query/key rotation for gfx950: Qwen multimodal rotary embedding (mRoPE) with an
// optional orthonormal FWHT-128, one wave per (request, head, token) row.  Lane t holds the
// rotate-half pair (d = t, d = t + 64), so both halves of the rotation and the stride-64
// butterfly of the FWHT stay inside the lane.
//
// Semantics follow _qwen_qk_mrope_kernel / _qwen_batched_qk_mrope_kernel
// (triton_qwen_mrope.py:45-211): x * cos + rotate_half(x) * sin in fp32, where dimension d takes
// its cos/sin from axis 0, 1 or 2 of the [3, B, S, 128] tables by its position d % 64 within the
// mRoPE sections, then the optional FWHT, then one rounding to the input dtype.
#include "r2o_common.hpp"

namespace {

__device__ __forceinline__ float load_table(const void* base, int code, int64_t idx) {
    if (code == 2) return reinterpret_cast<const float*>(base)[idx];
    const uint32_t b = reinterpret_cast<const uint16_t*>(base)[idx];
    return code == 0 ? r2o_bf16_to_f32(b) : r2o_f16_to_f32(b);
}

struct RopeArgs {
    const uint16_t* q;
    const uint16_t* k;
    uint16_t* q_out;
    uint16_t* k_out;
    const void* cos;
    const void* sin;
    int64_t cs[4];  // cos strides (axis, batch, token, dim) in elements
    int64_t ss[4];  // sin strides
    int64_t hq, hkv, tokens, rows;
    int dtype, table_code, s0, s1, hadamard;
};

__global__ __launch_bounds__(256) void qk_mrope_kernel(RopeArgs a) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // whole-wave exit: the FWHT shuffles stay within live waves
    const int t = threadIdx.x & 63;
    const int64_t per_req = (a.hq + a.hkv) * a.tokens;
    const int64_t b = row / per_req, local = row % per_req;
    const int64_t head = local / a.tokens, token = local % a.tokens;
    const bool is_q = head < a.hq;
    const int64_t off = is_q ? ((b * a.hq + head) * a.tokens + token) * 128 : ((b * a.hkv + head - a.hq) * a.tokens + token) * 128;
    const uint16_t* src = is_q ? a.q : a.k;
    uint16_t* dst = is_q ? a.q_out : a.k_out;
    const float x0 = a.dtype == 0 ? r2o_bf16_to_f32(src[off + t]) : r2o_f16_to_f32(src[off + t]);
    const float x1 = a.dtype == 0 ? r2o_bf16_to_f32(src[off + t + 64]) : r2o_f16_to_f32(src[off + t + 64]);
    const int axis = t < a.s0 ? 0 : (t < a.s0 + a.s1 ? 1 : 2);  // section of d % 64 == t
    const int64_t c0 = axis * a.cs[0] + b * a.cs[1] + token * a.cs[2], sn0 = axis * a.ss[0] + b * a.ss[1] + token * a.ss[2];
    const float cos0 = load_table(a.cos, a.table_code, c0 + t * a.cs[3]);
    const float cos1 = load_table(a.cos, a.table_code, c0 + (t + 64) * a.cs[3]);
    const float sin0 = load_table(a.sin, a.table_code, sn0 + t * a.ss[3]);
    const float sin1 = load_table(a.sin, a.table_code, sn0 + (t + 64) * a.ss[3]);
    float y0 = x0 * cos0 + (-x1) * sin0;  // rotate_half: (-x[d + 64], x[d - 64])
    float y1 = x1 * cos1 + x0 * sin1;
    if (a.hadamard) r2o_fwht128_pair(y0, y1, t);
    dst[off + t] = (uint16_t)(a.dtype == 0 ? r2o_f32_to_bf16(y0) : r2o_f32_to_f16(y0));
    dst[off + t + 64] = (uint16_t)(a.dtype == 0 ? r2o_f32_to_bf16(y1) : r2o_f32_to_f16(y1));
}

}  // namespace

extern "C" {

int r2o_qk_mrope(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out, int64_t dtype, int64_t batch,
                 int64_t hq, int64_t hkv, int64_t tokens, const void* cos, const void* sin, int64_t table_dtype,
                 const int64_t* cos_strides, const int64_t* sin_strides, int64_t section0, int64_t section1,
                 int64_t apply_hadamard, void* stream) {
    if (!q || !k || !q_out || !k_out || !cos || !sin || !cos_strides || !sin_strides) return R2O_EINVAL;
    if ((dtype != 0 && dtype != 1) || table_dtype < 0 || table_dtype > 2) return R2O_EINVAL;
    if (batch <= 0 || hq <= 0 || hkv <= 0 || tokens <= 0) return R2O_EINVAL;
    if (section0 < 0 || section1 < 0 || section0 + section1 > 64) return R2O_EINVAL;
    RopeArgs a;
    a.q = q;
    a.k = k;
    a.q_out = q_out;
    a.k_out = k_out;
    a.cos = cos;
    a.sin = sin;
    for (int i = 0; i < 4; ++i) {
        a.cs[i] = cos_strides[i];
        a.ss[i] = sin_strides[i];
    }
    a.hq = hq;
    a.hkv = hkv;
    a.tokens = tokens;
    a.rows = batch * (hq + hkv) * tokens;
    a.dtype = (int)dtype;
    a.table_code = (int)table_dtype;
    a.s0 = (int)section0;
    a.s1 = (int)section1;
    a.hadamard = apply_hadamard ? 1 : 0;
    if ((a.rows + 3) / 4 > 0x7fffffff) return R2O_EINVAL;
    hipLaunchKernelGGL(qk_mrope_kernel, dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

}  // extern "C"
