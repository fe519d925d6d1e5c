// Decode-step query/key rotation for gfx950: Qwen multimodal rotary embedding (mRoPE) with an
// optional orthonormal FWHT-128, one wave per (request, head, token) row.  Lane t holds the
// rotate-half pair (d = t, d = t + 64), so both halves of the rotation and the stride-64
// butterfly of the FWHT stay inside the lane.
//
// Semantics follow _qwen_qk_mrope_kernel / _qwen_batched_qk_mrope_kernel
// (triton_qwen_mrope.py:45-211): x * cos + rotate_half(x) * sin in fp32, where dimension d takes
// its cos/sin from axis 0, 1 or 2 of the [3, B, S, 128] tables by its position d % 64 within the
// mRoPE sections, then the optional FWHT, then one rounding to the input dtype.
//
// The Qwen3 branch of the same decode step (qwen_sspa_attention.py:1228-1235: q_norm / k_norm,
// apply_rotary_pos_emb, then triton_fwht_128 when keys are Hadamard-rotated) runs as one launch
// of qk_norm_rope_kernel, reproducing the rounding of every torch op of that sequence.
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
    const uint16_t* v;  // nullable: V rows take the FWHT alone
    uint16_t* q_out;
    uint16_t* k_out;
    uint16_t* v_out;
    const void* cos;
    const void* sin;
    int64_t cs[4];  // cos strides (axis, batch, token, dim) in elements
    int64_t ss[4];  // sin strides
    int64_t hq, hkv, hv, tokens, rows;  // hv: V heads (hkv with V rows, else 0)
    int dtype, table_code, s0, s1, hadamard;
};

__global__ __launch_bounds__(256) void qk_mrope_kernel(RopeArgs a) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // whole-wave exit: the FWHT's cross-lane butterflies need every lane of a live wave
    const int t = threadIdx.x & 63;
    const int64_t per_req = (a.hq + a.hkv + a.hv) * a.tokens;
    const int64_t b = row / per_req, local = row % per_req;
    const int64_t head = local / a.tokens, token = local % a.tokens;
    const bool is_q = head < a.hq, is_v = head >= a.hq + a.hkv;
    const int64_t kv_head = is_v ? head - a.hq - a.hkv : head - a.hq;
    const int64_t off = is_q ? ((b * a.hq + head) * a.tokens + token) * 128 : ((b * a.hkv + kv_head) * a.tokens + token) * 128;
    const uint16_t* src = is_q ? a.q : (is_v ? a.v : a.k);
    uint16_t* dst = is_q ? a.q_out : (is_v ? a.v_out : a.k_out);
    const float x0 = a.dtype == 0 ? r2o_bf16_to_f32(src[off + t]) : r2o_f16_to_f32(src[off + t]);
    const float x1 = a.dtype == 0 ? r2o_bf16_to_f32(src[off + t + 64]) : r2o_f16_to_f32(src[off + t + 64]);
    if (is_v) {  // wave-uniform: a V row is the FWHT of the row alone (triton_fwht_128)
        float y0 = x0, y1 = x1;
        r2o_fwht128_pair(y0, y1, t);
        dst[off + t] = (uint16_t)(a.dtype == 0 ? r2o_f32_to_bf16(y0) : r2o_f32_to_f16(y0));
        dst[off + t + 64] = (uint16_t)(a.dtype == 0 ? r2o_f32_to_bf16(y1) : r2o_f32_to_f16(y1));
        return;
    }
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


// Round to the tensor dtype (0 = bf16, 1 = fp16) and back: the result of one torch op.
__device__ __forceinline__ float round_to(float x, int dtype) {
    return dtype == 0 ? r2o_bf16_to_f32(r2o_f32_to_bf16(x)) : r2o_f16_to_f32(r2o_f32_to_f16(x));
}

__device__ __forceinline__ float load_elem(const uint16_t* p, int64_t i, int dtype) {
    return dtype == 0 ? r2o_bf16_to_f32(p[i]) : r2o_f16_to_f32(p[i]);
}

struct NormRopeArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;  // nullable: V rows take the FWHT alone
    uint16_t* q_out;
    uint16_t* k_out;
    uint16_t* v_out;
    const uint16_t* q_weight;  // [128] RMSNorm weights, input dtype
    const uint16_t* k_weight;
    const uint16_t* cos;       // input dtype, strides (batch, token, dim) in elements
    const uint16_t* sin;
    int64_t cs[3];
    int64_t ss[3];
    int64_t hq, hkv, hv, tokens, rows;  // hv: V heads (hkv with V rows, else 0)
    float eps;
    int dtype, hadamard;
};

// One wave per (request, head, token) row; lane t holds dims t and t + 64.
//   Qwen3RMSNorm (transformers 5.15.0 modeling_qwen3.py): v = mean(x^2) in fp32, n = dtype(x * rsqrt(v +
//   eps)) with rsqrt evaluated as 1 / sqrt (both correctly rounded, as torch's CPU kernel), then
//   w = dtype(weight * n);
//   apply_rotary_pos_emb: y = dtype(dtype(w * cos) + dtype(rotate_half(w) * sin)), rotate_half(w) =
//   (-w[d + 64], w[d - 64]);
//   optional FWHT-128 of y in fp32 (triton_fwht_128), rounded to dtype.
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(NormRopeArgs a) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;  // whole-wave exit: the cross-lane sums and butterflies need every lane of a live wave
    const int t = threadIdx.x & 63;
    const int64_t per_req = (a.hq + a.hkv + a.hv) * a.tokens;
    const int64_t b = row / per_req, local = row % per_req;
    const int64_t head = local / a.tokens, token = local % a.tokens;
    const bool is_q = head < a.hq, is_v = head >= a.hq + a.hkv;
    const int64_t kv_head = is_v ? head - a.hq - a.hkv : head - a.hq;
    const int64_t off = is_q ? ((b * a.hq + head) * a.tokens + token) * 128 : ((b * a.hkv + kv_head) * a.tokens + token) * 128;
    const uint16_t* src = is_q ? a.q : (is_v ? a.v : a.k);
    const uint16_t* wt = is_q ? a.q_weight : a.k_weight;
    uint16_t* dst = is_q ? a.q_out : (is_v ? a.v_out : a.k_out);
    const int dt = a.dtype;
    const float x0 = load_elem(src, off + t, dt), x1 = load_elem(src, off + t + 64, dt);
    if (is_v) {  // wave-uniform: a V row is the FWHT of the row alone (triton_fwht_128)
        float y0 = x0, y1 = x1;
        r2o_fwht128_pair(y0, y1, t);
        dst[off + t] = (uint16_t)(dt == 0 ? r2o_f32_to_bf16(y0) : r2o_f32_to_f16(y0));
        dst[off + t + 64] = (uint16_t)(dt == 0 ? r2o_f32_to_bf16(y1) : r2o_f32_to_f16(y1));
        return;
    }
    float sq = __fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sq = __fadd_rn(sq, __shfl_xor(sq, m, R2O_WAVE));
    const float var = __fdiv_rn(sq, 128.f);
    const float inv = __fdiv_rn(1.f, __fsqrt_rn(__fadd_rn(var, a.eps)));
    const float w0 = round_to(__fmul_rn(load_elem(wt, t, dt), round_to(__fmul_rn(x0, inv), dt)), dt);
    const float w1 = round_to(__fmul_rn(load_elem(wt, t + 64, dt), round_to(__fmul_rn(x1, inv), dt)), dt);
    const int64_t c = b * a.cs[0] + token * a.cs[1], sn = b * a.ss[0] + token * a.ss[1];
    const float cos0 = load_elem(a.cos, c + t * a.cs[2], dt), cos1 = load_elem(a.cos, c + (t + 64) * a.cs[2], dt);
    const float sin0 = load_elem(a.sin, sn + t * a.ss[2], dt), sin1 = load_elem(a.sin, sn + (t + 64) * a.ss[2], dt);
    float y0 = round_to(__fadd_rn(round_to(__fmul_rn(w0, cos0), dt), round_to(__fmul_rn(-w1, sin0), dt)), dt);
    float y1 = round_to(__fadd_rn(round_to(__fmul_rn(w1, cos1), dt), round_to(__fmul_rn(w0, sin1), dt)), dt);
    if (a.hadamard) r2o_fwht128_pair(y0, y1, t);
    dst[off + t] = (uint16_t)(dt == 0 ? r2o_f32_to_bf16(y0) : r2o_f32_to_f16(y0));
    dst[off + t + 64] = (uint16_t)(dt == 0 ? r2o_f32_to_bf16(y1) : r2o_f32_to_f16(y1));
}

}  // namespace

extern "C" {

int r2o_qkv_mrope(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* q_out, uint16_t* k_out,
                  uint16_t* v_out, int64_t dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t tokens,
                  const void* cos, const void* sin, int64_t table_dtype, const int64_t* cos_strides,
                  const int64_t* sin_strides, int64_t section0, int64_t section1, int64_t apply_hadamard,
                  void* stream) {
    if (!q || !k || !q_out || !k_out || !cos || !sin || !cos_strides || !sin_strides) return R2O_EINVAL;
    if ((v == nullptr) != (v_out == nullptr)) return R2O_EINVAL;
    if ((dtype != 0 && dtype != 1) || table_dtype < 0 || table_dtype > 2) return R2O_EINVAL;
    if (batch <= 0 || hq <= 0 || hkv <= 0 || tokens <= 0) return R2O_EINVAL;
    if (section0 < 0 || section1 < 0 || section0 + section1 > 64) return R2O_EINVAL;
    RopeArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_out = v_out;
    a.cos = cos;
    a.sin = sin;
    for (int i = 0; i < 4; ++i) {
        a.cs[i] = cos_strides[i];
        a.ss[i] = sin_strides[i];
    }
    a.hq = hq;
    a.hkv = hkv;
    a.hv = v ? hkv : 0;
    a.tokens = tokens;
    a.rows = batch * (hq + hkv + a.hv) * tokens;
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

int r2o_qk_mrope(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out, int64_t dtype, int64_t batch,
                 int64_t hq, int64_t hkv, int64_t tokens, const void* cos, const void* sin, int64_t table_dtype,
                 const int64_t* cos_strides, const int64_t* sin_strides, int64_t section0, int64_t section1,
                 int64_t apply_hadamard, void* stream) {
    return r2o_qkv_mrope(q, k, nullptr, q_out, k_out, nullptr, dtype, batch, hq, hkv, tokens, cos, sin, table_dtype,
                         cos_strides, sin_strides, section0, section1, apply_hadamard, stream);
}

int r2o_qkv_norm_rope(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* q_out, uint16_t* k_out,
                      uint16_t* v_out, int64_t dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t tokens,
                      const uint16_t* q_weight, const uint16_t* k_weight, float eps, const uint16_t* cos,
                      const uint16_t* sin, const int64_t* cos_strides, const int64_t* sin_strides,
                      int64_t apply_hadamard, void* stream) {
    if (!q || !k || !q_out || !k_out || !q_weight || !k_weight || !cos || !sin || !cos_strides || !sin_strides)
        return R2O_EINVAL;
    if ((v == nullptr) != (v_out == nullptr)) return R2O_EINVAL;
    if ((dtype != 0 && dtype != 1) || batch <= 0 || hq <= 0 || hkv <= 0 || tokens <= 0) return R2O_EINVAL;
    if (!(eps >= 0.f)) return R2O_EINVAL;
    NormRopeArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_out = v_out;
    a.q_weight = q_weight;
    a.k_weight = k_weight;
    a.cos = cos;
    a.sin = sin;
    for (int i = 0; i < 3; ++i) {
        a.cs[i] = cos_strides[i];
        a.ss[i] = sin_strides[i];
    }
    a.hq = hq;
    a.hkv = hkv;
    a.hv = v ? hkv : 0;
    a.tokens = tokens;
    a.rows = batch * (hq + hkv + a.hv) * tokens;
    a.eps = eps;
    a.dtype = (int)dtype;
    a.hadamard = apply_hadamard ? 1 : 0;
    if ((a.rows + 3) / 4 > 0x7fffffff) return R2O_EINVAL;
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)((a.rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_qk_norm_rope(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out, int64_t dtype,
                     int64_t batch, int64_t hq, int64_t hkv, int64_t tokens, const uint16_t* q_weight,
                     const uint16_t* k_weight, float eps, const uint16_t* cos, const uint16_t* sin,
                     const int64_t* cos_strides, const int64_t* sin_strides, int64_t apply_hadamard, void* stream) {
    return r2o_qkv_norm_rope(q, k, nullptr, q_out, k_out, nullptr, dtype, batch, hq, hkv, tokens, q_weight, k_weight,
                             eps, cos, sin, cos_strides, sin_strides, apply_hadamard, stream);
}

}  // extern "C"
