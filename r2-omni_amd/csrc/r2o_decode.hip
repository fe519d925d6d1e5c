// Split-K GQA decode over the SSPA packed cache for gfx950 (CDNA4, wave64, MFMA 16x16x32).
//
// Partial pass: one 256-thread block (4 waves) per work item, i.e. a run of 32-token tiles of
// one pool segment of one (request, kv head).  Each wave walks its share of the tiles with an
// online softmax in the log2 domain and keeps a 16 x 128 fp32 accumulator (query heads of the
// KV group padded to 16 MFMA rows).  Per tile:
//   QK  S^T[tok, h] = sum_c K[tok, c] * Q'[h, c]  as f16 MFMA on the raw INT4 codes:
//       the A operand is (1024 + code) built with one and-or per two nibbles, the B operand is
//       Q' = q * s (per-channel scale of the tile's K superblock, scaled by D^-1/2 * log2 e),
//       and the C operand starts at -sum_c Q'[h, c] * (1024 + z_c), itself one MFMA per
//       superblock, so the MFMA chain returns q . (code - z) * s exactly as the dequantised dot.
//       Recent-FP tiles use a bf16 MFMA on the bf16 K rows.
//   PV  O[h, d] += sum_tok P[h, tok] V[tok, d]: V rows are staged in LDS in their packed form
//       and read back transposed per lane (8 tokens of 8 adjacent dims) so that the MFMA B
//       operand holds consecutive tokens.  BF16 V: bf16 MFMA.  INT4 V: the per-token scale is
//       folded into P (P' = p * s) and the signed codes enter exactly as f16 ((1032 + c) built
//       with one and-or, minus 1032).  INT2 V: (c - z) * s is formed in f16 per element.
// The 4 waves' states are merged in LDS and one (max, sum, acc[GQA][128]) partial is written.
//
// Combine pass: one 128-thread block per (request, query head) merges the partials of its
// (request, kv head) group, divides, rounds to bf16, optionally applies the 128-point FWHT and
// performs the fused Recent-FP append of the step's K/V row and metadata.
//
// Semantics follow triton_fourq_splitk.py:456-1020 (tile attention, exact state merge, fused
// append :1007-1020, output Hadamard :1000-1006) and the oracle triton_fourq_attention.py:72-125.
#include "r2o_common.hpp"

namespace {

constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kStageBytes = 8192;                   // per wave: 32 rows x 256 B (bf16 V)
constexpr int kRowI4 = 80;                          // padded LDS row stride for INT4 V (64 B)
constexpr int kRowI2 = 48;                          // padded LDS row stride for INT2 V (32 B)
constexpr int kMergeFloats = 16 + 16 + 16 * 128;    // per wave: m, l, acc
constexpr int kSmemBytes = (kWaves * kMergeFloats * 4 > kWaves * kStageBytes) ? kWaves * kMergeFloats * 4
                                                                                : kWaves * kStageBytes;

enum Kind { kFP = 0, kI4 = 1, kI2 = 2, kRecent = 3 };

__device__ __forceinline__ void wave_lds_fence() {
    // LDS traffic of one wave is processed in order; keep the compiler from reordering the
    // staging writes and the transposed reads across this point and drain outstanding ops.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

// Lane's 8 tokens of a 32-token tile, in MFMA K order: tokens 4g..4g+3 then 16+4g..16+4g+3.
__device__ __forceinline__ int tile_token(int g, int k) { return (k < 4) ? 4 * g + k : 16 + 4 * g + (k - 4); }

struct WaveState {
    float m;        // running max (log2 domain) of head l16
    float l;        // partial sum of p over this lane's tokens
    r2o_f4 acc[8];  // O[4g+i][8*l16 + q] for q = 0..7
};

template <int KIND>
__device__ void run_item(const r2o_decode_params& p, const r2o_work_item& it, const r2o_request_desc& rq,
                         unsigned char* smem, WaveState& st) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
    const int gqa = (int)(p.hq / p.hkv);
    const int64_t kvh = it.kvh, b = it.req;
    const int per = (int)((it.ntiles + kWaves - 1) / kWaves);
    const int t_begin = wave * per;
    const int t_end = min((int)it.ntiles, t_begin + per);
    unsigned char* stage = smem + wave * kStageBytes;
    const float qscale = p.sm_scale * kLog2e;

    // ---- query operand (head l16 of the KV group; padded heads are zero)
    const bool head_ok = l16 < gqa;
    const uint16_t* qrow = p.query + ((b * p.hq) + kvh * gqa + (head_ok ? l16 : 0)) * 128 + 32 * g;
    uint32_t qp[4][4];  // f16 pairs (channel 8j+u, 8j+u+4) of 32g.. (INT4-K path) or bf16 pairs (recent)
    {
        const r2o_u4* q4 = reinterpret_cast<const r2o_u4*>(qrow);
        r2o_u4 raw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) raw[j] = head_ok ? q4[j] : r2o_u4{0, 0, 0, 0};
        float qf[32];
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            const uint32_t v = raw[w / 4][w % 4];
            qf[2 * w] = p.q_dtype == 0 ? r2o_bf16_to_f32(v & 0xffffu) : r2o_f16_to_f32(v & 0xffffu);
            qf[2 * w + 1] = p.q_dtype == 0 ? r2o_bf16_to_f32(v >> 16) : r2o_f16_to_f32(v >> 16);
        }
        if (KIND == kRecent) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u) qp[j][u] = r2o_pack_bf2(qf[8 * j + 2 * u], qf[8 * j + 2 * u + 1]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    qp[j][u] = r2o_pack_h2(qf[8 * j + u] * qscale, qf[8 * j + u + 4] * qscale);
        }
    }

    uint32_t qs[4][4];            // Q' = q * s for the current K superblock (f16 pairs)
    r2o_f4 negcorr = {0, 0, 0, 0};
    int64_t cur_sb = -1;
    const int recent_len = (KIND == kRecent) ? p.recent_len[b] : 0;
    const bool app = (KIND == kRecent) && p.do_append;

    for (int t = t_begin; t < t_end; ++t) {
        const int64_t a0 = it.tile0 + 32 * (int64_t)t;
        // ------------------------------------------------------------ QK^T for 32 tokens
        r2o_f4 s[2];
        if (KIND != kRecent) {
            const int64_t sb = a0 / p.superblock;
            if (sb != cur_sb) {
                cur_sb = sb;
                const int64_t meta = (kvh * rq.k_superblocks + sb) * 128 + 32 * g;
                const r2o_u4* s4 = reinterpret_cast<const r2o_u4*>(rq.k_scale + meta);
                const r2o_u4* z4 = reinterpret_cast<const r2o_u4*>(rq.k_zero + meta);
                uint32_t sd[16], zd[8];
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const r2o_u4 v = s4[w];
                    sd[4 * w] = v.x; sd[4 * w + 1] = v.y; sd[4 * w + 2] = v.z; sd[4 * w + 3] = v.w;
                }
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    const r2o_u4 v = z4[w];
                    zd[4 * w] = v.x; zd[4 * w + 1] = v.y; zd[4 * w + 2] = v.z; zd[4 * w + 3] = v.w;
                }
                negcorr = r2o_f4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    r2o_u4 zop;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const uint32_t sp = r2o_perm(sd[4 * j + 2 + u / 2], sd[4 * j + u / 2],
                                                     (u & 1) ? 0x07060302u : 0x05040100u);
                        qs[j][u] = r2o_h2_mul(qp[j][u], sp);
                        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + u) << 16) | (uint32_t)u;
                        zop[u] = r2o_perm(zd[2 * j + 1], zd[2 * j], sel) | 0xE400E400u;  // -(1024 + z)
                    }
                    negcorr = r2o_mfma_f16(zop, r2o_u4{qs[j][0], qs[j][1], qs[j][2], qs[j][3]}, negcorr);
                }
            }
#pragma unroll
            for (int mg = 0; mg < 2; ++mg) {
                const int64_t tok = a0 + 16 * mg + l16;
                const r2o_u4 kx = *reinterpret_cast<const r2o_u4*>(rq.k_packed + (kvh * rq.k_capacity + tok) * 64 + 16 * g);
                r2o_f4 acc = negcorr;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = kx[j];
                    const r2o_u4 a = {(w & 0x000F000Fu) | 0x64006400u, ((w >> 4) & 0x000F000Fu) | 0x64006400u,
                                      ((w >> 8) & 0x000F000Fu) | 0x64006400u, ((w >> 12) & 0x000F000Fu) | 0x64006400u};
                    acc = r2o_mfma_f16(a, r2o_u4{qs[j][0], qs[j][1], qs[j][2], qs[j][3]}, acc);
                }
                s[mg] = acc;
            }
        } else {
#pragma unroll
            for (int mg = 0; mg < 2; ++mg) {
                const int slot = (int)a0 + 16 * mg + l16;
                const uint16_t* krow = nullptr;
                if (slot < recent_len) krow = rq.recent_k + (kvh * rq.recent_capacity + slot) * 128;
                else if (app && slot == recent_len) krow = p.append_k + (b * p.hkv + kvh) * 128;
                r2o_f4 acc = {0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const r2o_u4 a = krow ? reinterpret_cast<const r2o_u4*>(krow + 32 * g)[j] : r2o_u4{0, 0, 0, 0};
                    acc = r2o_mfma_bf16(a, r2o_u4{qp[j][0], qp[j][1], qp[j][2], qp[j][3]}, acc);
                }
                s[mg] = acc * qscale;
            }
        }

        // ------------------------------------------------------------ V tile -> LDS
        const int64_t vbase = a0 - it.v_delta;  // V row of tile row 0 (segment kinds)
        auto row_valid = [&](int r) -> bool {
            if (KIND == kRecent) return (int)a0 + r < recent_len + (app ? 1 : 0);
            const int64_t pos = a0 + r;
            return pos >= it.lo && pos < it.hi;
        };
        if (KIND == kFP || KIND == kRecent) {
#pragma unroll
            for (int itn = 0; itn < 8; ++itn) {
                const int c = itn * 64 + lane, r = c >> 4, col = c & 15;
                r2o_u4 v = {0, 0, 0, 0};
                if (row_valid(r)) {
                    const uint16_t* vrow;
                    if (KIND == kFP) vrow = rq.fp_v + (kvh * rq.fp_stride + vbase + r) * 128;
                    else if ((int)a0 + r < recent_len) vrow = rq.recent_v + (kvh * rq.recent_capacity + a0 + r) * 128;
                    else vrow = p.append_v + (b * p.hkv + kvh) * 128;
                    v = reinterpret_cast<const r2o_u4*>(vrow)[col];
                }
                *reinterpret_cast<r2o_u4*>(stage + r * 256 + col * 16) = v;
            }
        } else if (KIND == kI4) {
#pragma unroll
            for (int itn = 0; itn < 2; ++itn) {
                const int c = itn * 64 + lane, r = c >> 2, col = c & 3;
                r2o_u4 v = {0, 0, 0, 0};
                if (row_valid(r)) v = reinterpret_cast<const r2o_u4*>(rq.i4_v + (kvh * rq.i4_stride + vbase + r) * 64)[col];
                *reinterpret_cast<r2o_u4*>(stage + r * kRowI4 + col * 16) = v;
            }
        } else {
            const int r = lane >> 1, col = lane & 1;
            r2o_u4 v = {0, 0, 0, 0};
            if (row_valid(r)) v = reinterpret_cast<const r2o_u4*>(rq.i2_v + (kvh * rq.i2_stride + vbase + r) * 32)[col];
            *reinterpret_cast<r2o_u4*>(stage + r * kRowI2 + col * 16) = v;
        }

        // ------------------------------------------------------------ online softmax
        float sv[8];
        bool vk[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int r = tile_token(g, k);
            vk[k] = row_valid(r) && head_ok;
            sv[k] = vk[k] ? s[k >> 2][k & 3] : -INFINITY;
        }
        float tmax = sv[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) tmax = fmaxf(tmax, sv[k]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, R2O_WAVE));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, R2O_WAVE));
        const float m_new = fmaxf(st.m, tmax);
        if (__any(m_new > st.m)) {
            const float alpha = (m_new > st.m) ? (st.m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m - m_new)) : 1.f;
            st.l *= alpha;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float ai = __shfl(alpha, 4 * g + i, R2O_WAVE);
#pragma unroll
                for (int q = 0; q < 8; ++q) st.acc[q][i] *= ai;
            }
            st.m = m_new;
        }
        const float m_use = st.m == -INFINITY ? 0.f : st.m;
        float pk[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            pk[k] = vk[k] ? __builtin_amdgcn_exp2f(sv[k] - m_use) : 0.f;
            st.l += pk[k];
        }

        // ------------------------------------------------------------ P operand
        r2o_u4 ap;
        if (KIND == kFP || KIND == kRecent) {
#pragma unroll
            for (int u = 0; u < 4; ++u) ap[u] = r2o_pack_bf2(pk[2 * u], pk[2 * u + 1]);
        } else if (KIND == kI4) {
            float pv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int r = tile_token(g, k);
                const float sc = row_valid(r) ? rq.i4_scale[kvh * rq.i4_stride + vbase + r] : 0.f;
                pv[k] = pk[k] * sc;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) ap[u] = r2o_pack_h2(pv[2 * u], pv[2 * u + 1]);
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) ap[u] = r2o_pack_h2(pk[2 * u], pk[2 * u + 1]);
        }

        // ------------------------------------------------------------ PV from LDS
        wave_lds_fence();
        if (KIND == kFP || KIND == kRecent) {
            r2o_u4 R[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) R[k] = *reinterpret_cast<const r2o_u4*>(stage + tile_token(g, k) * 256 + 16 * l16);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t sel = (q & 1) ? 0x07060302u : 0x05040100u;
                const r2o_u4 bop = {r2o_perm(R[1][q >> 1], R[0][q >> 1], sel), r2o_perm(R[3][q >> 1], R[2][q >> 1], sel),
                                    r2o_perm(R[5][q >> 1], R[4][q >> 1], sel), r2o_perm(R[7][q >> 1], R[6][q >> 1], sel)};
                st.acc[q] = r2o_mfma_bf16(ap, bop, st.acc[q]);
            }
        } else if (KIND == kI4) {
            uint32_t X[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                X[k] = *reinterpret_cast<const uint32_t*>(stage + tile_token(g, k) * kRowI4 + 4 * l16) ^ 0x88888888u;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + bb) << 16) | (uint32_t)bb;
                uint32_t y[4];
#pragma unroll
                for (int pr = 0; pr < 4; ++pr) y[pr] = r2o_perm(X[2 * pr + 1], X[2 * pr], sel);
                const r2o_u4 lo = {(y[0] & 0x000F000Fu) | 0x64006400u, (y[1] & 0x000F000Fu) | 0x64006400u,
                                   (y[2] & 0x000F000Fu) | 0x64006400u, (y[3] & 0x000F000Fu) | 0x64006400u};
                const r2o_u4 hi = {((y[0] >> 4) & 0x000F000Fu) | 0x64006400u, ((y[1] >> 4) & 0x000F000Fu) | 0x64006400u,
                                   ((y[2] >> 4) & 0x000F000Fu) | 0x64006400u, ((y[3] >> 4) & 0x000F000Fu) | 0x64006400u};
                r2o_u4 lo2, hi2;
#pragma unroll
                for (int pr = 0; pr < 4; ++pr) {  // (1032 + c) - 1032 = c exactly in fp16
                    lo2[pr] = r2o_h2_sub(lo[pr], 0x64086408u);
                    hi2[pr] = r2o_h2_sub(hi[pr], 0x64086408u);
                }
                st.acc[2 * bb] = r2o_mfma_f16(ap, lo2, st.acc[2 * bb]);
                st.acc[2 * bb + 1] = r2o_mfma_f16(ap, hi2, st.acc[2 * bb + 1]);
            }
        } else {
            const int groups = (int)(128 / p.int2_group);
            const int gamma = (8 * l16) / (int)p.int2_group;
            uint32_t Y[8], zh[8], sh[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int r = tile_token(g, k);
                Y[k] = *reinterpret_cast<const uint16_t*>(stage + r * kRowI2 + 2 * l16);
                if (row_valid(r)) {
                    const int64_t mrow = (kvh * rq.i2_stride + vbase + r) * groups + gamma;
                    zh[k] = 0x6400u | rq.i2_zero[mrow];
                    sh[k] = rq.i2_scale[mrow];
                } else {
                    zh[k] = 0x6400u;
                    sh[k] = 0u;
                }
            }
            uint32_t yp[4], zp[4], sp[4];
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                yp[pr] = Y[2 * pr] | (Y[2 * pr + 1] << 16);
                zp[pr] = zh[2 * pr] | (zh[2 * pr + 1] << 16);
                sp[pr] = sh[2 * pr] | (sh[2 * pr + 1] << 16);
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int shift = (q < 4) ? 2 * q : 8 + 2 * (q - 4);
                r2o_u4 bop;
#pragma unroll
                for (int pr = 0; pr < 4; ++pr) {
                    const uint32_t c = ((yp[pr] >> shift) & 0x00030003u) | 0x64006400u;
                    bop[pr] = r2o_h2_mul(r2o_h2_sub(c, zp[pr]), sp[pr]);
                }
                st.acc[q] = r2o_mfma_f16(ap, bop, st.acc[q]);
            }
        }
        wave_lds_fence();
    }
}

__global__ __launch_bounds__(256, 2) void decode_partial_kernel(r2o_decode_params p) {
    __shared__ __align__(16) unsigned char smem[kSmemBytes];
    const r2o_work_item it = p.items[blockIdx.x];
    const r2o_request_desc rq = p.reqs[it.req];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
    const int gqa = (int)(p.hq / p.hkv);

    WaveState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) st.acc[q] = r2o_f4{0, 0, 0, 0};

    switch (it.kind) {
        case kFP: run_item<kFP>(p, it, rq, smem, st); break;
        case kI4: run_item<kI4>(p, it, rq, smem, st); break;
        case kI2: run_item<kI2>(p, it, rq, smem, st); break;
        default: run_item<kRecent>(p, it, rq, smem, st); break;
    }

    // ---- per-wave epilogue: reduce l (and u) over the 4 lane groups of each head
    float l_h = st.l;
    l_h += __shfl_xor(l_h, 16, R2O_WAVE);
    l_h += __shfl_xor(l_h, 32, R2O_WAVE);
    __syncthreads();  // every wave is done with its staging area
    float* mrg = reinterpret_cast<float*>(smem) + wave * kMergeFloats;
    if (g == 0) {
        mrg[l16] = st.m;
        mrg[16 + l16] = l_h;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < 8; ++q) mrg[32 + (4 * g + i) * 128 + 8 * l16 + q] = st.acc[q][i];
    __syncthreads();

    // ---- merge the 4 wave states of this block and write the partial
    const float* base = reinterpret_cast<const float*>(smem);
    for (int e = threadIdx.x; e < gqa * 128; e += blockDim.x) {
        const int h = e >> 7, d = e & 127;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, base[w * kMergeFloats + h]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float mw = base[w * kMergeFloats + h];
                const float sc = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
                L += base[w * kMergeFloats + 16 + h] * sc;
                A += base[w * kMergeFloats + 32 + h * 128 + d] * sc;
            }
        }
        const int64_t slot = (int64_t)blockIdx.x * 16 + h;
        p.partial_out[slot * 128 + d] = A;
        if (d == 0) {
            p.partial_max[slot] = M;
            p.partial_sum[slot] = L;
        }
    }
}

__global__ __launch_bounds__(128) void decode_combine_kernel(r2o_decode_params p) {
    __shared__ float buf[128];
    const int64_t b = blockIdx.y;
    const int hqi = blockIdx.x;
    const int d = threadIdx.x;
    const int gqa = (int)(p.hq / p.hkv);
    const int kvh = hqi / gqa, h = hqi % gqa;
    const int beg = p.group_begin[b * p.hkv + kvh], end = p.group_begin[b * p.hkv + kvh + 1];
    float M = -INFINITY;
    for (int i = beg; i < end; ++i) M = fmaxf(M, p.partial_max[(int64_t)i * 16 + h]);
    float L = 0.f, A = 0.f;
    if (M != -INFINITY) {
        for (int i = beg; i < end; ++i) {
            const int64_t slot = (int64_t)i * 16 + h;
            const float m = p.partial_max[slot];
            const float sc = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
            L += p.partial_sum[slot] * sc;
            A += p.partial_out[slot * 128 + d] * sc;
        }
    }
    float y = r2o_bf16_to_f32(r2o_f32_to_bf16(A / L));
    if (p.output_hadamard) {
        buf[d] = y;
        __syncthreads();
        for (int stride = 1; stride < 128; stride <<= 1) {
            float a = 0.f, c = 0.f;
            int i0 = 0;
            if (d < 64) {
                i0 = (d / stride) * 2 * stride + (d & (stride - 1));
                a = buf[i0];
                c = buf[i0 + stride];
            }
            __syncthreads();
            if (d < 64) {
                buf[i0] = a + c;
                buf[i0 + stride] = a - c;
            }
            __syncthreads();
        }
        y = buf[d] * 0.08838834764831845f;
    }
    p.out[(b * p.hq + hqi) * 128 + d] = (uint16_t)r2o_f32_to_bf16(y);

    if (p.do_append && hqi < p.hkv) {  // fused Recent-FP append (triton_fourq_splitk.py:1007-1020)
        const r2o_request_desc& rq = p.reqs[b];
        const int64_t pos = p.recent_len[b];
        rq.recent_k[(hqi * rq.recent_capacity + pos) * 128 + d] = p.append_k[(b * p.hkv + hqi) * 128 + d];
        rq.recent_v[(hqi * rq.recent_capacity + pos) * 128 + d] = p.append_v[(b * p.hkv + hqi) * 128 + d];
        if (hqi == 0 && d == 0) {
            rq.recent_global[pos] = p.append_global[b];
            rq.recent_logical[pos] = p.append_logical[b];
            *rq.recent_length = (int32_t)(pos + 1);
            rq.recent_page_lengths[pos / p.page_size] = pos % p.page_size + 1;
        }
    }
}

int validate(const r2o_decode_params* p) {
    if (!p || !p->reqs || !p->items || !p->group_begin || !p->partial_max || !p->partial_sum || !p->partial_out ||
        !p->query || !p->out)
        return R2O_EINVAL;
    if (p->n_items <= 0 || p->n_items > 0x7fffffff || p->batch <= 0 || p->batch > R2O_MAX_BATCH) return R2O_EINVAL;
    if (p->hkv <= 0 || p->hq <= 0 || p->hq % p->hkv || p->hq / p->hkv > R2O_MAX_GQA) return R2O_EINVAL;
    if (!(p->superblock == 32 || p->superblock == 64 || p->superblock == 128)) return R2O_EINVAL;
    if (!(p->int2_group == 32 || p->int2_group == 64 || p->int2_group == 128)) return R2O_EINVAL;
    if (p->q_dtype != 0 && p->q_dtype != 1) return R2O_EINVAL;
    if (p->page_size <= 0) return R2O_EINVAL;
    if (p->do_append && (!p->append_k || !p->append_v)) return R2O_EINVAL;
    return R2O_OK;
}

}  // namespace

extern "C" {

int r2o_decode_partial(const r2o_decode_params* params, void* stream) {
    const int rc = validate(params);
    if (rc) return rc;
    hipLaunchKernelGGL(decode_partial_kernel, dim3((unsigned)params->n_items), dim3(256), 0, (hipStream_t)stream,
                       *params);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int r2o_decode_combine(const r2o_decode_params* params, void* stream) {
    const int rc = validate(params);
    if (rc) return rc;
    hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)params->hq, (unsigned)params->batch), dim3(128), 0,
                       (hipStream_t)stream, *params);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

}  // extern "C"
