// Split-K GQA decode over the SSPA packed cache for gfx950 (CDNA4, wave64, MFMA 16x16x32).
//
// Partial pass: one 256-thread block (4 waves) per work item, i.e. a run of 32-token tiles of
// one pool segment of one (request, kv head).  Each wave walks its share of the tiles with an
// online softmax in the log2 domain and keeps a 16 x 128 fp32 accumulator (query heads of the
// KV group padded to 16 MFMA rows).  The history keys come in one of three formats
// (r2o_decode_params.k_format), each a template instance of the kernel.  Per tile:
//   QK  S^T[tok, h] = sum_c K[tok, c] * Q'[h, c]  as f16 MFMA on the raw codes.
//       INT4-K: the A operand is (1024 + code) built in place from the nibbles, the B operand
//       is Q' = q * s (per-channel scale of the tile's K superblock, times D^-1/2 * log2 e), and
//       -sum_c Q'[h, c] * (1024 + z_c) is added by one more MFMA per channel block, so the chain
//       returns q . (code - z) * s exactly as the dequantised dot.
//       INT2-K: the crumb at bit position 2u of a 16-bit lane enters as 1024 + 4^u * code, the
//       B operand carries s / 4^u, and two correction MFMAs add sum_c q * offset_c and remove
//       the 1024 offsets, so the chain returns q . (code * s + offset).
//       The per-superblock operand pairs of both are written at pack time and arrive with the
//       tile.  BF16-K history and Recent-FP tiles use a bf16 MFMA on the bf16 K rows.
//   PV  O[h, d] += sum_tok P[h, tok] V[tok, d]: each lane holds the 8 adjacent dims 8*l16.. of
//       its 8 tokens, the MFMA B operand of 8 consecutive tokens after a byte permute (output
//       dim 8*l16 + q of MFMA q).  BF16 V: bf16 MFMA.  INT4 V: the per-token scale is folded
//       into P (P' = p * s) and the signed codes enter exactly as f16 (1032 + c, low nibbles,
//       and 1152 + 16 c in place for the high nibbles), the offsets being removed after the
//       last tile.  INT2 V: (c - z) * s is formed in f16 per element, or, when a group spans all
//       128 dims (one scale and zero point per token), the scale is folded into P and the crumbs
//       enter as 1024 + c, sum P' (1024 + z) being removed after the last tile.
//   Pool tiles arrive by global->LDS DMA into a one-stage-per-wave ring (no VGPRs held while in
//   flight); Recent-FP tiles are loaded straight into registers, all loads of a tile first.
// The 4 waves' states are merged in LDS and one (max, sum, acc[GQA][128]) fp32 partial is
// written with streaming stores (read once, by the combine).
//
// Combine pass: one block per (request, query head) merges the partials of its (request,
// kv head) group, divides, rounds to bf16, optionally applies the 128-point FWHT and performs
// the fused Recent-FP append of the step's K/V row and metadata.
//
// Semantics follow triton_fourq_splitk.py:456-1020 (tile attention, exact state merge, fused
// append :1007-1020, output Hadamard :1000-1006) and the oracle triton_fourq_attention.py:72-125.
#include <atomic>

#include "r2o_common.hpp"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMergeFloats = 16 + 16 + 16 * 128;    // per wave: m, l, acc

// History-key formats (r2o_decode_params.k_format): the compact INT4 arena, bf16 rows
// (matched-FP and v_fourq_k_bf16 caches) or the compact INT2 arena (v_fourq_k_int2_compact).
enum KFormat { kKInt4 = 0, kKBf16 = 1, kKInt2 = 2 };

// Element type of the 16-bit rows (FP-V pool, Recent-FP ring, BF16-K arena, appended token):
// r2o_decode_params.row_dtype.  Their MFMAs take the rows as they are, with P and the query packed to
// the same type.
enum RowFormat { kRowBf16 = 0, kRowF16 = 1 };

template <int RF>
__device__ __forceinline__ uint32_t pack_row2(float lo, float hi) {
    return RF == kRowF16 ? r2o_pack_h2(lo, hi) : r2o_pack_bf2(lo, hi);
}
template <int RF>
__device__ __forceinline__ r2o_f4 mfma_rows(r2o_u4 a, r2o_u4 b, r2o_f4 c) {
    if constexpr (RF == kRowF16) return r2o_mfma_f16(a, b, c);
    else return r2o_mfma_bf16(a, b, c);
}

// Per-kernel LDS / occupancy configuration.
// Build-time tuning knob (the default is the measured best on MI355X).
#ifndef R2O_DMA_STAGES
#define R2O_DMA_STAGES 1          // LDS stages per wave: tiles in flight while one is computed
#endif
constexpr int kDmaStages = R2O_DMA_STAGES;
static_assert(kDmaStages >= 1 && kDmaStages <= 3, "1 to 3 LDS stages per wave");

template <int KF>
struct KernelCfg {
    static constexpr int kWaves = 4;  // waves per workgroup
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kStage = KF == kKBf16 ? 16384 : 10752;  // one tile stage (sized for BF16 V, see StageLayout)
    static constexpr int kWaveLds = kDmaStages * kStage;
    static constexpr int kSmem = (kWaves * kMergeFloats * 4 > kWaves * kWaveLds) ? kWaves * kMergeFloats * 4
                                                                                 : kWaves * kWaveLds;
    static constexpr int kBlocksPerCU = 2;  // resident partial workgroups per CU (the planner launches 2 per CU)
    static constexpr int kWavesPerSimd = kBlocksPerCU * kWaves / 4;  // __launch_bounds__' second argument
};
static_assert(2 * KernelCfg<kKInt4>::kSmem <= 160 * 1024 && 2 * KernelCfg<kKBf16>::kSmem <= 160 * 1024,
              "two partial workgroups fit one CU's LDS");
constexpr int kRotLdsBytes = 18 * 136 * 2;  // the rows of a folded rotation (kRotBytes, below)
static_assert(2 * (KernelCfg<kKBf16>::kSmem + kRotLdsBytes) <= 160 * 1024, "with the rotation's rows as well");

enum Kind { kFP = 0, kI4 = 1, kI2 = 2, kRecent = 3 };

// Phase stamps of the measurement build (-DR2O_TIMELINE, libr2o_timeline.so, bench.py --timeline): each
// wave keeps real-time counter reads (100 MHz, one clock for the whole GPU) in registers and stores
// them once at its end.  In the product build the struct is empty and every stamp compiles to nothing.
struct Stamps {
#ifdef R2O_TIMELINE
    unsigned long long t[12];
#endif
};
__device__ __forceinline__ void stamp(Stamps& s, int i) {
#ifdef R2O_TIMELINE
    s.t[i] = __builtin_amdgcn_s_memrealtime();
#endif
}
#ifdef R2O_TIMELINE
// partial kernel: per (block, wave) 12 slots: 0 entry, 1 work item arrived, 2 first DMA issued, 3 first
// tile landed, 4 last tile landed, 5 tile loop done, 6 block done (partial stores issued), 7 XCC id |
// HW_ID << 32, 8 tiles | kind << 32.  combine: per (block, wave) 12 slots: 0 entry, 1 arguments
// arrived, 2 first round of partials landed, 3 merged, 4 (wave 0) output stored.
constexpr int kTimelineBlocks = 4096;
constexpr int kTimelineWaves = 4;  // stamp slots per partial workgroup (one per wave)
__device__ unsigned long long g_timeline_partial[kTimelineBlocks * kTimelineWaves * 12];
__device__ unsigned long long g_timeline_combine[kTimelineBlocks * 8 * 12];
__device__ __forceinline__ void stamps_store(unsigned long long* dst, int block, int wave, int waves, const Stamps& s) {
    if ((threadIdx.x & 63) == 0 && block < kTimelineBlocks)
#pragma unroll
        for (int k = 0; k < 12; ++k) dst[((int64_t)block * waves + wave) * 12 + k] = s.t[k];
}
#endif

// Lane's 8 tokens of a 32-token tile, in MFMA K order: tokens 4g..4g+3 then 16+4g..16+4g+3.
__device__ __forceinline__ int tile_token(int g, int k) { return (k < 4) ? 4 * g + k : 16 + 4 * g + (k - 4); }

struct WaveState {
    float m;        // running max (log2 domain) of head l16
    float l;        // partial sum of p over this lane's tokens
    r2o_f4 acc[8];  // O[4g+i][8*l16 + q] for q = 0..7
};

// ------------------------------------------------------------------ folded decode-step rotation
// With r2o_decode_params.rope_mode 1 the query and the appended key arrive as raw projections and the
// partial kernel applies the decode step's Qwen mRoPE (and FWHT) itself, bit-identically to
// qk_mrope_kernel (r2o_rope.hip): y = x * cos + rotate_half(x) * sin in fp32, channel c taking cos/sin
// from table axis 0, 1 or 2 by c % 64 against the sections, then optionally the orthonormal FWHT in
// the stage order 1, 2, .., 64, then one rounding to the row's dtype; the appended value takes the
// FWHT alone.  A row is rotated by one 16-lane group, lane c8 holding channels 8 c8 .. 8 c8 + 7 (FWHT
// strides 1 .. 4 inside the lane, 8 .. 64 across lanes c8 ^ 1 .. c8 ^ 8 of the group; every fp32 sum
// takes the same operands in the same order as the separate launch).  The 4 waves of a work item
// share the rows (4 per wave), which meet in LDS; after a barrier each lane reads the channels it holds
// as an MFMA operand, as it would read rotated rows in memory.
enum RopeMode { kRopeNone = 0, kRopeMrope = 1, kRopeQwen3 = 2 };

// A work item's LDS rows of a folded rotation (row dtype): the KV group's query heads 0 .. 15, then the
// appended key (row 16) and value (row 17); 272 bytes apart, so that 16 lanes' reads of one channel
// range from different rows fall on different banks.
constexpr int kRotStride = 136;
constexpr int kRotKeyRow = 16;
constexpr int kRotBytes = 18 * kRotStride * 2;
static_assert(kRotBytes == kRotLdsBytes, "one size for the rotation's LDS rows");

// Orthonormal FWHT-128 of a row whose dims 8 l16 .. 8 l16 + 7 this lane holds (the V layout of a
// Recent-FP tile): strides 1 .. 4 inside the lane, 8 .. 64 across lanes l16 ^ 1 .. l16 ^ 8 of a row.
__device__ __forceinline__ void fwht_row8(float (&y)[8], int l16) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if ((i & h) == 0) {
                const float a = y[i], c = y[i + h];
                y[i] = a + c;
                y[i + h] = a - c;
            }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float v = y[i], o;
        o = r2o_lane_xor<1>(v);
        v = (l16 & 1) ? o - v : v + o;
        o = r2o_lane_xor<2>(v);
        v = (l16 & 2) ? o - v : v + o;
        o = r2o_lane_xor<4>(v);
        v = (l16 & 4) ? o - v : v + o;
        o = r2o_lane_xor<8>(v);
        v = (l16 & 8) ? o - v : v + o;
        y[i] = v * 0.08838834764831845f;
    }
}

// Elements from one request's query (appended) rows to the next.  Only calls with a folded rotation
// take strided rows (views of a fused projection; the launch helpers spell a stride of 0 out as the
// dense figure); the other calls' rows are dense, as the reference requires, and the kernels
// compute their addresses without reading a stride, which would sit on the path to the first tile.
template <int RO>
__device__ __forceinline__ int64_t q_stride(const r2o_decode_params& p) {
    return RO != kRopeNone ? p.query_batch_stride : p.hq * 128;
}

// The query row of head l16 of the KV group (padded heads read head 0; their operand is zeroed).
template <int RO>
__device__ __forceinline__ const uint16_t* query_row(const r2o_decode_params& p, int64_t b, int64_t kvh, int gqa,
                                                     int l16) {
    return p.query + b * q_stride<RO>(p) + (kvh * gqa + (l16 < gqa ? l16 : 0)) * 128;
}

// The inputs of a lane's part of a rotation, put out ahead of the work item's first tile DMAs: the cos /
// sin table runs of the lane's 8 channels c = 8 c8 .. 8 c8 + 7 for the three axes, as whole 16-byte
// pieces (one each for 16-bit tables, two for fp32; the host requires unit channel strides and 16-byte
// aligned rows), and the raw row (its 8 channels and their rotate-half partners c -/+ 64).  Offsets
// from the request's table base are 32-bit byte offsets (below 2^31, checked on the host).
struct RotPrefetch {
    r2o_u4 tab[2][3][2];  // [cos, sin][axis][piece]
    r2o_u4 x, xp;
};

__device__ __forceinline__ void rot_row_loads(const uint16_t* row, int c8, r2o_u4& x, r2o_u4& xp) {
    x = r2o_ldg(reinterpret_cast<const r2o_u4*>(row + 8 * c8));
    xp = r2o_ldg(reinterpret_cast<const r2o_u4*>(row + 8 * (c8 ^ 8)));
}

// The source of rotation row r of a work item: query head r < gqa, the appended key (r == gqa) or value.
__device__ __forceinline__ const uint16_t* rot_source(const r2o_decode_params& p, int64_t b, int64_t kvh, int gqa,
                                                      int r) {
    if (r < gqa) return query_row<kRopeMrope>(p, b, kvh, gqa, r);
    return (r == gqa ? p.append_k : p.append_v) + b * p.append_batch_stride + kvh * 128;
}

// (RM: kRopeMrope reads the three axes' runs, kRopeQwen3 the one table's: 16-bit, one piece.)
template <int RM>
__device__ __forceinline__ void rot_prefetch(const r2o_decode_params& p, int64_t b, const uint16_t* row, int c8,
                                             RotPrefetch& f) {
    constexpr int kAxes = RM == kRopeQwen3 ? 1 : 3;
    const int pieces = RM == kRopeQwen3 ? 1 : (p.rope_table_dtype == 2 ? 2 : 1);
    const int64_t esize = RM == kRopeQwen3 ? 2 : (p.rope_table_dtype == 2 ? 4 : 2);
    const char* tab[2] = {reinterpret_cast<const char*>(p.rope_cos) + b * p.rope_cos_strides[1] * esize,
                          reinterpret_cast<const char*>(p.rope_sin) + b * p.rope_sin_strides[1] * esize};
    const uint32_t axis_bytes[2] = {(uint32_t)(p.rope_cos_strides[0] * esize), (uint32_t)(p.rope_sin_strides[0] * esize)};
    const uint32_t o = (uint32_t)(8 * c8 * esize);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int a = 0; a < kAxes; ++a)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                if (q < pieces) f.tab[t][a][q] = r2o_ldg(reinterpret_cast<const r2o_u4*>(tab[t] + (a * axis_bytes[t] + o + 16 * q)));
    rot_row_loads(row, c8, f.x, f.xp);
}

// Channel k of 8 packed 16-bit channels, as fp32.
__device__ __forceinline__ float row_channel(const r2o_u4& w, int k, int dt) {
    const uint32_t h = (k & 1) ? w[k >> 1] >> 16 : w[k >> 1] & 0xffffu;
    return dt == 0 ? r2o_bf16_to_f32(h) : r2o_f16_to_f32(h);
}

// cos / sin of the lane's 8 channels as fp32: channel k takes axis 1 from bit k of m1 and axis 2 from
// bit k of m2 (bit masks of the lane's channels against the sections, d = c % 64), selected by bit
// operations (per-channel condition masks would hold a pair of scalar registers each).
template <int RM>
__device__ __forceinline__ void rot_tables(const r2o_decode_params& p, int c8, const RotPrefetch& f, float (&cs)[8],
                                           float (&sn)[8]) {
    const int code = (int)p.rope_table_dtype;
    if constexpr (RM == kRopeQwen3) {  // one table in the row dtype
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            cs[k] = row_channel(f.tab[0][0][0], k, code);
            sn[k] = row_channel(f.tab[1][0][0], k, code);
        }
        return;
    }
    const int d0 = (8 * c8) & 63, t0 = (int)p.rope_section0 - d0, t1 = t0 + (int)p.rope_section1;
    const uint32_t m1 = t0 <= 0 ? 0xffu : (t0 >= 8 ? 0u : (0xffu << t0) & 0xffu);
    const uint32_t m2 = t1 <= 0 ? 0xffu : (t1 >= 8 ? 0u : (0xffu << t1) & 0xffu);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t v[2][3];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                const uint32_t w16 = f.tab[t][a][0][k >> 1];
                v[t][a] = code == 2 ? f.tab[t][a][k >> 2][k & 3] : ((k & 1) ? w16 >> 16 : w16 & 0xffffu);
            }
        const uint32_t f1 = 0u - ((m1 >> k) & 1u), f2 = 0u - ((m2 >> k) & 1u);
        float out[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t v01 = v[t][0] ^ ((v[t][0] ^ v[t][1]) & f1);
            const uint32_t bits = v01 ^ ((v01 ^ v[t][2]) & f2);
            out[t] = code == 2 ? __uint_as_float(bits) : (code == 0 ? r2o_bf16_to_f32(bits) : r2o_f16_to_f32(bits));
        }
        cs[k] = out[0];
        sn[k] = out[1];
    }
}

// One row of a folded rotation in a 16-lane group (lane c8: channels 8 c8 .. 8 c8 + 7): mRoPE then, with
// `had`, the FWHT (rope = false: the FWHT alone, for the appended value), one rounding to the row dtype,
// as the packed 16-bit channels.
// With rope_mode 2 (`qwen3`, the Qwen3 branch) the rotation is that of qk_norm_rope_kernel
// (r2o_rope.hip): the RMSNorm with `weight` (the row's q_norm or k_norm weights), then
// apply_rotary_pos_emb with every product and the sum rounded to the row dtype.  The sum of squares
// follows that kernel's butterfly: pair sums x[t]^2 + x[t + 64]^2 for t = 8 (c8 % 8) + k, combined over
// t's bits 5, 4, 3 across lanes c8 ^ 4, ^ 2, ^ 1 and bits 2, 1, 0 inside the lane, so the mean and the
// rounding of every product are those of the separate launch.
template <int RM>
__device__ __forceinline__ r2o_u4 rot_row(const r2o_decode_params& p, const r2o_u4& x, const r2o_u4& xp,
                                          const float (&cs)[8], const float (&sn)[8], int c8, bool rope, bool had,
                                          const uint16_t* weight) {
    const int dt = (int)p.row_dtype;
    float y[8];
    if (RM == kRopeQwen3 && rope) {  // whole 16-lane groups take the same branch
        float xv[8], xpv[8], s[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            xv[k] = row_channel(x, k, dt);
            xpv[k] = row_channel(xp, k, dt);
            const float lo = c8 < 8 ? xv[k] : xpv[k], hi = c8 < 8 ? xpv[k] : xv[k];  // x[t], x[t + 64]
            s[k] = __fadd_rn(__fmul_rn(lo, lo), __fmul_rn(hi, hi));
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            s[k] = __fadd_rn(s[k], r2o_lane_xor<4>(s[k]));
            s[k] = __fadd_rn(s[k], r2o_lane_xor<2>(s[k]));
            s[k] = __fadd_rn(s[k], r2o_lane_xor<1>(s[k]));
        }
#pragma unroll
        for (int m = 4; m >= 1; m >>= 1)
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if ((k & m) == 0) {
                    const float a = __fadd_rn(s[k], s[k + m]);
                    s[k] = a;
                    s[k + m] = a;
                }
        const float inv = __fdiv_rn(1.f, __fsqrt_rn(__fadd_rn(__fdiv_rn(s[0], 128.f), p.norm_eps)));
        const r2o_u4 wo = r2o_ldg(reinterpret_cast<const r2o_u4*>(weight + 8 * c8));
        const r2o_u4 wp = r2o_ldg(reinterpret_cast<const r2o_u4*>(weight + 8 * (c8 ^ 8)));
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float w = r2o_round_dtype(__fmul_rn(row_channel(wo, k, dt), r2o_round_dtype(__fmul_rn(xv[k], inv), dt)), dt);
            const float wq = r2o_round_dtype(__fmul_rn(row_channel(wp, k, dt), r2o_round_dtype(__fmul_rn(xpv[k], inv), dt)), dt);
            y[k] = r2o_round_dtype(__fadd_rn(r2o_round_dtype(__fmul_rn(w, cs[k]), dt),
                                             r2o_round_dtype(__fmul_rn(c8 < 8 ? -wq : wq, sn[k]), dt)), dt);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float xv = row_channel(x, k, dt), xpv = row_channel(xp, k, dt);
            const float rk = xv * cs[k] + (c8 < 8 ? -xpv : xpv) * sn[k];  // rotate_half: (-x[c + 64], x[c - 64])
            y[k] = rope ? rk : xv;
        }
    }
    if (had) fwht_row8(y, c8);  // whole 16-lane groups take the same branch
    r2o_u4 out;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t lo = dt == 0 ? r2o_f32_to_bf16(y[2 * u]) : r2o_f32_to_f16(y[2 * u]);
        const uint32_t hi = dt == 0 ? r2o_f32_to_bf16(y[2 * u + 1]) : r2o_f32_to_f16(y[2 * u + 1]);
        out[u] = lo | (hi << 16);
    }
    return out;
}

// Rotation row r of the work item in the 16-lane group lane >> 4 of wave (r / 4) % 4 (rows 16, 17 in
// a second round): query heads rounded into LDS rows 0 .. gqa - 1; with `kv` (the Recent-FP item of a
// call with an append) the appended key and value into rows 16, 17 and to rotated_k / rotated_v for
// the combine's append (that item is their only reader).  The waves meet at a barrier after this;
// each then reads the rows it needs.
template <int RM>
__device__ __forceinline__ void rot_block_row(const r2o_decode_params& p, int64_t b, int64_t kvh, int gqa, int r,
                                              int c8, const RotPrefetch& f, uint16_t* rot) {
    float cs[8], sn[8];
    rot_tables<RM>(p, c8, f, cs, sn);
    const bool is_q = r < gqa, is_v = r == gqa + 1;
    const r2o_u4 out = rot_row<RM>(p, f.x, f.xp, cs, sn, c8, !is_v, is_v ? p.value_hadamard != 0 : p.rope_hadamard != 0,
                                   is_q ? p.q_norm_weight : p.k_norm_weight);
    *reinterpret_cast<r2o_u4*>(rot + (is_q ? r : kRotKeyRow + (r - gqa)) * kRotStride + 8 * c8) = out;
    if (!is_q) *reinterpret_cast<r2o_u4*>((is_v ? p.rotated_v : p.rotated_k) + (b * p.hkv + kvh) * 128 + 8 * c8) = out;
}

// The lane's rotated query channels 32g .. 32g + 31 of head l16 (zero for the padded heads), after
// the barrier.
__device__ __forceinline__ void rot_read_query(const uint16_t* rot, int gqa, int l16, int g, r2o_u4 (&q)[4]) {
    const r2o_u4* src = reinterpret_cast<const r2o_u4*>(rot + (l16 < gqa ? l16 : 0) * kRotStride + 32 * g);
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = l16 < gqa ? src[j] : r2o_u4{0, 0, 0, 0};
}

// Query operand of head l16 of the KV group (padded heads are zero), channels 32g .. 32g+31, in
// the K operand order of the format: f16 pairs (8j+u, 8j+u+4) for INT4-K, f16 pairs
// (16(j/2) + 4(j%2) + u, +8) for INT2-K, both scaled by D^-1/2 log2(e), or bf16 pairs in channel
// order for bf16 keys (BF16-K pools and the Recent-FP ring; fp16 pairs for fp16 rows).  With a folded
// rotation (RO) `qrot` holds the lane's rotated channels (rot_read_query).
template <int KF, int RF, int RO>
__device__ __forceinline__ void load_query(const r2o_decode_params& p, int64_t b, int64_t kvh, int gqa, int l16,
                                           int g, float qscale, uint32_t (&qp)[4][4], const r2o_u4 (&qrot)[4]) {
    const bool head_ok = l16 < gqa;
    float qf[32];
    {
        r2o_u4 raw[4];
        if constexpr (RO != kRopeNone) {
#pragma unroll
            for (int j = 0; j < 4; ++j) raw[j] = qrot[j];
        } else {
            const r2o_u4* q4 = reinterpret_cast<const r2o_u4*>(query_row<RO>(p, b, kvh, gqa, l16) + 32 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j) raw[j] = head_ok ? r2o_ldg(q4 + j) : r2o_u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            const uint32_t v = raw[w / 4][w % 4];
            qf[2 * w] = p.q_dtype == 0 ? r2o_bf16_to_f32(v & 0xffffu) : r2o_f16_to_f32(v & 0xffffu);
            qf[2 * w + 1] = p.q_dtype == 0 ? r2o_bf16_to_f32(v >> 16) : r2o_f16_to_f32(v >> 16);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u)
            qp[j][u] = KF == kKBf16 ? pack_row2<RF>(qf[8 * j + 2 * u], qf[8 * j + 2 * u + 1])
                     : KF == kKInt4 ? r2o_pack_h2(qf[8 * j + u] * qscale, qf[8 * j + u + 4] * qscale)
                                    : r2o_pack_h2(qf[16 * (j >> 1) + 4 * (j & 1) + u] * qscale,
                                                  qf[16 * (j >> 1) + 4 * (j & 1) + u + 8] * qscale);
}

// Max / sum over the 4 lanes l16 + 16g (g = 0..3) that hold one head, with VALU lane swaps.
__device__ __forceinline__ float head_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}

// Online-softmax update for one tile: sv are the lane's 8 logits (log2 domain, -inf = masked).
// Returns the probabilities in pk.  The running max is raised lazily: only when a tile's max
// exceeds it by more than kRescaleSlack (log2 units) are the state and the NE accumulators at `extra`
// (4-row accumulators in the PV output layout) rescaled, so p = exp2(s - m) stays below
// 2^kRescaleSlack while the rescale branch is taken only a few times per work item.  (m, l, acc)
// always refer to the same m, so the state and its later merges are exact.
constexpr float kRescaleSlack = 4.f;

template <int N, int NE, bool ACC_L = true>
__device__ __forceinline__ void softmax_step(WaveState& st, const float (&sv)[N], float (&pk)[N], int g, float add,
                                             r2o_f4* extra) {
    float tmax = sv[0];
#pragma unroll
    for (int k = 1; k < N; ++k) tmax = fmaxf(tmax, sv[k]);
    tmax = head_max(tmax) + add;  // -inf + add = -inf
    if (__any(tmax > st.m + kRescaleSlack)) {  // -inf + slack = -inf: the first valid tile rescales
        const float m_new = fmaxf(st.m, tmax);
        // exp2(-inf) = 0 when the state was empty; a head with no valid token keeps alpha = 1
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(st.m - m_new);
        st.l *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * g + i, R2O_WAVE);
#pragma unroll
            for (int q = 0; q < 8; ++q) st.acc[q][i] *= ai;
#pragma unroll
            for (int e = 0; e < NE; ++e) extra[e][i] *= ai;
        }
        st.m = m_new;
    }
    const float d = (st.m == -INFINITY ? 0.f : st.m) - add;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        pk[k] = __builtin_amdgcn_exp2f(sv[k] - d);  // exp2(-inf) = 0 for masked tokens
        if constexpr (ACC_L) st.l += pk[k];
    }
}

// Online-softmax update for one tile whose logits are sv + add (log2 domain, -inf = masked).  With
// ACC_L false the caller accumulates the sum of p itself (in one of the `extra` accumulators).
template <int NE = 0, bool ACC_L = true>
__device__ __forceinline__ void softmax_tile(WaveState& st, const float (&sv)[8], float (&pk)[8], int g,
                                             float add = 0.f, r2o_f4* extra = nullptr) {
    softmax_step<8, NE, ACC_L>(st, sv, pk, g, add, extra);
}

// PV for 16-bit V rows held as R[k] = 8 dims (8*l16 ..) of token tile_token(g, k).
template <int RF>
__device__ __forceinline__ void pv_rows(WaveState& st, const r2o_u4& ap, const r2o_u4 (&R)[8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const uint32_t sel = (q & 1) ? 0x07060302u : 0x05040100u;
        const r2o_u4 bop = {r2o_perm(R[1][q >> 1], R[0][q >> 1], sel), r2o_perm(R[3][q >> 1], R[2][q >> 1], sel),
                            r2o_perm(R[5][q >> 1], R[4][q >> 1], sel), r2o_perm(R[7][q >> 1], R[6][q >> 1], sel)};
        st.acc[q] = mfma_rows<RF>(ap, bop, st.acc[q]);
    }
}

// Constants kept in VGPRs so that (x & mask) | magic selects one v_and_or_b32 (gfx9 VOP3 can
// take at most one literal/SGPR operand).
struct VConst {
    uint32_t nib;     // 0x000F000F
    uint32_t nib_hi;  // 0x00F000F0
    uint32_t crumb;   // 0x00030003
    uint32_t magic;   // 0x64006400 = fp16 (1024, 1024)
};

__device__ __forceinline__ VConst make_vconst() {
    VConst c;
    asm volatile("v_mov_b32 %0, 0x000F000F" : "=v"(c.nib));
    asm volatile("v_mov_b32 %0, 0x00F000F0" : "=v"(c.nib_hi));
    asm volatile("v_mov_b32 %0, 0x00030003" : "=v"(c.crumb));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(c.magic));
    return c;
}

// ------------------------------------------------------------------ pool segment tiles
// Registers of one tile, read from its LDS stage: INT4-K codes of tokens 16 mg + l16 (channels
// 32g ..), the tile's K superblock operands of lane group g, and for each of the lane's 8 tokens
// tile_token(g, k) the 8 V dims 8*l16 .. 8*l16+7 (bf16: 16 B, INT4: 4 B, INT2: 2 B) plus the
// token's V metadata.
template <int KF>
struct KRegs;
template <>
struct KRegs<kKInt4> {  // INT4-K: codes of tokens 16 mg + l16 (channels 32g ..)
    r2o_u4 kx[2];
};
template <>
struct KRegs<kKBf16> {  // BF16-K: channels 32g + 8j .. 32g + 8j + 7 of tokens 16 mg + l16
    r2o_u4 kb[2][4];
};
template <>
struct KRegs<kKInt2> {  // INT2-K: codes of tokens 16 mg + l16 (channels 32g .., 8 bytes)
    uint32_t kx[2][2];
};
template <int KIND>
struct VRegs;
template <>
struct VRegs<kFP> {
    r2o_u4 v[8];
};
template <>
struct VRegs<kI4> {
    uint32_t v[8];
    uint32_t vm[8];  // f32 scale bits
};
template <>
struct VRegs<kI2> {
    uint32_t v[8];
    uint32_t vm[8];  // fp16 scale bits (group of dims 8*l16); one token per group: [pr] = pair (2pr, 2pr + 1)
    uint32_t vz[8];  // u8 zero point; one token per group: [pr] = z(2pr) | z(2pr + 1) << 16
};
template <int KIND, int KF>
struct TileRegs : KRegs<KF>, VRegs<KIND> {};

// Valid arena positions of the segment (partial tiles mask the rest).
struct SegCtx {
    int lo, hi;
};

template <int KIND>
struct SegState {
    uint32_t qp[4][4];   // q (scaled), f16 pairs in the K-unpack channel order
    r2o_f4 bias[KIND == kI2 ? 3 : 2];  // INT4-V: [0] = sum_k P'_k per head row; INT2-V with one group
                         // per token: [0] = sum_k P'_k (1024 + z_k), [1] = sum_k P'_k (code offsets and
                         // the in-place crumb factors removed at the end), [2] = sum_k p_k (the softmax
                         // denominator, from the same f16 p the P' are formed of)
};

// QK operands of one K superblock for the lane's channel group: Q'_j per MFMA j and the logit
// correction, which is the same for every token of a head and so a lane scalar added by the
// softmax.  They change only when a tile starts a new superblock (every tile at SB 32, every fourth
// at SB 128), so the tile loop keeps them across the tiles of a superblock.
struct QkOps {
    r2o_u4 q[4];
    float corr;
};

// INT4-K: Q'_j = q * s (superblock scale pairs; the pairs of high-nibble channels carry s / 16)
// and corr = -sum Q'_j (1024 + z) by one MFMA per j.  ko = the 4 scale-pair and the 4 zero-pair
// operand vectors of the lane's channel group.
__device__ __forceinline__ void qk_ops_int4k(const uint32_t (&qp)[4][4], const r2o_u4 (&ko)[8], QkOps& o) {
    r2o_f4 cz = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const r2o_u4 sj = ko[j];
        o.q[j] = r2o_u4{r2o_h2_mul(qp[j][0], sj[0]), r2o_h2_mul(qp[j][1], sj[1]), r2o_h2_mul(qp[j][2], sj[2]),
                        r2o_h2_mul(qp[j][3], sj[3])};
        cz = r2o_mfma_f16(ko[4 + j], o.q[j], cz);
    }
    o.corr = cz[0];  // every row of the correction product is the same
}

// QK^T of one INT4-K tile: the codes of the dword read in place (1024 + c for the low nibble of
// each byte, 1024 + 16 c for the high one) against Q'_j.
__device__ __forceinline__ void qk_int4k(const QkOps& o, const VConst& vc, const r2o_u4 (&kx)[2], r2o_f4 (&s)[2]) {
    s[0] = r2o_f4{0, 0, 0, 0};
    s[1] = r2o_f4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int mg = 0; mg < 2; ++mg) {
            const uint32_t w = kx[mg][j], w8 = w >> 8;
            const r2o_u4 a = {(w & vc.nib) | vc.magic, (w & vc.nib_hi) | vc.magic, (w8 & vc.nib) | vc.magic,
                              (w8 & vc.nib_hi) | vc.magic};
            s[mg] = r2o_mfma_f16(a, o.q[j], s[mg]);
        }
    }
}

// INT2-K (k = code * s + o per channel and superblock): Q'_j = q * s / 4^u for the crumb u each
// lane of MFMA j carries, and corr = sum_c q_c o_c - 1024 sum_c Q'_c by two MFMAs per j (the offset
// pairs against q, and -1024 against Q'_j, the very f16 values the code MFMAs use).  ko = the 4
// scale-pair and the 4 offset-pair vectors.
__device__ __forceinline__ void qk_ops_int2k(const uint32_t (&qp)[4][4], const r2o_u4 (&ko)[8], QkOps& o) {
    r2o_f4 cz = {0, 0, 0, 0};
    const r2o_u4 neg1024 = {0xE400E400u, 0xE400E400u, 0xE400E400u, 0xE400E400u};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const r2o_u4 sj = ko[j];
        const r2o_u4 qraw = {qp[j][0], qp[j][1], qp[j][2], qp[j][3]};
        o.q[j] = r2o_u4{r2o_h2_mul(qp[j][0], sj[0]), r2o_h2_mul(qp[j][1], sj[1]), r2o_h2_mul(qp[j][2], sj[2]),
                        r2o_h2_mul(qp[j][3], sj[3])};
        cz = r2o_mfma_f16(ko[4 + j], qraw, cz);
        cz = r2o_mfma_f16(neg1024, o.q[j], cz);
    }
    o.corr = cz[0];
}

// QK^T of one INT2-K tile: per MFMA j the codes of half a dword enter in place as 1024 + 4^u c
// (crumb u of bytes 0/2 or 1/3) against Q'_j.
__device__ __forceinline__ void qk_int2k(const QkOps& o, const VConst& vc, const uint32_t (&kx)[2][2],
                                         r2o_f4 (&s)[2]) {
    s[0] = r2o_f4{0, 0, 0, 0};
    s[1] = r2o_f4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int mg = 0; mg < 2; ++mg) {
            const uint32_t w = (j & 1) ? (kx[mg][j >> 1] >> 8) : kx[mg][j >> 1];
            const r2o_u4 a = {(w & vc.crumb) | vc.magic, (w & (vc.crumb << 2)) | vc.magic,
                              (w & (vc.crumb << 4)) | vc.magic, (w & (vc.crumb << 6)) | vc.magic};
            s[mg] = r2o_mfma_f16(a, o.q[j], s[mg]);
        }
    }
}

// Logits of a tile in the lane's token order (masks only on partial tiles; padded heads have
// q = 0, so their logits are 0: harmless, and their rows are never written out).
__device__ __forceinline__ void tile_logits(const SegCtx& c, int a0, int g, const r2o_f4 (&s)[2], float (&sv)[8]) {
    const bool full = __builtin_amdgcn_readfirstlane(a0 >= c.lo && a0 + 32 <= c.hi);
    if (full) {
#pragma unroll
        for (int k = 0; k < 8; ++k) sv[k] = s[k >> 2][k & 3];
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int pos = a0 + tile_token(g, k);
            sv[k] = ((pos >= c.lo) & (pos < c.hi)) ? s[k >> 2][k & 3] : -INFINITY;
        }
    }
}

// PV of one tile with probabilities pk (the lane's 8 tokens).
template <int KIND, bool TS, int RF>  // TS: INT2 values with one scale and zero point per token (group 128)
__device__ __forceinline__ void pv_tile(WaveState& st, SegState<KIND>& ss, const VConst& vc, const float (&pk)[8],
                                        const VRegs<KIND>& cur) {
    r2o_u4 ap;
    if constexpr (KIND == kFP) {
#pragma unroll
        for (int u = 0; u < 4; ++u) ap[u] = pack_row2<RF>(pk[2 * u], pk[2 * u + 1]);
        pv_rows<RF>(st, ap, cur.v);
    } else if constexpr (KIND == kI4) {
        // P' = p * s_t; the signed codes (xor 8) enter as 1032 + c (low nibble) and, read in
        // place, 1152 + 16 c (high nibble).  sum_k P'_k is accumulated by one more MFMA on the
        // same A operand (so both see identical f16 inputs) and the offsets are removed at the end.
#pragma unroll
        for (int u = 0; u < 4; ++u)
            ap[u] = r2o_pack_h2(pk[2 * u] * __uint_as_float(cur.vm[2 * u]), pk[2 * u + 1] * __uint_as_float(cur.vm[2 * u + 1]));
        ss.bias[0] = r2o_mfma_f16(ap, r2o_u4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u}, ss.bias[0]);
        uint32_t X[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) X[k] = cur.v[k] ^ 0x88888888u;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + bb) << 16) | (uint32_t)bb;
            r2o_u4 lo, hi;
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                const uint32_t y = r2o_perm(X[2 * pr + 1], X[2 * pr], sel);
                lo[pr] = (y & vc.nib) | vc.magic;
                hi[pr] = (y & vc.nib_hi) | vc.magic;
            }
            st.acc[2 * bb] = r2o_mfma_f16(ap, lo, st.acc[2 * bb]);
            st.acc[2 * bb + 1] = r2o_mfma_f16(ap, hi, st.acc[2 * bb + 1]);
        }
    } else if constexpr (TS) {
        // one scale and zero point per token (a group of all 128 dims): P' = p * s_t.  The crumbs
        // of dims q < 4 (bits 2q of each token's word) and q >= 4 (bits 8 + 2(q - 4)) enter in place,
        // from the token words and from them shifted by 8, as f16 1024 + 4^u c with u = q % 4, so
        // column q of the product carries 4^u sum P' c.  sum_k P'_k (1024 + z_k) and sum_k P'_k
        // accumulate by two more MFMAs on the same A operand; the offsets and the 4^u factors are
        // removed after the last tile.
        // p in f16 pairs, P' = p * s in packed f16 against the tokens' scale pairs; sum_k p_k accumulates
        // by one more MFMA (the softmax leaves l to it)
        r2o_u4 p2;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            p2[u] = r2o_pack_h2(pk[2 * u], pk[2 * u + 1]);
            ap[u] = r2o_h2_mul(p2[u], cur.vm[u]);
        }
        const r2o_u4 ones = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
        ss.bias[2] = r2o_mfma_f16(p2, ones, ss.bias[2]);
        uint32_t yp[4], y8[4];
        r2o_u4 zb;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
            yp[pr] = cur.v[2 * pr] | (cur.v[2 * pr + 1] << 16);
            y8[pr] = yp[pr] >> 8;
            zb[pr] = cur.vz[pr] | vc.magic;
        }
        ss.bias[0] = r2o_mfma_f16(ap, zb, ss.bias[0]);
        ss.bias[1] = r2o_mfma_f16(ap, ones, ss.bias[1]);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t mask = 0x00030003u << (2 * (q & 3));
            r2o_u4 bop;
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) bop[pr] = ((q < 4 ? yp[pr] : y8[pr]) & mask) | vc.magic;
            st.acc[q] = r2o_mfma_f16(ap, bop, st.acc[q]);
        }
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) ap[u] = r2o_pack_h2(pk[2 * u], pk[2 * u + 1]);
        uint32_t yp[4], zp[4], sp[4];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
            yp[pr] = cur.v[2 * pr] | (cur.v[2 * pr + 1] << 16);
            zp[pr] = (cur.vz[2 * pr] | (cur.vz[2 * pr + 1] << 16)) | vc.magic;
            sp[pr] = cur.vm[2 * pr] | (cur.vm[2 * pr + 1] << 16);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int shift = (q < 4) ? 2 * q : 8 + 2 * (q - 4);
            r2o_u4 bop;
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                const uint32_t cc = ((yp[pr] >> shift) & vc.crumb) | vc.magic;
                bop[pr] = r2o_h2_mul(r2o_h2_sub(cc, zp[pr]), sp[pr]);
            }
            st.acc[q] = r2o_mfma_f16(ap, bop, st.acc[q]);
        }
    }
}

// QK^T of one BF16-K tile: per MFMA j the bf16 key rows (channels 32g + 8j ..) against the bf16
// query pairs, scaled by D^-1/2 log2(e) afterwards (the recent-ring formulation).
template <int RF>
__device__ __forceinline__ void qk_bf16k(const uint32_t (&qp)[4][4], float qscale, const r2o_u4 (&kb)[2][4],
                                         r2o_f4 (&s)[2]) {
#pragma unroll
    for (int mg = 0; mg < 2; ++mg) {
        r2o_f4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = mfma_rows<RF>(kb[mg][j], r2o_u4{qp[j][0], qp[j][1], qp[j][2], qp[j][3]}, acc);
        s[mg] = acc * qscale;
    }
}

// One tile: QK, masks, online softmax, PV.
template <int KIND, int KF, bool TS, int RF>
__device__ __forceinline__ void seg_compute(const SegCtx& c, WaveState& st, SegState<KIND>& ss, const VConst& vc,
                                            int a0, int g, float qscale, const QkOps& qo,
                                            const TileRegs<KIND, KF>& cur) {
    r2o_f4 s[2];
    float corr = 0.f;
    if constexpr (KF == kKBf16) qk_bf16k<RF>(ss.qp, qscale, cur.kb, s);
    else if constexpr (KF == kKInt4) qk_int4k(qo, vc, cur.kx, s);
    else qk_int2k(qo, vc, cur.kx, s);
    if constexpr (KF != kKBf16) corr = qo.corr;
    float sv[8], pk[8];
    tile_logits(c, a0, g, s, sv);
    softmax_tile<TS ? 3 : (KIND == kI4 ? 1 : 0), !TS>(st, sv, pk, g, corr, ss.bias);
    pv_tile<KIND, TS, RF>(st, ss, vc, pk, cur);
}

// ------------------------------------------------------------------ pool tiles via LDS DMA
// Every pool tile is moved by global->LDS DMA (16-byte chunks; no VGPRs held while in flight)
// into one stage of a per-wave ring of kDmaStages stages.  The wave waits for tile i, reads the
// whole stage into registers, refills the stage with tile i + kDmaStages, then computes tile i,
// so kDmaStages tiles stay in flight during the compute.  The 16-byte chunks are placed so that
// the transposed per-lane reads hit distinct LDS banks (see the slot functions).  A DMA of 16
// bytes per lane fills LDS at lane * 16; one of 1, 2 or 4 bytes per lane fills the low bytes of
// the dword at lane * 4, so sub-dword metadata rows sit in dword slots.
template <int KIND, int KF>
struct StageLayout {  // byte offsets within a stage: K | V payload | K operands (INT4/INT2-K) | V metadata
    static constexpr bool kBK = KF == kKBf16;
    static constexpr int kKBytes = kBK ? 8192 : (KF == kKInt4 ? 2048 : 1024);
    static constexpr int kV = kKBytes;
    static constexpr int kVBytes = KIND == kFP ? 8192 : (KIND == kI4 ? 2048 : 1024);
    static constexpr int kOps = kV + kVBytes;                  // INT4-K and INT2-K only
    static constexpr int kScale = kBK ? kV + kVBytes : kOps + 512;
    static constexpr int kZero = kScale + 256;                 // INT2 only
    static constexpr int kDma = kKBytes / 1024 + kVBytes / 1024 + (kBK ? 0 : 1) + (KIND == kFP ? 0 : (KIND == kI4 ? 1 : 2));
    static constexpr int kEnd = KIND == kFP ? kScale : (KIND == kI4 ? kScale + 128 : kZero + 128);
};
template <int KF>
constexpr bool stages_fit() {
    return StageLayout<kFP, KF>::kEnd <= KernelCfg<KF>::kStage && StageLayout<kI4, KF>::kEnd <= KernelCfg<KF>::kStage &&
           StageLayout<kI2, KF>::kEnd <= KernelCfg<KF>::kStage;
}
static_assert(stages_fit<kKInt4>() && stages_fit<kKBf16>() && stages_fit<kKInt2>(),
              "every tile stage fits its kernel's stage size");

// K codes: token t (0..31), 16-byte chunk c (0..3) of its 64-byte row.  Reads: 8 lanes take 8
// consecutive tokens of one chunk, so the chunk is rotated by (t >> 1) & 3.
__device__ __forceinline__ int k_slot(int t, int c) { return 4 * t + (c ^ ((t >> 1) & 3)); }
// INT4 V: token t, chunk c (0..3) of its 64-byte row.  Reads: 32 lanes take chunks 0..3 of
// tokens t and t + 4, which land in distinct 16-byte bank groups.
__device__ __forceinline__ int v4_slot(int t, int c) { return 8 * ((t & 3) + 4 * (t >> 3)) + 2 * c + ((t >> 2) & 1); }
// INT2 V: token t, chunk c (0..1) of its 32-byte row; tokens t, t+4, t+8, t+12 share 8 slots.
__device__ __forceinline__ int v2_slot(int t, int c) { return 8 * (t & 3) + 32 * (t >> 4) + 2 * ((t >> 2) & 3) + c; }
// INT2-K codes: token t, chunk c (0..1) of its 32-byte row.  Reads: 16 lanes take 8 bytes of one
// chunk of 16 consecutive tokens, so tokens 8..15 of a group swap their two chunks.  (Their 16-lane
// passes still meet 2-way bank conflicts, which a layout cannot remove while 16 lanes read the same
// half of 16 chunks; reading each chunk once with 16 bytes a lane and two row swaps removes them, but
// the swaps cost this VALU-bound loop more than the conflicts do.)
__device__ __forceinline__ int k2_slot(int t, int c) { return 2 * t + (c ^ ((t >> 3) & 1)); }
// BF16 V rows stay in natural order: 8 lanes read 8 consecutive chunks of one 256-byte row.
// BF16 K: token t, chunk c (0..15) of its 256-byte row.  Reads: 8 lanes take one chunk of 8
// consecutive tokens, so the chunk is rotated by t.
__device__ __forceinline__ int kb_slot(int t, int c) { return 16 * t + (c ^ (t & 15)); }

template <int SIZE>
__device__ __forceinline__ void dma(const void* gsrc, unsigned char* lds) {
    const auto g = (const __attribute__((address_space(1))) void*)gsrc;
    const auto l = (__attribute__((address_space(3))) void*)lds;
    constexpr int kNT = 2;  // cache policy: nontemporal (each KV byte is read once per call)
    if constexpr (SIZE == 16) __builtin_amdgcn_global_load_lds(g, l, 16, 0, kNT);
    else if constexpr (SIZE == 4) __builtin_amdgcn_global_load_lds(g, l, 4, 0, kNT);
    else if constexpr (SIZE == 2) __builtin_amdgcn_global_load_lds(g, l, 2, 0, kNT);
    else __builtin_amdgcn_global_load_lds(g, l, 1, 0, kNT);
}

constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Wait until at most `later` tiles of PER DMAs each are still in flight.
template <int PER>
__device__ __forceinline__ void wait_tiles(int later) {
    static_assert(kDmaStages <= 3 && 2 * PER < 64, "vmcnt holds the DMAs of two later tiles");
    if (later >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER));
    else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

struct DmaCtx {
    const uint8_t* kcode;   // K codes of this head
    const uint32_t* kops;   // K superblock operands of this head
    const uint8_t* vrows;   // V rows of this head
    const uint8_t* vscale;  // V scales of this head (bytes)
    const uint8_t* vzero;   // INT2 zero points of this head
    int lo, hi, vdelta, sb_shift, groups;
    int koff0, koff1;       // this lane's K source offset (bytes) for the K DMAs (INT4: two, INT2: one)
    int vt0, vt1, vc0, vc1; // this lane's V source token / chunk for the INT V DMAs
};

template <int KIND, int KF>
__device__ __forceinline__ void dma_tile(const DmaCtx& c, int a0, unsigned char* stage, int lane, bool ops = true) {
    using Lay = StageLayout<KIND, KF>;
    if constexpr (KF == kKBf16) {  // 8 x 1 KB of bf16 rows: slot s = 64 j + lane holds chunk c of token t
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int sl = 64 * j + lane, t = sl >> 4, ch = (sl & 15) ^ (t & 15);
            dma<16>(c.kcode + (a0 + t) * 256 + ch * 16, stage + 1024 * j);
        }
    } else if constexpr (KF == kKInt4) {
        dma<16>(c.kcode + a0 * 64 + c.koff0, stage);
        dma<16>(c.kcode + a0 * 64 + c.koff1, stage + 1024);
    } else {
        dma<16>(c.kcode + a0 * 32 + c.koff0, stage);
    }
    const bool full = __builtin_amdgcn_readfirstlane(a0 >= c.lo && a0 + 32 <= c.hi);  // wave-uniform
    // rows outside [lo, hi) read a clamped valid row (finite data, probability 0)
    auto row = [&](int t) { return (full ? a0 + t : min(max(a0 + t, c.lo), c.hi - 1)) - c.vdelta; };
    if constexpr (KIND == kFP) {  // 8 x 1 KB: instruction j covers tokens 4j..4j+3 (16 chunks each)
#pragma unroll
        for (int j = 0; j < 8; ++j) dma<16>(c.vrows + row(4 * j + (lane >> 4)) * 256 + (lane & 15) * 16, stage + Lay::kV + 1024 * j);
    } else if constexpr (KIND == kI4) {
        dma<16>(c.vrows + row(c.vt0) * 64 + c.vc0 * 16, stage + Lay::kV);
        dma<16>(c.vrows + row(c.vt1) * 64 + c.vc1 * 16, stage + Lay::kV + 1024);
    } else {
        dma<16>(c.vrows + row(c.vt0) * 32 + c.vc0 * 16, stage + Lay::kV);
    }
    if constexpr (KF != kKBf16)  // the tile's superblock operands, when the tile loop needs them
        if (ops && lane < 32) dma<16>(c.kops + (a0 >> c.sb_shift) * 128 + lane * 4, stage + Lay::kOps);
    if constexpr (KIND == kI4) {
        if (lane < 32) dma<4>(c.vscale + row(lane) * 4, stage + Lay::kScale);
    } else if constexpr (KIND == kI2) {
        if (c.groups == 4) {  // G = 32: 8-byte scale rows, 4-byte zero rows
            dma<4>(c.vscale + row(lane >> 1) * 8 + (lane & 1) * 4, stage + Lay::kScale);
            if (lane < 32) dma<4>(c.vzero + row(lane) * 4, stage + Lay::kZero);
        } else if (c.groups == 2) {
            if (lane < 32) dma<4>(c.vscale + row(lane) * 4, stage + Lay::kScale);
            if (lane < 32) dma<2>(c.vzero + row(lane) * 2, stage + Lay::kZero);
        } else {
            if (lane < 32) dma<2>(c.vscale + row(lane) * 2, stage + Lay::kScale);
            if (lane < 32) dma<1>(c.vzero + row(lane), stage + Lay::kZero);
        }
    }
}

// The K superblock operand vectors of lane group g (INT4-K and INT2-K stages).
template <int KIND, int KF>
__device__ __forceinline__ void read_ops(const unsigned char* stage, int g, r2o_u4 (&ko)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        ko[j] = *reinterpret_cast<const r2o_u4*>(stage + StageLayout<KIND, KF>::kOps + g * 128 + 16 * j);
}

template <int KIND, int KF, bool TS = false>
__device__ __forceinline__ void read_tile(const unsigned char* stage, int l16, int g, int gamma, int groups,
                                          TileRegs<KIND, KF>& tr) {
    using Lay = StageLayout<KIND, KF>;
    if constexpr (KF == kKBf16) {
#pragma unroll
        for (int mg = 0; mg < 2; ++mg)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                tr.kb[mg][j] = *reinterpret_cast<const r2o_u4*>(stage + 16 * kb_slot(16 * mg + l16, 4 * g + j));
    } else {
#pragma unroll
        for (int mg = 0; mg < 2; ++mg) {
            if constexpr (KF == kKInt4) {
                tr.kx[mg] = *reinterpret_cast<const r2o_u4*>(stage + 16 * k_slot(16 * mg + l16, g));
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(stage + 16 * k2_slot(16 * mg + l16, g >> 1) + 8 * (g & 1));
                tr.kx[mg][0] = w.x;
                tr.kx[mg][1] = w.y;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int t = tile_token(g, k);
        if constexpr (KIND == kFP) {
            tr.v[k] = *reinterpret_cast<const r2o_u4*>(stage + Lay::kV + 256 * t + 16 * l16);
        } else if constexpr (KIND == kI4) {
            tr.v[k] = *reinterpret_cast<const uint32_t*>(stage + Lay::kV + 16 * v4_slot(t, l16 >> 2) + 4 * (l16 & 3));
            tr.vm[k] = *reinterpret_cast<const uint32_t*>(stage + Lay::kScale + 4 * t);
        } else if constexpr (TS) {  // one group per token: scales and zeros of tokens t, t + 1 (t even) together
            tr.v[k] = *reinterpret_cast<const uint16_t*>(stage + Lay::kV + 16 * v2_slot(t, l16 >> 3) + 2 * (l16 & 7));
            if ((k & 1) == 0) {  // one dword slot per token: the 8 bytes at 4t hold both tokens' slots
                const uint2 sc = *reinterpret_cast<const uint2*>(stage + Lay::kScale + 4 * t);
                const uint2 zr = *reinterpret_cast<const uint2*>(stage + Lay::kZero + 4 * t);
                tr.vm[k >> 1] = r2o_perm(sc.y, sc.x, 0x05040100u);  // (s_t, s_t+1) as an f16 pair
                tr.vz[k >> 1] = r2o_perm(zr.y, zr.x, 0x0C040C00u);  // z_t | z_t+1 << 16
            }
        } else {  // scale rows: 8 bytes (G = 32) or one dword slot; zero rows: one dword slot
            tr.v[k] = *reinterpret_cast<const uint16_t*>(stage + Lay::kV + 16 * v2_slot(t, l16 >> 3) + 2 * (l16 & 7));
            tr.vm[k] = *reinterpret_cast<const uint16_t*>(stage + Lay::kScale + t * (groups == 4 ? 8 : 4) + 2 * gamma);
            tr.vz[k] = *(stage + Lay::kZero + 4 * t + gamma);
        }
    }
}

// Slot ranges of up to kInlineGroups groups travel in the combine launch's own arguments, next
// to r2o_decode_params: a merge block's partial loads then wait on nothing but the launch
// arguments (reading group_begin from device memory first cost one more dependent round trip).
constexpr int kInlineGroups = 32;
struct CombineArgs {
    int32_t n_groups;                  // groups whose range is below; 0: read p.group_begin
    int32_t gqa;                       // query heads per KV head
    int32_t begin[kInlineGroups + 1];  // slots of group g: [begin[g], begin[g + 1])
};

// The first read of each 64-byte line of the launch arguments waits on memory.  The combine kernel
// reads every argument word its merge path uses at entry (partial pointers and n_items, output
// pointer, output_hadamard, the head count and the block's inline slot range, which may sit on a
// line of its own), so that those misses overlap instead of each one queueing behind the loads
// that first use its line.  (The partial kernel reads lines 0x00 and 0x40 at entry by itself;
// forcing line 0x80 there as well measured slower.)
__device__ __forceinline__ void touch_combine_kernarg(const r2o_decode_params& p, const CombineArgs& ca,
                                                      int range_begin, int range_end) {
    asm volatile("" ::"s"(p.partial_out), "s"(p.partial_max), "s"(p.partial_sum), "s"(p.n_items), "s"(p.out),
                 "s"(p.output_hadamard), "s"(ca.gqa), "s"(ca.n_groups), "s"(range_begin), "s"(range_end));
}

template <int KIND, int KF, bool TS, int RF, int RO>
__device__ __forceinline__ void run_segment(const r2o_decode_params& p, const r2o_work_item& it,
                                            unsigned char* smem, WaveState& st, Stamps& ts) {
    using Cfg = KernelCfg<KF>;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
    const int gqa = __builtin_amdgcn_readfirstlane(r2o_div_small((int)p.hq, (int)p.hkv));
    const int64_t kvh = it.kvh, b = it.req;
    const int per = (int)((it.ntiles + Cfg::kWaves - 1) / Cfg::kWaves);
    const int t_begin = wave * per;
    const int t_end = min((int)it.ntiles, t_begin + per);
    if constexpr (RO == kRopeNone) {
        if (t_begin >= t_end) return;
    }  // with a folded rotation a wave without tiles still rotates its rows and meets the barrier
    unsigned char* ring = smem + wave * Cfg::kWaveLds;

    DmaCtx c;
    c.kcode = reinterpret_cast<const uint8_t*>(it.k_base);
    c.kops = it.k_ops;
    c.lo = (int)it.lo;
    c.hi = (int)it.hi;
    c.vdelta = (int)it.v_delta;
    c.sb_shift = p.superblock == 32 ? 5 : (p.superblock == 64 ? 6 : 7);
    const int g_shift = it.v_group == 32 ? 5 : (it.v_group == 64 ? 6 : 7);  // INT2-V only
    c.groups = 128 >> g_shift;
    const int gamma = (8 * l16) >> g_shift;
    c.vrows = reinterpret_cast<const uint8_t*>(it.v_base);
    c.vscale = reinterpret_cast<const uint8_t*>(it.v_scale);
    c.vzero = it.v_zero;
    {  // lane -> (token, chunk) sources of the K and INT V DMAs (inverse of the slot functions)
        const int s0 = lane, s1 = 64 + lane;
        const int t0 = s0 >> 2, t1 = s1 >> 2;
        if constexpr (KF == kKInt2) {  // one 1 KB DMA: slot s holds chunk (s & 1) ^ ((t >> 3) & 1) of token s >> 1
            c.koff0 = (s0 >> 1) * 32 + 16 * ((s0 & 1) ^ ((s0 >> 4) & 1));
            c.koff1 = 0;
        } else {
            c.koff0 = t0 * 64 + 16 * ((s0 & 3) ^ ((t0 >> 1) & 3));
            c.koff1 = t1 * 64 + 16 * ((s1 & 3) ^ ((t1 >> 1) & 3));
        }
        if constexpr (KIND == kI2) {
            c.vt0 = 16 * (s0 >> 5) + 4 * ((s0 >> 1) & 3) + ((s0 >> 3) & 3);
            c.vc0 = s0 & 1;
            c.vt1 = c.vt0;
            c.vc1 = c.vc0;
        } else {
            c.vt0 = 8 * (s0 >> 5) + 4 * (s0 & 1) + ((s0 >> 3) & 3);
            c.vc0 = (s0 >> 1) & 3;
            c.vt1 = 8 * (s1 >> 5) + 4 * (s1 & 1) + ((s1 >> 3) & 3);
            c.vc1 = (s1 >> 1) & 3;
        }
    }
    const int n = t_end - t_begin;
    const int a_first = (int)it.tile0 + 32 * t_begin;
    // With one stage per wave the superblock operands are moved and read only for the first tile of
    // the wave and of each superblock (a ring of more stages moves them with every tile, so that
    // its wait counts stay fixed).
    const int sb_mask = (1 << c.sb_shift) - 1;
    auto needs_ops = [&](int i) { return kDmaStages > 1 || i == 0 || ((a_first + 32 * i) & sb_mask) == 0; };
#pragma unroll
    for (int j = 0; j < kDmaStages; ++j)
        if (j < n) dma_tile<KIND, KF>(c, a_first + 32 * j, ring + j * Cfg::kStage, lane, true);
    stamp(ts, 2);
    r2o_u4 qrot[4];
    if constexpr (RO != kRopeNone) {  // the waves share the rotation while their first tiles are in flight
        uint16_t* rot = reinterpret_cast<uint16_t*>(smem + Cfg::kSmem);
        const int r = 4 * wave + (lane >> 4);
        if (r < gqa) {  // whole 16-lane groups
            RotPrefetch f;
            rot_prefetch<RO>(p, b, query_row<RO>(p, b, kvh, gqa, r), l16, f);
            rot_block_row<RO>(p, b, kvh, gqa, r, l16, f, rot);
        }
        __syncthreads();
        if (n <= 0) return;
        rot_read_query(rot, gqa, l16, g, qrot);
    }

    const VConst vc = make_vconst();
    const float qscale = p.sm_scale * kLog2e;
    SegState<KIND> ss;
    load_query<KF, RF, RO>(p, b, kvh, gqa, l16, g, qscale, ss.qp, qrot);  // BF16-K: row-type pairs, scaled after the MFMA
#pragma unroll
    for (int e = 0; e < (KIND == kI2 ? 3 : 2); ++e) ss.bias[e] = r2o_f4{0, 0, 0, 0};
    const SegCtx sc = {c.lo, c.hi};
    QkOps qo;  // operands of the current K superblock (INT4-K / INT2-K)
    for (int i = 0; i < n; ++i) {
        wait_tiles<StageLayout<KIND, KF>::kDma>(min(kDmaStages, n - i) - 1);  // tile i has landed
        __builtin_amdgcn_wave_barrier();
        if (i == 0) stamp(ts, 3);
        if (i == n - 1) stamp(ts, 4);
        unsigned char* stage = ring + (i % kDmaStages) * Cfg::kStage;
        TileRegs<KIND, KF> cur;
        read_tile<KIND, KF, TS>(stage, l16, g, gamma, c.groups, cur);
        const bool fresh = __builtin_amdgcn_readfirstlane(needs_ops(i));  // wave-uniform
        r2o_u4 ko[8];
        if constexpr (KF != kKBf16)
            if (fresh) read_ops<KIND, KF>(stage, g, ko);
        if (i + kDmaStages < n) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the whole stage is in registers
            __builtin_amdgcn_wave_barrier();
            dma_tile<KIND, KF>(c, a_first + 32 * (i + kDmaStages), stage, lane, needs_ops(i + kDmaStages));
        }
        if constexpr (KF == kKInt4) {
            if (fresh) qk_ops_int4k(ss.qp, ko, qo);
        } else if constexpr (KF == kKInt2) {
            if (fresh) qk_ops_int2k(ss.qp, ko, qo);
        }
        seg_compute<KIND, KF, TS, RF>(sc, st, ss, vc, a_first + 32 * i, g, qscale, qo, cur);
    }
    if constexpr (TS) {  // column q = 4^-u (sum P' (1024 + 4^u c)) - sum P' (1024 + z) + 1024 (1 - 4^-u) sum P'
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float f = 1.f / (float)(1 << (2 * (q & 3)));
            st.acc[q] = st.acc[q] * f - ss.bias[0] + ss.bias[1] * (1024.f * (1.f - f));
        }
        // sum p of head 4g' + i sits in row i of every lane of group g'; the epilogue expects head l16's
        // share in lanes l16 + 16 g, summed over g: lane 16 (l16 >> 2) + l16 holds it as row l16 & 3
        const int r = l16 & 3;
        const float mine = r == 0 ? ss.bias[2][0] : (r == 1 ? ss.bias[2][1] : (r == 2 ? ss.bias[2][2] : ss.bias[2][3]));
        const float head_l = __shfl(mine, 16 * (l16 >> 2) + l16, R2O_WAVE);
        st.l = g == 0 ? head_l : 0.f;
    }
    if constexpr (KIND == kI4) {  // remove the code offsets: lo dims 1032 * sum P', hi dims (1152 * sum P') / 16
#pragma unroll
        for (int q = 0; q < 8; q += 2) {
            st.acc[q] -= 1032.f * ss.bias[0];
            st.acc[q + 1] = (st.acc[q + 1] - 1152.f * ss.bias[0]) * 0.0625f;
        }
    }
}

// Recent-FP ring tiles (bf16 K and V, plus the fused-append token).  Every load of a tile is
// issued before any is used (rows past the valid end read the last valid row, whose
// probability is 0); a tile with no valid token is skipped.  With a folded rotation (RO) the item's
// waves rotate the query heads and the appended K and V rows together (rot_block_row, which also
// stores the appended rows for the combine's fused append), and the tile holding the appended token
// takes its rows from LDS.
template <int KF, int RF, int RO>
__device__ __forceinline__ void run_recent(const r2o_decode_params& p, const r2o_work_item& it,
                                           unsigned char* smem, WaveState& st) {
    constexpr int kWaves = KernelCfg<KF>::kWaves;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
    const int gqa = __builtin_amdgcn_readfirstlane(r2o_div_small((int)p.hq, (int)p.hkv));
    const int64_t kvh = it.kvh, b = it.req;
    const int per = (int)((it.ntiles + kWaves - 1) / kWaves);
    const int t_begin = wave * per;
    const int t_end = min((int)it.ntiles, t_begin + per);
    // device-state mode: the ring length lives in device memory (advanced by the previous step's
    // combine), so a captured launch stays valid from step to step
    const int recent_len = min(p.step_positions ? *it.ring_length : p.recent_len[b], (int)it.hi);
    const bool app = p.do_append != 0;
    const int valid_end = recent_len + (app ? 1 : 0);
    uint16_t* rot = reinterpret_cast<uint16_t*>(smem + KernelCfg<KF>::kSmem);
    if constexpr (RO != kRopeNone) {  // every wave, before any returns: the rows meet in LDS
        const int nrows = gqa + (app ? 2 : 0);
        for (int r0 = 4 * wave; r0 < nrows; r0 += 16) {  // wave-uniform
            const int r = r0 + (lane >> 4);
            if (r < nrows) {  // whole 16-lane groups
                RotPrefetch f;
                rot_prefetch<RO>(p, b, rot_source(p, b, kvh, gqa, r), l16, f);
                rot_block_row<RO>(p, b, kvh, gqa, r, l16, f, rot);
            }
        }
        __syncthreads();
    }
    if (t_begin >= t_end || valid_end == 0) return;
    const float qscale = p.sm_scale * kLog2e;
    const bool head_ok = l16 < gqa;
    uint32_t qp[4][4];
    r2o_u4 qrot[4];
    if constexpr (RO != kRopeNone) rot_read_query(rot, gqa, l16, g, qrot);
    load_query<kKBf16, RF, RO>(p, b, kvh, gqa, l16, g, qscale, qp, qrot);
    // folded rotation: the tile holding the appended token takes the rotated rows from LDS
    const int t_new = RO != kRopeNone && app && recent_len >= (int)it.tile0 ? (recent_len - (int)it.tile0) >> 5 : -1;
    const uint16_t* ring_k = reinterpret_cast<const uint16_t*>(it.k_base);
    const uint16_t* ring_v = reinterpret_cast<const uint16_t*>(it.v_base);
    // (with a folded rotation the appended token's rows come from LDS: ring row 0 stands in)
    const uint16_t* new_k = app && RO == kRopeNone ? p.append_k + (b * p.hkv + kvh) * 128 : ring_k;
    const uint16_t* new_v = app && RO == kRopeNone ? p.append_v + (b * p.hkv + kvh) * 128 : ring_v;
    for (int t = t_begin; t < t_end; ++t) {
        const int a0 = (int)it.tile0 + 32 * t;
        if (a0 >= valid_end) break;  // wave-uniform
        r2o_u4 kr[2][4], R[8];
#pragma unroll
        for (int mg = 0; mg < 2; ++mg) {
            const int slot = min(a0 + 16 * mg + l16, valid_end - 1);
            const uint16_t* krow = slot == recent_len ? new_k : ring_k + slot * 128;
#pragma unroll
            for (int j = 0; j < 4; ++j) kr[mg][j] = r2o_ldg(reinterpret_cast<const r2o_u4*>(krow + 32 * g) + j);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int slot = min(a0 + tile_token(g, k), valid_end - 1);
            const uint16_t* vrow = slot == recent_len ? new_v : ring_v + slot * 128;
            R[k] = r2o_ldg(reinterpret_cast<const r2o_u4*>(vrow + 8 * l16));
        }
        if constexpr (RO != kRopeNone) {
            if (t == t_new) {  // wave-uniform: the appended token's tile takes its rotated rows
                const r2o_u4* nk = reinterpret_cast<const r2o_u4*>(rot + kRotKeyRow * kRotStride + 32 * g);
                const r2o_u4 nv = *reinterpret_cast<const r2o_u4*>(rot + (kRotKeyRow + 1) * kRotStride + 8 * l16);
#pragma unroll
                for (int mg = 0; mg < 2; ++mg) {
                    const bool mine = min(a0 + 16 * mg + l16, valid_end - 1) == recent_len;
#pragma unroll
                    for (int j = 0; j < 4; ++j) kr[mg][j] = mine ? nk[j] : kr[mg][j];
                }
#pragma unroll
                for (int k = 0; k < 8; ++k) R[k] = min(a0 + tile_token(g, k), valid_end - 1) == recent_len ? nv : R[k];
            }
        }
        r2o_f4 s[2];
#pragma unroll
        for (int mg = 0; mg < 2; ++mg) {
            r2o_f4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = mfma_rows<RF>(kr[mg][j], r2o_u4{qp[j][0], qp[j][1], qp[j][2], qp[j][3]}, acc);
            s[mg] = acc * qscale;
        }
        float sv[8], pk[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) sv[k] = ((a0 + tile_token(g, k) < valid_end) & head_ok) ? s[k >> 2][k & 3] : -INFINITY;
        softmax_tile(st, sv, pk, g);
        r2o_u4 ap;
#pragma unroll
        for (int u = 0; u < 4; ++u) ap[u] = pack_row2<RF>(pk[2 * u], pk[2 * u + 1]);
        pv_rows<RF>(st, ap, R);
    }
}

template <int KF, int RF, int RO>
__global__ __launch_bounds__(KernelCfg<KF>::kThreads, KernelCfg<KF>::kWavesPerSimd) void decode_partial_kernel(
        r2o_decode_params p) {
    constexpr int kWaves = KernelCfg<KF>::kWaves;
    __shared__ __align__(16) unsigned char smem[KernelCfg<KF>::kSmem + (RO != kRopeNone ? kRotBytes : 0)];
    Stamps ts{};
    stamp(ts, 0);
    const r2o_work_item it = p.items[blockIdx.x];
#ifdef R2O_TIMELINE
    {
        const int64_t kind0 = it.kind;
        asm volatile("s_waitcnt lgkmcnt(0)" ::"s"(kind0) : "memory");
        stamp(ts, 1);
        ts.t[7] = (unsigned long long)__builtin_amdgcn_s_getreg((3 << 11) | 20) |          // XCC_ID
                  ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 4) << 32);   // HW_ID
        ts.t[8] = (unsigned long long)(uint32_t)it.ntiles | ((unsigned long long)(uint32_t)it.kind << 32);
    }
#endif
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
    const int gqa = __builtin_amdgcn_readfirstlane(r2o_div_small((int)p.hq, (int)p.hkv));

    WaveState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) st.acc[q] = r2o_f4{0, 0, 0, 0};

    switch (it.kind) {
        case kFP: run_segment<kFP, KF, false, RF, RO>(p, it, smem, st, ts); break;
        case kI4: run_segment<kI4, KF, false, RF, RO>(p, it, smem, st, ts); break;
        case kI2:  // INT2 values: one scale and zero point per token when a group spans all 128 dims
            if (it.v_group == 128) run_segment<kI2, KF, true, RF, RO>(p, it, smem, st, ts);
            else run_segment<kI2, KF, false, RF, RO>(p, it, smem, st, ts);
            break;
        default: run_recent<KF, RF, RO>(p, it, smem, st); break;
    }

    // ---- per-wave epilogue: reduce l (and u) over the 4 lane groups of each head
    float l_h = st.l;
    l_h = r2o_sum_lane_pair<16>(l_h);
    l_h = r2o_sum_lane_pair<32>(l_h);
    stamp(ts, 5);
    // each wave's state goes to the start of its own DMA ring, whose tiles it has all read: no wave
    // waits for the others before writing (one barrier less than a shared merge area)
    constexpr int kWaveFloats = KernelCfg<KF>::kWaveLds / 4;
    static_assert(KernelCfg<KF>::kWaveLds >= kMergeFloats * 4, "a wave's state fits its own ring");
    float* mrg = reinterpret_cast<float*>(smem) + wave * kWaveFloats;
    if (g == 0) {
        mrg[l16] = st.m;
        mrg[16 + l16] = l_h;
    }
    // rows 4g + i of the accumulator (the padded heads past the KV group are not needed): the
    // lane's 8 dims 8 l16 .. 8 l16 + 7 of a row are two 16-byte LDS writes
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (4 * g + i < gqa) {
            r2o_f4* row = reinterpret_cast<r2o_f4*>(mrg + 32 + (4 * g + i) * 128 + 8 * l16);
            row[0] = r2o_f4{st.acc[0][i], st.acc[1][i], st.acc[2][i], st.acc[3][i]};
            row[1] = r2o_f4{st.acc[4][i], st.acc[5][i], st.acc[6][i], st.acc[7][i]};
        }
    }
    __syncthreads();

    // ---- merge the 4 wave states of this block and write the partial: 4 dims per thread
    // (the planner numbers the slots 0 .. n_items - 1; a slot outside that range writes nothing)
    const float* base = reinterpret_cast<const float*>(smem);
    const int nmerge = (it.slot >= 0 && it.slot < p.n_items) ? gqa * 32 : 0;
    for (int e = threadIdx.x; e < nmerge; e += blockDim.x) {
        const int h = e >> 5, d4 = (e & 31) * 4;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, base[w * kWaveFloats + h]);
        float L = 0.f;
        r2o_f4 A = {0.f, 0.f, 0.f, 0.f};
        if (M != -INFINITY) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float mw = base[w * kWaveFloats + h];
                const float sc = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
                L += base[w * kWaveFloats + 16 + h] * sc;
                A += *reinterpret_cast<const r2o_f4*>(base + w * kWaveFloats + 32 + h * 128 + d4) * sc;
            }
        }
        // plain (write-back) stores: the end-of-kernel writeback leaves the partials in the Infinity
        // Cache, where the combine launch reads them.  Streaming (non-temporal) stores shorten this
        // kernel by ~0.6 us but send them to DRAM, and the combine's reads then cost more than that
        // (cfg2 layer call 24.3 vs 23.7 us); write-through stores are slower still.
        const int64_t slot = it.slot * 16 + h;
        *reinterpret_cast<r2o_f4*>(p.partial_out + slot * 128 + d4) = A;
        if (d4 == 0) {
            p.partial_max[slot] = M;
            p.partial_sum[slot] = L;
        }
    }
    stamp(ts, 6);
#ifdef R2O_TIMELINE
    stamps_store(g_timeline_partial, blockIdx.x, wave, kTimelineWaves, ts);
#endif
}

// Fused Recent-FP append (triton_fourq_splitk.py:1007-1020) of every KV head of request b, by one
// extra block of the combine grid: no merge block reads the ring, and this block is the only reader
// and writer of the ring length (and, in device-state mode, of the step positions) during the launch.
// 16-byte pieces of one token's K (or V) rows of every KV head that each combine thread moves:
// 4 x 512 threads cover hkv <= 128 (checked on the host).
constexpr int kAppendPieces = 4;

__device__ __forceinline__ void fused_append(const r2o_decode_params& p, int64_t b, int tid) {
    const r2o_request_desc& rq = p.reqs[b];
    // Every load that does not depend on the ring position is issued before it is known: the
    // appended rows (16 bytes a piece) and this step's (global, logical) positions.
    const int pieces = (int)p.hkv * 16;
    const r2o_u4* src_k = reinterpret_cast<const r2o_u4*>(p.append_k + b * p.hkv * 128);  // dense rows (the
    const r2o_u4* src_v = reinterpret_cast<const r2o_u4*>(p.append_v + b * p.hkv * 128);  // rotated ones too)
    r2o_u4 rk[kAppendPieces], rv[kAppendPieces];
#pragma unroll
    for (int k = 0; k < kAppendPieces; ++k) {  // unconditional loads (clamped index), guarded stores
        const int e = min(tid + k * (int)blockDim.x, pieces - 1);
        rk[k] = r2o_ldg(src_k + e);
        rv[k] = r2o_ldg(src_v + e);
    }
    int64_t gidx = 0, lpos = 0;
    if (tid == 0) {
        if (p.step_positions) {  // this step's positions, advanced for the next replay
            gidx = p.step_positions[2 * b];
            lpos = p.step_positions[2 * b + 1];
        } else {
            gidx = p.append_global[b];
            lpos = p.append_logical[b];
        }
    }
    const int64_t pos = p.step_positions ? (int64_t)*rq.recent_length : p.recent_len[b];
    if (pos >= rq.recent_capacity) return;  // a full ring takes no append (the host flushes first)
#pragma unroll
    for (int k = 0; k < kAppendPieces; ++k) {
        const int e = tid + k * (int)blockDim.x;
        if (e < pieces) {
            const int64_t hh = e >> 4, c = e & 15;
            const int64_t row = (hh * rq.recent_capacity + pos) * 16 + c;  // in 16-byte pieces
            reinterpret_cast<r2o_u4*>(rq.recent_k)[row] = rk[k];
            reinterpret_cast<r2o_u4*>(rq.recent_v)[row] = rv[k];
        }
    }
    if (tid == 0) {
        if (p.step_positions) {
            p.step_positions[2 * b] = gidx + 1;
            p.step_positions[2 * b + 1] = lpos + 1;
        }
        rq.recent_global[pos] = gidx;
        rq.recent_logical[pos] = lpos;
        *rq.recent_length = (int32_t)(pos + 1);
        rq.recent_page_lengths[pos / p.page_size] = pos % p.page_size + 1;
    }
}

// One 512-thread block per (group, query head of the group), a group being one (request, KV
// head): 16 slices of 32 lanes, lane l owning dims 4l..4l+3.  Slice s merges partials beg+s,
// beg+s+16, ... kCombineUnroll at a time with every load of a round issued before any is used, so
// a group of up to 128 partials costs one memory round trip.  The two slices of each wave then
// fold through a cross-half lane swap, the 8 wave states merge through LDS in wave 0, which also
// runs the output FWHT with DPP and permlane butterflies.  Every merge is the exact fp32
// softmax-state merge (triton_fourq_attention.py:58-69; triton_fourq_splitk.py:977-999).
constexpr int kCombineSlices = 16;
constexpr int kCombineWaves = kCombineSlices / 2;
#ifndef R2O_COMBINE_UNROLL
#define R2O_COMBINE_UNROLL 8
#endif
constexpr int kCombineUnroll = R2O_COMBINE_UNROLL;  // partials per slice per round: 16 x 8 = 128 per round trip

// Exact merge of softmax state (m2, l2, a2) into (m, l, a), both in the log2 domain.
__device__ __forceinline__ void merge_state(float& m, float& l, r2o_f4& a, float m2, float l2, r2o_f4 a2) {
    const float mn = fmaxf(m, m2);
    const float w1 = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mn);
    const float w2 = (m2 == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m2 - mn);
    l = l * w1 + l2 * w2;
    a = a * w1 + a2 * w2;
    m = mn;
}

__global__ __launch_bounds__(512) void decode_combine_kernel(r2o_decode_params p, CombineArgs ca) {
    __shared__ float sl_m[kCombineWaves], sl_l[kCombineWaves];
    __shared__ __align__(16) float sl_a[kCombineWaves][128];
    const int g = blockIdx.y;   // group: request g / hkv, KV head g % hkv
    const int h = blockIdx.x;   // query head within the group
    const int tid = threadIdx.x, lane = tid & 31, slice = tid >> 5;
    Stamps ts{};
    stamp(ts, 0);
    // the inline range of this group (a clamped index keeps the read inside the arguments for any
    // group; it is used only when g < ca.n_groups)
    const int gi = min(g, kInlineGroups - 1);
    const int inline_beg = ca.begin[gi], inline_end = ca.begin[gi + 1];
    touch_combine_kernarg(p, ca, inline_beg, inline_end);
#ifdef R2O_TIMELINE
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
    stamp(ts, 1);
    if (h == ca.gqa) {  // the extra block of a fused append: request g / hkv, on its KV head 0 group
        const int hkv = (int)p.hkv;
        const int b = __builtin_amdgcn_readfirstlane(r2o_div_small(g, hkv));
        if (g == b * hkv) fused_append(p, b, tid);
        return;
    }
    // slot range of the group, clamped to the slots a launch of n_items items writes
    int beg, end;
    if (g < ca.n_groups) {
        beg = inline_beg;
        end = inline_end;
    } else {
        beg = r2o_ldg(p.group_begin + g);
        end = r2o_ldg(p.group_begin + g + 1);
    }
    beg = max(beg, 0);
    end = min(end, (int)p.n_items);
    float m = -INFINITY, l = 0.f;
    r2o_f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int base = beg + slice; base < end; base += kCombineUnroll * kCombineSlices) {
        float mm[kCombineUnroll], ll[kCombineUnroll];
        r2o_f4 aa[kCombineUnroll];
#pragma unroll
        for (int k = 0; k < kCombineUnroll; ++k) {  // all loads of the round first
            const int i = base + k * kCombineSlices;
            const int64_t slot = (int64_t)(i < end ? i : base) * 16 + h;
            mm[k] = r2o_ldg(p.partial_max + slot);
            ll[k] = r2o_ldg(p.partial_sum + slot);
            aa[k] = r2o_ldg(reinterpret_cast<const r2o_f4*>(p.partial_out + slot * 128) + lane);
        }
        float mn = m;
#ifdef R2O_TIMELINE
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (base == beg + slice) stamp(ts, 2);
#endif
#pragma unroll
        for (int k = 0; k < kCombineUnroll; ++k) {
            if (base + k * kCombineSlices >= end) mm[k] = -INFINITY;
            mn = fmaxf(mn, mm[k]);
        }
        const float keep = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mn);
        l *= keep;
        acc *= keep;
#pragma unroll
        for (int k = 0; k < kCombineUnroll; ++k) {
            const float w = (mm[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mm[k] - mn);
            l += ll[k] * w;
            acc += aa[k] * w;
        }
        m = mn;
    }
    // ---- fold the wave's two slices (lanes l and l + 32 own the same dims): both halves merge
    // (slice 2w, slice 2w + 1) in that order
    {
        float m0, m1, l0, l1;
        r2o_f4 a0, a1;
        r2o_row_swap<32>(m, m0, m1);
        r2o_row_swap<32>(l, l0, l1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float x0, x1;
            r2o_row_swap<32>(acc[j], x0, x1);
            a0[j] = x0;
            a1[j] = x1;
        }
        merge_state(m0, l0, a0, m1, l1, a1);
        m = m0;
        l = l0;
        acc = a0;
    }
    const int wave = tid >> 6;
    stamp(ts, 3);
#ifdef R2O_TIMELINE
    if (wave != 0) stamps_store(g_timeline_combine, g * gridDim.x + h, wave, 8, ts);
#endif
    if ((tid & 32) == 0) {  // lanes 0..31 of each wave
        reinterpret_cast<r2o_f4*>(sl_a[wave])[lane] = acc;
        if (lane == 0) {
            sl_m[wave] = m;
            sl_l[wave] = l;
        }
    }
    __syncthreads();
    if (tid >= 64) return;
    // ---- wave 0: lane t owns dims t and t + 64
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kCombineWaves; ++w) M = fmaxf(M, sl_m[w]);
    float L = 0.f, y0 = 0.f, y1 = 0.f;
#pragma unroll
    for (int w = 0; w < kCombineWaves; ++w) {
        const float ms = sl_m[w];
        const float sc = (ms == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms - M);
        L += sl_l[w] * sc;
        y0 += sl_a[w][tid] * sc;
        y1 += sl_a[w][tid + 64] * sc;
    }
    y0 = r2o_bf16_to_f32(r2o_f32_to_bf16(y0 / L));
    y1 = r2o_bf16_to_f32(r2o_f32_to_bf16(y1 / L));
    if (p.output_hadamard) r2o_fwht128_pair(y0, y1, tid);  // of the bf16-rounded row (triton_fourq_splitk.py:1000-1006)
    // output row of (request b, query head kvh * gqa + h) = g * gqa + h
    uint16_t* orow = p.out + ((int64_t)g * ca.gqa + h) * 128;
    orow[tid] = (uint16_t)r2o_f32_to_bf16(y0);
    orow[tid + 64] = (uint16_t)r2o_f32_to_bf16(y1);
    stamp(ts, 4);
#ifdef R2O_TIMELINE
    stamps_store(g_timeline_combine, g * gridDim.x + h, 0, 8, ts);
#endif
}

int validate(const r2o_decode_params* p) {
    if (!p || !p->reqs || !p->items || !p->group_begin || !p->partial_max || !p->partial_sum || !p->partial_out ||
        !p->query || !p->out)
        return R2O_EINVAL;
    if (p->n_items <= 0 || p->n_items > 0x7fffffff || p->batch <= 0 || p->batch > R2O_MAX_BATCH) return R2O_EINVAL;
    if (p->n_items > p->partial_capacity) return R2O_EINVAL;  // every item writes one partial-state slot
    if (p->hkv <= 0 || p->hq <= 0 || p->hq > R2O_MAX_HEADS || p->hq % p->hkv || p->hq / p->hkv > R2O_MAX_GQA)
        return R2O_EINVAL;
    if (!(p->superblock == 32 || p->superblock == 64 || p->superblock == 128)) return R2O_EINVAL;
    if (!(p->int2_group == 32 || p->int2_group == 64 || p->int2_group == 128)) return R2O_EINVAL;
    if (p->q_dtype != 0 && p->q_dtype != 1) return R2O_EINVAL;
    if (p->page_size <= 0) return R2O_EINVAL;
    if (p->k_format != kKInt4 && p->k_format != kKBf16 && p->k_format != kKInt2) return R2O_EINVAL;
    if (p->row_dtype != kRowBf16 && p->row_dtype != kRowF16) return R2O_EINVAL;
    if (p->do_append && (!p->append_k || !p->append_v)) return R2O_EINVAL;
    // the fused append moves the new rows in 16-byte pieces, 4 per thread of a 512-thread block
    if (p->do_append && (p->hkv > 128 || reinterpret_cast<uintptr_t>(p->append_k) % 16 ||
                         reinterpret_cast<uintptr_t>(p->append_v) % 16))
        return R2O_EINVAL;
    if (reinterpret_cast<uintptr_t>(p->partial_out) % 16) return R2O_EINVAL;  // 16-byte vector rows
    if (reinterpret_cast<uintptr_t>(p->query) % 16) return R2O_EINVAL;        // 16-byte query loads
    // strided query / appended rows: whole 16-byte pieces per row, rows of one request not overlapping
    if (p->query_batch_stride && (p->query_batch_stride % 8 || p->query_batch_stride < p->hq * 128)) return R2O_EINVAL;
    if (p->append_batch_stride && (p->append_batch_stride % 8 || p->append_batch_stride < p->hkv * 128))
        return R2O_EINVAL;
    // strided rows only with a folded rotation (the other instances address dense rows)
    if (p->rope_mode == kRopeNone && ((p->query_batch_stride && p->query_batch_stride != p->hq * 128) ||
                                      (p->append_batch_stride && p->append_batch_stride != p->hkv * 128)))
        return R2O_EINVAL;
#ifdef R2O_TIMELINE
    if (p->rope_mode != kRopeNone) return R2O_EINVAL;
#endif
    if (p->rope_mode != kRopeNone) {  // folded rotation: the tables, sections and rotated-row outputs
        if ((p->rope_mode != kRopeMrope && p->rope_mode != kRopeQwen3) || !p->rope_cos || !p->rope_sin)
            return R2O_EINVAL;
        if (p->rope_mode == kRopeQwen3) {  // norm weights, epsilon, tables in the row dtype, one axis
            if (!p->q_norm_weight || !p->k_norm_weight || reinterpret_cast<uintptr_t>(p->q_norm_weight) % 16 ||
                reinterpret_cast<uintptr_t>(p->k_norm_weight) % 16 || !(p->norm_eps >= 0.f) ||
                p->rope_table_dtype != p->row_dtype || p->rope_section0 != 64 || p->rope_section1 != 0)
                return R2O_EINVAL;
        }
        if (p->rope_table_dtype < 0 || p->rope_table_dtype > 2) return R2O_EINVAL;
        const int64_t esize = p->rope_table_dtype == 2 ? 4 : 2, piece = 16 / esize;
        for (const int64_t* st : {p->rope_cos_strides, p->rope_sin_strides}) {
            for (int i = 0; i < 4; ++i)
                if (st[i] < 0) return R2O_EINVAL;
            // channel runs read as whole 16-byte pieces: unit channel stride, axis and request rows on
            // 16 bytes; a request's entries within 2^31 bytes of its base (32-bit offsets in the kernel)
            if (st[3] != 1 || st[0] % piece || st[1] % piece || st[0] >= (int64_t(1) << 29) ||
                (2 * st[0] + 128) * esize >= (int64_t(1) << 31))
                return R2O_EINVAL;
        }
        if (reinterpret_cast<uintptr_t>(p->rope_cos) % 16 || reinterpret_cast<uintptr_t>(p->rope_sin) % 16)
            return R2O_EINVAL;
        if (p->rope_section0 < 0 || p->rope_section1 < 0 || p->rope_section0 + p->rope_section1 > 64) return R2O_EINVAL;
        if (p->q_dtype != p->row_dtype) return R2O_EINVAL;  // one dtype for the rotated query and key
        if (p->do_append && (!p->rotated_k || !p->rotated_v || reinterpret_cast<uintptr_t>(p->rotated_k) % 16 ||
                             reinterpret_cast<uintptr_t>(p->rotated_v) % 16))
            return R2O_EINVAL;
    }
    return R2O_OK;
}

// ------------------------------------------------------------- workspace-free decode
// The partial states of r2o_decode_noalloc live in this array: one per GPU for the life of the
// process, kScratchSlots work items of (acc [16][128], max [16], sum [16]) fp32 = 8.1 MiB.
constexpr int64_t kScratchSlots = 1024;
constexpr int64_t kScratchFloats = kScratchSlots * (16 * 128 + 16 + 16);
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];

}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

// Device address of `scratch` on `dev` (the host-side name is only a stand-in): looked up once per
// device, with that device current for the lookup (the caller's current device is restored), by
// r2o_decode_noalloc_init or by the first r2o_decode_noalloc call on that device.  Returns nullptr if
// the lookup fails.
float* scratch_address(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    float* ptr = g_scratch[dev].load(std::memory_order_acquire);
    if (ptr != nullptr) return ptr;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return nullptr;
    if (e != hipSuccess || addr == nullptr) return nullptr;
    ptr = static_cast<float*>(addr);
    g_scratch[dev].store(ptr, std::memory_order_release);
    return ptr;
}

template <int RO>
void launch_partial(const r2o_decode_params& p, hipStream_t stream) {
    const dim3 grid((unsigned)p.n_items);
    const dim3 block(KernelCfg<kKInt4>::kThreads), block_bf16(KernelCfg<kKBf16>::kThreads);
    static_assert(KernelCfg<kKInt4>::kThreads == KernelCfg<kKInt2>::kThreads, "one workgroup size for the low-bit K formats");
    const bool f16 = p.row_dtype == kRowF16;
    switch (p.k_format) {
        case kKInt4:
            if (f16) hipLaunchKernelGGL((decode_partial_kernel<kKInt4, kRowF16, RO>), grid, block, 0, stream, p);
            else hipLaunchKernelGGL((decode_partial_kernel<kKInt4, kRowBf16, RO>), grid, block, 0, stream, p);
            break;
        case kKBf16:
            if (f16) hipLaunchKernelGGL((decode_partial_kernel<kKBf16, kRowF16, RO>), grid, block_bf16, 0, stream, p);
            else hipLaunchKernelGGL((decode_partial_kernel<kKBf16, kRowBf16, RO>), grid, block_bf16, 0, stream, p);
            break;
        default:
            if (f16) hipLaunchKernelGGL((decode_partial_kernel<kKInt2, kRowF16, RO>), grid, block, 0, stream, p);
            else hipLaunchKernelGGL((decode_partial_kernel<kKInt2, kRowBf16, RO>), grid, block, 0, stream, p);
            break;
    }
}

// The kernels' copy of the arguments: row strides of 0 (dense) spelled out.
r2o_decode_params kernel_params(const r2o_decode_params& params) {
    r2o_decode_params p = params;
    if (p.query_batch_stride == 0) p.query_batch_stride = p.hq * 128;
    if (p.append_batch_stride == 0) p.append_batch_stride = p.hkv * 128;
    return p;
}

int launch_decode(const r2o_decode_params& params, hipStream_t stream) {
    const r2o_decode_params p = kernel_params(params);
#ifndef R2O_TIMELINE  // the phase-stamp build (bench.py --timeline) has no rotating instances
    if (p.rope_mode == kRopeMrope) launch_partial<kRopeMrope>(p, stream);
    else if (p.rope_mode == kRopeQwen3) launch_partial<kRopeQwen3>(p, stream);
    else
#endif
        launch_partial<kRopeNone>(p, stream);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

int launch_combine(const r2o_decode_params& params, hipStream_t stream) {
    r2o_decode_params p = kernel_params(params);
    if (p.rope_mode != kRopeNone) {  // the fused append copies the rows the partial pass rotated
        p.append_k = p.rotated_k;
        p.append_v = p.rotated_v;
        p.append_batch_stride = p.hkv * 128;
    }
    CombineArgs ca{};
    const int64_t groups = p.batch * p.hkv;
    ca.gqa = (int32_t)(p.hq / p.hkv);
    if (p.group_begin_host && groups <= kInlineGroups) {
        ca.n_groups = (int32_t)groups;
        for (int64_t i = 0; i <= groups; ++i) ca.begin[i] = p.group_begin_host[i];
    }
    hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)(ca.gqa + (p.do_append ? 1 : 0)), (unsigned)groups),
                       dim3(512), 0, stream, p, ca);
    R2O_CHECK_LAUNCH();
    return R2O_OK;
}

}  // namespace

extern "C" {

int r2o_decode_partial(const r2o_decode_params* params, void* stream) {
    const int rc = validate(params);
    if (rc) return rc;
    return launch_decode(*params, (hipStream_t)stream);
}

int r2o_decode_combine(const r2o_decode_params* params, void* stream) {
    const int rc = validate(params);
    if (rc) return rc;
    return launch_combine(*params, (hipStream_t)stream);
}

int r2o_decode(const r2o_decode_params* params, void* stream) {
    const int rc = validate(params);
    if (rc) return rc;
    const int lrc = launch_decode(*params, (hipStream_t)stream);
    if (lrc) return lrc;
    return launch_combine(*params, (hipStream_t)stream);
}

int r2o_decode_noalloc_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return R2O_ELAUNCH;
    if (device < 0 || device >= n || device >= kMaxDevices) return R2O_EINVAL;
    return scratch_address(device) ? R2O_OK : R2O_ELAUNCH;
}

int r2o_decode_noalloc(const r2o_decode_params* params, void* stream) {
    if (!params) return R2O_EINVAL;
    if (params->n_items > kScratchSlots) return R2O_EINVAL;  // more partial states than `scratch` holds
    int dev = -1;  // the array of the GPU the stream runs on, whatever device is current
    if (hipStreamGetDevice((hipStream_t)stream, &dev) != hipSuccess) return R2O_EINVAL;
    float* base = scratch_address(dev);
    if (base == nullptr) return R2O_ELAUNCH;
    r2o_decode_params p = *params;  // the caller's partial pointers are ignored
    p.partial_out = base;
    p.partial_max = base + kScratchSlots * 16 * 128;
    p.partial_sum = p.partial_max + kScratchSlots * 16;
    p.partial_capacity = kScratchSlots;
    const int rc = validate(&p);
    if (rc) return rc;
    const int lrc = launch_decode(p, (hipStream_t)stream);
    if (lrc) return lrc;
    return launch_combine(p, (hipStream_t)stream);
}

#ifdef R2O_TIMELINE
// Measurement build only: copies the last launch's phase stamps to the host (which 0: partial kernel,
// [4096 blocks][4 waves][12]; 1: combine, [4096 blocks][8 waves][12]; u64 each).
int r2o_timeline_read(int which, void* dst, size_t bytes) {
    if (!dst || (which != 0 && which != 1)) return R2O_EINVAL;
    const size_t cap = which == 0 ? sizeof(g_timeline_partial) : sizeof(g_timeline_combine);
    if (bytes > cap) return R2O_EINVAL;
    const hipError_t e = which == 0 ? hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_timeline_partial), bytes, 0, hipMemcpyDeviceToHost)
                                    : hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_timeline_combine), bytes, 0, hipMemcpyDeviceToHost);
    return e == hipSuccess ? R2O_OK : R2O_ELAUNCH;
}
#endif

}  // extern "C"
