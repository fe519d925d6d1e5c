/*
 * r2o_sspa.h — C ABI of the MI355X (gfx950) SSPA packed-KV decode library (libr2o_sspa.so).
 *
 * The reference (Fabulous1496/R2-Omni) is pure Python: its hot path is Triton kernels launched
 * from r2omni/sspa/kernels/triton_fourq_splitk.py and the runtime packers in
 * r2omni/sspa/runtime/ (*.py).  There is no FFI in the reference; each entry point below replaces
 * one Triton launch (or one torch-op sequence) of that Python API and is bound with ctypes by
 * r2omni_amd/_lib.py.  Every entry point:
 *   - takes plain device pointers, int64 sizes and an opaque hipStream_t (as void*);
 *   - launches asynchronously on that stream and allocates nothing;
 *   - returns 0 on success, R2O_EINVAL for an argument the kernel's grid cannot honour
 *     (checked on the host before any launch), R2O_ELAUNCH if the launch itself failed.
 * Tensor layouts are the reference's "wire format" (compact_int4_key.py:83-110, quantization.py:19-116,
 * int2_reference.py:96-151) so caches built by the
 * reference and by this library are byte-identical.
 *
 * dtype codes: 0 = bfloat16, 1 = float16 (element type of K/V/Q rows).
 */
#ifndef R2O_SSPA_H
#define R2O_SSPA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define R2O_OK 0
#define R2O_EINVAL 1
#define R2O_ELAUNCH 2

#define R2O_HEAD_DIM 128
#define R2O_MAX_GQA 16
#define R2O_MAX_BATCH 32
#define R2O_MAX_HEADS 4096 /* query heads per decode launch */

/* r2o_decode_params.k_format */
#define R2O_K_INT4 0
#define R2O_K_BF16 1
#define R2O_K_INT2 2

/* ---------------------------------------------------------------- decode (hot path) ---- */

/* One request's static cache geometry; an array of these lives in device memory and is
 * rebuilt only when the cache layout changes (prefill, flush), like the reference's
 * prepare_splitk_executor (triton_fourq_splitk.py:1695-1907).  All fields are 8 bytes. */
typedef struct r2o_request_desc {
    const uint8_t* k_packed;      /* R2O_K_INT4: compact INT4-K arena u8 [Hkv, k_capacity, 64];  */
                                  /* R2O_K_INT2: compact INT2-K arena u8 [Hkv, k_capacity, 32];  */
                                  /* R2O_K_BF16: 16-bit key rows [Hkv, k_capacity, 128]          */
    const uint16_t* k_scale;      /* fp16 [Hkv, k_superblocks, 128]                              */
    const uint8_t* k_zero;        /* u8 zero points (INT4) or fp16 offsets (INT2) [Hkv, k_sb, 128] */
    int64_t k_capacity;
    int64_t k_superblocks;
    const uint32_t* k_operands;   /* u32  [Hkv, k_superblocks, 128]  QK MFMA operands (see pack) */
    const uint16_t* fp_v;         /* 16-bit [Hkv, fp_stride, 128]  (FP-V pool, row_dtype)        */
    int64_t fp_stride;
    const uint8_t* i4_v;          /* u8   [Hkv, i4_stride, 64]   (per-token symmetric INT4-V)   */
    const float* i4_scale;        /* f32  [Hkv, i4_stride]                                       */
    int64_t i4_stride;
    const uint8_t* i2_v;          /* u8   [Hkv, i2_stride, 32]   (per-token-group INT2-V)       */
    const uint16_t* i2_scale;     /* fp16 [Hkv, i2_stride, 128/G]                                */
    const uint8_t* i2_zero;       /* u8   [Hkv, i2_stride, 128/G]                                */
    int64_t i2_stride;
    uint16_t* recent_k;           /* 16-bit [Hkv, recent_capacity, 128]  Recent-FP ring (row_dtype), 16-byte aligned */
    uint16_t* recent_v;
    int64_t recent_capacity;
    int32_t* recent_length;       /* device int32 active length (written by the fused append)   */
    int64_t* recent_global;       /* int64 [recent_capacity]                                     */
    int64_t* recent_logical;      /* int64 [recent_capacity]                                     */
    int64_t* recent_page_lengths; /* int64 [recent_capacity / page_size]                         */
} r2o_request_desc;

/* One unit of split-K work: a run of 32-token tiles of one pool segment of one (request,
 * kv head).  Tiles are aligned to 32 positions of the compact K arena so that every tile lies
 * in one K superblock; positions outside [lo, hi) are masked.  For the Recent-FP ring, arena
 * positions are ring slots.  V row = arena position - v_delta.  Items may be launched in any
 * order (largest first); each writes its partial to `slot`.  The item carries the base pointers
 * of its (request, kv head) rows, so the partial kernel reads nothing else before its first
 * loads.  All fields are 8 bytes (16 words, 128 bytes). */
typedef struct r2o_work_item {
    int64_t req;
    int64_t kvh;
    int64_t kind;      /* 0 = FP-V (bf16), 1 = INT4-V, 2 = INT2-V, 3 = Recent-FP (bf16 K and V) */
    int64_t tile0;     /* arena position of the first tile (multiple of 32)                      */
    int64_t ntiles;    /* tiles of the item; each of the 4 waves takes a contiguous quarter       */
    int64_t lo;        /* valid arena positions [lo, hi)                                          */
    int64_t hi;
    int64_t v_delta;
    int64_t slot;      /* partial-state slot; slots of one (request, kv head) are contiguous     */
    const void* k_base;          /* K rows of the head: INT4 / INT2 codes, bf16 rows, or ring K   */
    const uint32_t* k_ops;       /* QK operands of the head's K superblocks (INT4/INT2-K) or NULL */
    const void* v_base;          /* V rows of the head in this pool, or ring V                    */
    const void* v_scale;         /* INT4-V f32 / INT2-V fp16 scales of the head, or NULL          */
    const uint8_t* v_zero;       /* INT2-V zero points of the head, or NULL                       */
    const int32_t* ring_length;  /* Recent-FP items: the request's device ring length, or NULL    */
    int64_t v_group;             /* INT2-V items: the V group size (32, 64 or 128), so the kernel's */
                                 /* start-up needs no launch argument beyond the first two lines;  */
                                 /* 0 for the other kinds (the planner fills it)                   */
} r2o_work_item;

/* One run of the planner's input: the 32-token tiles of one pool segment of one (request, kv head)
 * (or its Recent-FP ring, kind 3), runs of one (request, kv head) adjacent, groups in order. */
typedef struct r2o_plan_run {
    int64_t req, kvh, kind, tile0, ntiles, lo, hi, v_delta;
} r2o_plan_run;

/* Planner settings (the Python side owns the tuned values). */
typedef struct r2o_plan_config {
    int64_t num_cus;             /* compute units of the GPU                                        */
    int64_t blocks_per_cu;       /* at most this many items per CU                                  */
    int64_t tiles_per_item;      /* small caches: about this many tiles per item, >= num_cus items  */
    int64_t waves_per_item;      /* item sizes are multiples of this many tiles (one share a wave)  */
    int64_t min_tiles_per_item;  /* a run is not split into items smaller than this                 */
    double tile_cost[4];         /* weight of one tile of kind FP-V, INT4-V, INT2-V, Recent-FP      */
    double late_share;           /* single-kind plans over more than num_cus items: the work of the
                                    later-launched half of each run's items, relative to the first */
} r2o_plan_config;

/* Work-item plan of one decode launch (host code, no GPU work).  Splits every run into items of
 * about equal weighted cost (water-filling up to min(blocks_per_cu * num_cus, max(num_cus,
 * tiles / tiles_per_item)) items), numbers their partial slots in (request, kv head) order into
 * group_begin [n_groups + 1], and writes the items to items[0 .. *n_items) largest first.  With
 * reqs (host copies of the request descriptors) each item's base pointers are filled in, else they
 * are 0; INT2-V items get v_group = int2_group either way (int2_group must be 32, 64 or 128 whenever
 * a run has kind 2).  Every run needs tile0 >= 0, tile0 % 32 == 0, tile0 <= lo <= hi <=
 * tile0 + 32 * ntiles; with reqs also 0 <= kvh < n_groups / n_reqs, its tiles inside the K arena
 * (k_capacity) or the ring (recent_capacity), and its V rows [lo - v_delta, hi - v_delta) inside the
 * pool (fp_stride / i4_stride / i2_stride), since the partial kernel reads whole K tiles at the
 * items' base pointers.  Returns R2O_EINVAL for an inconsistent input or when more than max_items
 * would result.
 * No counterpart in the reference's launch plan (one program per BLOCK_N tile, counted while
 * preparing the executor, triton_fourq_splitk.py:1772-1817); it replaces that preparation step. */
int r2o_plan_work_items(const r2o_plan_run* runs, int64_t n_runs, const r2o_plan_config* cfg,
                        const r2o_request_desc* reqs, int64_t n_reqs, int64_t k_format, int64_t int2_group,
                        r2o_work_item* items, int64_t max_items, int32_t* group_begin, int64_t n_groups,
                        int64_t* n_items);

typedef struct r2o_decode_params {
    const r2o_request_desc* reqs;   /* device [batch]                                  */
    const r2o_work_item* items;     /* device [n_items] in launch order                */
    const int32_t* group_begin;     /* device [batch*hkv + 1] slot range of each group */
    int64_t n_items;
    float* partial_max;             /* device f32 [n_items, 16]      (log2 domain)     */
    float* partial_sum;             /* device f32 [n_items, 16]                        */
    float* partial_out;             /* device f32 [n_items, 16, 128], 16-byte aligned  */
    const uint16_t* query;          /* device [batch, hq, 128] (dtype q_dtype)         */
    int64_t query_batch_stride;     /* elements from one request's query rows to the next (0: hq*128),
                                       so that the query can be a view into a fused QKV projection;
                                       a multiple of 8, at least hq*128.  Only with rope_mode 1: other
                                       calls take dense rows (0 or hq*128), as the reference does. */
    const uint16_t* append_k;       /* device bf16 [batch, hkv, 128] or NULL; 16-byte
                                       aligned, and hkv <= 128 when do_append is set  */
    const uint16_t* append_v;
    int64_t* step_positions;        /* device int64 [batch, 2] or NULL.  Non-NULL selects device-state
                                       mode: both kernels read each ring length from
                                       reqs[b].recent_length (not recent_len[]), the fused append takes
                                       (global, logical) from here instead of append_global/logical and
                                       advances them by one, so one captured launch pair replays
                                       correctly from step to step (until a flush re-plans the items). */
    int64_t batch;
    int64_t hq;
    int64_t hkv;
    int64_t superblock;             /* K superblock: 32, 64 or 128                     */
    int64_t int2_group;             /* INT2-V group: 32, 64 or 128                     */
    int64_t page_size;              /* Recent-FP page size (16, 32, 64)                */
    int64_t q_dtype;                /* 0 = bf16, 1 = fp16                              */
    int64_t output_hadamard;        /* 1: out = bf16(FWHT128(bf16(out)))               */
    int64_t do_append;              /* 1: fused Recent-FP append of append_k/append_v  */
    int64_t k_format;               /* R2O_K_INT4 / R2O_K_BF16 / R2O_K_INT2: the history key layout  */
                                    /* of every request (see r2o_request_desc.k_packed)               */
    float sm_scale;                 /* softmax scale (head_dim^-1/2 by default)        */
    uint16_t* out;                  /* device bf16 [batch, hq, 128]                    */
    int64_t append_batch_stride;    /* the same for append_k / append_v (0: hkv*128; at least hkv*128;
                                       only with rope_mode 1)                                          */
    int32_t recent_len[R2O_MAX_BATCH];     /* host-tracked Recent-FP active length     */
    int64_t append_global[R2O_MAX_BATCH];  /* global token index of the appended token */
    int64_t append_logical[R2O_MAX_BATCH]; /* logical position of the appended token   */
    int64_t row_dtype;              /* 0 = bf16, 1 = fp16: element type of every 16-bit row (FP-V pool,
                                       Recent-FP ring, BF16-K arena, append_k / append_v); the output
                                       stays bf16, as the reference's (triton_fourq_splitk.py:1653-1655) */
    const int32_t* group_begin_host; /* host [batch*hkv + 1] copy of group_begin, or NULL.  When given
                                       and batch*hkv <= 32, r2o_decode_combine passes the slot ranges
                                       in its launch arguments instead of reading group_begin on the
                                       device (one dependent memory round trip less); it must equal
                                       the device array.  Read on the host during the call only. */
    int64_t partial_capacity;       /* partial-state slots the workspace holds (rows of partial_max /
                                       partial_sum / partial_out): every entry point returns R2O_EINVAL
                                       before any launch when n_items exceeds it, as the reference sizes
                                       and checks its workspace first (triton_fourq_splitk.py:1607-1692,
                                       qwen_sspa_attention.py:1157-1160).  r2o_decode_noalloc sets it
                                       itself. */
    /* The decode step's rotation folded into the call (qwen_sspa_attention.py:1239-1247, 230-235):
     * rope_mode 0: query and append rows are used as given (already rotated).  rope_mode 1 (Qwen mRoPE,
     * triton_qwen_mrope.py:45-124): query and append_k are the raw projections; the partial kernel
     * applies x * cos + rotate_half(x) * sin in fp32 (dimension d taking axis 0, 1 or 2 of the tables
     * by d % 64 against the sections), then with rope_hadamard the orthonormal FWHT-128, rounding each
     * row once to its dtype, exactly as r2o_qkv_mrope does; append_v takes the FWHT alone with
     * value_hadamard.  rope_mode 2: the Qwen3 norm + RoPE (below).  The rotated appended rows go to
     * rotated_k / rotated_v, from which the combine's fused append writes the ring.  The tables' channel
     * stride must be 1 and their axis and batch strides and base addresses whole 16-byte pieces. */
    int64_t rope_mode;
    const void* rope_cos;           /* [3, batch, tokens, 128] tables of the step (token 0 is used)  */
    const void* rope_sin;
    int64_t rope_cos_strides[4];    /* element strides of rope_cos: axis, batch, token, dimension     */
    int64_t rope_sin_strides[4];
    int64_t rope_table_dtype;       /* 0 = bf16, 1 = fp16, 2 = fp32                                    */
    int64_t rope_section0;          /* mRoPE sections s0, s1 (the third is 64 - s0 - s1)               */
    int64_t rope_section1;
    int64_t rope_hadamard;          /* 1: FWHT-128 of the rotated query and key rows                   */
    int64_t value_hadamard;         /* 1: FWHT-128 of the appended value row                           */
    uint16_t* rotated_k;            /* device [batch, hkv, 128] (row_dtype), 16-byte aligned: written  */
    uint16_t* rotated_v;            /* by the partial pass when rope_mode and do_append are set        */
    /* rope_mode 2 (the Qwen3 branch, qwen_sspa_attention.py:1228-1235): the query and appended key rows
     * first take their per-head RMSNorm (transformers' Qwen3RMSNorm: mean of squares in fp32, x *
     * rsqrt(mean + eps) rounded to the row dtype, times the weight, rounded), then apply_rotary_pos_emb
     * with every product and the sum rounded to the row dtype, then with rope_hadamard the FWHT-128,
     * exactly as r2o_qkv_norm_rope does.  The tables are passed as [1, batch, tokens, 128] views (axis
     * stride 0, rope_section0 = 64, rope_section1 = 0) in the row dtype. */
    const uint16_t* q_norm_weight;  /* [128], row dtype, 16-byte aligned (rope_mode 2)                */
    const uint16_t* k_norm_weight;
    float norm_eps;                 /* RMSNorm epsilon, >= 0 (one for both norms, as r2o_qkv_norm_rope) */
} r2o_decode_params;

/* Split-K partial pass.  Replaces _fourq_page_partial_kernel / _full_head_page_partial_kernel
 * (triton_fourq_splitk.py:456-931, :144-375, launched at :1393-1462). */
int r2o_decode_partial(const r2o_decode_params* params, void* stream);

/* Split-K combine + output (bf16, optional FWHT) + fused Recent-FP append.  Replaces
 * _fourq_hierarchical_group_reduce_kernel and _fourq_partial_reduce_kernel
 * (triton_fourq_splitk.py:1023-1155, :936-1020, launched at :1467-1541). */
int r2o_decode_combine(const r2o_decode_params* params, void* stream);

/* The whole decode call: r2o_decode_partial then r2o_decode_combine on `stream`, after one check of
 * the arguments.  Replaces the launch sequence of SplitKExecutor.__call__ (triton_fourq_splitk.py:
 * 1393-1541: the partial, group-reduce and final-reduce launches); one host call instead of two. */
int r2o_decode(const r2o_decode_params* params, void* stream);

/* Workspace-free decode: r2o_decode_partial then r2o_decode_combine on `stream`, with the split-K
 * partial states held in a library-owned device array (one per GPU, kept until the process ends)
 * instead of params->partial_max / partial_sum / partial_out / partial_capacity, which are ignored
 * and may be NULL / 0.  The array of the stream's device is used (hipStreamGetDevice); its address
 * is looked up once per device, by r2o_decode_noalloc_init or else by the first call on that device.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops).  Allocates nothing (no hipMalloc / hipFree).
 * Limit: params->n_items <= 1024 work items (8.1 MiB of partial states), else R2O_EINVAL before any
 * launch.  The array is shared by every call on one GPU and keeps the last call's contents (every
 * slot a launch reads is written first by that launch): calls that overlap on one GPU (different
 * streams, or threads without ordering) race on it. */
int r2o_decode_noalloc(const r2o_decode_params* params, void* stream);

/* Set-up of r2o_decode_noalloc on `device`: looks up the device address of that GPU's partial-state
 * array (with the device current for the lookup; the caller's current device is restored).  No
 * counterpart in the reference; for the same callers as r2o_decode_noalloc.  Call it once per device
 * before capturing r2o_decode_noalloc into a HIP graph, so that no runtime lookup falls inside the
 * capture.  Allocates nothing.  R2O_EINVAL for a device index out of range, R2O_ELAUNCH if the
 * lookup fails. */
int r2o_decode_noalloc_init(int device);

/* ----------------------------------------------------------------- pack / append --------- */

/* Per-channel affine INT4-K over `superblock`-token blocks into the compact arena.
 * Arena positions [dst_start, dst_start + tail + n) are (re)written; dst_start must be a
 * multiple of `superblock`.  The first `tail` positions are read back from the arena itself
 * (dequantised, rounded to `dtype`) — the flush rule of CompactInt4KeyArena.append_superblock
 * (compact_int4_key.py:210-220); the next n come from src[h, index[i]] (index NULL: i).
 * `operands` (nullable) receives, per superblock, the QK MFMA operands derived from the
 * stored scale/zero: for lane group g (channels 32g..32g+31), MFMA j and pair u, with
 * c = 32g + 8j + u, dword g*32 + 4j + u = fp16 (s[c], s[c+4]) and dword g*32 + 16 + 4j + u =
 * fp16 (-(1024 + z[c]), -(1024 + z[c+4])) for even u; for odd u (codes read 4 bits up, as
 * 1024 + 16 code) the pairs are (s/16) and -(1024 + 16 z).
 * Replaces _gather_pack_int4_key_kernel (compact_int4_key.py:22-76) and the torch flush path. */
int r2o_pack_int4_k(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens,
                    const int64_t* index, int64_t n, int64_t tail, int64_t dst_start,
                    uint8_t* packed, uint16_t* scale, uint8_t* zero, uint32_t* operands,
                    int64_t capacity, int64_t superblocks, int64_t superblock, void* stream);

/* Per-channel affine INT2-K (OScaR form) over superblocks of 32/64/128 tokens, same gather /
 * tail / superblock-aligned-destination contract as r2o_pack_int4_k.  packed u8 [Hkv, capacity, 32]
 * (byte j = channels 4j..4j+3, low bits first), scale and offset fp16 [Hkv, superblocks, 128]
 * (dequant = code * scale + offset).  With operands != NULL also writes the QK MFMA operands
 * u32 [Hkv, superblocks, 128]: per lane group g and MFMA j, pair u covers channels (c, c + 8),
 * c = 32g + 16(j/2) + 4(j%2) + u, whose codes enter the MFMA as 1024 + 4^u code; words
 * [32g + 4j + u] hold (scale / 4^u) pairs and [32g + 16 + 4j + u] offset pairs.
 * Replaces quantize_int2_key_per_channel (int2_reference.py:159-214) in
 * build_compact_int2_key_arena (compact_int2_key.py:125-153) and append_superblock (:110-122). */
int r2o_pack_int2_k(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens,
                    const int64_t* index, int64_t n, int64_t tail, int64_t dst_start,
                    uint8_t* packed, uint16_t* scale, uint16_t* offset, uint32_t* operands,
                    int64_t capacity, int64_t superblocks, int64_t superblock, void* stream);

/* Per-token symmetric INT4-V: packed[h, dst+i] / scale[h, dst+i] from src[h, index[i]] (index
 * NULL: src[h, i], n <= src_tokens).  Replaces _gather_pack_int4_value_kernel
 * (fused_value_pack.py:28-70), in the static gather and in CompactInt4ValueArena.append_block
 * (fused_value_pack.py:263-299), the flush of generated INT4 values. */
int r2o_pack_int4_v(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens,
                    const int64_t* index, int64_t n, int64_t dst_start,
                    uint8_t* packed, float* scale, int64_t capacity, void* stream);

/* Per-token-group affine INT2-V (group 32/64/128) from src[h, index[i]] (index NULL: src[h, i],
 * n <= src_tokens).  Replaces _gather_pack_int2_value_kernel (fused_value_pack.py:75-149), both
 * the gathered prefill and the contiguous flush forms. */
int r2o_pack_int2_v(const uint16_t* src, int64_t dtype, int64_t hkv, int64_t src_tokens,
                    const int64_t* index, int64_t n, int64_t dst_start, int64_t group,
                    uint8_t* packed, uint16_t* scale, uint8_t* zero, int64_t capacity,
                    void* stream);

/* Row gather dst[h, i, :] = src[h, index[i], :] of 16-bit elements (FP-V pool build,
 * replaces value.index_select(1, tokens) at precision_pool.py:697-698). */
int r2o_gather_rows(const uint16_t* src, int64_t hkv, int64_t src_tokens, const int64_t* index,
                    int64_t n, uint16_t* dst, int64_t dst_stride, void* stream);

/* Non-fused Recent-FP append of one token at `position` + metadata.  Replaces
 * _append_recent_fp_kernel (triton_fourq_splitk.py:413-447, host :1557-1604). */
int r2o_recent_append(uint16_t* recent_k, uint16_t* recent_v, int64_t hkv, int64_t capacity,
                      const uint16_t* new_k, const uint16_t* new_v, int64_t position,
                      int64_t global_index, int64_t logical_position, int32_t* length,
                      int64_t* global_buf, int64_t* logical_buf, int64_t* page_lengths,
                      int64_t page_size, void* stream);

/* Flush bookkeeping of the ring: move slots [flush, active) to [0, active - flush) for K, V
 * and both index buffers, then refresh page lengths for the new active length.  Replaces the
 * clone/copy sequence of dynamic_fourq_cache.py:246-253 and _refresh_recent_pages :108-117. */
int r2o_recent_shift(uint16_t* recent_k, uint16_t* recent_v, int64_t hkv, int64_t capacity,
                     int64_t flush, int64_t active, int64_t* global_buf, int64_t* logical_buf,
                     int32_t* length, int64_t* page_lengths, int64_t page_size, void* stream);

/* Orthonormal 128-point FWHT of `rows` rows (in place allowed), dtype in/out.  Replaces
 * triton_fwht_128 (triton_qwen_mrope.py:325-346). */
int r2o_fwht128(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t dtype, void* stream);

/* Decode-step Q/K rotation: Qwen multimodal RoPE (rotate-half, dimension d takes its cos/sin
 * from table axis 0, 1 or 2 by d % 64 against the sections (section0, section1, 64 - s0 - s1)),
 * computed in fp32, optionally followed by the orthonormal FWHT-128, rounded once to `dtype`.
 * q [batch, hq, tokens, 128], k [batch, hkv, tokens, 128] contiguous; cos/sin [3, batch, tokens,
 * 128] with element strides (axis, batch, token, dim) and table_dtype 0 = bf16, 1 = fp16,
 * 2 = fp32.  Replaces _qwen_qk_mrope_kernel / _qwen_batched_qk_mrope_kernel
 * (triton_qwen_mrope.py:45-211, host wrapper qwen_qk_mrope :214-322). */
int r2o_qk_mrope(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out, int64_t dtype,
                 int64_t batch, int64_t hq, int64_t hkv, int64_t tokens, const void* cos, const void* sin,
                 int64_t table_dtype, const int64_t* cos_strides, const int64_t* sin_strides,
                 int64_t section0, int64_t section1, int64_t apply_hadamard, void* stream);

/* r2o_qk_mrope plus, when v / v_out are non-NULL, the orthonormal FWHT-128 of the V rows
 * v [batch, hkv, tokens, 128] (same dtype) into v_out, in the same launch: the decode step's
 * K/V rotation (qwen_sspa_attention.py:1239-1247) and V Hadamard (triton_fwht_128 at :230-235,
 * triton_qwen_mrope.py:325-346) as one launch instead of two.  Every FWHT here (Q, K, V) runs the
 * reference's stage order (stride 1 .. 64), so V equals r2o_fwht128's result bit for bit.
 * v and v_out must both be NULL or both be set. */
int r2o_qkv_mrope(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* q_out, uint16_t* k_out,
                  uint16_t* v_out, int64_t dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t tokens,
                  const void* cos, const void* sin, int64_t table_dtype, const int64_t* cos_strides,
                  const int64_t* sin_strides, int64_t section0, int64_t section1, int64_t apply_hadamard,
                  void* stream);

/* Decode-step Q/K transform of Qwen3-style attention (MiniCPM-o's LLM): per-head RMSNorm with
 * weights q_weight / k_weight [128] and epsilon eps (mean of squares in fp32, x * 1/sqrt(v + eps)
 * rounded to dtype, times the weight rounded to dtype), then rotate-half RoPE with cos/sin
 * [batch, tokens, 128] of the same dtype (element strides (batch, token, dim); each product and the
 * sum rounded to dtype, as torch evaluates them), then optionally the orthonormal FWHT-128.
 * q/k/q_out/k_out as for r2o_qk_mrope; dtype 0 = bf16, 1 = fp16 for every tensor.  Replaces the
 * q_norm / k_norm / apply_rotary_pos_emb / triton_fwht_128 sequence of the Qwen3 branch
 * (qwen_sspa_attention.py:1228-1235). */
int r2o_qk_norm_rope(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out, int64_t dtype,
                     int64_t batch, int64_t hq, int64_t hkv, int64_t tokens, const uint16_t* q_weight,
                     const uint16_t* k_weight, float eps, const uint16_t* cos, const uint16_t* sin,
                     const int64_t* cos_strides, const int64_t* sin_strides, int64_t apply_hadamard, void* stream);

/* r2o_qk_norm_rope plus, when v / v_out are non-NULL, the orthonormal FWHT-128 of the V rows
 * v [batch, hkv, tokens, 128] (same dtype) into v_out in the same launch: the Qwen3 branch's Q/K
 * transform and the decode step's V Hadamard (triton_fwht_128 at qwen_sspa_attention.py:230-235)
 * as one launch, V rows as in r2o_qkv_mrope.  v and v_out must both be NULL or both be set. */
int r2o_qkv_norm_rope(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* q_out, uint16_t* k_out,
                      uint16_t* v_out, int64_t dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t tokens,
                      const uint16_t* q_weight, const uint16_t* k_weight, float eps, const uint16_t* cos,
                      const uint16_t* sin, const int64_t* cos_strides, const int64_t* sin_strides,
                      int64_t apply_hadamard, void* stream);

/* Library identification: returns the gfx target the code objects were built for. */
const char* r2o_build_target(void);

#ifdef __cplusplus
}
#endif
#endif /* R2O_SSPA_H */
