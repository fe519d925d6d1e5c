"""Split-K executor over the SSPA packed cache: the drop-in decode call surface.

Same names, arguments, return values and error behaviour as the reference
(r2omni/sspa/kernels/triton_fourq_splitk.py):
  allocate_splitk_workspace   :1607-1676   required_splitk_blocks :1679-1692
  prepare_splitk_executor     :1695-1907   SplitKExecutor.__call__ :1243-1547
  append_recent_fp_triton     :1557-1604   (name kept; it launches r2o_recent_append)
  stack_homogeneous_splitk_executors :1995-2241 (here also for ragged batches; the read-only
                                     payload is shared, each request's Recent-FP ring is copied)
  allocated_workspace_bytes   :2244-2256
Launch knobs of the Triton kernels (block_n, num_warps, num_stages, tensor-core flags, ...)
are accepted and ignored: the gfx950 kernels fix their own tiling.  A "block" of the
workspace is one split-K work item (a run of 32-token tiles handled by one workgroup).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Sequence

import torch

from . import _lib
from .cache import ThreePrecisionCache

TILE = 32
_WAVES_PER_ITEM = 4          # waves of the partial kernel's workgroup (each takes a contiguous share)
_MIN_TILES_PER_ITEM = 4      # one tile per wave
_BLOCKS_PER_CU = 2           # work items planned per CU: the kernel holds 2 resident, and more queue behind them
# Small caches: fewer, longer items (about two tiles per wave) while every CU still gets one; more
# items would only add partial states for the combine (measured on MI355X: a 3B layer at 32k
# tokens takes 13.0 us per call at 256 items against 14.9 at 512).
_TILES_PER_ITEM_TARGET = 8
# Two workgroups share each CU (slots j and j + CUs of the launch), and the hardware favours the
# older one: with equal work the later-launched sibling ends ~20 % after it (measured on MI355X for
# an all-INT2 131k-token layer: 6 us of a 30 us kernel with the CU half occupied).  When every item
# is of one kind, the items split from a run are therefore uneven: the later-launched half gets
# this share of the work of the earlier half.  Plans that mix kinds already launch their larger
# items first and keep an even split (an uneven one measured 1 us slower on the mixed-tier layer).
_LATE_SHARE = 0.7
# The share that measured best per key format (single-kind cfg3 plans, nontemporal tile loads): INT4-K
# 0.8 (layer call 0.55 us shorter than at 0.7), INT2-K 0.7 (0.8 was 0.3-0.5 us longer); BF16-K keeps 0.7.
_LATE_SHARE_BY_K = {_lib.K_INT4: 0.8}


@dataclass
class SplitKWorkspace:
    partial_max: torch.Tensor      # f32 [total_blocks, 16]
    partial_sum: torch.Tensor      # f32 [total_blocks, 16]
    partial_output: torch.Tensor   # f32 [total_blocks, 16, 128]
    output: torch.Tensor           # bf16 [B, Hq, 128]
    total_blocks: int
    block_n: int = 128
    hierarchical_group_blocks: int = 64
    empty_bf16: torch.Tensor | None = None


def _num_cus(device: torch.device) -> int:
    return int(torch.cuda.get_device_properties(device).multi_processor_count)


def _segments(cache: ThreePrecisionCache, extra_int2: int = 0):
    """(kind, lo, hi, v_delta) K-arena ranges of the FP, INT4 and INT2 pools and of the generated
    tokens: a V row is K position - v_delta.  ``extra_int2`` adds tokens to the tier that generated
    tokens flush into (the INT2 pool, the INT4 pool with INT4 generated values, the FP pool of a
    matched-FP cache).

    With INT4 generated values the INT4 pool is two runs, as the reference's mixed reference
    reassembles it (triton_fourq_attention.py:95-111): its static tokens at the INT4 segment of the
    K arena, and its generated tokens at ``generated_k_offset`` (after the static INT2 segment),
    whose values follow the static ones in the INT4-V arena."""
    ck = cache.compact_key if cache.compact_key is not None else cache.bf16_key
    if ck is None:
        raise NotImplementedError("the gfx950 decode path requires a compact INT4/INT2-K or a bf16 K arena")
    k_fp, k_i4, k_i2 = ck.segment_offsets
    extra = int(extra_int2)
    int4_values = cache.compact_int4_value is not None and not cache.matched_fp
    s_fp = cache.fp_pool.token_count + (extra if cache.matched_fp else 0)
    s_i4 = cache.int4_pool.token_count
    gen_i4 = 0
    if int4_values:
        static = min(cache.static_int4_tokens, s_i4)
        s_i4, gen_i4 = static, s_i4 - static + extra
    s_i2 = (0 if cache.compact_value is None else cache.compact_value.active_length) \
        + (0 if cache.matched_fp or int4_values else extra)
    out = []
    for kind, lo, n in ((_lib.KIND_FP, k_fp, s_fp), (_lib.KIND_INT4, k_i4, s_i4), (_lib.KIND_INT2, k_i2, s_i2)):
        if n > 0:
            out.append((kind, lo, lo + n, lo))
    if gen_i4 > 0:
        g = int(cache.generated_k_offset)
        out.append((_lib.KIND_INT4, g, g + gen_i4, g - s_i4))
    return out


def _tiles(lo: int, hi: int) -> tuple[int, int]:
    t0 = lo // TILE * TILE
    return t0, -(-(hi - t0) // TILE)


# Relative cost of one 32-token tile per kind (partial kernel, measured on MI355X): the
# planner sizes items so that every workgroup slot gets about the same amount of work.
_TILE_COST = {_lib.KIND_FP: 1.45, _lib.KIND_INT4: 1.0, _lib.KIND_INT2: 1.4, _lib.KIND_RECENT: 1.6}


def _plan_runs(caches: Sequence[ThreePrecisionCache], hkv: int, extra_int2: int = 0) -> list[tuple]:
    """(req, kv head, kind, first tile position, tiles, lo, hi, v_delta) of every pool segment and
    Recent-FP ring, grouped by (request, kv head) in order."""
    runs = []
    for r, c in enumerate(caches):
        ss = _segments(c, extra_int2)
        rcap = c.recent_fp_pool.capacity
        if rcap % TILE:
            raise ValueError("Recent-FP capacity must be a multiple of 32 for the gfx950 decode path")
        for h in range(hkv):
            for kind, lo, hi, vd in ss:
                t0, nt = _tiles(lo, hi)
                runs.append((r, h, kind, t0, nt, lo, hi, vd))
            runs.append((r, h, _lib.KIND_RECENT, 0, rcap // TILE, 0, rcap, 0))
    return runs


def _plan(caches: Sequence[ThreePrecisionCache], hkv: int, num_cus: int, extra_int2: int = 0,
          reqs: torch.Tensor | None = None, k_format: int = _lib.K_INT4, int2_group: int = 32):
    """r2o_plan_work_items over the caches' runs: (work items int64 [n, 16] in launch order, with their
    base pointers when ``reqs`` (host int64 [B, 22] request descriptors) is given, group_begin int32
    [B*hkv + 1]) on the host."""
    runs = _plan_runs(caches, hkv, extra_int2)
    n_runs, n_groups = len(runs), len(caches) * hkv
    cus = max(1, int(num_cus))
    cap = max(_BLOCKS_PER_CU * cus, n_runs)
    cfg = _lib.PlanConfig(num_cus=cus, blocks_per_cu=_BLOCKS_PER_CU, tiles_per_item=_TILES_PER_ITEM_TARGET,
                          waves_per_item=_WAVES_PER_ITEM, min_tiles_per_item=_MIN_TILES_PER_ITEM,
                          late_share=_LATE_SHARE_BY_K.get(k_format, _LATE_SHARE))
    for k in (_lib.KIND_FP, _lib.KIND_INT4, _lib.KIND_INT2, _lib.KIND_RECENT):
        cfg.tile_cost[k] = _TILE_COST[k]
    run_arr = (_lib.PlanRun * n_runs)(*[_lib.PlanRun(*r) for r in runs])
    items = torch.zeros(cap, 16, dtype=torch.int64)
    begins = torch.empty(n_groups + 1, dtype=torch.int32)
    n = ctypes.c_int64(0)
    if reqs is not None:
        reqs = reqs.contiguous()
    _lib.check(_lib.load().r2o_plan_work_items(run_arr, n_runs, ctypes.byref(cfg),
                                               None if reqs is None else reqs.data_ptr(), len(caches), k_format,
                                               int2_group, items.data_ptr(), cap, begins.data_ptr(), n_groups,
                                               ctypes.byref(n)), "r2o_plan_work_items")
    return items[: n.value], begins


def plan_work_items(caches: Sequence[ThreePrecisionCache], hkv: int, num_cus: int, extra_int2: int = 0):
    """Split every (request, kv head, pool segment) into runs of 32-token tiles.

    The partial kernel runs two 4-wave workgroups per CU, so the plan aims at no more than
    2 x CUs items of about equal cost (tiles weighted by kind), each a multiple of 4 tiles (one
    share per wave): all items then start together and finish together (a single-kind plan that
    puts two items on each CU splits its runs unevenly, see _LATE_SHARE).  A small cache aims at
    about _TILES_PER_ITEM_TARGET tiles per item instead, but at no fewer than CUs items.  Items keep a partial
    slot in (request, kv head) order, so the combine reads one contiguous slot range per group,
    and are launched largest first.  The planning runs in native code (r2o_plan_work_items).
    Returns (items [n, 9] int64 in launch order, group_begin [B*hkv + 1] int32) on the host.
    """
    items, begins = _plan(caches, hkv, num_cus, extra_int2)
    return items[:, :9].contiguous(), begins


def max_work_items(num_requests: int, hkv: int, num_cus: int) -> int:
    """Upper bound of ``plan_work_items`` for any cache sizes: the water-filling stops at
    _BLOCKS_PER_CU x CUs items unless the runs alone (one per request, KV head and pool segment,
    at most 5 per head: FP, static INT4, INT2, generated INT4 and the Recent-FP ring) are more."""
    return max(_BLOCKS_PER_CU * max(1, num_cus), 5 * int(num_requests) * int(hkv))


def required_splitk_blocks(cache: ThreePrecisionCache, *, block_n: int = 128, reserve_tokens: int = 0) -> int:
    """Partial-state slots a workspace needs for ``cache`` at any growth (``reserve_tokens`` is
    accepted for the reference's signature; the planner's item count is bounded independently of
    the cache size, so every flush fits)."""
    if block_n < 1:
        raise ValueError("block_n must be positive")
    dev = cache.recent_fp_pool.fp_k.device
    hkv = int(cache.recent_fp_pool.fp_k.shape[0])
    cus = _num_cus(dev) if dev.type == "cuda" else 256
    return max_work_items(1, hkv, cus)


def allocate_splitk_workspace(cache: ThreePrecisionCache, *, num_query_heads: int = 16, block_n: int = 128,
                              reserve_tokens: int = 0, device: torch.device | None = None,
                              partial_output_dtype: torch.dtype = torch.float32,
                              hierarchical_group_blocks: int = 64, batch_size: int = 1,
                              total_blocks: int | None = None) -> SplitKWorkspace:
    if partial_output_dtype not in (torch.float16, torch.float32):
        raise ValueError("partial_output_dtype must be float16 or float32")
    if hierarchical_group_blocks not in (16, 32, 64):
        raise ValueError("hierarchical_group_blocks must be 16, 32, or 64")
    if int(num_query_heads) < 1:
        raise ValueError("num_query_heads must be positive")
    if cache.survivor_count <= 0 and cache.recent_fp_pool.capacity <= 0:
        raise ValueError("cannot allocate workspace for an empty cache")
    dev = device if device is not None else cache.recent_fp_pool.fp_k.device
    total = int(total_blocks) if total_blocks is not None else \
        required_splitk_blocks(cache, block_n=block_n, reserve_tokens=reserve_tokens)
    # Partials stay fp32 whatever the requested dtype: the split-K merge is exact in fp32.
    return SplitKWorkspace(
        partial_max=torch.empty((total, 16), device=dev, dtype=torch.float32),
        partial_sum=torch.empty((total, 16), device=dev, dtype=torch.float32),
        partial_output=torch.empty((total, 16, 128), device=dev, dtype=torch.float32),
        output=torch.empty((int(batch_size), int(num_query_heads), 128), device=dev, dtype=torch.bfloat16),
        total_blocks=total, block_n=int(block_n), hierarchical_group_blocks=int(hierarchical_group_blocks),
        empty_bf16=torch.empty(1, device=dev, dtype=torch.bfloat16),
    )


def allocated_workspace_bytes(workspace: SplitKWorkspace) -> int:
    return int(sum(t.numel() * t.element_size() for t in (workspace.partial_max, workspace.partial_sum,
                                                          workspace.partial_output, workspace.output)))


def _k_format(cache: ThreePrecisionCache) -> int:
    if cache.bf16_key is not None:
        return _lib.K_BF16
    return _lib.K_INT2 if cache.compact_key.bit_width == 2 else _lib.K_INT4


def _request_words(cache: ThreePrecisionCache, ring=None) -> dict[str, int]:
    """Pool pointers of one request; ``ring`` replaces the cache's Recent-FP pool (the private ring
    copy of a stacked executor)."""
    ck, cv = cache.compact_key, cache.compact_value
    fp, i4 = cache.fp_pool, cache.int4_pool
    rec = cache.recent_fp_pool if ring is None else ring
    row = rec.fp_k.dtype
    if row not in (torch.bfloat16, torch.float16):
        raise ValueError("the gfx950 decode path requires bfloat16 or float16 FP-V / Recent-FP rows")
    rows = [t for t in (rec.fp_v, fp.fp_v if fp.token_count else None,
                        cache.bf16_key.rows if cache.bf16_key is not None else None) if t is not None]
    if any(t.dtype != row for t in rows):
        raise ValueError("FP-V, Recent-FP and BF16-K rows of one cache must share one dtype")
    i4_packed = i4.packed_v.packed if i4.token_count or cache.compact_int4_value is not None else None
    i4_scale = i4.packed_v.scale if i4.token_count or cache.compact_int4_value is not None else None
    # per-head stride of the INT4-V rows: the arena's capacity when generated values are INT4
    i4_stride = cache.compact_int4_value.capacity if cache.compact_int4_value is not None else i4.token_count
    if ck is not None:
        kw = {"k_packed": ck.packed.data_ptr(), "k_scale": ck.scale.data_ptr(), "k_zero": ck.zero_point.data_ptr(),
              "k_capacity": ck.capacity, "k_superblocks": ck.superblock_count,
              "k_operands": ck.kernel_operands.data_ptr()}
    else:  # bf16 key rows: the kernel reads k_packed as rows [Hkv, k_capacity, 128]
        kb = cache.bf16_key
        kw = {"k_packed": kb.rows.data_ptr(), "k_scale": 0, "k_zero": 0, "k_capacity": kb.capacity,
              "k_superblocks": 0, "k_operands": 0}
    words = {
        **kw,
        "fp_v": fp.fp_v.data_ptr() if fp.token_count else 0, "fp_stride": fp.token_count,
        "i4_v": i4_packed.data_ptr() if i4_packed is not None else 0,
        "i4_scale": i4_scale.data_ptr() if i4_scale is not None else 0, "i4_stride": i4_stride,
        "i2_v": cv.packed.data_ptr() if cv is not None else 0,
        "i2_scale": cv.scale.data_ptr() if cv is not None else 0,
        "i2_zero": cv.zero_point.data_ptr() if cv is not None else 0,
        "i2_stride": cv.capacity if cv is not None else 0,
        "recent_k": rec.fp_k.data_ptr(), "recent_v": rec.fp_v.data_ptr(), "recent_capacity": rec.capacity,
        "recent_length": rec.length_device.data_ptr(), "recent_global": rec.global_index_buffer.data_ptr(),
        "recent_logical": rec.logical_position_buffer.data_ptr(),
        "recent_page_lengths": rec.page_index.lengths.data_ptr(),
    }
    return {k: int(v) for k, v in words.items()}


def _request_desc(cache: ThreePrecisionCache) -> list[int]:
    words = _request_words(cache)
    return [words[f] for f in _lib.REQUEST_FIELDS]


@dataclass
class SplitKExecutor:
    caches: list
    workspace: SplitKWorkspace
    reqs: torch.Tensor          # device int64 [B, 22]
    items: torch.Tensor         # device int64 [n, 16] (r2o_work_item rows)
    group_begin: torch.Tensor   # device int32 [B*Hkv + 1]
    n_items: int
    num_query_heads: int
    num_key_value_heads: int
    head_dim: int = 128
    superblock: int = 32
    int2_group: int = 32
    page_size: int = 32
    output_hadamard: bool = False
    block_n: int = 128
    batched: bool = False
    host_items: torch.Tensor | None = None
    host_group_begin: torch.Tensor | None = None  # host int32 copy of group_begin (inline slot ranges)
    # Stacked executors (stack_homogeneous_splitk_executors) own a copy of each request's Recent-FP
    # ring and track its length here, as the reference's batched_recent / batched_recent_lengths
    # (triton_fourq_splitk.py:1232-1241, 1543-1546): the source caches are never written.
    batched_recent: list | None = None
    batched_recent_lengths: list | None = None
    # [B, Hkv, 128] rows of the ring dtype: with a folded rotation (FusedRotary) the partial pass writes
    # the rotated appended K / V rows here and the combine's fused append copies them into the ring
    rotated_k: torch.Tensor | None = None
    rotated_v: torch.Tensor | None = None
    _keep: list = field(default_factory=list)
    _template: tuple | None = field(default=None, repr=False, compare=False)

    @property
    def cache(self) -> ThreePrecisionCache:
        return self.caches[0]

    @property
    def total(self) -> int:
        return self.n_items

    def _static_params(self) -> _lib.DecodeParams:
        """The launch arguments that stay the same from call to call, built once per executor (again if
        its workspace or output transform is replaced).  Building the whole ctypes struct per call
        cost about as much host time as one of the two launches."""
        t = self._template
        if t is not None and t[0] is self.workspace and t[1] == self.output_hadamard:
            return t[2]
        p = _lib.DecodeParams()
        ws = self.workspace
        p.reqs, p.items, p.group_begin = self.reqs.data_ptr(), self.items.data_ptr(), self.group_begin.data_ptr()
        if self.host_group_begin is not None:
            p.group_begin_host = self.host_group_begin.data_ptr()
        p.n_items = self.n_items
        p.partial_max, p.partial_sum = ws.partial_max.data_ptr(), ws.partial_sum.data_ptr()
        p.partial_out = ws.partial_output.data_ptr()
        p.partial_capacity = min(int(ws.partial_max.shape[0]), int(ws.partial_sum.shape[0]),
                                 int(ws.partial_output.shape[0]))
        p.batch, p.hq, p.hkv = len(self.caches), self.num_query_heads, self.num_key_value_heads
        p.superblock, p.int2_group, p.page_size = self.superblock, self.int2_group, self.page_size
        p.row_dtype = _lib.dtype_code(self.caches[0].recent_fp_pool.fp_k.dtype)
        p.output_hadamard = int(self.output_hadamard)
        p.k_format = _k_format(self.caches[0])
        p.sm_scale = float(self.head_dim ** -0.5)
        self._template = (ws, self.output_hadamard, p)
        return p

    def _params(self, query: torch.Tensor, out: torch.Tensor, append, *,
                step_positions: torch.Tensor | None = None, rotary=None) -> _lib.DecodeParams:
        """Launch arguments.  With ``step_positions`` (device int64 [B, 2]) the launch runs in
        device-state mode: ring lengths and append positions are read (and advanced) on the device,
        so the same arguments stay valid for every later step (graph capture).  ``query`` and the
        appended rows are [B, H, 128] with unit strides inside a request (``_row_stride``); ``rotary``
        (a ``FusedRotary``) folds the decode step's rotation into the launch."""
        p = _lib.DecodeParams.from_buffer_copy(self._static_params())
        if step_positions is not None:
            p.step_positions = step_positions.data_ptr()
        p.query, p.out = query.data_ptr(), out.data_ptr()
        if rotary is not None:
            p.query_batch_stride = _row_stride(query, self.num_query_heads, "query")
        elif not query.is_contiguous():
            raise ValueError("strided query rows need a folded rotation (FusedRotary); pass a contiguous query")
        p.q_dtype = _lib.dtype_code(query.dtype)
        lengths = self._ring_lengths()
        p.recent_len[: len(lengths)] = lengths  # one ctypes slice store: ~0.1 us per request less than a loop
        if append is not None:
            ak, av, gidx, lpos = append
            p.append_k, p.append_v, p.do_append = ak.data_ptr(), av.data_ptr(), 1
            if rotary is not None:
                sk = _row_stride(ak, self.num_key_value_heads, "append K")
                if _row_stride(av, self.num_key_value_heads, "append V") != sk:
                    raise ValueError("append K/V must share one layout")
                p.append_batch_stride = sk
            elif not (ak.is_contiguous() and av.is_contiguous()):
                raise ValueError("strided append K/V rows need a folded rotation (FusedRotary)")
            b = len(self.caches)
            p.append_global[:b] = gidx  # lists of b ints (_per_request)
            p.append_logical[:b] = lpos
        if rotary is not None:
            rotary.fill(p, len(self.caches), query.device)
            p.rotated_k, p.rotated_v = self.rotated_k.data_ptr(), self.rotated_v.data_ptr()
        return p

    def _ring_lengths(self) -> list[int]:
        if self.batched_recent_lengths is not None:
            return list(self.batched_recent_lengths)
        return [int(c.recent_fp_pool.active_length) for c in self.caches]

    def __call__(self, query: torch.Tensor, append=None, *, rotary=None) -> torch.Tensor:
        """The split-K decode call (partial + combine), with the fused Recent-FP append when ``append`` =
        (K, V, global index, logical position) is given.  With ``rotary`` (a ``FusedRotary``) the query
        and the appended rows are the raw projections and the launch applies the decode step's mRoPE
        (and FWHT) itself, in place of a separate ``qwen_qk_mrope`` launch (an extension of the
        reference's call, which takes rotated rows)."""
        p, query, fused = self._prepare_call(query, append, self.workspace.output, rotary)
        self._launch(p, query.device)
        self._finish_call(fused)
        return self.workspace.output

    def call_noalloc(self, query: torch.Tensor, append=None, *, out: torch.Tensor | None = None,
                     rotary=None) -> torch.Tensor:
        """``__call__`` through ``r2o_decode_noalloc``: the partial states live in the library's
        per-GPU device array instead of the workspace, and nothing is allocated (unless ``append``
        rows need a 16-byte-aligned copy).  At most ``_lib.NOALLOC_MAX_ITEMS`` work items; calls that
        overlap on one GPU race on that array.  ``out`` (bf16 [B, Hq, 128]) defaults to the
        workspace's output."""
        out = self.workspace.output if out is None else out
        if out.dtype != torch.bfloat16 or not out.is_contiguous():
            raise ValueError("split-K output must be a contiguous bfloat16 tensor")
        if self.n_items > _lib.NOALLOC_MAX_ITEMS:
            raise ValueError(f"workspace-free decode holds at most {_lib.NOALLOC_MAX_ITEMS} work items")
        p, query, fused = self._prepare_call(query, append, out, rotary)
        p.partial_max = p.partial_sum = p.partial_out = None
        p.partial_capacity = 0
        _noalloc_init(query.device)
        _lib.check(_lib.load().r2o_decode_noalloc(ctypes.byref(p), ctypes.c_void_p(_lib.stream_of(query.device))),
                   "r2o_decode_noalloc")
        self._finish_call(fused)
        return out

    def _prepare_call(self, query: torch.Tensor, append, out: torch.Tensor, rotary=None):
        """Checks of a decode call (before any launch) and its launch arguments.  Contiguous rows
        without a folded rotation (every call of the manager) are checked as they are: slicing the
        token axis away costs ~1 us of host time per tensor, so only the other rows are sliced."""
        b = len(self.caches)
        strided = rotary is not None
        # contiguous, as the reference requires; with a folded rotation also rows readable in place (a
        # view into a fused QKV projection: unit strides inside a request, requests a multiple of 8
        # elements apart)
        shape = tuple(query.shape)
        if len(shape) == 4 and shape[2] == 1:
            shape = (shape[0], shape[1], shape[3])
            if strided or not query.is_contiguous():
                query = query[:, :, 0]
        if shape != (b, self.num_query_heads, self.head_dim) or query.device != out.device \
                or not (query.is_contiguous() or (strided and _row_layout_ok(query, self.num_query_heads))):
            raise ValueError("query does not match prepared split-K executor")
        if tuple(out.shape) != (b, self.num_query_heads, self.head_dim):
            raise ValueError("split-K workspace geometry is inconsistent")
        fused = None
        if append is not None:
            ak, av, gidx, lpos = append
            n = b * self.num_key_value_heads * self.head_dim
            if ak.device != query.device or av.device != query.device:
                raise ValueError("append K/V must be contiguous [B,Hkv,1,D] or [B,Hkv,D]")
            if ak.ndim == 4 and (strided or not (ak.is_contiguous() and av.is_contiguous())):
                ak, av = ak[:, :, 0], av[:, :, 0]
            if ak.is_contiguous() and av.is_contiguous():
                if ak.numel() != n or av.numel() != n:
                    raise ValueError("append K/V must be contiguous [B,Hkv,1,D] or [B,Hkv,D]")
                if ak.data_ptr() % 16 or av.data_ptr() % 16:  # the kernels move the rows in 16-byte pieces
                    ak, av = ak.clone(), av.clone()
            else:  # views of a projection row: with a folded rotation only
                shape = (b, self.num_key_value_heads, self.head_dim)
                if not strided or tuple(ak.shape) != shape or tuple(av.shape) != shape:
                    raise ValueError("append K/V must be contiguous [B,Hkv,1,D] or [B,Hkv,D]")
                if not _row_layout_ok(ak, self.num_key_value_heads) or not _row_layout_ok(av, self.num_key_value_heads) \
                        or ak.stride() != av.stride():
                    ak, av = ak.contiguous().clone(), av.contiguous().clone()
            ring_dtype = self.caches[0].recent_fp_pool.fp_k.dtype
            if ak.dtype != ring_dtype or av.dtype != ring_dtype:
                raise ValueError(f"append K/V must be {ring_dtype} like the Recent-FP ring")
            capacity = self.caches[0].recent_fp_pool.capacity
            if self.batched_recent_lengths is not None:
                if max(self.batched_recent_lengths) >= capacity:
                    raise RuntimeError("prepared batched executor cannot fuse an append into a full Recent-FP pool")
            else:
                for c in self.caches:
                    rec = c.recent_fp_pool
                    if rec.active_length is None or rec.active_length >= rec.capacity:
                        raise RuntimeError(
                            "prepared batched executor cannot fuse an append into a full Recent-FP pool"
                            if self.batched else "prepared executor cannot fuse an append into a full Recent-FP pool")
            gl = _per_request(gidx, b)
            lp = _per_request(lpos, b)
            fused = (ak, av, gl, lp)
        if rotary is not None and query.dtype != self.caches[0].recent_fp_pool.fp_k.dtype:
            raise ValueError("Q/K device and dtype must match")
        return self._params(query, out, fused, rotary=rotary), query, fused

    def _finish_call(self, fused) -> None:
        # A stacked executor advances its private ring lengths; a B=1 executor leaves the cache's
        # host length to the caller (qwen_sspa_attention.py:1824-1826), as the reference does.
        if fused is not None and self.batched_recent_lengths is not None:
            self.batched_recent_lengths[:] = [n + 1 for n in self.batched_recent_lengths]


    @staticmethod
    def _launch(p: _lib.DecodeParams, device: torch.device) -> None:
        # one host call for the partial and combine launches (r2o_decode): each ctypes crossing costs
        # ~2 us of host time, which launch-bound small caches pay per call
        _lib.check(_lib.load().r2o_decode(ctypes.byref(p), ctypes.c_void_p(_lib.stream_of(device))), "r2o_decode")


_NOALLOC_READY: set[int] = set()


def _noalloc_init(device: torch.device) -> None:
    """Look up the device's partial-state array once (r2o_decode_noalloc_init), so that a later
    call under HIP graph capture makes no runtime lookup."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _NOALLOC_READY:
        _lib.call("r2o_decode_noalloc_init", index)
        _NOALLOC_READY.add(index)


def _row_layout_ok(t: torch.Tensor, heads: int) -> bool:
    """Whether [B, heads, 128] rows can be read in place: unit strides inside a request, whole 16-byte
    pieces, requests apart by a multiple of 8 elements without overlapping."""
    if t.ndim != 3 or int(t.shape[1]) != heads or int(t.shape[2]) != 128:
        return False
    if t.stride(2) != 1 or (heads > 1 and t.stride(1) != 128) or t.data_ptr() % 16:
        return False
    return int(t.shape[0]) == 1 or (t.stride(0) % 8 == 0 and t.stride(0) >= heads * 128)


def _row_stride(t: torch.Tensor, heads: int, what: str) -> int:
    """r2o_decode_params' batch stride of [B, heads, 128] rows (0: dense)."""
    if not _row_layout_ok(t, heads):
        raise ValueError(f"{what} rows must be [B,{heads},128] with unit strides inside a request")
    dense = heads * 128
    return 0 if int(t.shape[0]) == 1 or t.stride(0) == dense else int(t.stride(0))


def _per_request(value, b: int) -> list[int]:
    t = type(value)  # the manager's plain ints and lists of ints first (host time on every call)
    if t is int:
        return [value] * b
    if (t is list or t is tuple) and len(value) == b:
        for v in value:
            if type(v) is not int:
                break
        else:
            return list(value)
    if isinstance(value, int):
        return [int(value)] * b
    if isinstance(value, (list, tuple)) and all(isinstance(v, int) for v in value):
        vals = list(value)  # plain positions: no tensor round trip (a few microseconds of host time per call)
    else:
        vals = torch.as_tensor(value).reshape(-1).tolist()
    if len(vals) == 1:
        return [int(vals[0])] * b
    if len(vals) != b:
        raise ValueError("batched append indices must contain one value per request")
    return [int(v) for v in vals]


_UPLOAD_STREAMS: dict[int, torch.cuda.Stream] = {}


def _upload_stream(dev: torch.device) -> torch.cuda.Stream:
    """The device's stream for plan uploads (created once, default priority)."""
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = _UPLOAD_STREAMS.get(index)
    if stream is None:
        stream = _UPLOAD_STREAMS[index] = torch.cuda.Stream(device=index)
    return stream


def _upload_plan(dev: torch.device, *host: torch.Tensor) -> list[torch.Tensor]:
    """Device copies of the host tensors of a plan, uploaded as one pinned block on a stream of their
    own.  A host-to-device copy queued behind the launches already on the compute stream could make
    the host wait until they had drained (milliseconds at a flush step, after which the GPU idled
    while the host re-planned); on its own stream the copy runs at once.  The device block is
    allocated on the upload stream and marked as used by the compute stream, so the allocator reuses
    it only after the compute stream's later work has run, and the compute stream waits for the copy
    before its next launch."""
    align = 256
    offsets, total = [], 0
    for t in host:
        offsets.append(total)
        total += -(-t.numel() * t.element_size() // align) * align
    staging = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    for t, o in zip(host, offsets):
        raw = t.contiguous().reshape(-1).view(torch.uint8)
        staging[o : o + raw.numel()].copy_(raw)
    compute = torch.cuda.current_stream(dev)
    side = _upload_stream(dev)
    with torch.cuda.stream(side):
        block = torch.empty(total, dtype=torch.uint8, device=dev)
        block.copy_(staging, non_blocking=True)
    block.record_stream(compute)
    compute.wait_stream(side)
    return [block[o : o + t.numel() * t.element_size()].view(t.dtype).view(t.shape) for t, o in zip(host, offsets)]


def _build_executor(caches: Sequence[ThreePrecisionCache], workspace: SplitKWorkspace, *, output_hadamard: bool,
                    block_n: int, batched: bool, rings: Sequence | None = None) -> SplitKExecutor:
    """Plan the work items and resolve the pool pointers of ``caches``.  ``rings`` (one Recent-FP
    pool per request) replaces the caches' own rings: the kernels then read and append to those."""
    first = caches[0]
    rec = first.recent_fp_pool
    if rec.fp_k is None or rec.fp_k.ndim != 3:
        raise ValueError("Recent-FP pool must expose [Hkv,capacity,D] K storage")
    if rec.length_device is None:
        raise ValueError("Recent-FP pool must expose a device-side active length")
    hkv, head_dim = int(rec.fp_k.shape[0]), int(rec.fp_k.shape[2])
    hq = int(workspace.output.shape[1])
    if head_dim != 128:
        raise ValueError("split-K executor currently requires head_dim=128")
    if hq % hkv:
        raise ValueError("query heads must be divisible by key/value heads")
    if hq // hkv > 16:
        raise ValueError("split-K executor supports at most 16 GQA heads per KV head")
    if len(caches) > _lib.MAX_BATCH:
        raise ValueError(f"split-K executor supports at most {_lib.MAX_BATCH} requests per launch")
    kf = _k_format(first)
    bf16k = kf == _lib.K_BF16
    sb = 32 if bf16k else first.compact_key.superblock_size
    group = 32 if first.compact_value is None else first.compact_value.group_size
    for r, c in enumerate(caches):
        if _k_format(c) != kf or c.recent_fp_pool.fp_k.dtype != rec.fp_k.dtype \
                or (not bf16k and c.compact_key.superblock_size != sb) \
                or (c.compact_value is not None and c.compact_value.group_size != group) \
                or int(c.recent_fp_pool.fp_k.shape[0]) != hkv or c.page_size != first.page_size:
            raise ValueError(f"batched split-K geometry differs for request {r}")
    dev = workspace.output.device
    words = [_request_words(c, None if rings is None else rings[r]) for r, c in enumerate(caches)]
    host_reqs = torch.tensor([[w[f] for f in _lib.REQUEST_FIELDS] for w in words], dtype=torch.int64)
    host_items, begins = _plan(caches, hkv, _num_cus(dev), reqs=host_reqs, k_format=kf, int2_group=group)
    n = int(host_items.shape[0])
    if n > workspace.total_blocks:
        raise ValueError("workspace block capacity is smaller than the active cache")
    reqs, items, group_begin = _upload_plan(dev, host_reqs, host_items, begins)
    rotated = torch.empty((2, len(caches), hkv, head_dim), device=dev, dtype=rec.fp_k.dtype)
    return SplitKExecutor(
        caches=list(caches), workspace=workspace, reqs=reqs, items=items, group_begin=group_begin,
        n_items=n, num_query_heads=hq, num_key_value_heads=hkv, head_dim=head_dim, superblock=sb, int2_group=group,
        page_size=first.page_size, output_hadamard=bool(output_hadamard), block_n=block_n, batched=batched,
        host_items=host_items, host_group_begin=begins.contiguous(),
        batched_recent=None if rings is None else list(rings),
        batched_recent_lengths=None if rings is None else [int(r.active_length) for r in rings],
        rotated_k=rotated[0], rotated_v=rotated[1],
    )


def prepare_splitk_executor(cache: ThreePrecisionCache, workspace: SplitKWorkspace, *, block_n: int = 128,
                            num_warps: int = 8, num_stages: int = 2, reduce_num_warps: int = 8,
                            use_tensor_cores_qk: bool = True, use_tensor_cores_pv: bool = False,
                            broadcast_k_metadata: bool = False, single_request_fastpath: bool | None = None,
                            tight_metadata_rows: bool | None = None, output_hadamard: bool = False,
                            hierarchical_reduce: bool = True) -> SplitKExecutor:
    if workspace.block_n != block_n:
        raise ValueError("cache/workspace is incompatible with a mixed split-K executor")
    if int(workspace.output.shape[0]) != 1:
        raise ValueError("split-K workspace geometry is inconsistent")
    return _build_executor([cache], workspace, output_hadamard=output_hadamard, block_n=block_n, batched=False)


def stack_homogeneous_splitk_executors(executors: Sequence[SplitKExecutor], *,
                                       workspace: SplitKWorkspace | None = None,
                                       throughput_use_tensor_cores_pv: bool = False,
                                       throughput_direct_reduce_max_splits: int = 0) -> SplitKExecutor:
    """One launch pair over several requests; unlike the reference, lengths may differ (ragged).

    As in the reference, the stacked executor keeps its own copy of each request's Recent-FP ring
    (rows, index buffers, page lengths and device length) and its own host lengths, so the same
    executor may be stacked several times ((ex,) * B) and the source caches stay unchanged.  The
    packed history is only read, so it is shared instead of copied.  A fused append fills the
    copies; like the reference, the stacked executor refuses an append into a full ring (a flush is
    a scheduler boundary: re-stack from the source caches, or use ``BatchedDecoder``)."""
    if len(executors) < 2:
        raise ValueError("batched split-K requires at least two executors")
    caches = [e.cache for e in executors]
    first = executors[0]
    for r, e in enumerate(executors[1:], start=1):
        if e.num_query_heads != first.num_query_heads or e.output_hadamard != first.output_hadamard:
            raise ValueError(f"batched split-K executor {r} differs in heads or output transform")
    hkv = first.num_key_value_heads
    dev = first.workspace.output.device
    if workspace is None:
        workspace = allocate_splitk_workspace(caches[0], num_query_heads=first.num_query_heads,
                                              block_n=first.block_n, batch_size=len(caches),
                                              total_blocks=max_work_items(len(caches), hkv, _num_cus(dev)))
    if int(workspace.output.shape[0]) != len(caches):
        raise ValueError("batched workspace output must hold one row per request")
    rings = [_copy_ring(e.cache.recent_fp_pool) for e in executors]
    return _build_executor(caches, workspace, output_hadamard=first.output_hadamard, block_n=first.block_n,
                           batched=True, rings=rings)


def _copy_ring(pool):
    """A private copy of a Recent-FP ring: rows, index buffers, page table and device length."""
    from .cache import PhysicalPageIndex, PrecisionPool

    if any(t is None for t in (pool.fp_k, pool.fp_v, pool.global_index_buffer, pool.logical_position_buffer,
                               pool.length_device)) or pool.active_length is None:
        raise ValueError("batched Recent-FP metadata buffers are incomplete")
    gbuf = pool.global_index_buffer.clone()
    lbuf = pool.logical_position_buffer.clone()
    idx = pool.page_index
    index = PhysicalPageIndex(original_page_ids=idx.original_page_ids.clone(),
                              physical_offsets=idx.physical_offsets.clone(), lengths=idx.lengths.clone(),
                              global_token_indices=gbuf, logical_positions=lbuf)
    return PrecisionPool(name=pool.name, page_index=index, fp_k=pool.fp_k.clone(), fp_v=pool.fp_v.clone(),
                         active_length=int(pool.active_length), capacity=pool.capacity,
                         length_device=pool.length_device.clone(), global_index_buffer=gbuf,
                         logical_position_buffer=lbuf)


def append_recent_fp_triton(cache: ThreePrecisionCache, new_key: torch.Tensor, new_value: torch.Tensor, *,
                            global_token_index: int, logical_position: int) -> None:
    """Append one decode token to the Recent-FP ring with one launch (non-fused path)."""
    pool = cache.recent_fp_pool
    if new_key.ndim == 4:
        new_key, new_value = new_key[0], new_value[0]
    if new_key.shape != new_value.shape or new_key.ndim != 3 or int(new_key.shape[1]) != 1:
        raise ValueError("new K/V must be [Hkv,1,D] or [1,Hkv,1,D]")
    if pool.active_length is None or pool.active_length >= pool.capacity:
        raise RuntimeError("Recent-FP staging buffer has no append capacity")
    if any(v is None for v in (pool.fp_k, pool.fp_v, pool.global_index_buffer, pool.logical_position_buffer,
                               pool.length_device)):
        raise RuntimeError("Recent-FP staging buffers are incomplete")
    _lib.require_device(new_key, "new_key")
    h = int(new_key.shape[0])
    nk = new_key.reshape(h, -1).contiguous()
    nv = new_value.reshape(h, -1).contiguous()
    _lib.call("r2o_recent_append", _lib.ptr(pool.fp_k), _lib.ptr(pool.fp_v), h, pool.capacity, _lib.ptr(nk),
              _lib.ptr(nv), pool.active_length, int(global_token_index), int(logical_position),
              _lib.ptr(pool.length_device), _lib.ptr(pool.global_index_buffer),
              _lib.ptr(pool.logical_position_buffer), _lib.ptr(pool.page_index.lengths), cache.page_size,
              _lib.stream_of(new_key.device))
    pool.active_length += 1


def triton_fwht_128(tensor: torch.Tensor, *, output: torch.Tensor | None = None) -> torch.Tensor:
    """Normalised 128-wide FWHT in one launch (name kept from triton_qwen_mrope.py:325)."""
    if tensor.shape[-1] != 128 or not torch.is_floating_point(tensor):
        raise ValueError("fused FWHT requires a floating tensor with last dimension 128")
    _lib.require_device(tensor, "FWHT input")
    tensor = tensor.contiguous()
    if output is None:
        output = torch.empty_like(tensor)
    elif output.shape != tensor.shape or output.device != tensor.device or output.dtype != tensor.dtype:
        raise ValueError("fused FWHT output must match input shape, device, and dtype")
    _lib.call("r2o_fwht128", _lib.ptr(tensor), _lib.ptr(output), tensor.numel() // 128, _lib.dtype_code(tensor.dtype),
              _lib.stream_of(tensor.device))
    return output
