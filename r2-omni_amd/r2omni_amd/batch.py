"""Batched decode steps with flushes inside the batch and a HIP graph of the per-step launches.

The reference batches decode only for homogeneous requests whose generation fits the Recent-FP
ring: ``enable_homogeneous_decode_batch`` (r2omni/sspa/integration/qwen_sspa_attention.py:278-317)
stacks B=1 executors, and a step fuses the ring append into the split-K call while the ring has
room (:1794-1807); a flush re-prepares that request's executor (:1808-1818).  ``BatchedDecoder``
runs one (partial + combine) launch pair per step over requests of any lengths, flushes each
request whose ring is full before the step (``flush_full_recent_pool``, the flush half of
``append_generated_token``, dynamic_fourq_cache.py:185-253), re-plans the work items only after a
flush, and can replay the launch pair from a captured HIP graph: the kernels then read the ring
lengths and advance the (global, logical) positions on the device, so the captured arguments
stay valid until the next flush.
"""
from __future__ import annotations

from typing import Sequence

import torch

from .cache import DynamicCacheStats, ThreePrecisionCache, flush_full_recent_pool
from .splitk import (
    SplitKExecutor,
    _build_executor,
    _num_cus,
    _per_request,
    allocate_splitk_workspace,
    max_work_items,
)


def _capture_launches(device: torch.device, side: torch.cuda.Stream, launch) -> torch.cuda.CUDAGraph:
    """Capture ``launch()`` into a HIP graph on ``side``, a stream kept for the captures of one
    decoder (a fresh pool stream would set up a hardware queue at its first use, milliseconds per
    re-capture), after making it wait for the current stream.  The capture is begun and ended
    directly: ``torch.cuda.graph`` would also synchronise the device, run the Python garbage
    collector and empty the allocator cache on every re-capture."""
    graph = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            launch()
        finally:
            graph.capture_end()
    torch.cuda.current_stream(device).wait_stream(side)
    return graph


class BatchedDecoder:
    """Decode steps over ``caches`` (one per request, same head geometry and K format).

    ``step(query, new_key, new_value, positions)`` returns the workspace's bf16 [B, Hq, 128]
    attention output of the step (query over history + ring + the new token, whose K/V row is
    appended to each ring by the same launch).  Inputs are copied into static buffers, so the
    caller may reuse its tensors; a caller that writes ``query_buffer`` / ``key_buffer`` /
    ``value_buffer`` directly can call ``step_in_place``, and ``bind_inputs`` makes those buffers
    views the caller owns (for instance slices of a fused QKV projection's output).  With ``rotary``
    (a ``FusedRotary`` whose tables the caller rewrites in place every step) the inputs are the raw
    projections and every step's launch applies the mRoPE / FWHT itself.
    """

    def __init__(self, caches: Sequence[ThreePrecisionCache], *, num_query_heads: int,
                 output_hadamard: bool = False, use_graph: bool = True,
                 stats: Sequence[DynamicCacheStats] | None = None, rotary=None):
        self.caches = list(caches)
        if not self.caches:
            raise ValueError("a decode batch needs at least one request")
        # each request appends to (and flushes) its own cache in place: a cache listed twice would
        # take two appends into one ring per step
        rings = [c.recent_fp_pool.fp_k.data_ptr() for c in self.caches]
        if len(set(map(id, self.caches))) != len(self.caches) or len(set(rings)) != len(rings):
            raise ValueError("BatchedDecoder requests must be distinct caches (a cache appears twice)")
        first = self.caches[0].recent_fp_pool
        self.device = first.fp_k.device
        self.hkv = int(first.fp_k.shape[0])
        self.hq = int(num_query_heads)
        self.output_hadamard = bool(output_hadamard)
        self.use_graph = bool(use_graph)
        self.rotary = rotary
        self.stats = list(stats) if stats is not None else [DynamicCacheStats() for _ in self.caches]
        if len(self.stats) != len(self.caches):
            raise ValueError("one DynamicCacheStats per request")
        b = len(self.caches)
        # the planner's item count is bounded whatever the cache sizes: one workspace serves every flush
        self.workspace = allocate_splitk_workspace(self.caches[0], num_query_heads=self.hq, batch_size=b,
                                                   total_blocks=max_work_items(b, self.hkv, _num_cus(self.device)))
        rows = first.fp_k.dtype  # the step's query and appended rows in the cache's row dtype
        self.query_buffer = torch.zeros((b, self.hq, 128), device=self.device, dtype=rows)
        self.key_buffer = torch.zeros((b, self.hkv, 128), device=self.device, dtype=rows)
        self.value_buffer = torch.zeros_like(self.key_buffer)
        self.step_positions = torch.zeros((b, 2), device=self.device, dtype=torch.int64)
        self._next_positions: list[tuple[int, int]] | None = None  # what the device holds for the next step
        self.executor: SplitKExecutor | None = None
        self._graph: torch.cuda.CUDAGraph | None = None
        self._capture_stream: torch.cuda.Stream | None = None
        self._params = None
        self.replans = 0
        self.graph_captures = 0
        self._replan()

    # ------------------------------------------------------------------ planning and capture
    def _replan(self) -> None:
        self._graph = None
        self.executor = _build_executor(self.caches, self.workspace, output_hadamard=self.output_hadamard,
                                        block_n=128, batched=len(self.caches) > 1)
        self._params = self.executor._params(self.query_buffer, self.workspace.output,
                                             (self.key_buffer, self.value_buffer, [0] * len(self.caches),
                                              [0] * len(self.caches)),
                                             step_positions=self.step_positions, rotary=self.rotary)
        self.replans += 1

    def bind_inputs(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
        """Read each step's query [B, Hq, 128] and new K / V rows [B, Hkv, 128] from the caller's tensors
        (in the ring dtype) instead of the decoder's own buffers: contiguous, or, for a decoder with a
        folded rotation, with unit strides inside a request and requests a multiple of 8 elements
        apart (e.g. ``qkv[:, a:b].view(B, H, 128)`` of a fused projection).  They are read when the
        step's launch runs: a captured graph reads them at every replay."""
        from .splitk import _row_layout_ok

        b, rows = len(self.caches), self.caches[0].recent_fp_pool.fp_k.dtype
        for t, heads, what in ((query, self.hq, "query"), (key, self.hkv, "key"), (value, self.hkv, "value")):
            if tuple(t.shape) != (b, heads, 128) or t.dtype != rows or t.device != self.device \
                    or not _row_layout_ok(t, heads):
                raise ValueError(f"bound {what} rows must be [B,{heads},128] of the ring dtype, with unit strides "
                                 "inside a request and requests a multiple of 8 elements apart")
            if self.rotary is None and not t.is_contiguous():
                raise ValueError(f"bound {what} rows must be contiguous without a folded rotation (FusedRotary)")
        if key.stride() != value.stride():
            raise ValueError("bound key and value rows must share one layout")
        self.query_buffer, self.key_buffer, self.value_buffer = query, key, value
        self._replan()

    def _capture(self) -> None:
        # one eager launch first (no append, host-provided lengths: it only rewrites the output) so
        # that nothing is loaded or initialised for the first time while the stream is capturing
        self.executor._launch(self.executor._params(self.query_buffer, self.workspace.output, None, rotary=self.rotary),
                              self.device)
        if self._capture_stream is None:
            self._capture_stream = torch.cuda.Stream(device=self.device)
        self._graph = _capture_launches(self.device, self._capture_stream,
                                        lambda: self.executor._launch(self._params, self.device))
        self.graph_captures += 1

    # ------------------------------------------------------------------------------ steps
    def step(self, query: torch.Tensor, new_key: torch.Tensor, new_value: torch.Tensor, *,
             global_token_index, logical_position) -> torch.Tensor:
        b = len(self.caches)
        if query.ndim == 4:
            query = query[:, :, 0]
        if new_key.ndim == 4:
            new_key, new_value = new_key[:, :, 0], new_value[:, :, 0]
        if tuple(query.shape) != (b, self.hq, 128):
            raise ValueError("query must be [B, Hq, 128] for the prepared batch")
        if tuple(new_key.shape) != (b, self.hkv, 128) or new_value.shape != new_key.shape:
            raise ValueError("new K/V must be [B, Hkv, 128] or [B, Hkv, 1, 128]")
        self.query_buffer.copy_(query)
        self.key_buffer.copy_(new_key)
        self.value_buffer.copy_(new_value)
        return self.step_in_place(global_token_index=global_token_index, logical_position=logical_position)

    def _prepare(self, global_token_index, logical_position) -> bool:
        """Flush full rings, re-plan after a flush and load the step's positions if they are not the
        previous step's + 1.  Returns whether the launch arguments changed (a new plan)."""
        b = len(self.caches)
        gl = _per_request(global_token_index, b)
        lp = _per_request(logical_position, b)
        flushed = False
        for cache, stats in zip(self.caches, self.stats):
            flushed |= flush_full_recent_pool(cache, stats)
        if flushed:
            self._replan()
        want = list(zip(gl, lp))
        if want != self._next_positions:  # the device positions only advance by one per step
            self.step_positions.copy_(torch.tensor(want, dtype=torch.int64))
        self._want = want
        return flushed

    def _advance(self) -> None:
        """Host bookkeeping after the step's launch pair (the device advanced itself)."""
        for cache, stats in zip(self.caches, self.stats):
            cache.recent_fp_pool.active_length += 1
            stats.appended_tokens += 1
        self._next_positions = [(g + 1, l + 1) for g, l in self._want]

    def step_in_place(self, *, global_token_index, logical_position) -> torch.Tensor:
        self._prepare(global_token_index, logical_position)
        if self.use_graph:
            if self._graph is None:
                self._capture()
            self._graph.replay()
        else:
            self.executor._launch(self._params, self.device)
        self._advance()
        return self.workspace.output


class DecodeStepGraph:
    """One HIP graph holding the launch pairs of every layer of a decode step.

    ``layers`` are per-layer ``BatchedDecoder``s over the same requests (their rings fill and flush
    together, as every layer appends one token per step).  ``step_in_place`` flushes and re-plans the
    layers that need it, captures the step again only then, and otherwise replays one graph for
    all layers; each layer's inputs are its decoder's ``query_buffer`` / ``key_buffer`` /
    ``value_buffer``.
    """

    def __init__(self, layers: Sequence[BatchedDecoder]):
        self.layers = list(layers)
        if not self.layers:
            raise ValueError("a decode step needs at least one layer")
        self.device = self.layers[0].device
        self._graph: torch.cuda.CUDAGraph | None = None
        self._capture_stream = torch.cuda.Stream(device=self.device)
        self.graph_captures = 0

    def _capture(self) -> None:
        for d in self.layers:  # eager warm-up without append (rewrites the outputs only)
            d.executor._launch(d.executor._params(d.query_buffer, d.workspace.output, None, rotary=d.rotary),
                               self.device)

        def launches():
            for d in self.layers:
                d.executor._launch(d._params, self.device)

        self._graph = _capture_launches(self.device, self._capture_stream, launches)
        self.graph_captures += 1

    def step_in_place(self, *, global_token_index, logical_position) -> list[torch.Tensor]:
        changed = False
        for d in self.layers:
            changed |= d._prepare(global_token_index, logical_position)
        if changed or self._graph is None:
            self._capture()
        self._graph.replay()
        for d in self.layers:
            d._advance()
        return [d.workspace.output for d in self.layers]
