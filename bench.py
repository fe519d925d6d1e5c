"""Benchmark of the gfx950 SSPA packed-KV decode attention (one line of JSON on stdout).

Workload (the headline decode shape): Qwen2.5-Omni-7B attention geometry
(28 query / 4 KV heads, head_dim 128), batch 4 with ragged contexts 8k/16k/32k/64k, INT4 keys,
BF16/INT4/INT2 value pages at 15/45/40 %, 128-token BF16 Recent-FP window.  Synthetic seeded
data.  A step is one decode-attention layer call (split-K partial + combine) over the batch.
To make the bytes come from HBM rather than the 256 MB Infinity Cache, the steps rotate over
``--layers`` distinct layer caches (default 8, 8 x 80 MB).

Reported: ``value`` = algorithmic GB/s of a layer call, ``ms_per_step`` = time per layer call,
``roofline`` for the dominant partial kernel (its average duration from HIP events on its
stream), ``cpu_baseline`` = the reference's CPU dequantise+attention path (restated in torch) on
the same packed data, ``hbm_copy`` / ``hbm_read`` = the box's measured device copy and streaming-read
rates, ``drop_in_call`` = the same call through the Python drop-in ``SplitKExecutor.__call__``,
``graph_call`` = the same calls replayed from a HIP graph (no host launch cost),
``dma_floor`` = the time a compute-free kernel of the partial kernel's launch shape and DMA pattern
takes to move the call's bytes, and ``e2e`` = the rest of the metric: configuration 4's decode tok/s (a random-init 28-layer
Qwen2.5-Omni-7B decoder, batch 8 x 32k, 128 greedy steps on this path).  Other modes (--prefill, --decode-steps, --sweep, --e2e)
print their own line instead.
"""
from __future__ import annotations

import argparse
import contextlib
import ctypes
import dataclasses
import gc
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "r2-omni_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _clock_warmup(dev, ms: float = 50.0) -> None:
    """Keep the GPU busy for ``ms`` milliseconds right before a timed window, with memory-bound work
    (device copies of 256 MiB) like the kernels measured here: after the host-side setup the clocks
    are low and take ~20 ms of load to come up.  (Matrix products as the warm-up load measured ~2 %
    slower decode calls afterwards than this build's own calls did; an idle gap of 50 ms, ~12 %.)"""
    import torch

    a = torch.empty(1 << 28, device=dev, dtype=torch.uint8)
    b = torch.empty_like(a)
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(8):
            b.copy_(a)
        torch.cuda.synchronize()
    del a, b


@contextlib.contextmanager
def _gc_paused():
    """Run a timed region with Python's garbage collector paused, as ``timeit`` does: a full
    collection of this process takes tens of milliseconds, a pause of the Python host that would
    otherwise land in a timed window now and then.  No collection is run on entry: that many idle
    milliseconds just before the window let the GPU clocks fall, and the timed launches then paid
    for the ramp back up (~2 us per cfg2 layer call over 200 calls)."""
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was_enabled:
            gc.enable()


def _time_events(fn, steps: int, stream, warm_ms: float = 30.0, lead: int = 16) -> float:
    """Average milliseconds of ``fn(i)`` over ``steps`` calls, HIP events on ``stream``.

    Steady state: ``fn`` itself runs untimed for ``warm_ms`` milliseconds first (synchronising every 64
    calls, so the host never runs far ahead), which brings the GPU clocks up under the very load that
    is timed, and then ``lead`` more untimed calls are queued right before the start event, with no
    host synchronisation in between, so that the timed calls start on a busy GPU and none of them
    waits on the host's first launch."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with _gc_paused():
        t0, i = time.perf_counter(), 0
        while (time.perf_counter() - t0) * 1e3 < warm_ms:
            for _ in range(64):
                fn(i)
                i += 1
            torch.cuda.synchronize()
        for _ in range(lead):
            fn(i)
            i += 1
        start.record(stream)
        for k in range(steps):
            fn(i + k)
        stop.record(stream)
        torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps  # ms


def cpu_baseline(caches, queries, hq: int, budget_s: float = 12.0) -> dict:
    """Time the reference's CPU path restated in torch (oracle/torch_path.py: every pool dequantised
    with torch ops on each call, as triton_mixed_reference does, then the softmax states merged) on
    the same packed data, on all of this process's host cores."""
    import numpy as np
    import torch

    from oracle import torch_path
    from oracle.cache import OracleCache
    from r2omni_amd.workloads import algorithmic_bytes

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    oc_list = []
    for c in caches:
        ck, cv, rec = c.compact_key, c.compact_value, c.recent_fp_pool
        h = int(rec.fp_k.shape[0])
        fp = c.fp_pool.fp_v.float().cpu().numpy() if c.fp_pool.token_count else np.zeros((h, 0, 128), np.float32)
        i4 = c.int4_pool
        if ck is not None:
            kw = dict(variant="int2k" if ck.bit_width == 2 else "int4k", k_packed=ck.packed.cpu().numpy(), k_scale=ck.scale.cpu().numpy(),
                      k_zero=ck.zero_point.cpu().numpy(), k_active=ck.active_length, k_capacity=ck.capacity,
                      k_segments=ck.segment_offsets, superblock=ck.superblock_size)
        else:  # bf16 key rows
            kb = c.bf16_key
            kw = dict(variant="matched" if c.matched_fp else "bf16k", k_rows=kb.rows.float().cpu().numpy(),
                      k_packed=np.zeros((h, 0, 64), np.uint8), k_scale=np.zeros((h, 0, 128), np.float16),
                      k_zero=np.zeros((h, 0, 128), np.uint8), k_active=kb.active_length, k_capacity=kb.capacity,
                      k_segments=kb.segment_offsets, superblock=32)
        if cv is not None:
            v2 = dict(v2_packed=cv.packed.cpu().numpy(), v2_scale=cv.scale.cpu().numpy(),
                      v2_zero=cv.zero_point.cpu().numpy(), v2_active=cv.active_length, v2_capacity=cv.capacity,
                      group=cv.group_size)
        else:
            v2 = dict(v2_packed=np.zeros((h, 0, 32), np.uint8), v2_scale=np.zeros((h, 0, 4, 1), np.float16),
                      v2_zero=np.zeros((h, 0, 4, 1), np.uint8), v2_active=0, v2_capacity=0, group=32)
        a4 = c.compact_int4_value  # INT4 generated values: the INT4 pool's rows are an arena
        gen4 = {} if a4 is None else dict(gen_values="int4", v4_capacity=a4.capacity,
                                          static_i4=c.static_int4_tokens, gen_k_offset=c.generated_k_offset)
        oc = OracleCache(
            dtype="bfloat16", hkv=h, page_size=c.page_size, flush_size=128, fp_v=fp,
            v4_packed=i4.packed_v.packed.cpu().numpy().reshape(h, -1, 64)[:, :i4.token_count] if i4.token_count
            else np.zeros((h, 0, 64), np.uint8),
            v4_scale=i4.packed_v.scale.cpu().numpy()[:, :i4.token_count] if i4.token_count
            else np.zeros((h, 0, 1), np.float32),
            recent_k=rec.fp_k.float().cpu().numpy(), recent_v=rec.fp_v.float().cpu().numpy(),
            recent_active=rec.active_length, recent_global=rec.global_index_buffer.cpu().numpy(),
            recent_logical=rec.logical_position_buffer.cpu().numpy(),
            recent_page_lengths=rec.page_index.lengths.cpu().numpy(),
            pool_tokens=[c.fp_pool.token_count, i4.token_count, v2["v2_active"]], **kw, **v2, **gen4,
        )
        oc_list.append(torch_path.from_oracle(oc))  # the packed cache as torch tensors, as the reference holds it
    qs = [q.float().cpu().numpy() for q in queries]

    def one_pass():
        for tc, q in zip(oc_list, qs):
            torch_path.mixed_reference(q, tc)

    one_pass()  # warm-up
    reps, t0 = 0, time.perf_counter()
    times = []
    while reps < 5 and time.perf_counter() - t0 < budget_s:
        s = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - s)
        reps += 1
    med = sorted(times)[len(times) // 2]
    nbytes = algorithmic_bytes(caches, hq)
    what = "request" if len(caches) == 1 else f"{len(caches)} ragged requests"
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"one decode-attention call over the same {what} (layer 0 of the GPU run), median of "
                      f"{reps} after 1 warm-up: {med * 1e6:.0f} us/call on {threads} threads (torch CPU restatement "
                      "of triton_mixed_reference: every pool dequantised with torch ops per call, fp32 softmax "
                      "states per pool, exact merge)"}


def read_bandwidth(dev, mib: int = 2048, reps: int = 20, blocks: int = 8192) -> dict:
    """The box's read-only HBM rate: one pass of ``r2o_bench_stream_read`` (16-byte nontemporal loads,
    nothing written) over ``mib`` MiB, bytes / time, median of ``reps`` HIP-event timings.  The
    practical ceiling of a read-dominated kernel such as the partial kernel."""
    import torch

    from r2omni_amd.build import BENCH_LIB_PATH

    lib = ctypes.CDLL(BENCH_LIB_PATH)
    lib.r2o_bench_stream_read.restype = ctypes.c_int
    lib.r2o_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_int, ctypes.c_void_p]
    nbytes = mib * (1 << 20)
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(blocks, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def one():
        rc = lib.r2o_bench_stream_read(src.data_ptr(), nbytes, sink.data_ptr(), blocks, 1, stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"r2o_bench_stream_read failed ({rc})")

    for _ in range(3):
        one()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        one()
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b))
    ms = sorted(times)[reps // 2]
    del src, sink
    torch.cuda.empty_cache()
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"GBs": round(gbs, 1), "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 1), "bytes_per_read": nbytes,
            "method": f"one streaming read of {mib} MiB (16-byte nontemporal loads, {blocks} workgroups, nothing "
                      f"written), bytes / time, median of {reps} HIP-event timings"}


def dma_floor(dev, nbytes: int, *, steps: int = 200, warmup: int = 300, blocks: int = 512, tile_kb: int = 4) -> dict:
    """What moving ``nbytes`` costs at the partial kernel's launch shape with no compute:
    ``r2o_bench_dma_read`` (512 blocks of 4 waves, two per CU, each wave streaming its own contiguous
    run of ``tile_kb`` KiB tiles by nontemporal global->LDS DMA, one tile in flight), back-to-back
    launches rotating over 8 buffers (so the bytes come from HBM), timed like the layer calls."""
    import torch

    from r2omni_amd.build import BENCH_LIB_PATH

    lib = ctypes.CDLL(BENCH_LIB_PATH)
    lib.r2o_bench_dma_read.restype = ctypes.c_int
    lib.r2o_bench_dma_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                       ctypes.c_void_p]
    nb = nbytes // (tile_kb * 1024) * (tile_kb * 1024)
    bufs = [torch.empty(nb, dtype=torch.uint8, device=dev) for _ in range(8)]
    sink = torch.zeros(blocks, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def one(i):
        rc = lib.r2o_bench_dma_read(bufs[i % 8].data_ptr(), nb, sink.data_ptr(), blocks, tile_kb, stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"r2o_bench_dma_read failed ({rc})")

    for i in range(warmup):
        one(i)
    ms = _time_events(one, steps, stream)
    del bufs, sink
    torch.cuda.empty_cache()
    gbs = nb / (ms * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 3), "GBs": round(gbs, 1), "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
            "bytes": nb, "method": f"the partial kernel's launch shape without compute: {blocks} blocks x 4 waves "
                                   f"(2 per CU), each wave streaming its own run of {tile_kb} KiB tiles by "
                                   f"nontemporal global->LDS DMA, one tile in flight; {steps} back-to-back launches "
                                   f"over 8 rotated buffers, HIP events"}


def copy_bandwidth(dev, mib: int = 1024, reps: int = 20) -> dict:
    """The box's device-to-device copy rate: a torch copy of ``mib`` MiB, (bytes read + written) /
    time, median of ``reps`` HIP-event timings."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    stream = torch.cuda.current_stream(dev)
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        dst.copy_(src)
        b.record(stream)
        b.synchronize()
        times.append(a.elapsed_time(b))
    ms = sorted(times)[reps // 2]
    moved = 2 * n * 4
    del src, dst
    torch.cuda.empty_cache()
    return {"GBs": round(moved / (ms * 1e-3) / 1e9, 1), "pct_of_peak": round(100 * moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
            "bytes_per_copy": moved, "method": f"device-to-device torch copy of {mib} MiB, (read + write bytes) / "
                                             f"time, median of {reps} HIP-event timings"}


def summarize_pmc(directory: str) -> dict:
    """Mean per-dispatch counter values of a rocprofv3 --pmc CSV run, keyed by kernel then counter."""
    import collections
    import csv
    import glob

    acc = collections.defaultdict(list)
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"]
                kernel = ("decode_partial_kernel" if "decode_partial_kernel" in name else
                          "decode_combine_kernel" if "decode_combine_kernel" in name else
                          "copy" if "copyBuffer" in name else None)
                if kernel:
                    acc[(kernel, row["Counter_Name"])].append(float(row["Counter_Value"]))
    out: dict = {}
    for (kernel, counter), vals in sorted(acc.items()):
        out.setdefault(kernel, {})[counter] = {"mean": sum(vals) / len(vals), "dispatches": len(vals)}
    return out


def summarize_trace(directory: str, tail: int = 200) -> dict:
    """Per-dispatch durations of the decode kernels in a rocprofv3 --kernel-trace CSV run, in launch
    order: partial dispatches followed by a combine (layer calls) apart from back-to-back partial-only
    ones, the combine, and the gap from a partial's end to its combine's start.  Besides the average
    over every dispatch, ``tail_avg_us`` averages the last ``tail`` of each kind: the timed calls,
    after the warm-up calls during which the clocks come up."""
    import csv
    import glob

    rows = []
    for path in glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"]
                kind = ("partial" if "decode_partial_kernel" in name else
                        "combine" if "decode_combine_kernel" in name else None)
                if kind:
                    rows.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]), kind))
    rows.sort()
    acc: dict = {"partial_in_call": [], "partial_only": [], "combine": [], "partial_end_to_combine_start": []}
    for k, (t0, t1, kind) in enumerate(rows):
        if kind == "combine":
            acc["combine"].append(t1 - t0)
            continue
        nxt = rows[k + 1] if k + 1 < len(rows) else None
        if nxt is not None and nxt[2] == "combine":
            acc["partial_in_call"].append(t1 - t0)
            acc["partial_end_to_combine_start"].append(nxt[0] - t1)
        else:
            acc["partial_only"].append(t1 - t0)
    return {key: {"dispatches": len(v), "avg_us": round(sum(v) / len(v) / 1e3, 3) if v else None,
                  "tail_avg_us": round(sum(v[-tail:]) / len(v[-tail:]) / 1e3, 3) if v else None}
            for key, v in acc.items()}


def traffic_from_profile() -> tuple[int | None, str | None]:
    """HBM bytes per partial-kernel launch recorded in the committed PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", "decode_partial_cfg2_hbm_traffic.md")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip()), "profiles/decode_partial_cfg2_hbm_traffic.md"
    return None, None


def prefill_bench(cfg, config_id: int, dev) -> dict:
    """Time build_three_precision_cache (tier-sorted gather + INT4-K / INT4-V / INT2-V packing) for
    the longest request of the configuration; bytes = bf16 K and V read + packed arenas written."""
    import torch

    from r2omni_amd.cache import build_three_precision_cache
    from r2omni_amd.policy import plan_from_pages
    from r2omni_amd.workloads import make_request

    total = max(cfg.lengths)
    data = make_request(cfg, total, seed=7, device=dev)
    plan = plan_from_pages(data.page_offsets, data.page_lengths, data.page_classes, recent_fp_capacity=128,
                           device=dev)

    def build():
        return build_three_precision_cache(data.key, data.value, plan, page_size=cfg.page,
                                           key_quantization_superblock=cfg.superblock, int2_group_size=cfg.group,
                                           compact_key_append_capacity=260, recent_flush_size=128)

    for _ in range(2):
        cache = build()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    start.record(stream)
    for _ in range(reps):
        cache = build()
    stop.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / reps
    hist = int(data.key.shape[1])
    read = 2 * cfg.hkv * hist * 128 * 2
    h = cfg.hkv
    sbs = -(-hist // cfg.superblock)
    written = h * (hist * 64 + sbs * 128 * (2 + 1 + 4) + cache.fp_pool.token_count * 256
                   + cache.int4_pool.token_count * 68 + cache.compact_value.active_length * (32 + 3 * (128 // cfg.group)))
    return {"metric": "prefill cache build (quantise + pack)", "config": f"cfg{config_id} {cfg.name}",
            "tokens": hist, "hkv": cfg.hkv, "us_per_build": round(ms * 1e3, 1),
            "GBs": round((read + written) / (ms * 1e-3) / 1e9, 1), "bytes_read": read, "bytes_written": written,
            "note": "one call of build_three_precision_cache on resident bf16 K/V, host launch gaps included"}


def flush_bench(cfg, config_id: int, dev, flushes: int = 8) -> dict:
    """The flush of a full Recent-FP ring (its oldest 128 tokens quantised and packed into the compact
    K arena and the INT2-V arena, metadata appended, the ring shifted: ``flush_full_recent_pool``) on the
    longest request of the configuration, one layer.  Between timed flushes 128 single-token appends
    refill the ring (untimed).  GPU time from HIP events around the flush's launches; host time from the
    wall clock of the call."""
    import torch

    from r2omni_amd.cache import DynamicCacheStats, append_generated_token, flush_full_recent_pool
    from r2omni_amd.workloads import build_request_cache, make_request

    total = max(cfg.lengths)
    data = make_request(cfg, total, seed=11, device=dev)
    cache = build_request_cache(cfg, data, append_capacity=(flushes + 2) * 128 + 128)
    hist = int(data.key.shape[1]) + cfg.recent
    stats = DynamicCacheStats()
    gen = torch.Generator(device=dev).manual_seed(3)
    h = cfg.hkv
    stream = torch.cuda.current_stream(dev)
    gpu, host = [], []
    pos = hist
    for k in range(flushes + 1):
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        t0 = time.perf_counter()
        if not flush_full_recent_pool(cache, stats):
            raise RuntimeError("the Recent-FP ring was not full")
        t1 = time.perf_counter()
        b.record(stream)
        b.synchronize()
        if k:  # the first flush warms the allocator and the code paths
            gpu.append(a.elapsed_time(b) * 1e3)
            host.append((t1 - t0) * 1e6)
        for _ in range(int(cache.recent_fp_pool.capacity)):  # refill the ring (untimed)
            nk = torch.randn((h, 1, 128), generator=gen, device=dev).to(data.key.dtype)
            nv = torch.randn((h, 1, 128), generator=gen, device=dev).to(data.key.dtype)
            append_generated_token(cache, nk, nv, global_token_index=pos, logical_position=pos, stats=stats)
            pos += 1
    med = lambda v: round(sorted(v)[len(v) // 2], 2)  # noqa: E731
    return {"metric": f"Recent-FP flush (128 tokens -> compact K + {cfg.gen_values.upper()}-V, ring shift), one layer",
            "config": f"cfg{config_id} {cfg.name}", "k_format": cfg.variant, "gen_values": cfg.gen_values,
            "hkv": h, "flush_tokens": 128,
            "flushes": flushes, "us_gpu_median": med(gpu), "us_host_median": med(host),
            "note": "GPU: HIP events around the flush's launches on the compute stream; host: wall clock of "
                    "flush_full_recent_pool (the launches are asynchronous); median over the timed flushes"}


def decode_steps_bench(cfg, config_id: int, dev, steps: int, layers: int) -> dict:
    """Per-step wall time of ``layers`` BatchedDecoder layers over the batch of the configuration:
    eager launches vs one HIP graph per decode step (DecodeStepGraph), flushes inside the run."""
    import torch

    import r2omni_amd as ro
    from r2omni_amd.workloads import build_request_cache, make_request

    out = {"metric": "batched decode step (flush inside the batch)", "config": f"cfg{config_id} {cfg.name}",
           "k_format": cfg.variant, "gen_values": cfg.gen_values, "steps": steps, "layers": layers,
           "requests": len(cfg.lengths)}
    for mode in ("eager", "step_graph"):
        decs, positions = [], None
        for layer in range(layers):
            datas = [make_request(cfg, total, seed=1000 * layer + r, device=dev) for r, total in enumerate(cfg.lengths)]
            caches = [build_request_cache(cfg, d, append_capacity=steps + 512) for d in datas]
            positions = [int(d.key.shape[1]) + cfg.recent for d in datas]
            del datas
            d = ro.BatchedDecoder(caches, num_query_heads=cfg.hq, output_hadamard=True,
                                  use_graph=False)
            gen = torch.Generator(device=dev).manual_seed(5 + layer)
            d.query_buffer.copy_(torch.randn(d.query_buffer.shape, generator=gen, device=dev))
            d.key_buffer.copy_(torch.randn(d.key_buffer.shape, generator=gen, device=dev))
            d.value_buffer.copy_(torch.randn(d.value_buffer.shape, generator=gen, device=dev))
            decs.append(d)
        graph = ro.DecodeStepGraph(decs) if mode == "step_graph" else None

        def one_step():
            nonlocal positions
            if graph is not None:
                graph.step_in_place(global_token_index=positions, logical_position=positions)
            else:
                for d in decs:
                    d.step_in_place(global_token_index=positions, logical_position=positions)
            positions = [p + 1 for p in positions]

        for _ in range(4):  # the rings start full: the first step flushes every request of every layer
            one_step()
        torch.cuda.synchronize()
        _clock_warmup(dev)
        steady = 100
        with _gc_paused():
            t0 = time.perf_counter()
            for _ in range(steady):
                one_step()
            torch.cuda.synchronize()
            t_steady = (time.perf_counter() - t0) / steady
        flushes0 = sum(st.flushed_superblocks for d in decs for st in d.stats)
        with _gc_paused():
            t0 = time.perf_counter()
            for _ in range(steps):
                one_step()
            torch.cuda.synchronize()
            t_all = (time.perf_counter() - t0) / steps
        out[mode] = {"us_per_step_steady": round(t_steady * 1e6, 2),
                     "us_per_layer_call_steady": round(t_steady * 1e6 / layers, 2),
                     "us_per_step_with_flushes": round(t_all * 1e6, 2),
                     "flush_steps_in_timed_run": (sum(st.flushed_superblocks for d in decs for st in d.stats)
                                                  - flushes0) // (layers * len(cfg.lengths)),
                     "graph_captures": graph.graph_captures if graph is not None else 0}
        del decs, graph
        torch.cuda.empty_cache()
    out["note"] = ("host wall clock per decode step (all layers) over back-to-back steps, no per-step sync: "
                   "launch overhead, flush packing, re-plans and graph re-captures included; 'steady' = 100 "
                   "steps without a flush; Python's garbage collector paused in the timed loops")
    return out


class E2EQwenDecoder:
    """Configuration 4: greedy decode of a random-init Qwen2.5-Omni-7B language model on this path.

    Model: 28 layers (``n_layers``), hidden 3584, 28 query / 4 KV heads of 128, SwiGLU 18944, vocab
    152064, RMSNorm 1e-6, mRoPE sections (16, 24, 24) with theta 1e6, bf16 weights N(0, 0.02).  Each of
    ``batch`` sequences of ``context`` seeded random token ids is prefilled through the whole model
    (flash attention); per layer its Hadamard-rotated K/V (keys after RoPE) go into an SSPA cache:
    INT4 keys, BF16/INT4/INT2 value pages drawn per 64-token page at 15/45/40 %, the newest 128 tokens
    in the Recent-FP ring.  Then greedy steps: fused mRoPE + FWHT of Q/K and the FWHT of V in one
    launch, the packed-KV attention with fused append (BatchedDecoder; the first step flushes every ring
    inside the batch), projections / MLP / lm_head as torch GEMMs.  The greedy loop is the reference's
    (qwen_r2omni_decode.py:248-292) with the manager's decode step (qwen_sspa_attention.py:1239-1247,
    1794-1826) in place of HF attention.
    """

    HID, NH, NKV, HD, INTER, VOCAB, EPS = 3584, 28, 4, 128, 18944, 152064, 1e-6
    SECTIONS, RECENT, PAGE, TIERS = (16, 24, 24), 128, 64, (0.15, 0.45, 0.4)

    def __init__(self, dev, *, batch: int, context: int, n_layers: int):
        import torch

        self.dev, self.batch, self.context, self.n_layers = dev, batch, context, n_layers
        bf = torch.bfloat16
        gen = torch.Generator(device=dev).manual_seed(0)
        self.cpu_gen = torch.Generator().manual_seed(0)

        def weight(*shape):
            return (torch.randn(shape, generator=gen, device=dev) * 0.02).to(bf)

        hid, nkv, hd, inter = self.HID, self.NKV, self.HD, self.INTER
        self.layers = []
        for _ in range(n_layers):
            wq, bq, wk, bk = weight(hid, hid), weight(hid), weight(nkv * hd, hid), weight(nkv * hd)
            wv, bv, wo, wg, wu = weight(nkv * hd, hid), weight(nkv * hd), weight(hid, hid), weight(inter, hid), \
                weight(inter, hid)
            # q/k/v and gate/up projections as one GEMM each (the weights stacked along the output dim)
            self.layers.append({"w_qkv": torch.cat((wq, wk, wv)), "b_qkv": torch.cat((bq, bk, bv)), "wo": wo,
                                "w_gu": torch.cat((wg, wu)), "wd": weight(hid, inter),
                                "n1": torch.ones(hid, device=dev, dtype=bf), "n2": torch.ones(hid, device=dev, dtype=bf)})
            del wq, wk, wv, wg, wu
        self.embed, self.lm_head = weight(self.VOCAB, hid), weight(self.VOCAB, hid)
        self.n_final = torch.ones(hid, device=dev, dtype=bf)
        self.inv_freq = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device=dev, dtype=torch.float32) / hd))
        self.kv = None
        self.first = None
        self.prefill_s = 0.0
        self.tiers = None

    # ------------------------------------------------------------------ model pieces
    def rms(self, x, w):
        import torch

        xf = x.float()
        return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.EPS)).to(torch.bfloat16)

    def tables(self, pos):
        """Text positions: the three mRoPE axes are equal; cos/sin [3, B, T, 128] in bf16."""
        import torch

        ang = pos.float()[..., None] * self.inv_freq
        ang = torch.cat([ang, ang], dim=-1)
        return ang.cos().to(torch.bfloat16)[None].expand(3, *ang.shape), \
            ang.sin().to(torch.bfloat16)[None].expand(3, *ang.shape)

    def mlp(self, x, lw):
        import torch.nn.functional as F

        h = self.rms(x, lw["n2"])
        gate, up = F.linear(h, lw["w_gu"]).split(self.INTER, dim=-1)
        return x + F.linear(F.silu(gate) * up, lw["wd"])

    # ------------------------------------------------------------------------- prefill
    def prefill(self) -> None:
        """Every sequence through the model (flash attention); keeps each layer's rotated K/V and the
        first greedy token of every sequence."""
        import torch
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel

        import r2omni_amd as ro

        dev, context, nh, nkv, hd, hid = self.dev, self.context, self.NH, self.NKV, self.HD, self.HID
        t0 = time.perf_counter()
        self.kv = [[None] * self.batch for _ in range(self.n_layers)]
        self.first = torch.empty(self.batch, dtype=torch.int64, device=dev)
        with torch.no_grad():
            for s_i in range(self.batch):
                tok = torch.randint(0, self.VOCAB, (context,), generator=self.cpu_gen).to(dev)
                x = self.embed[tok]
                cos, sin = self.tables(torch.arange(context, device=dev)[None])
                for li, lw in enumerate(self.layers):
                    h = self.rms(x, lw["n1"])
                    q, k, v = F.linear(h, lw["w_qkv"], lw["b_qkv"]).split((nh * hd, nkv * hd, nkv * hd), dim=-1)
                    q = q.reshape(context, nh, hd).transpose(0, 1)[None]
                    k = k.reshape(context, nkv, hd).transpose(0, 1)[None]
                    v = v.reshape(context, nkv, hd).transpose(0, 1)[None].contiguous()
                    q, k = ro.qwen_qk_mrope(q, k, cos, sin, self.SECTIONS)
                    with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                        a = F.scaled_dot_product_attention(q, k.repeat_interleave(nh // nkv, dim=1),
                                                           v.repeat_interleave(nh // nkv, dim=1), is_causal=True)
                    x = x + F.linear(a[0].transpose(0, 1).reshape(context, hid), lw["wo"])
                    x = self.mlp(x, lw)
                    self.kv[li][s_i] = (ro.triton_fwht_128(k[0]), ro.triton_fwht_128(v[0]))
                self.first[s_i] = F.linear(self.rms(x[-1:], self.n_final), self.lm_head).argmax(-1)[0]
                torch.cuda.synchronize()
                _log(f"e2e prefill sequence {s_i + 1}/{self.batch} ({time.perf_counter() - t0:.1f} s)")
        self.prefill_s = time.perf_counter() - t0
        hist = context - self.RECENT
        pages = hist // self.PAGE
        self.tiers = [torch.multinomial(torch.tensor(self.TIERS), pages, replacement=True, generator=self.cpu_gen)
                      for _ in range(self.n_layers * self.batch)]

    def request_data(self, layer: int, seq: int):
        """The cache inputs of one (layer, sequence): history K/V, the ring's 128 newest rows, pages."""
        import torch

        from r2omni_amd.workloads import TIER_CLASS, RequestData

        hist = self.context - self.RECENT
        pages = hist // self.PAGE
        k, v = self.kv[layer][seq]
        classes = torch.tensor(TIER_CLASS, dtype=torch.long)[self.tiers[layer * self.batch + seq]]
        return RequestData(None, k[:, :hist], v[:, :hist], k[:, hist:].transpose(0, 1), v[:, hist:].transpose(0, 1),
                           torch.arange(pages, dtype=torch.long) * self.PAGE,
                           torch.full((pages,), self.PAGE, dtype=torch.long), classes, None)

    def cache_config(self):
        from r2omni_amd.workloads import DecodeConfig

        return DecodeConfig("e2e", self.NH, self.NKV, (self.context,), self.TIERS, recent=self.RECENT, page=self.PAGE)

    def build_caches(self, steps: int):
        import torch

        from r2omni_amd.workloads import build_request_cache

        cfg = self.cache_config()
        out = [[build_request_cache(cfg, self.request_data(li, s_i), append_capacity=steps + 256)
                for s_i in range(self.batch)] for li in range(self.n_layers)]
        torch.cuda.synchronize()
        return out

    # -------------------------------------------------------------------------- decode
    def decode(self, steps: int, use_graph: bool, inspect=None, fused_rotation: bool = True):
        """``steps`` greedy steps from fresh caches: eager launches, or (``use_graph``) the steps
        after the first replayed from one HIP graph per step (the argmax stays outside the graph).
        ``fused_rotation``: each layer's QKV projection is written into one static buffer whose views
        the layer's decoder reads, and the attention call applies the mRoPE / FWHT itself (two launches
        per layer for the attention); otherwise a separate rotation launch writes the decoder's buffers.
        ``inspect(step, decoders)`` runs after each step's synchronisation (not for timing).
        Returns (decode ms from HIP events, tokens [steps, B], whether every step's logits were finite)."""
        import torch
        import torch.nn.functional as F

        import r2omni_amd as ro

        dev, batch, nh, nkv, hd, hid = self.dev, self.batch, self.NH, self.NKV, self.HD, self.HID
        caches = self.build_caches(steps)
        cos_buf = torch.empty(3, batch, 1, hd, device=dev, dtype=torch.bfloat16)
        sin_buf = torch.empty_like(cos_buf)
        qkv_buf = torch.empty(batch, (nh + 2 * nkv) * hd, device=dev, dtype=torch.bfloat16)
        rotary = ro.FusedRotary(cos_buf, sin_buf, self.SECTIONS, True, True) if fused_rotation else None
        decs = [ro.BatchedDecoder(c, num_query_heads=nh, output_hadamard=True, use_graph=False, rotary=rotary)
                for c in caches]
        if fused_rotation:
            for d in decs:  # every layer reads the one projection buffer, written right before its call
                d.bind_inputs(qkv_buf[:, : nh * hd].view(batch, nh, hd),
                              qkv_buf[:, nh * hd : (nh + nkv) * hd].view(batch, nkv, hd),
                              qkv_buf[:, (nh + nkv) * hd :].view(batch, nkv, hd))
        tok = self.first.clone()
        pos_dev = torch.full((1, 1), self.context, dtype=torch.int64, device=dev)
        logits = torch.empty(batch, self.VOCAB, device=dev, dtype=torch.bfloat16)
        finite = torch.ones((), dtype=torch.bool, device=dev)
        positions = [self.context] * batch
        tokens = []

        def body(attend):
            x = self.embed[tok]
            cos, sin = self.tables(pos_dev.expand(batch, 1))
            if fused_rotation:
                cos_buf.copy_(cos)
                sin_buf.copy_(sin)
            for lw, d in zip(self.layers, decs):
                h = self.rms(x, lw["n1"])
                if fused_rotation:  # raw projections; the attention call rotates them
                    torch.addmm(lw["b_qkv"], h, lw["w_qkv"].t(), out=qkv_buf)
                else:
                    q, k, v = F.linear(h, lw["w_qkv"], lw["b_qkv"]).split((nh * hd, nkv * hd, nkv * hd), dim=-1)
                    # Q/K rotation + FWHT and the V FWHT in one launch
                    ro.qwen_qk_mrope(q.reshape(batch, nh, 1, hd), k.reshape(batch, nkv, 1, hd), cos, sin,
                                     self.SECTIONS, apply_hadamard=True, value=v.reshape(batch, nkv, 1, hd),
                                     output=(d.query_buffer.view(batch, nh, 1, hd),
                                             d.key_buffer.view(batch, nkv, 1, hd),
                                             d.value_buffer.view(batch, nkv, 1, hd)))
                attend(d)
                x = x + F.linear(d.workspace.output.view(batch, hid), lw["wo"])
                x = self.mlp(x, lw)
            logits.copy_(F.linear(self.rms(x, self.n_final), self.lm_head))
            pos_dev.add_(1)

        def eager_attend(d):
            d.step_in_place(global_token_index=positions, logical_position=positions)

        def graph_attend(d):
            d.executor._launch(d._params, dev)

        def greedy(step):
            tok.copy_(logits.argmax(-1))
            finite.logical_and_(torch.isfinite(logits).all())
            tokens.append(tok.clone())
            if inspect is not None:
                torch.cuda.synchronize()
                inspect(step, decs)

        stream = torch.cuda.current_stream(dev)
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        graph = None
        with torch.no_grad(), _gc_paused():
            torch.cuda.synchronize()
            e[0].record(stream)
            body(eager_attend)  # step 1: every ring is full and flushes inside the batch
            greedy(0)
            e[1].record(stream)
            positions = [p + 1 for p in positions]
            if use_graph:
                for d in decs:  # the step's host bookkeeping; the captured launches advance the device state
                    assert not d._prepare(positions, positions), "no flush may fall inside the captured steps"
                graph = torch.cuda.CUDAGraph()
                side = torch.cuda.Stream(device=dev)
                side.wait_stream(stream)
                with torch.cuda.graph(graph, stream=side):
                    body(graph_attend)
                stream.wait_stream(side)
                torch.cuda.synchronize()
                # the capture recorded the step without running it: replay it as step 2
            e[2].record(stream)
            for i in range(1, steps):
                if use_graph:
                    if i > 1:
                        for d in decs:
                            assert not d._prepare(positions, positions)
                    graph.replay()
                    for d in decs:
                        d._advance()
                else:
                    body(eager_attend)
                greedy(i)
                positions = [p + 1 for p in positions]
            e[3].record(stream)
            torch.cuda.synchronize()
        ms = e[0].elapsed_time(e[1]) + e[2].elapsed_time(e[3])
        del decs, caches, graph
        torch.cuda.empty_cache()
        return ms, torch.stack(tokens), bool(finite.item())


def e2e_decode_bench(dev, *, batch: int, context: int, steps: int, n_layers: int) -> dict:
    """Configuration 4 decode tok/s: the decode runs twice from the same caches, eager launches and
    then one HIP graph per step; the faster is reported (a graph run only if its tokens equal the
    eager run's)."""
    import torch

    model = E2EQwenDecoder(dev, batch=batch, context=context, n_layers=n_layers)
    model.prefill()
    # PyTorch-ROCm's own GEMM selection for the decode shapes (M = batch): TunableOp times the
    # hipBLASLt / rocBLAS candidates once in a short untimed decode, then the choice is frozen so that
    # the eager and graph runs use the same kernels
    tunable = torch.cuda.tunable
    tunable.enable(True)
    tunable.set_filename(os.path.join(tempfile.gettempdir(), "r2o_tunableop_results.csv"))  # not into the repo
    tunable.set_max_tuning_duration(30)
    tunable.tuning_enable(True)
    t_tune = time.perf_counter()
    model.decode(2, False)
    tunable.tuning_enable(False)
    tune_s = time.perf_counter() - t_tune
    _log(f"e2e GEMM tuning (TunableOp) {tune_s:.1f} s")
    eager_ms, eager_tokens, eager_finite = model.decode(steps, False)
    _log(f"e2e eager decode: {eager_ms:.1f} ms for {steps} steps")
    graph_ms, graph_tokens, graph_finite = model.decode(steps, True)
    _log(f"e2e graph decode: {graph_ms:.1f} ms for {steps} steps")
    sep_ms, sep_tokens, _ = model.decode(steps, True, fused_rotation=False)
    _log(f"e2e graph decode with a separate rotation launch: {sep_ms:.1f} ms for {steps} steps")
    match = bool(torch.equal(eager_tokens, graph_tokens))
    use_graph = match and graph_ms < eager_ms
    best_ms = graph_ms if use_graph else eager_ms
    result = {"metric": "e2e decode tok/s", "value": round(batch * steps / (best_ms * 1e-3), 1), "unit": "tok/s",
              "higher_is_better": True, "steps": steps, "ms_per_step": round(best_ms / steps, 3),
              "mode": "hip_graph_per_step" if use_graph else "eager",
              "eager_tok_s": round(batch * steps / (eager_ms * 1e-3), 1),
              "graph_tok_s": round(batch * steps / (graph_ms * 1e-3), 1), "graph_matches_eager": match,
              "rotation": "folded into the attention call (FusedRotary): per layer one QKV GEMM into a static "
                          "buffer, then the partial and combine launches",
              "graph_tok_s_separate_rotation": round(batch * steps / (sep_ms * 1e-3), 1),
              "separate_rotation_tokens_match": bool(torch.equal(sep_tokens, graph_tokens)),
              "logits_finite": eager_finite and graph_finite,
              "dtype": "bf16", "data": "synthetic (random-init weights N(0, 0.02), seeded random token ids)",
              "config": {"workload": "cfg4 qwen25omni7b e2e decode", "layers": n_layers, "batch": batch,
                         "prefill_tokens": context, "decode_steps": steps, "value_tiers": "15/45/40 per 64-token page",
                         "keys": "compact INT4", "hadamard": True},
              "prefill_s": round(model.prefill_s, 1),
              "gemm_selection": f"PyTorch TunableOp over hipBLASLt / rocBLAS, tuned in an untimed 2-step decode "
                                f"({tune_s:.1f} s) and frozen; q/k/v and gate/up weights stacked into one GEMM each",
              "note": "HIP events around the decode steps (first step eager with the flush of every ring; graph "
                      "capture outside the timed span); greedy argmax in eager launches"}
    tunable.enable(False)
    del model
    torch.cuda.empty_cache()
    return result


def time_decode_layers(cfg, dev, *, n_layers: int, steps: int, warmup: int, seed_base: int = 0) -> dict:
    """Build ``n_layers`` distinct layer caches of ``cfg`` (seeds 1000 * layer + request) and time the
    decode-attention layer call rotating over them with HIP events on the launch stream.

    The call is timed as the manager issues it at every decode step (qwen_sspa_attention.py:1794-1826):
    partial + combine with the step's K/V row appended to each Recent-FP ring by the fused append.  Each
    ring then holds min(its tokens, capacity - 1) tokens (host-mode ring lengths, so every call rewrites
    the same slot) and the call attends over those plus the new token: at a full 128-token window the
    same 128 ring tokens as the call without the append, which is timed too.  The partial kernel alone
    is timed by back-to-back partial launches (an event pair around each partial inside the call
    sequence would add ~2 us of its own).  Every timed window follows ~30 ms of its own untimed calls and
    a queued lead of them (``_time_events``) and times exactly ``steps`` calls."""
    import torch

    import r2omni_amd as ro
    from r2omni_amd import _lib
    from r2omni_amd.workloads import algorithmic_bytes, build_request_cache, make_request

    _log(f"building {n_layers} layer caches of {cfg.name} {list(cfg.lengths)} ...")
    layers = []
    for layer in range(n_layers):
        datas = [make_request(cfg, total, seed=seed_base + 1000 * layer + r, device=dev)
                 for r, total in enumerate(cfg.lengths)]
        caches = [build_request_cache(cfg, d) for d in datas]
        q = torch.cat([d.query for d in datas]).contiguous()
        wss = [ro.allocate_splitk_workspace(c, num_query_heads=cfg.hq) for c in caches]
        exs = [ro.prepare_splitk_executor(c, w, output_hadamard=True) for c, w in zip(caches, wss)]
        ex = exs[0] if len(exs) == 1 else ro.stack_homogeneous_splitk_executors(exs)
        del datas
        layers.append((caches, q, ex))
    _log(f"{n_layers} layers ready ({layers[0][2].n_items} work items in layer 0)")
    torch.cuda.synchronize()
    nbytes = algorithmic_bytes(layers[0][0], cfg.hq)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    params = [ex._params(q, ex.workspace.output, None) for _, q, ex in layers]
    refs = [ctypes.byref(p) for p in params]

    # the step's new K/V rows ([B, Hkv, 128], the model dtype) and the ring lengths they are appended at
    b = len(cfg.lengths)
    gen = torch.Generator(device=dev).manual_seed(97)
    row_dtype = layers[0][0][0].recent_fp_pool.fp_k.dtype
    app_k = torch.randn(b, cfg.hkv, 128, generator=gen, device=dev).to(row_dtype)
    app_v = torch.randn(b, cfg.hkv, 128, generator=gen, device=dev).to(row_dtype)
    ring_n = [min(int(c.recent_fp_pool.active_length), c.recent_fp_pool.capacity - 1) for c in layers[0][0]]
    nbytes_app = nbytes + sum(cfg.hkv * 512 * (n + 1 - int(c.recent_fp_pool.active_length)) + cfg.hkv * 512
                              for n, c in zip(ring_n, layers[0][0]))
    params_app = []
    for caches, q, ex in layers:
        p = _lib.DecodeParams.from_buffer_copy(ex._params(q, ex.workspace.output, None))
        p.do_append, p.append_k, p.append_v = 1, app_k.data_ptr(), app_v.data_ptr()
        for r, c in enumerate(caches):
            p.recent_len[r] = ring_n[r]
            p.append_global[r] = p.append_logical[r] = int(c.compact_key.active_length if c.compact_key is not None
                                                           else c.bf16_key.active_length) + ring_n[r]
        params_app.append(p)
    refs_app = [ctypes.byref(p) for p in params_app]
    n_rot = len(layers)
    f_call, f_partial = lib.r2o_decode, lib.r2o_decode_partial

    def call(i):  # the manager's call (r2o_decode: partial + combine) with the fused append
        f_call(refs_app[i % n_rot], sp)

    def call_no_append(i):
        f_call(refs[i % n_rot], sp)

    def partial_only(i):
        f_partial(refs[i % n_rot], sp)

    # the drop-in: SplitKExecutor.__call__ with the append (checks, arguments, the two launches); the
    # host ring lengths are set back before each call, since a stacked executor advances them
    k4, v4 = app_k[:, :, None], app_v[:, :, None]
    gpos = [int(params_app[0].append_global[r]) for r in range(b)]
    ring_full = [[int(c.recent_fp_pool.active_length) for c in caches] for caches, _, _ in layers]
    for caches, _, ex in layers:
        for r, c in enumerate(caches):
            c.recent_fp_pool.active_length = ring_n[r]

    def drop_in(i):
        _, q, ex = layers[i % n_rot]
        if ex.batched_recent_lengths is not None:
            ex.batched_recent_lengths[:] = ring_n
        ex(q, append=(k4, v4, gpos, gpos))

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    ms_step = _time_events(call, steps, stream)
    ms_no_append = _time_events(call_no_append, steps, stream)
    ms_partial = _time_events(partial_only, steps, stream)
    ms_drop_in = _time_events(drop_in, steps, stream)
    for (caches, _, _), lengths in zip(layers, ring_full):
        for c, n in zip(caches, lengths):
            c.recent_fp_pool.active_length = n

    # the same calls replayed from one HIP graph holding a layer call per rotated cache: no host
    # launch cost, so on small caches this is the GPU's own time per call
    from r2omni_amd.batch import _capture_launches

    side = torch.cuda.Stream(device=dev)

    def rotation():
        cs = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for r in refs_app:
            f_call(r, cs)

    graph = _capture_launches(dev, side, rotation)
    for _ in range(20):
        graph.replay()
    replays = max(1, -(-steps // n_rot))
    ms_graph = _time_events(lambda i: graph.replay(), replays, stream, lead=2) / n_rot
    del graph
    return {"layers": layers, "bytes": nbytes_app, "bytes_no_append": nbytes, "ms_step": ms_step,
            "ms_no_append": ms_no_append, "ms_partial": ms_partial, "ms_drop_in": ms_drop_in, "ms_graph": ms_graph,
            "graph_calls": replays * n_rot, "n_items": layers[0][2].n_items, "ring_tokens": ring_n}


def rotation_bench(cfg, dev, *, n_layers: int, steps: int) -> dict:
    """The decode step's attention with the Q/K mRoPE + FWHT and the V FWHT folded into the split-K call
    (``FusedRotary``: two launches) against the same call on rows rotated by a separate ``qwen_qk_mrope``
    launch (three launches, as the reference's layer: qwen_sspa_attention.py:1239-1247, 230-235), both
    with the fused append, rotating ``n_layers`` layer caches; and the partial kernel alone with and
    without the folded rotation.  Every window as ``_time_events``."""
    import torch

    import r2omni_amd as ro
    from r2omni_amd import _lib
    from r2omni_amd.workloads import build_request_cache, make_request

    b = len(cfg.lengths)
    layers = []
    for layer in range(n_layers):
        datas = [make_request(cfg, total, seed=1000 * layer + r, device=dev) for r, total in enumerate(cfg.lengths)]
        caches = [build_request_cache(cfg, d) for d in datas]
        exs = [ro.prepare_splitk_executor(c, ro.allocate_splitk_workspace(c, num_query_heads=cfg.hq),
                                          output_hadamard=True) for c in caches]
        layers.append((caches, exs[0] if b == 1 else ro.stack_homogeneous_splitk_executors(exs)))
        del datas
    torch.cuda.synchronize()
    gen = torch.Generator(device=dev).manual_seed(98)
    row_dtype = layers[0][0][0].recent_fp_pool.fp_k.dtype
    # the step's raw projections, views of one fused QKV row per request, and its mRoPE tables
    qkv = torch.randn(b, (cfg.hq + 2 * cfg.hkv) * 128, generator=gen, device=dev).to(row_dtype)
    q = qkv[:, : cfg.hq * 128].view(b, cfg.hq, 128)
    k = qkv[:, cfg.hq * 128 : (cfg.hq + cfg.hkv) * 128].view(b, cfg.hkv, 128)
    v = qkv[:, (cfg.hq + cfg.hkv) * 128 :].view(b, cfg.hkv, 128)
    ang = torch.rand(3, b, 1, 64, generator=gen, device=dev) * 6.0
    ang = torch.cat([ang, ang], dim=-1)
    cos, sin = ang.cos().to(row_dtype), ang.sin().to(row_dtype)
    sections = (16, 24, 24)
    rot = ro.FusedRotary(cos, sin, sections, True, True)
    qr, kr, vr = (torch.empty(t.shape, device=dev, dtype=row_dtype) for t in (q, k, v))  # the separate launch's rows
    ring_n = [min(int(c.recent_fp_pool.active_length), c.recent_fp_pool.capacity - 1) for c in layers[0][0]]

    def with_append(p, caches, kk, vv):
        p.do_append, p.append_k, p.append_v = 1, kk.data_ptr(), vv.data_ptr()
        p.append_batch_stride = 0 if kk.is_contiguous() else int(kk.stride(0))
        for r, c in enumerate(caches):
            p.recent_len[r] = ring_n[r]
            p.append_global[r] = p.append_logical[r] = int(c.compact_key.active_length if c.compact_key is not None
                                                           else c.bf16_key.active_length) + ring_n[r]
        return p

    fused = [with_append(ex._params(q, ex.workspace.output, None, rotary=rot), caches, k, v) for caches, ex in layers]
    plain = [with_append(ex._params(qr, ex.workspace.output, None), caches, kr, vr) for caches, ex in layers]
    part_f = [ex._params(q, ex.workspace.output, None, rotary=rot) for _, ex in layers]
    part_p = [ex._params(qr, ex.workspace.output, None) for _, ex in layers]
    refs = {name: [ctypes.byref(p) for p in ps] for name, ps in
            (("fused", fused), ("plain", plain), ("part_f", part_f), ("part_p", part_p))}
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    n = len(layers)
    q4, k4, v4 = q[:, :, None], k[:, :, None], v[:, :, None]
    out4 = (qr[:, :, None], kr[:, :, None], vr[:, :, None])

    def separate(i):  # the rotation launch, then the call on its rows
        ro.qwen_qk_mrope(q4, k4, cos, sin, sections, apply_hadamard=True, value=v4, output=out4)
        lib.r2o_decode(refs["plain"][i % n], sp)

    res = {
        "call_fused_us": _time_events(lambda i: lib.r2o_decode(refs["fused"][i % n], sp), steps, stream) * 1e3,
        "call_separate_rotation_us": _time_events(separate, steps, stream) * 1e3,
        "call_on_rotated_rows_us": _time_events(lambda i: lib.r2o_decode(refs["plain"][i % n], sp), steps, stream) * 1e3,
        "partial_fused_us": _time_events(lambda i: lib.r2o_decode_partial(refs["part_f"][i % n], sp), steps, stream) * 1e3,
        "partial_us": _time_events(lambda i: lib.r2o_decode_partial(refs["part_p"][i % n], sp), steps, stream) * 1e3,
    }
    return {"metric": "decode-step attention with the rotation folded in vs a separate rotation launch",
            "config": {"workload": cfg.name, "lengths": list(cfg.lengths), "layers": n_layers,
                       "mrope_sections": list(sections), "hadamard": True, "tables": str(row_dtype)},
            **{kk: round(vv, 3) for kk, vv in res.items()}, "steps": steps,
            "note": "call = r2o_decode (partial + combine with the fused append); separate = qwen_qk_mrope "
                    "(Q/K mRoPE + FWHT and the V FWHT in one launch) then the call on its rows"}


def timeline_bench(cfg, dev, *, n_layers: int, warmup: int, trials: int = 3) -> dict:
    """Phase breakdown of the layer call from the measurement build (libr2o_timeline.so, the decode
    library compiled with -DR2O_TIMELINE: every wave keeps real-time counter stamps in registers and
    stores them at its end).  After the warm-up, ``trials`` times: 200 back-to-back layer calls, then
    the stamps of the last call are read.  Times in microseconds; each entry lists the 0/10/50/90/100th
    percentiles over work items (partial kernel) or blocks (combine), median over the trials."""
    import numpy as np
    import torch

    from r2omni_amd import _lib

    lib = _lib.load()
    if not hasattr(lib, "r2o_timeline_read"):
        raise RuntimeError(f"{_lib.LIB_PATH} has no phase stamps: run bench.py --timeline (it loads libr2o_timeline.so)")
    lib.r2o_timeline_read.restype = ctypes.c_int
    lib.r2o_timeline_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]
    r = time_decode_layers(cfg, dev, n_layers=n_layers, steps=200, warmup=warmup)
    layers = r["layers"]
    n = layers[(200 - 1) % len(layers)][2].n_items  # the stamps read are the last call's, on this layer
    if n > 4096:
        raise RuntimeError("the stamp arrays hold 4096 work items")
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    params = [ex._params(q, ex.workspace.output, None) for _, q, ex in layers]
    n_comb = len(cfg.lengths) * cfg.hq  # combine blocks: one per (request, query head) without an append
    pct = (0, 10, 50, 90, 100)

    def q(v):
        v = np.asarray(v, dtype=np.float64)
        v = v[np.isfinite(v)]
        return [round(float(x), 2) for x in np.percentile(v, pct)] if v.size else None

    runs = []
    for _ in range(trials):
        with _gc_paused():
            for i in range(200):
                pp = ctypes.byref(params[i % len(params)])
                lib.r2o_decode_partial(pp, sp)
                lib.r2o_decode_combine(pp, sp)
        torch.cuda.synchronize()
        a = np.zeros(4096 * 4 * 12, dtype=np.uint64)
        c = np.zeros(4096 * 8 * 12, dtype=np.uint64)
        _lib.check(lib.r2o_timeline_read(0, a.ctypes.data, a.nbytes), "r2o_timeline_read")
        _lib.check(lib.r2o_timeline_read(1, c.ctypes.data, c.nbytes), "r2o_timeline_read")
        a = a.reshape(4096, 4, 12)[:n].astype(np.int64)
        c = c.reshape(4096, 8, 12)[:n_comb].astype(np.int64)
        t0 = a[:, :, 0].min()
        kind = a[:, 0, 8] >> 32
        tiles = a[:, 0, 8] & 0xFFFFFFFF

        def at(x, j):  # stamp j in us from the first entry; NaN where a wave took no such step
            return np.where(x[..., j] > 0, (x[..., j] - t0) / 100.0, np.nan)

        seg = kind != 3
        loop_end = np.nanmax(at(a, 5), 1)
        block_end = at(a[:, 0], 6)
        last = float(np.nanmax(block_end))
        res = {
            "work_item_arrival": q(at(a[:, 0], 1)),
            "first_dma_after_item": q(np.nanmin(at(a[seg], 2), 1) - at(a[seg, 0], 1)),
            "first_tile_after_dma": q(np.nanmin(at(a[seg], 3), 1) - np.nanmin(at(a[seg], 2), 1)),
            "first_tile": q(np.nanmin(at(a[seg], 3), 1)),
            "wave_loop_end_spread": q(np.nanmax(at(a, 5), 1) - np.nanmin(at(a, 5), 1)),
            "epilogue": q(block_end - loop_end),
            "block_end": q(block_end),
            "xcc_blocks": np.bincount(a[:, 0, 7] & 0xF, minlength=8).tolist(),
        }
        for k, name in ((0, "bf16_v"), (1, "int4_v"), (2, "int2_v"), (3, "recent")):
            m = kind == k
            if not m.any():
                continue
            d = {"items": int(m.sum()), "block_end": q(block_end[m])}
            if k != 3:
                per_wave = np.ceil(tiles[m] / 4.0)
                d["us_per_tile"] = q((np.nanmax(at(a[m], 4), 1) - np.nanmin(at(a[m], 3), 1)) / np.maximum(per_wave - 1, 1))
            res[f"kind_{name}"] = d
        res["combine"] = {
            "blocks": n_comb,
            "start_after_partial_end": q(np.nanmin(at(c, 0), 1) - last),
            "arguments": q(np.nanmax(at(c, 1) - at(c, 0), 1)),
            "first_partials": q(np.nanmax(at(c, 2) - at(c, 1), 1)),
            "merge": q(np.nanmax(at(c, 3) - at(c, 2), 1)),
            "tail": q(at(c[:, 0], 4) - np.nanmax(at(c, 3), 1)),
            "end_after_partial_end": q(at(c[:, 0], 4) - last),
        }
        res["partial_last_block_end"] = round(last, 2)
        runs.append(res)

    def med(objs):
        if isinstance(objs[0], dict):
            return {k: med([o[k] for o in objs]) for k in objs[0]}
        if isinstance(objs[0], list):
            if any(o is None for o in objs):
                return None
            return [round(float(np.median([o[i] for o in objs])), 2) for i in range(len(objs[0]))]
        return objs[len(objs) // 2]

    return {"metric": "layer-call phase timeline (us; 0/10/50/90/100th percentiles, median of trials)",
            "config": cfg.name, "work_items": n, "us_call": round(r["ms_step"] * 1e3, 3),
            "us_partial": round(r["ms_partial"] * 1e3, 3), "trials": trials, "timeline": med(runs),
            "note": "measurement build (-DR2O_TIMELINE): the product kernels with real-time stamps kept in registers"}


def context_sweep(cfg, dev, *, factors, n_layers: int, steps: int, warmup: int) -> dict:
    """The layer call of ``cfg`` at context lengths scaled by ``factors`` (the recent window kept at
    128, the history rounded to whole pages), and a least-squares fit time = fixed + bytes / rate of
    the whole call and of the partial kernel: the fixed part is the per-launch cost (start-up, tail,
    combine), the rate the sustained streaming rate of the steady state."""
    import numpy as np
    import torch

    points = []
    for f in factors:
        lengths = tuple(int(round((t - cfg.recent) * f / cfg.page)) * cfg.page + cfg.recent for t in cfg.lengths)
        c = dataclasses.replace(cfg, lengths=lengths)
        r = time_decode_layers(c, dev, n_layers=n_layers, steps=steps, warmup=warmup)
        points.append({"factor": f, "context_lengths": list(lengths), "bytes": r["bytes_no_append"],
                       "work_items": r["n_items"], "us_call": round(r["ms_no_append"] * 1e3, 3),
                       "us_call_with_append": round(r["ms_step"] * 1e3, 3),
                       "us_partial": round(r["ms_partial"] * 1e3, 3),
                       "call_GBs": round(r["bytes_no_append"] / (r["ms_no_append"] * 1e-3) / 1e9, 1),
                       "partial_GBs": round(r["bytes_no_append"] / (r["ms_partial"] * 1e-3) / 1e9, 1)})
        _log(f"sweep x{f}: {points[-1]}")
        del r
        torch.cuda.empty_cache()
    b = np.array([p["bytes"] for p in points], dtype=np.float64)
    fits = {}
    for key in ("us_call", "us_partial"):
        t = np.array([p[key] for p in points], dtype=np.float64)
        slope, fixed = np.polyfit(b, t, 1)
        fits[key.replace("us_", "")] = {"fixed_us": round(float(fixed), 3),
                                        "rate_GBs": round(float(1e-3 / slope), 1),
                                        "rate_pct_of_peak": round(float(1e-3 / slope) / HBM_PEAK_GBS * 100, 1)}
    return {"metric": "decode-attention layer call vs context (fit: time = fixed + bytes / rate)",
            "config": f"{cfg.name} geometry, history x {list(factors)}", "points": points, "fit": fits}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed calls before the timed ones (default 2000, ~50 ms on cfg2: the GPU clocks take "
                         "~20 ms of load to come up after the idle cache build)")
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--variant", choices=("int4k", "int2k", "bf16k", "matched"), default="int4k",
                    help="K format of the layer caches: compact INT4-K (default), compact INT2-K, "
                         "v_fourq_k_bf16 or matched-FP")
    ap.add_argument("--gen-values", choices=("int2", "int4"), default="int2",
                    help="generated_value_precision of the layer caches: flushed values INT2 (released, default) "
                         "or INT4 (the INT4 pool's values in a compact arena with append room)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="leave configuration 4 (decode tok/s) out of the line")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (HBM counter calibration)")
    ap.add_argument("--prefill", action="store_true",
                    help="only time the prefill-side cache build (quantise + pack on the GPU) of the longest "
                         "request of --config and print one JSON line")
    ap.add_argument("--decode-steps", type=int, default=0, metavar="N",
                    help="only time N decode steps of --layers BatchedDecoder layers of --config (eager launches "
                         "and one HIP graph per step, flushes inside the batch) and print one JSON line")
    ap.add_argument("--flush", action="store_true",
                    help="only time the flush of a full Recent-FP ring (128 tokens quantised and packed, ring "
                         "shifted) on the longest request of --config and print one JSON line")
    ap.add_argument("--sweep", type=str, default="", metavar="F1,F2,...",
                    help="only time the layer call of --config with its history scaled by each factor and print "
                         "the points and the fit time = fixed + bytes / rate as one JSON line")
    ap.add_argument("--e2e", action="store_true",
                    help="only run configuration 4: prefill and greedy decode of a random-init Qwen2.5-Omni-7B "
                         "language model on this path, and print one JSON line (decode tok/s)")
    ap.add_argument("--e2e-batch", type=int, default=8)
    ap.add_argument("--e2e-context", type=int, default=32768)
    ap.add_argument("--e2e-steps", type=int, default=128)
    ap.add_argument("--e2e-layers", type=int, default=28)
    ap.add_argument("--fused-rotation", action="store_true",
                    help="only time the layer call of --config with the decode step's rotation folded in "
                         "(FusedRotary) against a separate rotation launch before the call, and print one "
                         "JSON line")
    ap.add_argument("--timeline", action="store_true",
                    help="only print the phase breakdown of the layer call of --config (work-item start-up, "
                         "first tile, per-kind tile times, epilogue, combine phases) from libr2o_timeline.so, "
                         "the decode library built with per-wave real-time stamps")
    ap.add_argument("--summarize-pmc", metavar="DIR",
                    help="only print the mean per-dispatch value of every counter in a rocprofv3 --pmc CSV "
                         "output directory, per decode kernel (and the calibration copy kernel)")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="only print the decode kernels' average durations in a rocprofv3 --kernel-trace CSV "
                         "output directory: partials inside layer calls and partial-only launches apart")
    args = ap.parse_args()
    if args.summarize_trace:
        print(json.dumps(summarize_trace(args.summarize_trace)))
        return 0
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(args.summarize_pmc)))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (the decode path "
                                   "shards by (request, kv head) or token range across GPUs by design, "
                                   "but no multi-GPU run is implemented)"}))
        return 2

    if args.timeline:  # before the package is imported: it binds the library named here
        os.environ["R2O_SSPA_LIB"] = os.path.join(ROOT, "r2-omni_amd", "r2omni_amd", "libr2o_timeline.so")

    import torch

    from r2omni_amd.workloads import CONFIGS

    dev = torch.device("cuda:0")
    e2e_kw = dict(batch=args.e2e_batch, context=args.e2e_context, steps=args.e2e_steps, n_layers=args.e2e_layers)
    if args.e2e:
        print(json.dumps(e2e_decode_bench(dev, **e2e_kw)), flush=True)
        return 0
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4}))
        return 0
    cfg = CONFIGS[args.config]
    if args.variant != "int4k":
        cfg = dataclasses.replace(cfg, variant=args.variant)
    if args.gen_values != "int2":
        cfg = dataclasses.replace(cfg, gen_values=args.gen_values)
    if args.prefill:
        print(json.dumps(prefill_bench(cfg, args.config, dev)), flush=True)
        return 0
    if args.flush:
        print(json.dumps(flush_bench(cfg, args.config, dev)), flush=True)
        return 0
    if args.decode_steps:
        print(json.dumps(decode_steps_bench(cfg, args.config, dev, args.decode_steps, args.layers)), flush=True)
        return 0
    if args.timeline:
        print(json.dumps(timeline_bench(cfg, dev, n_layers=args.layers, warmup=args.warmup)), flush=True)
        return 0
    if args.fused_rotation:
        print(json.dumps(rotation_bench(cfg, dev, n_layers=args.layers, steps=args.steps)), flush=True)
        return 0
    if args.sweep:
        factors = [float(f) for f in args.sweep.split(",")]
        print(json.dumps(context_sweep(cfg, dev, factors=factors, n_layers=args.layers, steps=args.steps,
                                       warmup=args.warmup)), flush=True)
        return 0
    _log("timing ...")
    t0 = time.perf_counter()
    r = time_decode_layers(cfg, dev, n_layers=args.layers, steps=args.steps, warmup=args.warmup)
    wall = time.perf_counter() - t0
    nbytes, ms_step, ms_partial, ms_drop_in = r["bytes"], r["ms_step"], r["ms_partial"], r["ms_drop_in"]
    nbytes_na, ms_na, ms_graph = r["bytes_no_append"], r["ms_no_append"], r["ms_graph"]
    ring_tokens, graph_calls = r["ring_tokens"], r["graph_calls"]
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    part_gbs = nbytes_na / (ms_partial * 1e-3) / 1e9
    _log(f"call {ms_step * 1e3:.2f} us ({gbs:.0f} GB/s), without append {ms_na * 1e3:.2f} us, partial "
         f"{ms_partial * 1e3:.2f} us ({part_gbs:.0f} GB/s), wall {wall:.2f} s")
    cpu = None
    if not args.no_cpu_baseline:
        _log("cpu baseline ...")
        caches0, q0, _ = r["layers"][0]
        cpu = cpu_baseline(caches0, [q0[i : i + 1] for i in range(len(cfg.lengths))], cfg.hq)
    del r
    torch.cuda.empty_cache()
    _log("copy and read bandwidth ...")
    copy = copy_bandwidth(dev)
    copy["partial_kernel_pct_of_copy"] = round(100 * part_gbs / copy["GBs"], 1)
    read = read_bandwidth(dev)
    read["partial_kernel_pct_of_read"] = round(100 * part_gbs / read["GBs"], 1)
    _log("dma floor at the call's bytes ...")
    floor = dma_floor(dev, nbytes_na)
    floor["partial_kernel_pct_of_floor"] = round(100 * floor["us"] / (ms_partial * 1e3), 1)
    e2e = None
    if not args.no_e2e:
        _log("e2e (configuration 4) ...")
        e2e = e2e_decode_bench(dev, **e2e_kw)
    traffic, traffic_src = traffic_from_profile() if args.config == 2 and args.variant == "int4k" \
        and args.gen_values == "int2" else (None, None)
    line = {
        "metric": "packed-KV decode attn: HBM GB/s (% peak), us/layer @32k ctx; decode tok/s",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "us_per_layer_call": round(ms_step * 1e3, 3),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-k/bf16|int4|int2-v, f16/bf16 mfma, f32 accumulate",
        "data": "synthetic (seeded N(0,1) bf16, 4 key outlier channels x8, seeded per-page V tiers)",
        "config": {"workload": f"cfg{args.config} {cfg.name}" + ("" if args.variant == "int4k" else f" {args.variant}")
                               + ("" if args.gen_values == "int2" else " int4-generated"),
                   "k_format": args.variant, "gen_values": args.gen_values, "hq": cfg.hq, "hkv": cfg.hkv,
                   "context_lengths": list(cfg.lengths), "v_tiers_bf16_int4_int2": list(cfg.tier_probs),
                   "recent_window": cfg.recent, "k_superblock": cfg.superblock, "int2_group": cfg.group,
                   "rotated_layer_caches": args.layers, "algorithmic_bytes_per_call": nbytes, "output_hadamard": True,
                   "fused_append": True, "ring_tokens_before_append": ring_tokens},
        "roofline": {"bound": "hbm", "achieved": round(part_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(part_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "decode_partial_kernel", "avg_us": round(ms_partial * 1e3, 3),
                     "algorithmic_bytes": nbytes_na,
                     "avg_us_source": "HIP events over back-to-back partial launches on the launch stream "
                                      "(after 30 ms of the same launches untimed and a queued lead of them)"},
        "call_without_append": {"us": round(ms_na * 1e3, 3), "GBs": round(nbytes_na / (ms_na * 1e-3) / 1e9, 1),
                                "bytes": nbytes_na,
                                "method": "the same rotated layer calls without the fused append, HIP events"},
        "graph_call": {"us": round(ms_graph * 1e3, 3), "GBs": round(nbytes / (ms_graph * 1e-3) / 1e9, 1),
                       "calls": graph_calls,
                       "method": "the same layer calls (fused append) replayed from one HIP graph per rotation of "
                                 "the layer caches (no host launch cost), HIP events over the replays"},
        "drop_in_call": {"us": round(ms_drop_in * 1e3, 3), "GBs": round(nbytes / (ms_drop_in * 1e-3) / 1e9, 1),
                         "method": "the same layer calls through SplitKExecutor.__call__(query, append=...) (the "
                                   "Python drop-in the manager calls: checks, launch arguments, the two launches), "
                                   "HIP events"},
        "cpu_baseline": cpu,
        "hbm_copy": copy,
        "hbm_read": read,
        "dma_floor": floor,
        "e2e": e2e,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
