"""CPU checks of the C-ABI library: it loads and exports every symbol include/r2o_sspa.h declares."""
import ctypes
import os
import re
import subprocess

import pytest

from r2omni_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "r2o_sspa.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(r2o_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert sorted(_lib.EXPORTED) == _declared()


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built: run `python -m r2omni_amd.build` in r2-omni_amd/")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    for name in _declared():
        assert re.search(rf"\bT {name}\b", out), name


def _c_layout(struct: str, fields, tmp_path):
    """offsetof() of each field and sizeof() of an include/r2o_sspa.h struct, from the host C compiler."""
    src = tmp_path / "probe.c"
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "r2o_sspa.h"', "int main(void) {"]
    for f in fields:
        lines.append(f'  printf("%zu\\n", offsetof({struct}, {f}));')
    lines += [f'  printf("%zu\\n", sizeof({struct}));', "  return 0;", "}"]
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    return vals[:-1], vals[-1]


def test_params_struct_layout_matches_header(tmp_path):
    p = _lib.DecodeParams
    names = [f[0] for f in p._fields_]
    offsets, size = _c_layout("r2o_decode_params", names, tmp_path)
    assert [getattr(p, n).offset for n in names] == offsets
    assert ctypes.sizeof(p) == size


def test_planner_struct_layouts_match_header(tmp_path):
    for struct, cls in (("r2o_plan_run", _lib.PlanRun), ("r2o_plan_config", _lib.PlanConfig)):
        names = [f[0] for f in cls._fields_]
        offsets, size = _c_layout(struct, names, tmp_path)
        assert [getattr(cls, n).offset for n in names] == offsets, struct
        assert ctypes.sizeof(cls) == size, struct


def test_descriptor_word_layouts_match_header(tmp_path):
    # the request descriptor and work item are rows of int64 words written by the host planner
    for struct, fields in (("r2o_request_desc", _lib.REQUEST_FIELDS), ("r2o_work_item", _lib.ITEM_FIELDS)):
        offsets, size = _c_layout(struct, fields, tmp_path)
        assert offsets == [8 * i for i in range(len(fields))] and size == 8 * len(fields), struct


def test_host_side_validation_rejects_bad_arguments_without_a_gpu():
    lib = _lib.load()
    # superblock 48 is rejected before any launch
    rc = lib.r2o_pack_int4_k(None, 0, 2, 10, None, 10, 0, 0, None, None, None, None, 128, 3, 48, None)
    assert rc == 1
    rc = lib.r2o_pack_int2_v(None, 0, 2, 10, None, 10, 0, 48, None, None, None, 128, None)
    assert rc == 1
    params = _lib.DecodeParams()
    assert lib.r2o_decode_partial(ctypes.byref(params), None) == 1
    # a workspace with fewer partial-state slots than work items is refused before any launch (the
    # pointers are never dereferenced on the host, so placeholders do)
    params = _lib.DecodeParams(reqs=0x1000, items=0x2000, group_begin=0x3000, n_items=40, partial_max=0x4000,
                               partial_sum=0x5000, partial_out=0x6000, query=0x7000, out=0x8000, batch=1, hq=28,
                               hkv=4, superblock=32, int2_group=32, page_size=64, k_format=_lib.K_INT4,
                               partial_capacity=39)
    assert lib.r2o_decode_partial(ctypes.byref(params), None) == 1
    assert lib.r2o_decode_combine(ctypes.byref(params), None) == 1
    assert lib.r2o_decode(ctypes.byref(params), None) == 1
    params.partial_capacity = 0
    assert lib.r2o_decode_partial(ctypes.byref(params), None) == 1


def test_folded_rotation_and_row_strides_are_checked_without_a_gpu():
    """The rotation fields and the strided query / appended rows are refused before any launch when the
    kernels could not honour them (placeholder pointers: nothing is dereferenced on the host)."""
    lib = _lib.load()

    def params(**kw):
        p = _lib.DecodeParams(reqs=0x1000, items=0x2000, group_begin=0x3000, n_items=40, partial_max=0x4000,
                              partial_sum=0x5000, partial_out=0x6000, query=0x7000, out=0x8000, batch=2, hq=28,
                              hkv=4, superblock=32, int2_group=32, page_size=64, k_format=_lib.K_INT4,
                              partial_capacity=40, append_k=0x9000, append_v=0xA000, do_append=1,
                              rope_mode=1, rope_cos=0xB000, rope_sin=0xC000, rope_section0=16, rope_section1=24,
                              rotated_k=0xD000, rotated_v=0xE000,
                              rope_cos_strides=(ctypes.c_int64 * 4)(256, 128, 128, 1),
                              rope_sin_strides=(ctypes.c_int64 * 4)(256, 128, 128, 1))
        for k, v in kw.items():
            setattr(p, k, v)
        return p

    bad = {
        "unknown rotation": dict(rope_mode=2),
        "no cos table": dict(rope_cos=None),
        "table dtype": dict(rope_table_dtype=3),
        "sections past 64": dict(rope_section0=40, rope_section1=30),
        "query and row dtypes differ": dict(q_dtype=0, row_dtype=1),
        "no rotated-row output": dict(rotated_k=None),
        "misaligned rotated rows": dict(rotated_v=0xE008),
        "query stride not whole pieces": dict(query_batch_stride=28 * 128 + 4),
        "query stride below a request": dict(query_batch_stride=128),
        "append stride below a request": dict(append_batch_stride=256),
        "misaligned query": dict(query=0x7008),
        "negative table stride": dict(rope_sin_strides=(ctypes.c_int64 * 4)(-256, 128, 128, 1)),
        "table past 2 GiB": dict(rope_cos_strides=(ctypes.c_int64 * 4)(1 << 30, 128, 128, 1)),
        "table channels not unit-strided": dict(rope_cos_strides=(ctypes.c_int64 * 4)(512, 256, 128, 2)),
        "table rows off 16 bytes": dict(rope_sin_strides=(ctypes.c_int64 * 4)(256, 132, 128, 1)),
        "misaligned table": dict(rope_cos=0xB008),
        "Qwen3 rotation without norm weights": dict(rope_mode=2, rope_section0=64, rope_section1=0),
        "Qwen3 rotation with misaligned weights": dict(rope_mode=2, rope_section0=64, rope_section1=0,
                                                       q_norm_weight=0xF008, k_norm_weight=0xF100),
        "Qwen3 rotation with a negative epsilon": dict(rope_mode=2, rope_section0=64, rope_section1=0,
                                                       q_norm_weight=0xF000, k_norm_weight=0xF100, norm_eps=-1.0),
        "Qwen3 rotation with mRoPE sections": dict(rope_mode=2, q_norm_weight=0xF000, k_norm_weight=0xF100),
        "Qwen3 rotation with fp32 tables": dict(rope_mode=2, rope_section0=64, rope_section1=0, rope_table_dtype=2,
                                                q_norm_weight=0xF000, k_norm_weight=0xF100),
        "strided query without the rotation": dict(rope_mode=0, query_batch_stride=36 * 128),
        "strided append rows without the rotation": dict(rope_mode=0, append_batch_stride=36 * 128),
    }
    for what, kw in bad.items():
        p = params(**kw)
        for fn in (lib.r2o_decode_partial, lib.r2o_decode_combine, lib.r2o_decode):
            assert fn(ctypes.byref(p), None) == 1, what
    assert lib.r2o_build_target() == b"gfx950"
    # the planner refuses runs whose groups do not match the group count, without a GPU
    run = _lib.PlanRun(0, 0, _lib.KIND_RECENT, 0, 4, 0, 128, 0)
    cfg = _lib.PlanConfig(num_cus=8, blocks_per_cu=2, tiles_per_item=8, waves_per_item=4, min_tiles_per_item=4,
                          late_share=1.0)
    n = ctypes.c_int64(0)
    items = (ctypes.c_int64 * (16 * 16))()
    begins = (ctypes.c_int32 * 4)()
    assert lib.r2o_plan_work_items(ctypes.byref(run), 1, ctypes.byref(cfg), None, 1, 0, 32, items, 16, begins, 3,
                                   ctypes.byref(n)) == 1
    assert lib.r2o_plan_work_items(ctypes.byref(run), 1, ctypes.byref(cfg), None, 1, 0, 32, items, 16, begins, 1,
                                   ctypes.byref(n)) == 0 and n.value >= 1


def test_stream_lookup_refuses_a_cpu_device():
    """Launches take their stream from the tensor's device; a CPU tensor is refused before any
    launch instead of being handed to a kernel."""
    import torch

    with pytest.raises(RuntimeError, match="GPU tensor"):
        _lib.stream_of(torch.device("cpu"))


def test_bench_read_probe_library_rejects_bad_arguments_without_a_gpu():
    """bench.py's streaming-read probe library checks its arguments on the host before any launch."""
    from r2omni_amd.build import BENCH_LIB_PATH

    lib = ctypes.CDLL(BENCH_LIB_PATH)
    fn = lib.r2o_bench_stream_read
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    assert fn(None, 1024, 64, 8, 1, None) == 1          # no source
    assert fn(4096, 1000, 64, 8, 1, None) == 1          # not a multiple of 16 bytes
    assert fn(4096 + 8, 1024, 64, 8, 1, None) == 1      # source not 16-byte aligned
    assert fn(4096, 1024, 64, 0, 1, None) == 1          # no workgroups


def test_bench_dma_read_probe_rejects_bad_arguments_without_a_gpu():
    """bench.py's DMA read-floor probe checks its arguments on the host before any launch."""
    from r2omni_amd.build import BENCH_LIB_PATH

    lib = ctypes.CDLL(BENCH_LIB_PATH)
    fn = lib.r2o_bench_dma_read
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    assert fn(None, 8192, 64, 8, 4, None) == 1          # no source
    assert fn(4096 + 8, 8192, 64, 8, 4, None) == 1      # source not 16-byte aligned
    assert fn(4096, 8192, 64, 0, 4, None) == 1          # no workgroups
    assert fn(4096, 8192, 64, 8, 2, None) == 1          # tile size other than 4 or 8 KiB
    assert fn(4096, 2048, 64, 8, 4, None) == 1          # less than one tile
    assert fn(4096, 8192, None, 8, 4, None) == 1        # no sink


def test_phase_stamps_live_only_in_the_measurement_library():
    """libr2o_timeline.so (bench.py --timeline) is the decode library with -DR2O_TIMELINE: it exports the
    stamp reader and every product symbol; the product library has no stamp code at all."""
    from r2omni_amd.build import TIMELINE_LIB_PATH

    def defined(path):
        return subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True).stdout

    product, timeline = defined(_lib.LIB_PATH), defined(TIMELINE_LIB_PATH)
    assert "r2o_timeline_read" not in product
    assert re.search(r"\bT r2o_timeline_read\b", timeline)
    for name in _declared():
        assert re.search(rf"\bT {name}\b", timeline), name


def test_built_kernels_keep_their_state_in_registers_and_lds():
    """The build records the compiler's resource figures of every kernel beside its object and fails
    on scratch use; here every decode partial instance (3 key formats x 2 row dtypes x no rotation, the
    folded mRoPE or the folded Qwen3 norm+RoPE) and the combine are listed, with no scratch, no spills
    and two workgroups per CU."""
    from r2omni_amd.build import ROOT_DIR

    path = os.path.join(ROOT_DIR, "_build", "r2o_decode.resources.txt")
    if not os.path.exists(path):
        pytest.fail(f"{path} not written: run `python -m r2omni_amd.build` in r2-omni_amd/")
    rows = [ln.split(" ", 1) for ln in open(path).read().splitlines()[1:]]
    table = {name: [int(x) for x in vals.split(" | ")] for name, vals in rows}
    partial = [n for n in table if "decode_partial_kernel" in n]
    assert len(partial) == 18 and any("decode_combine_kernel" in n for n in table)
    for name, (vgpr, agpr, sgpr, scratch, vspill, sspill, occupancy, lds) in table.items():
        assert scratch == 0 and vspill == 0 and sspill == 0, name
        if name in partial:
            assert vgpr + agpr <= 256 and occupancy >= 2, name


def test_resource_check_rejects_a_kernel_with_scratch(tmp_path):
    from r2omni_amd.build import _check_resources, kernel_resources

    def remarks(name, scratch):
        return "\n".join(f"x.hip:1:1: remark: {body} [-Rpass-analysis=kernel-resource-usage]" for body in (
            f"Function Name: {name}", "VGPRs: 188", "AGPRs: 0", "TotalSGPRs: 86",
            f"ScratchSize [bytes/lane]: {scratch}", "VGPRs Spill: 0", "SGPRs Spill: 0",
            "Occupancy [waves/SIMD]: 2", "LDS Size [bytes/block]: 43008"))

    text = remarks("k_clean", 0) + "\n" + remarks("k_stack", 1296)
    res = kernel_resources(text)
    assert res["k_clean"]["VGPRs"] == 188 and res["k_stack"]["ScratchSize [bytes/lane]"] == 1296
    _check_resources("x.hip", remarks("k_clean", 0), str(tmp_path / "ok.txt"))
    with pytest.raises(RuntimeError, match="k_stack"):
        _check_resources("x.hip", text, str(tmp_path / "bad.txt"))
