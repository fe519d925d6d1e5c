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


def test_params_struct_layout_matches_header():
    # offsets computed by the C compiler for the same struct, via a tiny host-only probe
    p = _lib.DecodeParams
    assert p.recent_len.offset == p.sm_scale.offset + 4
    assert p.append_global.offset % 8 == 0
    assert ctypes.sizeof(p) == p.append_logical.offset + 8 * _lib.MAX_BATCH


def test_host_side_validation_rejects_bad_arguments_without_a_gpu():
    lib = _lib.load()
    # superblock 48 is rejected before any launch
    rc = lib.r2o_pack_int4_k(None, 0, 2, 10, None, 10, 0, 0, None, None, None, None, 128, 3, 48, None)
    assert rc == 1
    rc = lib.r2o_pack_int2_v(None, 0, 2, 10, None, 10, 0, 48, None, None, None, 128, None)
    assert rc == 1
    params = _lib.DecodeParams()
    assert lib.r2o_decode_partial(ctypes.byref(params), None) == 1
    assert lib.r2o_build_target() == b"gfx950"
