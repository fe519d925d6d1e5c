"""ctypes binding of ``libr2o_sspa.so`` (declared in include/r2o_sspa.h).

The library is loaded lazily on first use and the load fails loudly: there is no CPU or
PyTorch fallback for any entry point.  Every call checks the returned status code and raises
``ValueError`` (R2O_EINVAL) or ``RuntimeError`` (R2O_ELAUNCH).
"""
from __future__ import annotations

import ctypes
import os

import torch

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("R2O_SSPA_LIB", os.path.join(_PKG_DIR, "libr2o_sspa.so"))

MAX_BATCH = 32
MAX_GQA = 16
NOALLOC_MAX_ITEMS = 1024  # work items r2o_decode_noalloc's device array holds

c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p


class DecodeParams(ctypes.Structure):
    """Mirror of ``r2o_decode_params``."""

    _fields_ = [
        ("reqs", c_vp),
        ("items", c_vp),
        ("group_begin", c_vp),
        ("n_items", c_i64),
        ("partial_max", c_vp),
        ("partial_sum", c_vp),
        ("partial_out", c_vp),
        ("query", c_vp),
        ("query_batch_stride", c_i64),
        ("append_k", c_vp),
        ("append_v", c_vp),
        ("step_positions", c_vp),
        ("batch", c_i64),
        ("hq", c_i64),
        ("hkv", c_i64),
        ("superblock", c_i64),
        ("int2_group", c_i64),
        ("page_size", c_i64),
        ("q_dtype", c_i64),
        ("output_hadamard", c_i64),
        ("do_append", c_i64),
        ("k_format", c_i64),
        ("sm_scale", ctypes.c_float),
        ("out", c_vp),
        ("append_batch_stride", c_i64),
        ("recent_len", ctypes.c_int32 * MAX_BATCH),
        ("append_global", c_i64 * MAX_BATCH),
        ("append_logical", c_i64 * MAX_BATCH),
        ("row_dtype", c_i64),
        ("group_begin_host", ctypes.c_void_p),
        ("partial_capacity", c_i64),
        ("rope_mode", c_i64),
        ("rope_cos", c_vp),
        ("rope_sin", c_vp),
        ("rope_cos_strides", c_i64 * 4),
        ("rope_sin_strides", c_i64 * 4),
        ("rope_table_dtype", c_i64),
        ("rope_section0", c_i64),
        ("rope_section1", c_i64),
        ("rope_hadamard", c_i64),
        ("value_hadamard", c_i64),
        ("rotated_k", c_vp),
        ("rotated_v", c_vp),
        ("q_norm_weight", c_vp),
        ("k_norm_weight", c_vp),
        ("norm_eps", ctypes.c_float),
    ]


# r2o_request_desc: 22 eight-byte words, in header order.
REQUEST_FIELDS = (
    "k_packed", "k_scale", "k_zero", "k_capacity", "k_superblocks", "k_operands",
    "fp_v", "fp_stride",
    "i4_v", "i4_scale", "i4_stride",
    "i2_v", "i2_scale", "i2_zero", "i2_stride",
    "recent_k", "recent_v", "recent_capacity", "recent_length",
    "recent_global", "recent_logical", "recent_page_lengths",
)
# r2o_work_item: 16 eight-byte words.
ITEM_FIELDS = ("req", "kvh", "kind", "tile0", "ntiles", "lo", "hi", "v_delta", "slot",
               "k_base", "k_ops", "v_base", "v_scale", "v_zero", "ring_length", "v_group")
WORK_FIELDS = ("req", "kvh", "kind", "tile0", "ntiles", "lo", "hi", "v_delta", "slot")
KIND_FP, KIND_INT4, KIND_INT2, KIND_RECENT = 0, 1, 2, 3
# r2o_decode_params.k_format: how the request descriptors' k_* fields hold the history keys
K_INT4, K_BF16, K_INT2 = 0, 1, 2

class PlanRun(ctypes.Structure):  # r2o_plan_run
    _fields_ = [(f, c_i64) for f in ("req", "kvh", "kind", "tile0", "ntiles", "lo", "hi", "v_delta")]


class PlanConfig(ctypes.Structure):  # r2o_plan_config
    _fields_ = [
        ("num_cus", c_i64),
        ("blocks_per_cu", c_i64),
        ("tiles_per_item", c_i64),
        ("waves_per_item", c_i64),
        ("min_tiles_per_item", c_i64),
        ("tile_cost", ctypes.c_double * 4),
        ("late_share", ctypes.c_double),
    ]


_SIGNATURES = {
    "r2o_plan_work_items": (ctypes.POINTER(PlanRun), c_i64, ctypes.POINTER(PlanConfig), c_vp, c_i64, c_i64, c_i64,
                            c_vp, c_i64, c_vp, c_i64, ctypes.POINTER(c_i64)),
    "r2o_decode_partial": (ctypes.POINTER(DecodeParams), c_vp),
    "r2o_decode_combine": (ctypes.POINTER(DecodeParams), c_vp),
    "r2o_decode": (ctypes.POINTER(DecodeParams), c_vp),
    "r2o_decode_noalloc": (ctypes.POINTER(DecodeParams), c_vp),
    "r2o_decode_noalloc_init": (ctypes.c_int,),
    "r2o_pack_int4_k": (c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                        c_vp),
    "r2o_pack_int2_k": (c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                        c_vp),
    "r2o_pack_int4_v": (c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp),
    "r2o_pack_int2_v": (c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp),
    "r2o_gather_rows": (c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp),
    "r2o_recent_append": (c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp),
    "r2o_recent_shift": (c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp),
    "r2o_fwht128": (c_vp, c_vp, c_i64, c_i64, c_vp),
    "r2o_qk_mrope": (c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp,
                     c_i64, c_i64, c_i64, c_vp),
    "r2o_qkv_mrope": (c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_vp,
                      c_vp, c_i64, c_i64, c_i64, c_vp),
    "r2o_qkv_norm_rope": (c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp,
                          ctypes.c_float, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp),
    "r2o_qk_norm_rope": (c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp, ctypes.c_float,
                         c_vp, c_vp, c_vp, c_vp, c_i64, c_vp),
}
EXPORTED = tuple(_SIGNATURES) + ("r2o_build_target",)

_LIB = None


def load() -> ctypes.CDLL:
    """Load and bind the library (raises if it is missing: no fallback exists)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m r2omni_amd.build` "
                "(the SSPA decode path has no CPU or PyTorch fallback)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = list(args)
            fn.restype = ctypes.c_int
        lib.r2o_build_target.restype = ctypes.c_char_p
        lib.r2o_build_target.argtypes = []
        _LIB = lib
    return _LIB


def check(rc: int, name: str) -> None:
    if rc == 0:
        return
    if rc == 1:
        raise ValueError(f"{name}: invalid argument (rejected by the host-side check before launch)")
    raise RuntimeError(f"{name}: HIP launch failed (status {rc})")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The device's current stream handle.  torch's raw lookup (the one its generated code uses)
    takes ~0.1 us; ``torch.cuda.current_stream(device).cuda_stream`` builds a Stream object, ~2 us
    per launch on the eager path."""
    if device.type != "cuda":
        raise RuntimeError(f"expected a GPU tensor, got one on {device}: the SSPA packed-KV path runs only "
                           "as HIP kernels on gfx950 (no CPU fallback)")
    if _RAW_STREAM is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return 0
    if dtype == torch.float16:
        return 1
    raise ValueError(f"K/V/Q rows must be bfloat16 or float16, got {dtype}")


def require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{what} must live on the GPU: the SSPA packed-KV path runs only as HIP kernels "
            "on gfx950 (no CPU fallback)"
        )
