"""Compile the gfx950 HIP sources into the in-tree C-ABI library ``libr2o_sspa.so``.

Usage: ``python -m r2omni_amd.build`` (from ``r2-omni_amd/``) or ``build_library()``.
Every HIP translation unit is compiled for gfx950 only, with packed-FP32 instruction
selection disabled and FP contraction off (the quantisers must round exactly like the
reference's torch CPU path).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)                 # r2-omni_amd/
REPO_DIR = os.path.dirname(ROOT_DIR)
CSRC = os.path.join(ROOT_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "libr2o_sspa.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ("r2o_decode.hip", "r2o_pack.hip", "r2o_rope.hip", "r2o_plan.cpp")  # r2o_plan.cpp: host code only
# bench.py's streaming-read probe, a library of its own (not part of the decode C-ABI)
BENCH_LIB_PATH = os.path.join(PKG_DIR, "libr2o_bench.so")
BENCH_SOURCES = ("bench_read.hip",)
# the same decode library built with per-wave phase stamps (-DR2O_TIMELINE), for bench.py --timeline only
TIMELINE_LIB_PATH = os.path.join(PKG_DIR, "libr2o_timeline.so")
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libr2o_sspa.so")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-fPIC",
        "-std=c++17",
        "-ffp-contract=off",
        "-munsafe-fp-atomics",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE,
        "-I", CSRC,
    ]


def build_library(verbose: bool = False) -> str:
    """Compile every source and link ``libr2o_sspa.so`` (and bench.py's ``libr2o_bench.so`` and
    ``libr2o_timeline.so``) next to this file; returns the decode library's path."""
    _link(SOURCES, LIB_PATH, verbose)
    _link(BENCH_SOURCES, BENCH_LIB_PATH, verbose)
    _link(SOURCES, TIMELINE_LIB_PATH, verbose, defines=("R2O_TIMELINE",), rebuild=("r2o_decode.hip",))
    return LIB_PATH


def _link(sources, path: str, verbose: bool, defines=(), rebuild=None) -> None:
    """Compile ``sources`` (only those in ``rebuild`` when given, reusing the other objects of the
    plain build) with ``defines`` and link them into ``path``."""
    hipcc = _hipcc()
    build_dir = os.path.join(ROOT_DIR, "_build")
    os.makedirs(build_dir, exist_ok=True)
    suffix = "".join("_" + d.lower() for d in defines)
    objects = []
    for src in sources:
        stem = os.path.splitext(src)[0]
        if rebuild is not None and src not in rebuild:
            objects.append(os.path.join(build_dir, stem + ".o"))
            continue
        obj = os.path.join(build_dir, stem + suffix + ".o")
        cmd = [hipcc, *common_flags(), *[f"-D{d}" for d in defines], "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".hip"):
            cmd.append("-Rpass-analysis=kernel-resource-usage")
        stderr = _run(cmd, verbose)
        if src.endswith(".hip"):
            _check_resources(src + suffix, stderr, os.path.join(build_dir, stem + suffix + ".resources.txt"))
        objects.append(obj)
    tmp = path + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", tmp], verbose)
    os.replace(tmp, path)


def _run(cmd: list[str], verbose: bool) -> str:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"HIP build failed: {' '.join(cmd[:3])} ... ({res.returncode})")
    noise = ("is not a recognized feature for this target", "-Rpass-analysis=kernel-resource-usage")
    rest = [ln for ln in (res.stderr or "").splitlines() if not any(n in ln for n in noise) and ln.strip()
            and not ln.startswith(" ")]
    if verbose and rest:
        sys.stderr.write("\n".join(rest) + "\n")
    return res.stderr or ""


_RESOURCE_KEYS = ("VGPRs", "AGPRs", "TotalSGPRs", "ScratchSize [bytes/lane]", "VGPRs Spill", "SGPRs Spill",
                  "Occupancy [waves/SIMD]", "LDS Size [bytes/block]")


def kernel_resources(stderr: str) -> dict[str, dict[str, int]]:
    """Per-kernel register, scratch and LDS figures from the compiler's kernel-resource-usage remarks."""
    out: dict[str, dict[str, int]] = {}
    name = None
    for ln in stderr.splitlines():
        if "remark:" not in ln:
            continue
        body = ln.split("remark:", 1)[1].strip()
        if body.startswith("Function Name:"):
            name = body.split(":", 1)[1].split("[")[0].strip()
            out[name] = {}
            continue
        for key in _RESOURCE_KEYS:
            if name is not None and body.startswith(key + ":"):
                out[name][key] = int(body.split(":", 1)[1].split()[0])
    return out


def _check_resources(what: str, stderr: str, path: str) -> None:
    """Every kernel keeps its state in registers and LDS: a kernel with scratch (a spill, a private
    array indexed at run time, or a device function left as a call, whose arguments and saved
    registers go through the stack) fails the build.  The figures are kept beside the object."""
    res = kernel_resources(stderr)
    with open(path, "w") as f:
        f.write("kernel " + " | ".join(_RESOURCE_KEYS) + "\n")
        for k, v in sorted(res.items()):
            f.write(k + " " + " | ".join(str(v.get(key, "?")) for key in _RESOURCE_KEYS) + "\n")
    bad = [k for k, v in res.items() if v.get("ScratchSize [bytes/lane]", 0) or v.get("VGPRs Spill", 0)
           or v.get("SGPRs Spill", 0)]
    if bad:
        raise RuntimeError(f"{what}: kernels using scratch memory: {', '.join(sorted(bad))}")


if __name__ == "__main__":
    print(build_library(verbose=True))
