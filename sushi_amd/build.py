"""Builds libsushi_exl3_hip.so in-tree with hipcc for gfx950 (one object per translation unit, in parallel).

Run as ``python -m sushi_amd.build`` or through ``__graft_entry__.build()``.  Every call recompiles (the driver's
"does it build" check); ``load()`` in ``sushi_amd._lib`` only loads what is built.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsushi_exl3_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("EXL3_OFFLOAD_ARCH", "gfx950")

SOURCES = [
    "exl3_capi.hip",
    "exl3_decode.hip",
    "exl3_moe.hip",
    "exl3_gemm.hip",
    "exl3_gemv_mcg.hip",
    "exl3_gemv_mul1.hip",
    "exl3_gemv_hash.hip",
    "exl3_gemv_pair.hip",
    "exl3_gemv_3inst.hip",
    "exl3_encode.hip",
    "exl3_quantize.hip",
]

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # Packed FP32 (v_pk_*_f32) stays off: hipcc would otherwise form it from scalar float code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading scalar kernel arguments arrive preloaded in SGPRs (the GEMV's first loads need no argument load).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # Kernels take their argument structs by value.  The compiler reads such a struct straight from the argument
    # segment only after walking every use of its local copy, and its default walk stops at 300 uses; the fused
    # shared-expert windows kernels have over a thousand, and past the limit every wave copied the struct to scratch
    # memory and read its fields from there (2.2x slower per window).
    "-mllvm", "-instcombine-max-copied-from-constant-users=4096",
    "-I", os.path.join(HERE, "..", "include"),
]


def _stale(src: str, obj: str) -> bool:
    """An object older than its source or than any header it may include (csrc/*.h, *.cuh, include/*.h)."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith((".h", ".cuh"))]
    inc = os.path.join(HERE, "..", "include")
    deps += [os.path.join(inc, h) for h in os.listdir(inc) if h.endswith(".h")]
    return any(os.path.getmtime(d) > t for d in deps)


INCREMENTAL = False


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    if INCREMENTAL and not _stale(src, obj):
        return obj
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    noise = "is not a recognized feature for this target"
    warn = "\n".join(l for l in r.stderr.splitlines() if l.strip() and noise not in l)
    if warn:
        print(f"[build] {src}:\n{warn[-3000:]}", file=sys.stderr)
    return obj


BENCH_SOURCES = ["bench_stream.hip"]
BENCH_LIB = os.path.join(HERE, "libsushi_bench_hip.so")


def _link(objs, out: str) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, out)


def build(jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    t0 = time.time()
    jobs = jobs or min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES + BENCH_SOURCES))
    _link(objs[:len(SOURCES)], LIB)
    _link(objs[len(SOURCES):], BENCH_LIB)  # bench.py's measurement kernels, outside the hot path's library
    if verbose:
        print(f"[build] {LIB} ({os.path.getsize(LIB) / 1e6:.1f} MB) in {time.time() - t0:.0f}s", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    # --incremental (development only): recompile only objects older than their sources or headers
    INCREMENTAL = "--incremental" in sys.argv[1:]
    build()
