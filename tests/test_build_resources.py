"""Every kernel of the built gfx950 library runs without scratch memory and without VGPR spills.

Read from the code-object metadata of the objects `python -m sushi_amd.build` leaves in sushi_amd/_build
(`.private_segment_fixed_size`, `.vgpr_spill_count`).  Scratch in these kernels has meant the compiler copying a
by-value argument struct into every wave's private memory (the fused shared-expert windows kernels did, at 2.2x the
time per window), and a VGPR spill is a memory round trip inside a hot loop; either is a regression to catch at build
time, not on the GPU.  Runs on the CPU with the ROCm binutils; skipped where the objects or the tools are absent.
"""
import glob
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "sushi_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
BUNDLER = os.path.join(LLVM, "clang-offload-bundler")
READELF = os.path.join(LLVM, "llvm-readelf")

OBJECTS = sorted(glob.glob(os.path.join(BUILD, "exl3_*.o")))


def _kernels(obj: str, tmp) -> list:
    """(name, private segment bytes, VGPR spills) of every kernel in obj's gfx950 code object."""
    fat = os.path.join(tmp, "fat.bin")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", obj, fat], check=True)
    targets = subprocess.run([BUNDLER, "--list", "--type=o", f"--input={fat}"], capture_output=True, text=True,
                             check=True).stdout.split()
    target = next(t for t in targets if "gfx950" in t)
    dev = os.path.join(tmp, "dev.o")
    subprocess.run([BUNDLER, "--unbundle", "--type=o", f"--input={fat}", f"--targets={target}", f"--output={dev}"],
                   check=True)
    notes = subprocess.run([READELF, "--notes", dev], capture_output=True, text=True, check=True).stdout
    out = []
    for block in re.split(r"\n\s+- \.agpr_count", notes)[1:]:
        field = lambda k: re.search(r"\." + k + r":\s+(\S+)", block)  # noqa: E731
        name = field("name")
        if name is None:
            continue
        out.append((name.group(1), int(field("private_segment_fixed_size").group(1)),
                    int(field("vgpr_spill_count").group(1))))
    return out


@pytest.mark.skipif(not OBJECTS or not (os.path.exists(BUNDLER) and os.path.exists(READELF) and shutil.which("objcopy")),
                    reason="needs the built objects (python -m sushi_amd.build) and the ROCm binutils")
def test_no_kernel_uses_scratch_or_spills(tmp_path):
    kernels = {os.path.basename(o): _kernels(o, str(tmp_path)) for o in OBJECTS}
    # the GEMV, GEMM, MoE, decode and encoder objects all hold kernels (the C-ABI object holds none)
    for name in ("exl3_gemv_3inst.o", "exl3_gemm.o", "exl3_moe.o", "exl3_decode.o", "exl3_encode.o"):
        assert kernels.get(name), f"no kernel metadata read from {name}"
    bad = [(o, n, scratch, spills) for o, ks in kernels.items() for n, scratch, spills in ks if scratch or spills]
    assert not bad, f"{len(bad)} kernels with scratch bytes / VGPR spills, e.g. {bad[:3]}"
