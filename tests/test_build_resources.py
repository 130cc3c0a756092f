"""Every kernel of the built gfx950 library runs without scratch memory and without VGPR spills, and no matrix
instruction reads a VGPR that a vector instruction wrote fewer than three instructions before it.

Read from the code-object metadata of the objects `python -m sushi_amd.build` leaves in sushi_amd/_build
(`.private_segment_fixed_size`, `.vgpr_spill_count`).  Scratch in these kernels has meant the compiler copying a
by-value argument struct into every wave's private memory (the fused shared-expert windows kernels did, at 2.2x the
time per window), and a VGPR spill is a memory round trip inside a hot loop; either is a regression to catch at build
time, not on the GPU.  The MFMA check guards a hazard the compiler does not count for inline asm: the decode's
half sums are SDWA adds written in asm, and an MFMA that read one two instructions after it was written read the
stale register (wrong weights, silently).  The compiler keeps its own writes three or more instructions ahead of an
MFMA that reads them; the decode's fenced phases keep the asm ones so.  Runs on the CPU with the ROCm binutils;
skipped where the objects or the tools are absent.
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
OBJDUMP = os.path.join(LLVM, "llvm-objdump")

OBJECTS = sorted(glob.glob(os.path.join(BUILD, "exl3_*.o")))


def _device_object(obj: str, tmp) -> str:
    """obj's gfx950 code object, unbundled into tmp."""
    fat = os.path.join(tmp, "fat.bin")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", obj, fat], check=True)
    targets = subprocess.run([BUNDLER, "--list", "--type=o", f"--input={fat}"], capture_output=True, text=True,
                             check=True).stdout.split()
    target = next(t for t in targets if "gfx950" in t)
    dev = os.path.join(tmp, "dev.o")
    subprocess.run([BUNDLER, "--unbundle", "--type=o", f"--input={fat}", f"--targets={target}", f"--output={dev}"],
                   check=True)
    return dev


def _kernels(obj: str, tmp) -> list:
    """(name, private segment bytes, VGPR spills) of every kernel in obj's gfx950 code object."""
    dev = _device_object(obj, tmp)
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


_VREG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")


def _vregs(text: str) -> set:
    out = set()
    for m in _VREG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _close_mfma_reads(obj: str, tmp, window: int = 2) -> list:
    """(kernel, distance, writer) for every MFMA whose A or B VGPRs a vector instruction wrote `window` or fewer
    issued instructions before it (s_nop N counting N + 1), within one basic block."""
    dev = _device_object(obj, tmp)
    proc = subprocess.Popen([OBJDUMP, "-d", "--no-show-raw-insn", dev], stdout=subprocess.PIPE, text=True)
    bad, kernel, recent = [], None, []  # recent: (issue slots, vector destination VGPRs, opcode), newest last
    for line in proc.stdout:
        head = re.match(r"^[0-9a-f]+ <(.*)>:", line)
        if head:
            kernel, recent = head.group(1), []
            continue
        ins = line.split("//")[0].strip()
        if not ins or ins.endswith(":"):
            continue
        op, _, rest = ins.partition(" ")
        if op.startswith("s_cbranch") or op == "s_branch" or op == "s_endpgm":
            recent = []
            continue
        if op.startswith("v_mfma"):
            ops = [o.strip() for o in rest.split(",")]
            src = _vregs(ops[1]) | _vregs(ops[2])
            dist = 0
            for slots, dst, wop in reversed(recent):
                dist += slots
                if dist > window:
                    break
                if dst & src:
                    bad.append((kernel, dist, wop))
                    break
        slots = int(rest) + 1 if op == "s_nop" else 1
        dst = _vregs(rest.split(",")[0]) if op.startswith("v_") and not op.startswith("v_mfma") else set()
        recent.append((slots, dst, op))
        recent = recent[-8:]
    proc.wait()
    return bad


@pytest.mark.skipif(not OBJECTS or not (os.path.exists(BUNDLER) and os.path.exists(OBJDUMP) and shutil.which("objcopy")),
                    reason="needs the built objects (python -m sushi_amd.build) and the ROCm binutils")
def test_no_mfma_reads_a_vgpr_written_just_before(tmp_path):
    objs = [o for o in OBJECTS if re.search(r"exl3_(gemv_\w+|gemm|moe)\.o$", o)]
    assert len(objs) >= 7, objs
    bad = [(os.path.basename(o),) + b for o in objs for b in _close_mfma_reads(o, str(tmp_path))]
    assert not bad, f"{len(bad)} MFMAs read a VGPR written two or fewer instructions before, e.g. {bad[:3]}"
