"""The C-ABI library loads and exports every entry point include/*.h declares; host-side refusals happen before any
launch.  No compute call here needs a GPU."""
import ctypes
import glob
import os
import re

import pytest

import sushi_amd._lib as L
from sushi_amd import exl3

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", src))
    return names


def test_header_declares_the_exports_the_binding_uses():
    assert set(L.EXPORTS) == _declared()


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(L.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_and_host_side_refusals():
    lib = L.load()
    assert lib.exl3_abi_version() == 5
    d = L.DecodeT(1, 16, -1)
    # bad shape: in not a multiple of 128 -> refused before any launch (null pointers never touched)
    assert lib.exl3_linear(None, 0, 1, 100, 128, None, 64, None, None, d, None, 0, None, 0, None) == -1
    assert "multiples of 128" in L.last_error()
    # unadmitted rate
    assert lib.exl3_linear(None, 0, 1, 128, 128, None, 130, None, None, d, None, 0, None, 0, None) == -1
    # a tabled codebook without its table: Exl3CodebookTableUnknown
    assert lib.exl3_linear(None, 0, 1, 128, 128, None, 64, None, None, L.DecodeT(2, 15, -1), None, 0, None, 0,
                           None) == -3
    # STD1 has no row at n=16: Exl3CodebookTableRateMissing
    assert lib.exl3_linear(None, 0, 1, 128, 128, None, 16, None, None, L.DecodeT(4, 15, 3), None, 0, None, 0,
                           None) == -10
    # bad window
    assert lib.exl3_linear(None, 0, 1, 128, 128, None, 64, None, None, L.DecodeT(1, 7, -1), None, 0, None, 0,
                           None) == -11
    # dtype
    assert lib.exl3_linear(None, 9, 1, 128, 128, None, 64, None, None, d, None, 0, None, 0, None) == -2
    # rows == 0 is a no-op
    assert lib.exl3_linear(None, 0, 0, 128, 128, None, 64, None, None, d, None, 0, None, 0, None) == 0
    # workspace too small (rows=1 needs counters)
    assert lib.exl3_linear(4, 0, 1, 128, 128, 1, 64, 1, 1, d, 1, 0, None, 0, None) == -9
    # x must be 4-byte aligned (the kernels read activations as aligned 32-bit words)
    assert lib.exl3_linear(2, 0, 1, 128, 128, 1, 64, 1, 1, d, 1, 0, None, 0, None) == -1
    assert "aligned" in L.last_error()


def test_moe_refusals():
    lib = L.load()
    d = L.DecodeT(1, 16, -1)
    bank = L.BankT()
    args = lambda topk, clamp, sdt=0: (None, 0, 1, 128, 128, 4, ctypes.byref(bank), None, None, sdt, topk, d, 0,
                                       clamp, None, None, 0, None, 0, None)
    assert lib.exl3_moe(*args(33, 0)) == -4  # Exl3TopKExceedsReduceBank
    assert lib.exl3_moe(*args(8, 129)) == -6  # InvalidExl3Clamp
    assert lib.exl3_moe(*args(8, 0)) == -1  # projections missing
    assert lib.exl3_moe(*args(8, 0, sdt=7)) == -2  # scores dtype: f32, bf16 or f16 (root.zig:114)
    for sdt in (1, 2):
        assert lib.exl3_moe(*args(8, 0, sdt=sdt)) == -1  # bf16 / f16 scores admitted (then the missing projections)
    # the gated shared expert needs both its output and its gate
    gargs = (None, 0, 1, 128, 128, 4, ctypes.byref(bank), None, None, 0, 8, d, 0, None, None, None, 0, None, 0, None)
    assert lib.exl3_moe_with_gated_shared(*gargs) == -1
    assert "gate" in L.last_error()
    assert lib.exl3_route_topk(None, 1, 2000, 8, None, None, None) == -1


def test_moe_groups_and_linear_pair_refusals():
    """moeGroups without banks is Exl3GroupMissing (root.zig:647); a bad group bank is refused before any launch;
    linearPair past one decode launch's rows declines (status 1, the reference's null) before any launch (the fake
    pointers are never dereferenced)."""
    lib = L.load()
    d = L.DecodeT(1, 16, -1)
    counts = (ctypes.c_int32 * 2)(4, 4)
    banks = (L.BankT * 2)()
    assert lib.exl3_moe_groups(None, 0, 1, 128, 128, 0, banks, counts, None, None, 0, 8, d, 0, None, 0, None, 0,
                               None) == -16
    assert lib.exl3_moe_groups(None, 0, 1, 128, 128, 2, banks, counts, None, None, 0, 8, d, 0, None, 0, None, 0,
                               None) == -1  # the banks' projections are missing
    fake = 0x1000
    assert lib.exl3_linear_pair(fake, 0, 2, 17, 128, 128, 256, fake, 32, fake, fake, d, fake, 32, fake, fake, d, fake,
                                0, None, 0, None) == 1
    assert "declined" in L.last_error()
    assert lib.exl3_linear_pair(fake, 0, 2, 4, 128, 100, 256, fake, 32, fake, fake, d, fake, 32, fake, fake, d, fake,
                                0, None, 0, None) == -1  # mid not a multiple of 128
    assert lib.exl3_linear_pair_workspace_size(2, 4, 128, 128, 256) > 0
    assert lib.exl3_linear_pair_workspace_size(2, 17, 128, 128, 256) == 0


def test_tiled_refusals():
    """Per-tile-rate banks: only the K1 / K2 pair, tables that hold both rates, the hash-product families, a 4-byte
    aligned mask table; every refusal before any launch (the fake pointers are never dereferenced)."""
    lib = L.load()
    fake = ctypes.c_void_p(0x1000)
    tb = L.TiledT()
    for i in range(3):
        tb.trellis[i] = tb.seg_off[i] = tb.seg_k1[i] = tb.suh[i] = tb.svh[i] = fake.value
    tb.experts, tb.n_a, tb.n_b = 4, 16, 32

    def moe(dec, bank=tb):
        return lib.exl3_moe_tiled(None, 0, 0, 128, 128, ctypes.byref(bank), None, None, 2, 8, dec, 0, 0, None, None,
                                  None, 0, None, 0, None)

    assert moe(L.DecodeT(2, 15, 1)) == 0  # spec1-w15 has rows at 16 and 32; zero rows: nothing to launch
    assert moe(L.DecodeT(1, 16, -1)) == 0  # MCG
    assert moe(L.DecodeT(4, 15, 3)) == -10  # std1 has no row at n = 16
    assert moe(L.DecodeT(2, 16, 2)) == -10  # nor spec1-w16
    assert moe(L.DecodeT(3, 16, 0)) == -10  # PAIR1 has no pair row at 16
    assert moe(L.DecodeT(0, 16, -1)) == -12  # MUL1: not a hash-product family
    tb.n_b = 48
    assert moe(L.DecodeT(1, 16, -1)) == -1 and "16 / 32" in L.last_error()
    tb.n_b = 32
    tb.seg_k1[1] = 0x1002
    assert moe(L.DecodeT(1, 16, -1)) == -1 and "aligned" in L.last_error()
    tb.seg_k1[1] = fake.value
    tb.suh[2] = None
    assert moe(L.DecodeT(1, 16, -1)) == -1 and "null" in L.last_error()
    assert lib.exl3_reconstruct_tiled(fake, fake, fake, 0, 128, 100, 16, 32, L.DecodeT(1, 16, -1), fake, None) == -1
    assert lib.exl3_reconstruct_tiled(fake, fake, fake, 0, 128, 128, 16, 24, L.DecodeT(1, 16, -1), fake, None) == -1


def test_workspace_sizes_are_aligned_and_monotone():
    lib = L.load()
    a = lib.exl3_linear_workspace_size(1, 4096, 4096, 64)
    b = lib.exl3_linear_workspace_size(8, 4096, 4096, 64)
    c = lib.exl3_linear_workspace_size(64, 4096, 4096, 64)
    assert a % 256 == 0 and b >= a and c > 0
    assert lib.exl3_moe_workspace_size(1, 8, 2048, 768) > 0


def test_python_mirror_refuses_by_name():
    with pytest.raises(exl3.Exl3CodebookTableUnknown):
        exl3.Decode(exl3.Codebook.spec1).require_table()
    with pytest.raises(exl3.InvalidExl3Clamp):
        exl3.moe_clamped(None, None, None, None, exl3.MCG, 0)
    with pytest.raises(exl3.Exl3TopKExceedsReduceBank):
        exl3.admit_top_k(33)
    assert exl3.k_from_packed_dim(41) is None and exl3.k_from_packed_dim(40).n == 40
    assert exl3.Rate(44).fresh_bits(1) == 3 and exl3.Rate(64).bit_end(255) == 1024
    assert exl3.Decode.tabled(exl3.Codebook.std1).table == exl3.Table.std1


def test_synth_is_deterministic_and_name_keyed():
    from sushi_amd import synth

    a = synth.codes(0, "w", (4, 8))
    b = synth.codes(0, "w", (4, 8))
    c = synth.codes(0, "v", (4, 8))
    assert (a == b).all() and not (a == c).all()
    s = synth.sign_scale(0, "s", (1000,)).float()
    assert ((s.abs() >= 0.5) & (s.abs() <= 1.5)).all() and (s < 0).any() and (s > 0).any()
    x = synth.normal(0, "x", (20000,)).float()
    assert abs(float(x.mean())) < 0.05 and abs(float(x.std()) - 1) < 0.05


def test_bench_refuses_more_than_one_gpu_before_touching_one():
    """bench.py measures one GPU: N > 1 exits with status 2 and a message saying so (no GPU is touched)."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "4"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2 and "one GPU only" in r.stderr and r.stdout == ""


def test_set_override_refuses_unknown_knobs_and_the_reserved_value():
    lib = L.load()
    assert lib.exl3_set_override(99, 1, 1) == -1
    assert lib.exl3_set_override(0, -2 ** 31, 1) == -1
    assert lib.exl3_set_override(0, 4, 1) == 0 and lib.exl3_set_override(0, 0, 0) == 0
    with exl3.arm_overrides(gemv_splits=2, moe_fold=0):
        pass  # set and unset again on exit


class _CpuWorkspace(exl3._Workspace):
    """The workspace cache with its device hooks replaced: streams are plain handles, buffers CPU tensors."""

    def __init__(self):
        super().__init__()
        self.stream = 1
        self.capturing = False
        self.made = []

    def _stream_handle(self, dev):
        return self.stream

    def _capturing(self):
        return self.capturing

    def _new(self, dev, size, handle):
        import torch

        self.made.append((handle, size))
        return torch.zeros(size, dtype=torch.uint8)


def test_workspace_is_one_buffer_per_stream_and_keeps_grown_out_buffers():
    import torch

    ws = _CpuWorkspace()
    dev = torch.device("cpu")
    a = ws.get(dev, 100)
    assert ws.get(dev, 100) is a                      # the same stream reuses its buffer
    ws.stream = 2
    b = ws.get(dev, 100)
    assert b is not a                                  # another stream (a capture's side stream) gets its own
    ws.stream = 1
    c = ws.get(dev, (1 << 20) + 1)                     # growth replaces stream 1's buffer...
    assert c is not a and c.numel() >= (1 << 20) + 1
    assert any(r is a for r in ws._retired)            # ...and keeps the old one alive for graphs that hold it
    ws.capturing = True
    assert ws.get(dev, 10) is c                        # inside a capture an existing buffer serves
    with pytest.raises(exl3.Exl3WorkspaceTooSmall):
        ws.get(dev, 1 << 24)                           # but nothing is allocated there
    ws.stream = 3
    with pytest.raises(exl3.Exl3WorkspaceTooSmall):
        ws.get(dev, 10)                                # a stream first seen inside a capture is refused
    assert [h for h, _ in ws.made] == [1, 2, 1]
