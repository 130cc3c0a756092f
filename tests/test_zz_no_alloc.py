"""exl3_linear_noalloc (the linear with a static device scratch, no workspace) against exl3_linear through the C ABI:
two calls in a row, the second with a smaller input, each equal byte for byte to the workspace entry point (the same
kernels and plan run on the same inputs) and within the north-star bar of the oracle."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import _lib, exl3, synth
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3


def _noalloc(L, x, pd, dec, y):
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    dt = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
    return L.exl3_linear_noalloc(x.data_ptr(), dt[x.dtype], x.shape[0], pd.in_features, pd.out_features,
                                 pd.trellis.data_ptr(), pd.n, pd.suh.data_ptr(), pd.svh.data_ptr(), dec.c(),
                                 y.data_ptr(), dt[y.dtype], stream)


def _one(dev, L, seed, rows, in_f, out_f, n, dec, odec, ydt=torch.float16, same_arm=True):
    """same_arm: both entry points take the same arm, so their outputs are equal bit for bit (else both hold the
    oracle's bar)."""
    print(f"[noalloc] rows={rows} {in_f}x{out_f} n={n} y={ydt}", flush=True)
    p = synth.proj(seed, f"na{in_f}x{out_f}", 1, in_f, out_f, n)
    x = synth.normal(seed, f"na.x{rows}", (rows, in_f))
    pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))
    xd = x.to(dev)
    want_bytes = exl3.linear(xd, pd, dec, out_dtype=ydt)
    y = torch.full((rows, out_f), float("nan"), dtype=ydt, device=dev)
    rc = _noalloc(L, xd, pd, dec, y)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    if same_arm:
        assert torch.equal(y, want_bytes)
    want = O.project_rows(x.float().numpy(), p.trellis.numpy().view(np.uint16), p.suh.numpy().view(np.uint16),
                          p.svh.numpy().view(np.uint16), in_f, out_f, n, odec, threads=8)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    assert max_abs_rel(want_bytes.float().cpu().numpy(), want) < BAR


def test_noalloc_gemv_two_calls_second_smaller(dev):
    """16 rows at 4096 x 4096 K4 (the decode GEMV, split, folded), then 1 row at 2048 x 1024 K2."""
    L = _lib.load()
    _one(dev, L, 41, 16, 4096, 4096, 64, exl3.INST3, O.decode(O.CB_3INST))
    _one(dev, L, 42, 1, 2048, 1024, 32, exl3.MCG, O.decode(O.CB_MCG))


def test_noalloc_gemm_and_f32_planes_two_calls_second_smaller(dev):
    """The GEMM arm (300 rows: prepared input in the scratch), then 3 rows with an f32 output (counters + planes)."""
    L = _lib.load()
    _one(dev, L, 43, 300, 2048, 1024, 48, exl3.INST3, O.decode(O.CB_3INST))
    _one(dev, L, 44, 3, 1024, 512, 48, exl3.MCG, O.decode(O.CB_MCG), ydt=torch.float32)


def test_noalloc_keeps_to_its_scratch_where_the_k_split_would_not_fit(dev):
    """400 rows at 2048 x 14336 K3: exl3_linear takes the 512-row tile with k in halves (112 tiles, 57 MiB of
    partials in its workspace); the static scratch cannot hold those, so exl3_linear_noalloc takes the decode-wave tile
    and still holds the bar."""
    L = _lib.load()
    assert L.exl3_linear_workspace_size(400, 2048, 14336, 48) > 32 << 20
    _one(dev, L, 45, 400, 2048, 14336, 48, exl3.INST3, O.decode(O.CB_3INST), same_arm=False)


def test_noalloc_refuses_past_its_scratch(dev):
    """A GEMM whose prepared input (2048 x 14336 f16 = 56 MiB) exceeds the static scratch is refused before any
    launch, with the workspace status."""
    L = _lib.load()
    x = torch.zeros(2048, 14336, dtype=torch.float16, device=dev)
    y = torch.empty(2048, 128, dtype=torch.float16, device=dev)
    t = torch.zeros(1, 14336 // 16, 128 // 16, 48, dtype=torch.int16, device=dev)
    s = torch.ones(1, 14336, dtype=torch.float16, device=dev)
    pd = exl3.Proj(t, s, s[:, :128].contiguous())
    assert _noalloc(L, x, pd, exl3.MCG, y) == exl3.Exl3WorkspaceTooSmall.status
    assert "static scratch" in _lib.last_error()
