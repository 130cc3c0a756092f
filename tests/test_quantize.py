"""Whole-tensor quantizer: the CPU oracle against the reference's tensor fixture and its own properties, then the GPU
quantizer (``exl3_quantize_tensor``) against the fixture and the oracle, code for code.

The oracle restates src/encoder/quantize.zig; the checks follow the reference's tests (quantize.zig:683-993).
``exl3_encode_tensor.safetensors`` holds a 256x128 weight W, a Hessian H, the sign vectors, the regularized scales and
inner matrix, and for five (codebook, rate, window, rows, out-scales) points the packed codes, f16 scales and global
scale of the whole tensor.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import oracle as O

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref", "exl3_encode_tensor.safetensors")
TENSOR_CONFIGS = [  # quantize.zig:658-664
    ("mcg_n32_w12_r256_auto", O.CB_MCG, 32, 12, 256, "auto"),
    ("mul1_n40_w12_r256_always", O.CB_MUL1, 40, 12, 256, "always"),
    ("mcg_n24_w12_r256_never", O.CB_MCG, 24, 12, 256, "never"),
    ("mcg_n40_w15_r128_auto", O.CB_MCG, 40, 15, 128, "auto"),
    ("mul1_n64_w12_r128_always", O.CB_MUL1, 64, 12, 128, "always"),
]
BRACKET = {O.CB_MCG: (0.5, 1.5), O.CB_MUL1: (0.4, 1.2)}


@pytest.fixture(scope="module")
def fx():
    from safetensors.numpy import load_file

    d = load_file(FIXTURE)
    d["W32"] = d["W"].astype(np.float32)
    d["H32"] = d["H"].astype(np.float32)
    return d


def _close(want, got, rel, floor):
    want = np.asarray(want, np.float32)
    got = np.asarray(got, np.float32)
    assert want.shape == got.shape
    bad = np.abs(want - got) > rel * np.abs(want) + floor
    assert not bad.any(), f"{bad.sum()} values off, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("rows,mode", [(256, "always"), (256, "never"), (256, "auto"), (128, "auto"), (128, "always")])
def test_regularize_reproduces_the_reference_scales_and_inner_matrix(fx, rows, mode):  # quantize.zig:683-709
    hdiag = np.diag(fx["H32"])[:rows].copy()
    inner, suh, svh = O.quant_regularize(fx["W32"][:rows], fx[f"sign_in_r{rows}"], fx["sign_out"], mode, hdiag)
    _close(fx[f"reg_r{rows}_{mode}.suh"], suh, 2e-6, 1e-9)
    _close(fx[f"reg_r{rows}_{mode}.svh"], svh, 2e-6, 1e-9)
    if rows == 256 and mode == "always":
        _close(fx["reg_r256_always.inner"].astype(np.float32), inner, 1.5e-3, 1e-5)


def test_the_decoders_transform_chain_turns_the_inner_matrix_back_into_the_weight(fx):  # quantize.zig:711-737
    w = fx["W32"]
    inner, suh, svh = O.quant_regularize(w, fx["sign_in_r256"], fx["sign_out"], "always", None)
    pub = inner.copy()
    for b in range(0, 256, 128):
        for c in range(128):
            pub[b:b + 128, c] = O.hadamard128(pub[b:b + 128, c])
    pub *= suh[:, None]
    for r in range(256):
        pub[r] = O.hadamard128(pub[r])
    pub *= svh[None, :]
    _close(w, pub, 1e-3, 1e-6)


def test_the_block_ldl_factor_carries_h10_equal_l10_h00():  # quantize.zig:739-767
    rng = np.random.default_rng(5)
    n = 32
    a = rng.standard_normal((n, n)).astype(np.float32)
    h = (a @ a.T / n).astype(np.float32)
    l = O.quant_ldl_factor(h)
    mean = float(np.float32(np.diag(h).astype(np.float64).sum() / n))
    for i in range(n):
        for j in range(n):
            if i // 16 == j // 16 or j > i:
                assert l[i, j] == 0
    h00 = h[:16, :16].astype(np.float64) + np.eye(16) * (0.025 * mean)
    np.testing.assert_allclose(l[16:, :16].astype(np.float64) @ h00, h[16:, :16], atol=2e-4)


def test_the_cholesky_factor_reproduces_its_matrix_and_names_a_failing_pivot():  # quantize.zig:862-891
    rng = np.random.default_rng(31)
    n = 200
    x = rng.standard_normal((n, 96))
    a = x @ x.T + 0.5 * np.eye(n)
    bad, l = O.cholesky_lower(a)
    assert bad == 0
    low = np.tril(l)
    np.testing.assert_allclose(low @ low.T, a, atol=1e-9)
    broken = a.copy()
    broken[70, 70] = -1
    assert O.cholesky_lower(broken)[0] == 71
    broken[70, 70] = np.nan
    assert O.cholesky_lower(broken)[0] != 0


def test_a_hessian_that_stays_indefinite_is_refused():
    h = -np.eye(128, dtype=np.float32)
    with pytest.raises(ValueError, match="HessianNotPositiveDefinite"):
        O.quant_ldl_factor(h)


@pytest.mark.parametrize("case", TENSOR_CONFIGS, ids=lambda c: c[0])
def test_oracle_whole_tensor_reproduces_the_reference_trellis_scales_and_global_scale(fx, case):  # :769-797
    name, cb, n, w, rows, mode = case
    h = np.ascontiguousarray(fx["H32"][:rows, :rows])
    packed, suh, svh, g = O.quantize_tensor(fx["W32"][:rows], h, fx[f"sign_in_r{rows}"], fx["sign_out"], n,
                                            O.decode(cb, w), mode)
    np.testing.assert_array_equal(packed.reshape(-1), fx[name + ".packed"].reshape(-1))
    lo, hi = BRACKET[cb]
    assert lo < g < hi and abs(g - float(fx[name + ".g"][0])) <= 1e-5
    np.testing.assert_array_equal(suh, fx[name + ".suh"].view(np.uint16))
    np.testing.assert_array_equal(svh, fx[name + ".svh"].view(np.uint16))


def test_sign_vectors_are_a_pure_function_of_seed_and_name():  # quantize.zig:800-815
    from sushi_amd import exl3

    name = "language_model.model.layers.0.mlp.switch_mlp.gate_proj"
    a, b = exl3.signs(7, name, 128), exl3.signs(7, name, 128)
    other = exl3.signs(7, "language_model.model.layers.0.mlp.switch_mlp.up_proj", 128)
    reseeded = exl3.signs(8, name, 128)
    np.testing.assert_array_equal(a, b)
    assert set(np.unique(a)) <= {-1.0, 1.0} and len(a) == 128
    assert (a != other).any() and (a != reseeded).any()
    np.testing.assert_array_equal(a, O.quant_signs(7, name, 128))
    assert abs(float(exl3.signs(3, "x", 4096).mean())) < 0.1


def test_the_c_abi_refuses_geometry_rate_and_window_before_any_launch():  # quantize.zig:843-860
    from sushi_amd import _lib, exl3

    L = _lib.load()
    mcg12 = exl3.Decode(exl3.Codebook.mcg, exl3.Window(12))
    cases = [((192, 128, 32, mcg12), exl3.BadExl3Shape), ((0, 0, 32, mcg12), exl3.BadExl3Shape),
             ((128, 128, 15, mcg12), exl3.RateUnsupported), ((128, 128, 130, mcg12), exl3.RateUnsupported),
             ((128, 128, 32, exl3.Decode(exl3.Codebook.mcg, exl3.Window(11))), exl3.Exl3WindowUnsupported),
             ((128, 128, 32, exl3.Decode(exl3.Codebook.mcg, exl3.Window(8))), exl3.Exl3WindowUnsupported),
             ((128, 128, 32, exl3.Decode(exl3.Codebook.pair1)), exl3.CodebookUnsupported)]
    for (rows, cols, n, dec), err in cases:
        rc = L.exl3_quantize_tensor(0, 0, rows, cols, 0, 0, n, dec.c(), 0, 0, 0, 0, 0, 0, 0, 0)
        assert rc == err.status, (rows, cols, n, _lib.last_error())
        assert L.exl3_quantize_workspace_size(rows, cols, n, dec.c()) == 0
    assert L.exl3_quantize_tensor(0, 0, 128, 128, 0, 0, 32, mcg12.c(), 3, 0, 0, 0, 0, 0, 0, 0) == exl3.BadExl3Shape.status


# ---- GPU quantizer -----------------------------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("case", TENSOR_CONFIGS, ids=lambda c: c[0])
def test_gpu_whole_tensor_reproduces_the_reference_fixture(dev, fx, case):
    from sushi_amd import exl3

    name, cb, n, w, rows, mode = case
    h = np.ascontiguousarray(fx["H32"][:rows, :rows])
    dec = exl3.Decode(exl3.Codebook(cb), exl3.Window(w))
    packed, suh, svh, g = exl3.quantize_tensor(fx["W32"][:rows], h, fx[f"sign_in_r{rows}"], fx["sign_out"], n, dec,
                                               mode, device=dev)
    np.testing.assert_array_equal(packed.reshape(-1), fx[name + ".packed"].reshape(-1))
    assert abs(g - float(fx[name + ".g"][0])) <= 1e-5
    np.testing.assert_array_equal(suh, fx[name + ".suh"].view(np.uint16))
    np.testing.assert_array_equal(svh, fx[name + ".svh"].view(np.uint16))


def _spd(rng, n, k):
    x = rng.standard_normal((n, k)).astype(np.float32) * 0.1
    h = (x @ x.T).astype(np.float32)
    h[np.arange(n), np.arange(n)] += 0.05
    return h


@pytest.mark.gpu
@pytest.mark.parametrize("cb,n,w,rows,cols,mode", [(O.CB_MCG, 32, 12, 512, 256, "auto"),
                                                   (O.CB_MUL1, 48, 13, 256, 384, "always"),
                                                   (O.CB_3INST, 40, 12, 384, 128, "never")])
def test_gpu_quantizer_is_the_oracle_code_for_code(dev, cb, n, w, rows, cols, mode):
    from sushi_amd import exl3

    rng = np.random.default_rng(rows + cols + n)
    wt = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    h = _spd(rng, rows, 48)
    si, so = exl3.signs(1, "t.in", rows), exl3.signs(1, "t.out", cols)
    want = O.quantize_tensor(wt, h, si, so, n, O.decode(cb, w), mode)
    got = exl3.quantize_tensor(wt, h, si, so, n, exl3.Decode(exl3.Codebook(cb), exl3.Window(w)), mode, device=dev)
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1], want[1])
    np.testing.assert_array_equal(got[2], want[2])
    assert got[3] == want[3]


@pytest.mark.gpu
def test_gpu_same_seed_and_name_quantize_to_the_same_bytes_and_decode_near_the_weight(dev):  # quantize.zig:817-841
    import torch

    from sushi_amd import exl3

    rng = np.random.default_rng(3)
    rows = cols = 128
    wt = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    h = (wt[:, :8] @ wt[:, :8].T).astype(np.float32)
    h[np.arange(rows), np.arange(rows)] += 0.1
    name = "language_model.model.layers.3.mlp.switch_mlp.down_proj"
    dec = exl3.Decode(exl3.Codebook.mcg, exl3.Window(12))
    first = exl3.quantize_named(wt, h, 11, name, 32, dec, "never", device=dev)
    second = exl3.quantize_named(wt, h, 11, name, 32, dec, "never", device=dev)
    for a, b in zip(first[:3], second[:3]):
        np.testing.assert_array_equal(a, b)
    assert first[3] == second[3]
    # The packed tensor decodes (the engine's own dequant) to an approximation of the weight.
    packed, suh, svh, _ = first
    tr = torch.from_numpy(packed.view(np.int16)).reshape(1, rows // 16, cols // 16, 32).to(dev)
    proj = exl3.Proj(tr, torch.from_numpy(suh.view(np.float16)).reshape(1, rows).to(dev),
                     torch.from_numpy(svh.view(np.float16)).reshape(1, cols).to(dev))
    eye = torch.eye(rows, dtype=torch.float16, device=dev)
    dense = exl3.linear(eye, proj, dec).float().cpu().numpy()
    rel = np.linalg.norm(dense - wt) / np.linalg.norm(wt)
    assert rel < 0.5, rel
