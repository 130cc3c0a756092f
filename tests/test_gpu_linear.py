"""GPU parity of the dense trellis linear (GEMV arm for 1..8 rows, MFMA GEMM arm above) against the oracle.

Bar: max |y - y_ref| / max |y_ref| <= 2e-3 with fp16 inputs and fp32 accumulation, where
y_ref is the oracle's `project` (src/exl3/expert_exl3.zig:546-566).  The oracle rounds its inner sum to f16 and the
GPU keeps it in f32, so the two differ by about one f16 ulp of the result; the bar leaves ample room.
"""
import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3

DECODES = {
    "mcg": (exl3.Decode(exl3.Codebook.mcg), O.decode(O.CB_MCG)),
    "mul1": (exl3.Decode(exl3.Codebook.mul1), O.decode(O.CB_MUL1)),
    "3inst": (exl3.Decode(exl3.Codebook.inst3), O.decode(O.CB_3INST)),
    "spec1": (exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    "std1": (exl3.Decode(exl3.Codebook.std1, exl3.Window(15), 3), O.decode(O.CB_STD1, 15, 3)),
    "pair1": (exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1)),
    "mcg_w12": (exl3.Decode(exl3.Codebook.mcg, exl3.Window(12)), O.decode(O.CB_MCG, 12)),
}


def _case(dev, seed, rows, in_f, out_f, n, dtype=torch.float16):
    p = synth.proj(seed, "lin", 1, in_f, out_f, n)
    x = synth.normal(seed, "x", (rows, in_f))
    pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))
    return p, pd, x, x.to(dtype).to(dev)


def _oracle(p, x, in_f, out_f, n, odec):
    return O.project_rows(x.float().numpy(), p.trellis.numpy().view(np.uint16), p.suh.numpy().view(np.uint16),
                          p.svh.numpy().view(np.uint16), in_f, out_f, n, odec, threads=8)


def _run(pd, xd, dec):
    y = exl3.linear(xd, pd, dec)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8, 12, 16])
@pytest.mark.parametrize("n", [16, 24, 32, 40, 48, 64])
def test_gemv_rows_and_rates_mcg(dev, rows, n):
    print(f"[gemv] rows={rows} n={n}", flush=True)
    p, pd, x, xd = _case(dev, 100 + n, rows, 512, 384, n)
    dec, odec = DECODES["mcg"]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, 512, 384, n, odec)) < BAR


@pytest.mark.parametrize("label", list(DECODES))
@pytest.mark.parametrize("n", [32, 48, 64])
def test_gemv_codebooks(dev, label, n):
    print(f"[gemv] {label} n={n}", flush=True)
    p, pd, x, xd = _case(dev, 7, 2, 256, 512, n)
    dec, odec = DECODES[label]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, 256, 512, n, odec)) < BAR


@pytest.mark.parametrize("n,rows", [(18, 3), (22, 3), (44, 3), (58, 3), (66, 3), (96, 3), (128, 3), (22, 12), (66, 16),
                                    (44, 16)])
def test_gemv_generic_rates(dev, n, rows):
    print(f"[gemv] generic n={n} rows={rows}", flush=True)
    p, pd, x, xd = _case(dev, 3, rows, 256, 256, n)
    dec, odec = DECODES["spec1"] if n < 24 or n > 64 else DECODES["pair1"]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, 256, 256, n, odec)) < BAR


@pytest.mark.parametrize("splits,separate,fold", [(1, 0, 1), (2, 0, 1), (2, 0, 0), (4, 1, 1), (8, 0, 1), (8, 0, 0)])
def test_gemv_split_and_finish_arms_agree(dev, splits, separate, fold):
    """Direct finish, the fold (fixed-point accumulation), counters + planes, and the separate finish kernel."""
    print(f"[gemv] splits={splits} separate={separate} fold={fold}", flush=True)
    p, pd, x, xd = _case(dev, 9, 4, 1024, 256, 48)
    dec, odec = DECODES["3inst"]
    want = _oracle(p, x, 1024, 256, 48, odec)
    with exl3.arm_overrides(gemv_splits=splits, gemv_separate_finish=separate, gemv_fold=fold):
        for _ in range(3):  # fused finish counters / accumulators must come back to zero between calls
            assert max_abs_rel(_run(pd, xd, dec), want) < BAR


@pytest.mark.parametrize("rows,per_group", [(6, 0), (7, 0), (8, 0), (11, 0), (13, 0), (16, 0), (16, 4), (15, 4),
                                            (9, 2), (16, 1)])
@pytest.mark.parametrize("splits,separate,fold", [(0, 0, 1), (4, 0, 0), (4, 1, 1)])
@pytest.mark.parametrize("ydt", [torch.float16, torch.float32])
def test_gemv_row_groups_against_oracle(dev, rows, per_group, splits, separate, fold, ydt):
    """A batch of rows run as groups of rows over the one bank (the default from 6 rows, or pinned), the last group
    holding the rest: every row against the oracle to the bar under the fold, the counters + planes finish and the
    separate finish kernel, twice in a row (the accumulators and counters come back to zero); the rows kept whole
    agree with it to the same bar."""
    print(f"[gemv] row groups rows={rows} per_group={per_group} splits={splits} sep={separate} fold={fold} {ydt}",
          flush=True)
    p, pd, x, xd = _case(dev, 21 + rows, rows, 1024, 384, 32)
    dec, odec = DECODES["mcg"]
    want = _oracle(p, x, 1024, 384, 32, odec)
    knobs = dict(gemv_splits=splits, gemv_separate_finish=separate, gemv_fold=fold)
    if per_group:
        knobs["gemv_rows_per_group"] = per_group
    with exl3.arm_overrides(**knobs):
        for _ in range(2):
            y = exl3.linear(xd, pd, dec, out_dtype=ydt)
            torch.cuda.synchronize()
            assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    with exl3.arm_overrides(gemv_rows_per_group=16, **dict(gemv_splits=splits, gemv_separate_finish=separate,
                                                            gemv_fold=fold)):
        whole = exl3.linear(xd, pd, dec, out_dtype=ydt)
        torch.cuda.synchronize()
    assert max_abs_rel(whole.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("fold", [1, 0])
def test_gemv_non_finite_rows(dev, fold):
    """A row whose input holds an inf comes out non-finite in every output under both split finishes (the fold marks
    non-finite contributions and yields NaN); the other rows stay within the bar and the accumulators stay clean."""
    print(f"[gemv] non-finite fold={fold}", flush=True)
    p, pd, x, xd = _case(dev, 11, 3, 1024, 256, 64)
    dec, odec = DECODES["mcg"]
    want = _oracle(p, x, 1024, 256, 64, odec)
    xbad = xd.clone()
    xbad[1, 5] = float("inf")
    with exl3.arm_overrides(gemv_splits=8, gemv_fold=fold):
        y = _run(pd, xbad, dec)
        assert not np.isfinite(y[1]).any()
        assert max_abs_rel(y[[0, 2]], want[[0, 2]]) < BAR
        assert max_abs_rel(_run(pd, xd, dec), want) < BAR  # the next call starts from clean words


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gemm_activation_dtypes_odd_blocks(dev, dtype):
    """The GEMM arm (24 rows) over three 128-blocks of input in bf16 and f32: the prepare's one-block workgroups of
    each input dtype, against the oracle (which rounds its input to f16 as prepareInput does)."""
    p, pd, x, xd = _case(dev, 17, 24, 384, 256, 64, dtype)
    dec, odec = DECODES["mcg"]
    want = _oracle(p, xd.float().cpu(), 384, 256, 64, odec)
    assert max_abs_rel(exl3.linear(xd, pd, dec, out_dtype=torch.float32).cpu().numpy(), want) < BAR


@pytest.mark.parametrize("rows", [2, 12, 24])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_activation_dtypes(dev, dtype, rows):
    p, pd, x, xd = _case(dev, 13, rows, 256, 256, 64, dtype)
    dec, odec = DECODES["mcg"]
    xo = xd.float().cpu()  # the oracle rounds its input to f16 as prepareInput does
    want = _oracle(p, xo, 256, 256, 64, odec)
    y32 = exl3.linear(xd, pd, dec, out_dtype=torch.float32)  # the input dtype's own path, f32 out
    assert max_abs_rel(y32.cpu().numpy(), want) < BAR
    y = exl3.linear(xd, pd, dec)
    assert y.dtype == dtype
    # a bf16 result carries its own rounding (2^-9 relative) on top of the f16 bar
    bar = BAR + (2.0 ** -8 if dtype == torch.bfloat16 else 0.0)
    assert max_abs_rel(y.float().cpu().numpy(), want) < bar


def test_arms_share_one_workspace(dev):
    """GEMM and MoE scratch never lands on the GEMV's fused-finish counters: interleave the arms on one workspace."""
    p, pd, x, xd = _case(dev, 17, 40, 1024, 1024, 64)
    dec, odec = DECODES["mcg"]
    want = _oracle(p, x, 1024, 1024, 64, odec)
    for _ in range(3):
        assert max_abs_rel(_run(pd, xd, dec), want) < BAR                      # GEMM arm (40 rows)
        assert max_abs_rel(_run(pd, xd[:3].contiguous(), dec), want[:3]) < BAR  # GEMV arm, fused finish


def test_fused_finish_repeated_across_shapes(dev):
    """The single-launch finish (arrival counters, partials in the XCD's L2 or written through) stays correct over
    back-to-back calls on one workspace, across shapes whose output groups map to different XCDs."""
    cases = []
    for seed, in_f, out_f in ((31, 4096, 4096), (32, 2048, 3584), (33, 1024, 384)):
        p, pd, x, xd = _case(dev, seed, 1, in_f, out_f, 64)
        cases.append((pd, xd, _oracle(p, x, in_f, out_f, 64, DECODES["mcg"][1])))
    for _ in range(3):
        for pd, xd, want in cases:
            exl3.linear(xd, pd, DECODES["mcg"][0])  # queued back to back, no host sync in between
        for pd, xd, want in cases:
            assert max_abs_rel(_run(pd, xd, DECODES["mcg"][0]), want) < BAR


def test_linear_grouped(dev):
    g, rows, in_f, out_f, n = 3, 2, 256, 384, 32
    p = synth.proj(21, "grp", g, in_f, out_f, n)
    x = synth.normal(21, "x", (g, rows, in_f))
    pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))
    y = exl3.linear_grouped(x.to(dev), pd, exl3.MCG).float().cpu().numpy()
    for b in range(g):
        want = O.project_rows(x[b].float().numpy(), p.trellis[b].numpy().view(np.uint16),
                              p.suh[b].numpy().view(np.uint16), p.svh[b].numpy().view(np.uint16), in_f, out_f, n,
                              O.decode(O.CB_MCG), threads=8)
        assert max_abs_rel(y[b], want) < BAR


@pytest.mark.parametrize("rows", [17, 33, 130])
@pytest.mark.parametrize("n", [32, 48, 64, 40])
def test_gemm_arm(dev, rows, n):
    print(f"[gemm] rows={rows} n={n}", flush=True)
    p, pd, x, xd = _case(dev, 40 + rows, rows, 512, 256, n)
    dec, odec = DECODES["3inst"]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, 512, 256, n, odec)) < BAR


@pytest.mark.parametrize("in_f,rows", [(128, 20), (384, 40), (640, 300)])
def test_gemm_odd_k_steps_and_row_tails(dev, in_f, rows):
    """k spans of 1, 3 and 5 GEMM k-steps (the unrolled step pair plus a tail step) and row counts that leave a
    partial 256-row tile."""
    p, pd, x, xd = _case(dev, 60 + in_f, rows, in_f, 256, 48)
    dec, odec = DECODES["3inst"]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, in_f, 256, 48, odec)) < BAR


@pytest.mark.parametrize("label", ["spec1", "pair1", "mul1"])
def test_gemm_codebooks(dev, label):
    p, pd, x, xd = _case(dev, 77, 24, 256, 256, 48)
    dec, odec = DECODES[label]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, 256, 256, 48, odec)) < BAR


def test_gemm_rows_equal_gemv_rows(dev):
    """Byte-exactness is not claimed between arms, but the two arms agree to the bar on the same rows."""
    p, pd, x, xd = _case(dev, 5, 24, 512, 512, 64)
    dec = DECODES["mcg"][0]
    wide = _run(pd, xd, dec)
    narrow = np.concatenate([_run(pd, xd[i:i + 4].contiguous(), dec) for i in range(0, 24, 4)])
    assert max_abs_rel(wide, narrow) < BAR


@pytest.mark.parametrize("rows", [1, 16, 24])
def test_c1_full_size_3inst_k4(dev, rows):
    """Config 1's shape at full size: 4096 x 4096, K4, 3INST, against the oracle."""
    print(f"[c1] rows={rows}", flush=True)
    p, pd, x, xd = _case(dev, 0, rows, 4096, 4096, 64)
    dec, odec = DECODES["3inst"]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, 4096, 4096, 64, odec)) < BAR


@pytest.mark.parametrize("in_f,out_f,n", [(4096, 14336, 32), (14336, 4096, 48), (2048, 2048, 64)])
def test_c2_shapes_mcg(dev, in_f, out_f, n):
    print(f"[c2] {in_f}x{out_f} n={n}", flush=True)
    p, pd, x, xd = _case(dev, 1, 4, in_f, out_f, n)
    dec, odec = DECODES["mcg"]
    assert max_abs_rel(_run(pd, xd, dec), _oracle(p, x, in_f, out_f, n, odec)) < BAR


def _big_case(dev, seed, rows, in_f, out_f, n, svh_scale, x_scale):
    """Outputs far past the fold's fixed-point range: svh times svh_scale (still f16), x times x_scale; the exact
    f64 truth of the f16 inputs."""
    from tests import _parity as P

    p = synth.proj(seed, "big", 1, in_f, out_f, n)
    svh = (p.svh.float() * svh_scale).half()
    x = (synth.normal(seed, "xbig", (rows, in_f)).float() * x_scale).half()
    pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), svh.to(dev))
    pr = P.prepared_rows(x.float().numpy(), p.suh.numpy().view(np.uint16)[0])
    w = P.decoded(p.trellis.numpy().view(np.uint16)[0], in_f, out_f, n, DECODES["3inst"][1])
    y64 = P.f16_bits(svh.numpy().view(np.uint16)[0]) * P.hadamard_blocks(pr @ w)
    return pd, x.to(dev), y64


@pytest.mark.parametrize("splits", [8, 16])
@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16, torch.float32])
def test_outputs_past_the_fold_range(dev, ydt, splits):
    """Split partials past 2^21 (the fold's fixed-point range) take its f64 overflow words: bf16 and f32 outputs of
    ~10^7 come out finite and within the bar of the exact value, and f16 outputs past 65504 come out +-inf with the
    exact value's sign (never NaN); the words are clean for the next call."""
    print(f"[gemv] big outputs {ydt} splits={splits}", flush=True)
    pd, xd, y64 = _big_case(dev, 23, 2, 4096, 1024, 64, 1024.0, 128.0)
    assert np.abs(y64).max() > 2.0 ** 23
    dec = DECODES["3inst"][0]
    with exl3.arm_overrides(gemv_splits=splits):
        for _ in range(2):
            y = exl3.linear(xd, pd, dec, out_dtype=ydt).float().cpu().numpy().astype(np.float64)
            if ydt == torch.float16:
                over = np.abs(y64) > 65520.0 * 1.002
                under = np.abs(y64) < 65504.0 * 0.998
                assert over.any() and under.any()
                assert np.isinf(y[over]).all() and (np.sign(y[over]) == np.sign(y64[over])).all()
                assert np.isfinite(y[under]).all()
                # the north-star metric: error over the largest exact output (the finite outputs here are
                # cancellations of partials near 10^7, so one f16 ulp of a prepared input moves them by hundreds)
                assert np.max(np.abs(y[under] - y64[under])) / np.abs(y64).max() < BAR
            else:
                bar = BAR + (2.0 ** -8 if ydt == torch.bfloat16 else 0.0)
                assert max_abs_rel(y, y64) < bar
    # the overflow and fold words are back at zero: an ordinary call on the same workspace is exact
    p, pd2, x, xd2 = _case(dev, 11, 3, 1024, 256, 64)
    with exl3.arm_overrides(gemv_splits=8):
        assert max_abs_rel(_run(pd2, xd2, DECODES["mcg"][0]), _oracle(p, x, 1024, 256, 64, DECODES["mcg"][1])) < BAR
