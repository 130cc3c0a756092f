"""GPU parity on the summand-relative bar (tests/_parity.py), with the reference's mutation arms and seed sweep.

Every arm runs with f32 outputs; its finish is undone exactly and each inner element is held to the f64 dot product
of the oracle's decoded weights, relative to that element's summand scale (src/exl3/expert_exl3_kernels.zig:
3310-3330).  Each case then checks that the same bar FAILS when the truth reads the wrong codeword window or one
flipped trellis bit (:3330-3352), so a decode defect that touches a single weight cannot pass.  The headline shapes
sweep PARITY_SEEDS = 8 seeds (:4550).  The north-star bar (max-abs-rel 2e-3 of the f16 output) is in
test_gpu_linear.py / test_gpu_moe.py; this bar is the stricter one.
"""
import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import _lib, exl3, synth
from tests import _parity as P

pytestmark = pytest.mark.gpu

DECODES = {
    "mcg": (exl3.Decode(exl3.Codebook.mcg), O.decode(O.CB_MCG)),
    "mul1": (exl3.Decode(exl3.Codebook.mul1), O.decode(O.CB_MUL1)),
    "3inst": (exl3.Decode(exl3.Codebook.inst3), O.decode(O.CB_3INST)),
    "spec1": (exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    "std1": (exl3.Decode(exl3.Codebook.std1, exl3.Window(15), 3), O.decode(O.CB_STD1, 15, 3)),
    "pair1": (exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1)),
    "mcg_w12": (exl3.Decode(exl3.Codebook.mcg, exl3.Window(12)), O.decode(O.CB_MCG, 12)),
}


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


class Dense:
    """One seeded dense projection [in, out] at rate n and `rows` input rows, on the device and as oracle inputs."""

    def __init__(self, dev, seed, rows, in_f, out_f, n):
        self.in_f, self.out_f, self.n = in_f, out_f, n
        p = synth.proj(seed, f"par{in_f}x{out_f}.{n}", 1, in_f, out_f, n)
        self.x = synth.normal(seed, f"par.x{rows}.{in_f}", (rows, in_f))
        self.t, self.suh, self.svh = _u16(p.trellis)[0], _u16(p.suh)[0], _u16(p.svh)[0]
        self.pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))
        self.xd = self.x.to(dev)
        self.p = P.prepared_rows(self.x.float().numpy(), self.suh)

    def inner(self, dec) -> np.ndarray:
        y = exl3.linear(self.xd, self.pd, dec, out_dtype=torch.float32)
        torch.cuda.synchronize()
        return P.inner_from_output(y.cpu().numpy(), self.svh)

    def truth(self, odec) -> P.Truth:
        return P.truth(self.p, P.decoded(self.t, self.in_f, self.out_f, self.n, odec))


def _hold(got: np.ndarray, d: Dense, odec, seed: int, mutate: bool = True, what: str = "") -> None:
    """The arm passes the bar; with `mutate`, the same output fails it against the window and flipped-bit mutants."""
    t = d.truth(odec)
    print(f"[parity] {what} worst error / ceiling = {P.worst_ratio(got, t):.4f}", flush=True)
    why = P.verdict(got, t)
    assert why is None, f"{what}: {why}"
    if not mutate:
        return
    tw = P.with_inner(t, d.p @ P.decoded(d.t, d.in_f, d.out_f, d.n, P.mutated_window(odec)))
    assert P.verdict(got, tw) is not None, f"{what}: the window mutation passed the bar"
    tb, where = P.flipped_truth(t, d.p, d.t, d.n, odec, np.random.default_rng(seed))
    assert P.verdict(got, tb) is not None, f"{what}: the flipped bit {where} passed the bar"


# ---- decode GEMV (1..16 rows) -------------------------------------------------------------------------------------


@pytest.mark.parametrize("rows", [1, 4, 16])
@pytest.mark.parametrize("n", [32, 48, 64])
@pytest.mark.parametrize("label", list(DECODES))
def test_gemv_codebooks_rates_rows(dev, label, n, rows):
    d = Dense(dev, 300 + n + rows, rows, 512, 384, n)
    dec, odec = DECODES[label]
    _hold(d.inner(dec), d, odec, seed=n + rows, what=f"gemv {label} n={n} rows={rows}")


@pytest.mark.parametrize("n,label", [(16, "spec1"), (24, "pair1"), (40, "3inst"), (22, "spec1"), (44, "pair1"),
                                     (96, "spec1"), (128, "spec1")])
def test_gemv_other_rates(dev, n, label):
    """n = 16, 24, 40 on the lane reader; 22, 44, 96, 128 on the generic reader."""
    d = Dense(dev, 400 + n, 3, 256, 256, n)
    dec, odec = DECODES[label]
    _hold(d.inner(dec), d, odec, seed=n, what=f"gemv {label} n={n}")


@pytest.mark.parametrize("splits,separate", [(1, 0), (2, 0), (4, 1), (8, 0)])
def test_gemv_split_arms(dev, splits, separate):
    """Direct finish, counters + planes, and the separate finish kernel (an f32 output never takes the fold)."""
    d = Dense(dev, 17, 4, 1024, 256, 48)
    dec, odec = DECODES["3inst"]
    with exl3.arm_overrides(gemv_splits=splits, gemv_separate_finish=separate):
        for _ in range(2):
            _hold(d.inner(dec), d, odec, seed=splits, mutate=False, what=f"split {splits} separate {separate}")


@pytest.mark.parametrize("seed", range(P.PARITY_SEEDS))
def test_c1_headline_shape_every_seed(dev, seed):
    """configs[0]'s shape as bench.py runs it: 4096 x 4096, K4 (n64), 3INST, batch 1."""
    d = Dense(dev, seed, 1, 4096, 4096, 64)
    dec, odec = DECODES["3inst"]
    _hold(d.inner(dec), d, odec, seed=seed, what=f"c1 seed {seed}")


def _f16_ulp(v: np.ndarray) -> np.ndarray:
    """The spacing of f16 values at |v| (2^-24 in the subnormal range)."""
    a = np.abs(np.asarray(v, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -14))) - 10)


def _butterfly_prepared(x_row: np.ndarray, suh_bits: np.ndarray) -> np.ndarray:
    """prepareInput f16(H128(f16(x) * suh)) (expert_exl3.zig:490-501) with the Hadamard as the GPU prologue forms it:
    f32 butterflies over index bits 6, 5, ..., 0 (each a + b and a - b rounded once), then times f32(1/sqrt(128)),
    then f16.  The reference's CPU path sums the dense O(128^2) Hadamard in another order, so a few elements round
    to the neighbouring f16 (the summand bar's PREP_ULPS term allows for that); here the fold's own rounding is under
    test, so the truth takes the prepared input the kernel multiplies with."""
    v = (np.asarray(x_row, np.float16).astype(np.float32) * P.f16_bits(suh_bits).astype(np.float32)).reshape(-1, 128)
    for h in (64, 32, 16, 8, 4, 2, 1):
        w = v.reshape(v.shape[0], 128 // (2 * h), 2, h)
        a, b = w[:, :, 0, :], w[:, :, 1, :]
        v = np.stack([a + b, a - b], axis=2).reshape(-1, 128)
    return (v.reshape(-1) * np.float32(0.08838834764831845)).astype(np.float16).astype(np.float64)


def _fold_truth(d: "Dense", w: np.ndarray, p: np.ndarray, splits: int):
    """y = svh * H(p w) in f64 (finishOutput, expert_exl3.zig:534-544) and each output's allowance beyond one f16 ulp:
    the f32 accumulation of the inner sums (ACC_FACTOR sqrt(depth) 2^-24 of the largest inner magnitude of the block,
    the summand bar's factor) and the fold's fixed point (half of 2^-24 per split term)."""
    sv = P.f16_bits(d.svh)
    inner = p[None] @ w
    y = sv * P.hadamard_blocks(inner)[0]
    blockmax = np.repeat(np.abs(inner[0]).reshape(-1, 128).max(axis=1), 128)
    return y, np.abs(sv) * P.ACC_FACTOR * np.sqrt(d.in_f) * P.U_F32 * blockmax + splits * 2.0 ** -25


def _within_one_ulp(got: np.ndarray, y: np.ndarray, allow: np.ndarray):
    """(passes, exact fraction, worst excess): every f16 output within one f16 ulp of round_f16(truth) plus its
    allowance."""
    want = y.astype(np.float16).astype(np.float64)
    err = np.abs(np.asarray(got, np.float64).reshape(-1) - want)
    lim = _f16_ulp(want) + allow
    return bool((err <= lim).all()), float(np.mean(err == 0)), float(np.max(err / lim))


@pytest.mark.parametrize("label,seed", [("3inst", s) for s in range(P.PARITY_SEEDS)] + [("mcg", 0), ("mcg", 1)])
def test_c1_fold_arm_every_output_within_one_f16_ulp(dev, label, seed):
    """The arm bench.py times: configs[0]'s 4096 x 4096 K4 at batch 1 with an f16 output, which takes the fixed-point
    fold over 8 splits (f32 outputs take the counters + planes arm, so the summand bar above never reaches it).  Every
    f16 output must sit within one f16 ulp of round_f16 of the f64 truth built from the oracle's decoded weights
    (src/exl3/expert_exl3_kernels.zig:3300-3352's standard, held per element; the allowance is a small fraction of an
    ulp except where outputs cancel to near zero); the same outputs must fail that bar against the wrong codeword
    window and against one flipped trellis bit.  3INST over PARITY_SEEDS seeds; MCG (the reference-pinned codebook of
    the bench line's twin) over two."""
    print(f"[parity] c1 fold arm {label} seed {seed}", flush=True)
    d = Dense(dev, seed, 1, 4096, 4096, 64)
    dec, odec = DECODES[label]
    got = exl3.linear(d.xd, d.pd, dec).float().cpu().numpy().astype(np.float64)  # f16 output: the fold arm
    p = _butterfly_prepared(d.x.numpy()[0], d.suh)
    # the same values as the oracle's prepareInput up to the two transforms' f32 error: a neighbouring f16, or, where
    # the block's inputs cancel to near zero, a few f32 roundings of the block's magnitude
    moved = np.nonzero(p != d.p[0])[0]
    tol = _f16_ulp(d.p[0][moved]) + 64 * P.U_F32 * np.abs(d.p[0]).max()
    assert moved.size <= 32 and (np.abs(p - d.p[0])[moved] <= tol).all(), moved
    w = P.decoded(d.t, d.in_f, d.out_f, d.n, odec)
    y, allow = _fold_truth(d, w, p, splits=8)
    ok, exact, worst = _within_one_ulp(got, y, allow)
    frac = float(np.median(allow / _f16_ulp(y.astype(np.float16).astype(np.float64))))
    print(f"[parity] c1 fold {label} seed {seed}: prepared input off the oracle's at {moved.size}, median allowance "
          f"{frac:.4f} ulp, exact {exact:.5f}, worst error / (ulp + allowance) {worst:.3f}", flush=True)
    assert ok, f"worst error / (ulp + allowance) = {worst:.3f}"
    assert exact > 0.99
    ww = P.decoded(d.t, d.in_f, d.out_f, d.n, P.mutated_window(odec))
    assert not _within_one_ulp(got, _fold_truth(d, ww, p, 8)[0], allow)[0]
    t = P.truth(p[None], w)
    tb, where = P.flipped_truth(t, p[None], d.t, d.n, odec, np.random.default_rng(seed))
    yb = P.f16_bits(d.svh) * P.hadamard_blocks(tb.inner)[0]
    assert not _within_one_ulp(got, yb, allow)[0], where


@pytest.mark.parametrize("rows", [1, 4, 16])
@pytest.mark.parametrize("n", [32, 48, 64])
@pytest.mark.parametrize("in_f,out_f", [(2048, 2048), (4096, 14336), (14336, 4096)])
def test_c2_shapes(dev, in_f, out_f, n, rows):
    """configs[1] at full size: MCG, K = 2/3/4, batch 1/4/16."""
    d = Dense(dev, 1, rows, in_f, out_f, n)
    dec, odec = DECODES["mcg"]
    _hold(d.inner(dec), d, odec, seed=rows, mutate=in_f == out_f, what=f"c2 {in_f}x{out_f} n={n} rows={rows}")


# ---- GEMM arm (rows > 16) -----------------------------------------------------------------------------------------


@pytest.mark.parametrize("rows", [17, 40, 130, 300])
@pytest.mark.parametrize("n", [32, 40, 48, 64])
def test_gemm_rates_rows(dev, n, rows):
    d = Dense(dev, 500 + rows, rows, 1024, 512, n)
    dec, odec = DECODES["3inst"]
    _hold(d.inner(dec), d, odec, seed=rows, what=f"gemm n={n} rows={rows}")


@pytest.mark.parametrize("rows", [40, 300])
def test_gemm_odd_block_count(dev, rows):
    """An input width of three 128-blocks: the prepare's one-block workgroups (two where the blocks pair up) and the
    tiles' k range, to the bar with its mutation arms."""
    d = Dense(dev, 610 + rows, rows, 384, 256, 32)
    dec, odec = DECODES["3inst"]
    _hold(d.inner(dec), d, odec, seed=rows, what=f"gemm in=384 rows={rows}")


@pytest.mark.parametrize("label", ["mcg", "mul1", "spec1", "std1", "pair1", "mcg_w12"])
def test_gemm_codebooks(dev, label):
    d = Dense(dev, 77, 24, 512, 256, 48)
    dec, odec = DECODES[label]
    _hold(d.inner(dec), d, odec, seed=5, what=f"gemm {label}")


@pytest.mark.parametrize("seed", range(P.PARITY_SEEDS))
def test_gemm_every_seed(dev, seed):
    d = Dense(dev, 900 + seed, 64, 2048, 1024, 48)
    dec, odec = DECODES["3inst"]
    _hold(d.inner(dec), d, odec, seed=seed, what=f"gemm seed {seed}")


@pytest.mark.parametrize("rows,out_f", [(512, 14336), (2048, 1024), (2048, 14336)])
def test_c3_prefill_shapes(dev, rows, out_f):
    """4096 x 14336, K3, 3INST at M = 512 (row tiles 2: the XCD remap with 4 output groups per XCD
    round) and M = 2048 (row tiles 8: one output group per XCD round), and M = 2048 at out 1024 (the same branch on a
    grid of one round)."""
    d = Dense(dev, 3, rows, 4096, out_f, 48)
    dec, odec = DECODES["3inst"]
    _hold(d.inner(dec), d, odec, seed=rows, mutate=out_f == 1024, what=f"c3 M={rows} out={out_f}")


# ---- ping-pong GEMM body (gemm_arm 5 / 6: 512- / 256-row tiles, every wave decoding half a k-tile row and running
# the MFMAs of its own rows; 7: the 512-row tile with k in two halves whose partials meet through the workspace),
# forced at small shapes; the row-count policy takes arm 5 past 512 rows


@pytest.mark.parametrize("arm", [5, 6, 7])
@pytest.mark.parametrize("n", [16, 24, 32, 40, 48, 64])
def test_gemm_pingpong_rates(dev, arm, n):
    d = Dense(dev, 700 + n, 300, 1024, 512, n)
    dec, odec = DECODES["3inst"]
    with exl3.arm_overrides(gemm_arm=arm):
        got = d.inner(dec)
    _hold(got, d, odec, seed=n, what=f"pingpong arm={arm} n={n}")


@pytest.mark.parametrize("arm", [5, 6, 7])
@pytest.mark.parametrize("rows", [17, 257, 700])
def test_gemm_pingpong_row_tails(dev, arm, rows):
    """Row counts that leave partial 16-row blocks, partial waves and a partial last tile (k spans of 2, 6 and 10
    steps: the three-slot words ring ends on every phase)."""
    in_f = {17: 128, 257: 384, 700: 640}[rows]
    d = Dense(dev, 710 + rows, rows, in_f, 256, 48)
    dec, odec = DECODES["3inst"]
    with exl3.arm_overrides(gemm_arm=arm):
        got = d.inner(dec)
    _hold(got, d, odec, seed=rows, what=f"pingpong arm={arm} rows={rows} in={in_f}")


@pytest.mark.parametrize("label", ["mcg", "spec1", "std1", "mcg_w12", "pair1", "mul1"])
def test_gemm_pingpong_codebooks(dev, label):
    """Hash-product families take the ping-pong body; PAIR1 and MUL1 fall back to the decode-wave tile."""
    d = Dense(dev, 720, 300, 512, 256, 48)
    dec, odec = DECODES[label]
    with exl3.arm_overrides(gemm_arm=5):
        got = d.inner(dec)
    _hold(got, d, odec, seed=7, what=f"pingpong {label}")


@pytest.mark.parametrize("label", ["mcg", "3inst", "spec1", "std1", "mcg_w12"])
@pytest.mark.parametrize("n", [16, 24, 32, 40, 48, 64])
def test_gemm_pingpong_half_decoder_is_bit_exact(dev, label, n):
    """The ping-pong body decodes through the half-chunk reader; the decode-wave tile through the lane reader that
    test_gpu_decode.py pins bit for bit.  Both accumulate every output in the same k order, so equal outputs on a
    matrix of 32 x 32 tiles show every weight of the half reader equal to the lane reader's."""
    table = {"spec1": 1, "std1": 3}.get(label)
    if table is not None and O.table_row(table, n) is None:
        pytest.skip(f"{label} has no row at n={n}")
    d = Dense(dev, 730 + n, 300, 512, 512, n)
    dec = DECODES[label][0]
    outs = {}
    for arm in (4, 6):
        with exl3.arm_overrides(gemm_arm=arm):
            outs[arm] = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32)
    if n != 40:
        with exl3.arm_overrides(gemm_arm=5):
            outs[5] = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32)
    torch.cuda.synchronize()
    for arm, y in outs.items():
        assert torch.equal(y, outs[4]), f"arm {arm} differs from the decode-wave tile ({label} n={n})"


def test_gemm_ksplit_repeats_and_groups(dev):
    """Arm 7 leaves its tile counters at zero: the same call twice gives the same output bit for bit (the two halves
    meet in a sum of two, whichever arrives last), GEMV calls that share the zeroed region run between them, and a
    grouped call (two weight groups, their own counters) holds the bar per group."""
    d = Dense(dev, 740, 640, 1024, 768, 48)
    dec, odec = DECODES["3inst"]
    with exl3.arm_overrides(gemm_arm=7):
        y1 = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32)
        g = Dense(dev, 741, 3, 1024, 768, 48)
        exl3.linear(g.xd, g.pd, dec)
        y2 = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32)
        exl3.linear(g.xd, g.pd, dec)
        y3 = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    with exl3.arm_overrides(gemm_arm=7):
        got = d.inner(dec)
    _hold(got, d, odec, seed=11, what="ksplit repeat")
    groups, rows, in_f, out_f, n = 2, 40, 512, 384, 48
    p = synth.proj(742, "ksg", groups, in_f, out_f, n)
    x = synth.normal(742, "ksg.x", (groups, rows, in_f))
    pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))
    with exl3.arm_overrides(gemm_arm=7):
        y = exl3.linear_grouped(x.float().to(dev), pd, dec)  # f32 x: f32 outputs (rounded to f16 on input alike)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    for b in range(groups):
        t = P.truth(P.prepared_rows(x[b].float().numpy(), _u16(p.suh)[b]),
                    P.decoded(_u16(p.trellis)[b], in_f, out_f, n, odec))
        why = P.verdict(P.inner_from_output(y[b], _u16(p.svh)[b]), t)
        assert why is None, f"ksplit group {b}: {why}"


def test_gemm_ksplit_shared_finish_and_handover_agree(dev):
    """Arm 7 finishes a tile one of two ways: each half finishes its own rows after a bounded wait for the other, or
    the first half to arrive hands the whole tile to the second (a zero wait forces that).  Both give the same outputs
    bit for bit (every output is the same sum of two), call after call, and hold the bar; a row tile with a short
    tail (640 rows: 512 + 128) is included."""
    print("[ksplit finish] rows=640 in=1024 out=768 n=48", flush=True)
    d = Dense(dev, 743, 640, 1024, 768, 48)
    dec, odec = DECODES["3inst"]
    outs = {}
    for wait in (None, 0, 1_000_000):  # the library's choice, never wait, wait up to 10 ms
        knobs = {"gemm_arm": 7} if wait is None else {"gemm_arm": 7, "gemm_split_wait": wait}
        with exl3.arm_overrides(**knobs):
            ys = [exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32) for _ in range(3)]
        torch.cuda.synchronize()
        assert all(torch.equal(y, ys[0]) for y in ys[1:]), f"wait {wait}: repeated calls differ"
        outs[wait] = ys[0]
    assert torch.equal(outs[0], outs[None]) and torch.equal(outs[1_000_000], outs[None])
    with exl3.arm_overrides(gemm_arm=7, gemm_split_wait=0):
        got = d.inner(dec)
    _hold(got, d, odec, seed=12, what="ksplit handover")


@pytest.mark.parametrize("arm", [4, 5, 6, 7])
def test_gemm_16bit_outputs_round_the_f32_outputs(dev, arm):
    """The GEMM bodies round each f32 output once to y's 16-bit dtype (the ping-pong tile stages 16-bit rows through
    LDS for wide stores): f16 and bf16 outputs equal the f32 outputs rounded, rows past a 16-row block included; and a
    y that is not 16-byte aligned (an offset view, through the C ABI) takes the lane-layout stores with the same
    result."""
    d = Dense(dev, 750 + arm, 300, 512, 384, 48)
    dec = DECODES["3inst"][0]
    with exl3.arm_overrides(gemm_arm=arm):
        y32 = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float32)
        y16 = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.float16)
        yb = exl3.linear(d.xd, d.pd, dec, out_dtype=torch.bfloat16)
        rows, out_f = d.xd.shape[0], d.out_f
        buf = torch.zeros(rows * out_f + 1, dtype=torch.float16, device=dev)
        yo = buf[1:].view(rows, out_f)  # 2 bytes past a 256-byte boundary
        L = _lib.load()
        ws = exl3.workspace.get(d.xd.device, L.exl3_linear_workspace_size(rows, d.in_f, out_f, d.n))
        f16 = exl3._dt(y16, "y")
        rc = L.exl3_linear(d.xd.data_ptr(), exl3._dt(d.xd, "x"), rows, d.in_f, out_f, d.pd.trellis.data_ptr(), d.n,
                           d.pd.suh.data_ptr(), d.pd.svh.data_ptr(), dec.c(), yo.data_ptr(), f16, ws.data_ptr(),
                           ws.numel(), exl3._stream(dev))
        assert rc == 0, rc
    torch.cuda.synchronize()
    assert torch.equal(y16, y32.half()), f"arm {arm}: f16 outputs differ from the rounded f32 outputs"
    assert torch.equal(yb, y32.bfloat16()), f"arm {arm}: bf16 outputs differ from the rounded f32 outputs"
    assert torch.equal(yo, y16), f"arm {arm}: the unaligned output differs"


def test_gemm_pingpong_equals_decode_wave_tile_at_c3(dev):
    """At C3's shape (4096 x 14336, K3, 3INST, 1024 rows) the two GEMM bodies accumulate every output in the same k
    order, so their outputs are identical bit for bit."""
    torch.manual_seed(0)
    p = synth.proj(3, "c3eq", 1, 4096, 14336, 48)
    pd = exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))
    x = synth.normal(3, "c3eq.x", (1024, 4096)).to(dev)
    dec = DECODES["3inst"][0]
    outs = {}
    for arm in (4, 5, 6):
        with exl3.arm_overrides(gemm_arm=arm):
            outs[arm] = exl3.linear(x, pd, dec, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(outs[4], outs[5]) and torch.equal(outs[4], outs[6])


# ---- routed experts -------------------------------------------------------------------------------------------------
#
# The routed layer sums its slots with per-expert svh, which no single inverse undoes; so these cases route every
# slot of a row to ONE expert (topk = 1, or topk copies of it with scores summing to 1), where
# y = (sum of scores) * svh_down[e] * H(inner_down) is undone exactly.  The routed decode, the per-slot and sorted
# arms, the mid and the slot reduce all run as usual.


def _moe_truth(bank, x, experts_of_row, odecs, clamp=0.0):
    """Exact down inner products of each row's expert, the chain's rounding points (tests/_parity.down_prepared)."""
    hidden = x.shape[1]
    g, u, dn = bank.gate, bank.up, bank.down
    inter = g.out_features
    ng, nu, nd = g.n, u.n, dn.n
    cache = {}
    rows_p, rows_w = [], []
    for r, e in enumerate(experts_of_row):
        if e not in cache:
            wg = P.decoded(_u16(g.trellis)[e], hidden, inter, ng, odecs[0])
            wu = P.decoded(_u16(u.trellis)[e], hidden, inter, nu, odecs[1])
            wd = P.decoded(_u16(dn.trellis)[e], inter, hidden, nd, odecs[2])
            cache[e] = (wg, wu, wd)
        wg, wu, wd = cache[e]
        pg = P.prepared_rows(x[r:r + 1], _u16(g.suh)[e])
        pu = P.prepared_rows(x[r:r + 1], _u16(u.suh)[e])
        gv = P.f16_bits(_u16(g.svh)[e]) * P.hadamard_blocks(pg @ wg)
        uv = P.f16_bits(_u16(u.svh)[e]) * P.hadamard_blocks(pu @ wu)
        pd = P.down_prepared(gv, uv, _u16(dn.suh)[e], clamp)
        rows_p.append(pd[0])
        rows_w.append(wd)
    inner = np.stack([p @ w for p, w in zip(rows_p, rows_w)])
    amag = np.stack([np.abs(p) @ np.abs(w) for p, w in zip(rows_p, rows_w)])
    bound = np.stack([np.abs(p).max() * np.abs(w).max(axis=0) for p, w in zip(rows_p, rows_w)])
    return P.Truth(inner, amag, bound, inter, P.MID_ULPS)


def _moe_inner(y, bank, experts_of_row, score_sum):
    svh = _u16(bank.down.svh)
    return np.stack([P.inner_from_output(y[r] / score_sum[r], svh[e]) for r, e in enumerate(experts_of_row)])


def _moe_case(dev, seed, rows, topk, E=32, hidden=512, inter=256, n=32):
    b = synth.bank(seed, f"pmoe{E}.{n}", E, hidden, inter, n)
    bd = exl3.Bank(*(exl3.Proj(q.trellis.to(dev), q.suh.to(dev), q.svh.to(dev)) for q in (b.gate, b.up, b.down)))
    x = synth.normal(seed, f"pmoe.x{rows}", (rows, hidden))
    rng = np.random.default_rng(seed)
    experts = rng.integers(0, E, size=rows)
    inds = np.repeat(experts[:, None], topk, axis=1).astype(np.int32)
    sc = rng.uniform(0.5, 1.5, size=(rows, topk)).astype(np.float32)
    sc /= sc.sum(axis=1, keepdims=True)
    score_sum = sc.sum(axis=1, dtype=np.float64)[:, None]
    return b, bd, x, experts, torch.from_numpy(inds).to(dev), torch.from_numpy(sc).to(dev), score_sum


@pytest.mark.parametrize("rows", [1, 5, 12, 40])
@pytest.mark.parametrize("topk", [1, 4])
def test_moe_chain_per_slot_and_sorted_arms(dev, rows, topk):
    """Up to 8 rows the per-slot arm, above it the expert windows; the planes + reduce finish (f32 output)."""
    b, bd, x, experts, inds, sc, ssum = _moe_case(dev, 60 + rows, rows, topk)
    odec = O.decode(O.CB_MCG)
    y = exl3.moe(x.to(dev).float(), bd, inds, sc, exl3.MCG)
    torch.cuda.synchronize()
    got = _moe_inner(y.cpu().numpy().astype(np.float64), b, experts, ssum)
    xf = x.float().numpy()
    t = _moe_truth(b, xf, experts, (odec, odec, odec))
    print(f"[parity] moe rows={rows} topk={topk} worst error / ceiling = {P.worst_ratio(got, t):.4f}", flush=True)
    assert P.verdict(got, t) is None, P.verdict(got, t)
    # mutations: the truth reads w15, or one flipped bit in the down bank / the gate bank of row 0's expert
    w15 = P.mutated_window(odec)
    assert P.verdict(got, _moe_truth(b, xf, experts, (w15, w15, w15))) is not None
    e0 = int(experts[0])
    for proj in ("down", "gate"):
        q = getattr(b, proj)
        tr = _u16(q.trellis).copy()
        pin = P.prepared_rows(xf[:1], _u16(b.gate.suh)[e0]) if proj == "gate" else np.ones((1, q.in_features))
        tr[e0], where = P.flip_one_bit(tr[e0], q.n, odec, pin, np.random.default_rng(rows + topk))
        mb = exl3.Bank(b.gate, b.up, b.down)
        setattr(mb, proj, exl3.Proj(torch.from_numpy(tr.view(np.int16)), q.suh, q.svh))
        assert P.verdict(got, _moe_truth(mb, xf, experts, (odec, odec, odec))) is not None, (proj, where)


@pytest.mark.parametrize("seed", range(P.PARITY_SEEDS))
def test_moe_every_seed(dev, seed):
    b, bd, x, experts, inds, sc, ssum = _moe_case(dev, 700 + seed, 6, 1, E=64, hidden=1024, inter=512, n=32)
    odec = O.decode(O.CB_MCG)
    y = exl3.moe(x.to(dev).float(), bd, inds, sc, exl3.MCG)
    torch.cuda.synchronize()
    got = _moe_inner(y.cpu().numpy().astype(np.float64), b, experts, ssum)
    t = _moe_truth(b, x.float().numpy(), experts, (odec, odec, odec))
    assert P.verdict(got, t) is None, P.verdict(got, t)


@pytest.mark.parametrize("rows", [3, 20])
def test_moe_ragged_spec1_k1_k2(dev, rows):
    """The rate-grouped bank (rate_groups.zig:22-140): SPEC1 (spec1-w15 table) experts at n16 and n32."""
    E1, E2, hidden, inter = 8, 24, 512, 256
    dec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1)
    odec = O.decode(O.CB_SPEC1, 15, 1)
    g1 = synth.bank(81, "prg1", E1, hidden, inter, 16)
    g2 = synth.bank(81, "prg2", E2, hidden, inter, 32)
    todev = lambda b: exl3.Bank(*(exl3.Proj(q.trellis.to(dev), q.suh.to(dev), q.svh.to(dev))  # noqa: E731
                                  for q in (b.gate, b.up, b.down)))
    rb = exl3.Ragged.init([todev(g1), todev(g2)])
    x = synth.normal(81, f"prg.x{rows}", (rows, hidden))
    rng = np.random.default_rng(rows)
    experts = rng.integers(0, E1 + E2, size=rows)
    inds = torch.from_numpy(experts[:, None].astype(np.int32)).to(dev)
    sc = torch.ones(rows, 1, dtype=torch.float32, device=dev)
    y = exl3.moe_ragged(x.to(dev).float(), rb, inds, sc, dec).cpu().numpy().astype(np.float64)
    xf = x.float().numpy()
    for r, e in enumerate(experts):
        grp, local = (g1, e) if e < E1 else (g2, e - E1)
        got = P.inner_from_output(y[r:r + 1], _u16(grp.down.svh)[local])
        t = _moe_truth(grp, xf[r:r + 1], [local], (odec, odec, odec))
        assert P.verdict(got, t) is None, (r, e, P.verdict(got, t))


@pytest.mark.parametrize("rows,topk", [(40, 4), (300, 1)])
def test_moe_gemm_arm(dev, rows, topk):
    """The routed GEMM arm on the summand-relative bar, with the mutation arms (every slot of a row on one expert)."""
    b, bd, x, experts, inds, sc, ssum = _moe_case(dev, 80 + rows, rows, topk, E=8, hidden=512, inter=256)
    odec = O.decode(O.CB_MCG)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe(x.to(dev).float(), bd, inds, sc, exl3.MCG)
    torch.cuda.synchronize()
    got = _moe_inner(y.cpu().numpy().astype(np.float64), b, experts, ssum)
    xf = x.float().numpy()
    t = _moe_truth(b, xf, experts, (odec, odec, odec))
    print(f"[parity] moe gemm rows={rows} worst error / ceiling = {P.worst_ratio(got, t):.4f}", flush=True)
    assert P.verdict(got, t) is None, P.verdict(got, t)
    w15 = P.mutated_window(odec)
    assert P.verdict(got, _moe_truth(b, xf, experts, (w15, w15, w15))) is not None
    e0 = int(experts[0])
    q = b.down
    tr = _u16(q.trellis).copy()
    tr[e0], where = P.flip_one_bit(tr[e0], q.n, odec, np.ones((1, q.in_features)), np.random.default_rng(rows))
    mb = exl3.Bank(b.gate, b.up, exl3.Proj(torch.from_numpy(tr.view(np.int16)), q.suh, q.svh))
    assert P.verdict(got, _moe_truth(mb, xf, experts, (odec, odec, odec))) is not None, where
