"""GPU parity of the routed SwiGLU expert chain (moe / moeWithShared / moeClamped / moeRagged) and the router.

Reference oracle: moeSwigluHost (src/exl3/expert_exl3_kernels.zig:3059-3114), per row.  Bar: max-abs-rel 2e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3


def _np(p):
    return (p.trellis.numpy().view(np.uint16), p.suh.numpy().view(np.uint16), p.svh.numpy().view(np.uint16))


def _to(b, dev):
    return exl3.Bank(*(exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev)) for p in (b.gate, b.up, b.down)))


def _route(seed, rows, experts, k):
    logits = synth.normal(seed, "logits", (rows, experts), dtype=torch.float32).numpy()
    return O.route_topk(logits, k)


def _oracle_moe(b, x, inds, scores, hidden, inter, n, odec, clamp=0.0):
    ys = []
    for r in range(x.shape[0]):
        ys.append(O.moe_swiglu_host(x[r], _np(b.gate), _np(b.up), _np(b.down), inds[r], scores[r], hidden, inter,
                                    (n, n, n), odec, clamp))
    return np.stack(ys)


@pytest.mark.parametrize("rows", [1, 3, 8, 16, 17, 40])
@pytest.mark.parametrize("n", [32, 48])
def test_moe_decode_chain(dev, rows, n):
    """Up to 8 rows: the per-slot decode chain; above: the sorted arm (slots grouped into expert windows)."""
    print(f"[moe] rows={rows} n={n}", flush=True)
    E, hidden, inter, k = 16, 256, 384, 4
    b = synth.bank(3, "moe", E, hidden, inter, n)
    x = synth.normal(3, "x", (rows, hidden))
    inds, scores = _route(3 + rows, rows, E, k)
    want = _oracle_moe(b, x.float().numpy(), inds, scores, hidden, inter, n, O.decode(O.CB_MCG))
    y = exl3.moe(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                 torch.from_numpy(scores).to(dev), exl3.MCG)
    assert y.shape == x.shape and y.dtype == torch.float16
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("label,dec,odec", [
    ("spec1", exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    ("pair1", exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1)),
    ("3inst", exl3.INST3, O.decode(O.CB_3INST)),
])
@pytest.mark.parametrize("rows", [2, 20])
def test_moe_codebooks(dev, label, dec, odec, rows):
    E, hidden, inter, k, n = 8, 256, 256, 3, 32
    b = synth.bank(8, "moe" + label, E, hidden, inter, n)
    x = synth.normal(8, "x", (rows, hidden))
    inds, scores = _route(8, rows, E, k)
    want = _oracle_moe(b, x.float().numpy(), inds, scores, hidden, inter, n, odec)
    y = exl3.moe(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                 torch.from_numpy(scores).to(dev), dec)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("rows", [3, 24])
def test_moe_with_shared_and_clamped(dev, rows):
    E, hidden, inter, k, n = 8, 256, 128, 2, 32
    b = synth.bank(4, "moes", E, hidden, inter, n)
    x = synth.normal(4, "x", (rows, hidden))
    inds, scores = _route(4, rows, E, k)
    shared = synth.normal(4, "shared", (rows, hidden))
    bd = _to(b, dev)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    want = _oracle_moe(b, x.float().numpy(), inds, scores, hidden, inter, n, O.decode(O.CB_MCG))
    y = exl3.moe_with_shared(x.to(dev), bd, xi, sc, exl3.MCG, False, shared.to(dev))
    assert max_abs_rel(y.float().cpu().numpy(), want + shared.float().numpy()) < BAR
    wantc = _oracle_moe(b, x.float().numpy(), inds, scores, hidden, inter, n, O.decode(O.CB_MCG), clamp=4.0)
    yc = exl3.moe_clamped(x.to(dev), bd, xi, sc, exl3.MCG, 4)
    assert max_abs_rel(yc.float().cpu().numpy(), wantc) < BAR
    assert max_abs_rel(wantc, want) > 10 * BAR  # the clamp is live on this data


@pytest.mark.parametrize("rows,groups", [
    (3, [(6, (32, 32, 48)), (10, (16, 16, 32))]),
    (21, [(6, (32, 32, 48)), (10, (16, 16, 32))]),
    # rates off the lane-reader set (20, 36, 56) beside lane rates: both ragged launches must run
    (3, [(6, (20, 32, 56)), (10, (16, 36, 32))]),
    (21, [(6, (20, 32, 56)), (10, (16, 36, 32))]),
])
def test_moe_ragged_rate_groups(dev, rows, groups):
    hidden, inter, k = 256, 256, 4
    banks = [synth.bank(20 + g, f"rg{g}", e, hidden, inter, rates) for g, (e, rates) in enumerate(groups)]
    rb = exl3.Ragged.init([_to(b, dev) for b in banks])
    E = sum(e for e, _ in groups)
    x = synth.normal(20, "x", (rows, hidden))
    inds, scores = _route(20, rows, E, k)
    want = np.zeros((rows, hidden))
    odec = O.decode(O.CB_MCG)
    for r in range(rows):
        for j in range(k):
            e = int(inds[r, j])
            g = 0 if e < groups[0][0] else 1
            local = e - (0 if g == 0 else groups[0][0])
            b = banks[g]
            want[r] += O.moe_swiglu_host(x[r].float().numpy(), _np(b.gate), _np(b.up), _np(b.down), [local],
                                         [scores[r, j]], hidden, inter, groups[g][1], odec)
    y = exl3.moe_ragged(x.to(dev), rb, torch.from_numpy(inds.view(np.int32)).to(dev),
                        torch.from_numpy(scores).to(dev), exl3.MCG)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    lane_only = all(n in exl3.LANE_RATES for _, rates in groups for n in rates)
    assert rb.c().lane_rates_only == int(lane_only)


def test_moe_ragged_lane_flag_clear_is_correct(dev, monkeypatch):
    """A zeroed `lane_rates_only` (the C default) also runs the generic-rate launch; the result must not change."""
    hidden, inter, k, rows = 256, 128, 4, 5
    groups = [(5, (16, 32, 48)), (7, (64, 24, 40))]
    banks = [synth.bank(60 + g, f"lf{g}", e, hidden, inter, rates) for g, (e, rates) in enumerate(groups)]
    rb = exl3.Ragged.init([_to(b, dev) for b in banks])
    E = sum(e for e, _ in groups)
    x = synth.normal(60, "x", (rows, hidden)).to(dev)
    inds, scores = _route(60, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    assert rb.c().lane_rates_only == 1
    y1 = exl3.moe_ragged(x, rb, xi, sc, exl3.MCG)
    c0 = exl3.Ragged.c

    def cleared(self):
        r = c0(self)
        r.lane_rates_only = 0
        return r
    monkeypatch.setattr(exl3.Ragged, "c", cleared)
    y0 = exl3.moe_ragged(x, rb, xi, sc, exl3.MCG)
    assert torch.equal(y0, y1)


def test_moe_ragged_stq_rates_k1_k2(dev):
    """configs[4]'s layer in its reference-expressible form: per-expert rate groups at K=1 and K=2 (1:3), SPEC1
    with the spec1-w15 table (the SPEC1 table with K=1 rows), plus a shared expert, against the oracle."""
    hidden, inter, k, rows = 256, 128, 8, 5
    groups = [(4, (16, 16, 16)), (12, (32, 32, 32))]
    banks = [synth.bank(40 + g, f"stq{g}", e, hidden, inter, rates) for g, (e, rates) in enumerate(groups)]
    rb = exl3.Ragged.init([_to(b, dev) for b in banks])
    E = sum(e for e, _ in groups)
    dec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1)
    odec = O.decode(O.CB_SPEC1, 15, 1)
    x = synth.normal(40, "x", (rows, hidden))
    inds, scores = _route(40, rows, E, k)
    sh = synth.normal(41, "shared", (rows, hidden))
    want = np.zeros((rows, hidden))
    for r in range(rows):
        for j in range(k):
            e = int(inds[r, j])
            g = 0 if e < groups[0][0] else 1
            local = e - (0 if g == 0 else groups[0][0])
            b = banks[g]
            want[r] += O.moe_swiglu_host(x[r].float().numpy(), _np(b.gate), _np(b.up), _np(b.down), [local],
                                         [scores[r, j]], hidden, inter, groups[g][1], odec)
    # the routed sum is rounded to the output dtype before the shared expert is added
    want = want.astype(np.float16).astype(np.float64) + sh.float().numpy()
    y = exl3.moe_ragged(x.to(dev), rb, torch.from_numpy(inds.view(np.int32)).to(dev),
                        torch.from_numpy(scores).to(dev), dec, shared=sh.to(dev))
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


def test_moe_sorted_arm_concentrated_routing(dev):
    """Every row routes to the same experts (40 slots per expert, ten windows each) and some ids sit past the bank
    (clamped to the last expert, as the decode chain does)."""
    E, hidden, inter, k, rows, n = 6, 256, 128, 4, 40, 32
    b = synth.bank(9, "moec", E, hidden, inter, n)
    x = synth.normal(9, "x", (rows, hidden))
    inds = np.tile(np.array([[3, 0, 5, 1]], dtype=np.uint32), (rows, 1))
    inds[::7, 2] = 9  # past the bank: clamped to expert 5
    _, scores = _route(9, rows, E, k)
    want = _oracle_moe(b, x.float().numpy(), np.minimum(inds, E - 1), scores, hidden, inter, n, O.decode(O.CB_MCG))
    y = exl3.moe(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                 torch.from_numpy(scores).to(dev), exl3.MCG)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


def test_moe_sorted_and_per_slot_arms_agree(dev):
    """The sorted arm (expert windows) and the per-slot chain give the same layer to the bar on one routing."""
    E, hidden, inter, k, rows, n = 32, 256, 256, 8, 24, 32
    b = _to(synth.bank(11, "moea", E, hidden, inter, n), dev)
    x = synth.normal(11, "x", (rows, hidden)).to(dev)
    inds, scores = _route(11, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    sorted_arm = exl3.moe(x, b, xi, sc, exl3.MCG).float().cpu().numpy()
    with exl3.arm_overrides(moe_windows=0):
        per_slot = exl3.moe(x, b, xi, sc, exl3.MCG).float().cpu().numpy()
    assert max_abs_rel(sorted_arm, per_slot) < BAR


@pytest.mark.parametrize("rows", [1, 5, 24])
@pytest.mark.parametrize("with_shared", [False, True])
def test_moe_fold_and_reduce_arms_agree(dev, rows, with_shared):
    """The down projection folded straight into y and the planes + reduce launch agree to the bar against the
    oracle (per-slot arm up to 8 rows, sorted arm above), with and without a shared expert, and the accumulators
    are clean for the next call."""
    print(f"[moe] fold arms rows={rows} shared={with_shared}", flush=True)
    E, hidden, inter, k, n = 24, 256, 384, 6, 32
    b = synth.bank(13, "moef", E, hidden, inter, n)
    bd = _to(b, dev)
    x = synth.normal(13, "x", (rows, hidden))
    inds, scores = _route(13 + rows, rows, E, k)
    want = _oracle_moe(b, x.float().numpy(), inds, scores, hidden, inter, n, O.decode(O.CB_MCG))
    sh = synth.normal(14, "shared", (rows, hidden)) if with_shared else None
    if with_shared:
        want = want.astype(np.float16).astype(np.float64) + sh.float().numpy()
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    shd = None if sh is None else sh.to(dev)
    got = {}
    for fold in (1, 0, 1):
        with exl3.arm_overrides(moe_fold=fold):
            y = exl3.moe_with_shared(x.to(dev), bd, xi, sc, exl3.MCG, False, shd) if with_shared else \
                exl3.moe(x.to(dev), bd, xi, sc, exl3.MCG)
        got.setdefault(fold, []).append(y.float().cpu().numpy())
    for ys in got.values():
        for y in ys:
            assert max_abs_rel(y, want) < BAR
    assert np.array_equal(got[1][0], got[1][1])  # exact accumulation: the same bytes on every call


def test_router_matches_oracle(dev):
    logits = synth.normal(2, "logits", (9, 256), dtype=torch.float32)
    inds, scores = exl3.moe_routing_chain(logits.to(dev), 8)
    oi, os_ = O.route_topk(logits.numpy(), 8)
    assert (inds.cpu().numpy().view(np.uint32) == oi).all()
    assert np.allclose(scores.cpu().numpy(), os_, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("experts,k", [(40, 8), (100, 8), (256, 8), (300, 32), (1024, 32)])
def test_router_non_finite_logits_match_oracle(dev, experts, k):
    """All-NaN, partly NaN, all -inf, mostly -inf and +inf rows: every pick is a distinct expert in range, equal to
    the oracle's (NaN selects as -inf, ties to the lower index), and the scores match it, NaN where it has NaN."""
    print(f"[router] non-finite E={experts} k={k}", flush=True)
    rng = np.random.default_rng(experts + k)
    lg = rng.standard_normal((7, experts)).astype(np.float32)
    lg[0, :] = np.nan
    lg[1, ::3] = np.nan
    lg[2, :] = -np.inf
    lg[2, [5, experts - 1]] = [1.0, -2.0]
    lg[3, :] = -np.inf
    lg[3, experts // 2] = np.nan
    lg[4, [0, 1, 2]] = np.inf
    lg[5, :] = 0.0
    inds, scores = exl3.moe_routing_chain(torch.from_numpy(lg).to(dev), k)
    torch.cuda.synchronize()
    oi, os_ = O.route_topk(lg, k)
    gi = inds.cpu().numpy().view(np.uint32)
    assert (gi == oi).all()
    assert all(len(set(r.tolist())) == k for r in gi) and gi.max() < experts
    assert np.allclose(scores.cpu().numpy(), os_, rtol=1e-5, atol=1e-7, equal_nan=True)


def test_tile_major_matches_oracle(dev):
    t = synth.codes(1, "tm", (3, 4, 6, 40))
    got = exl3.tile_major(t.to(dev)).cpu().numpy().view(np.uint16)
    src = t.numpy().view(np.uint16)
    for e in range(3):
        assert (got[e].reshape(-1) == O.tile_major(src[e].reshape(-1), 4, 6, 40)).all()
    back = exl3.tile_major(torch.from_numpy(got.view(np.int16)).to(dev), inverse=True).cpu().numpy()
    assert (back.view(np.uint16) == src).all()


def _two_calls(x, bd, sd, xi, sc, dec, limit=0):
    """The reference callers' pair: the shared expert as a one-expert chain, then moeWithShared / moeClamped."""
    rows = x.shape[0]
    z = torch.zeros(rows, 1, dtype=torch.int32, device=x.device)
    o = torch.ones(rows, 1, dtype=torch.float32, device=x.device)
    if limit:
        s = exl3.moe_clamped(x, sd, z, o, dec, limit)
        return exl3.moe_clamped(x, bd, xi, sc, dec, limit, shared=s)
    s = exl3.moe(x, sd, z, o, dec)
    return exl3.moe_with_shared(x, bd, xi, sc, dec, False, s)


@pytest.mark.parametrize("rows", [1, 3, 8, 16, 17, 33])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("limit", [0, 4])
def test_moe_with_shared_bank_is_the_two_calls(dev, rows, dtype, limit):
    """The fused shared expert (two launches) against the two calls it replaces (four launches), T(T(routed) +
    T(shared)) in both (their k splits may differ, so the f32 partial sums may round an output to a neighbouring
    value), and against the oracle (routed + shared expert) at the bar."""
    print(f"[moe shared bank] rows={rows} dtype={dtype} limit={limit}", flush=True)
    E, hidden, inter, k, n = 8, 256, 256, 4, 32
    b = synth.bank(31, "msb", E, hidden, inter, n)
    s = synth.bank(31, "msb.shared", 1, hidden, inter, n)
    x = synth.normal(31, f"x{rows}", (rows, hidden)).to(dtype)
    inds, scores = _route(31 + rows, rows, E, k)
    bd, sd = _to(b, dev), _to(s, dev)
    xd = x.to(dev)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    y = exl3.moe_with_shared_bank(xd, bd, sd, xi, sc, exl3.MCG, limit)
    ref = _two_calls(xd, bd, sd, xi, sc, exl3.MCG, limit)
    assert y.dtype == dtype and y.shape == x.shape
    bar = BAR if dtype == torch.float16 else 8e-3  # bf16 output rounding alone is 2^-9 relative
    assert max_abs_rel(y.float().cpu().numpy(), ref.float().cpu().numpy()) < bar
    odec = O.decode(O.CB_MCG)
    xf = x.float().numpy()
    want = _oracle_moe(b, xf, inds, scores, hidden, inter, n, odec, clamp=float(limit))
    want = want + _oracle_moe(s, xf, np.zeros((rows, 1), np.uint32), np.ones((rows, 1), np.float32), hidden, inter,
                              n, odec, clamp=float(limit))
    assert max_abs_rel(y.float().cpu().numpy(), want) < bar


@pytest.mark.parametrize("rows", [17, 40])
def test_moe_with_shared_bank_serves_wide_batches_in_the_sorted_arm(dev, rows):
    """Past 8 rows the fused form runs in the expert-window launches (the C ABI does not decline) and equals the two
    calls at the bar.  The GEMM arm is held off: at 40 rows (10 slots per expert) the layer would take it, and the fused
    form declines that arm."""
    E, hidden, inter, k, n = 16, 256, 128, 4, 32
    b = synth.bank(35, "msw", E, hidden, inter, n)
    s = synth.bank(35, "msw.shared", 1, hidden, inter, n)
    x = synth.normal(35, f"x{rows}", (rows, hidden))
    inds, scores = _route(35 + rows, rows, E, k)
    bd, sd = _to(b, dev), _to(s, dev)
    xd = x.to(dev)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    L = exl3._lib.load()
    cb = exl3._lib.BankT(bd.gate.c(), bd.up.c(), bd.down.c())
    cs = exl3._lib.BankT(sd.gate.c(), sd.up.c(), sd.down.c())
    ws = exl3.workspace.get(dev, L.exl3_moe_with_shared_bank_workspace_size(rows, k, hidden, inter))
    y = torch.empty_like(xd)
    x2 = xd.contiguous()
    with exl3.arm_overrides(moe_gemm=0):
        rc = L.exl3_moe_with_shared_bank(x2.data_ptr(), exl3._dt(x2, "x"), rows, hidden, inter, E, ctypes.byref(cb),
                                         ctypes.byref(cs), xi.data_ptr(), sc.data_ptr(), 2, k, exl3.MCG.c(), 0, 0,
                                         y.data_ptr(), exl3._dt(y, "y"), ws.data_ptr(), ws.numel(),
                                         exl3._stream(dev))
        assert rc == 0, exl3._lib.last_error()
        ref = _two_calls(xd, bd, sd, xi, sc, exl3.MCG)
    torch.cuda.synchronize()
    assert max_abs_rel(y.float().cpu().numpy(), ref.float().cpu().numpy()) < BAR


@pytest.mark.parametrize("case", ["rows700", "f32", "rates"])
def test_moe_with_shared_bank_declines_to_the_two_calls(dev, case):
    """Where the fused form does not serve, the C ABI declines before any launch and the wrapper makes the two
    calls; the result is the two calls' own.  700 rows: the routed, shared and combine fold words (3 x 700 x 256)
    exceed the fused finish's region (with the GEMM arm held off: at 175 slots per expert it would take the layer and
    serve the shared bank in its own launches)."""
    E, hidden, inter, k, n = 8, 256, 128, 2, 32
    rows = 700 if case == "rows700" else 2
    b = synth.bank(33, "msd", E, hidden, inter, n)
    s = synth.bank(33, "msd.shared", 1, hidden, inter, 48 if case == "rates" else n)
    x = synth.normal(33, "x", (rows, hidden)).to(torch.float32 if case == "f32" else torch.float16)
    inds, scores = _route(33, rows, E, k)
    bd, sd = _to(b, dev), _to(s, dev)
    xd = x.to(dev)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    L = exl3._lib.load()
    cb = exl3._lib.BankT(bd.gate.c(), bd.up.c(), bd.down.c())
    cs = exl3._lib.BankT(sd.gate.c(), sd.up.c(), sd.down.c())
    ws = exl3.workspace.get(dev, L.exl3_moe_with_shared_bank_workspace_size(rows, k, hidden, inter))
    y0 = torch.full_like(xd, 7.0)
    x2 = xd.contiguous()
    with exl3.arm_overrides(moe_gemm=0):
        rc = L.exl3_moe_with_shared_bank(x2.data_ptr(), exl3._dt(x2, "x"), rows, hidden, inter, E, ctypes.byref(cb),
                                         ctypes.byref(cs), xi.data_ptr(), sc.data_ptr(), 2, k, exl3.MCG.c(), 0, 0,
                                         y0.data_ptr(), exl3._dt(y0, "y"), ws.data_ptr(), ws.numel(),
                                         exl3._stream(dev))
        torch.cuda.synchronize()
        assert rc == exl3.EXL3_DECLINED and bool((y0 == 7.0).all())  # nothing launched
        y = exl3.moe_with_shared_bank(xd, bd, sd, xi, sc, exl3.MCG)
        ref = _two_calls(xd, bd, sd, xi, sc, exl3.MCG)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("rows", [1, 5, 20])
def test_moe_ragged_with_shared_bank_is_the_two_calls(dev, rows):
    """Rate-grouped routed experts (K1/K2 under SPEC1, lane and generic readers both) with a K4 shared expert in the
    same launches, against the shared one-expert chain followed by moeRagged with `shared`."""
    hidden, inter, k = 256, 256, 4
    dec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1)
    groups = [(6, (16, 16, 16)), (10, (32, 36, 32))]
    banks = [synth.bank(40 + g, f"rgs{g}", e, hidden, inter, rates) for g, (e, rates) in enumerate(groups)]
    rb = exl3.Ragged.init([_to(b, dev) for b in banks])
    sd = _to(synth.bank(40, "rgs.shared", 1, hidden, inter, 64), dev)
    E = sum(e for e, _ in groups)
    x = synth.normal(40, "x", (rows, hidden)).to(dev)
    inds, scores = _route(40, rows, E, k)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    y = exl3.moe_ragged_with_shared_bank(x, rb, sd, xi, sc, dec)
    z = torch.zeros(rows, 1, dtype=torch.int32, device=dev)
    o = torch.ones(rows, 1, dtype=torch.float32, device=dev)
    ref = exl3.moe_ragged(x, rb, xi, sc, dec, shared=exl3.moe(x, sd, z, o, dec))
    assert max_abs_rel(y.float().cpu().numpy(), ref.float().cpu().numpy()) < BAR


@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16])
def test_moe_down_fold_outputs_past_its_range(dev, ydt):
    """The down projection's fold across slots with contributions past 2^21: bf16 outputs finite within the bar of
    the exact chain, f16 outputs past 65504 +-inf (never NaN)."""
    from tests import _parity as P

    print(f"[moe] big outputs {ydt}", flush=True)
    E, hidden, inter, k, rows, n = 8, 256, 256, 4, 3, 32
    b = synth.bank(29, "moebig", E, hidden, inter, n)
    b.down.svh = (b.down.svh.float() * 1024).half()
    x = (synth.normal(29, "x", (rows, hidden)).float() * 4).half()
    inds, scores = _route(29, rows, E, k)
    bd = _to(b, dev)
    y = exl3.moe(x.to(dev).to(ydt), bd, torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev),
                 exl3.MCG).float().cpu().numpy().astype(np.float64)
    odec = O.decode(O.CB_MCG)
    svh = b.down.svh.numpy().view(np.uint16)
    y64 = np.zeros((rows, hidden))
    from tests.test_gpu_parity import _moe_truth
    xf = x.to(ydt).float().numpy()
    for r in range(rows):
        for j in range(k):
            e = int(inds[r, j])
            t = _moe_truth(b, xf[r:r + 1], [e], (odec, odec, odec))
            y64[r] += float(scores[r, j]) * P.f16_bits(svh[e]) * P.hadamard_blocks(t.inner[0])
    assert np.abs(y64).max() > 2.0 ** 21
    if ydt == torch.float16:
        over, under = np.abs(y64) > 65520.0 * 1.002, np.abs(y64) < 65504.0 * 0.998
        assert np.isinf(y[over]).all() and (np.sign(y[over]) == np.sign(y64[over])).all()
        assert np.isfinite(y[under]).all()
    else:
        assert max_abs_rel(y, y64) < BAR + 2.0 ** -8


@pytest.mark.parametrize("rows", [2, 20])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16])
def test_moe_scores_in_bf16_and_f16(dev, rows, sdt):
    """Scores in bf16 / f16 (root.zig:114 admits them) are read as they are: the layer equals the call with the same
    values in f32 byte for byte (fold finish at 2 rows, sorted arm at 20), and the oracle to the bar."""
    print(f"[moe] scores {sdt} rows={rows}", flush=True)
    E, hidden, inter, k, n = 16, 256, 256, 4, 32
    b = synth.bank(31, "moesc", E, hidden, inter, n, norm=True)
    bd = _to(b, dev)
    x = synth.normal(31, "x", (rows, hidden))
    inds, scores = _route(31 + rows, rows, E, k)
    sc_low = torch.from_numpy(scores).to(sdt)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    y_low = exl3.moe(x.to(dev), bd, xi, sc_low.to(dev), exl3.MCG)
    y_f32 = exl3.moe(x.to(dev), bd, xi, sc_low.float().to(dev), exl3.MCG)
    assert torch.equal(y_low, y_f32)
    want = _oracle_moe(b, x.float().numpy(), inds, sc_low.float().numpy(), hidden, inter, n, O.decode(O.CB_MCG))
    assert max_abs_rel(y_low.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("fold", [1, 0])
@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float16])
def test_moe_gated_shared_term_every_gate_logit(dev, ydt, fold):
    """`moeWithGatedShared` (root.zig:71-90) over every non-NaN bf16 / f16 gate logit, one per row, both finishes:
    with scores 0 the routed sum is exactly 0, so each output is T(sigmoid(gate) * shared) and must equal the
    oracle's rounding chain (REDUCE_GATED_SHARED_SOURCE, expert_exl3_kernels.zig:2410-2431) bit for bit (the
    reference's test, :7258-7315, holds its kernel to MLX's ops the same way)."""
    print(f"[moe] gated shared every logit {ydt} fold={fold}", flush=True)
    hidden, inter, rows = 128, 128, 4096
    b = synth.bank(33, "gsh", 1, hidden, inter, 32, norm=True)
    bd = _to(b, dev)
    bits = np.arange(1 << 16, dtype=np.uint32)
    if ydt == torch.bfloat16:
        allg = torch.from_numpy((bits << 16).view(np.float32)).to(torch.bfloat16)
    else:
        allg = torch.from_numpy(bits.astype(np.uint16).view(np.float16))
    allg = allg[~torch.isnan(allg.float())]
    shared_vals = torch.from_numpy(np.linspace(-3.0, 3.0, hidden, dtype=np.float32)).to(ydt)
    dt_code = 1 if ydt == torch.bfloat16 else 0
    with exl3.arm_overrides(moe_fold=fold):
        for start in range(0, allg.numel(), rows):
            g = allg[start:start + rows]
            r = g.numel()
            x = synth.normal(33, f"gsh.x{r}", (r, hidden)).to(ydt)
            shared = shared_vals.repeat(r, 1)
            y = exl3.moe_with_gated_shared(x.to(dev), bd, torch.zeros(r, 1, dtype=torch.int32, device=dev),
                                           torch.zeros(r, 1, dtype=torch.float32, device=dev), exl3.MCG, False,
                                           shared.to(dev), g.reshape(r, 1).to(dev))
            got = y.float().cpu().numpy()
            want = O.gated_shared_terms(g.float().numpy(), shared.float().numpy(), dt_code)
            same = (got == want) | (np.isnan(got) & np.isnan(want))
            bad = np.argwhere(~same)
            assert bad.size == 0, (len(bad), [(float(g[i]), got[i, j], want[i, j]) for i, j in bad[:4]])


@pytest.mark.parametrize("ydt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows", [1, 6, 24])
def test_moe_with_gated_shared_against_oracle(dev, rows, ydt):
    """routed + sigmoid(gate) * shared with real scores: T(T(routed) + T(sig * shared)) against the oracle's routed
    sum and its gated term.  In bf16 the kernel's routed sum (gate and up kept in f32) and the oracle's (rounded to
    f16 by its project) may round one bf16 ulp apart, and the final rounding another: the bar allows those two."""
    print(f"[moe] gated shared rows={rows} {ydt}", flush=True)
    E, hidden, inter, k, n = 16, 256, 256, 4, 32
    b = synth.bank(35, "gsh2", E, hidden, inter, n, norm=True)
    x = synth.normal(35, "x", (rows, hidden)).to(ydt)
    inds, scores = _route(35 + rows, rows, E, k)
    shared = synth.normal(36, "sh", (rows, hidden)).to(ydt)
    gate = (synth.normal(37, "g", (rows, 1)) * 3).to(ydt)
    y = exl3.moe_with_gated_shared(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                                   torch.from_numpy(scores).to(dev), exl3.MCG, False, shared.to(dev), gate.to(dev))
    routed = _oracle_moe(b, x.float().numpy(), inds, scores, hidden, inter, n, O.decode(O.CB_MCG))
    routed_t = torch.from_numpy(routed).to(ydt).float().numpy()
    sh, gv = shared.float().numpy(), gate.float().numpy()
    term = O.gated_shared_terms(gv[:, 0], sh, 1 if ydt == torch.bfloat16 else 2)
    want = torch.from_numpy((routed_t + term).astype(np.float32)).to(ydt).float().numpy()
    bar = BAR + (2 * 2.0 ** -8 if ydt == torch.bfloat16 else 0.0)
    assert max_abs_rel(y.float().cpu().numpy(), want) < bar


@pytest.mark.parametrize("rows", [1, 5, 20])
@pytest.mark.parametrize("rates", [(32, 48, 40), (48, 32, 32), (32, 32, 64)])
def test_moe_mixed_projection_rates(dev, rows, rates):
    """A uniform bank whose gate, up and down sit at different rates (moeMixedDecode, root.zig:705-722): gate and up
    run one launch each when they differ, down at its own rate; per-slot arm up to 8 rows, the sorted arm above.
    The fused shared-bank form declines (the wrapper makes the pair of calls)."""
    print(f"[moe] mixed rates {rates} rows={rows}", flush=True)
    E, hidden, inter, k = 12, 256, 256, 3
    b = synth.bank(39, "mixed", E, hidden, inter, rates, norm=True)
    x = synth.normal(39, "x", (rows, hidden))
    inds, scores = _route(39 + rows, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    odec = O.decode(O.CB_MCG)
    want = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, scores, hidden, inter,
                             rates, odec, threads=8)
    y = exl3.moe(x.to(dev), _to(b, dev), xi, sc, exl3.MCG)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    sh = synth.bank(40, "mixed.sh", 1, hidden, inter, 32, norm=True)
    y2 = exl3.moe_with_shared_bank(x.to(dev), _to(b, dev), _to(sh, dev), xi, sc, exl3.MCG)
    shared = O.moe_swiglu_rows(x.float().numpy(), _np(sh.gate), _np(sh.up), _np(sh.down), np.zeros((rows, 1)),
                               np.ones((rows, 1)), hidden, inter, (32, 32, 32), odec, threads=8)
    want2 = want.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
    assert max_abs_rel(y2.float().cpu().numpy(), want2) < BAR


@pytest.mark.parametrize("rows,E,k", [(1, 8, 2), (5, 16, 4), (40, 16, 4), (300, 32, 6)])
@pytest.mark.parametrize("label,dec,odec", [
    ("mcg", exl3.MCG, O.decode(O.CB_MCG)),
    ("3inst", exl3.INST3, O.decode(O.CB_3INST)),
    ("spec1", exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    ("pair1", exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1)),
])
def test_moe_gemm_arm_against_oracle(dev, rows, E, k, label, dec, odec):
    """The routed GEMM arm (moePrefill's sorted windows on the matrix cores, expert_exl3_kernels.zig:2861-2931),
    forced at every width: windows of up to 256 rows per expert, prepared inputs in fragment order, the decode-once
    GEMM for gate/up, the mid, the down GEMM and the reduce, against the oracle to the bar."""
    print(f"[moe gemm] {label} rows={rows} E={E} k={k}", flush=True)
    hidden, inter, n = 256, 384, 48
    b = synth.bank(41, f"mg.{label}", E, hidden, inter, n, norm=True)
    x = synth.normal(41, f"x{rows}", (rows, hidden))
    inds, scores = _route(41 + rows, rows, E, k)
    want = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, scores, hidden, inter,
                             (n, n, n), odec, threads=8)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                     torch.from_numpy(scores).to(dev), dec)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_moe_gemm_arm_odd_hidden_blocks(dev, dtype):
    """The routed GEMM arm at a hidden width of three 128-blocks: the prepare's one-block workgroups (gate and up
    from one gather) for f16 and bf16 inputs, the down GEMM's k range and the reduce's partial block group, against
    the oracle to the bar."""
    rows, E, k, hidden, inter, n = 96, 8, 2, 384, 256, 32
    b = synth.bank(53, "mgodd", E, hidden, inter, n, norm=True)
    x = synth.normal(53, "xodd", (rows, hidden), dtype=dtype)
    inds, scores = _route(53, rows, E, k)
    want = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, scores, hidden, inter,
                             (n, n, n), O.decode(O.CB_MCG), threads=8)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                     torch.from_numpy(scores).to(dev), exl3.MCG)
    bar = BAR + (2.0 ** -8 if dtype == torch.bfloat16 else 0.0)
    assert max_abs_rel(y.float().cpu().numpy(), want) < bar


@pytest.mark.parametrize("rows,E,k", [(40, 16, 4), (300, 8, 2)])
@pytest.mark.parametrize("n", [16, 24, 32, 40, 48, 64])
@pytest.mark.parametrize("label,dec,odec", [
    ("mcg", exl3.MCG, O.decode(O.CB_MCG)),
    ("3inst", exl3.INST3, O.decode(O.CB_3INST)),
])
def test_moe_gemm_arm_every_lane_rate(dev, rows, E, k, n, label, dec, odec):
    """The routed GEMM arm's kernel is built per lane rate (16, 24, 32, 40, 48 and 64 bits a row of 16 weights):
    forced at a sorted-window width and at a prefill width, each rate against the oracle to the bar."""
    print(f"[moe gemm rate] {label} n={n} rows={rows} E={E} k={k}", flush=True)
    hidden, inter = 256, 384
    b = synth.bank(43, f"mgr.{label}.{n}", E, hidden, inter, n, norm=True)
    x = synth.normal(43, f"x{rows}", (rows, hidden))
    inds, scores = _route(43 + rows, rows, E, k)
    want = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, scores, hidden, inter,
                             (n, n, n), odec, threads=8)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe(x.to(dev), _to(b, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                     torch.from_numpy(scores).to(dev), dec)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("routing", ["topk", "skewed"])
def test_moe_gemm_arm_windows_past_one_ranking_pass(dev, routing):
    """4608 tokens x top-8 + the shared expert's rows: 41472 slots, more than 64 chunks of 512 hold, so each chunk of
    the window sort spans 1024 slots and is ranked in two passes.  Top-k routing, and a skewed one (most slots on
    three experts, whose runs cross many chunk boundaries and fill windows of 256 rows, and several experts with no
    slot at all): the GEMM arm's layer against the oracle to the bar."""
    print(f"[moe gemm] two ranking passes routing={routing}", flush=True)
    E, hidden, inter, k, rows, n = 16, 128, 128, 8, 4608, 32
    b = synth.bank(57, "mgp", E, hidden, inter, n, norm=True)
    sh = synth.bank(57, "mgp.shared", 1, hidden, inter, n, norm=True)
    x = synth.normal(57, "x", (rows, hidden))
    inds, scores = _route(57, rows, E, k)
    if routing == "skewed":
        r = np.arange(rows)[:, None]
        c = np.arange(k)[None, :]
        inds = np.where(c < 3, c, 3 + (r + c) % 5).astype(np.uint32)  # distinct per row; experts 8..15 get none
    odec = O.decode(O.CB_MCG)
    routed = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, scores, hidden, inter,
                               (n, n, n), odec, threads=8)
    shared = O.moe_swiglu_rows(x.float().numpy(), _np(sh.gate), _np(sh.up), _np(sh.down), np.zeros((rows, 1)),
                               np.ones((rows, 1)), hidden, inter, (n, n, n), odec, threads=8)
    want = routed.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
    y = exl3.moe_with_shared_bank(x.to(dev), _to(b, dev), _to(sh, dev), torch.from_numpy(inds.view(np.int32)).to(dev),
                                  torch.from_numpy(scores).to(dev), exl3.MCG)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("rows,E,k", [(64, 16, 4), (300, 8, 2)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("limit", [0, 5])
def test_moe_gemm_arm_serves_the_shared_bank_in_its_launches(dev, rows, E, k, dtype, limit):
    """At GEMM-arm widths the fused shared-bank call runs the shared expert as one more expert of the routed launches
    (its rows as extra slots, windows of up to 256 of them) and equals the reference callers' pair of calls -- the
    shared expert as a one-expert layer, then moeWithShared / moeClamped -- bit for bit, for every y dtype; and the
    routed + shared sum matches the oracle at the bar."""
    print(f"[moe gemm shared] rows={rows} E={E} k={k} {dtype} limit={limit}", flush=True)
    hidden, inter, n = 256, 128, 32
    b = synth.bank(47, f"mgs{E}", E, hidden, inter, n, norm=True)
    s = synth.bank(47, "mgs.shared", 1, hidden, inter, n, norm=True)
    x = synth.normal(47, f"x{rows}", (rows, hidden), dtype=dtype)
    inds, scores = _route(47 + rows, rows, E, k)
    bd, sd = _to(b, dev), _to(s, dev)
    xd = x.to(dev)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    L = exl3._lib.load()
    cb = exl3._lib.BankT(bd.gate.c(), bd.up.c(), bd.down.c())
    cs = exl3._lib.BankT(sd.gate.c(), sd.up.c(), sd.down.c())
    ws = exl3.workspace.get(dev, L.exl3_moe_with_shared_bank_workspace_size(rows, k, hidden, inter))
    y = torch.empty_like(xd)
    rc = L.exl3_moe_with_shared_bank(xd.data_ptr(), exl3._dt(xd, "x"), rows, hidden, inter, E, ctypes.byref(cb),
                                     ctypes.byref(cs), xi.data_ptr(), sc.data_ptr(), 2, k, exl3.MCG.c(), 0, limit,
                                     y.data_ptr(), exl3._dt(y, "y"), ws.data_ptr(), ws.numel(), exl3._stream(dev))
    assert rc == 0, exl3._lib.last_error()
    ref = _two_calls(xd, bd, sd, xi, sc, exl3.MCG, limit)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    if dtype == torch.float16 and limit == 0:
        odec = O.decode(O.CB_MCG)
        routed = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, scores, hidden,
                                   inter, (n, n, n), odec, threads=8)
        shared = O.moe_swiglu_rows(x.float().numpy(), _np(s.gate), _np(s.up), _np(s.down), np.zeros((rows, 1)),
                                   np.ones((rows, 1)), hidden, inter, (n, n, n), odec, threads=8)
        want = routed.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
        assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


@pytest.mark.parametrize("E", [1023, 1024])
def test_moe_gemm_arm_shared_bank_at_the_expert_table_limit(dev, E):
    """The GEMM arm's window tables hold 1024 experts: 1023 routed + the shared one run in the same launches and
    equal the pair of calls bit for bit; 1024 routed + shared decline before any launch (the wrapper then makes the
    two calls itself)."""
    print(f"[moe gemm shared limit] E={E}", flush=True)
    hidden, inter, n, k = 128, 128, 16, 8
    rows = E  # 8 slots per expert
    bd = synth.bank(48, f"lim{E}", E, hidden, inter, n, device=dev, norm=True)
    sd = synth.bank(48, "lim.shared", 1, hidden, inter, n, device=dev, norm=True)
    x = synth.normal(48, f"x{E}", (rows, hidden)).to(dev)
    inds, scores = _route(48, rows, E, k)
    xi = torch.from_numpy(inds.view(np.int32)).to(dev)
    sc = torch.from_numpy(scores).to(dev)
    L = exl3._lib.load()
    cb = exl3._lib.BankT(bd.gate.c(), bd.up.c(), bd.down.c())
    cs = exl3._lib.BankT(sd.gate.c(), sd.up.c(), sd.down.c())
    ws = exl3.workspace.get(dev, L.exl3_moe_with_shared_bank_workspace_size(rows, k, hidden, inter))
    y = torch.full_like(x, 7.0)
    rc = L.exl3_moe_with_shared_bank(x.data_ptr(), exl3._dt(x, "x"), rows, hidden, inter, E, ctypes.byref(cb),
                                     ctypes.byref(cs), xi.data_ptr(), sc.data_ptr(), 2, k, exl3.MCG.c(), 0, 0,
                                     y.data_ptr(), exl3._dt(y, "y"), ws.data_ptr(), ws.numel(), exl3._stream(dev))
    ref = _two_calls(x, bd, sd, xi, sc, exl3.MCG)
    torch.cuda.synchronize()
    if E < 1024:
        assert rc == 0, exl3._lib.last_error()
        assert torch.equal(y, ref)
    else:
        assert rc == exl3.EXL3_DECLINED and bool((y == 7.0).all())
        assert torch.equal(exl3.moe_with_shared_bank(x, bd, sd, xi, sc, exl3.MCG), ref)


def test_moe_gemm_arm_long_windows_clamp_and_shared(dev):
    """One expert takes 450 slots (windows of 256 + 194 rows), clamped SwiGLU, a shared expert added after the
    routed rounding, then the same with a gate; and the arm equals the decode chain to the bar."""
    E, hidden, inter, k, rows, n = 4, 256, 256, 2, 300, 32
    b = synth.bank(43, "mgl", E, hidden, inter, n, norm=True)
    x = synth.normal(43, "x", (rows, hidden))
    inds = np.zeros((rows, k), np.uint32)
    inds[:, 1] = np.arange(rows) % 3 + 1          # expert 0 gets every row's first slot: 300 rows
    inds[:150, 1] = 0                             # ... and 150 more (450 in all -- its second slot repeats it)
    sc = np.full((rows, k), 0.5, np.float32)
    xi, scd = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(sc).to(dev)
    odec = O.decode(O.CB_MCG)
    want = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, sc, hidden, inter,
                             (n, n, n), odec, clamp_limit=7.0, threads=8)
    sh = synth.normal(44, "sh", (rows, hidden))
    gate = synth.normal(45, "g", (rows, 1))
    bd = _to(b, dev)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe_clamped(x.to(dev), bd, xi, scd, exl3.MCG, 7)
        y_sh = exl3.moe_clamped(x.to(dev), bd, xi, scd, exl3.MCG, 7, shared=sh.to(dev))
        y_g = exl3.moe_with_gated_shared(x.to(dev), bd, xi, scd, exl3.MCG, False, sh.to(dev), gate.to(dev))
    with exl3.arm_overrides(moe_gemm=0):
        y_chain = exl3.moe_clamped(x.to(dev), bd, xi, scd, exl3.MCG, 7)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    assert max_abs_rel(y.float().cpu().numpy(), y_chain.float().cpu().numpy()) < BAR
    want_sh = want.astype(np.float16).astype(np.float32) + sh.float().numpy()
    assert max_abs_rel(y_sh.float().cpu().numpy(), want_sh) < BAR
    want_g = O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), inds, sc, hidden, inter,
                               (n, n, n), odec, threads=8)
    term = O.gated_shared_terms(gate.float().numpy()[:, 0], sh.float().numpy(), 0)
    want_g = (want_g.astype(np.float16).astype(np.float32) + term).astype(np.float16).astype(np.float32)
    assert max_abs_rel(y_g.float().cpu().numpy(), want_g) < BAR


@pytest.mark.parametrize("rows", [1, 3, 8])
@pytest.mark.parametrize("case", ["moe", "shared_bank", "gated", "clamp_f32scores", "bf16"])
def test_moe_chain_in_one_launch_equals_two_launches(dev, rows, case):
    """The per-slot decode chain fused into one launch (down workgroups wait on their slot's gate/up arrivals) equals
    the two-launch chain bit for bit, call after call (its counters return to zero) and from a replayed HIP graph."""
    print(f"[moe chain] {case} rows={rows}", flush=True)
    E, hidden, inter, k, n = 16, 512, 384, 4, 32
    dtype = torch.bfloat16 if case == "bf16" else torch.float16
    b = synth.bank(49, "chain", E, hidden, inter, n, device=dev, norm=True)
    sd = synth.bank(49, "chain.shared", 1, hidden, inter, n, device=dev, norm=True)
    calls = []
    for c in range(3):
        x = synth.normal(49 + c, f"cx{rows}", (rows, hidden), device=dev).to(dtype)
        inds, scores = _route(49 + c + rows, rows, E, k)
        xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
        sh = synth.normal(50 + c, "csh", (rows, hidden), device=dev).to(dtype)
        g = synth.normal(51 + c, "cg", (rows, 1), device=dev).to(dtype)
        if case == "moe" or case == "bf16":
            calls.append(lambda x=x, xi=xi, sc=sc: exl3.moe(x, b, xi, sc, exl3.MCG))
        elif case == "shared_bank":
            calls.append(lambda x=x, xi=xi, sc=sc: exl3.moe_with_shared_bank(x, b, sd, xi, sc, exl3.MCG))
        elif case == "gated":
            calls.append(lambda x=x, xi=xi, sc=sc, sh=sh, g=g: exl3.moe_with_gated_shared(x, b, xi, sc, exl3.MCG,
                                                                                         False, sh, g))
        else:
            calls.append(lambda x=x, xi=xi, sc=sc: exl3.moe_clamped(x, b, xi, sc, exl3.MCG, 5))
    with exl3.arm_overrides(moe_chain=0):
        ref = [f() for f in calls]
    with exl3.arm_overrides(moe_chain=1):
        got = [f() for f in calls] + [f() for f in calls]
    torch.cuda.synchronize()
    for i, y in enumerate(got):
        assert torch.equal(y, ref[i % len(ref)]), i
    outs = []
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side), exl3.arm_overrides(moe_chain=1):
        [f() for f in calls]  # the side stream's workspace, made and zeroed before the capture
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            outs = [f() for f in calls]
    torch.cuda.current_stream(dev).wait_stream(side)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for i, y in enumerate(outs):
            assert torch.equal(y, ref[i]), ("graph", i)
