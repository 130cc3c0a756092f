"""Per-tile-rate banks (configs[4]'s seeded K1 / K2 tile mix) on the GPU, against the oracle's per-tile functions.

  * exl3_reconstruct_tiled -- the routed GEMV's tiled reader and decoder -- is bit-exact with
    reconstruct_inner_tiled (each tile through decodeTile at its own rate, src/exl3/expert_exl3.zig:338-357) for the
    hash-product codebooks, masked and unmasked windows, and maps of every mix (all K1, all K2, 25 %, 50 %);
  * the routed chain over such a bank (per-slot arm up to 8 rows, expert windows past it; with and without a fused
    shared expert) meets the north-star bar (max-abs-rel 2e-3) against moeSwigluHost restated per tile;
  * the summand-relative bar (tests/_parity.py) holds on the chain, and fails when the truth reads the wrong window
    or one flipped bit of a K1 tile (expert_exl3_kernels.zig:3310-3352's mutation arms).
"""
import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth
from tests import _parity as P
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3
DECODES = {
    "spec1": (exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    "mcg": (exl3.MCG, O.decode(O.CB_MCG)),
    "3inst": (exl3.Decode(exl3.Codebook.inst3), O.decode(O.CB_3INST)),
    "mcg_w12": (exl3.Decode(exl3.Codebook.mcg, exl3.Window(12)), O.decode(O.CB_MCG, 12)),
}


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def _to(tp: exl3.TiledProj, dev) -> exl3.TiledProj:
    return exl3.TiledProj(*(t.to(dev) for t in (tp.trellis, tp.seg_off, tp.seg_k1, tp.suh, tp.svh)))


def _arrays(tp: exl3.TiledProj):
    """(trellis, seg_off, seg_k1, suh, svh) as the oracle takes them."""
    return (_u16(tp.trellis), tp.seg_off.cpu().numpy().view(np.uint32), tp.seg_k1.cpu().numpy(), _u16(tp.suh),
            _u16(tp.svh))


@pytest.mark.parametrize("p_k1", [0.25, 0.0, 1.0, 0.5])
@pytest.mark.parametrize("label", list(DECODES))
def test_reconstruct_tiled_bit_exact(dev, label, p_k1):
    print(f"[tiled] reconstruct {label} p_k1={p_k1}", flush=True)
    dec, odec = DECODES[label]
    tp = synth.tiled_proj(11, f"gtl.{label}", 3, 256, 384, p_k1)
    d = _to(tp, dev)
    tr, off, msk, _, _ = _arrays(tp)
    for e in range(3):
        got = _u16(exl3.reconstruct_tiled(d, e, dec))
        want = O.reconstruct_inner_tiled(tr, off, msk, e, 256, 384, 16, 32, odec)
        bad = np.argwhere(got != want)
        assert bad.size == 0, f"expert {e}: {len(bad)} weights differ, first at {bad[0].tolist()}"


def _bank(dev, seed, E, hidden, inter, p_k1=0.25):
    b = synth.tiled_bank(seed, f"gtm{E}.{hidden}", E, hidden, inter, p_k1, norm=True)
    return b, exl3.Tiled(*(_to(p, dev) for p in (b.gate, b.up, b.down))), [_arrays(p) for p in (b.gate, b.up, b.down)]


def _routing(dev, seed, rows, E, k):
    logits = synth.normal(seed, f"gtm.l{rows}.{E}", (rows, E), dtype=torch.float32)
    inds, scores = exl3.moe_routing_chain(logits.to(dev), k)
    oi, osc = O.route_topk(logits.numpy(), k)
    assert (inds.cpu().numpy().view(np.uint32) == oi).all()
    return inds, scores, oi, osc


@pytest.mark.parametrize("rows", [1, 5, 12, 40])
@pytest.mark.parametrize("label", ["spec1", "mcg"])
def test_moe_tiled_against_oracle(dev, rows, label):
    """Per-slot arm (rows <= 8) and expert windows; f16 output through the fold (or the reduce)."""
    print(f"[tiled] moe {label} rows={rows}", flush=True)
    dec, odec = DECODES[label]
    E, hidden, inter, k = 16, 512, 256, 4
    b, bd, arrs = _bank(dev, 30 + rows, E, hidden, inter)
    x = synth.normal(30 + rows, f"gtm.x{rows}", (rows, hidden))
    inds, scores, oi, osc = _routing(dev, 30 + rows, rows, E, k)
    y = exl3.moe_tiled(x.to(dev), bd, inds, scores, dec).float().cpu().numpy()
    want = O.moe_swiglu_tiled_rows(x.float().numpy(), arrs, oi, osc, hidden, inter, 16, 32, odec)
    assert max_abs_rel(y, want) < BAR
    # with the reduce finish instead of the fold: the same result at the bar
    with exl3.arm_overrides(moe_fold=0):
        y2 = exl3.moe_tiled(x.to(dev), bd, inds, scores, dec).float().cpu().numpy()
    assert max_abs_rel(y2, want) < BAR


@pytest.mark.parametrize("rows", [1, 6, 20])
def test_moe_tiled_with_shared_bank(dev, rows):
    """A K4 shared expert (uniform one-expert bank) in the routed launches: T(T(routed) + T(shared)); with an f32
    output the fused form declines and the wrapper makes the pair of calls."""
    print(f"[tiled] moe+shared rows={rows}", flush=True)
    dec, odec = DECODES["spec1"]
    E, hidden, inter, k = 16, 512, 256, 4
    b, bd, arrs = _bank(dev, 50 + rows, E, hidden, inter)
    sh = synth.bank(50 + rows, "gtm.shared", 1, hidden, inter, 64, norm=True)
    shd = exl3.Bank(*(exl3.Proj(q.trellis.to(dev), q.suh.to(dev), q.svh.to(dev)) for q in (sh.gate, sh.up, sh.down)))
    x = synth.normal(50 + rows, f"gtm.sx{rows}", (rows, hidden))
    inds, scores, oi, osc = _routing(dev, 50 + rows, rows, E, k)
    xf = x.float().numpy()
    routed = O.moe_swiglu_tiled_rows(xf, arrs, oi, osc, hidden, inter, 16, 32, odec)
    shared = O.moe_swiglu_rows(xf, *[tuple(_u16(a) for a in (q.trellis, q.suh, q.svh)) for q in (sh.gate, sh.up,
                                                                                                   sh.down)],
                               np.zeros((rows, 1)), np.ones((rows, 1)), hidden, inter, (64, 64, 64), odec)
    y = exl3.moe_tiled_with_shared_bank(x.to(dev), bd, shd, inds, scores, dec).float().cpu().numpy()
    want = routed.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
    assert max_abs_rel(y, want) < BAR
    y32 = exl3.moe_tiled_with_shared_bank(x.to(dev).float(), bd, shd, inds, scores, dec).cpu().numpy()
    assert max_abs_rel(y32, routed + shared) < BAR


# ---- the summand-relative bar: every slot of a row on one expert, so the down finish undoes exactly ----------------


def _tiled_truth(arrs, x, experts_of_row, odec, hidden, inter):
    """Exact down inner products of each row's expert at the chain's rounding points (tests/_parity.down_prepared)."""
    rows_p, rows_w = [], []
    for r, e in enumerate(experts_of_row):
        w = [P.f16_bits(O.reconstruct_inner_tiled(a[0], a[1], a[2], e, i, o, 16, 32, odec))
             for a, (i, o) in zip(arrs, ((hidden, inter), (hidden, inter), (inter, hidden)))]
        g, u, d = arrs
        gv = P.f16_bits(g[4][e]) * P.hadamard_blocks(P.prepared_rows(x[r:r + 1], g[3][e]) @ w[0])
        uv = P.f16_bits(u[4][e]) * P.hadamard_blocks(P.prepared_rows(x[r:r + 1], u[3][e]) @ w[1])
        rows_p.append(P.down_prepared(gv, uv, d[3][e])[0])
        rows_w.append(w[2])
    inner = np.stack([p @ w for p, w in zip(rows_p, rows_w)])
    amag = np.stack([np.abs(p) @ np.abs(w) for p, w in zip(rows_p, rows_w)])
    bound = np.stack([np.abs(p).max() * np.abs(w).max(axis=0) for p, w in zip(rows_p, rows_w)])
    return P.Truth(inner, amag, bound, inter, P.MID_ULPS)


def _flip_k1_bit(arr, e, in_f, out_f, odec, xk, rng, min_effect=0.5):
    """The projection's arrays with one bit of one K1 tile of expert e flipped, chosen so the flip moves some weight by
    |dw| * max|x_k| >= min_effect; and where it is."""
    tr, off, msk = arr[0], arr[1], arr[2]
    it, segs = in_f // 16, out_f // 128
    before = P.f16_bits(O.reconstruct_inner_tiled(tr, off, msk, e, in_f, out_f, 16, 32, odec))
    for _ in range(2000):
        tk, s = int(rng.integers(it)), int(rng.integers(segs))
        m = int(msk[e, tk, s])
        k1_tiles = [o for o in range(8) if m >> o & 1]
        if not k1_tiles:
            continue
        o = k1_tiles[int(rng.integers(len(k1_tiles)))]
        hw = 2 * int(off[e, tk, s]) + sum(16 if m >> q & 1 else 32 for q in range(o)) + int(rng.integers(16))
        bit = int(rng.integers(16))
        t2 = tr.copy()
        t2[hw] ^= np.uint16(1 << bit)
        after = P.f16_bits(O.reconstruct_inner_tiled(t2, off, msk, e, in_f, out_f, 16, 32, odec))
        if np.nanmax(np.abs(after - before) * xk[:, None]) >= min_effect:
            return (t2,) + tuple(arr[1:]), (tk, s, o, hw, bit)
    raise AssertionError("no K1-tile bit flip moved a weight")


@pytest.mark.parametrize("rows,topk", [(1, 1), (5, 4), (12, 1), (40, 4)])
def test_moe_tiled_summand_bar_with_mutations(dev, rows, topk):
    print(f"[tiled] parity rows={rows} topk={topk}", flush=True)
    dec, odec = DECODES["spec1"]
    E, hidden, inter = 12, 512, 256
    b, bd, arrs = _bank(dev, 70 + rows, E, hidden, inter)
    x = synth.normal(70 + rows, f"gtp.x{rows}", (rows, hidden))
    rng = np.random.default_rng(rows)
    experts = rng.integers(0, E, size=rows)
    inds = torch.from_numpy(np.repeat(experts[:, None], topk, axis=1).astype(np.int32)).to(dev)
    sc = rng.uniform(0.5, 1.5, size=(rows, topk)).astype(np.float32)
    sc /= sc.sum(axis=1, keepdims=True)
    ssum = sc.sum(axis=1, dtype=np.float64)[:, None]
    y = exl3.moe_tiled(x.to(dev).float(), bd, inds, torch.from_numpy(sc).to(dev), dec).cpu().numpy().astype(np.float64)
    svh_d = arrs[2][4]
    got = np.stack([P.inner_from_output(y[r] / ssum[r], svh_d[e]) for r, e in enumerate(experts)])
    xf = x.float().numpy()
    t = _tiled_truth(arrs, xf, experts, odec, hidden, inter)
    print(f"[parity] tiled moe rows={rows} topk={topk} worst error / ceiling = {P.worst_ratio(got, t):.4f}", flush=True)
    assert P.verdict(got, t) is None, P.verdict(got, t)
    assert P.verdict(got, _tiled_truth(arrs, xf, experts, P.mutated_window(odec), hidden, inter)) is not None
    e0 = int(experts[0])
    for pi, (i, o) in ((2, (inter, hidden)), (0, (hidden, inter))):
        xk = np.ones(i) if pi == 2 else np.abs(P.prepared_rows(xf[:1], arrs[0][3][e0])).max(axis=0)
        m, where = _flip_k1_bit(arrs[pi], e0, i, o, odec, xk, np.random.default_rng(rows + pi))
        ma = list(arrs)
        ma[pi] = m
        assert P.verdict(got, _tiled_truth(ma, xf, experts, odec, hidden, inter)) is not None, (pi, where)
