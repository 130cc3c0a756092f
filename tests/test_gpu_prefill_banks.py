"""The routed GEMM arm (prefill widths) over ragged and per-tile-rate banks.

The reference sends a rate-grouped layer past DECODE_ROWS_MAX rows to `rate_groups.moePrefill`, per-group sorted GEMMs
(src/exl3/rate_groups.zig:2039-2075, dispatched at src/exl3/root.zig:602-609).  Here one launch serves every rate: each
workgroup's decode waves read its expert's rate (ragged meta) or each k-step's segment offset and rate mask (per-tile
banks) while the MFMA waves are the uniform arm's.  Checked:

  * against the oracle (moeSwigluHost over every row, max-abs-rel 2e-3) for the codebooks and rates each form admits,
    with and without a clamp and a (gated) shared expert;
  * a fused shared bank in the same launches equals the reference callers' pair of calls bit for bit;
  * configs[4]'s layer (hidden 4096, inter 2048, 1.75 bpw, SPEC1 spec1-w15) at 1024 tokens on the summand-relative bar
    (tests/_parity.py), with the reference's mutation arms: the wrong codeword window and one flipped trellis bit must
    fail it (src/exl3/expert_exl3_kernels.zig:3310-3352).
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth
from tests import _parity as P
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3
THREADS = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
DECODES = {
    "mcg": (exl3.MCG, O.decode(O.CB_MCG)),
    "3inst": (exl3.INST3, O.decode(O.CB_3INST)),
    "spec1": (exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    "pair1": (exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1)),
}


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def _np(p):
    return (_u16(p.trellis), _u16(p.suh), _u16(p.svh))


def _to(b, dev):
    return exl3.Bank(*(exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev)) for p in (b.gate, b.up, b.down)))


def _to_tiled(tb, dev):
    return exl3.Tiled(*(exl3.TiledProj(*(t.to(dev) for t in (q.trellis, q.seg_off, q.seg_k1, q.suh, q.svh)))
                        for q in (tb.gate, tb.up, tb.down)))


def _tiled_arrays(tb):
    return [(_u16(q.trellis), q.seg_off.cpu().numpy().view(np.uint32), q.seg_k1.cpu().numpy(), _u16(q.suh),
             _u16(q.svh)) for q in (tb.gate, tb.up, tb.down)]


def _route(seed, rows, experts, k):
    logits = synth.normal(seed, "logits", (rows, experts), dtype=torch.float32).numpy()
    return O.route_topk(logits, k)


def _ragged(dev, seed, groups, hidden, inter):
    banks = [synth.bank(seed + g, f"pb{seed}.{g}", e, hidden, inter, r, norm=True) for g, (e, r) in enumerate(groups)]
    rb = exl3.Ragged.init([_to(b, dev) for b in banks])
    oracle_banks = []
    for nm in ("gate", "up", "down"):
        qs = [getattr(b, nm) for b in banks]
        oracle_banks.append((np.concatenate([_np(q)[0].reshape(-1) for q in qs]),
                             np.concatenate([_np(q)[1] for q in qs]), np.concatenate([_np(q)[2] for q in qs])))
    rates = [np.concatenate([np.full(e, r[i]) for e, r in groups]) for i in range(3)]
    return banks, rb, oracle_banks, rates


RAGGED_GROUPS = {
    "mcg": [(5, (16, 24, 32)), (6, (40, 48, 64)), (5, (32, 32, 16))],
    "3inst": [(5, (16, 24, 32)), (6, (40, 48, 64)), (5, (32, 32, 16))],
    "spec1": [(6, (16, 16, 16)), (10, (32, 24, 48))],
    "pair1": [(6, (24, 40, 64)), (10, (32, 48, 24))],
}


@pytest.mark.parametrize("rows,k", [(5, 4), (40, 4), (300, 6)])
@pytest.mark.parametrize("label", list(DECODES))
def test_ragged_bank_on_the_gemm_arm_against_oracle(dev, label, rows, k):
    print(f"[prefill ragged] {label} rows={rows} k={k}", flush=True)
    dec, odec = DECODES[label]
    hidden, inter = 256, 384
    groups = RAGGED_GROUPS[label]
    _, rb, ob, rates = _ragged(dev, 90, groups, hidden, inter)
    E = sum(e for e, _ in groups)
    x = synth.normal(90, f"x{rows}", (rows, hidden))
    inds, scores = _route(90 + rows, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    want = O.moe_swiglu_rows(x.float().numpy(), *ob, inds, scores, hidden, inter, rates, odec, threads=THREADS)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe_ragged(x.to(dev), rb, xi, sc, dec)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    if rows == 300 and label == "mcg":  # clamp, then a gated shared expert, on the same arm
        wc = O.moe_swiglu_rows(x.float().numpy(), *ob, inds, scores, hidden, inter, rates, odec, clamp_limit=6.0,
                               threads=THREADS)
        sh = synth.normal(91, "sh", (rows, hidden))
        g = synth.normal(92, "g", (rows, 1))
        with exl3.arm_overrides(moe_gemm=1):
            yc = exl3.moe_ragged(x.to(dev), rb, xi, sc, dec, limit=6)
            yg = exl3.moe_ragged(x.to(dev), rb, xi, sc, dec, False, sh.to(dev), g.to(dev))
        assert max_abs_rel(yc.float().cpu().numpy(), wc) < BAR
        term = O.gated_shared_terms(g.float().numpy()[:, 0], sh.float().numpy(), 0)
        wg = (want.astype(np.float16).astype(np.float32) + term).astype(np.float16).astype(np.float32)
        assert max_abs_rel(yg.float().cpu().numpy(), wg) < BAR


@pytest.mark.parametrize("rows,k", [(5, 4), (40, 4), (300, 6)])
@pytest.mark.parametrize("label", ["mcg", "3inst", "spec1"])
@pytest.mark.parametrize("p_k1", [0.25, 1.0])
def test_tiled_bank_on_the_gemm_arm_against_oracle(dev, label, rows, k, p_k1):
    print(f"[prefill tiled] {label} rows={rows} k={k} p_k1={p_k1}", flush=True)
    dec, odec = DECODES[label]
    E, hidden, inter = 12, 256, 384
    tb = synth.tiled_bank(93, f"pt.{label}", E, hidden, inter, p_k1, norm=True)
    td = _to_tiled(tb, dev)
    x = synth.normal(93, f"x{rows}", (rows, hidden))
    inds, scores = _route(93 + rows, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    want = O.moe_swiglu_tiled_rows(x.float().numpy(), _tiled_arrays(tb), inds, scores, hidden, inter, 16, 32, odec,
                                   threads=THREADS)
    with exl3.arm_overrides(moe_gemm=1):
        y = exl3.moe_tiled(x.to(dev), td, xi, sc, dec)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR
    with exl3.arm_overrides(moe_gemm=0):
        y_chain = exl3.moe_tiled(x.to(dev), td, xi, sc, dec)
    assert max_abs_rel(y.float().cpu().numpy(), y_chain.float().cpu().numpy()) < BAR


def _two_calls_ragged(x, rb, sd, xi, sc, dec, form, td=None):
    z = torch.zeros(x.shape[0], 1, dtype=torch.int32, device=x.device)
    o = torch.ones(x.shape[0], 1, dtype=torch.float32, device=x.device)
    shared = exl3.moe(x, sd, z, o, dec)
    if form == "ragged":
        return exl3.moe_ragged(x, rb, xi, sc, dec, shared=shared)
    return exl3.moe_tiled(x, td, xi, sc, dec, shared=shared)


@pytest.mark.parametrize("form", ["ragged", "tiled"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("sh_n", [32, 64])
def test_shared_bank_rides_the_gemm_arm_of_ragged_and_tiled_banks(dev, form, dtype, sh_n):
    """At a prefill width (64 rows, E = 8, top-8) the fused shared bank is one more expert of the GEMM arm's launches,
    decoded at its own rate, and y equals the pair of calls (the one-expert chain, then `shared`) bit for bit."""
    print(f"[prefill shared] {form} {dtype} sh_n={sh_n}", flush=True)
    E, hidden, inter, k, rows = 8, 256, 256, 8, 64
    x = synth.normal(95, "x", (rows, hidden), dtype=dtype).to(dev)
    inds, scores = _route(95, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    dec = exl3.MCG
    sd = _to(synth.bank(96, "pbs.shared", 1, hidden, inter, sh_n, norm=True), dev)
    rb = td = None
    if form == "ragged":
        _, rb, _, _ = _ragged(dev, 97, [(3, (16, 16, 16)), (5, (32, 48, 32))], hidden, inter)
        y = exl3.moe_ragged_with_shared_bank(x, rb, sd, xi, sc, dec)
    else:
        td = _to_tiled(synth.tiled_bank(98, "pts", E, hidden, inter, 0.25, norm=True), dev)
        y = exl3.moe_tiled_with_shared_bank(x, td, sd, xi, sc, dec)
    ref = _two_calls_ragged(x, rb, sd, xi, sc, dec, form, td)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


# ---- configs[4]'s layer at a 1024-token prefill on the summand-relative bar ----------------------------------------
#
# Each token routes all 8 of its slots to one expert (scores summing to 1), so y = svh_down[e] * H(inner_down) of that
# expert is undone exactly (tests/test_gpu_parity.py routes the same way); 1024 tokens over 16 experts, half of them
# K1 and half K2 in the ragged form, give 512 slots per expert (two 256-row windows each).

C5_HIDDEN, C5_INTER, C5_TOKENS, C5_HIT = 4096, 2048, 1024, 16


def _c5_routing(seed, E, hit):
    rng = np.random.default_rng(seed)
    experts = rng.choice(hit, size=C5_TOKENS)
    sc = rng.uniform(0.5, 1.5, size=(C5_TOKENS, 8)).astype(np.float32)
    sc /= sc.sum(axis=1, keepdims=True)
    return experts, sc, sc.sum(axis=1, dtype=np.float64)[:, None]


def _c5_truth(weights_of, suh_svh_of, x, experts):
    """Exact down inner products at the chain's rounding points, rows grouped by expert (weights decoded once each)."""
    inner = np.zeros((len(experts), C5_HIDDEN))
    amag = np.zeros_like(inner)
    bound = np.zeros_like(inner)
    for e in np.unique(experts):
        rows = np.nonzero(experts == e)[0]
        wg, wu, wd = weights_of(int(e))
        sg, su, vg, vu, sd = suh_svh_of(int(e))
        gv = P.f16_bits(vg) * P.hadamard_blocks(P.prepared_rows(x[rows], sg) @ wg)
        uv = P.f16_bits(vu) * P.hadamard_blocks(P.prepared_rows(x[rows], su) @ wu)
        pd = P.down_prepared(gv, uv, sd)
        inner[rows] = pd @ wd
        amag[rows] = np.abs(pd) @ np.abs(wd)
        bound[rows] = np.abs(pd).max(axis=1, keepdims=True) * np.abs(wd).max(axis=0)
    return P.Truth(inner, amag, bound, C5_INTER, P.MID_ULPS)


@pytest.mark.parametrize("form", ["ragged", "tiled"])
def test_c5_prefill_1024_tokens_summand_bar_with_mutations(dev, form):
    print(f"[c5 prefill] {form} 1024 tokens", flush=True)
    dec, odec = DECODES["spec1"]
    E = 256
    x = synth.normal(99, "c5p.x", (C5_TOKENS, C5_HIDDEN))
    xf = x.float().numpy()
    hit = np.concatenate([np.arange(8), 64 + np.arange(8)]) if form == "ragged" else np.arange(C5_HIT) * 16
    experts_idx, sc, ssum = _c5_routing(99, E, C5_HIT)
    experts = hit[experts_idx]
    inds = torch.from_numpy(np.repeat(experts[:, None], 8, axis=1).astype(np.int32)).to(dev)
    scd = torch.from_numpy(sc).to(dev)
    dims = ((C5_HIDDEN, C5_INTER), (C5_HIDDEN, C5_INTER), (C5_INTER, C5_HIDDEN))
    if form == "ragged":
        g1 = synth.bank(99, "c5p.k1", 64, C5_HIDDEN, C5_INTER, 16, norm=True)
        g2 = synth.bank(99, "c5p.k2", 192, C5_HIDDEN, C5_INTER, 32, norm=True)
        rb = exl3.Ragged.init([_to(g1, dev), _to(g2, dev)])
        with exl3.arm_overrides(moe_gemm=1):
            y = exl3.moe_ragged(x.to(dev).float(), rb, inds, scd, dec).cpu().numpy().astype(np.float64)
        del rb

        def proj_of(e):
            return (g1, e) if e < 64 else (g2, e - 64)

        def weights_of(e, odecs=(odec, odec, odec), down=None):
            b, l = proj_of(e)
            ws = [P.decoded(_u16(q.trellis)[l], i, o, q.n, od) for q, (i, o), od in zip((b.gate, b.up, b.down), dims,
                                                                                      odecs)]
            if down is not None:
                ws[2] = P.decoded(down, C5_INTER, C5_HIDDEN, b.down.n, odecs[2])
            return ws

        def suh_svh_of(e):
            b, l = proj_of(e)
            return (_u16(b.gate.suh)[l], _u16(b.up.suh)[l], _u16(b.gate.svh)[l], _u16(b.up.svh)[l],
                    _u16(b.down.suh)[l])

        svh_down = lambda e: _u16(proj_of(e)[0].down.svh)[proj_of(e)[1]]  # noqa: E731
    else:
        tb = synth.tiled_bank(99, "c5p.t", E, C5_HIDDEN, C5_INTER, 0.25, norm=True)
        bpw = sum(p.bits_per_weight() for p in (tb.gate, tb.up, tb.down)) / 3
        assert abs(bpw - 1.75) < 0.01, bpw
        td = _to_tiled(tb, dev)
        with exl3.arm_overrides(moe_gemm=1):
            y = exl3.moe_tiled(x.to(dev).float(), td, inds, scd, dec).cpu().numpy().astype(np.float64)
        del td
        arrs = _tiled_arrays(tb)

        def weights_of(e, odecs=(odec, odec, odec), down=None):
            ws = [P.f16_bits(O.reconstruct_inner_tiled(a[0], a[1], a[2], e, i, o, 16, 32, od))
                  for a, (i, o), od in zip(arrs, dims, odecs)]
            if down is not None:
                a = arrs[2]
                ws[2] = P.f16_bits(O.reconstruct_inner_tiled(down, a[1], a[2], e, C5_INTER, C5_HIDDEN, 16, 32,
                                                             odecs[2]))
            return ws

        def suh_svh_of(e):
            return arrs[0][3][e], arrs[1][3][e], arrs[0][4][e], arrs[1][4][e], arrs[2][3][e]

        svh_down = lambda e: arrs[2][4][e]  # noqa: E731
    got = np.stack([P.inner_from_output(y[r] / ssum[r], svh_down(int(e))) for r, e in enumerate(experts)])
    cache = {}

    def cached(e):
        if e not in cache:
            cache[e] = weights_of(e)
        return cache[e]

    t = _c5_truth(cached, suh_svh_of, xf, experts)
    print(f"[parity] c5 prefill {form} worst error / ceiling = {P.worst_ratio(got, t):.4f}", flush=True)
    assert P.verdict(got, t) is None, P.verdict(got, t)
    # mutation arms on the rows of one expert of each rate: the wrong codeword window, then one flipped trellis bit
    w16 = P.mutated_window(odec)
    for e0 in (int(hit[0]), int(hit[-1])):
        rows = np.nonzero(experts == e0)[0]
        tw = _c5_truth(lambda e: weights_of(e, (w16, w16, w16)), suh_svh_of, xf[rows], experts[rows])
        assert P.verdict(got[rows], tw) is not None, e0
        rng = np.random.default_rng(e0)
        if form == "ragged":
            b, l = proj_of(e0)
            tr = _u16(b.down.trellis)[l]
            mut, where = P.flip_one_bit(tr, b.down.n, odec, np.ones((1, C5_INTER)), rng)
        else:
            a = arrs[2]
            base = P.f16_bits(O.reconstruct_inner_tiled(a[0], a[1], a[2], e0, C5_INTER, C5_HIDDEN, 16, 32, odec))
            mut = None
            for _ in range(2000):  # one bit of one tile of e0's down projection that moves a weight by >= 0.5
                tk, s, o = int(rng.integers(C5_INTER // 16)), int(rng.integers(C5_HIDDEN // 128)), int(rng.integers(8))
                m = int(a[2][e0, tk, s])
                hw = 2 * int(a[1][e0, tk, s]) + sum(16 if m >> q & 1 else 32 for q in range(o))
                hw += int(rng.integers(16 if m >> o & 1 else 32))
                cand = a[0].copy()
                cand[hw] ^= np.uint16(1 << int(rng.integers(16)))
                after = P.f16_bits(O.reconstruct_inner_tiled(cand, a[1], a[2], e0, C5_INTER, C5_HIDDEN, 16, 32, odec))
                if np.nanmax(np.abs(after - base)) >= 0.5:
                    mut, where = cand, (tk, s, o, hw)
                    break
            assert mut is not None
        tm = _c5_truth(lambda e: weights_of(e, down=mut), suh_svh_of, xf[rows], experts[rows])
        assert P.verdict(got[rows], tm) is not None, (e0, where)
