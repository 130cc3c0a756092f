"""The routed configurations at their full shapes against the oracle (max-abs-rel 2e-3).

configs[3] (C4): 256 routed experts + 1 shared, hidden 2048, inter 768, K2 MCG, top-8 over N(0,1) logits, batch 1 / 8 /
32 -- the shapes bench.py times, through the same calls (moe_with_shared_bank; and moe alone).  configs[4] (C5) in the
reference's rate-group form: 64 experts at K1 and 192 at K2 (1.75 bpw), SPEC1 with the spec1-w15 table, hidden 4096,
inter 2048, top-8, batch 64 on the sorted arm, plus a K4 shared expert; and as stated, a seeded per-tile K1 / K2 mix in
every expert (exl3.Tiled).  The oracle is moeSwigluHost
(src/exl3/expert_exl3_kernels.zig:3059-3114) over every row on the host's cores (ox_moe_swiglu_rows).  The banks'
svh carry 1/sqrt(in) (synth norm), so f16 outputs stay far from overflow.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3
THREADS = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)


def _np(p):
    return tuple(a.numpy().view(np.uint16) for a in (p.trellis, p.suh, p.svh))


def _to(b, dev):
    return exl3.Bank(*(exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev)) for p in (b.gate, b.up, b.down)))


def _cat(b, s):
    """Bank b with the one-expert bank s appended as its last expert (the oracle's shared-expert slot)."""
    return [tuple(np.concatenate([a, c]) for a, c in zip(_np(q), _np(qs)))
            for q, qs in ((b.gate, s.gate), (b.up, s.up), (b.down, s.down))]


@pytest.fixture(scope="module")
def c4(dev):
    E, hidden, inter = 256, 2048, 768
    b = synth.bank(3, "c4", E, hidden, inter, 32, norm=True)
    sh = synth.bank(3, "c4.shared", 1, hidden, inter, 32, norm=True)
    return b, sh, _to(b, dev), _to(sh, dev), _cat(b, sh)


@pytest.mark.parametrize("batch", [1, 8, 32])
def test_c4_layer_with_shared_expert(dev, c4, batch):
    print(f"[c4] batch={batch}", flush=True)
    b, sh, bd, shd, banks = c4
    E, hidden, inter, k = 256, 2048, 768, 8
    x = synth.normal(3, f"c4.t{batch}", (batch, hidden))
    logits = synth.normal(3, f"c4.tl{batch}", (batch, E), dtype=torch.float32)
    inds, scores = exl3.moe_routing_chain(logits.to(dev), k)
    oi, osc = O.route_topk(logits.numpy(), k)
    assert (inds.cpu().numpy().view(np.uint32) == oi).all()
    xd = x.to(dev)
    dec, odec = exl3.MCG, O.decode(O.CB_MCG)
    xf = x.float().numpy()
    routed = O.moe_swiglu_rows(xf, *banks, oi, osc, hidden, inter, (32, 32, 32), odec, threads=THREADS)
    shared = O.moe_swiglu_rows(xf, *banks, np.full((batch, 1), E), np.ones((batch, 1)), hidden, inter, (32, 32, 32),
                               odec, threads=THREADS)
    # moe alone (routed), then the layer with its shared expert: T(T(routed) + T(shared)) as the pair of calls rounds
    y = exl3.moe(xd, bd, inds, scores, dec).float().cpu().numpy()
    assert max_abs_rel(y, routed) < BAR
    y2 = exl3.moe_with_shared_bank(xd, bd, shd, inds, scores, dec).float().cpu().numpy()
    want = routed.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
    assert max_abs_rel(y2, want) < BAR


def test_c5_rate_group_layer_batch_64(dev):
    """configs[4] in the rate-group form: SPEC1 K1/K2 experts (a ragged bank), K4 shared expert, batch 64."""
    print("[c5] batch=64", flush=True)
    E1, E2, hidden, inter, k, batch = 64, 192, 4096, 2048, 8, 64
    dec, odec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)
    g1 = synth.bank(5, "c5.k1", E1, hidden, inter, 16, norm=True)
    g2 = synth.bank(5, "c5.k2", E2, hidden, inter, 32, norm=True)
    sh = synth.bank(5, "c5.shared", 1, hidden, inter, 64, norm=True)
    rb = exl3.Ragged.init([_to(g1, dev), _to(g2, dev)])
    x = synth.normal(5, "c5.t64", (batch, hidden))
    logits = synth.normal(5, "c5.tl64", (batch, E1 + E2), dtype=torch.float32)
    inds, scores = exl3.moe_routing_chain(logits.to(dev), k)
    oi, osc = O.route_topk(logits.numpy(), k)
    y = exl3.moe_ragged_with_shared_bank(x.to(dev), rb, _to(sh, dev), inds, scores, dec).float().cpu().numpy()
    xf = x.float().numpy()
    # the ragged bank as the oracle sees it: each projection's experts concatenated in expert order
    banks = []
    for nm in ("gate", "up", "down"):
        q1, q2 = getattr(g1, nm), getattr(g2, nm)
        t = np.concatenate([_np(q1)[0].reshape(-1), _np(q2)[0].reshape(-1)])
        banks.append((t, np.concatenate([_np(q1)[1], _np(q2)[1]]), np.concatenate([_np(q1)[2], _np(q2)[2]])))
    rates = [np.array([16] * E1 + [32] * E2)] * 3
    routed = O.moe_swiglu_rows(xf, *banks, oi, osc, hidden, inter, rates, odec, threads=THREADS)
    shared = O.moe_swiglu_rows(xf, *[_np(q) for q in (sh.gate, sh.up, sh.down)], np.zeros((batch, 1)),
                               np.ones((batch, 1)), hidden, inter, (64, 64, 64), odec, threads=THREADS)
    want = routed.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
    assert max_abs_rel(y, want) < BAR


def test_c5_per_tile_layer_batch_64(dev):
    """configs[4] as stated: every expert at a seeded per-tile K1 / K2 mix (25 % K1), SPEC1 (spec1-w15), hidden 4096,
    inter 2048, top-8 over 256 experts, batch 64 on the sorted arm, with a K4 shared expert in the same launches."""
    print("[c5] per-tile batch=64", flush=True)
    E, hidden, inter, k, batch = 256, 4096, 2048, 8, 64
    dec, odec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)
    tb = synth.tiled_bank(5, "c5t", E, hidden, inter, 0.25, device=dev, norm=True)
    sh = synth.bank(5, "c5.shared", 1, hidden, inter, 64, norm=True)
    bpw = sum(p.bits_per_weight() for p in (tb.gate, tb.up, tb.down)) / 3
    assert abs(bpw - 1.75) < 0.01, bpw
    x = synth.normal(5, "c5.t64", (batch, hidden))
    logits = synth.normal(5, "c5t.tl64", (batch, E), dtype=torch.float32)
    inds, scores = exl3.moe_routing_chain(logits.to(dev), k)
    oi, osc = O.route_topk(logits.numpy(), k)
    y = exl3.moe_tiled_with_shared_bank(x.to(dev), tb, _to(sh, dev), inds, scores, dec).float().cpu().numpy()
    arrs = [(p.trellis.cpu().numpy().view(np.uint16), p.seg_off.cpu().numpy().view(np.uint32), p.seg_k1.cpu().numpy(),
             p.suh.cpu().numpy().view(np.uint16), p.svh.cpu().numpy().view(np.uint16)) for p in (tb.gate, tb.up, tb.down)]
    del tb
    xf = x.float().numpy()
    routed = O.moe_swiglu_tiled_rows(xf, arrs, oi, osc, hidden, inter, 16, 32, odec, threads=THREADS)
    shared = O.moe_swiglu_rows(xf, *[_np(q) for q in (sh.gate, sh.up, sh.down)], np.zeros((batch, 1)),
                               np.ones((batch, 1)), hidden, inter, (64, 64, 64), odec, threads=THREADS)
    want = routed.astype(np.float16).astype(np.float32) + shared.astype(np.float16).astype(np.float32)
    assert max_abs_rel(y, want) < BAR


def test_c4_prefill_width_takes_the_gemm_arm(dev, c4):
    """configs[3]'s layer at a 512-token prefill (4096 slots, 16 per expert on average): the routed GEMM arm (taken
    by itself at this width) against the oracle, and equal to the decode chain at the bar."""
    print("[c4] prefill 512", flush=True)
    b, sh, bd, shd, banks = c4
    E, hidden, inter, k, batch = 256, 2048, 768, 8, 512
    x = synth.normal(3, "c4.p512", (batch, hidden))
    logits = synth.normal(3, "c4.pl512", (batch, E), dtype=torch.float32)
    inds, scores = exl3.moe_routing_chain(logits.to(dev), k)
    oi, osc = O.route_topk(logits.numpy(), k)
    y = exl3.moe(x.to(dev), bd, inds, scores, exl3.MCG).float().cpu().numpy()
    with exl3.arm_overrides(moe_gemm=0):
        y_chain = exl3.moe(x.to(dev), bd, inds, scores, exl3.MCG).float().cpu().numpy()
    routed = O.moe_swiglu_rows(x.float().numpy(), *banks, oi, osc, hidden, inter, (32, 32, 32), O.decode(O.CB_MCG),
                               threads=THREADS)
    assert max_abs_rel(y, routed) < BAR
    assert max_abs_rel(y, y_chain) < BAR
