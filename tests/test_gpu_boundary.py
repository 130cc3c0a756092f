"""GPU tests of the boundary's MoE flags: speculative-verify rows and the gated shared expert of `moeRagged`.

* verify_rows: the reference sends verify rows down the decode chain at any width (`rows <= DECODE_ROWS_MAX or
  verify_rows`, src/exl3/root.zig:169, :602), so they round as decode rows do.  At a width where the routed GEMM arm
  engages (E = 8, 64 rows, top-8: 64 slots per expert) a verify call must equal the decode chain (the GEMM arm held
  off) bit for bit, for every MoE entry point, while the same call without the flag takes the GEMM arm.
* `moeRagged(..., verify_rows, shared, shared_gate)` (src/exl3/root.zig:582-644; the trunk's ragged call passes both,
  src/trunk.zig:4092): y = T(T(routed) + T(sigmoid(gate) * shared)) against the oracle's routed sum and its gated term.
"""
import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth
from tests._util import max_abs_rel

pytestmark = pytest.mark.gpu

BAR = 2e-3
DT_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _np(p):
    return tuple(a.numpy().view(np.uint16) for a in (p.trellis, p.suh, p.svh))


def _to(b, dev):
    return exl3.Bank(*(exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev)) for p in (b.gate, b.up, b.down)))


def _route(seed, rows, experts, k):
    logits = synth.normal(seed, "logits", (rows, experts), dtype=torch.float32).numpy()
    return O.route_topk(logits, k)


def _ragged_oracle_banks(banks):
    """A ragged bank as the oracle reads it: each projection's experts concatenated in expert order."""
    out = []
    for nm in ("gate", "up", "down"):
        qs = [getattr(b, nm) for b in banks]
        out.append((np.concatenate([_np(q)[0].reshape(-1) for q in qs]), np.concatenate([_np(q)[1] for q in qs]),
                    np.concatenate([_np(q)[2] for q in qs])))
    return out


def _verify_case(dev, variant):
    """(call(verify_rows) -> y) for one MoE entry point at E = 8, 64 rows, top-8."""
    E, hidden, inter, k, rows, n = 8, 256, 256, 8, 64, 32
    x = synth.normal(70, "vx", (rows, hidden)).to(dev)
    inds, scores = _route(70, rows, E, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    if variant in ("moe", "gated", "shared_bank"):
        bd = _to(synth.bank(70, "vb", E, hidden, inter, n, norm=True), dev)
        if variant == "moe":
            return lambda v: exl3.moe(x, bd, xi, sc, exl3.MCG, v)
        if variant == "gated":
            sh = synth.normal(71, "vsh", (rows, hidden)).to(dev)
            g = synth.normal(72, "vg", (rows, 1)).to(dev)
            return lambda v: exl3.moe_with_gated_shared(x, bd, xi, sc, exl3.MCG, v, sh, g)
        sd = _to(synth.bank(70, "vb.shared", 1, hidden, inter, n, norm=True), dev)
        return lambda v: exl3.moe_with_shared_bank(x, bd, sd, xi, sc, exl3.MCG, verify_rows=v)
    if variant in ("ragged", "ragged_shared_bank"):
        groups = [(3, (16, 16, 16)), (5, (32, 32, 32))]
        rb = exl3.Ragged.init([_to(synth.bank(73 + g, f"vr{g}", e, hidden, inter, r, norm=True), dev)
                               for g, (e, r) in enumerate(groups)])
        if variant == "ragged":
            return lambda v: exl3.moe_ragged(x, rb, xi, sc, exl3.MCG, v)
        sd = _to(synth.bank(75, "vr.shared", 1, hidden, inter, 64, norm=True), dev)
        return lambda v: exl3.moe_ragged_with_shared_bank(x, rb, sd, xi, sc, exl3.MCG, verify_rows=v)
    tb = synth.tiled_bank(76, "vt", E, hidden, inter, 0.25, device=dev, norm=True)
    if variant == "tiled":
        return lambda v: exl3.moe_tiled(x, tb, xi, sc, exl3.MCG, verify_rows=v)
    sd = _to(synth.bank(77, "vt.shared", 1, hidden, inter, 32, norm=True), dev)
    return lambda v: exl3.moe_tiled_with_shared_bank(x, tb, sd, xi, sc, exl3.MCG, verify_rows=v)


VARIANTS = ["moe", "gated", "shared_bank", "ragged", "ragged_shared_bank", "tiled", "tiled_shared_bank"]


@pytest.mark.parametrize("variant", VARIANTS)
def test_verify_rows_equal_the_decode_chain(dev, variant):
    print(f"[verify] {variant}", flush=True)
    call = _verify_case(dev, variant)
    y_verify = call(True)
    with exl3.arm_overrides(moe_gemm=0):
        y_chain = call(False)
    torch.cuda.synchronize()
    assert torch.equal(y_verify, y_chain)
    # without the flag the layer takes the GEMM arm (rounded differently, within the bar of the chain)
    y_gemm = call(False)
    assert not torch.equal(y_gemm, y_chain)
    assert max_abs_rel(y_gemm.float().cpu().numpy(), y_chain.float().cpu().numpy()) < BAR


@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows", [3, 24])
def test_moe_ragged_gated_shared_against_oracle(dev, rows, ydt):
    """Ragged bank (two rate groups) with a gated shared expert: 3 rows fold the gated term into the down
    projection's completing arrival (16-bit y) or the reduce (f32 y); 24 rows run the expert windows."""
    print(f"[ragged gated] rows={rows} {ydt}", flush=True)
    hidden, inter, k = 256, 256, 4
    groups = [(6, (32, 32, 48)), (10, (16, 16, 32))]
    banks = [synth.bank(80 + g, f"rgs{g}", e, hidden, inter, r, norm=True) for g, (e, r) in enumerate(groups)]
    rb = exl3.Ragged.init([_to(b, dev) for b in banks])
    E = sum(e for e, _ in groups)
    x = synth.normal(80, "x", (rows, hidden)).to(ydt)
    inds, scores = _route(80 + rows, rows, E, k)
    shared = synth.normal(81, "sh", (rows, hidden)).to(ydt)
    gate = (synth.normal(82, "g", (rows, 1)) * 3).to(ydt)
    y = exl3.moe_ragged(x.to(dev), rb, torch.from_numpy(inds.view(np.int32)).to(dev),
                        torch.from_numpy(scores).to(dev), exl3.MCG, False, shared.to(dev), gate.to(dev))
    rates = [np.concatenate([np.full(e, r[i]) for e, r in groups]) for i in range(3)]
    routed = O.moe_swiglu_rows(x.float().numpy(), *_ragged_oracle_banks(banks), inds, scores, hidden, inter, rates,
                               O.decode(O.CB_MCG), threads=8)
    routed_t = torch.from_numpy(routed).to(ydt).float().numpy()
    term = O.gated_shared_terms(gate.float().numpy()[:, 0], shared.float().numpy(), DT_CODE[ydt])
    want = torch.from_numpy((routed_t + term).astype(np.float32)).to(ydt).float().numpy()
    # bf16: the kernel's routed sum and the oracle's may round one bf16 ulp apart, and the final rounding another
    bar = BAR + (2 * 2.0 ** -8 if ydt == torch.bfloat16 else 0.0)
    assert max_abs_rel(y.float().cpu().numpy(), want) < bar
    # the gate is live: the ungated add differs
    y_plain = exl3.moe_ragged(x.to(dev), rb, torch.from_numpy(inds.view(np.int32)).to(dev),
                              torch.from_numpy(scores).to(dev), exl3.MCG, False, shared.to(dev))
    assert max_abs_rel(y_plain.float().cpu().numpy(), want) > 10 * bar


def test_moe_ragged_gate_needs_its_shared_expert(dev):
    hidden, inter = 256, 128
    rb = exl3.Ragged.init([_to(synth.bank(83, "rgn", 4, hidden, inter, 32), dev)])
    x = synth.normal(83, "x", (2, hidden)).to(dev)
    inds, scores = _route(83, 2, 4, 2)
    g = torch.zeros(2, 1, dtype=torch.float16, device=dev)
    with pytest.raises(exl3.BadExl3Shape):
        exl3.moe_ragged(x, rb, torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev),
                        exl3.MCG, False, None, g)


# ---- linearPair (src/exl3/linear.zig:60-95) and moeGroups (src/exl3/root.zig:646-703) ----------------------------


def _proj(seed, name, groups, in_f, out_f, n, dev):
    p = synth.proj(seed, name, groups, in_f, out_f, n, norm=True)
    return p, exl3.Proj(p.trellis.to(dev), p.suh.to(dev), p.svh.to(dev))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("groups,rows", [(2, 1), (4, 3), (3, 16)])
def test_linear_pair_is_grouped_then_linear(dev, groups, rows, dtype):
    """x [G, rows, in] through the G-bank a, read as [rows, G * mid] by the one-bank b: bit-equal to linear_grouped,
    the transpose and linear; and against the oracle's projections (the intermediate rounded to x's dtype) at the
    north-star bar."""
    print(f"[linear pair] G={groups} rows={rows} {dtype}", flush=True)
    in_f, mid, out_f = 256, 384, 512
    pa, a = _proj(84, f"lpa{groups}", groups, in_f, mid, 48, dev)
    pb, b = _proj(85, f"lpb{groups}", 1, groups * mid, out_f, 32, dev)
    dec_a, dec_b = exl3.MCG, exl3.INST3
    x = synth.normal(84, f"lpx{groups}.{rows}", (groups, rows, in_f)).to(dtype).to(dev)
    y = exl3.linear_pair(x, a, b, dec_a, dec_b)
    mid_t = exl3.linear_grouped(x, a, dec_a).transpose(0, 1).reshape(rows, groups * mid).contiguous()
    ref = exl3.linear(mid_t, b, dec_b)
    torch.cuda.synchronize()
    assert y is not None and y.dtype == dtype and torch.equal(y, ref)
    xa = x.float().cpu().numpy()
    hs = []
    for g in range(groups):
        t, su, sv = _np(pa)
        hs.append(O.project_rows(xa[g], t[g], su[g], sv[g], in_f, mid, 48, O.decode(O.CB_MCG), threads=8))
    h = torch.from_numpy(np.concatenate(hs, axis=1)).to(dtype).float().numpy()
    t, su, sv = _np(pb)
    want = O.project_rows(h, t[0], su[0], sv[0], groups * mid, out_f, 32, O.decode(O.CB_3INST), threads=8)
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR + (2 ** -8 if dtype == torch.bfloat16 else 0.0)


def test_linear_pair_declines_past_one_decode_launch(dev):
    in_f, mid, out_f, groups, rows = 256, 128, 256, 2, 17
    _, a = _proj(86, "lpd.a", groups, in_f, mid, 32, dev)
    _, b = _proj(86, "lpd.b", 1, groups * mid, out_f, 32, dev)
    x = synth.normal(86, "lpd.x", (groups, rows, in_f)).to(dev)
    assert exl3.linear_pair(x, a, b, exl3.MCG, exl3.MCG) is None


def _group_banks(dev, seed, groups, hidden, inter):
    banks = [synth.bank(seed + g, f"mg{seed}.{g}", e, hidden, inter, n, norm=True) for g, (e, n) in enumerate(groups)]
    return banks, [_to(b, dev) for b in banks]


@pytest.mark.parametrize("rows", [1, 5, 24])
@pytest.mark.parametrize("ydt", [torch.float16, torch.float32])
def test_moe_groups_against_oracle(dev, rows, ydt):
    """Three uniform banks (3, 5 and 8 experts at K2, K3, K4): each group's partial in f32 over every slot (slots of
    other groups as local expert 0 with score 0), summed in group order and rounded once -- the oracle does the same
    with moeSwigluHost per group."""
    print(f"[moe groups] rows={rows} {ydt}", flush=True)
    hidden, inter, k = 256, 256, 4
    groups = [(3, 32), (5, 48), (8, 64)]
    banks, bds = _group_banks(dev, 87, groups, hidden, inter)
    E = sum(e for e, _ in groups)
    x = synth.normal(87, f"x{rows}", (rows, hidden)).to(ydt)
    inds, scores = _route(87 + rows, rows, E, k)
    y = exl3.moe_groups(x.to(dev), bds, torch.from_numpy(inds.view(np.int32)).to(dev),
                        torch.from_numpy(scores).to(dev), exl3.MCG)
    total = np.zeros((rows, hidden), np.float32)
    lo = 0
    for b, (e, n) in zip(banks, groups):
        inside = (inds >= lo) & (inds < lo + e)
        local = np.where(inside, inds - lo, 0).astype(np.uint32)
        w = np.where(inside, scores, 0.0).astype(np.float32)
        total += O.moe_swiglu_rows(x.float().numpy(), _np(b.gate), _np(b.up), _np(b.down), local, w, hidden, inter,
                                   (n, n, n), O.decode(O.CB_MCG), threads=8)
        lo += e
    want = torch.from_numpy(total).to(ydt).float().numpy()
    assert max_abs_rel(y.float().cpu().numpy(), want) < BAR


def test_moe_groups_of_one_bank_is_moe_and_verify_rows_hold(dev):
    """One bank is `moe` itself (root.zig:648), bit for bit; and verify rows at a GEMM-arm width equal the decode
    chain bit for bit through the group path as well."""
    hidden, inter, k, rows = 256, 256, 8, 64
    banks, bds = _group_banks(dev, 88, [(8, 32)], hidden, inter)
    x = synth.normal(88, "x", (rows, hidden)).to(dev)
    inds, scores = _route(88, rows, 8, k)
    xi, sc = torch.from_numpy(inds.view(np.int32)).to(dev), torch.from_numpy(scores).to(dev)
    assert torch.equal(exl3.moe_groups(x, bds, xi, sc, exl3.MCG), exl3.moe(x, bds[0], xi, sc, exl3.MCG))
    banks2, bds2 = _group_banks(dev, 89, [(3, 32), (5, 32)], hidden, inter)
    yv = exl3.moe_groups(x, bds2, xi, sc, exl3.MCG, verify_rows=True)
    with exl3.arm_overrides(moe_gemm=0):
        yc = exl3.moe_groups(x, bds2, xi, sc, exl3.MCG)
    torch.cuda.synchronize()
    assert torch.equal(yv, yc)
