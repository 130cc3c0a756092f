"""Pins the oracle's arithmetic layer: Hadamard, project, decodeDense, the MoE host oracle, routing and layout.

Each restatement is checked against something independent of its own code: the reference's fixtures (`public`),
closed forms (Sylvester Hadamard, H*H = I) and numpy products built from the fixture/dense weights.
"""
import numpy as np
import pytest

import oracle as O
from tests._util import LINEAR_FIXTURES, f16_bits_to_f32, load_fixture, rel_rms

CB = {"mul1": O.CB_MUL1, "mcg": O.CB_MCG}


def _sylvester(n=128):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(n)


def test_hadamard128_is_the_scaled_sylvester_matrix():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(128).astype(np.float32)
    h = _sylvester()
    assert np.allclose(O.hadamard128(v), h @ v, atol=1e-5)
    assert np.allclose(O.hadamard128(O.hadamard128(v)), v, atol=1e-5)  # H is an involution
    assert np.allclose(O.fwht128(v), O.hadamard128(v), atol=1e-5)


@pytest.mark.parametrize("name,n,cb,w", LINEAR_FIXTURES)
def test_project_matches_dense_matvec_over_public(name, n, cb, w):
    """The reference's own bar (expert_exl3.zig:897-914): project() vs x . public, relRms < 0.02."""
    d = load_fixture(name)
    rng = np.random.default_rng(7)
    x = (rng.random(128, dtype=np.float32) * 2 - 1)
    dec = O.decode(CB[cb], w)
    y = O.project(x, d["trellis"], d["suh"], d["svh"], 128, 128, n, dec)
    dense = x.astype(np.float64) @ f16_bits_to_f32(d["public"]).astype(np.float64)
    assert rel_rms(y, dense) < 0.02


@pytest.mark.parametrize("name,n,cb,w", LINEAR_FIXTURES)
def test_decode_dense_is_suh_h_m_h_svh(name, n, cb, w):
    d = load_fixture(name)
    dec = O.decode(CB[cb], w)
    dense = O.decode_dense(d["trellis"], d["suh"], d["svh"], 128, 128, n, dec)
    m = f16_bits_to_f32(d["inner"]).astype(np.float64)
    h = _sylvester()
    want = np.diag(f16_bits_to_f32(d["suh"])) @ h @ m @ h @ np.diag(f16_bits_to_f32(d["svh"]))
    assert np.allclose(dense, want, atol=1e-4)
    # and it is the public matrix before its f16 rounding
    assert np.allclose(dense, f16_bits_to_f32(d["public"]), rtol=2e-3, atol=2e-4)


def _bank(rng, e, i, o, n):
    t = rng.integers(0, 1 << 16, size=(e, i // 16, o // 16, n), dtype=np.uint32).astype(np.uint16)
    su = (rng.choice([-1.0, 1.0], size=(e, i)) * rng.uniform(0.5, 1.5, size=(e, i))).astype(np.float16).view(np.uint16)
    sv = (rng.choice([-1.0, 1.0], size=(e, o)) * rng.uniform(0.5, 1.5, size=(e, o))).astype(np.float16).view(np.uint16)
    return t, su, sv


def test_project_rows_threads_give_the_same_bytes():
    rng = np.random.default_rng(11)
    t, su, sv = _bank(rng, 1, 256, 384, 48)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    dec = O.decode(O.CB_MCG)
    one = O.project_rows(x, t, su, sv, 256, 384, 48, dec, threads=1)
    many = O.project_rows(x, t, su, sv, 256, 384, 48, dec, threads=4)
    assert (one == many).all()


def test_moe_swiglu_host_against_numpy_over_dense_weights():
    rng = np.random.default_rng(5)
    e, hid, inter, n = 6, 256, 128, 32
    g, u, d = _bank(rng, e, hid, inter, n), _bank(rng, e, hid, inter, n), _bank(rng, e, inter, hid, n)
    dec = O.decode(O.CB_MCG)
    x = rng.standard_normal(hid).astype(np.float16).astype(np.float32)
    slots = np.array([4, 1, 3], np.uint32)
    wts = np.array([0.5, 0.3, 0.2], np.float32)
    y = O.moe_swiglu_host(x, g, u, d, slots, wts, hid, inter, (n, n, n), dec)

    def dense(p, ex, i, o):
        return O.decode_dense(p[0][ex], p[1][ex], p[2][ex], i, o, n, dec).astype(np.float64)

    want = np.zeros(hid)
    for s, w in zip(slots, wts):
        gy = x @ dense(g, s, hid, inter)
        uy = x @ dense(u, s, hid, inter)
        h = gy / (1 + np.exp(-gy)) * uy
        want += w * (h @ dense(d, s, inter, hid))
    assert rel_rms(y, want) < 5e-3


def test_moe_clamp_limits_gate_above_and_up_both_ways():
    rng = np.random.default_rng(6)
    e, hid, inter, n = 2, 128, 128, 32
    g, u, d = _bank(rng, e, hid, inter, n), _bank(rng, e, hid, inter, n), _bank(rng, e, inter, hid, n)
    dec = O.decode(O.CB_MCG)
    x = (4 * rng.standard_normal(hid)).astype(np.float16).astype(np.float32)
    a = O.moe_swiglu_host(x, g, u, d, [0, 1], [0.5, 0.5], hid, inter, (n, n, n), dec, clamp_limit=1.0)
    b = O.moe_swiglu_host(x, g, u, d, [0, 1], [0.5, 0.5], hid, inter, (n, n, n), dec)
    assert not np.allclose(a, b)


def test_route_topk_against_numpy():
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((5, 64)).astype(np.float32)
    logits[0, 3] = logits[0, 9] = 9.0  # a tie: the lower index comes first
    inds, scores = O.route_topk(logits, 8)
    for r in range(5):
        order = sorted(range(64), key=lambda i: (-logits[r, i], i))[:8]
        assert inds[r].tolist() == order
        p = np.exp(logits[r] - logits[r].max())
        p /= p.sum()
        assert np.allclose(scores[r], p[order] / p[order].sum(), rtol=1e-6)
    assert inds[0, 0] == 3 and inds[0, 1] == 9


def test_moe_swiglu_rows_is_the_host_function_row_by_row_uniform_and_ragged():
    """ox_moe_swiglu_rows (rows of moeSwigluHost, OpenMP over rows) equals the single-row function row by row, on a
    uniform bank and on a ragged one (experts at their own rates), and its threaded run gives the same bytes."""
    from sushi_amd import synth

    dec = O.decode(O.CB_SPEC1, 15, 1)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 256)).astype(np.float16).astype(np.float32)
    sl = rng.integers(0, 6, (5, 3))
    w = rng.random((5, 3)).astype(np.float32)
    b = synth.bank(3, "rows", 6, 256, 128, 32)
    banks = [tuple(a.numpy().view(np.uint16) for a in (q.trellis, q.suh, q.svh)) for q in (b.gate, b.up, b.down)]
    y = O.moe_swiglu_rows(x, *banks, sl, w, 256, 128, (32, 32, 32), dec, threads=4)
    assert np.array_equal(y, O.moe_swiglu_rows(x, *banks, sl, w, 256, 128, (32, 32, 32), dec, threads=1))
    for r in range(5):
        assert np.array_equal(y[r], O.moe_swiglu_host(x[r], *banks, sl[r], w[r], 256, 128, (32, 32, 32), dec))
    # ragged: experts 0..2 at n16, 3..5 at n32, one flat trellis per projection in expert order
    g1, g2 = synth.bank(5, "r1", 3, 256, 128, 16), synth.bank(5, "r2", 3, 256, 128, 32)
    rag = []
    for nm in ("gate", "up", "down"):
        q1, q2 = getattr(g1, nm), getattr(g2, nm)
        rag.append(tuple(np.concatenate([a1.numpy().view(np.uint16).reshape(-1), a2.numpy().view(np.uint16).reshape(-1)])
                         if i == 0 else np.concatenate([a1.numpy().view(np.uint16), a2.numpy().view(np.uint16)])
                         for i, (a1, a2) in enumerate(zip((q1.trellis, q1.suh, q1.svh), (q2.trellis, q2.suh, q2.svh)))))
    rates = [np.array([16] * 3 + [32] * 3)] * 3
    yr = O.moe_swiglu_rows(x, *rag, sl, w, 256, 128, rates, dec, threads=4)
    for r in range(5):
        want = np.zeros(256, np.float32)
        for k in range(3):
            e = int(sl[r, k])
            grp, local, n = (g1, e, 16) if e < 3 else (g2, e - 3, 32)
            one = [tuple(a.numpy().view(np.uint16)[local] for a in (q.trellis, q.suh, q.svh))
                   for q in (grp.gate, grp.up, grp.down)]
            want += w[r, k] * O.moe_swiglu_host(x[r], *one, [0], [1.0], 256, 128, (n, n, n), dec)
        assert np.array_equal(yr[r], want), r


def _gated_term_independent(g, sh, dtype):
    """The gated shared term restated with numpy float16 / torch bfloat16 rounding (not the oracle's helpers)."""
    import torch

    if dtype == 0:
        r = lambda v: np.float32(np.float16(np.float32(v)))  # noqa: E731
    else:
        r = lambda v: np.float32(torch.tensor(np.float32(v)).to(torch.bfloat16).float().item())  # noqa: E731
    ex = r(np.float32(np.exp(abs(np.float64(g)))))
    rc = r(np.float32(1.0) / r(np.float32(1.0) + ex))
    sig = rc if g < 0 else r(np.float32(1.0) - rc)
    return r(np.float32(sig) * np.float32(sh))


@pytest.mark.parametrize("dtype", [0, 1])
def test_gated_shared_term_every_gate_value(dtype):
    """ox_gated_shared_term (REDUCE_GATED_SHARED_SOURCE's rounding chain, expert_exl3_kernels.zig:2410-2431) over
    every non-NaN f16 (dtype 0) or bf16 (dtype 1) gate, against an independent rounding of the same chain, and the
    sigmoid's closed form to within T's rounding."""
    import torch

    bits = np.arange(1 << 16, dtype=np.uint32)
    if dtype == 0:
        g_all = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    else:
        g_all = (bits << 16).view(np.float32)
    g_all = g_all[~np.isnan(g_all)]
    rng = np.random.default_rng(dtype)
    for g in g_all[rng.permutation(g_all.size)[:3000]]:  # a sample with the independent (slow, per-value) restatement
        for sh in (1.0, -2.75, 0.3):
            got, want = O.gated_shared_term(float(g), sh, dtype), _gated_term_independent(float(g), sh, dtype)
            assert got == want or (np.isnan(got) and np.isnan(want)), (g, sh, got, want)
    ulp = 2.0 ** -10 if dtype == 0 else 2.0 ** -7
    big = np.log(65504.0) if dtype == 0 else np.log(np.finfo(np.float32).max)  # exp|g| past T's range
    for g in g_all[np.isfinite(g_all)][::7]:
        sig = O.gated_shared_term(float(g), 1.0, dtype)
        if abs(g) > big:  # T(exp|g|) is inf: the chain's sigmoid is exactly 0 below and 1 above
            assert sig == (0.0 if g < 0 else 1.0), (g, sig)
            continue
        exact = 1.0 / (1.0 + np.exp(-np.float64(g)))
        assert abs(sig - exact) <= 3 * ulp * max(exact, 2.0 ** -14) + 2.0 ** -24, (g, sig, exact)


def _nonfinite_logit_rows():
    rng = np.random.default_rng(12)
    rows = rng.standard_normal((6, 40)).astype(np.float32)
    rows[0, :] = np.nan                                   # all NaN
    rows[1, ::3] = np.nan                                 # partly NaN
    rows[2, :] = -np.inf                                  # all -inf
    rows[2, [5, 17]] = [1.0, -2.0]                        # mostly -inf: two finite experts
    rows[3, :] = -np.inf
    rows[3, 7] = np.nan                                   # -inf with one NaN
    rows[4, [0, 1, 2]] = np.inf                           # +inf ties: lowest index first
    rows[5, :] = 0.0                                      # every key tied
    return rows


def test_route_topk_non_finite_rows_pick_distinct_experts_in_range():
    """NaN selects as -inf and an expert is never picked twice, so every pick is a distinct index in range; the
    order is the stable descending sort of the keys (numpy's argsort, an independent statement)."""
    logits = _nonfinite_logit_rows()
    k = 8
    inds, scores = O.route_topk(logits, k)
    for r in range(logits.shape[0]):
        keys = np.where(np.isnan(logits[r]), -np.inf, logits[r]).astype(np.float64)
        want = np.argsort(-keys, kind="stable")[:k]
        assert inds[r].tolist() == want.tolist(), r
        assert len(set(inds[r].tolist())) == k and inds[r].max() < logits.shape[1]
    assert np.isnan(scores[[0, 1, 3]]).all()              # a NaN logit reaches the softmax
    assert np.isnan(scores[4]).all()                      # +inf - max(+inf) is NaN
    p = np.exp(np.array([0.0, -3.0]))                     # two finite experts carry all the mass, the rest none
    assert np.allclose(scores[2][:2], p / p.sum()) and (scores[2][2:] == 0).all()
    assert np.isfinite(scores[5]).all() and np.allclose(scores[5], 1.0 / k)


def test_tile_major_round_trip_and_reference_layout_case():  # layout.zig:160-175
    it, ot, n = 5, 4, 3
    src = np.arange(it * ot * n, dtype=np.uint16)
    dst = O.tile_major(src, it, ot, n)
    for pair in range(ot // 2):
        for tk in range(it):
            for o in range(2):
                want = src[(tk * ot + pair * 2 + o) * n:][:n]
                assert (dst[((pair * it + tk) * 2 + o) * n:][:n] == want).all()
    assert (O.tile_major_inverse(dst, it, ot, n) == src).all()
