"""Pins the oracle's per-tile-rate functions (configs[4]'s K1 / K2 tile mix, a layout extension with no reference
counterpart) and the host packer that lays such a bank out (exl3.TiledProj.pack).

The tile arithmetic is decodeTile's at each tile's own rate (src/exl3/expert_exl3.zig:338-357), which the golden
vectors pin (test_oracle_format.py); what is new is the layout, so every check here rebuilds the expected result
from the UNPACKED per-tile codes (never from the flat stream and its segment tables):
  * reconstruct_inner_tiled equals the weights reassembled tile by tile with decode_tile at the map's rate;
  * with a one-rate map the tiled functions equal the uniform ones (reconstruct_inner, project, moe_swiglu_rows);
  * project_tiled equals finishOutput(f16(prepared x . W)) over those reassembled weights;
  * moe_swiglu_tiled_rows equals a numpy SwiGLU over project_tiled.
"""
import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3, synth

DEC = O.decode(O.CB_SPEC1, 15, 1)


def _np(t: torch.Tensor) -> np.ndarray:
    """Codes and f16 scales as u16 bits (what the oracle takes)."""
    return t.cpu().numpy().view(np.uint16) if t.dtype in (torch.int16, torch.float16) else t.cpu().numpy()


def _mixed(seed, e, in_f, out_f, p_k1=0.25):
    """A packed per-tile-rate projection with its unpacked codes [E, IT, OT, 32] and rate map."""
    shape = (e, in_f // 16, out_f // 16)
    k1 = synth.tile_map(seed, "otl.k1", shape, p_k1)
    cb = synth.codes(seed, "otl.tr", shape + (32,))
    su = synth.sign_scale(seed, "otl.suh", (e, in_f))
    sv = synth.sign_scale(seed, "otl.svh", (e, out_f))
    return exl3.TiledProj.pack(cb[..., :16], cb, k1, su, sv), _np(cb), k1.numpy()


def _arrays(tp):
    return _np(tp.trellis), tp.seg_off.numpy().view(np.uint32), tp.seg_k1.numpy()


def _reassembled(codes, k1, e, dec=DEC) -> np.ndarray:
    it, ot = k1.shape[1], k1.shape[2]
    out = np.zeros((it * 16, ot * 16), np.uint16)
    for tk in range(it):
        for tn in range(ot):
            n = 16 if k1[e, tk, tn] else 32
            out[tk * 16:tk * 16 + 16, tn * 16:tn * 16 + 16] = O.decode_tile(codes[e, tk, tn, :n], n, dec).reshape(16, 16)
    return out


def test_pack_layout_and_realised_rate():
    tp, codes, k1 = _mixed(1, 2, 256, 256)
    tr, off, msk = _arrays(tp)
    e, it, ot = k1.shape
    assert tr.size == int(np.where(k1, 16, 32).sum())
    assert tp.bits_per_weight() == pytest.approx(16 * tr.size / (e * it * ot * 256))
    assert 1.5 < tp.bits_per_weight() < 2.0
    # segment masks are the map's bits; the first segment starts at word 0; in (e, s, tk) order each segment's words
    # follow the last's, so a column group's k-tile rows are one run of the stream
    bits = (k1.reshape(e, it, ot // 8, 8) << np.arange(8)).sum(-1)
    assert (msk == bits).all()
    seg_words = np.where(k1, 8, 16).reshape(e, it, ot // 8, 8).sum(-1).transpose(0, 2, 1).reshape(-1)
    assert (off.transpose(0, 2, 1).reshape(-1) == np.concatenate([[0], np.cumsum(seg_words)[:-1]])).all()
    # a K1 tile holds the first 16 halfwords of its draw, a K2 tile all 32, at its place in the stream
    hw = 2 * int(off[1, 3, 1])
    for o in range(8):
        tn = 8 + o
        n = 16 if k1[1, 3, tn] else 32
        assert (tr[hw:hw + n] == codes[1, 3, tn, :n]).all()
        hw += n


@pytest.mark.parametrize("cb", ["spec1", "mcg", "3inst"])
def test_reconstruct_tiled_is_per_tile_decode(cb):
    dec = {"spec1": DEC, "mcg": O.decode(O.CB_MCG), "3inst": O.decode(O.CB_3INST)}[cb]
    tp, codes, k1 = _mixed(2, 2, 128, 256)
    tr, off, msk = _arrays(tp)
    for e in range(2):
        got = O.reconstruct_inner_tiled(tr, off, msk, e, 128, 256, 16, 32, dec)
        assert np.array_equal(got, _reassembled(codes, k1, e, dec)), e


@pytest.mark.parametrize("p_k1,n", [(0.0, 32), (1.0, 16)])
def test_one_rate_maps_are_the_uniform_functions(p_k1, n):
    tp, codes, k1 = _mixed(3, 2, 256, 128, p_k1)
    assert k1.all() if n == 16 else not k1.any()
    tr, off, msk = _arrays(tp)
    su, sv = _np(tp.suh), _np(tp.svh)
    x = synth.normal(3, "otl.x", (256,)).float().numpy()
    for e in range(2):
        uni = np.ascontiguousarray(codes[e, :, :, :n])
        assert np.array_equal(O.reconstruct_inner_tiled(tr, off, msk, e, 256, 128, 16, 32, DEC),
                              O.reconstruct_inner(uni, 256, 128, n, DEC))
        assert np.array_equal(O.project_tiled(x, tr, off, msk, e, su[e], sv[e], 256, 128, 16, 32, DEC),
                              O.project(x, uni, su[e], sv[e], 256, 128, n, DEC))


def test_project_tiled_over_reassembled_weights():
    tp, codes, k1 = _mixed(4, 3, 256, 256)
    tr, off, msk = _arrays(tp)
    su, sv = _np(tp.suh), _np(tp.svh)
    x = synth.normal(4, "otl.x2", (256,)).float().numpy()
    for e in range(3):
        got = O.project_tiled(x, tr, off, msk, e, su[e], sv[e], 256, 256, 16, 32, DEC)
        w = _reassembled(codes, k1, e).view(np.float16).astype(np.float64)
        inner = (O.prepare_input(x, su[e]).astype(np.float64) @ w).astype(np.float32)
        want = O.finish_output(inner.astype(np.float16).astype(np.float32), sv[e])
        # the oracle sums in f32 tile by tile; its f16 inner may sit one ulp from the f64 sum's
        assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max(), e


def test_moe_swiglu_tiled_rows_uniform_and_mixed():
    hidden, inter, E = 256, 128, 4
    projs = [_mixed(5 + i, E, *shape) for i, shape in enumerate([(hidden, inter), (hidden, inter), (inter, hidden)])]
    arrs = [(*_arrays(tp), _np(tp.suh), _np(tp.svh)) for tp, _, _ in projs]
    rng = np.random.default_rng(5)
    x = synth.normal(5, "otl.x3", (3, hidden)).float().numpy()
    sl = rng.integers(0, E, (3, 2)).astype(np.uint32)
    w = rng.random((3, 2)).astype(np.float32)
    y = O.moe_swiglu_tiled_rows(x, arrs, sl, w, hidden, inter, 16, 32, DEC, threads=3)
    assert np.array_equal(y, O.moe_swiglu_tiled_rows(x, arrs, sl, w, hidden, inter, 16, 32, DEC, threads=1))
    for r in range(3):
        want = np.zeros(hidden, np.float32)
        for k in range(2):
            e = int(sl[r, k])
            pt = lambda v, a, i, o: O.project_tiled(v, a[0], a[1], a[2], e, a[3][e], a[4][e], i, o, 16, 32, DEC)  # noqa: E731
            g, u = pt(x[r], arrs[0], hidden, inter), pt(x[r], arrs[1], hidden, inter)
            h = (g / (np.float32(1) + np.exp(-g))) * u
            want += w[r, k] * pt(h.astype(np.float32), arrs[2], inter, hidden)
        assert np.allclose(y[r], want, rtol=1e-5, atol=1e-5 * np.abs(want).max()), r
    # a one-rate (K2) bank: the uniform rows function, byte for byte
    uni = [_mixed(9 + i, E, *shape, p_k1=0.0) for i, shape in enumerate([(hidden, inter), (hidden, inter),
                                                                         (inter, hidden)])]
    ua = [(*_arrays(tp), _np(tp.suh), _np(tp.svh)) for tp, _, _ in uni]
    banks = [(np.ascontiguousarray(c), _np(tp.suh), _np(tp.svh)) for tp, c, _ in uni]
    yt = O.moe_swiglu_tiled_rows(x, ua, sl, w, hidden, inter, 16, 32, DEC)
    assert np.array_equal(yt, O.moe_swiglu_rows(x, *banks, sl, w, hidden, inter, (32, 32, 32), DEC))
