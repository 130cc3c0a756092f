"""The summand-relative parity bar on the CPU: arithmetic of the kind a correct arm does passes, and the reference's
mutation arms -- one wrong weight, the wrong codeword window, one flipped trellis bit -- fail it (the reference's
pure-function check of its verdict, src/exl3/expert_exl3_kernels.zig:3372-3399, and its mutations, :3330-3352).
Every mutation is planted in the oracle's decode, on the CPU."""
import numpy as np
import pytest

import oracle as O
from tests import _parity as P


def _case(seed, rows, in_f, out_f, n, odec):
    rng = np.random.default_rng(seed)
    t = rng.integers(0, 1 << 16, size=(in_f // 16, out_f // 16, n), dtype=np.uint32).astype(np.uint16)
    suh = (np.where(rng.random(in_f) < 0.5, -1.0, 1.0) * rng.uniform(0.5, 1.5, in_f)).astype(np.float16)
    x = rng.standard_normal((rows, in_f)).astype(np.float16).astype(np.float32)
    p = P.prepared_rows(x, suh.view(np.uint16))
    w = P.decoded(t, in_f, out_f, n, odec)
    return rng, t, p, w


def _f32_arm(p, w, splits=4):
    """A correct arm's arithmetic: f32 partial sums over k splits, added in f32."""
    k = p.shape[1] // splits
    acc = np.zeros((p.shape[0], w.shape[1]), np.float32)
    for s in range(splits):
        acc += p[:, s * k:(s + 1) * k].astype(np.float32) @ w[s * k:(s + 1) * k].astype(np.float32)
    return acc.astype(np.float64)


@pytest.mark.parametrize("in_f,n,cb", [(128, 64, O.CB_MCG), (512, 48, O.CB_3INST), (2048, 32, O.CB_MUL1)])
def test_correct_f32_arithmetic_passes_and_each_mutation_fails(in_f, n, cb):
    odec = O.decode(cb)
    rng, t, p, w = _case(in_f + n, 3, in_f, 256, n, odec)
    truth = P.truth(p, w)
    got = _f32_arm(p, w)
    assert P.verdict(got, truth) is None
    assert P.worst_ratio(got, truth) < 0.25  # f32 accumulation sits well inside the ceiling

    # an input element one f16 ulp off (the kernel's FWHT order rounding the other way) still passes
    p2 = p.copy()
    j = int(np.argmax(np.abs(p2[0])))
    p2[0, j] = np.float64(np.nextafter(np.float16(p2[0, j]), np.float16(np.inf)))
    assert P.verdict(_f32_arm(p2, w), truth) is None

    # one wrong weight
    w2 = w.copy()
    w2[in_f // 2, 17] += 1.0
    assert P.verdict(_f32_arm(p, w2), truth).startswith("gross_element")

    # the reference reads the other window (w16 -> w15): the truth moves, the arm did not
    tw = P.truth(p, P.decoded(t, in_f, 256, n, P.mutated_window(odec)))
    assert P.verdict(got, tw) is not None

    # one flipped trellis bit in the truth's decode
    tm, where = P.flip_one_bit(t, n, odec, p, rng)
    assert P.verdict(got, P.truth(p, P.decoded(tm, in_f, 256, n, odec))) is not None, where


def test_non_finite_fails():
    odec = O.decode(O.CB_MCG)
    _, _, p, w = _case(1, 1, 128, 128, 32, odec)
    truth = P.truth(p, w)
    got = _f32_arm(p, w)
    got[0, 3] = np.nan
    assert P.verdict(got, truth) == "nonfinite"


def test_finish_inverts_exactly():
    """inner = H(y / svh) undoes y = svh * H(inner) (H orthonormal and symmetric)."""
    rng = np.random.default_rng(3)
    inner = rng.standard_normal((2, 256))
    svh = (np.where(rng.random(256) < 0.5, -1.0, 1.0) * rng.uniform(0.5, 1.5, 256)).astype(np.float16)
    y = P.f16_bits(svh.view(np.uint16)) * P.hadamard_blocks(inner)
    assert np.allclose(P.inner_from_output(y, svh.view(np.uint16)), inner, rtol=0, atol=1e-12)
    # and the orthonormal Hadamard is the oracle's hadamard128
    v = rng.standard_normal(128).astype(np.float32)
    assert np.allclose(P.hadamard_blocks(v), O.hadamard128(v), rtol=0, atol=1e-5)
