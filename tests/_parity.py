"""Summand-relative parity for the trellis kernels, with the reference's mutation arms.

The reference scores a GEMM/GEMV arm against the exact dot product of the same decoded weights, relative to the
SUMMANDS (sum |w_i x_i|), because a trellis dot product cancels and a bar written against the result measures noise
(src/exl3/expert_exl3_kernels.zig:3310-3330).  It then injects a defect between the arm and its reference -- the
wrong codeword window, or one flipped trellis bit -- to show the bar FAILS on a wrong arm and not only passes on a
right one (:3330-3352), over PARITY_SEEDS = 8 seeds (:4550).

Here the arms finish in the same launch (output FWHT-128 and svh), so the test reads f32 outputs and undoes the
finish exactly in f64: y = svh * H(inner) with H the orthonormal Sylvester matrix (symmetric, H H = I), so
inner = H(y / svh).  Each element of that inner is compared with the f64 dot product of the oracle's decoded f16
weights and the oracle's prepared input, relative to that element's sum |x_k w_kj|.  Unlike the north-star bar
(max-abs-rel 2e-3 of the output), this bar sees one wrong weight: it moves one inner element by |dw x_k|, about
1 / (0.64 depth) of its summand scale, far above the ceiling below.

The element ceiling has two terms:
  * f32 accumulation: ACC_FACTOR * sqrt(depth) * 2^-24 of the summand scale (a random walk over `depth` f32 adds,
    with a wide margin);
  * the prepared input: the kernel and the oracle round H(x * suh) to f16 after summing in different orders, so an
    input element can land one f16 ulp apart; that moves an output by at most 2^-11 |x_k| |w_kj|, bounded by
    PREP_ULPS * 2^-11 * max|x| * max_k |w_kj| per element.  The routed chain's down input (the SwiGLU mid) is built
    from gate / up sums of depth `hidden` held in f32, so its rounding lands apart more often: MID_ULPS.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import scipy.linalg

import oracle as O

PARITY_SEEDS = 8
U_F32 = 2.0 ** -24
U_F16 = 2.0 ** -11
ACC_FACTOR = 4.0
PREP_ULPS = 4.0
MID_ULPS = 8.0

_H128 = scipy.linalg.hadamard(128).astype(np.float64) / np.sqrt(128.0)


def f16_bits(a) -> np.ndarray:
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float64)


def hadamard_blocks(v: np.ndarray) -> np.ndarray:
    """The orthonormal 128-point Hadamard over each 128-block of the last axis, in f64."""
    v = np.asarray(v, np.float64)
    shp = v.shape
    return (v.reshape(*shp[:-1], shp[-1] // 128, 128) @ _H128).reshape(shp)


def inner_from_output(y, svh_bits) -> np.ndarray:
    """Undoes finishOutput on f32 outputs: inner = H(y / svh), exact up to y's own f32 rounding."""
    return hadamard_blocks(np.asarray(y, np.float64) / f16_bits(svh_bits))


def prepared_rows(x, suh_bits) -> np.ndarray:
    """The oracle's prepareInput (f16(H128(f16(x) * suh)), src/exl3/expert_exl3.zig:490-501) of every row, in f64."""
    x = np.asarray(x, np.float32).reshape(-1, np.asarray(suh_bits).size)
    return np.stack([O.prepare_input(r, suh_bits) for r in x]).astype(np.float64)


@dataclass
class Truth:
    inner: np.ndarray   # exact f64 dot products [rows, out]
    amag: np.ndarray    # sum_k |x_k w_kj| [rows, out]
    bound: np.ndarray   # max|x| * max_k |w_kj| [rows, out]: the largest summand's bound
    depth: int
    prep_ulps: float = PREP_ULPS  # f16 ulps of the largest summand the prepared input may move an element


def truth(p: np.ndarray, w: np.ndarray) -> Truth:
    """Exact products of prepared rows p [rows, in] and decoded weights w [in, out] (f64; an f16 x f16 product is
    exact in f64, so these sums are the dot products up to f64's own rounding)."""
    return Truth(p @ w, np.abs(p) @ np.abs(w), np.abs(p).max(axis=1, keepdims=True) * np.abs(w).max(axis=0),
                 int(w.shape[0]))


def ceiling(t: Truth) -> np.ndarray:
    """Per-element bar on |got - exact| in units of that element's summand scale."""
    prep = t.prep_ulps * U_F16 * t.bound / np.maximum(t.amag, 1e-30)
    return ACC_FACTOR * np.sqrt(t.depth) * U_F32 + prep


def verdict(got_inner: np.ndarray, t: Truth) -> Optional[str]:
    """None when the arm passes; else why it failed ("nonfinite" or "gross_element: ...")."""
    g = np.asarray(got_inner, np.float64)
    if not np.isfinite(g).all() or not np.isfinite(t.inner).all():
        return "nonfinite"
    e = np.abs(g - t.inner) / np.maximum(t.amag, 1e-30)
    c = ceiling(t)
    if (e > c).any():
        i = np.unravel_index(np.argmax(e / c), e.shape)
        return f"gross_element at {tuple(int(v) for v in i)}: {e[i]:.3e} > {c[i]:.3e}"
    return None


def worst_ratio(got_inner: np.ndarray, t: Truth) -> float:
    """max over elements of error / ceiling (< 1 passes): how much room the arm leaves."""
    e = np.abs(np.asarray(got_inner, np.float64) - t.inner) / np.maximum(t.amag, 1e-30)
    return float(np.max(e / ceiling(t)))


# ---- mutations (src/exl3/expert_exl3_kernels.zig:3330-3352) -----------------------------------------------------


def mutated_window(odec: "O.Decode") -> "O.Decode":
    """The reference reads another codeword window than the pack names: w16 <-> w15 (mutatedDecode, :3346-3349)."""
    return O.decode(odec.codebook, 15 if odec.window_bits == 16 else 16, odec.table)


def decoded(trellis: np.ndarray, in_f: int, out_f: int, n: int, odec: "O.Decode") -> np.ndarray:
    return f16_bits(O.reconstruct_inner(trellis, in_f, out_f, n, odec))


def flip_one_bit(trellis: np.ndarray, n: int, odec: "O.Decode", p: np.ndarray, rng: np.random.Generator,
                 min_effect: float = 0.5):
    """One bit of one trellis halfword flipped, which moves the weights whose sliding window covers it.  The bit is
    drawn at random until the flip moves some weight w_kj by |dw| * max|x_k| >= min_effect (a defect of ordinary
    size, not one the decoder's masks happen to hide).  Returns (mutated copy, (tile k, tile n, halfword, bit))."""
    it, ot = trellis.shape[0], trellis.shape[1]
    xk = np.abs(p).max(axis=0)  # over rows, per input
    for _ in range(10000):
        tk, tn, hw, bit = int(rng.integers(it)), int(rng.integers(ot)), int(rng.integers(n)), int(rng.integers(16))
        tile = trellis[tk, tn].copy()
        before = f16_bits(O.decode_tile(tile, n, odec)).reshape(16, 16)
        tile[hw] ^= np.uint16(1 << bit)
        after = f16_bits(O.decode_tile(tile, n, odec)).reshape(16, 16)
        effect = np.abs(after - before) * xk[tk * 16:tk * 16 + 16, None]
        if np.nanmax(effect) >= min_effect:
            m = trellis.copy()
            m[tk, tn, hw] ^= np.uint16(1 << bit)
            return m, (tk, tn, hw, bit)
    raise AssertionError("no single-bit flip moved a weight")


def with_inner(t: Truth, inner: np.ndarray) -> Truth:
    """A mutated truth: the same summand scale, other exact products."""
    return Truth(inner, t.amag, t.bound, t.depth, t.prep_ulps)


def flipped_truth(t: Truth, p: np.ndarray, trellis: np.ndarray, n: int, odec: "O.Decode", rng: np.random.Generator):
    """The truth of `t` after one flipped trellis bit (flip_one_bit), recomputed for the one tile it touches."""
    _, (tk, tn, hw, bit) = flip_one_bit(trellis, n, odec, p, rng)
    tile = trellis[tk, tn].copy()
    before = f16_bits(O.decode_tile(tile, n, odec)).reshape(16, 16)
    tile[hw] ^= np.uint16(1 << bit)
    after = f16_bits(O.decode_tile(tile, n, odec)).reshape(16, 16)
    inner = t.inner.copy()
    inner[:, tn * 16:tn * 16 + 16] += p[:, tk * 16:tk * 16 + 16] @ (after - before)
    return with_inner(t, inner), (tk, tn, hw, bit)


def silu(g: np.ndarray) -> np.ndarray:
    return g / (1.0 + np.exp(-g))


def down_prepared(g: np.ndarray, u: np.ndarray, suh_down_bits, clamp_limit: float = 0.0) -> np.ndarray:
    """The routed chain's mid (DOWN_FUSED_SOURCE, src/exl3/expert_exl3_kernels.zig:1838-1925): gate and up stay
    unrounded, the gate is clamped from above and up both ways when a limit is set, SiLU(gate) * up * suh_down goes
    through the Hadamard and is rounded to f16 once, as the down projection's prepared input."""
    if clamp_limit > 0:
        g = np.minimum(g, clamp_limit)
        u = np.clip(u, -clamp_limit, clamp_limit)
    h = silu(g) * u * f16_bits(suh_down_bits)
    return hadamard_blocks(h).astype(np.float16).astype(np.float64)
