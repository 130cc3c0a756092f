"""Shared test helpers: the reference's golden fixtures, error metrics."""
from __future__ import annotations

import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF_FIXTURES = os.path.join(GOLDEN, "ref")

# (file, n, codebook, window): the reference's fixture table (src/exl3/expert_exl3.zig:571-591, :864-997).
LINEAR_FIXTURES = [
    ("exl3_k4_linear", 64, "mul1", 16),
    ("exl3_k3_linear", 48, "mul1", 16),
    ("exl3_k2_linear", 32, "mul1", 16),
    ("exl3_k2p5_mcg_linear", 40, "mcg", 16),
    ("exl3_k3_mcg_linear", 48, "mcg", 16),
    ("exl3_k2p5_mcg_w12_linear", 40, "mcg", 12),
]


def load_fixture(name: str) -> dict:
    from safetensors.numpy import load_file

    d = load_file(os.path.join(REF_FIXTURES, name + ".safetensors"))
    out = {}
    for k, v in d.items():
        out[k] = v.view(np.uint16) if v.dtype in (np.float16, np.int16) else v
    return out


def f16_bits_to_f32(a) -> np.ndarray:
    return np.asarray(a, np.uint16).view(np.float16).astype(np.float32)


def max_abs_rel(got, want) -> float:
    """max |got - want| / max |want| -- the north-star tolerance metric (bar 2e-3)."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    assert np.isfinite(g).all(), "non-finite output"
    return float(np.max(np.abs(g - w)) / max(np.max(np.abs(w)), 1e-30))


def rel_rms(got, want) -> float:
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    return float(np.sqrt(np.sum((g - w) ** 2) / max(np.sum(w * w), 1e-30)))
