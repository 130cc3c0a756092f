"""Seeded synthetic banks and activations (the counterpart of src/exl3/synth.zig, with a reproducible generator).

Every tensor comes from its own SplitMix64 stream, seed = mix(config seed, tensor name), so a tensor depends only on
(seed, name, shape) and not on generation order.  Integer streams (codes, signs) are bit-identical on CPU and GPU;
floating ones (N(0,1) activations, U(0.5,1.5) scales) are produced on the CPU and copied, so every consumer sees the
same bytes.

  codes  : uniform u16, 4 per 64-bit draw (little-endian halfwords)
  suh/svh: sign (+-1, from bit 63) x U(0.5, 1.5), rounded to f16
  x      : N(0, 1) by Box-Muller over two uniform draws, rounded to f16
  k1 map : a tile is K1 where its U[0, 1) draw is below p_k1 (configs[4]: 0.25), else K2
"""
from __future__ import annotations

import math

import torch

_GOLDEN = 0x9E3779B97F4A7C15
_M1 = 0xBF58476D1CE4E5B9
_M2 = 0x94D049BB133111EB
_MASK64 = (1 << 64) - 1


def _i64(v: int) -> int:
    v &= _MASK64
    return v - (1 << 64) if v >= (1 << 63) else v


def _srl(z: torch.Tensor, s: int) -> torch.Tensor:
    """Logical right shift of int64 lanes holding u64 bits."""
    return (z >> s) & ((1 << (64 - s)) - 1)


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & _MASK64
    return h


def seed_of(seed: int, name: str) -> int:
    return ((seed * _GOLDEN) ^ fnv1a64(name)) & _MASK64


def splitmix64(seed: int, count: int, device="cpu") -> torch.Tensor:
    """SplitMix64 outputs 1..count of the stream seeded with `seed`, as int64 lanes holding u64 bits."""
    i = torch.arange(1, count + 1, dtype=torch.int64, device=device)
    z = i * _i64(_GOLDEN) + _i64(seed)
    z = (z ^ _srl(z, 30)) * _i64(_M1)
    z = (z ^ _srl(z, 27)) * _i64(_M2)
    return z ^ _srl(z, 31)


def uniform01(seed: int, count: int) -> torch.Tensor:
    """U[0, 1) doubles on the CPU (53 high bits of each draw)."""
    return _srl(splitmix64(seed, count), 11).to(torch.float64) * (2.0 ** -53)


def codes(seed: int, name: str, shape, device="cpu") -> torch.Tensor:
    """Uniform u16 codes as an int16 tensor of `shape` (the bytes are what matter)."""
    numel = math.prod(shape)
    draws = splitmix64(seed_of(seed, name), (numel + 3) // 4, device=device)
    return draws.view(torch.int16)[:numel].reshape(shape).clone()


def sign_scale(seed: int, name: str, shape, device="cpu") -> torch.Tensor:
    """+-1 x U(0.5, 1.5) in f16."""
    numel = math.prod(shape)
    s = seed_of(seed, name)
    bits = splitmix64(s, numel)
    sign = torch.where(bits < 0, -1.0, 1.0).to(torch.float64)
    mag = 0.5 + uniform01(seed_of(s, "mag"), numel)
    return (sign * mag).to(torch.float16).reshape(shape).to(device)


def normal(seed: int, name: str, shape, device="cpu", dtype=torch.float16) -> torch.Tensor:
    """N(0, 1) by Box-Muller, rounded to `dtype`."""
    numel = math.prod(shape)
    s = seed_of(seed, name)
    u1 = uniform01(s, numel)
    u2 = uniform01(seed_of(s, "u2"), numel)
    z = torch.sqrt(-2.0 * torch.log1p(-u1)) * torch.cos(2.0 * math.pi * u2)
    return z.to(dtype).reshape(shape).to(device)


def proj(seed: int, name: str, experts: int, in_f: int, out_f: int, n: int, device="cpu", norm: bool = False):
    """A bank (trellis [E, in/16, out/16, n] int16, suh [E, in] f16, svh [E, out] f16).  `norm` divides svh by
    sqrt(in) (rounded to f16), so the projection keeps N(0, 1) activations near unit scale (the codebook's weights
    are near unit variance); without it outputs grow by sqrt(in) per projection."""
    from .exl3 import Proj

    svh = sign_scale(seed, name + ".svh", (experts, out_f))
    if norm:
        svh = (svh.double() / math.sqrt(in_f)).to(torch.float16)
    return Proj(codes(seed, name + ".trellis", (experts, in_f // 16, out_f // 16, n), device),
                sign_scale(seed, name + ".suh", (experts, in_f), device), svh.to(device))


def bank(seed: int, name: str, experts: int, hidden: int, inter: int, n, device="cpu", norm: bool = False):
    """gate / up [E, hidden -> inter] and down [E, inter -> hidden] at rates n (one rate or (n_gate, n_up, n_down));
    `norm` as in proj (the routed configs use it, so a chain of layers stays finite in f16)."""
    from .exl3 import Bank

    ng, nu, nd = (n, n, n) if isinstance(n, int) else n
    return Bank(proj(seed, name + ".gate", experts, hidden, inter, ng, device, norm),
                proj(seed, name + ".up", experts, hidden, inter, nu, device, norm),
                proj(seed, name + ".down", experts, inter, hidden, nd, device, norm))


def tile_map(seed: int, name: str, shape, p_k1: float = 0.25, device="cpu") -> torch.Tensor:
    """configs[4]'s seeded per-tile rate map: each tile K1 (True) with probability p_k1, else K2."""
    return (uniform01(seed_of(seed, name), math.prod(shape)) < p_k1).reshape(shape).to(device)


def tiled_proj(seed: int, name: str, experts: int, in_f: int, out_f: int, p_k1: float = 0.25, device="cpu",
               norm: bool = False):
    """A per-tile-rate projection (exl3.TiledProj): the tile map from `name`.k1; every tile's codes are the first n of
    a 32-halfword uniform draw (`name`.trellis), so a K1 tile holds the first 16 halfwords of its K2 draw."""
    from .exl3 import TiledProj

    shape = (experts, in_f // 16, out_f // 16)
    k1 = tile_map(seed, name + ".k1", shape, p_k1, device)
    cb = codes(seed, name + ".trellis", shape + (32,), device)
    svh = sign_scale(seed, name + ".svh", (experts, out_f))
    if norm:
        svh = (svh.double() / math.sqrt(in_f)).to(torch.float16)
    tp = TiledProj.pack(cb[..., :16], cb, k1, sign_scale(seed, name + ".suh", (experts, in_f), device), svh.to(device))
    return tp


def tiled_bank(seed: int, name: str, experts: int, hidden: int, inter: int, p_k1: float = 0.25, device="cpu",
               norm: bool = False):
    """gate / up / down as per-tile-rate projections (exl3.Tiled)."""
    from .exl3 import Tiled

    return Tiled(tiled_proj(seed, name + ".gate", experts, hidden, inter, p_k1, device, norm),
                 tiled_proj(seed, name + ".up", experts, hidden, inter, p_k1, device, norm),
                 tiled_proj(seed, name + ".down", experts, inter, hidden, p_k1, device, norm))
