"""CPU oracle for the EXL3/STQ trellis hot path -- TEST INFRASTRUCTURE ONLY.

This package wraps ``liboracle_exl3.so``, a plain-C restatement of beamivalice/sushi's CPU decoder
(``src/exl3/expert_exl3.zig``) and host oracles.  It is the *checker*: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it.  The product
(``sushi_amd``) never imports it and has no CPU fallback.

Which check pins each function is listed in ``exl3_oracle.h``.  ``decode_3inst`` is an extension the
reference does not have: it is pinned by closed form only ("parity unpinned" against the reference).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_exl3.so")

CB_MUL1, CB_MCG, CB_SPEC1, CB_PAIR1, CB_STD1, CB_3INST = 0, 1, 2, 3, 4, 5
TABLE_NONE, TABLE_PAIR1_W16_V1, TABLE_SPEC1_W15, TABLE_SPEC1_W16, TABLE_STD1 = -1, 0, 1, 2, 3


class Decode(ctypes.Structure):
    _fields_ = [("codebook", ctypes.c_int32), ("window_bits", ctypes.c_int32), ("table", ctypes.c_int32)]

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return f"Decode(cb={self.codebook}, w={self.window_bits}, table={self.table})"


def decode(codebook: int, window_bits: int = 16, table: int = TABLE_NONE) -> Decode:
    return Decode(codebook, window_bits, table)


class _Pair(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("mult", "rot", "mask0", "mask1", "scale")]


def build() -> None:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _declare(L: ctypes.CDLL) -> None:
    vp, sz, u32, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int32
    L.ox_f32_to_f16.restype = ctypes.c_uint16
    L.ox_f32_to_f16.argtypes = [ctypes.c_float]
    L.ox_f16_to_f32.restype = ctypes.c_float
    L.ox_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.ox_bit_end.restype = u32
    L.ox_bit_end.argtypes = [u32, u32]
    L.ox_rate_admitted.argtypes = [u32]
    for name in ("ox_decode_mcg", "ox_decode_mul1", "ox_decode_3inst"):
        getattr(L, name).restype = ctypes.c_uint16
        getattr(L, name).argtypes = [ctypes.c_uint16]
    L.ox_decode_hashmask.restype = ctypes.c_uint16
    L.ox_decode_hashmask.argtypes = [ctypes.c_uint16, u32, u32, u32]
    L.ox_decode_pair.argtypes = [ctypes.c_uint16, ctypes.POINTER(_Pair), vp]
    L.ox_pair1_row.argtypes = [u32, ctypes.POINTER(_Pair)]
    L.ox_table_row.argtypes = [i32, u32, vp]
    L.ox_table_info.argtypes = [i32, vp, vp, vp, vp, vp]
    L.ox_unpack_tile.argtypes = [vp, u32, vp]
    L.ox_tensor_core_perm.argtypes = [vp]
    L.ox_decode_tile.argtypes = [vp, u32, Decode, vp]
    L.ox_decode_codewords.argtypes = [vp, sz, u32, Decode, vp]
    L.ox_hadamard128.argtypes = [vp]
    L.ox_fwht128.argtypes = [vp]
    L.ox_reconstruct_inner.argtypes = [vp, sz, sz, u32, Decode, vp]
    L.ox_reconstruct_public.argtypes = [vp, vp, vp, sz, sz, u32, Decode, vp]
    L.ox_prepare_input.argtypes = [vp, vp, sz, vp]
    L.ox_inner_gemv.argtypes = [vp, vp, sz, sz, u32, Decode, vp]
    L.ox_finish_output.argtypes = [vp, vp, sz, vp]
    L.ox_project.argtypes = [vp, vp, vp, vp, sz, sz, u32, Decode, vp]
    L.ox_project_rows.argtypes = [vp, sz, vp, vp, vp, sz, sz, u32, Decode, ctypes.c_int, vp]
    L.ox_moe_swiglu_host.argtypes = [vp] * 12 + [sz, sz, sz, u32, u32, u32, Decode, ctypes.c_float, vp]
    L.ox_moe_swiglu_rows.argtypes = [vp, sz] + [vp] * 17 + [sz, sz, sz, Decode, ctypes.c_float, ctypes.c_int, vp]
    L.ox_decode_dense.argtypes = [vp, vp, vp, sz, sz, u32, Decode, vp]
    L.ox_reconstruct_inner_tiled.argtypes = [vp, vp, vp, sz, sz, sz, u32, u32, Decode, vp]
    L.ox_project_tiled.argtypes = [vp, vp, vp, vp, sz, vp, vp, sz, sz, u32, u32, Decode, vp]
    L.ox_moe_swiglu_tiled_rows.argtypes = [vp, sz, vp, vp, vp, vp, vp, u32, u32, vp, vp, sz, sz, sz, Decode,
                                           ctypes.c_float, ctypes.c_int, vp]
    L.ox_gated_shared_term.restype = ctypes.c_float
    L.ox_gated_shared_term.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int]
    L.ox_gated_shared_terms.argtypes = [vp, vp, sz, sz, ctypes.c_int, vp]
    L.ox_route_topk.argtypes = [vp, sz, sz, sz, vp, vp]
    L.ox_tile_major.argtypes = [vp, vp, sz, sz, sz]
    L.ox_tile_major_inverse.argtypes = [vp, vp, sz, sz, sz]
    L.ox_viterbi_pass.argtypes = [vp, vp, sz, vp, u32, ctypes.c_int64, vp]
    L.ox_viterbi_pass.restype = ctypes.c_double
    L.ox_exact_tail_biting.argtypes = [vp, vp, sz, vp, u32, vp]
    L.ox_exact_tail_biting.restype = ctypes.c_double
    L.ox_pack_states.argtypes = [u32, vp, vp]
    L.ox_encode_tile.argtypes = [vp, u32, Decode, vp, vp, ctypes.POINTER(ctypes.c_double)]
    L.ox_quant_regularize.argtypes = [vp, sz, sz, vp, vp, ctypes.c_int, vp, vp, vp, vp]
    L.ox_quant_rotated_hessian.argtypes = [vp, vp, sz, vp]
    L.ox_cholesky_lower.argtypes = [vp, sz]
    L.ox_cholesky_lower.restype = sz
    L.ox_quant_ldl_factor.argtypes = [vp, sz, vp]
    L.ox_quant_global_scale.argtypes = [vp, sz, sz, u32, Decode, vp]
    L.ox_quant_ldlq.argtypes = [vp, vp, sz, sz, u32, Decode, vp, vp]
    L.ox_quant_signs.argtypes = [ctypes.c_uint64, ctypes.c_char_p, sz, vp]
    L.ox_quantize_tensor.argtypes = [vp, vp, sz, sz, vp, vp, u32, Decode, ctypes.c_int, vp, vp, vp, vp]


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} refused (rc={rc}): no codebook row for this rate")


# ---- scalar decoders -------------------------------------------------------------------------


def f32_to_f16(v: float) -> int:
    return lib().ox_f32_to_f16(v)


def f16_to_f32(h: int) -> float:
    return lib().ox_f16_to_f32(h)


def bit_end(n: int, t: int) -> int:
    return lib().ox_bit_end(n, t)


def decode_mcg(cw: int) -> int:
    return lib().ox_decode_mcg(cw)


def decode_mul1(cw: int) -> int:
    return lib().ox_decode_mul1(cw)


def decode_3inst(cw: int) -> int:
    return lib().ox_decode_3inst(cw)


def decode_hashmask(cw: int, mult: int, mask: int, scale: int = 4096) -> int:
    return lib().ox_decode_hashmask(cw, mult, mask, scale)


@dataclass(frozen=True)
class Pair:
    mult: int
    rot: int
    mask0: int
    mask1: int
    scale: int = 4096


def pair1_row(n: int):
    p = _Pair()
    return Pair(p.mult, p.rot, p.mask0, p.mask1, p.scale) if lib().ox_pair1_row(n, ctypes.byref(p)) else None


def decode_pair(cw: int, pair: Pair) -> tuple:
    p = _Pair(pair.mult, pair.rot, pair.mask0, pair.mask1, pair.scale)
    out = np.zeros(2, np.uint16)
    lib().ox_decode_pair(cw, ctypes.byref(p), _p(out))
    return int(out[0]), int(out[1])


def table_row(table: int, n: int):
    row = np.zeros(4, np.uint32)
    return tuple(int(v) for v in row) if lib().ox_table_row(table, n, _p(row)) else None


def table_info(table: int):
    vals = [np.zeros(1, np.int32), np.zeros(1, np.int32), np.zeros(1, np.uint32), np.zeros(1, np.uint32),
            np.zeros(1, np.uint32)]
    if not lib().ox_table_info(table, *[_p(v) for v in vals]):
        return None
    cb, win, n_lo, rows, fields = (int(v[0]) for v in vals)
    return dict(codebook=cb, window_bits=win, n_lo=n_lo, rows=rows, fields=fields)


# ---- tiles -------------------------------------------------------------------------------------


def unpack_tile(words, n: int) -> np.ndarray:
    w = _u16(words)
    assert w.size == n
    out = np.zeros(256, np.uint16)
    lib().ox_unpack_tile(_p(w), n, _p(out))
    return out


def tensor_core_perm() -> np.ndarray:
    out = np.zeros(256, np.uint32)
    lib().ox_tensor_core_perm(_p(out))
    return out


def decode_tile(words, n: int, dec: Decode) -> np.ndarray:
    w = _u16(words)
    out = np.zeros(256, np.uint16)
    _check(lib().ox_decode_tile(_p(w), n, dec, _p(out)), "decode_tile")
    return out


def decode_codewords(cws, n: int, dec: Decode) -> np.ndarray:
    c = _u16(cws).ravel()
    out = np.zeros(c.size * (2 if dec.codebook == CB_PAIR1 else 1), np.uint16)
    _check(lib().ox_decode_codewords(_p(c), c.size, n, dec, _p(out)), "decode_codewords")
    return out


def hadamard128(v) -> np.ndarray:
    a = _f32(v).copy()
    lib().ox_hadamard128(_p(a))
    return a


def fwht128(v) -> np.ndarray:
    a = _f32(v).copy()
    lib().ox_fwht128(_p(a))
    return a


def reconstruct_inner(trellis, in_f: int, out_f: int, n: int, dec: Decode) -> np.ndarray:
    t = _u16(trellis)
    out = np.zeros((in_f, out_f), np.uint16)
    _check(lib().ox_reconstruct_inner(_p(t), in_f, out_f, n, dec, _p(out)), "reconstruct_inner")
    return out


def reconstruct_public(trellis, suh, svh, in_f: int, out_f: int, n: int, dec: Decode) -> np.ndarray:
    t, su, sv = _u16(trellis), _u16(suh), _u16(svh)
    out = np.zeros((in_f, out_f), np.uint16)
    _check(lib().ox_reconstruct_public(_p(t), _p(su), _p(sv), in_f, out_f, n, dec, _p(out)), "reconstruct_public")
    return out


# ---- project -----------------------------------------------------------------------------------


def prepare_input(x, suh) -> np.ndarray:
    xv, su = _f32(x), _u16(suh)
    out = np.zeros(xv.size, np.float32)
    lib().ox_prepare_input(_p(xv), _p(su), xv.size, _p(out))
    return out


def inner_gemv(trellis, transformed, in_f: int, out_f: int, n: int, dec: Decode) -> np.ndarray:
    t, xv = _u16(trellis), _f32(transformed)
    out = np.zeros(out_f, np.float32)
    _check(lib().ox_inner_gemv(_p(t), _p(xv), in_f, out_f, n, dec, _p(out)), "inner_gemv")
    return out


def finish_output(inner, svh) -> np.ndarray:
    iv, sv = _f32(inner), _u16(svh)
    out = np.zeros(iv.size, np.float32)
    lib().ox_finish_output(_p(iv), _p(sv), iv.size, _p(out))
    return out


def project(x, trellis, suh, svh, in_f: int, out_f: int, n: int, dec: Decode) -> np.ndarray:
    xv, t, su, sv = _f32(x), _u16(trellis), _u16(suh), _u16(svh)
    out = np.zeros(out_f, np.float32)
    _check(lib().ox_project(_p(xv), _p(t), _p(su), _p(sv), in_f, out_f, n, dec, _p(out)), "project")
    return out


def project_rows(x, trellis, suh, svh, in_f: int, out_f: int, n: int, dec: Decode, threads: int = 1) -> np.ndarray:
    xv = _f32(x).reshape(-1, in_f)
    t, su, sv = _u16(trellis), _u16(suh), _u16(svh)
    out = np.zeros((xv.shape[0], out_f), np.float32)
    rc = lib().ox_project_rows(_p(xv), xv.shape[0], _p(t), _p(su), _p(sv), in_f, out_f, n, dec, threads, _p(out))
    _check(rc, "project_rows")
    return out


def moe_swiglu_host(x, gate, up, down, slots, weights, hidden: int, inter: int, n: tuple, dec: Decode,
                    clamp_limit: float = 0.0) -> np.ndarray:
    """One token through the routed experts: gate/up/down are (trellis, suh, svh) banks."""
    xv = _f32(x)
    arrs = [_u16(a) for p in (gate, up, down) for a in p]
    sl = np.ascontiguousarray(slots, np.uint32)
    wv = _f32(weights)
    y = np.zeros(hidden, np.float32)
    rc = lib().ox_moe_swiglu_host(_p(xv), *[_p(a) for a in arrs], _p(sl), _p(wv), sl.size, hidden, inter,
                                  n[0], n[1], n[2], dec, clamp_limit, _p(y))
    _check(rc, "moe_swiglu_host")
    return y


def moe_swiglu_rows(x, gate, up, down, slots, weights, hidden: int, inter: int, n, dec: Decode,
                    clamp_limit: float = 0.0, threads: int = 8) -> np.ndarray:
    """Rows of tokens x [rows, hidden] through moeSwigluHost, slots / weights [rows, topk].  gate/up/down are
    (trellis, suh [E, in], svh [E, out]) banks; n is (n_gate, n_up, n_down), each an int (a uniform bank, trellis
    [E, in/16, out/16, n]) or a per-expert rate array (a ragged bank: each expert's tiles contiguous, in expert
    order, at its own rate)."""
    xv = _f32(x).reshape(-1, hidden)
    sl = np.ascontiguousarray(slots, np.uint32).reshape(xv.shape[0], -1)
    wv = _f32(weights).reshape(sl.shape)
    experts = _u16(gate[1]).size // hidden
    dims = ((hidden, inter), (hidden, inter), (inter, hidden))
    offs, rates = [], []
    for ni, (din, dout) in zip(n, dims):
        r = np.full(experts, ni, np.uint32) if np.isscalar(ni) else np.ascontiguousarray(ni, np.uint32)
        tiles = (din // 16) * (dout // 16)
        offs.append(np.concatenate([[0], np.cumsum(r.astype(np.uint64) * tiles)[:-1]]).astype(np.uint64))
        rates.append(r)
    arrs = [_u16(a) for p in (gate, up, down) for a in p]
    y = np.zeros((xv.shape[0], hidden), np.float32)
    rc = lib().ox_moe_swiglu_rows(_p(xv), xv.shape[0], *[_p(a) for a in arrs], *[_p(o) for o in offs],
                                  *[_p(r) for r in rates], _p(sl), _p(wv), sl.shape[1], hidden, inter, dec,
                                  clamp_limit, threads, _p(y))
    _check(rc, "moe_swiglu_rows")
    return y


# ---- per-tile rates (configs[4]'s K1/K2 tile mix; an extension with no reference counterpart) ----------------


def reconstruct_inner_tiled(trellis, seg_off, seg_k1, expert: int, in_f: int, out_f: int, n_a: int, n_b: int,
                            dec: Decode) -> np.ndarray:
    t, o, k = _u16(trellis), np.ascontiguousarray(seg_off, np.uint32), np.ascontiguousarray(seg_k1, np.uint8)
    out = np.zeros((in_f, out_f), np.uint16)
    _check(lib().ox_reconstruct_inner_tiled(_p(t), _p(o), _p(k), expert, in_f, out_f, n_a, n_b, dec, _p(out)),
           "reconstruct_inner_tiled")
    return out


def project_tiled(x, trellis, seg_off, seg_k1, expert: int, suh, svh, in_f: int, out_f: int, n_a: int, n_b: int,
                  dec: Decode) -> np.ndarray:
    xv, t = _f32(x), _u16(trellis)
    o, k = np.ascontiguousarray(seg_off, np.uint32), np.ascontiguousarray(seg_k1, np.uint8)
    su, sv = _u16(suh), _u16(svh)
    out = np.zeros(out_f, np.float32)
    _check(lib().ox_project_tiled(_p(xv), _p(t), _p(o), _p(k), expert, _p(su), _p(sv), in_f, out_f, n_a, n_b, dec,
                                  _p(out)), "project_tiled")
    return out


def moe_swiglu_tiled_rows(x, projs, slots, weights, hidden: int, inter: int, n_a: int, n_b: int, dec: Decode,
                          clamp_limit: float = 0.0, threads: int = 8) -> np.ndarray:
    """Rows of tokens through moeSwigluHost on per-tile-rate banks; projs = [(trellis, seg_off, seg_k1, suh, svh)]
    for gate, up and down."""
    xv = _f32(x).reshape(-1, hidden)
    sl = np.ascontiguousarray(slots, np.uint32).reshape(xv.shape[0], -1)
    wv = _f32(weights).reshape(sl.shape)
    keep = [(_u16(p[0]), np.ascontiguousarray(p[1], np.uint32), np.ascontiguousarray(p[2], np.uint8), _u16(p[3]),
             _u16(p[4])) for p in projs]
    arr = lambda i: (ctypes.c_void_p * 3)(*[k[i].ctypes.data for k in keep])  # noqa: E731
    y = np.zeros((xv.shape[0], hidden), np.float32)
    rc = lib().ox_moe_swiglu_tiled_rows(_p(xv), xv.shape[0], arr(0), arr(1), arr(2), arr(3), arr(4), n_a, n_b,
                                        _p(sl), _p(wv), sl.shape[1], hidden, inter, dec, clamp_limit, threads, _p(y))
    _check(rc, "moe_swiglu_tiled_rows")
    return y


def gated_shared_term(gate: float, shared: float, dtype: int) -> float:
    """T(sigmoid(gate) * shared) rounded where MLX's bf16 Sigmoid and Multiply round (dtype 0 f16, 1 bf16, 2 f32)."""
    return lib().ox_gated_shared_term(gate, shared, dtype)


def gated_shared_terms(gate, shared, dtype: int) -> np.ndarray:
    """gated_shared_term over a block: gate [rows], shared [rows, cols] -> [rows, cols] f32."""
    g = _f32(gate).reshape(-1)
    sh = _f32(shared).reshape(g.size, -1)
    out = np.zeros_like(sh)
    lib().ox_gated_shared_terms(_p(g), _p(sh), g.size, sh.shape[1], dtype, _p(out))
    return out


def decode_dense(words, suh, svh, in_f: int, out_f: int, n: int, dec: Decode) -> np.ndarray:
    w, su, sv = _u16(words), _u16(suh), _u16(svh)
    out = np.zeros((in_f, out_f), np.float32)
    _check(lib().ox_decode_dense(_p(w), _p(su), _p(sv), in_f, out_f, n, dec, _p(out)), "decode_dense")
    return out


def route_topk(logits, k: int):
    lg = _f32(logits)
    rows, experts = lg.shape
    inds = np.zeros((rows, k), np.uint32)
    scores = np.zeros((rows, k), np.float32)
    lib().ox_route_topk(_p(lg), rows, experts, k, _p(inds), _p(scores))
    return inds, scores


def tile_major(src, it: int, ot: int, n: int) -> np.ndarray:
    s = _u16(src)
    dst = np.zeros_like(s)
    lib().ox_tile_major(_p(s), _p(dst), it, ot, n)
    return dst


def tile_major_inverse(src, it: int, ot: int, n: int) -> np.ndarray:
    s = _u16(src)
    dst = np.zeros_like(s)
    lib().ox_tile_major_inverse(_p(s), _p(dst), it, ot, n)
    return dst


# ---- encoder search (src/encoder/encode.zig) ------------------------------------------------------------------


def viterbi_pass(x, ks, table, w: int, pin=None):
    """`viterbiPass` (encode.zig:46-101) in f64: (cost, path)."""
    xs = np.ascontiguousarray(x, np.float64)
    k = np.ascontiguousarray(ks, np.uint8)
    t = np.ascontiguousarray(table, np.float64)
    path = np.zeros(len(xs), np.uint16)
    c = lib().ox_viterbi_pass(_p(xs), _p(k), len(xs), _p(t), w, -1 if pin is None else int(pin), _p(path))
    return c, path


def exact_tail_biting(x, ks, table, w: int):
    xs = np.ascontiguousarray(x, np.float64)
    k = np.ascontiguousarray(ks, np.uint8)
    t = np.ascontiguousarray(table, np.float64)
    path = np.zeros(len(xs), np.uint16)
    return lib().ox_exact_tail_biting(_p(xs), _p(k), len(xs), _p(t), w, _p(path)), path


def pack_states(n: int, states) -> np.ndarray:
    s = _u16(states)
    out = np.zeros(n, np.uint16)
    lib().ox_pack_states(n, _p(s), _p(out))
    return out


ENCODE_ERRORS = {-1: "CodebookUnsupported", -2: "RateUnsupported", -3: "WindowUnsupported", -4: "WindowTooNarrow"}


def encode_tile(tile, n: int, dec: Decode):
    """`Encoder.encodeTile` (encode.zig:170-294): (packed [n] u16, sse f64, recon [256] f32) of one row-major tile."""
    x = _f32(tile).reshape(256)
    packed = np.zeros(n, np.uint16)
    recon = np.zeros(256, np.float32)
    sse = ctypes.c_double()
    rc = lib().ox_encode_tile(_p(x), n, dec, _p(packed), _p(recon), ctypes.byref(sse))
    if rc != 0:
        raise ValueError(ENCODE_ERRORS.get(rc, str(rc)))
    return packed, sse.value, recon


# ---- quantizer (src/encoder/quantize.zig) ------------------------------------------------------------------------

OUT_SCALES = {"auto": 0, "always": 1, "never": 2}


def quant_regularize(w, sign_in, sign_out, mode: str, hdiag=None):
    w = _f32(w)
    rows, cols = w.shape
    inner = np.zeros_like(w)
    suh = np.zeros(rows, np.float32)
    svh = np.zeros(cols, np.float32)
    hd = None if hdiag is None else _f32(hdiag)
    rc = lib().ox_quant_regularize(_p(w), rows, cols, _p(_f32(sign_in)), _p(_f32(sign_out)), OUT_SCALES[mode],
                                   None if hd is None else _p(hd), _p(inner), _p(suh), _p(svh))
    _check(rc, "quant_regularize")
    return inner, suh, svh


def quant_rotated_hessian(h, suh) -> np.ndarray:
    h = _f32(h)
    out = np.zeros_like(h)
    _check(lib().ox_quant_rotated_hessian(_p(h), _p(_f32(suh)), h.shape[0], _p(out)), "rotated_hessian")
    return out


def cholesky_lower(a):
    m = np.ascontiguousarray(a, np.float64).copy()
    bad = lib().ox_cholesky_lower(_p(m), m.shape[0])
    return bad, m


def quant_ldl_factor(h) -> np.ndarray:
    h = _f32(h)
    out = np.zeros_like(h)
    rc = lib().ox_quant_ldl_factor(_p(h), h.shape[0], _p(out))
    if rc != 0:
        raise ValueError("HessianNotPositiveDefinite" if rc == -2 else "GeometryUnsupported")
    return out


def quant_global_scale(inner, n: int, dec: Decode) -> float:
    x = _f32(inner)
    g = np.zeros(1, np.float32)
    _check(lib().ox_quant_global_scale(_p(x), x.shape[0], x.shape[1], n, dec, _p(g)), "global_scale")
    return float(g[0])


def quant_ldlq(inner, l, n: int, dec: Decode):
    x = _f32(inner)
    rows, cols = x.shape
    packed = np.zeros((rows // 16, cols // 16, n), np.uint16)
    recon = np.zeros_like(x)
    _check(lib().ox_quant_ldlq(_p(x), _p(_f32(l)), rows, cols, n, dec, _p(packed), _p(recon)), "ldlq")
    return packed, recon


def quant_signs(seed: int, name: str, length: int) -> np.ndarray:
    out = np.zeros(length, np.float32)
    lib().ox_quant_signs(seed, name.encode(), length, _p(out))
    return out


def quantize_tensor(w, h, sign_in, sign_out, n: int, dec: Decode, mode: str):
    """`quantizeTensor` (quantize.zig:600-626): (packed [in/16, out/16, n] u16, suh f16 bits, svh f16 bits, g)."""
    w = _f32(w)
    rows, cols = w.shape
    packed = np.zeros((rows // 16, cols // 16, n), np.uint16)
    suh = np.zeros(rows, np.uint16)
    svh = np.zeros(cols, np.uint16)
    g = np.zeros(1, np.float32)
    rc = lib().ox_quantize_tensor(_p(w), _p(_f32(h)), rows, cols, _p(_f32(sign_in)), _p(_f32(sign_out)), n, dec,
                                  OUT_SCALES[mode], _p(packed), _p(suh), _p(svh), _p(g))
    _check(rc, "quantize_tensor")
    return packed, suh, svh, float(g[0])
