"""ctypes binding of libsushi_exl3_hip.so (the C ABI declared in include/sushi_exl3_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsushi_exl3_hip.so")

EXPORTS = (
    "exl3_abi_version",
    "exl3_last_error",
    "exl3_set_override",
    "exl3_decode_codewords",
    "exl3_reconstruct_inner",
    "exl3_linear_workspace_size",
    "exl3_linear",
    "exl3_linear_grouped_workspace_size",
    "exl3_linear_grouped",
    "exl3_linear_noalloc",
    "exl3_linear_pair_workspace_size",
    "exl3_linear_pair",
    "exl3_workspace_init",
    "exl3_moe_workspace_size",
    "exl3_moe",
    "exl3_moe_with_gated_shared",
    "exl3_moe_ragged",
    "exl3_moe_groups_workspace_size",
    "exl3_moe_groups",
    "exl3_moe_with_shared_bank_workspace_size",
    "exl3_moe_with_shared_bank",
    "exl3_moe_ragged_with_shared_bank",
    "exl3_reconstruct_tiled",
    "exl3_moe_tiled",
    "exl3_moe_tiled_with_shared_bank",
    "exl3_route_topk",
    "exl3_tile_major",
    "exl3_encode_workspace_size",
    "exl3_encode_tiles",
    "exl3_quantize_workspace_size",
    "exl3_quantize_tensor",
)


class DecodeT(ctypes.Structure):
    _fields_ = [("codebook", ctypes.c_int32), ("window_bits", ctypes.c_int32), ("table", ctypes.c_int32)]


class ProjT(ctypes.Structure):
    _fields_ = [("trellis", ctypes.c_void_p), ("suh", ctypes.c_void_p), ("svh", ctypes.c_void_p),
                ("n", ctypes.c_int32)]


class BankT(ctypes.Structure):
    _fields_ = [("gate", ProjT), ("up", ProjT), ("down", ProjT)]


class RaggedT(ctypes.Structure):
    _fields_ = [("trellis", ctypes.c_void_p * 3), ("suh", ctypes.c_void_p * 3), ("svh", ctypes.c_void_p * 3),
                ("meta", ctypes.c_void_p), ("experts", ctypes.c_int32), ("lane_rates_only", ctypes.c_int32)]


class TiledT(ctypes.Structure):
    _fields_ = [("trellis", ctypes.c_void_p * 3), ("seg_off", ctypes.c_void_p * 3), ("seg_k1", ctypes.c_void_p * 3),
                ("suh", ctypes.c_void_p * 3), ("svh", ctypes.c_void_p * 3), ("experts", ctypes.c_int32),
                ("n_a", ctypes.c_int32), ("n_b", ctypes.c_int32)]


_lib = None


def load() -> ctypes.CDLL:
    """The built library; raises if it is not built (build with ``python -m sushi_amd.build``)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m sushi_amd.build` (no CPU fallback exists)")
    L = ctypes.CDLL(LIB_PATH)
    i32, vp, sz, i64 = ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64
    L.exl3_abi_version.restype = i32
    L.exl3_last_error.restype = ctypes.c_char_p
    L.exl3_set_override.argtypes = [i32, i32, i32]
    L.exl3_decode_codewords.argtypes = [vp, i64, i32, DecodeT, vp, vp]
    L.exl3_reconstruct_inner.argtypes = [vp, i32, i32, i32, DecodeT, vp, vp]
    L.exl3_linear_workspace_size.restype = sz
    L.exl3_linear_workspace_size.argtypes = [i32, i32, i32, i32]
    L.exl3_linear.argtypes = [vp, i32, i32, i32, i32, vp, i32, vp, vp, DecodeT, vp, i32, vp, sz, vp]
    L.exl3_linear_grouped_workspace_size.restype = sz
    L.exl3_linear_grouped_workspace_size.argtypes = [i32, i32, i32, i32, i32]
    L.exl3_linear_grouped.argtypes = [vp, i32, i32, i32, i32, i32, vp, i32, vp, vp, DecodeT, vp, i32, vp, sz, vp]
    L.exl3_linear_noalloc.argtypes = [vp, i32, i32, i32, i32, vp, i32, vp, vp, DecodeT, vp, i32, vp]
    L.exl3_linear_pair_workspace_size.restype = sz
    L.exl3_linear_pair_workspace_size.argtypes = [i32, i32, i32, i32, i32]
    L.exl3_linear_pair.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, i32, vp, vp, DecodeT, vp, i32, vp, vp,
                                   DecodeT, vp, i32, vp, sz, vp]
    L.exl3_workspace_init.argtypes = [vp, sz, vp]
    L.exl3_moe_workspace_size.restype = sz
    L.exl3_moe_workspace_size.argtypes = [i32, i32, i32, i32]
    L.exl3_moe.argtypes = [vp, i32, i32, i32, i32, i32, ctypes.POINTER(BankT), vp, vp, i32, i32, DecodeT, i32, i32,
                           vp, vp, i32, vp, sz, vp]
    L.exl3_moe_with_gated_shared.argtypes = [vp, i32, i32, i32, i32, i32, ctypes.POINTER(BankT), vp, vp, i32, i32,
                                             DecodeT, i32, vp, vp, vp, i32, vp, sz, vp]
    L.exl3_moe_ragged.argtypes = [vp, i32, i32, i32, i32, ctypes.POINTER(RaggedT), vp, vp, i32, i32, DecodeT, i32,
                                  i32, vp, vp, vp, i32, vp, sz, vp]
    L.exl3_moe_groups_workspace_size.restype = sz
    L.exl3_moe_groups_workspace_size.argtypes = [i32, i32, i32, i32]
    L.exl3_moe_groups.argtypes = [vp, i32, i32, i32, i32, i32, ctypes.POINTER(BankT), ctypes.POINTER(ctypes.c_int32),
                                  vp, vp, i32, i32, DecodeT, i32, vp, i32, vp, sz, vp]
    L.exl3_moe_with_shared_bank_workspace_size.restype = sz
    L.exl3_moe_with_shared_bank_workspace_size.argtypes = [i32, i32, i32, i32]
    L.exl3_moe_with_shared_bank.argtypes = [vp, i32, i32, i32, i32, i32, ctypes.POINTER(BankT), ctypes.POINTER(BankT),
                                            vp, vp, i32, i32, DecodeT, i32, i32, vp, i32, vp, sz, vp]
    L.exl3_moe_ragged_with_shared_bank.argtypes = [vp, i32, i32, i32, i32, ctypes.POINTER(RaggedT),
                                                   ctypes.POINTER(BankT), vp, vp, i32, i32, DecodeT, i32, i32, vp,
                                                   i32, vp, sz, vp]
    L.exl3_reconstruct_tiled.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, DecodeT, vp, vp]
    L.exl3_moe_tiled.argtypes = [vp, i32, i32, i32, i32, ctypes.POINTER(TiledT), vp, vp, i32, i32, DecodeT, i32, i32,
                                 vp, vp, vp, i32, vp, sz, vp]
    L.exl3_moe_tiled_with_shared_bank.argtypes = [vp, i32, i32, i32, i32, ctypes.POINTER(TiledT),
                                                  ctypes.POINTER(BankT), vp, vp, i32, i32, DecodeT, i32, i32, vp,
                                                  i32, vp, sz, vp]
    L.exl3_route_topk.argtypes = [vp, i32, i32, i32, vp, vp, vp]
    L.exl3_tile_major.argtypes = [vp, vp, i32, i32, i32, i32, i32, vp]
    L.exl3_encode_workspace_size.restype = sz
    L.exl3_encode_workspace_size.argtypes = [i32, DecodeT, ctypes.c_int64]
    L.exl3_encode_tiles.argtypes = [vp, ctypes.c_int64, i32, DecodeT, vp, vp, vp, sz, vp]
    L.exl3_quantize_workspace_size.restype = sz
    L.exl3_quantize_workspace_size.argtypes = [i32, i32, i32, DecodeT]
    L.exl3_quantize_tensor.argtypes = [vp, vp, i32, i32, vp, vp, i32, DecodeT, i32, vp, vp, vp, vp, vp, sz, vp]
    for name in EXPORTS:
        if name in ("exl3_abi_version", "exl3_last_error") or name.endswith("workspace_size"):
            continue
        getattr(L, name).restype = i32
    _lib = L
    return L


def last_error() -> str:
    return load().exl3_last_error().decode()
