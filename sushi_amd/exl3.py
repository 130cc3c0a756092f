"""Host-side mirror of beamivalice/sushi's ``sushi_exl3`` operator API for the EXL3/STQ trellis hot path, on MI355X.

Names, argument meaning and error behaviour follow the reference:

* formats: ``Codebook``/``Window``/``Decode``/``Rate`` (src/exl3/expert_exl3.zig:54-226), ``Proj``/``Bank``
  (src/exl3/root.zig:28-39), ``Ragged`` (src/exl3/rate_groups.zig:22-140);
* dense: ``linear``/``linear_grouped`` (src/exl3/linear.zig:27-53), ``reconstruct_inner`` (expert_exl3.zig:416);
* routed experts: ``moe``/``moe_with_shared``/``moe_clamped``/``moe_ragged`` (src/exl3/root.zig:51-124, :582-644);
* routing: ``moe_routing_chain`` (src/moe_router.zig:16-62); layout: ``tile_major`` (src/exl3/layout.zig:139-158).

Every call runs the HIP library through its C ABI on the caller's current torch stream; nothing falls back to the
CPU.  Refusals raise the reference's named errors before any launch.
"""
from __future__ import annotations

import contextlib
import ctypes
import enum
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from . import _lib

# ---------------------------------------------------------------------------------------------------------------
# Errors (src/exl3/root.zig:104-133, :421-423; src/exl3/expert_exl3_kernels.zig:2569, :1475)


class Exl3Error(RuntimeError):
    status = None


class BadExl3Shape(Exl3Error):
    status = -1


class BadExl3Dtype(Exl3Error):
    status = -2


class Exl3CodebookTableUnknown(Exl3Error):
    status = -3


class Exl3TopKExceedsReduceBank(Exl3Error):
    status = -4


class Exl3TopkUnsupported(Exl3Error):
    status = -5


class InvalidExl3Clamp(Exl3Error):
    status = -6


class Exl3SharedNeedsDecodeRows(Exl3Error):
    status = -7


class Exl3LaunchFailed(Exl3Error):
    status = -8


class Exl3WorkspaceTooSmall(Exl3Error):
    status = -9


class Exl3CodebookTableRateMissing(Exl3Error):
    status = -10


class Exl3WindowUnsupported(Exl3Error):
    status = -11


class CodebookUnsupported(Exl3Error):
    """The encoder searches MCG and MUL1 (and the 3INST extension) only (src/encoder/encode.zig:7-12)."""
    status = -12


class RateUnsupported(Exl3Error):
    status = -13


class WindowTooNarrow(Exl3Error):
    status = -14


class HessianNotPositiveDefinite(Exl3Error):
    status = -15


class Exl3GroupMissing(Exl3Error):
    status = -16


_BY_STATUS = {c.status: c for c in Exl3Error.__subclasses__()}


def _check(rc: int) -> None:
    if rc == 0:
        return
    raise _BY_STATUS.get(rc, Exl3Error)(f"[exl3 status {rc}] {_lib.last_error()}")


# ---------------------------------------------------------------------------------------------------------------
# Format types


class Codebook(enum.IntEnum):
    """`Codebook` (expert_exl3.zig:54-61) plus ``inst3``, QTIP's 3INST LCG codebook (an extension)."""

    mul1 = 0
    mcg = 1
    spec1 = 2
    pair1 = 3
    std1 = 4
    inst3 = 5

    @classmethod
    def from_name(cls, name: str) -> Optional["Codebook"]:
        return {"mcg": cls.mcg, "mul1": cls.mul1, "std1": cls.std1, "spec1": cls.spec1, "pair1": cls.pair1,
                "3inst": cls.inst3}.get(name)

    def tabled_hash_mask(self) -> bool:
        return self in (Codebook.spec1, Codebook.std1)

    def has_table(self) -> bool:
        return self.tabled_hash_mask() or self == Codebook.pair1


class Table(enum.IntEnum):
    """The shipped codebook tables, in codebook_tables.zig `shipped` order (:101-106)."""

    pair1_w16_v1 = 0
    spec1_w15 = 1
    spec1_w16 = 2
    std1 = 3


TABLE_NAMES = {"pair1-w16-v1": Table.pair1_w16_v1, "spec1-w15": Table.spec1_w15, "spec1-w16": Table.spec1_w16,
               "std1": Table.std1}


@dataclass(frozen=True)
class Window:
    """The codeword width a pack's search hashed (`Window`, expert_exl3.zig:102-137)."""

    bits: int = 16

    MIN_BITS = 8

    @classmethod
    def from_bits(cls, w: int) -> Optional["Window"]:
        return cls(w) if cls.MIN_BITS <= w <= 16 else None

    def mask(self) -> int:
        return (1 << self.bits) - 1


@dataclass(frozen=True)
class Decode:
    """How a pack's trellis decodes (`Decode`, expert_exl3.zig:141-174)."""

    codebook: Codebook
    window: Window = field(default_factory=Window)
    table: Optional[int] = None

    @classmethod
    def tabled(cls, codebook: Codebook, window: Window = Window()) -> "Decode":
        table = {Codebook.spec1: Table.spec1_w15, Codebook.std1: Table.std1}.get(codebook)
        return cls(codebook, window, table)

    def require_table(self) -> None:
        if self.codebook.tabled_hash_mask() and self.table is None:
            raise Exl3CodebookTableUnknown(f"{self.codebook.name} decode needs a codebook table")

    def c(self) -> _lib.DecodeT:
        return _lib.DecodeT(int(self.codebook), int(self.window.bits), -1 if self.table is None else int(self.table))


MUL1 = Decode(Codebook.mul1)
MCG = Decode(Codebook.mcg)
INST3 = Decode(Codebook.inst3)


@dataclass(frozen=True)
class Rate:
    """K = n/16 bits per weight (`Rate`, expert_exl3.zig:180-226)."""

    n: int

    MIN_N = 16
    MAX_N = 128

    @classmethod
    def from_k(cls, k: int) -> "Rate":
        return cls(16 * k)

    def bit_end(self, t: int) -> int:
        return ((t + 1) * self.n) >> 4

    def fresh_bits(self, t: int) -> int:
        return self.bit_end(t) - (0 if t == 0 else self.bit_end(t - 1))

    def words(self) -> int:
        return self.n // 2

    def total_bits(self) -> int:
        return 16 * self.n

    def is_integer(self) -> bool:
        return self.n % 16 == 0


def k_from_packed_dim(packed_hw: int) -> Optional[Rate]:
    """`kFromPackedDim` (expert_exl3.zig:241-245): even n in 16..128."""
    if packed_hw % 2 != 0 or packed_hw < Rate.MIN_N or packed_hw > Rate.MAX_N:
        return None
    return Rate(packed_hw)


@dataclass
class Proj:
    """One projection's bank: trellis u16 [E, in/16, out/16, n], suh f16 [E, in], svh f16 [E, out]."""

    trellis: torch.Tensor
    suh: torch.Tensor
    svh: torch.Tensor

    @property
    def n(self) -> int:
        return int(self.trellis.shape[-1])

    @property
    def experts(self) -> int:
        return int(self.trellis.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.trellis.shape[1]) * 16

    @property
    def out_features(self) -> int:
        return int(self.trellis.shape[2]) * 16

    def c(self) -> _lib.ProjT:
        return _lib.ProjT(self.trellis.data_ptr(), self.suh.data_ptr(), self.svh.data_ptr(), self.n)


@dataclass
class Bank:
    gate: Proj
    up: Proj
    down: Proj


META_WORDS = 8

# Rates the kernels read with a per-lane fixed-width reader; any other rate takes the generic reader.
LANE_RATES = (16, 24, 32, 40, 48, 64)


@dataclass
class Ragged:
    """A rate-grouped layer as one ragged trellis per projection (`Ragged`, rate_groups.zig:22-140).

    ``meta`` [E, 8] u32 per expert: {n_gate, n_up, n_down, group, off_gate, off_up, off_down, local}, offsets in u32
    words into the ragged trellis of that projection.
    """

    trellis: list
    suh: list
    svh: list
    meta: torch.Tensor
    experts: int
    hidden: int
    inter: int
    rates: list

    @classmethod
    def init(cls, banks: Sequence[Bank]) -> "Ragged":
        if not banks:
            raise BadExl3Shape("no rate groups")
        hidden = banks[0].gate.in_features
        inter = banks[0].gate.out_features
        meta, words = [], [0, 0, 0]
        rates = []
        for g, bank in enumerate(banks):
            projs = (bank.gate, bank.up, bank.down)
            e = bank.gate.experts
            for pi, p in enumerate(projs):
                want_in, want_out = (inter, hidden) if pi == 2 else (hidden, inter)
                if p.experts != e or p.in_features != want_in or p.out_features != want_out:
                    raise BadExl3Shape(f"group {g} projection {pi} shape {tuple(p.trellis.shape)}")
                if k_from_packed_dim(p.n) is None:
                    raise BadExl3Shape(f"group {g} projection {pi} rate n={p.n}")
            rates.append(tuple(p.n for p in projs))
            tiles = (hidden // 16) * (inter // 16)
            for local in range(e):
                row = [projs[0].n, projs[1].n, projs[2].n, g]
                row += [words[pi] + local * tiles * projs[pi].n // 2 for pi in range(3)]
                row.append(local)
                meta.append(row)
            for pi in range(3):
                words[pi] += e * tiles * projs[pi].n // 2
        dev = banks[0].gate.trellis.device
        trellis = [torch.cat([getattr(b, nm).trellis.reshape(-1) for b in banks]) for nm in ("gate", "up", "down")]
        suh = [torch.cat([getattr(b, nm).suh for b in banks]) for nm in ("gate", "up", "down")]
        svh = [torch.cat([getattr(b, nm).svh for b in banks]) for nm in ("gate", "up", "down")]
        if max(max(r) for r in meta[:]) >= 2 ** 32:
            raise BadExl3Shape("ragged offsets overflow u32")
        meta_t = torch.tensor(meta, dtype=torch.int64).to(torch.int32).to(dev)
        return cls(trellis, suh, svh, meta_t, len(meta), hidden, inter, rates)

    def c(self) -> _lib.RaggedT:
        r = _lib.RaggedT()
        for i in range(3):
            r.trellis[i] = self.trellis[i].data_ptr()
            r.suh[i] = self.suh[i].data_ptr()
            r.svh[i] = self.svh[i].data_ptr()
        r.meta = self.meta.data_ptr()
        r.experts = self.experts
        r.lane_rates_only = int(all(n in LANE_RATES for group in self.rates for n in group))
        return r


# Per-tile rates: the two tile rates of a per-tile-rate bank (K1 and K2).
TILED_RATES = (16, 32)


def _as_i32(t: torch.Tensor) -> torch.Tensor:
    """u32 values held in int64 as int32 lanes with the same bits."""
    return torch.where(t >= 2 ** 31, t - 2 ** 32, t).to(torch.int32)


@dataclass
class TiledProj:
    """One projection of a per-tile-rate bank (configs[4]'s K1 / K2 tile mix), a layout extension: the reference fixes
    a rate per tensor (layout.zig:56-62) or per expert group (rate_groups.zig:22-140), while each tile's arithmetic is
    decodeTile's at that tile's own n (expert_exl3.zig:338-357).

    ``trellis`` is one flat u16 stream; segment (e, tk, s) -- the tiles (tk, 8s .. 8s + 7) of expert e -- lies
    contiguous from u32 word ``seg_off[e, tk, s]`` (the stream in (e, s, tk) order), tiles in column order, tile o at
    16 halfwords when bit o of ``seg_k1[e, tk, s]`` is set, else at 32.  suh [E, in], svh [E, out] as for a uniform
    bank.
    """

    trellis: torch.Tensor
    seg_off: torch.Tensor  # [E, in/16, out/128] int32 (u32 bits)
    seg_k1: torch.Tensor   # [E, in/16, out/128] uint8
    suh: torch.Tensor
    svh: torch.Tensor

    @property
    def experts(self) -> int:
        return int(self.seg_off.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.seg_off.shape[1]) * 16

    @property
    def out_features(self) -> int:
        return int(self.seg_off.shape[2]) * 128

    def bits_per_weight(self) -> float:
        """The realised rate: packed bits over weights."""
        return self.trellis.numel() * 16 / (self.experts * self.in_features * self.out_features)

    @classmethod
    def pack(cls, codes_a: torch.Tensor, codes_b: torch.Tensor, k1: torch.Tensor, suh: torch.Tensor,
             svh: torch.Tensor) -> "TiledProj":
        """Tile (e, tk, tn) takes codes_a[e, tk, tn] (16 halfwords) where k1[e, tk, tn] is set, else codes_b (32);
        codes are int16 [E, in/16, out/16, n]."""
        if k1.dim() != 3 or k1.shape[2] % 8:
            raise BadExl3Shape(f"tile map {tuple(k1.shape)}: [E, in/16, out/16] with out a multiple of 128")
        e, it, ot = (int(v) for v in k1.shape)
        if tuple(codes_a.shape) != (e, it, ot, 16) or tuple(codes_b.shape) != (e, it, ot, 32):
            raise BadExl3Shape(f"codes {tuple(codes_a.shape)} / {tuple(codes_b.shape)} for tile map {(e, it, ot)}")
        dev = codes_b.device
        # The stream holds the segments in (e, s, tk) order: a column group's k-tile rows follow one another, so the
        # workgroup that reads them (a GEMM tile's k-steps, a GEMV split's waves) shares a 128-byte line only with
        # itself at a segment boundary.  In (e, tk, s) order neighbouring column groups -- other workgroups, often
        # on another XCD's L2 -- would each fetch the boundary line.
        def by_group(t: torch.Tensor) -> torch.Tensor:  # [E, IT, OT, ...] -> (e, s, tk, o)-major rows
            return t.reshape(e, it, ot // 8, 8, *t.shape[3:]).transpose(1, 2).reshape(e * it * ot, *t.shape[3:])
        kg = by_group(k1.to(dev))
        words = torch.where(kg, 8, 16).to(torch.int64)
        start = torch.cumsum(words, 0) - words
        total = int(words.sum())
        if total >= 2 ** 32:
            raise BadExl3Shape("per-tile-rate trellis past 2^32 words")
        flat = torch.zeros(2 * total, dtype=torch.int16, device=dev)
        ia, ib = torch.nonzero(kg).squeeze(1), torch.nonzero(~kg).squeeze(1)
        flat[(2 * start[ia])[:, None] + torch.arange(16, device=dev)] = by_group(codes_a)[ia]
        flat[(2 * start[ib])[:, None] + torch.arange(32, device=dev)] = by_group(codes_b)[ib]
        seg_off = _as_i32(start.reshape(e, ot // 8, it, 8)[..., 0].transpose(1, 2))
        bits = torch.tensor([1 << o for o in range(8)], dtype=torch.int32, device=dev)
        seg_k1 = (k1.to(dev).reshape(e, it, ot // 8, 8).to(torch.int32) * bits).sum(-1).to(torch.uint8)
        return cls(flat, seg_off.contiguous(), seg_k1.contiguous(), suh, svh)


@dataclass
class Tiled:
    """A routed layer whose three projections are per-tile-rate (TiledProj)."""

    gate: TiledProj
    up: TiledProj
    down: TiledProj

    @property
    def experts(self) -> int:
        return self.gate.experts

    @property
    def hidden(self) -> int:
        return self.gate.in_features

    @property
    def inter(self) -> int:
        return self.gate.out_features

    def check(self) -> None:
        e, h, i = self.experts, self.hidden, self.inter
        for nm, p, shape in (("gate", self.gate, (e, h, i)), ("up", self.up, (e, h, i)), ("down", self.down, (e, i, h))):
            if (p.experts, p.in_features, p.out_features) != shape:
                raise BadExl3Shape(f"tiled {nm}: {(p.experts, p.in_features, p.out_features)}, expected {shape}")

    def c(self) -> _lib.TiledT:
        r = _lib.TiledT()
        for i, p in enumerate((self.gate, self.up, self.down)):
            r.trellis[i] = p.trellis.data_ptr()
            r.seg_off[i] = p.seg_off.data_ptr()
            r.seg_k1[i] = p.seg_k1.data_ptr()
            r.suh[i] = p.suh.data_ptr()
            r.svh[i] = p.svh.data_ptr()
        r.experts = self.experts
        r.n_a, r.n_b = TILED_RATES
        return r


# ---------------------------------------------------------------------------------------------------------------
# Plumbing

_DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
_U16 = {torch.int16, getattr(torch, "uint16", torch.int16)}


def _dt(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise BadExl3Dtype(f"{what} dtype {t.dtype} (f16, bf16 or f32)") from None


def _need_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise BadExl3Shape("operands must be device tensors (the HIP path has no CPU fallback)")
        if not t.is_contiguous():
            raise BadExl3Shape("operands must be contiguous")


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


class _Workspace:
    """Scratch owned by this host layer (the C ABI itself never allocates), one buffer per (device, stream).

    The C ABI wants one workspace per stream: its first 8 MiB hold fold words and arrival counters that every call
    returns to zero, so two streams (a HIP-graph capture runs on a side stream) must not share it.  A buffer is
    allocated and zeroed eagerly; inside a capture it must already exist, since an allocation there would come from
    the graph's pool and its zero-fill would only be recorded.  A buffer that a larger one replaces stays alive for
    the life of the process: a captured graph may still point at it."""

    def __init__(self) -> None:
        self._buf: dict = {}
        self._retired: list = []

    # The three hooks below are the only places that touch the device (a CPU test replaces them).
    def _stream_handle(self, dev: torch.device) -> int:
        return torch.cuda.current_stream(dev).cuda_stream

    def _capturing(self) -> bool:
        return torch.cuda.is_current_stream_capturing()

    def _new(self, dev: torch.device, size: int, handle: int) -> torch.Tensor:
        buf = torch.empty(size, dtype=torch.uint8, device=dev)
        _check(_lib.load().exl3_workspace_init(buf.data_ptr(), buf.numel(), ctypes.c_void_p(handle)))
        return buf

    def get(self, dev: torch.device, nbytes: int) -> torch.Tensor:
        handle = self._stream_handle(dev)
        key = (dev.type, dev.index, handle)
        buf = self._buf.get(key)
        if buf is None or buf.numel() < nbytes:
            if self._capturing():
                raise Exl3WorkspaceTooSmall(
                    f"workspace of {nbytes} bytes is not allocated for this stream: make one eager call on the "
                    "capturing stream (or workspace.reserve) before the capture")
            size = max(nbytes, 1 << 20, 0 if buf is None else buf.numel() * 2)
            new = self._new(dev, size, handle)
            if buf is not None:
                self._retired.append(buf)
            self._buf[key] = buf = new
        return buf

    def reserve(self, dev: torch.device, nbytes: int) -> None:
        """Allocates (outside any capture) the current stream's buffer of at least `nbytes`."""
        self.get(dev, nbytes)


workspace = _Workspace()


def _u16_check(t: torch.Tensor, what: str) -> None:
    if t.element_size() != 2 or t.dtype.is_floating_point:
        raise BadExl3Dtype(f"{what} must be a 16-bit integer tensor (u16 codes)")


def _f16_check(t: torch.Tensor, what: str) -> None:
    if t.dtype != torch.float16:
        raise BadExl3Dtype(f"{what} must be float16")


# ---------------------------------------------------------------------------------------------------------------
# Arm overrides (tests and tuning sweeps; exl3_set_override in the C ABI)

KNOBS = {"gemv_splits": 0, "gemv_separate_finish": 1, "gemv_fold": 2, "moe_decode_rows_max": 3, "moe_splits1": 4,
         "moe_splits2": 5, "moe_windows": 6, "moe_fold": 7, "moe_gemm": 8, "gemm_arm": 9, "moe_chain": 10,
         "gemv_rows_per_group": 11, "gemm_split_wait": 12}


@contextlib.contextmanager
def arm_overrides(**knobs: int):
    """Pins library arms for the duration of a ``with`` block (e.g. ``arm_overrides(gemv_splits=8, gemv_fold=0)``);
    every knob named is unset again on exit."""
    L = _lib.load()
    try:
        for name, value in knobs.items():
            _check(L.exl3_set_override(KNOBS[name], int(value), 1))
        yield
    finally:
        for name in knobs:
            L.exl3_set_override(KNOBS[name], 0, 0)


# ---------------------------------------------------------------------------------------------------------------
# Decode / dequant


def decode_codewords(codewords: torch.Tensor, n: int, dec: Decode) -> torch.Tensor:
    """f16 weights of a flat list of codewords (PAIR1: two per codeword) -- the exhaustive decode check."""
    _need_gpu(codewords)
    _u16_check(codewords, "codewords")
    count = codewords.numel()
    per = 2 if dec.codebook == Codebook.pair1 else 1
    out = torch.empty(count * per, dtype=torch.float16, device=codewords.device)
    _check(_lib.load().exl3_decode_codewords(codewords.data_ptr(), count, n, dec.c(), out.data_ptr(),
                                             _stream(codewords.device)))
    return out


def reconstruct_inner(trellis: torch.Tensor, dec: Decode) -> torch.Tensor:
    """`reconstructInner` (expert_exl3.zig:416-438): f16 [in, out] of a [in/16, out/16, n] (or [1, ...]) trellis."""
    t = trellis.reshape(trellis.shape[-3:]) if trellis.dim() == 4 else trellis
    _need_gpu(t)
    _u16_check(t, "trellis")
    it, ot, n = (int(v) for v in t.shape)
    out = torch.empty(it * 16, ot * 16, dtype=torch.float16, device=t.device)
    _check(_lib.load().exl3_reconstruct_inner(t.data_ptr(), it * 16, ot * 16, n, dec.c(), out.data_ptr(),
                                              _stream(t.device)))
    return out


# ---------------------------------------------------------------------------------------------------------------
# Dense linears


def linear(x: torch.Tensor, p: Proj, dec: Decode, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """`linear.linear` (linear.zig:27-34): x [rows, in] through the one-bank projection -> [rows, out]."""
    if x.dim() != 2 or p.trellis.dim() != 4 or p.trellis.shape[0] != 1 or p.in_features != x.shape[1]:
        raise BadExl3Shape(f"linear: x {tuple(x.shape)} vs trellis {tuple(p.trellis.shape)}")
    dec.require_table()
    _need_gpu(x, p.trellis, p.suh, p.svh)
    _u16_check(p.trellis, "trellis")
    _f16_check(p.suh, "suh")
    _f16_check(p.svh, "svh")
    rows, in_f, out_f = int(x.shape[0]), p.in_features, p.out_features
    y = torch.empty(rows, out_f, dtype=out_dtype or x.dtype, device=x.device)
    L = _lib.load()
    ws_bytes = L.exl3_linear_workspace_size(rows, in_f, out_f, p.n)
    ws = workspace.get(x.device, ws_bytes)
    _check(L.exl3_linear(x.data_ptr(), _dt(x, "x"), rows, in_f, out_f, p.trellis.data_ptr(), p.n, p.suh.data_ptr(),
                         p.svh.data_ptr(), dec.c(), y.data_ptr(), _dt(y, "y"), ws.data_ptr(), ws.numel(),
                         _stream(x.device)))
    return y


def linear_grouped(x: torch.Tensor, p: Proj, dec: Decode) -> torch.Tensor:
    """`linear.linearGrouped` (linear.zig:37-53): x [G, rows, in] through the G-bank projection -> [G, rows, out]."""
    if x.dim() != 3 or p.trellis.dim() != 4 or p.trellis.shape[0] != x.shape[0] or p.in_features != x.shape[2]:
        raise BadExl3Shape(f"linear_grouped: x {tuple(x.shape)} vs trellis {tuple(p.trellis.shape)}")
    dec.require_table()
    _need_gpu(x, p.trellis, p.suh, p.svh)
    groups, rows = int(x.shape[0]), int(x.shape[1])
    in_f, out_f = p.in_features, p.out_features
    y = torch.empty(groups, rows, out_f, dtype=x.dtype, device=x.device)
    L = _lib.load()
    ws_bytes = L.exl3_linear_grouped_workspace_size(groups, rows, in_f, out_f, p.n)
    ws = workspace.get(x.device, ws_bytes)
    _check(L.exl3_linear_grouped(x.data_ptr(), _dt(x, "x"), groups, rows, in_f, out_f, p.trellis.data_ptr(), p.n,
                                 p.suh.data_ptr(), p.svh.data_ptr(), dec.c(), y.data_ptr(), _dt(y, "y"),
                                 ws.data_ptr(), ws.numel(), _stream(x.device)))
    return y


def linear_pair(x: torch.Tensor, a: Proj, b: Proj, dec_a: Decode, dec_b: Decode) -> Optional[torch.Tensor]:
    """`linear.linearPair` (linear.zig:60-95): x [G, rows, in] through the G-bank `a`, then that result as
    [rows, G * mid] through the one-bank `b` -> [rows, out] in x's dtype; linear_grouped, the transpose and linear, bit
    for bit, in two launches.  None, with nothing launched, past one decode launch's rows (the reference's null)."""
    if x.dim() != 3 or a.trellis.dim() != 4 or b.trellis.dim() != 4 or a.trellis.shape[0] != x.shape[0] or \
            b.trellis.shape[0] != 1 or a.in_features != x.shape[2] or b.in_features != x.shape[0] * a.out_features:
        raise BadExl3Shape(f"linear_pair: x {tuple(x.shape)}, a {tuple(a.trellis.shape)}, b {tuple(b.trellis.shape)}")
    dec_a.require_table()
    dec_b.require_table()
    for p in (a, b):
        _need_gpu(p.trellis, p.suh, p.svh)
        _u16_check(p.trellis, "trellis")
        _f16_check(p.suh, "suh")
        _f16_check(p.svh, "svh")
    _need_gpu(x)
    x = x.contiguous()
    groups, rows, in_f = int(x.shape[0]), int(x.shape[1]), int(x.shape[2])
    mid, out_f = a.out_features, b.out_features
    y = torch.empty(rows, out_f, dtype=x.dtype, device=x.device)
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_linear_pair_workspace_size(groups, rows, in_f, mid, out_f))
    rc = L.exl3_linear_pair(x.data_ptr(), _dt(x, "x"), groups, rows, in_f, mid, out_f, a.trellis.data_ptr(), a.n,
                            a.suh.data_ptr(), a.svh.data_ptr(), dec_a.c(), b.trellis.data_ptr(), b.n, b.suh.data_ptr(),
                            b.svh.data_ptr(), dec_b.c(), y.data_ptr(), _dt(y, "y"), ws.data_ptr(), ws.numel(),
                            _stream(x.device))
    if rc == EXL3_DECLINED:
        return None
    _check(rc)
    return y


# ---------------------------------------------------------------------------------------------------------------
# Routed experts

REDUCE_MAX_TOPK = 32
DECODE_ROWS_MAX = 16


def admit_top_k(topk: int) -> None:
    """`admitTopK` (root.zig:421-423)."""
    if topk > REDUCE_MAX_TOPK:
        raise Exl3TopKExceedsReduceBank(f"top-k {topk} > {REDUCE_MAX_TOPK}")


def _moe_prep(x: torch.Tensor, inds: torch.Tensor, scores: torch.Tensor):
    if x.dim() < 2 or inds.shape[:-1] != x.shape[:-1] or tuple(scores.shape) != tuple(inds.shape):
        raise BadExl3Shape(f"moe: x {tuple(x.shape)}, inds {tuple(inds.shape)}, scores {tuple(scores.shape)}")
    if inds.dtype not in (torch.int32, getattr(torch, "uint32", torch.int32)):
        raise BadExl3Dtype(f"moe: inds dtype {inds.dtype} (u32/i32)")
    if scores.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise BadExl3Dtype(f"moe: scores dtype {scores.dtype}")
    topk = int(inds.shape[-1])
    admit_top_k(topk)
    rows = x.numel() // x.shape[-1]
    x2 = x.reshape(rows, x.shape[-1])
    inds2 = inds.reshape(rows * topk).contiguous()
    sc2 = scores.reshape(rows * topk).contiguous()  # f32, bf16 or f16: the library reads each as it is
    return x2, inds2, sc2, rows, topk


def _bank_shape(bank: Bank, hidden: int):
    """(experts, inter) of a bank over hidden features (validateClampedProjection, root.zig:126-135)."""
    g, u, d = bank.gate, bank.up, bank.down
    experts = g.experts
    inter = g.out_features
    for p, (pin, pout) in ((g, (hidden, inter)), (u, (hidden, inter)), (d, (inter, hidden))):
        if p.experts != experts or p.in_features != pin or p.out_features != pout:
            raise BadExl3Shape(f"moe: projection shape {tuple(p.trellis.shape)}")
        _u16_check(p.trellis, "trellis")
        _f16_check(p.suh, "suh")
        _f16_check(p.svh, "svh")
        _need_gpu(p.trellis, p.suh, p.svh)
    return experts, inter


def _moe(x: torch.Tensor, bank: Bank, inds: torch.Tensor, scores: torch.Tensor, dec: Decode, verify_rows: bool,
         shared: Optional[torch.Tensor], limit: int, gate: Optional[torch.Tensor] = None) -> torch.Tensor:
    dec.require_table()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    g, u, d = bank.gate, bank.up, bank.down
    experts, inter = _bank_shape(bank, hidden)
    _need_gpu(x2, inds2, sc2, shared)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    if shared is not None:
        if shared.numel() != y.numel() or shared.dtype != y.dtype:
            raise BadExl3Shape("moe: shared expert output must match the routed output's size and dtype")
        shared = shared.reshape(rows, hidden).contiguous()
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_workspace_size(rows, topk, hidden, inter))
    cb = _lib.BankT(g.c(), u.c(), d.c())
    if gate is not None:
        if gate.numel() != rows or gate.dtype != y.dtype or shared is None:
            raise BadExl3Shape("moe: the shared expert's gate is one logit per row in the output's dtype")
        gate = gate.reshape(rows).contiguous()
        _need_gpu(gate)
        _check(L.exl3_moe_with_gated_shared(x2.data_ptr(), _dt(x2, "x"), rows, hidden, inter, experts,
                                            ctypes.byref(cb), inds2.data_ptr(), sc2.data_ptr(), _dt(sc2, "scores"),
                                            topk, dec.c(), int(verify_rows), shared.data_ptr(), gate.data_ptr(),
                                            y.data_ptr(), _dt(y, "y"), ws.data_ptr(), ws.numel(), _stream(x.device)))
        return y.reshape(x.shape)
    _check(L.exl3_moe(x2.data_ptr(), _dt(x2, "x"), rows, hidden, inter, experts, ctypes.byref(cb), inds2.data_ptr(),
                      sc2.data_ptr(), _dt(sc2, "scores"), topk, dec.c(), int(verify_rows), int(limit),
                      None if shared is None else shared.data_ptr(), y.data_ptr(), _dt(y, "y"), ws.data_ptr(),
                      ws.numel(), _stream(x.device)))
    return y.reshape(x.shape)


def moe(x, bank: Bank, inds, scores, dec: Decode, verify_rows: bool = False) -> torch.Tensor:
    """`moe` (root.zig:51-53): routed SwiGLU experts over x [..., D] for top-k inds/scores [..., K]."""
    return _moe(x, bank, inds, scores, dec, verify_rows, None, 0)


def moe_with_shared(x, bank: Bank, inds, scores, dec: Decode, verify_rows: bool, shared) -> torch.Tensor:
    """`moeWithShared` (root.zig:56-67): adds an already gated shared expert after the routed output's rounding."""
    return _moe(x, bank, inds, scores, dec, verify_rows, shared, 0)


def moe_with_gated_shared(x, bank: Bank, inds, scores, dec: Decode, verify_rows: bool, down, gate) -> torch.Tensor:
    """`moeWithGatedShared` (root.zig:71-90): routed + sigmoid(gate) * down, with `down` the shared expert's output
    [..., D] and `gate` its logit [..., 1], both in x's dtype, rounded where MLX's Sigmoid, Multiply and Add round."""
    return _moe(x, bank, inds, scores, dec, verify_rows, down, 0, gate)


def moe_clamped(x, bank: Bank, inds, scores, dec: Decode, limit: int, shared=None) -> torch.Tensor:
    """`moeClamped` / `moeClampedWithShared` (root.zig:98-124): gate upper-clamped, up clamped to [-limit, limit]."""
    if limit <= 0 or limit > 128:
        raise InvalidExl3Clamp(f"clamp limit {limit} outside 1..128")
    return _moe(x, bank, inds, scores, dec, False, shared, limit)


def _shared_operands(y: torch.Tensor, rows: int, shared, shared_gate, what: str):
    """`shared` [rows][D] and `shared_gate` [rows] (one logit per row) in the output's dtype, as the C ABI reads them."""
    if shared is not None:
        if shared.numel() != y.numel() or shared.dtype != y.dtype:
            raise BadExl3Shape(f"{what}: the shared expert's output must match the routed output's size and dtype")
        shared = shared.reshape(y.shape).contiguous()
        _need_gpu(shared)
    if shared_gate is not None:
        if shared is None or shared_gate.numel() != rows or shared_gate.dtype != y.dtype:
            raise BadExl3Shape(f"{what}: the shared expert's gate is one logit per row in the output's dtype")
        shared_gate = shared_gate.reshape(rows).contiguous()
        _need_gpu(shared_gate)
    return shared, shared_gate


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def moe_ragged(x, rb: Ragged, inds, scores, dec: Decode, verify_rows: bool = False, shared=None,
               shared_gate=None, limit: int = 0) -> torch.Tensor:
    """`moeRagged` (root.zig:582-644): each expert decodes at its own rate group's rates; `shared` is added after the
    routed output's rounding, as `sigmoid(shared_gate) * shared` when the gate logit [..., 1] is given (the trunk's
    ragged call passes both, trunk.zig:4092)."""
    dec.require_table()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    if hidden != rb.hidden:
        raise BadExl3Shape(f"moe_ragged: hidden {hidden} vs bank {rb.hidden}")
    _need_gpu(x2, inds2, sc2, rb.meta)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    shared, shared_gate = _shared_operands(y, rows, shared, shared_gate, "moe_ragged")
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_workspace_size(rows, topk, hidden, rb.inter))
    cr = rb.c()
    _check(L.exl3_moe_ragged(x2.data_ptr(), _dt(x2, "x"), rows, hidden, rb.inter, ctypes.byref(cr), inds2.data_ptr(),
                             sc2.data_ptr(), _dt(sc2, "scores"), topk, dec.c(), int(verify_rows), int(limit),
                             _ptr(shared), _ptr(shared_gate), y.data_ptr(), _dt(y, "y"), ws.data_ptr(), ws.numel(),
                             _stream(x.device)))
    return y.reshape(x.shape)


EXL3_DECLINED = 1


def moe_groups(x, banks: Sequence[Bank], inds, scores, dec: Decode, verify_rows: bool = False) -> torch.Tensor:
    """`moeGroups` (root.zig:646-703): experts split over several uniform banks (router ids counted across them in
    order); each group's output in f32, summed in group order, rounded to x's dtype once."""
    if len(banks) == 0:
        raise Exl3GroupMissing("moe_groups: no banks")
    dec.require_table()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    shapes = [_bank_shape(b, hidden) for b in banks]
    inter = shapes[0][1]
    if any(i != inter for _, i in shapes):
        raise BadExl3Shape("moe_groups: every bank must share the intermediate width")
    _need_gpu(x2, inds2, sc2)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_groups_workspace_size(rows, topk, hidden, inter))
    cbanks = (_lib.BankT * len(banks))(*[_lib.BankT(b.gate.c(), b.up.c(), b.down.c()) for b in banks])
    counts = (ctypes.c_int32 * len(banks))(*[e for e, _ in shapes])
    _check(L.exl3_moe_groups(x2.data_ptr(), _dt(x2, "x"), rows, hidden, inter, len(banks), cbanks, counts,
                             inds2.data_ptr(), sc2.data_ptr(), _dt(sc2, "scores"), topk, dec.c(), int(verify_rows),
                             y.data_ptr(), _dt(y, "y"), ws.data_ptr(), ws.numel(), _stream(x.device)))
    return y.reshape(x.shape)


_ONE_EXPERT: dict = {}
_ONE_EXPERT_RETIRED: list = []


def _one_expert_routing(rows: int, device: torch.device):
    """Routing of a one-expert chain (every row to expert 0 with score 1), kept per device and grown on demand so a
    call launches no fill kernels (the tensors are never written after they are made)."""
    z, o = _ONE_EXPERT.get(device, (None, None))
    if z is None or z.shape[0] < rows:
        if torch.cuda.is_current_stream_capturing():
            raise Exl3WorkspaceTooSmall("the one-expert routing tensors must exist before a capture: make one eager "
                                        "call first")
        cap = max(rows, 64, 2 * (0 if z is None else z.shape[0]))
        if z is not None:
            _ONE_EXPERT_RETIRED.append((z, o))  # a captured graph may still read the smaller pair
        z = torch.zeros(cap, 1, dtype=torch.int32, device=device)
        o = torch.ones(cap, 1, dtype=torch.float32, device=device)
        torch.cuda.current_stream(device).synchronize()  # filled before any other stream reads them
        _ONE_EXPERT[device] = (z, o)
    return z[:rows], o[:rows]


def _shared_rows(x: torch.Tensor, shared_bank: Bank, dec: Decode, limit: int) -> torch.Tensor:
    """The shared expert as a one-expert chain (inds 0, score 1), the reference callers' pattern
    (src/dsv41/dsv41_model.zig:3000)."""
    lead = tuple(x.shape[:-1])
    rows = x.numel() // int(x.shape[-1])
    z, o = _one_expert_routing(rows, x.device)
    return _moe(x, shared_bank, z.reshape(*lead, 1), o.reshape(*lead, 1), dec, False, None, limit)


def moe_with_shared_bank(x, bank: Bank, shared_bank: Bank, inds, scores, dec: Decode, limit: int = 0,
                         verify_rows: bool = False) -> torch.Tensor:
    """The routed layer and its shared expert in one call: T(T(routed) + T(shared)), the rounding of the reference
    callers' pair of calls (the shared expert as a one-expert chain, then `moeWithShared`, root.zig:56-67).  Where
    the fused form declines (f32 output, a shared rate other than the routed one, rows past the fused finish's
    region) it makes those two calls itself.  ``limit`` > 0 clamps both as `moeClamped` does (root.zig:98-124)."""
    if limit < 0 or limit > 128:
        raise InvalidExl3Clamp(f"clamp limit {limit} outside 1..128 (0 = none)")
    dec.require_table()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    experts, inter = _bank_shape(bank, hidden)
    if _bank_shape(shared_bank, hidden) != (1, inter):
        raise BadExl3Shape("moe_with_shared_bank: the shared bank must be one expert of the routed inter")
    _need_gpu(x2, inds2, sc2)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_with_shared_bank_workspace_size(rows, topk, hidden, inter))
    cb = _lib.BankT(bank.gate.c(), bank.up.c(), bank.down.c())
    cs = _lib.BankT(shared_bank.gate.c(), shared_bank.up.c(), shared_bank.down.c())
    rc = L.exl3_moe_with_shared_bank(x2.data_ptr(), _dt(x2, "x"), rows, hidden, inter, experts, ctypes.byref(cb),
                                     ctypes.byref(cs), inds2.data_ptr(), sc2.data_ptr(), _dt(sc2, "scores"), topk,
                                     dec.c(), int(verify_rows), int(limit), y.data_ptr(), _dt(y, "y"), ws.data_ptr(),
                                     ws.numel(), _stream(x.device))
    if rc == EXL3_DECLINED:
        return _moe(x, bank, inds, scores, dec, verify_rows, _shared_rows(x, shared_bank, dec, limit), limit)
    _check(rc)
    return y.reshape(x.shape)


def moe_ragged_with_shared_bank(x, rb: Ragged, shared_bank: Bank, inds, scores, dec: Decode,
                                limit: int = 0, verify_rows: bool = False) -> torch.Tensor:
    """`moeRagged` (root.zig:582-644) with its shared expert in the same launches (see moe_with_shared_bank); the
    shared bank decodes with the routed codebook at its own rate."""
    if limit < 0 or limit > 128:
        raise InvalidExl3Clamp(f"clamp limit {limit} outside 1..128 (0 = none)")
    dec.require_table()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    if hidden != rb.hidden:
        raise BadExl3Shape(f"moe_ragged_with_shared_bank: hidden {hidden} vs bank {rb.hidden}")
    if _bank_shape(shared_bank, hidden) != (1, rb.inter):
        raise BadExl3Shape("moe_ragged_with_shared_bank: the shared bank must be one expert of the routed inter")
    _need_gpu(x2, inds2, sc2, rb.meta)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_with_shared_bank_workspace_size(rows, topk, hidden, rb.inter))
    cr = rb.c()
    cs = _lib.BankT(shared_bank.gate.c(), shared_bank.up.c(), shared_bank.down.c())
    rc = L.exl3_moe_ragged_with_shared_bank(x2.data_ptr(), _dt(x2, "x"), rows, hidden, rb.inter, ctypes.byref(cr),
                                            ctypes.byref(cs), inds2.data_ptr(), sc2.data_ptr(), _dt(sc2, "scores"),
                                            topk, dec.c(), int(verify_rows), int(limit), y.data_ptr(), _dt(y, "y"),
                                            ws.data_ptr(), ws.numel(), _stream(x.device))
    if rc == EXL3_DECLINED:
        return moe_ragged(x, rb, inds, scores, dec, verify_rows, _shared_rows(x, shared_bank, dec, limit),
                          limit=limit)
    _check(rc)
    return y.reshape(x.shape)


def reconstruct_tiled(tp: TiledProj, expert: int, dec: Decode) -> torch.Tensor:
    """`reconstructInner` (expert_exl3.zig:416-438) of one expert of a per-tile-rate projection, each tile at its own
    rate: [in, out] f16 bits as int16, through the routed GEMV's own decoder."""
    dec.require_table()
    _need_gpu(tp.trellis, tp.seg_off, tp.seg_k1)
    if not 0 <= expert < tp.experts:
        raise BadExl3Shape(f"expert {expert} of {tp.experts}")
    out = torch.empty(tp.in_features, tp.out_features, dtype=torch.int16, device=tp.trellis.device)
    _check(_lib.load().exl3_reconstruct_tiled(tp.trellis.data_ptr(), tp.seg_off.data_ptr(), tp.seg_k1.data_ptr(),
                                              int(expert), tp.in_features, tp.out_features, TILED_RATES[0],
                                              TILED_RATES[1], dec.c(), out.data_ptr(), _stream(out.device)))
    return out


def moe_tiled(x, tb: Tiled, inds, scores, dec: Decode, shared=None, limit: int = 0, verify_rows: bool = False,
              shared_gate=None) -> torch.Tensor:
    """The routed SwiGLU chain (`moeRagged`, root.zig:582-644) over a per-tile-rate bank; `shared`, `shared_gate`,
    `verify_rows` and `limit` as for moe_ragged."""
    if limit < 0 or limit > 128:
        raise InvalidExl3Clamp(f"clamp limit {limit} outside 1..128 (0 = none)")
    dec.require_table()
    tb.check()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    if hidden != tb.hidden:
        raise BadExl3Shape(f"moe_tiled: hidden {hidden} vs bank {tb.hidden}")
    _need_gpu(x2, inds2, sc2, tb.gate.trellis)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    shared, shared_gate = _shared_operands(y, rows, shared, shared_gate, "moe_tiled")
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_workspace_size(rows, topk, hidden, tb.inter))
    ct = tb.c()
    _check(L.exl3_moe_tiled(x2.data_ptr(), _dt(x2, "x"), rows, hidden, tb.inter, ctypes.byref(ct), inds2.data_ptr(),
                            sc2.data_ptr(), _dt(sc2, "scores"), topk, dec.c(), int(verify_rows), int(limit),
                            _ptr(shared), _ptr(shared_gate), y.data_ptr(), _dt(y, "y"), ws.data_ptr(), ws.numel(),
                            _stream(x.device)))
    return y.reshape(x.shape)


def moe_tiled_with_shared_bank(x, tb: Tiled, shared_bank: Bank, inds, scores, dec: Decode,
                               limit: int = 0, verify_rows: bool = False) -> torch.Tensor:
    """moe_tiled with its shared expert (a uniform one-expert bank) in the same launches, as moe_with_shared_bank;
    where the fused form declines, the shared expert runs as a one-expert chain and joins through `shared`."""
    if limit < 0 or limit > 128:
        raise InvalidExl3Clamp(f"clamp limit {limit} outside 1..128 (0 = none)")
    dec.require_table()
    tb.check()
    x2, inds2, sc2, rows, topk = _moe_prep(x, inds, scores)
    hidden = int(x.shape[-1])
    if hidden != tb.hidden:
        raise BadExl3Shape(f"moe_tiled_with_shared_bank: hidden {hidden} vs bank {tb.hidden}")
    if _bank_shape(shared_bank, hidden) != (1, tb.inter):
        raise BadExl3Shape("moe_tiled_with_shared_bank: the shared bank must be one expert of the routed inter")
    _need_gpu(x2, inds2, sc2, tb.gate.trellis)
    y = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    L = _lib.load()
    ws = workspace.get(x.device, L.exl3_moe_with_shared_bank_workspace_size(rows, topk, hidden, tb.inter))
    ct = tb.c()
    cs = _lib.BankT(shared_bank.gate.c(), shared_bank.up.c(), shared_bank.down.c())
    rc = L.exl3_moe_tiled_with_shared_bank(x2.data_ptr(), _dt(x2, "x"), rows, hidden, tb.inter, ctypes.byref(ct),
                                           ctypes.byref(cs), inds2.data_ptr(), sc2.data_ptr(), _dt(sc2, "scores"),
                                           topk, dec.c(), int(verify_rows), int(limit), y.data_ptr(), _dt(y, "y"),
                                           ws.data_ptr(), ws.numel(), _stream(x.device))
    if rc == EXL3_DECLINED:
        return moe_tiled(x, tb, inds, scores, dec, _shared_rows(x, shared_bank, dec, limit), limit, verify_rows)
    _check(rc)
    return y.reshape(x.shape)


def moe_routing_chain(router_logits: torch.Tensor, k: int):
    """`moeRoutingChain` (moe_router.zig:16-62): (inds [.., k] i32, norm_scores [.., k] f32)."""
    lg = router_logits.to(torch.float32).contiguous()
    _need_gpu(lg)
    experts = int(lg.shape[-1])
    rows = lg.numel() // experts
    inds = torch.empty(*lg.shape[:-1], k, dtype=torch.int32, device=lg.device)
    scores = torch.empty(*lg.shape[:-1], k, dtype=torch.float32, device=lg.device)
    _check(_lib.load().exl3_route_topk(lg.data_ptr(), rows, experts, k, inds.data_ptr(), scores.data_ptr(),
                                       _stream(lg.device)))
    return inds, scores


def tile_major(trellis: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """`layout.tileMajor` (layout.zig:139-158) over [E, IT, OT, n]; ``inverse`` undoes it."""
    _need_gpu(trellis)
    e, it, ot, n = (int(v) for v in trellis.shape)
    out = torch.empty_like(trellis)
    _check(_lib.load().exl3_tile_major(trellis.data_ptr(), out.data_ptr(), e, it, ot, n, int(inverse),
                                       _stream(trellis.device)))
    return out


def encode_tiles(tiles: torch.Tensor, n: int, dec: Decode, with_sse: bool = True):
    """`Encoder.encodeTile` (src/encoder/encode.zig:170-309) over a batch on the GPU: row-major 16x16 f32 tiles
    [..., 256] (or [..., 16, 16]) -> (packed codes [..., n] as int16, f64 squared errors [...] or None)."""
    t = tiles.to(torch.float32).contiguous()
    _need_gpu(t)
    count = t.numel() // 256
    if t.numel() != count * 256:
        raise BadExl3Shape(f"tiles of {t.numel()} values are not whole 16x16 tiles")
    lead = t.shape[:-2] if t.dim() >= 2 and tuple(t.shape[-2:]) == (16, 16) else t.shape[:-1]
    L = _lib.load()
    ws_bytes = L.exl3_encode_workspace_size(n, dec.c(), count)
    if ws_bytes == 0 and count > 0:
        _check(L.exl3_encode_tiles(0, count, n, dec.c(), 0, 0, 0, 0, _stream(t.device)))
    packed = torch.empty(count, n, dtype=torch.int16, device=t.device)
    sse = torch.empty(count, dtype=torch.float64, device=t.device) if with_sse else None
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=t.device)
    _check(L.exl3_encode_tiles(t.data_ptr(), count, n, dec.c(), packed.data_ptr(),
                               0 if sse is None else sse.data_ptr(), ws.data_ptr(), ws.numel(), _stream(t.device)))
    return packed.reshape(*lead, n), (None if sse is None else sse.reshape(lead))


# ---------------------------------------------------------------------------------------------------------------
# Quantizer (src/encoder/quantize.zig)

OUT_SCALES = {"auto": 0, "always": 1, "never": 2}
_M64 = (1 << 64) - 1


def _splitmix(x: int) -> int:
    z = (x + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def signs(seed: int, name: str, length: int):
    """`signs` (quantize.zig:567-583): a +-1 f32 vector, a pure function of (seed, name, length): splitmix64 seeded by
    mixing `seed` with every byte of `name`, -1 where bit 0 of the i-th output is set."""
    import numpy as np

    state = seed & _M64
    for b in name.encode():
        state = _splitmix(state ^ b)
    state = _splitmix(state)
    out = np.empty(length, np.float32)
    for i in range(length):
        state = _splitmix(state)
        out[i] = -1.0 if state & 1 else 1.0
    return out


def quantize_tensor(w, h, sign_in, sign_out, n: int, dec: Decode, out_scales: str = "auto", device="cuda"):
    """`quantizeTensor` (quantize.zig:600-626) on the GPU: public weight w [in, out] and input Hessian h [in, in] (host
    arrays) -> (packed [in/16, out/16, n] u16, suh [in] and svh [out] as f16 bits, global scale g)."""
    import numpy as np

    w = np.ascontiguousarray(w, np.float32)
    h = np.ascontiguousarray(h, np.float32)
    si = np.ascontiguousarray(sign_in, np.float32)
    so = np.ascontiguousarray(sign_out, np.float32)
    if w.ndim != 2 or h.shape != (w.shape[0], w.shape[0]) or si.shape != (w.shape[0],) or so.shape != (w.shape[1],):
        raise BadExl3Shape(f"w {w.shape}, h {h.shape}, signs {si.shape} / {so.shape}")
    rows, cols = w.shape
    L = _lib.load()
    dev = torch.device(device)
    ws_bytes = L.exl3_quantize_workspace_size(rows, cols, n, dec.c())
    packed = np.zeros((max(rows // 16, 0), max(cols // 16, 0), n), np.uint16)
    suh = np.zeros(rows, np.uint16)
    svh = np.zeros(cols, np.uint16)
    g = np.zeros(1, np.float32)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    _check(L.exl3_quantize_tensor(p(w), p(h), rows, cols, p(si), p(so), n, dec.c(), OUT_SCALES[out_scales], p(packed),
                                  p(suh), p(svh), p(g), ws.data_ptr(), ws.numel(), _stream(dev)))
    return packed, suh, svh, float(g[0])


def quantize_named(w, h, seed: int, name: str, n: int, dec: Decode, out_scales: str = "auto", device="cuda"):
    """`quantizeNamed` (quantize.zig:592-598): `quantize_tensor` with the sign vectors of (seed, name)."""
    both = signs(seed, name, w.shape[0] + w.shape[1])
    return quantize_tensor(w, h, both[:w.shape[0]], both[w.shape[0]:], n, dec, out_scales, device)
