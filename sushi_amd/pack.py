"""EXL3/STQ pack loader: the on-disk format the trellis kernels consume, read into device banks.

Follows the reference's consumer contract for packs:

* ``expert_quant`` / ``trunk_quant`` parse with its named refusals (src/exl3/root.zig:190-292) and the codebook-table
  resolution (src/exl3/codebook_tables.zig:266-279);
* shard stamps in a shard's safetensors ``__metadata__`` (src/exl3/root.zig:264-292, src/pack_index.zig:36-50,
  :259-292);
* routed-expert tensor names, rate groups ``.gN`` and the ``trellis_pm`` (pair-major) tile order, validated per layer
  (src/exl3/layout.zig:1-137, src/exl3/pack.zig:70-175, src/pack_index.zig:317-338);
* the safetensors index and shard headers (src/pack_index.zig:100-258);
* trunk linears stored as trellis banks under ``trunk_quant`` (src/trunk_stq.zig:31-71).

A layer's tensors are read from the shards (memory-mapped), copied to the device as they are stored, and a pair-major
trellis is put back into the pack order on the GPU by the library's tile-major kernel; nothing is reshuffled on the
CPU.  A uniform layer becomes an ``exl3.Bank``; a rate-grouped one an ``exl3.Ragged`` (experts in group order, so
router index e is (group, local) by cumulative group sizes).
"""
from __future__ import annotations

import json
import math
import os
import re
from dataclasses import dataclass, field
from typing import Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np

from . import exl3
from .exl3 import Codebook, Exl3Error, Rate, Table, Window

# ---------------------------------------------------------------------------------------------------------------
# Named refusals (the reference's error names; src/exl3/root.zig, layout.zig, codebook_tables.zig, pack_index.zig)


class PackError(Exl3Error):
    """A pack the loader refuses; the subclass name is the reference's error name."""


def _err(name: str) -> type:
    cls = type(name, (PackError,), {})
    globals()[name] = cls
    return cls


for _name in (
        "ExpertLayoutUnsupported", "Exl3TileOrderUnsupported", "Exl3TileOrderMixed", "Exl3TileOrderMismatch",
        "Exl3TileOrderNeedsGroups", "Exl3ShardStampMismatch", "Exl3CodebookTableDigestMismatch",
        "Exl3CodebookTableLegacyConfig", "Exl3CodebookTableCodebookMismatch", "Exl3CodebookTableWindowMismatch",
        "Exl3GroupNameInvalid", "Exl3GroupMissing", "Exl3GroupGeometry", "Exl3GroupDtype", "Exl3MixedGroupLayout",
        "Exl3TrellisGeometry", "Exl3RouterWidthMismatch", "Exl3TopKExceedsExperts", "ExpertOutOfRange", "MissingWeight",
        "InvalidSafetensorsIndex", "AmbiguousSafetensorsIndex", "InvalidSafetensorsHeader", "SafetensorsHeaderTooLarge",
        "AmbiguousSafetensorsTensor", "SafetensorsPayloadMismatch", "MissingIndexedSafetensorsTensor",
        "MissingPackShard", "UnsupportedPackTensorDtype", "TrunkQuantMissing", "TrunkStqLayout"):
    _err(_name)

# The named errors the format types already raise (exl3.py) keep their classes.
Exl3CodebookTableUnknown = exl3.Exl3CodebookTableUnknown
Exl3CodebookTableRateMissing = exl3.Exl3CodebookTableRateMissing
Exl3WindowUnsupported = exl3.Exl3WindowUnsupported
Exl3TopKExceedsReduceBank = exl3.Exl3TopKExceedsReduceBank


def _refuse(name: str, detail: str = "") -> PackError:
    return globals()[name](f"{name}: {detail}" if detail else name)


# ---------------------------------------------------------------------------------------------------------------
# Codebook tables the library holds (sushi_amd/csrc/exl3_tables.h), as a pack names them (codebook_tables.zig:101-106)


@dataclass(frozen=True)
class CodebookTable:
    name: str
    table: Table
    codebook: Codebook
    digest: str
    n_lo: int
    n_hi: int
    own_window: Optional[int] = None   # PAIR1 reads the whole 16-bit window: it holds at its own window only
    superseded: Tuple[str, ...] = ()   # retired digests of the same table (Exl3CodebookTableLegacyConfig)

    def rates(self) -> frozenset:
        return frozenset(range(self.n_lo, self.n_hi + 1, 2))

    def admits(self, window: Window) -> bool:
        return self.own_window is None or window.bits == self.own_window


SHIPPED_TABLES: Dict[str, CodebookTable] = {t.name: t for t in (
    CodebookTable("pair1-w16-v1", Table.pair1_w16_v1, Codebook.pair1, "c089b4eb", 24, 64, own_window=16),
    CodebookTable("spec1-w15", Table.spec1_w15, Codebook.spec1, "37f72431", 16, 128, superseded=("2ac2594d",)),
    CodebookTable("spec1-w16", Table.spec1_w16, Codebook.spec1, "753ffa03", 24, 64),
    CodebookTable("std1", Table.std1, Codebook.std1, "c5dba171", 24, 64),
)}


def resolve_table(block: Mapping, codebook: Codebook, window: Window) -> CodebookTable:
    """`codebook_tables.resolve` (codebook_tables.zig:266-279): the table ``block`` names, refusing by name."""
    if not codebook.has_table():
        raise _refuse("Exl3CodebookTableCodebookMismatch", f"{codebook.name} has no table")
    name = block.get("codebook_table")
    if not isinstance(name, str) or name not in SHIPPED_TABLES:
        raise Exl3CodebookTableUnknown(f"Exl3CodebookTableUnknown: {name!r}")
    table = SHIPPED_TABLES[name]
    digest = block.get("codebook_digest")
    if not isinstance(digest, str):
        raise _refuse("Exl3CodebookTableDigestMismatch", "no digest")
    if digest in table.superseded:
        raise _refuse("Exl3CodebookTableLegacyConfig", f"{name} digest {digest} was retired for {table.digest}")
    if digest != table.digest:
        raise _refuse("Exl3CodebookTableDigestMismatch", f"{name}: {digest} != {table.digest}")
    if table.codebook != codebook:
        raise _refuse("Exl3CodebookTableCodebookMismatch", f"{name} is a {table.codebook.name} table")
    if not table.admits(window):
        raise _refuse("Exl3CodebookTableWindowMismatch", f"{name} holds at window {table.own_window} only")
    return table


# ---------------------------------------------------------------------------------------------------------------
# expert_quant / trunk_quant (src/exl3/root.zig:190-262)

PACK = "pack"
PAIR_MAJOR = "pair_major"


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def rate_from_config_k(k) -> Optional[Rate]:
    """`rateFromConfigK` (root.zig:203-215): a JSON number whose 16k is a whole, even, admitted halfword count."""
    if _is_int(k):
        scaled = float(k) * 16.0
    elif isinstance(k, float):
        scaled = k * 16.0
    else:
        return None
    if not math.isfinite(scaled):
        return None
    rounded = round(scaled)
    if abs(scaled - rounded) > 1e-6 or rounded < 0 or rounded > 1024:
        return None
    return exl3.k_from_packed_dim(int(rounded))


def window_from_config(block: Mapping) -> Optional[Window]:
    """`windowFromConfig` (root.zig:217-224): absent is 16; an integer 8..16 otherwise, never rounded."""
    if "window" not in block:
        return Window(16)
    raw = block["window"]
    return Window.from_bits(raw) if _is_int(raw) else None


@dataclass(frozen=True)
class Spec:
    """`Spec` (root.zig:190-201): a pack's rate ceiling, codebook, window, table and routed tile order."""

    rate: Rate
    codebook: Codebook
    window: Window = Window(16)
    rates: Optional[frozenset] = None    # the table's rates; None admits every rate up to the ceiling
    table: Optional[Table] = None
    tile_order: str = PACK

    def admits(self, n: int) -> bool:
        return self.rates is None or n in self.rates

    def decode(self) -> exl3.Decode:
        return exl3.Decode(self.codebook, self.window, None if self.table is None else int(self.table))


def parse_quant_block(block) -> Spec:
    """`parseQuantBlock` (root.zig:237-262): format, k, codebook, window and the STQ table of one quant block.

    ``format`` ``exl3`` carries the untabled codebooks (``mul1``, ``mcg``, and this build's ``3inst`` extension),
    ``stq`` the ones that name a table (``std1``, ``spec1``, ``pair1``)."""
    if not isinstance(block, dict):
        raise _refuse("ExpertLayoutUnsupported", "quant block is not an object")
    fmt = block.get("format")
    if not isinstance(fmt, str) or fmt not in ("exl3", "stq"):
        raise _refuse("ExpertLayoutUnsupported", f"format {fmt!r}")
    stq = fmt == "stq"
    if "k" not in block:
        raise _refuse("ExpertLayoutUnsupported", "no k")
    rate = rate_from_config_k(block["k"])
    if rate is None:
        raise _refuse("ExpertLayoutUnsupported", f"k {block['k']!r}")
    cb_name = block.get("codebook")
    codebook = Codebook.from_name(cb_name) if isinstance(cb_name, str) else None
    if codebook is None:
        raise _refuse("ExpertLayoutUnsupported", f"codebook {cb_name!r}")
    if codebook.has_table() != stq:
        raise _refuse("ExpertLayoutUnsupported", f"codebook {cb_name} under format {fmt}")
    window = window_from_config(block)
    if window is None:
        raise Exl3WindowUnsupported(f"Exl3WindowUnsupported: window {block.get('window')!r}")
    if not codebook.has_table():
        if "codebook_table" in block:
            raise _refuse("Exl3CodebookTableCodebookMismatch", f"{cb_name} names no table")
        return Spec(rate, codebook, window)
    table = resolve_table(block, codebook, window)
    if rate.n not in table.rates():
        raise Exl3CodebookTableRateMissing(f"Exl3CodebookTableRateMissing: {table.name} has no row for n={rate.n}")
    return Spec(rate, codebook, window, table.rates(), table.table)


def parse_expert_quant(config: Mapping) -> Spec:
    """`parseExpertQuant` (root.zig:226-235): the routed experts' block and its ``tile_order``."""
    block = config.get("expert_quant")
    if block is None:
        raise _refuse("ExpertLayoutUnsupported", "config has no expert_quant")
    spec = parse_quant_block(block)
    if "tile_order" in block:
        v = block["tile_order"]
        if v != PAIR_MAJOR:
            raise _refuse("Exl3TileOrderUnsupported", f"tile_order {v!r}")
        spec = Spec(spec.rate, spec.codebook, spec.window, spec.rates, spec.table, PAIR_MAJOR)
    return spec


def shard_tile_order_agrees(order: str, stamp: Optional[str]) -> None:
    """`shardTileOrderAgrees` (root.zig:264-269): a shard of routed trellis tensors stamps ``pair_major`` or nothing."""
    if stamp is None:
        stamped = PACK
    elif stamp == PAIR_MAJOR:
        stamped = PAIR_MAJOR
    else:
        raise _refuse("Exl3ShardStampMismatch", f"tile_order stamp {stamp!r}")
    if stamped != order:
        raise _refuse("Exl3ShardStampMismatch", f"shard stamps {stamped}, config names {order}")


def shard_stamp_agrees(spec: Spec, k: Optional[str], codebook: Optional[str], window: Optional[str]) -> None:
    """`shardStampAgrees` (root.zig:271-292): a shard's decoder stamps, every one a string, must be the config's.

    A narrower ``k`` is over-billed, not wrong; only a wider stamp refuses."""
    if codebook is not None and Codebook.from_name(codebook) != spec.codebook:
        raise _refuse("Exl3ShardStampMismatch", f"codebook stamp {codebook!r}")
    if window is not None:
        if not re.fullmatch(r"[+-]?[0-9]+", window):
            raise _refuse("Exl3ShardStampMismatch", f"window stamp {window!r}")
        w = Window.from_bits(int(window))
        if w is None or w != spec.window:
            raise _refuse("Exl3ShardStampMismatch", f"window stamp {window!r}")
    if k is not None:
        try:
            if not re.fullmatch(r"[0-9A-Za-z.+-]+", k):
                raise ValueError(k)
            rate_k = float(k)
        except ValueError:
            raise _refuse("Exl3ShardStampMismatch", f"k stamp {k!r}") from None
        if not math.isfinite(rate_k):
            raise _refuse("Exl3ShardStampMismatch", f"k stamp {k!r}")
        scaled = round(rate_k * 16.0)
        if abs(rate_k * 16.0 - scaled) > 1e-6 or scaled < Rate.MIN_N or scaled > Rate.MAX_N:
            raise _refuse("Exl3ShardStampMismatch", f"k stamp {k!r}")
        rate = exl3.k_from_packed_dim(int(scaled))
        if rate is None or rate.n > spec.rate.n:
            raise _refuse("Exl3ShardStampMismatch", f"k stamp {k!r} above the config's {spec.rate.n / 16:g}")


# ---------------------------------------------------------------------------------------------------------------
# Routed-expert tensor names and a layer's group layout (src/exl3/layout.zig:1-137)

MAX_GROUPS = 32
REDUCE_MAX_TOPK = 32   # top-k the MoE finish holds per row (REDUCE_MAX_TOPK, expert_exl3_kernels.zig:2562)
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
PARTS = ("trellis", "suh", "svh")


@dataclass(frozen=True)
class Name:
    """`Name.parse` (layout.zig:14-33): ``<gate|up|down>_proj[.gN].<trellis|trellis_pm|suh|svh>``."""

    group: int
    projection: int
    part: int
    grouped: bool
    pair_major: bool = False

    @classmethod
    def parse(cls, suffix: str) -> "Name":
        bits = suffix.split(".")
        if len(bits) < 2 or bits[0] not in PROJECTIONS:
            raise _refuse("Exl3GroupNameInvalid", suffix)
        proj = PROJECTIONS.index(bits[0])
        rest = bits[1:]
        group, grouped = 0, rest[0].startswith("g")
        if grouped:
            g = rest[0]
            if len(g) < 2 or (len(g) > 2 and g[1] == "0") or not g[1:].isdigit() or not g[1:].isascii():
                raise _refuse("Exl3GroupNameInvalid", suffix)
            group = int(g[1:])
            if group >= MAX_GROUPS:
                raise _refuse("Exl3GroupNameInvalid", suffix)
            rest = rest[1:]
        if len(rest) != 1:
            raise _refuse("Exl3GroupNameInvalid", suffix)
        leaf = rest[0]
        pair_major = leaf == "trellis_pm"
        if pair_major or leaf == "trellis":
            part = 0
        elif leaf in ("suh", "svh"):
            part = PARTS.index(leaf)
        else:
            raise _refuse("Exl3GroupNameInvalid", suffix)
        return cls(group, proj, part, grouped, pair_major)

    @property
    def tile_order(self) -> str:
        return PAIR_MAJOR if self.pair_major else PACK


def tile_dims(order: str, shape: Sequence[int]) -> Optional[Tuple[int, int, int]]:
    """`tileDims` (layout.zig:40-47): (IT, OT, n) of ``[E, IT, OT, n]``, or of ``[E, OT/2, IT, 2, n]`` pair-major."""
    if order == PACK:
        return (shape[1], shape[2], shape[3]) if len(shape) == 4 else None
    if len(shape) == 5 and shape[3] == 2:
        return (shape[2], shape[1] * 2, shape[4])
    return None


def trellis_rate(order: str, shape: Sequence[int], inp: int, out: int) -> Rate:
    """`trellisRate` (layout.zig:56-62): a trellis's grid must be its projection's; its n an admitted rate."""
    dims = tile_dims(order, shape)
    if dims is None or dims[0] != inp // 16 or dims[1] != out // 16:
        raise _refuse("Exl3GroupGeometry", f"{order} trellis {tuple(shape)} for {inp}x{out}")
    rate = exl3.k_from_packed_dim(int(dims[2]))
    if rate is None:
        raise _refuse("Exl3TrellisGeometry", f"n={dims[2]}")
    return rate


@dataclass
class Group:
    experts: int = 0
    rates: List[int] = field(default_factory=lambda: [0, 0, 0])
    mask: int = 0


class Layout:
    """`Layout` (layout.zig:64-137): one MoE layer's routed banks, validated tensor by tensor, then as a whole."""

    def __init__(self, hidden: int, intermediate: int, ceiling: Rate, rates: Optional[frozenset] = None):
        self.hidden = hidden
        self.intermediate = intermediate
        self.ceiling = ceiling
        self.rates = rates
        self.groups = [Group() for _ in range(MAX_GROUPS)]
        self.count = 0
        self.grouped: Optional[bool] = None
        self.tile_order: Optional[str] = None
        self.bytes = 0

    def add(self, suffix: str, shape: Sequence[int], dtype: str) -> Name:
        """`Layout.add` (layout.zig:86-120); ``dtype`` is the safetensors dtype name."""
        name = Name.parse(suffix)
        if self.grouped is not None and self.grouped != name.grouped:
            raise _refuse("Exl3MixedGroupLayout", suffix)
        if dtype != ("U16" if name.part == 0 else "F16"):
            raise _refuse("Exl3GroupDtype", f"{suffix} is {dtype}")
        inp, out = (self.intermediate, self.hidden) if name.projection == 2 else (self.hidden, self.intermediate)
        if inp <= 0 or out <= 0 or inp % 128 or out % 128:
            raise _refuse("Exl3GroupGeometry", f"{inp}x{out} is off the 128 grid")
        if name.part != 0 and len(shape) != 2:
            raise _refuse("Exl3GroupGeometry", f"{suffix} {tuple(shape)}")
        if len(shape) == 0 or shape[0] == 0 or shape[0] > 2 ** 31 - 1:
            raise _refuse("Exl3GroupGeometry", f"{suffix} {tuple(shape)}")
        group = self.groups[name.group]
        if group.experts != 0 and group.experts != shape[0]:
            raise _refuse("Exl3GroupGeometry", f"{suffix}: {shape[0]} experts, the group has {group.experts}")
        n = 0
        if name.part == 0:
            if self.tile_order is not None and self.tile_order != name.tile_order:
                raise _refuse("Exl3TileOrderMixed", suffix)
            n = trellis_rate(name.tile_order, shape, inp, out).n
            if n > self.ceiling.n:
                raise _refuse("Exl3TrellisGeometry", f"{suffix}: n={n} above the config's n={self.ceiling.n}")
            if self.rates is not None and n not in self.rates:
                raise Exl3CodebookTableRateMissing(f"Exl3CodebookTableRateMissing: {suffix} n={n}")
        elif shape[1] != (inp if name.part == 1 else out):
            raise _refuse("Exl3GroupGeometry", f"{suffix} {tuple(shape)}")
        bit = 1 << (name.projection * 3 + name.part)
        if group.mask & bit:
            raise _refuse("Exl3GroupNameInvalid", f"{suffix} twice")
        self.bytes += 2 * int(np.prod([int(d) for d in shape], dtype=np.uint64))
        self.grouped = name.grouped
        if name.part == 0:
            self.tile_order = name.tile_order
        self.count = max(self.count, name.group + 1)
        group.experts = int(shape[0])
        group.mask |= bit
        if name.part == 0:
            group.rates[name.projection] = n
        return name

    def finish(self, router_experts: int, topk: int) -> None:
        """`Layout.finish` (layout.zig:122-134), without the streaming engine's checks (every layer is resident)."""
        if self.count == 0:
            raise _refuse("MissingWeight", "no routed tensors")
        total = 0
        for g in self.groups[:self.count]:
            if g.mask != 511:
                raise _refuse("Exl3GroupMissing" if self.grouped else "MissingWeight", f"group mask {g.mask:#x}")
            total += g.experts
        if total != router_experts or total > 2 ** 31 - 1:
            raise _refuse("Exl3RouterWidthMismatch", f"{total} experts, the router has {router_experts}")
        if topk > router_experts:
            raise _refuse("Exl3TopKExceedsExperts", f"top-{topk} of {router_experts}")
        if topk > REDUCE_MAX_TOPK:
            raise Exl3TopKExceedsReduceBank(f"Exl3TopKExceedsReduceBank: top-{topk}")

    def locate(self, expert: int) -> Tuple[int, int]:
        """`Layout.locate` (layout.zig:128-136): router index -> (group, local) by cumulative group sizes."""
        offset = 0
        for i, g in enumerate(self.groups[:self.count]):
            if offset <= expert < offset + g.experts:
                return i, expert - offset
            offset += g.experts
        raise _refuse("ExpertOutOfRange", str(expert))


# ---------------------------------------------------------------------------------------------------------------
# safetensors shards and the index (src/pack_index.zig:100-258)

MAX_HEADER_BYTES = 512 * 1024 * 1024
PAD_PREFIX = "__pad__."
INDEX_FILE = "model.safetensors.index.json"
SINGLE_FILE = "model.safetensors"

DTYPES: Dict[str, np.dtype] = {
    "F16": np.dtype("<f2"), "BF16": np.dtype("<u2"), "F32": np.dtype("<f4"), "F64": np.dtype("<f8"),
    "U8": np.dtype("u1"), "I8": np.dtype("i1"), "U16": np.dtype("<u2"), "I16": np.dtype("<i2"),
    "U32": np.dtype("<u4"), "I32": np.dtype("<i4"), "U64": np.dtype("<u8"), "I64": np.dtype("<i8"),
    "BOOL": np.dtype("u1"), "F8_E4M3": np.dtype("u1"), "F8_E4M3FN": np.dtype("u1"), "F8_E5M2": np.dtype("u1"),
}


def _no_duplicates(what: str):
    def hook(pairs):
        out = {}
        for k, v in pairs:
            if k in out:
                raise _refuse(what, f"key {k!r} twice")
            out[k] = v
        return out
    return hook


@dataclass(frozen=True)
class TensorMeta:
    dtype: str
    shape: Tuple[int, ...]
    start: int      # data_offsets, relative to the data section
    end: int
    base: int       # file offset of the data section (8 + header length)
    file: str

    @property
    def nbytes(self) -> int:
        return self.end - self.start


def _shape(v) -> Tuple[int, ...]:
    if not isinstance(v, list) or not all(_is_int(d) and d >= 0 for d in v):
        raise _refuse("InvalidSafetensorsHeader", f"shape {v!r}")
    return tuple(v)


def _offsets(v) -> Tuple[int, int]:
    if not isinstance(v, list) or len(v) != 2 or not all(_is_int(d) and d >= 0 for d in v) or v[1] < v[0]:
        raise _refuse("InvalidSafetensorsHeader", f"data_offsets {v!r}")
    return v[0], v[1]


class Shard:
    """One safetensors file: its header (tensors and ``__metadata__``), read without loading any data."""

    def __init__(self, path: str):
        self.path = path
        self.file = os.path.basename(path)
        try:
            size = os.path.getsize(path)
            with open(path, "rb") as f:
                head = f.read(8)
                if len(head) != 8:
                    raise _refuse("InvalidSafetensorsHeader", f"{self.file}: shorter than 8 bytes")
                hlen = int.from_bytes(head, "little")
                if hlen > MAX_HEADER_BYTES:
                    raise _refuse("SafetensorsHeaderTooLarge", f"{self.file}: {hlen} bytes")
                if 8 + hlen > size:
                    raise _refuse("InvalidSafetensorsHeader", f"{self.file}: header past the end of the file")
                raw = f.read(hlen)
        except FileNotFoundError:
            raise _refuse("MissingPackShard", path) from None
        try:
            header = json.loads(raw.decode("utf-8"), object_pairs_hook=_no_duplicates("AmbiguousSafetensorsTensor"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise _refuse("InvalidSafetensorsHeader", f"{self.file}: {e}") from None
        if not isinstance(header, dict):
            raise _refuse("InvalidSafetensorsHeader", f"{self.file}: not an object")
        self.base = 8 + hlen
        meta = header.pop("__metadata__", None)
        self.metadata: Dict[str, str] = {k: v for k, v in meta.items() if isinstance(v, str)} \
            if isinstance(meta, dict) else {}
        self.tensors: Dict[str, TensorMeta] = {}
        spans = []
        for key, v in header.items():
            if not isinstance(v, dict) or not isinstance(v.get("dtype"), str):
                raise _refuse("InvalidSafetensorsHeader", f"{self.file}: {key}")
            shape = _shape(v.get("shape"))
            start, end = _offsets(v.get("data_offsets"))
            if self.base + end > size:
                raise _refuse("InvalidSafetensorsHeader", f"{self.file}: {key} runs past the end of the file")
            t = TensorMeta(v["dtype"], shape, start, end, self.base, self.file)
            dt = DTYPES.get(t.dtype)
            if dt is not None and int(np.prod(shape, dtype=np.uint64)) * dt.itemsize != t.nbytes:
                raise _refuse("SafetensorsPayloadMismatch", f"{self.file}: {key} {t.dtype} {shape} in {t.nbytes} B")
            self.tensors[key] = t
            spans.append((start, end, key))
        spans.sort()
        for (s0, e0, k0), (s1, e1, k1) in zip(spans, spans[1:]):
            if s1 < e0 and e0 > s0 and e1 > s1:
                raise _refuse("InvalidSafetensorsHeader", f"{self.file}: {k0} and {k1} overlap")

    def stamp(self) -> Tuple[Optional[str], Optional[str], Optional[str]]:
        """`readShardStamp` (pack_index.zig:259-270): the decoder a converter stamped (k, codebook, window)."""
        return self.metadata.get("k"), self.metadata.get("codebook"), self.metadata.get("window")

    def read(self, key: str) -> np.ndarray:
        """The tensor's stored bytes, memory-mapped (copy-on-write: the file is never written)."""
        t = self.tensors[key]
        dt = DTYPES.get(t.dtype)
        if dt is None:
            raise _refuse("UnsupportedPackTensorDtype", f"{key}: {t.dtype}")
        count = t.nbytes // dt.itemsize
        if count == 0:
            return np.zeros(t.shape, dtype=dt)
        mm = np.memmap(self.path, dtype=dt, mode="c", offset=t.base + t.start, shape=(count,))
        return mm.reshape(t.shape)


def write_shard(path: str, tensors: Mapping[str, np.ndarray], metadata: Optional[Mapping[str, str]] = None,
                dtypes: Optional[Mapping[str, str]] = None, align: int = 8) -> None:
    """Writes one safetensors file: 8-byte little-endian header length, the JSON header padded with spaces so the data
    starts on ``align`` bytes, then each tensor's bytes in the order given.  ``dtypes`` names a tensor's safetensors
    dtype where numpy's cannot (``U16`` trellis tiles held as int16, ``BF16``)."""
    np_names = {np.dtype("<f2"): "F16", np.dtype("<f4"): "F32", np.dtype("<f8"): "F64", np.dtype("u1"): "U8",
                np.dtype("i1"): "I8", np.dtype("<u2"): "U16", np.dtype("<i2"): "I16", np.dtype("<u4"): "U32",
                np.dtype("<i4"): "I32", np.dtype("<u8"): "U64", np.dtype("<i8"): "I64"}
    header: Dict[str, object] = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    blobs, off = [], 0
    for key, arr in tensors.items():
        a = np.ascontiguousarray(arr)
        name = (dtypes or {}).get(key) or np_names[a.dtype.newbyteorder("<") if a.dtype.byteorder == ">" else a.dtype]
        b = a.tobytes()
        header[key] = {"dtype": name, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    text = json.dumps(header, separators=(",", ":")).encode()
    pad = (-(8 + len(text))) % align
    text += b" " * pad
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little"))
        f.write(text)
        for b in blobs:
            f.write(b)


# ---------------------------------------------------------------------------------------------------------------
# A pack directory

# The routed nesting of each arch (pack.zig:70-72); a pack uses one of them for every routed layer it owns.
EXL3_PREFIXES = ("language_model.model.layers.", "model.layers.", "model.language_model.layers.")
SWITCH = ".mlp.switch_mlp."


def tile_order_of_keys(keys) -> str:
    """`tileOrderOfMap` (pack.zig:159-170): the order every routed trellis key names; both is mixed."""
    seen_pack = seen_major = False
    for key in keys:
        at = key.find(SWITCH)
        if at < 0:
            continue
        try:
            name = Name.parse(key[at + len(SWITCH):])
        except PackError:
            continue
        if name.part != 0:
            continue
        if name.pair_major:
            seen_major = True
        else:
            seen_pack = True
    if seen_pack and seen_major:
        raise _refuse("Exl3TileOrderMixed", "the index names trellis and trellis_pm")
    return PAIR_MAJOR if seen_major else PACK


def _cfg_int(config: Mapping, *names: str) -> Optional[int]:
    for scope in (config, config.get("text_config") or {}):
        for n in names:
            v = scope.get(n)
            if _is_int(v):
                return v
    return None


class Pack:
    """An EXL3/STQ pack directory: ``config.json``, ``model.safetensors.index.json`` (or one ``model.safetensors``)
    and its shards.  Opening parses the config's quant blocks, reads every shard header, and checks the index, the
    tile order and every shard's stamps before any tensor is read (`loadSourceIndex`, pack_index.zig:181-257;
    model.zig:1186)."""

    def __init__(self, path: str):
        self.path = path
        cfg_path = os.path.join(path, "config.json")
        self.config: Dict = {}
        if os.path.exists(cfg_path):
            with open(cfg_path, "rb") as f:
                self.config = json.loads(f.read().decode("utf-8"))
        self.spec: Optional[Spec] = parse_expert_quant(self.config) if "expert_quant" in self.config else None
        self.trunk_spec: Optional[Spec] = (parse_quant_block(self.config["trunk_quant"])
                                           if "trunk_quant" in self.config else None)
        self.weight_map: Dict[str, str] = self._weight_map()
        self.shards: Dict[str, Shard] = {}
        self.tensors: Dict[str, TensorMeta] = {}
        for fname in sorted(set(self.weight_map.values())):
            shard = Shard(os.path.join(path, fname))
            self.shards[fname] = shard
        for key, fname in self.weight_map.items():
            t = self.shards[fname].tensors.get(key)
            if t is None:
                raise _refuse("MissingIndexedSafetensorsTensor", f"{key} is not in {fname}")
            if key.startswith(PAD_PREFIX):
                continue
            self.tensors[key] = t
        self.tile_order = tile_order_of_keys(self.tensors)
        if self.spec is not None:
            if self.tile_order != self.spec.tile_order:
                raise _refuse("Exl3TileOrderMismatch",
                              f"the index names {self.tile_order}, expert_quant names {self.spec.tile_order}")
            for fname, shard in self.shards.items():
                shard_stamp_agrees(self.spec, *shard.stamp())
                if any(SWITCH in k and k.endswith((".trellis", ".trellis_pm")) for k in shard.tensors):
                    shard_tile_order_agrees(self.spec.tile_order, shard.metadata.get("tile_order"))

    def _weight_map(self) -> Dict[str, str]:
        index = os.path.join(self.path, INDEX_FILE)
        if os.path.exists(index):
            with open(index, "rb") as f:
                raw = f.read()
            try:
                doc = json.loads(raw.decode("utf-8"), object_pairs_hook=_no_duplicates("AmbiguousSafetensorsIndex"))
            except (UnicodeDecodeError, json.JSONDecodeError) as e:
                raise _refuse("InvalidSafetensorsIndex", str(e)) from None
            wm = doc.get("weight_map") if isinstance(doc, dict) else None
            if not isinstance(wm, dict) or not wm:
                raise _refuse("InvalidSafetensorsIndex", "no weight_map")
            for k, v in wm.items():
                if not isinstance(v, str) or not v or os.path.basename(v) != v:
                    raise _refuse("InvalidSafetensorsIndex", f"{k} -> {v!r}")
            return dict(wm)
        single = os.path.join(self.path, SINGLE_FILE)
        if os.path.exists(single):
            return {k: SINGLE_FILE for k in Shard(single).tensors}
        raise _refuse("InvalidSafetensorsIndex", f"{self.path} has neither {INDEX_FILE} nor {SINGLE_FILE}")

    # -- host side ---------------------------------------------------------------------------------------------

    def read(self, key: str) -> np.ndarray:
        t = self.tensors.get(key)
        if t is None:
            raise _refuse("MissingWeight", key)
        return self.shards[t.file].read(key)

    def layer_prefix(self, layer) -> str:
        """``<prefix>{L}`` of a routed layer: an int takes the arch nesting the pack uses; a string is the prefix."""
        if isinstance(layer, str):
            return layer
        for p in EXL3_PREFIXES:
            start = f"{p}{layer}{SWITCH}"
            if any(k.startswith(start) for k in self.tensors):
                return f"{p}{layer}"
        raise _refuse("MissingWeight", f"no routed tensors for layer {layer}")

    def moe_layout(self, layer, router_experts: Optional[int] = None, topk: Optional[int] = None,
                   hidden: Optional[int] = None, intermediate: Optional[int] = None) -> Tuple[Layout, List[str]]:
        """Validates one routed layer (`validateExl3Layer`, pack_index.zig:317-338) and returns its layout and keys.

        Geometry comes from the config (``hidden_size``, ``moe_intermediate_size``) unless given; the router width
        from ``<layer>.mlp.gate.weight`` when the pack holds it, else the config's expert count, else the layer's own
        total; top-k from ``num_experts_per_tok``."""
        if self.spec is None:
            raise _refuse("ExpertLayoutUnsupported", "config has no expert_quant")
        lp = self.layer_prefix(layer)
        hidden = hidden or _cfg_int(self.config, "hidden_size")
        intermediate = intermediate or _cfg_int(self.config, "moe_intermediate_size", "intermediate_size")
        if not hidden or not intermediate:
            raise _refuse("Exl3GroupGeometry", "no hidden_size / moe_intermediate_size")
        plan = Layout(hidden, intermediate, self.spec.rate, self.spec.rates)
        start = lp + SWITCH
        keys = sorted(k for k in self.tensors if k.startswith(start))
        for k in keys:
            t = self.tensors[k]
            plan.add(k[len(start):], t.shape, t.dtype)
        if router_experts is None:
            router = self.tensors.get(f"{lp}.mlp.gate.weight")
            if router is not None:
                if len(router.shape) != 2:
                    raise _refuse("Exl3RouterWidthMismatch", f"router {router.shape}")
                router_experts = router.shape[0]
            else:
                router_experts = _cfg_int(self.config, "n_routed_experts", "num_experts", "num_local_experts")
        if router_experts is None:
            router_experts = sum(g.experts for g in plan.groups[:plan.count])
        if topk is None:
            topk = _cfg_int(self.config, "num_experts_per_tok") or 1
        plan.finish(router_experts, topk)
        if plan.tile_order == PAIR_MAJOR and not plan.grouped:
            raise _refuse("Exl3TileOrderNeedsGroups", lp)
        return plan, keys

    def moe_layer_host(self, layer, **kw) -> Tuple[Layout, List[Dict[str, np.ndarray]]]:
        """The layer's tensors as stored (memory-mapped), one dict per group: ``{P}.{trellis|suh|svh}``."""
        plan, keys = self.moe_layout(layer, **kw)
        lp = self.layer_prefix(layer)
        start = lp + SWITCH
        groups: List[Dict[str, np.ndarray]] = [dict() for _ in range(plan.count)]
        for k in keys:
            name = Name.parse(k[len(start):])
            groups[name.group][f"{PROJECTIONS[name.projection]}.{PARTS[name.part]}"] = self.read(k)
        return plan, groups

    # -- device side -------------------------------------------------------------------------------------------

    def moe_layer(self, layer, device="cuda", **kw):
        """One routed layer on ``device``: an ``exl3.Bank`` (one ungrouped bank) or an ``exl3.Ragged`` (rate groups).

        Trellis tiles land on the device as stored; a pair-major trellis is put back into the pack order
        ``[E, IT, OT, n]`` by the library's tile-major kernel (`layout.tileMajorInverse`, layout.zig:150-158)."""
        plan, groups = self.moe_layer_host(layer, **kw)
        banks = []
        for gi, g in enumerate(groups):
            projs = []
            for pi, p in enumerate(PROJECTIONS):
                inp, out = (plan.intermediate, plan.hidden) if pi == 2 else (plan.hidden, plan.intermediate)
                tr = _to_device(g[f"{p}.trellis"].view(np.int16), device)
                e = tr.shape[0]
                if plan.tile_order == PAIR_MAJOR:
                    tr = exl3.tile_major(tr.reshape(e, inp // 16, out // 16, -1), inverse=True)
                suh = _to_device(g[f"{p}.suh"], device)
                svh = _to_device(g[f"{p}.svh"], device)
                projs.append(exl3.Proj(tr, suh, svh))
            banks.append(exl3.Bank(*projs))
        if not plan.grouped:
            return banks[0]
        return exl3.Ragged.init(banks)

    def linear(self, base: str, device="cuda") -> Tuple[exl3.Proj, exl3.Decode]:
        """A trunk projection stored as a trellis bank (`trunk_stq.load`, trunk_stq.zig:31-71): ``<base>.trellis`` U16
        ``[in/16, out/16, n]`` (or the grouped bank form ``[G, in/16, out/16, n]``), ``<base>.suh`` F16 ``[in]``,
        ``<base>.svh`` F16 ``[out]``; returns the projection and the ``trunk_quant`` decode."""
        tk, uk, vk = f"{base}.trellis", f"{base}.suh", f"{base}.svh"
        tr = self.tensors.get(tk)
        if tr is None:
            raise _refuse("MissingWeight", tk)
        if self.trunk_spec is None:
            raise _refuse("TrunkQuantMissing", f"{base} is a trellis bank and config.json has no trunk_quant")
        su, sv = self.tensors.get(uk), self.tensors.get(vk)
        if su is None or sv is None:
            raise _refuse("MissingWeight", uk if su is None else vk)
        shape = tr.shape
        groups = 1 if len(shape) == 3 else (shape[0] if len(shape) == 4 else 0)
        grid = shape[-3:] if groups else (0, 0, 0)
        inp, out = grid[0] * 16, grid[1] * 16
        rate = exl3.k_from_packed_dim(int(grid[2])) if groups else None
        ok = (groups > 0 and tr.dtype == "U16" and su.dtype == "F16" and sv.dtype == "F16" and rate is not None
              and inp > 0 and out > 0 and inp % 128 == 0 and out % 128 == 0
              and int(np.prod(su.shape)) == groups * inp and int(np.prod(sv.shape)) == groups * out)
        if not ok:
            raise _refuse("TrunkStqLayout", f"{base} is not a trellis bank (U16 [in/16, out/16, n], F16 scales "
                                            f"[in] and [out], both on the 128 grid)")
        if rate.n > self.trunk_spec.rate.n:
            raise _refuse("Exl3TrellisGeometry", f"{base}: n={rate.n} above trunk_quant's n={self.trunk_spec.rate.n}")
        if not self.trunk_spec.admits(rate.n):
            raise Exl3CodebookTableRateMissing(f"Exl3CodebookTableRateMissing: {base} n={rate.n}")
        t = _to_device(self.read(tk).view(np.int16).reshape(groups, *grid), device)
        s = _to_device(self.read(uk).reshape(groups, inp), device)
        v = _to_device(self.read(vk).reshape(groups, out), device)
        return exl3.Proj(t, s, v), self.trunk_spec.decode()


def _to_device(arr: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr)).to(device)


def open_pack(path: str) -> Pack:
    return Pack(path)
