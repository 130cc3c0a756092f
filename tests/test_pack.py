"""Pack loader: ``expert_quant`` parse, shard stamps, routed-layer layouts, safetensors packs on disk, device banks.

The CPU cases restate the reference's own tests of the same functions (src/exl3/root.zig:294-577,
src/exl3/layout.zig:160-230, src/exl3/codebook_tables.zig:281-430, src/pack_index.zig:452-467) with this build's
names; the GPU cases load synthetic packs written to the documented format (docs/pack-format.md:15-240) and check
the device banks and the MoE / linear outputs against banks built directly from the same arrays.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from sushi_amd import pack as P
from sushi_amd.exl3 import Codebook, Rate, Table, Window

SPEC1_TABLE = {"codebook_table": "spec1-w15", "codebook_digest": "37f72431"}
PAIR1_TABLE = {"codebook_table": "pair1-w16-v1", "codebook_digest": "c089b4eb"}
STD1_TABLE = {"codebook_table": "std1", "codebook_digest": "c5dba171"}


def spec_of(**block):
    return P.parse_expert_quant({"expert_quant": block})


def spec_of_text(text: str):
    return P.parse_expert_quant(json.loads(text))


# ---- expert_quant (root.zig:294-487) ------------------------------------------------------------------------------


def test_window_is_16_unless_the_config_names_one_this_build_decodes():  # root.zig:294-308
    base = dict(format="exl3", k=2.5, codebook="mcg")
    assert spec_of(**base).window == Window(16)
    for w in (16, 12, 11, 10, 8):
        assert spec_of(**base, window=w).window == Window(w)
    for bad in (17, 7, "12", None, 12.0):
        with pytest.raises(P.Exl3WindowUnsupported):
            spec_of(**base, window=bad)


def test_tile_order_names_pair_major_and_refuses_anything_else():  # root.zig:310-320
    base = dict(format="exl3", k=2.5, codebook="mcg")
    assert spec_of(**base).tile_order == P.PACK
    assert spec_of(**base, tile_order="pair_major").tile_order == P.PAIR_MAJOR
    for bad in ("pack", "Pair_Major", "", 1, None, True):
        with pytest.raises(P.Exl3TileOrderUnsupported):
            spec_of(**base, tile_order=bad)


def test_a_codebook_this_build_does_not_decode_is_refused():  # root.zig:322-327
    with pytest.raises(P.ExpertLayoutUnsupported):
        spec_of(format="exl3", k=2.5, codebook="mul2", window=12)


def test_an_stq_pack_names_its_table_and_every_rate_the_table_has_a_row_for():  # root.zig:333-346
    spec1 = spec_of(format="stq", k=2.5, codebook="spec1", window=15, **SPEC1_TABLE)
    assert spec1.codebook == Codebook.spec1 and spec1.rate.n == 40 and spec1.table == Table.spec1_w15
    pair1 = spec_of(format="stq", k=3, codebook="pair1", window=16, **PAIR1_TABLE)
    assert pair1.codebook == Codebook.pair1 and pair1.table == Table.pair1_w16_v1
    assert all(pair1.admits(n) for n in (24, 32, 36, 48, 64))
    assert not any(pair1.admits(n) for n in (16, 22, 66, 128))
    assert all(spec1.admits(n) for n in (16, 22, 66, 128))
    assert not spec1.admits(14) and not spec1.admits(130)
    assert spec_of(format="exl3", k=3, codebook="mcg").admits(36)


def test_spec1_decodes_at_every_window_pair1_only_at_its_own():  # root.zig:348-366
    for w in range(8, 17):
        s = spec_of(format="stq", k=2.5, codebook="spec1", window=w, **SPEC1_TABLE)
        assert s.window == Window(w) and s.table == Table.spec1_w15
    assert spec_of(format="stq", k=2, codebook="spec1", **SPEC1_TABLE).window == Window(16)
    for w in (7, 17):
        with pytest.raises(P.Exl3WindowUnsupported):
            spec_of(format="stq", k=2, codebook="spec1", window=w, **SPEC1_TABLE)
    with pytest.raises(P.Exl3CodebookTableWindowMismatch):
        spec_of(format="stq", k=2, codebook="pair1", window=15, **PAIR1_TABLE)
    assert spec_of(format="exl3", k=3, codebook="mcg").table is None
    # The reference's test-only table is not one this build holds.
    with pytest.raises(P.Exl3CodebookTableUnknown):
        spec_of(format="stq", k=3, codebook="spec1", window=8, codebook_table="spec1-test-per-rate",
                codebook_digest="a2f2fe40")


def test_std1_names_the_std1_table_at_every_window():  # root.zig:368-378
    for w in range(8, 17):
        s = spec_of(format="stq", k=2.5, codebook="std1", window=w, **STD1_TABLE)
        assert s.codebook == Codebook.std1 and s.window == Window(w) and s.table == Table.std1


@pytest.mark.parametrize("block,want", [  # root.zig:380-397
    (dict(k=2, codebook="spec1", window=15), "Exl3CodebookTableUnknown"),
    (dict(k=2, codebook="spec1", window=15, codebook_table="spec1-w15-v2", codebook_digest="c5dba171"),
     "Exl3CodebookTableUnknown"),
    (dict(k=2, codebook="spec1", window=15, codebook_table="spec1-w15", codebook_digest="00000000"),
     "Exl3CodebookTableDigestMismatch"),
    (dict(k=2, codebook="spec1", window=15, **STD1_TABLE), "Exl3CodebookTableCodebookMismatch"),
    (dict(k=2, codebook="spec1", window=15, **PAIR1_TABLE), "Exl3CodebookTableCodebookMismatch"),
    (dict(k=2, codebook="pair1", window=15, **PAIR1_TABLE), "Exl3CodebookTableWindowMismatch"),
    (dict(k=2, codebook="spec1", window=15, codebook_table="spec1-w15", codebook_digest="2ac2594d"),
     "Exl3CodebookTableLegacyConfig"),
    (dict(k=1, codebook="pair1", **PAIR1_TABLE), "Exl3CodebookTableRateMissing"),
    (dict(k=4.5, codebook="std1", window=15, **STD1_TABLE), "Exl3CodebookTableRateMissing"),
    (dict(k=2, codebook="mcg", format="exl3", **SPEC1_TABLE), "Exl3CodebookTableCodebookMismatch"),
    (dict(k=2, codebook="pair1", window=16, codebook_table="pair1-w16-v1"), "Exl3CodebookTableDigestMismatch"),
])
def test_an_stq_pack_with_a_missing_foreign_or_legacy_table_is_refused_by_name(block, want):
    block = dict(block)
    block.setdefault("format", "stq")
    with pytest.raises(getattr(P, want)):
        spec_of(**block)


def test_stq_is_for_the_tabled_codebooks_and_exl3_for_the_rest():  # root.zig:399-404
    for block in (dict(format="stq", k=2.5, codebook="mcg"),
                  dict(format="exl3", k=2.5, codebook="std1", window=15, **STD1_TABLE),
                  dict(format="exq", k=2.5, codebook="mcg")):
        with pytest.raises(P.ExpertLayoutUnsupported):
            spec_of(**block)


@pytest.mark.parametrize("text,n", [("2", 32), ("2.5", 40), ("2.75", 44), ("3", 48), ("3.5", 56), ("4", 64)])
@pytest.mark.parametrize("cb", ["mul1", "mcg", "spec1", "std1", "pair1", "3inst"])
def test_k_admits_integer_and_fractional_rates_under_every_served_codebook(text, n, cb):  # root.zig:443-470
    keys = {"spec1": ',"window":15,"codebook_table":"spec1-w15","codebook_digest":"37f72431"',
            "std1": ',"window":15,"codebook_table":"std1","codebook_digest":"c5dba171"',
            "pair1": ',"codebook_table":"pair1-w16-v1","codebook_digest":"c089b4eb"'}.get(cb, "")
    fmt = "stq" if cb in ("spec1", "std1", "pair1") else "exl3"
    s = spec_of_text(f'{{"expert_quant":{{"format":"{fmt}","k":{text},"codebook":"{cb}"{keys}}}}}')
    assert s.rate.n == n and s.codebook == Codebook.from_name(cb)


@pytest.mark.parametrize("bad", ["2.3", "8.125", "9", "0.875", "2.0625", '"2"', "true", "null", "1e400"])
def test_k_off_the_sixteenth_grid_or_the_served_range_is_refused(bad):  # root.zig:471-486
    with pytest.raises(P.ExpertLayoutUnsupported):
        spec_of_text(f'{{"expert_quant":{{"format":"exl3","k":{bad},"codebook":"mul1"}}}}')


def test_a_config_without_expert_quant_is_refused():
    with pytest.raises(P.ExpertLayoutUnsupported):
        P.parse_expert_quant({})
    with pytest.raises(P.ExpertLayoutUnsupported):
        P.parse_expert_quant({"expert_quant": [1]})


def test_config_k_and_packed_shapes_admit_k1_through_k8():  # root.zig:522-538
    for n in range(145):
        admitted = 16 <= n <= 128 and n % 2 == 0
        assert (P.rate_from_config_k(n / 16) is not None) == admitted, n
        plan = P.Layout(128, 256, Rate(128))
        if admitted:
            assert plan.add("gate_proj.trellis", (2, 8, 16, n), "U16").group == 0
            for cb in ("mul1", "mcg"):
                assert spec_of(format="exl3", k=n / 16, codebook=cb).rate.n == n
            if n > 16:
                with pytest.raises(P.Exl3TrellisGeometry):
                    P.Layout(128, 256, Rate(n - 2)).add("gate_proj.trellis", (2, 8, 16, n), "U16")
        else:
            with pytest.raises(P.Exl3TrellisGeometry):
                plan.add("gate_proj.trellis", (2, 8, 16, n), "U16")
    for k in range(1, 9):
        assert P.rate_from_config_k(k).n == 16 * k


def test_shipped_tables_are_the_library_rows_and_their_pinned_digests():
    """The loader's table registry against the HIP library's own rows (parsed from its source) and digests."""
    from tests.test_oracle_format import TABLE_DIGESTS, _digest, _header_tables

    rows = _header_tables()
    for name, t in P.SHIPPED_TABLES.items():
        n_lo, table_rows = rows[int(t.table)]
        ns = [n_lo + 2 * i for i in range(len(table_rows))]
        assert t.rates() == frozenset(ns), name
        assert t.digest == TABLE_DIGESTS[int(t.table)] == _digest(4 if t.codebook == Codebook.pair1 else 2, ns,
                                                                    table_rows)


# ---- shard stamps (pack_index.zig:452-467; dsv41/repack_test.zig:513-515) -----------------------------------------


def test_shard_k_stamp_refuses_invalid_nonfinite_and_wider_rates():
    spec = P.Spec(Rate(64), Codebook.mcg)
    for k in ("0", "0.5", "2.0625", "4.5", "nan", "inf", "-inf", "", "2 ", "k4"):
        with pytest.raises(P.Exl3ShardStampMismatch):
            P.shard_stamp_agrees(spec, k, None, None)
    for k in ("1", "1.5", "2", "2.125", "2.5", "3", "4"):
        P.shard_stamp_agrees(spec, k, None, None)


def test_shard_codebook_and_window_stamps_must_be_the_configs():
    spec = spec_of(format="stq", k=2, codebook="spec1", window=15, **SPEC1_TABLE)
    P.shard_stamp_agrees(spec, None, "spec1", "15")
    P.shard_stamp_agrees(spec, None, None, None)
    for cb, w in (("mcg", None), ("SPEC1", None), (None, "16"), (None, "x"), (None, "7")):
        with pytest.raises(P.Exl3ShardStampMismatch):
            P.shard_stamp_agrees(spec, None, cb, w)


def test_shard_tile_order_stamp():
    P.shard_tile_order_agrees(P.PACK, None)
    P.shard_tile_order_agrees(P.PAIR_MAJOR, "pair_major")
    for order, stamp in ((P.PACK, "pair_major"), (P.PAIR_MAJOR, None), (P.PACK, "pack"), (P.PAIR_MAJOR, "PM")):
        with pytest.raises(P.Exl3ShardStampMismatch):
            P.shard_tile_order_agrees(order, stamp)


# ---- names and layer layouts (layout.zig:14-137, :174-214; root.zig:406-423, :540-577) ------------------------


def test_a_pair_major_trellis_is_named_trellis_pm_and_its_5d_shape_is_the_same_grid():  # layout.zig:174-188
    name = P.Name.parse("gate_proj.g1.trellis_pm")
    assert name.pair_major and name.part == 0 and name.group == 1 and name.tile_order == P.PAIR_MAJOR
    assert not P.Name.parse("gate_proj.g1.trellis").pair_major
    for bad in ("gate_proj.g1.suh_pm", "gate_proj.trellis_pm.x", "gate.trellis", "gate_proj", "up_proj.g.suh",
                "up_proj.g1x.suh", "up_proj.g１.suh", "down_proj.g1.g2.suh"):
        with pytest.raises(P.Exl3GroupNameInvalid):
            P.Name.parse(bad)
    assert P.tile_dims(P.PAIR_MAJOR, (3, 4, 16, 2, 24)) == (16, 8, 24)
    assert P.tile_dims(P.PACK, (3, 16, 8, 24)) == (16, 8, 24)
    assert P.tile_dims(P.PAIR_MAJOR, (3, 16, 8, 24)) is None
    assert P.tile_dims(P.PAIR_MAJOR, (3, 4, 16, 3, 24)) is None
    assert P.tile_dims(P.PACK, (3, 4, 16, 2, 24)) is None


def test_a_layer_admits_a_pair_major_bank_and_refuses_a_wrong_grid_or_a_mixed_one():  # layout.zig:190-214
    ok = P.Layout(256, 128, Rate(64))
    ok.add("gate_proj.g0.trellis_pm", (3, 4, 16, 2, 32), "U16")
    ok.add("down_proj.g0.trellis_pm", (3, 8, 8, 2, 32), "U16")
    assert ok.tile_order == P.PAIR_MAJOR and ok.groups[0].rates[0] == 32 and ok.groups[0].rates[2] == 32
    for shape, err in (((3, 16, 8, 32), P.Exl3GroupGeometry), ((3, 4, 16, 4, 32), P.Exl3GroupGeometry),
                       ((3, 8, 16, 2, 32), P.Exl3GroupGeometry), ((3, 16, 4, 2, 32), P.Exl3GroupGeometry),
                       ((3, 4, 16, 2, 66), P.Exl3TrellisGeometry)):
        with pytest.raises(err):
            P.Layout(256, 128, Rate(64)).add("gate_proj.g0.trellis_pm", shape, "U16")
    with pytest.raises(P.Exl3GroupGeometry):
        P.Layout(256, 128, Rate(64)).add("gate_proj.g0.trellis", (3, 4, 16, 2, 32), "U16")
    mixed = P.Layout(256, 128, Rate(64))
    mixed.add("gate_proj.g0.trellis_pm", (3, 4, 16, 2, 32), "U16")
    with pytest.raises(P.Exl3TileOrderMixed):
        mixed.add("up_proj.g0.trellis", (3, 16, 8, 32), "U16")


def test_a_table_layer_whose_bank_rate_the_table_lacks_is_refused():  # root.zig:406-423
    rates = P.SHIPPED_TABLES["std1"].rates()
    plan = P.Layout(128, 128, Rate(48), rates)
    plan.add("gate_proj.trellis", (1, 8, 8, 32), "U16")
    plan.add("up_proj.trellis", (1, 8, 8, 48), "U16")
    with pytest.raises(P.Exl3CodebookTableRateMissing):
        plan.add("down_proj.trellis", (1, 8, 8, 16), "U16")
    grouped = P.Layout(128, 128, Rate(48), rates)
    grouped.add("gate_proj.g0.trellis", (1, 8, 8, 32), "U16")
    grouped.add("gate_proj.g1.trellis", (2, 8, 8, 48), "U16")
    with pytest.raises(P.Exl3CodebookTableRateMissing):
        grouped.add("up_proj.g1.trellis", (2, 8, 8, 16), "U16")


def _two_group_plan():
    plan = P.Layout(128, 128, Rate(64))
    for g, e in enumerate((2, 1)):
        for p, proj in enumerate(("gate", "up", "down")):
            n = 32 + 16 * ((g + p) % 3)
            plan.add(f"{proj}_proj.g{g}.trellis", (e, 8, 8, n), "U16")
            plan.add(f"{proj}_proj.g{g}.suh", (e, 128), "F16")
            plan.add(f"{proj}_proj.g{g}.svh", (e, 128), "F16")
    return plan


def test_layouts_validate_groups_route_slots_and_bill_stored_bytes():  # root.zig:540-562
    plan = _two_group_plan()
    plan.finish(3, 2)
    assert plan.count == 2 and plan.grouped
    assert plan.bytes == 3 * (8 * 8 * (32 + 48 + 64) * 2 + 3 * 256 * 2)
    assert plan.locate(2) == (1, 0) and plan.locate(1) == (0, 1) and plan.locate(0) == (0, 0)
    with pytest.raises(P.ExpertOutOfRange):
        plan.locate(3)
    with pytest.raises(P.Exl3RouterWidthMismatch):
        plan.finish(4, 2)
    with pytest.raises(P.Exl3TopKExceedsExperts):
        plan.finish(3, 4)


def test_top_k_above_the_reduce_bank_is_refused():  # root.zig:435-441
    plan = P.Layout(128, 128, Rate(64))
    for proj in ("gate", "up", "down"):
        plan.add(f"{proj}_proj.trellis", (40, 8, 8, 32), "U16")
        plan.add(f"{proj}_proj.suh", (40, 128), "F16")
        plan.add(f"{proj}_proj.svh", (40, 128), "F16")
    plan.finish(40, 32)
    with pytest.raises(P.Exl3TopKExceedsReduceBank):
        plan.finish(40, 33)


def test_layouts_refuse_malformed_missing_mixed_and_unsupported_groups():  # root.zig:564-577
    plan = P.Layout(128, 128, Rate(64))
    with pytest.raises(P.Exl3GroupNameInvalid):
        plan.add("gate_proj.g01.trellis", (1, 8, 8, 32), "U16")
    with pytest.raises(P.Exl3TrellisGeometry):
        plan.add("gate_proj.g0.trellis", (1, 8, 8, 33), "U16")
    with pytest.raises(P.Exl3GroupGeometry):
        plan.add("gate_proj.g0.trellis", (0, 8, 8, 32), "U16")
    with pytest.raises(P.Exl3GroupGeometry):
        plan.add("gate_proj.g0.suh", (1, 64), "F16")
    plan.add("gate_proj.g1.trellis", (1, 8, 8, 32), "U16")
    with pytest.raises(P.Exl3GroupMissing):
        plan.finish(1, 1)
    with pytest.raises(P.Exl3GroupGeometry):
        plan.add("up_proj.g1.trellis", (2, 8, 8, 32), "U16")
    with pytest.raises(P.Exl3MixedGroupLayout):
        plan.add("gate_proj.trellis", (1, 8, 8, 32), "U16")
    with pytest.raises(P.Exl3GroupDtype):
        plan.add("up_proj.g1.suh", (1, 128), "U16")
    with pytest.raises(P.Exl3GroupDtype):
        plan.add("up_proj.g1.suh", (1, 128), "BF16")
    with pytest.raises(P.Exl3GroupNameInvalid):
        plan.add("gate_proj.g32.trellis", (1, 8, 8, 32), "U16")
    with pytest.raises(P.Exl3GroupNameInvalid):
        plan.add("gate_proj.g1.trellis", (1, 8, 8, 32), "U16")  # the same tensor twice
    with pytest.raises(P.MissingWeight):
        P.Layout(128, 128, Rate(64)).finish(1, 1)


# ---- packs on disk --------------------------------------------------------------------------------------------

HIDDEN, INTER = 256, 128
LAYER = "model.layers.3"


def synth_group(seed: int, experts: int, rates):
    """Pack-order arrays of one rate group: {proj: (trellis u16 [E, in/16, out/16, n], suh f16, svh f16)}."""
    rng = np.random.default_rng(seed)
    out = {}
    for p, n in zip(P.PROJECTIONS, rates):
        inp, o = (INTER, HIDDEN) if p == "down_proj" else (HIDDEN, INTER)
        tr = rng.integers(0, 1 << 16, size=(experts, inp // 16, o // 16, n), dtype=np.uint16)
        suh = (rng.choice([-1.0, 1.0], size=(experts, inp)) * rng.uniform(0.5, 1.5, (experts, inp))).astype(np.float16)
        svh = (rng.choice([-1.0, 1.0], size=(experts, o)) * rng.uniform(0.5, 1.5, (experts, o))).astype(np.float16)
        out[p] = (tr, suh, svh)
    return out


def pair_major_of(tr: np.ndarray) -> np.ndarray:
    """[E, IT, OT, n] -> [E, OT/2, IT, 2, n] through the oracle's tile-major (layout.zig:139-148)."""
    from oracle import tile_major

    e, it, ot, n = tr.shape
    pm = np.stack([tile_major(tr[i].reshape(-1), it, ot, n) for i in range(e)])
    return pm.reshape(e, ot // 2, it, 2, n)


def write_pack(root, groups, *, grouped=True, order=P.PACK, expert_quant=None, stamp=None, tile_stamp="auto",
               router=True, single=False, extra=None, pad=True, config_extra=None):
    """A one-layer pack: the routed tensors in one shard (with a `__pad__.` tensor), the router in another."""
    os.makedirs(root, exist_ok=True)
    if expert_quant is None:
        expert_quant = dict(format="stq", k=4, codebook="spec1", window=15, **SPEC1_TABLE)
        if order == P.PAIR_MAJOR:
            expert_quant["tile_order"] = "pair_major"
    eq = dict(expert_quant)
    cfg = {"hidden_size": HIDDEN, "moe_intermediate_size": INTER, "num_experts_per_tok": 2, "expert_quant": eq}
    cfg.update(config_extra or {})
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump(cfg, f)
    tensors = {}
    for g, arrs in enumerate(groups):
        for p in P.PROJECTIONS:
            tr, suh, svh = arrs[p]
            stem = f"{LAYER}.mlp.switch_mlp.{p}" + (f".g{g}" if grouped else "")
            if order == P.PAIR_MAJOR:
                tensors[stem + ".trellis_pm"] = pair_major_of(tr)
            else:
                tensors[stem + ".trellis"] = tr
            tensors[stem + ".suh"] = suh
            tensors[stem + ".svh"] = svh
            if pad:
                tensors[f"__pad__.experts.{len(tensors)}"] = np.zeros(7, np.uint8)
    tensors.update(extra or {})
    meta = dict(stamp or {})
    if tile_stamp == "auto":
        if order == P.PAIR_MAJOR:
            meta["tile_order"] = "pair_major"
    elif tile_stamp is not None:
        meta["tile_order"] = tile_stamp
    experts = sum(next(iter(a.values()))[0].shape[0] for a in groups)
    other = {f"{LAYER}.mlp.gate.weight": np.zeros((experts, HIDDEN), np.float16)} if router else {}
    if single:
        P.write_shard(os.path.join(root, P.SINGLE_FILE), {**tensors, **other}, meta)
        return root
    P.write_shard(os.path.join(root, "experts.safetensors"), tensors, meta)
    wm = {k: "experts.safetensors" for k in tensors}
    if other:
        P.write_shard(os.path.join(root, "trunk.safetensors"), other)
        wm.update({k: "trunk.safetensors" for k in other})
    with open(os.path.join(root, P.INDEX_FILE), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    return root


GROUP_RATES = [((32, 48, 16), 3), ((64, 32, 24), 2), ((16, 16, 40), 1)]


def three_groups(seed=0):
    return [synth_group(seed + g, e, r) for g, (r, e) in enumerate(GROUP_RATES)]


@pytest.mark.parametrize("order", [P.PACK, P.PAIR_MAJOR])
def test_a_grouped_pack_reads_back_each_group_in_the_pack_order(tmp_path, order):
    from oracle import tile_major_inverse

    groups = three_groups()
    pk = P.Pack(write_pack(str(tmp_path), groups, order=order))
    assert pk.tile_order == order and pk.spec.tile_order == order
    assert not any(k.startswith(P.PAD_PREFIX) for k in pk.tensors)
    plan, host = pk.moe_layout(3)[0], pk.moe_layer_host(3)[1]
    assert plan.grouped and plan.count == 3 and [g.experts for g in plan.groups[:3]] == [3, 2, 1]
    assert [tuple(g.rates) for g in plan.groups[:3]] == [r for r, _ in GROUP_RATES]
    assert plan.locate(4) == (1, 1) and plan.locate(5) == (2, 0)
    for g, arrs in enumerate(groups):
        for p in P.PROJECTIONS:
            tr, suh, svh = arrs[p]
            got = host[g][f"{p}.trellis"]
            if order == P.PAIR_MAJOR:
                e, it, ot, n = tr.shape
                assert got.shape == (e, ot // 2, it, 2, n)
                got = np.stack([tile_major_inverse(got[i].reshape(-1), it, ot, n) for i in range(e)]).reshape(tr.shape)
            np.testing.assert_array_equal(got, tr)
            np.testing.assert_array_equal(host[g][f"{p}.suh"], suh)
            np.testing.assert_array_equal(host[g][f"{p}.svh"], svh)


def test_an_ungrouped_single_file_pack_is_one_bank(tmp_path):
    groups = [synth_group(7, 4, (32, 32, 32))]
    pk = P.Pack(write_pack(str(tmp_path), groups, grouped=False, single=True,
                           expert_quant=dict(format="exl3", k=2, codebook="mcg")))
    plan, host = pk.moe_layer_host(3)
    assert not plan.grouped and plan.count == 1 and plan.groups[0].experts == 4
    np.testing.assert_array_equal(host[0]["down_proj.trellis"], groups[0]["down_proj"][0])
    assert pk.spec.decode().codebook == Codebook.mcg and pk.spec.decode().table is None


def test_pack_level_refusals(tmp_path):
    groups = three_groups(3)
    d = lambda name: str(tmp_path / name)  # noqa: E731
    # config names pair_major, the index names the pack order (and the reverse)
    cfg_pm = dict(format="stq", k=4, codebook="spec1", window=15, tile_order="pair_major", **SPEC1_TABLE)
    with pytest.raises(P.Exl3TileOrderMismatch):
        P.Pack(write_pack(d("a"), groups, expert_quant=cfg_pm, tile_stamp=None))
    with pytest.raises(P.Exl3TileOrderMismatch):
        P.Pack(write_pack(d("b"), groups, order=P.PAIR_MAJOR,
                          expert_quant=dict(format="stq", k=4, codebook="spec1", window=15, **SPEC1_TABLE)))
    # a pair-major shard without its stamp; a pack-order shard that stamps one
    with pytest.raises(P.Exl3ShardStampMismatch):
        P.Pack(write_pack(d("c"), groups, order=P.PAIR_MAJOR, tile_stamp=None))
    with pytest.raises(P.Exl3ShardStampMismatch):
        P.Pack(write_pack(d("c2"), groups, tile_stamp="pair_major"))
    # decoder stamps
    with pytest.raises(P.Exl3ShardStampMismatch):
        P.Pack(write_pack(d("e"), groups, stamp={"k": "4.5"}))
    with pytest.raises(P.Exl3ShardStampMismatch):
        P.Pack(write_pack(d("f"), groups, stamp={"codebook": "mcg"}))
    P.Pack(write_pack(d("g"), groups, stamp={"k": "2", "codebook": "spec1", "window": "15"}))
    # both orders in one index
    tr = groups[0]["gate_proj"][0]
    with pytest.raises(P.Exl3TileOrderMixed):
        P.Pack(write_pack(d("h"), groups, extra={f"{LAYER}.mlp.switch_mlp.gate_proj.g9.trellis_pm":
                                                 pair_major_of(tr)}))
    # a pair-major layer must be rate-grouped
    pk = P.Pack(write_pack(d("i"), groups[:1], grouped=False, order=P.PAIR_MAJOR))
    with pytest.raises(P.Exl3TileOrderNeedsGroups):
        pk.moe_layout(3)
    # the router's width is the layer's expert total
    pk = P.Pack(write_pack(d("j"), groups))
    with pytest.raises(P.Exl3RouterWidthMismatch):
        pk.moe_layout(3, router_experts=7)
    with pytest.raises(P.Exl3TopKExceedsExperts):
        pk.moe_layout(3, topk=7)
    # a layer missing one group's tensor
    pk = P.Pack(write_pack(d("k"), groups, extra={f"{LAYER}.mlp.switch_mlp.up_proj.g3.suh":
                                                   np.zeros((1, HIDDEN), np.float16)}))
    with pytest.raises(P.Exl3GroupMissing):
        pk.moe_layout(3)
    # a routed bank above the config's rate
    pk = P.Pack(write_pack(d("l"), groups, expert_quant=dict(format="stq", k=2, codebook="spec1", window=15,
                                                             **SPEC1_TABLE)))
    with pytest.raises(P.Exl3TrellisGeometry):
        pk.moe_layout(3)
    with pytest.raises(P.MissingWeight):
        pk.moe_layout(4)


def _rewrite_header(path, edit):
    raw = open(path, "rb").read()
    hlen = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + hlen])
    edit(header)
    text = json.dumps(header).encode()
    text += b" " * ((-(8 + len(text))) % 8)
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little") + text + raw[8 + hlen:])


def test_safetensors_header_and_index_refusals(tmp_path):
    groups = [synth_group(11, 2, (32, 32, 32))]
    key = f"{LAYER}.mlp.switch_mlp.gate_proj.suh"

    def fresh(name):
        return write_pack(str(tmp_path / name), groups, grouped=False,
                          expert_quant=dict(format="exl3", k=2, codebook="mcg"))

    root = fresh("a")
    _rewrite_header(os.path.join(root, "experts.safetensors"),
                    lambda h: h[key].update(shape=[2, HIDDEN + 16]))
    with pytest.raises(P.SafetensorsPayloadMismatch):
        P.Pack(root)
    root = fresh("b")
    _rewrite_header(os.path.join(root, "experts.safetensors"),
                    lambda h: h[key].update(data_offsets=[0, 10 ** 9]))
    with pytest.raises(P.InvalidSafetensorsHeader):
        P.Pack(root)
    root = fresh("c")
    _rewrite_header(os.path.join(root, "experts.safetensors"), lambda h: h[key].update(shape=[2, -HIDDEN]))
    with pytest.raises(P.InvalidSafetensorsHeader):
        P.Pack(root)
    root = fresh("d")
    _rewrite_header(os.path.join(root, "experts.safetensors"), lambda h: h.pop(key))
    with pytest.raises(P.MissingIndexedSafetensorsTensor):
        P.Pack(root)
    root = fresh("e")
    with open(os.path.join(root, "experts.safetensors"), "r+b") as f:
        f.write((1 << 40).to_bytes(8, "little"))
    with pytest.raises(P.SafetensorsHeaderTooLarge):
        P.Pack(root)
    root = fresh("f")
    idx = os.path.join(root, P.INDEX_FILE)
    text = open(idx).read().replace('"weight_map": {', '"weight_map": {"' + key + '": "trunk.safetensors", ', 1)
    open(idx, "w").write(text)
    with pytest.raises(P.AmbiguousSafetensorsIndex):
        P.Pack(root)
    root = fresh("g")
    open(os.path.join(root, P.INDEX_FILE), "w").write('{"weight_map": {}}')
    with pytest.raises(P.InvalidSafetensorsIndex):
        P.Pack(root)
    root = fresh("h")
    wm = json.load(open(os.path.join(root, P.INDEX_FILE)))
    wm["weight_map"][key] = "missing.safetensors"
    json.dump(wm, open(os.path.join(root, P.INDEX_FILE), "w"))
    with pytest.raises(P.MissingPackShard):
        P.Pack(root)
    root = fresh("i")
    tkey = f"{LAYER}.mlp.switch_mlp.gate_proj.trellis"

    def overlap(h):
        s0 = h[tkey]["data_offsets"][0]
        h[key]["data_offsets"] = [s0, s0 + h[key]["data_offsets"][1] - h[key]["data_offsets"][0]]

    _rewrite_header(os.path.join(root, "experts.safetensors"), overlap)
    with pytest.raises(P.InvalidSafetensorsHeader):
        P.Pack(root)


def test_trunk_linear_refusals(tmp_path):
    rng = np.random.default_rng(5)
    base = "model.layers.0.self_attn.o_proj"
    good = {base + ".trellis": rng.integers(0, 1 << 16, (16, 8, 48), dtype=np.uint16),
            base + ".suh": np.ones(256, np.float16), base + ".svh": np.ones(128, np.float16)}
    root = str(tmp_path / "a")
    os.makedirs(root)
    P.write_shard(os.path.join(root, P.SINGLE_FILE), good)
    json.dump({"hidden_size": 256}, open(os.path.join(root, "config.json"), "w"))
    with pytest.raises(P.TrunkQuantMissing):
        P.Pack(root).linear(base, device="cpu")
    json.dump({"trunk_quant": dict(format="stq", k=4, codebook="std1", window=15, **STD1_TABLE)},
              open(os.path.join(root, "config.json"), "w"))
    proj, dec = P.Pack(root).linear(base, device="cpu")
    assert tuple(proj.trellis.shape) == (1, 16, 8, 48) and proj.in_features == 256 and proj.out_features == 128
    assert dec.codebook == Codebook.std1 and dec.table == int(Table.std1)
    for edit, err in (({base + ".suh": np.ones(128, np.float16)}, P.TrunkStqLayout),
                      ({base + ".svh": np.ones(128, np.float32)}, P.TrunkStqLayout),
                      ({base + ".trellis": rng.integers(0, 1 << 16, (12, 8, 48), dtype=np.uint16)}, P.TrunkStqLayout),
                      ({base + ".trellis": rng.integers(0, 1 << 16, (16, 8, 16), dtype=np.uint16)},
                       P.Exl3CodebookTableRateMissing)):
        r = str(tmp_path / f"t{len(os.listdir(tmp_path))}")
        os.makedirs(r)
        P.write_shard(os.path.join(r, P.SINGLE_FILE), {**good, **edit})
        json.dump({"trunk_quant": dict(format="stq", k=4, codebook="std1", window=15, **STD1_TABLE)},
                  open(os.path.join(r, "config.json"), "w"))
        with pytest.raises(err):
            P.Pack(r).linear(base, device="cpu")


# ---- device banks (GPU) ---------------------------------------------------------------------------------------


def _bank_of(arrs, dev):
    import torch

    from sushi_amd import exl3

    projs = []
    for p in P.PROJECTIONS:
        tr, suh, svh = arrs[p]
        projs.append(exl3.Proj(torch.from_numpy(tr.view(np.int16)).to(dev), torch.from_numpy(suh).to(dev),
                               torch.from_numpy(svh).to(dev)))
    return exl3.Bank(*projs)


@pytest.mark.gpu
@pytest.mark.parametrize("order", [P.PACK, P.PAIR_MAJOR])
def test_a_grouped_pack_on_the_device_is_the_written_ragged_bank(tmp_path, dev, order):
    import torch

    from sushi_amd import exl3

    groups = three_groups(21)
    pk = P.Pack(write_pack(str(tmp_path), groups, order=order))
    rb = pk.moe_layer(3, device=dev)
    want = exl3.Ragged.init([_bank_of(g, dev) for g in groups])
    for i in range(3):
        assert torch.equal(rb.trellis[i], want.trellis[i]), f"projection {i} trellis"
        assert torch.equal(rb.suh[i], want.suh[i]) and torch.equal(rb.svh[i], want.svh[i])
    assert torch.equal(rb.meta, want.meta)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, HIDDEN, generator=g).to(torch.float16).to(dev)
    inds = torch.stack([torch.randperm(6, generator=g)[:2] for _ in range(5)]).to(torch.int32).to(dev)
    scores = torch.softmax(torch.randn(5, 2, generator=g), -1).to(dev)
    dec = pk.spec.decode()
    y = exl3.moe_ragged(x, rb, inds, scores, dec)
    y_want = exl3.moe_ragged(x, want, inds, scores, dec)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.equal(y, y_want)


@pytest.mark.gpu
def test_an_ungrouped_pack_on_the_device_is_the_written_bank(tmp_path, dev):
    import torch

    from sushi_amd import exl3

    groups = [synth_group(31, 6, (32, 32, 32))]
    pk = P.Pack(write_pack(str(tmp_path), groups, grouped=False, expert_quant=dict(format="exl3", k=2,
                                                                                   codebook="mcg")))
    bank = pk.moe_layer(3, device=dev)
    want = _bank_of(groups[0], dev)
    for p in ("gate", "up", "down"):
        assert torch.equal(getattr(bank, p).trellis, getattr(want, p).trellis)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(3, HIDDEN, generator=g).to(torch.float16).to(dev)
    inds = torch.stack([torch.randperm(6, generator=g)[:2] for _ in range(3)]).to(torch.int32).to(dev)
    scores = torch.softmax(torch.randn(3, 2, generator=g), -1).to(dev)
    y = exl3.moe(x, bank, inds, scores, pk.spec.decode())
    torch.cuda.synchronize()
    assert torch.equal(y, exl3.moe(x, want, inds, scores, pk.spec.decode()))


@pytest.mark.gpu
def test_a_trunk_linear_from_a_pack_is_the_written_projection(tmp_path, dev):
    import torch

    from sushi_amd import exl3

    rng = np.random.default_rng(9)
    base = "model.layers.0.mlp.down_proj"
    tr = rng.integers(0, 1 << 16, (16, 8, 48), dtype=np.uint16)
    suh, svh = (rng.uniform(0.5, 1.5, 256).astype(np.float16), rng.uniform(0.5, 1.5, 128).astype(np.float16))
    root = str(tmp_path)
    P.write_shard(os.path.join(root, P.SINGLE_FILE), {base + ".trellis": tr, base + ".suh": suh, base + ".svh": svh})
    json.dump({"trunk_quant": dict(format="stq", k=3, codebook="spec1", window=15, **SPEC1_TABLE)},
              open(os.path.join(root, "config.json"), "w"))
    proj, dec = P.Pack(root).linear(base, device=dev)
    want = exl3.Proj(torch.from_numpy(tr.view(np.int16)).reshape(1, 16, 8, 48).to(dev),
                     torch.from_numpy(suh).reshape(1, 256).to(dev), torch.from_numpy(svh).reshape(1, 128).to(dev))
    x = torch.randn(4, 256, generator=torch.Generator().manual_seed(3)).to(torch.float16).to(dev)
    y = exl3.linear(x, proj, dec)
    torch.cuda.synchronize()
    assert torch.equal(y, exl3.linear(x, want, dec))
