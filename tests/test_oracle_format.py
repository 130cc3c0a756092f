"""Pins the CPU oracle's format layer (decoders, bitstream, tile order, tables) against the reference's own known
answers and golden fixtures, plus independent restatements where the reference holds none.

Every check here is chosen so a plausible mistake (a wrong shift, a transposed position, a bad table row) fails it.
"""
import hashlib
import os
import re

import numpy as np
import pytest

import oracle as O
from tests._util import LINEAR_FIXTURES, load_fixture

CB = {"mul1": O.CB_MUL1, "mcg": O.CB_MCG}


# ---- binary16 conversion: exhaustive vs numpy's IEEE conversion ------------------------------------------------


def test_f16_to_f32_is_exact_for_every_half():
    halves = np.arange(1 << 16, dtype=np.uint16)
    want = halves.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(h)) for h in halves[::97]], np.float32)
    w = want[::97]
    same = (got == w) | (np.isnan(got) & np.isnan(w))
    assert same.all()


def test_f32_to_f16_rounds_to_nearest_even():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, size=4000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    # plus exact ties and the subnormal/overflow boundaries
    extra = np.array([2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -24, 65504.0, 65519.99, 65520.0, 1.0 + 2.0 ** -11,
                      1.0 + 3 * 2.0 ** -11, -0.0, 6.1e-5, 5.96e-8], np.float32)
    vals = np.concatenate([vals, extra])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in vals], np.uint16)
    nan = np.isnan(vals)
    assert (got[~nan] == want[~nan]).all()
    assert ((got[nan] & 0x7C00) == 0x7C00).all() and ((got[nan] & 0x3FF) != 0).all()


# ---- rates: the reference's hand table (expert_exl3.zig:661-697) ------------------------------------------------


@pytest.mark.parametrize("n,ends,fresh", [
    (40, [2, 5, 7, 10, 12, 15, 17, 20], [2, 3] * 8),
    (44, [2, 5, 8, 11, 13, 16, 19, 22], [2, 3, 3, 3] * 4),
    (48, [3, 6, 9, 12, 15, 18, 21, 24], [3] * 16),
    (64, [4, 8, 12, 16, 20, 24, 28, 32], [4] * 16),
])
def test_bit_end_hand_table(n, ends, fresh):
    assert [O.bit_end(n, i) for i in range(8)] == ends
    got_fresh = [O.bit_end(n, i) - (O.bit_end(n, i - 1) if i else 0) for i in range(16)]
    assert got_fresh == fresh
    assert O.bit_end(n, 255) == 16 * n


# ---- bitstream: an independent per-bit circular extraction (the reference's check, expert_exl3.zig:1051-1072) ----


def _brute_codewords(words: np.ndarray, n: int) -> np.ndarray:
    # Stream bit b is bit 15 - b%16 of halfword 2*(b//32) + (1 - (b%32)//16): each u32 word is hw[2i] | hw[2i+1] << 16
    # read MSB first.  Codeword t is the 16 bits ending at bitEnd(t), wrapping around the tile.
    total = 16 * n
    out = np.zeros(256, np.uint16)
    for t in range(256):
        end = ((t + 1) * n) // 16
        v = 0
        for bit in range(16):
            at = (end - 16 + bit) % total
            hw = int(words[2 * (at // 32) + (1 - (at % 32) // 16)])
            v = (v << 1) | ((hw >> (15 - at % 16)) & 1)
        out[t] = v
    return out


@pytest.mark.parametrize("n", list(range(16, 129, 2)))
def test_unpack_tile_matches_brute_force(n):
    rng = np.random.default_rng(0x51555348 + n)
    for _ in range(3):
        words = rng.integers(0, 1 << 16, size=n, dtype=np.uint32).astype(np.uint16)
        assert (O.unpack_tile(words, n) == _brute_codewords(words, n)).all()


def test_tensor_core_perm_is_the_fragment_order():
    perm = O.tensor_core_perm()
    assert sorted(perm.tolist()) == list(range(256))
    # spot values of tensorCorePerm (expert_exl3.zig:379-398): thread 5 -> rows {2,3,10,11}, cols {1,9}
    assert perm[40:48].tolist() == [2 * 16 + 1, 3 * 16 + 1, 10 * 16 + 1, 11 * 16 + 1,
                                    2 * 16 + 9, 3 * 16 + 9, 10 * 16 + 9, 11 * 16 + 9]


# ---- codebooks: the reference's known answers ---------------------------------------------------------------------


def test_mul1_known_codewords():  # expert_exl3.zig:699-704
    assert (O.decode_mul1(0), O.decode_mul1(1), O.decode_mul1(7)) == (49896, 14625, 47511)


def test_hash_mask_known_codewords_with_rounded_half_sums():  # expert_exl3.zig:729-739
    pair = (0x840C1F37, 0x8FFE8FD0)
    want = {0: 0x0000, 1: 0x3E0D, 7: 0xBF94, 0x15: 0xC060, 0x3E: 0xC164, 0x1234: 0xBAD0, 0xFFFF: 0xBB8A}
    for cw, w in want.items():
        assert O.decode_hashmask(cw, *pair) == w, hex(cw)


def test_mcg_zero_codeword_closed_form():  # expert_exl3.zig:853-862
    lo = np.uint16(0x3B60).view(np.float16).astype(np.float32)
    assert O.decode_mcg(0) == np.float16(lo + lo).view(np.uint16)


PAIR_KATS = [  # expert_exl3.zig:770-795, sashimi's v2rot tables
    (24, 0x1, (0x3C74, 0xBDAA)), (24, 0x1234, (0x3A7C, 0xB8CB)), (32, 0x0, (0x0000, 0x0000)),
    (32, 0x1, (0xB440, 0xB804)), (32, 0x1234, (0x3822, 0xB086)), (32, 0xFFFF, (0xB19E, 0x3DA0)),
    (38, 0x1, (0x3FA4, 0x3610)), (38, 0x1234, (0x3A99, 0xB898)), (40, 0x1, (0x3FA6, 0x3610)),
    (40, 0x1234, (0x3A6D, 0xB898)), (48, 0x1, (0xB5B2, 0xB7AF)), (48, 0x15, (0x37C6, 0xA9D0)),
    (48, 0x8000, (0xA6E0, 0xB3EE)), (56, 0x1, (0xBF92, 0xB91E)), (56, 0x1234, (0xBCF0, 0xBAD6)),
    (58, 0x1, (0xBC90, 0x3608)), (58, 0x1234, (0x3CB0, 0xB102)), (64, 0x7, (0xAA00, 0xBA80)),
    (64, 0x15, (0xC010, 0x34F7)), (64, 0xFFFF, (0x3B10, 0x3C0C)),
]


@pytest.mark.parametrize("n,cw,want", PAIR_KATS)
def test_pair1_known_pairs(n, cw, want):
    assert O.decode_pair(cw, O.pair1_row(n)) == want


def test_pair1_rows_exist_only_at_even_rates_24_to_64():  # expert_exl3.zig:749-767
    for n in range(16, 73):
        assert (O.pair1_row(n) is not None) == (n % 2 == 0 and 24 <= n <= 64)
    assert O.pair1_row(38).mask0 == 0x8E6E8F9A and O.pair1_row(36).mask0 == 0x8F9A8E6E


def test_pair1_tiles_fixture():  # expert_exl3.zig:797-815 (sashimi's numpy decode)
    d = load_fixture("exl3_pair1_tiles")
    for n in range(24, 65, 2):
        t, want = d[f"trellis_n{n}"], d[f"decoded_n{n}"]
        for i in range(t.shape[0]):
            assert (O.decode_tile(t[i], n, O.decode(O.CB_PAIR1)) == want[i]).all(), n


# ---- golden fixtures: inner and public bit-exact (expert_exl3.zig:864-997) ----------------------------------------


@pytest.mark.parametrize("name,n,cb,w", LINEAR_FIXTURES)
def test_linear_fixture_inner_and_public_bit_exact(name, n, cb, w):
    d = load_fixture(name)
    dec = O.decode(CB[cb], w)
    assert d["trellis"].shape == (8, 8, n)
    inner = O.reconstruct_inner(d["trellis"], 128, 128, n, dec)
    assert (inner == d["inner"]).all()
    pub = O.reconstruct_public(d["trellis"], d["suh"], d["svh"], 128, 128, n, dec)
    assert (pub == d["public"]).all()


def test_w12_fixture_read_at_w16_is_a_different_matrix():  # expert_exl3.zig:987-996
    d = load_fixture("exl3_k2p5_mcg_w12_linear")
    wide = O.reconstruct_inner(d["trellis"], 128, 128, 40, O.decode(O.CB_MCG, 16))
    assert not (wide == d["inner"]).all()


def test_narrow_windows_mask_the_codeword():  # expert_exl3.zig:1015-1039
    d = load_fixture("exl3_k2p5_mcg_linear")
    tile = d["trellis"].reshape(-1)[:40]
    cws = O.unpack_tile(tile, 40)
    perm = O.tensor_core_perm()
    wide = O.decode_tile(tile, 40, O.decode(O.CB_MCG))
    for bits in (8, 10):
        got = O.decode_tile(tile, 40, O.decode(O.CB_MCG, bits))
        want = np.zeros(256, np.uint16)
        want[perm] = [O.decode_mcg(int(c) & ((1 << bits) - 1)) for c in cws]
        assert (got == want).all() and not (got == wide).all()


# ---- codebook tables: sha256 digests pinned by the reference (codebook_tables.zig:243-307) -----------------------


def _digest(fields, ns, rows):
    h = hashlib.sha256()
    for n, r in zip(ns, rows):
        h.update((f"{n}" + "".join(f",{v:08x}" for v in r[:fields]) + "\n").encode())
    return h.hexdigest()[:8]


def test_digest_fixed_vector():  # codebook_tables.zig:281-285
    assert _digest(4, [24, 64], [(1, 2, 3, 4), (0xFFFFFFFF, 0, 0x80000000, 0x7FFFFFFF)]) == "72fc0906"


TABLE_DIGESTS = {0: "c089b4eb", 1: "37f72431", 2: "753ffa03", 3: "c5dba171"}


@pytest.mark.parametrize("table", [0, 1, 2, 3])
def test_oracle_tables_hash_to_the_pinned_digests(table):
    info = O.table_info(table)
    ns = [info["n_lo"] + 2 * i for i in range(info["rows"])]
    rows = [O.table_row(table, n) for n in ns]
    assert _digest(info["fields"], ns, rows) == TABLE_DIGESTS[table]


def test_spec1_w15_legacy_digest_is_its_k4_rows():  # codebook_tables.zig:418-426
    ns = list(range(24, 65, 2))
    assert _digest(2, ns, [O.table_row(1, n) for n in ns]) == "2ac2594d"


def _header_tables():
    """The HIP library's own copy of the tables (sushi_amd/csrc/exl3_tables.h), parsed from its source."""
    src = open(os.path.join(os.path.dirname(__file__), "..", "sushi_amd", "csrc", "exl3_tables.h")).read()

    def block(name):
        body = re.search(name + r"\[[^\]]*\](?:\[[^\]]*\])? = \{(.*?)\};", src, re.S).group(1)
        return [tuple(int(v.rstrip("u"), 0) for v in re.findall(r"0x[0-9A-Fa-f]+u?|\b\d+\b", row))
                for row in re.findall(r"\{([^{}]*)\}", body)]

    pair = block("kPair1Rows")
    w15 = block("kSpec1W15")
    w16 = block("kSpec1W16")
    std = tuple(int(v.rstrip("u"), 0) for v in re.findall(r"0x[0-9A-Fa-f]+u?",
                                                          re.search(r"kStd1Pair\[2\] = \{(.*?)\}", src).group(1)))
    return {0: (24, [(r[0], r[1], r[2], r[3]) for r in pair]), 1: (16, w15), 2: (24, w16), 3: (24, [std] * 21)}


@pytest.mark.parametrize("table", [0, 1, 2, 3])
def test_hip_library_tables_hash_to_the_pinned_digests(table):
    n_lo, rows = _header_tables()[table]
    fields = 4 if table == 0 else 2
    ns = [n_lo + 2 * i for i in range(len(rows))]
    assert _digest(fields, ns, rows) == TABLE_DIGESTS[table]


# ---- decodeTile over every codebook x window x even rate (expert_exl3.zig:1073-1087) -----------------------------


@pytest.mark.parametrize("n", [16, 24, 32, 40, 46, 48, 56, 64, 66, 96, 128])
def test_decode_tile_composes_unpack_perm_and_codebook(n):
    rng = np.random.default_rng(n)
    words = rng.integers(0, 1 << 16, size=n, dtype=np.uint32).astype(np.uint16)
    cws = _brute_codewords(words, n)
    perm = O.tensor_core_perm()
    for bits in (8, 12, 15, 16):
        mask = (1 << bits) - 1
        for cb, fn in ((O.CB_MCG, O.decode_mcg), (O.CB_MUL1, O.decode_mul1), (O.CB_3INST, O.decode_3inst)):
            got = O.decode_tile(words, n, O.decode(cb, bits))
            assert all(got[perm[i]] == fn(int(c) & mask) for i, c in enumerate(cws))
        for table in (1, 3):
            row = O.table_row(table, n)
            cb = O.CB_SPEC1 if table == 1 else O.CB_STD1
            if row is None:
                with pytest.raises(ValueError):
                    O.decode_tile(words, n, O.decode(cb, bits, table))
                continue
            got = O.decode_tile(words, n, O.decode(cb, bits, table))
            assert all(got[perm[i]] == O.decode_hashmask(int(c) & mask, row[0], row[1]) for i, c in enumerate(cws))
        p = O.pair1_row(n)
        if p is not None:
            got = O.decode_tile(words, n, O.decode(O.CB_PAIR1, bits))
            for i in range(256):
                assert got[perm[i]] == O.decode_pair(int(cws[i | 1]) & mask, p)[i & 1]


# ---- 3INST (extension, absent from the reference): closed-form pins ----------------------------------------------


def test_3inst_is_the_lcg_step_then_the_mcg_mask_xor_and_half_sum():
    # The LCG x -> 89226354 x + 64248484 (mod 2^32) followed by (x & 0x8FFF8FFF) ^ 0x3B603B60 and the f16 sum of
    # the two halves: the same post-processing MCG uses, which the reference's fixtures pin (test above).  So a
    # codeword whose LCG image equals some MCG product must decode to the MCG value of that codeword.
    # Codewords whose masked LCG image equals a masked MCG product share the post-processing exactly.
    cws = np.arange(1 << 16, dtype=np.uint64)
    m = 0x8FFF8FFF
    lcg = ((cws * 89226354 + 64248484) & 0xFFFFFFFF) & m
    mcg = ((cws * 0xCBAC1FED) & 0xFFFFFFFF) & m
    where = {int(v): int(c) for c, v in zip(cws, mcg)}
    hits = [(int(c), where[int(v)]) for c, v in zip(cws, lcg) if int(v) in where]
    assert len(hits) >= 32
    for c3, cm in hits:
        assert O.decode_3inst(c3) == O.decode_mcg(cm)
    # and the zero codeword lands on b itself
    b = 64248484
    h = (b & 0x8FFF8FFF) ^ 0x3B603B60
    lo = np.uint16(h & 0xFFFF).view(np.float16).astype(np.float32)
    hi = np.uint16(h >> 16).view(np.float16).astype(np.float32)
    assert O.decode_3inst(0) == np.float16(lo + hi).view(np.uint16)


def test_3inst_values_are_roughly_unit_gaussian():
    vals = np.array([O.decode_3inst(c) for c in range(0, 1 << 16, 3)], np.uint16).view(np.float16).astype(np.float64)
    assert abs(vals.mean()) < 0.05 and 0.7 < vals.std() < 1.3
