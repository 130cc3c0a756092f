"""GPU decode parity: every codeword of every codebook, and dequantized tiles, bit-exact with the oracle.

Mirrors the reference's exhaustive GPU decode tests (src/exl3/kernel_source.zig:409-517), its "every admitted rate
reads exactly on every reader" check (src/exl3/expert_exl3_kernels.zig:6615) and its fixture tests.  `reconstruct_inner`
runs the decoder the GEMV and the GEMM multiply with (the lane reader + lane decoder at n = 16/24/32/40/48/64, the
generic reader elsewhere), so these tests pin the hot path's own dequantized weights.
"""
import numpy as np
import pytest
import torch

import oracle as O
from sushi_amd import exl3
from tests._util import LINEAR_FIXTURES, load_fixture

pytestmark = pytest.mark.gpu

ALL = np.arange(1 << 16, dtype=np.uint16)

# (label, exl3.Decode, oracle decode, rate n)
CASES = [
    ("mcg", exl3.Decode(exl3.Codebook.mcg), O.decode(O.CB_MCG), 64),
    ("mul1", exl3.Decode(exl3.Codebook.mul1), O.decode(O.CB_MUL1), 64),
    ("3inst", exl3.Decode(exl3.Codebook.inst3), O.decode(O.CB_3INST), 64),
    ("mcg_w12", exl3.Decode(exl3.Codebook.mcg, exl3.Window(12)), O.decode(O.CB_MCG, 12), 64),
    ("mcg_w8", exl3.Decode(exl3.Codebook.mcg, exl3.Window(8)), O.decode(O.CB_MCG, 8), 64),
    ("std1", exl3.Decode(exl3.Codebook.std1, exl3.Window(15), 3), O.decode(O.CB_STD1, 15, 3), 40),
] + [
    (f"spec1_w15_n{n}", exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1), n)
    for n in (16, 24, 32, 48, 64, 96, 128)
] + [
    (f"spec1_w16_n{n}", exl3.Decode(exl3.Codebook.spec1, exl3.Window(16), 2), O.decode(O.CB_SPEC1, 16, 2), n)
    for n in (24, 40, 64)
] + [
    (f"pair1_n{n}", exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1), n) for n in range(24, 65, 2)
]


@pytest.mark.parametrize("label,dec,odec,n", CASES, ids=[c[0] for c in CASES])
def test_every_codeword_decodes_bit_exact(dev, label, dec, odec, n):
    print(f"[decode] {label}", flush=True)
    got = exl3.decode_codewords(torch.from_numpy(ALL.view(np.int16)).to(dev), n, dec)
    want = O.decode_codewords(ALL, n, odec)
    got = got.cpu().numpy().view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{label}: {bad.size} mismatches, first cw index {bad[:4]}"


CB = {"mul1": exl3.Codebook.mul1, "mcg": exl3.Codebook.mcg}


@pytest.mark.parametrize("name,n,cb,w", LINEAR_FIXTURES)
def test_reconstruct_inner_matches_the_reference_fixtures(dev, name, n, cb, w):
    d = load_fixture(name)
    t = torch.from_numpy(d["trellis"].view(np.int16)).to(dev)
    got = exl3.reconstruct_inner(t, exl3.Decode(CB[cb], exl3.Window(w))).cpu().numpy().view(np.uint16)
    assert (got == d["inner"]).all()


DEC_RT = [
    ("mcg", exl3.Decode(exl3.Codebook.mcg), O.decode(O.CB_MCG)),
    ("mul1", exl3.Decode(exl3.Codebook.mul1), O.decode(O.CB_MUL1)),
    ("3inst_w13", exl3.Decode(exl3.Codebook.inst3, exl3.Window(13)), O.decode(O.CB_3INST, 13)),
    ("spec1", exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1), O.decode(O.CB_SPEC1, 15, 1)),
    ("pair1", exl3.Decode(exl3.Codebook.pair1), O.decode(O.CB_PAIR1)),
]


@pytest.mark.parametrize("n", [16, 22, 24, 32, 40, 44, 48, 62, 64, 66, 96, 128])
@pytest.mark.parametrize("label,dec,odec", DEC_RT, ids=[c[0] for c in DEC_RT])
def test_reconstruct_inner_every_rate(dev, n, label, dec, odec):
    if label == "pair1" and not (24 <= n <= 64):
        pytest.skip("PAIR1 has rows only at n = 24..64")
    rng = np.random.default_rng(n * 31 + len(label))
    t = rng.integers(0, 1 << 16, size=(4, 8, n), dtype=np.uint32).astype(np.uint16)
    want = O.reconstruct_inner(t, 64, 128, n, odec)
    got = exl3.reconstruct_inner(torch.from_numpy(t.view(np.int16)).to(dev), dec).cpu().numpy().view(np.uint16)
    assert (got == want).all()


# Every lane-reader rate x every codebook family x three windows, over 4221 random tiles (63 x 67: the last wave of
# the lane kernel holds 5 live tiles), bit for bit against the oracle's decodeTile composition.
LANE_RATES = (16, 24, 32, 40, 48, 64)
READER_CODEBOOKS = [
    ("mcg", exl3.Codebook.mcg, None, O.CB_MCG),
    ("mul1", exl3.Codebook.mul1, None, O.CB_MUL1),
    ("3inst", exl3.Codebook.inst3, None, O.CB_3INST),
    ("spec1_w15tab", exl3.Codebook.spec1, 1, O.CB_SPEC1),
    ("spec1_w16tab", exl3.Codebook.spec1, 2, O.CB_SPEC1),
    ("std1", exl3.Codebook.std1, 3, O.CB_STD1),
    ("pair1", exl3.Codebook.pair1, None, O.CB_PAIR1),
]


def _has_rows(label, table, n):
    if label == "pair1":
        return O.pair1_row(n) is not None
    return table is None or O.table_row(table, n) is not None


@pytest.mark.parametrize("window", [16, 12, 8])
@pytest.mark.parametrize("n", LANE_RATES)
@pytest.mark.parametrize("label,cb,table,ocb", READER_CODEBOOKS, ids=[c[0] for c in READER_CODEBOOKS])
def test_lane_reader_decodes_every_rate_codebook_and_window_bit_exact(dev, label, cb, table, ocb, n, window):
    if not _has_rows(label, table, n):
        pytest.skip(f"{label} has no row at n={n}")
    print(f"[reader] {label} n={n} w{window}", flush=True)
    it, ot = 63, 67
    rng = np.random.default_rng(1000 * n + 10 * window + len(label))
    t = rng.integers(0, 1 << 16, size=(it, ot, n), dtype=np.uint32).astype(np.uint16)
    odec = O.decode(ocb, window, O.TABLE_NONE if table is None else table)
    want = O.reconstruct_inner(t, it * 16, ot * 16, n, odec)
    dec = exl3.Decode(cb, exl3.Window(window), table)
    got = exl3.reconstruct_inner(torch.from_numpy(t.view(np.int16)).to(dev), dec).cpu().numpy().view(np.uint16)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{label} n={n} w{window}: {len(bad)} weights differ, first at (k, out) {bad[:3].tolist()}"


@pytest.mark.parametrize("n", list(range(24, 65, 2)))
def test_reconstruct_inner_matches_the_reference_pair1_tiles(dev, n):
    """The reference's PAIR1 fixture (src/exl3/expert_exl3.zig:797-815): three tiles per rate, decoded tile by tile
    through the reader each rate takes (lane reader at 24/32/40/48/64, generic elsewhere)."""
    d = load_fixture("exl3_pair1_tiles")
    t, want = d[f"trellis_n{n}"], d[f"decoded_n{n}"]
    got = exl3.reconstruct_inner(torch.from_numpy(t.reshape(1, 3, n).view(np.int16)).to(dev),
                                 exl3.Decode(exl3.Codebook.pair1)).cpu().numpy().view(np.uint16)
    for i in range(3):
        assert (got[:, 16 * i:16 * i + 16].reshape(256) == want[i]).all(), i
