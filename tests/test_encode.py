"""Trellis encoder search: the CPU oracle against the reference's own search fixture and brute force, then the GPU
search (``exl3_encode_tiles``) against the oracle and the fixture, code for code.

The oracle restates src/encoder/encode.zig; its checks follow the reference's tests (encode.zig:313-503):
``exl3_encode_tiles.safetensors`` holds, for 13 codebook x rate x window configs, eight tiles with the packed codes and
costs of the reference search.
"""
from __future__ import annotations

import ctypes
import itertools
import os

import numpy as np
import pytest

import oracle as O

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref", "exl3_encode_tiles.safetensors")


def _fixture():
    from safetensors.numpy import load_file

    d = load_file(FIXTURE)
    cfgs = sorted({k.split(".")[0] for k in d})
    out = []
    for c in cfgs:
        cb, n, w = c.split("_")
        out.append((c, O.CB_MCG if cb == "mcg" else O.CB_MUL1, int(n[1:]), int(w[1:]), d[c + ".x"], d[c + ".packed"],
                    d[c + ".cost"]))
    return out


def fresh_bits(n):
    return np.array([(((t + 1) * n) >> 4) - ((t * n) >> 4) for t in range(256)], np.uint8)


def test_the_fixture_covers_the_reference_configs():
    names = [c[0] for c in _fixture()]
    assert len(names) == 13 and "mcg_n64_w16" in names and "mul1_n44_w12" in names  # encode.zig:433-447


@pytest.mark.parametrize("case", _fixture(), ids=lambda c: c[0])
def test_oracle_packed_codes_match_the_reference_search(case):  # encode.zig:453-471
    name, cb, n, w, xs, packed, costs = case
    for i in range(len(costs)):
        p, sse, _ = O.encode_tile(xs[i], n, O.decode(cb, w))
        np.testing.assert_array_equal(p, packed[i], err_msg=f"{name} tile {i}")
        assert abs(sse - costs[i]) <= 1e-12 * abs(costs[i])


@pytest.mark.parametrize("cb,n,w", [(O.CB_MCG, 24, 12), (O.CB_MCG, 36, 12), (O.CB_MCG, 40, 15), (O.CB_MCG, 52, 16),
                                    (O.CB_MUL1, 44, 12), (O.CB_MUL1, 48, 15), (O.CB_MUL1, 64, 16),
                                    (O.CB_3INST, 32, 14), (O.CB_MCG, 16, 13), (O.CB_MCG, 128, 12)])
def test_every_code_the_search_writes_decodes_to_the_values_it_scored(cb, n, w):  # encode.zig:313-335
    rng = np.random.default_rng(7 + n + w)
    dec = O.decode(cb, w)
    for _ in range(2):
        tile = rng.standard_normal(256).astype(np.float32)
        packed, sse, recon = O.encode_tile(tile, n, dec)
        decoded = O.decode_tile(packed, n, dec)
        np.testing.assert_array_equal(decoded, recon.astype(np.float16).view(np.uint16))
        err = tile.astype(np.float64) - decoded.view(np.float16).astype(np.float64)
        assert abs(float((err * err).sum()) - sse) <= 1e-9 * sse


def _brute(xs, ks, table, w):
    """Every tail-biting path by enumeration: min cost per closing register (encode.zig:337-374)."""
    total = int(sum(ks))
    k0 = int(ks[0])
    mask, reg_mask = (1 << w) - 1, (1 << (w - k0)) - 1
    best = np.full(1 << (w - k0), np.inf)
    fs = np.arange(1 << total, dtype=np.int64)
    for pre in range(1 << w):
        cw = np.full(fs.shape, pre, np.int64)
        rest = fs.copy()
        cost = np.zeros(fs.shape)
        for k, xv in zip(ks, xs):
            f = rest & ((1 << int(k)) - 1)
            rest >>= int(k)
            cw = ((cw << int(k)) | f) & mask
            cost += (xv - table[cw]) ** 2
        ok = (cw & reg_mask) == (pre & reg_mask)
        if ok.any():
            best[pre & reg_mask] = min(best[pre & reg_mask], cost[ok].min())
    return best


@pytest.mark.parametrize("ks", [(2, 3, 2, 2, 3, 2), (1, 2, 1, 2, 1, 2), (3, 3, 3, 3, 3)])
def test_the_pinned_pass_equals_brute_force_over_every_tail_biting_path(ks):  # encode.zig:337-393
    rng = np.random.default_rng(11 + sum(ks))
    w = 5
    ks = np.array(ks, np.uint8)
    for _ in range(3):
        table = rng.random(1 << w) * 4 - 2
        xs = rng.standard_normal(len(ks))
        brute = _brute(xs, ks, table, w)
        best = np.inf
        for reg in range(1 << (w - int(ks[0]))):
            c, path = O.viterbi_pass(xs, ks, table, w, reg)
            assert abs(brute[reg] - c) <= 1e-12
            assert abs(c - float(((xs - table[path.astype(np.int64)]) ** 2).sum())) <= 1e-12
            for i in range(1, len(ks)):
                k = int(ks[i])
                assert int(path[i]) >> k == int(path[i - 1]) & ((1 << (w - k)) - 1)
            best = min(best, c)
        exact, _ = O.exact_tail_biting(xs, ks, table, w)
        assert abs(best - exact) <= 1e-12
        free, _ = O.viterbi_pass(xs, ks, table, w)
        assert free <= best + 1e-12


@pytest.mark.parametrize("n", [24, 40, 44, 56])
def test_the_half_tile_warm_up_pin_reaches_the_exact_optimum_on_a_narrow_window(n):  # encode.zig:396-431
    rng = np.random.default_rng(23 + n)
    w = 9
    table = O.decode_codewords(np.arange(1 << w, dtype=np.uint16), 16, O.decode(O.CB_MCG)).view(np.float16)
    table = table.astype(np.float64)
    ks = fresh_bits(n)
    perm = O.tensor_core_perm()
    k0 = int(ks[0])
    for _ in range(4):
        tile = rng.standard_normal(256).astype(np.float32)
        x = tile[perm].astype(np.float64)
        rolled_x = np.roll(x, -128)
        rolled_k = np.roll(ks, -128)
        _, path = O.viterbi_pass(rolled_x, rolled_k, table, w)
        reg = int(path[127]) & ((1 << (w - k0)) - 1)
        cost, _ = O.viterbi_pass(x, ks, table, w, reg)
        exact, _ = O.exact_tail_biting(x, ks, table, w)
        assert exact == cost


def test_a_rate_or_window_the_trellis_cannot_carry_is_refused():  # encode.zig:486-503
    tile = np.zeros(256, np.float32)
    for n, w, want in ((41, 16, "RateUnsupported"), (8, 16, "RateUnsupported"), (128, 8, "WindowUnsupported"),
                       (32, 11, "WindowUnsupported"), (15, 16, "RateUnsupported")):
        with pytest.raises(ValueError, match=want):
            O.encode_tile(tile, n, O.decode(O.CB_MCG, w))
    with pytest.raises(ValueError, match="CodebookUnsupported"):
        O.encode_tile(tile, 32, O.decode(O.CB_PAIR1, 16))


def test_the_c_abi_refuses_before_any_launch():
    """Status codes of ``exl3_encode_tiles`` for the encoder's named refusals (no GPU work: the plan refuses first)."""
    from sushi_amd import _lib, exl3

    L = _lib.load()
    for n, dec, want in ((41, exl3.MCG, exl3.RateUnsupported), (32, exl3.Decode(exl3.Codebook.pair1),
                                                                 exl3.CodebookUnsupported),
                         (32, exl3.Decode(exl3.Codebook.mcg, exl3.Window(11)), exl3.Exl3WindowUnsupported),
                         (32, exl3.Decode(exl3.Codebook.spec1), exl3.CodebookUnsupported)):
        assert L.exl3_encode_tiles(0, 1, n, dec.c(), 0, 0, 0, 0, 0) == want.status
        assert L.exl3_encode_workspace_size(n, dec.c(), 1) == 0
    assert L.exl3_encode_workspace_size(64, exl3.MCG.c(), 1000) > 0


# ---- GPU search ---------------------------------------------------------------------------------------------------


def _gpu_encode(dev, tiles, n, cb, w):
    import torch

    from sushi_amd import exl3

    dec = exl3.Decode(exl3.Codebook(cb), exl3.Window(w))
    packed, sse = exl3.encode_tiles(torch.from_numpy(np.ascontiguousarray(tiles, np.float32)).to(dev), n, dec)
    torch.cuda.synchronize()
    return packed.cpu().numpy().view(np.uint16), sse.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("case", _fixture(), ids=lambda c: c[0])
def test_gpu_search_matches_the_reference_fixture(dev, case):
    name, cb, n, w, xs, packed, costs = case
    got, sse = _gpu_encode(dev, xs, n, cb, w)
    np.testing.assert_array_equal(got, packed, err_msg=name)
    np.testing.assert_allclose(sse, costs, rtol=1e-12, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("cb,n,w,count", [(O.CB_MCG, 16, 12, 37), (O.CB_MCG, 32, 16, 3), (O.CB_MUL1, 48, 13, 21),
                                          (O.CB_3INST, 64, 15, 5), (O.CB_MCG, 128, 12, 19), (O.CB_MUL1, 24, 14, 9),
                                          (O.CB_MCG, 16, 16, 2), (O.CB_3INST, 40, 12, 33)])
def test_gpu_search_is_the_oracle_code_for_code(dev, cb, n, w, count):
    rng = np.random.default_rng(1000 + n * 17 + w)
    tiles = (rng.standard_normal((count, 256)) * rng.uniform(0.2, 3.0, (count, 1))).astype(np.float32)
    got, sse = _gpu_encode(dev, tiles, n, cb, w)
    for i in range(count):
        want, want_sse, _ = O.encode_tile(tiles[i], n, O.decode(cb, w))
        np.testing.assert_array_equal(got[i], want, err_msg=f"tile {i}")
        assert sse[i] == want_sse


@pytest.mark.gpu
def test_gpu_search_with_a_one_workgroup_workspace_runs_every_batch(dev):
    """A workspace for one workgroup: the grid shrinks to it and that workgroup walks every batch of tiles."""
    import torch

    from sushi_amd import _lib, exl3

    L = _lib.load()
    n, w, count = 32, 12, 70
    rng = np.random.default_rng(3)
    tiles = rng.standard_normal((count, 256)).astype(np.float32)
    t = torch.from_numpy(tiles).to(dev)
    packed = torch.zeros(count, n, dtype=torch.int16, device=dev)
    sse = torch.zeros(count, dtype=torch.float64, device=dev)
    dec = exl3.Decode(exl3.Codebook.mcg, exl3.Window(w))
    full = L.exl3_encode_workspace_size(n, dec.c(), count)
    one = L.exl3_encode_workspace_size(n, dec.c(), 1)
    assert 0 < one < full
    ws = torch.empty(one, dtype=torch.uint8, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rc = L.exl3_encode_tiles(t.data_ptr(), count, n, dec.c(), packed.data_ptr(), sse.data_ptr(), ws.data_ptr(),
                             ws.numel(), stream)
    assert rc == 0, _lib.last_error()
    assert L.exl3_encode_tiles(t.data_ptr(), count, n, dec.c(), packed.data_ptr(), sse.data_ptr(), ws.data_ptr(),
                               one - 1, stream) == exl3.Exl3WorkspaceTooSmall.status
    torch.cuda.synchronize()
    want, want_sse = _gpu_encode(dev, tiles, n, O.CB_MCG, w)
    np.testing.assert_array_equal(packed.cpu().numpy().view(np.uint16), want)
    np.testing.assert_array_equal(sse.cpu().numpy(), want_sse)
    for i in itertools.islice(range(count), 0, count, 7):
        p, s, _ = O.encode_tile(tiles[i], n, O.decode(O.CB_MCG, w))
        np.testing.assert_array_equal(want[i], p)
