"""Headline benchmark: EXL3 K=4 4096x4096 decode GEMV at batch 1 (BASELINE.json configs[0]'s shape, run on the GPU)
plus the MoE gathered-expert layer (configs[3], batch 1) as a secondary figure.

A step is one call of the hot path (prepare + trellis-decode GEMV + finish) on one token of seeded synthetic fp16
input.  Weights rotate over 64 resident copies (537 MB > the 256 MB Infinity Cache).  The calls are captured as HIP
graphs: one graph of the 64 copies and one of the first (steps mod 64).  A timed round is exactly `--steps` calls
(whole 64-copy replays, then the tail), and an untimed replay of the 64-copy graph precedes every round, so each
timed call reads a copy last read 64 calls (537 MB of other weights) earlier: from HBM.  Seven rounds are timed
(each bracketed by synchronisations) and the median round is reported.  The kernel's per-launch time comes from HIP
events around two graphs, the 64-copy sequence and the same sequence followed by the `--steps` timed calls: their
difference is the timed calls back to back inside one graph, without the start cost of a second graph.

Prints one JSON line (the driver's contract).  `cpu_baseline` times the C restatement of the reference's CPU path
(oracle/, `expert_exl3.project`) on a bounded sample of the same workload, on every host core and on one.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor figure
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, vendor figure (no sparsity)
COPIES = 64
ROUNDS = 7
SWEEP_GRAPHS = True  # --no-graph: the sweep issues every call from Python (for counter passes, one dispatch each)


def _algorithmic_bytes(in_f: int, out_f: int, n: int, rows: int) -> int:
    """Packed trellis + suh + svh + x + y (f16), per call."""
    return in_f * out_f * n // 128 + 2 * (in_f + out_f) + 2 * rows * (in_f + out_f)


def _capture(calls, dev):
    """One HIP graph holding `calls()` (captured on a side stream, outside any timed region).  One eager pass on the
    side stream first: the library's per-stream workspace is allocated and zeroed there before the capture."""
    import torch

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        calls()
        side.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            calls()
    torch.cuda.current_stream(dev).wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    return g


def bench_linear(steps: int, warmup: int, graph_mode: bool = True, rounds: int = ROUNDS, codebook: str = "3inst"):
    """C1's GEMV; `codebook` "3inst" (the configuration's, an extension the reference lacks) or "mcg" (the same codes
    through the reference's MCG decode, whose arithmetic the reference's fixtures pin)."""
    import statistics

    import torch

    from sushi_amd import exl3, synth

    dev = torch.device("cuda:0")
    in_f = out_f = 4096
    n, rows = 64, 1
    trellis = synth.codes(0, "c1.trellis", (COPIES, in_f // 16, out_f // 16, n), device=dev)
    suh = synth.sign_scale(0, "c1.suh", (1, in_f), device=dev)
    svh = synth.sign_scale(0, "c1.svh", (1, out_f), device=dev)
    x = synth.normal(0, "c1.x", (rows, in_f), device=dev)
    projs = [exl3.Proj(trellis[i:i + 1], suh, svh) for i in range(COPIES)]
    dec = exl3.INST3 if codebook == "3inst" else exl3.MCG
    y = exl3.linear(x, projs[0], dec)  # workspace, library load
    for i in range(warmup):
        exl3.linear(x, projs[i % COPIES], dec)
    torch.cuda.synchronize()
    # The host side of a call (Python checks + ctypes) costs more than the kernel, so the calls are captured, one per
    # weight copy, into HIP graphs (outside the timed region) and replayed: a round then holds exactly `steps`
    # library launches back to back, as a native caller would issue them.
    full = tail = merged = None
    if graph_mode:
        full = _capture(lambda: [exl3.linear(x, projs[i], dec) for i in range(COPIES)], dev)
        if steps % COPIES:
            tail = _capture(lambda: [exl3.linear(x, projs[i], dec) for i in range(steps % COPIES)], dev)
        # the eviction sequence and then the timed calls, in one graph (each timed call's copy last read 64 calls
        # earlier, as in the two-graph round)
        merged = _capture(lambda: [exl3.linear(x, projs[i % COPIES], dec) for i in list(range(COPIES)) +
                                   list(range(steps))], dev)
    stream = torch.cuda.current_stream(dev)

    def evict():
        # the 64-copy sequence, untimed: every copy the round reads was last read 64 calls earlier
        if graph_mode:
            full.replay()
        else:
            for i in range(COPIES):
                exl3.linear(x, projs[i], dec)

    def timed_calls():
        if graph_mode:
            for _ in range(steps // COPIES):
                full.replay()
            if tail is not None:
                tail.replay()
        else:
            for i in range(steps):
                exl3.linear(x, projs[i % COPIES], dec)

    def event_ms(pre, body):
        # HIP events on the launch stream around body(), submitted while pre() still runs, so the events bracket
        # the GPU's work back to back and not the host's launch latency ahead of it
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        pre()
        e0.record(stream)
        body()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    # Each round times the `steps` calls right after an untimed eviction pass: by wall clock, bracketed by
    # synchronisations, so it holds the host's submission of the calls too (the whole-job figure); and by HIP events
    # on the launch stream, twice: around the timed calls' own graphs (`direct`: this holds the start of a second
    # graph behind the eviction graph, which costs the GPU some 10-15 us whatever the graph holds), and as the
    # difference between the merged graph and the eviction graph alone (`in_graph`: the timed calls back to back
    # inside one graph, the per-launch time a caller's longer graph sees).
    walls, events, in_graph = [], [], []
    for _ in range(rounds):
        evict()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        timed_calls()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        events.append(event_ms(evict, timed_calls))
        if graph_mode:  # three differences a round: each is two ~0.5 ms spans whose jitter the median absorbs
            in_graph += [event_ms(evict, merged.replay) - event_ms(evict, full.replay) for _ in range(3)]
    bytes_per_call = _algorithmic_bytes(in_f, out_f, n, rows)
    del full, tail, merged, trellis, projs
    torch.cuda.empty_cache()
    return dict(wall_s=statistics.median(walls), event_ms=statistics.median(events),
                in_graph_ms=statistics.median(in_graph) if in_graph else None, bytes=bytes_per_call, rows=rows,
                y=y, steps=steps, rounds=rounds, wall_rounds_s=walls)


def bench_moe(batch: int, layers: int = 16, rounds: int = ROUNDS):
    """E=256 routed + shared, hidden 2048, inter 768, K2 MCG, top-8; microseconds per token.

    `layers` MoE layers back to back on one stream, captured once as a HIP graph and replayed: the stream runs them
    in order, as the reference's dependent chain (bench_util.zig:20-58) runs its calls, but each layer reads its own
    N(0,1) hidden state (an unnormalised chain of SwiGLU layers squares its scale per layer and is inf by the fourth)
    and every layer has its own routing, so the distinct experts hit change from layer to layer.  Every layer has its
    own bank (16 x 302 MB), as a model's layers do: the weights a layer reads were last read 15 layers (4.5 GB, far
    past the 256 MB Infinity Cache) earlier, so they come from HBM.  The banks' svh carry 1/sqrt(in) (synth norm),
    keeping each layer's output near unit scale.  Per layer: HIP events around a graph of the layers twice over less
    those around the graph of the layers once, median of `rounds` rounds."""
    import statistics

    import torch

    from sushi_amd import exl3, synth

    dev = torch.device("cuda:0")
    E, hidden, inter, n, k = 256, 2048, 768, 32, 8
    banks = [synth.bank(3, f"c4.l{layer}", E, hidden, inter, n, device=dev, norm=True) for layer in range(layers)]
    shareds = [synth.bank(3, f"c4.shared.l{layer}", 1, hidden, inter, n, device=dev, norm=True)
               for layer in range(layers)]
    xs = [synth.normal(3, f"c4.x{batch}.{layer}", (batch, hidden), device=dev) for layer in range(layers)]
    routes = []
    for layer in range(layers):
        logits = synth.normal(3, f"c4.logits{batch}.{layer}", (batch, E), dtype=torch.float32).to(dev)
        routes.append(exl3.moe_routing_chain(logits, k))

    def chain():
        # routed experts + the shared expert in one call: the fused form runs both in the same launches; where it
        # declines, the wrapper runs the shared expert as a one-expert chain first
        return [exl3.moe_with_shared_bank(x, bank, shared, inds, scores, exl3.MCG)
                for x, (inds, scores), bank, shared in zip(xs, routes, banks, shareds)]

    chain()
    torch.cuda.synchronize()
    g = _capture(chain, dev)
    # the layers twice over in one graph: the second pass reads each bank 15 layers after the first
    g2 = _capture(lambda: (chain(), chain()), dev)
    stream = torch.cuda.current_stream(dev)

    def event_us(body):
        # events submitted behind a running replay, so they bracket the GPU's work back to back
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g.replay()
        e0.record(stream)
        body()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3

    # Per layer: the doubled graph less the single one (the layers back to back inside one graph, without the GPU's
    # start of a graph behind another); `direct`: events around the single graph.
    times, direct = [], []
    for _ in range(rounds):
        t1 = event_us(g.replay)
        times.append((event_us(g2.replay) - t1) / layers)
        direct.append(t1 / layers)
    layer_us = statistics.median(times)
    distinct = sum(len(set(i.flatten().tolist())) for i, _ in routes) / layers
    per_expert = 3 * (hidden * inter * n // 128 + 2 * (hidden + inter))
    del g, g2, banks, shareds
    torch.cuda.empty_cache()
    return dict(batch=batch, layer_us=layer_us, layer_us_direct=statistics.median(direct),
                us_per_token=layer_us / batch, distinct=distinct,
                bytes=(distinct + 1) * per_expert)


def _time_linear(in_f, out_f, n, rows, dec, codec_name, seed, min_pool_bytes=640 << 20, replays=6):
    """Average microseconds per exl3.linear call over a rotating pool of weight copies (pool > the 256 MB Infinity
    Cache), timed as HIP-graph replays between HIP events."""
    import torch

    from sushi_amd import exl3, synth

    dev = torch.device("cuda:0")
    wbytes = in_f * out_f * n // 128  # n halfwords per 256-weight tile
    copies = max(2, min(256, -(-min_pool_bytes // wbytes)))
    trellis = synth.codes(seed, f"sw.{codec_name}.{in_f}x{out_f}.{n}", (copies, in_f // 16, out_f // 16, n), device=dev)
    suh = synth.sign_scale(seed, "sw.suh", (1, in_f), device=dev)
    svh = synth.sign_scale(seed, "sw.svh", (1, out_f), device=dev)
    x = synth.normal(seed, f"sw.x{rows}", (rows, in_f), device=dev)
    projs = [exl3.Proj(trellis[i:i + 1], suh, svh) for i in range(copies)]
    exl3.linear(x, projs[0], dec)
    torch.cuda.synchronize()
    calls = lambda: [exl3.linear(x, projs[i], dec) for i in range(copies)]  # noqa: E731
    g = _capture(calls, dev) if SWEEP_GRAPHS else None
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        g.replay() if g is not None else calls()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * copies)
    del g, trellis, projs
    torch.cuda.empty_cache()
    return us, copies


def _bench_lib():
    import ctypes

    path = os.path.join(ROOT, "sushi_amd", "libsushi_bench_hip.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python -m sushi_amd.build`")
    L = ctypes.CDLL(path)
    L.sb_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    L.sb_stream_read.restype = ctypes.c_int32
    return L


def measured_ceilings(small_bytes: int):
    """Practical ceilings measured on this box beside the vendor peaks, with this build's streaming-read kernel
    (sushi_amd/csrc/bench_stream.hip: 16-byte loads, four in flight per thread, nothing written):
      * hbm_read_GBps: a 1 GiB read, best grid of three, median of 7 launches;
      * read_small_graph_us: a read of `small_bytes` (C1's packed bytes) per launch, 64 rotating buffers (537 MB, past
        the Infinity Cache) replayed from a HIP graph, median of 7 rounds: the floor a kernel with C1's traffic sits
        on, launch cost included;
      * launch_floor_us: a 16-byte read per launch, from a graph of 64 launches: the launch cost alone."""
    import ctypes
    import statistics

    import torch

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    L = _bench_lib()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    hs = ctypes.c_void_p(stream.cuda_stream)

    def read(buf, nbytes, blocks, s=None):
        rc = L.sb_stream_read(buf.data_ptr(), nbytes, blocks, sink.data_ptr(),
                              hs if s is None else ctypes.c_void_p(s.cuda_stream))
        if rc:
            raise RuntimeError(f"sb_stream_read: hip error {rc}")

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        out = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1) / 1e3)
        return statistics.median(out)

    big = torch.zeros(1 << 30, dtype=torch.uint8, device=dev)
    best = max(((1 << 30) / timed(lambda b=b: read(big, 1 << 30, b), ROUNDS), b) for b in (1024, 2048, 4096))
    del big
    nb = (small_bytes + 15) // 16 * 16
    bufs = [torch.zeros(nb, dtype=torch.uint8, device=dev) for _ in range(COPIES)]
    floor = [torch.zeros(16, dtype=torch.uint8, device=dev) for _ in range(COPIES)]

    def graph(fn):
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            fn(side)
            side.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                fn(side)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        return g

    g_small = graph(lambda s: [read(b, nb, 1024, s) for b in bufs])
    g_floor = graph(lambda s: [read(b, 16, 1, s) for b in floor])
    small_s = timed(g_small.replay, ROUNDS) / COPIES
    floor_s = timed(g_floor.replay, ROUNDS) / COPIES
    del g_small, g_floor, bufs, floor
    torch.cuda.empty_cache()
    return {"hbm_read_GBps": round(best[0] / 1e9, 1), "hbm_read_grid": best[1],
            "read_small_graph_us": round(small_s * 1e6, 3), "read_small_bytes": nb,
            "read_small_GBps": round(nb / small_s / 1e9, 1), "launch_floor_us": round(floor_s * 1e6, 3),
            "how": "sushi_amd/csrc/bench_stream.hip streaming read: 1 GiB (best of 1024/2048/4096 workgroups, median "
                   "of 7); C1's packed bytes per launch over 64 rotating buffers from a HIP graph (median of 7 "
                   "rounds); a 16-byte read per launch from a graph (the launch cost)"}


def blas_f16_gemm_us(rows: int, in_f: int, out_f: int, reps: int = 20) -> float:
    """The practical MFMA ceiling: a plain f16 GEMM [rows, in] x [in, out] through torch.matmul (hipBLASLt), f32
    accumulate, both operands contiguous."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(rows, in_f, device=dev, generator=g).to(torch.float16)
    w = torch.randn(in_f, out_f, device=dev, generator=g).to(torch.float16)
    y = torch.matmul(x, w)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        torch.matmul(x, w, out=y)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    del x, w, y
    torch.cuda.empty_cache()
    return us


def bench_encode(cb_name: str, n: int, w: int, tiles: int, replays: int = 2):
    """The trellis encoder search (exl3.encode_tiles) over `tiles` random N(0,1) tiles: microseconds per tile, timed
    between HIP events after one untimed call."""
    import torch

    from sushi_amd import exl3, synth

    dev = torch.device("cuda:0")
    dec = exl3.Decode(exl3.Codebook.from_name(cb_name), exl3.Window(w))
    x = synth.normal(7, f"enc.{cb_name}.{n}.{w}", (tiles, 256), device=dev, dtype=torch.float32)
    exl3.encode_tiles(x[:64], n, dec)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        exl3.encode_tiles(x, n, dec)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / replays
    # The reference's CPU search (the single-threaded C port of Encoder.encodeTile) on a few of the same tiles.
    import oracle as O

    sample = x[:4].cpu().numpy()
    cb = {"mcg": O.CB_MCG, "mul1": O.CB_MUL1, "3inst": O.CB_3INST}[cb_name]
    t0 = time.perf_counter()
    for tile in sample:
        O.encode_tile(tile, n, O.decode(cb, w))
    cpu_us = (time.perf_counter() - t0) / len(sample) * 1e6
    return {"config": "encode", "codebook": cb_name, "K": n / 16, "window": w, "tiles": tiles,
            "us_per_call": round(us, 1), "us_per_tile": round(us / tiles, 3), "tiles_per_s": round(tiles / (us * 1e-6)),
            "weights_per_s": round(256 * tiles / (us * 1e-6)),
            "cpu_baseline": {"us_per_tile": round(cpu_us, 1), "cores": 1, "kind": "port",
                             "sample": f"{len(sample)} of the same tiles through the C port of encodeTile"}}


def bench_quantize(in_f: int, out_f: int, n: int, cb_name: str, w: int):
    """The whole-tensor quantizer (exl3.quantize_named) on a random weight [in, out] with a random SPD Hessian: wall
    seconds per tensor (host factor + GPU searches), and the decoded weight's relative error."""
    import numpy as np
    import torch

    from sushi_amd import exl3

    rng = np.random.default_rng(in_f + out_f)
    wt = (rng.standard_normal((in_f, out_f)) * 0.02).astype(np.float32)
    x = (rng.standard_normal((in_f, 256)) * 0.1).astype(np.float32)
    h = (x @ x.T).astype(np.float32)
    h[np.arange(in_f), np.arange(in_f)] += 0.01
    dec = exl3.Decode(exl3.Codebook.from_name(cb_name), exl3.Window(w))
    torch.cuda.synchronize()
    t0 = time.time()
    packed, suh, svh, g = exl3.quantize_named(wt, h, 1, f"bench.{in_f}x{out_f}", n, dec, "auto")
    secs = time.time() - t0
    dev = torch.device("cuda:0")
    proj = exl3.Proj(torch.from_numpy(packed.view(np.int16)).reshape(1, in_f // 16, out_f // 16, n).to(dev),
                     torch.from_numpy(suh.view(np.float16)).reshape(1, in_f).to(dev),
                     torch.from_numpy(svh.view(np.float16)).reshape(1, out_f).to(dev))
    dense = exl3.linear(torch.eye(in_f, dtype=torch.float16, device=dev), proj, dec).float().cpu().numpy()
    rel = float(np.linalg.norm(dense - wt) / np.linalg.norm(wt))
    return {"config": "quantize", "codebook": cb_name, "K": n / 16, "window": w, "in": in_f, "out": out_f,
            "seconds": round(secs, 3), "tiles_per_s": round(in_f * out_f / 256 / secs), "g": round(g, 5),
            "decoded_rel_err": round(rel, 4)}


def bench_pack(pair_major: bool, experts: int = 256, hidden: int = 2048, inter: int = 768, n: int = 32):
    """The pack loader on one C4-shaped routed layer (E=256, hidden 2048, inter 768, K2: 302 MB of trellis) written as
    a safetensors pack under a temporary directory: seconds from Pack() to the device bank (page cache warm: the
    shard was just written; after one untimed load), against reading the same shard bytes and copying them to the
    device raw."""
    import shutil
    import tempfile

    import numpy as np
    import torch

    from sushi_amd import pack as P

    root = tempfile.mkdtemp(prefix="exl3pack")
    try:
        rng = np.random.default_rng(1)
        tensors = {}
        for g in range(2):  # two rate groups of experts / 2 each (pair-major packs are rate-grouped)
            e = experts // 2
            for proj in P.PROJECTIONS:
                inp, out = (inter, hidden) if proj == "down_proj" else (hidden, inter)
                tr = rng.integers(0, 1 << 16, size=(e, inp // 16, out // 16, n), dtype=np.uint16)
                key = f"model.layers.0.mlp.switch_mlp.{proj}.g{g}"
                if pair_major:
                    tr = tr.reshape(e, inp // 16, out // 32, 2, n).transpose(0, 2, 1, 3, 4).copy()
                    tensors[key + ".trellis_pm"] = tr
                else:
                    tensors[key + ".trellis"] = tr
                tensors[key + ".suh"] = np.ones((e, inp), np.float16)
                tensors[key + ".svh"] = np.ones((e, out), np.float16)
        eq = {"format": "exl3", "k": n / 16, "codebook": "mcg"}
        if pair_major:
            eq["tile_order"] = "pair_major"
        with open(os.path.join(root, "config.json"), "w") as f:
            json.dump({"hidden_size": hidden, "moe_intermediate_size": inter, "num_experts_per_tok": 8,
                       "expert_quant": eq}, f)
        P.write_shard(os.path.join(root, P.SINGLE_FILE), tensors, {"tile_order": "pair_major"} if pair_major else {})
        nbytes = sum(a.nbytes for a in tensors.values())
        del tensors
        dev = torch.device("cuda:0")
        del P.Pack(root).moe_layer(0, device=dev).meta  # untimed: library load and first-use set-up
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        pk = P.Pack(root)
        layer = pk.moe_layer(0, device=dev)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t0
        del layer
        t0 = time.perf_counter()
        raw = np.fromfile(os.path.join(root, P.SINGLE_FILE), dtype=np.uint8)
        torch.from_numpy(raw).to(dev)
        torch.cuda.synchronize()
        raw_secs = time.perf_counter() - t0
        return {"config": "pack_load", "tile_order": "pair_major" if pair_major else "pack", "bytes": nbytes,
                "seconds": round(secs, 3), "GBps": round(nbytes / secs / 1e9, 2),
                "raw_read_copy_GBps": round(raw.nbytes / raw_secs / 1e9, 2)}
    finally:
        shutil.rmtree(root, ignore_errors=True)


def sweep(which: str, prefill_batches=None, prefill_arms=("gemm", "windows"), c2_filter=None):
    """configs[1] (C2: MCG GEMV sweep), configs[2] (C3: prefill GEMM) and configs[4] (C5: ragged STQ MoE layer):
    one JSON line per case."""
    from sushi_amd import exl3

    cases = []
    if which in ("c2", "all"):
        for in_f, out_f in ((2048, 2048), (4096, 14336), (14336, 4096)):
            for n in (32, 48, 64):
                for rows in (1, 4, 16):
                    if c2_filter and (f"{in_f}x{out_f}", n, rows) not in c2_filter:
                        continue
                    cases.append(("c2", in_f, out_f, n, rows, exl3.MCG, "mcg"))
    if which in ("c3", "all"):
        for rows in (512, 2048):
            cases.append(("c3", 4096, 14336, 48, rows, exl3.INST3, "3inst"))
    if which in ("c5", "all"):
        print(json.dumps(bench_moe_c5()), flush=True)
        for line in bench_moe_c5_tiled():
            print(json.dumps(line), flush=True)
    if which in ("moe_prefill", "all"):
        if prefill_batches:
            bench_moe_prefill(prefill_batches, arms=prefill_arms)
        else:
            bench_moe_prefill(arms=prefill_arms)
    if which in ("moe_prefill", "c5_prefill", "all"):
        if prefill_batches:
            bench_moe_prefill_c5(prefill_batches, arms=prefill_arms)
        else:
            bench_moe_prefill_c5(arms=prefill_arms)
    if which in ("pack", "all"):
        for pm in (False, True):
            print(json.dumps(bench_pack(pm)), flush=True)
    if which in ("enc", "all"):
        for cb_name, n, w, tiles in (("mcg", 32, 12, 65536), ("mcg", 40, 15, 8192), ("mcg", 64, 16, 4096),
                                     ("mul1", 48, 15, 8192), ("mcg", 32, 16, 2048)):
            print(json.dumps(bench_encode(cb_name, n, w, tiles)), flush=True)
        for in_f, out_f, n, cb_name, w in ((2048, 768, 32, "mcg", 15), (4096, 4096, 32, "mcg", 12)):
            print(json.dumps(bench_quantize(in_f, out_f, n, cb_name, w)), flush=True)
    for cfg, in_f, out_f, n, rows, dec, name in cases:
        us, copies = _time_linear(in_f, out_f, n, rows, dec, name, 1 if cfg == "c2" else 2)
        alg = _algorithmic_bytes(in_f, out_f, n, rows)
        line = {"config": cfg, "codebook": name, "in": in_f, "out": out_f, "K": n // 16, "rows": rows,
                "us_per_call": round(us, 3), "copies": copies, "tok_per_s": round(rows / (us * 1e-6), 1),
                "effective_GBps": round(alg / (us * 1e-6) / 1e9, 1),
                "hbm_frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if cfg == "c3":
            tflops = 2.0 * rows * in_f * out_f / (us * 1e-6) / 1e12
            line["TFLOPs"] = round(tflops, 1)
            line["mfma_frac_f16_dense"] = round(tflops / MFMA_F16_PEAK_TFLOPS, 4)
            blas_us = blas_f16_gemm_us(rows, in_f, out_f)
            blas_tflops = 2.0 * rows * in_f * out_f / (blas_us * 1e-6) / 1e12
            line["blas_f16_gemm"] = {"us_per_call": round(blas_us, 3), "TFLOPs": round(blas_tflops, 1),
                                     "mfma_frac_f16_dense": round(blas_tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                     "what": "torch.matmul f16 (hipBLASLt) of the same shape on decoded weights"}
            line["frac_of_blas_f16"] = round(tflops / blas_tflops, 4)
        print(json.dumps(line), flush=True)


def _graph_layer_us(chain, dev, layers: int, rounds: int = ROUNDS) -> float:
    """Median over `rounds` graph replays of `chain` (captured once), per layer."""
    import statistics

    import torch

    chain()
    torch.cuda.synchronize()
    g = _capture(chain, dev) if SWEEP_GRAPHS else None  # --no-graph: issued from Python (counter passes)
    stream = torch.cuda.current_stream(dev)
    times = []
    for _ in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        if g is not None:
            g.replay()
        else:
            chain()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) * 1e3 / layers)
    return statistics.median(times)


def _c5_inputs(E: int, batch: int, layers: int, dev):
    """configs[4]'s per-layer inputs: each layer its own N(0,1) hidden state and top-8 routing over N(0,1) logits."""
    import torch

    from sushi_amd import exl3, synth

    xs = [synth.normal(5, f"c5.x{batch}.{layer}", (batch, 4096), device=dev) for layer in range(layers)]
    routes = []
    for layer in range(layers):
        logits = synth.normal(5, f"c5.logits{batch}.{layer}", (batch, E), dtype=torch.float32).to(dev)
        routes.append(exl3.moe_routing_chain(logits, 8))
    return xs, routes


def _c5_line(variant: str, batch: int, E: int, bpw: float, layer_us: float, alg: float, **extra):
    line = {"config": "c5", "variant": variant, "batch": batch, "experts": E, "bpw": round(bpw, 4),
            "layer_us": round(layer_us, 3), "us_per_token": round(layer_us / batch, 3), "bytes_per_layer": int(alg),
            "effective_GBps": round(alg / (layer_us * 1e-6) / 1e9, 1),
            "hbm_frac": round(alg / (layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    line.update(extra)
    return line


def bench_moe_c5(batch: int = 64, layers: int = 4):
    """configs[4] in the reference-expressible form: the per-expert rate groups of rate_groups.zig (64 experts at
    K=1, 192 at K=2: 1.75 bpw on average) as one ragged bank, hidden 4096, inter 2048, SPEC1 (spec1-w15 table: the
    one with K=1 rows), top-8 over N(0,1) logits, batch 64, plus a K=4 shared expert run as a one-expert chain whose
    output the routed call adds.  `layers` layers, each with its own input and routing, captured once; median of
    ROUNDS replays.  Bytes: the distinct experts' packed tiles and scales plus the shared expert's."""
    from sushi_amd import exl3, synth

    import torch

    dev = torch.device("cuda:0")
    E1, E2, hidden, inter = 64, 192, 4096, 2048
    dec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1)
    g1 = synth.bank(5, "c5.k1", E1, hidden, inter, 16, device=dev, norm=True)
    g2 = synth.bank(5, "c5.k2", E2, hidden, inter, 32, device=dev, norm=True)
    rb = exl3.Ragged.init([g1, g2])
    del g1, g2
    shared = synth.bank(5, "c5.shared", 1, hidden, inter, 64, device=dev, norm=True)
    xs, routes = _c5_inputs(E1 + E2, batch, layers, dev)
    sh_inds = torch.zeros(batch, 1, dtype=torch.int32, device=dev)
    sh_sc = torch.ones(batch, 1, dtype=torch.float32, device=dev)

    def chain():
        out = []
        for x, (inds, scores) in zip(xs, routes):
            s = exl3.moe(x, shared, sh_inds, sh_sc, dec)
            out.append(exl3.moe_ragged(x, rb, inds, scores, dec, shared=s))
        return out

    layer_us = _graph_layer_us(chain, dev, layers)
    # packed tiles + suh + svh of the three projections (down's in + out is gate's out + in)
    per_expert = {n: 3 * _algorithmic_bytes(hidden, inter, n, 0) for n in (16, 32)}
    distinct = [sum(per_expert[16] if e < E1 else per_expert[32] for e in set(inds.flatten().tolist()))
                for inds, _ in routes]
    alg = sum(distinct) / layers + 3 * _algorithmic_bytes(hidden, inter, 64, 0)
    return _c5_line("rate_groups", batch, E1 + E2, 1.75, layer_us, alg)


def bench_moe_c5_tiled(batch: int = 64, layers: int = 4):
    """configs[4] as stated: every expert's tiles at a seeded per-tile mix of K=1 and K=2 (25% K1; the realised rate is
    reported), 256 experts, hidden 4096, inter 2048, SPEC1 (spec1-w15), top-8 over N(0,1) logits, batch 64, plus a
    K=4 shared expert -- in the same launches (moe_tiled_with_shared_bank, "tiled_fused") and as the pair of calls
    (one-expert chain, then moe_tiled with its output, "tiled_pair").  Bytes: the distinct experts' packed tiles,
    segment tables and scales, plus the shared expert's."""
    from sushi_amd import exl3, synth

    import torch

    dev = torch.device("cuda:0")
    E, hidden, inter = 256, 4096, 2048
    dec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1)
    tb = synth.tiled_bank(5, "c5t", E, hidden, inter, 0.25, device=dev, norm=True)
    shared = synth.bank(5, "c5.shared", 1, hidden, inter, 64, device=dev, norm=True)
    xs, routes = _c5_inputs(E, batch, layers, dev)
    sh_inds = torch.zeros(batch, 1, dtype=torch.int32, device=dev)
    sh_sc = torch.ones(batch, 1, dtype=torch.float32, device=dev)
    # bytes of each expert: tile words (8 per K1 tile, 16 per K2) + 5 table bytes per segment + scales
    popc = torch.tensor([bin(v).count("1") for v in range(256)], dtype=torch.int64, device=dev)
    per_expert = torch.zeros(E, dtype=torch.int64, device=dev)
    for p in (tb.gate, tb.up, tb.down):
        segs = p.seg_k1.shape[1] * p.seg_k1.shape[2]
        k1 = popc[p.seg_k1.long()].reshape(E, -1).sum(1)
        per_expert += 4 * (128 * segs - 8 * k1) + 5 * segs + 2 * (p.in_features + p.out_features)
    per_expert = per_expert.cpu().tolist()
    words = sum(p.trellis.numel() for p in (tb.gate, tb.up, tb.down))
    bpw = words * 16 / (3 * E * hidden * inter)
    distinct = [sum(per_expert[e] for e in set(inds.flatten().tolist())) for inds, _ in routes]
    alg = sum(distinct) / layers + 3 * _algorithmic_bytes(hidden, inter, 64, 0)

    def fused():
        return [exl3.moe_tiled_with_shared_bank(x, tb, shared, inds, scores, dec) for x, (inds, scores) in
                zip(xs, routes)]

    def pair():
        out = []
        for x, (inds, scores) in zip(xs, routes):
            s = exl3.moe(x, shared, sh_inds, sh_sc, dec)
            out.append(exl3.moe_tiled(x, tb, inds, scores, dec, shared=s))
        return out

    lines = []
    for variant, fn in (("tiled_fused", fused), ("tiled_pair", pair)):
        lines.append(_c5_line(variant, batch, E, bpw, _graph_layer_us(fn, dev, layers), alg,
                              k1_fraction=0.25, distinct_experts=round(sum(len(set(i.flatten().tolist()))
                                                                           for i, _ in routes) / layers, 1)))
    return lines


def bench_moe_prefill(batches=(64, 128, 256, 512, 1024, 2048), layers: int = 4, arms=("gemm", "windows")):
    """configs[3]'s layer (E=256 + shared, hidden 2048, inter 768, K2 MCG, top-8) at prefill widths, on the routed
    GEMM arm and on the decode chain's expert windows (arm overrides): microseconds per layer and per token, each a
    median of 7 replays of `layers` layers from a HIP graph."""
    import statistics

    import torch

    from sushi_amd import exl3, synth

    dev = torch.device("cuda:0")
    E, hidden, inter, n, k = 256, 2048, 768, 32, 8
    bank = synth.bank(3, "c4", E, hidden, inter, n, device=dev, norm=True)
    shared = synth.bank(3, "c4.shared", 1, hidden, inter, n, device=dev, norm=True)
    out = []
    for batch in batches:
        xs = [synth.normal(3, f"c4.pf{batch}.{l}", (batch, hidden), device=dev) for l in range(layers)]
        routes = [exl3.moe_routing_chain(synth.normal(3, f"c4.pfl{batch}.{l}", (batch, E), dtype=torch.float32)
                                         .to(dev), k) for l in range(layers)]
        line = {"config": "c4_prefill", "batch": batch, "slots_per_expert": round(batch * k / E, 2)}
        for arm, knob in (("gemm", 1), ("windows", 0)):
            if arm not in arms:
                continue
            with exl3.arm_overrides(moe_gemm=knob):
                def chain():
                    return [exl3.moe_with_shared_bank(x, bank, shared, i, s, exl3.MCG)
                            for x, (i, s) in zip(xs, routes)]
                chain()
                torch.cuda.synchronize()
                g = _capture(chain, dev) if SWEEP_GRAPHS else None  # --no-graph: issued from Python (counter passes)
                stream = torch.cuda.current_stream(dev)
                ts = []
                for _ in range(ROUNDS):
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    if g is not None:
                        g.replay()
                    else:
                        chain()
                    e1.record(stream)
                    torch.cuda.synchronize()
                    ts.append(e0.elapsed_time(e1) * 1e3 / layers)
                us = statistics.median(ts)
                line[arm] = {"layer_us": round(us, 1), "us_per_token": round(us / batch, 3)}
                del g
        print(json.dumps(line), flush=True)
        out.append(line)
    return out


def bench_moe_prefill_c5(batches=(256, 512, 1024, 2048), layers: int = 2, arms=("gemm", "windows"),
                         forms=("ragged", "tiled")):
    """configs[4]'s layer (hidden 4096, inter 2048, 256 experts at 1.75 bpw, SPEC1 spec1-w15, top-8, plus a K=4 shared
    expert) at prefill widths, on the routed GEMM arm and on the GEMV expert windows (arm overrides), for the ragged
    rate-group bank (64 experts at K1, 192 at K2) and the per-tile K1 / K2 bank; the shared expert rides the routed
    launches where the fused form serves, else runs as the pair of calls.  Median of 7 replays of `layers` layers
    from a HIP graph."""
    import statistics

    import torch

    from sushi_amd import exl3, synth

    dev = torch.device("cuda:0")
    hidden, inter, k = 4096, 2048, 8
    dec = exl3.Decode(exl3.Codebook.spec1, exl3.Window(15), 1)
    shared = synth.bank(5, "c5.shared", 1, hidden, inter, 64, device=dev, norm=True)
    out = []
    for form in forms:
        if form == "ragged":
            g1 = synth.bank(5, "c5.k1", 64, hidden, inter, 16, device=dev, norm=True)
            g2 = synth.bank(5, "c5.k2", 192, hidden, inter, 32, device=dev, norm=True)
            bank = exl3.Ragged.init([g1, g2])
            del g1, g2
            call = lambda x, i, s: exl3.moe_ragged_with_shared_bank(x, bank, shared, i, s, dec)  # noqa: E731
        else:
            bank = synth.tiled_bank(5, "c5t", 256, hidden, inter, 0.25, device=dev, norm=True)
            call = lambda x, i, s: exl3.moe_tiled_with_shared_bank(x, bank, shared, i, s, dec)  # noqa: E731
        for batch in batches:
            xs = [synth.normal(5, f"c5.pf{batch}.{l}", (batch, hidden), device=dev) for l in range(layers)]
            routes = [exl3.moe_routing_chain(synth.normal(5, f"c5.pfl{batch}.{l}", (batch, 256), dtype=torch.float32)
                                             .to(dev), k) for l in range(layers)]
            line = {"config": "c5_prefill", "form": form, "batch": batch, "slots_per_expert": round(batch * k / 256, 2)}
            for arm, knob in (("gemm", 1), ("windows", 0)):
                if arm not in arms:
                    continue
                with exl3.arm_overrides(moe_gemm=knob):
                    chain = lambda: [call(x, i, s) for x, (i, s) in zip(xs, routes)]  # noqa: E731
                    chain()
                    torch.cuda.synchronize()
                    g = _capture(chain, dev) if SWEEP_GRAPHS else None
                    stream = torch.cuda.current_stream(dev)
                    ts = []
                    for _ in range(ROUNDS):
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record(stream)
                        if g is not None:
                            g.replay()
                        else:
                            chain()
                        e1.record(stream)
                        torch.cuda.synchronize()
                        ts.append(e0.elapsed_time(e1) * 1e3 / layers)
                    us = statistics.median(ts)
                    line[arm] = {"layer_us": round(us, 1), "us_per_token": round(us / batch, 3)}
                    del g
            if "gemm" in line and "windows" in line:
                line["windows_over_gemm"] = round(line["windows"]["layer_us"] / line["gemm"]["layer_us"], 2)
            print(json.dumps(line), flush=True)
            out.append(line)
        del bank, call
        torch.cuda.empty_cache()
    return out


def copy_calibration(mib: int, reps: int = 4):
    """A plain device-to-device copy of `mib` MiB, `reps` times: the reference kernel whose FETCH_SIZE/WRITE_SIZE
    counters calibrate the HBM-traffic figures of the GEMV (expected: exactly `mib` MiB read and written)."""
    import torch

    src = torch.empty(mib << 19, dtype=torch.float16, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def _profiled_traffic():
    """HBM bytes per GEMV launch from the committed counter summary (two rocprofv3 --pmc passes, FETCH_SIZE then
    WRITE_SIZE, scaled by the same counters read over a plain copy kernel): the sum of the last column ("bytes per
    launch") of its FETCH_SIZE and WRITE_SIZE table rows, or None if the summary or either row is absent."""
    path = os.path.join(ROOT, "profiles", "gemv_c1_3inst_k4_b1_hbm_traffic.md")
    found = {}
    try:
        with open(path) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if cells and cells[0] in ("FETCH_SIZE", "WRITE_SIZE"):
                    found[cells[0]] = int(float(cells[-1]))
    except (OSError, ValueError):
        return None
    return found["FETCH_SIZE"] + found["WRITE_SIZE"] if len(found) == 2 else None


def _cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    return model, os.cpu_count() or 1, threads


def cpu_baseline(sample_calls: int):
    """The C port of the reference's CPU path (prepareInput / innerGemv / finishOutput with the dense O(128^2)
    Hadamard, expert_exl3.zig:490-566) on the same 4096x4096 K4 3INST workload: on every host core the build may use
    (OpenMP over output tiles, the same arithmetic per element) and on one (the reference's own single-threaded
    path); each the median of 7 samples."""
    import statistics

    import numpy as np

    import oracle as O
    from sushi_amd import synth

    model, nproc, threads = _cpu_info()
    p = synth.proj(0, "cpu", 1, 4096, 4096, 64)
    x = synth.normal(0, "cpu.x", (1, 4096)).float().numpy()
    t, su, sv = (a.numpy().view(np.uint16) for a in (p.trellis, p.suh, p.svh))
    dec = O.decode(O.CB_3INST)
    alg = _algorithmic_bytes(4096, 4096, 64, 1)

    def per_call(th, calls):
        O.project_rows(x, t, su, sv, 4096, 4096, 64, dec, threads=th)
        samples = []
        for _ in range(ROUNDS):
            t0 = time.perf_counter()
            for _ in range(calls):
                O.project_rows(x, t, su, sv, 4096, 4096, 64, dec, threads=th)
            samples.append((time.perf_counter() - t0) / calls)
        return statistics.median(samples)

    one = per_call(1, max(1, sample_calls // 8))
    many = per_call(threads, sample_calls)
    return dict(value=round(alg / many / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                sample=f"median of 7 samples of {sample_calls} single-row calls of the 4096x4096 K4 3INST project "
                       f"on {threads} threads ({many * 1e3:.1f} ms per call)",
                tok_per_s=round(1.0 / many, 2), nproc=nproc, cpu_model=model,
                single_thread={"value": round(alg / one / 1e9, 3), "unit": "GB/s", "cores": 1,
                               "ms_per_call": round(one * 1e3, 1), "tok_per_s": round(1.0 / one, 2),
                               "sample": f"median of 7 samples of {max(1, sample_calls // 8)} calls"})


def cpu_moe_baseline(batch: int = 16):
    """moeSwigluHost (expert_exl3_kernels.zig:3059-3114) over configs[3]'s layer: 256 experts, hidden 2048, inter 768,
    K2 MCG, top-8 over N(0,1) logits plus the shared expert as a ninth slot of weight 1; us per token on every core
    (OpenMP over `batch` rows) and on one (a single token); median of 7 samples."""
    import statistics

    import numpy as np

    import oracle as O
    from sushi_amd import synth

    model, nproc, threads = _cpu_info()
    E, hidden, inter, k = 256, 2048, 768, 8
    b = synth.bank(3, "c4", E, hidden, inter, 32, norm=True)
    sh = synth.bank(3, "c4.shared", 1, hidden, inter, 32, norm=True)
    # the shared expert as expert E of a 257-expert bank (weight 1 in every row)
    banks = [tuple(np.concatenate([a.numpy().view(np.uint16), c.numpy().view(np.uint16)])
                   for a, c in zip((q.trellis, q.suh, q.svh), (qs.trellis, qs.suh, qs.svh)))
             for q, qs in zip((b.gate, b.up, b.down), (sh.gate, sh.up, sh.down))]
    x = synth.normal(3, f"c4.cpu{batch}", (batch, hidden)).float().numpy()
    inds, scores = O.route_topk(synth.normal(3, f"c4.cpu.logits{batch}", (batch, E), dtype=__import__("torch").float32)
                                .numpy(), k)
    slots = np.concatenate([inds, np.full((batch, 1), E, np.uint32)], axis=1)
    weights = np.concatenate([scores, np.ones((batch, 1), np.float32)], axis=1)
    dec = O.decode(O.CB_MCG)

    def per_token(th, rows):
        O.moe_swiglu_rows(x[:rows], *banks, slots[:rows], weights[:rows], hidden, inter, (32, 32, 32), dec,
                          threads=th)
        samples = []
        for _ in range(ROUNDS):
            t0 = time.perf_counter()
            O.moe_swiglu_rows(x[:rows], *banks, slots[:rows], weights[:rows], hidden, inter, (32, 32, 32), dec,
                              threads=th)
            samples.append((time.perf_counter() - t0) / rows)
        return statistics.median(samples)

    one = per_token(1, 1)
    many = per_token(threads, batch)
    return dict(value=round(many * 1e6, 1), unit="us/token", cores=threads, kind="port", nproc=nproc,
                cpu_model=model,
                sample=f"median of 7 samples of {batch} rows (8 routed experts + the shared one each) on {threads} "
                       "threads",
                single_thread={"value": round(one * 1e6, 1), "unit": "us/token", "cores": 1,
                               "sample": "median of 7 samples of one row"})


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-sample", type=int, default=40, help="calls per all-core CPU sample (0: no CPU baseline)")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-twin", action="store_true", help="skip the MCG twin of the headline GEMV")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the measured read/copy/8 MiB-launch ceilings")
    ap.add_argument("--no-graph", action="store_true", help="issue every call from Python instead of a HIP graph")
    ap.add_argument("--moe-batches", default="1,8,32", help="MoE layer batches (configs[3]); the first is headline")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device 4 times (the counter-calibration kernel)")
    ap.add_argument("--sweep", choices=("c2", "c3", "c5", "moe_prefill", "c5_prefill", "enc", "pack", "all"), help="time configs[1]/[2] cases instead (one JSON line each)")
    ap.add_argument("--prefill-batches", default="", help="moe_prefill sweep: token counts (default 64 .. 2048)")
    ap.add_argument("--prefill-arms", default="gemm,windows", help="moe_prefill sweep: arms to time")
    ap.add_argument("--c2-cases", default="", help="c2 sweep: only these cases, e.g. 2048x2048:32:1,2048x2048:32:16 "
                                                   "(shape:n:rows)")
    args = ap.parse_args()
    if args.sweep:
        global SWEEP_GRAPHS
        SWEEP_GRAPHS = not args.no_graph
        pb = tuple(int(b) for b in args.prefill_batches.split(",") if b)
        c2f = {(c.split(":")[0], int(c.split(":")[1]), int(c.split(":")[2])) for c in args.c2_cases.split(",") if c}
        sweep(args.sweep, pb or None, tuple(a for a in args.prefill_arms.split(",") if a), c2f or None)
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the multi-GPU layout is a design "
              "note (expert/output-tile sharding), not a runnable path", file=sys.stderr)
        return 2

    if args.copy_calibration > 0:
        copy_calibration(args.copy_calibration)
    lin = bench_linear(args.steps, args.warmup, not args.no_graph)
    twin = None if args.no_twin else bench_linear(args.steps, args.warmup, not args.no_graph, codebook="mcg")
    steps = lin["steps"]
    ms_per_step = lin["wall_s"] / steps * 1e3
    value = lin["bytes"] / (lin["wall_s"] / steps) / 1e9
    launch_direct_s = lin["event_ms"] / 1e3 / steps
    launch_s = lin["in_graph_ms"] / 1e3 / steps if lin["in_graph_ms"] is not None else launch_direct_s
    achieved = lin["bytes"] / launch_s / 1e9
    moe = [] if args.no_moe else [bench_moe(int(b)) for b in args.moe_batches.split(",") if b]
    ceilings = measured_ceilings(4096 * 4096 * 64 // 128) if not args.no_ceilings else None
    cpu = cpu_baseline(args.cpu_sample) if args.cpu_sample > 0 else None
    cpu_moe = cpu_moe_baseline() if args.cpu_sample > 0 and moe else None
    traffic = _profiled_traffic()
    out = {
        "metric": "effective HBM GB/s + tok/s, EXL3 K=4 4096x4096 GEMV b=1; MoE layer us/token",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded SplitMix64 codes, +-U(0.5,1.5) f16 suh/svh, N(0,1) f16 x)",
        "config": {"workload": "EXL3 dense linear 4096x4096, K=4 (n=64), 3INST codebook, 16x16 tiles, batch 1, "
                               "64 rotating weight copies", "global_batch": 1, "parallelism": "none (1 GPU)"},
        "tok_per_s": round(1.0 / (lin["wall_s"] / steps), 1),
        "timing": f"median of {lin['rounds']} rounds of exactly {steps} calls, each after an untimed replay of the "
                  "64-copy sequence (every timed call reads a copy last read 64 calls, 537 MB, earlier); value: wall "
                  "clock between synchronisations; roofline.achieved: HIP events on the launch stream, the graph of "
                  "the eviction sequence followed by the timed calls less the eviction graph alone (the timed calls "
                  "back to back inside one graph; launch_us_direct: events around the timed calls' own graph behind "
                  "the eviction graph, which adds the GPU's start of a second graph)"
                  if not args.no_graph else "clock between synchronisations; roofline.achieved: HIP events around "
                  "the calls, issued from Python behind the eviction pass",
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": "profiles/gemv_c1_3inst_k4_b1_hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE passes of bench.py, scaled by a copy kernel's counters)"
                                       if traffic else None,
                     "algorithmic_bytes": lin["bytes"], "launch_us": round(launch_s * 1e6, 3),
                     "launch_us_direct": round(launch_direct_s * 1e6, 3),
                     "measured_ceilings": ceilings},
        "cpu_baseline": cpu,
    }
    if twin:
        t_direct = twin["event_ms"] / 1e3 / twin["steps"]
        t_launch = twin["in_graph_ms"] / 1e3 / twin["steps"] if twin["in_graph_ms"] is not None else t_direct
        t_ach = twin["bytes"] / t_launch / 1e9
        out["mcg_twin"] = {
            "what": "the headline GEMV with the same codes through the reference's MCG decode (3INST, the configured "
                    "codebook, has no counterpart in the reference; MCG's arithmetic is pinned by its fixtures)",
            "value": round(twin["bytes"] / (twin["wall_s"] / twin["steps"]) / 1e9, 2), "unit": "GB/s",
            "ms_per_step": round(twin["wall_s"] / twin["steps"] * 1e3, 6),
            "roofline": {"bound": "hbm", "achieved": round(t_ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(t_ach / HBM_PEAK_GBS, 4), "launch_us": round(t_launch * 1e6, 3),
                         "launch_us_direct": round(t_direct * 1e6, 3)}}
    if ceilings:
        out["roofline"]["frac_of_measured_read"] = round(achieved / ceilings["hbm_read_GBps"], 4)
        out["roofline"]["launch_us_over_read_floor"] = round(launch_s * 1e6 / ceilings["read_small_graph_us"], 3)
    if moe:
        out["moe_layer"] = {"config": "E=256 routed + 1 shared, hidden 2048, inter 768, K2 MCG, top-8; 16 layers back "
                                      "to back on one stream from a HIP graph, each its own bank (16 x 302 MB, so "
                                      "weights come from HBM), N(0,1) input and routing (svh with 1/sqrt(in)); "
                                      "layer_us: HIP events, the 16 layers twice over in one graph less once "
                                      "(layer_us_direct: events around the one graph), median of 7 rounds",
                            "us_per_token": round(moe[0]["us_per_token"], 3),
                            "batches": [{"batch": m["batch"], "layer_us": round(m["layer_us"], 3),
                                         "layer_us_direct": round(m["layer_us_direct"], 3),
                                         "us_per_token": round(m["us_per_token"], 3),
                                         "distinct_experts": round(m["distinct"], 2),
                                         "effective_GBps": round(m["bytes"] / (m["layer_us"] * 1e-6) / 1e9, 2)}
                                        for m in moe],
                            "cpu_baseline": cpu_moe}
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
