#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

The headline line measures BASELINE config 2: ragged batched decode attention
(B=4, per-row KV lengths ~ U[256, 2048], 14 q / 2 kv heads, head_dim 64) over
24 independent per-layer caches.  One step = the 24 per-layer decode-attention
launches of one decode token, captured once into a hipGraph and replayed.
Replicated cache sets (> 256 MB, the MI355X Infinity Cache) are cycled so each
step reads its K/V from HBM.  ``value`` = algorithmic bytes (valid K/V + q +
out) per step / step time, in GB/s.

Extra keys report the long-context decode (config 3), the bandwidth-bound
decode shapes (dense and paged caches), the fused RoPE+append prefill
(config 4) and the end-to-end Qwen2.5-0.5B-shaped decode step (config 5:
dense, ragged, paged and continuous batching).  ``cpu_baseline`` times the
CPU oracle on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
MALL_BYTES = 256 << 20


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-extras", action="store_true", help="headline line only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="time budget of the attention rows of the CPU baseline (all threads; "
                        "the one-thread rows take a third more)")
    p.add_argument("--prefill-only", action="store_true",
                   help="time only the config-4 prefill leg (for kernel profiles)")
    p.add_argument("--only", choices=("cfg1", "cfg2", "cfg3", "prefill", "e2e", "floor", "valu"),
                   help="time one leg and print its JSON (for per-leg kernel profiles)")
    p.add_argument("--trace-summary", metavar="TRACE",
                   help="summarise a rocprofv3 kernel trace of one leg (kernel_trace.csv or "
                        "the rocpd results.db) as Markdown and exit (no GPU); with --leg, "
                        "--trace-steps and --trace-launches")
    p.add_argument("--leg", default="cfg2", help="leg name for --trace-summary")
    p.add_argument("--trace-steps", type=int, default=0,
                   help="timed steps of the traced leg (--trace-summary)")
    p.add_argument("--trace-launches", type=int, default=24,
                   help="hot-path dispatches per step of the traced leg (--trace-summary)")
    p.add_argument("--pmc-sample", action="store_true",
                   help="run a short fixed kernel sequence for rocprofv3 --pmc and exit")
    p.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                   help="summarise two rocprofv3 --pmc passes over --pmc-sample (FETCH_SIZE, "
                        "then WRITE_SIZE counter_collection.csv) into "
                        "profiles/decode_split_cfg2_traffic.json and exit (no GPU)")
    return p.parse_args()


class GraphStep:
    """A list of launches captured once into a hipGraph (torch.cuda.CUDAGraph)."""

    def __init__(self, fn):
        import torch

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            fn()
        torch.cuda.synchronize()

    def replay(self):
        self.graph.replay()


def _time_graphs(graphs, steps, warmup):
    """Replay graphs round-robin; return ms per replay (HIP events on the replay
    stream).  The timed replays continue the warm-up's rotation, so the first
    timed graph is the one after the last warm-up graph: with a rotation set
    larger than the MALL, no timed replay starts on data a warm-up replay has
    just left in the caches."""
    import torch

    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        graphs[(warmup + i) % len(graphs)].replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# Untimed GPU time before a matrix-core-bound leg is timed.  After the GPU has
# been idle, the prefill kernels run up to 12% slower for their first ~25 ms of
# work (S=2048: 25.7 µs per call in the first 2.3 ms, 23.0 µs from about 25 ms
# on) while the clocks ramp; the memory-bound decode legs show no such ramp
# (config 2 within 0.3% from the first 20 steps).
PREFILL_WARM_MS = 60.0


def _warm_for(graphs, ms_target):
    """Replay `graphs` round-robin, untimed, until `ms_target` of GPU time has
    passed; returns the GPU time spent (ms)."""
    import torch

    spent, i = 0.0, 0
    while spent < ms_target:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(8):
            graphs[i % len(graphs)].replay()
            i += 1
        end.record()
        end.synchronize()
        spent += start.elapsed_time(end)
    return spent


def _replay_spans(graphs, n, first):
    """Median GPU time inside one graph replay, ms: each of `n` replays
    (continuing the rotation at graph `first`) is bracketed by HIP events on
    the replay stream, so the figure excludes the gap between one replay's
    last node and the next replay's first (the per-graph launch cost, which
    ``_time_graphs`` includes) -- the counterpart of a kernel trace's span
    from a replay's first dispatch start to its last dispatch end."""
    import torch

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    for i in range(n):
        ev[i][0].record()
        graphs[(first + i) % len(graphs)].replay()
        ev[i][1].record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in ev)


def bench_ragged_decode(steps, warmup, dev):
    """Config 2: 24 per-layer decode-attention launches per step."""
    import torch

    from qwenforge_amd import ops, workloads

    layers = workloads.decode_ragged_layers(24, 4, seed=0)
    set_bytes = sum(c.key_cache.numel() * 2 * 2 for c in layers)
    replicas = max(2, -(-2 * MALL_BYTES // set_bytes))
    cap_max = max(c.key_cache.shape[2] for c in layers)
    splits, fused = ops.decode_plan(4, 2, cap_max)
    flash = ops.make_flash_scratch(4, 2, 7, cap_max, dev, splits=splits, fused=fused)
    sets = []
    for _ in range(replicas):
        sets.append([c.to(dev) for c in layers])
    kv_last = [torch.tensor([n - 1 for n in c.lengths], dtype=torch.int64, device=dev) for c in layers]
    outs = [torch.empty(4, 2, 7, 64, dtype=torch.float16, device=dev) for _ in layers]

    def step_fn(cs):
        def run():
            for i, c in enumerate(cs):
                fl = tuple(t if j != 3 else outs[i] for j, t in enumerate(flash))
                ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, c.bias, fl,
                                           kv_last=kv_last[i])
        return run

    graphs = [GraphStep(step_fn(cs)) for cs in sets]
    ms = _time_graphs(graphs, steps, warmup)
    ms_span = _replay_spans(graphs, max(len(graphs), steps), warmup + steps)
    step_bytes = sum(c.valid_bytes for c in layers)
    fused = len(flash) > 4

    # The dominant kernel alone.  With the single-launch merge the call is one
    # kernel, so the full call is that kernel; otherwise the split launch
    # (qf_decode_split) over the same 24 layers, then the combine alone.
    ms_split, ms_combine = ms, None
    if not fused:
        def split_fn(cs):
            def run():
                for i, c in enumerate(cs):
                    ops.flash_decode_split(c.grouped, c.key_cache, c.value_cache, c.bias,
                                           flash[:4], kv_last=kv_last[i])
            return run

        split_graphs = [GraphStep(split_fn(cs)) for cs in sets]
        ms_split = _time_graphs(split_graphs, steps, warmup)
        comb = GraphStep(lambda: [ops.flash_decode_combine(flash[:4]) for _ in layers])
        ms_combine = _time_graphs([comb], steps, warmup)
    return dict(ms_per_step=ms, step_bytes=step_bytes, launches=len(layers), splits=splits,
                replicas=replicas, layers=layers, fused=fused, ms_split=ms_split,
                ms_combine=ms_combine, ms_span=ms_span)


def bench_decode_cfg1(steps, warmup, dev):
    """Config 1: B=1, L=cap=512, one layer (265,728 algorithmic bytes per call).
    Caches rotated past the MALL (2 x 256 MB of distinct 256 KB caches, 64
    calls per graph) and, separately, one cache-resident layer called 64 times
    per graph."""
    import torch

    from qwenforge_amd import ops, workloads

    base = workloads.decode_uniform(1, 512, seed=0)
    per = base.key_cache.numel() * 2 * 2
    reps = -(-2 * MALL_BYTES // per)
    q = base.grouped.to(dev)
    k0, v0 = base.key_cache.to(dev), base.value_cache.to(dev)
    ks = [k0] + [k0.clone() for _ in range(reps - 1)]
    vs = [v0] + [v0.clone() for _ in range(reps - 1)]
    splits, fused = ops.decode_plan(1, 2, 512)
    flash = ops.make_flash_scratch(1, 2, 7, 512, dev, splits=splits, fused=fused)
    per_graph = 64

    def run_fn(g):
        def run():
            for j in range(per_graph):
                r = (g * per_graph + j) % reps
                ops.flash_decode_attention(q, ks[r], vs[r], None, flash)
        return run

    graphs = [GraphStep(run_fn(g)) for g in range(reps // per_graph)]
    n = max(len(graphs), steps // 4)
    ms = _time_graphs(graphs, n, max(1, warmup // 4)) / per_graph
    resident = GraphStep(lambda: [ops.flash_decode_attention(q, k0, v0, None, flash)
                                  for _ in range(per_graph)])
    ms_res = _time_graphs([resident], max(8, steps // 4), max(1, warmup // 4)) / per_graph
    name = ops.decode_kernel_name(1, 2, 7, 512, splits, len(flash) > 4, bias="none")
    return dict(us_per_layer=ms * 1e3, us_resident=ms_res * 1e3, bytes=base.valid_bytes,
                splits=splits, kernel=name, caches=reps)


def bench_long_decode(steps, warmup, dev):
    """Config 3: B=1, L=32768 with 1% of keys x8; caches rotated past the MALL."""
    import torch

    from qwenforge_amd import ops, workloads

    base = workloads.decode_uniform(1, 32768, seed=0, heavy_frac=0.01)
    per = base.key_cache.numel() * 2 * 2
    reps = max(2, -(-2 * MALL_BYTES // per))
    q = base.grouped.to(dev)
    ks = [base.key_cache.to(dev) for _ in range(reps)]
    vs = [base.value_cache.to(dev) for _ in range(reps)]
    splits, fused = ops.decode_plan(1, 2, 32768)
    flash = ops.make_flash_scratch(1, 2, 7, 32768, dev, splits=splits, fused=fused)
    per_graph = 8

    def run_fn(g):
        def run():
            for j in range(per_graph):
                r = (g * per_graph + j) % reps
                ops.flash_decode_attention(q, ks[r], vs[r], None, flash)
        return run

    graphs = [GraphStep(run_fn(g)) for g in range(max(1, reps // per_graph))]
    # Whole passes over every cache set (reps calls), at least 16 replays: the
    # first replay's launch latency is inside the timed region, and over few
    # replays it shows (config 3 at 4 replays read 10.09 us against 9.6).
    n = len(graphs) * max(1, -(-max(16, steps // 8) // len(graphs)))
    ms = _time_graphs(graphs, n, max(1, warmup // 8)) / per_graph
    return dict(us_per_layer=ms * 1e3, bytes=base.valid_bytes, splits=splits, calls=n * per_graph,
                caches=reps, fused=len(flash) > 4)


def bench_bandwidth_decode(steps, warmup, dev, batch, length):
    """Decode attention where K/V streaming dominates (the >= 60%-of-HBM regime,
    KV length >= 4096): B x L slots per kv head, no bias, caches rotated so the
    set is at least twice the MALL.  Returns the full call (split + merge)
    and the split kernel alone, per layer."""
    import torch

    from qwenforge_amd import ops, workloads

    base = workloads.decode_uniform(batch, length, seed=1)
    per = base.key_cache.numel() * 2 * 2
    reps = max(2, -(-2 * MALL_BYTES // per))
    q = base.grouped.to(dev)
    k0, v0 = base.key_cache.to(dev), base.value_cache.to(dev)
    ks = [k0] + [k0.clone() for _ in range(reps - 1)]
    vs = [v0] + [v0.clone() for _ in range(reps - 1)]
    splits, fused = ops.decode_plan(batch, 2, length)
    flash = ops.make_flash_scratch(batch, 2, 7, length, dev, splits=splits, fused=fused)

    def full():
        for r in range(reps):
            ops.flash_decode_attention(q, ks[r], vs[r], None, flash)

    def split_only():
        for r in range(reps):
            ops.flash_decode_split(q, ks[r], vs[r], None, flash[:4])

    ms_full = _time_graphs([GraphStep(full)], max(16, steps // 4), max(1, warmup // 4)) / reps
    ms_split = _time_graphs([GraphStep(split_only)], max(16, steps // 4), max(1, warmup // 4)) / reps
    nbytes = base.valid_bytes
    return dict(batch=batch, length=length, splits=splits, fused=len(flash) > 4,
                us_full=ms_full * 1e3, us_split=ms_split * 1e3, bytes=nbytes)


def _to_pages(dense, page, perm):
    """(B, KVH, cap, D) cache -> (B*cap/page, KVH, page, D) pool whose page
    b*ppr + j holds logical page j of row b at physical index perm[b*ppr + j]."""
    b, kvh, cap, d = dense.shape
    ppr = cap // page
    pages = dense.view(b, kvh, ppr, page, d).permute(0, 2, 1, 3, 4).reshape(b * ppr, kvh, page, d)
    pool = dense.new_empty(pages.shape)
    pool[perm] = pages
    return pool


def bench_paged_decode(steps, warmup, dev, batch, length, page=64):
    """The bandwidth-regime decode over a paged cache: the same K/V as
    ``bench_bandwidth_decode`` cut into 64-slot pages placed by a random
    permutation, read through the block table."""
    import torch

    from qwenforge_amd import ops, paged, workloads

    base = workloads.decode_uniform(batch, length, seed=1)
    per = base.key_cache.numel() * 2 * 2
    reps = max(2, -(-2 * MALL_BYTES // per))
    q = base.grouped.to(dev)
    ppr = length // page
    perm = torch.randperm(batch * ppr, generator=torch.Generator().manual_seed(0)).to(dev)
    table = perm.view(batch, ppr).to(torch.int32)
    k0, v0 = base.key_cache.to(dev), base.value_cache.to(dev)
    kp = [_to_pages(k0, page, perm)] + [None] * (reps - 1)
    vp = [_to_pages(v0, page, perm)] + [None] * (reps - 1)
    for r in range(1, reps):
        kp[r], vp[r] = kp[0].clone(), vp[0].clone()
    del k0, v0
    splits, fused = ops.decode_plan(batch, 2, length)
    flash = ops.make_flash_scratch(batch, 2, 7, length, dev, splits=splits, fused=fused)

    def full():
        for r in range(reps):
            paged.flash_decode_attention_paged(q, kp[r], vp[r], table, None, flash)

    def split_only():
        for r in range(reps):
            paged.flash_decode_split_paged(q, kp[r], vp[r], table, None, flash[:4])

    ms_full = _time_graphs([GraphStep(full)], max(16, steps // 4), max(1, warmup // 4)) / reps
    ms_split = _time_graphs([GraphStep(split_only)], max(16, steps // 4), max(1, warmup // 4)) / reps
    return dict(batch=batch, length=length, splits=splits, page=page,
                us_full=ms_full * 1e3, us_split=ms_split * 1e3, bytes=base.valid_bytes)


def bench_paged_e2e(dev, new_tokens=128):
    """Config-5 model over a paged cache: the ragged batch of ``bench_e2e``
    through ``generate_paged`` (each row holds only its own pages, no holes),
    and continuous batching of 16 requests through 4 rows (``serve``)."""
    import torch

    from qwenforge_amd.model import Qwen2Config, init_weights
    from qwenforge_amd.paged_engine import PagedDecodeEngine

    cfg = Qwen2Config()
    eng = PagedDecodeEngine(cfg, init_weights(cfg, dev, seed=0), dev)
    lengths = (512, 700, 896, 1024)
    gen = torch.Generator().manual_seed(7)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in lengths]
    eng.generate_paged(prompts, 8)
    timing = {}
    eng.generate_paged(prompts, new_tokens, timing=timing)
    steps = new_tokens - 1
    out = {"ragged_bs4": {
        "lengths": list(lengths),
        "decode_tok_s": round(len(lengths) * steps / (timing["decode_ms"] * 1e-3), 1),
        "ms_per_step": round(timing["decode_ms"] / steps, 4),
        "prefill_ms": round(timing["prefill_ms"], 3),
        "pages": timing["pages"],
    }}
    gen = torch.Generator().manual_seed(8)
    n_req = 16
    req_len = torch.randint(128, 1025, (n_req,), generator=gen).tolist()
    req_new = torch.randint(16, 129, (n_req,), generator=gen).tolist()
    reqs = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in req_len]
    eng.serve(reqs[:4], 4, max_batch=4)
    torch.cuda.synchronize(dev)
    stats = {}
    t0 = time.perf_counter()
    res = eng.serve(reqs, req_new, max_batch=4, stats=stats)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    n_tok = sum(int(x.numel()) for x in res)
    out["serve"] = {
        "requests": n_req, "max_batch": 4, "tokens": n_tok, "replays": stats["replays"],
        "tok_s": round(n_tok / wall, 1), "wall_ms": round(wall * 1e3, 1),
        "what": "16 requests (prompt 128-1024, 16-128 new tokens) through 4 rows, per-request "
                "prefill on admission, wall clock including prefills and host scheduling",
    }
    return out


def hbm_copy_ceiling(dev, mib=512, reps=20):
    """Practical HBM rate on this box: a plain device copy of `mib` MiB
    (torch.Tensor.copy_), counted as read + write bytes per second."""
    import torch

    src = torch.empty(mib << 19, device=dev, dtype=torch.float16)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    return 2 * src.numel() * 2 / (ms * 1e-3) / 1e9


def hbm_read_ceiling(dev, sizes_mib=(16, 256), workgroups=(512, 1024, 2048, 4096)):
    """Read-only HBM rate (qf_stream_read: 16-byte loads, grid-stride) at the
    config-3 size and the bandwidth-regime size, over buffers rotated past the
    MALL (at least 512 MiB per pass), best over a few workgroup counts."""
    import torch

    from qwenforge_amd import _lib

    lib = _lib.load()
    sink = torch.zeros(4 * max(workgroups), device=dev, dtype=torch.int32)
    out = {}
    for mib in sizes_mib:
        nbuf = max(2, -(-512 // mib))
        bufs = [torch.empty(mib << 18, device=dev, dtype=torch.int32).fill_(i) for i in range(nbuf)]
        best = None
        for wg in workgroups:
            def run(wg=wg):
                for b in bufs:
                    _lib.check(lib.qf_stream_read(b.data_ptr(), mib << 20, sink.data_ptr(), wg,
                                                  torch.cuda.current_stream().cuda_stream),
                               "qf_stream_read")
            ms = _time_graphs([GraphStep(run)], 10, 2) / nbuf
            gbs = (mib << 20) / (ms * 1e-3) / 1e9
            if best is None or gbs > best[0]:
                best = (gbs, wg, ms)
        out[f"{mib}MiB"] = {"GBps": round(best[0], 1), "us": round(best[2] * 1e3, 2),
                            "workgroups": best[1], "frac_of_peak": round(best[0] / HBM_PEAK_GBS, 4)}
        del bufs
        torch.cuda.empty_cache()
    out["what"] = ("qf_stream_read (include/qf_probe.h): read-only 16-byte loads, "
                   f"{nbuf}+ buffers rotated per graph so reads miss the MALL; best of "
                   f"{list(workgroups)} workgroups")
    return out


def launch_floor(dev, shapes=((128, 512, "config 2: 16 splits x 8 (b, kv head), 8 waves"),
                               (256, 256, "config 3: 128 splits x 2 kv heads, 4 waves")),
                 per_graph=24, steps=40, warmup=4):
    """What a decode launch of a given shape cannot go under: graph-replayed
    qf_launch_probe kernels (include/qf_probe.h) of the decode launch's grid,
    24 nodes per graph as in a config-2 step -- an empty kernel (the cost of
    a graph node), one dependent HBM round trip (every thread loads 16 bytes
    of a region no earlier launch in the rotation touched) and two (a device
    index read first, as a decode split reads kv_last before its first tile).
    Per-launch microseconds."""
    import torch

    from qwenforge_amd import _lib

    lib = _lib.load()
    out = {}
    pool = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    index = torch.zeros(1, dtype=torch.int64, device=dev)
    for wg, threads, what in shapes:
        region = wg * threads * 16
        n_regions = pool.numel() // region
        sink = torch.zeros(wg * threads // 64, dtype=torch.int32, device=dev)
        row = {"workgroups": wg, "threads": threads, "what": what}
        for trips, key in ((0, "empty_us"), (1, "one_round_trip_us"), (2, "two_round_trips_us")):
            def run(g, trips=trips):
                def body():
                    for j in range(per_graph):
                        r = (g * per_graph + j) % n_regions
                        _lib.check(lib.qf_launch_probe(pool.data_ptr() + r * region, region,
                                                       index.data_ptr(), sink.data_ptr(), wg,
                                                       threads, trips,
                                                       torch.cuda.current_stream().cuda_stream),
                                   "qf_launch_probe")
                return body
            graphs = [GraphStep(run(g)) for g in range(max(1, n_regions // per_graph))]
            n = len(graphs) * max(1, -(-steps // len(graphs)))
            row[key] = round(_time_graphs(graphs, n, warmup) / per_graph * 1e3, 3)
        out[f"{wg}x{threads}"] = row
    del pool
    torch.cuda.empty_cache()
    return out


def bench_valu_vs_mfma(steps, warmup, dev):
    """The decode split launch as GQA-packed MFMA tiles (qf_decode_split, the
    product) against VALU dot products (qf_decode_split_valu, a comparison
    kernel) at the same split count, on the same caches rotated past the MALL,
    no bias: config 1 (B=1 L=512), config 2 (B=4 ragged, kv_last per row),
    config 3 (B=1 L=32768, 1% keys x8) and B=16 L=32768 (bandwidth regime).
    Split kernel alone (graph-replayed), per call; both partial sets merge to
    within 2e-3 of each other through the combine launch (tests cover the
    oracle)."""
    import torch

    from qwenforge_amd import _lib, ops, workloads

    lib = _lib.load()
    shapes = (("config1", workloads.decode_uniform(1, 512, seed=0), 16),
              ("config2", workloads.decode_ragged(4, seed=0), 32),
              ("config3", workloads.decode_uniform(1, 32768, seed=0, heavy_frac=0.01), 128),
              ("B16_L32768", workloads.decode_uniform(16, 32768, seed=1), 8))
    out = {}
    for name, base, splits in shapes:
        b = base.grouped.shape[0]
        cap = base.key_cache.shape[2]
        per = base.key_cache.numel() * 2 * 2
        reps = max(2, -(-2 * MALL_BYTES // per))
        q = base.grouped.to(dev)
        k0, v0 = base.key_cache.to(dev), base.value_cache.to(dev)
        ks = [k0] + [k0.clone() for _ in range(reps - 1)]
        vs = [v0] + [v0.clone() for _ in range(reps - 1)]
        kv_last = torch.tensor([n - 1 for n in base.lengths], dtype=torch.int64, device=dev)
        flash = ops.make_flash_scratch(b, 2, 7, cap, dev, splits=splits, fused=False)
        acc, m, l = flash[:3]

        def call(fn, r):
            st = torch.cuda.current_stream().cuda_stream
            common = (q.data_ptr(), *q.stride()[:3], ks[r].data_ptr(), *ks[r].stride()[:3],
                      vs[r].data_ptr(), *vs[r].stride()[:3])
            if fn == "mfma":
                rc = lib.qf_decode_split(*common, None, 0, kv_last.data_ptr(), 1, acc.data_ptr(),
                                         m.data_ptr(), l.data_ptr(), splits, b, 2, 7, 64, cap,
                                         0.125, st)
            else:
                rc = lib.qf_decode_split_valu(*common, kv_last.data_ptr(), 1, acc.data_ptr(),
                                              m.data_ptr(), l.data_ptr(), splits, b, 2, 7, 64,
                                              cap, 0.125, st)
            _lib.check(rc, fn)

        row = {"splits": splits, "bytes": base.valid_bytes, "caches": reps}
        outs = {}
        for fn in ("mfma", "valu"):
            call(fn, 0)
            outs[fn] = ops.flash_decode_combine(flash).clone()
            g = GraphStep(lambda fn=fn: [call(fn, r) for r in range(reps)])
            us = _time_graphs([g], max(16, steps // 10), max(1, warmup // 10)) / reps * 1e3
            row[f"{fn}_split_us"] = round(us, 3)
            row[f"{fn}_GBps"] = round(base.valid_bytes / (us * 1e-6) / 1e9, 1)
        torch.cuda.synchronize()
        row["valu_over_mfma"] = round(row["valu_split_us"] / row["mfma_split_us"], 3)
        row["max_abs_diff"] = float((outs["mfma"].float() - outs["valu"].float()).abs().max())
        out[name] = row
        del ks, vs
        torch.cuda.empty_cache()
    return out


def _trace_dispatches(path):
    """(kernel name, grid in workgroups, start ns, end ns) of every dispatch in
    a rocprofv3 kernel trace: the CSV of ``--output-format csv`` or the rocpd
    database rocprofv3 writes by default."""
    out = []
    if path.endswith(".db"):
        import sqlite3

        con = sqlite3.connect(path)
        q = "select name, grid_x, workgroup_x, grid_y, grid_z, start, end from kernels"
        for name, gx, wx, gy, gz, st, en in con.execute(q):
            out.append((name, (int(gx) // max(1, int(wx)), int(gy), int(gz)), int(st), int(en)))
        con.close()
    else:
        import csv

        for r in csv.DictReader(open(path)):
            grid = (int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])),
                    int(r["Grid_Size_Y"]), int(r["Grid_Size_Z"]))
            out.append((r["Kernel_Name"], grid, int(r["Start_Timestamp"]),
                        int(r["End_Timestamp"])))
    return [(n.split("(")[0].replace("void ", "").strip(), g, st, en) for n, g, st, en in out]


def trace_summary(path, leg, steps, launches, hot=("decode_", "prefill", "rope_kv"),
                  gap_us=5.0):
    """Per-kernel and per-step figures of one bench leg from a rocprofv3
    kernel trace (``--kernel-trace``), as Markdown.

    The leg's hot-path dispatches (kernel names containing one of ``hot``)
    are cut into replays wherever one starts more than ``gap_us`` after the
    previous one ends; the timed region is the last ``steps`` replays of
    exactly ``launches`` dispatches (the eager warm-up calls and the earlier
    replays come before it).  Reported over the timed region: per kernel the
    dispatch count and mean / median duration; per replay the span (first
    start to last end) and that span per launch, the trace's counterpart of
    the bench's HIP-event time per launch (which also holds the gaps between
    replays, where the profiler slows the host's graph submission)."""
    ds = sorted(_trace_dispatches(path), key=lambda d: d[2])
    lines = [f"Kernel trace `{os.path.basename(path)}`, leg `{leg}`.", ""]
    hot_d = [d for d in ds if any(h in d[0] for h in hot)]
    groups, cur = [], []
    for d in hot_d:
        if cur and (d[2] - cur[-1][3]) / 1e3 > gap_us:
            groups.append(cur)
            cur = []
        cur.append(d)
    if cur:
        groups.append(cur)
    full = [g for g in groups if len(g) == launches]
    timed = full[-steps:] if steps > 0 else full
    lines.append(f"{len(hot_d)} hot-path dispatches in {len(groups)} bursts; {len(full)} bursts of "
                 f"exactly {launches} (one replay); the timed region is the last {len(timed)}.")
    if timed:
        per = {}
        for g in timed:
            for name, grid, st, en in g:
                per.setdefault((name, grid), []).append((en - st) / 1e3)
        lines += ["", "| kernel (timed region) | grid (workgroups) | dispatches | mean µs | "
                      "median µs |", "|---|---|---:|---:|---:|"]
        for (name, grid), durs in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"| `{name}` | {grid[0]}x{grid[1]}x{grid[2]} | {len(durs)} | "
                         f"{statistics.mean(durs):.3f} | {statistics.median(durs):.3f} |")
        spans = [(max(d[3] for d in g) - g[0][2]) / 1e3 for g in timed]
        busy = [sum(d[3] - d[2] for d in g) / 1e3 for g in timed]
        lines += ["", "| per replay (timed region) | µs |", "|---|---:|",
                  f"| span, median (first start to last end) | {statistics.median(spans):.3f} |",
                  f"| span / {launches} launches | {statistics.median(spans) / launches:.3f} |",
                  f"| sum of kernel durations, median | {statistics.median(busy):.3f} |"]
    alln = {}
    for name, grid, st, en in ds:
        alln.setdefault((name, grid), []).append((en - st) / 1e3)
    lines += ["", "| kernel (whole run) | grid (workgroups) | dispatches | mean µs | median µs |",
              "|---|---|---:|---:|---:|"]
    for (name, grid), durs in sorted(alln.items(), key=lambda kv: -sum(kv[1]))[:25]:
        lines.append(f"| `{name}` | {grid[0]}x{grid[1]}x{grid[2]} | {len(durs)} | "
                     f"{statistics.mean(durs):.3f} | {statistics.median(durs):.3f} |")
    return "\n".join(lines)


def bench_prefill(steps, warmup, dev, seq=2048):
    """Config 4: causal prefill S=2048 with fused RoPE + cache append (other
    lengths for the long-prompt leg)."""
    import torch

    from qwenforge_amd import ops, workloads

    case = workloads.prefill_case(seq, seed=0)
    c = case.to(dev)
    kc = torch.zeros(1, 2, seq, 64, dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    per_graph = 8

    def run():
        for _ in range(per_graph):
            ops.gqa_flash_prefill_rope_append(c.query, c.key, c.value, c.cos, c.sin, kc, vc, 0)

    g = GraphStep(run)
    warm_ms = _warm_for([g], PREFILL_WARM_MS)
    ms = _time_graphs([g], max(12, steps // 8), max(1, warmup // 8)) / per_graph
    return dict(us_per_layer=ms * 1e3, flops=case.flops, warm_ms=warm_ms)


def bench_e2e(dev, batches=(1, 4), prefix=1024, new_tokens=128):
    """Config 5: Qwen2.5-0.5B-shaped greedy decode, random-init fp16 weights,
    the HIP RoPE/append/attention kernels inside a hipGraph-captured step."""
    import torch

    from qwenforge_amd.engine import DecodeEngine
    from qwenforge_amd.model import Qwen2Config, init_weights

    cfg = Qwen2Config()
    eng = DecodeEngine(cfg, init_weights(cfg, dev, seed=0), dev)
    out = {}
    for b in batches:
        ids = torch.randint(0, cfg.vocab, (b, prefix), generator=torch.Generator().manual_seed(b)).to(dev)
        eng.generate(ids, 8)                      # warm-up (allocator, hipBLASLt plans)
        timing = {}
        eng.generate(ids, new_tokens, timing)
        steps = new_tokens - 1
        out[b] = {
            "decode_tok_s": round(b * steps / (timing["decode_ms"] * 1e-3), 1),
            "ms_per_step": round(timing["decode_ms"] / steps, 4),
            "prefill_ms": round(timing["prefill_ms"], 3),
            "weight_GBps": round(cfg.weight_bytes() / (timing["decode_ms"] / steps * 1e-3) / 1e9, 1),
        }
        del ids
    # Ragged batch (the reference's padded-batch path, SE:1241-1335): four
    # prompts of different lengths, packed prefill, decode over masked holes.
    lengths = (512, 700, 896, 1024)
    gen = torch.Generator().manual_seed(7)
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=gen).to(dev) for n in lengths]
    eng.generate_ragged(prompts, 8)
    timing = {}
    eng.generate_ragged(prompts, new_tokens, timing)
    steps = new_tokens - 1
    out["ragged"] = {
        "lengths": list(lengths),
        "decode_tok_s": round(len(lengths) * steps / (timing["decode_ms"] * 1e-3), 1),
        "ms_per_step": round(timing["decode_ms"] / steps, 4),
        "prefill_ms": round(timing["prefill_ms"], 3),
    }
    return out


def pmc_sample(dev):
    """A short fixed sequence for ``rocprofv3 --pmc`` passes (no timing):
    a plain 64 MiB device copy (calibrates FETCH_SIZE / WRITE_SIZE against a
    known byte count), then one config-2 step: 24 decode-attention calls with
    the headline's split count and merge (single launch per call)."""
    import torch

    from qwenforge_amd import ops, workloads

    src = torch.randn(32 << 20, device=dev, dtype=torch.float16)   # 64 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    layers = [c.to(dev) for c in workloads.decode_ragged_layers(24, 4, seed=0)]
    cap_max = max(c.key_cache.shape[2] for c in layers)
    splits, fused = ops.decode_plan(4, 2, cap_max)
    flash = ops.make_flash_scratch(4, 2, 7, cap_max, dev, splits=splits, fused=fused)
    for c in layers:
        kv_last = torch.tensor([n - 1 for n in c.lengths], dtype=torch.int64, device=dev)
        ops.flash_decode_attention(c.grouped, c.key_cache, c.value_cache, c.bias, flash,
                                   kv_last=kv_last)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_sample": "done", "copy_bytes": 2 * src.numel() * 2,
                      "split_launches": len(layers),
                      "split_bytes_mean": sum(c.valid_bytes for c in layers) / len(layers)}))


def traffic_summary(fetch_csv, write_csv):
    """HBM bytes per launch of the headline kernel from two PMC passes over
    ``--pmc-sample``: the 64 MiB device copies calibrate each counter (bytes
    known to be read / written per copy), then the mean per-dispatch value of
    the decode kernel is scaled by that factor.  Writes the JSON the bench
    line's ``roofline.traffic`` reads, stamped with the kernel source hash and
    instance so that a later kernel change makes the figure stale (null)."""
    import csv
    import subprocess

    from qwenforge_amd import ops, workloads

    layers = workloads.decode_ragged_layers(24, 4, seed=0)
    cap_max = max(c.key_cache.shape[2] for c in layers)
    splits, fused = ops.decode_plan(4, 2, cap_max)
    kernel = ops.decode_kernel_name(4, 2, 7, cap_max, splits, fused)
    copy_bytes = 64 << 20

    def read(path, counter):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        copies = [r for r in rows if r["Kernel_Name"].startswith("__amd_rocclr_copyBuffer")]
        big = max(int(r["Grid_Size"]) for r in copies)
        cal = [float(r["Counter_Value"]) for r in copies if int(r["Grid_Size"]) == big]
        ker = [float(r["Counter_Value"]) for r in rows
               if r["Kernel_Name"].split("(")[0].replace("void ", "").strip() == kernel]
        if len(cal) < 1 or len(ker) != len(layers):
            raise SystemExit(f"{path}: {len(cal)} calibration copies, {len(ker)} dispatches of "
                             f"{kernel} (expected {len(layers)})")
        return statistics.mean(cal), statistics.mean(ker)

    f_cal, f_ker = read(fetch_csv, "FETCH_SIZE")
    w_cal, w_ker = read(write_csv, "WRITE_SIZE")
    f_fac, w_fac = copy_bytes / 1024 / f_cal, copy_bytes / 1024 / w_cal
    fetch_b, write_b = f_ker * 1024 * f_fac, w_ker * 1024 * w_fac
    try:
        commit = subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], cwd=ROOT,
                                capture_output=True, text=True).stdout.strip() or None
    except OSError:
        commit = None
    rec = {
        "kernel": kernel,
        "workload": f"config 2 (B=4 ragged, 24 layers, {splits} splits), one launch per layer",
        "source_sha16": _kernel_source_hash(),
        "commit": commit,
        "fetch_kib_per_launch": round(f_ker, 2),
        "write_kib_per_launch": round(w_ker, 2),
        "copy_calibration": {"bytes_read": copy_bytes, "bytes_written": copy_bytes,
                             "FETCH_SIZE_kib": round(f_cal, 2), "WRITE_SIZE_kib": round(w_cal, 2),
                             "fetch_factor": round(f_fac, 5), "write_factor": round(w_fac, 5)},
        "algorithmic_bytes_per_launch": int(sum(c.valid_bytes for c in layers) / len(layers)),
        "fetch_bytes_per_launch": int(fetch_b),
        "write_bytes_per_launch": int(write_b),
        "traffic_bytes_per_launch": int(fetch_b + write_b),
    }
    path = os.path.join(ROOT, "profiles", "decode_split_cfg2_traffic.json")
    with open(path, "w") as f:
        json.dump(rec, f, indent=1)
        f.write("\n")
    print(json.dumps(rec))


def _kernel_source_hash():
    """sha256 prefix of the decode kernel's source and build: decode_attn.hip,
    decode_attn_fused_vec.hip (the headline instances' unit), qf_common.h and
    the compiler flags ``qwenforge_amd.build`` gives those two units."""
    import hashlib

    from qwenforge_amd import build

    h = hashlib.sha256()
    for rel in ("decode_attn.hip", "decode_attn_fused_vec.hip", "qf_common.h"):
        with open(os.path.join(ROOT, "qwenforge_amd", "csrc", rel), "rb") as f:
            h.update(f.read())
    flags = [build.COMMON_FLAGS[:-1], build.DEVICE_FLAGS,
             build.UNIT_FLAGS.get("decode_attn.hip", []),
             build.UNIT_FLAGS.get("decode_attn_fused_vec.hip", [])]
    h.update(repr(flags).encode())
    return h.hexdigest()[:16]


def _traffic(kernel):
    """HBM bytes per launch of the headline's dominant kernel, measured with
    rocprofv3 counters (profiles/decode_split_cfg2_traffic.json), with the
    source hash and kernel instance the passes ran.  None when the kernel
    source or instance has changed since (the figure would be stale)."""
    path = os.path.join(ROOT, "profiles", "decode_split_cfg2_traffic.json")
    if not os.path.exists(path):
        return None, "no counter passes recorded"
    with open(path) as f:
        rec = json.load(f)
    if rec.get("source_sha16") != _kernel_source_hash():
        return None, "stale: the decode kernel source changed after the counter passes"
    if rec.get("kernel") != kernel:
        return None, f"stale: the counter passes ran {rec.get('kernel')}"
    return rec.get("traffic_bytes_per_launch"), (
        f"rocprofv3 FETCH_SIZE + WRITE_SIZE passes at commit {rec.get('commit', '?')}, "
        f"source {rec['source_sha16']}")


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name plus family / model /
    stepping (a virtualised host may report a generic model name)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if info:
                        break
                    continue
                k, v = (x.strip() for x in line.split(":", 1))
                if k in ("vendor_id", "model name", "cpu family", "model", "stepping",
                         "cpu MHz", "cache size") and k not in info:
                    info[k] = v
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    return (f"{name} (vendor {info.get('vendor_id', '?')}, family {info.get('cpu family', '?')}, "
            f"model {info.get('model', '?')}, stepping {info.get('stepping', '?')}, "
            f"{info.get('cpu MHz', '?')} MHz, cache {info.get('cache size', '?')}, "
            f"{os.cpu_count()} logical CPUs)")


def _time_oracle(layers, seconds, threads, form="fp32"):
    """Decode-attention layer calls of the CPU oracle for about `seconds` at
    `threads` threads (3 warm-up calls first, at least 20 timed calls);
    `form` is "fp32" (the fp32-accumulated oracle) or "fp16" (the reference's
    own fp16 form, SE:968-971).  Returns (GB/s, calls, median s, total s)."""
    import torch

    import oracle

    fn = (oracle.grouped_decode_attention if form == "fp32"
          else oracle.grouped_decode_attention_fp16)
    torch.set_num_threads(threads)
    for c in layers[:3]:
        fn(c.grouped, c.key_cache, c.value_cache, c.bias)
    t_end = time.perf_counter() + seconds
    done_bytes, n_layers, times = 0, 0, []
    while time.perf_counter() < t_end or n_layers < 20:
        c = layers[n_layers % len(layers)]
        t0 = time.perf_counter()
        fn(c.grouped, c.key_cache, c.value_cache, c.bias)
        times.append(time.perf_counter() - t0)
        done_bytes += c.valid_bytes
        n_layers += 1
    total = sum(times)
    return done_bytes / total / 1e9, n_layers, statistics.median(times), total


def _cpu_row(layers, seconds, threads, form, what):
    gbs, n, med, total = _time_oracle(layers, seconds, threads, form)
    gbs1, n1, med1, total1 = _time_oracle(layers, seconds / 3, 1, form)
    return {
        "GBps": round(gbs, 3), "us_per_layer": round(med * 1e6, 1), "threads": threads,
        "sample": f"{n} {what} layer calls ({form}), median {med * 1e6:.0f} us/layer, "
                  f"{total:.1f} s total",
        "single_thread": {"GBps": round(gbs1, 3), "us_per_layer": round(med1 * 1e6, 1),
                          "sample": f"{n1} calls, {total1:.1f} s"},
    }


def _cpu_decode_step(threads, reps=20, warm=3):
    """Config 5 on the CPU: the fp32 oracle's decode step (SE:876-982,
    oracle.model.decode_step) of the full Qwen2.5-0.5B shape at B=1 and B=4
    over 1152-slot caches with 1024 valid slots.  The cache holds random
    values (the step's work does not depend on them), so no CPU prefill runs;
    weights are upcast to fp32 once, outside the timed region."""
    import torch

    import oracle.model as om
    from qwenforge_amd.model import Qwen2Config, init_weights

    torch.set_num_threads(threads)
    cfg = Qwen2Config()
    w16 = init_weights(cfg, "cpu", seed=0)
    embed = w16["embed"].float()
    w = {"embed": embed, "final_norm": w16["final_norm"].float(), "lm_head": embed,
         "layers": [{k: v.float() for k, v in layer.items()} for layer in w16["layers"]]}
    del w16
    out = {}
    gen = torch.Generator().manual_seed(0)
    state = {}
    for b in (1, 4):
        caches = [(torch.randn(b, 2, 1152, 64, generator=gen),
                   torch.randn(b, 2, 1152, 64, generator=gen)) for _ in range(cfg.layers)]
        state[b] = (caches, torch.randint(0, cfg.vocab, (b,), generator=gen))
    # Warm-up steps at both batch sizes first (thread pool, first touch of the
    # fp32 weights), then the timed steps, alternating the batch sizes.  The
    # steps write cache slots 1024 .. 1024 + warm + reps - 1 (< 1152).
    for i in range(warm):
        for b in (1, 4):
            caches, tok = state[b]
            om.decode_step(w, cfg, tok, torch.full((b,), 1024 + i), caches, 1024 + i)
    times = {1: [], 4: []}
    for i in range(reps):
        for b in (1, 4):
            caches, tok = state[b]
            p = 1024 + warm + i
            t0 = time.perf_counter()
            om.decode_step(w, cfg, tok, torch.full((b,), p), caches, p)
            times[b].append(time.perf_counter() - t0)
    for b in (1, 4):
        med = statistics.median(times[b])
        out[f"tok_s_bs{b}"] = round(b / med, 2)
        out[f"ms_per_step_bs{b}"] = round(med * 1e3, 1)
    out["threads"] = threads
    out["sample"] = (f"median of {reps} timed steps per batch after {warm} warm-up steps at each, "
                     "fp32 oracle decode step, 24 layers + lm_head, 1024+ valid cache slots")
    return out


def _cpu_prefill(threads, reps, warm, seq=2048, reps16=None, warm16=None):
    """Config 4 on the CPU (RoPE theta=1e6 + causal prefill + cache append,
    B=1, S=2048, 14q/2kv, hd64), in the fp32 oracle form (oracle.apply_rope_fp16
    + oracle.causal_prefill + oracle.append_prefill) and in the reference's
    own fp16 eager form (the same RoPE and append around
    oracle.eager_attention_fp16, SE:579-599).  Median of `reps` calls after
    `warm` warm-ups, at `threads` threads; the fp16 form, whose fp16 matrix
    products run far slower on a CPU, takes `reps16` / `warm16` (default the
    same) so the baseline stays a bounded sample."""
    import torch

    import oracle
    from qwenforge_amd import workloads

    torch.set_num_threads(threads)
    case = workloads.prefill_case(seq, seed=0)
    kc = torch.zeros(1, 2, seq, 64, dtype=torch.float16)
    vc = torch.zeros_like(kc)

    def fp32():
        q = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
        k = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
        oracle.append_prefill(kc, vc, k, case.value)
        return oracle.causal_prefill(q, k, case.value)

    def fp16():
        q = oracle.apply_rope_fp16(case.query, case.cos, case.sin)
        k = oracle.apply_rope_fp16(case.key, case.cos, case.sin)
        oracle.append_prefill(kc, vc, k, case.value)
        return oracle.eager_attention_fp16(q, k, case.value)

    out = {}
    plan = (("fp32_oracle", fp32, reps, warm),
            ("fp16_reference_form", fp16, reps if reps16 is None else reps16,
             warm if warm16 is None else warm16))
    for name, fn, n_rep, n_warm in plan:
        if n_rep < 1:
            continue
        for _ in range(n_warm):
            fn()
        times = []
        for _ in range(n_rep):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        out[name] = {"us_per_call": round(med * 1e6, 1),
                     "TFLOPs": round(case.flops / med / 1e12, 4),
                     "sample": f"median of {n_rep} calls after {n_warm} warm-ups, "
                               f"{sum(times):.1f} s timed"}
    out["threads"] = threads
    return out



def cpu_baseline(layers, seconds):
    """The CPU restatements timed on the host's cores, per BASELINE's CPU plan:
    the fp32 oracle (SE:939-972 / SE:629-661 restated) and the reference's own
    fp16 form (SE:968-971), on config-2 layers (the headline `value`: fp32,
    all affine threads) and on config 1, each at all threads and at one; plus
    the config-5 decode step in fp32."""
    from qwenforge_amd import workloads

    threads = len(os.sched_getaffinity(0))
    share = seconds / 4
    cfg1 = [workloads.decode_uniform(1, 512, seed=i) for i in range(8)]
    cfg3 = [workloads.decode_uniform(1, 32768, seed=i, heavy_frac=0.01) for i in range(2)]
    c2_32 = _cpu_row(layers, share * 1.6, threads, "fp32", "config-2")
    c2_16 = _cpu_row(layers, share * 0.8, threads, "fp16", "config-2")
    c1_32 = _cpu_row(cfg1, share * 0.8, threads, "fp32", "config-1")
    c1_16 = _cpu_row(cfg1, share * 0.8, threads, "fp16", "config-1")
    c3_32 = _cpu_row(cfg3, share * 0.4, threads, "fp32", "config-3")
    c3_16 = _cpu_row(cfg3, share * 0.4, threads, "fp16", "config-3")
    # The fp16 eager form takes about 1.7 s per call on the GPU box's host (fp16
    # matrix products on a CPU): 3 calls after one warm-up, and no one-thread row.
    c4 = _cpu_prefill(threads, reps=20, warm=3, reps16=3, warm16=1)
    c4_1 = _cpu_prefill(1, reps=3, warm=1, reps16=0)
    return {
        "value": c2_32["GBps"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": "config 2 (B=4 ragged) layer calls of the fp32 oracle: " + c2_32["sample"],
        "single_thread": {"value": c2_32["single_thread"]["GBps"], "unit": "GB/s",
                          "sample": c2_32["single_thread"]["sample"]},
        "config2": {"fp32_oracle": c2_32, "fp16_reference_form": c2_16},
        "config1": {"fp32_oracle": c1_32, "fp16_reference_form": c1_16,
                    "what": "B=1, L=512, 14q/2kv, hd64, one layer (265,728 B)"},
        "config3": {"fp32_oracle": c3_32, "fp16_reference_form": c3_16,
                    "what": "B=1, L=32768, 1% of keys x8, 14q/2kv, hd64, one layer "
                            "(16,780,800 B); two distinct caches"},
        "config4": {**c4, "single_thread": c4_1,
                    "what": "B=1, S=2048 prefill: RoPE (theta 1e6) + causal attention + cache "
                            "append, 7,519,862,784 FLOP per call"},
        "config5": _cpu_decode_step(threads),
        "cpu_model": _cpu_model(),
    }


def _only(leg, steps, warmup, dev):
    """One leg's figures, for profiling a leg's kernels by themselves."""
    if leg == "cfg1":
        r = bench_decode_cfg1(steps, warmup, dev)
        return {"decode_cfg1": {k: r[k] for k in ("us_per_layer", "us_resident", "splits", "kernel")}}
    if leg == "cfg2":
        r = bench_ragged_decode(steps, warmup, dev)
        return {"decode_cfg2": {"us_per_layer": r["ms_per_step"] * 1e3 / r["launches"],
                                "us_per_launch_in_replay": r["ms_span"] * 1e3 / r["launches"],
                                "splits": r["splits"], "fused": r["fused"]}}
    if leg == "cfg3":
        return {"long_decode_cfg3": bench_long_decode(steps, warmup, dev)}
    if leg == "floor":
        return {"launch_floor": launch_floor(dev)}
    if leg == "valu":
        return {"valu_vs_mfma": bench_valu_vs_mfma(steps, warmup, dev)}
    if leg == "prefill":
        pf = bench_prefill(steps, warmup, dev)
        return {"prefill_cfg4": {"us_per_layer": pf["us_per_layer"],
                                 "TFLOPs": pf["flops"] / (pf["us_per_layer"] * 1e-6) / 1e12}}
    e2e = bench_e2e(dev)
    return {"decode_e2e_cfg5": {str(k): v for k, v in e2e.items()}}


def main():
    args = _args()
    if args.traffic_from:
        traffic_summary(*args.traffic_from)
        return
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.leg, args.trace_steps, args.trace_launches))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every box here has one MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    from qwenforge_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pmc_sample:
        pmc_sample(dev)
        return
    if args.only:
        print(json.dumps(_only(args.only, args.steps, args.warmup, dev)), flush=True)
        return
    if args.prefill_only:
        pf = bench_prefill(args.steps, args.warmup, dev)
        tf = pf["flops"] / (pf["us_per_layer"] * 1e-6) / 1e12
        print(json.dumps({"prefill_cfg4": {"us_per_layer": round(pf["us_per_layer"], 3),
                                           "TFLOPs": round(tf, 2),
                                           "mfma_frac": round(tf / FP16_MFMA_PEAK_TFLOPS, 4)}}))
        return

    r = bench_ragged_decode(args.steps, args.warmup, dev)
    from qwenforge_amd import ops

    cap_max = max(c.key_cache.shape[2] for c in r["layers"])
    kernel = ops.decode_kernel_name(4, 2, 7, cap_max, r["splits"], r["fused"])
    traffic, traffic_src = _traffic(kernel)
    ms = r["ms_per_step"]
    gbs = r["step_bytes"] / (ms * 1e-3) / 1e9
    us_layer = ms * 1e3 / r["launches"]
    launch_bytes = r["step_bytes"] / r["launches"]
    # The roofline's per-launch time: the whole timed step over its launches
    # (the driver's clock around the run sees the same), or with split +
    # combine launches the split launch alone, timed the same way.  The median
    # span of one replay (HIP events right before and after each replay) is
    # reported beside it; on some boxes the events' own serialisation makes
    # it longer than a step in the back-to-back loop, on others shorter.
    us_split = (ms if r["fused"] else r["ms_split"]) * 1e3 / r["launches"]
    split_gbs = launch_bytes / (us_split * 1e-6) / 1e9
    line = {
        "metric": "flash-decode µs/layer + HBM GB/s (% of peak); decode tok/s at bs=1/4",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) fp16 q/k/v, zero-padded caches, fp16-min bias)",
        "config": {
            "workload": "config 2: ragged decode attention, B=4, L_b~U[256,2048], cap=roundup64, "
                        "14q/2kv heads, hd64, 24 per-layer caches; one step = 24 graph-replayed launches",
            "global_batch": 4,
            "kv_lengths_mean": round(sum(sum(c.lengths) for c in r["layers"]) / (4 * 24), 1),
            "splits": r["splits"],
            "cache_replicas": r["replicas"],
        },
        "us_per_layer": round(us_layer, 3),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(split_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(split_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": kernel,
            "kernel_role": ("qf_decode_attn: the whole call is this one launch (single-launch merge)"
                            if r["fused"] else "qf_decode_split: the split launch (partial mode)"),
            "bytes_per_launch": int(launch_bytes),
            "avg_launch_us": round(us_split, 3),
            "avg_launch_us_what": ("ms_per_step / 24 launches: the whole timed step, gaps "
                                   "between graph replays included"),
            "replay_span_us_per_launch": round(r["ms_span"] * 1e3 / r["launches"], 3),
            "replay_span_what": ("median span of one graph replay, HIP events right before and "
                                 "after each replay, / 24 launches"),
            "combine_kernel_avg_us": (None if r["ms_combine"] is None
                                      else round(r["ms_combine"] * 1e3 / r["launches"], 3)),
            "merge": "fused single launch" if r["fused"] else "split + combine launches",
        },
    }
    floor = launch_floor(dev)
    f2 = floor["128x512"]
    line["roofline"]["launch_floor_us"] = {
        "empty": f2["empty_us"], "one_round_trip": f2["one_round_trip_us"],
        "two_round_trips": f2["two_round_trips_us"],
        "what": "graph-replayed qf_launch_probe kernels of this launch's grid (128 workgroups x "
                "512 threads), 24 per graph: an empty node, one dependent HBM round trip, two "
                "(a device index, then the tile, as kv_last then the first K/V tile)"}
    line["launch_floor"] = floor
    if not args.no_extras:
        c1 = bench_decode_cfg1(args.steps, args.warmup, dev)
        line["decode_cfg1"] = {
            "us_per_layer": round(c1["us_per_layer"], 3),
            "GBps": round(c1["bytes"] / (c1["us_per_layer"] * 1e-6) / 1e9, 1),
            "hbm_frac": round(c1["bytes"] / (c1["us_per_layer"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_layer_cache_resident": round(c1["us_resident"], 3),
            "bytes_per_layer": c1["bytes"],
            "splits": c1["splits"],
            "kernel": c1["kernel"],
            "what": f"B=1, L=cap=512, no bias; {c1['caches']} distinct caches rotated past the "
                    "MALL, 64 graph-replayed calls per graph",
        }
        lg = bench_long_decode(args.steps, args.warmup, dev)
        line["long_decode_cfg3"] = {
            "us_per_layer": round(lg["us_per_layer"], 3),
            "GBps": round(lg["bytes"] / (lg["us_per_layer"] * 1e-6) / 1e9, 1),
            "hbm_frac": round(lg["bytes"] / (lg["us_per_layer"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "splits": lg["splits"],
            "merge": "fused single launch" if lg["fused"] else "split + combine launches",
            "timed_calls": lg["calls"],
            "caches": lg["caches"],
        }
        bw = {}
        for b, L in ((12, 5760), (16, 32768), (64, 4096)):
            x = bench_bandwidth_decode(args.steps, args.warmup, dev, b, L)
            gbs_full = x["bytes"] / (x["us_full"] * 1e-6) / 1e9
            gbs_split = x["bytes"] / (x["us_split"] * 1e-6) / 1e9
            bw[f"B{b}_L{L}"] = {
                **({"note": "the reference's own flash-decode benchmark shape (0.180 ms/layer, "
                            "~197 GB/s on its RTX 2080 Ti, README.md:61)"}
                   if (b, L) == (12, 5760) else {}),
                "us_per_layer": round(x["us_full"], 3),
                "GBps": round(gbs_full, 1),
                "hbm_frac": round(gbs_full / HBM_PEAK_GBS, 4),
                "split_kernel_us": round(x["us_split"], 3),
                "split_kernel_hbm_frac": round(gbs_split / HBM_PEAK_GBS, 4),
                "splits": x["splits"],
                "merge": "fused single launch" if x["fused"] else "split + combine launches",
            }
        line["bandwidth_decode"] = bw
        pg = {}
        for b, L in ((16, 32768), (64, 4096)):
            x = bench_paged_decode(args.steps, args.warmup, dev, b, L)
            gbs_full = x["bytes"] / (x["us_full"] * 1e-6) / 1e9
            dense = bw[f"B{b}_L{L}"]
            pg[f"B{b}_L{L}"] = {
                "page": x["page"],
                "us_per_layer": round(x["us_full"], 3),
                "GBps": round(gbs_full, 1),
                "hbm_frac": round(gbs_full / HBM_PEAK_GBS, 4),
                "split_kernel_us": round(x["us_split"], 3),
                "vs_dense_cache": round(dense["us_per_layer"] / x["us_full"], 3),
            }
        line["paged_decode"] = pg
        copy_gbs = hbm_copy_ceiling(dev)
        line["hbm_copy_ceiling"] = {"GBps": round(copy_gbs, 1),
                                    "frac_of_peak": round(copy_gbs / HBM_PEAK_GBS, 4),
                                    "what": "torch copy_ of 512 MiB, read + write bytes / time"}
        line["hbm_read_ceiling"] = hbm_read_ceiling(dev)
        pf = bench_prefill(args.steps, args.warmup, dev)
        tf = pf["flops"] / (pf["us_per_layer"] * 1e-6) / 1e12
        line["prefill_cfg4"] = {
            "us_per_layer": round(pf["us_per_layer"], 3),
            "TFLOPs": round(tf, 2),
            "mfma_frac": round(tf / FP16_MFMA_PEAK_TFLOPS, 4),
            "untimed_warm_ms": round(pf["warm_ms"], 1),
        }
        # The same prefill on a long prompt (same shape otherwise), where the
        # causal imbalance between query tiles weighs less.
        pl = bench_prefill(max(8, args.steps // 4), max(8, args.warmup // 2), dev, seq=8192)
        tl = pl["flops"] / (pl["us_per_layer"] * 1e-6) / 1e12
        line["prefill_long_s8192"] = {
            "us_per_layer": round(pl["us_per_layer"], 3),
            "TFLOPs": round(tl, 2),
            "mfma_frac": round(tl / FP16_MFMA_PEAK_TFLOPS, 4),
            "untimed_warm_ms": round(pl["warm_ms"], 1),
        }
        e2e = bench_e2e(dev)
        line["decode_e2e_cfg5"] = {
            "tok_s_bs1": e2e[1]["decode_tok_s"],
            "tok_s_bs4": e2e[4]["decode_tok_s"],
            "ms_per_step_bs1": e2e[1]["ms_per_step"],
            "ms_per_step_bs4": e2e[4]["ms_per_step"],
            "prefill_ms_bs1": e2e[1]["prefill_ms"],
            "prefill_ms_bs4": e2e[4]["prefill_ms"],
            "weight_stream_GBps_bs1": e2e[1]["weight_GBps"],
            "ragged_bs4": e2e["ragged"],
            "paged": bench_paged_e2e(dev),
            "workload": "24 layers, hidden 896, 14/2 heads, vocab 151936, random-init fp16 "
                        "(std 0.02), 1024-token random prefix, 128 greedy tokens; "
                        "tok/s = B*127 / graph-replay decode time",
        }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline([c for c in r["layers"]], args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
