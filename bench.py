#!/usr/bin/env python3
"""Throughput of the quantized-KV attention hot path on one MI355X.

Headline (BASELINE.json `metric`, config C2): decode attention of Qwen3-32B shapes -- 64 query
heads / 8 KV heads, head_dim 128, 8-bit affine KV cache with group 64, 32768 cached tokens,
batch 1, one fp16 query token -- reported as algorithmic HBM GB/s and as a fraction of the
8 TB/s HBM3E peak.

A step is one attention call (the decode kernel launch(es) of libkvq.so) over one 32K-token
cache. Inputs are resident in HBM before the timed region starts. Steps rotate over enough
distinct caches (>= 3, and more than 2.5x the 256 MB Infinity Cache in total) that every step
streams its cache from HBM rather than from the MALL.

Timing:
  * value / ms_per_step: the K steps are captured once in a HIP graph and replayed; HIP events
    on the launch stream bracket the replay (after a device synchronize on both sides).
  * roofline.achieved: the average duration of one call (the decode kernel and the split-merge
    kernel it launches), from one HIP event pair around a batch of eager calls queued behind a
    spin kernel, so the GPU runs them back to back and the pair brackets their kernels only.
  * prefill.roofline.achieved: the attention kernels' share of the graph-replayed prefill step,
    that is the step minus the same appends replayed alone in a graph of their own (an event
    pair around each eager launch, kept only for the per-chunk breakdown, adds a few us each).
  * roofline.traffic: HBM bytes per call (decode) / per chunk launch (prefill), read from the
    committed rocprofv3 FETCH_SIZE and WRITE_SIZE summary in profiles/, whose counters are scaled
    by what they read for a plain 256 MiB device copy (`bench.py --calibrate-copy`).
  * cpu_baseline: the CPU restatement of the reference algorithm (a torch-CPU port of
    m5engine/attention.py with the reference's dtype casts) timed on the host's cores on one
    cache of the same workload, for a bounded number of calls.

Algorithmic bytes of one decode call:
  sum_b S_b * Hkv * 2 * (D*bits/8 + 2*(D/G)*2)   (K and V codes, scales, biases)
  + 2 * B * Hq * D * 2                           (the query in, the output out)
= 272 B per cached token and KV head at 8 bits, 144 B at 4 bits (D = 128, G = 64); an
unquantized cache (the "-dense" extras) reads D*2 bytes per row, 512 B per token and KV head.

The "extra" object also times the other decode configurations, C2 at batch 8 over a paged pool
(64-row pages in shuffled order, read through block tables), the C3 chunk's cache update with and
without fused RoPE (device time from a graph replay, and the host time of an eager call), and,
over unquantized caches, the
C5 window layer's decode step and prefill chunk and a C3 chunk (attention FLOPs: 4 * D * Hq per
unmasked query-key pair), and head_dim-256 legs (Gemma-3-12B heads: a quantized and an unquantized
window prefill chunk, an unquantized decode step).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--no-parity]
                       [--no-prefill | --prefill-only] [--calibrate-copy]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "decode-attn HBM GB/s (% of peak) @32K 8-bit KV; prefill TFLOP/s (% MFMA)"
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, published
PEAK_MFMA_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, published
MALL_BYTES = 256 << 20  # Infinity Cache


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(seq_lens, Hq, Hkv, D, bits, G=64, elem=2, window=0):
    """Algorithmic HBM bytes of one decode call (see the module docstring). With a sliding
    window only the keys the query can see count: min(S_b, window) per sequence."""
    row = D * elem if bits == 16 else D * bits // 8 + 2 * (D // G) * elem  # bits 16: unquantized rows
    keys = sum(min(s, window) if window > 0 else s for s in seq_lens)
    return keys * Hkv * 2 * row + 2 * len(seq_lens) * Hq * D * elem


# Decode workloads (seed = 1000 + config number). The headline is C2 at batch 1.
DECODE = {
    "C2-b1": dict(desc="Qwen3-32B decode attention, 8-bit KV, 32K context, batch 1", B=1, Hq=64, Hkv=8, D=128,
                  S=32768, bits=8, dtype="float16", seed=1002),
    "C1": dict(desc="Qwen3-0.6B decode attention, 8-bit KV, 4096+1 context", B=1, Hq=16, Hkv=8, D=128, S=4097,
               bits=8, dtype="float16", seed=1001),
    "C2-b8": dict(desc="Qwen3-32B decode attention, 8-bit KV, batch 8, S_b ~ U[16384, 32768]", B=8, Hq=64, Hkv=8,
                  D=128, S=32768, bits=8, dtype="float16", seed=1002, varlen=(16384, 32768)),
    # one GPU's share of C2 at tensor parallelism 8 (each GPU owns one KV head and its 8 query heads)
    "C2-tp8": dict(desc="Qwen3-32B decode attention at TP=8, one GPU's shard: 1 KV head, 8 query heads, 8-bit KV, 32K "
                        "context, batch 8", B=8, Hq=8, Hkv=1, D=128, S=32768, bits=8, dtype="float16", seed=1008),
    "C4": dict(desc="Qwen3-32B decode attention, 4-bit KV, 131072 context, 1% K outlier channels x8", B=1, Hq=64,
               Hkv=8, D=128, S=131072, bits=4, dtype="float16", seed=1004, outliers=True),
    "C5-global": dict(desc="Gemma-3-27B decode step after 8192 prefill, global causal layer, batch 4", B=4, Hq=32,
                      Hkv=16, D=128, S=8193, bits=8, dtype="bfloat16", seed=1005, causal=True),
    "C5-window": dict(desc="Gemma-3-27B decode step after 8192 prefill, window-1024 layer, batch 4", B=4, Hq=32,
                      Hkv=16, D=128, S=8193, bits=8, dtype="bfloat16", seed=1006, causal=True, window=1024),
    # the window layer as the reference runs it: a RotatingKVCache of 1024 rows, left unquantized
    # (m5engine/attention.py:106-112), attention over all of its rows
    "C5-window-dense": dict(desc="Gemma-3-27B decode step, window-1024 layer on its unquantized rotating cache, "
                                 "batch 4", B=4, Hq=32, Hkv=16, D=128, S=1024, bits=16, dtype="bfloat16", seed=1007),
}


def seq_lens_of(cfg):
    import torch

    if "varlen" not in cfg:
        return [cfg["S"]] * cfg["B"]
    lo, hi = cfg["varlen"]
    g = torch.Generator().manual_seed(cfg["seed"])
    return torch.randint(lo, hi + 1, (cfg["B"],), generator=g).tolist()


def make_cache(cfg, seed, device):
    """One seeded cache: K/V ~ N(0,1) in T, quantized by the append kernel into MLX-layout triples
    (bits 16: left unquantized, two [B, Hkv, S, D] tensors)."""
    import torch

    from myinfer_amd import kernels

    B, Hkv, S, D, bits = cfg["B"], cfg["Hkv"], cfg["S"], cfg["D"], cfg["bits"]
    T = getattr(torch, cfg["dtype"])
    g = torch.Generator(device=device).manual_seed(seed)
    if bits == 16:
        return tuple(torch.randn((B, Hkv, S, D), generator=g, device=device, dtype=torch.float32).to(T)
                     for _ in range(2))
    trip = []
    for which in ("k", "v"):
        x = torch.randn((B, Hkv, S, D), generator=g, device=device, dtype=torch.float32)
        if which == "k" and cfg.get("outliers"):
            gc = torch.Generator().manual_seed(seed + 7)
            nch = max(1, round(0.01 * D))
            for h in range(Hkv):
                ch = torch.randperm(D, generator=gc)[:nch].to(device)
                x[:, h, :, ch] *= 8.0
        x = x.to(T)
        codes = torch.empty((B, Hkv, S, D * bits // 32), dtype=torch.int32, device=device).view(torch.uint32)
        scales = torch.empty((B, Hkv, S, D // 64), dtype=T, device=device)
        biases = torch.empty_like(scales)
        kernels.quantize_append(x, (codes, scales, biases), row_offset=0, group_size=64, bits=bits)
        del x
        trip.append((codes, scales, biases))
    return trip[0], trip[1]


def calibrate_spin(torch, target_ms):
    """Cycles of torch.cuda._sleep that keep the GPU busy for about target_ms."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 1 << 20
    torch.cuda.synchronize()
    s.record()
    torch.cuda._sleep(n)
    e.record()
    torch.cuda.synchronize()
    ms = max(s.elapsed_time(e), 1e-3)
    return int(min(n * target_ms / ms, 1 << 34))


def time_decode(cfg, steps, warmup, device, want_parity=False):
    """Run one decode workload; returns a dict of timings (and the caches for the CPU leg)."""
    import torch

    from myinfer_amd import kernels

    lens = seq_lens_of(cfg)
    nbytes = decode_bytes(lens, cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["bits"], window=cfg.get("window", 0))
    ncache = max(3, math.ceil(2.5 * MALL_BYTES / nbytes))  # the bytes a call reads must miss the MALL
    T = getattr(torch, cfg["dtype"])
    log(f"[bench] {cfg['desc']}: {nbytes / 1e6:.2f} MB per call, rotating {ncache} caches")
    caches = [make_cache(cfg, cfg["seed"] * 100 + i, device) for i in range(ncache)]
    gq = torch.Generator(device=device).manual_seed(cfg["seed"] + 2)
    q = torch.randn((cfg["B"], cfg["Hq"], 1, cfg["D"]), generator=gq, device=device).to(T)
    out = torch.empty_like(q)
    sl = None if "varlen" not in cfg else torch.tensor(lens, dtype=torch.int32, device=device)
    scale = 1.0 / math.sqrt(cfg["D"])
    calls = [kernels.prepare_attention(q, kt, vt, scale, causal=cfg.get("causal", False),
                                       window=cfg.get("window", 0), seq_lens=sl, bits=cfg["bits"], out=out,
                                       kernel="decode") for kt, vt in caches]
    for i in range(warmup):
        calls[i % ncache]()
    torch.cuda.synchronize()

    # per-call duration: one event pair around a batch of eager calls queued behind a spin kernel,
    # so the GPU runs the calls back to back and the pair brackets their kernels only
    nev = min(steps, 100)
    ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    cycles = calibrate_spin(torch, 20.0 + 0.05 * nev)
    torch.cuda.synchronize()
    torch.cuda._sleep(cycles)
    ev[0].record()
    for i in range(nev):
        calls[i % ncache]()
    ev[1].record()
    torch.cuda.synchronize()
    call_us_mean = 1e3 * ev[0].elapsed_time(ev[1]) / nev
    call_us_median = call_us_mean

    # the timed region: K steps captured in one HIP graph, replayed
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        # the prepared calls launch on the stream that was current when they were built; rebuild
        # them on the capture stream
        gcalls = [kernels.prepare_attention(q, kt, vt, scale, causal=cfg.get("causal", False),
                                            window=cfg.get("window", 0), seq_lens=sl, bits=cfg["bits"], out=out,
                                            kernel="decode") for kt, vt in caches]
    with torch.cuda.graph(graph, stream=side):
        for i in range(steps):
            gcalls[i % ncache]()
    graph.replay()  # untimed graph warm-up
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    graph.replay()
    e.record()
    torch.cuda.synchronize()
    total_ms = s.elapsed_time(e)
    ms_per_step = total_ms / steps

    res = dict(bytes=nbytes, ncache=ncache, ms_per_step=ms_per_step, gbs=nbytes / (ms_per_step * 1e-3) / 1e9,
               call_us_mean=call_us_mean, call_us_median=call_us_median,
               kernel_gbs=nbytes / (call_us_mean * 1e-6) / 1e9, seq_lens=lens)
    if want_parity:
        res["parity"], res["parity_arrays"] = parity_check(cfg, q, caches[0], sl, scale)
        res["cpu_inputs"] = (q, caches[0], scale)
    del graph, calls, gcalls
    return res


def time_paged_decode(cfg, steps, warmup, device):
    """The decode workload over a paged pool: each sequence's rows in shuffled 64-row pages read
    through its block table. Enough disjoint page sets that every call streams from HBM."""
    import torch

    from myinfer_amd import kernels

    PAGE = kernels.PAGE_ROWS
    lens = seq_lens_of(cfg)
    B, Hq, Hkv, D, bits = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["bits"]
    T = getattr(torch, cfg["dtype"])
    nbytes = decode_bytes(lens, Hq, Hkv, D, bits)
    ncache = max(3, math.ceil(2.5 * MALL_BYTES / nbytes))
    per_set = sum(math.ceil(n / PAGE) for n in lens)
    npages = ncache * per_set
    log(f"[bench] {cfg['desc']} (paged): {nbytes / 1e6:.2f} MB per call, {ncache} page sets of {per_set} pages")
    W, G = D * bits // 32, D // 64
    pools = []
    for _ in range(2):
        codes = torch.empty((npages, Hkv, PAGE, W), dtype=torch.int32, device=device).view(torch.uint32)
        sc = torch.empty((npages, Hkv, PAGE, G), dtype=T, device=device)
        pools.append((codes, sc, torch.empty_like(sc)))
    g = torch.Generator().manual_seed(cfg["seed"] + 11)
    perm = torch.randperm(npages, generator=g).tolist()
    width = max(math.ceil(n / PAGE) for n in lens)
    gd = torch.Generator(device=device).manual_seed(cfg["seed"] + 12)
    tables, k = [], 0
    for _ in range(ncache):
        rows = []
        for n in lens:
            need = math.ceil(n / PAGE)
            rows.append(perm[k:k + need] + [perm[k + need - 1]] * (width - need))
            k += need
        t = torch.tensor(rows, dtype=torch.int32, device=device)
        for b, n in enumerate(lens):
            x = torch.randn((1, Hkv, n, D), generator=gd, device=device).to(T)
            y = torch.randn((1, Hkv, n, D), generator=gd, device=device).to(T)
            kernels.paged_quantize_append(x, pools[0], y, pools[1], t[b:b + 1], bits=bits)
        tables.append(t)
    q = torch.randn((B, Hq, 1, D), generator=gd, device=device).to(T)
    out = torch.empty_like(q)
    sl = torch.tensor(lens, dtype=torch.int32, device=device)
    scale = 1.0 / math.sqrt(D)
    S = max(lens)

    def call(i):
        kernels.paged_attention(q, pools[0], pools[1], tables[i % ncache], sl, scale, bits=bits, max_len=S, out=out,
                                kernel="decode")

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(0)  # the side stream's workspace exists before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(steps):
            call(i)
    graph.replay()
    torch.cuda.synchronize()
    s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_.record()
    graph.replay()
    e_.record()
    torch.cuda.synchronize()
    ms = s_.elapsed_time(e_) / steps
    del graph
    # the last replayed call read page set (steps - 1) % ncache: its first sequence, gathered out of
    # the pools through its block table, against the exact fp64 oracle
    t = tables[(steps - 1) % ncache]
    n0 = lens[0]
    pages = t[0, :math.ceil(n0 / PAGE)].long()

    def gather(pool):  # (codes indexed as int32: torch has no uint32 gather on the device)
        return tuple((x.view(torch.int32) if x.dtype == torch.uint32 else x)[pages].permute(1, 0, 2, 3)
                     .reshape(1, Hkv, -1, x.shape[-1])[:, :, :n0] for x in pool)

    parity = tail_parity(q[:1], gather(pools[0]), gather(pools[1]), out[:1], scale, bits=bits)
    parity["rows"] = "sequence 0 of the last page set"
    return dict(bytes=nbytes, ms_per_step=ms, gbs=nbytes / (ms * 1e-3) / 1e9, parity=parity)


def parity_check(cfg, q, cache, sl, scale):
    """One call against the exact fp64 oracle (the bench's own sanity check of what it times)."""
    import numpy as np
    import torch

    from myinfer_amd import kernels
    from oracle import attention as OA
    from oracle import quantize as OQ

    dense = cfg["bits"] == 16
    out = kernels.attention(q, cache[0], cache[1], scale, causal=cfg.get("causal", False),
                            window=cfg.get("window", 0), seq_lens=sl, kernel="decode",
                            **({} if dense else {"bits": cfg["bits"]}))
    torch.cuda.synchronize()
    dt = cfg["dtype"]

    def trip(tr):
        if dense:  # an unquantized cache: the tensor itself
            return tr.float().cpu().double().numpy()
        c, s, b = tr
        return OQ.dequantize(c.cpu().view(torch.int32).numpy().view(np.uint32),
                             s.cpu().view(torch.int16).numpy().view(np.uint16),
                             b.cpu().view(torch.int16).numpy().view(np.uint16), dt, 64, cfg["bits"])

    kdq = trip(cache[0])
    vdq = trip(cache[1])
    ref = OA.exact_attention(q.cpu().double().numpy(), kdq, vdq, scale, causal=cfg.get("causal", False),
                             window=cfg.get("window", 0), seq_lens=None if sl is None else sl.cpu().tolist())
    got = out.cpu().double().numpy()
    return parity_record(got, ref, dt), (got, ref)


def parity_record(got, ref, dtype: str, **extra):
    """Error against the exact fp64 oracle and the bar it is judged by: the north-star bar for fp16
    outputs (max-abs 2e-3, relative L2 1e-3); for bf16 outputs half an ulp of the output rounding on
    top (max-abs 2^-8 max|ref| + 1e-3, relative L2 3e-3), as in tests/helpers.py."""
    import numpy as np

    from oracle import attention as OA

    st = OA.error_stats(got, ref)
    bar = (2e-3, 1e-3) if dtype == "float16" else (2.0**-8 * float(np.abs(ref).max()) + 1e-3, 3e-3)
    return {"vs": "exact fp64 oracle", **extra, "max_abs": st["max_abs"], "rel_l2": st["rel_l2"],
            "bar": {"max_abs": bar[0], "rel_l2": bar[1]},
            "within_bar": bool(st["max_abs"] <= bar[0] and st["rel_l2"] <= bar[1])}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def reference_mask(cfg, lens, L, S):
    """The mask the reference's caller would pass for this workload (m5engine/attention.py:55-58,
    70-81): None (every key visible), "causal", or a bool [B, 1, L, S] array for per-sequence
    lengths and sliding windows."""
    import numpy as np
    import torch

    from oracle import attention as OA

    window, causal = cfg.get("window", 0), cfg.get("causal", False)
    if window == 0 and all(n == S for n in lens):
        return "causal" if causal and L > 1 else None
    m = np.stack([OA.key_mask(L, S, n, causal, window) for n in lens])[:, None]
    return torch.from_numpy(m)


def cpu_trip(tr):
    import torch

    c, s, b = tr
    return (c.cpu().view(torch.int32).to(torch.int64) & 0xFFFFFFFF, s.cpu(), b.cpu())


def cpu_baseline(cfg, q, cache, scale, lens, budget_s=15.0, max_calls=8, min_calls=5):
    """The reference algorithm restated for the CPU (oracle.attention.reference_sdpa: mlx-lm's
    quantized SDPA for L == 1 with the reference's dtype casts and masks), timed on the host's
    cores over the same workload (one cache, every sequence of the batch): at least `min_calls`
    calls, more while the time budget lasts, up to `max_calls`; the median is reported."""
    import torch

    from oracle import attention as OA

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    qc = q.cpu()
    kt, vt = cpu_trip(cache[0]), cpu_trip(cache[1])
    mask = reference_mask(cfg, lens, 1, cfg["S"])
    OA.reference_sdpa(qc, kt, vt, scale, mask, 64, cfg["bits"])  # warm-up (allocator, threads)
    times = []
    t_all = time.perf_counter()
    while len(times) < max_calls and (len(times) < min_calls or (time.perf_counter() - t_all) < budget_s):
        t0 = time.perf_counter()
        ref_out = OA.reference_sdpa(qc, kt, vt, scale, mask, 64, cfg["bits"])
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    nbytes = decode_bytes(lens, cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["bits"], window=cfg.get("window", 0))
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} calls of this workload (one cache, B={cfg['B']}) through "
                   f"oracle.attention.reference_sdpa on the host CPU ({cpu_model()}); median {med * 1e3:.1f} ms/call"),
    }, ref_out.float().double().numpy()


# Prefill workload C3 (seed 1003): Qwen3-30B-A3B shapes, a 16384-token prompt in 512-token chunks;
# each chunk is quantize-appended to an 8-bit cache and then attends causally to all prior keys.
PREFILL = dict(desc="Qwen3-30B-A3B chunked prefill, 16384 tokens in 512-token chunks, 8-bit KV, bf16", B=1,
               Hq=32, Hkv=4, D=128, N=16384, chunk=512, bits=8, dtype="bfloat16", seed=1003)


# C5 (Gemma-3-27B shapes) prefill legs over the quantized cache: B=4 sequences of 8192 tokens in
# 2048-token chunks, 32 query heads / 16 KV heads, bf16; the global causal layer and a window-1024
# layer (5 of every 6 layers; quantized here, as the C5 workload's 8-bit KV cache states, although
# the reference leaves sliding-window caches unquantized: m5engine/attention.py:106-112).
PREFILL_C5 = {
    "C5-global-prefill": dict(desc="Gemma-3-27B global-layer chunked prefill, B=4 x 8192 tokens in 2048-token "
                                   "chunks, 8-bit KV, bf16", B=4, Hq=32, Hkv=16, D=128, N=8192, chunk=2048, bits=8,
                              dtype="bfloat16", seed=1015),
    "C5-window-prefill": dict(desc="Gemma-3-27B window-1024-layer chunked prefill, B=4 x 8192 tokens in 2048-token "
                                   "chunks, 8-bit KV, bf16", B=4, Hq=32, Hkv=16, D=128, N=8192, chunk=2048, bits=8,
                              dtype="bfloat16", seed=1016, window=1024),
}


def prefill_flops(N, Hq, D, L0=0, L1=None, window=0, B=1):
    """Algorithmic FLOPs of causal attention for query positions [L0, L1) of B N-token prompts:
    4 * D * Hq per unmasked (query, key) pair; position p sees p + 1 keys, or min(p + 1, window)."""
    L1 = N if L1 is None else L1
    if window > 0:
        pairs = sum(min(p + 1, window) for p in range(L0, L1))
    else:
        pairs = (L1 * (L1 + 1) - L0 * (L0 + 1)) // 2
    return 4 * D * Hq * pairs * B


def time_prefill(cfg, steps, warmup, device, want_parity=False):
    """One step = the whole prompt: per chunk, the fused quantize-append of its K/V rows and the
    causal attention of its queries over the cache so far."""
    import torch

    from myinfer_amd import kernels

    B, Hq, Hkv, D, N, C, bits = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["D"], cfg["N"], cfg["chunk"], cfg["bits"]
    W = cfg.get("window", 0)
    T = getattr(torch, cfg["dtype"])
    g = torch.Generator(device=device).manual_seed(cfg["seed"])
    k = torch.randn((B, Hkv, N, D), generator=g, device=device).to(T)
    v = torch.randn((B, Hkv, N, D), generator=g, device=device).to(T)
    q = torch.randn((B, Hq, N, D), generator=g, device=device).to(T)
    out = torch.empty_like(q)
    kc = torch.zeros((B, Hkv, N, D * bits // 32), dtype=torch.int32, device=device).view(torch.uint32)
    vc = torch.zeros_like(kc)
    ks, kb, vs, vb = (torch.zeros((B, Hkv, N, D // 64), dtype=T, device=device) for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    nchunk = N // C
    flops = prefill_flops(N, Hq, D, window=W, B=B)
    log(f"[bench] {cfg['desc']}: {flops / 1e12:.3f} TFLOP of attention per step")

    def make_calls():
        appends, attns = [], []
        for c in range(nchunk):
            lo, hi = c * C, (c + 1) * C
            appends.append((k[:, :, lo:hi], v[:, :, lo:hi], lo))
            attns.append(kernels.prepare_attention(q[:, :, lo:hi], (kc[:, :, :hi], ks[:, :, :hi], kb[:, :, :hi]),
                                                   (vc[:, :, :hi], vs[:, :, :hi], vb[:, :, :hi]), scale, causal=True,
                                                   window=W, bits=bits, out=out[:, :, lo:hi], kernel="prefill"))
        return appends, attns

    def append(a):
        kernels.quantize_append(a[0], (kc, ks, kb), a[1], (vc, vs, vb), row_offset=a[2], group_size=64, bits=bits)

    appends, attns = make_calls()
    for _ in range(max(1, warmup // nchunk)):
        for a, f in zip(appends, attns):
            append(a)
            f()
    torch.cuda.synchronize()

    # per-chunk breakdown: event pairs around each append and attention call, all queued behind a
    # spin kernel. Each pair also holds the gap between its event packets and the kernel (a few us),
    # so the attention total below comes from a graph of the attention launches instead.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(2 * nchunk)]
    cycles = calibrate_spin(torch, 30.0)
    torch.cuda.synchronize()
    torch.cuda._sleep(cycles)
    for c, (a, f) in enumerate(zip(appends, attns)):
        ev[2 * c][0].record()
        append(a)
        ev[2 * c][1].record()
        ev[2 * c + 1][0].record()
        f()
        ev[2 * c + 1][1].record()
    torch.cuda.synchronize()
    append_ms = [ev[2 * c][0].elapsed_time(ev[2 * c][1]) for c in range(nchunk)]
    attn_ms = [ev[2 * c + 1][0].elapsed_time(ev[2 * c + 1][1]) for c in range(nchunk)]

    # the timed region: `steps` whole prompts captured in one HIP graph and replayed
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gappends, gattns = make_calls()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(steps):
            for a, f in zip(gappends, gattns):
                kernels.quantize_append(a[0], (kc, ks, kb), a[1], (vc, vs, vb), row_offset=a[2], group_size=64,
                                        bits=bits)
                f()
    graph.replay()
    torch.cuda.synchronize()
    s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_.record()
    graph.replay()
    e_.record()
    torch.cuda.synchronize()
    ms_per_step = s_.elapsed_time(e_) / steps
    del graph

    # The attention kernels' share of the timed step: the step minus the same appends replayed alone
    # (a graph of the prompt's append launches; they rewrite the same rows). For reference, the
    # attention launches replayed alone (the cache already holds every chunk's rows, and a chunk's
    # call reads only the rows before its end). Each graph holds `steps` prompts and is timed by one
    # event pair.
    def replay_ms(body):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=side):
            for _ in range(steps):
                body()
        gr.replay()
        torch.cuda.synchronize()
        s_.record()
        gr.replay()
        e_.record()
        torch.cuda.synchronize()
        return s_.elapsed_time(e_) / steps

    def appends_only():
        for a in gappends:
            kernels.quantize_append(a[0], (kc, ks, kb), a[1], (vc, vs, vb), row_offset=a[2], group_size=64, bits=bits)

    def attns_only():
        for f in gattns:
            f()

    append_graph_ms = replay_ms(appends_only)
    attn_alone_ms = replay_ms(attns_only)
    attn_step_ms = ms_per_step - append_graph_ms
    res = dict(flops=flops, ms_per_step=ms_per_step, tflops=flops / (ms_per_step * 1e-3) / 1e12,
               attn_ms=attn_step_ms, append_ms=append_graph_ms, attn_alone_ms=attn_alone_ms,
               attn_events_ms=sum(attn_ms), append_events_ms=sum(append_ms),
               attn_tflops=flops / (attn_step_ms * 1e-3) / 1e12,
               chunk_attn_us={c: round(1e3 * attn_ms[c], 2) for c in (0, nchunk // 2, nchunk - 1)})
    if want_parity:
        res["parity"], res["parity_arrays"] = prefill_parity(cfg, q, out, (kc, ks, kb), (vc, vs, vb), scale,
                                                             nchunk - 1)
        last = nchunk - 1
        res["cpu_inputs"] = (q[:, :, last * C:], (kc, ks, kb), (vc, vs, vb), scale)
    return res


def time_attention_shape(desc, q, k, v, scale, flops, steps, device, check=None, **mask):
    """Attention-kernel TFLOP/s of one prefill call shape (k, v: unquantized tensors, or quantized
    triples with bits / group_size among the keyword arguments): `steps` calls captured in a HIP
    graph and replayed once, timed with events. `check(out)`, when given, judges the output the
    timed replay left and its record goes in as "parity"."""
    import torch

    from myinfer_amd import kernels

    out = torch.empty_like(q)
    log(f"[bench] {desc}: {flops / 1e12:.4f} TFLOP per call")
    kernels.prepare_attention(q, k, v, scale, out=out, kernel="prefill", **mask)()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call = kernels.prepare_attention(q, k, v, scale, out=out, kernel="prefill", **mask)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(steps):
            call()
    graph.replay()
    torch.cuda.synchronize()
    s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_.record()
    graph.replay()
    e_.record()
    torch.cuda.synchronize()
    ms = s_.elapsed_time(e_) / steps
    del graph
    res = {"tflops": round(flops / (ms * 1e-3) / 1e12, 2), "frac": round(flops / (ms * 1e-3) / 1e12 / PEAK_MFMA_TFLOPS, 4),
           "us_per_call": round(ms * 1e3, 2), "flops": flops}
    if check is not None:
        res["parity"] = check(out)
    return res


def tail_parity(q, k, v, out, scale, rows=128, bits=None, window=0):
    """The last `rows` queries of a causal call (all heads) against the exact fp64 oracle: queries
    align to the end of the keys, as in the kernels. k, v: unquantized tensors, or quantized
    triples of group 64 with `bits`."""
    import numpy as np
    import torch

    from oracle import attention as OA
    from oracle import quantize as OQ

    dt = str(q.dtype).replace("torch.", "")

    def host(x):
        if bits is None:
            return x.float().cpu().double().numpy()
        cc, ss, bb = x
        return OQ.dequantize(cc.cpu().view(torch.int32).numpy().view(np.uint32),
                             ss.cpu().view(torch.int16).numpy().view(np.uint16),
                             bb.cpu().view(torch.int16).numpy().view(np.uint16), dt, 64, bits)

    L = q.shape[2]
    r = min(rows, L)
    qs = q[:, :, L - r:].float().cpu().double().numpy()
    ref = OA.exact_attention(qs, host(k), host(v), scale, causal=True, window=window)
    got = out[:, :, L - r:].float().cpu().double().numpy()
    return parity_record(got, ref, dt, rows=f"last {r} of {L} queries")


def dense_prefill_extras(steps, device):
    """Prefill over unquantized caches: the C5 window layer's steady-state 2048-row chunk (its
    rotating cache returns 1023 earlier rows + the chunk; every query sees 1024 keys), and the last
    C3 chunk over an unquantized cache (the plain cache before quantized_kv_start)."""
    import torch

    g = torch.Generator(device=device).manual_seed(1008)
    res = {}
    B, Hq, Hkv, D, W, C = 4, 32, 16, 128, 1024, 2048
    T = torch.bfloat16
    q = torch.randn((B, Hq, C, D), generator=g, device=device).to(T)
    k = torch.randn((B, Hkv, W - 1 + C, D), generator=g, device=device).to(T)
    v = torch.randn((B, Hkv, W - 1 + C, D), generator=g, device=device).to(T)
    res["C5-window-prefill-dense"] = time_attention_shape(
        "C5 window-layer prefill chunk, unquantized bf16 (B=4, 2048 queries, window 1024)", q, k, v,
        1.0 / math.sqrt(D), 4 * D * Hq * B * C * W, steps, device, causal=True, window=W,
        check=lambda out: tail_parity(q, k, v, out, 1.0 / math.sqrt(D), window=W))
    B, Hq, Hkv, N, C = 1, 32, 4, 16384, 512
    q = torch.randn((B, Hq, C, D), generator=g, device=device).to(T)
    k = torch.randn((B, Hkv, N, D), generator=g, device=device).to(T)
    v = torch.randn((B, Hkv, N, D), generator=g, device=device).to(T)
    res["C3-last-chunk-dense"] = time_attention_shape(
        "C3 last chunk over an unquantized bf16 cache (512 queries, 16384 keys, causal)", q, k, v,
        1.0 / math.sqrt(D), prefill_flops(N, Hq, D, N - C, N), steps, device, causal=True,
        check=lambda out: tail_parity(q, k, v, out, 1.0 / math.sqrt(D)))
    return res


def wide_extras(steps, device):
    """Head_dim 256 (Gemma-3-12B attention: 16 query / 8 KV heads): a 2048-token prefill chunk after
    6144 earlier tokens over an 8-bit quantized bf16 cache, a sliding-window (1024) chunk of the same
    size over an unquantized cache, and a batch-4 decode step over 8192 unquantized rows (graph
    replay; HBM bytes = the K/V rows read plus the query and output)."""
    import torch

    from myinfer_amd import kernels

    g = torch.Generator(device=device).manual_seed(1010)
    res = {}
    B, Hq, Hkv, D, S, C = 1, 16, 8, 256, 8192, 2048
    T = torch.bfloat16
    k = torch.randn((B, Hkv, S, D), generator=g, device=device).to(T)
    v = torch.randn((B, Hkv, S, D), generator=g, device=device).to(T)
    q = torch.randn((B, Hq, C, D), generator=g, device=device).to(T)
    trip = []
    for x in (k, v):
        c = torch.zeros((B, Hkv, S, D // 4), dtype=torch.int32, device=device).view(torch.uint32)
        sc = torch.zeros((B, Hkv, S, D // 64), dtype=T, device=device)
        bi = torch.zeros_like(sc)
        kernels.quantize_append(x, (c, sc, bi), group_size=64, bits=8)
        trip.append((c, sc, bi))
    res["D256-prefill-q8"] = time_attention_shape(
        "head_dim 256 prefill chunk over an 8-bit cache (Gemma-3-12B heads, 2048 queries, 8192 keys, causal)",
        q, trip[0], trip[1], 1.0 / math.sqrt(D), prefill_flops(S, Hq, D, S - C, S), steps, device, causal=True,
        bits=8, group_size=64, check=lambda out: tail_parity(q, trip[0], trip[1], out, 1.0 / math.sqrt(D), bits=8))
    W = 1024
    res["D256-window-prefill-dense"] = time_attention_shape(
        "head_dim 256 window-1024 prefill chunk over an unquantized bf16 cache (2048 queries, 8192 keys)",
        q, k, v, 1.0 / math.sqrt(D), prefill_flops(S, Hq, D, S - C, S, window=W), steps, device, causal=True,
        window=W, check=lambda out: tail_parity(q, k, v, out, 1.0 / math.sqrt(D), window=W))
    del trip
    B = 4
    k = torch.randn((B, Hkv, S, D), generator=g, device=device).to(T)
    v = torch.randn((B, Hkv, S, D), generator=g, device=device).to(T)
    q = torch.randn((B, Hq, 1, D), generator=g, device=device).to(T)
    out = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call = kernels.prepare_attention(q, k, v, 1.0 / math.sqrt(D), out=out)
    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(steps):
            call()
    graph.replay()
    torch.cuda.synchronize()
    s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_.record()
    graph.replay()
    e_.record()
    torch.cuda.synchronize()
    us = s_.elapsed_time(e_) / steps * 1e3
    nbytes = 2 * k.numel() * 2 + 2 * q.numel() * 2
    res["D256-decode-dense-b4"] = {"gbs": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4),
                                   "us_per_step": round(us, 3), "bytes": nbytes, "kernel": call.symbol,
                                   "parity": tail_parity(q, k, v, out, 1.0 / math.sqrt(D))}
    del graph
    return res


def plain_read_reference(nbytes, steps, device):
    """What a plain read of the same number of bytes costs on this GPU, for reading the decode
    roofline fraction against: torch's own reduction kernel (an fp32 sum) and its
    device copy (nbytes read and nbytes written), each timed like the decode call (one event pair
    around a batch of eager calls queued behind a spin kernel) over buffers that rotate past the
    MALL like the decode caches. A reference point, not a bound."""
    import torch

    nbuf = max(3, math.ceil(2.5 * MALL_BYTES / nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device=device) for _ in range(nbuf)]
    dsts = [torch.empty_like(b) for b in bufs]
    acc = torch.zeros((), dtype=torch.float32, device=device)

    n = min(steps, 100)

    def timed(fn):
        for i in range(3):
            fn(i)
        cycles = calibrate_spin(torch, 20.0 + 0.05 * n)
        torch.cuda.synchronize()
        s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(cycles)
        s_.record()
        for i in range(n):
            fn(i)
        e_.record()
        torch.cuda.synchronize()
        return s_.elapsed_time(e_) / n * 1e3  # us

    sum_us = timed(lambda i: torch.sum(bufs[i % nbuf], dim=0, out=acc))
    copy_us = timed(lambda i: dsts[i % nbuf].copy_(bufs[i % nbuf]))
    del bufs, dsts
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "torch_sum_us": round(sum_us, 3), "torch_sum_gbs": round(nbytes / sum_us / 1e3, 1),
            "torch_copy_us": round(copy_us, 3), "torch_copy_gbs": round(2 * nbytes / copy_us / 1e3, 1),
            "note": "torch's fp32 sum and device copy over buffers of the call's size rotated past the MALL, "
                    "timed like the decode call; copy counts read + write bytes"}


def append_extras(device, calls=200):
    """The C3 chunk's cache update: quantize-append of 512 rows x 4 KV heads (bf16, 8-bit), plain and
    with the keys rotated in the same launch (kvq_rope_quantize_append); device microseconds per call
    (graph replay) and the HBM bytes it moves (reads 2 B and writes 1.0625 B per element, K and V),
    and the host microseconds of one eager call from Python, plain and through prepare_append."""
    import torch

    from myinfer_amd import kernels

    g = torch.Generator(device=device).manual_seed(1009)
    k = torch.randn((1, 4, 512, 128), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((1, 4, 512, 128), generator=g, device=device).to(torch.bfloat16)

    def triple():
        c = torch.zeros((1, 4, 16384, 32), dtype=torch.int32, device=device).view(torch.uint32)
        sc = torch.zeros((1, 4, 16384, 2), dtype=torch.bfloat16, device=device)
        return c, sc, torch.zeros_like(sc)

    kd, vd = triple(), triple()
    rope = kernels.Rope(128, False, 1000000.0)
    res = {}
    for name, kw in (("append", {}), ("rope_append", {"rope": rope})):
        kernels.quantize_append(k, kd, v, vd, row_offset=15872, bits=8, **kw)
        torch.cuda.synchronize()
        # device time: the calls captured in a HIP graph and replayed
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(calls):
                kernels.quantize_append(k, kd, v, vd, row_offset=15872, bits=8, **kw)
        graph.replay()
        torch.cuda.synchronize()
        s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_.record()
        graph.replay()
        e_.record()
        torch.cuda.synchronize()
        us = 1e3 * s_.elapsed_time(e_) / calls
        # host cost of one eager call from Python (descriptor packing and the foreign call)
        t0 = time.perf_counter()
        for _ in range(calls):
            kernels.quantize_append(k, kd, v, vd, row_offset=15872, bits=8, **kw)
        host_us = 1e6 * (time.perf_counter() - t0) / calls
        torch.cuda.synchronize()
        # the same through a prepared call (descriptors built once, as the cache objects do)
        call = kernels.prepare_append(kd, vd, bits=8, **kw)
        t0 = time.perf_counter()
        for _ in range(calls):
            call(k, v, 15872)
        prep_us = 1e6 * (time.perf_counter() - t0) / calls
        torch.cuda.synchronize()
        nbytes = 2 * 4 * 512 * (128 * 2 + 128 + 8)
        res[name] = {"us_per_call": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "host_us_per_eager_call": round(host_us, 2), "host_us_per_prepared_call": round(prep_us, 2)}
        del graph
    return res


def prefill_parity(cfg, q, out, kt, vt, scale, c):
    """Chunk c's output (as left by the timed steps) against the exact fp64 oracle."""
    import numpy as np
    import torch

    from oracle import attention as OA
    from oracle import quantize as OQ

    C = cfg["chunk"]
    hi = (c + 1) * C

    def trip(tr):
        cc, ss, bb = (x[:, :, :hi] for x in tr)
        return (cc.cpu().view(torch.int32).numpy().view(np.uint32), ss.cpu().view(torch.int16).numpy().view(np.uint16),
                bb.cpu().view(torch.int16).numpy().view(np.uint16))

    kdq = OQ.dequantize(*trip(kt), cfg["dtype"], 64, cfg["bits"])
    vdq = OQ.dequantize(*trip(vt), cfg["dtype"], 64, cfg["bits"])
    qc = q[:, :, c * C:hi].float().cpu().double().numpy()
    ref = OA.exact_attention(qc, kdq, vdq, scale, causal=True, window=cfg.get("window", 0))
    got = out[:, :, c * C:hi].float().cpu().double().numpy()
    return parity_record(got, ref, cfg["dtype"], chunk=c), (got, ref)


def prefill_cpu_baseline(cfg, q_last, kt, vt, scale, budget_s=20.0):
    """The reference algorithm (oracle.attention.reference_sdpa: m5engine/attention.py's blocked
    loop with its dtype casts and masks) on the last chunk of the prompt of the first sequence,
    timed on the host's cores. Returns the baseline and the port's output for that sequence."""
    import torch

    from oracle import attention as OA

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    N, C, W = cfg["N"], cfg["chunk"], cfg.get("window", 0)
    qc = q_last[:1].cpu()
    ktc, vtc = (tuple(x[:1] for x in cpu_trip(t)) for t in (kt, vt))
    mask = reference_mask(dict(cfg, causal=True), [N], C, N)
    mask = "causal" if mask is None and W == 0 else mask
    times = []
    t_all = time.perf_counter()
    while not times or (time.perf_counter() - t_all < budget_s and len(times) < 3):
        t0 = time.perf_counter()
        ref_out = OA.reference_sdpa(qc, ktc, vtc, scale, mask, 64, cfg["bits"])
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    fl = prefill_flops(N, cfg["Hq"], cfg["D"], N - C, N, window=W)
    return {"value": round(fl / med / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} run(s) of the last {C}-token chunk ({N} keys{f', window {W}' if W else ''}) of "
                      f"one sequence through oracle.attention.reference_sdpa on the host CPU ({cpu_model()}); "
                      f"median {med:.2f} s"}, ref_out.float().double().numpy()


def add_faithful(parity, arrays, faithful):
    """Extend a parity record with the error against the reference-faithful CPU port (the output
    the CPU baseline computed on the same inputs) and that port's own error against exact fp64."""
    if parity is None or arrays is None or faithful is None:
        return parity
    from oracle import attention as OA

    got, exact = arrays
    n = faithful.shape[0]  # the port may have run on the first sequences only
    got, exact = got[:n], exact[:n]
    a, b, g = OA.error_stats(got, faithful), OA.error_stats(faithful, exact), OA.error_stats(got, exact)
    parity["vs_faithful_oracle"] = {"max_abs": a["max_abs"], "rel_l2": a["rel_l2"]}
    parity["faithful_oracle_vs_exact"] = {"max_abs": b["max_abs"], "rel_l2": b["rel_l2"]}
    if n < arrays[0].shape[0]:
        parity["faithful_sequences"] = n
    # the bound the GPU-to-port distance must meet: within (GPU error + port error), the triangle
    # inequality through the exact answer (both errors measured against it); and whether the GPU is
    # at least as close to the exact answer as the reference's own algorithm (same sequences)
    parity["checks"] = {
        "port_distance_within_gpu_plus_port_error": bool(
            a["max_abs"] <= (g["max_abs"] + b["max_abs"]) * (1 + 1e-9) and
            a["rel_l2"] <= (g["rel_l2"] + b["rel_l2"]) * (1 + 1e-9)),
        "gpu_no_less_accurate_than_port": bool(g["max_abs"] <= b["max_abs"] and g["rel_l2"] <= b["rel_l2"]),
    }
    return parity


TRAFFIC_FILE = Path(__file__).resolve().parent / "profiles" / "hbm_traffic_decode_c2_b1_prefill_c3.md"


def measured_traffic(key: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by
    the copy-kernel calibration recorded there), or None when the summary has no such line."""
    try:
        text = TRAFFIC_FILE.read_text()
    except OSError:
        return None
    m = re.search(rf"^bytes_per_(?:call|launch) {re.escape(key)}: (\d+)$", text, re.M)
    return int(m.group(1)) if m else None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="time only the headline workload")
    ap.add_argument("--no-parity", action="store_true", help="skip the oracle check of the headline output")
    ap.add_argument("--no-prefill", action="store_true", help="skip the C3 chunked-prefill leg")
    ap.add_argument("--prefill-only", action="store_true", help="time only the C3 chunked-prefill leg")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 10 device copies of 256 MiB (reference for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--config", choices=sorted(DECODE) + sorted(PREFILL_C5) + ["C3", "D256"],
                    help="time only this workload (no CPU leg, no parity) and print its numbers: for profiling")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one GPU: the attention path here runs on a single MI355X (multi-GPU sharding "
            "is a design note only). Run with --gpus 1.")
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        ap.error("--steps must be >= 1 and --warmup >= 0")

    import torch

    from myinfer_amd import _lib

    if not torch.cuda.is_available():
        log("bench.py needs a GPU (torch.cuda.is_available() is False)")
        sys.exit(1)
    _lib.lib()  # the HIP library must be built; there is no fallback
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    log(f"[bench] device: {torch.cuda.get_device_name(device)}")
    if args.calibrate_copy:
        # A plain copy whose HBM traffic is known (256 MiB read, 256 MiB written per dispatch): the
        # FETCH_SIZE / WRITE_SIZE counters of these dispatches give the counters' scale.
        n = 256 * 1024**2
        src = torch.empty(n // 4, dtype=torch.int32, device=device).random_()
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibrate-copy: 10 copies of {n} bytes")
        return

    if args.config:
        # one workload alone, as a profiler run needs it
        if args.config == "D256":
            print(json.dumps({"config": "D256", **wide_extras(min(args.steps, 20), device)}), flush=True)
            return
        if args.config in DECODE:
            r = time_decode(DECODE[args.config], args.steps, args.warmup, device)
            out = {"config": args.config, "gbs": round(r["gbs"], 1), "frac": round(r["gbs"] / PEAK_HBM_GBS, 4),
                   "us_per_step": round(r["ms_per_step"] * 1e3, 3), "kernel_us": round(r["call_us_mean"], 3),
                   "bytes": r["bytes"]}
        else:
            cfg = PREFILL if args.config == "C3" else PREFILL_C5[args.config]
            r = time_prefill(cfg, max(1, min(args.steps, 3)), args.warmup, device)
            out = {"config": args.config, "attn_tflops": round(r["attn_tflops"], 2),
                   "frac": round(r["attn_tflops"] / PEAK_MFMA_TFLOPS, 4), "attn_ms": round(r["attn_ms"], 4),
                   "flops": r["flops"]}
        print(json.dumps(out), flush=True)
        return

    prefill = None
    if not args.no_prefill:
        pr = time_prefill(PREFILL, max(1, min(args.steps, 3)), args.warmup, device, want_parity=not args.no_parity)
        log(f"[bench] C3 prefill: {pr['tflops']:.1f} TFLOP/s whole step ({pr['ms_per_step']:.3f} ms incl. appends); "
            f"attention kernels {pr['attn_ms']:.3f} ms -> {pr['attn_tflops']:.1f} TFLOP/s; appends {pr['append_ms']:.3f} ms")
        pcpu = None
        if not args.no_cpu and "cpu_inputs" in pr:
            pcpu, faithful = prefill_cpu_baseline(PREFILL, *pr["cpu_inputs"])
            add_faithful(pr.get("parity"), pr.get("parity_arrays"), faithful)
            log(f"[bench] C3 CPU baseline: {pcpu['value']} TFLOP/s on {pcpu['cores']} cores")
        prefill = {
            "metric": "prefill TFLOP/s (% MFMA)",
            "value": round(pr["tflops"], 2),
            "unit": "TFLOP/s",
            "ms_per_step": round(pr["ms_per_step"], 4),
            "config": {"workload": "C3 chunked prefill (Qwen3-30B-A3B shapes): B=1, Hq=32, Hkv=4, D=128, 16384-token "
                                   "prompt in 32 chunks of 512, each quantize-appended (8-bit, G=64) then causal "
                                   "attention over all prior keys, bf16",
                       "flops_per_step": pr["flops"], "steps": max(1, min(args.steps, 3))},
            "roofline": {"bound": "mfma", "achieved": round(pr["attn_tflops"], 2), "peak": PEAK_MFMA_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(pr["attn_tflops"] / PEAK_MFMA_TFLOPS, 4),
                         "traffic": measured_traffic("prefill_c3_chunk"),
                         "kernel_ms": round(pr["attn_ms"], 4),
                         "kernel": "prefill_attn_kernel (one launch per chunk; split keys are merged inside it), "
                                   "summed over the 32 chunks: the timed step's graph minus a graph of its "
                                   "appends alone"},
            "append_ms": round(pr["append_ms"], 4),
            "attn_alone_ms": round(pr["attn_alone_ms"], 4),
            "attn_events_ms": round(pr["attn_events_ms"], 4),
            "chunk_attn_us": pr["chunk_attn_us"],
            "cpu_baseline": pcpu,
            "parity": pr.get("parity"),
        }
        torch.cuda.empty_cache()
        if args.prefill_only:
            print(json.dumps({"metric": prefill["metric"], "value": prefill["value"], "unit": "TFLOP/s", "n_gpus": 1,
                              "higher_is_better": True, "prefill": prefill}), flush=True)
            return

    head = DECODE["C2-b1"]
    res = time_decode(head, args.steps, args.warmup, device, want_parity=not args.no_parity)
    log(f"[bench] C2-b1: {res['gbs']:.1f} GB/s (graph, {res['ms_per_step'] * 1e3:.2f} us/step); "
        f"per call {res['call_us_mean']:.2f} us mean -> {res['kernel_gbs']:.1f} GB/s")
    extra = {}
    if not args.no_extra:
        for name in ("C1", "C2-b8", "C2-tp8", "C4", "C5-global", "C5-window", "C5-window-dense"):
            cfg = DECODE[name]
            quantized = cfg["bits"] != 16
            r = time_decode(cfg, args.steps, args.warmup, device, want_parity=True)
            extra[name] = {"gbs": round(r["gbs"], 1), "frac": round(r["gbs"] / PEAK_HBM_GBS, 4),
                           "us_per_step": round(r["ms_per_step"] * 1e3, 3), "bytes": r["bytes"],
                           "kernel_us": round(r["call_us_mean"], 3), "parity": r.get("parity")}
            log(f"[bench] {name}: {r['gbs']:.1f} GB/s ({r['ms_per_step'] * 1e3:.2f} us/step)")
            if quantized and not args.no_cpu:
                q, cache, scale = r["cpu_inputs"]
                c, faithful = cpu_baseline(cfg, q, cache, scale, r["seq_lens"], budget_s=6.0, max_calls=5)
                add_faithful(extra[name]["parity"], r.get("parity_arrays"), faithful)
                extra[name]["cpu_baseline"] = c
                log(f"[bench] {name} CPU baseline: {c['value']} GB/s on {c['cores']} cores")
            del r
            torch.cuda.empty_cache()
        for name, cfg in PREFILL_C5.items():
            pr = time_prefill(cfg, 1, max(1, args.warmup // 10), device, want_parity=not args.no_parity)
            e = {"tflops": round(pr["tflops"], 2), "attn_tflops": round(pr["attn_tflops"], 2),
                 "frac": round(pr["attn_tflops"] / PEAK_MFMA_TFLOPS, 4), "ms_per_step": round(pr["ms_per_step"], 4),
                 "attn_ms": round(pr["attn_ms"], 4), "append_ms": round(pr["append_ms"], 4),
                 "flops": pr["flops"], "chunk_attn_us": pr["chunk_attn_us"], "parity": pr.get("parity")}
            if not args.no_cpu and "cpu_inputs" in pr:
                c, faithful = prefill_cpu_baseline(cfg, *pr["cpu_inputs"], budget_s=10.0)
                add_faithful(e["parity"], pr.get("parity_arrays"), faithful)
                e["cpu_baseline"] = c
            extra[name] = e
            log(f"[bench] {name}: {pr['attn_tflops']:.1f} TFLOP/s attention ({pr['attn_ms']:.3f} ms), "
                f"{pr['tflops']:.1f} TFLOP/s whole step")
            del pr
            torch.cuda.empty_cache()
        r = time_paged_decode(DECODE["C2-b8"], args.steps, args.warmup, device)
        extra["C2-b8-paged"] = {"gbs": round(r["gbs"], 1), "frac": round(r["gbs"] / PEAK_HBM_GBS, 4),
                                "us_per_step": round(r["ms_per_step"] * 1e3, 3), "bytes": r["bytes"],
                                "parity": r["parity"]}
        log(f"[bench] C2-b8-paged: {r['gbs']:.1f} GB/s ({r['ms_per_step'] * 1e3:.2f} us/step)")
        torch.cuda.empty_cache()
        for name, r in append_extras(device).items():
            extra["C3-chunk-" + name] = r
            log(f"[bench] C3-chunk-{name}: {r['us_per_call']:.2f} us/call on the device ({r['gbs']:.0f} GB/s); "
                f"{r['host_us_per_eager_call']:.1f} us of host time per eager call")
        for name, r in dense_prefill_extras(min(args.steps, 20), device).items():
            extra[name] = r
            log(f"[bench] {name}: {r['tflops']:.1f} TFLOP/s ({r['us_per_call']:.1f} us/call)")
        torch.cuda.empty_cache()
        for name, r in wide_extras(min(args.steps, 20), device).items():
            extra[name] = r
            log(f"[bench] {name}: " + (f"{r['tflops']:.1f} TFLOP/s ({r['us_per_call']:.1f} us/call)" if "tflops" in r
                                       else f"{r['gbs']:.1f} GB/s ({r['us_per_step']:.2f} us/step)"))
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        q, cache, scale = res["cpu_inputs"] if "cpu_inputs" in res else (None, None, None)
        if q is None:
            r2 = time_decode(head, 1, 0, device, want_parity=True)
            q, cache, scale = r2["cpu_inputs"]
        cpu, faithful = cpu_baseline(head, q, cache, scale, seq_lens_of(head))
        add_faithful(res.get("parity"), res.get("parity_arrays"), faithful)
        log(f"[bench] CPU baseline: {cpu['value']} GB/s on {cpu['cores']} cores")

    achieved = res["kernel_gbs"]
    read_ref = plain_read_reference(res["bytes"], args.steps, device)
    log(f"[bench] plain read of {res['bytes']} B: torch sum {read_ref['torch_sum_us']} us "
        f"({read_ref['torch_sum_gbs']} GB/s), torch copy {read_ref['torch_copy_gbs']} GB/s")
    line = {
        "metric": METRIC,
        "value": round(res["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) fp16 Q/K/V; K/V quantized to 8-bit affine (G=64) by the append kernel",
        "config": {
            "workload": "C2 decode attention (Qwen3-32B shapes): B=1, Hq=64, Hkv=8, D=128, S=32768, "
                        "8-bit affine KV, group 64, fp16 query/scales/output, 1 query token",
            "B": 1, "Hq": 64, "Hkv": 8, "head_dim": 128, "context": 32768, "kv_bits": 8, "group_size": 64,
            "bytes_per_step": res["bytes"], "caches_rotated": res["ncache"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic("decode_c2_b1"),
            "kernel_us": round(res["call_us_mean"], 3),
            "kernel": "decode_attn_kernel + combine_kernel (the two launches of one kvq_decode_attn call)",
            "plain_read_reference": read_ref,
        },
        "cpu_baseline": cpu,
        "parity": res.get("parity"),
        "prefill": prefill,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
