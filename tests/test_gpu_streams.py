"""Attention calls on several streams at once. The Python layer keeps one workspace per (device,
stream), so calls that run concurrently on different streams never share split partials or
arrival counters: two streams alternate decode calls (combine launch and in-kernel merge) and
prefill calls with no synchronisation between them, and every output equals the same call made
alone on the default stream."""

import torch
import pytest

from myinfer_amd import kernels
from tests.helpers import seeded_normal
from tests.test_gpu_decode import make_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_concurrent_streams_match_serial_calls():
    print("two streams, interleaved decode and prefill calls", flush=True)
    D, bits, dtype = 128, 8, torch.bfloat16
    # decode with the combine launch (32 splits) and with the in-kernel merge (few splits), and a
    # split prefill chunk
    shapes = [("decode", 1, 64, 8, 1, 32768), ("decode", 8, 32, 8, 1, 4096), ("prefill", 1, 32, 4, 512, 8192)]
    cases = []
    for i, (kernel, B, Hq, Hkv, L, S) in enumerate(shapes):
        kt, vt = make_cache(B, Hkv, S, D, bits, dtype, 1500 + i)
        qs = [seeded_normal((B, Hq, L, D), 1510 + 10 * i + j, dtype, DEV) for j in range(2)]
        cases.append((kernel, kt, vt, qs))
    ref = [[kernels.attention(q, kt, vt, 0.09, causal=True, bits=bits, kernel=kernel) for q in qs]
           for kernel, kt, vt, qs in cases]
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[[] for _ in cases] for _ in streams]
    for rep in range(3):
        for c, (kernel, kt, vt, qs) in enumerate(cases):
            for j, s in enumerate(streams):
                with torch.cuda.stream(s):
                    outs[j][c].append(kernels.attention(qs[j], kt, vt, 0.09, causal=True, bits=bits, kernel=kernel))
    torch.cuda.synchronize()
    for j in range(len(streams)):
        for c in range(len(cases)):
            for o in outs[j][c]:
                assert torch.equal(o, ref[c][j]), f"stream {j}, case {c}: differs from the serial call"
