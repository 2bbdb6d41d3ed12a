"""HIP-graph capture of the prepared entry points (the bench's timed region, and the serving use that
``AttentionCall`` and ``AppendCall`` are built for): a graph holding a quantize-append of new rows
and the attention call that reads the cache is replayed several times, with the program's own eager
work and synchronisations between the replays, and every replay is checked bit for bit against the
same calls run eagerly.

The plans cover both decode split merges (the in-kernel merge, whose arrival counters each call
leaves at zero, and the combine launch), the prefill kernel's in-kernel split merge, and a
serving step over paged pools (per-sequence append positions and lengths read on the device).
Nothing in the graphs is a memset: the workspaces are zeroed once, when they are allocated,
outside the capture.
"""

import math

import pytest
import torch

from myinfer_amd import kernels
from tests.helpers import seeded_normal

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cache(B, Hkv, cap, D, bits, dtype, group=64):
    codes = torch.zeros((B, Hkv, cap, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
    sc = torch.zeros((B, Hkv, cap, D // group), dtype=dtype, device=DEV)
    return codes, sc, torch.zeros_like(sc)


def _view(tr, S):
    return tuple(x[:, :, :S] for x in tr)


@pytest.mark.parametrize("name,B,Hq,Hkv,S,L,kernel,dtype", [
    ("decode, in-kernel merge", 8, 64, 8, 4096, 1, "decode", torch.float16),
    ("decode, combine launch", 1, 16, 8, 6000, 1, "decode", torch.bfloat16),
    ("prefill, split merge", 1, 32, 4, 4096, 256, "prefill", torch.bfloat16),
])
def test_graph_replays_match_eager(name, B, Hq, Hkv, S, L, kernel, dtype):
    print(f"graph replay: {name} B={B} Hq={Hq} Hkv={Hkv} S={S} L={L} {dtype}", flush=True)
    D, bits = 128, 8
    scale = 1.0 / math.sqrt(D)
    kt, vt = _cache(B, Hkv, S + 64, D, bits, dtype), _cache(B, Hkv, S + 64, D, bits, dtype)
    # the history, appended eagerly; the graph appends rows [S - L, S) and attends to all S
    kernels.quantize_append(seeded_normal((B, Hkv, S - L, D), 1300, dtype, DEV), kt,
                            seeded_normal((B, Hkv, S - L, D), 1301, dtype, DEV), vt, row_offset=0, bits=bits)
    new_k = seeded_normal((B, Hkv, L, D), 1302, dtype, DEV)
    new_v = seeded_normal((B, Hkv, L, D), 1303, dtype, DEV)
    q = seeded_normal((B, Hq, L, D), 1304, dtype, DEV)
    out = torch.empty((B, Hq, L, D), dtype=dtype, device=DEV)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        # prepared calls launch on the stream current at preparation: the capture stream
        app = kernels.prepare_append(kt, vt, bits=bits)
        att = kernels.prepare_attention(q, _view(kt, S), _view(vt, S), scale, causal=True, bits=bits, out=out,
                                        kernel=kernel)
        app(new_k, new_v, S - L)  # warm-up on the capture stream
        att()
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        app(new_k, new_v, S - L)
        att()

    for r in range(4):
        # the program's eager work between replays: new rows and queries written in place, and an
        # unrelated eager attention call with a plan of its own
        new_k.copy_(seeded_normal((B, Hkv, L, D), 1310 + r, dtype, DEV))
        new_v.copy_(seeded_normal((B, Hkv, L, D), 1320 + r, dtype, DEV))
        q.copy_(seeded_normal((B, Hq, L, D), 1330 + r, dtype, DEV))
        other = kernels.attention(q[:, :, :1], _view(kt, S // 2), _view(vt, S // 2), scale, bits=bits)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got_out = out.clone()
        got_rows = [x[:, :, S - L:S].clone() for x in (*kt, *vt)]
        # the same calls, eagerly: the append rewrites the same rows, the attention goes to a new
        # output
        kernels.quantize_append(new_k, kt, new_v, vt, row_offset=S - L, bits=bits)
        ref_out = kernels.attention(q, _view(kt, S), _view(vt, S), scale, causal=True, bits=bits, kernel=kernel)
        torch.cuda.synchronize()
        for a, x in zip(got_rows, (*kt, *vt)):
            assert torch.equal(a.view(torch.int16) if a.dtype != torch.uint32 else a.view(torch.int32),
                               x[:, :, S - L:S].view(torch.int16) if x.dtype != torch.uint32
                               else x[:, :, S - L:S].view(torch.int32)), f"replay {r}: appended rows differ"
        assert torch.equal(got_out, ref_out), f"replay {r}: the graph's attention differs from the eager call"
        assert torch.isfinite(other).all()
    del graph


def test_paged_decode_step_replays_match_eager():
    """A serving step over paged pools captured as one graph: each sequence's new token appended at
    its own position (starts) and the paged decode over seq_lens = starts + 1. New tokens and
    queries are written in place between replays; every replay equals the same calls run eagerly,
    bit for bit, and reads no poisoned pool row."""
    from tests.test_gpu_paged import build

    print("graph replay: paged decode step", flush=True)
    B, Hq, Hkv, D, bits, dtype = 3, 16, 4, 128, 8, torch.float16
    lens = [700, 300, 65]  # the next row of each sequence lies in its last page
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 1350)
    starts = torch.tensor(lens, dtype=torch.int32, device=DEV)
    seq = starts + 1
    S = max(lens) + 1
    new_k = seeded_normal((B, Hkv, 1, D), 1351, dtype, DEV)
    new_v = seeded_normal((B, Hkv, 1, D), 1352, dtype, DEV)
    q = seeded_normal((B, Hq, 1, D), 1353, dtype, DEV)
    out = torch.empty((B, Hq, 1, D), dtype=dtype, device=DEV)

    def step(dst):
        kernels.paged_quantize_append(new_k, kp, new_v, vp, tables, starts=starts, bits=bits)
        return kernels.paged_attention(q, kp, vp, tables, seq, 0.1, causal=True, bits=bits, max_len=S, out=dst,
                                       kernel="decode")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(out)  # warm-up on the capture stream: its workspace is allocated and zeroed here
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        step(out)

    for r in range(4):
        new_k.copy_(seeded_normal((B, Hkv, 1, D), 1360 + r, dtype, DEV))
        new_v.copy_(seeded_normal((B, Hkv, 1, D), 1370 + r, dtype, DEV))
        q.copy_(seeded_normal((B, Hq, 1, D), 1380 + r, dtype, DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref = step(None)  # the same calls, eagerly, into a new output
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all(), f"replay {r}: a poisoned pool row was read"
        assert torch.equal(got, ref), f"replay {r}: the graph's paged decode differs from the eager call"
    del graph
