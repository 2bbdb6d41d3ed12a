"""GPU split-K decode attention vs the exact fp64 oracle over the dequantized cache.

Caches are filled by the quantize kernel (bit-exact with the oracle, see test_gpu_quantize.py);
the oracle dequantizes the very triples the kernel reads. Covers GQA ratios 1..8, head_dim 64 and
128, 4- and 8-bit, fp16/bf16, ragged key counts (tile and split tails), variable-length batches,
sliding windows, several query rows (L > 1, causal), capacity-padded cache views, and the
BASELINE decode configurations at full size.
"""

import math

import pytest
import torch

from myinfer_amd import kernels
from tests.helpers import assert_close, exact_reference, seeded_normal

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_cache(B, Hkv, S, D, bits, dtype, seed, cap=None, outliers=False, group=64):
    cap = cap or S
    k = seeded_normal((B, Hkv, S, D), seed, torch.float32)
    if outliers:
        # 1% of the channels of every KV head at 8x magnitude (RoPE'd-K stress, C4)
        g = torch.Generator().manual_seed(seed + 7)
        nch = max(1, round(0.01 * D))
        for h in range(Hkv):
            ch = torch.randperm(D, generator=g)[:nch]
            k[:, h, :, ch] *= 8.0
    k = k.to(dtype).to(DEV)
    v = seeded_normal((B, Hkv, S, D), seed + 1, dtype, DEV)
    trip = []
    for x in (k, v):
        codes = torch.zeros((B, Hkv, cap, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
        sc = torch.zeros((B, Hkv, cap, D // group), dtype=dtype, device=DEV)
        bi = torch.zeros_like(sc)
        kernels.quantize_append(x, (codes, sc, bi), row_offset=0, group_size=group, bits=bits)
        trip.append((codes[:, :, :S], sc[:, :, :S], bi[:, :, :S]))
    return trip[0], trip[1]


def run_case(B, Hq, Hkv, L, S, D, bits, dtype, *, causal=False, window=0, seq_lens=None, seed=0, cap=None,
             outliers=False, group=64, what=""):
    print(f"decode case {what} B={B} Hq={Hq} Hkv={Hkv} L={L} S={S} D={D} bits={bits} group={group} {dtype} "
          f"causal={causal} window={window} var={seq_lens is not None}", flush=True)
    kt, vt = make_cache(B, Hkv, S, D, bits, dtype, seed, cap=cap, outliers=outliers, group=group)
    q = seeded_normal((B, Hq, L, D), seed + 2, dtype, DEV)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, causal=causal, window=window, seq_lens=sl, bits=bits,
                            group_size=group, kernel="decode")
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, scale, bits=bits, group_size=group, causal=causal, window=window, seq_lens=sl)
    return assert_close(out, ref, what)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (64, 8)])
def test_gqa_ratios(dtype, bits, Hq, Hkv):
    run_case(1, Hq, Hkv, 1, 1000, 128, bits, dtype, seed=10 + Hq, what="gqa")


@pytest.mark.parametrize("S", [1, 2, 31, 32, 33, 100, 511, 513, 4097])
def test_ragged_lengths(S):
    run_case(1, 16, 2, 1, S, 128, 8, torch.float16, seed=S, what="ragged")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("Hq,Hkv,L", [(4, 4, 1), (8, 2, 1), (16, 4, 1), (4, 4, 6), (8, 2, 6)])
def test_head_dim_64(bits, Hq, Hkv, L):
    # the shapes of the reference's own test (tests/test_core.py:27: D=64, S=700, L=6)
    run_case(1, Hq, Hkv, L, 700, 64, bits, torch.float16, causal=L > 1, seed=L + Hq, what="d64")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group,D", [(32, 128), (128, 128), (32, 64)])
@pytest.mark.parametrize("Hq,Hkv,L,S", [(8, 1, 1, 1000), (16, 2, 1, 4097), (4, 4, 1, 33), (8, 2, 3, 700)])
def test_group_sizes(dtype, bits, group, D, Hq, Hkv, L, S):
    # 32 and 128 are mlx's other group sizes; a pass then serves 16*group/D query rows
    run_case(2, Hq, Hkv, L, S, D, bits, dtype, causal=L > 1, seed=400 + group + S, group=group, what="group")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("Hq,Hkv,L,S", [(8, 1, 1, 1000), (16, 2, 1, 4097), (4, 4, 1, 33), (8, 2, 3, 700)])
def test_head_dim_256(dtype, bits, group, Hq, Hkv, L, S):
    # head_dim 256 (Gemma-style): a pass serves 16*group/256 query rows
    run_case(2, Hq, Hkv, L, S, 256, bits, dtype, causal=L > 1, seed=700 + group + S, group=group, what="d256")


def test_head_dim_256_window_lengths_and_prompt():
    run_case(3, 16, 2, 1, 3000, 256, 8, torch.bfloat16, window=700, seq_lens=[3000, 1, 1777], seed=81, group=64,
             what="d256-window")
    # a prompt chunk: many query rows take many decode passes over the keys
    run_case(1, 8, 4, 70, 900, 256, 4, torch.float16, causal=True, seed=82, group=64, what="d256-chunk")


def test_group_sizes_window_and_lengths():
    run_case(3, 16, 2, 1, 3000, 128, 4, torch.float16, window=700, seq_lens=[3000, 1, 1777], seed=77, group=32,
             what="group32-window")
    run_case(3, 32, 4, 1, 3000, 128, 8, torch.bfloat16, window=513, seq_lens=[2, 3000, 999], seed=78, group=128,
             what="group128-window")


@pytest.mark.parametrize("L,Hq,Hkv", [(2, 8, 2), (4, 8, 4), (3, 4, 2), (2, 16, 2)])
def test_multi_query_causal(L, Hq, Hkv):
    # rows = (Hq/Hkv)*L up to 16: one or two passes of 8 rows
    run_case(2, Hq, Hkv, L, 777, 128, 8, torch.float16, causal=True, seed=50 + L, what="multi-query")


def test_variable_lengths_and_window():
    run_case(3, 16, 4, 1, 3000, 128, 8, torch.bfloat16, seq_lens=[3000, 17, 1500], causal=True, seed=5,
             what="varlen")
    run_case(2, 16, 8, 1, 5000, 128, 8, torch.float16, causal=True, window=1024, seed=6, what="window")
    run_case(2, 8, 2, 3, 2000, 128, 4, torch.float16, causal=True, window=100, seq_lens=[2000, 150], seed=7,
             what="window-varlen")


def test_capacity_padded_views():
    # cache views [..., :S, :] of larger buffers (the layout QuantizedKVCache.update_and_fetch returns)
    run_case(2, 16, 8, 1, 1000, 128, 8, torch.float16, cap=1280, seed=8, what="padded")
    run_case(1, 8, 2, 1, 4097, 128, 4, torch.bfloat16, cap=4352, seed=9, what="padded-4bit")


@pytest.mark.parametrize("name", ["C1", "C2-b1", "C2-b8", "C2-tp8", "C4", "C5-decode"])
def test_baseline_configs(name):
    if name == "C1":
        # Qwen3-0.6B shapes, 4096 cached + 1 appended token
        st = run_case(1, 16, 8, 1, 4097, 128, 8, torch.float16, seed=1001, what=name)
    elif name == "C2-b1":
        st = run_case(1, 64, 8, 1, 32768, 128, 8, torch.float16, seed=1002, what=name)
    elif name == "C2-b8":
        g = torch.Generator().manual_seed(1002)
        lens = torch.randint(16384, 32769, (8,), generator=g).tolist()
        st = run_case(8, 64, 8, 1, 32768, 128, 8, torch.float16, seq_lens=lens, seed=1012, what=name)
    elif name == "C2-tp8":
        # one GPU's share of C2 at tensor parallelism 8: one KV head, so the keys split 128 ways
        st = run_case(1, 8, 1, 1, 32768, 128, 8, torch.float16, seed=1013, what=name)
    elif name == "C4":
        st = run_case(1, 64, 8, 1, 131072, 128, 4, torch.float16, seed=1004, outliers=True, what=name)
    else:
        # Gemma-3-27B decode step after an 8192-token prefill: a global and a window-1024 layer
        st = run_case(4, 32, 16, 1, 8193, 128, 8, torch.bfloat16, causal=True, seed=1005, what=name + "-global")
        st = run_case(4, 32, 16, 1, 8193, 128, 8, torch.bfloat16, causal=True, window=1024, seed=1006,
                      what=name + "-window")
    print(name, st, flush=True)


def test_repeated_calls_are_bit_identical():
    """Calls of different shapes share one workspace (split counters and partials) and run back to
    back: every repetition must reproduce its first output bit for bit, which fails if the split
    merge ever reads a partial of another call or a counter is left non-zero."""
    cases = []
    for seed, (B, Hq, Hkv, S, bits, sl) in enumerate([(1, 64, 8, 32768, 8, None), (1, 16, 8, 4097, 8, None),
                                                       (3, 16, 4, 3001, 4, [3001, 17, 1500]),
                                                       (2, 8, 2, 777, 8, [700, 777])]):
        kt, vt = make_cache(B, Hkv, S, 128, bits, torch.float16, 300 + seed)
        q = seeded_normal((B, Hq, 1, 128), 400 + seed, torch.float16, DEV)
        lens = None if sl is None else torch.tensor(sl, dtype=torch.int32, device=DEV)
        call = kernels.prepare_attention(q, kt, vt, 1.0 / math.sqrt(128), seq_lens=lens, bits=bits, kernel="decode",
                                         causal=sl is not None)
        cases.append(call)
    first = [c().clone() for c in cases]
    for rep in range(25):
        for i, c in enumerate(cases):
            out = c()
            assert torch.equal(out, first[i]), f"repetition {rep}, case {i}: output changed"
    torch.cuda.synchronize()


def test_large_batch_variable_lengths():
    """32 sequences of lengths from 0 to 3000 (one empty, one of a single key) in one decode call:
    many units, split and unsplit, merged in the kernel or by the combine launch."""
    g = torch.Generator().manual_seed(1400)
    lens = torch.randint(2, 3001, (32,), generator=g).tolist()
    lens[5], lens[17], lens[30] = 0, 1, 3000
    for dtype, bits in ((torch.float16, 8), (torch.bfloat16, 4)):
        run_case(32, 32, 8, 1, 3000, 128, bits, dtype, seq_lens=lens, seed=1401 + bits, what=f"batch 32 {bits}-bit")
