"""GPU attention over an unquantized fp16/bf16 cache (kvq_decode_attn_dense, kvq_prefill_attn_dense)
vs the exact fp64 oracle, and the sliding-window cache (RotatingKVCache) driven through it.

These are the kernels behind mx.fast.scaled_dot_product_attention in the reference's stack: the
plain cache before quantized_kv_start and the sliding-window layers m5engine/attention.py:106-112
leaves unquantized. Covers decode (head_dim 64 and 128, GQA 1..8, several query rows, ragged key
counts, variable lengths, windows, capacity-padded views), prefill (GQA, causal / full, windows,
variable lengths, ragged shapes, long split key ranges) and the C5 window-layer shapes, plus
step-by-step decoding and chunked prefill through RotatingKVCache against window attention over
the whole history. Bars as for the quantized kernels (tests/helpers.py).
"""

import math

import numpy as np
import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd import kernels
from myinfer_amd.cache import KVCache, QuantizedKVCache, RotatingKVCache
from oracle import attention as OA
from tests.helpers import assert_close, seeded_normal

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_kv(B, Hkv, S, D, dtype, seed, cap=None):
    cap = cap or S
    k = torch.zeros((B, Hkv, cap, D), dtype=dtype, device=DEV)
    v = torch.zeros_like(k)
    k[:, :, :S] = seeded_normal((B, Hkv, S, D), seed, dtype, DEV)
    v[:, :, :S] = seeded_normal((B, Hkv, S, D), seed + 1, dtype, DEV)
    return k[:, :, :S], v[:, :, :S]


def exact(q, k, v, scale, **mask):
    f = lambda t: t.detach().cpu().double().numpy()  # noqa: E731
    sl = mask.pop("seq_lens", None)
    sl = None if sl is None else [int(x) for x in sl.cpu().tolist()]
    return OA.exact_attention(f(q), f(k), f(v), scale, seq_lens=sl, **mask)


def run_case(kernel, B, Hq, Hkv, L, S, D, dtype, *, causal=False, window=0, seq_lens=None, seed=0, cap=None,
             what=""):
    print(f"dense {kernel} case {what} B={B} Hq={Hq} Hkv={Hkv} L={L} S={S} D={D} {dtype} causal={causal} "
          f"window={window} var={seq_lens is not None}", flush=True)
    k, v = make_kv(B, Hkv, S, D, dtype, seed, cap=cap)
    q = seeded_normal((B, Hq, L, D), seed + 2, dtype, DEV)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, k, v, scale, causal=causal, window=window, seq_lens=sl, kernel=kernel)
    torch.cuda.synchronize()
    ref = exact(q, k, v, scale, causal=causal, window=window, seq_lens=sl)
    return assert_close(out, ref, f"dense {kernel} {what}")


# ---- decode


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 16), (64, 8)])
def test_decode_gqa(dtype, Hq, Hkv):
    run_case("decode", 1, Hq, Hkv, 1, 3000, 128, dtype, seed=Hq + Hkv, what="gqa")


@pytest.mark.parametrize("S", [1, 2, 31, 32, 33, 100, 513, 4097])
def test_decode_ragged(S):
    run_case("decode", 2, 16, 4, 1, S, 128, torch.float16, seed=S, what="ragged")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,L", [(4, 4, 1), (8, 2, 1), (16, 4, 1), (8, 2, 6)])
def test_decode_head_dim_64(dtype, Hq, Hkv, L):
    run_case("decode", 2, Hq, Hkv, L, 777, 64, dtype, causal=L > 1, seed=Hq * L, what="d64")


def test_decode_masks_and_views():
    run_case("decode", 3, 32, 16, 1, 5000, 128, torch.bfloat16, seq_lens=[5000, 1023, 1], seed=1, what="varlen")
    run_case("decode", 2, 32, 16, 1, 5000, 128, torch.bfloat16, window=1024, seed=2, what="window")
    run_case("decode", 2, 8, 2, 4, 900, 128, torch.float16, causal=True, window=100, seed=3, what="multi-row window")
    run_case("decode", 2, 16, 8, 1, 1000, 128, torch.float16, cap=1280, seed=4, what="capacity view")


# ---- prefill


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 4), (32, 4), (32, 16)])
def test_prefill_gqa(dtype, Hq, Hkv):
    run_case("prefill", 1, Hq, Hkv, 96, 700, 128, dtype, causal=True, seed=30 + Hq + Hkv, what="gqa")


@pytest.mark.parametrize("L,S", [(1, 1), (2, 2), (5, 5), (17, 40), (64, 64), (65, 300), (200, 2048)])
def test_prefill_ragged(L, S):
    run_case("prefill", 1, 8, 2, L, S, 128, torch.float16, causal=True, seed=L + S, what="ragged")


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_full_and_causal(causal):
    run_case("prefill", 2, 16, 4, 77, 1500, 128, torch.bfloat16, causal=causal, seed=9, what="mask")


def test_prefill_windows_varlen_long():
    run_case("prefill", 2, 16, 8, 300, 3000, 128, torch.bfloat16, causal=True, window=1024, seed=11, what="window")
    run_case("prefill", 3, 16, 4, 64, 2500, 128, torch.float16, causal=True, seq_lens=[2500, 900, 64], seed=12,
             what="varlen")
    run_case("prefill", 1, 32, 4, 512, 16384, 128, torch.bfloat16, causal=True, seed=13, what="long split")


def test_c5_window_layer_shapes():
    # Gemma-3-27B window layers: Hq 32, Hkv 16, window 1024, a 2048-row prefill chunk at 6144 and
    # one decode step at 8192, four sequences
    run_case("prefill", 4, 32, 16, 2048, 8192, 128, torch.bfloat16, causal=True, window=1024, seed=14,
             what="C5 window prefill")
    run_case("decode", 4, 32, 16, 1, 8192, 128, torch.bfloat16, causal=True, window=1024, seed=15,
             what="C5 window decode")


def test_rejects_bad_dense_arguments():
    q = torch.zeros((1, 8, 1, 128), dtype=torch.float16, device=DEV)
    k = torch.zeros((1, 2, 64, 128), dtype=torch.float16, device=DEV)
    with pytest.raises(ValueError):
        kernels.attention(q, k, k.to(torch.bfloat16), 0.1)
    with pytest.raises(ValueError):
        kernels.attention(q, k[:, :, :, :64], k[:, :, :, :64], 0.1)
    with pytest.raises(ValueError):
        kernels.attention(q, k, (k, k, k), 0.1)
    # no kernel past 256 dims
    q264 = torch.zeros((1, 8, 1, 264), dtype=torch.float16, device=DEV)
    k264 = torch.zeros((1, 2, 64, 264), dtype=torch.float16, device=DEV)
    with pytest.raises(NotImplementedError):
        kernels.attention(q264, k264, k264, 0.1, kernel="prefill")


# ---- the sliding-window cache through the kernels


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rotating_cache_decode_equals_window_attention(dtype):
    print(f"rotating decode {dtype}", flush=True)
    W, B, Hq, Hkv, D, T = 96, 2, 8, 4, 128, 300
    k_all = seeded_normal((B, Hkv, T, D), 41, dtype, DEV)
    v_all = seeded_normal((B, Hkv, T, D), 42, dtype, DEV)
    q_all = seeded_normal((B, Hq, T, D), 43, dtype, DEV)
    scale = 1.0 / math.sqrt(D)
    c = RotatingKVCache(W, keep=0, step=32)
    P = 40  # a prompt chunk first, then one token at a time
    c.update_and_fetch(k_all[:, :, :P], v_all[:, :, :P])
    worst = 0.0
    for t in range(P, T):
        mask = c.make_mask(1)
        kf, vf = c.update_and_fetch(k_all[:, :, t:t + 1], v_all[:, :, t:t + 1])
        out = A.scaled_dot_product_attention(q_all[:, :, t:t + 1], kf, vf, c, scale, mask)
        if t % 37 == 0 or t == T - 1:
            torch.cuda.synchronize()
            lo = max(0, t - W + 1)
            ref = exact(q_all[:, :, t:t + 1], k_all[:, :, lo:t + 1], v_all[:, :, lo:t + 1], scale)
            worst = max(worst, assert_close(out, ref, f"rotating decode t={t}")["max_abs"])
    print(f"worst max_abs {worst:.2e}", flush=True)


def test_rotating_cache_chunked_prefill_equals_window_attention():
    print("rotating chunked prefill", flush=True)
    W, B, Hq, Hkv, D, T = 256, 1, 16, 4, 128, 1100
    dtype = torch.bfloat16
    k_all = seeded_normal((B, Hkv, T, D), 51, dtype, DEV)
    v_all = seeded_normal((B, Hkv, T, D), 52, dtype, DEV)
    q_all = seeded_normal((B, Hq, T, D), 53, dtype, DEV)
    scale = 1.0 / math.sqrt(D)
    c = RotatingKVCache(W, keep=0)
    lo = 0
    for L in (300, 300, 7, 493):
        mask = c.make_mask(L)
        kf, vf = c.update_and_fetch(k_all[:, :, lo:lo + L], v_all[:, :, lo:lo + L])
        out = A.fast_scaled_dot_product_attention(q_all[:, :, lo:lo + L], kf, vf, scale, mask)
        torch.cuda.synchronize()
        # every query row sees the W newest tokens up to itself
        ref = exact(q_all[:, :, lo:lo + L], k_all[:, :, :lo + L], v_all[:, :, :lo + L], scale, causal=True, window=W)
        assert_close(out, ref, f"rotating prefill chunk at {lo}")
        lo += L


def test_dispatcher_routes_by_cache_type():
    print("sdpa dispatcher", flush=True)
    B, Hq, Hkv, L, S, D = 1, 16, 4, 1, 600, 128
    dtype = torch.float16
    k, v = make_kv(B, Hkv, S, D, dtype, 61)
    q = seeded_normal((B, Hq, L, D), 62, dtype, DEV)
    scale = 1.0 / math.sqrt(D)
    plain = KVCache()
    kf, vf = plain.update_and_fetch(k.contiguous(), v.contiguous())
    out = A.scaled_dot_product_attention(q, kf, vf, plain, scale, None)
    torch.cuda.synchronize()
    assert_close(out, exact(q, k, v, scale), "plain cache")
    qc = plain.to_quantized(group_size=64, bits=8)
    qk, qv = qc.fetch()
    out_q = A.scaled_dot_product_attention(q, qk, qv, qc, scale, None)
    ref_q = kernels.attention(q, qk, qv, scale, bits=8)
    torch.cuda.synchronize()
    assert torch.equal(out_q, ref_q)
    # quantization moves the result by at most a little
    assert float((out_q.float() - out.float()).abs().max()) < 0.05
    with pytest.raises(NotImplementedError):
        A.scaled_dot_product_attention(q, kf, vf, plain, scale, None, sinks=torch.zeros(Hq, device=DEV))
    assert isinstance(qc, QuantizedKVCache)


def test_dense_repeated_calls_are_bit_identical():
    print("dense repeat", flush=True)
    k, v = make_kv(2, 8, 3000, 128, torch.bfloat16, 71)
    q = seeded_normal((2, 32, 1, 128), 72, torch.bfloat16, DEV)
    a = kernels.attention(q, k, v, 0.08)
    b = kernels.attention(q, k, v, 0.08)
    qp = seeded_normal((2, 32, 256, 128), 73, torch.bfloat16, DEV)
    c = kernels.attention(qp, k, v, 0.08, causal=True)
    d = kernels.attention(qp, k, v, 0.08, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)
    assert np.isfinite(c.float().cpu().numpy()).all()


def test_prefill_output_views():
    """The D = 128 prefill kernel stores whole output rows 16 bytes a lane: a 16-byte aligned view
    with a row stride of D + 16 elements gets the contiguous call's bits and keeps its neighbours;
    an 8-byte aligned view is rejected by the entry point."""
    print("dense prefill output view", flush=True)
    B, Hq, Hkv, L, S, D = 1, 16, 4, 77, 700, 128  # 308 rows: a full and a partial row block
    k, v = make_kv(B, Hkv, S, D, torch.bfloat16, 74)
    q = seeded_normal((B, Hq, L, D), 75, torch.bfloat16, DEV)
    ref = kernels.attention(q, k, v, 0.09, causal=True, kernel="prefill")
    big = torch.full((B, Hq, L, D + 16), 3.0, dtype=torch.bfloat16, device=DEV)
    view = big[..., 8:8 + D]
    kernels.attention(q, k, v, 0.09, causal=True, kernel="prefill", out=view)
    torch.cuda.synchronize()
    assert torch.equal(view, ref)
    assert torch.all(big[..., :8] == 3.0) and torch.all(big[..., 8 + D:] == 3.0)
    assert_close(ref, exact(q, k, v, 0.09, causal=True), "dense prefill into a view")
    with pytest.raises(ValueError, match="16-byte aligned"):
        kernels.attention(q, k, v, 0.09, causal=True, kernel="prefill", out=big[..., 4:4 + D])


@pytest.mark.parametrize("D,L,kernel", [(128, 6, "decode"), (128, 90, "prefill"), (64, 90, "prefill"),
                                        (256, 33, "prefill")])
def test_sequences_shorter_than_the_chunk(D, L, kernel):
    """Unquantized caches: a sequence with fewer keys than the chunk has queries leaves its first
    rows at negative causal positions; they see no key and come out 0."""
    print(f"dense short sequence D={D} L={L} {kernel}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 300
    lens = [300, L // 2]
    k, v = make_kv(B, Hkv, S, D, torch.float16, 76 + D)
    q = seeded_normal((B, Hq, L, D), 77 + L, torch.float16, DEV)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = kernels.attention(q, k, v, 0.1, causal=True, seq_lens=seq, kernel=kernel)
    torch.cuda.synchronize()
    assert_close(out, exact(q, k, v, 0.1, causal=True, seq_lens=seq), f"dense short sequence D={D} {kernel}")
    assert torch.all(out[1, :, :L - lens[1]] == 0)


@pytest.mark.parametrize("D,L,kernel", [(128, 1, "decode"), (128, 64, "prefill"), (64, 64, "prefill"),
                                        (256, 20, "prefill")])
def test_empty_sequence_in_batch(D, L, kernel):
    """Unquantized caches: a batch row with seq_lens 0 returns 0 in every row."""
    print(f"dense empty sequence D={D} L={L} {kernel}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 3000
    k, v = make_kv(B, Hkv, S, D, torch.bfloat16, 78 + D)
    q = seeded_normal((B, Hq, L, D), 79 + L, torch.bfloat16, DEV)
    seq = torch.tensor([S, 0], dtype=torch.int32, device=DEV)
    out = kernels.attention(q, k, v, 0.1, causal=True, seq_lens=seq, kernel=kernel)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0)
    assert_close(out, exact(q, k, v, 0.1, causal=True, seq_lens=seq), f"dense empty sequence D={D} {kernel}")
