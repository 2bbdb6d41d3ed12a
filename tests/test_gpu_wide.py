"""GPU attention through wide_attn_kernel vs the exact fp64 oracle.

Head_dim 256 is the Gemma family's width (Gemma-2 and the smaller Gemma-3 models). The kernel
serves prefill over quantized caches (4/8-bit, groups 64 and 128) and every call, decode included,
over unquantized caches (the plain cache before quantized_kv_start and the sliding-window layers).
At head_dim 64 (Llama-3.2-1B, Qwen2.5-0.5B) it serves prefill over unquantized caches.
Covers GQA ratios, causal / full / sliding-window masks, variable-length batches, ragged query and
key counts (partial tiles and row blocks, row blocks spanning two heads), capacity-padded views,
split key ranges merged by combine_kernel, a Gemma-3-12B prefill chunk, and the public API's
dispatch. Bars as for the other kernels (tests/helpers.py).
"""

import math

import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd import kernels
from tests.helpers import assert_close, exact_reference, seeded_normal
from tests.test_gpu_decode import make_cache
from tests.test_gpu_dense import exact, make_kv

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 256


def quant_case(B, Hq, Hkv, L, S, bits, dtype, *, group=64, causal=True, window=0, seq_lens=None, seed=0, cap=None,
               what=""):
    print(f"wide quantized case {what} B={B} Hq={Hq} Hkv={Hkv} L={L} S={S} bits={bits} group={group} {dtype} "
          f"causal={causal} window={window} var={seq_lens is not None}", flush=True)
    kt, vt = make_cache(B, Hkv, S, D, bits, dtype, seed, cap=cap, group=group)
    q = seeded_normal((B, Hq, L, D), seed + 2, dtype, DEV)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, causal=causal, window=window, seq_lens=sl, bits=bits, group_size=group,
                            kernel="prefill")
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, scale, bits=bits, group_size=group, causal=causal, window=window, seq_lens=sl)
    return assert_close(out, ref, what)


def dense_case(kernel, B, Hq, Hkv, L, S, dtype, *, causal=False, window=0, seq_lens=None, seed=0, cap=None, what="",
               head_dim=D):
    print(f"wide dense {kernel} case {what} B={B} Hq={Hq} Hkv={Hkv} L={L} S={S} D={head_dim} {dtype} causal={causal} "
          f"window={window} var={seq_lens is not None}", flush=True)
    k, v = make_kv(B, Hkv, S, head_dim, dtype, seed, cap=cap)
    q = seeded_normal((B, Hq, L, head_dim), seed + 2, dtype, DEV)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(head_dim)
    out = kernels.attention(q, k, v, scale, causal=causal, window=window, seq_lens=sl, kernel=kernel)
    torch.cuda.synchronize()
    ref = exact(q, k, v, scale, causal=causal, window=window, seq_lens=sl)
    return assert_close(out, ref, f"wide dense {kernel} {what}")


# ---- quantized caches (prefill)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [64, 128])
def test_quantized_bits_groups(dtype, bits, group):
    quant_case(1, 8, 4, 150, 1300, bits, dtype, group=group, seed=10 + bits + group, what="bits-groups")


@pytest.mark.parametrize("Hq,Hkv", [(4, 4), (8, 4), (16, 8), (16, 2)])
def test_quantized_gqa(Hq, Hkv):
    quant_case(1, Hq, Hkv, 96, 700, 8, torch.float16, seed=30 + Hq + Hkv, what="gqa")


@pytest.mark.parametrize("L,S", [(2, 2), (5, 40), (33, 33), (65, 300), (129, 129), (200, 2048)])
def test_quantized_ragged(L, S):
    # partial tiles and row blocks; L = 65 and 129 put row blocks across two heads
    quant_case(1, 8, 4, L, S, 8, torch.float16, seed=L + S, what="ragged-causal")
    quant_case(2, 6, 2, L, S, 4, torch.bfloat16, causal=False, seed=L + S + 1, what="ragged-full")


def test_quantized_window_varlen_capacity():
    quant_case(2, 8, 2, 33, 5000, 8, torch.float16, window=1024, seq_lens=[5000, 700], seed=41, what="window-varlen")
    quant_case(3, 8, 4, 40, 900, 4, torch.bfloat16, seq_lens=[900, 41, 333], seed=42, cap=1280, what="varlen-cap")
    quant_case(1, 16, 8, 300, 3000, 8, torch.bfloat16, window=512, seed=43, group=128, what="window")


def test_quantized_long_split():
    # few row blocks over a long key range: the keys split over workgroups and combine_kernel merges
    quant_case(1, 8, 4, 16, 12000, 8, torch.float16, seed=51, what="split-f16")
    quant_case(1, 4, 2, 7, 9000, 4, torch.bfloat16, causal=False, seed=52, group=128, what="split-bf16")


def test_quantized_gemma3_chunk():
    # Gemma-3-12B attention (16 query / 8 KV heads, head_dim 256): a 512-token chunk over 4096 keys
    quant_case(1, 16, 8, 512, 4096, 8, torch.bfloat16, seed=61, what="gemma3-12b-chunk")


# ---- unquantized caches (decode and prefill)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,S", [(8, 4, 3000), (16, 8, 777), (4, 1, 33), (16, 16, 4097)])
def test_dense_decode(dtype, Hq, Hkv, S):
    dense_case("decode", 2, Hq, Hkv, 1, S, dtype, seed=70 + Hq + S, what="decode")


def test_dense_decode_window_varlen_capacity():
    dense_case("decode", 3, 8, 4, 1, 3000, torch.bfloat16, window=1024, seq_lens=[3000, 1, 1777], seed=81,
               what="decode-window")
    dense_case("decode", 2, 16, 8, 3, 2000, torch.float16, causal=True, seq_lens=[2000, 5], seed=82, cap=2304,
               what="decode-rows-cap")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("L,S,causal,window", [(150, 1300, True, 0), (64, 64, True, 0), (100, 2100, False, 0),
                                               (300, 3000, True, 1024), (7, 9000, True, 0)])
def test_dense_prefill(dtype, L, S, causal, window):
    dense_case("prefill", 1, 8, 4, L, S, dtype, causal=causal, window=window, seed=90 + L + S, what="prefill")


def test_dense_gemma3_window_chunk():
    # a sliding-window layer of Gemma-3-12B: 512 queries, window 1024, after 3584 earlier tokens
    dense_case("prefill", 1, 16, 8, 512, 4096, torch.bfloat16, causal=True, window=1024, seed=95, what="gemma3-window")


# ---- unquantized caches at head_dim 64 (prefill)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Hq,Hkv,L,S,causal,window", [(32, 8, 150, 1300, True, 0), (8, 8, 64, 64, True, 0),
                                                      (14, 2, 100, 2100, False, 0), (16, 4, 300, 3000, True, 1024),
                                                      (8, 2, 7, 9000, True, 0), (32, 8, 33, 5000, True, 0)])
def test_dense_prefill_head_dim_64(dtype, Hq, Hkv, L, S, causal, window):
    dense_case("prefill", 1, Hq, Hkv, L, S, dtype, causal=causal, window=window, seed=110 + L + S, what="d64",
               head_dim=64)


def test_dense_head_dim_64_varlen_capacity_and_dispatch():
    dense_case("prefill", 3, 16, 4, 40, 900, torch.bfloat16, causal=True, seq_lens=[900, 41, 333], seed=121, cap=1280,
               what="d64-varlen-cap", head_dim=64)
    # the public entry point sends a head_dim-64 prompt chunk over an unquantized cache here
    k, v = make_kv(1, 8, 600, 64, torch.float16, 122)
    q = seeded_normal((1, 32, 128, 64), 124, torch.float16, DEV)
    call = kernels.prepare_attention(q, k, v, 0.125, causal=True)
    assert call.symbol == "kvq_prefill_attn_dense"
    out = call()
    torch.cuda.synchronize()
    assert_close(out, exact(q, k, v, 0.125, causal=True), "d64 dispatch")


# ---- the public API routes head_dim 256 here


def test_api_dispatch_head_dim_256():
    print("wide case api dispatch", flush=True)
    torch.manual_seed(0)
    B, Hq, Hkv, L, S = 1, 8, 4, 64, 700
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 5, group=64)
    q = seeded_normal((B, Hq, L, D), 7, torch.float16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = A.blocked_quantized_sdpa(q, kt, vt, scale, "causal", group_size=64, bits=8)
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, scale, bits=8, group_size=64, causal=True)
    assert_close(out, ref, "api d256 prefill")
    call = kernels.prepare_attention(q, kt, vt, scale, causal=True, bits=8)
    assert call.kernel == "prefill" and call.symbol == "kvq_prefill_attn"
    k, v = make_kv(B, Hkv, S, D, torch.float16, 8)
    call = kernels.prepare_attention(q[:, :, :1], k, v, scale)
    assert call.symbol == "kvq_decode_attn_dense"
    o1 = call()
    torch.cuda.synchronize()
    assert_close(o1, exact(q[:, :, :1], k, v, scale), "api d256 dense decode")


def test_shared_workspace_keeps_counters_zero():
    # the split partials sit past the arrival-counter block that the other kernels' in-kernel merges
    # count in; a head_dim-256 split call leaves it zero, so a D=128 prefill and a fused decode on the
    # same cached workspace stay exact
    from tests import test_gpu_decode as TD
    from tests import test_gpu_prefill as TP

    print("wide case shared workspace", flush=True)
    quant_case(1, 8, 4, 16, 12000, 8, torch.float16, seed=53, what="split-before-shared")
    dev = torch.device(DEV)
    ws = kernels._workspace(dev, kernels._lib.stream_ptr(dev), 1)
    nctr = 65536  # the counter block's 32-bit words (merge.h kMaxCountedUnits)
    assert int(ws.view(torch.int32)[:nctr].abs().sum().item()) == 0
    TP.run_case(1, 8, 2, 40, 9000, 8, torch.float16, seed=54, what="d128-after-wide")
    TD.run_case(4, 32, 16, 1, 4000, 128, 8, torch.bfloat16, seed=55, what="fused-decode-after-wide")
