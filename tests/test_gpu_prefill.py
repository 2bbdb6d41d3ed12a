"""GPU chunked-prefill attention (MFMA kernel) vs the exact fp64 oracle over the dequantized cache.

Caches are filled by the quantize kernel (bit-exact with the oracle); the oracle dequantizes the
very triples the kernel reads. Covers GQA ratios 1..8, 4- and 8-bit, fp16/bf16, causal and full
masks, sliding windows, variable-length batches, ragged L and S (partial tiles and row blocks),
capacity-padded cache views, split key ranges (long contexts), and the C3 / C5 prefill shapes.
"""

import math

import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd import kernels
from tests.helpers import assert_close, exact_reference, seeded_normal
from tests.test_gpu_decode import make_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def run_case(B, Hq, Hkv, L, S, bits, dtype, *, causal=True, window=0, seq_lens=None, seed=0, cap=None, group=64,
             D=128, what=""):
    print(f"prefill case {what} B={B} Hq={Hq} Hkv={Hkv} L={L} S={S} D={D} bits={bits} group={group} {dtype} "
          f"causal={causal} window={window} var={seq_lens is not None}", flush=True)
    kt, vt = make_cache(B, Hkv, S, D, bits, dtype, seed, cap=cap, group=group)
    q = seeded_normal((B, Hq, L, D), seed + 2, dtype, DEV)
    sl = None if seq_lens is None else torch.tensor(seq_lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, kt, vt, scale, causal=causal, window=window, seq_lens=sl, bits=bits,
                            group_size=group, kernel="prefill")
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, scale, bits=bits, group_size=group, causal=causal, window=window, seq_lens=sl)
    return assert_close(out, ref, what)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (16, 4), (32, 4)])
def test_gqa_ratios(dtype, bits, Hq, Hkv):
    run_case(1, Hq, Hkv, 96, 700, bits, dtype, seed=20 + Hq + Hkv, what="gqa")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [32, 128])
def test_group_sizes(dtype, bits, group):
    run_case(2, 16, 4, 150, 1300, bits, dtype, seed=500 + group + bits, group=group, what="group")
    run_case(2, 8, 2, 33, 5000, bits, dtype, window=1024, seq_lens=[5000, 700], seed=600 + group, group=group,
             what="group-window")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [32, 64])
def test_head_dim_64(dtype, bits, group):
    # head_dim 64 (Llama-3.2-1B, Qwen2.5-0.5B shapes): half the MFMAs per tile, waves 0-3 dequantize
    run_case(2, 16, 4, 150, 1300, bits, dtype, seed=800 + group + bits, group=group, D=64, what="d64")
    run_case(2, 8, 2, 33, 5000, bits, dtype, window=1024, seq_lens=[5000, 700], seed=900 + group, group=group, D=64,
             what="d64-window")


@pytest.mark.parametrize("L,S", [(1, 1), (5, 5), (65, 300), (200, 2048)])
def test_head_dim_64_ragged_and_full(L, S):
    run_case(1, 8, 2, L, S, 8, torch.float16, seed=L + S + 64, D=64, what="d64-ragged")
    run_case(2, 14, 2, L, S, 4, torch.bfloat16, causal=False, seed=L + S + 65, D=64, what="d64-full")


def test_head_dim_64_long_context_and_auto_dispatch():
    run_case(1, 16, 4, 512, 8192, 8, torch.bfloat16, seed=66, D=64, what="d64-long")
    # kernel="auto" picks the prefill kernel for a D=64 prompt chunk
    D = 64
    kt, vt = make_cache(1, 2, 1000, D, 8, torch.float16, 67)
    q = seeded_normal((1, 8, 100, D), 68, torch.float16, DEV)
    call = kernels.prepare_attention(q, kt, vt, 0.125, causal=True, bits=8)
    assert call.kernel == "prefill"


@pytest.mark.parametrize("L,S", [(1, 1), (2, 2), (5, 5), (17, 40), (64, 64), (65, 300), (128, 1000), (200, 2048)])
def test_ragged_shapes(L, S):
    run_case(1, 8, 2, L, S, 8, torch.float16, seed=L + S, what="ragged")


@pytest.mark.parametrize("causal", [True, False])
def test_full_and_causal(causal):
    run_case(2, 16, 4, 77, 1500, 8, torch.bfloat16, causal=causal, seed=3, what="mask")


def test_windows_and_varlen():
    run_case(2, 16, 8, 300, 3000, 8, torch.bfloat16, window=1024, seed=5, what="window")
    run_case(2, 16, 8, 300, 3000, 8, torch.float16, window=100, seed=6, what="small-window")
    run_case(3, 16, 4, 64, 2500, 8, torch.float16, seq_lens=[2500, 900, 64], seed=7, what="varlen")
    run_case(2, 8, 2, 40, 1200, 4, torch.bfloat16, window=200, seq_lens=[1200, 333], seed=8, what="window-varlen")


def test_capacity_padded_views():
    run_case(1, 16, 4, 100, 1000, 8, torch.bfloat16, cap=1280, seed=9, what="padded")


def test_long_context_splits():
    # key ranges long enough to be split over several workgroups and merged
    run_case(1, 32, 4, 64, 8192, 8, torch.bfloat16, seed=10, what="split")
    run_case(1, 8, 8, 32, 6000, 4, torch.float16, causal=False, seed=11, what="split-full")


@pytest.mark.parametrize("chunk", [0, 1, 31])
def test_c3_chunk(chunk):
    # Qwen3-30B-A3B chunked prefill: 32 Q / 4 KV heads, 512-token chunks, 8-bit KV, bf16
    L = 512
    S = L * (chunk + 1)
    run_case(1, 32, 4, L, S, 8, torch.bfloat16, seed=1003 + chunk, what=f"C3-chunk{chunk}")


def test_c5_prefill_chunk():
    # Gemma-3-27B: 32 Q / 16 KV heads, a 2048-token chunk of an 8192 prefill, global and window layers
    run_case(1, 32, 16, 2048, 4096, 8, torch.bfloat16, seed=1005, what="C5-global")
    run_case(1, 32, 16, 2048, 4096, 8, torch.bfloat16, window=1024, seed=1006, what="C5-window")


def test_blocked_sdpa_string_mask_routes_to_prefill():
    # the reference's causal string mask (m5engine/attention.py:55-58) through the public entry point
    B, Hq, Hkv, L, S, D = 1, 16, 4, 48, 600, 128
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 21)
    q = seeded_normal((B, Hq, L, D), 22, torch.float16, DEV)
    out = A.blocked_quantized_sdpa(q, kt, vt, 1.0 / math.sqrt(D), "causal", 64, 8)
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, 1.0 / math.sqrt(D), bits=8, causal=True)
    assert_close(out, ref, "string-mask")


@pytest.mark.parametrize("D,S", [(128, 300), (128, 6000), (64, 300)])
def test_output_views(D, S):
    """Output rows stored whole from LDS, 16 bytes a lane: into a view 16 bytes past the start of
    each row, with a row stride of D + 16 elements, and a partial last row block (with S = 6000 the
    keys are split and merged). Every row matches the contiguous call bit for bit and the elements
    around the rows keep their values. The prefill entry point requires 16-byte aligned rows and
    strides; an 8-byte aligned view is rejected."""
    print(f"prefill output view D={D} S={S}", flush=True)
    B, Hq, Hkv, L = 1, 16, 4, 77  # 16 / 4 * 77 = 308 rows: a full and a partial row block
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 40 + D)
    q = seeded_normal((B, Hq, L, D), 41 + D, torch.float16, DEV)
    ref = kernels.attention(q, kt, vt, 0.1, causal=True, bits=8, kernel="prefill")
    big = torch.full((B, Hq, L, D + 16), 5.0, dtype=torch.float16, device=DEV)
    view = big[..., 8:8 + D]
    out = kernels.attention(q, kt, vt, 0.1, causal=True, bits=8, kernel="prefill", out=view)
    torch.cuda.synchronize()
    assert out.data_ptr() == view.data_ptr()
    assert torch.equal(view, ref)
    assert torch.all(big[..., :8] == 5.0) and torch.all(big[..., 8 + D:] == 5.0)
    assert_close(ref, exact_reference(q, kt, vt, 0.1, bits=8, causal=True), f"D={D} S={S}")
    with pytest.raises(ValueError, match="16-byte aligned"):
        kernels.attention(q, kt, vt, 0.1, causal=True, bits=8, kernel="prefill", out=big[..., 4:4 + D])


def test_repeated_calls_are_bit_identical():
    # the key splits are merged in split order whichever workgroup merges them
    print("prefill repeat", flush=True)
    kt, vt = make_cache(1, 4, 16384, 128, 8, torch.bfloat16, 81)
    q = seeded_normal((1, 32, 512, 128), 82, torch.bfloat16, DEV)
    outs = [kernels.attention(q, kt, vt, 0.088, causal=True, bits=8, kernel="prefill") for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal,bits", [(False, 8), (True, 8), (False, 4)])
def test_running_max_moves_mid_split(dtype, causal, bits):
    # every query shares a +-1 component u, the keys are small noise except three "spike" keys
    # beta * u that score about 16 beta (log2 units) above the rest. The spikes sit in the third
    # and fourth tiles of one 256-key split and in the second tile of the last split, so each row's
    # running maximum is stale by far more than the rescale bound mid-split, with live
    # accumulators: the probabilities against it would overflow fp16 unless the kernel moves the
    # maximum, rescales and recomputes. Scores stay moderate, so fp16 operand rounding keeps the
    # result within the usual bar.
    print(f"prefill mid-split maxima dtype={dtype} causal={causal} bits={bits}", flush=True)
    B, Hq, Hkv, L, S, D = 1, 16, 4, 96, 2048, 128
    g = torch.Generator().manual_seed(95)
    u = torch.randint(0, 2, (D,), generator=g).float() * 2 - 1
    k = 0.3 * seeded_normal((B, Hkv, S, D), 96, torch.float32)
    for pos, beta in ((400, 1.0), (480, 2.0), (1850, 1.5)):
        k[:, :, pos] = beta * u
    k = k.to(dtype).to(DEV)
    v = seeded_normal((B, Hkv, S, D), 97, dtype, DEV)
    trip = []
    for x in (k, v):
        codes = torch.zeros((B, Hkv, S, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
        sc = torch.zeros((B, Hkv, S, D // 64), dtype=dtype, device=DEV)
        bi = torch.zeros_like(sc)
        kernels.quantize_append(x, (codes, sc, bi), row_offset=0, group_size=64, bits=bits)
        trip.append((codes, sc, bi))
    q = (u + 0.3 * seeded_normal((B, Hq, L, D), 98, torch.float32)).to(dtype).to(DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, trip[0], trip[1], scale, causal=causal, bits=bits, kernel="prefill")
    torch.cuda.synchronize()
    ref = exact_reference(q, trip[0], trip[1], scale, bits=bits, causal=causal)
    assert_close(out, ref, "mid-split maxima")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal,bits", [(False, 8), (True, 8), (False, 4)])
def test_rising_key_norms(dtype, causal, bits):
    # Key norms grow x1 -> x65 along the sequence, so each row's maximum keeps rising tile after
    # tile (the running maximum moves, rescales and recomputes again and again) and the scores
    # reach about 300 in natural-log units. At that magnitude fp16 key operands alone move a
    # score by about 300 * 2^-11 / sqrt(3) ~ 0.08, so no kernel that dequantizes keys to fp16 --
    # the reference's fp16 quantized_matmul included -- meets the north-star bar of N(0,1)
    # inputs here. The bar is therefore derived on the same inputs:
    #   floor = error of exact fp64 attention over the dequantized keys rounded to fp16
    #   the kernel: error <= floor + the north-star (fp16) or bf16 bar
    # and the kernel must also be closer to the exact answer than the reference-faithful port
    # (the reference's blocked loop with its roundings to T, m5engine/attention.py:49, 66-69,
    # 87-90), which the reference itself would produce.
    import numpy as np

    from oracle import attention as OA
    from tests.helpers import TOL, fp16_key_floor

    print(f"prefill rising key norms dtype={dtype} causal={causal} bits={bits}", flush=True)
    B, Hq, Hkv, L, S, D = 1, 16, 4, 96, 2048, 128
    growth = 1.0 + torch.arange(S, dtype=torch.float32) / 32.0
    k = (seeded_normal((B, Hkv, S, D), 91, torch.float32) * growth[None, None, :, None]).to(dtype).to(DEV)
    v = seeded_normal((B, Hkv, S, D), 92, dtype, DEV)
    trip = []
    for x in (k, v):
        codes = torch.zeros((B, Hkv, S, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32)
        sc = torch.zeros((B, Hkv, S, D // 64), dtype=dtype, device=DEV)
        bi = torch.zeros_like(sc)
        kernels.quantize_append(x, (codes, sc, bi), row_offset=0, group_size=64, bits=bits)
        trip.append((codes, sc, bi))
    q = seeded_normal((B, Hq, L, D), 93, dtype, DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, trip[0], trip[1], scale, causal=causal, bits=bits, kernel="prefill")
    torch.cuda.synchronize()
    ref = exact_reference(q, trip[0], trip[1], scale, bits=bits, causal=causal)
    o = out.cpu().float().numpy().astype(np.float64)
    assert np.isfinite(o).all()
    st = OA.error_stats(o, ref)
    floor = fp16_key_floor(q, trip[0], trip[1], scale, ref, bits=bits, causal=causal)
    ns_abs, ns_rel = TOL[dtype](ref)
    if dtype == torch.float16:  # (bf16 4-bit codes times bf16 scales mostly fit fp16 exactly)
        assert floor["max_abs"] > ns_abs, "the case must exercise scores beyond the north-star regime"
    assert st["max_abs"] <= floor["max_abs"] + ns_abs and st["rel_l2"] <= floor["rel_l2"] + ns_rel, (st, floor)
    cpu = [tuple(t.cpu() for t in tr) for tr in trip]
    port = OA.reference_sdpa(q.cpu(), cpu[0], cpu[1], scale, "causal" if causal else None, 64, bits)
    pst = OA.error_stats(port.float().numpy().astype(np.float64), ref)
    print(f"  gpu {st}  fp16-key floor {floor}  reference port {pst}", flush=True)
    assert st["max_abs"] <= pst["max_abs"] and st["rel_l2"] <= pst["rel_l2"], (st, pst)


@pytest.mark.parametrize("D,L,kernel,window", [
    (128, 5, "decode", 0), (128, 100, "prefill", 0), (128, 100, "prefill", 48), (64, 70, "prefill", 0),
    (256, 40, "prefill", 0),
])
def test_sequences_shorter_than_the_chunk(D, L, kernel, window):
    """A batch row whose sequence holds fewer keys than the chunk has queries: under the causal
    mask its first rows sit at negative positions and see no key, so they come out 0 (the
    reference's blocked path gives acc / max(denom, 1e-30) = 0); the rest see the keys up to their
    position."""
    print(f"short sequence D={D} L={L} {kernel} window={window}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 400
    lens = [400, L // 2]
    G = 64
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.bfloat16, 90 + D + L, group=G)
    q = seeded_normal((B, Hq, L, D), 91 + L, torch.bfloat16, DEV)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    kw = dict(causal=True, window=window, seq_lens=seq, bits=8, group_size=G)
    out = kernels.attention(q, kt, vt, 0.1, kernel=kernel, **kw)
    torch.cuda.synchronize()
    ref = exact_reference(q, kt, vt, 0.1, **kw)
    assert_close(out, ref, f"short sequence D={D} L={L} {kernel}")
    dark = L - lens[1]  # rows of sequence 1 at negative positions
    assert torch.all(out[1, :, :dark] == 0)
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("D,L,kernel,causal", [
    (128, 1, "decode", False), (128, 1, "decode", True), (128, 64, "prefill", True), (64, 64, "prefill", False),
    (256, 20, "prefill", True),
])
def test_empty_sequence_in_batch(D, L, kernel, causal):
    """A batch row with no keys at all (seq_lens 0): every one of its rows sees no key and comes
    out 0, with and without the causal mask, and with the keys split over workgroups for the
    other row (S = 3000)."""
    print(f"empty sequence D={D} L={L} {kernel} causal={causal}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 3000
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 95 + D + L)
    q = seeded_normal((B, Hq, L, D), 96 + L, torch.float16, DEV)
    seq = torch.tensor([S, 0], dtype=torch.int32, device=DEV)
    kw = dict(causal=causal, seq_lens=seq, bits=8)
    out = kernels.attention(q, kt, vt, 0.1, kernel=kernel, **kw)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0)
    assert_close(out, exact_reference(q, kt, vt, 0.1, **kw), f"empty sequence D={D} {kernel}")
