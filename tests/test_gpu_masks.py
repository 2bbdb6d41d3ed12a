"""General masks (kvq_decode_attn_masked / kvq_decode_attn_dense_masked): boolean masks with no
causal / window / padding structure, per-head masks and additive masks, through the drop-in
entry points, against the exact fp64 oracle (oracle.attention.exact_attention's vis / add).

The expected per-query-head mask is built here by hand from the reference's broadcasting: a rank
>= 3 mask gains a KV-head axis before it meets the grouped [B, Hkv, rep, L, S] scores, in the
blocked loop (m5engine/attention.py:55-56) and in the hand-off to mlx-lm's quantized SDPA (:42-45,
restated by oracle.attention.original_sdpa); mx.fast's SDPA broadcasts against [B, Hq, L, S].
"""

import math

import numpy as np
import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd import kernels
from oracle import attention as OA
from oracle import quantize as OQ
from tests.helpers import NP_DTYPE, assert_close, seeded_normal, triple_to_np
from tests.test_gpu_decode import make_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _exact(q, kt, vt, scale, bits, group, vis=None, add=None):
    dt = NP_DTYPE[q.dtype]
    qn = q.detach().cpu().float().numpy().astype(np.float64)
    kdq = OQ.dequantize(*triple_to_np(kt), dt, group, bits)
    vdq = OQ.dequantize(*triple_to_np(vt), dt, group, bits)
    return OA.exact_attention(qn, kdq, vdq, scale, vis=vis, add=add)


def _random_vis(shape, seed, p=0.7):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(*shape, generator=g) < p
    m[..., 0] = True  # no row is fully hidden unless a test says so
    return m


@pytest.mark.parametrize("D,G,bits,dtype,L,S", [
    (128, 64, 8, torch.float16, 1, 3000),
    (128, 64, 8, torch.bfloat16, 37, 700),
    (64, 32, 4, torch.float16, 9, 513),
    (256, 64, 8, torch.bfloat16, 5, 1100),
    (128, 128, 4, torch.float16, 130, 300),
])
def test_random_bool_mask_quantized(D, G, bits, dtype, L, S):
    print(f"masked quantized bool D={D} G={G} bits={bits} {dtype} L={L} S={S}", flush=True)
    B, Hq, Hkv = 2, 8, 2
    kt, vt = make_cache(B, Hkv, S, D, bits, dtype, 900 + D + L, group=G)
    q = seeded_normal((B, Hq, L, D), 901 + L, dtype, DEV)
    vis = _random_vis((B, 1, L, S), 902 + S)
    scale = 1.0 / math.sqrt(D)
    out = A.blocked_quantized_sdpa(q, kt, vt, scale, vis.to(DEV), group_size=G, bits=bits)
    assert_close(out, _exact(q, kt, vt, scale, bits, G, vis=vis.numpy()), f"bool mask D={D} L={L}")


def test_per_kv_head_mask_blocked_layout(monkeypatch):
    """L > 1 with S above one block: a [B, Hkv, L, S] mask indexes KV heads (query head h reads
    mask[:, h // rep])."""
    monkeypatch.setattr(A, "score_budget_bytes", 1)  # one MIN_BLOCK: S = 700 takes the blocked loop
    B, Hq, Hkv, L, S, D = 2, 8, 2, 12, 700, 128
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 910)
    q = seeded_normal((B, Hq, L, D), 911, torch.float16, DEV)
    m = _random_vis((B, Hkv, L, S), 912)
    rep = Hq // Hkv
    vis = m.numpy()[:, np.arange(Hq) // rep]
    out = A.blocked_quantized_sdpa(q, kt, vt, 0.09, m.to(DEV), group_size=64, bits=8)
    assert_close(out, _exact(q, kt, vt, 0.09, 8, 64, vis=vis), "per-KV-head mask, blocked layout")


def test_batched_decode_mask_indexes_sequences():
    """L == 1 (the hand-off to mlx-lm's quantized SDPA): a [B, 1, 1, S] mask gains a KV-head axis
    before it meets the grouped [B, Hkv, rep, 1, S] scores, so sequence b reads mask[b]."""
    B, Hq, Hkv, L, S, D = 2, 8, 2, 1, 900, 128
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 920)
    q = seeded_normal((B, Hq, L, D), 921, torch.float16, DEV)
    m = _random_vis((B, 1, 1, S), 922)
    out = A.blocked_quantized_sdpa(q, kt, vt, 0.09, m.to(DEV), group_size=64, bits=8)
    assert_close(out, _exact(q, kt, vt, 0.09, 8, 64, vis=m.numpy()), "batched decode mask")


@pytest.mark.parametrize("mdtype", [torch.float32, torch.bfloat16, torch.float16])
def test_additive_mask(mdtype):
    print(f"masked additive {mdtype}", flush=True)
    B, Hq, Hkv, L, S, D = 2, 8, 4, 20, 600, 128
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.bfloat16, 930)
    q = seeded_normal((B, Hq, L, D), 931, torch.bfloat16, DEV)
    g = torch.Generator().manual_seed(932)
    add = (torch.rand(B, 1, L, S, generator=g) * 6.0 - 3.0).to(mdtype)
    add[:, :, :, 100:140] = float("-inf")  # hidden keys as -inf
    exact_add = add.float().numpy().astype(np.float64)
    out = A.blocked_quantized_sdpa(q, kt, vt, 0.09, add.to(DEV), group_size=64, bits=8)
    assert_close(out, _exact(q, kt, vt, 0.09, 8, 64, add=exact_add), f"additive {mdtype}")


def test_fully_hidden_rows_return_zero():
    B, Hq, Hkv, L, S, D = 1, 4, 4, 6, 400, 64
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 940)
    q = seeded_normal((B, Hq, L, D), 941, torch.float16, DEV)
    m = _random_vis((B, Hq, L, S), 942)
    m[0, 2, 3] = False
    m[0, 0, 5] = False
    out = A.blocked_quantized_sdpa(q, kt, vt, 0.12, m.to(DEV), group_size=64, bits=8)
    assert torch.all(out[0, 2, 3] == 0) and torch.all(out[0, 0, 5] == 0)
    assert_close(out, _exact(q, kt, vt, 0.12, 8, 64, vis=m.numpy()), "fully hidden rows")


@pytest.mark.parametrize("D,dtype", [(128, torch.float16), (64, torch.bfloat16), (256, torch.bfloat16)])
def test_unquantized_per_query_head_mask(D, dtype):
    """mx.fast's layout: a [B, Hq, L, S] mask is per query head."""
    print(f"masked dense D={D} {dtype}", flush=True)
    B, Hq, Hkv, L, S = 2, 8, 2, 33, 500
    k = seeded_normal((B, Hkv, S, D), 950, dtype, DEV)
    v = seeded_normal((B, Hkv, S, D), 951, dtype, DEV)
    q = seeded_normal((B, Hq, L, D), 952, dtype, DEV)
    m = _random_vis((B, Hq, L, S), 953)
    scale = 1.0 / math.sqrt(D)
    out = A.fast_scaled_dot_product_attention(q, k, v, scale, m.to(DEV))
    kn = k.cpu().float().numpy().astype(np.float64)
    vn = v.cpu().float().numpy().astype(np.float64)
    qn = q.cpu().float().numpy().astype(np.float64)
    assert_close(out, OA.exact_attention(qn, kn, vn, scale, vis=m.numpy()), f"dense mask D={D}")


def test_structured_masks_still_take_the_structured_path(monkeypatch):
    """A causal boolean mask is recognised and runs as causal (no general-mask launch)."""
    calls = []
    real = kernels.masked_attention
    monkeypatch.setattr(kernels, "masked_attention", lambda *a, **k: calls.append(1) or real(*a, **k))
    B, Hq, Hkv, L, S, D = 1, 8, 2, 16, 300, 128
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 960)
    q = seeded_normal((B, Hq, L, D), 961, torch.float16, DEV)
    causal = torch.arange(S - L, S)[:, None] >= torch.arange(S)[None]
    out = A.blocked_quantized_sdpa(q, kt, vt, 0.09, causal.to(DEV), group_size=64, bits=8)
    assert not calls
    assert_close(out, _exact(q, kt, vt, 0.09, 8, 64, vis=causal.numpy()), "causal bool mask")


@pytest.mark.parametrize("L,S", [(1, 2048), (40, 700)])
def test_unquantized_head_dim_256_additive_mask(L, S):
    """The unquantized head_dim-256 cache runs through the head_dim-256 kernel: an additive mask with
    -inf entries, per query head, at decode and prefill lengths."""
    print(f"masked dense D=256 additive L={L} S={S}", flush=True)
    B, Hq, Hkv, D = 2, 8, 4, 256
    dtype = torch.bfloat16
    k = seeded_normal((B, Hkv, S, D), 970, dtype, DEV)
    v = seeded_normal((B, Hkv, S, D), 971, dtype, DEV)
    q = seeded_normal((B, Hq, L, D), 972, dtype, DEV)
    g = torch.Generator().manual_seed(973)
    add = torch.rand(B, Hq, L, S, generator=g) * 4.0 - 2.0
    add[:, :, :, 50:90] = float("-inf")
    scale = 1.0 / math.sqrt(D)
    out = A.fast_scaled_dot_product_attention(q, k, v, scale, add.to(DEV))
    kn = k.cpu().float().numpy().astype(np.float64)
    vn = v.cpu().float().numpy().astype(np.float64)
    qn = q.cpu().float().numpy().astype(np.float64)
    ref = OA.exact_attention(qn, kn, vn, scale, add=add.numpy().astype(np.float64))
    assert_close(out, ref, f"dense D=256 additive L={L}")
