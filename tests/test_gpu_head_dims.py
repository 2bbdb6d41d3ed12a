"""Head dimensions other than 64, 128 and 256: any multiple of 8 up to 256 (for quantized caches the
group size must divide it and lie between a quarter of the kernel width and the width). They run
at the next width (64, 128 or 256) for every query length, with zero queries past the row's last
dim and only its own dims stored: on the decode kernel, or for unquantized rows past 128 dims on the
head_dim-256 kernel. The reference takes D from the queries (m5engine/attention.py:38) and is
generic over it; mlx-lm's quantized cache needs D to be a multiple of the group size.

Every case is checked against the exact fp64 oracle. Rows past each sequence's end hold NaN scales
and biases (NaN values in the unquantized caches), and paged pools are poisoned the same way, so a
read past a row's own dims that leaves the cache's valid rows shows up as a non-finite output.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from myinfer_amd import _lib
from myinfer_amd import attention as A
from myinfer_amd import kernels
from oracle import attention as OA
from tests.helpers import assert_close, exact_reference, seeded_normal
from tests.test_gpu_decode import make_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _poison_tail(tr, seq_lens):
    """NaN scales and biases for the rows of sequence b at or past seq_lens[b]."""
    for b, n in enumerate(seq_lens):
        tr[1][b, :, n:] = float("nan")
        tr[2][b, :, n:] = float("nan")


@pytest.mark.parametrize("D,G,bits,dtype,L,causal,window", [
    (96, 32, 8, torch.float16, 1, False, 0),
    (96, 32, 4, torch.bfloat16, 1, False, 0),
    (96, 32, 8, torch.bfloat16, 40, True, 0),
    (96, 32, 4, torch.float16, 17, True, 100),
    (32, 32, 8, torch.float16, 1, False, 0),
    (32, 32, 4, torch.bfloat16, 25, True, 0),
    (192, 64, 8, torch.bfloat16, 1, False, 0),
    (192, 64, 4, torch.float16, 1, False, 0),
    (192, 64, 8, torch.float16, 33, True, 0),
])
def test_quantized_head_dims(D, G, bits, dtype, L, causal, window):
    print(f"head dim D={D} G={G} bits={bits} {dtype} L={L} causal={causal} window={window}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 700
    lens = [700, 513]
    kt, vt = make_cache(B, Hkv, S, D, bits, dtype, 1200 + D + L, group=G)
    _poison_tail(kt, lens)
    _poison_tail(vt, lens)
    q = seeded_normal((B, Hq, L, D), 1201 + D, dtype, DEV)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    kw = dict(causal=causal, window=window, seq_lens=seq, group_size=G, bits=bits)
    out = kernels.attention(q, kt, vt, scale, **kw)
    ref = exact_reference(q, kt, vt, scale, bits=bits, group_size=G, causal=causal, window=window, seq_lens=seq)
    assert_close(out, ref, f"D={D} G={G} bits={bits} L={L}")
    # the prefill entry point serves these widths with the same kernel: the same bits
    out_p = kernels.attention(q, kt, vt, scale, kernel="prefill", **kw)
    assert torch.equal(out_p, out)


def test_output_rows_keep_their_neighbours():
    """Only D dims of each output row are written: an output view with wider rows keeps the
    elements past D."""
    B, Hq, Hkv, S, D, G = 1, 8, 2, 300, 96, 32
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 1210, group=G)
    q = seeded_normal((B, Hq, 1, D), 1211, torch.float16, DEV)
    wide = torch.full((B, Hq, 1, 128), 7.0, dtype=torch.float16, device=DEV)
    out = kernels.attention(q, kt, vt, 0.1, group_size=G, bits=8, out=wide[..., :D])
    assert torch.all(wide[..., D:] == 7.0)
    assert_close(out, exact_reference(q, kt, vt, 0.1, bits=8, group_size=G), "D=96 into a wider row")


@pytest.mark.parametrize("L", [1, 12])
def test_drop_in_blocked_sdpa(monkeypatch, L):
    """The drop-in entry point over a head_dim-96 cache (Phi-3-mini's heads, groups of 32), the
    string causal mask and an additive mask."""
    monkeypatch.setattr(A, "score_budget_bytes", 1)  # S = 600 takes the blocked loop at L > 1
    B, Hq, Hkv, S, D, G = 2, 8, 4, 600, 96, 32
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.float16, 1220 + L, group=G)
    q = seeded_normal((B, Hq, L, D), 1221 + L, torch.float16, DEV)
    scale = 1.0 / math.sqrt(D)
    out = A.blocked_quantized_sdpa(q, kt, vt, scale, "causal", group_size=G, bits=8)
    assert_close(out, exact_reference(q, kt, vt, scale, bits=8, group_size=G, causal=True), f"drop-in causal L={L}")
    g = torch.Generator().manual_seed(1222)
    add = (torch.rand(B, 1, L, S, generator=g) * 4.0 - 2.0).to(torch.float16)
    out = A.blocked_quantized_sdpa(q, kt, vt, scale, add.to(DEV), group_size=G, bits=8)
    from tests.test_gpu_masks import _exact

    assert_close(out, _exact(q, kt, vt, scale, 8, G, add=add.float().numpy().astype(np.float64)),
                 f"drop-in additive L={L}")


@pytest.mark.parametrize("D,dtype,L,causal,window", [
    (80, torch.float16, 1, False, 0),
    (80, torch.bfloat16, 29, True, 0),
    (96, torch.bfloat16, 1, False, 0),
    (112, torch.float16, 20, True, 64),
    (32, torch.float16, 9, True, 0),
    (48, torch.bfloat16, 1, False, 0),
    (160, torch.bfloat16, 1, False, 0),
    (192, torch.float16, 37, True, 0),
    (224, torch.bfloat16, 20, True, 96),
    (136, torch.float16, 130, True, 0),
])
def test_unquantized_head_dims(D, dtype, L, causal, window):
    print(f"unquantized head dim D={D} {dtype} L={L} causal={causal} window={window}", flush=True)
    B, Hq, Hkv, S = 2, 8, 2, 520
    lens = [520, 301]
    k = seeded_normal((B, Hkv, S, D), 1230 + D, dtype, DEV)
    v = seeded_normal((B, Hkv, S, D), 1231 + D, dtype, DEV)
    for b, n in enumerate(lens):
        k[b, :, n:] = float("nan")
        v[b, :, n:] = float("nan")
    q = seeded_normal((B, Hq, L, D), 1232 + L, dtype, DEV)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out = kernels.attention(q, k, v, scale, causal=causal, window=window, seq_lens=seq)
    ref = OA.exact_attention(q.cpu().double().numpy(), k.cpu().double().numpy(), v.cpu().double().numpy(), scale,
                             causal=causal, window=window, seq_lens=lens)
    assert_close(out, ref, f"unquantized D={D} L={L}")
    out_p = kernels.attention(q, k, v, scale, causal=causal, window=window, seq_lens=seq, kernel="prefill")
    assert torch.equal(out_p, out)


@pytest.mark.parametrize("D", [80, 192])
def test_unquantized_per_head_mask(D):
    """mx.fast's SDPA with a per-query-head boolean mask over Phi-2-shaped heads (D = 80, the decode
    kernel) and 192-dim heads (the head_dim-256 kernel)."""
    B, Hq, Hkv, L, S = 1, 8, 8, 21, 333
    k = seeded_normal((B, Hkv, S, D), 1240, torch.float16, DEV)
    v = seeded_normal((B, Hkv, S, D), 1241, torch.float16, DEV)
    q = seeded_normal((B, Hq, L, D), 1242, torch.float16, DEV)
    g = torch.Generator().manual_seed(1243)
    m = torch.rand(B, Hq, L, S, generator=g) < 0.6
    m[..., 0] = True
    out = A.fast_scaled_dot_product_attention(q, k, v, 0.11, m.to(DEV))
    ref = OA.exact_attention(q.cpu().double().numpy(), k.cpu().double().numpy(), v.cpu().double().numpy(), 0.11,
                             vis=m.numpy())
    assert_close(out, ref, f"D={D} per-head mask")


def test_paged_head_dim_96():
    """Paged pools at head_dim 96 (groups of 32): bit-identical to the contiguous caches and within
    the bar of the oracle, decode and a causal chunk."""
    from tests.test_gpu_paged import build

    B, Hkv, Hq, D, G = 3, 2, 8, 96, 32
    lens = [300, 64, 129]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, 8, torch.float16, 1250, group=G)
    seq = torch.tensor(lens, dtype=torch.int32, device=DEV)
    for L in (1, 10):
        q = seeded_normal((B, Hq, L, D), 1251 + L, torch.float16, DEV)
        out = kernels.paged_attention(q, kp, vp, tables, seq, 0.1, causal=True, group_size=G, bits=8)
        cont = kernels.attention(q, kc, vc, 0.1, causal=True, seq_lens=seq, group_size=G, bits=8)
        assert torch.equal(out, cont), f"paged D=96 L={L} differs from the contiguous call"
        assert_close(out, exact_reference(q, kc, vc, 0.1, bits=8, group_size=G, causal=True, seq_lens=seq),
                     f"paged D=96 L={L}")


def test_static_entry_point_head_dim_96():
    """kvq_decode_attn_static at head_dim 96: bit-identical to kvq_decode_attn."""
    from tests.test_zz_no_alloc import _static_call

    B, Hq, Hkv, S, D, G = 1, 16, 8, 1000, 96, 32
    kt, vt = make_cache(B, Hkv, S, D, 8, torch.bfloat16, 1260, group=G)
    q = seeded_normal((B, Hq, 1, D), 1261, torch.bfloat16, DEV)
    ref_out = kernels.attention(q, kt, vt, 0.1, bits=8, group_size=G, kernel="decode")
    out = torch.full_like(ref_out, float("nan"))
    _lib.check(_static_call(q, kt, vt, out, 0.1, bits=8, group=G), "kvq_decode_attn_static")
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)


def test_rejected_head_dims_raise():
    q = torch.zeros((1, 4, 1, 160), dtype=torch.float16, device=DEV)
    kt, vt = make_cache(1, 2, 64, 160, 8, torch.float16, 1270, group=32)
    with pytest.raises((ValueError, NotImplementedError, RuntimeError)):
        kernels.attention(q, kt, vt, 0.1, group_size=32, bits=8)  # width 256 needs groups of 64 or 128
    q = torch.zeros((1, 4, 1, 264), dtype=torch.float16, device=DEV)
    k = torch.zeros((1, 2, 64, 264), dtype=torch.float16, device=DEV)
    with pytest.raises((ValueError, NotImplementedError, RuntimeError)):
        kernels.attention(q, k, k, 0.1)  # past 256 dims
    assert ctypes  # the C ABI's own rejections are covered by the CPU tests
