"""The C5 configuration end to end: Gemma-3-27B attention shapes (32 query heads / 16 KV heads,
head_dim 128, bf16) with five window-1024 layers and one global causal layer, B = 4 sequences,
an 8192-token prefill in 2048-token chunks and then decode steps, driven through the cache objects
the way mlx-lm's generate_step drives them:

  * make_prompt_cache(layer_windows=[1024] * 5 + [None]) builds a RotatingKVCache per window
    layer and a KVCache for the global layer;
  * each chunk appends its K/V rows to every layer's cache (update_and_fetch), and attention runs
    through scaled_dot_product_attention with the cache's mask (make_mask for window layers);
  * after each model call safe_maybe_quantize_kv_cache(quantized_kv_start=0, group 64, 8 bits)
    converts the plain global cache to a QuantizedKVCache (m5engine/attention.py:106-112): chunk 0
    of the global layer attends unquantized rows, every later chunk and every decode step attends
    the 8-bit cache, while the window layers stay unquantized, as the reference leaves them.

Every layer's output is compared with the exact fp64 oracle on sampled query rows (all heads,
all sequences): the oracle sees each sampled query at its absolute position over the layer's whole
history -- the exact bf16 rows for unquantized layers, the dequantized triples the kernels read
for the quantized one -- with the window applied to absolute positions.
"""

import math

import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd.cache import QuantizedKVCache, RotatingKVCache, make_prompt_cache
from oracle import attention as OA
from oracle import quantize as OQ
from tests.helpers import TOL, seeded_normal, triple_to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, HQ, HKV, D, N, C, W = 4, 32, 16, 128, 8192, 2048, 1024
WINDOWS = [W] * 5 + [None]


def _check(out, q, layer, cache, hist_k, hist_v, pos0, rows, scale, what):
    """Sampled rows `rows` (indices into this call's queries, at positions pos0 + row) of `out`
    against the exact oracle over the layer's history."""
    win = WINDOWS[layer] or 0
    if isinstance(cache, QuantizedKVCache):
        kdq = OQ.dequantize(*triple_to_np(cache.fetch()[0]), "bfloat16", 64, 8)
        vdq = OQ.dequantize(*triple_to_np(cache.fetch()[1]), "bfloat16", 64, 8)
    else:
        kdq = torch.cat(hist_k, dim=2).double().numpy()
        vdq = torch.cat(hist_v, dim=2).double().numpy()
    qn = q.float().cpu().double().numpy()
    got = out.float().cpu().double().numpy()
    for r in rows:
        p = pos0 + r
        ref = OA.exact_attention(qn[:, :, r:r + 1], kdq[:, :, :p + 1], vdq[:, :, :p + 1], scale, window=win)
        st = OA.error_stats(got[:, :, r:r + 1], ref)
        max_abs, rel = TOL[torch.bfloat16](ref)
        assert st["max_abs"] <= max_abs and st["rel_l2"] <= rel, f"{what} row {r} (position {p}): {st}"


def test_c5_window_and_global_layers_prefill_then_decode():
    scale = 1.0 / math.sqrt(D)
    caches = make_prompt_cache(len(WINDOWS), layer_windows=WINDOWS)
    assert [type(c) for c in caches] == [RotatingKVCache] * 5 + [type(caches[5])]
    hist_k = [[] for _ in WINDOWS]
    hist_v = [[] for _ in WINDOWS]
    g = torch.Generator().manual_seed(1500)
    quantized_seen = False
    for c in range(N // C):
        rows = sorted(set([0, C - 1] + torch.randint(0, C, (6,), generator=g).tolist()))
        for layer in range(len(WINDOWS)):
            print(f"C5 prefill chunk {c} layer {layer} ({'window' if WINDOWS[layer] else 'global'}, "
                  f"{type(caches[layer]).__name__})", flush=True)
            seed = 1600 + 10 * c + layer
            k = seeded_normal((B, HKV, C, D), seed, torch.bfloat16, DEV)
            v = seeded_normal((B, HKV, C, D), seed + 100, torch.bfloat16, DEV)
            q = seeded_normal((B, HQ, C, D), seed + 200, torch.bfloat16, DEV)
            hist_k[layer].append(k.float().cpu())
            hist_v[layer].append(v.float().cpu())
            cache = caches[layer]
            # the mask is built before the cache update, as mlx-lm's models build it
            mask = cache.make_mask(C, window_size=W) if WINDOWS[layer] else "causal"
            kf, vf = cache.update_and_fetch(k, v)
            out = A.scaled_dot_product_attention(q, kf, vf, cache, scale, mask)
            torch.cuda.synchronize()
            quantized_seen |= isinstance(cache, QuantizedKVCache)
            _check(out, q, layer, cache, hist_k[layer], hist_v[layer], c * C, rows, scale, f"chunk {c} layer {layer}")
        # after the model call, as mlx-lm's generate_step does
        A.safe_maybe_quantize_kv_cache(caches, quantized_kv_start=0, kv_group_size=64, kv_bits=8)
        assert isinstance(caches[5], QuantizedKVCache) and all(isinstance(x, RotatingKVCache) for x in caches[:5])
    assert quantized_seen, "the global layer must attend its 8-bit cache from chunk 1 on"
    assert caches[5].offset == N and caches[5].keys[0].shape[0] == B
    # decode steps: one new token per sequence per step
    for step in range(3):
        for layer in range(len(WINDOWS)):
            print(f"C5 decode step {step} layer {layer}", flush=True)
            seed = 1900 + 10 * step + layer
            k = seeded_normal((B, HKV, 1, D), seed, torch.bfloat16, DEV)
            v = seeded_normal((B, HKV, 1, D), seed + 100, torch.bfloat16, DEV)
            q = seeded_normal((B, HQ, 1, D), seed + 200, torch.bfloat16, DEV)
            hist_k[layer].append(k.float().cpu())
            hist_v[layer].append(v.float().cpu())
            cache = caches[layer]
            mask = cache.make_mask(1, window_size=W) if WINDOWS[layer] else None
            kf, vf = cache.update_and_fetch(k, v)
            out = A.scaled_dot_product_attention(q, kf, vf, cache, scale, mask)
            torch.cuda.synchronize()
            _check(out, q, layer, cache, hist_k[layer], hist_v[layer], N + step, [0], scale,
                   f"decode step {step} layer {layer}")
        A.safe_maybe_quantize_kv_cache(caches, quantized_kv_start=0, kv_group_size=64, kv_bits=8)
    assert caches[5].offset == N + 3 and caches[0].offset == N + 3
