"""GPU KV caches in MLX layout (myinfer_amd/cache.py) against the oracle's bookkeeping model of
mlx-lm's caches (oracle/cache.py) and its quantizer: step-256 growth, offset, trim and re-append
(the contract m5engine/prefix_cache.py:77-123 relies on, restated from tests/test_core.py:79-97),
nbytes (m5engine/context.py:41-47, :169), to_quantized / safe_maybe_quantize_kv_cache
(m5engine/attention.py:106-112), and attention over the fetched views."""

import math

import numpy as np
import pytest
import torch

from myinfer_amd import attention as A
from myinfer_amd.cache import KVCache, QuantizedKVCache, can_trim_prompt_cache, make_prompt_cache, trim_prompt_cache
from oracle import cache as OC
from oracle import quantize as OQ
from tests.helpers import assert_close, exact_reference, seeded_normal, to_np_bits, triple_to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rows(n, seed, H=2, D=128, dtype=torch.float16):
    return seeded_normal((1, H, n, D), seed, dtype, DEV)


@pytest.mark.parametrize("cls", ["plain", "quantized"])
def test_growth_matches_model(cls):
    c = KVCache() if cls == "plain" else QuantizedKVCache(group_size=64, bits=8)
    model = OC.CacheModel()
    for i, L in enumerate([5, 1, 300, 1, 1, 251, 512, 1, 3]):
        k, v = rows(L, 10 + i), rows(L, 50 + i)
        c.update_and_fetch(k, v)
        model.update(L)
        cap = (c.keys.shape[2] if cls == "plain" else c.keys[0].shape[2])
        assert (c.offset, cap) == (model.offset, model.capacity), f"append {i} (L={L})"
    assert c.is_trimmable()
    assert c.trim(10) == model.trim(10) and c.offset == model.offset
    assert c.trim(10**6) == model.trim(10**6) and c.offset == 0


def test_quantized_contents_bit_exact_after_appends_and_trim():
    c = QuantizedKVCache(group_size=64, bits=4)
    ks, vs = [], []
    for i, L in enumerate([7, 1, 260, 1]):
        k, v = rows(L, 100 + i), rows(L, 200 + i)
        fk, fv = c.update_and_fetch(k, v)
        ks.append(k)
        vs.append(v)
    # prefix reuse: drop the last 3 tokens, then append 2 new ones at the trimmed offset
    assert c.trim(3) == 3
    k2, v2 = rows(2, 300), rows(2, 301)
    fk, fv = c.update_and_fetch(k2, v2)
    allk = torch.cat(ks, dim=2)[:, :, :c.offset - 2]
    allk = torch.cat([allk, k2], dim=2)
    allv = torch.cat([torch.cat(vs, dim=2)[:, :, :c.offset - 2], v2], dim=2)
    assert fk[0].shape[2] == c.offset == 268  # 269 appended, 3 trimmed, 2 re-appended
    for got, x in ((fk, allk), (fv, allv)):
        rc, rs, rb = OQ.quantize(to_np_bits(x), "float16", 64, 4)
        gc, gs, gb = triple_to_np(got)
        assert np.array_equal(gc, rc) and np.array_equal(gs, rs) and np.array_equal(gb, rb)


def test_prefix_cache_contract():
    # tests/test_core.py:79-87 restated on this cache: 5 tokens cached, a request sharing 3 of them
    # trims back to offset 3 and re-appends from there
    cache = make_prompt_cache(1)
    cache[0].update_and_fetch(rows(5, 1, H=2, D=64), rows(5, 2, H=2, D=64))
    assert can_trim_prompt_cache(cache)
    assert trim_prompt_cache(cache, 5 - 3) == 2 and cache[0].offset == 3
    cache[0].update_and_fetch(rows(1, 3, H=2, D=64), rows(1, 4, H=2, D=64))
    assert cache[0].offset == 4
    assert trim_prompt_cache([], 1) == 0


@pytest.mark.parametrize("bits", [8, 4])
def test_nbytes(bits):
    c = QuantizedKVCache(group_size=64, bits=bits)
    c.update_and_fetch(rows(10, 5), rows(10, 6))
    cap = c.keys[0].shape[2]
    per_row = OC.row_bytes(128, bits)  # D*bits/8 + 2*(D/64)*2 bytes, context.py:169 per element
    assert c.nbytes == 2 * 1 * 2 * cap * per_row  # K and V, B=1, H=2
    p = KVCache()
    p.update_and_fetch(rows(10, 5), rows(10, 6))
    assert p.nbytes == 2 * 2 * p.keys.shape[2] * OC.row_bytes(128, None)


def test_to_quantized_and_safe_maybe_quantize():
    plain = KVCache()
    plain.update_and_fetch(rows(300, 7), rows(300, 8))

    class Rotating(KVCache):  # stands in for a sliding-window cache: never quantized
        pass

    rot = Rotating()
    rot.update_and_fetch(rows(300, 9), rows(300, 10))
    small = KVCache()
    small.update_and_fetch(rows(10, 11), rows(10, 12))
    caches = [plain, rot, small]
    A.safe_maybe_quantize_kv_cache(caches, quantized_kv_start=256, kv_group_size=64, kv_bits=8)
    assert isinstance(caches[0], QuantizedKVCache) and caches[0].offset == 300
    assert caches[1] is rot and caches[2] is small
    # the whole allocated buffer is quantized (mlx-lm semantics), offset rows included
    q = caches[0]
    rc, rs, rb = OQ.quantize(to_np_bits(plain.keys), "float16", 64, 8)
    gc, gs, gb = triple_to_np(q.keys)
    assert np.array_equal(gc, rc) and np.array_equal(gs, rs) and np.array_equal(gb, rb)
    A.safe_maybe_quantize_kv_cache(caches, 0, 64, None)  # kv_bits None: no-op
    assert caches[1] is rot


def test_decode_through_cache_views():
    # per-step decode as mlx-lm drives it: update_and_fetch, then attention over the views
    c = QuantizedKVCache(group_size=64, bits=8)
    c.update_and_fetch(rows(700, 20, H=4), rows(700, 21, H=4))
    for step in range(3):
        fk, fv = c.update_and_fetch(rows(1, 30 + step, H=4), rows(1, 40 + step, H=4))
        q = seeded_normal((1, 16, 1, 128), 50 + step, torch.float16, DEV)
        out = A.blocked_quantized_sdpa(q, fk, fv, 1.0 / math.sqrt(128), None)
        torch.cuda.synchronize()
        ref = exact_reference(q, fk, fv, 1.0 / math.sqrt(128), bits=8)
        assert_close(out, ref, f"step {step}")


@pytest.mark.parametrize("group,bits", [(32, 4), (128, 8)])
def test_group_sizes_through_cache_views(group, bits):
    # mlx-lm's other kv_group_size values: quantize a plain cache, then prefill and decode over it
    plain = KVCache()
    plain.update_and_fetch(rows(600, 60, H=4), rows(600, 61, H=4))
    caches = [plain]
    A.safe_maybe_quantize_kv_cache(caches, quantized_kv_start=0, kv_group_size=group, kv_bits=bits)
    c = caches[0]
    assert c.group_size == group and c.keys[1].shape[-1] == 128 // group
    scale = 1.0 / math.sqrt(128)
    for step, n in enumerate((90, 1, 1)):
        fk, fv = c.update_and_fetch(rows(n, 70 + step, H=4), rows(n, 80 + step, H=4))
        q = seeded_normal((1, 16, n, 128), 90 + step, torch.float16, DEV)
        out = A.blocked_quantized_sdpa(q, fk, fv, scale, "causal" if n > 1 else None, group_size=group, bits=bits)
        torch.cuda.synchronize()
        ref = exact_reference(q, fk, fv, scale, bits=bits, group_size=group, causal=n > 1)
        assert_close(out, ref, f"group={group} step {step}")
