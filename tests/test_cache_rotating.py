"""The sliding-window cache (RotatingKVCache) on CPU tensors: its bookkeeping model in oracle/cache.py
is pinned by the properties a sliding-window cache must have, and the torch cache must match the
model row for row (keys carry their token position, so every fetched row names the token it holds).

Properties pinned: one-token updates keep exactly the `keep` first tokens plus the newest
max_size - keep tokens; multi-token updates return rows in temporal order ending with the new
tokens and carrying at least max_size - 1 earlier tokens; with make_mask, each new query sees
exactly the max_size newest tokens up to itself (keep = 0); trim / is_trimmable / state / nbytes
follow the cache contract the reference's prefix cache and footprint code read.
"""

import pytest
import torch

from myinfer_amd.cache import KVCache, RotatingKVCache, make_prompt_cache
from oracle.cache import RotatingCacheModel


def _tokens(lo, L, H=2, D=8):
    pos = torch.arange(lo, lo + L, dtype=torch.float32)
    k = pos[None, None, :, None].expand(1, H, L, D).clone()
    return k, -k


def _positions(t: torch.Tensor):
    return [int(x) for x in t[0, 0, :, 0].tolist()]


SCHEDULES = [
    [1] * 40,
    [5] + [1] * 30,
    [3, 1, 1, 7, 1, 1, 1, 12, 1, 1, 2, 1],
    [1] * 9 + [16] + [1] * 20 + [4] + [1] * 5,
    [20, 20, 1, 1, 20],
]


@pytest.mark.parametrize("max_size,keep,step", [(8, 0, 4), (8, 2, 3), (16, 4, 256), (5, 0, 2)])
@pytest.mark.parametrize("schedule", SCHEDULES)
def test_model_properties(max_size, keep, step, schedule):
    m = RotatingCacheModel(max_size, keep, step)
    for L in schedule:
        prev = m.offset
        rows = m.update(L)
        assert None not in rows
        assert len(set(rows)) == len(rows)
        new = list(range(prev, prev + L))
        if L == 1:
            if m.offset <= max_size:
                assert sorted(rows) == list(range(m.offset))
            else:
                assert len(rows) == max_size
                pinned = [p for p in rows if p < keep]
                assert len(pinned) == min(keep, len(rows))
                recent = sorted(p for p in rows if p >= keep)
                # the newest tokens, contiguous and ending with this one
                assert recent == list(range(m.offset - len(recent), m.offset))
        else:
            assert rows == sorted(rows), "multi-token fetch is not in temporal order"
            assert rows[-L:] == new
            earlier = rows[:-L]
            assert len(earlier) >= min(prev, max_size - 1)
            assert earlier[-1:] == ([prev - 1] if prev else [])


@pytest.mark.parametrize("max_size,keep,step", [(8, 0, 4), (8, 2, 3), (16, 4, 256), (5, 0, 2)])
@pytest.mark.parametrize("schedule", SCHEDULES)
def test_cache_matches_model(max_size, keep, step, schedule):
    c = RotatingKVCache(max_size, keep, step)
    m = RotatingCacheModel(max_size, keep, step)
    for L in schedule:
        k, v = _tokens(c.offset, L)
        fk, fv = c.update_and_fetch(k, v)
        rows = m.update(L)
        assert _positions(fk) == rows
        assert torch.equal(fv, -fk)
        assert c.offset == m.offset
        assert c.keys.shape[2] == len(m.rows)
        assert c.is_trimmable() == (c.offset < max_size)


@pytest.mark.parametrize("schedule", [[1] * 30, [6, 1, 1, 9, 1, 13, 1, 1]])
def test_make_mask_gives_each_query_its_window(schedule):
    W = 8
    c = RotatingKVCache(W, keep=0, step=4)
    for L in schedule:
        mask = c.make_mask(L)
        lo = c.offset
        k, v = _tokens(lo, L)
        fk, _ = c.update_and_fetch(k, v)
        pos = torch.tensor(_positions(fk))
        S = pos.numel()
        if mask is None:
            vis = torch.ones(L, S, dtype=torch.bool)
        elif isinstance(mask, str):
            vis = torch.arange(S)[None, :] <= (S - L + torch.arange(L))[:, None]
        else:
            vis = mask
        for i in range(L):
            q = lo + i
            want = sorted(p for p in range(max(0, q - W + 1), q + 1))
            got = sorted(int(p) for p in pos[vis[i]])
            assert got == want, (L, i, got, want)


def test_window_shorter_than_ring_rotated_mask():
    c = RotatingKVCache(8, keep=0, step=8)
    for t in range(13):
        c.update_and_fetch(*_tokens(t, 1))
    mask = c.make_mask(1, window_size=4)
    k, v = _tokens(13, 1)
    fk, _ = c.update_and_fetch(k, v)
    got = sorted(int(p) for p in torch.tensor(_positions(fk))[mask])
    assert got == [10, 11, 12, 13]


def test_trim_state_nbytes():
    c = RotatingKVCache(16, keep=0, step=8)
    assert c.state == (None, None) and c.nbytes == 0
    c.update_and_fetch(*_tokens(0, 5))
    assert c.is_trimmable()
    assert c.trim(2) == 2 and c.offset == 3
    k, _ = c.state
    assert _positions(k) == [0, 1, 2]
    c.update_and_fetch(*_tokens(3, 1))
    assert _positions(c.state[0]) == [0, 1, 2, 3]
    assert c.nbytes == c.keys.nbytes + c.values.nbytes
    with pytest.raises(NotImplementedError):
        c.to_quantized()


def test_rejects_bad_sizes():
    with pytest.raises(ValueError):
        RotatingKVCache(4, keep=4)
    with pytest.raises(ValueError):
        RotatingKVCache(0)


def test_make_prompt_cache_patterns():
    caches = make_prompt_cache(6, layer_windows=[1024] * 5 + [None])
    assert [type(c) for c in caches] == [RotatingKVCache] * 5 + [KVCache]
    assert all(c.max_size == 1024 and c.keep == 0 for c in caches[:5])
    caches = make_prompt_cache(3, max_kv_size=4096)
    assert all(isinstance(c, RotatingKVCache) and c.max_size == 4096 and c.keep == 4 for c in caches)
    assert all(type(c) is KVCache for c in make_prompt_cache(2))
    with pytest.raises(ValueError):
        make_prompt_cache(3, layer_windows=[None])
