"""The paged radix prefix cache (kvq_radix_*, host C++ in libkvq.so) on CPU.

The model in oracle/radix.py is pinned by the behaviour the reference's PagedRadixKVCache
documents (native/include/kv_cache.hpp:28-44, native/src/kv_cache.cpp:76-160): a committed
prompt re-submitted matches all its full pages but never the last prompt token; prompts sharing
k full pages share those k pages; a differing token stops the match; the pool size caps the
allocation and an exhausted pool is an error; eviction takes the least recently used cached
page. Pages held by a running sequence are never evicted (the reference count this build adds).
The C++ cache must then equal the model step for step on random workloads.
"""

import ctypes
import random

import pytest

from myinfer_amd import _lib
from myinfer_amd.paged import PageRadix
from oracle.radix import RadixModel


@pytest.mark.parametrize("P", [4, 16, 64])
def test_model_rematch_leaves_last_token(P):
    m = RadixModel(64, P)
    for n in (1, P - 1, P, P + 1, 3 * P, 3 * P + 5):
        toks = list(range(1000 * n, 1000 * n + n))
        table, got = m.match_and_allocate(toks, 0)
        assert got == 0
        m.commit(toks, table, n)
        m.release(table)
        table2, got2 = m.match_and_allocate(toks, 0)
        assert got2 == ((n - 1) // P) * P
        assert table2[: got2 // P] == table[: got2 // P]
        m.release(table2)


def test_model_shared_prefix_and_divergence():
    P = 4
    m = RadixModel(32, P)
    a = list(range(20))
    t, _ = m.match_and_allocate(a, 0)
    m.commit(a, t, len(a))
    b = a[:9] + [777] + a[10:]  # differs inside page 2
    tb, got = m.match_and_allocate(b, 0)
    assert got == 8 and tb[:2] == t[:2] and tb[2] not in t
    c = [5] + a[1:]  # differs in page 0
    tc, gotc = m.match_and_allocate(c, 0)
    assert gotc == 0


def test_model_capacity_holds_and_lru():
    P = 4
    m = RadixModel(6, P)
    a = list(range(8))  # 8 + 16 margin -> 6 pages
    ta, _ = m.match_and_allocate(a, 0)
    assert len(ta) == 6
    assert m.match_and_allocate(list(range(100, 104)), 0) is None  # every page is held
    m.commit(a, ta, 8)
    m.release(ta)
    # two cached pages; the oldest-touched one is evicted first once free pages run out
    tb, _ = m.match_and_allocate(list(range(200, 204)), 0)  # 5 pages: 4 free + 1 eviction
    assert len(tb) == 5
    st = m.stats()
    assert st["cached_pages"] == 1 and st["in_use_pages"] == 5
    # the first page was committed (touched) first, so it went first; the chain is now broken
    assert tuple(a[:4]) not in m.index and m.index[tuple(a[:8])] == ta[1]
    m.release(tb)
    t2, got = m.match_and_allocate(a, 0)
    assert got == 0


def test_model_held_pages_survive_eviction_pressure():
    P = 4
    m = RadixModel(10, P)
    a = list(range(12))
    ta, _ = m.match_and_allocate(a, 0)  # 7 pages, held
    m.commit(a, ta, 12)
    with pytest.raises(AssertionError):
        m.commit(a, [9], 4)  # page 9 is not held
    assert m.match_and_allocate(list(range(50, 60)), 0) is None  # needs 7, only 3 free
    st = m.stats()
    assert st["in_use_pages"] == 7 and st["cached_pages"] == 3


def _cxx_vs_model(seed, num_pages, P, steps):
    rng = random.Random(seed)
    r, m = PageRadix(num_pages, P), RadixModel(num_pages, P)
    bases = [[rng.randrange(50) for _ in range(rng.randrange(1, 6 * P))] for _ in range(5)]
    live = []
    for _ in range(steps):
        op = rng.random()
        if op < 0.5:
            base = rng.choice(bases)
            toks = base[: rng.randrange(1, len(base) + 1)] + [rng.randrange(50) for _ in range(rng.randrange(0, 2 * P))]
            new = rng.randrange(0, 2 * P)
            want = m.match_and_allocate(toks, new)
            if want is None:
                with pytest.raises(RuntimeError):
                    r.match_and_allocate(toks, new)
            else:
                got = r.match_and_allocate(toks, new)
                assert (got.block_table, got.matched_tokens) == want
                live.append((toks, got.block_table))
        elif op < 0.75 and live:
            toks, table = rng.choice(live)
            valid = rng.randrange(0, len(toks) + 1)
            m.commit(toks, table, valid)
            r.commit_prefix_blocks(toks, table, valid)
        elif op < 0.97 and live:
            toks, table = live.pop(rng.randrange(len(live)))
            m.release(table)
            r.release(table)
        else:
            m.clear()
            r.clear_cache()
        st = r.stats()
        for k, v in m.stats().items():
            assert st[k] == v, (k, st[k], v)


@pytest.mark.parametrize("seed", range(6))
def test_cxx_matches_model(seed):
    _cxx_vs_model(seed, num_pages=[12, 40, 200][seed % 3], P=[4, 16, 64][seed % 3], steps=400)


def test_errors():
    with pytest.raises(ValueError):
        PageRadix(0, 64)
    r = PageRadix(4, 4)
    t = r.match_and_allocate([1, 2, 3, 4, 5], 0)
    assert t.total_blocks_allocated == 4  # 5 + 16 margin -> 6 pages, capped at the pool
    with pytest.raises(ValueError):
        r.commit_prefix_blocks([1, 2, 3, 4, 5], [0, 1, 2, 3], 6)  # more valid tokens than tokens
    r.release(t.block_table)
    with pytest.raises(ValueError):
        r.commit_prefix_blocks([1, 2, 3, 4], [0], 4)  # page 0 is no longer held
    lib = _lib.lib()
    h = lib.kvq_radix_create(4, 4)
    table = (ctypes.c_int32 * 1)()
    a, b = ctypes.c_int(), ctypes.c_int()
    toks = (ctypes.c_int32 * 3)(1, 2, 3)
    assert lib.kvq_radix_match_and_allocate(h, toks, 3, 0, table, 1, ctypes.byref(a), ctypes.byref(b)) == _lib.ERR_INVALID
    assert b"capacity" in lib.kvq_radix_last_error()
    lib.kvq_radix_destroy(h)
