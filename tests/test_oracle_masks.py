"""Pins the general-mask arguments of oracle.attention.exact_attention (vis: visible keys, add:
added to the scores), by what the mathematics fixes rather than by a second restatement:

* a boolean mask equal to the causal (or windowed) key mask gives exactly the causal result;
* adding log(c_j) to key j's score weights it c_j times: the same as a cache where key j appears
  c_j times; adding a per-row constant changes nothing (softmax invariance);
* a row whose keys are all hidden returns 0; hiding key j equals deleting it from the cache;
* a scalar brute force (one query, explicit sums) on a tiny case with both masks.
"""

import math

import numpy as np

from oracle import attention as A


def _data(seed, B=2, Hq=4, Hkv=2, L=5, S=23, D=8):
    r = np.random.default_rng(seed)
    return (r.standard_normal((B, Hq, L, D)), r.standard_normal((B, Hkv, S, D)), r.standard_normal((B, Hkv, S, D)))


def test_bool_mask_equal_to_causal_window():
    q, k, v = _data(1)
    B, Hq, L, _ = q.shape
    S = k.shape[2]
    for window in (0, 6):
        m = A.key_mask(L, S, S, True, window)  # [L, S]
        got = A.exact_attention(q, k, v, 0.3, vis=m)
        ref = A.exact_attention(q, k, v, 0.3, causal=True, window=window)
        assert np.array_equal(got, ref)


def test_additive_log_multiplicity_and_row_shift():
    q, k, v = _data(2, B=1)
    S = k.shape[2]
    counts = np.random.default_rng(3).integers(1, 4, size=S)
    idx = np.repeat(np.arange(S), counts)
    got = A.exact_attention(q, k, v, 0.25, add=np.log(counts)[None, None, None, :])
    ref = A.exact_attention(q, k[:, :, idx], v[:, :, idx], 0.25)
    assert np.abs(got - ref).max() < 1e-12
    shift = np.log(counts)[None, None, None, :] + np.arange(q.shape[2])[None, None, :, None] * 5.0
    got2 = A.exact_attention(q, k, v, 0.25, add=shift)
    assert np.abs(got2 - got).max() < 1e-12


def test_hidden_rows_and_deleted_keys():
    q, k, v = _data(4)
    B, Hq, L, _ = q.shape
    S = k.shape[2]
    vis = np.ones((B, Hq, L, S), bool)
    vis[1, 3, 2] = False  # one row sees nothing
    vis[:, :, :, 7] = False  # key 7 hidden everywhere
    got = A.exact_attention(q, k, v, 0.4, vis=vis)
    assert np.all(got[1, 3, 2] == 0.0)
    keep = np.array([j for j in range(S) if j != 7])
    ref = A.exact_attention(q, k[:, :, keep], v[:, :, keep], 0.4)
    rows = np.ones((B, Hq, L), bool)
    rows[1, 3, 2] = False
    assert np.abs(got[rows] - ref[rows]).max() < 1e-12


def test_scalar_brute_force_with_both_masks():
    q, k, v = _data(5, B=1, Hq=2, Hkv=1, L=2, S=6, D=3)
    r = np.random.default_rng(6)
    vis = r.random((1, 2, 2, 6)) > 0.3
    vis[..., 0] = True
    add = r.standard_normal((1, 2, 2, 6))
    got = A.exact_attention(q, k, v, 0.7, vis=vis, add=add)
    for h in range(2):
        for l in range(2):
            sc = [sum(q[0, h, l, d] * k[0, 0, j, d] for d in range(3)) * 0.7 + add[0, h, l, j] for j in range(6)]
            w = [math.exp(sc[j]) if vis[0, h, l, j] else 0.0 for j in range(6)]
            z = sum(w)
            for d in range(3):
                assert abs(got[0, h, l, d] - sum(w[j] * v[0, 0, j, d] for j in range(6)) / z) < 1e-12
