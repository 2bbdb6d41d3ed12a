"""kernels.mask_view (CPU): the (tensor, strides) a general mask is read through must address, for
query head h = kvh * rep + j, the element each reference path broadcasts to that head."""

import pytest
import torch

from myinfer_amd import kernels


def _read(view, strides, B, Hkv, rep, L, S):
    t, (sb, skv, srep, sl) = view, strides
    flat = torch.as_strided(t, (B, Hkv, rep, L, S), (sb, skv, srep, sl, 1))
    return flat.reshape(B, Hkv * rep, L, S)


@pytest.mark.parametrize("shape", [(7, 30), (2, 1, 7, 30), (2, 8, 7, 30), (1, 1, 1, 30), (7, 1)])
def test_heads_layout(shape):
    B, Hq, Hkv, L, S = 2, 8, 2, 7, 30
    m = torch.rand(*shape) < 0.5
    v, st = kernels.mask_view(m, B, Hq, Hkv, L, S, "heads")
    assert torch.equal(_read(v, st, B, Hkv, Hq // Hkv, L, S), torch.broadcast_to(m, (B, Hq, L, S)))


def test_blocked_layout_indexes_kv_heads():
    B, Hq, Hkv, L, S = 2, 8, 2, 5, 16
    m = torch.rand(B, Hkv, L, S) < 0.5
    v, st = kernels.mask_view(m, B, Hq, Hkv, L, S, "blocked")
    want = m[:, torch.arange(Hq) // (Hq // Hkv)]
    assert torch.equal(_read(v, st, B, Hkv, Hq // Hkv, L, S), want)
    # rank 2 gains no head axis
    m2 = torch.rand(L, S) < 0.5
    v2, st2 = kernels.mask_view(m2, B, Hq, Hkv, L, S, "blocked")
    assert torch.equal(_read(v2, st2, B, Hkv, Hq // Hkv, L, S), torch.broadcast_to(m2, (B, Hq, L, S)))


def test_grouped_layout_indexes_the_repeat_axis():
    B, Hq, Hkv, L, S = 1, 8, 2, 1, 16
    rep = Hq // Hkv
    m = torch.rand(1, rep, 1, S) < 0.5
    v, st = kernels.mask_view(m, B, Hq, Hkv, L, S, "grouped")
    want = m[0][torch.arange(Hq) % rep][None]
    assert torch.equal(_read(v, st, B, Hkv, rep, L, S), want)


def test_rejects_what_does_not_broadcast():
    with pytest.raises(ValueError):
        kernels.mask_view(torch.ones(3, 7, 30, dtype=torch.bool), 2, 8, 2, 7, 30, "heads")
    with pytest.raises(ValueError):
        kernels.mask_view(torch.ones(7, 29, dtype=torch.bool), 2, 8, 2, 7, 30, "heads")
    with pytest.raises(ValueError):
        kernels.mask_view(torch.ones(7, 30, dtype=torch.int32), 2, 8, 2, 7, 30, "heads")
