"""Host-side logic of the reference-named API (myinfer_amd/attention.py) without a GPU: the block
rule and module globals of m5engine/attention.py:21-22, :40-41 (patched by tests/test_core.py:36-37),
the translation of reference-style masks into (causal, window, seq_lens), _slice_keys, install()."""

import types

import pytest
import torch

from myinfer_amd import attention as A
from oracle import attention as OA


def test_block_rule_reads_module_globals(monkeypatch):
    assert A.block_size(1, 32, 512) == OA.block_size(1, 32, 512)
    monkeypatch.setattr(A, "score_budget_bytes", 1)
    monkeypatch.setattr(A, "MIN_BLOCK", 128)
    assert A.block_size(1, 4, 6) == 128


def test_slice_keys():
    t = tuple(torch.arange(2 * 3 * 10 * 4).reshape(2, 3, 10, 4) for _ in range(3))
    s = A._slice_keys(t, 2, 7)
    assert all(x.shape == (2, 3, 5, 4) for x in s)
    assert torch.equal(s[0], t[0][..., 2:7, :])


def test_mask_none_and_string():
    assert A.mask_structure(None, 1, 8, 4, 100) == (False, 0, None)
    assert A.mask_structure("causal", 1, 8, 4, 100) == (True, 0, None)


def _mask(B, L, S, S_b, causal, window):
    k = torch.arange(S)[None, None, :]
    pos = (torch.tensor(S_b)[:, None] - L + torch.arange(L)[None, :])[:, :, None]
    m = k < torch.tensor(S_b)[:, None, None]
    if causal:
        m = m & (k <= pos)
    if window:
        m = m & (k > pos - window)
    return m[:, None]  # [B, 1, L, S]


@pytest.mark.parametrize("causal,window,lens", [(True, 0, [50, 50]), (True, 16, [50, 50]), (True, 0, [50, 21]),
                                                (False, 0, [50, 30]), (True, 8, [50, 33])])
def test_bool_masks_are_recognised(causal, window, lens):
    B, L, S = 2, 4, 50
    m = _mask(B, L, S, lens, causal, window)
    c, w, sl = A.mask_structure(m, B, 8, L, S)
    assert w == window
    if window:
        assert c
    elif L > 1:
        assert c == causal
    if all(x == S for x in lens):
        assert sl is None
    else:
        assert sl.tolist() == lens


def test_additive_and_unsupported_masks():
    assert A.mask_structure(torch.zeros(1, 1, 4, 50), 1, 8, 4, 50) == (False, 0, None)
    with pytest.raises(NotImplementedError):
        A.mask_structure(torch.full((1, 1, 4, 50), -1.0), 1, 8, 4, 50)
    random = torch.rand(1, 1, 4, 50) > 0.5
    with pytest.raises(NotImplementedError):
        A.mask_structure(random, 1, 8, 4, 50)
    with pytest.raises(ValueError):
        A.mask_structure(torch.ones(1, 1, 3, 50, dtype=torch.bool), 1, 8, 4, 50)


def test_install_is_idempotent(monkeypatch):
    monkeypatch.setattr(A, "_installed", False)
    monkeypatch.setattr(A, "_patched", set())
    base, gen = types.SimpleNamespace(), types.SimpleNamespace()
    A.install(base, gen)
    assert A._installed
    assert base.quantized_scaled_dot_product_attention is A.blocked_quantized_sdpa
    assert gen.maybe_quantize_kv_cache is A.safe_maybe_quantize_kv_cache
    # a second call on the same modules leaves an attribute a user changed since alone
    base.quantized_scaled_dot_product_attention = "user"
    A.install(base, gen)
    assert base.quantized_scaled_dot_product_attention == "user"
    # other modules are still patched
    other = types.SimpleNamespace()
    A.install(other, None)
    assert other.quantized_scaled_dot_product_attention is A.blocked_quantized_sdpa


def test_install_engine_sequence_without_host_framework(monkeypatch):
    # the reference engine calls install() with no arguments (m5engine/engine.py:138); without the
    # host framework that raises and patches nothing, so a later call with modules still installs
    monkeypatch.setattr(A, "_installed", False)
    monkeypatch.setattr(A, "_patched", set())
    monkeypatch.setattr(A, "HOST_BASE_MODULE", "no_such_host_framework.models.base")
    with pytest.raises(ImportError, match="no host framework"):
        A.install()
    assert not A._installed and not A._patched
    base, gen = types.SimpleNamespace(), types.SimpleNamespace()
    A.install(base, gen)
    assert base.quantized_scaled_dot_product_attention is A.blocked_quantized_sdpa
    assert gen.maybe_quantize_kv_cache is A.safe_maybe_quantize_kv_cache


def test_install_without_arguments_patches_named_modules(monkeypatch):
    import sys

    monkeypatch.setattr(A, "_installed", False)
    monkeypatch.setattr(A, "_patched", set())
    base, gen = types.ModuleType("fakehost_base"), types.ModuleType("fakehost_generate")
    monkeypatch.setitem(sys.modules, "fakehost_base", base)
    monkeypatch.setitem(sys.modules, "fakehost_generate", gen)
    monkeypatch.setattr(A, "HOST_BASE_MODULE", "fakehost_base")
    monkeypatch.setattr(A, "HOST_GENERATE_MODULE", "fakehost_generate")
    A.install()
    A.install()  # idempotent
    assert A._installed
    assert base.quantized_scaled_dot_product_attention is A.blocked_quantized_sdpa
    assert gen.maybe_quantize_kv_cache is A.safe_maybe_quantize_kv_cache


def test_mask_analysis_runs_once_per_mask(monkeypatch):
    # the layers of one forward pass share one mask object: it is analysed once, on the host, and
    # analysed again only after it is modified in place
    calls = []
    real = A._analyse_mask

    def counting(*a):
        calls.append(1)
        return real(*a)

    monkeypatch.setattr(A, "_analyse_mask", counting)
    monkeypatch.setattr(A, "_mask_cache", {})
    L, S = 4, 50
    m = torch.ones(1, 1, L, S, dtype=torch.bool).tril(S - L)
    first = A.mask_structure(m, 1, 8, L, S)
    for _ in range(5):
        assert A.mask_structure(m, 1, 8, L, S) == first
    assert len(calls) == 1 and first == (True, 0, None)
    m.fill_(True)  # modified in place: a new analysis, a new answer (every key visible)
    assert A.mask_structure(m, 1, 8, L, S) == (False, 0, None)
    assert len(calls) == 2


def test_mask_structure_under_inference_mode(monkeypatch):
    """A mask built under torch.inference_mode() has no version counter: it is analysed on every
    call (no cache entry), gives the same answers, and an in-place edit is seen."""
    calls = []
    real = A._analyse_mask

    def counting(*a):
        calls.append(1)
        return real(*a)

    monkeypatch.setattr(A, "_analyse_mask", counting)
    monkeypatch.setattr(A, "_mask_cache", {})
    L, S = 4, 50
    with torch.inference_mode():
        m = torch.ones(1, 1, L, S, dtype=torch.bool).tril(S - L)
        assert m.is_inference()
        assert A.mask_structure(m, 1, 8, L, S) == (True, 0, None)
        assert A.mask_structure(m, 1, 8, L, S) == (True, 0, None)
        w = A.mask_structure(m & ~torch.ones(L, S, dtype=torch.bool).tril(S - L - 3), 1, 8, L, S)
        assert w == (True, 3, None)
        m.fill_(True)
        assert A.mask_structure(m, 1, 8, L, S) == (False, 0, None)
    assert len(calls) == 4 and A._mask_cache == {}
    # outside inference mode too (the tensor is still an inference tensor)
    assert A.mask_structure(m, 1, 8, L, S) == (False, 0, None)


def test_prepared_call_rejects_inputs_it_would_copy(monkeypatch):
    """A prepared call reads its tensors in place on every launch; a query or unquantized K/V that
    the kernels cannot read directly (here: strided along D) raises instead of being snapshotted.
    The checks run on the host before any library call (the device check is stubbed to run here)."""
    from myinfer_amd import kernels as K

    monkeypatch.setattr(K, "_require_cuda", lambda *t: t[0].device)
    B, Hq, Hkv, L, S, D = 1, 8, 2, 4, 64, 128
    q = torch.zeros(B, Hq, L, 2 * D, dtype=torch.float16)[..., ::2]  # stride 2 along D
    k = torch.zeros(B, Hkv, S, D, dtype=torch.float16)
    v = torch.zeros(B, Hkv, S, D, dtype=torch.float16)
    with pytest.raises(ValueError, match="queries need unit stride"):
        K.prepare_attention(q, k, v, 0.1)
    with pytest.raises(ValueError, match="keys need unit stride"):
        K.prepare_attention(q.contiguous(), torch.zeros(B, Hkv, S, 2 * D, dtype=torch.float16)[..., ::2], v, 0.1)
    codes = torch.zeros(B, Hkv, S, D // 4, dtype=torch.int32).view(torch.uint32)
    sb = torch.zeros(B, Hkv, S, D // 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="queries need unit stride"):
        K.prepare_attention(q, (codes, sb, sb), (codes, sb, sb), 0.1)
