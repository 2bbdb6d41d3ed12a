"""Memory-bounded attention over a quantized KV cache, on MI355X.

Drop-in counterpart of m5engine/attention.py: the same public names and argument meaning,
over torch tensors in MLX layout on the GPU, executed by libkvq.so's HIP kernels.

  blocked_quantized_sdpa(queries, q_keys, q_values, scale, mask, group_size=64, bits=8)
      reference: m5engine/attention.py:29-103. The GPU kernels stream the cache in 32-key
      tiles with an online softmax (split-K decode for small L, MFMA tiles for prefill), so no
      score matrix is ever materialised; the only transient memory is the split workspace.
  quantized_scaled_dot_product_attention(...)
      the L == 1 entry mlx-lm calls (captured at m5engine/attention.py:19, used at :42-45);
      here it is the same kernels.
  fast_scaled_dot_product_attention(queries, keys, values, scale, mask)
      attention over an unquantized cache (mlx's mx.fast.scaled_dot_product_attention, which
      mlx-lm uses for the caches m5engine/attention.py:106-112 leaves unquantized: the plain
      cache before quantized_kv_start and the sliding-window RotatingKVCache layers).
  scaled_dot_product_attention(queries, keys, values, cache, scale, mask)
      mlx-lm's dispatcher between the two, by the cache's type.
  safe_maybe_quantize_kv_cache(prompt_cache, quantized_kv_start, kv_group_size, kv_bits)
      reference: m5engine/attention.py:106-112.
  install(base_module=None, generate_module=None)
      reference: m5engine/attention.py:115-126 (idempotent patch of the host framework's
      quantized-SDPA and cache-quantization hooks).

``score_budget_bytes`` and ``MIN_BLOCK`` keep the reference's values (:21-22) and its block rule
(:40-41, ``block_size``) for callers and tests that read them; the GPU path does not need them.

Masks (the reference accepts None, a string, or an array):
  None                  every cached key is visible
  any str               causal, queries at positions S - L .. S - 1 (reference :55-58)
  bool tensor           a causal mask, a causal sliding window, or either with right padding per
                        batch row (keys >= S_b masked), is recognised and runs as that structure;
                        any other boolean mask (per-head masks included) is read by the kernel
  additive float        all-zero runs unmasked; any other is added to the scores by the kernel
General masks (kernels.masked_attention) run on the decode kernel for any L, broadcast as the
reference broadcasts them on the same path; a row that sees no key returns 0.
Keyword extensions: ``window=`` (sliding window) and ``seq_lens=`` (int32 [B] valid key counts)
give the same structure without building a mask.
"""

from __future__ import annotations

import weakref
from typing import Optional

import torch

from . import kernels
from .cache import KVCache

score_budget_bytes = 512 * 1024**2
MIN_BLOCK = 256


def block_size(B: int, n_q_heads: int, L: int) -> int:
    """The reference's key-block length (m5engine/attention.py:40-41), read at call time."""
    per_key = B * n_q_heads * L * 4 * 3
    return max(MIN_BLOCK, score_budget_bytes // max(per_key, 1))


def _slice_keys(q, start, end):
    """Slice every member of a (codes, scales, biases) triple along the key axis (:25-26)."""
    return tuple(x[..., start:end, :] for x in q)


def _expected_mask(L: int, S: int, S_b: torch.Tensor, causal: bool, window: int, device) -> torch.Tensor:
    k = torch.arange(S, device=device)[None, None, :]
    pos = (S_b[:, None] - L + torch.arange(L, device=device)[None, :])[:, :, None]
    m = k < S_b[:, None, None]
    if causal:
        m = m & (k <= pos)
    if window > 0:
        m = m & (k > pos - window)
    return m.expand(S_b.shape[0], L, S)


# Analysed boolean / float masks: id(mask) -> (weak reference, version, shape key, result). A model
# builds one mask per forward pass and hands it to every layer; the analysis (a host pass over the
# mask) then runs once for all of them, and a mask on the host never costs a device synchronization.
_mask_cache: dict = {}


def mask_structure(mask, B: int, n_q_heads: int, L: int, S: int, device=None):
    """Translate a reference-style mask into (causal, window, seq_lens) for the kernels.

    String and None masks cost nothing. An array mask is analysed on the host (a device mask is
    copied there once) and the result is cached for that mask object until it is modified, so the
    layers of one forward pass share one analysis. A mask created under torch.inference_mode() has
    no version counter and is analysed on every call (callers in a serving loop pass ``window=`` /
    ``seq_lens=`` to skip the analysis). seq_lens comes back as an int32 tensor on `device`
    (default: the mask's device)."""
    if mask is None:
        return False, 0, None
    if isinstance(mask, str):
        return True, 0, None
    if not torch.is_tensor(mask):
        raise NotImplementedError(f"unsupported mask type {type(mask)}")
    device = torch.device(device) if device is not None else mask.device
    # A tensor made under torch.inference_mode() has no version counter, so an in-place edit of it
    # could not be told from the cached analysis: such masks are analysed on every call.
    versioned = not mask.is_inference()
    key = (B, n_q_heads, L, S, str(device))
    if versioned:
        hit = _mask_cache.get(id(mask))
        if hit is not None and hit[0]() is mask and hit[1] == mask._version and hit[2] == key:
            if isinstance(hit[3], NotImplementedError):
                raise NotImplementedError(str(hit[3]))
            return hit[3]
    try:
        causal, window, seq = _analyse_mask(mask.detach().cpu(), B, n_q_heads, L, S)
        res = (causal, window, None if seq is None else seq.to(device))
    except NotImplementedError as e:
        res = e  # remembered too: the layers of a forward pass do not analyse a general mask again
    if versioned:
        if len(_mask_cache) > 64:
            _mask_cache.clear()
        _mask_cache[id(mask)] = (weakref.ref(mask), mask._version, key, res)
    if isinstance(res, NotImplementedError):
        raise NotImplementedError(str(res))
    return res


def _analyse_mask(mask: torch.Tensor, B: int, n_q_heads: int, L: int, S: int):
    """mask_structure for a host tensor (seq_lens on the host)."""
    if mask.dtype != torch.bool:
        if bool((mask == 0).all()):
            return False, 0, None
        raise NotImplementedError("additive masks other than all-zero are not supported by the GPU kernels")
    m = mask
    while m.dim() < 4:
        m = m.unsqueeze(0)
    if m.shape[-1] != S or m.shape[-2] not in (1, L):
        raise ValueError(f"mask's last two dims {tuple(m.shape[-2:])} do not broadcast to (L, S) = {(L, S)}")
    m = m.expand(B, m.shape[1], L, S)  # a size-1 query axis broadcasts, as in the reference's slicing
    if m.shape[1] > 1 and not bool((m == m[:, :1]).all()):
        raise NotImplementedError("per-head masks are not supported by the GPU kernels")
    m = m[:, 0]  # [B, L, S]
    # valid key count of each sequence = one past the last visible key of its last query row
    last = m[:, L - 1]
    idx = torch.arange(1, S + 1, device=m.device)
    S_b = torch.where(last, idx, torch.zeros_like(idx)).amax(dim=1)
    first_row_count = m[:, L - 1].sum(dim=1)
    full = bool((S_b == S).all())
    for causal in (True, False):
        # window = number of visible keys of the last row when it is smaller than S_b
        win_t = torch.where(first_row_count < S_b, first_row_count, torch.zeros_like(first_row_count))
        windows = set(win_t.tolist())
        if len(windows) != 1:
            continue
        window = int(windows.pop())
        if window and not causal:
            continue
        if bool(torch.equal(m, _expected_mask(L, S, S_b, causal, window, m.device))):
            seq = None if full else S_b.to(torch.int32)
            return causal, window, seq
    raise NotImplementedError("this boolean mask is not a causal / sliding-window / right-padding mask")


def blocked_quantized_sdpa(queries: torch.Tensor, q_keys, q_values, scale: float, mask, group_size: int = 64,
                           bits: int = 8, *, window: int = 0, seq_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(scale * Q K^T + mask) V over an affine-quantized cache (m5engine/attention.py:29-103).

    queries [B, Hq, L, D] (float16/bfloat16, CUDA); q_keys, q_values: (codes uint32
    [B, Hkv, S, D*bits/32], scales, biases [B, Hkv, S, D/group_size]) in the queries' dtype.
    Query head h reads KV head h // (Hq / Hkv) (:47-53). Returns [B, Hq, L, D] in the queries'
    dtype. Rows that see no key return 0, as the reference's blocked path does.
    """
    B, n_q_heads, L, D = queries.shape
    S = q_keys[0].shape[-2]
    try:
        causal, window, seq_lens = _resolve_mask(mask, B, n_q_heads, L, S, window, seq_lens, queries.device)
    except NotImplementedError:
        if window or seq_lens is not None:
            raise
        # a general mask, broadcast as the reference does: a rank >= 3 mask gains a KV-head axis
        # before it meets the grouped [B, Hkv, rep, L, S] scores, in the blocked loop (:55-56) and in
        # the hand-off to mlx-lm's quantized SDPA (:42-45) alike
        return kernels.masked_attention(queries, tuple(q_keys), tuple(q_values), scale, mask, layout="blocked",
                                        group_size=group_size, bits=bits)
    return kernels.attention(queries, tuple(q_keys), tuple(q_values), scale, causal=causal, window=window,
                             seq_lens=seq_lens, group_size=group_size, bits=bits)


def _resolve_mask(mask, B: int, n_q_heads: int, L: int, S: int, window: int, seq_lens, device=None):
    """(causal, window, seq_lens) from a reference-style mask plus the keyword extensions."""
    causal, mwin, mseq = mask_structure(mask, B, n_q_heads, L, S, device=device)
    if window and mwin and window != mwin:
        raise ValueError(f"window={window} disagrees with the mask's window {mwin}")
    window = window or mwin
    if seq_lens is None:
        seq_lens = mseq
    if window and not causal:
        causal = True
    return causal, window, seq_lens


def fast_scaled_dot_product_attention(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float,
                                      mask=None, *, window: int = 0,
                                      seq_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(scale * Q K^T + mask) V over an unquantized cache: the counterpart of
    mx.fast.scaled_dot_product_attention, which mlx-lm calls for every cache that is not quantized
    (the KVCache before quantized_kv_start, and the RotatingKVCache sliding-window layers that
    m5engine/attention.py:106-112 leaves unquantized).

    queries [B, Hq, L, D]; keys, values [B, Hkv, S, D] in the queries' dtype (float16/bfloat16,
    CUDA). Masks as for blocked_quantized_sdpa. Returns [B, Hq, L, D].
    """
    B, n_q_heads, L, D = queries.shape
    S = keys.shape[-2]
    try:
        causal, window, seq_lens = _resolve_mask(mask, B, n_q_heads, L, S, window, seq_lens, queries.device)
    except NotImplementedError:
        if window or seq_lens is not None:
            raise
        # a general mask broadcasts against the [B, Hq, L, S] scores, as mx.fast's does
        return kernels.masked_attention(queries, keys, values, scale, mask, layout="heads")
    return kernels.attention(queries, keys, values, scale, causal=causal, window=window, seq_lens=seq_lens)


def scaled_dot_product_attention(queries, keys, values, cache, scale: float, mask, sinks=None):
    """mlx-lm's models.base.scaled_dot_product_attention: a quantized cache (one with ``bits``)
    goes to the quantized path, any other cache to the unquantized kernels."""
    if sinks is not None:
        raise NotImplementedError("attention sinks are not supported by the GPU kernels")
    if hasattr(cache, "bits"):
        return quantized_scaled_dot_product_attention(queries, keys, values, scale, mask,
                                                      group_size=cache.group_size, bits=cache.bits)
    return fast_scaled_dot_product_attention(queries, keys, values, scale, mask)


def quantized_scaled_dot_product_attention(queries, q_keys, q_values, scale, mask, group_size: int = 64,
                                           bits: int = 8):
    """The entry mlx-lm's models call for quantized caches; same kernels as the blocked path."""
    return blocked_quantized_sdpa(queries, q_keys, q_values, scale, mask, group_size, bits)


def safe_maybe_quantize_kv_cache(prompt_cache, quantized_kv_start, kv_group_size, kv_bits) -> None:
    """Quantize only plain KV caches; sliding-window and recurrent caches stay as-is
    (m5engine/attention.py:106-112). Mutates `prompt_cache` in place."""
    if kv_bits is None:
        return
    for i, c in enumerate(prompt_cache):
        if type(c) is KVCache and c.offset >= quantized_kv_start:
            prompt_cache[i] = c.to_quantized(group_size=kv_group_size, bits=kv_bits)


# The host framework's modules that install() patches when it is called without arguments, as the
# reference's engine calls it (m5engine/engine.py:138): the same two mlx-lm modules the reference
# patches (m5engine/attention.py:122-125). A host framework with other module names sets these.
HOST_BASE_MODULE = "mlx_lm.models.base"
HOST_GENERATE_MODULE = "mlx_lm.generate"

_installed = False
_patched: set = set()  # (id(module), attribute) pairs already routed here


def _patch(module, attr: str, fn) -> None:
    setattr(module, attr, fn)
    _patched.add((id(module), attr))


def install(base_module=None, generate_module=None) -> None:
    """Route a host framework's quantized attention and cache quantization to this module
    (m5engine/attention.py:118-126): sets `quantized_scaled_dot_product_attention` on the base
    module and `maybe_quantize_kv_cache` on the generate module.

    Called with no arguments (the reference engine's call, m5engine/engine.py:138) it imports the
    modules named by HOST_BASE_MODULE / HOST_GENERATE_MODULE and patches them; if they cannot be
    imported it raises ImportError and patches nothing, so a later call can still install. Modules
    passed in are patched whatever an earlier call did. Idempotent per module."""
    global _installed
    if base_module is None and generate_module is None:
        import importlib

        try:
            base_module = importlib.import_module(HOST_BASE_MODULE)
            generate_module = importlib.import_module(HOST_GENERATE_MODULE)
        except ImportError as e:
            raise ImportError(
                f"install() found no host framework to patch ({HOST_BASE_MODULE}, {HOST_GENERATE_MODULE}: {e}); "
                "pass the modules, as install(base_module, generate_module), or set HOST_BASE_MODULE / "
                "HOST_GENERATE_MODULE") from e
    if base_module is not None and (id(base_module), "quantized_scaled_dot_product_attention") not in _patched:
        _patch(base_module, "quantized_scaled_dot_product_attention", blocked_quantized_sdpa)
    if generate_module is not None and (id(generate_module), "maybe_quantize_kv_cache") not in _patched:
        _patch(generate_module, "maybe_quantize_kv_cache", safe_maybe_quantize_kv_cache)
    _installed = bool(_patched)
