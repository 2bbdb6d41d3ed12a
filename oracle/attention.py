"""CPU oracles for attention over a quantized KV cache. TEST INFRASTRUCTURE ONLY.

exact_attention   softmax(scale * q K^T + mask) V over the exactly dequantized cache, in fp64.
                  This is the parity gate for the GPU kernels. It restates the quantity that
                  m5engine/attention.py:29-103 computes and that tests/test_core.py:16-20
                  (_ref_attention) takes as ground truth: dense scores over mx.dequantize'd
                  K/V, GQA by repeating each KV head over its Hq/Hkv query heads (:32-33),
                  causal as q_pos = arange(S - L, S) >= key index (:34).
reference_sdpa    a torch-CPU port of m5engine/attention.py:29-103 with the reference's block
                  rule (:38-45) and dtype casts (:49, :66-69, :87-90, :100), falling back to
                  mlx-lm's original quantized SDPA for L == 1 or short S (:42-45). Used as the
                  timed CPU baseline and as an informative "reference-faithful" comparison.
                  Unknowns of the third-party kernels it models are choices stated below.

Mask structure (the build's drop-in boundary converts the reference's masks to it):
  seq_lens[b]  keys [0, S_b) exist for sequence b (None: S_b = S)
  causal       query l sits at position S_b - L + l and sees keys <= position
  window       if > 0, keys k > position - window only
"""

from __future__ import annotations

import math

import numpy as np

from . import quantize as Q

NEG = -1e30


def key_mask(L: int, S: int, S_b: int, causal: bool, window: int) -> np.ndarray:
    """bool [L, S]: which keys each query row of a sequence with S_b keys may see."""
    k = np.arange(S)[None, :]
    pos = (S_b - L + np.arange(L))[:, None]
    m = np.broadcast_to(k < S_b, (L, S)).copy()
    if causal:
        m &= k <= pos
    if window > 0:
        m &= k > pos - window
    return m


def exact_attention(q: np.ndarray, kdq: np.ndarray, vdq: np.ndarray, scale: float, *, causal: bool = False,
                    window: int = 0, seq_lens=None, vis=None, add=None) -> np.ndarray:
    """fp64 attention. q [B, Hq, L, D]; kdq/vdq dequantized [B, Hkv, S, D]. Rows with no visible
    key return 0 (the value the reference's blocked path yields: acc / max(denom, 1e-30)).

    General masks, per query head (m5engine/attention.py:76-80 after its GQA broadcast): vis, a
    boolean array broadcastable to [B, Hq, L, S] (False hides the key, :77-78 and :81-82); add, an
    array broadcastable to [B, Hq, L, S] added to scale * q.k (:79-80)."""
    q = np.asarray(q, np.float64)
    B, Hq, L, D = q.shape
    Hkv, S = kdq.shape[1], kdq.shape[2]
    rep = Hq // Hkv
    vis = None if vis is None else np.broadcast_to(np.asarray(vis, bool), (B, Hq, L, S))
    add = None if add is None else np.broadcast_to(np.asarray(add, np.float64), (B, Hq, L, S))
    out = np.zeros((B, Hq, L, vdq.shape[-1]), np.float64)
    for b in range(B):
        S_b = S if seq_lens is None else int(seq_lens[b])
        if S_b <= 0:
            continue  # no key at all: every row of the sequence stays 0
        m = key_mask(L, S, S_b, causal, window)[:, :S_b]
        for h in range(Hkv):
            K = np.asarray(kdq[b, h, :S_b], np.float64)
            V = np.asarray(vdq[b, h, :S_b], np.float64)
            qg = q[b, h * rep:(h + 1) * rep].reshape(rep * L, D)
            s = (qg @ K.T) * scale
            s = s.reshape(rep, L, S_b)
            s = np.where(m[None], s, -np.inf)
            if vis is not None:
                s = np.where(vis[b, h * rep:(h + 1) * rep, :, :S_b], s, -np.inf)
            if add is not None:
                s = s + add[b, h * rep:(h + 1) * rep, :, :S_b]
            mx = s.max(axis=-1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            p = np.exp(s - mx)
            den = p.sum(axis=-1, keepdims=True)
            o = (p.reshape(rep * L, S_b) @ V).reshape(rep, L, -1)
            out[b, h * rep:(h + 1) * rep] = np.where(den > 0, o / np.where(den > 0, den, 1.0), 0.0)
    return out


def exact_from_quantized(q, k_triple, v_triple, dtype: str, scale: float, *, group_size=64, bits=8, **mask):
    """exact_attention over (codes, scale_bits, bias_bits) triples (numpy, uint16 storage)."""
    kdq = Q.dequantize(*k_triple, dtype, group_size, bits)
    vdq = Q.dequantize(*v_triple, dtype, group_size, bits)
    return exact_attention(q, kdq, vdq, scale, **mask)


# ---------------------------------------------------------------- reference-faithful port
def _torch():
    import torch

    return torch


def _dequant_T(triple, group_size, bits, T):
    """mx.quantized_matmul's dequantization on the CPU: scale * T(code) + bias, each op in T
    (chosen model: MLX's CPU kernels form the weight in the activation type)."""
    torch = _torch()
    codes, scales, biases = triple
    per = 32 // bits
    shifts = torch.arange(per, dtype=torch.int64) * bits
    w = (codes.to(torch.int64)[..., None] >> shifts) & ((1 << bits) - 1)
    w = w.reshape(*codes.shape[:-1], codes.shape[-1] * per)
    D = w.shape[-1]
    wg = w.reshape(*w.shape[:-1], D // group_size, group_size).to(T)
    prod = (wg.float() * scales.float()[..., None]).to(T)
    return (prod.float() + biases.float()[..., None]).to(T).reshape(*w.shape)


def _qmm(x, triple, transpose: bool, group_size, bits):
    """mx.quantized_matmul: x @ W^T (transpose) or x @ W, output in x's dtype. Chosen model of the
    unpinned third-party kernel: weights dequantized in T, fp32 accumulation, one rounding."""
    T = x.dtype
    W = _dequant_T(triple, group_size, bits, T).float()
    out = x.float() @ (W.transpose(-1, -2) if transpose else W)
    return out.to(T)


def block_size(B: int, n_q_heads: int, L: int, score_budget_bytes: int = 512 * 1024**2, min_block: int = 256) -> int:
    """The reference's key-block rule, m5engine/attention.py:40-41."""
    per_key = B * n_q_heads * L * 4 * 3
    return max(min_block, score_budget_bytes // max(per_key, 1))


def original_sdpa(queries, q_keys, q_values, scale, mask, group_size=64, bits=8):
    """mlx-lm quantized_scaled_dot_product_attention (third-party, mlx-lm==0.31.3), restated:
    q *= scale (T); scores = qmm(q, K) (T); masks; softmax(precise) -> T; out = qmm(p, V)."""
    torch = _torch()
    B, Hq, L, D = queries.shape
    Hkv, S = q_keys[0].shape[-3], q_keys[0].shape[-2]
    rep = Hq // Hkv
    T = queries.dtype
    q = (queries.float() * scale).to(T)
    if rep > 1:
        q = q.reshape(B, Hkv, rep, L, D)
        q_keys = tuple(x.unsqueeze(-3) for x in q_keys)
        q_values = tuple(x.unsqueeze(-3) for x in q_values)
    scores = _qmm(q, q_keys, True, group_size, bits)
    if mask is not None:
        if isinstance(mask, str):
            qi = torch.arange(S - L, S)[:, None]
            ki = torch.arange(S)[None]
            valid = qi >= ki
            scores = torch.where(valid, scores, torch.tensor(torch.finfo(T).min, dtype=T))
        elif mask.dtype == torch.bool:
            mk = mask.unsqueeze(-3) if (rep > 1 and mask.dim() >= 3) else mask
            scores = torch.where(mk, scores, torch.tensor(torch.finfo(T).min, dtype=T))
        else:
            scores = (scores.float() + mask.float()).to(T)
    p = torch.softmax(scores.float(), dim=-1).to(T)
    out = _qmm(p, q_values, False, group_size, bits)
    return out.reshape(B, Hq, L, -1) if rep > 1 else out


def reference_sdpa(queries, q_keys, q_values, scale, mask, group_size=64, bits=8, *,
                   score_budget_bytes=512 * 1024**2, min_block=256):
    """Port of blocked_quantized_sdpa, m5engine/attention.py:29-103, in torch on the CPU.
    queries: torch T [B, Hq, L, D]; q_keys/q_values: torch (codes int32/uint32, scales T, biases T)."""
    torch = _torch()
    B, n_q_heads, L, D = queries.shape
    S = q_keys[0].shape[-2]
    block = block_size(B, n_q_heads, L, score_budget_bytes, min_block)
    if S <= block or L == 1:
        return original_sdpa(queries, q_keys, q_values, scale, mask, group_size, bits)
    n_kv_heads = q_keys[0].shape[-3]
    n_repeats = n_q_heads // n_kv_heads
    T = queries.dtype
    q = (queries.float() * scale).to(T)
    if n_repeats > 1:
        q = q.reshape(B, n_kv_heads, n_repeats, L, D)
        q_keys = tuple(x.unsqueeze(-3) for x in q_keys)
        q_values = tuple(x.unsqueeze(-3) for x in q_values)
    causal = isinstance(mask, str)
    if mask is not None and not causal and n_repeats > 1 and mask.dim() >= 3:
        mask = mask.unsqueeze(-3)
    q_pos = torch.arange(S - L, S)[:, None] if causal else None
    m = denom = acc = None
    for start in range(0, S, block):
        end = min(S, start + block)
        ks = tuple(x[..., start:end, :] for x in q_keys)
        vs = tuple(x[..., start:end, :] for x in q_values)
        scores = _qmm(q, ks, True, group_size, bits).float()
        valid = None
        if causal:
            if end > S - L:
                valid = q_pos >= torch.arange(start, end)[None]
        elif mask is not None:
            blk = mask[..., start:end]
            if blk.dtype == torch.bool:
                valid = blk
            else:
                scores = scores + blk.float()
        if valid is not None:
            scores = torch.where(valid, scores, torch.tensor(NEG, dtype=torch.float32))
        blk_max = scores.amax(dim=-1, keepdim=True)
        m_new = blk_max if m is None else torch.maximum(m, blk_max)
        p = torch.exp(scores - m_new)
        if valid is not None:
            p = torch.where(valid, p, torch.zeros((), dtype=torch.float32))
        pv = _qmm(p.to(T), vs, False, group_size, bits).float()
        if m is None:
            denom = p.sum(dim=-1, keepdim=True)
            acc = pv
        else:
            corr = torch.exp(m - m_new)
            denom = denom * corr + p.sum(dim=-1, keepdim=True)
            acc = acc * corr + pv
        m = m_new
    out = (acc / torch.clamp(denom, min=1e-30)).to(T)
    if n_repeats > 1:
        out = out.reshape(B, n_q_heads, L, -1)
    return out


def error_stats(out: np.ndarray, ref: np.ndarray) -> dict:
    """max-abs and relative-L2 error of `out` against `ref` (fp64)."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    diff = out - ref
    nref = math.sqrt(float((ref * ref).sum()))
    return {
        "max_abs": float(np.abs(diff).max()) if diff.size else 0.0,
        "rel_l2": math.sqrt(float((diff * diff).sum())) / max(nref, 1e-300),
    }
