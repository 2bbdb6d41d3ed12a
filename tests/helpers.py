"""Helpers shared by the GPU parity tests: seeded inputs, oracle comparison, tolerances."""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention as OA
from oracle import quantize as OQ

NP_DTYPE = {torch.float16: "float16", torch.bfloat16: "bfloat16"}

# Tolerances against the exact fp64 oracle.
#  fp16 outputs: the north-star bound, max-abs 2e-3 and relative L2 1e-3.
#  bf16 outputs: rounding the output alone costs up to 2^-9 |o| per element (half an ulp with
#  8 significant bits) and about 2^-9/sqrt(3) ~ 1.1e-3 in relative L2; the bound allows that
#  plus the fp16-level kernel error: max-abs <= 2^-8 * max|ref| + 1e-3, relative L2 <= 3e-3.
TOL = {
    torch.float16: lambda ref: (2e-3, 1e-3),
    torch.bfloat16: lambda ref: (2.0**-8 * float(np.abs(ref).max()) + 1e-3, 3e-3),
}


def seeded_normal(shape, seed, dtype, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype).to(device)


def to_np_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def triple_to_np(tr):
    c, s, b = tr
    return c.detach().cpu().view(torch.int32).numpy().view(np.uint32), to_np_bits(s), to_np_bits(b)


def exact_reference(q: torch.Tensor, k_tr, v_tr, scale, *, bits, group_size=64, causal=False, window=0,
                    seq_lens=None):
    dt = NP_DTYPE[q.dtype]
    qn = q.detach().cpu().float().numpy().astype(np.float64)
    kdq = OQ.dequantize(*triple_to_np(k_tr), dt, group_size, bits)
    vdq = OQ.dequantize(*triple_to_np(v_tr), dt, group_size, bits)
    sl = None if seq_lens is None else [int(x) for x in seq_lens.cpu().tolist()]
    return OA.exact_attention(qn, kdq, vdq, scale, causal=causal, window=window, seq_lens=sl)


def fp16_key_floor(q: torch.Tensor, k_tr, v_tr, scale, ref: np.ndarray, *, bits, group_size=64, causal=False,
                   window=0, seq_lens=None) -> dict:
    """Error (vs the exact fp64 answer `ref`) of exact fp64 attention whose dequantized keys were
    rounded to fp16 first: the error floor of any kernel that feeds the dequantized keys to fp16
    operands (as mlx-lm's fp16 quantized_matmul does when it dequantizes in T). It grows with the
    score magnitude: a key element k carries a rounding of up to 2^-11 |k|, so a score of size s
    moves by about 2^-11 s / sqrt(3) times a mixing factor; at N(0,1) inputs it is far below the
    north-star bar, with keys of norm 65x it is not."""
    dt = NP_DTYPE[q.dtype]
    qn = q.detach().cpu().float().numpy().astype(np.float64)
    kdq = OQ.dequantize(*triple_to_np(k_tr), dt, group_size, bits).astype(np.float16).astype(np.float64)
    vdq = OQ.dequantize(*triple_to_np(v_tr), dt, group_size, bits)
    sl = None if seq_lens is None else [int(x) for x in seq_lens.cpu().tolist()]
    floor = OA.exact_attention(qn, kdq, vdq, scale, causal=causal, window=window, seq_lens=sl)
    return OA.error_stats(floor, ref)


def assert_close(out: torch.Tensor, ref: np.ndarray, what: str = ""):
    o = out.detach().cpu().float().numpy().astype(np.float64)
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    st = OA.error_stats(o, ref)
    max_abs, rel = TOL[out.dtype](ref)
    assert st["max_abs"] <= max_abs and st["rel_l2"] <= rel, f"{what}: {st} vs bounds max_abs {max_abs}, rel_l2 {rel}"
    return st
