"""Writes the golden fixtures in this directory from the CPU oracle (never from MLX: it is not
installed here). Run from the repository root: `python tests/golden/make_golden.py`.

quantize.npz   inputs (fp16 / bf16 bit patterns) with known-answer groups (all-zero, constant,
               integer ramps) and stress rows (outliers, all-positive / all-negative groups,
               repeated values), and the expected codes / scales / biases at 8, 4 and 2 bits.
attention.npz  small quantized caches, queries and the exact fp64 outputs for decode (L = 1,
               GQA 1/4/8, ragged S, variable lengths) and prefill (L > 1, causal, window).

Every array is small (about a megabyte in all, mostly incompressible codes); the GPU tests recompute
nothing from the oracle for these cases, they compare kernel outputs with the stored ones.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import attention as OA  # noqa: E402
from oracle import quantize as OQ  # noqa: E402


def quantize_inputs(rng, dtype: str, D: int = 128) -> np.ndarray:
    rows = []
    rows.append(np.zeros(D, np.float32))
    rows.append(np.full(D, 0.5, np.float32))
    rows.append(np.full(D, -3.25, np.float32))
    ramp = np.concatenate([np.arange(64, dtype=np.float32), -np.arange(64, dtype=np.float32)])
    rows.append(ramp)
    x = rng.standard_normal((28, D)).astype(np.float32)
    x[::5] *= 8.0
    x[1::7, 3] = 40.0
    x[2::7] = np.abs(x[2::7])
    x[3::7] = -np.abs(x[3::7])
    x[4::9] = 0.75
    x[5::9, :64] = 1e-3 * x[5::9, :64]
    rows.extend(list(x))
    a = np.stack(rows).astype(np.float32)
    return OQ.to_bits(a, dtype)


def make_quantize(rng) -> dict:
    out = {}
    for dtype in ("float16", "bfloat16"):
        xb = quantize_inputs(rng, dtype)
        out[f"x_{dtype}"] = xb
        for bits in (8, 4, 2):
            for G in (64, 32):
                c, s, b = OQ.quantize(xb, dtype, G, bits)
                key = f"{dtype}_b{bits}_g{G}"
                out[f"codes_{key}"] = c
                out[f"scales_{key}"] = s
                out[f"biases_{key}"] = b
    return out


ATTN_CASES = [
    # name, B, Hq, Hkv, L, S, bits, dtype, causal, window, seq_lens
    ("dec_gqa1", 1, 2, 2, 1, 130, 8, "float16", False, 0, None),
    ("dec_gqa4", 1, 8, 2, 1, 257, 8, "float16", False, 0, None),
    ("dec_gqa8_4bit", 1, 8, 1, 1, 300, 4, "float16", False, 0, None),
    ("dec_varlen_bf16", 2, 8, 2, 1, 200, 8, "bfloat16", True, 0, [200, 33]),
    ("dec_window", 1, 4, 1, 1, 250, 8, "bfloat16", True, 64, None),
    ("pre_causal", 1, 8, 2, 24, 180, 8, "float16", True, 0, None),
    ("pre_window_bf16", 1, 4, 1, 40, 200, 8, "bfloat16", True, 50, None),
    ("pre_full_4bit", 1, 4, 2, 33, 97, 4, "float16", False, 0, None),
]


def make_attention(rng) -> dict:
    out = {}
    D = 128
    for name, B, Hq, Hkv, L, S, bits, dtype, causal, window, seq_lens in ATTN_CASES:
        k = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
        v = rng.standard_normal((B, Hkv, S, D)).astype(np.float32)
        q = rng.standard_normal((B, Hq, L, D)).astype(np.float32)
        kb, vb, qb = OQ.to_bits(k, dtype), OQ.to_bits(v, dtype), OQ.to_bits(q, dtype)
        kt = OQ.quantize(kb, dtype, 64, bits)
        vt = OQ.quantize(vb, dtype, 64, bits)
        scale = 1.0 / np.sqrt(D)
        ref = OA.exact_from_quantized(OQ.from_bits(qb, dtype).astype(np.float64), kt, vt, dtype, scale,
                                      group_size=64, bits=bits, causal=causal, window=window, seq_lens=seq_lens)
        out[f"{name}/q"] = qb
        for tag, (c, s, b) in (("k", kt), ("v", vt)):
            out[f"{name}/{tag}_codes"] = c
            out[f"{name}/{tag}_scales"] = s
            out[f"{name}/{tag}_biases"] = b
        out[f"{name}/ref"] = ref.astype(np.float32)  # fp32 is far finer than the parity tolerances
        out[f"{name}/meta"] = np.array([B, Hq, Hkv, L, S, bits, int(causal), window], np.int64)
        out[f"{name}/seq_lens"] = np.array(seq_lens if seq_lens is not None else [], np.int32)
        out[f"{name}/dtype"] = np.array(dtype)
    return out


def build() -> dict:
    rng = np.random.default_rng(20261201)
    return {"quantize": make_quantize(rng), "attention": make_attention(rng)}


def main() -> None:
    data = build()
    for name, arrays in data.items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(f"wrote {HERE / (name + '.npz')} ({len(arrays)} arrays)")


if __name__ == "__main__":
    main()
