"""Seeded random shapes for the attention kernels against the exact fp64 oracle.

Each case draws batch, GQA ratio, head dim, query and key lengths, cache capacity, bits, dtype,
causal and window masks and per-sequence lengths from a fixed seed, so a failure names a case
that reruns identically. The hand-written tests pin the edges one at a time; these cover their
combinations (partial tiles and row blocks with windows, variable lengths and capacity views
together, grids that are and are not a multiple of the XCD count).
"""

import random

import pytest
import torch

from tests import test_gpu_decode as TD
from tests import test_gpu_dense as TN
from tests import test_gpu_prefill as TP

pytestmark = pytest.mark.gpu
DTYPES = (torch.float16, torch.bfloat16)


def _masks(rng, B, L, S):
    causal = rng.random() < 0.5
    window = rng.choice([0, 0, rng.randrange(1, S + 1)])
    seq_lens = None
    if B > 1 and rng.random() < 0.5:
        seq_lens = [S] + [rng.randrange(L, S + 1) for _ in range(B - 1)]
        rng.shuffle(seq_lens)
    return causal, window, seq_lens


@pytest.mark.parametrize("case", range(24))
def test_decode_fuzz(case):
    rng = random.Random(7100 + case)
    D, bits, dtype = rng.choice([64, 128]), rng.choice([4, 8]), rng.choice(DTYPES)
    Hkv, rep = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 3, 4, 8])
    B, L = rng.choice([1, 2, 3]), rng.choice([1, 1, 2, 4])
    S = rng.randrange(L, 2500)
    cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
    causal, window, seq_lens = _masks(rng, B, L, S)
    TD.run_case(B, Hkv * rep, Hkv, L, S, D, bits, dtype, causal=causal, window=window, seq_lens=seq_lens,
                seed=7100 + case, cap=cap, outliers=rng.random() < 0.3, what=f"fuzz {case}")


@pytest.mark.parametrize("case", range(24))
def test_prefill_fuzz(case):
    rng = random.Random(7200 + case)
    bits, dtype = rng.choice([4, 8]), rng.choice(DTYPES)
    Hkv, rep = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 4, 8])
    B, L = rng.choice([1, 2]), rng.randrange(1, 400)
    S = rng.randrange(L, 3000)
    cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
    causal, window, seq_lens = _masks(rng, B, L, S)
    TP.run_case(B, Hkv * rep, Hkv, L, S, bits, dtype, causal=causal, window=window, seq_lens=seq_lens,
                seed=7200 + case, cap=cap, what=f"fuzz {case}")


@pytest.mark.parametrize("case", range(24))
def test_unquantized_fuzz(case):
    rng = random.Random(7300 + case)
    kernel = rng.choice(["decode", "prefill"])
    D = 128 if kernel == "prefill" else rng.choice([64, 128])
    dtype = rng.choice(DTYPES)
    Hkv, rep = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 4, 8])
    B = rng.choice([1, 2])
    L = rng.choice([1, 2, 4]) if kernel == "decode" else rng.randrange(1, 300)
    S = rng.randrange(L, 2500)
    cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
    causal, window, seq_lens = _masks(rng, B, L, S)
    TN.run_case(kernel, B, Hkv * rep, Hkv, L, S, D, dtype, causal=causal, window=window, seq_lens=seq_lens,
                seed=7300 + case, cap=cap, what=f"fuzz {case}")
