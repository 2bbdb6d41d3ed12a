"""Seeded random shapes for the attention kernels against the exact fp64 oracle.

Each case draws batch, GQA ratio, head dim, query and key lengths, cache capacity, bits, dtype,
causal and window masks and per-sequence lengths from a fixed seed, so a failure names a case
that reruns identically. The hand-written tests pin the edges one at a time; these cover their
combinations (partial tiles and row blocks with windows, variable lengths and capacity views
together, grids that are and are not a multiple of the XCD count), and the paged pools against
the contiguous caches.
"""

import math
import random

import pytest
import torch

from myinfer_amd import kernels
from tests import test_gpu_decode as TD
from tests import test_gpu_dense as TN
from tests import test_gpu_paged as TG
from tests import test_gpu_prefill as TP
from tests.helpers import assert_close, exact_reference, seeded_normal

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


@pytest.mark.parametrize("case", range(48))
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


@pytest.mark.parametrize("case", range(48))
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


def _group(rng, D):
    return rng.choice([g for g in (32, 64, 128) if D // 4 <= g <= D])


@pytest.mark.parametrize("case", range(32))
def test_decode_fuzz_groups_and_head_dims(case):
    # group sizes 32/64/128 and head_dim 64/128/256, with the masks, lengths and views above
    rng = random.Random(7500 + case)
    D, bits, dtype = rng.choice([64, 128, 256]), rng.choice([4, 8]), rng.choice(DTYPES)
    group = _group(rng, D)
    Hkv, rep = rng.choice([1, 2, 4]), rng.choice([1, 2, 3, 4, 8])
    B, L = rng.choice([1, 2, 3]), rng.choice([1, 1, 2, 5])
    S = rng.randrange(L, 2500)
    cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
    causal, window, seq_lens = _masks(rng, B, L, S)
    TD.run_case(B, Hkv * rep, Hkv, L, S, D, bits, dtype, causal=causal, window=window, seq_lens=seq_lens,
                seed=7500 + case, cap=cap, outliers=rng.random() < 0.3, group=group, what=f"fuzz-gd {case}")


@pytest.mark.parametrize("case", range(32))
def test_prefill_fuzz_groups_and_head_dims(case):
    rng = random.Random(7600 + case)
    D, bits, dtype = rng.choice([64, 128]), rng.choice([4, 8]), rng.choice(DTYPES)
    group = _group(rng, D)
    Hkv, rep = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 4, 8])
    B, L = rng.choice([1, 2]), rng.randrange(1, 400)
    S = rng.randrange(L, 3000)
    cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
    causal, window, seq_lens = _masks(rng, B, L, S)
    TP.run_case(B, Hkv * rep, Hkv, L, S, bits, dtype, causal=causal, window=window, seq_lens=seq_lens,
                seed=7600 + case, cap=cap, group=group, D=D, what=f"fuzz-gd {case}")


@pytest.mark.parametrize("case", range(32))
def test_head_dim_256_fuzz(case):
    # the head_dim-256 kernel: quantized prefill (groups 64/128) and unquantized decode / prefill
    rng = random.Random(7700 + case)
    dtype = rng.choice(DTYPES)
    Hkv, rep = rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 4])
    B = rng.choice([1, 2])
    if case % 2 == 0:
        bits, group = rng.choice([4, 8]), rng.choice([64, 128])
        L = rng.randrange(1, 300)
        S = rng.randrange(L, 3000)
        cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
        causal, window, seq_lens = _masks(rng, B, L, S)
        TP.run_case(B, Hkv * rep, Hkv, L, S, bits, dtype, causal=causal, window=window, seq_lens=seq_lens,
                    seed=7700 + case, cap=cap, group=group, D=256, what=f"fuzz-d256 {case}")
    else:
        kernel = rng.choice(["decode", "prefill"])
        L = rng.choice([1, 2, 4]) if kernel == "decode" else rng.randrange(1, 300)
        S = rng.randrange(L, 2500)
        cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
        causal, window, seq_lens = _masks(rng, B, L, S)
        TN.run_case(kernel, B, Hkv * rep, Hkv, L, S, 256, dtype, causal=causal, window=window, seq_lens=seq_lens,
                    seed=7700 + case, cap=cap, what=f"fuzz-d256 {case}")


@pytest.mark.parametrize("case", range(32))
def test_other_head_dims_fuzz(case):
    # head dims other than 64/128/256 (the decode kernel at the next width, any query length):
    # quantized 32/96/192 at their groups, unquantized multiples of 8 up to 248, through either
    # entry point
    rng = random.Random(7900 + case)
    dtype = rng.choice(DTYPES)
    Hkv, rep = rng.choice([1, 2, 4]), rng.choice([1, 2, 4, 8])
    B = rng.choice([1, 2, 3])
    L = rng.choice([1, 1, 3, rng.randrange(1, 200)])
    S = rng.randrange(L, 2500)
    cap = S + rng.choice([0, 0, rng.randrange(1, 300)])
    causal, window, seq_lens = _masks(rng, B, L, S)
    if case % 2 == 0:
        D, group = rng.choice([(32, 32), (96, 32), (192, 64)])
        TD.run_case(B, Hkv * rep, Hkv, L, S, D, rng.choice([4, 8]), dtype, causal=causal, window=window,
                    seq_lens=seq_lens, seed=7900 + case, cap=cap, group=group, what=f"fuzz-hd {case}")
    else:
        D = rng.choice([16, 24, 40, 48, 72, 80, 96, 112, 120, 136, 160, 192, 248])
        TN.run_case(rng.choice(["decode", "prefill"]), B, Hkv * rep, Hkv, L, S, D, dtype, causal=causal,
                    window=window, seq_lens=seq_lens, seed=7900 + case, cap=cap, what=f"fuzz-hd {case}")


@pytest.mark.parametrize("case", range(48))
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


@pytest.mark.parametrize("case", range(32))
def test_paged_fuzz(case):
    # pools in shuffled 64-row pages, unused rows poisoned with NaN scales; the paged kernels must
    # equal the contiguous ones bit for bit, and both the oracle
    rng = random.Random(7400 + case)
    kernel = rng.choice(["decode", "prefill"])
    D = 128 if kernel == "prefill" else rng.choice([64, 128])
    bits, dtype = rng.choice([4, 8]), rng.choice(DTYPES)
    Hkv, rep, B = rng.choice([1, 2, 4]), rng.choice([1, 2, 4, 8]), rng.choice([1, 2, 3])
    L = rng.choice([1, 2, 4]) if kernel == "decode" else rng.randrange(1, 300)
    lens = [rng.randrange(L, 2500) for _ in range(B)]
    causal, window = rng.random() < 0.5, rng.choice([0, 0, rng.randrange(1, max(lens) + 1)])
    print(f"paged fuzz {case}: {kernel} B={B} Hq={Hkv * rep} Hkv={Hkv} L={L} lens={lens} D={D} bits={bits} "
          f"{dtype} causal={causal} window={window}", flush=True)
    rows, tables, kp, vp, kc, vc = TG.build(B, Hkv, lens, D, bits, dtype, 7400 + case)
    q = seeded_normal((B, Hkv * rep, L, D), 7500 + case, dtype, "cuda")
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(D)
    out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, causal=causal, window=window, bits=bits,
                                    max_len=max(lens), kernel=kernel)
    out_c = kernels.attention(q, kc, vc, scale, causal=causal, window=window, seq_lens=sl, bits=bits, kernel=kernel)
    torch.cuda.synchronize()
    assert torch.isfinite(out_p.float()).all(), "a row past a sequence's end was read"
    assert torch.equal(out_p, out_c)
    assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, causal=causal, window=window, seq_lens=sl),
                 f"paged fuzz {case}")
