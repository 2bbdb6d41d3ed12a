"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py) are
re-derived from the CPU oracle: quantized codes / scales / biases bit for bit, exact attention to
the fp32 rounding it is stored with. A change to the oracle that moves any fixture fails here."""

from pathlib import Path

import numpy as np
import pytest

from oracle import attention as OA
from oracle import quantize as OQ

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("G", [64, 32])
def test_quantize_fixtures(dtype, bits, G):
    z = load("quantize")
    c, s, b = OQ.quantize(z[f"x_{dtype}"], dtype, G, bits)
    key = f"{dtype}_b{bits}_g{G}"
    assert np.array_equal(c, z[f"codes_{key}"])
    assert np.array_equal(s, z[f"scales_{key}"])
    assert np.array_equal(b, z[f"biases_{key}"])


def test_quantize_fixture_known_answers():
    # rows 0..3 of the fixture input are the hand-derived groups of the oracle's own tests
    z = load("quantize")
    codes = OQ.unpack(z["codes_float16_b8_g64"], 8)
    assert (codes[0] == 0).all() and (codes[1] == 0).all() and (codes[2] == 0).all()
    assert int(z["scales_float16_b8_g64"][0, 0]) == 0x8002  # s = -1e-7 rounded to fp16
    j = np.arange(64)
    assert np.array_equal(codes[3, :64], np.round((63 - j) * 85 / 21).astype(np.uint32))
    assert np.array_equal(codes[3, 64:], np.round((63 - j) * 85 / 21).astype(np.uint32))


def attention_cases():
    z = load("attention")
    return sorted({k.split("/")[0] for k in z})


@pytest.mark.parametrize("name", attention_cases())
def test_attention_fixtures(name):
    z = load("attention")
    B, Hq, Hkv, L, S, bits, causal, window = (int(x) for x in z[f"{name}/meta"])
    dtype = str(z[f"{name}/dtype"])
    sl = z[f"{name}/seq_lens"].tolist() or None
    q = OQ.from_bits(z[f"{name}/q"], dtype).astype(np.float64)
    kt = tuple(z[f"{name}/k_{t}"] for t in ("codes", "scales", "biases"))
    vt = tuple(z[f"{name}/v_{t}"] for t in ("codes", "scales", "biases"))
    ref = OA.exact_from_quantized(q, kt, vt, dtype, 1.0 / np.sqrt(128), group_size=64, bits=bits,
                                  causal=bool(causal), window=window, seq_lens=sl)
    assert ref.shape == (B, Hq, L, 128)
    # stored as fp32: equal to the fp64 oracle up to that rounding
    np.testing.assert_allclose(ref, z[f"{name}/ref"].astype(np.float64), rtol=0, atol=1e-6)
