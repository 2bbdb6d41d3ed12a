"""GPU kernels against the committed golden fixtures (tests/golden/*.npz): the quantize-append
kernel must reproduce the stored codes / scales / biases bit for bit, the attention kernels the
stored exact outputs within the parity tolerance."""

from pathlib import Path

import numpy as np
import pytest
import torch

from myinfer_amd import kernels
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"
TORCH = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits_to_tensor(a, dtype):
    return torch.from_numpy(a.astype(np.int16)).view(TORCH[dtype]).to(DEV)


def u32(a):
    return torch.from_numpy(a.view(np.int32)).to(DEV).view(torch.uint32)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("bits", [8, 4, 2])
@pytest.mark.parametrize("G", [64, 32])
def test_quantize_matches_fixtures(dtype, bits, G):
    z = load("quantize")
    x = bits_to_tensor(z[f"x_{dtype}"], dtype)
    c, s, b = kernels.quantize(x, G, bits)
    key = f"{dtype}_b{bits}_g{G}"
    assert np.array_equal(c.cpu().view(torch.int32).numpy().view(np.uint32), z[f"codes_{key}"])
    assert np.array_equal(s.cpu().view(torch.int16).numpy().view(np.uint16), z[f"scales_{key}"])
    assert np.array_equal(b.cpu().view(torch.int16).numpy().view(np.uint16), z[f"biases_{key}"])


def attention_cases():
    with np.load(GOLDEN / "attention.npz", allow_pickle=False) as z:
        return sorted({k.split("/")[0] for k in z.files})


@pytest.mark.parametrize("name", attention_cases())
def test_attention_matches_fixtures(name):
    print(f"golden attention case {name}", flush=True)
    z = load("attention")
    B, Hq, Hkv, L, S, bits, causal, window = (int(x) for x in z[f"{name}/meta"])
    dtype = str(z[f"{name}/dtype"])
    sl = z[f"{name}/seq_lens"]
    q = bits_to_tensor(z[f"{name}/q"], dtype)
    kt = (u32(z[f"{name}/k_codes"]), bits_to_tensor(z[f"{name}/k_scales"], dtype), bits_to_tensor(z[f"{name}/k_biases"], dtype))
    vt = (u32(z[f"{name}/v_codes"]), bits_to_tensor(z[f"{name}/v_scales"], dtype), bits_to_tensor(z[f"{name}/v_biases"], dtype))
    seq = torch.from_numpy(sl).to(DEV) if sl.size else None
    out = kernels.attention(q, kt, vt, 1.0 / np.sqrt(128), causal=bool(causal), window=window, seq_lens=seq, bits=bits)
    torch.cuda.synchronize()
    assert_close(out, z[f"{name}/ref"], name)
