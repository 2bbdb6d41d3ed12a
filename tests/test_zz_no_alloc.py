"""kvq_decode_attn_static: the decode entry point that allocates nothing (its scratch is a static
device array in the library). Called through the C ABI and compared with kvq_decode_attn, whose
kernels it shares: the outputs must be bit-identical, over consecutive calls of different plans
(an in-kernel split merge that uses the arrival counters, then a smaller call merged by the
combine launch, then the first plan again, so the counters must have been left at zero)."""

import ctypes
import math

import pytest
import torch

from myinfer_amd import _lib, kernels
from tests.helpers import assert_close, exact_reference, seeded_normal


def _static_call(q, kt, vt, out, scale, *, bits=8, group=64, causal=False, window=0, seq_lens=None):
    lib = _lib.lib()
    B, Hq, L, D = q.shape
    Hkv, S = kt[0].shape[1], kt[0].shape[2]
    qr, orr = _lib.rows(q), _lib.rows(out)
    kq, vq = _lib.qtensor(*kt), _lib.qtensor(*vt)
    sl = None if seq_lens is None else seq_lens.data_ptr()
    return lib.kvq_decode_attn_static(ctypes.byref(qr), ctypes.byref(kq), ctypes.byref(vq), sl, ctypes.byref(orr), B, Hq,
                                      Hkv, L, D, S, bits, group, _lib.dtype_code(q.dtype), float(scale), int(causal),
                                      int(window), _lib.stream_ptr(q.device))


def test_static_rejects_plans_beyond_its_scratch():
    # checked on the host before any HIP call: a batch whose partials exceed the static scratch
    lib = _lib.lib()
    B, Hq, Hkv, L, D, S = 512, 64, 8, 1, 128, 4096
    need = lib.kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, 0)
    assert need > 8 << 20
    w = D * 8 // 32
    rows = _lib.Rows(1 << 20, Hq * L * D, L * D, D)
    qt = _lib.QTensor(1 << 30, 1 << 31, (1 << 31) + (1 << 28), Hkv * S * w, S * w, w, Hkv * S * 2, S * 2, 2)
    rc = lib.kvq_decode_attn_static(ctypes.byref(rows), ctypes.byref(qt), ctypes.byref(qt), None, ctypes.byref(rows), B,
                                    Hq, Hkv, L, D, S, 8, 64, 0, 0.1, 0, 0, None)
    assert rc == _lib.ERR_WORKSPACE and "static scratch" in _lib.last_error()
    rc = lib.kvq_decode_attn_static(ctypes.byref(rows), ctypes.byref(qt), ctypes.byref(qt), None, ctypes.byref(rows), 1,
                                    Hq, Hkv, L, D, S, 3, 64, 0, 0.1, 0, 0, None)
    assert rc == _lib.ERR_UNSUPPORTED


def _cache(B, Hkv, S, D, bits, dtype, seed, group=64):
    from tests.test_gpu_decode import make_cache

    return make_cache(B, Hkv, S, D, bits, dtype, seed, group=group)


@pytest.mark.gpu
def test_static_matches_workspace_entry_point():
    dev = "cuda"
    cases = [
        # (B, Hq, Hkv, S, D, group, bits, dtype, seq_lens): fused merge (4 splits, arrival counters) ...
        (8, 64, 8, 4096, 128, 64, 8, torch.float16, [4096, 3000, 4096, 17, 2500, 4096, 1, 4000]),
        # ... then a smaller call merged by the combine launch (many splits) ...
        (1, 16, 8, 2000, 128, 64, 4, torch.bfloat16, None),
        # ... then the fused plan again: the counters must have been left at zero
        (8, 64, 8, 4096, 128, 64, 8, torch.float16, None),
        # head_dim 256 (Gemma-2 / Gemma-3 heads) at groups 64 and 128: the scratch holds the
        # quantized plan the call runs
        (1, 16, 8, 4096, 256, 64, 8, torch.bfloat16, None),
        (2, 16, 8, 1024, 256, 128, 4, torch.float16, [1024, 700]),
    ]
    for i, (B, Hq, Hkv, S, D, G, bits, dtype, sl) in enumerate(cases):
        print(f"no-alloc case {i}: B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} G={G} bits={bits} {dtype} "
              f"varlen={sl is not None}", flush=True)
        kt, vt = _cache(B, Hkv, S, D, bits, dtype, 700 + i, group=G)
        q = seeded_normal((B, Hq, 1, D), 710 + i, dtype, dev)
        seq = None if sl is None else torch.tensor(sl, dtype=torch.int32, device=dev)
        scale = 1.0 / math.sqrt(D)
        ref_out = kernels.attention(q, kt, vt, scale, seq_lens=seq, bits=bits, group_size=G, kernel="decode")
        out = torch.full_like(ref_out, float("nan"))
        rc = _static_call(q, kt, vt, out, scale, bits=bits, group=G, seq_lens=seq)
        _lib.check(rc, "kvq_decode_attn_static")
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"case {i}: the static-scratch call differs from kvq_decode_attn"
        assert_close(out, exact_reference(q, kt, vt, scale, bits=bits, group_size=G, seq_lens=seq),
                     f"no-alloc case {i}")
