"""The C ABI (include/kvq.h) without a GPU: the library loads, exports every declared entry point,
reports its ABI version, and rejects bad arguments with a status code and a message before any
HIP call is made."""

import ctypes
import re
from pathlib import Path

import pytest

from myinfer_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvq.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvq_[a-z_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert "kvq_decode_attn" in names and "kvq_quantize_append" in names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in kvq.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"


def test_abi_version():
    assert _lib.lib().kvq_abi_version() == _lib.ABI_VERSION
    text = HEADER.read_text()
    assert f"#define KVQ_ABI_VERSION {_lib.ABI_VERSION}" in text


def _fake_rows(ptr=16 * 1024, D=128):
    return _lib.Rows(ptr, 8 * D, 4 * D, D)


def _fake_q(ptr=1 << 20, D=128, bits=8):
    w = D * bits // 32
    return _lib.QTensor(ptr, ptr + (1 << 16), ptr + (1 << 17), 8 * 256 * w, 256 * w, w, 8 * 512, 512, 2)


def _attn(fn, **kw):
    args = dict(q=_fake_rows(), k=_fake_q(), v=_fake_q(), seq=None, out=_fake_rows(), B=1, Hq=8, Hkv=1, L=1, D=128,
                S=256, bits=8, group=64, dtype=0, scale=0.1, causal=0, window=0, ws=None, wsb=0, stream=None)
    args.update(kw)
    byref = ctypes.byref
    return fn(byref(args["q"]), byref(args["k"]), byref(args["v"]), args["seq"], byref(args["out"]), args["B"],
              args["Hq"], args["Hkv"], args["L"], args["D"], args["S"], args["bits"], args["group"], args["dtype"],
              args["scale"], args["causal"], args["window"], args["ws"], args["wsb"], args["stream"])


@pytest.mark.parametrize("kw,code,needle", [
    (dict(bits=3), _lib.ERR_UNSUPPORTED, "bits"),
    (dict(group=48), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(group=128, D=64, S=256), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(D=96), _lib.ERR_UNSUPPORTED, "dividing head_dim"),  # groups of 64 do not divide 96
    (dict(D=160, group=32), _lib.ERR_UNSUPPORTED, "group_size"),  # runs at width 256: groups of 64 or 128
    (dict(D=100), _lib.ERR_UNSUPPORTED, "multiples of 8"),
    (dict(D=512), _lib.ERR_UNSUPPORTED, "head_dim"),
    (dict(group=32, D=256, S=256), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(Hq=7, Hkv=2), _lib.ERR_INVALID, "multiple"),
    (dict(dtype=5), _lib.ERR_INVALID, "dtype"),
    (dict(S=0), _lib.ERR_INVALID, "positive"),
    (dict(window=-1), _lib.ERR_INVALID, "window"),
    (dict(scale=float("nan")), _lib.ERR_INVALID, "scale"),
    (dict(), _lib.ERR_WORKSPACE, "workspace"),
])
def test_decode_rejects_bad_arguments(kw, code, needle):
    lib = _lib.lib()
    rc = _attn(lib.kvq_decode_attn, **kw)
    assert rc == code
    assert needle in _lib.last_error()
    with pytest.raises((ValueError, NotImplementedError, RuntimeError)):
        _lib.check(rc, "decode")


def test_decode_rejects_misaligned_pointers():
    lib = _lib.lib()
    ws = 1 << 30
    n = lib.kvq_decode_workspace_size(1, 8, 1, 1, 128, 256, 0)
    assert n > 0
    rc = _attn(lib.kvq_decode_attn, q=_fake_rows(ptr=16 * 1024 + 2), ws=ws, wsb=n)
    assert rc == _lib.ERR_INVALID and "16-byte" in _lib.last_error()
    k = _fake_q()
    k.codes += 4
    rc = _attn(lib.kvq_decode_attn, k=k, ws=ws, wsb=n)
    assert rc == _lib.ERR_INVALID and "codes" in _lib.last_error()
    rc = _attn(lib.kvq_decode_attn, ws=ws + 64, wsb=n)
    assert rc == _lib.ERR_WORKSPACE and "aligned" in _lib.last_error()
    rc = _attn(lib.kvq_decode_attn, ws=ws, wsb=n - 1)
    assert rc == _lib.ERR_WORKSPACE


def test_quantize_append_rejects_bad_arguments():
    lib = _lib.lib()
    r = _fake_rows()
    q = _fake_q()
    byref = ctypes.byref
    assert lib.kvq_quantize_append(byref(r), byref(q), None, None, 0, 1, 1, 1, 128, 3, 64, 0, None) == _lib.ERR_UNSUPPORTED
    assert lib.kvq_quantize_append(byref(r), byref(q), None, None, 0, 1, 1, 1, 128, 8, 48, 0, None) == _lib.ERR_UNSUPPORTED
    assert lib.kvq_quantize_append(byref(r), byref(q), None, None, 0, 1, 1, 1, 96, 8, 64, 0, None) == _lib.ERR_INVALID
    assert "multiple" in _lib.last_error()
    assert lib.kvq_quantize_append(byref(r), byref(q), byref(r), None, 0, 1, 1, 1, 128, 8, 64, 0, None) == _lib.ERR_INVALID
    assert lib.kvq_quantize_append(byref(r), byref(q), None, None, -1, 1, 1, 1, 128, 8, 64, 0, None) == _lib.ERR_INVALID
    assert lib.kvq_quantize_append(None, byref(q), None, None, 0, 1, 1, 1, 128, 8, 64, 0, None) == _lib.ERR_INVALID
    # zero rows is a successful no-op that never touches the device
    assert lib.kvq_quantize_append(byref(r), byref(q), None, None, 0, 1, 1, 0, 128, 8, 64, 0, None) == _lib.OK
    assert _lib.last_error() == ""


def test_workspace_sizes():
    lib = _lib.lib()
    a = lib.kvq_decode_workspace_size(1, 64, 8, 1, 128, 32768, 0)
    b = lib.kvq_decode_workspace_size(8, 64, 8, 1, 128, 32768, 0)
    # the split count targets a fixed number of workgroups, so the partials do not shrink with B
    assert 0 < a <= b
    # head dims other than 64/128/256 run at the next width: the same partials as that width
    assert lib.kvq_decode_workspace_size(1, 64, 8, 1, 96, 32768, 0) == a
    assert lib.kvq_decode_workspace_size(1, 64, 8, 1, 100, 32768, 0) == 0
    assert lib.kvq_decode_workspace_size(1, 64, 8, 1, 264, 32768, 0) == 0
    assert lib.kvq_decode_workspace_size(1, 64, 8, 1, 256, 32768, 0) > 0  # head_dim 256 (quantized caches)
    # a sliding window never needs more splits than the full context
    assert 0 < lib.kvq_decode_workspace_size(4, 32, 16, 1, 128, 8192, 1024) <= lib.kvq_decode_workspace_size(4, 32, 16, 1, 128, 8192, 0)


def test_rope_entry_points_reject_bad_arguments():
    lib = _lib.lib()
    r = _fake_rows()
    q = _fake_q()
    byref = ctypes.byref

    def rp(**kw):
        a = dict(dims=128, traditional=0, base=10000.0, scale=1.0, offset=0)
        a.update(kw)
        return _lib.RopeParams(a["dims"], a["traditional"], a["base"], a["scale"], a["offset"])

    for bad, code, needle in [
        (rp(dims=24), _lib.ERR_UNSUPPORTED, "dims"),
        (rp(dims=256), _lib.ERR_UNSUPPORTED, "dims"),  # more than D = 128
        (rp(dims=0), _lib.ERR_UNSUPPORTED, "dims"),
        (rp(base=0.0), _lib.ERR_INVALID, "base"),
        (rp(base=float("inf")), _lib.ERR_INVALID, "base"),
        (rp(scale=float("nan")), _lib.ERR_INVALID, "scale"),
        (rp(offset=-1), _lib.ERR_INVALID, "offset"),
    ]:
        assert lib.kvq_rope(byref(r), byref(bad), 1, 1, 1, 128, 0, None) == code
        assert needle in _lib.last_error()
        assert lib.kvq_rope_quantize_append(byref(r), byref(q), None, None, byref(bad), 0, 1, 1, 1, 128, 8, 64, 0,
                                            None) == code
        assert needle in _lib.last_error()
    good = rp(dims=64, traditional=1, offset=5)
    assert lib.kvq_rope(byref(r), None, 1, 1, 1, 128, 0, None) == _lib.ERR_INVALID
    assert lib.kvq_rope(byref(r), byref(good), 1, 1, 1, 128, 7, None) == _lib.ERR_INVALID
    assert lib.kvq_rope(_lib.Rows(16 * 1024 + 2, 1024, 512, 128), byref(good), 1, 1, 1, 128, 0, None) == _lib.ERR_INVALID
    assert lib.kvq_rope_quantize_append(byref(r), byref(q), None, None, byref(good), 0, 1, 1, 1, 128, 3, 64, 0,
                                        None) == _lib.ERR_UNSUPPORTED
    # zero rows are a successful no-op that never touches the device
    assert lib.kvq_rope(byref(r), byref(good), 1, 1, 0, 128, 0, None) == _lib.OK
    assert lib.kvq_rope_quantize_append(byref(r), byref(q), None, None, byref(good), 0, 1, 1, 0, 128, 8, 64, 0,
                                        None) == _lib.OK
    assert _lib.last_error() == ""
