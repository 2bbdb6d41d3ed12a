"""Argument checks of the prefill, unquantized and paged attention entry points (include/kvq.h),
without a GPU. Every case here fails validation, so no call reaches a HIP launch: the descriptors
hold fake device addresses. Each failure returns its status code and names the offending argument
in kvq_last_error(), as the reference's callers expect an error rather than a crash
(m5engine/attention.py:29-37 takes shapes from the caller; mlx raises on a mismatch)."""

import ctypes

import pytest

from myinfer_amd import _lib
from tests.test_abi import _attn, _fake_q, _fake_rows

byref = ctypes.byref
WS = 1 << 30  # a 256-byte aligned fake address; never dereferenced


def _prefill(**kw):
    return _attn(_lib.lib().kvq_prefill_attn, **kw)


def _dense(fn, **kw):
    a = dict(q=_fake_rows(), k=_fake_rows(ptr=1 << 21), v=_fake_rows(ptr=1 << 22), seq=None, out=_fake_rows(ptr=1 << 23),
             B=1, Hq=8, Hkv=1, L=1, D=128, S=256, dtype=0, scale=0.1, causal=0, window=0, ws=None, wsb=0, stream=None)
    a.update(kw)
    return fn(byref(a["q"]), byref(a["k"]), byref(a["v"]), a["seq"], byref(a["out"]), a["B"], a["Hq"], a["Hkv"],
              a["L"], a["D"], a["S"], a["dtype"], a["scale"], a["causal"], a["window"], a["ws"], a["wsb"], a["stream"])


def _paged(fn, **kw):
    a = dict(q=_fake_rows(), k=_fake_q(), v=_fake_q(ptr=1 << 24), pages=16, table=1 << 25, table_stride=4, seq=None,
             out=_fake_rows(ptr=1 << 23), B=1, Hq=8, Hkv=1, L=1, D=128, S=256, bits=8, group=64, dtype=0, scale=0.1,
             causal=0, window=0, ws=None, wsb=0, stream=None)
    a.update(kw)
    return fn(byref(a["q"]), byref(a["k"]), byref(a["v"]), a["pages"], a["table"], a["table_stride"], a["seq"],
              byref(a["out"]), a["B"], a["Hq"], a["Hkv"], a["L"], a["D"], a["S"], a["bits"], a["group"], a["dtype"],
              a["scale"], a["causal"], a["window"], a["ws"], a["wsb"], a["stream"])


def _expect(rc, code, needle):
    assert rc == code, (rc, _lib.last_error())
    assert needle in _lib.last_error()


def test_prefill_workspace_size():
    lib = _lib.lib()
    c3 = lib.kvq_prefill_workspace_size(1, 32, 4, 512, 128, 16384, 0)
    assert c3 >= 256 and c3 % 256 == 0
    # a split takes at least about 4 key tiles of 64: two tiles need no split, only the shared
    # counter block
    assert lib.kvq_prefill_workspace_size(1, 32, 4, 128, 128, 128, 0) == 256
    assert lib.kvq_prefill_workspace_size(1, 32, 4, 512, 128, 512, 0) > 256
    # head dims other than 64/128/256 run the decode kernel: its workspace
    assert lib.kvq_prefill_workspace_size(1, 32, 4, 512, 96, 16384, 0) == lib.kvq_decode_workspace_size(1, 32, 4, 512, 96,
                                                                                                      16384, 0) > 0
    assert lib.kvq_prefill_workspace_size(1, 32, 4, 512, 100, 16384, 0) == 0
    assert 0 < lib.kvq_prefill_workspace_size(1, 32, 4, 512, 64, 16384, 0) < c3  # half the dims per partial row
    assert lib.kvq_prefill_workspace_size(1, 30, 4, 512, 128, 16384, 0) == 0  # Hq not a multiple of Hkv
    assert lib.kvq_prefill_workspace_size(1, 32, 4, 0, 128, 16384, 0) == 0
    assert lib.kvq_prefill_workspace_size(1, 32, 4, 512, 128, 16384, -1) == 0


@pytest.mark.parametrize("kw,code,needle", [
    (dict(D=512), _lib.ERR_UNSUPPORTED, "head_dim 64, 128, 256"),
    (dict(D=96), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(D=256, group=32), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(D=64, group=128), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(bits=3), _lib.ERR_UNSUPPORTED, "bits"),
    (dict(group=16), _lib.ERR_UNSUPPORTED, "group_size"),
    (dict(Hq=6, Hkv=4), _lib.ERR_INVALID, "multiple"),
    (dict(L=0), _lib.ERR_INVALID, "positive"),
    (dict(dtype=2), _lib.ERR_INVALID, "dtype"),
    (dict(scale=float("inf")), _lib.ERR_INVALID, "scale"),
    (dict(window=-2), _lib.ERR_INVALID, "window"),
    (dict(), _lib.ERR_WORKSPACE, "workspace"),
])
def test_prefill_rejects_bad_arguments(kw, code, needle):
    _expect(_prefill(**kw), code, needle)


def test_prefill_rejects_bad_layouts():
    n = _lib.lib().kvq_prefill_workspace_size(1, 8, 1, 1, 128, 256, 0)
    # the output rows are written 8 bytes at a time: 16-byte alignment, as for the queries
    _expect(_prefill(out=_fake_rows(ptr=(1 << 23) + 8), ws=WS, wsb=n), _lib.ERR_INVALID, "out")
    k = _fake_q()
    k.codes_stride_s = 16  # fewer words than one 8-bit row of D = 128
    _expect(_prefill(k=k, ws=WS, wsb=n), _lib.ERR_INVALID, "row stride")
    v = _fake_q()
    v.sb_stride_s = 1
    _expect(_prefill(v=v, ws=WS, wsb=n), _lib.ERR_INVALID, "scales row stride")
    # 32-bit buffer offsets: S rows of a 8 KiB stride do not fit
    k = _fake_q()
    k.codes_stride_s = 2048
    big = 1 << 20
    nb = _lib.lib().kvq_prefill_workspace_size(1, 8, 1, 1, 128, big, 0)
    _expect(_prefill(k=k, S=big, ws=WS, wsb=nb), _lib.ERR_UNSUPPORTED, "4 GiB")
    _expect(_prefill(ws=WS + 128, wsb=n), _lib.ERR_WORKSPACE, "aligned")


@pytest.mark.parametrize("entry", ["kvq_decode_attn_dense", "kvq_prefill_attn_dense"])
def test_dense_entry_points_reject_bad_arguments(entry):
    fn = getattr(_lib.lib(), entry)
    _expect(_dense(fn, D=264), _lib.ERR_UNSUPPORTED, "multiples of 8 up to 256")
    _expect(_dense(fn, D=100), _lib.ERR_UNSUPPORTED, "multiples of 8")
    _expect(_dense(fn, dtype=3), _lib.ERR_INVALID, "dtype")
    _expect(_dense(fn, Hq=5, Hkv=2), _lib.ERR_INVALID, "multiple")
    _expect(_dense(fn, k=_lib.Rows(1 << 21, 8 * 128, 4 * 128, 120)), _lib.ERR_INVALID, "row stride")
    _expect(_dense(fn, v=_lib.Rows((1 << 22) + 4, 8 * 128, 4 * 128, 128)), _lib.ERR_INVALID, "values")
    _expect(_dense(fn, k=_lib.Rows(0, 8 * 128, 4 * 128, 128)), _lib.ERR_INVALID, "keys")
    big = 1 << 22
    _expect(_dense(fn, k=_lib.Rows(1 << 21, 0, 0, 1024), S=big), _lib.ERR_UNSUPPORTED, "4 GiB")
    _expect(_dense(fn), _lib.ERR_WORKSPACE, "workspace")


@pytest.mark.parametrize("entry", ["kvq_paged_decode_attn", "kvq_paged_prefill_attn"])
def test_paged_entry_points_reject_bad_arguments(entry):
    lib = _lib.lib()
    fn = getattr(lib, entry)
    _expect(_paged(fn, D=96), _lib.ERR_UNSUPPORTED, "group_size")
    _expect(_paged(fn, D=100), _lib.ERR_UNSUPPORTED, "head_dim")
    _expect(_paged(fn, bits=2), _lib.ERR_UNSUPPORTED, "bits")
    _expect(_paged(fn, pages=0), _lib.ERR_INVALID, "num_pages")
    _expect(_paged(fn, table=None), _lib.ERR_INVALID, "block_table")
    _expect(_paged(fn, table_stride=0), _lib.ERR_INVALID, "table_stride")
    # S = 256 rows need 4 pages of 64 rows per sequence
    _expect(_paged(fn, table_stride=3), _lib.ERR_INVALID, "cannot hold")
    k = _fake_q()
    k.codes_stride_h = 100  # pages of 64 rows of 32 words cannot be 100 words apart
    _expect(_paged(fn, k=k), _lib.ERR_INVALID, "overlap")
    v = _fake_q(ptr=1 << 24)
    v.sb_stride_b = 8  # the page stride is smaller than the heads it holds
    _expect(_paged(fn, v=v, Hkv=2, Hq=8), _lib.ERR_INVALID, "overlap")
    v = _fake_q(ptr=(1 << 24) + 8)
    _expect(_paged(fn, v=v), _lib.ERR_INVALID, "16-byte")
    _expect(_paged(fn), _lib.ERR_WORKSPACE, "workspace")


def test_paged_append_rejects_bad_arguments():
    lib = _lib.lib()
    r = _fake_rows()
    q = _fake_q()

    def call(**kw):
        a = dict(pages=16, table=1 << 25, table_stride=4, starts=None, row_offset=0, B=1, H=1, L=1, D=128, bits=8)
        a.update(kw)
        return lib.kvq_paged_quantize_append(byref(r), byref(q), None, None, a["pages"], a["table"], a["table_stride"],
                                             a["starts"], a["row_offset"], None, a["B"], a["H"], a["L"], a["D"],
                                             a["bits"], 64, 0, None)

    _expect(call(pages=0), _lib.ERR_INVALID, "num_pages")
    _expect(call(table=None), _lib.ERR_INVALID, "block_table")
    # rows 255 .. 256 need 5 pages in the table
    _expect(call(row_offset=255, L=2), _lib.ERR_INVALID, "cannot hold")
    _expect(call(bits=3), _lib.ERR_UNSUPPORTED, "bits")
    _expect(call(row_offset=-1), _lib.ERR_INVALID, "row_offset")


@pytest.mark.parametrize("field,value", [("sb_stride_s", 3), ("sb_stride_h", 8 * 256 + 1), ("scales", (1 << 16) + 2)])
def test_prefill_rejects_unaligned_scale_rows(field, value):
    # with two or more scale groups per row the prefill kernel loads a row's groups in pairs
    # (4 bytes): scale and bias rows must be 4-byte aligned
    n = _lib.lib().kvq_prefill_workspace_size(1, 8, 1, 1, 128, 256, 0)
    k = _fake_q()
    setattr(k, field, value)
    _expect(_prefill(k=k, ws=WS, wsb=n), _lib.ERR_INVALID, "4-byte aligned")
    _expect(_paged(_lib.lib().kvq_paged_prefill_attn, k=k, ws=WS, wsb=n), _lib.ERR_INVALID, "4-byte aligned")


def test_unquantized_head_dims():
    # the unquantized kernels take head_dim 64/128/256 (decode and prefill)
    lib = _lib.lib()
    _expect(_dense(lib.kvq_prefill_attn_dense, D=512), _lib.ERR_UNSUPPORTED, "head_dim 64, 128, 256")
    _expect(_dense(lib.kvq_decode_attn_dense, D=512), _lib.ERR_UNSUPPORTED, "head_dim 64, 128, 256")
    # head_dim 256 needs a workspace from both size queries
    assert lib.kvq_prefill_workspace_size(1, 8, 4, 512, 256, 4096, 0) >= 256
    assert lib.kvq_decode_workspace_size(1, 8, 4, 1, 256, 4096, 0) >= lib.kvq_prefill_workspace_size(1, 8, 4, 1, 256,
                                                                                                    4096, 0)


def _rows96(ptr, D=96):
    return _lib.Rows(ptr, 8 * D, 4 * D, D)


def _q96(ptr=1 << 20, D=96, bits=8, G=32):
    w, ng = D * bits // 32, D // G
    return _lib.QTensor(ptr, ptr + (1 << 16), ptr + (1 << 17), 8 * 256 * w, 256 * w, w, 8 * 256 * ng, 256 * ng, ng)


@pytest.mark.parametrize("entry", ["kvq_decode_attn", "kvq_prefill_attn", "kvq_decode_attn_static"])
def test_narrow_head_dims_need_tight_scale_rows(entry):
    """A head dimension below its kernel's width (96 -> 128) reads the next row's first scale groups
    past its own, so scale/bias rows must hold exactly D/G elements; a well-formed call reaches the
    workspace check (no device memory is touched)."""
    lib = _lib.lib()
    fn = getattr(lib, entry)
    common = dict(q=_rows96(16 * 1024), out=_rows96(1 << 23), D=96, group=32)
    static = entry.endswith("static")

    def call(**kw):
        a = dict(common, **kw)
        if static:
            return fn(byref(a["q"]), byref(a["k"]), byref(a["v"]), None, byref(a["out"]), 1, 8, 1, 1, 96, 256, 8, 32,
                      0, 0.1, 0, 0, None)
        return _attn(fn, **a)

    k = _q96()
    k.sb_stride_s = 4  # a padded scale row
    _expect(call(k=k, v=_q96(1 << 24)), _lib.ERR_UNSUPPORTED, "exactly D/group=3")
    if not static:
        _expect(call(k=_q96(), v=_q96(1 << 24)), _lib.ERR_WORKSPACE, "workspace")


def test_narrow_unquantized_head_dims_need_tight_key_rows():
    lib = _lib.lib()
    for fn in (lib.kvq_decode_attn_dense, lib.kvq_prefill_attn_dense):
        q, out = _rows96(16 * 1024, 80), _rows96(1 << 23, 80)
        padded = _lib.Rows(1 << 21, 8 * 88 * 256, 88 * 256, 88)
        _expect(_dense(fn, q=q, out=out, D=80, k=padded, v=_rows96(1 << 22, 80)), _lib.ERR_UNSUPPORTED,
                "key rows of exactly D")
        _expect(_dense(fn, q=q, out=out, D=80, k=_rows96(1 << 21, 80), v=_rows96(1 << 22, 80)), _lib.ERR_WORKSPACE,
                "workspace")
