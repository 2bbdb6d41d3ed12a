"""Typed wrappers around libkvq.so's entry points (torch tensors in, torch tensors out).

Every wrapper validates shapes on the host, passes raw pointers and strides through the C ABI
and launches on the tensors' current HIP stream. Scratch memory (the attention workspace) is a
zero-filled torch allocation cached per (device, stream); the library itself allocates nothing.
"""

from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

Triple = Tuple[torch.Tensor, torch.Tensor, torch.Tensor]

_workspaces: dict = {}


def new_workspace(nbytes: int, device) -> torch.Tensor:
    """A zero-filled attention workspace. The kernels keep their split counters in it and leave
    them at zero after every call, so a workspace is zeroed once, when it is allocated."""
    return torch.zeros(max(int(nbytes), 1 << 20), dtype=torch.uint8, device=device)


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index, stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = new_workspace(nbytes, device)
        _workspaces[key] = buf
    return buf


def _require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"libkvq operates on GPU tensors; got a tensor on {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}; got {t.device}")
    return dev


def _check_triple(tr: Sequence[torch.Tensor], name: str) -> None:
    if len(tr) != 3:
        raise ValueError(f"{name} must be a (codes, scales, biases) triple")


# ---- range exponents (include/kvq.h, kvq_qtensor.range_exp)
#
# A quantized cache keeps one int32 in device memory, its range exponent E: the appends raise it to
# the smallest E >= 0 with every dequantized value within 2^15 * 2^E, and the quantized prefill
# kernels stage their fp16 operands times 2^-E, so a bf16 cache whose values leave the fp16 range
# still gives finite results. The word belongs to the cache's buffers: it is registered here under
# the storage of the codes buffer, and every call that is handed a view of those buffers (the
# reference-style entry points pass only the (codes, scales, biases) views) finds it again.

_range_words: dict = {}  # codes storage address -> (weak reference to the codes buffer, int32 word)


def register_range_word(codes: torch.Tensor, word: torch.Tensor) -> None:
    """Attach a cache's range word (a one-element int32 tensor on the codes' device) to the codes
    buffer: appends into views of it raise the word, attention over views of it reads it."""
    if word.dtype != torch.int32 or word.numel() != 1 or word.device != codes.device:
        raise ValueError("a range word is a one-element int32 tensor on the cache's device")
    key = codes.untyped_storage().data_ptr()
    if len(_range_words) > 4096:  # drop entries whose buffers are gone
        for k in [k for k, (ref, _) in _range_words.items() if ref() is None]:
            del _range_words[k]
    _range_words[key] = (weakref.ref(codes), word)


def range_word(codes: torch.Tensor) -> Optional[torch.Tensor]:
    """The range word registered for the buffer `codes` is a view of, or None."""
    hit = _range_words.get(codes.untyped_storage().data_ptr())
    if hit is None:
        return None
    buf = hit[0]()
    if buf is None or buf.untyped_storage().data_ptr() != codes.untyped_storage().data_ptr():
        return None
    return hit[1]


def range_exponent(triple: Triple, bits: int) -> torch.Tensor:
    """The range exponent of a (codes, scales, biases) triple computed from its scales and biases on
    its device (no host synchronization): the smallest E >= 0 with max(|b|, |b + (2^bits - 1) s|)
    <= 2^15 * 2^E over every group, as a one-element int32 tensor. For triples that carry no
    registered word."""
    _, scales, biases = triple
    s, b = scales.float(), biases.float()
    if s.numel() == 0:
        return torch.zeros(1, dtype=torch.int32, device=scales.device)
    top = b + float((1 << bits) - 1) * s
    bound = torch.nan_to_num(torch.maximum(b.abs(), top.abs()), nan=0.0, posinf=float("inf")).amax()
    e = torch.ceil(torch.log2(bound * (1.0 / 32768.0)))
    e = torch.nan_to_num(e, nan=127.0, posinf=127.0, neginf=0.0).clamp(0.0, 127.0)
    return e.to(torch.int32).reshape(1)


@dataclass(frozen=True)
class Rope:
    """Rotary position embedding as mlx's nn.RoPE(dims, traditional, base, scale) applies it: row l
    of a call at position offset + l, pair i turned by (position * scale) * base^(-2i/dims)."""

    dims: int
    traditional: bool = False
    base: float = 10000.0
    scale: float = 1.0

    def params(self, offset: int) -> "_lib.RopeParams":
        return _lib.RopeParams(int(self.dims), int(bool(self.traditional)), float(self.base), float(self.scale),
                               int(offset))


def rope(x: torch.Tensor, r: Rope, offset: int = 0) -> torch.Tensor:
    """Rotate x [B, H, L, D] (float16/bfloat16, CUDA) in place, rows at positions offset + l, and
    return it: the query side of a fused RoPE + cache update (kernels.metal:106-160)."""
    dev = _require_cuda(x)
    if x.dim() != 4:
        raise ValueError(f"x must be [B, H, L, D], got {tuple(x.shape)}")
    B, H, L, D = x.shape
    xr, rp = _lib.rows(x), r.params(offset)
    rc = _lib.lib().kvq_rope(ctypes.byref(xr), ctypes.byref(rp), B, H, L, D, _lib.dtype_code(x.dtype),
                             _lib.stream_ptr(dev))
    _lib.check(rc, "kvq_rope")
    return x


def quantize_append(k: torch.Tensor, k_dst: Triple, v: Optional[torch.Tensor] = None, v_dst: Optional[Triple] = None,
                    row_offset: int = 0, group_size: int = 64, bits: int = 8, rope: Optional[Rope] = None,
                    rope_offset: Optional[int] = None) -> None:
    """Quantize k (and v) [B, H, L, D] and store them at rows [row_offset, row_offset + L) of the
    (codes, scales, biases) buffers k_dst (and v_dst), in one kernel launch. With `rope`, the keys
    are rotated first (row l at position rope_offset + l, rope_offset defaulting to row_offset) and
    rounded to their dtype before they are quantized; k itself is not modified."""
    _check_triple(k_dst, "k_dst")
    tens = [k, *k_dst]
    if v is not None:
        if v_dst is None:
            raise ValueError("v_dst is required with v")
        _check_triple(v_dst, "v_dst")
        if v.shape != k.shape or v.dtype != k.dtype:
            raise ValueError("k and v must have the same shape and dtype")
        tens += [v, *v_dst]
    dev = _require_cuda(*tens)
    B, H, L, D = k.shape
    for tr in [k_dst] + ([v_dst] if v is not None else []):
        codes, scales, _ = tr
        if codes.shape[:2] != (B, H) or scales.shape[:2] != (B, H):
            raise ValueError(f"destination leads {tuple(codes.shape[:2])} do not match source {(B, H)}")
        if row_offset + L > codes.shape[2] or row_offset + L > scales.shape[2]:
            raise ValueError(f"rows [{row_offset}, {row_offset + L}) exceed the destination's {codes.shape[2]} rows")
        if codes.shape[3] != D * bits // 32 or scales.shape[3] != D // group_size:
            raise ValueError("destination row widths do not match D, bits and group_size")
        if scales.dtype != k.dtype:
            raise ValueError("scales/biases must have the dtype of the rows (MLX stores them in T)")
    L_ = _lib.lib()
    kr, kq = _lib.rows(k), _lib.qtensor(*k_dst, range_exp=range_word(k_dst[0]))
    if v is not None:
        vr, vq = _lib.rows(v), _lib.qtensor(*v_dst, range_exp=range_word(v_dst[0]))
        vr_p, vq_p = ctypes.byref(vr), ctypes.byref(vq)
    else:
        vr_p = vq_p = None
    if rope is None:
        rc = L_.kvq_quantize_append(ctypes.byref(kr), ctypes.byref(kq), vr_p, vq_p, int(row_offset), B, H, L, D,
                                    int(bits), int(group_size), _lib.dtype_code(k.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "kvq_quantize_append")
    else:
        rp = rope.params(row_offset if rope_offset is None else rope_offset)
        rc = L_.kvq_rope_quantize_append(ctypes.byref(kr), ctypes.byref(kq), vr_p, vq_p, ctypes.byref(rp),
                                         int(row_offset), B, H, L, D, int(bits), int(group_size),
                                         _lib.dtype_code(k.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "kvq_rope_quantize_append")


class AppendCall:
    """A quantize-append into fixed destination buffers with its C-ABI descriptors built once.

    ``prepare_append`` validates the destinations; calling the object with new source rows fills
    two preallocated row descriptors and makes one foreign call, so a decode loop pays a few
    microseconds of host time per layer instead of rebuilding every descriptor. Launches go to
    the stream that was current at preparation time.
    """

    def __init__(self, k_dst: Triple, v_dst: Optional[Triple], group_size: int, bits: int,
                 rope: Optional[Rope]):
        _check_triple(k_dst, "k_dst")
        tens = list(k_dst)
        if v_dst is not None:
            _check_triple(v_dst, "v_dst")
            tens += list(v_dst)
        self._dev = _require_cuda(*tens)
        self._k_dst, self._v_dst = k_dst, v_dst  # the descriptors point into these
        codes, scales, _ = k_dst
        self._lead = tuple(codes.shape[:2])
        self._rows = min(codes.shape[2], scales.shape[2])
        self._widths = (codes.shape[3], scales.shape[3])
        if v_dst is not None:
            if tuple(v_dst[0].shape) != tuple(codes.shape) or tuple(v_dst[1].shape) != tuple(scales.shape):
                raise ValueError("k_dst and v_dst must have the same shapes")
            if v_dst[1].dtype != scales.dtype:
                raise ValueError("k_dst and v_dst must share a dtype")
        self._kq = _lib.qtensor(*k_dst, range_exp=range_word(k_dst[0]))
        self._vq = _lib.qtensor(*v_dst, range_exp=range_word(v_dst[0])) if v_dst is not None else None
        self._kr, self._vr = _lib.Rows(), _lib.Rows()
        self._dtype = k_dst[1].dtype
        self._code = _lib.dtype_code(self._dtype)
        self._bits, self._group = int(bits), int(group_size)
        self._rope = rope
        self._rp = rope.params(0) if rope is not None else None
        lib = _lib.lib()
        self._fn = lib.kvq_rope_quantize_append if rope is not None else lib.kvq_quantize_append
        self._stream = _lib.stream_ptr(self._dev)

    def __call__(self, k: torch.Tensor, v: Optional[torch.Tensor], row_offset: int,
                 rope_offset: Optional[int] = None) -> None:
        if k.dtype != self._dtype or k.device != self._dev or k.dim() != 4 or k.stride(-1) != 1:
            raise ValueError("rows must match the prepared dtype and device, as [B, H, L, D] with D contiguous")
        B, H, L, D = k.shape
        if (B, H) != self._lead:
            raise ValueError(f"destination leads {self._lead} do not match source {(B, H)}")
        if row_offset < 0 or row_offset + L > self._rows:
            raise ValueError(f"rows [{row_offset}, {row_offset + L}) exceed the destination's {self._rows} rows")
        if self._widths != (D * self._bits // 32, D // self._group):
            raise ValueError("destination row widths do not match D, bits and group_size")
        kr = self._kr
        kr.data = k.data_ptr()
        kr.stride_b, kr.stride_h, kr.stride_l = k.stride()[:3]
        vr_p = vq_p = None
        if v is not None:
            if self._vq is None or v.shape != k.shape or v.dtype != k.dtype or v.stride(-1) != 1:
                raise ValueError("values must match the keys and a prepared value destination")
            vr = self._vr
            vr.data = v.data_ptr()
            vr.stride_b, vr.stride_h, vr.stride_l = v.stride()[:3]
            vr_p, vq_p = ctypes.byref(vr), ctypes.byref(self._vq)
        if self._rp is None:
            rc = self._fn(ctypes.byref(kr), ctypes.byref(self._kq), vr_p, vq_p, int(row_offset), B, H, L, D,
                          self._bits, self._group, self._code, self._stream)
        else:
            self._rp.offset = int(row_offset if rope_offset is None else rope_offset)
            rc = self._fn(ctypes.byref(kr), ctypes.byref(self._kq), vr_p, vq_p, ctypes.byref(self._rp),
                          int(row_offset), B, H, L, D, self._bits, self._group, self._code, self._stream)
        if rc:
            _lib.check(rc, "kvq_rope_quantize_append" if self._rp is not None else "kvq_quantize_append")


def prepare_append(k_dst: Triple, v_dst: Optional[Triple] = None, *, group_size: int = 64, bits: int = 8,
                   rope: Optional[Rope] = None) -> AppendCall:
    """Build an ``AppendCall`` for repeated appends into the same (codes, scales, biases) buffers."""
    return AppendCall(k_dst, v_dst, group_size, bits, rope)


def quantize(x: torch.Tensor, group_size: int = 64, bits: int = 8) -> Triple:
    """Counterpart of mx.quantize(x, group_size, bits) for x [..., D] on the GPU:
    returns (codes uint32 [..., D*bits/32], scales [..., D/G], biases [..., D/G])."""
    _require_cuda(x)
    lead = x.shape[:-1]
    D = x.shape[-1]
    x4 = x.reshape(1, 1, -1, D)
    if x4.stride(-1) != 1:
        x4 = x4.contiguous()
    n = x4.shape[2]
    codes = torch.empty((1, 1, n, D * bits // 32), dtype=torch.uint32, device=x.device)
    scales = torch.empty((1, 1, n, D // group_size), dtype=x.dtype, device=x.device)
    biases = torch.empty_like(scales)
    quantize_append(x4, (codes, scales, biases), row_offset=0, group_size=group_size, bits=bits)
    return (codes.reshape(*lead, -1), scales.reshape(*lead, -1), biases.reshape(*lead, -1))


FP16_MAX = 65504.0


def fits_fp16_operands(triple: Triple, bits: int) -> bool:
    """Whether every dequantized value s * c + b (c in [0, 2^bits - 1]) of a (codes, scales,
    biases) triple lies inside the fp16 range. The prefill kernel's dequantized operands are fp16:
    for a bf16 cache with a group outside that range its query rows come back NaN (decode is exact
    either way), so a caller whose bf16 K/V can exceed 65504 checks its cache once with this and
    routes those layers through decode. Works on the triple's device; returns a Python bool (a
    synchronisation on the GPU)."""
    _check_triple(triple, "triple")
    _, scales, biases = triple
    s, b = scales.float(), biases.float()
    hi = b + s * float((1 << bits) - 1)
    worst = torch.maximum(b.abs(), hi.abs())
    return bool(torch.isfinite(worst).all().item()) and bool((worst <= FP16_MAX).all().item())


NATIVE_HEAD_DIMS = (64, 128, 256)


def kernel_dim(D: int) -> int:
    """The width the kernels compute head dimension D at: 64, 128 or 256. Other multiples of 8 (up to
    256 for quantized caches, 128 for unquantized ones) run the decode kernel at the next width, with
    zero queries past their last dim, for every query length."""
    return 64 if D <= 64 else 128 if D <= 128 else 256


def decode_rows_per_pass(D: int, group_size: int = 64) -> int:
    """Query rows (heads of a GQA group x query positions) one decode pass serves: the 16 MFMA
    columns hold each row once per scale group of the kernel's width (an unquantized cache counts as
    group 64)."""
    return 16 * group_size // kernel_dim(D)


def _auto_kernel(rep_rows: int, D: int, group_size: int) -> str:
    """Decode while a KV head's query rows fit at most two decode passes over its keys (one pass for
    group 64, where 8 rows fit one pass), the prefill kernel otherwise (head dims 64, 128 and 256 have
    one; the others run the decode kernel at every length). At head_dim 256 the unquantized entry
    points run the head_dim-256 kernel for every query length."""
    if D not in NATIVE_HEAD_DIMS:
        return "decode"
    return "decode" if rep_rows <= max(decode_rows_per_pass(D, group_size), 8) else "prefill"


class AttentionCall:
    """A validated attention launch with its C-ABI arguments built once.

    ``prepare_attention`` checks shapes and dtypes, sizes the workspace and packs the ctypes
    descriptors; calling the object launches the kernels on the stream that was current at
    preparation time, with no further host-side work beyond one foreign call. Tensors are held
    by reference, so refilling them in place (a new query, appended cache rows inside the same
    views) is picked up by the next launch. Used by serving loops and HIP-graph capture.
    """

    def __init__(self, fn, args, keep, kernel: str, out: torch.Tensor, symbol: str):
        self._fn = fn
        self._args = args
        self._keep = keep  # tensors and ctypes structs whose addresses are baked into _args
        self.kernel = kernel  # "decode" or "prefill"
        self.symbol = symbol  # the C entry point
        self.out = out

    def __call__(self) -> torch.Tensor:
        rc = self._fn(*self._args)
        if rc:
            _lib.check(rc, self.symbol)
        return self.out


def _rows_ok(t: torch.Tensor) -> bool:
    """Rows the kernels can read directly: unit stride, 16-byte aligned, strides of 8 elements."""
    return t.stride(-1) == 1 and not any(st % 8 for st in t.stride()[:3]) and t.data_ptr() % 16 == 0


def _check_out(out: Optional[torch.Tensor], queries: torch.Tensor, dev) -> torch.Tensor:
    """A fresh output, or the caller's after the checks the kernels' stores rely on: the queries'
    shape, dtype and device, unit stride along D, 8-byte alignment and strides of 4 elements (the
    kernels write 4 elements at a time; prefill also needs 16-byte rows, checked by the library)."""
    B, Hq, L, D = queries.shape
    if out is None:
        return torch.empty((B, Hq, L, D), dtype=queries.dtype, device=dev)
    if tuple(out.shape) != (B, Hq, L, D) or out.dtype != queries.dtype or out.device != dev:
        raise ValueError(f"out must be a {queries.dtype} tensor of shape {(B, Hq, L, D)} on {dev}")
    if out.stride(-1) != 1 or any(st % 4 for st in out.stride()[:3]) or out.data_ptr() % 8:
        raise ValueError("out must have unit stride along D, 8-byte alignment and strides that are multiples of 4")
    return out


def _copy_for_one_shot(t: torch.Tensor, name: str, one_shot: bool) -> torch.Tensor:
    """A contiguous copy of a tensor the kernels cannot read in place. Only a one-shot call may take
    it: a prepared call holds its tensors by reference, so a copy would silently freeze them."""
    if not one_shot:
        raise ValueError(
            f"prepare_attention: {name} need unit stride along D, 16-byte alignment and strides that are multiples "
            f"of 8 elements (got strides {tuple(t.stride())}); a prepared call reads its tensors in place on every "
            f"launch, so pass .contiguous() tensors (and refill those)")
    return t.contiguous()


def prepare_attention(queries: torch.Tensor, keys, values, scale: float, *, causal: bool = False,
                      window: int = 0, seq_lens: Optional[torch.Tensor] = None, group_size: int = 64,
                      bits: int = 8, out: Optional[torch.Tensor] = None, kernel: str = "auto",
                      workspace: Optional[torch.Tensor] = None, _one_shot: bool = False) -> AttentionCall:
    """Validate one attention launch and return it as an ``AttentionCall`` (see ``attention``).

    The queries and unquantized keys/values must be readable in place (unit stride along D, 16-byte
    aligned, strides in multiples of 8 elements): a prepared call reads the same memory on every
    launch, so a tensor that would need a copy raises ValueError rather than being snapshotted."""
    if queries.dim() != 4:
        raise ValueError(f"queries must be [B, Hq, L, D], got {tuple(queries.shape)}")
    B, Hq, L, D = queries.shape
    dense = torch.is_tensor(keys)
    if dense:
        if not torch.is_tensor(values):
            raise ValueError("keys and values must both be tensors (unquantized) or both be triples")
        dev = _require_cuda(queries, keys, values)
        Hkv, S = keys.shape[1], keys.shape[2]
        for name, t in (("keys", keys), ("values", values)):
            if t.dim() != 4 or tuple(t.shape) != (B, Hkv, S, D):
                raise ValueError(f"{name} must be [B, Hkv, S, D] = {(B, Hkv, S, D)}, got {tuple(t.shape)}")
            if t.dtype != queries.dtype:
                raise ValueError(f"{name} are {t.dtype}, queries are {queries.dtype}")
        if not _rows_ok(keys):
            keys = _copy_for_one_shot(keys, "keys", _one_shot)
        if not _rows_ok(values):
            values = _copy_for_one_shot(values, "values", _one_shot)
    else:
        _check_triple(keys, "keys")
        _check_triple(values, "values")
        dev = _require_cuda(queries, *keys, *values)
        Hkv, S = keys[0].shape[1], keys[0].shape[2]
        for name, tr in (("keys", keys), ("values", values)):
            c, s, b = tr
            if c.shape[0] != B or c.shape[1] != Hkv or c.shape[2] != S or s.shape[:3] != c.shape[:3]:
                raise ValueError(f"{name} triple shapes {tuple(c.shape)}, {tuple(s.shape)} do not match B={B}, Hkv={Hkv}, S={S}")
            if c.shape[3] * 32 // bits != D:
                raise ValueError(f"{name} codes hold {c.shape[3] * 32 // bits} dims at {bits} bits, queries have {D}")
            if s.shape[3] * group_size != D:
                raise ValueError(f"{name} scales hold {s.shape[3]} groups, expected D/group_size = {D // group_size}")
            if s.dtype != queries.dtype:
                raise ValueError(f"{name} scales are {s.dtype}, queries are {queries.dtype}")
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if not _rows_ok(queries):
        queries = _copy_for_one_shot(queries, "queries", _one_shot)
    out = _check_out(out, queries, dev)
    sl_ptr = None
    if seq_lens is not None:
        if seq_lens.dtype != torch.int32 or seq_lens.device != dev or seq_lens.numel() != B:
            raise ValueError("seq_lens must be an int32 tensor of B entries on the queries' device")
        sl_ptr = seq_lens.data_ptr()
    rep = Hq // Hkv
    if kernel == "auto":
        kernel = _auto_kernel(rep * L, D, 64 if dense else group_size)
    if kernel not in ("decode", "prefill"):
        raise ValueError(f"kernel must be 'decode', 'prefill' or 'auto', got {kernel!r}")
    lib = _lib.lib()
    ws_fn = lib.kvq_decode_workspace_size if kernel == "decode" else lib.kvq_prefill_workspace_size
    symbol = f"kvq_{kernel}_attn" + ("_dense" if dense else "")
    fn = getattr(lib, symbol)
    nbytes = ws_fn(B, Hq, Hkv, L, D, S, int(window))
    if nbytes == 0:
        raise NotImplementedError(f"{kernel} attention does not support B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} S={S}")
    stream = _lib.stream_ptr(dev)
    if workspace is None:
        ws = _workspace(dev, stream, nbytes)
    else:
        if workspace.device != dev or workspace.numel() * workspace.element_size() < nbytes:
            raise ValueError(f"workspace must hold at least {nbytes} bytes on {dev}")
        ws = workspace
    qr, orr = _lib.rows(queries), _lib.rows(out)
    tail = (_lib.dtype_code(queries.dtype), float(scale), int(bool(causal)), int(window), ws.data_ptr(),
            ws.numel() * ws.element_size(), stream)
    if dense:
        kq, vq = _lib.rows(keys), _lib.rows(values)
        args = (ctypes.byref(qr), ctypes.byref(kq), ctypes.byref(vq), sl_ptr, ctypes.byref(orr), B, Hq, Hkv, L, D, S,
                *tail)
    else:
        # the caches' range words: registered with their buffers, else (one-shot prefill calls)
        # computed from the scales and biases on the device; decode applies scales in fp32 and
        # reads none
        kw, vw = range_word(keys[0]), range_word(values[0])
        if kernel == "prefill" and _one_shot:
            kw = range_exponent(keys, bits) if kw is None else kw
            vw = range_exponent(values, bits) if vw is None else vw
        kq, vq = _lib.qtensor(*keys, range_exp=kw), _lib.qtensor(*values, range_exp=vw)
        args = (ctypes.byref(qr), ctypes.byref(kq), ctypes.byref(vq), sl_ptr, ctypes.byref(orr), B, Hq, Hkv, L, D, S,
                int(bits), int(group_size), *tail)
        keep_words = (kw, vw)
    keep = (queries, keys, values, seq_lens, ws, qr, orr, kq, vq) + (() if dense else keep_words)
    return AttentionCall(fn, args, keep, kernel, out, symbol)


def attention(queries: torch.Tensor, keys, values, scale: float, *, causal: bool = False,
              window: int = 0, seq_lens: Optional[torch.Tensor] = None, group_size: int = 64, bits: int = 8,
              out: Optional[torch.Tensor] = None, kernel: str = "auto") -> torch.Tensor:
    """softmax(scale * q K^T + mask) V. queries [B, Hq, L, D]; keys/values either quantized triples
    (codes [B, Hkv, S, D*bits/32], scales/biases [B, Hkv, S, D/G]) or unquantized tensors
    [B, Hkv, S, D] in the queries' dtype; returns [B, Hq, L, D] (or fills `out`). kernel: "decode",
    "prefill" or "auto" (decode while a KV head's query rows fit max(16*G/D, 8) columns, that is
    at most two decode passes over its keys, prefill otherwise)."""
    return prepare_attention(queries, keys, values, scale, causal=causal, window=window, seq_lens=seq_lens,
                             group_size=group_size, bits=bits, out=out, kernel=kernel, _one_shot=True)()


# ---- general masks (kvq_mask): boolean masks with no causal / window / padding structure, per-head
# masks and additive masks, read by the decode kernel beside every tile

_MASK_KINDS = {torch.bool: _lib.MASK_BOOL, torch.float16: _lib.MASK_F16, torch.bfloat16: _lib.MASK_BF16,
               torch.float32: _lib.MASK_F32}


def mask_view(mask: torch.Tensor, B: int, Hq: int, Hkv: int, L: int, S: int, layout: str = "heads"):
    """The mask as the kernels read it: (tensor, (stride_b, stride_kvh, stride_rep, stride_l)) over the
    [B, Hkv, Hq / Hkv, L, S] score layout, keys contiguous, broadcast dimensions at stride 0.

    ``layout`` is how the caller's reference broadcasts the mask against the scores:
      "heads"    against [B, Hq, L, S] (mx.fast.scaled_dot_product_attention);
      "grouped"  against [B, Hkv, Hq / Hkv, L, S] as given (mlx-lm's quantized SDPA, the L == 1 /
                 short-S hand-off of m5engine/attention.py:42-45);
      "blocked"  a mask of rank 3 or more gains an axis at -3 first (m5engine/attention.py:55-56),
                 so its head axis indexes KV heads.
    With Hq == Hkv the three agree."""
    if layout not in ("heads", "grouped", "blocked"):
        raise ValueError(f"layout must be 'heads', 'grouped' or 'blocked', got {layout!r}")
    m = mask
    if m.dtype == torch.float64:
        m = m.float()
    if m.dtype not in _MASK_KINDS:
        raise ValueError(f"masks are bool (visible keys) or float (additive), got {m.dtype}")
    if m.dim() == 0 or m.shape[-1] not in (1, S):
        raise ValueError(f"the mask's last dimension {tuple(m.shape)[-1:]} does not broadcast to S = {S}")
    if m.shape[-1] == 1 and S != 1:
        m = m.expand(*m.shape[:-1], S)
    if m.stride(-1) != 1:
        m = m.contiguous()
    rep = Hq // Hkv
    try:
        if rep == 1 or layout == "heads":
            m4 = torch.broadcast_to(m, (B, Hq, L, S))
            sb, sh, sl, _ = m4.stride()
            return m4, (sb, rep * sh, sh, sl)
        if layout == "blocked" and m.dim() >= 3:
            m = m.unsqueeze(-3)
        m5 = torch.broadcast_to(m, (B, Hkv, rep, L, S))
    except RuntimeError as e:
        raise ValueError(f"mask of shape {tuple(mask.shape)} does not broadcast to the scores: {e}") from None
    sb, skv, srep, sl, _ = m5.stride()
    return m5, (sb, skv, srep, sl)


def masked_attention(queries: torch.Tensor, keys, values, scale: float, mask: torch.Tensor, *, layout: str = "heads",
                     group_size: int = 64, bits: int = 8, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(scale * q K^T + mask) V under a general mask (boolean: visible keys; float: added to
    the scores), keys/values quantized triples or unquantized tensors as for ``attention``. Runs the
    decode kernel (any L: rows beyond one pass take more passes over the keys), or, for an
    unquantized head_dim-256 cache, the head_dim-256 kernel. A row that sees no key returns 0."""
    if queries.dim() != 4:
        raise ValueError(f"queries must be [B, Hq, L, D], got {tuple(queries.shape)}")
    B, Hq, L, D = queries.shape
    dense = torch.is_tensor(keys)
    if dense:
        dev = _require_cuda(queries, keys, values)
        Hkv, S = keys.shape[1], keys.shape[2]
        for name, t in (("keys", keys), ("values", values)):
            if t.dim() != 4 or tuple(t.shape) != (B, Hkv, S, D) or t.dtype != queries.dtype:
                raise ValueError(f"{name} must be {queries.dtype} [B, Hkv, S, D] = {(B, Hkv, S, D)}")
        keys = keys if _rows_ok(keys) else keys.contiguous()
        values = values if _rows_ok(values) else values.contiguous()
    else:
        _check_triple(keys, "keys")
        _check_triple(values, "values")
        dev = _require_cuda(queries, *keys, *values)
        Hkv, S = keys[0].shape[1], keys[0].shape[2]
        if keys[0].shape[0] != B or keys[0].shape[3] * 32 // bits != D or keys[1].shape[3] * group_size != D:
            raise ValueError("keys triple does not match the queries' B and D at these bits and group_size")
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if not torch.is_tensor(mask):
        raise ValueError("mask must be a tensor")
    if mask.device != dev:
        mask = mask.to(dev)
    mview, strides = mask_view(mask, B, Hq, Hkv, L, S, layout)
    desc = _lib.Mask(mview.data_ptr(), _MASK_KINDS[mview.dtype], *strides)
    if not _rows_ok(queries):
        queries = queries.contiguous()
    out = _check_out(out, queries, dev)
    lib = _lib.lib()
    nbytes = lib.kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, 0)
    if nbytes == 0:
        raise NotImplementedError(f"decode attention does not support B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} S={S}")
    stream = _lib.stream_ptr(dev)
    ws = _workspace(dev, stream, nbytes)
    qr, orr = _lib.rows(queries), _lib.rows(out)
    tail = (float(scale), ctypes.byref(desc), ws.data_ptr(), ws.numel() * ws.element_size(), stream)
    if dense:
        kr, vr = _lib.rows(keys), _lib.rows(values)
        rc = lib.kvq_decode_attn_dense_masked(ctypes.byref(qr), ctypes.byref(kr), ctypes.byref(vr), ctypes.byref(orr),
                                              B, Hq, Hkv, L, D, S, _lib.dtype_code(queries.dtype), *tail)
        _lib.check(rc, "kvq_decode_attn_dense_masked")
    else:
        kq, vq = _lib.qtensor(*keys), _lib.qtensor(*values)
        rc = lib.kvq_decode_attn_masked(ctypes.byref(qr), ctypes.byref(kq), ctypes.byref(vq), ctypes.byref(orr), B, Hq,
                                        Hkv, L, D, S, int(bits), int(group_size), _lib.dtype_code(queries.dtype), *tail)
        _lib.check(rc, "kvq_decode_attn_masked")
    return out


# ---- paged pools (64-row pages; include/kvq.h "Paged layout")

PAGE_ROWS = _lib.PAGE_ROWS


def _check_table(block_tables: torch.Tensor, B: int, dev) -> None:
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.shape[0] != B:
        raise ValueError(f"block_tables must be int32 [B={B}, max_pages], got {block_tables.dtype} "
                         f"{tuple(block_tables.shape)}")
    if block_tables.device != dev or block_tables.stride(1) != 1:
        raise ValueError("block_tables must be on the queries' device with contiguous rows")


def paged_quantize_append(k: torch.Tensor, k_pool: Triple, v: Optional[torch.Tensor], v_pool: Optional[Triple],
                          block_tables: torch.Tensor, *, starts: Optional[torch.Tensor] = None, row_offset: int = 0,
                          group_size: int = 64, bits: int = 8, rope: Optional[Rope] = None) -> None:
    """Quantize k (and v) [B, H, L, D] into paged pools ([num_pages, H, 64, *] triples): row l of
    sequence b goes to row starts[b] + l (or row_offset + l) of that sequence's pages. With `rope`
    the keys are rotated at those positions first."""
    _check_triple(k_pool, "k_pool")
    tens = [k, *k_pool]
    if v is not None:
        _check_triple(v_pool, "v_pool")
        tens += [v, *v_pool]
    dev = _require_cuda(*tens)
    B, H, L, D = k.shape
    _check_table(block_tables, B, dev)
    st_ptr = None
    if starts is not None:
        if starts.dtype != torch.int32 or starts.numel() != B or starts.device != dev:
            raise ValueError("starts must be an int32 tensor of B entries on the same device")
        st_ptr = starts.data_ptr()
    kr, kq = _lib.rows(k), _lib.qtensor(*k_pool, range_exp=range_word(k_pool[0]))
    vr_p = vq_p = None
    if v is not None:
        vr, vq = _lib.rows(v), _lib.qtensor(*v_pool, range_exp=range_word(v_pool[0]))
        vr_p, vq_p = ctypes.byref(vr), ctypes.byref(vq)
    rp = None
    if rope is not None:
        rparams = rope.params(0 if starts is not None else row_offset)
        rp = ctypes.byref(rparams)
    rc = _lib.lib().kvq_paged_quantize_append(
        ctypes.byref(kr), ctypes.byref(kq), vr_p, vq_p, k_pool[0].shape[0], block_tables.data_ptr(),
        block_tables.stride(0), st_ptr, int(row_offset), rp, B, H, L, D, int(bits), int(group_size),
        _lib.dtype_code(k.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "kvq_paged_quantize_append")


def paged_attention(queries: torch.Tensor, k_pool: Triple, v_pool: Triple, block_tables: torch.Tensor,
                    seq_lens: torch.Tensor, scale: float, *, causal: bool = False, window: int = 0,
                    group_size: int = 64, bits: int = 8, max_len: Optional[int] = None,
                    out: Optional[torch.Tensor] = None, kernel: str = "auto") -> torch.Tensor:
    """softmax(scale * q K^T + mask) V over paged pools: sequence b holds seq_lens[b] rows in the
    pages block_tables[b]; queries [B, Hq, L, D] sit at its last L positions. max_len bounds
    seq_lens (default: the table's capacity) and sizes the split plan."""
    _check_triple(k_pool, "k_pool")
    _check_triple(v_pool, "v_pool")
    dev = _require_cuda(queries, *k_pool, *v_pool)
    if queries.dim() != 4:
        raise ValueError(f"queries must be [B, Hq, L, D], got {tuple(queries.shape)}")
    B, Hq, L, D = queries.shape
    _check_table(block_tables, B, dev)
    if seq_lens.dtype != torch.int32 or seq_lens.numel() != B or seq_lens.device != dev:
        raise ValueError("seq_lens must be an int32 tensor of B entries on the queries' device")
    Hkv = k_pool[0].shape[1]
    if k_pool[0].shape[2] != PAGE_ROWS or k_pool[1].dtype != queries.dtype:
        raise ValueError(f"pools must be [num_pages, Hkv, {PAGE_ROWS}, *] with scales in the queries' dtype")
    for a, b_ in zip(k_pool, v_pool):
        if tuple(a.shape) != tuple(b_.shape) or a.dtype != b_.dtype:
            raise ValueError("v_pool must match k_pool in every shape and dtype (the kernels read both through "
                             "one block table over k_pool's page count)")
    if k_pool[0].shape[3] * 32 // bits != D or k_pool[1].shape[3] * group_size != D or k_pool[1].shape[:3] != \
            k_pool[0].shape[:3]:
        raise ValueError(f"pools' row widths do not match D={D}, bits={bits} and group_size={group_size}")
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    S = int(max_len) if max_len is not None else block_tables.shape[1] * PAGE_ROWS
    if not _rows_ok(queries):
        queries = _copy_for_one_shot(queries, "queries", True)
    out = _check_out(out, queries, dev)
    if kernel == "auto":
        kernel = _auto_kernel((Hq // Hkv) * L, D, group_size)
    lib = _lib.lib()
    ws_fn = lib.kvq_decode_workspace_size if kernel == "decode" else lib.kvq_prefill_workspace_size
    nbytes = ws_fn(B, Hq, Hkv, L, D, S, int(window))
    if nbytes == 0:
        raise NotImplementedError(f"{kernel} attention does not support B={B} Hq={Hq} Hkv={Hkv} L={L} D={D} S={S}")
    stream = _lib.stream_ptr(dev)
    ws = _workspace(dev, stream, nbytes)
    qr, orr = _lib.rows(queries), _lib.rows(out)
    # (only registered words: the unused rows of a pool's pages hold whatever was there)
    kw, vw = range_word(k_pool[0]), range_word(v_pool[0])
    kq, vq = _lib.qtensor(*k_pool, range_exp=kw), _lib.qtensor(*v_pool, range_exp=vw)
    fn = lib.kvq_paged_decode_attn if kernel == "decode" else lib.kvq_paged_prefill_attn
    rc = fn(ctypes.byref(qr), ctypes.byref(kq), ctypes.byref(vq), k_pool[0].shape[0], block_tables.data_ptr(),
            block_tables.stride(0), seq_lens.data_ptr(), ctypes.byref(orr), B, Hq, Hkv, L, D, S, int(bits),
            int(group_size), _lib.dtype_code(queries.dtype), float(scale), int(bool(causal)), int(window),
            ws.data_ptr(), ws.numel() * ws.element_size(), stream)
    _lib.check(rc, f"kvq_paged_{kernel}_attn")
    return out
