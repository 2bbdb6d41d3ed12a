"""ctypes binding of libkvq.so (declared in include/kvq.h).

The library is loaded once, after torch, so that it binds to the HIP runtime torch already
loaded (it is linked against torch/lib/libamdhip64.so). A missing or stale library raises at
load time; there is no fallback path.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch  # noqa: F401  (binds the HIP runtime before libkvq.so is loaded)

# The in-tree build, the only library this package loads.
LIB_PATH = Path(__file__).resolve().parent / "libkvq.so"
ABI_VERSION = 6

DTYPE_F16 = 0
DTYPE_BF16 = 1

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_HIP = -4
ERR_CAPACITY = -5
PAGE_ROWS = 64  # KVQ_PAGE_ROWS

# Function name -> (restype, argtypes); the complete export list of include/kvq.h.


class Rows(ctypes.Structure):
    """kvq_rows: a strided T[B][H][L][D] array (D contiguous)."""

    _fields_ = [("data", c_void_p), ("stride_b", c_int64), ("stride_h", c_int64), ("stride_l", c_int64)]


class QTensor(ctypes.Structure):
    """kvq_qtensor: the (codes, scales, biases) triple of one quantized K or V cache view."""

    _fields_ = [
        ("codes", c_void_p),
        ("scales", c_void_p),
        ("biases", c_void_p),
        ("codes_stride_b", c_int64),
        ("codes_stride_h", c_int64),
        ("codes_stride_s", c_int64),
        ("sb_stride_b", c_int64),
        ("sb_stride_h", c_int64),
        ("sb_stride_s", c_int64),
        ("range_exp", c_void_p),  # int32 range exponent in device memory, or NULL (include/kvq.h)
    ]


class RopeParams(ctypes.Structure):
    """kvq_rope_params: rotary embedding of the rows of one call (row l at position offset + l)."""

    _fields_ = [("dims", c_int), ("traditional", c_int), ("base", c_float), ("scale", c_float),
                ("offset", c_int64)]


_ATTN_ARGS = [
    POINTER(Rows), POINTER(QTensor), POINTER(QTensor), c_void_p, POINTER(Rows),
    c_int, c_int, c_int, c_int, c_int, c_int,  # B Hq Hkv L D S
    c_int, c_int, c_int,  # bits group dtype
    c_float, c_int, c_int,  # scale causal window
    c_void_p, c_size_t, c_void_p,  # workspace bytes stream
]
_DENSE_ARGS = [
    POINTER(Rows), POINTER(Rows), POINTER(Rows), c_void_p, POINTER(Rows),
    c_int, c_int, c_int, c_int, c_int, c_int,  # B Hq Hkv L D S
    c_int,  # dtype
    c_float, c_int, c_int,  # scale causal window
    c_void_p, c_size_t, c_void_p,  # workspace bytes stream
]
_WS_ARGS = [c_int, c_int, c_int, c_int, c_int, c_int, c_int]
_PAGED_ATTN_ARGS = [
    POINTER(Rows), POINTER(QTensor), POINTER(QTensor), c_int, c_void_p, c_int64, c_void_p, POINTER(Rows),
    c_int, c_int, c_int, c_int, c_int, c_int,  # B Hq Hkv L D S
    c_int, c_int, c_int,  # bits group dtype
    c_float, c_int, c_int,  # scale causal window
    c_void_p, c_size_t, c_void_p,  # workspace bytes stream
]


MASK_BOOL, MASK_F16, MASK_BF16, MASK_F32 = 1, 2, 3, 4  # KVQ_MASK_*


class Mask(ctypes.Structure):
    """kvq_mask: a general mask over the [B][Hkv][Hq / Hkv][L][S] score layout (keys contiguous;
    strides in elements, 0 broadcasts)."""

    _fields_ = [("data", c_void_p), ("kind", ctypes.c_int32), ("stride_b", c_int64), ("stride_kvh", c_int64),
                ("stride_rep", c_int64), ("stride_l", c_int64)]


_MASKED_ARGS = [
    POINTER(Rows), POINTER(QTensor), POINTER(QTensor), POINTER(Rows),
    c_int, c_int, c_int, c_int, c_int, c_int,  # B Hq Hkv L D S
    c_int, c_int, c_int,  # bits group dtype
    c_float, POINTER(Mask),  # scale mask
    c_void_p, c_size_t, c_void_p,  # workspace bytes stream
]
_DENSE_MASKED_ARGS = [
    POINTER(Rows), POINTER(Rows), POINTER(Rows), POINTER(Rows),
    c_int, c_int, c_int, c_int, c_int, c_int,  # B Hq Hkv L D S
    c_int,  # dtype
    c_float, POINTER(Mask),  # scale mask
    c_void_p, c_size_t, c_void_p,  # workspace bytes stream
]


class RadixInfo(ctypes.Structure):
    """kvq_radix_info: counters of a radix prefix cache."""

    _fields_ = [("num_pages", c_int), ("page_tokens", c_int), ("cached_pages", c_int), ("free_pages", c_int),
                ("in_use_pages", c_int), ("prefix_hit_tokens", c_int64), ("prompt_tokens", c_int64)]

SIGNATURES = {
    "kvq_abi_version": (c_int, []),
    "kvq_last_error": (c_char_p, []),
    "kvq_quantize_append": (
        c_int,
        [POINTER(Rows), POINTER(QTensor), POINTER(Rows), POINTER(QTensor), c_int64,
         c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "kvq_rope": (c_int, [POINTER(Rows), POINTER(RopeParams), c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "kvq_rope_quantize_append": (
        c_int,
        [POINTER(Rows), POINTER(QTensor), POINTER(Rows), POINTER(QTensor), POINTER(RopeParams), c_int64,
         c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "kvq_decode_attn": (c_int, _ATTN_ARGS),
    "kvq_decode_attn_static": (c_int, _ATTN_ARGS[:-3] + [c_void_p]),  # no workspace: the library's scratch
    "kvq_decode_attn_masked": (c_int, _MASKED_ARGS),
    "kvq_decode_attn_dense_masked": (c_int, _DENSE_MASKED_ARGS),
    "kvq_paged_quantize_append": (
        c_int,
        [POINTER(Rows), POINTER(QTensor), POINTER(Rows), POINTER(QTensor), c_int, c_void_p, c_int64, c_void_p, c_int64,
         POINTER(RopeParams), c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "kvq_paged_decode_attn": (c_int, _PAGED_ATTN_ARGS),
    "kvq_paged_prefill_attn": (c_int, _PAGED_ATTN_ARGS),
    "kvq_radix_create": (c_void_p, [c_int, c_int]),
    "kvq_radix_destroy": (None, [c_void_p]),
    "kvq_radix_match_and_allocate": (
        c_int, [c_void_p, POINTER(ctypes.c_int32), c_int, c_int, POINTER(ctypes.c_int32), c_int, POINTER(c_int),
                POINTER(c_int)],
    ),
    "kvq_radix_commit": (c_int, [c_void_p, POINTER(ctypes.c_int32), c_int, POINTER(ctypes.c_int32), c_int, c_int]),
    "kvq_radix_release": (c_int, [c_void_p, POINTER(ctypes.c_int32), c_int]),
    "kvq_radix_clear": (None, [c_void_p]),
    "kvq_radix_stats": (c_int, [c_void_p, POINTER(RadixInfo)]),
    "kvq_radix_last_error": (c_char_p, []),
    "kvq_decode_attn_dense": (c_int, _DENSE_ARGS),
    "kvq_prefill_attn_dense": (c_int, _DENSE_ARGS),
    "kvq_decode_workspace_size": (c_size_t, _WS_ARGS),
    "kvq_prefill_attn": (c_int, _ATTN_ARGS),
    "kvq_prefill_workspace_size": (c_size_t, _WS_ARGS),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load libkvq.so (once) and declare its signatures. Raises if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m myinfer_amd._build` "
                "(the HIP kernels have no fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.kvq_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = handle
        return handle


def last_error() -> str:
    msg = lib().kvq_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Map a kvq status code to a Python exception."""
    if rc == OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == ERR_INVALID:
        raise ValueError(msg)
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(f"{msg} (status {rc})")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return DTYPE_F16
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise ValueError(f"unsupported dtype {dtype}: expected float16 or bfloat16")


def rows(t: torch.Tensor) -> Rows:
    """Descriptor of a [B, H, L, D] tensor whose last dimension is contiguous."""
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D [B, H, L, D] tensor, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError("the last dimension must be contiguous")
    return Rows(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def qtensor(codes: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
            range_exp: torch.Tensor | None = None) -> QTensor:
    """Descriptor of a quantized [B, H, S, *] triple (codes uint32, scales/biases in T), with the
    cache's range exponent (a one-element int32 device tensor) when it keeps one."""
    for name, t in (("codes", codes), ("scales", scales), ("biases", biases)):
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D [B, H, S, *], got shape {tuple(t.shape)}")
        if t.stride(-1) != 1:
            raise ValueError(f"{name}: the last dimension must be contiguous")
    if codes.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"codes must be uint32, got {codes.dtype}")
    if scales.dtype != biases.dtype:
        raise ValueError("scales and biases must share a dtype")
    if scales.stride() != biases.stride() or scales.shape != biases.shape:
        raise ValueError("scales and biases must have identical shapes and strides")
    if range_exp is not None and (range_exp.dtype != torch.int32 or range_exp.numel() < 1
                                  or range_exp.device != codes.device):
        raise ValueError("range_exp must be an int32 tensor on the cache's device")
    return QTensor(
        codes.data_ptr(), scales.data_ptr(), biases.data_ptr(),
        codes.stride(0), codes.stride(1), codes.stride(2),
        scales.stride(0), scales.stride(1), scales.stride(2),
        None if range_exp is None else range_exp.data_ptr(),
    )


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
