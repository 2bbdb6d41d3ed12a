"""KV caches in MLX layout on the GPU: the objects the reference's attention path reads and
appends to.

Counterparts of mlx-lm's ``KVCache`` / ``QuantizedKVCache`` (third-party, mlx-lm==0.31.3,
requirements.txt:4), with the contract the reference relies on:
  * ``update_and_fetch(keys, values)`` appends [B, H, L, D] rows at ``offset`` and returns the
    ``[..., :offset, :]`` views (for the quantized cache: two (codes, scales, biases) triples);
  * storage grows in steps of 256 rows (cut to ``offset`` first when it is not step-aligned);
  * ``trim(n)`` / ``is_trimmable()`` / ``offset`` as used by m5engine/prefix_cache.py:77-123;
  * ``nbytes`` (allocated bytes) and ``state`` as used by m5engine/context.py:41-47, 56-68;
  * ``KVCache.to_quantized(group_size, bits)`` as used by m5engine/attention.py:106-112.
The quantized append is one launch of the fused quantize-and-append kernel for K and V.

MI355X addition: ``reserve(capacity)`` preallocates rows up front (one step-aligned buffer), so a
long generation does not re-copy the cache every 256 tokens; the contract above is unchanged.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import kernels

STEP = 256


def _grow_rows(prev: int, capacity: int, L: int, step: int = STEP) -> Tuple[int, int]:
    """(rows to keep, new capacity) when `L` rows are appended at `prev` and do not fit."""
    grow = (step + L - 1) // step * step
    if capacity == 0:
        return 0, grow
    keep = prev if prev % step != 0 else capacity
    return keep, keep + grow


def _new_like(t: torch.Tensor, rows: int) -> torch.Tensor:
    shape = list(t.shape)
    shape[2] = rows
    if t.dtype == torch.uint32:
        return torch.zeros(shape, dtype=torch.int32, device=t.device).view(torch.uint32)
    return torch.zeros(shape, dtype=t.dtype, device=t.device)


def _copy_rows(dst: torch.Tensor, src: torch.Tensor, rows: int) -> None:
    if rows == 0:
        return
    if dst.dtype == torch.uint32:
        dst[..., :rows, :].view(torch.int32).copy_(src[..., :rows, :].view(torch.int32))
    else:
        dst[..., :rows, :].copy_(src[..., :rows, :])


class KVCache:
    """Unquantized K/V rows [B, H, cap, D] (the cache before ``quantized_kv_start``)."""

    step = STEP

    def __init__(self) -> None:
        self.keys: Optional[torch.Tensor] = None
        self.values: Optional[torch.Tensor] = None
        self.offset = 0

    def _resize(self, like_k: torch.Tensor, like_v: torch.Tensor, L: int) -> None:
        cap = 0 if self.keys is None else self.keys.shape[2]
        keep, new_cap = _grow_rows(self.offset, cap, L, self.step)
        B, H, _, Dk = like_k.shape
        nk = torch.zeros((B, H, new_cap, Dk), dtype=like_k.dtype, device=like_k.device)
        nv = torch.zeros((B, H, new_cap, like_v.shape[3]), dtype=like_v.dtype, device=like_v.device)
        if self.keys is not None:
            _copy_rows(nk, self.keys, keep)
            _copy_rows(nv, self.values, keep)
        self.keys, self.values = nk, nv

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        prev = self.offset
        L = keys.shape[2]
        if self.keys is None or prev + L > self.keys.shape[2]:
            self._resize(keys, values, L)
        self.offset += L
        self.keys[..., prev:self.offset, :] = keys
        self.values[..., prev:self.offset, :] = values
        return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]

    @property
    def state(self):
        if self.keys is None:
            return None, None
        if self.offset == self.keys.shape[2]:
            return self.keys, self.values
        return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n

    @property
    def nbytes(self) -> int:
        if self.keys is None:
            return 0
        return self.keys.nbytes + self.values.nbytes

    def empty(self) -> bool:
        return self.keys is None

    def to_quantized(self, group_size: int = 64, bits: int = 4) -> "QuantizedKVCache":
        """Quantize the whole allocated buffer (mlx-lm semantics) into a QuantizedKVCache."""
        qc = QuantizedKVCache(group_size=group_size, bits=bits)
        qc.offset = self.offset
        if self.keys is not None:
            qc.keys = qc._alloc_like(self.keys, self.keys.shape[2])
            qc.values = qc._alloc_like(self.values, self.values.shape[2])
            kernels.quantize_append(self.keys, qc.keys, self.values, qc.values, row_offset=0,
                                    group_size=group_size, bits=bits)
        return qc


class QuantizedKVCache:
    """Affine-quantized K/V: per head, codes uint32 [B, H, cap, D*bits/32] and scales / biases in
    the K/V dtype [B, H, cap, D/group_size] (MLX layout)."""

    step = STEP

    def __init__(self, group_size: int = 64, bits: int = 8) -> None:
        if bits not in (2, 4, 8):
            raise ValueError(f"bits must be 2, 4 or 8, got {bits}")
        self.keys: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None
        self.values: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None
        self.offset = 0
        self.group_size = group_size
        self.bits = bits

    def _alloc_like(self, rows: torch.Tensor, cap: int):
        B, H, _, D = rows.shape
        if D % self.group_size or (D * self.bits) % 32:
            raise ValueError(f"head_dim {D} is not a multiple of group_size {self.group_size}")
        codes = torch.zeros((B, H, cap, D * self.bits // 32), dtype=torch.int32, device=rows.device).view(torch.uint32)
        scales = torch.zeros((B, H, cap, D // self.group_size), dtype=rows.dtype, device=rows.device)
        biases = torch.zeros_like(scales)
        return codes, scales, biases

    def _resize(self, keys: torch.Tensor, values: torch.Tensor, L: int, capacity: Optional[int] = None) -> None:
        cap = 0 if self.keys is None else self.keys[0].shape[2]
        if capacity is None:
            keep, new_cap = _grow_rows(self.offset, cap, L, self.step)
        else:
            keep, new_cap = (self.offset if self.keys is not None else 0), capacity
        nk = self._alloc_like(keys, new_cap)
        nv = self._alloc_like(values, new_cap)
        if self.keys is not None:
            for dst, src in zip(nk + nv, self.keys + self.values):
                _copy_rows(dst, src, keep)
        self.keys, self.values = nk, nv

    def reserve(self, like: torch.Tensor, capacity: int) -> None:
        """Preallocate `capacity` rows (rounded up to the step) shaped like `like` [B, H, *, D]."""
        capacity = (capacity + self.step - 1) // self.step * self.step
        if self.keys is None or self.keys[0].shape[2] < capacity:
            self._resize(like, like, 0, capacity=capacity)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor, rope: Optional["kernels.Rope"] = None):
        """Append keys/values [B, H, L, D] at `offset` and return the fetched views. With `rope`,
        the keys are rotated (positions offset .. offset + L - 1) in the same launch that
        quantizes them: the RoPE + cache update an attention layer does, fused."""
        prev = self.offset
        L = keys.shape[2]
        if self.keys is None or prev + L > self.keys[0].shape[2]:
            self._resize(keys, values, L)
        kernels.quantize_append(keys, self.keys, values, self.values, row_offset=prev,
                                group_size=self.group_size, bits=self.bits, rope=rope)
        self.offset += L
        return self.fetch()

    def fetch(self):
        """The (codes, scales, biases) views of the first `offset` rows, for K and for V."""
        o = self.offset
        return tuple(x[..., :o, :] for x in self.keys), tuple(x[..., :o, :] for x in self.values)

    @property
    def state(self):
        if self.keys is None:
            return None, None
        if self.offset == self.keys[0].shape[2]:
            return self.keys, self.values
        return self.fetch()

    def is_trimmable(self) -> bool:
        return True

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n

    @property
    def nbytes(self) -> int:
        if self.keys is None:
            return 0
        return sum(x.nbytes for x in self.keys + self.values)

    def empty(self) -> bool:
        return self.keys is None


def can_trim_prompt_cache(cache: List) -> bool:
    """mlx-lm's can_trim_prompt_cache, used at m5engine/prefix_cache.py:90."""
    return all(c.is_trimmable() for c in cache)


def trim_prompt_cache(cache: List, num_tokens: int) -> int:
    """mlx-lm's trim_prompt_cache, used at m5engine/prefix_cache.py:99."""
    if not can_trim_prompt_cache(cache) or len(cache) == 0:
        return 0
    return [c.trim(num_tokens) for c in cache][0]


def make_prompt_cache(num_layers: int) -> List[KVCache]:
    """One unquantized cache per attention layer (mlx-lm make_prompt_cache for plain models)."""
    return [KVCache() for _ in range(num_layers)]
