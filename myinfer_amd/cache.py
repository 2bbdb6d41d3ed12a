"""KV caches in MLX layout on the GPU: the objects the reference's attention path reads and
appends to.

Counterparts of mlx-lm's ``KVCache`` / ``QuantizedKVCache`` / ``RotatingKVCache`` (third-party,
mlx-lm==0.31.3, requirements.txt:4), with the contract the reference relies on:
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
            qc.keys, qc.values = qc._buffers_like(self.keys, self.values, self.keys.shape[2])
            kernels.quantize_append(self.keys, qc.keys, self.values, qc.values, row_offset=0,
                                    group_size=group_size, bits=bits)
        return qc


class RotatingKVCache:
    """Sliding-window K/V rows [B, H, rows, D]: mlx-lm's RotatingKVCache, the cache of windowed
    attention layers. m5engine/attention.py:106-112 leaves it unquantized (its attention runs on
    the unquantized kernels) and m5engine/context.py:65-66 sizes it by ``max_size``.

    * One-token updates write in place into a ring of ``max_size`` rows (grown in steps of
      ``step`` until full); its first ``keep`` rows are never overwritten. The fetched rows are in
      ring order, which attention of a single query does not depend on.
    * Multi-token updates return the rows in temporal order: the ``keep`` first tokens, the newest
      ``max_size - 1 - keep`` earlier ones and the new tokens, so that with ``make_mask`` every new
      token sees a full window.
    """

    def __init__(self, max_size: int, keep: int = 0, step: int = STEP) -> None:
        if max_size <= 0 or keep < 0 or keep >= max_size:
            raise ValueError(f"need 0 <= keep < max_size, got keep={keep}, max_size={max_size}")
        self.max_size, self.keep, self.step = int(max_size), int(keep), int(step)
        self.keys: Optional[torch.Tensor] = None
        self.values: Optional[torch.Tensor] = None
        self.offset = 0
        self._idx = 0  # next ring row to write (one-token updates)

    def _drop_oldest(self, x: torch.Tensor, n: int, append: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x without its n oldest rows after the first `keep` (x in temporal order), plus `append`."""
        parts = [x[..., : self.keep, :], x[..., n + self.keep:, :]] if n > 0 else [x]
        if append is not None:
            parts.append(append)
        return torch.cat(parts, dim=2) if len(parts) > 1 else parts[0]

    def _in_time_order(self, x: torch.Tensor) -> torch.Tensor:
        if self._idx == x.shape[2]:
            return x
        if self._idx < self.offset:  # the ring has wrapped: the oldest rows follow the write point
            return torch.cat([x[..., : self.keep, :], x[..., self._idx:, :], x[..., self.keep: self._idx, :]], dim=2)
        return x[..., : self._idx, :]

    def _append_chunk(self, keys: torch.Tensor, values: torch.Tensor):
        if self.keys is None:
            self.keys, self.values = keys.clone(), values.clone()
        else:
            k, v = self._in_time_order(self.keys), self._in_time_order(self.values)
            self._idx = k.shape[2]
            drop = self._idx - self.max_size + 1
            self.keys, self.values = self._drop_oldest(k, drop, keys), self._drop_oldest(v, drop, values)
        self.offset += keys.shape[2]
        self._idx = self.keys.shape[2]
        return self.keys, self.values

    def _write_one(self, keys: torch.Tensor, values: torch.Tensor):
        prev = self.offset
        if self.keys is None or (prev >= self.keys.shape[2] and self.keys.shape[2] < self.max_size):
            grow = min(self.step, self.max_size - prev)
            B, H, _, Dk = keys.shape
            nk = torch.zeros((B, H, grow, Dk), dtype=keys.dtype, device=keys.device)
            nv = torch.zeros((B, H, grow, values.shape[3]), dtype=values.dtype, device=values.device)
            if self.keys is None:
                self.keys, self.values = nk, nv
            else:
                self.keys, self.values = torch.cat([self.keys, nk], dim=2), torch.cat([self.values, nv], dim=2)
            self._idx = prev
        extra = self.keys.shape[2] - self.max_size
        if extra > 0:  # after a multi-token update: back to a ring of max_size rows
            self.keys, self.values = self._drop_oldest(self.keys, extra), self._drop_oldest(self.values, extra)
            self._idx = self.max_size
        if self._idx == self.max_size:
            self._idx = self.keep
        self.keys[..., self._idx: self._idx + 1, :] = keys
        self.values[..., self._idx: self._idx + 1, :] = values
        self.offset += 1
        self._idx += 1
        if self.offset < self.max_size:
            return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]
        return self.keys, self.values

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        if keys.shape[2] == 1:
            return self._write_one(keys, values)
        return self._append_chunk(keys, values)

    def make_mask(self, N: int, window_size: Optional[int] = None):
        """The mask mlx-lm builds for N new queries over this cache: None or "causal" where that
        suffices, else a bool [N, S] causal sliding-window mask (ring-rotated for one query when
        the window is shorter than the ring)."""
        if N > 1:
            window_size = window_size or self.max_size
            off = min(self.max_size - 1, self.offset)
            if off + N > window_size:
                q = torch.arange(off, off + N)[:, None]
                k = torch.arange(off + N)[None, :]
                return (k <= q) & (k > q - window_size)
            return "causal"
        if window_size is None:
            return None
        if self.offset >= window_size and self.max_size > window_size:
            idx = self._idx if self._idx < self.max_size else 0
            n = min(self.max_size, self.offset + 1)
            return torch.roll(torch.arange(n) >= n - window_size, shifts=idx + 1)
        return None

    @property
    def state(self):
        if self.keys is None:
            return None, None
        if self.offset < self.keys.shape[2]:
            return self.keys[..., : self.offset, :], self.values[..., : self.offset, :]
        return self.keys, self.values

    def is_trimmable(self) -> bool:
        return self.offset < self.max_size

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        self._idx -= n
        return n

    @property
    def nbytes(self) -> int:
        if self.keys is None:
            return 0
        return self.keys.nbytes + self.values.nbytes

    def empty(self) -> bool:
        return self.keys is None

    def to_quantized(self, group_size: int = 64, bits: int = 4):
        raise NotImplementedError("RotatingKVCache quantization is not supported (mlx-lm raises too)")


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
        # the K and V range exponents (kernels.register_range_word): int32 [2] on the cache's device,
        # raised by the appends, read by the prefill kernels; it outlives buffer growth
        self.range_exp: Optional[torch.Tensor] = None

    def _buffers_like(self, like_k: torch.Tensor, like_v: torch.Tensor, cap: int):
        """New K and V buffers of `cap` rows, registered with the cache's range words."""
        if self.range_exp is None:
            self.range_exp = torch.zeros(2, dtype=torch.int32, device=like_k.device)
        nk, nv = self._alloc_like(like_k, cap), self._alloc_like(like_v, cap)
        kernels.register_range_word(nk[0], self.range_exp[0:1])
        kernels.register_range_word(nv[0], self.range_exp[1:2])
        return nk, nv

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
        nk, nv = self._buffers_like(keys, values, new_cap)
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
        # the append's descriptors are built once per buffer set, RoPE and stream
        key = (id(self.keys[0]), id(self.values[0]), rope, torch.cuda.current_stream(keys.device).cuda_stream)
        if getattr(self, "_append_key", None) != key:
            self._append = kernels.prepare_append(self.keys, self.values, group_size=self.group_size,
                                                  bits=self.bits, rope=rope)
            self._append_key = key
        self._append(keys, values, prev)
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

    def range_exponents(self) -> Tuple[int, int]:
        """The K and V range exponents the appends have raised (0, 0 while every value fits the fp16
        operands as it is). Reads device memory: a synchronization."""
        if self.range_exp is None:
            return 0, 0
        k, v = self.range_exp.tolist()
        return int(k), int(v)

    def fits_fp16_operands(self) -> bool:
        """Whether the cached K and V rows dequantize inside the fp16 range as they are
        (kernels.fits_fp16_operands); an empty cache fits. A cache that does not still gives finite
        prefill results: its range words scale the operands."""
        if self.keys is None or self.offset == 0:
            return True
        keys, values = self.fetch()
        return kernels.fits_fp16_operands(keys, self.bits) and kernels.fits_fp16_operands(values, self.bits)


def can_trim_prompt_cache(cache: List) -> bool:
    """mlx-lm's can_trim_prompt_cache, used at m5engine/prefix_cache.py:90."""
    return all(c.is_trimmable() for c in cache)


def trim_prompt_cache(cache: List, num_tokens: int) -> int:
    """mlx-lm's trim_prompt_cache, used at m5engine/prefix_cache.py:99."""
    if not can_trim_prompt_cache(cache) or len(cache) == 0:
        return 0
    return [c.trim(num_tokens) for c in cache][0]


def make_prompt_cache(num_layers: int, max_kv_size: Optional[int] = None,
                      layer_windows: Optional[List[Optional[int]]] = None) -> List:
    """One cache per attention layer, as mlx-lm's make_prompt_cache builds them: a KVCache per
    layer, or a RotatingKVCache(max_kv_size, keep=4) per layer when max_kv_size is given.
    layer_windows gives a model's own pattern instead (a model's make_cache(): a window size for
    each sliding-window layer, None for a global layer), e.g. five 1024-token windows then one
    global layer."""
    if layer_windows is not None:
        if len(layer_windows) != num_layers:
            raise ValueError(f"layer_windows has {len(layer_windows)} entries for {num_layers} layers")
        return [RotatingKVCache(max_size=w, keep=0) if w else KVCache() for w in layer_windows]
    if max_kv_size is not None:
        return [RotatingKVCache(max_size=max_kv_size, keep=4) for _ in range(num_layers)]
    return [KVCache() for _ in range(num_layers)]
