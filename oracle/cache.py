"""Bookkeeping model of mlx-lm's KVCache / QuantizedKVCache (third-party, mlx-lm==0.31.3,
requirements.txt:4). TEST INFRASTRUCTURE ONLY.

What the reference relies on (prefix_cache.py:17-38, 77-123; context.py:41-47, 56-68):
  * storage grows in steps of 256 rows: when offset + L exceeds the capacity, the buffers are
    first cut to `offset` if it is not a multiple of 256, then extended by ceil(L/256)*256 rows;
  * update_and_fetch(k, v) writes rows [offset, offset + L) and returns views [..., :offset, :];
  * trim(n) lowers offset by min(offset, n) and returns that amount; is_trimmable() is True;
  * nbytes is the byte size of the allocated buffers (capacity rows, not offset rows);
  * to_quantized(group_size, bits) quantizes the whole allocated buffer and keeps offset.
This model tracks (offset, capacity) only; the GPU cache classes must match it step for step.

RotatingCacheModel follows mlx-lm's RotatingKVCache (sliding-window layers; the caches
m5engine/attention.py:106-112 leaves unquantized and context.py:65-66 sizes by max_size) on token
positions instead of rows: which position each buffer row holds. Parity with mlx-lm itself is
unpinned (the module is absent here); tests/test_cache_rotating.py pins the model by the
properties a sliding-window cache must have.
"""

from __future__ import annotations

STEP = 256


class CacheModel:
    def __init__(self) -> None:
        self.offset = 0
        self.capacity = 0

    def update(self, L: int) -> None:
        prev = self.offset
        if self.capacity == 0 or prev + L > self.capacity:
            grow = (STEP + L - 1) // STEP * STEP
            if self.capacity:
                if prev % STEP != 0:
                    self.capacity = prev
                self.capacity += grow
            else:
                self.capacity = grow
        self.offset += L

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        return n


def row_bytes(D: int, bits: int | None, elem_bytes: int = 2, group_size: int = 64) -> int:
    """Bytes of one cached row of one head: D*bits/8 code bytes + 2 * (D/G) scale/bias elements,
    or D elements unquantized. Matches m5engine/context.py:169 (bits/8 + 4/64 bytes per element)."""
    if not bits:
        return D * elem_bytes
    return D * bits // 8 + 2 * (D // group_size) * elem_bytes


class RotatingCacheModel:
    """Buffer rows as token positions (None = an allocated row never written).

    Single-token updates write in place into a ring of max_size rows whose first `keep` rows are
    never overwritten, growing the buffer in steps of `step` until it reaches max_size. Multi-token
    updates first put the buffer in temporal order, keep its first `keep` rows and the newest
    max_size - 1 - keep others, and append the new tokens, so every new token sees at least
    max_size - 1 earlier ones (the buffer then holds up to max_size - 1 + L rows).
    """

    def __init__(self, max_size: int, keep: int = 0, step: int = STEP) -> None:
        self.max_size, self.keep, self.step = max_size, keep, step
        self.rows: list | None = None
        self.offset = 0
        self.idx = 0

    def _trim(self, n: int, rows: list, append: list | None = None) -> list:
        out = rows[: self.keep] + rows[n + self.keep:] if n > 0 else list(rows)
        return out + (append or [])

    def _temporal(self, rows: list) -> list:
        if self.idx == len(rows):
            return list(rows)
        if self.idx < self.offset:
            return rows[: self.keep] + rows[self.idx:] + rows[self.keep: self.idx]
        return rows[: self.idx]

    def update(self, L: int) -> list:
        """Append positions offset .. offset + L - 1; returns the fetched rows (as positions)."""
        new = list(range(self.offset, self.offset + L))
        if L > 1:
            if self.rows is None:
                self.rows = new
            else:
                self.rows = self._temporal(self.rows)
                self.idx = len(self.rows)
                self.rows = self._trim(self.idx - self.max_size + 1, self.rows, new)
            self.offset += L
            self.idx = len(self.rows)
            return list(self.rows)
        prev = self.offset
        if self.rows is None or (prev >= len(self.rows) and len(self.rows) < self.max_size):
            grow = min(self.step, self.max_size - prev)
            self.rows = (self.rows or []) + [None] * grow
            self.idx = prev
        extra = len(self.rows) - self.max_size
        if extra > 0:
            self.rows = self._trim(extra, self.rows)
            self.idx = self.max_size
        if self.idx == self.max_size:
            self.idx = self.keep
        self.rows[self.idx] = new[0]
        self.offset += 1
        self.idx += 1
        if self.offset < self.max_size:
            return self.rows[: self.offset]
        return list(self.rows)

    def trim(self, n: int) -> int:
        n = min(self.offset, n)
        self.offset -= n
        self.idx -= n
        return n
