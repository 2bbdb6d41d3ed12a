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
