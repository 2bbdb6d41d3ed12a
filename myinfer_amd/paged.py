"""Paged quantized KV pools with a radix prefix cache: the MI355X counterpart of the reference's
PagedRadixKVCache (native/include/kv_cache.hpp, native/src/kv_cache.cpp:73-157).

The reference keeps whole caches and moves them in and out of its prefix cache
(m5engine/prefix_cache.py:1-5); its native engine instead pages the KV cache (16-token blocks
through a block table, native/src/kernels.metal:106-160, 384-450) and shares prompt prefixes
page by page. Here the pages hold the MLX-layout quantized cache:

  * ``PageRadix`` -- the host-side radix over page numbers (libkvq's kvq_radix_*, C++): which
    pages hold which token prefixes, with reference counts so that pages of running sequences
    are never evicted;
  * ``PagedRadixKVCache`` -- per-layer pools on the GPU, codes [max_blocks, Hkv, 64, D*bits/32]
    and scales/biases [max_blocks, Hkv, 64, D/64], plus a PageRadix; sequences append through
    ``kernels.paged_quantize_append`` and attend through ``kernels.paged_attention`` with
    int32 block tables.

Names follow the reference: match_and_allocate, commit_prefix_blocks, clear_cache, block_size,
max_blocks, cached_prefix_blocks, total_prefix_hits, total_prompt_tokens, kv_memory_bytes,
k_cache(layer), v_cache(layer); ``release`` is new (the hold on a finished sequence's pages).
Pages are 64 tokens (the reference's are 16): a 64-key prefill tile then reads exactly one page.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import _lib, kernels

PAGE_ROWS = _lib.PAGE_ROWS


@dataclass
class PrefixMatchResult:
    """native/include/kv_cache.hpp:10-14."""

    block_table: List[int]
    matched_tokens: int
    total_blocks_allocated: int


def _i32(seq: Sequence[int]):
    arr = (ctypes.c_int32 * max(len(seq), 1))(*seq)
    return arr


class PageRadix:
    """Radix prefix cache over `num_pages` pages of `page_tokens` tokens (host memory only)."""

    def __init__(self, num_pages: int, page_tokens: int = PAGE_ROWS) -> None:
        self._lib = _lib.lib()
        h = self._lib.kvq_radix_create(int(num_pages), int(page_tokens))
        if not h:
            raise ValueError(f"kvq_radix_create: {self._lib.kvq_radix_last_error().decode()}")
        self._h = h
        self.num_pages, self.page_tokens = int(num_pages), int(page_tokens)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.kvq_radix_destroy(h)

    def _err(self) -> str:
        return self._lib.kvq_radix_last_error().decode()

    def match_and_allocate(self, prompt_tokens: Sequence[int], max_new_tokens: int) -> PrefixMatchResult:
        toks = _i32(prompt_tokens)
        cap = self.num_pages
        table = (ctypes.c_int32 * cap)()
        matched, npages = ctypes.c_int(0), ctypes.c_int(0)
        rc = self._lib.kvq_radix_match_and_allocate(self._h, toks, len(prompt_tokens), int(max_new_tokens), table, cap,
                                                   ctypes.byref(matched), ctypes.byref(npages))
        if rc == _lib.ERR_CAPACITY:
            raise RuntimeError(f"PagedRadixKVCache: {self._err()}")
        if rc != _lib.OK:
            raise ValueError(f"match_and_allocate: {self._err()}")
        return PrefixMatchResult(list(table[: npages.value]), matched.value, npages.value)

    def commit_prefix_blocks(self, tokens: Sequence[int], block_table: Sequence[int], valid_token_count: int) -> None:
        rc = self._lib.kvq_radix_commit(self._h, _i32(tokens), len(tokens), _i32(block_table), len(block_table),
                                        int(valid_token_count))
        if rc != _lib.OK:
            raise ValueError(f"commit_prefix_blocks: {self._err()}")

    def release(self, block_table: Sequence[int]) -> None:
        self._lib.kvq_radix_release(self._h, _i32(block_table), len(block_table))

    def clear_cache(self) -> None:
        self._lib.kvq_radix_clear(self._h)

    def stats(self) -> dict:
        info = _lib.RadixInfo()
        self._lib.kvq_radix_stats(self._h, ctypes.byref(info))
        return {name: getattr(info, name) for name, _ in _lib.RadixInfo._fields_}


class PagedRadixKVCache:
    """Quantized K/V pools of `num_layers` layers in pages of 64 tokens, with a radix prefix cache."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, max_blocks: int = 1024, *, bits: int = 8,
                 group_size: int = 64, dtype: torch.dtype = torch.float16, device="cuda") -> None:
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8 (the attention kernels' formats), got {bits}")
        self.num_layers, self.num_kv_heads, self.head_dim = num_layers, num_kv_heads, head_dim
        self.bits, self.group_size, self.dtype = bits, group_size, dtype
        self.radix = PageRadix(max_blocks, PAGE_ROWS)
        W, G = head_dim * bits // 32, head_dim // group_size

        def pool():
            codes = torch.zeros((max_blocks, num_kv_heads, PAGE_ROWS, W), dtype=torch.int32, device=device)
            scales = torch.zeros((max_blocks, num_kv_heads, PAGE_ROWS, G), dtype=dtype, device=device)
            codes = codes.view(torch.uint32)
            # the pool's range exponent: raised by the paged appends, read by the paged prefill
            kernels.register_range_word(codes, torch.zeros(1, dtype=torch.int32, device=device))
            return codes, scales, torch.zeros_like(scales)

        self._k = [pool() for _ in range(num_layers)]
        self._v = [pool() for _ in range(num_layers)]

    # ---- the reference's interface (native/include/kv_cache.hpp:28-54)

    @property
    def block_size(self) -> int:
        return PAGE_ROWS

    @property
    def max_blocks(self) -> int:
        return self.radix.num_pages

    def match_and_allocate(self, prompt_tokens: Sequence[int], max_new_tokens: int) -> PrefixMatchResult:
        return self.radix.match_and_allocate(prompt_tokens, max_new_tokens)

    def commit_prefix_blocks(self, tokens: Sequence[int], block_table: Sequence[int], valid_token_count: int) -> None:
        self.radix.commit_prefix_blocks(tokens, block_table, valid_token_count)

    def release(self, block_table: Sequence[int]) -> None:
        """Drop a finished sequence's hold on its pages (cached ones stay matchable until evicted)."""
        self.radix.release(block_table)

    def clear_cache(self) -> None:
        self.radix.clear_cache()

    def k_cache(self, layer: int):
        return self._k[layer]

    def v_cache(self, layer: int):
        return self._v[layer]

    @property
    def cached_prefix_blocks(self) -> int:
        return self.radix.stats()["cached_pages"]

    @property
    def total_prefix_hits(self) -> int:
        return self.radix.stats()["prefix_hit_tokens"]

    @property
    def total_prompt_tokens(self) -> int:
        return self.radix.stats()["prompt_tokens"]

    @property
    def kv_memory_bytes(self) -> int:
        return sum(x.nbytes for tr in self._k + self._v for x in tr)

    # ---- device work

    def tables(self, block_tables: Sequence[Sequence[int]], device=None) -> torch.Tensor:
        """int32 [B, max pages] device tensor of per-sequence page lists (short rows padded with
        their last page)."""
        width = max(len(t) for t in block_tables)
        rows = [list(t) + [t[-1]] * (width - len(t)) for t in block_tables]
        return torch.tensor(rows, dtype=torch.int32, device=device or self._k[0][0].device)

    def append(self, layer: int, keys: torch.Tensor, values: torch.Tensor, block_tables: torch.Tensor, *,
               starts: Optional[torch.Tensor] = None, row_offset: int = 0,
               rope: Optional[kernels.Rope] = None) -> None:
        """Quantize keys/values [B, Hkv, L, D] into the layer's pages (fused, one launch)."""
        kernels.paged_quantize_append(keys, self._k[layer], values, self._v[layer], block_tables, starts=starts,
                                      row_offset=row_offset, group_size=self.group_size, bits=self.bits, rope=rope)

    def attention(self, layer: int, queries: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
                  scale: float, *, causal: bool = False, window: int = 0, max_len: Optional[int] = None,
                  kernel: str = "auto") -> torch.Tensor:
        return kernels.paged_attention(queries, self._k[layer], self._v[layer], block_tables, seq_lens, scale,
                                       causal=causal, window=window, group_size=self.group_size, bits=self.bits,
                                       max_len=max_len, kernel=kernel)

    def gather(self, layer: int, block_table: Sequence[int], length: int):
        """The first `length` rows of one sequence as contiguous [1, Hkv, length, *] triples (K, V)."""
        idx = torch.tensor(list(block_table), dtype=torch.long, device=self._k[0][0].device)

        def one(pool):
            out = []
            for x in pool:
                y = x.view(torch.int32) if x.dtype == torch.uint32 else x
                g = y.index_select(0, idx).transpose(0, 1).reshape(1, self.num_kv_heads, -1, x.shape[-1])[:, :, :length]
                g = g.contiguous()
                out.append(g.view(torch.uint32) if x.dtype == torch.uint32 else g)
            return tuple(out)

        return one(self._k[layer]), one(self._v[layer])
