"""Model of the paged radix prefix cache (myinfer_amd/csrc/radix.cpp). TEST INFRASTRUCTURE ONLY.

Follows the reference's PagedRadixKVCache (native/src/kv_cache.cpp:73-157,
native/include/kv_cache.hpp:17-77):
  * match_and_allocate (kv_cache.cpp:76-133): pages for prompt + max_new + 16 tokens, capped at the
    pool; full prompt pages are matched in order while the prefix is cached with exactly the same
    tokens, never the last prompt token; the rest are free pages, else the least recently used
    cached pages (kv_cache.cpp:42-72); an exhausted pool is an error;
  * commit_prefix_blocks (kv_cache.cpp:136-160): full pages of the valid tokens become cached
    under their prefix;
  * clear_cache (kv_cache.cpp:162-170).
Keys here are the exact token prefixes (tuples), which is what the reference's chained hash plus
token verification decides. The C++ code adds, and this model restates: page reference counts
(held pages are never evicted; release drops a hold), a free list whose top is the lowest free
page at start and then the most recently freed one, eviction by the oldest access tick, and a
duplicate commit keeping the page that is already cached.
"""

from __future__ import annotations


class RadixModel:
    def __init__(self, num_pages: int, page_tokens: int) -> None:
        self.num_pages, self.P = num_pages, page_tokens
        self.clock = 0
        self.refs = [0] * num_pages
        self.tick = [0] * num_pages
        self.key = [None] * num_pages  # the cached prefix (a tuple of tokens), or None
        self.index: dict = {}  # prefix -> page
        self.free = list(range(num_pages - 1, -1, -1))  # stack: pop() gives the next free page
        self.hits = 0
        self.prompts = 0

    def _touch(self, p: int) -> None:
        self.clock += 1
        self.tick[p] = self.clock

    def _evictable(self):
        return [p for p in range(self.num_pages) if self.key[p] is not None and self.refs[p] == 0]

    def _take(self):
        if self.free:
            p = self.free.pop()
        else:
            ev = self._evictable()
            if not ev:
                return None
            p = min(ev, key=lambda q: self.tick[q])
            self._uncache(p)
        self.refs[p] = 1
        self._touch(p)
        return p

    def _uncache(self, p: int) -> None:
        k = self.key[p]
        if k is not None and self.index.get(k) == p:
            del self.index[k]
        self.key[p] = None

    def _drop(self, p: int) -> None:
        if self.refs[p] <= 0:
            return
        self.refs[p] -= 1
        if self.refs[p] == 0 and self.key[p] is None:
            self.free.append(p)

    def match_and_allocate(self, tokens, max_new: int):
        P = self.P
        need = min((len(tokens) + max_new + 16 + P - 1) // P, self.num_pages)
        self.prompts += len(tokens)
        max_match = (len(tokens) - 1) // P if len(tokens) > 1 else 0
        table = []
        for blk in range(min(max_match, need)):
            prefix = tuple(tokens[: (blk + 1) * P])
            p = self.index.get(prefix)
            if p is None:
                break
            self.refs[p] += 1
            self._touch(p)
            table.append(p)
        got = len(table)
        while len(table) < need:
            p = self._take()
            if p is None:
                for q in table:
                    self._drop(q)
                return None
            table.append(p)
        self.hits += got * P
        return table, got * P

    def commit(self, tokens, table, valid: int) -> None:
        P = self.P
        for blk in range(min(valid // P, len(table))):
            p = table[blk]
            assert self.refs[p] > 0, "commit of a page the caller does not hold"
            prefix = tuple(tokens[: (blk + 1) * P])
            if self.key[p] == prefix:
                self._touch(p)
            elif prefix not in self.index:
                self._uncache(p)
                self.key[p] = prefix
                self.index[prefix] = p
                self._touch(p)

    def release(self, table) -> None:
        for p in table:
            self._drop(p)

    def clear(self) -> None:
        self.index.clear()
        self.key = [None] * self.num_pages
        self.tick = [0] * self.num_pages
        self.free = [p for p in range(self.num_pages - 1, -1, -1) if self.refs[p] == 0]

    def stats(self):
        return dict(cached_pages=len(self.index), free_pages=len(self.free),
                    in_use_pages=sum(r > 0 for r in self.refs), prefix_hit_tokens=self.hits,
                    prompt_tokens=self.prompts)
