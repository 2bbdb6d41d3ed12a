// Paged radix prefix cache, host side: which pages of a KV pool hold which token prefixes.
//
// Counterpart of the reference's PagedRadixKVCache (native/src/kv_cache.cpp:73-157,
// native/include/kv_cache.hpp): the pool is cut into pages of P tokens; a full page is keyed by a
// 64-bit hash chained over its tokens and its parent page's key; a new prompt walks its full pages
// while the chain hits and the stored tokens match exactly, and reuses those pages; the rest of the
// sequence gets free pages, or evicts the least recently used cached ones.
//
// Differences from the reference, on purpose:
//  * pages carry reference counts: a page held by a running sequence is never evicted or re-keyed
//    by another sequence's allocation, and kvq_radix_release drops the hold (the reference pins
//    only within one call, which serves its one-request-at-a-time engine);
//  * free pages and evictable cached pages sit in a free list and an LRU-ordered set, so
//    allocation costs O(log pages) instead of a scan of the pool (pools of 10^5 pages fit in HBM);
//  * committing content that another page already caches keeps the cached page (the reference
//    re-points the key, leaving the old page keyed but unreachable);
//  * the page size is a parameter (64 tokens for the MI355X kernels, whose 64-key tiles then
//    read one page each).
// The hash is this file's own (a splitmix64-style mix); keys are internal, never stored.

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <new>
#include <set>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/kvq.h"

namespace {

thread_local char g_radix_err[256] = "";

struct Page {
  uint64_t key = 0;
  uint64_t tick = 0;
  int32_t refs = 0;
  bool cached = false;
  std::vector<int32_t> tokens;  // the page's tokens, for exact verification
};

uint64_t mix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

}  // namespace

struct kvq_radix {
  int num_pages = 0, page_tokens = 0;
  uint64_t clock = 0, hit_tokens = 0, prompt_tokens = 0;
  std::vector<Page> pages;
  std::unordered_map<uint64_t, int32_t> index;  // key -> cached page
  std::vector<int32_t> free_list;               // uncached, unreferenced (lowest index on top)
  std::set<std::pair<uint64_t, int32_t>> lru;   // (tick, page) of cached, unreferenced pages

  uint64_t page_key(uint64_t parent, const int32_t* toks) const {
    uint64_t h = mix64(parent ^ 0x6b76715f72616478ull);
    for (int i = 0; i < page_tokens; ++i) h = mix64(h ^ (uint64_t)(uint32_t)toks[i]);
    return h;
  }
  bool same_tokens(const Page& pg, const int32_t* toks) const {
    return (int)pg.tokens.size() == page_tokens && memcmp(pg.tokens.data(), toks, sizeof(int32_t) * page_tokens) == 0;
  }
  void hold(int32_t p) {
    Page& pg = pages[p];
    if (pg.refs == 0 && pg.cached) lru.erase({pg.tick, p});
    pg.refs++;
    pg.tick = ++clock;
  }
  void drop(int32_t p) {
    Page& pg = pages[p];
    if (pg.refs <= 0) return;
    if (--pg.refs == 0) {
      if (pg.cached)
        lru.insert({pg.tick, p});
      else
        free_list.push_back(p);
    }
  }
  void uncache(int32_t p) {
    Page& pg = pages[p];
    auto it = index.find(pg.key);
    if (it != index.end() && it->second == p) index.erase(it);
    pg.cached = false;
    pg.tokens.clear();
    pg.key = 0;
  }
  // an unreferenced page for a new sequence: a free one, else the least recently used cached one
  int32_t take() {
    int32_t p = -1;
    if (!free_list.empty()) {
      p = free_list.back();
      free_list.pop_back();
    } else if (!lru.empty()) {
      p = lru.begin()->second;
      lru.erase(lru.begin());
      uncache(p);
    } else {
      return -1;
    }
    pages[p].refs = 1;
    pages[p].tick = ++clock;
    return p;
  }
};

extern "C" {

const char* kvq_radix_last_error(void) { return g_radix_err; }

kvq_radix* kvq_radix_create(int num_pages, int page_tokens) {
  if (num_pages <= 0 || page_tokens <= 0) {
    snprintf(g_radix_err, sizeof(g_radix_err), "num_pages and page_tokens must be positive (%d, %d)", num_pages,
             page_tokens);
    return nullptr;
  }
  kvq_radix* r = new (std::nothrow) kvq_radix;
  if (!r) return nullptr;
  r->num_pages = num_pages;
  r->page_tokens = page_tokens;
  r->pages.resize(num_pages);
  r->free_list.reserve(num_pages);
  for (int32_t p = num_pages - 1; p >= 0; --p) r->free_list.push_back(p);
  g_radix_err[0] = '\0';
  return r;
}

void kvq_radix_destroy(kvq_radix* r) { delete r; }

int kvq_radix_match_and_allocate(kvq_radix* r, const int32_t* tokens, int n_tokens, int max_new_tokens,
                                 int32_t* table, int table_capacity, int* matched_tokens, int* n_pages) {
  if (!r || (!tokens && n_tokens > 0) || !table || !matched_tokens || !n_pages || n_tokens < 0 || max_new_tokens < 0) {
    snprintf(g_radix_err, sizeof(g_radix_err), "bad argument");
    return KVQ_ERR_INVALID;
  }
  const int P = r->page_tokens;
  // the prompt, the new tokens and a margin of 16 (speculative tokens), as kv_cache.cpp:84-88
  int64_t need = ((int64_t)n_tokens + max_new_tokens + 16 + P - 1) / P;
  if (need > r->num_pages) need = r->num_pages;
  if (need > table_capacity) {
    snprintf(g_radix_err, sizeof(g_radix_err), "table capacity %d < %lld pages", table_capacity, (long long)need);
    return KVQ_ERR_INVALID;
  }
  r->prompt_tokens += (uint64_t)n_tokens;
  // full pages that may match, always leaving the last prompt token to be computed
  const int max_match = n_tokens > 1 ? (n_tokens - 1) / P : 0;
  uint64_t parent = 0;
  int got = 0;
  for (int blk = 0; blk < max_match && blk < need; ++blk) {
    const int32_t* t = tokens + (int64_t)blk * P;
    const uint64_t key = r->page_key(parent, t);
    auto it = r->index.find(key);
    if (it == r->index.end() || !r->same_tokens(r->pages[it->second], t)) break;
    r->hold(it->second);
    table[blk] = it->second;
    parent = key;
    got++;
  }
  for (int blk = got; blk < need; ++blk) {
    const int32_t p = r->take();
    if (p < 0) {
      for (int b2 = 0; b2 < blk; ++b2) r->drop(table[b2]);
      snprintf(g_radix_err, sizeof(g_radix_err), "out of KV pages: %lld needed, the pool holds %d", (long long)need,
               r->num_pages);
      return KVQ_ERR_CAPACITY;
    }
    table[blk] = p;
  }
  *matched_tokens = got * P;
  *n_pages = (int)need;
  r->hit_tokens += (uint64_t)got * P;
  g_radix_err[0] = '\0';
  return KVQ_OK;
}

int kvq_radix_commit(kvq_radix* r, const int32_t* tokens, int n_tokens, const int32_t* table, int n_pages,
                     int valid_tokens) {
  if (!r || (!tokens && n_tokens > 0) || (!table && n_pages > 0) || valid_tokens < 0 || valid_tokens > n_tokens) {
    snprintf(g_radix_err, sizeof(g_radix_err), "bad argument");
    return KVQ_ERR_INVALID;
  }
  const int P = r->page_tokens;
  const int full = valid_tokens / P;
  uint64_t parent = 0;
  for (int blk = 0; blk < full && blk < n_pages; ++blk) {
    const int32_t p = table[blk];
    if (p < 0 || p >= r->num_pages) {
      snprintf(g_radix_err, sizeof(g_radix_err), "page %d out of range", p);
      return KVQ_ERR_INVALID;
    }
    Page& pg = r->pages[p];
    if (pg.refs == 0) {
      snprintf(g_radix_err, sizeof(g_radix_err), "page %d is not held by the caller", p);
      return KVQ_ERR_INVALID;
    }
    const int32_t* t = tokens + (int64_t)blk * P;
    const uint64_t key = r->page_key(parent, t);
    if (pg.cached && pg.key == key) {
      pg.tick = ++r->clock;
    } else if (r->index.count(key) == 0) {
      if (pg.cached) r->uncache(p);  // held, so not in the LRU set
      pg.key = key;
      pg.tokens.assign(t, t + P);
      pg.cached = true;
      pg.tick = ++r->clock;
      r->index[key] = p;
    }  // else: another page caches this content already; it stays the cached copy
    parent = key;
  }
  g_radix_err[0] = '\0';
  return KVQ_OK;
}

int kvq_radix_release(kvq_radix* r, const int32_t* table, int n_pages) {
  if (!r || (!table && n_pages > 0)) return KVQ_ERR_INVALID;
  for (int i = 0; i < n_pages; ++i)
    if (table[i] >= 0 && table[i] < r->num_pages) r->drop(table[i]);
  return KVQ_OK;
}

void kvq_radix_clear(kvq_radix* r) {
  if (!r) return;
  r->index.clear();
  r->lru.clear();
  r->free_list.clear();
  for (int32_t p = r->num_pages - 1; p >= 0; --p) {
    Page& pg = r->pages[p];
    pg.cached = false;
    pg.tokens.clear();
    pg.key = 0;
    pg.tick = 0;
    if (pg.refs == 0) r->free_list.push_back(p);
  }
}

int kvq_radix_stats(const kvq_radix* r, kvq_radix_info* out) {
  if (!r || !out) return KVQ_ERR_INVALID;
  int in_use = 0;
  for (const Page& pg : r->pages) in_use += pg.refs > 0;
  out->num_pages = r->num_pages;
  out->page_tokens = r->page_tokens;
  out->cached_pages = (int)r->index.size();
  out->free_pages = (int)r->free_list.size();
  out->in_use_pages = in_use;
  out->prefix_hit_tokens = (int64_t)r->hit_tokens;
  out->prompt_tokens = (int64_t)r->prompt_tokens;
  return KVQ_OK;
}

}  // extern "C"
