"""GPU paged pools: the quantize-append into 64-row pages, and decode / prefill attention through
block tables, against the contiguous kernels (bit-identical: same rows, same tiles, same split
plan) and the exact fp64 oracle; and prefix sharing through the radix cache.

Pages are handed out in a shuffled order, and every row of the pools that no sequence writes
holds NaN scales and biases, so reading a row past a sequence's end, or a page that is not in
its table, shows up as a non-finite output.
"""

import math

import pytest
import torch

from myinfer_amd import kernels
from myinfer_amd.paged import PAGE_ROWS, PagedRadixKVCache
from tests.helpers import assert_close, exact_reference, seeded_normal

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAN_BITS = {torch.float16: 0x7E00, torch.bfloat16: 0x7FC0}


def poisoned_pool(npages, H, D, bits, dtype, group=64):
    codes = torch.randint(0, 2**31 - 1, (npages, H, PAGE_ROWS, D * bits // 32), dtype=torch.int32, device=DEV)
    sc = torch.full((npages, H, PAGE_ROWS, D // group), NAN_BITS[dtype], dtype=torch.int16, device=DEV).view(dtype)
    return codes.view(torch.uint32), sc, sc.clone()


def page_tables(lens, npages, seed):
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(npages, generator=g).tolist()
    width = max(math.ceil(n / PAGE_ROWS) for n in lens)
    rows, k = [], 0
    for n in lens:
        need = math.ceil(n / PAGE_ROWS)
        row = perm[k:k + need]
        k += need
        rows.append(row + [row[-1]] * (width - need))
    return rows, torch.tensor(rows, dtype=torch.int32, device=DEV)


def build(B, Hkv, lens, D, bits, dtype, seed, npages=None, group=64):
    """Paged pools and the equivalent contiguous caches (quantized by the same kernel)."""
    S = max(lens)
    npages = npages or sum(math.ceil(n / PAGE_ROWS) for n in lens) + 7
    rows, tables = page_tables(lens, npages, seed)
    kp, vp = poisoned_pool(npages, Hkv, D, bits, dtype, group), poisoned_pool(npages, Hkv, D, bits, dtype, group)
    k = seeded_normal((B, Hkv, S, D), seed, dtype, DEV)
    v = seeded_normal((B, Hkv, S, D), seed + 1, dtype, DEV)
    # append in two uneven pieces per sequence, as a prefill chunk and then decode steps would
    cut = [n // 3 for n in lens]
    for b in range(B):
        kb, vb = k[b:b + 1], v[b:b + 1]
        t = tables[b:b + 1]
        kernels.paged_quantize_append(kb[:, :, :cut[b]], kp, vb[:, :, :cut[b]], vp, t, row_offset=0, bits=bits,
                                      group_size=group)
        if lens[b] > cut[b]:
            st = torch.full((1,), cut[b], dtype=torch.int32, device=DEV)
            kernels.paged_quantize_append(kb[:, :, cut[b]:lens[b]], kp, vb[:, :, cut[b]:lens[b]], vp, t, starts=st,
                                          bits=bits, group_size=group)
    kc = [torch.zeros((B, Hkv, S, D * bits // 32), dtype=torch.int32, device=DEV).view(torch.uint32),
          torch.zeros((B, Hkv, S, D // group), dtype=dtype, device=DEV),
          torch.zeros((B, Hkv, S, D // group), dtype=dtype, device=DEV)]
    vc = [x.clone() for x in kc]
    kernels.quantize_append(k, kc, v, vc, row_offset=0, bits=bits, group_size=group)
    return rows, tables, kp, vp, tuple(kc), tuple(vc)


def test_paged_append_bit_exact():
    print("paged append", flush=True)
    B, Hkv, D, bits, dtype = 3, 4, 128, 8, torch.bfloat16
    lens = [300, 64, 129]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 5)
    for b in range(B):
        for pool, cont in ((kp, kc), (vp, vc)):
            idx = torch.tensor(rows[b], dtype=torch.long, device=DEV)
            for x, y in zip(pool, cont):
                xi = x.view(torch.int32) if x.dtype == torch.uint32 else x.view(torch.int16)
                yi = y.view(torch.int32) if y.dtype == torch.uint32 else y.view(torch.int16)
                g = xi.index_select(0, idx).transpose(0, 1).reshape(Hkv, -1, x.shape[-1])[:, :lens[b]]
                assert torch.equal(g, yi[b, :, :lens[b]])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [8, 4])
def test_paged_decode_equals_contiguous(dtype, bits):
    print(f"paged decode {dtype} bits={bits}", flush=True)
    B, Hq, Hkv, D = 3, 32, 8, 128
    lens = [5000, 777, 64]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 11)
    q = seeded_normal((B, Hq, 1, D), 12, dtype, DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    S = max(lens)
    out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, bits=bits, max_len=S, kernel="decode")
    out_c = kernels.attention(q, kc, vc, scale, seq_lens=sl, bits=bits, kernel="decode")
    torch.cuda.synchronize()
    assert torch.isfinite(out_p.float()).all(), "a row past a sequence's end was read"
    assert torch.equal(out_p, out_c)
    assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, seq_lens=sl), "paged decode")


@pytest.mark.parametrize("D", [64, 128])
def test_paged_decode_window_and_multirow(D):
    print(f"paged decode window D={D}", flush=True)
    B, Hq, Hkv, L = 2, 8, 2, 3
    dtype, bits = torch.float16, 8
    lens = [2000, 1500]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 21)
    q = seeded_normal((B, Hq, L, D), 22, dtype, DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, causal=True, window=333, bits=bits,
                                    max_len=max(lens), kernel="decode")
    out_c = kernels.attention(q, kc, vc, scale, causal=True, window=333, seq_lens=sl, bits=bits, kernel="decode")
    torch.cuda.synchronize()
    assert torch.equal(out_p, out_c)
    assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, causal=True, window=333, seq_lens=sl),
                 "paged decode window")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paged_prefill_equals_contiguous(dtype):
    print(f"paged prefill {dtype}", flush=True)
    B, Hq, Hkv, D, bits, L = 2, 16, 4, 128, 8, 300
    lens = [3000, 1211]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 31)
    q = seeded_normal((B, Hq, L, D), 32, dtype, DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    for causal, window in ((True, 0), (True, 700), (False, 0)):
        out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, causal=causal, window=window, bits=bits,
                                        max_len=max(lens), kernel="prefill")
        out_c = kernels.attention(q, kc, vc, scale, causal=causal, window=window, seq_lens=sl, bits=bits,
                                  kernel="prefill")
        torch.cuda.synchronize()
        assert torch.isfinite(out_p.float()).all()
        assert torch.equal(out_p, out_c), (causal, window)
        assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, causal=causal, window=window, seq_lens=sl),
                     f"paged prefill causal={causal} window={window}")


def test_paged_rope_append_matches_contiguous():
    print("paged rope append", flush=True)
    B, H, D, L = 2, 4, 128, 70
    r = kernels.Rope(128, False, 1000000.0)
    k = seeded_normal((B, H, L, D), 41, torch.bfloat16, DEV)
    v = seeded_normal((B, H, L, D), 42, torch.bfloat16, DEV)
    starts = torch.tensor([100, 7], dtype=torch.int32, device=DEV)
    rows, tables = page_tables([170, 77], 8, 43)
    kp, vp = poisoned_pool(8, H, D, 8, torch.bfloat16), poisoned_pool(8, H, D, 8, torch.bfloat16)
    kernels.paged_quantize_append(k, kp, v, vp, tables, starts=starts, rope=r)
    torch.cuda.synchronize()
    for b, st in enumerate((100, 7)):
        kc = [torch.zeros((1, H, st + L, 32), dtype=torch.int32, device=DEV).view(torch.uint32),
              torch.zeros((1, H, st + L, 2), dtype=torch.bfloat16, device=DEV),
              torch.zeros((1, H, st + L, 2), dtype=torch.bfloat16, device=DEV)]
        kernels.quantize_append(k[b:b + 1], kc, row_offset=st, rope=r)
        idx = torch.tensor(rows[b], dtype=torch.long, device=DEV)
        for x, y in zip(kp, kc):
            xi = x.view(torch.int32) if x.dtype == torch.uint32 else x.view(torch.int16)
            yi = y.view(torch.int32) if y.dtype == torch.uint32 else y.view(torch.int16)
            g = xi.index_select(0, idx).transpose(0, 1).reshape(H, -1, x.shape[-1])[:, st:st + L]
            assert torch.equal(g, yi[0, :, st:st + L])


def test_prefix_sharing_through_the_radix():
    print("paged radix prefix sharing", flush=True)
    Hq, Hkv, D, dtype = 16, 4, 128, torch.float16
    cache = PagedRadixKVCache(1, Hkv, D, max_blocks=64, bits=8, dtype=dtype)
    prompt_a = list(range(1000, 1000 + 700))
    prompt_b = prompt_a[:520] + list(range(5000, 5100))  # shares 8 full pages (512 tokens)
    k_all = seeded_normal((1, Hkv, 1200, D), 51, dtype, DEV)
    v_all = seeded_normal((1, Hkv, 1200, D), 52, dtype, DEV)
    # keys/values of a token depend only on the prefix here: B's first 520 rows are A's
    kb_rows = torch.cat([k_all[:, :, :520], k_all[:, :, 700:800]], dim=2)
    vb_rows = torch.cat([v_all[:, :, :520], v_all[:, :, 700:800]], dim=2)

    ma = cache.match_and_allocate(prompt_a, 16)
    assert ma.matched_tokens == 0
    ta = cache.tables([ma.block_table])
    cache.append(0, k_all[:, :, :700], v_all[:, :, :700], ta)
    cache.commit_prefix_blocks(prompt_a, ma.block_table, 700)
    cache.release(ma.block_table)

    mb = cache.match_and_allocate(prompt_b, 16)
    assert mb.matched_tokens == 512 and mb.block_table[:8] == ma.block_table[:8]
    tb = cache.tables([mb.block_table])
    m = mb.matched_tokens
    cache.append(0, kb_rows[:, :, m:].contiguous(), vb_rows[:, :, m:].contiguous(), tb, row_offset=m)
    q = seeded_normal((1, Hq, 1, D), 53, dtype, DEV)
    sl = torch.tensor([620], dtype=torch.int32, device=DEV)
    out = cache.attention(0, q, tb, sl, 1.0 / math.sqrt(D), max_len=620)
    kc = kernels.quantize(kb_rows, bits=8)
    vc = kernels.quantize(vb_rows, bits=8)
    ref = kernels.attention(q, kc, vc, 1.0 / math.sqrt(D), bits=8)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    gk, gv = cache.gather(0, mb.block_table, 620)
    for x, y in zip(gk, kc):
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.uint32 else x,
                           y.view(torch.int32) if y.dtype == torch.uint32 else y)
    assert cache.total_prefix_hits == 512 and cache.cached_prefix_blocks == 10
    assert cache.kv_memory_bytes == 2 * 64 * Hkv * 64 * (128 + 2 * 2 * 2)  # K and V: codes, scales, biases


@pytest.mark.parametrize("group", [32, 128])
@pytest.mark.parametrize("bits", [8, 4])
def test_paged_group_sizes(group, bits):
    print(f"paged group={group} bits={bits}", flush=True)
    B, Hq, Hkv, D, dtype = 2, 16, 4, 128, torch.bfloat16
    lens = [2100, 517]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 41 + group, group=group)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    for L, kernel in ((1, "decode"), (2, "decode"), (120, "prefill")):
        q = seeded_normal((B, Hq, L, D), 42 + L, dtype, DEV)
        out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, causal=True, bits=bits, group_size=group,
                                        max_len=max(lens), kernel=kernel)
        out_c = kernels.attention(q, kc, vc, scale, causal=True, seq_lens=sl, bits=bits, group_size=group,
                                  kernel=kernel)
        torch.cuda.synchronize()
        assert torch.isfinite(out_p.float()).all()
        assert torch.equal(out_p, out_c), (L, kernel)
        assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, group_size=group, causal=True, seq_lens=sl),
                     f"paged {kernel} group={group}")


@pytest.mark.parametrize("bits", [8, 4])
def test_paged_head_dim_256(bits):
    print(f"paged D=256 bits={bits}", flush=True)
    B, Hq, Hkv, D, dtype = 2, 8, 2, 256, torch.float16
    lens = [1500, 333]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 51, group=64)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    for L in (1, 3, 200):
        q = seeded_normal((B, Hq, L, D), 52 + L, dtype, DEV)
        out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, causal=True, bits=bits, group_size=64,
                                        max_len=max(lens))
        # L = 1 runs the decode kernel, L = 3 and 200 the head_dim-256 prefill kernel, on both layouts
        out_c = kernels.attention(q, kc, vc, scale, causal=True, seq_lens=sl, bits=bits, group_size=64)
        torch.cuda.synchronize()
        assert torch.isfinite(out_p.float()).all()
        assert torch.equal(out_p, out_c), L
        assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, group_size=64, causal=True, seq_lens=sl),
                     f"paged D=256 L={L}")


@pytest.mark.parametrize("bits,group", [(8, 64), (4, 32)])
def test_paged_prefill_head_dim_64(bits, group):
    print(f"paged prefill D=64 bits={bits} group={group}", flush=True)
    B, Hq, Hkv, D, L, dtype = 2, 16, 4, 64, 200, torch.bfloat16
    lens = [2500, 901]
    rows, tables, kp, vp, kc, vc = build(B, Hkv, lens, D, bits, dtype, 61, group=group)
    q = seeded_normal((B, Hq, L, D), 62, dtype, DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out_p = kernels.paged_attention(q, kp, vp, tables, sl, scale, causal=True, bits=bits, group_size=group,
                                    max_len=max(lens), kernel="prefill")
    out_c = kernels.attention(q, kc, vc, scale, causal=True, seq_lens=sl, bits=bits, group_size=group,
                              kernel="prefill")
    torch.cuda.synchronize()
    assert torch.isfinite(out_p.float()).all()
    assert torch.equal(out_p, out_c)
    assert_close(out_p, exact_reference(q, kc, vc, scale, bits=bits, group_size=group, causal=True, seq_lens=sl),
                 "paged prefill D=64")


@pytest.mark.parametrize("D,L,kernel", [(128, 1, "decode"), (128, 40, "prefill"), (256, 20, "prefill")])
def test_paged_short_and_empty_sequences(D, L, kernel):
    """Paged pools with one sequence shorter than the chunk (its first rows at negative causal
    positions) and one with no keys at all: those rows come out 0, the pools' poisoned rows are
    never read, and the result equals the contiguous call's bit for bit."""
    print(f"paged short/empty sequences D={D} L={L} {kernel}", flush=True)
    B, Hq, Hkv, bits, dtype = 3, 8, 2, 8, torch.float16
    rows, tables, kp, vp, kc, vc = build(B, Hkv, [700, 64, 64], D, bits, dtype, 41)
    lens = [700, L // 2, 0]
    q = seeded_normal((B, Hq, L, D), 42, dtype, DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out_p = kernels.paged_attention(q, kp, vp, tables, sl, 0.1, causal=True, bits=bits, max_len=700, kernel=kernel)
    out_c = kernels.attention(q, kc, vc, 0.1, causal=True, seq_lens=sl, bits=bits, kernel=kernel)
    torch.cuda.synchronize()
    assert torch.isfinite(out_p.float()).all()
    assert torch.all(out_p[2] == 0) and torch.all(out_p[1, :, :L - lens[1]] == 0)
    assert torch.equal(out_p, out_c)
    assert_close(out_p, exact_reference(q, kc, vc, 0.1, bits=bits, causal=True, seq_lens=sl), "paged short/empty")
