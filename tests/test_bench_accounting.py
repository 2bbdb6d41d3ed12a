"""The bench's accounting, without a GPU: the algorithmic FLOP and byte counts that its roofline
fractions divide by, checked against brute-force counts on small shapes and against the figures
the headline configurations are quoted with, and the committed traffic summary it reads."""

import bench


def _pairs_brute(L0, L1, window):
    # unmasked (query, key) pairs: query position p sees keys k <= p, and k > p - window if set
    n = 0
    for p in range(L0, L1):
        for k in range(p + 1):
            if window <= 0 or k > p - window:
                n += 1
    return n


def test_prefill_flops_counts_unmasked_pairs():
    for L0, L1, window in [(0, 64, 0), (0, 97, 0), (40, 97, 0), (0, 64, 16), (30, 130, 33), (5, 6, 0)]:
        for Hq, D, B in [(1, 1, 1), (8, 128, 2)]:
            want = 4 * D * Hq * B * _pairs_brute(L0, L1, window)
            assert bench.prefill_flops(L1, Hq, D, L0, L1, window=window, B=B) == want


def test_prefill_flops_headline():
    # C3: a 16384-token causal prompt, 32 query heads of 128 dims: N (N + 1) / 2 pairs
    assert bench.prefill_flops(16384, 32, 128) == 4 * 128 * 32 * 16384 * 16385 // 2 == 2199157473280
    # the chunks of the prompt add up to the whole
    total = sum(bench.prefill_flops(16384, 32, 128, c * 512, (c + 1) * 512) for c in range(32))
    assert total == bench.prefill_flops(16384, 32, 128)


def test_decode_bytes():
    # 8 bits, D = 128, G = 64: 128 code bytes + 2 groups x (scale + bias) x 2 bytes = 136 B per row,
    # K and V; plus the fp16 query in and output out
    assert bench.decode_bytes([32768], 64, 8, 128, 8) == 32768 * 8 * 2 * 136 + 2 * 64 * 128 * 2 == 71335936
    # 4 bits: 64 + 8 = 72 B per row
    assert bench.decode_bytes([131072], 64, 8, 128, 4) == 131072 * 8 * 2 * 72 + 2 * 64 * 128 * 2
    # group 32 doubles the scale/bias bytes; unquantized rows are D * 2 bytes
    assert bench.decode_bytes([100], 8, 2, 128, 8, G=32) == 100 * 2 * 2 * (128 + 16) + 2 * 8 * 128 * 2
    assert bench.decode_bytes([1024] * 4, 32, 16, 128, 16) == 4 * 1024 * 16 * 2 * 256 + 2 * 4 * 32 * 128 * 2
    # ragged batch and a sliding window: only the keys a query can see count
    assert bench.decode_bytes([10, 2000, 700], 4, 1, 64, 8, window=1024) == (10 + 1024 + 700) * 2 * (64 + 4) + 2 * 3 * 4 * 64 * 2


def test_measured_traffic_reads_the_committed_summary():
    decode = bench.measured_traffic("decode_c2_b1")
    prefill = bench.measured_traffic("prefill_c3_chunk")
    assert decode is not None and prefill is not None
    # the cache is read once: within a few percent of the algorithmic bytes
    assert 1.0 <= decode / bench.decode_bytes([32768], 64, 8, 128, 8) < 1.1
    assert bench.measured_traffic("no_such_kernel") is None


def test_tail_parity_judges_the_last_rows():
    # the bench's parity record of a prefill shape: an output formed by the oracle itself is within
    # the bar, and one whose last rows are perturbed by 1% fails it; rows before the checked tail
    # are not looked at
    import numpy as np
    import torch

    from oracle import attention as OA

    g = torch.Generator().manual_seed(5)
    q = torch.randn((1, 4, 40, 64), generator=g).to(torch.float16)
    k = torch.randn((1, 2, 90, 64), generator=g).to(torch.float16)
    v = torch.randn((1, 2, 90, 64), generator=g).to(torch.float16)
    ref = OA.exact_attention(q.double().numpy(), k.double().numpy(), v.double().numpy(), 0.125, causal=True, window=30)
    out = torch.from_numpy(ref).to(torch.float16)
    rec = bench.tail_parity(q, k, v, out, 0.125, rows=16, window=30)
    assert rec["within_bar"] and rec["rows"] == "last 16 of 40 queries"
    bad = out.clone()
    bad[:, :, :24] = 7.0  # outside the checked tail
    assert bench.tail_parity(q, k, v, bad, 0.125, rows=16, window=30)["within_bar"]
    bad[:, :, -1] *= 1.01
    assert not bench.tail_parity(q, k, v, bad, 0.125, rows=16, window=30)["within_bar"]
    # a window the oracle is not told about changes the reference: the record catches it
    assert not bench.tail_parity(q, k, v, out, 0.125, rows=16)["within_bar"]
    assert np.isfinite(rec["max_abs"])
