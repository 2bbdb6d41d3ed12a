"""Pins oracle.cache.CacheModel (mlx-lm 0.31.3's KVCache / QuantizedKVCache bookkeeping) with
capacities derived by hand from the published growth rule, not from a second restatement:

  an update of L rows at offset `prev` fits when prev + L <= capacity; otherwise the buffers are
  cut to `prev` rows when prev is not a multiple of 256, then extended by ceil(L / 256) * 256 rows.

Each table row below was worked out on paper from that sentence. The same tables check the
unquantized KVCache of the package (which runs on CPU tensors) and the byte accounting that
m5engine/prefix_cache.py:17-24 and m5engine/context.py:41-47 read through ``nbytes``: bytes per
allocated row must be the reference's own per-token estimate, context.py:169
(bits/8 + 4/64 bytes per element, 2 bytes unquantized) times 2 (K and V) times D.
"""

import pytest
import torch

from myinfer_amd import cache as C
from oracle import cache as OC

# (operations, capacity after each, offset after each); ("t", n) is trim(n), an int is an append
TABLES = [
    # 5 rows -> one step; 1 more fits; 300 more at offset 6: cut to 6, grow by 512 -> 518
    ([5, 1, 300], [256, 256, 518], [5, 6, 306]),
    # a step-aligned offset grows with no cut
    ([256, 1], [256, 512], [256, 257]),
    ([512, 300], [512, 1024], [512, 812]),
    # prefill chunks of 2048
    ([2048, 2048, 2048], [2048, 4096, 6144], [2048, 4096, 6144]),
    # trim then refill inside the capacity: nothing moves
    ([100, ("t", 50), 200], [256, 256, 256], [100, 50, 250]),
    # trim to an unaligned offset, then overflow: cut to 70, grow by 512 -> 582
    ([100, ("t", 30), 300], [256, 256, 582], [100, 70, 370]),
    # trim below a full step, then overflow by a little: cut to 246, grow by 256 -> 502
    ([256, ("t", 10), 20], [256, 256, 502], [256, 246, 266]),
    # trimming more than the offset removes only the offset
    ([5, ("t", 10), 3], [256, 256, 256], [5, 0, 3]),
    # 257 rows take 2 steps; 513 more at offset 257 (unaligned): cut to 257, grow by 768 -> 1025
    ([257, 513], [512, 1025], [257, 770]),
    # 300 at offset 257 (unaligned): cut to 257, grow by 512 -> 769
    ([257, 300], [512, 769], [257, 557]),
]


def _run_model(ops):
    m = OC.CacheModel()
    caps, offs = [], []
    for op in ops:
        if isinstance(op, tuple):
            m.trim(op[1])
        else:
            m.update(op)
        caps.append(m.capacity)
        offs.append(m.offset)
    return caps, offs


@pytest.mark.parametrize("ops,caps,offs", TABLES)
def test_cache_model_growth(ops, caps, offs):
    got_caps, got_offs = _run_model(ops)
    assert got_caps == caps
    assert got_offs == offs


def test_trim_returns_amount():
    m = OC.CacheModel()
    m.update(5)
    assert m.trim(3) == 3 and m.offset == 2
    assert m.trim(10) == 2 and m.offset == 0


def test_token_by_token_growth():
    m = OC.CacheModel()
    for i in range(1, 600):
        m.update(1)
        assert m.capacity == ((i + 255) // 256) * 256


@pytest.mark.parametrize("ops,caps,offs", TABLES)
def test_plain_cache_follows_the_tables(ops, caps, offs):
    """The package's unquantized KVCache (CPU tensors) keeps the same capacities and offsets,
    and keeps the rows below the cut."""
    B, H, D = 1, 2, 8
    c = C.KVCache()
    pos = 0
    for op, cap, off in zip(ops, caps, offs):
        if isinstance(op, tuple):
            c.trim(op[1])
            pos = c.offset
        else:
            k = torch.arange(pos, pos + op, dtype=torch.float32)[None, None, :, None].expand(B, H, op, D)
            kk, vv = c.update_and_fetch(k.contiguous(), -k.contiguous())
            pos += op
            assert torch.equal(kk[0, 0, :, 0], torch.arange(pos, dtype=torch.float32))
            assert torch.equal(vv[0, 1, :, 3], -torch.arange(pos, dtype=torch.float32))
        assert c.keys.shape[2] == cap
        assert c.offset == off
        assert c.nbytes == 2 * B * H * cap * D * 4


@pytest.mark.parametrize("bits,D,elem", [(8, 128, 2), (4, 128, 2), (8, 64, 2), (None, 128, 2), (None, 256, 2)])
def test_row_bytes_is_the_reference_estimate(bits, D, elem):
    """context.py:169: per element bytes = bits/8 + 4/64 (quantized, G = 64, 2-byte scale and
    bias) or 2 (unquantized); K and V give the factor 2 of kv_estimate_per_token."""
    per_elem = 2.0 if not bits else bits / 8 + 4 / 64
    assert 2 * OC.row_bytes(D, bits, elem) == 2 * D * per_elem
    # C2's figure: 272 B per token and KV head at 8 bits, 144 B at 4 bits
    if D == 128 and bits:
        assert 2 * OC.row_bytes(D, bits, elem) == {8: 272, 4: 144}[bits]
