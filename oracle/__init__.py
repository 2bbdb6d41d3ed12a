"""CPU oracle for the quantized-KV attention path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or, for the baseline, as the thing timed on the host):
the product path (``myinfer_amd``) never calls it and has no CPU fallback.

Contents
  quantize.py   restatement of MLX's affine quantizer (mx.quantize / mx.dequantize) as used by
                mlx-lm's QuantizedKVCache, bit-exact target for the append kernel.
  attention.py  exact fp64 attention over the dequantized cache (the parity gate), and a
                torch-CPU port of m5engine/attention.py's blocked algorithm with the reference's
                dtype casts (the CPU baseline and an informative second oracle).
  cache.py      a list-based model of mlx-lm's KVCache / QuantizedKVCache bookkeeping
                (step-256 growth, offset, trim), the contract prefix_cache.py relies on.

How each function is pinned (checks live in tests/test_oracle_*.py):
  quantize      hand-derived known-answer groups (all-zero, constant, integer ramps of both
                signs), the bound |x - xhat| <= |s|/2 (+ rounding of the stored s, b), the
                extreme-maps-to-code-0 invariant, agreement of the numpy and C restatements,
                and torch's own fp16/bf16 rounding for the stored scales/biases.
                MLX-exactness itself is "parity unpinned": mlx is not installed here and the
                reference holds no quantized fixtures (its only test, tests/test_core.py:23-40,
                calls mx.quantize on both sides).
  attention     brute-force softmax on tiny shapes, closed forms (S = 1 -> V0; equal keys ->
                mean of V; a dominant logit -> that row of V), invariance under key
                permutation, and the reference test's dense-equivalence cases
                (tests/test_core.py:16-40) for the blocked port.
  cache         the expectations of tests/test_core.py:79-97 (prefix take / trim / offset).
"""
