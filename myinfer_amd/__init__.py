"""MI355X-native quantized-KV attention (the hot path of tdcb/myinfer's M5Engine).

Public modules:
  myinfer_amd.attention  reference-named API (blocked_quantized_sdpa, safe_maybe_quantize_kv_cache,
                         install, score_budget_bytes, MIN_BLOCK)
  myinfer_amd.cache      KVCache / QuantizedKVCache in MLX layout on the GPU
  myinfer_amd.kernels    typed wrappers of libkvq.so (quantize, quantize_append, attention)
  myinfer_amd._lib       ctypes binding of include/kvq.h
"""

__version__ = "0.1.0"
