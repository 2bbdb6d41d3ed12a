/*
 * kvq.h - C ABI of libkvq.so, the MI355X (gfx950) quantized-KV attention library.
 *
 * The library implements the hot path of the reference's memory-bounded attention over an
 * MLX-layout affine-quantized KV cache:
 *   - quantize-and-append of new K/V rows into the cache   (reference: mlx-lm
 *     QuantizedKVCache.update_and_fetch, reached from m5engine/attention.py:106-112 and the
 *     per-layer attention call; the quantizer is mx.quantize, restated in oracle/quantize.py)
 *   - attention of queries against the quantized cache      (reference:
 *     m5engine/attention.py:29-103 blocked_quantized_sdpa, and the L == 1 fallback at :42-45)
 *
 * Layout (MLX conventions, all little-endian):
 *   queries / outputs   T[B][Hq][L][D], last dimension contiguous, other strides free.
 *   K or V cache        codes  uint32[B][H][S_cap][D*bits/32]  (code k of a word at bits
 *                                                               [k*bits, (k+1)*bits), LSB first)
 *                       scales T[B][H][S_cap][D/group]
 *                       biases T[B][H][S_cap][D/group]
 *                       dequantized value = scale * code + bias
 *   T is float16 or bfloat16; scales and biases have the same dtype as the K/V rows.
 *
 * Conventions:
 *   - Every entry point returns KVQ_OK (0) or a negative status; it never throws and never
 *     aborts. kvq_last_error() returns a message for the calling thread's last failure.
 *   - All pointers are device pointers, except the kvq_rows / kvq_qtensor descriptors
 *     themselves, which are read on the host during the call.
 *   - Launches are asynchronous on `stream` (a hipStream_t; NULL = the default stream).
 *   - The library allocates no device memory: scratch space (the attention workspace) is
 *     owned by the caller; its size comes from the *_workspace_size functions. A workspace must
 *     be zero-filled once, when it is allocated (hipMemset): the kernels keep per-call split
 *     counters in it and reset them before they finish, so it stays valid for later calls of any
 *     shape. Calls that share one workspace must be ordered (same stream, or synchronized).
 *   - Strides are in elements of the pointed-to type.
 */
#ifndef KVQ_H
#define KVQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVQ_ABI_VERSION 6

/* Element types of queries, K/V rows, outputs, scales and biases. */
#define KVQ_DTYPE_F16 0
#define KVQ_DTYPE_BF16 1

/* Status codes. */
#define KVQ_OK 0
#define KVQ_ERR_INVALID (-1)     /* bad argument: null pointer, shape, stride, dtype, bits    */
#define KVQ_ERR_UNSUPPORTED (-2) /* well-formed but not built: head_dim, group size, head ratio */
#define KVQ_ERR_WORKSPACE (-3)   /* workspace missing or smaller than *_workspace_size()       */
#define KVQ_ERR_HIP (-4)         /* the HIP runtime reported an error at launch                */
#define KVQ_ERR_CAPACITY (-5)    /* the page pool cannot hold the request                      */

/* A strided T[B][H][L][D] array (D contiguous). */
typedef struct kvq_rows {
  void* data;
  int64_t stride_b, stride_h, stride_l;
} kvq_rows;

/* A quantized K or V cache view: the (codes, scales, biases) triple of the reference.
 *
 * range_exp (may be NULL) is the cache's range exponent E, one int32 in device memory, kept by
 * the appends and read by the quantized prefill kernels:
 *   - kvq_*quantize_append raise it (atomic max) to the smallest E >= 0 with every dequantized
 *     value s * c + b of every group they write at most 2^15 * 2^E in magnitude (it starts at 0
 *     and never decreases: a trimmed cache keeps it);
 *   - the quantized prefill kernels stage their fp16 MFMA operands as (s * c + b) * 2^-E and fold
 *     2^E back into the fp32 scores (K) and the output (V), so a bf16 cache whose values leave the
 *     fp16 range still gives finite results (values below 2^(E - 24) then lose precision in the
 *     operands). E = 0 (or NULL) stages the values as they are: there a bf16 group beyond the fp16
 *     range makes the row blocks that read it return NaN, never a finite wrong value;
 *   - decode ignores it: it applies scales and biases in fp32.
 * This field has no counterpart in the reference, whose MLX kernels dequantize in bf16. */
typedef struct kvq_qtensor {
  uint32_t* codes;
  void* scales;
  void* biases;
  int64_t codes_stride_b, codes_stride_h, codes_stride_s; /* in uint32 words; the row itself is contiguous */
  int64_t sb_stride_b, sb_stride_h, sb_stride_s;          /* in T elements; shared by scales and biases    */
  int32_t* range_exp;                                     /* the range exponent E above, or NULL           */
} kvq_qtensor;

/* ABI version the library was built with (KVQ_ABI_VERSION). */
int kvq_abi_version(void);

/* Message describing the calling thread's most recent failure ("" if none). */
const char* kvq_last_error(void);

/*
 * Quantize rows [0, L) of k_src (and v_src, when not NULL) with MLX's affine quantizer and
 * write them to rows [row_offset, row_offset + L) of k_dst (and v_dst), in one launch.
 * Replaces: mx.quantize inside mlx-lm QuantizedKVCache.update_and_fetch (third-party, called
 * per layer by the model's attention) and KVCache.to_quantized, used by
 * m5engine/attention.py:106-112 (safe_maybe_quantize_kv_cache). Codes, scales and biases are
 * bit-identical to the CPU restatement in oracle/quantize.py.
 * Supported: bits in {2, 4, 8}; group_size in {32, 64, 128}; D a multiple of group_size and of 8.
 */
int kvq_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst,
                        const kvq_rows* v_src, const kvq_qtensor* v_dst,
                        int64_t row_offset, int B, int H, int L, int D,
                        int bits, int group_size, int dtype, void* stream);

/* Rotary position embedding of the rows passed to kvq_rope / kvq_rope_quantize_append
 * (the rotation mlx-lm's attention layers apply with nn.RoPE / mx.fast.rope before the cache
 * update; fused with the KV write as in native/src/kernels.metal:106-160). Row l of a call sits
 * at position offset + l; pair i turns by the angle (position * scale) * freq_i in fp32, with
 * freq_i = 1 / base^(2i / dims) evaluated in double precision and rounded to fp32. */
typedef struct kvq_rope_params {
  int dims;        /* rotated leading dims: a multiple of 16, <= min(D, 256); the rest pass through */
  int traditional; /* 0: pairs (i, i + dims/2) (NeoX; mlx traditional=False); 1: pairs (2i, 2i+1) */
  float base;      /* theta                                                                        */
  float scale;     /* position scale (1 = none; linear RoPE scaling divides positions)             */
  int64_t offset;  /* position of row 0                                                            */
} kvq_rope_params;

/*
 * In-place RoPE of rows [0, L) of x (T[B][H][L][D], the query rows of a step).
 * Replaces: the query rotation mlx-lm's attention layers apply before attention.
 * The rotation runs in fp32 and the result is rounded to T.
 */
int kvq_rope(const kvq_rows* x, const kvq_rope_params* rope, int B, int H, int L, int D, int dtype, void* stream);

/*
 * kvq_quantize_append with the keys rotated first: k_src is read, rotated by `rope`, rounded to
 * T (the dtype RoPE returns) and quantized; v_src is quantized as is. k_src is not modified.
 * Replaces: the key rotation followed by QuantizedKVCache.update_and_fetch in mlx-lm's attention
 * layers (the fused RoPE + KV write of native/src/kernels.metal:106-160, here into the
 * quantized cache). Same support as kvq_quantize_append, and rope->dims as in kvq_rope.
 */
int kvq_rope_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst,
                             const kvq_rows* v_src, const kvq_qtensor* v_dst, const kvq_rope_params* rope,
                             int64_t row_offset, int B, int H, int L, int D,
                             int bits, int group_size, int dtype, void* stream);

/*
 * Attention of L query rows per sequence against a quantized cache, for small L (decode):
 * out = softmax(scale * q K^T + mask) V over the dequantized K/V.
 * Replaces: m5engine/attention.py:42-45 (the L == 1 hand-off to mlx-lm's
 * quantized_scaled_dot_product_attention) and, for L > 1, the blocked loop at :64-103.
 * Requirements: D a multiple of 8 up to 256 and of group_size; group_size in {32, 64, 128} with
 *   W / 4 <= group_size <= W, where W is the kernel width: D itself for D in {64, 128, 256}, else
 *   the next of them (32 dims run at 64, 96 at 128, 192 at 256: the queries' dims past D are zero,
 *   and each K/V row is read W wide at its own stride, so the scale and bias rows of such a cache
 *   must hold exactly D / group_size elements); bits in {4, 8}. One pass of the kernel serves
 *   16 * group_size / W query rows ((Hq / Hkv) * L) of a KV head; more rows take more passes over
 *   the keys. Only D dims of each output row are written.
 *   seq_lens: NULL (every sequence has S keys) or device int32[B] with 1 <= seq_lens[b] <= S.
 *   causal:   query l of sequence b sits at position seq_len_b - L + l and sees keys <= it.
 *   window:   0 = none; otherwise keys k > position - window only (sliding window).
 *   workspace: device buffer of at least kvq_decode_workspace_size(...) bytes, 256-byte aligned,
 *              zero-filled at allocation (see the conventions above).
 * The key range is split over workgroups; their log-sum-exp partials are merged by the last
 * workgroup of each unit to finish when there are at most 4 splits, otherwise by a second, small
 * launch on the same stream (both are enqueued by this call).
 */
int kvq_decode_attn(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v,
                    const int32_t* seq_lens, const kvq_rows* out,
                    int B, int Hq, int Hkv, int L, int D, int S,
                    int bits, int group_size, int dtype,
                    float scale, int causal, int window,
                    void* workspace, size_t workspace_bytes, void* stream);

size_t kvq_decode_workspace_size(int B, int Hq, int Hkv, int L, int D, int S, int window);

/*
 * kvq_decode_attn without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference: its MLX path allocates freely.
 * The split partials and arrival counters live in a static device array of
 * KVQ_STATIC_SCRATCH_BYTES that the library holds on every GPU it runs on until the process
 * ends; the call allocates nothing. A call whose plan needs more scratch than that
 * (kvq_decode_workspace_size(...) > KVQ_STATIC_SCRATCH_BYTES, e.g. B * Hq * L above about
 * 15 000 rows at D = 128) returns KVQ_ERR_WORKSPACE and launches nothing.
 * Every call on one GPU shares that GPU's scratch: calls that overlap on one GPU (different
 * streams or threads without ordering between them) race and give undefined results. The first
 * call on a GPU also zeroes the scratch's counters on `stream` (a kernel, not a memset).
 * Arguments, requirements and results are those of kvq_decode_attn; the kernels are the same.
 */
#define KVQ_STATIC_SCRATCH_BYTES (8u << 20)
int kvq_decode_attn_static(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v,
                           const int32_t* seq_lens, const kvq_rows* out,
                           int B, int Hq, int Hkv, int L, int D, int S,
                           int bits, int group_size, int dtype,
                           float scale, int causal, int window, void* stream);

/*
 * A general attention mask: element (b, kvh, j, l, key) of the [B][Hkv][Hq / Hkv][L][S] score
 * layout the reference's GQA reshape uses (query head h = kvh * (Hq / Hkv) + j) sits at
 *   data + b * stride_b + kvh * stride_kvh + j * stride_rep + l * stride_l + key
 * (strides in elements; 0 broadcasts a dimension; keys are contiguous).
 *   KVQ_MASK_BOOL: uint8, nonzero = the key is visible (the reference's boolean masks);
 *   KVQ_MASK_F16 / _BF16 / _F32: additive, added to scale * q.k before the softmax.
 * A row that sees no key returns 0 (the reference's blocked path does the same).
 */
#define KVQ_MASK_BOOL 1
#define KVQ_MASK_F16 2
#define KVQ_MASK_BF16 3
#define KVQ_MASK_F32 4
typedef struct kvq_mask {
  const void* data;
  int32_t kind; /* KVQ_MASK_* */
  int64_t stride_b, stride_kvh, stride_rep, stride_l;
} kvq_mask;

/*
 * kvq_decode_attn (any L) under a general mask instead of causal / window / seq_lens: boolean
 * masks that are not causal, sliding-window or right-padding masks, per-head masks and additive
 * masks. Replaces: m5engine/attention.py:55-56 and :76-80 (the array-mask branches of the
 * blocked loop) and the mask handling of the L == 1 hand-off at :42-45. The decode kernel reads
 * the mask beside each 32-key tile; rows beyond one pass take more passes over the keys, so long
 * prompts under such masks run at the decode kernel's rate. Same requirements and workspace
 * (kvq_decode_workspace_size with window 0) as kvq_decode_attn.
 */
int kvq_decode_attn_masked(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v,
                           const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S,
                           int bits, int group_size, int dtype, float scale, const kvq_mask* mask,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * The same over an unquantized cache (kvq_decode_attn_dense's arguments and head dims).
 * Replaces the mask handling of mx.fast.scaled_dot_product_attention for array masks.
 */
int kvq_decode_attn_dense_masked(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v,
                                 const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S,
                                 int dtype, float scale, const kvq_mask* mask,
                                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * Attention for prefill chunks (any L): same contract as kvq_decode_attn, MFMA tiles with
 * K/V tiles dequantized into LDS. Replaces m5engine/attention.py:29-103 for L > 1.
 * Requirements: those of kvq_decode_attn; Hq a multiple of Hkv; at D = 64 or 128 the output rows
 *   are stored 16 bytes at a time, so out 16-byte aligned with strides in multiples of 8 elements;
 *   there too, with two or more scale groups per row, scale and bias rows 4-byte aligned (even
 *   strides; MLX's contiguous layout is).
 * D = 256 runs a kernel of its own (128 query rows per workgroup, 32-key tiles) whose split key
 * ranges are merged by a second, small launch on the same stream. Head dims other than 64, 128
 * and 256 run the decode kernel (any L) and take kvq_decode_attn's workspace size.
 */
int kvq_prefill_attn(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v,
                     const int32_t* seq_lens, const kvq_rows* out,
                     int B, int Hq, int Hkv, int L, int D, int S,
                     int bits, int group_size, int dtype,
                     float scale, int causal, int window,
                     void* workspace, size_t workspace_bytes, void* stream);

size_t kvq_prefill_workspace_size(int B, int Hq, int Hkv, int L, int D, int S, int window);

/*
 * Attention over an unquantized cache: K and V are T[B][Hkv][S_cap][D] rows (kvq_rows, viewed
 * as [..., :S, :]) in the queries' dtype. Same masks, outputs, workspace and streams as the
 * quantized entry points; the workspace sizes above cover these calls too.
 * Replaces: mx.fast.scaled_dot_product_attention, which mlx-lm's scaled_dot_product_attention
 * calls for every cache that is not quantized: the plain KVCache before quantized_kv_start and
 * the RotatingKVCache (sliding-window) layers that m5engine/attention.py:106-112 leaves
 * unquantized.
 * The products run on MFMA in the cache's own type (fp16 or bf16, exact operands) with fp32
 * accumulation; the probabilities enter the PV product in that type.
 * Requirements: D in {64, 128, 256}, or another multiple of 8 up to 256, run at the next of those
 * widths for any L (by the decode kernel up to 128 dims, by the head_dim-256 kernel past them; the
 * key rows must then be exactly D elements apart); rows 16-byte aligned with strides that are
 * multiples of 8 elements. At D = 256 both entry points run the head_dim-256 prefill kernel (any
 * L); the prefill entry point runs the same kernel at D = 64. At D = 128 the prefill entry point
 * stores output rows 16 bytes at a time, so out must be 16-byte aligned with strides in multiples
 * of 8 elements there too.
 */
int kvq_decode_attn_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v,
                          const int32_t* seq_lens, const kvq_rows* out,
                          int B, int Hq, int Hkv, int L, int D, int S, int dtype,
                          float scale, int causal, int window,
                          void* workspace, size_t workspace_bytes, void* stream);

int kvq_prefill_attn_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v,
                           const int32_t* seq_lens, const kvq_rows* out,
                           int B, int Hq, int Hkv, int L, int D, int S, int dtype,
                           float scale, int causal, int window,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * ---- Paged layout ----
 * A paged pool holds one layer's K (or V) for many sequences in pages of KVQ_PAGE_ROWS rows:
 * codes u32 [num_pages][H][KVQ_PAGE_ROWS][D*bits/32], scales/biases T [num_pages][H][KVQ_PAGE_ROWS][D/G]
 * (head-major within a page), described by a kvq_qtensor whose batch strides are page strides.
 * Row r of sequence b lives in page block_table[b * table_stride + r / KVQ_PAGE_ROWS], at row
 * r % KVQ_PAGE_ROWS. The attention kernels clamp table entries to [0, num_pages) (a read of a
 * wrong page is harmless); the paged append drops a row whose entry lies outside [0, num_pages),
 * such as a -1 "unallocated" sentinel, so it never writes into a page it was not given.
 * Replaces: the reference's paged KV layout (native/src/kv_cache.cpp:8-27, 16-token blocks read
 * through a block table in native/src/kernels.metal:106-160, 384-450), here for the quantized MLX
 * cache, as the alternative to whole-cache move-reuse (m5engine/prefix_cache.py:1-5). Pages are
 * 64 rows so that a prefill tile (64 keys) reads one page and a decode tile (32 keys) half of one.
 */
#define KVQ_PAGE_ROWS 64

/*
 * kvq_quantize_append into a paged pool: row l of sequence b goes to row starts[b] + l (starts: a
 * device int32 [B], or NULL for row_offset + l for every sequence). With `rope` the keys are
 * rotated first, row l of sequence b at position rope->offset + (starts ? starts[b] : 0) + l.
 * Rows whose page index is at or past table_stride, or whose table entry lies outside
 * [0, num_pages), are dropped.
 */
int kvq_paged_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_pool,
                              const kvq_rows* v_src, const kvq_qtensor* v_pool, int num_pages,
                              const int32_t* block_table, int64_t table_stride, const int32_t* starts,
                              int64_t row_offset, const kvq_rope_params* rope,
                              int B, int H, int L, int D, int bits, int group_size, int dtype, void* stream);

/*
 * kvq_decode_attn / kvq_prefill_attn over paged pools (same arguments, masks, workspace sizes and
 * outputs; S is the longest sequence, table_stride >= ceil(S / KVQ_PAGE_ROWS)). The results are
 * bit-identical to the contiguous entry points over the same rows.
 */
int kvq_paged_decode_attn(const kvq_rows* q, const kvq_qtensor* k_pool, const kvq_qtensor* v_pool,
                          int num_pages, const int32_t* block_table, int64_t table_stride,
                          const int32_t* seq_lens, const kvq_rows* out,
                          int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size, int dtype,
                          float scale, int causal, int window,
                          void* workspace, size_t workspace_bytes, void* stream);

int kvq_paged_prefill_attn(const kvq_rows* q, const kvq_qtensor* k_pool, const kvq_qtensor* v_pool,
                           int num_pages, const int32_t* block_table, int64_t table_stride,
                           const int32_t* seq_lens, const kvq_rows* out,
                           int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size, int dtype,
                           float scale, int causal, int window,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * Radix prefix cache over a page pool (host memory and host code only; no HIP calls).
 * Replaces: PagedRadixKVCache (native/include/kv_cache.hpp, native/src/kv_cache.cpp:73-157):
 * match_and_allocate / commit_prefix_blocks / clear_cache, with page reference counts added:
 * pages returned by match_and_allocate are held until kvq_radix_release, and held pages are
 * never evicted. Not thread-safe: one radix per thread, or a lock around it.
 */
typedef struct kvq_radix kvq_radix;
typedef struct kvq_radix_info {
  int num_pages, page_tokens, cached_pages, free_pages, in_use_pages;
  int64_t prefix_hit_tokens, prompt_tokens;
} kvq_radix_info;

kvq_radix* kvq_radix_create(int num_pages, int page_tokens);  /* NULL on bad sizes */
void kvq_radix_destroy(kvq_radix* r);
/* Match the longest cached prefix of whole pages (leaving the last prompt token unmatched) and
 * allocate pages for the rest of n_tokens + max_new_tokens + 16 tokens (capped at the pool):
 * table[0 .. *n_pages) holds them, the first *matched_tokens / page_tokens of them matched.
 * KVQ_ERR_CAPACITY (nothing held) when free and evictable pages run out. */
int kvq_radix_match_and_allocate(kvq_radix* r, const int32_t* tokens, int n_tokens, int max_new_tokens,
                                 int32_t* table, int table_capacity, int* matched_tokens, int* n_pages);
/* Key the full pages of tokens[0 .. valid_tokens) (held pages of `table`) for later matches. */
int kvq_radix_commit(kvq_radix* r, const int32_t* tokens, int n_tokens, const int32_t* table, int n_pages,
                     int valid_tokens);
int kvq_radix_release(kvq_radix* r, const int32_t* table, int n_pages);
void kvq_radix_clear(kvq_radix* r);
int kvq_radix_stats(const kvq_radix* r, kvq_radix_info* out);
const char* kvq_radix_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KVQ_H */
