// Internal launchers shared between the kernels' translation units and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/kvq.h"

namespace kvq {

hipError_t launch_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst, const kvq_rows* v_src,
                                  const kvq_qtensor* v_dst, const kvq_rope_params* rope, int64_t row_offset, int B, int H,
                                  int L, int D, int bits, int group_size, int dtype, hipStream_t stream);
hipError_t launch_paged_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_pool, const kvq_rows* v_src,
                                        const kvq_qtensor* v_pool, int num_pages, const int32_t* table,
                                        int64_t table_stride, const int32_t* starts, int64_t row_offset,
                                        const kvq_rope_params* rope, int B, int H, int L, int D, int bits,
                                        int group_size, int dtype, hipStream_t stream);
hipError_t launch_rope(const kvq_rows* x, const kvq_rope_params* rope, int B, int H, int L, int dtype, hipStream_t stream);

// The decode kernel's width for head dimension D: 64, 128 or 256. A narrower row (D a multiple of 8)
// runs at the next width: its K/V rows are read that wide at their own stride (the bytes past the row
// are the next row's or, past the sequence, zero), the queries' dims past D are zero and only D dims
// of the output are stored.
int decode_kernel_dim(int D);
size_t decode_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window, int bits, int G);
// mask: a general mask (kvq_mask) or nullptr
hipError_t launch_decode(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                         const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype,
                         float scale, int causal, int window, void* workspace, hipStream_t stream,
                         const kvq_mask* mask = nullptr);

hipError_t launch_decode_paged(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                               const int32_t* table, int64_t table_stride, const int32_t* seq_lens, const kvq_rows* out,
                               int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype, float scale,
                               int causal, int window, void* workspace, hipStream_t stream);
hipError_t launch_decode_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                               const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype, float scale,
                               int causal, int window, void* workspace, hipStream_t stream,
                               const kvq_mask* mask = nullptr);

size_t prefill_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window, int bits);
hipError_t launch_prefill(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                          const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype,
                          float scale, int causal, int window, void* workspace, hipStream_t stream);
hipError_t launch_prefill_paged(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                                const int32_t* table, int64_t table_stride, const int32_t* seq_lens, const kvq_rows* out,
                                int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype, float scale,
                                int causal, int window, void* workspace, hipStream_t stream);
// wide.hip: head_dim 256 over quantized (4/8 bits, groups 64/128) and unquantized caches, and head_dim 64
// over unquantized caches, any query length
size_t wide_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window);
hipError_t launch_wide(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                       const kvq_rows* out, int B, int Hq, int Hkv, int L, int S, int bits, int G, int dtype,
                       float scale, int causal, int window, void* workspace, hipStream_t stream);
hipError_t launch_wide_paged(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                             const int32_t* table, int64_t table_stride, const int32_t* seq_lens, const kvq_rows* out,
                             int B, int Hq, int Hkv, int L, int S, int bits, int G, int dtype, float scale, int causal,
                             int window, void* workspace, hipStream_t stream);
hipError_t launch_wide_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                             const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype, float scale,
                             int causal, int window, void* workspace, hipStream_t stream,
                             const kvq_mask* mask = nullptr);
hipError_t launch_prefill_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                                const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype,
                                float scale, int causal, int window, void* workspace, hipStream_t stream);

}  // namespace kvq
