// C ABI of libkvq.so: argument validation, error reporting, dispatch to the kernel launchers.
// Every check runs on the host before any HIP call, so a rejected call touches no device state.

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "launch.h"
#include "merge.h"

// Scratch of kvq_decode_attn_static: device memory the library owns, one copy per GPU, held until
// the process ends. In host code `scratch` is a host-side stand-in for the symbol, not a device
// address: the kernels get the per-device address hipGetSymbolAddress returns (static_scratch
// below), never the name.
static __device__ __align__(256) uint8_t scratch[KVQ_STATIC_SCRATCH_BYTES];

// Zero `n` words (the scratch's arrival counters, once per device). A kernel rather than
// hipMemsetAsync, so that a caller may capture the first call into a HIP graph.
__global__ void zero_words_kernel(uint32_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return KVQ_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(KVQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

int check_dtype(int dtype) {
  if (dtype != KVQ_DTYPE_F16 && dtype != KVQ_DTYPE_BF16) return fail(KVQ_ERR_INVALID, "dtype %d is not f16 (0) or bf16 (1)", dtype);
  return KVQ_OK;
}

int check_qtensor(const kvq_qtensor* t, const char* name) {
  if (!t) return fail(KVQ_ERR_INVALID, "%s descriptor is NULL", name);
  if (!t->codes || !t->scales || !t->biases) return fail(KVQ_ERR_INVALID, "%s has a NULL codes/scales/biases pointer", name);
  if (t->codes_stride_b < 0 || t->codes_stride_h < 0 || t->codes_stride_s <= 0 || t->sb_stride_b < 0 ||
      t->sb_stride_h < 0 || t->sb_stride_s <= 0)
    return fail(KVQ_ERR_INVALID, "%s has a negative or zero stride", name);
  if (!aligned(t->scales, 2) || !aligned(t->biases, 2)) return fail(KVQ_ERR_INVALID, "%s scales/biases are not 2-byte aligned", name);
  return KVQ_OK;
}

int check_rows(const kvq_rows* r, const char* name, int D, bool vec16) {
  if (!r || !r->data) return fail(KVQ_ERR_INVALID, "%s is NULL", name);
  if (r->stride_b < 0 || r->stride_h < 0 || r->stride_l < 0) return fail(KVQ_ERR_INVALID, "%s has a negative stride", name);
  if (vec16) {
    if (!aligned(r->data, 16) || r->stride_b % 8 || r->stride_h % 8 || r->stride_l % 8 || D % 8)
      return fail(KVQ_ERR_INVALID, "%s must be 16-byte aligned with strides that are multiples of 8 elements", name);
  } else if (!aligned(r->data, 2)) {
    return fail(KVQ_ERR_INVALID, "%s is not 2-byte aligned", name);
  }
  return KVQ_OK;
}


// Shared checks of the attention entry points (shape, dtype, scale, window, queries, output).
int check_attn_common(const kvq_rows* q, const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype,
                      float scale, int window) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || S <= 0) return fail(KVQ_ERR_INVALID, "B, Hq, Hkv, L and S must be positive (got %d, %d, %d, %d, %d)", B, Hq, Hkv, L, S);
  if (Hq % Hkv) return fail(KVQ_ERR_INVALID, "Hq=%d is not a multiple of Hkv=%d", Hq, Hkv);
  if (window < 0) return fail(KVQ_ERR_INVALID, "window must be >= 0, got %d", window);
  if (!isfinite(scale)) return fail(KVQ_ERR_INVALID, "scale is not finite");
  if ((rc = check_rows(q, "queries", D, true))) return rc;
  if ((rc = check_rows(out, "out", D, false))) return rc;
  // every attention kernel writes 4 output elements (8 bytes) at a time
  if (!aligned(out->data, 8) || out->stride_b % 4 || out->stride_h % 4 || out->stride_l % 4)
    return fail(KVQ_ERR_INVALID, "out must be 8-byte aligned with strides that are multiples of 4 elements");
  return KVQ_OK;
}

// Head dimensions 64, 128 and 256 have kernels of their own width; any other multiple of 8 up to 256
// runs at the next width (kvq::decode_kernel_dim), for every query length: on the decode kernel, or
// for unquantized rows past 128 dims on the head_dim-256 kernel.
bool native_dim(int D) { return D == 64 || D == 128 || D == 256; }

int check_head_dim(int D, const char* what) {
  if (D > 0 && D % 8 == 0 && D <= 256) return KVQ_OK;
  return fail(KVQ_ERR_UNSUPPORTED, "%s supports head_dim 64, 128, 256 and other multiples of 8 up to 256, got %d", what,
              D);
}

int check_workspace(size_t ws_needed, void* workspace, size_t workspace_bytes) {
  if (!workspace || workspace_bytes < ws_needed)
    return fail(KVQ_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", ws_needed, workspace ? workspace_bytes : (size_t)0);
  if (!aligned(workspace, 256)) return fail(KVQ_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return KVQ_OK;
}

// Scale-group sizes the attention kernels are built for: 32, 64 and 128, at most the kernel width and
// at least a quarter of it (a decode lane's quarter of a row lies in one group), dividing D.
int check_attn_group(int group_size, int D) {
  const int Dk = kvq::decode_kernel_dim(D);
  if ((group_size != 32 && group_size != 64 && group_size != 128) || group_size > Dk || 4 * group_size < Dk ||
      D % group_size)
    return fail(KVQ_ERR_UNSUPPORTED,
                "attention supports group_size 32, 64 and 128 dividing head_dim (%d) and between %d/4 and %d, got %d",
                D, Dk, Dk, group_size);
  return KVQ_OK;
}

// Everything check_attn checks but the workspace.
int check_attn_args(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const kvq_rows* out, int B, int Hq,
                    int Hkv, int L, int D, int S, int bits, int group_size, int dtype, float scale, int window) {
  int rc;
  if ((rc = check_attn_common(q, out, B, Hq, Hkv, L, D, S, dtype, scale, window))) return rc;
  if (bits != 4 && bits != 8) return fail(KVQ_ERR_UNSUPPORTED, "attention supports 4- and 8-bit caches, got bits=%d", bits);
  if ((rc = check_attn_group(group_size, D))) return rc;
  if ((rc = check_qtensor(k, "keys"))) return rc;
  if ((rc = check_qtensor(v, "values"))) return rc;
  const int64_t row_words = (int64_t)D * bits / 32;
  for (const kvq_qtensor* t : {k, v}) {
    if (!aligned(t->codes, 16) || (t->codes_stride_s * 4) % 16 || (t->codes_stride_h * 4) % 16 || (t->codes_stride_b * 4) % 16)
      return fail(KVQ_ERR_INVALID, "codes must be 16-byte aligned with 16-byte-multiple row, head and batch strides");
    if (t->codes_stride_s < row_words) return fail(KVQ_ERR_INVALID, "codes row stride %lld is smaller than D*bits/32=%lld", (long long)t->codes_stride_s, (long long)row_words);
    if (t->sb_stride_s < D / group_size)
      return fail(KVQ_ERR_INVALID, "scales row stride %lld is smaller than D/group=%d", (long long)t->sb_stride_s, D / group_size);
    // a row narrower than its kernel reads the next row's first groups past its own: they must be
    // rows of the cache, not padding
    if (D < kvq::decode_kernel_dim(D) && t->sb_stride_s != D / group_size)
      return fail(KVQ_ERR_UNSUPPORTED, "head_dim %d needs scale and bias rows of exactly D/group=%d elements, got a stride "
                  "of %lld", D, D / group_size, (long long)t->sb_stride_s);
    // the kernels address each (sequence, KV head)'s rows with 32-bit byte offsets
    if ((int64_t)S * t->codes_stride_s * 4 > (int64_t)UINT32_MAX || (int64_t)S * t->sb_stride_s * 2 > (int64_t)UINT32_MAX)
      return fail(KVQ_ERR_UNSUPPORTED, "attention needs S times each row stride within 4 GiB (S=%d)", S);
  }
  return KVQ_OK;
}

int check_attn(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const kvq_rows* out, int B, int Hq,
               int Hkv, int L, int D, int S, int bits, int group_size, int dtype, float scale, int window,
               size_t ws_needed, void* workspace, size_t workspace_bytes) {
  int rc;
  if ((rc = check_attn_args(q, k, v, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, window))) return rc;
  return check_workspace(ws_needed, workspace, workspace_bytes);
}

// Attention over an unquantized cache: K and V are strided T rows like the queries.
int check_attn_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const kvq_rows* out, int B, int Hq,
                     int Hkv, int L, int D, int S, int dtype, float scale, int window, size_t ws_needed,
                     void* workspace, size_t workspace_bytes) {
  int rc;
  if ((rc = check_attn_common(q, out, B, Hq, Hkv, L, D, S, dtype, scale, window))) return rc;
  if ((rc = check_rows(k, "keys", D, true))) return rc;
  if ((rc = check_rows(v, "values", D, true))) return rc;
  // a key row narrower than its kernel reads the next row's first elements past its own: they must
  // be a row of the cache, not padding
  if (D < kvq::decode_kernel_dim(D) && k->stride_l != D)
    return fail(KVQ_ERR_UNSUPPORTED, "head_dim %d needs key rows of exactly D elements, got a stride of %lld", D,
                (long long)k->stride_l);
  for (const kvq_rows* t : {k, v}) {
    if (t->stride_l < D) return fail(KVQ_ERR_INVALID, "K/V row stride %lld is smaller than D=%d", (long long)t->stride_l, D);
    // the kernels address each (sequence, KV head)'s rows with 32-bit byte offsets
    if ((int64_t)S * t->stride_l * 2 > (int64_t)UINT32_MAX)
      return fail(KVQ_ERR_UNSUPPORTED, "attention needs S times the K/V row stride within 4 GiB (S=%d)", S);
  }
  return check_workspace(ws_needed, workspace, workspace_bytes);
}

int check_quantize(const kvq_rows* k_src, const kvq_qtensor* k_dst, const kvq_rows* v_src, const kvq_qtensor* v_dst,
                   int64_t row_offset, int B, int H, int L, int D, int bits, int group_size, int dtype) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (bits != 2 && bits != 4 && bits != 8) return fail(KVQ_ERR_UNSUPPORTED, "bits must be 2, 4 or 8, got %d", bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(KVQ_ERR_UNSUPPORTED, "group_size must be 32, 64 or 128, got %d", group_size);
  if (B < 0 || H < 0 || L < 0 || D <= 0) return fail(KVQ_ERR_INVALID, "negative shape (B=%d H=%d L=%d D=%d)", B, H, L, D);
  if (D % group_size) return fail(KVQ_ERR_INVALID, "D=%d is not a multiple of group_size=%d", D, group_size);
  if (row_offset < 0) return fail(KVQ_ERR_INVALID, "row_offset must be >= 0");
  if ((v_src == nullptr) != (v_dst == nullptr)) return fail(KVQ_ERR_INVALID, "v_src and v_dst must both be given or both be NULL");
  if ((rc = check_rows(k_src, "k_src", D, true))) return rc;
  if ((rc = check_qtensor(k_dst, "k_dst"))) return rc;
  if (v_src) {
    if ((rc = check_rows(v_src, "v_src", D, true))) return rc;
    if ((rc = check_qtensor(v_dst, "v_dst"))) return rc;
  }
  const int64_t row_words = (int64_t)D * bits / 32;
  for (const kvq_qtensor* t : {k_dst, v_dst}) {
    if (!t) continue;
    if (t->codes_stride_s < row_words) return fail(KVQ_ERR_INVALID, "codes row stride is smaller than D*bits/32");
    if (bits == 8 && (!aligned(t->codes, 8) || t->codes_stride_s % 2 || t->codes_stride_h % 2 || t->codes_stride_b % 2))
      return fail(KVQ_ERR_INVALID, "8-bit codes must be 8-byte aligned with even word strides");
    if (t->sb_stride_s < D / group_size) return fail(KVQ_ERR_INVALID, "scales row stride is smaller than D/group_size");
  }
  return KVQ_OK;
}

// A paged pool described by a kvq_qtensor whose batch strides are page strides: pages of
// KVQ_PAGE_ROWS rows per head, head-major within a page.
int check_pool(const kvq_qtensor* t, const char* name, int H, int D, int bits, int group_size, int num_pages) {
  int rc;
  if ((rc = check_qtensor(t, name))) return rc;
  if (num_pages <= 0) return fail(KVQ_ERR_INVALID, "num_pages must be positive, got %d", num_pages);
  const int64_t row_words = (int64_t)D * bits / 32, groups = D / group_size;
  if (t->codes_stride_s < row_words || t->sb_stride_s < groups)
    return fail(KVQ_ERR_INVALID, "%s row strides are smaller than one row", name);
  if (D < kvq::decode_kernel_dim(D) && t->sb_stride_s != groups)
    return fail(KVQ_ERR_UNSUPPORTED, "head_dim %d needs %s scale and bias rows of exactly D/group=%lld elements", D, name,
                (long long)groups);
  if (t->codes_stride_h < KVQ_PAGE_ROWS * t->codes_stride_s || t->sb_stride_h < KVQ_PAGE_ROWS * t->sb_stride_s ||
      t->codes_stride_b < H * t->codes_stride_h || t->sb_stride_b < H * t->sb_stride_h)
    return fail(KVQ_ERR_INVALID, "%s is not [num_pages][H][%d][row]: its strides overlap", name, KVQ_PAGE_ROWS);
  return KVQ_OK;
}

int check_table(const int32_t* table, int64_t table_stride, int64_t rows_needed) {
  if (!table) return fail(KVQ_ERR_INVALID, "block_table is NULL");
  if (table_stride <= 0) return fail(KVQ_ERR_INVALID, "table_stride must be positive");
  if ((rows_needed + KVQ_PAGE_ROWS - 1) / KVQ_PAGE_ROWS > table_stride)
    return fail(KVQ_ERR_INVALID, "table_stride %lld pages cannot hold %lld rows", (long long)table_stride,
                (long long)rows_needed);
  return KVQ_OK;
}

// The address of this device's copy of `scratch`, looked up once per device (with the device
// current) by hipGetSymbolAddress; the first call on a device also zeroes its arrival counters on
// `stream` (every later call leaves them at zero).
constexpr int kMaxDevices = 64;
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

int static_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(KVQ_ERR_UNSUPPORTED, "device %d is beyond the %d the library tracks", dev, kMaxDevices);
  ScratchSlot& s = g_scratch[dev];
  std::call_once(s.once, [&] {
    void* p = nullptr;
    s.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (s.err != hipSuccess) return;
    const size_t words = kvq::kCounterBytes / 4;
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream, (uint32_t*)p, words);
    s.err = hipGetLastError();
    if (s.err == hipSuccess) s.ptr = p;
  });
  if (!s.ptr) return hip_status(s.err != hipSuccess ? s.err : hipErrorInvalidSymbol, "static scratch set-up");
  *out = s.ptr;
  return KVQ_OK;
}

int check_rope(const kvq_rope_params* r, int D) {
  if (!r) return fail(KVQ_ERR_INVALID, "rope descriptor is NULL");
  if (r->dims <= 0 || r->dims > D || r->dims > 256 || r->dims % 16)
    return fail(KVQ_ERR_UNSUPPORTED, "rope dims must be a positive multiple of 16, at most D=%d and 256, got %d", D,
                r->dims);
  if (!(r->base > 0.0f) || !isfinite(r->base)) return fail(KVQ_ERR_INVALID, "rope base must be positive and finite");
  if (!isfinite(r->scale)) return fail(KVQ_ERR_INVALID, "rope scale is not finite");
  if (r->offset < 0) return fail(KVQ_ERR_INVALID, "rope offset must be >= 0");
  return KVQ_OK;
}

}  // namespace

extern "C" {

int kvq_abi_version(void) { return KVQ_ABI_VERSION; }

const char* kvq_last_error(void) { return g_err; }

int kvq_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst, const kvq_rows* v_src,
                        const kvq_qtensor* v_dst, int64_t row_offset, int B, int H, int L, int D, int bits,
                        int group_size, int dtype, void* stream) {
  int rc;
  if ((rc = check_quantize(k_src, k_dst, v_src, v_dst, row_offset, B, H, L, D, bits, group_size, dtype))) return rc;
  if (B == 0 || H == 0 || L == 0) return ok();
  return hip_status(kvq::launch_quantize_append(k_src, k_dst, v_src, v_dst, nullptr, row_offset, B, H, L, D, bits,
                                                group_size, dtype, (hipStream_t)stream),
                    "quantize_append launch");
}

int kvq_rope(const kvq_rows* x, const kvq_rope_params* rope, int B, int H, int L, int D, int dtype, void* stream) {
  int rc;
  if ((rc = check_dtype(dtype))) return rc;
  if (B < 0 || H < 0 || L < 0 || D <= 0 || D % 8) return fail(KVQ_ERR_INVALID, "bad shape (B=%d H=%d L=%d D=%d)", B, H, L, D);
  if ((rc = check_rope(rope, D))) return rc;
  if ((rc = check_rows(x, "x", D, true))) return rc;
  if (B == 0 || H == 0 || L == 0) return ok();
  return hip_status(kvq::launch_rope(x, rope, B, H, L, dtype, (hipStream_t)stream), "rope launch");
}

int kvq_rope_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst, const kvq_rows* v_src,
                             const kvq_qtensor* v_dst, const kvq_rope_params* rope, int64_t row_offset, int B, int H, int L,
                             int D, int bits, int group_size, int dtype, void* stream) {
  int rc;
  if ((rc = check_rope(rope, D))) return rc;
  if ((rc = check_quantize(k_src, k_dst, v_src, v_dst, row_offset, B, H, L, D, bits, group_size, dtype))) return rc;
  if (B == 0 || H == 0 || L == 0) return ok();
  return hip_status(kvq::launch_quantize_append(k_src, k_dst, v_src, v_dst, rope, row_offset, B, H, L, D, bits,
                                                group_size, dtype, (hipStream_t)stream),
                    "rope_quantize_append launch");
}

int kvq_paged_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_pool, const kvq_rows* v_src,
                              const kvq_qtensor* v_pool, int num_pages, const int32_t* block_table,
                              int64_t table_stride, const int32_t* starts, int64_t row_offset,
                              const kvq_rope_params* rope, int B, int H, int L, int D, int bits, int group_size,
                              int dtype, void* stream) {
  int rc;
  if ((rc = check_quantize(k_src, k_pool, v_src, v_pool, row_offset, B, H, L, D, bits, group_size, dtype))) return rc;
  if ((rc = check_pool(k_pool, "k_pool", H, D, bits, group_size, num_pages))) return rc;
  if (v_pool && (rc = check_pool(v_pool, "v_pool", H, D, bits, group_size, num_pages))) return rc;
  if ((rc = check_table(block_table, table_stride, starts ? 1 : row_offset + L))) return rc;
  if (rope && (rc = check_rope(rope, D))) return rc;
  if (B == 0 || H == 0 || L == 0) return ok();
  return hip_status(kvq::launch_paged_quantize_append(k_src, k_pool, v_src, v_pool, num_pages, block_table, table_stride,
                                                      starts, row_offset, rope, B, H, L, D, bits, group_size, dtype,
                                                      (hipStream_t)stream),
                    "paged_quantize_append launch");
}

size_t kvq_decode_workspace_size(int B, int Hq, int Hkv, int L, int D, int S, int window) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || S <= 0 || D <= 0 || D > 256 || D % 8 || window < 0) return 0;
  // one size serves every cache format: the quantized (8-, 4-bit) and the unquantized (16) plans
  // and every scale-group size (the group sets the query rows per workgroup)
  const int Dk = kvq::decode_kernel_dim(D);
  size_t n = 0;
  for (int bits : {8, 4, 16})
    for (int G : {32, 64, 128}) {
      if (G > Dk || 4 * G < Dk || (bits == 16 && Dk > 128)) continue;
      const size_t x = kvq::decode_workspace_bytes(B, Hq, Hkv, L, D, S, window, bits, G);
      n = x > n ? x : n;
    }
  if (Dk == 256) {  // unquantized rows past 128 dims run through the head_dim-256 kernel
    const size_t x = kvq::wide_workspace_bytes(B, Hq, Hkv, L, Dk, S, window);
    n = x > n ? x : n;
  }
  return n;
}

int kvq_decode_attn(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                    const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size,
                    int dtype, float scale, int causal, int window, void* workspace, size_t workspace_bytes,
                    void* stream) {
  if (check_head_dim(D, "decode")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn(q, k, v, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, window,
                      kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, window), workspace, workspace_bytes);
  if (rc) return rc;
  return hip_status(kvq::launch_decode(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale,
                                       causal, window, workspace, (hipStream_t)stream),
                    "decode_attn launch");
}

int kvq_decode_attn_static(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                           const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size,
                           int dtype, float scale, int causal, int window, void* stream) {
  if (check_head_dim(D, "decode")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn_args(q, k, v, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, window);
  if (rc) return rc;
  // the scratch has to hold this call's own plan (its format and group size), not the largest plan
  // any cache format could need at these shapes
  const size_t need = kvq::decode_workspace_bytes(B, Hq, Hkv, L, D, S, window, bits, group_size);
  if (need > (size_t)KVQ_STATIC_SCRATCH_BYTES)
    return fail(KVQ_ERR_WORKSPACE, "this call needs %zu bytes of scratch; the static scratch holds %zu (use kvq_decode_attn "
                "with a workspace)", need, (size_t)KVQ_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = static_scratch((hipStream_t)stream, &ws))) return rc;
  return hip_status(kvq::launch_decode(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale,
                                       causal, window, ws, (hipStream_t)stream),
                    "decode_attn_static launch");
}

size_t kvq_prefill_workspace_size(int B, int Hq, int Hkv, int L, int D, int S, int window) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || S <= 0 || window < 0 || Hq % Hkv) return 0;
  if (!native_dim(D)) return kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, window);  // the decode kernel serves
  if (D == 256) return kvq::wide_workspace_bytes(B, Hq, Hkv, L, D, S, window);
  const size_t n = kvq::prefill_workspace_bytes(B, Hq, Hkv, L, D, S, window, 8);
  if (D == 64) {  // the unquantized cache at head_dim 64 runs through wide.hip's kernel
    const size_t x = kvq::wide_workspace_bytes(B, Hq, Hkv, L, D, S, window);
    return x > n ? x : n;
  }
  return n;
}

// The prefill kernel loads two scale groups of a row at once when a row has several: scale and
// bias rows then have to be 4-byte aligned.
static int check_prefill_sb(const kvq_qtensor* k, const kvq_qtensor* v, int D, int group_size) {
  if (D / group_size < 2) return KVQ_OK;
  for (const kvq_qtensor* t : {k, v})
    if (!aligned(t->scales, 4) || !aligned(t->biases, 4) || (t->sb_stride_s | t->sb_stride_h | t->sb_stride_b) & 1)
      return fail(KVQ_ERR_INVALID, "prefill with %d scale groups per row needs 4-byte aligned scales and biases with "
                  "even row, head and batch (page) strides", D / group_size);
  return KVQ_OK;
}

int kvq_prefill_attn(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                     const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size,
                     int dtype, float scale, int causal, int window, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (check_head_dim(D, "prefill")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn(q, k, v, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, window,
                      kvq_prefill_workspace_size(B, Hq, Hkv, L, D, S, window), workspace, workspace_bytes);
  if (rc) return rc;
  if (!native_dim(D))
    return hip_status(kvq::launch_decode(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale,
                                         causal, window, workspace, (hipStream_t)stream),
                      "prefill_attn launch (the decode kernel, head_dim other than 64/128/256)");
  if (D == 256)
    return hip_status(kvq::launch_wide(q, k, v, seq_lens, out, B, Hq, Hkv, L, S, bits, group_size, dtype, scale, causal,
                                       window, workspace, (hipStream_t)stream),
                      "prefill_attn launch (head_dim 256)");
  if ((rc = check_rows(out, "out", D, true))) return rc;  // rows are stored 16 bytes at a time
  if ((rc = check_prefill_sb(k, v, D, group_size))) return rc;
  return hip_status(kvq::launch_prefill(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale,
                                        causal, window, workspace, (hipStream_t)stream),
                    "prefill_attn launch");
}

// Attention over paged pools: the quantized checks with the pool geometry and the block table.
static int check_paged_attn(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                            const int32_t* table, int64_t table_stride, const kvq_rows* out, int B, int Hq, int Hkv,
                            int L, int D, int S, int bits, int group_size, int dtype, float scale, int window,
                            size_t ws_needed, void* workspace, size_t workspace_bytes) {
  int rc;
  if ((rc = check_attn_common(q, out, B, Hq, Hkv, L, D, S, dtype, scale, window))) return rc;
  if (bits != 4 && bits != 8) return fail(KVQ_ERR_UNSUPPORTED, "attention supports 4- and 8-bit caches, got bits=%d", bits);
  if ((rc = check_attn_group(group_size, D))) return rc;
  if ((rc = check_pool(k, "k_pool", Hkv, D, bits, group_size, num_pages))) return rc;
  if ((rc = check_pool(v, "v_pool", Hkv, D, bits, group_size, num_pages))) return rc;
  for (const kvq_qtensor* t : {k, v})
    if (!aligned(t->codes, 16) || (t->codes_stride_s * 4) % 16 || (t->codes_stride_h * 4) % 16 || (t->codes_stride_b * 4) % 16)
      return fail(KVQ_ERR_INVALID, "codes must be 16-byte aligned with 16-byte-multiple row, head and page strides");
  if ((rc = check_table(table, table_stride, S))) return rc;
  return check_workspace(ws_needed, workspace, workspace_bytes);
}

int kvq_paged_decode_attn(const kvq_rows* q, const kvq_qtensor* k_pool, const kvq_qtensor* v_pool, int num_pages,
                          const int32_t* block_table, int64_t table_stride, const int32_t* seq_lens,
                          const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size,
                          int dtype, float scale, int causal, int window, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (check_head_dim(D, "decode")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_paged_attn(q, k_pool, v_pool, num_pages, block_table, table_stride, out, B, Hq, Hkv, L, D, S, bits,
                            group_size, dtype, scale, window, kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, window),
                            workspace, workspace_bytes);
  if (rc) return rc;
  return hip_status(kvq::launch_decode_paged(q, k_pool, v_pool, num_pages, block_table, table_stride, seq_lens, out, B,
                                             Hq, Hkv, L, D, S, bits, group_size, dtype, scale, causal, window,
                                             workspace, (hipStream_t)stream),
                    "paged_decode_attn launch");
}

int kvq_paged_prefill_attn(const kvq_rows* q, const kvq_qtensor* k_pool, const kvq_qtensor* v_pool, int num_pages,
                           const int32_t* block_table, int64_t table_stride, const int32_t* seq_lens,
                           const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int group_size,
                           int dtype, float scale, int causal, int window, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (check_head_dim(D, "prefill")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_paged_attn(q, k_pool, v_pool, num_pages, block_table, table_stride, out, B, Hq, Hkv, L, D, S, bits,
                            group_size, dtype, scale, window, kvq_prefill_workspace_size(B, Hq, Hkv, L, D, S, window),
                            workspace, workspace_bytes);
  if (rc) return rc;
  if (!native_dim(D))
    return hip_status(kvq::launch_decode_paged(q, k_pool, v_pool, num_pages, block_table, table_stride, seq_lens, out,
                                               B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, causal, window,
                                               workspace, (hipStream_t)stream),
                      "paged_prefill_attn launch (the decode kernel, head_dim other than 64/128/256)");
  if (D == 256)
    return hip_status(kvq::launch_wide_paged(q, k_pool, v_pool, num_pages, block_table, table_stride, seq_lens, out, B,
                                             Hq, Hkv, L, S, bits, group_size, dtype, scale, causal, window, workspace,
                                             (hipStream_t)stream),
                      "paged_prefill_attn launch (head_dim 256)");
  if ((rc = check_rows(out, "out", D, true))) return rc;  // rows are stored 16 bytes at a time
  if ((rc = check_prefill_sb(k_pool, v_pool, D, group_size))) return rc;
  return hip_status(kvq::launch_prefill_paged(q, k_pool, v_pool, num_pages, block_table, table_stride, seq_lens, out, B,
                                              Hq, Hkv, L, D, S, bits, group_size, dtype, scale, causal, window,
                                              workspace, (hipStream_t)stream),
                    "paged_prefill_attn launch");
}

int kvq_decode_attn_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                          const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype, float scale,
                          int causal, int window, void* workspace, size_t workspace_bytes, void* stream) {
  if (check_head_dim(D, "unquantized decode")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn_dense(q, k, v, out, B, Hq, Hkv, L, D, S, dtype, scale, window,
                            kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, window), workspace, workspace_bytes);
  if (rc) return rc;
  if (D > 128)
    return hip_status(kvq::launch_wide_dense(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, dtype, scale, causal, window,
                                             workspace, (hipStream_t)stream),
                      "decode_attn_dense launch (the head_dim-256 kernel)");
  return hip_status(kvq::launch_decode_dense(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, dtype, scale, causal, window,
                                             workspace, (hipStream_t)stream),
                    "decode_attn_dense launch");
}

// A general mask: a known kind, a pointer aligned to its element, non-negative strides (the key
// stride is 1 by definition).
static int check_mask(const kvq_mask* m) {
  if (!m || !m->data) return fail(KVQ_ERR_INVALID, "mask and mask->data must not be NULL");
  if (m->kind < KVQ_MASK_BOOL || m->kind > KVQ_MASK_F32) return fail(KVQ_ERR_INVALID, "unknown mask kind %d", m->kind);
  const uintptr_t el = m->kind == KVQ_MASK_BOOL ? 1 : m->kind == KVQ_MASK_F32 ? 4 : 2;
  if (!aligned(m->data, el)) return fail(KVQ_ERR_INVALID, "mask data is not aligned to its %zu-byte elements", (size_t)el);
  if (m->stride_b < 0 || m->stride_kvh < 0 || m->stride_rep < 0 || m->stride_l < 0)
    return fail(KVQ_ERR_INVALID, "mask strides must be non-negative");
  return KVQ_OK;
}

int kvq_decode_attn_masked(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const kvq_rows* out, int B,
                           int Hq, int Hkv, int L, int D, int S, int bits, int group_size, int dtype, float scale,
                           const kvq_mask* mask, void* workspace, size_t workspace_bytes, void* stream) {
  if (check_head_dim(D, "decode")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn(q, k, v, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, 0,
                      kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, 0), workspace, workspace_bytes);
  if (rc || (rc = check_mask(mask))) return rc;
  return hip_status(kvq::launch_decode(q, k, v, nullptr, out, B, Hq, Hkv, L, D, S, bits, group_size, dtype, scale, 0, 0,
                                       workspace, (hipStream_t)stream, mask),
                    "decode_attn_masked launch");
}

int kvq_decode_attn_dense_masked(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const kvq_rows* out, int B,
                                 int Hq, int Hkv, int L, int D, int S, int dtype, float scale, const kvq_mask* mask,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  if (check_head_dim(D, "masked unquantized attention")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn_dense(q, k, v, out, B, Hq, Hkv, L, D, S, dtype, scale, 0,
                            kvq_decode_workspace_size(B, Hq, Hkv, L, D, S, 0), workspace, workspace_bytes);
  if (rc || (rc = check_mask(mask))) return rc;
  if (D > 128)  // unquantized rows past 128 dims run through the head_dim-256 kernel
    return hip_status(kvq::launch_wide_dense(q, k, v, nullptr, out, B, Hq, Hkv, L, D, S, dtype, scale, 0, 0, workspace,
                                             (hipStream_t)stream, mask),
                      "decode_attn_dense_masked launch (the head_dim-256 kernel)");
  return hip_status(kvq::launch_decode_dense(q, k, v, nullptr, out, B, Hq, Hkv, L, D, S, dtype, scale, 0, 0, workspace,
                                             (hipStream_t)stream, mask),
                    "decode_attn_dense_masked launch");
}

int kvq_prefill_attn_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                           const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype, float scale,
                           int causal, int window, void* workspace, size_t workspace_bytes, void* stream) {
  if (check_head_dim(D, "unquantized prefill")) return KVQ_ERR_UNSUPPORTED;
  int rc = check_attn_dense(q, k, v, out, B, Hq, Hkv, L, D, S, dtype, scale, window,
                            kvq_prefill_workspace_size(B, Hq, Hkv, L, D, S, window), workspace, workspace_bytes);
  if (rc) return rc;
  if (D > 128 && D < 256)
    return hip_status(kvq::launch_wide_dense(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, dtype, scale, causal, window,
                                             workspace, (hipStream_t)stream),
                      "prefill_attn_dense launch (the head_dim-256 kernel)");
  if (!native_dim(D))
    return hip_status(kvq::launch_decode_dense(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, dtype, scale, causal, window,
                                               workspace, (hipStream_t)stream),
                      "prefill_attn_dense launch (the decode kernel, head_dim other than 64/128/256)");
  if (D != 128)
    return hip_status(kvq::launch_wide_dense(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, dtype, scale, causal, window,
                                             workspace, (hipStream_t)stream),
                      "prefill_attn_dense launch (head_dim 64 / 256)");
  if ((rc = check_rows(out, "out", D, true))) return rc;  // rows are stored 16 bytes at a time
  return hip_status(kvq::launch_prefill_dense(q, k, v, seq_lens, out, B, Hq, Hkv, L, D, S, dtype, scale, causal, window,
                                              workspace, (hipStream_t)stream),
                    "prefill_attn_dense launch");
}

}  // extern "C"
