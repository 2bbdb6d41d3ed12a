// Fused quantize-and-append: new K/V rows -> MLX-layout affine cache (codes, scales, biases).
//
// Algorithm (per group of G consecutive elements of a row), the affine quantizer of
// mx.quantize that mlx-lm's QuantizedKVCache.update_and_fetch applies to every appended row
// (reached from m5engine/attention.py:106-112 and the per-layer cache update):
//   xmax, xmin over the group in fp32; n = 2^bits - 1
//   s = max((xmax - xmin) / n, 1e-7), negated unless |xmin| > |xmax|
//   edge = |xmin| > |xmax| ? xmin : xmax;  q0 = rint(edge / s)
//   if q0 != 0: s = edge / q0, bias = edge   else bias = 0
//   code = clamp(rint((x - bias) / s), 0, n)          (fp32 s and bias, before rounding)
//   stored scale = T(s), bias = T(bias)               (round to nearest even)
// Every operation is IEEE fp32 with round-to-nearest-even (correctly rounded division, rint
// half-to-even), so codes, scales and biases are bit-identical to the CPU restatement.
//
// Thread mapping: one thread per 8 consecutive elements (one 16-byte load); the G/8 threads of a
// group reduce min/max with lane permutes. Grid.y selects the K or the V job of one launch.

#include "common.h"
#include "launch.h"

namespace kvq {

struct QuantJob {
  const uint16_t* src;
  int64_t s_b, s_h, s_l;
  uint32_t* codes;
  uint16_t* scales;
  uint16_t* biases;
  int64_t c_b, c_h, c_s;
  int64_t g_b, g_h, g_s;
};

template <typename T, int BITS, int G>
__global__ __launch_bounds__(256) void quantize_append_kernel(QuantJob job0, QuantJob job1, int H, int L,
                                                              int D, int64_t total, int64_t row_offset) {
#pragma clang fp contract(off)
  const QuantJob job = blockIdx.y == 0 ? job0 : job1;
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool active = tid < total;
  const int per_row = D / 8;
  const int64_t t = active ? tid : 0;
  const int chunk = (int)(t % per_row);
  const int64_t row = t / per_row;
  const int l = (int)(row % L);
  const int h = (int)((row / L) % H);
  const int64_t b = row / ((int64_t)L * H);

  const uint16_t* src = job.src + b * job.s_b + h * job.s_h + (int64_t)l * job.s_l + chunk * 8;
  u4 raw = *(const u4*)src;
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = to_float((uint16_t)(raw[i] & 0xffffu), T{});
    x[2 * i + 1] = to_float((uint16_t)(raw[i] >> 16), T{});
  }
  float mx = x[0], mn = x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mx = fmaxf(mx, x[i]);
    mn = fminf(mn, x[i]);
  }
#pragma unroll
  for (int off = 1; off < G / 8; off <<= 1) {
    mx = fmaxf(mx, shfl_xor(mx, off));
    mn = fminf(mn, shfl_xor(mn, off));
  }
  if (!active) return;

  constexpr float n_bins = (float)((1 << BITS) - 1);
  const bool neg = fabsf(mn) > fabsf(mx);
  float s = fmaxf((mx - mn) / n_bins, 1e-7f);
  s = neg ? s : -s;
  const float edge = neg ? mn : mx;
  const float q0 = rintf(edge / s);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    s = edge / q0;
    bias = edge;
  }

  uint32_t packed[BITS] = {};  // 8 codes * BITS bits = BITS bytes -> BITS/4 words (at least 1)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float c = rintf((x[i] - bias) / s);
    c = fminf(fmaxf(c, 0.0f), n_bins);
    const uint32_t code = (uint32_t)c;
    const int bit = i * BITS;
    packed[bit / 32] |= code << (bit % 32);
  }

  const int64_t drow = row_offset + l;
  uint32_t* cdst = job.codes + b * job.c_b + h * job.c_h + drow * job.c_s;
  if constexpr (BITS == 8) {
    *(u2*)(cdst + chunk * 2) = u2{packed[0], packed[1]};
  } else if constexpr (BITS == 4) {
    cdst[chunk] = packed[0];
  } else {  // 2-bit: 8 codes fill 16 bits; two neighbouring threads share a word
    const uint32_t other = (uint32_t)__builtin_amdgcn_ds_bpermute((__lane_id() ^ 1) << 2, (int)packed[0]);
    if ((chunk & 1) == 0) cdst[chunk / 2] = packed[0] | (other << 16);
  }
  if (chunk % (G / 8) == 0) {
    const int64_t gi = b * job.g_b + h * job.g_h + drow * job.g_s + chunk / (G / 8);
    job.scales[gi] = from_float(s, T{});
    job.biases[gi] = from_float(bias, T{});
  }
}

template <typename T, int BITS, int G>
static hipError_t launch_quant(const QuantJob& k, const QuantJob& v, int njobs, int B, int H, int L, int D,
                               int64_t row_offset, hipStream_t stream) {
  const int64_t total = (int64_t)B * H * L * (D / 8);
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G>), dim3((unsigned)blocks, njobs), dim3(256), 0, stream, k,
                     v, H, L, D, total, row_offset);
  return hipGetLastError();
}

template <typename T, int BITS>
static hipError_t dispatch_group(int G, const QuantJob& k, const QuantJob& v, int njobs, int B, int H, int L, int D,
                                 int64_t row_offset, hipStream_t stream) {
  switch (G) {
    case 32: return launch_quant<T, BITS, 32>(k, v, njobs, B, H, L, D, row_offset, stream);
    case 64: return launch_quant<T, BITS, 64>(k, v, njobs, B, H, L, D, row_offset, stream);
    default: return launch_quant<T, BITS, 128>(k, v, njobs, B, H, L, D, row_offset, stream);
  }
}

template <typename T>
static hipError_t dispatch_bits(int bits, int G, const QuantJob& k, const QuantJob& v, int njobs, int B, int H, int L,
                                int D, int64_t row_offset, hipStream_t stream) {
  switch (bits) {
    case 2: return dispatch_group<T, 2>(G, k, v, njobs, B, H, L, D, row_offset, stream);
    case 4: return dispatch_group<T, 4>(G, k, v, njobs, B, H, L, D, row_offset, stream);
    default: return dispatch_group<T, 8>(G, k, v, njobs, B, H, L, D, row_offset, stream);
  }
}

static QuantJob make_job(const kvq_rows* src, const kvq_qtensor* dst) {
  QuantJob j;
  j.src = (const uint16_t*)src->data;
  j.s_b = src->stride_b;
  j.s_h = src->stride_h;
  j.s_l = src->stride_l;
  j.codes = dst->codes;
  j.scales = (uint16_t*)dst->scales;
  j.biases = (uint16_t*)dst->biases;
  j.c_b = dst->codes_stride_b;
  j.c_h = dst->codes_stride_h;
  j.c_s = dst->codes_stride_s;
  j.g_b = dst->sb_stride_b;
  j.g_h = dst->sb_stride_h;
  j.g_s = dst->sb_stride_s;
  return j;
}

hipError_t launch_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst, const kvq_rows* v_src,
                                  const kvq_qtensor* v_dst, int64_t row_offset, int B, int H, int L, int D, int bits,
                                  int group_size, int dtype, hipStream_t stream) {
  QuantJob k = make_job(k_src, k_dst);
  QuantJob v = v_src ? make_job(v_src, v_dst) : k;
  const int njobs = v_src ? 2 : 1;
  if (dtype == KVQ_DTYPE_BF16) return dispatch_bits<BF16>(bits, group_size, k, v, njobs, B, H, L, D, row_offset, stream);
  return dispatch_bits<F16>(bits, group_size, k, v, njobs, B, H, L, D, row_offset, stream);
}

}  // namespace kvq
