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
//
// RoPE (kvq_rope_quantize_append): the K job rotates its rows before quantizing, the way mlx-lm's
// attention layers rotate keys before the cache update and the reference's native kernel fuses
// the rotation with the KV write (native/src/kernels.metal:106-160). Pair i of a row at position
// p turns by angle = (p * scale) * freq_i, freq_i = 1 / base^(2i / dims), in fp32; the rotated
// value is rounded to T (what RoPE returns) before it is quantized. NeoX pairs (i, i + dims/2)
// are read by each thread from its own chunk and the partner chunk, so no lanes exchange data.

#include "common.h"
#include "launch.h"

namespace kvq {

constexpr int kMaxRopePairs = 128;

// freq[i] = 1 / base^(2i / dims), computed once on the host in double precision and rounded to
// fp32, so that the angles do not depend on the device's pow (at position 1e5 one ulp of freq
// moves the angle by about 6e-3 rad).
struct RopeArgs {
  int dims, traditional;
  float scale;
  int64_t offset;
  float freq[kMaxRopePairs];
};

// cos and sin of the angle of pair `pair` at position `pos`
__device__ __forceinline__ void rope_cs(const RopeArgs& r, int64_t pos, int pair, float& c, float& s) {
#pragma clang fp contract(off)
  const float ang = ((float)pos * r.scale) * r.freq[pair];
  sincosf(ang, &s, &c);
}

static RopeArgs make_rope_args(const kvq_rope_params* p) {
  RopeArgs r{};
  r.dims = p->dims;
  r.traditional = p->traditional;
  r.scale = p->scale;
  r.offset = p->offset;
  for (int i = 0; i < p->dims / 2 && i < kMaxRopePairs; ++i)
    r.freq[i] = (float)(1.0 / pow((double)p->base, 2.0 * i / (double)p->dims));
  return r;
}

// Rotate the 8 values x of dims [d0, d0 + 8) of a row at position pos. For NeoX pairs, xp holds
// the 8 values at the partner dims (d0 -+ dims/2). Dims at or past r.dims pass through.
__device__ __forceinline__ void rope8(const RopeArgs& r, int64_t pos, int d0, float (&x)[8], const float (&xp)[8]) {
#pragma clang fp contract(off)
  if (d0 >= r.dims) return;
  if (r.traditional) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float c, sn;
      rope_cs(r, pos, d0 / 2 + i, c, sn);
      const float a = x[2 * i], b = x[2 * i + 1];
      x[2 * i] = a * c - b * sn;
      x[2 * i + 1] = a * sn + b * c;
    }
  } else {
    const int half = r.dims / 2;
    const bool lo = d0 < half;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float c, sn;
      rope_cs(r, pos, (lo ? d0 : d0 - half) + e, c, sn);
      x[e] = lo ? x[e] * c - xp[e] * sn : x[e] * c + xp[e] * sn;
    }
  }
}

template <typename T>
__device__ __forceinline__ void load8(const uint16_t* p, float (&x)[8]) {
  const u4 raw = *(const u4*)p;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = to_float((uint16_t)(raw[i] & 0xffffu), T{});
    x[2 * i + 1] = to_float((uint16_t)(raw[i] >> 16), T{});
  }
}

struct QuantJob {
  const uint16_t* src;
  int64_t s_b, s_h, s_l;
  uint32_t* codes;
  uint16_t* scales;
  uint16_t* biases;
  int64_t c_b, c_h, c_s;
  int64_t g_b, g_h, g_s;
  int32_t* range_exp;  // the destination cache's range exponent (kvq_qtensor), or null
};

// The range exponent a group needs: the smallest E >= 0 with max(|b|, |b + n s|) <= 2^15 * 2^E,
// from the stored (rounded) scale and bias, whose dequantized values s * c + b (c in [0, n]) have
// their extremes at c = 0 and c = n.
__device__ __forceinline__ int group_range_exp(float s, float b, float n) {
#pragma clang fp contract(off)
  const float bound = fmaxf(fabsf(b), fabsf(b + n * s));
  if (!(bound > 32768.0f)) return 0;           // within range (or a NaN group, which no scale mends)
  if (__builtin_isinf(bound)) return 127;      // the largest exponent the kernels accept
  int k;
  const float m = frexpf(bound * (1.0f / 32768.0f), &k);  // bound / 2^15 = m 2^k, m in [0.5, 1)
  return m == 0.5f ? k - 1 : k;
}

// Paged destination: row r of sequence b goes to row r % 64 of page table[b][r / 64] (the job's
// batch strides are then page strides); r = starts[b] + l when `starts` is given, else
// row_offset + l. table == nullptr: the contiguous cache.
struct PageMap {
  const int32_t* table;
  int64_t table_stride;
  const int32_t* starts;
  int num_pages;
};

template <typename T, int BITS, int G, bool ROPE>
__global__ __launch_bounds__(256) void quantize_append_kernel(QuantJob job0, QuantJob job1, int H, int L,
                                                              int D, int64_t total, int64_t row_offset, RopeArgs rope,
                                                              PageMap pm) {
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

  const uint16_t* srow = job.src + b * job.s_b + h * job.s_h + (int64_t)l * job.s_l;
  float x[8];
  load8<T>(srow + chunk * 8, x);
  if constexpr (ROPE) {
    if (blockIdx.y == 0) {  // the K job
      const int d0 = chunk * 8, half = rope.dims / 2;
      float xp[8];
      if (!rope.traditional && d0 < rope.dims) load8<T>(srow + (d0 < half ? d0 + half : d0 - half), xp);
      rope8(rope, rope.offset + (pm.starts ? pm.starts[b] : 0) + l, d0, x, xp);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = to_float(from_float(x[i], T{}), T{});
    }
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

  int64_t drow = row_offset + l, bb = b;
  if (pm.table) {
    const int64_t r = (pm.starts ? (int64_t)pm.starts[b] : row_offset) + l;
    if (r < 0 || (r >> 6) >= pm.table_stride) return;  // a row outside the sequence's table is dropped
    // A table entry outside the pool (such as a -1 "unallocated" sentinel) drops the row too:
    // clamping it would write into a page that may belong to another sequence.
    const int pg = pm.table[b * pm.table_stride + (r >> 6)];
    if (pg < 0 || pg >= pm.num_pages) return;
    bb = pg;
    drow = r & 63;
  }
  uint32_t* cdst = job.codes + bb * job.c_b + h * job.c_h + drow * job.c_s;
  if constexpr (BITS == 8) {
    *(u2*)(cdst + chunk * 2) = u2{packed[0], packed[1]};
  } else if constexpr (BITS == 4) {
    cdst[chunk] = packed[0];
  } else {  // 2-bit: 8 codes fill 16 bits; two neighbouring threads share a word
    const uint32_t other = (uint32_t)__builtin_amdgcn_ds_bpermute((__lane_id() ^ 1) << 2, (int)packed[0]);
    if ((chunk & 1) == 0) cdst[chunk / 2] = packed[0] | (other << 16);
  }
  if (chunk % (G / 8) == 0) {
    const int64_t gi = bb * job.g_b + h * job.g_h + drow * job.g_s + chunk / (G / 8);
    const uint16_t sT = from_float(s, T{}), bT = from_float(bias, T{});
    job.scales[gi] = sT;
    job.biases[gi] = bT;
    if (job.range_exp) {
      const int e = group_range_exp(to_float(sT, T{}), to_float(bT, T{}), n_bins);
      if (e > 0) atomicMax(job.range_exp, e);
    }
  }
}

template <typename T, int BITS, int G>
static hipError_t launch_quant(const QuantJob& k, const QuantJob& v, int njobs, int B, int H, int L, int D,
                               int64_t row_offset, const RopeArgs* rope, const PageMap& pm, hipStream_t stream) {
  const int64_t total = (int64_t)B * H * L * (D / 8);
  const int64_t blocks = (total + 255) / 256;
  if (rope)
    hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G, true>), dim3((unsigned)blocks, njobs), dim3(256), 0, stream,
                       k, v, H, L, D, total, row_offset, *rope, pm);
  else
    hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G, false>), dim3((unsigned)blocks, njobs), dim3(256), 0,
                       stream, k, v, H, L, D, total, row_offset, RopeArgs{}, pm);
  return hipGetLastError();
}

template <typename T, int BITS>
static hipError_t dispatch_group(int G, const QuantJob& k, const QuantJob& v, int njobs, int B, int H, int L, int D,
                                 int64_t row_offset, const RopeArgs* rope, const PageMap& pm, hipStream_t stream) {
  switch (G) {
    case 32: return launch_quant<T, BITS, 32>(k, v, njobs, B, H, L, D, row_offset, rope, pm, stream);
    case 64: return launch_quant<T, BITS, 64>(k, v, njobs, B, H, L, D, row_offset, rope, pm, stream);
    default: return launch_quant<T, BITS, 128>(k, v, njobs, B, H, L, D, row_offset, rope, pm, stream);
  }
}

template <typename T>
static hipError_t dispatch_bits(int bits, int G, const QuantJob& k, const QuantJob& v, int njobs, int B, int H, int L,
                                int D, int64_t row_offset, const RopeArgs* rope, const PageMap& pm, hipStream_t stream) {
  switch (bits) {
    case 2: return dispatch_group<T, 2>(G, k, v, njobs, B, H, L, D, row_offset, rope, pm, stream);
    case 4: return dispatch_group<T, 4>(G, k, v, njobs, B, H, L, D, row_offset, rope, pm, stream);
    default: return dispatch_group<T, 8>(G, k, v, njobs, B, H, L, D, row_offset, rope, pm, stream);
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
  j.range_exp = dst->range_exp;
  return j;
}

hipError_t launch_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_dst, const kvq_rows* v_src,
                                  const kvq_qtensor* v_dst, const kvq_rope_params* rope, int64_t row_offset, int B, int H,
                                  int L, int D, int bits, int group_size, int dtype, hipStream_t stream) {
  QuantJob k = make_job(k_src, k_dst);
  QuantJob v = v_src ? make_job(v_src, v_dst) : k;
  const int njobs = v_src ? 2 : 1;
  RopeArgs ra{};
  if (rope) ra = make_rope_args(rope);
  const RopeArgs* rp = rope ? &ra : nullptr;
  const PageMap pm{nullptr, 0, nullptr, 0};
  if (dtype == KVQ_DTYPE_BF16)
    return dispatch_bits<BF16>(bits, group_size, k, v, njobs, B, H, L, D, row_offset, rp, pm, stream);
  return dispatch_bits<F16>(bits, group_size, k, v, njobs, B, H, L, D, row_offset, rp, pm, stream);
}

hipError_t launch_paged_quantize_append(const kvq_rows* k_src, const kvq_qtensor* k_pool, const kvq_rows* v_src,
                                        const kvq_qtensor* v_pool, int num_pages, const int32_t* table,
                                        int64_t table_stride, const int32_t* starts, int64_t row_offset,
                                        const kvq_rope_params* rope, int B, int H, int L, int D, int bits,
                                        int group_size, int dtype, hipStream_t stream) {
  QuantJob k = make_job(k_src, k_pool);
  QuantJob v = v_src ? make_job(v_src, v_pool) : k;
  const int njobs = v_src ? 2 : 1;
  RopeArgs ra{};
  if (rope) ra = make_rope_args(rope);
  const RopeArgs* rp = rope ? &ra : nullptr;
  const PageMap pm{table, table_stride, starts, num_pages};
  if (dtype == KVQ_DTYPE_BF16)
    return dispatch_bits<BF16>(bits, group_size, k, v, njobs, B, H, L, D, row_offset, rp, pm, stream);
  return dispatch_bits<F16>(bits, group_size, k, v, njobs, B, H, L, D, row_offset, rp, pm, stream);
}

// In-place RoPE: one thread per rotated pair of 8-value chunks (NeoX: dims [8j, +8) and
// [8j + dims/2, +8); interleaved: one chunk), so no thread reads what another writes.
template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(uint16_t* x, int64_t s_b, int64_t s_h, int64_t s_l, int H, int L,
                                                   int64_t total, int per_row, RopeArgs r) {
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (tid >= total) return;
  const int j = (int)(tid % per_row);
  const int64_t row = tid / per_row;
  const int l = (int)(row % L), h = (int)((row / L) % H);
  const int64_t b = row / ((int64_t)L * H);
  uint16_t* xr = x + b * s_b + h * s_h + (int64_t)l * s_l;
  const int64_t pos = r.offset + l;
  auto store8 = [&](uint16_t* p, const float (&v)[8]) {
    u4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)from_float(v[2 * i], T{}) | ((uint32_t)from_float(v[2 * i + 1], T{}) << 16);
    *(u4*)p = w;
  };
  float a[8], c[8];
  if (r.traditional) {
    load8<T>(xr + 8 * j, a);
    rope8(r, pos, 8 * j, a, c);
    store8(xr + 8 * j, a);
  } else {
    const int half = r.dims / 2;
    load8<T>(xr + 8 * j, a);
    load8<T>(xr + 8 * j + half, c);
    float a2[8], c2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a2[i] = a[i];
      c2[i] = c[i];
    }
    rope8(r, pos, 8 * j, a2, c);         // first half: a * cos - c * sin
    rope8(r, pos, 8 * j + half, c2, a);  // second half: c * cos + a * sin
    store8(xr + 8 * j, a2);
    store8(xr + 8 * j + half, c2);
  }
}

hipError_t launch_rope(const kvq_rows* x, const kvq_rope_params* rope, int B, int H, int L, int dtype, hipStream_t stream) {
  const RopeArgs r = make_rope_args(rope);
  const int per_row = rope->traditional ? rope->dims / 8 : rope->dims / 16;
  const int64_t total = (int64_t)B * H * L * per_row;
  const int64_t blocks = (total + 255) / 256;
  if (dtype == KVQ_DTYPE_BF16)
    hipLaunchKernelGGL((rope_kernel<BF16>), dim3((unsigned)blocks), dim3(256), 0, stream, (uint16_t*)x->data,
                       x->stride_b, x->stride_h, x->stride_l, H, L, total, per_row, r);
  else
    hipLaunchKernelGGL((rope_kernel<F16>), dim3((unsigned)blocks), dim3(256), 0, stream, (uint16_t*)x->data,
                       x->stride_b, x->stride_h, x->stride_l, H, L, total, per_row, r);
  return hipGetLastError();
}

}  // namespace kvq
