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
// Thread mapping: one thread per 32 (large launches) or 8 consecutive elements, 16 bytes a load, all
// loads in flight at once; the threads of a group are neighbouring lanes and reduce min/max with
// DPP lane permutes. Grid.y selects the K or the V job of one launch.
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

// The rows [l0, l0 + L) of every (sequence, head) in one launch: thread t quantizes chunk
// t % per_row of row t / per_row (per_row = D / EPT), rows ordered (b, h, l); total < 2^31.
struct RowMap {
  uint32_t total, L, H, per_row;
  Div31 div_c, div_l, div_h;
  int64_t l0;
};

// Paged destination: row r of sequence b goes to row r % 64 of page table[b][r / 64] (the job's
// batch strides are then page strides); r = starts[b] + l when `starts` is given, else
// row_offset + l. table == nullptr: the contiguous cache.
struct PageMap {
  const int32_t* table;
  int64_t table_stride;
  const int32_t* starts;
  int num_pages;
};

// v of another lane by a DPP lane permutation: quad_perm [1, 0, 3, 2] and [2, 3, 0, 1] (the lane
// index XOR 1 and XOR 2), row_half_mirror (lane 7 - i of each 8) and row_mirror (15 - i of each 16)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kHalfMirror = 0x141, kMirror = 0x140;

// Max and min over the TPG neighbouring lanes of a group (TPG a power of two up to 16): after the
// quad steps every lane of a quad holds its quad's value, so the mirrors exchange whole quads, then
// whole 8-lane halves.
template <int TPG>
__device__ __forceinline__ void group_minmax(float& mx, float& mn) {
  if constexpr (TPG >= 2) {
    mx = fmaxf(mx, dpp<kQuadXor1>(mx));
    mn = fminf(mn, dpp<kQuadXor1>(mn));
  }
  if constexpr (TPG >= 4) {
    mx = fmaxf(mx, dpp<kQuadXor2>(mx));
    mn = fminf(mn, dpp<kQuadXor2>(mn));
  }
  if constexpr (TPG >= 8) {
    mx = fmaxf(mx, dpp<kHalfMirror>(mx));
    mn = fminf(mn, dpp<kHalfMirror>(mn));
  }
  if constexpr (TPG >= 16) {
    mx = fmaxf(mx, dpp<kMirror>(mx));
    mn = fminf(mn, dpp<kMirror>(mn));
  }
}

// EPT elements per thread (EPT / 8 16-byte loads in flight): 32 for launches large enough to fill
// the GPU several times over (fewer instructions per element), 8 for small, latency-bound ones.
template <typename T, int BITS, int G, bool ROPE, int EPT>
__global__ __launch_bounds__(256) void quantize_append_kernel(QuantJob job0, QuantJob job1, RowMap rm,
                                                              int64_t row_offset, RopeArgs rope, PageMap pm) {
#pragma clang fp contract(off)
  constexpr int kEPT = EPT;
  constexpr int TPG = G / kEPT;  // threads per group: neighbouring lanes
  const QuantJob job = blockIdx.y == 0 ? job0 : job1;
  const uint32_t tid = blockIdx.x * 256u + threadIdx.x;
  const bool active = tid < rm.total;
  const uint32_t t = active ? tid : 0u;
  const uint32_t row = div31(t, rm.div_c);
  const int chunk = (int)(t - row * rm.per_row);
  const uint32_t bh = div31(row, rm.div_l);
  const int64_t l = rm.l0 + (int64_t)(row - bh * rm.L);  // the row's position among the appended rows
  const uint32_t b32 = div31(bh, rm.div_h);
  const int h = (int)(bh - b32 * rm.H);
  const int64_t b = b32;

  const uint16_t* srow = job.src + b * job.s_b + h * job.s_h + l * job.s_l;
  float x[kEPT];
  {
    u4 raw[kEPT / 8];  // every load in flight before any conversion
#pragma unroll
    for (int j = 0; j < kEPT / 8; ++j) raw[j] = *(const u4*)(srow + chunk * kEPT + 8 * j);
#pragma unroll
    for (int j = 0; j < kEPT / 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[8 * j + 2 * i] = to_float((uint16_t)(raw[j][i] & 0xffffu), T{});
        x[8 * j + 2 * i + 1] = to_float((uint16_t)(raw[j][i] >> 16), T{});
      }
  }
  if constexpr (ROPE) {
    if (blockIdx.y == 0) {  // the K job
      const int half = rope.dims / 2;
      const int64_t pos = rope.offset + (pm.starts ? pm.starts[b] : 0) + l;
#pragma unroll
      for (int j = 0; j < kEPT / 8; ++j) {
        const int d0 = chunk * kEPT + 8 * j;
        float xs[8], xp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xs[i] = x[8 * j + i];
        if (!rope.traditional && d0 < rope.dims) load8<T>(srow + (d0 < half ? d0 + half : d0 - half), xp);
        rope8(rope, pos, d0, xs, xp);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[8 * j + i] = to_float(from_float(xs[i], T{}), T{});
      }
    }
  }
  float mx = x[0], mn = x[0];
#pragma unroll
  for (int i = 1; i < kEPT; ++i) {
    mx = fmaxf(mx, x[i]);
    mn = fminf(mn, x[i]);
  }
  group_minmax<TPG>(mx, mn);
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

  // code = rint((x - bias) / s) with the quotient rounded as the IEEE division rounds it. The
  // reciprocal estimate (v_rcp_f32, within 1 ulp) refined by one residual step gives q1 within one
  // ulp of that correctly rounded quotient, so rint(q1) can differ from its rint only when a
  // half-integer lies within one ulp. A thread with any quotient within 2 ulp (|q1| 2^-22) of a
  // half-integer, or of magnitude 2^21 or more, or not finite, divides all its elements exactly:
  // the codes stay bit-identical and the division is the rare path.
  constexpr int W = kEPT * BITS / 32 > 0 ? kEPT * BITS / 32 : 1;  // code words per thread (2-bit, 8 elements: half a word)
  uint32_t packed[W];
  auto put = [&](int i, float c) {
    c = fminf(fmaxf(c, 0.0f), n_bins);
    const int bit = i * BITS;
    if (bit % 32 == 0) packed[bit / 32] = 0u;
    packed[bit / 32] |= (uint32_t)c << (bit % 32);
  };
  const float rs = __builtin_amdgcn_rcpf(s);
  bool exact = false;
#pragma unroll
  for (int i = 0; i < kEPT; ++i) {
    const float a = x[i] - bias;
    const float qa = a * rs;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-qa, s, a), rs, qa);
    const float c = rintf(q1);
    exact |= !(fabsf(q1 - c) < __builtin_fmaf(fabsf(q1), -0x1p-22f, 0.5f));
    put(i, c);
  }
  if (exact) {
#pragma unroll
    for (int i = 0; i < kEPT; ++i) put(i, rintf((x[i] - bias) / s));
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
  if constexpr (kEPT * BITS < 32) {  // 2-bit, 8 elements: 16 bits; two neighbouring threads share a word
    const uint32_t other = (uint32_t)__builtin_amdgcn_ds_bpermute((__lane_id() ^ 1) << 2, (int)packed[0]);
    if ((chunk & 1) == 0) cdst[chunk / 2] = packed[0] | (other << 16);
  } else if constexpr (BITS == 8) {  // 8-byte aligned (checked on the host)
#pragma unroll
    for (int w = 0; w < W; w += 2) *(u2*)(cdst + chunk * W + w) = u2{packed[w], packed[w + 1]};
  } else {
#pragma unroll
    for (int w = 0; w < W; ++w) cdst[chunk * W + w] = packed[w];
  }
  if (chunk % TPG == 0) {
    const int64_t gi = bb * job.g_b + h * job.g_h + drow * job.g_s + chunk / TPG;
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
  // rows per launch: the thread index of every launch stays below 2^31 (more rows take more launches)
  // 32 elements per thread when that launch still has 8 or more workgroups per CU (2048 in all)
  const bool wide = (int64_t)B * H * L * (D / 32) * njobs >= 2048 * 256;
  const int ept = wide ? 32 : 8;
  const int64_t per_l = (int64_t)B * H * (D / ept);
  if (per_l >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  const int64_t max_l = (((int64_t)1 << 31) - 1) / per_l;
  RowMap rm{};
  rm.H = (uint32_t)H;
  rm.div_h = make_div31((uint32_t)H);
  rm.per_row = (uint32_t)(D / ept);
  rm.div_c = make_div31(rm.per_row);
  for (int64_t l0 = 0; l0 < L; l0 += max_l) {
    const int64_t nl = L - l0 < max_l ? L - l0 : max_l;
    rm.L = (uint32_t)nl;
    rm.div_l = make_div31((uint32_t)nl);
    rm.total = (uint32_t)(per_l * nl);
    rm.l0 = l0;
    const unsigned blocks = (unsigned)((rm.total + 255u) / 256u);
    const RopeArgs ra = rope ? *rope : RopeArgs{};
    if (rope && wide)
      hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G, true, 32>), dim3(blocks, njobs), dim3(256), 0, stream, k, v,
                         rm, row_offset, ra, pm);
    else if (rope)
      hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G, true, 8>), dim3(blocks, njobs), dim3(256), 0, stream, k, v,
                         rm, row_offset, ra, pm);
    else if (wide)
      hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G, false, 32>), dim3(blocks, njobs), dim3(256), 0, stream, k,
                         v, rm, row_offset, ra, pm);
    else
      hipLaunchKernelGGL((quantize_append_kernel<T, BITS, G, false, 8>), dim3(blocks, njobs), dim3(256), 0, stream, k,
                         v, rm, row_offset, ra, pm);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
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
