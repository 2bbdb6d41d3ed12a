// Log-sum-exp merge of key-split attention partials, shared by the decode and prefill kernels.
//
// A kernel that splits the keys of a query row over `nsplit` workgroups leaves, per row and split,
// (m, l) = (running maximum in log2 units, sum of 2^(s - m)) and o[D] = sum of 2^(s - m) v. The
// merged output is sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s with M = max_s m_s (splits with
// l_s = 0 saw no key and drop out); a row no split saw is written as 0.
//
// Partials are laid out by "unit" -- the (sequence, KV head, row block) a workgroup serves -- with
// R rows per unit, split-major: o of (unit, split, r) at part_o[((unit * nsplit + split) * R + r) * D],
// (m, l) at part_ml[2 * ((unit * nsplit + split) * R + r)]. Row r of a unit is query position
// r % L of local head r / L.
#pragma once

#include <math.h>

#include "common.h"

namespace kvq {

constexpr int kMaxSplit = 128;

// Launches whose last-arriving workgroup merges the splits count arrivals per unit in a counter
// block at the start of the workspace. Every launch reserves the same block, so launches of
// different shapes that share one workspace never place partials over another launch's counters;
// a launch with more units than this does not split (prefill) or merges with combine_kernel
// (decode). Counters start at zero (the workspace is zero-filled once) and the merging workgroup
// resets its own.
constexpr int kMaxCountedUnits = 65536;
constexpr size_t kCounterBytes = (size_t)kMaxCountedUnits * sizeof(unsigned);

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v = fmaxf(v, shfl_xor(v, m));
  return max_xor32(max_xor16(v));
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) v += shfl_xor(v, m);
  return add_xor32(add_xor16(v));
}

struct MergeParams {
  const float* part_o;
  const float* part_ml;
  uint16_t* out;
  int64_t o_sb, o_sh, o_sl;
  int Hq, Hkv, L, rep, R, rowblocks, nsplit;
  int xcd_remap;  // 1: the decode launch numbered its workgroups by XCD (see decode_attn_kernel)
  Div31 d_l, d_hq, d_rep;  // L, Hq and rep as multiply-shift divisors (set by launch_combine)
};

// Quad lane exchanges (lane i with lane i ^ 1, i ^ 2) through DPP quad permutes.
template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, quad_perm<0xB1>(v));     // [1, 0, 3, 2]
  return fmaxf(v, quad_perm<0x4E>(v));  // [2, 3, 0, 1]
}
__device__ __forceinline__ float quad_sum(float v) {
  v += quad_perm<0xB1>(v);
  return v + quad_perm<0x4E>(v);
}

// Four threads per (output row, 4 columns): thread q of a quad takes splits q, q + 4, q + 8, ...,
// loads its float4 and (m, l) of each in one round (a quarter of the loads a thread would issue
// alone: the merge is bound by the latency of these loads), forms the split weights against the
// quad's maximum, and the quad sums its terms with two DPP exchanges. Fixed order, so repeated
// calls are bit-identical. 256 / D rows per workgroup of 256 threads. When the decode launch
// placed each unit's splits on one XCD, the workgroups here are numbered the same way (a grid that
// is a multiple of 8, rows in unit order), so a unit's partials are merged on the XCD that wrote
// them (+1% at 32 splits).
// NARROW: output rows of dv < D dims (the partials stay D wide); otherwise dv is not read.
template <typename T, int D, int R, bool NARROW = false>
__global__ __launch_bounds__(256) void combine_kernel(MergeParams p, int nrows, int dv) {
  constexpr int F4 = D / 4;              // float4s per row
  constexpr int RPB = 256 / (4 * F4);    // rows per workgroup
  constexpr int CH = 8;                  // splits per thread loaded in the first round
  const int t = threadIdx.x;
  const int q = t & 3, j = (t >> 2) % F4;
  const int bx = p.xcd_remap ? (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8 : blockIdx.x;
  const int grow = bx * RPB + t / (4 * F4);
  const bool ok = grow < nrows;
  const int g = ok ? grow : 0;
  const int gl = (int)div31((uint32_t)g, p.d_l);  // g / L: the (sequence, head) of the row
  const int l = g - gl * p.L;
  const int b = (int)div31((uint32_t)gl, p.d_hq);
  const int h = gl - b * p.Hq;
  const int kvh = (int)div31((uint32_t)h, p.d_rep);
  const int rw = (h - kvh * p.rep) * p.L + l;
  const int unit = (b * p.Hkv + kvh) * p.rowblocks + rw / R;
  const int64_t base = (int64_t)unit * p.nsplit * R + rw % R;  // split s at base + s * R
  const f4* po = (const f4*)(p.part_o + base * D) + j;
  const float2* ml = (const float2*)p.part_ml + base;
  constexpr int ss = R * D / 4;  // float4s between splits
  // loads past the last split re-read it (in bounds, no per-split branches) and count with l = 0
  // (held in a VGPR, so that the clamped offsets are vector values, not scalar registers)
  int last;
  asm volatile("v_mov_b32 %0, %1" : "=v"(last) : "s"(p.nsplit - 1));
  f4 o[CH];
  float2 mv[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int s = q + 4 * u;
    o[u] = po[min(s, last) * ss];
    mv[u] = ml[min(s, last) * R];
    if (s > last) mv[u].y = 0.0f;
  }
  // the row's maximum over the splits that saw a key (l > 0)
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < CH; ++u)
    if (mv[u].y > 0.0f) M = fmaxf(M, mv[u].x);
  for (int s = 4 * CH + q; s < p.nsplit; s += 4) {
    const float2 v = ml[s * R];
    if (v.y > 0.0f) M = fmaxf(M, v.x);
  }
  M = quad_max(M);
  f4 acc = {0, 0, 0, 0};
  float Ls = 0.0f;
  auto add = [&](const float2 v, const f4 ov) __attribute__((always_inline)) {
    const float w = (v.y > 0.0f) ? exp2_fast(v.x - M) : 0.0f;  // M is finite when any l > 0
    acc += w * ov;
    Ls += w * v.y;
  };
#pragma unroll
  for (int u = 0; u < CH; ++u) add(mv[u], o[u]);
  for (int s = 4 * CH + q; s < p.nsplit; s += 4) add(ml[s * R], po[s * ss]);
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = quad_sum(acc[e]);
  Ls = quad_sum(Ls);
  acc *= Ls > 0.0f ? 1.0f / Ls : 0.0f;
  if (!ok || q != 0 || (NARROW && 4 * j >= dv)) return;
  uint16_t* dst = p.out + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)l * p.o_sl + 4 * j;
  u2 w;
  w[0] = (uint32_t)from_float(acc[0], T{}) | ((uint32_t)from_float(acc[1], T{}) << 16);
  w[1] = (uint32_t)from_float(acc[2], T{}) | ((uint32_t)from_float(acc[3], T{}) << 16);
  *(u2*)dst = w;
}

template <typename T, int D>
// dv: dims of an output row (D unless the decode kernel ran narrower rows at width D)
inline hipError_t launch_combine(const MergeParams& m, int B, hipStream_t stream, int dv = D) {
  const int nrows = B * m.Hq * m.L;
  constexpr int rpb = 256 / D;  // rows per 256-thread workgroup
  const dim3 grid((nrows + rpb - 1) / rpb);
  MergeParams mm = m;
  mm.xcd_remap = m.xcd_remap && grid.x % 8 == 0;
  mm.d_l = make_div31((uint32_t)m.L);
  mm.d_hq = make_div31((uint32_t)m.Hq);
  mm.d_rep = make_div31((uint32_t)m.rep);
  // R (rows per unit: 16 / scale groups per row for decode, 128 for the head_dim-256 kernel) fixes
  // the kernel's split strides
  if (dv != D) {
    switch (m.R) {
      case 4: hipLaunchKernelGGL((combine_kernel<T, D, 4, true>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
      case 8: hipLaunchKernelGGL((combine_kernel<T, D, 8, true>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
      case 16: hipLaunchKernelGGL((combine_kernel<T, D, 16, true>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
      case 128: hipLaunchKernelGGL((combine_kernel<T, D, 128, true>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (m.R) {
    case 4: hipLaunchKernelGGL((combine_kernel<T, D, 4>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
    case 8: hipLaunchKernelGGL((combine_kernel<T, D, 8>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
    case 16: hipLaunchKernelGGL((combine_kernel<T, D, 16>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
    case 128: hipLaunchKernelGGL((combine_kernel<T, D, 128>), grid, dim3(256), 0, stream, mm, nrows, dv); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kvq
