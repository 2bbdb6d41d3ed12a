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
};

// One thread per (output row, 4 columns): the D/4 threads of a row load its float4 of every split
// at once, share the split weights through LDS (computed by the row's threads from the (m, l)
// pairs, a few splits each) and sum the splits in split order. One wave per workgroup: 64 / (D/4)
// rows, so a call spreads its partial reads over many CUs.
template <typename T, int D>
__global__ __launch_bounds__(64) void combine_kernel(MergeParams p, int nrows) {
  constexpr int TPR = D / 4;      // threads per row
  constexpr int RPW = 64 / TPR;   // rows per workgroup
  constexpr int SPT = kMaxSplit / TPR;  // splits whose (m, l) one thread reads
  constexpr int CH = 32;          // partial loads in flight per thread
  __shared__ float s_w[RPW][kMaxSplit];
  const int tr = threadIdx.x / TPR, j = threadIdx.x % TPR;
  const int grow = blockIdx.x * RPW + tr;
  const bool ok = grow < nrows;
  const int g = ok ? grow : 0;
  const int l = g % p.L, h = (g / p.L) % p.Hq, b = g / (p.L * p.Hq);
  const int kvh = h / p.rep;
  const int rw = (h - kvh * p.rep) * p.L + l;
  const int unit = (b * p.Hkv + kvh) * p.rowblocks + rw / p.R;
  const int64_t base = (int64_t)unit * p.nsplit * p.R + rw % p.R;  // split s at base + s * R
  const f4* po = (const f4*)(p.part_o + base * D) + j;
  const int64_t sstride = (int64_t)p.R * D / 4;  // float4s between splits
  f4 o[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) o[u] = u < p.nsplit ? po[u * sstride] : f4{0, 0, 0, 0};
  // the row's weights 2^(m_s - M) / sum_s 2^(m_s - M) l_s, this thread's splits j, j + TPR, ...
  const float2* ml = (const float2*)p.part_ml + base;
  float mk[SPT], lk[SPT];
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    const int sp = j + TPR * k;
    const float2 v = sp < p.nsplit ? ml[(int64_t)sp * p.R] : make_float2(-INFINITY, 0.0f);
    mk[k] = v.y > 0.0f ? v.x : -INFINITY;
    lk[k] = v.y;
    M = fmaxf(M, mk[k]);
  }
#pragma unroll
  for (int m = 1; m < TPR; m <<= 1) M = fmaxf(M, shfl_xor(M, m));
  float Ls = 0.0f;
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    mk[k] = (M == -INFINITY || mk[k] == -INFINITY) ? 0.0f : exp2_fast(mk[k] - M);
    Ls += mk[k] * lk[k];
  }
#pragma unroll
  for (int m = 1; m < TPR; m <<= 1) Ls += shfl_xor(Ls, m);
  const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
  for (int k = 0; k < SPT; ++k)
    if (j + TPR * k < p.nsplit) s_w[tr][j + TPR * k] = mk[k] * inv;
  __syncthreads();
  f4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < CH; ++u)
    if (u < p.nsplit) acc += s_w[tr][u] * o[u];
  for (int s0 = CH; s0 < p.nsplit; s0 += CH) {
#pragma unroll
    for (int u = 0; u < CH; ++u) o[u] = s0 + u < p.nsplit ? po[(s0 + u) * sstride] : f4{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < CH; ++u)
      if (s0 + u < p.nsplit) acc += s_w[tr][s0 + u] * o[u];
  }
  if (!ok) return;
  uint16_t* dst = p.out + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)l * p.o_sl + 4 * j;
  u2 w;
  w[0] = (uint32_t)from_float(acc[0], T{}) | ((uint32_t)from_float(acc[1], T{}) << 16);
  w[1] = (uint32_t)from_float(acc[2], T{}) | ((uint32_t)from_float(acc[3], T{}) << 16);
  *(u2*)dst = w;
}

template <typename T, int D>
inline hipError_t launch_combine(const MergeParams& m, int B, hipStream_t stream) {
  const int nrows = B * m.Hq * m.L;
  const int grid = (nrows + (256 / D) - 1) / (256 / D);  // 64 / (D / 4) rows per workgroup
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3(grid), dim3(64), 0, stream, m, nrows);
  return hipGetLastError();
}

}  // namespace kvq
