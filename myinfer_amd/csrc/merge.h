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
// at once, and each of them also reads all of the row's (m, l) pairs (the same addresses for the
// whole row) and forms the split weights itself, so no exchange between threads is needed. The
// splits are summed in split order; the weighted sum is divided by the weighted sum of the l's.
// One wave per workgroup: 64 / (D/4) rows, so a call spreads its partial reads over many CUs.
template <typename T, int D>
__global__ __launch_bounds__(64) void combine_kernel(MergeParams p, int nrows) {
  constexpr int TPR = D / 4;      // threads per row
  constexpr int RPW = 64 / TPR;   // rows per workgroup
  constexpr int CH = 32;          // partial loads in flight per thread
  constexpr int R = 1024 / D;     // rows per decode unit (16 / groups per row); the host checks p.R
  const int tr = threadIdx.x / TPR, j = threadIdx.x % TPR;
  const int grow = blockIdx.x * RPW + tr;
  const bool ok = grow < nrows;
  const int g = ok ? grow : 0;
  const int l = g % p.L, h = (g / p.L) % p.Hq, b = g / (p.L * p.Hq);
  const int kvh = h / p.rep;
  const int rw = (h - kvh * p.rep) * p.L + l;
  const int unit = (b * p.Hkv + kvh) * p.rowblocks + rw / R;
  const int64_t base = (int64_t)unit * p.nsplit * R + rw % R;  // split s at base + s * R
  const f4* po = (const f4*)(p.part_o + base * D) + j;
  const float2* ml = (const float2*)p.part_ml + base;
  constexpr int ss = R * D / 4;  // float4s between splits
  // loads past the last split re-read it (in bounds, no per-split branches) and count with l = 0
  // (held in a VGPR, so that the 64 clamped offsets are vector values, not scalar registers)
  int last;
  asm volatile("v_mov_b32 %0, %1" : "=v"(last) : "s"(p.nsplit - 1));
  f4 o[CH];
  float2 mv[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) o[u] = po[min(u, last) * ss];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    mv[u] = ml[min(u, last) * R];
    if (u > last) mv[u].y = 0.0f;
  }
  // the row's maximum over the splits that saw a key (l > 0)
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < CH; ++u)
    if (mv[u].y > 0.0f) M = fmaxf(M, mv[u].x);
  for (int s = CH; s < p.nsplit; ++s) {
    const float2 v = ml[s * R];
    if (v.y > 0.0f) M = fmaxf(M, v.x);
  }
  f4 acc = {0, 0, 0, 0};
  float Ls = 0.0f;
  auto add = [&](const float2 v, const f4 ov) __attribute__((always_inline)) {
    const float w = (v.y > 0.0f) ? exp2_fast(v.x - M) : 0.0f;  // M is finite when any l > 0
    acc += w * ov;
    Ls += w * v.y;
  };
#pragma unroll
  for (int u = 0; u < CH; ++u) add(mv[u], o[u]);
  for (int s0 = CH; s0 <= last; s0 += CH) {
#pragma unroll
    for (int u = 0; u < CH; ++u) o[u] = po[min(s0 + u, last) * ss];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      mv[u] = ml[min(s0 + u, last) * R];
      if (s0 + u > last) mv[u].y = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) add(mv[u], o[u]);
  }
  acc *= Ls > 0.0f ? 1.0f / Ls : 0.0f;
  if (!ok) return;
  uint16_t* dst = p.out + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)l * p.o_sl + 4 * j;
  u2 w;
  w[0] = (uint32_t)from_float(acc[0], T{}) | ((uint32_t)from_float(acc[1], T{}) << 16);
  w[1] = (uint32_t)from_float(acc[2], T{}) | ((uint32_t)from_float(acc[3], T{}) << 16);
  *(u2*)dst = w;
}

template <typename T, int D>
inline hipError_t launch_combine(const MergeParams& m, int B, hipStream_t stream) {
  if (m.R != 1024 / D) return hipErrorInvalidValue;  // the kernel's split strides assume this
  const int nrows = B * m.Hq * m.L;
  const int grid = (nrows + (256 / D) - 1) / (256 / D);  // 64 / (D / 4) rows per workgroup
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3(grid), dim3(64), 0, stream, m, nrows);
  return hipGetLastError();
}

}  // namespace kvq
