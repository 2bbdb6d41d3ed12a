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

// One wave per (output row, 64 columns) item, grid-stride over the items beyond two waves of
// resident workgroups. Every lane issues all its partial
// loads (32 at a time) before the weights are formed, so an item costs one round trip.
template <typename T, int D>
__global__ __launch_bounds__(64) void combine_kernel(MergeParams p, int nitems) {
  constexpr int CH = 32;
  __shared__ float s_w[kMaxSplit];
  const int lane = threadIdx.x;
  for (int item = blockIdx.x; item < nitems; item += gridDim.x) {
    const int grow = item / (D / 64), d = (item % (D / 64)) * 64 + lane;
    const int l = grow % p.L, h = (grow / p.L) % p.Hq, b = grow / (p.L * p.Hq);
    const int kvh = h / p.rep;
    const int rw = (h - kvh * p.rep) * p.L + l;
    const int unit = (b * p.Hkv + kvh) * p.rowblocks + rw / p.R;
    const int64_t base = (int64_t)unit * p.nsplit * p.R + rw % p.R;  // split s at base + s * R
    const float* po = p.part_o + base * D + d;
    float o[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) o[u] = u < p.nsplit ? po[(int64_t)u * p.R * D] : 0.0f;
    {
      const float2* ml = (const float2*)p.part_ml + base;
      const float2 v0 = lane < p.nsplit ? ml[(int64_t)lane * p.R] : make_float2(-INFINITY, 0.0f);
      const float2 v1 = lane + 64 < p.nsplit ? ml[(int64_t)(lane + 64) * p.R] : make_float2(-INFINITY, 0.0f);
      const float m0 = v0.y > 0.0f ? v0.x : -INFINITY, m1 = v1.y > 0.0f ? v1.x : -INFINITY;
      const float M = wave_max(fmaxf(m0, m1));
      const float w0 = (M == -INFINITY || m0 == -INFINITY) ? 0.0f : exp2_fast(m0 - M);
      const float w1 = (M == -INFINITY || m1 == -INFINITY) ? 0.0f : exp2_fast(m1 - M);
      const float Lsum = wave_sum(w0 * v0.y + w1 * v1.y);
      const float inv = Lsum > 0.0f ? 1.0f / Lsum : 0.0f;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // the previous item's reads of s_w are done
      __builtin_amdgcn_wave_barrier();
      if (lane < p.nsplit) s_w[lane] = w0 * inv;
      if (lane + 64 < p.nsplit) s_w[lane + 64] = w1 * inv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < CH; ++u)
      if (u < p.nsplit) acc += s_w[u] * o[u];
    for (int s0 = CH; s0 < p.nsplit; s0 += CH) {
#pragma unroll
      for (int u = 0; u < CH; ++u) o[u] = s0 + u < p.nsplit ? po[(int64_t)(s0 + u) * p.R * D] : 0.0f;
#pragma unroll
      for (int u = 0; u < CH; ++u)
        if (s0 + u < p.nsplit) acc += s_w[s0 + u] * o[u];
    }
    p.out[(int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)l * p.o_sl + d] = from_float(acc, T{});
  }
}

template <typename T, int D>
inline hipError_t launch_combine(const MergeParams& m, int B, hipStream_t stream) {
  const int nitems = B * m.Hq * m.L * (D / 64);
  const int grid = nitems < 16384 ? nitems : 16384;
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3(grid), dim3(64), 0, stream, m, nitems);
  return hipGetLastError();
}

}  // namespace kvq
