// Split-K flash-decoding over an MLX-layout affine-quantized KV cache (small L), with the
// log-sum-exp merge of the key splits fused into the same launch.
//
// Computes, per (sequence b, query head h, query row l):
//   out = softmax(scale * q K^T + mask) V,   K = sK * codesK + bK,  V = sV * codesV + bV
// i.e. the quantity m5engine/attention.py:29-103 evaluates (blocked online softmax, :64-100)
// and that its L == 1 branch (:42-45) hands to mlx-lm's quantized SDPA.
//
// Design (one wave = 16 MFMA columns; group size 64, NG = D/64 groups per row):
//  * The rep*L query rows that share a KV head are the MFMA columns. Column n holds query row
//    n % R (R = 16/NG) restricted to group n / R, so one accumulator yields per-group partial dot
//    products and a DPP row rotation adds the groups; every lane then owns a complete score.
//  * Codes enter the MFMA unconverted: a byte c placed in the low bits of an f16 is the subnormal
//    c * 2^-24, exact. Scales and biases are applied in fp32 after the MFMA:
//      q.k = sum_g s_g * (sum_{d in g} q_d c_d) + b_g * (sum_{d in g} q_d)
//      p.V = sum_t (p_t s_t) c_t + sum_t p_t b_t      (p_t s_t is the f16 A operand)
//    4-bit codes are masked in place; nibbles at odd positions arrive scaled by 16, which the Q
//    operand (QK) or the final accumulator scale (PV) undoes exactly.
//  * The score tile is computed transposed (keys are MFMA rows), which leaves each lane with
//    the probabilities of its own query row at 8 keys: exactly the A operand of the PV MFMA,
//    with no shuffle and no LDS round trip.
//  * K codes: each lane loads 16-32 contiguous bytes of one key row (128-bit loads). V codes:
//    each lane loads its 4-16 byte column slice of 8 key rows. Scales/biases of a 32-key tile
//    are fetched with one coalesced load per lane and redistributed through a per-wave LDS slab.
//  * Each wave streams its tiles through a ring of NBUF register buffers, so NBUF - 1 tiles are
//    in flight while one is computed.
//  * Online softmax in the log2 domain; rescaling of the output accumulators is lazy (only when a
//    row maximum grows). The waves of a workgroup merge in LDS into one (m, l, o[D]) partial per
//    query row. The last workgroup of each (sequence, KV head, row block) to finish -- found with
//    a device-scope counter that it resets afterwards -- merges the splits and writes the output.
//  * Workgroups are numbered so that the splits of one KV head land on one XCD (hardware hands
//    consecutive workgroups to the 8 XCDs in turn), keeping the merge inside one L2.

#include <math.h>
#include <stdlib.h>

#include "common.h"
#include "launch.h"
#include "merge.h"

namespace kvq {

constexpr int kTile = 32;
constexpr int kXcds = 8;

template <int D, int BITS>
struct DecCfg {
  static constexpr int NG = D / 64;            // scale groups per row
  static constexpr int R = 16 / NG;            // query rows per wave
  static constexpr int KSTEPS = D / 32;        // QK MFMA k-steps (8 dims per lane each)
  static constexpr int NBLK = D / 16;          // PV MFMA column blocks
  static constexpr int ROWB = D * BITS / 8;    // code bytes per key row
  static constexpr int KLB = ROWB / 4;         // K code bytes per lane per key (4 lane groups)
  static constexpr int VLB = ROWB / 16;        // V code bytes per lane per key (16 columns)
  static constexpr int SBB = 4 * NG;           // bytes of one cooperative scale/bias load (2 keys)
};

struct DecParams {
  const uint16_t* q;
  int64_t q_sb, q_sh, q_sl;
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t kc_sb, kc_sh, kc_ss;  // bytes
  int64_t vc_sb, vc_sh, vc_ss;  // bytes
  const uint16_t* ks;
  const uint16_t* kb;
  const uint16_t* vs;
  const uint16_t* vb;
  int64_t ksb_sb, ksb_sh, ksb_ss;  // elements
  int64_t vsb_sb, vsb_sh, vsb_ss;
  const int32_t* seq_lens;
  uint16_t* out;
  int64_t o_sb, o_sh, o_sl;
  unsigned* counters;
  float* part_o;
  float* part_ml;  // (m, l) pairs
  int Hq, Hkv, L, S, rep, nrows, rowblocks, nsplit, chunk, nunits;
  int xcd_remap;  // 1: number workgroups so that consecutive splits share an XCD
  int fused;      // 1: the last workgroup of a unit merges the splits; 0: combine_kernel does
  int sb_vec;     // scale/bias rows adjacent and aligned for one vector load per key pair
  int fast;       // sb_vec, and a tile's row offsets fit in 32 bits: full tiles use load_tile_fast
  float scale_log2;
  int causal, window;
};

template <int D, int BITS>
struct TileRegs {
  using C = DecCfg<D, BITS>;
  Bytes<C::KLB> kc[2];
  Bytes<(C::VLB < 2 ? 2 : C::VLB)> vc[8];
  Bytes<C::SBB> sb;
};

// Token (relative to the tile) of V slot i' (the MFMA k index 8*lg + i') for lane group lg.
__device__ __forceinline__ int v_token(int lg, int i) { return (i < 4) ? 4 * lg + i : 16 + 4 * lg + (i - 4); }

template <int D, int BITS>
__device__ __forceinline__ void load_tile(TileRegs<D, BITS>& R, const DecParams& p, const uint8_t* kbase,
                                          const uint8_t* vbase, const uint8_t* sbase, int64_t sb_row_bytes, int k0,
                                          int S_b, int n, int lg) {
  using C = DecCfg<D, BITS>;
  const bool partial = k0 + kTile > S_b;
#pragma unroll
  for (int beta = 0; beta < 2; ++beta) {
    int t = k0 + 16 * beta + n;
    if (partial) t = min(t, S_b - 1);
    R.kc[beta].load(kbase + (int64_t)t * p.kc_ss + lg * C::KLB);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int t = k0 + v_token(lg, i);
    if (partial) t = min(t, S_b - 1);
    R.vc[i].load(vbase + (int64_t)t * p.vc_ss + n * C::VLB);
  }
  // cooperative scale/bias load: lane -> (array a = lane/16, key pair tp = lane%16)
  const int tp = __lane_id() & 15;
  const int t0 = k0 + 2 * tp;
  if (!partial && p.sb_vec) {
    R.sb.load(sbase + (int64_t)t0 * sb_row_bytes);
  } else {
    const int ta = min(t0, S_b - 1), tb = min(t0 + 1, S_b - 1);
    if constexpr (C::NG == 1) {
      const uint32_t lo = *(const uint16_t*)(sbase + (int64_t)ta * sb_row_bytes);
      const uint32_t hi = *(const uint16_t*)(sbase + (int64_t)tb * sb_row_bytes);
      R.sb.w[0] = lo | (hi << 16);
    } else {
#pragma unroll
      for (int w = 0; w < C::NG / 2; ++w) {
        R.sb.w[w] = *(const uint32_t*)(sbase + (int64_t)ta * sb_row_bytes + 4 * w);
        R.sb.w[C::NG / 2 + w] = *(const uint32_t*)(sbase + (int64_t)tb * sb_row_bytes + 4 * w);
      }
    }
  }
}

// K operand (A of S^T = K Q^T) for k-step j: 8 codes of the lane's key as f16 subnormals.
template <int D, int BITS>
__device__ __forceinline__ h8 k_operand(const Bytes<DecCfg<D, BITS>::KLB>& kc, int j) {
  u4 r;
  if constexpr (BITS == 8) {
    const uint32_t w0 = kc.w[2 * j], w1 = kc.w[2 * j + 1];
    r[0] = perm(w0, w0, 0x0C010C00u);
    r[1] = perm(w0, w0, 0x0C030C02u);
    r[2] = perm(w1, w1, 0x0C010C00u);
    r[3] = perm(w1, w1, 0x0C030C02u);
  } else {
    const uint32_t w = kc.w[j];
    const uint32_t w8 = w >> 8;
    r[0] = w & 0x000F000Fu;   // nibbles 0, 4
    r[1] = w & 0x00F000F0u;   // nibbles 1, 5 (x16)
    r[2] = w8 & 0x000F000Fu;  // nibbles 2, 6
    r[3] = w8 & 0x00F000F0u;  // nibbles 3, 7 (x16)
  }
  return __builtin_bit_cast(h8, r);
}

// Dimension offset (within the lane's 8-dim slice of a k-step) and weight of operand slot i.
template <int BITS>
__device__ __forceinline__ int k_slot_dim(int i) {
  if constexpr (BITS == 8) return i;
  constexpr int m[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  return m[i];
}
template <int BITS>
__device__ __forceinline__ float k_slot_weight(int i) {
  if constexpr (BITS == 8) return 1.0f;
  return ((i >> 1) & 1) ? 0.0625f : 1.0f;
}

// V operand (B of O = P' V) for column block jN: codes of 8 keys at the lane's column.
template <int D, int BITS>
__device__ __forceinline__ h8 v_operand(const TileRegs<D, BITS>& R, int jN) {
  const int byte_off = (jN * BITS) / 8;  // byte of the lane's slice holding code jN
  const int wi = byte_off / 4;
  const uint32_t jb = (uint32_t)(byte_off % 4);
  const uint32_t sel = 0x0C000C00u | ((4u + jb) << 16) | jb;
  u4 r;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    uint32_t y = perm(R.vc[2 * a + 1].w[wi], R.vc[2 * a].w[wi], sel);
    if constexpr (BITS == 4) y &= (jN & 1) ? 0x00F000F0u : 0x000F000Fu;
    r[a] = y;
  }
  return __builtin_bit_cast(h8, r);
}

// Agent-scope (device-coherent) accesses to the split partials.
__device__ __forceinline__ void st_agent(float* ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* ptr) {
  return __hip_atomic_load(const_cast<float*>(ptr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Per-lane byte offsets of a tile's code loads, relative to the tile's first key row.
template <int D, int BITS>
struct LaneOff {
  uint32_t k[2];
  uint32_t v[8];
};

// Full-tile load: buffer loads with the tile's byte offset as the wave-uniform offset and fixed
// 32-bit lane offsets, so the code loads need no per-tile address arithmetic; `st` is this lane's
// scale/bias pointer for the tile.
template <int D, int BITS>
__device__ __forceinline__ void load_tile_fast(TileRegs<D, BITS>& R, __amdgpu_buffer_rsrc_t kr, uint32_t ks,
                                               __amdgpu_buffer_rsrc_t vr, uint32_t vs, const uint8_t* st,
                                               const LaneOff<D, BITS>& o) {
#pragma unroll
  for (int beta = 0; beta < 2; ++beta) R.kc[beta].load_buf(kr, o.k[beta], ks);
#pragma unroll
  for (int i = 0; i < 8; ++i) R.vc[i].load_buf(vr, o.v[i], vs);
  R.sb.load(st);
}

// Rescaling slack, log2 units: a row's running maximum is raised only when a tile's maximum
// exceeds it by more than this, so most tiles skip the accumulator rescale. Probabilities stay
// below 2^kSlack; with fp16 scales (|s| <= 514) the fp16 PV operand p*s stays finite.
constexpr float kSlack = 6.0f;

template <typename T, int D, int BITS, int NW, int NBUF>
__global__ __launch_bounds__(NW * 64, 8 / NW) void decode_attn_kernel(DecParams p) {
  using C = DecCfg<D, BITS>;
  constexpr int R = C::R;
  constexpr int NT = NW * 64;
  __shared__ __align__(16) uint16_t sb_lds[NW][4][C::NG][kTile];
  __shared__ float w_m[NW][R], w_l[NW][R];
  __shared__ __align__(16) float w_o[NW][R][D];
  __shared__ float s_w[R][kMaxSplit];
  __shared__ unsigned s_prev;

  const int lane = __lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, lg = lane >> 4;

  // ---- workgroup -> (unit, split); a unit is (sequence, KV head, row block)
  int wg = blockIdx.x;
  if (p.xcd_remap) {
    const int per_xcd = (p.nunits * p.nsplit) / kXcds;
    wg = (wg % kXcds) * per_xcd + wg / kXcds;
  }
  const int unit = wg / p.nsplit;
  const int split = wg % p.nsplit;
  const int b = unit / (p.Hkv * p.rowblocks);
  const int kvh = (unit / p.rowblocks) % p.Hkv;
  const int rb = unit % p.rowblocks;

  const int S_b = p.seq_lens ? min(max(p.seq_lens[b], 0), p.S) : p.S;  // clamped: never read past the view
  const int key_base = p.window > 0 ? max(0, S_b - p.L - p.window + 1) : 0;
  const int k_begin = key_base + split * p.chunk;
  const int k_end = min(k_begin + p.chunk, S_b);
  const int ntile = k_end > k_begin ? (k_end - k_begin + kTile - 1) / kTile : 0;
  // full tiles run through the register ring; a ragged last tile (and every tile of a cache
  // whose layout the fast loads do not cover) takes the clamped path afterwards
  const bool ragged = ntile > 0 && (k_end - k_begin) % kTile != 0;
  const int nfull = p.fast ? ntile - (ragged ? 1 : 0) : 0;
  const int nring = nfull > wave ? (nfull - wave + NW - 1) / NW : 0;  // ring tiles of this wave

  // ---- per-(b, kv head) bases
  const uint8_t* kbase = p.kc + (int64_t)b * p.kc_sb + (int64_t)kvh * p.kc_sh;
  const uint8_t* vbase = p.vc + (int64_t)b * p.vc_sb + (int64_t)kvh * p.vc_sh;
  const int arr = lane >> 4;  // cooperative scale/bias array of this lane: sK, bK, sV, bV
  const uint16_t* sbp;
  {
    const int64_t ko = (int64_t)b * p.ksb_sb + (int64_t)kvh * p.ksb_sh;
    const int64_t vo = (int64_t)b * p.vsb_sb + (int64_t)kvh * p.vsb_sh;
    sbp = arr == 0 ? p.ks + ko : arr == 1 ? p.kb + ko : arr == 2 ? p.vs + vo : p.vb + vo;
  }
  const int64_t sb_row_bytes = (arr < 2 ? p.ksb_ss : p.vsb_ss) * 2;
  const uint8_t* sbase = (const uint8_t*)sbp;

  LaneOff<D, BITS> off;
#pragma unroll
  for (int beta = 0; beta < 2; ++beta) off.k[beta] = (uint32_t)((16 * beta + n) * p.kc_ss + lg * C::KLB);
#pragma unroll
  for (int i = 0; i < 8; ++i) off.v[i] = (uint32_t)(v_token(lg, i) * p.vc_ss + n * C::VLB);
  const uint8_t* sb_lane = sbase + (int64_t)(2 * (lane & 15)) * sb_row_bytes;
  // ring tile i of this wave (clamped to the wave's last ring tile: look-ahead loads past the end
  // re-read a tile the wave already holds)
  auto ring_k0 = [&](int i) { return k_begin + kTile * (wave + NW * min(i, nring - 1)); };
  // code buffers of this (sequence, KV head): the S_b valid rows (the host checks the byte range
  // fits 32 bits before it enables the fast path)
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)(p.fast ? (int64_t)S_b * p.kc_ss : 0));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, (uint32_t)(p.fast ? (int64_t)S_b * p.vc_ss : 0));
  auto ring_load = [&](TileRegs<D, BITS>& buf, int i) {
    const int k0 = ring_k0(i);
    load_tile_fast<D, BITS>(buf, krs, (uint32_t)(k0 * p.kc_ss), vrs, (uint32_t)(k0 * p.vc_ss),
                            sb_lane + (int64_t)k0 * sb_row_bytes, off);
  };

  TileRegs<D, BITS> buf[NBUF];
  if (nring > 0) {
#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j) ring_load(buf[j], j);
  }

  // ---- this lane's query row / group
  const int r = n % R, g = n / R;
  const int row = rb * R + r;
  const bool row_ok = row < p.nrows;
  const int hq = kvh * p.rep + (row_ok ? row / p.L : 0);
  const int lq = row_ok ? row % p.L : 0;
  const int qpos = S_b - p.L + lq;
  const int lo_r = p.window > 0 ? max(0, qpos - p.window + 1) : 0;
  const int hi_r = p.causal ? min(S_b, qpos + 1) : S_b;
  const int lo_all = p.window > 0 ? max(0, S_b - p.window) : 0;
  const int hi_all = p.causal ? S_b - p.L + 1 : S_b;

  // ---- Q operand: slot i of k-step j is q[row][lg*D/4 + 8j + dim(i)] if that dim is in group g
  const bool in_group = (lg * (D / 4)) / 64 == g;
  float qv[C::KSTEPS][8];
  float qmax = 0.0f, qsum = 0.0f;
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)lq * p.q_sl + lg * (D / 4);
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j) {
      u4 raw = (row_ok && in_group) ? *(const u4*)(qrow + 8 * j) : u4{0, 0, 0, 0};
      float e[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[2 * i] = to_float((uint16_t)(raw[i] & 0xffffu), T{});
        e[2 * i + 1] = to_float((uint16_t)(raw[i] >> 16), T{});
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qv[j][i] = e[k_slot_dim<BITS>(i)];
        qmax = fmaxf(qmax, fabsf(qv[j][i]));
        qsum += qv[j][i];
      }
    }
  }
#pragma unroll
  for (int m = R; m < 16; m <<= 1) qmax = fmaxf(qmax, shfl_xor(qmax, m));
  qmax = max_xor32(max_xor16(qmax));
  qsum = add_xor32(add_xor16(qsum));
  int qexp = 0;
  if (qmax > 0.0f) {
    frexpf(qmax, &qexp);
    qexp = 15 - qexp;  // |q| * 2^qexp < 2^15
  }
  const float qscale = ldexpf(1.0f, qexp);
  h8 qop[C::KSTEPS];
#pragma unroll
  for (int j = 0; j < C::KSTEPS; ++j) {
#pragma unroll
    for (int i = 0; i < 8; ++i) qop[j][i] = (_Float16)(qv[j][i] * qscale * k_slot_weight<BITS>(i));
  }
  // score = sK * (acc * kf) + bK * qs2, then summed over the NG groups of the row
  const float kf = ldexpf(1.0f, 24 - qexp) * p.scale_log2;
  const float qs2 = qsum * p.scale_log2;

  float m_run = -INFINITY, l_part = 0.0f, ob_part = 0.0f;
  f4 acc_o[C::NBLK];
#pragma unroll
  for (int jn = 0; jn < C::NBLK; ++jn) acc_o[jn] = f4{0, 0, 0, 0};

  auto compute = [&](const TileRegs<D, BITS>& Rg, int k0) {
    // scales/biases -> LDS as [array][group][key], then each lane reads its keys' values
    {
      const int tp = lane & 15;
#pragma unroll
      for (int gg = 0; gg < C::NG; ++gg) {
        uint32_t v;
        if constexpr (C::NG == 1) {
          v = Rg.sb.w[0];
        } else {
          const int wlo = gg / 2;
          const uint32_t sel = (gg & 1) ? 0x07060302u : 0x05040100u;
          v = perm(Rg.sb.w[C::NG / 2 + wlo], Rg.sb.w[wlo], sel);
        }
        *(uint32_t*)&sb_lds[wave][arr][gg][2 * tp] = v;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    u2 sbr[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int beta = 0; beta < 2; ++beta) sbr[a][beta] = *(const u2*)&sb_lds[wave][a][g][16 * beta + 4 * lg];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    auto sbv = [&](int a, int beta, int i) -> float {
      const uint32_t w = sbr[a][beta][i >> 1];
      return to_float((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)), T{});
    };

    // S^T = K Q^T: rows = 16 keys of block beta, columns = (query row, group)
    f4 sacc[2];
#pragma unroll
    for (int beta = 0; beta < 2; ++beta) {
      sacc[beta] = f4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < C::KSTEPS; ++j)
        sacc[beta] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand<D, BITS>(Rg.kc[beta], j), qop[j], sacc[beta],
                                                            0, 0, 0);
    }
    float sc[8];
#pragma unroll
    for (int beta = 0; beta < 2; ++beta)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = sbv(0, beta, i) * (sacc[beta][i] * kf) + sbv(1, beta, i) * qs2;
        if constexpr (C::NG >= 2) x += row_rotate<8>(x);
        if constexpr (C::NG >= 4) x += row_rotate<4>(x);
        sc[4 * beta + i] = x;
      }
    const bool need_mask = !(k0 >= lo_all && k0 + kTile <= hi_all);
    if (need_mask) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int t = k0 + 16 * (s >> 2) + 4 * lg + (s & 3);
        if (!(t >= lo_r && t < hi_r)) sc[s] = -INFINITY;
      }
    }
    float tm = sc[0];
#pragma unroll
    for (int s = 1; s < 8; ++s) tm = fmaxf(tm, sc[s]);
    tm = max_xor32(max_xor16(tm));
    if (__builtin_amdgcn_ballot_w64(tm > m_run + kSlack) != 0) {
      const float m_new = fmaxf(m_run, tm);
      const float corr = (m_new == -INFINITY) ? 1.0f : exp2_fast(m_run - m_new);
      l_part *= corr;
      ob_part *= corr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ci = shfl(corr, (4 * lg + i) % R);
#pragma unroll
        for (int jn = 0; jn < C::NBLK; ++jn) acc_o[jn][i] *= ci;
      }
      m_run = m_new;
    }
    const float msub = (m_run == -INFINITY) ? 0.0f : m_run;
    float pa[8];
    float psum = 0.0f, pb = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float pr = exp2_fast(sc[s] - msub);
      psum += pr;
      pb += pr * sbv(3, s >> 2, s & 3);
      pa[s] = pr * sbv(2, s >> 2, s & 3);
    }
    l_part += psum;
    ob_part += pb;
    u4 aw;
#pragma unroll
    for (int a = 0; a < 4; ++a) aw[a] = pack_f16x2(pa[2 * a], pa[2 * a + 1]);
    const h8 aop = __builtin_bit_cast(h8, aw);
#pragma unroll
    for (int jn = 0; jn < C::NBLK; ++jn)
      acc_o[jn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, v_operand<D, BITS>(Rg, jn), acc_o[jn], 0, 0, 0);
  };

  // ---- main loop: a ring of NBUF tile buffers, NBUF - 1 loads ahead of the compute
  if (nring > 0) {
    int i = 0;
    for (; i + NBUF <= nring; i += NBUF) {
#pragma unroll
      for (int j = 0; j < NBUF; ++j) {
        ring_load(buf[(j + NBUF - 1) % NBUF], i + j + NBUF - 1);
        compute(buf[j], ring_k0(i + j));
      }
    }
    // the fewer than NBUF tiles left are already in buf[0 .. NBUF-2]
#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j)
      if (i + j < nring) compute(buf[j], ring_k0(i + j));
  }
  // ---- clamped tiles: the ragged last tile, or every tile when the fast loads do not apply
  for (int t = p.fast ? ntile - 1 : wave; t < ntile; t += NW) {
    if (p.fast && (!ragged || t % NW != wave)) break;
    const int k0 = k_begin + kTile * t;
    load_tile<D, BITS>(buf[0], p, kbase, vbase, sbase, sb_row_bytes, k0, S_b, n, lg);
    compute(buf[0], k0);
  }

  // ---- wave epilogue: sums over the 4 lane groups, then stage (m, l, o) in LDS
  l_part = add_xor32(add_xor16(l_part));
  ob_part = add_xor32(add_xor16(ob_part));
  float obi[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) obi[i] = shfl(ob_part, 4 * lg + i);
  if (lg == 0 && n < R) {
    w_m[wave][n] = m_run;
    w_l[wave][n] = l_part;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * lg + i;
    if (m / R == n / R) {
#pragma unroll
      for (int jn = 0; jn < C::NBLK; ++jn) {
        float sc = 16777216.0f;
        if constexpr (BITS == 4) sc = (jn & 1) ? 1048576.0f : 16777216.0f;
        w_o[wave][m % R][(D / 16) * n + jn] = acc_o[jn][i] * sc + obi[i];
      }
    }
  }
  __syncthreads();

  // ---- merge the waves: this workgroup's (m, l, o) per row; a single split writes the output
  const bool single = p.nsplit == 1;
  for (int idx = threadIdx.x; idx < R * D; idx += NT) {
    const int rr = idx / D, d = idx % D;
    const int rw = rb * R + rr;
    if (rw >= p.nrows) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, w_m[w][rr]);
    float o = 0.0f, lsum = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = w_m[w][rr];
        if (mw != -INFINITY) {
          const float f = exp2_fast(mw - M);
          o += f * w_o[w][rr][d];
          lsum += f * w_l[w][rr];
        }
      }
    }
    if (single) {
      const int hh = kvh * p.rep + rw / p.L, ll = rw % p.L;
      uint16_t* orow = p.out + (int64_t)b * p.o_sb + (int64_t)hh * p.o_sh + (int64_t)ll * p.o_sl;
      orow[d] = from_float(lsum > 0.0f ? o / lsum : 0.0f, T{});
    } else {
      const int64_t slot = ((int64_t)unit * R + rr) * p.nsplit + split;
      if (p.fused) {
        st_agent(p.part_o + slot * D + d, o);
        if (d == 0) {
          st_agent(p.part_ml + 2 * slot, M);
          st_agent(p.part_ml + 2 * slot + 1, lsum);
        }
      } else {
        p.part_o[slot * D + d] = o;
        if (d == 0) ((float2*)p.part_ml)[slot] = make_float2(M, lsum);
      }
    }
  }
  if (single || !p.fused) return;

  // ---- the last workgroup of this unit to finish merges the splits. The partials were written
  // with agent-scope stores; once they are acknowledged (s_waitcnt) the counter increment is
  // ordered after them at the device's coherence point, and the merging workgroup reads them with
  // agent-scope loads. No device-scope fence is needed (on gfx950 one writes back the XCD's L2).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_prev = __hip_atomic_fetch_add(&p.counters[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_prev != (unsigned)(p.nsplit - 1)) return;
  if (threadIdx.x == 0) __hip_atomic_store(&p.counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // weights w_s / sum_s w_s l_s per row, one wave per row
  for (int rr = wave; rr < R; rr += NW) {
    const int64_t base = ((int64_t)unit * R + rr) * p.nsplit;
    float m0 = -INFINITY, l0 = 0.0f, m1 = -INFINITY, l1 = 0.0f;
    if (lane < p.nsplit) {
      m0 = ld_agent(p.part_ml + 2 * (base + lane));
      l0 = ld_agent(p.part_ml + 2 * (base + lane) + 1);
    }
    if (lane + 64 < p.nsplit) {
      m1 = ld_agent(p.part_ml + 2 * (base + lane + 64));
      l1 = ld_agent(p.part_ml + 2 * (base + lane + 64) + 1);
    }
    m0 = l0 > 0.0f ? m0 : -INFINITY;
    m1 = l1 > 0.0f ? m1 : -INFINITY;
    const float M = wave_max(fmaxf(m0, m1));
    const float w0 = (M == -INFINITY || m0 == -INFINITY) ? 0.0f : exp2_fast(m0 - M);
    const float w1 = (M == -INFINITY || m1 == -INFINITY) ? 0.0f : exp2_fast(m1 - M);
    const float Lsum = wave_sum(w0 * l0 + w1 * l1);
    const float inv = Lsum > 0.0f ? 1.0f / Lsum : 0.0f;
    if (lane < p.nsplit) s_w[rr][lane] = w0 * inv;
    if (lane + 64 < p.nsplit) s_w[rr][lane + 64] = w1 * inv;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * D; idx += NT) {
    const int rr = idx / D, d = idx % D;
    const int rw = rb * R + rr;
    if (rw >= p.nrows) continue;
    const float* po = p.part_o + ((int64_t)unit * R + rr) * p.nsplit * D + d;
    float acc = 0.0f;
    int s = 0;
    for (; s + 8 <= p.nsplit; s += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = ld_agent(po + (int64_t)(s + u) * D);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += s_w[rr][s + u] * v[u];
    }
    for (; s < p.nsplit; ++s) acc += s_w[rr][s] * ld_agent(po + (int64_t)s * D);
    const int hh = kvh * p.rep + rw / p.L, ll = rw % p.L;
    p.out[(int64_t)b * p.o_sb + (int64_t)hh * p.o_sh + (int64_t)ll * p.o_sl + d] = from_float(acc, T{});
  }
}

// ------------------------------------------------------------------------------------------
// Host side: plan, workspace, launch.

struct DecPlan {
  int R, rowblocks, chunk, nsplit, span, nunits, nw, nbuf, fused;
};

struct DecTune {
  int nw, nbuf, target_wgs, fused;
};

// Launch-shape defaults; KVQ_DECODE_TUNE="waves,buffers,workgroups,fused" overrides them (read
// once per process).
static DecTune decode_tune() {
  static DecTune t = [] {
    DecTune d{8, 2, 256, 0};
    if (const char* e = getenv("KVQ_DECODE_TUNE")) {
      int a = 0, b = 0, c = 0, f = 1;
      if (sscanf(e, "%d,%d,%d,%d", &a, &b, &c, &f) >= 3 && (a == 4 || a == 8) && b >= 2 && b <= 4 && c >= 1)
        d = {a, b, c, f != 0};
    }
    return d;
  }();
  return t;
}

DecPlan decode_plan(int B, int Hq, int Hkv, int L, int D, int S, int window, int) {
  DecPlan pl;
  const DecTune tune = decode_tune();
  pl.nw = D == 128 ? tune.nw : 4;
  pl.nbuf = D == 128 ? tune.nbuf : 2;
  pl.R = 16 / (D / 64);
  const int nrows = (Hq / Hkv) * L;
  pl.rowblocks = (nrows + pl.R - 1) / pl.R;
  pl.span = window > 0 ? std::min(S, window + L - 1) : S;
  const int64_t tiles_seq = (pl.span + kTile - 1) / kTile;
  pl.nunits = B * Hkv * pl.rowblocks;
  int64_t tpw = (pl.nunits * tiles_seq + tune.target_wgs - 1) / tune.target_wgs;
  tpw = std::max<int64_t>(tpw, (tiles_seq + kMaxSplit - 1) / kMaxSplit);
  tpw = std::max<int64_t>(pl.nw, (tpw + pl.nw - 1) / pl.nw * pl.nw);
  pl.chunk = (int)(tpw * kTile);
  pl.nsplit = (pl.span + pl.chunk - 1) / pl.chunk;
  pl.fused = tune.fused && pl.nunits <= kMaxCountedUnits;
  return pl;
}

// Workspace: [split counters (the shared block), zero between calls][(m, l) per row and split]
// [o per row and split]
struct DecLayout {
  size_t counters, ml, o, total;
};
static DecLayout decode_layout(const DecPlan& pl, int D) {
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  DecLayout l;
  const size_t prow = (size_t)pl.nunits * pl.R * pl.nsplit;
  l.counters = 0;
  l.ml = kCounterBytes;
  l.o = l.ml + up(prow * sizeof(float2));
  l.total = l.o + up(prow * D * sizeof(float));
  return l;
}

size_t decode_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window, int bits) {
  const DecPlan pl = decode_plan(B, Hq, Hkv, L, D, S, window, bits);
  return decode_layout(pl, D).total;
}

template <typename T, int D, int BITS, int NW, int NBUF>
static hipError_t launch_decode_t(const DecParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((decode_attn_kernel<T, D, BITS, NW, NBUF>), dim3(p.nunits * p.nsplit), dim3(NW * 64), 0, stream,
                     p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.nsplit == 1 || p.fused) return e;
  MergeParams m;
  m.part_o = p.part_o;
  m.part_ml = p.part_ml;
  m.out = p.out;
  m.o_sb = p.o_sb;
  m.o_sh = p.o_sh;
  m.o_sl = p.o_sl;
  m.Hq = p.Hq;
  m.Hkv = p.Hkv;
  m.L = p.L;
  m.rep = p.rep;
  m.R = DecCfg<D, BITS>::R;
  m.rowblocks = p.rowblocks;
  m.nsplit = p.nsplit;
  m.position_major = 0;
  return launch_combine<T, D>(m, p.nunits / (p.Hkv * p.rowblocks), stream);
}

template <typename T, int D, int BITS>
static hipError_t launch_decode_shape(const DecParams& p, const DecPlan& pl, hipStream_t stream) {
  if constexpr (D == 128) {
    if (pl.nw == 8) {
      if (pl.nbuf == 2) return launch_decode_t<T, D, BITS, 8, 2>(p, stream);
      return launch_decode_t<T, D, BITS, 8, 3>(p, stream);
    }
    if (pl.nbuf == 2) return launch_decode_t<T, D, BITS, 4, 2>(p, stream);
    if (pl.nbuf == 3) return launch_decode_t<T, D, BITS, 4, 3>(p, stream);
    return launch_decode_t<T, D, BITS, 4, 4>(p, stream);
  } else {
    return launch_decode_t<T, D, BITS, 4, 2>(p, stream);
  }
}

hipError_t launch_decode(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                         const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int dtype,
                         float scale, int causal, int window, void* workspace, hipStream_t stream) {
  const DecPlan pl = decode_plan(B, Hq, Hkv, L, D, S, window, bits);
  const DecLayout lay = decode_layout(pl, D);
  DecParams p;
  p.q = (const uint16_t*)q->data;
  p.q_sb = q->stride_b;
  p.q_sh = q->stride_h;
  p.q_sl = q->stride_l;
  p.kc = (const uint8_t*)k->codes;
  p.vc = (const uint8_t*)v->codes;
  p.kc_sb = k->codes_stride_b * 4;
  p.kc_sh = k->codes_stride_h * 4;
  p.kc_ss = k->codes_stride_s * 4;
  p.vc_sb = v->codes_stride_b * 4;
  p.vc_sh = v->codes_stride_h * 4;
  p.vc_ss = v->codes_stride_s * 4;
  p.ks = (const uint16_t*)k->scales;
  p.kb = (const uint16_t*)k->biases;
  p.vs = (const uint16_t*)v->scales;
  p.vb = (const uint16_t*)v->biases;
  p.ksb_sb = k->sb_stride_b;
  p.ksb_sh = k->sb_stride_h;
  p.ksb_ss = k->sb_stride_s;
  p.vsb_sb = v->sb_stride_b;
  p.vsb_sh = v->sb_stride_h;
  p.vsb_ss = v->sb_stride_s;
  p.seq_lens = seq_lens;
  p.out = (uint16_t*)out->data;
  p.o_sb = out->stride_b;
  p.o_sh = out->stride_h;
  p.o_sl = out->stride_l;
  p.counters = (unsigned*)((char*)workspace + lay.counters);
  p.part_ml = (float*)((char*)workspace + lay.ml);
  p.part_o = (float*)((char*)workspace + lay.o);
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.L = L;
  p.S = S;
  p.rep = Hq / Hkv;
  p.nrows = p.rep * L;
  p.rowblocks = pl.rowblocks;
  p.nsplit = pl.nsplit;
  p.chunk = pl.chunk;
  p.nunits = pl.nunits;
  p.xcd_remap = ((int64_t)pl.nunits * pl.nsplit) % kXcds == 0;
  p.fused = pl.fused;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.causal = causal;
  p.window = window;
  {
    const int NG = D / 64;
    const int64_t vb = 4 * NG;  // bytes of one 2-key vector load
    auto ok = [&](const void* base, int64_t sbb, int64_t sbh, int64_t sbs) {
      return sbs == NG && ((uintptr_t)base % vb) == 0 && (sbb * 2) % vb == 0 && (sbh * 2) % vb == 0;
    };
    p.sb_vec = ok(k->scales, k->sb_stride_b, k->sb_stride_h, k->sb_stride_s) &&
               ok(k->biases, k->sb_stride_b, k->sb_stride_h, k->sb_stride_s) &&
               ok(v->scales, v->sb_stride_b, v->sb_stride_h, v->sb_stride_s) &&
               ok(v->biases, v->sb_stride_b, v->sb_stride_h, v->sb_stride_s);
    p.fast = p.sb_vec && (int64_t)S * std::max(p.kc_ss, p.vc_ss) < ((int64_t)1 << 31);
  }
  const bool bf = dtype == KVQ_DTYPE_BF16;
#define KVQ_DEC(TT, DD, BB) return launch_decode_shape<TT, DD, BB>(p, pl, stream)
  if (D == 128) {
    if (bits == 8) { if (bf) KVQ_DEC(BF16, 128, 8); else KVQ_DEC(F16, 128, 8); }
    else { if (bf) KVQ_DEC(BF16, 128, 4); else KVQ_DEC(F16, 128, 4); }
  } else {
    if (bits == 8) { if (bf) KVQ_DEC(BF16, 64, 8); else KVQ_DEC(F16, 64, 8); }
    else { if (bf) KVQ_DEC(BF16, 64, 4); else KVQ_DEC(F16, 64, 4); }
  }
#undef KVQ_DEC
}

}  // namespace kvq
