// Causal chunked-prefill attention over an MLX-layout affine-quantized KV cache, on MFMA.
//
// Computes, per (sequence b, query head h, query row l), the quantity m5engine/attention.py:29-103
// evaluates for L > 1 (blocked online softmax over key blocks, :64-100, causal when the mask is a
// string, :55-58/:70-73):
//   out = softmax(scale * q K^T + mask) V,  K = sK * codesK + bK,  V = sV * codesV + bV
// with query l at position S_b - L + l, keys <= position when causal, keys > position - window
// when a sliding window is set.
//
// Design (head_dim 128, 64-key tiles, a workgroup = 4 waves = 128 query rows):
//  * A workgroup serves 128 consecutive rows of one (sequence, KV head) in position-major order
//    (row = position * rep + local head), so all rep query heads of a position share each K/V
//    tile and a causal boundary cuts only a few positions.
//  * Each 64-key tile is dequantized once per workgroup into LDS as fp16: K row-major, V
//    transposed (V^T[d][slot]) with its key slots permuted to match the score layout below.
//    Double-buffered: the codes of tile t+1 are in flight while tile t is computed.
//  * Per wave (32 rows = the columns of a 32x32 MFMA): S^T = K Q^T (v_mfma_f32_32x32x16_f16;
//    A = K rows from LDS, B = Q^T held in registers). In the MFMA result layout every lane holds
//    16 keys of one query column, so the row max / sum are lane-local plus one permlane swap, and
//    the probabilities converted to fp16 are already the B operand of O^T = V^T P^T: no shuffle.
//  * Q carries the softmax scale in log2 units and a per-row power of two that keeps it inside
//    the fp16 range; scores are fp32 and are corrected by that power before the softmax.
//  * Online softmax with threshold rescaling (a row's running maximum moves only when a tile's
//    maximum exceeds it by more than 2^6), fp32 accumulators.
//  * Long key ranges are split over several workgroups; their (m, l, o) partials are merged by
//    the log-sum-exp combine kernel of merge.h.

#include <math.h>

#include "common.h"
#include "launch.h"
#include "merge.h"

namespace kvq {

constexpr int kPT = 64;       // keys per tile
constexpr int kPRows = 128;   // query rows per workgroup (4 waves x 32 MFMA columns)
constexpr int kPW = 4;        // waves per workgroup
constexpr int kKS = 136;      // fp16 per K row in LDS: 128 + 8 (rows shift by 4 banks)
constexpr int kVS = 72;       // fp16 per V^T row in LDS: 64 + 8
constexpr float kPSlack = 6.0f;
constexpr int kPTargetWgs = 512;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

struct PreParams {
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
  float* part_o;
  float* part_ml;
  unsigned* counters;  // arrivals per unit, zero between launches
  int Hq, Hkv, L, S, rep, nrows, rowblocks, nsplit, nunits;
  int fast;    // scale/bias rows [.., 2] contiguous and 16-byte aligned, byte ranges fit 32 bits
  float scale_log2;
  int causal, window;
};

// V^T slot of key `kk` (0..63) inside a tile: the 16 keys of PV k-step j = kk / 16 are stored so
// that slots 16j + 8h + i hold the keys the score layout gives lane half h at i.
__device__ __forceinline__ int v_slot_key(int slot) {
  const int j = slot >> 4, h = (slot >> 3) & 1, i = slot & 7;
  return 16 * j + (i < 4 ? 4 * h + i : 8 + 4 * h + (i - 4));
}

// Codes and scales of one tile as staged by one thread. Waves 0-1 stage V: thread t < 128 takes the
// 8 keys of V^T slot chunk t % 8 at dims [8 * (t / 8), +8) -- the 8 lanes of a row group write 8
// different slot chunks of one V^T row, and 32 consecutive rows are read per operand, both free of
// bank conflicts with 144-byte rows. Waves 2-3 stage K: thread t takes dims
// [64 * ((t - 128) / 64), +64) of key (t % 64), one scale group.
template <int BITS>
struct PreStage {
  uint32_t c[2 * BITS];  // V: key i's 8 codes at c[i * BITS / 4 ..]; K: 64 codes
  uint16_t s[8], b[8];   // V: per key; K: s[0], b[0]
};

// Per-thread constant byte offsets of the staging loads (relative to the tile's first row).
struct PreOff {
  uint32_t code[8];  // V: one per key; K: code[0]
  uint32_t sb[2];    // V: the two 4-key scale runs; K: sb[0]
};

template <int BITS>
__device__ __forceinline__ PreOff stage_offsets(const PreParams& p, int tid) {
  PreOff o;
  if (tid < 128) {
    const int c8 = tid & 7, o8 = tid >> 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) o.code[i] = (uint32_t)(v_slot_key(8 * c8 + i) * p.vc_ss + o8 * BITS);
#pragma unroll
    for (int r = 0; r < 2; ++r) o.sb[r] = (uint32_t)(v_slot_key(8 * c8 + 4 * r) * 4);
  } else {
    const int key = tid & 63, half = (tid >> 6) & 1;
    o.code[0] = (uint32_t)(key * p.kc_ss + half * 8 * BITS);
#pragma unroll
    for (int i = 1; i < 8; ++i) o.code[i] = 0;
    o.sb[0] = (uint32_t)((key * p.ksb_ss + half) * 2);
    o.sb[1] = 0;
  }
  return o;
}

// Buffer resources of one (sequence, KV head): codes and scales of the S_b valid rows.
struct PreRsrc {
  __amdgpu_buffer_rsrc_t kc, vc, ks, kb, vs, vb;
};

// Full tile (all 64 rows valid, scale rows [.., 2] contiguous): buffer loads, no address math.
template <int BITS>
__device__ __forceinline__ void stage_load_fast(PreStage<BITS>& st, const PreParams& p, const PreRsrc& rs,
                                                const PreOff& o, int k0, int tid) {
  if (tid < 128) {
    const int g = ((tid >> 3) * 8) >> 6;
    const uint32_t so = (uint32_t)(k0 * p.vc_ss);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (BITS == 8) {
        const u2 v = __builtin_amdgcn_raw_buffer_load_b64(rs.vc, o.code[i], so, 0);
        st.c[2 * i] = v[0];
        st.c[2 * i + 1] = v[1];
      } else {
        st.c[i] = __builtin_amdgcn_raw_buffer_load_b32(rs.vc, o.code[i], so, 0);
      }
    }
    const uint32_t ss = (uint32_t)(k0 * 4);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const u4 s4 = __builtin_amdgcn_raw_buffer_load_b128(rs.vs, o.sb[r], ss, 0);
      const u4 b4 = __builtin_amdgcn_raw_buffer_load_b128(rs.vb, o.sb[r], ss, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st.s[4 * r + i] = (uint16_t)(g ? (s4[i] >> 16) : (s4[i] & 0xffffu));
        st.b[4 * r + i] = (uint16_t)(g ? (b4[i] >> 16) : (b4[i] & 0xffffu));
      }
    }
  } else {
    const uint32_t so = (uint32_t)(k0 * p.kc_ss);
#pragma unroll
    for (int w = 0; w < 2 * BITS; w += 4) {
      const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs.kc, o.code[0] + 4 * w, so, 0);
      st.c[w] = v[0];
      st.c[w + 1] = v[1];
      st.c[w + 2] = v[2];
      st.c[w + 3] = v[3];
    }
    const uint32_t ss = (uint32_t)(k0 * p.ksb_ss * 2);
    st.s[0] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs.ks, o.sb[0], ss, 0);
    st.b[0] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs.kb, o.sb[0], ss, 0);
  }
}

// Any tile, any scale layout: rows clamped to the last valid one (the rows past it are masked).
template <int BITS>
__device__ __forceinline__ void stage_load_clamped(PreStage<BITS>& st, const PreParams& p, const uint8_t* kbase,
                                                   const uint8_t* vbase, const uint16_t* ksb, const uint16_t* kbb,
                                                   const uint16_t* vsb, const uint16_t* vbb, int k0, int S_b,
                                                   int tid) {
  if (tid < 128) {
    const int c8 = tid & 7, o8 = tid >> 3, g = (o8 * 8) >> 6;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = min(k0 + v_slot_key(8 * c8 + i), S_b - 1);
      const uint8_t* src = vbase + (int64_t)row * p.vc_ss + o8 * BITS;
      if constexpr (BITS == 8) {
        const u2 v = *(const u2*)src;
        st.c[2 * i] = v[0];
        st.c[2 * i + 1] = v[1];
      } else {
        st.c[i] = *(const uint32_t*)src;
      }
      st.s[i] = vsb[(int64_t)row * p.vsb_ss + g];
      st.b[i] = vbb[(int64_t)row * p.vsb_ss + g];
    }
  } else {
    const int key = tid & 63, half = (tid >> 6) & 1;
    const int row = min(k0 + key, S_b - 1);
    const uint8_t* src = kbase + (int64_t)row * p.kc_ss + half * 8 * BITS;
#pragma unroll
    for (int w = 0; w < 2 * BITS; w += 4) {
      const u4 v = *(const u4*)(src + 4 * w);
      st.c[w] = v[0];
      st.c[w + 1] = v[1];
      st.c[w + 2] = v[2];
      st.c[w + 3] = v[3];
    }
    st.s[0] = ksb[(int64_t)row * p.ksb_ss + half];
    st.b[0] = kbb[(int64_t)row * p.ksb_ss + half];
  }
}

__device__ __forceinline__ _Float16 to_half(uint16_t r, F16) { return __builtin_bit_cast(_Float16, r); }
__device__ __forceinline__ _Float16 to_half(uint16_t r, BF16) { return (_Float16)__uint_as_float((uint32_t)r << 16); }

// 1024 + c as fp16 for two codes: the code bytes selected by `sel` become the low mantissa bytes of
// 0x64xx (= 1024 + c exactly); subtracting 1024 and one packed FMA give c * s + b in fp16.
constexpr uint32_t kF16x1024 = 0x64646464u;
__device__ __forceinline__ uint32_t dequant_pair(uint32_t bytes, uint32_t sel, h2 s2, h2 b2) {
  h2 x = __builtin_bit_cast(h2, perm(kF16x1024, bytes, sel)) - h2{(_Float16)1024.0f, (_Float16)1024.0f};
  x = x * s2 + b2;
  return __builtin_bit_cast(uint32_t, x);
}

// The 8 codes of `n` (8-bit: two words; 4-bit: one word) dequantized to 4 fp16 pairs (dims 2m, 2m+1).
template <int BITS>
__device__ __forceinline__ void dequant8(const uint32_t* w, h2 s2, h2 b2, uint32_t* out) {
  if constexpr (BITS == 8) {
    out[0] = dequant_pair(w[0], 0x04010400u, s2, b2);
    out[1] = dequant_pair(w[0], 0x04030402u, s2, b2);
    out[2] = dequant_pair(w[1], 0x04010400u, s2, b2);
    out[3] = dequant_pair(w[1], 0x04030402u, s2, b2);
  } else {
    const uint32_t lo = w[0] & 0x0F0F0F0Fu, hi = (w[0] >> 4) & 0x0F0F0F0Fu;
    const uint32_t t0 = perm(hi, lo, 0x05010400u), t1 = perm(hi, lo, 0x07030602u);  // codes 0..3, 4..7 as bytes
    out[0] = dequant_pair(t0, 0x04010400u, s2, b2);
    out[1] = dequant_pair(t0, 0x04030402u, s2, b2);
    out[2] = dequant_pair(t1, 0x04010400u, s2, b2);
    out[3] = dequant_pair(t1, 0x04030402u, s2, b2);
  }
}

template <typename T, int BITS>
__device__ __forceinline__ void stage_store(const PreStage<BITS>& st, _Float16* klds, _Float16* vlds, int tid) {
  constexpr int W = BITS / 4;  // words per 8 codes
  if (tid < 128) {
    const int c8 = tid & 7, o8 = tid >> 3;
    uint32_t x[8][4];  // key i, dim pair m
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const _Float16 sh = to_half(st.s[i], T{}), bh = to_half(st.b[i], T{});
      dequant8<BITS>(&st.c[W * i], h2{sh, sh}, h2{bh, bh}, x[i]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      u4 v;
#pragma unroll
      for (int ip = 0; ip < 4; ++ip) v[ip] = perm(x[2 * ip + 1][e >> 1], x[2 * ip][e >> 1], sel);
      *(u4*)&vlds[(8 * o8 + e) * kVS + 8 * c8] = v;
    }
  } else {
    const int key = tid & 63, half = (tid >> 6) & 1;
    const _Float16 sh = to_half(st.s[0], T{}), bh = to_half(st.b[0], T{});
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      uint32_t x[4];
      dequant8<BITS>(&st.c[W * c], h2{sh, sh}, h2{bh, bh}, x);
      *(u4*)&klds[key * kKS + 64 * half + 8 * c] = u4{x[0], x[1], x[2], x[3]};
    }
  }
}

template <typename T, int BITS>
__global__ __launch_bounds__(256, 2) void prefill_attn_kernel(PreParams p) {
  __shared__ __align__(16) _Float16 k_lds[2][kPT * kKS];
  __shared__ __align__(16) _Float16 v_lds[2][128 * kVS];
  __shared__ unsigned s_arrived;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qc = lane & 31, hh = lane >> 5;

  const int unit = blockIdx.x / p.nsplit, split = blockIdx.x % p.nsplit;
  const int b = unit / (p.Hkv * p.rowblocks);
  const int kvh = (unit / p.rowblocks) % p.Hkv;
  const int rb = unit % p.rowblocks;
  const int S_b = p.seq_lens ? min(max(p.seq_lens[b], 0), p.S) : p.S;

  // ---- the workgroup's rows, their positions, and the key range they see
  const int fr0 = rb * kPRows;
  const int frl = min(fr0 + kPRows, p.nrows) - 1;
  const int pos_min = S_b - p.L + fr0 / p.rep, pos_max = S_b - p.L + frl / p.rep;
  const int hi_wg = p.causal ? min(S_b, pos_max + 1) : S_b;
  const int lo_wg = p.window > 0 ? max(0, pos_min - p.window + 1) : 0;
  // keys every row of the workgroup sees: tiles inside need no mask
  const int hi_all = p.causal ? min(S_b, pos_min + 1) : S_b;
  const int lo_all = p.window > 0 ? max(0, pos_max - p.window + 1) : 0;
  // splits cover [lo_wg rounded down to a tile, hi_wg) in whole tiles (tile starts stay 64-aligned)
  const int lo_al = lo_wg & ~(kPT - 1);
  const int span = max(hi_wg - lo_al, 0);
  const int chunk = ((span + p.nsplit - 1) / p.nsplit + kPT - 1) / kPT * kPT;
  const int k_begin = lo_al + split * chunk;
  const int k_end = min(k_begin + chunk, hi_wg);
  const int ntile = k_end > k_begin ? (k_end - k_begin + kPT - 1) / kPT : 0;

  // ---- this lane's query row (MFMA column qc of this wave)
  const int fr = fr0 + wave * 32 + qc;
  const bool row_ok = fr < p.nrows;
  const int lq = row_ok ? fr / p.rep : 0;
  const int head = kvh * p.rep + (row_ok ? fr % p.rep : 0);
  const int pos = S_b - p.L + lq;
  const int lo_r = p.window > 0 ? max(0, pos - p.window + 1) : 0;
  const int hi_r = p.causal ? min(S_b, pos + 1) : S_b;

  // ---- Q^T operand: k-step j holds dims 16j + 8hh .. +7, times scale*log2(e)*2^qe in fp16
  h8 qop[8];
  float inv2;
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)head * p.q_sh + (int64_t)lq * p.q_sl + 8 * hh;
    float qv[8][8];
    float qmax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u4 raw = row_ok ? *(const u4*)(qrow + 16 * j) : u4{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qv[j][2 * i] = to_float((uint16_t)(raw[i] & 0xffffu), T{});
        qv[j][2 * i + 1] = to_float((uint16_t)(raw[i] >> 16), T{});
        qmax = fmaxf(qmax, fmaxf(fabsf(qv[j][2 * i]), fabsf(qv[j][2 * i + 1])));
      }
    }
    qmax = max_xor32(qmax) * p.scale_log2;
    int e = 0;
    if (qmax > 0.0f) frexpf(qmax, &e);
    const int qe = 14 - e;  // |q * scale * log2(e)| * 2^qe < 2^14
    const float qmul = ldexpf(p.scale_log2, qe);
    inv2 = ldexpf(1.0f, -qe);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) qop[j][i] = (_Float16)(qv[j][i] * qmul);
  }

  const uint8_t* kbase = p.kc + (int64_t)b * p.kc_sb + (int64_t)kvh * p.kc_sh;
  const uint8_t* vbase = p.vc + (int64_t)b * p.vc_sb + (int64_t)kvh * p.vc_sh;
  const uint16_t* ksb = p.ks + (int64_t)b * p.ksb_sb + (int64_t)kvh * p.ksb_sh;
  const uint16_t* kbb = p.kb + (int64_t)b * p.ksb_sb + (int64_t)kvh * p.ksb_sh;
  const uint16_t* vsb = p.vs + (int64_t)b * p.vsb_sb + (int64_t)kvh * p.vsb_sh;
  const uint16_t* vbb = p.vb + (int64_t)b * p.vsb_sb + (int64_t)kvh * p.vsb_sh;
  PreRsrc rs;
  {
    const int64_t nr = p.fast ? S_b : 0;  // the host checks these byte ranges fit 32 bits
    rs.kc = make_rsrc(kbase, (uint32_t)(nr * p.kc_ss));
    rs.vc = make_rsrc(vbase, (uint32_t)(nr * p.vc_ss));
    rs.ks = make_rsrc(ksb, (uint32_t)(nr * p.ksb_ss * 2));
    rs.kb = make_rsrc(kbb, (uint32_t)(nr * p.ksb_ss * 2));
    rs.vs = make_rsrc(vsb, (uint32_t)(nr * p.vsb_ss * 2));
    rs.vb = make_rsrc(vbb, (uint32_t)(nr * p.vsb_ss * 2));
  }
  const PreOff off = stage_offsets<BITS>(p, tid);
  auto stage_load = [&](PreStage<BITS>& s_, int k0) {
    if (p.fast && k0 + kPT <= S_b) stage_load_fast<BITS>(s_, p, rs, off, k0, tid);
    else stage_load_clamped<BITS>(s_, p, kbase, vbase, ksb, kbb, vsb, vbb, k0, S_b, tid);
  };

  float m_run = -INFINITY, l_run = 0.0f;
  f16v oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = f16v{};

  PreStage<BITS> st;
  if (ntile > 0) {
    stage_load(st, k_begin);
    stage_store<T, BITS>(st, k_lds[0], v_lds[0], tid);
  }
  __syncthreads();

  for (int t = 0; t < ntile; ++t) {
    const int cur = t & 1;
    const int k0 = k_begin + kPT * t;
    const bool has_next = t + 1 < ntile;
    if (has_next) stage_load(st, k0 + kPT);

    // S^T = K Q^T for the two 32-key blocks of the tile (scores in log2 units times 2^qe)
    f16v sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = f16v{};
      const _Float16* krow = &k_lds[cur][(32 * kb + qc) * kKS + 8 * hh];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const h8*)(krow + 16 * j), qop[j], sacc[kb], 0, 0, 0);
    }
    // this lane's query sees keys k0 + 32kb + 8(i/4) + 4hh + i%4
    const bool need_mask = !(k0 >= lo_all && k0 + kPT <= hi_all);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
          if (key < lo_r || key >= hi_r) sacc[kb][i] = -INFINITY;
        }
    }
    float tm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) tm = fmaxf(tm, sacc[kb][i]);
    tm = max_xor32(tm) * inv2;
    if (__builtin_amdgcn_ballot_w64(tm > m_run + kPSlack) != 0) {
      const float m_new = tm > m_run + kPSlack ? fmaxf(m_run, tm) : m_run;
      const float corr = m_new == m_run ? 1.0f : exp2_fast(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] *= corr;
      m_run = m_new;
    }
    // p = 2^(acc * 2^-qe - m): rounded to fp16 it is the B operand of O^T = V^T P^T; the row sum
    // is kept in fp32
    const float nm = m_run == -INFINITY ? 0.0f : -m_run;
    h8 pop[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = exp2_fast(fmaf(sacc[j >> 1][8 * (j & 1) + 2 * e], inv2, nm));
        const float p1 = exp2_fast(fmaf(sacc[j >> 1][8 * (j & 1) + 2 * e + 1], inv2, nm));
        w[e] = pack_f16x2(p0, p1);
        l_run += p0 + p1;
      }
      pop[j] = __builtin_bit_cast(h8, w);
    }
    // O^T += V^T P^T
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const _Float16* vrow = &v_lds[cur][(32 * db + qc) * kVS + 8 * hh];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const h8*)(vrow + 16 * j), pop[j], oacc[db], 0, 0, 0);
    }

    if (has_next) stage_store<T, BITS>(st, k_lds[cur ^ 1], v_lds[cur ^ 1], tid);
    __syncthreads();
  }

  // ---- epilogue: this lane holds O^T[d][row] for d = 32db + 8(i/4) + 4hh + i%4
  float l_tot = add_xor32(l_run);
  if (p.nsplit > 1) {
    // Key split: publish this split's partials, count the arrival, and let the unit's last split to
    // arrive merge them into its own registers. Partials keep the register image, so every access
    // is a coalesced 1 KiB per wave: o word (4 db + c) of lane `lane` of wave `wave` of split s at
    // byte ((s * kPW + wave) * 16 + 4 db + c) * 1024 + 16 lane of the unit's o block; (m, l) of
    // row r at byte 8 (s * kPRows + r) of the unit's (m, l) block.
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.part_o + (int64_t)unit * p.nsplit * (kPRows * 128),
                                                (uint32_t)p.nsplit * (kPRows * 128 * 4));
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(p.part_ml + (int64_t)unit * p.nsplit * (kPRows * 2),
                                                (uint32_t)p.nsplit * (kPRows * 8));
    const uint32_t lo = (uint32_t)wave * (16 * 1024) + 16 * lane;
    const uint32_t split_o = kPW * 16 * 1024;
    const uint32_t row_ml = 8 * (wave * 32 + qc);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        store_agent_b128(ro, lo + (4 * db + c) * 1024 + split * split_o,
                         f4{oacc[db][4 * c], oacc[db][4 * c + 1], oacc[db][4 * c + 2], oacc[db][4 * c + 3]});
    if (hh == 0) store_agent_b64(rm, row_ml + split * (kPRows * 8), make_float2(m_run, l_tot));
    // The stores are acknowledged (written through to the device's coherence point) before the
    // arrival is counted, so the last arrival sees every split's partials.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) s_arrived = __hip_atomic_fetch_add(&p.counters[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != (unsigned)(p.nsplit - 1)) return;
    if (tid == 0) __hip_atomic_store(&p.counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // M = max over the splits that saw a key; weights 2^(m_s - M)
    float M = l_tot > 0.0f ? m_run : -INFINITY;
    for (int s2 = 0; s2 < p.nsplit; ++s2) {
      if (s2 == split) continue;
      const float2 ml = load_agent_b64(rm, row_ml, s2 * (kPRows * 8));
      if (ml.y > 0.0f) M = fmaxf(M, ml.x);
    }
    const float w_own = (M == -INFINITY || l_tot <= 0.0f) ? 0.0f : exp2_fast(m_run - M);
    l_tot *= w_own;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[db][i] *= w_own;
    for (int s2 = 0; s2 < p.nsplit; ++s2) {
      if (s2 == split) continue;
      const float2 ml = load_agent_b64(rm, row_ml, s2 * (kPRows * 8));
      f4 po[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) po[u] = load_agent_b128(ro, lo + u * 1024, s2 * split_o);
      const float w = (M == -INFINITY || ml.y <= 0.0f) ? 0.0f : exp2_fast(ml.x - M);
      l_tot += w * ml.y;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) oacc[db][4 * c + e] += w * po[4 * db + c][e];
    }
  }
  if (!row_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  uint16_t* orow = p.out + (int64_t)b * p.o_sb + (int64_t)head * p.o_sh + (int64_t)lq * p.o_sl;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = 32 * db + 8 * c + 4 * hh;
      u2 w;
      w[0] = (uint32_t)from_float(oacc[db][4 * c] * inv, T{}) | ((uint32_t)from_float(oacc[db][4 * c + 1] * inv, T{}) << 16);
      w[1] = (uint32_t)from_float(oacc[db][4 * c + 2] * inv, T{}) | ((uint32_t)from_float(oacc[db][4 * c + 3] * inv, T{}) << 16);
      *(u2*)(orow + d) = w;
    }
}

// ------------------------------------------------------------------------------------------
// Host side: plan, workspace, launch.

struct PrePlan {
  int rowblocks, nunits, nsplit;
};

static PrePlan prefill_plan(int B, int Hq, int Hkv, int L, int S, int window) {
  PrePlan pl;
  const int nrows = (Hq / Hkv) * L;
  pl.rowblocks = (nrows + kPRows - 1) / kPRows;
  pl.nunits = B * Hkv * pl.rowblocks;
  // keys a row block sees: the whole context, or about a window
  const int span = window > 0 ? std::min(S, window + kPRows) : S;
  const int tiles = (span + kPT - 1) / kPT;
  int ns = (kPTargetWgs + pl.nunits - 1) / pl.nunits;
  ns = std::min(ns, std::max(1, tiles / 4));  // at least about 4 tiles per split
  pl.nsplit = pl.nunits > kMaxCountedUnits ? 1 : std::max(1, std::min(ns, kMaxSplit));
  return pl;
}

// Workspace: [arrival counters (the block shared with decode)][o partials][(m, l) partials]
struct PreLayout {
  size_t o, ml, total;
};
static PreLayout prefill_layout(const PrePlan& pl) {
  PreLayout l;
  const size_t slots = (size_t)pl.nunits * pl.nsplit * kPRows;
  l.o = kCounterBytes;
  l.ml = l.o + slots * 128 * sizeof(float);
  l.total = l.ml + (slots * 2 * sizeof(float) + 255) / 256 * 256;
  return l;
}

size_t prefill_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window, int) {
  const PrePlan pl = prefill_plan(B, Hq, Hkv, L, S, window);
  if (pl.nsplit == 1) return 256;
  return prefill_layout(pl).total;
}

template <typename T, int BITS>
static hipError_t launch_prefill_t(const PreParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((prefill_attn_kernel<T, BITS>), dim3(p.nunits * p.nsplit), dim3(kPW * 64), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_prefill(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                          const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int dtype,
                          float scale, int causal, int window, void* workspace, hipStream_t stream) {
  const PrePlan pl = prefill_plan(B, Hq, Hkv, L, S, window);
  PreParams p;
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
  const PreLayout lay = prefill_layout(pl);
  p.counters = (unsigned*)workspace;
  p.part_o = (float*)((char*)workspace + lay.o);
  p.part_ml = (float*)((char*)workspace + lay.ml);
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.L = L;
  p.S = S;
  p.rep = Hq / Hkv;
  p.nrows = p.rep * L;
  p.rowblocks = pl.rowblocks;
  p.nsplit = pl.nsplit;
  p.nunits = pl.nunits;
  auto vec_ok = [](const void* base, int64_t sbb, int64_t sbh, int64_t sbs) {
    return sbs == 2 && ((uintptr_t)base % 16) == 0 && (sbb * 2) % 16 == 0 && (sbh * 2) % 16 == 0;
  };
  const int64_t big = std::max(std::max(p.kc_ss, p.vc_ss), 2 * std::max(p.ksb_ss, p.vsb_ss));
  p.fast = vec_ok(v->scales, v->sb_stride_b, v->sb_stride_h, v->sb_stride_s) &&
           vec_ok(v->biases, v->sb_stride_b, v->sb_stride_h, v->sb_stride_s) && (int64_t)S * big < ((int64_t)1 << 31);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.causal = causal;
  p.window = window;
  (void)D;
  if (dtype == KVQ_DTYPE_BF16) {
    if (bits == 8) return launch_prefill_t<BF16, 8>(p, stream);
    return launch_prefill_t<BF16, 4>(p, stream);
  }
  if (bits == 8) return launch_prefill_t<F16, 8>(p, stream);
  return launch_prefill_t<F16, 4>(p, stream);
}

}  // namespace kvq
