// Attention at head_dim 256: the reference's blocked attention over a quantized cache
// (m5engine/attention.py:29-103) for models whose heads are 256 wide, and every call over an
// unquantized cache of that width (the plain KVCache before quantized_kv_start and the sliding-window
// RotatingKVCache, which the reference leaves to mlx-lm's SDPA, attention.py:106-112). The same
// kernel at head_dim 64 serves prefill over unquantized caches of that width.
//
//   out = softmax(scale * q K^T + mask) V,  K = sK * codesK + bK,  V = sV * codesV + bV
//
// Design (gfx950):
//  * Workgroup: 4 waves, one per SIMD (up to 512 registers each: the 256-wide head needs 128
//    accumulator registers per 32 query rows and 64 for the query operand), 128 query rows of one
//    KV head, 32 per wave. Rows are head-major within the KV head (row r is position r % L of GQA
//    head r / L), the order the split merge (combine_kernel) uses.
//  * Keys stream in 32-key tiles through a ring of raw slots filled by buffer->LDS DMA (codes, and
//    scales/biases into 4-byte cells, cell 32 g + k = group g of key k; raw T rows for an
//    unquantized cache). Each tile is dequantized once per workgroup, LDS to LDS, into MFMA operands:
//    K row-major with padded rows, V transposed with its key slots permuted to the score layout.
//    The staging of tile t + 1 runs beside the MFMAs of tile t, one barrier per tile.
//  * Scores S^T = K Q^T with v_mfma_f32_32x32x16 (16 k-steps over the head): each lane holds 16
//    keys of one query, so the row max / sum are lane-local plus one permlane swap; the packed
//    probabilities are the B operand of O^T = V^T P^T (2 k-steps x 8 column blocks). The softmax
//    scale is applied to the fp32 scores.
//  * Operands: an unquantized cache's own rows (T, on the T MFMA); a quantized cache is dequantized
//    to fp16 whatever T is (a packed fp16 subtract and FMA per pair of elements: the code enters
//    exactly as 1024 + c, the FMA rounds once), with the query entering the
//    fp16 MFMA exactly as q * 2^qe (the power of two that puts the row's largest element in
//    [2^13, 2^14)) and 2^-qe folded into the softmax scale. A bf16 cache whose groups exceed the
//    fp16 range is staged times 2^-E (its range exponent, include/kvq.h) with 2^E folded back into
//    the score scale and the output; with no range word such a group dequantizes to inf and the
//    rows that read it come out NaN, never a finite wrong value.
//  * Online softmax in log2 units with threshold rescaling (the running maximum moves only when a
//    tile's maximum exceeds it by more than 2^6, so probabilities stay below 64).
//  * Keys are split over workgroups when the row blocks alone do not fill the GPU; the splits
//    leave (m, l, o) partials that combine_kernel merges (merge.h).
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "dma.h"
#include "launch.h"
#include "merge.h"

namespace kvq {

constexpr int kWT = 32;      // keys per tile
constexpr int kWW = 4;       // waves per workgroup
constexpr int kWRows = 128;  // query rows per workgroup
constexpr float kWSlack = 6.0f;

template <int D, int BITS, int G>
struct WideCfg {
  static constexpr bool DENSE = BITS == 16;
  static_assert(DENSE || ((BITS == 4 || BITS == 8) && (G == 64 || G == 128)), "4/8 bits, groups 64/128");
  static_assert(D == 256 || (D == 64 && DENSE), "head_dim 256, or 64 over an unquantized cache");
  static constexpr int NG = DENSE ? 1 : D / G;             // scale groups per row
  static constexpr int KSTEPS = D / 16;                    // QK MFMA k-steps
  static constexpr int NDB = D / 32;                       // PV MFMA column blocks
  static constexpr int KCH = D / 64;                       // K staging: 16-byte chunks per thread
  static constexpr int VPT = D / 64;                       // V^T staging: dims per thread
  static constexpr int ROWB = D * BITS / 8;                // raw bytes per key row: 128, 256, 512 (D 256)
  static constexpr int TB = kWT * ROWB;                    // raw bytes of a K (or V) tile
  static constexpr int CI = TB / 1024;                     // 1 KiB DMAs per K (or V) tile
  static constexpr int CPR = ROWB / 16;                    // 16-byte chunks per raw row
  static constexpr int RPI = 64 / CPR;                     // raw rows per 1 KiB DMA
  static constexpr int SBA = DENSE ? 0 : 4 * kWT * NG;     // bytes of one scale/bias cell array
  static constexpr int NSB = DENSE ? 0 : NG / 2;           // 64-cell DMAs per array (2 groups x 32 keys)
  static constexpr int SLOT = 2 * TB + 4 * SBA;            // [K raw][V raw][sK][bK][sV][bV]
  static constexpr int NR = DENSE ? 2 : 3;                 // raw ring slots
  static constexpr int CPW = 2 * CI / kWW;                 // code DMAs per wave per tile
  static constexpr int IPW = CPW + NSB;                    // DMAs per wave per tile (wave a loads array a)
  static constexpr int KROW = D * 2 + 16;                  // K operand row pitch: the row + 16 bytes of padding
  static constexpr int KOPB = kWT * KROW;                  // bytes of a K operand tile
  static constexpr int VOPB = D * kWT * 2;                 // bytes of a V^T operand tile
  static constexpr int LDS = NR * SLOT + 2 * (KOPB + VOPB);  // ring + double-buffered K and V^T
  // The raw K rows land with their 16-byte chunks XOR-swizzled: position x of row r holds chunk
  // x ^ kswz(r). The K staging reads a chunk of 32 consecutive rows per 32-lane half; rows r and
  // r + 32 / CPR share banks (128 banks of 4 bytes), and kswz gives the CPR rows of each such class
  // distinct positions, so those reads are free of bank conflicts.
  static_assert(CPR >= 8 && CPR <= 32, "raw rows of 128 to 512 bytes");
  static constexpr int kswz(int r) { return (r / (32 / CPR)) % CPR; }
  static_assert(2 * CI % kWW == 0, "code DMAs divide over the waves");
  static_assert(LDS <= 160 * 1024, "fits the LDS");
};

struct WideParams {
  const uint16_t* q;
  int64_t q_sb, q_sh, q_sl;  // elements
  const uint8_t* kc;         // codes (quantized) or raw T rows (unquantized)
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
  float* part_o;   // nsplit > 1: o per (unit, split, row), D floats
  float* part_ml;  // (m, l) pairs, same index
  int Hq, Hkv, L, S, rep, nrows, rowblocks, nsplit, nunits;
  float scale_log2;
  int causal, window;
  // paged pools (PAGED kernels): rows of sequence b live in 64-row pages, page table[b][r / 64]; the
  // codes / scales / biases batch strides above are then page strides
  const int32_t* table;
  int64_t table_stride;
  int num_pages;
  // the caches' range exponents (kvq_qtensor.range_exp), or null: the fp16 operands are staged
  // times 2^-E, and 2^E returns in the score scale (K) and the output (V)
  const int32_t* k_rexp;
  const int32_t* v_rexp;
  // general mask (kvq_mask, MASKED kernels): kind 0 = none
  const void* mask;
  int mask_kind;
  int64_t m_sb, m_skv, m_srep, m_sl;
  // the head dimension of the rows (NARROW kernels: a multiple of 8 below D, the unquantized rows
  // past 128 dims): their queries' dims from dv on are zero and only dv dims are stored
  int dv;
};

// A general mask (kvq_mask) on the lane's 16 scores of a tile (keys k0 + 8 (i / 4) + 4 h + i % 4 of
// query row (b, kvh, j, l)), in the raw product units the kernel scales by kf later: a boolean mask
// sends hidden keys to -inf, an additive one adds its value times log2(e) / kf. Keys outside
// [lo, hi) are already -inf and are not read.
__device__ __forceinline__ void wide_apply_mask(const WideParams& p, int b, int kvh, int j, int l, int k0, int h, int lo,
                                                int hi, float add_scale, float (&s)[16]) {
  const int64_t row = (int64_t)b * p.m_sb + (int64_t)kvh * p.m_skv + (int64_t)j * p.m_srep + (int64_t)l * p.m_sl;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int k = k0 + 8 * (i >> 2) + 4 * h + (i & 3);
    if (k < lo || k >= hi) continue;
    const int64_t e = row + k;
    if (p.mask_kind == KVQ_MASK_BOOL) {
      if (((const uint8_t*)p.mask)[e] == 0) s[i] = -INFINITY;
    } else {
      float a;
      if (p.mask_kind == KVQ_MASK_F32) {
        a = ((const float*)p.mask)[e];
      } else if (p.mask_kind == KVQ_MASK_BF16) {
        a = to_float(((const uint16_t*)p.mask)[e], BF16{});
      } else {
        a = to_float(((const uint16_t*)p.mask)[e], F16{});
      }
      s[i] += a * add_scale;
    }
  }
}

// The key held in V^T slot 8 c + e (c = 0..3, e = 0..7): PV k-step c / 2 takes, in lane half c % 2,
// the probabilities the score layout gives that half as its values 8 (c / 2) + e, which are keys
// 16 (c / 2) + 4 (c % 2) + (e < 4 ? e : e + 4).
__host__ __device__ constexpr int w_slot_key(int c, int e) { return 16 * (c >> 1) + 4 * (c & 1) + (e < 4 ? e : e + 4); }

// A scale/bias cell (the value in its low half, the cache's dtype) as fp16. A bf16 value beyond the
// fp16 range becomes inf, and the rows that read the group come out non-finite.
__device__ __forceinline__ _Float16 cell_half(uint32_t cell, F16) { return __builtin_bit_cast(_Float16, (uint16_t)cell); }
__device__ __forceinline__ _Float16 cell_half(uint32_t cell, BF16) { return (_Float16)__uint_as_float(cell << 16); }
// The same times m = 2^-E (the cache's range exponent) when SCALED, exact in fp32 and rounded once
// to fp16.
template <typename T, bool SCALED>
__device__ __forceinline__ _Float16 cell_half_e(uint32_t cell, float m) {
  if constexpr (!SCALED) {
    return cell_half(cell, T{});
  } else {
    return (_Float16)(to_float((uint16_t)cell, T{}) * m);
  }
}

// Two codes as fp16 s * c + b in packed arithmetic: the code bytes `sel` picks become the low
// mantissa bytes of 0x64xx (1024 + c, exact), then one packed subtract and one packed FMA (rounded
// once to fp16).
__device__ __forceinline__ uint32_t dq_pair(uint32_t bytes, uint32_t sel, h2 s2, h2 b2) {
  h2 x = __builtin_bit_cast(h2, perm(0x64646464u, bytes, sel)) - h2{(_Float16)1024.0f, (_Float16)1024.0f};
  return __builtin_bit_cast(uint32_t, x * s2 + b2);
}
constexpr uint32_t kSelLo = 0x04010400u;  // bytes 0, 1 -> fp16 pair
constexpr uint32_t kSelHi = 0x04030402u;  // bytes 2, 3 -> fp16 pair
// 4-bit codes 0..3 (or 4..7) of a word as one byte each
__device__ __forceinline__ uint32_t nibbles_lo(uint32_t w) {
  return perm((w >> 4) & 0x0F0F0F0Fu, w & 0x0F0F0F0Fu, 0x05010400u);
}
__device__ __forceinline__ uint32_t nibbles_hi(uint32_t w) {
  return perm((w >> 4) & 0x0F0F0F0Fu, w & 0x0F0F0F0Fu, 0x07030602u);
}

// K of a raw tile into the K operand tile (OT elements): thread t dequantizes dims
// [D/8 p, D/8 (p + 1)) of key r (t = 32 p + r) and writes them as KCH chunks of 8 dims. Rows are 16
// bytes longer than the data (528 bytes at D = 256), so the 32 lanes that read one 16-byte column of
// 32 keys hit distinct banks and a lane's reads of one row are one base address plus immediates.
// Consecutive lanes take consecutive keys: a 16-byte LDS write is served 8 lanes at a time over 128
// bytes, and 8 rows 528 bytes apart fill those 128 bytes without a conflict (8 lanes of one row,
// 64 bytes apart, met 4 to a bank: 2.3x the write time). The raw reads follow kswz.
template <typename T, typename OT, int D, int BITS, int G, bool SCALED = false>
__device__ __forceinline__ void wide_stage_k(const uint8_t* raw, uint8_t* kop, int t, bool& range_bad, float kmul) {
  using C = WideCfg<D, BITS, G>;
  const int r = t & 31, p = t >> 5, sw = C::kswz(r);
  const uint8_t* row = raw + r * C::ROWB;
  u4 w[C::KCH];
  if constexpr (C::DENSE) {
#pragma unroll
    for (int c = 0; c < C::KCH; ++c) w[c] = *(const u4*)(row + 16 * ((C::KCH * p + c) ^ sw));
  } else {
    const int g = 32 * p / G;
    const uint32_t* cells = (const uint32_t*)(raw + 2 * C::TB);
    const _Float16 sh = cell_half_e<T, SCALED>(cells[32 * g + r], kmul);
    const _Float16 bh = cell_half_e<T, SCALED>(cells[C::SBA / 4 + 32 * g + r], kmul);
    // MLX's bias is the group's larger-magnitude extreme: it converts to inf exactly when some
    // value of the group lies beyond the fp16 range
    if constexpr (T::id == KVQ_DTYPE_BF16) range_bad |= __builtin_isinf((float)bh);
    const h2 s2 = {sh, sh}, b2 = {bh, bh};
    if constexpr (BITS == 8) {
      const u4 a = *(const u4*)(row + 16 * ((2 * p) ^ sw)), b = *(const u4*)(row + 16 * ((2 * p + 1) ^ sw));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wa = i < 2 ? a[2 * i] : b[2 * (i - 2)], wb = i < 2 ? a[2 * i + 1] : b[2 * (i - 2) + 1];
        w[i] = u4{dq_pair(wa, kSelLo, s2, b2), dq_pair(wa, kSelHi, s2, b2), dq_pair(wb, kSelLo, s2, b2),
                  dq_pair(wb, kSelHi, s2, b2)};
      }
    } else {
      const u4 a = *(const u4*)(row + 16 * (p ^ sw));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = nibbles_lo(a[i]), hi = nibbles_hi(a[i]);
        w[i] = u4{dq_pair(lo, kSelLo, s2, b2), dq_pair(lo, kSelHi, s2, b2), dq_pair(hi, kSelLo, s2, b2),
                  dq_pair(hi, kSelHi, s2, b2)};
      }
    }
  }
#pragma unroll
  for (int c = 0; c < C::KCH; ++c) *(u4*)(kop + r * C::KROW + 16 * (C::KCH * p + c)) = w[c];
}

// V of a raw tile into the V^T operand tile: thread t = 64 c + j dequantizes dims
// [VPT j, VPT (j + 1)) (VPT = D / 64) of the 8 keys of slot chunk c and writes, for each of those
// dims, the chunk's 8 slots (16 bytes) to row d at chunk position c ^ ((d >> 2) & 3) (rows are 64
// bytes: 32 slots), the row itself stored at row d ^ ((d >> 4) & 1).
template <typename T, typename OT, int D, int BITS, int G, bool SCALED = false>
__device__ __forceinline__ void wide_stage_v(const uint8_t* raw, uint8_t* vop, int t, bool& range_bad, float vmul) {
  using C = WideCfg<D, BITS, G>;
  const int c = t >> 6, j = t & 63;
  const uint8_t* vraw = raw + C::TB;
  // xp[e][q]: key e's dims 2q, 2q + 1 of the thread's VPT as a packed pair (one 16-bit value when
  // VPT is 1)
  uint32_t xp[8][(C::VPT + 1) / 2];
  if constexpr (C::DENSE) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (C::VPT == 4) {
        const u2 v = *(const u2*)(vraw + w_slot_key(c, e) * C::ROWB + 8 * j);
        xp[e][0] = v[0];
        xp[e][1] = v[1];
      } else {
        xp[e][0] = *(const uint16_t*)(vraw + w_slot_key(c, e) * C::ROWB + 2 * j);
      }
    }
  } else {
    static_assert(C::VPT == 4, "quantized caches at head_dim 256");
    const int g = 4 * j / G;
    const uint8_t* cells = raw + 2 * C::TB + 2 * C::SBA + 4 * 32 * g;  // sV, then bV one array later
    const int kb0 = w_slot_key(c, 0);
    const u4 s_lo = *(const u4*)(cells + 4 * kb0), s_hi = *(const u4*)(cells + 4 * (kb0 + 8));
    const u4 b_lo = *(const u4*)(cells + C::SBA + 4 * kb0), b_hi = *(const u4*)(cells + C::SBA + 4 * (kb0 + 8));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 sh = cell_half_e<T, SCALED>(e < 4 ? s_lo[e] : s_hi[e - 4], vmul);
      const _Float16 bh = cell_half_e<T, SCALED>(e < 4 ? b_lo[e] : b_hi[e - 4], vmul);
      if constexpr (T::id == KVQ_DTYPE_BF16) range_bad |= __builtin_isinf((float)bh);
      uint32_t bytes;  // codes of the thread's 4 dims, one byte each
      if constexpr (BITS == 8) {
        bytes = *(const uint32_t*)(vraw + w_slot_key(c, e) * C::ROWB + 4 * j);
      } else {
        bytes = nibbles_lo(*(const uint16_t*)(vraw + w_slot_key(c, e) * C::ROWB + 2 * j));
      }
      xp[e][0] = dq_pair(bytes, kSelLo, h2{sh, sh}, h2{bh, bh});
      xp[e][1] = dq_pair(bytes, kSelHi, h2{sh, sh}, h2{bh, bh});
    }
  }
  // V^T row of dim i: slots e = 0..7, packed (2a, 2a + 1): the matching halves of two keys' pairs
#pragma unroll
  for (int i = 0; i < C::VPT; ++i) {
    u4 o;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      if constexpr (C::VPT == 1) {
        o[a] = (xp[2 * a][0] & 0xffffu) | (xp[2 * a + 1][0] << 16);
      } else {
        o[a] = perm(xp[2 * a + 1][i >> 1], xp[2 * a][i >> 1], (i & 1) ? 0x07060302u : 0x05040100u);
      }
    }
    // row d is stored at row d ^ ((d >> 4) & 1): the 8 consecutive lanes of a write (rows 4 apart)
    // then fill both 64-byte halves of a 128-byte bank window, 8 distinct 16-byte slots
    const int d = C::VPT * j + i;
    *(u4*)(vop + (d ^ ((d >> 4) & 1)) * (kWT * 2) + 16 * (c ^ ((d >> 2) & 3))) = o;
  }
}

// MASKED: compiled with a general mask (kvq_mask) read beside every tile; the other instantiations
// carry no trace of it.
template <typename T, int D, int BITS, int G, bool PAGED = false, bool MASKED = false, bool NARROW = false>
__global__ __launch_bounds__(kWW * 64, 1) void wide_attn_kernel(WideParams p) {
  using C = WideCfg<D, BITS, G>;
  static_assert(!NARROW || C::DENSE, "narrow rows: unquantized caches");
  static_assert(!PAGED || !C::DENSE, "paged pools hold quantized caches");
  using OT = std::conditional_t<C::DENSE, T, F16>;  // operand type
  __shared__ __align__(16) uint8_t smem[C::LDS];
  uint8_t* const ring = smem;
  uint8_t* const kop = smem + C::NR * C::SLOT;  // [2][KOPB]
  uint8_t* const vop = kop + 2 * C::KOPB;       // [2][VOPB]

  const int tid = threadIdx.x;
  const int lane = __lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, h = lane >> 5;

  // ---- workgroup -> (unit, split); a unit is (sequence, KV head, row block)
  const int unit = blockIdx.x / p.nsplit, split = blockIdx.x % p.nsplit;
  const int b = unit / (p.Hkv * p.rowblocks);
  const int kvh = (unit / p.rowblocks) % p.Hkv;
  const int rb = unit % p.rowblocks;
  const int S_b = p.seq_lens ? min(max(load_uniform_i32(p.seq_lens, b), 0), p.S) : p.S;

  // the row block's positions: one head's contiguous run, or every position when it spans heads
  const int r0 = rb * kWRows, r1 = min(r0 + kWRows, p.nrows) - 1;
  const bool one_head = r0 / p.L == r1 / p.L;
  const int lq_min = one_head ? r0 % p.L : 0, lq_max = one_head ? r1 % p.L : p.L - 1;
  const int key_hi = p.causal ? min(S_b, max(0, S_b - p.L + lq_max + 1)) : S_b;
  const int key_lo = p.window > 0 ? min(key_hi, max(0, S_b - p.L + lq_min - p.window + 1)) : 0;
  const int t_lo = key_lo / kWT, t_hi = (key_hi + kWT - 1) / kWT;
  const int cps = (t_hi - t_lo + p.nsplit - 1) / p.nsplit;
  const int t_begin = min(t_hi, t_lo + split * cps), t_end = min(t_hi, t_begin + cps);
  const int ntile = t_end - t_begin;

  // ---- raw tile DMAs: wave w issues code DMAs [w CPW, (w + 1) CPW) (K first, then V) and the NSB
  // loads of scale/bias array w (sK, bK, sV, bV)
  const uint8_t* kbase = p.kc + (int64_t)b * p.kc_sb + (int64_t)kvh * p.kc_sh;
  const uint8_t* vbase = p.vc + (int64_t)b * p.vc_sb + (int64_t)kvh * p.vc_sh;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)((int64_t)S_b * p.kc_ss));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, (uint32_t)((int64_t)S_b * p.vc_ss));
  __amdgpu_buffer_rsrc_t code_r[C::CPW];
  uint32_t code_vo[C::CPW], code_lds[C::CPW];
  int64_t code_ss[C::CPW];
  // waves 0 and 1 load K (swizzled rows), waves 2 and 3 load V: a mask the compiler does not split
  // the offsets on
  static_assert(2 * C::CPW == C::CI, "two waves load each of K and V");
  const int kmask = opaque(wave < 2 ? C::CPR - 1 : 0);
#pragma unroll
  for (int j = 0; j < C::CPW; ++j) {
    const int q = wave * C::CPW + j;
    const bool is_k = q < C::CI;
    const int i = is_k ? q : q - C::CI;
    code_r[j] = is_k ? krs : vrs;
    code_ss[j] = is_k ? p.kc_ss : p.vc_ss;
    const int rr = i * C::RPI + lane / C::CPR;  // the row of the tile this lane's 16 bytes belong to
    code_vo[j] = (uint32_t)(rr * code_ss[j] + 16 * ((lane % C::CPR) ^ (C::kswz(rr) & kmask)));
    code_lds[j] = (is_k ? 0 : C::TB) + 1024 * i;
  }
  __amdgpu_buffer_rsrc_t sb_r = krs;
  int64_t sb_ss = 0;
  uint32_t sb_vo[C::NSB > 0 ? C::NSB : 1] = {};
  const uint8_t* sb_page0 = nullptr;  // paged pools: the wave's scale/bias array at page 0 of this head
  int64_t sb_ps = 0;                  // ... and its page stride in bytes
  if constexpr (!C::DENSE) {
    const uint16_t* arr = wave == 0 ? p.ks : wave == 1 ? p.kb : wave == 2 ? p.vs : p.vb;
    const int64_t sb_b = wave < 2 ? p.ksb_sb : p.vsb_sb, sb_h = wave < 2 ? p.ksb_sh : p.vsb_sh;
    sb_ss = wave < 2 ? p.ksb_ss : p.vsb_ss;
    sb_r = make_rsrc(arr + (int64_t)b * sb_b + (int64_t)kvh * sb_h, (uint32_t)((int64_t)S_b * sb_ss * 2));
    sb_page0 = (const uint8_t*)(arr + (int64_t)kvh * sb_h);
    sb_ps = 2 * sb_b;
#pragma unroll
    for (int j = 0; j < C::NSB; ++j) sb_vo[j] = (uint32_t)(2 * ((lane & 31) * sb_ss + 2 * j + (lane >> 5)));
  }
  const uint32_t ring_lds = lds_addr(ring);
  const int t_last = max(ntile - 1, 0);
  // paged pools: a 32-key tile (32-aligned) lies in one 64-row page; its page number is read one
  // tile ahead (a scalar load that the next issue consumes), clamped to the pool, and the tile's
  // buffer resources span only that page's valid rows, so rows past S_b still read as zero
  auto page_of = [&](int i) -> int {
    const int k0 = (t_begin + min(i, t_last)) * kWT;
    const int pi = min(k0, max(S_b - 1, 0)) >> 6;
    return __builtin_amdgcn_readfirstlane(min(max(p.table[(int64_t)b * p.table_stride + pi], 0), p.num_pages - 1));
  };
  int pg_next = PAGED ? page_of(0) : 0;
  // tile i of this split into ring slot i % NR; past the last tile it re-reads the last one, so every
  // wait below sees the same number of loads in flight
  auto issue = [&](int i) {
    const int k0 = (t_begin + min(i, t_last)) * kWT;
    const uint32_t slot = ring_lds + (uint32_t)((i % C::NR) * C::SLOT);
    if constexpr (PAGED) {
      const int pg = pg_next;
      pg_next = page_of(i + 1);
      const int nv = __builtin_amdgcn_readfirstlane(max(min(64, S_b - (k0 & ~63)), 0));  // valid rows of the page
      const int r0p = k0 & 63;                                                          // the tile's first row in it
#pragma unroll
      for (int j = 0; j < C::CPW; ++j) {
        const bool is_k = wave * C::CPW + j < C::CI;
        const uint8_t* base = is_k ? p.kc + (int64_t)kvh * p.kc_sh + (int64_t)pg * p.kc_sb
                                   : p.vc + (int64_t)kvh * p.vc_sh + (int64_t)pg * p.vc_sb;
        dma_b128(make_rsrc(base, (uint32_t)(nv * code_ss[j])), slot + code_lds[j], code_vo[j], (uint32_t)(r0p * code_ss[j]));
      }
      const __amdgpu_buffer_rsrc_t r = make_rsrc(sb_page0 + (int64_t)pg * sb_ps, (uint32_t)(nv * sb_ss * 2));
#pragma unroll
      for (int j = 0; j < C::NSB; ++j)
        dma_b16(r, slot + 2 * C::TB + C::SBA * wave + 256 * j, sb_vo[j], (uint32_t)(2 * r0p * sb_ss));
    } else {
#pragma unroll
      for (int j = 0; j < C::CPW; ++j) dma_b128(code_r[j], slot + code_lds[j], code_vo[j], (uint32_t)(k0 * code_ss[j]));
      if constexpr (!C::DENSE) {
#pragma unroll
        for (int j = 0; j < C::NSB; ++j)
          dma_b16(sb_r, slot + 2 * C::TB + C::SBA * wave + 256 * j, sb_vo[j], (uint32_t)(2 * k0 * sb_ss));
      }
    }
  };

  // ---- this lane's query row and its operand (rows past the block's end read row 0 of the head
  // and are never stored)
  const int row = r0 + 32 * wave + n;
  const bool row_ok = row < p.nrows;
  const int hq = kvh * p.rep + (row_ok ? row / p.L : 0);
  const int lq = row_ok ? row % p.L : 0;
  const int qpos = S_b - p.L + lq;
  const int lo_r = p.window > 0 ? max(0, qpos - p.window + 1) : 0;
  const int hi_r = p.causal ? min(S_b, qpos + 1) : S_b;
  // keys every row of the block sees: tiles inside need no mask
  const int lo_all = p.window > 0 ? max(0, S_b - p.L + lq_max - p.window + 1) : 0;
  const int hi_all = p.causal ? S_b - p.L + lq_min + 1 : S_b;

  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < C::NR; ++i) issue(i);
  __builtin_amdgcn_sched_barrier(0);

  u4 qop[C::KSTEPS];
  float kf = p.scale_log2;  // fp32 score -> log2 units
  // range exponents of the K and V caches (0 for an unquantized cache, an fp16 cache -- whose
  // values always fit the fp16 operands -- or a null pointer), read after the query and the first
  // tiles are requested, so that waiting for the word delays no load
  int ek = 0, ev = 0;
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)lq * p.q_sl + 8 * h;
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j)
      qop[j] = (!NARROW || 16 * j + 8 * h < p.dv) ? *(const u4*)(qrow + 16 * j) : u4{0, 0, 0, 0};
    if constexpr (!C::DENSE && T::id == KVQ_DTYPE_BF16) {
      if (p.k_rexp) ek = min(max(*p.k_rexp, 0), 127);
      if (p.v_rexp) ev = min(max(*p.v_rexp, 0), 127);
    }
    if constexpr (!C::DENSE) {
      // q * 2^qe in fp16, exact: the row's largest |q| lands in [2^13, 2^14)
      float qmax = 0.0f;
#pragma unroll
      for (int j = 0; j < C::KSTEPS; ++j)
#pragma unroll
        for (int a = 0; a < 8; ++a) qmax = fmaxf(qmax, fabsf(to_float((uint16_t)(qop[j][a >> 1] >> (16 * (a & 1))), T{})));
      qmax = max_xor32(qmax);
      int qe = 0;
      if (qmax > 0.0f) {
        frexpf(qmax, &qe);
        qe = 14 - qe;
      }
      const float qs = ldexpf(1.0f, qe);
      kf = ldexpf(p.scale_log2, ek - qe);  // the K operands are staged times 2^-ek
#pragma unroll
      for (int j = 0; j < C::KSTEPS; ++j)
#pragma unroll
        for (int a = 0; a < 4; ++a)
          qop[j][a] = pack_f16x2(to_float((uint16_t)(qop[j][a] & 0xffffu), T{}) * qs,
                                 to_float((uint16_t)(qop[j][a] >> 16), T{}) * qs);
    }
  }

  const float kmul = ldexpf(1.0f, -ek), vmul = ldexpf(1.0f, -ev);  // the staging's factors 2^-E
  float m_run = -INFINITY, l_run = 0.0f;
  bool range_bad = false;  // a tile this thread staged holds a bf16 group beyond the fp16 range
  f16v oacc[C::NDB];
#pragma unroll
  for (int db = 0; db < C::NDB; ++db) oacc[db] = f16v{};

  // K operand of k-step j: key n, dims 16 j + 8 h .. + 8; V^T operand of column block db, k-step s:
  // row d = 32 db + n (stored at row d ^ ((d >> 4) & 1)), chunk position (2 s + h) ^ ((n >> 2) & 3)
  const uint32_t k_off = (uint32_t)(n * C::KROW + 16 * h);
  const uint32_t v_off = (uint32_t)((n ^ ((n >> 4) & 1)) * (kWT * 2));  // row n's place (see wide_stage_v)
  const int v_sw = (n >> 2) & 3;

  // One step: tile t's products from operand buffers (kt, vt), and tile t + 1's staging from raw
  // slot raw1 into (kd, vd). The step is one basic block: each product's operand reads are issued
  // ahead of its MFMA chain, and the staging's independent VALU work fills the chain's issue slots.
  auto step = [&](auto scaled, const uint8_t* kt, const uint8_t* vt, int k0, const uint8_t* raw1, uint8_t* kd,
                  uint8_t* vd) {
    constexpr bool SC = decltype(scaled)::value;
    // K operands through a ring of KR registers, read KR MFMAs ahead
    constexpr int KR = C::KSTEPS < 8 ? C::KSTEPS : 8;
    u4 ka[KR];
#pragma unroll
    for (int j = 0; j < KR; ++j) ka[j] = *(const u4*)(kt + k_off + 32 * j);
    wide_stage_k<T, OT, D, BITS, G, SC>(raw1, kd, tid, range_bad, kmul);
    f16v s = f16v{};
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j) {
      s = mfma_32x32x16(ka[j % KR], qop[j], s, OT{});
      if (j + KR < C::KSTEPS) ka[j % KR] = *(const u4*)(kt + k_off + 32 * (j + KR));
    }
    // value i of the lane is key k0 + 8 (i / 4) + 4 h + i % 4 of query row n
    if (MASKED || !(k0 >= lo_all && k0 + kWT <= hi_all)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int k = k0 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (k < lo_r || k >= hi_r) s[i] = -INFINITY;
      }
      if constexpr (MASKED) {
        float sv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = s[i];
        if (row_ok) wide_apply_mask(p, b, kvh, hq - kvh * p.rep, lq, k0, h, lo_r, hi_r, 1.4426950408889634f / kf, sv);
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = sv[i];
      }
    }
    float tm = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) tm = fmaxf(tm, s[i]);
    tm = max_xor32(tm) * kf;
    if (__builtin_amdgcn_ballot_w64(tm > m_run + kWSlack) != 0) {
      const float m_new = tm > m_run + kWSlack ? fmaxf(m_run, tm) : m_run;
      const float corr = m_new == m_run ? 1.0f : exp2_fast(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) oacc[db] *= corr;
      m_run = m_new;
    }
    const float nm = m_run == -INFINITY ? 0.0f : -m_run;
    u4 pop[2];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float p0 = exp2_fast(fmaf(s[8 * st + 2 * a], kf, nm));
        const float p1 = exp2_fast(fmaf(s[8 * st + 2 * a + 1], kf, nm));
        pop[st][a] = pack2(p0, p1, OT{});
        l_run = add_pair(pop[st][a], l_run, OT{});
      }
    // V^T operands likewise, VR MFMAs ahead
    constexpr int NV = 2 * C::NDB, VR = NV < 8 ? NV : 8;
    auto vop_at = [&](int i) {
      return *(const u4*)(vt + 32 * (i >> 1) * (kWT * 2) + v_off + 16 * ((2 * (i & 1) + h) ^ v_sw));
    };
    u4 va[VR];
#pragma unroll
    for (int i = 0; i < VR; ++i) va[i] = vop_at(i);
    wide_stage_v<T, OT, D, BITS, G, SC>(raw1, vd, tid, range_bad, vmul);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      oacc[i >> 1] = mfma_32x32x16(va[i % VR], pop[i & 1], oacc[i >> 1], OT{});
      if (i + VR < NV) va[i % VR] = vop_at(i + VR);
    }
  };

  // ---- the tile loop: tile t is computed from operand buffer t % 2 while tile t + 1 is staged into
  // the other; raw slot t % NR is refilled with tile t + NR once tile t is staged. Every step stages:
  // past the last tile the raw slot holds a re-read of the last tile, staged into a buffer no step
  // reads. Every wave computes (rows past the block's end are clamped and never stored).
  // The loop is compiled twice: staging the cache as it is, and staging it times 2^-E (a bf16 cache
  // whose range exponent is not 0), so that the common case carries no scaling work.
  auto tile_loop = [&](auto scaled) {
    constexpr bool SC = decltype(scaled)::value;
    wait_vm<0>();  // the query and the first NR raw tiles
    __syncthreads();
    wide_stage_k<T, OT, D, BITS, G, SC>(ring, kop, tid, range_bad, kmul);
    wide_stage_v<T, OT, D, BITS, G, SC>(ring, vop, tid, range_bad, vmul);
    for (int t = 0; t < ntile; ++t) {
      if constexpr (C::NR == 3) {
        wait_vm<C::IPW>();  // tile t + 1 has landed (tile t + 2 may be in flight)
      } else {
        wait_vm<0>();
      }
      __syncthreads();  // operand buffer t % 2 is complete; raw slot t % NR is free
      issue(t + C::NR);
      const int ck = opaque((t & 1) * C::KOPB), nk = opaque(((t + 1) & 1) * C::KOPB);
      const int cv = opaque((t & 1) * C::VOPB), nv = opaque(((t + 1) & 1) * C::VOPB);
      step(scaled, kop + ck, vop + cv, (t_begin + t) * kWT, ring + opaque(((t + 1) % C::NR) * C::SLOT), kop + nk,
           vop + nv);
    }
  };
  if (ntile > 0) {
    if constexpr (!C::DENSE && T::id == KVQ_DTYPE_BF16) {
      if (ek != 0 || ev != 0) {
        tile_loop(std::integral_constant<bool, true>{});
      } else {
        tile_loop(std::integral_constant<bool, false>{});
      }
    } else {
      tile_loop(std::integral_constant<bool, false>{});
    }
  }
  wait_vm<0>();  // the look-ahead loads land before the workgroup's LDS is released
  float l_tot = add_xor32(l_run);
  if constexpr (!C::DENSE && T::id == KVQ_DTYPE_BF16) {
    // a group beyond the fp16 range poisons every row of the workgroup: NaN output rows, or NaN
    // partials with (m, l) = (0, 1), which the split merge counts and carries to the output rows
    // (its weight times NaN is NaN, zero weight included)
    if (__syncthreads_or(range_bad)) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) oacc[db] = f16v{} + __builtin_nanf("");
      m_run = 0.0f;
      l_tot = 1.0f;
    }
  }

  // ---- epilogue: lane (n, h) holds O^T rows 32 db + 8 i + 4 h + j (j = 0..3) of query row n
  if (!row_ok) return;
  if (p.nsplit == 1) {
    const float inv = l_tot > 0.0f ? ldexpf(1.0f / l_tot, ev) : 0.0f;  // the V operands were staged times 2^-ev
    uint16_t* orow = p.out + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)lq * p.o_sl + 4 * h;
#pragma unroll
    for (int db = 0; db < C::NDB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u2 w;
        w[0] = pack2(oacc[db][4 * i] * inv, oacc[db][4 * i + 1] * inv, T{});
        w[1] = pack2(oacc[db][4 * i + 2] * inv, oacc[db][4 * i + 3] * inv, T{});
        if (!NARROW || 32 * db + 8 * i + 4 * h < p.dv) *(u2*)(orow + 32 * db + 8 * i) = w;
      }
  } else {
    const int64_t pi = ((int64_t)unit * p.nsplit + split) * kWRows + (row - r0);
    float* po = p.part_o + pi * D + 4 * h;
    const float vs = ldexpf(1.0f, ev);  // the partial in the cache's units (the V operands were staged times 2^-ev)
#pragma unroll
    for (int db = 0; db < C::NDB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *(f4*)(po + 32 * db + 8 * i) =
            f4{oacc[db][4 * i] * vs, oacc[db][4 * i + 1] * vs, oacc[db][4 * i + 2] * vs, oacc[db][4 * i + 3] * vs};
    if (h == 0) ((float2*)p.part_ml)[pi] = make_float2(m_run, l_tot);
  }
}

// ------------------------------------------------------------------------------------------
// Host side: plan, workspace, launch.

struct WidePlan {
  int rowblocks, nunits, nsplit;
};

// Splits fill about 256 workgroups when the row blocks alone do not; each split keeps at least two
// tiles of the widest row block's keys.
static WidePlan wide_plan(int B, int Hq, int Hkv, int L, int S, int window) {
  WidePlan pl;
  const int nrows = (Hq / Hkv) * L;
  pl.rowblocks = (nrows + kWRows - 1) / kWRows;
  pl.nunits = B * Hkv * pl.rowblocks;
  const int span = window > 0 ? std::min(S, window + std::min(L, kWRows) - 1 + kWT) : S;
  const int tiles = (span + kWT - 1) / kWT;
  pl.nsplit = 1;
  if (pl.nunits < 192) pl.nsplit = std::max(1, std::min({(256 + pl.nunits - 1) / pl.nunits, tiles / 2, kMaxSplit}));
  return pl;
}

// Workspace: [the arrival counter block every launch reserves (merge.h), left untouched][(m, l) per
// row and split][o per row and split]; a launch without splits writes none of it.
size_t wide_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window) {
  const WidePlan pl = wide_plan(B, Hq, Hkv, L, S, window);
  if (pl.nsplit == 1) return kCounterBytes;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t rows = (size_t)pl.nunits * pl.nsplit * kWRows;
  return kCounterBytes + up(rows * sizeof(float2)) + up(rows * D * sizeof(float));
}

template <typename T, int D, int BITS, int G, bool PAGED = false>
static hipError_t launch_wide_t(const WideParams& p, hipStream_t stream) {
  if (p.dv != D) {
    // unquantized rows narrower than 256 dims (decode_kernel_dim), plain or masked
    if constexpr (D == 256 && BITS == 16 && !PAGED) {
      if (p.mask_kind != 0) {
        hipLaunchKernelGGL((wide_attn_kernel<T, D, BITS, G, PAGED, true, true>), dim3(p.nunits * p.nsplit),
                           dim3(kWW * 64), 0, stream, p);
      } else {
        hipLaunchKernelGGL((wide_attn_kernel<T, D, BITS, G, PAGED, false, true>), dim3(p.nunits * p.nsplit),
                           dim3(kWW * 64), 0, stream, p);
      }
    } else {
      return hipErrorInvalidValue;
    }
  } else if (p.mask_kind != 0) {
    if constexpr (D == 256 && BITS == 16 && !PAGED) {
      hipLaunchKernelGGL((wide_attn_kernel<T, D, BITS, G, PAGED, true>), dim3(p.nunits * p.nsplit), dim3(kWW * 64), 0,
                         stream, p);
    } else {
      return hipErrorInvalidValue;  // general masks: the unquantized head_dim-256 cache only
    }
  } else {
    hipLaunchKernelGGL((wide_attn_kernel<T, D, BITS, G, PAGED>), dim3(p.nunits * p.nsplit), dim3(kWW * 64), 0, stream,
                       p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.nsplit == 1) return e;
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
  m.R = kWRows;
  m.rowblocks = p.rowblocks;
  m.nsplit = p.nsplit;
  m.xcd_remap = 0;
  return launch_combine<T, D>(m, p.nunits / (p.Hkv * p.rowblocks), stream, p.dv);
}

static WideParams wide_params(const kvq_rows* q, const int32_t* seq_lens, const kvq_rows* out, int B, int Hq, int Hkv,
                              int L, int S, float scale, int causal, int window, void* workspace) {
  const WidePlan pl = wide_plan(B, Hq, Hkv, L, S, window);
  WideParams p{};
  p.q = (const uint16_t*)q->data;
  p.q_sb = q->stride_b;
  p.q_sh = q->stride_h;
  p.q_sl = q->stride_l;
  p.seq_lens = seq_lens;
  p.out = (uint16_t*)out->data;
  p.o_sb = out->stride_b;
  p.o_sh = out->stride_h;
  p.o_sl = out->stride_l;
  const size_t rows = (size_t)pl.nunits * pl.nsplit * kWRows;
  p.part_ml = (float*)((char*)workspace + kCounterBytes);
  p.part_o = (float*)((char*)workspace + kCounterBytes + (rows * sizeof(float2) + 255) / 256 * 256);
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.L = L;
  p.S = S;
  p.rep = Hq / Hkv;
  p.nrows = p.rep * L;
  p.rowblocks = pl.rowblocks;
  p.nsplit = pl.nsplit;
  p.nunits = pl.nunits;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.causal = causal;
  p.window = window;
  p.dv = 256;  // the quantized launches run head_dim 256; launch_wide_dense sets its own
  return p;
}

static void wide_quant_params(WideParams& p, const kvq_qtensor* k, const kvq_qtensor* v) {
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
  p.k_rexp = k->range_exp;
  p.v_rexp = v->range_exp;
}

template <bool PAGED>
static hipError_t launch_wide_quant(const WideParams& p, int bits, int G, int dtype, hipStream_t stream) {
  auto go = [&](auto t) -> hipError_t {
    using T = decltype(t);
    if (bits == 8 && G == 64) return launch_wide_t<T, 256, 8, 64, PAGED>(p, stream);
    if (bits == 8 && G == 128) return launch_wide_t<T, 256, 8, 128, PAGED>(p, stream);
    if (bits == 4 && G == 64) return launch_wide_t<T, 256, 4, 64, PAGED>(p, stream);
    if (bits == 4 && G == 128) return launch_wide_t<T, 256, 4, 128, PAGED>(p, stream);
    return hipErrorInvalidValue;
  };
  return dtype == KVQ_DTYPE_BF16 ? go(BF16{}) : go(F16{});
}

hipError_t launch_wide(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                       const kvq_rows* out, int B, int Hq, int Hkv, int L, int S, int bits, int G, int dtype,
                       float scale, int causal, int window, void* workspace, hipStream_t stream) {
  WideParams p = wide_params(q, seq_lens, out, B, Hq, Hkv, L, S, scale, causal, window, workspace);
  wide_quant_params(p, k, v);
  return launch_wide_quant<false>(p, bits, G, dtype, stream);
}

// Paged pools: the k / v descriptors' batch strides are page strides (include/kvq.h "Paged layout").
hipError_t launch_wide_paged(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                             const int32_t* table, int64_t table_stride, const int32_t* seq_lens, const kvq_rows* out,
                             int B, int Hq, int Hkv, int L, int S, int bits, int G, int dtype, float scale, int causal,
                             int window, void* workspace, hipStream_t stream) {
  WideParams p = wide_params(q, seq_lens, out, B, Hq, Hkv, L, S, scale, causal, window, workspace);
  wide_quant_params(p, k, v);
  p.table = table;
  p.table_stride = table_stride;
  p.num_pages = num_pages;
  return launch_wide_quant<true>(p, bits, G, dtype, stream);
}

hipError_t launch_wide_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                             const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype, float scale,
                             int causal, int window, void* workspace, hipStream_t stream, const kvq_mask* mask) {
  WideParams p = wide_params(q, seq_lens, out, B, Hq, Hkv, L, S, scale, causal, window, workspace);
  if (mask) {
    p.mask = mask->data;
    p.mask_kind = mask->kind;
    p.m_sb = mask->stride_b;
    p.m_skv = mask->stride_kvh;
    p.m_srep = mask->stride_rep;
    p.m_sl = mask->stride_l;
  }
  p.kc = (const uint8_t*)k->data;
  p.vc = (const uint8_t*)v->data;
  p.kc_sb = k->stride_b * 2;
  p.kc_sh = k->stride_h * 2;
  p.kc_ss = k->stride_l * 2;
  p.vc_sb = v->stride_b * 2;
  p.vc_sh = v->stride_h * 2;
  p.vc_ss = v->stride_l * 2;
  p.dv = D;
  if (D > 128 && D < 256) D = 256;  // rows narrower than the kernel: read 256 wide at their own stride
  if (D == 64)
    return dtype == KVQ_DTYPE_BF16 ? launch_wide_t<BF16, 64, 16, 64>(p, stream) : launch_wide_t<F16, 64, 16, 64>(p, stream);
  if (D == 256)
    return dtype == KVQ_DTYPE_BF16 ? launch_wide_t<BF16, 256, 16, 64>(p, stream)
                                   : launch_wide_t<F16, 256, 16, 64>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace kvq
