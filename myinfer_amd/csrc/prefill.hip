// Causal chunked-prefill attention over an MLX-layout affine-quantized KV cache, on MFMA.
//
// Computes, per (sequence b, query head h, query row l), the quantity m5engine/attention.py:29-103
// evaluates for L > 1 (blocked online softmax over key blocks, :64-100, causal when the mask is a
// string, :55-58/:70-73):
//   out = softmax(scale * q K^T + mask) V,  K = sK * codesK + bK,  V = sV * codesV + bV
// with query l at position S_b - L + l, keys <= position when causal, keys > position - window
// when a sliding window is set.
//
// Design (head_dim D = 128 or 64, 64-key tiles, a workgroup = 8 waves = 256 query rows, one per CU):
//  * A workgroup serves 256 consecutive rows of one (sequence, KV head) in position-major order
//    (row = position * rep + local head), so all rep query heads of a position share each K/V
//    tile and a causal boundary cuts only a few positions.
//  * The raw tiles (codes, scales, biases) stream into a 3-slot LDS ring by buffer->LDS DMA, two
//    steps ahead of their use, with no registers held in flight; rows past the sequence end read
//    as zero through the buffer range check (they are masked). Each 64-key tile is then
//    dequantized once per workgroup, LDS to LDS, into fp16 operands: K row-major, V transposed
//    (V^T[d][slot]) with its key slots permuted to match the score layout below. The fp16
//    operands are triple-buffered: tile t + 2 is dequantized while tile t is computed (the
//    quantized tile loop below says how the steps overlap).
//  * Per wave (32 rows = the columns of a 32x32 MFMA): S^T = K Q^T (v_mfma_f32_32x32x16_f16;
//    A = K rows from LDS, B = Q^T held in registers). In the MFMA result layout every lane holds
//    16 keys of one query column, so the row max / sum are lane-local plus one permlane swap, and
//    the probabilities converted to fp16 are already the B operand of O^T = V^T P^T: no shuffle.
//  * Q enters the MFMA exactly (times a per-row power of two that keeps it inside the fp16
//    range); the softmax scale in log2 units and that power are applied to the fp32 scores.
//  * A bf16 cache group beyond the fp16 range (its bias overflows on conversion) cannot be held by
//    the fp16 operands: the row blocks that read one return NaN rather than wrong finite values.
//  * Online softmax with threshold rescaling (a row's running maximum moves only when a tile's
//    maximum exceeds it by more than 2^6), fp32 accumulators.
//  * Long key ranges are split over several workgroups; the last split of a row block to finish
//    merges the (m, l, o) partials of the others (log-sum-exp) and writes the output.
//  * An unquantized fp16/bf16 cache (BITS == 16) takes a simpler loop: K operands straight from
//    the raw ring, only V^T staged, the MFMAs in the cache's type.

#include <math.h>

#include <type_traits>

#include "common.h"
#include "dma.h"
#include "launch.h"
#include "merge.h"

namespace kvq {

constexpr int kPT = 64;       // keys per tile
constexpr int kPRows = 256;   // query rows per workgroup (8 waves x 32 MFMA columns)
constexpr int kPW = 8;        // waves per workgroup
// fp16 per K row in LDS: D + 8 (rows shift by 4 banks)
template <int D>
constexpr int kKS = D + 8;
constexpr int kVS = 72;       // fp16 per V^T row in LDS: 64 + 8
constexpr float kPSlack = 6.0f;
constexpr int kPTargetWgs = 256;  // one workgroup per CU
constexpr int kRawSlots = 3;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2

// The raw tile ring. A slot holds one 64-key tile as loaded: [K codes][V codes][sK, bK, sV, bV],
// code rows with their 16-byte chunks XOR-swizzled by row (chunk c of row r at position
// c ^ swz(r)), each scale/bias array as 64 PC 4-byte cells: with NG = D / G >= 2 scale groups
// per row, cell PC key + c holds groups 2c and 2c + 1 of the key (PC = NG / 2); with one group,
// cell key holds it in its low half (PC = 1).
// BITS == 16 is the unquantized cache: raw T rows, no scales or biases.
template <int BITS, int G = 64, int D = 128>
struct RawCfg {
  static constexpr bool DENSE = BITS == 16;
  static_assert(G == 32 || G == 64 || G == 128, "group sizes 32, 64, 128");
  static_assert(D == 128 || (D == 64 && !DENSE), "head_dim 128, or 64 for quantized caches");
  static_assert(G <= D, "a group lies in one row");
  static constexpr int NG = D / G;                  // scale groups per key row
  static constexpr int ROWB = D * BITS / 8;         // code bytes per key row
  static constexpr int CPR = ROWB / 16;             // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;              // rows per 1 KiB DMA instruction
  static constexpr int CI = kPT / RPI;              // DMA instructions per K (or V) code tile
  static constexpr int KB = kPT * ROWB;             // bytes of a K (or V) code tile
  static constexpr int PC = NG >= 2 ? NG / 2 : 1;  // 4-byte cells per key in a scale/bias array
  static constexpr int SBB = DENSE ? 0 : 256 * PC;  // bytes of one scale/bias array
  static constexpr int SLOT = 2 * KB + 4 * SBB;
  // code DMA instructions per wave: with fewer than one per wave (4-bit, D = 64) waves 0 .. 2 CI - 1
  // issue one each and the others none
  static constexpr int CPW = 2 * CI >= kPW ? 2 * CI / kPW : 1;
  static constexpr int CODE_WAVES = 2 * CI >= kPW ? kPW : 2 * CI;
  // The chunk swizzle of row r. Quantized tiles fold in r / 16: the V^T staging reads one dim
  // quad of 8 keys per lane, and keys 16 apart (the same key % CPR) would otherwise share LDS
  // banks (a 4-way conflict at 8 bits); this spreads them over the banks. Unquantized rows keep
  // r % CPR (their staging and operand reads index it directly).
  static __device__ __forceinline__ constexpr int swz(int r) { return (DENSE ? r : r ^ (r >> 4)) % CPR; }
  // the waves that dequantize: V^T in waves [0, NSW), K in [NSW, 2 NSW) (256 threads each for
  // D = 128, 128 for D = 64); the other waves only compute
  static constexpr int NSW = D / 32;
  // 64-cell scale/bias DMA instructions per wave: 4 PC of them fill the four arrays, one per wave
  // (with PC = 1 two waves fill the same cells)
  static constexpr int SBW = DENSE ? 0 : 1;
  static constexpr int IPT = CPW + SBW;             // DMA instructions per tile of a wave that loads codes
  static constexpr int IPT_NOCODE = SBW;            // ... and of one that does not
  static_assert(CPW * CODE_WAVES == 2 * CI, "code DMAs divide evenly over the waves that issue them");
  static_assert(CODE_WAVES >= 2 * NSW, "the dequantizing waves load codes");
  static_assert(DENSE || 4 * PC <= kPW, "scale/bias DMAs fit one per wave");
  // byte offset of group g of key `key` inside a scale/bias array
  static __host__ __device__ constexpr int sb_off(int key, int g) { return 4 * (PC * key + g / 2) + 2 * (g & 1); }
};

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
  int xcd_remap;       // 1: the grid is a multiple of the XCD count (see the numbering in the kernel)
  int Hq, Hkv, L, S, rep, nrows, rowblocks, nsplit, nunits;
  float scale_log2;
  int causal, window;
  // paged cache (PAGED kernels): rows of sequence b live in 64-row pages, page table[b][r / 64];
  // the codes/scales/biases batch strides above are then page strides
  const int32_t* table;
  int64_t table_stride;
  int num_pages;
  // the caches' range exponents (kvq_qtensor.range_exp), or null: the fp16 operands are staged
  // times 2^-E, and 2^E returns in the score scale (K) and the output (V)
  const int32_t* k_rexp;
  const int32_t* v_rexp;
};

// V^T slot of key `kk` (0..63) inside a tile: the 16 keys of PV k-step j = kk / 16 are stored so
// that slots 16j + 8h + i hold the keys the score layout gives lane half h at i.
__host__ __device__ constexpr int v_slot_key(int slot) {
  return 16 * (slot >> 4) + ((slot & 7) < 4 ? 4 * ((slot >> 3) & 1) + (slot & 7) : 8 + 4 * ((slot >> 3) & 1) + (slot & 7) - 4);
}
// The 8 keys of V^T slot chunk c8 are v_base_key(c8) + v_key_offset(i): a per-lane base plus
// compile-time offsets, so the staging addresses them with immediate offsets.
__host__ __device__ constexpr int v_base_key(int c8) { return 16 * (c8 >> 1) + 4 * (c8 & 1); }
__host__ __device__ constexpr int v_key_offset(int i) { return i < 4 ? i : i + 4; }
constexpr bool v_keys_split() {
  for (int c8 = 0; c8 < 8; ++c8)
    for (int i = 0; i < 8; ++i)
      if (v_slot_key(8 * c8 + i) != v_base_key(c8) + v_key_offset(i) || (v_base_key(c8) & 3) != 0 ||
          (v_key_offset(i) & 7) != (i & 3) || ((v_base_key(c8) + v_key_offset(i)) >> 4) != (v_base_key(c8) >> 4))
        return false;
  return true;
}
static_assert(v_keys_split(), "slot keys are a per-lane base (low two bits clear) plus i-dependent offsets below 16");


// This wave's share of a raw tile: CPW 1 KiB code loads (K instructions first, then V; none for
// waves from CODE_WAVES on) and one 64-cell scale/bias load (array wave / 2, cells 64 part .. with
// part = (wave % 2) % PC; 4-byte cells, or 2-byte values into the low halves when PC = 1 holds a
// single group).
template <int BITS, int G = 64, int D = 128>
struct RawShare {
  using C = RawCfg<BITS, G, D>;
  static constexpr int SBN = C::SBW > 0 ? C::SBW : 1;
  __amdgpu_buffer_rsrc_t code_r[C::CPW], sb_r[SBN];
  uint32_t code_vo[C::CPW], code_lds[C::CPW], sb_vo[SBN], sb_lds[SBN];
  int64_t code_ss[C::CPW], sb_ss[SBN];  // bytes per key row
  bool code_on;                         // this wave issues code loads (wave-uniform)

  __device__ __forceinline__ void init(const PreParams& p, __amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                       const __amdgpu_buffer_rsrc_t (&sr)[4], int wave, int lane) {
    code_on = wave < C::CODE_WAVES;
#pragma unroll
    for (int j = 0; j < C::CPW; ++j) {
      const int q = code_on ? wave * C::CPW + j : 0;
      const bool is_k = q < C::CI;
      const int i = is_k ? q : q - C::CI;
      const int r = i * C::RPI + lane / C::CPR;
      const int c = (lane % C::CPR) ^ C::swz(r);
      code_r[j] = is_k ? kr : vr;
      code_ss[j] = is_k ? p.kc_ss : p.vc_ss;
      code_vo[j] = (uint32_t)(r * code_ss[j] + 16 * c);
      code_lds[j] = (is_k ? 0 : C::KB) + 1024 * i;
    }
#pragma unroll
    for (int j = 0; j < SBN; ++j) {
      const int li = wave * C::SBW + j, a = li / 2, part = (li % 2) % C::PC;
      const int cell = 64 * part + lane;  // cell cell % PC of key cell / PC
      sb_r[j] = a == 0 ? sr[0] : a == 1 ? sr[1] : a == 2 ? sr[2] : sr[3];
      sb_ss[j] = C::DENSE ? 0 : 2 * (a < 2 ? p.ksb_ss : p.vsb_ss);
      sb_vo[j] = (uint32_t)((cell / C::PC) * sb_ss[j] + 4 * (cell % C::PC));
      sb_lds[j] = 2 * C::KB + C::SBB * a + 256 * part;
    }
  }
  // raw tile of keys [k0, k0 + 64) into the slot at LDS address `slot`
  __device__ __forceinline__ void issue(uint32_t slot, int k0) const {
    if (code_on) {
#pragma unroll
      for (int j = 0; j < C::CPW; ++j) dma_b128(code_r[j], slot + code_lds[j], code_vo[j], (uint32_t)(k0 * code_ss[j]));
    }
#pragma unroll
    for (int j = 0; j < C::SBW; ++j) dma_sb(sb_r[j], slot + sb_lds[j], sb_vo[j], (uint32_t)(k0 * sb_ss[j]));
  }
  static __device__ __forceinline__ void dma_sb(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t vo, uint32_t so) {
    if constexpr (C::NG >= 2) {
      dma_b32(r, lds, vo, so);
    } else {
      dma_b16(r, lds, vo, so);
    }
  }

  // Paged cache: the wave's arrays at page 0 of this KV head, and their page strides (bytes).
  const uint8_t* code_base[C::CPW];
  const uint8_t* sb_base[SBN];
  int64_t code_ps[C::CPW], sb_ps[SBN];
  __device__ __forceinline__ void init_paged(const PreParams& p, int kvh, int wave) {
#pragma unroll
    for (int j = 0; j < C::CPW; ++j) {
      const bool is_k = (code_on ? wave * C::CPW + j : 0) < C::CI;
      code_base[j] = is_k ? p.kc + (int64_t)kvh * p.kc_sh : p.vc + (int64_t)kvh * p.vc_sh;
      code_ps[j] = is_k ? p.kc_sb : p.vc_sb;
    }
#pragma unroll
    for (int j = 0; j < SBN; ++j) {
      const int a = (wave * C::SBW + j) / 2;
      const uint16_t* arr = a == 0 ? p.ks : a == 1 ? p.kb : a == 2 ? p.vs : p.vb;
      sb_base[j] = (const uint8_t*)(arr + (int64_t)kvh * (a < 2 ? p.ksb_sh : p.vsb_sh));
      sb_ps[j] = 2 * (a < 2 ? p.ksb_sb : p.vsb_sb);
    }
  }
  // raw tile of page `pg` (its first nv rows valid) into the slot at LDS address `slot`
  __device__ __forceinline__ void issue_paged(uint32_t slot, int pg, int nv) const {
    if (code_on) {
#pragma unroll
      for (int j = 0; j < C::CPW; ++j)
        dma_b128(make_rsrc(code_base[j] + (int64_t)pg * code_ps[j], (uint32_t)(nv * code_ss[j])), slot + code_lds[j],
                 code_vo[j], 0u);
    }
#pragma unroll
    for (int j = 0; j < C::SBW; ++j)
      dma_sb(make_rsrc(sb_base[j] + (int64_t)pg * sb_ps[j], (uint32_t)(nv * sb_ss[j])), slot + sb_lds[j], sb_vo[j],
             0u);
  }
};

__device__ __forceinline__ _Float16 to_half(uint16_t r, F16) { return __builtin_bit_cast(_Float16, r); }
__device__ __forceinline__ _Float16 to_half(uint16_t r, BF16) { return (_Float16)__uint_as_float((uint32_t)r << 16); }
// A scale or bias as its fp16 operand value times m = 2^-E (the cache's range exponent, include/kvq.h):
// exact in fp32, rounded once. An fp16 cache never needs the factor (its values fit the operands).
__device__ __forceinline__ _Float16 to_half_scaled(uint16_t r, float, F16) { return __builtin_bit_cast(_Float16, r); }
__device__ __forceinline__ _Float16 to_half_scaled(uint16_t r, float m, BF16) {
  return (_Float16)(__uint_as_float((uint32_t)r << 16) * m);
}

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

// Dequantize the raw tile at `raw` into the fp16 operands. Threads 0 .. 64 NSW - 1 (NSW = D / 32
// waves) build V^T: thread t takes the 8 keys of slot chunk t % 8 at dims [4 (t / 8), +4) and writes
// 4 V^T rows of 8 slots. The next 64 NSW threads build K: thread 64 NSW + u takes dims [32 q, +32)
// of key u % 64, q = u / 64. Threads beyond take no part.
//
// V^T, first part: the wave's lanes convert the scale and bias of the wave's group (dims
// [32 w, 32 w + 32) lie in one group) for the 64 keys (lane = key) into a per-wave table of fp16
// (scale, bias) pairs, which stage_v then reads for its 8 keys. Only this wave touches its table,
// and the LDS operations of one wave complete in program order, so a wave barrier (which keeps
// the compiler from moving the lanes' accesses across it) is all the ordering the reads need.
template <typename T, int BITS, int G, int D>
__device__ __forceinline__ void stage_v_table(const uint8_t* raw, uint32_t* sbt, int tid, bool& range_bad, float vmul) {
  using C = RawCfg<BITS, G, D>;
  const int key = tid & 63, g = (4 * (tid >> 3)) / G;
  const uint8_t* sbase = raw + 2 * C::KB + C::sb_off(key, g);
  const uint16_t sv = *(const uint16_t*)(sbase + 2 * C::SBB), bv = *(const uint16_t*)(sbase + 3 * C::SBB);
  const h2 sbp = {to_half_scaled(sv, vmul, T{}), to_half_scaled(bv, vmul, T{})};
  sbt[key] = __builtin_bit_cast(uint32_t, sbp);
  // a bf16 group beyond the fp16 range has a bias (its largest-magnitude element) that converts to
  // inf; the operands cannot hold it
  if constexpr (T::id == KVQ_DTYPE_BF16) range_bad |= __builtin_isinf((float)sbp[1]);
}

// V^T, second part (after stage_v_table of the same tile), in two halves: half H builds dims
// 4 d4 + 2H and + 2H + 1 (V^T rows 2H, 2H + 1 of the thread's four).
template <int BITS, int G, int D, int H>
__device__ __forceinline__ void stage_v(const uint8_t* raw, _Float16* vlds, const uint32_t* sbt, int tid) {
  using C = RawCfg<BITS, G, D>;
  const int c8 = tid & 7, d4 = tid >> 3;
  // key i of the chunk is kb + v_key_offset(i), and its swizzle swz(key) is
  // (((kb % CPR) | (i & 3)) ^ (kb >> 4)) % CPR: kb has its low two bits clear and kb % 16 is 0 or
  // 4, the offsets are i & 3 modulo 8 and below 12 (so key >> 4 == kb >> 4), CPR is a power of
  // two. Four code addresses per lane; everything else is an immediate offset
  const int kb = v_base_key(c8);
  const uint8_t* vr = raw + C::KB + kb * C::ROWB;
  uint32_t x[8];  // key i: the dim pair of this half
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ko = v_key_offset(i);
    const int sw = (((kb % C::CPR) | (i & 3)) ^ (kb >> 4)) % C::CPR;
    uint32_t bytes;  // codes of dims 4 d4 .. 4 d4 + 3 as 4 bytes
    if constexpr (BITS == 8) {
      bytes = *(const uint32_t*)(vr + ko * C::ROWB + 16 * ((d4 >> 2) ^ sw) + 4 * (d4 & 3));
    } else {
      const uint32_t h = *(const uint16_t*)(vr + ko * C::ROWB + 16 * ((d4 >> 3) ^ sw) + 2 * (d4 & 7));
      bytes = perm((h >> 4) & 0x0F0Fu, h & 0x0F0Fu, 0x05010400u);
    }
    const h2 sbp = __builtin_bit_cast(h2, sbt[kb + ko]);
    const _Float16 sh = sbp[0], bh = sbp[1];
    x[i] = dequant_pair(bytes, H == 0 ? 0x04010400u : 0x04030402u, h2{sh, sh}, h2{bh, bh});
  }
#pragma unroll
  for (int e = 2 * H; e < 2 * H + 2; ++e) {
    const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
    u4 v;
#pragma unroll
    for (int ip = 0; ip < 4; ++ip) v[ip] = perm(x[2 * ip + 1], x[2 * ip], sel);
    *(u4*)&vlds[(4 * d4 + e) * kVS + 8 * c8] = v;
  }
}

// K, in two halves: half H builds dims [32 q + 16 H, +16) of key u % 64.
template <typename T, int BITS, int G, int D, int H>
__device__ __forceinline__ void stage_k(const uint8_t* raw, _Float16* klds, int tid, bool& range_bad, float kmul) {
  using C = RawCfg<BITS, G, D>;
  const int u = tid - 64 * C::NSW;
  const int key = u & 63, q = u >> 6;
  const uint8_t* kr = raw + key * C::ROWB;
  uint32_t w[4];  // the half's 16 codes
  if constexpr (BITS == 8) {
    const u4 a = *(const u4*)(kr + 16 * ((2 * q + H) ^ C::swz(key)));
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = a[i];
  } else {
    const u2 a = *(const u2*)(kr + 16 * (q ^ C::swz(key)) + 8 * H);
    w[0] = a[0];
    w[1] = a[1];
  }
  const uint8_t* sbase = raw + 2 * C::KB + C::sb_off(key, (32 * q + 16 * H) / G);
  const _Float16 sh = to_half_scaled(*(const uint16_t*)sbase, kmul, T{});
  const _Float16 bh = to_half_scaled(*(const uint16_t*)(sbase + C::SBB), kmul, T{});
  if constexpr (T::id == KVQ_DTYPE_BF16) range_bad |= __builtin_isinf((float)bh);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    uint32_t x[4];
    dequant8<BITS>(&w[(BITS / 4) * c], h2{sh, sh}, h2{bh, bh}, x);
    *(u4*)&klds[key * kKS<D> + 32 * q + 16 * H + 8 * c] = u4{x[0], x[1], x[2], x[3]};
  }
}

// The whole tile, all threads.
template <typename T, int BITS, int G, int D>
__device__ __forceinline__ void stage_from_raw(const uint8_t* raw, _Float16* klds, _Float16* vlds, uint32_t* sbt,
                                               int tid, bool& range_bad, float kmul, float vmul) {
  constexpr int NST = 64 * RawCfg<BITS, G, D>::NSW;  // threads per operand
  if (tid < NST) {
    stage_v_table<T, BITS, G, D>(raw, sbt, tid, range_bad, vmul);
    __builtin_amdgcn_wave_barrier();
    stage_v<BITS, G, D, 0>(raw, vlds, sbt, tid);
    stage_v<BITS, G, D, 1>(raw, vlds, sbt, tid);
  } else if (tid < 2 * NST) {
    stage_k<T, BITS, G, D, 0>(raw, klds, tid, range_bad, kmul);
    stage_k<T, BITS, G, D, 1>(raw, klds, tid, range_bad, kmul);
  }
}

// Unquantized cache: build half of V^T from the raw V rows of a tile (phase 0: slots 0-31, phase
// 1: slots 32-63). Thread t (0..255) takes slot chunk c8 = 4 phase + t % 4 and dims 2 (t / 4),
// 2 (t / 4) + 1: 8 keys x 2 dims read as 32-bit words, written as two 8-slot V^T rows.
__device__ __forceinline__ void stage_v_raw(const uint8_t* raw, _Float16* vlds, int t, int phase) {
  constexpr int ROWB = RawCfg<16>::ROWB, CPR = RawCfg<16>::CPR;
  const int c8 = 4 * phase + (t & 3), d2 = t >> 2;
  const uint8_t* vr = raw + RawCfg<16>::KB;
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = v_slot_key(8 * c8 + i);
    w[i] = *(const uint32_t*)(vr + key * ROWB + 16 * ((d2 >> 2) ^ (key % CPR)) + 4 * (d2 & 3));
  }
  u4 lo, hi;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    lo[a] = perm(w[2 * a + 1], w[2 * a], 0x05040100u);
    hi[a] = perm(w[2 * a + 1], w[2 * a], 0x07060302u);
  }
  *(u4*)&vlds[(2 * d2) * kVS + 8 * c8] = lo;
  *(u4*)&vlds[(2 * d2 + 1) * kVS + 8 * c8] = hi;
}

template <typename T, int BITS, bool PAGED = false, int G = 64, int D = 128>
__global__ __launch_bounds__(kPW * 64, 1) void prefill_attn_kernel(PreParams p) {
  using RC = RawCfg<BITS, G, D>;
  constexpr bool DENSE = RC::DENSE;  // unquantized cache: K operands are read from the raw ring
  constexpr int KS = kKS<D>;
  constexpr int KSTEPS = D / 16;   // k-steps of S^T = K Q^T over the head dimension
  constexpr int NDB = D / 32;      // 32-dim blocks of O^T
  constexpr int QW = D / 16;       // 16-byte words of a lane's packed output row
  __shared__ __align__(16) _Float16 k_lds[DENSE ? 1 : 3][DENSE ? 8 : kPT * KS];
  __shared__ __align__(16) _Float16 v_lds[DENSE ? 2 : 3][D * kVS];
  __shared__ __align__(16) uint8_t raw[kRawSlots][RC::SLOT];
  __shared__ uint32_t sb_tab[DENSE ? 1 : kPW / 2][64];  // per V^T-building wave: (scale, bias) pairs
  // after the tile loop the table's storage holds per-wave flags (words 0-7) and the split arrival
  // count (word 8): the LDS budget has no room for more
  unsigned* const s_flags = &sb_tab[0][0];
  unsigned* const s_arrived = &sb_tab[0][8];
  bool range_bad = false;  // some tile this lane staged held a group beyond the fp16 range
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qc = lane & 31, hh = lane >> 5;

  // Workgroup numbering: the row blocks of one (sequence, KV head, split) share every K/V tile, so
  // they are consecutive, and consecutive workgroups are placed on one XCD (the hardware hands
  // workgroups to the 8 XCDs in turn): each tile is fetched into one L2 rather than eight.
  int wg = blockIdx.x;
  if (p.xcd_remap) {
    const int per_xcd = (int)(gridDim.x / kXcds);
    wg = (wg % kXcds) * per_xcd + wg / kXcds;
  }
  const int rb = wg % p.rowblocks;
  const int split = (wg / p.rowblocks) % p.nsplit;
  const int bk = wg / (p.rowblocks * p.nsplit);  // b * Hkv + kvh
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;
  const int unit = bk * p.rowblocks + rb;
  const int S_b = p.seq_lens ? min(max(load_uniform_i32(p.seq_lens, b), 0), p.S) : p.S;

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

  // ---- the raw query slice (loaded before the tile stream; row and head are clamped, so every
  // lane's load is in bounds)
  u4 qraw[KSTEPS];
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)head * p.q_sh + (int64_t)lq * p.q_sl + 8 * hh;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) qraw[j] = *(const u4*)(qrow + 16 * j);
  }

  // ---- raw tile stream: buffer resources over the S_b valid rows of this (sequence, KV head)
  // (the host checks S * row stride fits 32 bits); tiles past the last re-read the last one
  RawShare<BITS, G, D> share;
  {
    const __amdgpu_buffer_rsrc_t kr =
        make_rsrc(p.kc + (int64_t)b * p.kc_sb + (int64_t)kvh * p.kc_sh, (uint32_t)((int64_t)S_b * p.kc_ss));
    const __amdgpu_buffer_rsrc_t vr =
        make_rsrc(p.vc + (int64_t)b * p.vc_sb + (int64_t)kvh * p.vc_sh, (uint32_t)((int64_t)S_b * p.vc_ss));
    const int64_t ko = (int64_t)b * p.ksb_sb + (int64_t)kvh * p.ksb_sh;
    const int64_t vo = (int64_t)b * p.vsb_sb + (int64_t)kvh * p.vsb_sh;
    const uint32_t kn = (uint32_t)((int64_t)S_b * p.ksb_ss * 2), vn = (uint32_t)((int64_t)S_b * p.vsb_ss * 2);
    __amdgpu_buffer_rsrc_t sr[4] = {kr, kr, kr, kr};
    if constexpr (!DENSE) {
      sr[0] = make_rsrc(p.ks + ko, kn);
      sr[1] = make_rsrc(p.kb + ko, kn);
      sr[2] = make_rsrc(p.vs + vo, vn);
      sr[3] = make_rsrc(p.vb + vo, vn);
    }
    share.init(p, kr, vr, sr, wave, lane);
    if constexpr (PAGED) share.init_paged(p, kvh, wave);
  }
  const uint32_t raw_lds = lds_addr(&raw[0][0]);
  const int last = max(ntile - 1, 0);
  // paged cache: a tile (64 rows, 64-aligned) is one page; its page number is read one tile ahead
  // (a scalar load), clamped to the pool, and the tile's buffer resources span only that page's
  // valid rows, so rows past S_b still read as zero
  auto page_of = [&](int k0) -> int {
    const int pi = min(k0, max(S_b - 1, 0)) >> 6;
    return __builtin_amdgcn_readfirstlane(min(max(p.table[(int64_t)b * p.table_stride + pi], 0), p.num_pages - 1));
  };
  int pg_next = PAGED ? page_of(k_begin) : 0;
  auto issue_raw = [&](int i) {
    const int k0 = k_begin + kPT * min(i, last);
    const uint32_t slot = raw_lds + (i % kRawSlots) * RC::SLOT;
    if constexpr (PAGED) {
      const int pg = pg_next;
      pg_next = page_of(k_begin + kPT * min(i + 1, last));
      share.issue_paged(slot, pg, __builtin_amdgcn_readfirstlane(max(min(kPT, S_b - k0), 0)));
    } else {
      share.issue(slot, k0);
    }
  };
  // the first tiles of the ring (the tile loops below say how far ahead each runs)
  if (ntile > 0) {
#pragma unroll
    for (int j = 0; j < (DENSE ? 2 : kRawSlots); ++j) issue_raw(j);
  }

  // ---- range exponents of the K and V caches (0 for an unquantized cache, an fp16 cache -- whose
  // values always fit the fp16 operands -- or a null pointer) and the factors 2^-E the staging
  // applies to the scales and biases; 2^E_K returns in the score scale, 2^E_V in the output. Read
  // here, after the first tile loads are issued, so that waiting for the word delays no load. (The
  // factors are held in VGPRs: the tile loop has spare vector registers and no spare scalar ones.)
  float kmul = 1.0f, vmul = 1.0f, kback = 1.0f, vback = 1.0f;
  if constexpr (!DENSE && T::id == KVQ_DTYPE_BF16) {
    const int ek = p.k_rexp ? min(max(*p.k_rexp, 0), 127) : 0;
    const int ev = p.v_rexp ? min(max(*p.v_rexp, 0), 127) : 0;
    kmul = ldexpf(1.0f, -ek);
    vmul = ldexpf(1.0f, -ev);
    kback = ldexpf(1.0f, ek);
    vback = ldexpf(1.0f, ev);
    asm volatile("" : "+v"(kmul), "+v"(vmul), "+v"(kback), "+v"(vback));
  }

  // ---- Q^T operand: k-step j holds dims 16j + 8hh .. +7. Quantized cache: the query times 2^qe in
  // fp16 (exact: a power of two, with qe chosen so the row's largest element lands in [2^13, 2^14);
  // a bf16 query has 8 significant bits, so only elements below 2^-14 of the operand's scale lose
  // bits), and the scores are multiplied by inv2 = scale * log2(e) * 2^-qe in fp32. Folding the
  // softmax scale into the fp16 operand instead would round every query element. Unquantized
  // cache: the raw query (exact), the scores multiplied by scale*log2(e) in fp32.
  u4 qop[KSTEPS];
  float inv2;
  if constexpr (DENSE) {
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) qop[j] = row_ok ? qraw[j] : u4{0, 0, 0, 0};
    inv2 = p.scale_log2;
  } else {
    float qv[KSTEPS][8];
    float qmax = 0.0f;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      const u4 raw_q = row_ok ? qraw[j] : u4{0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qv[j][2 * i] = to_float((uint16_t)(raw_q[i] & 0xffffu), T{});
        qv[j][2 * i + 1] = to_float((uint16_t)(raw_q[i] >> 16), T{});
        qmax = fmaxf(qmax, fmaxf(fabsf(qv[j][2 * i]), fabsf(qv[j][2 * i + 1])));
      }
    }
    qmax = max_xor32(qmax);
    int e = 0;
    if (qmax > 0.0f) frexpf(qmax, &e);
    const int qe = 14 - e;  // |q| * 2^qe < 2^14
    const float qmul = ldexpf(1.0f, qe);
    inv2 = ldexpf(p.scale_log2, -qe) * kback;  // the K operands are staged times 2^-E_K
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) qop[j][i] = pack_f16x2(qv[j][2 * i] * qmul, qv[j][2 * i + 1] * qmul);
  }
  // MFMA operand type: bf16 for an unquantized bf16 cache, else fp16
  using OT = typename std::conditional<DENSE && T::id == KVQ_DTYPE_BF16, BF16, F16>::type;

  float m_run = -INFINITY, l_run = 0.0f;
  f16v oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = f16v{};

  if constexpr (DENSE) {
    // ---- the pieces of a tile step (head_dim 128)
    // this lane's query sees keys k0 + 32kb + 8(i/4) + 4hh + i%4. Only tiles on a causal diagonal or
    // window edge need a mask (a branch the whole workgroup takes or skips); there, each element's
    // offset c = 32kb + 8(i/4) + i%4 is a constant compared with the lane's bounds
    auto mask_tile = [&](f16v (&acc)[2], int k0) {
      const bool need_mask = !(k0 >= lo_all && k0 + kPT <= hi_all);
      if (__builtin_expect(need_mask, 0)) {
        const int lo = lo_r - k0 - 4 * hh, hi = hi_r - k0 - 4 * hh;
        if (lo <= 0) {  // no key of the tile is below the lane's window
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (32 * kb + 8 * (i >> 2) + (i & 3) >= hi) acc[kb][i] = -INFINITY;
        } else {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int c = 32 * kb + 8 * (i >> 2) + (i & 3);
              if (c < lo || c >= hi) acc[kb][i] = -INFINITY;
            }
        }
      }
    };
    // the tile's row maximum in log2 units; the running maximum moves (and the accumulators are
    // rescaled) only when it exceeds the running one by more than the slack
    auto update_max = [&](const f16v (&acc)[2]) {
      float tm = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) tm = fmaxf(tm, acc[kb][i]);
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
    };
    // p = 2^(acc * inv2 - m): rounded to the operand type it is the B operand of O^T = V^T P^T; the
    // row sum is kept in fp32 (of the rounded values, so the output stays a convex combination of V
    // rows), in two chains
    auto probs = [&](const f16v (&acc)[2], u4 (&pop)[4]) {
      const float nm = m_run == -INFINITY ? 0.0f : -m_run;
      float lsum[2] = {0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = exp2_fast(fmaf(acc[j >> 1][8 * (j & 1) + 2 * e], inv2, nm));
          const float p1 = exp2_fast(fmaf(acc[j >> 1][8 * (j & 1) + 2 * e + 1], inv2, nm));
          pop[j][e] = pack2(p0, p1, OT{});
          lsum[e & 1] = add_pair(pop[j][e], lsum[e & 1], OT{});
        }
      }
      l_run += lsum[0] + lsum[1];
    };
    // O^T += V^T P^T: the 16 V^T operands stream through a 4-deep register ring; the 4 dim blocks
    // alternate. vl = this lane's start in a V^T buffer.
    auto pv = [&](const _Float16* vl, const u4 (&pop)[4]) {
      auto vop = [&](int i) { return *(const u4*)(vl + (i & 3) * 32 * kVS + 16 * (i >> 2)); };
      u4 ring[4] = {vop(0), vop(1), vop(2), vop(3)};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        oacc[i & 3] = mfma_32x32x16(ring[i & 3], pop[i >> 2], oacc[i & 3], OT{});
        if (i + 4 < 16) ring[i & 3] = vop(i + 4);
      }
    };

    // ---- unquantized cache: K operands are read from the raw ring while tile t is computed, so
    // tile t + 2 is issued into the slot of tile t - 1 and lands within the step (issued once the
    // step's QK MFMAs are, which measured 4-5% faster than at the step's start); V^T is built from
    // the raw rows into a double buffer, half by waves 4-7 before their MFMAs and half by waves 0-3
    // after theirs (the two waves that share a SIMD are in opposite phases)
    if (ntile > 0) {
      wait_vm<0>();
      __syncthreads();
      stage_v_raw(raw[0], v_lds[0], tid & 255, tid >> 8);
      __syncthreads();
    }
    // this lane's K operand bytes within a raw slot: key row 32 (i & 1) + qc, 16-byte chunk
    // 2 (i >> 1) + hh at its swizzled position
    const int kswz = qc % RawCfg<16>::CPR;
    for (int t = 0; t < ntile; ++t) {
      const int cur = t & 1;
      const int k0 = k_begin + kPT * t;
      if (t + 1 < ntile && wave >= kPW / 2) stage_v_raw(raw[(t + 1) % kRawSlots], v_lds[cur ^ 1], tid - 256, 0);
      f16v sacc[2] = {f16v{}, f16v{}};
      {
        const uint8_t* kraw = raw[t % kRawSlots] + qc * RawCfg<16>::ROWB;
        auto kop = [&](int i) -> u4 {
          return *(const u4*)(kraw + (i & 1) * 32 * RawCfg<16>::ROWB + 16 * ((2 * (i >> 1) + hh) ^ kswz));
        };
        u4 ring[4] = {kop(0), kop(1), kop(2), kop(3)};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          sacc[i & 1] = mfma_32x32x16(ring[i & 3], qop[i >> 1], sacc[i & 1], OT{});
          if (i + 4 < 16) ring[i & 3] = kop(i + 4);
        }
      }
      if (t + 2 < ntile) issue_raw(t + 2);  // into the slot of tile t - 1 (read in the last step)
      mask_tile(sacc, k0);
      update_max(sacc);
      u4 pop[4];
      probs(sacc, pop);
      pv(&v_lds[cur][qc * kVS + 8 * hh], pop);
      if (t + 1 < ntile && wave < kPW / 2) stage_v_raw(raw[(t + 1) % kRawSlots], v_lds[cur ^ 1], tid, 1);
      wait_vm<0>();  // tile t + 2 has landed
      __syncthreads();
    }
  } else if (ntile > 0) {
    // ---- quantized cache, software-pipelined over 32-key blocks. Step t (tile t) runs two halves;
    // half h takes the scores of block h of the tile, already computed, and
    //  * takes their row maximum (and the rare rescale) first, then issues the MFMAs of the next
    //    block's scores (block 1 of tile t, then block 0 of tile t + 1) and runs the exponentials
    //    while they execute (the maximum first measured about 1% faster than after two MFMAs), then
    //  * accumulates O += V P for the block while the dequantizing waves build half of tile t + 2
    //    (the V^T waves its V^T, the K waves its K),
    // so every wave always has MFMA work beside its VALU work, and two 16-register score blocks are
    // live rather than two tiles.
    //  * fp16 operands: tile j in k_lds[j % 3] and v_lds[j % 3] (step t reads K of tiles t and
    //    t + 1 and V of tile t, and writes tile t + 2);
    //  * raw ring: tile j in slot j % 3; step t reads tile t + 2 and issues tile t + 4 into the slot
    //    of tile t + 1 (dequantized in step t - 1), so every tile is loaded two steps ahead;
    //  * one barrier per step orders all of it.
    constexpr int KBUF = kPT * KS, VBUF = D * kVS;
    const _Float16* kl_lane = &k_lds[0][qc * KS + 8 * hh];  // this lane's K operands, V^T operands
    const _Float16* vl_lane = &v_lds[0][qc * kVS + 8 * hh];
    // S^T = K Q^T for the 32-key block whose K rows start at kl (this lane's offset included):
    // KSTEPS MFMAs over the head dimension, the K operands streamed through a 4-deep register ring
    // (deeper rings of 6 and 8, and an 8-deep V^T ring, measured slower); MFMAs [J0, J1) of them
    auto qk_ring = [&](u4 (&ring)[4], const _Float16* kl) {
#pragma unroll
      for (int j = 0; j < 4; ++j) ring[j] = *(const u4*)(kl + 16 * j);
    };
    auto qk_run = [&](auto j0, auto j1, f16v& acc, u4 (&ring)[4], const _Float16* kl) {
#pragma unroll
      for (int j = decltype(j0)::value; j < decltype(j1)::value; ++j) {
        acc = mfma_32x32x16(ring[j & 3], qop[j], j == 0 ? f16v{} : acc, OT{});
        if (j + 4 < KSTEPS) ring[j & 3] = *(const u4*)(kl + 16 * (j + 4));
      }
    };
    using J0 = std::integral_constant<int, 0>;
    using JE = std::integral_constant<int, KSTEPS>;
    // the block's keys [k, k + 32): mask (only on a causal diagonal or window edge), row maximum
    auto mask_blk = [&](f16v& acc, int k) {
      if (__builtin_expect(!(k >= lo_all && k + 32 <= hi_all), 0)) {
        const int lo = lo_r - k - 4 * hh, hi = hi_r - k - 4 * hh;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int c = 8 * (i >> 2) + (i & 3);
          if (c < lo || c >= hi) acc[i] = -INFINITY;
        }
      }
    };
    auto max_blk = [&](const f16v& acc) {
      float tm = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) tm = fmaxf(tm, acc[i]);
      return max_xor32(tm) * inv2;
    };
    auto rescale = [&](float tm) {
      if (__builtin_amdgcn_ballot_w64(tm > m_run + kPSlack) != 0) {
        const float m_new = tm > m_run + kPSlack ? fmaxf(m_run, tm) : m_run;
        const float corr = m_new == m_run ? 1.0f : exp2_fast(m_run - m_new);
        l_run *= corr;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) oacc[db][i] *= corr;
        m_run = m_new;
      }
    };
    // p = 2^(acc * inv2 - m) for the block's 32 keys: the B operands of its two PV k-steps
    auto probs_blk = [&](const f16v& acc, u4 (&pop)[2]) {
      const float nm = m_run == -INFINITY ? 0.0f : -m_run;
      float lsum[2] = {0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = exp2_fast(fmaf(acc[8 * j + 2 * e], inv2, nm));
          const float p1 = exp2_fast(fmaf(acc[8 * j + 2 * e + 1], inv2, nm));
          pop[j][e] = pack2(p0, p1, OT{});
          lsum[e & 1] = add_pair(pop[j][e], lsum[e & 1], OT{});
        }
      l_run += lsum[0] + lsum[1];
    };
    // O^T += V^T P^T over block kb's two k-steps (V^T slots 32 kb .. 32 kb + 31): 2 NDB MFMAs, the
    // NDB dim blocks alternating, V^T operands through a 4-deep ring
    auto pv_blk = [&](const _Float16* vl, const u4 (&pop)[2], auto kb) {
      constexpr int KB = decltype(kb)::value;
      auto vop = [&](int i) { return *(const u4*)(vl + (i % NDB) * 32 * kVS + 16 * (2 * KB + i / NDB)); };
      u4 ring[4] = {vop(0), vop(1), vop(2), vop(3)};
#pragma unroll
      for (int i = 0; i < 2 * NDB; ++i) {
        oacc[i % NDB] = mfma_32x32x16(ring[i & 3], pop[i / NDB], oacc[i % NDB], OT{});
        if (i + 4 < 2 * NDB) ring[i & 3] = vop(i + 4);
      }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;

    // The wave's role: 0 builds V^T (waves [0, NSW)), 1 builds K (waves [NSW, 2 NSW)), 2 only
    // computes (head_dim 64: waves from 2 NSW on). The loop is compiled once per role, so each copy
    // keeps only its own staging addresses live, and waits for its own number of loads per tile.
    static_assert(RC::CODE_WAVES == kPW || RC::CODE_WAVES == 2 * RC::NSW, "computing-only waves all load codes or none");
    f16v sX, sY;  // the scores of block 0 (entering a step: tile t's) and block 1 of a tile
    auto step = [&](auto role, auto qkn, auto stg, int t) {
      constexpr int ROLE = decltype(role)::value;
      constexpr bool QKN = decltype(qkn)::value, STG = decltype(stg)::value;
      constexpr int IPT = (ROLE < 2 || RC::CODE_WAVES == kPW) ? RC::IPT : RC::IPT_NOCODE;
      // the step's buffers, as element (byte, for the raw ring) offsets from each array's start
      const int k_t = opaque((t % 3) * KBUF), k_t1 = opaque(((t + 1) % 3) * KBUF);
      const int k_w = opaque(((t + 2) % 3) * KBUF);
      const int v_t = opaque((t % 3) * VBUF), v_w = opaque(((t + 2) % 3) * VBUF);
      const uint8_t* raw2 = &raw[0][0] + opaque(((t + 2) % kRawSlots) * RC::SLOT);
      if constexpr (STG && ROLE == 0) {
        stage_v_table<T, BITS, G, D>(raw2, sb_tab[wave & 3], tid, range_bad, vmul);
        __builtin_amdgcn_wave_barrier();
      }
      const int k0 = k_begin + kPT * t;
      const _Float16* vl = vl_lane + v_t;
      u4 ring[4];
      u4 pop[2];
      // half 0: softmax of block 0 beside S(block 1) = K(t) rows 32-63 Q^T
      {
        const _Float16* kl = kl_lane + k_t + 32 * KS;
        mask_blk(sX, k0);
        const float tm = max_blk(sX);
        rescale(tm);
        qk_ring(ring, kl);
        qk_run(J0{}, JE{}, sY, ring, kl);
        probs_blk(sX, pop);
      }
      pv_blk(vl, pop, B0{});
      if constexpr (STG && ROLE == 0) stage_v<BITS, G, D, 0>(raw2, &v_lds[0][0] + v_w, sb_tab[wave & 3], tid);
      if constexpr (STG && ROLE == 1) stage_k<T, BITS, G, D, 0>(raw2, &k_lds[0][0] + k_w, tid, range_bad, kmul);
      // tile t + 4 into the slot of tile t + 1, issued between the halves (at the step's start
      // it delays the first half: about 2% slower on C3, as are the other positions tried)
      issue_raw(t + 4);
      // half 1: softmax of block 1 beside S(block 0 of tile t + 1) = K(t + 1) rows 0-31 Q^T
      {
        const _Float16* kl = kl_lane + k_t1;
        mask_blk(sY, k0 + 32);
        const float tm = max_blk(sY);
        rescale(tm);
        if constexpr (QKN) {
          qk_ring(ring, kl);
          qk_run(J0{}, JE{}, sX, ring, kl);
        }
        probs_blk(sY, pop);
      }
      pv_blk(vl, pop, B1{});
      if constexpr (STG && ROLE == 0) stage_v<BITS, G, D, 1>(raw2, &v_lds[0][0] + v_w, sb_tab[wave & 3], tid);
      if constexpr (STG && ROLE == 1) stage_k<T, BITS, G, D, 1>(raw2, &k_lds[0][0] + k_w, tid, range_bad, kmul);
      wait_vm<IPT>();  // tile t + 3 has landed (tile t + 4 may be in flight)
      __syncthreads();
    };
    using Y = std::true_type;
    using N = std::false_type;

    auto run = [&](auto role) {
      constexpr int ROLE = decltype(role)::value;
      constexpr int IPT = (ROLE < 2 || RC::CODE_WAVES == kPW) ? RC::IPT : RC::IPT_NOCODE;
      // prologue: tiles 0 and 1 dequantized, S(tile 0, block 0) computed, tile 2 landed, tile 3 in
      // flight
      wait_vm<2 * IPT>();
      __syncthreads();
      stage_from_raw<T, BITS, G, D>(raw[0], k_lds[0], v_lds[0], sb_tab[wave & 3], tid, range_bad, kmul, vmul);
      wait_vm<IPT>();
      __syncthreads();
      issue_raw(3);  // into the slot of tile 0
      stage_from_raw<T, BITS, G, D>(raw[1], k_lds[1], v_lds[1], sb_tab[wave & 3], tid, range_bad, kmul, vmul);
      {
        u4 ring[4];
        qk_ring(ring, kl_lane);
        qk_run(J0{}, JE{}, sX, ring, kl_lane);
      }
      wait_vm<IPT>();
      __syncthreads();
      int t = 0;
      for (; t + 2 < ntile; ++t) step(role, Y{}, Y{}, t);
      if (t + 1 < ntile) step(role, Y{}, N{}, t++);
      step(role, N{}, N{}, t);
    };
    if (wave < RC::NSW) {
      run(std::integral_constant<int, 0>{});
    } else if constexpr (2 * RC::NSW == kPW) {
      run(std::integral_constant<int, 1>{});
    } else {
      if (wave < 2 * RC::NSW) {
        run(std::integral_constant<int, 1>{});
      } else {
        run(std::integral_constant<int, 2>{});
      }
    }
  }
  wait_vm<0>();  // no load into this workgroup's LDS outlives it
  if constexpr (!DENSE && T::id == KVQ_DTYPE_BF16) {
    // a group beyond the fp16 range poisons the workgroup's rows: NaN propagates through the split
    // merge (0 * NaN is NaN) to every output row of the row block. (The tables are free: the last
    // tile step staged nothing and ended with a barrier.)
    const bool wave_bad = __builtin_amdgcn_ballot_w64(range_bad) != 0;
    if (lane == 0) s_flags[wave] = wave_bad;
    __syncthreads();
    unsigned any_bad = 0;
#pragma unroll
    for (int w = 0; w < kPW; ++w) any_bad |= s_flags[w];
    if (any_bad) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = __builtin_nanf("");
    }
  }

  // ---- epilogue: this lane holds O^T[d][row] for d = 32db + 8(i/4) + 4hh + i%4
  float l_tot = add_xor32(l_run);
  if (p.nsplit > 1) {
    // Key split: publish this split's partials, count the arrival, and let the unit's last split to
    // arrive merge them into its own registers.
    //  * A partial row is o / l in fp16, times 2^-e with e chosen per row so every stored value is
    //    below 2^14, and the row's record (m, l, 2^e). The merge scales row s by w_s l_s 2^e_s.
    //  * The merging split rounds its own partial through the same fp16 packing, so every split's
    //    term is formed from the same values whichever split merges: the result is
    //    bit-reproducible from call to call.
    //  * The packed row keeps the register image: lane `lane` of wave `wave` of split s holds words
    //    u (0 .. QW - 1) of 16 bytes at byte ((s * kPW + wave) * QW + u) * 1024 + 16 lane of the unit's o
    //    block; word u packs value groups 2u and 2u + 1 (group 4 db + c = oacc[db][4c .. 4c+3]).
    //    Record of row r at byte 16 (s * kPRows + r) of the unit's record block.
    const __amdgpu_buffer_rsrc_t ro = make_rsrc((const uint8_t*)p.part_o + (int64_t)unit * p.nsplit * (kPRows * 2 * D),
                                                (uint32_t)p.nsplit * (kPRows * 2 * D));
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(p.part_ml + (int64_t)unit * p.nsplit * (kPRows * 4),
                                                (uint32_t)p.nsplit * (kPRows * 16));
    const uint32_t lo = (uint32_t)wave * (QW * 1024) + 16 * lane;
    const uint32_t split_o = kPW * QW * 1024;
    const uint32_t row_ml = 16 * (wave * 32 + qc);
    u4 own[QW];
    float own_sc;
    {
      const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      float mx = 0.0f;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(oacc[db][i]));
      mx = max_xor32(mx) * inv_l;
      // mx * 2^-e lies in [2^13, 2^14): every row uses the full fp16 mantissa whatever its
      // magnitude (small rows would otherwise be stored as subnormals)
      int ex = 0;
      if (mx > 0.0f) frexpf(mx, &ex);
      const int e = mx > 0.0f ? min(max(ex - 14, -100), 100) : 0;
      own_sc = ldexpf(1.0f, e) * vback;  // the V operands were staged times 2^-E_V
      const float f = ldexpf(inv_l, -e);
#pragma unroll
      for (int u = 0; u < QW; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = 2 * u + h, db = g >> 2, c = g & 3;
          own[u][2 * h] = pack_f16x2(oacc[db][4 * c] * f, oacc[db][4 * c + 1] * f);
          own[u][2 * h + 1] = pack_f16x2(oacc[db][4 * c + 2] * f, oacc[db][4 * c + 3] * f);
        }
    }
#pragma unroll
    for (int u = 0; u < QW; ++u) store_agent_b128(ro, lo + u * 1024 + split * split_o, __builtin_bit_cast(f4, own[u]));
    if (hh == 0) store_agent_b128(rm, row_ml + split * (kPRows * 16), f4{m_run, l_tot, own_sc, 0.0f});
    // The stores are acknowledged (written through to the device's coherence point) before the
    // arrival is counted, so the last arrival sees every split's partials.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) *s_arrived = __hip_atomic_fetch_add(&p.counters[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*s_arrived != (unsigned)(p.nsplit - 1)) return;
    if (tid == 0) __hip_atomic_store(&p.counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // M = max over the splits that saw a key; weights 2^(m_s - M)
    float M = l_tot > 0.0f ? m_run : -INFINITY;
    for (int s2 = 0; s2 < p.nsplit; ++s2) {
      if (s2 == split) continue;
      const f4 rec = load_agent_b128(rm, row_ml, s2 * (kPRows * 16));
      if (rec[1] > 0.0f) M = fmaxf(M, rec[0]);
    }
    // the splits are summed in split order, each term one explicit fma
    f16v macc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) macc[db] = f16v{};
    float l_acc = 0.0f;
    for (int s2 = 0; s2 < p.nsplit; ++s2) {
      f4 rec;
      u4 po[QW];
      if (s2 == split) {
        rec = f4{m_run, l_tot, own_sc, 0.0f};
#pragma unroll
        for (int u = 0; u < QW; ++u) po[u] = own[u];
      } else {
        rec = load_agent_b128(rm, row_ml, s2 * (kPRows * 16));
#pragma unroll
        for (int u = 0; u < QW; ++u) po[u] = __builtin_bit_cast(u4, load_agent_b128(ro, lo + u * 1024, s2 * split_o));
      }
      const float w = (M == -INFINITY || rec[1] <= 0.0f) ? 0.0f : exp2_fast(rec[0] - M);
      l_acc = fmaf(w, rec[1], l_acc);
      const float F = (w * rec[1]) * rec[2];
#pragma unroll
      for (int u = 0; u < QW; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = 2 * u + h, db = g >> 2, c = g & 3;
          // halves are extracted with integer shifts: converting the elements of an h2 bit-cast
          // from a u4 element let the compiler (ROCm 7.2) fold all four words of a u4 into the
          // first one's register in v_fma_mix_f32
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t w = po[u][2 * h + (k >> 1)];
            const float x = (float)__builtin_bit_cast(_Float16, (uint16_t)((k & 1) ? w >> 16 : w & 0xffffu));
            macc[db][4 * c + k] = fmaf(F, x, macc[db][4 * c + k]);
          }
        }
    }
    l_tot = l_acc;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[db] = macc[db];
  }
  // ---- output. A lane holds 8-byte pieces of one row; stored directly, each store instruction
  // would write 8 bytes into each of 32 rows. Each wave instead stages its 32 rows in LDS (the
  // rings are free once every wave is past this barrier) and stores whole rows: 16 bytes a lane, so
  // an instruction writes 4 (D = 128) or 8 (D = 64) complete rows.
  // (after a split merge l_tot and oacc are in true units; else the V operands' 2^-ev returns here)
  const float inv = l_tot > 0.0f ? (1.0f / l_tot) * (p.nsplit > 1 ? 1.0f : vback) : 0.0f;
  constexpr int OP = D + 8;                 // fp16 per staged row: rows shift by 4 banks
  constexpr int WSB = 32 * OP * 2;          // staging bytes per wave
  constexpr int NRW = kRawSlots * RC::SLOT / WSB;           // waves staged in the raw ring
  constexpr int NVW = (DENSE ? 2 : 3) * D * kVS * 2 / WSB;  // ... and in the V^T ring
  static_assert(NRW + NVW >= kPW, "every wave's rows fit the raw and V^T rings");
  __syncthreads();
  uint16_t* const stage =
      (uint16_t*)(wave < NRW ? &raw[0][0] + wave * WSB : (uint8_t*)&v_lds[0][0] + (wave - NRW) * WSB);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u2 w;
      w[0] = (uint32_t)from_float(oacc[db][4 * c] * inv, T{}) | ((uint32_t)from_float(oacc[db][4 * c + 1] * inv, T{}) << 16);
      w[1] = (uint32_t)from_float(oacc[db][4 * c + 2] * inv, T{}) | ((uint32_t)from_float(oacc[db][4 * c + 3] * inv, T{}) << 16);
      *(u2*)(stage + qc * OP + 32 * db + 8 * c + 4 * hh) = w;
    }
  // the output offset of this lane's row (lanes 0-31 own the wave's rows), read by the lanes that
  // store it
  const int64_t roff = (int64_t)b * p.o_sb + (int64_t)head * p.o_sh + (int64_t)lq * p.o_sl;
  const int roff_lo = (int)(uint32_t)roff, roff_hi = (int)(roff >> 32);
  __builtin_amdgcn_wave_barrier();  // the wave's LDS writes are issued before its reads (LDS keeps a wave's order)
  constexpr int CPR = D / 8;   // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per store instruction
  const int cc = lane % CPR;
#pragma unroll
  for (int it = 0; it < 32 / RPI; ++it) {
    const int r = it * RPI + lane / CPR;
    const u4 v = *(const u4*)(stage + r * OP + 8 * cc);
    const int64_t ro = (int64_t)(((uint64_t)(uint32_t)__shfl(roff_hi, r) << 32) | (uint32_t)__shfl(roff_lo, r));
    if (fr0 + wave * 32 + r < p.nrows) {
      *(u4*)(p.out + ro + 8 * cc) = v;  // the host checks 16-byte aligned rows and strides
    }
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
static PreLayout prefill_layout(const PrePlan& pl, int D) {
  PreLayout l;
  const size_t slots = (size_t)pl.nunits * pl.nsplit * kPRows;
  l.o = kCounterBytes;
  l.ml = l.o + slots * D * sizeof(uint16_t);  // fp16 rows
  l.total = l.ml + (slots * 4 * sizeof(float) + 255) / 256 * 256;  // (m, l, 2^e, -) records
  return l;
}

size_t prefill_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window, int) {
  const PrePlan pl = prefill_plan(B, Hq, Hkv, L, S, window);
  if (pl.nsplit == 1) return 256;
  return prefill_layout(pl, D).total;
}

template <typename T, int BITS, bool PAGED = false, int G = 64, int D = 128>
static hipError_t launch_prefill_t(const PreParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((prefill_attn_kernel<T, BITS, PAGED, G, D>), dim3(p.nunits * p.nsplit), dim3(kPW * 64), 0, stream,
                     p);
  return hipGetLastError();
}

// The quantized instantiation for (dtype, D in {64, 128}, bits in {4, 8}, G in {32, 64, 128}, G <= D).
template <bool PAGED>
static hipError_t launch_prefill_quant(const PreParams& p, int dtype, int D, int bits, int G, hipStream_t stream) {
  auto by_g = [&](auto t, auto d, auto b) -> hipError_t {
    using TT = decltype(t);
    constexpr int DD = decltype(d)::value;
    constexpr int BB = decltype(b)::value;
    if (G == 32) return launch_prefill_t<TT, BB, PAGED, 32, DD>(p, stream);
    if constexpr (DD >= 128) {
      if (G == 128) return launch_prefill_t<TT, BB, PAGED, 128, DD>(p, stream);
    }
    return launch_prefill_t<TT, BB, PAGED, 64, DD>(p, stream);
  };
  auto by_d = [&](auto t, auto b) -> hipError_t {
    return D == 64 ? by_g(t, std::integral_constant<int, 64>{}, b) : by_g(t, std::integral_constant<int, 128>{}, b);
  };
  auto by_b = [&](auto t) -> hipError_t {
    return bits == 8 ? by_d(t, std::integral_constant<int, 8>{}) : by_d(t, std::integral_constant<int, 4>{});
  };
  return dtype == KVQ_DTYPE_BF16 ? by_b(BF16{}) : by_b(F16{});
}

// Everything but the K/V operands.
static PreParams prefill_params(const kvq_rows* q, const int32_t* seq_lens, const kvq_rows* out, int Hq, int Hkv, int L, int D,
                                int S, float scale, int causal, int window, void* workspace, const PrePlan& pl) {
  PreParams p{};
  p.q = (const uint16_t*)q->data;
  p.q_sb = q->stride_b;
  p.q_sh = q->stride_h;
  p.q_sl = q->stride_l;
  p.seq_lens = seq_lens;
  p.out = (uint16_t*)out->data;
  p.o_sb = out->stride_b;
  p.o_sh = out->stride_h;
  p.o_sl = out->stride_l;
  const PreLayout lay = prefill_layout(pl, D);
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
  p.xcd_remap = ((int64_t)pl.nunits * pl.nsplit) % kXcds == 0;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.causal = causal;
  p.window = window;
  return p;
}

hipError_t launch_prefill(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                          const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype,
                          float scale, int causal, int window, void* workspace, hipStream_t stream) {
  const PrePlan pl = prefill_plan(B, Hq, Hkv, L, S, window);
  PreParams p = prefill_params(q, seq_lens, out, Hq, Hkv, L, D, S, scale, causal, window, workspace, pl);
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
  return launch_prefill_quant<false>(p, dtype, D, bits, G, stream);
}

hipError_t launch_prefill_paged(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                                const int32_t* table, int64_t table_stride, const int32_t* seq_lens, const kvq_rows* out,
                                int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype, float scale,
                                int causal, int window, void* workspace, hipStream_t stream) {
  const PrePlan pl = prefill_plan(B, Hq, Hkv, L, S, window);
  PreParams p = prefill_params(q, seq_lens, out, Hq, Hkv, L, D, S, scale, causal, window, workspace, pl);
  p.kc = (const uint8_t*)k->codes;
  p.vc = (const uint8_t*)v->codes;
  p.kc_sb = k->codes_stride_b * 4;  // page strides
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
  p.table = table;
  p.table_stride = table_stride;
  p.num_pages = num_pages;
  return launch_prefill_quant<true>(p, dtype, D, bits, G, stream);
}

hipError_t launch_prefill_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                                const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype,
                                float scale, int causal, int window, void* workspace, hipStream_t stream) {
  const PrePlan pl = prefill_plan(B, Hq, Hkv, L, S, window);
  PreParams p = prefill_params(q, seq_lens, out, Hq, Hkv, L, D, S, scale, causal, window, workspace, pl);
  p.kc = (const uint8_t*)k->data;
  p.vc = (const uint8_t*)v->data;
  p.kc_sb = k->stride_b * 2;
  p.kc_sh = k->stride_h * 2;
  p.kc_ss = k->stride_l * 2;
  p.vc_sb = v->stride_b * 2;
  p.vc_sh = v->stride_h * 2;
  p.vc_ss = v->stride_l * 2;
  if (dtype == KVQ_DTYPE_BF16) return launch_prefill_t<BF16, 16>(p, stream);
  return launch_prefill_t<F16, 16>(p, stream);
}

}  // namespace kvq
