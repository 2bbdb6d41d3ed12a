// Split-K flash-decoding over an MLX-layout affine-quantized KV cache (small L), or over an
// unquantized fp16/bf16 cache, with a log-sum-exp merge of the key splits.
//
// Computes, per (sequence b, query head h, query row l):
//   out = softmax(scale * q K^T + mask) V,   K = sK * codesK + bK,  V = sV * codesV + bV
// i.e. the quantity m5engine/attention.py:29-103 evaluates (blocked online softmax, :64-100)
// and that its L == 1 branch (:42-45) hands to mlx-lm's quantized SDPA.
//
// Design (one wave = 16 MFMA columns; NG = D/G scale groups per row, head_dim 64, 128 or 256):
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
//  * Each wave streams its 32-key tiles through a ring of NSLOT LDS slots filled by buffer->LDS
//    DMA: every code load is one contiguous KiB (16 bytes a lane), scales and biases arrive as
//    16-bit loads, and no VGPR holds data in flight, so NSLOT - 1 tiles stream while one is
//    computed. Rows past the sequence end read as zero through the buffer range check. K rows
//    are stored with their 16-byte chunks XOR-swizzled by row, so the MFMA operand reads (one
//    key row per lane) are free of LDS bank conflicts.
//  * Online softmax in the log2 domain; rescaling of the output accumulators is lazy (only when a
//    row maximum grows). The waves of a workgroup merge in LDS into one (m, l, o[D]) partial per
//    query row. A second small launch (combine_kernel) merges the splits and writes the output;
//    optionally (fused mode) the last workgroup of each (sequence, KV head, row block) to finish --
//    found with a device-scope counter that it resets afterwards -- merges them instead.
//  * The unquantized cache (BITS == 16) takes the same path with raw 16-bit rows as MFMA operands
//    (bf16 MFMA for bf16 caches), no scales or biases, and the raw query as the Q operand.
//  * Workgroups are numbered so that the splits of one KV head land on one XCD (hardware hands
//    consecutive workgroups to the 8 XCDs in turn), keeping the merge inside one L2.

#include <math.h>
#include <stdlib.h>

#include <type_traits>

#include "common.h"
#include "launch.h"
#include "merge.h"

namespace kvq {

constexpr int kTile = 32;
constexpr int kXcds = 8;

// BITS == 16 is the unquantized cache: raw T rows, no scales or biases. It keeps the column
// layout of the quantized cache (R query rows, each in NG columns), with every column computing the
// row's full dot product, so the wave epilogue below serves both.
template <int D, int BITS, int G = 64>
struct DecCfg {
  static constexpr bool DENSE = BITS == 16;
  static_assert(G == 32 || G == 64 || G == 128, "group sizes 32, 64, 128");
  static_assert(D % G == 0 && D / 4 <= G, "a lane group's quarter of a row lies in one scale group");
  static constexpr int NG = D / G;             // scale groups per row
  static constexpr int R = 16 / NG;            // query rows per wave
  static constexpr int KSTEPS = D / 32;        // QK MFMA k-steps (8 dims per lane each)
  static constexpr int NBLK = D / 16;          // PV MFMA column blocks
  static constexpr int ROWB = D * BITS / 8;    // code bytes per key row
  static constexpr int KLB = ROWB / 4;         // K code bytes per lane per key (4 lane groups)
  static constexpr int VLB = ROWB / 16;        // V code bytes per lane per key (16 columns)
  static constexpr int CPR = ROWB / 16;        // 16-byte chunks per code row
  static constexpr int RPI = 64 / CPR;         // code rows per 1 KiB DMA instruction
  static constexpr int CI = kTile / RPI;       // DMA instructions per K (or V) tile
  static constexpr int TB = kTile * ROWB;      // bytes of a K (or V) tile
  // a ring slot: [K tile][V tile][sK, bK, sV, bV: SBC 4-byte cells each, value in the low half;
  // cell 32 g + k holds group g of key k] (no scale/bias cells for the unquantized cache). One
  // 2-byte DMA fills 64 cells (two groups of 32 keys), so NSB of them fill an array.
  static constexpr int NSB = NG > 2 ? NG / 2 : 1;
  static constexpr int SBC = 64 * NSB;
  static constexpr int AS = 4 * SBC;  // bytes between the arrays
  static constexpr int SLOT = 2 * TB + (DENSE ? 0 : 4 * AS);
  static constexpr int IPT = 2 * CI + (DENSE ? 0 : 4 * NSB);  // DMA instructions per tile
  // The XOR swizzle of the 16-byte chunks of K row r: r % CPR with one more bit of r folded in, so
  // that the 16 keys x 2 lane groups of a 32-lane half of each operand read (ds_read_b128, 128
  // banks of 4 bytes) fall on 32 distinct 16-byte bank groups. With r % CPR alone, keys r and r + 8
  // (CPR 8, 4) or r and r + 4 (CPR 16) met in one bank group: a 2-way conflict on every K read.
  static constexpr int kswz(int r) {
    return (r % CPR) ^ (CPR == 16 ? (r >> 2) & 1 : CPR == 8 ? (r >> 3) & 1 : CPR == 4 ? 2 * ((r >> 3) & 1) : 0);
  }
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
  float scale_log2;
  int causal, window;
  // paged cache (PAGED kernels): rows of sequence b live in 64-row pages, page table[b][r / 64];
  // the codes/scales/biases batch strides above are then page strides
  const int32_t* table;
  int64_t table_stride;
  int num_pages;
  // general mask (kvq_mask): kind 0 = none; otherwise every tile is masked element by element
  const void* mask;
  int mask_kind;
  int64_t m_sb, m_skv, m_srep, m_sl;
  // the head dimension of the rows (a multiple of 8, at most the kernel's D): a narrower row is
  // computed as a D-wide one whose dims past dv carry zero queries, and only dims below dv are stored
  int dv;
  // nsplit, rowblocks, Hkv and L as multiply-shift divisors (the workgroup and row numbering)
  Div31 d_nsplit, d_rowblocks, d_hkv, d_l;
};

// A general mask (kvq_mask) on the lane's 8 scores of a tile (keys k0 + 16 (s / 4) + 4 lg + s % 4 of
// query row (b, kvh, j, l), log2 units): a boolean mask sends hidden keys to -inf, an additive one
// adds its value times log2(e). Keys outside [lo, hi) are already -inf and are not read.
__device__ __forceinline__ void apply_mask(const DecParams& p, int b, int kvh, int j, int l, int k0, int lg, int lo, int hi,
                                        float (&sc)[8]) {
  const int64_t row = (int64_t)b * p.m_sb + (int64_t)kvh * p.m_skv + (int64_t)j * p.m_srep + (int64_t)l * p.m_sl;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int t = k0 + 16 * (s >> 2) + 4 * lg + (s & 3);
    if (!(t >= lo && t < hi)) continue;
    const int64_t i = row + t;
    if (p.mask_kind == KVQ_MASK_BOOL) {
      if (((const uint8_t*)p.mask)[i] == 0) sc[s] = -INFINITY;
    } else {
      float a;
      if (p.mask_kind == KVQ_MASK_F32) {
        a = ((const float*)p.mask)[i];
      } else if (p.mask_kind == KVQ_MASK_BF16) {
        a = to_float(((const uint16_t*)p.mask)[i], BF16{});
      } else {
        a = to_float(((const uint16_t*)p.mask)[i], F16{});
      }
      sc[s] += a * 1.4426950408889634f;
    }
  }
}

// Token (relative to the tile) of V slot i' (the MFMA k index 8*lg + i') for lane group lg.
__device__ __forceinline__ int v_token(int lg, int i) { return (i < 4) ? 4 * lg + i : 16 + 4 * lg + (i - 4); }

// Buffer->LDS DMA: lane i's 16 bytes (dma16) or 2 bytes (dma2, in the low half of a 4-byte cell)
// land at lds + 16 i (+ 4 i); `lds` is wave-uniform. Device-only wrappers keep the target builtin
// out of the host pass.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t vo, uint32_t so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, vo, so, 0, 0);
}
__device__ __forceinline__ void dma2(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t vo, uint32_t so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 2, vo, so, 0, 0);
}

// 32-bit LDS address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// The LDS operands of one 32-key tile, read by one asm block that also waits for them. The reads
// are asm so that the compiler does not tie them to the buffer->LDS loads still in flight into
// other ring slots (it would otherwise wait for every outstanding load before any LDS read); the
// ring's own vmcnt waits order each slot's fill before its read.
//   k[beta]  : the lane's KLB bytes of key 16 beta + n (XOR-swizzled chunks)
//   sb[a][b] : 4 cells of array a (sK, bK, sV, bV) for the lane's group at keys 16 b + 4 lg .. +3
//   v[i]     : the lane's VLB-byte column slice of key v_token(lg, i)
template <int ROWB>
struct TileOps;
template <>
struct TileOps<256> {
  u4 k[2][4];
  u4 sb[4][2];
  u4 v[8];
};
template <>
struct TileOps<128> {
  u4 k[2][2];
  u4 sb[4][2];
  u2 v[8];
};
template <>
struct TileOps<64> {
  u4 k[2];
  u4 sb[4][2];
  uint32_t v[8];
};
template <>
struct TileOps<32> {
  u2 k[2];
  u4 sb[4][2];
  uint32_t v[8];
};

// ka: the K chunk addresses of key n (one per 16-byte chunk of the lane's quarter row; rows below
// 128 bytes use the first); sa: the sb base; va: the V slice address of key 4 lg. AS: bytes between
// the scale/bias arrays of a slot.
template <int AS>
__device__ __forceinline__ void read_tile(TileOps<256>& t, const uint32_t (&ka)[4], uint32_t sa, uint32_t va) {
  asm volatile(
      "ds_read_b128 %0, %24\n"
      "ds_read_b128 %1, %25\n"
      "ds_read_b128 %2, %26\n"
      "ds_read_b128 %3, %27\n"
      "ds_read_b128 %4, %24 offset:4096\n"
      "ds_read_b128 %5, %25 offset:4096\n"
      "ds_read_b128 %6, %26 offset:4096\n"
      "ds_read_b128 %7, %27 offset:4096\n"
      "ds_read_b128 %8, %28\n"
      "ds_read_b128 %9, %28 offset:64\n"
      "ds_read_b128 %10, %28 offset:%30\n"
      "ds_read_b128 %11, %28 offset:%31\n"
      "ds_read_b128 %12, %28 offset:%32\n"
      "ds_read_b128 %13, %28 offset:%33\n"
      "ds_read_b128 %14, %28 offset:%34\n"
      "ds_read_b128 %15, %28 offset:%35\n"
      "ds_read_b128 %16, %29\n"
      "ds_read_b128 %17, %29 offset:256\n"
      "ds_read_b128 %18, %29 offset:512\n"
      "ds_read_b128 %19, %29 offset:768\n"
      "ds_read_b128 %20, %29 offset:4096\n"
      "ds_read_b128 %21, %29 offset:4352\n"
      "ds_read_b128 %22, %29 offset:4608\n"
      "ds_read_b128 %23, %29 offset:4864\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t.k[0][0]), "=&v"(t.k[0][1]), "=&v"(t.k[0][2]), "=&v"(t.k[0][3]), "=&v"(t.k[1][0]), "=&v"(t.k[1][1]),
        "=&v"(t.k[1][2]), "=&v"(t.k[1][3]), "=&v"(t.sb[0][0]), "=&v"(t.sb[0][1]), "=&v"(t.sb[1][0]),
        "=&v"(t.sb[1][1]), "=&v"(t.sb[2][0]), "=&v"(t.sb[2][1]), "=&v"(t.sb[3][0]), "=&v"(t.sb[3][1]), "=&v"(t.v[0]),
        "=&v"(t.v[1]), "=&v"(t.v[2]), "=&v"(t.v[3]), "=&v"(t.v[4]), "=&v"(t.v[5]), "=&v"(t.v[6]), "=&v"(t.v[7])
      : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(sa), "v"(va), "i"(AS), "i"(AS + 64), "i"(2 * AS),
        "i"(2 * AS + 64), "i"(3 * AS), "i"(3 * AS + 64)
      : "memory");
}
template <int AS>
__device__ __forceinline__ void read_tile(TileOps<128>& t, const uint32_t (&ka)[4], uint32_t sa, uint32_t va) {
  const uint32_t ka0 = ka[0], ka1 = ka[1];
  asm volatile(
      "ds_read_b128 %0, %20\n"
      "ds_read_b128 %1, %21\n"
      "ds_read_b128 %2, %20 offset:2048\n"
      "ds_read_b128 %3, %21 offset:2048\n"
      "ds_read_b128 %4, %22\n"
      "ds_read_b128 %5, %22 offset:64\n"
      "ds_read_b128 %6, %22 offset:%24\n"
      "ds_read_b128 %7, %22 offset:%25\n"
      "ds_read_b128 %8, %22 offset:%26\n"
      "ds_read_b128 %9, %22 offset:%27\n"
      "ds_read_b128 %10, %22 offset:%28\n"
      "ds_read_b128 %11, %22 offset:%29\n"
      "ds_read_b64 %12, %23\n"
      "ds_read_b64 %13, %23 offset:128\n"
      "ds_read_b64 %14, %23 offset:256\n"
      "ds_read_b64 %15, %23 offset:384\n"
      "ds_read_b64 %16, %23 offset:2048\n"
      "ds_read_b64 %17, %23 offset:2176\n"
      "ds_read_b64 %18, %23 offset:2304\n"
      "ds_read_b64 %19, %23 offset:2432\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t.k[0][0]), "=&v"(t.k[0][1]), "=&v"(t.k[1][0]), "=&v"(t.k[1][1]), "=&v"(t.sb[0][0]), "=&v"(t.sb[0][1]),
        "=&v"(t.sb[1][0]), "=&v"(t.sb[1][1]), "=&v"(t.sb[2][0]), "=&v"(t.sb[2][1]), "=&v"(t.sb[3][0]),
        "=&v"(t.sb[3][1]), "=&v"(t.v[0]), "=&v"(t.v[1]), "=&v"(t.v[2]), "=&v"(t.v[3]), "=&v"(t.v[4]), "=&v"(t.v[5]),
        "=&v"(t.v[6]), "=&v"(t.v[7])
      : "v"(ka0), "v"(ka1), "v"(sa), "v"(va), "i"(AS), "i"(AS + 64), "i"(2 * AS), "i"(2 * AS + 64), "i"(3 * AS),
        "i"(3 * AS + 64)
      : "memory");
}
template <int AS>
__device__ __forceinline__ void read_tile(TileOps<64>& t, const uint32_t (&ka)[4], uint32_t sa, uint32_t va) {
  const uint32_t ka0 = ka[0];
  asm volatile(
      "ds_read_b128 %0, %18\n"
      "ds_read_b128 %1, %18 offset:1024\n"
      "ds_read_b128 %2, %19\n"
      "ds_read_b128 %3, %19 offset:64\n"
      "ds_read_b128 %4, %19 offset:%21\n"
      "ds_read_b128 %5, %19 offset:%22\n"
      "ds_read_b128 %6, %19 offset:%23\n"
      "ds_read_b128 %7, %19 offset:%24\n"
      "ds_read_b128 %8, %19 offset:%25\n"
      "ds_read_b128 %9, %19 offset:%26\n"
      "ds_read_b32 %10, %20\n"
      "ds_read_b32 %11, %20 offset:64\n"
      "ds_read_b32 %12, %20 offset:128\n"
      "ds_read_b32 %13, %20 offset:192\n"
      "ds_read_b32 %14, %20 offset:1024\n"
      "ds_read_b32 %15, %20 offset:1088\n"
      "ds_read_b32 %16, %20 offset:1152\n"
      "ds_read_b32 %17, %20 offset:1216\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t.k[0]), "=&v"(t.k[1]), "=&v"(t.sb[0][0]), "=&v"(t.sb[0][1]), "=&v"(t.sb[1][0]), "=&v"(t.sb[1][1]),
        "=&v"(t.sb[2][0]), "=&v"(t.sb[2][1]), "=&v"(t.sb[3][0]), "=&v"(t.sb[3][1]), "=&v"(t.v[0]), "=&v"(t.v[1]),
        "=&v"(t.v[2]), "=&v"(t.v[3]), "=&v"(t.v[4]), "=&v"(t.v[5]), "=&v"(t.v[6]), "=&v"(t.v[7])
      : "v"(ka0), "v"(sa), "v"(va), "i"(AS), "i"(AS + 64), "i"(2 * AS), "i"(2 * AS + 64), "i"(3 * AS), "i"(3 * AS + 64)
      : "memory");
}
template <int AS>
__device__ __forceinline__ void read_tile(TileOps<32>& t, const uint32_t (&ka)[4], uint32_t sa, uint32_t va) {
  const uint32_t ka0 = ka[0];
  asm volatile(
      "ds_read_b64 %0, %18\n"
      "ds_read_b64 %1, %18 offset:512\n"
      "ds_read_b128 %2, %19\n"
      "ds_read_b128 %3, %19 offset:64\n"
      "ds_read_b128 %4, %19 offset:%21\n"
      "ds_read_b128 %5, %19 offset:%22\n"
      "ds_read_b128 %6, %19 offset:%23\n"
      "ds_read_b128 %7, %19 offset:%24\n"
      "ds_read_b128 %8, %19 offset:%25\n"
      "ds_read_b128 %9, %19 offset:%26\n"
      "ds_read_u16 %10, %20\n"
      "ds_read_u16 %11, %20 offset:32\n"
      "ds_read_u16 %12, %20 offset:64\n"
      "ds_read_u16 %13, %20 offset:96\n"
      "ds_read_u16 %14, %20 offset:512\n"
      "ds_read_u16 %15, %20 offset:544\n"
      "ds_read_u16 %16, %20 offset:576\n"
      "ds_read_u16 %17, %20 offset:608\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t.k[0]), "=&v"(t.k[1]), "=&v"(t.sb[0][0]), "=&v"(t.sb[0][1]), "=&v"(t.sb[1][0]), "=&v"(t.sb[1][1]),
        "=&v"(t.sb[2][0]), "=&v"(t.sb[2][1]), "=&v"(t.sb[3][0]), "=&v"(t.sb[3][1]), "=&v"(t.v[0]), "=&v"(t.v[1]),
        "=&v"(t.v[2]), "=&v"(t.v[3]), "=&v"(t.v[4]), "=&v"(t.v[5]), "=&v"(t.v[6]), "=&v"(t.v[7])
      : "v"(ka0), "v"(sa), "v"(va), "i"(AS), "i"(AS + 64), "i"(2 * AS), "i"(2 * AS + 64), "i"(3 * AS), "i"(3 * AS + 64)
      : "memory");
}

// The LDS operands of one 32-key tile of the unquantized cache (raw T rows):
//   k[beta][c] : chunk c of the lane's D/4 dims of key 16 beta + n (chunk position swizzled by
//                key, so each chunk has its own address: ka[c])
//   v[i]       : the lane's D/16 dims of key v_token(lg, i)
template <int D>
struct DenseOps;
template <>
struct DenseOps<128> {
  u4 k[2][4];
  u4 v[8];
};
template <>
struct DenseOps<64> {
  u4 k[2][2];
  u2 v[8];
};

__device__ __forceinline__ void read_tile_dense(DenseOps<128>& t, const uint32_t (&ka)[4], uint32_t va) {
  asm volatile(
      "ds_read_b128 %0, %16\n"
      "ds_read_b128 %1, %17\n"
      "ds_read_b128 %2, %18\n"
      "ds_read_b128 %3, %19\n"
      "ds_read_b128 %4, %16 offset:4096\n"
      "ds_read_b128 %5, %17 offset:4096\n"
      "ds_read_b128 %6, %18 offset:4096\n"
      "ds_read_b128 %7, %19 offset:4096\n"
      "ds_read_b128 %8, %20\n"
      "ds_read_b128 %9, %20 offset:256\n"
      "ds_read_b128 %10, %20 offset:512\n"
      "ds_read_b128 %11, %20 offset:768\n"
      "ds_read_b128 %12, %20 offset:4096\n"
      "ds_read_b128 %13, %20 offset:4352\n"
      "ds_read_b128 %14, %20 offset:4608\n"
      "ds_read_b128 %15, %20 offset:4864\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t.k[0][0]), "=&v"(t.k[0][1]), "=&v"(t.k[0][2]), "=&v"(t.k[0][3]), "=&v"(t.k[1][0]), "=&v"(t.k[1][1]),
        "=&v"(t.k[1][2]), "=&v"(t.k[1][3]), "=&v"(t.v[0]), "=&v"(t.v[1]), "=&v"(t.v[2]), "=&v"(t.v[3]), "=&v"(t.v[4]),
        "=&v"(t.v[5]), "=&v"(t.v[6]), "=&v"(t.v[7])
      : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(va)
      : "memory");
}
__device__ __forceinline__ void read_tile_dense(DenseOps<64>& t, const uint32_t (&ka)[2], uint32_t va) {
  asm volatile(
      "ds_read_b128 %0, %12\n"
      "ds_read_b128 %1, %13\n"
      "ds_read_b128 %2, %12 offset:2048\n"
      "ds_read_b128 %3, %13 offset:2048\n"
      "ds_read_b64 %4, %14\n"
      "ds_read_b64 %5, %14 offset:128\n"
      "ds_read_b64 %6, %14 offset:256\n"
      "ds_read_b64 %7, %14 offset:384\n"
      "ds_read_b64 %8, %14 offset:2048\n"
      "ds_read_b64 %9, %14 offset:2176\n"
      "ds_read_b64 %10, %14 offset:2304\n"
      "ds_read_b64 %11, %14 offset:2432\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(t.k[0][0]), "=&v"(t.k[0][1]), "=&v"(t.k[1][0]), "=&v"(t.k[1][1]), "=&v"(t.v[0]), "=&v"(t.v[1]),
        "=&v"(t.v[2]), "=&v"(t.v[3]), "=&v"(t.v[4]), "=&v"(t.v[5]), "=&v"(t.v[6]), "=&v"(t.v[7])
      : "v"(ka[0]), "v"(ka[1]), "v"(va)
      : "memory");
}

// V operand of the unquantized cache for column block jN: the 16-bit value at the lane's dim jN
// of each of its 8 keys, packed in key order.
template <typename VT>
__device__ __forceinline__ u4 v_operand_dense(const VT (&vr)[8], int jN) {
  const uint32_t sel = (jN & 1) ? 0x07060302u : 0x05040100u;
  u4 r;
#pragma unroll
  for (int a = 0; a < 4; ++a) r[a] = perm(vr[2 * a + 1][jN >> 1], vr[2 * a][jN >> 1], sel);
  return r;
}

// s_waitcnt vmcnt(N) (N < 64), other counters left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// K operand (A of S^T = K Q^T) for k-step j: 8 codes of the lane's key as f16 subnormals.
template <int D, int BITS>
__device__ __forceinline__ h8 k_operand(const Bytes<D * BITS / 32>& kc, int j) {
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
template <int D, int BITS, int VB>
__device__ __forceinline__ h8 v_operand(const Bytes<VB> (&vc)[8], int jN) {
  const int byte_off = (jN * BITS) / 8;  // byte of the lane's slice holding code jN
  const int wi = byte_off / 4;
  const uint32_t jb = (uint32_t)(byte_off % 4);
  const uint32_t sel = 0x0C000C00u | ((4u + jb) << 16) | jb;
  u4 r;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    uint32_t y = perm(vc[2 * a + 1].w[wi], vc[2 * a].w[wi], sel);
    // 4 bits: an even block takes the byte's low nibble; an odd block takes the whole byte,
    // lo + 16 hi, and the even block's sum is subtracted from it at the end (one AND fewer)
    if constexpr (BITS == 4) {
      if (!(jN & 1)) y &= 0x000F000Fu;
    }
    r[a] = y;
  }
  return __builtin_bit_cast(h8, r);
}

// Rescaling slack, log2 units: a row's running maximum is raised only when a tile's maximum
// exceeds it by more than this, so most tiles skip the accumulator rescale. Probabilities stay
// below 2^kSlack; with fp16 scales (|s| <= 514) the fp16 PV operand p*s stays finite.
constexpr float kSlack = 6.0f;

// Split counts up to which the in-kernel merge loads every split's partial in one round.
constexpr int kFewSplits = 4;

// Workgroups per CU the launch bounds ask for: two 4-wave workgroups when their rings fit in LDS
// together, else one.
template <int D, int BITS, int NW, int NSLOT, int G>
constexpr int dec_min_wgs() {
  return (NW == 4 && 2 * NW * NSLOT * DecCfg<D, BITS, G>::SLOT <= 160 * 1024) ? 2 : 1;
}

// MASKED: compiled with a general mask (kvq_mask) read beside every tile; NARROW: for rows of p.dv < D
// dims. The other instantiations carry no trace of either.
template <typename T, int D, int BITS, int NW, int NSLOT, bool PAGED = false, int G = 64, bool MASKED = false,
          bool NARROW = false>
__global__ __launch_bounds__(NW * 64, (dec_min_wgs<D, BITS, NW, NSLOT, G>())) void decode_attn_kernel(DecParams p) {
  using C = DecCfg<D, BITS, G>;
  constexpr int R = C::R;
  constexpr int NT = NW * 64;
  // the tile ring while streaming; the waves' (m, l, o) and the split weights afterwards
  constexpr int kRing = NW * NSLOT * C::SLOT;
  constexpr int kEpi = (2 * NW * R + NW * R * D + R * kMaxSplit) * 4;
  __shared__ __align__(16) uint8_t smem[kRing > kEpi ? kRing : kEpi];
  __shared__ unsigned s_prev;

  const int lane = __lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, lg = lane >> 4;

  // ---- workgroup -> (unit, split); a unit is (sequence, KV head, row block)
  // Kernel arguments arrive in dependent rounds of scalar loads wherever a branch separates their
  // uses. The pointers and strides the query and first tile loads need are requested up front
  // (an empty asm takes them as operands) and the workgroup numbering is a select, so they arrive
  // in one round.
  asm volatile("" ::"s"(p.q), "s"(p.kc), "s"(p.vc), "s"(p.ks), "s"(p.kb), "s"(p.vs), "s"(p.vb));
  asm volatile("" ::"s"(p.q_sb), "s"(p.q_sh), "s"(p.q_sl), "s"(p.kc_sb), "s"(p.kc_sh), "s"(p.kc_ss), "s"(p.vc_sb),
               "s"(p.vc_sh), "s"(p.vc_ss));
  asm volatile("" ::"s"(p.ksb_sb), "s"(p.ksb_sh), "s"(p.ksb_ss), "s"(p.vsb_sb), "s"(p.vsb_sh), "s"(p.vsb_ss));
  const int dims = NARROW ? p.dv : D;  // dims of a row (a compile-time D unless NARROW)
  if constexpr (NARROW) asm volatile("" ::"s"(dims));
  const int wg0 = blockIdx.x;
  const int wg = p.xcd_remap ? (wg0 % kXcds) * ((p.nunits * p.nsplit) / kXcds) + wg0 / kXcds : wg0;
  const int unit = (int)div31((uint32_t)wg, p.d_nsplit);
  const int split = wg - unit * p.nsplit;
  const int bk = (int)div31((uint32_t)unit, p.d_rowblocks);  // b * Hkv + kvh
  const int rb = unit - bk * p.rowblocks;
  const int b = (int)div31((uint32_t)bk, p.d_hkv);
  const int kvh = bk - b * p.Hkv;

  const int S_b = p.seq_lens ? min(max(load_uniform_i32(p.seq_lens, b), 0), p.S) : p.S;  // clamped: never read past the view
  // the first key any row sees, rounded down to a tile boundary (tiles stay 32-aligned, so a tile of
  // a paged cache lies in one page; the keys before the window are masked)
  const int key_base = p.window > 0 ? max(0, S_b - p.L - p.window + 1) & ~(kTile - 1) : 0;
  const int k_begin = key_base + split * p.chunk;
  const int k_end = min(k_begin + p.chunk, S_b);
  const int ntile = k_end > k_begin ? (k_end - k_begin + kTile - 1) / kTile : 0;
  const int nmine = ntile > wave ? (ntile - wave + NW - 1) / NW : 0;  // tiles wave, wave + NW, ...

  // ---- this lane's query row / group, and its raw query slice (loaded before the tile stream
  // so that waiting for it does not wait for the tiles)
  const int r = n % R, g = n / R;
  const int row = rb * R + r;
  const bool row_ok = row < p.nrows;
  const int rq = (int)div31((uint32_t)row, p.d_l);  // row / L
  const int hq = kvh * p.rep + (row_ok ? rq : 0);
  const int lq = row_ok ? row - rq * p.L : 0;
  const bool in_group = (lg * (D / 4)) / G == g;
  u4 qraw[C::KSTEPS];
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)lq * p.q_sl + lg * (D / 4);
    // in bounds: row and head are clamped, and dims from dv on (a row narrower than D) are not read
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j)
      qraw[j] = (!NARROW || lg * (D / 4) + 8 * j < dims) ? *(const u4*)(qrow + 8 * j) : u4{0, 0, 0, 0};
  }

  // ---- tile stream: buffer resources over the S_b valid rows of this (sequence, KV head); the
  // host checks that S * row stride fits 32 bits for every array
  const uint8_t* kbase = p.kc + (int64_t)b * p.kc_sb + (int64_t)kvh * p.kc_sh;
  const uint8_t* vbase = p.vc + (int64_t)b * p.vc_sb + (int64_t)kvh * p.vc_sh;
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kbase, (uint32_t)((int64_t)S_b * p.kc_ss));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vbase, (uint32_t)((int64_t)S_b * p.vc_ss));
  __amdgpu_buffer_rsrc_t srs[4] = {krs, krs, krs, krs};
  if constexpr (!C::DENSE) {
    const int64_t ko = (int64_t)b * p.ksb_sb + (int64_t)kvh * p.ksb_sh;
    const int64_t vo = (int64_t)b * p.vsb_sb + (int64_t)kvh * p.vsb_sh;
    const uint32_t kn = (uint32_t)((int64_t)S_b * p.ksb_ss * 2), vn = (uint32_t)((int64_t)S_b * p.vsb_ss * 2);
    srs[0] = make_rsrc(p.ks + ko, kn);
    srs[1] = make_rsrc(p.kb + ko, kn);
    srs[2] = make_rsrc(p.vs + vo, vn);
    srs[3] = make_rsrc(p.vb + vo, vn);
  }
  // lane offsets: code lane l fills 16-byte cell l of each KiB, i.e. row l / CPR and -- for K,
  // swizzled -- chunk (l % CPR) ^ kswz(row); scale/bias lane l reads group l / 32 of key l % 32
  // (for NG == 1 the upper half re-reads the lower half's keys)
  uint32_t dk[C::CI], dv[C::CI], dsb[4][C::NSB];
  {
    const int rr = lane / C::CPR, cc = lane % C::CPR;
#pragma unroll
    for (int c = 0; c < C::CI; ++c) {
      const int kr = c * C::RPI + rr;
      dk[c] = (uint32_t)((int64_t)kr * p.kc_ss + 16 * (cc ^ C::kswz(kr)));
      dv[c] = (uint32_t)((int64_t)(c * C::RPI + rr) * p.vc_ss + 16 * cc);
    }
#pragma unroll
    for (int h = 0; h < C::NSB; ++h) {
      // DMA h of an array fills cells 64 h + lane: group 2 h + lane / 32 of key lane % 32
      const int sk = lane & 31, sg = C::NG >= 2 ? 2 * h + (lane >> 5) : 0;
      dsb[0][h] = dsb[1][h] = C::DENSE ? 0u : (uint32_t)(sk * p.ksb_ss * 2 + 2 * sg);
      dsb[2][h] = dsb[3][h] = C::DENSE ? 0u : (uint32_t)(sk * p.vsb_ss * 2 + 2 * sg);
    }
  }
  uint8_t* const ring = smem + wave * (NSLOT * C::SLOT);
  auto tile_k0 = [&](int i) { return k_begin + kTile * (wave + NW * i); };
  // tile i of this wave -> slot `slot`; past the wave's last tile it re-reads that tile, so the
  // number of loads in flight behind any tile is always (NSLOT - 1) * IPT
  const int last = max(nmine - 1, 0);
  // paged cache: a tile (32 rows, 32-aligned) lies in one 64-row page; its page number is read one
  // tile ahead (a scalar load that the ring's waits cover), clamped to the pool, and the tile's
  // buffer resources span only that page's valid rows, so rows past S_b still read as zero
  auto page_of = [&](int k0) -> int {
    const int pi = min(k0, max(S_b - 1, 0)) >> 6;
    return __builtin_amdgcn_readfirstlane(min(max(p.table[(int64_t)b * p.table_stride + pi], 0), p.num_pages - 1));
  };
  int pg_next = PAGED ? page_of(tile_k0(0)) : 0;
  auto issue = [&](int i, int slot) {
    const int k0 = tile_k0(min(i, last));
    uint8_t* sl = ring + slot * C::SLOT;
    __amdgpu_buffer_rsrc_t kr = krs, vr = vrs, sr[4] = {srs[0], srs[1], srs[2], srs[3]};
    int rk0 = k0;  // the tile's first row within the buffer resources
    if constexpr (PAGED) {
      const int pg = pg_next;
      pg_next = page_of(tile_k0(min(i + 1, last)));
      const int nv = __builtin_amdgcn_readfirstlane(max(min(64, S_b - (k0 & ~63)), 0));  // keeps the rsrc in SGPRs
      kr = make_rsrc(p.kc + (int64_t)pg * p.kc_sb + (int64_t)kvh * p.kc_sh, (uint32_t)(nv * p.kc_ss));
      vr = make_rsrc(p.vc + (int64_t)pg * p.vc_sb + (int64_t)kvh * p.vc_sh, (uint32_t)(nv * p.vc_ss));
      if constexpr (!C::DENSE) {
        const int64_t ko = (int64_t)pg * p.ksb_sb + (int64_t)kvh * p.ksb_sh;
        const int64_t vo = (int64_t)pg * p.vsb_sb + (int64_t)kvh * p.vsb_sh;
        const uint32_t kn = (uint32_t)(nv * p.ksb_ss * 2), vn = (uint32_t)(nv * p.vsb_ss * 2);
        sr[0] = make_rsrc(p.ks + ko, kn);
        sr[1] = make_rsrc(p.kb + ko, kn);
        sr[2] = make_rsrc(p.vs + vo, vn);
        sr[3] = make_rsrc(p.vb + vo, vn);
      }
      rk0 = k0 & 63;
    }
    const uint32_t ko = (uint32_t)((int64_t)rk0 * p.kc_ss), vo = (uint32_t)((int64_t)rk0 * p.vc_ss);
#pragma unroll
    for (int c = 0; c < C::CI; ++c) dma16(kr, sl + 1024 * c, dk[c], ko);
#pragma unroll
    for (int c = 0; c < C::CI; ++c) dma16(vr, sl + C::TB + 1024 * c, dv[c], vo);
    if constexpr (!C::DENSE) {
      const uint32_t kso = (uint32_t)((int64_t)rk0 * p.ksb_ss * 2), vso = (uint32_t)((int64_t)rk0 * p.vsb_ss * 2);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int h = 0; h < C::NSB; ++h) dma2(sr[a], sl + 2 * C::TB + C::AS * a + 256 * h, dsb[a][h], a < 2 ? kso : vso);
    }
  };
  // nothing that waits for the query loads may be scheduled into (or before) the first tile loads
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < NSLOT; ++j) issue(j, j);
  __builtin_amdgcn_sched_barrier(0);

  const int qpos = S_b - p.L + lq;
  const int lo_r = p.window > 0 ? max(0, qpos - p.window + 1) : 0;
  const int hi_r = p.causal ? min(S_b, qpos + 1) : S_b;
  const int lo_all = p.window > 0 ? max(0, S_b - p.window) : 0;
  const int hi_all = p.causal ? S_b - p.L + 1 : S_b;

  // ---- Q operand. Unquantized cache: the raw query slice itself (exact), the scale applied to the
  // fp32 scores. Quantized cache:
  h8 qop[C::KSTEPS];
  u4 qd[C::KSTEPS];
  float kf, qs2 = 0.0f;
  if constexpr (C::DENSE) {
    (void)in_group;
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j) qd[j] = row_ok ? qraw[j] : u4{0, 0, 0, 0};
    kf = p.scale_log2;
  } else {
    // slot i of k-step j is q[row][lg*D/4 + 8j + dim(i)] if that dim is in group g
    float qv[C::KSTEPS][8];
    float qmax = 0.0f, qsum = 0.0f;
    const bool q_on = row_ok && in_group;
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j) {
      if (!q_on) qraw[j] = u4{0, 0, 0, 0};
      float e[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[2 * i] = to_float((uint16_t)(qraw[j][i] & 0xffffu), T{});
        e[2 * i + 1] = to_float((uint16_t)(qraw[j][i] >> 16), T{});
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qv[j][i] = e[k_slot_dim<BITS>(i)];
        qmax = fmaxf(qmax, fabsf(qv[j][i]));
        qsum += qv[j][i];
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
#pragma unroll
    for (int j = 0; j < C::KSTEPS; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qop[j][i] = (_Float16)(qv[j][i] * qscale * k_slot_weight<BITS>(i));
    }
    // score = sK * (acc * kf) + bK * qs2, then summed over the NG groups of the row
    kf = ldexpf(1.0f, 24 - qexp) * p.scale_log2;
    qs2 = qsum * p.scale_log2;
  }

  float m_run = -INFINITY, l_part = 0.0f, ob_part = 0.0f;
  f4 acc_o[C::NBLK];
#pragma unroll
  for (int jn = 0; jn < C::NBLK; ++jn) acc_o[jn] = f4{0, 0, 0, 0};

  // per-lane LDS offsets of the tile operands, relative to a slot
  const int sw = C::kswz(n);  // the swizzle of key n (and of key 16 + n)
  // K: chunk c of the lane's quarter row of key n (KLB / 16 chunks; below 16 bytes a half chunk)
  uint32_t off_k[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if constexpr (C::KLB >= 16) {
      off_k[c] = n * C::ROWB + 16 * (((C::KLB / 16) * lg + min(c, C::KLB / 16 - 1)) ^ sw);
    } else {
      off_k[c] = n * C::ROWB + 16 * ((lg >> 1) ^ sw) + 8 * (lg & 1);
    }
  }
  const uint32_t off_sb = 2 * C::TB + 4 * (32 * g + 4 * lg);
  const uint32_t off_v = C::TB + 4 * lg * C::ROWB + n * C::VLB;
  // unquantized cache: chunk c of the lane's D/4 dims of key n sits at position (KCH lg + c) ^ sw
  constexpr int KCH = C::DENSE ? C::KLB / 16 : 1;
  uint32_t off_kd[KCH];
#pragma unroll
  for (int c = 0; c < KCH; ++c) off_kd[c] = n * C::ROWB + 16 * ((KCH * lg + c) ^ sw);

  auto compute = [&](const auto& op, int k0) {
    auto sbv = [&](int a, int beta, int i) -> float {
      if constexpr (C::DENSE) {
        return 0.0f;
      } else {
        return to_float((uint16_t)(op.sb[a][beta][i] & 0xffffu), T{});
      }
    };
    float sc[8];
    if constexpr (C::DENSE) {
      // S^T = K Q^T on the raw 16-bit rows: rows = 16 keys of block beta, columns = query rows
#pragma unroll
      for (int beta = 0; beta < 2; ++beta) {
        f4 sacc = f4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < C::KSTEPS; ++j) sacc = mfma_16x16x32(op.k[beta][j], qd[j], sacc, T{});
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[4 * beta + i] = sacc[i] * kf;
      }
    } else {
      // S^T = K Q^T: rows = 16 keys of block beta, columns = (query row, group)
      f4 sacc[2];
#pragma unroll
      for (int beta = 0; beta < 2; ++beta) {
        Bytes<C::KLB> kc;
        if constexpr (C::KLB == 64) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int w = 0; w < 4; ++w) kc.w[4 * c + w] = op.k[beta][c][w];
        } else if constexpr (C::KLB == 32) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            kc.w[w] = op.k[beta][0][w];
            kc.w[4 + w] = op.k[beta][1][w];
          }
        } else if constexpr (C::KLB == 16) {
#pragma unroll
          for (int w = 0; w < 4; ++w) kc.w[w] = op.k[beta][w];
        } else {
          kc.w[0] = op.k[beta][0];
          kc.w[1] = op.k[beta][1];
        }
        sacc[beta] = f4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < C::KSTEPS; ++j)
          sacc[beta] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k_operand<D, BITS>(kc, j), qop[j], sacc[beta], 0, 0, 0);
      }
#pragma unroll
      for (int beta = 0; beta < 2; ++beta)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = sbv(0, beta, i) * (sacc[beta][i] * kf) + sbv(1, beta, i) * qs2;
          if constexpr (C::NG >= 2) x += row_rotate<8>(x);
          if constexpr (C::NG >= 4) x += row_rotate<4>(x);
          sc[4 * beta + i] = x;
        }
    }
    const bool need_mask = MASKED || !(k0 >= lo_all && k0 + kTile <= hi_all);
    if (need_mask) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int t = k0 + 16 * (s >> 2) + 4 * lg + (s & 3);
        if (!(t >= lo_r && t < hi_r)) sc[s] = -INFINITY;
      }
      if constexpr (MASKED) {
        if (row_ok) apply_mask(p, b, kvh, hq - kvh * p.rep, lq, k0, lg, lo_r, hi_r, sc);
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
    if constexpr (C::DENSE) {
      // P' (A operand) in the cache's type; the row sum adds the rounded probabilities, so the
      // output stays a convex combination of V rows whatever the rounding
      float pr[8];
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) pr[s2] = exp2_fast(sc[s2] - msub);
      u4 aw;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        if constexpr (T::id == KVQ_DTYPE_BF16) {
          aw[a] = pack_bf16x2(pr[2 * a], pr[2 * a + 1]);
        } else {
          aw[a] = pack_f16x2(pr[2 * a], pr[2 * a + 1]);
        }
        l_part += pr[2 * a] + pr[2 * a + 1];
      }
#pragma unroll
      for (int jn = 0; jn < C::NBLK; ++jn) acc_o[jn] = mfma_16x16x32(aw, v_operand_dense(op.v, jn), acc_o[jn], T{});
    } else {
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
      // V codes of the lane's column slice at its 8 keys
      constexpr int VB = C::VLB < 2 ? 2 : C::VLB;
      Bytes<VB> vc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (C::VLB == 16) {
#pragma unroll
          for (int w = 0; w < 4; ++w) vc[i].w[w] = op.v[i][w];
        } else if constexpr (C::VLB == 8) {
          vc[i].w[0] = op.v[i][0];
          vc[i].w[1] = op.v[i][1];
        } else {
          vc[i].w[0] = op.v[i];
        }
      }
#pragma unroll
      for (int jn = 0; jn < C::NBLK; ++jn)
        acc_o[jn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, v_operand<D, BITS, VB>(vc, jn), acc_o[jn], 0, 0, 0);
    }
  };

  // ---- main loop: tile i is read out of its slot, the slot is refilled with tile i + NSLOT, and
  // tile i is computed while NSLOT tiles stream
  const uint32_t ring_lds = lds_addr(ring);
  for (int i = 0; i < nmine; ++i) {
    const int slot = i % NSLOT;
    wait_vmcnt<(NSLOT - 1) * C::IPT>();  // tile i has landed
    const uint32_t sa = ring_lds + slot * C::SLOT;
    if constexpr (C::DENSE) {
      DenseOps<D> op;
      uint32_t ka[KCH];
#pragma unroll
      for (int c = 0; c < KCH; ++c) ka[c] = sa + off_kd[c];
      read_tile_dense(op, ka, sa + off_v);
      issue(i + NSLOT, slot);
      compute(op, tile_k0(i));
    } else {
      TileOps<C::ROWB> op;
      const uint32_t ka[4] = {sa + off_k[0], sa + off_k[1], sa + off_k[2], sa + off_k[3]};
      read_tile<C::AS>(op, ka, sa + off_sb, sa + off_v);
      issue(i + NSLOT, slot);
      compute(op, tile_k0(i));
    }
  }
  wait_vmcnt<0>();  // the look-ahead loads past the last tile land before the ring is reused
  __syncthreads();  // every wave is done with its ring: the space is reused below

  float* const w_m = (float*)smem;     // [NW][R]
  float* const w_l = w_m + NW * R;     // [NW][R]
  float* const w_o = w_l + NW * R;     // [NW][R][D]
  float* const s_w = w_o + NW * R * D;  // [R][kMaxSplit]
  // ---- wave epilogue: sums over the 4 lane groups, then stage (m, l, o) in LDS
  l_part = add_xor32(add_xor16(l_part));
  ob_part = add_xor32(add_xor16(ob_part));
  float obi[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) obi[i] = shfl(ob_part, 4 * lg + i);
  if (lg == 0 && n < R) {
    w_m[wave * R + n] = m_run;
    w_l[wave * R + n] = l_part;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * lg + i;
    if (m / R == n / R) {
#pragma unroll
      for (int jn = 0; jn < C::NBLK; ++jn) {
        // codes entered the MFMA as fp16 subnormals c 2^-24; at 4 bits an odd block holds the sums
        // over lo + 16 hi of its byte, so the hi nibbles' sum is (odd - even) / 16
        float x = C::DENSE ? acc_o[jn][i] : acc_o[jn][i] * 16777216.0f;
        if constexpr (BITS == 4) {
          if (jn & 1) x = (acc_o[jn][i] - acc_o[jn - 1][i]) * 1048576.0f;
        }
        w_o[(wave * R + m % R) * D + (D / 16) * n + jn] = x + obi[i];
      }
    }
  }
  __syncthreads();

  // ---- merge the waves: this workgroup's (m, l, o) per row, NPT float4s of o per thread; a single
  // split writes the output, otherwise the partial goes to the workspace split-major:
  // o at ((unit * nsplit + split) * R + row) * D, (m, l) at the same index in pairs
  constexpr int NV = R * D / 4;
  constexpr int NPT = (NV + NT - 1) / NT;
  static_assert(NV % NT == 0 || NV < NT, "whole float4s of a partial per thread");
  const bool single = p.nsplit == 1;
  struct Slot {
    int i4, rr, d0;
    bool mine;
    uint16_t* orow;
  };
  auto slot_of = [&](int it) {
    Slot s;
    s.i4 = threadIdx.x + it * NT;
    s.rr = (4 * s.i4) / D;
    s.d0 = (4 * s.i4) % D;
    const int rw = rb * R + s.rr;
    s.mine = s.i4 < NV && rw < p.nrows && (!NARROW || s.d0 < dims);
    const int rq = (int)div31((uint32_t)rw, p.d_l);
    const int hh = kvh * p.rep + rq, ll = rw - rq * p.L;
    s.orow = p.out + (int64_t)b * p.o_sb + (int64_t)hh * p.o_sh + (int64_t)ll * p.o_sl + s.d0;
    return s;
  };
  auto write_out = [&](const Slot& s, f4 o, float inv) {
#pragma unroll
    for (int e = 0; e < 4; ++e) s.orow[e] = from_float(o[e] * inv, T{});
  };
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.part_o + (int64_t)unit * p.nsplit * (R * D), (uint32_t)(p.nsplit * R * D * 4));
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(p.part_ml + (int64_t)unit * p.nsplit * (2 * R), (uint32_t)(p.nsplit * R * 8));
#pragma unroll
  for (int it = 0; it < NPT; ++it) {
    const Slot sl = slot_of(it);
    if (sl.i4 >= NV) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, w_m[w * R + sl.rr]);
    f4 o = {0, 0, 0, 0};
    float lsum = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = w_m[w * R + sl.rr];
        if (mw != -INFINITY) {
          const float f = exp2_fast(mw - M);
          o += f * *(const f4*)&w_o[(w * R + sl.rr) * D + sl.d0];
          lsum += f * w_l[w * R + sl.rr];
        }
      }
    }
    if (single) {
      if (sl.mine) write_out(sl, o, lsum > 0.0f ? 1.0f / lsum : 0.0f);
    } else if (p.fused) {
      store_agent_b128(ro, 16 * sl.i4 + split * (R * D * 4), o);
      if (sl.d0 == 0) store_agent_b64(rm, 8 * sl.rr + split * (R * 8), make_float2(M, lsum));
    } else {
      const int64_t pi = ((int64_t)unit * p.nsplit + split) * R + sl.rr;
      *(f4*)(p.part_o + pi * D + sl.d0) = o;
      if (sl.d0 == 0) ((float2*)p.part_ml)[pi] = make_float2(M, lsum);
    }
  }
  if (single || !p.fused) return;

  // ---- the last workgroup of this unit to finish merges the splits. The partials were written
  // with agent-scope (sc1) stores; once they are acknowledged (s_waitcnt) the counter increment is
  // ordered after them at the device's coherence point, and the merging workgroup reads them with
  // agent-scope loads. No device-scope fence is needed (on gfx950 one writes back the XCD's L2).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_prev = __hip_atomic_fetch_add(&p.counters[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_prev != (unsigned)(p.nsplit - 1)) return;
  if (threadIdx.x == 0) __hip_atomic_store(&p.counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  if (NPT > 1 || p.nsplit <= kFewSplits) {
    // few splits (the plan's choice for this form, and the only one with several float4s per
    // thread): each thread loads its float4 and its row's (m, l) of every split in one round (loads
    // past the last split re-read it and count with l = 0) and forms the weights itself: no wave
    // reductions, no exchange through LDS
    const int last = p.nsplit - 1;
#pragma unroll
    for (int it = 0; it < NPT; ++it) {
      const Slot sl = slot_of(it);
      if (!sl.mine) continue;
      f4 po[kFewSplits];
      float2 mv[kFewSplits];
#pragma unroll
      for (int u = 0; u < kFewSplits; ++u) {
        const int su = min(u, last);
        po[u] = load_agent_b128(ro, 16 * sl.i4, su * (R * D * 4));
        mv[u] = load_agent_b64(rm, 8 * sl.rr, su * (R * 8));
      }
      float Mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < kFewSplits; ++u)
        if (u <= last && mv[u].y > 0.0f) Mx = fmaxf(Mx, mv[u].x);
      f4 acc = {0, 0, 0, 0};
      float Ls = 0.0f;
#pragma unroll
      for (int u = 0; u < kFewSplits; ++u) {
        const float w = (u <= last && mv[u].y > 0.0f) ? exp2_fast(mv[u].x - Mx) : 0.0f;
        acc += w * po[u];
        Ls += w * mv[u].y;
      }
      write_out(sl, acc, Ls > 0.0f ? 1.0f / Ls : 0.0f);
    }
    return;
  }
  if constexpr (NPT == 1) {
    const Slot sl = slot_of(0);
    const int i4 = sl.i4;
    // this thread's float4 of the first 32 splits, in flight while the weights are formed
    constexpr int CH = 32;
    f4 po[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u)
      po[u] = (i4 < NV && u < p.nsplit) ? load_agent_b128(ro, 16 * i4, u * (R * D * 4)) : f4{0, 0, 0, 0};
    // weights w_s / sum_s w_s l_s per row: one wave per row, lane = split
    for (int r2 = wave; r2 < R; r2 += NW) {
      float2 v0 = make_float2(-INFINITY, 0.0f), v1 = v0;
      if (lane < p.nsplit) v0 = load_agent_b64(rm, 8 * r2, lane * (R * 8));
      if (lane + 64 < p.nsplit) v1 = load_agent_b64(rm, 8 * r2, (lane + 64) * (R * 8));
      const float m0 = v0.y > 0.0f ? v0.x : -INFINITY, m1 = v1.y > 0.0f ? v1.x : -INFINITY;
      const float Mx = wave_max(fmaxf(m0, m1));
      const float w0 = (Mx == -INFINITY || m0 == -INFINITY) ? 0.0f : exp2_fast(m0 - Mx);
      const float w1 = (Mx == -INFINITY || m1 == -INFINITY) ? 0.0f : exp2_fast(m1 - Mx);
      const float Lsum = wave_sum(w0 * v0.y + w1 * v1.y);
      const float inv = Lsum > 0.0f ? 1.0f / Lsum : 0.0f;
      if (lane < p.nsplit) s_w[r2 * kMaxSplit + lane] = w0 * inv;
      if (lane + 64 < p.nsplit) s_w[r2 * kMaxSplit + lane + 64] = w1 * inv;
    }
    __syncthreads();
    if (!sl.mine) return;
    const float* wrow = s_w + sl.rr * kMaxSplit;
    f4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < CH; ++u)
      if (u < p.nsplit) acc += wrow[u] * po[u];
    for (int s0 = CH; s0 < p.nsplit; s0 += CH) {
#pragma unroll
      for (int u = 0; u < CH; ++u)
        po[u] = s0 + u < p.nsplit ? load_agent_b128(ro, 16 * i4, (s0 + u) * (R * D * 4)) : f4{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < CH; ++u)
        if (s0 + u < p.nsplit) acc += wrow[s0 + u] * po[u];
    }
    write_out(sl, acc, 1.0f);
  }
}

// ------------------------------------------------------------------------------------------
// Host side: plan, workspace, launch.

struct DecPlan {
  int R, rowblocks, chunk, nsplit, span, nunits, nw, nslot, fused;
};

struct DecTune {
  int nw, nslot, target_wgs, fused;
};

// The in-kernel split merge (the last split of a unit merges) costs an arrival counter and a
// round trip per split partial in one workgroup; the combine launch costs a kernel boundary. With
// few splits the in-kernel merge is faster (3-4 splits: C5 window layer 12.5 against 13.3 us, C2 at
// batch 8 and C5's global layer about 1% faster), with many it is slower (17 splits: C1 12.6 against
// 11.4 us; 32: C2 at batch 1 24.2 against 21.7 us).
constexpr int kFusedMaxSplit = kFewSplits;

// Launch-shape defaults; KVQ_DECODE_TUNE="waves,slots,workgroups[,fused]" overrides them (read
// once per process; fused 0 or 1 forces the split merge's form, omitted leaves it to the plan).
// 8-wave workgroups take 2 ring slots (the ring of 3 would not fit in LDS).
static DecTune decode_tune() {
  static DecTune t = [] {
    DecTune d{4, 2, 256, -1};
    if (const char* e = getenv("KVQ_DECODE_TUNE")) {
      int a = 0, b = 0, c = 0, f = -1;
      if (sscanf(e, "%d,%d,%d,%d", &a, &b, &c, &f) >= 3 && (a == 4 || (a == 8 && b == 2)) && b >= 2 && b <= 4 && c >= 1)
        d = {a, b, c, f < 0 ? -1 : f != 0};
    }
    return d;
  }();
  return t;
}

DecPlan decode_plan(int B, int Hq, int Hkv, int L, int D, int S, int window, int bits, int G) {
  DecPlan pl;
  const DecTune tune = decode_tune();
  const bool dense = bits == 16;
  if (dense) G = 64;  // the unquantized kernels keep the column layout of group 64
  const bool tuned = D == 128 && !dense && G == 64;  // the launch shapes built for other than 4 waves x 2 slots
  pl.nw = tuned ? tune.nw : 4;
  pl.nslot = tuned ? tune.nslot : 2;
  pl.R = 16 / (D / G);
  const int nrows = (Hq / Hkv) * L;
  pl.rowblocks = (nrows + pl.R - 1) / pl.R;
  pl.span = window > 0 ? std::min(S, window + L - 1 + kTile - 1) : S;  // the window, from a tile boundary
  const int64_t tiles_seq = (pl.span + kTile - 1) / kTile;
  pl.nunits = B * Hkv * pl.rowblocks;
  int64_t tpw = (pl.nunits * tiles_seq + tune.target_wgs - 1) / tune.target_wgs;
  tpw = std::max<int64_t>(tpw, (tiles_seq + kMaxSplit - 1) / kMaxSplit);
  tpw = std::max<int64_t>(pl.nw, (tpw + pl.nw - 1) / pl.nw * pl.nw);
  pl.chunk = (int)(tpw * kTile);
  pl.nsplit = (pl.span + pl.chunk - 1) / pl.chunk;
  const bool fused = tune.fused < 0 ? pl.nsplit <= kFusedMaxSplit : tune.fused != 0;
  // (with 16 query rows of 128 dims a thread owns two float4s of a partial; the in-kernel merge
  // then handles at most kFewSplits splits)
  const bool few_only = pl.R * D / 4 > 4 * 64;
  pl.fused = fused && pl.nunits <= kMaxCountedUnits && (!few_only || pl.nsplit <= kFewSplits);
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

int decode_kernel_dim(int D) { return D <= 64 ? 64 : D <= 128 ? 128 : 256; }

size_t decode_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S, int window, int bits, int G) {
  const int Dk = decode_kernel_dim(D);
  const DecPlan pl = decode_plan(B, Hq, Hkv, L, Dk, S, window, bits, G);
  return decode_layout(pl, Dk).total;
}

// Whether kernel width D with scale group G serves narrower rows: head dims that run at width D
// (decode_kernel_dim) and are multiples of G, i.e. 32 dims at width 64 (G 32), 96 at 128 (G 32) and
// 192 at 256 (G 64); unquantized rows (G stands at 64) of any multiple of 8 at width 64 or 128.
template <int D, int BITS, int G>
constexpr bool narrow_rows() {
  if constexpr (BITS == 16) return D <= 128;
  const int lo = D == 64 ? 0 : D / 2;  // the widths below D end here
  return (lo / G + 1) * G < D;
}

template <typename T, int D, int BITS, int NW, int NSLOT, bool PAGED = false, int G = 64>
static hipError_t launch_decode_t(const DecParams& p, hipStream_t stream) {
  if (p.dv != D) {
    // rows narrower than the kernel (decode_kernel_dim): the default launch shape, plain, paged or
    // masked
    if constexpr (NW == 4 && NSLOT == 2 && narrow_rows<D, BITS, G>()) {
      if (p.mask_kind != 0) {
        if constexpr (!PAGED) {
          hipLaunchKernelGGL((decode_attn_kernel<T, D, BITS, NW, NSLOT, PAGED, G, true, true>),
                             dim3(p.nunits * p.nsplit), dim3(NW * 64), 0, stream, p);
        } else {
          return hipErrorInvalidValue;
        }
      } else {
        hipLaunchKernelGGL((decode_attn_kernel<T, D, BITS, NW, NSLOT, PAGED, G, false, true>), dim3(p.nunits * p.nsplit),
                           dim3(NW * 64), 0, stream, p);
      }
    } else {
      return hipErrorInvalidValue;
    }
  } else if (p.mask_kind != 0) {
    if constexpr (NW == 4 && NSLOT == 2 && !PAGED) {
      hipLaunchKernelGGL((decode_attn_kernel<T, D, BITS, NW, NSLOT, PAGED, G, true>), dim3(p.nunits * p.nsplit),
                         dim3(NW * 64), 0, stream, p);
    } else {
      return hipErrorInvalidValue;  // masked calls always take the default launch shape
    }
  } else {
    hipLaunchKernelGGL((decode_attn_kernel<T, D, BITS, NW, NSLOT, PAGED, G>), dim3(p.nunits * p.nsplit), dim3(NW * 64),
                       0, stream, p);
  }
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
  m.R = DecCfg<D, BITS, G>::R;
  m.rowblocks = p.rowblocks;
  m.nsplit = p.nsplit;
  m.xcd_remap = p.xcd_remap;
  return launch_combine<T, D>(m, p.nunits / (p.Hkv * p.rowblocks), stream, p.dv);
}

template <typename T, int D, int BITS, int G = 64>
static hipError_t launch_decode_shape(const DecParams& p, const DecPlan& pl, hipStream_t stream) {
  if (p.mask_kind != 0 || p.dv != D) return launch_decode_t<T, D, BITS, 4, 2, false, G>(p, stream);
  if constexpr (BITS == 16) {
    return launch_decode_t<T, D, BITS, 4, 2>(p, stream);  // a 3-slot ring of raw rows does not fit
  } else if constexpr (G != 64) {
    return launch_decode_t<T, D, BITS, 4, 2, false, G>(p, stream);
  } else if constexpr (D == 128) {
    if (pl.nw == 8) return launch_decode_t<T, D, BITS, 8, 2>(p, stream);
    if (pl.nslot == 2) return launch_decode_t<T, D, BITS, 4, 2>(p, stream);
    if (pl.nslot == 3) return launch_decode_t<T, D, BITS, 4, 3>(p, stream);
    return launch_decode_t<T, D, BITS, 4, 4>(p, stream);
  } else {
    return launch_decode_t<T, D, BITS, 4, 2>(p, stream);
  }
}

// Everything but the K/V operands.
static DecParams decode_params(const kvq_rows* q, const int32_t* seq_lens, const kvq_rows* out, int Hq, int Hkv,
                               int L, int D, int S, float scale, int causal, int window, void* workspace,
                               const DecPlan& pl) {
  const DecLayout lay = decode_layout(pl, D);
  DecParams p{};
  p.q = (const uint16_t*)q->data;
  p.q_sb = q->stride_b;
  p.q_sh = q->stride_h;
  p.q_sl = q->stride_l;
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
  p.dv = D;
  p.d_nsplit = make_div31((uint32_t)pl.nsplit);
  p.d_rowblocks = make_div31((uint32_t)pl.rowblocks);
  p.d_hkv = make_div31((uint32_t)Hkv);
  p.d_l = make_div31((uint32_t)L);
  return p;
}

// Calls f(T{}, D, BITS, G) (the last three as std::integral_constant) for the quantized
// instantiation that matches the runtime arguments: D in {64, 128, 256}, bits in {4, 8}, G in {32,
// 64, 128} with D / 4 <= G <= D.
template <int N>
using IC = std::integral_constant<int, N>;
template <typename F>
static hipError_t dispatch_quant(int dtype, int D, int bits, int G, F&& f) {
  auto by_g = [&](auto t, auto d, auto b) -> hipError_t {
    constexpr int DD = decltype(d)::value;
    if constexpr (DD / 4 <= 32) {
      if (G == 32) return f(t, d, b, IC<32>{});
    }
    if constexpr (DD >= 128) {
      if (G == 128) return f(t, d, b, IC<128>{});
    }
    return f(t, d, b, IC<64>{});
  };
  auto by_b = [&](auto t, auto d) -> hipError_t { return bits == 8 ? by_g(t, d, IC<8>{}) : by_g(t, d, IC<4>{}); };
  auto by_d = [&](auto t) -> hipError_t {
    if (D == 256) return by_b(t, IC<256>{});
    return D == 128 ? by_b(t, IC<128>{}) : by_b(t, IC<64>{});
  };
  return dtype == KVQ_DTYPE_BF16 ? by_d(BF16{}) : by_d(F16{});
}

static void set_mask(DecParams& p, const kvq_mask* mask) {
  if (!mask) return;
  p.mask = mask->data;
  p.mask_kind = mask->kind;
  p.m_sb = mask->stride_b;
  p.m_skv = mask->stride_kvh;
  p.m_srep = mask->stride_rep;
  p.m_sl = mask->stride_l;
}

hipError_t launch_decode(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, const int32_t* seq_lens,
                         const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype,
                         float scale, int causal, int window, void* workspace, hipStream_t stream, const kvq_mask* mask) {
  const int Dk = decode_kernel_dim(D);
  const DecPlan pl = decode_plan(B, Hq, Hkv, L, Dk, S, window, bits, G);
  DecParams p = decode_params(q, seq_lens, out, Hq, Hkv, L, Dk, S, scale, causal, window, workspace, pl);
  p.dv = D;
  set_mask(p, mask);
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
  return dispatch_quant(dtype, Dk, bits, G, [&](auto t, auto d, auto b, auto g) {
    return launch_decode_shape<decltype(t), decltype(d)::value, decltype(b)::value, decltype(g)::value>(p, pl, stream);
  });
}

hipError_t launch_decode_paged(const kvq_rows* q, const kvq_qtensor* k, const kvq_qtensor* v, int num_pages,
                               const int32_t* table, int64_t table_stride, const int32_t* seq_lens, const kvq_rows* out,
                               int B, int Hq, int Hkv, int L, int D, int S, int bits, int G, int dtype, float scale,
                               int causal, int window, void* workspace, hipStream_t stream) {
  const int Dk = decode_kernel_dim(D);
  const DecPlan pl = decode_plan(B, Hq, Hkv, L, Dk, S, window, bits, G);
  DecParams p = decode_params(q, seq_lens, out, Hq, Hkv, L, Dk, S, scale, causal, window, workspace, pl);
  p.dv = D;
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
  p.table = table;
  p.table_stride = table_stride;
  p.num_pages = num_pages;
  return dispatch_quant(dtype, Dk, bits, G, [&](auto t, auto d, auto b, auto g) {
    return launch_decode_t<decltype(t), decltype(d)::value, decltype(b)::value, 4, 2, true, decltype(g)::value>(p, stream);
  });
}

hipError_t launch_decode_dense(const kvq_rows* q, const kvq_rows* k, const kvq_rows* v, const int32_t* seq_lens,
                               const kvq_rows* out, int B, int Hq, int Hkv, int L, int D, int S, int dtype, float scale,
                               int causal, int window, void* workspace, hipStream_t stream, const kvq_mask* mask) {
  const int Dk = decode_kernel_dim(D);
  const DecPlan pl = decode_plan(B, Hq, Hkv, L, Dk, S, window, 16, 64);
  DecParams p = decode_params(q, seq_lens, out, Hq, Hkv, L, Dk, S, scale, causal, window, workspace, pl);
  p.dv = D;
  set_mask(p, mask);
  p.kc = (const uint8_t*)k->data;
  p.vc = (const uint8_t*)v->data;
  p.kc_sb = k->stride_b * 2;
  p.kc_sh = k->stride_h * 2;
  p.kc_ss = k->stride_l * 2;
  p.vc_sb = v->stride_b * 2;
  p.vc_sh = v->stride_h * 2;
  p.vc_ss = v->stride_l * 2;
  const bool bf = dtype == KVQ_DTYPE_BF16;
  if (Dk == 256) return hipErrorInvalidValue;  // unquantized rows past 128 dims run through the head_dim-256 kernel
  if (Dk == 128) return bf ? launch_decode_shape<BF16, 128, 16>(p, pl, stream) : launch_decode_shape<F16, 128, 16>(p, pl, stream);
  return bf ? launch_decode_shape<BF16, 64, 16>(p, pl, stream) : launch_decode_shape<F16, 64, 16>(p, pl, stream);
}

}  // namespace kvq
