// Shared device helpers for the gfx950 kernels of libkvq.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvq.h"

namespace kvq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// Element-type tags. Raw storage is always a 16-bit pattern.
struct F16 {
  static constexpr int id = KVQ_DTYPE_F16;
};
struct BF16 {
  static constexpr int id = KVQ_DTYPE_BF16;
};

__device__ __forceinline__ float to_float(uint16_t r, F16) {
  return (float)__builtin_bit_cast(_Float16, r);
}
__device__ __forceinline__ float to_float(uint16_t r, BF16) {
  return __uint_as_float((uint32_t)r << 16);
}
// float -> 16-bit pattern, round to nearest even (the hardware default mode for f16).
__device__ __forceinline__ uint16_t from_float(float f, F16) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint16_t from_float(float f, BF16) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Two f16 values packed in a u32 (low half first), rounded to nearest even.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  h2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

// Two bf16 values packed in a u32 (low half first), rounded to nearest even; lo and hi are
// replaced by the rounded values (callers keep sums consistent with the operands they pack).
__device__ __forceinline__ uint32_t pack_bf16x2(float& lo, float& hi) {
  const bf2 v = {(__bf16)lo, (__bf16)hi};
  lo = (float)v[0];
  hi = (float)v[1];
  return __builtin_bit_cast(uint32_t, v);
}

// Two values packed as the operand type (f16 or bf16 by the element tag), rounded to nearest even.
__device__ __forceinline__ uint32_t pack2(float lo, float hi, F16) { return pack_f16x2(lo, hi); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi, BF16) { return pack_bf16x2(lo, hi); }

// acc + lo + hi of two packed 16-bit values (one dot-product instruction against (1, 1)): sums the
// rounded probabilities exactly as the MFMA consumes them.
__device__ __forceinline__ float add_pair(uint32_t packed, float acc, F16) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, packed), h2{(_Float16)1.0f, (_Float16)1.0f}, acc, false);
}
__device__ __forceinline__ float add_pair(uint32_t packed, float acc, BF16) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, packed), bf2{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
}

// MFMA on 16-bit operands given as raw bit patterns, f16 or bf16 by the element tag.
__device__ __forceinline__ f4 mfma_16x16x32(u4 a, u4 b, f4 c, F16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_16x16x32(u4 a, u4 b, f4 c, BF16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f16v mfma_32x32x16(u4 a, u4 b, f16v c, F16) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f16v mfma_32x32x16(u4 a, u4 b, f16v c, BF16) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane helpers (wave64).
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  const int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}
__device__ __forceinline__ float shfl(float v, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}
// Reductions between lane i and lane i ^ 32 (or i ^ 16) with the gfx950 VALU permlane swaps:
// with both operands equal, each lane ends up holding its own value and its partner's, so a
// symmetric combine of the pair is the butterfly step without a trip through the LDS unit.
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Rotate within each row of 16 lanes: lane c receives lane (c + n) % 16 of its row.
template <int N>
__device__ __forceinline__ float row_rotate(float v) {
  static_assert(N > 0 && N < 16, "rotation within a DPP row");
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + (16 - N) % 16, 0xF, 0xF, false));
}

// Byte selection: bytes 0..3 come from `lo`, 4..7 from `hi`; selector byte 0x0C yields 0.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit data format, no
// swizzle). Loads through it take a 32-bit lane offset plus a wave-uniform offset, and read 0
// outside the range instead of faulting.
// n / d for 0 <= n < 2^31 as one multiply and shift: with l = ceil(log2 d) and
// m = ceil(2^(31 + l) / d) (which fits 32 bits), floor(n m / 2^(31 + l)) = floor(n / d)
// (Granlund and Montgomery, "Division by invariant integers using multiplication", 1994, for
// 31-bit dividends: the error n (m - 2^(31 + l) / d) / 2^(31 + l) stays below 1 / d). The host
// builds the pair for a launch's divisors; a runtime division on the device is a long sequence.
struct Div31 {
  uint32_t m;
  uint32_t sh;  // 31 + l
};
inline Div31 make_div31(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  return {(uint32_t)((((uint64_t)1 << (31 + l)) + d - 1) / d), 31 + l};
}
__device__ __forceinline__ uint32_t div31(uint32_t n, Div31 q) { return (uint32_t)(((uint64_t)n * q.m) >> q.sh); }

// A read-only int32 at a wave-uniform index, read through the constant address space so that it is
// one scalar load: a plain load of caller memory is a vector load (the compiler cannot rule out
// that the kernel writes it), whose whole round trip the first address computations would wait
// for. Used for the per-sequence lengths, which no kernel writes.
__device__ __forceinline__ int load_uniform_i32(const int32_t* p, int i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Device-coherent vector accesses through a buffer resource, for data one workgroup publishes and
// a workgroup on another XCD reads in the same launch: cache policy sc1 is the agent-scope form of
// the gfx94x/gfx950 memory model (stores write through the XCD's L2, loads do not hit a stale copy
// in it), the same bits an agent-scope atomic store or load carries.
constexpr int kCpolAgent = 16;  // sc1
__device__ __forceinline__ void store_agent_b128(__amdgpu_buffer_rsrc_t r, uint32_t vo, f4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, v), r, vo, 0, kCpolAgent);
}
__device__ __forceinline__ void store_agent_b64(__amdgpu_buffer_rsrc_t r, uint32_t vo, float2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, v), r, vo, 0, kCpolAgent);
}
__device__ __forceinline__ f4 load_agent_b128(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, kCpolAgent));
}
__device__ __forceinline__ float2 load_agent_b64(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, kCpolAgent));
}

// NBYTES consecutive bytes held as 32-bit words; load() from a generic pointer, load_buf() through
// a buffer resource (lane offset `vo`, uniform offset `so`).
template <int NBYTES>
struct Bytes;
template <>
struct Bytes<2> {
  uint32_t w[1];
  __device__ __forceinline__ void load(const uint8_t* p) { w[0] = *(const uint16_t*)p; }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0);
  }
};
template <>
struct Bytes<4> {
  uint32_t w[1];
  __device__ __forceinline__ void load(const uint8_t* p) { w[0] = *(const uint32_t*)p; }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
  }
};
template <>
struct Bytes<8> {
  uint32_t w[2];
  __device__ __forceinline__ void load(const uint8_t* p) {
    u2 v = *(const u2*)p;
    w[0] = v[0];
    w[1] = v[1];
  }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0);
    w[0] = v[0];
    w[1] = v[1];
  }
};
template <>
struct Bytes<16> {
  uint32_t w[4];
  __device__ __forceinline__ void load(const uint8_t* p) {
    u4 v = *(const u4*)p;
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  }
};
template <>
struct Bytes<32> {
  uint32_t w[8];
  __device__ __forceinline__ void load(const uint8_t* p) {
    u4 a = *(const u4*)p;
    u4 b = *(const u4*)(p + 16);
    w[0] = a[0];
    w[1] = a[1];
    w[2] = a[2];
    w[3] = a[3];
    w[4] = b[0];
    w[5] = b[1];
    w[6] = b[2];
    w[7] = b[3];
  }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    u4 a = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
    u4 b = __builtin_amdgcn_raw_buffer_load_b128(r, vo + 16, so, 0);
    w[0] = a[0];
    w[1] = a[1];
    w[2] = a[2];
    w[3] = a[3];
    w[4] = b[0];
    w[5] = b[1];
    w[6] = b[2];
    w[7] = b[3];
  }
};
template <>
struct Bytes<64> {
  uint32_t w[16];
  __device__ __forceinline__ void load(const uint8_t* p) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u4 v = *(const u4*)(p + 16 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[4 * c + i] = v[i];
    }
  }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, vo + 16 * c, so, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[4 * c + i] = v[i];
    }
  }
};

}  // namespace kvq

// Host-side launch plumbing shared by the C-ABI layer.
namespace kvq_host {
struct Status {
  int code;
  const char* msg;
};
void set_error(const char* fmt, ...);
}  // namespace kvq_host
