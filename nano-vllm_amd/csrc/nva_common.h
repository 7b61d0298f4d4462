// Shared device helpers for the gfx950 attention kernels.
//
// Element storage: bf16 values travel as raw 16-bit words (uint16_t) and fp8
// values as raw bytes (OCP e4m3fn, the format gfx950 converts natively).
// MFMA operands are 8 x bf16 vectors; accumulators are 4 x f32 vectors.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nva {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) { return __builtin_bit_cast(u32x4, v); }

// D = A(16x32) * B(32x16) + C.  Lane l supplies A row (l % 16) and B column
// (l % 16), each with 8 contraction elements owned by lane group (l / 16).
// Lane l receives C rows 4*(l/16) + r, r = 0..3, of column (l % 16).
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// D = A(32x16) * B(16x32) + C.  Lane l supplies A row (l % 32) and B column
// (l % 32) with 8 contraction elements owned by lane half (l / 32); lane l
// receives C rows 8*(i/4) + 4*(l/32) + i%4, i = 0..15, of column (l % 32).
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_permlane32_swap: swaps the upper 32 lanes of `a` with the lower 32 lanes
// of `b`, so with a = b = x the pair holds x[l & 31] and x[l | 32], i.e. lanes
// l and l^32 in some order.  Inline asm because this compiler's builtin loses
// the second result (the optimiser replaces it by the first).  The s_nop
// gives the wait states a VALU write of an operand needs before the swap.
__device__ __forceinline__ void permlane32_swap(uint32_t& a, uint32_t& b) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// Max / sum over lanes l and l^32 (the two halves holding one 32x32 MFMA column).
__device__ __forceinline__ float max_across_halves(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane32_swap(a, b);
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

__device__ __forceinline__ float sum_across_halves(float v) {
  uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
  permlane32_swap(a, b);
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// 16-byte and 8-byte global loads / stores through plain vector memory ops.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// The same loads with the non-temporal hint (`nt`): for data a kernel streams
// once, such as the cache rows of a decode step, so they do not displace data
// that is reused (decode at config 5: 548.7 -> 514.3 us).
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld8_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
// Cache-policy operand of the buffer-load builtins: the non-temporal bit.
constexpr int kBufNonTemporal = 2;

// Round-to-nearest-even f32 -> bf16 pair packed in one dword (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// f32 -> OCP e4m3fn with round-to-nearest-even on the grid extended by 480
// (the NaN code 0x7f): magnitudes above 464, the midpoint of 448 and 480, and
// infinities and NaNs map to NaN (0x7f) with the input's sign bit; exactly 464
// ties to even (448).
//  - |x| < 2^-6 (the subnormal range): adding 2^14 rounds |x| to a multiple of
//    2^-9, the subnormal step, and the low mantissa bits of the sum are the code.
//  - otherwise: round the 23-bit mantissa to 3 bits (ties to even) and rebias
//    the exponent from 127 to 7.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
  uint32_t bits = __builtin_bit_cast(uint32_t, x);
  const uint32_t sign = (bits >> 24) & 0x80u;
  bits &= 0x7fffffffu;
  uint32_t code;
  if (bits > 0x43e80000u) {  // > 464.0f, inf or NaN
    code = 0x7fu;
  } else if (bits < 0x3c800000u) {  // < 2^-6
    const float y = __builtin_bit_cast(float, bits) + 16384.0f;
    code = __builtin_bit_cast(uint32_t, y) - 0x46800000u;
  } else {
    const uint32_t odd = (bits >> 20) & 1u;
    bits += 0x7ffffu + odd;
    code = (bits >> 20) - (120u << 3);
  }
  return code | sign;
}

// Eight bf16 values (16 bytes, element e in bits 16 (e % 2) of word e / 2)
// divided by `scale`, as eight e4m3fn codes (8 bytes, code e in byte e).
__device__ __forceinline__ u32x2 bf16x8_to_e4m3fn(u32x4 w, float scale) {
  u32x2 out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t word = w[2 * h + (e >> 1)];
      const uint32_t b16 = (e & 1) ? (word >> 16) : (word & 0xffffu);
      packed |= f32_to_e4m3fn(bf16_bits_to_f32(b16) / scale) << (8 * e);
    }
    out[h] = packed;
  }
  return out;
}

// Two e4m3fn bytes (selected 16-bit half of `w`) -> two bf16 in one dword.
// The conversion is exact: every e4m3fn value is representable in bf16.
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  bf16x2 v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane xor shuffle within the 64-lane wavefront.
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  int lane = __lane_id();
  int src = lane ^ mask;
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src << 2, __builtin_bit_cast(int, v)));
}

// v_perm_b32: selector byte k picks byte (sel_k) of the 8-byte value {hi:a, lo:b}.
__device__ __forceinline__ uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
  return __builtin_amdgcn_perm(a, b, sel);
}

}  // namespace nva
