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
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;      // head_dim of every supported shape
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) { return __builtin_bit_cast(u32x4, v); }

// D = A(16x32) * B(32x16) + C.  Lane l supplies A row (l % 16) and B column
// (l % 16), each with 8 contraction elements owned by lane group (l / 16).
// Lane l receives C rows 4*(l/16) + r, r = 0..3, of column (l % 16).
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16-byte and 8-byte global loads / stores through plain vector memory ops.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Round-to-nearest-even f32 -> bf16 pair packed in one dword (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
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

// Max over lanes l, l^16, l^32, l^48 (the four lane groups holding one MFMA
// column) with gfx950 row swaps: called with the same value as both operands,
// v_permlane16_swap / v_permlane32_swap return {x[l], x[l^16]} /
// {x[l], x[l^32]} in some order, so combining the pair is order-free.
__device__ __forceinline__ float max_across_groups(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto r16 = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  v = fmaxf(__builtin_bit_cast(float, r16[0]), __builtin_bit_cast(float, r16[1]));
  const uint32_t c = __builtin_bit_cast(uint32_t, v);
  const auto r32 = __builtin_amdgcn_permlane32_swap(c, c, false, false);
  return fmaxf(__builtin_bit_cast(float, r32[0]), __builtin_bit_cast(float, r32[1]));
}

// v_perm_b32: selector byte k picks byte (sel_k) of the 8-byte value {hi:a, lo:b}.
__device__ __forceinline__ uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
  return __builtin_amdgcn_perm(a, b, sel);
}

}  // namespace nva
