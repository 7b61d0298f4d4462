// Fused per-head RMSNorm + rotary embedding of q and k, the producer step just
// before attention in Qwen3Attention.forward (qwen3.py:91-105):
//   q = RMSNorm(q per head) * q_norm.weight      layernorm.py:17-27 (rms_forward)
//   k = RMSNorm(k per head) * k_norm.weight
//   q, k = rotary_emb(positions, q, k)           rotary_embedding.py:6-17, 37-55
// With no norm weights it is the rotary embedding alone (Qwen2, qwen2.py:91-92).
//
// One (token, head) row per 16 lanes, 4 rows per wavefront.  Lane j of a row
// holds E = D/32 consecutive elements of each half of the head dimension,
// [E j, E j + E) and [D/2 + E j, ...), so the rotation pairs (i, i + D/2) are
// lane-local and only the sum of squares crosses lanes (4 xor shuffles).
//
// Arithmetic follows the reference's eager op sequence, rounding where it
// rounds: fp32 x, mean of squares, x * rsqrt(mean + eps) rounded to bf16, times
// the bf16 weight rounded to bf16; then fp32 x1*cos - x2*sin and x2*cos + x1*sin
// with every product and sum rounded separately (no FMA contraction), rounded
// to bf16.  The sum of squares runs in this kernel's order (a lane's squares,
// then a 16-lane butterfly), which can move the mean by an fp32 ulp against
// torch's reduction and so, rarely, an output by one bf16 ulp.  Memory-bound:
// each row is read once and written once; the cos/sin row of a token is shared
// by its heads through the caches.
#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

namespace {

template <int E>
struct Half;
template <>
struct Half<4> {  // head_dim 128: 4 bf16 = 8 bytes per half
  typedef u32x2 T;
  __device__ static T load(const uint16_t* p) { return ld8(p); }
  __device__ static void store(uint16_t* p, T v) { *reinterpret_cast<u32x2*>(p) = v; }
  __device__ static uint32_t word(const T& v, int i) { return v[i]; }
  __device__ static void set(T& v, int i, uint32_t w) { v[i] = w; }
};
template <>
struct Half<2> {  // head_dim 64: 2 bf16 = 4 bytes per half
  typedef uint32_t T;
  __device__ static T load(const uint16_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
  __device__ static void store(uint16_t* p, T v) { *reinterpret_cast<uint32_t*>(p) = v; }
  __device__ static uint32_t word(const T& v, int) { return v; }
  __device__ static void set(T& v, int, uint32_t w) { v = w; }
};

__device__ __forceinline__ float bf16_round(float x) {
  return bf16_bits_to_f32(pack_bf16x2(x, 0.f) & 0xffffu);
}

__device__ __forceinline__ float sum16(float v) {
  // xor butterflies within each 16-lane row group
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 16);
  return v;
}

}  // namespace

template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QKNormRopeParams p) {
  // every product and sum rounds on its own, as the reference's separate ops do:
  // no FMA contraction anywhere in this function
#pragma clang fp contract(off)
  constexpr int E = D / 32;
  using H = Half<E>;
  const int lane = threadIdx.x & 63;
  const int j = lane & 15;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  const int heads = p.num_heads + p.num_kv_heads;
  const bool valid = row < p.num_tokens * heads;  // no early return: the shuffles need the whole group
  const int64_t t = valid ? row / heads : 0;
  const int hh = valid ? static_cast<int>(row - t * heads) : 0;
  const bool is_q = hh < p.num_heads;
  const uint16_t* src = is_q ? p.q + t * p.q_row_stride + hh * D
                             : p.k + t * p.k_row_stride + (hh - p.num_heads) * D;
  uint16_t* dst = is_q ? p.q_out + t * p.q_out_row_stride + hh * D
                       : p.k_out + t * p.k_out_row_stride + (hh - p.num_heads) * D;

  typename H::T lo = H::load(src + E * j), hi = H::load(src + D / 2 + E * j);
  float x1[E], x2[E];
#pragma unroll
  for (int w = 0; w < E / 2; ++w) {
    x1[2 * w] = bf16_bits_to_f32(H::word(lo, w) & 0xffffu);
    x1[2 * w + 1] = bf16_bits_to_f32(H::word(lo, w) >> 16);
    x2[2 * w] = bf16_bits_to_f32(H::word(hi, w) & 0xffffu);
    x2[2 * w + 1] = bf16_bits_to_f32(H::word(hi, w) >> 16);
  }

  if (p.q_weight) {  // RMSNorm over the head dimension (uniform branch)
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) ss = (ss + x1[e] * x1[e]) + x2[e] * x2[e];
    ss = sum16(ss);
    const float r = rsqrtf(ss / static_cast<float>(D) + p.eps);
    const uint16_t* wt = is_q ? p.q_weight : p.k_weight;
    typename H::T wl = H::load(wt + E * j), wh = H::load(wt + D / 2 + E * j);
#pragma unroll
    for (int w = 0; w < E / 2; ++w) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const float w1 = bf16_bits_to_f32(b ? H::word(wl, w) >> 16 : H::word(wl, w) & 0xffffu);
        const float w2 = bf16_bits_to_f32(b ? H::word(wh, w) >> 16 : H::word(wh, w) & 0xffffu);
        x1[2 * w + b] = bf16_round(bf16_round(x1[2 * w + b] * r) * w1);
        x2[2 * w + b] = bf16_round(bf16_round(x2[2 * w + b] * r) * w2);
      }
    }
  }

  // rotary embedding: cache row = [cos(D/2) | sin(D/2)] of the clamped position
  int64_t pos = valid ? p.positions[t] : 0;
  pos = pos < 0 ? 0 : (pos >= p.max_position ? p.max_position - 1 : pos);
  const float* cs = p.cos_sin + pos * D;
  float c[E], s[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    c[e] = cs[E * j + e];
    s[e] = cs[D / 2 + E * j + e];
  }
  typename H::T o1, o2;
#pragma unroll
  for (int w = 0; w < E / 2; ++w) {
    float y1[2], y2[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int e = 2 * w + b;
      y1[b] = x1[e] * c[e] - x2[e] * s[e];
      y2[b] = x2[e] * c[e] + x1[e] * s[e];
    }
    H::set(o1, w, pack_bf16x2(y1[0], y1[1]));
    H::set(o2, w, pack_bf16x2(y2[0], y2[1]));
  }
  if (valid) {
    H::store(dst + E * j, o1);
    H::store(dst + D / 2 + E * j, o2);
  }
}

hipError_t launch_qk_norm_rope(const QKNormRopeParams& p, hipStream_t stream) {
  const int64_t rows = p.num_tokens * (p.num_heads + p.num_kv_heads);
  if (rows <= 0) return hipSuccess;
  const int64_t blocks = (rows + 15) / 16;  // 4 wavefronts x 4 rows
  if (p.head_dim == 128)
    hipLaunchKernelGGL(qk_norm_rope_kernel<128>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<64>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nva
