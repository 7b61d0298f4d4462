// Paged GQA decode attention for gfx950 (replaces flash_attn_with_kvcache at
// nanovllm/layers/attention.py:75-77).
//
// Work item = (sequence b, kv head, split).  One 64-lane wavefront owns a work
// item and every query head of the kv head's group (up to 16), so each K/V byte
// of the split is read from HBM exactly once.  The split's keys are visited 32
// at a time:
//
//   S^T (32 keys x 16 heads) = K (32 x 128) . Q^T (128 x 16)   two key tiles x
//                                                              four 16x16x32 MFMAs
//   O^T (128 x 16 heads)    += V^T (128 x 32) . P^T (32 x 16)  eight MFMAs
//
// Lane l (n = l % 16, g = l / 16) supplies K row n of each key tile and query
// head n; the tile rows are ordered so that the S^T accumulator of lane l holds
// head n's scores for keys 8g .. 8g+7 of the step -- exactly the P^T operand
// layout of the PV MFMA, so softmax probabilities never leave the lane.  The V
// operand needs 8 keys of one column per lane: the lane loads 8 value rows
// (16 B each, columns 8n .. 8n+7) and transposes them with v_perm_b32.
// The O^T accumulator of lane l then holds head n, columns 32g .. 32g+31.
//
// Online softmax runs in the exp2 domain per head; the row max is shared by the
// four lanes of a head through two xor shuffles.  With more than one split per
// sequence each wave writes (unnormalised O, max, sum) and decode_merge_kernel
// combines the splits with a log-sum-exp merge.  The split count depends only
// on host-side sizes, so the launch is graph-capture safe.
#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

// Contraction index (head-dim position) of element e of lane group g in MFMA s.
// Any bijection works as long as K and Q use the same one; these make each lane
// load contiguous 16-byte pieces.
template <bool FP8>
__device__ __forceinline__ int qk_dim(int s, int g) {
  return FP8 ? (64 * (s >> 1) + 16 * g + 8 * (s & 1)) : (32 * s + 8 * g);
}

// Transpose 8 bf16 value rows (row i: 8 columns) into the 8 V^T MFMA operands
// (operand j: column j of rows 0..7).
__device__ __forceinline__ void transpose_v_bf16(const u32x4 (&vr)[8], bf16x8 (&vt)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    u32x4 o;
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) o[pp] = perm(vr[2 * pp + 1][j >> 1], vr[2 * pp][j >> 1], sel);
    vt[j] = as_bf16x8(o);
  }
}

// Same for 8 fp8 value rows (row i: 8 e4m3fn bytes), converting to bf16.
__device__ __forceinline__ void transpose_v_fp8(const u32x2 (&vr)[8], bf16x8 (&vt)[8]) {
  u32x4 o[8];
#pragma unroll
  for (int jp = 0; jp < 4; ++jp) {  // column pair (2jp, 2jp+1)
    const int w = jp >> 1;
    const uint32_t sel = (jp & 1) ? 0x07030602u : 0x05010400u;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const uint32_t x = perm(vr[2 * pp + 1][w], vr[2 * pp][w], sel);
      o[2 * jp][pp] = fp8x2_to_bf16x2<false>(x);
      o[2 * jp + 1][pp] = fp8x2_to_bf16x2<true>(x);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) vt[j] = as_bf16x8(o[j]);
}

// 16 fp8 -> two 8 x bf16 MFMA operands.
__device__ __forceinline__ void fp8x16_to_ops(u32x4 w, bf16x8& lo, bf16x8& hi) {
  u32x4 a, b;
  a[0] = fp8x2_to_bf16x2<false>(w[0]);
  a[1] = fp8x2_to_bf16x2<true>(w[0]);
  a[2] = fp8x2_to_bf16x2<false>(w[1]);
  a[3] = fp8x2_to_bf16x2<true>(w[1]);
  b[0] = fp8x2_to_bf16x2<false>(w[2]);
  b[1] = fp8x2_to_bf16x2<true>(w[2]);
  b[2] = fp8x2_to_bf16x2<false>(w[3]);
  b[3] = fp8x2_to_bf16x2<true>(w[3]);
  lo = as_bf16x8(a);
  hi = as_bf16x8(b);
}

}  // namespace

template <bool FP8>
__global__ __launch_bounds__(64) void paged_decode_kernel(DecodeParams p) {
  constexpr int EB = FP8 ? 1 : 2;  // bytes per cache element
  const int lane = threadIdx.x;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int G = p.group;
  const int h = kvh * G + n;
  const bool head_ok = n < G;
  const bool direct = p.num_splits == 1;

  int ctx = p.seqlens[b];
  const int cap = p.max_blocks * p.block_size;
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int k_begin = split * p.keys_per_split;
  const int k_end = min(ctx, k_begin + p.keys_per_split);
  if (k_begin >= k_end) {
    if (direct && head_ok) {
      uint16_t* orow = p.out + b * p.out_row_stride + h * kHeadDim + 32 * g;
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < 4; ++r) st16(orow + 8 * r, z);
    }
    return;
  }

  // Q^T operand: head n, 8 contraction elements per MFMA.
  bf16x8 qop[4];
  {
    const uint16_t* qrow = p.q + b * p.q_row_stride + h * kHeadDim;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[s] = as_bf16x8(head_ok ? ld16(qrow + qk_dim<FP8>(s, g)) : z);
    }
  }

  const int64_t slot_bytes = static_cast<int64_t>(p.num_kv_heads) * kHeadDim * EB;
  const char* kbase = static_cast<const char*>(p.k_cache) + static_cast<int64_t>(kvh) * kHeadDim * EB;
  const char* vbase = static_cast<const char*>(p.v_cache) + static_cast<int64_t>(kvh) * kHeadDim * EB;
  const int32_t* bt = p.block_table + b * p.bt_row_stride;
  const float sl2 = FP8 ? p.scale_log2 * p.k_scale[kvh] : p.scale_log2;

  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;
  float l_run = 0.f;

  // K tile row n of tile t holds key 8*(n/4) + 4*t + (n%4) of the step.
  const int krow0 = 8 * (n >> 2) + (n & 3);
  const int bs = p.block_size;

  for (int blk = k_begin / bs; blk * bs < k_end; ++blk) {
    const int page = bt[blk];
    if (page < 0 || page >= p.num_blocks) continue;  // inconsistent table: keys stay masked
    const int kp_end = min(k_end, (blk + 1) * bs);
    for (int key0 = blk * bs; key0 < kp_end; key0 += 32) {
      const int64_t row0 = static_cast<int64_t>(page) * bs + (key0 - blk * bs);
      const int nvalid = kp_end - key0;  // keys of this step that exist (may exceed 32)

      // ---- loads ---------------------------------------------------------
      bf16x8 kop[2][4];
      bf16x8 vt[8];
      if constexpr (!FP8) {
        u32x4 kr[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const char* rp = kbase + (row0 + krow0 + 4 * t) * slot_bytes;
#pragma unroll
          for (int s = 0; s < 4; ++s) kr[t][s] = ld16(rp + qk_dim<false>(s, g) * 2);
        }
        u32x4 vr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) vr[i] = ld16(vbase + (row0 + 8 * g + i) * slot_bytes + 16 * n);
        if (nvalid < 32) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (8 * g + i >= nvalid) vr[i] = u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int s = 0; s < 4; ++s) kop[t][s] = as_bf16x8(kr[t][s]);
        transpose_v_bf16(vr, vt);
      } else {
        u32x4 kr[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const char* rp = kbase + (row0 + krow0 + 4 * t) * slot_bytes;
#pragma unroll
          for (int u = 0; u < 2; ++u) kr[t][u] = ld16(rp + 64 * u + 16 * g);
        }
        u32x2 vr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) vr[i] = ld8(vbase + (row0 + 8 * g + i) * slot_bytes + 8 * n);
        if (nvalid < 32) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (8 * g + i >= nvalid) vr[i] = u32x2{0u, 0u};
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          fp8x16_to_ops(kr[t][0], kop[t][0], kop[t][1]);
          fp8x16_to_ops(kr[t][1], kop[t][2], kop[t][3]);
        }
        transpose_v_fp8(vr, vt);
      }

      // ---- scores ----------------------------------------------------------
      f32x4 st[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) st[t] = mfma16x16x32(kop[t][s], qop[s], st[t]);
      }
      float sv[8];
      float mx = kNegInf;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = st[i >> 2][i & 3] * sl2;
        sv[i] = (8 * g + i < nvalid) ? x : kNegInf;
        mx = fmaxf(mx, sv[i]);
      }
      mx = fmaxf(mx, shfl_xor(mx, 16));
      mx = fmaxf(mx, shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);  // finite: key0 itself is valid
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
      float pv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pv[i] = fast_exp2(sv[i] - m_new);
        psum += pv[i];
      }
      l_run = l_run * alpha + psum;
      u32x4 pw;
#pragma unroll
      for (int w = 0; w < 4; ++w) pw[w] = pack_bf16x2(pv[2 * w], pv[2 * w + 1]);
      const bf16x8 pop = as_bf16x8(pw);

      // ---- O^T += V^T . P^T ---------------------------------------------
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc[j] *= alpha;
        acc[j] = mfma16x16x32(vt[j], pop, acc[j]);
      }
    }
  }

  float l = l_run;
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
  const float vscale = FP8 ? p.v_scale[kvh] : 1.0f;
  if (!head_ok) return;
  if (direct) {
    const float inv = l > 0.f ? vscale / l : 0.f;
    uint16_t* orow = p.out + b * p.out_row_stride + h * kHeadDim + 32 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) o[w] = pack_bf16x2(acc[2 * w][r] * inv, acc[2 * w + 1][r] * inv);
      st16(orow + 8 * r, o);
    }
  } else {
    const int64_t idx = (static_cast<int64_t>(b) * p.num_heads + h) * p.num_splits + split;
    float* wo = p.ws_o + idx * kHeadDim + 32 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f32x4 lo, hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = acc[j][r] * vscale;
        hi[j] = acc[4 + j][r] * vscale;
      }
      *reinterpret_cast<f32x4*>(wo + 8 * r) = lo;
      *reinterpret_cast<f32x4*>(wo + 8 * r + 4) = hi;
    }
    if (g == 0) {
      f32x2 ml = {m_run, l};
      *reinterpret_cast<f32x2*>(p.ws_ml + idx * 2) = ml;
    }
  }
}

// Log-sum-exp merge of the split partials: one wavefront per (sequence, head),
// two output columns per lane.
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeParams p) {
  const int bh = blockIdx.x;
  const int b = bh / p.num_heads;
  const int lane = threadIdx.x;
  int ctx = p.seqlens[b];
  const int cap = p.max_blocks * p.block_size;
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  const int nvalid = (ctx + p.keys_per_split - 1) / p.keys_per_split;
  const float* ml = p.ws_ml + static_cast<int64_t>(bh) * p.num_splits * 2;
  const float* wo = p.ws_o + static_cast<int64_t>(bh) * p.num_splits * kHeadDim + 2 * lane;
  float M = kNegInf;
  for (int s = 0; s < nvalid; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.f, o0 = 0.f, o1 = 0.f;
  if (M != kNegInf) {
    for (int s = 0; s < nvalid; ++s) {
      const float w = fast_exp2(ml[2 * s] - M);
      L += w * ml[2 * s + 1];
      const f32x2 v = *reinterpret_cast<const f32x2*>(wo + static_cast<int64_t>(s) * kHeadDim);
      o0 += w * v[0];
      o1 += w * v[1];
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const int h = bh - b * p.num_heads;
  uint32_t* orow = reinterpret_cast<uint32_t*>(p.out + b * p.out_row_stride + h * kHeadDim + 2 * lane);
  *orow = pack_bf16x2(o0 * inv, o1 * inv);
}

DecodePlan plan_decode(int32_t batch, int32_t num_kv_heads, int32_t max_blocks, int32_t block_size,
                       int32_t kv_dtype, int32_t requested_splits) {
  (void)block_size;
  (void)kv_dtype;
  DecodePlan plan;
  int32_t pps = 1;
  if (requested_splits > 0) {
    pps = (max_blocks + requested_splits - 1) / requested_splits;
  } else {
    // Widest split that still leaves >= 8192 work items (about 32 per CU):
    // fewer partials to merge without starving the 256 CUs.
    const int64_t pairs = static_cast<int64_t>(batch) * num_kv_heads;
    while (pps < max_blocks) {
      const int64_t next = 2 * pps;
      const int64_t items = pairs * ((max_blocks + next - 1) / next);
      if (items < 8192) break;
      pps = static_cast<int32_t>(next);
    }
  }
  if (pps < 1) pps = 1;
  if (pps > max_blocks) pps = max_blocks > 0 ? max_blocks : 1;
  plan.pages_per_split = pps;
  plan.num_splits = max_blocks > 0 ? (max_blocks + pps - 1) / pps : 1;
  return plan;
}

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, hipStream_t stream) {
  if (p.batch <= 0) return hipSuccess;
  const dim3 grid(p.num_splits, p.num_kv_heads, p.batch);
  if (kv_dtype == 1)
    hipLaunchKernelGGL(paged_decode_kernel<true>, grid, dim3(64), 0, stream, p);
  else
    hipLaunchKernelGGL(paged_decode_kernel<false>, grid, dim3(64), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.num_splits == 1) return e;
  const dim3 mgrid(static_cast<unsigned>(p.batch * p.num_heads));
  hipLaunchKernelGGL(decode_merge_kernel, mgrid, dim3(64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nva
