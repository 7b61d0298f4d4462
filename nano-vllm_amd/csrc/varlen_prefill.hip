// Varlen causal prefill attention for gfx950 (replaces flash_attn_varlen_func at
// nanovllm/layers/attention.py:67-73), with K/V either packed by cu_seqlens_k
// or gathered from the paged cache through block_table (prefix-cache case,
// cu_seqlens_k > cu_seqlens_q, bottom-right causal alignment).
//
// Workgroup = 4 wavefronts = 128 query rows of one (sequence, query head); each
// wave owns 32 rows (two 16-row MFMA column tiles).  Keys are visited in 64-key
// tiles staged in LDS by the whole workgroup:
//   sK  [64 keys][128 dims]   16-byte chunks XOR-swizzled by key row
//   sVt [128 dims][64 keys]   transposed while staging (v_perm), swizzled
// Per 32-key step a wave computes S^T = K . Q^T (keys x rows) with 16x16x32 bf16
// MFMAs.  Key tile rows are ordered so that the S^T accumulator of lane l holds
// query row (l % 16)'s scores for keys 8*(l/16) .. +7 -- the P^T operand layout
// of O^T += V^T . P^T -- so probabilities stay in registers.  Softmax runs
// online in the exp2 domain, one running (max, sum) per lane and row.
#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

namespace {

constexpr int kRowsPerWave = 32;
constexpr int kWaves = 4;
constexpr int kBQ = kRowsPerWave * kWaves;  // query rows per workgroup
constexpr int kBK = 64;                     // keys per LDS tile
constexpr float kNegInf = -__builtin_huge_valf();

// Swizzle of the 16-byte chunk index inside a K row: the 16 rows one MFMA
// operand read touches map to 16 distinct bank groups.
__device__ __forceinline__ int k_swz(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
// Same for the transposed V rows (8 chunks of 8 keys per 128-byte row).
__device__ __forceinline__ int vt_swz(int r) { return (r >> 1) & 7; }

}  // namespace

template <bool PAGED>
__global__ __launch_bounds__(256) void varlen_prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[kBK * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[kHeadDim * kBK];

  const int tile = p.num_q_tiles - 1 - static_cast<int>(blockIdx.x);  // heavy tiles first
  const int h = blockIdx.y;
  const int s = blockIdx.z;
  const int q_start = p.cu_q[s];
  const int Lq = p.cu_q[s + 1] - q_start;
  const int k_start = p.cu_k[s];
  const int Lk = p.cu_k[s + 1] - k_start;
  const int i0 = tile * kBQ;
  if (i0 >= Lq) return;
  const int off = Lk - Lq;  // bottom-right causal offset
  const int kvh = h / p.group;

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int g = lane >> 4;

  // Q^T operands for this wave's two 16-row tiles.
  bf16x8 qop[2][4];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int pos = i0 + kRowsPerWave * w + 16 * nt + n;
    const uint16_t* qrow = p.q + static_cast<int64_t>(q_start + pos) * p.q_row_stride + h * kHeadDim;
#pragma unroll
    for (int sidx = 0; sidx < 4; ++sidx) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[nt][sidx] = as_bf16x8(pos < Lq ? ld16(qrow + 32 * sidx + 8 * g) : z);
    }
  }

  const int last_row = min(i0 + kBQ, Lq) - 1;
  const int kmax = min(Lk, last_row + off + 1);  // keys [0, kmax) are visible to some row
  const int wave_last = min(i0 + kRowsPerWave * w + kRowsPerWave, Lq) - 1;
  const int wave_kmax = min(kmax, wave_last + off + 1);

  f32x4 acc[2][8];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[nt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {kNegInf, kNegInf};
  float l_run[2] = {0.f, 0.f};
  const float sl2 = p.scale_log2;

  const int krow0 = 8 * (n >> 2) + (n & 3);
  const int32_t* bt = PAGED ? p.block_table + s * p.bt_row_stride : nullptr;
  const uint16_t* kbase = p.k + kvh * kHeadDim;
  const uint16_t* vbase = p.v + kvh * kHeadDim;

  for (int kb = 0; kb < kmax; kb += kBK) {
    // ---- stage the 64-key K and V^T tiles ---------------------------------
    int64_t slot0;  // cache / packed row of key kb
    bool tile_ok = true;
    if constexpr (PAGED) {
      const int bi = kb / p.block_size;
      const int page = bi < p.max_blocks ? bt[bi] : -1;
      tile_ok = page >= 0 && page < p.num_blocks;  // inconsistent table: the tile reads as zeros
      slot0 = static_cast<int64_t>(tile_ok ? page : 0) * p.block_size + (kb % p.block_size);
    } else {
      slot0 = static_cast<int64_t>(k_start) + kb;
    }
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 4;
      const int ch = c & 15;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (tile_ok && kb + row < kmax) v = ld16(kbase + (slot0 + row) * p.k_row_stride + ch * 8);
      *reinterpret_cast<u32x4*>(&sK[row * kHeadDim + ((ch ^ k_swz(row)) * 8)]) = v;
    }
    {
      const int kg = tid >> 4;  // keys 4kg .. 4kg+3
      const int cg = tid & 15;  // dims 8cg .. 8cg+7
      u32x4 vr[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = kb + 4 * kg + e;
        vr[e] = u32x4{0u, 0u, 0u, 0u};
        if (tile_ok && key < kmax) vr[e] = ld16(vbase + (slot0 + 4 * kg + e) * p.v_row_stride + cg * 8);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        u32x2 o;
        o[0] = perm(vr[1][j >> 1], vr[0][j >> 1], sel);
        o[1] = perm(vr[3][j >> 1], vr[2][j >> 1], sel);
        const int R = 16 * j + cg;
        const int kc = kg >> 1;
        *reinterpret_cast<u32x2*>(&sVt[R * kBK + ((kc ^ vt_swz(R)) * 8) + (kg & 1) * 4]) = o;
      }
    }
    __syncthreads();

    // ---- two 32-key steps ------------------------------------------------
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int key0 = kb + 32 * sub;
      if (key0 >= wave_kmax) break;  // every key of this step is masked for this wave
      bf16x8 kop[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 32 * sub + krow0 + 4 * t;
#pragma unroll
        for (int sidx = 0; sidx < 4; ++sidx) {
          const int ch = 4 * sidx + g;
          kop[t][sidx] = as_bf16x8(*reinterpret_cast<const u32x4*>(&sK[row * kHeadDim + ((ch ^ k_swz(row)) * 8)]));
        }
      }
      bf16x8 vt[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int R = 16 * j + n;
        const int kc = g + 4 * sub;
        vt[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(&sVt[R * kBK + ((kc ^ vt_swz(R)) * 8)]));
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        f32x4 st[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sidx = 0; sidx < 4; ++sidx) st[t] = mfma16x16x32(kop[t][sidx], qop[nt][sidx], st[t]);
        }
        const int pos = i0 + kRowsPerWave * w + 16 * nt + n;
        const int limit = min(pos + off, kmax - 1);  // last visible key of this row
        float sv[8];
        float mx = kNegInf;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int key = key0 + 8 * g + i;
          const float x = st[i >> 2][i & 3] * sl2;
          sv[i] = key <= limit ? x : kNegInf;
          mx = fmaxf(mx, sv[i]);
        }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run[nt], mx);
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const float alpha = fast_exp2(m_run[nt] - m_use);
        m_run[nt] = m_new;
        float psum = 0.f;
        float pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pv[i] = fast_exp2(sv[i] - m_use);
          psum += pv[i];
        }
        l_run[nt] = l_run[nt] * alpha + psum;
        u32x4 pw;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) pw[q2] = pack_bf16x2(pv[2 * q2], pv[2 * q2 + 1]);
        const bf16x8 pop = as_bf16x8(pw);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          acc[nt][j] *= alpha;
          acc[nt][j] = mfma16x16x32(vt[j], pop, acc[nt][j]);
        }
      }
    }
  }

  // ---- epilogue: normalise and write rows ------------------------------------
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float l = l_run[nt];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
    const int pos = i0 + kRowsPerWave * w + 16 * nt + n;
    if (pos >= Lq) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* orow = p.out + static_cast<int64_t>(q_start + pos) * p.out_row_stride + h * kHeadDim + 32 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 o;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2)
        o[q2] = pack_bf16x2(acc[nt][2 * q2][r] * inv, acc[nt][2 * q2 + 1][r] * inv);
      st16(orow + 8 * r, o);
    }
  }
}

hipError_t launch_prefill(const PrefillParams& p0, int max_seqlen_q, hipStream_t stream) {
  if (p0.num_seqs <= 0 || max_seqlen_q <= 0) return hipSuccess;
  PrefillParams p = p0;
  p.num_q_tiles = (max_seqlen_q + kBQ - 1) / kBQ;
  const dim3 grid(p.num_q_tiles, p.num_heads, p.num_seqs);
  if (p.block_table)
    hipLaunchKernelGGL(varlen_prefill_kernel<true>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(varlen_prefill_kernel<false>, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nva
