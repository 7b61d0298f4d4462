// Varlen causal prefill attention for gfx950 (replaces flash_attn_varlen_func at
// nanovllm/layers/attention.py:67-73), with K/V either packed by cu_seqlens_k
// or gathered from the paged cache through block_table (prefix-cache case,
// cu_seqlens_k > cu_seqlens_q, bottom-right causal alignment).
//
// Workgroup = (sequence, kv head, query tile): 8 wavefronts x 32 rows, where a
// row is one (query position, query head) pair of the kv head's GQA group
// (rows are position-major: row r = position r / G, head r % G).  All G heads
// therefore share every K/V tile the workgroup stages.  Keys are visited in
// 64-key tiles, double-buffered in LDS:
//   sK  [64 keys][128 dims]   16-byte chunks XOR-swizzled by key row
//   sVt [128 dims][64 keys]   transposed while staging (v_perm), swizzled
// The next tile's global loads are issued before the current tile's math and
// written to the other buffer afterwards (one barrier per tile).
//
// Per 32-key step a wave computes S^T = K . Q^T (keys x rows) for its two
// 16-row column tiles with 16x16x32 bf16 MFMAs.  32 rows per wave keep Q, the
// O accumulators, the K/V operands and the staging registers within 256 VGPRs
// (two waves per SIMD, no accumulator traffic to AGPRs); gfx950's LDS read
// rate covers the K/V operand reads this costs.  Key tile rows are ordered so
// that the S^T accumulator of lane l holds row (l % 16)'s scores for keys
// 8*(l/16) .. +7 -- the P^T operand layout of O^T += V^T . P^T -- so the
// probabilities never leave the lane.  The row sums of the probabilities come
// from the matrix pipe as well (one extra MFMA against an all-ones operand per
// column tile), so they use the same bf16 weights as the numerator and cost no
// VALU adds.  Softmax runs online in the exp2 domain
// with a lazily updated row maximum: the maximum used for the exponent moves
// only when a new score exceeds it by more than kTau (so p <= 2^kTau), which
// makes the rescale of the 32 accumulator registers per tile rare.  Masks are
// evaluated only on tiles that cross the causal diagonal or the key end.
#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

namespace {

constexpr int kWaves = 8;
constexpr int kRowsPerWave = 32;
constexpr int kNT = kRowsPerWave / 16;      // MFMA column tiles per wave
constexpr int kRows = kWaves * kRowsPerWave;  // (position, head) rows per workgroup
constexpr int kBK = 64;                     // keys per LDS tile
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kTau = 8.0f;                // lazy-rescale threshold (log2 units)

// Swizzle of the 16-byte chunk index inside a K row: the 16 rows one MFMA
// operand read touches map to 16 distinct bank groups.
__device__ __forceinline__ int k_swz(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
// Same for the transposed V rows (8 chunks of 8 keys per 128-byte row).
__device__ __forceinline__ int vt_swz(int r) { return (r >> 1) & 7; }

// One 64-key tile of K and V held in registers between its global load and
// its LDS store: threads 0..255 carry four 16-byte K chunks each, threads
// 256..511 four V rows x 8 dims each (transposed on the way into LDS).
struct TileRegs {
  u32x4 r[4];
};

}  // namespace

template <bool PAGED>
__device__ __forceinline__ void load_tile(TileRegs& t, const PrefillParams& p, const uint16_t* kbase,
                                          const uint16_t* vbase, const int32_t* bt, int k_start, int kb,
                                          int kmax, int tid) {
  int64_t slot0;
  bool ok = true;
  if constexpr (PAGED) {
    const int bi = kb / p.block_size;
    const int page = bi < p.max_blocks ? bt[bi] : -1;
    ok = page >= 0 && page < p.num_blocks;  // inconsistent table: the tile reads as zeros
    slot0 = static_cast<int64_t>(ok ? page : 0) * p.block_size + (kb % p.block_size);
  } else {
    slot0 = static_cast<int64_t>(k_start) + kb;
  }
  if (tid < 256) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 4;
      const int ch = c & 15;
      t.r[u] = u32x4{0u, 0u, 0u, 0u};
      if (ok && kb + row < kmax) t.r[u] = ld16(kbase + (slot0 + row) * p.k_row_stride + ch * 8);
    }
  } else {
    const int kg = (tid - 256) >> 4;  // keys 4kg .. 4kg+3
    const int cg = tid & 15;          // dims 8cg .. 8cg+7
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t.r[e] = u32x4{0u, 0u, 0u, 0u};
      if (ok && kb + 4 * kg + e < kmax) t.r[e] = ld16(vbase + (slot0 + 4 * kg + e) * p.v_row_stride + cg * 8);
    }
  }
}

__device__ __forceinline__ void store_tile(const TileRegs& t, uint16_t* sK, uint16_t* sVt, int tid) {
  if (tid < 256) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = tid + 256 * u;
      const int row = c >> 4;
      const int ch = c & 15;
      *reinterpret_cast<u32x4*>(&sK[row * kHeadDim + ((ch ^ k_swz(row)) * 8)]) = t.r[u];
    }
  } else {
    const int kg = (tid - 256) >> 4;
    const int cg = tid & 15;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x2 o;
      o[0] = perm(t.r[1][j >> 1], t.r[0][j >> 1], sel);
      o[1] = perm(t.r[3][j >> 1], t.r[2][j >> 1], sel);
      const int R = 16 * j + cg;  // transposed row of dim 8cg + j
      const int kc = kg >> 1;
      *reinterpret_cast<u32x2*>(&sVt[R * kBK + ((kc ^ vt_swz(R)) * 8) + (kg & 1) * 4]) = o;
    }
  }
}

template <bool PAGED>
__global__ __launch_bounds__(64 * kWaves) void varlen_prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][kBK * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[2][kHeadDim * kBK];

  const int s = blockIdx.x / p.num_kv_heads;
  const int kvh = blockIdx.x - s * p.num_kv_heads;
  const int tile = p.num_q_tiles - 1 - static_cast<int>(blockIdx.y);  // heavy tiles first
  const int q_start = p.cu_q[s];
  const int Lq = p.cu_q[s + 1] - q_start;
  const int k_start = p.cu_k[s];
  const int Lk = p.cu_k[s + 1] - k_start;
  const int G = p.group;
  const int BP = p.positions_per_tile;  // query positions per workgroup (BP * G <= kRows)
  const int i0 = tile * BP;
  if (i0 >= Lq) return;
  const int off = Lk - Lq;  // bottom-right causal offset

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int nrows = BP * G;

  // rows of this lane: r = 64w + 16nt + n
  int pos[kNT];
  bf16x8 qop[kNT][4];
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    const int r = kRowsPerWave * w + 16 * nt + n;
    const int qp = i0 + r / G;
    const int h = kvh * G + r % G;
    const bool ok = r < nrows && qp < Lq;
    pos[nt] = ok ? qp : -1;
    const uint16_t* qrow = p.q + static_cast<int64_t>(q_start + qp) * p.q_row_stride + h * kHeadDim;
#pragma unroll
    for (int sidx = 0; sidx < 4; ++sidx) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[nt][sidx] = as_bf16x8(ok ? ld16(qrow + 32 * sidx + 8 * g) : z);
    }
  }

  const int last_pos = min(i0 + BP, Lq) - 1;
  const int kmax = max(0, min(Lk, last_pos + off + 1));  // keys [0, kmax) are visible to some row
  const int w_first = kRowsPerWave * w;
  const int w_last = min(kRowsPerWave * w + kRowsPerWave, nrows) - 1;
  // positions spanned by this wave's rows (empty when the wave holds only padding)
  const int wpos_lo = i0 + w_first / G;
  const int wpos_hi = w_last >= w_first ? min(i0 + w_last / G, Lq - 1) : wpos_lo - 1;
  const int wave_kmax = wpos_hi >= wpos_lo ? max(0, min(kmax, wpos_hi + off + 1)) : 0;
  const int wave_full = wpos_lo + off + 1;  // keys below this are visible to every row of the wave

  f32x4 acc[kNT][8];
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[nt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[kNT];
  f32x4 lacc[kNT];  // row sums of the probabilities (every element of the 4 holds the sum)
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    m_run[nt] = kNegInf;
    lacc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bf16x8 ones = as_bf16x8(u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  const float sl2 = p.scale_log2;

  const int krow0 = 8 * (n >> 2) + (n & 3);
  const int32_t* bt = PAGED ? p.block_table + s * p.bt_row_stride : nullptr;
  const uint16_t* kbase = p.k + kvh * kHeadDim;
  const uint16_t* vbase = p.v + kvh * kHeadDim;
  const int ntiles = (kmax + kBK - 1) / kBK;

  TileRegs pre;
  if (ntiles > 0) {
    load_tile<PAGED>(pre, p, kbase, vbase, bt, k_start, 0, kmax, tid);
    store_tile(pre, sK[0], sVt[0], tid);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int kb = it * kBK;
    const int buf = it & 1;
    const bool more = it + 1 < ntiles;
    if (more) load_tile<PAGED>(pre, p, kbase, vbase, bt, k_start, kb + kBK, kmax, tid);

    const uint16_t* cK = sK[buf];
    const uint16_t* cV = sVt[buf];
#pragma unroll 1
    for (int sub = 0; sub < 2; ++sub) {
      const int key0 = kb + 32 * sub;
      if (key0 >= wave_kmax) break;  // every key of this step is masked for this wave
      const bool need_mask = key0 + 32 > wave_full || key0 + 32 > kmax;
      bf16x8 kop[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int row = 32 * sub + krow0 + 4 * t;
#pragma unroll
        for (int sidx = 0; sidx < 4; ++sidx) {
          const int ch = 4 * sidx + g;
          kop[t][sidx] = as_bf16x8(*reinterpret_cast<const u32x4*>(&cK[row * kHeadDim + ((ch ^ k_swz(row)) * 8)]));
        }
      }
      bf16x8 vt[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int R = 16 * j + n;
        const int kc = g + 4 * sub;
        vt[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(&cV[R * kBK + ((kc ^ vt_swz(R)) * 8)]));
      }
      // Column tiles one after another, software-pipelined by one tile: the
      // QK^T MFMAs of tile nt+1 are issued before the softmax of tile nt, so the
      // VALU work overlaps the matrix pipe while only two score sets are live.
      f32x4 st[2][2];
      auto qk = [&](f32x4 (&d)[2], int nt) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          d[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int sidx = 0; sidx < 4; ++sidx) d[t] = mfma16x16x32(kop[t][sidx], qop[nt][sidx], d[t]);
        }
      };
      qk(st[0], 0);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        const int cur = nt & 1;
        if (nt + 1 < kNT) qk(st[cur ^ 1], nt + 1);
        float sv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) sv[i] = st[cur][i >> 2][i & 3];
        if (need_mask) {
          const int limit = pos[nt] < 0 ? -1 : min(pos[nt] + off, kmax - 1);  // last visible key
#pragma unroll
          for (int i = 0; i < 8; ++i) sv[i] = (key0 + 8 * g + i <= limit) ? sv[i] : kNegInf;
        }
        float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mx = max_across_groups(mx) * sl2;  // log2 domain (sl2 > 0)
        // lazy maximum: move it only when a score exceeds it by more than kTau
        const bool grow = mx > m_run[nt] + kTau;
        if (__builtin_amdgcn_ballot_w64(grow)) {
          const float m_new = grow ? mx : m_run[nt];
          const float alpha = fast_exp2(m_run[nt] - m_new);  // 1 for lanes that keep their maximum
          lacc[nt] *= alpha;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[nt][j] *= alpha;
          m_run[nt] = m_new;
        }
        const float m_use = m_run[nt] == kNegInf ? 0.f : m_run[nt];
        float pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pv[i] = fast_exp2(__builtin_fmaf(sv[i], sl2, -m_use));
        u32x4 pw;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) pw[q2] = pack_bf16x2(pv[2 * q2], pv[2 * q2 + 1]);
        const bf16x8 pop = as_bf16x8(pw);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[nt][j] = mfma16x16x32(vt[j], pop, acc[nt][j]);
        lacc[nt] = mfma16x16x32(ones, pop, lacc[nt]);
      }
    }
    if (more) store_tile(pre, sK[buf ^ 1], sVt[buf ^ 1], tid);
    __syncthreads();
  }

  // ---- epilogue: normalise and write rows ------------------------------------
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    const float l = lacc[nt][0];
    if (pos[nt] < 0) continue;
    const int r = kRowsPerWave * w + 16 * nt + n;
    const int h = kvh * G + r % G;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* orow = p.out + static_cast<int64_t>(q_start + pos[nt]) * p.out_row_stride + h * kHeadDim + 32 * g;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      u32x4 o;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2)
        o[q2] = pack_bf16x2(acc[nt][2 * q2][rr] * inv, acc[nt][2 * q2 + 1][rr] * inv);
      st16(orow + 8 * rr, o);
    }
  }
}

int prefill_positions_per_tile(int group) { return group >= 1 && group <= kRows ? kRows / group : 1; }

hipError_t launch_prefill(const PrefillParams& p0, int max_seqlen_q, hipStream_t stream) {
  if (p0.num_seqs <= 0 || max_seqlen_q <= 0) return hipSuccess;
  PrefillParams p = p0;
  p.positions_per_tile = prefill_positions_per_tile(p.group);
  p.num_q_tiles = (max_seqlen_q + p.positions_per_tile - 1) / p.positions_per_tile;
  // x: (sequence, kv head) pairs, y: query tiles heaviest first.  Workgroup id
  // x + y * gridDim.x keeps every tile of one (sequence, kv head) on the same
  // XCD (and its L2) whenever gridDim.x is a multiple of 8.
  const dim3 grid(static_cast<unsigned>(p.num_seqs * p.num_kv_heads), static_cast<unsigned>(p.num_q_tiles));
  if (p.block_table)
    hipLaunchKernelGGL(varlen_prefill_kernel<true>, grid, dim3(64 * kWaves), 0, stream, p);
  else
    hipLaunchKernelGGL(varlen_prefill_kernel<false>, grid, dim3(64 * kWaves), 0, stream, p);
  return hipGetLastError();
}

}  // namespace nva
