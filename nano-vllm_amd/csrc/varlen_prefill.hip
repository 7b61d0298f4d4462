// Varlen causal prefill attention for gfx950 (replaces flash_attn_varlen_func at
// nanovllm/layers/attention.py:67-73), with K/V either packed by cu_seqlens_k
// or gathered from the paged cache through block_table (prefix-cache case,
// cu_seqlens_k > cu_seqlens_q, bottom-right causal alignment).
//
// Workgroup = (sequence, kv head, query tile): 8 wavefronts x 32 rows, where a
// row is one (query position, query head) pair of the kv head's GQA group
// (rows are position-major: row r = position r / G, head r % G).  All G heads
// therefore share every K/V tile the workgroup stages.  Keys are visited in
// 64-key tiles, triple-buffered in LDS and filled by global->LDS DMA
// (global_load_lds_dwordx4: no registers, no VALU):
//   K [64 keys][256 B]  16-byte pieces XOR-swizzled by key row
//   V [64 keys][256 B]  32-byte chunks XOR-swizzled by key row
// Each lane of a DMA instruction lands 16 B at LDS base + 16 * lane, so the
// swizzles are made by choosing every lane's source address.  The DMA of tile
// i+2 is issued before the math of tile i, so a tile has two tiles of math to
// arrive (one barrier per tile).  The
// V^T MFMA operand (8 consecutive keys of one dim per lane) is read with
// gfx950's transposing LDS read ds_read_b64_tr_b16: within a 16-lane group,
// lane i receives element i % 4 of the 8 bytes addressed by lanes
// 4e + i / 4 (e = 0..3), so when lane j addresses key row base + j / 4 at dims
// 4 (j % 4) .. +3, lane i holds dim i of keys base .. base + 3.
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

// Swizzle of the 16-byte piece index inside a K row: the 16 rows one MFMA
// operand read touches map to 16 distinct bank groups.
__device__ __forceinline__ int k_swz(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
// Swizzle of the 32-byte chunk index inside a V row: the 16 rows (4 per lane
// group) of one transposing read map to 8 chunk positions, two rows each --
// the minimum of two passes for a 512-byte read.
__device__ __forceinline__ int v_swz(int row) { return (row & 3) | (((row >> 3) & 1) << 2); }

constexpr int kTileBytes = kBK * kHeadDim * 2;  // one K (or V) tile: 16 KiB
constexpr int kStageBytes = 2 * kTileBytes;      // K + V

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// All but the last tile's four DMA instructions have completed.
__device__ __forceinline__ void wait_vmem_keep4() { asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); }

constexpr float kInitMax = -1e30f;  // finite: exp2(fma(s, c, -m)) never sees -inf - -inf

}  // namespace

// Per-lane constants of the DMA that fills a stage: every wave issues four
// 1 KiB instructions; lane `lane` of instruction u fills key row `row[u]`,
// element offset `col[u]` inside that row (K for waves 0..3, V for 4..7).
struct DmaLane {
  int row[4];
  int col[4];
};

__device__ __forceinline__ DmaLane dma_lane(int w, int lane) {
  DmaLane d;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int off = (4 * w + u) * 1024;
    const int local = (off & (kTileBytes - 1)) + 16 * lane;
    const int row = local >> 8;
    const int piece = (local >> 4) & 15;
    d.row[u] = row;
    d.col[u] = off < kTileBytes ? (piece ^ k_swz(row)) * 8
                                : ((piece >> 1) ^ v_swz(row)) * 16 + (piece & 1) * 8;
  }
  return d;
}

// DMA of one 64-key K/V tile into LDS stage `st` (32 KiB).  Keys at or beyond
// kmax are redirected to the tile's first key, a valid row whose scores the
// masks remove; a block id outside the pool redirects the tile to slot 0.
template <bool PAGED>
__device__ __forceinline__ void dma_tile(char* st, const PrefillParams& p, const uint16_t* base, int64_t stride,
                                         const DmaLane& d, const int32_t* bt, int k_start, int kb, int kmax,
                                         int w) {
  int64_t slot0;
  if constexpr (PAGED) {
    const int bi = kb / p.block_size;
    const int page = bi < p.max_blocks ? bt[bi] : -1;
    const bool ok = page >= 0 && page < p.num_blocks;
    slot0 = ok ? static_cast<int64_t>(page) * p.block_size + (kb % p.block_size) : 0;
  } else {
    slot0 = static_cast<int64_t>(k_start) + kb;
  }
  const uint16_t* tile = base + slot0 * stride;
  const int nrow = kmax - kb;  // rows that exist (>= 64 except in the last tile)
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = d.row[u] < nrow ? d.row[u] : 0;
    const uint16_t* src = tile + row * stride + d.col[u];
    __builtin_amdgcn_global_load_lds((gvoid*)src, (lvoid*)(st + (4 * w + u) * 1024), 16, 0, 0);
  }
}

template <bool PAGED>
__global__ __launch_bounds__(64 * kWaves) void varlen_prefill_kernel(PrefillParams p) {
  // Three stages as separate objects, so the compiler can prove that reads of
  // one stage never alias the DMA filling another and need not wait for it.
  __shared__ __attribute__((aligned(1024))) char smem0[kStageBytes];
  __shared__ __attribute__((aligned(1024))) char smem1[kStageBytes];
  __shared__ __attribute__((aligned(1024))) char smem2[kStageBytes];

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

  // rows of this lane: r = 32w + 16nt + n
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
    m_run[nt] = kInitMax;
    lacc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bf16x8 ones = as_bf16x8(u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
  const float sl2 = p.scale_log2;

  // Per-lane LDS byte offsets of the MFMA operand reads inside a stage; the key
  // tile (t), the 32-key half (sub) and the 4-key half (hh) add constants.
  //   K: row krow0 + 4t + 32sub, piece (4 sidx + g) ^ k_swz(row) = (4 sidx + g) ^ n
  //   V: row 8g + 4hh + n/4 + 32sub, chunk j ^ v_swz(row) = j ^ (n/4 | (g&1) << 2)
  const int krow0 = 8 * (n >> 2) + (n & 3);
  int kaddr[4];
#pragma unroll
  for (int sidx = 0; sidx < 4; ++sidx) kaddr[sidx] = krow0 * 256 + ((4 * sidx + g) ^ n) * 16;
  const int vs = (n >> 2) | ((g & 1) << 2);
  int vaddr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) vaddr[j] = kTileBytes + (8 * g + (n >> 2)) * 256 + 8 * (n & 3) + (j ^ vs) * 32;

  const DmaLane dl = dma_lane(w, lane);
  const bool k_wave = w < 4;  // waves 0..3 stage K, 4..7 stage V
  const int32_t* bt = PAGED ? p.block_table + s * p.bt_row_stride : nullptr;
  const uint16_t* dbase = (k_wave ? p.k : p.v) + kvh * kHeadDim;
  const int64_t dstride = k_wave ? p.k_row_stride : p.v_row_stride;
  const int ntiles = (kmax + kBK - 1) / kBK;

  // One 64-key tile: start the DMA of tile it+2 into `nxt`, run the math on
  // `cur`, wait for tile it+1 and synchronise.
  auto tile_step = [&](int it, const char* cur, char* nxt) {
    const int kb = it * kBK;
    const bool issue = it + 2 < ntiles;
    if (issue) dma_tile<PAGED>(nxt, p, dbase, dstride, dl, bt, k_start, kb + 2 * kBK, kmax, w);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int key0 = kb + 32 * sub;
      if (key0 < wave_kmax) {  // otherwise every key of this step is masked for this wave
        const bool need_mask = key0 + 32 > wave_full || key0 + 32 > kmax;
        const char* sb = cur + 8192 * sub;
        bf16x8 kop[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int sidx = 0; sidx < 4; ++sidx)
            kop[t][sidx] = as_bf16x8(*reinterpret_cast<const u32x4*>(sb + kaddr[sidx] + 1024 * t));
        // V^T operands: dims 16j .. 16j+15 of keys 8g .. 8g+7 (two transposing reads)
        bf16x8 vt[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(sb + vaddr[j]));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(sb + vaddr[j] + 1024));
          const u32x2 a = __builtin_bit_cast(u32x2, lo);
          const u32x2 b = __builtin_bit_cast(u32x2, hi);
          vt[j] = as_bf16x8(u32x4{a[0], a[1], b[0], b[1]});
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
          const int curb = nt & 1;
          if (nt + 1 < kNT) qk(st[curb ^ 1], nt + 1);
          float sv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) sv[i] = st[curb][i >> 2][i & 3];
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
          const float mneg = -m_run[nt];
          float pv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) pv[i] = fast_exp2(__builtin_fmaf(sv[i], sl2, mneg));
          u32x4 pw;
#pragma unroll
          for (int q2 = 0; q2 < 4; ++q2) pw[q2] = pack_bf16x2(pv[2 * q2], pv[2 * q2 + 1]);
          const bf16x8 pop = as_bf16x8(pw);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[nt][j] = mfma16x16x32(vt[j], pop, acc[nt][j]);
          lacc[nt] = mfma16x16x32(ones, pop, lacc[nt]);
        }
      }
    }
    if (issue)
      wait_vmem_keep4();  // tile it+1 has landed; tile it+2 may still be in flight ...
    else
      wait_vmem_all();
    __syncthreads();  // ... for every wave; stage `cur` is free again
  };

  if (ntiles > 0) dma_tile<PAGED>(smem0, p, dbase, dstride, dl, bt, k_start, 0, kmax, w);
  if (ntiles > 1) {
    dma_tile<PAGED>(smem1, p, dbase, dstride, dl, bt, k_start, kBK, kmax, w);
    wait_vmem_keep4();
  } else {
    wait_vmem_all();
  }
  __syncthreads();
  for (int it = 0; it < ntiles; it += 3) {
    tile_step(it, smem0, smem2);
    if (it + 1 < ntiles) tile_step(it + 1, smem1, smem0);
    if (it + 2 < ntiles) tile_step(it + 2, smem2, smem1);
  }

  // ---- epilogue: normalise and write rows ------------------------------------
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    const float l = lacc[nt][0];
    if (pos[nt] < 0) continue;
    const int r = kRowsPerWave * w + 16 * nt + n;
    const int h = kvh * G + r % G;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* orow = p.out + static_cast<int64_t>(q_start + pos[nt]) * p.out_row_stride + h * kHeadDim + 4 * g;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x2 o;
      o[0] = pack_bf16x2(acc[nt][j][0] * inv, acc[nt][j][1] * inv);
      o[1] = pack_bf16x2(acc[nt][j][2] * inv, acc[nt][j][3] * inv);
      *reinterpret_cast<u32x2*>(orow + 16 * j) = o;
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
