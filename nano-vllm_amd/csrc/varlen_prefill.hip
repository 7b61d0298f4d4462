// Varlen causal prefill attention for gfx950 (replaces flash_attn_varlen_func at
// nanovllm/layers/attention.py:67-73), with K/V either packed by cu_seqlens_k
// or gathered from the paged cache through block_table (prefix-cache case,
// cu_seqlens_k > cu_seqlens_q, bottom-right causal alignment).
//
// Workgroup = (sequence, kv head, query tile): 8 wavefronts x 32 rows, where a
// row is one (query position, query head) pair of the kv head's GQA group
// (rows are position-major: row r = position r / G, head r % G).  All G heads
// therefore share every K/V tile the workgroup stages.  Keys are visited in
// 64-key tiles held in a 4-stage LDS ring:
//   K [64 keys][256 B]  16-byte pieces XOR-swizzled by key row (row & 15)
//   V [64 keys][256 B]  32-byte chunks XOR-swizzled by key row (2 * (row & 3))
// Tiles are copied global -> LDS by global_load_lds_dwordx4 (no registers),
// two tiles ahead: every lane moves 16-byte pieces to 16 * lane inside its
// wave's KiB, so the swizzles are made by choosing each lane's source address.
// One barrier per tile, placed between the tile's two 32-key steps.
//
// Per 32-key step a wave computes the 32 keys x 32 rows tile S^T = K . Q^T with
// one chain of 32x32x16 bf16 MFMAs over the head dim, and the MFMAs of the
// next step's S^T (their K operands read at the start of the step) are issued
// between the exponentials of the current one, so the matrix pipe and the VALU
// overlap.  Lane l owns
// row l % 32 and keys 8b + 4h + r (h = l / 32, b, r = 0..3) of the step, so
// the row maximum needs one permlane32 swap, and the probabilities of
// registers 8u .. 8u+7 are exactly the P^T operand of PV MFMA u (keys
// 16u + 8(e/4) + 4h + e%4) -- they never leave the lane.  The matching V^T
// operand (those 8 keys of one head dim per lane) is read with gfx950's
// transposing LDS read ds_read_b64_tr_b16: within a 16-lane group, lane i
// receives element i % 4 of the 8 bytes addressed by lanes 4e + i / 4, so
// when lane j addresses key row base + j / 4 at dims 4 (j % 4) .. +3, lane i
// holds dim i of keys base .. base + 3.
//
// Softmax runs online in the exp2 domain with a lazily updated row maximum m:
// Q is scaled by softmax_scale * log2(e) once per item, and every QK chain
// starts from the accumulator value -m, so the MFMAs deliver s - m directly and
// each probability is a single exp2.  The first step sets m to the row
// maximum; after that m moves only when a score exceeds it by more than kTau
// (so p <= 2^kTau), which makes the rescale of the accumulators rare.  Masks
// are evaluated only on tiles that cross the causal diagonal or the key end.
#include <algorithm>

#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

namespace {

constexpr int kWaves = 8;
constexpr int kRowsPerWave = 32;
constexpr int kRows = kWaves * kRowsPerWave;  // (position, head) rows per workgroup
constexpr int kBK = 64;                       // keys per LDS tile
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kTau = 8.0f;                  // lazy-rescale threshold (log2 units)

constexpr int kStages = 4;                    // LDS ring depth

// Tile geometry for head dimension D (64 or 128): a key row is RB = 2D bytes.
template <int D>
struct Geom {
  static constexpr int RB = 2 * D;
  static constexpr int kTileBytes = kBK * RB;        // one K (or V) tile: 16 KiB at D = 128
  static constexpr int kStageBytes = 2 * kTileBytes;  // K + V
  // K tiles of the ring first, V tiles after them: with the loop unrolled over
  // the stages every operand read is a per-lane base plus an immediate < 64 KiB.
  static constexpr int kVRing = kStages * kTileBytes;
  static constexpr int KP = RB / 16;                  // 16-byte pieces per row
  static constexpr int P = kStageBytes / 1024 / kWaves;  // 1 KiB staging pieces per wave
  // K: 16-byte piece swizzle; the consecutive rows one quarter-wave of an
  // operand read touches land in distinct bank groups.
  __device__ static int k_swz(int row) { return row & (KP - 1); }
  // V: 32-byte chunk swizzle; each half-wave of a transposing read (4 rows x
  // 2 chunks) lands in distinct 32-byte bank groups.
  __device__ static int v_swz(int row) { return D == 128 ? 2 * (row & 3) : (row & 3); }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Workgroup barrier after this wave's LDS accesses have completed.  Unlike
// __syncthreads it does not also wait for the tile copies still in flight;
// those are waited for explicitly (wait_vmem) where a tile must be complete.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ bf16x8 read_tr_pair(const char* p0, const char* p1) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
  const u32x2 a = __builtin_bit_cast(u32x2, lo);
  const u32x2 b = __builtin_bit_cast(u32x2, hi);
  return as_bf16x8(u32x4{a[0], a[1], b[0], b[1]});
}

}  // namespace

// Per-lane constants of the staging of a tile: every wave moves P 1 KiB
// pieces; lane `lane` of piece u carries key row `row[u]`, element offset
// `col[u]` inside that row (K for waves 0..3, V for 4..7).
template <int P>
struct StageLane {
  int row[P];
  int col[P];
  uint32_t off[P];  // byte offset of (row, col) from the tile's first key
};

template <int D>
__device__ __forceinline__ StageLane<Geom<D>::P> stage_lane(int w, int lane, int64_t stride) {
  using Gm = Geom<D>;
  StageLane<Gm::P> d;
#pragma unroll
  for (int u = 0; u < Gm::P; ++u) {
    const int off = (Gm::P * w + u) * 1024;
    const int local = (off & (Gm::kTileBytes - 1)) + 16 * lane;
    const int row = local / Gm::RB;
    const int piece = (local >> 4) & (Gm::KP - 1);
    d.row[u] = row;
    d.col[u] = off < Gm::kTileBytes ? (piece ^ Gm::k_swz(row)) * 8
                                    : ((piece >> 1) ^ Gm::v_swz(row)) * 16 + (piece & 1) * 8;
    d.off[u] = static_cast<uint32_t>((row * stride + d.col[u]) * 2);
  }
  return d;
}

typedef const __attribute__((address_space(4))) int32_t const_i32;

// Block id of the page holding key kb (-1 past the mb entries of the table row
// at bt).  The block table is read through the constant address space: a
// scalar load, counted by lgkmcnt, not vmcnt.
__device__ __forceinline__ int page_of(const PrefillParams& p, const_i32* bt, int mb, int kb) {
  const int bi = kb / p.block_size;
  return bi < mb ? bt[bi] : -1;
}

// Address of the first key of the 64-key tile at kb: packed K/V from
// k_start, or the page `page` (paged caches only).  A block id outside
// [0, num_blocks) redirects the tile to slot 0, so no access leaves the cache;
// those keys are not masked (the result of such a sequence is unspecified,
// other sequences are unaffected).  Masking them costs the loop ~3% (scalar
// state per ring stage), so only decode masks them.
template <bool PAGED>
__device__ __forceinline__ const char* tile_base(const PrefillParams& p, const uint16_t* base, int64_t stride, int page,
                                                 int k_start, int kb) {
  int64_t slot0;
  if constexpr (PAGED) {
    const bool ok = page >= 0 && page < p.num_blocks;
    slot0 = ok ? static_cast<int64_t>(page) * p.block_size + (kb % p.block_size) : 0;
  } else {
    slot0 = static_cast<int64_t>(k_start) + kb;
  }
  return reinterpret_cast<const char*>(base + slot0 * stride);
}

typedef __attribute__((address_space(3))) char lds_char;

// LDS byte address of a pointer into the workgroup's shared memory.
__device__ __forceinline__ uint32_t lds_addr(const char* ptr) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_char*)ptr));
}

// Copy 16 bytes per lane from base + off (base uniform, in SGPRs) straight into
// LDS at lds + 16 * lane (global_load_lds_dwordx4).  Inline asm, so that the
// compiler sees no LDS store it would have to order against the operand reads
// of other stages; ordering comes from wait_vmem and the barriers instead.
__device__ __forceinline__ void dma16(const char* base, uint32_t off, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// Wait until at most N of this wave's vector-memory operations are in flight.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Copy this wave's P KiB of one 64-key K/V tile (at `tile`, key kb) into the
// stage whose K tile is at `st` (its V tile v_skip + tile bytes further on):
// lane `lane` of piece u lands at (P w + u) KiB + 16 lane and carries the
// swizzled (row, col) of StageLane.  Keys at or beyond kmax (only in the last
// tile) are redirected to the tile's first key, a valid row whose scores the
// masks remove.
template <int P, int U0 = 0, int U1 = P>
__device__ __forceinline__ void dma_tile(char* st, const char* tile, const StageLane<P>& d, int kb, int kmax, int w,
                                         int v_skip) {
  const uint32_t dst = lds_addr(st) + v_skip + P * w * 1024;
  if (kb + kBK <= kmax) {
#pragma unroll
    for (int u = U0; u < U1; ++u) dma16(tile, d.off[u], dst + u * 1024);
  } else {
    const int nrow = kmax - kb;
#pragma unroll
    for (int u = U0; u < U1; ++u)
      dma16(tile, d.row[u] < nrow ? d.off[u] : static_cast<uint32_t>(d.col[u] * 2), dst + u * 1024);
  }
}

// A work item -- query tile `tile` of sequence s, kv head kvh (its GQA
// group's heads) -- with the per-item scalars read from cu_seqlens.
struct ItemDesc {
  int s, kvh, tile;
  int q_start, Lq, k_start, Lk;
  int i0;      // first query position of the tile
  int kmax;    // keys [0, kmax) are visible to some row of the tile
  int ntiles;  // 64-key tiles spanning [0, kmax)
  int split_slot;  // >= 0: one key half of a split item (workspace slot); -1: a whole item
  int bt_off;      // paged: block-table entries before the item's first key (a second key half)
  bool valid;  // false: no item (s < 0) or a tile past the sequence's end
};

// cu_q / cu_k: cu_seqlens_q / cu_seqlens_k, in global memory or a copy in LDS.
__device__ __forceinline__ ItemDesc item_desc(const PrefillParams& p, const int* cu_q, const int* cu_k, int s, int kvh,
                                              int tile) {
  ItemDesc d{};
  d.s = s;
  d.kvh = kvh;
  d.tile = tile;
  d.split_slot = -1;
  d.bt_off = 0;
  d.valid = false;
  if (s < 0) return d;
  d.q_start = __builtin_amdgcn_readfirstlane(cu_q[s]);
  d.Lq = __builtin_amdgcn_readfirstlane(cu_q[s + 1]) - d.q_start;
  d.k_start = __builtin_amdgcn_readfirstlane(cu_k[s]);
  d.Lk = __builtin_amdgcn_readfirstlane(cu_k[s + 1]) - d.k_start;
  d.i0 = tile * p.positions_per_tile;
  d.valid = d.i0 < d.Lq;
  const int last_pos = min(d.i0 + p.positions_per_tile, d.Lq) - 1;
  d.kmax = max(0, min(d.Lk, last_pos + (d.Lk - d.Lq) + 1));
  d.ntiles = (d.kmax + kBK - 1) / kBK;
  return d;
}

// Work item of cell c of the direct grid under key halving.  When the cap
// below is 0 (the launch is oversubscribed, so nothing splits) the cells are
// those of the plain grid -- x = (sequence, kv head), y = query tile from the
// last -- flattened.  Otherwise the grid is compact: c = num_kv_heads *
// position + kv head, over the (sequence, query tile) pairs in level order --
// query tile descending, then sequence: the heaviest tiles first -- where a
// split pair takes two consecutive positions, its key halves.  A pair splits
// when its tile sees at least split_tiles key tiles (keys [0, min(Lk,
// (t + 1) BP + Lk - Lq))) and fewer such pairs precede it in this order than
// the cap: split_slots / num_kv_heads, and the CUs the real items leave free,
// over num_kv_heads: a half beyond those waits for a CU, and an oversubscribed
// launch has no idle CU for it to fill.  When the lightest item sees at most
// half the key tiles of the heaviest, split_cus / kSplitSpareDiv more may
// split: the items that then wait for a CU are the lightest ones, which fit
// beside the halves (with a long cached prefix every item is heavy, and a
// waiting one would end after the halves).  Its slots are rank *
// num_kv_heads + kv head.
// Every workgroup derives it from cu_seqlens with ballots over 64 sequences at
// a time, so the result is wave-uniform; s = -1 past the last pair.  (The
// scan over the levels costs the lighter items time that an oversubscribed
// launch would put on its critical path, hence the plain cells there.)
constexpr int kSplitSpareDiv = 8;  // halves may exceed the free CUs by split_cus / kSplitSpareDiv

struct CellItem {
  int s, kvh, t, half;
  int pair;  // rank of a split pair, -1 for a whole item
};

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

__device__ __forceinline__ CellItem compact_cell(const PrefillParams& p, int c) {
  const int lane = threadIdx.x & 63;
  CellItem ci;
  ci.s = -1;
  ci.kvh = 0;
  ci.t = 0;
  ci.half = 0;
  ci.pair = -1;
  const int BP = p.positions_per_tile;
  const int thr = (p.split_tiles - 1) * kBK;
  int pos = 0;    // positions before this level and chunk
  int cands = 0;  // split candidates before them
  // the first 64 sequences' lengths stay in registers across the levels
  int lq0 = 0, lk0 = 0;
  if (lane < p.num_seqs) {
    lq0 = p.cu_q[lane + 1] - p.cu_q[lane];
    lk0 = p.cu_k[lane + 1] - p.cu_k[lane];
  }
  // real items (num_kv_heads * the sequences' query tiles), and the keys the
  // lightest (a sequence's first tile) and the heaviest (its last) item see
  auto lens_stats = [&](int lq, int lk, int& ntq, int& kmin, int& kmax) {
    if (lq > 0) {
      ntq += (lq + BP - 1) / BP;
      kmin = min(kmin, min(lk, min(BP, lq) + lk - lq));
      kmax = max(kmax, lk);
    }
  };
  int ntq = 0, kmin = 0x7fffffff, kmax = 0;
  lens_stats(lq0, lk0, ntq, kmin, kmax);
  for (int c0 = 64; c0 < p.num_seqs; c0 += 64) {
    const int sq = c0 + lane;
    if (sq < p.num_seqs) lens_stats(p.cu_q[sq + 1] - p.cu_q[sq], p.cu_k[sq + 1] - p.cu_k[sq], ntq, kmin, kmax);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ntq += __shfl_xor(ntq, o);
    kmin = min(kmin, __shfl_xor(kmin, o));
    kmax = max(kmax, __shfl_xor(kmax, o));
  }
  const int items = p.num_kv_heads * __builtin_amdgcn_readfirstlane(ntq);
  const int kmin_u = __builtin_amdgcn_readfirstlane(min(kmin, 1 << 30));  // no sequence with queries: 2^30
  const bool light_tail = 2 * ((kmin_u + kBK - 1) / kBK) <= (__builtin_amdgcn_readfirstlane(kmax) + kBK - 1) / kBK;
  const int spare = p.split_cus + (light_tail ? p.split_cus / kSplitSpareDiv : 0) - items;
  const int cap = min(p.split_slots, max(0, spare)) / p.num_kv_heads;
  if (cap == 0) {
    const int gx = p.num_seqs * p.num_kv_heads;
    if (c >= gx * p.num_q_tiles) return ci;
    const int x = c % gx;
    ci.s = x / p.num_kv_heads;
    ci.kvh = x - ci.s * p.num_kv_heads;
    ci.t = p.num_q_tiles - 1 - c / gx;
    return ci;  // may be a tile past the sequence's end: item_desc marks it invalid
  }
  ci.kvh = c % p.num_kv_heads;
  const int k = c / p.num_kv_heads;
  for (int t = p.num_q_tiles - 1; t >= 0; --t) {
    for (int c0 = 0; c0 < p.num_seqs; c0 += 64) {
      const int sq = c0 + lane;
      bool alive = false, cand = false;
      if (sq < p.num_seqs) {
        const int Lq = c0 == 0 ? lq0 : p.cu_q[sq + 1] - p.cu_q[sq];
        const int Lk = c0 == 0 ? lk0 : p.cu_k[sq + 1] - p.cu_k[sq];
        alive = t * BP < Lq;
        cand = alive && min(Lk, min((t + 1) * BP, Lq) + Lk - Lq) > thr;
      }
      const uint64_t am = __builtin_amdgcn_ballot_w64(alive);
      const uint64_t cm = __builtin_amdgcn_ballot_w64(cand);
      const int rank = cands + lanes_below(cm);
      const bool sp = cand && rank < cap;
      const uint64_t sm = __builtin_amdgcn_ballot_w64(sp);
      const int n = __builtin_popcountll(am) + __builtin_popcountll(sm);
      if (k < pos + n) {
        const int first = pos + lanes_below(am) + lanes_below(sm);  // this lane's first position
        const uint64_t hm = __builtin_amdgcn_ballot_w64(alive && k >= first && k < first + (sp ? 2 : 1));
        if (hm == 0) return ci;  // cannot happen: the level's positions are the lanes' runs
        const int L = static_cast<int>(__builtin_ctzll(hm));
        ci.s = c0 + L;
        ci.t = t;
        ci.half = __builtin_amdgcn_readlane(k - first, L);
        ci.pair = __builtin_amdgcn_readlane(sp ? rank : -1, L);
        return ci;
      }
      pos += n;
      cands += __builtin_popcountll(cm);
    }
  }
  return ci;
}

// Restrict item d to key half `half` of its tiles: half 0 takes tiles
// [0, mid), half 1 [mid, ntiles).  The item's keys are re-based at the half's
// first key (k_start and Lk move together, so the causal offset Lk - Lq
// follows), and kmax stops at the half's end.  Paged, mid is the page
// boundary nearest the middle (tiles per page tpp; a tile never straddles
// pages), and the second half starts mid / tpp entries into the block-table
// row; mid may reach ntiles, leaving the second half no key (its partial then
// weighs nothing in the merge).
template <bool PAGED>
__device__ __forceinline__ void key_half(const PrefillParams& p, ItemDesc& d, int half, int slot) {
  int mid = (d.ntiles + 1) / 2;
  if constexpr (PAGED) {
    const int tpp = p.block_size / kBK;
    mid = min(d.ntiles, max(tpp, (mid + tpp / 2) / tpp * tpp));
    d.bt_off = half ? mid / tpp : 0;
  }
  const int t_lo = half ? mid : 0;
  const int t_hi = half ? d.ntiles : mid;
  const int k0 = t_lo * kBK;
  d.kmax = max(0, min(d.kmax, t_hi * kBK) - k0);
  d.ntiles = t_hi - t_lo;
  d.k_start += k0;
  d.Lk -= k0;
  d.split_slot = slot;
}

// Bound on the merging workgroup's wait for the other half's partial.  With
// the control words consistent, that half arrived first and only its stores
// remain, so the wait ends within microseconds (and with the arrival count out
// of step the other half is already running or next in line); the bound keeps
// a wave from spinning for ever should that ever fail.  Each poll sleeps ~128
// cycles after a device-scope load: about 30 ms in all.
constexpr uint32_t kSplitSpinMax = 1u << 16;

// End of one key half of a split item, after the loop.  Thread 0 counts the
// arrival and reads the slot's epoch E and the poll limit in one round trip.
// The even arrival writes its unnormalised O, row maxima and row sums to the
// item's slot, publishes them with the ready word E + 1 and returns false.
// The odd arrival waits for that ready word, folds the partial into its own
// acc and l (both rescaled to the larger maximum), advances the slot to epoch
// E + 1 (arrival count 2E + 2) and returns true.  A ready word from an earlier
// epoch never equals E + 1, so nothing published by an earlier call (or late,
// after a wait gave up) is taken for this call's partial.  If the wait gives
// up, the item's rows become NaN, the error bit is set in split_err[0] and the
// slot advances all the same.
template <int D>
__device__ __forceinline__ bool merge_key_halves(const PrefillParams& p, char* smem_all, int slot,
                                                 f32x16 (&acc)[D / 32], float m_run, float& l) {
  constexpr int NJD = D / 32;
  constexpr int kThreads = 64 * kWaves;
  uint32_t* ctl = p.split_ctl + kPrefillSplitCtlWords * slot;
  float* part = p.split_part + static_cast<int64_t>(slot) * kPrefillSplitPartFloats;
  float4* pacc = reinterpret_cast<float4*>(part);
  float* pm = part + kRows * 128;
  const int tid = threadIdx.x;
  uint32_t* s_ctl = reinterpret_cast<uint32_t*>(smem_all);
  barrier_lds();  // every wave is done with the ring
  if (tid == 0) {
    s_ctl[0] = atomicAdd(ctl, 1u);
    s_ctl[1] = __hip_atomic_load(ctl + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_ctl[2] = __hip_atomic_load(p.split_err + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  barrier_lds();
  const uint32_t arrival = __builtin_amdgcn_readfirstlane(s_ctl[0]);
  const uint32_t epoch = __builtin_amdgcn_readfirstlane(s_ctl[1]);
  if ((arrival & 1u) == 0) {
#pragma unroll
    for (int jd = 0; jd < NJD; ++jd)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        pacc[(4 * jd + b) * kThreads + tid] =
            float4{acc[jd][4 * b], acc[jd][4 * b + 1], acc[jd][4 * b + 2], acc[jd][4 * b + 3]};
    pm[tid] = m_run;
    pm[kThreads + tid] = l;
    // Every wave waits for its stores to reach L2, then one release at device
    // scope publishes them all: an agent-scope fence writes back the whole L2
    // of this XCD, so one per workgroup rather than one per wave.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    barrier_lds();
    if (tid == 0) __hip_atomic_store(ctl + 1, epoch + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    return false;
  }
  if (tid == 0) {
    // Poll with relaxed loads (an acquire per poll would invalidate this XCD's
    // L2 each time, under every other workgroup on it), then acquire once.
    const uint32_t lim = s_ctl[2];
    const uint32_t polls = lim == 0u ? kSplitSpinMax : lim - 1u;
    uint32_t got = 0u;
    for (uint32_t k = 0; k < polls; ++k) {
      if (__hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch + 1u) {
        got = 1u;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (!got) atomicOr(p.split_err, kPrefillErrSplitWait);
    __hip_atomic_store(ctl, 2u * (epoch + 1u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctl + 2, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_ctl[3] = got;
  }
  barrier_lds();
  if (__builtin_amdgcn_readfirstlane(s_ctl[3]) == 0u) {
    // The partial never came: the item's rows become NaN (bits laundered
    // through an empty asm, so no arithmetic on them is folded).
    uint32_t nan_bits = 0x7fc00000u;
    asm volatile("" : "+v"(nan_bits));
    const float qnan = __builtin_bit_cast(float, nan_bits);
#pragma unroll
    for (int jd = 0; jd < NJD; ++jd)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[jd][e] = qnan;
    l = 1.f;
    return true;
  }
  // the other waves' loads of the partial come after thread 0's acquire (the
  // barrier orders them); a workgroup-scope acquire keeps them after it
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // a half whose rows saw no key (sum 0) has no maximum: weight 0
  const float la = pm[kThreads + tid];
  const float ma = la > 0.f ? pm[tid] : kNegInf;
  const float mb = l > 0.f ? m_run : kNegInf;
  const float mm = fmaxf(ma, mb);
  const float wa = ma == kNegInf ? 0.f : fast_exp2(ma - mm);
  const float wb = mb == kNegInf ? 0.f : fast_exp2(mb - mm);
  l = wa * la + wb * l;
#pragma unroll
  for (int jd = 0; jd < NJD; ++jd)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float4 a = pacc[(4 * jd + b) * kThreads + tid];
      acc[jd][4 * b] = wa * a.x + wb * acc[jd][4 * b];
      acc[jd][4 * b + 1] = wa * a.y + wb * acc[jd][4 * b + 1];
      acc[jd][4 * b + 2] = wa * a.z + wb * acc[jd][4 * b + 2];
      acc[jd][4 * b + 3] = wa * a.w + wb * acc[jd][4 * b + 3];
    }
  return true;
}

// The thread index passes through an empty asm so that everything derived
// from it (operand addresses, staging offsets) is formed where it is used:
// hoisted out of the persistent kernel's item loop, those values would stay
// live across items and push the register count past 256.
__device__ __forceinline__ int laundered_tid() {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  return tid;
}

// Q^T operand of item `it` for this lane: row r = 32w + n, head dims
// 16 ks + 8h .. +7 for MFMA step ks (zeros for padding rows).
template <int D>
__device__ __forceinline__ void item_fetch_q(const PrefillParams& p, const ItemDesc& it, bf16x8 (&qop)[D / 16]) {
  const int tid = laundered_tid();
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 31;
  const int h = lane >> 5;
  const int G = p.group;
  const int r = kRowsPerWave * w + n;
  const int qp = it.i0 + r / G;
  const int qh = it.kvh * G + r % G;
  const bool row_ok = r < p.positions_per_tile * G && qp < it.Lq;
  const uint16_t* qrow = p.q + static_cast<int64_t>(it.q_start + qp) * p.q_row_stride + qh * D + 8 * h;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const u32x4 z = {0u, 0u, 0u, 0u};
    qop[ks] = as_bf16x8(row_ok ? ld16(qrow + 16 * ks) : z);
  }
}

// Per-wave staging constants of item `it`'s K/V tiles (waves 0..3 copy K,
// 4..7 copy V).
template <bool PAGED, int D>
struct ItemStaging {
  const_i32* bt;
  int mb;  // entries of the block-table row from bt on
  const uint16_t* dbase;
  int64_t dstride;
  StageLane<Geom<D>::P> dl;
  int v_skip;
  int w;

  __device__ __forceinline__ ItemStaging(const PrefillParams& p, const ItemDesc& it) {
    using Gm = Geom<D>;
    const int tid = laundered_tid();
    w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: staging bases stay scalar
    const bool k_wave = w < 4;
    bt = PAGED ? (const_i32*)(p.block_table + static_cast<int64_t>(it.s) * p.bt_row_stride + it.bt_off) : nullptr;
    mb = p.max_blocks - it.bt_off;
    dbase = (k_wave ? p.k : p.v) + it.kvh * D;
    dstride = k_wave ? p.k_row_stride : p.v_row_stride;
    dl = stage_lane<D>(w, tid & 63, dstride);
    v_skip = k_wave ? 0 : Gm::kVRing - Gm::kTileBytes;
  }
  // first key of tile t in global memory
  __device__ __forceinline__ const char* tile(const PrefillParams& p, const ItemDesc& it, int page, int t) const {
    return tile_base<PAGED>(p, dbase, dstride, page, it.k_start, t * kBK);
  }
  __device__ __forceinline__ void copy(const PrefillParams& p, const ItemDesc& it, char* st, int page, int t) const {
    dma_tile<Geom<D>::P>(st, tile(p, it, page, t), dl, t * kBK, it.kmax, w, v_skip);
  }
  // pieces [U0, U1) of this wave's share of tile t, whose first key is at src
  template <int U0, int U1>
  __device__ __forceinline__ void copy_part(const ItemDesc& it, char* st, const char* src, int t) const {
    dma_tile<Geom<D>::P, U0, U1>(st, src, dl, t * kBK, it.kmax, w, v_skip);
  }
};

// Start the copies of item `it`'s tiles 0 and 1 into ring stages 0 and 1.
template <bool PAGED, int D>
__device__ __forceinline__ void item_fetch_tiles(const PrefillParams& p, char* smem_all, const ItemDesc& it) {
  const ItemStaging<PAGED, D> st(p, it);
#pragma unroll
  for (int t = 0; t < 2; ++t)
    if (t < it.ntiles) st.copy(p, it, smem_all + t * Geom<D>::kTileBytes, PAGED ? page_of(p, st.bt, st.mb, t * kBK) : 0, t);
}

// Run work item `it` on the whole workgroup.  Its Q operands (qop) and the
// copies of its tiles 0 and 1 were issued before (item_fetch_q,
// item_fetch_tiles).  When `next` is valid, this issues next's Q loads into
// qop once the last QK has been issued and next's first two tile copies right
// after the epilogue's barrier, so their latency overlaps the epilogue; the
// epilogue's transpose therefore uses ring stages 2 and 3 only.  SPLIT: the
// item may be one key half, merged at the end (merge_key_halves); only the
// direct grid splits, so the persistent grid's code carries no merge.
template <bool PAGED, int D, bool SPLIT>
__device__ __forceinline__ void prefill_run(const PrefillParams& p, char* smem_all, const ItemDesc& item,
                                            bf16x8 (&qop)[D / 16], const ItemDesc& next, uint32_t* claim_ctr,
                                            uint32_t& claim) {
  using Gm = Geom<D>;
  constexpr int RB = Gm::RB;
  constexpr int KP = Gm::KP;
  constexpr int P = Gm::P;
  constexpr int NKS = D / 16;  // QK MFMAs (16 head dims each) per 32-key step
  constexpr int NJD = D / 32;  // PV MFMAs (32 head dims each) per 16 keys
  // The ring: stage i % 4 holds 64-key tile i, its K at i % 4 * kTileBytes
  // and its V kVRing further on.
  auto stage = [&](int i) { return smem_all + (i & (kStages - 1)) * Gm::kTileBytes; };

  const int s = item.s;
  const int q_start = item.q_start;
  const int Lq = item.Lq;
  const int k_start = item.k_start;
  const int kvh = item.kvh;
  const int G = p.group;
  const int BP = p.positions_per_tile;  // query positions per workgroup (BP * G <= kRows)
  const int i0 = item.i0;
  const int off = item.Lk - Lq;  // bottom-right causal offset
  const int kmax = item.kmax;
  const int ntiles = item.ntiles;

  const int tid = laundered_tid();
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31;  // row of this lane within the wave's 32
  const int h = lane >> 5;  // lane half
  const int nrows = BP * G;
  const int r = kRowsPerWave * w + n;
  const int qp = i0 + r / G;
  const bool row_ok = r < nrows && qp < Lq;
  const int pos = row_ok ? qp : -1;

  const int w_first = kRowsPerWave * w;
  const int w_last = min(kRowsPerWave * w + kRowsPerWave, nrows) - 1;
  // positions spanned by this wave's rows (empty when the wave holds only padding)
  const int wpos_lo = i0 + w_first / G;
  const int wpos_hi = w_last >= w_first ? min(i0 + w_last / G, Lq - 1) : wpos_lo - 1;
  const int wave_kmax = wpos_hi >= wpos_lo ? max(0, min(kmax, wpos_hi + off + 1)) : 0;
  const int wave_full = wpos_lo + off + 1;  // keys below this are visible to every row of the wave
  const int limit = pos < 0 ? -1 : min(pos + off, kmax - 1);  // last key this row sees

  f32x16 acc[NJD];  // O^T, head dims 32 jd + 8 b + 4 h + r of row n
#pragma unroll
  for (int jd = 0; jd < NJD; ++jd) acc[jd] = f32x16{};
  float m_run = 0.f;  // row maximum (log2 units); scores leave the QK product relative to it
  f32x16 negm = f32x16{};  // -m_run in every register: the C operand of the QK chain
  float l_run[2] = {0.f, 0.f};  // this lane's half of the row sum, two dot2 chains
  const float sl2 = p.scale_log2;

  // Per-lane LDS byte offsets of the MFMA operand reads inside a stage; the
  // 32-key half (sub), PV MFMA (u) and 4-key block (eb) add constants.
  //   K: row n + 32 sub, piece (2 ks + h) ^ k_swz(row)
  //   V: row 16u + 8eb + 4h + j/4 + 32 sub (j = lane % 16),
  //      chunk (2 jd + (lane/16 & 1)) ^ v_swz(j/4), byte 8 (j % 4)
  int kaddr[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) kaddr[ks] = n * RB + ((2 * ks + h) ^ Gm::k_swz(n)) * 16;
  const int jl = lane & 15;
  int vaddr[NJD];
#pragma unroll
  for (int jd = 0; jd < NJD; ++jd)
    vaddr[jd] = Gm::kVRing + (4 * h + (jl >> 2)) * RB +
                ((2 * jd + ((lane >> 4) & 1)) ^ Gm::v_swz(jl >> 2)) * 32 + 8 * (jl & 3);

  const ItemStaging<PAGED, D> stg(p, item);
  (void)s;
  (void)k_start;
  (void)kvh;

  // S^T = K . Q^T for the 32 keys at `sb`: one accumulation chain over the
  // head dims (dependent MFMAs of one shape issue back to back).
  auto k_read = [&](const char* sb, bf16x8 (&kr)[NKS]) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) kr[ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(sb + kaddr[ks]));
  };
  auto qk_mfma = [&](const bf16x8 (&kr)[NKS], f32x16& sacc) {
    sacc = mfma32x32x16(kr[0], qop[0], negm);
#pragma unroll
    for (int ks = 1; ks < NKS; ++ks) sacc = mfma32x32x16(kr[ks], qop[ks], sacc);
  };
  auto qk = [&](const char* sb, f32x16& sacc) {
    bf16x8 kr[NKS];
    k_read(sb, kr);
    qk_mfma(kr, sacc);
  };

  // One 32-key step: softmax of the scores s_cur of keys key0 .. key0+31
  // and O^T += V^T P^T with V from `sb_v`; the QK MFMAs of the following step
  // (keys at `sb_next`) are issued in between, so the matrix pipe works on
  // them while the VALU does the exponentials.  After the last tile there is
  // no following step: they still read `sb_next`, the ring stage after the
  // last tile (no copy writes it then, so the stale read is harmless), and
  // their result is unused.  Reading it unconditionally keeps the block
  // branch-free and every operand address a base plus an immediate (choosing
  // between two stages cost a VALU add per K read: 2.5% at config 4).
  auto step = [&](f32x16& sv, f32x16& s_next, int key0, const char* sb_v, const char* sb_next) {
    if (key0 < wave_kmax) {  // otherwise every key of this step is masked for this wave
      // K operands of the following QK, read first so that they have landed
      // by the time its MFMAs issue between the exponentials
      bf16x8 kr[NKS];
      k_read(sb_next, kr);
      if (key0 + 32 > wave_full || key0 + 32 > kmax) {
        // score i is key key0 + 4h + c_i (c_i = 8 (i / 4) + i % 4): it stays
        // when c_i <= limit - key0 - 4h, one compare against an immediate each
        const int rel = limit - key0 - 4 * h;
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = 8 * (i >> 2) + (i & 3) <= rel ? sv[i] : kNegInf;
      }
      float mx = sv[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sv[i]);
      // Lazy maximum, shared by the two lanes holding a row (n and n + 32): it
      // moves only when a score exceeds it by more than kTau.  Each lane first
      // checks only its own 16 scores; the cross-lane maximum and the rescale
      // run only when some lane exceeds it (the first step, rare outliers).
      const bool first = key0 == 0;  // the first step sets the maximum
      if (first || __builtin_amdgcn_ballot_w64(mx > kTau)) {
        mx = max_across_halves(mx);
        const bool grow = first ? mx > kNegInf : mx > kTau;  // the same in both lanes of a row
        const float delta = grow ? mx : 0.f;
        const float alpha = first ? 1.f : fast_exp2(-delta);  // nothing accumulated before the first step
        l_run[0] *= alpha;
        l_run[1] *= alpha;
#pragma unroll
        for (int jd = 0; jd < NJD; ++jd) acc[jd] *= alpha;
        m_run += delta;
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] -= delta;
        negm = f32x16{} - m_run;
      }
      qk_mfma(kr, s_next);
      const bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
      bf16x8 pop[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        u32x4 pw;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          const float a = fast_exp2(sv[8 * u + 2 * q2]);
          const float b = fast_exp2(sv[8 * u + 2 * q2 + 1]);
          // The row sum adds the rounded probabilities the PV product uses,
          // two at a time (v_dot2 against (1, 1)).  The dot2 takes the bf16
          // pair itself: this compiler misselects the register when its
          // operand is a bitcast element of a 4-dword vector.
          const bf16x2 pb = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
          pw[q2] = __builtin_bit_cast(uint32_t, pb);
          l_run[q2 & 1] = __builtin_amdgcn_fdot2_f32_bf16(pb, ones, l_run[q2 & 1], false);
        }
        pop[u] = as_bf16x8(pw);
      }
      // V^T operands: head dims 32 jd .. +31 of PV MFMA u's 16 keys
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int jd = 0; jd < NJD; ++jd) {
          const bf16x8 vt = read_tr_pair(sb_v + vaddr[jd] + 16 * RB * u, sb_v + vaddr[jd] + 16 * RB * u + 8 * RB);
          acc[jd] = mfma32x32x16(vt, pop[u], acc[jd]);
        }
    }
  };

  // Tile `it` (in stage `cur`, tile it+1 in `nxt`): step over its first 32
  // keys; wait for this wave's copy of tile it+1 (issued two tiles ago) and
  // synchronise, after which every wave is done with tile it-1 and tile it+1
  // is visible; start the copy of tile it+3 into the stage `fill` that tile
  // it-1 left; then step over the last 32 keys while the QK of tile it+1's
  // first step issues.  Copies thus have two tiles of math to land.
  // Scores ping-pong between two buffers: the first step of a tile reads s0
  // and issues the QK of the second into s1, which issues the next tile's into s0.
  f32x16 s0 = f32x16{}, s1 = f32x16{};
  // Cursor over the tiles still to copy (from tile 2 on): c_ptr is the first
  // key of the next one.  Inside a page it moves by one tile of rows; at a
  // page boundary it takes the page id read one page earlier (a block id
  // outside the pool redirects to slot 0).  Block sizes are multiples of 64,
  // so a tile never straddles two pages, and the loop needs no division and
  // no 64-bit multiply per tile.
  const int64_t tile_step = static_cast<int64_t>(kBK) * stg.dstride * 2;
  const int tpp = PAGED ? p.block_size / kBK : 1;  // tiles per page
  const uint32_t nb32 = p.num_blocks > 0x7fffffff ? 0x7fffffffu : static_cast<uint32_t>(p.num_blocks);
  auto page_at = [&](int idx) { return idx < stg.mb ? stg.bt[idx] : -1; };
  auto page_base = [&](int page) {
    const int64_t slot = static_cast<uint32_t>(page) < nb32 ? static_cast<int64_t>(page) * p.block_size : 0;
    return reinterpret_cast<const char*>(stg.dbase + slot * stg.dstride);
  };
  int c_pg = PAGED ? 2 / tpp : 0;        // block-table index of the next tile's page
  int c_left = PAGED ? tpp - 2 % tpp : 0;  // tiles of that page from the next one on
  int c_next = PAGED ? page_at(c_pg + 1) : 0;
  const char* c_ptr = PAGED ? page_base(page_at(c_pg)) + (2 % tpp) * tile_step
                            : reinterpret_cast<const char*>(stg.dbase + (static_cast<int64_t>(item.k_start) + 2 * kBK) * stg.dstride);
  auto advance = [&]() {
    if constexpr (PAGED) {
      if (--c_left > 0) {
        c_ptr += tile_step;
      } else {
        ++c_pg;
        c_left = tpp;
        c_ptr = page_base(c_next);
        c_next = page_at(c_pg + 1);  // scalar load, a page of tiles ahead of its use
      }
    } else {
      c_ptr += tile_step;
    }
  };
  auto tile_iter = [&](int it, const char* cur, const char* nxt, char* fill) {
    const int kb = it * kBK;
    step(s0, s1, kb, cur, cur + 32 * RB);
    if (it + 2 < ntiles)
      wait_vmem<P>();  // tile it+2's copy may stay in flight
    else
      wait_vmem<0>();
    barrier_lds();
    // tile it+3's copy in two halves, one on each side of the second step, so
    // its LDS writes do not all land at once among the operand reads
    const char* src3 = c_ptr;
    if (it + 3 < ntiles) {
      stg.template copy_part<0, P / 2>(item, fill, src3, it + 3);
      advance();
    }
    step(s1, s0, kb + 32, cur + 32 * RB, nxt);
    if (it + 3 < ntiles) stg.template copy_part<P / 2, P>(item, fill, src3, it + 3);
  };

  // prologue: tiles 0 and 1 (copies issued before this call) and the Q
  // operands landed and visible; tile 2's copy starts after the barrier; the
  // first QK is issued
  wait_vmem<0>();
  // Q scaled by softmax_scale * log2(e) once per item: the QK product is then
  // in the exp2 domain
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    u32x4 wq = as_u32x4(qop[ks]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wq[j] = pack_bf16x2(__builtin_bit_cast(float, wq[j] << 16) * sl2, __builtin_bit_cast(float, wq[j] & 0xffff0000u) * sl2);
    qop[ks] = as_bf16x8(wq);
  }
  // The scaling above is an unconditional use of the Q operands, so the
  // compiler's own wait for their loads lands here.  Its only other use before the loop is conditional, and
  // the compiler would then keep those loads pending into the loop and wait
  // for all vector memory there -- which, unknown to it, also drains the tile
  // copies in flight -- on every step.
  barrier_lds();
  if (2 < ntiles) {
    stg.template copy_part<0, P>(item, stage(2), c_ptr, 2);
    advance();
  }
  if (0 < wave_kmax) qk(stage(0), s0);
  // unrolled over the ring's stages, so the stage offsets are immediates
  for (int it0 = 0; it0 < ntiles; it0 += kStages) {
#pragma unroll
    for (int t = 0; t < kStages; ++t) {
      const int it = it0 + t;
      if (it >= ntiles) break;
      tile_iter(it, stage(t), stage(t + 1), stage(t + 3));
    }
  }

  // ---- epilogue: normalise, transpose through LDS, write whole rows --------
  // The next item's Q operands first: the last QK has been issued, so qop is
  // free, and the loads have the epilogue to land.
  if (next.valid) item_fetch_q<D>(p, next, qop);
  float l = sum_across_halves(l_run[0] + l_run[1]);
  if constexpr (SPLIT) {
    if (item.split_slot >= 0 && !merge_key_halves<D>(p, smem_all, item.split_slot, acc, m_run, l)) return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  barrier_lds();  // every wave is done with the ring
  // stages 0 and 1 take the next item's first tiles
  if (next.valid) item_fetch_tiles<PAGED, D>(p, smem_all, next);
  // A work-queue grid claims the item after `next` here, one item ahead; the
  // caller reads the result after its own barrier, once the epilogue has run.
  if (claim_ctr != nullptr && next.valid && threadIdx.x == 0) claim = atomicAdd(claim_ctr, 1u);
  // Each wave owns 32 rows in ring stages 2 and 3 (waves 0..3 in the K half,
  // 4..7 in the V half, two waves per tile): row n at n * RB, 16-byte chunk c
  // (dims 8c .. 8c+7) at position c ^ k_swz(n).  Read back, KP consecutive
  // lanes cover one row, so every store writes whole lines.
  static_assert(2 * kRowsPerWave == kBK, "two waves' rows fill one tile");
  char* ot = smem_all + (w >> 2) * Gm::kVRing + (2 + ((w >> 1) & 1)) * Gm::kTileBytes + (w & 1) * kRowsPerWave * RB;
#pragma unroll
  for (int jd = 0; jd < NJD; ++jd)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      u32x2 o;
      o[0] = pack_bf16x2(acc[jd][4 * b] * inv, acc[jd][4 * b + 1] * inv);
      o[1] = pack_bf16x2(acc[jd][4 * b + 2] * inv, acc[jd][4 * b + 3] * inv);
      const int c = 4 * jd + b;
      *reinterpret_cast<u32x2*>(ot + n * RB + ((c ^ Gm::k_swz(n)) * 16) + 8 * h) = o;
    }
  const int c = lane & (KP - 1);
#pragma unroll
  for (int i = 0; i < KP / 2; ++i) {
    const int rr = (64 / KP) * i + lane / KP;  // row within the wave
    const int r2 = 32 * w + rr;
    const int qp2 = i0 + r2 / G;
    const u32x4 v = *reinterpret_cast<const u32x4*>(ot + rr * RB + ((c ^ Gm::k_swz(rr)) * 16));
    if (r2 < nrows && qp2 < Lq) {
      uint16_t* dst = p.out + static_cast<int64_t>(q_start + qp2) * p.out_row_stride + (kvh * G + r2 % G) * D + 8 * c;
      st16(dst, v);
    }
  }
}

// Direct grid: x = (sequence, kv head), y = query tile, heaviest tiles first.
// Workgroup id x + y * gridDim.x keeps every tile of one (sequence, kv head)
// on the same XCD (and its L2) whenever gridDim.x is a multiple of 8.  Tiles
// past a sequence's end exit at once.  Used when the persistent grid's tables
// would not fit its LDS.
template <bool PAGED, int D>
__global__ __launch_bounds__(64 * kWaves) void varlen_prefill_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(1024))) char smem_all[kStages * Geom<D>::kStageBytes];
  int s, kvh, tile, half = 0, pair = -1;
  if (p.split_tiles > 0) {
    // key halving: the compact grid (the real items first, heaviest first;
    // one kv head's items on one XCD when num_kv_heads is a multiple of 8),
    // or the plain one when nothing can split
    const CellItem ci = compact_cell(p, static_cast<int>(blockIdx.x));
    if (ci.s < 0) return;
    s = ci.s;
    kvh = ci.kvh;
    tile = ci.t;
    half = ci.half;
    pair = ci.pair;
  } else {
    s = blockIdx.x / p.num_kv_heads;
    kvh = blockIdx.x - s * p.num_kv_heads;
    tile = p.num_q_tiles - 1 - static_cast<int>(blockIdx.y);
  }
  ItemDesc it = item_desc(p, p.cu_q, p.cu_k, s, kvh, tile);
  if (!it.valid) return;
  if (pair >= 0) key_half<PAGED>(p, it, half, pair * p.num_kv_heads + kvh);
  bf16x8 qop[D / 16];
  item_fetch_q<D>(p, it, qop);
  item_fetch_tiles<PAGED, D>(p, smem_all, it);
  ItemDesc none{};
  none.valid = false;
  uint32_t unused = 0;
  prefill_run<PAGED, D, true>(p, smem_all, it, qop, none, nullptr, unused);
}

// Persistent grid: one workgroup per CU walks the real work items.
//
// A grid with one workgroup per (sequence, kv head, query tile) also holds the
// tiles past the shorter sequences' ends; they exit at once, but a workgroup
// dispatcher that waits for a particular busy CU then leaves other CUs idle
// for a whole workgroup's duration (measured: half the CUs idle for the first
// ~40 us of config 4).  Here every workgroup copies cu_seqlens_q/k into LDS
// (so locating an item needs no global load, whose scalar-cache wait would
// also hold up the LDS waits around it) and builds the same table of real
// items from them -- item order: query tile index descending (the
// heavier tiles first), then sequence, then kv head -- and takes items
// g, then 2 NW - 1 - g, ... (a snake over the NW workgroups, which balances
// their totals).  Workgroup g = 8 m + x runs on XCD x, and the snake reverses
// m only, so one kv head's items stay on one XCD (and its L2) when
// num_kv_heads is 8.
//
// With a work queue (p.queue) the order after the first item is dynamic
// instead: lane x = g % 8 (the XCD) owns items 8 k + x, its workgroups start
// with k = g / 8 and then claim k = NW / 8 + queue[x]++, each claim issued in
// the previous item's epilogue so its latency is hidden.  A workgroup that
// meets a slow CU or a heavy item simply claims fewer; a static order cannot
// adapt (measured per-workgroup end times spread over ~75 us of ~225 us at
// config 4).  The last workgroup to finish (queue[8] counts them) zeroes the
// queue, so every completed launch leaves it as it found it.
constexpr int kPersistMaxSeqs = 1024;
constexpr int kPersistMaxTiles = 1024;
constexpr int kThreads = 64 * kWaves;

// The rank-th sequence (ascending, 0-based) with more than t query tiles, or
// -1.  Every wave computes it on its own (ballots over 64 sequences at a time),
// so the lookup needs no workgroup barrier and the result is wave-uniform.
__device__ __forceinline__ int find_seq(const int* s_ntq, int S, int t, int rank) {
  const int lane = threadIdx.x & 63;
  for (int c0 = 0; c0 < S; c0 += 64) {
    const int sq = c0 + lane;
    const bool f = sq < S && s_ntq[sq] > t;
    const uint64_t m = __builtin_amdgcn_ballot_w64(f);
    const int cnt = __builtin_popcountll(m);
    if (rank < cnt) {
      const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
      const uint64_t hit = __builtin_amdgcn_ballot_w64(f && below == rank);
      return c0 + static_cast<int>(__builtin_ctzll(hit));
    }
    rank -= cnt;
  }
  return -1;
}

template <bool PAGED, int D, bool QUEUE>
__global__ __launch_bounds__(64 * kWaves) void varlen_prefill_persistent_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(1024))) char smem_all[kStages * Geom<D>::kStageBytes];
  __shared__ int s_ntq[kPersistMaxSeqs];           // query tiles of each sequence
  __shared__ int s_start[kPersistMaxTiles + 1];    // first item of each tile level (level T_max: total)
  __shared__ int s_cu[2][kPersistMaxSeqs + 1];     // cu_seqlens_q and cu_seqlens_k
  __shared__ uint32_t s_claim;                     // the queue claim, broadcast by thread 0
  const int tid = threadIdx.x;
  const int S = p.num_seqs;
  const int T = p.num_q_tiles;
  const int BP = p.positions_per_tile;
  const int nkv = p.num_kv_heads;
  constexpr int L = kPrefillQueueLanes;
  const int NW = static_cast<int>(gridDim.x);
  const int g = static_cast<int>(blockIdx.x);
  // QUEUE: the launch guarantees NW % 8 == 0, so lane x is the XCD
  const int x = g % L;
  uint32_t* const claim_ctr = QUEUE ? p.queue + x : nullptr;
  // The first claim goes out before the table is built, so its round trip
  // overlaps the cu_seqlens loads (config 4: 203.2 -> 201.9 us).  A workgroup
  // with no first item claims only indices >= NW, past every real item, so
  // nothing it claims is lost.
  uint32_t claim = 0;
  if (QUEUE && tid == 0) claim = atomicAdd(claim_ctr, 1u);

  // level table: cnt[t] = #{s : ntq_s > t}; items of level t (query tile t of
  // those sequences, all kv heads) start at s_start[t] = nkv * sum_{t' > t} cnt[t']
  for (int i = tid; i <= T; i += kThreads) s_start[i] = 0;
  for (int i = tid; i <= S; i += kThreads) {
    s_cu[0][i] = p.cu_q[i];
    s_cu[1][i] = p.cu_k[i];
  }
  __syncthreads();
  for (int i = tid; i < S; i += kThreads) {
    const int lq = s_cu[0][i + 1] - s_cu[0][i];
    const int nt = lq > 0 ? min((lq + BP - 1) / BP, T) : 0;
    s_ntq[i] = nt;
    if (nt > 0) atomicAdd(&s_start[nt - 1], 1);  // histogram of ntq (bin nt - 1)
  }
  __syncthreads();
  if (tid < 64) {
    // suffix sums over the levels in chunks of C per lane: first cnt[t] =
    // sum_{k >= t} hist[k], then start[t] = nkv * sum_{t' > t} cnt[t']
    const int lane = tid;
    constexpr int C = kPersistMaxTiles / 64;
    for (int pass = 0; pass < 2; ++pass) {
      int local = 0;
      for (int k = 0; k < C; ++k) {
        const int t = lane * C + k;
        local += t < T ? s_start[t] : 0;
      }
      // exclusive suffix over lanes (lanes above this one)
      int suf = local;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int src = lane + d < 64 ? lane + d : lane;
        const int x = __builtin_amdgcn_ds_bpermute(src << 2, suf);
        if (lane + d < 64) suf += x;
      }
      int acc = suf - local;  // sum over t beyond this lane's chunk
      for (int k = C - 1; k >= 0; --k) {
        const int t = lane * C + k;
        if (t < T) {
          const int v = s_start[t];
          if (pass == 0) {
            acc += v;
            s_start[t] = acc;  // inclusive: cnt[t]
          } else {
            s_start[t] = nkv * acc;  // exclusive: start[t]
            acc += v;
          }
        }
      }
      if (pass == 1 && lane == 0) s_start[T] = nkv * (suf);  // total items
    }
  }
  __syncthreads();
  const int total = s_start[T];
  // Table item `item` (every item below `total` is a real tile: its sequence
  // has more than t query tiles), or an invalid descriptor past the end.
  auto desc_of = [&](int item) {
    if (item >= total) return item_desc(p, s_cu[0], s_cu[1], -1, 0, 0);
    // level t: the smallest t with start[t] <= item (start decreases in t)
    int lo = 0, hi = T - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (__builtin_amdgcn_readfirstlane(s_start[mid]) <= item) hi = mid;
      else lo = mid + 1;
    }
    const int t = lo;
    const int j = item - __builtin_amdgcn_readfirstlane(s_start[t]);
    const int rank = j / nkv;
    const int kvh = j - rank * nkv;
    return item_desc(p, s_cu[0], s_cu[1], find_seq(s_ntq, S, t, rank), kvh, t);
  };
  auto finish = [&]() {
    if (QUEUE && tid == 0 &&
        atomicAdd(p.queue + kPrefillQueueLanes, 1u) == static_cast<uint32_t>(NW - 1)) {
      for (int y = 0; y < kPrefillQueueWords; ++y) atomicExch(p.queue + y, 0u);
    }
  };
  ItemDesc cur = desc_of(g);  // round 0 of either order
  if (!cur.valid) {
    finish();
    return;
  }
  bf16x8 qop[D / 16];
  item_fetch_q<D>(p, cur, qop);
  item_fetch_tiles<PAGED, D>(p, smem_all, cur);
  for (int round = 1;; ++round) {
    // the next item is located (from the LDS tables) while this one's
    // first copies are in flight; its own first copies start in this one's
    // epilogue
    ItemDesc nxt;
    if (QUEUE) {
      if (tid == 0) s_claim = claim;
      __syncthreads();
      nxt = desc_of(L * (NW / L + static_cast<int>(__builtin_amdgcn_readfirstlane(s_claim))) + x);
    } else {
      const int q = (round & 1) ? (NW % 8 == 0 ? 8 * (NW / 8 - 1 - g / 8) + g % 8 : NW - 1 - g) : g;
      const int64_t item64 = static_cast<int64_t>(round) * NW + q;
      nxt = desc_of(item64 < total ? static_cast<int>(item64) : total);
    }
    prefill_run<PAGED, D, false>(p, smem_all, cur, qop, nxt, claim_ctr, claim);
    if (!nxt.valid) break;
    cur = nxt;
  }
  finish();
}


int prefill_positions_per_tile(int group) { return group >= 1 && group <= kRows ? kRows / group : 1; }

// Compute units of the current device (cached per device).
static int device_cu_count() {
  static int counts[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

// Key halving of the direct grid (with a workspace): with at most
// two grid cells per CU, the longest items set the launch's length while CUs
// sit idle.  Items of at least kSplitNum / kSplitDen of the longest key span
// (and at least kSplitMin tiles) then run as two key halves, on the compact
// grid (compact_cell).
constexpr int kSplitNum = 3;
constexpr int kSplitDen = 5;
constexpr int kSplitMin = 8;
constexpr int kSplitMaxPageTiles = 8;  // paged key halving for block sizes up to 512

hipError_t launch_prefill(const PrefillParams& p0, int max_seqlen_q, int max_seqlen_k, hipStream_t stream) {
  if (p0.num_seqs <= 0 || max_seqlen_q <= 0) return hipSuccess;
  PrefillParams p = p0;
  p.positions_per_tile = prefill_positions_per_tile(p.group);
  p.num_q_tiles = (max_seqlen_q + p.positions_per_tile - 1) / p.positions_per_tile;
  // Persistent grid when there are enough items to balance; with at most two
  // per CU its table set-up (one more dependent global load and a few
  // barriers) costs more than it saves (measured on config 2).
  const int64_t max_items = static_cast<int64_t>(p.num_seqs) * p.num_kv_heads * p.num_q_tiles;
  const int cus = device_cu_count();
  if (p.num_seqs <= kPersistMaxSeqs && p.num_q_tiles <= kPersistMaxTiles && max_items > 2 * int64_t{cus}) {
    // one workgroup per CU (the ring takes most of a CU's LDS); the work queue
    // needs whole XCD lanes
    const unsigned nw = static_cast<unsigned>(cus);
    const dim3 grid(nw);
    const bool queue = p.queue != nullptr && nw % kPrefillQueueLanes == 0;
#define NVA_PERSIST(PG, DD)                                                                                  \
  do {                                                                                                       \
    if (queue)                                                                                               \
      hipLaunchKernelGGL((varlen_prefill_persistent_kernel<PG, DD, true>), grid, dim3(kThreads), 0, stream, p); \
    else                                                                                                     \
      hipLaunchKernelGGL((varlen_prefill_persistent_kernel<PG, DD, false>), grid, dim3(kThreads), 0, stream, p); \
  } while (0)
    if (p.head_dim == 64) {
      if (p.block_table) NVA_PERSIST(true, 64);
      else NVA_PERSIST(false, 64);
    } else {
      if (p.block_table) NVA_PERSIST(true, 128);
      else NVA_PERSIST(false, 128);
    }
#undef NVA_PERSIST
    return hipGetLastError();
  }
  // max_seqlen_k only sizes the cut: a wrong value changes which items are
  // split, never the result beyond rounding
  const int64_t kt_max = (std::max<int64_t>(max_seqlen_k, 0) + kBK - 1) / kBK;
  p.split_tiles = 0;
  p.split_slots = kPrefillSplitSlots;
  p.split_cus = cus;
  const int64_t pairs_split = kPrefillSplitSlots / p.num_kv_heads;  // at most this many pairs split
  // paged: the halves meet at a page boundary, so only items of at least two
  // pages' tiles split (tpp tiles per page; pages of at most kSplitMaxPageTiles)
  const int tpp = p.block_table ? p.block_size / kBK : 1;
  if (p.split_ctl != nullptr && p.split_part != nullptr && max_items <= 2 * int64_t{cus} && kt_max >= kSplitMin &&
      pairs_split > 0 && tpp <= kSplitMaxPageTiles)
    p.split_tiles = static_cast<int>(
        std::max<int64_t>(std::max(kSplitMin, 2 * tpp), (kSplitNum * kt_max + kSplitDen - 1) / kSplitDen));
  // compact grid with key halving: every (sequence, tile) pair's position, one
  // more for each pair that may split
  const dim3 grid = p.split_tiles > 0
                        ? dim3(static_cast<unsigned>(max_items + pairs_split * p.num_kv_heads))
                        : dim3(static_cast<unsigned>(p.num_seqs * p.num_kv_heads), static_cast<unsigned>(p.num_q_tiles));
  if (p.head_dim == 64) {
    if (p.block_table)
      hipLaunchKernelGGL((varlen_prefill_kernel<true, 64>), grid, dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((varlen_prefill_kernel<false, 64>), grid, dim3(kThreads), 0, stream, p);
  } else {
    if (p.block_table)
      hipLaunchKernelGGL((varlen_prefill_kernel<true, 128>), grid, dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((varlen_prefill_kernel<false, 128>), grid, dim3(kThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace nva
