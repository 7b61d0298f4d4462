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
#include <type_traits>

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

// Raw loads of one 32-key step for one kv head (see the file comment for the
// lane layout).  bf16: K tile rows as 16-byte MFMA operands, 8 value rows of 8
// columns; fp8: the same positions, half the bytes.
template <bool FP8>
struct StepRegs;
template <>
struct StepRegs<false> {
  u32x4 k[2][4];
  u32x4 v[8];
};
template <>
struct StepRegs<true> {
  u32x4 k[2][2];
  u32x2 v[8];
};

typedef const __attribute__((address_space(4))) int32_t const_i32;

// Per-wave constants of a work item.
struct WaveItem {
  const char* kbase;      // k_cache + kv head offset (bytes)
  const char* vbase;
  int64_t slot_bytes;     // bytes between consecutive slots
  // Block table row of the sequence, read with ordinary loads: through the
  // constant address space (scalar loads) the balanced decode measured 2 us
  // slower at config 3.
  const int32_t* bt;
  int64_t num_blocks;
  int block_size;
  int k_begin;
  int k_end;
  int krow0;              // K tile row this lane supplies (tile 0)
  int n;                  // lane % 16
  int g;                  // lane / 16
};

// Slot of the first key of step i and how many of its 32 keys exist (0 when the
// block id is outside the pool: those keys stay masked and nothing is read from
// the bad page).  HOIST: lane j of bt_row holds block-table entry j (the whole
// row, read before the loop), so the step needs no dependent load.
template <bool HOIST = false>
__device__ __forceinline__ int64_t step_row(const WaveItem& w, int i, int& nvalid, int bt_row = 0) {
  const int key0 = w.k_begin + 32 * i;
  const int blk = key0 / w.block_size;
  const int page = HOIST ? __builtin_amdgcn_readlane(bt_row, blk) : w.bt[blk];
  const bool ok = page >= 0 && page < w.num_blocks;
  nvalid = ok ? min(32, w.k_end - key0) : 0;
  return static_cast<int64_t>(ok ? page : 0) * w.block_size + (key0 - blk * w.block_size);
}

// D = 64: two QK MFMAs per key tile, and only lanes n < 8 hold value columns
// (the other V^T rows are zero, so half of each PV MFMA is idle work).
template <bool FP8, int D>
__device__ __forceinline__ void load_step(StepRegs<FP8>& r, const WaveItem& w, int64_t row0) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const char* rp = w.kbase + (row0 + w.krow0 + 4 * t) * w.slot_bytes;
    if constexpr (!FP8) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s) r.k[t][s] = ld16_nt(rp + qk_dim<false>(s, w.g) * 2);
    } else {
#pragma unroll
      for (int u = 0; u < D / 64; ++u) r.k[t][u] = ld16_nt(rp + 64 * u + 16 * w.g);
    }
  }
  const bool has_cols = D == 128 || w.n < D / 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const char* rp = w.vbase + (row0 + 8 * w.g + i) * w.slot_bytes;
    if constexpr (!FP8)
      r.v[i] = has_cols ? ld16_nt(rp + 16 * w.n) : u32x4{0u, 0u, 0u, 0u};
    else
      r.v[i] = has_cols ? ld8_nt(rp + 8 * w.n) : u32x2{0u, 0u};
  }
}

// A step as two buffer resources (its 32 K rows and 32 V rows of this kv head)
// and its count of keys.  Rows past the last valid key, every row of a block
// id outside the pool and every row of a step past the segment's end lie
// outside the resource's records: their loads return zeros without touching
// memory.  Loads can thus be issued for steps that do not exist, so every
// path issues the same loads and the compiler's wait before a step's compute
// covers only that step's loads (a prefetch issued on one path only makes it
// wait for everything in flight).
struct StepRsrc {
  __amdgpu_buffer_rsrc_t k, v;
  int nvalid;
  int row0;  // cache slot of the step's first key (low 32 bits)
};

// Records covering rows [0, nvalid) of a step whose row 0 is at `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const char* base, int nvalid, int slot_bytes, int row_bytes) {
  const int records = nvalid > 0 ? (nvalid - 1) * slot_bytes + row_bytes : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, records, 0x00020000);
}

template <bool HOIST, int ROW_BYTES>
__device__ __forceinline__ StepRsrc step_rsrc(const WaveItem& w, int i, int nsteps, int bt_row) {
  StepRsrc r;
  int nvalid = 0;
  int64_t row0 = 0;
  if (i < nsteps) row0 = step_row<HOIST>(w, i, nvalid, bt_row);
  const int sb = static_cast<int>(w.slot_bytes);
  r.k = rows_rsrc(w.kbase + row0 * w.slot_bytes, nvalid, sb, ROW_BYTES);
  r.v = rows_rsrc(w.vbase + row0 * w.slot_bytes, nvalid, sb, ROW_BYTES);
  r.nvalid = nvalid;
  r.row0 = static_cast<int>(row0);
  return r;
}

// load_step through the step's buffer resources; lanes with no value columns
// (D = 64) read at an offset past every record.
template <bool FP8, int D>
__device__ __forceinline__ void load_step_buf(StepRegs<FP8>& r, const WaveItem& w, const StepRsrc& rs) {
  const int sb = static_cast<int>(w.slot_bytes);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int ro = (w.krow0 + 4 * t) * sb;
    if constexpr (!FP8) {
#pragma unroll
      for (int s = 0; s < D / 32; ++s)
        r.k[t][s] = __builtin_amdgcn_raw_buffer_load_b128(rs.k, ro + qk_dim<false>(s, w.g) * 2, 0, kBufNonTemporal);
    } else {
#pragma unroll
      for (int u = 0; u < D / 64; ++u)
        r.k[t][u] = __builtin_amdgcn_raw_buffer_load_b128(rs.k, ro + 64 * u + 16 * w.g, 0, kBufNonTemporal);
    }
  }
  const bool has_cols = D == 128 || w.n < D / 8;
  const int col = has_cols ? (FP8 ? 8 : 16) * w.n : 0x7fffffff - 32 * sb;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int off = (8 * w.g + i) * sb + col;
    if constexpr (!FP8)
      r.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs.v, off, 0, kBufNonTemporal);
    else
      r.v[i] = __builtin_amdgcn_raw_buffer_load_b64(rs.v, off, 0, kBufNonTemporal);
  }
}

// Online-softmax update of one step: scores, running max/sum, O^T += V^T P^T.
template <bool FP8, int D, bool ZERO_ROWS = true>
__device__ __forceinline__ void compute_step(StepRegs<FP8>& r, int nvalid, int g, const bf16x8 (&qop)[4],
                                             float sl2, f32x4 (&acc)[8], float& m_run, float& l_run) {
  if (ZERO_ROWS && nvalid < 32) {  // keys past the end (or on a bad page) contribute nothing
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (8 * g + i >= nvalid) {
        if constexpr (!FP8)
          r.v[i] = u32x4{0u, 0u, 0u, 0u};
        else
          r.v[i] = u32x2{0u, 0u};
      }
  }
  bf16x8 kop[2][4];
  if constexpr (!FP8) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < D / 32; ++s) kop[t][s] = as_bf16x8(r.k[t][s]);
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < D / 64; ++u) fp8x16_to_ops(r.k[t][u], kop[t][2 * u], kop[t][2 * u + 1]);
  }
  f32x4 st[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < D / 32; ++s) st[t] = mfma16x16x32(kop[t][s], qop[s], st[t]);
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
  const float m_new = fmaxf(m_run, mx);
  const float m_use = m_new == kNegInf ? 0.f : m_new;  // a step with no valid key changes nothing
  const float alpha = fast_exp2(m_run - m_use);
  m_run = m_new;
  float psum = 0.f;
  float pv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pv[i] = fast_exp2(sv[i] - m_use);
    psum += pv[i];
  }
  l_run = l_run * alpha + psum;
  u32x4 pw;
#pragma unroll
  for (int w = 0; w < 4; ++w) pw[w] = pack_bf16x2(pv[2 * w], pv[2 * w + 1]);
  const bf16x8 pop = as_bf16x8(pw);
  bf16x8 vt[8];
  if constexpr (!FP8)
    transpose_v_bf16(r.v, vt);
  else
    transpose_v_fp8(r.v, vt);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    acc[j] *= alpha;
    acc[j] = mfma16x16x32(vt[j], pop, acc[j]);
  }
}

// No register patch (every caller but the fused store).
struct NoPatch {
  template <class R>
  __device__ __forceinline__ void apply(R&, int, int) const {}
};

// The new token's key and value of one kv head, as this lane holds them in a
// step's registers (StepRegs layout), and where they go: local step `step`
// of the segment, row `row` of that step (step -1: nowhere).  The spread
// kernel with a fused store patches them into the step's freshly loaded
// registers instead of waiting for its own store to reach the cache.  The
// bf16 source pieces are kept as loaded; fp8 quantises them (as the store
// does) only in the patched step, so no wait for them precedes the step loads.
template <bool FP8, int D>
struct NewRow {
  static constexpr int NK = D / 32;  // 16-byte bf16 source pieces of the key row per lane
  int step = -1;     // local step holding the new key (-1: none)
  int row = 0;       // its row in that step
  int slot = -1;     // the new token's slot (the pool has fewer than 2^31 slots)
  float ks = 1.f, vs = 1.f;
  u32x4 k[NK];
  u32x4 v;

  // Source pieces for lane (n, g): bf16 K dims qk_dim(s, g) .. +7 (bf16
  // cache) or 64 u + 16 g .. +15 (fp8 cache, pieces 2u and 2u+1); V columns
  // 8 n .. 8 n + 7.
  __device__ __forceinline__ void load(const uint16_t* kin, const uint16_t* vin, int n, int g, float kscale,
                                       float vscale) {
    ks = kscale;
    vs = vscale;
#pragma unroll
    for (int s = 0; s < NK; ++s)
      k[s] = ld16(kin + (FP8 ? 64 * (s >> 1) + 16 * g + 8 * (s & 1) : qk_dim<false>(s, g)));
    v = ld16(vin + 8 * (D == 128 || n < D / 8 ? n : 0));
  }

  // Registers of local step i, whose first key is at cache slot row0: the
  // K tile row `row` lives in lanes n = 4 (row / 8) + row % 4 (tile
  // t = row / 4 % 2), the V row in lanes g = row / 8 (register row % 8).  Only
  // a step that read the new token's slot is patched (slot_mapping[b] is then
  // the slot of key ctx-1, as every decode step produces it).
  __device__ __forceinline__ void apply(StepRegs<FP8>& r, int i, int row0) const {
    if (i != step || row0 + row != slot) return;
    // a side effect: the selects below stay behind the branch (if-converted,
    // they would run on every step of the loop)
    asm volatile("");
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int t = (row >> 2) & 1;
    const bool kl = n == 4 * (row >> 3) + (row & 3);
    const bool vl = g == (row >> 3);
    if constexpr (!FP8) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int s = 0; s < NK; ++s) r.k[tt][s] = (tt == t && kl) ? k[s] : r.k[tt][s];
      const u32x4 vv = D == 128 || n < D / 8 ? v : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int ii = 0; ii < 8; ++ii) r.v[ii] = (ii == (row & 7) && vl) ? vv : r.v[ii];
    } else {
      // the empty asm keeps the quantisation here (hoisted out of the step
      // loop, it would wait for the source loads before the first step's loads)
      u32x4 kk[NK];
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        kk[s] = k[s];
        asm volatile("" : "+v"(kk[s]));
      }
      u32x4 vr = v;
      asm volatile("" : "+v"(vr));
#pragma unroll
      for (int u = 0; u < D / 64; ++u) {
        const u32x2 lo = bf16x8_to_e4m3fn(kk[2 * u], ks);
        const u32x2 hi = bf16x8_to_e4m3fn(kk[2 * u + 1], ks);
        const u32x4 c = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) r.k[tt][u] = (tt == t && kl) ? c : r.k[tt][u];
      }
      const u32x2 vc = bf16x8_to_e4m3fn(vr, vs);
#pragma unroll
      for (int ii = 0; ii < 8; ++ii) r.v[ii] = (ii == (row & 7) && vl) ? vc : r.v[ii];
    }
  }
};

// One wave, one kv head: the unnormalised attention state of the head group's
// queries over keys [k_begin, k_end) of sequence b -- O^T in acc (lane (n, g):
// head n, columns 32g .. 32g+31), the running maximum m_run (log2 units) and
// the row sum `l` (summed over the four lanes of a head).
template <bool FP8, bool PREFETCH, int D, bool HOIST = false, bool BUF = false, class Patch = NoPatch>
__device__ __forceinline__ void segment_accumulate(const DecodeParams& p, int kvh, int b, int k_begin, int k_end,
                                                   f32x4 (&acc)[8], float& m_run, float& l, int bt_row = 0,
                                                   const Patch& patch = Patch{}) {
  constexpr int EB = FP8 ? 1 : 2;  // bytes per cache element
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int h = kvh * p.group + n;
  const bool head_ok = n < p.group;

  WaveItem w;
  w.slot_bytes = static_cast<int64_t>(p.num_kv_heads) * D * EB;
  w.kbase = static_cast<const char*>(p.k_cache) + static_cast<int64_t>(kvh) * D * EB;
  w.vbase = static_cast<const char*>(p.v_cache) + static_cast<int64_t>(kvh) * D * EB;
  w.bt = p.block_table + b * p.bt_row_stride;
  w.num_blocks = p.num_blocks;
  w.block_size = p.block_size;
  w.k_begin = k_begin;
  w.k_end = k_end;
  w.krow0 = 8 * (n >> 2) + (n & 3);  // K tile row n of tile t holds key 8*(n/4) + 4*t + n%4
  w.n = n;
  w.g = g;

  // Q^T operand: head n, 8 contraction elements per MFMA.
  bf16x8 qop[4];
  {
    const uint16_t* qrow = p.q + b * p.q_row_stride + h * D;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      qop[s] = as_bf16x8(head_ok ? ld16(qrow + qk_dim<FP8>(s, g)) : z);
    }
  }
  const float sl2 = FP8 ? p.scale_log2 * p.k_scale[kvh] : p.scale_log2;

#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  m_run = kNegInf;
  float l_run = 0.f;

  // Two register buffers: with PREFETCH the loads of step i+1 are in flight
  // while step i is computed.
  const int nsteps = (k_end - k_begin + 31) >> 5;
  if (BUF && nsteps > 0) {
    // two steps in flight: step i+1's loads go out before step i is computed,
    // step i+2's before step i+1 (past the end they return zeros).  With a
    // patch (only ever of the last step) the loop stops one step short and the
    // last step, already loaded into A or B by it, is patched and computed
    // after it: inside the loop the patch's branch would move the waits for
    // each step's loads to the step's start.
    constexpr int RB = D * EB;
    StepRegs<FP8> A, B;
    StepRsrc ra = step_rsrc<HOIST, RB>(w, 0, nsteps, bt_row);
    load_step_buf<FP8, D>(A, w, ra);
    if constexpr (std::is_same<Patch, NoPatch>::value) {
      for (int i = 0; i < nsteps; i += 2) {
        const StepRsrc rb = step_rsrc<HOIST, RB>(w, i + 1, nsteps, bt_row);
        load_step_buf<FP8, D>(B, w, rb);
        compute_step<FP8, D, false>(A, ra.nvalid, g, qop, sl2, acc, m_run, l_run);
        ra = step_rsrc<HOIST, RB>(w, i + 2, nsteps, bt_row);
        load_step_buf<FP8, D>(A, w, ra);
        if (i + 1 < nsteps) compute_step<FP8, D, false>(B, rb.nvalid, g, qop, sl2, acc, m_run, l_run);
      }
    } else {
      const int nloop = nsteps - 1;
      StepRsrc rb = ra;
      for (int i = 0; i < nloop; i += 2) {
        rb = step_rsrc<HOIST, RB>(w, i + 1, nsteps, bt_row);
        load_step_buf<FP8, D>(B, w, rb);
        compute_step<FP8, D, false>(A, ra.nvalid, g, qop, sl2, acc, m_run, l_run);
        ra = step_rsrc<HOIST, RB>(w, i + 2, nsteps, bt_row);
        load_step_buf<FP8, D>(A, w, ra);
        if (i + 1 < nloop) compute_step<FP8, D, false>(B, rb.nvalid, g, qop, sl2, acc, m_run, l_run);
      }
      // step nloop: in A when nloop is even (loaded as step i + 2 of the last
      // iteration, or before the loop), else in B (step i + 1)
      if ((nloop & 1) == 0) {
        patch.apply(A, nloop, ra.row0);
        compute_step<FP8, D, false>(A, ra.nvalid, g, qop, sl2, acc, m_run, l_run);
      } else {
        patch.apply(B, nloop, rb.row0);
        compute_step<FP8, D, false>(B, rb.nvalid, g, qop, sl2, acc, m_run, l_run);
      }
    }
  } else if (nsteps > 0) {
    StepRegs<FP8> A, B;
    int nvA = 0, nvB = 0;
    load_step<FP8, D>(A, w, step_row<HOIST>(w, 0, nvA, bt_row));
    for (int i = 0; i < nsteps; i += 2) {
      const bool has1 = i + 1 < nsteps;
      const bool has2 = i + 2 < nsteps;
      if (PREFETCH && has1) load_step<FP8, D>(B, w, step_row<HOIST>(w, i + 1, nvB, bt_row));
      compute_step<FP8, D>(A, nvA, g, qop, sl2, acc, m_run, l_run);
      if (has1) {
        if (!PREFETCH) load_step<FP8, D>(B, w, step_row<HOIST>(w, i + 1, nvB, bt_row));
        if (PREFETCH && has2) load_step<FP8, D>(A, w, step_row<HOIST>(w, i + 2, nvA, bt_row));
        compute_step<FP8, D>(B, nvB, g, qop, sl2, acc, m_run, l_run);
      }
      if (!PREFETCH && has2) load_step<FP8, D>(A, w, step_row<HOIST>(w, i + 2, nvA, bt_row));
    }
  }

  l = l_run;
  l += shfl_xor(l, 16);
  l += shfl_xor(l, 32);
}

__device__ __forceinline__ int clamped_len(const DecodeParams& p, int b) {
  const int ctx = p.seqlens[b];
  const int cap = p.max_blocks * p.block_size;
  return ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
}

// One wave, one kv head: attention of the head group's queries over keys
// [k_begin, k_end) of sequence b.  Writes the normalised output when `direct`,
// otherwise the unnormalised partial (O * v_scale, running max, sum) at `slot`.
// STORE: the segment holding key ctx-1 also stores the new token's K and V
// rows of this kv head at slot_mapping[b], after its own steps, and -- when
// that slot is key ctx-1's (what every decode step produces) -- patches the
// rows into its registers in place of the stale ones it loaded, so the result
// equals store-then-decode without waiting for the store (no other segment
// reads key ctx-1).
template <bool FP8, bool PREFETCH, int D, bool BUF = false, bool STORE = false>
__device__ __forceinline__ void decode_segment(const DecodeParams& p, int kvh, int b, int k_begin, int k_end,
                                               bool direct, int64_t slot, int ctx = 0) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int h = kvh * p.group + n;
  const bool head_ok = n < p.group;
  f32x4 acc[8];
  float m_run, l;
  if constexpr (STORE) {
    // ctx: the sequence's (clamped) length; the segment ending at ctx holds
    // key ctx-1.  slot_mapping[b] is read with a scalar load (constant address
    // space); it is needed only at the last step and for the store.
    const bool holder = ctx > 0 && k_end == ctx;
    if (holder) {
      NewRow<FP8, D> nr;
      // lanes 0..D/8-1 store the key row, lanes 32.. the value row, 8 elements each
      const int j = lane & 31;
      const bool is_v = lane >= 32;
      const uint16_t* kin = p.new_k + b * p.new_k_stride + kvh * D;
      const uint16_t* vin = p.new_v + b * p.new_v_stride + kvh * D;
      nr.load(kin, vin, n, g, FP8 ? p.k_scale[kvh] : 1.f, FP8 ? p.v_scale[kvh] : 1.f);
      const u32x4 x = ld16((is_v ? vin : kin) + 8 * (j & (D / 8 - 1)));
      nr.step = ((ctx - 1) >> 5) - (k_begin >> 5);
      nr.row = (ctx - 1) & 31;
      const int64_t nslot = ((const_i32*)p.slot_mapping)[b];
      // an invalid slot matches no row0 + row, so nothing is patched
      nr.slot = static_cast<int>(nslot);
      segment_accumulate<FP8, PREFETCH, D, false, BUF>(p, kvh, b, k_begin, k_end, acc, m_run, l, 0, nr);
      if (j < D / 8 && nslot >= 0 && nslot < static_cast<int64_t>(p.num_blocks) * p.block_size) {
        constexpr int EB = FP8 ? 1 : 2;
        char* dst = static_cast<char*>(const_cast<void*>(is_v ? p.v_cache : p.k_cache)) +
                    (nslot * p.num_kv_heads + kvh) * D * EB + 8 * j * EB;
        if constexpr (FP8)
          *reinterpret_cast<u32x2*>(dst) = bf16x8_to_e4m3fn(x, is_v ? p.v_scale[kvh] : p.k_scale[kvh]);
        else
          *reinterpret_cast<u32x4*>(dst) = x;
      }
    } else {
      segment_accumulate<FP8, PREFETCH, D, false, BUF>(p, kvh, b, k_begin, k_end, acc, m_run, l);
    }
  } else {
    segment_accumulate<FP8, PREFETCH, D, false, BUF>(p, kvh, b, k_begin, k_end, acc, m_run, l);
  }
  const float vscale = FP8 ? p.v_scale[kvh] : 1.0f;
  if (!head_ok || 32 * g >= D) return;  // lanes g >= D/32 hold no output columns
  if (direct) {
    const float inv = l > 0.f ? vscale / l : 0.f;
    uint16_t* orow = p.out + b * p.out_row_stride + h * D + 32 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 o;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) o[q2] = pack_bf16x2(acc[2 * q2][r] * inv, acc[2 * q2 + 1][r] * inv);
      st16(orow + 8 * r, o);
    }
  } else {
    const int64_t idx = slot * p.num_heads + h;
    float* wo = p.ws_o + idx * D + 32 * g;
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

// Launch shape per cache dtype, chosen by measurement on MI355X (config 3 /
// config 5 shapes): waves per workgroup (kv heads sharing a key range), whether
// the next step's loads are issued before the current step's math, and the
// total number of waves the balanced mode spreads the steps over.
//   bf16: 4 waves, prefetch (256 VGPRs, one wave per SIMD), 1024 waves
//   fp8 : 8 waves, no prefetch (half the bytes per step), 2048 waves
template <bool FP8>
struct DecodeShape;
template <>
struct DecodeShape<false> {
  static constexpr int kWaves = 4;
  static constexpr bool kPrefetch = true;
  static constexpr bool kBuf = true;  // buffer-resource steps, two in flight (-1.4% at config 3)
  static constexpr int kTargetWaves = 1024;
};
template <>
struct DecodeShape<true> {
  static constexpr int kWaves = 8;
  // buffer-resource steps, two in flight: with non-temporal loads, config 5 516.5 -> 508.6 us and
  // its TP8 share 84.6 -> 82.1 us (plain loads without prefetch had been 0.8% ahead before)
  static constexpr bool kPrefetch = true;
  static constexpr bool kBuf = true;
  static constexpr int kTargetWaves = 2048;
};

// ---------------------------------------------------------------------------
// Fixed split-K: workgroup = WAVES kv heads of one sequence over one split of
// keys_per_split keys.  Grid: (head groups, splits, batch).  Partial slot of
// split s of sequence b: b * num_splits + s.
// ---------------------------------------------------------------------------
template <bool FP8, int WAVES, bool PREFETCH, int D>
__global__ __launch_bounds__(64 * WAVES) void paged_decode_split_kernel(DecodeParams p) {
  const int kvh = blockIdx.x * WAVES + (threadIdx.x >> 6);
  if (kvh >= p.num_kv_heads) return;
  const int split = blockIdx.y;
  const int b = blockIdx.z;
  const int ctx = clamped_len(p, b);
  const int k_begin = split * p.keys_per_split;
  const int k_end = min(ctx, k_begin + p.keys_per_split);
  const bool direct = p.num_splits == 1;
  if (k_begin >= k_end && !direct) return;  // the merge reads only splits that hold keys
  decode_segment<FP8, PREFETCH, D>(p, kvh, b, k_begin, max(k_begin, k_end), direct,
                                   static_cast<int64_t>(b) * p.num_splits + split);
}

// ---------------------------------------------------------------------------
// Spread split-K for small batches: one wave per workgroup; workgroup
// (r, kvh, b) takes the r-th share of sequence b's 32-key steps.  One CU moves
// a step's 16 KiB slowly (about 16 bytes per cycle with eight waves loading,
// measured), so a small batch is spread over many CUs: S shares per
// (sequence, kv head), S = kSpreadTargetWaves / (batch * num_kv_heads) capped
// by the table's steps (plan_decode).  Shares are ceil(steps / S) steps; the
// S_b = ceil(steps / share) non-empty ones each write their partial
// (O * v_scale, max, sum) to slot b * S + r for decode_spread_merge_kernel.  A
// sequence with one share (or none: zeros) is written directly.  (Merging in
// this launch instead -- the last share to arrive on a device counter merges --
// measured slower: arrivals on one counter serialise at ~500 cycles each, and
// the release/acquire fences cost as much again.)  Grid: (S, num_kv_heads, batch).
// ---------------------------------------------------------------------------
// Steps per share and the number of non-empty shares of a sequence of `steps`
// steps cut into at most S shares.
__device__ __forceinline__ void spread_shares(int steps, int S, int& per, int& shares) {
  per = steps > 0 ? (steps + S - 1) / S : 1;
  shares = (steps + per - 1) / per;
}

template <bool FP8, int D, bool STORE>
__global__ __launch_bounds__(64) void paged_decode_spread_kernel(DecodeParams p) {
  const int r = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int S = p.spread;
  const int lane = threadIdx.x;
  // the whole block-table row (at most kWgMaxBlocks entries), read together
  // with the context length instead of one dependent read per step
  const int bt_row = lane < p.max_blocks ? p.block_table[b * p.bt_row_stride + lane] : -1;
  const int ctx = __builtin_amdgcn_readfirstlane(clamped_len(p, b));
  int per, shares;  // shares: the non-empty ones (0 for an empty sequence)
  spread_shares((ctx + 31) >> 5, S, per, shares);
  const bool direct = shares <= 1;
  if (r >= (direct ? 1 : shares)) return;
  const int k_begin = min(ctx, 32 * per * r);
  const int k_end = min(ctx, 32 * per * (r + 1));
  f32x4 acc[8];
  float m_run, l;
  const int n = lane & 15;
  const int g = lane >> 4;
  if constexpr (STORE) {
    // The share holding key ctx-1 stores the new token's rows of this kv
    // head.  When slot_mapping[b] is key ctx-1's slot -- what every decode
    // step produces -- that share's own read of the key is patched from
    // registers, so no other share reads the slot and the result equals
    // store-then-decode without waiting for the store.  An empty sequence's
    // rows are stored by the merge kernel, after every read of this launch.
    const int64_t slot = __builtin_amdgcn_readfirstlane(p.slot_mapping[b]);
    const int holder = ctx > 0 ? (ctx - 1) / (32 * per) : -1;
    NewRow<FP8, D> nr;
    const bool stores = r == holder && slot >= 0 && slot < static_cast<int64_t>(p.num_blocks) * p.block_size;
    // lanes 0..D/8-1 store the key row, lanes 32.. the value row, 8 elements
    // each; the rows are loaded now and stored after the steps, so the store
    // never holds up this share's own loads
    const int j = lane & 31;
    const bool is_v = lane >= 32;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (stores) {
      const uint16_t* kin = p.new_k + b * p.new_k_stride + kvh * D;
      const uint16_t* vin = p.new_v + b * p.new_v_stride + kvh * D;
      nr.load(kin, vin, n, g, FP8 ? p.k_scale[kvh] : 1.f, FP8 ? p.v_scale[kvh] : 1.f);
      x = ld16((is_v ? vin : kin) + 8 * (j & (D / 8 - 1)));  // every lane loads (no branch), D/8 of them store
      nr.step = ((ctx - 1) >> 5) - (k_begin >> 5);
      nr.row = (ctx - 1) & 31;
      nr.slot = static_cast<int>(slot);
    }
    if (stores)
      segment_accumulate<FP8, true, D, true, true>(p, kvh, b, k_begin, k_end, acc, m_run, l, bt_row, nr);
    else
      segment_accumulate<FP8, true, D, true, true>(p, kvh, b, k_begin, k_end, acc, m_run, l, bt_row);
    if (stores && j < D / 8) {
      constexpr int EB = FP8 ? 1 : 2;
      char* dst = static_cast<char*>(const_cast<void*>(is_v ? p.v_cache : p.k_cache)) +
                  (slot * p.num_kv_heads + kvh) * D * EB + 8 * j * EB;
      if constexpr (FP8)
        *reinterpret_cast<u32x2*>(dst) = bf16x8_to_e4m3fn(x, is_v ? p.v_scale[kvh] : p.k_scale[kvh]);
      else
        *reinterpret_cast<u32x4*>(dst) = x;
    }
  } else {
    segment_accumulate<FP8, true, D, true, true>(p, kvh, b, k_begin, k_end, acc, m_run, l, bt_row);
  }
  const bool cols = n < p.group && 32 * g < D;  // lanes holding a head's output columns
  const int h = kvh * p.group + n;
  const float vscale = FP8 ? p.v_scale[kvh] : 1.0f;
  if (direct) {
    if (!cols) return;
    const float inv = l > 0.f ? vscale / l : 0.f;
    uint16_t* orow = p.out + b * p.out_row_stride + h * D + 32 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      u32x4 o;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) o[q2] = pack_bf16x2(acc[2 * q2][q] * inv, acc[2 * q2 + 1][q] * inv);
      st16(orow + 8 * q, o);
    }
    return;
  }
  if (!cols) return;
  const int64_t idx = (static_cast<int64_t>(b) * S + r) * p.num_heads + h;
  float* wo = p.ws_o + idx * D + 32 * g;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f32x4 lo, hi;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo[j] = acc[j][q] * vscale;
      hi[j] = acc[4 + j][q] * vscale;
    }
    *reinterpret_cast<f32x4*>(wo + 8 * q) = lo;
    *reinterpret_cast<f32x4*>(wo + 8 * q + 4) = hi;
  }
  if (g == 0) *reinterpret_cast<f32x2*>(p.ws_ml + idx * 2) = f32x2{m_run, l};
}

// ---------------------------------------------------------------------------
// Balanced split-K.  Every sequence is cut into 32-key steps and the steps of
// all sequences, in sequence order, form one list of T entries (T from a
// device-side scan of the lengths, so nothing is read back to the host).
// Range r of the P ranges [r*T/P, (r+1)*T/P) goes to workgroup r, whose WAVES
// waves are WAVES kv heads; every wave does the same number of steps whatever
// the length mix.  A range covering a whole sequence writes its output
// directly; otherwise the piece of sequence b in range r goes to partial slot
// b + r (distinct for all pieces: ranges and sequences both advance
// monotonically).  Workgroup (0, 0) also stores the exclusive step prefix of
// every sequence for the merge.  Grid: (P, head groups).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int shfl_up_i(int v, int d) {
  const int lane = __lane_id();
  const int src = lane >= d ? lane - d : lane;
  return __builtin_amdgcn_ds_bpermute(src << 2, v);
}

// Inclusive scan over the workgroup (WAVES waves); `total` gets the sum.
template <int WAVES>
__device__ __forceinline__ int block_scan_incl(int v, int* s_wsum, int& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = shfl_up_i(v, d);
    if (lane >= d) v += t;
  }
  if (lane == 63) s_wsum[wave] = v;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < WAVES; ++i) {
    const int s = s_wsum[i];
    before += i < wave ? s : 0;
    total += s;
  }
  __syncthreads();
  return v + before;
}

__device__ __forceinline__ int64_t range_start(int64_t r, int64_t T, int64_t P) { return r * T / P; }

// Ranges used for T steps: the planned P, but no more than one per
// kMinRangeSteps steps.  The host plans P from the block-table width, an upper
// bound on the steps; short actual totals (small batches) would otherwise be
// cut into one-step pieces whose partials the merge then has to fold.
constexpr int64_t kMinRangeSteps = 4;
__device__ __forceinline__ int64_t used_ranges(int64_t P, int64_t T) {
  const int64_t cap = T / kMinRangeSteps;
  return cap < 1 ? 1 : (P < cap ? P : cap);
}

template <bool FP8, int WAVES, bool PREFETCH, int D, bool STORE = false>
__global__ __launch_bounds__(64 * WAVES) void paged_decode_balanced_kernel(DecodeParams p) {
  constexpr int CH = 64 * WAVES;  // sequences per scan chunk
  __shared__ int s_wsum[WAVES];
  // (b, first step, end step) of the chunk's pieces.  (Carrying each
  // sequence's length here too, instead of re-reading it per segment, measured
  // 2 us slower at config 3.)
  __shared__ int s_seg[3 * CH];
  const int tid = threadIdx.x;
  // wave-uniform (readfirstlane): the step buffer resources stay in scalar registers
  const int kvh = __builtin_amdgcn_readfirstlane(blockIdx.y * WAVES + (tid >> 6));
  const int r = blockIdx.x;
  const int B = p.batch;
  const bool write_prefix = blockIdx.x == 0 && blockIdx.y == 0;

  // pass 1: total step count T (and the prefix array for the merge)
  int T = 0;
  for (int c0 = 0; c0 < B; c0 += CH) {
    const int b = c0 + tid;
    const int st = b < B ? (clamped_len(p, b) + 31) >> 5 : 0;
    int tot;
    const int incl = block_scan_incl<WAVES>(st, s_wsum, tot);
    if (write_prefix && b < B) p.ws_prefix[b] = T + incl - st;
    T += tot;
  }
  if (write_prefix && tid == 0) p.ws_prefix[B] = T;
  const int64_t P = used_ranges(p.balanced_ranges, T);
  if (r >= P) return;
  const int start = static_cast<int>(range_start(r, T, P));
  const int end = static_cast<int>(range_start(r + 1, T, P));
  if (start >= end) return;  // uniform over the workgroup

  // pass 2: walk the sequences overlapping [start, end), one chunk at a time
  int carry = 0;
  for (int c0 = 0; c0 < B && carry < end; c0 += CH) {
    const int b = c0 + tid;
    const int st = b < B ? (clamped_len(p, b) + 31) >> 5 : 0;
    int tot;
    const int incl = block_scan_incl<WAVES>(st, s_wsum, tot);
    const int s0 = carry + incl - st;  // first step of sequence b
    const int s1 = carry + incl;
    const bool hit = b < B && st > 0 && s0 < end && s1 > start;
    int nseg;
    const int pos = block_scan_incl<WAVES>(hit ? 1 : 0, s_wsum, nseg) - 1;
    if (hit) {
      s_seg[3 * pos] = b;
      s_seg[3 * pos + 1] = max(start, s0) - s0;
      s_seg[3 * pos + 2] = min(end, s1) - s0;
    }
    __syncthreads();
    if (kvh < p.num_kv_heads) {
      for (int i = 0; i < nseg; ++i) {
        const int sb = __builtin_amdgcn_readfirstlane(s_seg[3 * i]);
        const int lo = __builtin_amdgcn_readfirstlane(s_seg[3 * i + 1]);
        const int hi = __builtin_amdgcn_readfirstlane(s_seg[3 * i + 2]);
        const int len = __builtin_amdgcn_readfirstlane(clamped_len(p, sb));
        const bool whole = lo == 0 && hi == ((len + 31) >> 5);
        decode_segment<FP8, PREFETCH, D, DecodeShape<FP8>::kBuf, STORE>(p, kvh, sb, 32 * lo, min(32 * hi, len),
                                                                        whole, static_cast<int64_t>(sb) + r, len);
      }
    }
    __syncthreads();  // s_seg is rewritten by the next chunk
    carry += tot;
  }
}

// Log-sum-exp merge of the partials: one wavefront per (sequence, head), four
// heads of one sequence per workgroup, two output columns per lane.  Fixed
// splits: slots b*num_splits + s for the splits that hold keys.  Balanced:
// slots b + r for the ranges r that overlap the sequence; a sequence inside
// one range was written directly and is skipped, an empty one gets zeros.
// One pass: the loads of up to eight partials are issued together and folded
// into a running (max, sum, output) online, so the only dependent load before
// them is the step prefix.
// WIDE (plans with many partials per sequence): one workgroup per (sequence,
// head) instead; its four waves fold a quarter of the partials each and wave 0
// combines their states through LDS, so a long list costs a quarter of the
// dependent load batches (a one-kv-head fp8 decode at B=64, 32 ranges per
// sequence: 16.7 us as one wave per head).
constexpr int kMergeHeads = 4;    // heads (waves) per merge workgroup
constexpr int kMergeWideMin = 8;  // ranges per sequence (on average) from which the merge is WIDE

// The new token's K and V rows of (b, kvh) for a sequence with no keys, when
// the store is fused into the decode launch: no decode wave reads key ctx-1 of
// such a sequence, so the merge kernel -- stream-ordered after every read of
// the decode launch -- stores them.  One wave: lanes 0..d/8-1 write the key
// row, lanes 32..32+d/8-1 the value row, 8 elements each (fp8: quantised as
// the store kernel does).  Slots outside the pool are skipped.
__device__ void store_empty_rows_wave(const DecodeParams& p, int b, int kvh, int lane) {
  const int64_t slot = p.slot_mapping[b];
  const int j = lane & 31;
  if (slot < 0 || slot >= p.num_blocks * p.block_size || 8 * j >= p.head_dim) return;
  const bool is_v = lane >= 32;
  const u32x4 x = ld16((is_v ? p.new_v + b * p.new_v_stride : p.new_k + b * p.new_k_stride) +
                       static_cast<int64_t>(kvh) * p.head_dim + 8 * j);
  const int64_t elem = (slot * p.num_kv_heads + kvh) * p.head_dim + 8 * j;
  char* base = static_cast<char*>(const_cast<void*>(is_v ? p.v_cache : p.k_cache));
  if (p.kv_fp8)
    *reinterpret_cast<u32x2*>(base + elem) = bf16x8_to_e4m3fn(x, is_v ? p.v_scale[kvh] : p.k_scale[kvh]);
  else
    *reinterpret_cast<u32x4*>(base + 2 * elem) = x;
}

template <bool WIDE>
__global__ __launch_bounds__(64 * kMergeHeads) void decode_merge_kernel(DecodeParams p) {
  const int hgroups = (p.num_heads + kMergeHeads - 1) / kMergeHeads;
  const int b = WIDE ? blockIdx.x / p.num_heads : blockIdx.x / hgroups;
  const int wq = threadIdx.x >> 6;  // WIDE: the wave's quarter of the partials
  const int h = WIDE ? static_cast<int>(blockIdx.x) - b * p.num_heads : (blockIdx.x - b * hgroups) * kMergeHeads + wq;
  const int lane = threadIdx.x & 63;
  int64_t first, count;
  bool zero = false;
  if (p.balanced_ranges > 0) {
    const int64_t s0 = p.ws_prefix[b], s1 = p.ws_prefix[b + 1], T = p.ws_prefix[p.batch];
    const int64_t P = used_ranges(p.balanced_ranges, T);
    if (s1 <= s0) {
      zero = true;
      first = count = 0;
    } else {
      const int64_t rf = ((s0 + 1) * P - 1) / T;  // range holding step s0
      const int64_t rl = (s1 * P - 1) / T;        // range holding step s1 - 1
      if (rf == rl) return;
      first = b + rf;
      count = rl - rf + 1;
    }
  } else {
    const int ctx = clamped_len(p, b);
    first = static_cast<int64_t>(b) * p.num_splits;
    count = (ctx + p.keys_per_split - 1) / p.keys_per_split;
    zero = count == 0;
  }
  if (h >= p.num_heads) return;
  if (zero && p.new_k && h % p.group == 0 && (!WIDE || wq == 0)) store_empty_rows_wave(p, b, h / p.group, lane);
  // A partial slot holds data unless it is a balanced range with no steps (P > T).
  const int64_t T = p.balanced_ranges > 0 ? p.ws_prefix[p.batch] : 0;
  const int64_t PU = p.balanced_ranges > 0 ? used_ranges(p.balanced_ranges, T) : 0;
  auto has_data = [&](int64_t s) {
    if (p.balanced_ranges <= 0) return true;
    const int64_t rr = first - b + s;
    return range_start(rr, T, PU) != range_start(rr + 1, T, PU);
  };
  const bool cols = 2 * lane < p.head_dim;  // lane owns output columns 2 lane, 2 lane + 1
  float M = kNegInf, L = 0.f, o0 = 0.f, o1 = 0.f;
  const int64_t s_lo = WIDE ? count * wq / kMergeHeads : 0;
  const int64_t s_hi = WIDE ? count * (wq + 1) / kMergeHeads : count;
  if (!zero) {
    for (int64_t s0 = s_lo; s0 < s_hi; s0 += 8) {
      f32x2 ml[8], v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t s = s0 + u;
        const bool ok = s < s_hi && has_data(s);
        const int64_t idx = (first + (ok ? s : 0)) * p.num_heads + h;
        ml[u] = ok ? *reinterpret_cast<const f32x2*>(p.ws_ml + idx * 2) : f32x2{kNegInf, 0.f};
        v[u] = ok && cols ? *reinterpret_cast<const f32x2*>(p.ws_o + idx * p.head_dim + 2 * lane) : f32x2{0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (ml[u][0] == kNegInf) continue;  // no slot, or no valid key in it
        const float m_new = fmaxf(M, ml[u][0]);
        const float a = fast_exp2(M - m_new);  // 0 while M is still -inf
        const float w = fast_exp2(ml[u][0] - m_new);
        L = L * a + w * ml[u][1];
        o0 = o0 * a + w * v[u][0];
        o1 = o1 * a + w * v[u][1];
        M = m_new;
      }
    }
  }
  if constexpr (WIDE) {
    __shared__ float s_m[kMergeHeads], s_l[kMergeHeads];
    __shared__ f32x2 s_o[kMergeHeads][64];
    if (lane == 0) {
      s_m[wq] = M;
      s_l[wq] = L;
    }
    s_o[wq][lane] = f32x2{o0, o1};
    __syncthreads();
    if (wq != 0) return;
    M = kNegInf;
    L = o0 = o1 = 0.f;
#pragma unroll
    for (int q = 0; q < kMergeHeads; ++q) {
      const float mq = s_m[q];
      if (mq == kNegInf) continue;  // a quarter with no partial holding keys
      const float m_new = fmaxf(M, mq);
      const float a = fast_exp2(M - m_new);
      const float w = fast_exp2(mq - m_new);
      const f32x2 oq = s_o[q][lane];
      L = L * a + w * s_l[q];
      o0 = o0 * a + w * oq[0];
      o1 = o1 * a + w * oq[1];
      M = m_new;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (!cols) return;
  uint32_t* orow = reinterpret_cast<uint32_t*>(p.out + b * p.out_row_stride + h * p.head_dim + 2 * lane);
  *orow = pack_bf16x2(o0 * inv, o1 * inv);
}

// Merge of the spread mode's partials: one wavefront per (sequence, head) and
// per workgroup (a small batch has few of them: one CU each, since one CU
// moves partials as slowly as cache rows), two output columns per lane; slots b * spread + r for
// the sequence's non-empty shares (one share or none: written directly by the
// decode kernel, skipped here).  The loads of kSpreadMergeBatch partials are
// issued unconditionally, so they are all in flight together: the merge costs
// one memory round trip per batch, not one per partial.  16 per batch: a
// small-batch step is latency-bound and this kernel's code is fetched cold by
// each CU, so a 32-way unrolled batch (twice the code) measured slower
// (captured batch 1: 12.6 vs 13.1 us per layer; batch 16: 22.4 vs 24.0).
constexpr int kSpreadMergeBatch = kSpreadMaxShares;  // one batch holds every share

__global__ __launch_bounds__(64) void decode_spread_merge_kernel(DecodeParams p) {
  const int b = blockIdx.x / p.num_heads;
  const int h = blockIdx.x - b * p.num_heads;
  const int lane = threadIdx.x;
  const int64_t first = static_cast<int64_t>(b) * p.spread;
  const int col = 2 * lane < p.head_dim ? 2 * lane : 0;  // lane owns output columns col, col + 1
  // The first batch's loads do not wait for the context length: slots of
  // shares this launch left empty hold stale partials and are not folded.
  f32x2 ml[kSpreadMergeBatch], v[kSpreadMergeBatch];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int u = 0; u < kSpreadMergeBatch; ++u) {
      const int64_t idx = (first + min(s0 + u, p.spread - 1)) * p.num_heads + h;
      ml[u] = *reinterpret_cast<const f32x2*>(p.ws_ml + idx * 2);
      v[u] = *reinterpret_cast<const f32x2*>(p.ws_o + idx * p.head_dim + col);
    }
  };
  load_batch(0);
  int per, shares;
  spread_shares((clamped_len(p, b) + 31) >> 5, p.spread, per, shares);
  if (shares == 0 && p.new_k && h % p.group == 0) store_empty_rows_wave(p, b, h / p.group, lane);
  if (shares <= 1) return;  // written directly by the decode kernel
  float M = kNegInf, L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int s0 = 0;;) {
    // the batch's maximum first, then every weight at once: no chain of
    // dependent exponentials through the shares
    float mx = kNegInf;
#pragma unroll
    for (int u = 0; u < kSpreadMergeBatch; ++u)
      if (s0 + u < shares) mx = fmaxf(mx, ml[u][0]);
    const float m_new = fmaxf(M, mx);
    if (m_new != kNegInf) {  // otherwise no valid key so far
      const float a = fast_exp2(M - m_new);  // 0 while M is still -inf
      L *= a;
      o0 *= a;
      o1 *= a;
#pragma unroll
      for (int u = 0; u < kSpreadMergeBatch; ++u) {
        if (s0 + u >= shares) continue;  // a stale slot: never read into the sums
        const float w = fast_exp2(ml[u][0] - m_new);  // 0 for a share with no valid key (max -inf)
        L += w * ml[u][1];
        o0 += w * v[u][0];
        o1 += w * v[u][1];
      }
      M = m_new;
    }
    s0 += kSpreadMergeBatch;
    if (s0 >= shares) break;
    load_batch(s0);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (2 * lane >= p.head_dim) return;
  uint32_t* orow = reinterpret_cast<uint32_t*>(p.out + b * p.out_row_stride + h * p.head_dim + 2 * lane);
  *orow = pack_bf16x2(o0 * inv, o1 * inv);
}

// The two-wave shape is not used: with two kv heads it returned an illegal
// address on the GPU once and unnormalised garbage (fp8) in another run, for
// a cause not yet found; one wave per workgroup serves those head counts.
int decode_waves_per_group(int32_t num_kv_heads, int32_t kv_dtype) {
  int w = kv_dtype == 1 ? DecodeShape<true>::kWaves : DecodeShape<false>::kWaves;
  while (w > 1 && w / 2 >= num_kv_heads) w /= 2;
  return w == 2 ? 1 : w;
}

DecodePlan plan_decode(int32_t batch, int32_t num_kv_heads, int32_t max_blocks, int32_t block_size,
                       int32_t kv_dtype, int32_t requested_splits) {
  DecodePlan plan{};
  // small batch, short table: spread over many CUs, merged in the same launch
  const int64_t table_steps = (static_cast<int64_t>(max_blocks) * block_size + 31) / 32;
  const int64_t pairs = static_cast<int64_t>(batch) * num_kv_heads;
  if (requested_splits == 0 && pairs <= kSpreadMaxPairs && max_blocks <= kWgMaxBlocks) {
    int64_t S = kSpreadTargetWaves / pairs;
    if (S > table_steps) S = table_steps;
    if (S > kSpreadMaxShares) S = kSpreadMaxShares;
    if (S < 1) S = 1;
    plan.pages_per_split = max_blocks;
    plan.num_splits = 1;
    plan.balanced_ranges = 0;
    plan.spread = static_cast<int32_t>(S);
    plan.partial_slots = S > 1 ? static_cast<int64_t>(batch) * S : 0;
    return plan;
  }
  if (requested_splits < 0) requested_splits = 0;  // -1: balanced whatever the sizes
  if (requested_splits > 0) {  // fixed: about requested_splits splits per sequence
    int32_t pps = (max_blocks + requested_splits - 1) / requested_splits;
    if (pps < 1) pps = 1;
    plan.pages_per_split = pps;
    plan.num_splits = (max_blocks + pps - 1) / pps;
    plan.balanced_ranges = 0;
    plan.partial_slots = plan.num_splits > 1 ? static_cast<int64_t>(batch) * plan.num_splits : 0;
    return plan;
  }
  // balanced: about kTargetWaves waves in total, never more ranges than there
  // can be steps
  const int w = decode_waves_per_group(num_kv_heads, kv_dtype);
  const int64_t groups = (num_kv_heads + w - 1) / w;
  const int target = kv_dtype == 1 ? DecodeShape<true>::kTargetWaves : DecodeShape<false>::kTargetWaves;
  int64_t P = target / (w * groups);
  const int64_t max_steps = static_cast<int64_t>(batch) * ((static_cast<int64_t>(max_blocks) * block_size + 31) / 32);
  if (max_steps >= (int64_t{1} << 31)) return plan_decode(batch, num_kv_heads, max_blocks, block_size, kv_dtype, 1);
  if (P > max_steps) P = max_steps;
  if (P < 1) P = 1;
  plan.pages_per_split = max_blocks;
  plan.num_splits = 1;
  plan.balanced_ranges = static_cast<int32_t>(P);
  plan.partial_slots = batch + P;
  return plan;
}

#define NVA_COMMA ,
template <bool FP8, int D>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  constexpr bool PF = DecodeShape<FP8>::kPrefetch;
  const int w = decode_waves_per_group(p.num_kv_heads, FP8 ? 1 : 0);
  const unsigned groups = static_cast<unsigned>((p.num_kv_heads + w - 1) / w);
  constexpr int WMAX = DecodeShape<FP8>::kWaves;  // wider shapes are never launched for this dtype
// EXTRA: further template arguments (", true" or nothing)
#define NVA_LAUNCH_W(KERNEL, GRID, EXTRA)                                                               \
  if (w >= 8 && WMAX >= 8)                                                                              \
    hipLaunchKernelGGL((KERNEL<FP8, (WMAX >= 8 ? 8 : 1), PF, D EXTRA>), GRID, dim3(64 * (WMAX >= 8 ? 8 : 1)), \
                       0, stream, p);                                                                   \
  else if (w >= 4)                                                                                      \
    hipLaunchKernelGGL((KERNEL<FP8, 4, PF, D EXTRA>), GRID, dim3(256), 0, stream, p);                   \
  else                                                                                                  \
    hipLaunchKernelGGL((KERNEL<FP8, 1, PF, D EXTRA>), GRID, dim3(64), 0, stream, p);
  bool merge;
  if (p.spread > 0) {
    const dim3 grid(static_cast<unsigned>(p.spread), static_cast<unsigned>(p.num_kv_heads),
                    static_cast<unsigned>(p.batch));
    if (p.new_k)
      hipLaunchKernelGGL((paged_decode_spread_kernel<FP8, D, true>), grid, dim3(64), 0, stream, p);
    else
      hipLaunchKernelGGL((paged_decode_spread_kernel<FP8, D, false>), grid, dim3(64), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.spread == 1) return e;
    hipLaunchKernelGGL(decode_spread_merge_kernel, dim3(static_cast<unsigned>(p.batch * p.num_heads)), dim3(64), 0,
                       stream, p);
    return hipGetLastError();
  } else if (p.balanced_ranges > 0) {
    const dim3 grid(static_cast<unsigned>(p.balanced_ranges), groups);
    // The store is fused for a bf16 cache only: its buffer-step loop takes the
    // patch (an fp8 cache stores first, a few microseconds).
    bool fused = false;
    if constexpr (!FP8) {
      if (p.new_k) {
        NVA_LAUNCH_W(paged_decode_balanced_kernel, grid, NVA_COMMA true);
        fused = true;
      }
    }
    if (!fused) {
      NVA_LAUNCH_W(paged_decode_balanced_kernel, grid, );
    }
    merge = true;
  } else {
    const dim3 grid(groups, p.num_splits, p.batch);
    NVA_LAUNCH_W(paged_decode_split_kernel, grid, );
    merge = p.num_splits > 1;
  }
#undef NVA_LAUNCH_W
#undef NVA_COMMA
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !merge) return e;
  const int64_t per_seq = p.balanced_ranges > 0 ? p.balanced_ranges / p.batch : p.num_splits;
  if (per_seq >= kMergeWideMin) {
    hipLaunchKernelGGL(decode_merge_kernel<true>, dim3(static_cast<unsigned>(p.batch * p.num_heads)),
                       dim3(64 * kMergeHeads), 0, stream, p);
  } else {
    const dim3 mgrid(static_cast<unsigned>(p.batch * ((p.num_heads + kMergeHeads - 1) / kMergeHeads)));
    hipLaunchKernelGGL(decode_merge_kernel<false>, mgrid, dim3(64 * kMergeHeads), 0, stream, p);
  }
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams& p, int kv_dtype, hipStream_t stream) {
  if (p.batch <= 0) return hipSuccess;
  if (p.head_dim == 64)
    return kv_dtype == 1 ? launch_decode_t<true, 64>(p, stream) : launch_decode_t<false, 64>(p, stream);
  return kv_dtype == 1 ? launch_decode_t<true, 128>(p, stream) : launch_decode_t<false, 128>(p, stream);
}

}  // namespace nva
