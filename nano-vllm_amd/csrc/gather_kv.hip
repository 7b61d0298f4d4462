// Paged cache -> packed rows: the keys and values of every sequence, gathered
// through its block table and written as bf16 rows at cu_seqlens_k[s] + j.
// This is how a prefix-cached prefill (nanovllm/layers/attention.py:68-73)
// reads an fp8 e4m3fn cache: the rows are dequantised here (x = e4m3 * scale
// of the kv head, rounded to bf16) and the packed prefill kernel runs on them,
// so the MFMA prefill keeps its global->LDS copies.  A bf16 cache is copied
// bit for bit.
//
// Workgroup = (kRowsPerGroup key rows of one sequence); threadIdx.y selects K
// (0) or V (1), and every lane moves 8 elements of each of the rows (8 or 16
// bytes in, 16 bytes out).  The loads of all the rows are issued before any of
// them is converted or stored, so a lane has kRowsPerGroup loads in flight
// instead of one memory round trip per row.  HBM-bound: each cache byte is read
// once, each output byte written once.  Rows on a page outside [0,
// num_blocks), past the block table's width or past the output rows are zeros
// (or not written).
#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

namespace {

constexpr int kRowsPerGroup = 16;

template <bool FP8>
__global__ __launch_bounds__(256) void gather_kv_kernel(GatherParams p) {
  const int s = blockIdx.y;
  const int k_start = p.cu_k[s];
  const int Lk = p.cu_k[s + 1] - k_start;
  const int j0 = blockIdx.x * kRowsPerGroup;
  if (j0 >= Lk) return;
  const bool is_v = threadIdx.y != 0;
  const int D = p.row_elems;
  const int pieces = D / 8;
  const int32_t* bt = p.block_table + static_cast<int64_t>(s) * p.bt_row_stride;
  const float* scale = is_v ? p.v_scale : p.k_scale;
  const char* cache = static_cast<const char*>(is_v ? p.v_cache : p.k_cache);
  char* out = static_cast<char*>(is_v ? p.v_out : p.k_out);
  // source slot of each row (-1: a zero row), its output row (-1: not written)
  int64_t slot[kRowsPerGroup], row[kRowsPerGroup];
#pragma unroll
  for (int r = 0; r < kRowsPerGroup; ++r) {
    const int j = j0 + r;
    const int64_t orow = static_cast<int64_t>(k_start) + j;
    row[r] = j < Lk && orow >= 0 && orow < p.out_rows ? orow : -1;
    const int bi = j / p.block_size;
    const int page = j < Lk && bi < p.max_blocks ? bt[bi] : -1;
    slot[r] = page >= 0 && page < p.num_blocks ? static_cast<int64_t>(page) * p.block_size + (j - bi * p.block_size)
                                               : -1;
  }
  for (int c = threadIdx.x; c < pieces; c += blockDim.x) {
    if constexpr (FP8) {
      const float sc = scale[(c * 8) / p.head_dim];
      u32x2 w[kRowsPerGroup];
#pragma unroll
      for (int r = 0; r < kRowsPerGroup; ++r) w[r] = slot[r] >= 0 ? ld8(cache + slot[r] * D + c * 8) : u32x2{0u, 0u};
#pragma unroll
      for (int r = 0; r < kRowsPerGroup; ++r) {
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // fp8 -> bf16 is exact; the scale is applied in f32, then one rounding
          const uint32_t lo = fp8x2_to_bf16x2<false>(w[r][h]);
          const uint32_t hi = fp8x2_to_bf16x2<true>(w[r][h]);
          o[2 * h] = pack_bf16x2(bf16_bits_to_f32(lo & 0xffffu) * sc, bf16_bits_to_f32(lo >> 16) * sc);
          o[2 * h + 1] = pack_bf16x2(bf16_bits_to_f32(hi & 0xffffu) * sc, bf16_bits_to_f32(hi >> 16) * sc);
        }
        if (row[r] >= 0) st16(out + (row[r] * p.out_row_stride + c * 8) * 2, o);
      }
    } else {
      u32x4 w[kRowsPerGroup];
#pragma unroll
      for (int r = 0; r < kRowsPerGroup; ++r)
        w[r] = slot[r] >= 0 ? ld16(cache + (slot[r] * D + c * 8) * 2) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < kRowsPerGroup; ++r)
        if (row[r] >= 0) st16(out + (row[r] * p.out_row_stride + c * 8) * 2, w[r]);
    }
  }
}

}  // namespace

hipError_t launch_gather_kv(const GatherParams& p, int max_seqlen_k, int kv_dtype, hipStream_t stream) {
  if (p.num_seqs <= 0 || max_seqlen_k <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((max_seqlen_k + kRowsPerGroup - 1) / kRowsPerGroup),
                  static_cast<unsigned>(p.num_seqs));
  const int pieces = p.row_elems / 8;
  const dim3 block(pieces < 128 ? pieces : 128, 2);
  if (kv_dtype == 1)
    hipLaunchKernelGGL(gather_kv_kernel<true>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(gather_kv_kernel<false>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace nva
