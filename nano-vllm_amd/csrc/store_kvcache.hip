// Paged KV-cache scatter (replaces the Triton store_kvcache_kernel of
// nanovllm/layers/attention.py:10-29).
//
// One workgroup per new token.  Its threads stream the token's key row and
// value row (D = num_kv_heads * head_dim bf16 each) in 16-byte pieces and write
// them to slot `slot_mapping[token]` of the paged caches.  Every lane issues
// one coalesced vector load and one vector store per piece; offsets are 64-bit
// (slot * D overflows int32 beyond 2^21 slots).  The stores are non-temporal:
// the cache rows are not read again by this launch, and streaming them past
// the caches took prefill-sized batches from 54% to 59% of HBM peak
// (several tokens per workgroup, tried for more bytes in flight, did not help).
#include "nva_common.h"
#include "nva_kernels.h"

namespace nva {

// VB bytes per lane per access (16, 8, 4 or 2: chosen on the host from the
// alignment of pointers and row strides).
template <int VB>
__global__ __launch_bounds__(256) void store_kvcache_bf16_kernel(StoreParams p) {
  const int64_t t = blockIdx.x;
  const int row_bytes = p.row_elems * 2;
  const int pieces = row_bytes / VB;
  const char* ksrc = static_cast<const char*>(p.key) + t * p.key_row_stride * 2;
  const char* vsrc = static_cast<const char*>(p.value) + t * p.value_row_stride * 2;
  // threadIdx.y selects key (0) or value (1)
  const char* src = threadIdx.y ? vsrc : ksrc;
  // The first 16-byte piece is loaded together with the slot (the source row
  // does not depend on it): a small batch then waits for one memory round trip
  // before its stores instead of two.
  const int c0 = threadIdx.x;
  u32x4 first = {0u, 0u, 0u, 0u};
  if (VB == 16 && c0 < pieces) first = ld16(src + c0 * 16);
  const int64_t slot = p.slot_mapping[t];
  if (slot < 0 || slot >= p.num_slots) return;
  char* kdst = static_cast<char*>(p.k_cache) + slot * row_bytes;
  char* vdst = static_cast<char*>(p.v_cache) + slot * row_bytes;
  char* dst = threadIdx.y ? vdst : kdst;
  if (VB == 16 && c0 < pieces) __builtin_nontemporal_store(first, reinterpret_cast<u32x4*>(dst + c0 * 16));
  for (int c = VB == 16 ? c0 + blockDim.x : c0; c < pieces; c += blockDim.x) {
    if constexpr (VB == 16) {
      __builtin_nontemporal_store(ld16(src + c * 16), reinterpret_cast<u32x4*>(dst + c * 16));
    } else if constexpr (VB == 8) {
      __builtin_nontemporal_store(ld8(src + c * 8), reinterpret_cast<u32x2*>(dst + c * 8));
    } else if constexpr (VB == 4) {
      __builtin_nontemporal_store(*reinterpret_cast<const uint32_t*>(src + c * 4), reinterpret_cast<uint32_t*>(dst + c * 4));
    } else {
      __builtin_nontemporal_store(*reinterpret_cast<const uint16_t*>(src + c * 2), reinterpret_cast<uint16_t*>(dst + c * 2));
    }
  }
}

// bf16 rows -> fp8 cache rows, 8 elements (16 B in, 8 B out) per lane.
__global__ __launch_bounds__(256) void store_kvcache_fp8_kernel(StoreParams p) {
  const int64_t t = blockIdx.x;
  const int64_t slot = p.slot_mapping[t];
  if (slot < 0 || slot >= p.num_slots) return;
  const int pieces = p.row_elems / 8;
  const bool is_v = threadIdx.y != 0;
  const char* src = static_cast<const char*>(is_v ? p.value : p.key) +
                    t * (is_v ? p.value_row_stride : p.key_row_stride) * 2;
  char* dst = static_cast<char*>(is_v ? p.v_cache : p.k_cache) + slot * p.row_elems;
  const float* scale = is_v ? p.v_scale : p.k_scale;
  for (int c = threadIdx.x; c < pieces; c += blockDim.x) {
    const float s = scale[(c * 8) / p.head_dim];
    *reinterpret_cast<u32x2*>(dst + c * 8) = bf16x8_to_e4m3fn(ld16(src + c * 16), s);
  }
}

hipError_t launch_store_kvcache(const StoreParams& p, int vec_bytes, hipStream_t stream) {
  if (p.num_tokens == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(p.num_tokens));
  if (p.cache_dtype == 1) {
    const int pieces = p.row_elems / 8;
    const dim3 block(pieces < 128 ? pieces : 128, 2);
    hipLaunchKernelGGL(store_kvcache_fp8_kernel, grid, block, 0, stream, p);
    return hipGetLastError();
  }
  const int pieces = p.row_elems * 2 / vec_bytes;
  const dim3 block(pieces < 128 ? pieces : 128, 2);
  switch (vec_bytes) {
    case 16: hipLaunchKernelGGL(store_kvcache_bf16_kernel<16>, grid, block, 0, stream, p); break;
    case 8: hipLaunchKernelGGL(store_kvcache_bf16_kernel<8>, grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL(store_kvcache_bf16_kernel<4>, grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL(store_kvcache_bf16_kernel<2>, grid, block, 0, stream, p); break;
  }
  return hipGetLastError();
}

}  // namespace nva
