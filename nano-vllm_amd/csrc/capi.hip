// extern "C" entry points declared in include/nva_attention.h: argument
// validation, launch planning and error reporting.  Validation never touches
// the GPU, so a rejected call is safe (and testable) on a host without one.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "nva_attention.h"
#include "nva_kernels.h"

// The static decode scratch of nva_decode_noalloc (see scratch_on_current_device).
static __device__ __align__(256) char scratch[nva::kDecodeScratchBytes];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return NVA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(NVA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace

extern "C" {

int nva_version(void) { return 100; }

const char* nva_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"

namespace {

// Validate a store and fill its parameters and vector width (the launch is
// the caller's).  Shared by nva_store_kvcache and nva_store_decode.
int store_setup(const void* key, int64_t key_row_stride, const void* value, int64_t value_row_stride,
                void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping, int64_t num_tokens,
                int32_t num_kv_heads, int32_t head_dim, int32_t cache_dtype, const float* k_scale,
                const float* v_scale, nva::StoreParams& p, int& vec) {
  if (num_tokens < 0) return fail(NVA_ERR_INVALID_ARGUMENT, "num_tokens must be >= 0 (got %lld)", (long long)num_tokens);
  if (num_tokens > 0x7fffffffLL) return fail(NVA_ERR_UNSUPPORTED, "num_tokens above 2^31-1");
  if (num_kv_heads <= 0 || head_dim <= 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_kv_heads and head_dim must be positive (got %d, %d)", num_kv_heads, head_dim);
  if (cache_dtype != NVA_DTYPE_BF16 && cache_dtype != NVA_DTYPE_FP8_E4M3)
    return fail(NVA_ERR_INVALID_ARGUMENT, "unknown cache dtype %d", cache_dtype);
  if (num_tokens == 0) return ok();
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(NVA_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int64_t D = static_cast<int64_t>(num_kv_heads) * head_dim;
  if (key_row_stride < D || value_row_stride < D)
    return fail(NVA_ERR_INVALID_ARGUMENT, "key/value row strides (%lld, %lld) must be >= num_kv_heads*head_dim (%lld)",
                (long long)key_row_stride, (long long)value_row_stride, (long long)D);
  if (num_slots <= 0) return fail(NVA_ERR_INVALID_ARGUMENT, "num_slots must be positive");
  if (D > (1 << 20)) return fail(NVA_ERR_UNSUPPORTED, "num_kv_heads*head_dim above 2^20");
  if (!aligned(slot_mapping, 4)) return fail(NVA_ERR_INVALID_ARGUMENT, "slot_mapping must be 4-byte aligned");

  p = nva::StoreParams{};
  p.key = key;
  p.value = value;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.slot_mapping = slot_mapping;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.key_row_stride = key_row_stride;
  p.value_row_stride = value_row_stride;
  p.num_slots = num_slots;
  p.num_tokens = num_tokens;
  p.row_elems = static_cast<int32_t>(D);
  p.head_dim = head_dim;
  p.cache_dtype = cache_dtype;

  vec = 2;
  if (cache_dtype == NVA_DTYPE_FP8_E4M3) {
    if (!k_scale || !v_scale) return fail(NVA_ERR_INVALID_ARGUMENT, "fp8 cache needs k_scale and v_scale");
    if (head_dim % 8 != 0) return fail(NVA_ERR_UNSUPPORTED, "fp8 store needs head_dim %% 8 == 0");
    if (!aligned(key, 16) || !aligned(value, 16) || (key_row_stride % 8) || (value_row_stride % 8))
      return fail(NVA_ERR_UNSUPPORTED, "fp8 store needs 16-byte aligned key/value rows");
    if (!aligned(k_cache, 8) || !aligned(v_cache, 8))
      return fail(NVA_ERR_INVALID_ARGUMENT, "fp8 caches must be 8-byte aligned");
    if (!aligned(k_scale, 4) || !aligned(v_scale, 4)) return fail(NVA_ERR_INVALID_ARGUMENT, "scales must be 4-byte aligned");
  } else {
    for (int cand : {16, 8, 4}) {
      if ((D * 2) % cand == 0 && (key_row_stride * 2) % cand == 0 && (value_row_stride * 2) % cand == 0 &&
          aligned(key, cand) && aligned(value, cand) && aligned(k_cache, cand) && aligned(v_cache, cand)) {
        vec = cand;
        break;
      }
    }
    if (!aligned(key, 2) || !aligned(value, 2) || !aligned(k_cache, 2) || !aligned(v_cache, 2))
      return fail(NVA_ERR_INVALID_ARGUMENT, "bf16 tensors must be 2-byte aligned");
  }
  return ok();
}

}  // namespace

extern "C" {

int nva_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                      int64_t value_row_stride, void* k_cache, void* v_cache, int64_t num_slots,
                      const int32_t* slot_mapping, int64_t num_tokens, int32_t num_kv_heads,
                      int32_t head_dim, int32_t cache_dtype, const float* k_scale,
                      const float* v_scale, void* stream) {
  nva::StoreParams p{};
  int vec = 2;
  const int rc = store_setup(key, key_row_stride, value, value_row_stride, k_cache, v_cache, num_slots, slot_mapping,
                             num_tokens, num_kv_heads, head_dim, cache_dtype, k_scale, v_scale, p, vec);
  if (rc != NVA_OK || num_tokens == 0) return rc;
  return hip_status(nva::launch_store_kvcache(p, vec, static_cast<hipStream_t>(stream)), "store_kvcache launch");
}

int nva_prefill(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride, const void* v,
                int64_t v_row_stride, const int32_t* block_table, int64_t bt_row_stride,
                int32_t max_blocks_per_seq, int32_t block_size, int64_t num_blocks,
                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads,
                int32_t head_dim, float softmax_scale, void* out, int64_t out_row_stride, void* workspace,
                int64_t workspace_bytes, void* stream) {
  if (head_dim != 128 && head_dim != 64)
    return fail(NVA_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_heads, num_kv_heads);
  if (num_heads > 65535) return fail(NVA_ERR_UNSUPPORTED, "num_heads above 65535");
  if (num_seqs < 0 || max_seqlen_q < 0) return fail(NVA_ERR_INVALID_ARGUMENT, "num_seqs and max_seqlen_q must be >= 0");
  if (num_seqs > 65535) return fail(NVA_ERR_UNSUPPORTED, "num_seqs above 65535");
  if (num_seqs == 0 || max_seqlen_q == 0) return ok();
  if (!q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k) return fail(NVA_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int64_t hd = static_cast<int64_t>(num_heads) * head_dim;
  const int64_t kd = static_cast<int64_t>(num_kv_heads) * head_dim;
  if (q_row_stride < hd || out_row_stride < hd)
    return fail(NVA_ERR_INVALID_ARGUMENT, "q/out row strides must be >= num_heads*head_dim");
  if (k_row_stride < kd || v_row_stride < kd)
    return fail(NVA_ERR_INVALID_ARGUMENT, "k/v row strides must be >= num_kv_heads*head_dim");
  if (k_row_stride > (int64_t{1} << 24) || v_row_stride > (int64_t{1} << 24))
    return fail(NVA_ERR_UNSUPPORTED, "k/v row strides above 2^24 elements not supported");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16) || (q_row_stride % 8) ||
      (k_row_stride % 8) || (v_row_stride % 8) || (out_row_stride % 8))
    return fail(NVA_ERR_UNSUPPORTED, "q/k/v/out must be 16-byte aligned with row strides a multiple of 8 elements");
  if (!(softmax_scale > 0.f)) return fail(NVA_ERR_INVALID_ARGUMENT, "softmax_scale must be positive");
  if (num_heads / num_kv_heads > nva::kPrefillMaxGroup)
    return fail(NVA_ERR_UNSUPPORTED, "GQA group %d above %d not supported", num_heads / num_kv_heads,
                nva::kPrefillMaxGroup);
  {
    const int bp = nva::prefill_positions_per_tile(num_heads / num_kv_heads);
    if ((static_cast<int64_t>(max_seqlen_q) + bp - 1) / bp > 65535)
      return fail(NVA_ERR_UNSUPPORTED, "max_seqlen_q %d too long for the launch grid", max_seqlen_q);
    if (static_cast<int64_t>(num_seqs) * num_kv_heads > 0x7fffffffLL)
      return fail(NVA_ERR_UNSUPPORTED, "num_seqs*num_kv_heads above 2^31-1");
  }
  if (block_table) {
    if (block_size <= 0 || block_size % 64 != 0)
      return fail(NVA_ERR_UNSUPPORTED, "paged prefill needs block_size a positive multiple of 64 (got %d)", block_size);
    if (max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq || num_blocks <= 0)
      return fail(NVA_ERR_INVALID_ARGUMENT, "block table shape is inconsistent");
    if (!aligned(block_table, 4)) return fail(NVA_ERR_INVALID_ARGUMENT, "block_table must be 4-byte aligned");
  }
  if (workspace && (workspace_bytes < nva::kPrefillWorkspaceBytes || !aligned(workspace, 256)))
    return fail(NVA_ERR_INVALID_ARGUMENT, "prefill workspace must be 256-byte aligned and hold %lld bytes",
                static_cast<long long>(nva::kPrefillWorkspaceBytes));
  nva::PrefillParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.block_table = block_table;
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.out = static_cast<uint16_t*>(out);
  p.q_row_stride = q_row_stride;
  p.k_row_stride = k_row_stride;
  p.v_row_stride = v_row_stride;
  p.out_row_stride = out_row_stride;
  p.bt_row_stride = bt_row_stride;
  p.num_blocks = num_blocks;
  p.max_blocks = max_blocks_per_seq;
  p.block_size = block_size;
  p.num_seqs = num_seqs;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.head_dim = head_dim;
  p.scale_log2 = softmax_scale * kLog2e;
  p.queue = static_cast<uint32_t*>(workspace);
  if (workspace) {
    p.split_ctl = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + nva::kPrefillSplitCtlOffset);
    p.split_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + nva::kPrefillSplitPartOffset);
    p.split_err = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + nva::kPrefillErrOffset);
  }
  return hip_status(nva::launch_prefill(p, max_seqlen_q, max_seqlen_k, static_cast<hipStream_t>(stream)),
                    "prefill launch");
}

int64_t nva_prefill_workspace_bytes(void) { return nva::kPrefillWorkspaceBytes; }

int nva_prefill_workspace_errors(void* workspace, int64_t workspace_bytes, uint32_t* errors, void* stream) {
  if (!workspace || !errors) return fail(NVA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (workspace_bytes < nva::kPrefillWorkspaceBytes || !aligned(workspace, 256))
    return fail(NVA_ERR_INVALID_ARGUMENT, "prefill workspace must be 256-byte aligned and hold %lld bytes",
                static_cast<long long>(nva::kPrefillWorkspaceBytes));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* word = static_cast<char*>(workspace) + nva::kPrefillErrOffset;
  uint32_t host = 0;
  hipError_t e = hipMemcpyAsync(&host, word, sizeof(host), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemsetAsync(word, 0, sizeof(uint32_t), s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_status(e, "prefill workspace error word");
  *errors = host;
  return ok();
}

int64_t nva_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t max_blocks_per_seq, int32_t block_size, int32_t kv_dtype,
                                   int32_t num_splits) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || max_blocks_per_seq <= 0 || head_dim <= 0 ||
      block_size <= 0 || num_splits < -1)
    return 0;
  const nva::DecodePlan plan =
      nva::plan_decode(batch, num_kv_heads, max_blocks_per_seq, block_size, kv_dtype, num_splits);
  if (plan.partial_slots <= 0) return 0;
  const int64_t rows = plan.partial_slots * num_heads;
  int64_t bytes = rows * head_dim * 4 + rows * 2 * 4;
  if (plan.balanced_ranges > 0) bytes += (static_cast<int64_t>(batch) + 1) * 4;
  return (bytes + 255) & ~static_cast<int64_t>(255);
}

}  // extern "C"

namespace {

// Static decode scratch for nva_decode_noalloc: device memory of the library
// itself, so that entry point allocates nothing.  Each GPU holds its own copy
// of the array until the process ends; its device address on the current GPU
// is looked up once per device (hipGetSymbolAddress) and kept.  In host code
// the name `scratch` is only a host-side stand-in: kernels get the looked-up
// address, never the name.
constexpr int64_t kDecodeScratchBytes = nva::kDecodeScratchBytes;

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;
char g_scratch_error[256] = "";

void* scratch_on_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    snprintf(g_scratch_error, sizeof(g_scratch_error), "hipGetDevice: %s (device %d)", hipGetErrorString(e), dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      snprintf(g_scratch_error, sizeof(g_scratch_error), "hipGetSymbolAddress: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

// nva_decode's body.  `scratch_max` > 0 selects the no-allocation variant: the
// workspace is the library's static scratch array (`workspace` its device
// address, fetched lazily by `get_scratch` once the arguments are valid) and a
// launch that needs more than scratch_max bytes is refused before any HIP call.
int decode_impl(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache, int32_t kv_dtype,
                const float* k_scale, const float* v_scale, int64_t num_blocks, const int32_t* cache_seqlens,
                const int32_t* block_table, int64_t bt_row_stride, int32_t max_blocks_per_seq, int32_t block_size,
                int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
                int32_t num_splits, void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                void* stream, int64_t scratch_max, void* (*get_scratch)(),
                const nva::StoreParams* store = nullptr, int store_vec = 0) {
  if (head_dim != 128 && head_dim != 64)
    return fail(NVA_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_heads (%d) must be a positive multiple of num_kv_heads (%d)", num_heads, num_kv_heads);
  if (num_heads / num_kv_heads > 16)
    return fail(NVA_ERR_UNSUPPORTED, "GQA group %d above 16 not supported", num_heads / num_kv_heads);
  if (num_kv_heads > 65535) return fail(NVA_ERR_UNSUPPORTED, "num_kv_heads above 65535");
  if (kv_dtype != NVA_DTYPE_BF16 && kv_dtype != NVA_DTYPE_FP8_E4M3)
    return fail(NVA_ERR_INVALID_ARGUMENT, "unknown kv dtype %d", kv_dtype);
  // fp8 decode at head_dim 64 faulted on the GPU (an address outside every
  // aperture) for a cause not yet found; it stays refused until then.
  if (kv_dtype == NVA_DTYPE_FP8_E4M3 && head_dim != 128)
    return fail(NVA_ERR_UNSUPPORTED, "fp8 kv cache decode supports head_dim 128 only");
  if (batch < 0) return fail(NVA_ERR_INVALID_ARGUMENT, "batch must be >= 0");
  if (batch > 65535) return fail(NVA_ERR_UNSUPPORTED, "batch above 65535");
  if (num_splits < -1) return fail(NVA_ERR_INVALID_ARGUMENT, "num_splits must be >= -1");
  if (block_size <= 0 || block_size % 32 != 0)
    return fail(NVA_ERR_UNSUPPORTED, "decode needs block_size a positive multiple of 32 (got %d)", block_size);
  if (max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq)
    return fail(NVA_ERR_INVALID_ARGUMENT, "block table width %d / row stride %lld inconsistent", max_blocks_per_seq,
                (long long)bt_row_stride);
  if (static_cast<int64_t>(max_blocks_per_seq) * block_size > 0x7fffffffLL)
    return fail(NVA_ERR_UNSUPPORTED, "max_blocks_per_seq*block_size above 2^31-1");
  if (num_blocks <= 0) return fail(NVA_ERR_INVALID_ARGUMENT, "num_blocks must be positive");
  if (batch == 0) return ok();
  if (!q || !k_cache || !v_cache || !cache_seqlens || !block_table || !out)
    return fail(NVA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (kv_dtype == NVA_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(NVA_ERR_INVALID_ARGUMENT, "fp8 kv cache needs k_scale and v_scale");
  const int64_t hd = static_cast<int64_t>(num_heads) * head_dim;
  if (q_row_stride < hd || out_row_stride < hd)
    return fail(NVA_ERR_INVALID_ARGUMENT, "q/out row strides must be >= num_heads*head_dim");
  if (!aligned(q, 16) || !aligned(out, 16) || (q_row_stride % 8) || (out_row_stride % 8))
    return fail(NVA_ERR_UNSUPPORTED, "q/out must be 16-byte aligned with row strides a multiple of 8 elements");
  if (!aligned(k_cache, 16) || !aligned(v_cache, 16)) return fail(NVA_ERR_INVALID_ARGUMENT, "caches must be 16-byte aligned");
  if (!aligned(cache_seqlens, 4) || !aligned(block_table, 4))
    return fail(NVA_ERR_INVALID_ARGUMENT, "index tensors must be 4-byte aligned");
  if (!(softmax_scale > 0.f)) return fail(NVA_ERR_INVALID_ARGUMENT, "softmax_scale must be positive");

  const nva::DecodePlan plan =
      nva::plan_decode(batch, num_kv_heads, max_blocks_per_seq, block_size, kv_dtype, num_splits);
  const int64_t need = nva_decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                                  block_size, kv_dtype, num_splits);
  if (scratch_max > 0) {
    if (need > scratch_max)
      return fail(NVA_ERR_WORKSPACE,
                  "decode needs %lld bytes of workspace, above the %lld-byte static scratch of nva_decode_noalloc "
                  "(use nva_decode with a caller-allocated workspace)",
                  (long long)need, (long long)scratch_max);
    workspace = need > 0 ? get_scratch() : nullptr;
    if (need > 0 && !workspace) return fail(NVA_ERR_HIP, "static decode scratch unavailable: %s", g_scratch_error);
    workspace_bytes = scratch_max;
  }
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(NVA_ERR_WORKSPACE, "decode needs a workspace of %lld bytes (got %lld)", (long long)need,
                  (long long)(workspace ? workspace_bytes : 0));
    if (!aligned(workspace, 16)) return fail(NVA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }
  nva::DecodeParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.seqlens = cache_seqlens;
  p.block_table = block_table;
  p.out = static_cast<uint16_t*>(out);
  const int64_t rows = plan.partial_slots * num_heads;
  p.ws_o = need > 0 ? static_cast<float*>(workspace) : nullptr;
  p.ws_ml = need > 0 ? static_cast<float*>(workspace) + rows * head_dim : nullptr;
  p.ws_prefix = need > 0 && plan.balanced_ranges > 0
                    ? reinterpret_cast<int32_t*>(static_cast<float*>(workspace) + rows * (head_dim + 2))
                    : nullptr;
  p.q_row_stride = q_row_stride;
  p.out_row_stride = out_row_stride;
  p.bt_row_stride = bt_row_stride;
  p.num_blocks = num_blocks;
  p.batch = batch;
  p.max_blocks = max_blocks_per_seq;
  p.block_size = block_size;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.group = num_heads / num_kv_heads;
  p.keys_per_split = plan.pages_per_split * block_size;
  p.num_splits = plan.num_splits;
  p.balanced_ranges = plan.balanced_ranges;
  p.spread = plan.spread;
  p.head_dim = head_dim;
  p.scale_log2 = softmax_scale * kLog2e;
  p.kv_fp8 = kv_dtype == NVA_DTYPE_FP8_E4M3 ? 1 : 0;
  if (store) {
    // The spread mode with more than one share, and the balanced mode over a
    // bf16 cache, store inside their own launch (16-byte source pieces): the
    // rows of sequences with keys in the decode kernel, those of sequences
    // with none in the merge kernel that follows it.  Otherwise the store
    // kernel runs first.
    // (The fused kernels compare slots in 32 bits: pools below 2^31 slots.)
    const bool bf16_vec = kv_dtype == NVA_DTYPE_BF16 && store_vec == 16;
    const bool small_pool = num_blocks * block_size < (int64_t{1} << 31);
    if (small_pool && ((plan.spread > 1 && (kv_dtype == NVA_DTYPE_FP8_E4M3 || store_vec == 16)) ||
                       (plan.balanced_ranges > 0 && bf16_vec))) {
      p.new_k = static_cast<const uint16_t*>(store->key);
      p.new_v = static_cast<const uint16_t*>(store->value);
      p.new_k_stride = store->key_row_stride;
      p.new_v_stride = store->value_row_stride;
      p.slot_mapping = store->slot_mapping;
    } else {
      const hipError_t e = nva::launch_store_kvcache(*store, store_vec, static_cast<hipStream_t>(stream));
      if (e != hipSuccess) return hip_status(e, "store_kvcache launch");
    }
  }
  return hip_status(nva::launch_decode(p, kv_dtype, static_cast<hipStream_t>(stream)), "decode launch");
}

}  // namespace

extern "C" {

int nva_decode(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache, int32_t kv_dtype,
               const float* k_scale, const float* v_scale, int64_t num_blocks, const int32_t* cache_seqlens,
               const int32_t* block_table, int64_t bt_row_stride, int32_t max_blocks_per_seq, int32_t block_size,
               int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
               int32_t num_splits, void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
               void* stream) {
  return decode_impl(q, q_row_stride, k_cache, v_cache, kv_dtype, k_scale, v_scale, num_blocks, cache_seqlens,
                     block_table, bt_row_stride, max_blocks_per_seq, block_size, batch, num_heads, num_kv_heads,
                     head_dim, softmax_scale, num_splits, out, out_row_stride, workspace, workspace_bytes, stream, 0,
                     nullptr);
}

int nva_store_decode(const void* key, int64_t key_row_stride, const void* value, int64_t value_row_stride,
                     const int32_t* slot_mapping, const void* q, int64_t q_row_stride, void* k_cache, void* v_cache,
                     int32_t kv_dtype, const float* k_scale, const float* v_scale, int64_t num_blocks,
                     const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_row_stride,
                     int32_t max_blocks_per_seq, int32_t block_size, int32_t batch, int32_t num_heads,
                     int32_t num_kv_heads, int32_t head_dim, float softmax_scale, int32_t num_splits, void* out,
                     int64_t out_row_stride, void* workspace, int64_t workspace_bytes, void* stream) {
  if (num_blocks <= 0 || block_size <= 0 || num_blocks > INT64_MAX / block_size)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_blocks and block_size must be positive");
  nva::StoreParams sp{};
  int vec = 2;
  const int rc = store_setup(key, key_row_stride, value, value_row_stride, k_cache, v_cache, num_blocks * block_size,
                             slot_mapping, batch, num_kv_heads, head_dim, kv_dtype, k_scale, v_scale, sp, vec);
  if (rc != NVA_OK) return rc;
  return decode_impl(q, q_row_stride, k_cache, v_cache, kv_dtype, k_scale, v_scale, num_blocks, cache_seqlens,
                     block_table, bt_row_stride, max_blocks_per_seq, block_size, batch, num_heads, num_kv_heads,
                     head_dim, softmax_scale, num_splits, out, out_row_stride, workspace, workspace_bytes, stream, 0,
                     nullptr, batch > 0 ? &sp : nullptr, vec);
}

int64_t nva_decode_noalloc_max_workspace_bytes(void) { return kDecodeScratchBytes; }

int nva_decode_noalloc(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                       int32_t kv_dtype, const float* k_scale, const float* v_scale, int64_t num_blocks,
                       const int32_t* cache_seqlens, const int32_t* block_table, int64_t bt_row_stride,
                       int32_t max_blocks_per_seq, int32_t block_size, int32_t batch, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, float softmax_scale, int32_t num_splits, void* out,
                       int64_t out_row_stride, void* stream) {
  return decode_impl(q, q_row_stride, k_cache, v_cache, kv_dtype, k_scale, v_scale, num_blocks, cache_seqlens,
                     block_table, bt_row_stride, max_blocks_per_seq, block_size, batch, num_heads, num_kv_heads,
                     head_dim, softmax_scale, num_splits, out, out_row_stride, nullptr, 0, stream,
                     kDecodeScratchBytes, scratch_on_current_device);
}

int nva_gather_kv(const void* k_cache, const void* v_cache, int32_t kv_dtype, const float* k_scale,
                  const float* v_scale, int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                  int32_t max_blocks_per_seq, int32_t block_size, const int32_t* cu_seqlens_k, int32_t num_seqs,
                  int32_t max_seqlen_k, int32_t num_kv_heads, int32_t head_dim, void* k_out, void* v_out,
                  int64_t out_rows, int64_t out_row_stride, void* stream) {
  if (kv_dtype != NVA_DTYPE_BF16 && kv_dtype != NVA_DTYPE_FP8_E4M3)
    return fail(NVA_ERR_INVALID_ARGUMENT, "unknown kv dtype %d", kv_dtype);
  if (num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 != 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_kv_heads must be positive and head_dim a positive multiple of 8");
  if (num_seqs < 0 || max_seqlen_k < 0 || out_rows < 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_seqs, max_seqlen_k and out_rows must be >= 0");
  if (num_seqs > 65535) return fail(NVA_ERR_UNSUPPORTED, "num_seqs above 65535");
  if (block_size <= 0 || max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq || num_blocks <= 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "block table shape is inconsistent");
  const int64_t D = static_cast<int64_t>(num_kv_heads) * head_dim;
  if (D > (1 << 20)) return fail(NVA_ERR_UNSUPPORTED, "num_kv_heads*head_dim above 2^20");
  if (out_row_stride < D || out_row_stride % 8)
    return fail(NVA_ERR_INVALID_ARGUMENT, "out_row_stride must be >= num_kv_heads*head_dim and a multiple of 8");
  if (num_seqs == 0 || max_seqlen_k == 0 || out_rows == 0) return ok();
  if (!k_cache || !v_cache || !block_table || !cu_seqlens_k || !k_out || !v_out)
    return fail(NVA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (kv_dtype == NVA_DTYPE_FP8_E4M3 && (!k_scale || !v_scale))
    return fail(NVA_ERR_INVALID_ARGUMENT, "fp8 kv cache needs k_scale and v_scale");
  if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(k_out, 16) || !aligned(v_out, 16))
    return fail(NVA_ERR_INVALID_ARGUMENT, "caches and outputs must be 16-byte aligned");
  if (!aligned(block_table, 4) || !aligned(cu_seqlens_k, 4))
    return fail(NVA_ERR_INVALID_ARGUMENT, "index tensors must be 4-byte aligned");
  nva::GatherParams p{};
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.block_table = block_table;
  p.cu_k = cu_seqlens_k;
  p.k_out = k_out;
  p.v_out = v_out;
  p.bt_row_stride = bt_row_stride;
  p.num_blocks = num_blocks;
  p.out_rows = out_rows;
  p.out_row_stride = out_row_stride;
  p.max_blocks = max_blocks_per_seq;
  p.block_size = block_size;
  p.num_seqs = num_seqs;
  p.row_elems = static_cast<int32_t>(D);
  p.head_dim = head_dim;
  return hip_status(nva::launch_gather_kv(p, max_seqlen_k, kv_dtype, static_cast<hipStream_t>(stream)),
                    "gather_kv launch");
}

int nva_qk_norm_rope(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride, void* q_out,
                     int64_t q_out_row_stride, void* k_out, int64_t k_out_row_stride, const void* q_norm_weight,
                     const void* k_norm_weight, float eps, const float* cos_sin_cache, int64_t max_position,
                     const int64_t* positions, int64_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, void* stream) {
  if (num_tokens < 0) return fail(NVA_ERR_INVALID_ARGUMENT, "num_tokens must be >= 0 (got %lld)", (long long)num_tokens);
  if (num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return fail(NVA_ERR_INVALID_ARGUMENT, "num_heads, num_kv_heads and head_dim must be positive");
  if (head_dim != 64 && head_dim != 128)
    return fail(NVA_ERR_UNSUPPORTED, "head_dim %d not supported (64 or 128)", head_dim);
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr))
    return fail(NVA_ERR_INVALID_ARGUMENT, "pass both norm weights (qk-norm) or neither (rotary embedding only)");
  if (q_norm_weight && !(eps >= 0.f)) return fail(NVA_ERR_INVALID_ARGUMENT, "eps must be >= 0");
  if (max_position <= 0) return fail(NVA_ERR_INVALID_ARGUMENT, "max_position must be positive");
  if (num_tokens == 0) return ok();
  if (!q || !k || !q_out || !k_out || !cos_sin_cache || !positions)
    return fail(NVA_ERR_INVALID_ARGUMENT, "null pointer argument");
  const int64_t hd = static_cast<int64_t>(num_heads) * head_dim;
  const int64_t kd = static_cast<int64_t>(num_kv_heads) * head_dim;
  if (q_row_stride < hd || q_out_row_stride < hd)
    return fail(NVA_ERR_INVALID_ARGUMENT, "q/q_out row strides must be >= num_heads*head_dim");
  if (k_row_stride < kd || k_out_row_stride < kd)
    return fail(NVA_ERR_INVALID_ARGUMENT, "k/k_out row strides must be >= num_kv_heads*head_dim");
  const uintptr_t a = head_dim == 128 ? 8 : 4;  // bytes each lane moves per half row
  if (!aligned(q, a) || !aligned(k, a) || !aligned(q_out, a) || !aligned(k_out, a) ||
      (q_norm_weight && (!aligned(q_norm_weight, a) || !aligned(k_norm_weight, a))) ||
      (q_row_stride * 2) % a || (k_row_stride * 2) % a || (q_out_row_stride * 2) % a || (k_out_row_stride * 2) % a)
    return fail(NVA_ERR_UNSUPPORTED, "q/k rows and weights must be %d-byte aligned", (int)a);
  if (!aligned(cos_sin_cache, 4) || !aligned(positions, 8))
    return fail(NVA_ERR_INVALID_ARGUMENT, "cos_sin_cache must be 4-byte and positions 8-byte aligned");
  if (num_tokens * (num_heads + num_kv_heads) > (int64_t{1} << 36))
    return fail(NVA_ERR_UNSUPPORTED, "num_tokens*(num_heads+num_kv_heads) above 2^36");

  nva::QKNormRopeParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.q_out = static_cast<uint16_t*>(q_out);
  p.k_out = static_cast<uint16_t*>(k_out);
  p.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  p.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  p.cos_sin = cos_sin_cache;
  p.positions = positions;
  p.q_row_stride = q_row_stride;
  p.k_row_stride = k_row_stride;
  p.q_out_row_stride = q_out_row_stride;
  p.k_out_row_stride = k_out_row_stride;
  p.num_tokens = num_tokens;
  p.max_position = max_position;
  p.num_heads = num_heads;
  p.num_kv_heads = num_kv_heads;
  p.head_dim = head_dim;
  p.eps = eps;
  return hip_status(nva::launch_qk_norm_rope(p, static_cast<hipStream_t>(stream)), "qk_norm_rope launch");
}

}  // extern "C"
