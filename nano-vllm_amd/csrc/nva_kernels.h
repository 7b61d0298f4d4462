// Kernel parameter blocks and launchers (internal; the public surface is
// include/nva_attention.h).  All sizes and strides are in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nva {

struct StoreParams {
  const void* key;            // bf16 (T, nkv, d)
  const void* value;          // bf16 (T, nkv, d)
  void* k_cache;              // (num_slots, nkv*d) bf16 or fp8
  void* v_cache;
  const int32_t* slot_mapping;
  const float* k_scale;       // [nkv], fp8 only
  const float* v_scale;
  int64_t key_row_stride;
  int64_t value_row_stride;
  int64_t num_slots;
  int64_t num_tokens;
  int32_t row_elems;          // nkv * d
  int32_t head_dim;
  int32_t cache_dtype;        // 0 bf16, 1 fp8 e4m3fn
};

struct DecodeParams {
  const uint16_t* q;          // (B, nh, d) bf16, head stride d
  const void* k_cache;        // (num_blocks, block_size, nkv, d)
  const void* v_cache;
  const float* k_scale;       // [nkv] (fp8) or null
  const float* v_scale;
  const int32_t* seqlens;     // [B]
  const int32_t* block_table; // [B, bt_row_stride]
  uint16_t* out;              // (B, nh, d) bf16
  float* ws_o;                // [slots, nh, d] partial numerators
  float* ws_ml;               // [slots, nh, 2] partial (max, sum)
  int32_t* ws_prefix;         // [B + 1] step prefix (balanced mode)
  int64_t q_row_stride;
  int64_t out_row_stride;
  int64_t bt_row_stride;
  int64_t num_blocks;
  int32_t batch;
  int32_t max_blocks;         // usable block-table width
  int32_t block_size;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t group;              // num_heads / num_kv_heads
  int32_t keys_per_split;     // fixed mode: multiple of block_size
  int32_t num_splits;         // fixed mode: splits per sequence
  int32_t balanced_ranges;    // balanced mode: number of step ranges P (0 = fixed mode)
  int32_t spread;             // > 0: spread mode with that many shares per sequence (small batches)
  int32_t head_dim;           // 64 or 128
  // Store fused into the decode launch (null new_k: none): row b of new_k /
  // new_v (bf16, nkv * d elements) goes to cache slot slot_mapping[b].  Rows
  // of sequences with keys are stored by the wave that reads key ctx-1; rows
  // of sequences with none are stored by the merge kernel, after every read.
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t new_k_stride;
  int64_t new_v_stride;
  const int32_t* slot_mapping;
  float scale_log2;           // softmax_scale * log2(e)
  int32_t kv_fp8;             // 1: e4m3fn cache (k_scale / v_scale), 0: bf16
};

struct PrefillParams {
  const uint16_t* q;          // (Tq, nh, d) bf16
  const uint16_t* k;          // packed (Tk, nkv, d) or cache (slots, nkv, d)
  const uint16_t* v;
  const int32_t* block_table; // null => packed
  const int32_t* cu_q;        // [S+1]
  const int32_t* cu_k;        // [S+1]
  uint16_t* out;              // (Tq, nh, d)
  int64_t q_row_stride;
  int64_t k_row_stride;
  int64_t v_row_stride;
  int64_t out_row_stride;
  int64_t bt_row_stride;
  int64_t num_blocks;
  int32_t max_blocks;
  int32_t block_size;
  int32_t num_seqs;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t group;
  int32_t num_q_tiles;        // ceil(max_seqlen_q / positions_per_tile)
  int32_t positions_per_tile; // query positions per workgroup (x group = rows)
  int32_t head_dim;           // 64 or 128
  float scale_log2;
  uint32_t* queue;            // null: static item order; else kPrefillQueueWords zeroed words
  // Key halving of the direct grid: items of at least split_tiles
  // key tiles (0: off) run as two workgroups over the two halves of their key
  // tiles, merged by the second to arrive.  At most split_slots such items;
  // each has kPrefillSplitCtlWords control words in split_ctl and
  // kPrefillSplitPartFloats floats of partial results in split_part.
  int32_t split_tiles;
  int32_t split_slots;
  int32_t split_cus;          // compute units: with the real items, they cap the split items
  uint32_t* split_ctl;
  float* split_part;
  // split_err[0]: error bits (kPrefillErrSplitWait), set by the kernel, cleared
  // only by the host; split_err[1]: the merge wait's poll limit (0: the
  // default bound, n > 0: n - 1 polls), written by the host.
  uint32_t* split_err;
};

struct QKNormRopeParams {
  const uint16_t* q;          // (T, nh, d) bf16, head stride d
  const uint16_t* k;          // (T, nkv, d) bf16, head stride d
  uint16_t* q_out;            // may alias q
  uint16_t* k_out;            // may alias k
  const uint16_t* q_weight;   // (d,) bf16 q_norm weight, or null: rotary embedding only
  const uint16_t* k_weight;   // (d,) bf16 k_norm weight (null iff q_weight is)
  const float* cos_sin;       // (max_position, d) fp32: [cos(d/2) | sin(d/2)] per position
  const int64_t* positions;   // (T,)
  int64_t q_row_stride, k_row_stride, q_out_row_stride, k_out_row_stride;
  int64_t num_tokens;
  int64_t max_position;
  int32_t num_heads, num_kv_heads, head_dim;
  float eps;
};

// Paged cache -> packed bf16 rows (gather_kv.hip).
struct GatherParams {
  const void* k_cache;        // (num_blocks, block_size, nkv, d) bf16 or fp8
  const void* v_cache;
  const float* k_scale;       // [nkv] (fp8) or null
  const float* v_scale;
  const int32_t* block_table; // [num_seqs, bt_row_stride]
  const int32_t* cu_k;        // [num_seqs + 1]
  void* k_out;                // packed (out_rows, out_row_stride) bf16
  void* v_out;
  int64_t bt_row_stride;
  int64_t num_blocks;
  int64_t out_rows;
  int64_t out_row_stride;
  int32_t max_blocks;
  int32_t block_size;
  int32_t num_seqs;
  int32_t row_elems;          // nkv * d
  int32_t head_dim;
};

hipError_t launch_store_kvcache(const StoreParams& p, int vec_bytes, hipStream_t stream);
hipError_t launch_gather_kv(const GatherParams& p, int max_seqlen_k, int kv_dtype, hipStream_t stream);
hipError_t launch_qk_norm_rope(const QKNormRopeParams& p, hipStream_t stream);
hipError_t launch_decode(const DecodeParams& p, int kv_dtype, hipStream_t stream);
hipError_t launch_prefill(const PrefillParams& p, int max_seqlen_q, int max_seqlen_k, hipStream_t stream);
int prefill_positions_per_tile(int group);  // query positions one prefill workgroup covers
constexpr int kPrefillMaxGroup = 256;        // rows per prefill workgroup bound the GQA group
// Work queue of the persistent prefill grid: one claim counter per XCD lane,
// then the count of finished workgroups.  Zero on entry, zero again on exit.
constexpr int kPrefillQueueLanes = 8;
constexpr int kPrefillQueueWords = kPrefillQueueLanes + 1;
// Key-halved items of the direct grid: three control words per slot at byte
// kPrefillSplitCtlOffset -- an arrival count (two per use: the even arrival
// publishes its partial, the odd one merges), a ready word (the slot's epoch
// + 1 once the partial is published) and the slot's epoch (uses completed) --
// then one partial per slot from kPrefillSplitPartOffset: O (256 rows x up to
// 128 head dims, float32, unnormalised) and each row's maximum and sum.  A
// zeroed workspace is a valid start; every call leaves the words consistent
// (arrival count = 2 x epoch, ready word <= epoch), so a ready word left by
// an earlier call never matches a later one.
// 128 slots: a one-kv-head launch (a tensor-parallel share) splits up to 128 items,
// as many as its free CUs take (64 slots held config 4's TP8 share at 44.3 us, 128
// bring it to 41.9 us).
constexpr int kPrefillSplitSlots = 128;
constexpr int kPrefillSplitCtlWords = 3;
constexpr int64_t kPrefillSplitPartFloats = 256 * 128 + 2 * 512;
constexpr int64_t kPrefillErrOffset = 128;  // error word, then the poll-limit word
constexpr int64_t kPrefillSplitCtlOffset = 256;
constexpr int64_t kPrefillSplitPartOffset = 2048;
constexpr int64_t kPrefillWorkspaceBytes = kPrefillSplitPartOffset + kPrefillSplitSlots * kPrefillSplitPartFloats * 4;
static_assert(kPrefillSplitCtlOffset + 4 * kPrefillSplitCtlWords * kPrefillSplitSlots <= kPrefillSplitPartOffset,
              "control words fit");
static_assert(kPrefillQueueWords * 4 <= kPrefillErrOffset && kPrefillErrOffset + 8 <= kPrefillSplitCtlOffset,
              "error words fit between the queue and the control words");
// Error bit: a key-half merge gave up waiting for its partial (the item's rows
// were written as NaN).
constexpr uint32_t kPrefillErrSplitWait = 1u;
// Static device scratch of nva_decode_noalloc (bytes, per GPU).
constexpr int64_t kDecodeScratchBytes = int64_t{32} << 20;
static_assert(kPrefillQueueWords * 4 <= kPrefillSplitCtlOffset, "queue fits the workspace");

// Split-K plan shared by nva_decode and nva_decode_workspace_bytes.
// balanced_ranges > 0: balanced mode with that many step ranges; otherwise
// fixed mode with num_splits splits of pages_per_split pages per sequence.
struct DecodePlan {
  int32_t pages_per_split;
  int32_t num_splits;
  int32_t balanced_ranges;
  int32_t spread;             // > 0: spread mode, shares per sequence
  int64_t partial_slots;      // partial (O, max, sum) slots the workspace holds
};
// Spread mode (small batches): the largest batch * num_kv_heads it serves, the
// waves it aims for in total, and the widest block table (one wave holds a row,
// one entry per lane).
constexpr int kSpreadMaxPairs = 256;
constexpr int kSpreadTargetWaves = 1024;
// Shares per (sequence, kv head): the merge then folds one batch of loads
// (captured batch 1, context 1024: 16 shares 9.6 us per layer, 8 shares 10.6, 32 shares 11.6).
constexpr int kSpreadMaxShares = 16;
constexpr int kWgMaxBlocks = 64;

DecodePlan plan_decode(int32_t batch, int32_t num_kv_heads, int32_t max_blocks,
                       int32_t block_size, int32_t kv_dtype, int32_t requested_splits);

}  // namespace nva
