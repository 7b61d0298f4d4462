/*
 * nva_attention.h -- C ABI of the MI355X (gfx950) attention hot path of nano-vllm.
 *
 * Three device operations replace the three native calls inside
 * nanovllm/layers/attention.py (reference, read-only):
 *   nva_store_kvcache  <- store_kvcache / store_kvcache_kernel   attention.py:10-39
 *   nva_prefill        <- flash_attn_varlen_func(..., causal=True,
 *                         block_table=None | block_tables)         attention.py:67-73
 *   nva_decode         <- flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 *                         cache_seqlens, block_table, softmax_scale,
 *                         causal=True)                             attention.py:74-77
 * plus the decode branch of Attention.forward as one call (store, then decode):
 *   nva_store_decode   <- store_kvcache + flash_attn_with_kvcache    attention.py:58-79
 * and one fused producer step just before attention:
 *   nva_qk_norm_rope   <- q_norm / k_norm + rotary_emb             qwen3.py:91-105
 *
 * Conventions shared by every entry point
 *   - Plain pointers to device memory, sizes and strides in ELEMENTS (not bytes).
 *   - Queries, keys, values and outputs are bf16 (the model dtype, model_runner.py:33).
 *   - Paged caches are (num_blocks, block_size, num_kv_heads, head_dim), contiguous:
 *     one slot is num_kv_heads*head_dim elements (the layout model_runner.py:136-148
 *     allocates and attention.py:37 asserts).  A cache may hold bf16 or OCP fp8 e4m3fn
 *     (NVA_DTYPE_FP8_E4M3) with one fp32 scale per kv head: real = fp8 * scale[h].
 *   - Index tensors (slot_mapping, cu_seqlens, cache_seqlens, block tables) are int32,
 *     as the reference's producers build them (model_runner.py:151-249).
 *   - `stream` is a hipStream_t; every launch is enqueued on it, nothing synchronises,
 *     nothing reads device memory on the host and nothing allocates device memory, so
 *     the calls can be captured into a HIP graph (model_runner.py:296-336).
 *   - Return 0 on success, otherwise an NVA_ERR_* code with a message retrievable by
 *     nva_last_error() (thread-local).  Argument checks run before any HIP call, so
 *     they are testable on a machine without a GPU; a rejected call writes nothing.
 */
#ifndef NVA_ATTENTION_H
#define NVA_ATTENTION_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVA_OK 0
#define NVA_ERR_INVALID_ARGUMENT 1 /* shape, stride, alignment or pointer is wrong */
#define NVA_ERR_UNSUPPORTED 2      /* valid but not implemented (e.g. head_dim 96) */
#define NVA_ERR_HIP 3              /* the HIP runtime rejected a launch */
#define NVA_ERR_WORKSPACE 4        /* workspace missing or smaller than required */

#define NVA_DTYPE_BF16 0
#define NVA_DTYPE_FP8_E4M3 1

/* Library version (major*10000 + minor*100 + patch). */
int nva_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* nva_last_error(void);

/*
 * Scatter new keys/values into the paged caches.
 * Replaces store_kvcache(key, value, k_cache, v_cache, slot_mapping), attention.py:32-39,
 * and its Triton kernel store_kvcache_kernel, attention.py:10-29:
 *   k_cache.flat[slot*D : slot*D + D] = key[i]      (D = num_kv_heads * head_dim)
 * key/value are (num_tokens, num_kv_heads, head_dim) with head stride head_dim and
 * element stride 1 (the asserts at attention.py:35-36); their row strides are free
 * (value is a strided view of the fused qkv projection, qwen3.py:89).
 * A slot outside [0, num_slots) is skipped (the reference has no guard; CUDA-graph
 * padding rows would otherwise write slot 0).  For a bf16 cache the copy is bit-exact.
 * For an fp8 cache each element is stored as e4m3fn(float(x) / scale[h]) with
 * round-to-nearest-even; a magnitude above 464 (one that rounds past 448), an
 * infinity or a NaN becomes NaN (0x7f | sign), bit-identical to
 * (x.float() / scale).to(torch.float8_e4m3fn).
 */
int nva_store_kvcache(const void* key, int64_t key_row_stride,
                      const void* value, int64_t value_row_stride,
                      void* k_cache, void* v_cache, int64_t num_slots,
                      const int32_t* slot_mapping, int64_t num_tokens,
                      int32_t num_kv_heads, int32_t head_dim, int32_t cache_dtype,
                      const float* k_scale, const float* v_scale, void* stream);

/*
 * Varlen causal prefill.  Replaces flash_attn_varlen_func(q, k, v, max_seqlen_q,
 * cu_seqlens_q, max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True, block_table),
 * attention.py:67-73.
 * q: (total_q, num_heads, head_dim); out: same shape.
 * block_table == NULL: k/v are packed (total_k, num_kv_heads, head_dim) rows addressed by
 *   cu_seqlens_k (row strides k_row_stride / v_row_stride, head stride head_dim).
 * block_table != NULL: k/v are the paged caches (prefix-cache case, attention.py:68-69);
 *   key j of sequence s lives in block block_table[s*bt_row_stride + j/block_size].
 * Causal masking is bottom-right aligned: query i of a sequence with Lq queries and Lk
 * keys sees keys j <= i + (Lk - Lq).  A query row with no visible key yields zeros.
 * max_seqlen_q bounds the launch grid (host value, graph-capture safe).
 * head_dim 64 or 128; a paged cache needs block_size % 64 == 0 and bf16.
 * workspace: NULL, or nva_prefill_workspace_bytes() bytes (about 17.3 MB), 256-byte aligned,
 *   holding zeros before its first use.  With it, a prefill over many work items hands
 *   them out dynamically (a work queue per XCD), and a prefill over few items (at most two
 *   per CU; paged caches with blocks of at most 512 keys) runs its longest items as two
 *   halves of their key range (cut at a page boundary when paged), merged
 *   in the launch through float32 partials kept in the workspace.  Every completed call
 *   leaves the workspace's control words consistent (queue counters zero; each half slot's
 *   arrival count, ready word and epoch advanced together), so it is allocated and cleared
 *   once and reused.  Calls that may run at the same time (different streams) need
 *   different workspaces.  NULL selects a static item order and whole items: bit-identical
 *   to the work queue, and within float32 rounding of the halves (the merge reassociates
 *   sums).  Should a half's wait for the other half's partial ever give up (a bounded wait
 *   of about 30 ms; words out of step), that item's rows are written as NaN and bit
 *   NVA_PREFILL_ERR_SPLIT_WAIT is set in the workspace's error word (read and cleared by
 *   nva_prefill_workspace_errors).  The 32-bit word at byte 132 of the workspace bounds
 *   that wait: 0 (as zeroed) is the default bound, n > 0 allows n - 1 polls (a test hook).
 */
int nva_prefill(const void* q, int64_t q_row_stride,
                const void* k, int64_t k_row_stride,
                const void* v, int64_t v_row_stride,
                const int32_t* block_table, int64_t bt_row_stride,
                int32_t max_blocks_per_seq, int32_t block_size, int64_t num_blocks,
                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                float softmax_scale,
                void* out, int64_t out_row_stride,
                void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the optional nva_prefill workspace (a constant of the library). */
int64_t nva_prefill_workspace_bytes(void);

/*
 * Error bits a prefill workspace has collected, copied to *errors and cleared (no
 * counterpart in the reference, where flash-attn keeps no state between calls).
 * NVA_PREFILL_ERR_SPLIT_WAIT: a key-half merge gave up waiting; that item's output rows
 * were written as NaN.  Ordered on `stream` after the calls before it, and the one entry
 * point that waits for the stream: for diagnostics and tests, not for captured graphs.
 */
#define NVA_PREFILL_ERR_SPLIT_WAIT 1u
int nva_prefill_workspace_errors(void* workspace, int64_t workspace_bytes, uint32_t* errors, void* stream);

/*
 * Workspace bytes nva_decode needs for these launch parameters (0 if it needs none).
 * Depends only on host-side sizes, never on device contents.
 */
int64_t nva_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t max_blocks_per_seq,
                                   int32_t block_size, int32_t kv_dtype, int32_t num_splits);

/*
 * Paged GQA decode: one query token per sequence over cache_seqlens[b] cached keys.
 * Replaces flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 * cache_seqlens=context_lens, block_table=block_tables, softmax_scale, causal=True),
 * attention.py:75-77 (causal is a no-op for one query).
 * q/out: (batch, num_heads, head_dim).  block_table: (batch, >= max_blocks_per_seq).
 * num_splits: 0 picks a split-K count from the sizes; n > 0 requests about n splits per
 * sequence (as flash-attn's num_splits).  The key range of a sequence is clamped to
 * max_blocks_per_seq*block_size; a block id outside [0, num_blocks) makes its keys
 * masked; a sequence with no key yields zeros.
 * kv_dtype NVA_DTYPE_FP8_E4M3: caches are e4m3fn with per-kv-head scales k_scale/v_scale.
 * head_dim 64 or 128 for a bf16 cache; an fp8 cache needs head_dim 128.  GQA group <= 16,
 * block_size a multiple of 32.
 */
int nva_decode(const void* q, int64_t q_row_stride,
               const void* k_cache, const void* v_cache, int32_t kv_dtype,
               const float* k_scale, const float* v_scale, int64_t num_blocks,
               const int32_t* cache_seqlens, const int32_t* block_table,
               int64_t bt_row_stride, int32_t max_blocks_per_seq, int32_t block_size,
               int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
               float softmax_scale, int32_t num_splits,
               void* out, int64_t out_row_stride,
               void* workspace, int64_t workspace_bytes, void* stream);

/*
 * One decode step of Attention.forward (attention.py:58-79, decode branch): the store of the
 * new token's key/value rows (store_kvcache, attention.py:32-39 / 10-29) followed by the paged
 * decode (flash_attn_with_kvcache, attention.py:75-77).  key/value: (batch, num_kv_heads,
 * head_dim) bf16 rows at key_row_stride / value_row_stride; slot_mapping: (batch,) int32, slots
 * outside [0, num_blocks*block_size) skipped; every other argument as nva_decode (same workspace,
 * nva_decode_workspace_bytes).  It has no single counterpart in the reference.
 * When nva_decode's plan is the small-batch spread mode (with more than one share per
 * sequence), or the balanced mode over a bf16 cache, the store runs inside the decode call
 * with no extra launch: for a sequence with keys, the wave that reads key cache_seqlens[b]-1
 * writes the new rows and uses them from registers; the rows of a sequence with none
 * (cache_seqlens[b] == 0, e.g. a padded graph row) are written by the merge kernel, after
 * every read of the call.  The result is deterministic for any input and equals
 * store-then-decode when (a) slot_mapping[b] is the slot of key cache_seqlens[b]-1 for every
 * sequence with keys, as every decode step the reference runs has it (prepare_decode,
 * model_runner.py:218-229), and (b) no sequence reads the slot of a row with no keys.  The
 * reference's graph replay breaks (b): run_model zero-fills slot_mapping
 * (model_runner.py:271-273), so padded rows write slot 0, which a live sequence may own; here
 * that sequence reads slot 0's previous contents, the two calls would show it the padded row.
 * A runner that pads with slot -1 meets (b).  A sequence with keys whose slot breaks (a)
 * leaves the attention over that slot unspecified (the store itself is done).  Other plans
 * (fixed splits, an fp8 cache in balanced mode, one spread share) run the store kernel, then
 * the decode: exactly the two calls.  The fused paths need fewer than 2^31 slots in the pool
 * (num_blocks * block_size); larger pools store first.
 */
int nva_store_decode(const void* key, int64_t key_row_stride,
                     const void* value, int64_t value_row_stride,
                     const int32_t* slot_mapping,
                     const void* q, int64_t q_row_stride,
                     void* k_cache, void* v_cache, int32_t kv_dtype,
                     const float* k_scale, const float* v_scale, int64_t num_blocks,
                     const int32_t* cache_seqlens, const int32_t* block_table,
                     int64_t bt_row_stride, int32_t max_blocks_per_seq, int32_t block_size,
                     int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                     float softmax_scale, int32_t num_splits,
                     void* out, int64_t out_row_stride,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Gather each sequence's keys and values from the paged caches into packed bf16 rows:
 * key j of sequence s (block block_table[s*bt_row_stride + j/block_size], j < cu_seqlens_k[s+1] -
 * cu_seqlens_k[s]) goes to row cu_seqlens_k[s] + j of k_out / v_out.  An fp8 e4m3fn cache is
 * dequantised (bf16(e4m3 * scale[h]), round to nearest even); a bf16 cache is copied bit for bit.
 * This is the prefix-cached prefill over an fp8 cache (attention.py:68-73 reads k_cache/v_cache
 * through block_table): gather, then nva_prefill on the packed rows (block_table NULL).  It has no
 * single counterpart in the reference, where flash_attn_varlen_func reads the pages itself.
 * Keys on a block id outside [0, num_blocks) or past max_blocks_per_seq become zero rows; rows at or
 * beyond out_rows are not written.  max_seqlen_k bounds the launch grid (keys of a sequence beyond
 * it are not gathered).  head_dim a multiple of 8; out_row_stride a multiple of 8 elements.
 */
int nva_gather_kv(const void* k_cache, const void* v_cache, int32_t kv_dtype,
                  const float* k_scale, const float* v_scale, int64_t num_blocks,
                  const int32_t* block_table, int64_t bt_row_stride,
                  int32_t max_blocks_per_seq, int32_t block_size,
                  const int32_t* cu_seqlens_k, int32_t num_seqs, int32_t max_seqlen_k,
                  int32_t num_kv_heads, int32_t head_dim,
                  void* k_out, void* v_out, int64_t out_rows, int64_t out_row_stride,
                  void* stream);

/*
 * nva_decode without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP-graph capture, tight serving loops, harnesses that forbid hipMalloc).  It has
 * no counterpart in the reference.  Same arguments, checks and results as nva_decode (the same
 * kernels, bit for bit); the split-K partials live in a static __device__ array of the library
 * (nva_decode_noalloc_max_workspace_bytes() bytes, 32 MiB, on each GPU the library runs on,
 * held until the process ends).  A call whose nva_decode_workspace_bytes exceeds that size is
 * refused with NVA_ERR_WORKSPACE before any HIP call.  Nothing is allocated or freed, and nothing
 * in the array needs to start at zero.  Every call on one GPU shares that GPU's array: calls
 * that can overlap on one GPU (different streams, or a graph replay concurrent with another
 * call) race and must not be issued.
 */
int nva_decode_noalloc(const void* q, int64_t q_row_stride,
                       const void* k_cache, const void* v_cache, int32_t kv_dtype,
                       const float* k_scale, const float* v_scale, int64_t num_blocks,
                       const int32_t* cache_seqlens, const int32_t* block_table,
                       int64_t bt_row_stride, int32_t max_blocks_per_seq, int32_t block_size,
                       int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                       float softmax_scale, int32_t num_splits,
                       void* out, int64_t out_row_stride, void* stream);

/* Size in bytes of nva_decode_noalloc's static scratch (the largest workspace it serves). */
int64_t nva_decode_noalloc_max_workspace_bytes(void);

/*
 * Fused per-head RMSNorm + rotary embedding of q and k: the producer step feeding the
 * path.  Replaces, in Qwen3Attention.forward (qwen3.py:91-105),
 *   q = q_norm(q.view(T, nh, d)); k = k_norm(k.view(T, nkv, d))   layernorm.py:17-27
 *   q, k = rotary_emb(positions, q, k)                             rotary_embedding.py:37-55
 * q/k: (num_tokens, heads, head_dim) bf16 rows with head stride head_dim and free row
 * strides (views into the fused qkv projection, qwen3.py:89); outputs have the same
 * layout and may alias the inputs (in place).  q_norm_weight/k_norm_weight: bf16
 * (head_dim,), both NULL for the rotary embedding alone (Qwen2, qwen2.py:91-92).
 * cos_sin_cache: fp32 (max_position, head_dim), row p = [cos(p*f) | sin(p*f)] as
 * RotaryEmbedding builds it (rotary_embedding.py:29-35); positions: int64 (num_tokens,),
 * clamped to [0, max_position).  head_dim 64 or 128.  Results follow the reference's
 * eager rounding steps; the sum of squares runs in a different order, so an output can
 * differ from the reference's by one bf16 ulp.
 */
int nva_qk_norm_rope(const void* q, int64_t q_row_stride,
                     const void* k, int64_t k_row_stride,
                     void* q_out, int64_t q_out_row_stride,
                     void* k_out, int64_t k_out_row_stride,
                     const void* q_norm_weight, const void* k_norm_weight, float eps,
                     const float* cos_sin_cache, int64_t max_position,
                     const int64_t* positions, int64_t num_tokens,
                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVA_ATTENTION_H */
