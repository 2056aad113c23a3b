/*
 * nvs_attention.h — C ABI of the MI355X (gfx950) paged-KV attention library
 * (libnvs_attention.so).
 *
 * These entry points replace the tensor-level operations behind
 * nanovllm/layers/attention.py:PagedAttention in the reference (nanovllm_self):
 * the KV-cache write, the per-token KV quantisation, the paged gather used by
 * the eager path, and the varlen / paged causal attention that the reference
 * delegates to flash_attn_varlen_func.  Each declaration cites the reference
 * code it replaces.
 *
 * Conventions shared by every entry point
 *  - All pointers are device pointers owned by the caller; the library never
 *    allocates, frees or retains them.  `stream` is a hipStream_t (NULL = the
 *    default stream).  Every call is asynchronous on `stream`: no host sync,
 *    no device allocation, so calls are safe inside HIP-graph capture as long
 *    as the caller's buffers stay alive.
 *  - Strides are in elements, not bytes.  The innermost (head_dim) dimension
 *    of every tensor must be contiguous.
 *  - KV cache layout (reference model_runner.py:40-50, 302-331): one layer's
 *    K (or V) cache is a contiguous [num_blocks, block_size, num_kv_heads,
 *    head_dim] array; a token at slot s = block_id * block_size + offset lives
 *    at element offset (s * num_kv_heads + h) * head_dim.  Quantised caches add
 *    a contiguous fp32 scale array [num_blocks, block_size, num_kv_heads]
 *    (reference model_runner.py:52-73, the trailing dim of 1 is implicit).
 *  - Return value: NVS_OK (0) on success, a negative NVS_ERR_* code otherwise;
 *    nvs_last_error() then returns a message describing the failure (per
 *    calling thread).  Arguments are validated before anything is launched.
 */
#ifndef NVS_ATTENTION_H
#define NVS_ATTENTION_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types.  INT8 is the reference's "int8_mock" symmetric per-token,
 * per-kv-head quantisation (attention.py:63-98); FP8_E4M3 is OCP
 * float8_e4m3fn with the same per-token, per-kv-head scale layout. */
enum nvs_dtype {
  NVS_DTYPE_BF16 = 0,
  NVS_DTYPE_FP16 = 1,
  NVS_DTYPE_FP32 = 2,
  NVS_DTYPE_INT8 = 3,
  NVS_DTYPE_FP8_E4M3 = 4
};

enum nvs_status {
  NVS_OK = 0,
  NVS_ERR_INVALID = -1,     /* bad shape / stride / pointer argument   */
  NVS_ERR_UNSUPPORTED = -2, /* valid request this build does not serve */
  NVS_ERR_WORKSPACE = -3,   /* workspace missing or too small          */
  NVS_ERR_LAUNCH = -4       /* HIP reported an error at launch         */
};

/* Message for the last failing call on this thread ("" if none). */
const char* nvs_last_error(void);

/* Library version, major * 10000 + minor * 100 + patch. */
int nvs_version(void);

/*
 * KV-cache write.  Replaces PagedAttention.store_kv_cache_torch
 * (reference attention.py:139-189, dispatched from write_kv_cache :120-136).
 *   k, v          [num_tokens, num_kv_heads, head_dim] of src_dtype
 *                 (BF16 / FP16 / FP32), strides (tok, head) in elements.
 *   slot_mapping  [num_tokens] int32; block = slot / block_size, offset =
 *                 slot % block_size.  Precondition (what the engine's
 *                 prepare_model_input builds, model_runner.py:461-532):
 *                 every slot >= 0.  Outside it, slots < 0 are skipped (the
 *                 reference's slot // bs, slot % bs would wrap -1 to the
 *                 last row of the last block, attention.py:158-159); slots
 *                 >= num_blocks * block_size are skipped as well, so the
 *                 kernel never writes outside the cache.
 *   cache_dtype   BF16 / FP16 / FP32: the row is cast to the cache dtype with
 *                 round-to-nearest-even (the reference's k.to(cache_dtype)).
 *                 INT8: absmax = max|x| over head_dim in fp32,
 *                 scale = max(absmax / 127, 1e-6),
 *                 code = clamp(rint(x / scale), -127, 127), bit-exact with
 *                 quantize_int8_per_token (attention.py:94-98).
 *                 FP8_E4M3: scale = max(absmax / 448, 1e-6),
 *                 code = e4m3fn(clamp(x / scale, -448, 448)) with RNE.
 *   k_scale, v_scale  fp32 scale caches, required for INT8 / FP8_E4M3,
 *                 ignored otherwise.
 *   head_dim must be a multiple of 8 with head_dim / 8 a power of two <= 64.
 */
int nvs_store_kvcache(const void* k, const void* v, int src_dtype,
                      int64_t k_tok_stride, int64_t k_head_stride,
                      int64_t v_tok_stride, int64_t v_head_stride,
                      const int32_t* slot_mapping, int64_t num_tokens,
                      void* k_cache, void* v_cache, int cache_dtype,
                      float* k_scale, float* v_scale,
                      int64_t num_blocks, int block_size, int num_kv_heads,
                      int head_dim, void* stream);

/*
 * Fused pre-attention step of a Qwen3 attention layer: per-head RMSNorm of q
 * and k, rotary embedding of both, and the KV-cache write of the rotated k and
 * of v.  Replaces the sequence q_norm(q); k_norm(k); rotary_embedding(
 * positions, q, k); write_kv_cache(k, v, slot_mapping) of the reference
 * (nanovllm/models/qwen3.py:100-104 and :118 via attention.py:500-546, with
 * layers/RMSNorm.py:11-18, layers/RoPE.py:5-25 and 60-74,
 * attention.py:139-189).
 *   q [num_tokens, num_heads, head_dim], k, v [num_tokens, num_kv_heads,
 *     head_dim]: BF16, strides (tok, head) in elements.
 *   positions       [num_tokens] int64, clamped into [0, max_position).
 *   q/k_norm_weight [head_dim] BF16; eps the layers' rms_norm_eps.
 *   cos_sin_cache   [max_position, head_dim] fp32 (the rotary layer's buffer:
 *                   cos of the head_dim / 2 frequencies, then their sin).
 *   Per (token, head), in fp32 with every product and sum rounded on its own:
 *     rms = sqrt(mean(x^2) + eps); n = bf16((w * x) / rms);
 *     y1 = n1 cos - n2 sin, y2 = n2 cos + n1 sin over the halves n1, n2 of n;
 *     out = bf16(y1 ++ y2).
 *   q_out receives the rotated q; k_out (may be NULL) the rotated k; the
 *   cache write of the rotated k and of v follows nvs_store_kvcache (same
 *   slot rule, casts and quantisation).  head_dim must be 128.
 */
int nvs_qk_norm_rope_store(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                           const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                           const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                           const int64_t* positions, int64_t num_tokens,
                           const void* q_norm_weight, const void* k_norm_weight, float eps,
                           const float* cos_sin_cache, int64_t max_position,
                           const int32_t* slot_mapping, void* k_cache, void* v_cache,
                           int cache_dtype, float* k_scale, float* v_scale,
                           int64_t num_blocks, int block_size, int num_heads,
                           int num_kv_heads, int head_dim,
                           void* q_out, int64_t q_out_tok_stride, int64_t q_out_head_stride,
                           void* k_out, int64_t k_out_tok_stride, int64_t k_out_head_stride,
                           void* stream);

/*
 * Per-token, per-head quantisation of a [num_tokens, num_heads, head_dim]
 * tensor into contiguous codes (same shape) and fp32 scales
 * [num_tokens, num_heads].  Replaces PagedAttention.quantize_int8_per_token
 * (reference attention.py:63-98); code_dtype INT8 or FP8_E4M3, same
 * arithmetic as nvs_store_kvcache.
 */
int nvs_quantize_per_token(const void* x, int src_dtype, int64_t tok_stride,
                           int64_t head_stride, int64_t num_tokens,
                           int num_heads, int head_dim, void* codes,
                           int code_dtype, float* scales, void* stream);

/*
 * Dequantisation (codes * scale) rounded to out_dtype (BF16 / FP16 / FP32),
 * contiguous [num_tokens, num_heads, head_dim] in and out, scales
 * [num_tokens, num_heads].  Replaces dequantize_int8_per_token
 * (reference attention.py:100-117).
 */
int nvs_dequantize_per_token(const void* codes, int code_dtype,
                             const float* scales, int64_t num_tokens,
                             int num_heads, int head_dim, void* out,
                             int out_dtype, void* stream);

/*
 * Paged gather of the visible K/V of a batch, the eager path's
 * PagedAttention.get_kv_cache (reference attention.py:201-285).
 * For sequence i the non-negative entries of block_tables[i] are taken in
 * order (entries < 0 are dropped; the reference's row[row != -1] drops only
 * -1, and would index other negative ids from the end of the pool), flattened to
 * tokens and truncated to context_lens[i]; codes are dequantised to out_dtype
 * when cache_dtype is INT8 / FP8_E4M3, otherwise cast.  Positions past the
 * gathered length are zero and kv_mask (uint8, [num_seqs, max_len]) is 1
 * exactly on gathered positions.
 *   k_out, v_out  contiguous [num_seqs, max_len, num_kv_heads, head_dim].
 */
int nvs_gather_kvcache(const void* k_cache, const void* v_cache,
                       int cache_dtype, const float* k_scale,
                       const float* v_scale, const int32_t* block_tables,
                       int64_t bt_stride, int max_blocks_per_seq,
                       const int32_t* context_lens, int num_seqs, int max_len,
                       int64_t num_blocks, int block_size, int num_kv_heads,
                       int head_dim, void* k_out, void* v_out, int out_dtype,
                       uint8_t* kv_mask, void* stream);

/*
 * Workspace (bytes) that nvs_paged_attention / nvs_varlen_attention need for
 * a batch with these bounds: the prefill work plan the device builds from
 * cu_seqlens (a 256-byte header and the list of prefill query tiles)
 * followed by the decode partials (two slots of (num_heads / num_kv_heads) x
 * (head_dim + 2) floats per decode wave, for rows whose keys are split
 * across wave groups).  num_kv_heads <= 0 asks for an upper bound over every
 * kv-head count.  The workspace must be 256-byte aligned; it needs no
 * initialisation and is scratch between calls; calls that share one
 * workspace must be ordered on one stream.
 */
int64_t nvs_attention_workspace_bytes(int num_seqs, int max_seqlen_q,
                                      int max_seqlen_k, int num_heads,
                                      int num_kv_heads, int head_dim,
                                      int block_size);

/*
 * The same with the cache dtype: for an int8 / fp8 cache and a batch with
 * prefill rows (max_seqlen_q > 1) it adds room for a bf16 copy of the
 * prefill rows' keys and values (min(num_seqs x ceil(max_seqlen_k / 64),
 * 1 GiB / (64 x num_kv_heads x 128 x 4)) tiles of 64 keys), the copy the
 * reference's prefill_torch makes per sequence before it attends
 * (attention.py:268-273: (code.float() * scale).to(bf16)).  Given at least
 * this much, nvs_paged_attention dequantises into the copy and runs the
 * MFMA tile-loop prefill kernel on it; given only
 * nvs_attention_workspace_bytes(...), or a batch whose prefill rows need
 * more tiles, its prefill kernel dequantises inside its tile fill instead
 * (the same values, slower).  Other dtypes: the same as
 * nvs_attention_workspace_bytes.  num_kv_heads must be given (> 0).
 */
int64_t nvs_attention_workspace_bytes_cache(int num_seqs, int max_seqlen_q,
                                            int max_seqlen_k, int num_heads,
                                            int num_kv_heads, int head_dim,
                                            int block_size, int cache_dtype);

/*
 * Causal varlen attention over a paged KV cache: the paged call of
 * prefill_flashattn (reference attention.py:356-375,
 * flash_attn_varlen_func(..., block_table=...)) and equally the
 * prefix branch of prefill_torch (attention.py:441-498).  Serves prefix-hit
 * prefill, chunked prefill, decode (q_len == 1) and mixed batches in one call.
 *   q             [num_tokens, num_heads, head_dim] BF16 (FP16 with an FP16
 *                 cache), strides in elements.
 *   cu_seqlens_q  [num_seqs + 1] int32 prefix sums of the new-token counts.
 *   cu_seqlens_k  [num_seqs + 1] int32 prefix sums of the visible KV lengths
 *                 (cached prefix + new tokens, already written to the cache).
 *   block_tables  [num_seqs, bt_stride] int32; logical block j of sequence i
 *                 is block_tables[i * bt_stride + j].  Precondition (what
 *                 prepare_block_tables builds, model_runner.py:334-344):
 *                 -1 entries only after the last block that k_len keys
 *                 need.  Outside it, an entry < 0 inside k_len reads as
 *                 all-zero K and V at its logical positions, where the
 *                 reference's gather compacts (row[row != -1] drops a -1
 *                 and shifts later keys left, attention.py:255-275).
 *   Mask: query row r of a sequence with q_len new and k_len visible tokens
 *   attends keys j <= r + (k_len - q_len) (bottom-right causal); rows with no
 *   visible key produce 0.  GQA: query head hq reads kv head
 *   hq / (num_heads / num_kv_heads).
 *   cache_dtype   BF16, FP16, INT8 or FP8_E4M3 (scales required for the last
 *                 two).  An FP16 cache computes in fp16 (q, P and out fp16,
 *                 fp16 MFMA), as the reference's flash path computes in the
 *                 cache's dtype (attention.py:326-336); the others in bf16.
 *   out           [num_tokens, num_heads, head_dim] BF16 (FP16 with an FP16
 *                 cache).
 *   Rows with q_len == 1 run the split-K decode kernels, the others the MFMA
 *   prefill kernel; `workspace` holds at least
 *   nvs_attention_workspace_bytes(...) bytes.
 *   head_dim must be 128; num_heads / num_kv_heads must be 1..16;
 *   block_size must be a multiple of 64.
 */
int nvs_paged_attention(const void* q, int64_t q_tok_stride,
                        int64_t q_head_stride, const void* k_cache,
                        const void* v_cache, int cache_dtype,
                        const float* k_scale, const float* v_scale,
                        const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k,
                        const int32_t* block_tables, int64_t bt_stride,
                        int num_seqs, int64_t num_tokens, int max_seqlen_q,
                        int max_seqlen_k, int num_heads, int num_kv_heads,
                        int head_dim, int block_size, int64_t num_blocks,
                        float softmax_scale, void* out, int64_t out_tok_stride,
                        int64_t out_head_stride, void* workspace,
                        int64_t workspace_bytes, void* stream);

/*
 * The layer's forward in one call: the KV-cache write of the step's k / v
 * (as nvs_store_kvcache) and then the attention (as nvs_paged_attention).
 * Replaces PagedAttention.forward_unified's write_kv_cache(k, v,
 * slot_mapping) + prefill_flashattn(q, k, v, context) (reference
 * attention.py:500-546).  When every row is a decode row (max_seqlen_q ==
 * 1), the sources are BF16 and the rows 16-byte aligned, the decode kernel
 * writes each row's new token itself (BF16 values, or fp8 / int8 codes and
 * their scales); otherwise the store kernel runs first.  In the decode
 * kernel, the wave that reads a row's last tile writes the row's token just
 * before that read when slot_mapping[row] is the row's own last position
 * (block_tables[row][(k_len-1) / block_size] * block_size + (k_len-1) %
 * block_size, the slot the engine forms for a decode row); any other slot
 * >= 0 (a keyless row, a missing block, a position in another row's keys or
 * an earlier tile of its own) is detected on the device and written by every
 * wave of its kv head before that wave's first load.
 * Precondition: slot_mapping entries are distinct (a repeated slot leaves
 * the rows that share it unspecified), and no row reads another row's
 * own-last-position slot through a shared block (a sequence appends only
 * into its own last block, as the engine's block manager guarantees).
 * Under it, the cache contents and the output equal nvs_store_kvcache
 * followed by nvs_paged_attention, bit for bit.
 */
int nvs_paged_attention_store(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                              const void* k, const void* v, int src_dtype,
                              int64_t k_tok_stride, int64_t k_head_stride,
                              int64_t v_tok_stride, int64_t v_head_stride,
                              const int32_t* slot_mapping, void* k_cache, void* v_cache,
                              int cache_dtype, float* k_scale, float* v_scale,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              const int32_t* block_tables, int64_t bt_stride, int num_seqs,
                              int64_t num_tokens, int max_seqlen_q, int max_seqlen_k,
                              int num_heads, int num_kv_heads, int head_dim, int block_size,
                              int64_t num_blocks, float softmax_scale, void* out,
                              int64_t out_tok_stride, int64_t out_head_stride,
                              void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of nvs_paged_attention_store, with no counterpart
 * in the reference: for callers that cannot allocate device memory or pass a
 * workspace (code under HIP-graph capture, tight serving loops, hosts that
 * forbid hipMalloc).  Same arguments, semantics and kernels as
 * nvs_paged_attention_store without workspace / workspace_bytes: the
 * workspace is the library's static per-device scratch of
 * NVS_NOALLOC_SCRATCH_BYTES (32 MiB on every GPU the library is loaded on,
 * held until the process ends), looked up on the first call with the device
 * current; the stream must belong to the current device.  A batch whose
 * nvs_attention_workspace_bytes(...) exceeds the scratch is refused with
 * NVS_ERR_WORKSPACE before anything is launched.  The call allocates
 * nothing.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (different streams or threads) race; calls ordered on
 * one stream do not.
 */
#define NVS_NOALLOC_SCRATCH_BYTES (32ll << 20)
int nvs_paged_attention_store_noalloc(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                      const void* k, const void* v, int src_dtype,
                                      int64_t k_tok_stride, int64_t k_head_stride,
                                      int64_t v_tok_stride, int64_t v_head_stride,
                                      const int32_t* slot_mapping, void* k_cache, void* v_cache,
                                      int cache_dtype, float* k_scale, float* v_scale,
                                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                      const int32_t* block_tables, int64_t bt_stride, int num_seqs,
                                      int64_t num_tokens, int max_seqlen_q, int max_seqlen_k,
                                      int num_heads, int num_kv_heads, int head_dim, int block_size,
                                      int64_t num_blocks, float softmax_scale, void* out,
                                      int64_t out_tok_stride, int64_t out_head_stride, void* stream);

/*
 * Causal varlen attention over the step's own (not cached) K/V: the
 * block_tables-is-None call of prefill_flashattn (reference
 * attention.py:338-354, flash_attn_varlen_func without block_table) and the
 * no-prefix branch of prefill_torch (attention.py:400-439).
 *   q, out        [num_tokens, num_heads, head_dim] with strides.
 *   k, v          [num_kv_tokens, num_kv_heads, head_dim] BF16 with strides;
 *                 keys of sequence i are rows cu_seqlens_k[i] ..
 *                 cu_seqlens_k[i+1]-1 (as flash_attn_varlen_func, the key
 *                 rows need not match the query rows; reads are clamped to
 *                 [0, num_kv_tokens)).  Same mask, GQA map, output and
 *                 workspace rule as nvs_paged_attention; head_dim 128.
 */
int nvs_varlen_attention(const void* q, int64_t q_tok_stride,
                         int64_t q_head_stride, const void* k, const void* v,
                         int64_t k_tok_stride, int64_t k_head_stride,
                         int64_t v_tok_stride, int64_t v_head_stride,
                         const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_k, int num_seqs,
                         int64_t num_tokens, int64_t num_kv_tokens,
                         int max_seqlen_q, int max_seqlen_k, int num_heads,
                         int num_kv_heads, int head_dim, float softmax_scale,
                         void* out, int64_t out_tok_stride,
                         int64_t out_head_stride, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * nvs_varlen_attention with the element type of q, k, v and out given:
 * dtype BF16 or FP16 (fp16 compute, the reference's flash_attn_varlen_func
 * on fp16 tensors, attention.py:338-354 with attention_compute_dtype
 * float16).  nvs_varlen_attention is this call with dtype BF16.
 */
int nvs_varlen_attention_dtype(const void* q, int64_t q_tok_stride,
                               int64_t q_head_stride, const void* k, const void* v,
                               int64_t k_tok_stride, int64_t k_head_stride,
                               int64_t v_tok_stride, int64_t v_head_stride,
                               const int32_t* cu_seqlens_q,
                               const int32_t* cu_seqlens_k, int num_seqs,
                               int64_t num_tokens, int64_t num_kv_tokens,
                               int max_seqlen_q, int max_seqlen_k, int num_heads,
                               int num_kv_heads, int head_dim, float softmax_scale,
                               void* out, int64_t out_tok_stride,
                               int64_t out_head_stride, void* workspace,
                               int64_t workspace_bytes, void* stream, int dtype);

/*
 * Step metadata built on the device.  Replaces the per-token loops of
 * ModelRunner.prepare_model_input (reference model_runner.py:461-532) that
 * form cu_seqlens_q/k, context_lens, positions and slot_mapping, and the
 * padding of prepare_block_tables (model_runner.py:334-344).
 *   num_cached_tokens, num_new_tokens  [num_seqs] int32: the Sequence fields
 *                 the runner reads; num_seqs <= 4096.
 *   block_ids     the sequences' block lists concatenated, int32
 *                 [num_block_ids]; sequence b's list is block_ids[
 *                 block_offsets[b] .. block_offsets[b+1]-1] (block_offsets
 *                 int32 [num_seqs + 1]; offsets outside [0, num_block_ids]
 *                 count as 0, a decreasing pair as an empty list).
 *   num_tokens    the sum of num_new_tokens (the host knows it; it sizes
 *                 slot_mapping and positions).
 * Writes cu_seqlens_q / cu_seqlens_k [num_seqs + 1] (running sums of
 * num_new and of num_cached + num_new), context_lens [num_seqs]
 * (num_cached + num_new), and for query token t of sequence b at position
 * p = num_cached[b] + (t - cu_seqlens_q[b]): positions[t] = p (int64; may
 * be NULL) and slot_mapping[t] = list_b[p / block_size] * block_size +
 * p % block_size.  A position past the end of its list or on a -1 entry gets
 * slot -1 (the store skips it), as do tokens past the sum of num_new_tokens.
 * block_tables (may be NULL) [num_seqs, block_table_width] receives each
 * list padded (or cut) to the width with -1.  Slots and running sums are
 * int32, as in the reference.
 */
int nvs_build_context(const int32_t* num_cached_tokens, const int32_t* num_new_tokens,
                      int num_seqs, const int32_t* block_offsets,
                      const int32_t* block_ids, int64_t num_block_ids,
                      int block_size, int64_t num_tokens,
                      int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                      int32_t* context_lens, int32_t* slot_mapping,
                      int64_t* positions, int32_t* block_tables,
                      int block_table_width, void* stream);

/*
 * Whole-block copies between a paged cache and a packed block snapshot, one
 * launch per tensor.  Replaces the KV handoff copies of the reference's PD
 * connector: the export kv_cache[:, :, src_block_ids].contiguous() (and the
 * same of kv_scale_cache) in _export_kv_snapshot
 * (pd_self/kv_connector.py:94-110), and the per-block loop
 * kv_cache[:, :, block_id].copy_(blocks[:, :, i]) of load_kv_item
 * (kv_connector.py:282-311).
 *   src, dst      [num_planes, src/dst_num_blocks, block_bytes] byte arrays
 *                 (num_planes = 2 x layers; block_bytes = block_size x
 *                 kv_heads x head_dim x element size for the codes,
 *                 block_size x kv_heads x 4 for the fp32 scales), 16-byte
 *                 aligned, block_bytes a multiple of 16.
 *   copy i moves block src_block_ids[i] (i when NULL) of every plane to block
 *   dst_block_ids[i] (i when NULL) of the same plane.  Ids outside
 *   [0, num_blocks) skip the copy.  Destinations must be distinct and the
 *   source and destination regions disjoint (copies run in no fixed order).
 */
int nvs_copy_blocks(const void* src, int64_t src_num_blocks, const int32_t* src_block_ids,
                    void* dst, int64_t dst_num_blocks, const int32_t* dst_block_ids,
                    int64_t num_planes, int64_t block_bytes, int64_t num_copies,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVS_ATTENTION_H */
