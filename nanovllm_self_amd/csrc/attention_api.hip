// C ABI of the attention kernels: argument validation and dispatch of decode
// rows (q_len == 1, split-K decode) and prefill rows (MFMA flash prefill).
#include <algorithm>
#include <cstdlib>
#include <string>

#include "nvs_common.h"
#include "attention_common.h"
#include "decode_merge.h"

using namespace nvs;

static int validate_common(const AttnParams& P, const char* who) {
  NVS_REQUIRE(P.B >= 0 && P.T >= 0, NVS_ERR_INVALID, "%s: negative batch size", who);
  NVS_REQUIRE(P.B < 65536, NVS_ERR_UNSUPPORTED, "%s: at most 65535 sequences per call", who);
  NVS_REQUIRE(P.q && P.out && P.cu_q && P.cu_k, NVS_ERR_INVALID, "%s: null tensor pointer", who);
  NVS_REQUIRE(P.Hq > 0 && P.Hkv > 0 && P.Hq % P.Hkv == 0, NVS_ERR_INVALID,
              "%s: num_heads (%d) must be a positive multiple of num_kv_heads (%d)", who, P.Hq,
              P.Hkv);
  NVS_REQUIRE(P.Hkv <= 256, NVS_ERR_UNSUPPORTED, "%s: at most 256 kv heads, got %d", who, P.Hkv);
  NVS_REQUIRE(P.Hq / P.Hkv <= 16, NVS_ERR_UNSUPPORTED,
              "%s: at most 16 query heads per kv head, got %d", who, P.Hq / P.Hkv);
  NVS_REQUIRE(P.max_seqlen_q >= 0 && P.max_seqlen_k >= 0, NVS_ERR_INVALID,
              "%s: negative max_seqlen", who);
  // The kernels take the row max of the unscaled scores, which needs a
  // positive scale (the layer passes head_dim^-0.5).
  NVS_REQUIRE(P.softmax_scale > 0.0f && P.softmax_scale < INFINITY, NVS_ERR_INVALID,
              "%s: softmax_scale must be positive and finite, got %g", who, (double)P.softmax_scale);
  NVS_REQUIRE(P.q_ts % 8 == 0 && P.q_hs % 8 == 0 && ((uintptr_t)P.q % 16) == 0, NVS_ERR_INVALID,
              "%s: q rows must be 16-byte aligned", who);
  NVS_REQUIRE(P.out_ts % 8 == 0 && P.out_hs % 8 == 0 && ((uintptr_t)P.out % 16) == 0,
              NVS_ERR_INVALID, "%s: out rows must be 16-byte aligned", who);
  // The decode kernel addresses a group's heads with 32-bit lane offsets.
  NVS_REQUIRE(P.q_hs >= 0 && P.q_hs < (1ll << 26) && P.out_hs >= 0 && P.out_hs < (1ll << 26),
              NVS_ERR_UNSUPPORTED, "%s: head strides must lie in [0, 2^26) elements", who);
  return NVS_OK;
}

namespace nvs {
// Query positions per prefill tile for num_heads / num_kv_heads (the
// smallest tile when the group size is unknown).
static int prefill_pbm(int num_heads, int num_kv_heads) {
  const int g = (num_kv_heads > 0 && num_heads % num_kv_heads == 0) ? num_heads / num_kv_heads : 0;
  return prefill_positions(g);
}

static int prefill_tiles(int max_seqlen_q, int pbm) {
  const int t = (max_seqlen_q + pbm - 1) / pbm;
  return t < 1 ? 1 : t;
}

// Workspace: the prefill plan, then the decode partials (256-byte aligned).
// With an unknown kv-head count (num_kv_heads <= 0, or not dividing
// num_heads) both parts are sized for their worst case: the smallest prefill
// tile, and one kv head whose group is every query head (waves x group is
// largest there).
int64_t attention_workspace_bytes(int num_seqs, int max_seqlen_q, int max_seqlen_k, int num_heads,
                                  int num_kv_heads) {
  if (num_seqs <= 0 || num_heads <= 0) return 0;
  const bool known = num_kv_heads > 0 && num_heads % num_kv_heads == 0;
  const int hk = known ? num_kv_heads : 1;
  const int group = known ? num_heads / num_kv_heads : num_heads;
  const int waves = decode_wave_cap(num_seqs, max_seqlen_k, hk);
  const int ntq = prefill_tiles(max_seqlen_q, prefill_pbm(num_heads, num_kv_heads));
  return align256(plan_bytes(num_seqs, ntq)) + decode_workspace_bytes(waves, group);
}

// The plan's tile of query positions is the kernel's work-item height; the
// classic kernel's tile is never larger than the MFMA tile-loop kernel's,
// so the workspace sized for it holds either plan.
static Plan make_plan(void* ws, const AttnParams& P) {
  const int pbm = prefill_mx_serves(P) ? prefill_mx_positions(P.Hq / P.Hkv) : prefill_pbm(P.Hq, P.Hkv);
  return plan_at(ws, P.B, prefill_tiles(P.max_seqlen_q, pbm), pbm);
}

// fp16 elements run only on the tile-loop kernel (the classic kernel is
// bf16 and code caches); a call with prefill work it does not serve is
// refused before any launch.  Paged calls have prefill work when
// max_seqlen_q > 1 (q_len == 1 rows go to the decode kernel), local calls
// always.
static int check_f16_served(const AttnParams& P, const char* who) {
  const bool prefill = P.bt ? P.max_seqlen_q > 1 : P.max_seqlen_q > 0;
  NVS_REQUIRE(P.cache_dtype != NVS_DTYPE_FP16 || !prefill || prefill_mx_serves(P),
              NVS_ERR_UNSUPPORTED,
              "%s: fp16 prefill runs on the tile-loop kernel only, which does not serve this call "
              "(NVS_PREFILL_KERNEL=classic, or strides past its 32-bit lane offsets)", who);
  return NVS_OK;
}

static int launch_prefill_any(const AttnParams& P, const Plan& plan, hipStream_t s) {
  return prefill_mx_serves(P) ? launch_prefill_mx(P, plan, s) : launch_prefill(P, plan, s);
}

// Whether a paged call over a code cache can serve its prefill rows from a
// bf16 copy through the tile-loop kernel: the workspace holds the copy after
// the plan and the decode partials, and both prefill kernels tile the query
// positions alike (the plan is shared; which one runs is decided on the
// device).  NVS_PREFILL_KERNEL=classic keeps every call on the classic
// kernel.
static bool shadow_serves(const AttnParams& P) {
  if (!is_quant(P.cache_dtype) || P.max_seqlen_q <= 1 || P.bt == nullptr) return false;
  const int g = P.Hq / P.Hkv;
  if (prefill_mx_positions(g) != prefill_positions(g)) return false;
  const int64_t base = align256(attention_workspace_bytes(P.B, P.max_seqlen_q, P.max_seqlen_k, P.Hq, P.Hkv));
  if (shadow_cap(P.B, P.max_seqlen_k, P.Hkv) <= 0) return false;
  if (P.ws_bytes < base + shadow_bytes(P.B, P.max_seqlen_k, P.Hkv)) return false;
  // The copy is read as a bf16 cache of block size 64.
  AttnParams C = P;
  C.cache_dtype = NVS_DTYPE_BF16;
  C.bs = kShadowTile;
  C.NB = shadow_cap(P.B, P.max_seqlen_k, P.Hkv);
  return prefill_mx_serves(C);
}

// Work-groups of a prefill launch that also streams the call's decode rows
// (0: the decode keeps a launch of its own): every work-group slot of the
// device, when the tile-loop kernel serves the prefill rows (from the cache,
// or from a code cache's bf16 copy), the step's new tokens are already
// stored, and the device holds two decode waves per kv head on each XCD.
// NVS_CODECODE=0 turns it off.
static int co_decode_wgs(const AttnParams& P) {
  static const bool off = [] {
    const char* e = std::getenv("NVS_CODECODE");
    return e && std::string(e) == "0";
  }();
  if (off || P.kn || P.max_seqlen_q <= 1) return 0;
  const int wgs = device_slots(1) & ~7;
  return wgs >= std::max(8, (2 * P.Hkv + 7) & ~7) ? wgs : 0;
}

static float env_rate(const char* name, float dflt) {
  const char* e = std::getenv(name);
  return e ? std::strtof(e, nullptr) : dflt;
}

// Decode beside the prefill: a work-group of four decode waves (one per
// SIMD) streams about 44 GB/s of a bf16 cache's decode rows while the other
// CUs run prefill tiles (mixed_32b's 3.56 GB on 32 CUs in 2.5 ms) and about
// 28 GB/s of an fp8 one's (1.84 GB on 32 CUs in 2.3 ms: a code tile carries
// half the bytes for the same VALU work), the chip about 6 TB/s; a CU runs
// about 5 TFLOP/s of prefill (1.89 TFLOP in 1.47 ms on 256 CUs).
// NVS_CODECODE_{CU_BPS,HBM_BPS,CU_FLOPS,FINISH} override them.
CoDecodeRates co_decode_rates(int cache_dtype) {
  const bool half = cache_dtype == NVS_DTYPE_BF16 || cache_dtype == NVS_DTYPE_FP16;
  static const float cu16 = env_rate("NVS_CODECODE_CU_BPS", 44e9f), cu8 = env_rate("NVS_CODECODE_CU_BPS", 28e9f);
  static const CoDecodeRates r = {0.0f, env_rate("NVS_CODECODE_HBM_BPS", 6.0e12f),
                                  env_rate("NVS_CODECODE_CU_FLOPS", 5.0e12f), env_rate("NVS_CODECODE_FINISH", 0.85f)};
  CoDecodeRates x = r;
  x.cu_bps = half ? cu16 : cu8;
  return x;
}

int decode_launch_waves(int max_waves, int Hkv) {
  const int w = std::min(max_waves, device_slots(4 * kDecodeWavesPerEU));
  return std::max(Hkv, w / Hkv * Hkv);
}
}  // namespace nvs

extern "C" int64_t nvs_attention_workspace_bytes(int num_seqs, int max_seqlen_q, int max_seqlen_k,
                                                 int num_heads, int num_kv_heads, int head_dim,
                                                 int block_size) {
  (void)head_dim;
  (void)block_size;
  return attention_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads);
}

extern "C" int64_t nvs_attention_workspace_bytes_cache(int num_seqs, int max_seqlen_q, int max_seqlen_k,
                                                       int num_heads, int num_kv_heads, int head_dim,
                                                       int block_size, int cache_dtype) {
  (void)head_dim;
  (void)block_size;
  const int64_t base = attention_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads);
  if (base <= 0 || !is_quant(cache_dtype) || max_seqlen_q <= 1 || num_kv_heads <= 0 ||
      num_heads % num_kv_heads != 0)
    return base;
  return align256(base) + shadow_bytes(num_seqs, max_seqlen_k, num_kv_heads);
}

static int check_workspace(const AttnParams& P, const char* who) {
  const int64_t need = attention_workspace_bytes(P.B, P.max_seqlen_q, P.max_seqlen_k, P.Hq, P.Hkv);
  NVS_REQUIRE(P.ws && P.ws_bytes >= need && ((uintptr_t)P.ws % 256) == 0, NVS_ERR_WORKSPACE,
              "%s: workspace of %lld bytes (256-byte aligned) needed, %lld given", who,
              (long long)need, (long long)P.ws_bytes);
  return NVS_OK;
}

// nvs_paged_attention's body; P.kn != null asks the decode kernel to store
// the step's new tokens itself (decode rows only).
static int paged_attention_impl(AttnParams& P, const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                const void* k_cache, const void* v_cache, int cache_dtype,
                                const float* k_scale, const float* v_scale,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                const int32_t* block_tables, int64_t bt_stride, int num_seqs,
                                int64_t num_tokens, int max_seqlen_q, int max_seqlen_k,
                                int num_heads, int num_kv_heads, int head_dim, int block_size,
                                int64_t num_blocks, float softmax_scale, void* out,
                                int64_t out_tok_stride, int64_t out_head_stride,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  P.q = q; P.q_ts = q_tok_stride; P.q_hs = q_head_stride;
  P.kc = k_cache; P.vc = v_cache; P.cache_dtype = cache_dtype; P.ks = k_scale; P.vs = v_scale;
  P.bt = block_tables; P.bt_stride = bt_stride; P.bs = block_size; P.NB = num_blocks;
  P.cu_q = cu_seqlens_q; P.cu_k = cu_seqlens_k;
  P.B = num_seqs; P.T = num_tokens; P.max_seqlen_q = max_seqlen_q; P.max_seqlen_k = max_seqlen_k;
  P.Hq = num_heads; P.Hkv = num_kv_heads; P.softmax_scale = softmax_scale;
  P.out = out; P.out_ts = out_tok_stride; P.out_hs = out_head_stride;
  P.ws = workspace; P.ws_bytes = workspace_bytes;
  if (num_seqs == 0 || num_tokens == 0) return NVS_OK;
  int rc = validate_common(P, "paged_attention");
  if (rc != NVS_OK) return rc;
  NVS_REQUIRE(head_dim == kHeadDim, NVS_ERR_UNSUPPORTED,
              "paged_attention: head_dim must be %d, got %d", kHeadDim, head_dim);
  NVS_REQUIRE(k_cache && v_cache && block_tables, NVS_ERR_INVALID,
              "paged_attention: null cache / block_tables pointer");
  NVS_REQUIRE(cache_dtype == NVS_DTYPE_BF16 || cache_dtype == NVS_DTYPE_FP16 || cache_dtype == NVS_DTYPE_INT8 ||
                  cache_dtype == NVS_DTYPE_FP8_E4M3,
              NVS_ERR_UNSUPPORTED, "paged_attention: cache dtype %d not served (bf16/fp16/int8/fp8)",
              cache_dtype);
  NVS_REQUIRE(!is_quant(cache_dtype) || (k_scale && v_scale), NVS_ERR_INVALID,
              "paged_attention: quantised cache needs k_scale and v_scale");
  NVS_REQUIRE(block_size > 0 && block_size % 64 == 0, NVS_ERR_UNSUPPORTED,
              "paged_attention: block_size must be a multiple of 64, got %d", block_size);
  NVS_REQUIRE(num_blocks > 0, NVS_ERR_INVALID, "paged_attention: empty cache");
  NVS_REQUIRE(num_blocks < (1ll << 31) && bt_stride < (1ll << 31) &&
                  (int64_t)num_seqs * bt_stride < (1ll << 31),
              NVS_ERR_UNSUPPORTED, "paged_attention: block pool / block_tables too large");
  NVS_REQUIRE(bt_stride > 0 && ((int64_t)max_seqlen_k + block_size - 1) / block_size <= bt_stride,
              NVS_ERR_INVALID,
              "paged_attention: block_tables rows (%lld) too short for max_seqlen_k %d",
              (long long)bt_stride, max_seqlen_k);
  NVS_REQUIRE((int64_t)num_seqs * (((int64_t)max_seqlen_k + kDecodeTile - 1) / kDecodeTile) < (1ll << 31),
              NVS_ERR_UNSUPPORTED, "paged_attention: batch too large for one call (decode tiles exceed 2^31)");
  if (max_seqlen_q <= 0) return NVS_OK;
  rc = check_workspace(P, "paged_attention");
  if (rc != NVS_OK) return rc;
  rc = check_f16_served(P, "paged_attention");
  if (rc != NVS_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const bool shadow = shadow_serves(P);
  const Plan plan = shadow ? plan_at(workspace, P.B, prefill_tiles(P.max_seqlen_q, prefill_mx_positions(P.Hq / P.Hkv)),
                                     prefill_mx_positions(P.Hq / P.Hkv))
                           : make_plan(workspace, P);
  char* partials = (char*)workspace + align256(plan_bytes(num_seqs, plan.ntq));
  const int max_waves = decode_wave_cap(num_seqs, max_seqlen_k, num_kv_heads);
  // The tile-loop kernel serving the prefill rows streams the decode rows
  // too (its first work-groups, before they join the prefill); the merge of
  // split rows follows it.
  const int co_wgs = (shadow || prefill_mx_serves(P)) ? co_decode_wgs(P) : 0;
  if (co_wgs > 0) {
    CoDecode co;
    co.a = decode_args(P, max_waves, partials);
    co.bt = P.bt;
    co.kv = P.cache_dtype;
    co.groups = std::min(8 * ((co_wgs / 2) / P.Hkv), max_waves / P.Hkv);
    co.wgs = co_wgs;
    if (!shadow) {
      rc = launch_plan(P, plan, /*paged=*/true, s, nullptr, nullptr, &co);
      if (rc != NVS_OK) return rc;
      rc = launch_prefill_mx(P, plan, s, &co);
      if (rc != NVS_OK) return rc;
      return launch_decode_merge(co.a, co.groups, s);
    }
    // Code cache: the prefill reads the bf16 copy, the decode waves the
    // codes; they run whichever prefill kernel the plan lets serve.
    const ShadowLayout sh = shadow_at((char*)workspace + align256(attention_workspace_bytes(
                                          P.B, P.max_seqlen_q, P.max_seqlen_k, P.Hq, P.Hkv)),
                                      P.B, P.max_seqlen_k, P.Hkv);
    rc = launch_plan(P, plan, /*paged=*/true, s, &sh, nullptr, &co);
    if (rc != NVS_OK) return rc;
    rc = launch_shadow_fill(P, plan, sh, s);
    if (rc != NVS_OK) return rc;
    AttnParams C = P;
    C.kc = sh.k; C.vc = sh.v; C.cache_dtype = NVS_DTYPE_BF16; C.ks = nullptr; C.vs = nullptr;
    C.bt = sh.table; C.bt_stride = sh.ST; C.bs = kShadowTile; C.NB = sh.cap;
    C.gate = &plan.hdr->shadow_on; C.gate_run = 1;
    rc = launch_prefill_mx(C, plan, s, &co);
    if (rc != NVS_OK) return rc;
    if ((int64_t)sh.cap < (int64_t)P.B * sh.ST) {
      AttnParams F = P;
      F.gate = &plan.hdr->shadow_on; F.gate_run = 0;
      rc = launch_prefill(F, plan, s);
      if (rc != NVS_OK) return rc;
    }
    return launch_decode_merge(co.a, co.groups, s);
  }
  // With prefill rows the plan launch also merges the split decode rows.
  MergeJob merge;
  rc = launch_decode(P, max_waves, decode_launch_waves(max_waves, num_kv_heads), partials, s,
                     max_seqlen_q > 1 ? &merge : nullptr);
  if (rc != NVS_OK || max_seqlen_q == 1) return rc;  // no prefill rows: no plan
  if (!shadow) {
    rc = launch_plan(P, plan, /*paged=*/true, s, nullptr, &merge);
    if (rc != NVS_OK) return rc;
    return launch_prefill_any(P, plan, s);
  }
  // Code cache: the prefill rows' keys and values dequantised into the bf16
  // copy, read by the tile-loop kernel; the classic kernel serves the call
  // instead where the plan finds that the copy would not fit.
  const ShadowLayout sh = shadow_at((char*)workspace + align256(attention_workspace_bytes(
                                        P.B, P.max_seqlen_q, P.max_seqlen_k, P.Hq, P.Hkv)),
                                    P.B, P.max_seqlen_k, P.Hkv);
  rc = launch_plan(P, plan, /*paged=*/true, s, &sh, &merge);
  if (rc != NVS_OK) return rc;
  rc = launch_shadow_fill(P, plan, sh, s);
  if (rc != NVS_OK) return rc;
  AttnParams C = P;
  C.kc = sh.k; C.vc = sh.v; C.cache_dtype = NVS_DTYPE_BF16; C.ks = nullptr; C.vs = nullptr;
  C.bt = sh.table; C.bt_stride = sh.ST; C.bs = kShadowTile; C.NB = sh.cap;
  C.gate = &plan.hdr->shadow_on; C.gate_run = 1;
  rc = launch_prefill_mx(C, plan, s);
  if (rc != NVS_OK) return rc;
  // When every row's tiles fit the copy whatever the lengths, the plan
  // cannot turn the copy off and the classic kernel would only exit.
  if ((int64_t)sh.cap >= (int64_t)P.B * sh.ST) return NVS_OK;
  AttnParams F = P;
  F.gate = &plan.hdr->shadow_on; F.gate_run = 0;
  return launch_prefill(F, plan, s);
}

extern "C" int nvs_paged_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                   const void* k_cache, const void* v_cache, int cache_dtype,
                                   const float* k_scale, const float* v_scale,
                                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   const int32_t* block_tables, int64_t bt_stride, int num_seqs,
                                   int64_t num_tokens, int max_seqlen_q, int max_seqlen_k,
                                   int num_heads, int num_kv_heads, int head_dim, int block_size,
                                   int64_t num_blocks, float softmax_scale, void* out,
                                   int64_t out_tok_stride, int64_t out_head_stride,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  AttnParams P = {};
  return paged_attention_impl(P, q, q_tok_stride, q_head_stride, k_cache, v_cache, cache_dtype, k_scale, v_scale,
                              cu_seqlens_q, cu_seqlens_k, block_tables, bt_stride, num_seqs, num_tokens,
                              max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, block_size,
                              num_blocks, softmax_scale, out, out_tok_stride, out_head_stride, workspace,
                              workspace_bytes, stream);
}

extern "C" int nvs_paged_attention_store(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                         const void* k, const void* v, int src_dtype, int64_t k_tok_stride,
                                         int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                                         const int32_t* slot_mapping, void* k_cache, void* v_cache,
                                         int cache_dtype, float* k_scale, float* v_scale,
                                         const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                         const int32_t* block_tables, int64_t bt_stride, int num_seqs,
                                         int64_t num_tokens, int max_seqlen_q, int max_seqlen_k,
                                         int num_heads, int num_kv_heads, int head_dim, int block_size,
                                         int64_t num_blocks, float softmax_scale, void* out,
                                         int64_t out_tok_stride, int64_t out_head_stride,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  AttnParams P = {};
  // A batch of decode rows with bf16 sources: the decode kernel stores the
  // new tokens itself (one launch less), values into a bf16 cache, codes and
  // scales into an fp8 / int8 one.  Otherwise the store kernel first.
  const bool cache_ok = cache_dtype == NVS_DTYPE_BF16 ||
                        ((cache_dtype == NVS_DTYPE_FP8_E4M3 || cache_dtype == NVS_DTYPE_INT8) && k_scale && v_scale);
  const bool fused = num_tokens > 0 && max_seqlen_q == 1 && cache_ok &&
                     src_dtype == NVS_DTYPE_BF16 && k && v && slot_mapping && head_dim == kHeadDim &&
                     k_tok_stride % 8 == 0 && k_head_stride % 8 == 0 && v_tok_stride % 8 == 0 &&
                     v_head_stride % 8 == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                     k_tok_stride >= 0 && k_head_stride >= 0 && v_tok_stride >= 0 && v_head_stride >= 0;
  if (fused) {
    P.kn = k; P.vn = v; P.slots = slot_mapping;
    P.kn_ts = k_tok_stride; P.kn_hs = k_head_stride; P.vn_ts = v_tok_stride; P.vn_hs = v_head_stride;
  } else {
    const int rc = nvs_store_kvcache(k, v, src_dtype, k_tok_stride, k_head_stride, v_tok_stride, v_head_stride,
                                     slot_mapping, num_tokens, k_cache, v_cache, cache_dtype, k_scale, v_scale,
                                     num_blocks, block_size, num_kv_heads, head_dim, stream);
    if (rc != NVS_OK) return rc;
  }
  return paged_attention_impl(P, q, q_tok_stride, q_head_stride, k_cache, v_cache, cache_dtype, k_scale, v_scale,
                              cu_seqlens_q, cu_seqlens_k, block_tables, bt_stride, num_seqs, num_tokens,
                              max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, block_size,
                              num_blocks, softmax_scale, out, out_tok_stride, out_head_stride, workspace,
                              workspace_bytes, stream);
}

static int varlen_attention_impl(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                 const void* k, const void* v, int64_t k_tok_stride,
                                 int64_t k_head_stride, int64_t v_tok_stride,
                                 int64_t v_head_stride, const int32_t* cu_seqlens_q,
                                 const int32_t* cu_seqlens_k, int num_seqs, int64_t num_tokens,
                                 int64_t num_kv_tokens, int max_seqlen_q, int max_seqlen_k, int num_heads,
                                 int num_kv_heads, int head_dim, float softmax_scale, void* out,
                                 int64_t out_tok_stride, int64_t out_head_stride,
                                 void* workspace, int64_t workspace_bytes, void* stream, int dtype) {
  AttnParams P = {};
  P.cache_dtype = dtype;  // the element type of q, k, v and out
  P.ws = workspace; P.ws_bytes = workspace_bytes;
  P.q = q; P.q_ts = q_tok_stride; P.q_hs = q_head_stride;
  P.k = k; P.v = v; P.k_ts = k_tok_stride; P.k_hs = k_head_stride;
  P.v_ts = v_tok_stride; P.v_hs = v_head_stride;
  P.bt = nullptr;
  P.cu_q = cu_seqlens_q; P.cu_k = cu_seqlens_k;
  P.B = num_seqs; P.T = num_tokens; P.Tk = num_kv_tokens;
  P.max_seqlen_q = max_seqlen_q; P.max_seqlen_k = max_seqlen_k;
  P.Hq = num_heads; P.Hkv = num_kv_heads; P.softmax_scale = softmax_scale;
  P.out = out; P.out_ts = out_tok_stride; P.out_hs = out_head_stride;
  if (num_seqs == 0 || num_tokens == 0) return NVS_OK;
  NVS_REQUIRE(num_kv_tokens >= 1, NVS_ERR_INVALID, "varlen_attention: num_kv_tokens must be >= 1");
  int rc = validate_common(P, "varlen_attention");
  if (rc != NVS_OK) return rc;
  NVS_REQUIRE(head_dim == kHeadDim, NVS_ERR_UNSUPPORTED,
              "varlen_attention: head_dim must be %d, got %d", kHeadDim, head_dim);
  NVS_REQUIRE(dtype == NVS_DTYPE_BF16 || dtype == NVS_DTYPE_FP16, NVS_ERR_UNSUPPORTED,
              "varlen_attention: dtype %d not served (bf16 / fp16)", dtype);
  NVS_REQUIRE(k && v, NVS_ERR_INVALID, "varlen_attention: null k/v pointer");
  NVS_REQUIRE(k_tok_stride % 8 == 0 && k_head_stride % 8 == 0 && v_tok_stride % 8 == 0 &&
                  v_head_stride % 8 == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0,
              NVS_ERR_INVALID, "varlen_attention: k/v rows must be 16-byte aligned");
  if (max_seqlen_q <= 0) return NVS_OK;
  rc = check_workspace(P, "varlen_attention");
  if (rc != NVS_OK) return rc;
  rc = check_f16_served(P, "varlen_attention");
  if (rc != NVS_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const Plan plan = make_plan(workspace, P);
  rc = launch_plan(P, plan, /*paged=*/false, s);
  if (rc != NVS_OK) return rc;
  return launch_prefill_any(P, plan, s);
}

extern "C" int nvs_varlen_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                    const void* k, const void* v, int64_t k_tok_stride,
                                    int64_t k_head_stride, int64_t v_tok_stride,
                                    int64_t v_head_stride, const int32_t* cu_seqlens_q,
                                    const int32_t* cu_seqlens_k, int num_seqs, int64_t num_tokens,
                                    int64_t num_kv_tokens, int max_seqlen_q, int max_seqlen_k, int num_heads,
                                    int num_kv_heads, int head_dim, float softmax_scale, void* out,
                                    int64_t out_tok_stride, int64_t out_head_stride,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  return varlen_attention_impl(q, q_tok_stride, q_head_stride, k, v, k_tok_stride, k_head_stride, v_tok_stride,
                               v_head_stride, cu_seqlens_q, cu_seqlens_k, num_seqs, num_tokens, num_kv_tokens,
                               max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, out,
                               out_tok_stride, out_head_stride, workspace, workspace_bytes, stream,
                               NVS_DTYPE_BF16);
}

extern "C" int nvs_varlen_attention_dtype(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                          const void* k, const void* v, int64_t k_tok_stride,
                                          int64_t k_head_stride, int64_t v_tok_stride,
                                          int64_t v_head_stride, const int32_t* cu_seqlens_q,
                                          const int32_t* cu_seqlens_k, int num_seqs, int64_t num_tokens,
                                          int64_t num_kv_tokens, int max_seqlen_q, int max_seqlen_k,
                                          int num_heads, int num_kv_heads, int head_dim, float softmax_scale,
                                          void* out, int64_t out_tok_stride, int64_t out_head_stride,
                                          void* workspace, int64_t workspace_bytes, void* stream, int dtype) {
  clear_error();
  return varlen_attention_impl(q, q_tok_stride, q_head_stride, k, v, k_tok_stride, k_head_stride, v_tok_stride,
                               v_head_stride, cu_seqlens_q, cu_seqlens_k, num_seqs, num_tokens, num_kv_tokens,
                               max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, out,
                               out_tok_stride, out_head_stride, workspace, workspace_bytes, stream, dtype);
}
