// KV-cache write (with fused per-token quantisation), standalone
// quantise / dequantise, and the eager path's paged gather.
//
// Reference semantics: nanovllm/layers/attention.py
//   quantize_int8_per_token   :63-98
//   dequantize_int8_per_token :100-117
//   store_kv_cache_torch      :139-189
//   get_kv_cache              :201-285
#include <stdarg.h>
#include <stdio.h>

#include "nvs_common.h"
#include "store_common.h"

namespace nvs {

// ---------------------------------------------------------------------------
// Error plumbing
// ---------------------------------------------------------------------------
static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return NVS_ERR_LAUNCH;
  }
  return NVS_OK;
}

// ---------------------------------------------------------------------------
// KV-cache write.  One thread owns 8 consecutive head_dim elements of one
// (token, kv_head) row of both K and V; lpr = head_dim / 8 lanes form a row.
// With IDENT the destination row is the token index itself (used by
// nvs_quantize_per_token), otherwise slot_mapping[token].
// ---------------------------------------------------------------------------
struct StoreArgs {
  const void* k;
  const void* v;
  int64_t k_ts, k_hs, v_ts, v_hs;
  const int32_t* slots;
  int64_t rows;         // num_tokens * H
  int64_t total_slots;  // num_blocks * block_size
  void* kc;
  void* vc;
  float* ks;
  float* vs;
  int H, D, lpr_log2;
};

template <int SRC, int DST, bool IDENT, bool HAS_V>
__global__ __launch_bounds__(256) void store_kv_kernel(StoreArgs a) {
  const int lpr = 1 << a.lpr_log2;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid >> a.lpr_log2;
  const int c = (int)(gid & (lpr - 1));
  const bool active = row < a.rows;
  const int64_t t = active ? row / a.H : 0;
  const int h = active ? (int)(row - t * a.H) : 0;
  int64_t slot = -1;
  if (active) slot = IDENT ? t : (int64_t)a.slots[t];
  const bool valid = active && slot >= 0 && slot < a.total_slots;

  constexpr int SRC_BYTES = (SRC == NVS_DTYPE_FP32) ? 4 : 2;
  float xk[8], xv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xk[i] = xv[i] = 0.0f;
  if (valid) {
    load8<SRC>((const char*)a.k + (t * a.k_ts + h * a.k_hs + c * 8) * SRC_BYTES, xk);
    if constexpr (HAS_V)
      load8<SRC>((const char*)a.v + (t * a.v_ts + h * a.v_hs + c * 8) * SRC_BYTES, xv);
  }
  const int64_t dst_row = slot * a.H + h;  // (block*bs + off) * H + h
  const int64_t dst_elem = dst_row * a.D + c * 8;

  if constexpr (DST == NVS_DTYPE_INT8 || DST == NVS_DTYPE_FP8_E4M3) {
    // All lanes of a row take part in the reduction, valid or not.
    constexpr float qmax = (DST == NVS_DTYPE_INT8) ? QuantInt8::kQmax : QuantFp8::kQmax;
    const float sk = quant_scale(row_absmax(xk, lpr), qmax);
    float sv = 0.0f;
    if constexpr (HAS_V) sv = quant_scale(row_absmax(xv, lpr), qmax);
    if (valid) {
      *reinterpret_cast<u32x2*>((uint8_t*)a.kc + dst_elem) = quant8<DST, SRC != NVS_DTYPE_FP32>(xk, sk);
      if (c == 0) a.ks[dst_row] = sk;
      if constexpr (HAS_V) {
        *reinterpret_cast<u32x2*>((uint8_t*)a.vc + dst_elem) = quant8<DST, SRC != NVS_DTYPE_FP32>(xv, sv);
        if (c == 0) a.vs[dst_row] = sv;
      }
    }
  } else {
    constexpr int DST_BYTES = (DST == NVS_DTYPE_FP32) ? 4 : 2;
    if (valid) {
      store8_float<DST>((char*)a.kc + dst_elem * DST_BYTES, xk);
      if constexpr (HAS_V) store8_float<DST>((char*)a.vc + dst_elem * DST_BYTES, xv);
    }
  }
}

static int lpr_log2_for(int D) {
  if (D <= 0 || D % 8 != 0) return -1;
  int lpr = D / 8, l2 = 0;
  while ((1 << l2) < lpr) ++l2;
  if ((1 << l2) != lpr || lpr > 64) return -1;
  return l2;
}

template <bool IDENT, bool HAS_V>
static int launch_store(const StoreArgs& a, int src, int dst, hipStream_t s) {
  const int64_t threads = a.rows << a.lpr_log2;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks == 0) return NVS_OK;
  NVS_REQUIRE(blocks < (1ll << 31), NVS_ERR_INVALID, "too many rows (%lld)", (long long)a.rows);
  dim3 grid((unsigned)blocks), block(256);
#define NVS_STORE_CASE(S, D)                                                   \
  if (src == S && dst == D) {                                                  \
    hipLaunchKernelGGL((store_kv_kernel<S, D, IDENT, HAS_V>), grid, block, 0, s, a); \
    return check_launch("store_kvcache");                                      \
  }
#define NVS_STORE_SRC(S)                  \
  NVS_STORE_CASE(S, NVS_DTYPE_BF16)       \
  NVS_STORE_CASE(S, NVS_DTYPE_FP16)       \
  NVS_STORE_CASE(S, NVS_DTYPE_FP32)       \
  NVS_STORE_CASE(S, NVS_DTYPE_INT8)       \
  NVS_STORE_CASE(S, NVS_DTYPE_FP8_E4M3)
  NVS_STORE_SRC(NVS_DTYPE_BF16)
  NVS_STORE_SRC(NVS_DTYPE_FP16)
  NVS_STORE_SRC(NVS_DTYPE_FP32)
#undef NVS_STORE_SRC
#undef NVS_STORE_CASE
  set_error("store_kvcache: unsupported dtype pair src=%d cache=%d", src, dst);
  return NVS_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Dequantisation: out = round_to_out(code * scale)
// ---------------------------------------------------------------------------
template <int CODE>
__device__ __forceinline__ float code_to_f32(uint32_t c) {
  if constexpr (CODE == NVS_DTYPE_INT8)
    return (float)(int32_t)(int8_t)(uint8_t)c;
  else
    return e4m3_to_f32(c);
}

// Widen 8 cache elements of any cache dtype (scale applied for codes).
template <int CACHE>
__device__ __forceinline__ void load8_cache(const void* base, int64_t elem,
                                            float scale, float (&x)[8]) {
  if constexpr (CACHE == NVS_DTYPE_INT8 || CACHE == NVS_DTYPE_FP8_E4M3) {
    u32x2 w = *reinterpret_cast<const u32x2*>((const uint8_t*)base + elem);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      x[i] = code_to_f32<CACHE>((w[i >> 2] >> (8 * (i & 3))) & 0xffu) * scale;
  } else {
    constexpr int B = (CACHE == NVS_DTYPE_FP32) ? 4 : 2;
    load8<CACHE>((const char*)base + elem * B, x);
  }
}

template <int CODE, int OUT>
__global__ __launch_bounds__(256) void dequant_kernel(const void* codes, const float* scales,
                                                      int64_t n_chunks, int chunks_per_row,
                                                      void* out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= n_chunks) return;
  const int64_t row = gid / chunks_per_row;
  constexpr int OB = (OUT == NVS_DTYPE_FP32) ? 4 : 2;
  float x[8];
  load8_cache<CODE>(codes, gid * 8, scales[row], x);
  store8_float<OUT>((char*)out + gid * 8 * OB, x);
}

// ---------------------------------------------------------------------------
// Paged gather (get_kv_cache).  Grid (position tiles, seq).  Each work-group
// first compacts the sequence's non-negative block-table entries into LDS,
// then copies positions [p0, p0 + kGatherPos) of all heads.
// ---------------------------------------------------------------------------
constexpr int kGatherPos = 64;

struct GatherArgs {
  const void* kc;
  const void* vc;
  const float* ks;
  const float* vs;
  const int32_t* bt;
  int64_t bt_stride;
  int max_blocks;
  int64_t NB;
  const int32_t* ctx;
  int max_len;
  int bs, H, D;
  void* ko;
  void* vo;
  uint8_t* mask;
};

template <int CACHE, int OUT>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
  extern __shared__ int32_t lds_blocks[];
  __shared__ int32_t wave_counts[4];
  __shared__ int32_t total_valid;
  const int seq = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t* row = a.bt + (int64_t)seq * a.bt_stride;

  // Stream compaction of row[row >= 0] into lds_blocks, in order.
  int base = 0;
  for (int e0 = 0; e0 < a.max_blocks; e0 += 256) {
    const int e = e0 + tid;
    const int32_t id = (e < a.max_blocks) ? row[e] : -1;
    const bool keep = id >= 0;
    const uint64_t bal = __ballot(keep);
    const int before_in_wave = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wave_counts[wave] = __popcll(bal);
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      before += (w < wave) ? wave_counts[w] : 0;
      tot += wave_counts[w];
    }
    if (keep) lds_blocks[base + before + before_in_wave] = id;
    base += tot;
    __syncthreads();
  }
  if (tid == 0) total_valid = base;
  __syncthreads();
  const int nvalid = total_valid;
  const int ctx = a.ctx[seq];
  int glen = nvalid * a.bs;
  if (ctx < glen) glen = ctx;
  if (glen < 0) glen = 0;

  const int chunks_per_pos = (a.H * a.D) >> 3;
  const int p0 = blockIdx.x * kGatherPos;
  const int p1 = min(p0 + kGatherPos, a.max_len);
  constexpr int OB = (OUT == NVS_DTYPE_FP32) ? 4 : 2;
  for (int idx = tid; idx < (p1 - p0) * chunks_per_pos; idx += 256) {
    const int p = p0 + idx / chunks_per_pos;
    const int cc = idx - (p - p0) * chunks_per_pos;  // (head, chunk)
    const int64_t out_elem = ((int64_t)seq * a.max_len + p) * a.H * a.D + (int64_t)cc * 8;
    float xk[8], xv[8];
    const int blk = p < glen ? lds_blocks[p / a.bs] : -1;
    if (blk >= 0 && blk < a.NB) {
      const int64_t slot = (int64_t)blk * a.bs + (p % a.bs);
      const int h = (cc * 8) / a.D;
      const int64_t src_elem = slot * a.H * a.D + (int64_t)cc * 8;
      float sk = 1.0f, sv = 1.0f;
      if constexpr (CACHE == NVS_DTYPE_INT8 || CACHE == NVS_DTYPE_FP8_E4M3) {
        sk = a.ks[slot * a.H + h];
        sv = a.vs[slot * a.H + h];
      }
      load8_cache<CACHE>(a.kc, src_elem, sk, xk);
      load8_cache<CACHE>(a.vc, src_elem, sv, xv);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) xk[i] = xv[i] = 0.0f;
    }
    store8_float<OUT>((char*)a.ko + out_elem * OB, xk);
    store8_float<OUT>((char*)a.vo + out_elem * OB, xv);
  }
  for (int p = p0 + tid; p < p1; p += 256) a.mask[(int64_t)seq * a.max_len + p] = (p < glen) ? 1 : 0;
}

}  // namespace nvs

using namespace nvs;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" const char* nvs_last_error(void) { return g_err; }

extern "C" int nvs_version(void) { return 100; }

extern "C" int nvs_store_kvcache(const void* k, const void* v, int src_dtype,
                                 int64_t k_tok_stride, int64_t k_head_stride,
                                 int64_t v_tok_stride, int64_t v_head_stride,
                                 const int32_t* slot_mapping, int64_t num_tokens,
                                 void* k_cache, void* v_cache, int cache_dtype,
                                 float* k_scale, float* v_scale, int64_t num_blocks,
                                 int block_size, int num_kv_heads, int head_dim,
                                 void* stream) {
  clear_error();
  NVS_REQUIRE(num_tokens >= 0, NVS_ERR_INVALID, "store_kvcache: num_tokens < 0");
  if (num_tokens == 0) return NVS_OK;
  NVS_REQUIRE(k && v && slot_mapping && k_cache && v_cache, NVS_ERR_INVALID,
              "store_kvcache: null tensor pointer");
  NVS_REQUIRE(src_dtype == NVS_DTYPE_BF16 || src_dtype == NVS_DTYPE_FP16 ||
                  src_dtype == NVS_DTYPE_FP32,
              NVS_ERR_UNSUPPORTED, "store_kvcache: unsupported k/v dtype %d", src_dtype);
  NVS_REQUIRE(dtype_size(cache_dtype) > 0, NVS_ERR_UNSUPPORTED,
              "store_kvcache: unsupported cache dtype %d", cache_dtype);
  NVS_REQUIRE(!is_quant(cache_dtype) || (k_scale && v_scale), NVS_ERR_INVALID,
              "store_kvcache: quantised cache needs k_scale and v_scale");
  NVS_REQUIRE(num_kv_heads > 0 && block_size > 0 && num_blocks > 0, NVS_ERR_INVALID,
              "store_kvcache: bad cache shape");
  const int l2 = lpr_log2_for(head_dim);
  NVS_REQUIRE(l2 >= 0, NVS_ERR_UNSUPPORTED,
              "store_kvcache: head_dim %d must be 8 * 2^n <= 512", head_dim);
  const int sb = dtype_size(src_dtype);
  NVS_REQUIRE((k_tok_stride * sb) % 16 == 0 && (k_head_stride * sb) % 16 == 0 &&
                  (v_tok_stride * sb) % 16 == 0 && (v_head_stride * sb) % 16 == 0 &&
                  ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0,
              NVS_ERR_INVALID, "store_kvcache: k/v rows must be 16-byte aligned");
  StoreArgs a;
  a.k = k; a.v = v;
  a.k_ts = k_tok_stride; a.k_hs = k_head_stride;
  a.v_ts = v_tok_stride; a.v_hs = v_head_stride;
  a.slots = slot_mapping;
  a.rows = num_tokens * num_kv_heads;
  a.total_slots = num_blocks * (int64_t)block_size;
  a.kc = k_cache; a.vc = v_cache; a.ks = k_scale; a.vs = v_scale;
  a.H = num_kv_heads; a.D = head_dim; a.lpr_log2 = l2;
  return launch_store<false, true>(a, src_dtype, cache_dtype, (hipStream_t)stream);
}

extern "C" int nvs_quantize_per_token(const void* x, int src_dtype, int64_t tok_stride,
                                      int64_t head_stride, int64_t num_tokens, int num_heads,
                                      int head_dim, void* codes, int code_dtype, float* scales,
                                      void* stream) {
  clear_error();
  NVS_REQUIRE(num_tokens >= 0 && num_heads > 0, NVS_ERR_INVALID, "quantize: bad shape");
  if (num_tokens == 0) return NVS_OK;
  NVS_REQUIRE(x && codes && scales, NVS_ERR_INVALID, "quantize: null tensor pointer");
  NVS_REQUIRE(is_quant(code_dtype), NVS_ERR_UNSUPPORTED,
              "quantize: code dtype must be INT8 or FP8_E4M3, got %d", code_dtype);
  NVS_REQUIRE(src_dtype == NVS_DTYPE_BF16 || src_dtype == NVS_DTYPE_FP16 ||
                  src_dtype == NVS_DTYPE_FP32,
              NVS_ERR_UNSUPPORTED, "quantize: unsupported input dtype %d", src_dtype);
  const int l2 = lpr_log2_for(head_dim);
  NVS_REQUIRE(l2 >= 0, NVS_ERR_UNSUPPORTED, "quantize: head_dim %d must be 8 * 2^n <= 512",
              head_dim);
  const int sb = dtype_size(src_dtype);
  NVS_REQUIRE((tok_stride * sb) % 16 == 0 && (head_stride * sb) % 16 == 0 &&
                  ((uintptr_t)x % 16) == 0,
              NVS_ERR_INVALID, "quantize: rows must be 16-byte aligned");
  StoreArgs a;
  a.k = x; a.v = x;
  a.k_ts = a.v_ts = tok_stride; a.k_hs = a.v_hs = head_stride;
  a.slots = nullptr;
  a.rows = num_tokens * num_heads;
  a.total_slots = num_tokens;
  a.kc = codes; a.vc = codes; a.ks = scales; a.vs = scales;
  a.H = num_heads; a.D = head_dim; a.lpr_log2 = l2;
  return launch_store<true, false>(a, src_dtype, code_dtype, (hipStream_t)stream);
}

extern "C" int nvs_dequantize_per_token(const void* codes, int code_dtype, const float* scales,
                                        int64_t num_tokens, int num_heads, int head_dim,
                                        void* out, int out_dtype, void* stream) {
  clear_error();
  NVS_REQUIRE(num_tokens >= 0 && num_heads > 0 && head_dim > 0 && head_dim % 8 == 0,
              NVS_ERR_INVALID, "dequantize: bad shape");
  if (num_tokens == 0) return NVS_OK;
  NVS_REQUIRE(codes && scales && out, NVS_ERR_INVALID, "dequantize: null tensor pointer");
  NVS_REQUIRE(is_quant(code_dtype), NVS_ERR_UNSUPPORTED, "dequantize: bad code dtype %d",
              code_dtype);
  const int64_t n_chunks = num_tokens * num_heads * (head_dim / 8);
  const int64_t blocks = (n_chunks + 255) / 256;
  NVS_REQUIRE(blocks < (1ll << 31), NVS_ERR_INVALID, "dequantize: too large");
  hipStream_t s = (hipStream_t)stream;
#define NVS_DQ(C, O)                                                                      \
  if (code_dtype == C && out_dtype == O) {                                                \
    hipLaunchKernelGGL((dequant_kernel<C, O>), dim3((unsigned)blocks), dim3(256), 0, s, codes, \
                       scales, n_chunks, head_dim / 8, out);                              \
    return check_launch("dequantize");                                                    \
  }
  NVS_DQ(NVS_DTYPE_INT8, NVS_DTYPE_BF16)
  NVS_DQ(NVS_DTYPE_INT8, NVS_DTYPE_FP16)
  NVS_DQ(NVS_DTYPE_INT8, NVS_DTYPE_FP32)
  NVS_DQ(NVS_DTYPE_FP8_E4M3, NVS_DTYPE_BF16)
  NVS_DQ(NVS_DTYPE_FP8_E4M3, NVS_DTYPE_FP16)
  NVS_DQ(NVS_DTYPE_FP8_E4M3, NVS_DTYPE_FP32)
#undef NVS_DQ
  set_error("dequantize: unsupported output dtype %d", out_dtype);
  return NVS_ERR_UNSUPPORTED;
}

extern "C" int nvs_gather_kvcache(const void* k_cache, const void* v_cache, int cache_dtype,
                                  const float* k_scale, const float* v_scale,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  int max_blocks_per_seq, const int32_t* context_lens,
                                  int num_seqs, int max_len, int64_t num_blocks, int block_size,
                                  int num_kv_heads, int head_dim, void* k_out, void* v_out,
                                  int out_dtype, uint8_t* kv_mask, void* stream) {
  clear_error();
  NVS_REQUIRE(num_seqs >= 0 && max_len >= 0 && max_blocks_per_seq >= 0, NVS_ERR_INVALID,
              "gather: bad shape");
  if (num_seqs == 0 || max_len == 0) return NVS_OK;
  NVS_REQUIRE(k_cache && v_cache && block_tables && context_lens && k_out && v_out && kv_mask,
              NVS_ERR_INVALID, "gather: null tensor pointer");
  NVS_REQUIRE(!is_quant(cache_dtype) || (k_scale && v_scale), NVS_ERR_INVALID,
              "gather: quantised cache needs scales");
  NVS_REQUIRE(head_dim % 8 == 0 && block_size > 0 && num_kv_heads > 0 && num_blocks > 0,
              NVS_ERR_INVALID, "gather: bad cache shape");
  NVS_REQUIRE(max_blocks_per_seq <= 16384, NVS_ERR_UNSUPPORTED,
              "gather: at most 16384 blocks per sequence");
  NVS_REQUIRE(num_seqs < 65536, NVS_ERR_UNSUPPORTED, "gather: at most 65535 sequences");
  GatherArgs a;
  a.kc = k_cache; a.vc = v_cache; a.ks = k_scale; a.vs = v_scale;
  a.bt = block_tables; a.bt_stride = bt_stride; a.max_blocks = max_blocks_per_seq;
  a.NB = num_blocks;
  a.ctx = context_lens; a.max_len = max_len;
  a.bs = block_size; a.H = num_kv_heads; a.D = head_dim;
  a.ko = k_out; a.vo = v_out; a.mask = kv_mask;
  dim3 grid((max_len + kGatherPos - 1) / kGatherPos, num_seqs);
  const size_t lds = (size_t)(max_blocks_per_seq > 0 ? max_blocks_per_seq : 1) * sizeof(int32_t);
  hipStream_t s = (hipStream_t)stream;
#define NVS_GA(C, O)                                                                   \
  if (cache_dtype == C && out_dtype == O) {                                            \
    hipLaunchKernelGGL((gather_kernel<C, O>), grid, dim3(256), lds, s, a);             \
    return check_launch("gather_kvcache");                                             \
  }
#define NVS_GA_OUT(C)                 \
  NVS_GA(C, NVS_DTYPE_BF16)           \
  NVS_GA(C, NVS_DTYPE_FP16)           \
  NVS_GA(C, NVS_DTYPE_FP32)
  NVS_GA_OUT(NVS_DTYPE_BF16)
  NVS_GA_OUT(NVS_DTYPE_FP16)
  NVS_GA_OUT(NVS_DTYPE_FP32)
  NVS_GA_OUT(NVS_DTYPE_INT8)
  NVS_GA_OUT(NVS_DTYPE_FP8_E4M3)
#undef NVS_GA_OUT
#undef NVS_GA
  set_error("gather: unsupported dtype pair cache=%d out=%d", cache_dtype, out_dtype);
  return NVS_ERR_UNSUPPORTED;
}
