// Fused pre-attention step of a Qwen3 attention layer for gfx950: per-head
// RMSNorm of q and k, rotary embedding of both, and the KV-cache write of
// the rotated k and of v (quantised for int8 / fp8 caches).
//
// Reference semantics (nanovllm/models/qwen3.py:100-104 and the layers it
// calls):
//   RMSNorm (layers/RMSNorm.py:11-18), per (token, head) in fp32:
//     rms = sqrt(mean(x^2) + eps);  y = bf16((w * x) / rms)
//   rotary embedding (layers/RoPE.py:5-25, 60-74), cos/sin from the model's
//   fp32 cos_sin_cache [max_position, 1, 2 * (D / 2)] at the token's position:
//     x1, x2 = first and second half of the normalised head (as fp32)
//     y1 = x1 cos - x2 sin;  y2 = x2 cos + x1 sin;  out = bf16(cat(y1, y2))
//   KV write (layers/attention.py:139-189): as nvs_store_kvcache, from the
//   rotated bf16 k and the raw v.
// Each product and sum is rounded on its own (no fused multiply-add), as the
// eager torch ops compute them.
//
// Work: one wave per token.  Its rows (units) are the Hq query heads, then
// the Hkv key heads, then the Hkv value heads; the wave's four 16-lane groups
// take rows g, g + 4, g + 8, ..., four passes at a time with every load of
// the four issued before any is used.  Lane j holds elements 8 j .. 8 j + 7
// of its head (head_dim 128) as one 16-byte load, its rotary partners
// (elements +-64) sit in lane j ^ 8, and the norm's sum is a butterfly over
// the row's 16 lanes.  The token's position, cos/sin and the two norm
// weights are loaded once per wave.
#include <algorithm>

#include "nvs_common.h"
#include "store_common.h"

namespace nvs {

namespace {

constexpr int kPrepD = 128;
constexpr int kRowLanes = 16;  // lanes per head row, 8 elements each
constexpr int kPrepThreads = 256;
constexpr int kPrepTokens = kPrepThreads / 64;  // one wave per token
constexpr int kPrepUnroll = 4;                  // passes whose loads are issued together

struct PrepArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_ts, q_hs, k_ts, k_hs, v_ts, v_hs;
  const int64_t* pos;
  int64_t T;
  const uint16_t* qw;
  const uint16_t* kw;
  float eps;
  const float* cs;  // [max_pos, 128]: cos at 0..63, sin at 64..127
  int64_t max_pos;
  const int32_t* slots;
  int64_t total_slots;
  void* kc;
  void* vc;
  float* ks;
  float* vs;
  int Hq, Hkv;
  uint16_t* qo;
  int64_t qo_ts, qo_hs;
  uint16_t* ko;  // may be null
  int64_t ko_ts, ko_hs;
};

// The 8 values rounded to bf16 in place, two per conversion; `bits` holds
// them packed (element 2 m in the low half of word m), as a store wants them.
__device__ __forceinline__ void round8_bf16(float (&v)[8], u32x4& bits) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t w = pack_bf16x2(v[2 * m], v[2 * m + 1]);
    bits[m] = w;
    v[2 * m] = __uint_as_float(w << 16);
    v[2 * m + 1] = __uint_as_float(w & 0xffff0000u);
  }
}

__device__ __forceinline__ void unpack8_bf16(const u32x4& w, float (&x)[8]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    x[2 * m] = __uint_as_float(w[m] << 16);
    x[2 * m + 1] = __uint_as_float(w[m] & 0xffff0000u);
  }
}

// Products and sums rounded one by one: with contraction off the compiler
// cannot fuse x * c - y * s into a multiply-add.  (Division is correctly
// rounded in this build's float model.)
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// a / b correctly rounded from y = RN(1 / b), with one multiply and two
// fused multiply-adds instead of a division per element (Markstein's
// theorem: q0 = RN(a y) is within an ulp of a / b, r = a - b q0 is exact in
// an FMA, and RN(q0 + r y) = RN(a / b)).  It needs b normal and finite and
// r not to underflow, which |a| >= 2^-100 (or a = 0) ensures.
__device__ __forceinline__ float div_by_recip(float a, float b, float y) {
  const float q0 = mul_rn(a, y);
  const float r = __builtin_fmaf(-b, q0, a);
  return __builtin_fmaf(r, y, q0);
}

// Lane j ^ m of the lane's 16-lane row, for m = 1, 2, 4, 8, as DPP moves
// (VALU, no trip through the LDS crossbar): quad_perm for 1 and 2,
// row_half_mirror (j ^ 7) then quad_perm j ^ 3 for 4, and a rotation of the
// row by 8 for 8.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int M>
__device__ __forceinline__ float row_xor(float v) {
  if constexpr (M == 1) return dpp<0xB1>(v);  // quad_perm(1, 0, 3, 2)
  if constexpr (M == 2) return dpp<0x4E>(v);  // quad_perm(2, 3, 0, 1)
  if constexpr (M == 4) return dpp<0x1B>(dpp<0x141>(v));  // half mirror, then quad_perm(3, 2, 1, 0)
  return dpp<0x128>(v);  // row_ror:8
}

// Sum over the 16 lanes of a head row: a butterfly, lane partners j ^ 1,
// j ^ 2, j ^ 4, j ^ 8.
__device__ __forceinline__ float row_sum16(float v) {
  v = add_rn(v, row_xor<1>(v));
  v = add_rn(v, row_xor<2>(v));
  v = add_rn(v, row_xor<4>(v));
  return add_rn(v, row_xor<8>(v));
}

// Every source row is read once and every destination row written once:
// both marked non-temporal (`nt`), which keeps the stream from displacing
// other lines in the caches (36 864 tokens: 180 -> 165 us; the loads alone
// marked: 186 us, the stores alone: 174 us).
#ifndef NVS_PREP_NT
#define NVS_PREP_NT 1
#endif
#ifndef NVS_PREP_NTS
#define NVS_PREP_NTS 1
#endif
__device__ __forceinline__ u32x4 prep_load(const u32x4* p) {
  if constexpr (NVS_PREP_NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <typename V>
__device__ __forceinline__ void prep_store(V* p, V v) {
  if constexpr (NVS_PREP_NTS) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Writes lane j's 8 elements of head row `row` of a cache of dtype DST;
// quantised caches take the row scale from the absmax over the row's lanes.
template <int DST>
__device__ __forceinline__ void cache_row(void* cache, float* scales, int64_t row, const float (&x)[8],
                                          bool write) {
  const int j = threadIdx.x & (kRowLanes - 1);
  const int64_t e = row * kPrepD + 8 * j;
  if constexpr (DST == NVS_DTYPE_INT8 || DST == NVS_DTYPE_FP8_E4M3) {
    constexpr float qmax = (DST == NVS_DTYPE_INT8) ? QuantInt8::kQmax : QuantFp8::kQmax;
    const float sc = quant_scale(row_absmax(x, kRowLanes), qmax);
    if (write) {
      prep_store(reinterpret_cast<u32x2*>((uint8_t*)cache + e), quant8<DST, true>(x, sc));
      if (j == 0) scales[row] = sc;
    }
  } else {
    constexpr int B = (DST == NVS_DTYPE_FP32) ? 4 : 2;
    if (write) store8_float<DST>((char*)cache + e * B, x);
  }
}

// The per-token values a section needs: the lane's cos / sign-folded sin,
// the token's cache row and output rows.
struct PrepToken {
  float c[8], s[8];
  bool ok;           // the slot is inside the cache
  int64_t cslot;     // the slot (0 when not ok; nothing is written then)
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* qo;
  uint16_t* ko;      // null: the rotated k is not returned
};

// The token's q heads (KIND 0) or its k and v heads (KIND 1), four rows a
// pass (head g + 4 p on lane group g), the loads of kPrepUnroll rows issued
// before any is used (KIND 1: the k and v rows of kPrepUnroll / 2 passes).
// Rows past the heads re-read the last one and write nothing.  q and k rows:
// RMSNorm (mean of squares over the 128 elements, division by 128 exact),
// rounding to bf16, rotation, rounding to bf16; q goes to q_out, k to k_out
// and the cache; v rows go to the cache as they are (cast or quantised).
template <int KIND, int DST>
__device__ __forceinline__ void prep_section(const PrepArgs& a, const PrepToken& tk, const uint16_t* src, int hs,
                                             const uint16_t* vsrc, int vhs, int H, const float (&w)[8], int g,
                                             int j) {
  constexpr int PER = KIND == 0 ? kPrepUnroll : kPrepUnroll / 2;  // passes per round of loads
  const int passes = (H + 3) / 4;
  for (int p0 = 0; p0 < passes; p0 += PER) {
    u32x4 xw[kPrepUnroll];
#pragma unroll
    for (int k = 0; k < kPrepUnroll; ++k) {
      const bool isv = KIND == 1 && k >= PER;
      const int h = min(g + 4 * (p0 + k % PER), H - 1);
      xw[k] = prep_load(reinterpret_cast<const u32x4*>((isv ? vsrc : src) + (uint32_t)(h * (isv ? vhs : hs) + 8 * j)));
    }
#pragma unroll
    for (int k = 0; k < kPrepUnroll; ++k) {
      if (p0 + k % PER >= passes) continue;
      const int h = g + 4 * (p0 + k % PER);
      if (h >= H) continue;
      if (KIND == 1 && k >= PER) {  // value head: copy / cast / quantise into the cache
        const int64_t row = tk.cslot * a.Hkv + h;
        if constexpr (DST == NVS_DTYPE_BF16) {
          if (tk.ok) prep_store(reinterpret_cast<u32x4*>((uint16_t*)a.vc + row * kPrepD + 8 * j), xw[k]);
        } else {
          float x[8];
          unpack8_bf16(xw[k], x);
          cache_row<DST>(a.vc, a.vs, row, x, tk.ok);
        }
        continue;
      } else {
        float x[8];
        unpack8_bf16(xw[k], x);
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = add_rn(ss, mul_rn(x[i], x[i]));
        ss = row_sum16(ss);
        // __builtin_sqrtf is the correctly rounded square root (HIP's
        // __fsqrt_rn is the raw v_sqrt_f32 here, off by an ulp at times).
        const float rms = __builtin_sqrtf(add_rn(mul_rn(ss, 1.0f / kPrepD), a.eps));
        float n[8];
        if (rms >= 0x1p-126f && rms <= 0x1p126f) {
          const float inv = __fdiv_rn(1.0f, rms);
#pragma unroll
          for (int i = 0; i < 8; ++i) n[i] = div_by_recip(mul_rn(w[i], x[i]), rms, inv);
        } else {  // rms 0, subnormal, huge or not finite: divide
#pragma unroll
          for (int i = 0; i < 8; ++i) n[i] = __fdiv_rn(mul_rn(w[i], x[i]), rms);
        }
        u32x4 nb;
        round8_bf16(n, nb);
        // Rotary pairs (e, e + 64): lanes j and j ^ 8 hold the two halves.
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = add_rn(mul_rn(n[i], tk.c[i]), mul_rn(row_xor<8>(n[i]), tk.s[i]));
        u32x4 yb;
        round8_bf16(y, yb);
        if constexpr (KIND == 0) {
          prep_store(reinterpret_cast<u32x4*>(tk.qo + (uint32_t)(h * (int)a.qo_hs + 8 * j)), yb);
        } else {
          if (tk.ko) prep_store(reinterpret_cast<u32x4*>(tk.ko + (uint32_t)(h * (int)a.ko_hs + 8 * j)), yb);
          if constexpr (DST == NVS_DTYPE_BF16) {
            if (tk.ok) prep_store(reinterpret_cast<u32x4*>((uint16_t*)a.kc + (tk.cslot * a.Hkv + h) * kPrepD + 8 * j), yb);
          } else {
            cache_row<DST>(a.kc, a.ks, tk.cslot * a.Hkv + h, y, tk.ok);
          }
        }
      }
    }
  }
}

template <int DST>
__global__ __launch_bounds__(kPrepThreads) void qk_prep_kernel(PrepArgs a) {
  // The token is wave-uniform (through readfirstlane, so its pointers are
  // scalar); a lane adds a 32-bit offset for its head row and elements.
  const int64_t t = (int64_t)blockIdx.x * kPrepTokens + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= a.T) return;  // whole waves exit together
  const int g = (threadIdx.x >> 4) & 3, j = threadIdx.x & (kRowLanes - 1);
  PrepToken tk;
  const int64_t slot = a.slots[t];
  tk.ok = slot >= 0 && slot < a.total_slots;
  tk.cslot = tk.ok ? slot : 0;

  // Per token: rotary cos / sin of the lane's elements and the norm weights.
  int64_t p = a.pos[t];
  p = p < 0 ? 0 : (p >= a.max_pos ? a.max_pos - 1 : p);
  const float* cs = a.cs + p * kPrepD + 8 * (j & 7);
  float qw[8], kw[8];
  *reinterpret_cast<f32x4*>(tk.c) = *reinterpret_cast<const f32x4*>(cs);
  *reinterpret_cast<f32x4*>(tk.c + 4) = *reinterpret_cast<const f32x4*>(cs + 4);
  *reinterpret_cast<f32x4*>(tk.s) = *reinterpret_cast<const f32x4*>(cs + 64);
  *reinterpret_cast<f32x4*>(tk.s + 4) = *reinterpret_cast<const f32x4*>(cs + 68);
  load8<NVS_DTYPE_BF16>(a.qw + 8 * j, qw);
  load8<NVS_DTYPE_BF16>(a.kw + 8 * j, kw);
  // First half: y1 = x1 cos - x2 sin; second half: y2 = x2 cos + x1 sin.
  // a - b and a + (-b) round identically, so both halves are one add of a
  // product whose sine carries the sign.
  const bool first = j < 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) tk.s[i] = first ? -tk.s[i] : tk.s[i];
  tk.qo = a.qo + t * a.qo_ts;
  tk.ko = a.ko ? a.ko + t * a.ko_ts : nullptr;
  prep_section<0, DST>(a, tk, a.q + t * a.q_ts, (int)a.q_hs, nullptr, 0, a.Hq, qw, g, j);
  prep_section<1, DST>(a, tk, a.k + t * a.k_ts, (int)a.k_hs, a.v + t * a.v_ts, (int)a.v_hs, a.Hkv, kw, g, j);
}

bool is_code_dtype(int dt) { return dt == NVS_DTYPE_INT8 || dt == NVS_DTYPE_FP8_E4M3; }

}  // namespace
}  // namespace nvs

using namespace nvs;

extern "C" int nvs_qk_norm_rope_store(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                      const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                                      const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                      const int64_t* positions, int64_t num_tokens,
                                      const void* q_norm_weight, const void* k_norm_weight, float eps,
                                      const float* cos_sin_cache, int64_t max_position,
                                      const int32_t* slot_mapping, void* k_cache, void* v_cache,
                                      int cache_dtype, float* k_scale, float* v_scale, int64_t num_blocks,
                                      int block_size, int num_heads, int num_kv_heads, int head_dim,
                                      void* q_out, int64_t q_out_tok_stride, int64_t q_out_head_stride,
                                      void* k_out, int64_t k_out_tok_stride, int64_t k_out_head_stride,
                                      void* stream) {
  clear_error();
  const char* who = "qk_norm_rope_store";
  NVS_REQUIRE(num_tokens >= 0, NVS_ERR_INVALID, "%s: num_tokens < 0", who);
  NVS_REQUIRE(head_dim == kPrepD, NVS_ERR_UNSUPPORTED, "%s: head_dim %d (this build serves 128)", who,
              head_dim);
  NVS_REQUIRE(num_heads > 0 && num_kv_heads > 0, NVS_ERR_INVALID, "%s: head counts must be positive", who);
  NVS_REQUIRE(q_norm_weight && k_norm_weight && cos_sin_cache && k_cache && v_cache, NVS_ERR_INVALID,
              "%s: null pointer argument", who);
  // Per-token arrays may be null for an empty batch.
  NVS_REQUIRE(num_tokens == 0 || (q && k && v && positions && slot_mapping && q_out), NVS_ERR_INVALID,
              "%s: null pointer argument", who);
  NVS_REQUIRE(max_position > 0, NVS_ERR_INVALID, "%s: max_position must be positive", who);
  NVS_REQUIRE(eps >= 0.0f, NVS_ERR_INVALID, "%s: eps must be >= 0", who);
  NVS_REQUIRE(num_blocks > 0 && block_size > 0, NVS_ERR_INVALID, "%s: empty cache", who);
  NVS_REQUIRE(cache_dtype == NVS_DTYPE_BF16 || cache_dtype == NVS_DTYPE_FP16 || cache_dtype == NVS_DTYPE_FP32 ||
                  is_code_dtype(cache_dtype),
              NVS_ERR_UNSUPPORTED, "%s: cache dtype %d", who, cache_dtype);
  NVS_REQUIRE(!is_code_dtype(cache_dtype) || (k_scale && v_scale), NVS_ERR_INVALID,
              "%s: quantised caches need k_scale and v_scale", who);
  NVS_REQUIRE((int64_t)num_heads * q_head_stride < (1ll << 30) && (int64_t)num_heads * q_out_head_stride < (1ll << 30) &&
                  (int64_t)num_kv_heads * (k_head_stride + v_head_stride + k_out_head_stride) < (1ll << 30),
              NVS_ERR_INVALID, "%s: head strides too large", who);
  NVS_REQUIRE(q_tok_stride >= 0 && q_head_stride >= 0 && k_tok_stride >= 0 && k_head_stride >= 0 &&
                  v_tok_stride >= 0 && v_head_stride >= 0 && q_out_tok_stride >= 0 && q_out_head_stride >= 0 &&
                  k_out_tok_stride >= 0 && k_out_head_stride >= 0,
              NVS_ERR_INVALID, "%s: negative stride", who);
  if (num_tokens == 0) return NVS_OK;
  const int64_t blocks = (num_tokens + kPrepTokens - 1) / kPrepTokens;
  NVS_REQUIRE(blocks < (1ll << 31), NVS_ERR_INVALID, "%s: too many tokens (%lld)", who, (long long)num_tokens);
  PrepArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.q_ts = q_tok_stride; a.q_hs = q_head_stride; a.k_ts = k_tok_stride; a.k_hs = k_head_stride;
  a.v_ts = v_tok_stride; a.v_hs = v_head_stride;
  a.pos = positions; a.T = num_tokens;
  a.qw = (const uint16_t*)q_norm_weight; a.kw = (const uint16_t*)k_norm_weight; a.eps = eps;
  a.cs = cos_sin_cache; a.max_pos = max_position;
  a.slots = slot_mapping; a.total_slots = num_blocks * (int64_t)block_size;
  a.kc = k_cache; a.vc = v_cache; a.ks = k_scale; a.vs = v_scale;
  a.Hq = num_heads; a.Hkv = num_kv_heads;
  a.qo = (uint16_t*)q_out; a.qo_ts = q_out_tok_stride; a.qo_hs = q_out_head_stride;
  a.ko = (uint16_t*)k_out; a.ko_ts = k_out_tok_stride; a.ko_hs = k_out_head_stride;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)blocks), block(kPrepThreads);
  switch (cache_dtype) {
    case NVS_DTYPE_BF16: hipLaunchKernelGGL(qk_prep_kernel<NVS_DTYPE_BF16>, grid, block, 0, s, a); break;
    case NVS_DTYPE_FP16: hipLaunchKernelGGL(qk_prep_kernel<NVS_DTYPE_FP16>, grid, block, 0, s, a); break;
    case NVS_DTYPE_FP32: hipLaunchKernelGGL(qk_prep_kernel<NVS_DTYPE_FP32>, grid, block, 0, s, a); break;
    case NVS_DTYPE_INT8: hipLaunchKernelGGL(qk_prep_kernel<NVS_DTYPE_INT8>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(qk_prep_kernel<NVS_DTYPE_FP8_E4M3>, grid, block, 0, s, a); break;
  }
  return check_launch(who);
}
