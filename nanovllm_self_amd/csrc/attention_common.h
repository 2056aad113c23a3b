// Definitions shared by the decode and prefill attention kernels.
#pragma once

#include "nvs_common.h"

namespace nvs {

constexpr int kHeadDim = 128;    // head_dim served by the attention kernels
constexpr int kDecodePart = 256; // keys per decode wave (one split-K partition)

inline int decode_max_parts(int max_seqlen_k) {
  const int p = (max_seqlen_k + kDecodePart - 1) / kDecodePart;
  return p < 1 ? 1 : p;
}

// 2^x on the hardware transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two fp32 values that are exactly bf16-representable -> packed bf16x2 by
// keeping their upper halves (no rounding needed).
__device__ __forceinline__ uint32_t pack_exact_bf16x2(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Codes in bytes (0,1) (HI = false) or (2,3) (HI = true) of x -> two fp32,
// exact.  gfx950 converts OCP e4m3 in hardware.
template <int KV, bool HI>
__device__ __forceinline__ void code_pair_to_f32(uint32_t x, float& f0, float& f1) {
  if constexpr (KV == NVS_DTYPE_FP8_E4M3) {
    const auto f = __builtin_amdgcn_cvt_pk_f32_fp8(x, HI);
    f0 = f[0];
    f1 = f[1];
  } else {
    constexpr int sh = HI ? 16 : 0;
    f0 = (float)(int32_t)(int8_t)(uint8_t)(x >> sh);
    f1 = (float)(int32_t)(int8_t)(uint8_t)(x >> (sh + 8));
  }
}

// Same pair -> packed bf16x2; int8 and e4m3 values are exactly representable
// in bf16, so no rounding happens.
template <int KV, bool HI>
__device__ __forceinline__ uint32_t code_pair_to_bf16x2(uint32_t x) {
  float f0, f1;
  code_pair_to_f32<KV, HI>(x, f0, f1);
  return pack_exact_bf16x2(f0, f1);
}

// 8 codes (bytes of lo then hi) -> bf16x8 operand.
template <int KV>
__device__ __forceinline__ bf16x8 codes8_to_bf16x8(uint32_t lo, uint32_t hi) {
  u32x4 w;
  w[0] = code_pair_to_bf16x2<KV, false>(lo);
  w[1] = code_pair_to_bf16x2<KV, true>(lo);
  w[2] = code_pair_to_bf16x2<KV, false>(hi);
  w[3] = code_pair_to_bf16x2<KV, true>(hi);
  return __builtin_bit_cast(bf16x8, w);
}

// Validated launch parameters of one attention call.
struct AttnParams {
  const void* q;
  int64_t q_ts, q_hs;
  // paged mode
  const void* kc;
  const void* vc;
  int cache_dtype;
  const float* ks;
  const float* vs;
  const int32_t* bt;  // null selects the local (non-paged) mode
  int64_t bt_stride;
  int bs;
  int64_t NB;
  // local mode
  const void* k;
  const void* v;
  int64_t k_ts, k_hs, v_ts, v_hs;
  // batch
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B;
  int64_t T;
  int max_seqlen_q, max_seqlen_k;
  int Hq, Hkv;
  float softmax_scale;
  void* out;
  int64_t out_ts, out_hs;
  void* ws;
  int64_t ws_bytes;
};

int64_t decode_workspace_bytes(int num_seqs, int max_seqlen_k, int num_heads);
int launch_decode(const AttnParams& P, hipStream_t stream);
int launch_prefill(const AttnParams& P, bool skip_decode_rows, hipStream_t stream);

}  // namespace nvs
