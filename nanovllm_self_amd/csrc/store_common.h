// Per-thread helpers of the KV-cache kernels: 8 consecutive head_dim
// elements per thread, widened to fp32, stored, or quantised.
#pragma once

#include "nvs_common.h"

namespace nvs {

// ---------------------------------------------------------------------------
// Loading 8 consecutive source elements as fp32 (exact widening).
// ---------------------------------------------------------------------------
template <int SRC>
__device__ __forceinline__ void load8(const void* p, float (&x)[8]) {
  if constexpr (SRC == NVS_DTYPE_FP32) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 a = q[0], b = q[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (SRC == NVS_DTYPE_BF16) {
        x[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
        x[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
      } else {
        x[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
        x[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
      }
    }
  }
}

// Store 8 values rounded to a float/half element type.
template <int DST>
__device__ __forceinline__ void store8_float(void* p, const float (&x)[8]) {
  if constexpr (DST == NVS_DTYPE_FP32) {
    float4* q = reinterpret_cast<float4*>(p);
    q[0] = make_float4(x[0], x[1], x[2], x[3]);
    q[1] = make_float4(x[4], x[5], x[6], x[7]);
  } else {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DST == NVS_DTYPE_BF16)
        w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);  // one conversion per pair, the same bits
      else
        w[i] = f32_to_f16_bits(x[2 * i]) | (f32_to_f16_bits(x[2 * i + 1]) << 16);
    }
    *reinterpret_cast<u32x4*>(p) = w;
  }
}

// Quantise a row chunk (8 values) given the row scale; 8 one-byte codes.
template <int DST>
__device__ __forceinline__ u32x2 quant8(const float (&x)[8], float scale) {
  if constexpr (DST == NVS_DTYPE_FP8_E4M3) {
    // A finite scale means a finite row, so every clamped quotient is a
    // finite value in [-448, 448]: gfx950's conversion (OCP e4m3, round to
    // nearest even, two values per instruction) encodes it as f32_to_e4m3
    // does, without that encoder's per-value branches.  Rows holding inf or
    // NaN (scale inf or NaN) take the bit-level encoder below.
    if (__builtin_isfinite(scale)) {
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = x[i] / scale;
        y[i] = v < -448.0f ? -448.0f : (v > 448.0f ? 448.0f : v);
      }
      u32x2 w;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int c = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * h], y[4 * h + 1], 0, false);
        c = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * h + 2], y[4 * h + 3], c, true);
        w[h] = (uint32_t)c;
      }
      return w;
    }
  }
  u32x2 w = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t c = (DST == NVS_DTYPE_INT8) ? quant_int8(x[i], scale)
                                         : quant_fp8(x[i], scale);
    w[i >> 2] |= c << (8 * (i & 3));
  }
  return w;
}

// absmax over the lanes of one row; rows are 2^lpr_log2 consecutive lanes.
__device__ __forceinline__ float row_absmax(const float (&x)[8], int lpr) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
  for (int s = 1; s < lpr; s <<= 1) m = fmaxf(m, shfl_xor(m, s));
  return m;
}

}  // namespace nvs
