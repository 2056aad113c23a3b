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

// The quotients x[i] / scale that decide the codes.  With SRC16 (every x[i]
// a bf16 or fp16 value, the row's scale max(absmax / qmax, 1e-6) finite)
// they come from one reciprocal and an FMA correction,
//   q0 = x r,  q = q0 + (x - q0 scale) r   (r = 1 / scale, q = q0 for x = 0),
// whose int8 and e4m3 codes equal those of the correctly rounded x / scale
// for every pair of bf16 values and every pair of fp16 values with |x| <=
// absmax, for both qmax: tests/test_store_quotient.py enumerates all of
// them (about 2^30 pairs per source type) with the same IEEE fp32 operations
// on the CPU; the quotients differ for about 4.6e5 bf16 pairs, the codes for
// none.  fp32 sources, and rows with inf or NaN, take an IEEE divide per value.
template <bool SRC16>
__device__ __forceinline__ void quotients8(const float (&x)[8], float scale, float (&q)[8]) {
  if (SRC16 && __builtin_isfinite(scale)) {
    const float r = 1.0f / scale;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float q0 = x[i] * r;
      q[i] = q0 == 0.0f ? q0 : __builtin_fmaf(__builtin_fmaf(-q0, scale, x[i]), r, q0);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = x[i] / scale;
  }
}

// Quantise a row chunk (8 values) given the row scale; 8 one-byte codes.
// SRC16: the values are bf16 / fp16 ones (see quotients8).
template <int DST, bool SRC16 = false>
__device__ __forceinline__ u32x2 quant8(const float (&x)[8], float scale) {
  float q[8];
  quotients8<SRC16>(x, scale, q);
  u32x2 w = {0u, 0u};
  if constexpr (DST == NVS_DTYPE_FP8_E4M3) {
    // A finite scale means a finite row, so every clamped quotient is a
    // finite value in [-448, 448]: gfx950's conversion (OCP e4m3, round to
    // nearest even, two values per instruction) encodes it as f32_to_e4m3
    // does, without that encoder's per-value branches.  Rows holding inf or
    // NaN (scale inf or NaN) take the bit-level encoder.
    if (__builtin_isfinite(scale)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = q[i] < -448.0f ? -448.0f : (q[i] > 448.0f ? 448.0f : q[i]);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int c = __builtin_amdgcn_cvt_pk_fp8_f32(q[4 * h], q[4 * h + 1], 0, false);
        c = __builtin_amdgcn_cvt_pk_fp8_f32(q[4 * h + 2], q[4 * h + 3], c, true);
        w[h] = (uint32_t)c;
      }
      return w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float y = q[i] < -448.0f ? -448.0f : (q[i] > 448.0f ? 448.0f : q[i]);
      w[i >> 2] |= f32_to_e4m3(y) << (8 * (i & 3));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i >> 2] |= int8_code(q[i]) << (8 * (i & 3));
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
