// Shared device/host helpers for the gfx950 paged-KV attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/nvs_attention.h"

namespace nvs {

// ---------------------------------------------------------------------------
// Error plumbing: one message per calling thread, returned by nvs_last_error.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();
int check_launch(const char* what);

#define NVS_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      ::nvs::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)

// ---------------------------------------------------------------------------
// Vector types
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Per-lane address offsets.  global_load/store take a 64-bit wave-uniform base
// in scalar registers plus a 32-bit lane offset when the address is built as
// base + zext(offset) in the same block.  A loop-invariant offset would be
// zero-extended once before the loop and kept as a 64-bit lane address in two
// registers; passing it through an empty asm at the use keeps the extension
// in the block, so the offset stays one 32-bit register.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lane_off(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// ---------------------------------------------------------------------------
// Scalar conversions.  Widening bf16/fp16 -> fp32 is exact; narrowing uses
// round-to-nearest-even, the rounding torch's .to(dtype) applies.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// fp32 -> bf16 bits, round-to-nearest-even, NaN kept quiet.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16x2 (low half = a), RNE: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed fp16x2 (low half = a), RNE.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// acc + lo(x) + hi(x) for a packed bf16x2 x, in fp32 (v_dot2c_f32_bf16 with 1.0).
__device__ __forceinline__ float add_bf16x2(uint32_t x, float acc) {
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), ones, acc, false);
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// fp32 -> OCP float8_e4m3fn code with round-to-nearest-even.
// Format: 1 sign, 4 exponent (bias 7), 3 mantissa bits; the largest finite
// magnitude is 448 (S.1111.110) and S.1111.111 is NaN; there is no infinity.
// Normal range |x| >= 2^-6; below it codes are m * 2^-9, m = 0..7.
// Magnitudes that round above 448 (>= 464 rounds up) encode as NaN, like a
// non-saturating cast; callers clamp to +-448 first.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  if (u >= 0x43f00000u) return sign | 0x7fu;  // >= 480, inf or NaN
  uint32_t code;
  if (u >= 0x3c800000u) {
    // Normal: keep 3 of 23 mantissa bits, RNE on the dropped 20 bits, then
    // rebias the exponent from 127 to 7 (difference 120 << 3 in code units).
    const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);
    code = (r >> 20) - (120u << 3);
    if (code > 0x7eu) code = 0x7fu;  // rounded past 448 -> NaN code
  } else {
    // Subnormal / zero: the value is m * 2^-9; |x| * 512 is exact, rint is RNE.
    // m == 8 is the smallest normal (code 0x08), which the encoding absorbs.
    code = (uint32_t)__builtin_rintf(__uint_as_float(u) * 512.0f);
  }
  return sign | code;
}

// Per-token quantisation constants.
struct QuantInt8 {
  static constexpr float kQmax = 127.0f;
};
struct QuantFp8 {
  static constexpr float kQmax = 448.0f;
};

// scale = max(absmax / qmax, 1e-6) with an IEEE (correctly rounded) divide and
// NaN propagation, as torch's (absmax / q).clamp(min=1e-6) does.
__device__ __forceinline__ float quant_scale(float absmax, float qmax) {
  float s = absmax / qmax;
  return (s < 1e-6f) ? 1e-6f : s;
}

// int8 code of a quotient x / scale: round half to even, clamp to +-127.
__device__ __forceinline__ uint32_t int8_code(float quotient) {
  float q = __builtin_rintf(quotient);
  q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
  return ((uint32_t)(int32_t)q) & 0xffu;
}


// e4m3 code (low byte) -> fp32, exact.  gfx950 converts OCP e4m3 in hardware.
__device__ __forceinline__ float e4m3_to_f32(uint32_t code) {
  return __builtin_amdgcn_cvt_f32_fp8(code, 0);
}

// ---------------------------------------------------------------------------
// Lane shuffles (wave64)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Element-size of an nvs_dtype (0 if unknown).
inline int dtype_size(int dt) {
  switch (dt) {
    case NVS_DTYPE_BF16:
    case NVS_DTYPE_FP16:
      return 2;
    case NVS_DTYPE_FP32:
      return 4;
    case NVS_DTYPE_INT8:
    case NVS_DTYPE_FP8_E4M3:
      return 1;
    default:
      return 0;
  }
}

inline bool is_quant(int dt) {
  return dt == NVS_DTYPE_INT8 || dt == NVS_DTYPE_FP8_E4M3;
}

}  // namespace nvs
