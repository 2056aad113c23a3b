/* Exhaustive check of the KV store's quantisation quotient (CPU, C99 + OpenMP).
 *
 * The store kernel (nanovllm_self_amd/csrc/store_common.h, quotients8) forms
 * the quotient x / scale of a bf16 or fp16 source value with one reciprocal
 * per row and one FMA correction per value:
 *     r = 1 / scale,  q0 = x * r,  q = (q0 == 0) ? q0 : fma(fma(-q0, scale, x), r, q0)
 * The reference divides (nanovllm/layers/attention.py:94-98: x_fp32 / scale).
 * This program enumerates every pair (x, absmax) of finite source values with
 * |x| <= absmax, sets scale = max(absmax / qmax, 1e-6) as the store does, and
 * counts the pairs whose int8 code (rint, clamp +-127) or OCP e4m3 code
 * (clamp +-448, round to nearest even) differs between the two quotients.
 *
 * Every operation is an IEEE binary32 operation with round-to-nearest-even:
 * build with -ffp-contract=off and without -ffast-math (x86-64 SSE arithmetic;
 * fmaf is the correctly rounded fused multiply-add).  gfx950's v_mul_f32,
 * v_fma_f32 and the compiler's default (correctly rounded) fp32 divide give
 * the same bits, so the result holds for the kernel.
 *
 * Usage: store_quotient_check <bf16|fp16> <127|448> [plain]
 *   "plain" drops the FMA correction (q = x * r) to show that the check
 *   detects a quotient that is not the divide's.
 * Prints: "pairs N diff_quotients D diff_codes C" and exits 0.
 * Mode "encoder" checks the e4m3 encoder below against a brute-force nearest
 * (ties to even) search over every bf16 value in [-448, 448] and every
 * midpoint between adjacent e4m3 values +-1 ulp; prints "encoder_errors E".
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bf16_to_f32(uint32_t h) { return bits_f32(h << 16); }

static float f16_to_f32(uint32_t h) {
  const uint32_t s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0)
    v = ldexpf((float)m, -24); /* exact */
  else
    v = ldexpf((float)(m | 0x400), (int)e - 25);
  return s ? -v : v;
}

/* OCP e4m3 (float8_e4m3fn) code of a finite value |y| <= 448, round to
 * nearest even; written from the format: 1 sign bit, 4 exponent bits (bias
 * 7), 3 mantissa bits, subnormals m * 2^-9. */
static uint32_t e4m3_code(float y) {
  uint32_t u = f32_bits(y);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  if (u >= 0x3c800000u) { /* |y| >= 2^-6: normal */
    const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);
    return sign | ((r >> 20) - (120u << 3));
  }
  /* subnormal range: multiples of 2^-9, nearest even multiple on ties */
  const float a = bits_f32(u) * 512.0f; /* exact scaling by 2^9 */
  const float m = rintf(a);
  return sign | (uint32_t)m;
}

static float e4m3_value(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xf, m = c & 7;
  const float v = e ? ldexpf((float)(8 + m), (int)e - 10) : ldexpf((float)m, -9);
  return (c & 0x80) ? -v : v;
}

static uint32_t int8_code(float q) {
  float r = rintf(q);
  r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
  return (uint32_t)(int32_t)r & 0xffu;
}

static uint32_t fp8_code(float q) {
  const float y = q < -448.0f ? -448.0f : (q > 448.0f ? 448.0f : q);
  return e4m3_code(y);
}

/* brute force: the e4m3 value nearest to y (|y| <= 448), ties to the even
 * code; returns the code (sign from y, so -0 for small negative y). */
static uint32_t e4m3_brute(float y) {
  const uint32_t sign = (f32_bits(y) >> 24) & 0x80u;
  const double a = fabs((double)y);
  uint32_t best = 0;
  double bd = 1e300;
  for (uint32_t c = 0; c <= 0x7e; ++c) {
    const double d = fabs((double)e4m3_value(c) - a);
    if (d < bd || (d == bd && (c & 1u) == 0)) {
      bd = d;
      best = c;
    }
  }
  return sign | best;
}

static int encoder_mode(void) {
  long errors = 0, n = 0;
  for (uint32_t h = 0; h < 0x10000; ++h) {
    const float y = bf16_to_f32(h);
    if (!(fabsf(y) <= 448.0f)) continue;
    ++n;
    if (e4m3_code(y) != e4m3_brute(y)) ++errors;
  }
  for (uint32_t c = 0; c < 0x7e; ++c) {
    const float mid = (float)(((double)e4m3_value(c) + (double)e4m3_value(c + 1)) / 2.0);
    const float cand[3] = {nextafterf(mid, 0.0f), mid, nextafterf(mid, 1e9f)};
    for (int k = 0; k < 3; ++k)
      for (int s = 0; s < 2; ++s) {
        const float y = s ? -cand[k] : cand[k];
        ++n;
        if (e4m3_code(y) != e4m3_brute(y)) ++errors;
      }
  }
  printf("encoder_checked %ld encoder_errors %ld\n", n, errors);
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 2 && strcmp(argv[1], "encoder") == 0) return encoder_mode();
  if (argc < 3) {
    fprintf(stderr, "usage: %s <bf16|fp16> <127|448> [plain]\n", argv[0]);
    return 2;
  }
  const int is_bf16 = strcmp(argv[1], "bf16") == 0;
  const float qmax = (float)atof(argv[2]);
  const int plain = argc >= 4 && strcmp(argv[3], "plain") == 0;
  const int fp8 = qmax == 448.0f;
  /* every finite non-negative value, in increasing order of magnitude */
  const uint32_t top = is_bf16 ? 0x7f7fu : 0x7bffu;
  const int nv = (int)top + 1;
  float* pos = (float*)malloc(sizeof(float) * nv);
  for (int i = 0; i < nv; ++i) pos[i] = is_bf16 ? bf16_to_f32((uint32_t)i) : f16_to_f32((uint32_t)i);

  long long pairs = 0, dq = 0, dc = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, dq, dc)
  for (int ia = 0; ia < nv; ++ia) {
    const float absmax = pos[ia];
    float scale = absmax / qmax;
    scale = scale < 1e-6f ? 1e-6f : scale;
    const float r = 1.0f / scale;
    for (int ix = 0; ix <= ia; ++ix) {
      for (int s = 0; s < 2; ++s) {
        const float x = s ? -pos[ix] : pos[ix];
        const float q0 = x * r;
        const float q = plain ? q0 : (q0 == 0.0f ? q0 : fmaf(fmaf(-q0, scale, x), r, q0));
        const float qd = x / scale;
        ++pairs;
        if (f32_bits(q) != f32_bits(qd)) {
          ++dq;
          const uint32_t c1 = fp8 ? fp8_code(q) : int8_code(q);
          const uint32_t c2 = fp8 ? fp8_code(qd) : int8_code(qd);
          if (c1 != c2) ++dc;
        }
      }
    }
  }
  printf("pairs %lld diff_quotients %lld diff_codes %lld\n", pairs, dq, dc);
  free(pos);
  return 0;
}
