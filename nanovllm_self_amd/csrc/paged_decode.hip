// Split-K paged decode (q_len == 1 rows) for gfx950.
//
// Reference semantics: the q_len == 1 rows of prefill_flashattn's paged call
// (nanovllm/layers/attention.py:356-375) and of prefill_torch's prefix branch
// (:441-498): out[h] = softmax(q[h] . K^T * scale) V over the sequence's
// k_len cached keys, kv head h / (Hq / Hkv).
//
// Work decomposition: one wave64 per (sequence, kv head, partition of
// kPart keys).  The wave serves every query head of its kv head, so each
// K/V byte is read from HBM exactly once.  Per 32-key tile:
//   S^T[32 keys x 16 heads] = K[32 x 128] . Q^T   (8 x mfma_f32_16x16x32_bf16)
//   O^T[128 x 16 heads]    += V^T[128 x 32] . P^T (8 x mfma_f32_16x16x32_bf16)
// With keys as the MFMA row index, the S^T accumulator layout (lane = head
// column, 4 consecutive keys per lane group) is exactly the B-operand layout
// that P^T needs, so P never leaves registers.  V rows are loaded with full
// 256-byte coalescing and transposed in registers with v_perm_b32.  Quantised
// codes are converted to bf16 exactly in registers (int8 and e4m3 values are
// bf16-representable); the per-key scales multiply S (K) and P (V).
// Each wave writes a partial (m, l, o[128]) per head; decode_reduce_kernel
// merges the partitions with a log-sum-exp.
#include "nvs_common.h"
#include "attention_common.h"

namespace nvs {

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const void* kc;
  const void* vc;
  const float* ks;
  const float* vs;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* bt;
  int64_t bt_stride;  // row stride == number of columns
  int64_t NB;
  int64_t T;  // query / output rows
  int Hq, Hkv, g, bs;
  int max_parts;
  float scale_log2;
  float* ws_o;   // [B, Hq, max_parts, 128]
  float* ws_ml;  // [B, Hq, max_parts, 2]
  uint16_t* out;
  int64_t out_ts, out_hs;
};

// Registers of one 32-key tile as loaded from HBM.
template <int KV>
struct DecodeTile;

template <>
struct DecodeTile<NVS_DTYPE_BF16> {
  u32x4 k[2][4];  // [subtile t][d step s]: key 16t + col, d = 32 grp + 8 s
  u32x4 v[8];     // [slot e]: key 16(e/4) + 4 grp + e%4, d = 8 col .. +7
};

template <int KV>
struct DecodeTile {
  u32x4 k[2][2];  // [t][half]: 32 codes, d = 32 grp + 16 half .. +15
  u32x2 v[8];     // [e]: 8 codes, d = 8 col .. +7
  float ksc[8];   // scales of the 8 keys the lane owns (slot order)
  float vsc[8];
};

template <int KV>
__device__ __forceinline__ void decode_load(DecodeTile<KV>& T, const DecodeArgs& a, int b, int h,
                                            int kt, int col, int grp) {
  const int lblk = kt / a.bs;
  int blk = lblk < a.bt_stride ? a.bt[(int64_t)b * a.bt_stride + lblk] : -1;
  if (blk >= a.NB) blk = -1;  // never read outside the pool
  const int64_t slot0 = (int64_t)blk * a.bs + (kt - lblk * a.bs);
  constexpr int D = kHeadDim;
  if (blk < 0) {
    // Missing block: zero K and V (the eager path's zero padding).
    if constexpr (KV == NVS_DTYPE_BF16) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) T.k[t][s] = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; ++e) T.v[e] = u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t) T.k[t][0] = T.k[t][1] = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        T.v[e] = u32x2{0, 0};
        T.ksc[e] = 0.0f;
        T.vsc[e] = 0.0f;
      }
    }
    return;
  }
  if constexpr (KV == NVS_DTYPE_BF16) {
    const uint16_t* kc = (const uint16_t*)a.kc;
    const uint16_t* vc = (const uint16_t*)a.vc;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint16_t* kr = kc + ((slot0 + 16 * t + col) * a.Hkv + h) * D + 32 * grp;
#pragma unroll
      for (int s = 0; s < 4; ++s) T.k[t][s] = *reinterpret_cast<const u32x4*>(kr + 8 * s);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = 16 * (e >> 2) + 4 * grp + (e & 3);
      T.v[e] = *reinterpret_cast<const u32x4*>(vc + ((slot0 + key) * a.Hkv + h) * D + 8 * col);
    }
  } else {
    const uint8_t* kc = (const uint8_t*)a.kc;
    const uint8_t* vc = (const uint8_t*)a.vc;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint8_t* kr = kc + ((slot0 + 16 * t + col) * a.Hkv + h) * D + 32 * grp;
      T.k[t][0] = *reinterpret_cast<const u32x4*>(kr);
      T.k[t][1] = *reinterpret_cast<const u32x4*>(kr + 16);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = 16 * (e >> 2) + 4 * grp + (e & 3);
      const int64_t row = (slot0 + key) * a.Hkv + h;
      T.v[e] = *reinterpret_cast<const u32x2*>(vc + row * D + 8 * col);
      T.ksc[e] = a.ks[row];
      T.vsc[e] = a.vs[row];
    }
  }
}

template <int KV>
__device__ __forceinline__ void decode_tile_compute(const DecodeTile<KV>& T, const bf16x8 (&qop)[4],
                                                    f32x4 (&o)[8], float& m_run, float& l_run,
                                                    int kt, int kend, int grp, float scale_log2) {
  // ---- S^T = K . Q^T -------------------------------------------------------
  f32x4 s[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      bf16x8 kop;
      if constexpr (KV == NVS_DTYPE_BF16) {
        kop = __builtin_bit_cast(bf16x8, T.k[t][st]);
      } else {
        const u32x4 w = T.k[t][st >> 1];
        kop = codes8_to_bf16x8<KV>(w[2 * (st & 1)], w[2 * (st & 1) + 1]);
      }
      s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[st], s[t], 0, 0, 0);
    }
  }
  // ---- online softmax (log2 domain) -----------------------------------------
  const bool partial = kt + 32 > kend;
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float f = scale_log2;
    if constexpr (KV != NVS_DTYPE_BF16) f *= T.ksc[e];
    float x = s[e >> 2][e & 3] * f;
    if (partial) {
      const int key = kt + 16 * (e >> 2) + 4 * grp + (e & 3);
      x = key < kend ? x : -INFINITY;
    }
    sv[e] = x;
  }
  float mt = sv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mt = fmaxf(mt, sv[e]);
  mt = fmaxf(mt, shfl_xor(mt, 16));
  mt = fmaxf(mt, shfl_xor(mt, 32));
  const float m_new = fmaxf(m_run, mt);
  const float alpha = fast_exp2(m_run - m_new);
  m_run = m_new;
  l_run *= alpha;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] *= alpha;
  float pv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = fast_exp2(sv[e] - m_new);
    l_run += p;
    float pw = p;
    if constexpr (KV != NVS_DTYPE_BF16) pw = (sv[e] == -INFINITY) ? 0.0f : p * T.vsc[e];
    pv[e] = pw;
  }
  u32x4 pw;
#pragma unroll
  for (int m = 0; m < 4; ++m) pw[m] = pack_bf16x2(pv[2 * m], pv[2 * m + 1]);
  const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);

  // ---- V^T operands (transpose in registers) and O^T += V^T . P^T ---------
  if constexpr (KV == NVS_DTYPE_BF16) {
    u32x4 v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = T.v[e];
    if (partial) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = kt + 16 * (e >> 2) + 4 * grp + (e & 3);
        if (key >= kend) v[e] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4 aw;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        aw[m] = __builtin_amdgcn_perm(v[2 * m + 1][j >> 1], v[2 * m][j >> 1], sel);
      o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, aw), pop, o[j], 0,
                                                     0, 0);
    }
  } else {
    u32x2 v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = T.v[e];
    if (partial) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = kt + 16 * (e >> 2) + 4 * grp + (e & 3);
        if (key >= kend) v[e] = u32x2{0, 0};
      }
    }
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {  // d pair (2jp, 2jp+1) within the lane's 8
      const int wsel = jp >> 1;        // code word holding bytes 2jp, 2jp+1
      const int b0 = (jp & 1) * 2;     // byte index of 2jp inside that word
      // bytes: [w0.b0, w1.b0, w0.b0+1, w1.b0+1]
      const uint32_t sel = (uint32_t)(b0) | ((uint32_t)(4 + b0) << 8) |
                           ((uint32_t)(b0 + 1) << 16) | ((uint32_t)(5 + b0) << 24);
      u32x4 a0, a1;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t x = __builtin_amdgcn_perm(v[2 * m + 1][wsel], v[2 * m][wsel], sel);
        a0[m] = code_pair_to_bf16x2<KV, false>(x);
        a1[m] = code_pair_to_bf16x2<KV, true>(x);
      }
      o[2 * jp] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), pop,
                                                          o[2 * jp], 0, 0, 0);
      o[2 * jp + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), pop,
                                                              o[2 * jp + 1], 0, 0, 0);
    }
  }
}

template <int KV>
__global__ __launch_bounds__(64) void paged_decode_kernel(DecodeArgs a) {
  const int p = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int q0 = a.cu_q[b];
  if (a.cu_q[b + 1] - q0 != 1 || q0 < 0 || q0 >= a.T) return;
  const int klen = a.cu_k[b + 1] - a.cu_k[b];
  const int kbeg = p * kDecodePart;
  if (kbeg >= klen) return;
  const int kend = min(kbeg + kDecodePart, klen);
  const int col = lane & 15, grp = lane >> 4;

  // Q^T as the B operand: column = head (col < g), d = 32 grp + 8 s .. +7.
  bf16x8 qop[4];
  if (col < a.g) {
    const uint16_t* qp = a.q + (int64_t)q0 * a.q_ts + (int64_t)(h * a.g + col) * a.q_hs + 32 * grp;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = *reinterpret_cast<const bf16x8*>(qp + 8 * s);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = __builtin_bit_cast(bf16x8, u32x4{0, 0, 0, 0});
  }

  f32x4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  DecodeTile<KV> ta, tb;
  decode_load<KV>(ta, a, b, h, kbeg, col, grp);
  for (int kt = kbeg; kt < kend; kt += 64) {
    const bool two = kt + 32 < kend;
    if (two) decode_load<KV>(tb, a, b, h, kt + 32, col, grp);
    decode_tile_compute<KV>(ta, qop, o, m_run, l_run, kt, kend, grp, a.scale_log2);
    if (!two) break;
    if (kt + 64 < kend) decode_load<KV>(ta, a, b, h, kt + 64, col, grp);
    decode_tile_compute<KV>(tb, qop, o, m_run, l_run, kt + 32, kend, grp, a.scale_log2);
  }
  l_run += shfl_xor(l_run, 16);
  l_run += shfl_xor(l_run, 32);

  if (col < a.g) {
    const int hq = h * a.g + col;
    // Lane (col, grp) holds O[hq][d] for d = 32 grp + 8 r + j.
    if (a.max_parts == 1) {
      // Single partition: finish here.
      const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
      uint16_t* op = a.out + (int64_t)q0 * a.out_ts + (int64_t)hq * a.out_hs + 32 * grp;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x4 w;
#pragma unroll
        for (int m = 0; m < 4; ++m) w[m] = pack_bf16x2(o[2 * m][r] * inv, o[2 * m + 1][r] * inv);
        *reinterpret_cast<u32x4*>(op + 8 * r) = w;
      }
    } else {
      const int64_t base = ((int64_t)b * a.Hq + hq) * a.max_parts + p;
      float* op = a.ws_o + base * kHeadDim + 32 * grp;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        *reinterpret_cast<f32x4*>(op + 8 * r) = f32x4{o[0][r], o[1][r], o[2][r], o[3][r]};
        *reinterpret_cast<f32x4*>(op + 8 * r + 4) = f32x4{o[4][r], o[5][r], o[6][r], o[7][r]};
      }
      if (grp == 0) {
        a.ws_ml[base * 2] = m_run;
        a.ws_ml[base * 2 + 1] = l_run;
      }
    }
  }
}

// Merge the partitions of every (decode sequence, query head).
// 64 threads, each owning 2 of the 128 head_dim elements.
__global__ __launch_bounds__(64) void decode_reduce_kernel(DecodeArgs a) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int q0 = a.cu_q[b];
  if (a.cu_q[b + 1] - q0 != 1 || q0 < 0 || q0 >= a.T) return;
  const int klen = a.cu_k[b + 1] - a.cu_k[b];
  const int parts = klen > 0 ? min((klen + kDecodePart - 1) / kDecodePart, a.max_parts) : 0;
  const int d = 2 * threadIdx.x;
  const int64_t base = ((int64_t)b * a.Hq + hq) * a.max_parts;
  float M = -INFINITY;
  for (int p = 0; p < parts; ++p) M = fmaxf(M, a.ws_ml[(base + p) * 2]);
  float L = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
  for (int p = 0; p < parts; ++p) {
    const float w = fast_exp2(a.ws_ml[(base + p) * 2] - M);
    L += w * a.ws_ml[(base + p) * 2 + 1];
    const float2 ov = *reinterpret_cast<const float2*>(a.ws_o + (base + p) * kHeadDim + d);
    acc0 += w * ov.x;
    acc1 += w * ov.y;
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  uint16_t* op = a.out + (int64_t)q0 * a.out_ts + (int64_t)hq * a.out_hs + d;
  *reinterpret_cast<uint32_t*>(op) = pack_bf16x2(acc0 * inv, acc1 * inv);
}

int64_t decode_workspace_bytes(int num_seqs, int max_seqlen_k, int num_heads) {
  const int64_t parts = decode_max_parts(max_seqlen_k);
  if (parts <= 1) return 0;
  return (int64_t)num_seqs * num_heads * parts * (kHeadDim + 2) * (int64_t)sizeof(float);
}

int launch_decode(const AttnParams& P, hipStream_t stream) {
  DecodeArgs a;
  a.q = (const uint16_t*)P.q; a.q_ts = P.q_ts; a.q_hs = P.q_hs;
  a.kc = P.kc; a.vc = P.vc; a.ks = P.ks; a.vs = P.vs;
  a.cu_q = P.cu_q; a.cu_k = P.cu_k; a.bt = P.bt; a.bt_stride = P.bt_stride; a.NB = P.NB; a.T = P.T;
  a.Hq = P.Hq; a.Hkv = P.Hkv; a.g = P.Hq / P.Hkv; a.bs = P.bs;
  a.max_parts = decode_max_parts(P.max_seqlen_k);
  a.scale_log2 = P.softmax_scale * 1.4426950408889634f;
  a.out = (uint16_t*)P.out; a.out_ts = P.out_ts; a.out_hs = P.out_hs;
  a.ws_o = nullptr; a.ws_ml = nullptr;
  if (a.max_parts > 1) {
    const int64_t need = decode_workspace_bytes(P.B, P.max_seqlen_k, P.Hq);
    NVS_REQUIRE(P.ws && P.ws_bytes >= need, NVS_ERR_WORKSPACE,
                "paged_attention: decode workspace of %lld bytes needed, %lld given",
                (long long)need, (long long)P.ws_bytes);
    a.ws_o = (float*)P.ws;
    a.ws_ml = a.ws_o + (int64_t)P.B * P.Hq * a.max_parts * kHeadDim;
  }
  dim3 grid(a.max_parts, P.Hkv, P.B), block(64);
  switch (P.cache_dtype) {
    case NVS_DTYPE_BF16:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_BF16>, grid, block, 0, stream, a);
      break;
    case NVS_DTYPE_INT8:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_INT8>, grid, block, 0, stream, a);
      break;
    case NVS_DTYPE_FP8_E4M3:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_FP8_E4M3>, grid, block, 0, stream, a);
      break;
    default:
      set_error("paged_attention: decode does not serve cache dtype %d", P.cache_dtype);
      return NVS_ERR_UNSUPPORTED;
  }
  int rc = check_launch("paged_decode");
  if (rc != NVS_OK || a.max_parts == 1) return rc;
  hipLaunchKernelGGL(decode_reduce_kernel, dim3(P.Hq, P.B), dim3(64), 0, stream, a);
  return check_launch("decode_reduce");
}

}  // namespace nvs
