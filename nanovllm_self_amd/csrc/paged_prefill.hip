// Varlen causal prefill attention (q_len > 1 rows, or every row of the
// non-paged mode) for gfx950.
//
// Reference semantics: prefill_flashattn (nanovllm/layers/attention.py:303-375)
// and prefill_torch (:378-498).  Query row r of a sequence with L new and K
// visible keys attends keys j <= r + (K - L); GQA head map hq -> hq / g;
// softmax in fp32; output rounded to bf16.  Paged mode reads K/V (prefix and
// the step's own tokens, already stored) through block_tables; quantised
// caches are dequantised as bf16(code * scale), the eager path's
// dequantize_int8_per_token rounding (:100-117).  Local mode reads the step's
// k/v rows directly (block_tables is None).
//
// Work decomposition: one 256-thread work-group per (sequence, 128-row query
// tile, query head).  Each wave owns 32 query rows.  Per 64-key tile, K
// (row-major) and V^T are staged in LDS by all four waves; then each wave
//   S^T[64 x 32] = K . Q^T         (32 x mfma_f32_16x16x32_bf16)
//   O^T[128 x 32] += V^T . P^T     (32 x mfma_f32_16x16x32_bf16)
// P^T is consumed from registers: the S^T accumulator layout equals the
// B-operand layout of the PV product.  The next tile's global loads are in
// flight while the current tile is computed.
//
// Scheduling: work-groups are dispatched longest-first (last query tiles of
// every sequence first) and the g query heads that share a kv head land on
// the same XCD so their K/V tiles are fetched into that XCD's L2 once.
#include <algorithm>

#include "nvs_common.h"
#include "attention_common.h"

namespace nvs {

constexpr int kBM = kPrefillBM;  // query rows per work item
constexpr int kBN = 64;        // keys per tile
constexpr int kKStride = 136;  // bf16 per K row in LDS (272 B: conflict-free b128 reads)
constexpr int kVStride = 68;   // bf16 per V^T row in LDS (136 B: conflict-free b64 access)

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const void* kc;
  const void* vc;
  const float* ks;
  const float* vs;
  const int32_t* bt;
  int bt_stride;      // row stride == number of columns (32-bit: scalar lookup)
  int NB;
  int64_t T;          // rows of the local k/v
  int bs;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_ts, k_hs, v_ts, v_hs;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B, Hq, Hkv, g;
  Plan plan;
  float scale_log2;
  uint16_t* out;
  int64_t out_ts, out_hs;
};

// Global-load staging of one K/V tile.
template <int KV>
struct FillRegs {
  u32x4 k[4];  // K: key tid/16 + 16 i, d chunk tid%16 (8 elements)
  u32x4 v[4];  // V: key 4 kg + e, d chunk 4 w + lane/16
};
template <>
struct FillRegs<NVS_DTYPE_INT8> {
  u32x2 k[4];
  u32x2 v[4];
  float ksc[4], vsc[4];
};
template <>
struct FillRegs<NVS_DTYPE_FP8_E4M3> {
  u32x2 k[4];
  u32x2 v[4];
  float ksc[4], vsc[4];
};

template <int KV, bool PAGED>
__device__ __forceinline__ void prefill_fill_load(FillRegs<KV>& R, const PrefillArgs& a, int b,
                                                  int hkv, int k0, int K, int kt, int tid) {
  const int lane = tid & 63, w = tid >> 6;
  int64_t slot0 = 0;
  bool have = true;
  if constexpr (PAGED) {
    const int lblk = kt / a.bs;
    const int blk = lblk < a.bt_stride ? a.bt[b * a.bt_stride + lblk] : -1;
    have = blk >= 0 && blk < a.NB;  // never read outside the pool
    slot0 = (int64_t)blk * a.bs + (kt - lblk * a.bs);
  }
  // K rows
  const int kc = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = (tid >> 4) + 16 * i;
    const bool ok = have && (kt + key < K);
    if constexpr (PAGED) {
      const int64_t row = (slot0 + key) * a.Hkv + hkv;
      if constexpr (KV == NVS_DTYPE_BF16) {
        R.k[i] = ok ? *reinterpret_cast<const u32x4*>((const uint16_t*)a.kc + row * kHeadDim + 8 * kc)
                    : u32x4{0, 0, 0, 0};
      } else {
        R.k[i] = ok ? *reinterpret_cast<const u32x2*>((const uint8_t*)a.kc + row * kHeadDim + 8 * kc)
                    : u32x2{0, 0};
        R.ksc[i] = ok ? a.ks[row] : 0.0f;
      }
    } else {
      const bool in = ok && (int64_t)k0 + kt + key < a.T;
      R.k[i] = in ? *reinterpret_cast<const u32x4*>(a.k + (int64_t)(k0 + kt + key) * a.k_ts +
                                                    (int64_t)hkv * a.k_hs + 8 * kc)
                  : u32x4{0, 0, 0, 0};
    }
  }
  // V rows
  const int kg = lane & 15, vc = 4 * w + (lane >> 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int key = 4 * kg + e;
    const bool ok = have && (kt + key < K);
    if constexpr (PAGED) {
      const int64_t row = (slot0 + key) * a.Hkv + hkv;
      if constexpr (KV == NVS_DTYPE_BF16) {
        R.v[e] = ok ? *reinterpret_cast<const u32x4*>((const uint16_t*)a.vc + row * kHeadDim + 8 * vc)
                    : u32x4{0, 0, 0, 0};
      } else {
        R.v[e] = ok ? *reinterpret_cast<const u32x2*>((const uint8_t*)a.vc + row * kHeadDim + 8 * vc)
                    : u32x2{0, 0};
        R.vsc[e] = ok ? a.vs[row] : 0.0f;
      }
    } else {
      const bool in = ok && (int64_t)k0 + kt + key < a.T;
      R.v[e] = in ? *reinterpret_cast<const u32x4*>(a.v + (int64_t)(k0 + kt + key) * a.v_ts +
                                                    (int64_t)hkv * a.v_hs + 8 * vc)
                  : u32x4{0, 0, 0, 0};
    }
  }
}

// 8 codes * scale -> 8 bf16 (RNE), as bf16(code.float() * scale).
template <int KV>
__device__ __forceinline__ u32x4 dequant8_bf16(u32x2 w, float scale) {
  u32x4 r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float f0, f1, f2, f3;
    code_pair_to_f32<KV, false>(w[h], f0, f1);
    code_pair_to_f32<KV, true>(w[h], f2, f3);
    r[2 * h] = pack_bf16x2(f0 * scale, f1 * scale);
    r[2 * h + 1] = pack_bf16x2(f2 * scale, f3 * scale);
  }
  return r;
}

template <int KV>
__device__ __forceinline__ void prefill_fill_store(const FillRegs<KV>& R, uint16_t* Ks, uint16_t* Vt,
                                                   int tid) {
  const int lane = tid & 63, w = tid >> 6;
  const int kc = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = (tid >> 4) + 16 * i;
    u32x4 val;
    if constexpr (KV == NVS_DTYPE_BF16)
      val = R.k[i];
    else
      val = dequant8_bf16<KV>(R.k[i], R.ksc[i]);
    *reinterpret_cast<u32x4*>(Ks + key * kKStride + 8 * kc) = val;
  }
  const int kg = lane & 15, vc = 4 * w + (lane >> 4);
  u32x4 v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (KV == NVS_DTYPE_BF16)
      v[e] = R.v[e];
    else
      v[e] = dequant8_bf16<KV>(R.v[e], R.vsc[e]);
  }
  // 4 keys x 8 d -> 8 d-rows x 4 keys.
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    u32x2 t;
    t[0] = __builtin_amdgcn_perm(v[1][j >> 1], v[0][j >> 1], sel);
    t[1] = __builtin_amdgcn_perm(v[3][j >> 1], v[2][j >> 1], sel);
    *reinterpret_cast<u32x2*>(Vt + (8 * vc + j) * kVStride + 4 * kg) = t;
  }
}

// One work item: (sequence b, query tile qt, query head hkv * g + cg).  Every
// thread of the work-group runs the same items, so the barriers inside match.
template <int KV, bool PAGED>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, int b, int qt, int hkv, int cg,
                                             uint16_t* Ks, uint16_t* Vt) {
  const int hq = hkv * a.g + cg;
  const int q0 = a.cu_q[b];
  const int L = a.cu_q[b + 1] - q0;
  const int m0 = qt * kBM;
  if (m0 >= L) return;
  const int k0 = a.cu_k[b];
  const int K = a.cu_k[b + 1] - k0;
  const int off = K - L;
  const int kv_end = min(K, m0 + kBM + off);
  const int ntiles = kv_end > 0 ? (kv_end + kBN - 1) / kBN : 0;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int wrow0 = m0 + 32 * w;  // first query row of this wave
  const bool wave_active = wrow0 < L;
  const int wave_last_key = min(K - 1, wrow0 + 31 + off);

  // Q^T operands: column = query row wrow0 + 16 c + col, d = 32 grp + 8 s.
  bf16x8 qop[2][4];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int row = wrow0 + 16 * c + col;
    if (row < L) {
      const uint16_t* qp = a.q + (int64_t)(q0 + row) * a.q_ts + (int64_t)hq * a.q_hs + 32 * grp;
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[c][s] = *reinterpret_cast<const bf16x8*>(qp + 8 * s);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) qop[c][s] = __builtin_bit_cast(bf16x8, u32x4{0, 0, 0, 0});
    }
  }

  f32x4 o[8][2];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n][0] = o[n][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  FillRegs<KV> R;
  if (ntiles > 0) {
    prefill_fill_load<KV, PAGED>(R, a, b, hkv, k0, K, 0, tid);
    prefill_fill_store<KV>(R, Ks, Vt, tid);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int kt = it * kBN;
    const bool more = it + 1 < ntiles;
    if (more) prefill_fill_load<KV, PAGED>(R, a, b, hkv, k0, K, kt + kBN, tid);

    if (wave_active && kt <= wave_last_key) {
      // ---- S^T = K . Q^T --------------------------------------------------
      f32x4 sacc[4][2];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        sacc[t][0] = sacc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8 kop =
              *reinterpret_cast<const bf16x8*>(Ks + (16 * t + col) * kKStride + 32 * grp + 8 * s);
          sacc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[0][s], sacc[t][0], 0, 0, 0);
          sacc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop[1][s], sacc[t][1], 0, 0, 0);
        }
      }
      // ---- online softmax per query row (lane column) --------------------
      const bool need_mask = kt + kBN - 1 > wrow0 + off;
      bf16x8 pop[2][2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int lim = wrow0 + 16 * c + col + off;  // last visible key of this row
        float sv[16];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float x = sacc[t][c][r] * a.scale_log2;
            if (need_mask) {
              const int key = kt + 16 * t + 4 * grp + r;
              x = key <= lim ? x : -INFINITY;
            }
            sv[4 * t + r] = x;
          }
        float mt = sv[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mt = fmaxf(mt, sv[e]);
        mt = fmaxf(mt, shfl_xor(mt, 16));
        mt = fmaxf(mt, shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run[c], mt);
        const float m_safe = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = fast_exp2(m_run[c] - m_safe);
        m_run[c] = m_new;
        l_run[c] *= alpha;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[n][c] *= alpha;
        float pv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          pv[e] = fast_exp2(sv[e] - m_safe);
          l_run[c] += pv[e];
        }
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
          u32x4 pw;
          pw[0] = pack_bf16x2(pv[8 * uu + 0], pv[8 * uu + 1]);
          pw[1] = pack_bf16x2(pv[8 * uu + 2], pv[8 * uu + 3]);
          pw[2] = pack_bf16x2(pv[8 * uu + 4], pv[8 * uu + 5]);
          pw[3] = pack_bf16x2(pv[8 * uu + 6], pv[8 * uu + 7]);
          pop[c][uu] = __builtin_bit_cast(bf16x8, pw);
        }
      }
      // ---- O^T += V^T . P^T ----------------------------------------------
#pragma unroll
      for (int n = 0; n < 8; ++n) {
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
          const uint16_t* vr = Vt + (16 * n + col) * kVStride + 32 * uu + 4 * grp;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vr);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vr + 16);
          const bf16x8 vop = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
          o[n][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[0][uu], o[n][0], 0, 0, 0);
          o[n][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop[1][uu], o[n][1], 0, 0, 0);
        }
      }
    }
    __syncthreads();
    if (more) {
      prefill_fill_store<KV>(R, Ks, Vt, tid);
      __syncthreads();
    }
  }

  if (!wave_active) return;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float l = l_run[c];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int row = wrow0 + 16 * c + col;
    if (row < L) {
      uint16_t* op = a.out + (int64_t)(q0 + row) * a.out_ts + (int64_t)hq * a.out_hs + 4 * grp;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        u32x2 wv;
        wv[0] = pack_bf16x2(o[n][c][0] * inv, o[n][c][1] * inv);
        wv[1] = pack_bf16x2(o[n][c][2] * inv, o[n][c][3] * inv);
        *reinterpret_cast<u32x2*>(op + 16 * n) = wv;
      }
    }
  }
}

// Persistent, dynamically scheduled: work k maps to (unit u, head-in-group
// c) with u = (list index, kv head); work with k % 8 == x is claimed from XCD
// x's counter by the work-groups on XCD x (work-group i runs on XCD i % 8), so
// the g query heads of a unit run on one XCD and fetch its K/V tiles into that
// XCD's L2 once, and each XCD's work-groups take the heaviest remaining work
// first.  The next claim is made while the current item runs.
template <int KV, bool PAGED>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kHeadDim * kVStride];
  __shared__ int s_claim[2];
  const int units = a.plan.hdr->n_prefill * a.Hkv;
  const int total = ((units + 7) / 8) * 8 * a.g;
  const int xcd = blockIdx.x & 7;
  int* counter = a.plan.hdr->prefill_next + xcd;
  if (threadIdx.x == 0) s_claim[0] = atomicAdd(counter, 1);
  __syncthreads();
  for (int it = 0;; ++it) {
    const int c = s_claim[it & 1];
    const int k = 8 * c + xcd;
    if (k >= total) break;
    int next = 0;
    if (threadIdx.x == 0) next = atomicAdd(counter, 1);
    const int cg = c % a.g;
    const int u = 8 * (c / a.g) + xcd;
    if (u < units) {
      const int idx = u / a.Hkv;
      const int hkv = u - idx * a.Hkv;
      const int item = __builtin_amdgcn_readfirstlane(a.plan.plist[idx]);
      const int b = item / a.plan.ntq;
      prefill_item<KV, PAGED>(a, b, item - b * a.plan.ntq, hkv, cg, Ks, Vt);
    }
    // The claim slot read next iteration was last read two iterations ago,
    // before the barrier below.
    if (threadIdx.x == 0) s_claim[(it + 1) & 1] = next;
    __syncthreads();
  }
}

int launch_prefill(const AttnParams& P, const Plan& plan, hipStream_t stream) {
  PrefillArgs a;
  a.q = (const uint16_t*)P.q; a.q_ts = P.q_ts; a.q_hs = P.q_hs;
  a.kc = P.kc; a.vc = P.vc; a.ks = P.ks; a.vs = P.vs;
  a.bt = P.bt; a.bt_stride = (int)P.bt_stride; a.bs = P.bs; a.NB = (int)P.NB; a.T = P.T;
  a.k = (const uint16_t*)P.k; a.v = (const uint16_t*)P.v;
  a.k_ts = P.k_ts; a.k_hs = P.k_hs; a.v_ts = P.v_ts; a.v_hs = P.v_hs;
  a.cu_q = P.cu_q; a.cu_k = P.cu_k;
  a.B = P.B; a.Hq = P.Hq; a.Hkv = P.Hkv; a.g = P.Hq / P.Hkv;
  a.plan = plan;
  a.scale_log2 = P.softmax_scale * 1.4426950408889634f;
  a.out = (uint16_t*)P.out; a.out_ts = P.out_ts; a.out_hs = P.out_hs;
  if (plan.ntq <= 0 || P.B <= 0) return NVS_OK;
  // One work-group per CU (a multiple of 8), never more than the work there can be.
  const int64_t upper = (((int64_t)P.B * plan.ntq * P.Hkv + 7) / 8) * 8 * a.g;
  int64_t wgs = std::min<int64_t>(upper, (int64_t)device_slots(1));
  wgs = std::max<int64_t>(8, wgs & ~(int64_t)7);
  dim3 grid((unsigned)wgs), block(256);
  const bool paged = P.bt != nullptr;
  if (!paged) {
    hipLaunchKernelGGL((prefill_kernel<NVS_DTYPE_BF16, false>), grid, block, 0, stream, a);
  } else {
    switch (P.cache_dtype) {
      case NVS_DTYPE_BF16:
        hipLaunchKernelGGL((prefill_kernel<NVS_DTYPE_BF16, true>), grid, block, 0, stream, a);
        break;
      case NVS_DTYPE_INT8:
        hipLaunchKernelGGL((prefill_kernel<NVS_DTYPE_INT8, true>), grid, block, 0, stream, a);
        break;
      case NVS_DTYPE_FP8_E4M3:
        hipLaunchKernelGGL((prefill_kernel<NVS_DTYPE_FP8_E4M3, true>), grid, block, 0, stream, a);
        break;
      default:
        set_error("paged_attention: prefill does not serve cache dtype %d", P.cache_dtype);
        return NVS_ERR_UNSUPPORTED;
    }
  }
  return check_launch("prefill");
}

}  // namespace nvs
