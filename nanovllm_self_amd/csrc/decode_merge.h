// The decode waves' arguments and the merge of their split rows, shared by
// the decode file (the merge's own launch: decode-only calls, and calls
// whose prefill launch streamed the decode rows) and the planning kernel
// (which runs the merge beside the plan in one launch when a paged call's
// decode launch comes before prefill rows).
#pragma once

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
  int bt_stride;  // row stride == number of columns
  int NB;
  int Hq, Hkv, g, bs;
  float scale_log2;
  float* ws_o;   // [max_waves, 2 slots, g, 128]
  float* ws_ml;  // [max_waves, 2 slots, g, 2]
  int32_t* ws_rec;  // [4 + 4 waves]: (T, Kw), then per wave the split row it merges
  // New tokens (bf16) stored by the decode waves themselves: copied into a
  // bf16 cache, quantised per token and kv head into an fp8 / int8 one with
  // their scales into ks / vs (kn null: none).
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t kn_ts, kn_hs, vn_ts, vn_hs;
  const int32_t* slots;
  int64_t total_slots;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B;
  int64_t T;  // query / output rows
  uint16_t* out;
  int64_t out_ts, out_hs;
  int f16;  // q and out are fp16 (an fp16 cache), else bf16
};

// First tile of decode group k of Kw over T tiles.
__device__ __forceinline__ int group_start(int T, int Kw, int k) { return (int)((int64_t)k * T / Kw); }

// Heads c0 + lane / 16 + 4 i (i < NH) of the row: NH head passes at once,
// so a group of more than four heads waits for its partials' loads once
// rather than once per four heads.
template <int NH>
__device__ __forceinline__ void merge_heads(const DecodeArgs& a, int h, int k, int k_last, int slot_k, int q_row,
                                            int c0, int lane) {
  const int j = lane & 15;
  int cc[NH];
  bool use[NH];
  float M[NH], L[NH];
  f32x4 acc0[NH], acc1[NH];
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    const int c = c0 + (lane >> 4) + 4 * i;
    use[i] = c < a.g;
    cc[i] = use[i] ? c : 0;
    M[i] = -INFINITY;
    L[i] = 0.0f;
    acc0[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc1[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int x0 = k; x0 <= k_last; x0 += 4) {
    f32x2 ml[4][NH];
    f32x4 o0[4][NH], o1[4][NH];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int x = min(x0 + u, k_last);
#pragma unroll
      for (int i = 0; i < NH; ++i) {
        const int64_t base = (((int64_t)x * a.Hkv + h) * 2 + (x == k ? slot_k : 0)) * a.g + cc[i];
        ml[u][i] = *reinterpret_cast<const f32x2*>(a.ws_ml + base * 2);
        o0[u][i] = *reinterpret_cast<const f32x4*>(a.ws_o + base * kHeadDim + 8 * j);
        o1[u][i] = *reinterpret_cast<const f32x4*>(a.ws_o + base * kHeadDim + 8 * j + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (x0 + u > k_last) break;
#pragma unroll
      for (int i = 0; i < NH; ++i) {
        const float m_new = fmaxf(M[i], ml[u][i][0]);
        const float al = M[i] == -INFINITY ? 0.0f : fast_exp2(M[i] - m_new);
        const float be = ml[u][i][0] == -INFINITY ? 0.0f : fast_exp2(ml[u][i][0] - m_new);
        M[i] = m_new;
        L[i] = L[i] * al + ml[u][i][1] * be;
        acc0[i] = acc0[i] * al + o0[u][i] * be;
        acc1[i] = acc1[i] * al + o1[u][i] * be;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    if (!use[i]) continue;
    const float inv = L[i] > 0.0f ? 1.0f / L[i] : 0.0f;
    const f32x4 x0 = acc0[i] * inv, x1 = acc1[i] * inv;
    u32x4 v;
    if (a.f16) {
      v[0] = pack_f16x2(x0[0], x0[1]);
      v[1] = pack_f16x2(x0[2], x0[3]);
      v[2] = pack_f16x2(x1[0], x1[1]);
      v[3] = pack_f16x2(x1[2], x1[3]);
    } else {
      v[0] = pack_bf16x2(x0[0], x0[1]);
      v[1] = pack_bf16x2(x0[2], x0[3]);
      v[2] = pack_bf16x2(x1[0], x1[1]);
      v[3] = pack_bf16x2(x1[2], x1[3]);
    }
    *reinterpret_cast<u32x4*>(a.out + (int64_t)q_row * a.out_ts + (int64_t)(h * a.g + cc[i]) * a.out_hs + 8 * j) = v;
  }
}

// Log-sum-exp merge of the rows split across groups.  Wave k Hkv + h owns kv
// head h of the row recorded by decode wave k Hkv + h (the row that crosses
// the boundary after group k and starts inside group k's range); its
// partials sit in wave k Hkv + h (the recorded slot) and in waves x Hkv + h
// for groups x = k + 1 .. k_last (slot 0).  Lane l serves head 4 p + l / 16
// of the group (pass p) and head_dim elements 8 (l % 16) .. + 7; one pass
// over the partials keeps a running max, sum and output, with the loads of
// four partials in flight at a time, for up to two head passes together.
__device__ __forceinline__ void merge_split_row(const DecodeArgs& a, int unit, int lane) {
  const int k = unit / a.Hkv, h = unit - k * a.Hkv;
  // Groups k >= Kw - 1 merge nothing (a launch may hold more merge waves
  // than the decode had groups; their records are not this call's).
  const int Kw = __builtin_amdgcn_readfirstlane(a.ws_rec[1]);
  if (k >= Kw - 1) return;
  const int32_t* rec = a.ws_rec + 4 + 4 * unit;
  if (__builtin_amdgcn_readfirstlane(rec[3]) == 0) return;
  const int T = __builtin_amdgcn_readfirstlane(a.ws_rec[0]);
  const int q_row = __builtin_amdgcn_readfirstlane(rec[0]);
  const int last = group_start(T, Kw, k + 1) - 1 + __builtin_amdgcn_readfirstlane(rec[1]);  // the row's last tile
  const int k_last = (int)(((int64_t)(last + 1) * Kw - 1) / T);
  const int slot_k = __builtin_amdgcn_readfirstlane(rec[2]);
  if (a.g <= 4) {
    merge_heads<1>(a, h, k, k_last, slot_k, q_row, 0, lane);
  } else {
    for (int c0 = 0; c0 < a.g; c0 += 8) merge_heads<2>(a, h, k, k_last, slot_k, q_row, c0, lane);
  }
}

// A merge left to the plan launch: the decode launch's arguments and the
// number of merge waves ((groups - 1) x Hkv; 0: no row can be split).
struct MergeJob {
  DecodeArgs a;
  int units;
};

// Decode rows streamed by the MFMA prefill launch: their arguments and
// block tables, the cache type, the decode groups the partial workspace
// holds, and the work-groups the launch runs.
struct CoDecode {
  DecodeArgs a;
  const int32_t* bt;
  int kv;
  int groups;
  int wgs;
};

}  // namespace nvs
