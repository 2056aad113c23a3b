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
// Work decomposition: one 512-thread work-group (8 waves, two per SIMD) per
// (sequence, tile of query positions, kv head, group of up to 8 query heads).
// Each wave owns 32 query positions of one query head, so the g heads that
// share a kv head share every K/V tile the work-group stages.  Per 64-key
// tile, K and V are staged row-major in LDS (double-buffered: the next tile's
// global loads are in flight during the current tile, one barrier per tile)
// and each wave computes, with v_mfma_f32_32x32x16_bf16,
//   S^T[64 keys x 32 q] = K . Q^T      (16 MFMAs; Q^T stays in registers)
//   O^T[128 d x 32 q] += V^T . P^T     (16 MFMAs)
// The S^T accumulator layout (lane = query column, keys along registers) is
// the B-operand layout of P^T, so P never leaves registers; the V^T operand
// is read from the row-major V tile with ds_read_b64_tr_b16, which transposes
// 4 x 16 bf16 blocks across each 16-lane group.  One query per lane makes the
// row max a single cross-lane exchange.  Two waves per SIMD let one wave's
// softmax run under the other's MFMAs.
//
// LDS tiles are row-major with 16-byte chunks XOR-swizzled per key
// (chunk ^ swz(key)): both the K reads (16 keys x one chunk per 16 lanes)
// and the transposed V reads (4 keys x 4 chunks per 16 lanes) hit 16
// distinct 16-byte bank groups.
#include <algorithm>

#include "nvs_common.h"
#include "attention_common.h"

namespace nvs {

constexpr int kWaves = kPrefillWaves;  // 8
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = kPrefillWaveRows;  // query positions per wave
constexpr int kBN = 64;                  // keys per tile
constexpr int kTile = kBN * kHeadDim;    // bf16 elements of one K (or V) tile
constexpr int kBlockWindow = 512;        // block-table entries staged in LDS at a time

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const void* kc;
  const void* vc;
  const float* ks;
  const float* vs;
  const int32_t* bt;
  int bt_stride;  // row stride == number of columns
  int NB;
  int64_t T;  // rows of the local k/v (clamp bound of their reads)
  int bs;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_ts, k_hs, v_ts, v_hs;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B, Hq, Hkv, g;
  int hpw, nblk, hgroups;  // heads per item, position blocks per item, head groups per kv head
  Plan plan;
  float scale_log2;
  uint16_t* out;
  int64_t out_ts, out_hs;
  const int* gate;  // run only where *gate == gate_run (null: always)
  int gate_run;
};

// 16-byte chunk swizzle of key row `key`: a bijection of key % 16 that maps
// 4 consecutive keys to 4 different chunk quads.
__device__ __forceinline__ int swz(int key) { return ((key & 3) << 2) | ((key >> 2) & 3); }
// Element offset of (key, d) in a swizzled tile (d a multiple of 4).
__device__ __forceinline__ int tile_at(int key, int d) {
  return key * kHeadDim + (((d >> 3) ^ swz(key)) << 3) + (d & 7);
}

// ---------------------------------------------------------------------------
// Tile fill: global -> registers (issued at the start of an iteration) ->
// swizzled LDS (stored at its end).  K and V tiles are filled separately:
// their LDS lifetimes are offset by two tiles.  bf16: thread t owns 16-byte
// chunk t % 16 of key rows t / 16 and t / 16 + 32; codes: thread t owns 16
// codes (d = 16 (t % 8) ..) of key row t / 8.  Rows past the sequence or in
// a missing block are stored as zeros.
// ---------------------------------------------------------------------------
template <int KV>
struct Half {
  u32x4 x;
  float sc;
  bool ok;  // row holds a visible key (else stored as zeros)
};
template <>
struct Half<NVS_DTYPE_BF16> {
  u32x4 x[2];
  bool ok[2];
};

struct ItemKV {
  int b, hkv, k0, K;
  int win0;  // first logical block staged in blk_lds
};

// Loads are issued unconditionally from in-bounds addresses (a missing block
// reads block 0, a row outside the local k/v reads its first or last row) and
// replaced by zeros when stored: with no load behind a branch and no use of
// the loaded values before the store, the compiler's wait counts stay exact
// and the compute never waits for a later tile's loads.
template <int KV, bool PAGED, bool ISV>
__device__ __forceinline__ void half_load(Half<KV>& F, const PrefillArgs& a, const ItemKV& it, int kt,
                                          const int* blk_lds) {
  const int tid = threadIdx.x;
  int64_t slot0 = 0;
  bool have = true;
  if constexpr (PAGED) {
    const int lblk = kt / a.bs;  // a 64-key tile never spans two blocks (bs % 64 == 0)
    const int blk = blk_lds[lblk - it.win0];
    have = blk >= 0;
    slot0 = (int64_t)(have ? blk : 0) * a.bs + (kt - lblk * a.bs);
  }
  if constexpr (KV == NVS_DTYPE_BF16) {
    const int c = tid & 15;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = (tid >> 4) + 32 * i;
      F.ok[i] = have && kt + key < it.K;
      if constexpr (PAGED) {
        const int64_t row = (slot0 + key) * a.Hkv + it.hkv;
        const uint16_t* src = (const uint16_t*)(ISV ? a.vc : a.kc);
        F.x[i] = *reinterpret_cast<const u32x4*>(src + row * kHeadDim + 8 * c);
      } else {
        const int64_t row = max((int64_t)0, min((int64_t)it.k0 + kt + key, a.T - 1));
        const uint16_t* src = ISV ? a.v + row * a.v_ts + (int64_t)it.hkv * a.v_hs
                                  : a.k + row * a.k_ts + (int64_t)it.hkv * a.k_hs;
        F.x[i] = *reinterpret_cast<const u32x4*>(src + 8 * c);
      }
    }
  } else {
    const int key = tid >> 3, c = tid & 7;
    F.ok = have && kt + key < it.K;
    const int64_t row = (slot0 + key) * a.Hkv + it.hkv;
    const uint8_t* src = (const uint8_t*)(ISV ? a.vc : a.kc);
    F.x = *reinterpret_cast<const u32x4*>(src + row * kHeadDim + 16 * c);
    F.sc = (ISV ? a.vs : a.ks)[row];
  }
}

// 8 codes * scale -> 8 bf16 (RNE), as bf16(code.float() * scale).
template <int KV>
__device__ __forceinline__ u32x4 dequant8_bf16(uint32_t w0, uint32_t w1, float scale) {
  u32x4 r;
  float f0, f1, f2, f3;
  code_pair_to_f32<KV, false>(w0, f0, f1);
  code_pair_to_f32<KV, true>(w0, f2, f3);
  r[0] = pack_bf16x2(f0 * scale, f1 * scale);
  r[1] = pack_bf16x2(f2 * scale, f3 * scale);
  code_pair_to_f32<KV, false>(w1, f0, f1);
  code_pair_to_f32<KV, true>(w1, f2, f3);
  r[2] = pack_bf16x2(f0 * scale, f1 * scale);
  r[3] = pack_bf16x2(f2 * scale, f3 * scale);
  return r;
}

template <int KV>
__device__ __forceinline__ void half_store(const Half<KV>& F, uint16_t* S) {
  const int tid = threadIdx.x;
  const u32x4 zero = {0, 0, 0, 0};
  if constexpr (KV == NVS_DTYPE_BF16) {
    const int c = tid & 15;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int key = (tid >> 4) + 32 * i;
      *reinterpret_cast<u32x4*>(S + tile_at(key, 8 * c)) = F.ok[i] ? F.x[i] : zero;
    }
  } else {
    const int key = tid >> 3, c = tid & 7;
    const u32x4 x = F.ok ? F.x : zero;
    const float sc = F.ok ? F.sc : 0.0f;
    *reinterpret_cast<u32x4*>(S + tile_at(key, 16 * c)) = dequant8_bf16<KV>(x[0], x[1], sc);
    *reinterpret_cast<u32x4*>(S + tile_at(key, 16 * c + 8)) = dequant8_bf16<KV>(x[2], x[3], sc);
  }
}

// Block ids of logical blocks [win0, win0 + kBlockWindow) of sequence b, -1
// where the table has none, the block is outside the pool or past the keys
// the item reads.
__device__ __forceinline__ void load_block_window(const PrefillArgs& a, int b, int win0, int kv_end,
                                                  int* blk_lds) {
  for (int i = threadIdx.x; i < kBlockWindow; i += kThreads) {
    const int lb = win0 + i;
    int blk = -1;
    if ((int64_t)lb * a.bs < kv_end && lb < a.bt_stride) blk = a.bt[(int64_t)b * a.bt_stride + lb];
    blk_lds[i] = (blk >= 0 && blk < a.NB) ? blk : -1;
  }
}

// ---------------------------------------------------------------------------
// One wave's 32 query positions against 64-key tiles.
// Lane (qc = lane % 32, h = lane / 32).  S^T accumulator t, register v holds
// key 32 t + 8 (v / 4) + 4 h + v % 4 for query qc; O^T accumulator n,
// register v holds d = 32 n + 8 (v / 4) + 4 h + v % 4.
// ---------------------------------------------------------------------------
constexpr float kLazyRescale = 8.0f;  // log2 units; p stays below 2^8

// S^T = K . Q^T (16 MFMAs).
__device__ __forceinline__ void qk_tile(const uint16_t* Ks, const bf16x8 (&qop)[8], f32x16 (&s)[2]) {
  const int lane = threadIdx.x & 63;
  const int qc = lane & 31, h = lane >> 5;
  const int ksw = swz(qc);  // swz(32 t + qc) == swz(qc)
  s[0] = f32x16{};
  s[1] = f32x16{};
#pragma unroll
  for (int st = 0; st < 8; ++st) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bf16x8 kop =
          *reinterpret_cast<const bf16x8*>(Ks + (32 * t + qc) * kHeadDim + (((2 * st + h) ^ ksw) << 3));
      s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qop[st], s[t], 0, 0, 0);
    }
  }
}

// O^T += V^T . P^T (16 MFMAs, 16 keys each).  P^T slice m = keys 16m + 4h +
// 0..3 and 16m + 8 + 4h + 0..3 (registers 8 (m % 2) .. + 7 of S^T accumulator
// m / 2).  Its V^T operand at d = 32n + lane % 32 takes two transposing
// reads: lane (r, c) of a 16-lane group supplies key 16m + 4h + r (+ 8),
// d = 32n + 16 (lane / 16 % 2) + 4c.
__device__ __forceinline__ void pv_tile(const uint16_t* Vs, const u32x4 (&pw)[4], f32x16 (&o)[4]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, r = (lane >> 2) & 3, c = lane & 3;
  const int dq = 16 * ((lane >> 4) & 1) + 4 * c;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const bf16x8 pop = __builtin_bit_cast(bf16x8, pw[m]);
    const int key0 = 16 * m + 4 * h + r;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (i16x4 __attribute__((address_space(3)))*)(Vs + tile_at(key0, 32 * n + dq)));
      const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (i16x4 __attribute__((address_space(3)))*)(Vs + tile_at(key0 + 8, 32 * n + dq)));
      const i16x8 vv = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      o[n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vv), pop, o[n], 0, 0, 0);
    }
  }
}

// One pipelined step of a wave (iteration j of the tile loop):
//   block 1: O += V_{j-1}^T P_{j-1}^T (PV) beside the row max of S_j (SM);
//   then the lazy rescale of O and l when the max moved;
//   block 2: S_{j+1} = K_{j+1} Q^T (QK) beside P_j = 2^(S_j scale - m) (SM).
// Each block's MFMAs and VALU work are independent, so they overlap.
// MASK: tile j crosses the wave's causal diagonal; key kt + k is visible to
// this lane's query when k <= rel + 4 h (rel = last visible key - kt - 4 h,
// so the per-register key offsets are compile-time constants).
// Scores are scaled inside the exponent: with softmax_scale > 0 the row max
// of the raw scores scaled is the max of the scaled scores, and
// p = 2^(s * scale_log2 - m) is one v_fma + one v_exp.  The row sum adds the
// bf16-rounded p, the values the MFMA multiplies.
template <bool MASK, bool PV, bool QK, bool SM>
__device__ __forceinline__ void step(const uint16_t* Vp, const uint16_t* Kn, const bf16x8 (&qop)[8],
                                     f32x16 (&sc)[2], f32x16 (&sn)[2], u32x4 (&pw)[4], f32x16 (&o)[4],
                                     float& m_run, float& l_run, int rel, float scale_log2) {
  if constexpr (PV) pv_tile(Vp, pw, o);
  if constexpr (SM) {
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        if constexpr (MASK) {
          const int k = 32 * t + 8 * (v >> 2) + (v & 3);  // key - kt - 4 h
          sc[t][v] = k <= rel ? sc[t][v] : -INFINITY;
        }
        mx = fmaxf(mx, sc[t][v]);
      }
    mx = fmaxf(mx, shfl_xor(mx, 32)) * scale_log2;
    if (__any(mx > m_run + kLazyRescale)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.0f : m_new));
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < 4; ++n) o[n] *= alpha;
    }
  }
  if constexpr (QK) qk_tile(Kn, qop, sn);
  if constexpr (SM) {
    const float nms = m_run == -INFINITY ? 0.0f : -m_run;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int t = m >> 1, v0 = 8 * (m & 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pw[m][e] = pack_bf16x2(fast_exp2(fmaf(sc[t][v0 + 2 * e], scale_log2, nms)),
                               fast_exp2(fmaf(sc[t][v0 + 2 * e + 1], scale_log2, nms)));
        l_run = add_bf16x2(pw[m][e], l_run);
      }
    }
  }
}

// Iteration j of a wave whose last tile with a visible key is lt (-1: none).
__device__ __forceinline__ void wave_iteration(int j, int lt, bool mask, const uint16_t* Vp, const uint16_t* Kn,
                                               const bf16x8 (&qop)[8], f32x16 (&sc)[2], f32x16 (&sn)[2],
                                               u32x4 (&pw)[4], f32x16 (&o)[4], float& m_run, float& l_run,
                                               int rel, float scale_log2) {
  const bool pv = j >= 1 && j - 1 <= lt, qk = j + 1 <= lt, sm = j <= lt;
#define NVS_STEP(M, P, Q, S) step<M, P, Q, S>(Vp, Kn, qop, sc, sn, pw, o, m_run, l_run, rel, scale_log2)
  if (pv && qk && sm) {
    if (mask) NVS_STEP(true, true, true, true); else NVS_STEP(false, true, true, true);
  } else if (sm) {
    if (pv) {
      if (mask) NVS_STEP(true, true, false, true); else NVS_STEP(false, true, false, true);
    } else if (qk) {
      if (mask) NVS_STEP(true, false, true, true); else NVS_STEP(false, false, true, true);
    } else {
      if (mask) NVS_STEP(true, false, false, true); else NVS_STEP(false, false, false, true);
    }
  } else if (pv) {
    NVS_STEP(false, true, false, false);
  }
#undef NVS_STEP
}

// One work item: (sequence b, position tile qt, kv head hkv, head group hg).
// Every thread of the work-group runs the same items and iterations, so the
// barriers match.
//
// Software pipeline over 64-key tiles, one barrier per iteration.
// Iteration j reads V_{j-1} (Vbuf[(j-1) % 2]) and K_{j+1} (Kbuf[(j+1) % 2]);
// its fill loads K_{j+2} and V_j at the start and stores them into Kbuf[j % 2]
// and Vbuf[j % 2] at the end, buffers whose tiles (K_j, V_{j-2}) were last
// read in iteration j - 1, before the previous barrier.
template <int KV, bool PAGED>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, int b, int qt, int hkv, int hg,
                                             uint16_t* lds, int* blk_lds) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int qc = lane & 31, h = lane >> 5;
  const int q0 = a.cu_q[b];
  const int L = a.cu_q[b + 1] - q0;
  const int p0 = qt * a.plan.pbm;
  if (p0 >= L) return;
  ItemKV it;
  it.b = b;
  it.hkv = hkv;
  it.k0 = a.cu_k[b];
  it.K = a.cu_k[b + 1] - it.k0;
  it.win0 = 0;
  const int off = it.K - L;
  const int p_last = min(L, p0 + a.plan.pbm) - 1;
  const int kv_end = min(it.K, p_last + off + 1);
  const int ntiles = kv_end > 0 ? (kv_end + kBN - 1) / kBN : 0;

  const int hsub = w % a.hpw, pblk = w / a.hpw;
  const int hin = hg * kWaves + hsub;
  const int hq = hkv * a.g + hin;
  const int wp0 = p0 + kRows * pblk;
  const bool wave_active = pblk < a.nblk && hin < a.g && wp0 < L;
  const int my_p = wp0 + qc;
  const int wave_last_key = min(it.K - 1, min(L - 1, wp0 + kRows - 1) + off);
  // Last tile with a key visible to this wave (-1: none).
  const int lt = (wave_active && wave_last_key >= 0) ? wave_last_key / kBN : -1;

  // Q^T operand: column = query position my_p, d = 16 s + 8 h + 0..7 (read
  // unconditionally from a clamped row and head, then zeroed if unused).
  bf16x8 qop[8];
  {
    const bool qok = wave_active && my_p < L;
    const uint16_t* qp = a.q + (int64_t)(q0 + min(my_p, L - 1)) * a.q_ts +
                         (int64_t)min(hq, a.Hq - 1) * a.q_hs + 8 * h;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(qp + 16 * st);
      qop[st] = __builtin_bit_cast(bf16x8, qok ? x : u32x4{0, 0, 0, 0});
    }
  }
  f32x16 o[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) o[n] = f32x16{};
  float m_run = -INFINITY, l_run = 0.0f;
  f32x16 s0[2], s1[2];
  u32x4 pw[4];

  uint16_t* const Kb = lds;              // Kbuf[2]
  uint16_t* const Vb = lds + 2 * kTile;  // Vbuf[2]
  // Fill tiles are clamped to the item's last tile, so every iteration issues
  // the same loads and stores; a clamped tile lands in a buffer that is not
  // read again.
  const int last_kt = max(ntiles - 1, 0) * kBN;
  if constexpr (PAGED) load_block_window(a, b, 0, kv_end, blk_lds);
  __syncthreads();
  Half<KV> FK, FV;
  half_load<KV, PAGED, false>(FK, a, it, 0, blk_lds);  // all zeros when there is no key
  half_load<KV, PAGED, false>(FV, a, it, min(kBN, last_kt), blk_lds);
  half_store<KV>(FK, Kb);
  half_store<KV>(FV, Kb + kTile);
  __syncthreads();
  if (lt >= 0) qk_tile(Kb, qop, s0);
  __syncthreads();

  // One iteration; S_j lives in sc, S_{j+1} is produced into sn.
  auto iteration = [&](int j, f32x16(&sc)[2], f32x16(&sn)[2]) {
    if constexpr (PAGED) {
      if (j + 2 < ntiles && ((j + 2) * kBN) / a.bs >= it.win0 + kBlockWindow) {
        // Every read of the old window happened before the last barrier.
        it.win0 = (j * kBN) / a.bs;
        load_block_window(a, b, it.win0, kv_end, blk_lds);
        __syncthreads();
      }
    }
    half_load<KV, PAGED, false>(FK, a, it, min((j + 2) * kBN, last_kt), blk_lds);
    half_load<KV, PAGED, true>(FV, a, it, min(j * kBN, last_kt), blk_lds);
    const int kt = j * kBN;
    const bool mask = kt + kBN - 1 > wp0 + off;  // tile j crosses the wave's diagonal
    wave_iteration(j, lt, mask, Vb + ((j - 1) & 1) * kTile, Kb + ((j + 1) & 1) * kTile, qop, sc, sn, pw, o,
                   m_run, l_run, my_p + off - kt - 4 * h, a.scale_log2);
    half_store<KV>(FK, Kb + (j & 1) * kTile);
    half_store<KV>(FV, Vb + (j & 1) * kTile);
    __syncthreads();
  };
  for (int j = 0; j <= ntiles; j += 2) {
    iteration(j, s0, s1);
    if (j + 1 > ntiles) break;
    iteration(j + 1, s1, s0);
  }

  if (!wave_active) return;
  const float l = l_run + shfl_xor(l_run, 32);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (my_p < L) {
    uint16_t* op = a.out + (int64_t)(q0 + my_p) * a.out_ts + (int64_t)hq * a.out_hs + 4 * h;
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        u32x2 wv;
        wv[0] = pack_bf16x2(o[n][4 * jj] * inv, o[n][4 * jj + 1] * inv);
        wv[1] = pack_bf16x2(o[n][4 * jj + 2] * inv, o[n][4 * jj + 3] * inv);
        *reinterpret_cast<u32x2*>(op + 32 * n + 8 * jj) = wv;
      }
  }
}

// Persistent, dynamically scheduled: unit u = (list entry, kv head, head
// group); units with u % 8 == x are claimed from XCD x's counter by the
// work-groups running on XCD x (work-group i runs on XCD i % 8), heaviest
// remaining first.  The next claim is made while the current item runs.
template <int KV, bool PAGED>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * kTile];  // Kbuf[2], Vbuf[2]
  __shared__ int blk_lds[kBlockWindow];
  __shared__ int s_claim[2];
  if (a.gate && *a.gate != a.gate_run) return;  // the other prefill kernel serves this call
  const int per_entry = a.Hkv * a.hgroups;
  const int units = a.plan.hdr->n_prefill * per_entry;
  const int xcd = blockIdx.x & 7;
  int* counter = a.plan.hdr->prefill_next + xcd;
  if (threadIdx.x == 0) s_claim[0] = atomicAdd(counter, 1);
  __syncthreads();
  for (int it = 0;; ++it) {
    const int u = 8 * s_claim[it & 1] + xcd;
    if (u >= units) break;
    int next = 0;
    if (threadIdx.x == 0) next = atomicAdd(counter, 1);
    const int idx = u / per_entry;
    const int rem = u - idx * per_entry;
    const int hkv = rem / a.hgroups;
    const int hg = rem - hkv * a.hgroups;
    const int item = __builtin_amdgcn_readfirstlane(a.plan.plist[idx]);
    const int b = item / a.plan.ntq;
    prefill_item<KV, PAGED>(a, b, item - b * a.plan.ntq, hkv, hg, lds, blk_lds);
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
  a.bt = P.bt; a.bt_stride = (int)P.bt_stride; a.bs = P.bs; a.NB = (int)P.NB; a.T = P.Tk;
  a.k = (const uint16_t*)P.k; a.v = (const uint16_t*)P.v;
  a.k_ts = P.k_ts; a.k_hs = P.k_hs; a.v_ts = P.v_ts; a.v_hs = P.v_hs;
  a.cu_q = P.cu_q; a.cu_k = P.cu_k;
  a.B = P.B; a.Hq = P.Hq; a.Hkv = P.Hkv; a.g = P.Hq / P.Hkv;
  a.hpw = prefill_heads_per_item(a.g);
  a.nblk = kWaves / a.hpw;
  a.hgroups = prefill_head_groups(a.g);
  a.plan = plan;
  a.scale_log2 = P.softmax_scale * 1.4426950408889634f;
  a.out = (uint16_t*)P.out; a.out_ts = P.out_ts; a.out_hs = P.out_hs;
  a.gate = P.gate; a.gate_run = P.gate_run;
  if (plan.ntq <= 0 || P.B <= 0) return NVS_OK;
  if (plan.pbm != kRows * a.nblk) {
    set_error("prefill: plan tile of %d positions does not match %d heads per kv head", plan.pbm, a.g);
    return NVS_ERR_INVALID;
  }
  // One work-group per CU (a multiple of 8), never more than the work there can be.
  const int64_t upper = (((int64_t)P.B * plan.ntq * P.Hkv * a.hgroups + 7) / 8) * 8;
  int64_t wgs = std::min<int64_t>(upper, (int64_t)device_slots(1));
  wgs = std::max<int64_t>(8, wgs & ~(int64_t)7);
  dim3 grid((unsigned)wgs), block(kThreads);
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
