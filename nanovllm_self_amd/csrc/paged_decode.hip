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
// merges the partitions with a log-sum-exp (a second launch: the kernel
// boundary makes the partials visible across XCDs without device-scope
// fences, which on a multi-XCD part write back the L2).
#include <algorithm>

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
  int bt_stride;  // row stride == number of columns (32-bit: keeps the
  int NB;         // block-table lookup a scalar compare + scalar load)
  int64_t T;      // query / output rows
  int Hq, Hkv, g, bs;
  int max_parts;
  float scale_log2;
  float* ws_o;   // [B, Hq, max_parts, 128]
  float* ws_ml;  // [B, Hq, max_parts, 2]
  Plan plan;
  uint16_t* out;
  int64_t out_ts, out_hs;
};

// Registers of one 32-key tile as loaded from HBM.  `has` is false when the
// tile's block-table entry is missing (< 0 or outside the pool); the loads
// then read block 0 and the compute treats the keys as zero vectors.
template <int KV>
struct DecodeTile;

template <>
struct DecodeTile<NVS_DTYPE_BF16> {
  u32x4 k[2][4];  // [subtile t][d step s]: key 16t + col, d = 32 s + 8 grp
  u32x4 v[8];     // [slot e]: key 16(e/4) + 4 grp + e%4, d = 8 col .. +7
  bool has;
};

template <int KV>
struct DecodeTile {
  u32x4 k[2][2];  // [t][half]: 32 codes, d = 32 grp + 16 half .. +15
  u32x2 v[8];     // [e]: 8 codes, d = 8 col .. +7
  float ksc[8];   // scales of the 8 keys the lane owns (slot order)
  float vsc[8];
  bool has;
};

__device__ __forceinline__ int slot_key(int e, int grp) { return 16 * (e >> 2) + 4 * grp + (e & 3); }

// head_dim elements of MFMA step s / lane group grp in the QK^T product:
// d = kKStepStride * s + kKGroupStride * grp + 0..7.  Any split works as long
// as K and Q use the same one; bf16 K uses d = 32 s + 8 grp so that one load
// instruction reads 64 contiguous bytes of each of its 16 rows, code caches
// keep d = 32 grp + 8 s (one 128-byte row per lane group pair of loads).
template <int KV>
constexpr int kKStepStride = (KV == NVS_DTYPE_BF16) ? 32 : 8;
template <int KV>
constexpr int kKGroupStride = (KV == NVS_DTYPE_BF16) ? 8 : 32;

// Per-lane byte offsets from a tile's first row, identical for every tile:
// loads take a wave-uniform 64-bit base (scalar registers) plus these 32-bit
// lane offsets, so no per-load address arithmetic remains in the loop.
struct LaneOffsets {
  uint32_t k[2];   // key 16t + col, d = 8 grp (bf16) / 32 grp (codes)
  uint32_t v[8];   // key slot_key(e), d = 8 col
  uint32_t sc[8];  // scale of key slot_key(e)
};

template <int KV>
__device__ __forceinline__ LaneOffsets lane_offsets(int Hkv, int col, int grp) {
  constexpr uint32_t ESZ = (KV == NVS_DTYPE_BF16) ? 2 : 1;
  const uint32_t row = (uint32_t)Hkv * kHeadDim * ESZ;  // bytes per token row (all heads)
  LaneOffsets o;
#pragma unroll
  for (int t = 0; t < 2; ++t) o.k[t] = (uint32_t)(16 * t + col) * row + kKGroupStride<KV> * grp * ESZ;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o.v[e] = (uint32_t)slot_key(e, grp) * row + 8 * col * ESZ;
    o.sc[e] = (uint32_t)slot_key(e, grp) * Hkv * 4;
  }
  return o;
}

// One decode work item as the wave holds it: scalars plus the block ids of
// the partition in a vector value (a private array here would be placed in
// LDS and re-read per tile).
typedef int idxvec __attribute__((ext_vector_type(kDecodeItemBlocks)));

struct ItemRegs {
  int q0, b, p, kend;
  int lb0;      // logical block of the partition's first key
  idxvec blk;   // -1: missing block
};

// Scalars of a record from its words.
__device__ __forceinline__ ItemRegs unpack_item(const int (&w)[kDecodeItemWords], int bs) {
  ItemRegs it;
  it.q0 = w[0];
  it.b = w[1];
  it.p = w[2];
  it.kend = w[3];
  it.lb0 = it.p * kDecodePart / bs;
#pragma unroll
  for (int j = 0; j < kDecodeItemBlocks; ++j) it.blk[j] = w[4 + j];
  return it;
}

template <int KV>
__device__ __forceinline__ void decode_load(DecodeTile<KV>& T, const DecodeArgs& a, const LaneOffsets& lo,
                                            const ItemRegs& it, int h, int kt) {
  constexpr int ESZ = (KV == NVS_DTYPE_BF16) ? 2 : 1;
  const int lblk = kt / a.bs;
  const int j = lblk - it.lb0;
  int blk = it.blk[0];
#pragma unroll
  for (int i = 1; i < kDecodeItemBlocks; ++i) blk = (j == i) ? it.blk[i] : blk;
  T.has = blk >= 0;  // the plan stores -1 for missing and out-of-pool blocks
  const int64_t row0 = ((int64_t)(T.has ? blk : 0) * a.bs + (kt - lblk * a.bs)) * a.Hkv + h;
  const char* kb = (const char*)a.kc + row0 * kHeadDim * ESZ;
  const char* vb = (const char*)a.vc + row0 * kHeadDim * ESZ;
  if constexpr (KV == NVS_DTYPE_BF16) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) T.k[t][s] = *reinterpret_cast<const u32x4*>(kb + lo.k[t] + 64 * s);
#pragma unroll
    for (int e = 0; e < 8; ++e) T.v[e] = *reinterpret_cast<const u32x4*>(vb + lo.v[e]);
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      T.k[t][0] = *reinterpret_cast<const u32x4*>(kb + lo.k[t]);
      T.k[t][1] = *reinterpret_cast<const u32x4*>(kb + lo.k[t] + 16);
    }
    const char* ksb = (const char*)(a.ks + row0);
    const char* vsb = (const char*)(a.vs + row0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      T.v[e] = *reinterpret_cast<const u32x2*>(vb + lo.v[e]);
      T.ksc[e] = *reinterpret_cast<const float*>(ksb + lo.sc[e]);
      T.vsc[e] = *reinterpret_cast<const float*>(vsb + lo.sc[e]);
    }
  }
}

// A missing block reads as all-zero keys and values: clear the tile in place
// (the loads fetched block 0).
template <int KV>
__device__ __forceinline__ void zero_tile(DecodeTile<KV>& T) {
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
}

// v_perm_b32 selector bytes >= 0x0C produce 0x00: masked slots are zeroed
// inside the transpose instead of by copying registers.
__device__ __forceinline__ uint32_t masked_sel(uint32_t sel, uint32_t keep) {
  return (sel & keep) | (0x0c0c0c0cu & ~keep);
}

// The running max is only moved (and O, l rescaled) when a tile raises it by
// more than 2^kLazyRescale: until then p = 2^(s - m) stays below 2^8, which
// bf16 P and the fp32 accumulators carry exactly as well.
constexpr float kLazyRescale = 8.0f;

// MASKED: the partition's last tile; keys outside [kt, kend) are masked (score
// -inf, value slot zeroed inside the transpose so stale cache contents can
// never reach the sum).
template <int KV, bool MASKED>
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
  bool valid[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) valid[e] = !MASKED || (kt + slot_key(e, grp) < kend);
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float f = scale_log2;
    if constexpr (KV != NVS_DTYPE_BF16) f *= T.ksc[e];
    float x = s[e >> 2][e & 3] * f;
    if constexpr (MASKED) x = valid[e] ? x : -INFINITY;  // outside the partition
    sv[e] = x;
  }
  float mt = sv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mt = fmaxf(mt, sv[e]);
  mt = fmaxf(mt, shfl_xor(mt, 16));
  mt = fmaxf(mt, shfl_xor(mt, 32));
  if (__any(mt > m_run + kLazyRescale)) {
    const float m_new = fmaxf(m_run, mt);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] *= alpha;
  }
  float pv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = fast_exp2(sv[e] - m_run);
    l_run += p;
    float pw = p;
    if constexpr (KV != NVS_DTYPE_BF16) pw = p * T.vsc[e];
    if constexpr (MASKED) pw = valid[e] ? pw : 0.0f;
    pv[e] = pw;
  }
  u32x4 pw;
#pragma unroll
  for (int m = 0; m < 4; ++m) pw[m] = pack_bf16x2(pv[2 * m], pv[2 * m + 1]);
  const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);

  // ---- V^T operands (transpose in registers) and O^T += V^T . P^T ---------
  uint32_t keep[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const bool v0 = valid[2 * m], v1 = valid[2 * m + 1];
    if constexpr (KV == NVS_DTYPE_BF16)
      keep[m] = (v0 ? 0x0000ffffu : 0u) | (v1 ? 0xffff0000u : 0u);
    else
      keep[m] = (v0 ? 0x00ff00ffu : 0u) | (v1 ? 0xff00ff00u : 0u);
  }
  if constexpr (KV == NVS_DTYPE_BF16) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4 aw;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        aw[m] = __builtin_amdgcn_perm(T.v[2 * m + 1][j >> 1], T.v[2 * m][j >> 1],
                                      MASKED ? masked_sel(sel, keep[m]) : sel);
      o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, aw), pop, o[j], 0,
                                                     0, 0);
    }
  } else {
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
        const uint32_t x = __builtin_amdgcn_perm(T.v[2 * m + 1][wsel], T.v[2 * m][wsel],
                                                 MASKED ? masked_sel(sel, keep[m]) : sel);
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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v = fmaxf(v, shfl_xor(v, s));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v += shfl_xor(v, s);
  return v;
}

// One work item: (decode sequence, kv head h, partition), as planned.
template <int KV, int NBUF>
__device__ __forceinline__ void paged_decode_item(const DecodeArgs& a, const ItemRegs& it, int h) {
  const int lane = threadIdx.x;
  const int q0 = it.q0, b = it.b, p = it.p;
  const int kbeg = p * kDecodePart;
  if (kbeg >= it.kend) {
    if (p == 0 && a.max_parts == 1) {  // no visible key: output 0 (the merge handles max_parts > 1)
      for (int i = lane; i < a.g * (kHeadDim / 2); i += 64) {
        const int c = i / (kHeadDim / 2), d = 2 * (i % (kHeadDim / 2));
        *reinterpret_cast<uint32_t*>(a.out + (int64_t)q0 * a.out_ts + (int64_t)(h * a.g + c) * a.out_hs + d) = 0u;
      }
    }
    return;
  }
  const int kend = it.kend;
  const int ntiles = (kend - kbeg + 31) >> 5;
  const int col = lane & 15, grp = lane >> 4;

  // Q^T as the B operand: column = head (col < g); step s, lane group grp
  // holds the same 8 d values as the K operand: d = 32 s + 8 grp for bf16
  // caches, 32 grp + 8 s for code caches.
  bf16x8 qop[4];
  if (col < a.g) {
    const uint16_t* qp = a.q + (int64_t)q0 * a.q_ts + (int64_t)(h * a.g + col) * a.q_hs +
                         kKGroupStride<KV> * grp;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = *reinterpret_cast<const bf16x8*>(qp + kKStepStride<KV> * s);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = __builtin_bit_cast(bf16x8, u32x4{0, 0, 0, 0});
  }

  f32x4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  // Ring of NBUF tiles, fully unrolled over the partition so every buffer
  // index is a compile-time constant: NBUF - 1 tiles are in flight while one
  // is consumed.
  // The scheduling barriers keep each tile's loads in issue order: the
  // hardware's load counter retires in order, so a later tile's load hoisted
  // above an earlier one would make the wait for the earlier tile drain it too.
  // Loads are issued unconditionally (tiles past the end re-read the last
  // tile, an L2 hit) so that every path issues the same loads in the same
  // order and each wait covers exactly the tile about to be used.
  constexpr int NT = kDecodePart / 32;
  const LaneOffsets lo = lane_offsets<KV>(a.Hkv, col, grp);
  DecodeTile<KV> ring[NBUF];
  const int last = ntiles - 1;
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i) {
    decode_load<KV>(ring[i], a, lo, it, h, kbeg + 32 * min(i, last));
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    if (i + NBUF - 1 < NT)
      decode_load<KV>(ring[(i + NBUF - 1) % NBUF], a, lo, it, h, kbeg + 32 * min(i + NBUF - 1, last));
    __builtin_amdgcn_sched_barrier(0);
    if (i < last) {  // every tile but the last is full: no masking
      if (!ring[i % NBUF].has) zero_tile(ring[i % NBUF]);
      decode_tile_compute<KV, false>(ring[i % NBUF], qop, o, m_run, l_run, kbeg + 32 * i, kend, grp,
                                     a.scale_log2);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // The last tile (possibly partial) runs the masked path; its ring slot is
  // last % NBUF (later clamped loads only re-read the same tile).
#pragma unroll
  for (int r = 0; r < NBUF; ++r) {
    if (last % NBUF == r) {
      if (!ring[r].has) zero_tile(ring[r]);
      decode_tile_compute<KV, true>(ring[r], qop, o, m_run, l_run, kbeg + 32 * last, kend, grp,
                                    a.scale_log2);
    }
  }
  l_run += shfl_xor(l_run, 16);
  l_run += shfl_xor(l_run, 32);

  if (a.max_parts == 1) {
    // Single partition: normalise and write the output here.
    if (col < a.g) {
      const int hq = h * a.g + col;
      const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
      uint16_t* op = a.out + (int64_t)q0 * a.out_ts + (int64_t)hq * a.out_hs + 32 * grp;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u32x4 w;
#pragma unroll
        for (int m = 0; m < 4; ++m) w[m] = pack_bf16x2(o[2 * m][r] * inv, o[2 * m + 1][r] * inv);
        *reinterpret_cast<u32x4*>(op + 8 * r) = w;
      }
    }
    return;
  }
  // Lane (col, grp) holds O[hq][d] for d = 32 grp + 8 r + j.
  if (col < a.g) {
    const int hq = h * a.g + col;
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

// Persistent: each wave walks the plan's decode records with a grid stride,
// kv head fastest, so the Hkv waves reading one block's rows run side by
// side.  The next item's record is loaded while the current item runs: it
// comes through the scalar cache (the restrict-qualified pointer lets the
// compiler prove no store of this kernel clobbers it), so waiting for it never
// waits for this wave's vector loads or stores.
template <int KV>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kDecodeWavesPerEU)))
void paged_decode_kernel(DecodeArgs a, const int* __restrict__ rec_words) {
  const int total = a.plan.hdr->n_decode * a.Hkv;
  int k = blockIdx.x;
  if (k >= total) return;
  int w[kDecodeItemWords];
  const int* r = rec_words + (int64_t)(k / a.Hkv) * kDecodeItemWords;
#pragma unroll
  for (int i = 0; i < kDecodeItemWords; ++i) w[i] = r[i];
  for (; k < total; k += gridDim.x) {
    const int h = k % a.Hkv;
    const ItemRegs it = unpack_item(w, a.bs);
    const int kn = min(k + (int)gridDim.x, total - 1);
    r = rec_words + (int64_t)(kn / a.Hkv) * kDecodeItemWords;
#pragma unroll
    for (int i = 0; i < kDecodeItemWords; ++i) w[i] = r[i];
    paged_decode_item<KV, kDecodeBuffers>(a, it, h);
  }
}

// Log-sum-exp merge of the partitions of every (decode sequence, query
// head); one wave each.  Lane l owns head_dim elements 2l, 2l + 1.  Partition
// weights are computed lane-parallel and broadcast with a shuffle, and the
// partial-output loads are unrolled so many are in flight at once.
__global__ __launch_bounds__(64) void decode_reduce_kernel(DecodeArgs a) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const int q0 = a.cu_q[b];
  if (a.cu_q[b + 1] - q0 != 1 || q0 < 0 || q0 >= a.T) return;
  const int klen = a.cu_k[b + 1] - a.cu_k[b];
  const int parts = klen > 0 ? min((klen + kDecodePart - 1) / kDecodePart, a.max_parts) : 0;
  const int64_t base = ((int64_t)b * a.Hq + hq) * a.max_parts;
  const float* ml = a.ws_ml + base * 2;
  float M = -INFINITY;
  for (int p = lane; p < parts; p += 64) M = fmaxf(M, ml[2 * p]);
  M = wave_max(M);
  float L = 0.0f;
  for (int p = lane; p < parts; p += 64) L += fast_exp2(ml[2 * p] - M) * ml[2 * p + 1];
  L = wave_sum(L);
  const float* po = a.ws_o + base * kHeadDim + 2 * lane;
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int p0 = 0; p0 < parts; p0 += 64) {
    const int n = min(64, parts - p0);
    const float wl = lane < n ? fast_exp2(ml[2 * (p0 + lane)] - M) : 0.0f;
    int i = 0;
    for (; i + 8 <= n; i += 8) {
      float2 ov[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) ov[u] = *reinterpret_cast<const float2*>(po + (int64_t)(p0 + i + u) * kHeadDim);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float w = __shfl(wl, i + u, 64);
        acc0 += w * ov[u].x;
        acc1 += w * ov[u].y;
      }
    }
    for (; i < n; ++i) {
      const float w = __shfl(wl, i, 64);
      const float2 ov = *reinterpret_cast<const float2*>(po + (int64_t)(p0 + i) * kHeadDim);
      acc0 += w * ov.x;
      acc1 += w * ov.y;
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  uint16_t* op = a.out + (int64_t)q0 * a.out_ts + (int64_t)hq * a.out_hs + 2 * lane;
  *reinterpret_cast<uint32_t*>(op) = pack_bf16x2(acc0 * inv, acc1 * inv);
}

int64_t decode_workspace_bytes(int num_seqs, int max_seqlen_k, int num_heads) {
  const int64_t parts = decode_max_parts(max_seqlen_k);
  if (parts <= 1) return 0;
  return (int64_t)num_seqs * num_heads * parts * (kHeadDim + 2) * (int64_t)sizeof(float);
}

int launch_decode(const AttnParams& P, const Plan& plan, void* partials, hipStream_t stream) {
  DecodeArgs a;
  a.q = (const uint16_t*)P.q; a.q_ts = P.q_ts; a.q_hs = P.q_hs;
  a.kc = P.kc; a.vc = P.vc; a.ks = P.ks; a.vs = P.vs;
  a.cu_q = P.cu_q; a.cu_k = P.cu_k; a.bt = P.bt; a.bt_stride = (int)P.bt_stride; a.NB = (int)P.NB; a.T = P.T;
  a.Hq = P.Hq; a.Hkv = P.Hkv; a.g = P.Hq / P.Hkv; a.bs = P.bs;
  a.max_parts = plan.max_parts;
  a.scale_log2 = P.softmax_scale * 1.4426950408889634f;
  a.out = (uint16_t*)P.out; a.out_ts = P.out_ts; a.out_hs = P.out_hs;
  a.plan = plan;
  a.ws_o = nullptr; a.ws_ml = nullptr;
  if (a.max_parts > 1) {
    a.ws_o = (float*)partials;
    a.ws_ml = a.ws_o + (int64_t)P.B * P.Hq * a.max_parts * kHeadDim;
  }
  // One wave per SIMD slot (2 per SIMD), never more than the items that can exist.
  const int64_t upper = (int64_t)P.B * a.max_parts * P.Hkv;
  const int waves = (int)std::min<int64_t>(upper, device_slots(4 * kDecodeWavesPerEU));
  dim3 grid(waves), block(64);
  const int* words = reinterpret_cast<const int*>(plan.drec);
  switch (P.cache_dtype) {
    case NVS_DTYPE_BF16:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_BF16>, grid, block, 0, stream, a, words);
      break;
    case NVS_DTYPE_INT8:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_INT8>, grid, block, 0, stream, a, words);
      break;
    case NVS_DTYPE_FP8_E4M3:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_FP8_E4M3>, grid, block, 0, stream, a, words);
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
