// The decode wave of the split-K paged decode (q_len == 1 rows): everything
// a decode wave runs, shared by the decode kernel (one wave per work-group,
// the whole chip) and the MFMA prefill kernel, whose first work-groups
// stream a call's decode rows before they join the prefill.  The work
// decomposition, the tile formulation and the store of the step's new
// tokens are described in paged_decode.hip.
#pragma once

#include <climits>

#include "nvs_common.h"
#include "attention_common.h"
#include "store_common.h"
#include "decode_merge.h"

namespace nvs {

// Element i of a read-only input (block tables, cu_seqlens) at a
// wave-uniform index, as a scalar load: through the constant address space
// the compiler issues s_load whatever the kernel stores elsewhere.  As a
// vector load, its wait (followed by readfirstlane) would also wait for
// every tile load the wave has in flight.
template <typename T>
__device__ __forceinline__ T scalar_read(const T* p, int64_t i) {
  return ((const __attribute__((address_space(4))) T*)p)[i];
}

// Caches of 16-bit values (bf16, fp16) share the tile layout and loads; the
// MFMA and the packing of P and of the output follow the element type.
// Code caches compute in bf16.
template <int KV>
constexpr bool kHalf = KV == NVS_DTYPE_BF16 || KV == NVS_DTYPE_FP16;

template <int KV>
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (KV == NVS_DTYPE_FP16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int KV>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (KV == NVS_DTYPE_FP16)
    return pack_f16x2(a, b);
  else
    return pack_bf16x2(a, b);
}

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

template <>
struct DecodeTile<NVS_DTYPE_FP16> : DecodeTile<NVS_DTYPE_BF16> {};

template <int KV>
struct DecodeTile {
  u32x4 k[2][2];  // [t][half]: 32 codes, d = 32 grp + 16 half .. +15
  u32x2 v[8];     // [e]: 8 codes, d = 8 col .. +7
  float sc;       // lanes 0-31: k scale of key l; lanes 32-63: v scale of key l - 32
  bool has;
};

__device__ __forceinline__ int slot_key(int e, int grp) { return 16 * (e >> 2) + 4 * grp + (e & 3); }

// head_dim elements of MFMA step s / lane group grp in the QK^T product:
// d = kKStepStride * s + kKGroupStride * grp + 0..7.  Any split works as long
// as K and Q use the same one; bf16 K uses d = 32 s + 8 grp so that one load
// instruction reads 64 contiguous bytes of each of its 16 rows, code caches
// keep d = 32 grp + 8 s (one 128-byte row per lane group pair of loads).
template <int KV>
constexpr int kKStepStride = kHalf<KV> ? 32 : 8;
template <int KV>
constexpr int kKGroupStride = kHalf<KV> ? 8 : 32;

// Per-lane byte offsets from a tile's first row, identical for every tile.
// A load of slot e adds the wave-uniform offset of key row slot_key(e, 0)
// (or 16 t) to a scalar base, so each kind of load needs one lane offset.
struct LaneOffsets {
  uint32_t k;   // key col, d = 8 grp (bf16) / 32 grp (codes)
  uint32_t v;   // key 4 grp, d = 8 col
};

template <int KV>
__device__ __forceinline__ LaneOffsets lane_offsets(int Hkv, int col, int grp) {
  constexpr uint32_t ESZ = kHalf<KV> ? 2 : 1;
  const uint32_t row = (uint32_t)Hkv * kHeadDim * ESZ;  // bytes per token row (all heads)
  LaneOffsets o;
  o.k = (uint32_t)col * row + kKGroupStride<KV> * grp * ESZ;
  o.v = (uint32_t)(4 * grp) * row + 8 * col * ESZ;
  return o;
}

// The cache's V bytes are read once per call, each load instruction taking
// whole 128-byte lines: those loads are marked non-temporal (`nt`), which
// keeps the stream from displacing other lines in the caches on its way
// (decode_8b: 252 -> 228 us per call; decode_quant bf16 471 -> 429, fp8
// 256 -> 240 us).  A K load instruction takes half of each line it touches
// (16 key rows x 64 bytes), the other half coming with the next instruction:
// K stays a plain load, since an `nt` line can leave the cache in between
// (K marked `nt` as well: fp8 233 -> 240 us, bf16 428 -> 429 us).
//
// V is read through a buffer resource whose base is the tile's first row:
// the loop-invariant lane offset and the slot's row offset (a scalar) form
// each address.  Built as 64-bit lane addresses instead, the compiler reused
// one address register as the destination of a V load, and since the loop
// can reach its next iteration from either unrolled step, it then waited
// for every load in flight (vmcnt(0)) at each step before issuing the next
// tile's loads: a wave had one tile in flight, not D - 1.
constexpr int kNtAux = 2;  // the `nt` bit of a buffer load's cache policy

// Loads of one 32-key tile of kv head h whose first key sits at offset koff
// of pool block blk (-1: missing; the loads then read block 0, in bounds).
// Every address is a wave-uniform row base plus a 32-bit lane offset.
template <int KV>
__device__ __forceinline__ void decode_load(DecodeTile<KV>& T, const DecodeArgs& a, const LaneOffsets& lo,
                                            int blk, int koff, int h) {
  constexpr int ESZ = kHalf<KV> ? 2 : 1;
  T.has = blk >= 0;
  const int64_t row0 = ((int64_t)(T.has ? blk : 0) * a.bs + koff) * a.Hkv + h;
  const int64_t rowb = (int64_t)a.Hkv * kHeadDim * ESZ;  // bytes per token row
  const char* kb = (const char*)a.kc + row0 * kHeadDim * ESZ;
  const char* vb = (const char*)a.vc + row0 * kHeadDim * ESZ;
  const uint32_t ok = lane_off(lo.k);
  // num_records past any row offset a tile uses; a raw buffer's loads are
  // range-checked against it (an access past it reads 0).
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)vb, 0, 0x7fffffff, 0x20000);
  if constexpr (kHalf<KV>) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) T.k[t][s] = *reinterpret_cast<const u32x4*>(kb + 16 * t * rowb + 64 * s + ok);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      T.v[e] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, lo.v, (int)(slot_key(e, 0) * rowb),
                                                                                kNtAux));
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      T.k[t][0] = *reinterpret_cast<const u32x4*>(kb + 16 * t * rowb + ok);
      T.k[t][1] = *reinterpret_cast<const u32x4*>(kb + 16 * t * rowb + 16 + ok);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      T.v[e] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(vr, lo.v, (int)(slot_key(e, 0) * rowb),
                                                                               kNtAux));
    // One scale per lane (lanes 0-31 the k scales of the tile's keys, 32-63
    // the v scales); the compute hands each lane its keys' scales with
    // cross-lane reads.
    const uint32_t so = lane_off((uint32_t)(threadIdx.x & 31) * (uint32_t)a.Hkv * 4u);
    const char* sb = (const char*)(((threadIdx.x & 32) == 0 ? a.ks : a.vs) + row0);
    // A plain load: 4-byte scales of rows Hkv x 4 bytes apart, marked
    // non-temporal, made the fp8 decode_quant call 5 % slower (251 against
    // 239 us).
    T.sc = *reinterpret_cast<const float*>(sb + so);
  }
}

// A missing block reads as all-zero keys and values: clear the tile in place
// (the loads fetched block 0).
template <int KV>
__device__ __forceinline__ void zero_tile(DecodeTile<KV>& T) {
  if constexpr (kHalf<KV>) {
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
    for (int e = 0; e < 8; ++e) T.v[e] = u32x2{0, 0};
    T.sc = 0.0f;
  }
}

// Scales of a lane's 8 key slots from the tile's one-scale-per-lane register
// (lanes 0-31: k scale of key l, lanes 32-63: v scale of key l - 32).  Slot e
// is key slot_key(e, grp).  ds_bpermute_b32 reads lane (address + offset) / 4,
// so all 16 reads share one address register (16 grp bytes) and carry the
// slot's key as the instruction's offset; one wait ends the block.
__device__ __forceinline__ void tile_scales(float sc, int grp, float (&ksc)[8], float (&vsc)[8]) {
  const int base = 16 * grp;
  asm("ds_bpermute_b32 %0, %16, %17 offset:0\n\t"
      "ds_bpermute_b32 %1, %16, %17 offset:4\n\t"
      "ds_bpermute_b32 %2, %16, %17 offset:8\n\t"
      "ds_bpermute_b32 %3, %16, %17 offset:12\n\t"
      "ds_bpermute_b32 %4, %16, %17 offset:64\n\t"
      "ds_bpermute_b32 %5, %16, %17 offset:68\n\t"
      "ds_bpermute_b32 %6, %16, %17 offset:72\n\t"
      "ds_bpermute_b32 %7, %16, %17 offset:76\n\t"
      "ds_bpermute_b32 %8, %16, %17 offset:128\n\t"
      "ds_bpermute_b32 %9, %16, %17 offset:132\n\t"
      "ds_bpermute_b32 %10, %16, %17 offset:136\n\t"
      "ds_bpermute_b32 %11, %16, %17 offset:140\n\t"
      "ds_bpermute_b32 %12, %16, %17 offset:192\n\t"
      "ds_bpermute_b32 %13, %16, %17 offset:196\n\t"
      "ds_bpermute_b32 %14, %16, %17 offset:200\n\t"
      "ds_bpermute_b32 %15, %16, %17 offset:204\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(ksc[0]), "=&v"(ksc[1]), "=&v"(ksc[2]), "=&v"(ksc[3]), "=&v"(ksc[4]), "=&v"(ksc[5]),
        "=&v"(ksc[6]), "=&v"(ksc[7]), "=&v"(vsc[0]), "=&v"(vsc[1]), "=&v"(vsc[2]), "=&v"(vsc[3]),
        "=&v"(vsc[4]), "=&v"(vsc[5]), "=&v"(vsc[6]), "=&v"(vsc[7])
      : "v"(base), "v"(sc));
}
static_assert(4 * (16 + 3) + 4 * 32 + 16 * 3 < 256, "scale reads stay inside the wave's 64 lanes");

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
      if constexpr (kHalf<KV>) {
        kop = __builtin_bit_cast(bf16x8, T.k[t][st]);
      } else {
        const u32x4 w = T.k[t][st >> 1];
        kop = codes8_to_bf16x8<KV>(w[2 * (st & 1)], w[2 * (st & 1) + 1]);
      }
      s[t] = mfma16x16x32<KV>(kop, qop[st], s[t]);
    }
  }
  // ---- per-key scales of quantised caches: slot e of this lane is key
  // slot_key(e, grp), whose k scale lane slot_key(e, grp) holds and whose v
  // scale lane 32 + slot_key(e, grp) holds.
  float ksc[8], vsc[8];
  if constexpr (!kHalf<KV>) tile_scales(T.sc, grp, ksc, vsc);
  // ---- online softmax (log2 domain) -----------------------------------------
  bool valid[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) valid[e] = !MASKED || (kt + slot_key(e, grp) < kend);
  float sv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float f = scale_log2;
    if constexpr (!kHalf<KV>) f *= ksc[e];
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
    if constexpr (!kHalf<KV>) pw = p * vsc[e];
    if constexpr (MASKED) pw = valid[e] ? pw : 0.0f;
    pv[e] = pw;
  }
  u32x4 pw;
#pragma unroll
  for (int m = 0; m < 4; ++m) pw[m] = pack2<KV>(pv[2 * m], pv[2 * m + 1]);
  const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);

  // ---- V^T operands (transpose in registers) and O^T += V^T . P^T ---------
  uint32_t keep[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const bool v0 = valid[2 * m], v1 = valid[2 * m + 1];
    if constexpr (kHalf<KV>)
      keep[m] = (v0 ? 0x0000ffffu : 0u) | (v1 ? 0xffff0000u : 0u);
    else
      keep[m] = (v0 ? 0x00ff00ffu : 0u) | (v1 ? 0xff00ff00u : 0u);
  }
  if constexpr (kHalf<KV>) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4 aw;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        aw[m] = __builtin_amdgcn_perm(T.v[2 * m + 1][j >> 1], T.v[2 * m][j >> 1],
                                      MASKED ? masked_sel(sel, keep[m]) : sel);
      o[j] = mfma16x16x32<KV>(__builtin_bit_cast(bf16x8, aw), pop, o[j]);
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

// ---------------------------------------------------------------------------
// Scheduling, on the device and without a planning launch: decode work is
// counted in 32-key tiles of the decode rows (q_len == 1 rows with at least
// one visible key), in row order, T in all.  Every wave derives T, the group
// count Kw and its group's first tile from cu_seqlens itself, scanning the
// batch 64 rows at a time (one row per lane).
// ---------------------------------------------------------------------------

// Row b of the batch: whether it is a decode row (q_len == 1; malformed rows
// are skipped), its output row and key count.
struct RowInfo {
  bool dec;
  int q0, K;
};

__device__ __forceinline__ RowInfo row_info(const DecodeArgs& a, const int32_t* __restrict__ cu_q,
                                            const int32_t* __restrict__ cu_k, int b) {
  RowInfo r;
  r.q0 = scalar_read(cu_q, b);
  const int q1 = scalar_read(cu_q, b + 1);
  r.K = scalar_read(cu_k, b + 1) - scalar_read(cu_k, b);
  r.dec = q1 - r.q0 == 1 && r.q0 >= 0 && (int64_t)q1 <= a.T;
  return r;
}

__device__ __forceinline__ int row_tiles(const RowInfo& r) {
  return r.dec && r.K > 0 ? (r.K + kDecodeTile - 1) / kDecodeTile : 0;
}

// A scan round: the 256 rows c0 .. c0 + 255 of the batch, lane l holding
// rows c0 + 4 l .. + 3 as the cu_seqlens entries around them (q[i], k[i] =
// cu_seqlens_q/k[c0 + 4 l + i], i = 0..4; entries past B read entry B, so
// those rows are empty).  A lane issues its ten loads together, so a batch
// of up to 256 rows costs one load round trip.
constexpr int kScanRows = 4;
constexpr int kScanSpan = 64 * kScanRows;

struct ScanRound {
  int c0;
  int q[kScanRows + 1];
  int k[kScanRows + 1];
};

__device__ __forceinline__ ScanRound load_round(const DecodeArgs& a, const int32_t* __restrict__ cu_q,
                                                const int32_t* __restrict__ cu_k, int c0) {
  ScanRound r;
  r.c0 = c0;
  const int b0 = c0 + kScanRows * (int)(threadIdx.x & 63);
#pragma unroll
  for (int i = 0; i <= kScanRows; ++i) {
    const int b = min(b0 + i, a.B);
    r.q[i] = cu_q[b];
    r.k[i] = cu_k[b];
  }
  return r;
}

// Tiles of the row with cu_seqlens entries (q0, q1) and (k0, k1); the same
// rule as row_info / row_tiles.
__device__ __forceinline__ int tiles_of(const DecodeArgs& a, int q0, int q1, int k0, int k1) {
  const int K = k1 - k0;
  const bool dec = q1 - q0 == 1 && q0 >= 0 && (int64_t)q1 <= a.T;
  return dec && K > 0 ? (K + kDecodeTile - 1) / kDecodeTile : 0;
}

__device__ __forceinline__ int lane_tiles(const DecodeArgs& a, const ScanRound& r) {
  int n = 0;
#pragma unroll
  for (int i = 0; i < kScanRows; ++i) n += tiles_of(a, r.q[i], r.q[i + 1], r.k[i], r.k[i + 1]);
  return n;
}

// Wave sum; every lane holds it after the butterfly, and readfirstlane tells
// the compiler it is wave-uniform (else everything derived from it, down to
// the tile cursors, would be treated as divergent and kept in VGPRs).
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
  return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}

// The step's new token of a decode row (query row q0), kv head h, written
// into the cache at `slot` (slot_mapping[q0]): lanes 0-15 take the k row,
// lanes 16-31 the v row, 8 elements each.  A bf16 cache receives the
// values; an fp8 / int8 cache the codes and the per-token scale, computed by
// the store kernel's own helpers (absmax over the row's 16 lanes,
// quant_scale, quant8), so the bytes are identical whichever wave writes
// them.  Slots outside the cache are skipped, as the store kernel skips
// them.
template <int KV>
__device__ __forceinline__ void store_new_token(const DecodeArgs& a, int q0, int64_t slot, int h) {
  const int lane = threadIdx.x & 63;
  if (slot < 0 || slot >= a.total_slots || lane >= 32) return;
  const int c = lane & 15;
  const uint32_t off = lane_off(16u * (uint32_t)c);
  const bool isv = lane >= 16;
  const char* src = (const char*)(isv ? a.vn + (int64_t)q0 * a.vn_ts + (int64_t)h * a.vn_hs
                                      : a.kn + (int64_t)q0 * a.kn_ts + (int64_t)h * a.kn_hs);
  const int64_t row = slot * a.Hkv + h;
  if constexpr (KV == NVS_DTYPE_BF16) {
    char* dst = (char*)(isv ? a.vc : a.kc) + row * (int64_t)(kHeadDim * 2);
    *reinterpret_cast<u32x4*>(dst + off) = *reinterpret_cast<const u32x4*>(src + off);
  } else if constexpr (KV == NVS_DTYPE_FP16) {  // bf16 sources cast to fp16 (RNE)
    float x[8];
    load8<NVS_DTYPE_BF16>(src + off, x);
    char* dst = (char*)(isv ? a.vc : a.kc) + row * (int64_t)(kHeadDim * 2);
    store8_float<NVS_DTYPE_FP16>(dst + off, x);
  } else {
    float x[8];
    load8<NVS_DTYPE_BF16>(src + off, x);
    constexpr float qmax = (KV == NVS_DTYPE_INT8) ? QuantInt8::kQmax : QuantFp8::kQmax;
    const float sc = quant_scale(row_absmax(x, kHeadDim / 8), qmax);
    char* dst = (char*)(isv ? a.vc : a.kc) + row * (int64_t)kHeadDim;
    *reinterpret_cast<u32x2*>(dst + 8 * c) = quant8<KV, true>(x, sc);
    if (c == 0) const_cast<float*>(isv ? a.vs : a.ks)[row] = sc;
  }
}

// Zeroes the output of the round's decode rows that see no key (row b by
// decode wave b % nw): no tile covers them, so no wave writes them otherwise.
template <int KV>
__device__ __forceinline__ void zero_keyless_rows(const DecodeArgs& a, const ScanRound& rd, int wi, int nw) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < kScanRows; ++i) {
    const int b = rd.c0 + kScanRows * lane + i;
    const bool dec = rd.q[i + 1] - rd.q[i] == 1 && rd.q[i] >= 0 && (int64_t)rd.q[i + 1] <= a.T;
    uint64_t z = __ballot(b < a.B && dec && rd.k[i + 1] - rd.k[i] <= 0 && b % nw == wi);
    while (z) {
      const int li = __builtin_ctzll(z);
      z &= z - 1;
      const int q0 = __builtin_amdgcn_readlane(rd.q[i], li);
      for (int x = lane; x < a.Hq * (kHeadDim / 8); x += 64) {
        const int hq = x / (kHeadDim / 8), d = 8 * (x % (kHeadDim / 8));
        *reinterpret_cast<u32x4*>(a.out + (int64_t)q0 * a.out_ts + (int64_t)hq * a.out_hs + d) = u32x4{0, 0, 0, 0};
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Where the step's new tokens may be written from.  The owner of a decode
// row's last tile writes the row's token ahead of its own load of that tile
// when the slot is the row's own last position (slot == block_table[row][
// (k_len - 1) / bs] * bs + (k_len - 1) % bs, the slot the engine forms for a
// decode row): no other wave reads that position as long as no other row of
// the batch reads the row's last block at that offset (a sequence appends
// only into its own last block).  Any other valid slot (a keyless row, a
// missing block, a slot in another row's keys or in an earlier tile of its
// own row) could be read by any wave of the kv head, so every such wave
// writes it before its first load: the bytes are the same from every wave,
// so each wave reads the new token (its own write, or an identical one), as
// after the reference's write-then-read.  Negative slots and slots outside
// the cache are skipped, as the store kernel skips them.
// ---------------------------------------------------------------------------
struct SlotCheck {
  int slot[kScanRows];  // slot_mapping of the lane's rows (-1 for non-decode rows)
  int blk[kScanRows];   // block-table entry of their last position (-1: none)
  int off[kScanRows];   // that position's offset in its block (-1: keyless row)
};

// Loads of a scan round's slots and last-position block ids (vector loads,
// issued early; the values are used after the tile search).
__device__ __forceinline__ SlotCheck issue_slot_check(const DecodeArgs& a, const int32_t* __restrict__ bt,
                                                      const ScanRound& rd) {
  SlotCheck c;
  const int b0 = rd.c0 + kScanRows * (int)(threadIdx.x & 63);
#pragma unroll
  for (int i = 0; i < kScanRows; ++i) {
    const int b = b0 + i;
    const bool dec = b < a.B && rd.q[i + 1] - rd.q[i] == 1 && rd.q[i] >= 0 && (int64_t)rd.q[i + 1] <= a.T;
    const int K = rd.k[i + 1] - rd.k[i];
    const int lb = K > 0 ? (K - 1) / a.bs : 0;
    c.slot[i] = -1;
    c.blk[i] = -1;
    c.off[i] = K > 0 ? K - 1 - lb * a.bs : -1;
    if (dec) c.slot[i] = a.slots[rd.q[i]];
    if (dec && K > 0 && lb < a.bt_stride) c.blk[i] = bt[(int64_t)b * a.bt_stride + lb];
  }
  return c;
}

// Whether a decode row's token may be left to the owner of its last tile:
// its slot is skipped, or it is the row's last position, offset `off`
// (-1: the row has no key) in block `blk` (-1: none).
__device__ __forceinline__ bool owner_writes(const DecodeArgs& a, int64_t slot, int blk, int off) {
  if (slot < 0 || slot >= a.total_slots) return true;  // skipped by every writer
  if (off < 0 || blk < 0 || blk >= a.NB) return false;
  return slot == (int64_t)blk * a.bs + off;
}

// Every wave of kv head h writes the round's rows that no owner writes
// (ballot over the lanes' rows); true if there was one.
template <int KV>
__device__ __forceinline__ bool write_nonconforming(const DecodeArgs& a, const ScanRound& rd,
                                                    const SlotCheck& c, int h) {
  bool any = false;
#pragma unroll
  for (int i = 0; i < kScanRows; ++i) {
    const bool bad = !owner_writes(a, c.slot[i], c.blk[i], c.off[i]);
    uint64_t z = __ballot(bad);
    any |= z != 0;
    while (z) {
      const int li = __builtin_ctzll(z);
      z &= z - 1;
      store_new_token<KV>(a, __builtin_amdgcn_readlane(rd.q[i], li), __builtin_amdgcn_readlane(c.slot[i], li), h);
    }
  }
  return any;
}

// The all-waves writes of the whole batch: round 0 from the checks issued at
// the start, later rounds (more than 256 rows) loaded here.
template <int KV>
__device__ __forceinline__ bool write_all_nonconforming(const DecodeArgs& a, const int32_t* __restrict__ bt,
                                                        const int32_t* __restrict__ cu_q,
                                                        const int32_t* __restrict__ cu_k, const ScanRound& r0,
                                                        const SlotCheck& c0, int h) {
  bool any = write_nonconforming<KV>(a, r0, c0, h);
  for (int s = kScanSpan; s < a.B; s += kScanSpan) {
    const ScanRound rd = load_round(a, cu_q, cu_k, s);
    any |= write_nonconforming<KV>(a, rd, issue_slot_check(a, bt, rd), h);
  }
  return any;
}

// Total decode tiles of the batch; r0 receives the first scan round, which
// locate_tile reuses.  Keyless decode rows are zeroed on the way.
template <int KV>
__device__ __forceinline__ int decode_tiles(const DecodeArgs& a, const int32_t* __restrict__ cu_q,
                                            const int32_t* __restrict__ cu_k, ScanRound& r0, int wi, int nw) {
  r0 = load_round(a, cu_q, cu_k, 0);
  int tot = wave_sum_i(lane_tiles(a, r0));
  zero_keyless_rows<KV>(a, r0, wi, nw);
  for (int c0 = kScanSpan; c0 < a.B; c0 += kScanSpan) {
    const ScanRound rd = load_round(a, cu_q, cu_k, c0);
    tot += wave_sum_i(lane_tiles(a, rd));
    zero_keyless_rows<KV>(a, rd, wi, nw);
  }
  return tot;
}

// Position of a decode wave in its tile stream: a decode row and a tile.
// All members are wave-uniform (scalar registers).
struct Cursor {
  int b, q0, K, n;  // the row
  int t;            // tile
  int lb, koff;     // its logical block and key offset in the block (kept
                    // incrementally: a division by block_size would be VALU)
};

// The decode row and tile of tile index s (< T), and the row's first tile
// index.  r0 is the first scan round (rows 0 .. 255); later rounds are loaded
// as the search reaches them.  The row is read from the found lane's
// registers, so the cursor needs no further loads.
__device__ __forceinline__ void locate_tile(const DecodeArgs& a, const int32_t* __restrict__ cu_q,
                                            const int32_t* __restrict__ cu_k, int s, const ScanRound& r0,
                                            Cursor& c, int& first) {
  int base = 0;
  for (int c0 = 0; c0 < a.B; c0 += kScanSpan) {
    const ScanRound rd = c0 == 0 ? r0 : load_round(a, cu_q, cu_k, c0);
    const int nl = lane_tiles(a, rd);
    const int incl = base + wave_incl_scan(nl);
    const uint64_t m = __ballot(incl > s);
    if (m) {
      const int li = __builtin_amdgcn_readfirstlane(__builtin_ctzll(m));
      int e = __builtin_amdgcn_readlane(incl, li) - __builtin_amdgcn_readlane(nl, li);
      int q[kScanRows + 1], k[kScanRows + 1];
#pragma unroll
      for (int i = 0; i <= kScanRows; ++i) {
        q[i] = __builtin_amdgcn_readlane(rd.q[i], li);
        k[i] = __builtin_amdgcn_readlane(rd.k[i], li);
      }
      // The lane's rows in order: the first whose tiles reach past s.  Its
      // total exceeds s - e, so one of them does.
      bool found = false;
#pragma unroll
      for (int i = 0; i < kScanRows; ++i) {
        const int n = tiles_of(a, q[i], q[i + 1], k[i], k[i + 1]);
        if (!found && e + n > s) {
          found = true;
          c.b = rd.c0 + kScanRows * li + i;
          c.q0 = q[i];
          c.K = k[i + 1] - k[i];
          c.n = n;
          first = e;
        }
        if (!found) e += n;
      }
      c.t = s - first;
      c.lb = (c.t * kDecodeTile) / a.bs;
      c.koff = c.t * kDecodeTile - c.lb * a.bs;
      return;
    }
    base = __builtin_amdgcn_readlane(incl, 63);
  }
  // Unreachable for s < T; an in-bounds cursor at row 0 keeps every access valid.
  c.b = 0;
  c.q0 = __builtin_amdgcn_readlane(r0.q[0], 0);
  c.K = 0;
  c.n = 1;
  c.t = c.lb = c.koff = 0;
  first = 0;
}

// Moves cursor x to the next decode row with keys (scalar loads; in a pure
// decode batch that is the next row).  Past the last row the cursor stays.
__device__ __forceinline__ void next_row(const DecodeArgs& a, const int32_t* __restrict__ cu_q,
                                         const int32_t* __restrict__ cu_k, Cursor& x) {
  for (int b = x.b + 1; b < a.B; ++b) {
    const RowInfo r = row_info(a, cu_q, cu_k, b);
    const int n = row_tiles(r);
    if (n > 0) {
      x.b = b;
      x.q0 = r.q0;
      x.K = r.K;
      x.n = n;
      break;
    }
  }
  x.t = x.lb = x.koff = 0;
}

// Block id of cursor c's tile (-1 where the table has none or it is outside
// the pool); a 32-key tile never spans two blocks (block_size % 64 == 0).
__device__ __forceinline__ int tile_block(const DecodeArgs& a, const int32_t* __restrict__ bt, const Cursor& c) {
  const int blk = c.lb < a.bt_stride ? scalar_read(bt, (int64_t)c.b * a.bt_stride + c.lb) : -1;
  return (blk >= 0 && blk < a.NB) ? blk : -1;
}

// Q^T as the B operand for query row q0, kv head h: column = head (col < g);
// step s, lane group grp holds the same 8 d values as the K operand: d = 32 s
// + 8 grp for bf16 caches, 32 grp + 8 s for code caches.  Columns past the
// group's heads hold head 0's values: every column's scores, softmax and
// output are its own (the MFMAs never mix columns, the row max and sum
// reduce over one column's lanes) and those columns are never stored.
// Zeroing them would wait for the loads right away, and with them for every
// tile load in flight; this way the wait falls at the next tile's MFMAs.
template <int KV>
__device__ __forceinline__ void load_q(bf16x8 (&qop)[4], const DecodeArgs& a, int q0, int h, int col, int grp) {
  const bool use = col < a.g;
  // Row base of the group's first head plus a 32-bit lane offset (head
  // strides are below 2^26 elements, so (g - 1) heads fit).
  const char* qb = (const char*)(a.q + (int64_t)q0 * a.q_ts + (int64_t)h * a.g * a.q_hs);
  const uint32_t lo =
      lane_off(((uint32_t)(use ? col : 0) * (uint32_t)a.q_hs + kKGroupStride<KV> * grp) * 2u);
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qop[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(qb + lo + kKStepStride<KV> * s * 2));
}

// The end of a row segment of kv head h: a row the wave saw whole is
// normalised and written; a split row leaves its partial in slot `slot` of
// wave w.  Lane (col, grp) holds O[hq][d] for d = 32 grp + 8 r + j in o[j][r].
__device__ __forceinline__ void finish_segment(const DecodeArgs& a, const Cursor& c, int h, bool whole, int w,
                                               int slot, const f32x4 (&o)[8], float m_run, float l_run, int col,
                                               int grp) {
  if (col >= a.g) return;
  if (whole) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    // Row base of the group's first head plus a 32-bit lane offset, as in load_q.
    char* ob = (char*)(a.out + (int64_t)c.q0 * a.out_ts + (int64_t)h * a.g * a.out_hs);
    const uint32_t lo = lane_off(((uint32_t)col * (uint32_t)a.out_hs + 32u * grp) * 2u);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 v;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        v[m] = a.f16 ? pack_f16x2(o[2 * m][r] * inv, o[2 * m + 1][r] * inv)
                     : pack_bf16x2(o[2 * m][r] * inv, o[2 * m + 1][r] * inv);
      *reinterpret_cast<u32x4*>(ob + lo + 16 * r) = v;
    }
  } else {
    const int64_t base = ((int64_t)w * 2 + slot) * a.g;  // partial row of head 0 of the group
    char* ob = (char*)(a.ws_o + base * kHeadDim);
    const uint32_t lo = lane_off(((uint32_t)col * kHeadDim + 32u * grp) * 4u);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      *reinterpret_cast<f32x4*>(ob + lo + 32 * r) = f32x4{o[0][r], o[1][r], o[2][r], o[3][r]};
      *reinterpret_cast<f32x4*>(ob + lo + 32 * r + 16) = f32x4{o[4][r], o[5][r], o[6][r], o[7][r]};
    }
    if (grp == 0)
      *reinterpret_cast<f32x2*>((char*)(a.ws_ml + base * 2) + lane_off((uint32_t)col * 8u)) =
          f32x2{m_run, l_run};
  }
}

// Decode ranges: Kw groups of Hkv waves (one per kv head) share the T tiles,
// group k taking [floor(k T / Kw), floor((k + 1) T / Kw)); Kw = min(launched
// groups, T / kDecodeMinUnits), at least 1.
__device__ __forceinline__ int decode_groups(int T, int G) {
  return T > 0 ? min(G, max(1, T / kDecodeMinUnits)) : 0;
}


// One decode wave (kv head h of group k of the G groups the launch has
// room for; wave wi of the nw decode waves): tiles [s0, s0 + left) of the
// stream, streamed one by one, partials at index w.  Cursor n[0] is the
// tile being computed, n[1] .. n[D - 1] the next ones (their loads are in
// flight during n[0]'s compute) and n[D] the one after (its block id is
// fetched during n[0]'s compute), D the ring depth.  Loads are issued
// unconditionally (past the wave's last tile the cursors stop advancing, so
// the surplus loads re-read the last tile) and the ring is unrolled so every
// buffer index is a compile-time constant.  The block table is read through
// a restrict-qualified pointer, so its entries are scalar loads whose waits
// never wait for the wave's vector loads.
template <int KV, int D>
__device__ __forceinline__ void decode_wave(const DecodeArgs& a, const int32_t* __restrict__ bt,
                                            const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
                                            int h, int k, int G, int wi, int nw) {
  const int w = k * a.Hkv + h;  // partial slot index (k < G)
  const int lane = threadIdx.x & 63;

  ScanRound r0;
  const int T = decode_tiles<KV>(a, cu_q, cu_k, r0, wi, nw);
  const int Kw = decode_groups(T, G);
  if (w == 0 && lane < 2) a.ws_rec[lane] = lane == 0 ? T : Kw;
  // The slot checks of the first 256 rows, waited for after the tile search.
  SlotCheck chk0;
  if (a.kn) chk0 = issue_slot_check(a, bt, r0);
  if (k >= Kw) {
    if (lane == 0 && k < G) a.ws_rec[4 + 4 * w + 3] = 0;
    // With no tile at all no wave reads the cache; group 0 still writes the
    // rows no owner writes.
    if (a.kn && k == 0) write_all_nonconforming<KV>(a, bt, cu_q, cu_k, r0, chk0, h);
    return;
  }
  const int s0 = group_start(T, Kw, k);
  const int left = group_start(T, Kw, k + 1) - s0;  // >= 1 (Kw <= T)

  const int col = lane & 15, grp = lane >> 4;
  const LaneOffsets lo = lane_offsets<KV>(a.Hkv, col, grp);

  // Cursors.
  Cursor n[D + 1];
  {
    int first;
    locate_tile(a, cu_q, cu_k, s0, r0, n[0], first);
  }
  // The new tokens of the rows whose last tile lies in this range and whose
  // slot is their own last position are written by this wave (a.kn set),
  // all of them here, before the ring's state exists, so the walk's
  // registers are free again by the main loop; then the rows no owner
  // writes, by every wave.  The wave's own load of a row's last tile must
  // follow the row's write in the wave's program order (one wave's vector
  // memory operations reach its CU's L1 in issue order): a workgroup-scope
  // release fence, which keeps the compiler from moving the load above the
  // write and, with one wave per work-group, adds no wait, goes before the
  // first loads if a row ends in the tiles they cover or the wave wrote a
  // row no owner writes, otherwise just before the load of the first
  // written row's last tile (fence_tile).
  int fence_tile = INT_MAX;
  if (a.kn) {
    Cursor c = n[0];
    int tile = s0;  // global index of c's tile
    for (;;) {
      const int last = tile + (c.n - 1 - c.t);
      if (last >= s0 + left) break;  // the row ends in a later group's range
      const int64_t slot = a.slots[c.q0];
      const int lb = (c.K - 1) / a.bs;  // c.K >= 1: the row has tiles
      const int blk = lb < a.bt_stride ? scalar_read(bt, (int64_t)c.b * a.bt_stride + lb) : -1;
      if (owner_writes(a, slot, blk, c.K - 1 - lb * a.bs)) {
        store_new_token<KV>(a, c.q0, slot, h);
        fence_tile = min(fence_tile, last);
      }
      tile = last + 1;
      if (tile >= s0 + left) break;
      next_row(a, cu_q, cu_k, c);
    }
    if (write_all_nonconforming<KV>(a, bt, cu_q, cu_k, r0, chk0, h)) fence_tile = s0;
    if (fence_tile < s0 + D - 1) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      fence_tile = INT_MAX;
    }
  }
  auto advance = [&](Cursor& x) {
    if (++x.t == x.n) {
      next_row(a, cu_q, cu_k, x);
    } else if ((x.koff += kDecodeTile) == a.bs) {
      x.koff = 0;
      ++x.lb;
    }
  };
#pragma unroll
  for (int j = 1; j <= D; ++j) {
    n[j] = n[j - 1];
    if (left > j) advance(n[j]);
  }

  bf16x8 qop[4];
  load_q<KV>(qop, a, n[0].q0, h, col, grp);
  f32x4 o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  int seg_t0 = n[0].t;  // first tile of the current segment
  int slot = 0;         // partial slot of the current segment (0: the item's first)

  DecodeTile<KV> r[D];
#pragma unroll
  for (int j = 0; j < D - 1; ++j) decode_load<KV>(r[j], a, lo, tile_block(a, bt, n[j]), n[j].koff, h);
  int blk_last = tile_block(a, bt, n[D - 1]);

  // Tile i (cursor n[0]) from ring slot cur; the loads of tile i + D - 1 go
  // to slot nxt_t.
  auto step = [&](DecodeTile<KV>& cur, DecodeTile<KV>& nxt_t, int i) {
    if (s0 + i + D - 1 == fence_tile) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    decode_load<KV>(nxt_t, a, lo, blk_last, n[D - 1].koff, h);
    const int blk_next = tile_block(a, bt, n[D]);
    __builtin_amdgcn_sched_barrier(0);
    const Cursor& c = n[0];
    if (!cur.has) zero_tile(cur);
    const int kt = c.t * kDecodeTile;
    if (kt + kDecodeTile > c.K)  // the row's last, partial tile
      decode_tile_compute<KV, true>(cur, qop, o, m_run, l_run, kt, c.K, grp, a.scale_log2);
    else
      decode_tile_compute<KV, false>(cur, qop, o, m_run, l_run, kt, c.K, grp, a.scale_log2);
    __builtin_amdgcn_sched_barrier(0);
    if (c.t == c.n - 1 || i == left - 1) {  // the segment ends with tile i
      if (i == left - 1 && lane < 4) {
        // The wave's record: its last row (output row, tiles left after the
        // group's range, partial slot), valid if the row continues past the
        // range and starts inside it (this group merges it).
        const int v = lane == 0   ? c.q0
                      : lane == 1 ? c.n - 1 - c.t
                      : lane == 2 ? slot
                                  : (int)(c.t != c.n - 1 && seg_t0 == 0);
        a.ws_rec[4 + 4 * w + lane] = v;
      }
      float l = l_run + shfl_xor(l_run, 16);
      l += shfl_xor(l, 32);
      finish_segment(a, c, h, seg_t0 == 0 && c.t == c.n - 1, w, slot, o, m_run, l, col, grp);
      // The next tile clears o: with m_run = -inf its rescale always runs,
      // with alpha = 2^-inf = 0 (its first key is visible, so its max is
      // finite).  Not writing o here keeps it in one register set.
      m_run = -INFINITY;
      l_run = 0.0f;
      seg_t0 = 0;
      slot = 1;
      // The next segment's q (tile i + 1 starts it); its wait falls at tile
      // i + 1's compute, which waits for that tile's loads anyway.
      if (i + 1 < left) load_q<KV>(qop, a, n[1].q0, h, col, grp);
    }
#pragma unroll
    for (int j = 0; j < D; ++j) n[j] = n[j + 1];
    if (i + D + 1 < left) advance(n[D]);
    blk_last = blk_next;
  };
  for (int i = 0; i < left; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      if (i + j >= left) break;
      step(r[j], r[(j + D - 1) % D], i + j);
    }
  }
}

}  // namespace nvs
