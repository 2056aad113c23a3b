// Definitions shared by the decode and prefill attention kernels.
#pragma once

#include "nvs_common.h"

namespace nvs {

constexpr int kHeadDim = 128;    // head_dim served by the attention kernels
#ifndef NVS_DECODE_WAVES_PER_EU
#define NVS_DECODE_WAVES_PER_EU 2
#endif
constexpr int kDecodeWavesPerEU = NVS_DECODE_WAVES_PER_EU;  // decode waves per SIMD
constexpr int kDecodeTile = 32;         // keys per decode tile (one unit of decode work)
constexpr int kDecodeMaxWaves = 2048;   // decode waves per call at most (256 CUs x 8)
constexpr int kDecodeMinUnits = 4;      // fewest tiles a decode group is given

// 2^x on the hardware transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two fp32 values that are exactly bf16-representable -> packed bf16x2 by
// keeping their upper halves (no rounding needed).
__device__ __forceinline__ uint32_t pack_exact_bf16x2(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Codes in bytes (0,1) (HI = false) or (2,3) (HI = true) of x -> two fp32,
// exact.  gfx950 converts OCP e4m3 in hardware.
template <int KV, bool HI>
__device__ __forceinline__ void code_pair_to_f32(uint32_t x, float& f0, float& f1) {
  if constexpr (KV == NVS_DTYPE_FP8_E4M3) {
    const auto f = __builtin_amdgcn_cvt_pk_f32_fp8(x, HI);
    f0 = f[0];
    f1 = f[1];
  } else {
    constexpr int sh = HI ? 16 : 0;
    f0 = (float)(int32_t)(int8_t)(uint8_t)(x >> sh);
    f1 = (float)(int32_t)(int8_t)(uint8_t)(x >> (sh + 8));
  }
}

// Same pair -> packed bf16x2; int8 and e4m3 values are exactly representable
// in bf16, so no rounding happens.
template <int KV, bool HI>
__device__ __forceinline__ uint32_t code_pair_to_bf16x2(uint32_t x) {
  if constexpr (KV == NVS_DTYPE_FP8_E4M3) {
    // gfx950 converts two e4m3 codes straight to packed bf16 (scale 2^0).
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, HI));
  } else {
    float f0, f1;
    code_pair_to_f32<KV, HI>(x, f0, f1);
    return pack_exact_bf16x2(f0, f1);
  }
}

// 8 codes (bytes of lo then hi) -> bf16x8 operand.
template <int KV>
__device__ __forceinline__ bf16x8 codes8_to_bf16x8(uint32_t lo, uint32_t hi) {
  u32x4 w;
  w[0] = code_pair_to_bf16x2<KV, false>(lo);
  w[1] = code_pair_to_bf16x2<KV, true>(lo);
  w[2] = code_pair_to_bf16x2<KV, false>(hi);
  w[3] = code_pair_to_bf16x2<KV, true>(hi);
  return __builtin_bit_cast(bf16x8, w);
}

// ---------------------------------------------------------------------------
// Decode scheduling (paged calls): decode work is counted in 32-key tiles of
// the decode rows (q_len == 1 rows with a visible key), in row order, T in
// all.  Waves form groups of Hkv, one wave per kv head; of the Kw groups with
// work, group k takes tiles [floor(k T / Kw), floor((k + 1) T / Kw)) for its
// Hkv heads (stream-K: every wave gets the same work and streams across row
// boundaries).  The decode waves derive all of this from cu_seqlens
// themselves; rows split across groups leave partials in the workspace.
//
// Prefill work plan: a one-work-group planning kernel turns cu_seqlens into
// the prefill list in the workspace, on the device, so the prefill kernel
// launches a fixed persistent grid and never dispatches empty work-groups
// (each costs the dispatcher several nanoseconds; an upper-bound grid is
// mostly empty on ragged batches).
//   prefill list: b * ntq + qt, one entry per (q_len > 1 row, tile of
//                 prefill_positions(g) query positions), row by row, each
//                 row's tiles in descending qt (heaviest first).
// ---------------------------------------------------------------------------

// Prefill work item: one 8-wave work-group serves up to 8 query heads of one
// kv head (all of them when g <= 8) over a tile of query positions, 32 rows
// (positions) per wave; fewer heads per item means more positions per item.
constexpr int kPrefillWaves = 8;
constexpr int kPrefillWaveRows = 32;
__host__ __device__ inline int prefill_heads_per_item(int g) { return g < kPrefillWaves ? g : kPrefillWaves; }
__host__ __device__ inline int prefill_positions(int g) {
  return g <= 0 ? kPrefillWaveRows : kPrefillWaveRows * (kPrefillWaves / prefill_heads_per_item(g));
}
__host__ __device__ inline int prefill_head_groups(int g) { return (g + kPrefillWaves - 1) / kPrefillWaves; }

struct PlanHeader {
  int n_prefill;        // prefill list entries
  int prefill_next[8];  // per-XCD work counters of the prefill kernel (zeroed by the plan)
  int shadow_tiles;     // code caches: 64-key tiles of the prefill rows' bf16 copy
  int shadow_on;        // 1: the copy fits and the tile-loop kernel serves the prefill
  int dec_wgs;          // work-groups of the prefill launch that stream the decode rows first
  int pad[52];          // keeps the list 256-byte aligned
};
static_assert(sizeof(PlanHeader) == 256, "plan header is one 256-byte line");

// What a work-group of the MFMA prefill kernel needs to start a list entry,
// in one 64-byte load: the entry, its sequence's query and key ranges,
// (paged) the block ids of its first three 64-key tiles (-1: missing), and
// what the kernel derives from them per entry: the entry's first query
// position p0, the 64-key tiles its rows see, the key rows its fills may
// read (local mode: never past the k / v tensors), K - L, the first key row
// clamped into the local k / v, the sequence and the bytes of its
// block-table row the kernel may read.
struct PlanRecord {
  int item, q0, L, k0, K, blk0, blk1, blk2;
  int p0, ntiles, kf, off, k0c, b, bt_bytes, pad;
};
static_assert(sizeof(PlanRecord) == 64, "plan record is 64 bytes");

struct Plan {
  PlanHeader* hdr;
  int* plist;
  PlanRecord* rec;  // per list entry, beside plist
  int ntq;          // prefill query tiles per sequence (list stride)
  int pbm;          // query positions per prefill tile
};

inline int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Decode waves a call may use: Hkv per group, at most kDecodeMaxWaves in
// all, and no more groups than the tiles there can be (B rows x
// ceil(max_seqlen_k / 32)) allow at kDecodeMinUnits each, rounded up to a
// multiple of 8 groups (one per XCD of a launch round).
inline int decode_wave_cap(int B, int max_seqlen_k, int Hkv) {
  const int hk = Hkv > 0 ? Hkv : 1;
  const int64_t tiles = (int64_t)B * ((max_seqlen_k + kDecodeTile - 1) / kDecodeTile);
  int64_t groups = (tiles + kDecodeMinUnits - 1) / kDecodeMinUnits;
  groups = (groups + 7) / 8 * 8;
  const int64_t gmax = kDecodeMaxWaves / hk > 0 ? kDecodeMaxWaves / hk : 1;
  groups = groups < 1 ? 1 : (groups > gmax ? gmax : groups);
  return (int)(groups * hk);
}

// Bytes of the plan for a batch; it sits at the start of the workspace.
inline int64_t plan_bytes(int B, int ntq) {
  return (int64_t)sizeof(PlanHeader) + align256((int64_t)B * ntq * 4) +
         align256((int64_t)B * ntq * (int64_t)sizeof(PlanRecord));
}

inline Plan plan_at(void* ws, int B, int ntq, int pbm) {
  Plan p;
  p.hdr = (PlanHeader*)ws;
  p.plist = (int*)((char*)ws + sizeof(PlanHeader));
  p.rec = (PlanRecord*)((char*)ws + sizeof(PlanHeader) + align256((int64_t)B * ntq * 4));
  p.ntq = ntq;
  p.pbm = pbm;
  return p;
}

// Number of work-group slots the device runs at once for a kernel with
// `per_cu` resident work-groups per CU (CU count cached per device).
int device_slots(int per_cu);

// Validated launch parameters of one attention call.
struct AttnParams {
  const void* q;
  int64_t q_ts, q_hs;
  // paged mode
  const void* kc;
  const void* vc;
  int cache_dtype;
  const float* ks;
  const float* vs;
  const int32_t* bt;  // null selects the local (non-paged) mode
  int64_t bt_stride;
  int bs;
  int64_t NB;
  // local mode
  const void* k;
  const void* v;
  int64_t k_ts, k_hs, v_ts, v_hs;
  // batch
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B;
  // The step's new k / v rows (bf16) that the decode kernel stores into a
  // bf16 cache itself (null: the caller stored them).
  const void* kn;
  const void* vn;
  int64_t kn_ts, kn_hs, vn_ts, vn_hs;
  const int32_t* slots;
  int64_t T;   // query / output rows
  int64_t Tk;  // rows of the local k/v (varlen mode)
  int max_seqlen_q, max_seqlen_k;
  int Hq, Hkv;
  float softmax_scale;
  void* out;
  int64_t out_ts, out_hs;
  void* ws;
  int64_t ws_bytes;
  // Prefill kernels launched side by side run only where *gate == gate_run
  // (null: always): the plan decides on the device which one serves.
  const int* gate;
  int gate_run;
};

// Code caches (int8 / fp8): the prefill rows' keys and values are first
// dequantised, bf16(code x scale) exactly as the reference's prefill_torch
// does per sequence (attention.py:268-273), into a bf16 copy in the
// workspace made of 64-key tiles [tile, 64, Hkv, 128], one run of tiles per
// prefill row, with a table row per sequence mapping its 64-key tile t to a
// copy tile; the MFMA tile-loop kernel then reads the copy as a bf16 paged
// cache of block size 64.  The copy's capacity is the batch bound (rows x
// ceil(max_seqlen_k / 64) tiles), at most kShadowMaxBytes; a batch whose
// prefill rows need more tiles falls back, on the device, to the classic
// kernel, which dequantises in its tile fill.
constexpr int kShadowTile = 64;
constexpr int64_t kShadowMaxBytes = 1ll << 30;  // K + V copy
struct ShadowLayout {
  int* base;    // [B + 1]: first copy tile of row b (exclusive prefix; base[B] = all)
  int* table;   // [B, ST]: copy tile of row b's 64-key tile t
  uint16_t* k;  // [cap, 64, Hkv, 128] bf16
  uint16_t* v;
  int ST;       // table row length: ceil(max_seqlen_k / 64)
  int cap;      // copy tiles
};
inline int64_t shadow_tile_bytes(int Hkv) { return (int64_t)kShadowTile * Hkv * kHeadDim * 2; }
inline int shadow_cap(int B, int max_seqlen_k, int Hkv) {
  const int64_t st = ((int64_t)max_seqlen_k + kShadowTile - 1) / kShadowTile;
  const int64_t most = kShadowMaxBytes / (2 * shadow_tile_bytes(Hkv > 0 ? Hkv : 1));
  const int64_t c = (int64_t)B * st < most ? (int64_t)B * st : most;
  return (int)(c > 0 ? c : 0);
}
inline int64_t shadow_bytes(int B, int max_seqlen_k, int Hkv) {
  const int64_t st = ((int64_t)max_seqlen_k + kShadowTile - 1) / kShadowTile;
  return align256((int64_t)(B + 1) * 4) + align256((int64_t)B * st * 4) +
         2 * (int64_t)shadow_cap(B, max_seqlen_k, Hkv) * shadow_tile_bytes(Hkv);
}
inline ShadowLayout shadow_at(void* p, int B, int max_seqlen_k, int Hkv) {
  ShadowLayout s;
  s.ST = (int)(((int64_t)max_seqlen_k + kShadowTile - 1) / kShadowTile);
  s.cap = shadow_cap(B, max_seqlen_k, Hkv);
  char* c = (char*)p;
  s.base = (int*)c;
  c += align256((int64_t)(B + 1) * 4);
  s.table = (int*)c;
  c += align256((int64_t)B * s.ST * 4);
  s.k = (uint16_t*)c;
  s.v = (uint16_t*)(c + (int64_t)s.cap * shadow_tile_bytes(Hkv));
  return s;
}

int64_t decode_workspace_bytes(int max_waves, int group);
int64_t attention_workspace_bytes(int num_seqs, int max_seqlen_q, int max_seqlen_k, int num_heads,
                                  int num_kv_heads);
// Decode waves a paged call launches: whole groups of Hkv, its workspace
// bound (max_waves) and the device's resident wave slots, whichever is
// smaller.
int decode_launch_waves(int max_waves, int Hkv);
struct MergeJob;
struct CoDecode;
// The plan kernel; with `merge` it also runs the decode launch's merge of
// split rows (extra work-groups beside the plan's); with `co` it sizes the
// decode part of the prefill launch (PlanHeader::dec_wgs) and clears the
// decode waves' header.
int launch_plan(const AttnParams& P, const Plan& plan, bool paged, hipStream_t stream,
                const ShadowLayout* shadow = nullptr, const MergeJob* merge = nullptr,
                const CoDecode* co = nullptr);
// Rates the plan sizes the co-scheduled decode with: decode bytes per
// second of one CU beside the prefill and of the whole chip, prefill FLOP
// per second of one CU, and the fraction of the call by which the decode
// should end.
struct CoDecodeRates {
  float cu_bps, hbm_bps, pre_cu_flops, finish;
};
CoDecodeRates co_decode_rates(int cache_dtype);
// Dequantises the prefill rows' tiles into the copy (runs only where the
// plan set shadow_on).
int launch_shadow_fill(const AttnParams& P, const Plan& plan, const ShadowLayout& sh, hipStream_t stream);
// The decode kernel, then the merge of split rows: its own launch, or, with
// `defer`, left to the plan launch (defer receives what it needs).
int launch_decode(const AttnParams& P, int max_waves, int waves, void* partials, hipStream_t stream,
                  MergeJob* defer = nullptr);
// The decode waves' arguments (partials for max_waves waves at `partials`),
// and the merge of rows split across `groups` decode groups as a launch.
struct DecodeArgs;
DecodeArgs decode_args(const AttnParams& P, int max_waves, void* partials);
int launch_decode_merge(const DecodeArgs& a, int groups, hipStream_t stream);
int launch_prefill(const AttnParams& P, const Plan& plan, hipStream_t stream);
// The MFMA tile-loop prefill kernel (paged_prefill_mx.hip): whether it serves
// a call, its query positions per work item for a group of g query heads,
// and its launch.
bool prefill_mx_serves(const AttnParams& P);
int prefill_mx_positions(int g);
// With `co`, the launch's first work-groups stream the call's decode rows
// before they join the prefill (co->kv: the cache type of the decode rows,
// which a code cache's prefill reads through its bf16 copy); the plan has
// sized their number for co->wgs work-groups.
int launch_prefill_mx(const AttnParams& P, const Plan& plan, hipStream_t stream, const CoDecode* co = nullptr);

}  // namespace nvs
