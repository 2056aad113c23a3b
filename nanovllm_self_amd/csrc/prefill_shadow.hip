// The bf16 copy of a code cache's prefill keys and values that the MFMA
// tile-loop prefill kernel reads (layout and capacity: ShadowLayout in
// attention_common.h).
//
// Reference semantics: prefill_torch's dequantisation of a sequence's cached
// keys and values (nanovllm/layers/attention.py:268-273, 100-117):
// (code.float() * scale.float()).to(bf16), per token and kv head, with
// missing blocks read as zeros (the eager gather pads them with zeros).
//
// Work: tile s (64 consecutive keys of one prefill row, every kv head, K and
// V), or half of it when the copy has fewer tiles than work-groups, per
// work-group iteration; the plan kernel numbered the tiles row by row
// (ShadowLayout::base).  A work-group finds the row of its tile by a binary
// search over those numbers, writes the table entry (first half), and
// converts its token rows of K and of V: 16 lanes to a row (8 codes, one
// 8-byte load, a 16-byte store each), 16 rows per pass of 256 threads.
// Keys past the row's length are not written (the prefill kernel never
// reads them).
#include <algorithm>

#include "nvs_common.h"
#include "attention_common.h"

namespace nvs {

namespace {

constexpr int kShadowThreads = 256;

struct ShadowArgs {
  const uint8_t* kc;
  const uint8_t* vc;
  const float* ks;
  const float* vs;
  const int32_t* bt;
  int64_t bt_stride;
  int64_t NB;
  int bs;
  const int32_t* cu_k;
  int B, Hkv;
  const PlanHeader* hdr;
  ShadowLayout sh;
};

// Eight codes (bytes of w) times the row's scale, rounded to bf16 (one
// conversion per pair, round-to-nearest-even as torch's .to(bf16)).
template <int KV>
__device__ __forceinline__ u32x4 dequant8(u32x2 w, float sc) {
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float f0, f1;
    if (i & 1)
      code_pair_to_f32<KV, true>(w[i >> 1], f0, f1);
    else
      code_pair_to_f32<KV, false>(w[i >> 1], f0, f1);
    o[i] = pack_bf16x2(f0 * sc, f1 * sc);
  }
  return o;
}

template <int KV>
__global__ __launch_bounds__(kShadowThreads) void shadow_fill_kernel(ShadowArgs a) {
  if (a.hdr->shadow_on == 0) return;
  const int total = a.hdr->shadow_tiles;
  const int j = threadIdx.x & 15;
  const int rows = kShadowTile * a.Hkv;  // token rows of a tile (token-major, then kv head)
  // A copy whose half tiles (32 keys x Hkv token rows) all fit one pass of
  // the grid is cut into them, so that it spreads over twice as many
  // work-groups (mixed_32b's 504 tiles: 45.7 -> 38.3 us); a larger one keeps
  // whole tiles (prefill_8b's 833 tiles as half tiles: 49.3 -> 53.5 us).
  const int split = 2 * total <= (int)gridDim.x ? 2 : 1;
  for (int u = blockIdx.x; u < split * total; u += gridDim.x) {
    const int s = split == 2 ? u >> 1 : u, half = split == 2 ? u & 1 : 0;
    // Row b of tile s: base[b] <= s < base[b + 1] (base is non-decreasing
    // with base[B] = total > s, so the largest such b has tiles).
    int lo = 0, hi = a.B;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.sh.base[mid] <= s) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int t = s - a.sh.base[b];  // < ST: the plan keeps a row's tiles within its table row
    if (threadIdx.x == 0 && half == 0) a.sh.table[(int64_t)b * a.sh.ST + t] = s;
    const int K = a.cu_k[b + 1] - a.cu_k[b];
    // The tile's keys lie in one block (block_size is a multiple of 64).
    const int lb = kShadowTile * t / a.bs;
    const int64_t nblk = min(((int64_t)K + a.bs - 1) / a.bs, a.bt_stride);
    int blk = lb < nblk ? a.bt[(int64_t)b * a.bt_stride + lb] : -1;
    if (blk >= a.NB) blk = -1;
    const int64_t row0 = blk >= 0 ? ((int64_t)blk * a.bs + (kShadowTile * t) % a.bs) * a.Hkv : 0;
    const int keys = min(K - kShadowTile * t, kShadowTile);
    const int64_t out0 = (int64_t)s * rows;
    const int span = kShadowTile / split;  // keys of the work item
    const int r_end = min(keys, span * (half + 1)) * a.Hkv;
    for (int r = span * half * a.Hkv + (threadIdx.x >> 4); r < r_end; r += kShadowThreads / 16) {
      u32x4 ko = {0u, 0u, 0u, 0u}, vo = {0u, 0u, 0u, 0u};
      if (blk >= 0) {
        const int64_t cr = row0 + r;  // cache row (token, kv head)
        const u32x2 kw = *reinterpret_cast<const u32x2*>(a.kc + cr * kHeadDim + 8 * j);
        const u32x2 vw = *reinterpret_cast<const u32x2*>(a.vc + cr * kHeadDim + 8 * j);
        ko = dequant8<KV>(kw, a.ks[cr]);
        vo = dequant8<KV>(vw, a.vs[cr]);
      }
      *reinterpret_cast<u32x4*>(a.sh.k + (out0 + r) * kHeadDim + 8 * j) = ko;
      *reinterpret_cast<u32x4*>(a.sh.v + (out0 + r) * kHeadDim + 8 * j) = vo;
    }
  }
}

}  // namespace

int launch_shadow_fill(const AttnParams& P, const Plan& plan, const ShadowLayout& sh, hipStream_t stream) {
  ShadowArgs a;
  a.kc = (const uint8_t*)P.kc;
  a.vc = (const uint8_t*)P.vc;
  a.ks = P.ks;
  a.vs = P.vs;
  a.bt = P.bt;
  a.bt_stride = P.bt_stride;
  a.NB = P.NB;
  a.bs = P.bs;
  a.cu_k = P.cu_k;
  a.B = P.B;
  a.Hkv = P.Hkv;
  a.hdr = plan.hdr;
  a.sh = sh;
  if (P.B <= 0 || sh.cap <= 0) return NVS_OK;
  // Persistent: a few work-groups per CU, never more than the copy's half tiles.
  const int wgs = (int)std::min<int64_t>(2 * (int64_t)sh.cap, (int64_t)device_slots(4));
  dim3 grid((unsigned)std::max(1, wgs)), block(kShadowThreads);
  switch (P.cache_dtype) {
    case NVS_DTYPE_INT8:
      hipLaunchKernelGGL(shadow_fill_kernel<NVS_DTYPE_INT8>, grid, block, 0, stream, a);
      break;
    case NVS_DTYPE_FP8_E4M3:
      hipLaunchKernelGGL(shadow_fill_kernel<NVS_DTYPE_FP8_E4M3>, grid, block, 0, stream, a);
      break;
    default:
      set_error("paged_attention: no bf16 copy for cache dtype %d", P.cache_dtype);
      return NVS_ERR_UNSUPPORTED;
  }
  return check_launch("shadow_fill");
}

}  // namespace nvs
