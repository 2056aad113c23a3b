// Split-K paged decode (q_len == 1 rows) for gfx950.
//
// Reference semantics: the q_len == 1 rows of prefill_flashattn's paged call
// (nanovllm/layers/attention.py:356-375) and of prefill_torch's prefix branch
// (:441-498): out[h] = softmax(q[h] . K^T * scale) V over the sequence's
// k_len cached keys, kv head h / (Hq / Hkv).
//
// Work decomposition (stream-K): decode work is counted in 32-key tiles of
// the decode rows, in row order (T in all).  Waves form Kw groups of Hkv,
// one wave per kv head; group k processes tiles [floor(k T / Kw),
// floor((k + 1) T / Kw)) as one continuous stream, so every wave has the
// same work, the load pipeline never restarts at row boundaries, and the Hkv
// waves of a group read the same token rows (each its 256-byte slice of a
// 2 KiB row) side by side.  A wave serves every query head of its kv head,
// so each K/V byte is read from HBM exactly once.  Per 32-key tile:
//   S^T[32 keys x 16 heads] = K[32 x 128] . Q^T   (8 x mfma_f32_16x16x32_bf16)
//   O^T[128 x 16 heads]    += V^T[128 x 32] . P^T (8 x mfma_f32_16x16x32_bf16)
// With keys as the MFMA row index, the S^T accumulator layout (lane = head
// column, 4 consecutive keys per lane group) is exactly the B-operand layout
// that P^T needs, so P never leaves registers.  V rows are loaded with full
// 256-byte coalescing and transposed in registers with v_perm_b32.  Quantised
// codes are converted to bf16 exactly in registers (int8 and e4m3 values are
// bf16-representable); the per-key scales multiply S (K) and P (V).
// A row that lies inside one group's range is normalised and written by the
// group's waves; a row split across groups leaves one partial (m, l,
// o[128]) per query head in each wave, merged by decode_merge_kernel with a
// log-sum-exp (a second launch: the kernel boundary makes the partials
// visible across XCDs without device-scope fences, which on a multi-XCD part
// write back the L2).  The group where a split row starts leaves a record
// (output row, last group, slot) for the merge, so the merge needs no scan
// of its own.
// Given the step's new k / v rows (nvs_paged_attention_store), the wave that
// owns a decode row's last tile also writes the row's new token into the
// cache (values, or codes and scales), ahead of its own load of that tile,
// when the row's slot is its own last position k_len - 1 under its block
// table (the slot the engine gives a decode row).  Every other slot is
// checked for on the device and written, before any load, by every wave that
// reads the cache (see write_nonconforming).
#include <algorithm>

#include "nvs_common.h"
#include "attention_common.h"
#include "store_common.h"
#include "decode_merge.h"
#include "decode_wave.h"

namespace nvs {

// Depth D of a decode wave's tile ring: the oldest tile is computed while
// the loads of the D - 1 after it are in flight.  D = 2 for every cache: a
// code tile carries half a bf16 tile's bytes, yet a third code tile in
// flight measured no faster (the stream is bound by HBM throughput, not by
// the bytes a wave keeps in flight).
#ifndef NVS_DECODE_RING_BF16
#define NVS_DECODE_RING_BF16 2
#endif
#ifndef NVS_DECODE_RING_CODES
#define NVS_DECODE_RING_CODES 2
#endif
template <int KV>
constexpr int kDecodeRing = kHalf<KV> ? NVS_DECODE_RING_BF16 : NVS_DECODE_RING_CODES;

// Launch index -> (kv head h, group k) with the group fastest: work-group i
// runs on XCD i % 8, so with a multiple of 8 launched groups the Hkv waves
// of a group share an XCD and their slices of each 2 KiB token row reach HBM
// together (7 % faster than one XCD per kv head, measured).
template <int KV>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kDecodeWavesPerEU)))
void paged_decode_kernel(DecodeArgs a, const int32_t* __restrict__ bt, const int32_t* __restrict__ cu_q,
                         const int32_t* __restrict__ cu_k) {
  const int G = gridDim.x / a.Hkv;
  const int h = blockIdx.x / G, k = blockIdx.x - h * G;
  decode_wave<KV, kDecodeRing<KV>>(a, bt, cu_q, cu_k, h, k, G, blockIdx.x, gridDim.x);
}

// The merge of split rows as a launch of its own (decode-only calls, and
// after a prefill launch that streamed the decode rows); calls whose decode
// has a launch of its own beside prefill rows run it in the plan launch
// (merge_split_row).
// Sixteen merge waves a work-group: a launch of a few large work-groups
// is dispatched sooner than one of many single-wave ones.
constexpr int kMergeWaves = 16;
__global__ __launch_bounds__(64 * kMergeWaves) void decode_merge_kernel(DecodeArgs a, int units) {
  const int unit = (int)blockIdx.x * kMergeWaves + (int)(threadIdx.x >> 6);
  if (unit < units) merge_split_row(a, __builtin_amdgcn_readfirstlane(unit), threadIdx.x & 63);
}

int64_t decode_workspace_bytes(int max_waves, int group) {
  // Partials, then a 4-int header and one 4-int record per wave (sized for
  // the most waves any call launches, so the size only grows with group).
  return (int64_t)max_waves * 2 * group * (kHeadDim + 2) * (int64_t)sizeof(float) +
         ((int64_t)kDecodeMaxWaves + 1) * 4 * (int64_t)sizeof(int32_t);
}

DecodeArgs decode_args(const AttnParams& P, int max_waves, void* partials) {
  DecodeArgs a;
  a.q = (const uint16_t*)P.q; a.q_ts = P.q_ts; a.q_hs = P.q_hs;
  a.kc = P.kc; a.vc = P.vc; a.ks = P.ks; a.vs = P.vs;
  a.bt_stride = (int)P.bt_stride; a.NB = (int)P.NB;
  a.Hq = P.Hq; a.Hkv = P.Hkv; a.g = P.Hq / P.Hkv; a.bs = P.bs;
  a.scale_log2 = P.softmax_scale * 1.4426950408889634f;
  a.cu_q = P.cu_q; a.cu_k = P.cu_k; a.B = P.B; a.T = P.T;
  a.kn = (const uint16_t*)P.kn; a.vn = (const uint16_t*)P.vn;
  a.kn_ts = P.kn_ts; a.kn_hs = P.kn_hs; a.vn_ts = P.vn_ts; a.vn_hs = P.vn_hs;
  a.slots = P.slots; a.total_slots = P.NB * (int64_t)P.bs;
  a.out = (uint16_t*)P.out; a.out_ts = P.out_ts; a.out_hs = P.out_hs;
  a.f16 = P.cache_dtype == NVS_DTYPE_FP16 ? 1 : 0;
  a.ws_o = (float*)partials;
  a.ws_ml = a.ws_o + (int64_t)max_waves * 2 * a.g * kHeadDim;
  a.ws_rec = (int32_t*)(a.ws_ml + (int64_t)max_waves * 2 * a.g * 2);
  return a;
}

int launch_decode_merge(const DecodeArgs& a, int groups, hipStream_t stream) {
  if (groups <= 1) return NVS_OK;
  const int units = (groups - 1) * a.Hkv;
  hipLaunchKernelGGL(decode_merge_kernel, dim3((units + kMergeWaves - 1) / kMergeWaves), dim3(64 * kMergeWaves), 0,
                     stream, a, units);
  return check_launch("decode_merge");
}

int launch_decode(const AttnParams& P, int max_waves, int waves, void* partials, hipStream_t stream,
                  MergeJob* defer) {
  if (defer) defer->units = 0;
  const DecodeArgs a = decode_args(P, max_waves, partials);
  if (waves <= 0) return NVS_OK;
  dim3 grid(waves), block(64);
  switch (P.cache_dtype) {
    case NVS_DTYPE_BF16:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_BF16>, grid, block, 0, stream, a, P.bt, P.cu_q, P.cu_k);
      break;
    case NVS_DTYPE_FP16:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_FP16>, grid, block, 0, stream, a, P.bt, P.cu_q, P.cu_k);
      break;
    case NVS_DTYPE_INT8:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_INT8>, grid, block, 0, stream, a, P.bt, P.cu_q, P.cu_k);
      break;
    case NVS_DTYPE_FP8_E4M3:
      hipLaunchKernelGGL(paged_decode_kernel<NVS_DTYPE_FP8_E4M3>, grid, block, 0, stream, a, P.bt, P.cu_q,
                         P.cu_k);
      break;
    default:
      set_error("paged_attention: decode does not serve cache dtype %d", P.cache_dtype);
      return NVS_ERR_UNSUPPORTED;
  }
  int rc = check_launch("paged_decode");
  if (rc != NVS_OK) return rc;
  // With one group no row is split (keyless rows were zeroed by the decode
  // kernel's scan).
  const int groups = waves / P.Hkv;
  if (defer) {  // the plan launch runs the merge
    defer->a = a;
    defer->units = groups > 1 ? (groups - 1) * P.Hkv : 0;
    return NVS_OK;
  }
  return launch_decode_merge(a, groups, stream);
}

}  // namespace nvs
