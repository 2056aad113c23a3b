// Step metadata on the device: what prepare_model_input builds on the host
// with a per-token Python loop (nanovllm/engine/model_runner.py:461-532).
//
// Per sequence b the host supplies num_cached[b] and num_new[b] (the
// Sequence fields the runner reads) and its block list, the lists
// concatenated in block_ids with sequence b's at block_offsets[b] ..
// block_offsets[b+1]-1; one launch then writes
//   cu_seqlens_q[b+1] = cu_seqlens_q[b] + num_new[b]                 (:497)
//   cu_seqlens_k[b+1] = cu_seqlens_k[b] + num_cached[b] + num_new[b] (:498)
//   context_lens[b]   = num_cached[b] + num_new[b]                   (:488)
//   for query token t of sequence b at position p = num_cached[b] + i:
//     positions[t]    = p                                            (:495)
//     slot_mapping[t] = block_table[b][p / bs] * bs + p % bs         (:503-507)
//   block_tables[b][j] = block_table[b][j], -1 past its end     (:334-344)
//
// Every work-group rescans the (at most kCtxMaxSeqs) per-sequence counts in
// LDS, so no work-group waits for another; a token finds its sequence by a
// binary search over cu_seqlens_q in LDS.  Work-group 0 also writes the
// per-sequence outputs; the padded table is written grid-stride by all.  A
// position past the end of its sequence's block list, or on a -1 entry, gets
// slot -1, which the KV store skips; the reference would fail on such a
// sequence (a list index error), and the host wrapper rejects it before the
// launch.  Offsets outside [0, num_block_ids] read as empty lists, so no
// argument makes the kernel read outside block_ids.
#include "nvs_common.h"

namespace nvs {
namespace {

constexpr int kCtxThreads = 1024;
constexpr int kCtxWaves = kCtxThreads / 64;
constexpr int kCtxPerThread = 4;  // sequences per thread in the scan
constexpr int kCtxMaxSeqs = kCtxThreads * kCtxPerThread;
constexpr int kCtxTokensPerThread = 4;
constexpr int kCtxTokensPerBlock = kCtxThreads * kCtxTokensPerThread;

struct CtxArgs {
  const int32_t* cached;
  const int32_t* fresh;
  const int32_t* boff;
  const int32_t* bids;
  int64_t n_bids;
  int32_t* table;
  int width;
  int32_t* cu_q;
  int32_t* cu_k;
  int32_t* ctx_lens;
  int32_t* slots;
  int64_t* positions;
  int64_t T;
  int B;
  int bs;
};

// Inclusive prefix sum of one int per lane across the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// Length of sequence b's block list; a decreasing pair of offsets is empty.
__device__ __forceinline__ int list_len(const int* s_boff, int b) {
  const int n = s_boff[b + 1] - s_boff[b];
  return n > 0 ? n : 0;
}

__global__ __launch_bounds__(kCtxThreads) void context_kernel(CtxArgs a) {
  __shared__ int s_cuq[kCtxMaxSeqs + 1];
  __shared__ int s_cached[kCtxMaxSeqs];
  __shared__ int s_boff[kCtxMaxSeqs + 1];
  __shared__ int s_wq[kCtxWaves], s_wk[kCtxWaves];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int base = tid * kCtxPerThread;
  for (int b = tid; b <= a.B; b += kCtxThreads) {
    const int o = a.boff[b];
    s_boff[b] = (o < 0 || o > a.n_bids) ? 0 : o;
  }

  // Each thread owns kCtxPerThread consecutive sequences: local sums, then a
  // block-wide exclusive scan of the per-thread totals.
  int nq[kCtxPerThread], nk[kCtxPerThread];
  int tq = 0, tk = 0;
#pragma unroll
  for (int i = 0; i < kCtxPerThread; ++i) {
    const int b = base + i;
    const int c = b < a.B ? a.cached[b] : 0;
    const int n = b < a.B ? a.fresh[b] : 0;
    if (b < a.B) s_cached[b] = c;
    nq[i] = n;
    nk[i] = c + n;
    tq += n;
    tk += c + n;
  }
  const int iq = wave_inclusive_scan(tq);
  const int ik = wave_inclusive_scan(tk);
  if (lane == 63) {
    s_wq[wave] = iq;
    s_wk[wave] = ik;
  }
  __syncthreads();
  int oq = 0, ok = 0;
  for (int w = 0; w < wave; ++w) {
    oq += s_wq[w];
    ok += s_wk[w];
  }
  int eq = oq + iq - tq, ek = ok + ik - tk;  // exclusive prefix of this thread
  const bool writer = blockIdx.x == 0;
#pragma unroll
  for (int i = 0; i < kCtxPerThread; ++i) {
    const int b = base + i;
    if (b < a.B) {
      s_cuq[b] = eq;
      if (writer) {
        a.cu_q[b] = eq;
        a.cu_k[b] = ek;
        a.ctx_lens[b] = nk[i];
      }
    }
    eq += nq[i];
    ek += nk[i];
  }
  // The thread holding the last sequence (thread 0 when there is none) ends
  // with the totals, entry B of both running sums.
  if (tid == (a.B > 0 ? (a.B - 1) / kCtxPerThread : 0)) {
    s_cuq[a.B] = eq;
    if (writer) {
      a.cu_q[a.B] = eq;
      a.cu_k[a.B] = ek;
    }
  }
  __syncthreads();

  const int total = s_cuq[a.B];
  const int64_t t0 = (int64_t)blockIdx.x * kCtxTokensPerBlock;
#pragma unroll
  for (int j = 0; j < kCtxTokensPerThread; ++j) {
    const int64_t t = t0 + (int64_t)j * kCtxThreads + tid;
    if (t >= a.T) break;
    int slot = -1;
    int64_t pos = 0;
    if (t < total) {
      // Largest b with cu_q[b] <= t: sequences with no new tokens are skipped.
      int lo = 0, hi = a.B - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_cuq[mid] <= (int)t) lo = mid; else hi = mid - 1;
      }
      pos = (int64_t)s_cached[lo] + (t - s_cuq[lo]);
      const int64_t blk = pos / a.bs;
      if (blk < list_len(s_boff, lo)) {
        const int id = a.bids[s_boff[lo] + blk];
        if (id >= 0) slot = (int)((int64_t)id * a.bs + (pos - blk * a.bs));
      }
    }
    a.slots[t] = slot;
    if (a.positions) a.positions[t] = pos;
  }

  if (a.table) {
    const int64_t cells = (int64_t)a.B * a.width;
    for (int64_t e = (int64_t)blockIdx.x * kCtxThreads + tid; e < cells; e += (int64_t)gridDim.x * kCtxThreads) {
      const int b = (int)(e / a.width);
      const int j = (int)(e - (int64_t)b * a.width);
      a.table[e] = j < list_len(s_boff, b) ? a.bids[s_boff[b] + j] : -1;
    }
  }
}

}  // namespace
}  // namespace nvs

using namespace nvs;

extern "C" int nvs_build_context(const int32_t* num_cached_tokens, const int32_t* num_new_tokens, int num_seqs,
                                 const int32_t* block_offsets, const int32_t* block_ids, int64_t num_block_ids,
                                 int block_size, int64_t num_tokens, int32_t* cu_seqlens_q,
                                 int32_t* cu_seqlens_k, int32_t* context_lens, int32_t* slot_mapping,
                                 int64_t* positions, int32_t* block_tables, int block_table_width,
                                 void* stream) {
  clear_error();
  const char* who = "build_context";
  NVS_REQUIRE(num_seqs >= 0 && num_seqs <= kCtxMaxSeqs, NVS_ERR_UNSUPPORTED,
              "%s: num_seqs %d outside [0, %d]", who, num_seqs, kCtxMaxSeqs);
  NVS_REQUIRE(num_tokens >= 0 && num_tokens < (1ll << 31), NVS_ERR_INVALID, "%s: num_tokens %lld out of range",
              who, (long long)num_tokens);
  NVS_REQUIRE(num_block_ids >= 0 && num_block_ids < (1ll << 31), NVS_ERR_INVALID,
              "%s: num_block_ids %lld out of range", who, (long long)num_block_ids);
  NVS_REQUIRE(block_size > 0, NVS_ERR_INVALID, "%s: block_size must be positive", who);
  NVS_REQUIRE(block_table_width >= 0, NVS_ERR_INVALID, "%s: negative block_table_width", who);
  NVS_REQUIRE(cu_seqlens_q && cu_seqlens_k && block_offsets, NVS_ERR_INVALID, "%s: null pointer argument", who);
  NVS_REQUIRE(num_seqs == 0 || (num_cached_tokens && num_new_tokens && context_lens), NVS_ERR_INVALID,
              "%s: null pointer argument", who);
  NVS_REQUIRE(num_block_ids == 0 || block_ids, NVS_ERR_INVALID, "%s: null block_ids", who);
  NVS_REQUIRE(num_tokens == 0 || slot_mapping, NVS_ERR_INVALID, "%s: null slot_mapping", who);
  NVS_REQUIRE(num_tokens == 0 || num_seqs > 0, NVS_ERR_INVALID, "%s: tokens without sequences", who);
  CtxArgs a;
  a.cached = num_cached_tokens; a.fresh = num_new_tokens;
  a.boff = block_offsets; a.bids = block_ids; a.n_bids = num_block_ids;
  a.table = (num_seqs > 0 && block_table_width > 0) ? block_tables : nullptr;
  a.width = block_table_width;
  a.cu_q = cu_seqlens_q; a.cu_k = cu_seqlens_k; a.ctx_lens = context_lens;
  a.slots = slot_mapping; a.positions = positions;
  a.T = num_tokens; a.B = num_seqs; a.bs = block_size;
  const int64_t by_tokens = (num_tokens + kCtxTokensPerBlock - 1) / kCtxTokensPerBlock;
  const int64_t by_cells = a.table ? ((int64_t)num_seqs * block_table_width + kCtxTokensPerBlock - 1) /
                                         kCtxTokensPerBlock : 0;
  const int64_t blocks = by_tokens > by_cells ? (by_tokens > 0 ? by_tokens : 1) : (by_cells > 0 ? by_cells : 1);
  hipLaunchKernelGGL(context_kernel, dim3((unsigned)blocks), dim3(kCtxThreads), 0, (hipStream_t)stream, a);
  return check_launch(who);
}
