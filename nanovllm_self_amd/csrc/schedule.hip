// Planning kernel: the prefill work list from cu_seqlens, on the device and
// without a host round trip.
#include "nvs_common.h"
#include "attention_common.h"

namespace nvs {

struct PlanArgs {
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B;
  int64_t T;
  int paged;
  Plan plan;
};

// Inclusive scan of one int per thread over the 1024-thread work-group:
// shuffle scan inside each wave, then the 16 wave totals through LDS.  Also
// returns the work-group total.  Two barriers.
__device__ __forceinline__ int block_scan_1024(int v, int* lds, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  if (lane == 63) lds[w] = v;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int x = lds[i];
    before += i < w ? x : 0;
    all += x;
  }
  __syncthreads();
  total = all;
  return v + before;
}

// Row b's work: a decode row (q_len == 1 row of a paged call) or prefill
// query tiles (every other row); also its first query row and key count.
__device__ __forceinline__ void row_work(const PlanArgs& a, int b, bool& dec, int& np, int& q0, int& kl) {
  dec = false;
  np = 0;
  q0 = kl = 0;
  if (b >= a.B) return;
  q0 = a.cu_q[b];
  const int ql = a.cu_q[b + 1] - q0;
  kl = a.cu_k[b + 1] - a.cu_k[b];
  if (q0 < 0 || ql <= 0 || (int64_t)q0 + ql > a.T) return;  // malformed rows are skipped
  if (a.paged && ql == 1)
    dec = true;
  else
    np = min((ql + a.plan.pbm - 1) / a.plan.pbm, a.plan.ntq);
}

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kPlanFastLevels = 512;  // prefill tiles per row the one-pass ordering serves

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanArgs a) {
  __shared__ int scan_lds[kPlanWaves];
  __shared__ int lev_cnt[kPlanFastLevels * kPlanWaves];
  __shared__ int lev_off[kPlanFastLevels];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const Plan& pl = a.plan;
  if (tid < 8) pl.hdr->prefill_next[tid] = 0;

  // ---- prefill tiles level by level from the deepest query tile down, so
  // the heaviest tiles (most keys under the causal mask) of every row come
  // first; rows in order within a level.
  int deepest = 0, np0 = 0;
  for (int b0 = 0; b0 < a.B; b0 += kPlanThreads) {
    bool dec;
    int np, q0, kl;
    row_work(a, b0 + tid, dec, np, q0, kl);
    if (b0 == 0) np0 = np;
    deepest = max(deepest, np);
  }
  int nlev;
  {
    int v = deepest;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    if (lane == 0) scan_lds[w] = v;
    __syncthreads();
    nlev = 0;
#pragma unroll
    for (int i = 0; i < kPlanWaves; ++i) nlev = max(nlev, scan_lds[i]);
    __syncthreads();
  }
  if (a.B <= kPlanThreads && nlev <= kPlanFastLevels) {
    // One pass: per (level, wave) counts by ballot, their prefixes over waves
    // and over deeper levels, then each row writes its tiles directly.
    for (int lev = 0; lev < nlev; ++lev) {
      const int c = __popcll(__ballot(np0 > lev));
      if (lane == 0) lev_cnt[lev * kPlanWaves + w] = c;
    }
    __syncthreads();
    for (int lev = tid; lev < nlev; lev += kPlanThreads) {
      int run = 0;
#pragma unroll
      for (int x = 0; x < kPlanWaves; ++x) {
        const int c = lev_cnt[lev * kPlanWaves + x];
        lev_cnt[lev * kPlanWaves + x] = run;
        run += c;
      }
      lev_off[lev] = run;  // level total, turned into its offset below
    }
    __syncthreads();
    const int lev = nlev - 1 - tid;  // deepest level first
    const int v = lev >= 0 ? lev_off[lev] : 0;
    int total;
    const int incl = block_scan_1024(v, scan_lds, total);
    if (lev >= 0) lev_off[lev] = incl - v;
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int l = 0; l < nlev; ++l) {
      const uint64_t m = __ballot(np0 > l);
      if (np0 > l)
        pl.plist[lev_off[l] + lev_cnt[l * kPlanWaves + w] + __popcll(m & below)] = tid * pl.ntq + l;
    }
    if (tid == 0) pl.hdr->n_prefill = total;
    return;
  }
  // General case: one block scan per (level, chunk of rows).
  int base = 0;
  for (int lev = nlev - 1; lev >= 0; --lev) {
    for (int b0 = 0; b0 < a.B; b0 += kPlanThreads) {
      const int b = b0 + tid;
      bool dec;
      int np, q0, kl, tot;
      row_work(a, b, dec, np, q0, kl);
      const int f = np > lev ? 1 : 0;
      const int incl = block_scan_1024(f, scan_lds, tot);
      if (f) pl.plist[base + incl - 1] = b * pl.ntq + lev;
      base += tot;
    }
  }
  if (tid == 0) pl.hdr->n_prefill = base;
}

static int g_cus[64] = {0};

int device_slots(int per_cu) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev] * per_cu;
}

int launch_plan(const AttnParams& P, const Plan& plan, bool paged, hipStream_t stream) {
  PlanArgs a;
  a.cu_q = P.cu_q;
  a.cu_k = P.cu_k;
  a.B = P.B;
  a.T = P.T;
  a.paged = paged ? 1 : 0;
  a.plan = plan;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(1024), 0, stream, a);
  return check_launch("plan");
}

}  // namespace nvs
