// Planning kernel: compact decode / prefill work lists from cu_seqlens, on
// the device and without a host round trip.
#include "nvs_common.h"
#include "attention_common.h"

namespace nvs {

struct PlanArgs {
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* bt;  // paged calls only
  int64_t bt_stride;
  int64_t NB;
  int bs;
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

// Row b's work counts: decode partitions (q_len == 1 rows of a paged call)
// or prefill query tiles (every other row); also its first query row and key
// count.
__device__ __forceinline__ void row_work(const PlanArgs& a, int b, int& nd, int& np, int& q0, int& kl) {
  nd = np = 0;
  q0 = kl = 0;
  if (b >= a.B) return;
  q0 = a.cu_q[b];
  const int ql = a.cu_q[b + 1] - q0;
  kl = a.cu_k[b + 1] - a.cu_k[b];
  if (q0 < 0 || ql <= 0 || (int64_t)q0 + ql > a.T) return;  // malformed rows are skipped
  if (a.paged && ql == 1)
    nd = kl > 0 ? min((kl + kDecodePart - 1) / kDecodePart, a.plan.max_parts) : 1;
  else
    np = min((ql + a.plan.pbm - 1) / a.plan.pbm, a.plan.ntq);
}

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kPlanFastLevels = 512;  // prefill tiles per row the one-pass ordering serves

// The full record of decode entry i of a chunk whose rows' record offsets,
// first query rows and key counts sit in LDS.
__device__ __forceinline__ void fill_decode_record(const PlanArgs& a, DecodeItem* rec, int i, int b0,
                                                   const int* row_off, const int* row_q0,
                                                   const int* row_kl) {
  // Row: the last r with row_off[r] <= i (rows without records share the
  // next row's offset, so they never win).
  int lo = 0, hi = kPlanThreads - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (row_off[mid] <= i) lo = mid; else hi = mid - 1;
  }
  const int p = i - row_off[lo];
  const int b = b0 + lo, kl = row_kl[lo];
  const int kbeg = p * kDecodePart;
  const int kend = kl > 0 ? min(kbeg + kDecodePart, kl) : kl;
  const int lb0 = kbeg / a.bs;
  const int lb1 = kend > kbeg ? (kend - 1) / a.bs : lb0 - 1;
  DecodeItem r;
  r.q0 = row_q0[lo];
  r.b = b;
  r.p = p;
  r.kend = kend;
#pragma unroll
  for (int j = 0; j < kDecodeItemBlocks; ++j) {
    const int lblk = lb0 + j;
    int blk = -1;
    if (lblk <= lb1 && lblk < a.bt_stride) blk = a.bt[(int64_t)b * a.bt_stride + lblk];
    r.blk[j] = (blk >= 0 && blk < a.NB) ? blk : -1;
  }
  *rec = r;
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanArgs a) {
  __shared__ int scan_lds[kPlanWaves];
  __shared__ int row_off[kPlanThreads];
  __shared__ int row_q0[kPlanThreads];
  __shared__ int row_kl[kPlanThreads];
  __shared__ int lev_cnt[kPlanFastLevels * kPlanWaves];
  __shared__ int lev_off[kPlanFastLevels];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const Plan& pl = a.plan;
  if (tid < 8) pl.hdr->prefill_next[tid] = 0;

  // ---- decode records, 1024 rows at a time: scan the rows' partition
  // counts, stage the rows in LDS, then every thread fills whole records.
  int base = 0, deepest = 0, np0 = 0;
  for (int b0 = 0; b0 < a.B; b0 += kPlanThreads) {
    int nd, np, q0, kl, tot;
    row_work(a, b0 + tid, nd, np, q0, kl);
    if (b0 == 0) np0 = np;
    deepest = max(deepest, np);
    const int incl = block_scan_1024(nd, scan_lds, tot);
    row_off[tid] = incl - nd;
    row_q0[tid] = q0;
    row_kl[tid] = kl;
    __syncthreads();
    for (int i = tid; i < tot; i += kPlanThreads)
      fill_decode_record(a, pl.drec + base + i, i, b0, row_off, row_q0, row_kl);
    base += tot;
    __syncthreads();
  }
  if (tid == 0) pl.hdr->n_decode = base;

  // ---- prefill tiles level by level from the deepest query tile down, so
  // the heaviest tiles (most keys under the causal mask) of every row come
  // first; rows in order within a level.
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
  base = 0;
  for (int lev = nlev - 1; lev >= 0; --lev) {
    for (int b0 = 0; b0 < a.B; b0 += kPlanThreads) {
      const int b = b0 + tid;
      int nd, np, q0, kl, tot;
      row_work(a, b, nd, np, q0, kl);
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
  a.bt = P.bt;
  a.bt_stride = P.bt_stride;
  a.NB = P.NB;
  a.bs = P.bs > 0 ? P.bs : 1;
  a.B = P.B;
  a.T = P.T;
  a.paged = paged ? 1 : 0;
  a.plan = plan;
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(1024), 0, stream, a);
  return check_launch("plan");
}

}  // namespace nvs
