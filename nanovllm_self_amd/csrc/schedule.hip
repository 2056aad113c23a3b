// Planning kernel: compact decode / prefill work lists from cu_seqlens, on
// the device and without a host round trip.
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

// Row b's work counts: decode partitions (q_len == 1 rows of a paged call)
// or prefill query tiles (every other row).
__device__ __forceinline__ void row_work(const PlanArgs& a, int b, int& nd, int& np) {
  nd = np = 0;
  if (b >= a.B) return;
  const int q0 = a.cu_q[b];
  const int ql = a.cu_q[b + 1] - q0;
  const int kl = a.cu_k[b + 1] - a.cu_k[b];
  if (q0 < 0 || ql <= 0 || (int64_t)q0 + ql > a.T) return;  // malformed rows are skipped
  if (a.paged && ql == 1)
    nd = kl > 0 ? min((kl + kDecodePart - 1) / kDecodePart, a.plan.max_parts) : 1;
  else
    np = min((ql + kPrefillBM - 1) / kPrefillBM, a.plan.ntq);
}

__global__ __launch_bounds__(1024) void plan_kernel(PlanArgs a) {
  __shared__ int lds[16];
  const int tid = threadIdx.x;
  const Plan& pl = a.plan;
  // Decode partitions, row by row.
  int base = 0, deepest = 0;
  for (int b0 = 0; b0 < a.B; b0 += 1024) {
    const int b = b0 + tid;
    int nd, np, tot;
    row_work(a, b, nd, np);
    deepest = max(deepest, np);
    const int incl = block_scan_1024(nd, lds, tot);
    for (int i = 0; i < nd; ++i) pl.dlist[base + incl - nd + i] = b * pl.max_parts + i;
    base += tot;
  }
  if (tid == 0) pl.hdr->n_decode = base;
  // Prefill tiles level by level from the deepest query tile down, so the
  // heaviest tiles (most keys under the causal mask) of every row come first.
  int nlev;
  {
    int v = deepest;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    if ((tid & 63) == 0) lds[tid >> 6] = v;
    __syncthreads();
    nlev = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) nlev = max(nlev, lds[i]);
    __syncthreads();
  }
  base = 0;
  for (int lev = nlev - 1; lev >= 0; --lev) {
    for (int b0 = 0; b0 < a.B; b0 += 1024) {
      const int b = b0 + tid;
      int nd, np, tot;
      row_work(a, b, nd, np);
      const int f = np > lev ? 1 : 0;
      const int incl = block_scan_1024(f, lds, tot);
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
