// Planning kernel: the prefill work list from cu_seqlens, on the device and
// without a host round trip.
#include "nvs_common.h"
#include "attention_common.h"
#include "decode_merge.h"

namespace nvs {

struct PlanArgs {
  const int32_t* cu_q;
  const int32_t* cu_k;
  int B;
  int64_t T;
  int paged;
  const int32_t* bt;  // paged: block tables
  int64_t bt_stride;
  int64_t NB;
  int bs;
  Plan plan;
  int* shadow_base;  // code caches: per-row first tile of the bf16 copy (null: no copy)
  int shadow_cap;
  int shadow_st;     // tiles of a table row: a row's tiles past it are not copied
  int64_t Tk;        // rows of the local k / v (local mode)
  // Decode rows streamed by the prefill launch's first work-groups (co_wgs
  // > 0: the launch's work-group count; 0: the decode has a launch of its
  // own).  The plan picks how many from the decode bytes and the prefill
  // FLOPs at the per-CU rates below.
  int co_wgs;
  int32_t* dec_rec;  // the decode waves' header (T, Kw), zeroed here: with no decode work-group the
                     // merge after the prefill launch must find no groups, not a stale count
  int Hq, Hkv;
  float dec_tile_bytes;  // HBM bytes of one 32-key decode tile over all kv heads
  float dec_cu_bps;      // decode bytes per second one CU streams beside the prefill
  float dec_hbm_bps;     // decode bytes per second of the whole chip
  float pre_cu_flops;    // prefill FLOP per second of one CU
  float dec_finish;      // the decode should end by this fraction of the call
};

// Tiles of the bf16 copy for a prefill row with kl keys.
__device__ __forceinline__ int shadow_row_tiles(const PlanArgs& a, int np, int kl) {
  return np > 0 && kl > 0 ? min((kl + kShadowTile - 1) / kShadowTile, a.shadow_st) : 0;
}

// Block id of the tile of keys [64 t, 64 t + 64) of row b: -1 past the
// row's blocks or outside the pool.
__device__ __forceinline__ int tile_block(const PlanArgs& a, int b, int kl, int t) {
  const int lb = 64 * t / a.bs;
  const int64_t nblk = min((int64_t)(kl + a.bs - 1) / a.bs, a.bt_stride);
  if (lb >= nblk) return -1;
  const int blk = a.bt[(int64_t)b * a.bt_stride + lb];
  return (blk >= 0 && blk < a.NB) ? blk : -1;
}

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

// Sums of three floats per thread over the 1024-thread work-group (every
// thread gets them).  Two barriers.
__device__ __forceinline__ void block_sum3_1024(float (&v)[3], float (*lds)[3]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v[i] += __shfl_xor(v[i], off, 64);
  if (lane == 0)
    for (int i = 0; i < 3; ++i) lds[w][i] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float all = 0.0f;
#pragma unroll
    for (int x = 0; x < kPlanWaves; ++x) all += lds[x][i];
    v[i] = all;
  }
  __syncthreads();
}

// Query-key pairs of a prefill row with L new and K visible keys under the
// causal mask (row r sees keys j <= r + K - L).
__device__ __forceinline__ float causal_pairs(int L, int K) {
  const float off = (float)(K - L);
  return K >= L ? (float)L * off + 0.5f * (float)L * (float)(L + 1) : 0.5f * (float)K * (float)(K + 1);
}

// Work-groups of the prefill launch that stream the decode rows before they
// join the prefill: the fewest whose decode, at dec_cu_bps a CU and at most
// dec_hbm_bps in all, ends by dec_finish of the call's estimated time (the
// prefill's CU time, its FLOPs at pre_cu_flops a CU, plus the decode's,
// shared by all work-groups); all of them when none does; none without
// decode rows.  Counts step in multiples of 8 (as many on every XCD) and of
// 2 Hkv (an XCD's decode waves form whole groups: at 24 work-groups and Hkv
// = 8 a third of them idled) when the launch holds such a step.
__device__ int pick_decode_wgs(const PlanArgs& a, float dec_rows, float dec_tiles, float pairs) {
  if (a.co_wgs <= 0 || dec_rows <= 0.0f) return 0;  // a keyless decode row still needs its zeros
  const int top = a.co_wgs & ~7;
  int step = 8;
  while (step % (2 * a.Hkv) != 0 && step <= top) step += 8;
  if (step > top) step = 8;
  const int lo = min(top, max(step, (2 * a.Hkv + 7) & ~7));
  const float bytes = dec_tiles * a.dec_tile_bytes;
  const float pre = pairs * 4.0f * (float)a.Hq * (float)kHeadDim / a.pre_cu_flops;  // CU seconds
  for (int nd = lo; nd <= top; nd += step) {
    const float td = bytes / fminf((float)nd * a.dec_cu_bps, a.dec_hbm_bps);
    const float t = (pre + (float)nd * td) / (float)a.co_wgs;
    if (td <= a.dec_finish * t) return nd;
  }
  return top;
}

// What the plan keeps of each row of a 1024-row step in LDS while the
// step's list entries are written, one entry per thread.
struct PlanRows {
  int end[kPlanThreads];  // inclusive prefix of the rows' entry counts
  int q0[kPlanThreads], L[kPlanThreads], k0[kPlanThreads], K[kPlanThreads];
  int blk[3][kPlanThreads];
};

// Work-group 0 writes the plan; the others (a paged call whose decode
// launch left its merge to this one) merge the decode rows split across
// groups, one merge wave per wave.
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanArgs a, DecodeArgs m, int merge_units) {
  if (blockIdx.x > 0) {
    const int unit = (blockIdx.x - 1) * kPlanWaves + (threadIdx.x >> 6);
    if (unit < merge_units) merge_split_row(m, __builtin_amdgcn_readfirstlane(unit), threadIdx.x & 63);
    return;
  }
  __shared__ int scan_lds[kPlanWaves];
  __shared__ float sum_lds[kPlanWaves][3];
  __shared__ PlanRows rows;
  const int tid = threadIdx.x;
  const Plan& pl = a.plan;
  if (tid < 8) pl.hdr->prefill_next[tid] = 0;
  // ---- code caches: the prefill rows' 64-key tiles of the bf16 copy, row
  // by row (an exclusive scan of ceil(k_len / 64)); the copy serves the call
  // if they fit.
  bool shadow = false;
  if (a.shadow_base) {
    int sbase = 0;
    for (int b0 = 0; b0 < a.B; b0 += kPlanThreads) {
      bool dec;
      int np, q0, kl, tot;
      row_work(a, b0 + tid, dec, np, q0, kl);
      const int nt = shadow_row_tiles(a, np, kl);
      const int incl = block_scan_1024(nt, scan_lds, tot);
      if (b0 + tid < a.B) a.shadow_base[b0 + tid] = sbase + incl - nt;
      sbase += tot;
    }
    shadow = sbase <= a.shadow_cap;
    if (tid == 0) {
      a.shadow_base[a.B] = sbase;
      pl.hdr->shadow_tiles = sbase;
      pl.hdr->shadow_on = shadow ? 1 : 0;
    }
  } else if (tid == 0) {
    pl.hdr->shadow_tiles = 0;
    pl.hdr->shadow_on = 0;
  }
  // ---- prefill tiles row by row (1024 rows per step: a scan of the rows'
  // tile counts), each row's tiles deepest first (most keys under the causal
  // mask).  Row-major order keeps the work-groups of an XCD on the same
  // sequence at the same time, so the K/V tiles they all read come from HBM
  // once and from L2 after that.  Each thread then writes entries e, e +
  // 1024, ... of the step, finding its row by a binary search of the prefix.
  int base = 0;
  // this thread's rows: decode rows and their tiles, prefill query-key pairs
  float dec_rows = 0.0f, dec_tiles = 0.0f, pairs = 0.0f;
  for (int b0 = 0; b0 < a.B; b0 += kPlanThreads) {
    bool dec;
    int np, q0, kl, tot;
    const int b = b0 + tid;
    row_work(a, b, dec, np, q0, kl);
    if (dec) dec_rows += 1.0f;
    if (dec && kl > 0) dec_tiles += (float)((kl + kDecodeTile - 1) / kDecodeTile);
    if (np > 0) pairs += causal_pairs(a.cu_q[b + 1] - q0, kl);
    const int incl = block_scan_1024(np, scan_lds, tot);
    rows.end[tid] = incl;
    if (np > 0) {
      rows.q0[tid] = q0;
      rows.L[tid] = a.cu_q[b + 1] - q0;
      rows.k0[tid] = a.cu_k[b];
      rows.K[tid] = kl;
      if (shadow) {  // tiles of the copy (the thread wrote shadow_base[b] itself)
        const int sb = a.shadow_base[b], nt = shadow_row_tiles(a, np, kl);
        for (int t = 0; t < 3; ++t) rows.blk[t][tid] = t < nt ? sb + t : -1;
      } else {
        for (int t = 0; t < 3; ++t) rows.blk[t][tid] = a.paged ? tile_block(a, b, kl, t) : -1;
      }
    }
    __syncthreads();
    for (int e = tid; e < tot; e += kPlanThreads) {
      int lo = 0, hi = kPlanThreads - 1;  // the first row whose prefix passes e
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (rows.end[mid] > e) hi = mid; else lo = mid + 1;
      }
      const int r = lo, rb = b0 + r;
      const int qt = rows.end[r] - 1 - e;  // the row's first entry is its deepest tile
      PlanRecord rec;
      rec.q0 = rows.q0[r];
      rec.L = rows.L[r];
      rec.k0 = rows.k0[r];
      rec.K = rows.K[r];
      rec.blk0 = rows.blk[0][r];
      rec.blk1 = rows.blk[1][r];
      rec.blk2 = rows.blk[2][r];
      // What the MFMA kernel derives per entry.  The table it reads is the
      // copy's (64-key tiles, shadow_st a row) when the copy serves the call.
      rec.off = rec.K - rec.L;
      rec.b = rb;
      if (a.paged) {
        rec.k0c = 0;
        rec.kf = rec.K;
        const int tbs = shadow ? kShadowTile : a.bs;
        const int64_t tst = shadow ? a.shadow_st : a.bt_stride;
        rec.bt_bytes = 4 * (int)min((int64_t)(rec.K + tbs - 1) / tbs, tst);
      } else {
        const int64_t k0c = min(max((int64_t)rec.k0, (int64_t)0), a.Tk);
        rec.k0c = (int)k0c;
        rec.kf = (int)max((int64_t)0, min((int64_t)rec.K, a.Tk - k0c));
        rec.bt_bytes = 0;
      }
      rec.pad = 0;
      rec.item = rb * pl.ntq + qt;
      rec.p0 = qt * pl.pbm;
      const int p_last = min(rec.L, rec.p0 + pl.pbm) - 1;
      const int kv_end = min(rec.K, p_last + rec.off + 1);
      rec.ntiles = (rec.p0 < rec.L && kv_end > 0) ? (kv_end + 63) / 64 : 0;
      pl.plist[base + e] = rec.item;
      pl.rec[base + e] = rec;
    }
    __syncthreads();  // the next step's rows overwrite the LDS
    base += tot;
  }
  if (tid == 0) pl.hdr->n_prefill = base;
  if (a.co_wgs > 0) {
    if (tid < 2) a.dec_rec[tid] = 0;
    float sums[3] = {dec_rows, dec_tiles, pairs};
    block_sum3_1024(sums, sum_lds);
    if (tid == 0) pl.hdr->dec_wgs = pick_decode_wgs(a, sums[0], sums[1], sums[2]);
  } else if (tid == 0) {
    pl.hdr->dec_wgs = 0;
  }
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

int launch_plan(const AttnParams& P, const Plan& plan, bool paged, hipStream_t stream, const ShadowLayout* shadow,
                const MergeJob* merge, const CoDecode* co) {
  PlanArgs a;
  a.cu_q = P.cu_q;
  a.cu_k = P.cu_k;
  a.B = P.B;
  a.T = P.T;
  a.paged = paged ? 1 : 0;
  a.bt = P.bt;
  a.bt_stride = P.bt_stride;
  a.NB = P.NB;
  a.bs = P.bs > 0 ? P.bs : 64;
  a.plan = plan;
  a.shadow_base = shadow ? shadow->base : nullptr;
  a.shadow_cap = shadow ? shadow->cap : 0;
  a.shadow_st = shadow ? shadow->ST : 0;
  a.Tk = P.Tk;
  a.co_wgs = co ? co->wgs : 0;
  a.dec_rec = co ? co->a.ws_rec : nullptr;
  a.Hq = P.Hq;
  a.Hkv = P.Hkv;
  const float esz = (P.cache_dtype == NVS_DTYPE_BF16 || P.cache_dtype == NVS_DTYPE_FP16) ? 2.0f : 1.0f;
  a.dec_tile_bytes = (float)kDecodeTile * P.Hkv * (2.0f * kHeadDim * esz + (esz < 2.0f ? 8.0f : 0.0f));
  const CoDecodeRates r = co_decode_rates(P.cache_dtype);
  a.dec_cu_bps = r.cu_bps;
  a.dec_hbm_bps = r.hbm_bps;
  a.pre_cu_flops = r.pre_cu_flops;
  a.dec_finish = r.finish;
  DecodeArgs m = {};
  int units = 0;
  if (merge && merge->units > 0) {
    m = merge->a;
    units = merge->units;
  }
  const int grid = 1 + (units + kPlanWaves - 1) / kPlanWaves;
  hipLaunchKernelGGL(plan_kernel, dim3(grid), dim3(kPlanThreads), 0, stream, a, m, units);
  return check_launch("plan");
}

}  // namespace nvs
