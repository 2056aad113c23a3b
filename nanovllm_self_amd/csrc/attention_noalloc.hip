// Allocation-free variant of nvs_paged_attention_store for callers that may
// not allocate device memory (code under HIP-graph capture, tight serving
// loops, hosts that forbid hipMalloc): the workspace (the prefill work plan
// and the decode partials of rows split across wave groups) comes from a
// file-scope static device array instead of a caller argument.
//
// The array holds kScratchBytes on every GPU the library is loaded on, for
// the life of the process.  Its device address is looked up once per device
// (hipGetSymbolAddress, on the entry point's first call with that device
// current) and only that address is ever passed to kernels: the array's name
// in host code is a host-side stand-in, not a device pointer.  Every call on
// one GPU shares that GPU's array, so calls that overlap on one GPU (on
// different streams, or from different threads) race; calls ordered on one
// stream do not.  Nothing in the array needs to start at zero: the plan
// kernel clears the prefill work counters and the decode kernel writes its
// records before the merge reads them, on every call.
#include <atomic>
#include <mutex>

#include "nvs_common.h"
#include "attention_common.h"

namespace {

constexpr int64_t kScratchBytes = NVS_NOALLOC_SCRATCH_BYTES;  // 32 MiB per device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> g_scratch[kMaxDevices];  // per-device address of `scratch`
std::mutex g_scratch_mu;

// Device address of the current device's copy of `scratch`.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  NVS_REQUIRE(e == hipSuccess, NVS_ERR_LAUNCH, "paged_attention_store_noalloc: hipGetDevice failed: %s",
              hipGetErrorString(e));
  NVS_REQUIRE(dev >= 0 && dev < kMaxDevices, NVS_ERR_UNSUPPORTED,
              "paged_attention_store_noalloc: device %d beyond the %d devices served", dev, kMaxDevices);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      NVS_REQUIRE(e == hipSuccess && p, NVS_ERR_LAUNCH,
                  "paged_attention_store_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
      NVS_REQUIRE(((uintptr_t)p % 256) == 0, NVS_ERR_LAUNCH,
                  "paged_attention_store_noalloc: scratch on device %d is not 256-byte aligned", dev);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return NVS_OK;
}

}  // namespace

extern "C" int nvs_paged_attention_store_noalloc(
    const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k, const void* v, int src_dtype,
    int64_t k_tok_stride, int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
    const int32_t* slot_mapping, void* k_cache, void* v_cache, int cache_dtype, float* k_scale, float* v_scale,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, const int32_t* block_tables, int64_t bt_stride,
    int num_seqs, int64_t num_tokens, int max_seqlen_q, int max_seqlen_k, int num_heads, int num_kv_heads,
    int head_dim, int block_size, int64_t num_blocks, float softmax_scale, void* out, int64_t out_tok_stride,
    int64_t out_head_stride, void* stream) {
  nvs::clear_error();
  const int64_t need =
      nvs::attention_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads);
  NVS_REQUIRE(need <= kScratchBytes, NVS_ERR_WORKSPACE,
              "paged_attention_store_noalloc: this batch needs %lld bytes of scratch, more than the "
              "library's static %lld (call nvs_paged_attention_store with a workspace instead)",
              (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != NVS_OK) return rc;
  return nvs_paged_attention_store(q, q_tok_stride, q_head_stride, k, v, src_dtype, k_tok_stride, k_head_stride,
                                   v_tok_stride, v_head_stride, slot_mapping, k_cache, v_cache, cache_dtype,
                                   k_scale, v_scale, cu_seqlens_q, cu_seqlens_k, block_tables, bt_stride, num_seqs,
                                   num_tokens, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim,
                                   block_size, num_blocks, softmax_scale, out, out_tok_stride, out_head_stride, ws,
                                   kScratchBytes, stream);
}
