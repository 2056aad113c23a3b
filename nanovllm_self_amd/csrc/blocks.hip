// Whole-block copies between a paged cache and a packed block snapshot: the
// KV handoff of prefill/decode disaggregation (pd_self/kv_connector.py).
//
//   export  kv_cache[:, :, src_block_ids]      (_export_kv_snapshot :94-110)
//   import  kv_cache[:, :, dst_block_ids[i]] = blocks[:, :, i]
//                                               (load_kv_item :282-311)
//
// The caches are [planes, num_blocks, block] arrays of bytes (planes = 2 x
// layers; a block is block_size x kv_heads x head_dim codes, or the
// block_size x kv_heads fp32 scales), so one kernel serves bf16, fp16, fp32,
// int8 and fp8 codes and the scales alike.  Work item = one 16 KiB chunk of
// one block of one plane: each of 256 threads issues four 16 B loads, then
// the four stores, so four loads per thread are in flight.  Copies must not
// overlap each other (distinct destination blocks, source and destination
// regions disjoint): the work-groups run in no particular order.
#include "nvs_common.h"

namespace nvs {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;
constexpr int64_t kCopyStep = kCopyThreads * 16;
constexpr int64_t kChunk = kCopyStep * kCopyUnroll;

struct CopyArgs {
  const char* src;
  char* dst;
  const int32_t* src_ids;  // NULL: copy i reads block i
  const int32_t* dst_ids;  // NULL: copy i writes block i
  int64_t src_nb, dst_nb;
  int64_t block_bytes;
  int64_t chunks;  // chunks per block
  int64_t copies;
  int64_t items;   // planes * copies * chunks
};

__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(CopyArgs a) {
  for (int64_t it = blockIdx.x; it < a.items; it += gridDim.x) {
    const int64_t chunk = it % a.chunks;
    const int64_t pc = it / a.chunks;
    const int64_t i = pc % a.copies;
    const int64_t plane = pc / a.copies;
    const int64_t s = a.src_ids ? a.src_ids[i] : i;
    const int64_t d = a.dst_ids ? a.dst_ids[i] : i;
    if (s < 0 || s >= a.src_nb || d < 0 || d >= a.dst_nb) continue;  // uniform per work-group
    const char* from = a.src + (plane * a.src_nb + s) * a.block_bytes;
    char* to = a.dst + (plane * a.dst_nb + d) * a.block_bytes;
    const int64_t base = chunk * kChunk + threadIdx.x * 16;
    u32x4 v[kCopyUnroll];
#pragma unroll
    for (int k = 0; k < kCopyUnroll; ++k) {
      const int64_t off = base + k * kCopyStep;
      if (off < a.block_bytes) v[k] = __builtin_nontemporal_load((const u32x4*)(from + off));
    }
#pragma unroll
    for (int k = 0; k < kCopyUnroll; ++k) {
      const int64_t off = base + k * kCopyStep;
      if (off < a.block_bytes) *(u32x4*)(to + off) = v[k];
    }
  }
}

}  // namespace
}  // namespace nvs

using namespace nvs;

extern "C" int nvs_copy_blocks(const void* src, int64_t src_num_blocks, const int32_t* src_block_ids,
                               void* dst, int64_t dst_num_blocks, const int32_t* dst_block_ids,
                               int64_t num_planes, int64_t block_bytes, int64_t num_copies, void* stream) {
  clear_error();
  const char* who = "copy_blocks";
  NVS_REQUIRE(num_planes >= 0 && num_copies >= 0 && src_num_blocks >= 0 && dst_num_blocks >= 0,
              NVS_ERR_INVALID, "%s: negative size", who);
  NVS_REQUIRE(block_bytes > 0 && block_bytes % 16 == 0, NVS_ERR_INVALID,
              "%s: block_bytes %lld must be a positive multiple of 16", who, (long long)block_bytes);
  NVS_REQUIRE(src_block_ids || num_copies <= src_num_blocks, NVS_ERR_INVALID,
              "%s: %lld copies from a %lld-block source without ids", who, (long long)num_copies,
              (long long)src_num_blocks);
  NVS_REQUIRE(dst_block_ids || num_copies <= dst_num_blocks, NVS_ERR_INVALID,
              "%s: %lld copies into a %lld-block destination without ids", who, (long long)num_copies,
              (long long)dst_num_blocks);
  const int64_t chunks = (block_bytes + kChunk - 1) / kChunk;
  const int64_t items = num_planes * num_copies * chunks;
  if (items == 0) return NVS_OK;
  NVS_REQUIRE(src && dst, NVS_ERR_INVALID, "%s: null pointer argument", who);
  NVS_REQUIRE(((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0, NVS_ERR_INVALID,
              "%s: buffers must be 16-byte aligned", who);
  CopyArgs a;
  a.src = (const char*)src; a.dst = (char*)dst;
  a.src_ids = src_block_ids; a.dst_ids = dst_block_ids;
  a.src_nb = src_num_blocks; a.dst_nb = dst_num_blocks;
  a.block_bytes = block_bytes; a.chunks = chunks; a.copies = num_copies; a.items = items;
  // Enough work-groups to keep every CU streaming; each loops over the rest.
  const int64_t grid = items < 8192 ? items : 8192;
  hipLaunchKernelGGL(copy_blocks_kernel, dim3((unsigned)grid), dim3(kCopyThreads), 0, (hipStream_t)stream, a);
  return check_launch(who);
}
