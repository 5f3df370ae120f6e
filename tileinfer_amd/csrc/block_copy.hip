// Whole-block copies between paged KV caches: swap-out to / swap-in from pinned host memory and
// device-to-device block copies, driven by a (source block, destination block) list.
//
// tileInfer accepts a swap budget but never moves KV blocks (engine/config.py:22,
// engine/block_manager.py:29); this is the data path a SWAP policy needs. A block id names
// `n_chunks` chunks (K and V of every attention layer) of `chunk_bytes` each, chunk c of block b at
// base + c * chunk_stride + b * chunk_bytes — the [2, layers, blocks, block_size, H_kv, D] slab.
// One launch moves the whole list: each workgroup copies one chunk with 16-byte vector accesses.
// Pinned host memory is addressed directly by the kernel (it is mapped into the device's address
// space), so a swap is one launch instead of one copy call per chunk.
#include "ti_common.h"

namespace ti {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 8;

__global__ __launch_bounds__(kCopyThreads) void copy_blocks_kernel(
    const u32x4* __restrict__ src, u32x4* __restrict__ dst, const int64_t* __restrict__ pairs,
    int64_t n_items, int32_t n_chunks, int64_t chunk_vecs, int64_t src_chunk_stride,
    int64_t dst_chunk_stride, int64_t src_blocks, int64_t dst_blocks) {
  // Strides are in 16-byte vectors.
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int64_t pair = item / n_chunks;
    const int64_t chunk = item - pair * n_chunks;
    const int64_t s = pairs[2 * pair];
    const int64_t d = pairs[2 * pair + 1];
    if (s < 0 || s >= src_blocks || d < 0 || d >= dst_blocks) continue;  // uniform per workgroup
    const u32x4* from = src + chunk * src_chunk_stride + s * chunk_vecs;
    u32x4* to = dst + chunk * dst_chunk_stride + d * chunk_vecs;
    for (int64_t base = threadIdx.x; base < chunk_vecs; base += kCopyThreads * kCopyUnroll) {
      u32x4 v[kCopyUnroll];
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + int64_t(u) * kCopyThreads;
        if (i < chunk_vecs) v[u] = __builtin_nontemporal_load(from + i);
      }
#pragma unroll
      for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + int64_t(u) * kCopyThreads;
        if (i < chunk_vecs) __builtin_nontemporal_store(v[u], to + i);
      }
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The address at which the device reaches `p`: device memory as is, pinned (page-locked, mapped)
// host memory through its device mapping. Anything else is refused before a kernel could touch it.
int device_address(const void* p, const char* what, const void** out) {
  hipPointerAttribute_t attr;
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // the failed query must not surface as a later launch error
    return fail(TI_EINVAL, "ti_copy_blocks: %s is neither device memory nor pinned host memory",
                what);
  }
  if (attr.type == hipMemoryTypeHost) {
    if (attr.devicePointer == nullptr) {
      return fail(TI_EINVAL, "ti_copy_blocks: %s is host memory without a device mapping", what);
    }
    const char* base_host = static_cast<const char*>(attr.hostPointer);
    const char* base_dev = static_cast<const char*>(attr.devicePointer);
    *out = base_host ? base_dev + (static_cast<const char*>(p) - base_host) : base_dev;
    return TI_OK;
  }
  if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
      attr.type == hipMemoryTypeUnified) {
    *out = p;
    return TI_OK;
  }
  return fail(TI_EINVAL,
              "ti_copy_blocks: %s is neither device memory nor pinned host memory (memory type %d)",
              what, int(attr.type));
}

}  // namespace
}  // namespace ti

extern "C" int ti_copy_blocks(const void* src, void* dst, const int64_t* block_pairs,
                              int64_t n_pairs, int32_t n_chunks, int64_t chunk_bytes,
                              int64_t src_chunk_stride_bytes, int64_t dst_chunk_stride_bytes,
                              int64_t src_num_blocks, int64_t dst_num_blocks, void* stream) {
  using namespace ti;
  if (n_pairs < 0 || n_chunks <= 0 || chunk_bytes <= 0 || src_num_blocks < 0 ||
      dst_num_blocks < 0) {
    return fail(TI_EINVAL, "ti_copy_blocks: bad sizes pairs=%lld chunks=%d chunk_bytes=%lld",
                (long long)n_pairs, n_chunks, (long long)chunk_bytes);
  }
  if (n_pairs == 0) return TI_OK;
  if (!src || !dst || !block_pairs) return fail(TI_EINVAL, "ti_copy_blocks: null pointer");
  if (chunk_bytes % 16 || src_chunk_stride_bytes % 16 || dst_chunk_stride_bytes % 16 ||
      !aligned16(src) || !aligned16(dst)) {
    return fail(TI_EINVAL, "ti_copy_blocks: chunks, strides and bases must be 16-byte aligned");
  }
  if (src_chunk_stride_bytes < src_num_blocks * chunk_bytes ||
      dst_chunk_stride_bytes < dst_num_blocks * chunk_bytes) {
    return fail(TI_EINVAL, "ti_copy_blocks: chunk stride smaller than num_blocks * chunk_bytes");
  }
  const void *dsrc = nullptr, *ddst = nullptr, *dpairs = nullptr;
  int rc = device_address(src, "src", &dsrc);
  if (rc == TI_OK) rc = device_address(dst, "dst", &ddst);
  if (rc == TI_OK) rc = device_address(block_pairs, "block_pairs", &dpairs);
  if (rc != TI_OK) return rc;
  const int64_t items = n_pairs * n_chunks;
  const int64_t cap = int64_t(device_cu_count()) * 16;
  const unsigned grid = unsigned(items < cap ? items : cap);
  hipLaunchKernelGGL(copy_blocks_kernel, dim3(grid), dim3(kCopyThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(dsrc),
                     static_cast<u32x4*>(const_cast<void*>(ddst)),
                     static_cast<const int64_t*>(dpairs), items, n_chunks, chunk_bytes / 16,
                     src_chunk_stride_bytes / 16, dst_chunk_stride_bytes / 16, src_num_blocks,
                     dst_num_blocks);
  return check_launch("ti_copy_blocks");
}
