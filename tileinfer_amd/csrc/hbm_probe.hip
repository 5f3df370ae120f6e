// HBM read ceiling probe: the bandwidth a plain streaming reader reaches on the decode's own
// access pattern (whole K and V pages, gathered through a page list), with no compute. It is the
// measured ceiling the decode kernel is judged against besides the 8 TB/s data-sheet peak.
//
// Workgroups take pages either in a grid-stride loop or, with `runs`, as contiguous runs of the
// page list (workgroup w reads entries [w*c, (w+1)*c), c = ceil(n_pages / workgroups): the
// decode's balanced assignment, one run of a sequence's pages per workgroup). Page ids outside
// [0, region_pages) are skipped. The 256 lanes of a workgroup read each page of K and of V as
// 16-byte vectors (one fully coalesced 4 KiB sweep per load instruction), eight loads per page
// per region in flight before any is consumed. The loaded words are folded with XOR and each lane
// stores one 16-byte word, so the loads cannot be dropped and the stores are negligible.
#include "ti_common.h"

namespace ti {
namespace {

constexpr int kProbeThreads = 256;

template <bool STREAM>
__device__ __forceinline__ u32x4 probe_load(const u32x4* p) {
  if constexpr (STREAM) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

template <bool STREAM>
__global__ __launch_bounds__(kProbeThreads) void hbm_read_pages_kernel(
    const unsigned char* k, const unsigned char* v, const int32_t* pages, int64_t n_pages,
    int64_t page_bytes, int64_t region_pages, int32_t runs, u32x4* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t per_pass = int64_t(kProbeThreads) * 16;
  const int64_t c = runs ? (n_pages + gridDim.x - 1) / gridDim.x : 1;
  const int64_t first = runs ? blockIdx.x * c : blockIdx.x;
  const int64_t end = runs ? (first + c < n_pages ? first + c : n_pages) : n_pages;
  const int64_t step = runs ? 1 : gridDim.x;
  for (int64_t i = first; i < end; i += step) {
    const int64_t id = pages ? pages[i] : i;
    if (id < 0 || id >= region_pages) continue;  // uniform
    const int64_t base = id * page_bytes + threadIdx.x * 16;
    for (int64_t off = 0; off < page_bytes; off += 8 * per_pass) {
      u32x4 w[16];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t o = off + u * per_pass;
        const bool in = o < page_bytes;  // uniform
        w[u] = in ? probe_load<STREAM>(reinterpret_cast<const u32x4*>(k + base + o))
                  : u32x4{0u, 0u, 0u, 0u};
        w[8 + u] = in ? probe_load<STREAM>(reinterpret_cast<const u32x4*>(v + base + o))
                      : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) acc ^= w[u];
    }
  }
  sink[int64_t(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

}  // namespace
}  // namespace ti

extern "C" int ti_hbm_read_probe(const void* k, const void* v, const int32_t* pages,
                                 int64_t n_pages, int64_t page_bytes, int64_t region_pages,
                                 int32_t streaming, int32_t runs, int32_t workgroups, void* sink,
                                 void* stream) {
  using namespace ti;
  // Whole 4 KiB sweeps only: a lane's last load then ends exactly at the page end.
  if (n_pages < 0 || page_bytes <= 0 || page_bytes % (kProbeThreads * 16) != 0 ||
      region_pages < 0 || workgroups <= 0 || workgroups > 65535) {
    return fail(TI_EINVAL,
                "ti_hbm_read_probe: n_pages=%lld page_bytes=%lld (a multiple of 4096) "
                "region_pages=%lld workgroups=%d",
                (long long)n_pages, (long long)page_bytes, (long long)region_pages, workgroups);
  }
  if (n_pages == 0) return TI_OK;
  if (!k || !v || !sink || (reinterpret_cast<uintptr_t>(k) & 15) ||
      (reinterpret_cast<uintptr_t>(v) & 15) || (reinterpret_cast<uintptr_t>(sink) & 15)) {
    return fail(TI_EINVAL, "ti_hbm_read_probe: null or unaligned pointer");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned char* kb = static_cast<const unsigned char*>(k);
  const unsigned char* vb = static_cast<const unsigned char*>(v);
  u32x4* out = static_cast<u32x4*>(sink);
  if (streaming) {
    hipLaunchKernelGGL(hbm_read_pages_kernel<true>, dim3(workgroups), dim3(kProbeThreads), 0, s,
                       kb, vb, pages, n_pages, page_bytes, region_pages, runs, out);
  } else {
    hipLaunchKernelGGL(hbm_read_pages_kernel<false>, dim3(workgroups), dim3(kProbeThreads), 0, s,
                       kb, vb, pages, n_pages, page_bytes, region_pages, runs, out);
  }
  return check_launch("ti_hbm_read_probe");
}
