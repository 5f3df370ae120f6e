// Slot-mapped K/V append into the paged cache (gfx950).
//
// Replaces tileInfer's store_kvcache (kernels/kvcache_store.py:43-71). The reference stages a
// block_N x D tile of K and V in shared memory and then scatters it (14-40); here every lane
// moves one 16-byte vector straight from the new-token row to its cache row, so a 2 KiB row
// (4 KV heads x 256 x bf16) is one fully coalesced 128-lane access for K and one for V, with no
// LDS round trip and no per-N specialisation.
#include "ti_common.h"

namespace ti {
namespace {

constexpr int kAppendThreads = 256;

// VecT is the per-lane access: u32x4 (16 B) when rows and strides allow it, else 16-bit.
template <typename VecT>
__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(
    const VecT* __restrict__ key, const VecT* __restrict__ value, int64_t key_stride,
    int64_t value_stride, VecT* __restrict__ k_cache, VecT* __restrict__ v_cache,
    int64_t cache_stride, const int32_t* __restrict__ slot_mapping, uint32_t total,
    uint32_t row_vecs, int64_t num_slots) {
  // Strides are in units of VecT. One item = one vector of one token's K row and the matching
  // vector of its V row.
  for (uint32_t i = blockIdx.x * kAppendThreads + threadIdx.x; i < total;
       i += gridDim.x * kAppendThreads) {
    const uint32_t tok = i / row_vecs;
    const uint32_t vec = i - tok * row_vecs;
    const int64_t slot = slot_mapping[tok];
    if (slot < 0 || slot >= num_slots) continue;  // -1 padding, or out of range: skip
    // The new rows are read once: streaming (nt) loads keep them out of the way of the cache rows.
    const VecT kx = __builtin_nontemporal_load(key + tok * key_stride + vec);
    const VecT vx = __builtin_nontemporal_load(value + tok * value_stride + vec);
    k_cache[slot * cache_stride + vec] = kx;
    v_cache[slot * cache_stride + vec] = vx;
  }
}

template <typename VecT>
int launch_append(const void* key, const void* value, int64_t key_stride, int64_t value_stride,
                  void* k_cache, void* v_cache, int64_t cache_stride,
                  const int32_t* slot_mapping, int64_t n_tokens, int64_t row_elems,
                  int64_t num_slots, hipStream_t stream) {
  constexpr int64_t per = sizeof(VecT) / 2;  // 16-bit elements per vector
  const int64_t row_vecs = row_elems / per;
  const int64_t total = n_tokens * row_vecs;
  if (total >= (int64_t(1) << 31)) {
    return fail(TI_EINVAL, "ti_kv_append: n_tokens*row_elems too large (%lld vectors)",
                (long long)total);
  }
  const int64_t blocks_needed = ceil_div(total, kAppendThreads);
  const int64_t max_blocks = int64_t(device_cu_count()) * 32;
  const unsigned grid = unsigned(blocks_needed < max_blocks ? blocks_needed : max_blocks);
  hipLaunchKernelGGL(kv_append_kernel<VecT>, dim3(grid), dim3(kAppendThreads), 0, stream,
                     static_cast<const VecT*>(key), static_cast<const VecT*>(value),
                     key_stride / per, value_stride / per, static_cast<VecT*>(k_cache),
                     static_cast<VecT*>(v_cache), cache_stride / per, slot_mapping,
                     uint32_t(total), uint32_t(row_vecs), num_slots);
  return check_launch("ti_kv_append");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace ti

extern "C" int ti_kv_append(const void* key, const void* value, int64_t key_row_stride,
                            int64_t value_row_stride, void* k_cache, void* v_cache,
                            int64_t cache_row_stride, const int32_t* slot_mapping,
                            int64_t n_tokens, int64_t row_elems, int64_t num_slots,
                            int32_t dtype, void* stream) {
  using namespace ti;
  if (dtype != TI_DTYPE_BF16 && dtype != TI_DTYPE_F16) {
    return fail(TI_EUNSUPPORTED, "ti_kv_append: dtype code %d is not bf16/fp16", dtype);
  }
  if (n_tokens < 0 || row_elems <= 0 || num_slots < 0) {
    return fail(TI_EINVAL, "ti_kv_append: bad sizes n_tokens=%lld row_elems=%lld num_slots=%lld",
                (long long)n_tokens, (long long)row_elems, (long long)num_slots);
  }
  if (n_tokens == 0) return TI_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) {
    return fail(TI_EINVAL, "ti_kv_append: null pointer");
  }
  if (key_row_stride < row_elems || value_row_stride < row_elems || cache_row_stride < row_elems) {
    return fail(TI_EINVAL, "ti_kv_append: row strides (%lld, %lld, %lld) < row_elems %lld",
                (long long)key_row_stride, (long long)value_row_stride,
                (long long)cache_row_stride, (long long)row_elems);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec16 = (row_elems % 8 == 0) && (key_row_stride % 8 == 0) &&
                     (value_row_stride % 8 == 0) && (cache_row_stride % 8 == 0) &&
                     aligned16(key) && aligned16(value) && aligned16(k_cache) &&
                     aligned16(v_cache);
  if (vec16) {
    return launch_append<u32x4>(key, value, key_row_stride, value_row_stride, k_cache, v_cache,
                                cache_row_stride, slot_mapping, n_tokens, row_elems, num_slots,
                                s);
  }
  return launch_append<uint16_t>(key, value, key_row_stride, value_row_stride, k_cache, v_cache,
                                 cache_row_stride, slot_mapping, n_tokens, row_elems, num_slots,
                                 s);
}
