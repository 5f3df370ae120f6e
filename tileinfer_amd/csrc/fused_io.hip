// The element-wise work on either side of the paged attention path, fused with it.
//
// Before attention (model/qwen_36.py:977-1018): per-head RMSNorm of q and k with a (1 + w)
// weight, partial rotary embedding on the first rotary_dim dimensions, then the slot-mapped append
// of k and v. The reference runs the first two as one TileLang kernel for a single sequence
// (kernels/qknorm_rope.py:9-56) and as separate torch ops otherwise, then store_kvcache.
//   ti_qknorm_rope         q or k alone (any number of tokens, per-token cos/sin)
//   ti_qknorm_rope_append  q, k and v of one step in one launch: q normalised and rotated to its
//                          output, k normalised and rotated and v as is, written straight into
//                          the cache rows at slot_mapping (no intermediate k)
// After attention (model/qwen_36.py:1083, kernels/act_mul.py:62-79): out = attn * sigmoid(gate).
//   ti_sigmoid_mul         the element-wise product alone (the decode kernel also applies it in
//                          its output epilogue, ti_gqa_decode_paged_gated)
//
// Numerics follow the reference's fused kernel (kernels/qknorm_rope.py:29-49): sum of squares and
// scale in fp32, normalised row rounded to the storage type, rotation in fp32 from those values
// with cos/sin[0 .. rotary_dim/2) for both halves (rotate-half pairing i <-> i + rotary_dim/2),
// rounded once. The fused append writes exactly what ti_qknorm_rope followed by the append would.
#include "decode_common.h"

namespace ti {
namespace {

struct NormRopeArgs {
  const uint16_t* x;
  int64_t x_st, x_sh;
  uint16_t* out;  // row outputs (q or k) or nullptr
  int64_t o_st, o_sh;
  const uint16_t* w;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cs_st;  // cos/sin token stride (0: one vector for every token)
  int32_t n_tokens, n_heads, rotary_dim;
  float eps;
  // Cache-row output (fused append): row slot of token t, head h at cache + slot*row + h*D.
  uint16_t* cache;
  int64_t cache_row;
  const int32_t* slots;
  int64_t num_slots;
};

// Normalises and rotates row (t, h) of `a.x` (one wave per row); returns the lane's EPL output
// values, packed. Lane l owns elements [EPL*l, EPL*l + EPL). `sh` is this wave's LDS row of D
// 16-bit values, through which the rotation partners (i <-> i +- rotary_dim/2) are exchanged.
template <int D, typename Tag>
__device__ __forceinline__ void norm_rope_row(const NormRopeArgs& a, int t, int h, uint16_t* sh,
                                              uint32_t (&res)[D / 128]) {
  constexpr int EPL = D / 64;  // 2 or 4 elements per lane
  const int lane = threadIdx.x & 63;
  const uint16_t* xr = a.x + int64_t(t) * a.x_st + int64_t(h) * a.x_sh + EPL * lane;
  float v[EPL], w[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j += 2) {
    const float2 p = unpack2(*reinterpret_cast<const uint32_t*>(xr + j), Tag{});
    const float2 q = unpack2(*reinterpret_cast<const uint32_t*>(a.w + EPL * lane + j), Tag{});
    v[j] = p.x;
    v[j + 1] = p.y;
    w[j] = q.x;
    w[j + 1] = q.y;
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) ss += v[j] * v[j];
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) ss += __shfl_xor(ss, d, 64);
  const float r = rsqrtf(ss / float(D) + a.eps);
  uint32_t nb[EPL / 2];
#pragma unroll
  for (int j = 0; j < EPL; j += 2) {
    nb[j / 2] = pack2(v[j] * r * (1.f + w[j]), v[j + 1] * r * (1.f + w[j + 1]), Tag{});
    *reinterpret_cast<uint32_t*>(sh + EPL * lane + j) = nb[j / 2];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int half = a.rotary_dim / 2;
  const uint16_t* cr = a.rotary_dim > 0 ? a.cos + int64_t(t) * a.cs_st : nullptr;
  const uint16_t* sr = a.rotary_dim > 0 ? a.sin + int64_t(t) * a.cs_st : nullptr;
#pragma unroll
  for (int j = 0; j < EPL; j += 2) {
    const float2 own = unpack2(nb[j / 2], Tag{});
    float o2[2] = {own.x, own.y};
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = EPL * lane + j + e;
      if (i < a.rotary_dim) {
        const int k = i < half ? i : i - half;          // cos/sin index
        const int pi = i < half ? i + half : i - half;  // rotation partner
        const uint16_t pb = sh[pi];
        const float partner = unpack2(uint32_t(pb), Tag{}).x;
        const float c = unpack2(uint32_t(cr[k]), Tag{}).x;
        const float s = unpack2(uint32_t(sr[k]), Tag{}).x;
        o2[e] = i < half ? o2[e] * c - partner * s : o2[e] * c + partner * s;
      }
    }
    res[j / 2] = pack2(o2[0], o2[1], Tag{});
  }
}

template <int D, typename Tag>
__global__ __launch_bounds__(256) void norm_rope_kernel(NormRopeArgs a) {
  constexpr int EPL = D / 64;
  __shared__ __align__(16) uint16_t sh[4][D];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + wave;
  if (row >= int64_t(a.n_tokens) * a.n_heads) return;  // uniform per wave
  const int t = int(row / a.n_heads);
  const int h = int(row % a.n_heads);
  uint32_t res[EPL / 2];
  norm_rope_row<D, Tag>(a, t, h, sh[wave], res);
  uint16_t* dst = a.out + int64_t(t) * a.o_st + int64_t(h) * a.o_sh + EPL * lane;
#pragma unroll
  for (int j = 0; j < EPL / 2; ++j) reinterpret_cast<uint32_t*>(dst)[j] = res[j];
}

// One launch for q, k and v of a step: rows [0, T*Hq) are q heads (to q_out), the next T*Hkv
// are k heads (to the k cache at their slots), the last T*Hkv are v heads (copied to the v cache).
struct StepArgs {
  NormRopeArgs q, k;
  const uint16_t* v;
  int64_t v_st, v_sh;
  uint16_t* v_cache;
  int32_t n_kv_heads;
};

template <int D, typename Tag>
__global__ __launch_bounds__(256) void norm_rope_append_kernel(StepArgs a) {
  constexpr int EPL = D / 64;
  __shared__ __align__(16) uint16_t sh[4][D];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int64_t row = int64_t(blockIdx.x) * 4 + wave;
  const int64_t nq = int64_t(a.q.n_tokens) * a.q.n_heads;
  const int64_t nk = int64_t(a.k.n_tokens) * a.k.n_heads;
  uint32_t res[EPL / 2];
  if (row < nq) {
    const int t = int(row / a.q.n_heads), h = int(row % a.q.n_heads);
    norm_rope_row<D, Tag>(a.q, t, h, sh[wave], res);
    uint16_t* dst = a.q.out + int64_t(t) * a.q.o_st + int64_t(h) * a.q.o_sh + EPL * lane;
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) reinterpret_cast<uint32_t*>(dst)[j] = res[j];
    return;
  }
  row -= nq;
  if (row < nk) {
    const int t = int(row / a.k.n_heads), h = int(row % a.k.n_heads);
    const int64_t slot = a.k.slots[t];
    norm_rope_row<D, Tag>(a.k, t, h, sh[wave], res);
    if (slot < 0 || slot >= a.k.num_slots) return;
    uint16_t* dst = a.k.cache + slot * a.k.cache_row + int64_t(h) * D + EPL * lane;
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) reinterpret_cast<uint32_t*>(dst)[j] = res[j];
    return;
  }
  row -= nk;
  if (row < nk) {
    const int t = int(row / a.n_kv_heads), h = int(row % a.n_kv_heads);
    const int64_t slot = a.k.slots[t];
    if (slot < 0 || slot >= a.k.num_slots) return;
    const uint16_t* src = a.v + int64_t(t) * a.v_st + int64_t(h) * a.v_sh + EPL * lane;
    uint16_t* dst = a.v_cache + slot * a.k.cache_row + int64_t(h) * D + EPL * lane;
#pragma unroll
    for (int j = 0; j < EPL / 2; ++j) {
      reinterpret_cast<uint32_t*>(dst)[j] = reinterpret_cast<const uint32_t*>(src)[j];
    }
  }
}

template <typename Tag>
__global__ __launch_bounds__(256) void sigmoid_mul_kernel(const uint32_t* a, const uint32_t* b,
                                                          uint32_t* out, int64_t n_pairs) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n_pairs;
       i += int64_t(gridDim.x) * 256) {
    out[i] = gate_mul2(a[i], b[i], Tag{});
  }
}

bool rows_aligned(const void* p, int64_t st, int64_t sh) {
  return (reinterpret_cast<uintptr_t>(p) & 3) == 0 && st % 2 == 0 && sh % 2 == 0;
}

int check_common(int32_t n_tokens, int32_t head_dim, int32_t rotary_dim, int32_t dtype,
                 const char* who) {
  if (dtype != TI_DTYPE_BF16 && dtype != TI_DTYPE_F16) {
    return fail(TI_EUNSUPPORTED, "%s: dtype code %d is not bf16/fp16", who, dtype);
  }
  if (head_dim != 128 && head_dim != 256) {
    return fail(TI_EUNSUPPORTED, "%s: head_dim %d not built (128, 256)", who, head_dim);
  }
  if (n_tokens < 0 || rotary_dim < 0 || rotary_dim > head_dim || rotary_dim % 2 != 0) {
    return fail(TI_EINVAL, "%s: bad sizes tokens=%d rotary_dim=%d", who, n_tokens, rotary_dim);
  }
  return TI_OK;
}

unsigned row_blocks(int64_t rows) { return unsigned((rows + 3) / 4); }

}  // namespace
}  // namespace ti

extern "C" int ti_qknorm_rope(const void* x, int64_t x_stride_t, int64_t x_stride_h, void* out,
                              int64_t out_stride_t, int64_t out_stride_h, const void* weight,
                              const void* cos, const void* sin, int64_t cs_stride_t,
                              int32_t n_tokens, int32_t n_heads, int32_t head_dim,
                              int32_t rotary_dim, float eps, int32_t dtype, void* stream) {
  using namespace ti;
  int rc = check_common(n_tokens, head_dim, rotary_dim, dtype, "ti_qknorm_rope");
  if (rc != TI_OK) return rc;
  if (n_heads <= 0) return fail(TI_EINVAL, "ti_qknorm_rope: n_heads %d", n_heads);
  if (n_tokens == 0) return TI_OK;
  if (!x || !out || !weight || (rotary_dim > 0 && (!cos || !sin))) {
    return fail(TI_EINVAL, "ti_qknorm_rope: null pointer");
  }
  if (!rows_aligned(x, x_stride_t, x_stride_h) || !rows_aligned(out, out_stride_t, out_stride_h) ||
      (reinterpret_cast<uintptr_t>(weight) & 3)) {
    return fail(TI_EINVAL, "ti_qknorm_rope: rows must be 4-byte aligned");
  }
  NormRopeArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_st = x_stride_t;
  a.x_sh = x_stride_h;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.w = static_cast<const uint16_t*>(weight);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.cs_st = cs_stride_t;
  a.n_tokens = n_tokens;
  a.n_heads = n_heads;
  a.rotary_dim = rotary_dim;
  a.eps = eps;
  const dim3 grid(row_blocks(int64_t(n_tokens) * n_heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == TI_DTYPE_BF16;
  if (head_dim == 256) {
    if (bf16) hipLaunchKernelGGL((norm_rope_kernel<256, Bf16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((norm_rope_kernel<256, F16>), grid, dim3(256), 0, s, a);
  } else {
    if (bf16) hipLaunchKernelGGL((norm_rope_kernel<128, Bf16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((norm_rope_kernel<128, F16>), grid, dim3(256), 0, s, a);
  }
  return check_launch("ti_qknorm_rope");
}

extern "C" int ti_qknorm_rope_append(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
    int64_t k_stride_h, const void* v, int64_t v_stride_t, int64_t v_stride_h,
    const void* q_weight, const void* k_weight, const void* cos, const void* sin,
    int64_t cs_stride_t, void* q_out, int64_t q_out_stride_t, int64_t q_out_stride_h,
    void* k_cache, void* v_cache, int64_t cache_row_stride, const int32_t* slot_mapping,
    int64_t num_slots, int32_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    int32_t rotary_dim, float eps, int32_t dtype, void* stream) {
  using namespace ti;
  int rc = check_common(n_tokens, head_dim, rotary_dim, dtype, "ti_qknorm_rope_append");
  if (rc != TI_OK) return rc;
  if (n_q_heads <= 0 || n_kv_heads <= 0 || num_slots < 0 ||
      cache_row_stride < int64_t(n_kv_heads) * head_dim) {
    return fail(TI_EINVAL, "ti_qknorm_rope_append: bad heads/slots/row stride");
  }
  if (n_tokens == 0) return TI_OK;
  if (!q || !k || !v || !q_weight || !k_weight || !q_out || !k_cache || !v_cache ||
      !slot_mapping || (rotary_dim > 0 && (!cos || !sin))) {
    return fail(TI_EINVAL, "ti_qknorm_rope_append: null pointer");
  }
  if (!rows_aligned(q, q_stride_t, q_stride_h) || !rows_aligned(k, k_stride_t, k_stride_h) ||
      !rows_aligned(v, v_stride_t, v_stride_h) ||
      !rows_aligned(q_out, q_out_stride_t, q_out_stride_h) ||
      !rows_aligned(k_cache, cache_row_stride, 2) || !rows_aligned(v_cache, 2, 2)) {
    return fail(TI_EINVAL, "ti_qknorm_rope_append: rows must be 4-byte aligned");
  }
  StepArgs a{};
  a.q.x = static_cast<const uint16_t*>(q);
  a.q.x_st = q_stride_t;
  a.q.x_sh = q_stride_h;
  a.q.out = static_cast<uint16_t*>(q_out);
  a.q.o_st = q_out_stride_t;
  a.q.o_sh = q_out_stride_h;
  a.q.w = static_cast<const uint16_t*>(q_weight);
  a.q.cos = static_cast<const uint16_t*>(cos);
  a.q.sin = static_cast<const uint16_t*>(sin);
  a.q.cs_st = cs_stride_t;
  a.q.n_tokens = n_tokens;
  a.q.n_heads = n_q_heads;
  a.q.rotary_dim = rotary_dim;
  a.q.eps = eps;
  a.k = a.q;
  a.k.x = static_cast<const uint16_t*>(k);
  a.k.x_st = k_stride_t;
  a.k.x_sh = k_stride_h;
  a.k.out = nullptr;
  a.k.w = static_cast<const uint16_t*>(k_weight);
  a.k.n_heads = n_kv_heads;
  a.k.cache = static_cast<uint16_t*>(k_cache);
  a.k.cache_row = cache_row_stride;
  a.k.slots = slot_mapping;
  a.k.num_slots = num_slots;
  a.v = static_cast<const uint16_t*>(v);
  a.v_st = v_stride_t;
  a.v_sh = v_stride_h;
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.n_kv_heads = n_kv_heads;
  const int64_t rows = int64_t(n_tokens) * (n_q_heads + 2 * n_kv_heads);
  const dim3 grid(row_blocks(rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == TI_DTYPE_BF16;
  if (head_dim == 256) {
    if (bf16) hipLaunchKernelGGL((norm_rope_append_kernel<256, Bf16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((norm_rope_append_kernel<256, F16>), grid, dim3(256), 0, s, a);
  } else {
    if (bf16) hipLaunchKernelGGL((norm_rope_append_kernel<128, Bf16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((norm_rope_append_kernel<128, F16>), grid, dim3(256), 0, s, a);
  }
  return check_launch("ti_qknorm_rope_append");
}

extern "C" int ti_sigmoid_mul(const void* a, const void* b, void* out, int64_t n, int32_t dtype,
                              void* stream) {
  using namespace ti;
  if (dtype != TI_DTYPE_BF16 && dtype != TI_DTYPE_F16) {
    return fail(TI_EUNSUPPORTED, "ti_sigmoid_mul: dtype code %d is not bf16/fp16", dtype);
  }
  if (n < 0 || n % 2 != 0) return fail(TI_EINVAL, "ti_sigmoid_mul: n=%lld must be even", (long long)n);
  if (n == 0) return TI_OK;
  if (!a || !b || !out) return fail(TI_EINVAL, "ti_sigmoid_mul: null pointer");
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
       reinterpret_cast<uintptr_t>(out)) & 3) {
    return fail(TI_EINVAL, "ti_sigmoid_mul: pointers must be 4-byte aligned");
  }
  const int64_t pairs = n / 2;
  const int64_t cap = int64_t(device_cu_count()) * 16;
  const int64_t want = (pairs + 255) / 256;
  const dim3 grid(unsigned(want < cap ? want : cap));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TI_DTYPE_BF16) {
    hipLaunchKernelGGL((sigmoid_mul_kernel<Bf16>), grid, dim3(256), 0, s,
                       static_cast<const uint32_t*>(a), static_cast<const uint32_t*>(b),
                       static_cast<uint32_t*>(out), pairs);
  } else {
    hipLaunchKernelGGL((sigmoid_mul_kernel<F16>), grid, dim3(256), 0, s,
                       static_cast<const uint32_t*>(a), static_cast<const uint32_t*>(b),
                       static_cast<uint32_t*>(out), pairs);
  }
  return check_launch("ti_sigmoid_mul");
}
