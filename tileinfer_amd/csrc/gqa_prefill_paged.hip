// Causal GQA prefill attention that reads K/V straight from the paged cache (gfx950).
//
// Replaces tileInfer's chunked-prefill attention, which first gathers every cached position of the
// sequence through the block table into contiguous K/V copies (model/qwen_36.py:1030-1044) and then
// runs varlen flash attention on them (kernels/gqa_varlen.py:40-185, dispatch 369-389). Here the
// cache pages are the operand: no gather copy, one launch for any number of sequences.
//
// Semantics (kernels/gqa_varlen.py:88-131, 144-175): sequence b has q_len = cu_q[b+1] - cu_q[b]
// query tokens and kv_len = seqlen_k[b] cached tokens (the chunk's own K/V already appended); the
// causal mask is bottom-right aligned, query i sees keys j <= kv_len - q_len + i. Scores are scaled
// by D^-1/2 log2 e and exponentiated in base 2, P is rounded to the cache dtype before P.V, fp32
// accumulation, a row with no visible key is zero. `causal = 0` drops the causal mask (every query
// sees all kv_len keys), the reference's is_causal=False. As in the decode kernel, a block id
// outside [0, num_blocks) inside the context is an absent page: its keys are masked, never loaded.
//
// Work unit: a workgroup = 64 query tokens of one query head (4 waves x 16 tokens); 32-key tiles of
// that head's KV head are staged in LDS (prefetched into registers one tile ahead, one barrier per
// tile) straight from the pages. Each wave uses the decode kernel's transposed MFMA layout with its
// 16 query tokens as the 16 columns:
//   S^T[16 keys x 16 queries] = K[16 keys x 32 d] . Q^T[32 d x 16 queries]    (16x16x32)
//   O^T[16 d x 16 queries]   += V^T[16 d x 16 keys] . P^T[16 keys x 16 queries] (16x16x16)
// so every accumulator's query is its lane's column and the softmax rescale stays in the lane.
#include "decode_common.h"

namespace ti {
namespace {

typedef __bf16 pf_bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 pf_f16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c, Bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(pf_bf16x4_t, a),
                                                   __builtin_bit_cast(pf_bf16x4_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c, F16) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(pf_f16x4_t, a),
                                               __builtin_bit_cast(pf_f16x4_t, b), c, 0, 0, 0);
}

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;  // q [T, hq, D] strides (elements)
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t page_stride, row_stride;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* cu_q;      // [B+1]
  const int32_t* seqlen_k;  // [B]
  uint16_t* out;
  int64_t o_st, o_sh;
  int32_t total_q, num_blocks32, hq, hkv, group, page_size, max_blocks, causal;
  float scale_log2;
};

constexpr int kQB = 64;   // query tokens per workgroup
constexpr int kKT = 32;   // keys per staged tile

template <int D, typename Tag>
__global__ __launch_bounds__(256) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int KK = D / 32;
  constexpr int NC = D / 128;
  constexpr int NT = D / 16;
  constexpr int ROW = D + 8;                 // padded LDS row (16-bit elements)
  constexpr int CPR = D / 8;                 // 16-byte chunks per row
  constexpr int CPT = kKT * CPR / 256;       // chunks per thread per tile, each of K and V
  static_assert(CPT * 256 == kKT * CPR, "tile must split evenly over 256 lanes");

  __shared__ __align__(16) uint16_t sk[2][kKT * ROW];
  __shared__ __align__(16) uint16_t sv[2][kKT * ROW];
  // Key j of the staged tile exists (inside the context, with a block id inside the cache): the
  // byte s_ok[buf][j] is 1. Keys that do not exist are masked out, like the decode kernel's.
  __shared__ __align__(4) uint8_t s_ok[2][kKT];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n = lane & 15;  // query column of S^T/O^T; key row of K; d-column of V^T
  const int g = lane >> 4;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int kvh = h / a.group;

  // Row ranges are clamped into [0, total_q): a malformed cu_seqlens_q cannot move an access
  // outside q/out.
  const int q_start = min(max(a.cu_q[b], 0), a.total_q);
  const int q_len = min(max(a.cu_q[b + 1], q_start), a.total_q) - q_start;
  const int qb0 = blockIdx.x * kQB;
  if (qb0 >= q_len) return;  // uniform over the workgroup
  int kv_len = a.seqlen_k[b];
  const int cap = a.max_blocks * a.page_size;
  kv_len = kv_len < 0 ? 0 : (kv_len > cap ? cap : kv_len);
  const int offset = kv_len - q_len;  // query i sits at absolute position offset + i

  const int q0 = qb0 + 16 * wave;        // this wave's first query token
  const bool row_ok = q0 + n < q_len;
  const int q_pos = offset + q0 + n;     // absolute position of this lane's query

  // Q^T operand of this lane's query row (zero for rows past the chunk).
  u32x4 qop[KK];
  {
    const uint16_t* qrow = a.q + int64_t(q_start + q0 + n) * a.q_st + int64_t(h) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qop[kk] = row_ok ? load16(qrow + 32 * kk + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  f32x4 o[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_run = 0.f;

  // Keys the workgroup can see: j < kv_len, and j < offset + qb0 + kQB under the causal mask.
  int k_end = a.causal ? min(kv_len, offset + qb0 + kQB) : kv_len;
  if (k_end < 0) k_end = 0;
  const int ntiles = (k_end + kKT - 1) / kKT;
  // Under the causal mask, keys past this one are masked for every row of the wave.
  const int wave_last_key = a.causal ? offset + q0 + 15 : INT32_MAX;

  u32x4 pk[CPT], pv[CPT];
  uint32_t pok = 0;  // bit j: chunk j's key exists
  auto fetch = [&](int k0) {
    pok = 0;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int ci = t + 256 * j;
      const int r = ci / CPR, col = ci % CPR;
      const int key = k0 + r;
      int bid = -1;
      if (key < kv_len) {
        bid = a.block_table[int64_t(b) * a.bt_stride + key / a.page_size];
        if (uint32_t(bid) >= uint32_t(a.num_blocks32)) bid = -1;
      }
      if (bid >= 0) {
        const int64_t off = int64_t(bid) * a.page_stride + int64_t(key % a.page_size) * a.row_stride +
                            int64_t(kvh) * D + 8 * col;
        pk[j] = load16(a.k_cache + off);
        pv[j] = load16(a.v_cache + off);
        pok |= 1u << j;
      } else {
        pk[j] = u32x4{0u, 0u, 0u, 0u};
        pv[j] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      const int ci = t + 256 * j;
      const int r = ci / CPR, col = ci % CPR;
      *reinterpret_cast<u32x4*>(&sk[buf][r * ROW + 8 * col]) = pk[j];
      *reinterpret_cast<u32x4*>(&sv[buf][r * ROW + 8 * col]) = pv[j];
      if (col == 0) s_ok[buf][r] = uint8_t((pok >> j) & 1u);
    }
  };

  auto compute_sub = [&](int buf, int key0, int sub) {
    // 16 keys [key0, key0 + 16) held in rows 16*sub.. of the staged tile.
    const uint16_t* kb = &sk[buf][(16 * sub) * ROW];
    const uint16_t* vb = &sv[buf][(16 * sub) * ROW];
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u32x4 kop = *reinterpret_cast<const u32x4*>(kb + n * ROW + 32 * kk + 8 * g);
      s = mfma16x16x32(kop, qop[kk], s, Tag{});
    }
    const uint32_t okw = *reinterpret_cast<const uint32_t*>(&s_ok[buf][16 * sub + 4 * g]);
    float sv_[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + 4 * g + r;
      const bool ok = row_ok && ((okw >> (8 * r)) & 1u) && (key <= q_pos || !a.causal);
      sv_[r] = ok ? s[r] * a.scale_log2 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sv_[0], sv_[1]), fmaxf(sv_[2], sv_[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sv_[r] - m_use);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
      for (int i = 0; i < NT; ++i) o[i] *= alpha;
    }
    u32x2 pop;
    pop[0] = pack2(p[0], p[1], Tag{});
    pop[1] = pack2(p[2], p[3], Tag{});
    u32x4 vr[4][NC];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        vr[r][c] = *reinterpret_cast<const u32x4*>(vb + (4 * g + r) * ROW + 128 * c + 8 * n);
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        u32x2 vop;
        vop[0] = __builtin_amdgcn_perm(vr[1][c][e >> 1], vr[0][c][e >> 1], sel);
        vop[1] = __builtin_amdgcn_perm(vr[3][c][e >> 1], vr[2][c][e >> 1], sel);
        o[8 * c + e] = mfma16x16x16(vop, pop, o[8 * c + e], Tag{});
      }
    }
  };

  if (ntiles > 0) fetch(0);
  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    stash(buf);
    __syncthreads();
    if (it + 1 < ntiles) fetch((it + 1) * kKT);
    const int k0 = it * kKT;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      // A sub-tile wholly above this wave's diagonal contributes nothing: skip it (uniform).
      if (k0 + 16 * sub <= wave_last_key) compute_sub(buf, k0 + 16 * sub, sub);
    }
  }

  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!row_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  uint16_t* orow = a.out + int64_t(q_start + q0 + n) * a.o_st + int64_t(h) * a.o_sh;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 w;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        w[k] = pack2(o[8 * c + 2 * k][r] * inv, o[8 * c + 2 * k + 1][r] * inv, Tag{});
      }
      *reinterpret_cast<u32x4*>(orow + 128 * c + 32 * g + 8 * r) = w;
    }
  }
}

}  // namespace
}  // namespace ti

extern "C" int ti_gqa_prefill_paged(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                    const void* k_cache, const void* v_cache,
                                    const int32_t* block_table, int64_t block_table_stride,
                                    const int32_t* cu_seqlens_q, const int32_t* seqlen_k,
                                    void* out, int64_t out_stride_t, int64_t out_stride_h,
                                    int32_t batch, int32_t total_q, int32_t max_seqlen_q,
                                    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t page_size,
                                    int64_t num_blocks, int32_t max_blocks_per_seq, int32_t causal,
                                    int32_t dtype, void* stream) {
  using namespace ti;
  if (dtype != TI_DTYPE_BF16 && dtype != TI_DTYPE_F16) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: dtype code %d is not bf16/fp16", dtype);
  }
  if (batch < 0 || total_q < 0 || max_seqlen_q < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || max_blocks_per_seq < 0 || num_blocks < 0) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged: bad sizes");
  }
  if (head_dim != 128 && head_dim != 256) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: head_dim %d not built (128, 256)",
                head_dim);
  }
  if (page_size <= 0 || page_size % 16 != 0) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: page_size %d not a multiple of 16",
                page_size);
  }
  if (batch == 0 || total_q == 0 || max_seqlen_q == 0) return TI_OK;
  if (!q || !k_cache || !v_cache || !block_table || !cu_seqlens_q || !seqlen_k || !out) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged: null pointer");
  }
  if (block_table_stride < max_blocks_per_seq || q_stride_h % 8 || q_stride_t % 8 ||
      out_stride_h % 8 || out_stride_t % 8 || (reinterpret_cast<uintptr_t>(q) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & 15) || (reinterpret_cast<uintptr_t>(k_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(v_cache) & 15)) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged: rows must be 16-byte aligned");
  }
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.row_stride = int64_t(num_kv_heads) * head_dim;
  a.page_stride = a.row_stride * page_size;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.cu_q = cu_seqlens_q;
  a.seqlen_k = seqlen_k;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.total_q = total_q;
  a.num_blocks32 = int32_t(num_blocks < INT32_MAX ? num_blocks : INT32_MAX);
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.page_size = page_size;
  a.max_blocks = max_blocks_per_seq;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = float(1.4426950408889634 / sqrt(double(head_dim)));
  const dim3 grid(unsigned(ceil_div(max_seqlen_q, kQB)), unsigned(num_q_heads), unsigned(batch));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == TI_DTYPE_BF16;
  if (head_dim == 256) {
    if (bf16) hipLaunchKernelGGL((prefill_mfma_kernel<256, Bf16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((prefill_mfma_kernel<256, F16>), grid, dim3(256), 0, s, a);
  } else {
    if (bf16) hipLaunchKernelGGL((prefill_mfma_kernel<128, Bf16>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((prefill_mfma_kernel<128, F16>), grid, dim3(256), 0, s, a);
  }
  return check_launch("ti_gqa_prefill_paged");
}
