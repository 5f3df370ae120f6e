// Scalar variant of the paged decode partial kernel (gfx950): no matrix cores.
//
// One workgroup of 256 lanes per (sequence, KV head, split-K partition). Every 64-token tile of
// the partition's K and V rows for that KV head is staged once in LDS (fetched into registers one
// tile ahead, so global latency overlaps the current tile's arithmetic) and shared by all query
// heads of the group:
//   q.k : lane (token t/4, quarter t%4) dots its quarter of the K row with each query head
//         (q pre-scaled by D^-1/2 log2 e, fp32 in LDS), then the 4 quarters are summed with
//         shuffles;
//   softmax: each wave owns 16 tokens of every tile and keeps its own running (max, sum) per head,
//         the max found by a butterfly of shuffles across the wave;
//   p.v : lane l of a wave accumulates d in [l*D/64, +D/64) of every head over the wave's tokens.
// The four waves' states are merged through LDS at the end of the partition. Output is the same
// (m, l, o) partial, or the normalised row, as the MFMA variant produces, and uses the same merge.
#include "decode_common.h"

namespace ti {
namespace {

__device__ __forceinline__ void unpack2(uint32_t w, float& x, float& y, Bf16) {
  x = __uint_as_float(w << 16);
  y = __uint_as_float(w & 0xffff0000u);
}
__device__ __forceinline__ void unpack2(uint32_t w, float& x, float& y, F16) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, w);
  x = static_cast<float>(h[0]);
  y = static_cast<float>(h[1]);
}
__device__ __forceinline__ float to_float(uint16_t v, Bf16) {
  return __uint_as_float(uint32_t(v) << 16);
}
__device__ __forceinline__ float to_float(uint16_t v, F16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}
__device__ __forceinline__ uint16_t from_float(float v, Bf16) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}
__device__ __forceinline__ uint16_t from_float(float v, F16) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

template <int D, int G, typename Tag, int POL>
__global__ __launch_bounds__(256) void decode_scalar_kernel(DecodeArgs a) {
  constexpr int TT = 64;                // tokens per staged tile
  constexpr int ROW = D + 8;            // padded LDS row (16-bit elements)
  constexpr int QD = D / 4;             // d per lane in q.k
  constexpr int QROW = QD + 4;          // padded fp32 quarter-row of q
  constexpr int DPL = D / 64;           // d per lane in p.v
  constexpr int CPR = D / 8;            // 16-byte chunks per row
  constexpr int CPT = TT * CPR / 256;   // chunks per thread per tile (each of K and V)
  constexpr int GP = (G + 3) & ~3;      // padded head count of a p row
  static_assert(CPT * 256 == TT * CPR, "tile must split evenly over 256 lanes");
  static_assert(4 * G * D * 4 <= TT * ROW * 2, "wave states must fit the K tile buffer");

  __shared__ __align__(16) uint16_t sk[TT * ROW];
  __shared__ __align__(16) uint16_t sv[TT * ROW];
  __shared__ __align__(16) float sq[G * 4 * QROW];
  __shared__ __align__(16) float sp[4][16][GP];
  __shared__ int s_bids[kMaxSplitPages];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int b = blockIdx.z;

  const int ctx = seq_len(a, b);
  const int nsplit = (ctx + a.split_tokens - 1) / a.split_tokens;
  if (split >= (nsplit > 0 ? nsplit : 1)) return;  // uniform over the workgroup
  const int tok0 = split * a.split_tokens;
  const int tok1 = min(tok0 + a.split_tokens, ctx);
  const int page0 = tok0 / a.page_size;
  const int npages = tok1 > tok0 ? (tok1 - tok0 + a.page_size - 1) / a.page_size : 0;
  for (int i = t; i < npages; i += 256) s_bids[i] = a.block_table[b * a.bt_stride + page0 + i];
  {
    const uint16_t* qg = a.q + b * a.q_sb + int64_t(kvh) * G * a.q_sh;
    for (int i = t; i < G * D; i += 256) {
      const int h = i / D, d = i % D;
      sq[h * 4 * QROW + (d / QD) * QROW + d % QD] = to_float(qg[h * a.q_sh + d], Tag{}) * a.scale_log2;
    }
  }
  __syncthreads();

  auto row_bid = [&](int pos) -> int {  // block id of token `pos`, -1 when absent
    if (pos >= tok1) return -1;
    const int bid = s_bids[(pos - tok0) / a.page_size];
    return (bid >= 0 && bid < a.num_blocks32) ? bid : -1;
  };

  u32x4 pk[CPT], pv[CPT];
  auto fetch = [&](int t0) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int ci = t + 256 * k;
      const int row = ci / CPR, col = ci % CPR;
      const int pos = t0 + row;
      const int bid = row_bid(pos);
      if (bid >= 0) {
        const int64_t off = int64_t(bid) * a.page_stride + int64_t(pos % a.page_size) * a.row_stride +
                            int64_t(kvh) * D + 8 * col;
        pk[k] = load16_policy<POL>(a.k_cache + off);
        pv[k] = load16_policy<POL>(a.v_cache + off);
      } else {
        pk[k] = u32x4{0u, 0u, 0u, 0u};
        pv[k] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int ci = t + 256 * k;
      const int row = ci / CPR, col = ci % CPR;
      *reinterpret_cast<u32x4*>(sk + row * ROW + 8 * col) = pk[k];
      *reinterpret_cast<u32x4*>(sv + row * ROW + 8 * col) = pv[k];
    }
  };

  const int tj = t >> 2;  // q.k: token of the tile
  const int qq = t & 3;   //      quarter of the head dim
  float m_run[G], l_run[G], o[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[h][e] = 0.f;
  }

  const int ntiles = (tok1 - tok0 + TT - 1) / TT;
  if (ntiles > 0) fetch(tok0);
  for (int it = 0; it < ntiles; ++it) {
    const int t0 = tok0 + it * TT;
    stash();
    __syncthreads();
    if (it + 1 < ntiles) fetch(t0 + TT);

    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = 0.f;
    const uint16_t* krow = sk + tj * ROW + qq * QD;
    const float* qb = sq + qq * QROW;
#pragma unroll 2
    for (int c = 0; c < QD / 8; ++c) {
      const u32x4 kx = *reinterpret_cast<const u32x4*>(krow + 8 * c);
      float kf[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) unpack2(kx[w], kf[2 * w], kf[2 * w + 1], Tag{});
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const f32x4 q0 = *reinterpret_cast<const f32x4*>(qb + h * 4 * QROW + 8 * c);
        const f32x4 q1 = *reinterpret_cast<const f32x4*>(qb + h * 4 * QROW + 8 * c + 4);
        s[h] += kf[0] * q0[0] + kf[1] * q0[1] + kf[2] * q0[2] + kf[3] * q0[3] + kf[4] * q1[0] +
                kf[5] * q1[1] + kf[6] * q1[2] + kf[7] * q1[3];
      }
    }
    const bool valid = row_bid(t0 + tj) >= 0;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s[h] += __shfl_xor(s[h], 1, 64);
      s[h] += __shfl_xor(s[h], 2, 64);
      if (!valid) s[h] = -INFINITY;
      float mx = s[h];
      mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run[h], mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[h] - m_use);
      const float p = fast_exp2(s[h] - m_use);
      l_run[h] = l_run[h] * alpha + (qq == 0 ? p : 0.f);
      m_run[h] = m_new;
#pragma unroll
      for (int e = 0; e < DPL; ++e) o[h][e] *= alpha;
      if (qq == 0) sp[wave][tj & 15][h] = p;
    }
    __builtin_amdgcn_wave_barrier();

#pragma unroll 4
    for (int jj = 0; jj < 16; ++jj) {
      const uint16_t* vrow = sv + (wave * 16 + jj) * ROW + lane * DPL;
      float vf[DPL];
      if constexpr (DPL == 4) {
        const uint2 vx = *reinterpret_cast<const uint2*>(vrow);
        unpack2(vx.x, vf[0], vf[1], Tag{});
        unpack2(vx.y, vf[2], vf[3], Tag{});
      } else {
        const uint32_t vx = *reinterpret_cast<const uint32_t*>(vrow);
        unpack2(vx, vf[0], vf[1], Tag{});
      }
      float pr[GP];
#pragma unroll
      for (int h4 = 0; h4 < GP; h4 += 4) {
        const f32x4 p4 = *reinterpret_cast<const f32x4*>(&sp[wave][jj][h4]);
        pr[h4] = p4[0];
        pr[h4 + 1] = p4[1];
        pr[h4 + 2] = p4[2];
        pr[h4 + 3] = p4[3];
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[h][e] += pr[h] * vf[e];
      }
    }
    __syncthreads();
  }

  // Merge the four waves' states through LDS (the K tile buffer is free now).
  float* so = reinterpret_cast<float*>(sk);
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float l = l_run[h];
    l += __shfl_xor(l, 1, 64);
    l += __shfl_xor(l, 2, 64);
    l += __shfl_xor(l, 4, 64);
    l += __shfl_xor(l, 8, 64);
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
#pragma unroll
    for (int e = 0; e < DPL; ++e) so[(wave * G + h) * D + lane * DPL + e] = o[h][e];
    if (lane == 0) {
      sp[wave][0][h] = m_run[h];
      sp[wave][1][h] = l;
    }
  }
  __syncthreads();
  for (int d = t; d < D; d += 256) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, sp[w][0][h]);
      float L = 0.f, O = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float mw = sp[w][0][h];
          const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - M);
          L += f * sp[w][1][h];
          O += f * so[(w * G + h) * D + d];
        }
      }
      const int hq = kvh * G + h;
      if (nsplit <= 1) {
        a.out[(int64_t(b) * a.hq + hq) * D + d] = from_float(L > 0.f ? O / L : 0.f, Tag{});
      } else {
        const int64_t slot = (int64_t(b) * a.hq + hq) * a.max_splits + split;
        a.part_o[slot * D + d] = O;
        if (d == 0) {
          a.part_ml[2 * slot] = M;
          a.part_ml[2 * slot + 1] = L;
        }
      }
    }
  }
}

template <int D, int G, typename Tag>
void launch_gp(const DecodeArgs& a, dim3 grid, bool reuse_kv, hipStream_t stream) {
  if (reuse_kv) {
    hipLaunchKernelGGL((decode_scalar_kernel<D, G, Tag, kPolicyKeep>), grid, dim3(256), 0, stream, a);
  } else {
    hipLaunchKernelGGL((decode_scalar_kernel<D, G, Tag, kPolicyStream>), grid, dim3(256), 0, stream,
                       a);
  }
}

template <int D, typename Tag>
int launch_g(const DecodeArgs& a, int batch, bool reuse_kv, hipStream_t stream) {
  const dim3 grid(a.hkv, a.max_splits, batch);
  switch (a.group) {
    case 4:
      launch_gp<D, 4, Tag>(a, grid, reuse_kv, stream);
      break;
    case 6:
      launch_gp<D, 6, Tag>(a, grid, reuse_kv, stream);
      break;
    case 8:
      launch_gp<D, 8, Tag>(a, grid, reuse_kv, stream);
      break;
    default:
      return fail(TI_EUNSUPPORTED, "scalar decode: query group %d not built (4, 6, 8)", a.group);
  }
  return check_launch("ti_gqa_decode_paged (scalar)");
}

}  // namespace

int launch_decode_scalar(const DecodeArgs& a, int batch, bool bf16, int head_dim, bool reuse_kv,
                         hipStream_t stream) {
  if (head_dim == 256) {
    return bf16 ? launch_g<256, Bf16>(a, batch, reuse_kv, stream)
                : launch_g<256, F16>(a, batch, reuse_kv, stream);
  }
  if (head_dim == 128) {
    return bf16 ? launch_g<128, Bf16>(a, batch, reuse_kv, stream)
                : launch_g<128, F16>(a, batch, reuse_kv, stream);
  }
  return fail(TI_EUNSUPPORTED, "scalar decode: head_dim %d not built", head_dim);
}

}  // namespace ti
