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
// Work unit: a workgroup = one (sequence, KV head, block of query tokens), whose rows are the
// (token, query head) pairs of the KV head's group, so each 64-key K/V tile staged in LDS is shared
// by every query head of the group (GQA packing) and each K/V operand read from LDS feeds C MFMAs
// (C column tiles of 16 rows per wave). Tiles are loaded straight from the pages one tile ahead,
// through per-page buffer descriptors. Each wave uses the transposed MFMA layout:
//   S^T[16 keys x 16 rows]  = K[16 keys x 32 d] . Q^T[32 d x 16 rows]       (16x16x32, D/32 steps)
//   O^T[16 d x 16 rows]    += V^T[16 d x 32 keys] . P^T[32 keys x 16 rows]   (16x16x32)
// so each accumulator's query row is its lane's column and the softmax stays inside the lane.
#include "decode_common.h"

namespace ti {
namespace {

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
  int32_t tq;  // query tokens per workgroup: floor(64 * C / group)
  float scale_log2;
};

// A staged tile holds NS 16-key sub-tiles (each inside one page): kKT = 16 * NS keys. Four
// (64 keys) measured 1-3 % faster than two in a same-process A/B on MI355X.
constexpr int kPrefillSubTiles = 4;
constexpr float kRescaleSlack = 8.f;  // exp2 units a row maximum may rise before O is rescaled

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// ds_read_b64_tr_b16 (measured on gfx950): within each 16-lane group, output lane j receives
// element j % 4 of the 8-byte rows addressed by lanes j/4, j/4 + 4, j/4 + 8, j/4 + 12.
__device__ __forceinline__ u32x2 lds_read_tr4(const uint16_t* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}

// LDS slot of 16-byte chunk c of K/V tile row r is c ^ lds_swizzle(r). On gfx950 a ds_read_b128
// serves 16 lanes per cycle over 64 banks: lanes {0-3, 12-15, 20-23, 24-27} together, then
// {4-11, 16-19, 28-31}, and the same for lanes 32-63 (measured with SQ_LDS_BANK_CONFLICT). With
// this swizzle both MFMA operand reads of the tile -- K rows across lanes, V rows across
// 16-lane groups -- hit 16 distinct bank quads per cycle, for head_dim 128 and 256.
__device__ __forceinline__ int lds_swizzle(int r) { return (r ^ ((r << 1) & 8)) & 15; }

// V tiles are read only by ds_read_b64_tr_b16, which serves 32 consecutive lanes per cycle (8 bytes
// each, measured the same way); the V operand reads of one half-wave touch 8 rows, 4 lanes per 32
// bytes of a row, so XOR-ing the chunk index with 2r puts every row's 32 bytes on distinct banks.
__device__ __forceinline__ int lds_swizzle_v(int r) { return (2 * r) & 14; }

// Max over the four 16-lane rows of the wave (lanes n, n+16, n+32, n+48).
__device__ __forceinline__ float row_group_max(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row_group_sum(float x) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// One workgroup = one (sequence, KV head, block of tq query tokens); its rows are the
// (token, query head) pairs of that KV head's group, row = token * group + head-in-group, 64*C rows
// over 4 waves (C column tiles of 16 rows per wave). Every staged K/V tile is thus shared by all
// query heads of the group, and every K/V operand read from LDS feeds C MFMAs.
//
// K/V tiles go from the pages straight into LDS (buffer loads with the LDS destination), two
// stages in distinct arrays so that the compiler's wait counting tells the stage being loaded from
// the stage being read. LDS rows are unpadded and swizzled (lds_swizzle) so that the MFMA operand
// reads are free of bank conflicts.
template <int D, int C, int W, int NS, typename Tag>
__global__ __launch_bounds__(64 * W) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kKT = 16 * NS;
  constexpr int KK = D / 32;
  constexpr int NT = D / 16;
  constexpr int CPR = D / 8;              // 16-byte chunks per row
  constexpr int RPB = 1024 / (2 * D);     // rows per 1 KiB load (64 lanes x 16 bytes)
  constexpr int LPW = kKT / RPB / W;      // 1 KiB loads per wave per tile, each of K and V
  static_assert(LPW * RPB * W == kKT && 16 % (kKT / W) == 0,
                "each wave's loads must lie inside one sub-tile");

  __shared__ __align__(1024) uint16_t sk0[kKT * D];
  __shared__ __align__(1024) uint16_t sv0[kKT * D];
  __shared__ __align__(1024) uint16_t sk1[kKT * D];
  __shared__ __align__(1024) uint16_t sv1[kKT * D];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const int kvh = blockIdx.x;
  const int b = blockIdx.z;
  const int G = a.group;

  const int q_start = min(max(a.cu_q[b], 0), a.total_q);
  const int q_len = min(max(a.cu_q[b + 1], q_start), a.total_q) - q_start;
  // Heaviest query blocks (latest tokens, longest causal range) are dispatched first.
  const int qb0 = (gridDim.y - 1 - blockIdx.y) * a.tq;
  if (qb0 >= q_len) return;  // uniform over the workgroup
  int kv_len = a.seqlen_k[b];
  const int cap = a.max_blocks * a.page_size;
  kv_len = kv_len < 0 ? 0 : (kv_len > cap ? cap : kv_len);
  const int offset = kv_len - q_len;  // query i sits at absolute position offset + i
  const int tq = min(a.tq, q_len - qb0);

  // This lane's C rows.
  bool row_ok[C];
  int q_pos[C];
  u32x4 qop[C][KK];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int rho = wave * 16 * C + 16 * c + n;
    const int tok = rho / G;
    const int hh = rho - tok * G;
    row_ok[c] = tok < tq;
    q_pos[c] = a.causal ? offset + qb0 + tok : INT32_MAX;
    const uint16_t* qrow =
        a.q + int64_t(q_start + qb0 + tok) * a.q_st + int64_t(kvh * G + hh) * a.q_sh + 8 * g;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qop[c][kk] = row_ok[c] ? load16(qrow + 32 * kk) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  f32x4 o[C][NT];
  float m_run[C], l_run[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
#pragma unroll
    for (int i = 0; i < NT; ++i) o[c][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[c] = -INFINITY;
    l_run[c] = 0.f;
  }

  // Keys the workgroup can see: j < kv_len, and j < offset + qb0 + tq under the causal mask.
  int k_end = a.causal ? min(kv_len, offset + qb0 + tq) : kv_len;
  if (k_end < 0) k_end = 0;
  const int ntiles = (k_end + kKT - 1) / kKT;
  // Under the causal mask, keys past this one are masked for every row of the wave.
  const int wave_tok = min(tq - 1, ((wave + 1) * 16 * C - 1) / G);
  const int wave_last_key = a.causal ? offset + qb0 + wave_tok : INT32_MAX;
  // Keys up to this one are visible to every row of the wave.
  const int wave_first_key = a.causal ? offset + qb0 + (wave * 16 * C) / G : INT32_MAX;

  // V^T operand addresses for the transposed reads, fixed for the whole kernel: lane (s, g)
  // (s = lane % 16) points at key row 16h + 4g + s/4 and columns d0 + 4(s%4) .. +3, so the read
  // gives output lane m the values V[16h + 4g + i][d0 + m], i = 0..3 -- the k-slots 8g + 4h + i
  // of the A operand (keys 4g + i of sub-tile h, matching P). voff[h][dt % 8] is the element
  // offset inside a stage of d-tile dt's piece; d-tiles dt and dt + 8 differ by 128 elements
  // (the swizzle only permutes chunks inside each group of 16).
  int voff[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int r = 16 * hh + 4 * g + (n >> 2);
    const int sw = lds_swizzle_v(r);
#pragma unroll
    for (int dl = 0; dl < 8; ++dl) {
      const int y = 2 * dl + ((n & 3) >> 1);
      voff[hh][dl] = r * D + ((y ^ sw) * 8) + (n & 1) * 4;
    }
  }
  const uint32_t row_bytes = uint32_t(a.row_stride) * 2u;
  const int32_t* bt_row = a.block_table + int64_t(b) * a.bt_stride;

  // Block ids of the next tile to load (uniform), fetched one tile ahead of their use.
  int nbid[NS], nrows[NS];
  auto load_ids = [&](int k0) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int key0 = k0 + 16 * j;
      int rows = min(max(kv_len - key0, 0), 16);
      int id = rows > 0 ? bt_row[key0 / a.page_size] : 0;
      if (uint32_t(id) >= uint32_t(a.num_blocks32)) {
        rows = 0;  // absent page: masked, never loaded
        id = 0;
      }
      nbid[j] = id;
      nrows[j] = rows;
    }
  };
  // Rows of each sub-tile that exist in the two stages (uniform).
  int rows_st[2][NS];
  // The sub-tile this wave loads (kKT / W rows per wave, inside one sub-tile).
  const int my_sub = (wave * (kKT / W)) / 16;
  // Issue this wave's loads of the tile at key k0 into stage (sk, sv). A sub-tile lies in one
  // page; its loads use a buffer descriptor spanning only the rows that exist, so rows past the
  // context or in an absent page land in LDS as zero without a memory access.
  auto fetch = [&](uint16_t* sk, uint16_t* sv, int (&rows_out)[NS], int k0) {
    int bid = nbid[0], rows = nrows[0];
#pragma unroll
    for (int j = 1; j < NS; ++j) {
      if (my_sub == j) {
        bid = nbid[j];
        rows = nrows[j];
      }
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) rows_out[j] = nrows[j];
    bid = __builtin_amdgcn_readfirstlane(bid);
    rows = __builtin_amdgcn_readfirstlane(rows);
    const int key0 = k0 + 16 * my_sub;
    const int64_t base = int64_t(bid) * a.page_stride +
                         int64_t(key0 % a.page_size) * a.row_stride + int64_t(kvh) * D;
    const uint32_t nbytes = rows > 0 ? uint32_t(rows - 1) * row_bytes + D * 2 : 0u;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(a.k_cache + base, nbytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v_cache + base, nbytes);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int blk = wave * LPW + i;                  // 1 KiB block of the tile (uniform)
      const int row = blk * RPB + lane / CPR;          // tile row of this lane's chunk
      const int slot = lane % CPR;
      const int chunk_k = slot ^ lds_swizzle(row);
      const int chunk_v = slot ^ lds_swizzle_v(row);
      const uint32_t off_k = uint32_t(row & 15) * row_bytes + uint32_t(chunk_k) * 16u;
      const uint32_t off_v = uint32_t(row & 15) * row_bytes + uint32_t(chunk_v) * 16u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)(sk + blk * 512), 16, off_k, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)(sv + blk * 512), 16, off_v, 0, 0, 0);
    }
  };

  auto compute = [&](const uint16_t* sk, const uint16_t* sv, const int (&rows_in)[NS], int k0) {
    // S^T of each sub-tile that holds a key some row of the wave can see; the rest stay zero.
    f32x4 s[NS][C];
    int rows[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int c = 0; c < C; ++c) s[j][c] = f32x4{0.f, 0.f, 0.f, 0.f};
      rows[j] = 0;
      if (k0 + 16 * j <= wave_last_key) {  // uniform
        rows[j] = rows_in[j];
        u32x4 kop[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          kop[kk] = *reinterpret_cast<const u32x4*>(
              sk + (16 * j + n) * D + (((4 * kk + g) ^ lds_swizzle(n)) * 8));
        }
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
          for (int c = 0; c < C; ++c) s[j][c] = mfma16x16x32(kop[kk], qop[c][kk], s[j][c], Tag{});
        }
      }
    }
    // A tile wholly below the wave's diagonal with every key present needs no mask (uniform).
    bool full = k0 + kKT - 1 <= wave_first_key;
#pragma unroll
    for (int j = 0; j < NS; ++j) full = full && rows[j] == 16;
    u32x4 pop[C][NS / 2];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      float v[4 * NS];
      if (full) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
#pragma unroll
          for (int r = 0; r < 4; ++r) v[4 * j + r] = s[j][c][r];
        }
      } else {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i0 = 4 * g + r;
            const bool ok = row_ok[c] & (i0 < rows[j]) & (k0 + 16 * j + i0 <= q_pos[c]);
            v[4 * j + r] = ok ? s[j][c][r] : -INFINITY;
          }
        }
      }
      float mx = v[0];
#pragma unroll
      for (int i = 1; i < 4 * NS; ++i) mx = fmaxf(mx, v[i]);
      mx = row_group_max(mx) * a.scale_log2;
      // The running maximum (exp2 units) moves only when the tile's maximum exceeds it by more
      // than kRescaleSlack: P then stays <= 2^kRescaleSlack and O is rescaled rarely. Which
      // maximum is used cancels in O / l; it only sets the scale at which P is rounded.
      const bool grow = mx > m_run[c] + kRescaleSlack;
      const float m_next = grow ? mx : m_run[c];
      const float alpha = grow ? fast_exp2(m_run[c] - m_next) : 1.f;
      const float m_use = (m_next == -INFINITY) ? 0.f : m_next;
      float p[4 * NS];
#pragma unroll
      for (int i = 0; i < 4 * NS; ++i) p[i] = fast_exp2(fmaf(v[i], a.scale_log2, -m_use));
      float psum = 0.f;
#pragma unroll
      for (int h = 0; h < NS / 2; ++h) {
        psum += ((p[8 * h] + p[8 * h + 1]) + (p[8 * h + 2] + p[8 * h + 3])) +
                ((p[8 * h + 4] + p[8 * h + 5]) + (p[8 * h + 6] + p[8 * h + 7]));
      }
      l_run[c] = l_run[c] * alpha + psum;
      m_run[c] = m_next;
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
        for (int i = 0; i < NT; ++i) o[c][i] *= alpha;
      }
#pragma unroll
      for (int h = 0; h < NS / 2; ++h) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          pop[c][h][w] = pack2(p[8 * h + 2 * w], p[8 * h + 2 * w + 1], Tag{});
        }
      }
    }
    // O^T[16 d x 16 rows] += V^T[16 d x 32 keys] . P^T[32 keys x 16 rows] per pair of sub-tiles,
    // d-tile dt covering d = 16 dt .. 16 dt + 15; the A operand comes from two transposed reads.
#pragma unroll
    for (int h = 0; h < NS / 2; ++h) {
      if (k0 + 32 * h > wave_last_key) continue;  // uniform: every P of the pair is zero
#pragma unroll
      for (int dt = 0; dt < NT; ++dt) {
        const int dh = dt >> 3, dl = dt & 7;
        const u32x2 lo = lds_read_tr4(sv + 32 * h * D + voff[0][dl] + 128 * dh);
        const u32x2 hi = lds_read_tr4(sv + 32 * h * D + voff[1][dl] + 128 * dh);
        const u32x4 vop = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int c = 0; c < C; ++c) o[c][dt] = mfma16x16x32(vop, pop[c][h], o[c][dt], Tag{});
      }
    }
  };

  if (ntiles > 0) {
    load_ids(0);
    fetch(sk0, sv0, rows_st[0], 0);
    if (ntiles > 1) load_ids(kKT);
  }
  // Two tiles per trip so that each stage is a compile-time array.
  for (int it = 0; it < ntiles; it += 2) {
    __syncthreads();  // stage 0 holds tile it; every wave is done with stage 1
    if (it + 1 < ntiles) {
      fetch(sk1, sv1, rows_st[1], (it + 1) * kKT);
      if (it + 2 < ntiles) load_ids((it + 2) * kKT);
    }
    if (it * kKT <= wave_last_key) compute(sk0, sv0, rows_st[0], it * kKT);
    if (it + 1 >= ntiles) break;
    __syncthreads();  // stage 1 holds tile it + 1; every wave is done with stage 0
    if (it + 2 < ntiles) {
      fetch(sk0, sv0, rows_st[0], (it + 2) * kKT);
      if (it + 3 < ntiles) load_ids((it + 3) * kKT);
    }
    if ((it + 1) * kKT <= wave_last_key) compute(sk1, sv1, rows_st[1], (it + 1) * kKT);
  }

#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float l_tot = row_group_sum(l_run[c]);
    if (!row_ok[c]) continue;
    const int rho = wave * 16 * C + 16 * c + n;
    const int tok = rho / G;
    const int hh = rho - tok * G;
    uint16_t* orow =
        a.out + int64_t(q_start + qb0 + tok) * a.o_st + int64_t(kvh * G + hh) * a.o_sh;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    // Lane (n, g) holds d = 16 dt + 4g .. +3 of its row in o[c][dt].
#pragma unroll
    for (int dt = 0; dt < NT; ++dt) {
      u32x2 w;
      w[0] = pack2(o[c][dt][0] * inv, o[c][dt][1] * inv, Tag{});
      w[1] = pack2(o[c][dt][2] * inv, o[c][dt][3] * inv, Tag{});
      *reinterpret_cast<u32x2*>(orow + 16 * dt + 4 * g) = w;
    }
  }
}

template <int D, int C, int W, int NS>
void launch_prefill(const PrefillArgs& a0, int batch, int max_q, bool bf16, hipStream_t s) {
  PrefillArgs a = a0;
  a.tq = (16 * C * W) / a.group;
  const dim3 grid(unsigned(a.hkv), unsigned(ceil_div(max_q, a.tq)), unsigned(batch));
  if (bf16) hipLaunchKernelGGL((prefill_mfma_kernel<D, C, W, NS, Bf16>), grid, dim3(64 * W), 0, s, a);
  else hipLaunchKernelGGL((prefill_mfma_kernel<D, C, W, NS, F16>), grid, dim3(64 * W), 0, s, a);
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
  if (num_q_heads / num_kv_heads > 64) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: %d query heads per KV head (max 64)",
                num_q_heads / num_kv_heads);
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == TI_DTYPE_BF16;
  if (head_dim == 256) launch_prefill<256, 1, 8, kPrefillSubTiles>(a, batch, max_seqlen_q, bf16, s);
  else launch_prefill<128, 2, 8, kPrefillSubTiles>(a, batch, max_seqlen_q, bf16, s);
  return check_launch("ti_gqa_prefill_paged");
}
