// Paged GQA decode attention with split-K for gfx950 (MI355X).
//
// Replaces tileInfer's gqa_decode_paged_fn (kernels/gqa_decode_paged.py:392-437), whose TileLang
// kernels run one CTA per (sequence, KV head) over the whole context (44-177, 191-367). Here the
// context of every (sequence, KV head) is cut into split-K partitions; one wavefront owns one
// (sequence, KV head, partition), and the waves of a workgroup are the KV heads of one
// (sequence, partition), so a workgroup streams whole 2 KiB token rows (all KV heads) of each
// page. Partitions write unnormalised (m, l, o) partials that a second kernel merges in a fixed
// order; a sequence that fits one partition is normalised and written directly.
//
// Math (the reference's recipe, ref_gqa_decode_paged, kernels/gqa_decode_paged.py:444-461):
//   s_j = q . k_j * D^-1/2 ;  p = softmax(s) ;  o = p @ V,
// evaluated with an online softmax in base 2 (scores pre-scaled by D^-1/2 * log2 e, as the
// reference kernel does at 50 and 138-142), fp32 accumulation, P rounded to the cache dtype before
// the P.V product (as the reference kernel does at 148 and the torch recipe at 459-460).
//
// Matrix-core layout, per 16-token tile (lane l: row/column l%16, k-group g = l/16):
//   S^T[16 tokens x 16 heads] = K[16 tokens x 32 d] . Q^T[32 d x 16 heads]
//     v_mfma_f32_16x16x32 x D/32: A = K rows straight from the page (lane (m,g): token m,
//     d in [32kk+8g, +8)); B = the query group with rows >= group zero. The accumulator leaves
//     lane (n,g) holding tokens 4g..4g+3 of head n.
//   O^T[16 d x 16 heads] += V^T[16 d x 16 tokens] . P^T[16 tokens x 16 heads]
//     v_mfma_f32_16x16x16 x D/16: B = P exactly as the S^T accumulator holds it (lane (n,g):
//     tokens 4g..4g+3 of head n, no transpose); A = V gathered so that lane (m,g) owns
//     d = 128c+8m+e (e < 8) of tokens 4g..4g+3, paired with v_perm_b32. The accumulator leaves
//     lane (n,g) holding head n at d in [128c+32g, +32).
// Every O^T accumulator's head is its lane's head, so the softmax rescale needs no cross-lane
// traffic; only the running max crosses the 4 lanes that share a head.
#include <mutex>
#include <type_traits>
#include <vector>

#include "decode_common.h"

namespace ti {
namespace {

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c, Bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                   __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c, F16) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a),
                                               __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
}

// One 16-token tile of one KV head in MFMA operand layout.
template <int D>
struct Tile {
  u32x4 k[D / 32];      // [k-step]: row n, d in [32kk+8g, +8)
  u32x4 v[4][D / 128];  // [row 4g+r][chunk c]: d in [128c+8n, +8)
  // Tokens of the tile that exist (uniform): pages of 16 tokens or more, a count of leading rows;
  // smaller pages, a mask (bit t: row t is in the partition and its page's block id is valid).
  int rows;
};

// Zeros that the small-page loads of absent rows read instead (one head's row, 512 bytes).
__device__ __align__(16) uint16_t g_zero_row[256] = {};

// Issues one tile's K and V loads (MFMA operand layout) with cache policy P.
template <int D, int P>
__device__ __forceinline__ void issue_tile(Tile<D>& T, __amdgpu_buffer_rsrc_t rk,
                                           __amdgpu_buffer_rsrc_t rv, uint32_t lane_k,
                                           uint32_t lane_v, uint32_t row_bytes) {
#pragma unroll
  for (int kk = 0; kk < D / 32; ++kk) T.k[kk] = buffer_load16<P>(rk, lane_k + 64 * kk);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int c = 0; c < D / 128; ++c) T.v[r][c] = buffer_load16<P>(rv, lane_v + r * row_bytes + 256 * c);
  }
}

// The batch's first-column block ids in an LDS hash set with a count per id, so that a sequence
// can ask whether another sequence starts with the same block (kPolicyAuto). Open addressing with
// linear probing over `slots` (a power of two: four times the ids inserted, at most kShareSlots,
// so at least twice).
constexpr int kShareSlots = 4096;
constexpr int kShareMaxBatch = kShareSlots / 2;

// Multiplicative (Fibonacci) hashing: the top log2(slots) bits of id * 2654435761 (a prime near
// 2^32 / phi) modulo 2^32, which depend on every bit of the id. The product's low bits depend only on the id's low bits, and a free-list
// allocator gives equal-length sequences first blocks k * L apart: with those, every id would
// start its probe in one of a few slots (batch 256 at L = 512: probes of up to 256 slots, against
// 1 here; simulated on the host).
__device__ __forceinline__ uint32_t share_hash(int id, int slots) {
  return (uint32_t(id) * 2654435761u) >> (32 - __builtin_ctz(uint32_t(slots)));
}

__device__ __forceinline__ void share_insert(int* keys, int* counts, int slots, int id) {
  uint32_t h = share_hash(id, slots);
  for (int probe = 0; probe < slots; ++probe) {
    const int old = atomicCAS(&keys[h], -1, id);
    if (old == -1 || old == id) {
      atomicAdd(&counts[h], 1);
      return;
    }
    h = (h + 1) & uint32_t(slots - 1);
  }
}

// Count of `id` in the set (uniform: every lane probes the same slots).
__device__ __forceinline__ int share_count(const int* keys, const int* counts, int slots, int id) {
  uint32_t h = share_hash(id, slots);
  for (int probe = 0; probe < slots; ++probe) {
    const int k = keys[h];
    if (k == id) return counts[h];
    if (k == -1) return 0;
    h = (h + 1) & uint32_t(slots - 1);
  }
  return 0;
}

// Wave-wide inclusive prefix sum.
__device__ __forceinline__ int wave_inclusive_scan(int x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// Batches of at most this many 16-token tiles in all take runs of kShortChunkTiles: there the
// runs' one round of tile loads matters more than the merge's extra parts (graph-timed GPU time,
// same box: config 1's 32 tiles 14.3 -> 12.6 us, 4 sequences of 67 tiles 18.4 -> 14.6, 2 of 76
// 16.1 -> 14.7; one sequence of 128 tiles went 17.6 -> 18.4 with them, so it keeps 4).
constexpr int kShortBatchTiles = 96;
constexpr int kShortChunkTiles = 2;

// Total 16-token tiles of the batch and the balanced run length (same in every workgroup and in
// the merge: a pure function of the sequence lengths and the plan).
__device__ __forceinline__ int balanced_chunk(const DecodeArgs& a, int total_tiles) {
  const int per = (total_tiles + a.balanced_wgs - 1) / a.balanced_wgs;
  const int least = total_tiles <= kShortBatchTiles ? min(kShortChunkTiles, a.chunk_min_tiles)
                                                    : a.chunk_min_tiles;
  return max(per, least);
}

// SMALL: pages of 1, 2, 4 or 8 tokens (a 16-token tile spans 16 / page_size pages, so each lane
// addresses its own rows' pages with a 64-bit address); otherwise pages of a multiple of 16
// tokens (a tile lies in one page: one buffer descriptor per tile).
// WS (wave split): one workgroup per (sequence, KV head) whose WPB waves take consecutive tile
// ranges of the sequence and combine their parts through LDS (short contexts of small batches: no
// merge launch). Otherwise each wave is one KV head of the workgroup's group.
template <int D, typename Tag, int WPB, int POL, bool SMALL, bool WS = false>
__global__ __launch_bounds__(64 * WPB) void decode_mfma_kernel(DecodeArgs a, int batch) {
  constexpr int KK = D / 32;
  constexpr int NC = D / 128;
  constexpr int NT = D / 16;
  static_assert(D % 128 == 0, "head_dim must be a multiple of 128");

  // Block ids of the current partition: pages smaller than a tile take more slots per token.
  constexpr int kBidSlots = SMALL ? kMaxRunPagesSmall : kMaxSplitPages;
  __shared__ int s_bids[kBidSlots];
  __shared__ int s_part[WPB + 4];

  const int lane = threadIdx.x & 63;
  // Uniform across the wave; readfirstlane lets the compiler keep it (and every page address
  // derived from it) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;  // MFMA row/col index: token row of K, head of S^T/O^T, d-col of V^T
  const int g = lane >> 4;  // MFMA k-group
  const int kvh = WS ? int(blockIdx.x) : int(blockIdx.x) * WPB + wave;
  const int h = kvh * a.group + n;
  const bool head_ok = n < a.group;

  // Byte offsets of this lane's loads inside one 16-token tile of its KV head.
  const uint32_t row_bytes = uint32_t(a.row_stride) * 2;
  const uint32_t lane_k = uint32_t(n) * row_bytes + 16 * g;
  const uint32_t lane_v = uint32_t(4 * g) * row_bytes + 16 * n;

  u32x4 qop[KK];
  f32x4 o[NT];
  float m_run, l_run, l_tot;
  int tok0, tok1;

  // Cache policy of the current sequence's K/V loads (uniform). kPolicyAuto: the batch's
  // first-column block ids go into an LDS hash set here, and a sequence whose first block another
  // sequence also starts with loads with kPolicyKeep (its pages are read again by the others and
  // are then served from L2/MALL); every other sequence streams. Rows of an empty table (id -1:
  // the runner's graph padding) and ids outside the cache are left out. A barrier follows before
  // the first lookup (the balanced scan's, or the one below for fixed splits).
  bool keep = POL == kPolicyKeep;
  int share_slots = 0;  // 0: no set (batch too large), every sequence streams
  int* s_skey = nullptr;
  int* s_scnt = nullptr;
  if constexpr (POL == kPolicyAuto) {
    __shared__ int s_share_key[kShareSlots];
    __shared__ int s_share_cnt[kShareSlots];
    s_skey = s_share_key;
    s_scnt = s_share_cnt;
    if (batch <= kShareMaxBatch && a.max_blocks > 0) {  // uniform
      share_slots = 64;
      while (share_slots < 4 * batch && share_slots < kShareSlots) share_slots <<= 1;
    }
  }
  // One wave fills the set (a wave's LDS operations take effect in order, so its clear precedes
  // its inserts without a barrier): the last wave, while wave 0 runs the balanced scan, so the
  // set costs no time on the start-up path; with one wave per workgroup, wave 0 after its scan.
  // The barrier at the end of the scan (or the one below, for fixed splits) publishes it.
  // First block ids of sequences [j0, j0 + 512), one per lane and step (the loads issued
  // together), and their inserts into the set.
  auto share_load_chunk = [&](int j0, int (&ids)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int j = j0 + 64 * u + lane;
      ids[u] = j < batch ? a.block_table[int64_t(j) * a.bt_stride] : -1;
    }
  };
  auto share_insert_chunk = [&](const int (&ids)[8]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (uint32_t(ids[u]) < uint32_t(a.num_blocks32)) {
        share_insert(s_skey, s_scnt, share_slots, ids[u]);
      }
    }
  };
  // Clears the set and inserts every sequence's first block id; `first` holds the ids of the
  // first 512 sequences when the caller has already requested them (one memory latency with its
  // own loads), nullptr otherwise.
  auto build_share_set = [&](const int (*first)[8] = nullptr) {
    if constexpr (POL == kPolicyAuto) {
      if (share_slots == 0) return;
      for (int e = lane; e < share_slots; e += 64) {
        s_skey[e] = -1;
        s_scnt[e] = 0;
      }
      for (int j0 = 0; j0 < batch; j0 += 8 * 64) {
        if (j0 == 0 && first != nullptr) {
          share_insert_chunk(*first);
          continue;
        }
        int ids[8];
        share_load_chunk(j0, ids);
        share_insert_chunk(ids);
      }
    }
  };
  // Sets `keep` for sequence b from its first block id (loaded by the caller ahead of a barrier).
  auto choose_policy = [&](int first_id) {
    if constexpr (POL == kPolicyAuto) {
      keep = false;
      const int id = __builtin_amdgcn_readfirstlane(first_id);
      if (share_slots > 0 && uint32_t(id) < uint32_t(a.num_blocks32)) {
        keep = __builtin_amdgcn_readfirstlane(share_count(s_skey, s_scnt, share_slots, id)) > 1;
      }
    }
  };

  // Loads the 16-token tile at position p into `T`. Every load is issued unconditionally through
  // a buffer descriptor that spans only the tile's rows that exist (in the partition and with a
  // valid block id); rows past it read as zero with no memory access. Branch-free loads keep the
  // compiler's count of outstanding loads exact, so waiting for one tile never waits for the tile
  // prefetched behind it.
  auto load_tile = [&](Tile<D>& T, int p) {
    if constexpr (SMALL) {
      // tok0 and p are multiples of 16, hence of the page size: the tile's pages are the
      // partition's slots [slot0, slot0 + 16 / page_size).
      const int L = a.page_log2;
      const int slot0 = (p - tok0) >> L;
      const int nrows = max(min(tok1 - p, 16), 0);
      int mask = 0;
      for (int j = 0; j < (16 >> L); ++j) {  // uniform
        const int id = __builtin_amdgcn_readfirstlane(s_bids[min(slot0 + j, kBidSlots - 1)]);
        if (uint32_t(id) < uint32_t(a.num_blocks32)) mask |= ((1 << a.page_size) - 1) << (j << L);
      }
      mask &= (1 << nrows) - 1;
      // The address of one of this lane's rows (t), or of the zero row when t is absent.
      auto row_ptr = [&](const uint16_t* cache, int t, int col) -> const uint16_t* {
        if (!((mask >> t) & 1)) return g_zero_row + col;
        const int id = s_bids[min(slot0 + (t >> L), kBidSlots - 1)];
        return cache + int64_t(id) * a.page_stride + int64_t(t & (a.page_size - 1)) * a.row_stride +
               kvh * D + col;
      };
      auto issue = [&](auto pol) {
        constexpr int P = decltype(pol)::value;
        const uint16_t* kp = row_ptr(a.k_cache, n, 8 * g);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) T.k[kk] = load16_policy<P>(kp + 32 * kk);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint16_t* vp = row_ptr(a.v_cache, 4 * g + r, 8 * n);
#pragma unroll
          for (int c = 0; c < NC; ++c) T.v[r][c] = load16_policy<P>(vp + 128 * c);
        }
      };
      if constexpr (POL == kPolicyAuto) {
        if (keep) issue(std::integral_constant<int, kPolicyKeep>{});
        else issue(std::integral_constant<int, kPolicyStream>{});
      } else {
        issue(std::integral_constant<int, POL>{});
      }
      T.rows = mask;
      return;
    }
    // Past the partition end the LDS entry may be stale; `rows` is 0 there and masks it.
    const int slot = min(p / a.page_size - tok0 / a.page_size, kBidSlots - 1);
    const int id = __builtin_amdgcn_readfirstlane(s_bids[slot]);
    const bool ok = (tok1 - p > 0) && (uint32_t(id) < uint32_t(a.num_blocks32));
    const int rows = ok ? min(tok1 - p, 16) : 0;
    const int bid = ok ? id : 0;
    const int64_t base =
        int64_t(bid) * a.page_stride + int64_t(p % a.page_size) * a.row_stride + kvh * D;
    const uint32_t nbytes = rows > 0 ? uint32_t(rows - 1) * row_bytes + D * 2 : 0u;
    const auto rk = make_rsrc(a.k_cache + base, nbytes);
    const auto rv = make_rsrc(a.v_cache + base, nbytes);
    if constexpr (POL == kPolicyAuto) {
      if (keep) issue_tile<D, kPolicyKeep>(T, rk, rv, lane_k, lane_v, row_bytes);
      else issue_tile<D, kPolicyStream>(T, rk, rv, lane_k, lane_v, row_bytes);
    } else {
      issue_tile<D, POL>(T, rk, rv, lane_k, lane_v, row_bytes);
    }
    T.rows = rows;
  };

  auto compute_tile = [&](Tile<D>& T) {
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) s = mfma16x16x32(T.k[kk], qop[kk], s, Tag{});
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool present = SMALL ? ((T.rows >> (4 * g + r)) & 1) != 0 : 4 * g + r < T.rows;
      sv[r] = present ? s[r] * a.scale_log2 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sv[r] - m_use);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] *= alpha;
    }
    // P^T operand: element j <-> token 4g + j.
    u32x2 pop;
    pop[0] = pack2(p[0], p[1], Tag{});
    pop[1] = pack2(p[2], p[3], Tag{});
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // V^T operand of d-tile 8c+e: (V[4g][d], V[4g+1][d]), (V[4g+2][d], V[4g+3][d]).
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        u32x2 vop;
        vop[0] = __builtin_amdgcn_perm(T.v[1][c][e >> 1], T.v[0][c][e >> 1], sel);
        vop[1] = __builtin_amdgcn_perm(T.v[3][c][e >> 1], T.v[2][c][e >> 1], sel);
        o[8 * c + e] = mfma16x16x16(vop, pop, o[8 * c + e], Tag{});
      }
    }
  };

  // Fused append: the wave whose tokens end at the sequence's last token writes that token's K/V
  // rows (its KV head) before any of its tiles is loaded. Its own later loads of the row then see
  // them (`attend` waits for the stores before the first tile load); no other wave or workgroup
  // reads that row.
  auto append_row = [&](int b) {
    const int slot = __builtin_amdgcn_readfirstlane(a.app_slot[b]);
    if (slot >= 0 && slot < a.app_num_slots && lane < D / 8) {  // uniform slot test
      const int64_t dst = int64_t(slot) * a.row_stride + kvh * D + 8 * lane;
      const u32x4 kw = load16(a.app_k + b * a.app_k_sb + kvh * D + 8 * lane);
      const u32x4 vw = load16(a.app_v + b * a.app_v_sb + kvh * D + 8 * lane);
      *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.k_cache) + dst) = kw;
      *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.v_cache) + dst) = vw;
    }
  };

  // Query group of sequence b as the B operand of S^T = K . Q^T; rows beyond the group stay zero.
  auto load_q = [&](int b) {
    const uint16_t* qrow = a.q + b * a.q_sb + int64_t(h) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qop[kk] = head_ok ? load16(qrow + 32 * kk + 8 * g) : u32x4{0u, 0u, 0u, 0u};
    }
  };

  // Attention of this wave's query group over tokens [w0, w1) (16-aligned w0), with the query
  // loaded and the block ids of the workgroup's partition, from token t0 (16-aligned), staged in
  // LDS: leaves the unnormalised (o, m_run) and the head's denominator l_tot.
  auto attend = [&](int t0, int w0, int w1, bool appended) {
    tok0 = t0;
    tok1 = w1;
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run = -INFINITY;
    l_run = 0.f;
    if (appended) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the appended rows are written
    // Two tiles in flight: the next tile's loads are issued before the current one is consumed.
    const int ntiles = (w1 - w0 + 15) / 16;
    if (ntiles > 0) {
      Tile<D> ta, tb;
      load_tile(ta, w0);
      int it = 0;
      for (; it + 2 <= ntiles; it += 2) {
        const int p0 = w0 + 16 * it;
        load_tile(tb, p0 + 16);
        compute_tile(ta);
        if (it + 2 < ntiles) load_tile(ta, p0 + 32);
        compute_tile(tb);
      }
      if (it < ntiles) compute_tile(ta);
    }
    // Sum the per-lane partial denominators of each head (lanes n, n+16, n+32, n+48).
    l_tot = l_run + __shfl_xor(l_run, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
  };

  // Balanced runs: attention over tokens [t0, t1) of sequence b (16-aligned t0), staging the
  // partition's block ids in LDS. Uniform over the workgroup. `ends`: t1 is the sequence's end.
  auto run_partition = [&](int b, int t0, int t1, bool ends) {
    const bool appended = a.app_slot != nullptr && ends;
    if (appended) append_row(b);
    const int page0 = t0 / a.page_size;
    // The plan keeps every partition within kBidSlots pages; the clamp only guards LDS.
    const int npages = t1 > t0 ? min((t1 - 1) / a.page_size - page0 + 1, kBidSlots) : 0;
    // The sequence's first block id (cache policy), requested with the partition's block ids.
    const int first_id =
        (POL == kPolicyAuto && share_slots > 0 && npages > 0) ? a.block_table[b * a.bt_stride] : -1;
    __syncthreads();  // the previous partition's tiles are done with s_bids
    for (int i = threadIdx.x; i < npages; i += 64 * WPB) {
      s_bids[i] = a.block_table[b * a.bt_stride + page0 + i];
    }
    __syncthreads();
    choose_policy(first_id);
    load_q(b);
    attend(t0, t0, t1, appended);
  };

  // Fixed partitions and wave splits, whose tokens follow from the grid position: everything a
  // workgroup needs before its first tile is requested together, before the sequence length is
  // known (one memory latency instead of three): the query group, the block ids of `npages`
  // pages from page0 (staged in LDS; the host bound, not the length), the sequence's first block
  // id and, for the cache policy, the batch's (the share set, wave 0). Ends with a barrier;
  // returns the sequence's first block id.
  auto prologue = [&](int b, int page0, int npages) -> int {
    load_q(b);
    constexpr int kRegIds = 4;  // ids per thread held in registers; the rest after them
    int ids_r[kRegIds];
#pragma unroll
    for (int k = 0; k < kRegIds; ++k) {
      const int i = int(threadIdx.x) + k * 64 * WPB;
      ids_r[k] = i < npages ? a.block_table[b * a.bt_stride + page0 + i] : -1;
    }
    const int first_id =
        (POL == kPolicyAuto && share_slots > 0 && npages > 0) ? a.block_table[b * a.bt_stride] : -1;
    int share_ids[8];
    const bool share_wave = POL == kPolicyAuto && share_slots > 0 && wave == 0;
    if (share_wave) share_load_chunk(0, share_ids);
#pragma unroll
    for (int k = 0; k < kRegIds; ++k) {
      const int i = int(threadIdx.x) + k * 64 * WPB;
      if (i < npages) s_bids[i] = ids_r[k];
    }
    for (int i = int(threadIdx.x) + kRegIds * 64 * WPB; i < npages; i += 64 * WPB) {
      s_bids[i] = a.block_table[b * a.bt_stride + page0 + i];
    }
    if (share_wave) build_share_set(&share_ids);
    __syncthreads();
    return first_id;
  };

  auto store_out = [&](int b) {
    uint16_t* orow = a.out + (int64_t(b) * a.hq + h) * D;
    const uint16_t* grow = a.gate ? a.gate + b * a.gate_sb + int64_t(h) * a.gate_sh : nullptr;
    auto put = [&](int d, u32x4 w) __attribute__((always_inline)) {
      if (grow) {
        const u32x4 gv = load16(grow + d);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = gate_mul2(w[k], gv[k], Tag{});
      }
      *reinterpret_cast<u32x4*>(orow + d) = w;
    };
    // A row shorter than the shared prefix (the runner's graph-padding rows: context 1, no
    // pages) is outside the prefix contract and gets no prefix part: zeros, as plain decode.
    if (!a.pre_o || a.seqlen[b] < a.ctx_offset) {  // uniform
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          u32x4 w;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            w[k] = pack2(o[8 * c + 2 * k][r] * inv, o[8 * c + 2 * k + 1][r] * inv, Tag{});
          }
          put(128 * c + 32 * g + 8 * r, w);
        }
      }
      return;
    }
    // With the prefix parts (m_s, l_s, o_s): out = (w o + sum_s w_s o_s) / (w l + sum_s w_s l_s),
    // weights 2^(m - M) and 2^(m_s - M), M the largest maximum; parts in order.
    const int64_t r0 = int64_t(b) * a.hq + h;
    const int64_t part_rows = int64_t(batch) * a.hq;
    float mm = m_run;
    for (int s = 0; s < a.pre_parts; ++s) mm = fmaxf(mm, a.pre_ml[2 * (s * part_rows + r0)]);
    const float ws = m_run == -INFINITY ? 0.f : fast_exp2(m_run - mm);
    float l = ws * l_tot;
    for (int s = 0; s < a.pre_parts; ++s) {
      const float me = a.pre_ml[2 * (s * part_rows + r0)];
      l += (me == -INFINITY ? 0.f : fast_exp2(me - mm)) * a.pre_ml[2 * (s * part_rows + r0) + 1];
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 128 * c + 32 * g + 8 * r;
        float acc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = o[8 * c + k][r] * ws;
        for (int s = 0; s < a.pre_parts; ++s) {
          const int64_t pr = s * part_rows + r0;
          const float me = a.pre_ml[2 * pr];
          const float we = me == -INFINITY ? 0.f : fast_exp2(me - mm);
          const f32x4 e0 = *reinterpret_cast<const f32x4*>(a.pre_o + pr * D + d);
          const f32x4 e1 = *reinterpret_cast<const f32x4*>(a.pre_o + pr * D + d + 4);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            acc[k] += e0[k] * we;
            acc[4 + k] += e1[k] * we;
          }
        }
        u32x4 w;
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = pack2(acc[2 * k] * inv, acc[2 * k + 1] * inv, Tag{});
        put(d, w);
      }
    }
  };

  auto store_partial = [&](int64_t slot) {
    float* prow = a.part_o + slot * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        f32x4 w0 = {o[8 * c + 0][r], o[8 * c + 1][r], o[8 * c + 2][r], o[8 * c + 3][r]};
        f32x4 w1 = {o[8 * c + 4][r], o[8 * c + 5][r], o[8 * c + 6][r], o[8 * c + 7][r]};
        f32x4* dst = reinterpret_cast<f32x4*>(prow + 128 * c + 32 * g + 8 * r);
        dst[0] = w0;
        dst[1] = w1;
      }
    }
    if (g == 0) {
      a.part_ml[2 * slot] = m_run;
      a.part_ml[2 * slot + 1] = l_tot;
    }
  };

  if constexpr (WS) {
    // One workgroup per (KV head, sequence b): wave w takes the tiles [w per, (w + 1) per) of the
    // sequence; the parts are combined through LDS in wave order.
    __shared__ float s_comb[WPB][4 * NT + 2][64];  // each wave's o values, then m and l, per lane
    const int b = blockIdx.z;
    const int ctx = seq_len(a, b);
    const int first_id = prologue(b, 0, min(a.max_blocks, kBidSlots));
    choose_policy(first_id);
    const int ntiles = (ctx + 15) >> 4;
    const int per = (ntiles + WPB - 1) / WPB;
    const int w0 = min(wave * per * 16, ctx);
    const int w1 = min((wave + 1) * per * 16, ctx);
    const int owner = ntiles > 0 ? (ntiles - 1) / per : 0;  // the wave holding the last token
    const bool appended = a.app_slot != nullptr && wave == owner;
    if (appended) append_row(b);
    attend(0, w0, w1, appended);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s_comb[wave][4 * t + r][lane] = o[t][r];
    }
    s_comb[wave][4 * NT][lane] = m_run;
    s_comb[wave][4 * NT + 1][lane] = l_tot;
    __syncthreads();
    if (!head_ok) return;
    // m = max m_s, w_s = 2^(m_s - m), out = sum_s w_s o_s / sum_s w_s l_s, in wave order.
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < WPB; ++w) mm = fmaxf(mm, s_comb[w][4 * NT][lane]);
    float wt[WPB];
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < WPB; ++w) {
      const float ms = s_comb[w][4 * NT][lane];
      wt[w] = ms == -INFINITY ? 0.f : fast_exp2(ms - mm);
      l += wt[w] * s_comb[w][4 * NT + 1][lane];
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* orow = a.out + (int64_t(b) * a.hq + h) * D;
    const uint16_t* grow = a.gate ? a.gate + b * a.gate_sb + int64_t(h) * a.gate_sh : nullptr;
    // Output group (c, r): d = 128 c + 32 g + 8 r + e holds o[8 c + e][r]; groups dealt to waves.
    for (int q = wave; q < 4 * NC; q += WPB) {
      const int c = q >> 2, r = q & 3;
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
      for (int w = 0; w < WPB; ++w) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += wt[w] * s_comb[w][4 * (8 * c + e) + r][lane];
      }
      u32x4 v;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = pack2(acc[2 * k] * inv, acc[2 * k + 1] * inv, Tag{});
      const int d = 128 * c + 32 * g + 8 * r;
      if (grow) {
        const u32x4 gv = load16(grow + d);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = gate_mul2(v[k], gv[k], Tag{});
      }
      *reinterpret_cast<u32x4*>(orow + d) = v;
    }
    return;
  }

  if (a.balanced_wgs == 0) {
    // One workgroup per (sequence, partition of split_tokens).
    const int split = blockIdx.y;
    const int b = blockIdx.z;
    const int ctx = seq_len(a, b);
    const int t0 = split * a.split_tokens;
    // The partition's pages up to the host bound (the length is not known yet).
    const int t_end = min(t0 + a.split_tokens, a.max_blocks * a.page_size);
    const int page0 = t0 / a.page_size;
    const int first_id = prologue(
        b, page0, t_end > t0 ? min((t_end - 1) / a.page_size - page0 + 1, kBidSlots) : 0);
    const int nsplit = (ctx + a.split_tokens - 1) / a.split_tokens;
    if (split >= (nsplit > 0 ? nsplit : 1)) return;  // uniform over the workgroup
    choose_policy(first_id);
    const int t1 = min(t0 + a.split_tokens, ctx);
    const bool appended = a.app_slot != nullptr && t1 == ctx;
    if (appended) append_row(b);
    attend(t0, t0, t1, appended);
    if (!head_ok) return;
    if (nsplit <= 1) store_out(b);
    else store_partial((int64_t(b) * a.hq + h) * a.max_splits + split);
    return;
  }

  // Balanced: workgroup i takes tiles [i * chunk, (i + 1) * chunk) of the batch's concatenated
  // 16-token tiles. Wave 0 finds the first and last sequence of that run with a prefix scan.
  const int i = blockIdx.y;
  if (WPB > 1 && wave == WPB - 1) build_share_set();
  if (wave == 0) {
    // Lane l owns sequences [l K, l K + K), K = ceil(batch / 64): it sums their tile counts (the
    // loads issued together, so any batch costs about one memory latency), the lane sums are
    // prefix-scanned, and the blocks holding the run's first tile T0 and last tile T1 - 1 are
    // searched.
    const int K = (batch + 63) >> 6;
    const int j0 = min(lane * K, batch);
    const int j1 = min(j0 + K, batch);
    int mine = 0;
#pragma unroll 8
    for (int j = j0; j < j1; ++j) mine += seq_tiles(a, j);
    const int incl = wave_inclusive_scan(mine, lane);
    const int excl = incl - mine;
    const int tot = __shfl(incl, 63, 64);
    if (i == 0 && blockIdx.x == 0 && lane == 0 && a.seq_first_tile) a.seq_first_tile[batch] = tot;
    const int chunk = balanced_chunk(a, tot);
    const int T0 = i * chunk;
    const int T1 = min(T0 + chunk, tot);
    int b_first = -1, s_first = 0, b_last = -1;
    if (T0 < T1) {
      // Each of the two tiles lies in exactly one lane's block; the whole wave then scans that
      // block 64 sequences at a time (one memory latency per 64 of its K sequences).
      const int lf = __builtin_ctzll(
          __builtin_amdgcn_ballot_w64(mine > 0 && excl <= T0 && T0 < incl));
      const int ll = __builtin_ctzll(
          __builtin_amdgcn_ballot_w64(mine > 0 && excl <= T1 - 1 && T1 - 1 < incl));
      // The sequence holding tile t of lane `owner`'s block and the first tile of that sequence.
      auto locate = [&](int owner, int t, int& b_at, int& s_at) {
        const int jb = min(owner * K, batch);
        const int je = min(jb + K, batch);
        int base = __shfl(excl, owner, 64);
        if (K == 1) {  // uniform: the owner's block is its one sequence, already scanned
          b_at = jb;
          s_at = base;
          return;
        }
        for (int c0 = jb; c0 < je; c0 += 64) {
          const int j = c0 + lane;
          const int nt = j < je ? seq_tiles(a, j) : 0;
          const int inc = wave_inclusive_scan(nt, lane) + base;
          const int exc = inc - nt;
          const uint64_t hit = __builtin_amdgcn_ballot_w64(nt > 0 && exc <= t && t < inc);
          if (hit) {  // uniform
            const int src = __builtin_ctzll(hit);
            b_at = c0 + src;
            s_at = __shfl(exc, src, 64);
            return;
          }
          base = __shfl(inc, 63, 64);
        }
      };
      int s_last = 0;
      locate(lf, T0, b_first, s_first);
      locate(ll, T1 - 1, b_last, s_last);
    }
    if (lane == 0) {
      s_part[0] = T0;
      s_part[1] = T1;
      s_part[2] = b_first;
      s_part[3] = s_first;
      s_part[4] = b_last;
    }
    if (WPB == 1) build_share_set();
  }
  __syncthreads();
  const int T0 = __builtin_amdgcn_readfirstlane(s_part[0]);
  const int T1 = __builtin_amdgcn_readfirstlane(s_part[1]);
  const int b_first = __builtin_amdgcn_readfirstlane(s_part[2]);
  const int b_last = __builtin_amdgcn_readfirstlane(s_part[4]);
  if (T0 >= T1 || b_first < 0 || b_last < b_first) return;  // uniform: no work
  int sb = __builtin_amdgcn_readfirstlane(s_part[3]);
  for (int b = b_first; b <= b_last; ++b) {
    const int nb = __builtin_amdgcn_readfirstlane(seq_tiles(a, b));
    if (nb > 0) {
      const int t0 = max(T0, sb) - sb;
      const int t1 = min(T1, sb + nb) - sb;
      // The workgroup holding the sequence's first tile records where it starts for the merge.
      if (t0 == 0 && blockIdx.x == 0 && threadIdx.x == 0 && a.seq_first_tile) {
        a.seq_first_tile[b] = sb;
      }
      const int ctx = __builtin_amdgcn_readfirstlane(seq_len(a, b));
      const int p1 = min(16 * t1, ctx);
      run_partition(b, 16 * t0, p1, p1 == ctx);
      if (head_ok) {
        if (t0 == 0 && t1 == nb) {
          // With precomputed prefix parts a whole sequence's row goes to its own part slot and
          // the merge folds the prefix parts in (in parallel over rows, not one dependent load
          // round per part in this epilogue).
          if (a.whole_rows) store_partial(a.whole_row0 + int64_t(b) * a.hq + h);
          else store_out(b);
        } else {
          store_partial((int64_t(i) * 2 + (b == b_first ? 0 : 1)) * a.hq + h);
        }
      }
    }
    sb += nb;
  }
}

// Combines the partials of every (sequence, q-head) whose context was split over more than one
// workgroup, in workgroup order (deterministic): m = max m_s, w_s = 2^(m_s - m),
// out = sum w_s o_s / sum w_s l_s. In balanced mode it also writes the zero rows of empty
// sequences (no workgroup covers them).
// W > 1 (balanced batches of at most kNarrowMergeRows rows): W waves per row; a row cut into
// more than 64 parts has them split into W contiguous ranges, each summed in order by one wave,
// the ranges then added in wave order (deterministic; a row of 64 parts or fewer takes the
// one-wave path unchanged).
template <int D, typename Tag, int W>
__global__ __launch_bounds__(64 * W) void decode_merge_kernel(DecodeArgs a, int batch) {
  constexpr int PER = D / 64;  // d-values per thread
  typedef float PartVec __attribute__((ext_vector_type(PER)));  // one lane's piece of a part row
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = W > 1 ? __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6) : 0;
  const int d0 = lane * PER;
  uint16_t* orow = a.out + (int64_t(b) * a.hq + h) * D + d0;
  const uint16_t* grow = a.gate ? a.gate + b * a.gate_sb + int64_t(h) * a.gate_sh + d0 : nullptr;
  // Writes one pair of output values, through the sigmoid gate when there is one.
  auto put = [&](int j, uint32_t w) {
    if (grow) w = gate_mul2(w, *reinterpret_cast<const uint32_t*>(grow + j), Tag{});
    *reinterpret_cast<uint32_t*>(orow + j) = w;
  };
  // The precomputed prefix parts of this row (none for rows shorter than the prefix, see the
  // partial kernel's store_out): their largest maximum, and their weighted sum at a given maximum.
  const int64_t pr = int64_t(b) * a.hq + h;
  const int64_t part_rows = int64_t(batch) * a.hq;
  const bool pre = a.pre_o != nullptr && a.seqlen[b] >= a.ctx_offset;
  float me = -INFINITY;
  if (pre) {  // uniform; lane s reads part s's maximum
    for (int s0 = 0; s0 < a.pre_parts; s0 += 64) {
      if (s0 + lane < a.pre_parts) me = fmaxf(me, a.pre_ml[2 * ((s0 + lane) * part_rows + pr)]);
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) me = fmaxf(me, __shfl_xor(me, d, 64));
  }
  // acc += sum_s 2^(m_s - m) o_s, returns sum_s 2^(m_s - m) l_s, summed in part order. Lane s
  // computes part s's weights; the o rows are loaded 16 parts at a time before any is used, so
  // their latencies overlap (one dependent load per part cost config 5's merge ~11 us).
  auto add_pre = [&](float m, float* acc) -> float {
    float l = 0.f;
    for (int s0 = 0; s0 < a.pre_parts; s0 += 64) {
      float w = 0.f, wl = 0.f;
      if (s0 + lane < a.pre_parts) {
        const int64_t r = (s0 + lane) * part_rows + pr;
        const float ms = a.pre_ml[2 * r];
        w = ms == -INFINITY ? 0.f : fast_exp2(ms - m);
        wl = w * a.pre_ml[2 * r + 1];
      }
      const int cnt = __builtin_amdgcn_readfirstlane(min(64, a.pre_parts - s0));
      for (int j0 = 0; j0 < cnt; j0 += 16) {
        PartVec v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int j = min(j0 + u, cnt - 1);  // past cnt: a valid row, left out below
          v[u] = *reinterpret_cast<const PartVec*>(a.pre_o + ((s0 + j) * part_rows + pr) * D + d0);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if (j0 + u < cnt) {  // uniform
            const float wj = __shfl(w, j0 + u, 64);
            const float lj = __shfl(wl, j0 + u, 64);
#pragma unroll
            for (int q = 0; q < PER; ++q) acc[q] += wj * v[u][q];
            l += lj;
          }
        }
      }
    }
    return l;
  };
  int64_t slot0 = 0, stride = 1;
  int nparts = 0;
  int first_part_slot1 = 0;  // balanced: the first part sits in slot 1 of its workgroup
  if (a.balanced_wgs == 0) {
    slot0 = (int64_t(b) * a.hq + h) * a.max_splits;
    if constexpr (W == 1) {
      nparts = -1;  // the row's first parts are requested below, before its length is known
    } else {
      const int ctx = seq_len(a, b);
      nparts = (ctx + a.split_tokens - 1) / a.split_tokens;
      if (nparts <= 1) return;
    }
  } else {
    const int nb = seq_tiles(a, b);
    if (nb == 0 && wave != 0) return;  // uniform: one wave writes what follows
    if (nb == 0 && h == 0 && a.app_slot != nullptr) {
      // Fused append of a sequence no partial workgroup covers: its whole K/V row, here.
      const int slot = a.app_slot[b];
      if (slot >= 0 && slot < a.app_num_slots) {
        for (int64_t e = 8 * lane; e < a.row_stride; e += 8 * 64) {
          *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.k_cache) + slot * a.row_stride + e) =
              load16(a.app_k + b * a.app_k_sb + e);
          *reinterpret_cast<u32x4*>(const_cast<uint16_t*>(a.v_cache) + slot * a.row_stride + e) =
              load16(a.app_v + b * a.app_v_sb + e);
        }
      }
    }
    if (nb == 0) {  // no token of this kernel's range: zeros, or the prefix parts alone
      float e[PER];
#pragma unroll
      for (int q = 0; q < PER; ++q) e[q] = 0.f;
      float inv = 0.f;
      if (me != -INFINITY) {
        const float l = add_pre(me, e);
        inv = l > 0.f ? 1.f / l : 0.f;
      }
#pragma unroll
      for (int j = 0; j < PER; j += 2) put(j, pack2(e[j] * inv, e[j + 1] * inv, Tag{}));
      return;
    }
    // Where the sequence's tiles start in the batch's tile order, and the batch's total, as the
    // partial kernel recorded them.
    const int pre_tiles = __builtin_amdgcn_readfirstlane(a.seq_first_tile[b]);
    const int tot = __builtin_amdgcn_readfirstlane(a.seq_first_tile[batch]);
    const int chunk = balanced_chunk(a, tot);
    const int i0 = pre_tiles / chunk;
    const int i1 = (pre_tiles + nb - 1) / chunk;
    if (i0 == i1) {  // one workgroup covered the whole sequence
      if (!a.whole_rows) return;  // and wrote its row
      nparts = 1;  // its row waits in the sequence's whole-row slot for the prefix parts
      slot0 = a.whole_row0 + int64_t(b) * a.hq + h;
    } else {
      nparts = i1 - i0 + 1;
      first_part_slot1 = (i0 * chunk < pre_tiles) ? 1 : 0;
      slot0 = int64_t(i0) * 2 * a.hq + h;
      stride = 2 * a.hq;
    }
  }
  // Part s lives at slot0 + s * stride (+ hq for a first part stored as its workgroup's last).
  auto part = [&](int s) -> int64_t {
    return slot0 + s * stride + ((s == 0 && first_part_slot1) ? a.hq : 0);
  };
  if constexpr (W > 1) {
    if (nparts <= 64) {  // uniform
      if (wave != 0) return;
    } else {
      __shared__ float s_red[W - 1][PER + 1][64];  // the other waves' sums (o, then l)
      const int quarter = (nparts + W - 1) / W;
      const int p0 = min(wave * quarter, nparts);
      const int p1 = min(p0 + quarter, nparts);
      // This wave's first 16 part rows and the (m, l) of its first 64 parts are requested with
      // every part's maximum, so one memory latency covers all three.
      const int cnt0 = __builtin_amdgcn_readfirstlane(min(64, p1 - p0));
      PartVec v0[16];
      float ms_own = -INFINITY, ls_own = 0.f;  // (m, l) of part p0 + lane
      if (cnt0 > 0) {  // uniform
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          v0[u] = *reinterpret_cast<const PartVec*>(a.part_o + part(p0 + min(u, cnt0 - 1)) * D + d0);
        }
        if (lane < cnt0) {
          ms_own = a.part_ml[2 * part(p0 + lane)];
          ls_own = a.part_ml[2 * part(p0 + lane) + 1];
        }
      }
      float m = -INFINITY;
#pragma unroll 4
      for (int s0 = 0; s0 < nparts; s0 += 64) {
        const int s = s0 + lane;
        m = fmaxf(m, s < nparts ? a.part_ml[2 * part(s)] : -INFINITY);
      }
#pragma unroll
      for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
      m = fmaxf(m, me);
      float acc[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) acc[j] = 0.f;
      float l = 0.f;
      if (wave == 0 && me != -INFINITY) l = add_pre(m, acc);  // the prefix parts first
      if (m != -INFINITY) {
        for (int s0 = p0; s0 < p1; s0 += 64) {
          const int s = s0 + lane;
          float w = 0.f, wl = 0.f;
          if (s < p1) {
            const float ms = s0 == p0 ? ms_own : a.part_ml[2 * part(s)];
            w = ms == -INFINITY ? 0.f : fast_exp2(ms - m);
            wl = w * (s0 == p0 ? ls_own : a.part_ml[2 * part(s) + 1]);
          }
          const int cnt = __builtin_amdgcn_readfirstlane(min(64, p1 - s0));
          auto add_part = [&](int j, const PartVec& v) __attribute__((always_inline)) {
            const float wj = __shfl(w, j, 64);
            const float lj = __shfl(wl, j, 64);
#pragma unroll
            for (int q = 0; q < PER; ++q) acc[q] += wj * v[q];
            l += lj;
          };
          int j0 = 0;
          if (s0 == p0) {  // uniform: the first 16 rows, requested above
#pragma unroll
            for (int u = 0; u < 16; ++u) {
              if (u < cnt) add_part(u, v0[u]);  // uniform
            }
            j0 = 16;
          }
          for (; j0 < cnt; j0 += 16) {
            PartVec v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
              const int j = min(j0 + u, cnt - 1);
              v[u] = *reinterpret_cast<const PartVec*>(a.part_o + part(s0 + j) * D + d0);
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
              if (j0 + u < cnt) add_part(j0 + u, v[u]);  // uniform
            }
          }
        }
      }
      if (wave > 0) {
#pragma unroll
        for (int q = 0; q < PER; ++q) s_red[wave - 1][q][lane] = acc[q];
        s_red[wave - 1][PER][lane] = l;
      }
      __syncthreads();
      if (wave != 0) return;
      for (int w = 0; w < W - 1; ++w) {
#pragma unroll
        for (int q = 0; q < PER; ++q) acc[q] += s_red[w][q][lane];
        l += s_red[w][PER][lane];
      }
      const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
      for (int j = 0; j < PER; j += 2) put(j, pack2(acc[j] * inv, acc[j + 1] * inv, Tag{}));
      return;
    }
  }
  // The o rows of the first kBurst parts are requested ahead of the (m, l) loads: they do not
  // depend on the weights, so one memory latency covers both. Past nparts the last part's row is
  // read again (a valid row) and left out of the sum. nburst is uniform; readfirstlane lets the
  // compiler see it, so these are plain vector loads.
  // Fixed partitions (nparts < 0 here): the part slots follow from the host-known max_splits, so
  // the first rows and (m, l) are requested with the row's length, one memory latency for all;
  // slots past the row's parts hold no value of this call and are left out below.
  const int spec = nparts < 0 ? a.max_splits : nparts;
  constexpr int kBurst = 16;
  const int nburst = __builtin_amdgcn_readfirstlane(min(spec, kBurst));
  PartVec vb[kBurst];
#pragma unroll
  for (int u = 0; u < kBurst; ++u) {
    vb[u] = *reinterpret_cast<const PartVec*>(a.part_o + part(min(u, nburst - 1)) * D + d0);
  }
  float ms_first = -INFINITY, ls_first = 0.f;  // (m, l) of part `lane`
  if (lane < spec) {
    ms_first = a.part_ml[2 * part(lane)];
    ls_first = a.part_ml[2 * part(lane) + 1];
  }
  if (nparts < 0) {
    const int ctx = seq_len(a, b);
    nparts = (ctx + a.split_tokens - 1) / a.split_tokens;
    if (nparts <= 1) return;
  }
  // Maximum over the parts' m (and the prefix parts'), lane-parallel; lane s keeps the (m, l) of
  // part s (parts 0-63) for the weights below.
  float m = -INFINITY, ms0 = -INFINITY, ls0 = 0.f;
#pragma unroll 4
  for (int s0 = 0; s0 < nparts; s0 += 64) {  // unrolled: the loads of 4 steps issued together
    const int s = s0 + lane;
    float ms = -INFINITY;
    if (s < nparts) {
      if (s0 == 0) {
        ms = ms_first;
        ls0 = ls_first;
      } else {
        ms = a.part_ml[2 * part(s)];
      }
    }
    if (s0 == 0) ms0 = ms;
    m = fmaxf(m, ms);
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  m = fmaxf(m, me);
  float acc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) acc[j] = 0.f;
  float l = 0.f;
  if (me != -INFINITY) l = add_pre(m, acc);  // the prefix parts first (fixed order)
  if (m != -INFINITY) {
    // Parts in chunks of 64: lane s holds part s0+s's weight w and w * l; part j's are broadcast
    // when it is added. Summation order is fixed (ascending part) for o and for l.
    float ms = ms0, ls = ls0;  // (m, l) of part s0 + lane of the current chunk
    for (int s0 = 0; s0 < nparts; s0 += 64) {
      // The next chunk's (m, l) are requested now, ahead of this chunk's o rows.
      float ms_next = -INFINITY, ls_next = 0.f;
      if (s0 + 64 + lane < nparts) {
        ms_next = a.part_ml[2 * part(s0 + 64 + lane)];
        ls_next = a.part_ml[2 * part(s0 + 64 + lane) + 1];
      }
      const float w = ms == -INFINITY ? 0.f : fast_exp2(ms - m);
      const float wl = w * ls;
      const int cnt = __builtin_amdgcn_readfirstlane(min(64, nparts - s0));
      auto add_part = [&](int j, const PartVec& v) __attribute__((always_inline)) {
        const float wj = __shfl(w, j, 64);
        const float lj = __shfl(wl, j, 64);
#pragma unroll
        for (int q = 0; q < PER; ++q) acc[q] += wj * v[q];
        l += lj;
      };
      int j0 = 0;
      if (s0 == 0) {
#pragma unroll
        for (int u = 0; u < kBurst; ++u) {
          if (u < cnt) add_part(u, vb[u]);  // uniform
        }
        j0 = kBurst;
      }
      // The rest 16 at a time, loaded back to back so that their latencies overlap.
      for (; j0 < cnt; j0 += 16) {
        PartVec v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int j = min(j0 + u, cnt - 1);
          v[u] = *reinterpret_cast<const PartVec*>(a.part_o + part(s0 + j) * D + d0);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if (j0 + u < cnt) add_part(j0 + u, v[u]);  // uniform
        }
      }
      ms = ms_next;
      ls = ls_next;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int j = 0; j < PER; j += 2) put(j, pack2(acc[j] * inv, acc[j + 1] * inv, Tag{}));
}

template <int D, typename Tag, int WPB, bool SMALL>
void launch_mfma_pages(const DecodeArgs& a, int batch, int policy, hipStream_t stream) {
  const dim3 grid = a.balanced_wgs > 0 ? dim3(a.hkv / WPB, a.balanced_wgs, 1)
                                        : dim3(a.hkv / WPB, a.max_splits, batch);
  if (policy == kPolicyKeep) {
    hipLaunchKernelGGL((decode_mfma_kernel<D, Tag, WPB, kPolicyKeep, SMALL>), grid, dim3(64 * WPB),
                       0, stream, a, batch);
  } else if (policy == kPolicyStream) {
    hipLaunchKernelGGL((decode_mfma_kernel<D, Tag, WPB, kPolicyStream, SMALL>), grid,
                       dim3(64 * WPB), 0, stream, a, batch);
  } else {
    hipLaunchKernelGGL((decode_mfma_kernel<D, Tag, WPB, kPolicyAuto, SMALL>), grid, dim3(64 * WPB),
                       0, stream, a, batch);
  }
}

// Wave split: one 4-wave workgroup per (KV head, sequence), no merge.
template <int D, typename Tag, bool SMALL>
void launch_wave_split_pages(const DecodeArgs& a, int batch, int policy, hipStream_t stream) {
  const dim3 grid(a.hkv, 1, batch);
  if (policy == kPolicyKeep) {
    hipLaunchKernelGGL((decode_mfma_kernel<D, Tag, 4, kPolicyKeep, SMALL, true>), grid, dim3(256),
                       0, stream, a, batch);
  } else if (policy == kPolicyStream) {
    hipLaunchKernelGGL((decode_mfma_kernel<D, Tag, 4, kPolicyStream, SMALL, true>), grid,
                       dim3(256), 0, stream, a, batch);
  } else {
    hipLaunchKernelGGL((decode_mfma_kernel<D, Tag, 4, kPolicyAuto, SMALL, true>), grid, dim3(256),
                       0, stream, a, batch);
  }
}

template <int D, typename Tag, int WPB>
int launch_mfma(const DecodeArgs& a, int batch, int policy, hipStream_t stream) {
  if (a.page_size < 16) launch_mfma_pages<D, Tag, WPB, true>(a, batch, policy, stream);
  else launch_mfma_pages<D, Tag, WPB, false>(a, batch, policy, stream);
  return check_launch("ti_gqa_decode_paged (mfma)");
}

// Balanced calls merge with 8 waves per row up to kWideMergeRows rows (q-heads x sequences), 4 up
// to kMidMergeRows and 2 up to kNarrowMergeRows, one above. A sequence holding more than a quarter
// of the batch's tiles is cut into more than 64 parts (up to 256), in any batch, and the merge of
// its rows is a chain of dependent loads that the waves shorten; rows of 64 parts or fewer leave
// the extra waves idle, and those occupy wave slots (the merge holds 160 VGPRs: 12 waves per CU,
// 3,072 per round on 256 CUs, so rows x waves fit one round up to 1,536 rows at 2 waves and 768 at
// 4). Graph time per call, same box (24 q-heads per sequence):
// * 8 waves against 4 at one to four sequences: B = 1 x 32k 39.1 -> 37.1 us, B = 1 x 128k
//   95.9 -> 93.9, B = 2 x 64k 92.0 -> 90.8 (16 waves, 128 registers each, spill and are slower).
// * 4 waves against 1 above four: one 128k sequence and 4, 7 or 15 of 512 tokens 117.8 -> 97.8,
//   118.4 -> 98.6, 120.9 -> 101.7 us; 64k + 15 x 1k 83.1 -> 68.0; 32k + 31 x 256 60.2 -> 45.2;
//   uniform batches within 0.2 us (config 2, 16 x 8k, 32 x 2k). At 64 sequences 4 waves cost
//   uniform batches more than they save (64 x 1k 51.6 -> 53.3; 32k + 63 x 512 64.0 -> 54.1): the
//   1,536 rows' workgroups no longer fit one round of wave slots. 8 waves up to 32 sequences:
//   +1.0-2.0 us on uniform batches.
// * 2 waves against 1 at 33 to 64 sequences: 32k + 63 x 512 66.0 -> 59.6 us, 32k + 47 x 512
//   65.3 -> 57.6; uniform batches +0.1-0.25 us (64 x 1k 52.2 -> 52.4, 64 x 2k, 48 x 1k, 40 x 4k).
constexpr int kWideMergeRows = 4 * 24;
constexpr int kMidMergeRows = 32 * 24;
constexpr int kNarrowMergeRows = 64 * 24;

template <int D, typename Tag>
int launch_decode(const DecodeArgs& a, int batch, int policy, hipStream_t stream) {
  int rc;
  if (a.wave_split) {
    if (a.page_size < 16) launch_wave_split_pages<D, Tag, true>(a, batch, policy, stream);
    else launch_wave_split_pages<D, Tag, false>(a, batch, policy, stream);
    return check_launch("ti_gqa_decode_paged (mfma, wave split)");
  }
  if (a.hkv % 4 == 0) {
    rc = launch_mfma<D, Tag, 4>(a, batch, policy, stream);
  } else if (a.hkv % 2 == 0) {
    rc = launch_mfma<D, Tag, 2>(a, batch, policy, stream);
  } else {
    rc = launch_mfma<D, Tag, 1>(a, batch, policy, stream);
  }
  if (rc != TI_OK) return rc;
  // A row is cut into more than 64 parts only if its sequence spans more than 63 runs of the
  // shortest chunk, which the table's bound tells; otherwise the extra waves would only idle.
  const int64_t rows = int64_t(a.hq) * batch;
  const int64_t bound_tiles = (int64_t(a.max_blocks) * a.page_size + 15) / 16;
  if (a.balanced_wgs > 0 && rows <= kNarrowMergeRows &&
      bound_tiles > int64_t(63) * a.chunk_min_tiles) {
    const dim3 grid(a.hq, batch);
    if (rows <= kWideMergeRows) {
      hipLaunchKernelGGL((decode_merge_kernel<D, Tag, 8>), grid, dim3(64 * 8), 0, stream, a, batch);
    } else if (rows <= kMidMergeRows) {
      hipLaunchKernelGGL((decode_merge_kernel<D, Tag, 4>), grid, dim3(64 * 4), 0, stream, a, batch);
    } else {
      hipLaunchKernelGGL((decode_merge_kernel<D, Tag, 2>), grid, dim3(64 * 2), 0, stream, a, batch);
    }
    return check_launch("ti_gqa_decode_paged (merge)");
  }
  if (a.balanced_wgs > 0 || a.max_splits > 1) {
    hipLaunchKernelGGL((decode_merge_kernel<D, Tag, 1>), dim3(a.hq, batch), dim3(64), 0, stream, a,
                       batch);
    return check_launch("ti_gqa_decode_paged (merge)");
  }
  return TI_OK;
}

int64_t lcm64(int64_t x, int64_t y) {
  int64_t p = x, q = y;
  while (q) {
    int64_t t = p % q;
    p = q;
    q = t;
  }
  return x / p * y;
}

// Launch plans of one decode call. `split`/`max_splits`/`ws_fixed`: one workgroup per
// (sequence, partition of `split` tokens) -- the requested split, or the heuristic one for the
// scalar variant. `balanced_wgs`/`ws_balanced`: the MFMA variant's balanced mode when no split was
// requested (0 otherwise). `short_split`/`short_splits`/`ws_short`: the MFMA variant's plan when no
// split was requested and the context bound is short (0 otherwise; see plan()).
struct Plan {
  int32_t split = 0, max_splits = 1, balanced_wgs = 0, chunk_min_tiles = 0;
  int32_t short_split = 0, short_splits = 0;
  bool wave_split = false;  // short bounds of small batches: one workgroup per (KV head, sequence)
  int64_t ws_fixed = 0, ws_balanced = 0, ws_short = 0;
};

constexpr int kMinChunkTiles = 4;  // 64 tokens: shorter runs are dominated by start-up
// Short contexts: with a context bound of at most this many tokens, the MFMA variant's default is
// fixed partitions of the smallest split (32 tokens at page size 16) whenever they fit one round
// of workgroups. Each workgroup then knows its tokens from its grid position, so its block ids and
// query are requested with its sequence length instead of after the balanced plan's scan, and the
// merge needs no per-sequence first tile (graph time per call, same box, balanced -> fixed:
// B = 1 x 512 12.7 -> 11.4 us, B = 16 x U[16, 512] 20.0 -> 14.8, B = 8 x 512 16.5 -> 13.3,
// B = 64 x 128 19.9 -> 18.0, B = 8 x 1k 19.0 -> 18.3). At 2k-token bounds and above the balanced
// plan is faster (B = 2 x 2k 18.5 against 18.8, B = 8 x 2k 24.1 against 33.9): each row is cut into
// as many parts as the split allows and the merge reads them all.
constexpr int64_t kShortBoundTokens = 1024;
// Bounds of at most this many tokens (2 tiles per wave) take one 4-wave workgroup per (KV head,
// sequence) instead, when the pairs fit one round: the waves split the sequence's tiles and
// combine their parts in LDS, so there is no partial to write and no merge launch (graph time per
// call against the fixed split: B = 16 x 64 11.3 -> 6.8 us, B = 1 x 128 10.7 -> 7.8). With more
// tiles per wave the split is slower: a wave keeps two tiles in flight, so its tiles are a chain
// of memory latencies (B = 1 x 512 11.2 -> 14.4 us, B = 4 x 1k 14.6 -> 28.3; B = 16 x 256, 4 tiles
// per wave, 13.6 -> 13.3).
constexpr int64_t kWaveSplitBoundTokens = 128;
// Bounds of at most this many tokens also take one workgroup per (KV head, sequence) when the
// pairs fill three quarters to all of one round (192-256 on 256 CUs), whatever the fixed split
// would need: every CU then streams one pair's pages, and neither partials nor a merge launch
// are paid. Graph time per call, same box, against the plan these shapes took before (balanced):
// B = 64 x 512 32.7 -> 25.0 us, 64 x U[16, 512] 28.1 -> 21.0, 64 x U[1, 512] 24.9 -> 20.8,
// 48 x 512 30.1 -> 22.7, 56 x 384 26.4 -> 19.5, 64 x 256 23.0 -> 15.3, 64 x U[1, 256]
// 24.4 -> 13.2. The cost is one long sequence among short ones, whose pair is a chain of up to 8
// tiles per wave: 512 + 63 x 16 tokens 15.5 -> 19.0 us, 512 + 63 x 64 17.1 -> 19.4. Longer bounds
// make that chain the whole call (2,048 + 63 x 64 tokens 19.3 -> 59.6 us; 64 x U[64, 2048]
// 56.9 -> 67.1), so they keep the balanced plan, though uniform batches would gain (64 x 1k
// 51.5 -> 46.5, 64 x 2k 90.0 -> 83.8).
constexpr int64_t kPairRoundBoundTokens = 512;

int plan(int32_t batch, int32_t hq, int32_t hkv, int32_t D, int32_t page_size, int32_t max_blocks,
         int32_t split_req, Plan* out) {
  if (batch < 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0) {
    return fail(TI_EINVAL, "decode: bad head counts batch=%d hq=%d hkv=%d", batch, hq, hkv);
  }
  if (hq / hkv > 16) {
    return fail(TI_EUNSUPPORTED, "decode: query group %d exceeds the 16-row MFMA tile", hq / hkv);
  }
  if (D != 128 && D != 256) {
    return fail(TI_EUNSUPPORTED, "decode: head_dim %d not built (128, 256)", D);
  }
  if (page_size <= 0 || (page_size % 16 != 0 && 16 % page_size != 0)) {
    return fail(TI_EUNSUPPORTED,
                "decode: page_size %d is neither 1, 2, 4, 8 nor a positive multiple of 16",
                page_size);
  }
  if (max_blocks < 0) return fail(TI_EINVAL, "decode: max_blocks_per_seq %d < 0", max_blocks);
  const int64_t bound = int64_t(max_blocks) * page_size;
  if (bound > (int64_t(1) << 30)) {
    return fail(TI_EINVAL, "decode: context bound %lld too large", (long long)bound);
  }
  const int64_t unit = lcm64(32, page_size);
  const int64_t cus = device_cu_count();
  int64_t split;
  if (split_req > 0) {
    split = split_req;
    if (split % unit != 0 || split > kMaxSplitTokens || split / page_size > kMaxSplitPages) {
      return fail(TI_EINVAL,
                  "decode: split_tokens %d must be a multiple of %lld and <= %d tokens / %d pages",
                  split_req, (long long)unit, kMaxSplitTokens, kMaxSplitPages);
    }
  } else {
    // Fewest, longest partitions that still give every CU a workgroup: each workgroup pays a
    // start-up (block ids, first tile) and drain that nothing else on its CU hides, so on MI355X
    // one full round of long workgroups streams fastest (config 3: 8,192 tokens, 256 workgroups).
    const int64_t wpb = (hkv % 4 == 0) ? 4 : (hkv % 2 == 0) ? 2 : 1;  // waves per workgroup
    const int64_t wgs_per_split = int64_t(batch) * (hkv / wpb);
    split = kMaxSplitTokens;
    while (split > 256 && wgs_per_split * ceil_div(bound, split) < cus) split /= 2;
    split = ceil_div(split, unit) * unit;
    while (split / page_size > kMaxSplitPages) split -= unit;
    if (split <= 0) split = unit;
  }
  int64_t max_splits = bound > 0 ? ceil_div(bound, split) : 1;
  if (max_splits > 65535) return fail(TI_EINVAL, "decode: %lld partitions", (long long)max_splits);
  out->split = int32_t(split);
  out->max_splits = int32_t(max_splits);
  out->ws_fixed = max_splits > 1 ? int64_t(batch) * hq * max_splits * (D + 2) * 4 : 0;
  out->balanced_wgs = 0;
  out->ws_balanced = 0;
  if (split_req <= 0) {
    // Balanced mode: one round of workgroups over the batch's tiles, one wave (KV head) per SIMD:
    // cus * 4 / hkv runs per KV-head group, each a workgroup of the group's waves. (A second
    // resident wave per SIMD, which head_dim 128 has room for, measured ~2 % slower at 8k-16k
    // contexts: shorter runs pay more start-ups.) When runs that long would exceed the block ids
    // one workgroup stages in LDS (a run may start mid-page: one page of slack), whole further
    // rounds: a partial last round would run alone after the others and nearly double the time.
    // (Pages smaller than a tile: runs start on a tile, hence on a page, so no slack page.)
    const int64_t max_chunk = page_size >= 16 ? int64_t(kMaxSplitPages - 1) * (page_size / 16)
                                              : int64_t(kMaxRunPagesSmall) / (16 / page_size);
    const int64_t bound_tiles = ceil_div(bound, 16);
    const int64_t per_round = cus * 4 / hkv > 0 ? cus * 4 / hkv : 1;
    const int64_t needed = ceil_div(int64_t(batch) * bound_tiles, max_chunk);
    int64_t wgs = per_round;
    if (needed > wgs) wgs = ceil_div(needed, per_round) * per_round;
    if (wgs > 65535) return fail(TI_EINVAL, "decode: %lld balanced workgroups", (long long)wgs);
    out->balanced_wgs = int32_t(wgs);
    out->chunk_min_tiles = int32_t(kMinChunkTiles < max_chunk ? kMinChunkTiles : max_chunk);
    // Partials, then the [batch + 1] first-tile entries (rounded to 256 bytes).
    out->ws_balanced = wgs * 2 * hq * (D + 2) * 4 + (int64_t(batch) * 4 + 4 + 255) / 256 * 256;
    const int64_t wpb = (hkv % 4 == 0) ? 4 : (hkv % 2 == 0) ? 2 : 1;  // waves per workgroup
    const int64_t short_splits = ceil_div(bound, unit);
    if (bound > 0 && bound <= kShortBoundTokens &&
        int64_t(batch) * short_splits * (hkv / wpb) <= cus) {
      out->short_split = int32_t(unit);
      out->short_splits = int32_t(short_splits);
      out->ws_short = short_splits > 1 ? int64_t(batch) * hq * short_splits * (D + 2) * 4 : 0;
      out->wave_split = bound <= kWaveSplitBoundTokens && int64_t(batch) * hkv <= cus;
    }
    if (bound > 0 && bound <= kPairRoundBoundTokens && int64_t(batch) * hkv * 4 >= cus * 3 &&
        int64_t(batch) * hkv <= cus) {
      out->wave_split = true;
    }
  }
  return TI_OK;
}

// Workspace bytes a balanced ti_gqa_decode_paged_prefixed call needs beyond the plan's: one part
// row (o, then (m, l)) per (sequence, q-head) for the whole sequences.
int64_t prefixed_extra_bytes(int64_t batch, int64_t hq, int64_t D) { return batch * hq * (D + 2) * 4; }

// The launch shape a call takes from its plan, and the workspace that shape needs. Short context
// bounds take fixed partitions by default (see plan()); one workgroup per (KV head, sequence), with
// no workspace, up to kWaveSplitBoundTokens, and up to kPairRoundBoundTokens when the pairs fill
// most of one round; not with prefix parts, whose balanced suffix decode leaves whole rows for
// the merge to fold them in parallel (one more part row per (sequence, q-head)).
struct EntryShape {
  bool short_fixed, wave_split, balanced;
  int64_t ws_need;
};

EntryShape entry_shape(const Plan& pl, int kind, int32_t split_tokens, bool prefixed,
                       int32_t batch, int32_t num_q_heads, int32_t head_dim) {
  EntryShape e;
  e.short_fixed =
      kind != TI_DECODE_SCALAR && split_tokens <= 0 && pl.short_split > 0 && !prefixed;
  e.wave_split = kind != TI_DECODE_SCALAR && split_tokens <= 0 && !prefixed && pl.wave_split;
  e.balanced = kind != TI_DECODE_SCALAR && !e.short_fixed && !e.wave_split && pl.balanced_wgs > 0;
  e.ws_need = (e.balanced ? pl.ws_balanced
               : e.wave_split ? 0
               : e.short_fixed ? pl.ws_short
                               : pl.ws_fixed) +
              (e.balanced && prefixed ? prefixed_extra_bytes(batch, num_q_heads, head_dim) : 0);
  return e;
}

}  // namespace
}  // namespace ti

extern "C" int ti_gqa_decode_plan(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t page_size, int32_t max_blocks_per_seq,
                                  int32_t split_tokens, int32_t* split_tokens_out,
                                  int32_t* max_splits_out, int64_t* workspace_bytes_out) {
  if (!split_tokens_out || !max_splits_out || !workspace_bytes_out) {
    return ti::fail(TI_EINVAL, "ti_gqa_decode_plan: null output pointer");
  }
  ti::Plan p;
  const int rc = ti::plan(batch, num_q_heads, num_kv_heads, head_dim, page_size,
                          max_blocks_per_seq, split_tokens, &p);
  if (rc != TI_OK) return rc;
  if (split_tokens > 0) {
    *split_tokens_out = p.split;
    *max_splits_out = p.max_splits;
    *workspace_bytes_out = p.ws_fixed;
  } else {
    // The MFMA variant's plan: fixed partitions for short bounds, else balanced. The workspace
    // covers every plan of these bounds (the shared-prefix call's suffix decode is balanced, the
    // scalar variant has its own split).
    if (p.wave_split) {
      *split_tokens_out = 0;
      *max_splits_out = 0;
    } else if (p.short_split > 0) {
      *split_tokens_out = p.short_split;
      *max_splits_out = p.short_splits;
    } else {
      *split_tokens_out = 0;
      *max_splits_out = p.balanced_wgs;
    }
    const int64_t ws = p.ws_balanced > p.ws_fixed ? p.ws_balanced : p.ws_fixed;
    *workspace_bytes_out = ws > p.ws_short ? ws : p.ws_short;
  }
  return TI_OK;
}

namespace ti {
namespace {

int decode_entry(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                 const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
                 const int32_t* seqlen, void* out, void* workspace, int64_t workspace_bytes,
                 int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                 int32_t page_size, int64_t num_blocks, int32_t max_blocks_per_seq,
                 int32_t split_tokens, int32_t variant, int32_t dtype, const void* gate,
                 int64_t gate_stride_b, int64_t gate_stride_h, void* stream,
                 const float* pre_o = nullptr, const float* pre_ml = nullptr,
                 int32_t prefix_tokens = 0, int32_t prefix_parts = 0,
                 const void* app_key = nullptr, const void* app_value = nullptr,
                 int64_t app_key_stride = 0, int64_t app_value_stride = 0,
                 const int32_t* app_slot = nullptr, int64_t app_num_slots = 0) {
  if (dtype != TI_DTYPE_BF16 && dtype != TI_DTYPE_F16) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_decode_paged: dtype code %d is not bf16/fp16", dtype);
  }
  const int kind = variant & 0xF;
  const bool reuse_kv = (variant & TI_DECODE_REUSE_KV) != 0;
  const bool stream_kv = (variant & TI_DECODE_STREAM_KV) != 0;
  if ((kind != TI_DECODE_AUTO && kind != TI_DECODE_MFMA && kind != TI_DECODE_SCALAR) ||
      (variant & ~(0xF | TI_DECODE_REUSE_KV | TI_DECODE_STREAM_KV)) != 0 ||
      (reuse_kv && stream_kv)) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged: unknown variant/flags 0x%x", variant);
  }
  // The MFMA kernel's K/V cache policy: forced by a flag, else chosen per sequence on the device.
  const int policy = reuse_kv ? kPolicyKeep : stream_kv ? kPolicyStream : kPolicyAuto;
  Plan pl;
  int rc = plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_blocks_per_seq,
                split_tokens, &pl);
  if (rc != TI_OK) return rc;
  const EntryShape shape =
      entry_shape(pl, kind, split_tokens, pre_o != nullptr, batch, num_q_heads, head_dim);
  const bool short_fixed = shape.short_fixed;
  const bool wave_split = shape.wave_split;
  const bool balanced = shape.balanced;
  const int32_t split = short_fixed ? pl.short_split : pl.split;
  const int32_t max_splits = short_fixed ? pl.short_splits : pl.max_splits;
  // Balanced calls with prefix parts: whole sequences leave their rows in the extra part rows.
  const bool whole_rows = balanced && pre_o != nullptr;
  const int64_t ws_need = shape.ws_need;
  if (batch == 0) return TI_OK;
  if (!q || !k_cache || !v_cache || !block_table || !seqlen || !out) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged: null pointer");
  }
  if (num_blocks < 0 || block_table_stride < max_blocks_per_seq) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged: num_blocks=%lld, block_table_stride=%lld < %d",
                (long long)num_blocks, (long long)block_table_stride, max_blocks_per_seq);
  }
  if (q_stride_h % 8 != 0 || q_stride_b % 8 != 0 || q_stride_h < head_dim ||
      (reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(k_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(v_cache) & 15) || (reinterpret_cast<uintptr_t>(out) & 15)) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged: q/cache/out must be 16-byte aligned rows");
  }
  if (ws_need > 0 && (workspace == nullptr || workspace_bytes < ws_need ||
                      (reinterpret_cast<uintptr_t>(workspace) & 15))) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged: workspace of %lld bytes (16-byte aligned) needed",
                (long long)ws_need);
  }
  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k_cache = static_cast<const uint16_t*>(k_cache);
  a.v_cache = static_cast<const uint16_t*>(v_cache);
  a.row_stride = int64_t(num_kv_heads) * head_dim;
  a.page_stride = a.row_stride * page_size;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.seqlen = seqlen;
  a.out = static_cast<uint16_t*>(out);
  a.part_o = static_cast<float*>(workspace);
  const int64_t n_parts =
      (balanced ? int64_t(pl.balanced_wgs) * 2 * num_q_heads : int64_t(batch) * num_q_heads * max_splits) +
      (whole_rows ? int64_t(batch) * num_q_heads : 0);
  a.whole_rows = whole_rows ? 1 : 0;
  a.whole_row0 = int64_t(pl.balanced_wgs) * 2 * num_q_heads;
  a.part_ml = a.part_o ? a.part_o + n_parts * head_dim : nullptr;
  a.seq_first_tile =
      balanced && a.part_o ? reinterpret_cast<int32_t*>(a.part_ml + n_parts * 2) : nullptr;
  a.balanced_wgs = balanced ? pl.balanced_wgs : 0;
  a.wave_split = wave_split ? 1 : 0;
  a.chunk_min_tiles = pl.chunk_min_tiles;
  a.num_blocks32 = int32_t(num_blocks < INT32_MAX ? num_blocks : INT32_MAX);
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.page_size = page_size;
  a.page_log2 = 0;
  while ((1 << a.page_log2) < page_size && a.page_log2 < 30) ++a.page_log2;
  a.max_blocks = max_blocks_per_seq;
  a.max_splits = max_splits;
  a.split_tokens = split;
  a.scale_log2 = float(1.4426950408889634 / sqrt(double(head_dim)));
  if (gate != nullptr) {
    if (kind == TI_DECODE_SCALAR) {
      return fail(TI_EUNSUPPORTED, "ti_gqa_decode_paged_gated: the gate epilogue is built for "
                                   "the MFMA variant only");
    }
    if ((reinterpret_cast<uintptr_t>(gate) & 15) || gate_stride_b % 8 || gate_stride_h % 8) {
      return fail(TI_EINVAL, "ti_gqa_decode_paged_gated: gate rows must be 16-byte aligned");
    }
  }
  a.gate = static_cast<const uint16_t*>(gate);
  a.gate_sb = gate_stride_b;
  a.gate_sh = gate_stride_h;
  a.pre_o = pre_o;
  a.pre_ml = pre_ml;
  a.pre_parts = pre_o ? prefix_parts : 0;
  a.ctx_offset = prefix_tokens;
  if (pre_o != nullptr && kind == TI_DECODE_SCALAR) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_decode_paged_prefixed: MFMA variant only");
  }
  a.app_k = static_cast<const uint16_t*>(app_key);
  a.app_v = static_cast<const uint16_t*>(app_value);
  a.app_k_sb = app_key_stride;
  a.app_v_sb = app_value_stride;
  a.app_slot = app_slot;
  a.app_num_slots = app_num_slots;
  if (app_slot != nullptr) {
    const int64_t row = a.row_stride;
    if (kind == TI_DECODE_SCALAR) {
      return fail(TI_EUNSUPPORTED, "ti_gqa_decode_paged_append: MFMA variant only");
    }
    if (!app_key || !app_value || app_num_slots < 0 ||
        app_num_slots > num_blocks * int64_t(page_size) || app_key_stride < row ||
        app_value_stride < row || app_key_stride % 8 || app_value_stride % 8 ||
        (reinterpret_cast<uintptr_t>(app_key) & 15) ||
        (reinterpret_cast<uintptr_t>(app_value) & 15)) {
      return fail(TI_EINVAL,
                  "ti_gqa_decode_paged_append: key/value must be 16-byte aligned rows of at least "
                  "%lld elements (row strides %lld, %lld), num_slots %lld at most the cache's rows",
                  (long long)row, (long long)app_key_stride, (long long)app_value_stride,
                  (long long)app_num_slots);
    }
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf16 = dtype == TI_DTYPE_BF16;
  if (kind == TI_DECODE_SCALAR) {
    rc = launch_decode_scalar(a, batch, bf16, head_dim, reuse_kv, s);
    if (rc != TI_OK) return rc;
    if (max_splits > 1) {
      if (head_dim == 256) {
        if (bf16) hipLaunchKernelGGL((decode_merge_kernel<256, Bf16, 1>), dim3(num_q_heads, batch), dim3(64), 0, s, a, batch);
        else hipLaunchKernelGGL((decode_merge_kernel<256, F16, 1>), dim3(num_q_heads, batch), dim3(64), 0, s, a, batch);
      } else {
        if (bf16) hipLaunchKernelGGL((decode_merge_kernel<128, Bf16, 1>), dim3(num_q_heads, batch), dim3(64), 0, s, a, batch);
        else hipLaunchKernelGGL((decode_merge_kernel<128, F16, 1>), dim3(num_q_heads, batch), dim3(64), 0, s, a, batch);
      }
      return check_launch("ti_gqa_decode_paged (merge)");
    }
    return TI_OK;
  }
  if (head_dim == 256) {
    return bf16 ? launch_decode<256, Bf16>(a, batch, policy, s)
                : launch_decode<256, F16>(a, batch, policy, s);
  }
  return bf16 ? launch_decode<128, Bf16>(a, batch, policy, s)
              : launch_decode<128, F16>(a, batch, policy, s);
}

}  // namespace
}  // namespace ti

extern "C" int ti_gqa_decode_paged(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                   const void* k_cache, const void* v_cache,
                                   const int32_t* block_table, int64_t block_table_stride,
                                   const int32_t* seqlen, void* out, void* workspace,
                                   int64_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                                   int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                   int64_t num_blocks, int32_t max_blocks_per_seq,
                                   int32_t split_tokens, int32_t variant, int32_t dtype,
                                   void* stream) {
  return ti::decode_entry(q, q_stride_b, q_stride_h, k_cache, v_cache, block_table,
                          block_table_stride, seqlen, out, workspace, workspace_bytes, batch,
                          num_q_heads, num_kv_heads, head_dim, page_size, num_blocks,
                          max_blocks_per_seq, split_tokens, variant, dtype, nullptr, 0, 0, stream);
}

extern "C" int ti_gqa_decode_paged_append(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache, const void* v_cache,
    const int32_t* block_table, int64_t block_table_stride, const int32_t* seqlen, void* out,
    void* workspace, int64_t workspace_bytes, int32_t batch, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int64_t num_blocks,
    int32_t max_blocks_per_seq, int32_t split_tokens, int32_t variant, int32_t dtype,
    const void* key, const void* value, int64_t key_row_stride, int64_t value_row_stride,
    const int32_t* slot_mapping, int64_t num_slots, void* stream) {
  if (!slot_mapping) return ti::fail(TI_EINVAL, "ti_gqa_decode_paged_append: null slot_mapping");
  return ti::decode_entry(q, q_stride_b, q_stride_h, k_cache, v_cache, block_table,
                          block_table_stride, seqlen, out, workspace, workspace_bytes, batch,
                          num_q_heads, num_kv_heads, head_dim, page_size, num_blocks,
                          max_blocks_per_seq, split_tokens, variant, dtype, nullptr, 0, 0, stream,
                          nullptr, nullptr, 0, 0, key, value, key_row_stride, value_row_stride,
                          slot_mapping, num_slots);
}

// ---- No-allocation entry point -----------------------------------------------------------------
//
// For callers that cannot allocate (code under graph capture, tight serving loops): the split-K
// partials live in a file-scope device array instead of a caller workspace. The array's host-side
// name is not a device address; its address on each device comes from hipGetSymbolAddress, taken
// once per device with that device current, and only that address is passed to kernels. Every call
// on one device shares that device's array (calls that overlap on one GPU race on it). Nothing in
// it needs to start at zero: the merge reads only partial slots the partial kernel of the same
// call wrote.

namespace ti {
namespace {
constexpr int64_t kDecodeScratchBytes = int64_t(32) << 20;  // 32 MiB per GPU, held for the process
}  // namespace
}  // namespace ti

static __device__ __align__(256) unsigned char scratch[ti::kDecodeScratchBytes];

namespace ti {
namespace {

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device id: that device's address of `scratch`

// The device address of `scratch` on the device `stream` belongs to (the current device for the
// null stream), looked up on the first call for that device.
int decode_scratch(hipStream_t stream, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return fail(TI_ELAUNCH, "no-alloc decode: hipGetDevice: %s", hipGetErrorString(e));
  int dev = cur;
  if (stream != nullptr) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) {
      return fail(TI_ELAUNCH, "no-alloc decode: hipStreamGetDevice: %s", hipGetErrorString(e));
    }
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (dev >= static_cast<int>(g_scratch_ptr.size())) g_scratch_ptr.resize(dev + 1, nullptr);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
      return fail(TI_ELAUNCH, "no-alloc decode: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr) {
      return fail(TI_ELAUNCH, "no-alloc decode: hipGetSymbolAddress(scratch) on device %d: %s",
                  dev, hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TI_OK;
}

}  // namespace
}  // namespace ti

extern "C" int64_t ti_gqa_decode_scratch_bytes(void) { return ti::kDecodeScratchBytes; }

extern "C" int ti_gqa_decode_paged_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                           const void* k_cache, const void* v_cache,
                                           const int32_t* block_table,
                                           int64_t block_table_stride, const int32_t* seqlen,
                                           void* out, int32_t batch, int32_t num_q_heads,
                                           int32_t num_kv_heads, int32_t head_dim,
                                           int32_t page_size, int64_t num_blocks,
                                           int32_t max_blocks_per_seq, int32_t split_tokens,
                                           int32_t variant, int32_t dtype, void* stream) {
  using namespace ti;
  Plan pl;
  int rc = plan(batch, num_q_heads, num_kv_heads, head_dim, page_size, max_blocks_per_seq,
                split_tokens, &pl);
  if (rc != TI_OK) return rc;
  // The shape ti_gqa_decode_paged would take, and so the scratch this call uses.
  const int64_t need =
      entry_shape(pl, variant & 0xF, split_tokens, false, batch, num_q_heads, head_dim).ws_need;
  if (need > kDecodeScratchBytes) {
    return fail(TI_EINVAL,
                "ti_gqa_decode_paged_noalloc: this call needs %lld bytes of split-K scratch, the "
                "no-allocation entry point has %lld; use ti_gqa_decode_paged with a workspace",
                (long long)need, (long long)kDecodeScratchBytes);
  }
  if (batch == 0) return TI_OK;
  void* ws = nullptr;
  rc = decode_scratch(static_cast<hipStream_t>(stream), &ws);
  if (rc != TI_OK) return rc;
  return decode_entry(q, q_stride_b, q_stride_h, k_cache, v_cache, block_table,
                      block_table_stride, seqlen, out, ws, kDecodeScratchBytes, batch, num_q_heads,
                      num_kv_heads, head_dim, page_size, num_blocks, max_blocks_per_seq,
                      split_tokens, variant, dtype, nullptr, 0, 0, stream);
}

extern "C" int ti_gqa_decode_paged_gated(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
    const int32_t* seqlen, void* out, void* workspace, int64_t workspace_bytes, int32_t batch,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
    int64_t num_blocks, int32_t max_blocks_per_seq, int32_t split_tokens, int32_t variant,
    int32_t dtype, const void* gate, int64_t gate_stride_b, int64_t gate_stride_h,
    void* stream) {
  if (batch > 0 && gate == nullptr) {
    return ti::fail(TI_EINVAL, "ti_gqa_decode_paged_gated: null gate");
  }
  return ti::decode_entry(q, q_stride_b, q_stride_h, k_cache, v_cache, block_table,
                          block_table_stride, seqlen, out, workspace, workspace_bytes, batch,
                          num_q_heads, num_kv_heads, head_dim, page_size, num_blocks,
                          max_blocks_per_seq, split_tokens, variant, dtype, gate, gate_stride_b,
                          gate_stride_h, stream);
}

extern "C" int ti_gqa_decode_paged_prefixed(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
    const int32_t* seqlen, void* out, void* workspace, int64_t workspace_bytes, int32_t batch,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
    int64_t num_blocks, int32_t max_blocks_per_seq, int32_t split_tokens, int32_t variant,
    int32_t dtype, const void* gate, int64_t gate_stride_b, int64_t gate_stride_h,
    const float* prefix_o, const float* prefix_ml, int32_t prefix_parts, int32_t prefix_tokens,
    void* stream) {
  using namespace ti;
  if (batch > 0 && (prefix_o == nullptr || prefix_ml == nullptr)) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged_prefixed: null prefix part");
  }
  if (prefix_parts < 1 || prefix_parts > 65535) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged_prefixed: prefix_parts %d outside [1, 65535]",
                prefix_parts);
  }
  if (prefix_tokens < 0 || page_size <= 0 || prefix_tokens % page_size != 0 ||
      prefix_tokens / page_size > max_blocks_per_seq) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged_prefixed: prefix_tokens %d must be a multiple of "
                           "page_size within the table", prefix_tokens);
  }
  if ((reinterpret_cast<uintptr_t>(prefix_o) & 15) || (reinterpret_cast<uintptr_t>(prefix_ml) & 7)) {
    return fail(TI_EINVAL, "ti_gqa_decode_paged_prefixed: prefix o 16-byte, (m, l) 8-byte aligned");
  }
  // The kernel covers tokens from prefix_tokens on: its table starts at that page.
  const int32_t skip = prefix_tokens / page_size;
  return decode_entry(q, q_stride_b, q_stride_h, k_cache, v_cache,
                      block_table ? block_table + skip : nullptr, block_table_stride, seqlen, out,
                      workspace, workspace_bytes, batch, num_q_heads, num_kv_heads, head_dim,
                      page_size, num_blocks, max_blocks_per_seq - skip, split_tokens, variant,
                      dtype, gate, gate_stride_b, gate_stride_h, stream, prefix_o, prefix_ml,
                      prefix_tokens, prefix_parts);
}
