// Causal GQA prefill attention that reads K/V straight from the paged cache (gfx950).
//
// Replaces tileInfer's chunked-prefill attention, which first gathers every cached position of the
// sequence through the block table into contiguous K/V copies (model/qwen_36.py:1030-1044) and then
// runs varlen flash attention on them (kernels/gqa_varlen.py:40-185, dispatch 369-389). Here the
// cache pages are the operand: no gather copy, any number of sequences per call (one launch per
// unit schedule; schedule + attention + merge launches for the balanced one, see below).
//
// Semantics (kernels/gqa_varlen.py:88-131, 144-175): sequence b has q_len = cu_q[b+1] - cu_q[b]
// query tokens and kv_len = seqlen_k[b] cached tokens (the chunk's own K/V already appended); the
// causal mask is bottom-right aligned, query i sees keys j <= kv_len - q_len + i. Scores are scaled
// by D^-1/2 log2 e and exponentiated in base 2, P is rounded to the cache dtype before P.V, fp32
// accumulation, a row with no visible key is zero. `causal = 0` drops the causal mask (every query
// sees all kv_len keys), the reference's is_causal=False. As in the decode kernel, a block id
// outside [0, num_blocks) inside the context is an absent page: its keys are masked, never loaded.
//
// Work unit: (sequence, KV head, block of query tokens), whose rows are the (token, query head)
// pairs of the KV head's group; a workgroup computes one unit (or, balanced, a run of key tiles
// over consecutive units), so each K/V tile staged in LDS (32 or 64 keys) is shared
// by every query head of the group (GQA packing) and each K/V operand read from LDS feeds C MFMAs
// (C column tiles of 16 rows per wave). Tiles are loaded straight from the pages one tile ahead,
// through per-page buffer descriptors. Each wave uses the transposed MFMA layout:
//   S^T[16 keys x 16 rows]  = K[16 keys x 32 d] . Q^T[32 d x 16 rows]       (16x16x32, D/32 steps)
//   O^T[16 d x 16 rows]    += V^T[16 d x 32 keys] . P^T[32 keys x 16 rows]   (16x16x32)
// so each accumulator's query row is its lane's column and the softmax stays inside the lane.
#include <atomic>
#include <type_traits>

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
  int32_t page_shift;  // log2(page_size) when it is a power of two, else -1
  int32_t tq;        // query tokens per unit: floor(rows per workgroup / group)
  int32_t key_tile;  // keys per staged tile
  float scale_log2;
  // Balanced schedule (balanced_wgs > 0; see prefill_plan_kernel), else one workgroup per unit.
  int32_t balanced_wgs, max_pairs, min_chunk;
  int32_t* plan;   // schedule tables
  float* part_o;   // [balanced_wgs][2][rows][D] unnormalised partial rows
  float* part_ml;  // [balanced_wgs][2][rows][2] their (m, l), m in exp2 units
  // Optional sigmoid gate of the output (out = attention * sigmoid(gate)), [total_q, hq, D] at
  // these strides; nullptr for the plain output.
  const uint16_t* gate;
  int64_t gate_st, gate_sh;
  // Unnormalised output (instead of out): fp32 o relative to 2^m, [key_splits][total_q][hq][D],
  // and (m, l) [key_splits][total_q][hq][2], m in exp2 units; nullptr for the normalised output.
  float* uo;
  float* uml;
  // Per-unit schedule only: each unit's key tiles are cut into key_splits contiguous ranges, one
  // workgroup each (grid z = sequence * key_splits + split), and split s writes its unnormalised
  // part to slot s of uo / uml (a range with no key writes m = -inf, l = 0, o = 0). 1 otherwise.
  int32_t key_splits;
};

constexpr float kRescaleSlack = 8.f;  // exp2 units a row maximum may rise before O is rescaled
constexpr int kMinChunkTiles = 11;    // shortest run of key tiles of a balanced workgroup
constexpr int kXcds = 8;              // MI355X: 8 XCDs of 32 CUs, one L2 each
// A unit's start-up and epilogue (Q load, pipeline fill, output or partial store), priced in key
// tiles. Measured: a causal 2,048-token first chunk (units of 1..64 tiles) takes 125 us at 2,
// 109 at 4, 97.5 at 6, 96 at 9 and 100 at 14; long units (a 8,192-key continuation) do not move.
constexpr int kUnitCost = 9;
static_assert(kMinChunkTiles > kUnitCost, "every balanced run must reach a key tile");

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One 1 KiB load into LDS: lane i's 16 bytes at rsrc + voff land at LDS byte lds + 16 i. Issued
// as assembly, which the compiler's wait insertion does not see: its own waits for the loads it
// knows stay at least as strict (vector memory operations complete in issue order, so hidden
// loads only add to what a count waits for), and the kernel waits for these loads explicitly
// before each stage barrier. The builtin form instead makes the compiler wait for every load
// into a stage array before reading that array, all loads issued since included, which defeats
// a pipeline that keeps two tiles in flight.
__device__ __forceinline__ void load_lds16(u32x4 rsrc, uint32_t voff, const uint16_t* lds) {
  const uint32_t m0 = uint32_t(reinterpret_cast<uintptr_t>((lds_ptr_t)(lds)));
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(m0)
               : "memory");
}

// The cache row at byte offset `off` from `base`.
__device__ __forceinline__ const uint16_t* at_bytes(const uint16_t* base, uint64_t off) {
  return reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(base) + off);
}

// Buffer descriptor words of [base, base + bytes) (raw, no stride), uniform.
__device__ __forceinline__ u32x4 rsrc_words(const uint16_t* base, uint32_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  return u32x4{uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(addr)))),
               uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(addr >> 32) & 0xffffu))),
               uint32_t(__builtin_amdgcn_readfirstlane(int(bytes))), uint32_t(kBufferRsrcWord3)};
}
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

// Query and key extent of sequence b, clamped as the entry point documents.
struct SeqExtent {
  int q_start, q_len, kv_len;
  int offset;  // query i sits at absolute position offset + i
};

__device__ __forceinline__ SeqExtent seq_extent(const PrefillArgs& a, int b) {
  SeqExtent s;
  s.q_start = min(max(a.cu_q[b], 0), a.total_q);
  s.q_len = min(max(a.cu_q[b + 1], s.q_start), a.total_q) - s.q_start;
  const int kv = a.seqlen_k[b];
  const int cap = a.max_blocks * a.page_size;
  s.kv_len = kv < 0 ? 0 : (kv > cap ? cap : kv);
  s.offset = s.kv_len - s.q_len;
  return s;
}

// Keys the query block starting at qb0 can see: j < kv_len, and j < offset + qb0 + tq under the
// causal mask.
__device__ __forceinline__ int block_key_end(const PrefillArgs& a, const SeqExtent& s, int qb0) {
  const int tq = min(a.tq, s.q_len - qb0);
  const int k_end = a.causal ? min(s.kv_len, s.offset + qb0 + tq) : s.kv_len;
  return k_end < 0 ? 0 : k_end;
}

// Keys the rows [r0, r0 + rows) of a sequence's (token, query head) rows can see (row = token *
// group + head): j < kv_len, and j <= offset + the last row's token under the causal mask.
__device__ __forceinline__ int rows_key_end(const PrefillArgs& a, const SeqExtent& s, int r0,
                                            int rows) {
  const int last_tok = (r0 + min(rows, s.q_len * a.group - r0) - 1) / a.group;
  const int k_end = a.causal ? min(s.kv_len, s.offset + last_tok + 1) : s.kv_len;
  return k_end < 0 ? 0 : k_end;
}

// Balanced schedule. A unit is (KV head, sequence, query block); its work is kUnitCost plus its key
// tiles (the fixed part prices a unit's start-up and epilogue in tiles). Units are concatenated KV
// head major, then by (sequence, query block) "pair", and run i of R takes work
// [floor(i T / R), floor((i + 1) T / R)) of the concatenation's T, so every workgroup gets the same
// work whatever the mix of prompt and context lengths (R: one per workgroup, fewer when a run
// would be shorter than min_chunk tiles). A sequence's query blocks are listed shortest and
// longest alternately (0, n - 1, 1, n - 2, ...): under a causal mask their works then sum in
// pairs to about two runs, so run boundaries fall on every other unit's end and half as many
// units are cut. A unit's key tiles sit at the end of its work; a unit cut between
// workgroups is finished by each as an unnormalised partial (slot 0 when it is the workgroup's
// first unit, 1 when its last) and merged afterwards in workgroup order. The tables, in the
// workspace (int32):
//   header   {pairs, work per KV head, runs, total work}
//   per pair {sequence, query block, key tiles, exclusive prefix of work}   (max_pairs each)
//   per workgroup {KV head, pair} of its first unit                        (balanced_wgs each)
struct PlanView {
  int32_t *hdr, *pair_b, *pair_qb, *pair_nt, *pair_pre, *wg_kvh, *wg_p;
};

__device__ __forceinline__ PlanView plan_view(const PrefillArgs& a) {
  PlanView v;
  v.hdr = a.plan;
  v.pair_b = a.plan + 4;
  v.pair_qb = v.pair_b + a.max_pairs;
  v.pair_nt = v.pair_qb + a.max_pairs;
  v.pair_pre = v.pair_nt + a.max_pairs;
  v.wg_kvh = v.pair_pre + a.max_pairs;
  v.wg_p = v.wg_kvh + a.balanced_wgs;
  return v;
}

int64_t plan_ints(int64_t max_pairs, int64_t wgs) { return 4 + 4 * max_pairs + 2 * wgs; }

constexpr int kPlanThreads = 1024;
constexpr int kMaxPlanSeqs = 8192;  // sequences of one balanced launch (first pairs kept in LDS)

__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

// Inclusive scan of x over the workgroup; `total` receives the workgroup's sum.
__device__ int block_incl_scan(int x, int* s_w, int& total) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int incl = wave_incl_scan(x, lane);
  if (lane == 63) s_w[w] = incl;
  __syncthreads();
  int pre = 0, tot = 0;
  for (int i = 0; i < kPlanThreads / 64; ++i) {
    const int y = s_w[i];
    pre += i < w ? y : 0;
    tot += y;
  }
  __syncthreads();  // s_w is reused by the next scan
  total = tot;
  return pre + incl;
}

// One workgroup builds the schedule tables from cu_seqlens_q / seqlen_k (device values, so the
// launch sequence stays free of host reads).
__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(PrefillArgs a, int batch) {
  __shared__ int s_off[kMaxPlanSeqs + 1];
  __shared__ int s_w[kPlanThreads / 64];
  const int t = threadIdx.x;
  const PlanView v = plan_view(a);
  // First pair of every sequence (query blocks of the sequences before it).
  int carry = 0;
  for (int b0 = 0; b0 < batch; b0 += kPlanThreads) {
    const int b = b0 + t;
    const int nq = b < batch ? (seq_extent(a, b).q_len + a.tq - 1) / a.tq : 0;
    int tot;
    const int incl = block_incl_scan(nq, s_w, tot);
    if (b < batch) s_off[b] = carry + incl - nq;
    carry += tot;
  }
  if (t == 0) s_off[batch] = carry;
  __syncthreads();
  // Cannot exceed max_pairs for non-decreasing cu_seqlens_q; a malformed one loses the excess.
  const int n_pairs = min(carry, a.max_pairs);
  // Key tiles of every pair and the exclusive prefix of their work.
  int work = 0;
  for (int p0 = 0; p0 < n_pairs; p0 += kPlanThreads) {
    const int p = p0 + t;
    int nt = 0;
    if (p < n_pairs) {
      int lo = 0, hi = batch;  // s_off[lo] <= p < s_off[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_off[mid] <= p) lo = mid;
        else hi = mid;
      }
      const int k = p - s_off[lo];
      const int nq = s_off[lo + 1] - s_off[lo];
      const int qb = (k & 1) ? nq - 1 - (k >> 1) : (k >> 1);
      nt = (block_key_end(a, seq_extent(a, lo), qb * a.tq) + a.key_tile - 1) / a.key_tile;
      v.pair_b[p] = lo;
      v.pair_qb[p] = qb;
      v.pair_nt[p] = nt;
    }
    const int w = nt > 0 ? nt + kUnitCost : 0;
    int tot;
    const int incl = block_incl_scan(w, s_w, tot);
    if (p < n_pairs) v.pair_pre[p] = work + incl - w;
    work += tot;
  }
  const int64_t total = int64_t(a.hkv) * work;
  const int64_t wgs = a.balanced_wgs;
  const int64_t runs = max(int64_t(1), min(wgs, total / a.min_chunk));
  if (t == 0) {
    v.hdr[0] = n_pairs;
    v.hdr[1] = work;
    v.hdr[2] = int32_t(runs);
    v.hdr[3] = int32_t(total);
  }
  for (int i = t; i < wgs; i += kPlanThreads) v.wg_p[i] = -1;
  __syncthreads();  // the -1 defaults land before the starts below
  // Workgroup i starts in the unit holding work position floor(i * total / runs) (units without
  // key tiles hold none; a position in a unit's fixed part starts that unit at its first key tile).
  const int units = a.hkv * n_pairs;
  for (int u = t; u < units; u += kPlanThreads) {
    const int kvh = u / n_pairs;
    const int p = u - kvh * n_pairs;
    const int nt = v.pair_nt[p];
    if (nt == 0) continue;
    const int64_t pre = int64_t(kvh) * work + v.pair_pre[p];
    const int64_t e = pre + kUnitCost + nt;  // the unit's work is [pre, e)
    for (int64_t i = (pre * runs + total - 1) / total; i < runs && i * total / runs < e; ++i) {
      v.wg_kvh[i] = kvh;
      v.wg_p[i] = p;
    }
  }
}

// A workgroup's rows are the (token, query head) pairs of one KV head's group, row = token * group
// + head-in-group, 16 * C * W rows over W waves (C column tiles of 16 rows per wave). Every staged
// K/V tile is thus shared by all query heads of the group, and every K/V operand read from LDS feeds
// C MFMAs. Without a balanced schedule a workgroup is one unit (sequence, KV head, query block);
// with one, it walks the units of its run of key tiles.
//
// K/V tiles go from the pages straight into LDS (buffer loads with the LDS destination), two
// stages in distinct arrays so that the compiler's wait counting tells the stage being loaded from
// the stage being read. LDS rows are unpadded and swizzled (lds_swizzle) so that the MFMA operand
// reads are free of bank conflicts.
// P2: page_size is a power of two (page_shift >= 0); pages are then found with shifts (a runtime
// division costs ~20 scalar instructions, several per tile).
// SMALL: pages of 4 or 8 tokens (P2 as well). A 16-key sub-tile then spans 16 / page_size pages:
// each 1 KiB load (2 or 4 rows) lies in one page and gets that page's descriptor, and the keys
// present in a stage are a bit mask (an absent page can share a sub-tile with a present one).
template <int D, int C, int W, int NS, bool P2, bool SMALL, typename Tag>
__global__ __launch_bounds__(64 * W) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int kKT = 16 * NS;
  constexpr int KK = D / 32;
  constexpr int NT = D / 16;
  constexpr int CPR = D / 8;              // 16-byte chunks per row
  constexpr int RPB = 1024 / (2 * D);     // rows per 1 KiB load (64 lanes x 16 bytes)
  // Waves 0-3 load the tiles; the others only compute. A wave issuing its loads stalls until the
  // texture path takes them (~500-1000 cycles per tile when 8 waves issue together), and the
  // SIMDs favour older waves, so the youngest waves set the pace of the stage barriers: loads go
  // to the oldest waves, which wait at the barriers longest (per-wave s_memtime stamps; 4 waves
  // loading: -6 % for 8-wave units, -3 % for 12-wave ones, against 8 waves loading).
  constexpr int LW = 4;
  constexpr int LPW = kKT / RPB / LW;     // 1 KiB loads per loading wave per tile, each of K and V
  constexpr int ROWS = 16 * C * W;        // rows of the workgroup
  // Register-lean forms for shapes above 8 waves (3 waves per SIMD leave 168 VGPRs): V offsets
  // computed per read, K operands read through a ring, load offsets recomputed per tile. Each
  // costs the 8-wave shape 1-3 % (same-process A/B), which therefore keeps the plain forms.
  constexpr bool kLean = W > 8;
  // K/V loads into LDS as assembly (load_lds16) or through the compiler's builtin: the 8-wave
  // shape gains 3-6 % from the former, the 12-wave one loses ~3 % (same-process A/Bs).
  constexpr bool kAsmLoads = !kLean;
  static_assert(W >= LW && LPW * RPB * LW == kKT && 16 % (kKT / LW) == 0,
                "each wave's loads must lie inside one sub-tile");

  __shared__ __align__(1024) uint16_t sk0[kKT * D];
  __shared__ __align__(1024) uint16_t sv0[kKT * D];
  __shared__ __align__(1024) uint16_t sk1[kKT * D];
  __shared__ __align__(1024) uint16_t sv1[kKT * D];
  // Pages of 16 tokens or more: each stage's empty sub-tiles (bit j), written by the loading
  // wave 0 at the fetch and read by every wave after the next stage barrier, so that only the
  // loading waves read the block ids.
  __shared__ uint32_t s_empty[2];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const int G = a.group;

  // V^T operand addresses for the transposed reads, fixed for the whole kernel: lane (s, g)
  // (s = lane % 16) points at key row 16h + 4g + s/4 and columns d0 + 4(s%4) .. +3, so the read
  // gives output lane m the values V[16h + 4g + i][d0 + m], i = 0..3 -- the k-slots 8g + 4h + i
  // of the A operand (keys 4g + i of sub-tile h, matching P). voff[h][dt % 8] is the element
  // offset inside a stage of d-tile dt's piece; d-tiles dt and dt + 8 differ by 128 elements
  // (the swizzle only permutes chunks inside each group of 16).
  // Lean form: the swizzle XORs the 16-byte chunk index 2 dl + ((s % 4) / 2) with the even
  // 2r & 14, i.e. element offset 16 (dl ^ (r & 7)) + 8 ((s % 4) / 2), so voff[h][dl] =
  // vbase[h] + (16 dl ^ vxor[h]): one v_xad per read instead of 16 live offsets.
  int voff[2][kLean ? 1 : 8];
  int vbase[2], vxor[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int r = 16 * hh + 4 * g + (n >> 2);
    vbase[hh] = r * D + ((n & 3) >> 1) * 8 + (n & 1) * 4;
    vxor[hh] = 16 * (r & 7);
    if constexpr (!kLean) {
      const int sw = lds_swizzle_v(r);
#pragma unroll
      for (int dl = 0; dl < 8; ++dl) {
        const int y = 2 * dl + ((n & 3) >> 1);
        voff[hh][dl] = r * D + ((y ^ sw) * 8) + (n & 1) * 4;
      }
    }
  }
  const uint32_t row_bytes = uint32_t(a.row_stride) * 2u;
  // A page's bytes fit 32 bits (the host refuses larger pages), so a page's byte offset is one
  // 32 x 32-bit product and the offsets inside a page are 32-bit.
  const uint32_t page_bytes = uint32_t(a.page_stride) * 2u;
  // The sub-tile this wave loads (kKT / W rows per wave, inside one sub-tile).
  const int my_sub = (min(wave, LW - 1) * (kKT / LW)) / 16;

  // The current unit (uniform) and this lane's C rows of it; the key split of the unit. A unit's
  // rows are the sequence's (token, query head) rows [qr0, qr0 + ROWS) (row = token * G + head):
  // per-unit workgroups take ROWS consecutive rows whether or not they start a token; balanced
  // units are whole query blocks of tq tokens (qr0 = block * tq * G).
  int b = 0, kvh = 0, qr0 = 0, split = 0;
  SeqExtent sx;
  const int32_t* bt_row = a.block_table;
  int wave_last_key = 0, wave_first_key = 0;
  // Pages of 16 tokens or more: the last tile start whose tile needs no mask for the wave (every
  // key inside the context and at or below every row's diagonal), one value per unit.
  int full_k0 = 0;
  bool row_ok[C];
  int q_pos[C];
  u32x4 qop[C][KK];
  f32x4 o[C][NT];
  float m_run[C], l_run[C];

  auto page_of = [&](int key) __attribute__((always_inline)) {
    if constexpr (P2) return key >> a.page_shift;
    else return key / a.page_size;
  };
  // Block ids of the next tile to load (uniform), fetched one tile ahead of their use; -1 for a
  // sub-tile past the context. An id outside the cache is an absent page (masked, never loaded);
  // the fetch that uses the id checks that, so nothing waits for the id's load before then.
  // The ids are read with scalar loads: a vector load would be counted with the K/V loads into
  // LDS, and waiting for the ids would then wait for the whole tile in flight.
  int nbid[NS];
  // SMALL: the next tile's present keys (bit 16 j + i: key i of sub-tile j is inside the context
  // and its page valid) and the block ids of the pages of this wave's sub-tile (-1: absent).
  uint64_t nmask = 0;
  int nsid0 = -1, nsid1 = -1, nsid2 = -1, nsid3 = -1;  // scalars: an array would go to LDS
  auto load_ids = [&](int k0) __attribute__((always_inline)) {
    typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
    const const_i32_ptr row = (const_i32_ptr)bt_row;
    if constexpr (SMALL) {
      const int ps = a.page_size;
      uint64_t mask = 0;
#pragma unroll
      for (int j = 0; j < NS; ++j) {
#pragma unroll
        for (int pj = 0; pj < 4; ++pj) {
          const int key0 = k0 + 16 * j + pj * ps;
          if (pj * ps < 16) {  // uniform
            const int id = key0 < sx.kv_len ? row[key0 >> a.page_shift] : -1;
            const bool ok = uint32_t(id) < uint32_t(a.num_blocks32);
            if (ok) mask |= uint64_t((1u << ps) - 1u) << (16 * j + pj * ps);
            if (j == my_sub) {
              const int v = ok ? id : -1;
              if (pj == 0) nsid0 = v;
              else if (pj == 1) nsid1 = v;
              else if (pj == 2) nsid2 = v;
              else nsid3 = v;
            }
          }
        }
      }
      const int live = min(max(sx.kv_len - k0, 0), 16 * NS);  // keys inside the context
      nmask = live >= 64 ? mask : mask & ((uint64_t(1) << live) - 1);
      return;
    }
    if (wave >= LW) return;  // uniform: the other waves take the stage's mask from LDS
    // Keys are non-negative, so the page's byte offset in the row is a 32-bit unsigned value
    // (a scalar load with a register offset, no 64-bit address arithmetic).
    typedef const __attribute__((address_space(4))) char* const_c_ptr;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int key0 = k0 + 16 * j;
      const uint32_t pg = P2 ? uint32_t(key0) >> a.page_shift
                             : uint32_t(key0) / uint32_t(a.page_size);
      nbid[j] = key0 < sx.kv_len ? *(const_i32_ptr)((const_c_ptr)row + pg * 4u) : -1;
    }
  };
  // Keys of the sub-tile at key0 that exist (uniform).
  auto sub_rows = [&](int key0) __attribute__((always_inline)) {
    return min(max(sx.kv_len - key0, 0), 16);
  };
  // Sub-tiles of each stage with nothing loaded (bit j; uniform). Kept as two masks rather than
  // per-sub-tile row counts: the tile loop is short of scalar registers. SMALL: the stage's
  // present keys instead (bit 16 j + i).
  typedef std::conditional_t<SMALL, uint64_t, uint32_t> StageMask;
  StageMask empty_st[2];
  // The mask of stage st, valid after the stage barrier that follows its fetch.
  auto stage_mask = [&](int st) __attribute__((always_inline)) -> StageMask {
    if constexpr (SMALL) return empty_st[st];
    else return StageMask(__builtin_amdgcn_readfirstlane(int(s_empty[st])));
  };
  // Issue this wave's loads of the tile at key k0 into stage (sk, sv). A sub-tile lies in one
  // page; its loads use a buffer descriptor spanning only the rows that exist, so rows past the
  // context or in an absent page land in LDS as zero without a memory access.
  auto fetch = [&](uint16_t* sk, uint16_t* sv, int st, int k0)
      __attribute__((always_inline)) {
    if constexpr (SMALL) {
      empty_st[st] = nmask;
      if (wave >= LW) return;  // uniform: the other waves only need the mask
      const int ps = a.page_size;
      const int key_sub = k0 + 16 * my_sub;
      const int q = lane / CPR;
      const int slot = lane % CPR;
      int wblk = wave * LPW;
      asm volatile("" : "+s"(wblk));
      const int bw = (wblk * RPB) & 15;
      const uint32_t lane_hi = __umul24(uint32_t(bw | q), row_bytes);
      const uint32_t lane_k = uint32_t(slot ^ lds_swizzle(bw | q)) * 16u;
      const uint32_t lane_v = uint32_t(slot ^ lds_swizzle_v(bw | q)) * 16u;
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int blk = wblk + i;                  // 1 KiB block of the tile (uniform)
        const int rb = bw + RPB * i;               // its first row in the sub-tile
        const int pj = rb >> a.page_shift;         // its page in the sub-tile (ps >= RPB)
        const int id = pj == 0 ? nsid0 : pj == 1 ? nsid1 : pj == 2 ? nsid2 : nsid3;
        const int present = id < 0 ? 0 : min(max(sx.kv_len - (key_sub + pj * ps), 0), ps);
        const uint32_t nbytes = present > 0 ? uint32_t(present - 1) * row_bytes + D * 2 : 0u;
        const uint64_t off = uint64_t(uint32_t(id < 0 ? 0 : id)) * page_bytes +
                             uint32_t(kvh) * uint32_t(D * 2);
        // Offsets as the page-16 form computes them (relative to the sub-tile), moved to the
        // page's first row.
        const uint32_t ri = uint32_t(RPB * i) * row_bytes - uint32_t(pj * ps) * row_bytes;
        const uint32_t off_k = ((lane_k ^ uint32_t(16 * lds_swizzle(RPB * i))) + lane_hi) + ri;
        const uint32_t off_v = ((lane_v ^ uint32_t(16 * lds_swizzle_v(RPB * i))) + lane_hi) + ri;
        if constexpr (kAsmLoads) {
          load_lds16(rsrc_words(at_bytes(a.k_cache, off), nbytes), off_k, sk + blk * 512);
          load_lds16(rsrc_words(at_bytes(a.v_cache, off), nbytes), off_v, sv + blk * 512);
        } else {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(at_bytes(a.k_cache, off), nbytes),
                                                   (lds_ptr_t)(sk + blk * 512), 16, off_k, 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(at_bytes(a.v_cache, off), nbytes),
                                                   (lds_ptr_t)(sv + blk * 512), 16, off_v, 0, 0, 0);
        }
      }
      return;
    }
    if (wave >= LW) return;  // uniform: the other waves take the stage's mask from LDS
    // A sub-tile is empty past the context (id -1) or when its id is outside the cache.
    auto absent = [&](int id) __attribute__((always_inline)) {
      return uint32_t(id) >= uint32_t(a.num_blocks32);
    };
    int bid = nbid[0];
    uint32_t empty = absent(nbid[0]) ? 1u : 0u;
#pragma unroll
    for (int j = 1; j < NS; ++j) {
      if (my_sub == j) bid = nbid[j];
      empty |= (absent(nbid[j]) ? 1u : 0u) << j;
    }
    if (t == 0) s_empty[st] = empty;
    bid = __builtin_amdgcn_readfirstlane(bid);
    const int key0 = k0 + 16 * my_sub;
    const bool gone = absent(bid);
    const int rows = __builtin_amdgcn_readfirstlane(gone ? 0 : sub_rows(key0));
    bid = gone ? 0 : bid;
    const uint32_t in_page = P2 ? uint32_t(key0) & uint32_t(a.page_size - 1)
                                : uint32_t(key0 - page_of(key0) * a.page_size);
    const uint64_t off = uint64_t(uint32_t(bid)) * page_bytes +
                         (in_page * row_bytes + uint32_t(kvh) * uint32_t(D * 2));
    const uint32_t nbytes = rows > 0 ? uint32_t(rows - 1) * row_bytes + D * 2 : 0u;
    // Lean form: the per-lane offsets are recomputed at every fetch (an opaque copy of the lane
    // index keeps the compiler from hoisting 2 * LPW of them out of the loop, where they would
    // be spilled).
    int ln = lane;
    if constexpr (kLean) asm volatile("" : "+v"(ln));
    // The wave's first 1 KiB block of the tile, recomputed at every fetch (an opaque copy of the
    // wave index): hoisted out of the loop, the 2 * LPW LDS addresses would occupy scalar
    // registers for the whole loop and be spilled.
    int wblk = wave * LPW;
    asm volatile("" : "+s"(wblk));
    // Byte offsets of this lane's chunk of the wave's block i (1 KiB) of the tile in K and V. The
    // chunk's tile row has low four bits bw | RPB i | q (bw: those of the wave's first block, a
    // multiple of RPB LPW; q = ln / CPR; disjoint bit fields), and both swizzles are XOR-linear in
    // those bits, so each offset is a lane term, computed once per fetch, combined with a term of
    // i alone (an XOR-add and a scalar add per load, no 32-bit multiply).
    const int q = int(uint32_t(ln) / CPR);
    const int slot = int(uint32_t(ln) % CPR);
    const int bw = (wblk * RPB) & 15;
    const uint32_t lane_hi = __umul24(uint32_t(bw | q), row_bytes);
    const uint32_t lane_k = uint32_t(slot ^ lds_swizzle(bw | q)) * 16u;
    const uint32_t lane_v = uint32_t(slot ^ lds_swizzle_v(bw | q)) * 16u;
    auto chunk_offsets = [&](int i, uint32_t& off_k, uint32_t& off_v)
        __attribute__((always_inline)) {
      const uint32_t ri = uint32_t(RPB * i) * row_bytes;  // uniform
      off_k = ((lane_k ^ uint32_t(16 * lds_swizzle(RPB * i))) + lane_hi) + ri;
      off_v = ((lane_v ^ uint32_t(16 * lds_swizzle_v(RPB * i))) + lane_hi) + ri;
    };
    if constexpr (kAsmLoads) {
      const u32x4 rk = rsrc_words(at_bytes(a.k_cache, off), nbytes);
      const u32x4 rv = rsrc_words(at_bytes(a.v_cache, off), nbytes);
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int blk = wblk + i;                  // 1 KiB block of the tile (uniform)
        uint32_t off_k, off_v;
        chunk_offsets(i, off_k, off_v);
        load_lds16(rk, off_k, sk + blk * 512);
        load_lds16(rv, off_v, sv + blk * 512);
      }
    } else {
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(at_bytes(a.k_cache, off), nbytes);
      const __amdgpu_buffer_rsrc_t rv = make_rsrc(at_bytes(a.v_cache, off), nbytes);
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int blk = wblk + i;
        uint32_t off_k, off_v;
        chunk_offsets(i, off_k, off_v);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)(sk + blk * 512), 16, off_k, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)(sv + blk * 512), 16, off_v, 0, 0, 0);
      }
    }
  };

  // Q.K^T of the tile at k0 (stage sk), the online softmax, and P^T in MFMA operand form.
  auto qk_softmax = [&](const uint16_t* sk, StageMask empty, int k0, u32x4 (&pop)[C][NS / 2])
      __attribute__((always_inline)) {
    // S^T of each sub-tile that holds a key some row of the wave can see; the rest stay zero.
    f32x4 s[NS][C];
    int rows[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int c = 0; c < C; ++c) s[j][c] = f32x4{0.f, 0.f, 0.f, 0.f};
      rows[j] = 0;
      if (k0 + 16 * j <= wave_last_key) {  // uniform
        if constexpr (SMALL) {
          rows[j] = int((empty >> (16 * j)) & 0xffffu);  // present keys of the sub-tile
        } else {
          rows[j] = ((empty >> j) & 1u) ? 0 : sub_rows(k0 + 16 * j);
        }
        auto read_k = [&](int kk) __attribute__((always_inline)) {
          return *reinterpret_cast<const u32x4*>(sk + (16 * j + n) * D +
                                                (((4 * kk + g) ^ lds_swizzle(n)) * 8));
        };
        if constexpr (kLean) {
          // K reads two k-steps ahead of their MFMAs (a ring of three operands).
          u32x4 kop[3];
          kop[0] = read_k(0);
          kop[1] = read_k(1);
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
            __builtin_amdgcn_sched_barrier(0);
            if (kk + 2 < KK) kop[(kk + 2) % 3] = read_k(kk + 2);
#pragma unroll
            for (int c = 0; c < C; ++c) {
              s[j][c] = mfma16x16x32(kop[kk % 3], qop[c][kk], s[j][c], Tag{});
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        } else {
          u32x4 kop[KK];
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) kop[kk] = read_k(kk);
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
            for (int c = 0; c < C; ++c) s[j][c] = mfma16x16x32(kop[kk], qop[c][kk], s[j][c], Tag{});
          }
        }
      }
    }
    // A tile wholly below the wave's diagonal with every key present needs no mask (uniform).
    bool full;
    if constexpr (SMALL) {
      full = k0 + kKT - 1 <= wave_first_key;
#pragma unroll
      for (int j = 0; j < NS; ++j) full = full && rows[j] == 0xffff;
    } else {
      // Every rows[j] == 16: the whole tile inside the context and no sub-tile empty (below the
      // wave's first key every sub-tile is also at or below its last).
      full = k0 <= full_k0 && empty == 0;
    }
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
            const bool present = SMALL ? ((rows[j] >> i0) & 1) != 0 : i0 < rows[j];
            const bool ok = row_ok[c] & present & (k0 + 16 * j + i0 <= q_pos[c]);
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
  };

  // O += P.V of the tile at k0 (stage sv), with P^T from qk_softmax.
  auto pv = [&](const uint16_t* sv, int k0, const u32x4 (&pop)[C][NS / 2])
      __attribute__((always_inline)) {
    // O^T[16 d x 16 rows] += V^T[16 d x 32 keys] . P^T[32 keys x 16 rows] per pair of sub-tiles,
    // d-tile dt covering d = 16 dt .. 16 dt + 15; the A operand comes from two transposed reads.
    // The reads run two d-tiles ahead of the MFMAs; the scheduling barriers keep that order (left
    // to itself the scheduler may serialise each read with its MFMA when scalar registers run
    // short).
#pragma unroll
    for (int h = 0; h < NS / 2; ++h) {
      if (k0 + 32 * h > wave_last_key) continue;  // uniform: every P of the pair is zero
      const uint16_t* svh = sv + 32 * h * D;
      auto read_v = [&](int dt) __attribute__((always_inline)) {
        const int dh = dt >> 3, dl = dt & 7;
        int o0, o1;
        if constexpr (kLean) {
          o0 = vbase[0] + ((16 * dl) ^ vxor[0]);
          o1 = vbase[1] + ((16 * dl) ^ vxor[1]);
        } else {
          o0 = voff[0][dl];
          o1 = voff[1][dl];
        }
        const u32x2 lo = lds_read_tr4(svh + o0 + 128 * dh);
        const u32x2 hi = lds_read_tr4(svh + o1 + 128 * dh);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vop[3];
      vop[0] = read_v(0);
      vop[1] = read_v(1);
#pragma unroll
      for (int dt = 0; dt < NT; ++dt) {
        __builtin_amdgcn_sched_barrier(0);
        if (dt + 2 < NT) vop[(dt + 2) % 3] = read_v(dt + 2);
#pragma unroll
        for (int c = 0; c < C; ++c) {
          o[c][dt] = mfma16x16x32(vop[dt % 3], pop[c][h], o[c][dt], Tag{});
        }
      }
    }
  };

  auto compute = [&](const uint16_t* sk, const uint16_t* sv, StageMask empty, int k0)
      __attribute__((always_inline)) {
    u32x4 pop[C][NS / 2];
    qk_softmax(sk, empty, k0, pop);
    pv(sv, k0, pop);
  };

  // Attention of unit (b, kvh, qr0) over its key tiles [t0, t1): leaves the unnormalised o and
  // the per-lane m_run / l_run. Uniform over the workgroup.
  auto run_unit = [&](int t0, int t1) __attribute__((always_inline)) {
    sx = seq_extent(a, b);
    sx.q_start = __builtin_amdgcn_readfirstlane(sx.q_start);
    sx.q_len = __builtin_amdgcn_readfirstlane(sx.q_len);
    sx.kv_len = __builtin_amdgcn_readfirstlane(sx.kv_len);
    sx.offset = __builtin_amdgcn_readfirstlane(sx.offset);
    // Rows of the unit: ROWS (per-unit) or its query block's tokens (balanced), clipped to the
    // sequence's rows.
    const int ur = min(a.balanced_wgs > 0 ? a.tq * G : ROWS, sx.q_len * G - qr0);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int rho = wave * 16 * C + 16 * c + n;
      const int tok = (qr0 + rho) / G;  // token of the row within the sequence
      const int hh = qr0 + rho - tok * G;
      row_ok[c] = rho < ur;
      q_pos[c] = a.causal ? sx.offset + tok : INT32_MAX;
      const uint16_t* qrow = a.q + int64_t(sx.q_start + tok) * a.q_st +
                             int64_t(kvh * G + hh) * a.q_sh + 8 * g;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        qop[c][kk] = row_ok[c] ? load16(qrow + 32 * kk) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < NT; ++i) o[c][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      m_run[c] = -INFINITY;
      l_run[c] = 0.f;
    }
    // Under the causal mask, keys past wave_last_key are masked for every row of the wave and
    // keys up to wave_first_key are visible to all of them.
    const int wave_row = min(ur - 1, (wave + 1) * 16 * C - 1);
    wave_last_key = a.causal ? sx.offset + (qr0 + wave_row) / G : INT32_MAX;
    wave_first_key = a.causal ? sx.offset + (qr0 + wave * 16 * C) / G : INT32_MAX;
    full_k0 = min(wave_first_key - (kKT - 1), sx.kv_len - kKT);
    bt_row = a.block_table + int64_t(b) * a.bt_stride;
    const int cnt = t1 - t0;
    if (cnt > 0) load_ids(t0 * kKT);
    // Every wave is done reading both stages (previous unit). LDS only: the previous unit's
    // output stores may still be in flight; they drain under this unit's first loads.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Q lands here, before the tile loads are issued: the compiler does not see loads issued as
    // assembly, and its wait for Q at the first use, inside the tile loop, would also wait for
    // them.
    if constexpr (kAsmLoads) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+v"(qop[c][kk]));
      }
    }
    if (cnt > 0) {
      fetch(sk0, sv0, 0, t0 * kKT);
      if (cnt > 1) load_ids((t0 + 1) * kKT);
    }
    // Two tiles per trip so that each stage is a compile-time array. Each wave loads only part
    // of a stage, so before the barrier every wave must wait for its own K/V loads into LDS to
    // land (vmcnt): the compiler's __syncthreads does not count those loads as writes to order,
    // and its per-wave waits before the LDS reads cover only the reading wave's own part.
    for (int it = 0; it < cnt; it += 2) {
      const int k0 = (t0 + it) * kKT;
      // Stage 0 holds tile it; every wave is done with stage 1.
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (it + 1 < cnt) fetch(sk1, sv1, 1, k0 + kKT);
      if (k0 <= wave_last_key) compute(sk0, sv0, stage_mask(0), k0);
      // The ids of the tile after next, issued after this tile's LDS reads: the stage barrier's
      // wait covers them, and the fetch after it is their first use.
      if (it + 2 < cnt) load_ids(k0 + 2 * kKT);
      if (it + 1 >= cnt) break;
      // Stage 1 holds tile it + 1; every wave is done with stage 0.
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (it + 2 < cnt) fetch(sk0, sv0, 0, k0 + 2 * kKT);
      if (k0 + kKT <= wave_last_key) compute(sk1, sv1, stage_mask(1), k0 + kKT);
      if (it + 3 < cnt) load_ids(k0 + 3 * kKT);
    }
  };

  // The unit's normalised rows into `out`.
  auto store_final = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float l_tot = row_group_sum(l_run[c]);
      if (!row_ok[c]) continue;
      const int rho = wave * 16 * C + 16 * c + n;
      const int tok = (qr0 + rho) / G;
      const int hh = qr0 + rho - tok * G;
      if (a.uo) {  // uniform: unnormalised rows for a later merge (slot of the key split)
        const int64_t r = (int64_t(split) * a.total_q + sx.q_start + tok) * a.hq + kvh * G + hh;
#pragma unroll
        for (int dt = 0; dt < NT; ++dt) {
          *reinterpret_cast<f32x4*>(a.uo + r * D + 16 * dt + 4 * g) = o[c][dt];
        }
        if (g == 0) {
          a.uml[2 * r] = m_run[c];
          a.uml[2 * r + 1] = l_tot;
        }
        continue;
      }
      uint16_t* orow =
          a.out + int64_t(sx.q_start + tok) * a.o_st + int64_t(kvh * G + hh) * a.o_sh;
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      // Lane (n, g) holds d = 16 dt + 4g .. +3 of its row in o[c][dt].
      const uint16_t* grow = a.gate ? a.gate + int64_t(sx.q_start + tok) * a.gate_st +
                                          int64_t(kvh * G + hh) * a.gate_sh
                                    : nullptr;
#pragma unroll
      for (int dt = 0; dt < NT; ++dt) {
        u32x2 w;
        w[0] = pack2(o[c][dt][0] * inv, o[c][dt][1] * inv, Tag{});
        w[1] = pack2(o[c][dt][2] * inv, o[c][dt][3] * inv, Tag{});
        if (grow) {  // uniform
          const u32x2 gv = *reinterpret_cast<const u32x2*>(grow + 16 * dt + 4 * g);
          w[0] = gate_mul2(w[0], gv[0], Tag{});
          w[1] = gate_mul2(w[1], gv[1], Tag{});
        }
        *reinterpret_cast<u32x2*>(orow + 16 * dt + 4 * g) = w;
      }
    }
  };

  // The unit's unnormalised rows (o relative to 2^m, with m and the row's l) into partial slot
  // rows [row0, row0 + ROWS).
  auto store_partial = [&](int64_t row0) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float l_tot = row_group_sum(l_run[c]);
      if (!row_ok[c]) continue;
      const int64_t r = row0 + wave * 16 * C + 16 * c + n;
      float* prow = a.part_o + r * D + 4 * g;
#pragma unroll
      for (int dt = 0; dt < NT; ++dt) *reinterpret_cast<f32x4*>(prow + 16 * dt) = o[c][dt];
      if (g == 0) {
        a.part_ml[2 * r] = m_run[c];
        a.part_ml[2 * r + 1] = l_tot;
      }
    }
  };

  // Work of this workgroup: one unit, or (balanced) a run of key tiles over consecutive units.
  // One call site per lambda keeps every per-lane array in registers.
  const bool balanced = a.balanced_wgs > 0;
  // Balanced runs are dealt to the XCDs in contiguous blocks: workgroup ids go round-robin over
  // the 8 XCDs, so run i = (id % 8) * (G / 8) + id / 8 keeps consecutive runs (one KV head,
  // query blocks of one sequence, the same K/V pages) in one XCD's L2.
  const int nwg = a.balanced_wgs;
  const int i = (nwg % kXcds == 0) ? int(blockIdx.x % kXcds) * (nwg / kXcds) + int(blockIdx.x / kXcds)
                                   : int(blockIdx.x);
  const PlanView v = plan_view(a);
  int p = 0, n_pairs = 1, grid_nt = 0, unit_work = 1;
  int64_t pos = 0, end = 0;  // this workgroup's work positions (balanced)
  int grid_t0 = 0;  // per-unit schedule: the key tiles [grid_t0, grid_nt) of this workgroup
  if (!balanced) {
    // The heaviest query blocks (latest tokens, longest causal range) are dispatched first.
    kvh = blockIdx.x;
    b = blockIdx.z / a.key_splits;
    split = blockIdx.z - b * a.key_splits;
    qr0 = (gridDim.y - 1 - blockIdx.y) * ROWS;
    const SeqExtent s0 = seq_extent(a, b);
    if (qr0 >= s0.q_len * G) return;  // uniform over the workgroup
    grid_nt = (rows_key_end(a, s0, qr0, ROWS) + kKT - 1) / kKT;
    if (a.key_splits > 1) {
      const int per = (grid_nt + a.key_splits - 1) / a.key_splits;
      grid_t0 = min(split * per, grid_nt);
      grid_nt = min(grid_t0 + per, grid_nt);
    }
  } else {
    p = __builtin_amdgcn_readfirstlane(v.wg_p[i]);
    if (p < 0) return;  // no work left for this workgroup
    kvh = __builtin_amdgcn_readfirstlane(v.wg_kvh[i]);
    n_pairs = __builtin_amdgcn_readfirstlane(v.hdr[0]);
    unit_work = __builtin_amdgcn_readfirstlane(v.hdr[1]);
    const int64_t runs = __builtin_amdgcn_readfirstlane(v.hdr[2]);
    const int64_t total = __builtin_amdgcn_readfirstlane(v.hdr[3]);
    pos = int64_t(i) * total / runs;
    end = int64_t(i + 1) * total / runs;
  }
  // A run that starts inside a unit defers that first piece (the unit's tail) to its end: every
  // run then starts at key 0 of a unit, and the deferred tail begins about where the run's last
  // piece (the next unit's head, same cut) ended, so an XCD's workgroups sweep the keys together
  // and share pages in L2. Partial slot 0 stays the run's first piece, slot 1 its last.
  bool first = true, deferred = false, replay = false;
  int d_p = 0, d_kvh = 0;
  for (;;) {
    int nt = grid_nt, t0 = grid_t0, t1 = grid_nt;
    bool last = true;
    if (balanced) {
      nt = __builtin_amdgcn_readfirstlane(v.pair_nt[p]);
      b = __builtin_amdgcn_readfirstlane(v.pair_b[p]);
      qr0 = __builtin_amdgcn_readfirstlane(v.pair_qb[p]) * a.tq * G;
      // The unit's key tiles occupy work [k_pos, k_pos + nt); this run covers [pos, end).
      const int64_t k_pos = int64_t(kvh) * unit_work +
                            __builtin_amdgcn_readfirstlane(v.pair_pre[p]) + kUnitCost;
      t0 = int(max(pos - k_pos, int64_t(0)));
      t1 = int(min(end - k_pos, int64_t(nt)));
      last = k_pos + nt >= end;
    }
    const bool slot0 = first || replay;
    // Units without keys get their zero rows from the merge (balanced) or here (grid: nt = 0).
    bool go = t0 < t1 || !balanced;
    if (go && first && t0 > 0 && !last) {  // balanced only (grid units start at 0)
      d_p = p;
      d_kvh = kvh;
      deferred = true;
      first = false;
      go = false;
    }
    if (go) {
      run_unit(t0, t1);
      // Per-unit workgroups store their rows (a key split's unnormalised part, into its slot).
      if (!balanced || (t0 == 0 && t1 == nt)) store_final();
      else store_partial((int64_t(i) * 2 + (slot0 ? 0 : 1)) * ROWS);
      first = false;
    }
    bool done = last || replay;
    if (!done && ++p == n_pairs) {
      p = 0;
      done = ++kvh == a.hkv;
    }
    if (done) {
      if (!deferred || replay) break;
      p = d_p;
      kvh = d_kvh;
      replay = true;
    }
  }
}

// Combines the partials of every unit that was cut between workgroups, in workgroup order, and
// writes the zero rows of units with no visible key: per row m = max m_s, w_s = 2^(m_s - m),
// out = sum w_s o_s / sum w_s l_s. One workgroup per (pair, KV head, block of kMergeRows rows);
// each thread takes 8 values of kMergeRowsPerThread rows, loads first, so that their latencies
// overlap.
constexpr int kMergeRowsPerThread = 1;

template <int D, int ROWS, typename Tag>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  constexpr int TPR = D / 8;                          // threads per row, 8 values each
  constexpr int RPT = kMergeRowsPerThread;
  constexpr int RPW = 256 / TPR * RPT;                // rows per workgroup
  const PlanView v = plan_view(a);
  const int p = blockIdx.x;
  const int kvh = blockIdx.y;
  const int n_pairs = v.hdr[0];
  if (p >= n_pairs) return;
  const int unit_work = v.hdr[1];
  const int64_t runs = v.hdr[2];
  const int64_t total = v.hdr[3];
  // The run holding work position x: the last i with floor(i * total / runs) <= x.
  auto run_of = [&](int64_t x) { return ((x + 1) * runs - 1) / total; };
  const int b = v.pair_b[p];
  const int qb0 = v.pair_qb[p] * a.tq;
  const int nt = v.pair_nt[p];
  int64_t i0 = 0;
  int nparts = 0, first_slot = 0;
  if (nt > 0) {
    const int64_t pre = int64_t(kvh) * unit_work + v.pair_pre[p];
    const int64_t k_pos = pre + kUnitCost;  // work position of the unit's first key tile
    i0 = run_of(k_pos);
    const int64_t i1 = run_of(k_pos + nt - 1);
    if (i0 == i1) return;  // one workgroup finished the unit
    nparts = int(i1 - i0 + 1);
    // The first part is slot 1 of a workgroup that started in an earlier unit.
    first_slot = i0 * total / runs < pre ? 1 : 0;
  }
  const SeqExtent sx = seq_extent(a, b);
  const int rows = min(a.tq, sx.q_len - qb0) * a.group;
  const int d0 = (threadIdx.x % TPR) * 8;
  const int r0 = int(blockIdx.z) * RPW + int(threadIdx.x) / TPR;  // rows r0 + j * (256 / TPR)
  if (r0 >= rows) return;
  auto part_row = [&](int s, int j) -> int64_t {
    return ((i0 + s) * 2 + (s == 0 ? first_slot : 0)) * ROWS + r0 + j * (256 / TPR);
  };
  float m[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) m[j] = -INFINITY;
  for (int s = 0; s < nparts; ++s) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) m[j] = fmaxf(m[j], a.part_ml[2 * part_row(s, j)]);
  }
  f32x4 acc[RPT][2];
  float l[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    acc[j][0] = acc[j][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    l[j] = 0.f;
  }
  for (int s = 0; s < nparts; ++s) {
    float ms[RPT], ls[RPT];
    f32x4 x[RPT][2];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int64_t pr = part_row(s, j);
      ms[j] = a.part_ml[2 * pr];
      ls[j] = a.part_ml[2 * pr + 1];
      const f32x4* src = reinterpret_cast<const f32x4*>(a.part_o + pr * D + d0);
      x[j][0] = src[0];
      x[j][1] = src[1];
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const float w = ms[j] == -INFINITY ? 0.f : fast_exp2(ms[j] - m[j]);
      l[j] += w * ls[j];
      acc[j][0] += w * x[j][0];
      acc[j][1] += w * x[j][1];
    }
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = r0 + j * (256 / TPR);
    if (r >= rows) break;
    const int tok = r / a.group;
    const int hh = r - tok * a.group;
    if (a.uo) {  // unnormalised rows for a later merge
      const int64_t ur = int64_t(sx.q_start + qb0 + tok) * a.hq + kvh * a.group + hh;
      f32x4* dst = reinterpret_cast<f32x4*>(a.uo + ur * D + d0);
      dst[0] = acc[j][0];
      dst[1] = acc[j][1];
      if (d0 == 0) {
        a.uml[2 * ur] = m[j];
        a.uml[2 * ur + 1] = l[j];
      }
      continue;
    }
    const float inv = l[j] > 0.f ? 1.f / l[j] : 0.f;
    uint16_t* orow = a.out + int64_t(sx.q_start + qb0 + tok) * a.o_st +
                     int64_t(kvh * a.group + hh) * a.o_sh + d0;
    u32x4 w;
    w[0] = pack2(acc[j][0][0] * inv, acc[j][0][1] * inv, Tag{});
    w[1] = pack2(acc[j][0][2] * inv, acc[j][0][3] * inv, Tag{});
    w[2] = pack2(acc[j][1][0] * inv, acc[j][1][1] * inv, Tag{});
    w[3] = pack2(acc[j][1][2] * inv, acc[j][1][3] * inv, Tag{});
    if (a.gate) {
      const u32x4 gv = *reinterpret_cast<const u32x4*>(
          a.gate + int64_t(sx.q_start + qb0 + tok) * a.gate_st +
          int64_t(kvh * a.group + hh) * a.gate_sh + d0);
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = gate_mul2(w[e], gv[e], Tag{});
    }
    *reinterpret_cast<u32x4*>(orow) = w;
  }
}

// Launch shape per head_dim and schedule: C column tiles per wave, W waves (16 C W rows), NS
// 16-key sub-tiles per staged tile (each inside one page). head_dim 256, measured in same-process
// A/Bs on MI355X (config 4, 6 query heads per KV head):
// - one workgroup per unit: 8 waves, 64-key tiles. Units of 128 rows keep a causal first chunk's
//   longest unit short (82 us for the 2048-token chunk; 12 waves x 192 rows: 106-115 us).
// - balanced: 12 waves (3 per SIMD, 168 VGPRs), 32-key tiles. 192 rows share each K/V tile, 1.5x
//   the rows of 8 waves, and the 32-key tile leaves the registers the third wave needs (64-key
//   tiles spill 22 VGPRs): continuation chunk 405 us against 444 us for 8 waves.
template <int D, bool BAL> struct PrefillShape;
template <> struct PrefillShape<256, false> { static constexpr int C = 1, W = 8, NS = 4; };
template <> struct PrefillShape<256, true> { static constexpr int C = 1, W = 12, NS = 2; };
template <bool BAL> struct PrefillShape<128, BAL> { static constexpr int C = 2, W = 8, NS = 4; };

int prefill_rows(int head_dim, bool balanced) {
  return head_dim == 256 ? (balanced ? 16 * 1 * 12 : 16 * 1 * 8) : 16 * 2 * 8;
}
int prefill_key_tile(int head_dim, bool balanced) {
  return head_dim == 256 && balanced ? 16 * 2 : 16 * 4;
}

template <int D, bool BAL, bool P2, typename Tag, bool SMALL = false>
constexpr auto prefill_kernel() {
  using S = PrefillShape<D, BAL>;
  return prefill_mfma_kernel<D, S::C, S::W, S::NS, P2, SMALL, Tag>;
}

// Workgroups of one balanced launch: every CU's resident workgroups (one round).
template <int D, typename Tag>
int balanced_wgs() {
  static std::atomic<int> cached{0};  // same code object on every gfx950 device
  int per_cu = cached.load(std::memory_order_relaxed);
  if (per_cu == 0) {
    const auto fn = prefill_kernel<D, true, true, Tag>();
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn),
                                                     64 * PrefillShape<D, true>::W, 0) !=
            hipSuccess ||
        per_cu <= 0) {
      (void)hipGetLastError();
      per_cu = 1;
    }
    cached.store(per_cu, std::memory_order_relaxed);
  }
  return device_cu_count() * per_cu;
}

// Upper bound of balanced_wgs (LDS bounds the resident workgroups per CU).
int balanced_wgs_bound(int head_dim) {
  const int lds = 4 * prefill_key_tile(head_dim, true) * head_dim * 2;
  return device_cu_count() * (160 * 1024 / lds);
}

template <int D, bool BAL, typename Tag>
int launch_prefill(const PrefillArgs& a, int batch, int max_q, hipStream_t s) {
  using S = PrefillShape<D, BAL>;
  const auto kern = a.page_size < 16   ? prefill_kernel<D, BAL, true, Tag, true>()
                    : a.page_shift >= 0 ? prefill_kernel<D, BAL, true, Tag>()
                                        : prefill_kernel<D, BAL, false, Tag>();
  if constexpr (!BAL) {
    const dim3 grid(unsigned(a.hkv), unsigned(ceil_div(int64_t(max_q) * a.group, S::C * S::W * 16)),
                    unsigned(batch * a.key_splits));
    hipLaunchKernelGGL(kern, grid, dim3(64 * S::W), 0, s, a);
    return check_launch("ti_gqa_prefill_paged");
  } else {
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, a, batch);
    int rc = check_launch("ti_gqa_prefill_paged (plan)");
    if (rc != TI_OK) return rc;
    hipLaunchKernelGGL(kern, dim3(unsigned(a.balanced_wgs)), dim3(64 * S::W), 0, s, a);
    rc = check_launch("ti_gqa_prefill_paged");
    if (rc != TI_OK) return rc;
    constexpr int kRows = 16 * S::C * S::W;
    constexpr int kMergeRows = 256 / (D / 8) * kMergeRowsPerThread;  // rows per merge workgroup
    static_assert(kRows % kMergeRows == 0, "merge row blocks must tile the unit");
    hipLaunchKernelGGL((prefill_merge_kernel<D, kRows, Tag>),
                       dim3(unsigned(a.max_pairs), unsigned(a.hkv), unsigned(kRows / kMergeRows)),
                       dim3(256), 0, s, a);
    return check_launch("ti_gqa_prefill_paged (merge)");
  }
}

// Balanced-schedule sizes of one call; false when the call runs one workgroup per unit (too many
// sequences for the schedule's tables, or tile counts beyond int32).
bool balanced_sizes(int32_t batch, int32_t total_q, int32_t hq, int32_t hkv, int32_t head_dim,
                    int32_t page_size, int32_t max_blocks, int64_t wgs, int64_t* max_pairs,
                    int64_t* bytes) {
  if (batch <= 0 || batch > kMaxPlanSeqs || hkv <= 0 || hq % hkv != 0) return false;
  const int64_t tq = prefill_rows(head_dim, true) / (hq / hkv);
  if (tq <= 0) return false;
  const int64_t pairs = ceil_div(total_q, tq) + batch;
  const int64_t kt = prefill_key_tile(head_dim, true);
  const int64_t tiles_bound =
      pairs * (ceil_div(int64_t(max_blocks) * page_size, kt) + kUnitCost) * hkv;
  if (pairs > INT32_MAX / 8 || tiles_bound > INT32_MAX / 2 || hkv * pairs > INT32_MAX / 2) {
    return false;
  }
  const int64_t ints = (plan_ints(pairs, wgs) + 63) / 64 * 64;  // 256-byte aligned floats after
  const int64_t rows = int64_t(wgs) * 2 * prefill_rows(head_dim, true);
  *max_pairs = pairs;
  *bytes = ints * 4 + rows * (head_dim + 2) * 4;
  return true;
}

}  // namespace
}  // namespace ti

extern "C" int ti_gqa_prefill_workspace_bytes(int32_t batch, int32_t total_q, int32_t num_q_heads,
                                              int32_t num_kv_heads, int32_t head_dim,
                                              int32_t page_size, int32_t max_blocks_per_seq,
                                              int64_t* bytes_out) {
  using namespace ti;
  if (!bytes_out) return fail(TI_EINVAL, "ti_gqa_prefill_workspace_bytes: null output pointer");
  if (head_dim != 128 && head_dim != 256) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_workspace_bytes: head_dim %d not built",
                head_dim);
  }
  int64_t pairs = 0, bytes = 0;
  if (total_q <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || page_size <= 0 ||
      max_blocks_per_seq < 0 ||
      !balanced_sizes(batch, total_q, num_q_heads, num_kv_heads, head_dim, page_size,
                      max_blocks_per_seq, balanced_wgs_bound(head_dim), &pairs, &bytes)) {
    bytes = 0;
  }
  *bytes_out = bytes;
  return TI_OK;
}

namespace ti {
namespace {

// Both entry points: gate == nullptr for the plain output.
int prefill_paged(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                  const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
                  const int32_t* cu_seqlens_q, const int32_t* seqlen_k, void* out,
                  int64_t out_stride_t, int64_t out_stride_h, void* workspace,
                  int64_t workspace_bytes, int32_t batch, int32_t total_q, int32_t max_seqlen_q,
                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                  int64_t num_blocks, int32_t max_blocks_per_seq, int32_t causal, int32_t dtype,
                  void* stream, const void* gate, int64_t gate_stride_t, int64_t gate_stride_h,
                  float* uo = nullptr, float* uml = nullptr, int32_t key_splits = 1) {
  if (dtype != TI_DTYPE_BF16 && dtype != TI_DTYPE_F16) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: dtype code %d is not bf16/fp16", dtype);
  }
  if (batch < 0 || total_q < 0 || max_seqlen_q < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads != 0 || max_blocks_per_seq < 0 || num_blocks < 0 ||
      workspace_bytes < 0) {
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
  if (page_size <= 0 || (page_size % 16 != 0 && page_size != 8 && page_size != 4)) {
    return fail(TI_EUNSUPPORTED,
                "ti_gqa_prefill_paged: page_size %d is neither 4, 8 nor a multiple of 16",
                page_size);
  }
  if (int64_t(num_kv_heads) * head_dim * page_size * 2 > int64_t(UINT32_MAX)) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: a page of %d tokens x %d KV heads "
                "exceeds 4 GiB", page_size, num_kv_heads);
  }
  if (key_splits < 1 || (key_splits > 1 && (workspace != nullptr || uo == nullptr)) ||
      int64_t(batch) * key_splits > 65535) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged_partial: key_splits %d needs the unnormalised "
                           "output, no workspace and batch * key_splits <= 65535", key_splits);
  }
  if (batch == 0 || total_q == 0 || max_seqlen_q == 0) return TI_OK;
  if (!q || !k_cache || !v_cache || !block_table || !cu_seqlens_q || !seqlen_k ||
      (!out && !(uo && uml))) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged: null pointer");
  }
  if (block_table_stride < max_blocks_per_seq || q_stride_h % 8 || q_stride_t % 8 ||
      out_stride_h % 8 || out_stride_t % 8 || (reinterpret_cast<uintptr_t>(q) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & 15) || (reinterpret_cast<uintptr_t>(k_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(v_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255)) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged: rows must be 16-byte aligned (workspace 256)");
  }
  if ((reinterpret_cast<uintptr_t>(uo) & 15) || (reinterpret_cast<uintptr_t>(uml) & 7)) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged_partial: o 16-byte, (m, l) 8-byte aligned");
  }
  if (gate && ((reinterpret_cast<uintptr_t>(gate) & 15) || gate_stride_t % 8 || gate_stride_h % 8)) {
    return fail(TI_EINVAL, "ti_gqa_prefill_paged_gated: gate rows must be 16-byte aligned");
  }
  const bool bf16 = dtype == TI_DTYPE_BF16;
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
  a.page_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctz(unsigned(page_size)) : -1;
  a.max_blocks = max_blocks_per_seq;
  a.causal = causal ? 1 : 0;
  const bool balanced = workspace != nullptr && workspace_bytes > 0;
  if (!balanced &&
      ceil_div(int64_t(max_seqlen_q) * a.group, prefill_rows(head_dim, false)) > 65535) {
    return fail(TI_EUNSUPPORTED, "ti_gqa_prefill_paged: %d query tokens per sequence exceed the "
                "per-unit grid (65,535 row blocks); pass a workspace", max_seqlen_q);
  }
  a.tq = prefill_rows(head_dim, balanced) / a.group;
  a.key_tile = prefill_key_tile(head_dim, balanced);
  a.scale_log2 = float(1.4426950408889634 / sqrt(double(head_dim)));
  a.balanced_wgs = 0;
  a.max_pairs = 0;
  a.min_chunk = kMinChunkTiles;
  a.plan = nullptr;
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.gate = static_cast<const uint16_t*>(gate);
  a.gate_st = gate_stride_t;
  a.gate_sh = gate_stride_h;
  a.uo = uo;
  a.uml = uml;
  a.key_splits = key_splits;
  if (balanced) {
    const int wgs = head_dim == 256 ? (bf16 ? balanced_wgs<256, Bf16>() : balanced_wgs<256, F16>())
                                    : (bf16 ? balanced_wgs<128, Bf16>() : balanced_wgs<128, F16>());
    int64_t pairs = 0, need = 0;
    if (!balanced_sizes(batch, total_q, num_q_heads, num_kv_heads, head_dim, page_size,
                        max_blocks_per_seq, wgs, &pairs, &need)) {
      return fail(TI_EINVAL, "ti_gqa_prefill_paged: no balanced schedule for this call (batch %d); "
                             "pass no workspace", batch);
    }
    if (workspace_bytes < need) {
      return fail(TI_EINVAL, "ti_gqa_prefill_paged: workspace of %lld bytes needed, %lld given",
                  (long long)need, (long long)workspace_bytes);
    }
    a.balanced_wgs = wgs;
    a.max_pairs = int32_t(pairs);
    a.plan = static_cast<int32_t*>(workspace);
    const int64_t ints = (plan_ints(pairs, wgs) + 63) / 64 * 64;
    a.part_o = reinterpret_cast<float*>(a.plan + ints);
    a.part_ml = a.part_o + int64_t(wgs) * 2 * prefill_rows(head_dim, true) * head_dim;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (head_dim == 256) {
    if (balanced) {
      return bf16 ? launch_prefill<256, true, Bf16>(a, batch, max_seqlen_q, s)
                  : launch_prefill<256, true, F16>(a, batch, max_seqlen_q, s);
    }
    return bf16 ? launch_prefill<256, false, Bf16>(a, batch, max_seqlen_q, s)
                : launch_prefill<256, false, F16>(a, batch, max_seqlen_q, s);
  }
  if (balanced) {
    return bf16 ? launch_prefill<128, true, Bf16>(a, batch, max_seqlen_q, s)
                : launch_prefill<128, true, F16>(a, batch, max_seqlen_q, s);
  }
  return bf16 ? launch_prefill<128, false, Bf16>(a, batch, max_seqlen_q, s)
              : launch_prefill<128, false, F16>(a, batch, max_seqlen_q, s);
}

}  // namespace
}  // namespace ti

extern "C" int ti_gqa_prefill_paged(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                    const void* k_cache, const void* v_cache,
                                    const int32_t* block_table, int64_t block_table_stride,
                                    const int32_t* cu_seqlens_q, const int32_t* seqlen_k,
                                    void* out, int64_t out_stride_t, int64_t out_stride_h,
                                    void* workspace, int64_t workspace_bytes, int32_t batch,
                                    int32_t total_q, int32_t max_seqlen_q, int32_t num_q_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                    int64_t num_blocks, int32_t max_blocks_per_seq, int32_t causal,
                                    int32_t dtype, void* stream) {
  return ti::prefill_paged(q, q_stride_t, q_stride_h, k_cache, v_cache, block_table,
                           block_table_stride, cu_seqlens_q, seqlen_k, out, out_stride_t,
                           out_stride_h, workspace, workspace_bytes, batch, total_q, max_seqlen_q,
                           num_q_heads, num_kv_heads, head_dim, page_size, num_blocks,
                           max_blocks_per_seq, causal, dtype, stream, nullptr, 0, 0);
}

extern "C" int ti_gqa_prefill_paged_gated(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
    const int32_t* cu_seqlens_q, const int32_t* seqlen_k, void* out, int64_t out_stride_t,
    int64_t out_stride_h, void* workspace, int64_t workspace_bytes, int32_t batch, int32_t total_q,
    int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, int64_t num_blocks, int32_t max_blocks_per_seq, int32_t causal,
    int32_t dtype, const void* gate, int64_t gate_stride_t, int64_t gate_stride_h, void* stream) {
  if (!gate) return ti::fail(TI_EINVAL, "ti_gqa_prefill_paged_gated: null gate");
  return ti::prefill_paged(q, q_stride_t, q_stride_h, k_cache, v_cache, block_table,
                           block_table_stride, cu_seqlens_q, seqlen_k, out, out_stride_t,
                           out_stride_h, workspace, workspace_bytes, batch, total_q, max_seqlen_q,
                           num_q_heads, num_kv_heads, head_dim, page_size, num_blocks,
                           max_blocks_per_seq, causal, dtype, stream, gate, gate_stride_t,
                           gate_stride_h);
}

extern "C" int ti_gqa_prefill_paged_partial(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
    const int32_t* cu_seqlens_q, const int32_t* seqlen_k, float* o_part, float* ml_part,
    void* workspace, int64_t workspace_bytes, int32_t batch, int32_t total_q,
    int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t page_size, int64_t num_blocks, int32_t max_blocks_per_seq, int32_t causal,
    int32_t dtype, int32_t key_splits, void* stream) {
  if (!o_part || !ml_part) {
    return ti::fail(TI_EINVAL, "ti_gqa_prefill_paged_partial: null output pointer");
  }
  return ti::prefill_paged(q, q_stride_t, q_stride_h, k_cache, v_cache, block_table,
                           block_table_stride, cu_seqlens_q, seqlen_k, nullptr, 0, 0, workspace,
                           workspace_bytes, batch, total_q, max_seqlen_q, num_q_heads,
                           num_kv_heads, head_dim, page_size, num_blocks, max_blocks_per_seq,
                           causal, dtype, stream, nullptr, 0, 0, o_part, ml_part, key_splits);
}

// Key splits of a one-sequence partial pass of `total_q` queries over `kv_tokens` keys (the shared
// prefix of a decode batch): enough (query block, KV head, key range) workgroups to give every CU
// one, each range at least kMinSplitTiles key tiles.
extern "C" int32_t ti_gqa_prefill_key_splits(int32_t total_q, int32_t num_q_heads,
                                             int32_t num_kv_heads, int32_t head_dim,
                                             int32_t kv_tokens) {
  using namespace ti;
  constexpr int kMinSplitTiles = 4;
  if (total_q <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0 || kv_tokens <= 0 ||
      (head_dim != 128 && head_dim != 256)) {
    return 1;
  }
  const int64_t units = int64_t(num_kv_heads) *
                        ceil_div(int64_t(total_q) * (num_q_heads / num_kv_heads),
                                 prefill_rows(head_dim, false));
  const int64_t tiles = ceil_div(kv_tokens, prefill_key_tile(head_dim, false));
  int64_t s = device_cu_count() / units;
  s = s < ceil_div(tiles, kMinSplitTiles) ? s : ceil_div(tiles, kMinSplitTiles);
  s = s < 65535 ? s : 65535;
  return int32_t(s > 1 ? s : 1);
}
