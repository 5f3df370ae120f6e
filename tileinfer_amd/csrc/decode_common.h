// Definitions shared by the paged decode kernels (MFMA and scalar variants).
#pragma once

#include <math.h>

#include "ti_common.h"

namespace ti {

constexpr int kMaxSplitPages = 1024;  // block ids of one partition staged in LDS
// The MFMA kernel's balanced runs over pages smaller than its 16-token tile stage up to this
// many block ids (8,192 tokens at page 2, 16,384 at page 4: one round of runs at config 3).
constexpr int kMaxRunPagesSmall = 4096;
constexpr int kMaxSplitTokens = 16384;

struct Bf16 {};
struct F16 {};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c, Bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c, F16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// Two floats -> two 16-bit values (round to nearest even), x in the low half.
__device__ __forceinline__ uint32_t pack2(float x, float y, Bf16) {
  bf16x2_t v = {static_cast<__bf16>(x), static_cast<__bf16>(y)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t pack2(float x, float y, F16) {
  f16x2_t v = {static_cast<_Float16>(x), static_cast<_Float16>(y)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two 16-bit values -> floats (exact), x in the low half.
__device__ __forceinline__ float2 unpack2(uint32_t v, Bf16) {
  return make_float2(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
}
__device__ __forceinline__ float2 unpack2(uint32_t v, F16) {
  const f16x2_t h = __builtin_bit_cast(f16x2_t, v);
  return make_float2(float(h[0]), float(h[1]));
}

// Logistic function 1 / (1 + e^-x) through the HIP device library's expf.
__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }

// a * sigmoid(g) for two packed 16-bit pairs, rounded back to the storage type: the output
// epilogue of the sigmoid gate (out = attention output * sigmoid(gate)).
template <typename Tag>
__device__ __forceinline__ uint32_t gate_mul2(uint32_t a, uint32_t g, Tag tag) {
  const float2 x = unpack2(a, tag);
  const float2 y = unpack2(g, tag);
  return pack2(x.x * sigmoidf(y.x), x.y * sigmoidf(y.y), tag);
}

__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Raw buffer descriptor over [base, base + bytes): loads at or past `bytes` return zero without
// touching memory. Word 3 is the gfx9-family raw 32-bit data format.
constexpr int kBufferRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, int(bytes),
                                           kBufferRsrcWord3);
}

// Cache policies of the K/V loads. kPolicyStream (the `nt` bit) is for pages read once per call:
// on MI355X a read stream issued that way sustains ~7.0 TB/s against ~6.3 TB/s with the default
// policy. kPolicyKeep (default policy) is for calls whose block tables share pages across
// sequences (prefix caching): the shared pages are then served from L2/MALL, which `nt` defeats
// (config 5: 450 us with kPolicyKeep against 770 us with kPolicyStream).
constexpr int kPolicyKeep = 0;
constexpr int kPolicyStream = 2;
// Chosen per sequence on the device (decode_mfma_kernel): kPolicyKeep when another sequence of the
// batch starts with the same block (prefix caching shares whole-block chains from a table's first
// column, so that finds every sequence whose pages other sequences also read), else kPolicyStream.
constexpr int kPolicyAuto = -1;

template <int POL>
__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
  return __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(rsrc, int(offset), 0, POL));
}

template <int POL>
__device__ __forceinline__ u32x4 load16_policy(const uint16_t* p) {
  if constexpr (POL == kPolicyStream) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  } else {
    return load16(p);
  }
}

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;  // q strides (elements)
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int64_t page_stride;  // elements per physical block: page_size * hkv * D
  int64_t row_stride;   // elements per token row: hkv * D
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* seqlen;
  uint16_t* out;   // [B, hq, D]
  float* part_o;   // [B, hq, max_splits, D]
  float* part_ml;  // [B, hq, max_splits, 2]  (running max in log2 units, sum of exp2)
  // Balanced mode: [B + 1] ints after the partials; entry b is sequence b's first tile in the
  // batch's concatenated tile order (written by the workgroup that holds that tile, for sequences
  // with tiles), entry B the batch's total tiles (written by workgroup 0). The merge reads them
  // instead of scanning every sequence length per row.
  int32_t* seq_first_tile;
  int32_t num_blocks32;  // block ids in [0, num_blocks32) are valid (int32 ids)
  int32_t hq, hkv, group, page_size, max_blocks, max_splits, split_tokens;
  int32_t page_log2;  // log2(page_size) when it is a power of two (the small-page path)
  // 1: one workgroup per (KV head, sequence) whose waves split the sequence's tiles and combine
  // their parts in LDS (no partials, no merge); 0 otherwise.
  int32_t wave_split;
  float scale_log2;
  // Balanced mode (> 0): this many workgroups share the batch's 16-token tiles evenly (every
  // workgroup takes a contiguous run of the concatenated tiles of all sequences); partials are
  // indexed [workgroup][first|last segment][q-head]. 0: one workgroup per (sequence, partition of
  // split_tokens), partials indexed [sequence][q-head][partition].
  int32_t balanced_wgs;
  int32_t chunk_min_tiles;  // lower bound on a balanced workgroup's run
  // Optional sigmoid gate of the output (out = attention * sigmoid(gate)), [B, hq, D] at these
  // strides; nullptr for the plain output.
  const uint16_t* gate;
  int64_t gate_sb, gate_sh;
  // Optional attention parts computed elsewhere (a prefix shared by the batch): pre_parts
  // unnormalised fp32 parts, o relative to 2^m [pre_parts][B][hq][D] and (m, l)
  // [pre_parts][B][hq][2], m in exp2 units, merged into every row in part order; the kernel itself
  // then covers tokens [ctx_offset, seqlen[b]) through the block table it gets (whose column 0 is
  // token ctx_offset's page). nullptr / 0 for plain decode.
  const float* pre_o;
  const float* pre_ml;
  int32_t pre_parts;
  int32_t ctx_offset;
  // Balanced calls with prefix parts (whole_rows = 1): a sequence one workgroup covers whole
  // stores its unnormalised row as part row whole_row0 + b * hq + h (after the workgroups' part
  // rows), and the merge folds the prefix parts into it.
  int32_t whole_rows;
  int64_t whole_row0;
  // Optional fused append (one new token per sequence, its K/V rows not yet in the cache): row b
  // of app_k / app_v ([B][hkv * D] at row strides app_k_sb / app_v_sb elements) is written to
  // cache row app_slot[b] (skipped when negative or >= app_num_slots) before it is read, by the
  // workgroup whose tiles end at the sequence's last token (the merge for sequences with none).
  // The caller guarantees that app_slot[b] is the slot of position seqlen[b] - 1. nullptr: none.
  const uint16_t* app_k;
  const uint16_t* app_v;
  int64_t app_k_sb, app_v_sb;
  const int32_t* app_slot;
  int64_t app_num_slots;
};


// Clamped context length of sequence b and its number of partitions.
__device__ __forceinline__ int seq_len(const DecodeArgs& a, int b) {
  int ctx = a.seqlen[b] - a.ctx_offset;
  const int cap = a.max_blocks * a.page_size;
  ctx = ctx < 0 ? 0 : (ctx > cap ? cap : ctx);
  return ctx;
}

// Tiles (16 tokens) of sequence b.
__device__ __forceinline__ int seq_tiles(const DecodeArgs& a, int b) { return (seq_len(a, b) + 15) >> 4; }


// Launches the LDS-staged scalar variant of the partial kernel (gqa_decode_scalar.hip).
int launch_decode_scalar(const DecodeArgs& a, int batch, bool bf16, int head_dim, bool reuse_kv,
                         hipStream_t stream);

}  // namespace ti
