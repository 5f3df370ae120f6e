/*
 * tileinfer_amd.h — C ABI of the MI355X (gfx950) paged KV-cache library.
 *
 * The library implements tileInfer's paged KV-cache hot path as hand-written HIP kernels:
 *   - the slot-mapped K/V append           (replaces kernels/kvcache_store.py:43-71, store_kvcache)
 *   - single-query paged GQA decode        (replaces kernels/gqa_decode_paged.py:392-437,
 *     attention with a split-K merge         gqa_decode_paged_fn)
 *   - block copies between caches           (swap out/in and copy-on-write; no reference kernel)
 *   - paged causal GQA prefill attention    (replaces the gather + varlen flash attention of
 *                                            model/qwen_36.py:1030-1065, kernels/gqa_varlen.py)
 *   - device-resident step metadata         (replaces the runner's per-step table / slot builders,
 *                                            engine/model_runner.py:538-637)
 *   - QK-norm + RoPE (+ append), sigmoid     (replace kernels/qknorm_rope.py, kernels/act_mul.py's
 *     gate (+ in decode's epilogue)          fused_sigmoid_mul around the path)
 *
 * Conventions shared by every entry point
 *   - All tensor pointers are DEVICE pointers owned by the caller. The library never allocates,
 *     frees or synchronises inside a call: every call only enqueues kernels on `stream`.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Calls on different streams
 *     are independent; a workspace buffer must not be shared by calls that can overlap.
 *   - Strides are in ELEMENTS, not bytes.
 *   - dtype codes: TI_DTYPE_BF16 or TI_DTYPE_F16 (the cache, key/value, q and out share it).
 *   - Return value: TI_OK (0) on success, otherwise one of the TI_E* codes below; the text of the
 *     most recent error on the calling thread is returned by ti_last_error().
 */
#ifndef TILEINFER_AMD_H_
#define TILEINFER_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TI_DTYPE_BF16 0
#define TI_DTYPE_F16 1

#define TI_OK 0
#define TI_EINVAL 1       /* bad argument: shape, stride, alignment or size out of range */
#define TI_ELAUNCH 2      /* the HIP runtime rejected a launch or a device query */
#define TI_EUNSUPPORTED 3 /* valid arguments that this build has no kernel for */

/* Decode kernel variants (argument `variant` of ti_gqa_decode_paged). */
#define TI_DECODE_AUTO 0   /* the measured-fastest variant for the shape */
#define TI_DECODE_MFMA 1   /* query group packed into a 16-row MFMA tile, K/V direct to registers */
#define TI_DECODE_SCALAR 2 /* K/V pages staged in LDS, fp32 FMA, DPP/shuffle softmax reductions */
/* Cache policy of the K/V loads. With neither flag (the default) the MFMA variant chooses per
 * sequence on the device: a sequence whose first block id another sequence of the batch also has
 * in its first column (prefix caching shares whole-block chains from there) loads with the default
 * cache policy, so the pages the other sequences read again are served from L2/MALL; every other
 * sequence loads its pages as a once-read stream (`nt`), faster when a page is read once per call.
 * (Batches above 2,048 sequences stream.) TI_DECODE_REUSE_KV forces the default policy for every
 * page, TI_DECODE_STREAM_KV forces `nt`; the scalar variant streams unless REUSE_KV is given.
 * Results are bitwise the same under every policy. */
#define TI_DECODE_REUSE_KV 0x10
#define TI_DECODE_STREAM_KV 0x20

/*
 * Slot-mapped K/V append: for every i in [0, n_tokens) with 0 <= slot_mapping[i] < num_slots,
 *   k_cache[slot_mapping[i], 0:row_elems] = key[i, 0:row_elems]
 *   v_cache[slot_mapping[i], 0:row_elems] = value[i, 0:row_elems]
 * Rows whose slot is negative are skipped (the reference's padding convention); slots at or beyond
 * num_slots are skipped as well instead of writing out of bounds. A bit copy: no arithmetic.
 * Duplicate non-negative slots within one call are unsupported (the surviving row is unspecified).
 *
 * Replaces: store_kvcache(key, value, k_cache, v_cache, slot_mapping)
 *           kernels/kvcache_store.py:43-71 (kernel body 14-40, torch semantics 74-84).
 *   key/value        [n_tokens, row_elems] rows at key_row_stride / value_row_stride (the
 *                    reference's key.reshape(N, num_heads*head_dim))
 *   k_cache/v_cache  [num_slots, row_elems] rows at cache_row_stride (kernels/kvcache_store.py:55-56)
 *   slot_mapping     [n_tokens] int32, -1 = skip (kernels/kvcache_store.py:57)
 */
int ti_kv_append(const void* key, const void* value, int64_t key_row_stride,
                 int64_t value_row_stride, void* k_cache, void* v_cache, int64_t cache_row_stride,
                 const int32_t* slot_mapping, int64_t n_tokens, int64_t row_elems, int64_t num_slots,
                 int32_t dtype, void* stream);

/*
 * Launch plan of a paged decode call and the fp32 workspace it needs.
 *   split_tokens > 0: fixed split-K -- one workgroup per (sequence, partition of split_tokens);
 *     outputs the split used, the maximum partitions per sequence, and the workspace (0 when every
 *     sequence fits one partition). The value must be a multiple of 32 and of page_size.
 *   split_tokens <= 0: the MFMA variant's own choice.
 *     - Bounds of at most 128 tokens whose (sequence, KV head) pairs fit one round (batch x
 *       num_kv_heads <= CUs), and bounds of at most 512 tokens whose pairs fill three quarters
 *       to all of one round (3/4 CUs <= batch x num_kv_heads <= CUs): one 4-wave workgroup per
 *       pair, its waves splitting the sequence's tiles and combining their parts in LDS (no
 *       partials, no merge); outputs split_tokens_out = 0, max_splits_out = 0.
 *     - Short bounds (max_blocks_per_seq * page_size <= 1024 tokens) whose fixed partitions of
 *       the smallest split (lcm(32, page_size) tokens) fit one round of workgroups (batch x
 *       partitions x KV-head groups <= CUs): that fixed split, output as for split_tokens > 0.
 *     - Otherwise balanced: one round of workgroups (one KV-head wave per SIMD; whole further
 *       rounds when a run would exceed the block ids one workgroup stages) shares the batch's
 *       16-token tiles evenly whatever the per-sequence lengths (sequences cut between
 *       workgroups are merged in a fixed order); outputs split_tokens_out = 0, max_splits_out =
 *       the number of runs per group of KV heads.
 *     The workspace covers both plans and the scalar variant's own plan (the partials, plus
 *     batch + 1 ints the balanced merge reads).
 * The plan depends only on host-known bounds, so it is valid for any seqlen values <=
 * max_blocks_per_seq * page_size and it is safe to compute once and reuse under graph capture.
 *
 * No reference counterpart: the reference decode has no split-K (kernels/gqa_decode_paged.py:73,
 * one CTA per (sequence, KV head)); this is the sizing half of the split-K design.
 */
int ti_gqa_decode_plan(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t page_size, int32_t max_blocks_per_seq, int32_t split_tokens,
                       int32_t* split_tokens_out, int32_t* max_splits_out,
                       int64_t* workspace_bytes_out);

/*
 * Paged GQA decode attention for one query token per sequence:
 *   out[b, h, :] = softmax_j( q[b,h,:] . K_b[j,:] * head_dim^-0.5 ) @ V_b[j,:],  j < seqlen[b]
 * where K_b[j] = k_cache[block_table[b, j / page_size], j % page_size, h / (Hq/Hkv), :] and V_b
 * likewise. fp32 accumulation and softmax; output rounded to the input dtype (RNE).
 * seqlen[b] == 0 gives a zero row. Block ids outside [0, num_blocks) at positions < seqlen[b]
 * are treated as absent (masked, never loaded); entries at or beyond ceil(seqlen[b]/page_size)
 * are never read, so the -1 padding of the reference's tables is harmless.
 *
 * Replaces: gqa_decode_paged_fn(q, k_cache, v_cache, block_table, seqlen_kv, page_size=16)
 *           kernels/gqa_decode_paged.py:392-437 (math: ref_gqa_decode_paged, 444-461).
 *   q            [batch, num_q_heads, head_dim], last dim contiguous, strides q_stride_b/_h
 *   k/v_cache    [num_blocks, page_size, num_kv_heads, head_dim] contiguous (one layer's slab);
 *                page_size 1, 2, 4, 8 or a multiple of 16 (the reference takes pages that divide
 *                its 64-token tile, kernels/gqa_decode_paged.py:57-62, 408; engine/config.py:20)
 *   block_table  [batch, >= ceil(max seqlen / page_size)] int32, row stride block_table_stride;
 *                max_blocks_per_seq bounds every seqlen: seqlen[b] <= max_blocks_per_seq*page_size
 *   seqlen       [batch] int32 (the reference's seqlen_kv / context_lens)
 *   out          [batch, num_q_heads, head_dim] contiguous
 *   workspace    >= workspace_bytes from ti_gqa_decode_plan with the same arguments (may be NULL
 *                when that is 0); contents need no initialisation.
 *   split_tokens as in ti_gqa_decode_plan; variant one of TI_DECODE_AUTO/MFMA/SCALAR, optionally
 *                OR'd with TI_DECODE_REUSE_KV or TI_DECODE_STREAM_KV.
 */
int ti_gqa_decode_paged(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                        const void* v_cache, const int32_t* block_table, int64_t block_table_stride,
                        const int32_t* seqlen, void* out, void* workspace, int64_t workspace_bytes,
                        int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t page_size, int64_t num_blocks, int32_t max_blocks_per_seq,
                        int32_t split_tokens, int32_t variant, int32_t dtype, void* stream);

/*
 * Whole-block copy between two paged caches (device or pinned host memory, in any direction):
 * for every pair i, block block_pairs[2i] of `src` is copied to block block_pairs[2i+1] of `dst`.
 * A block consists of `n_chunks` chunks of `chunk_bytes`; chunk c of block b starts at
 * base + c * chunk_stride_bytes + b * chunk_bytes (for the [2, layers, blocks, ...] cache slab:
 * n_chunks = 2 * layers, chunk_bytes = one layer's K or V block, chunk_stride = blocks *
 * chunk_bytes). `src`/`dst` must span n_chunks * their chunk stride; `block_pairs` is int64
 * [n_pairs, 2] in device-readable memory. Pairs with an id outside [0, num_blocks) are skipped.
 * Destination blocks must be distinct. One launch on `stream`; pinned host memory is accessed
 * directly by the kernel.
 *
 * No reference counterpart: tileInfer accepts a swap budget but never moves KV blocks
 * (engine/config.py:22, engine/block_manager.py:29); this is the data path of block swapping and
 * copy-on-write.
 */
int ti_copy_blocks(const void* src, void* dst, const int64_t* block_pairs, int64_t n_pairs,
                   int32_t n_chunks, int64_t chunk_bytes, int64_t src_chunk_stride_bytes,
                   int64_t dst_chunk_stride_bytes, int64_t src_num_blocks, int64_t dst_num_blocks,
                   void* stream);

/*
 * Causal (or full) GQA prefill attention reading K/V straight from the paged cache.
 *
 * Replaces the chunked-prefill path of model/qwen_36.py:1030-1065, which gathers every cached
 * position through block_tables into contiguous K/V and then calls the varlen flash-attention
 * kernel kernels/gqa_varlen.py:40-185 (dispatch 369-389); same arguments' meaning, with the K/V
 * source being the cache instead of the gathered copy. Sequence b owns query rows
 * [cu_seqlens_q[b], cu_seqlens_q[b+1]) of `q` and attends over its first seqlen_k[b] cached tokens
 * (the chunk's own K/V already appended), gathered through block_table[b]. With `causal` set the
 * mask is bottom-right aligned (query i sees keys j <= seqlen_k[b] - q_len + i); query head h reads
 * KV head h / (num_q_heads / num_kv_heads); scale = head_dim^-1/2; a row with no visible key is 0.
 * Block ids outside [0, num_blocks) inside the context are absent pages (their keys are masked,
 * never loaded); table entries past ceil(seqlen_k[b] / page_size) are never read.
 *   q            [total_q, num_q_heads, head_dim] (16-byte aligned rows, unit innermost stride)
 *   k/v_cache    as for ti_gqa_decode_paged
 *   cu_seqlens_q [batch + 1] int32, non-decreasing, cu_seqlens_q[batch] <= total_q (values are
 *                clamped into [0, total_q], so rows outside q/out are never touched)
 *   seqlen_k     [batch] int32, clamped to max_blocks_per_seq * page_size
 *   out          [total_q, num_q_heads, head_dim], written for every row covered by cu_seqlens_q
 *   max_seqlen_q >= every q_len (rows past it are not computed)
 *   workspace    NULL (workspace_bytes ignored): one workgroup per (sequence, KV head, block of
 *                consecutive (token, query head) rows), one launch; each row's result is then independent of the rest of
 *                the batch and of how the prompt was chunked (bitwise). Otherwise, at least
 *                ti_gqa_prefill_workspace_bytes() bytes, 256-byte aligned: a balanced schedule
 *                gives every CU the same number of key tiles (units cut between workgroups are
 *                merged in a fixed order; deterministic, but not batch-invariant); three launches
 *                (schedule, attention, merge). The workspace is scratch of this call only.
 * Launches on `stream`. head_dim 128 or 256; page_size 4, 8 or a multiple of 16; a page of
 * page_size x num_kv_heads x head_dim elements must fit 4 GiB (TI_EUNSUPPORTED otherwise).
 */
int ti_gqa_prefill_paged(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                         const void* k_cache, const void* v_cache, const int32_t* block_table,
                         int64_t block_table_stride, const int32_t* cu_seqlens_q,
                         const int32_t* seqlen_k, void* out, int64_t out_stride_t,
                         int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                         int32_t batch, int32_t total_q, int32_t max_seqlen_q,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                         int32_t page_size, int64_t num_blocks, int32_t max_blocks_per_seq,
                         int32_t causal, int32_t dtype, void* stream);

/*
 * ti_gqa_prefill_paged with the sigmoid gate in its output epilogue:
 *   out[t, h, :] = prefill(t, h) * sigmoid(gate[t * gate_stride_t + h * gate_stride_h + :])
 * bitwise what ti_gqa_prefill_paged followed by ti_sigmoid_mul gives (attention output rounded to
 * the storage type first, as the unfused pair does), without the extra pass over the output. The
 * gate of model/qwen_36.py:1083 on the prefill path is q_gate [1, q_len, H_q * D]
 * (gate_stride_t = H_q * D, gate_stride_h = D); gate rows 16-byte aligned. Both schedules.
 */
int ti_gqa_prefill_paged_gated(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                               const void* k_cache, const void* v_cache,
                               const int32_t* block_table, int64_t block_table_stride,
                               const int32_t* cu_seqlens_q, const int32_t* seqlen_k, void* out,
                               int64_t out_stride_t, int64_t out_stride_h, void* workspace,
                               int64_t workspace_bytes, int32_t batch, int32_t total_q,
                               int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t page_size, int64_t num_blocks,
                               int32_t max_blocks_per_seq, int32_t causal, int32_t dtype,
                               const void* gate, int64_t gate_stride_t, int64_t gate_stride_h,
                               void* stream);

/*
 * ti_gqa_prefill_paged with unnormalised fp32 output, for merging with attention over other keys:
 *   o_part  [key_splits, total_q, num_q_heads, head_dim] fp32, o relative to 2^m (16-byte aligned)
 *   ml_part [key_splits, total_q, num_q_heads, 2] fp32 (m, l): m the running maximum of the scaled
 *           scores in exp2 units (-inf: no visible key), l the sum of 2^(s - m)
 * so that out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s, M = max_s m_s. key_splits = 1 is
 * one part per row (any schedule); key_splits > 1 cuts every unit's keys into that many contiguous
 * ranges, one workgroup and one part each (per-unit schedule: workspace must be NULL). No reference
 * counterpart: it is the prefix half of ti_gqa_decode_paged_prefixed (a shared prefix attended once
 * for a whole decode batch).
 */
int ti_gqa_prefill_paged_partial(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                 const void* k_cache, const void* v_cache,
                                 const int32_t* block_table, int64_t block_table_stride,
                                 const int32_t* cu_seqlens_q, const int32_t* seqlen_k,
                                 float* o_part, float* ml_part, void* workspace,
                                 int64_t workspace_bytes, int32_t batch, int32_t total_q,
                                 int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t page_size, int64_t num_blocks,
                                 int32_t max_blocks_per_seq, int32_t causal, int32_t dtype,
                                 int32_t key_splits, void* stream);

/*
 * Key splits for a one-sequence ti_gqa_prefill_paged_partial pass of total_q queries over
 * kv_tokens keys (the shared prefix of a decode batch): enough workgroups to give every compute
 * unit one, each key range at least 4 key tiles; 1 when splitting does not pay. Host-only.
 */
int32_t ti_gqa_prefill_key_splits(int32_t total_q, int32_t num_q_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t kv_tokens);

/*
 * Workspace of the balanced ti_gqa_prefill_paged schedule for these sizes (host-only, no device
 * work). *bytes_out = 0 when the call must run without one (more than 8192 sequences, or tile
 * counts past int32). No reference counterpart (the reference's varlen kernel takes no workspace).
 */
int ti_gqa_prefill_workspace_bytes(int32_t batch, int32_t total_q, int32_t num_q_heads,
                                   int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                   int32_t max_blocks_per_seq, int64_t* bytes_out);

/*
 * Device-resident paged metadata for one step: persistent block tables updated in place, and the
 * step's slot mapping, context lengths and -1-padded batch block tables derived on the GPU.
 *
 * Replaces the per-step host builders engine/model_runner.py:538-584 (_prepare_decode_into_graph,
 * including graph padding 580-584), 586-593 (_build_block_tables) and 595-637 (slot mappings),
 * which rebuild and upload every sequence's whole table each step. Inputs (int32, device):
 *   tables       [num_rows, table_stride] persistent tables (row = a sequence's slot), updated
 *   batch_rows   [n] persistent row of batch entry i (distinct within a call)
 *   ctx_new      [n] context length of entry i after this step's tokens
 *   table_len    [n] length of entry i's block table (ids copied to bt_out; -1 past them)
 *   tok_off      [n+1] entry i's new tokens are slot_out[tok_off[i] .. tok_off[i+1]), the last
 *                tok_off[i+1]-tok_off[i] positions before ctx_new[i] (decode: one token each)
 *   upd_off      [n+1] entry i's table updates are upd_col/upd_id[upd_off[i] .. upd_off[i+1]):
 *                tables[batch_rows[i]][upd_col[k]] = upd_id[k] (the ids appended since the last
 *                step; a whole table for a sequence new to its row)
 * Outputs: slot_out [tok_off[n] + pad_to - n] (a position without a block gives -1),
 *   ctx_out [pad_to], bt_out [pad_to, width] at bt_stride (optional, NULL to skip; entries past
 *   table_len are -1). Entries [n, pad_to) are graph padding: slot -1, context length
 *   1, block -1 (engine/model_runner.py:524-527). One launch on `stream`.
 */
int ti_paged_metadata(int32_t* tables, int64_t table_stride, int32_t num_rows, int32_t max_blocks,
                      const int32_t* batch_rows, const int32_t* ctx_new,
                      const int32_t* table_len, const int32_t* tok_off,
                      const int32_t* upd_off, const int32_t* upd_col, const int32_t* upd_id,
                      int32_t n, int32_t pad_to, int32_t* slot_out, int32_t* ctx_out,
                      int32_t* bt_out, int64_t bt_stride, int32_t width, int32_t page_size,
                      void* stream);

/*
 * Per-head RMSNorm with a (1 + weight) scale, then rotary embedding of the first rotary_dim
 * dimensions (rotate-half pairing i <-> i + rotary_dim/2, cos/sin[0 .. rotary_dim/2) for both
 * halves), for n_tokens x n_heads rows of head_dim values:
 *   y = x * rsqrt(mean(x^2) + eps) * (1 + weight)   (fp32, rounded to the storage type)
 *   out[i] = y[i] c_i - y[i+h] s_i,  out[i+h] = y[i+h] c_i + y[i] s_i  (i < h = rotary_dim/2),
 *   out[i] = y[i] for i >= rotary_dim.
 * Replaces fused_qknorm_rope(x, weight, cos_flat, sin_flat, eps) (kernels/qknorm_rope.py:52-56,
 * kernel 9-50) and generalises it to many tokens with per-token cos/sin (row stride cs_stride_t;
 * 0 = one vector for all tokens, as the reference kernel takes). head_dim 128 or 256; rows 4-byte
 * aligned; x and out may alias.
 */
int ti_qknorm_rope(const void* x, int64_t x_stride_t, int64_t x_stride_h, void* out,
                   int64_t out_stride_t, int64_t out_stride_h, const void* weight,
                   const void* cos, const void* sin, int64_t cs_stride_t, int32_t n_tokens,
                   int32_t n_heads, int32_t head_dim, int32_t rotary_dim, float eps,
                   int32_t dtype, void* stream);

/*
 * One launch for the attention inputs of a step (model/qwen_36.py:977-1018): q heads normalised
 * and rotated into q_out; k heads normalised and rotated and written straight into the k cache row
 * of their slot; v heads copied into the v cache row of their slot (slots < 0 or >= num_slots are
 * skipped, as ti_kv_append does). Bitwise what ti_qknorm_rope on q and k followed by ti_kv_append
 * gives; no intermediate k tensor. Cache rows are [num_slots, cache_row_stride] with head h at
 * h * head_dim.
 */
int ti_qknorm_rope_append(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k,
                          int64_t k_stride_t, int64_t k_stride_h, const void* v,
                          int64_t v_stride_t, int64_t v_stride_h, const void* q_weight,
                          const void* k_weight, const void* cos, const void* sin,
                          int64_t cs_stride_t, void* q_out, int64_t q_out_stride_t,
                          int64_t q_out_stride_h, void* k_cache, void* v_cache,
                          int64_t cache_row_stride, const int32_t* slot_mapping, int64_t num_slots,
                          int32_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                          int32_t head_dim, int32_t rotary_dim, float eps, int32_t dtype,
                          void* stream);

/*
 * out[i] = a[i] * sigmoid(b[i]) for n (even) contiguous values, computed in fp32 and rounded to the
 * storage type. Replaces fused_sigmoid_mul(a, b) (kernels/act_mul.py:62-79), the attention output
 * gate of model/qwen_36.py:1083.
 */
int ti_sigmoid_mul(const void* a, const void* b, void* out, int64_t n, int32_t dtype,
                   void* stream);

/*
 * ti_gqa_decode_paged with the sigmoid gate in its output epilogue:
 *   out[b, h, :] = decode(b, h) * sigmoid(gate[b * gate_stride_b + h * gate_stride_h + :])
 * bitwise what ti_gqa_decode_paged followed by ti_sigmoid_mul gives (decode output rounded to the
 * storage type first, as the unfused pair does), without the extra pass over the output. The gate
 * of model/qwen_36.py:1083 is q_gate [B, 1, H_q * D]: gate_stride_b = H_q * D, gate_stride_h = D.
 * MFMA variant only (TI_DECODE_SCALAR returns TI_EUNSUPPORTED).
 */
int ti_gqa_decode_paged_gated(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                              const void* k_cache, const void* v_cache,
                              const int32_t* block_table, int64_t block_table_stride,
                              const int32_t* seqlen, void* out, void* workspace,
                              int64_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                              int64_t num_blocks, int32_t max_blocks_per_seq,
                              int32_t split_tokens, int32_t variant, int32_t dtype,
                              const void* gate, int64_t gate_stride_b, int64_t gate_stride_h,
                              void* stream);

/*
 * The decode step's append and attention in one call: ti_kv_append of one new token per sequence
 * (key/value row b [num_kv_heads * head_dim] at key_row_stride / value_row_stride elements, written
 * to cache row slot_mapping[b]; rows with a slot < 0 or >= num_slots are skipped) followed by
 * ti_gqa_decode_paged, bitwise what the two calls give, in the launches of the decode alone: the
 * workgroup whose tokens end at a sequence's last position writes that token's rows before it
 * reads them. Requires slot_mapping[b] to be the slot of position seqlen[b] - 1 (the reference
 * runner's decode step: engine/model_runner.py:628-637 with context_lens = num_tokens), so the
 * rows written are the rows the call reads. Cache rows are the decode's token rows
 * ([num_blocks * page_size, num_kv_heads * head_dim]). MFMA variant only.
 * Reference counterpart: store_kvcache(k, v, k_cache, v_cache, slot_mapping) then
 * gqa_decode_paged_fn(q, k_cache, v_cache, block_table, seqlen_kv) (model/qwen_36.py:1018, 1074;
 * kernels/kvcache_store.py:43-71, kernels/gqa_decode_paged.py:392-437).
 */
int ti_gqa_decode_paged_append(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                               const void* k_cache, const void* v_cache,
                               const int32_t* block_table, int64_t block_table_stride,
                               const int32_t* seqlen, void* out, void* workspace,
                               int64_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                               int64_t num_blocks, int32_t max_blocks_per_seq,
                               int32_t split_tokens, int32_t variant, int32_t dtype,
                               const void* key, const void* value, int64_t key_row_stride,
                               int64_t value_row_stride, const int32_t* slot_mapping,
                               int64_t num_slots, void* stream);

/*
 * ti_gqa_decode_paged (optionally gated) for a batch whose sequences share their first
 * prefix_tokens tokens (a multiple of page_size): the kernel attends to tokens
 * [prefix_tokens, seqlen[b]) of each sequence, through block_table columns from
 * prefix_tokens / page_size on, and merges into every row the precomputed prefix parts
 * (prefix_o [prefix_parts, B, H_q, D], prefix_ml [prefix_parts, B, H_q, 2], as
 * ti_gqa_prefill_paged_partial writes them with key_splits = prefix_parts), in part order. Rows
 * with seqlen[b] < prefix_tokens (graph padding) get no prefix part.
 * Same arguments as ti_gqa_decode_paged_gated otherwise (gate may be NULL); the workspace is
 * ti_gqa_decode_plan's for max_blocks_per_seq - prefix_tokens / page_size, plus
 * batch * num_q_heads * (head_dim + 2) * 4 bytes when split_tokens is 0 (the balanced plan keeps
 * the rows of sequences one workgroup covers whole there, for the merge to fold the prefix parts
 * into). MFMA variant only.
 * Reference counterpart: gqa_decode_paged_fn (kernels/gqa_decode_paged.py:392-437) on a batch
 * whose block tables share a prefix (engine/scheduler.py:161-189 share_blocks), which reads the
 * shared pages once per sequence.
 */
int ti_gqa_decode_paged_prefixed(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 const void* k_cache, const void* v_cache,
                                 const int32_t* block_table, int64_t block_table_stride,
                                 const int32_t* seqlen, void* out, void* workspace,
                                 int64_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                 int64_t num_blocks, int32_t max_blocks_per_seq,
                                 int32_t split_tokens, int32_t variant, int32_t dtype,
                                 const void* gate, int64_t gate_stride_b, int64_t gate_stride_h,
                                 const float* prefix_o, const float* prefix_ml,
                                 int32_t prefix_parts, int32_t prefix_tokens, void* stream);

/*
 * ti_gqa_decode_paged without a workspace argument, for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference (its decode allocates its output and a padded block table on every
 * call, kernels/gqa_decode_paged.py:421-437). Same arguments and results as ti_gqa_decode_paged;
 * the split-K partials go to a static device array of ti_gqa_decode_scratch_bytes() bytes
 * (32 MiB) that each GPU the library runs on holds until the process ends. Calls whose launch
 * needs more (the workspace ti_gqa_decode_paged would use for the same call, of which
 * ti_gqa_decode_plan's workspace_bytes, taken over every plan, is an upper bound) return
 * TI_EINVAL. Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (different streams, or host threads) race and must be
 * serialised by the caller. Allocates and frees nothing; the array's device address is looked up
 * once per device on the first call.
 */
int ti_gqa_decode_paged_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, const void* v_cache,
                                const int32_t* block_table, int64_t block_table_stride,
                                const int32_t* seqlen, void* out, int32_t batch,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t page_size, int64_t num_blocks, int32_t max_blocks_per_seq,
                                int32_t split_tokens, int32_t variant, int32_t dtype, void* stream);

/* Size in bytes of the per-GPU static scratch of ti_gqa_decode_paged_noalloc. */
int64_t ti_gqa_decode_scratch_bytes(void);

/* Text of the last error reported on the calling thread ("" when none). */
const char* ti_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int32_t ti_abi_version(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TILEINFER_AMD_H_ */
