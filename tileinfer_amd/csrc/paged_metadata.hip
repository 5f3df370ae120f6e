// Device-resident paged-attention metadata: persistent block tables updated incrementally, and the
// per-step slot mapping / context lengths / batch block tables derived on the GPU.
//
// Replaces the per-step host builders of tileInfer's model runner, which rebuild every sequence's
// whole block table as a Python list, convert it to a tensor and copy it host to device each step
// (engine/model_runner.py:538-584 _prepare_decode_into_graph, 586-593 _build_block_tables,
// 595-637 slot mappings; graph padding 524-527, 580-584). Here the host sends only what changed:
// each batch entry's persistent row, its context length after the step, its number of new tokens,
// and the block ids appended to its table since the last step. One launch then
//   1. writes the appended ids into the persistent table rows,
//   2. emits slot[t] = table[p / page] * page + p % page for every new token (position p counted
//      back from the new context length),
//   3. emits context_lens and the batch's block tables: each entry's first table_len ids gathered
//      from its persistent row, -1 past them (the runner's -1 padding),
//   4. fills graph-padding entries [n, pad_to) with slot -1, context length 1, block -1.
// One workgroup per batch entry: an entry's updates are applied and read back by the same
// workgroup, so no grid-wide ordering is needed. Rows must be distinct within one call.
#include "ti_common.h"

namespace ti {
namespace {

constexpr int kMetaThreads = 256;

struct MetaArgs {
  int32_t* tables;
  int64_t table_stride;
  int32_t num_rows, max_blocks;
  const int32_t* batch_rows;
  const int32_t* ctx_new;
  const int32_t* table_len;
  const int32_t* tok_off;
  const int32_t* upd_off;
  const int32_t* upd_col;
  const int32_t* upd_id;
  int32_t n, pad_to, page_size, width;
  int32_t* slot_out;
  int32_t* ctx_out;
  int32_t* bt_out;
  int64_t bt_stride;
};

__global__ __launch_bounds__(kMetaThreads) void paged_metadata_kernel(MetaArgs a) {
  const int i = blockIdx.x;
  const int t = threadIdx.x;
  if (i >= a.n) {
    // Graph padding entry: one slot -1, context length 1, an all -1 table row.
    const int pad = i - a.n;
    if (t == 0) {
      a.slot_out[a.tok_off[a.n] + pad] = -1;
      a.ctx_out[i] = 1;
    }
    if (a.bt_out) {
      for (int c = t; c < a.width; c += kMetaThreads) a.bt_out[int64_t(i) * a.bt_stride + c] = -1;
    }
    return;
  }
  const int r = a.batch_rows[i];
  const bool row_ok = r >= 0 && r < a.num_rows;
  int32_t* row = a.tables + int64_t(row_ok ? r : 0) * a.table_stride;
  if (row_ok) {
    for (int k = a.upd_off[i] + t; k < a.upd_off[i + 1]; k += kMetaThreads) {
      const int c = a.upd_col[k];
      if (c >= 0 && c < a.max_blocks) row[c] = a.upd_id[k];
    }
  }
  __syncthreads();  // this workgroup's table writes are visible to its reads below
  const int ctx = max(a.ctx_new[i], 0);
  if (t == 0) a.ctx_out[i] = ctx;
  const int nblk = row_ok ? min(max(a.table_len[i], 0), a.max_blocks) : 0;
  if (a.bt_out) {
    int32_t* dst = a.bt_out + int64_t(i) * a.bt_stride;
    for (int c = t; c < a.width; c += kMetaThreads) dst[c] = c < nblk ? row[c] : -1;
  }
  const int t0 = a.tok_off[i];
  const int nt = a.tok_off[i + 1] - t0;
  for (int j = t; j < nt; j += kMetaThreads) {
    const int p = ctx - nt + j;  // position of new token j
    const int blk = p >= 0 ? p / a.page_size : -1;
    int slot = -1;
    if (blk >= 0 && blk < nblk) {  // ids past the table length may be a previous owner's
      const int id = row[blk];
      slot = id >= 0 ? id * a.page_size + p % a.page_size : -1;
    }
    a.slot_out[t0 + j] = slot;
  }
}

}  // namespace
}  // namespace ti

extern "C" int ti_paged_metadata(int32_t* tables, int64_t table_stride, int32_t num_rows,
                                 int32_t max_blocks, const int32_t* batch_rows,
                                 const int32_t* ctx_new, const int32_t* table_len,
                                 const int32_t* tok_off,
                                 const int32_t* upd_off, const int32_t* upd_col,
                                 const int32_t* upd_id, int32_t n, int32_t pad_to,
                                 int32_t* slot_out, int32_t* ctx_out, int32_t* bt_out,
                                 int64_t bt_stride, int32_t width, int32_t page_size,
                                 void* stream) {
  using namespace ti;
  if (n < 0 || pad_to < n || num_rows < 0 || max_blocks < 0 || width < 0 || page_size <= 0 ||
      table_stride < max_blocks) {
    return fail(TI_EINVAL,
                "ti_paged_metadata: bad sizes n=%d pad_to=%d rows=%d max_blocks=%d width=%d "
                "page_size=%d",
                n, pad_to, num_rows, max_blocks, width, page_size);
  }
  if (pad_to == 0) return TI_OK;
  if (!tok_off || !slot_out || !ctx_out ||
      (n > 0 && (!tables || !batch_rows || !ctx_new || !table_len || !upd_off))) {
    return fail(TI_EINVAL, "ti_paged_metadata: null pointer");
  }
  if (bt_out && bt_stride < width) {
    return fail(TI_EINVAL, "ti_paged_metadata: bt_stride %lld < width %d", (long long)bt_stride,
                width);
  }
  MetaArgs a;
  a.tables = tables;
  a.table_stride = table_stride;
  a.num_rows = num_rows;
  a.max_blocks = max_blocks;
  a.batch_rows = batch_rows;
  a.ctx_new = ctx_new;
  a.table_len = table_len;
  a.tok_off = tok_off;
  a.upd_off = upd_off;
  a.upd_col = upd_col;
  a.upd_id = upd_id;
  a.n = n;
  a.pad_to = pad_to;
  a.page_size = page_size;
  a.width = width;
  a.slot_out = slot_out;
  a.ctx_out = ctx_out;
  a.bt_out = bt_out;
  a.bt_stride = bt_stride;
  hipLaunchKernelGGL(paged_metadata_kernel, dim3(unsigned(pad_to)), dim3(kMetaThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("ti_paged_metadata");
}
