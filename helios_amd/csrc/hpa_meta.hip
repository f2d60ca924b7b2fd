// Step metadata kept in HBM across scheduler steps.
//
// helios rebuilds every step's attention metadata from Python lists: the
// runner copies each item's block table into a fresh BatchedAttnMeta
// (exec/runner.py:205-225, 263-268), and every attention call of every layer
// turns those lists into device tensors again (exec/triton_attn.py:156-165,
// paged_attn.py:106, 347-348), each conversion a synchronising host-to-device
// copy.  Here the block table of each resident sequence lives in a
// persistent device array (one row per sequence).  Between steps a table
// changes only at its tail (a block appended every block_size tokens, a
// copy-on-write replacement, a re-admission), so a step uploads only the
// changed suffix of each row, and hpa_step_tables
//   1. writes those suffixes into the resident rows, and
//   2. gathers the rows of this step's sequences, in batch order, into the
//      zero-padded [n, step_width] table every attention entry point takes,
// in one launch.  The same step tables then serve every layer.
//
// entries: int32 [num_entries][5] = (row, n_blocks, upd_first, upd_count,
// upd_offset): resident row, live blocks of the table, first replaced index,
// number of replaced entries, and where they start in new_ids.
#include "hpa_host.h"

namespace hpa {

constexpr int kMetaEntryInts = 5;

__global__ __launch_bounds__(256) void step_tables_kernel(const int32_t* __restrict__ entries,
                                                          const int32_t* __restrict__ new_ids,
                                                          int num_new_ids, int32_t* __restrict__ resident,
                                                          int resident_rows, int resident_width,
                                                          int32_t* __restrict__ step_tables, int step_width) {
  const int e = blockIdx.y;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= step_width) return;
  const int32_t* en = entries + (long)e * kMetaEntryInts;
  const int row = en[0];
  const int n_blocks = min(en[1], resident_width);
  const int first = en[2], count = en[3], off = en[4];
  int32_t val = 0;
  if (row >= 0 && row < resident_rows && j < n_blocks) {
    int32_t* r = resident + (long)row * resident_width;
    const int u = j - first;
    if (u >= 0 && u < count && off + u < num_new_ids) {
      val = new_ids[off + u];
      r[j] = val;
    } else {
      val = r[j];
    }
  }
  step_tables[(long)e * step_width + j] = val;
}

}  // namespace hpa

using namespace hpa;

extern "C" int hpa_step_tables(const int32_t* entries, int num_entries, const int32_t* new_ids,
                               int num_new_ids, int32_t* resident, int resident_rows, int resident_width,
                               int32_t* step_tables, int step_width, hipStream_t stream) {
  if (num_entries == 0) return HPA_OK;
  if (!entries || !resident || !step_tables || (num_new_ids > 0 && !new_ids))
    return fail(HPA_ERR_ARG, "hpa_step_tables: null pointer argument");
  if (num_entries < 0 || num_entries > 65535 || num_new_ids < 0 || resident_rows <= 0 ||
      resident_width <= 0 || step_width <= 0 || step_width > resident_width)
    return fail(HPA_ERR_ARG,
                "hpa_step_tables: bad shape (entries %d, new ids %d, resident %d x %d, step width %d)",
                num_entries, num_new_ids, resident_rows, resident_width, step_width);
  dim3 grid((unsigned)((step_width + 255) / 256), (unsigned)num_entries);
  hipLaunchKernelGGL(step_tables_kernel, grid, dim3(256), 0, stream, entries, new_ids, num_new_ids, resident,
                     resident_rows, resident_width, step_tables, step_width);
  return check_launch("hpa_step_tables");
}
