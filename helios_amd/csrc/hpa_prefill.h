// Arguments shared by the chunked-prefill / verify kernels (hpa_prefill.hip,
// hpa_prefill_mfma.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hpa {

struct PrefillArgs {
  const void* q;
  void* out;
  const void* k;
  const void* v;
  const void* ks;
  const void* vs;
  const int32_t* tables;
  int table_stride;
  const int32_t* cu_q;
  const int32_t* q_pos;
  const int32_t* ctx_lens;
  int num_seqs, num_q_heads, num_kv_heads, group;
  int bs_log2, num_blocks;
  float scale_log2;
  // > 0: a speculative verify, uniform_q query tokens per sequence.  cu_q and
  // q_pos are not read: sequence b's tokens are [b uniform_q, (b + 1)
  // uniform_q) and its first token sits at ctx_lens[b] - uniform_q.
  // Honoured by the MFMA kernel only.
  int uniform_q;
};

// LDS-tiled 32x32 MFMA prefill for fp16 / bf16 queries over pools of the
// same dtype or int8 pools (fp16 / fp32 scales), head_dim 64 or 128 and
// block_size >= 16; returns false (launching nothing) for other shapes.
bool launch_prefill_mfma(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim,
                         int max_q_len, hipStream_t s);

}  // namespace hpa
