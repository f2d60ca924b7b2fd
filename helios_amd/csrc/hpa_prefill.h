// Arguments shared by the chunked-prefill / verify kernels (hpa_prefill.hip,
// hpa_prefill_mfma.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hpa {

// A piece slot of verify_i8_kernel's split-K: one wave pair's unnormalised O
// (64 floats per lane) and (m, l) per lane.
constexpr int kViSlotFloats = 2 * 64 * 64 + 2 * 64 * 2;

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
  int num_seqs;
  // rows of q / out: tokens at or past it are never read or written, so
  // metadata that disagrees with the tensors cannot address memory outside them
  int num_tokens;
  int num_q_heads, num_kv_heads, group;
  int bs_log2, num_blocks;
  float scale_log2;
  // > 0: a speculative verify, uniform_q query tokens per sequence.  cu_q and
  // q_pos are not read: sequence b's tokens are [b uniform_q, (b + 1)
  // uniform_q) and its first token sits at ctx_lens[b] - uniform_q.
  int uniform_q;
  // verify_i8_kernel's split-K (read by no other kernel): one arrival
  // counter per (sequence, KV head), zero between calls; piece_slots slots
  // of kViSlotFloats floats for cut units' pieces (0: no unit is cut).
  // xcd_slots: workgroups resident per XCD, which sets the length a unit
  // must exceed to be cut.
  int* counters = nullptr;
  float* pieces = nullptr;
  int piece_slots = 0;
  int xcd_slots = 0;
  int cut_budget = 0;  // units that may be cut per XCD (set by the launcher)
};

// Sequence b's query tokens [q0, q0 + qn), the first at position pos0, with
// qn cut at num_tokens.
struct SeqSpan {
  int q0, qn, pos0;
};
__device__ __forceinline__ SeqSpan seq_span(const PrefillArgs& a, int b) {
  SeqSpan sp;
  if (a.uniform_q > 0) {
    sp = {b * a.uniform_q, a.uniform_q, a.ctx_lens[b] - a.uniform_q};
  } else {
    const int q0 = a.cu_q[b];
    sp = {q0, a.cu_q[b + 1] - q0, a.q_pos[b]};
  }
  sp.qn = max(0, min(sp.qn, a.num_tokens - sp.q0));
  if (sp.q0 < 0) sp.qn = 0;
  return sp;
}

// Longest-first order within an XCD: workgroup 8 m + x (x = its XCD) runs
// the item of rank m by cost among the nk items 8 j + x.  An item's key
// packs its cost above its inverted index j, so keys are distinct (ties go
// to the lower j) and the ranks a permutation; a rank counts the larger
// keys, four per LDS read.  keys: LDS for nk rounded up to 4 ints, 16-byte
// aligned; pick: one LDS int.  Every thread of the workgroup calls it; the
// result is uniform.  nk <= kLptMax; cost(j) >= 0.
constexpr int kLptBits = 9;
constexpr int kLptMax = 1 << kLptBits;
template <int NTHREADS, class F>
__device__ __forceinline__ int lpt_pick(int* keys, int* pick, int nk, int m, int xcd, F cost) {
  const int nk4 = (nk + 3) & ~3;
  for (int j = threadIdx.x; j < nk4; j += NTHREADS)
    keys[j] = j < nk ? (min(cost(j), (1 << (30 - kLptBits)) - 1) << kLptBits) | (kLptMax - 1 - j) : -1;
  __syncthreads();
  for (int j = threadIdx.x; j < nk; j += NTHREADS) {
    const int kj = keys[j];
    int rank = 0;
#pragma unroll 4
    for (int i = 0; i < nk4; i += 4) {
      const int4 c = *reinterpret_cast<const int4*>(&keys[i]);
      rank += (c.x > kj) + (c.y > kj) + (c.z > kj) + (c.w > kj);
    }
    if (rank == m) *pick = 8 * j + xcd;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*pick);
}

// LDS-tiled 32x32 MFMA prefill for fp16 / bf16 queries over pools of the
// same dtype or int8 pools (fp16 / fp32 scales), head_dim 64 or 128 and
// block_size >= 16; returns false (launching nothing) for other shapes.
bool launch_prefill_mfma(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim,
                         int max_q_len, hipStream_t s);

// A verify (uniform_q > 0) of 17-64 rows per KV head over an int8 pool
// (fp16 or bf16 queries, fp16 / fp32 scales, head_dim 64 / 128, block_size >= 16),
// dequantised in registers (hpa_verify_i8.hip); returns false (launching
// nothing) for other shapes.
bool launch_verify_i8(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim, hipStream_t s);

// The generic prefill kernel (any supported dtype, head_dim and block size);
// returns HPA_OK or an HPA_ERR_* status (with its message) for shapes it
// has no kernel for.
int launch_prefill_generic(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim,
                           int max_q_len, hipStream_t s);

}  // namespace hpa
