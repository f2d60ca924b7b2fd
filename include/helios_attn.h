/* helios_attn.h -- C-ABI of the MI355X (gfx950) paged-attention library
 * (libheliosattn.so).
 *
 * The library is the GPU half of helios' paged-attention path.  Every entry
 * point takes raw device pointers, plain integers and a hipStream_t, launches
 * asynchronously on that stream, allocates nothing, keeps no pointer after it
 * returns and never synchronises the host.  The caller owns every buffer.
 * Return value: HPA_OK (0) or one of the HPA_ERR_* codes below, with a
 * message from hpa_last_error() (thread-local).
 *
 * Layouts are helios' own (reference python/helios/exec/paged_attn.py):
 *   K/V pool      [num_blocks, num_kv_heads, block_size, head_dim]   (:49-51)
 *   int8 scales   [num_blocks, num_kv_heads, block_size]             (:166-168)
 *   block tables  int32 [num_seqs, table_stride], zero padded
 *                 (reference exec/triton_attn.py:156-165)
 *   queries / out [tokens, num_q_heads, head_dim], query head h reads KV
 *                 head h / (num_q_heads / num_kv_heads)   (triton_attn.py:83)
 * Position p of a sequence lives in block table[p / block_size] at offset
 * p % block_size (paged_attn.py:74-85).  block_size must be a power of two
 * (>= 4 for attention).  head_dim is one of 8, 16, 32, 64, 128, 256.
 *
 * The tables are trusted: a block id outside [0, num_blocks) is read as
 * block 0 (attention, gather) or skipped (write, copy) so that a bad table can
 * never address memory outside the pool.  Callers that build tables on the
 * host validate them first (the Python layer raises IndexError there, like
 * paged_attn.py:78-82 and :101-104).
 */
#ifndef HELIOS_ATTN_H
#define HELIOS_ATTN_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HPA_VERSION 1

/* status codes */
#define HPA_OK 0
#define HPA_ERR_ARG 1         /* null pointer or inconsistent shape */
#define HPA_ERR_UNSUPPORTED 2 /* dtype / head_dim / block_size not built */
#define HPA_ERR_WORKSPACE 3   /* workspace smaller than hpa_decode_workspace_size() */
#define HPA_ERR_LAUNCH 4      /* the HIP runtime refused a launch */

/* element types */
#define HPA_F32 0
#define HPA_F16 1
#define HPA_BF16 2
#define HPA_I8 3

/* Library version (HPA_VERSION). */
int hpa_version(void);

/* Message describing the last failure on this thread. */
const char* hpa_last_error(void);

/* Bytes of split-K workspace hpa_paged_decode needs for these shapes
 * (0 when no sequence is split, or when the shapes run on the prefill
 * kernels).  part_tokens: 0 = library default. */
size_t hpa_decode_workspace_size(int num_seqs, int q_per_seq, int num_q_heads, int num_kv_heads,
                                 int head_dim, int max_context_len, int part_tokens);

/* Paged decode and speculative verify.
 * Replaces paged_attention_decode_batched (paged_attn.py:298-353),
 * paged_attention_decode (paged_attn.py:264-295) and the Triton kernel behind
 * paged_attention_decode_triton (triton_attn.py:54-183), extended with int8 KV
 * and with q_per_seq > 1 query tokens per sequence.
 *   q, out        [num_seqs * q_per_seq, num_q_heads, head_dim], dtype q_dtype
 *                 (F32, F16 or BF16; out has the same dtype)
 *   k/v_pool      kv_dtype == q_dtype, or HPA_I8 with k/v_scale of
 *                 scale_dtype (F16 as helios stores them, or F32)
 *   context_lens  int32 [num_seqs], each at most 2^30
 *   max_context_len  an upper bound of context_lens, used only to size the
 *                 launch and the workspace: every context is honoured as
 *                 given (one above the bound makes the call slower, never
 *                 wrong)
 * Token t of sequence b attends keys [0, context_lens[b] - q_per_seq + t]
 * (helios' causal rule, paged_attn.py:401-404, with start_pos = context -
 * q_per_seq).  An empty context yields zeros.  Softmax scale sm_scale.
 * Any number of query rows per KV head ((num_q_heads / num_kv_heads) *
 * q_per_seq) is taken.  17-64 rows with fp16 or bf16 queries over an int8
 * pool (head_dim 64 or 128, block_size >= 16) run on a verify kernel that
 * dequantises in registers; it uses the workspace, when given, to cut long
 * contexts (fewer cuts with a smaller one).  Over fp16 / bf16 pools, 17 rows
 * and more, and other shapes above 32 rows, run on the MFMA prefill kernel
 * when it takes the shape (fp16 / bf16 queries, head_dim 64 or 128,
 * block_size >= 16), and above 64 rows on the generic prefill kernel when it
 * does not, with the same results as hpa_paged_prefill over the same tokens;
 * the workspace is then unused.  Up to 64 rows the shapes no other kernel
 * takes run on the decode kernel.
 * part_tokens: smallest share of the context, in tokens, one wave streams
 * (0 = library default); it changes only the summation order.
 * workspace: at least hpa_decode_workspace_size(...) bytes of device memory
 * (may be NULL if that is 0), zero-filled before its first use.  It holds
 * per-(sequence, KV head) arrival counters that every completed call leaves
 * at zero again, so one workspace serves any number of calls ordered on one
 * stream; calls that may run concurrently need separate workspaces.  A call
 * that did not complete (a launch error, a device reset) may leave counters
 * set: zero-fill the workspace again before reusing it. */
int hpa_paged_decode(const void* q, void* out, int q_dtype, const void* k_pool, const void* v_pool,
                     int kv_dtype, const void* k_scale, const void* v_scale, int scale_dtype,
                     const int32_t* block_tables, int table_stride, const int32_t* context_lens,
                     int num_seqs, int q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                     int block_size, int num_blocks, int max_context_len, float sm_scale,
                     int part_tokens, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Bytes of the static scratch hpa_paged_decode_noalloc uses per GPU. */
#define HPA_NOALLOC_SCRATCH_BYTES (64u << 20)

/* hpa_paged_decode for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the same
 * arguments and results (bit for bit, except 17-64-row int8 verifies, which
 * it runs without cutting units: there it agrees within the fp16 bound, as
 * hpa_paged_decode does across workspace sizes), with the split-K workspace
 * taken from a static
 * device array of HPA_NOALLOC_SCRATCH_BYTES that the library holds on each
 * GPU it runs on until the process ends.  It calls no hipMalloc, hipFree or
 * allocating routine.  Each call first clears the arrival counters it uses
 * (a small kernel on `stream`, no memset).  Shapes whose workspace
 * (hpa_decode_workspace_size) exceeds the scratch are refused with
 * HPA_ERR_WORKSPACE.  Every call on one GPU shares that GPU's scratch: calls
 * that may overlap on one GPU (different streams) race and must not be
 * made.  No counterpart in the reference (helios allocates per call); this
 * is for the callers above. */
int hpa_paged_decode_noalloc(const void* q, void* out, int q_dtype, const void* k_pool,
                             const void* v_pool, int kv_dtype, const void* k_scale,
                             const void* v_scale, int scale_dtype, const int32_t* block_tables,
                             int table_stride, const int32_t* context_lens, int num_seqs,
                             int q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                             int block_size, int num_blocks, int max_context_len, float sm_scale,
                             int part_tokens, hipStream_t stream);

/* Chunked prefill / verify over a ragged batch, in one launch.
 * Replaces paged_attention_prefill (paged_attn.py:368-408) called once per
 * sequence by BatchedAttention.run (reference exec/model.py:303-317).
 *   q, out        [cu_q_lens[num_seqs], num_q_heads, head_dim]
 *   cu_q_lens     int32 [num_seqs + 1]: sequence b owns query tokens
 *                 [cu_q_lens[b], cu_q_lens[b+1]); max_q_len bounds their count
 *   q_positions   int32 [num_seqs]: absolute position of each sequence's first
 *                 query token (helios' start_pos)
 *   context_lens  int32 [num_seqs]: keys [0, context) exist
 *   num_tokens    rows of q and out: query tokens at or past it are neither
 *                 read nor written, whatever cu_q_lens says
 * Query token i of sequence b attends keys [0, min(q_positions[b] + i + 1,
 * context_lens[b])).  Rows with no key yield zeros. */
int hpa_paged_prefill(const void* q, void* out, int q_dtype, const void* k_pool, const void* v_pool,
                      int kv_dtype, const void* k_scale, const void* v_scale, int scale_dtype,
                      const int32_t* block_tables, int table_stride, const int32_t* cu_q_lens,
                      const int32_t* q_positions, const int32_t* context_lens, int num_seqs,
                      int max_q_len, int num_tokens, int num_q_heads, int num_kv_heads,
                      int head_dim, int block_size, int num_blocks, float sm_scale,
                      hipStream_t stream);

/* Scatter new K/V into the pool; int8 pools quantise on the fly.
 * Replaces PagedKVCache.write (paged_attn.py:57-85) and
 * QuantizedPagedKVCache.write + _quantize (paged_attn.py:177-211).
 *   k, v          [cu_tokens[num_seqs], num_kv_heads, head_dim], in_dtype
 *                 (F32, F16 or BF16)
 *   cu_tokens     int32 [num_seqs + 1]; start_positions int32 [num_seqs]:
 *                 token i of sequence b goes to position start_positions[b] + i
 *   pool_dtype    F32 / F16 / BF16 (converted, round to nearest even) or I8
 *                 (bit-exact helios quantisation, scales in scale_dtype)
 * The blocks written must be private to their sequence (the allocator's
 * copy-on-write remap, reference core/allocator.py:298-341, runs first);
 * positions whose block is missing from the table are skipped. */
int hpa_kv_write(const void* k, const void* v, int in_dtype, void* k_pool, void* v_pool,
                 int pool_dtype, void* k_scale, void* v_scale, int scale_dtype,
                 const int32_t* block_tables, int table_stride, const int32_t* cu_tokens,
                 const int32_t* start_positions, int num_seqs, int max_tokens, int num_kv_heads,
                 int head_dim, int block_size, int num_blocks, hipStream_t stream);

/* hpa_kv_write with K rotated rotate-half style (RoPE) by its write position
 * on the way into the pool: the step before attention fused into the write,
 * so K is written once, rotated (and, for int8 pools, quantized from the
 * rotated values).  rope_cos / rope_sin are fp32 [rope_rows][head_dim / 2]
 * tables, as helios' build_rope_cache makes them; with c, s = row pos, element
 * j < head_dim/2 becomes x[j] c[j] - x[j + head_dim/2] s[j] and element
 * j + head_dim/2 becomes x[j + head_dim/2] c[j] + x[j] s[j], every product and
 * sum rounded to fp32.  V is written as is.  Positions at or past rope_rows
 * are skipped, like positions without a block.  head_dim must be even.
 * Replaces apply_rope on K followed by the cache write (exec/model.py:135-153,
 * :196-206, :236-247). */
int hpa_kv_write_rope(const void* k, const void* v, int in_dtype, void* k_pool, void* v_pool,
                      int pool_dtype, void* k_scale, void* v_scale, int scale_dtype,
                      const int32_t* block_tables, int table_stride, const int32_t* cu_tokens,
                      const int32_t* start_positions, int num_seqs, int max_tokens, int num_kv_heads,
                      int head_dim, int block_size, int num_blocks, const float* rope_cos,
                      const float* rope_sin, int rope_rows, hipStream_t stream);

/* Gather one sequence's first context_len positions into contiguous
 * [context_len, num_kv_heads, head_dim] tensors of out_dtype; int8 pools are
 * dequantised as fp32(q) * fp32(scale) then rounded.
 * Replaces PagedKVCache.gather (paged_attn.py:87-110) and
 * QuantizedPagedKVCache.gather (paged_attn.py:213-235). */
int hpa_kv_gather(const void* k_pool, const void* v_pool, int pool_dtype, const void* k_scale,
                  const void* v_scale, int scale_dtype, const int32_t* block_table,
                  int context_len, void* k_out, void* v_out, int out_dtype, int num_kv_heads,
                  int head_dim, int block_size, int num_blocks, hipStream_t stream);

/* Copy-on-write / swap block copies for every layer in one launch.
 * Replaces the runner's per-layer copy_block loop (reference
 * exec/runner.py:155-165) over PagedKVCache.copy_block (paged_attn.py:112-115)
 * and QuantizedPagedKVCache.copy_block (paged_attn.py:237-245).
 *   k_pools, v_pools          device arrays [num_layers] of pool pointers
 *   k_scales, v_scales        device arrays [num_layers] of scale pointers, or
 *                             NULL for fp pools
 *   pairs                     device int32 [num_pairs][2] = (src, dst)
 *   block_bytes               bytes of one block of one pool
 *   scale_block_bytes         bytes of one block of one scale tensor
 * Destinations must be distinct and must not appear as sources in the same
 * call (copies run concurrently). */
int hpa_copy_blocks(void* const* k_pools, void* const* v_pools, void* const* k_scales,
                    void* const* v_scales, int num_layers, const int32_t* pairs, int num_pairs,
                    int num_blocks, size_t block_bytes, size_t scale_block_bytes,
                    hipStream_t stream);

/* One step's block tables from tables kept in device memory across steps.
 * Replaces rebuilding every table from Python lists each step
 * (reference exec/runner.py:205-225, 263-268) and converting them to device
 * tensors in every attention call of every layer (exec/triton_attn.py:156-165,
 * paged_attn.py:106, 347-348).
 *   resident       device int32 [resident_rows][resident_width]: one row per
 *                  resident sequence, updated in place
 *   entries        device int32 [num_entries][5] = (row, n_blocks, upd_first,
 *                  upd_count, upd_offset), one per sequence of the step, in
 *                  batch order; rows must be distinct within a call
 *   new_ids        device int32 [num_new_ids]: entry e's replaced table
 *                  entries upd_first .. upd_first + upd_count - 1 are
 *                  new_ids[upd_offset ..]
 *   step_tables    device int32 [num_entries][step_width], written: entry e's
 *                  row after the update, entries >= n_blocks as 0 (the
 *                  zero-padded table of triton_attn.py:156-165)
 * Rows outside [0, resident_rows) give all-zero step rows. */
int hpa_step_tables(const int32_t* entries, int num_entries, const int32_t* new_ids,
                    int num_new_ids, int32_t* resident, int resident_rows, int resident_width,
                    int32_t* step_tables, int step_width, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HELIOS_ATTN_H */
