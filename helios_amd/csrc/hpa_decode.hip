// C-ABI of the paged decode / speculative-verify attention (the kernels and
// their work decomposition are in hpa_decode_impl.h).
#include <mutex>

#include "hpa_decode_impl.h"
#include "hpa_prefill.h"

namespace hpa {

static DecodeFn pick_decode(int q_dtype, int kv_dtype, int scale_dtype, int d, int nt) {
  switch (q_dtype) {
    case HPA_F32: return pick_kv<F32>(kv_dtype, scale_dtype, d, nt);
    case HPA_F16: return pick_kv<F16>(kv_dtype, scale_dtype, d, nt);
    case HPA_BF16: return pick_kv<BF16>(kv_dtype, scale_dtype, d, nt);
  }
  return nullptr;
}

static int decode_nt(int rows) { return rows <= 16 ? 1 : rows <= 32 ? 2 : rows <= 64 ? 4 : 0; }

// Waves launched and the per-wave slice floor for these shapes.  The host
// sees only max_context_len, so the wave count is sized on the upper bound
// of the step count; the kernel computes the real slices from the real
// contexts (a context above max_context_len only makes the slices longer).
struct DecodePlan {
  int waves, min_steps;
};
static DecodePlan plan_decode(int num_seqs, int num_kv_heads, int max_context_len, int min_tokens) {
  DecodePlan p;
  const int mt = min_tokens > 0 ? std::min(min_tokens, 1 << 20) : kDefaultMinTokens;
  p.min_steps = std::max(1, (mt + 31) / 32);
  const long per_unit = std::max(1L, ((long)std::min(max_context_len, kMaxContext) + 31) / 32) + kUnitCost;
  const long ub = (long)num_seqs * num_kv_heads * per_unit;
  const long w = (ub + p.min_steps - 1) / p.min_steps;
  p.waves = (int)std::max(1L, std::min<long>(w, kWaveCap));
  return p;
}

// Workspace layout: a fixed region of kMaxUnits int32 arrival counters (one
// per (sequence, KV head)), then (m, l) [W][2][rows][2] and O
// [W][2][rows][max(head_dim, 16)] in fp32.  The counters sit at the same
// place whatever the shapes, so a zero-filled workspace stays valid across
// calls of any shape.
constexpr long kMaxUnits = 1L << 18;
constexpr size_t kCounterBytes = kMaxUnits * sizeof(int);
static size_t ws_bytes(int waves, int rows, int head_dim) {
  if (waves <= 1) return 0;
  const size_t ml = (size_t)waves * 2 * rows * 2 * sizeof(float);
  const size_t o = (size_t)waves * 2 * rows * std::max(head_dim, 16) * sizeof(float);
  return kCounterBytes + ml + o;
}

}  // namespace hpa

using namespace hpa;

extern "C" size_t hpa_decode_workspace_size(int num_seqs, int q_per_seq, int num_q_heads,
                                            int num_kv_heads, int head_dim, int max_context_len,
                                            int part_tokens) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || q_per_seq <= 0 || head_dim <= 0 ||
      num_q_heads % num_kv_heads)
    return 0;
  const int rows = (num_q_heads / num_kv_heads) * q_per_seq;
  if (!decode_nt(rows)) return 0;  // more than 64 rows: the prefill kernels, no workspace
  const DecodePlan p = plan_decode(num_seqs, num_kv_heads, std::max(0, max_context_len), part_tokens);
  return ws_bytes(p.waves, rows, head_dim);
}

namespace hpa {

// ---- the workspace of hpa_paged_decode_noalloc: a static array per GPU, for
// callers that cannot allocate.  In host code `scratch` names a host-side
// stand-in, not device memory: its device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
constexpr size_t kScratchBytes = (size_t)HPA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch[kMaxDevices];

// The current device's address of `scratch`, looked up on the first call
// on that device (with it current) and kept.
static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(HPA_ERR_LAUNCH, "hpa_paged_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(HPA_ERR_UNSUPPORTED, "hpa_paged_decode_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(HPA_ERR_LAUNCH, "hpa_paged_decode_noalloc: hipGetSymbolAddress(scratch): %s",
                  hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return HPA_OK;
}

// Zeroes the arrival counters [0, n) with vector stores (a kernel, not a
// memset, so the call stays capturable in a HIP graph).
__global__ __launch_bounds__(256) void clear_counters_kernel(int* counters, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) counters[i] = 0;
}

enum class Ws { Caller, Static };

static int paged_decode(const void* q, void* out, int q_dtype, const void* k_pool, const void* v_pool,
                        int kv_dtype, const void* k_scale, const void* v_scale, int scale_dtype,
                        const int32_t* block_tables, int table_stride, const int32_t* context_lens,
                        int num_seqs, int q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                        int block_size, int num_blocks, int max_context_len, float sm_scale,
                        int part_tokens, void* workspace, size_t workspace_bytes, Ws ws_kind,
                        hipStream_t stream) {
  if (num_seqs == 0) return HPA_OK;
  if (!q || !out || !k_pool || !v_pool || !block_tables || !context_lens)
    return fail(HPA_ERR_ARG, "hpa_paged_decode: null pointer argument");
  if (num_seqs < 0 || q_per_seq <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads || num_blocks <= 0 || table_stride <= 0 || max_context_len < 0)
    return fail(HPA_ERR_ARG,
                "hpa_paged_decode: bad shape (seqs %d, q/seq %d, Hq %d, Hkv %d, blocks %d, stride %d)",
                num_seqs, q_per_seq, num_q_heads, num_kv_heads, num_blocks, table_stride);
  const int bsl = ilog2_exact(block_size);
  if (bsl < 2 || bsl > 10)
    return fail(HPA_ERR_UNSUPPORTED, "hpa_paged_decode: block_size %d must be a power of two in [4, 1024]",
                block_size);
  if (kv_dtype == HPA_I8 && (!k_scale || !v_scale))
    return fail(HPA_ERR_ARG, "hpa_paged_decode: int8 KV needs k_scale and v_scale");
  const int group = num_q_heads / num_kv_heads;
  const int rows = group * q_per_seq;
  const int nt = decode_nt(rows);
  if (nt != 1) {
    // More than 16 query rows per KV head (a wide speculative verify).  With
    // fp16 or bf16 queries over an int8 pool, 17-64 rows run on the verify
    // kernel that dequantises in registers.  Over fp16 / bf16 pools, and for
    // other shapes above 32 rows, the MFMA prefill kernel (fp16 / bf16
    // queries, head_dim 64 / 128, block_size >= 16) runs the verify, about
    // twice as fast as the decode kernel's two and four row tiles; past 64
    // rows, which the decode kernel does not take, shapes the MFMA kernel does
    // not take run on the generic prefill kernel.  Both prefill kernels
    // compute the same causal rule as hpa_paged_prefill over the same tokens,
    // in a mode where sequence b's tokens are [b q_per_seq, (b + 1) q_per_seq)
    // and end at its context; no workspace is used.  Up to 64 rows, shapes no
    // other kernel takes run on the decode kernel.
    PrefillArgs pa;
    pa.q = q;
    pa.out = out;
    pa.k = k_pool;
    pa.v = v_pool;
    pa.ks = k_scale;
    pa.vs = v_scale;
    pa.tables = block_tables;
    pa.table_stride = table_stride;
    pa.cu_q = nullptr;
    pa.q_pos = nullptr;
    pa.ctx_lens = context_lens;
    pa.num_seqs = num_seqs;
    pa.num_tokens = num_seqs * q_per_seq;
    pa.num_q_heads = num_q_heads;
    pa.num_kv_heads = num_kv_heads;
    pa.group = group;
    pa.bs_log2 = bsl;
    pa.num_blocks = num_blocks;
    pa.scale_log2 = sm_scale * 1.4426950408889634f;
    pa.uniform_q = q_per_seq;
    // The int8 verify kernel may cut long units in two; the pieces use the
    // caller's workspace (its counter region, then piece slots), when given.
    if (ws_kind == Ws::Caller && workspace && workspace_bytes > kCounterBytes &&
        (long)num_seqs * num_kv_heads <= kMaxUnits) {
      pa.counters = reinterpret_cast<int*>(workspace);
      pa.pieces = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + kCounterBytes);
      pa.piece_slots = (int)std::min<size_t>((workspace_bytes - kCounterBytes) / (sizeof(float) * kViSlotFloats),
                                             (size_t)1 << 20);
    }
    if (nt != 0 && launch_verify_i8(pa, q_dtype, kv_dtype, scale_dtype, head_dim, stream))
      return check_launch("hpa_paged_decode");
    if ((nt != 2 || kv_dtype != HPA_I8) &&
        launch_prefill_mfma(pa, q_dtype, kv_dtype, scale_dtype, head_dim, q_per_seq, stream))
      return check_launch("hpa_paged_decode");
    if (nt == 0) {
      const int st = launch_prefill_generic(pa, q_dtype, kv_dtype, scale_dtype, head_dim, q_per_seq, stream);
      if (st != HPA_OK) return st;
      return check_launch("hpa_paged_decode");
    }
  }
  DecodeFn fn = pick_decode(q_dtype, kv_dtype, scale_dtype, head_dim, nt);
  if (!fn)
    return fail(HPA_ERR_UNSUPPORTED, "hpa_paged_decode: no kernel for q dtype %d, kv dtype %d, scale dtype %d, head_dim %d",
                q_dtype, kv_dtype, scale_dtype, head_dim);
  const DecodePlan p = plan_decode(num_seqs, num_kv_heads, max_context_len, part_tokens);
  if ((long)num_seqs * num_kv_heads > kMaxUnits)
    return fail(HPA_ERR_UNSUPPORTED, "hpa_paged_decode: %d sequences x %d KV heads exceed %ld",
                num_seqs, num_kv_heads, kMaxUnits);
  const size_t need = ws_bytes(p.waves, rows, head_dim);
  if (ws_kind == Ws::Static) {
    if (need > kScratchBytes)
      return fail(HPA_ERR_WORKSPACE,
                  "hpa_paged_decode_noalloc: these shapes need %zu bytes of workspace, the static scratch "
                  "holds %zu; use hpa_paged_decode with a caller-owned workspace",
                  need, kScratchBytes);
    if (need) {
      const int st = scratch_address(&workspace);
      if (st != HPA_OK) return st;
      workspace_bytes = kScratchBytes;
      // the counters this call uses start at zero, whatever an earlier call
      // that did not complete left there
      const int units = num_seqs * num_kv_heads;
      hipLaunchKernelGGL(clear_counters_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, stream,
                         reinterpret_cast<int*>(workspace), units);
      const int cl = check_launch("hpa_paged_decode_noalloc");
      if (cl != HPA_OK) return cl;
    }
  }
  if (need > workspace_bytes || (need && !workspace))
    return fail(HPA_ERR_WORKSPACE, "hpa_paged_decode: workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);

  DecodeArgs a;
  a.q = q;
  a.out = out;
  a.k = k_pool;
  a.v = v_pool;
  a.ks = k_scale;
  a.vs = v_scale;
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.ctx_lens = context_lens;
  a.num_seqs = num_seqs;
  a.q_per_seq = q_per_seq;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.rows = rows;
  a.bs_log2 = bsl;
  a.num_blocks = num_blocks;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.num_waves = p.waves;
  a.min_steps = p.min_steps;
  // with one wave every unit is whole and the workspace is never touched
  char* ws = reinterpret_cast<char*>(workspace);
  a.counters = need ? reinterpret_cast<int*>(ws) : nullptr;
  a.ws_ml = need ? reinterpret_cast<float*>(ws + kCounterBytes) : nullptr;
  a.ws_o = need ? a.ws_ml + (size_t)p.waves * 2 * rows * 2 : nullptr;
  // workspace offsets follow the cap; the launcher may run fewer waves
  return fn(a, p.waves, stream);
}

}  // namespace hpa

extern "C" int hpa_paged_decode(const void* q, void* out, int q_dtype, const void* k_pool,
                                const void* v_pool, int kv_dtype, const void* k_scale,
                                const void* v_scale, int scale_dtype, const int32_t* block_tables,
                                int table_stride, const int32_t* context_lens, int num_seqs,
                                int q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                                int block_size, int num_blocks, int max_context_len,
                                float sm_scale, int part_tokens, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  return paged_decode(q, out, q_dtype, k_pool, v_pool, kv_dtype, k_scale, v_scale, scale_dtype, block_tables,
                      table_stride, context_lens, num_seqs, q_per_seq, num_q_heads, num_kv_heads, head_dim,
                      block_size, num_blocks, max_context_len, sm_scale, part_tokens, workspace,
                      workspace_bytes, Ws::Caller, stream);
}

extern "C" int hpa_paged_decode_noalloc(const void* q, void* out, int q_dtype, const void* k_pool,
                                        const void* v_pool, int kv_dtype, const void* k_scale,
                                        const void* v_scale, int scale_dtype, const int32_t* block_tables,
                                        int table_stride, const int32_t* context_lens, int num_seqs,
                                        int q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                                        int block_size, int num_blocks, int max_context_len,
                                        float sm_scale, int part_tokens, hipStream_t stream) {
  return paged_decode(q, out, q_dtype, k_pool, v_pool, kv_dtype, k_scale, v_scale, scale_dtype, block_tables,
                      table_stride, context_lens, num_seqs, q_per_seq, num_q_heads, num_kv_heads, head_dim,
                      block_size, num_blocks, max_context_len, sm_scale, part_tokens, nullptr, 0, Ws::Static,
                      stream);
}
