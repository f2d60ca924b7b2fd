// Chunked-prefill / speculative-verify attention over a paged KV cache, gfx950.
//
// Replaces helios' paged_attention_prefill (exec/paged_attn.py:368-408) and
// the per-sequence loop of BatchedAttention.run (exec/model.py:303-317) with
// one launch over a ragged batch.  Sequence b owns query tokens
// [cu_q[b], cu_q[b+1]); its token i sits at absolute position q_pos[b] + i
// and attends keys [0, min(q_pos[b] + i + 1, context_len[b])) -- helios'
// causal mask `k_pos > start_pos + i` (paged_attn.py:401-404) restricted to
// the gathered context (paged_attn.py:391).
//
// A verify launch (uniform_q > 0, from hpa_paged_decode) gives every sequence
// uniform_q tokens ending at context_len[b] - 1 and reads neither cu_q nor
// q_pos.  Tokens at or past num_tokens are never read or written.
//
// Work decomposition: the (token, head-in-group) rows of each (sequence, KV
// head) are cut into tiles of NW * NT * 16 rows, one workgroup per tile; each
// wave owns NT * 16 consecutive rows and streams keys [0, its last row's
// limit) through the shared AttnCore with fp16/bf16 MFMA.  Only the steps
// that cross the causal diagonal pay for element-wise masking.
#include "hpa_attn_core.h"
#include "hpa_host.h"
#include "hpa_prefill.h"

namespace hpa {

constexpr int kPrefillWaves = 4;
constexpr int kPrefillNT = 2;

template <class CT, class KVT, class ST, int D, int NT, int NW, bool BIG>
__global__ __launch_bounds__(64 * NW) void prefill_kernel(const PrefillArgs a) {
  typedef AttnCore<CT, KVT, ST, D, NT> Core;
  typedef typename CT::storage q_t;
  const int b = blockIdx.z, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = a.group;
  const SeqSpan sp = seq_span(a, b);
  const int q0 = sp.q0;
  const int rows = sp.qn * G;
  const int row_base = (blockIdx.x * NW + w) * NT * 16;
  if (row_base >= rows) return;  // this kernel has no barriers
  const int ctx = a.ctx_lens[b];
  const int pos0 = sp.pos0;
  const q_t* q = reinterpret_cast<const q_t*>(a.q);
  q_t* out = reinterpret_cast<q_t*>(a.out);
  auto row_off = [&](int r) -> long {
    const int t = r / G, hh = r - t * G;
    return ((long)(q0 + t) * a.num_q_heads + kvh * G + hh) * D;
  };
  auto limit = [&](int r) -> int { return min(max(pos0 + r / G + 1, 0), max(ctx, 0)); };

  const int last = min(row_base + NT * 16, rows) - 1;
  const int maxlim = limit(last);
  const int minlim = limit(row_base);

  const q_t* rowq[NT];
  int rowlim[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = row_base + nt * 16 + n;
    rowq[nt] = r < rows ? q + row_off(r) : nullptr;
    rowlim[nt] = r < rows ? limit(r) : maxlim;
  }
  Core core;
  core.init(rowq, rowlim);
  PoolView pv{a.k, a.v, a.ks, a.vs, a.tables + (long)b * a.table_stride, a.table_stride, kvh,
              a.num_kv_heads,
              a.bs_log2, a.num_blocks, ctx};

  const typename Core::LaneOff lo = Core::lane_off();
  if (maxlim > 0) {
    TableWindow win;
    if (BIG) win.fill(pv.table, pv.table_stride, 0);
    int k0 = 0;
    typename Core::Raw cur;
    Core::template load_sel<BIG>(pv, win, k0, lo, cur);
    for (;;) {
      const int kn = k0 + 32;
      typename Core::Raw nxt;
      Core::template load_sel<BIG>(pv, win, kn, lo, nxt, kn < maxlim);
      core.compute(cur, k0, a.scale_log2, k0 + 32 > minlim, ctx);
      if (kn >= maxlim) break;
      cur = nxt;
      k0 = kn;
    }
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float lt = core.row_l(nt);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int r = row_base + nt * 16 + n;
    if (r >= rows) continue;
    q_t* orow = out + row_off(r);
#pragma unroll
    for (int j = 0; j < Core::J; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = Core::out_dim(g, j, i);
        if (d < D) orow[d] = Cvt<CT>::from_f32(core.out_val(nt, j, i) * inv);
      }
  }
}

typedef void (*PrefillFn)(const PrefillArgs&, dim3, hipStream_t);

template <class CT, class KVT, class ST, int D>
void launch_prefill(const PrefillArgs& a, dim3 grid, hipStream_t s) {
  if (a.bs_log2 >= 4)
    hipLaunchKernelGGL((prefill_kernel<CT, KVT, ST, D, kPrefillNT, kPrefillWaves, true>), grid,
                       dim3(64 * kPrefillWaves), 0, s, a);
  else
    hipLaunchKernelGGL((prefill_kernel<CT, KVT, ST, D, kPrefillNT, kPrefillWaves, false>), grid,
                       dim3(64 * kPrefillWaves), 0, s, a);
}
template <class CT, class KVT, class ST>
PrefillFn pick_pd(int d) {
  switch (d) {
    case 8: return launch_prefill<CT, KVT, ST, 8>;
    case 16: return launch_prefill<CT, KVT, ST, 16>;
    case 32: return launch_prefill<CT, KVT, ST, 32>;
    case 64: return launch_prefill<CT, KVT, ST, 64>;
    case 128: return launch_prefill<CT, KVT, ST, 128>;
    case 256: return launch_prefill<CT, KVT, ST, 256>;
  }
  return nullptr;
}
template <class CT>
PrefillFn pick_pkv(int kv_dtype, int scale_dtype, int d) {
  if (kv_dtype == HPA_I8) {
    if (scale_dtype == HPA_F16) return pick_pd<CT, I8, F16>(d);
    if (scale_dtype == HPA_F32) return pick_pd<CT, I8, F32>(d);
    return nullptr;
  }
  if (kv_dtype != CT::code) return nullptr;
  return pick_pd<CT, CT, F32>(d);
}
static PrefillFn pick_prefill(int q_dtype, int kv_dtype, int scale_dtype, int d) {
  switch (q_dtype) {
    case HPA_F32: return pick_pkv<F32>(kv_dtype, scale_dtype, d);
    case HPA_F16: return pick_pkv<F16>(kv_dtype, scale_dtype, d);
    case HPA_BF16: return pick_pkv<BF16>(kv_dtype, scale_dtype, d);
  }
  return nullptr;
}

int launch_prefill_generic(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim,
                           int max_q_len, hipStream_t s) {
  PrefillFn fn = pick_prefill(q_dtype, kv_dtype, scale_dtype, head_dim);
  if (!fn)
    return fail(HPA_ERR_UNSUPPORTED,
                "paged prefill: no kernel for q dtype %d, kv dtype %d, scale dtype %d, head_dim %d", q_dtype,
                kv_dtype, scale_dtype, head_dim);
  const long rows = (long)max_q_len * a.group;
  const long per_wg = (long)kPrefillWaves * kPrefillNT * 16;
  const long gx = (rows + per_wg - 1) / per_wg;
  if (gx > 0x7fffffffL || a.num_seqs > 65535 || a.num_kv_heads > 65535)
    return fail(HPA_ERR_UNSUPPORTED, "paged prefill: %d sequences x %ld rows is too large a grid", a.num_seqs,
                rows);
  fn(a, dim3((unsigned)gx, (unsigned)a.num_kv_heads, (unsigned)a.num_seqs), s);
  return HPA_OK;
}

}  // namespace hpa

using namespace hpa;

extern "C" int hpa_paged_prefill(const void* q, void* out, int q_dtype, const void* k_pool,
                                 const void* v_pool, int kv_dtype, const void* k_scale,
                                 const void* v_scale, int scale_dtype,
                                 const int32_t* block_tables, int table_stride,
                                 const int32_t* cu_q_lens, const int32_t* q_positions,
                                 const int32_t* context_lens, int num_seqs, int max_q_len,
                                 int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                                 int block_size, int num_blocks, float sm_scale, hipStream_t stream) {
  if (num_seqs == 0 || max_q_len == 0 || num_tokens == 0) return HPA_OK;
  if (!q || !out || !k_pool || !v_pool || !block_tables || !cu_q_lens || !q_positions ||
      !context_lens)
    return fail(HPA_ERR_ARG, "hpa_paged_prefill: null pointer argument");
  if (num_seqs < 0 || max_q_len < 0 || num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads || num_blocks <= 0 || table_stride <= 0)
    return fail(HPA_ERR_ARG, "hpa_paged_prefill: bad shape (seqs %d, max_q %d, tokens %d, Hq %d, Hkv %d)",
                num_seqs, max_q_len, num_tokens, num_q_heads, num_kv_heads);
  const int bsl = ilog2_exact(block_size);
  if (bsl < 2 || bsl > 10)
    return fail(HPA_ERR_UNSUPPORTED,
                "hpa_paged_prefill: block_size %d must be a power of two in [4, 1024]", block_size);
  if (kv_dtype == HPA_I8 && (!k_scale || !v_scale))
    return fail(HPA_ERR_ARG, "hpa_paged_prefill: int8 KV needs k_scale and v_scale");
  if (!pick_prefill(q_dtype, kv_dtype, scale_dtype, head_dim))
    return fail(HPA_ERR_UNSUPPORTED,
                "hpa_paged_prefill: no kernel for q dtype %d, kv dtype %d, scale dtype %d, head_dim %d",
                q_dtype, kv_dtype, scale_dtype, head_dim);
  PrefillArgs a;
  a.q = q;
  a.out = out;
  a.k = k_pool;
  a.v = v_pool;
  a.ks = k_scale;
  a.vs = v_scale;
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.cu_q = cu_q_lens;
  a.q_pos = q_positions;
  a.ctx_lens = context_lens;
  a.num_seqs = num_seqs;
  a.num_tokens = num_tokens;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  a.bs_log2 = bsl;
  a.num_blocks = num_blocks;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.uniform_q = 0;
  if (launch_prefill_mfma(a, q_dtype, kv_dtype, scale_dtype, head_dim, max_q_len, stream))
    return check_launch("hpa_paged_prefill");
  const int st = launch_prefill_generic(a, q_dtype, kv_dtype, scale_dtype, head_dim, max_q_len, stream);
  if (st != HPA_OK) return st;
  return check_launch("hpa_paged_prefill");
}
