// Paged decode / speculative-verify attention for gfx950.
//
// Replaces helios' paged_attention_decode_batched (exec/paged_attn.py:298-353)
// and the Triton kernel (exec/triton_attn.py:54-130).  Every sequence carries
// q_per_seq query tokens (1 for decode, gamma+1 for verify); token t of a
// sequence with context c sits at position c - q_per_seq + t and attends keys
// [0, c - q_per_seq + t], which is helios' prefill mask (paged_attn.py:401-404)
// with start_pos = c - q_per_seq.
//
// Work decomposition: one workgroup of NW waves per (sequence, KV head,
// context partition).  All G * q_per_seq query rows of the KV head live in
// every wave (GQA packing), the waves take interleaved 32-key steps of the
// partition, and merge their online-softmax states through LDS.  A sequence
// with one partition writes its output directly; longer ones write
// (O, m, l) partials that hpa_decode_reduce merges in a fixed order, so the
// result does not depend on scheduling.
#include <algorithm>

#include "hpa_attn_core.h"
#include "hpa_host.h"

namespace hpa {

struct DecodeArgs {
  const void* q;
  void* out;
  const void* k;
  const void* v;
  const void* ks;
  const void* vs;
  const int32_t* tables;
  int table_stride;
  const int32_t* ctx_lens;
  int num_seqs, q_per_seq, num_q_heads, num_kv_heads, group, rows;
  int bs_log2, num_blocks;
  float scale_log2;
  int part_tokens, max_parts;
  int ctx_cap;   // max_parts * part_tokens: contexts are clamped here
  float* ws_o;   // [num_seqs * Hkv * max_parts, rows, D]
  float* ws_ml;  // [num_seqs * Hkv * max_parts, rows, 2]
};

constexpr int kDecodeWaves = 4;
constexpr int kMaxParts = 512;

template <class CT, class KVT, class ST, int D, int NT, int NW>
__global__ __launch_bounds__(64 * NW) void decode_kernel(const DecodeArgs a) {
  typedef AttnCore<CT, KVT, ST, D, NT> Core;
  typedef typename CT::storage q_t;
  constexpr int DS = D + 4;  // padded LDS row
  __shared__ float sm_o[NW * 16 * DS];
  __shared__ float sm_m[NW * 16];
  __shared__ float sm_l[NW * 16];

  const int kvh = blockIdx.x % a.num_kv_heads;
  const int b = blockIdx.x / a.num_kv_heads;
  const int part = blockIdx.y;
  const int ctx = min(a.ctx_lens[b], a.ctx_cap);
  const int kbeg = part * a.part_tokens;
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = a.group, Tq = a.q_per_seq;
  q_t* out = reinterpret_cast<q_t*>(a.out);
  const q_t* q = reinterpret_cast<const q_t*>(a.q);

  auto out_row = [&](int r) -> q_t* {
    const int t = r / G, hh = r - t * G;
    return out + ((long)(b * Tq + t) * a.num_q_heads + kvh * G + hh) * D;
  };

  if (ctx <= 0) {
    // helios' softmax over an empty context is NaN (all -inf); this build
    // defines the output as zeros.
    if (part == 0)
      for (int idx = threadIdx.x; idx < a.rows * D; idx += 64 * NW)
        out_row(idx / D)[idx % D] = Cvt<CT>::from_f32(0.f);
    return;
  }
  if (kbeg >= ctx) return;
  const int kend = min(ctx, kbeg + a.part_tokens);
  const int nparts = (ctx + a.part_tokens - 1) / a.part_tokens;

  const q_t* rowq[NT];
  int rowlim[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r = nt * 16 + n;
    if (r < a.rows) {
      const int t = r / G, hh = r - t * G;
      rowq[nt] = q + ((long)(b * Tq + t) * a.num_q_heads + kvh * G + hh) * D;
      rowlim[nt] = min(max(ctx - Tq + t + 1, 0), kend);
    } else {
      rowq[nt] = nullptr;
      rowlim[nt] = kend;
    }
  }
  const int minlim = min(max(ctx - Tq + 1, 0), kend);

  Core core;
  core.init(rowq, rowlim);
  PoolView pv{a.k, a.v, a.ks, a.vs, a.tables + (long)b * a.table_stride, a.table_stride, kvh,
              a.num_kv_heads,
              a.bs_log2, a.num_blocks, ctx};

  const typename Core::LaneOff lo = Core::lane_off();
  int k0 = kbeg + 32 * w;
  if (k0 < kend) {
    typename Core::Raw cur;
    Core::load_any(pv, k0, lo, cur);
    for (;;) {
      const int kn = k0 + 32 * NW;
      typename Core::Raw nxt;
      if (kn < kend) Core::load_any(pv, kn, lo, nxt);
      core.compute(cur, k0, a.scale_log2, k0 + 32 > minlim, ctx);
      if (kn >= kend) break;
      cur = nxt;
      k0 = kn;
    }
  }

  // ---- merge the NW waves' states, one 16-row tile at a time
  const long unit = (long)b * a.num_kv_heads + kvh;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float lt = core.row_l(nt);
    if (g == 0) {
      sm_m[w * 16 + n] = core.m[nt];
      sm_l[w * 16 + n] = lt;
    }
#pragma unroll
    for (int j = 0; j < Core::J; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = Core::out_dim(g, j, i);
        if (d < D) sm_o[(w * 16 + n) * DS + d] = core.out_val(nt, j, i);
      }
    __syncthreads();
    for (int idx = threadIdx.x; idx < 16 * D; idx += 64 * NW) {
      const int rr = idx / D, d = idx - rr * D, r = nt * 16 + rr;
      if (r >= a.rows) continue;
      float M = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, sm_m[ww * 16 + rr]);
      const float Mref = M == -INFINITY ? 0.f : M;
      float L = 0.f, O = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float wt = __builtin_amdgcn_exp2f(sm_m[ww * 16 + rr] - Mref);
        L += wt * sm_l[ww * 16 + rr];
        O += wt * sm_o[(ww * 16 + rr) * DS + d];
      }
      if (nparts == 1) {
        out_row(r)[d] = Cvt<CT>::from_f32(L > 0.f ? O / L : 0.f);
      } else {
        const long slot = (unit * a.max_parts + part) * a.rows + r;
        a.ws_o[slot * D + d] = O;
        if (d == 0) {
          a.ws_ml[2 * slot] = M;
          a.ws_ml[2 * slot + 1] = L;
        }
      }
    }
    __syncthreads();
  }
}

// Merges the partition partials of every (sequence, KV head) that has more
// than one partition, in partition order (deterministic).  Rows are handled
// in groups whose weight table fits in LDS: one thread per row computes the
// row's merged max / sum, then all threads combine the partial outputs with
// coalesced reads along head_dim.
constexpr int kReduceLds = 4096;

template <class CT>
__global__ __launch_bounds__(256) void decode_reduce_kernel(const DecodeArgs a, int D) {
  typedef typename CT::storage q_t;
  __shared__ float sw[kReduceLds];
  const int unit = blockIdx.x;
  const int kvh = unit % a.num_kv_heads, b = unit / a.num_kv_heads;
  const int ctx = min(a.ctx_lens[b], a.ctx_cap);
  if (ctx <= 0) return;
  const int nparts = (ctx + a.part_tokens - 1) / a.part_tokens;
  if (nparts <= 1) return;
  const int G = a.group, Tq = a.q_per_seq;
  q_t* out = reinterpret_cast<q_t*>(a.out);
  const float* ml = a.ws_ml + (long)unit * a.max_parts * a.rows * 2;
  const float* po = a.ws_o + (long)unit * a.max_parts * a.rows * D;
  const int rg = max(1, min(a.rows, kReduceLds / nparts));
  for (int r0 = 0; r0 < a.rows; r0 += rg) {
    const int nr = min(rg, a.rows - r0);
    for (int rr = threadIdx.x; rr < nr; rr += 256) {
      const int r = r0 + rr;
      float M = -INFINITY;
      for (int p = 0; p < nparts; ++p) M = fmaxf(M, ml[2 * (p * a.rows + r)]);
      const float Mref = M == -INFINITY ? 0.f : M;
      float L = 0.f;
      for (int p = 0; p < nparts; ++p) {
        const float wt = __builtin_amdgcn_exp2f(ml[2 * (p * a.rows + r)] - Mref);
        sw[p * rg + rr] = wt;
        L += wt * ml[2 * (p * a.rows + r) + 1];
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
      for (int p = 0; p < nparts; ++p) sw[p * rg + rr] *= inv;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * D; idx += 256) {
      const int rr = idx / D, d = idx - rr * D, r = r0 + rr;
      float O = 0.f;
      for (int p = 0; p < nparts; ++p) O += sw[p * rg + rr] * po[((long)p * a.rows + r) * D + d];
      const int t = r / G, hh = r - t * G;
      out[((long)(b * Tq + t) * a.num_q_heads + kvh * G + hh) * D + d] = Cvt<CT>::from_f32(O);
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ dispatch
typedef void (*DecodeFn)(const DecodeArgs&, dim3, hipStream_t);

template <class CT, class KVT, class ST, int D, int NT>
void launch_decode(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((decode_kernel<CT, KVT, ST, D, NT, kDecodeWaves>), grid, dim3(64 * kDecodeWaves),
                     0, s, a);
}

template <class CT, class KVT, class ST, int D>
DecodeFn pick_nt(int nt) {
  switch (nt) {
    case 1: return launch_decode<CT, KVT, ST, D, 1>;
    case 2: return launch_decode<CT, KVT, ST, D, 2>;
    case 4: return launch_decode<CT, KVT, ST, D, 4>;
  }
  return nullptr;
}
template <class CT, class KVT, class ST>
DecodeFn pick_d(int d, int nt) {
  switch (d) {
    case 8: return pick_nt<CT, KVT, ST, 8>(nt);
    case 16: return pick_nt<CT, KVT, ST, 16>(nt);
    case 32: return pick_nt<CT, KVT, ST, 32>(nt);
    case 64: return pick_nt<CT, KVT, ST, 64>(nt);
    case 128: return pick_nt<CT, KVT, ST, 128>(nt);
    case 256: return pick_nt<CT, KVT, ST, 256>(nt);
  }
  return nullptr;
}
template <class CT>
DecodeFn pick_kv(int kv_dtype, int scale_dtype, int d, int nt) {
  if (kv_dtype == HPA_I8) {
    if (scale_dtype == HPA_F16) return pick_d<CT, I8, F16>(d, nt);
    if (scale_dtype == HPA_F32) return pick_d<CT, I8, F32>(d, nt);
    return nullptr;
  }
  if (kv_dtype != CT::code) return nullptr;
  return pick_d<CT, CT, F32>(d, nt);
}

static DecodeFn pick_decode(int q_dtype, int kv_dtype, int scale_dtype, int d, int nt) {
  switch (q_dtype) {
    case HPA_F32: return pick_kv<F32>(kv_dtype, scale_dtype, d, nt);
    case HPA_F16: return pick_kv<F16>(kv_dtype, scale_dtype, d, nt);
    case HPA_BF16: return pick_kv<BF16>(kv_dtype, scale_dtype, d, nt);
  }
  return nullptr;
}

static int decode_nt(int rows) { return rows <= 16 ? 1 : rows <= 32 ? 2 : rows <= 64 ? 4 : 0; }

static int choose_part_tokens(int num_seqs, int num_kv_heads, int max_context_len, int requested) {
  int part = requested > 0 ? requested : (num_seqs * num_kv_heads >= 512 ? 512 : 256);
  part = (part + 32 * kDecodeWaves - 1) / (32 * kDecodeWaves) * (32 * kDecodeWaves);
  while ((max_context_len + part - 1) / part > kMaxParts) part *= 2;
  return part;
}

}  // namespace hpa

using namespace hpa;

extern "C" size_t hpa_decode_workspace_size(int num_seqs, int q_per_seq, int num_q_heads,
                                            int num_kv_heads, int head_dim, int max_context_len,
                                            int part_tokens) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || q_per_seq <= 0 || head_dim <= 0)
    return 0;
  const int part = choose_part_tokens(num_seqs, num_kv_heads, max_context_len, part_tokens);
  const long max_parts = std::max(1, (max_context_len + part - 1) / part);
  if (max_parts <= 1) return 0;
  const long rows = (long)(num_q_heads / num_kv_heads) * q_per_seq;
  const long units = (long)num_seqs * num_kv_heads * max_parts * rows;
  return (size_t)(units * (head_dim + 2) * sizeof(float));
}

extern "C" int hpa_paged_decode(const void* q, void* out, int q_dtype, const void* k_pool,
                                const void* v_pool, int kv_dtype, const void* k_scale,
                                const void* v_scale, int scale_dtype, const int32_t* block_tables,
                                int table_stride, const int32_t* context_lens, int num_seqs,
                                int q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
                                int block_size, int num_blocks, int max_context_len,
                                float sm_scale, int part_tokens, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
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
  if (!nt)
    return fail(HPA_ERR_UNSUPPORTED,
                "hpa_paged_decode: %d query rows per KV head exceed 64; use hpa_paged_prefill", rows);
  DecodeFn fn = pick_decode(q_dtype, kv_dtype, scale_dtype, head_dim, nt);
  if (!fn)
    return fail(HPA_ERR_UNSUPPORTED, "hpa_paged_decode: no kernel for q dtype %d, kv dtype %d, scale dtype %d, head_dim %d",
                q_dtype, kv_dtype, scale_dtype, head_dim);
  const int part = choose_part_tokens(num_seqs, num_kv_heads, max_context_len, part_tokens);
  const int max_parts = std::max(1, (max_context_len + part - 1) / part);
  const size_t need = hpa_decode_workspace_size(num_seqs, q_per_seq, num_q_heads, num_kv_heads,
                                                head_dim, max_context_len, part_tokens);
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
  a.part_tokens = part;
  a.max_parts = max_parts;
  a.ctx_cap = max_parts * part;
  const long ws_units = (long)num_seqs * num_kv_heads * max_parts * rows;
  a.ws_o = reinterpret_cast<float*>(workspace);
  a.ws_ml = need ? a.ws_o + ws_units * head_dim : nullptr;

  dim3 grid((unsigned)(num_seqs * num_kv_heads), (unsigned)max_parts);
  fn(a, grid, stream);
  int st = check_launch("hpa_paged_decode");
  if (st) return st;
  if (max_parts > 1) {
    switch (q_dtype) {
      case HPA_F32:
        hipLaunchKernelGGL(decode_reduce_kernel<F32>, dim3(num_seqs * num_kv_heads), dim3(256), 0, stream, a, head_dim);
        break;
      case HPA_F16:
        hipLaunchKernelGGL(decode_reduce_kernel<F16>, dim3(num_seqs * num_kv_heads), dim3(256), 0, stream, a, head_dim);
        break;
      default:
        hipLaunchKernelGGL(decode_reduce_kernel<BF16>, dim3(num_seqs * num_kv_heads), dim3(256), 0, stream, a, head_dim);
        break;
    }
    st = check_launch("hpa_paged_decode (reduce)");
  }
  return st;
}
