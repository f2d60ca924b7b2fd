// KV-cache data movement for gfx950: scatter write (fp copy or fused int8
// quantize), gather (with int8 dequantisation) and batched block copies.
//
//  * hpa_kv_write replaces PagedKVCache.write (exec/paged_attn.py:57-85) and
//    QuantizedPagedKVCache.write (paged_attn.py:185-211) -- a Python loop of
//    2-4 indexed assignments per token -- with one launch over a ragged batch.
//    Position p of sequence b lands in block table[b][p / bs], offset p % bs.
//    The int8 path reproduces QuantizedPagedKVCache._quantize
//    (paged_attn.py:177-183) bit for bit: absmax over head_dim in fp32,
//    clamped to >= 1e-8, s = absmax / 127 (IEEE division), q = round-half-even
//    (x / s) (IEEE division per element) clamped to [-127, 127], and the scale
//    stored as fp16 (round to nearest even) or, optionally, fp32.
//  * hpa_kv_gather replaces PagedKVCache.gather / QuantizedPagedKVCache.gather
//    (paged_attn.py:87-110, 213-235): dequantised value = fp32(q) * fp32(s),
//    then rounded to the output dtype.
//  * hpa_copy_blocks replaces the per-layer, per-pair copy_block calls of the
//    runner's copy-on-write / swap step (exec/runner.py:155-165,
//    paged_attn.py:112-115, 237-245), scales included, in one launch.
#include "hpa_host.h"
#include "hpa_types.h"

namespace hpa {

struct WriteArgs {
  const void* k;
  const void* v;
  void* kp;
  void* vp;
  void* ks;
  void* vs;
  const int32_t* tables;
  int table_stride;
  const int32_t* cu_tokens;
  const int32_t* start_pos;
  int num_kv_heads, head_dim, bs_log2, num_blocks;
  // optional rotary tables [rope_rows][head_dim / 2] (fp32); K is rotated by
  // its write position when rope_cos is set
  const float* rope_cos;
  const float* rope_sin;
  int rope_rows;
};

// Element d of K rotated rotate-half style at position pos (reference
// exec/model.py:135-153): with c, s = cos/sin[pos][d mod D/2],
//   d <  D/2: x[d] c - x[d + D/2] s       d >= D/2: x[d] c + x[d - D/2] s
// Each product and the sum are rounded to fp32 separately, as torch's
// separate elementwise ops round them: contraction into a fused multiply-add
// (which HIP allows by default, also through __fmul_rn) is switched off here.
template <class IT>
__device__ __forceinline__ float rope_elem(const typename IT::storage* x, int d, int D, const float* cs_row,
                                           const float* sn_row) {
#pragma clang fp contract(off)
  const int half = D >> 1;
  const int j = d < half ? d : d - half;
  const float c = cs_row[j], sn = sn_row[j];
  const float xd = Cvt<IT>::to_f32(x[d]);
  if (d < half) {
    const float xo = Cvt<IT>::to_f32(x[d + half]);
    return xd * c - xo * sn;
  }
  const float xo = Cvt<IT>::to_f32(x[d - half]);
  return xd * c + xo * sn;
}

__device__ __forceinline__ long write_slot(const WriteArgs& a, int b, int i, int h) {
  const int pos = a.start_pos[b] + i;
  if (pos < 0) return -1;
  if (a.rope_cos && pos >= a.rope_rows) return -1;  // no rotary row for it
  const int lb = pos >> a.bs_log2;
  if (lb >= a.table_stride) return -1;
  const int phys = a.tables[(long)b * a.table_stride + lb];
  if ((unsigned)phys >= (unsigned)a.num_blocks) return -1;
  return ((long)(phys * a.num_kv_heads + h) << a.bs_log2) + (pos & ((1 << a.bs_log2) - 1));
}

// fp pool: one thread per element, converting the input dtype to the pool's.
template <class IT, class PT>
__global__ __launch_bounds__(256) void kv_write_fp_kernel(const WriteArgs a, int max_tokens) {
  const int b = blockIdx.y;
  const int t0 = a.cu_tokens[b], nt = a.cu_tokens[b + 1] - t0;
  const int D = a.head_dim, H = a.num_kv_heads;
  const long per_tok = (long)H * D;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < (long)nt * per_tok;
       e += (long)gridDim.x * blockDim.x) {
    const int i = (int)(e / per_tok);
    const int rem = (int)(e - (long)i * per_tok);
    const int h = rem / D, d = rem - h * D;
    const long slot = write_slot(a, b, i, h);
    if (slot < 0) continue;
    const long src = (long)(t0 + i) * per_tok + rem;
    typedef typename IT::storage i_t;
    typedef typename PT::storage p_t;
    float kx;
    if (a.rope_cos) {
      const long row = (long)(a.start_pos[b] + i) * (D >> 1);
      kx = rope_elem<IT>(reinterpret_cast<const i_t*>(a.k) + (src - d), d, D, a.rope_cos + row, a.rope_sin + row);
    } else {
      kx = Cvt<IT>::to_f32(reinterpret_cast<const i_t*>(a.k)[src]);
    }
    const float vx = Cvt<IT>::to_f32(reinterpret_cast<const i_t*>(a.v)[src]);
    reinterpret_cast<p_t*>(a.kp)[slot * D + d] = Cvt<PT>::from_f32(kx);
    reinterpret_cast<p_t*>(a.vp)[slot * D + d] = Cvt<PT>::from_f32(vx);
  }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

// int8 pool: one wave per (token, KV head) and tensor (K or V).  Lane l owns
// head_dim elements [l*EPL, l*EPL + EPL).
// One (token, head) row into registers: the lane's EPL values, rotated when
// cs_row is given.
template <class IT, int EPL>
__device__ __forceinline__ void load_row(const typename IT::storage* x, int D, const float* cs_row,
                                         const float* sn_row, float* v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int d = lane * EPL + e;
    v[e] = d < D ? (cs_row ? rope_elem<IT>(x, d, D, cs_row, sn_row) : Cvt<IT>::to_f32(x[d])) : 0.f;
  }
}

// helios' _quantize of one row held in registers, stored at qdst / sdst
template <class ST, int EPL>
__device__ __forceinline__ void quant_store(const float* v, int8_t* qdst, typename ST::storage* sdst, int D) {
  const int lane = threadIdx.x & 63;
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = wave_max(amax);
  const float s = fmaxf(amax, 1e-8f) / 127.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const int d = lane * EPL + e;
    if (d < D) {
      float r = rintf(v[e] / s);
      r = fminf(fmaxf(r, -127.f), 127.f);
      qdst[d] = (int8_t)(int)r;
    }
  }
  if (lane == 0) {
    if constexpr (std::is_same<ST, F16>::value) {
      *sdst = (uint16_t)f32_to_f16_bits(s);
    } else {
      *sdst = s;
    }
  }
}

template <class IT, class ST, int EPL>
__global__ __launch_bounds__(256) void kv_write_i8_kernel(const WriteArgs a) {
  const int b = blockIdx.y;
  const int t0 = a.cu_tokens[b], nt = a.cu_tokens[b + 1] - t0;
  const int H = a.num_kv_heads, D = a.head_dim;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);  // (token, head)
  if (item >= nt * H) return;
  const int i = item / H, h = item - i * H;
  typedef typename IT::storage i_t;
  typedef typename ST::storage s_t;
  // the rows are read before the slot is known, so these loads and the
  // block-table read are in flight together; a row whose slot turns out
  // invalid is dropped (its rotary rows are read only when they exist)
  const long src = ((long)(t0 + i) * H + h) * D;
  const int pos = a.start_pos[b] + i;
  const bool rot = a.rope_cos != nullptr && pos >= 0 && pos < a.rope_rows;
  const long row = (long)pos * (D >> 1);
  float kx[EPL], vx[EPL];
  load_row<IT, EPL>(reinterpret_cast<const i_t*>(a.k) + src, D, rot ? a.rope_cos + row : nullptr,
                    rot ? a.rope_sin + row : nullptr, kx);
  load_row<IT, EPL>(reinterpret_cast<const i_t*>(a.v) + src, D, nullptr, nullptr, vx);
  const long slot = write_slot(a, b, i, h);
  if (slot < 0) return;
  quant_store<ST, EPL>(kx, reinterpret_cast<int8_t*>(a.kp) + slot * D, reinterpret_cast<s_t*>(a.ks) + slot, D);
  quant_store<ST, EPL>(vx, reinterpret_cast<int8_t*>(a.vp) + slot * D, reinterpret_cast<s_t*>(a.vs) + slot, D);
}

// ------------------------------------------------------------------- gather
struct GatherArgs {
  const void* kp;
  const void* vp;
  const void* ks;
  const void* vs;
  void* ko;
  void* vo;
  const int32_t* table;
  int ctx, num_kv_heads, head_dim, bs_log2, num_blocks;
};

template <class PT, class ST, class OT>
__global__ __launch_bounds__(256) void kv_gather_kernel(const GatherArgs a) {
  const int D = a.head_dim, H = a.num_kv_heads;
  const long total = (long)a.ctx * H * D;
  typedef typename OT::storage o_t;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (long)gridDim.x * blockDim.x) {
    const int tok = (int)(e / ((long)H * D));
    const int rem = (int)(e - (long)tok * H * D);
    const int h = rem / D, d = rem - h * D;
    int phys = a.table[tok >> a.bs_log2];
    phys = (unsigned)phys < (unsigned)a.num_blocks ? phys : 0;
    const long slot = ((long)(phys * H + h) << a.bs_log2) + (tok & ((1 << a.bs_log2) - 1));
    float kx, vx;
    if constexpr (std::is_same<PT, I8>::value) {
      typedef typename ST::storage s_t;
      const float sk = Cvt<ST>::to_f32(reinterpret_cast<const s_t*>(a.ks)[slot]);
      const float sv = Cvt<ST>::to_f32(reinterpret_cast<const s_t*>(a.vs)[slot]);
      // helios rounds the product to fp32, then to the output dtype: the
      // empty asm keeps the compiler from fusing the two roundings into one
      // mixed-precision multiply (with fp32 scales the product is not exact)
      kx = (float)reinterpret_cast<const int8_t*>(a.kp)[slot * D + d] * sk;
      vx = (float)reinterpret_cast<const int8_t*>(a.vp)[slot * D + d] * sv;
      asm volatile("" : "+v"(kx), "+v"(vx));
    } else {
      typedef typename PT::storage p_t;
      kx = Cvt<PT>::to_f32(reinterpret_cast<const p_t*>(a.kp)[slot * D + d]);
      vx = Cvt<PT>::to_f32(reinterpret_cast<const p_t*>(a.vp)[slot * D + d]);
    }
    reinterpret_cast<o_t*>(a.ko)[e] = Cvt<OT>::from_f32(kx);
    reinterpret_cast<o_t*>(a.vo)[e] = Cvt<OT>::from_f32(vx);
  }
}

// -------------------------------------------------------------- block copies
// grid: (pairs, layers, 4 tensors).  Tensor 2/3 are the scales (skipped when
// the layer pointer is null).
__global__ __launch_bounds__(256) void copy_blocks_kernel(void* const* kp, void* const* vp,
                                                          void* const* ksp, void* const* vsp,
                                                          const int32_t* pairs, int num_blocks,
                                                          long block_bytes, long scale_bytes) {
  const int pr = blockIdx.x, layer = blockIdx.y, which = blockIdx.z;
  void* base = which == 0 ? kp[layer] : which == 1 ? vp[layer] : which == 2 ? (ksp ? ksp[layer] : nullptr)
                                                                            : (vsp ? vsp[layer] : nullptr);
  if (!base) return;
  const long nbytes = which < 2 ? block_bytes : scale_bytes;
  if (nbytes <= 0) return;
  const int src = pairs[2 * pr], dst = pairs[2 * pr + 1];
  if ((unsigned)src >= (unsigned)num_blocks || (unsigned)dst >= (unsigned)num_blocks || src == dst) return;
  char* s = reinterpret_cast<char*>(base) + (long)src * nbytes;
  char* d = reinterpret_cast<char*>(base) + (long)dst * nbytes;
  if ((nbytes & 15) == 0) {
    const long n16 = nbytes >> 4;
    for (long i = threadIdx.x; i < n16; i += blockDim.x)
      reinterpret_cast<u32x4*>(d)[i] = reinterpret_cast<const u32x4*>(s)[i];
  } else {
    for (long i = threadIdx.x; i < nbytes; i += blockDim.x) d[i] = s[i];
  }
}

// ------------------------------------------------------------------ dispatch
template <class IT>
static int launch_write_input(const WriteArgs& a, int pool_dtype, int scale_dtype, int num_seqs,
                              int max_tokens, hipStream_t s) {
  if (pool_dtype == HPA_I8) {
    const int items = max_tokens * a.num_kv_heads;
    dim3 grid((unsigned)((items + 3) / 4), (unsigned)num_seqs);
    const int D = a.head_dim;
    const int epl = D <= 64 ? 1 : D <= 128 ? 2 : D <= 256 ? 4 : 0;
    if (!epl) return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_write: head_dim %d > 256 for int8", D);
    if (scale_dtype == HPA_F16) {
      if (epl == 1) hipLaunchKernelGGL((kv_write_i8_kernel<IT, F16, 1>), grid, dim3(256), 0, s, a);
      else if (epl == 2) hipLaunchKernelGGL((kv_write_i8_kernel<IT, F16, 2>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((kv_write_i8_kernel<IT, F16, 4>), grid, dim3(256), 0, s, a);
    } else if (scale_dtype == HPA_F32) {
      if (epl == 1) hipLaunchKernelGGL((kv_write_i8_kernel<IT, F32, 1>), grid, dim3(256), 0, s, a);
      else if (epl == 2) hipLaunchKernelGGL((kv_write_i8_kernel<IT, F32, 2>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((kv_write_i8_kernel<IT, F32, 4>), grid, dim3(256), 0, s, a);
    } else {
      return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_write: scale dtype %d", scale_dtype);
    }
    return check_launch("hpa_kv_write (int8)");
  }
  const long elems = (long)max_tokens * a.num_kv_heads * a.head_dim;
  long blocks = (elems + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  dim3 grid((unsigned)(blocks > 0 ? blocks : 1), (unsigned)num_seqs);
  switch (pool_dtype) {
    case HPA_F32: hipLaunchKernelGGL((kv_write_fp_kernel<IT, F32>), grid, dim3(256), 0, s, a, max_tokens); break;
    case HPA_F16: hipLaunchKernelGGL((kv_write_fp_kernel<IT, F16>), grid, dim3(256), 0, s, a, max_tokens); break;
    case HPA_BF16: hipLaunchKernelGGL((kv_write_fp_kernel<IT, BF16>), grid, dim3(256), 0, s, a, max_tokens); break;
    default: return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_write: pool dtype %d", pool_dtype);
  }
  return check_launch("hpa_kv_write");
}

template <class PT, class ST>
static int launch_gather_out(const GatherArgs& a, int out_dtype, hipStream_t s) {
  const long total = (long)a.ctx * a.num_kv_heads * a.head_dim;
  long blocks = (total + 255) / 256;
  if (blocks > 65535) blocks = 65535;
  dim3 grid((unsigned)(blocks > 0 ? blocks : 1));
  switch (out_dtype) {
    case HPA_F32: hipLaunchKernelGGL((kv_gather_kernel<PT, ST, F32>), grid, dim3(256), 0, s, a); break;
    case HPA_F16: hipLaunchKernelGGL((kv_gather_kernel<PT, ST, F16>), grid, dim3(256), 0, s, a); break;
    case HPA_BF16: hipLaunchKernelGGL((kv_gather_kernel<PT, ST, BF16>), grid, dim3(256), 0, s, a); break;
    default: return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_gather: output dtype %d", out_dtype);
  }
  return check_launch("hpa_kv_gather");
}

}  // namespace hpa

using namespace hpa;

static int kv_write_impl(const char* who, const void* k, const void* v, int in_dtype, void* k_pool,
                         void* v_pool, int pool_dtype, void* k_scale, void* v_scale, int scale_dtype,
                         const int32_t* block_tables, int table_stride, const int32_t* cu_tokens,
                         const int32_t* start_positions, int num_seqs, int max_tokens, int num_kv_heads,
                         int head_dim, int block_size, int num_blocks, const float* rope_cos,
                         const float* rope_sin, int rope_rows, hipStream_t stream) {
  if (num_seqs == 0 || max_tokens == 0) return HPA_OK;
  if (!k || !v || !k_pool || !v_pool || !block_tables || !cu_tokens || !start_positions)
    return fail(HPA_ERR_ARG, "%s: null pointer argument", who);
  if (rope_cos && (!rope_sin || rope_rows <= 0 || (head_dim & 1)))
    return fail(HPA_ERR_ARG, "%s: rotary tables need sin, rows > 0 and an even head_dim", who);
  if (num_seqs < 0 || max_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || table_stride <= 0 ||
      num_blocks <= 0)
    return fail(HPA_ERR_ARG, "%s: bad shape", who);
  const int bsl = ilog2_exact(block_size);
  if (bsl < 0 || bsl > 10)
    return fail(HPA_ERR_UNSUPPORTED, "%s: block_size %d must be a power of two <= 1024", who, block_size);
  if (pool_dtype == HPA_I8 && (!k_scale || !v_scale))
    return fail(HPA_ERR_ARG, "%s: int8 pool needs k_scale and v_scale", who);
  if (pool_dtype != HPA_I8 && (pool_dtype < HPA_F32 || pool_dtype > HPA_BF16))
    return fail(HPA_ERR_UNSUPPORTED, "%s: pool dtype %d", who, pool_dtype);
  WriteArgs a{k, v, k_pool, v_pool, k_scale, v_scale, block_tables, table_stride, cu_tokens,
              start_positions, num_kv_heads, head_dim, bsl, num_blocks, rope_cos,
              rope_cos ? rope_sin : nullptr, rope_cos ? rope_rows : 0};
  switch (in_dtype) {
    case HPA_F32: return launch_write_input<F32>(a, pool_dtype, scale_dtype, num_seqs, max_tokens, stream);
    case HPA_F16: return launch_write_input<F16>(a, pool_dtype, scale_dtype, num_seqs, max_tokens, stream);
    case HPA_BF16: return launch_write_input<BF16>(a, pool_dtype, scale_dtype, num_seqs, max_tokens, stream);
  }
  return fail(HPA_ERR_UNSUPPORTED, "%s: input dtype %d", who, in_dtype);
}

extern "C" int hpa_kv_write(const void* k, const void* v, int in_dtype, void* k_pool, void* v_pool,
                            int pool_dtype, void* k_scale, void* v_scale, int scale_dtype,
                            const int32_t* block_tables, int table_stride,
                            const int32_t* cu_tokens, const int32_t* start_positions, int num_seqs,
                            int max_tokens, int num_kv_heads, int head_dim, int block_size,
                            int num_blocks, hipStream_t stream) {
  return kv_write_impl("hpa_kv_write", k, v, in_dtype, k_pool, v_pool, pool_dtype, k_scale, v_scale,
                       scale_dtype, block_tables, table_stride, cu_tokens, start_positions, num_seqs,
                       max_tokens, num_kv_heads, head_dim, block_size, num_blocks, nullptr, nullptr, 0,
                       stream);
}

extern "C" int hpa_kv_write_rope(const void* k, const void* v, int in_dtype, void* k_pool, void* v_pool,
                                 int pool_dtype, void* k_scale, void* v_scale, int scale_dtype,
                                 const int32_t* block_tables, int table_stride,
                                 const int32_t* cu_tokens, const int32_t* start_positions, int num_seqs,
                                 int max_tokens, int num_kv_heads, int head_dim, int block_size,
                                 int num_blocks, const float* rope_cos, const float* rope_sin,
                                 int rope_rows, hipStream_t stream) {
  if (!rope_cos || !rope_sin) return fail(HPA_ERR_ARG, "hpa_kv_write_rope: null rotary table");
  return kv_write_impl("hpa_kv_write_rope", k, v, in_dtype, k_pool, v_pool, pool_dtype, k_scale, v_scale,
                       scale_dtype, block_tables, table_stride, cu_tokens, start_positions, num_seqs,
                       max_tokens, num_kv_heads, head_dim, block_size, num_blocks, rope_cos, rope_sin,
                       rope_rows, stream);
}

extern "C" int hpa_kv_gather(const void* k_pool, const void* v_pool, int pool_dtype,
                             const void* k_scale, const void* v_scale, int scale_dtype,
                             const int32_t* block_table, int context_len, void* k_out, void* v_out,
                             int out_dtype, int num_kv_heads, int head_dim, int block_size,
                             int num_blocks, hipStream_t stream) {
  if (context_len <= 0) return HPA_OK;
  if (!k_pool || !v_pool || !block_table || !k_out || !v_out)
    return fail(HPA_ERR_ARG, "hpa_kv_gather: null pointer argument");
  if (num_kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0)
    return fail(HPA_ERR_ARG, "hpa_kv_gather: bad shape");
  const int bsl = ilog2_exact(block_size);
  if (bsl < 0 || bsl > 10)
    return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_gather: block_size %d must be a power of two <= 1024",
                block_size);
  GatherArgs a{k_pool, v_pool, k_scale, v_scale, k_out, v_out, block_table, context_len,
               num_kv_heads, head_dim, bsl, num_blocks};
  switch (pool_dtype) {
    case HPA_F32: return launch_gather_out<F32, F32>(a, out_dtype, stream);
    case HPA_F16: return launch_gather_out<F16, F32>(a, out_dtype, stream);
    case HPA_BF16: return launch_gather_out<BF16, F32>(a, out_dtype, stream);
    case HPA_I8:
      if (!k_scale || !v_scale) return fail(HPA_ERR_ARG, "hpa_kv_gather: int8 pool needs scales");
      if (scale_dtype == HPA_F16) return launch_gather_out<I8, F16>(a, out_dtype, stream);
      if (scale_dtype == HPA_F32) return launch_gather_out<I8, F32>(a, out_dtype, stream);
      return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_gather: scale dtype %d", scale_dtype);
  }
  return fail(HPA_ERR_UNSUPPORTED, "hpa_kv_gather: pool dtype %d", pool_dtype);
}

extern "C" int hpa_copy_blocks(void* const* k_pools, void* const* v_pools, void* const* k_scales,
                               void* const* v_scales, int num_layers, const int32_t* pairs,
                               int num_pairs, int num_blocks, size_t block_bytes,
                               size_t scale_block_bytes, hipStream_t stream) {
  if (num_pairs == 0 || num_layers == 0) return HPA_OK;
  if (!k_pools || !v_pools || !pairs) return fail(HPA_ERR_ARG, "hpa_copy_blocks: null pointer argument");
  if (num_pairs < 0 || num_layers < 0 || num_blocks <= 0 || num_pairs > 65535 || num_layers > 65535)
    return fail(HPA_ERR_ARG, "hpa_copy_blocks: bad shape (pairs %d, layers %d)", num_pairs, num_layers);
  dim3 grid((unsigned)num_pairs, (unsigned)num_layers, (k_scales || v_scales) ? 4u : 2u);
  hipLaunchKernelGGL(copy_blocks_kernel, grid, dim3(256), 0, stream, k_pools, v_pools, k_scales,
                     v_scales, pairs, num_blocks, (long)block_bytes, (long)scale_block_bytes);
  return check_launch("hpa_copy_blocks");
}
