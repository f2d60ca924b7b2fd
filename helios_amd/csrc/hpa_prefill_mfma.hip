// Chunked-prefill / verify attention for fp16 and bf16 pools on gfx950:
// LDS-shared K/V tiles and 32x32x16 MFMAs.
//
// Same contract as prefill_kernel (hpa_prefill.hip): sequence b owns query
// tokens [cu_q[b], cu_q[b+1]); its token i sits at position q_pos[b] + i and
// attends keys [0, min(q_pos[b] + i + 1, ctx[b])) -- helios' causal rule
// (reference exec/paged_attn.py:401-404).
//
// A workgroup of four waves owns 128 consecutive (token, head-in-group) rows
// of one (sequence, KV head); each wave owns 32 of them, one 32x32 MFMA tile.
// The workgroup walks the keys in steps of 32.  Every step's K and V tiles
// (32 keys x head_dim each) are copied once from the paged pool into LDS by
// direct global->LDS buffer loads issued by all four waves, two steps ahead
// of the compute, and then read by every wave, so each K/V byte leaves L2 once
// per 128 query rows instead of once per wave.
//
// Per wave and step:
//   S^T[key][row] = K[key][:] . Q[row][:]        head_dim / 16 MFMAs
//   online softmax down each row (column of S^T; the two halves of a row's
//   32 keys sit in lanes l and l ^ 32)
//   O^T[dim][row] += V^T[dim][key] P^T[key][row]  2 * head_dim / 32 MFMAs
// The S^T result layout (lane l: row l % 32, keys 8j + 4(l/32) + i) is the
// P^T operand layout once each 16-key MFMA chunk takes keys {8j + 4(l/32) + i:
// j in {2kc, 2kc+1}}, so probabilities never leave the lane.  V^T's operand
// wants one head dim across 8 keys per lane: lane m reads head dims
// [DB*m, DB*m + DB) of each key (DB = head_dim / 32) and PV MFMA db takes
// element db of every key, so the dims land as DB*M + db.
//
// LDS rows are 16-byte chunks XOR-swizzled by the key row (chunk j of row r at
// position j ^ (r % chunks_per_row)); the global->LDS loads apply the inverse
// permutation on the global side, so the per-lane LDS destinations stay the
// hardware's consecutive ones, and both the K reads (16 keys x one chunk) and
// the V reads (one key x all chunks) hit distinct banks.
#include <type_traits>

#include "hpa_attn_core.h"
#include "hpa_host.h"
#include "hpa_prefill.h"

namespace hpa {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <class CT> struct M32;
template <> struct M32<F16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                  c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    return f32_to_f16_bits(x) | (f32_to_f16_bits(y) << 16);
  }
  __device__ __forceinline__ static float lo_of(uint32_t w) { return f16_bits_to_f32(w & 0xffffu); }
  __device__ __forceinline__ static float hi_of(uint32_t w) { return f16_bits_to_f32(w >> 16); }
};
template <> struct M32<BF16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    return f32_to_bf16_bits(x) | (f32_to_bf16_bits(y) << 16);
  }
  __device__ __forceinline__ static float lo_of(uint32_t w) { return bf16_bits_to_f32(w & 0xffffu); }
  __device__ __forceinline__ static float hi_of(uint32_t w) { return bf16_bits_to_f32(w >> 16); }
};

constexpr int kPfWaves = 4;              // waves per workgroup, 32 rows each
constexpr int kPfRows = 32 * kPfWaves;   // rows per workgroup
constexpr int kPfStages = 3;             // LDS tiles: two steps of loads in flight
constexpr int kPfLazy = 8;               // rescale only when a row max grows by > 2^8

// x combined with the value of lane l ^ 32 (the other half of the same row)
__device__ __forceinline__ float pair_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

template <class CT, int D>
__global__ __launch_bounds__(64 * kPfWaves, 2) void prefill_mfma_kernel(const PrefillArgs a,
                                                                     const int32_t* __restrict__ tables,
                                                                     int tiles_per_unit) {
  typedef M32<CT> M;
  typedef typename CT::storage q_t;
  constexpr int NCH = D / 8;          // 16-byte chunks per key row
  constexpr int ROWB = D * 2;         // bytes per key row
  constexpr int TILEB = 32 * ROWB;    // one 32-key tile of K or of V
  constexpr int KCH = D / 16;         // QK MFMAs per step
  constexpr int DB = D / 32;          // PV dim blocks; lane m holds dims [DB*m, DB*m + DB)
  constexpr int VW = (DB * 2 + 3) / 4;  // u32 words of V per key per lane
  constexpr int IPW = NCH / 4;        // global->LDS instructions per wave per step
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(kPfStages == 3, "the step loop is unrolled by three");
  __shared__ __attribute__((aligned(16))) uint8_t smem[kPfStages][2 * TILEB];

  // heaviest (last) row tiles first; the units of one tile index spread over
  // consecutive workgroup ids, so a unit's tiles share an XCD when the unit
  // count is a multiple of 8
  const int unit = blockIdx.x;
  const int tile = tiles_per_unit - 1 - (int)blockIdx.y;
  const int b = unit / a.num_kv_heads, kvh = unit - b * a.num_kv_heads;
  const int G = a.group;
  const int q0 = a.cu_q[b];
  const int rows = (a.cu_q[b + 1] - q0) * G;
  if (tile * kPfRows >= rows) return;  // uniform over the workgroup, before any barrier
  const int ctx = a.ctx_lens[b];
  const int pos0 = a.q_pos[b];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, n = lane & 31;
  auto limit = [&](int r) -> int { return max(min(pos0 + r / G + 1, ctx), 0); };

  const int r0 = tile * kPfRows + 32 * w;           // this wave's first row
  const int r = r0 + n;                             // this lane's row
  const bool rv = r < rows;
  const int lim = rv ? limit(r) : 0;
  const bool wave_live = r0 < rows;
  const int wave_minlim = wave_live ? limit(r0) : 0;
  const int wave_maxlim = wave_live ? limit(min(r0 + 31, rows - 1)) : 0;
  const int wg_maxlim = limit(min(tile * kPfRows + kPfRows - 1, rows - 1));
  const int nsteps = (wg_maxlim + 31) >> 5;

  // ---- query rows into registers (B operand of S^T): lane half h holds dims
  // [h*D/2, (h+1)*D/2) as KCH chunks of 8
  const q_t* qp = reinterpret_cast<const q_t*>(a.q);
  u32x4 qf[KCH];
  {
    const int t = r / G, hh = r - t * G;
    const q_t* qrow = qp + ((long)(q0 + t) * a.num_q_heads + kvh * G + hh) * D + h * (D / 2);
#pragma unroll
    for (int c = 0; c < KCH; ++c)
      qf[c] = rv ? *reinterpret_cast<const u32x4*>(qrow + 8 * c) : (u32x4){0, 0, 0, 0};
  }

  // ---- cooperative global->LDS copy.  Wave w copies tensor w / 2 (K, V),
  // 16-key half w % 2 of every step: IPW instructions of 64 lanes x 16 bytes.
  // Lane offsets (global side, swizzle applied) are the same every step.
  const int tensor = w >> 1, half = w & 1;
  uint32_t voff[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int P = (w * IPW + i) * 64 + lane;     // chunk position in [K tile | V tile]
    const int row = (P % (32 * NCH)) / NCH, q = P % NCH;
    voff[i] = (uint32_t)((row & 15) * ROWB + (q ^ (row % NCH)) * 16);
  }
  const char* pool = reinterpret_cast<const char*>(tensor ? a.v : a.k);
  const long blk_rows = (long)a.num_kv_heads << a.bs_log2;   // key rows per block
  const long head_rows = (long)kvh << a.bs_log2;
  const int bsm = (1 << a.bs_log2) - 1;
  const int32_t* trow = tables + (long)b * a.table_stride;
  TableWindow win;
  if (nsteps > 0) win.fill(trow, a.table_stride, 0);
  auto issue_loads = [&](int step, int stage) {
    const int key0 = step * 32 + 16 * half;
    int valid = min(max(ctx - key0, 0), 16);     // rows past the context read as zeros
    int phys = 0;
    if (valid > 0) {
      const int lb = key0 >> a.bs_log2;
      if (!win.covers(lb)) win.fill_sync(trow, a.table_stride, lb);
      phys = win.get(lb);
      if ((unsigned)phys >= (unsigned)a.num_blocks) { phys = 0; valid = 0; }
    }
    const char* base = pool + ((long)phys * blk_rows + head_rows + (key0 & bsm)) * ROWB;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, valid * ROWB, 0x00020000);
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      // a local copy: the host pass of this builtin rejects a captured array
      // element, which would silently drop the kernel's launch stub
      const int vo = (int)voff[i];
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (__attribute__((address_space(3))) void*)(&smem[stage][0] + (w * IPW + i) * 64 * 16), 16, vo, 0, 0, 0);
    }
  };

  // ---- per-lane LDS offsets of the operand reads (same in every stage)
  uint32_t koff[KCH], vofs[2][8];
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    const int jj = h * (NCH / 2) + c;
    koff[c] = (uint32_t)((n * NCH + (jj ^ (n % NCH))) * 16);
  }
  {
    const int jv = (DB * 2 * n) / 16, off = (DB * 2 * n) % 16;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) {
        const int key = 8 * (2 * kc + (s2 >> 2)) + 4 * h + (s2 & 3);
        vofs[kc][s2] = (uint32_t)(TILEB + (key * NCH + (jv ^ (key % NCH))) * 16 + off);
      }
  }

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = (f32x16){};
  float m = -INFINITY, l = 0.f;
  const float cs = a.scale_log2;

  // one step: wait for its copies, barrier, issue the copies two steps ahead,
  // then compute (STAGE folds to a constant in every unrolled call)
  auto step = [&](int i, const int STAGE) {
    if (i + 1 < nsteps) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | IPW);  // vmcnt(IPW): this wave's copies for step i landed
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);        // vmcnt(0)
    }
    // After the barrier every wave's copies for step i are in LDS (each
    // waited for its own above) and every wave has consumed its reads of
    // the stage step i + 2 refills (step i - 1).  No memory fence: a
    // workgroup fence would also wait for the copies of step i + 1 still in
    // flight; the signal fences keep the compiler from moving LDS accesses.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (i + 2 < nsteps) issue_loads(i + 2, (STAGE + 2) % kPfStages);
    const int k0 = 32 * i;
    if (k0 >= wave_maxlim) return;
    const uint8_t* st_base = &smem[STAGE][0];

    // ---- S^T = K . Q^T
    f32x16 st = (f32x16){};
#pragma unroll
    for (int c = 0; c < KCH; ++c) st = M::mma(*reinterpret_cast<const u32x4*>(st_base + koff[c]), qf[c], st);
    // ---- V rows of this lane's 16 keys, dims [DB*n, DB*n + DB)
    uint32_t vr[2][8][VW];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int s2 = 0; s2 < 8; ++s2) {
        const uint8_t* p = st_base + vofs[kc][s2];
        if constexpr (VW == 2) {
          const u32x2 x = *reinterpret_cast<const u32x2*>(p);
          vr[kc][s2][0] = x[0];
          vr[kc][s2][VW - 1] = x[1];
        } else {
          vr[kc][s2][0] = *reinterpret_cast<const uint32_t*>(p);
        }
      }
    // ---- online softmax over the row's 32 keys (16 here, 16 in lane ^ 32);
    // only steps crossing some row's limit pay for the mask
    float x[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) x[v] = st[v];
    if (__builtin_expect(k0 + 32 > wave_minlim, 0)) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = k0 + 8 * (v >> 2) + 4 * h + (v & 3);
        x[v] = key < lim ? x[v] : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, x[v]);
    mx = pair_max(mx) * cs;  // scale_log2 > 0 keeps the order
    const bool grow = mx > m + (float)kPfLazy;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float mnew = grow ? mx : m;
      const float alpha = __builtin_amdgcn_exp2f(m - (mnew == -INFINITY ? 0.f : mnew));
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] = o[db] * alpha;
    }
    const float mref = m == -INFINITY ? 0.f : m;
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(x[v], cs, -mref));
      ps += p;
      x[v] = p;  // -inf scores give exactly 0
    }
    l += ps;
    // ---- O^T += V^T . P^T, two 16-key chunks
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      u32x4 pf, pl;
#pragma unroll
      for (int p = 0; p < 4; ++p) pf[p] = M::pack(x[8 * kc + 2 * p], x[8 * kc + 2 * p + 1]);
      if constexpr (std::is_same<CT, BF16>::value) {
        // bf16 keeps 8 significant bits; P = hi + lo carries ~16
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t wv = pf[p];
          pl[p] = M::pack(x[8 * kc + 2 * p] - M::lo_of(wv), x[8 * kc + 2 * p + 1] - M::hi_of(wv));
        }
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int wd = (db * 2) / 4, hb = db & 1;  // word and 16-bit half holding dim DB*n + db
        const uint32_t sel = (uint32_t)(2 * hb) | ((uint32_t)(2 * hb + 1) << 8) |
                             ((uint32_t)(4 + 2 * hb) << 16) | ((uint32_t)(5 + 2 * hb) << 24);
        u32x4 vf;
#pragma unroll
        for (int p = 0; p < 4; ++p)
          vf[p] = __builtin_amdgcn_perm(vr[kc][2 * p + 1][wd], vr[kc][2 * p][wd], sel);
        o[db] = M::mma(vf, pf, o[db]);
        if constexpr (std::is_same<CT, BF16>::value) o[db] = M::mma(vf, pl, o[db]);
      }
    }
  };

  // the query rows land before the first tile copy is issued, so no wait in
  // the loop has to cover them
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  if (nsteps > 0) issue_loads(0, 0);
  if (nsteps > 1) issue_loads(1, 1);
  for (int i0 = 0; i0 < nsteps; i0 += kPfStages) {
#pragma unroll
    for (int u = 0; u < kPfStages; ++u)
      if (i0 + u < nsteps) step(i0 + u, u);
  }

  // ---- epilogue: O = O^T / l; lane holds dims DB*M + db for M in its 16 rows of O^T
  const float lt = pair_sum(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (rv) {
    const int t = r / G, hh = r - t * G;
    q_t* orow = reinterpret_cast<q_t*>(a.out) + ((long)(q0 + t) * a.num_q_heads + kvh * G + hh) * D;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int Mi = 8 * (v >> 2) + 4 * h + (v & 3);
      if constexpr (DB == 4) {
        u32x2 pk;
        pk[0] = M::pack(o[0][v] * inv, o[1][v] * inv);
        pk[1] = M::pack(o[2][v] * inv, o[3][v] * inv);
        *reinterpret_cast<u32x2*>(orow + DB * Mi) = pk;
      } else {
        *reinterpret_cast<uint32_t*>(orow + DB * Mi) = M::pack(o[0][v] * inv, o[1][v] * inv);
      }
    }
  }
}


template <class CT, int D>
static void launch_one(const PrefillArgs& a, int max_q_len, hipStream_t s) {
  const int units = a.num_seqs * a.num_kv_heads;
  const int tiles = (max_q_len * a.group + kPfRows - 1) / kPfRows;
  hipLaunchKernelGGL((prefill_mfma_kernel<CT, D>), dim3((unsigned)units, (unsigned)tiles), dim3(64 * kPfWaves),
                     0, s, a, a.tables, tiles);
}

bool launch_prefill_mfma(const PrefillArgs& a, int q_dtype, int kv_dtype, int head_dim, int max_q_len,
                         hipStream_t s) {
  if (a.bs_log2 < 4 || kv_dtype != q_dtype || (head_dim != 64 && head_dim != 128)) return false;
  if ((long)max_q_len * a.group > (1L << 30)) return false;
  if (q_dtype == HPA_F16) {
    if (head_dim == 128) launch_one<F16, 128>(a, max_q_len, s);
    else launch_one<F16, 64>(a, max_q_len, s);
    return true;
  }
  if (q_dtype == HPA_BF16) {
    if (head_dim == 128) launch_one<BF16, 128>(a, max_q_len, s);
    else launch_one<BF16, 64>(a, max_q_len, s);
    return true;
  }
  return false;
}

}  // namespace hpa
