// Wave-level paged-attention core for gfx950, shared by the decode
// (split-K) and prefill/verify (row-tiled) kernels.
//
// One wavefront owns NT x 16 query rows of one (sequence, KV head) and walks
// a range of keys in steps of 32 (two 16-key tiles).  Rows are query
// (token, head-in-group) pairs, so the G = Hq / Hkv query heads that share a
// KV head share every K/V load (GQA packing).  Per step:
//
//   S^T[key][row] = K[key][:] . Q[row][:]       (A = K, B = Q^T)
//   online softmax down each row (column of S^T)
//   O^T[dim][row] += V^T[dim][key] P^T[key][row] (A = V^T, B = P^T)
//
// Computing the transposed products is what removes every LDS round trip:
//  * the S^T output layout (lane l: row l%16, keys 4*(l/16)+i) is exactly the
//    B-operand layout P^T needs, so probabilities never leave the lane;
//  * the K operand wants key l%16 with contiguous k-slots, and we choose the
//    slot -> head_dim mapping so that lane group g owns the contiguous span
//    [g*D/4, (g+1)*D/4) of the key row: one or two 16-byte loads per lane;
//  * the V^T operand wants, per lane, one head_dim index across 8 keys.
//    Splitting the PV product into J = D/16 MFMAs where MFMA j covers the
//    dims {J*m + j : m = 0..15}, lane m loads the J contiguous elements
//    [J*m, J*m + J) of each of its 8 keys and hands element j to MFMA j.
//    The result lands as 4J contiguous output dims per lane.
//  * the online-softmax rescale is lane-local because O^T's columns are the
//    same rows as S^T's columns.
//
// The pool layout is helios' [num_blocks, Hkv, block_size, D] (paged_attn.py
// :49-51), scales [num_blocks, Hkv, block_size] (paged_attn.py:166-168).
// INT8 values are dequantised in registers: the key scale multiplies the
// score of its key, the value scale multiplies the probability of its key
// before the PV product, so the int8 -> compute conversion is exact.
#pragma once

#include <type_traits>

#include "hpa_types.h"

namespace hpa {

struct PoolView {
  const void* k;        // [num_blocks, Hkv, bs, D] of the KV storage type
  const void* v;
  const void* ks;       // [num_blocks, Hkv, bs] scale type (int8 pools only)
  const void* vs;
  const int32_t* table; // this sequence's block table row
  int table_stride;     // entries in that row
  int kvh, num_kv_heads;
  int bs_log2;
  int num_blocks;
  int ctx;              // keys [0, ctx) exist for this sequence
};

template <int NB>
__device__ __forceinline__ void load_raw(uint32_t* r, const void* p) {
  if constexpr (NB >= 16) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      u32x4 x = reinterpret_cast<const u32x4*>(p)[i];
      r[4 * i + 0] = x[0];
      r[4 * i + 1] = x[1];
      r[4 * i + 2] = x[2];
      r[4 * i + 3] = x[3];
    }
  } else if constexpr (NB == 8) {
    u32x2 x = *reinterpret_cast<const u32x2*>(p);
    r[0] = x[0];
    r[1] = x[1];
  } else if constexpr (NB == 4) {
    r[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (NB == 2) {
    r[0] = *reinterpret_cast<const uint16_t*>(p);
  } else {
    r[0] = *reinterpret_cast<const uint8_t*>(p);
  }
}

template <class CT, class KVT, class ST, int D, int NT>
struct AttnCore {
  static constexpr bool QUANT = std::is_same<KVT, I8>::value;
  static constexpr int DP = D < 32 ? 32 : D;  // head_dim padded to one MFMA k-extent
  static constexpr int C = DP / 32;           // QK^T MFMAs per 16-key tile
  static constexpr int KPL = DP / 4;          // contiguous K elements per lane
  static constexpr int J = D < 16 ? 1 : D / 16;  // PV MFMAs per 32-key step
  typedef typename KVT::storage kv_t;
  typedef typename CT::storage q_t;
  static constexpr int ESZ = sizeof(kv_t);
  static constexpr int KW = (KPL * ESZ + 3) / 4;  // u32 registers of K per tile
  static constexpr int VB = J * ESZ;              // bytes of V per key slot
  static constexpr int VW = (VB + 3) / 4;
  static constexpr int SB = QUANT ? 4 * (int)sizeof(typename ST::storage) : 4;  // 4 scales
  static constexpr int SW = SB / 4;

  struct Raw {
    uint32_t k[2][KW];
    uint32_t v[8][VW];
    uint32_t ks[2][SW];
    uint32_t vs[2][SW];
  };

  // int8 KV with fp16 compute converts a byte x to the fp16 value 1152 + x
  // (two VALU ops per pair of values instead of three) and removes the
  // offset algebraically: S = S' - 1152 * sum(q) and O = O' - 1152 * sum(P').
  static constexpr bool I8F16 = QUANT && std::is_same<CT, F16>::value;
  static constexpr float kI8Off = 1152.f;
  // Rescale the accumulators only when a row max grows by more than 2^8;
  // probabilities then stay below 2^8 relative to the running reference.
  static constexpr float kLazy = 8.f;

  Frag<CT> q[NT][C];
  f32x4 o[NT][J];
  f32x4 ps[NT];     // I8F16: sum over keys of the fp16 P' fed to the PV MFMAs
  float qoff[NT];   // I8F16: 1152 * sum_d q[row][d]
  float m[NT], l[NT];
  int lim[NT];

  __device__ __forceinline__ static int lane() { return threadIdx.x & 63; }

  // Row pointer per n-tile (nullptr for padding rows) and key limit.
  __device__ __forceinline__ void init(const q_t* const* rowq, const int* rowlim) {
    const int g = lane() >> 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      lim[nt] = rowlim[nt];
      m[nt] = -INFINITY;
      l[nt] = 0.f;
#pragma unroll
      for (int j = 0; j < J; ++j) o[nt][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
      const q_t* p = rowq[nt];
      const bool has = p != nullptr && g * KPL < D;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (has) {
          if constexpr (std::is_same<CT, F32>::value) {
            uint32_t r[8];
            load_raw<32>(r, p + g * KPL + c * 8);
#pragma unroll
            for (int s = 0; s < 8; ++s) q[nt][c].f[s] = __builtin_bit_cast(float, r[s]);
          } else {
            uint32_t r[4];
            load_raw<16>(r, p + g * KPL + c * 8);
            q[nt][c].w = (u32x4){r[0], r[1], r[2], r[3]};
          }
        } else {
          frag_zero(q[nt][c]);
        }
      }
      if constexpr (I8F16) {
        float sq = 0.f;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // copy the element out first: a bit_cast applied directly to an
            // ext_vector element reads element 0 (seen with hipcc 7.2)
            const uint32_t wi = q[nt][c].w[i];
            const f16x2 h = __builtin_bit_cast(f16x2, wi);
            sq += (float)h[0] + (float)h[1];
          }
        qoff[nt] = kI8Off * xor_sum(sq);
        ps[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      }
    }
  }

  __device__ __forceinline__ static int phys_of(const PoolView& pv, int key) {
    key = key < pv.ctx ? key : pv.ctx - 1;  // keys past the context read a real key; P = 0 there
    int lb = key >> pv.bs_log2;
    lb = lb < pv.table_stride ? lb : pv.table_stride - 1;
    int b = pv.table[lb];
    b = (unsigned)b < (unsigned)pv.num_blocks ? b : 0;  // never leave the pool
    return b;
  }
  __device__ __forceinline__ static long slot_of(const PoolView& pv, int key, int phys) {
    key = key < pv.ctx ? key : pv.ctx - 1;
    return ((long)(phys * pv.num_kv_heads + pv.kvh) << pv.bs_log2) + (key & ((1 << pv.bs_log2) - 1));
  }

  // Issue every global load of the 32-key step starting at k0.
  __device__ __forceinline__ static void load(const PoolView& pv, int k0, Raw& r) {
    const int n = lane() & 15, g = lane() >> 4;
    const kv_t* kp = reinterpret_cast<const kv_t*>(pv.k);
    const kv_t* vp = reinterpret_cast<const kv_t*>(pv.v);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int kk = k0 + 16 * t + n;  // this lane's key in the K operand
      const long sk = slot_of(pv, kk, phys_of(pv, kk));
      if (g * KPL < D) {
        load_raw<KPL * ESZ>(r.k[t], kp + sk * D + g * KPL);
      } else {
#pragma unroll
        for (int i = 0; i < KW; ++i) r.k[t][i] = 0;
      }
      const int kv = k0 + 16 * t + 4 * g;  // first of this lane's 4 keys in S^T / P^T / V^T
      const int pvb = phys_of(pv, kv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const long sv = slot_of(pv, kv + i, pvb);
        if (J * n < D) {
          load_raw<VB>(r.v[4 * t + i], vp + sv * D + J * n);
        } else {
#pragma unroll
          for (int w = 0; w < VW; ++w) r.v[4 * t + i][w] = 0;
        }
      }
      if constexpr (QUANT) {
        // 4 scales of a 4-aligned key group; past the context, the group of
        // the last key (never straddles a block: block_size >= 4)
        const int kvs = kv < pv.ctx ? kv : ((pv.ctx - 1) & ~3);
        const long s0 = slot_of(pv, kvs, pvb);
        typedef typename ST::storage s_t;
        load_raw<SB>(r.ks[t], reinterpret_cast<const s_t*>(pv.ks) + s0);
        load_raw<SB>(r.vs[t], reinterpret_cast<const s_t*>(pv.vs) + s0);
      }
    }
  }

  // Lane-constant byte offsets of the fast path (block_size >= 16).
  struct LaneOff {
    uint32_t k, v, s;
  };
  __device__ __forceinline__ static LaneOff lane_off() {
    const int n = lane() & 15, g = lane() >> 4;
    LaneOff o;
    o.k = (uint32_t)(n * D * ESZ + g * KPL * ESZ);
    o.v = (uint32_t)(4 * g * D * ESZ + J * n * ESZ);
    o.s = (uint32_t)(4 * g * (QUANT ? (int)sizeof(typename ST::storage) : 0));
    return o;
  }

  // Fast path for block_size >= 16: a 16-key tile never leaves its block, so
  // the block base is one scalar table load and every lane address is that
  // uniform base plus a 32-bit lane-constant offset.  k0 must be
  // wave-uniform.  A tile at or past the context reads the tile holding the
  // last key (real memory; its keys are masked, and the fp V slots of keys
  // past the context are zeroed in compute()).
  __device__ __forceinline__ static void load_big(const PoolView& pv, int k0, const LaneOff& lo,
                                                  Raw& r) {
    const int n = lane() & 15, g = lane() >> 4;
    const int bsm = (1 << pv.bs_log2) - 1;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key0 = k0 + 16 * t;
      const int keyc = key0 < pv.ctx ? key0 : ((pv.ctx - 1) & ~15);
      int lb = keyc >> pv.bs_log2;
      lb = lb < pv.table_stride ? lb : pv.table_stride - 1;
      int phys = pv.table[lb];
      phys = (unsigned)phys < (unsigned)pv.num_blocks ? phys : 0;
      const long slot0 = ((long)(phys * pv.num_kv_heads + pv.kvh) << pv.bs_log2) + (keyc & bsm);
      const char* kb = reinterpret_cast<const char*>(pv.k) + slot0 * (D * ESZ);
      const char* vb = reinterpret_cast<const char*>(pv.v) + slot0 * (D * ESZ);
      if (g * KPL < D) {
        load_raw<KPL * ESZ>(r.k[t], kb + lo.k);
      } else {
#pragma unroll
        for (int i = 0; i < KW; ++i) r.k[t][i] = 0;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (J * n < D) {
          load_raw<VB>(r.v[4 * t + i], vb + lo.v + i * (D * ESZ));
        } else {
#pragma unroll
          for (int w = 0; w < VW; ++w) r.v[4 * t + i][w] = 0;
        }
      }
      if constexpr (QUANT) {
        typedef typename ST::storage s_t;
        const char* ksb = reinterpret_cast<const char*>(pv.ks) + slot0 * (long)sizeof(s_t);
        const char* vsb = reinterpret_cast<const char*>(pv.vs) + slot0 * (long)sizeof(s_t);
        load_raw<SB>(r.ks[t], ksb + lo.s);
        load_raw<SB>(r.vs[t], vsb + lo.s);
      }
    }
  }

  __device__ __forceinline__ static void load_any(const PoolView& pv, int k0, const LaneOff& lo,
                                                  Raw& r) {
    if (pv.bs_log2 >= 4) {
      load_big(pv, k0, lo, r);
    } else {
      load(pv, k0, r);
    }
  }

  __device__ __forceinline__ static float scale_at(const uint32_t* w, int i) {
    if constexpr (QUANT) {
      if constexpr (std::is_same<ST, F16>::value) {
        return f16_bits_to_f32((w[i >> 1] >> (16 * (i & 1))) & 0xffffu);
      } else {
        return __builtin_bit_cast(float, w[i]);
      }
    }
    return 1.f;
  }

  // K operand of one 16-key tile, chunk c, from its raw registers.
  __device__ __forceinline__ static void k_frag(const uint32_t* kr, int c, Frag<CT>& f) {
    if constexpr (QUANT) {
      const uint32_t w0 = kr[2 * c], w1 = kr[2 * c + 1];
      if constexpr (std::is_same<CT, F16>::value) {
        // [b0^0x80, 0x64, b1^0x80, 0x64] = fp16 (1152 + x0, 1152 + x1)
        const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
        f.w[0] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);
        f.w[1] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
        f.w[2] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
        f.w[3] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
      } else {
        float x[8];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          x[s] = i8_to_f32(w0, s);
          x[4 + s] = i8_to_f32(w1, s);
        }
        frag_from_f32(f, x);
      }
    } else if constexpr (std::is_same<CT, F32>::value) {
#pragma unroll
      for (int s = 0; s < 8; ++s) f.f[s] = __builtin_bit_cast(float, kr[8 * c + s]);
    } else {
      f.w = (u32x4){kr[4 * c], kr[4 * c + 1], kr[4 * c + 2], kr[4 * c + 3]};
    }
  }

  // V^T operand for MFMA j: element j of each of the 8 key slots.
  __device__ __forceinline__ static void v_frag(const Raw& r, int j, Frag<CT>& f) {
    if constexpr (QUANT) {
      if constexpr (std::is_same<CT, F16>::value) {
        // fp16 (1152 + x) pairs; the offset leaves through ps[]
#pragma unroll
        for (int p = 0; p < 4; ++p)
          f.w[p] = __builtin_amdgcn_perm(r.v[2 * p + 1][j >> 2], r.v[2 * p][j >> 2],
                                         perm_sel_bytes(j & 3, j & 3)) ^ 0x64806480u;
      } else {
        float x[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) x[s] = i8_to_f32(r.v[s][j >> 2], j & 3);
        frag_from_f32(f, x);
      }
    } else if constexpr (std::is_same<CT, F32>::value) {
#pragma unroll
      for (int s = 0; s < 8; ++s) f.f[s] = __builtin_bit_cast(float, r.v[s][j]);
    } else {
      const int h = j & 1;
      const uint32_t sel = (uint32_t)(2 * h) | ((uint32_t)(2 * h + 1) << 8) |
                           ((uint32_t)(4 + 2 * h) << 16) | ((uint32_t)(5 + 2 * h) << 24);
#pragma unroll
      for (int p = 0; p < 4; ++p)
        f.w[p] = __builtin_amdgcn_perm(r.v[2 * p + 1][j >> 1], r.v[2 * p][j >> 1], sel);
    }
  }

  __device__ __forceinline__ static float xor_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
  }
  __device__ __forceinline__ static float xor_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
  }

  // One 32-key step. `masked` must be true whenever any key of the step may
  // lie at or beyond some row's limit.
  __device__ __forceinline__ void compute(Raw& r, int k0, float scale_log2, bool masked, int ctx) {
    const int g = lane() >> 4;
    if constexpr (!QUANT) {
      // fp pools may hold NaN in slots never written; P = 0 there must stay 0
      if (masked) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int key = k0 + 16 * (s >> 2) + 4 * g + (s & 3);
          if (key >= ctx) {
#pragma unroll
            for (int w = 0; w < VW; ++w) r.v[s][w] = 0;
          }
        }
      }
    }
    f32x4 st[2][NT];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) st[t][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < C; ++c) {
        Frag<CT> kf;
        k_frag(r.k[t], c, kf);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) st[t][nt] = mma(kf, q[nt][c], st[t][nt]);
      }
    }
    float ksl[8], vsc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      ksl[s] = scale_log2 * scale_at(r.ks[s >> 2], s & 3);
      vsc[s] = scale_at(r.vs[s >> 2], s & 3);
    }
    Frag<CT> vf[J];
#pragma unroll
    for (int j = 0; j < J; ++j) v_frag(r, j, vf[j]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float x[8];
      float mx = -INFINITY;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        float v = st[s >> 2][nt][s & 3];
        if constexpr (I8F16) v -= qoff[nt];
        v *= ksl[s];
        if (masked) {
          const int key = k0 + 16 * (s >> 2) + 4 * g + (s & 3);
          v = key < lim[nt] ? v : -INFINITY;
        }
        x[s] = v;
        mx = fmaxf(mx, v);
      }
      mx = xor_max(mx);
      // lazy rescale: wave-uniform branch, taken when some row's max grew
      // by more than 2^kLazy (always on a row's first finite max)
      const bool grow = mx > m[nt] + kLazy;
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float mnew = grow ? mx : m[nt];
        const float alpha = __builtin_amdgcn_exp2f(m[nt] - (mnew == -INFINITY ? 0.f : mnew));
        m[nt] = mnew;
        l[nt] *= alpha;
#pragma unroll
        for (int j = 0; j < J; ++j) o[nt][j] = o[nt][j] * alpha;
        if constexpr (I8F16) ps[nt] = ps[nt] * alpha;
      }
      const float mref = m[nt] == -INFINITY ? 0.f : m[nt];
      float psum = 0.f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float p = __builtin_amdgcn_exp2f(x[s] - mref);
        psum += p;
        // a masked key contributes exactly 0, whatever its (unwritten) scale holds
        x[s] = (!masked || x[s] != -INFINITY) ? p * vsc[s] : 0.f;
      }
      l[nt] += psum;
      Frag<CT> pf;
      frag_from_f32(pf, x);
      if constexpr (std::is_same<CT, BF16>::value) {
        // bf16 keeps 8 significant bits; P = hi + lo with both halves in
        // bf16 carries ~16, so probabilities are not the error term.
        float lo[8];
#pragma unroll
        for (int s = 0; s < 8; ++s)
          lo[s] = x[s] - bf16_bits_to_f32((pf.w[s >> 1] >> (16 * (s & 1))) & 0xffffu);
        Frag<CT> pl;
        frag_from_f32(pl, lo);
#pragma unroll
        for (int j = 0; j < J; ++j) {
          o[nt][j] = mma(vf[j], pf, o[nt][j]);
          o[nt][j] = mma(vf[j], pl, o[nt][j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < J; ++j) o[nt][j] = mma(vf[j], pf, o[nt][j]);
        if constexpr (I8F16) {
          Frag<CT> ones;
          ones.w = (u32x4){0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};
          ps[nt] = mma(ones, pf, ps[nt]);
        }
      }
    }
  }

  // Accumulator element (j, i) of n-tile nt with the int8 offset removed.
  __device__ __forceinline__ float out_val(int nt, int j, int i) const {
    if constexpr (I8F16) return o[nt][j][i] - kI8Off * ps[nt][0];
    return o[nt][j][i];
  }

  // Row total of l for every lane of the row.
  __device__ __forceinline__ float row_l(int nt) const { return xor_sum(l[nt]); }

  // Output dim of accumulator element (j, i) for lane group g: the lane holds
  // the 4J contiguous dims [4Jg, 4Jg + 4J), element (j, i) at offset J*i + j.
  __device__ __forceinline__ static int out_dim(int g, int j, int i) { return J * (4 * g + i) + j; }
};

}  // namespace hpa
