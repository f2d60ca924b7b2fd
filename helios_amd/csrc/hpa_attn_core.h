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

// A window of one sequence's block table held in two VGPRs: lane i holds
// entries base + i and base + 64 + i.  Block ids are then read with
// v_readlane at a wave-uniform index, so the KV loads of a step never wait on
// a table read.  Entries past the table's end read as 0.
struct TableWindow {
  int base = 0, limit = 0;  // holds logical blocks [base, limit)
  uint32_t w0 = 0, w1 = 0;

  __device__ __forceinline__ bool covers(int lb) const { return lb >= base && lb < limit; }

  __device__ __forceinline__ void fill(const int32_t* row, int stride, int b0) {
    const int lane = threadIdx.x & 63;
    base = b0;
    limit = b0 + 128;
    w0 = b0 + lane < stride ? (uint32_t)row[b0 + lane] : 0u;
    w1 = b0 + 64 + lane < stride ? (uint32_t)row[b0 + 64 + lane] : 0u;
  }

  // Fill and wait for it here, so that later reads of the window never make
  // the compiler wait for loads that are still in flight (a KV prefetch
  // issued after a possible refill would otherwise be drained at every read).
  __device__ __forceinline__ void fill_sync(const int32_t* row, int stride, int b0) {
    fill(row, stride, b0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }

  // Takes entries [b0, b0 + 128) from an LDS copy made by stage_window.
  __device__ __forceinline__ void fill_lds(const uint32_t* lds, int b0) {
    const int lane = threadIdx.x & 63;
    base = b0;
    limit = b0 + 128;
    w0 = lds[lane];
    w1 = lds[64 + lane];
  }

  __device__ __forceinline__ int get(int lb) const {
    const int i = lb - base;
    return i < 64 ? __builtin_amdgcn_readlane((int)w0, i) : __builtin_amdgcn_readlane((int)w1, i - 64);
  }
};

typedef __attribute__((address_space(3))) void lds_void;

// Issues a direct global->LDS copy of table entries [b0, b0 + 128) of `row`
// (entries at or past `stride` read as 0) into 512 bytes of LDS at `lds`:
// two loads, no VGPR, nothing waits for them.  The copy has landed once
// vmcnt has fallen below the number of vector memory instructions issued
// after it.
__device__ __forceinline__ void stage_window(void* lds, const int32_t* row, int stride, int b0) {
  const int lane = threadIdx.x & 63;
  const int n = max(0, min(stride - b0, 128));
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(row + min(b0, stride)), (short)0, __builtin_amdgcn_readfirstlane(4 * n), 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 4, 4 * lane, 0, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)((char*)lds + 256), 4, 256 + 4 * lane, 0, 0, 0);
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

  // int8 KV with fp16 compute converts a key byte x to the fp16 subnormal
  // (128 + x) 2^-24 and a value byte to the fp16 value 1152 + x (two VALU
  // ops per pair of values instead of three) and removes the offsets
  // algebraically: S = 2^24 (S' - 128 2^-24 sum(q)) and O = O' - 1152 sum(P').
  // The small key offset keeps the fp32 sums of S' near the score's own
  // magnitude, so large key scales do not amplify their rounding.
  //
  // Over int8 pools the MFMAs run in fp16 for bf16 queries too (MT, the math
  // type): a bf16 value is exact in fp16 within fp16's range, and each
  // query row enters scaled by the power of two that brings its largest
  // element into [2^14, 2^15) (the scale returns in the row's score scale), so
  // the cheap fp16 form of the dequantisation serves both.  The output is
  // still written in the query dtype.
  typedef typename std::conditional<QUANT && std::is_same<CT, BF16>::value, F16, CT>::type MT;
  static constexpr bool I8F16 = QUANT && std::is_same<MT, F16>::value;
  static constexpr bool kBf16Q = QUANT && std::is_same<CT, BF16>::value;
  static constexpr float kI8KOff = 0x1p-17f;  // 128 * 2^-24
  static constexpr float kI8VOff = 1152.f;
  // P enters the PV MFMAs as two terms (hi + lo) for bf16 compute and for
  // int8 pools with fp16 compute
  static constexpr bool kSplitP = std::is_same<MT, BF16>::value || I8F16;
  // Rescale the accumulators only when a row max grows by more than 2^8;
  // probabilities then stay below 2^8 relative to the running reference.
  static constexpr float kLazy = 8.f;

  Frag<MT> q[NT][C];
  f32x4 o[NT][J];
  f32x4 ps[NT];     // I8F16: sum over keys of the fp16 P' fed to the PV MFMAs
  float qoff[NT];   // I8F16: 128 * 2^-24 * sum_d q[row][d]
  float qexp[NT];   // bf16 queries over int8: 2^e, the row entered fp16 as row * 2^-e
  float m[NT], l[NT];
  int lim[NT];

  __device__ __forceinline__ static int lane() { return threadIdx.x & 63; }

  // Row pointer per n-tile (nullptr for padding rows) and key limit.
  __device__ __forceinline__ void init(const q_t* const* rowq, const int* rowlim) {
    load_q(rowq);
    start(rowlim);
  }

  // Issues the loads of the query rows (the B operand of S^T), one row
  // pointer per n-tile (nullptr for padding rows).  Nothing waits for them
  // until start(), so loads issued in between (a table window, the first
  // K/V steps) are not waited for with them.
  __device__ __forceinline__ void load_q(const q_t* const* rowq) {
    const int g = lane() >> 4;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
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
    }
  }

  // Resets the softmax state for the rows load_q loaded, with their key
  // limits, and derives the query terms (this waits for the query rows).
  __device__ __forceinline__ void start(const int* rowlim) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      lim[nt] = rowlim[nt];
      m[nt] = -INFINITY;
      l[nt] = 0.f;
#pragma unroll
      for (int j = 0; j < J; ++j) o[nt][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
      qexp[nt] = 1.f;
      if constexpr (kBf16Q) {
        // bf16 bits -> fp16, the row scaled by the power of two 2^-e that
        // brings its largest magnitude into [2^14, 2^15): the fp16 row then
        // keeps the bf16 precision of every element down to 2^-28 of it
        float mx = 0.f;
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t wi = q[nt][c].w[i];
            mx = fmaxf(mx, fmaxf(fabsf(bf16_bits_to_f32(wi & 0xffffu)), fabsf(bf16_bits_to_f32(wi >> 16))));
          }
        mx = xor_max(mx);
        const int e = mx > 0.f ? max(min(__builtin_amdgcn_frexp_expf(mx) - 15, 240), -120) : 0;
        qexp[nt] = __builtin_ldexpf(1.f, e);
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t wi = q[nt][c].w[i];
            const f16x2 h = {(_Float16)__builtin_ldexpf(bf16_bits_to_f32(wi & 0xffffu), -e),
                             (_Float16)__builtin_ldexpf(bf16_bits_to_f32(wi >> 16), -e)};
            q[nt][c].w[i] = __builtin_bit_cast(uint32_t, h);
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
        qoff[nt] = kI8KOff * xor_sum(sq);
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

  // Lane-constant byte offsets of the fast path (block_size >= 16), relative
  // to the first key of a 16-key tile.
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
  // its four tensors (K, V and, for int8, their scales) are each one
  // contiguous range whose base is wave-uniform.  Each becomes a buffer
  // resource (base in SGPRs, lane offsets in one VGPR); a tile wholly past
  // the context gets a zero-length resource, so its loads return zeros
  // without touching memory.  The block id comes from the table window held
  // in registers, so no load waits on a table read.
  static constexpr int kTileBytes = 16 * D * ESZ;
  static constexpr int kTileScaleBytes = QUANT ? 16 * (int)sizeof(typename ST::storage) : 0;

  template <int NB>
  __device__ __forceinline__ static void buf_load(uint32_t* r, __amdgpu_buffer_rsrc_t rs, uint32_t off) {
    if constexpr (NB >= 16) {
#pragma unroll
      for (int i = 0; i < NB / 16; ++i) {
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * i, 0, 0);
        r[4 * i + 0] = x[0];
        r[4 * i + 1] = x[1];
        r[4 * i + 2] = x[2];
        r[4 * i + 3] = x[3];
      }
    } else if constexpr (NB == 8) {
      const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
      r[0] = x[0];
      r[1] = x[1];
    } else if constexpr (NB == 4) {
      r[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
    } else if constexpr (NB == 2) {
      r[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
    } else {
      r[0] = __builtin_amdgcn_raw_buffer_load_b8(rs, off, 0, 0);
    }
  }

  __device__ __forceinline__ static __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    // dword 3 = 0x00020000: 32-bit data format, the raw-buffer setting for gfx9 parts
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
  }

  // Loads tile t (keys key0 .. key0 + 15, key0 a multiple of 16) whose block
  // is `phys`; `valid` false gives zeros.
  __device__ __forceinline__ static void load_tile(const PoolView& pv, int t, int key0, int phys,
                                                   bool valid, const LaneOff& lo, Raw& r) {
    const int n = lane() & 15, g = lane() >> 4;
    const int bsm = (1 << pv.bs_log2) - 1;
    const long slot0 = ((long)(phys * pv.num_kv_heads + pv.kvh) << pv.bs_log2) + (key0 & bsm);
    const char* kb = reinterpret_cast<const char*>(pv.k) + slot0 * (D * ESZ);
    const char* vb = reinterpret_cast<const char*>(pv.v) + slot0 * (D * ESZ);
    const int nbytes = valid ? kTileBytes : 0;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb, nbytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb, nbytes);
    if (g * KPL < D) {
      buf_load<KPL * ESZ>(r.k[t], rk, lo.k);
    } else {
#pragma unroll
      for (int i = 0; i < KW; ++i) r.k[t][i] = 0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (J * n < D) {
        buf_load<VB>(r.v[4 * t + i], rv, lo.v + i * (D * ESZ));
      } else {
#pragma unroll
        for (int w = 0; w < VW; ++w) r.v[4 * t + i][w] = 0;
      }
    }
    if constexpr (QUANT) {
      typedef typename ST::storage s_t;
      const int sbytes = valid ? kTileScaleBytes : 0;
      const __amdgpu_buffer_rsrc_t rks =
          make_rsrc(reinterpret_cast<const char*>(pv.ks) + slot0 * (long)sizeof(s_t), sbytes);
      const __amdgpu_buffer_rsrc_t rvs =
          make_rsrc(reinterpret_cast<const char*>(pv.vs) + slot0 * (long)sizeof(s_t), sbytes);
      buf_load<SB>(r.ks[t], rks, lo.s);
      buf_load<SB>(r.vs[t], rvs, lo.s);
    }
  }

  // Both tiles of the 32-key step starting at k0 (wave-uniform), fast path.
  // With `enable` false every tile is a zero-length resource: the load
  // instructions still issue (so the compiler's wait counts do not depend on
  // a branch) but return zeros without touching memory.
  __device__ __forceinline__ static void load_big(const PoolView& pv, const TableWindow& win, int k0,
                                                  const LaneOff& lo, Raw& r, bool enable = true) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key0 = k0 + 16 * t;
      const bool valid = enable && key0 < pv.ctx;
      int phys = 0;
      if (valid) {
        // the caller keeps the window covering every valid tile it loads
        phys = win.get(key0 >> pv.bs_log2);
        phys = (unsigned)phys < (unsigned)pv.num_blocks ? phys : 0;  // never leave the pool
      }
      load_tile(pv, t, key0, phys, valid, lo, r);
    }
  }

  // Makes `win` cover the blocks of the 32-key step at k0 (fast path only);
  // a refill waits for its load.
  template <bool BIG>
  __device__ __forceinline__ static void cover(const PoolView& pv, TableWindow& win, int k0) {
    if constexpr (BIG) {
      const int last = min(k0 + 31, pv.ctx - 1);
      if (last >= k0 && !(win.covers(k0 >> pv.bs_log2) && win.covers(last >> pv.bs_log2)))
        win.fill_sync(pv.table, pv.table_stride, k0 >> pv.bs_log2);
    }
  }

  // One step's loads.  Fast path: issued unconditionally, `enable` false
  // makes them empty; general path: nothing is issued when disabled.
  template <bool BIG>
  __device__ __forceinline__ static void load_sel(const PoolView& pv, TableWindow& win, int k0,
                                                  const LaneOff& lo, Raw& r, bool enable = true) {
    if constexpr (BIG) {
      if (enable) cover<BIG>(pv, win, k0);
      load_big(pv, win, k0, lo, r, enable);
    } else {
      if (enable) load(pv, k0, r);
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
  __device__ __forceinline__ static void k_frag(const uint32_t* kr, int c, Frag<MT>& f) {
    if constexpr (QUANT) {
      const uint32_t w0 = kr[2 * c], w1 = kr[2 * c + 1];
      if constexpr (std::is_same<MT, F16>::value) {
        // [b0^0x80, 0x00, b1^0x80, 0x00] = fp16 ((128 + x0) 2^-24, (128 + x1) 2^-24)
        const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
        f.w[0] = __builtin_amdgcn_perm(0u, x0, 0x0C010C00u);
        f.w[1] = __builtin_amdgcn_perm(0u, x0, 0x0C030C02u);
        f.w[2] = __builtin_amdgcn_perm(0u, x1, 0x0C010C00u);
        f.w[3] = __builtin_amdgcn_perm(0u, x1, 0x0C030C02u);
      } else {
        float x[8];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          x[s] = i8_to_f32(w0, s);
          x[4 + s] = i8_to_f32(w1, s);
        }
        frag_from_f32(f, x);
      }
    } else if constexpr (std::is_same<MT, F32>::value) {
#pragma unroll
      for (int s = 0; s < 8; ++s) f.f[s] = __builtin_bit_cast(float, kr[8 * c + s]);
    } else {
      f.w = (u32x4){kr[4 * c], kr[4 * c + 1], kr[4 * c + 2], kr[4 * c + 3]};
    }
  }

  // V^T operand for MFMA j: element j of each of the 8 key slots.
  __device__ __forceinline__ static void v_frag(const Raw& r, int j, Frag<MT>& f) {
    if constexpr (QUANT) {
      if constexpr (std::is_same<MT, F16>::value) {
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

  // Reductions over the four 16-lane rows (lanes l, l^16, l^32, l^48) with
  // the gfx950 row-swap instructions instead of LDS permutes:
  // permlane16_swap(x, x) yields rows (0,0,2,2) and (1,1,3,3) of x,
  // permlane32_swap(x, x) yields rows (0,1,0,1) and (2,3,2,3).
  __device__ __forceinline__ static float xor_max(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float y = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
    const uint32_t v = __builtin_bit_cast(uint32_t, y);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
  }
  __device__ __forceinline__ static float xor_sum(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float y = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
    const uint32_t v = __builtin_bit_cast(uint32_t, y);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
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
        Frag<MT> kf;
        k_frag(r.k[t], c, kf);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) st[t][nt] = mma(kf, q[nt][c], st[t][nt]);
      }
    }
    // probabilities of every n-tile first, then the PV products one V^T
    // fragment at a time (each converted once and used by every n-tile), so
    // at most one converted V fragment is live
    Frag<MT> pf[NT];
    Frag<MT> pl[NT];  // bf16 and int8 -> fp16: the low half of P
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float x[8];
      float mx = -INFINITY;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        float v = st[s >> 2][nt][s & 3];
        if constexpr (I8F16) v -= qoff[nt];
        v *= (I8F16 ? scale_log2 * 0x1p24f * qexp[nt] : scale_log2) * scale_at(r.ks[s >> 2], s & 3);
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
        x[s] = (!masked || x[s] != -INFINITY) ? p * scale_at(r.vs[s >> 2], s & 3) : 0.f;
      }
      l[nt] += psum;
      frag_from_f32(pf[nt], x);
      if constexpr (kSplitP) {
        // bf16 keeps 8 significant bits, fp16 11: P = hi + lo with both
        // halves in the compute type carries twice that, so the rounding of
        // the weights is not the error term.  (On int8 pools P holds the
        // value scale, P * vs, whose per-key rounding would otherwise reach
        // the output undamped.)
        float lo[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const uint32_t hb = (pf[nt].w[s >> 1] >> (16 * (s & 1))) & 0xffffu;
          lo[s] = x[s] - (std::is_same<MT, BF16>::value ? bf16_bits_to_f32(hb) : f16_bits_to_f32(hb));
        }
        frag_from_f32(pl[nt], lo);
      }
      if constexpr (I8F16) {
        Frag<MT> ones;
        ones.w = (u32x4){0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};
        ps[nt] = mma(ones, pf[nt], ps[nt]);
        ps[nt] = mma(ones, pl[nt], ps[nt]);
      }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      Frag<MT> vf;
      v_frag(r, j, vf);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        o[nt][j] = mma(vf, pf[nt], o[nt][j]);
        if constexpr (kSplitP) o[nt][j] = mma(vf, pl[nt], o[nt][j]);
      }
    }
  }

  // Accumulator element (j, i) of n-tile nt with the int8 offset removed.
  __device__ __forceinline__ float out_val(int nt, int j, int i) const {
    if constexpr (I8F16) return o[nt][j][i] - kI8VOff * ps[nt][0];
    return o[nt][j][i];
  }

  // Row total of l for every lane of the row.
  __device__ __forceinline__ float row_l(int nt) const { return xor_sum(l[nt]); }

  // Output dim of accumulator element (j, i) for lane group g: the lane holds
  // the 4J contiguous dims [4Jg, 4Jg + 4J), element (j, i) at offset J*i + j.
  __device__ __forceinline__ static int out_dim(int g, int j, int i) { return J * (4 * g + i) + j; }
};

}  // namespace hpa
