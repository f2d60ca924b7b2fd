// Paged decode / speculative-verify attention for gfx950.
//
// Replaces helios' paged_attention_decode_batched (exec/paged_attn.py:298-353)
// and the Triton kernel (exec/triton_attn.py:54-130).  Every sequence carries
// q_per_seq query tokens (1 for decode, gamma+1 for verify); token t of a
// sequence with context c sits at position c - q_per_seq + t and attends keys
// [0, c - q_per_seq + t], which is helios' prefill mask (paged_attn.py:401-404)
// with start_pos = c - q_per_seq.
//
// Work decomposition (stream-K).  A "unit" is one (sequence, KV head); it
// holds ceil(context / 32) steps of 32 keys (one step for an empty context,
// which writes zeros).  Units are laid end to end, sequence-major, into one
// global step range of T steps, and the kernel's W waves (as many as the
// device keeps resident) each take an equal contiguous slice of ceil(T / W)
// steps.  A wave therefore streams the same number of KV bytes as every other
// wave whatever the context lengths are, with one step of loads in flight,
// and pays the unit prologue (block-table window and query rows into
// registers) only where its slice crosses a unit boundary.  All
// G * q_per_seq query rows of a KV head live in the wave (GQA packing), so
// every K/V byte is read from HBM once.
//
// A unit that lies wholly inside one wave's slice is normalised and written
// to `out` by that wave.  A unit cut by slice boundaries is split into
// pieces held by consecutive waves; each piece leaves its (O, m, l) in the
// workspace and bumps the unit's arrival counter, and the wave that brings
// the counter to the piece count merges all pieces in piece order, reading
// every piece (its own included) back from the workspace, and resets the
// counter to zero.  The merge order is fixed,
// so results do not depend on which wave arrives last.  No wave ever waits
// for another.
#pragma once

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
  int num_waves;   // W: waves launched
  int min_steps;   // lower bound on a wave's slice, in 32-key steps
  int* counters;   // [num_seqs * Hkv] arrival counters, zero between calls
  float* ws_ml;    // [W][2][rows][2]  (m, l) of partial pieces
  float* ws_o;     // [W][2][rows][max(D, 16)]  unnormalised O of partial pieces (lane-major)
};

constexpr int kWavesPerGroup = 4;
constexpr int kWaveCap = 4096;          // 256 CUs x 16 resident waves
// Steps of KV loads in flight per wave.  The kernel runs one wave per SIMD:
// two waves sharing a SIMD are served oldest-first, so with equal slices the
// younger one finishes long after the older, while a single wave with a deep
// pipeline keeps the SIMD's share of HBM busy on its own.
constexpr int kDepth = 3;
// Steps of loads in flight, where kDepth's ring would spill: head_dim 256,
// and key rows of 512 bytes or more (fp32 pools at head_dim 128), keep one (a
// step's K/V registers, 64 VGPRs per tensor, times a ring of four spilled
// over a thousand registers to scratch and cost two thirds of the
// bandwidth); with more row tiles, 256-byte rows keep two at two tiles and
// one at four, and int8 rows of head_dim 128 two at two tiles and one at
// four.
template <int D, class KVT, int NT>
constexpr int ring_depth() {
  constexpr int rowb = D * (int)sizeof(typename KVT::storage);
  constexpr bool i8 = sizeof(typename KVT::storage) == 1;
  if (D >= 256 || rowb >= 512) return 1;
  if (NT >= 4 && (rowb >= 256 || (i8 && D >= 128))) return 1;
  if (NT >= 2 && (rowb >= 256 || (i8 && D >= 128))) return 2;
  return kDepth;
}
constexpr int kDefaultMinTokens = 256;  // per-wave slice floor (8 steps)
// What a unit costs beyond its steps, in step-equivalents: its prologue
// (table window, query rows, first loads in flight) and epilogue (output or
// partial stores, arrival count, possibly the merge).  Slices are cut on
// steps plus this, so waves holding many short units get fewer steps.
constexpr int kUnitCost = 4;

// Contexts are honoured as given up to 2^30 tokens (keys are int32 and a
// step index times 32 must not overflow); the launch's max_context_len only
// sizes the grid.  Positions in a head's step space are 64-bit sums.
constexpr int kMaxContext = 1 << 30;

__device__ __forceinline__ int clamp_ctx(int ctx) { return min(ctx, kMaxContext); }

__device__ __forceinline__ int unit_steps(int ctx) {
  ctx = clamp_ctx(ctx);
  return ctx <= 0 ? 1 : (ctx + 31) >> 5;
}

__device__ __forceinline__ long wave_sum_l(long x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ long wave_incl_scan_l(long x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const long y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

__device__ __forceinline__ long uniform_l(long x) {
  const int lo = __builtin_amdgcn_readfirstlane((int)(x & 0xffffffffL));
  const int hi = __builtin_amdgcn_readfirstlane((int)(x >> 32));
  return (long)(((unsigned long)(unsigned)hi << 32) | (unsigned)lo);
}

// Position of a wave in the global step range.
struct UnitPos {
  int b, kvh;  // unit
  int n;       // its steps
  long g;      // global position where its cost range starts
};

// The prologue reads the context lengths once: the first kLocRegs * 64 stay
// in registers for the search after the total (later ones are read again).
constexpr int kLocRegs = 4;
struct LocCache {
  int c[kLocRegs];
};

// Cost (steps + kUnitCost per unit) per KV head summed over all sequences
// (identical in every wave).
__device__ long total_steps_per_head(const DecodeArgs& a, LocCache& lc) {
  const int lane = threadIdx.x & 63;
  long acc = 0;
#pragma unroll
  for (int i = 0; i < kLocRegs; ++i) {
    const int b = 64 * i + lane;
    lc.c[i] = b < a.num_seqs ? a.ctx_lens[b] : 0;
  }
#pragma unroll
  for (int i = 0; i < kLocRegs; ++i)
    if (64 * i + lane < a.num_seqs) acc += unit_steps(lc.c[i]) + kUnitCost;
  for (int base = 64 * kLocRegs; base < a.num_seqs; base += 256) {
    int c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = base + 64 * i + lane;
      c[i] = b < a.num_seqs ? a.ctx_lens[b] : 0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (base + 64 * i + lane < a.num_seqs) acc += unit_steps(c[i]) + kUnitCost;
  }
  return wave_sum_l(acc);
}

// The sequence whose cost range in one KV head's position space holds s0
// (< total), and its context.  A sequence's range is kUnitCost positions of
// overhead followed by its steps.  Wave-uniform result; the caller sets the
// head.
__device__ UnitPos locate(const DecodeArgs& a, long s0, const LocCache& lc, int& ctx) {
  const int lane = threadIdx.x & 63;
  long run = 0;  // positions before this chunk
  UnitPos p{0, 0, 1, 0};
  ctx = 0;
  auto chunk = [&](int base, int cv) -> bool {
    const int b = base + lane;
    const int n = b < a.num_seqs ? unit_steps(cv) : 0;
    const long c = b < a.num_seqs ? n + kUnitCost : 0;
    const long incl = wave_incl_scan_l(c);
    const long first = run + incl - c;  // first position of sequence b
    const long last = run + incl;       // one past its last
    const unsigned long long hit =
        __builtin_amdgcn_ballot_w64(b < a.num_seqs && first <= s0 && s0 < last);
    if (hit) {
      const int l = __builtin_ffsll((long long)hit) - 1;
      p.b = base + l;
      p.n = __builtin_amdgcn_readfirstlane(__shfl(n, l));
      p.g = uniform_l(__shfl(first, l));
      ctx = __builtin_amdgcn_readfirstlane(__shfl(clamp_ctx(cv), l));
      return true;
    }
    run += uniform_l(__shfl(incl, 63));
    return false;
  };
#pragma unroll
  for (int i = 0; i < kLocRegs; ++i)
    if (64 * i < a.num_seqs && chunk(64 * i, lc.c[i])) return p;
  for (int base = 64 * kLocRegs; base < a.num_seqs; base += 64) {
    const int b = base + lane;
    if (chunk(base, b < a.num_seqs ? a.ctx_lens[b] : 0)) return p;
  }
  return p;
}

// Partial pieces travel between waves that may sit on different XCDs, whose
// L2 caches are not coherent with each other.  They are written and read
// with device-scope (sc1) buffer accesses, which go through to / come from
// the device's coherence point, so publishing a piece needs only a wait for
// its stores to complete, not a device-wide cache write-back.
constexpr int kCoherent = 16;  // cache-policy bit sc1 (device scope)
// A buffer offset past every buffer's records (ws_rsrc sets 0x7fffffff): a
// load from it returns zeros without touching memory.
constexpr uint32_t kPastRecords = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// A wave-uniform element read with a scalar load (through the constant
// address space), so that it neither takes a VGPR nor joins the vector-load
// counter: waiting for it never waits for K/V loads in flight.  The array
// must not change during the kernel.
__device__ __forceinline__ int uniform_load(const int32_t* p, int i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

// Compiler barriers around an explicit wait, so no memory access is moved
// across it.
__device__ __forceinline__ void wait_vm_all() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ void wait_lgkm_all() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <class CT, class KVT, class ST, int D, int NT, bool BIG>
__global__ __launch_bounds__(64 * kWavesPerGroup) void decode_kernel(const DecodeArgs a) {
  typedef AttnCore<CT, KVT, ST, D, NT> Core;
  typedef typename CT::storage q_t;
  constexpr int J = Core::J;
  // split-K pieces loaded per round trip of a merge (one piece of 16 rows
  // at head_dim 256 is 64 VGPRs)
  constexpr int kMergeBatch = J <= 4 ? 4 : J <= 8 ? 2 : 1;
  const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerGroup + (threadIdx.x >> 6));
  if (wave >= a.num_waves) return;
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int H = a.num_kv_heads, G = a.group, Tq = a.q_per_seq;
  const q_t* q = reinterpret_cast<const q_t*>(a.q);
  q_t* out = reinterpret_cast<q_t*>(a.out);

  // ---- this wave's slice.  Waves form groups of H; a group takes the slice
  // [s0, s1) of one KV head's position space (sequences laid end to end)
  // and wave h of the group runs KV head h of it.  The H waves of a group
  // walk the same blocks at the same pace, so each block's K (and V) rows
  // of all heads -- one contiguous run of H slabs -- are fetched together.
  const int NG = max(1, a.num_waves / H);
  const int grp = wave / H, head = wave - grp * H;
  if (grp >= NG) return;
  LocCache lc;
  const long total = uniform_l(total_steps_per_head(a, lc));
  const long per = max((long)a.min_steps, (total + NG - 1) / NG);
  const long s0 = grp * per;
  if (s0 >= total) return;
  const long s1 = min(total, s0 + per);
  int ctx = 0;
  UnitPos u = locate(a, s0, lc, ctx);
  u.kvh = head;

  const typename Core::LaneOff lo = Core::lane_off();
  constexpr int DEP = ring_depth<D, KVT, NT>();
  constexpr int NB = DEP + 1;
  // A ring of DEP + 1 register buffers, unrolled so every index is a
  // compile-time constant: DEP steps of loads stay in flight while a step
  // computes, and no buffer is ever copied (a register copy of data still in
  // flight would make the compiler wait for it).
  typename Core::Raw rb[NB];
  auto make_pv = [&](const UnitPos& uu, int c) -> PoolView {
    return PoolView{a.k, a.v, a.ks, a.vs, a.tables + (long)uu.b * a.table_stride, a.table_stride,
                    uu.kvh, H, a.bs_log2, a.num_blocks, c};
  };

  // Query rows of unit uu, and the key limit of each row for context c.
  auto row_off = [&](const UnitPos& uu, int r) -> long {
    const int t = r / G, hh = r - t * G;
    return ((long)(uu.b * Tq + t) * a.num_q_heads + uu.kvh * G + hh) * D;
  };
  auto load_rows = [&](Core& core, const UnitPos& uu) {
    const q_t* rowq[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int r = nt * 16 + n;
      rowq[nt] = r < a.rows ? q + row_off(uu, r) : nullptr;
    }
    core.load_q(rowq);
  };

  // ---- per-wave LDS staging of table windows.  While a unit streams, the
  // next unit's first table window and the current unit's next window are
  // copied into LDS by direct global->LDS loads: no VGPR holds them and no
  // wait covers them until they are taken, by which time they have landed,
  // so neither a unit boundary nor a window refill waits for a table read
  // with K/V loads in flight.  (Query rows need no staging: loaded before a
  // unit's first K/V steps, they arrive with them.)
  __shared__ __attribute__((aligned(16))) uint32_t lds_windows[kWavesPerGroup][2][128];
  void* const lds_wnext = lds_windows[threadIdx.x >> 6][0];
  void* const lds_refill = lds_windows[threadIdx.x >> 6][1];
  // one step's loads; with block_size >= 16 the table window moves on by 128
  // entries when a step passes it, to the copy staged when the current window
  // was installed (64 or more steps ago: landed, since every later step's
  // data has been waited for), and the window after it is staged
  auto advance_window = [&](const PoolView& v, TableWindow& w, int key0, bool enable) {
    if (enable && key0 < v.ctx && (min(key0 + 31, v.ctx - 1) >> a.bs_log2) >= w.limit) {
      w.fill_lds(reinterpret_cast<const uint32_t*>(lds_refill), w.limit);
      wait_lgkm_all();
      stage_window(lds_refill, v.table, v.table_stride, w.limit);
    }
  };
  auto load_step = [&](const PoolView& v, TableWindow& w, int key0, typename Core::Raw& r, bool enable) {
    if constexpr (BIG) {
      advance_window(v, w, key0, enable);
      Core::load_big(v, w, key0, lo, r, enable);
    } else {
      Core::template load_sel<false>(v, w, key0, lo, r, enable);
    }
  };
  auto issue_first = [&](const PoolView& v, TableWindow& w, int first, int end) {
#pragma unroll
    for (int k = 0; k < DEP; ++k) load_step(v, w, 32 * (first + k), rb[k], first + k < end);
  };

  // ---- the first unit: its query rows, its table window, then its first
  // DEP steps of loads (in that order: waiting for the rows does not wait
  // for the K/V steps behind them)
  int lbeg = (int)max(s0 - (u.g + kUnitCost), 0L);  // first local step of the unit in the slice
  long sb = u.g + kUnitCost;  // global position of the unit's step 0
  int lend = (int)min((long)u.n, s1 - sb);  // steps of this unit in the slice: [lbeg, lend)
  if (lend <= lbeg) return;  // the slice ends inside the unit's overhead: the next group has it
  Core core;
  load_rows(core, u);
  PoolView pv = make_pv(u, ctx);
  TableWindow win;
  const int wb0 = (32 * lbeg) >> a.bs_log2;
  if (BIG && ctx > 0) {
    win.fill(pv.table, pv.table_stride, wb0);
    stage_window(lds_refill, pv.table, pv.table_stride, wb0 + 128);
  }
  if (ctx > 0) issue_first(pv, win, lbeg, lend);
  bool first_unit = true;

  for (;;) {
    // ---- unit prologue: the query rows (already requested) and row limits
    int rowlim[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int r = nt * 16 + n;
      rowlim[nt] = r < a.rows ? max(ctx - Tq + r / G + 1, 0) : max(ctx, 0);
    }
    const int minlim = max(ctx - Tq + 1, 0);
    core.start(rowlim);

    // ---- what the next unit (the next sequence, same head) needs to start:
    // its context (a scalar load) and first table window (staged in LDS),
    // requested now so that both are in place long before this unit ends.
    // The LDS copy of this unit's window was read (and waited for) before
    // this one overwrites it.
    const bool has_next = sb + lend < s1;
    int ctx_raw_n = 0;
    if (has_next) {
      ctx_raw_n = uniform_load(a.ctx_lens, u.b + 1);  // waited for at the boundary
      if (BIG) stage_window(lds_wnext, a.tables + (long)(u.b + 1) * a.table_stride, a.table_stride, 0);
    }

    // ---- stream the unit's steps [lbeg, lend); the first DEP are in flight
    if (ctx > 0) {
      bool done = false;
      for (int st = lbeg; !done; st += NB) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
          if (!done) {
            const int cur = st + k;
            load_step(pv, win, 32 * (cur + DEP), rb[(k + DEP) % NB], cur + DEP < lend);
            core.compute(rb[k], 32 * cur, a.scale_log2, 32 * cur + 32 > minlim, ctx);
            done = cur + 1 >= lend;
          }
        }
      }
    }

    // ---- the next unit's query rows, window and first DEP steps of loads
    // go out before this unit's epilogue, so they overlap its latency.  The
    // loads still in flight are this unit's trailing empty prefetches and
    // its staged window, long landed: waiting for them costs little.
    wait_vm_all();
    UnitPos un = u;
    int ctx_n = 0, lend_n = 0;
    if (has_next) {
      un.g += u.n + kUnitCost;
      ++un.b;
      un.n = unit_steps(ctx_raw_n);
      ctx_n = clamp_ctx(ctx_raw_n);
      lend_n = (int)min((long)un.n, s1 - (un.g + kUnitCost));
    }
    const bool go_next = has_next && lend_n > 0;
    const PoolView pv_n = make_pv(un, ctx_n);
    float lrow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) lrow[nt] = core.row_l(nt);
    TableWindow win_n;
    if (go_next) {
      load_rows(core, un);  // the epilogue below reads o, m and l, not the query rows
      if (BIG) win_n.fill_lds(reinterpret_cast<const uint32_t*>(lds_wnext), 0);
      wait_lgkm_all();
      if (BIG && ctx_n > 0) stage_window(lds_refill, pv_n.table, pv_n.table_stride, 128);
      if (ctx_n > 0) issue_first(pv_n, win_n, 0, lend_n);
    }

    // ---- output rows: the lane holds the 4J contiguous dims [4Jg, 4Jg + 4J)
    // of row r (element (j, i) of the accumulators at J*i + j), stored in
    // 16-byte pieces
    auto store_row = [&](const UnitPos& uu, int r, const float* vals, float inv) {
      if (4 * J * g >= D) return;  // head_dim below 16: lanes past it hold nothing
      q_t* orow = out + row_off(uu, r) + 4 * J * g;
      if constexpr (sizeof(q_t) == 2) {
        uint32_t w[2 * J];
#pragma unroll
        for (int k = 0; k < 2 * J; ++k)
          w[k] = (uint32_t)Cvt<CT>::from_f32(vals[2 * k] * inv) | ((uint32_t)Cvt<CT>::from_f32(vals[2 * k + 1] * inv) << 16);
        if constexpr (2 * J >= 4) {
#pragma unroll
          for (int c = 0; c < 2 * J / 4; ++c)
            *reinterpret_cast<u32x4*>(orow + 8 * c) = (u32x4){w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
        } else {
          *reinterpret_cast<u32x2*>(orow) = (u32x2){w[0], w[1]};
        }
      } else {
#pragma unroll
        for (int c = 0; c < J; ++c)
          *reinterpret_cast<f32x4*>(orow + 4 * c) =
              (f32x4){vals[4 * c] * inv, vals[4 * c + 1] * inv, vals[4 * c + 2] * inv, vals[4 * c + 3] * inv};
      }
    };
    // Merges the pieces of unit uu (held by groups wa_..wb_; group p's in
    // the slots of wave p H + head, group wa_'s first or second slot per
    // slot_a_) in piece order and stores its output rows.  This wave's own
    // piece comes from its registers -- the exact values it would have
    // stored -- and every other from the workspace, so the result does not
    // depend on which wave merges.
    const __amdgpu_buffer_rsrc_t ro = ws_rsrc(a.ws_o), rml = ws_rsrc(a.ws_ml);
    // A piece's O is stored lane-major: a slot holds a.rows * 4J 16-byte
    // chunks; n-tile nt (rt rows) starts at chunk 64 J nt, and its chunk c
    // holds the 16 bytes of each lane (n, g) with n < rt at g rt + n, so each
    // store (and load) instruction moves 64 rt consecutive bytes.  Row-major
    // pieces made each instruction 48 partial-line writes through to the
    // coherence point, several microseconds per published piece under the
    // K/V stream.  o_chunk is chunk 0's offset; chunk c is 64 rt c further.
    auto o_rt = [&](int nt) { return min(16, a.rows - 16 * nt); };
    auto o_chunk = [&](long sl, int nt) -> uint32_t {
      return (uint32_t)(((sl * a.rows + 16 * nt) * 4 * J + g * o_rt(nt) + n) * 16);
    };
    auto merge_pieces = [&](const UnitPos& uu, int wa_, int wb_, long slot_a_) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int r = nt * 16 + n;
        if (r >= a.rows) continue;
        float own[4 * J];
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) own[J * i + j] = core.out_val(nt, j, i);
        // running merge over pieces in order: (M, L, acc) rescaled as each
        // piece's (m, l, O) arrives
        float M = -INFINITY, L = 0.f;
        float acc[4 * J];
#pragma unroll
        for (int e = 0; e < 4 * J; ++e) acc[e] = 0.f;
        // pieces go in batches of kMergeBatch: a batch's loads are all issued
        // before its first piece is merged, so a unit cut into P pieces
        // waits ceil(P / kMergeBatch) round trips, not P
        for (int p0 = wa_; p0 <= wb_; p0 += kMergeBatch) {
          u32x2 ml[kMergeBatch];
          u32x4 ov[kMergeBatch][J];
#pragma unroll
          for (int k = 0; k < kMergeBatch; ++k) {
            const int p = p0 + k;
            // this wave's own piece, and pieces past wb_, read nothing: an
            // offset past the buffer's records returns zeros
            const bool ld = p <= wb_ && p != grp;
            const long sl = p == wa_ ? slot_a_ : 2L * (p * H + head);
            ml[k] = __builtin_amdgcn_raw_buffer_load_b64(rml, ld ? (uint32_t)((sl * a.rows + r) * 8) : kPastRecords,
                                                         0, kCoherent);
            const uint32_t ob = o_chunk(sl, nt);
#pragma unroll
            for (int c = 0; c < J; ++c)
              ov[k][c] = __builtin_amdgcn_raw_buffer_load_b128(ro, ld ? ob + 64 * o_rt(nt) * c : kPastRecords, 0,
                                                               kCoherent);
          }
#pragma unroll
          for (int k = 0; k < kMergeBatch; ++k) {
            const int p = p0 + k;
            if (p > wb_) break;
            float mp, lp, val[4 * J];
            if (p == grp) {
              mp = core.m[nt];
              lp = lrow[nt];
#pragma unroll
              for (int e = 0; e < 4 * J; ++e) val[e] = own[e];
            } else {
              // elements are copied out before bit_cast: a bit_cast applied
              // to an ext_vector element reads element 0 (hipcc 7.2)
#pragma unroll
              for (int c = 0; c < J; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const uint32_t oe = ov[k][c][e];
                  val[4 * c + e] = __builtin_bit_cast(float, oe);
                }
              const uint32_t m0 = ml[k][0], l0 = ml[k][1];
              mp = __builtin_bit_cast(float, m0);
              lp = __builtin_bit_cast(float, l0);
            }
            const float Mn = fmaxf(M, mp);
            const float Mref = Mn == -INFINITY ? 0.f : Mn;
            const float sa = __builtin_amdgcn_exp2f(M - Mref), sp = __builtin_amdgcn_exp2f(mp - Mref);
            L = __builtin_fmaf(L, sa, lp * sp);
#pragma unroll
            for (int e = 0; e < 4 * J; ++e) acc[e] = __builtin_fmaf(acc[e], sa, val[e] * sp);
            M = Mn;
          }
        }
        store_row(uu, r, acc, L > 0.f ? 1.f / L : 0.f);
      }
    };


    // ---- unit epilogue
    const bool finish = lbeg == 0 && lend == u.n;  // the whole unit is in this slice
    if (!finish) {
      // A piece of a unit cut by slice boundaries.  Group p's piece sits in
      // the slots of wave p H + head; group wa, whose slice ends in the unit,
      // saw the unit first iff its slice began inside the unit's range.
      const int wa = (int)(sb / per), wb = (int)((sb + u.n - 1) / per);  // groups holding the pieces
      const int unit = u.b * H + u.kvh;
      const long slot = 2L * wave + (first_unit ? 0 : 1);
      const long slot_a = 2L * (wa * H + head) + ((long)wa * per >= u.g ? 0 : 1);
      // With two pieces, group wa's holds the unit's first steps, streamed at
      // the end of its slice, while group wb streamed the rest at the start
      // of its own: wa is almost always the last to finish.  It first reads
      // the count; if the other piece is in, it merges at once from its own
      // registers and never publishes.  (With more pieces the middle ones
      // span whole slices and end with wa's, so the read rarely pays.)
      bool merge = false;
      if (grp == wa && wb == wa + 1) {
        int seen = 0;
        if (lane == 0) seen = __hip_atomic_load(a.counters + unit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        merge = __builtin_amdgcn_readfirstlane(seen) == wb - wa;
      }
      if (!merge) {
        // publish this piece
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int r = nt * 16 + n;
          if (r >= a.rows) continue;
          // the lane's 4J dims are contiguous from 4Jg, element (j, i) at
          // J*i + j (dims past D hold values no merge uses)
          float tmp[4 * J];
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) tmp[J * i + j] = core.out_val(nt, j, i);
          const uint32_t ob = o_chunk(slot, nt);
#pragma unroll
          for (int c = 0; c < J; ++c)
            __builtin_amdgcn_raw_buffer_store_b128(
                (u32x4){__builtin_bit_cast(uint32_t, tmp[4 * c]), __builtin_bit_cast(uint32_t, tmp[4 * c + 1]),
                        __builtin_bit_cast(uint32_t, tmp[4 * c + 2]), __builtin_bit_cast(uint32_t, tmp[4 * c + 3])},
                ro, ob + 64 * o_rt(nt) * c, 0, kCoherent);
          if (g == 0)
            __builtin_amdgcn_raw_buffer_store_b64(
                (u32x2){__builtin_bit_cast(uint32_t, core.m[nt]), __builtin_bit_cast(uint32_t, lrow[nt])}, rml,
                (uint32_t)((slot * a.rows + r) * 8), 0, kCoherent);
        }
        // count it in once its stores are complete (hence visible device-wide)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        int old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(a.counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        merge = __builtin_amdgcn_readfirstlane(old) == wb - wa;
      }
      if (merge) {
        if (lane == 0) __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        merge_pieces(u, wa, wb, slot_a);
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int r = nt * 16 + n;
        if (r < a.rows) {
          float vals[4 * J];
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) vals[J * i + j] = ctx > 0 ? core.out_val(nt, j, i) : 0.f;
          store_row(u, r, vals, lrow[nt] > 0.f ? 1.f / lrow[nt] : 0.f);
        }
      }
    }

    if (!go_next) break;
    u = un;
    ctx = ctx_n;
    sb = un.g + kUnitCost;
    lbeg = 0;
    lend = lend_n;
    pv = pv_n;
    win = win_n;
    first_unit = false;
  }
}

// ------------------------------------------------------------------ dispatch
// A launcher sets a.num_waves (at most `cap`) to what the device keeps
// resident at once, so that every wave's slice streams concurrently.
typedef int (*DecodeFn)(DecodeArgs&, int cap, hipStream_t);

static int device_cus() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

template <class CT, class KVT, class ST, int D, int NT, bool BIG>
int launch_decode_kernel(DecodeArgs& a, int cap, hipStream_t s) {
  static int groups_per_cu = 0;
  if (!groups_per_cu) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, reinterpret_cast<const void*>(&decode_kernel<CT, KVT, ST, D, NT, BIG>),
            64 * kWavesPerGroup, 0) != hipSuccess || nb <= 0)
      nb = 1;
    groups_per_cu = nb;
  }
  const long resident = (long)device_cus() * groups_per_cu * kWavesPerGroup;
  // whole groups of num_kv_heads waves, at least one; a single group never
  // cuts a unit, so it needs no workspace slots even when cap is smaller
  const long H = a.num_kv_heads;
  long nw = std::min<long>(cap, resident);
  nw = std::max(H, nw - nw % H);
  a.num_waves = (int)nw;
  const unsigned groups = (unsigned)((a.num_waves + kWavesPerGroup - 1) / kWavesPerGroup);
  hipLaunchKernelGGL((decode_kernel<CT, KVT, ST, D, NT, BIG>), dim3(groups), dim3(64 * kWavesPerGroup),
                     0, s, a);
  return check_launch("hpa_paged_decode");
}

template <class CT, class KVT, class ST, int D, int NT>
int launch_decode(DecodeArgs& a, int cap, hipStream_t s) {
  // block_size >= 16 takes the scalar-addressed fast path
  if (a.bs_log2 >= 4) return launch_decode_kernel<CT, KVT, ST, D, NT, true>(a, cap, s);
  return launch_decode_kernel<CT, KVT, ST, D, NT, false>(a, cap, s);
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

// Kernel tables, one per (compute type, KV storage, scale type); each is
// instantiated in its own translation unit (hpa_decode_<q>_<kv>.hip) so the
// builds run in parallel.
#define HPA_DECODE_TABLES(X) \
  X(F32, F32, F32)           \
  X(F32, I8, F16)            \
  X(F32, I8, F32)            \
  X(F16, F16, F32)           \
  X(F16, I8, F16)            \
  X(F16, I8, F32)            \
  X(BF16, BF16, F32)         \
  X(BF16, I8, F16)           \
  X(BF16, I8, F32)
#define HPA_EXTERN_TABLE(CT, KVT, ST) extern template DecodeFn pick_d<CT, KVT, ST>(int, int);
HPA_DECODE_TABLES(HPA_EXTERN_TABLE)
#undef HPA_EXTERN_TABLE

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

}  // namespace hpa
