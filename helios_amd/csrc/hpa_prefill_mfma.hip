// Chunked-prefill / verify attention for fp16 and bf16 pools on gfx950:
// LDS-shared K/V tiles and 32x32x16 MFMAs.
//
// Same contract as prefill_kernel (hpa_prefill.hip): sequence b owns query
// tokens [cu_q[b], cu_q[b+1]); its token i sits at position q_pos[b] + i and
// attends keys [0, min(q_pos[b] + i + 1, ctx[b])) -- helios' causal rule
// (reference exec/paged_attn.py:401-404).  A verify launch (uniform_q > 0,
// from hpa_paged_decode) gives every sequence uniform_q tokens ending at
// ctx[b] - 1 and reads neither cu_q nor q_pos.
//
// A workgroup of four waves owns 128 consecutive (token, head-in-group) rows
// of one (sequence, KV head); each wave owns 32 of them, one 32x32 MFMA tile.
// The workgroup walks the keys in steps of 32.  Every step's K and V tiles
// (32 keys x head_dim each) are copied once from the paged pool into LDS by
// direct global->LDS buffer loads issued by all four waves, four steps ahead
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
// wants one head dim across 8 keys per lane; ds_read_b64_tr_b16 delivers it
// straight from the key-major V tile: within each group of 16 lanes, output
// lane i receives element i % 4 of the 8 bytes addressed by lanes i / 4 + 4j
// (j = 0..3), so lanes 4j + c address key j, dims 4c..4c+3, and lane i ends up
// with dim i of keys 0..3 (layout measured on gfx950).
//
// LDS rows are 16-byte chunks XOR-swizzled per key row: K chunk j of row r sits
// at position j ^ (r % chunks_per_row), so the K reads (16 keys x one chunk)
// hit distinct banks; V chunk j sits at j ^ kVSwz[r % 4], which keeps the
// transpose reads (4 keys x 4 chunks per 32 lanes, 4 keys x 2 chunks per 16)
// conflict-free for 64 banks and for 32.  The global->LDS loads apply the
// inverse permutation on the global side, so the per-lane LDS destinations
// stay the hardware's consecutive ones.
//
// INT8 pools (QuantizedPagedKVCache) run the same MFMA path on dequantised
// tiles.  The int8 K/V rows of a step and their per-(token, head) scales are
// copied into LDS stages by the same direct loads; one step ahead of the
// compute, each wave dequantises exactly the 16 keys of one tensor it copied
// (so only its own load count, no barrier, guards the read) into one of two
// fp16/bf16 tiles laid out and swizzled like the fp16 path's, as
// (q * s).to(dtype) -- the reference's gather, exec/paged_attn.py:213-235.
// The step's barrier then publishes that tile and frees the other one.
#include <type_traits>

#include "hpa_attn_core.h"
#include "hpa_host.h"
#include "hpa_prefill.h"

namespace hpa {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

template <class CT> struct M32;
template <> struct M32<F16> {
  __device__ __forceinline__ static f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                  c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float x, float y) {
    return __builtin_bit_cast(uint32_t, (f16x2){(_Float16)x, (_Float16)y});  // v_cvt_pk_f16_f32, RNE
  }
  // acc + both halves of w, in fp32
  __device__ __forceinline__ static float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), (f16x2){1, 1}, acc, false);
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
    return __builtin_bit_cast(uint32_t, (bf16x2){(__bf16)x, (__bf16)y});  // v_cvt_pk_bf16_f32, RNE
  }
  __device__ __forceinline__ static float lo_of(uint32_t w) { return bf16_bits_to_f32(w & 0xffffu); }
  __device__ __forceinline__ static float hi_of(uint32_t w) { return bf16_bits_to_f32(w >> 16); }
};

// (q * s).to(CT) of the 4 NW int8 values in `in` (little-endian bytes) with
// one scale (raw ST bits), two values per output word: the reference's
// dequantisation, exec/paged_attn.py:213-235 (fp32 product, then the
// compute dtype).  Each value is rounded once, as there.
template <class CT, class ST, int NW>
__device__ __forceinline__ void dequant_words(const uint32_t* in, uint32_t sbits, uint32_t* out) {
#pragma clang fp contract(off)
  if constexpr (std::is_same<CT, F16>::value && std::is_same<ST, F16>::value) {
    // [q ^ 0x80, 0x64] is the fp16 value 1152 + q; less 1152 is q exactly,
    // and the fp16 product with the fp16 scale is q * s rounded once to fp16
    // (the fp32 product of an 8-bit and an 11-bit significand is exact)
    const f16x2 off = {(_Float16)-1152.f, (_Float16)-1152.f};
    const f16x2 sv = __builtin_bit_cast(f16x2, (sbits & 0xffffu) * 0x10001u);
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t x = in[w] ^ 0x80808080u;
      const f16x2 lo = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) + off;
      const f16x2 hi = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) + off;
      out[2 * w] = __builtin_bit_cast(uint32_t, lo * sv);
      out[2 * w + 1] = __builtin_bit_cast(uint32_t, hi * sv);
    }
  } else {
    // fp32: byte q ^ 0x80 = q + 128 exactly; fma(q + 128, s, -128 s) is
    // q * s rounded once to fp32 (-128 s is exact), then rounded to CT.  The
    // empty asm keeps the compiler from fusing the two roundings into one
    // mixed-precision fma: with fp32 scales the product is not exact, and
    // the reference rounds it to fp32 first.
    const float s = std::is_same<ST, F16>::value ? f16_bits_to_f32(sbits & 0xffffu) : __builtin_bit_cast(float, sbits);
    const float c = -128.f * s;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t x = in[w] ^ 0x80808080u;
      float f[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) f[k] = __builtin_fmaf((float)((x >> (8 * k)) & 0xffu), s, c);
      asm volatile("" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
      out[2 * w] = M32<CT>::pack(f[0], f[1]);
      out[2 * w + 1] = M32<CT>::pack(f[2], f[3]);
    }
  }
}

constexpr int kPfWaves = 4;              // waves per workgroup, 32 rows each
constexpr int kPfRows = 32 * kPfWaves;   // rows per workgroup
constexpr int kPfStages = 5;             // LDS tiles: copies run kPfStages - 1 steps ahead
constexpr int kPfLazy = 8;               // rescale only when a row max grows by > 2^8

// V-tile chunk swizzle by key row % 4 (chunks_per_row 16 and 8)
__device__ __forceinline__ constexpr int v_swz(int nch, int row) {
  return nch == 16 ? (row & 3) * 4 + ((row & 2) ? 2 : 0) : (row & 3) * 2;
}


// Work item i is the (i / units)-th heaviest row tile of unit i % units.
// Workgroups go to the 8 XCDs round-robin by id and, within an XCD, start in
// id order as slots free up.  The workgroup with id 8m + x runs the item of
// rank m -- by step count, longest first, ties by id -- among the items
// 8j + x, so each XCD schedules its own items longest-first (list
// scheduling's LPT rule) and a unit's tiles stay on one XCD's L2 whenever the
// unit count is a multiple of 8.  Returns steps + 1, or 0 for an empty tile.
__device__ __forceinline__ int item_cost(const PrefillArgs& a, int item, int units, int tiles) {
  const int unit = item % units, tile = tiles - 1 - item / units;
  const int b = unit / a.num_kv_heads;
  const SeqSpan sp = seq_span(a, b);
  const int rows = sp.qn * a.group;
  if (tile * kPfRows >= rows) return 0;
  const int rlast = min(tile * kPfRows + kPfRows - 1, rows - 1);
  const int lim = max(min(sp.pos0 + rlast / a.group + 1, a.ctx_lens[b]), 0);
  return ((lim + 31) >> 5) + 1;
}

// 4 x b16 transposed across each 16-lane group (see the layout above),
// issued through inline asm.  With the builtin, the compiler's wait pass
// cannot tell the read from the global->LDS copies still in flight and puts
// a vmcnt(0) before it, which drains every copy issued ahead; the copies are
// ordered by the kernel's own per-wave vmcnt waits and the step barrier
// instead.  The compiler does not track the asm's result, so the step waits
// for its reads with an explicit lgkmcnt(0) before any use of them.
template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr(uint32_t lds_addr) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(lds_addr), "i"(OFF));
  return r;
}

// LDS address of a pointer into the kernel's shared array
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

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

template <class CT, class KVT, class ST, int D>
__global__ __launch_bounds__(64 * kPfWaves, 2) void prefill_mfma_kernel(const PrefillArgs a,
                                                                     const int32_t* __restrict__ tables,
                                                                     int tiles_per_unit) {
  typedef M32<CT> M;
  typedef typename CT::storage q_t;
  constexpr bool QUANT = std::is_same<KVT, I8>::value;
  constexpr int NCH = D / 8;          // 16-byte chunks per key row
  constexpr int ROWB = D * 2;         // bytes per key row
  constexpr int TILEB = 32 * ROWB;    // one 32-key tile of K or of V
  constexpr int KCH = D / 16;         // QK MFMAs per step
  constexpr int DB = D / 32;          // PV MFMAs per 16-key chunk: O^T block db = dims [32db, 32db + 32)
  constexpr int IPW = NCH / 4;        // global->LDS instructions per wave per step
  // int8: a wave copies 16 keys x D bytes (R8) plus one scale per lane, and
  // dequantises them; NS stages run NS - 2 steps ahead of the dequantisation
  constexpr int R8 = 16 * D;
  constexpr int IPW8 = R8 / 1024;
  constexpr int G8 = IPW8 + 1;        // loads per wave per step
  constexpr int NS = QUANT ? 6 : kPfStages;
  constexpr int SSZ = QUANT ? (int)sizeof(typename ST::storage) : 4;
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(kPfStages >= 3 && (kPfStages - 2) * IPW <= 15 && (!QUANT || (NS - 2) * G8 <= 15),
                "the copy waits below fit vmcnt's low four bits");
  // fp pools: NS stages of [K tile | V tile].  int8 pools: two dequantised
  // [K tile | V tile] buffers, then NS int8 stages of 4 wave regions.
  constexpr int SMEM = QUANT ? 2 * 2 * TILEB + NS * 4 * R8 : NS * 2 * TILEB;
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  // ---- which (unit, row tile) this workgroup runs: longest-first per XCD
  const int units = a.num_seqs * a.num_kv_heads;
  int item = (int)blockIdx.x;
  {
    // the pick lives in the last stage, which is first written after the
    // first step's barrier (every wave has read the pick by then)
    int& s_pick = *reinterpret_cast<int*>(&smem[SMEM - 4]);
    const int xcd = item & 7, m = item >> 3;
    const int nk = ((int)gridDim.x - xcd + 7) >> 3;  // items on this XCD
    if (nk <= kLptMax)
      item = lpt_pick<64 * kPfWaves>(reinterpret_cast<int*>(&smem[0]), &s_pick, nk, m, xcd,
                                     [&](int j) { return item_cost(a, 8 * j + xcd, units, tiles_per_unit); });
  }
  const int unit = item % units;
  const int tile = tiles_per_unit - 1 - item / units;
  const int b = unit / a.num_kv_heads, kvh = unit - b * a.num_kv_heads;
  const int G = a.group;
  const SeqSpan sp = seq_span(a, b);
  const int q0 = sp.q0;
  const int rows = sp.qn * G;
  if (tile * kPfRows >= rows) return;  // uniform over the workgroup, before any barrier
  const int ctx = a.ctx_lens[b];
  const int pos0 = sp.pos0;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, n = lane & 31;
  auto limit = [&](int r) -> int { return max(min(pos0 + r / G + 1, ctx), 0); };

  const int r0 = tile * kPfRows + 32 * w;           // this wave's first row
  const int r = r0 + n;                             // this lane's row
  const bool rv = r < rows;
  const int lim = rv ? limit(r) : 0;
  // wave- and workgroup-uniform limits, pinned to scalar registers (the
  // compiler would otherwise merge them with the per-lane limit above)
  const bool wave_live = r0 < rows;
  const int wave_minlim = __builtin_amdgcn_readfirstlane(wave_live ? limit(r0) : 0);
  const int wave_maxlim = __builtin_amdgcn_readfirstlane(wave_live ? limit(min(r0 + 31, rows - 1)) : 0);
  const int wg_maxlim = limit(min(tile * kPfRows + kPfRows - 1, rows - 1));
  const int nsteps = __builtin_amdgcn_readfirstlane((wg_maxlim + 31) >> 5);

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
    const int swz = tensor ? v_swz(NCH, row) : row % NCH;
    voff[i] = (uint32_t)((row & 15) * ROWB + (q ^ swz) * 16);
  }
  const char* pool = reinterpret_cast<const char*>(tensor ? a.v : a.k);
  const char* spool = reinterpret_cast<const char*>(tensor ? a.vs : a.ks);
  uint32_t sc[NS];  // int8: this lane's key scale, per stage (raw bits)
  const long blk_rows = (long)a.num_kv_heads << a.bs_log2;   // key rows per block
  const long head_rows = (long)kvh << a.bs_log2;
  const int bsm = (1 << a.bs_log2) - 1;
  const int32_t* trow = tables + (long)b * a.table_stride;
  TableWindow win;
  if (nsteps > 0) win.fill(trow, a.table_stride, 0);
  auto issue_loads = [&](int step, int stage) {
    const int key0 = step * 32 + 16 * half;
    // rows past the context read as zeros; a step past the last one issues
    // empty copies, so every step has the same loads in flight
    int valid = step < nsteps ? min(max(ctx - key0, 0), 16) : 0;
    int phys = 0;
    if (valid > 0) {
      const int lb = key0 >> a.bs_log2;
      if (!win.covers(lb)) win.fill_sync(trow, a.table_stride, lb);
      phys = win.get(lb);
      if ((unsigned)phys >= (unsigned)a.num_blocks) { phys = 0; valid = 0; }
    }
    if constexpr (QUANT) {
      // 16 consecutive int8 rows of one block, copied as they lie: lane l's
      // 16 bytes of instruction i land at region + 1024 i + 16 l
      const long row0 = (long)phys * blk_rows + head_rows + (key0 & bsm);
      const int nbytes = __builtin_amdgcn_readfirstlane(valid * D);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(pool + row0 * D), (short)0, nbytes, 0x00020000);
      uint8_t* dst = &smem[2 * 2 * TILEB + stage * 4 * R8 + w * R8];
#pragma unroll
      for (int i = 0; i < IPW8; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16,
                                                 i * 1024 + lane * 16, 0, 0, 0);
      // the scale of the key this lane dequantises (key lane / 4); rows past
      // the context read as 0
      const int sbytes = __builtin_amdgcn_readfirstlane(valid * SSZ);
      const __amdgpu_buffer_rsrc_t srs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(spool + row0 * SSZ), (short)0, sbytes, 0x00020000);
      if constexpr (SSZ == 2)
        sc[stage] = __builtin_amdgcn_raw_buffer_load_b16(srs, (lane >> 2) * 2, 0, 0);
      else
        sc[stage] = __builtin_amdgcn_raw_buffer_load_b32(srs, (lane >> 2) * 4, 0, 0);
    } else {
      const char* base = pool + ((long)phys * blk_rows + head_rows + (key0 & bsm)) * ROWB;
      // the record count is computed on the VALU (min/max); pinning it to a
      // scalar keeps the resource uniform, with no per-lane loop around the loads
      const int nbytes = __builtin_amdgcn_readfirstlane(valid * ROWB);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, nbytes, 0x00020000);
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        // a local copy: the host pass of this builtin rejects a captured array
        // element, which would silently drop the kernel's launch stub
        const int vo = (int)voff[i];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(&smem[stage * 2 * TILEB] + (w * IPW + i) * 64 * 16), 16, vo,
            0, 0, 0);
      }
    }
  };

  // int8: dequantise this wave's 16 keys of step j (stage `stage`) into the
  // compute tile of step j.  Lane l holds key 16 half + l / 4, dims
  // [(l % 4) D / 4, +D / 4), written as D / 32 swizzled 16-byte chunks.
  auto dequant = [&](int j, int stage) {
    if constexpr (QUANT) {
      constexpr int BPL = D / 4;   // int8 bytes per lane
      const uint8_t* src = &smem[2 * 2 * TILEB + stage * 4 * R8 + w * R8 + lane * BPL];
      uint32_t in[BPL / 4];
#pragma unroll
      for (int c = 0; c < BPL / 16; ++c) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(src + 16 * c);
        in[4 * c] = x[0];
        in[4 * c + 1] = x[1];
        in[4 * c + 2] = x[2];
        in[4 * c + 3] = x[3];
      }
      uint32_t outw[BPL / 2];
      dequant_words<CT, ST, BPL / 4>(in, sc[stage], outw);
      const int row = 16 * half + (lane >> 2);
      const int swz = tensor ? v_swz(NCH, row) : row % NCH;
      uint8_t* tile = &smem[(j & 1) * 2 * TILEB + tensor * TILEB + row * ROWB];
      const int jc0 = (lane & 3) * (D / 32);
#pragma unroll
      for (int c = 0; c < D / 32; ++c)
        *reinterpret_cast<u32x4*>(tile + ((jc0 + c) ^ swz) * 16) =
            (u32x4){outw[4 * c], outw[4 * c + 1], outw[4 * c + 2], outw[4 * c + 3]};
    }
  };

  // ---- per-lane LDS offsets of the operand reads (same in every stage)
  uint32_t koff[KCH], vofs[DB];
#pragma unroll
  for (int c = 0; c < KCH; ++c) {
    const int jj = h * (NCH / 2) + c;
    koff[c] = (uint32_t)((n * NCH + (jj ^ (n % NCH))) * 16);
  }
  {
    // transpose-read source lane 16g + 4j + c: key 4(g/2) + j (+ 8 per key
    // group, an immediate), dims 32db + 16(g%2) + 4c
    const int g = lane >> 4, j = (lane >> 2) & 3, c = lane & 3;
    const int key = 4 * (g >> 1) + j;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int ch = 4 * db + 2 * (g & 1) + (c >> 1);
      vofs[db] = (uint32_t)(TILEB + key * ROWB + (ch ^ v_swz(NCH, key)) * 16 + 8 * (c & 1));
    }
  }

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = (f32x16){};
  float m = -INFINITY, l = 0.f;
  const float cs = a.scale_log2;

  // one step: wait for its copies, barrier, issue the copies kPfStages - 1
  // steps ahead, then compute (STAGE folds to a constant in every unrolled call)
  auto step = [&](int i, const int STAGE) {
    if constexpr (QUANT) {
      // this wave's copies for step i + 1 (dequantised below) have landed
      // once at most the later steps' groups (G8 loads each) are in flight
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((NS - 3) * G8));
    } else {
      // this wave's copies for step i have landed once at most the later
      // steps' groups (IPW loads each) are still in flight
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((kPfStages - 2) * IPW));
    }
    // After the barrier every wave's copies for step i are in LDS (each
    // waited for its own above) and every wave has consumed its reads of
    // the stage that step i + kPfStages - 1 refills (step i - 1).  No memory
    // fence: a workgroup fence would also wait for the later steps' copies
    // still in flight; the signal fences keep the compiler from moving LDS
    // accesses.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // int8: the barrier also published the tile of step i (dequantised in
    // step i - 1) and retired every read of the tile step i + 1 reuses
    issue_loads(i + NS - 1, (STAGE + NS - 1) % NS);
    if constexpr (QUANT) {
      if (i + 1 < nsteps) dequant(i + 1, (STAGE + 1) % NS);
    }
    const int k0 = 32 * i;
    if (k0 >= wave_maxlim) return;
    const uint8_t* st_base = QUANT ? &smem[(i & 1) * 2 * TILEB] : &smem[STAGE * 2 * TILEB];

    // ---- S^T = K . Q^T
    f32x16 st = (f32x16){};
#pragma unroll
    for (int c = 0; c < KCH; ++c) st = M::mma(*reinterpret_cast<const u32x4*>(st_base + koff[c]), qf[c], st);
    // ---- V^T operands: dims 32db + l % 32, keys 8(2kc + r) + 4(l/32) + 0..3
    u32x2 vtr[DB][4];
    const uint32_t st_lds = lds_addr(st_base);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      vtr[db][0] = lds_read_tr<0 * 8 * ROWB>(st_lds + vofs[db]);
      vtr[db][1] = lds_read_tr<1 * 8 * ROWB>(st_lds + vofs[db]);
      vtr[db][2] = lds_read_tr<2 * 8 * ROWB>(st_lds + vofs[db]);
      vtr[db][3] = lds_read_tr<3 * 8 * ROWB>(st_lds + vofs[db]);
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
#pragma unroll
    for (int v = 0; v < 16; ++v)
      x[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[v], cs, -mref));  // -inf scores give exactly 0
    // ---- wait for this wave's V^T reads.  The asm operands keep the wait
    // ahead of every use of the read results (the empty asms below) and
    // after the exponential of x[15], so the reads' latency overlaps the
    // softmax.
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x[15]));
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(vtr[db][r]));
    u32x4 vf[2][DB];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < DB; ++db)
        vf[kc][db] = (u32x4){vtr[db][2 * kc][0], vtr[db][2 * kc][1], vtr[db][2 * kc + 1][0], vtr[db][2 * kc + 1][1]};
    // ---- O^T += V^T . P^T, two 16-key chunks
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      u32x4 pf, pl;
#pragma unroll
      for (int p = 0; p < 4; ++p) pf[p] = M::pack(x[8 * kc + 2 * p], x[8 * kc + 2 * p + 1]);
      if constexpr (std::is_same<CT, BF16>::value) {
        // bf16 keeps 8 significant bits; P = hi + lo carries ~16, and the row
        // sum takes the unrounded values
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t wv = pf[p];
          pl[p] = M::pack(x[8 * kc + 2 * p] - M::lo_of(wv), x[8 * kc + 2 * p + 1] - M::hi_of(wv));
          l += x[8 * kc + 2 * p] + x[8 * kc + 2 * p + 1];
        }
      } else {
        // the row sum of exactly the fp16 weights the MFMA multiplies
#pragma unroll
        for (int p = 0; p < 4; ++p) l = M::sum2(pf[p], l);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        o[db] = M::mma(vf[kc][db], pf, o[db]);
        if constexpr (std::is_same<CT, BF16>::value) o[db] = M::mma(vf[kc][db], pl, o[db]);
      }
    }
  };

  // the query rows land before the first tile copy is issued, so no wait in
  // the loop has to cover them
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
  for (int u = 0; u < NS - 1; ++u) issue_loads(u, u);
  if constexpr (QUANT) {
    // step 0's tile: this wave's copies for step 0 landed once at most the
    // later groups are in flight
    if (nsteps > 0) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | ((NS - 2) * G8));
      dequant(0, 0);
    }
  }
  for (int i0 = 0; i0 < nsteps; i0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (i0 + u < nsteps) step(i0 + u, u);
  }
  // the empty copies issued past the last step still write LDS: they land
  // before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // ---- epilogue: O = O^T / l; o[db][v] is dim 32db + 8(v/4) + 4h + v%4 of
  // row n, so every 4 consecutive values are 4 consecutive dims
  const float lt = pair_sum(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (rv) {
    const int t = r / G, hh = r - t * G;
    q_t* orow = reinterpret_cast<q_t*>(a.out) + ((long)(q0 + t) * a.num_q_heads + kvh * G + hh) * D + 4 * h;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        u32x2 pk;
        pk[0] = M::pack(o[db][4 * v4] * inv, o[db][4 * v4 + 1] * inv);
        pk[1] = M::pack(o[db][4 * v4 + 2] * inv, o[db][4 * v4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * v4) = pk;
      }
  }
}


template <class CT, class KVT, class ST, int D>
static void launch_one(const PrefillArgs& a, int max_q_len, hipStream_t s) {
  const int units = a.num_seqs * a.num_kv_heads;
  const int tiles = (max_q_len * a.group + kPfRows - 1) / kPfRows;
  hipLaunchKernelGGL((prefill_mfma_kernel<CT, KVT, ST, D>), dim3((unsigned)(units * tiles)), dim3(64 * kPfWaves),
                     0, s, a, a.tables, tiles);
}

template <class CT, class KVT, class ST>
static bool launch_d(const PrefillArgs& a, int head_dim, int max_q_len, hipStream_t s) {
  if (head_dim == 128) launch_one<CT, KVT, ST, 128>(a, max_q_len, s);
  else launch_one<CT, KVT, ST, 64>(a, max_q_len, s);
  return true;
}

template <class CT>
static bool launch_ct(const PrefillArgs& a, int kv_dtype, int scale_dtype, int head_dim, int max_q_len,
                      hipStream_t s) {
  if (kv_dtype == CT::code) return launch_d<CT, CT, F32>(a, head_dim, max_q_len, s);
  if (kv_dtype != HPA_I8 || !a.ks || !a.vs) return false;
  if (scale_dtype == HPA_F16) return launch_d<CT, I8, F16>(a, head_dim, max_q_len, s);
  if (scale_dtype == HPA_F32) return launch_d<CT, I8, F32>(a, head_dim, max_q_len, s);
  return false;
}

bool launch_prefill_mfma(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim,
                         int max_q_len, hipStream_t s) {
  if (a.bs_log2 < 4 || (head_dim != 64 && head_dim != 128)) return false;
  if ((long)max_q_len * a.group > (1L << 30)) return false;
  if ((long)a.num_seqs * a.num_kv_heads * ((max_q_len * (long)a.group + kPfRows - 1) / kPfRows) > 0x7fffffffL)
    return false;
  if (q_dtype == HPA_F16) return launch_ct<F16>(a, kv_dtype, scale_dtype, head_dim, max_q_len, s);
  if (q_dtype == HPA_BF16) return launch_ct<BF16>(a, kv_dtype, scale_dtype, head_dim, max_q_len, s);
  return false;
}

}  // namespace hpa
