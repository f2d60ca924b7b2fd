// Wide speculative verify over int8 pools: 17-64 query rows per KV head
// (helios' verify prefill, exec/runner.py:354-362, batched over sequences),
// fp16 or bf16 queries (bf16 rows enter the fp16 MFMAs scaled by a power of
// two), head_dim 64 or 128, block_size >= 16.
//
// A workgroup of two waves owns one (sequence, KV head): wave w holds rows
// [32 w, 32 w + 32) of its G * q_per_seq rows, one 32x32 MFMA tile, and
// computes S^T = K Q^T and O^T += V^T P^T as prefill_mfma_kernel does.  The
// K/V tiles of each 32-key step travel into LDS as int8 (with their
// per-(token, head) scales) by direct global->LDS copies, three steps ahead
// of the compute, and each wave turns its own MFMA operands into fp16 in
// registers (one xor and one v_perm per pair of bytes) with offsets that
// leave algebraically:
//   K byte x -> fp16 subnormal (128 + x) 2^-24:
//     S = ks[key] * 2^24 * (S' - 128 * 2^-24 * sum(q))
//   V byte x -> fp16 1152 + x, and P * vs[key] = hi + lo (two fp16 values):
//     O = (O' - 1152 * sum(hi + lo)) / l
// The K offset stays small next to |x| <= 127, so large key scales do not
// amplify the cancellation in S', and the hi/lo pair carries P * vs to
// 2^-22, so no per-key rounding of the weights reaches the output.  No
// dequantised tile is written back to LDS and no step waits for one.
// A workgroup then needs only the int8 stages (33 KB at head_dim 128), four
// workgroups share a CU, and every wave holds rows (with 17-32 rows the
// second wave only copies).  With a workspace, the longest units of an XCD
// are cut into 2-4 pieces that run on separate workgroups; the last piece to
// finish merges them in piece order.
//
// Operand layouts (lane l, h = l / 32, n = l % 32):
//  - S^T's A operand row m is key pi(m) (bits 2 and 3 of m swapped), so the
//    16 scores a lane holds are keys 16 kc + 8 h + e (value 8 kc + e), e < 8:
//    the P^T operand of chunk kc is the lane's own 8 values, in key order.
//  - K: 8 consecutive dims of key pi(n) per MFMA (one ds_read_b64).
//  - V^T: dim 32 db + n of keys 16 kc + 8 h + e, e < 8, from one
//    ds_read_b64_tr_b8: within each 16-lane group, output lane i gets byte
//    i % 8 of the 8 bytes addressed by lanes i / 8 + 2 j (j = 0..7), so lane
//    s of group g addresses key 16 kc + 8 (g / 2) + (s % 16) / 2 at dims
//    32 db + 16 (g % 2) + 8 (s % 2) (layout measured on gfx950).
// LDS rows are 16-byte chunks XOR-swizzled by (row / 2) % (chunks per row);
// the copies apply the permutation on the global side.
#include <algorithm>
#include <type_traits>

#include "hpa_attn_core.h"
#include "hpa_host.h"
#include "hpa_prefill.h"

namespace hpa {

typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef __bf16 vi_bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kViWaves = 2;    // 32 rows each
constexpr int kViStages = 4;   // LDS stages; copies run kViStages - 1 steps ahead
// rescale only when a row max grows by more than 2^kViLazy, so P <= 16 and
// P * vs stays inside fp16 for every scale of an fp16-range value (vs < 517)
constexpr int kViLazy = 4;

// split-K: a unit is cut when its steps exceed its XCD's steps per resident
// workgroup and kViMinPiece (piece slots: kViSlotFloats)
constexpr int kViMinPiece = 16;
constexpr int kViMaxPieces = 4;  // pieces per cut unit
// device-scope (sc1) buffer accesses: pieces travel between workgroups on
// different XCDs, whose L2 caches are not coherent with each other
constexpr int kViCoherent = 16;

__host__ __device__ constexpr int vi_vmcnt(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// bytes b0..b7 of (w0, w1), signed, as the fp16 subnormals (128 + b) 2^-24,
// in order (the K operand: an offset of 128 next to |b| <= 127 keeps the fp32
// sums of S' within a few units of the score's own magnitude)
__device__ __forceinline__ u32x4 vi_i8_f16_sub(uint32_t w0, uint32_t w1) {
  const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  return (u32x4){__builtin_amdgcn_perm(0u, x0, 0x0C010C00u), __builtin_amdgcn_perm(0u, x0, 0x0C030C02u),
                 __builtin_amdgcn_perm(0u, x1, 0x0C010C00u), __builtin_amdgcn_perm(0u, x1, 0x0C030C02u)};
}

// bytes b0..b7 of (w0, w1), signed, as the fp16 values 1152 + b, in order
// (the V operand)
__device__ __forceinline__ u32x4 vi_i8_f16(uint32_t w0, uint32_t w1) {
  const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  return (u32x4){__builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u),
                 __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u),
                 __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u),
                 __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)};
}

__device__ __forceinline__ f32x16v vi_mma(u32x4 a, u32x4 b, f32x16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// x combined with the value of lane l ^ 32 (the other half of the same row)
__device__ __forceinline__ float vi_pair_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float vi_pair_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// LDS reads of the step's operands, issued through inline asm: the
// compiler's wait pass cannot tell an LDS read from the global->LDS copies
// in flight and would drain every one of them (vmcnt(0)) before it; the
// step counts these reads itself (vi_wait_lgkm).  LDS reads complete in
// issue order.
__device__ __forceinline__ u32x2 vi_read_tr8(uint32_t addr) {  // 8 transposed bytes (layout above)
  u32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ u32x2 vi_read_b64(uint32_t addr) {
  u32x2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
template <int OFF>
__device__ __forceinline__ u32x4 vi_read_b128(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// wait until at most N of this wave's LDS reads are outstanding (the
// counter saturates at 15, so a larger N waits for 15)
template <int N>
__device__ __forceinline__ void vi_wait_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N < 15 ? N : 15));
}
// f(std::integral_constant<int, I>) for I = 0 .. N-1, so that I can be a
// template argument (waits and immediate offsets)
template <int I, int N>
struct ViFor {
  template <class F>
  __device__ __forceinline__ static void run(F& f) {
    f(std::integral_constant<int, I>{});
    ViFor<I + 1, N>::run(f);
  }
};
template <int N>
struct ViFor<N, N> {
  template <class F>
  __device__ __forceinline__ static void run(F&) {}
};

__device__ __forceinline__ uint32_t vi_lds_addr(const uint8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

// the scale of entry e (0..7) of an 8-scale run, raw bits in w (fp16: two per
// word; fp32: one per word)
template <class ST>
__device__ __forceinline__ float vi_scale(const uint32_t* w, int e) {
  if constexpr (std::is_same<ST, F16>::value) return f16_bits_to_f32((w[e >> 1] >> (16 * (e & 1))) & 0xffffu);
  else return __builtin_bit_cast(float, w[e]);
}
// fma(x, scale e of the run, c); an fp16 scale enters as an operand of
// v_fma_mix_f32, so the product costs one instruction for either storage
template <class ST>
__device__ __forceinline__ float vi_fma_scale(float x, const uint32_t* w, int e, float c) {
  if constexpr (std::is_same<ST, F16>::value)
    return __builtin_fmaf(x, (float)__builtin_bit_cast(f16x2, w[e >> 1])[e & 1], c);
  else return __builtin_fmaf(x, __builtin_bit_cast(float, w[e]), c);
}

// BQ: bf16 queries and output.  The MFMAs still run in fp16: a bf16 value is
// exact in fp16 within fp16's range, each query row enters scaled by the
// power of two that brings its largest element into [2^14, 2^15), and that
// scale returns in the row's score scale.
template <class ST, int D, bool BQ>
__global__ __launch_bounds__(64 * kViWaves, 2) void verify_i8_kernel(const PrefillArgs a) {
  constexpr int CH = D / 16;                     // 16-byte chunks per key row (int8)
  constexpr int DB = D / 32;                     // O^T blocks of 32 dims
  constexpr int SSZ = (int)sizeof(typename ST::storage);
  constexpr int NI = D / 64;                     // 1 KB copies per 16-key half
  constexpr int NS = kViStages;
  constexpr int TILE = 32 * D;                   // one step's K (or V) tile
  constexpr int SB = 2 * TILE + 2 * 32 * SSZ;    // stage: K tile, V tile, K scales, V scales
  constexpr int LPW = 2 * NI + 2;                // copy instructions per wave per step
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert((NS & (NS - 1)) == 0 && (NS - 2) * LPW < 64, "stage mask; copy waits fit vmcnt");
  __shared__ __attribute__((aligned(16))) uint8_t smem[NS * SB];
  __shared__ int s_pick;
  __shared__ int s_red[2];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, n = lane & 31;
  const int units = a.num_seqs * a.num_kv_heads;
  const int T = a.uniform_q, G = a.group, H = a.num_kv_heads;

  // ---- the work item of this workgroup: a unit, longest-first per XCD
  // (workgroup 8 m + x, x its XCD, runs the item of rank m there).  With
  // cutting on, the `cuts` longest units of the XCD whose n steps exceed
  // both kViMinPiece and the XCD's steps per resident workgroup (at most
  // a.cut_budget of them) are cut into P pieces of steps [p n / P, (p + 1)
  // n / P): P = 2, or up to kViMaxPieces when that still leaves no item
  // waiting for a resident workgroup.  Items P r .. P r + P - 1 are the
  // pieces of the unit of rank r, then the other units follow
  // longest-first.  Workgroups past the XCD's item count return at once.
  int unit = (int)blockIdx.x;
  int s_begin = 0, s_end = -1, piece = -1, pieces = 0, slot = 0;
  {
    const int xcd = unit & 7, m = unit >> 3;
    int* lds = reinterpret_cast<int*>(&smem[0]);
    if (a.cut_budget <= 0) {
      const int nk = ((int)gridDim.x - xcd + 7) >> 3;
      if (nk <= kLptMax)
        unit = lpt_pick<64 * kViWaves>(lds, &s_pick, nk, m, xcd,
                                       [&](int j) { return max(a.ctx_lens[(8 * j + xcd) / H], 0); });
    } else {
      // the launcher cuts only when nk <= kLptMax / 2
      const int nk = (units - xcd + 7) >> 3, nk4 = (nk + 3) & ~3;
      int* ukey = lds;                 // [kLptMax / 2] steps above inverted index
      int* at = lds + kLptMax / 2;     // [kLptMax / 2] the unit of each rank
      if (threadIdx.x == 0) {
        s_red[0] = 0;
        s_red[1] = 0;
      }
      __syncthreads();
      int tot = 0;
      for (int j = threadIdx.x; j < nk4; j += 64 * kViWaves) {
        const int n = j < nk ? (max(a.ctx_lens[(8 * j + xcd) / H], 0) + 31) >> 5 : 0;
        ukey[j] = j < nk ? (min(n, (1 << (30 - kLptBits)) - 1) << kLptBits) | (kLptMax - 1 - j) : -1;
        tot += n;
      }
      atomicAdd(&s_red[0], tot);
      __syncthreads();
      const int cap = max((s_red[0] + a.xcd_slots - 1) / max(a.xcd_slots, 1), kViMinPiece);
      int over = 0;
      for (int j = threadIdx.x; j < nk; j += 64 * kViWaves) over += (ukey[j] >> kLptBits) > cap;
      atomicAdd(&s_red[1], over);
      __syncthreads();
      // (read through readfirstlane: values from LDS count as divergent, and
      // a divergent step range would put every copy's descriptor in a loop)
      const int cuts = __builtin_amdgcn_readfirstlane(min(s_red[1], a.cut_budget));  // ranks [0, cuts)
      const int np = cuts > 0 ? min(max((a.xcd_slots - nk + cuts) / cuts, 2), kViMaxPieces) : 2;
      if (m >= nk + (np - 1) * cuts) return;  // no item for this workgroup
      for (int j = threadIdx.x; j < nk; j += 64 * kViWaves) {
        const int kj = ukey[j];
        int rank = 0;
#pragma unroll 4
        for (int i = 0; i < nk4; i += 4) {
          const int4 c = *reinterpret_cast<const int4*>(&ukey[i]);
          rank += (c.x > kj) + (c.y > kj) + (c.z > kj) + (c.w > kj);
        }
        at[rank] = j;
      }
      __syncthreads();
      const int rk = __builtin_amdgcn_readfirstlane(m < np * cuts ? m / np : m - (np - 1) * cuts);
      const int j = __builtin_amdgcn_readfirstlane(at[rk]);
      unit = 8 * j + xcd;
      if (m < np * cuts) {
        const int n = __builtin_amdgcn_readfirstlane(ukey[j] >> kLptBits);
        piece = m - np * rk;
        pieces = np;
        // (the divisions by np run on the vector unit; readfirstlane keeps the
        // step range, and with it every copy's descriptor, in scalar registers)
        s_begin = __builtin_amdgcn_readfirstlane(piece * n / np);
        s_end = __builtin_amdgcn_readfirstlane((piece + 1) * n / np);
        slot = kViMaxPieces * (8 * rk + xcd);
      }
      __syncthreads();  // every thread has read its item before the copies reuse the LDS
    }
  }
  const int b = unit / H, kvh = unit - b * H;
  const int ctx = __builtin_amdgcn_readfirstlane(max(a.ctx_lens[b], 0));
  const int rows = T * G;
  const int nsteps = (ctx + 31) >> 5;
  if (piece < 0) s_end = nsteps;
  const int q0 = b * T, pos0 = ctx - T;

  // ---- this lane's row and its query fragments: MFMA c takes dims
  // [16 c + 8 h, + 8); the row's sum of q enters the offset term
  const int r = 32 * w + n;
  const bool busy = 32 * w < rows;  // wave-uniform: this wave holds rows
  const bool rv = r < rows && q0 + r / G < a.num_tokens;
  const int t = r / G, hh = r - t * G;
  const int lim = rv ? max(min(pos0 + t + 1, ctx), 0) : 0;
  const int minlim = __builtin_amdgcn_readfirstlane(max(min(pos0 + 1, ctx), 0));
  const uint16_t* qrow = reinterpret_cast<const uint16_t*>(a.q) + ((long)(q0 + t) * a.num_q_heads + kvh * G + hh) * D;
  u32x4 qf[CH];
  float qs = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) qf[c] = rv ? *reinterpret_cast<const u32x4*>(qrow + 16 * c + 8 * h) : (u32x4){0, 0, 0, 0};
  float qexp = 1.f;  // bf16: 2^e, the row entered fp16 as row * 2^-e
  if constexpr (BQ) {
    float mx = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t wd = qf[c][e];
        mx = fmaxf(mx, fmaxf(fabsf(bf16_bits_to_f32(wd & 0xffffu)), fabsf(bf16_bits_to_f32(wd >> 16))));
      }
    mx = vi_pair_max(mx);
    const int ex = mx > 0.f ? max(min(__builtin_amdgcn_frexp_expf(mx) - 15, 240), -120) : 0;
    qexp = __builtin_ldexpf(1.f, ex);
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t wd = qf[c][e];
        const f16x2 hv = {(_Float16)__builtin_ldexpf(bf16_bits_to_f32(wd & 0xffffu), -ex),
                          (_Float16)__builtin_ldexpf(bf16_bits_to_f32(wd >> 16), -ex)};
        qf[c][e] = __builtin_bit_cast(uint32_t, hv);
      }
  }
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t wd = qf[c][e];
      qs += f16_bits_to_f32(wd & 0xffffu) + f16_bits_to_f32(wd >> 16);
    }
  // the first S' MFMA of a step starts from -128 sum(q) 2^-24, so the score
  // times 2^-24 leaves the accumulator directly
  const float qoff = 0x1p-17f * vi_pair_sum(qs);
  f32x16v negq;
#pragma unroll
  for (int v = 0; v < 16; ++v) negq[v] = -qoff;

  // ---- copies: wave 0 copies K and its scales, wave 1 V and its scales,
  // both 16-key halves of every step.  Lane L of copy i lands at byte
  // 1024 i + 16 L of the half's 16 rows; it fetches the chunk that the
  // swizzle puts there.
  const char* pool = reinterpret_cast<const char*>(w ? a.v : a.k);
  const char* spool = reinterpret_cast<const char*>(w ? a.vs : a.ks);
  uint32_t voff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int off = 1024 * i + 16 * lane;        // byte within the half's 16 rows
    const int rl = off / D, p = (off % D) / 16;  // row in the half, chunk position
    // the half's first row is a multiple of 16, so the swizzle of row 16 hf + rl
    // is ((16 hf + rl) / 2) % CH = (rl / 2) % CH
    voff[i] = (uint32_t)(rl * D + ((p ^ ((rl >> 1) & (CH - 1))) * 16));
  }
  const long blk_rows = (long)H << a.bs_log2;
  const long head_rows = (long)kvh << a.bs_log2;
  const int bsm = (1 << a.bs_log2) - 1;
  const int32_t* trow = a.tables + (long)b * a.table_stride;
  constexpr int SL = 16 * SSZ / 4;  // dwords of one half's scales
  auto issue_copy = [&](int step) {
    uint8_t* st = &smem[(step & (NS - 1)) * SB];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int key0 = 32 * step + 16 * hf;
      const int left = ctx - key0;
      int valid = step >= s_end ? 0 : left >= 16 ? 16 : left > 0 ? left : 0;
      int phys = 0;
      if (valid > 0) {
        const int lb = key0 >> a.bs_log2;
        phys = lb < a.table_stride ? ((const __attribute__((address_space(4))) int32_t*)trow)[lb] : -1;
        if ((unsigned)phys >= (unsigned)a.num_blocks) { phys = 0; valid = 0; }
      }
      // uniform by construction; said so, because a descriptor the compiler
      // thinks divergent is issued in a readfirstlane loop
      valid = __builtin_amdgcn_readfirstlane(valid);
      phys = __builtin_amdgcn_readfirstlane(phys);
      const long row0 = (long)phys * blk_rows + head_rows + (key0 & bsm);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(pool + row0 * D), (short)0, valid * D, 0x00020000);
      uint8_t* dst = st + w * TILE + hf * 16 * D;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int vo = (int)voff[i];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + 1024 * i), 16,
                                                 vo, 0, 0, 0);
      }
      // the half's scales: SL dwords, one per lane of the first SL lanes.  The
      // record count is rounded up to whole dwords (a dword past the count
      // reads as zero, which would drop the last valid key's scale); the
      // extra slot lies in the same block, and its key is masked.
      const __amdgpu_buffer_rsrc_t ss = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(spool + row0 * SSZ), (short)0, (valid * SSZ + 3) & ~3, 0x00020000);
      uint8_t* sdst = st + 2 * TILE + w * 32 * SSZ + hf * 16 * SSZ;
      if (lane < SL)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ss, (__attribute__((address_space(3))) void*)sdst, 4, 4 * lane, 0, 0,
                                                 0);
    }
  };

  // ---- per-lane LDS offsets of the operand reads (same in every stage)
  const int kr = (n & ~12) | ((n & 4) << 1) | ((n & 8) >> 1);  // pi(n)
  uint32_t koff[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) koff[c] = (uint32_t)(kr * D + ((c ^ ((kr >> 1) & (CH - 1))) * 16) + 8 * h);
  uint32_t vofs[2][DB];
  {
    const int g = lane >> 4, sl = lane & 15;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const int key = 16 * kc + 8 * (g >> 1) + (sl >> 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int ch = 2 * db + (g & 1);
        vofs[kc][db] = (uint32_t)(TILE + key * D + ((ch ^ ((key >> 1) & (CH - 1))) * 16) + 8 * (sl & 1));
      }
    }
  }

  f32x16v o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = (f32x16v){};
  float m = -INFINITY, l = 0.f, loff = 0.f;
  const float cs = a.scale_log2 * 0x1p24f * qexp;  // the scores arrive times 2^-24 (and 2^-e)

  auto step = [&](int i) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(vi_vmcnt((NS - 2) * LPW));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // every wave has read step i - 1's stage, which step i + NS - 1 refills
    issue_copy(i + NS - 1);
    if (!busy) return;  // a wave without rows only copies
    const uint32_t sl = vi_lds_addr(&smem[(i & (NS - 1)) * SB]);
    // ---- LDS reads, in this order: the K operand bytes, the scales of the
    // lane's 16 keys (runs 16 kc + 8 h + [0, 8), K then V), the V^T bytes
    constexpr int NSR = 8 * SSZ / 16;  // 16-byte reads per 8-scale run
    constexpr int NSC = 4 * NSR, NV = 2 * DB;
    u32x2 kraw[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) kraw[c] = vi_read_b64(sl + koff[c]);
    u32x4 ksr[2][NSR], vsr[2][NSR];
    const uint32_t sa = sl + 8 * h * SSZ;
    auto read_scales = [&](auto ji) {
      constexpr int kc = decltype(ji)::value / NSR, c = decltype(ji)::value % NSR;
      ksr[kc][c] = vi_read_b128<2 * TILE + 16 * kc * SSZ + 16 * c>(sa);
      vsr[kc][c] = vi_read_b128<2 * TILE + 32 * SSZ + 16 * kc * SSZ + 16 * c>(sa);
    };
    ViFor<0, 2 * NSR>::run(read_scales);
    u32x2 vraw[2][DB];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < DB; ++db) vraw[kc][db] = vi_read_tr8(sl + vofs[kc][db]);
    // ---- S'^T over the 1152 + k values, each MFMA once its K bytes landed
    f32x16v s;
    auto qk = [&](auto ci) {
      constexpr int c = decltype(ci)::value;
      vi_wait_lgkm<CH - 1 - c + NSC + NV>();
      asm volatile("" : "+v"(kraw[c]));
      s = vi_mma(vi_i8_f16_sub(kraw[c][0], kraw[c][1]), qf[c], c == 0 ? negq : s);
    };
    ViFor<0, CH>::run(qk);
    vi_wait_lgkm<NV>();
    uint32_t ksw[2][4 * NSR], vsw[2][4 * NSR];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int c = 0; c < NSR; ++c) {
        asm volatile("" : "+v"(ksr[kc][c]), "+v"(vsr[kc][c]));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ksw[kc][4 * c + e] = ksr[kc][c][e];
          vsw[kc][4 * c + e] = vsr[kc][c][e];
        }
      }
    // ---- scores: value v is key 16 (v / 8) + 8 h + v % 8 of the step
    const int k0 = 32 * i;
    float x[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) x[v] = vi_fma_scale<ST>(s[v], ksw[v >> 3], v & 7, 0.f);
    if (__builtin_expect(k0 + 32 > minlim, 0)) {
#pragma unroll
      for (int v = 0; v < 16; ++v) x[v] = k0 + 16 * (v >> 3) + 8 * h + (v & 7) < lim ? x[v] : -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, x[v]);
    mx = vi_pair_max(mx) * cs;  // scale_log2 > 0 keeps the order
    const bool grow = mx > m + (float)kViLazy;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float mnew = grow ? mx : m;
      const float alpha = __builtin_amdgcn_exp2f(m - (mnew == -INFINITY ? 0.f : mnew));
      m = mnew;
      l *= alpha;
      loff *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] = o[db] * alpha;
    }
    const float mref = m == -INFINITY ? 0.f : m;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      x[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[v], cs, -mref));  // -inf scores give exactly 0
      l += x[v];
    }
    // P * vs[key] as the sum of two fp16 values hi + lo (hi rounded, lo the
    // rounded remainder, together within 2^-22 of the product): both feed
    // the O^T MFMAs as B operands, and their row sum (of exactly those
    // values) carries the 1152 offset out.  One fp16 P' alone would leave a
    // 2^-11 relative error per key in the output.
    u32x4 phi[2], plo[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int v = 8 * kc + 2 * p;
        const float p0 = vi_fma_scale<ST>(x[v], vsw[kc], 2 * p, 0.f);
        const float p1 = vi_fma_scale<ST>(x[v + 1], vsw[kc], 2 * p + 1, 0.f);
        const f16x2 hi = (f16x2){(_Float16)p0, (_Float16)p1};
        const f16x2 lo = (f16x2){(_Float16)vi_fma_scale<ST>(x[v], vsw[kc], 2 * p, -(float)hi[0]),
                                 (_Float16)vi_fma_scale<ST>(x[v + 1], vsw[kc], 2 * p + 1, -(float)hi[1])};
        phi[kc][p] = __builtin_bit_cast(uint32_t, hi);
        plo[kc][p] = __builtin_bit_cast(uint32_t, lo);
        loff = __builtin_amdgcn_fdot2(hi, (f16x2){1, 1}, loff, false);
        loff = __builtin_amdgcn_fdot2(lo, (f16x2){1, 1}, loff, false);
      }
    // ---- wait for the transpose reads (asm: the compiler does not track
    // them), then O'^T += V'^T P'^T
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(loff));
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < DB; ++db) asm volatile("" : "+v"(vraw[kc][db]));
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x4 vf = vi_i8_f16(vraw[kc][db][0], vraw[kc][db][1]);
        o[db] = vi_mma(vf, phi[kc], o[db]);
        o[db] = vi_mma(vf, plo[kc], o[db]);
      }
  };

  // the query rows land before the first copy is issued, so no wait in the
  // loop has to cover them
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  for (int u = 0; u < NS - 1; ++u) issue_copy(s_begin + u);
  for (int i = s_begin; i < s_end; ++i) step(i);
  // the empty copies issued past the last step still write LDS
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // ---- epilogue: O = (O'^T - 1152 sum(P')) / l; o[db][v] is dim
  // 32 db + 8 (v / 4) + 4 h + v % 4 of row n
  const float lt = vi_pair_sum(l), ot = 1152.f * vi_pair_sum(loff);
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = o[db] - ot;  // unnormalised O
  float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (piece >= 0) {
    // A cut unit.  The piece that arrives last merges all of them (in piece
    // order, so the result does not depend on which one that is) and
    // returns the unit's counter to zero; the others publish their (O, m,
    // l) and leave.  A piece that finds the others already counted merges
    // without publishing.
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(a.pieces, (short)0, 0x7fffffff, 0x00020000);
    const int li = 64 * w + lane;
    // O is stored lane-major: 16-byte chunk (db, c) of every lane of the
    // workgroup in lane order, so each store and load instruction moves 1 KB
    // of consecutive bytes rather than 64 partial cache lines
    auto uo = [&](int db, int c) { return (uint32_t)(((db * 4 + c) * 128 + li) * 16); };
    const uint32_t mlo = (uint32_t)(2 * 64 * 64 + 2 * li) * 4u;
    auto slot_off = [&](int p) { return (uint32_t)((slot + p) * kViSlotFloats) * 4u; };
    int* ctr = a.counters + unit;
    if (threadIdx.x == 0) s_red[0] = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    bool merge = s_red[0] == pieces - 1;
    __syncthreads();
    if (!merge) {
      const uint32_t own = slot_off(piece);
      // (elements are copied out before the bit casts: a bit_cast applied
      // directly to an ext_vector element reads element 0 with hipcc 7.2)
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float e0 = o[db][4 * c], e1 = o[db][4 * c + 1], e2 = o[db][4 * c + 2], e3 = o[db][4 * c + 3];
          __builtin_amdgcn_raw_buffer_store_b128(
              (u32x4){__builtin_bit_cast(uint32_t, e0), __builtin_bit_cast(uint32_t, e1),
                      __builtin_bit_cast(uint32_t, e2), __builtin_bit_cast(uint32_t, e3)},
              pr, own + uo(db, c), 0, kViCoherent);
        }
      __builtin_amdgcn_raw_buffer_store_b64((u32x2){__builtin_bit_cast(uint32_t, m), __builtin_bit_cast(uint32_t, lt)},
                                            pr, own + mlo, 0, kViCoherent);
      // counted once both waves' stores are complete (hence visible device-wide)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __syncthreads();
      if (threadIdx.x == 0) s_red[1] = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      merge = s_red[1] == pieces - 1;
    }
    if (!merge) return;
    if (threadIdx.x == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // every piece's (m, l): this one's from registers, the others' from
    // their slots; then the pieces' O in piece order, rescaled to the
    // largest m
    float mp[kViMaxPieces], lp[kViMaxPieces];
    float mm = -INFINITY;
#pragma unroll
    for (int p = 0; p < kViMaxPieces; ++p) {
      mp[p] = -INFINITY;
      lp[p] = 0.f;
      if (p < pieces) {
        if (p == piece) {
          mp[p] = m;
          lp[p] = lt;
        } else {
          const u32x2 mlx = __builtin_amdgcn_raw_buffer_load_b64(pr, slot_off(p) + mlo, 0, kViCoherent);
          const uint32_t mlx0 = mlx[0], mlx1 = mlx[1];
          mp[p] = __builtin_bit_cast(float, mlx0);
          lp[p] = __builtin_bit_cast(float, mlx1);
        }
        mm = fmaxf(mm, mp[p]);
      }
    }
    f32x16v acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = (f32x16v){};
    float ll = 0.f;
#pragma unroll
    for (int p = 0; p < kViMaxPieces; ++p) {
      if (p < pieces) {
        const float ap = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp[p] - mm);
        ll += lp[p] * ap;
        if (p == piece) {
#pragma unroll
          for (int db = 0; db < DB; ++db) acc[db] += o[db] * ap;
        } else {
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            f32x16v u;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(pr, slot_off(p) + uo(db, c), 0, kViCoherent);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint32_t xe = x[e];
                u[4 * c + e] = __builtin_bit_cast(float, xe);
              }
            }
            acc[db] += u * ap;
          }
        }
      }
    }
    inv = ll > 0.f ? 1.f / ll : 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = acc[db];
  }
  if (rv) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.out) + ((long)(q0 + t) * a.num_q_heads + kvh * G + hh) * D + 4 * h;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        u32x2 pk;
        const float e0 = o[db][4 * v4] * inv, e1 = o[db][4 * v4 + 1] * inv;
        const float e2 = o[db][4 * v4 + 2] * inv, e3 = o[db][4 * v4 + 3] * inv;
        if constexpr (BQ) {
          pk[0] = __builtin_bit_cast(uint32_t, (vi_bf16x2){(__bf16)e0, (__bf16)e1});
          pk[1] = __builtin_bit_cast(uint32_t, (vi_bf16x2){(__bf16)e2, (__bf16)e3});
        } else {
          pk[0] = __builtin_bit_cast(uint32_t, (f16x2){(_Float16)e0, (_Float16)e1});
          pk[1] = __builtin_bit_cast(uint32_t, (f16x2){(_Float16)e2, (_Float16)e3});
        }
        *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * v4) = pk;
      }
  }
}

template <class ST, int D, bool BQ>
static void vi_launch(PrefillArgs a, long units, hipStream_t s) {
  static int per_cu = 0;  // workgroups resident per CU
  if (!per_cu) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(&verify_i8_kernel<ST, D, BQ>),
                                                     64 * kViWaves, 0) != hipSuccess || nb <= 0)
      nb = 1;
    per_cu = nb;
  }
  static int cus_of[64];
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    if (!cus_of[dev] && (hipDeviceGetAttribute(&cus_of[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                         cus_of[dev] <= 0))
      cus_of[dev] = 256;
    cus = cus_of[dev];
  }
  // Cutting needs the workspace (two piece slots per cut unit, 8 XCDs) and
  // at most kLptMax / 2 units per XCD.  Per XCD it may cut up to a quarter of
  // its units, or as many as leave resident workgroups idle otherwise.
  const long nk = (units + 7) / 8;
  const int xcd_slots = std::max(1, cus * per_cu / 8);
  const long slots = std::min<long>(a.piece_slots, 0x7fffffffL / (4L * kViSlotFloats));
  long budget = std::max<long>(nk / 4, std::min<long>(nk, xcd_slots - nk));
  budget = std::min<long>(budget, slots / (8L * kViMaxPieces));
  const bool cut = a.counters && a.pieces && nk <= kLptMax / 2 && budget > 0;
  a.cut_budget = cut ? (int)budget : 0;
  a.xcd_slots = xcd_slots;
  // cutting: every XCD gets enough workgroups for every item: nk + budget
  // with two pieces per cut unit, at most xcd_slots with more
  const dim3 grid((unsigned)(cut ? 8 * std::max<long>(nk + budget, xcd_slots) : units)), block(64 * kViWaves);
  hipLaunchKernelGGL((verify_i8_kernel<ST, D, BQ>), grid, block, 0, s, a);
}

bool launch_verify_i8(const PrefillArgs& a, int q_dtype, int kv_dtype, int scale_dtype, int head_dim,
                      hipStream_t s) {
  if ((q_dtype != HPA_F16 && q_dtype != HPA_BF16) || kv_dtype != HPA_I8 || !a.ks || !a.vs || a.uniform_q <= 0)
    return false;
  if (a.bs_log2 < 4 || (head_dim != 64 && head_dim != 128)) return false;
  const long rows = (long)a.uniform_q * a.group;
  if (rows <= 16 || rows > 32 * kViWaves) return false;
  const long units = (long)a.num_seqs * a.num_kv_heads;
  if (units <= 0 || units > 0x3fffffffL) return false;
  if (scale_dtype != HPA_F16 && scale_dtype != HPA_F32) return false;
  const bool f16s = scale_dtype == HPA_F16, bq = q_dtype == HPA_BF16;
  if (head_dim == 128) {
    if (f16s) bq ? vi_launch<F16, 128, true>(a, units, s) : vi_launch<F16, 128, false>(a, units, s);
    else bq ? vi_launch<F32, 128, true>(a, units, s) : vi_launch<F32, 128, false>(a, units, s);
  } else {
    if (f16s) bq ? vi_launch<F16, 64, true>(a, units, s) : vi_launch<F16, 64, false>(a, units, s);
    else bq ? vi_launch<F32, 64, true>(a, units, s) : vi_launch<F32, 64, false>(a, units, s);
  }
  return true;
}

}  // namespace hpa
