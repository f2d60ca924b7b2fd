// Element types, MFMA fragments and register-level conversions for the
// gfx950 (CDNA4) paged-attention kernels.
//
// Every matrix product in this library is expressed as one 16x16x32 tile
// product:  C[16x16] += A[16x32] * B[32x16]  accumulated in fp32, where lane l
// of the 64-wide wavefront holds row (l % 16) of A, column (l % 16) of B and
// the eight k-slots  k = 8 * (l / 16) + s,  s = 0..7,  of both.  For fp16 and
// bf16 that is one v_mfma_f32_16x16x32_{f16,bf16}; for fp32 it is eight
// v_mfma_f32_16x16x4_f32 (one per slot).  The output C holds
// C[4 * (l / 16) + i][l % 16], i = 0..3, in lane l.
//
// Because a dot product does not care in which order its terms are summed,
// the kernels are free to decide which real index each (lane group, slot)
// pair stands for, as long as A and B agree.  That freedom is what lets
// every operand be loaded straight from the paged pool in wide, coalesced
// loads with no LDS transpose (see hpa_attn_core.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hpa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// dtype codes shared with the C-ABI (include/helios_attn.h)
enum DType : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I8 = 3 };

// ---------------------------------------------------------------- type tags
struct F32 {
  typedef float storage;
  static constexpr int code = DT_F32;
};
struct F16 {
  typedef uint16_t storage;
  static constexpr int code = DT_F16;
};
struct BF16 {
  typedef uint16_t storage;
  static constexpr int code = DT_BF16;
};
struct I8 {
  typedef int8_t storage;
  static constexpr int code = DT_I8;
};

// ------------------------------------------------------- scalar conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}
// Round-to-nearest-even fp32 -> bf16 bits (quiet NaN kept a NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
}

template <class T> struct Cvt;
template <> struct Cvt<F32> {
  __device__ static float to_f32(float x) { return x; }
  __device__ static float from_f32(float x) { return x; }
};
template <> struct Cvt<F16> {
  __device__ static float to_f32(uint16_t x) { return f16_bits_to_f32(x); }
  __device__ static uint16_t from_f32(float x) { return (uint16_t)f32_to_f16_bits(x); }
};
template <> struct Cvt<BF16> {
  __device__ static float to_f32(uint16_t x) { return bf16_bits_to_f32(x); }
  __device__ static uint16_t from_f32(float x) { return (uint16_t)f32_to_bf16_bits(x); }
};

// ---------------------------------------------------------------- fragments
// Eight k-slots of one MFMA operand in the compute type CT.
template <class CT> struct Frag;
template <> struct Frag<F16> { u32x4 w; };   // 8 x fp16, slot s in half s
template <> struct Frag<BF16> { u32x4 w; };  // 8 x bf16
template <> struct Frag<F32> { float f[8]; };

__device__ __forceinline__ f32x4 mma(const Frag<F16>& a, const Frag<F16>& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a.w),
                                                __builtin_bit_cast(f16x8, b.w), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(const Frag<BF16>& a, const Frag<BF16>& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.w),
                                                 __builtin_bit_cast(bf16x8, b.w), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma(const Frag<F32>& a, const Frag<F32>& b, f32x4 c) {
#pragma unroll
  for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f[s], b.f[s], c, 0, 0, 0);
  return c;
}

template <class CT> __device__ __forceinline__ void frag_zero(Frag<CT>& f);
template <> __device__ __forceinline__ void frag_zero(Frag<F16>& f) { f.w = (u32x4){0, 0, 0, 0}; }
template <> __device__ __forceinline__ void frag_zero(Frag<BF16>& f) { f.w = (u32x4){0, 0, 0, 0}; }
template <> __device__ __forceinline__ void frag_zero(Frag<F32>& f) {
#pragma unroll
  for (int s = 0; s < 8; ++s) f.f[s] = 0.f;
}

// Eight fp32 values -> fragment (RNE rounding to the compute type).
__device__ __forceinline__ void frag_from_f32(Frag<F16>& f, const float* x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) f.w[i] = f32_to_f16_bits(x[2 * i]) | (f32_to_f16_bits(x[2 * i + 1]) << 16);
}
__device__ __forceinline__ void frag_from_f32(Frag<BF16>& f, const float* x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) f.w[i] = f32_to_bf16_bits(x[2 * i]) | (f32_to_bf16_bits(x[2 * i + 1]) << 16);
}
__device__ __forceinline__ void frag_from_f32(Frag<F32>& f, const float* x) {
#pragma unroll
  for (int s = 0; s < 8; ++s) f.f[s] = x[s];
}

// ----------------------------------------------- int8 -> compute conversion
// Two signed bytes, already placed as [b0, 0x00, b1, 0x00] (little endian),
// become two exact fp16 values: the byte XOR 0x80 is x + 128 in [0, 255];
// under exponent field 0x64 that half is 1024 + (x + 128); subtracting 1152
// leaves x exactly (every integer below 2048 is an fp16).
__device__ __forceinline__ uint32_t i8x2_placed_to_f16x2(uint32_t placed) {
  f16x2 h = __builtin_bit_cast(f16x2, placed ^ 0x64806480u);
  h = h + (f16x2){(_Float16)-1152.0f, (_Float16)-1152.0f};
  return __builtin_bit_cast(uint32_t, h);
}
// v_perm_b32 selector that gathers byte `ja` of `lo` and byte `jb` of `hi`
// into [lo.ja, 0, hi.jb, 0]; selector 0x0c yields a zero byte.
__host__ __device__ constexpr uint32_t perm_sel_bytes(int ja, int jb) {
  return (uint32_t)ja | (0x0cu << 8) | ((uint32_t)(4 + jb) << 16) | (0x0cu << 24);
}
__device__ __forceinline__ uint32_t i8pair_to_f16x2(uint32_t lo, uint32_t hi, int ja, int jb) {
  return i8x2_placed_to_f16x2(__builtin_amdgcn_perm(hi, lo, perm_sel_bytes(ja, jb)));
}
__device__ __forceinline__ float i8_to_f32(uint32_t word, int j) {
  return (float)(int8_t)((word >> (8 * j)) & 0xffu);
}

}  // namespace hpa
