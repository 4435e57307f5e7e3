// Loads of the forward products' input x in its stored dtype XT (F32, or
// BF16 / F16 / E4M3 / E5M2 as a fused epilogue stores an activation), for
// gfx950.  The products run on bf16 MFMA, so every x element becomes bf16:
// F32 and F16 round to nearest even (the F16 value through its exact fp32
// widening), BF16 is taken as is, E4M3 / E5M2 decode exactly (every FP8 value
// is a bf16 value; the per-tensor scale is applied after accumulation).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"

namespace novaq {

typedef uint32_t xl_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t xl_u32x2 __attribute__((ext_vector_type(2)));
typedef float xl_f32x4 __attribute__((ext_vector_type(4)));
typedef float xl_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 xl_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 xl_f16x2 __attribute__((ext_vector_type(2)));

template <int XT>
struct XL {
  static constexpr int bits = dtype_bits(XT);
  static constexpr int bytes = bits / 8;
  static_assert(XT == F32 || XT == F16 || XT == BF16 || XT == E4M3 || XT == E5M2,
                "x dtype");
};

// Code of element e (raw bits in the low end).
template <int XT>
__device__ __forceinline__ uint32_t x_code(const uint8_t* __restrict__ x, int64_t e) {
  if constexpr (XL<XT>::bits == 32) return reinterpret_cast<const uint32_t*>(x)[e];
  else if constexpr (XL<XT>::bits == 16) return reinterpret_cast<const uint16_t*>(x)[e];
  else return x[e];
}

// Element e decoded to fp32 (exact; unscaled).
template <int XT>
__device__ __forceinline__ float x_val(const uint8_t* __restrict__ x, int64_t e) {
  return u2f(decode<XT>(x_code<XT>(x, e)));
}

// Raw codes of the 4 consecutive elements e .. e+3 (e a multiple of 4, the
// row 16-byte aligned for F32): words 0..3 (F32), 0..1 (16-bit), 0 (8-bit).
template <int XT>
__device__ __forceinline__ xl_u32x4 x4_raw(const uint8_t* __restrict__ x, int64_t e) {
  const uint8_t* p = x + e * XL<XT>::bytes;
  if constexpr (XL<XT>::bits == 32) {
    return *reinterpret_cast<const xl_u32x4*>(p);
  } else if constexpr (XL<XT>::bits == 16) {
    const xl_u32x2 v = *reinterpret_cast<const xl_u32x2*>(p);
    return xl_u32x4{v[0], v[1], 0u, 0u};
  } else {
    return xl_u32x4{*reinterpret_cast<const uint32_t*>(p), 0u, 0u, 0u};
  }
}

// Raw codes of elements e .. e+3, the ones at or past `end` read as 0.
template <int XT>
__device__ __forceinline__ xl_u32x4 x4_raw_guarded(const uint8_t* __restrict__ x, int64_t e,
                                                   int64_t end) {
  xl_u32x4 v = {0u, 0u, 0u, 0u};
  constexpr int B = XL<XT>::bits;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (e + q < end) v[(q * B) / 32] |= x_code<XT>(x, e + q) << ((q * B) % 32);
  return v;
}

// The 4 elements of a raw group as two bf16 pairs (element 2i in the low half).
template <int XT>
__device__ __forceinline__ xl_u32x2 x4_bf16(const xl_u32x4& r) {
  auto pair = [](xl_bf16x2 v) { return __builtin_bit_cast(uint32_t, v); };
  if constexpr (XT == F32) {
    const xl_f32x2 a = {u2f(r[0]), u2f(r[1])}, b = {u2f(r[2]), u2f(r[3])};
    return xl_u32x2{pair(__builtin_convertvector(a, xl_bf16x2)),
                    pair(__builtin_convertvector(b, xl_bf16x2))};
  } else if constexpr (XT == BF16) {
    return xl_u32x2{r[0], r[1]};
  } else if constexpr (XT == F16) {
    // through a scalar word: bit-casting a vector element directly makes
    // ROCm 7.2 clang reuse element 0 for both
    const uint32_t w0 = r[0], w1 = r[1];
    const xl_f32x2 a = __builtin_convertvector(__builtin_bit_cast(xl_f16x2, w0), xl_f32x2);
    const xl_f32x2 b = __builtin_convertvector(__builtin_bit_cast(xl_f16x2, w1), xl_f32x2);
    return xl_u32x2{pair(__builtin_convertvector(a, xl_bf16x2)),
                    pair(__builtin_convertvector(b, xl_bf16x2))};
  } else if constexpr (XT == E4M3) {
    return xl_u32x2{pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[0], 1.0f, false)),
                    pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(r[0], 1.0f, true))};
  } else {
    return xl_u32x2{pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(r[0], 1.0f, false)),
                    pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(r[0], 1.0f, true))};
  }
}

// 4 consecutive elements decoded to fp32 (exact), from an aligned group.
template <int XT>
__device__ __forceinline__ xl_f32x4 x4_f32(const uint8_t* __restrict__ x, int64_t e) {
  if constexpr (XT == F32) {
    return *reinterpret_cast<const xl_f32x4*>(x + e * 4);
  } else {
    const xl_u32x4 r = x4_raw<XT>(x, e);
    constexpr int B = XL<XT>::bits;
    xl_f32x4 f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t word = r[(q * B) / 32];
      f[q] = u2f(decode<XT>((word >> ((q * B) % 32)) & ((1u << B) - 1u)));
    }
    return f;
  }
}

// The combined per-tensor scale of a product: s_w * s_x (NULL = 1; with no
// x scale the result is s_w exactly).
__device__ __forceinline__ float product_scale(const float* w_scale, const float* x_scale) {
  float s = w_scale ? *w_scale : 1.0f;
  if (x_scale) s = s * *x_scale;
  return s;
}

}  // namespace novaq
