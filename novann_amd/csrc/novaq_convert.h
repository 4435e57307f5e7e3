// Device-side element conversions for gfx950.
//
// Every function works on raw bit patterns and reproduces the rules written
// in include/novaq.h exactly (RNE, saturation, NaN, signed zero, subnormals).
// The rounding is done with a few integer and fp32 operations per element so
// that the cast kernels stay HBM-bound:
//   - normal results: add (bias_t - 127) << 23 to rebias the exponent, add
//     (half ulp - 1) + the lsb of the kept mantissa (round-half-even), shift;
//   - subnormal results: add the fp32 "magic" 2^p whose ulp equals the target
//     quantum; the fp32 adder's own round-to-nearest-even then leaves the code
//     in the low bits, and subtracting bits(2^p) extracts it;
//   - decoding shifts the code into fp32 position and multiplies by a power
//     of two, which is exact for every code including subnormals (fp32
//     denormals are kept: the library is never built with flush-to-zero).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace novaq {

enum Dtype : int { F32 = 0, F16 = 1, BF16 = 2, E4M3 = 3, E5M2 = 4, E2M1 = 5 };

__host__ __device__ constexpr int dtype_bits(int dt) {
  return dt == F32 ? 32 : (dt == F16 || dt == BF16) ? 16 : (dt == E2M1) ? 4 : 8;
}
__host__ __device__ constexpr bool is_quant(int dt) {
  return dt == E4M3 || dt == E5M2 || dt == E2M1;
}
__host__ __device__ constexpr float fmt_max(int dt) {
  return dt == E4M3 ? 448.0f : dt == E5M2 ? 57344.0f : dt == E2M1 ? 6.0f : 1.0f;
}

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Magnitude code (sign clear) of the finite or infinite fp32 magnitude `a`
// for a format with MB mantissa bits and exponent bias BIAS, RNE.  Results
// past the largest finite code come back larger than it (callers clamp).
template <int MB, int BIAS>
__device__ __forceinline__ uint32_t round_mag(uint32_t a) {
  constexpr uint32_t kMinNormal = (uint32_t)(128 - BIAS) << 23;
  constexpr uint32_t kMagic = (uint32_t)(127 + 24 - BIAS - MB) << 23;
  constexpr uint32_t kRebias = (uint32_t)(BIAS - 127) << 23;  // wraps: subtracts
  constexpr uint32_t kHalfM1 = (1u << (22 - MB)) - 1u;
  uint32_t sub = f2u(u2f(a) + u2f(kMagic)) - kMagic;
  uint32_t nor = (a + kRebias + kHalfM1 + ((a >> (23 - MB)) & 1u)) >> (23 - MB);
  return a < kMinNormal ? sub : nor;
}

// ---- encoders: fp32 bits -> code ----

__device__ __forceinline__ uint32_t enc_bf16(uint32_t x) {
  uint32_t r = (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
  return (x & 0x7FFFFFFFu) > 0x7F800000u ? ((x >> 16) | 0x0040u) : r;
}

// Two fp32 values (bits a, b) to two bf16 codes in one word, a in the low
// half, with one gfx950 v_cvt_pk_bf16_f32: round to nearest even, a NaN
// quieted with its sign and payload kept -- the codes of enc_bf16 for every
// fp32 input (compared over all 2^32 patterns on the device).  The product
// epilogues' bf16 stores use it; their parity tests check it against the
// oracle's cast on every rounding class.  (The cast kernels keep enc_bf16:
// the packed convert made the fp32 -> bf16 cast 2% slower.)
typedef float cv_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 cv_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(uint32_t a, uint32_t b) {
  const cv_f32x2 f = {u2f(a), u2f(b)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, cv_bf16x2));
}

__device__ __forceinline__ uint32_t enc_f16(uint32_t x) {
  uint32_t a = x & 0x7FFFFFFFu;
  uint32_t c = min(round_mag<10, 15>(a), 0x7C00u);  // overflow -> Inf
  uint32_t nan = 0x7C00u | max((a & 0x7FFFFFu) >> 13, 1u);
  c = a > 0x7F800000u ? nan : c;
  return c | ((x >> 16) & 0x8000u);
}

__device__ __forceinline__ uint32_t enc_e4m3(uint32_t x) {
  uint32_t a = x & 0x7FFFFFFFu;
  uint32_t c = min(round_mag<3, 7>(a), 0x7Eu);  // satfinite, Inf -> 448
  c = a > 0x7F800000u ? 0x7Fu : c;
  return c | ((x >> 24) & 0x80u);
}

__device__ __forceinline__ uint32_t enc_e5m2(uint32_t x) {
  uint32_t a = x & 0x7FFFFFFFu;
  uint32_t c = min(round_mag<2, 15>(a), 0x7Bu);  // satfinite, Inf -> 57344
  c = a > 0x7F800000u ? 0x7Fu : c;
  return c | ((x >> 24) & 0x80u);
}

__device__ __forceinline__ uint32_t enc_e2m1(uint32_t x) {
  uint32_t a = x & 0x7FFFFFFFu;
  uint32_t c = min(round_mag<1, 1>(a), 0x7u) | ((x >> 28) & 0x8u);
  return a > 0x7F800000u ? 0u : c;  // NaN -> +0
}

template <int DT>
__device__ __forceinline__ uint32_t encode(uint32_t x) {
  if constexpr (DT == F32) return x;
  else if constexpr (DT == F16) return enc_f16(x);
  else if constexpr (DT == BF16) return enc_bf16(x);
  else if constexpr (DT == E4M3) return enc_e4m3(x);
  else if constexpr (DT == E5M2) return enc_e5m2(x);
  else return enc_e2m1(x);
}

// ---- decoders: code -> fp32 bits ----

__device__ __forceinline__ uint32_t dec_f16(uint32_t h) {
  uint32_t a = h & 0x7FFFu;
  uint32_t v = f2u(u2f(a << 13) * 0x1p112f);
  v = a >= 0x7C00u ? ((a << 13) | 0x7F800000u) : v;  // Inf / NaN keep payload
  return v | ((h & 0x8000u) << 16);
}

__device__ __forceinline__ uint32_t dec_bf16(uint32_t h) { return h << 16; }

__device__ __forceinline__ uint32_t dec_e4m3(uint32_t c) {
  uint32_t a = c & 0x7Fu;
  uint32_t v = f2u(u2f(a << 20) * 0x1p120f);
  v = a == 0x7Fu ? 0x7FC00000u : v;
  return v | ((c & 0x80u) << 24);
}

__device__ __forceinline__ uint32_t dec_e5m2(uint32_t c) {
  uint32_t a = c & 0x7Fu;
  uint32_t v = f2u(u2f(a << 21) * 0x1p112f);
  v = a == 0x7Cu ? 0x7F800000u : v;
  v = a > 0x7Cu ? 0x7FC00000u : v;
  return v | ((c & 0x80u) << 24);
}

__device__ __forceinline__ uint32_t dec_e2m1(uint32_t c) {
  uint32_t v = f2u(u2f((c & 0x7u) << 22) * 0x1p126f);
  return v | ((c & 0x8u) << 28);
}

template <int ST>
__device__ __forceinline__ uint32_t decode(uint32_t c) {
  if constexpr (ST == F32) return c;
  else if constexpr (ST == F16) return dec_f16(c);
  else if constexpr (ST == BF16) return dec_bf16(c);
  else if constexpr (ST == E4M3) return dec_e4m3(c);
  else if constexpr (ST == E5M2) return dec_e5m2(c);
  else return dec_e2m1(c);
}

// Multiply fp32 bits v by the scale m: the sign is the xor of the signs, the
// magnitude one RNE fp32 multiply; a NaN operand or product gives the
// canonical quiet NaN with that sign.
__device__ __forceinline__ uint32_t scale_mul(uint32_t v, float m) {
  uint32_t sign = (v ^ f2u(m)) & 0x80000000u;
  uint32_t mb = f2u(fabsf(u2f(v)) * fabsf(m));
  mb = ((v & 0x7FFFFFFFu) > 0x7F800000u || mb > 0x7F800000u) ? 0x7FC00000u : mb;
  return sign | mb;
}

// One element through the whole cast pipeline: widen, unscale, scale, narrow.
template <int ST, int DT, bool SCALED>
__device__ __forceinline__ uint32_t convert(uint32_t c, float s, float inv_s) {
  uint32_t v = decode<ST>(c);
  if constexpr (SCALED && is_quant(ST)) v = scale_mul(v, s);
  if constexpr (SCALED && is_quant(DT)) v = scale_mul(v, inv_s);
  return encode<DT>(v);
}

}  // namespace novaq
