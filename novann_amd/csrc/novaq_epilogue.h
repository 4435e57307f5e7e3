// Fused epilogue of the forward products (Linear, Conv2d) for gfx950.
//
// For output channel c (a Linear output feature or a Conv2d output channel)
// and the fp32 accumulator a of one output element:
//
//   v = a * s_w + bias[c]            the product itself (scale, then bias)
//   v = v * mul[c]                   when mul is given   } eval-mode BatchNorm
//   v = v + add[c]                   when add is given   } folded per channel
//   v = v * (v > 0 ? 1 : 0)          when relu is set (novann functional.relu:
//                                    negative -> -0, NaN and -Inf -> NaN)
//   store v as out_dtype             f32; bf16 / f16 (RNE); E4M3 / E5M2 as
//                                    enc(v * (1/s_out)) with the cast kernels'
//                                    rules (saturating, NaN kept)
//
// Every step is one fp32 operation rounded to nearest even (no contraction),
// so an epilogue equals the same steps applied to the fp32 output afterwards
// bit for bit, and an FP8 store equals novaq_cast of that fp32 value.  When
// amax is given, the largest |v| (before the store's cast, NaN ignored) of
// the launch is folded into *amax with an atomic max on the fp32 bits (the
// caller's entry point zeroes it first).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"

namespace novaq {

struct Epilogue {
  const float* bias;
  const float* mul;
  const float* add;
  const float* out_scale;  // FP8 output: s_out (NULL: 1)
  uint32_t* amax;          // fp32 bits of max |v|, or NULL
  int relu;
  int out_dtype;  // F32, F16, BF16, E4M3, E5M2
};

// Per-channel constants of the epilogue, loaded once per channel.
struct EpiChan {
  float bias, mul, add;
};

// (an absent mul / add is 1 / -0: the identities epi_value_nb relies on)
__device__ __forceinline__ EpiChan epi_chan(const Epilogue& e, int c) {
  EpiChan k;
  k.bias = e.bias ? e.bias[c] : 0.0f;
  k.mul = e.mul ? e.mul[c] : 1.0f;
  k.add = e.add ? e.add[c] : -0.0f;
  return k;
}

// 1 / s_out for the FP8 stores (correctly rounded division, as the casts).
__device__ __forceinline__ float epi_inv_scale(const Epilogue& e) {
  return (e.out_scale && is_quant(e.out_dtype)) ? 1.0f / *e.out_scale : 1.0f;
}

__device__ __forceinline__ float epi_value(const Epilogue& e, const EpiChan& k, float acc,
                                           float s) {
  float v = acc * s + k.bias;
  if (e.mul) v = v * k.mul;
  if (e.add) v = v + k.add;
  if (e.relu) v = v * (v > 0.0f ? 1.0f : 0.0f);
  return v;
}

// epi_value without branches on the epilogue's fields: an absent step is an
// exact identity (v * 1 = v and v + (-0) = v for every v, -0 and NaN
// included; the ReLU factor is z = 1 when relu is off, 0 when on), so the
// result has the same bits (NaN stays NaN).
__device__ __forceinline__ float epi_relu_factor(const Epilogue& e) {
  return e.relu ? 0.0f : 1.0f;
}

__device__ __forceinline__ float epi_value_nb(const EpiChan& k, float acc, float s, float z) {
  float v = acc * s + k.bias;
  v = v * k.mul;
  v = v + k.add;
  return v * (v > 0.0f ? 1.0f : z);
}

// Running max of |v| bits, NaN ignored (0 is the identity).
__device__ __forceinline__ uint32_t epi_track(uint32_t m, float v) {
  const uint32_t a = f2u(v) & 0x7FFFFFFFu;
  return a <= 0x7F800000u && a > m ? a : m;
}

// Wave-wide max, then one atomic per wave.
__device__ __forceinline__ void epi_amax_commit(const Epilogue& e, uint32_t m) {
  if (!e.amax) return;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t t = (uint32_t)__shfl_xor((int)m, o);
    m = t > m ? t : m;
  }
  if ((threadIdx.x & 63) == 0 && m) atomicMax(e.amax, m);
}

// Code of v in the output dtype (bits in the low end).
__device__ __forceinline__ uint32_t epi_encode(int dt, float v, float inv_s) {
  switch (dt) {
    case F16: return enc_f16(f2u(v));
    case BF16: return enc_bf16(f2u(v));
    case E4M3: return enc_e4m3(scale_mul(f2u(v), inv_s));
    case E5M2: return enc_e5m2(scale_mul(f2u(v), inv_s));
    default: return f2u(v);
  }
}

// Store one element at index i of the output.
__device__ __forceinline__ void epi_store(int dt, void* y, int64_t i, float v, float inv_s) {
  const uint32_t c = epi_encode(dt, v, inv_s);
  if (dt == F32) reinterpret_cast<float*>(y)[i] = v;
  else if (dt == F16 || dt == BF16) reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)c;
  else reinterpret_cast<uint8_t*>(y)[i] = (uint8_t)c;
}

// Store four consecutive elements at index i (a multiple of 4; the output is
// 16-byte aligned) with one 16 / 8 / 4-byte store.
__device__ __forceinline__ void epi_store4(int dt, void* y, int64_t i, const float* v,
                                           float inv_s) {
  if (dt == F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (dt == F16 || dt == BF16) {
    const uint32_t c0 = epi_encode(dt, v[0], inv_s), c1 = epi_encode(dt, v[1], inv_s);
    const uint32_t c2 = epi_encode(dt, v[2], inv_s), c3 = epi_encode(dt, v[3], inv_s);
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(y) + i) =
        make_uint2(c0 | (c1 << 16), c2 | (c3 << 16));
  } else {
    uint32_t w = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) w |= epi_encode(dt, v[q], inv_s) << (8 * q);
    *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(y) + i) = w;
  }
}

// The same encode / stores with the output dtype fixed at compile time.
template <int OD>
__device__ __forceinline__ uint32_t epi_encode_t(float v, float inv_s) {
  if constexpr (OD == F16) return enc_f16(f2u(v));
  else if constexpr (OD == BF16) return enc_bf16(f2u(v));
  else if constexpr (OD == E4M3) return enc_e4m3(scale_mul(f2u(v), inv_s));
  else if constexpr (OD == E5M2) return enc_e5m2(scale_mul(f2u(v), inv_s));
  else return f2u(v);
}

// Two 16-bit codes in one word (v0 in the low half).
template <int OD>
__device__ __forceinline__ uint32_t epi_encode2_t(float v0, float v1, float inv_s) {
  if constexpr (OD == BF16) return pack_bf16x2(f2u(v0), f2u(v1));
  else return epi_encode_t<OD>(v0, inv_s) | (epi_encode_t<OD>(v1, inv_s) << 16);
}

template <int OD>
__device__ __forceinline__ void epi_store_t(void* y, int64_t i, float v, float inv_s) {
  if constexpr (OD == F32) reinterpret_cast<float*>(y)[i] = v;
  else if constexpr (OD == F16 || OD == BF16)
    reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)epi_encode_t<OD>(v, inv_s);
  else reinterpret_cast<uint8_t*>(y)[i] = (uint8_t)epi_encode_t<OD>(v, inv_s);
}

template <int OD>
__device__ __forceinline__ void epi_store4_t(void* y, int64_t i, const float* v, float inv_s) {
  if constexpr (OD == F32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + i) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (OD == F16 || OD == BF16) {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(y) + i) =
        make_uint2(epi_encode2_t<OD>(v[0], v[1], inv_s), epi_encode2_t<OD>(v[2], v[3], inv_s));
  } else {
    uint32_t w = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) w |= epi_encode_t<OD>(v[q], inv_s) << (8 * q);
    *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(y) + i) = w;
  }
}

template <int OD>
struct OutDtype {
  static constexpr int value = OD;
};

}  // namespace novaq
