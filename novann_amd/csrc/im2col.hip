// The two intermediate arrays NovaNN's operators hand back with extras=True,
// materialised on the device for callers that keep them (the reference's
// Conv2d and MaxPool2d layers cache them for their backward):
//
//   im2col_kernel  the conv2d column matrix (novann/functional.py:346-368):
//                  col[(c, kh, kw), (n, oh, ow)] =
//                      xpad[n, c, oh * sh + kh, ow * sw + kw]
//                  as fp32, rows ordered (c, kh, kw) and columns (n, oh, ow)
//                  exactly as the reference's windows.transpose(1, 4, 5, 0,
//                  2, 3).reshape(C * KH * KW, -1) lays them out;
//   pad2d_kernel   the padded input (np.pad, functional.py:325-344 for conv2d
//                  and :495-514 for max_pool2d) in the input's own storage,
//                  over which the caller takes the (N, C, OH, OW, KH, KW)
//                  window view with strides, as the reference's as_strided
//                  does (:516-527).
//
// Both are pure data movement: every output element is one input element (or
// the zero pad), decoded for im2col (F16 / BF16 widened exactly, FP8 times its
// per-tensor scale as one fp32 multiply, the value novaq_cast's dequantize
// gives) and copied code for code by the pad.  HBM-bound: the column matrix is
// KH * KW times the input (config [5] conv2: 231 MB written), each input
// element read KH * KW times from L2.  Each lane makes 4 consecutive outputs
// and stores them with one vector store; consecutive lanes continue along the
// output row, so a wave's stores are one contiguous span.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "novaq_convert.h"
#include "novaq_internal.h"
#include "novaq_xload.h"

namespace novaq {
namespace {

constexpr int THREADS = 256;
constexpr int PER_LANE = 4;
constexpr int SPAN = THREADS * PER_LANE;  // outputs per workgroup and row
constexpr int MAX_GRID_Y = 65535;

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ColGeom {
  int C, H, W, KH, KW, sh, sw, ph, pw, pad_mode, OH, OW;
  int L;       // columns: N * OH * OW
  int rows;    // C * KH * KW
  int segs;    // workgroups along a row
};

// Workgroup (seg, y) writes columns [seg * SPAN, +SPAN) of rows y, y + gridDim.y, ...
template <int XT>
__global__ __launch_bounds__(THREADS) void im2col_kernel(const uint8_t* __restrict__ x,
                                                         const float* __restrict__ scale,
                                                         float* __restrict__ col, ColGeom g) {
  const int j0 = blockIdx.x * SPAN + threadIdx.x * PER_LANE;
  if (j0 >= g.L) return;
  float s = 1.0f;
  if constexpr (is_quant(XT)) {
    if (scale) s = *scale;
  }
  // column j0 -> (n, oh, ow), the next three by carrying
  const int q = j0 / g.OW;
  const int ow0 = j0 - q * g.OW;
  const int n0 = q / g.OH;
  const int oh0 = q - n0 * g.OH;
  const int plane_hw = g.H * g.W;
  const bool whole = (g.L & 3) == 0 && j0 + PER_LANE <= g.L;
  for (int r = blockIdx.y; r < g.rows; r += gridDim.y) {
    const int c = r / (g.KH * g.KW);
    const int kk = r - c * (g.KH * g.KW);
    const int kh = kk / g.KW, kw = kk - (kk / g.KW) * g.KW;
    int n = n0, oh = oh0, ow = ow0;
    float v[PER_LANE];
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) {
      float val = 0.0f;
      if (j0 + e < g.L) {
        const int hi = pad_index(oh * g.sh + kh - g.ph, g.H, g.pad_mode);
        const int wi = pad_index(ow * g.sw + kw - g.pw, g.W, g.pad_mode);
        if (hi >= 0 && wi >= 0) {
          const int64_t idx = ((int64_t)n * g.C + c) * plane_hw + (int64_t)hi * g.W + wi;
          uint32_t bits = decode<XT>(x_code<XT>(x, idx));
          if constexpr (is_quant(XT)) bits = scale_mul(bits, s);
          val = u2f(bits);
        }
      }
      v[e] = val;
      if (++ow == g.OW) {
        ow = 0;
        if (++oh == g.OH) {
          oh = 0;
          ++n;
        }
      }
    }
    float* dst = col + (int64_t)r * g.L + j0;
    if (whole) {
      __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(dst));
    } else {
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e)
        if (j0 + e < g.L) dst[e] = v[e];
    }
  }
}

struct PadGeom {
  int H, W, ph, pw, pad_mode, Hp, Wp;
  int64_t planes;
};

// Workgroup (seg, y) writes elements [seg * SPAN, +SPAN) of planes y,
// y + gridDim.y, ...; EB bytes per element (codes copied as they are).
template <int EB>
__global__ __launch_bounds__(THREADS) void pad2d_kernel(const uint8_t* __restrict__ x,
                                                        uint8_t* __restrict__ y, PadGeom g) {
  using T = typename std::conditional<EB == 4, uint32_t,
                                      typename std::conditional<EB == 2, uint16_t,
                                                                uint8_t>::type>::type;
  const int hw = g.Hp * g.Wp;
  const int i0 = blockIdx.x * SPAN + threadIdx.x * PER_LANE;
  if (i0 >= hw) return;
  const int hp0 = i0 / g.Wp, wp0 = i0 - hp0 * g.Wp;
  const T* src = reinterpret_cast<const T*>(x);
  T* dst = reinterpret_cast<T*>(y);
  const bool whole = (hw & 3) == 0 && i0 + PER_LANE <= hw;
  for (int64_t p = blockIdx.y; p < g.planes; p += gridDim.y) {
    const T* plane = src + p * g.H * g.W;
    int hp = hp0, wp = wp0;
    T v[PER_LANE];
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) {
      T val = 0;
      if (i0 + e < hw) {
        const int hi = pad_index(hp - g.ph, g.H, g.pad_mode);
        const int wi = pad_index(wp - g.pw, g.W, g.pad_mode);
        if (hi >= 0 && wi >= 0) val = plane[hi * g.W + wi];
      }
      v[e] = val;
      if (++wp == g.Wp) {
        wp = 0;
        ++hp;
      }
    }
    T* out = dst + p * hw + i0;
    if (whole) {
      if constexpr (EB == 4) {
        *reinterpret_cast<uint32_t __attribute__((ext_vector_type(4)))*>(out) =
            (uint32_t __attribute__((ext_vector_type(4)))){v[0], v[1], v[2], v[3]};
      } else if constexpr (EB == 2) {
        *reinterpret_cast<uint32_t __attribute__((ext_vector_type(2)))*>(out) =
            (uint32_t __attribute__((ext_vector_type(2)))){
                (uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
      } else {
        *reinterpret_cast<uint32_t*>(out) = (uint32_t)v[0] | ((uint32_t)v[1] << 8) |
                                            ((uint32_t)v[2] << 16) | ((uint32_t)v[3] << 24);
      }
    } else {
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e)
        if (i0 + e < hw) out[e] = v[e];
    }
  }
}

}  // namespace

int im2col_launch(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t C,
                  int64_t H, int64_t W, int KH, int KW, int sh, int sw, int ph, int pw,
                  int pad_mode, float* col, hipStream_t stream) {
  const int64_t OH = (H + 2 * (int64_t)ph - KH) / sh + 1;
  const int64_t OW = (W + 2 * (int64_t)pw - KW) / sw + 1;
  const int64_t L = N * OH * OW, rows = C * KH * KW;
  // 32-bit column and plane indices; the padded window positions fit int
  if (L > 0x7FFFFFFF - SPAN || rows > 0x7FFFFFFF || H * W > 0x7FFFFFFF || OH * sh + KH > 0x3FFFFFFF ||
      OW * sw + KW > 0x3FFFFFFF)
    return NOVAQ_EINVAL;
  if (L == 0) return NOVAQ_OK;
  ColGeom g{(int)C, (int)H, (int)W, KH, KW, sh, sw, ph, pw, pad_mode, (int)OH, (int)OW, (int)L,
            (int)rows, (int)((L + SPAN - 1) / SPAN)};
  const dim3 grid((unsigned)g.segs, (unsigned)(rows < MAX_GRID_Y ? rows : MAX_GRID_Y));
  const auto* xb = static_cast<const uint8_t*>(x);
  switch (x_dtype) {
    case F32: hipLaunchKernelGGL(im2col_kernel<F32>, grid, dim3(THREADS), 0, stream, xb, nullptr, col, g); break;
    case F16: hipLaunchKernelGGL(im2col_kernel<F16>, grid, dim3(THREADS), 0, stream, xb, nullptr, col, g); break;
    case BF16: hipLaunchKernelGGL(im2col_kernel<BF16>, grid, dim3(THREADS), 0, stream, xb, nullptr, col, g); break;
    case E4M3: hipLaunchKernelGGL(im2col_kernel<E4M3>, grid, dim3(THREADS), 0, stream, xb, x_scale, col, g); break;
    case E5M2: hipLaunchKernelGGL(im2col_kernel<E5M2>, grid, dim3(THREADS), 0, stream, xb, x_scale, col, g); break;
    default: return NOVAQ_EDTYPE;
  }
  return check_launch();
}

int pad2d_launch(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int ph,
                 int pw, int pad_mode, void* y, hipStream_t stream) {
  const int64_t Hp = H + 2 * (int64_t)ph, Wp = W + 2 * (int64_t)pw;
  if (Hp * Wp > 0x7FFFFFFF - SPAN || H * W > 0x7FFFFFFF) return NOVAQ_EINVAL;
  const int64_t planes = N * C;
  if (planes == 0) return NOVAQ_OK;
  PadGeom g{(int)H, (int)W, ph, pw, pad_mode, (int)Hp, (int)Wp, planes};
  const dim3 grid((unsigned)((Hp * Wp + SPAN - 1) / SPAN),
                  (unsigned)(planes < MAX_GRID_Y ? planes : MAX_GRID_Y));
  const auto* xb = static_cast<const uint8_t*>(x);
  auto* yb = static_cast<uint8_t*>(y);
  switch (dtype_bits(x_dtype)) {
    case 32: hipLaunchKernelGGL(pad2d_kernel<4>, grid, dim3(THREADS), 0, stream, xb, yb, g); break;
    case 16: hipLaunchKernelGGL(pad2d_kernel<2>, grid, dim3(THREADS), 0, stream, xb, yb, g); break;
    case 8: hipLaunchKernelGGL(pad2d_kernel<1>, grid, dim3(THREADS), 0, stream, xb, yb, g); break;
    default: return NOVAQ_EDTYPE;
  }
  return check_launch();
}

}  // namespace novaq
