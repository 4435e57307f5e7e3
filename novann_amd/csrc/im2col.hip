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
// output row, so a wave's stores are one contiguous span.  A workgroup covers
// a span of 1024 columns (elements) and walks a block of consecutive rows
// (im2col) or a strided set of planes (pad), about 16 workgroups per CU in
// all.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
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
constexpr int WG_PER_CU = 16;  // launch size: workgroups per CU (each loops over rows / planes)

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ColGeom {
  int C, H, W, KH, KW, sh, sw, ph, pw, pad_mode, OH, OW;
  int L;       // columns: N * OH * OW
  int rows;    // C * KH * KW
  int segs;    // workgroups along a row
};

// Workgroup (seg, y) writes columns [seg * SPAN, +SPAN) of the y-th block of
// ceil(rows / gridDim.y) consecutive rows.  A lane's 4 columns fix their
// (n, oh, ow) for every row, so the window origin and the image offset are
// worked out once; a row only adds its uniform (c, kh, kw).  ZEROS: the zeros
// padding mode (an out-of-range tap reads 0), no index folding.
template <int XT, bool ZEROS>
__global__ __launch_bounds__(THREADS) void im2col_kernel(const uint8_t* __restrict__ x,
                                                         const float* __restrict__ scale,
                                                         float* __restrict__ col, ColGeom g) {
  const int j0 = blockIdx.x * SPAN + threadIdx.x * PER_LANE;
  if (j0 >= g.L) return;
  float s = 1.0f;
  if constexpr (is_quant(XT)) {
    if (scale) s = *scale;
  }
  // columns j0 .. j0 + 3 -> image offset, window origin (row, column)
  int64_t xoff[PER_LANE];
  int hb[PER_LANE], wb[PER_LANE];
  bool live[PER_LANE];
  {
    const int q = j0 / g.OW;
    int ow = j0 - q * g.OW;
    int n = q / g.OH;
    int oh = q - n * g.OH;
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) {
      live[e] = j0 + e < g.L;
      xoff[e] = (int64_t)n * g.C * g.H * g.W;
      hb[e] = oh * g.sh - g.ph;
      wb[e] = ow * g.sw - g.pw;
      if (++ow == g.OW) {
        ow = 0;
        if (++oh == g.OH) {
          oh = 0;
          ++n;
        }
      }
    }
  }
  const int plane_hw = g.H * g.W;
  const int taps = g.KH * g.KW;
  const bool whole = (g.L & 3) == 0 && j0 + PER_LANE <= g.L;
  // a contiguous block of rows per workgroup: the KH * KW rows of one input
  // channel re-read the same input lines, from this CU's L1 / its XCD's L2
  const int rpw = (g.rows + gridDim.y - 1) / gridDim.y;
  const int r_end = min(g.rows, (int)(blockIdx.y + 1) * rpw);
  for (int r = blockIdx.y * rpw; r < r_end; ++r) {
    const int c = r / taps;
    const int kk = r - c * taps;
    const int kh = kk / g.KW, kw = kk - kh * g.KW;
    const int cbase = c * plane_hw;
    float v[PER_LANE];
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) {
      int hi = hb[e] + kh, wi = wb[e] + kw;
      bool in;
      if constexpr (ZEROS) {
        in = (unsigned)hi < (unsigned)g.H && (unsigned)wi < (unsigned)g.W;
      } else {
        hi = pad_index(hi, g.H, g.pad_mode);
        wi = pad_index(wi, g.W, g.pad_mode);
        in = hi >= 0 && wi >= 0;
      }
      float val = 0.0f;
      if (live[e] && in) {
        uint32_t bits = decode<XT>(x_code<XT>(x, xoff[e] + (cbase + hi * g.W + wi)));
        if constexpr (is_quant(XT)) bits = scale_mul(bits, s);
        val = u2f(bits);
      }
      v[e] = val;
    }
    float* dst = col + (int64_t)r * g.L + j0;
    if (whole) {
      __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(dst));
    } else {
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e)
        if (live[e]) dst[e] = v[e];
    }
  }
}

// fp32 x, zeros padding, stride 1, W and OW multiples of 4, KW <= 7, x
// 16-byte aligned and under 2 GiB: a lane's 4 columns share (n, oh) with ow a
// multiple of 4, so for row (c, kh, kw) its taps are the 4 consecutive
// elements from column ow + kw - pw of input row oh + kh - ph.  Rows start on
// 16-byte boundaries (W % 4 == 0), so the KW rows of one (c, kh) read columns
// ow - pw .. ow - pw + KW + 2, which lie in at most 4 aligned 4-element
// chunks from a0 = (ow - pw) >> 2; each row's taps start s0 + kw elements
// into them, s0 = (ow - pw) & 3 -- the same for every lane.  A chunk is
// wholly inside the row or wholly padding: the group's chunks are loaded
// once with aligned 16-byte buffer loads (a chunk outside the image carries
// an offset past the buffer and reads +0, the zero pad) and each row's 4
// values are selected from them -- 3 coalesced loads per 3 rows at 3 x 3,
// where the kernel above makes four 4-byte gathers per row.  A workgroup's
// block of rows is a whole number of (c, kh) groups (rpw a multiple of KW).
constexpr uint32_t COL_OOB = 0x80000000u;  // past the buffer of an input under 2 GiB

__device__ __forceinline__ f32x4 taps4(const f32x4& lo, const f32x4& hi, int sh) {
  if (sh == 0) return lo;
  if (sh == 1) return f32x4{lo[1], lo[2], lo[3], hi[0]};
  if (sh == 2) return f32x4{lo[2], lo[3], hi[0], hi[1]};
  return f32x4{lo[3], hi[0], hi[1], hi[2]};
}

__global__ __launch_bounds__(THREADS) void im2col_rows4_kernel(const float* __restrict__ x,
                                                              float* __restrict__ col, ColGeom g,
                                                              int x_bytes, int rpw) {
  const int j0 = blockIdx.x * SPAN + threadIdx.x * PER_LANE;
  if (j0 >= g.L) return;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(x), (short)0, x_bytes, 0x00020000);
  const int q = j0 / g.OW;
  const int ow = j0 - q * g.OW;
  const int n = q / g.OH;
  const int oh = q - n * g.OH;
  const int plane_hw = g.H * g.W;
  const int w4 = g.W >> 2;
  const int s_lo = ow - g.pw;
  const int a0 = s_lo >> 2, s0 = s_lo & 3;  // floor division: s_lo may be negative
  const int nch = (s0 + g.KW + 6) >> 2;     // chunks of columns s0 .. s0 + KW + 2 (<= 4)
  const int r_end = min(g.rows, (int)(blockIdx.y + 1) * rpw);
  int r = blockIdx.y * rpw;
  int ckh = r / g.KW;  // c * KH + kh
  for (; r < r_end; r += g.KW, ++ckh) {
    const int c = ckh / g.KH, kh = ckh - c * g.KH;
    const int hi = oh + kh - g.ph;
    const bool row_in = (unsigned)hi < (unsigned)g.H;
    const int e0 = n * g.C * plane_hw + c * plane_hw + hi * g.W + 4 * a0;
    uint32_t off[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      off[k] = row_in && k < nch && (unsigned)(a0 + k) < (unsigned)w4 ? (uint32_t)(e0 + 4 * k) * 4
                                                                   : COL_OOB;
    f32x4 ch[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      ch[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off[k], 0, 0));
    for (int kw = 0; kw < g.KW; ++kw) {
      const int t = s0 + kw, j = t >> 2;
      const f32x4 lo = j == 0 ? ch[0] : j == 1 ? ch[1] : j == 2 ? ch[2] : ch[3];
      const f32x4 nx = j == 0 ? ch[1] : j == 1 ? ch[2] : ch[3];
      __builtin_nontemporal_store(taps4(lo, nx, t & 3),
                                  reinterpret_cast<f32x4*>(col + (int64_t)(r + kw) * g.L + j0));
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
  // the lane's 4 padded positions are the same in every plane: their source
  // offsets in a plane (-1: the zero pad) are worked out once
  int soff[PER_LANE];
  {
    int hp = i0 / g.Wp, wp = i0 - (i0 / g.Wp) * g.Wp;
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) {
      const int hi = pad_index(hp - g.ph, g.H, g.pad_mode);
      const int wi = pad_index(wp - g.pw, g.W, g.pad_mode);
      soff[e] = (i0 + e < hw && hi >= 0 && wi >= 0) ? hi * g.W + wi : -1;
      if (++wp == g.Wp) {
        wp = 0;
        ++hp;
      }
    }
  }
  const T* src = reinterpret_cast<const T*>(x);
  T* dst = reinterpret_cast<T*>(y);
  const bool whole = (hw & 3) == 0 && i0 + PER_LANE <= hw;
  for (int64_t p = blockIdx.y; p < g.planes; p += gridDim.y) {
    const T* plane = src + p * g.H * g.W;
    T v[PER_LANE];
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) v[e] = soff[e] >= 0 ? plane[soff[e]] : (T)0;
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
  if (L > 0x7FFFFFFF - SPAN || rows > 0x7FFFFFFF || C * H * W > 0x7FFFFFFF || OH * sh + KH > 0x3FFFFFFF ||
      OW * sw + KW > 0x3FFFFFFF)
    return NOVAQ_EINVAL;
  if (L == 0) return NOVAQ_OK;
  ColGeom g{(int)C, (int)H, (int)W, KH, KW, sh, sw, ph, pw, pad_mode, (int)OH, (int)OW, (int)L,
            (int)rows, (int)((L + SPAN - 1) / SPAN)};
  // about WG_PER_CU workgroups per CU, each walking rows (one output row of
  // SPAN columns is a single 4 KB store per workgroup: too little per launch)
  const int64_t ry = std::max<int64_t>(1, (int64_t)device_cu_count() * WG_PER_CU / g.segs);
  const dim3 grid((unsigned)g.segs, (unsigned)std::min<int64_t>(std::min<int64_t>(rows, ry), MAX_GRID_Y));
  const auto* xb = static_cast<const uint8_t*>(x);
  const int64_t x_bytes = N * C * H * W * (dtype_bits(x_dtype) / 8);
  if (x_dtype == F32 && pad_mode == NOVAQ_PAD_ZEROS && sh == 1 && sw == 1 && W % 4 == 0 &&
      OW % 4 == 0 && KW <= 7 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
      x_bytes < (int64_t)COL_OOB) {
    // row blocks of whole (c, kh) groups
    const int64_t per = (rows + grid.y - 1) / grid.y;
    const int64_t rpw = (per + KW - 1) / KW * KW;
    const dim3 g2(grid.x, (unsigned)((rows + rpw - 1) / rpw));
    hipLaunchKernelGGL(im2col_rows4_kernel, g2, dim3(THREADS), 0, stream,
                       static_cast<const float*>(x), col, g, (int)x_bytes, (int)rpw);
    return check_launch();
  }
  auto go = [&](auto xt) {
    constexpr int XT = decltype(xt)::value;
    if (pad_mode == NOVAQ_PAD_ZEROS)
      hipLaunchKernelGGL((im2col_kernel<XT, true>), grid, dim3(THREADS), 0, stream, xb, x_scale, col, g);
    else
      hipLaunchKernelGGL((im2col_kernel<XT, false>), grid, dim3(THREADS), 0, stream, xb, x_scale, col, g);
    return check_launch();
  };
  switch (x_dtype) {
    case F32: return go(std::integral_constant<int, F32>{});
    case F16: return go(std::integral_constant<int, F16>{});
    case BF16: return go(std::integral_constant<int, BF16>{});
    case E4M3: return go(std::integral_constant<int, E4M3>{});
    case E5M2: return go(std::integral_constant<int, E5M2>{});
    default: return NOVAQ_EDTYPE;
  }
}

int pad2d_launch(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int ph,
                 int pw, int pad_mode, void* y, hipStream_t stream) {
  const int64_t Hp = H + 2 * (int64_t)ph, Wp = W + 2 * (int64_t)pw;
  if (Hp * Wp > 0x7FFFFFFF - SPAN || H * W > 0x7FFFFFFF) return NOVAQ_EINVAL;
  const int64_t planes = N * C;
  if (planes == 0) return NOVAQ_OK;
  PadGeom g{(int)H, (int)W, ph, pw, pad_mode, (int)Hp, (int)Wp, planes};
  const int64_t segs = (Hp * Wp + SPAN - 1) / SPAN;
  const int64_t py = std::max<int64_t>(1, (int64_t)device_cu_count() * WG_PER_CU / segs);
  const dim3 grid((unsigned)segs,
                  (unsigned)std::min<int64_t>(std::min<int64_t>(planes, py), MAX_GRID_Y));
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
