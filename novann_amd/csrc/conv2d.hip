// Quantized-weight Conv2d forward (NCHW, implicit im2col) on bf16 MFMA.
//
//   y[n, co, oh, ow] = bias[co] + s * sum_{c, kh, kw} dec(w[co, c, kh, kw]) *
//                      xpad[n, c, oh*sh + kh - ph, ow*sw + kw - pw]
//
// GEMM view: M = output channels, N = output pixels of one image, K = the
// (kh, kw, c) window.  NovaNN materialises the (C*KH*KW, N*OH*OW) column
// matrix (novann/functional.py:346-368); here no column matrix exists:
//   - a workgroup owns 64 output channels and a run of 256 consecutive output
//     pixels of one image (4 waves x 64 pixels);
//   - the input rows that run touches are staged in LDS channel-last,
//     [row][col][c] in bf16, with the padding mode (zeros / reflect /
//     replicate / circular, numpy.pad's index rules) resolved while staging,
//     so the MFMA loop has no bounds logic;
//   - K is ordered (kh, kw, c) with c padded to a multiple of 8, so the 8
//     consecutive K values an MFMA lane needs are 8 channels of one input
//     pixel: one 16-byte LDS read;
//   - the weights are decoded once per workgroup into LDS as a [co][k] bf16
//     matrix (exact for E4M3 / E5M2 / E2M1) and the scale and bias are
//     applied in fp32 after accumulation;
//   - the result is written straight to contiguous NCHW (32 consecutive
//     pixels of one channel per store instruction).
// Workgroups loop over pixel tiles (grid sized to the CU count) so the weight
// decode is paid once per workgroup, not once per tile.  More than 64 input
// channels are processed in blocks of 64 (weights then restaged per block).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int THREADS = 256;
constexpr int CO_TILE = 64;
constexpr int PIX_WAVE = 64;
constexpr int PIX_TILE = PIX_WAVE * (THREADS / 64);
constexpr int MAX_CB = 64;
constexpr size_t LDS_LIMIT = 160 * 1024;

struct ConvGeom {
  int N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, pad_mode;
  int OH, OW;
  int CB;        // channels per block (multiple of 8, <= 64)
  int cstride;   // bf16 per staged input pixel (CB, +8 if CB/8 is even)
  int groups;    // K groups of 8 per channel block = KH*KW*CB/8
  int ksteps;    // ceil(groups / 2)
  int wrow;      // bf16 per weight LDS row = 16*ksteps + 8
  int rows;      // staged input rows per tile
  int wp;        // staged input columns
  int tiles_per_image;
  int64_t tiles;
};

__device__ __forceinline__ int pad_index(int i, int n, int mode) {
  if (i >= 0 && i < n) return i;
  if (mode == NOVAQ_PAD_ZEROS) return -1;
  if (mode == NOVAQ_PAD_REPLICATE) return i < 0 ? 0 : n - 1;
  if (mode == NOVAQ_PAD_CIRCULAR) {
    int r = i % n;
    return r < 0 ? r + n : r;
  }
  if (n == 1) return 0;  // reflect, period 2(n-1)
  int p = 2 * (n - 1);
  int r = i % p;
  if (r < 0) r += p;
  return r >= n ? p - r : r;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return (uint16_t)enc_bf16(__float_as_uint(f));
}

// Decoded weight element e (flat (co, c, kh, kw) index) as bf16 bits.
template <int WT>
__device__ __forceinline__ uint16_t weight_bf16(const uint8_t* __restrict__ w, int64_t e) {
  uint32_t f;
  if constexpr (WT == E4M3) f = dec_e4m3(w[e]);
  else if constexpr (WT == E5M2) f = dec_e5m2(w[e]);
  else if constexpr (WT == E2M1) f = dec_e2m1((w[e >> 1] >> ((e & 1) * 4)) & 0xFu);
  else if constexpr (WT == BF16) return reinterpret_cast<const uint16_t*>(w)[e];
  else if constexpr (WT == F16) f = dec_f16(reinterpret_cast<const uint16_t*>(w)[e]);
  else f = reinterpret_cast<const uint32_t*>(w)[e];
  // FP8 / FP4 values are exact in bf16; fp16 / fp32 weights round to nearest even
  return (uint16_t)enc_bf16(f);
}

template <int WT>
__global__ __launch_bounds__(THREADS, 2) void conv2d_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ w_scale,
    const float* __restrict__ bias, float* __restrict__ y, ConvGeom g) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* wl = lds;                                  // [CO_TILE][g.wrow]
  uint16_t* xl = lds + CO_TILE * g.wrow;               // [rows][wp][cstride]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  const int co0 = blockIdx.y * CO_TILE;
  const int cblocks = (g.C + g.CB - 1) / g.CB;
  const int npix = g.OH * g.OW;
  const int c8 = g.CB / 8;
  const bool two_m = co0 + 32 < g.C_out;
  const float s = w_scale ? *w_scale : 1.0f;

  auto stage_weights = [&](int cb) {
    const int kcols = 16 * g.ksteps;
    for (int idx = tid; idx < CO_TILE * kcols; idx += THREADS) {
      const int co = idx / kcols, k = idx - co * kcols;
      const int grp = k >> 3;
      uint16_t v = 0;
      if (grp < g.groups && co0 + co < g.C_out) {
        const int khkw = grp / c8;
        const int c = cb * g.CB + (grp - khkw * c8) * 8 + (k & 7);
        if (c < g.C) {
          const int kh = khkw / g.KW, kw = khkw - kh * g.KW;
          const int64_t e = (((int64_t)(co0 + co) * g.C + c) * g.KH + kh) * g.KW + kw;
          v = weight_bf16<WT>(w, e);
        }
      }
      wl[co * g.wrow + k] = v;
    }
  };

  if (cblocks == 1) stage_weights(0);

  for (int64_t tile = blockIdx.x; tile < g.tiles; tile += gridDim.x) {
    const int n = (int)(tile / g.tiles_per_image);
    const int p0 = (int)(tile - (int64_t)n * g.tiles_per_image) * PIX_TILE;
    const int oh_first = p0 / g.OW;
    const int ih0 = oh_first * g.sh - g.ph;

    // per-lane pixel bases (in staged-input elements) for the two 32-pixel blocks
    int pbase[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      int p = p0 + wave * PIX_WAVE + nt * 32 + (lane & 31);
      if (p >= npix) p = p0;  // read something valid; never stored
      const int oh = p / g.OW, ow = p - oh * g.OW;
      pbase[nt] = (((oh - oh_first) * g.sh) * g.wp + ow * g.sw) * g.cstride;
    }

    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    for (int cb = 0; cb < cblocks; ++cb) {
      __syncthreads();  // previous readers of the LDS tile are done
      if (cblocks > 1) stage_weights(cb);
      // stage input rows [ih0, ih0 + rows) x cols [-pw, -pw + wp), channels of block cb
      const int per_c = g.rows * g.wp;
      for (int idx = tid; idx < g.CB * per_c; idx += THREADS) {
        const int c = idx / per_c;
        const int rc = idx - c * per_c;
        const int r = rc / g.wp, col = rc - r * g.wp;
        const int cg = cb * g.CB + c;
        float v = 0.0f;
        if (cg < g.C) {
          const int hi = pad_index(ih0 + r, g.H, g.pad_mode);
          const int wi = pad_index(col - g.pw, g.W, g.pad_mode);
          if (hi >= 0 && wi >= 0) v = x[(((int64_t)n * g.C + cg) * g.H + hi) * g.W + wi];
        }
        xl[(r * g.wp + col) * g.cstride + c] = f32_to_bf16_rne(v);
      }
      __syncthreads();

      for (int st = 0; st < g.ksteps; ++st) {
        const int grp = 2 * st + half;
        const bool live = grp < g.groups;
        int koff = 0;
        if (live) {
          const int khkw = grp / c8;
          const int kh = khkw / g.KW, kw = khkw - kh * g.KW;
          koff = (kh * g.wp + kw) * g.cstride + (grp - khkw * c8) * 8;
        }
        const int kcol = st * 16 + half * 8;
        bf16x8 a0 = *reinterpret_cast<const bf16x8*>(&wl[(lane & 31) * g.wrow + kcol]);
        bf16x8 a1 = *reinterpret_cast<const bf16x8*>(&wl[(32 + (lane & 31)) * g.wrow + kcol]);
        bf16x8 b[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          if (live) {
            b[nt] = *reinterpret_cast<const bf16x8*>(&xl[pbase[nt] + koff]);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) b[nt][j] = (__bf16)0.0f;
          }
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          acc[0][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b[nt], acc[0][nt], 0, 0, 0);
          if (two_m)
            acc[1][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b[nt], acc[1][nt], 0, 0, 0);
        }
      }
    }

    // epilogue: lane holds pixel (lane & 31) of each 32-block and channels
    // 8*(r/4) + 4*half + r%4 of each 32-channel block
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      if (mt == 1 && !two_m) break;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int p = p0 + wave * PIX_WAVE + nt * 32 + (lane & 31);
        if (p >= npix) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int co = co0 + mt * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          if (co < g.C_out) {
            const float bv = bias ? bias[co] : 0.0f;
            y[((int64_t)n * g.C_out + co) * npix + p] = acc[mt][nt][r] * s + bv;
          }
        }
      }
    }
  }
}

template <int WT>
int launch(const float* x, const void* w, const float* w_scale, const float* bias, float* y,
           ConvGeom g, hipStream_t stream) {
  // staged rows for a run of PIX_TILE pixels: it spans at most
  // ceil((PIX_TILE - 1) / OW) + 1 output rows
  const int out_rows = (PIX_TILE - 1) / g.OW + 2;
  g.rows = (out_rows - 1) * g.sh + g.KH;
  g.wp = (g.OW - 1) * g.sw + g.KW;
  const size_t lds = (size_t)CO_TILE * g.wrow * 2 + (size_t)g.rows * g.wp * g.cstride * 2;
  if (lds > LDS_LIMIT) return NOVAQ_ENOTSUP;  // rows too wide for one LDS tile
  auto kern = conv2d_kernel<WT>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return hip_fail(e);
  }
  const int64_t co_blocks = (g.C_out + CO_TILE - 1) / CO_TILE;
  int64_t grid = (int64_t)device_cu_count() * 2;
  if (grid > g.tiles) grid = g.tiles;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid, (unsigned)co_blocks), dim3(THREADS), lds, stream, x,
                     static_cast<const uint8_t*>(w), w_scale, bias, y, g);
  return check_launch();
}

}  // namespace

int conv2d_launch(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const void* w_q,
                  int w_dtype, const float* w_scale, int64_t C_out, int KH, int KW, int sh,
                  int sw, int ph, int pw, int pad_mode, const float* bias, float* y,
                  hipStream_t stream) {
  const int64_t OH = (H + 2 * (int64_t)ph - KH) / sh + 1;
  const int64_t OW = (W + 2 * (int64_t)pw - KW) / sw + 1;
  if (OH <= 0 || OW <= 0) return NOVAQ_ESHAPE;
  if (N > 0x7FFFFFFF || C > 0x7FFFFFFF || H * W > 0x7FFFFFFF || C_out > 65535 * CO_TILE ||
      OH * OW > 0x7FFFFFFF)
    return NOVAQ_EINVAL;
  ConvGeom g{};
  g.N = (int)N; g.C = (int)C; g.H = (int)H; g.W = (int)W; g.C_out = (int)C_out;
  g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw; g.ph = ph; g.pw = pw; g.pad_mode = pad_mode;
  g.OH = (int)OH; g.OW = (int)OW;
  const int cpad = (int)((C + 7) / 8 * 8);
  g.CB = cpad < MAX_CB ? cpad : MAX_CB;
  g.cstride = ((g.CB / 8) % 2 == 0) ? g.CB + 8 : g.CB;
  g.groups = KH * KW * g.CB / 8;
  g.ksteps = (g.groups + 1) / 2;
  g.wrow = 16 * g.ksteps + 8;
  g.tiles_per_image = (int)((OH * OW + PIX_TILE - 1) / PIX_TILE);
  g.tiles = (int64_t)N * g.tiles_per_image;
  switch (w_dtype) {
    case E4M3: return launch<E4M3>(x, w_q, w_scale, bias, y, g, stream);
    case E5M2: return launch<E5M2>(x, w_q, w_scale, bias, y, g, stream);
    case E2M1: return launch<E2M1>(x, w_q, w_scale, bias, y, g, stream);
    case BF16: return launch<BF16>(x, w_q, w_scale, bias, y, g, stream);
    case F16: return launch<F16>(x, w_q, w_scale, bias, y, g, stream);
    case F32: return launch<F32>(x, w_q, w_scale, bias, y, g, stream);
    default: return NOVAQ_EDTYPE;
  }
}

}  // namespace novaq
