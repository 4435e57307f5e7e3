// Quantized-weight Conv2d forward (NCHW, implicit im2col) on bf16 MFMA --
// kernels, included by one translation unit per stored dtype of x
// (conv2d.hip: fp32 x and the dispatch; conv2d_x*.hip: the others).
//
//   y[n, co, oh, ow] = epilogue(bias[co] + s_w * s_x * sum_{c, kh, kw}
//                      dec(w[co, c, kh, kw]) * xpad[n, c, oh*sh + kh - ph,
//                      ow*sw + kw - pw])
//
// x is fp32, or bf16 / f16 / FP8 as a fused epilogue stored it; it becomes
// bf16 while it is staged (fp32 and f16 rounded to nearest even, bf16 and
// FP8 exact).
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
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "novaq_convert.h"
#include "novaq_epilogue.h"
#include "novaq_internal.h"
#include "novaq_xload.h"

namespace novaq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int THREADS = 256;
constexpr int CO_TILE = 64;
constexpr int PIX_WAVE = 64;
constexpr int PIX_TILE = PIX_WAVE * (THREADS / 64);
constexpr int MAX_CB = 64;
// workgroups per CU the registers are sized for (the grid is CUs x this), and
// input-staging items per thread whose loads are issued together
#ifndef CONV_OCC
#define CONV_OCC 2
#endif
#ifndef CONV_IB
#define CONV_IB 4
#endif
constexpr size_t LDS_LIMIT = 160 * 1024;
// LDS bytes of a band workgroup that still lets four share a CU
constexpr size_t BAND_LDS_FOUR = 40 * 1024;

struct ConvGeom {
  int N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, pad_mode;
  int OH, OW;
  int CB;        // channels per block (multiple of 8, <= 64)
  int cstride;   // bf16 per staged input pixel (CB, +8 if CB/8 is even)
  int groups;    // K groups of 8 per channel block = KH*KW*CB/8
  int ksteps;    // ceil(groups / 2)
  int wrow;      // bytes per weight LDS row (2*ksteps K groups, padded for banks)
  int rows;      // staged input rows per tile
  int wp;        // staged input columns
  int tiles_per_image;
  int raw_in_lds;  // weights staged through a raw LDS copy (one channel block, fits)
  int64_t tiles;
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return (uint16_t)enc_bf16(__float_as_uint(f));
}

// Bytes of one 8-wide K group of a weight row in LDS: the packed codes for
// E2M1 (4 B) and E4M3 / E5M2 (8 B), decoded bf16 otherwise (16 B).
template <int WT>
__host__ __device__ constexpr int group_bytes() {
  return WT == E2M1 ? 4 : (WT == E4M3 || WT == E5M2) ? 8 : 16;
}

// Stored code of weight element e (E2M1 nibble or FP8 byte).
template <int WT>
__device__ __forceinline__ uint32_t weight_code(const uint8_t* __restrict__ w, int64_t e) {
  if constexpr (WT == E2M1) return (w[e >> 1] >> ((e & 1) * 4)) & 0xFu;
  else return w[e];
}

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

// One lane's A fragment (8 weights of one K group) from LDS as 8 bf16; FP8
// and FP4 codes are decoded exactly with gfx950's packed converts.
template <int WT>
__device__ __forceinline__ bf16x8 weight_frag(const uint8_t* p) {
  if constexpr (WT == E2M1) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    uint32_t o[4];
    o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 0));
    o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 1));
    o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 2));
    o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 3));
    return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
  } else if constexpr (WT == E4M3 || WT == E5M2) {
    const u32x2v v = *reinterpret_cast<const u32x2v*>(p);
    const uint32_t lo = v[0], hi = v[1];
    uint32_t o[4];
    if constexpr (WT == E4M3) {
      o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
      o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
      o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
      o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
    } else {
      o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(lo, 1.0f, false));
      o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(lo, 1.0f, true));
      o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(hi, 1.0f, false));
      o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(hi, 1.0f, true));
    }
    return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
  } else {
    return *reinterpret_cast<const bf16x8*>(p);
  }
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

template <int WT, int XT>
__global__ __launch_bounds__(THREADS, CONV_OCC) void conv2d_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale,
    Epilogue ep, void* __restrict__ y, ConvGeom g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int GB = group_bytes<WT>();
  uint8_t* wl = lds;                                                     // [CO_TILE][g.wrow B]
  uint16_t* xl = reinterpret_cast<uint16_t*>(lds + CO_TILE * g.wrow);    // [rows][wp][cstride]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  const int co0 = blockIdx.y * CO_TILE;
  const int cblocks = (g.C + g.CB - 1) / g.CB;
  const int npix = g.OH * g.OW;
  const int c8 = g.CB / 8;
  const bool two_m = co0 + 32 < g.C_out;
  const float s = product_scale(w_scale, x_scale);
  const float inv_o = epi_inv_scale(ep);
  uint32_t am = 0;

  // Weights: one item = (output channel, group of 8 consecutive K values), i.e.
  // 8 channels of one (kh, kw) tap, written as one LDS group: 8 packed E2M1
  // nibbles (4 B), 8 FP8 bytes (8 B) or 8 decoded bf16 (16 B).  Channels
  // past C and K groups past the window are zeros (code 0 is +0 in every
  // format).  `src` holds the (co, c, kh, kw) weights in storage order
  // starting at output channel `cofs` (the global tensor, or its raw copy).
  auto stage_weights = [&](int cb, const uint8_t* src, int cofs) {
    const int gpr = 2 * g.ksteps;  // 8-wide K groups per LDS row
    const int cstep = g.KH * g.KW;
    for (int it = tid; it < CO_TILE * gpr; it += THREADS) {
      const int co = it / gpr, grp = it - co * gpr;
      uint32_t p[4] = {0u, 0u, 0u, 0u};
      if (grp < g.groups && co0 + co < g.C_out) {
        const int khkw = grp / c8;
        const int cbase = cb * g.CB + (grp - khkw * c8) * 8;
        const int64_t e0 = ((int64_t)(co0 + co - cofs) * g.C + cbase) * cstep + khkw;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (cbase + j >= g.C) continue;
          if constexpr (GB == 4) {
            p[0] |= weight_code<WT>(src, e0 + j * cstep) << (4 * j);
          } else if constexpr (GB == 8) {
            p[j >> 2] |= weight_code<WT>(src, e0 + j * cstep) << (8 * (j & 3));
          } else {
            p[j >> 1] |= (uint32_t)weight_bf16<WT>(src, e0 + j * cstep) << ((j & 1) * 16);
          }
        }
      }
      uint8_t* d = wl + co * g.wrow + grp * GB;
      if constexpr (GB == 4) *reinterpret_cast<uint32_t*>(d) = p[0];
      else if constexpr (GB == 8) *reinterpret_cast<u32x2v*>(d) = u32x2v{p[0], p[1]};
      else *reinterpret_cast<uint4*>(d) = make_uint4(p[0], p[1], p[2], p[3]);
    }
  };
  // Raw copy of this workgroup's weight rows into the (not yet used) input
  // tile region with coalesced dword loads, all in flight at once; the
  // decode above then reads LDS instead of issuing dependent global loads.
  // Used when all channels fit one block and the raw rows fit the region.
  auto stage_weights_via_lds = [&]() {
    const int rows = min(CO_TILE, g.C_out - co0);
    const int64_t row_elems = (int64_t)g.C * g.KH * g.KW;
    const int64_t first = (int64_t)co0 * row_elems;  // first element (even: co0 % 64 == 0)
    const int nbytes = (int)(rows * row_elems * dtype_bits(WT) / 8 + (dtype_bits(WT) == 4 ? (rows * row_elems) & 1 : 0));
    const uint8_t* gsrc = w + first * dtype_bits(WT) / 8;  // 4-byte aligned (row_elems * 64 elems)
    uint8_t* raw = reinterpret_cast<uint8_t*>(xl);
    const int nwords = nbytes >> 2;
#pragma unroll 8
    for (int i = tid; i < nwords; i += THREADS)
      reinterpret_cast<uint32_t*>(raw)[i] = reinterpret_cast<const uint32_t*>(gsrc)[i];
    for (int i = (nwords << 2) + tid; i < nbytes; i += THREADS) raw[i] = gsrc[i];
    __syncthreads();
    stage_weights(0, raw, co0);
  };

  // window offset (in staged-input elements) of each 8-wide K group, -1 for
  // the padding group past the window
  int* ktab = reinterpret_cast<int*>(xl + g.rows * g.wp * g.cstride);
  for (int i = tid; i < 2 * g.ksteps; i += THREADS) {
    int koff = -1;
    if (i < g.groups) {
      const int khkw = i / c8;
      const int kh = khkw / g.KW, kw = khkw - kh * g.KW;
      koff = (kh * g.wp + kw) * g.cstride + (i - khkw * c8) * 8;
    }
    ktab[i] = koff;
  }

  if (cblocks == 1) {
    if (g.raw_in_lds) stage_weights_via_lds();
    else stage_weights(0, w, 0);
  }

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
      if (cblocks > 1) stage_weights(cb, w, 0);
      // Stage input rows [ih0, ih0 + rows) x cols [-pw, -pw + wp) of channel
      // block cb.  One item = one staged pixel x 8 channels: 8 independent
      // loads (consecutive lanes take consecutive pixels, so each load
      // instruction reads a contiguous row segment), 4 packed bf16 converts
      // (RNE) and one 16-byte LDS write.
      const int pix = g.rows * g.wp;
      const int total = pix * c8;
      const int64_t hw = (int64_t)g.H * g.W;
      // batches of IB items per thread: all 8*IB loads are issued before the
      // first conversion
      constexpr int IB = CONV_IB;
      for (int base = 0; base < total; base += IB * THREADS) {
        float v[IB][8];
        int dst[IB];
#pragma unroll
        for (int b = 0; b < IB; ++b) {
          const int it = base + b * THREADS + tid;
          dst[b] = -1;
#pragma unroll
          for (int j = 0; j < 8; ++j) v[b][j] = 0.0f;
          if (it < total) {
            const int cgi = it / pix, p = it - cgi * pix;
            const int r = p / g.wp, col = p - r * g.wp;
            const int hi = pad_index(ih0 + r, g.H, g.pad_mode);
            const int wi = pad_index(col - g.pw, g.W, g.pad_mode);
            const int cbase = cb * g.CB + cgi * 8;
            dst[b] = (r * g.wp + col) * g.cstride + cgi * 8;
            if (hi >= 0 && wi >= 0) {
              const int64_t src = ((int64_t)n * g.C + cbase) * hw + (int64_t)hi * g.W + wi;
#pragma unroll
              for (int j = 0; j < 8; ++j)
                if (cbase + j < g.C) v[b][j] = x_val<XT>(x, src + j * hw);
            }
          }
        }
#pragma unroll
        for (int b = 0; b < IB; ++b) {
          if (dst[b] < 0) continue;
          uint32_t q[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            f32x2 f = {v[b][2 * j], v[b][2 * j + 1]};
            q[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
          }
          *reinterpret_cast<uint4*>(&xl[dst[b]]) = make_uint4(q[0], q[1], q[2], q[3]);
        }
      }
      __syncthreads();

      // fragments of K step st into register set `buf`; the window offset
      // of each 8-wide K group comes from the per-workgroup table (-1: the
      // zero padding group past the window)
      bf16x8 fa0[2], fa1[2], fb[2][2];
      auto load = [&](int st, int buf) {
        const int koff = ktab[2 * st + half];
        const int kbyte = (2 * st + half) * GB;
        fa0[buf] = weight_frag<WT>(wl + (lane & 31) * g.wrow + kbyte);
        fa1[buf] = weight_frag<WT>(wl + (32 + (lane & 31)) * g.wrow + kbyte);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          if (koff >= 0) {
            fb[buf][nt] = *reinterpret_cast<const bf16x8*>(&xl[pbase[nt] + koff]);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) fb[buf][nt][j] = (__bf16)0.0f;
          }
        }
      };
      auto mfma = [&](int buf) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          acc[0][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa0[buf], fb[buf][nt], acc[0][nt], 0, 0, 0);
          if (two_m)
            acc[1][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa1[buf], fb[buf][nt], acc[1][nt], 0, 0, 0);
        }
      };
      // the next step's fragments are read while the current step multiplies
      load(0, 0);
      for (int st = 0; st < g.ksteps; st += 2) {
        if (st + 1 < g.ksteps) load(st + 1, 1);
        mfma(0);
        if (st + 1 < g.ksteps) {
          if (st + 2 < g.ksteps) load(st + 2, 0);
          mfma(1);
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
            const float v = epi_value(ep, epi_chan(ep, co), acc[mt][nt][r], s);
            if (ep.amax) am = epi_track(am, v);
            epi_store(ep.out_dtype, y, ((int64_t)n * g.C_out + co) * npix + p, v, inv_o);
          }
        }
      }
    }
  }
  epi_amax_commit(ep, am);
}

// ---------------------------------------------------------------------------
// Band kernel (C <= 64 input channels, at most 256 output pixels per band).
//
// A workgroup owns up to 64 output channels of one band of R whole output
// rows of one image; the band's output is R*OW consecutive floats of each
// channel plane.  GEMM orientation per band: M = the band's pixels in
// 16-pixel tiles, N = output channels in 16-channel tiles, K = (kh, kw, c) in
// 8-channel groups, on v_mfma_f32_16x16x32_bf16.  With pixels as rows, a
// lane's four accumulators are four consecutive pixels of one channel: one
// 16-byte store.
//   - the weights of the workgroup's output channels are regrouped once from
//     (co, c, kh, kw) order into (co, [kh, kw, 8 channels]) groups in LDS,
//     FP8 / FP4 codes kept packed and decoded per MFMA fragment (exact);
//   - the band's input rows are staged in LDS channel-last in bf16 (RNE);
//     whole 4-column groups of the interior come in as 16-byte loads of 8
//     channels (bf16 x: its codes as they are), issued into registers before
//     the weights are regrouped (when there is at most one such item per
//     thread) so their latency overlaps that work, and are transposed in
//     registers; padding columns are
//     resolved element-wise with numpy.pad's index rules;
//   - many small workgroups per CU: one's loads overlap another's MFMAs and
//     stores.

struct BandGeom {
  int N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, pad_mode, OH, OW;
  int c8;        // 8-channel groups (C padded to a multiple of 8)
  int passes;    // channel passes: the band's input staged pc8 groups at a time
  int pc8;       // 8-channel groups staged per pass
  int cstride;   // bf16 per staged pixel
  int taps;      // KH * KW
  int groups;    // taps * c8 K groups of 8
  int gpr;       // groups rounded up to whole MFMA K steps (4 groups)
  int wrow;      // bytes per weight row in LDS
  int co_rows;   // weight rows staged in LDS (C_out rounded up to 16, at most 64)
  int R;         // output rows per band
  int bands;     // bands per image
  int rows_in;   // staged input rows per band
  int wp;        // staged input columns
  int nborder;   // staged columns outside [0, W) (element-wise path)
  int vec;       // interior columns staged with 16-byte loads (W % 4 == 0)
  int vitems;    // 16-byte-load items per band and pass (rows_in * W/4 * pc8)
  int raw_ok;    // packed weights copied to LDS before regrouping
  int x_off;     // LDS byte offset of the staged input
  int x_bytes;   // bytes of the staged input (one pass)
  int ostage;    // narrow output stored through LDS (whole store units per channel row)
  // dividers for the per-item index arithmetic: c8, W / 4, OW, KW and the
  // element-wise staged columns (a run-time integer division is a long
  // instruction sequence; these are a multiply-high, an add and a shift)
  FastDiv fd_c8, fd_w4, fd_ow, fd_kw, fd_nc, fd_pc8;
};

typedef float f32x4 __attribute__((ext_vector_type(4)));

// A staging item's registers: 8 channels x 4 columns as fp32 values, or for
// bf16 x the raw codes (two words a channel): the staged layout is bf16, so
// bf16 codes move as they are, never widened and narrowed again.
template <int XT>
struct BandItem {
  f32x4 v[8];
};
template <>
struct BandItem<BF16> {
  uint32_t w[8][2];
};

// 16-byte-load items of one band held in registers: IPT items per thread.
template <int IPT, int XT>
struct BandRegs {
  BandItem<XT> v[IPT > 0 ? IPT : 1];
};

// K9: 3x3 window, C a multiple of 8 and packed FP8 / FP4 codes copied to LDS:
// the 8 channels x 9 taps of one (co, channel group) are 72 consecutive codes
// (aligned 32-bit words), regrouped with constant shifts.
template <int WT, int XT, int IPT, bool K9>
__global__ __launch_bounds__(THREADS, 2) void conv2d_band_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale,
    Epilogue ep, void* __restrict__ y, BandGeom g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int GB = group_bytes<WT>();
  uint8_t* wl = lds;                                           // [g.co_rows][g.wrow]
  int* ktab = reinterpret_cast<int*>(lds + g.co_rows * g.wrow);  // [g.gpr]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int band = blockIdx.x % g.bands, n = blockIdx.x / g.bands;
  const int co0 = blockIdx.y * CO_TILE;
  const int64_t HW = (int64_t)g.H * g.W;
  const int64_t xn = (int64_t)n * g.C * HW;  // element offset of image n
  const int W4 = g.W >> 2;

  // 16-byte-load item `it` of band b, pass ps: (row r, column group cg,
  // channel group q of the pass)
  auto vload = [&](int b, int ps, int it, BandItem<XT>& v) {
    const int rest = (int)fdiv((uint32_t)it, g.fd_pc8), q = it - rest * g.pc8;
    const int r = (int)fdiv((uint32_t)rest, g.fd_w4), cg = rest - r * W4;
    const int hi = pad_index(b * g.R * g.sh - g.ph + r, g.H, g.pad_mode);
    const bool used = cg * 4 + g.pw < g.wp;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = (ps * g.pc8 + q) * 8 + j;
      const bool live = used && hi >= 0 && c < g.C;
      const int64_t e = xn + c * HW + (int64_t)hi * g.W + cg * 4;
      if constexpr (XT == BF16) {
        v.w[j][0] = v.w[j][1] = 0u;
        if (live) {
          const xl_u32x4 raw = x4_raw<BF16>(x, e);
          const uint32_t w0 = raw[0], w1 = raw[1];
          v.w[j][0] = w0;
          v.w[j][1] = w1;
        }
      } else {
        v.v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (live) v.v[j] = x4_f32<XT>(x, e);
      }
    }
  };
  // --- weights: (co, c, kh, kw) -> [co][K group] ---------------------------
  const int row_elems = g.C * g.taps;
  const uint8_t* src = w;
  int cofs = 0;
  // packed codes of rows co0 .. co0+63 (the first element is even, so the
  // E2M1 byte boundary matches), coalesced dwords then bytes, into the
  // staged-input region.  The first RAW_REGS dwords per lane are loaded into
  // registers before the band's loads are issued, so writing them to LDS
  // waits for those few loads only, not for the band behind them.
  constexpr int RAW_REGS = 12;
  uint32_t rw[RAW_REGS];
  int nbytes = 0, nwords = 0;
  const uint8_t* gsrc = w;
  if (g.raw_ok) {
    const int rows = min(CO_TILE, g.C_out - co0);
    const int64_t first = (int64_t)co0 * row_elems;
    nbytes = (int)(((int64_t)rows * row_elems * dtype_bits(WT) + 7) / 8);
    gsrc = w + first * dtype_bits(WT) / 8;
    nwords = (reinterpret_cast<uintptr_t>(gsrc) & 3) ? 0 : nbytes >> 2;
#pragma unroll
    for (int k = 0; k < RAW_REGS; ++k) {
      const int i = tid + k * THREADS;
      rw[k] = i < nwords ? reinterpret_cast<const uint32_t*>(gsrc)[i] : 0u;
    }
  }
  // then the band's 16-byte loads
  BandRegs<IPT, XT> r0;
  if constexpr (IPT > 0) {
    if (tid < g.vitems) vload(band, 0, tid, r0.v[0]);
  }
  if (g.raw_ok) {
    uint8_t* raw = lds + g.x_off;
#pragma unroll
    for (int k = 0; k < RAW_REGS; ++k) {
      const int i = tid + k * THREADS;
      if (i < nwords) reinterpret_cast<uint32_t*>(raw)[i] = rw[k];
    }
    for (int i = tid + RAW_REGS * THREADS; i < nwords; i += THREADS)
      reinterpret_cast<uint32_t*>(raw)[i] = reinterpret_cast<const uint32_t*>(gsrc)[i];
    for (int i = (nwords << 2) + tid; i < nbytes; i += THREADS) raw[i] = gsrc[i];
    __syncthreads();
    src = raw;
    cofs = co0;
  }
  if constexpr (K9 && GB < 16) {
    constexpr int BITS = dtype_bits(WT);
    constexpr int NW = 72 * BITS / 32;  // words of one (co, q) run
    for (int item = tid; item < g.co_rows * g.c8; item += THREADS) {
      const int co = (int)fdiv((uint32_t)item, g.fd_c8), q = item - co * g.c8;
      uint32_t o[9][GB / 4];
      if (co0 + co < g.C_out) {
        const uint32_t* run = reinterpret_cast<const uint32_t*>(
            src + (size_t)(co * g.C + q * 8) * 9 * BITS / 8);
        uint32_t wv[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) wv[i] = run[i];
#pragma unroll
        for (int t = 0; t < 9; ++t) {
#pragma unroll
          for (int k = 0; k < GB / 4; ++k) o[t][k] = 0u;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            constexpr uint32_t mask = (1u << BITS) - 1u;
            const int e = 9 * j + t;
            const uint32_t code = (wv[e * BITS / 32] >> ((e * BITS) % 32)) & mask;
            o[t][(j * BITS) / 32] |= code << ((j * BITS) % 32);
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < 9; ++t)
#pragma unroll
          for (int k = 0; k < GB / 4; ++k) o[t][k] = 0u;
      }
#pragma unroll
      for (int t = 0; t < 9; ++t) {
        uint8_t* d = wl + co * g.wrow + (t * g.c8 + q) * GB;
        if constexpr (GB == 4) *reinterpret_cast<uint32_t*>(d) = o[t][0];
        else *reinterpret_cast<u32x2v*>(d) = u32x2v{o[t][0], o[t][1]};
      }
    }
    // zero groups past the window (K padding to whole MFMA steps)
    const int pad = g.gpr - g.groups;
    for (int item = tid; item < g.co_rows * pad; item += THREADS) {
      const int co = item / pad, gi = g.groups + (item - co * pad);
      uint8_t* d = wl + co * g.wrow + gi * GB;
      if constexpr (GB == 4) *reinterpret_cast<uint32_t*>(d) = 0u;
      else *reinterpret_cast<u32x2v*>(d) = u32x2v{0u, 0u};
    }
  } else {
    // four threads per output channel row, each taking every fourth group
    // (rows past g.co_rows are not staged)
    const int co = tid >> 2;
    const bool live = co0 + co < g.C_out;
    const int gend = co < g.co_rows ? g.gpr : 0;
    int tap = 0, q = tid & 3;
    while (q >= g.c8) { q -= g.c8; ++tap; }
    for (int gi = tid & 3; gi < gend; gi += 4) {
      uint32_t p[4] = {0u, 0u, 0u, 0u};
      if (live && gi < g.groups) {
        const int cbase = q * 8;
        const int64_t e0 = ((int64_t)(co0 + co - cofs) * g.C + cbase) * g.taps + tap;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (cbase + j >= g.C) break;
          if constexpr (GB == 4) {
            p[0] |= weight_code<WT>(src, e0 + j * g.taps) << (4 * j);
          } else if constexpr (GB == 8) {
            p[j >> 2] |= weight_code<WT>(src, e0 + j * g.taps) << (8 * (j & 3));
          } else {
            p[j >> 1] |= (uint32_t)weight_bf16<WT>(src, e0 + j * g.taps) << ((j & 1) * 16);
          }
        }
      }
      uint8_t* d = wl + co * g.wrow + gi * GB;
      if constexpr (GB == 4) *reinterpret_cast<uint32_t*>(d) = p[0];
      else if constexpr (GB == 8) *reinterpret_cast<u32x2v*>(d) = u32x2v{p[0], p[1]};
      else *reinterpret_cast<uint4*>(d) = make_uint4(p[0], p[1], p[2], p[3]);
      // advance (tap, q) by four groups
      q += 4;
      while (q >= g.c8) { q -= g.c8; ++tap; }
    }
  }
  // window offset (staged elements) of each K group; -1 past the window
  for (int gi = tid; gi < g.gpr; gi += THREADS) {
    int koff = -1;
    if (gi < g.groups) {
      const int tap = (int)fdiv((uint32_t)gi, g.fd_c8), q = gi - tap * g.c8;
      const int kh = (int)fdiv((uint32_t)tap, g.fd_kw), kw = tap - kh * g.KW;
      koff = (kh * g.wp + kw) * g.cstride + (q % g.pc8) * 8;  // within its pass's staging
    }
    ktab[gi] = koff;
  }
  __syncthreads();  // weights regrouped; the raw copy region is free

  auto vstore = [&](uint16_t* xl, int it, const BandItem<XT>& v) {
    const int rest = (int)fdiv((uint32_t)it, g.fd_pc8), q = it - rest * g.pc8;
    const int r = (int)fdiv((uint32_t)rest, g.fd_w4), cg = rest - r * W4;
    const int col0 = cg * 4 + g.pw;  // staged column of input column 4*cg
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = col0 + i;
      if (col >= g.wp) break;
      uint32_t pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (XT == BF16) {
          // column i's codes of channels 2j and 2j + 1
          const uint32_t a = v.w[2 * j][i >> 1], b2 = v.w[2 * j + 1][i >> 1];
          pk[j] = (i & 1) ? ((a >> 16) | (b2 & 0xFFFF0000u)) : ((a & 0xFFFFu) | (b2 << 16));
        } else {
          f32x2 f = {v.v[2 * j][i], v.v[2 * j + 1][i]};
          pk[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
        }
      }
      *reinterpret_cast<uint4*>(&xl[(r * g.wp + col) * g.cstride + q * 8]) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
  };
  // element-wise columns of pass ps of band b: the padding columns, or
  // every column when the rows are not 16-byte aligned
  auto stage_border = [&](int b, int ps, uint16_t* xl) {
    const int ncols = g.vec ? g.nborder : g.wp;
    const int left = min(g.pw, g.wp);
    const int items = g.rows_in * ncols * g.pc8;
    const int ih0 = b * g.R * g.sh - g.ph;
    for (int it = tid; it < items; it += THREADS) {
      const int rest = (int)fdiv((uint32_t)it, g.fd_pc8), q = it - rest * g.pc8;
      const int r = (int)fdiv((uint32_t)rest, g.fd_nc), bi = rest - r * ncols;
      const int col = !g.vec ? bi : (bi < left ? bi : g.pw + g.W + (bi - left));
      const int hi = pad_index(ih0 + r, g.H, g.pad_mode);
      const int wi = pad_index(col - g.pw, g.W, g.pad_mode);
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int c = (ps * g.pc8 + q) * 8 + j;
        v[j] = (hi >= 0 && wi >= 0 && c < g.C) ? x_val<XT>(x, xn + c * HW + (int64_t)hi * g.W + wi)
                                               : 0.0f;
      }
      uint32_t pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x2 f = {v[2 * j], v[2 * j + 1]};
        pk[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
      }
      *reinterpret_cast<uint4*>(&xl[(r * g.wp + col) * g.cstride + q * 8]) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
  };
  // The 16-byte-load items of pass ps > 0 of band b, while the products'
  // accumulators are live: four channels' loads in flight at a time, written
  // as channel pairs (4-byte LDS stores), so few registers hold staging data.
  auto stage_quads = [&](int b, int ps, uint16_t* xl) {
    for (int it = tid; it < g.vitems; it += THREADS) {
      const int rest = (int)fdiv((uint32_t)it, g.fd_pc8), q = it - rest * g.pc8;
      const int r = (int)fdiv((uint32_t)rest, g.fd_w4), cg = rest - r * W4;
      const int hi = pad_index(b * g.R * g.sh - g.ph + r, g.H, g.pad_mode);
      const int col0 = cg * 4 + g.pw;  // staged column of input column 4*cg
      const bool used = col0 < g.wp && hi >= 0;
      uint16_t* d = &xl[(r * g.wp + col0) * g.cstride + q * 8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = (ps * g.pc8 + q) * 8 + 4 * h + j;
          v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          if (used && c < g.C) v[j] = x4_f32<XT>(x, xn + c * HW + (int64_t)hi * g.W + cg * 4);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (col0 + i >= g.wp) break;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const f32x2 f = {v[2 * j][i], v[2 * j + 1][i]};
            *reinterpret_cast<uint32_t*>(d + i * g.cstride + 4 * h + 2 * j) =
                __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
          }
        }
      }
    }
  };
  // stage pass ps of band b into buffer xl (from the registers when IPT > 0)
  auto stage = [&](const BandRegs<IPT, XT>& rg, int b, int ps, uint16_t* xl) {
    if (g.vec) {
      if constexpr (IPT > 0) {
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
          const int it = tid + k * THREADS;
          if (it < g.vitems) vstore(xl, it, rg.v[k]);
        }
      } else {
        // two items a pass, both items' loads issued before either is
        // stored: one memory latency per pass
        for (int it = tid; it < g.vitems; it += 2 * THREADS) {
          BandItem<XT> v[2];
          const bool two = it + THREADS < g.vitems;
          vload(b, ps, it, v[0]);
          if (two) vload(b, ps, it + THREADS, v[1]);
          vstore(xl, it, v[0]);
          if (two) vstore(xl, it + THREADS, v[1]);
        }
      }
    }
    stage_border(b, ps, xl);
  };

  const float s = product_scale(w_scale, x_scale);
  const float inv_o = epi_inv_scale(ep);
  uint32_t am = 0;
  const bool plain = !ep.mul && !ep.add && !ep.relu && !ep.amax && ep.out_dtype == F32;
  const int64_t npix = (int64_t)g.OH * g.OW;
  const int nt_live = min(4, (min(CO_TILE, g.C_out - co0) + 15) >> 4);
  const uint8_t* wfrag = wl + lr * g.wrow + lg * GB;
  const int steps = g.gpr >> 2;
  const bf16x8 zero8 = __builtin_bit_cast(bf16x8, make_uint4(0u, 0u, 0u, 0u));

  // MFMA and store of band b from buffer xl, which holds pass 0's staging;
  // wave w takes M tiles w, w+4, ...
  auto compute = [&](int b, uint16_t* xl) {
    const int oh0 = b * g.R;
    const int P = min(g.R, g.OH - oh0) * g.OW;
    const int mtiles = (P + 15) >> 4;
    const int my_mt = wave < mtiles ? (mtiles - wave + 3) >> 2 : 0;
    int pb[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      int p = (wave + 4 * m) * 16 + lr;
      if (p >= P) p = 0;  // a valid address; the product is never stored
      const int ohr = (int)fdiv((uint32_t)p, g.fd_ow), ow = p - ohr * g.OW;
      pb[m] = ((ohr * g.sh) * g.wp + ow * g.sw) * g.cstride;
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[m][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // (the fragments are not double-buffered: the extra registers would cost
    // a workgroup per CU, and other workgroups hide the LDS latency)
    auto frags = [&](int st, bf16x8* af, bf16x8* bf) {
      const int koff = ktab[st * 4 + lg];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (t < nt_live) bf[t] = weight_frag<WT>(wfrag + t * 16 * g.wrow + st * 4 * GB);
#pragma unroll
      for (int m = 0; m < 4; ++m)
        if (m < my_mt) af[m] = koff >= 0 ? *reinterpret_cast<const bf16x8*>(&xl[pb[m] + koff]) : zero8;
    };
    auto mma = [&](const bf16x8* af, const bf16x8* bf) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= my_mt) break;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (t < nt_live)
            acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[m], bf[t], acc[m][t], 0, 0, 0);
      }
    };
    // pass ps owns the K steps st = ps (mod passes): the weights' (tap, 8
    // channels) groups run tap-major, so one step is one tap's four channel
    // groups of one pass (at most two passes)
    auto mma_pass = [&](int ps) {
      for (int st = ps; st < steps; st += g.passes) {
        bf16x8 af[4], bf[4];
        frags(st, af, bf);
        mma(af, bf);
      }
    };
    mma_pass(0);
    if (g.passes > 1) {
      __syncthreads();  // every wave's fragment reads of pass 0 are done
      if (g.vec) stage_quads(b, 1, xl);
      stage_border(b, 1, xl);
      __syncthreads();
      mma_pass(1);
    }
    // lane holds pixels 4*lg .. 4*lg+3 of channel lr of each tile; its four
    // channels' epilogue constants are loaded once
    EpiChan kc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int co = co0 + t * 16 + lr;
      kc[t] = (t < nt_live && co < g.C_out) ? epi_chan(ep, co) : EpiChan{0.0f, 1.0f, -0.0f};
    }
    if (plain && (npix & 3) == 0 && ((oh0 * g.OW) & 3) == 0 && (P & 3) == 0) {
      // bias only, fp32 output, every lane's four pixels one aligned 16-byte
      // run (uniform per band): one lane base pointer, constant steps
      // (plain stores: the 64-byte pieces of a line written by neighbouring
      // lanes and waves merge in L2 before they reach HBM)
      float* ybase = reinterpret_cast<float*>(y) +
                     (((int64_t)n * g.C_out + co0 + lr) * npix + (int64_t)oh0 * g.OW);
      const int64_t tstep = 16 * npix;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= my_mt) break;
        const int p = (wave + 4 * m) * 16 + 4 * lg;
        if (p >= P) continue;
        float* dm = ybase + p;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (t >= nt_live || co0 + t * 16 + lr >= g.C_out) continue;
          *reinterpret_cast<f32x4*>(dm + t * tstep) = acc[m][t] * s + kc[t].bias;
        }
      }
      return;
    }
    if (ep.out_dtype == F32 && (npix & 3) == 0 && ((oh0 * g.OW) & 3) == 0 && (P & 3) == 0) {
      // an fp32 output with the epilogue, the same addressing (the values of
      // the general loop below: epi_value_nb per element, the amax over the
      // band's pixels)
      const float z = epi_relu_factor(ep);
      const bool track = ep.amax != nullptr;
      float* ybase = reinterpret_cast<float*>(y) +
                     (((int64_t)n * g.C_out + co0 + lr) * npix + (int64_t)oh0 * g.OW);
      const int64_t tstep = 16 * npix;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= my_mt) break;
        const int p = (wave + 4 * m) * 16 + 4 * lg;
        if (p >= P) continue;
        float* dm = ybase + p;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (t >= nt_live || co0 + t * 16 + lr >= g.C_out) continue;
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = epi_value_nb(kc[t], acc[m][t][i], s, z);
          if (track) {
#pragma unroll
            for (int i = 0; i < 4; ++i) am = epi_track(am, v[i]);
          }
          *reinterpret_cast<f32x4*>(dm + t * tstep) = v;
        }
      }
      return;
    }
    if (plain) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= my_mt) break;
        const int p = (wave + 4 * m) * 16 + 4 * lg;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int co = co0 + t * 16 + lr;
          if (t >= nt_live || co >= g.C_out) continue;
          // bias only, fp32 output: one 16-byte store of the four pixels
          const int64_t di = ((int64_t)n * g.C_out + co) * npix + (int64_t)oh0 * g.OW + p;
          float* dst = reinterpret_cast<float*>(y) + di;
          const f32x4 v = acc[m][t] * s + kc[t].bias;
          if (p + 3 < P && (di & 3) == 0) {
            *reinterpret_cast<f32x4*>(dst) = v;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (p + i < P) dst[i] = v[i];
          }
        }
      }
      return;
    }
    // the epilogue, with the output dtype fixed per copy of the loop and no
    // branch on the epilogue's fields per element
    const float z = epi_relu_factor(ep);
    auto store_all = [&](auto od) {
      constexpr int OD = decltype(od)::value;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= my_mt) break;
        const int p = (wave + 4 * m) * 16 + 4 * lg;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int co = co0 + t * 16 + lr;
          if (t >= nt_live || co >= g.C_out) continue;
          const int64_t di = ((int64_t)n * g.C_out + co) * npix + (int64_t)oh0 * g.OW + p;
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = epi_value_nb(kc[t], acc[m][t][i], s, z);
            if (p + i < P) am = epi_track(am, v[i]);  // committed only with ep.amax
          }
          if (p + 3 < P && (di & 3) == 0) {
            epi_store4_t<OD>(y, di, v, inv_o);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (p + i < P) epi_store_t<OD>(y, di + i, v[i], inv_o);
          }
        }
      }
    };
    // A narrow output goes through LDS when its channel rows pack into whole
    // store units: the codes are written [channel][pixel] over the staged
    // input (every wave's MFMAs are done with it), then consecutive lanes
    // store each channel's run of P pixels in 8-byte (16-bit codes) or
    // 4-byte (8-bit) pieces -- contiguous spans, where the lanes' own stores
    // would be 32- or 16-byte pieces of 16 channel rows.
    const bool track = ep.amax != nullptr;  // uniform: the amax is asked for
    auto stage_out = [&](auto od) {
      constexpr int OD = decltype(od)::value;
      constexpr int ES = dtype_bits(OD) / 8;
      constexpr int SU = ES == 2 ? 8 : 4;
      uint8_t* ol = lds + g.x_off;
      const int rowb = P * ES;
      __syncthreads();
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= my_mt) break;
        const int p = (wave + 4 * m) * 16 + 4 * lg;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int co = co0 + t * 16 + lr;
          if (t >= nt_live || co >= g.C_out || p >= P) continue;
          // P is a multiple of 4 here, so all four pixels are in the band
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = epi_value_nb(kc[t], acc[m][t][i], s, z);
          if (track) {
#pragma unroll
            for (int i = 0; i < 4; ++i) am = epi_track(am, v[i]);
          }
          uint8_t* d = ol + (t * 16 + lr) * rowb + p * ES;
          if constexpr (ES == 2) {
            *reinterpret_cast<u32x2v*>(d) =
                u32x2v{epi_encode2_t<OD>(v[0], v[1], inv_o), epi_encode2_t<OD>(v[2], v[3], inv_o)};
          } else {
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) w |= epi_encode_t<OD>(v[i], inv_o) << (8 * i);
            *reinterpret_cast<uint32_t*>(d) = w;
          }
        }
      }
      __syncthreads();
      // wave w copies channel rows w, w + 4, ...: its lanes take consecutive
      // store units of the row, the row pointer steps by four planes
      const int live = min(CO_TILE, g.C_out - co0);
      const int per_row = rowb / SU;
      const int64_t cstep = 4 * npix * ES;
      uint8_t* dr = reinterpret_cast<uint8_t*>(y) +
                    (((int64_t)n * g.C_out + co0 + wave) * npix + (int64_t)oh0 * g.OW) * ES;
      for (int cl = wave; cl < live; cl += 4, dr += cstep) {
        const uint8_t* sr = ol + cl * rowb;
        for (int o = lane; o < per_row; o += 64) {
          if constexpr (SU == 8)
            *reinterpret_cast<u32x2v*>(dr + o * SU) = *reinterpret_cast<const u32x2v*>(sr + o * SU);
          else
            *reinterpret_cast<uint32_t*>(dr + o * SU) = *reinterpret_cast<const uint32_t*>(sr + o * SU);
        }
      }
    };
    if (g.ostage) {
      switch (ep.out_dtype) {
        case F16: stage_out(OutDtype<F16>{}); return;
        case BF16: stage_out(OutDtype<BF16>{}); return;
        case E4M3: stage_out(OutDtype<E4M3>{}); return;
        case E5M2: stage_out(OutDtype<E5M2>{}); return;
        default: break;
      }
    }
    switch (ep.out_dtype) {
      case F16: store_all(OutDtype<F16>{}); break;
      case BF16: store_all(OutDtype<BF16>{}); break;
      case E4M3: store_all(OutDtype<E4M3>{}); break;
      case E5M2: store_all(OutDtype<E5M2>{}); break;
      default: store_all(OutDtype<F32>{}); break;
    }
  };

  uint16_t* xl = reinterpret_cast<uint16_t*>(lds + g.x_off);
  stage(r0, band, 0, xl);
  __syncthreads();
  compute(band, xl);
  epi_amax_commit(ep, am);
}

// Band geometry for this convolution, or false when the band kernel does not
// apply (too many channels, rows too wide, or LDS too small).  *ipt is the
// number of 16-byte-load items per thread held in registers (0: loaded while
// staging).
template <int WT>
bool band_geometry_pass(const ConvGeom& cg, int pc8, BandGeom& b, size_t& lds, int* ipt,
                        int out_dtype) {
  if (cg.C > MAX_CB || cg.OW > 256) return false;
  b = BandGeom{};
  b.N = cg.N; b.C = cg.C; b.H = cg.H; b.W = cg.W; b.C_out = cg.C_out; b.KH = cg.KH;
  b.KW = cg.KW; b.sh = cg.sh; b.sw = cg.sw; b.ph = cg.ph; b.pw = cg.pw; b.pad_mode = cg.pad_mode;
  b.OH = cg.OH; b.OW = cg.OW;
  b.c8 = (cg.C + 7) / 8;
  b.pc8 = std::min(pc8, b.c8);
  b.passes = (b.c8 + b.pc8 - 1) / b.pc8;
  if (b.passes > 1 && b.c8 % b.pc8 != 0) return false;
  // pixel stride in LDS of 8 mod 16 bf16 (4 mod 8 banks): the 16 pixels of a
  // fragment read fall in distinct banks
  b.cstride = (b.pc8 % 2 == 0) ? b.pc8 * 8 + 8 : b.pc8 * 8;
  b.taps = cg.KH * cg.KW;
  b.groups = b.taps * b.c8;
  b.gpr = (b.groups + 3) / 4 * 4;
  // each K step (four groups) within one pass: a tap's pc8 groups in whole steps
  if (b.passes > 1 && b.pc8 % 4 != 0) return false;
  // bands of whole output rows, at most 256 pixels, balanced across the image
  const int64_t npix = (int64_t)cg.OH * cg.OW;
  const int nb = (int)((npix + 255) / 256);
  b.R = (cg.OH + nb - 1) / nb;
  while ((int64_t)b.R * cg.OW > 256) --b.R;
  if (b.R < 1) return false;
  b.bands = (cg.OH + b.R - 1) / b.R;
  b.rows_in = (b.R - 1) * cg.sh + cg.KH;
  b.wp = (cg.OW - 1) * cg.sw + cg.KW;
  b.vec = (cg.W % 4) == 0;
  b.nborder = std::min(cg.pw, b.wp) + std::max(0, b.wp - cg.pw - cg.W);
  b.vitems = b.vec ? b.rows_in * (cg.W / 4) * b.pc8 : 0;
  b.fd_c8 = fast_div((uint32_t)b.c8);
  b.fd_pc8 = fast_div((uint32_t)b.pc8);
  b.fd_w4 = fast_div((uint32_t)std::max(1, cg.W / 4));
  b.fd_ow = fast_div((uint32_t)cg.OW);
  b.fd_kw = fast_div((uint32_t)cg.KW);
  b.fd_nc = fast_div((uint32_t)std::max(1, b.vec ? b.nborder : b.wp));
  *ipt = (b.vec && b.vitems <= THREADS) ? 1 : 0;
  // weight row: gpr groups of GB bytes, stride padded so the 16 rows a
  // fragment read touches fall in distinct banks
  constexpr int GB = group_bytes<WT>();
  int stride_dw = b.gpr * GB / 4;
  while ((GB == 4 && stride_dw % 2 != 1) || (GB == 8 && stride_dw % 4 != 2) ||
         (GB == 16 && stride_dw % 8 != 4))
    stride_dw += GB / 4;
  b.wrow = stride_dw * 4;
  b.co_rows = std::min(CO_TILE, (cg.C_out + 15) / 16 * 16);
  b.x_off = (b.co_rows * b.wrow + 4 * b.gpr + 15) / 16 * 16;
  b.x_bytes = (int)(((size_t)b.rows_in * b.wp * b.cstride * 2 + 15) / 16 * 16);
  const size_t raw_bytes = ((size_t)b.co_rows * cg.C * b.taps * dtype_bits(WT) + 7) / 8;
  b.raw_ok = dtype_bits(WT) <= 8 && raw_bytes <= (size_t)b.x_bytes;
  // a narrow output through LDS: every channel row of every band (and a
  // plane) a whole number of store units, P a multiple of 4
  size_t region = (size_t)b.x_bytes;
  const int ob = dtype_bits(out_dtype) / 8, su = ob == 2 ? 8 : 4;
  b.ostage = 0;
  if (ob < 4 && ((int64_t)b.R * cg.OW) % 4 == 0 && ((int64_t)b.R * cg.OW * ob) % su == 0 &&
      (npix * ob) % su == 0) {
    const size_t out_bytes = ((size_t)b.co_rows * b.R * cg.OW * ob + 15) / 16 * 16;
    if (b.x_off + std::max(region, out_bytes) <= 80 * 1024) {
      region = std::max(region, out_bytes);
      b.ostage = 1;
    }
  }
  lds = b.x_off + region;
  return lds <= 80 * 1024;
}

// The band geometry: the whole band's channels staged at once, or, when that
// leaves room for fewer than four workgroups per CU (64 channels), in two
// passes of 32 channels over a smaller staging region.
template <int WT>
bool band_geometry(const ConvGeom& cg, BandGeom& b, size_t& lds, int* ipt, int out_dtype) {
  if (!band_geometry_pass<WT>(cg, MAX_CB / 8, b, lds, ipt, out_dtype)) return false;
  if (b.c8 == 8 && lds > BAND_LDS_FOUR) {
    BandGeom b2;
    size_t lds2 = 0;
    int ipt2 = 0;
    if (band_geometry_pass<WT>(cg, 4, b2, lds2, &ipt2, out_dtype) && lds2 <= BAND_LDS_FOUR) {
      b = b2;
      lds = lds2;
      *ipt = ipt2;
    }
  }
  return true;
}

template <int WT, int XT, int IPT, bool K9>
int launch_band(const uint8_t* x, const float* x_scale, const void* w, const float* w_scale,
                const Epilogue& ep, void* y, const BandGeom& b, size_t lds, int64_t co_blocks,
                hipStream_t stream) {
  auto kern = conv2d_band_kernel<WT, XT, IPT, K9>;
  static size_t lds_enabled = 64 * 1024;  // per instantiation: raise the limit once
  if (lds > lds_enabled) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_LIMIT);
    if (e != hipSuccess) return hip_fail(e);
    lds_enabled = LDS_LIMIT;
  }
  const int64_t blocks = (int64_t)b.N * b.bands;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks, (unsigned)co_blocks), dim3(THREADS), lds, stream,
                     x, x_scale, static_cast<const uint8_t*>(w), w_scale, ep, y, b);
  return check_launch();
}

// One output channel (C_out = 1, stride 1, zero padding, at most 16 taps,
// KW <= 8, C <= 64, W a multiple of 4: the input gradient of a one-channel
// convolution).  As the band kernel's GEMM its N would hold 1 of an MFMA
// tile's 16 output channels; instead the taps are N.  A workgroup owns a
// band of R output rows of one image and stages its R + KH - 1 input rows
// channel-last in bf16 as the band kernel does (16-byte loads of 4 columns of
// 8 channel planes, transposed in registers; padding columns and rows 0);
// then Y[q][t] = sum over c of x[c][q] w[c][t] for every staged pixel q on
// v_mfma_f32_16x16x32_bf16 (M = staged pixels, K = channels in steps of 32,
// N = taps; wave w takes pixel tiles w, w + 4, ...), and a lane makes output
// pixel p as the sum over taps, in tap order, of Y[p + (kh, kw)][t]; the
// epilogue as the other kernels.  The operands are the MFMA paths' (x and W
// rounded to bf16: products exact in fp32).
struct Co1Geom {
  int N, C, H, W, KH, KW, ph, pw, OH, OW;
  int R, bands, rows_in, wp, npin;  // band rows, bands per image, staged rows / columns / pixels
  int c8, ksteps, cstride, taps;    // 8-channel groups, K steps of 32, bf16 per staged pixel
  int vitems;                       // 16-byte-load items per band
  FastDiv fd_c8, fd_w4, fd_ow, fd_kw;
};
constexpr int CO1_MT = 8;   // pixel tiles per wave, at most (512 staged pixels)
constexpr int CO1_YP = 17;  // fp32 pitch of a staged pixel's Y row (odd: fewer bank conflicts)

//
// The body takes its band index (bid) and LDS from the caller, so a launch
// can run it beside other work.  FLIP1: w holds the weights of the
// one-input-channel convolution whose input gradient this is, (C, 1, KH, KW),
// and tap t of channel c is read at c * taps + (taps - 1 - t) -- the flipped
// weight without a flipped copy.
template <int WT, int XT, bool FLIP1>
__device__ __forceinline__ void co1_body(const uint8_t* __restrict__ x,
                                         const float* __restrict__ x_scale,
                                         const uint8_t* __restrict__ w,
                                         const float* __restrict__ w_scale, const Epilogue& ep,
                                         void* __restrict__ y, const Co1Geom& g, int bid,
                                         uint8_t* lds) {
  const int WS = g.ksteps * 32 + 8;                                 // Ws row pitch (bf16)
  uint16_t* ws = reinterpret_cast<uint16_t*>(lds);                 // [16 taps][WS]
  uint16_t* xs = ws + 16 * WS;                                     // [npin][cstride]
  float* ys = reinterpret_cast<float*>(xs);                        // [npin][CO1_YP] (after the products)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int band = bid % g.bands, n = bid / g.bands;
  const int oh0 = band * g.R;
  const int64_t HW = (int64_t)g.H * g.W;
  const int64_t xn = (int64_t)n * g.C * HW;
  const int W4 = g.W >> 2;

  // the band's 16-byte-load items into registers first: it = (staged row r,
  // column group cg, channel group q)
  constexpr int MAXI = 2;
  f32x4 v[MAXI][8];
#pragma unroll
  for (int k = 0; k < MAXI; ++k) {
    const int it = tid + 256 * k;
    const int rest = (int)fdiv((uint32_t)it, g.fd_c8), q = it - rest * g.c8;
    const int r = (int)fdiv((uint32_t)rest, g.fd_w4), cg = rest - r * W4;
    const int hi = oh0 - g.ph + r;
    const bool live = it < g.vitems && hi >= 0 && hi < g.H;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = q * 8 + j;
      v[k][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (live && c < g.C) v[k][j] = x4_f32<XT>(x, xn + c * HW + (int64_t)hi * g.W + cg * 4);
    }
  }
  // the weights (at most 64 x 16: four a lane), decoded while those loads fly
  uint16_t wv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int i = tid + 256 * k;
    int src = i;
    if constexpr (FLIP1) src = i + g.taps - 1 - 2 * (i % g.taps);
    wv[k] = i < g.C * g.taps ? weight_bf16<WT>(w, src) : (uint16_t)0;
  }
  // zero the staging (padding columns, channels past C), then the weights as
  // Ws[t][c] (bf16, taps and channels past the window 0)
  {
    uint32_t* z = reinterpret_cast<uint32_t*>(lds);
    const int words = (16 * WS + g.npin * g.cstride) / 2;
    for (int i = tid; i < words; i += 256) z[i] = 0u;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int i = tid + 256 * k;
    if (i >= g.C * g.taps) continue;
    const int c = (int)fdiv((uint32_t)i, g.fd_kw) / g.KH;  // i = c * taps + t
    const int t = i - c * g.taps;
    ws[t * WS + c] = wv[k];
  }
#pragma unroll
  for (int k = 0; k < MAXI; ++k) {
    const int it = tid + 256 * k;
    if (it >= g.vitems) continue;
    const int rest = (int)fdiv((uint32_t)it, g.fd_c8), q = it - rest * g.c8;
    const int r = (int)fdiv((uint32_t)rest, g.fd_w4), cg = rest - r * W4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = cg * 4 + g.pw + i;
      if (col >= g.wp) break;
      uint32_t pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x2 f = {v[k][2 * j][i], v[k][2 * j + 1][i]};
        pk[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
      }
      *reinterpret_cast<uint4*>(&xs[(r * g.wp + col) * g.cstride + q * 8]) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
  }
  __syncthreads();

  // Y tiles: lane holds Y[16 m + 4 (lane >> 4) + i][lane & 15]
  const int lr = lane & 15, lg = lane >> 4;
  const int mtiles = (g.npin + 15) >> 4;
  f32x4 acc[CO1_MT];
#pragma unroll
  for (int mt = 0; mt < CO1_MT; ++mt) {
    acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int m = wave + 4 * mt;
    if (m >= mtiles) continue;
    int q = m * 16 + lr;
    if (q >= g.npin) q = 0;  // a valid address; its Y row is never read
    for (int ks = 0; ks < g.ksteps; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(&xs[q * g.cstride + ks * 32 + lg * 8]);
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(&ws[lr * WS + ks * 32 + lg * 8]);
      acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[mt], 0, 0, 0);
    }
  }
  __syncthreads();  // every wave's staging reads are done: Y replaces the staging
#pragma unroll
  for (int mt = 0; mt < CO1_MT; ++mt) {
    const int m = wave + 4 * mt;
    if (m >= mtiles || lr >= g.taps) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = m * 16 + 4 * lg + i;
      if (q < g.npin) ys[q * CO1_YP + lr] = acc[mt][i];
    }
  }
  __syncthreads();

  const int P = min(g.R, g.OH - oh0) * g.OW;
  const float s = product_scale(w_scale, x_scale);
  const float inv_o = epi_inv_scale(ep);
  uint32_t am = 0;
  if (tid < P) {
    const int orow = (int)fdiv((uint32_t)tid, g.fd_ow), ocol = tid - orow * g.OW;
    float sum = 0.0f;
    for (int t = 0; t < g.taps; ++t) {
      const int kh = (int)fdiv((uint32_t)t, g.fd_kw), kw = t - kh * g.KW;
      sum += ys[((orow + kh) * g.wp + ocol + kw) * CO1_YP + t];
    }
    const float val = epi_value(ep, epi_chan(ep, 0), sum, s);
    am = epi_track(am, val);
    epi_store(ep.out_dtype, y, (int64_t)n * g.OH * g.OW + (int64_t)oh0 * g.OW + tid, val, inv_o);
  }
  epi_amax_commit(ep, am);
}

template <int WT, int XT>
__global__ __launch_bounds__(256) void conv2d_co1_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale, Epilogue ep, void* __restrict__ y, Co1Geom g) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  co1_body<WT, XT, false>(x, x_scale, w, w_scale, ep, y, g, blockIdx.x, lds);
}

// The one-output-channel geometry, or false when it does not apply.
inline bool co1_geometry(const ConvGeom& cg, Co1Geom& g, size_t& lds) {
  if (cg.C_out != 1 || cg.sh != 1 || cg.sw != 1 || cg.pad_mode != NOVAQ_PAD_ZEROS ||
      cg.W % 4 != 0 || cg.KH * cg.KW > 16 || cg.KW > 8 || cg.C > 64 || cg.C < 1 ||
      cg.OW > 256 || cg.OH < 1 || cg.OW < 1)
    return false;
  g = Co1Geom{};
  g.N = cg.N; g.C = cg.C; g.H = cg.H; g.W = cg.W; g.KH = cg.KH; g.KW = cg.KW; g.ph = cg.ph;
  g.pw = cg.pw; g.OH = cg.OH; g.OW = cg.OW;
  g.taps = cg.KH * cg.KW;
  g.c8 = (cg.C + 7) / 8;
  g.ksteps = (cg.C + 31) / 32;
  g.cstride = g.ksteps * 32 + 8;  // 8 mod 16 bf16: a fragment read's 16 pixels in distinct banks
  g.wp = cg.OW + cg.KW - 1;
  const int64_t npix = (int64_t)cg.OH * cg.OW;
  const int nb = (int)((npix + 255) / 256);
  g.R = (cg.OH + nb - 1) / nb;
  while ((int64_t)g.R * cg.OW > 256) --g.R;
  for (;; --g.R) {
    if (g.R < 1) return false;
    g.rows_in = g.R + cg.KH - 1;
    g.npin = g.rows_in * g.wp;
    g.vitems = g.rows_in * (cg.W / 4) * g.c8;
    if (g.npin <= 16 * 4 * CO1_MT && g.vitems <= 2 * 256) break;
  }
  g.bands = (cg.OH + g.R - 1) / g.R;
  g.fd_c8 = fast_div((uint32_t)g.c8);
  g.fd_w4 = fast_div((uint32_t)(cg.W / 4));
  g.fd_ow = fast_div((uint32_t)cg.OW);
  g.fd_kw = fast_div((uint32_t)cg.KW);
  const size_t wsb = (size_t)16 * (g.ksteps * 32 + 8) * 2;
  const size_t xsb = std::max((size_t)g.npin * g.cstride * 2, (size_t)g.npin * CO1_YP * 4);
  lds = wsb + xsb;
  return lds <= 64 * 1024;
}

// Any geometry whose staged input rows do not fit in LDS (very wide images):
// one lane per output element (grid-strided over the NCHW output), the window
// gathered straight from global memory with the padding mode resolved.  The
// operands are those of the MFMA paths -- x and W rounded to bf16, so every
// product is exact in fp32 -- summed in fp32 in (c, kh, kw) order, then the
// same epilogue.
template <int WT, int XT>
__global__ __launch_bounds__(256) void conv2d_direct_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale,
    const uint8_t* __restrict__ w, const float* __restrict__ w_scale, Epilogue ep,
    void* __restrict__ y, ConvGeom g) {
  const int64_t total = (int64_t)g.N * g.C_out * g.OH * g.OW;
  const float s = product_scale(w_scale, x_scale);
  const float inv_o = epi_inv_scale(ep);
  const int64_t hw = (int64_t)g.H * g.W;
  uint32_t am = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += stride) {
    const int ow = (int)(t % g.OW);
    int64_t r = t / g.OW;
    const int oh = (int)(r % g.OH);
    r /= g.OH;
    const int co = (int)(r % g.C_out);
    const int64_t n = r / g.C_out;
    float acc = 0.0f;
    for (int c = 0; c < g.C; ++c) {
      const int64_t xb = (n * g.C + c) * hw;
      const int64_t wb = ((int64_t)co * g.C + c) * g.KH * g.KW;
      for (int kh = 0; kh < g.KH; ++kh) {
        const int hi = pad_index(oh * g.sh + kh - g.ph, g.H, g.pad_mode);
        for (int kw = 0; kw < g.KW; ++kw) {
          const int wi = pad_index(ow * g.sw + kw - g.pw, g.W, g.pad_mode);
          if (hi < 0 || wi < 0) continue;  // zero padding adds +0 * w
          const float xv = u2f(enc_bf16(f2u(x_val<XT>(x, xb + (int64_t)hi * g.W + wi))) << 16);
          const float wv = u2f((uint32_t)weight_bf16<WT>(w, wb + kh * g.KW + kw) << 16);
          acc = acc + xv * wv;
        }
      }
    }
    const float v = epi_value(ep, epi_chan(ep, co), acc, s);
    am = epi_track(am, v);
    epi_store(ep.out_dtype, y, t, v, inv_o);
  }
  epi_amax_commit(ep, am);
}

// Few input channels (C <= 4, stride 1, windows up to 7 x 7): the GEMM's K is
// only C*KH*KW, so padding it to whole 8-channel MFMA groups would multiply
// the work (11x for MNIST's 1-channel 3 x 3 conv).  Instead a workgroup owns
// one image and SC_CO output channels: it stages the image's padded planes in
// LDS once (padding mode resolved, values rounded to bf16 as the MFMA paths
// round x) and the channels' weights decoded (exact bf16 values, laid out
// [c][kh][kw][8 channels] so one tap's 8 weights are two 16-byte reads), then
// each lane takes a chunk of 4 consecutive outputs of one row and makes them
// for all SC_CO channels with VALU FMAs from one input window in registers --
// every product exact in fp32, summed in (c, kh, kw) order -- and writes each
// channel's 4 values with one 16- (8-, 4-) byte store.  Consecutive lanes take
// consecutive chunks of a plane, so a wave's stores are one contiguous span.
// HBM-bound on the output.
constexpr int SC_CO = 8;          // output channels per workgroup
constexpr int SC_MAX_C = 4, SC_MAX_K = 7;
constexpr size_t SC_LDS = 64 * 1024;

struct SmallGeom {
  int N, C, H, W, C_out, KH, KW, ph, pw, pad_mode, OH, OW;
  int HP, WP;   // staged plane: HP padded rows, WP floats apart (16-byte aligned)
  int WS;       // staged columns of a row (WS <= WP; the pitch's extra floats are never read)
  int WV;       // columns of the padded image (W + 2 pw); staged columns past it are 0
  int cpr;      // 4-pixel chunks per output row
  int vec;      // OW % 4 == 0: whole chunks, vector stores
};

// F3: a 3 x 3 window with zeros padding (config [5]'s conv1), its loops and
// padding tests fixed at compile time; other windows and modes take F3 = false.
template <int WT, int XT, bool VEC, bool F3>
__global__ __launch_bounds__(256) void conv2d_smallc_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale,
    const uint8_t* __restrict__ w, const float* __restrict__ w_scale, Epilogue ep,
    void* __restrict__ y, SmallGeom g) {
  extern __shared__ __attribute__((aligned(16))) float sc_lds[];
  const int n = blockIdx.x;
  const int co0 = blockIdx.y * SC_CO;
  const int nco = min(SC_CO, g.C_out - co0);
  const int plane = g.HP * g.WP;
  const int KH = F3 ? 3 : g.KH, KW = F3 ? 3 : g.KW;
  const int taps = KH * KW;
  float* xs = sc_lds;                          // C planes of HP x WP
  float* ws = sc_lds + g.C * plane;            // C*KH*KW taps x SC_CO channels
  // stage the weights and the padded planes: every load of a round is issued
  // before the first LDS write, so the round pays one memory latency, not one
  // per element.  A lane covers rows (lane / 32) + 8 i and columns
  // (lane % 32) + 32 j of the C*HP staged rows, SC_SR x SC_SC slots a round.
  constexpr int SC_SR = 4, SC_SC = 2;
  const int64_t wb = (int64_t)co0 * g.C * taps;
  const int nwt = g.C * taps * SC_CO;
  float wv0[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = threadIdx.x + 256 * k;
    const int t = i / SC_CO, cl = i - t * SC_CO;
    wv0[k] = (i < nwt && cl < nco)
                 ? u2f((uint32_t)weight_bf16<WT>(w, wb + (int64_t)cl * g.C * taps + t) << 16)
                 : 0.0f;
  }
  // the scale and the bias of the plain store path, loaded before the
  // barrier so their latency hides behind the staging
  const bool plain = !ep.mul && !ep.add && !ep.relu && !ep.amax && ep.out_dtype == F32;
  const float s = product_scale(w_scale, x_scale);
  float bias[SC_CO];
#pragma unroll
  for (int cl = 0; cl < SC_CO; ++cl)
    bias[cl] = (plain && ep.bias && cl < nco) ? ep.bias[co0 + cl] : 0.0f;
  const uint8_t* xn = x + (int64_t)n * g.C * g.H * g.W * XL<XT>::bytes;
  const int rows = g.C * g.HP;
  auto stage_round = [&](int r0, int c0) {
    float v[SC_SR][SC_SC];
#pragma unroll
    for (int i = 0; i < SC_SR; ++i) {
      const int r = r0 + (threadIdx.x >> 5) + 8 * i;
      const int c = r / g.HP, hp = r - c * g.HP;
      int hi = -1;
      if (r < rows) {
        if constexpr (F3) hi = (unsigned)(hp - g.ph) < (unsigned)g.H ? hp - g.ph : -1;
        else hi = pad_index(hp - g.ph, g.H, g.pad_mode);
      }
      const int rb = (c * g.H + hi) * g.W;
#pragma unroll
      for (int j = 0; j < SC_SC; ++j) {
        const int col = c0 + (threadIdx.x & 31) + 32 * j;
        int wi = -1;
        if (col < g.WV) {
          if constexpr (F3) wi = (unsigned)(col - g.pw) < (unsigned)g.W ? col - g.pw : -1;
          else wi = pad_index(col - g.pw, g.W, g.pad_mode);
        }
        v[i][j] = (hi >= 0 && wi >= 0) ? x_val<XT>(xn, rb + wi) : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < SC_SR; ++i) {
      const int r = r0 + (threadIdx.x >> 5) + 8 * i;
#pragma unroll
      for (int j = 0; j < SC_SC; ++j) {
        const int col = c0 + (threadIdx.x & 31) + 32 * j;
        if (r < rows && col < g.WS) xs[r * g.WP + col] = u2f(enc_bf16(f2u(v[i][j])) << 16);
      }
    }
  };
  if (rows <= 8 * SC_SR && g.WS <= 32 * SC_SC) {
    stage_round(0, 0);  // one round covers the image: straight-line code
  } else {
    for (int r0 = 0; r0 < rows; r0 += 8 * SC_SR)
      for (int c0 = 0; c0 < g.WS; c0 += 32 * SC_SC) stage_round(r0, c0);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (threadIdx.x + 256 * k < nwt) ws[threadIdx.x + 256 * k] = wv0[k];
  for (int i = threadIdx.x + 512; i < nwt; i += 256) {  // windows past 8 x 8 x C
    const int t = i / SC_CO, cl = i - t * SC_CO;
    ws[i] = cl < nco ? u2f((uint32_t)weight_bf16<WT>(w, wb + (int64_t)cl * g.C * taps + t) << 16)
                     : 0.0f;
  }
  __syncthreads();

  const float inv_o = epi_inv_scale(ep);
  const float z = epi_relu_factor(ep);
  const int per_plane = g.OH * g.cpr;
  const int cstep = g.OH * g.OW;  // one output plane (elements)
  uint32_t am = 0;
  for (int p = threadIdx.x; p < per_plane; p += 256) {
    const int oh = p / g.cpr, ow0 = (p - oh * g.cpr) * 4;
    float acc[SC_CO][4];
#pragma unroll
    for (int cl = 0; cl < SC_CO; ++cl)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[cl][q] = 0.0f;
    for (int c = 0; c < g.C; ++c) {
      for (int kh = 0; kh < KH; ++kh) {
        const float4* row =
            reinterpret_cast<const float4*>(xs + (c * g.HP + oh + kh) * g.WP + ow0);
        float v[12];
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const float4 f = row[q];
          v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
        const float4* wk = reinterpret_cast<const float4*>(ws + (c * KH + kh) * KW * SC_CO);
#pragma unroll
        for (int kw = 0; kw < SC_MAX_K; ++kw) {
          if (kw < KW) {
            const float4 wa = wk[2 * kw], wbv = wk[2 * kw + 1];
            const float wv[SC_CO] = {wa.x, wa.y, wa.z, wa.w, wbv.x, wbv.y, wbv.z, wbv.w};
            // a bf16 x bf16 product is exact in fp32, so the fused
            // multiply-add rounds exactly as the separate add would
#pragma unroll
            for (int cl = 0; cl < SC_CO; ++cl)
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[cl][q] = __builtin_fmaf(v[q + kw], wv[cl], acc[cl][q]);
          }
        }
      }
    }
    const int64_t e0 = (((int64_t)n * g.C_out + co0) * g.OH + oh) * g.OW + ow0;
    if (plain) {
      // bias only, fp32 output: acc * s + bias, one 16-byte store per channel
      // (one lane pointer stepped by a plane)
      float* dst = reinterpret_cast<float*>(y) + e0;
#pragma unroll
      for (int cl = 0; cl < SC_CO; ++cl) {
        if (cl >= nco) break;
        float o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = acc[cl][q] * s + bias[cl];
        if constexpr (VEC) {
          *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (ow0 + q < g.OW) dst[q] = o[q];
        }
        dst += cstep;
      }
      continue;
    }
    // the epilogue, one copy of the store loop per output dtype, no branch on
    // the epilogue's fields per element
    auto store_all = [&](auto od) {
      constexpr int OD = decltype(od)::value;
#pragma unroll
      for (int cl = 0; cl < SC_CO; ++cl) {
        if (cl >= nco) break;
        const EpiChan k = epi_chan(ep, co0 + cl);
        float o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          o[q] = epi_value_nb(k, acc[cl][q], s, z);
          if (ow0 + q < g.OW) am = epi_track(am, o[q]);
        }
        const int64_t e = e0 + (int64_t)cl * cstep;
        if constexpr (VEC) {
          epi_store4_t<OD>(y, e, o, inv_o);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (ow0 + q < g.OW) epi_store_t<OD>(y, e + q, o[q], inv_o);
        }
      }
    };
    switch (ep.out_dtype) {
      case F16: store_all(OutDtype<F16>{}); break;
      case BF16: store_all(OutDtype<BF16>{}); break;
      case E4M3: store_all(OutDtype<E4M3>{}); break;
      case E5M2: store_all(OutDtype<E5M2>{}); break;
      default: store_all(OutDtype<F32>{}); break;
    }
  }
  epi_amax_commit(ep, am);
}

// The small-channel path when the shape fits it; returns false otherwise.
template <int WT, int XT>
bool launch_smallc(const uint8_t* x, const float* x_scale, const void* w, const float* w_scale,
                   const Epilogue& ep, void* y, const ConvGeom& cg, hipStream_t stream,
                   int* rc) {
  if (cg.C > SC_MAX_C || cg.sh != 1 || cg.sw != 1 || cg.KH > SC_MAX_K || cg.KW > SC_MAX_K)
    return false;
  SmallGeom g{};
  g.N = cg.N; g.C = cg.C; g.H = cg.H; g.W = cg.W; g.C_out = cg.C_out; g.KH = cg.KH;
  g.KW = cg.KW; g.ph = cg.ph; g.pw = cg.pw; g.pad_mode = cg.pad_mode; g.OH = cg.OH;
  g.OW = cg.OW;
  g.HP = cg.OH + cg.KH - 1;
  g.cpr = (cg.OW + 3) / 4;
  g.WV = cg.OW + cg.KW - 1;
  g.WS = 4 * g.cpr + 8;  // a chunk reads 12 floats (3 x 16 bytes) from its start
  g.vec = cg.OW % 4 == 0 && (reinterpret_cast<uintptr_t>(y) % 16) == 0;
  // row pitch 4 * cpr + 64 floats when it fits: the chunks' 16-byte reads then
  // fall on the banks of a contiguous run (pitch = one row of chunks mod 64
  // banks), with no conflicts where a group of lanes crosses a row
  const size_t wts = (size_t)SC_CO * g.C * g.KH * g.KW;
  g.WP = 4 * g.cpr + 64;
  if (((size_t)g.C * g.HP * g.WP + wts) * sizeof(float) > SC_LDS) g.WP = g.WS;
  const size_t lds = ((size_t)g.C * g.HP * g.WP + wts) * sizeof(float);
  // (within the default 64 KB of dynamic LDS: no attribute to raise); the
  // image's input offsets and one output plane fit 32-bit indices
  if (lds > SC_LDS || (int64_t)g.OH * g.cpr * SC_CO > 0x7FFFFFFF ||
      (int64_t)g.C * g.H * g.W > 0x7FFFFFFF || (int64_t)g.OH * g.OW > 0x7FFFFFFF)
    return false;
  const int64_t co_groups = (cg.C_out + SC_CO - 1) / SC_CO;
  if (co_groups > 65535) return false;
  const dim3 grid((unsigned)cg.N, (unsigned)co_groups);
  const auto* wq = static_cast<const uint8_t*>(w);
  const bool f3 = cg.KH == 3 && cg.KW == 3 && cg.pad_mode == NOVAQ_PAD_ZEROS;
  if (g.vec && f3)
    hipLaunchKernelGGL((conv2d_smallc_kernel<WT, XT, true, true>), grid, dim3(256), lds, stream, x,
                       x_scale, wq, w_scale, ep, y, g);
  else if (g.vec)
    hipLaunchKernelGGL((conv2d_smallc_kernel<WT, XT, true, false>), grid, dim3(256), lds, stream, x,
                       x_scale, wq, w_scale, ep, y, g);
  else
    hipLaunchKernelGGL((conv2d_smallc_kernel<WT, XT, false, false>), grid, dim3(256), lds, stream, x,
                       x_scale, wq, w_scale, ep, y, g);
  *rc = check_launch();
  return true;
}

template <int WT, int XT>
int launch(const uint8_t* x, const float* x_scale, const void* w, const float* w_scale,
           const Epilogue& ep, void* y, ConvGeom g, hipStream_t stream) {
  {
    int rc = NOVAQ_OK;
    if (launch_smallc<WT, XT>(x, x_scale, w, w_scale, ep, y, g, stream, &rc)) return rc;
  }
  {
    Co1Geom c1;
    size_t lds = 0;
    if (co1_geometry(g, c1, lds)) {
      if ((int64_t)g.N * c1.bands > 0x7FFFFFFF) return NOVAQ_EINVAL;
      hipLaunchKernelGGL((conv2d_co1_kernel<WT, XT>), dim3((unsigned)(g.N * c1.bands)), dim3(256),
                         lds, stream, x, x_scale, static_cast<const uint8_t*>(w), w_scale, ep, y, c1);
      return check_launch();
    }
  }
  {
    BandGeom b;
    size_t lds = 0;
    int ipt = 0;
    if (band_geometry<WT>(g, b, lds, &ipt, ep.out_dtype)) {
      const int64_t co_blocks = (g.C_out + CO_TILE - 1) / CO_TILE;
      if constexpr (group_bytes<WT>() < 16) {
        if (b.taps == 9 && g.C % 8 == 0 && b.raw_ok) {
          if (ipt == 1) return launch_band<WT, XT, 1, true>(x, x_scale, w, w_scale, ep, y, b, lds, co_blocks, stream);
          return launch_band<WT, XT, 0, true>(x, x_scale, w, w_scale, ep, y, b, lds, co_blocks, stream);
        }
      }
      if (ipt == 1) return launch_band<WT, XT, 1, false>(x, x_scale, w, w_scale, ep, y, b, lds, co_blocks, stream);
      return launch_band<WT, XT, 0, false>(x, x_scale, w, w_scale, ep, y, b, lds, co_blocks, stream);
    }
  }
  // staged rows for a run of PIX_TILE pixels: it spans at most
  // ceil((PIX_TILE - 1) / OW) + 1 output rows
  const int out_rows = (PIX_TILE - 1) / g.OW + 2;
  g.rows = (out_rows - 1) * g.sh + g.KH;
  g.wp = (g.OW - 1) * g.sw + g.KW;
  // weight row: 2*ksteps groups of GB bytes, padded so the 32 rows one
  // fragment read touches fall in distinct LDS banks (row stride in dwords
  // odd for 4-byte reads, 2 mod 4 for 8-byte reads, 4 mod 8 for 16-byte reads)
  constexpr int GB = group_bytes<WT>();
  int stride_dw = 2 * g.ksteps * GB / 4;
  while ((GB == 4 && stride_dw % 2 != 1) || (GB == 8 && stride_dw % 4 != 2) ||
         (GB == 16 && stride_dw % 8 != 4))
    stride_dw += GB / 4;
  g.wrow = stride_dw * 4;
  const size_t xl_bytes = (size_t)g.rows * g.wp * g.cstride * 2;
  // weights, staged input, then the K-group offset table (2*ksteps ints)
  const size_t lds = (size_t)CO_TILE * g.wrow + xl_bytes + (size_t)8 * g.ksteps;
  const size_t raw_bytes = ((size_t)CO_TILE * g.C * g.KH * g.KW * dtype_bits(WT) + 7) / 8;
  g.raw_in_lds = g.C <= g.CB && raw_bytes <= xl_bytes;
  if (lds > LDS_LIMIT) {  // rows too wide for one LDS tile: the direct gather
    const int64_t total = (int64_t)g.N * g.C_out * g.OH * g.OW;
    int64_t blocks = (total + 255) / 256;
    const int64_t cap = (int64_t)device_cu_count() * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL((conv2d_direct_kernel<WT, XT>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, x, x_scale, static_cast<const uint8_t*>(w), w_scale, ep, y, g);
    return check_launch();
  }
  auto kern = conv2d_kernel<WT, XT>;
  static size_t lds_enabled = 64 * 1024;  // per instantiation: raise the limit once
  if (lds > lds_enabled) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_LIMIT);
    if (e != hipSuccess) return hip_fail(e);
    lds_enabled = LDS_LIMIT;
  }
  const int64_t co_blocks = (g.C_out + CO_TILE - 1) / CO_TILE;
  int64_t grid = (int64_t)device_cu_count() * CONV_OCC;
  if (grid > g.tiles) grid = g.tiles;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid, (unsigned)co_blocks), dim3(THREADS), lds, stream, x,
                     x_scale, static_cast<const uint8_t*>(w), w_scale, ep, y, g);
  return check_launch();
}

}  // namespace

// The convolution for x stored as XT (one translation unit per XT instantiates it).
template <int XT>
int conv2d_launch_xt(const uint8_t* x, const float* x_scale, int64_t N, int64_t C, int64_t H,
                     int64_t W, const void* w_q, int w_dtype, const float* w_scale, int64_t C_out,
                     int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode,
                     const Epilogue& ep, void* y, hipStream_t stream) {
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
  g.tiles_per_image = (int)((OH * OW + PIX_TILE - 1) / PIX_TILE);
  g.tiles = (int64_t)N * g.tiles_per_image;
  switch (w_dtype) {
    case E4M3: return launch<E4M3, XT>(x, x_scale, w_q, w_scale, ep, y, g, stream);
    case E5M2: return launch<E5M2, XT>(x, x_scale, w_q, w_scale, ep, y, g, stream);
    case E2M1: return launch<E2M1, XT>(x, x_scale, w_q, w_scale, ep, y, g, stream);
    case BF16: return launch<BF16, XT>(x, x_scale, w_q, w_scale, ep, y, g, stream);
    case F16: return launch<F16, XT>(x, x_scale, w_q, w_scale, ep, y, g, stream);
    case F32: return launch<F32, XT>(x, x_scale, w_q, w_scale, ep, y, g, stream);
    default: return NOVAQ_EDTYPE;
  }
}

}  // namespace novaq
