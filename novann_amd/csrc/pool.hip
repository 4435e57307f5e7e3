// MaxPool2d and GlobalAvgPool2d forward for gfx950 (restate
// novann.functional.max_pool2d, functional.py:450-532, and avg_pool2d,
// :548-559), on x stored as F32 or as a fused epilogue stores activations
// (BF16, F16, E4M3, E5M2).
//
// max_pool2d: the input padded with numpy.pad's rules (zeros pads +0), then
// the max of each KH x KW window.  The reference reduces a strided window
// view with numpy's maximum; its result is the window's largest value, a
// later element in row-major window order replacing an equal one (so the sign
// of a zero maximum is that of the last zero), and NaN once a NaN is met.
// The kernel walks the window in the same order with the same rule; the
// result is one of the input codes, so every x dtype is exact (FP8 codes
// keep their per-tensor scale).  One lane per output element, consecutive
// lanes on consecutive output columns.  HBM-bound: read x ~once (the windows
// of a row overlap in L1/L2), write y once.
//
// global_avg_pool2d: np.mean over H and W of each (n, c) plane, which numpy
// evaluates in float32 as 0 plus, block by block of its default ufunc buffer
// size (8192 elements), the pairwise_sum of the block, followed by one float32
// division by H*W.  pairwise_sum is numpy's published algorithm: fewer than
// 8 elements summed in order from 0; up to 128 with 8 interleaved partial
// sums combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) plus the remainder in
// order; longer runs split at n/2 rounded down to a multiple of 8 and the two
// halves added.  The kernel evaluates exactly that, so the result equals the
// reference's bit for bit; narrow x is decoded and multiplied by its scale
// first (the dequantized array the reference would average).  Lanes per leaf
// of the tree, shuffles across leaves: several planes per wave when a plane's
// tree fits a wave's lanes (the tree kernel), else one wave per plane walking
// numpy's blocks (the plane kernel).
//
// Backward passes (MaxPool2d.backward, layers/pooling/maxpool/maxpool2d.py:
// 79-129; GlobalAvgPool2d.backward, layers/pooling/gap/global_avg_pool2d.py:
// 35-57): the max pool's input gradient, each window's grad split over the
// elements equal to its maximum, the windows' shares added per element in
// window order; the average pool's, grad times float32(1 / (H*W)) over the
// plane.  Both write fp32, HBM-bound.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "novaq_convert.h"
#include "novaq_gap_plan.h"
#include "novaq_internal.h"
#include "novaq_xload.h"

namespace novaq {
namespace {

#ifndef POOL_WG_PER_CU
#define POOL_WG_PER_CU 64
#endif

struct PoolGeom {
  int64_t N, C;
  int H, W, KH, KW, sh, sw, ph, pw, pad_mode, OH, OW;
};

template <int XT>
__device__ __forceinline__ void store_code(uint8_t* __restrict__ y, int64_t i, uint32_t c) {
  if constexpr (XL<XT>::bits == 32) reinterpret_cast<uint32_t*>(y)[i] = c;
  else if constexpr (XL<XT>::bits == 16) reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)c;
  else y[i] = (uint8_t)c;
}

// Lane t of the grid makes output element t (planes of OH x OW outputs back
// to back), so workgroups are full whatever the plane size.
template <int XT>
__global__ __launch_bounds__(256) void max_pool2d_kernel(const uint8_t* __restrict__ x,
                                                        uint8_t* __restrict__ y, PoolGeom g) {
  const int npix = g.OH * g.OW;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= g.N * g.C * npix) return;
  const int64_t plane = t / npix;  // n * C + c
  const int pix = (int)(t - plane * npix);
  const int oh = pix / g.OW, ow = pix - oh * g.OW;
  const int64_t base = plane * g.H * g.W;
  uint32_t best = 0;
  float bv = 0.0f;
  bool first = true;
  for (int kh = 0; kh < g.KH; ++kh) {
    const int hi = pad_index(oh * g.sh + kh - g.ph, g.H, g.pad_mode);
    for (int kw = 0; kw < g.KW; ++kw) {
      const int wi = pad_index(ow * g.sw + kw - g.pw, g.W, g.pad_mode);
      uint32_t c = 0;  // the zero padding's +0
      if (hi >= 0 && wi >= 0) c = x_code<XT>(x, base + (int64_t)hi * g.W + wi);
      const float v = u2f(decode<XT>(c));
      if (first) {
        best = c;
        bv = v;
        first = false;
      } else if (!isnan(bv) && (v >= bv || isnan(v))) {
        best = c;
        bv = v;
      }
    }
  }
  store_code<XT>(y, t, best);
}

// The window rule: v replaces the running maximum bv when it is larger or
// equal, or NaN, unless bv is NaN already.
__device__ __forceinline__ void take_max(uint32_t c, float v, uint32_t& best, float& bv) {
  if (!isnan(bv) && (v >= bv || isnan(v))) {
    best = c;
    bv = v;
  }
}


// 2-wide windows with stride 2 along W and no W padding (MaxPool2d(2, 2) and
// its (k, 2) / (k, 2) relatives): an item makes the two adjacent outputs
// 2u, 2u+1 of one output row from 4 consecutive inputs per window row, read
// with one 16 / 8 / 4-byte load when W is a multiple of 4.  Items t (planes
// of OH x ceil(OW/2) back to back, t < 2^31) go two per lane per step, grid-
// strided, all their window rows' loads issued before the first compare
// (KH2: the 2-row window, unrolled).
template <int XT, bool KH2>
__global__ __launch_bounds__(256) void max_pool2d_w2_kernel(const uint8_t* __restrict__ x,
                                                           uint8_t* __restrict__ y, PoolGeom g,
                                                           FastDiv dper, FastDiv dou,
                                                           uint32_t total) {
  const int OU = (g.OW + 1) / 2;  // output pairs per row
  const uint32_t per = (uint32_t)(g.OH * OU);
  const bool vec = (g.W & 3) == 0;
  const bool pair_store = (g.OW & 1) == 0;
  constexpr int B = XL<XT>::bits;
  constexpr int KR = KH2 ? 2 : 1;  // window rows loaded at once
  const uint32_t stride = gridDim.x * 256u;
  struct Item {
    bool live, two;
    int oh;
    int64_t base, out;
    int u;
  };
  auto locate = [&](uint32_t t) {
    Item it;
    it.live = t < total;
    const uint32_t plane = fdiv(t, dper), item = t - plane * per;
    it.oh = (int)fdiv(item, dou);
    it.u = (int)item - it.oh * OU;
    it.base = (int64_t)plane * g.H * g.W;
    it.out = (int64_t)plane * g.OH * g.OW + (int64_t)it.oh * g.OW + 2 * it.u;
    it.two = 2 * it.u + 1 < g.OW;
    return it;
  };
  auto load = [&](const Item& it, int kh, uint32_t* c) {
    c[0] = c[1] = c[2] = c[3] = 0u;  // the zero padding's +0
    if (!it.live) return;
    const int hi = pad_index(it.oh * g.sh + kh - g.ph, g.H, g.pad_mode);
    if (hi < 0) return;
    const int64_t e = it.base + (int64_t)hi * g.W + 4 * it.u;
    if (vec) {
      const xl_u32x4 r = x4_raw<XT>(x, e);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        c[q] = B == 32 ? r[q] : (r[(q * B) / 32] >> ((q * B) % 32)) & ((1u << (B & 31)) - 1u);
    } else {
      c[0] = x_code<XT>(x, e);
      c[1] = x_code<XT>(x, e + 1);
      if (it.two) {
        c[2] = x_code<XT>(x, e + 2);
        c[3] = x_code<XT>(x, e + 3);
      }
    }
  };
  auto fold = [&](const uint32_t* c, bool first, uint32_t* best, float* bv) {
#pragma unroll
    for (int o = 0; o < 2; ++o)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t code = c[2 * o + q];
        const float v = u2f(decode<XT>(code));
        if (first && q == 0) {
          best[o] = code;
          bv[o] = v;
        } else {
          take_max(code, v, best[o], bv[o]);
        }
      }
  };
  auto store = [&](const Item& it, const uint32_t* best) {
    if (!it.live) return;
    if (it.two && pair_store) {
      if constexpr (B == 32) {
        *reinterpret_cast<uint2*>(reinterpret_cast<uint32_t*>(y) + it.out) =
            make_uint2(best[0], best[1]);
      } else if constexpr (B == 16) {
        reinterpret_cast<uint32_t*>(y)[it.out >> 1] = best[0] | (best[1] << 16);
      } else {
        reinterpret_cast<uint16_t*>(y)[it.out >> 1] = (uint16_t)(best[0] | (best[1] << 8));
      }
    } else {
      store_code<XT>(y, it.out, best[0]);
      if (it.two) store_code<XT>(y, it.out + 1, best[1]);
    }
  };
  constexpr int IT = 2;  // items per lane per step
  for (uint32_t t = blockIdx.x * 256u + threadIdx.x; t < total; t += IT * stride) {
    Item it[IT];
    uint32_t best[IT][2];
    float bv[IT][2];
#pragma unroll
    for (int k = 0; k < IT; ++k) {
      // t + k * stride < 2^31 + IT * 2^31 would wrap; items past the end are
      // dead (locate's division needs n < 2^31)
      const uint64_t tk = (uint64_t)t + (uint64_t)k * stride;
      it[k] = locate(tk < total ? (uint32_t)tk : 0u);
      it[k].live = tk < total;
      best[k][0] = best[k][1] = 0u;
      bv[k][0] = bv[k][1] = 0.0f;
    }
    for (int kh0 = 0; kh0 < g.KH; kh0 += KR) {
      uint32_t c[IT][KR][4];
#pragma unroll
      for (int r = 0; r < KR; ++r)
#pragma unroll
        for (int k = 0; k < IT; ++k) load(it[k], kh0 + r, c[k][r]);
#pragma unroll
      for (int r = 0; r < KR; ++r)
#pragma unroll
        for (int k = 0; k < IT; ++k) fold(c[k][r], kh0 + r == 0, best[k], bv[k]);
    }
#pragma unroll
    for (int k = 0; k < IT; ++k) store(it[k], best[k]);
  }
}

// MaxPool2d(2, 2) without padding (2 x 2 windows, stride 2, W a multiple of
// 4, OW even): one lane per output pair of one row, flat over the planes'
// OH x OW/2 pairs -- two 4-element loads (one per window row), the window
// rule, one paired store.  The same comparisons as max_pool2d_w2_kernel, so
// the same results; without its grid-stride loop, padding lookups and
// per-row window loop (a stripped copy of that kernel ran 11.1 -> 7.5 us on
// a (256, 64, 28, 28) bf16 map).
template <int XT>
__global__ __launch_bounds__(256) void max_pool2d_22_kernel(const uint8_t* __restrict__ x,
                                                           uint8_t* __restrict__ y, int H, int W,
                                                           int OH, int OW, FastDiv dper,
                                                           FastDiv dou, uint32_t total) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= total) return;
  constexpr int B = XL<XT>::bits;
  const int OU = OW >> 1;
  const uint32_t per = (uint32_t)(OH * OU);
  const uint32_t plane = fdiv(t, dper), item = t - plane * per;
  const int oh = (int)fdiv(item, dou);
  const int u = (int)item - oh * OU;
  const int64_t e = (int64_t)plane * H * W + (int64_t)(2 * oh) * W + 4 * u;
  const xl_u32x4 r0 = x4_raw<XT>(x, e), r1 = x4_raw<XT>(x, e + W);
  auto code = [](const xl_u32x4& r, int q) {
    return B == 32 ? r[q] : (r[(q * B) / 32] >> ((q * B) % 32)) & ((1u << (B & 31)) - 1u);
  };
  uint32_t best[2];
#pragma unroll
  for (int o = 0; o < 2; ++o) {
    // row-major window order: (0, 0), (0, 1), (1, 0), (1, 1)
    best[o] = code(r0, 2 * o);
    float bv = u2f(decode<XT>(best[o]));
    take_max(code(r0, 2 * o + 1), u2f(decode<XT>(code(r0, 2 * o + 1))), best[o], bv);
    take_max(code(r1, 2 * o), u2f(decode<XT>(code(r1, 2 * o))), best[o], bv);
    take_max(code(r1, 2 * o + 1), u2f(decode<XT>(code(r1, 2 * o + 1))), best[o], bv);
  }
  const int64_t out = (int64_t)plane * OH * OW + (int64_t)oh * OW + 2 * u;
  if constexpr (B == 32) {
    *reinterpret_cast<uint2*>(reinterpret_cast<uint32_t*>(y) + out) = make_uint2(best[0], best[1]);
  } else if constexpr (B == 16) {
    reinterpret_cast<uint32_t*>(y)[out >> 1] = best[0] | (best[1] << 16);
  } else {
    reinterpret_cast<uint16_t*>(y)[out >> 1] = (uint16_t)(best[0] | (best[1] << 8));
  }
}

constexpr int64_t NP_BUFSIZE = 8192;  // numpy's default ufunc buffer (np.getbufsize())

// --- global average, every load issued at once (planes of at most 8192) ----
//
// The same leaves and the same tree as the wave kernel, with no staging and
// no plan table.  The tree is made complete: D is its deepest level, each of
// the 2^D virtual leaves either is a real leaf (a leaf at depth d < D owns the
// first of the 2^(D-d) virtual leaves below it) or holds -0.0f, the exact
// additive identity, so adding neighbours level by level (D levels of
// shuffles) associates exactly as numpy's recursion.  A lane finds its leaf
// by walking the D levels from the root with the bits of its virtual leaf
// index.  Each virtual leaf has 8/Q lanes; lane h of a leaf loads elements
// h*Q .. h*Q+Q-1 of every whole group of 8 with one Q-element vector load
// (Q chosen by the host so that every such load is aligned) and keeps Q of
// the 8 interleaved partial sums; the partials are added pairwise in the lane
// and shuffles finish ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)); the leaf's first
// lane adds the remainder in order.  W = (8/Q) * 2^D <= 64 lanes per plane,
// 64/W planes per wave.  The loads are buffer loads through a descriptor
// over the workgroup's planes: every lane issues the same NG loads (NG = 8
// or 16, at least the longest leaf's group count), with no branch, so all of
// them are in flight before the first add and each add waits only for its
// own load.  Load k of a lane whose leaf has ng <= k groups (and every load of
// a lane that owns no leaf) gets a vector offset past the descriptor's range
// and returns +0 without a memory access; the lane adds it like the others:
// adding +0 changes at most the sign of a zero partial sum, and zeros of
// either sign leave every non-zero sum as it is and give the same final
// 0 + sum.  This kernel is issue-bound as much as HBM-bound, so each element
// costs one add (plus its decode, and SCALED's multiply).
template <int XT, int Q>
__device__ __forceinline__ xl_u32x4 bload_q(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                            uint32_t soff = 0) {
  constexpr int BYTES = Q * XL<XT>::bits / 8;
  xl_u32x4 r = {0u, 0u, 0u, 0u};
  if constexpr (BYTES == 16) {
    r = __builtin_amdgcn_raw_buffer_load_b128(rs, off, soff, 0);
  } else if constexpr (BYTES == 8) {
    const xl_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, soff, 0);
    r[0] = v[0];
    r[1] = v[1];
  } else if constexpr (BYTES == 4) {
    r[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, soff, 0);
  } else if constexpr (BYTES == 2) {
    r[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, soff, 0);
  } else {
    r[0] = __builtin_amdgcn_raw_buffer_load_b8(rs, off, soff, 0);
  }
  return r;
}

constexpr uint32_t GAP_OOB = 0x40000000u;  // a vector offset past any descriptor's range (<= 8 MiB)

template <int XT, int Q, bool SCALED, int NG>
__global__ __launch_bounds__(256) void global_avg_pool2d_tree_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, float* __restrict__ y,
    int64_t planes, int hw, int D, int wshift) {
  constexpr int B = XL<XT>::bits, EB = B / 8;
  constexpr int LPL = 8 / Q;  // lanes per leaf
  constexpr int LSH = LPL == 8 ? 3 : LPL == 4 ? 2 : LPL == 2 ? 1 : 0;
  const int ppb = 256 >> wshift;  // planes per workgroup
  const int64_t p0 = (int64_t)blockIdx.x * ppb;
  const int lp = threadIdx.x >> wshift;
  const int l = threadIdx.x & ((1 << wshift) - 1);
  const int vi = l >> LSH, h = l & (LPL - 1);
  const int W = 1 << wshift;
  const int64_t left = planes - p0;
  const int nplanes = left < ppb ? (int)left : ppb;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(x + p0 * hw * EB), (short)0, nplanes * hw * EB, 0x00020000);
  const float s = SCALED ? *x_scale : 1.0f;
  int off, len;
  const bool owner = gap_detail::virtual_leaf(hw, D, vi, off, len) && lp < nplanes;
  const int ng = owner ? len >> 3 : 0;
  const int nr = owner && h == 0 ? len & 7 : 0;
  const uint32_t lb = (uint32_t)(lp * hw + off) * EB;  // the leaf's first byte
  const uint32_t lq = lb + (uint32_t)(h * Q * EB);
  // every address first, then the NG loads back to back: interleaving the
  // address arithmetic with the loads measured 20% slower
  uint32_t ad[NG];
#pragma unroll
  for (int k = 0; k < NG; ++k) ad[k] = (k < ng ? lq : GAP_OOB) + 8 * k * EB;
  __builtin_amdgcn_sched_barrier(0);
  xl_u32x4 v[NG];
#pragma unroll
  for (int k = 0; k < NG; ++k) v[k] = bload_q<XT, Q>(rs, ad[k]);
  __builtin_amdgcn_sched_barrier(0);
  float tail[7] = {};
  if (hw & 7) {  // only then has a leaf a remainder
#pragma unroll
    for (int q = 0; q < 7; ++q) {
      const float f =
          u2f(decode<XT>(bload_q<XT, 1>(rs, q < nr ? lb + (uint32_t)((8 * ng + q) * EB) : GAP_OOB)[0]));
      tail[q] = SCALED ? f * s : f;
    }
  }
  auto val = [&](const xl_u32x4& r, int q) {
    const uint32_t c =
        B == 32 ? r[q] : (r[(q * B) / 32] >> ((q * B) % 32)) & ((1u << (B & 31)) - 1u);
    const float f = u2f(decode<XT>(c));
    return SCALED ? f * s : f;
  };
  float r[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) r[q] = val(v[0], q);
#pragma unroll
  for (int k = 1; k < NG; ++k)
#pragma unroll
    for (int q = 0; q < Q; ++q) r[q] += val(v[k], q);
  // partials h*Q .. h*Q+Q-1 pairwise, neighbours first, then the other lanes'
#pragma unroll
  for (int w = 1; w < Q; w <<= 1)
#pragma unroll
    for (int q = 0; q < Q; q += 2 * w) r[q] = r[q] + r[q + w];
  float c = r[0];
#pragma unroll
  for (int d = 1; d < LPL; d <<= 1) c = c + __shfl_down(c, d, W);
  float res = ng > 0 ? c : 0.0f;  // below 8 elements: 0 plus the elements in order
#pragma unroll
  for (int q = 0; q < 7; ++q)
    if (q < nr) res += tail[q];
  if (!owner) res = -0.0f;
  for (int lvl = 0; lvl < D; ++lvl) res = res + __shfl_down(res, LPL << lvl, W);
  if (l == 0 && lp < nplanes) y[p0 + lp] = (0.0f + res) / (float)hw;
}

// --- global average, one wave per plane (any plane size) -------------------
//
// Planes whose tree is too deep for one wave's lanes, or over 8192 elements:
// the wave walks numpy's 8192-element blocks in order (total = 0, then total
// + each block's pairwise sum), and runs each block's complete tree (depth D)
// in passes of P = 64/LPL consecutive virtual leaves -- each pass a complete
// subtree, reduced by the same lanes, loads and shuffles as the tree kernel.
// Pass k's sum is parked in lane k, and the passes (a power of two) are then
// added neighbours first by shuffles, the upper levels of the same tree.
// Each block has its own buffer descriptor (at most 32 KiB), so no offset
// outgrows 32 bits whatever the plane size.
template <int XT, int Q, bool SCALED, int NG>
__global__ __launch_bounds__(256) void global_avg_pool2d_plane_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, float* __restrict__ y,
    int64_t planes, int64_t hw, int D_full, int D_last) {
  constexpr int B = XL<XT>::bits, EB = B / 8;
  constexpr int LPL = 8 / Q;  // lanes per leaf
  constexpr int LSH = LPL == 8 ? 3 : LPL == 4 ? 2 : LPL == 2 ? 1 : 0;
  constexpr int PSH = 6 - LSH;  // log2 of the virtual leaves per pass (64 / LPL)
  const int lane = threadIdx.x & 63;
  const int64_t plane = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (plane >= planes) return;  // the whole wave
  const int h = lane & (LPL - 1);
  const float s = SCALED ? *x_scale : 1.0f;
  auto val = [&](const xl_u32x4& r, int q) {
    const uint32_t c =
        B == 32 ? r[q] : (r[(q * B) / 32] >> ((q * B) % 32)) & ((1u << (B & 31)) - 1u);
    const float f = u2f(decode<XT>(c));
    return SCALED ? f * s : f;
  };
  float total = 0.0f;
  for (int64_t b0 = 0; b0 < hw; b0 += NP_BUFSIZE) {
    const int nb = (int)(hw - b0 < NP_BUFSIZE ? hw - b0 : NP_BUFSIZE);
    const int D = b0 + NP_BUFSIZE < hw ? D_full : D_last;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(x + (plane * hw + b0) * EB), (short)0, nb * EB, 0x00020000);
    const int passes = D > PSH ? 1 << (D - PSH) : 1;
    float coll = -0.0f;  // lane k: pass k's sum
    for (int ps = 0; ps < passes; ++ps) {
      const int vi = (ps << PSH) + (lane >> LSH);
      int off, len;
      const bool owner = gap_detail::virtual_leaf(nb, D, vi, off, len);
      const int ng = owner ? len >> 3 : 0;
      const int nr = owner && h == 0 ? len & 7 : 0;
      const uint32_t lb = (uint32_t)off * EB;
      const uint32_t lq = lb + (uint32_t)(h * Q * EB);
      uint32_t ad[NG];
#pragma unroll
      for (int k = 0; k < NG; ++k) ad[k] = (k < ng ? lq : GAP_OOB) + 8 * k * EB;
      __builtin_amdgcn_sched_barrier(0);
      xl_u32x4 v[NG];
#pragma unroll
      for (int k = 0; k < NG; ++k) v[k] = bload_q<XT, Q>(rs, ad[k]);
      __builtin_amdgcn_sched_barrier(0);
      float tail[7] = {};
      if (nb & 7) {
#pragma unroll
        for (int q = 0; q < 7; ++q) {
          const float f = u2f(
              decode<XT>(bload_q<XT, 1>(rs, q < nr ? lb + (uint32_t)((8 * ng + q) * EB) : GAP_OOB)[0]));
          tail[q] = SCALED ? f * s : f;
        }
      }
      float r[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) r[q] = val(v[0], q);
#pragma unroll
      for (int k = 1; k < NG; ++k)
#pragma unroll
        for (int q = 0; q < Q; ++q) r[q] += val(v[k], q);
#pragma unroll
      for (int w = 1; w < Q; w <<= 1)
#pragma unroll
        for (int q = 0; q < Q; q += 2 * w) r[q] = r[q] + r[q + w];
      float c = r[0];
#pragma unroll
      for (int d = 1; d < LPL; d <<= 1) c = c + __shfl_down(c, d, 64);
      float res = ng > 0 ? c : 0.0f;
#pragma unroll
      for (int q = 0; q < 7; ++q)
        if (q < nr) res += tail[q];
      if (!owner) res = -0.0f;
#pragma unroll
      for (int l = 0; l < PSH; ++l) res = res + __shfl_down(res, LPL << l, 64);
      const float pass_sum = __shfl(res, 0, 64);
      if (lane == ps) coll = pass_sum;
    }
    for (int w = 1; w < passes; w <<= 1) coll = coll + __shfl_down(coll, w, 64);
    total = total + __shfl(coll, 0, 64);
  }
  if (lane == 0) y[plane] = total / (float)hw;
}

template <int XT>
int launch_max(const void* x, void* y, const PoolGeom& g, hipStream_t stream) {
  const int64_t npix = (int64_t)g.OH * g.OW;
  if (npix > 0x7FFFFFFF) return NOVAQ_EINVAL;
  // the paired kernel reads 4 elements at once when W % 4 == 0 and stores
  // output pairs when OW is even: it needs x on a 4-element and y on a
  // 2-element boundary (views into a larger tensor need not be)
  constexpr uintptr_t EB = XL<XT>::bits / 8;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % (4 * EB)) == 0 &&
                       (reinterpret_cast<uintptr_t>(y) % (2 * EB)) == 0;
  if (g.KH == 2 && g.KW == 2 && g.sh == 2 && g.sw == 2 && g.ph == 0 && g.pw == 0 && aligned &&
      (g.W & 3) == 0 && (g.OW & 1) == 0) {
    const int64_t per = (int64_t)g.OH * (g.OW / 2);
    const int64_t items = g.N * g.C * per;
    if (items < ((int64_t)1 << 31) && per > 0) {
      const FastDiv dper = fast_div((uint32_t)per), dou = fast_div((uint32_t)(g.OW / 2));
      hipLaunchKernelGGL(max_pool2d_22_kernel<XT>, dim3((unsigned)((items + 255) / 256)),
                         dim3(256), 0, stream, static_cast<const uint8_t*>(x),
                         static_cast<uint8_t*>(y), g.H, g.W, g.OH, g.OW, dper, dou,
                         (uint32_t)items);
      return check_launch();
    }
  }
  if (g.KW == 2 && g.sw == 2 && g.pw == 0 && aligned) {
    const int64_t per = (int64_t)g.OH * ((g.OW + 1) / 2);
    const int64_t items = g.N * g.C * per;
    if (items < ((int64_t)1 << 31)) {
      // two items per lane per step, at most POOL_WG_PER_CU workgroups per CU
      int64_t blocks = (items + 511) / 512;
      const int64_t cap = (int64_t)device_cu_count() * POOL_WG_PER_CU;
      if (blocks > cap) blocks = cap;
      if (blocks < 1) blocks = 1;
      const FastDiv dper = fast_div((uint32_t)per), dou = fast_div((uint32_t)((g.OW + 1) / 2));
      auto kern = g.KH == 2 ? max_pool2d_w2_kernel<XT, true> : max_pool2d_w2_kernel<XT, false>;
      hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream,
                         static_cast<const uint8_t*>(x), static_cast<uint8_t*>(y), g, dper, dou,
                         (uint32_t)items);
      return check_launch();
    }
  }
  const int64_t blocks = (g.N * g.C * npix + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(max_pool2d_kernel<XT>, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(x), static_cast<uint8_t*>(y), g);
  return check_launch();
}

template <int XT>
int launch_gap(const void* x, const float* x_scale, float* y, int64_t planes, int64_t hw,
               hipStream_t stream) {
  // the widest Q-element vector (Q * bytes <= 16) that every plane's, block's,
  // leaf's and group's start keeps aligned
  constexpr int EB = XL<XT>::bits / 8;
  int Q = 16 / EB < 8 ? 16 / EB : 8;
  while (Q > 1 && (hw % Q != 0 || reinterpret_cast<uintptr_t>(x) % ((uintptr_t)Q * EB) != 0))
    Q >>= 1;
  int lsh = 0;
  for (int lpl = 8 / Q; lpl > 1; lpl >>= 1) ++lsh;
  const bool sc = is_quant(XT) && x_scale != nullptr;  // the C ABI refuses other scales
  // one block whose tree fits a wave's lanes: several planes per wave
  const int D1 = hw <= NP_BUFSIZE ? gap_detail::tree_depth((int)hw) : 0;
  const int wshift = D1 + lsh;
  if (hw <= NP_BUFSIZE && wshift <= 6) {
    const int64_t blocks = ((planes << wshift) + 255) / 256;
    if (blocks > 0x7FFFFFFF || planes > ((int64_t)1 << 40)) return NOVAQ_EINVAL;
    const int ngmax = gap_detail::leaf_len((int)hw, true) >> 3;
    using Kern = decltype(&global_avg_pool2d_tree_kernel<XT, 1, false, 16>);
    Kern kern = nullptr;
    auto choose = [&](auto qc) {
      constexpr int QC = decltype(qc)::value;
      if (Q != QC) return;
      if (ngmax <= 8)
        kern = sc ? global_avg_pool2d_tree_kernel<XT, QC, is_quant(XT), 8>
                  : global_avg_pool2d_tree_kernel<XT, QC, false, 8>;
      else
        kern = sc ? global_avg_pool2d_tree_kernel<XT, QC, is_quant(XT), 16>
                  : global_avg_pool2d_tree_kernel<XT, QC, false, 16>;
    };
    choose(std::integral_constant<int, 1>{});
    choose(std::integral_constant<int, 2>{});
    choose(std::integral_constant<int, 4>{});
    if constexpr (EB < 4) choose(std::integral_constant<int, 8>{});
    if (!kern) return NOVAQ_EINVAL;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(x), x_scale, y, planes, (int)hw, D1, wshift);
    return check_launch();
  }
  // one wave per plane, over numpy's blocks in order
  const int64_t full = hw / NP_BUFSIZE, rest = hw - full * NP_BUFSIZE;
  const int nb_last = rest ? (int)rest : (int)NP_BUFSIZE;
  const int D_full = gap_detail::tree_depth((int)NP_BUFSIZE), D_last = gap_detail::tree_depth(nb_last);
  int longest = gap_detail::leaf_len(nb_last, true);
  if (full > (rest ? 0 : 1)) longest = std::max(longest, gap_detail::leaf_len((int)NP_BUFSIZE, true));
  const int ngmax = longest >> 3;
  const int64_t blocks = (planes + 3) / 4;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  using Kern = decltype(&global_avg_pool2d_plane_kernel<XT, 1, false, 16>);
  Kern kern = nullptr;
  auto choose = [&](auto qc) {
    constexpr int QC = decltype(qc)::value;
    if (Q != QC) return;
    if (ngmax <= 8)
      kern = sc ? global_avg_pool2d_plane_kernel<XT, QC, is_quant(XT), 8>
                : global_avg_pool2d_plane_kernel<XT, QC, false, 8>;
    else
      kern = sc ? global_avg_pool2d_plane_kernel<XT, QC, is_quant(XT), 16>
                : global_avg_pool2d_plane_kernel<XT, QC, false, 16>;
  };
  choose(std::integral_constant<int, 1>{});
  choose(std::integral_constant<int, 2>{});
  choose(std::integral_constant<int, 4>{});
  if constexpr (EB < 4) choose(std::integral_constant<int, 8>{});
  if (!kern) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(x), x_scale, y, planes, hw, D_full, D_last);
  return check_launch();
}


// ---------------------------------------------------------------------------
// Backward passes.
//
// MaxPool2d (MaxPool2d.backward, novann/layers/pooling/maxpool/maxpool2d.py:
// 79-129): over the forward's windows of the padded input, a window's maximum
// is NaN when it holds one (numpy's max) and its count is the number of its
// elements equal to that maximum, 1 when none is (a NaN maximum).  An element
// equal to the maximum receives 1 * (grad / count), any other element of the
// window 0 * (grad / count) -- a NaN where grad is not finite, as the
// reference's mask product gives; an input element adds what the windows
// holding it give, in (oh, ow) order, to +0, and what lands on the padding is
// dropped (the reference scatters into the padded shape and crops it).  fp32
// throughout, the divide IEEE-rounded.

// Window (i, j)'s maximum and count over the padded plane at base.
template <int XT>
__device__ __forceinline__ void window_max_count(const uint8_t* __restrict__ x, int64_t base,
                                                 const PoolGeom& g, int i, int j, float& mx,
                                                 int& cnt) {
  bool nan = false;
  mx = -INFINITY;
  for (int kh = 0; kh < g.KH; ++kh) {
    const int hi = pad_index(i * g.sh + kh - g.ph, g.H, g.pad_mode);
    for (int kw = 0; kw < g.KW; ++kw) {
      const int wi = pad_index(j * g.sw + kw - g.pw, g.W, g.pad_mode);
      const float v = (hi >= 0 && wi >= 0) ? x_val<XT>(x, base + (int64_t)hi * g.W + wi) : 0.0f;
      nan |= isnan(v);
      mx = v > mx ? v : mx;
    }
  }
  if (nan) mx = __builtin_nanf("");
  cnt = 0;
  for (int kh = 0; kh < g.KH; ++kh) {
    const int hi = pad_index(i * g.sh + kh - g.ph, g.H, g.pad_mode);
    for (int kw = 0; kw < g.KW; ++kw) {
      const int wi = pad_index(j * g.sw + kw - g.pw, g.W, g.pad_mode);
      const float v = (hi >= 0 && wi >= 0) ? x_val<XT>(x, base + (int64_t)hi * g.W + wi) : 0.0f;
      cnt += v == mx;
    }
  }
  if (cnt == 0) cnt = 1;
}

// Any geometry: lane t makes input element t (planes of H x W back to back)
// from the windows holding it, each window's maximum and count recomputed.
template <int XT>
__global__ __launch_bounds__(256) void max_pool2d_bwd_kernel(const float* __restrict__ grad,
                                                            const uint8_t* __restrict__ x,
                                                            float* __restrict__ gi, PoolGeom g) {
  const int64_t hw = (int64_t)g.H * g.W;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= g.N * g.C * hw) return;
  const int64_t plane = t / hw;
  const int pix = (int)(t - plane * hw);
  const int h = pix / g.W, w = pix - h * g.W;
  const float xv = x_val<XT>(x, t);
  // windows i with i*sh <= h + ph < i*sh + KH (and j likewise)
  const int hp = h + g.ph, wp = w + g.pw;
  const int i0 = hp >= g.KH ? (hp - g.KH) / g.sh + 1 : 0, i1 = min(g.OH - 1, hp / g.sh);
  const int j0 = wp >= g.KW ? (wp - g.KW) / g.sw + 1 : 0, j1 = min(g.OW - 1, wp / g.sw);
  const float* gp = grad + plane * g.OH * g.OW;
  float sum = 0.0f;
  for (int i = i0; i <= i1; ++i)
    for (int j = j0; j <= j1; ++j) {
      float mx;
      int cnt;
      window_max_count<XT>(x, plane * hw, g, i, j, mx, cnt);
      const float q = gp[(int64_t)i * g.OW + j] / (float)cnt;
      sum += (xv == mx ? 1.0f : 0.0f) * q;
    }
  gi[t] = sum;
}

// 2 x 2 windows, stride 2, no padding, H and W even (every input element in
// exactly one window: config [5]'s MaxPool2d(2, 2)): lane t makes window t's
// four gradients, its two input rows read as 2-element loads and its two
// gradient rows written as 8-byte stores (x aligned to 2 elements, gi to 8
// bytes).  t < 2^31: the divisions by the plane's windows and by OW are
// multiply-shifts.
template <int XT>
__global__ __launch_bounds__(256) void max_pool2d_bwd_22_kernel(
    const float* __restrict__ grad, const uint8_t* __restrict__ x, float* __restrict__ gi,
    int W, int OW, FastDiv dnpix, FastDiv dow, uint32_t windows, uint32_t npix) {
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= windows) return;
  const uint32_t plane = fdiv(t, dnpix), pix = t - plane * npix;
  const uint32_t i = fdiv(pix, dow), j = pix - i * (uint32_t)OW;
  const int64_t e0 = (int64_t)plane * (4 * (int64_t)npix) + (int64_t)(2 * i) * W + 2 * j;
  constexpr int B = XL<XT>::bits;
  uint32_t c[4];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int64_t e = e0 + (int64_t)r * W;
    if constexpr (B == 32) {
      const uint2 v = *reinterpret_cast<const uint2*>(x + e * 4);
      c[2 * r] = v.x;
      c[2 * r + 1] = v.y;
    } else if constexpr (B == 16) {
      const uint32_t v = *reinterpret_cast<const uint32_t*>(x + e * 2);
      c[2 * r] = v & 0xFFFFu;
      c[2 * r + 1] = v >> 16;
    } else {
      const uint32_t v = *reinterpret_cast<const uint16_t*>(x + e);
      c[2 * r] = v & 0xFFu;
      c[2 * r + 1] = v >> 8;
    }
  }
  float v[4];
  bool nan = false;
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] = u2f(decode<XT>(c[k]));
    nan |= isnan(v[k]);
    mx = v[k] > mx ? v[k] : mx;
  }
  if (nan) mx = __builtin_nanf("");
  int cnt = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) cnt += v[k] == mx;
  if (cnt == 0) cnt = 1;
  const float q = grad[t] / (float)cnt;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const float a = 0.0f + (v[2 * r] == mx ? 1.0f : 0.0f) * q;
    const float b = 0.0f + (v[2 * r + 1] == mx ? 1.0f : 0.0f) * q;
    *reinterpret_cast<float2*>(gi + e0 + (int64_t)r * W) = make_float2(a, b);
  }
}

template <int XT>
int launch_max_bwd(const float* grad, const void* x, float* gi, const PoolGeom& g,
                   hipStream_t stream) {
  const auto* xb = static_cast<const uint8_t*>(x);
  constexpr uintptr_t EB = XL<XT>::bits / 8;
  const int64_t npix = (int64_t)g.OH * g.OW;
  const int64_t windows = g.N * g.C * npix;
  if (g.KH == 2 && g.KW == 2 && g.sh == 2 && g.sw == 2 && g.ph == 0 && g.pw == 0 &&
      g.H == 2 * g.OH && g.W == 2 * g.OW && windows < ((int64_t)1 << 31) &&
      reinterpret_cast<uintptr_t>(x) % (2 * EB) == 0 && reinterpret_cast<uintptr_t>(gi) % 8 == 0) {
    hipLaunchKernelGGL(max_pool2d_bwd_22_kernel<XT>, dim3((unsigned)((windows + 255) / 256)),
                       dim3(256), 0, stream, grad, xb, gi, g.W, g.OW,
                       fast_div((uint32_t)npix), fast_div((uint32_t)g.OW), (uint32_t)windows,
                       (uint32_t)npix);
    return check_launch();
  }
  const int64_t blocks = (g.N * g.C * g.H * (int64_t)g.W + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(max_pool2d_bwd_kernel<XT>, dim3((unsigned)blocks), dim3(256), 0, stream,
                     grad, xb, gi, g);
  return check_launch();
}

// GlobalAvgPool2d (GlobalAvgPool2d.backward, novann/layers/pooling/gap/
// global_avg_pool2d.py:35-57): every element of plane p is grad[p] * f, f =
// 1 / (H*W) rounded to fp32 by the host (the reference's Python float factor
// becomes float32 in its product with the float32 grad; the ones it then
// multiplies by change nothing).  VEC: 4 elements a lane, one 16-byte store
// (H*W a multiple of 4, gi 16-byte aligned, fewer than 2^31 lanes).
template <bool VEC>
__global__ __launch_bounds__(256) void global_avg_pool2d_bwd_kernel(
    const float* __restrict__ grad, float* __restrict__ gi, int64_t lanes, int64_t hw, float f,
    FastDiv dq, uint32_t q) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= lanes) return;
  if constexpr (VEC) {
    const float v = grad[fdiv((uint32_t)t, dq)] * f;
    *reinterpret_cast<float4*>(gi + 4 * t) = make_float4(v, v, v, v);
    (void)hw;
    (void)q;
  } else {
    gi[t] = grad[t / hw] * f;
  }
}

}  // namespace

int max_pool2d_launch(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W,
                      int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode, void* y,
                      hipStream_t stream) {
  PoolGeom g{};
  g.N = N; g.C = C; g.H = (int)H; g.W = (int)W; g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw;
  g.ph = ph; g.pw = pw; g.pad_mode = pad_mode;
  g.OH = (int)((H + 2 * (int64_t)ph - KH) / sh + 1);
  g.OW = (int)((W + 2 * (int64_t)pw - KW) / sw + 1);
  switch (x_dtype) {
    case F32: return launch_max<F32>(x, y, g, stream);
    case F16: return launch_max<F16>(x, y, g, stream);
    case BF16: return launch_max<BF16>(x, y, g, stream);
    case E4M3: return launch_max<E4M3>(x, y, g, stream);
    case E5M2: return launch_max<E5M2>(x, y, g, stream);
    default: return NOVAQ_EDTYPE;
  }
}

int global_avg_pool2d_launch(const void* x, int x_dtype, const float* x_scale, int64_t planes,
                             int64_t hw, float* y, hipStream_t stream) {
  switch (x_dtype) {
    case F32: return launch_gap<F32>(x, x_scale, y, planes, hw, stream);
    case F16: return launch_gap<F16>(x, x_scale, y, planes, hw, stream);
    case BF16: return launch_gap<BF16>(x, x_scale, y, planes, hw, stream);
    case E4M3: return launch_gap<E4M3>(x, x_scale, y, planes, hw, stream);
    case E5M2: return launch_gap<E5M2>(x, x_scale, y, planes, hw, stream);
    default: return NOVAQ_EDTYPE;
  }
}

int max_pool2d_backward_launch(const float* grad, const void* x, int x_dtype, int64_t N,
                               int64_t C, int64_t H, int64_t W, int KH, int KW, int sh, int sw,
                               int ph, int pw, int pad_mode, float* grad_input,
                               hipStream_t stream) {
  PoolGeom g{};
  g.N = N; g.C = C; g.H = (int)H; g.W = (int)W; g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw;
  g.ph = ph; g.pw = pw; g.pad_mode = pad_mode;
  g.OH = (int)((H + 2 * (int64_t)ph - KH) / sh + 1);
  g.OW = (int)((W + 2 * (int64_t)pw - KW) / sw + 1);
  if ((int64_t)g.OH * g.OW > 0x7FFFFFFF || H * W > 0x7FFFFFFF) return NOVAQ_EINVAL;
  switch (x_dtype) {
    case F32: return launch_max_bwd<F32>(grad, x, grad_input, g, stream);
    case F16: return launch_max_bwd<F16>(grad, x, grad_input, g, stream);
    case BF16: return launch_max_bwd<BF16>(grad, x, grad_input, g, stream);
    case E4M3: return launch_max_bwd<E4M3>(grad, x, grad_input, g, stream);
    case E5M2: return launch_max_bwd<E5M2>(grad, x, grad_input, g, stream);
    default: return NOVAQ_EDTYPE;
  }
}

int global_avg_pool2d_backward_launch(const float* grad, int64_t planes, int64_t hw,
                                      float factor, float* grad_input, hipStream_t stream) {
  const int64_t total = planes * hw;
  if (hw % 4 == 0 && total / 4 < ((int64_t)1 << 31) &&
      reinterpret_cast<uintptr_t>(grad_input) % 16 == 0) {
    const int64_t lanes = total / 4;
    hipLaunchKernelGGL(global_avg_pool2d_bwd_kernel<true>, dim3((unsigned)((lanes + 255) / 256)),
                       dim3(256), 0, stream, grad, grad_input, lanes, hw, factor,
                       fast_div((uint32_t)(hw / 4)), (uint32_t)(hw / 4));
    return check_launch();
  }
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(global_avg_pool2d_bwd_kernel<false>, dim3((unsigned)blocks), dim3(256), 0,
                     stream, grad, grad_input, total, hw, factor, FastDiv{}, 0u);
  return check_launch();
}

}  // namespace novaq
