// Quantized-weight Linear forward on bf16 MFMA (gfx950).
//
//   y[M, N] = x[M, K] . (s * dec(W[N, K]))^T + bias[N]
//
// Both operands are K-contiguous ("NT" GEMM).  One workgroup owns a
// BM x BN = 128 x 256 tile of y and walks K in BK = 64 steps:
//   - x (fp32) is read with 16-byte loads, rounded to bf16 (RNE,
//     v_cvt_pk_bf16_f32) and written to LDS;
//   - W is read in its stored format (E4M3 / E5M2 / E2M1 / bf16 / f16 / f32)
//     and decoded to bf16 on the way into LDS; the FP8 / FP4 decodes are exact
//     (every E4M3, E5M2 and E2M1 value is a bf16 value) and use gfx950's
//     packed converts (v_cvt_scalef32_pk_bf16_{fp8,bf8,fp4}, scale 1.0);
//   - four waves (2 x 2) each compute a 64 x 128 sub-tile with
//     v_mfma_f32_32x32x16_bf16 (fp32 accumulation), reading 16-byte fragments
//     from LDS rows padded to 72 bf16 (144 B) so a wave's 32 rows fall in
//     distinct banks;
//   - LDS is double-buffered: the next K block is fetched into registers
//     while the current one is multiplied, then converted and stored into the
//     other buffer (one barrier per K block).
// The per-tensor scale s and the bias are applied in fp32 after accumulation.
// Tiles are numbered so that the workgroups the hardware sends to one XCD
// (block id mod 8) cover a compact 4-row group of tiles, so their x rows and W
// rows are shared through that XCD's L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 256, BK = 64;
constexpr int LDS_ROW = BK + 8;  // bf16 per LDS row
constexpr int THREADS = 256;
constexpr int WM = 64, WN = 128;  // per-wave sub-tile
constexpr int MT = WM / 32, NT = WN / 32;
constexpr int XCH = BM * BK / 4 / THREADS;  // x 16-byte chunks per thread

template <int WT>
struct W {
  static constexpr int bits = dtype_bits(WT);
  static constexpr int epc = 128 / bits;           // elements per 16-byte chunk
  static constexpr int chunks = BN * BK / epc / THREADS;  // per thread per K block
  static constexpr int words = epc / 2;            // bf16 pairs per chunk
};

__device__ __forceinline__ uint32_t bf16_pair(bf16x2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ uint32_t f32x2_to_bf16(uint32_t lo, uint32_t hi) {
  f32x2 f = {__uint_as_float(lo), __uint_as_float(hi)};
  return bf16_pair(__builtin_convertvector(f, bf16x2));
}

// Decode one 16-byte chunk of W (epc elements) into epc/2 bf16 pairs.
template <int WT>
__device__ __forceinline__ void decode_chunk(const u32x4& c, uint32_t* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t v = c[i];
    if constexpr (WT == E4M3) {
      out[2 * i] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, false));
      out[2 * i + 1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, true));
    } else if constexpr (WT == E5M2) {
      out[2 * i] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(v, 1.0f, false));
      out[2 * i + 1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(v, 1.0f, true));
    } else if constexpr (WT == E2M1) {
      out[4 * i] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 0));
      out[4 * i + 1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 1));
      out[4 * i + 2] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 2));
      out[4 * i + 3] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 3));
    } else if constexpr (WT == BF16) {
      out[i] = v;
    } else if constexpr (WT == F16) {
      f16x2 h = __builtin_bit_cast(f16x2, v);
      f32x2 f = __builtin_convertvector(h, f32x2);  // exact widening
      out[i] = bf16_pair(__builtin_convertvector(f, bf16x2));
    } else {  // F32: two chunk words per bf16 pair
      if (i % 2 == 0) out[i / 2] = f32x2_to_bf16(c[i], c[i + 1]);
    }
  }
}

// Element e of a row of W in storage order, for the guarded (edge) loads.
template <int WT>
__device__ __forceinline__ uint32_t load_w_elem(const uint8_t* row, int e) {
  if constexpr (W<WT>::bits == 32) return reinterpret_cast<const uint32_t*>(row)[e];
  else if constexpr (W<WT>::bits == 16) return reinterpret_cast<const uint16_t*>(row)[e];
  else if constexpr (W<WT>::bits == 8) return row[e];
  else return (row[e >> 1] >> ((e & 1) * 4)) & 0xFu;
}

// 16-byte chunk of row `r` (< rows) starting at element k (multiple of epc):
// one vector load when it lies inside the row and rows are 16-byte aligned,
// element loads with zero fill otherwise.
template <int WT>
__device__ __forceinline__ u32x4 load_w_chunk(const uint8_t* __restrict__ w, int r, int rows,
                                              int k, int K, size_t row_bytes, bool vec_ok) {
  constexpr int EPC = W<WT>::epc;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (r >= rows) return v;
  const uint8_t* row = w + (size_t)r * row_bytes;
  if (vec_ok && k + EPC <= K) return *reinterpret_cast<const u32x4*>(row + (size_t)k * W<WT>::bits / 8);
  constexpr int bits = W<WT>::bits;
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    if (k + e < K) {
      uint32_t c = load_w_elem<WT>(row, k + e);
      v[(e * bits) / 32] |= c << ((e * bits) % 32);
    }
  }
  return v;
}

__device__ __forceinline__ u32x4 load_x_chunk(const float* __restrict__ x, int r, int rows, int k,
                                              int K, bool vec_ok) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (r >= rows) return v;
  const float* row = x + (size_t)r * K;
  if (vec_ok && k + 4 <= K) return *reinterpret_cast<const u32x4*>(row + k);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (k + e < K) v[e] = __float_as_uint(row[k + e]);
  return v;
}

template <int WT>
__global__ __launch_bounds__(THREADS, 1) void linear_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ w_scale,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n, int x_vec, int w_vec) {
  __shared__ __attribute__((aligned(16))) __bf16 As[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[2][BN * LDS_ROW];
  using WTr = W<WT>;
  constexpr int WCPR = BK / WTr::epc;  // W chunks per tile row
  const size_t w_row_bytes = (size_t)K * WTr::bits / 8;

  // tile index: XCD-contiguous, then 4-row groups walked column by column
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  constexpr int GM = 4;
  const int group = t / (GM * tiles_n);
  const int first_m = group * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int rem = t - group * GM * tiles_n;
  const int m0 = (first_m + rem % gm) * BM;
  const int n0 = (rem / gm) * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave & 1) * WM, wn = (wave >> 1) * WN;

  u32x4 xr[XCH];
  u32x4 wr[WTr::chunks];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      int c = tid + THREADS * i;
      xr[i] = load_x_chunk(x, m0 + (c >> 4), M, k0 + (c & 15) * 4, K, x_vec);
    }
#pragma unroll
    for (int i = 0; i < WTr::chunks; ++i) {
      int c = tid + THREADS * i;
      wr[i] = load_w_chunk<WT>(w, n0 + c / WCPR, N, k0 + (c % WCPR) * WTr::epc, K, w_row_bytes,
                               w_vec);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      int c = tid + THREADS * i;
      uint32_t p0 = f32x2_to_bf16(xr[i][0], xr[i][1]);
      uint32_t p1 = f32x2_to_bf16(xr[i][2], xr[i][3]);
      *reinterpret_cast<uint2*>(&As[buf][(c >> 4) * LDS_ROW + (c & 15) * 4]) = make_uint2(p0, p1);
    }
#pragma unroll
    for (int i = 0; i < WTr::chunks; ++i) {
      int c = tid + THREADS * i;
      uint32_t words[WTr::words];
      decode_chunk<WT>(wr[i], words);
      uint32_t* dst = reinterpret_cast<uint32_t*>(&Bs[buf][(c / WCPR) * LDS_ROW + (c % WCPR) * WTr::epc]);
      if constexpr (WTr::words == 2) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(words[0], words[1]);
      } else {
#pragma unroll
        for (int q = 0; q < WTr::words; q += 4)
          *reinterpret_cast<uint4*>(dst + q) =
              make_uint4(words[q], words[q + 1], words[q + 2], words[q + 3]);
      }
    }
  };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

  const int kblocks = (K + BK - 1) / BK;
  fetch(0);
  stage(0);
  __syncthreads();
  for (int kb = 0; kb < kblocks; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < kblocks;
    if (more) fetch((kb + 1) * BK);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int kk = s * 16 + (lane >> 5) * 8;
      bf16x8 a[MT], b[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(&As[buf][(wm + i * 32 + (lane & 31)) * LDS_ROW + kk]);
#pragma unroll
      for (int j = 0; j < NT; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(wn + j * 32 + (lane & 31)) * LDS_ROW + kk]);
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (more) stage(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column (lane & 31) and rows 8*(r/4) + 4*(lane/32) + r%4
  const float s = w_scale ? *w_scale : 1.0f;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int col = n0 + wn + j * 32 + (lane & 31);
    if (col >= N) continue;
    const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M) y[(size_t)row * N + col] = acc[i][j][r] * s + bv;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fast path: whole tiles only (M % 128 == 0, N % 256 == 0, K % 64 == 0), no
// bounds logic.  W stays in its stored format in LDS (1 byte per E4M3/E5M2
// element, half a byte per E2M1, 2 bytes for bf16/f16) and each wave decodes
// its B fragments after the LDS read, so LDS traffic for W is that of the
// packed codes.  The next K block is fetched into registers while the
// current one is multiplied; LDS fragments are double-buffered across the
// four 16-deep MFMA steps of a K block.

template <int WT, int FBN>
struct Fast {
  static constexpr int bits = dtype_bits(WT);
  static constexpr int row_bytes = BK * bits / 8;        // W bytes per tile row per K block
  // LDS row pitch: keeps a wave's 32-row fragment reads in distinct banks
  static constexpr int pitch = bits == 4 ? 36 : bits == 8 ? 72 : 144;
  static constexpr int chunks = FBN * row_bytes / 16 / THREADS;  // 16-byte W chunks per thread
  static constexpr int cpr = row_bytes / 16;             // chunks per W row
  static constexpr int frag_bytes = 8 * bits / 8;        // one lane's 8 elements
};

constexpr int A_PITCH = BK + 8;                      // bf16 per A row in LDS
constexpr int A_STAGE = BM * A_PITCH * 2;            // bytes

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 8 stored W elements (one lane's fragment) -> 8 bf16 for the MFMA B operand
template <int WT>
__device__ __forceinline__ bf16x8 frag_to_bf16(const uint8_t* p) {
  uint32_t o[4];
  if constexpr (WT == E4M3 || WT == E5M2) {
    u32x2 v = *reinterpret_cast<const u32x2*>(p);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if constexpr (WT == E4M3) {
        o[2 * i] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[i], 1.0f, false));
        o[2 * i + 1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v[i], 1.0f, true));
      } else {
        o[2 * i] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(v[i], 1.0f, false));
        o[2 * i + 1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(v[i], 1.0f, true));
      }
    }
  } else if constexpr (WT == E2M1) {
    uint32_t v = *reinterpret_cast<const uint32_t*>(p);
    o[0] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 0));
    o[1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 1));
    o[2] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 2));
    o[3] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 3));
  } else if constexpr (WT == BF16) {
    return *reinterpret_cast<const bf16x8*>(p);
  } else {  // F16
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // the element goes through a scalar first: bit-casting v[i] directly
      // makes this compiler (ROCm 7.2 clang) reuse element 0 for every i
      const uint32_t word = v[i];
      f32x2 f = __builtin_convertvector(__builtin_bit_cast(f16x2, word), f32x2);
      o[i] = bf16_pair(__builtin_convertvector(f, bf16x2));
    }
  }
  u32x4 r = {o[0], o[1], o[2], o[3]};
  return __builtin_bit_cast(bf16x8, r);
}

// FBN: tile width in outputs (128 or 256); OCC: workgroups per CU the
// register budget is sized for; PF: K blocks fetched ahead (1 or 2); WLM:
// waves along M (2: 2 x 2 waves of 64 x FBN/2; 1: 1 x 4 waves of 128 x
// FBN/4, where every W element is decoded by exactly one wave).
template <int WT, int FBN, int OCC, int PF, int WLM>
__global__ __launch_bounds__(THREADS, OCC) void linear_fast_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ w_scale,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n) {
  using F = Fast<WT, FBN>;
  constexpr int WM = BM / WLM;             // per-wave rows
  constexpr int MT = WM / 32;
  constexpr int FWN = FBN / (4 / WLM);     // per-wave width
  constexpr int FNT = FWN / 32;
  constexpr int B_STAGE = FBN * F::pitch;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (A_STAGE + B_STAGE)];

  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  constexpr int GM = 4;
  const int group = t / (GM * tiles_n);
  const int first_m = group * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int rem = t - group * GM * tiles_n;
  const int m0 = (first_m + rem % gm) * BM;
  const int n0 = (rem / gm) * FBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  const int wm = (wave % WLM) * WM, wn = (wave / WLM) * FWN;
  const size_t w_row_bytes = (size_t)K * F::bits / 8;

  // Global sources: a uniform tile base, one per-lane offset, and uniform
  // per-chunk strides (chunk i of a thread is 16*i rows of x / 256*i/cpr rows
  // of W further down), so addresses cost scalar registers, not vector ones.
  const float* xtile = x + (size_t)m0 * K;
  const uint32_t xlane = (uint32_t)((tid >> 4) * K + (tid & 15) * 4);  // floats
  const size_t xstep = (size_t)16 * K;                                   // floats per chunk
  const int xdst0 = ((tid >> 4) * A_PITCH + (tid & 15) * 4) * 2;        // LDS bytes
  constexpr int XDST_STEP = 16 * A_PITCH * 2;
  const uint8_t* wtile = w + (size_t)n0 * w_row_bytes;
  const uint32_t wlane = (uint32_t)((tid / F::cpr) * w_row_bytes + (tid % F::cpr) * 16);
  const size_t wstep = (size_t)(THREADS / F::cpr) * w_row_bytes;
  const int wdst0 = (tid / F::cpr) * F::pitch + (tid % F::cpr) * 16;
  constexpr int WDST_STEP = (THREADS / F::cpr) * F::pitch;

  struct Regs {
    u32x4 x[XCH];
    u32x4 w[F::chunks];
  };
  auto fetch = [&](Regs& r, int kb) {
    const float* xk = xtile + (size_t)kb * BK;
    const uint8_t* wk = wtile + (size_t)kb * F::row_bytes;
#pragma unroll
    for (int i = 0; i < XCH; ++i)
      r.x[i] = *reinterpret_cast<const u32x4*>(xk + i * xstep + xlane);
#pragma unroll
    for (int i = 0; i < F::chunks; ++i)
      r.w[i] = *reinterpret_cast<const u32x4*>(wk + i * wstep + wlane);
  };
  auto stage = [&](const Regs& r, int buf) {
    uint8_t* A = lds + buf * (A_STAGE + B_STAGE) + xdst0;
    uint8_t* B = lds + buf * (A_STAGE + B_STAGE) + A_STAGE + wdst0;
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      uint32_t p0 = f32x2_to_bf16(r.x[i][0], r.x[i][1]);
      uint32_t p1 = f32x2_to_bf16(r.x[i][2], r.x[i][3]);
      *reinterpret_cast<u32x2*>(A + i * XDST_STEP) = u32x2{p0, p1};
    }
#pragma unroll
    for (int i = 0; i < F::chunks; ++i) {
      uint8_t* d = B + i * WDST_STEP;
      if constexpr (F::pitch % 16 == 0) {
        *reinterpret_cast<u32x4*>(d) = r.w[i];
      } else if constexpr (F::pitch % 8 == 0) {
        *reinterpret_cast<u32x2*>(d) = u32x2{r.w[i][0], r.w[i][1]};
        *reinterpret_cast<u32x2*>(d + 8) = u32x2{r.w[i][2], r.w[i][3]};
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t*>(d + 4 * q) = r.w[i][q];
      }
    }
  };

  f32x16 acc[MT][FNT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < FNT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

  // fragment addresses (bytes) within a stage
  int aoff[MT], boff[FNT];
#pragma unroll
  for (int i = 0; i < MT; ++i) aoff[i] = ((wm + i * 32 + (lane & 31)) * A_PITCH + half * 8) * 2;
#pragma unroll
  for (int j = 0; j < FNT; ++j)
    boff[j] = A_STAGE + (wn + j * 32 + (lane & 31)) * F::pitch + half * F::frag_bytes;

  auto compute = [&](int buf) {
    const uint8_t* S = lds + buf * (A_STAGE + B_STAGE);
    bf16x8 a[2][MT], b[2][FNT];
#pragma unroll
    for (int i = 0; i < MT; ++i) a[0][i] = *reinterpret_cast<const bf16x8*>(S + aoff[i]);
#pragma unroll
    for (int j = 0; j < FNT; ++j) b[0][j] = frag_to_bf16<WT>(S + boff[j]);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
          a[nxt][i] = *reinterpret_cast<const bf16x8*>(S + aoff[i] + (s + 1) * 32);
#pragma unroll
        for (int j = 0; j < FNT; ++j)
          b[nxt][j] = frag_to_bf16<WT>(S + boff[j] + (s + 1) * 2 * F::frag_bytes);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < FNT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[cur][i], b[cur][j], acc[i][j], 0, 0, 0);
    }
  };

  // K blocks alternate between LDS buffers 0 and 1; a buffer is rewritten
  // only after the barrier that ends its last reads.
  const int kblocks = K / BK;
  if constexpr (PF == 1) {
    Regs r;
    fetch(r, 0);
    stage(r, 0);
    __syncthreads();
    for (int kb = 0; kb < kblocks; ++kb) {
      const bool more = kb + 1 < kblocks;
      if (more) fetch(r, kb + 1);
      compute(kb & 1);
      if (more) stage(r, (kb + 1) & 1);
      __syncthreads();
    }
  } else {
    // two register sets: K block kb+2 is in flight while kb+1 waits to be staged
    Regs ra, rb;
    fetch(ra, 0);
    if (kblocks > 1) fetch(rb, 1);
    stage(ra, 0);
    __syncthreads();
    for (int kb = 0; kb < kblocks; kb += 2) {
      if (kb + 2 < kblocks) fetch(ra, kb + 2);
      compute(0);
      if (kb + 1 < kblocks) stage(rb, 1);
      __syncthreads();
      if (kb + 1 < kblocks) {
        if (kb + 3 < kblocks) fetch(rb, kb + 3);
        compute(1);
        if (kb + 2 < kblocks) stage(ra, 0);
        __syncthreads();
      }
    }
  }

  const float s = w_scale ? *w_scale : 1.0f;
#pragma unroll
  for (int j = 0; j < FNT; ++j) {
    const int col = n0 + wn + j * 32 + (lane & 31);
    const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        __builtin_nontemporal_store(acc[i][j][r] * s + bv, &y[(size_t)row * N + col]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Staged-decode variant: W is decoded to bf16 once per workgroup while it is
// written to LDS (instead of once per wave after every LDS read), and the
// staging of K block kb+1 (x rounding, W decoding, LDS writes) is spread over
// MFMA steps 1..3 of block kb so the converts issue while the matrix core is
// busy.  The MFMA loop itself is then only 16-byte LDS reads and MFMAs.

constexpr int B_PITCH = BK + 8;  // bf16 per W row in LDS (144 B, conflict-free fragment reads)

template <int WT, int FBN, int OCC>
__global__ __launch_bounds__(THREADS, OCC) void linear_sd_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w, const float* __restrict__ w_scale,
    const float* __restrict__ bias, float* __restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n) {
  using WTr = W<WT>;
  constexpr int FWN = FBN / 2;
  constexpr int FNT = FWN / 32;
  constexpr int B_STAGE = FBN * B_PITCH * 2;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int WCH = FBN * BK / WTr::epc / THREADS;  // W chunks per thread
  constexpr int WCPR = BK / WTr::epc;                  // W chunks per row
  constexpr int UNITS = XCH + WCH;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  constexpr int GM = 4;
  const int group = t / (GM * tiles_n);
  const int first_m = group * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int rem = t - group * GM * tiles_n;
  const int m0 = (first_m + rem % gm) * BM;
  const int n0 = (rem / gm) * FBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  const int wm = (wave & 1) * WM, wn = (wave >> 1) * FWN;
  const size_t w_row_bytes = (size_t)K * WTr::bits / 8;

  const float* xtile = x + (size_t)m0 * K;
  const uint32_t xlane = (uint32_t)((tid >> 4) * K + (tid & 15) * 4);
  const size_t xstep = (size_t)16 * K;
  const int xdst0 = ((tid >> 4) * A_PITCH + (tid & 15) * 4) * 2;
  constexpr int XDST_STEP = 16 * A_PITCH * 2;
  const uint8_t* wtile = w + (size_t)n0 * w_row_bytes;
  const uint32_t wlane = (uint32_t)((tid / WCPR) * w_row_bytes + (tid % WCPR) * 16);
  const size_t wstep = (size_t)(THREADS / WCPR) * w_row_bytes;
  const int wdst0 = A_STAGE + ((tid / WCPR) * B_PITCH + (tid % WCPR) * WTr::epc) * 2;
  constexpr int WDST_STEP = (THREADS / WCPR) * B_PITCH * 2;

  u32x4 xr[XCH], wr[WCH];
  auto fetch = [&](int kb) {
    const float* xk = xtile + (size_t)kb * BK;
    const uint8_t* wk = wtile + (size_t)kb * (BK * WTr::bits / 8);
#pragma unroll
    for (int i = 0; i < XCH; ++i) xr[i] = *reinterpret_cast<const u32x4*>(xk + i * xstep + xlane);
#pragma unroll
    for (int i = 0; i < WCH; ++i) wr[i] = *reinterpret_cast<const u32x4*>(wk + i * wstep + wlane);
  };
  // staging units u in [u0, u1): x chunks first, then W chunks
  auto stage_units = [&](uint8_t* S, int u0, int u1) {
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      if (u < u0 || u >= u1) continue;
      if (u < XCH) {
        uint32_t p0 = f32x2_to_bf16(xr[u][0], xr[u][1]);
        uint32_t p1 = f32x2_to_bf16(xr[u][2], xr[u][3]);
        *reinterpret_cast<u32x2*>(S + xdst0 + u * XDST_STEP) = u32x2{p0, p1};
      } else {
        const int i = u - XCH;
        uint32_t words[WTr::words];
        decode_chunk<WT>(wr[i], words);
        uint8_t* d = S + wdst0 + i * WDST_STEP;
#pragma unroll
        for (int q = 0; q < WTr::words; q += 4)
          *reinterpret_cast<u32x4*>(d + 4 * q) = u32x4{words[q], words[q + 1], words[q + 2], words[q + 3]};
      }
    }
  };

  f32x16 acc[MT][FNT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < FNT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

  int aoff[MT], boff[FNT];
#pragma unroll
  for (int i = 0; i < MT; ++i) aoff[i] = ((wm + i * 32 + (lane & 31)) * A_PITCH + half * 8) * 2;
#pragma unroll
  for (int j = 0; j < FNT; ++j) boff[j] = A_STAGE + ((wn + j * 32 + (lane & 31)) * B_PITCH + half * 8) * 2;

  const int kblocks = K / BK;
  fetch(0);
  stage_units(lds, 0, UNITS);
  __syncthreads();
  for (int kb = 0; kb < kblocks; ++kb) {
    const uint8_t* S = lds + (kb & 1) * STAGE;
    uint8_t* Snext = lds + ((kb + 1) & 1) * STAGE;
    // The last block fetches and stages itself once more into the idle
    // buffer, so the loop body has no branch and schedules as one region.
    fetch(min(kb + 1, kblocks - 1));
    bf16x8 a[2][MT], b[2][FNT];
#pragma unroll
    for (int i = 0; i < MT; ++i) a[0][i] = *reinterpret_cast<const bf16x8*>(S + aoff[i]);
#pragma unroll
    for (int j = 0; j < FNT; ++j) b[0][j] = *reinterpret_cast<const bf16x8*>(S + boff[j]);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < BK / 16) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
          a[nxt][i] = *reinterpret_cast<const bf16x8*>(S + aoff[i] + (s + 1) * 32);
#pragma unroll
        for (int j = 0; j < FNT; ++j)
          b[nxt][j] = *reinterpret_cast<const bf16x8*>(S + boff[j] + (s + 1) * 32);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < FNT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[cur][i], b[cur][j], acc[i][j], 0, 0, 0);
      // a third of the next block's staging after each of MFMA steps 1..3
      if (s >= 1) stage_units(Snext, (s - 1) * UNITS / 3, s * UNITS / 3);
    }
    __syncthreads();
  }

  const float s = w_scale ? *w_scale : 1.0f;
#pragma unroll
  for (int j = 0; j < FNT; ++j) {
    const int col = n0 + wn + j * 32 + (lane & 31);
    const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        __builtin_nontemporal_store(acc[i][j][r] * s + bv, &y[(size_t)row * N + col]);
      }
    }
  }
}

// Whole-tile configuration: tile width, workgroups per CU, prefetch depth.
#ifndef NOVAQ_LINEAR_CFG
#define NOVAQ_LINEAR_CFG 5
#endif
constexpr int kCfg = NOVAQ_LINEAR_CFG;
constexpr bool kSD = kCfg >= 4;  // staged-decode kernel
constexpr int kFBN = (kCfg == 2 || kCfg == 3 || kCfg == 5) ? 128 : 256;
constexpr int kOCC = (kCfg == 2 || kCfg == 3 || kCfg == 5) ? 2 : 1;
constexpr int kPF = (kCfg == 1 || kCfg == 3) ? 2 : 1;
#ifndef NOVAQ_LINEAR_WLM
#define NOVAQ_LINEAR_WLM 2
#endif
constexpr int kWLM = NOVAQ_LINEAR_WLM;

template <int WT>
int launch(const float* x, int64_t M, int64_t K, const void* w, const float* w_scale,
           const float* bias, int64_t N, float* y, hipStream_t stream) {
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int64_t T = tiles_m * tiles_n;
  if (T > 0x7FFFFFFF || M > 0x7FFFFFFF || N > 0x7FFFFFFF || K > 0x7FFFFFFF) return NOVAQ_EINVAL;
  if constexpr (WT != F32) {
    const bool whole = M % BM == 0 && N % kFBN == 0 && K % BK == 0 && K > 0;
    if (whole) {
      const int64_t ftn = N / kFBN;
      if constexpr (kSD) {
        hipLaunchKernelGGL((linear_sd_kernel<WT, kFBN, kOCC>), dim3((unsigned)(tiles_m * ftn)),
                           dim3(THREADS), 0, stream, x, static_cast<const uint8_t*>(w), w_scale,
                           bias, y, (int)M, (int)N, (int)K, (int)tiles_m, (int)ftn);
      } else {
        hipLaunchKernelGGL((linear_fast_kernel<WT, kFBN, kOCC, kPF, kWLM>),
                           dim3((unsigned)(tiles_m * ftn)), dim3(THREADS), 0, stream, x,
                           static_cast<const uint8_t*>(w), w_scale, bias, y, (int)M, (int)N,
                           (int)K, (int)tiles_m, (int)ftn);
      }
      return check_launch();
    }
  }
  const int x_vec = (K % 4) == 0;
  const int w_vec = ((K * W<WT>::bits / 8) % 16) == 0 && (K * W<WT>::bits) % 8 == 0;
  hipLaunchKernelGGL((linear_kernel<WT>), dim3((unsigned)T), dim3(THREADS), 0, stream, x,
                     static_cast<const uint8_t*>(w), w_scale, bias, y, (int)M, (int)N, (int)K,
                     (int)tiles_m, (int)tiles_n, x_vec, w_vec);
  return check_launch();
}

}  // namespace

int linear_launch(const float* x, int64_t N, int64_t D_in, const void* w_q, int w_dtype,
                  const float* w_scale, const float* bias, int64_t D_out, float* y,
                  hipStream_t stream) {
  switch (w_dtype) {
    case E4M3: return launch<E4M3>(x, N, D_in, w_q, w_scale, bias, D_out, y, stream);
    case E5M2: return launch<E5M2>(x, N, D_in, w_q, w_scale, bias, D_out, y, stream);
    case E2M1: return launch<E2M1>(x, N, D_in, w_q, w_scale, bias, D_out, y, stream);
    case BF16: return launch<BF16>(x, N, D_in, w_q, w_scale, bias, D_out, y, stream);
    case F16: return launch<F16>(x, N, D_in, w_q, w_scale, bias, D_out, y, stream);
    case F32: return launch<F32>(x, N, D_in, w_q, w_scale, bias, D_out, y, stream);
    default: return NOVAQ_EDTYPE;
  }
}

}  // namespace novaq
