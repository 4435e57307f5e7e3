// Quantized-weight Linear forward on bf16 MFMA (gfx950) -- kernels, included
// by one translation unit per x dtype (linear.hip: fp32 x and the dispatch;
// linear_x*.hip: the others), so each file compiles in about the time one did.
//
//   y[M, N] = epilogue(x[M, K] . (s_w * dec(W[N, K]))^T * s_x + bias[N])
//
// Both operands are K-contiguous ("NT" GEMM).  x (fp32, or bf16 / f16 / FP8
// as a fused epilogue stored it) becomes bf16 on its way into LDS (fp32 and
// f16 rounded to nearest even, FP8 decoded exactly); W is read in its stored
// format (E4M3 / E5M2 / E2M1 / bf16 / f16 / f32) and decoded to bf16 with
// gfx950's packed converts (v_cvt_scalef32_pk_bf16_{fp8,bf8,fp4}, scale 1.0),
// which are exact: every E4M3, E5M2 and E2M1 value is a bf16 value.  Products
// run on v_mfma_f32_32x32x16_bf16 with fp32 accumulation; the per-tensor scale
// s and the bias are applied in fp32 after accumulation.
//
// Five kernels, chosen by shape and the operands' formats:
//   - linear_f8_kernel (x stored as E4M3 / E5M2 and FP8 / FP4 weights, M % 128,
//     N % 256, K % 128): both operands' codes on the FP8 MFMA
//     (v_mfma_f32_32x32x64_f8f6f4), loaded straight into LDS;
//   - linear_pingpong_kernel (FP8 weights, x in fp32 / bf16 / f16, M % 128,
//     N % 256, K % 128): the 128 x 256 tile on two wave groups that take
//     turns at the matrix cores and at the operand traffic;
//   - linear_wide_kernel (E2M1 weights, and FP8 weights in their [K][N]
//     layout for the backward; M % 128, N % 256, K % 128): one 128 x 256 tile
//     per workgroup of 8 waves, K blocks of 128 (one 128-byte line of an FP8
//     W row), W raw in LDS and decoded per MFMA fragment, buffer loads with
//     SGPR offsets;
//   - linear_pipe_kernel (whole 128-row tiles, K % 64): W decoded once per
//     workgroup into bf16 LDS tiles, loads kept up to 3 K blocks ahead;
//   - linear_kernel: any shape (guarded edge tiles) and fp32 weights.
// Tiles are numbered so that the workgroups the hardware sends to one XCD
// (block id mod 8) cover a compact 4-row group of tiles, so their x rows and W
// rows are shared through that XCD's L2.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"
#include "novaq_epilogue.h"
#include "novaq_internal.h"
#include "novaq_xload.h"

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

// Raw codes of x elements k .. k+3 of row r (zeros past the row or matrix).
template <int XT>
__device__ __forceinline__ u32x4 load_x_chunk(const uint8_t* __restrict__ x, int r, int rows,
                                              int k, int K, bool vec_ok) {
  if (r >= rows) return u32x4{0u, 0u, 0u, 0u};
  const int64_t e = (int64_t)r * K + k;
  if (vec_ok && k + 4 <= K) return x4_raw<XT>(x, e);
  return x4_raw_guarded<XT>(x, e, (int64_t)r * K + K);
}

template <int WT, int XT>
__global__ __launch_bounds__(THREADS, 1) void linear_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale,
    Epilogue ep, void* __restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n, int x_vec, int w_vec) {
  __shared__ __attribute__((aligned(16))) __bf16 As[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[2][BN * LDS_ROW];
  using WTr = W<WT>;
  constexpr int WCPR = BK / WTr::epc;  // W chunks per tile row
  // rows of whole bytes: an odd-length E2M1 row ends with a pad nibble
  const size_t w_row_bytes = ((size_t)K * WTr::bits + 7) / 8;

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
      xr[i] = load_x_chunk<XT>(x, m0 + (c >> 4), M, k0 + (c & 15) * 4, K, x_vec);
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
      const xl_u32x2 pr = x4_bf16<XT>(xr[i]);
      *reinterpret_cast<uint2*>(&As[buf][(c >> 4) * LDS_ROW + (c & 15) * 4]) = make_uint2(pr[0], pr[1]);
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
  const float s = product_scale(w_scale, x_scale);
  const float inv_o = epi_inv_scale(ep);
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int col = n0 + wn + j * 32 + (lane & 31);
    if (col >= N) continue;
    const EpiChan k = epi_chan(ep, col);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < M) {
          const float v = epi_value(ep, k, acc[i][j][r], s);
          if (ep.amax) am = epi_track(am, v);
          epi_store(ep.out_dtype, y, (size_t)row * N + col, v, inv_o);
        }
      }
    }
  }
  epi_amax_commit(ep, am);
}

// Epilogue of a whole tile of 32 x 32 MFMA accumulators (acc[i][j]: rows
// row0 + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4, column col0 + 32 j +
// lane % 32): one copy of the store loop per output dtype and no branch on
// the epilogue's fields per element (epi_value_nb, the same bits); fp32 goes
// out with non-temporal stores.
template <int OD, int MTn, int NTn>
__device__ __forceinline__ uint32_t store_tile(const Epilogue& ep, const f32x16 (&acc)[MTn][NTn],
                                               float s, float inv_o, float z, void* y, int N,
                                               int row0, int col0, int lane) {
  uint32_t am = 0;
  const int half = lane >> 5;
#pragma unroll
  for (int j = 0; j < NTn; ++j) {
    const int col = col0 + j * 32 + (lane & 31);
    const EpiChan k = epi_chan(ep, col);
#pragma unroll
    for (int i = 0; i < MTn; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        const float v = epi_value_nb(k, acc[i][j][r], s, z);
        am = epi_track(am, v);  // committed only with ep.amax
        if constexpr (OD == F32)
          __builtin_nontemporal_store(v, reinterpret_cast<float*>(y) + (size_t)row * N + col);
        else
          epi_store_t<OD>(y, (size_t)row * N + col, v, inv_o);
      }
    }
  }
  return am;
}

template <int MTn, int NTn>
__device__ __forceinline__ void tile_epilogue(const Epilogue& ep, const f32x16 (&acc)[MTn][NTn],
                                              float s, void* y, int N, int row0, int col0,
                                              int lane) {
  const float inv_o = epi_inv_scale(ep), z = epi_relu_factor(ep);
  uint32_t am;
  switch (ep.out_dtype) {
    case F16: am = store_tile<F16>(ep, acc, s, inv_o, z, y, N, row0, col0, lane); break;
    case BF16: am = store_tile<BF16>(ep, acc, s, inv_o, z, y, N, row0, col0, lane); break;
    case E4M3: am = store_tile<E4M3>(ep, acc, s, inv_o, z, y, N, row0, col0, lane); break;
    case E5M2: am = store_tile<E5M2>(ep, acc, s, inv_o, z, y, N, row0, col0, lane); break;
    default: am = store_tile<F32>(ep, acc, s, inv_o, z, y, N, row0, col0, lane); break;
  }
  epi_amax_commit(ep, am);
}

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

// gfx950's transposing LDS read (ds_read_b64_tr_b8), for W kept in its own
// [K][N] layout: within each group of 16 lanes, lane p names 8 bytes (row
// 2 j + h of the group's 8 rows, with j = (p % 16) / 2 and h = p % 2 picking
// the half of a 16-byte column run), and lane i receives byte i % 8 of the
// runs named by lanes 2 j + i / 8: 8 consecutive K of one N index.
typedef int i32x2_lds __attribute__((ext_vector_type(2)));

constexpr int B_PITCH = BK + 8;  // bf16 per W row in LDS (144 B, conflict-free fragment reads)

// ---------------------------------------------------------------------------
// Pipelined staged-decode kernel (whole tiles, any weight format but fp32):
// W is decoded to bf16 once per workgroup while it is written to LDS, so the
// MFMA loop is only 16-byte LDS reads and MFMAs.  NW waves (2 along M x NW/2
// along N, each 64 x FBN*2/NW); PF register sets keep global loads PF K
// blocks ahead: block kb+PF is loaded while block kb+1 (loaded PF-1 blocks
// earlier) is converted into the idle LDS buffer after MFMA steps 1..3.

template <int WT, int XT, int FBN, int NW, int OCC, int PF>
__global__ __launch_bounds__(NW * 64, OCC) void linear_pipe_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale,
    Epilogue ep, void* __restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n) {
  using WTr = W<WT>;
  constexpr int NTH = NW * 64;
  constexpr int FWN = FBN * 2 / NW;
  constexpr int FNT = FWN / 32;
  constexpr int B_STAGE = FBN * B_PITCH * 2;
  constexpr int STAGE = A_STAGE + B_STAGE;
  constexpr int XC = BM * BK / 4 / NTH;               // x chunks per thread
  constexpr int WCPR = BK / WTr::epc;                 // W chunks per row
  constexpr int WC = FBN * BK / WTr::epc / NTH;       // W chunks per thread
  constexpr int UNITS = XC + WC;
  static_assert(FNT >= 1 && XC >= 1 && WC >= 1 && NTH % WCPR == 0, "tile shape");
  static_assert(PF >= 1 && PF <= 3, "prefetch distance");
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

  const uint8_t* xtile = x + (size_t)m0 * K * XL<XT>::bytes;
  const uint32_t xlane = (uint32_t)((tid >> 4) * K + (tid & 15) * 4);
  const size_t xstep = (size_t)(NTH / 16) * K;
  const int xdst0 = ((tid >> 4) * A_PITCH + (tid & 15) * 4) * 2;
  constexpr int XDST_STEP = (NTH / 16) * A_PITCH * 2;
  const uint8_t* wtile = w + (size_t)n0 * w_row_bytes;
  const uint32_t wlane = (uint32_t)((tid / WCPR) * w_row_bytes + (tid % WCPR) * 16);
  const size_t wstep = (size_t)(NTH / WCPR) * w_row_bytes;
  const int wdst0 = A_STAGE + ((tid / WCPR) * B_PITCH + (tid % WCPR) * WTr::epc) * 2;
  constexpr int WDST_STEP = (NTH / WCPR) * B_PITCH * 2;

  struct Regs {
    u32x4 x[XC];
    u32x4 w[WC];
  };
  auto fetch = [&](Regs& r, int kb) {
    const size_t xk = (size_t)kb * BK;
    const uint8_t* wk = wtile + (size_t)kb * (BK * WTr::bits / 8);
#pragma unroll
    for (int i = 0; i < XC; ++i) r.x[i] = x4_raw<XT>(xtile, xk + i * xstep + xlane);
#pragma unroll
    for (int i = 0; i < WC; ++i) r.w[i] = *reinterpret_cast<const u32x4*>(wk + i * wstep + wlane);
  };
  // staging units u in [u0, u1): x chunks first, then W chunks
  auto stage_units = [&](const Regs& r, uint8_t* S, int u0, int u1) {
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      if (u < u0 || u >= u1) continue;
      if (u < XC) {
        const xl_u32x2 pr = x4_bf16<XT>(r.x[u]);
        *reinterpret_cast<u32x2*>(S + xdst0 + u * XDST_STEP) = u32x2{pr[0], pr[1]};
      } else {
        const int i = u - XC;
        uint32_t words[WTr::words];
        decode_chunk<WT>(r.w[i], words);
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
  // One K block: fetch block kb+PF into `rf` (free: its previous block is
  // already in LDS), multiply the LDS buffer of block kb, and convert block
  // kb+1 from `rs` into the other buffer after MFMA steps 1..3.  Past the end
  // the last block is fetched and staged again into the idle buffer, so the
  // body has no branch.
  auto body = [&](int kb, Regs& rf, const Regs& rs) {
    const uint8_t* S = lds + (kb & 1) * STAGE;
    uint8_t* Snext = lds + ((kb + 1) & 1) * STAGE;
    fetch(rf, min(kb + PF, kblocks - 1));
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
      if (s >= 1) stage_units(rs, Snext, (s - 1) * UNITS / 3, s * UNITS / 3);
    }
    __syncthreads();
  };

  Regs r0, r1, r2;
  fetch(r0, 0);
  if constexpr (PF >= 2) fetch(r1, min(1, kblocks - 1));
  if constexpr (PF >= 3) fetch(r2, min(2, kblocks - 1));
  stage_units(r0, lds, 0, UNITS);
  __syncthreads();
  if constexpr (PF == 1) {
    for (int kb = 0; kb < kblocks; ++kb) body(kb, r0, r0);
  } else if constexpr (PF == 2) {
    for (int kb = 0; kb < kblocks; kb += 2) {
      body(kb, r0, r1);
      if (kb + 1 < kblocks) body(kb + 1, r1, r0);
    }
  } else {
    for (int kb = 0; kb < kblocks; kb += 3) {
      body(kb, r0, r1);
      if (kb + 1 < kblocks) body(kb + 1, r1, r2);
      if (kb + 2 < kblocks) body(kb + 2, r2, r0);
    }
  }

  tile_epilogue(ep, acc, product_scale(w_scale, x_scale), y, N, m0 + wm, n0 + wn, lane);
}

// ---------------------------------------------------------------------------
// Wide-K kernel (dispatched for E2M1 weights; it also handles FP8, which the
// ping-pong kernel below takes; K % 128 == 0): K blocks of 128, so one K
// block of a W row is a whole 128-byte line for FP8 (64 bytes for E2M1) and
// each W load fetches no line it uses only half of; barriers are
// half as many.  W stays in its stored format in LDS (decoded per fragment),
// x is rounded to bf16 on the way in; two LDS stages, two register sets
// (block kb+2 is loaded while block kb+1 is staged).

template <int WT>
struct Wide {
  static constexpr int KB = 128;                        // K per block
  static constexpr int bits = dtype_bits(WT);
  static constexpr int row_bytes = KB * bits / 8;       // W bytes per row per block
  static constexpr int pitch = bits == 8 ? 136 : 68;    // W LDS row pitch (bytes)
  static constexpr int a_pitch = KB + 8;                // bf16 per x row in LDS
  static constexpr int frag_bytes = 8 * bits / 8;
  static constexpr int cpr = row_bytes / 16;            // W 16-byte chunks per row
};

template <int WT, int XT>
__global__ __launch_bounds__(512, 1) void linear_wide_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale,
    Epilogue ep, void* __restrict__ y, int M, int N, int K, int tiles_m,
    int tiles_n) {
  using F = Wide<WT>;
  constexpr int KB = F::KB;
  constexpr int FBN = 256, NTH = 512;
  constexpr int FWN = 64, FNT = 2;
  constexpr int A_ST = BM * F::a_pitch * 2;
  constexpr int B_ST = FBN * F::pitch;
  constexpr int STAGE = A_ST + B_ST;
  constexpr int XC = BM * KB / 4 / NTH;                 // 8 x chunks per thread
  constexpr int WC = FBN * F::row_bytes / 16 / NTH;     // 4 (FP8) or 2 (E2M1) W chunks
  constexpr int UNITS = XC + WC;
  constexpr int STEPS = KB / 16;
  static_assert(F::bits <= 8 && NTH % F::cpr == 0, "tile shape");
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

  // Global loads are buffer loads through per-tile descriptors: a 32-bit
  // per-lane byte offset in one VGPR, block and chunk offsets in SGPRs.
  // x: 32 chunks (512 B) per row, 16 rows per pass of the workgroup;
  // W: cpr chunks per row, NTH / cpr rows per pass.
  constexpr int XB = XL<XT>::bytes;
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(x + (size_t)m0 * K * XB), (short)0, BM * K * XB, 0x00020000);
  const uint32_t xlane = (uint32_t)((tid >> 5) * K + (tid & 31) * 4) * (uint32_t)XB;
  const uint32_t xstep = 16u * (uint32_t)K * (uint32_t)XB;
  const uint32_t w_row_bytes = (uint32_t)K * F::bits / 8;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(w + (size_t)n0 * w_row_bytes), (short)0, (int)(FBN * w_row_bytes),
      0x00020000);
  const uint32_t wlane = (uint32_t)(tid / F::cpr) * w_row_bytes + (uint32_t)(tid % F::cpr) * 16u;
  const uint32_t wstep = (uint32_t)(NTH / F::cpr) * w_row_bytes;

  // LDS: [A0 | A1 | B0 | B1].  Per-lane bases below; every other offset is a
  // compile-time constant that fits a ds instruction's 16-bit offset field.
  constexpr int XDST_STEP = 16 * F::a_pitch * 2;
  constexpr int WDST_STEP = (NTH / F::cpr) * F::pitch;
  constexpr int A_ROWS32 = 32 * F::a_pitch * 2;
  const int xw = ((tid >> 5) * F::a_pitch + (tid & 31) * 4) * 2;
  const int ww0 = 2 * A_ST + (tid / F::cpr) * F::pitch + (tid % F::cpr) * 16;
  const int ww1 = ww0 + B_ST;
  const int ar = ((wm + (lane & 31)) * F::a_pitch + half * 8) * 2;
  const int br0 = 2 * A_ST + (wn + (lane & 31)) * F::pitch + half * F::frag_bytes;
  const int br1 = br0 + B_ST;
  // B fragment offsets: per 32-column sub-tile and per 16-K step
  constexpr int BJ = 32 * F::pitch;
  constexpr int BSTEP = 2 * F::frag_bytes;
  auto bfrag = [](const uint8_t* p) { return frag_to_bf16<WT>(p); };

  struct Regs {
    u32x4 x[XC];
    u32x4 w[WC];
  };
  auto fetch = [&](Regs& r, int kb) {
    const uint32_t xk = (uint32_t)kb * (KB * XB);
    const uint32_t wk = (uint32_t)kb * F::row_bytes;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      if constexpr (XB == 4) {
        r.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xlane, xk + i * xstep, 0);
      } else if constexpr (XB == 2) {
        const xl_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(xrs, xlane, xk + i * xstep, 0);
        r.x[i] = u32x4{v[0], v[1], 0u, 0u};
      } else {
        r.x[i] = u32x4{__builtin_amdgcn_raw_buffer_load_b32(xrs, xlane, xk + i * xstep, 0), 0u,
                       0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < WC; ++i) r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wlane, wk + i * wstep, 0);
  };
  auto stage_units = [&](const Regs& r, const int BUF, int u0, int u1) {
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      if (u < u0 || u >= u1) continue;
      if (u < XC) {
        const xl_u32x2 pr = x4_bf16<XT>(r.x[u]);
        *reinterpret_cast<u32x2*>(lds + xw + BUF * A_ST + u * XDST_STEP) = u32x2{pr[0], pr[1]};
      } else {
        const int i = u - XC;
        uint8_t* d = lds + (BUF ? ww1 : ww0) + i * WDST_STEP;
        if constexpr (F::pitch % 8 == 0) {
          *reinterpret_cast<u32x2*>(d) = u32x2{r.w[i][0], r.w[i][1]};
          *reinterpret_cast<u32x2*>(d + 8) = u32x2{r.w[i][2], r.w[i][3]};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t*>(d + 4 * q) = r.w[i][q];
        }
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

  const int kblocks = K / KB;
  // Block kb in buffer BUF: fetch block kb+2 into `rf` (its block kb is in
  // LDS already), multiply, and stage block kb+1 from `rs` into buffer BUF^1
  // after MFMA steps 1..6.  Past the end the last block is fetched and staged
  // again into the idle buffer, so the body has no branch.
  auto body = [&](int kb, const int BUF, Regs& rf, const Regs& rs) {
    const uint8_t* SA = lds + ar + BUF * A_ST;
    const uint8_t* SB = lds + (BUF ? br1 : br0);
    fetch(rf, min(kb + 2, kblocks - 1));
    bf16x8 a[2][MT], b[2][FNT];
#pragma unroll
    for (int i = 0; i < MT; ++i) a[0][i] = *reinterpret_cast<const bf16x8*>(SA + i * A_ROWS32);
#pragma unroll
    for (int j = 0; j < FNT; ++j) b[0][j] = bfrag(SB + j * BJ);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < STEPS) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
          a[nxt][i] = *reinterpret_cast<const bf16x8*>(SA + i * A_ROWS32 + (s + 1) * 32);
#pragma unroll
        for (int j = 0; j < FNT; ++j)
          b[nxt][j] = bfrag(SB + j * BJ + (s + 1) * BSTEP);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < FNT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[cur][i], b[cur][j], acc[i][j], 0, 0, 0);
      if (s >= 1 && s <= 6) stage_units(rs, BUF ^ 1, (s - 1) * UNITS / 6, s * UNITS / 6);
    }
    __syncthreads();
  };

  Regs r0, r1;
  fetch(r0, 0);
  fetch(r1, min(1, kblocks - 1));
  stage_units(r0, 0, 0, UNITS);
  __syncthreads();
  for (int kb = 0; kb < kblocks; kb += 2) {
    body(kb, 0, r0, r1);
    if (kb + 1 < kblocks) body(kb + 1, 1, r1, r0);
  }

  tile_epilogue(ep, acc, product_scale(w_scale, x_scale), y, N, m0 + wm, n0 + wn, lane);
}

// ---------------------------------------------------------------------------
// Ping-pong kernel (E4M3 / E5M2 weights, x in fp32 / bf16 / f16, M % 128,
// N % 256, K % 128): the wide kernel's 128 x 256 tile and 64 x 64 wave tiles,
// scheduled so that the matrix cores are not idle while operands move.  The
// 8 waves form two groups of 4 (rows 0-63 and 64-127 of the tile); waves w
// and w + 4 share a SIMD.  Every wave runs the same program of phases
// separated by workgroup barriers -- per K block of 128: M0 (read the
// fragments of K 0-63, stage half of the next block), C0 (16 MFMAs), M1 (the
// fragments of K 64-127, the other half), C1 -- and group 1 passes one extra
// barrier first, so it runs one phase behind group 0: while one wave of a
// SIMD multiplies, the other reads LDS and issues loads.
//
// x: each group loads its own 64 rows into registers (two register sets, so a
// block's loads are issued two blocks before it is staged) and rounds them to
// bf16 into padded LDS rows.  W: group 0 copies each block straight into LDS
// with buffer_load ... lds, in two K halves of 256 rows x 64 bytes whose
// 16-byte chunks are XOR-swizzled by row (chunk c of row r at slot
// c ^ ((r / 4) % 4): the 16 rows one fragment read serves per LDS cycle hit
// distinct banks).  A lane's B fragment for two consecutive 16-K MFMA steps
// is one 16-byte read: lane half h holds K [16 h, 16 h + 16) of a 32-K pair,
// and the x fragments follow the same K order (MFMA step u of the pair takes
// K 16 h + 8 u .. + 7 in both operands).  Synchronisation: s_waitcnt
// lgkmcnt(0) then s_barrier at every phase end; after each multiply phase
// s_waitcnt vmcnt(12) -- group 0's copy of the previous memory phase has
// landed (the x loads issued after it may still be in flight).
//
// WN: W in its natural [K][N] layout (the Linear backward's grad_input =
// grad @ W on the forward's codes): a K half is 64 rows of the tile's 256
// columns, chunk c of row r at slot c ^ (2 (r % 8)), and B fragments come
// from gfx950's transposing read (8 consecutive K of one column per lane; the
// 32 lanes of a half-wave read 8 rows x 32 bytes, all in distinct banks) in
// the MFMA's own K order, which the x fragments then follow.

template <int WT, int XT, bool WN = false>
__global__ __launch_bounds__(512, 1) void linear_pingpong_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale, const uint8_t* __restrict__ w,
    const float* __restrict__ w_scale, Epilogue ep, void* __restrict__ y, int M, int N, int K,
    int tiles_m, int tiles_n) {
  static_assert(WT == E4M3 || WT == E5M2, "FP8 weights");
  constexpr int KB = 128, FBN = 256, FNT = 2;
  constexpr int XB = XL<XT>::bytes;
  static_assert(XB == 4 || XB == 2, "x in fp32 or a 16-bit format");
  constexpr int XP = 2 * KB + 16;     // bytes per bf16 x row in LDS
  constexpr int XS = BM * XP;         // x stage
  constexpr int WS = FBN * KB;        // W stage: two K halves of 256 rows x 64 bytes
  constexpr int WH = WS / 2;
  constexpr int WOFF = 2 * XS;
  // x moves in 16-byte chunks (4 fp32 or 8 16-bit elements): RL lanes cover
  // a row's 128 K, a pass of the group's 256 lanes 256 / RL rows, and each
  // lane holds XC chunks of a block (fp32: 32 lanes a row, 8 chunks; 16-bit:
  // 16 lanes a row, 4 chunks, so half the load and LDS-write instructions)
  constexpr int EPC = 16 / XB;        // elements per chunk
  constexpr int RL = KB / EPC;        // lanes per row
  constexpr int RP = 256 / RL;        // rows per pass
  constexpr int XC = 64 / RP;         // x chunks per lane per block
  static_assert(XC % 2 == 0, "x chunks split over the two memory phases");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * XS + 2 * WS];

  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((T & 7) == 0) t = (t & 7) * (T >> 3) + (t >> 3);
  constexpr int GM = 4;
  const int grp = t / (GM * tiles_n);
  const int first_m = grp * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int rem = t - grp * GM * tiles_n;
  const int m0 = (first_m + rem % gm) * BM;
  const int n0 = (rem / gm) * FBN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = wave >> 2, q = wave & 3;
  const int wm = g * 64, wn = q * 64;
  const int gt = tid & 255;
  const int la = lane & 31, h = lane >> 5;

  // x: the group's 64 rows, RP rows of 16-byte chunks per pass of its lanes
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(x + (size_t)(m0 + wm) * K * XB), (short)0, 64 * K * XB, 0x00020000);
  const uint32_t xlane = (uint32_t)((gt / RL) * K + (gt % RL) * EPC) * (uint32_t)XB;
  const uint32_t xstep = (uint32_t)RP * (uint32_t)K * (uint32_t)XB;
  const int xw = (wm + gt / RL) * XP + (gt % RL) * EPC * 2;

  // W: instruction j (= 4 i + q for wave q) of a K half fills LDS slots
  // 64 j + lane: row 16 j + lane / 4, slot lane % 4, holding that row's chunk
  // (lane % 4) ^ ((lane / 16) % 4) of the half.  WN: row 4 j + lane / 16 of
  // the half's 64, slot lane % 16, holding column chunk
  // (lane % 16) ^ (2 (row % 8)), row % 8 = 4 (q % 2) + lane / 16.
  const __amdgpu_buffer_rsrc_t wrs =
      WN ? __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w + n0), (short)0,
                                             (int)((size_t)K * N - n0), 0x00020000)
         : __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w + (size_t)n0 * K), (short)0,
                                             FBN * K, 0x00020000);
  const uint32_t wlane =
      WN ? (uint32_t)((lane >> 4) * N + (((lane & 15) ^ (2 * (4 * (q & 1) + (lane >> 4)))) << 4))
         : (uint32_t)((lane >> 2) * K + (((lane & 3) ^ (lane >> 4)) << 4));

  // fragment bases: A row wm + la (+ 32 i), bytes 32 h (+ 64 t + 16 u) of
  // the row; B row wn + la (+ 32 j), chunk 2 t + h of the K half at slot
  // (2 t + h) ^ ((la / 4) % 4), so step t only flips address bit 5.  WN: A
  // bytes 16 h (+ 64 t + 32 u); B rows 8 h + (lane % 16) / 2 (+ 16 (2 t + u))
  // of the half, column chunk 4 q + (lane / 16) % 2 (+ 2 j), 8 (lane % 2)
  // bytes in, so sub-tile j only flips address bit 5.
  const int abase = (wm + la) * XP + (WN ? 16 : 32) * h;
  const int bx = (lane & 15) >> 1;
  const int bbase =
      WN ? WOFF + (8 * h + bx) * 256 + (((4 * q + ((lane >> 4) & 1)) ^ (2 * bx)) << 4) + 8 * (lane & 1)
         : WOFF + (wn + la) * 64 + ((h ^ ((la >> 2) & 3)) << 4);

  const int nb = K / KB;
  u32x4 xr[2][XC];
  bf16x8 fa[2][2][MT];  // [32-K pair][step][M tile]
  u32x4 fb[2][FNT];     // [32-K pair][N tile]: 16 codes (WN: 8 per 16-K step)
  f32x16 acc[MT][FNT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < FNT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

  auto fetch_x = [&](u32x4 (&xs)[XC], int kb, const int i0, const int i1) {
    const uint32_t xk = (uint32_t)kb * (KB * XB);
#pragma unroll
    for (int i = i0; i < i1; ++i)
      xs[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xlane, xk + i * xstep, 0);
  };
  auto stage_x = [&](const u32x4 (&xs)[XC], int slot, const int i0, const int i1) {
    uint8_t* d = lds + slot * XS + xw;
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      if constexpr (XB == 4) {
        const xl_u32x2 pr = x4_bf16<XT>(xs[i]);
        *reinterpret_cast<u32x2*>(d + i * RP * XP) = u32x2{pr[0], pr[1]};
      } else {
        const xl_u32x2 lo = x4_bf16<XT>(xs[i]);
        const xl_u32x2 hi = x4_bf16<XT>(u32x4{xs[i][2], xs[i][3], 0u, 0u});
        *reinterpret_cast<u32x4*>(d + i * RP * XP) = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    }
  };
  auto copy_w = [&](int kb, int slot, const int hf) {
    typedef __attribute__((address_space(3))) void lds_void;
    uint8_t* d = lds + WOFF + slot * WS + hf * WH;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * i + q;
      const uint32_t so = WN ? (uint32_t)(kb * KB + 64 * hf + 4 * j) * (uint32_t)N
                             : (uint32_t)(16 * j) * (uint32_t)K + (uint32_t)kb * KB + 64u * hf;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void*)(d + j * 64 * 16), 16, wlane, so,
                                               0, 0);
    }
  };
  auto read_frags = [&](int kb, const int hf) {
    const uint8_t* sa = lds + (kb & 1) * XS + abase;
    const int sb = bbase + (kb & 1) * WS + hf * WH;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int t4 = 2 * hf + tt;
#pragma unroll
      for (int j = 0; j < FNT; ++j) {
        if constexpr (WN) {
          typedef __attribute__((address_space(3))) i32x2_lds lds_i32x2;
          const i32x2_lds r0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (lds_i32x2*)(lds + ((sb + 16 * (2 * tt) * 256) ^ (j << 5))));
          const i32x2_lds r1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (lds_i32x2*)(lds + ((sb + 16 * (2 * tt + 1) * 256) ^ (j << 5))));
          fb[tt][j] = u32x4{(uint32_t)r0[0], (uint32_t)r0[1], (uint32_t)r1[0], (uint32_t)r1[1]};
        } else {
          fb[tt][j] = *reinterpret_cast<const u32x4*>(lds + ((sb + j * 32 * 64) ^ (tt << 5)));
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < MT; ++i)
          fa[tt][u][i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * XP + 64 * t4 +
                                                          (WN ? 32 : 16) * u);
    }
  };
  auto dec = [](uint32_t w0, uint32_t w1) {
    uint32_t o[4];
    if constexpr (WT == E4M3) {
      o[0] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false));
      o[1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true));
      o[2] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false));
      o[3] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true));
    } else {
      o[0] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w0, 1.0f, false));
      o[1] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w0, 1.0f, true));
      o[2] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w1, 1.0f, false));
      o[3] = bf16_pair(__builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w1, 1.0f, true));
    }
    return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
  };
  auto multiply = [&]() {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        bf16x8 bb[FNT];
#pragma unroll
        for (int j = 0; j < FNT; ++j) bb[j] = dec(fb[tt][j][2 * u], fb[tt][j][2 * u + 1]);
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < FNT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[tt][u][i], bb[j], acc[i][j], 0, 0, 0);
      }
  };
  auto bar = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // Memory phase hf of block kb: its fragments of K half hf; group 0 copies
  // K half hf of block kb+1's W; half the x chunks of block kb+1 are staged
  // from register set (kb+1) % 2 and that set's loads for block kb+3 issued.
  // Past the last block the last one is copied and staged again into the
  // idle slot, so the loop has no tail.
  constexpr int XH = XC / 2;  // x chunks staged and loaded per memory phase
  auto mem = [&](u32x4 (&xs)[XC], int kb, const int hf) {
    read_frags(kb, hf);
    if (g == 0) copy_w(min(kb + 1, nb - 1), (kb + 1) & 1, hf);
    stage_x(xs, (kb + 1) & 1, XH * hf, XH * hf + XH);
    fetch_x(xs, min(kb + 3, nb - 1), XH * hf, XH * hf + XH);
  };
  // after a multiply phase: group 0's W copy of the memory phase before it
  // has landed (4 copies and XH x loads per memory phase, in that order: the
  // last phase's loads and copies and the phase before's x loads may still
  // be in flight)
  auto wait_copy = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 + 2 * XH) : "memory");
  };
  auto block = [&](u32x4 (&xs)[XC], int b) {
    mem(xs, b, 0);
    bar();
    multiply();  // C0(b)
    wait_copy();
    bar();
    mem(xs, b, 1);
    bar();
    multiply();  // C1(b)
    wait_copy();
    bar();
  };

  // Prologue: block 0 staged and its W copied, blocks 1 and 2 loaded.
  fetch_x(xr[0], 0, 0, XC);
  if (g == 0) {
    copy_w(0, 0, 0);
    copy_w(0, 0, 1);
  }
  stage_x(xr[0], 0, 0, XC);
  fetch_x(xr[1], min(1, nb - 1), 0, XC);
  fetch_x(xr[0], min(2, nb - 1), 0, XC);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * XC) : "memory");  // block 0's W copies
  bar();
  if (g == 1) bar();  // group 1 runs one phase behind
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    block(xr[1], b);
    block(xr[0], b + 1);
  }
  if (b < nb) block(xr[1], b);
  if (g == 0) bar();  // both groups pass the same number of barriers
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  tile_epilogue(ep, acc, product_scale(w_scale, x_scale), y, N, m0 + wm, n0 + wn, lane);
}

// ---------------------------------------------------------------------------
// FP8 product for x stored as E4M3 / E5M2 (the narrow activations a fused
// epilogue writes) with E4M3 / E5M2 / E2M1 weights; M % 128, N % 256,
// K % 128.  gfx950's v_mfma_f32_32x32x64_f8f6f4 takes both operands' codes
// as they are stored: every product is exact and sums in fp32, and the
// per-tensor scales s_x * s_w are applied in the epilogue, as on the other
// paths.  The MFMA runs FP8 at over twice the bf16 rate under the chip's
// power limit, and nothing is converted per fragment.
//
// The kernel keeps the 128 x 256 tile and 8 waves (2 x 4, 64 x 64 per wave)
// of the wide kernel.  x and W go from HBM straight into LDS with
// global_load_lds_dwordx4 (no staging registers) through a ring of 3 stages
// of 128 K (x 16 KB + W 32 / 16 KB each: whole 128-byte lines), each issued
// 2 stages ahead.  Rows are stored in 16-byte chunks XOR-swizzled by row so
// the 16 rows one fragment read touches per LDS cycle fall in distinct
// banks; a wave's load writes 64 consecutive chunk slots and each lane
// fetches the global chunk that belongs in its slot.  The operands' lane
// halves hold the K ranges the instruction pairs up (F8::x_chunk).  Fragments
// are read one 64-K step ahead of the MFMAs that use them.  Synchronisation:
// s_waitcnt vmcnt (this wave's loads of the next stage have landed) and
// lgkmcnt (its fragment reads are done), then s_barrier (every wave's loads
// have, and every wave is done with the slot the next load overwrites).

template <int WT, int XT>
struct F8 {
  static_assert(XT == E4M3 || XT == E5M2, "x codes feed the FP8 MFMA as stored");
  static constexpr int KS = 128;                         // K per stage: whole 128-byte lines
  static constexpr int w_row = KS * dtype_bits(WT) / 8;  // 128 (FP8) or 64 (E2M1)
  static constexpr int w_chunks = w_row / 16;            // 8 or 4
  static constexpr int x_bytes = BM * KS;                // 128 rows x 128 B
  static constexpr int w_bytes = 256 * w_row;
  static constexpr int stage = x_bytes + w_bytes;         // 48 KB (FP8 W) or 32 KB (E2M1)
  static constexpr int NS = 150 * 1024 / stage >= 3 ? 3 : 2;
  static constexpr int X_PER = BM * 8 / 512;              // x loads per lane per stage
  static constexpr int W_PER = 256 * w_chunks / 512;      // W loads per lane per stage
  static constexpr int L = X_PER + W_PER;                 // loads per lane per stage
  static constexpr int lds = NS * stage;
  static constexpr int fmt = WT == E4M3 ? 0 : WT == E5M2 ? 1 : 4;  // f8f6f4 format codes
  static constexpr int fmt_x = XT == E5M2 ? 1 : 0;
  // The instruction's K order within a 64-K step: an FP8 operand's lane half
  // h holds K [32h, 32h + 32); an E2M1 operand's holds K [16h, 16h + 16) then
  // [32 + 16h, 32 + 16h + 16).  W keeps its order (in step s, lane half h
  // reads chunk 2s + h for E2M1, chunks 4s + 2h and 4s + 2h + 1 for FP8), so
  // the x operand's two 16-byte chunks u = 0, 1 are chunks 4s + 2h + u
  // against FP8 W and 4s + h + 2u against E2M1 W.
  __device__ static constexpr int x_chunk(int s, int h, int u) {
    return 4 * s + (w_chunks == 8 ? 2 * h + u : h + 2 * u);
  }
  __device__ static constexpr int w_chunk(int s, int h, int u) {
    return w_chunks == 8 ? 4 * s + 2 * h + u : 2 * s + h;
  }
  // chunk c of row r sits at slot c ^ swz(r): the 16 rows one fragment read
  // touches per LDS cycle fall in distinct banks
  __device__ static constexpr int swz_x(int r) { return (r >> 1) & 7; }
  __device__ static constexpr int swz_w(int r) {
    return w_chunks == 8 ? ((r >> 1) & 7) : ((r >> 2) & 3);
  }
};

typedef int i32x8 __attribute__((ext_vector_type(8)));

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (lds is wave-uniform).  A plain device function: inside a kernel template
// the builtin's host-side checks would drop the kernel's host stub.
__device__ __forceinline__ void lds_dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

template <int WT, int XT>
__global__ __launch_bounds__(512, 1) void linear_f8_kernel(
    const uint8_t* __restrict__ x, const float* __restrict__ x_scale,
    const uint8_t* __restrict__ w, const float* __restrict__ w_scale, Epilogue ep,
    void* __restrict__ y, int M, int N, int K, int tiles_m, int tiles_n) {
  using D = F8<WT, XT>;
  constexpr int NS = D::NS, FBN = 256, FWN = 64, FNT = 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t dl[];

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

  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave & 1) * WM, wn = (wave >> 1) * FWN;

  // this lane's load sources (stage 0): slot q = i * 512 + tid of x or W,
  // row q / chunks
  const size_t w_row_bytes = (size_t)K * dtype_bits(WT) / 8;
  const uint8_t* xsrc[D::X_PER];
#pragma unroll
  for (int i = 0; i < D::X_PER; ++i) {
    const int q = i * 512 + tid, r = q >> 3, c = (q & 7) ^ D::swz_x(r);
    xsrc[i] = x + (size_t)(m0 + r) * K + c * 16;
  }
  const uint8_t* wsrc[D::W_PER];
#pragma unroll
  for (int i = 0; i < D::W_PER; ++i) {
    const int q = i * 512 + tid, r = q / D::w_chunks, c = (q % D::w_chunks) ^ D::swz_w(r);
    wsrc[i] = w + (size_t)(n0 + r) * w_row_bytes + c * 16;
  }
  const int kblocks = K / D::KS;
  auto issue = [&](int kb) {
    uint8_t* base = dl + (kb % NS) * D::stage + wave * 64 * 16;
    const size_t xk = (size_t)kb * D::KS, wk = (size_t)kb * D::w_row;
#pragma unroll
    for (int i = 0; i < D::X_PER; ++i) lds_dma16(xsrc[i] + xk, base + i * 512 * 16);
#pragma unroll
    for (int i = 0; i < D::W_PER; ++i)
      lds_dma16(wsrc[i] + wk, base + D::x_bytes + i * 512 * 16);
  };

  // fragment read offsets within a stage (bytes), per 64-K step; rows are
  // lane-fixed, so their swizzles are too
  const int ra = lane & 31;
  int xoff[2][MT][2], woff[2][FNT][2];
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
        xoff[st][i][u] =
            (wm + i * 32 + ra) * D::KS + ((D::x_chunk(st, half, u) ^ D::swz_x(ra)) << 4);
#pragma unroll
      for (int j = 0; j < FNT; ++j)
        woff[st][j][u] = D::x_bytes + (wn + j * 32 + ra) * D::w_row +
                         ((D::w_chunk(st, half, u) ^ D::swz_w(ra)) << 4);
    }

  f32x16 acc[MT][FNT];
#pragma unroll
  for (int a = 0; a < MT; ++a)
#pragma unroll
    for (int b = 0; b < FNT; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

  // one 64-K step's operands: x per M tile, W per N tile
  struct Frags {
    i32x8 a[MT];
    i32x8 b[FNT];
  };
  auto cat = [](const u32x4& p, const u32x4& q) {
    return __builtin_bit_cast(i32x8, (uint32_t __attribute__((ext_vector_type(8)))){
                                         p[0], p[1], p[2], p[3], q[0], q[1], q[2], q[3]});
  };
  auto read = [&](Frags& f, int kb, const int st) {
    const uint8_t* sb = dl + (kb % NS) * D::stage;
#pragma unroll
    for (int j = 0; j < FNT; ++j) {
      const u32x4 p = *reinterpret_cast<const u32x4*>(sb + woff[st][j][0]);
      u32x4 q = u32x4{0u, 0u, 0u, 0u};
      if constexpr (D::w_chunks == 8) q = *reinterpret_cast<const u32x4*>(sb + woff[st][j][1]);
      f.b[j] = cat(p, q);
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
      f.a[i] = cat(*reinterpret_cast<const u32x4*>(sb + xoff[st][i][0]),
                   *reinterpret_cast<const u32x4*>(sb + xoff[st][i][1]));
  };
  auto multiply = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < FNT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            f.a[i], f.b[j], acc[i][j], D::fmt_x, D::fmt, 0, 0, 0, 0);
  };
  // Wait until stage kb + 1 has landed (at most `ahead` later stages still
  // in flight) and this wave's fragment reads are done, then the barrier:
  // after it every wave's loads of stage kb + 1 are in LDS and every wave is
  // done reading stage kb, whose slot the next load may overwrite.
  auto wait_next = [&](int ahead) {
    if (NS == 3 && ahead >= 1)
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(D::L) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  // Stage kb in two 64-K steps: step 0's fragments were read one step
  // earlier; read step 1's and multiply step 0; then (wait for stage kb + 1,
  // barrier, refill stage kb's slot with stage kb + NS) read stage kb + 1's
  // step 0 and multiply step 1.  The loop runs while a next stage exists, so
  // its body has no branch around the reads (a join there costs a full LDS
  // wait).
  Frags f0, f1;
#pragma unroll
  for (int k = 0; k < NS; ++k)
    if (k < kblocks) issue(k);
  {
    const int ahead = min(NS - 1, kblocks - 1);  // stages in flight beyond stage 0
    if (ahead >= 2) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * D::L) : "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(D::L) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }
  read(f0, 0, 0);
  int kb = 0;
  for (; kb + 1 < kblocks; ++kb) {
    read(f1, kb, 1);
    multiply(f0);
    wait_next(min(NS - 2, kblocks - 2 - kb));
    if (kb + NS < kblocks) issue(kb + NS);
    read(f0, kb + 1, 0);
    multiply(f1);
  }
  read(f1, kb, 1);
  multiply(f0);
  multiply(f1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  tile_epilogue(ep, acc, product_scale(w_scale, x_scale), y, N, m0 + wm, n0 + wn, lane);
}

template <int WT, int XT>
int launch_f8(const uint8_t* x, const float* x_scale, int64_t M, int64_t K, const uint8_t* w,
              const float* w_scale, const Epilogue& ep, int64_t N, void* y, hipStream_t stream) {
  using D = F8<WT, XT>;
  static bool lds_raised = false;
  if (!lds_raised) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&linear_f8_kernel<WT, XT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, D::lds);
    if (e != hipSuccess) return hip_fail(e);
    lds_raised = true;
  }
  const int64_t tiles_m = M / BM, tiles_n = N / 256;
  hipLaunchKernelGGL((linear_f8_kernel<WT, XT>), dim3((unsigned)(tiles_m * tiles_n)), dim3(512),
                     D::lds, stream, x, x_scale, w, w_scale, ep, y, (int)M, (int)N, (int)K,
                     (int)tiles_m, (int)tiles_n);
  return check_launch();
}

template <int WT, int XT>
int launch(const uint8_t* x, const float* x_scale, int64_t M, int64_t K, const void* w,
           const float* w_scale, const Epilogue& ep, int64_t N, void* y, hipStream_t stream) {
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int64_t T = tiles_m * tiles_n;
  if (T > 0x7FFFFFFF || M > 0x7FFFFFFF || N > 0x7FFFFFFF || K > 0x7FFFFFFF) return NOVAQ_EINVAL;
  const auto* wq = static_cast<const uint8_t*>(w);
  const bool rows_whole = M % BM == 0 && K > 0;
  if constexpr (dtype_bits(WT) <= 8 && (XT == E4M3 || XT == E5M2)) {
    if (rows_whole && N % 256 == 0 && K % F8<WT, XT>::KS == 0)
      return launch_f8<WT, XT>(x, x_scale, M, K, wq, w_scale, ep, N, y, stream);
  }
  if constexpr ((WT == E4M3 || WT == E5M2) && XL<XT>::bytes >= 2) {
    // W tile (256 rows x K bytes) and x tile bytes must fit the buffer range
    if (rows_whole && N % 256 == 0 && K % 128 == 0 && K <= (1 << 21)) {
      hipLaunchKernelGGL((linear_pingpong_kernel<WT, XT>), dim3((unsigned)(tiles_m * (N / 256))),
                         dim3(512), 0, stream, x, x_scale, wq, w_scale, ep, y, (int)M, (int)N,
                         (int)K, (int)tiles_m, (int)(N / 256));
      return check_launch();
    }
  }
  if constexpr (WT == E2M1) {
    // tile byte sizes (BM * K * bytes(x) for x) must fit the 31-bit buffer range
    if (rows_whole && N % 256 == 0 && K % 128 == 0 && K <= (1 << 21)) {
      hipLaunchKernelGGL((linear_wide_kernel<WT, XT>), dim3((unsigned)(tiles_m * (N / 256))),
                         dim3(512), 0, stream, x, x_scale, wq, w_scale, ep, y, (int)M, (int)N,
                         (int)K, (int)tiles_m, (int)(N / 256));
      return check_launch();
    }
  }
  if constexpr (WT != F32) {
    if (rows_whole && N % 256 == 0 && K % BK == 0) {
      hipLaunchKernelGGL((linear_pipe_kernel<WT, XT, 256, 8, 1, 3>),
                         dim3((unsigned)(tiles_m * (N / 256))), dim3(512), 0, stream, x, x_scale,
                         wq, w_scale, ep, y, (int)M, (int)N, (int)K, (int)tiles_m, (int)(N / 256));
      return check_launch();
    }
    if (rows_whole && N % 128 == 0 && K % BK == 0) {
      hipLaunchKernelGGL((linear_pipe_kernel<WT, XT, 128, 4, 2, 2>),
                         dim3((unsigned)(tiles_m * (N / 128))), dim3(256), 0, stream, x, x_scale,
                         wq, w_scale, ep, y, (int)M, (int)N, (int)K, (int)tiles_m, (int)(N / 128));
      return check_launch();
    }
  }
  const int x_vec = (K % 4) == 0;
  const int w_vec = ((K * W<WT>::bits / 8) % 16) == 0 && (K * W<WT>::bits) % 8 == 0;
  hipLaunchKernelGGL((linear_kernel<WT, XT>), dim3((unsigned)T), dim3(THREADS), 0, stream, x,
                     x_scale, wq, w_scale, ep, y, (int)M, (int)N, (int)K, (int)tiles_m,
                     (int)tiles_n, x_vec, w_vec);
  return check_launch();
}

}  // namespace

// y[M, N] = x[M, K] @ (s * dec(W[K, N])) with W in its natural [K][N] layout
// (the Linear backward's grad_input = grad @ W on the forward's weight codes),
// FP8 codes only, M % 128, N % 256, K % 128; NOVAQ_ENOTSUP for anything else
// (the caller transposes W and uses the forward product instead).
template <int XT>
int linear_wn_launch_xt(const uint8_t* x, int64_t M, int64_t K, const void* w_q, int w_dtype,
                        const float* w_scale, const Epilogue& ep, int64_t N, void* y,
                        hipStream_t stream) {
  if (!linear_wn_supported(M, K, N, w_dtype)) return NOVAQ_ENOTSUP;
  const int64_t tiles_m = M / BM, tiles_n = N / 256;
  const auto* wq = static_cast<const uint8_t*>(w_q);
  if (w_dtype == E4M3)
    hipLaunchKernelGGL((linear_pingpong_kernel<E4M3, XT, true>),
                       dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, stream, x, nullptr, wq,
                       w_scale, ep, y, (int)M, (int)N, (int)K, (int)tiles_m, (int)tiles_n);
  else
    hipLaunchKernelGGL((linear_pingpong_kernel<E5M2, XT, true>),
                       dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, stream, x, nullptr, wq,
                       w_scale, ep, y, (int)M, (int)N, (int)K, (int)tiles_m, (int)tiles_n);
  return check_launch();
}

// The product for x stored as XT (one translation unit per XT instantiates it).
template <int XT>
int linear_launch_xt(const uint8_t* x, const float* x_scale, int64_t N, int64_t D_in,
                     const void* w_q, int w_dtype, const float* w_scale, const Epilogue& ep,
                     int64_t D_out, void* y, hipStream_t stream) {
  switch (w_dtype) {
    case E4M3: return launch<E4M3, XT>(x, x_scale, N, D_in, w_q, w_scale, ep, D_out, y, stream);
    case E5M2: return launch<E5M2, XT>(x, x_scale, N, D_in, w_q, w_scale, ep, D_out, y, stream);
    case E2M1: return launch<E2M1, XT>(x, x_scale, N, D_in, w_q, w_scale, ep, D_out, y, stream);
    case BF16: return launch<BF16, XT>(x, x_scale, N, D_in, w_q, w_scale, ep, D_out, y, stream);
    case F16: return launch<F16, XT>(x, x_scale, N, D_in, w_q, w_scale, ep, D_out, y, stream);
    case F32: return launch<F32, XT>(x, x_scale, N, D_in, w_q, w_scale, ep, D_out, y, stream);
    default: return NOVAQ_EDTYPE;
  }
}

}  // namespace novaq
