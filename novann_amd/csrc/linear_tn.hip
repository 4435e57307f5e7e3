// The weight-gradient product of the Linear backward ("TN" GEMM) on bf16 MFMA:
//
//   C[M, N] = sum over k of A[k, m] * B[k, n]
//
// with A (K x M) and B (K x N) row-major -- grad (batch x D_out) and x (batch x
// D_in) as the backward receives them, so grad_weight = grad^T @ x
// (novann/layers/linear/linear.py:101) needs no transposed copies.  Both
// operands are rounded to bf16 (nearest even) while staged into LDS in their
// own K-major layout, and read into MFMA fragments with gfx950's transposing
// LDS read (ds_read_b64_tr_b16): within each group of 16 lanes, lane p names
// an 8-byte run of 4 elements (row p / 4, columns 4 (p % 4) .. +3 of a 4 x 16
// block), and lane i receives column i of that block -- 4 consecutive K of
// one M (or N) index, the half of a 32x32x16 MFMA fragment.  Products sum in
// fp32 (v_mfma_f32_32x32x16_bf16).
//
// Tiles of 256 x 256 (8 waves of 128 x 64, K blocks of 32) where M % 256,
// N % 256 and K % 32 are 0 and the tiles fill the GPU, else 128 x 256 (8 waves
// of 64 x 64, K blocks of 64); two LDS stages.
//
// With a16 non-null the kernel also stores A rounded to bf16 (K x M, the
// values it multiplies), each K block by one workgroup of the tile row (the
// one whose column index is the block index mod the tiles per row), for a
// later product on the same operand.
//
// With colsum non-null the workgroups of the first column of tiles also sum
// A's columns in fp32 (the bias gradient, grad summed over the batch:
// linear.py:103-104) from the values they stage: each thread adds its 4
// columns over the rows it loads (one residue class of rows modulo the rows
// per staging pass), in row order, and a column's partial sums are added in
// order of that residue at the end.  The rows per pass depend on the tile
// size the launch picks (256 x 256 tiles when they fill the device's CUs,
// else 128 x 256), so the sums are reproducible bit for bit per device and
// shape, not across devices with other CU counts or across shapes.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "linear_impl.h"

namespace novaq {
namespace {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// Tile configurations: BM x BN of C per workgroup of NW waves, each wave
// WM x WN, K blocks of KB rows.  LDS rows are padded by 64 bytes so a row
// pitch is 16 (mod 64) banks: the 8 rows one transposing read touches land in
// 4 disjoint bank ranges per 32 lanes.
template <int BM_, int BN_, int KB_, int NW_, int WM_, int WN_>
struct TnCfg {
  static constexpr int BM = BM_, BN = BN_, KB = KB_, NW = NW_, WM = WM_, WN = WN_;
  static constexpr int NTH = NW * 64;
  static constexpr int PA = (BM + 32) * 2, PB = (BN + 32) * 2;
  static constexpr int A_ST = KB * PA, B_ST = KB * PB, STAGE = A_ST + B_ST;
  static_assert((BM / WM) * (BN / WN) == NW, "wave grid");
};
// 8 waves of 64 x 64 on 128 x 256; 8 waves of 128 x 64 on 256 x 256 (half
// the tiles, 25% fewer LDS reads per MFMA; K blocks of 32 keep the staging
// registers within 256 VGPRs).
using Tn128 = TnCfg<128, 256, 64, 8, 64, 64>;
using Tn256 = TnCfg<256, 256, 32, 8, 128, 64>;

// 4 elements (8 bytes of LDS) transposed across each 16-lane group.
__device__ __forceinline__ bf16x4 tr_read(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)p);
}

// A 4-element chunk of an fp32 (16 bytes) or 16-bit (8 bytes) operand.
template <int XB>
__device__ __forceinline__ u32x4 load4(const __amdgpu_buffer_rsrc_t& rs, uint32_t lo, uint32_t so) {
  if constexpr (XB == 4) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, lo, so, 0);
  } else {
    const xl_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, lo, so, 0);
    return u32x4{v[0], v[1], 0u, 0u};
  }
}

template <int AT, int BT, class C>
__global__ __launch_bounds__(C::NTH, 1) void linear_tn_kernel(const uint8_t* __restrict__ a,
                                                           const uint8_t* __restrict__ b,
                                                           float* __restrict__ c,
                                                           float* __restrict__ colsum,
                                                           uint16_t* __restrict__ a16, int M,
                                                           int N, int K, int tiles_m,
                                                           int tiles_n) {
  constexpr int BM = C::BM, BN = C::BN, KB = C::KB, PA = C::PA, PB = C::PB;
  constexpr int A_ST = C::A_ST, STAGE = C::STAGE, NTH = C::NTH;
  constexpr int MT = C::WM / 32, NT = C::WN / 32;
  constexpr int AB = XL<AT>::bytes, BB = XL<BT>::bytes;
  constexpr int CA = BM / 4, CB = BN / 4;      // 4-element chunks per row
  constexpr int RA = NTH / CA, RB = NTH / CB;  // rows per pass of the workgroup
  constexpr int AC = KB * CA / NTH, BC = KB * CB / NTH;  // chunks per thread
  constexpr int UNITS = AC + BC, STEPS = KB / 16;
  static_assert(NTH % CA == 0 && NTH % CB == 0 && KB % RA == 0 && KB % RB == 0, "staging");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * STAGE];

  // Workgroups of one XCD (block id mod 8) take a compact group of tiles.
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

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int WGM = BM / C::WM;
  const int wm = (wave % WGM) * C::WM, wn = (wave / WGM) * C::WN;

  // Buffer loads over the whole operands (the host checks K * M and K * N
  // bytes fit 31 bits): a 4-element chunk per lane, row and K-block offsets in
  // SGPRs.
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(a), (short)0, K * M * AB, 0x00020000);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(b), (short)0, K * N * BB, 0x00020000);
  const uint32_t alane = (uint32_t)((tid / CA) * M + m0 + (tid % CA) * 4) * AB;
  const uint32_t blane = (uint32_t)((tid / CB) * N + n0 + (tid % CB) * 4) * BB;
  const uint32_t astep = (uint32_t)RA * (uint32_t)M * AB;
  const uint32_t bstep = (uint32_t)RB * (uint32_t)N * BB;

  // LDS: [A0 | B0 | A1 | B1], rows of K.
  const int aw = (tid / CA) * PA + (tid % CA) * 8;
  const int bw = A_ST + (tid / CB) * PB + (tid % CB) * 8;
  constexpr int AW_STEP = RA * PA, BW_STEP = RB * PB;
  // Fragment reads: lane l names row 8 (l / 32) + (l % 16) / 4 and column
  // 16 ((l / 16) % 2) + 4 (l % 4) of the 16 x 32 block it helps read; the
  // second read of a fragment is 4 rows further.
  const int rowoff = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int coloff = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int ar = rowoff * PA + (wm + coloff) * 2;
  const int br = A_ST + rowoff * PB + (wn + coloff) * 2;

  struct Regs {
    u32x4 a[AC];
    u32x4 b[BC];
  };
  auto fetch = [&](Regs& r, int kb) {
    const uint32_t ak = (uint32_t)kb * KB * (uint32_t)M * AB;
    const uint32_t bk = (uint32_t)kb * KB * (uint32_t)N * BB;
#pragma unroll
    for (int i = 0; i < AC; ++i)
      r.a[i] = load4<AB>(ars, alane, ak + i * astep);
#pragma unroll
    for (int i = 0; i < BC; ++i)
      r.b[i] = load4<BB>(brs, blane, bk + i * bstep);
  };
  const bool sums = colsum != nullptr && n0 == 0;
  float cs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int ntile = n0 / BN;
  // kbs: the index of the staged block, -1 when the last block is staged again.
  auto stage_units = [&](const Regs& r, const int BUF, int u0, int u1, int kbs) {
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      if (u < u0 || u >= u1) continue;
      if (u < AC) {
        if constexpr (AT == F32) {
          if (sums && kbs >= 0) {
            cs[0] += u2f(r.a[u][0]);
            cs[1] += u2f(r.a[u][1]);
            cs[2] += u2f(r.a[u][2]);
            cs[3] += u2f(r.a[u][3]);
          }
        }
        const xl_u32x2 p = x4_bf16<AT>(r.a[u]);
        *reinterpret_cast<u32x2*>(lds + BUF * STAGE + aw + u * AW_STEP) = u32x2{p[0], p[1]};
        if (a16 && kbs >= 0 && kbs % tiles_n == ntile) {
          const int64_t row = (int64_t)kbs * KB + tid / CA + RA * u;
          *reinterpret_cast<u32x2*>(a16 + row * M + m0 + (tid % CA) * 4) = u32x2{p[0], p[1]};
        }
      } else {
        const int i = u - AC;
        const xl_u32x2 p = x4_bf16<BT>(r.b[i]);
        *reinterpret_cast<u32x2*>(lds + BUF * STAGE + bw + i * BW_STEP) = u32x2{p[0], p[1]};
      }
    }
  };
  auto frag = [&](const uint8_t* p, int pitch) {
    const bf16x4 lo = tr_read(p), hi = tr_read(p + 4 * pitch);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int kblocks = K / KB;
  // Block kb in buffer BUF: fetch block kb+2 into `rf`, multiply, and stage
  // block kb+1 from `rs` into buffer BUF^1 over the steps; past the end the
  // last block is fetched and staged again into the idle buffer.
  auto body = [&](int kb, const int BUF, Regs& rf, const Regs& rs) {
    const uint8_t* SA = lds + BUF * STAGE + ar;
    const uint8_t* SB = lds + BUF * STAGE + br;
    fetch(rf, min(kb + 2, kblocks - 1));
    bf16x8 fa[2][MT], fb[2][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i) fa[0][i] = frag(SA + i * 64, PA);
#pragma unroll
    for (int j = 0; j < NT; ++j) fb[0][j] = frag(SB + j * 64, PB);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int cur = s & 1, nxt = cur ^ 1;
      if (s + 1 < STEPS) {
#pragma unroll
        for (int i = 0; i < MT; ++i) fa[nxt][i] = frag(SA + (s + 1) * 16 * PA + i * 64, PA);
#pragma unroll
        for (int j = 0; j < NT; ++j) fb[nxt][j] = frag(SB + (s + 1) * 16 * PB + j * 64, PB);
      }
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i][j],
                                                              0, 0, 0);
      stage_units(rs, BUF ^ 1, s * UNITS / STEPS, (s + 1) * UNITS / STEPS,
                  kb + 1 < kblocks ? kb + 1 : -1);
    }
    __syncthreads();
  };

  Regs r0, r1;
  fetch(r0, 0);
  fetch(r1, min(1, kblocks - 1));
  stage_units(r0, 0, 0, UNITS, 0);
  __syncthreads();
  for (int kb = 0; kb < kblocks; kb += 2) {
    body(kb, 0, r0, r1);
    if (kb + 1 < kblocks) body(kb + 1, 1, r1, r0);
  }

  if (sums) {
    // the last body ended with a barrier: LDS is free
    float* part = reinterpret_cast<float*>(lds);  // [RA][BM]
#pragma unroll
    for (int q = 0; q < 4; ++q) part[(tid / CA) * BM + (tid % CA) * 4 + q] = cs[q];
    __syncthreads();
    for (int col = tid; col < BM; col += NTH) {
      float v = part[col];
#pragma unroll
      for (int t = 1; t < RA; ++t) v += part[t * BM + col];
      colsum[m0 + col] = v;
    }
  }
  Epilogue ep{};
  ep.out_dtype = F32;
  tile_epilogue(ep, acc, 1.0f, c, N, m0 + wm, n0 + wn, lane);
}

}  // namespace

bool linear_tn_supported(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 && M % Tn128::BM == 0 && N % Tn128::BN == 0 &&
         K % Tn128::KB == 0 && K * M * 4 < ((int64_t)1 << 31) && K * N * 4 < ((int64_t)1 << 31);
}

int linear_tn_launch(const float* a, const float* b, int64_t M, int64_t N, int64_t K, float* c,
                     float* colsum, uint16_t* a16, hipStream_t stream) {
  if (!linear_tn_supported(M, N, K)) return NOVAQ_ESHAPE;
  const uint8_t* ap = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* bp = reinterpret_cast<const uint8_t*>(b);
  if (M % Tn256::BM == 0 && N % Tn256::BN == 0 && K % Tn256::KB == 0 &&
      (M / Tn256::BM) * (N / Tn256::BN) >= device_cu_count()) {
    const int tm = (int)(M / Tn256::BM), tn = (int)(N / Tn256::BN);
    hipLaunchKernelGGL((linear_tn_kernel<F32, F32, Tn256>), dim3((unsigned)(tm * tn)),
                       dim3(Tn256::NTH), 0, stream, ap, bp, c, colsum, a16, (int)M, (int)N, (int)K, tm,
                       tn);
  } else {
    const int tm = (int)(M / Tn128::BM), tn = (int)(N / Tn128::BN);
    hipLaunchKernelGGL((linear_tn_kernel<F32, F32, Tn128>), dim3((unsigned)(tm * tn)),
                       dim3(Tn128::NTH), 0, stream, ap, bp, c, colsum, a16, (int)M, (int)N, (int)K, tm,
                       tn);
  }
  return check_launch();
}

}  // namespace novaq
