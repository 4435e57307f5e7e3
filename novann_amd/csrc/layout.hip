// Layout kernels for the backward products: 2-D transpose (with an optional
// fp32 -> bf16 / fp16 rounding on the way) and a column sum.
//
// Transpose: dst (cols x rows) = src (rows x cols)^T, both row-major.  A
// workgroup moves one 64 x 64 tile through LDS: every global load and store
// instruction of a wave covers 64 consecutive elements of one row.  Quantized
// codes are permuted, never re-encoded (E2M1: both sides nibble-packed along
// their rows, element 2i in the low nibble; a lane writes one byte, i.e. two
// consecutive elements of a destination row).  fp32 -> bf16 / fp16 rounds to
// nearest even with the same rules as the cast kernels.  Two shapes take
// 16-byte accesses instead: 8-bit codes with rows and cols multiples of 16
// (transpose_bytes_kernel) and fp32 -> bf16 / fp16 with rows % 8 == 0 and
// cols % 4 == 0 (transpose_round_kernel).
//
// Column sum: out[c] = sum over rows of x[r][c] in fp32, in a fixed order
// (each of 16 row slices summed in four interleaved row chains, the chains
// added in order, then the slices added in slice order), so repeated calls
// agree bit for bit.  A workgroup owns 64 columns (each wave load instruction
// reads 256 contiguous bytes of one row) and 16 waves split the rows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_colsum.h"
#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {
namespace {

constexpr int TILE = 64;
constexpr int TT = 256;  // threads per transpose workgroup

template <int DT>
__device__ __forceinline__ uint32_t load_code(const uint8_t* __restrict__ p, int64_t e) {
  if constexpr (dtype_bits(DT) == 32) return reinterpret_cast<const uint32_t*>(p)[e];
  else if constexpr (dtype_bits(DT) == 16) return reinterpret_cast<const uint16_t*>(p)[e];
  else if constexpr (dtype_bits(DT) == 8) return p[e];
  else return (p[e >> 1] >> ((e & 1) * 4)) & 0xFu;
}

template <int ST, int DT>
__device__ __forceinline__ uint32_t convert_code(uint32_t c) {
  if constexpr (ST == DT) return c;
  else if constexpr (DT == BF16) return enc_bf16(c);  // ST == F32
  else return enc_f16(c);                             // ST == F32, DT == F16
}

template <int ST, int DT>
__global__ __launch_bounds__(TT) void transpose_kernel(const uint8_t* __restrict__ src,
                                                       uint8_t* __restrict__ dst, int64_t rows,
                                                       int64_t cols) {
  __shared__ uint32_t tile[TILE][TILE + 1];
  const int64_t r0 = (int64_t)blockIdx.y * TILE, c0 = (int64_t)blockIdx.x * TILE;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < TILE / 4; ++k) {
    const int i = ty + 4 * k;
    const int64_t r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < rows && c < cols) ? load_code<ST>(src, r * cols + c) : 0u;
  }
  __syncthreads();
  if constexpr (DT == E2M1) {
    // lane tx < 32 writes destination elements (2tx, 2tx+1) of its row
#pragma unroll
    for (int k = 0; k < TILE / 4; ++k) {
      const int i = ty + 4 * k;  // destination row offset (source column)
      const int64_t c = c0 + i;
      if (tx >= TILE / 2 || c >= cols) continue;
      const int64_t r = r0 + 2 * tx;  // even; rows is even
      if (r >= rows) continue;
      const uint32_t lo = tile[2 * tx][i], hi = tile[2 * tx + 1][i];
      dst[(c * rows + r) >> 1] = (uint8_t)(lo | (hi << 4));
    }
  } else {
#pragma unroll
    for (int k = 0; k < TILE / 4; ++k) {
      const int i = ty + 4 * k;
      const int64_t c = c0 + i, r = r0 + tx;
      if (c >= cols || r >= rows) continue;
      const uint32_t v = convert_code<ST, DT>(tile[tx][i]);
      const int64_t e = c * rows + r;
      if constexpr (dtype_bits(DT) == 32) reinterpret_cast<uint32_t*>(dst)[e] = v;
      else if constexpr (dtype_bits(DT) == 16) reinterpret_cast<uint16_t*>(dst)[e] = (uint16_t)v;
      else dst[e] = (uint8_t)v;
    }
  }
}

// 8-bit codes with rows and cols multiples of 16: a workgroup moves a
// 128 x 128 byte tile.  Lane (rb, cb) loads 16 bytes of each of source rows
// 4rb .. 4rb+3 (a wave's load covers 8 rows x 128 contiguous bytes),
// transposes the 4 x 16 byte block in registers into 16 dwords (4 source
// rows of one source column each) and writes them to LDS as tile[col][rb];
// then 8 lanes per destination row write its 128 bytes with 16-byte stores.
// Rows and cols being multiples of 16 make every 16-byte access wholly in or
// out of range.
constexpr int TB = 128;            // tile edge in bytes
constexpr int TB_DW = TB / 4 + 1;  // LDS dwords per destination row (padded)

__global__ __launch_bounds__(TT) void transpose_bytes_kernel(const uint8_t* __restrict__ src,
                                                             uint8_t* __restrict__ dst,
                                                             int64_t rows, int64_t cols) {
  __shared__ uint32_t tile[TB][TB_DW];
  const int64_t r0 = (int64_t)blockIdx.y * TB, c0 = (int64_t)blockIdx.x * TB;
  const int t = threadIdx.x;
  const int rb = t >> 3, cb = t & 7;  // 4-row group, 16-byte column chunk
  uint4 a[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t r = r0 + 4 * rb + k, c = c0 + 16 * cb;
    a[k] = (r < rows && c < cols) ? *reinterpret_cast<const uint4*>(src + r * cols + c)
                                  : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t w0 = (&a[0].x)[d], w1 = (&a[1].x)[d], w2 = (&a[2].x)[d], w3 = (&a[3].x)[d];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // bytes j of the four rows' dwords: source column 16cb + 4d + j
      const uint32_t o = ((w0 >> (8 * j)) & 0xFFu) | (((w1 >> (8 * j)) & 0xFFu) << 8) |
                         (((w2 >> (8 * j)) & 0xFFu) << 16) | (((w3 >> (8 * j)) & 0xFFu) << 24);
      tile[16 * cb + 4 * d + j][rb] = o;
    }
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int oc = (t >> 3) + 32 * p, chunk = t & 7;  // destination row, 16-byte chunk
    const int64_t c = c0 + oc, r = r0 + 16 * chunk;
    if (c < cols && r < rows) {
      const uint32_t* q = &tile[oc][4 * chunk];
      *reinterpret_cast<uint4*>(dst + c * rows + r) = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
}

// fp32 -> bf16 / fp16 with rows a multiple of 8 and cols of 4: a workgroup
// moves a 64 x 64 tile.  Lane (rb, cb) loads 4 floats of each of source rows
// 4rb .. 4rb+3 (a wave's load covers 4 rows x 256 contiguous bytes), rounds
// them and writes each source column's 4 values as two packed dwords to LDS;
// then 8 lanes per destination row write its 128 bytes with 16-byte stores.
constexpr int TN = 64;                 // tile edge in elements
constexpr int TN_DW = TN / 2 + 1;      // LDS dwords per destination row (padded)

template <int DT>
__global__ __launch_bounds__(TT) void transpose_round_kernel(const float* __restrict__ src,
                                                             uint16_t* __restrict__ dst,
                                                             int64_t rows, int64_t cols) {
  __shared__ uint32_t tile[TN][TN_DW];
  const int64_t r0 = (int64_t)blockIdx.y * TN, c0 = (int64_t)blockIdx.x * TN;
  const int t = threadIdx.x;
  const int rb = t >> 4, cb = t & 15;  // 4-row group, 4-column chunk
  uint4 a[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t r = r0 + 4 * rb + k, c = c0 + 4 * cb;
    a[k] = (r < rows && c < cols) ? *reinterpret_cast<const uint4*>(src + r * cols + c)
                                  : make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) e[k] = convert_code<F32, DT>((&a[k].x)[j]);
    tile[4 * cb + j][2 * rb] = e[0] | (e[1] << 16);
    tile[4 * cb + j][2 * rb + 1] = e[2] | (e[3] << 16);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int oc = (t >> 3) + 32 * p, chunk = t & 7;  // destination row, 8-element chunk
    const int64_t c = c0 + oc, r = r0 + 8 * chunk;
    if (c < cols && r < rows) {
      const uint32_t* q = &tile[oc][4 * chunk];
      *reinterpret_cast<uint4*>(dst + c * rows + r) = make_uint4(q[0], q[1], q[2], q[3]);
    }
  }
}

// Column sums (the fixed summation order is novaq_colsum.h's).
__global__ __launch_bounds__(CS_COLS * CS_SLICES) void colsum_kernel(const float* __restrict__ x,
                                                                    int64_t rows, int64_t cols,
                                                                    float* __restrict__ out,
                                                                    int pt, int pco, int pc) {
  __shared__ float part[CS_SLICES][CS_COLS];
  colsum_block(x, rows, cols, out, pt, pco, pc, blockIdx.x, part);
}

template <int ST, int DT>
int launch_transpose(const void* src, void* dst, int64_t rows, int64_t cols, hipStream_t stream) {
  const int64_t gx = (cols + TILE - 1) / TILE, gy = (rows + TILE - 1) / TILE;
  if (gx > 0x7FFFFFFF || gy > 65535) return NOVAQ_EINVAL;
  hipLaunchKernelGGL((transpose_kernel<ST, DT>), dim3((unsigned)gx, (unsigned)gy), dim3(TT), 0,
                     stream, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), rows,
                     cols);
  return check_launch();
}

}  // namespace

int transpose_launch(const void* src, int st, int64_t rows, int64_t cols, void* dst, int dt,
                     hipStream_t stream) {
  if (rows == 0 || cols == 0) return NOVAQ_OK;
  if (st == dt) {
    if (dtype_bits(st) == 8 && rows % 16 == 0 && cols % 16 == 0) {
      const int64_t gx = (cols + TB - 1) / TB, gy = (rows + TB - 1) / TB;
      if (gx > 0x7FFFFFFF || gy > 65535) return NOVAQ_EINVAL;
      hipLaunchKernelGGL(transpose_bytes_kernel, dim3((unsigned)gx, (unsigned)gy), dim3(TT), 0,
                         stream, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst),
                         rows, cols);
      return check_launch();
    }
    switch (st) {
      case F32: return launch_transpose<F32, F32>(src, dst, rows, cols, stream);
      case F16: return launch_transpose<F16, F16>(src, dst, rows, cols, stream);
      case BF16: return launch_transpose<BF16, BF16>(src, dst, rows, cols, stream);
      case E4M3: return launch_transpose<E4M3, E4M3>(src, dst, rows, cols, stream);
      case E5M2: return launch_transpose<E5M2, E5M2>(src, dst, rows, cols, stream);
      case E2M1:
        if (rows % 2 || cols % 2) return NOVAQ_ESHAPE;
        return launch_transpose<E2M1, E2M1>(src, dst, rows, cols, stream);
      default: return NOVAQ_EDTYPE;
    }
  }
  if (st == F32 && (dt == BF16 || dt == F16) && rows % 8 == 0 && cols % 4 == 0) {
    const int64_t gx = (cols + TN - 1) / TN, gy = (rows + TN - 1) / TN;
    if (gx > 0x7FFFFFFF || gy > 65535) return NOVAQ_EINVAL;
    auto kern = dt == BF16 ? transpose_round_kernel<BF16> : transpose_round_kernel<F16>;
    hipLaunchKernelGGL(kern, dim3((unsigned)gx, (unsigned)gy), dim3(TT), 0, stream,
                       static_cast<const float*>(src), static_cast<uint16_t*>(dst), rows, cols);
    return check_launch();
  }
  if (st == F32 && dt == BF16) return launch_transpose<F32, BF16>(src, dst, rows, cols, stream);
  if (st == F32 && dt == F16) return launch_transpose<F32, F16>(src, dst, rows, cols, stream);
  return NOVAQ_EDTYPE;
}

int colsum_launch(const float* x, int64_t rows, int64_t cols, float* out, hipStream_t stream,
                  int pt, int pco, int pc) {
  if (cols == 0) return NOVAQ_OK;
  const int64_t blocks = (cols + CS_COLS - 1) / CS_COLS;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(colsum_kernel, dim3((unsigned)blocks), dim3(CS_COLS * CS_SLICES), 0, stream,
                     x, rows, cols, out, pt, pco, pc);
  return check_launch();
}

}  // namespace novaq
