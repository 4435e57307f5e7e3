// One workgroup's share of a column sum, shared by the column-sum kernel and
// the conv backward's finishing kernel.
//
// out[c] = sum over r of x[r * cols + c] in fp32 in a fixed order: each of
// SLICES row slices is summed in four chains (row r of a slice goes to chain
// r % 4, in row order), the chains are added (0 + 1) + (2 + 3), then the
// slices in slice order, so repeated calls with the same shape agree bit for
// bit.  A workgroup of COLS x SLICES lanes (1024, or 256) owns COLS columns:
// 64 by default (a wave's load reads 256 contiguous bytes of one row); 16
// with 64 slices for few columns over many rows (a quarter of the rows per
// lane), or 4 with 64 slices in a 256-lane workgroup -- the same slices, so
// the same sums bit for bit.  With pt > 0 the columns form a (pt, pco, pc) array and column (t, co, c)
// is stored at out[(co * pc + c) * pt + t].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace novaq {

constexpr int CS_COLS = 64;    // columns per workgroup
constexpr int CS_SLICES = 16;  // row slices per workgroup (one wave each)

// blk: the workgroup's column block; part: SLICES x COLS floats of LDS.
// Every lane of the workgroup calls it (it has a barrier).
template <int COLS = CS_COLS, int SLICES = CS_SLICES>
__device__ inline void colsum_block(const float* __restrict__ x, int64_t rows, int64_t cols,
                                    float* __restrict__ out, int pt, int pco, int pc,
                                    int64_t blk, float (*part)[COLS]) {
  static_assert(COLS * SLICES == 1024 || COLS * SLICES == 256, "a workgroup of 1024 or 256 lanes");
  const int tx = threadIdx.x % COLS, ty = threadIdx.x / COLS;
  const int64_t c = blk * COLS + tx;
  const int64_t per = (rows + SLICES - 1) / SLICES;
  const int64_t rb = ty * per, re = min(rows, rb + per);
  float s = 0.0f;
  if (c < cols) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int64_t r = rb;
    // unrolled by 4: 16 loads in flight per lane
#pragma unroll 4
    for (; r + 3 < re; r += 4) {
      a0 += x[r * cols + c];
      a1 += x[(r + 1) * cols + c];
      a2 += x[(r + 2) * cols + c];
      a3 += x[(r + 3) * cols + c];
    }
    for (; r < re; ++r) a0 += x[r * cols + c];
    s = (a0 + a1) + (a2 + a3);
  }
  part[ty][tx] = s;
  __syncthreads();
  if (ty == 0 && c < cols) {
    float t = part[0][tx];
#pragma unroll
    for (int k = 1; k < SLICES; ++k) t += part[k][tx];
    int64_t o = c;
    if (pt > 0) {
      const int64_t per_t = (int64_t)pco * pc;
      const int64_t tt = c / per_t, rest = c - tt * per_t;
      o = rest * pt + tt;  // rest = co * pc + c
    }
    out[o] = t;
  }
}

}  // namespace novaq
