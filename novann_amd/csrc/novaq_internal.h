// Internal glue shared by the kernel files and the C ABI (capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/novaq.h"

namespace novaq {

// Source index of padded position i (-1 .. n + pad) along an axis of length n
// under numpy.pad's index rules for NovaNN's padding modes
// (novann/functional.py:325-344): -1 where zeros mode pads a 0; edge
// (replicate) repeats the end element; wrap (circular) is i mod n; reflect
// mirrors without repeating the end element, period 2(n - 1), any width.
__device__ __forceinline__ int pad_index(int i, int n, int mode) {
  if (i >= 0 && i < n) return i;
  if (mode == NOVAQ_PAD_ZEROS) return -1;
  if (mode == NOVAQ_PAD_REPLICATE) return i < 0 ? 0 : n - 1;
  if (mode == NOVAQ_PAD_CIRCULAR) {
    const int r = i % n;
    return r < 0 ? r + n : r;
  }
  if (n == 1) return 0;  // reflect, period 2(n-1)
  const int p = 2 * (n - 1);
  int r = i % p;
  if (r < 0) r += p;
  return r >= n ? p - r : r;
}

// n / d for n < 2^31 by a multiply and a shift (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994): with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1, n / d =
// (mulhi(n, m) + n) >> l; the sum stays below 2^32 because n < 2^31.  The
// host works out (m, l) once per launch for a divisor d >= 1.
struct FastDiv {
  uint32_t m;
  int l;
};

inline FastDiv fast_div(uint32_t d) {
  FastDiv f;
  f.l = 0;
  while (((uint64_t)1 << f.l) < d) ++f.l;
  f.m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << f.l) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.l;
}

// Records a failed HIP call for novaq_last_hip_error() and maps it to a status.
int hip_fail(hipError_t e);

// Status of the most recent kernel launch on this thread.
inline int check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NOVAQ_OK : hip_fail(e);
}

// Compute units of the current device (cached per device).
int device_cu_count();

int cast_launch(const void* src, int st, void* dst, int dt, int64_t n, int smode,
                const float* scale, float* scale_out, hipStream_t stream);
int amax_launch(const void* x, int dt, int64_t n, float* amax, hipStream_t stream);
int scale_from_amax_launch(const float* amax, int dt, float* scale, hipStream_t stream);

struct Epilogue;  // novaq_epilogue.h

int linear_launch(const float* x, int64_t N, int64_t D_in, const void* w_q, int w_dtype,
                  const float* w_scale, const float* bias, int64_t D_out, float* y,
                  hipStream_t stream);
int linear_launch(const float* x, int64_t N, int64_t D_in, const void* w_q, int w_dtype,
                  const float* w_scale, const Epilogue& ep, int64_t D_out, void* y,
                  hipStream_t stream);
// x stored as x_dtype (F32, BF16, F16, E4M3, E5M2) with per-tensor scale x_scale (NULL = 1).
int linear_launch(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t D_in,
                  const void* w_q, int w_dtype, const float* w_scale, const Epilogue& ep,
                  int64_t D_out, void* y, hipStream_t stream);
// y[M, N] = x[M, K] @ (s * dec(W[K, N])) with W's codes in their natural
// [K][N] layout (no transposed copy): bf16 x, FP8 W, M % 128, N % 256,
// K % 128; NOVAQ_ENOTSUP otherwise.
inline bool linear_wn_supported(int64_t M, int64_t K, int64_t N, int w_dtype) {
  return (w_dtype == 3 || w_dtype == 4) && M > 0 && M % 128 == 0 && M <= 0x7FFFFFFF &&
         N > 0 && N % 256 == 0 && K > 0 && K % 128 == 0 && K <= (1 << 21) &&
         K * N < ((int64_t)1 << 31);
}
int linear_wn_launch(const void* x, int x_dtype, int64_t M, int64_t K, const void* w_q,
                     int w_dtype, const float* w_scale, const Epilogue& ep, int64_t N, void* y,
                     hipStream_t stream);
int conv2d_launch(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const void* w_q,
                  int w_dtype, const float* w_scale, int64_t C_out, int KH, int KW, int sh,
                  int sw, int ph, int pw, int pad_mode, const float* bias, float* y,
                  hipStream_t stream);
int conv2d_launch(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const void* w_q,
                  int w_dtype, const float* w_scale, int64_t C_out, int KH, int KW, int sh,
                  int sw, int ph, int pw, int pad_mode, const Epilogue& ep, void* y,
                  hipStream_t stream);
int conv2d_launch(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t C,
                  int64_t H, int64_t W, const void* w_q, int w_dtype, const float* w_scale,
                  int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode,
                  const Epilogue& ep, void* y, hipStream_t stream);

// One AdamW step of n fp32 weights (adamw.py:41-65); amax (optional) gets max |w|.
int adamw_launch(float* w, const float* g, float* m, float* v, int64_t n, double lr, double beta1,
                 double beta2, double eps, double weight_decay, int64_t step, int decay,
                 float* amax, hipStream_t stream);
// The same step on n float64 weights and moments, the gradient float32
// (g_f32) or float64, with numpy's promotion rules.
int adamw_f64_launch(double* w, const void* g, bool g_f32, double* m, double* v, int64_t n,
                     double lr, double beta1, double beta2, double eps, double weight_decay,
                     int64_t step, int decay, hipStream_t stream);

int max_pool2d_launch(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W,
                      int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode, void* y,
                      hipStream_t stream);
int global_avg_pool2d_launch(const void* x, int x_dtype, const float* x_scale, int64_t planes,
                             int64_t hw, float* y, hipStream_t stream);
int max_pool2d_backward_launch(const float* grad, const void* x, int x_dtype, int64_t N,
                               int64_t C, int64_t H, int64_t W, int KH, int KW, int sh, int sw,
                               int ph, int pw, int pad_mode, float* grad_input,
                               hipStream_t stream);
int global_avg_pool2d_backward_launch(const float* grad, int64_t planes, int64_t hw,
                                      float factor, float* grad_input, hipStream_t stream);

// col (C*KH*KW, N*OH*OW) fp32 = the conv2d column matrix of x in x_dtype
// (FP8 times *x_scale when given); pad modes resolved as pad_index does.
int im2col_launch(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t C,
                  int64_t H, int64_t W, int KH, int KW, int sh, int sw, int ph, int pw,
                  int pad_mode, float* col, hipStream_t stream);
// y (N, C, H + 2 ph, W + 2 pw) = x padded in pad_mode, codes copied as stored.
int pad2d_launch(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int ph,
                 int pw, int pad_mode, void* y, hipStream_t stream);

// Sets count 32-bit words at p to v (a kernel, so it may be captured in graphs).
int fill_u32_launch(uint32_t* p, uint32_t v, int count, hipStream_t stream);

int transpose_launch(const void* src, int st, int64_t rows, int64_t cols, void* dst, int dt,
                     hipStream_t stream);

// c[M, N] = sum over k of a[k, m] * b[k, n] (a: K x M, b: K x N, row-major
// fp32), both rounded to bf16, fp32 sums: the Linear weight gradient without
// transposed copies.  Shapes: M % 128, N % 256, K % 64, K * M and K * N
// fp32 bytes under 2 GiB.  colsum (optional): colsum[m] = sum over k of
// a[k, m] in fp32, in a fixed order.  a16 (optional): a rounded to bf16.
bool linear_tn_supported(int64_t M, int64_t N, int64_t K);
int linear_tn_launch(const float* a, const float* b, int64_t M, int64_t N, int64_t K, float* c,
                     float* colsum, uint16_t* a16, hipStream_t stream);

// Workspace parts of conv2d_backward_launch (byte offsets, 256-byte aligned):
// the flipped weights, the grad_weight partials (chunks x C_out x C*KH*KW
// fp32) and the grad_bias partials (chunks x C_out fp32).
struct ConvBwdWs {
  size_t wf, part, bpart, total;
  int chunks;
};
ConvBwdWs conv2d_bwd_workspace(int64_t N, int64_t C, int64_t C_out, int KH, int KW, int w_dtype,
                               int cus);
// Capacity of the static scratch the allocation-free Conv2d backward uses
// (novaq_conv2d_backward_noalloc): config [5] conv2 needs 30.8 MB.
constexpr size_t CONV_BWD_SCRATCH_BYTES = (size_t)32 << 20;
// The current device's address of that scratch (looked up on first use).
int conv2d_bwd_scratch(void** ptr);
int conv2d_backward_launch(const float* grad, const float* x, int64_t N, int64_t C, int64_t H,
                           int64_t W, const void* w_q, int w_dtype, const float* w_scale,
                           int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw,
                           int pad_mode, float* grad_input, float* grad_weight,
                           float* grad_bias, void* workspace, hipStream_t stream);
// out[c] = sum over r of x[r * cols + c] in a fixed order; with pt > 0 the
// columns form a (pt, pco, pc) array and column (t, co, c) goes to
// out[(co * pc + c) * pt + t].
int colsum_launch(const float* x, int64_t rows, int64_t cols, float* out, hipStream_t stream,
                  int pt = 0, int pco = 0, int pc = 0);

}  // namespace novaq
