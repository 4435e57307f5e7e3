// AdamW step on fp32 master weights, for gfx950 (restates AdamW.step,
// novann/optim/adamw.py:41-65), and the re-quantization that follows it.
//
// The reference's parameters and moments are float32 arrays and its
// hyper-parameters Python floats, so each of its numpy statements is one
// float32 operation with the scalar rounded to float32.  The kernel performs
// the same operations in the same order (no contraction; division and square
// root correctly rounded, as hipcc builds them by default), so its results
// equal the reference's bit for bit:
//   m = b1 * m + (1 - b1) * g;   v = b2 * v + (1 - b2) * (g * g)
//   w = w - (lr * (m / bc1)) / (sqrt(v / bc2) + eps)
//   w = w - (lr * wd) * w        (when the parameter decays)
// with bc1 = 1 - b1^t and bc2 = 1 - b2^t formed in double on the host.
//
// HBM-bound: 16 bytes read (w, g, m, v) and 12 written per element, one
// 16-byte access per lane and array; the kernel can also fold max |w| of the
// updated weights into an amax (NaN ignored) for the re-quantization, which
// then runs as the amax-scaled cast (4 + 1 or 0.5 bytes per element).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

struct AdamHP {
  float b1, omb1, b2, omb2, bc1, bc2, lr, eps, lrwd;
  int decay;
};

__device__ __forceinline__ float adam_elem(float w, float g, float& m, float& v, const AdamHP& h) {
  m = h.b1 * m + h.omb1 * g;
  v = h.b2 * v + h.omb2 * (g * g);
  const float m_hat = m / h.bc1;
  const float v_hat = v / h.bc2;
  w = w - (h.lr * m_hat) / (sqrtf(v_hat) + h.eps);
  if (h.decay) w = w - h.lrwd * w;
  return w;
}

__device__ __forceinline__ uint32_t abs_max(uint32_t am, float w) {
  const uint32_t a = __float_as_uint(w) & 0x7FFFFFFFu;
  return (a <= 0x7F800000u && a > am) ? a : am;
}

constexpr int ADAM_THREADS = 256;
constexpr int ADAM_UNROLL = 2;

// A workgroup takes ADAM_UNROLL * ADAM_THREADS consecutive 4-element groups
// an iteration (lane i the groups i and i + ADAM_THREADS of it, all eight
// 16-byte loads issued first), the workgroups a grid-stride apart; the last,
// partial span group by group and the ragged tail (n % 4 elements) on the
// first lanes of the grid.  Plain (not non-temporal) loads and stores: with
// both non-temporal the seven streams ran at 66% of HBM, plain at 79%.  The
// amax is reduced per workgroup (waves, then LDS) with one atomic each.
__global__ __launch_bounds__(ADAM_THREADS) void adamw_kernel(float* __restrict__ w,
                                                            const float* __restrict__ g,
                                                            float* __restrict__ m,
                                                            float* __restrict__ v, int64_t n,
                                                            AdamHP h, uint32_t* __restrict__ amax) {
  __shared__ uint32_t wave_max[ADAM_THREADS / 64];
  const int64_t n4 = n >> 2;
  constexpr int64_t SPAN = (int64_t)ADAM_UNROLL * ADAM_THREADS;
  const int64_t t0 = (int64_t)blockIdx.x * ADAM_THREADS + threadIdx.x;
  f4* W4 = reinterpret_cast<f4*>(w);
  const f4* G4 = reinterpret_cast<const f4*>(g);
  f4* M4 = reinterpret_cast<f4*>(m);
  f4* V4 = reinterpret_cast<f4*>(v);
  uint32_t am = 0;
  auto update = [&](f4& wv, const f4& gv, f4& mv, f4& vv) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float mq = mv[q], vq = vv[q];
      wv[q] = adam_elem(wv[q], gv[q], mq, vq, h);
      mv[q] = mq;
      vv[q] = vq;
      if (amax) am = abs_max(am, wv[q]);
    }
  };
  for (int64_t b0 = (int64_t)blockIdx.x * SPAN; b0 < n4; b0 += (int64_t)gridDim.x * SPAN) {
    const int64_t i0 = b0 + threadIdx.x;
    if (b0 + SPAN <= n4) {
      f4 wv[ADAM_UNROLL], gv[ADAM_UNROLL], mv[ADAM_UNROLL], vv[ADAM_UNROLL];
#pragma unroll
      for (int j = 0; j < ADAM_UNROLL; ++j) {
        const int64_t i = i0 + j * ADAM_THREADS;
        wv[j] = W4[i]; gv[j] = G4[i]; mv[j] = M4[i]; vv[j] = V4[i];
      }
#pragma unroll
      for (int j = 0; j < ADAM_UNROLL; ++j) update(wv[j], gv[j], mv[j], vv[j]);
#pragma unroll
      for (int j = 0; j < ADAM_UNROLL; ++j) {
        const int64_t i = i0 + j * ADAM_THREADS;
        W4[i] = wv[j]; M4[i] = mv[j]; V4[i] = vv[j];
      }
    } else {
      for (int j = 0; j < ADAM_UNROLL; ++j) {
        const int64_t i = i0 + j * ADAM_THREADS;
        if (i >= n4) break;
        f4 wv = W4[i], mv = M4[i], vv = V4[i];
        const f4 gv = G4[i];
        update(wv, gv, mv, vv);
        W4[i] = wv; M4[i] = mv; V4[i] = vv;
      }
    }
  }
  const int64_t e = (n4 << 2) + t0;
  if (e < n) {
    float mm = m[e], vv = v[e];
    const float wn = adam_elem(w[e], g[e], mm, vv, h);
    w[e] = wn;
    m[e] = mm;
    v[e] = vv;
    if (amax) am = abs_max(am, wn);
  }
  if (amax) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint32_t t = (uint32_t)__shfl_xor((int)am, o);
      am = t > am ? t : am;
    }
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = am;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t b = wave_max[0];
#pragma unroll
      for (int k = 1; k < ADAM_THREADS / 64; ++k) b = wave_max[k] > b ? wave_max[k] : b;
      if (b) atomicMax(amax, b);
    }
  }
}

// The same update on a float64 parameter (the reference's BatchNorm gamma /
// beta are float64 arrays, and np.zeros_like gives their moments that dtype):
// every operation in float64, except that numpy forms (1 - b1) * g and
// (1 - b2) * g**2 in float32 when the gradient array is float32 (a Python
// float does not widen an array) and widens them only for the float64 sums.
struct AdamHP64 {
  double b1, omb1, b2, omb2, bc1, bc2, lr, eps, lrwd;
  float omb1f, omb2f;
  int decay;
};

template <bool G32>
__global__ __launch_bounds__(ADAM_THREADS) void adamw_f64_kernel(double* __restrict__ w,
                                                                const void* __restrict__ g,
                                                                double* __restrict__ m,
                                                                double* __restrict__ v,
                                                                int64_t n, AdamHP64 h) {
  const int64_t stride = (int64_t)gridDim.x * ADAM_THREADS;
  for (int64_t i = (int64_t)blockIdx.x * ADAM_THREADS + threadIdx.x; i < n; i += stride) {
    double gm, gs;
    if constexpr (G32) {
      const float gf = reinterpret_cast<const float*>(g)[i];
      gm = (double)(h.omb1f * gf);
      gs = (double)(h.omb2f * (gf * gf));
    } else {
      const double gd = reinterpret_cast<const double*>(g)[i];
      gm = h.omb1 * gd;
      gs = h.omb2 * (gd * gd);
    }
    const double mm = h.b1 * m[i] + gm;
    const double vv = h.b2 * v[i] + gs;
    const double m_hat = mm / h.bc1;
    const double v_hat = vv / h.bc2;
    double ww = w[i] - (h.lr * m_hat) / (sqrt(v_hat) + h.eps);
    if (h.decay) ww = ww - h.lrwd * ww;
    w[i] = ww;
    m[i] = mm;
    v[i] = vv;
  }
}

}  // namespace

int adamw_launch(float* w, const float* g, float* m, float* v, int64_t n, double lr, double beta1,
                 double beta2, double eps, double weight_decay, int64_t step, int decay,
                 float* amax, hipStream_t stream) {
  AdamHP h;
  h.b1 = (float)beta1;
  h.omb1 = (float)(1.0 - beta1);
  h.b2 = (float)beta2;
  h.omb2 = (float)(1.0 - beta2);
  h.bc1 = (float)(1.0 - pow(beta1, (double)step));
  h.bc2 = (float)(1.0 - pow(beta2, (double)step));
  h.lr = (float)lr;
  h.eps = (float)eps;
  h.lrwd = (float)(lr * weight_decay);
  h.decay = weight_decay > 0.0 && decay;
  if (amax) {
    const int rc = fill_u32_launch(reinterpret_cast<uint32_t*>(amax), 0u, 1, stream);
    if (rc != NOVAQ_OK) return rc;
  }
  if (n == 0) return NOVAQ_OK;
  const int64_t n4 = n >> 2;
  int64_t blocks = std::max<int64_t>((n4 + ADAM_UNROLL * ADAM_THREADS - 1) /
                                         (ADAM_UNROLL * ADAM_THREADS),
                                     (n & 3) ? 1 : 0);
  // grid-stride beyond 8 workgroups per CU (also bounds the amax atomics)
  const int64_t cap = (int64_t)device_cu_count() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(ADAM_THREADS), 0, stream, w, g, m,
                     v, n, h, reinterpret_cast<uint32_t*>(amax));
  return check_launch();
}

int adamw_f64_launch(double* w, const void* g, bool g_f32, double* m, double* v, int64_t n,
                     double lr, double beta1, double beta2, double eps, double weight_decay,
                     int64_t step, int decay, hipStream_t stream) {
  if (n == 0) return NOVAQ_OK;
  AdamHP64 h;
  h.b1 = beta1;
  h.omb1 = 1.0 - beta1;
  h.b2 = beta2;
  h.omb2 = 1.0 - beta2;
  h.omb1f = (float)h.omb1;
  h.omb2f = (float)h.omb2;
  h.bc1 = 1.0 - pow(beta1, (double)step);
  h.bc2 = 1.0 - pow(beta2, (double)step);
  h.lr = lr;
  h.eps = eps;
  h.lrwd = lr * weight_decay;
  h.decay = weight_decay > 0.0 && decay;
  int64_t blocks = (n + ADAM_THREADS - 1) / ADAM_THREADS;
  const int64_t cap = (int64_t)device_cu_count() * 8;
  if (blocks > cap) blocks = cap;
  auto kern = g_f32 ? adamw_f64_kernel<true> : adamw_f64_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(ADAM_THREADS), 0, stream, w, g, m, v, n,
                     h);
  return check_launch();
}

}  // namespace novaq
