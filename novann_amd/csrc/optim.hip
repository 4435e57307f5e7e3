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

// Lane i of the grid takes the 4-element groups i, i + stride, ...; the
// ragged tail (n % 4 elements) goes to the first lanes of the grid.
__global__ __launch_bounds__(ADAM_THREADS) void adamw_kernel(float* __restrict__ w,
                                                            const float* __restrict__ g,
                                                            float* __restrict__ m,
                                                            float* __restrict__ v, int64_t n,
                                                            AdamHP h, uint32_t* __restrict__ amax) {
  const int64_t n4 = n >> 2;
  const int64_t stride = (int64_t)gridDim.x * ADAM_THREADS;
  const int64_t t0 = (int64_t)blockIdx.x * ADAM_THREADS + threadIdx.x;
  uint32_t am = 0;
  for (int64_t i = t0; i < n4; i += stride) {
    float4 wv = reinterpret_cast<const float4*>(w)[i];
    const float4 gv = reinterpret_cast<const float4*>(g)[i];
    float4 mv = reinterpret_cast<const float4*>(m)[i];
    float4 vv = reinterpret_cast<const float4*>(v)[i];
    wv.x = adam_elem(wv.x, gv.x, mv.x, vv.x, h);
    wv.y = adam_elem(wv.y, gv.y, mv.y, vv.y, h);
    wv.z = adam_elem(wv.z, gv.z, mv.z, vv.z, h);
    wv.w = adam_elem(wv.w, gv.w, mv.w, vv.w, h);
    reinterpret_cast<float4*>(w)[i] = wv;
    reinterpret_cast<float4*>(m)[i] = mv;
    reinterpret_cast<float4*>(v)[i] = vv;
    if (amax) am = abs_max(abs_max(abs_max(abs_max(am, wv.x), wv.y), wv.z), wv.w);
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
    if ((threadIdx.x & 63) == 0 && am) atomicMax(amax, am);
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
  int64_t blocks = (std::max<int64_t>(n4, n & 3) + ADAM_THREADS - 1) / ADAM_THREADS;
  const int64_t cap = (int64_t)device_cu_count() * 32;  // grid-stride beyond this
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(ADAM_THREADS), 0, stream, w, g, m,
                     v, n, h, reinterpret_cast<uint32_t*>(amax));
  return check_launch();
}

}  // namespace novaq
