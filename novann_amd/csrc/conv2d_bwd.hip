// Conv2d backward on quantized weights (restates Conv2d.backward,
// novann/layers/convolutional/conv2d.py:179-207, and its _col2im, :117-148).
//
//   grad_weight[co, c, kh, kw] = sum_{n, oh, ow} grad[n, co, oh, ow] *
//                                xpad[n, c, oh*sh + kh, ow*sw + kw]
//     (xpad: the input padded in pad_mode with numpy.pad's rules, i.e. the
//     column matrix the forward built);
//   grad_bias[co] = sum_{n, oh, ow} grad[n, co, oh, ow];
//   grad_input[n, c, h, w] = sum over (co, kh, kw) with h + ph - kh = oh*sh and
//     w + pw - kw = ow*sw of s*dec(W[co, c, kh, kw]) * grad[n, co, oh, ow]:
//     col2im into a zero-padded buffer with the border cropped, so the padding
//     mode does not enter (the reference crops; it does not fold the border
//     back onto the pixels the padding copied).
//
// Kernels:
//   - flip_weights_kernel: Wf[c, co, kh, kw] = W[co, c, KH-1-kh, KW-1-kw],
//     codes permuted (exact).  With stride 1 and padding < kernel size,
//     grad_input is the forward convolution of grad with Wf and zero padding
//     (KH-1-ph, KW-1-pw), run by conv2d.hip's kernels;
//   - dinput_direct_kernel: the sum above element by element in fp32, for the
//     other strides and paddings;
//   - dweight_kernel: implicit GEMM on bf16 MFMA (v_mfma_f32_32x32x16_bf16):
//     M = output channels (64 per workgroup), N = (c, kh, kw) (64 per
//     workgroup), K = the output pixels of a run of images, 64 per LDS stage
//     (grad rows staged with consecutive loads, the padded-input operand
//     gathered element-wise with the padding mode resolved); each workgroup
//     writes one partial to the workspace;
//   - chansum_partial_kernel: per-channel partial sums of grad over a slice
//     of (n, pixel);
//   - reduce_partials_kernel: adds the partials in slice order, so results do
//     not depend on scheduling.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int pad_idx(int i, int n, int mode) {
  if (i >= 0 && i < n) return i;
  if (mode == NOVAQ_PAD_ZEROS) return -1;
  if (mode == NOVAQ_PAD_REPLICATE) return i < 0 ? 0 : n - 1;
  if (mode == NOVAQ_PAD_CIRCULAR) {
    int r = i % n;
    return r < 0 ? r + n : r;
  }
  if (n == 1) return 0;  // reflect, period 2(n-1)
  const int p = 2 * (n - 1);
  int r = i % p;
  if (r < 0) r += p;
  return r >= n ? p - r : r;
}

template <int WT>
__device__ __forceinline__ uint32_t code_at(const uint8_t* __restrict__ w, int64_t e) {
  if constexpr (WT == E2M1) return (w[e >> 1] >> ((e & 1) * 4)) & 0xFu;
  else if constexpr (dtype_bits(WT) == 8) return w[e];
  else if constexpr (dtype_bits(WT) == 16) return reinterpret_cast<const uint16_t*>(w)[e];
  else return reinterpret_cast<const uint32_t*>(w)[e];
}

// Wf[c, co, kh, kw] = W[co, c, KH-1-kh, KW-1-kw]; one thread per output byte
// (E2M1: two elements; the total is even) or element.
template <int WT>
__global__ void flip_weights_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ wf,
                                    int C_out, int C, int KH, int KW) {
  constexpr int PER = WT == E2M1 ? 2 : 1;
  const int64_t total = (int64_t)C_out * C * KH * KW;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t * PER >= total) return;
  uint32_t out = 0;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int64_t e = t * PER + q;  // index into Wf (c, co, kh, kw)
    if (e >= total) break;          // E2M1 with an odd total: the last high nibble is 0
    const int kw = (int)(e % KW);
    int64_t r = e / KW;
    const int kh = (int)(r % KH);
    r /= KH;
    const int co = (int)(r % C_out);
    const int c = (int)(r / C_out);
    const int64_t src = (((int64_t)co * C + c) * KH + (KH - 1 - kh)) * KW + (KW - 1 - kw);
    out |= code_at<WT>(w, src) << (q * 4);
  }
  if constexpr (dtype_bits(WT) <= 8) wf[t] = (uint8_t)out;
  else if constexpr (dtype_bits(WT) == 16) reinterpret_cast<uint16_t*>(wf)[t] = (uint16_t)out;
  else reinterpret_cast<uint32_t*>(wf)[t] = out;
}

struct BwdGeom {
  int N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, pad_mode, OH, OW;
};

// grad_input, one element per thread, fp32 accumulation over (kh, kw, co).
template <int WT>
__global__ __launch_bounds__(256) void dinput_direct_kernel(const float* __restrict__ grad,
                                                           const uint8_t* __restrict__ w,
                                                           const float* __restrict__ w_scale,
                                                           float* __restrict__ gi, BwdGeom g) {
  const int64_t total = (int64_t)g.N * g.C * g.H * g.W;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int wx = (int)(t % g.W);
  int64_t r = t / g.W;
  const int hy = (int)(r % g.H);
  r /= g.H;
  const int c = (int)(r % g.C);
  const int n = (int)(r / g.C);
  const float s = w_scale ? *w_scale : 1.0f;
  float acc = 0.0f;
  for (int kh = 0; kh < g.KH; ++kh) {
    const int th = hy + g.ph - kh;
    if (th < 0 || th % g.sh) continue;
    const int oh = th / g.sh;
    if (oh >= g.OH) continue;
    for (int kw = 0; kw < g.KW; ++kw) {
      const int tw = wx + g.pw - kw;
      if (tw < 0 || tw % g.sw) continue;
      const int ow = tw / g.sw;
      if (ow >= g.OW) continue;
      for (int co = 0; co < g.C_out; ++co) {
        const float gv = grad[(((int64_t)n * g.C_out + co) * g.OH + oh) * g.OW + ow];
        const int64_t e = (((int64_t)co * g.C + c) * g.KH + kh) * g.KW + kw;
        acc += u2f(decode<WT>(code_at<WT>(w, e))) * s * gv;
      }
    }
  }
  gi[t] = acc;
}

constexpr int DW_THREADS = 256;
constexpr int DW_M = 64, DW_N = 64, DW_K = 64;  // workgroup tile and K stage
constexpr int DW_PITCH = DW_K + 8;              // bf16 per LDS row (144 B: conflict-free reads)

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
  f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Partial grad_weight of one (image chunk, co block, j block):
// part[chunk][co][j] fp32, j = (c, kh, kw) flattened (the weight's layout).
__global__ __launch_bounds__(DW_THREADS, 2) void dweight_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, float* __restrict__ part,
    BwdGeom g, int ckk, int chunks) {
  __shared__ __attribute__((aligned(16))) __bf16 As[DW_M * DW_PITCH];  // [co][k]
  __shared__ __attribute__((aligned(16))) __bf16 Bs[DW_N * DW_PITCH];  // [j][k]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  const int chunk = blockIdx.x, co0 = blockIdx.y * DW_M, j0 = blockIdx.z * DW_N;
  const int n_begin = (int)((int64_t)g.N * chunk / chunks);
  const int n_end = (int)((int64_t)g.N * (chunk + 1) / chunks);
  const int P = g.OH * g.OW;
  const int64_t HW = (int64_t)g.H * g.W;
  const int wm = (wave & 1) * 32, wn = (wave >> 1) * 32;

  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

  for (int n = n_begin; n < n_end; ++n) {
    const float* gn = grad + (int64_t)n * g.C_out * P;
    const float* xn = x + (int64_t)n * g.C * HW;
    for (int p0 = 0; p0 < P; p0 += DW_K) {
      // A: grad[n, co0 + i, p0 .. p0+63] -> As[i][k], four pixels per item
#pragma unroll
      for (int it = 0; it < DW_M * DW_K / 4 / DW_THREADS; ++it) {
        const int item = tid + it * DW_THREADS;
        const int i = item / (DW_K / 4), k4 = (item % (DW_K / 4)) * 4;
        const int co = co0 + i;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int p = p0 + k4 + q;
          v[q] = (co < g.C_out && p < P) ? gn[(int64_t)co * P + p] : 0.0f;
        }
        *reinterpret_cast<uint2*>(&As[i * DW_PITCH + k4]) =
            make_uint2(bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3]));
      }
      // B: xpad[n, c, oh*sh + kh - ph, ow*sw + kw - pw] for j = (c, kh, kw)
#pragma unroll
      for (int it = 0; it < DW_N * DW_K / 4 / DW_THREADS; ++it) {
        const int item = tid + it * DW_THREADS;
        const int jj = item / (DW_K / 4), k4 = (item % (DW_K / 4)) * 4;
        const int j = j0 + jj;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (j < ckk) {
          const int kw = j % g.KW, ckh = j / g.KW;
          const int kh = ckh % g.KH, c = ckh / g.KH;
          const float* xc = xn + (int64_t)c * HW;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int p = p0 + k4 + q;
            if (p < P) {
              const int oh = p / g.OW, ow = p - oh * g.OW;
              const int hi = pad_idx(oh * g.sh + kh - g.ph, g.H, g.pad_mode);
              const int wi = pad_idx(ow * g.sw + kw - g.pw, g.W, g.pad_mode);
              if (hi >= 0 && wi >= 0) v[q] = xc[(int64_t)hi * g.W + wi];
            }
          }
        }
        *reinterpret_cast<uint2*>(&Bs[jj * DW_PITCH + k4]) =
            make_uint2(bf16_pair(v[0], v[1]), bf16_pair(v[2], v[3]));
      }
      __syncthreads();
#pragma unroll
      for (int st = 0; st < DW_K / 16; ++st) {
        const int kk = st * 16 + half * 8;
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&As[(wm + (lane & 31)) * DW_PITCH + kk]);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(&Bs[(wn + (lane & 31)) * DW_PITCH + kk]);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
      }
      __syncthreads();
    }
  }
  // lane holds column wn + (lane & 31) and rows wm + 8*(r/4) + 4*half + r%4
  float* pc = part + (int64_t)chunk * g.C_out * ckk;
  const int j = j0 + wn + (lane & 31);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int co = co0 + wm + 8 * (r >> 2) + 4 * half + (r & 3);
    if (co < g.C_out && j < ckk) pc[(int64_t)co * ckk + j] = acc[r];
  }
}

constexpr int CH_THREADS = 256;

// bpart[slice][co] = sum of grad[n, co, p] over this slice's (n, p) range, in
// a fixed order (thread-strided, then a fixed tree through LDS).
__global__ __launch_bounds__(CH_THREADS) void chansum_partial_kernel(const float* __restrict__ grad,
                                                                    int N, int C_out, int P,
                                                                    int slices,
                                                                    float* __restrict__ bpart) {
  __shared__ float red[CH_THREADS];
  const int co = blockIdx.x, slice = blockIdx.y;
  const int64_t total = (int64_t)N * P;
  const int64_t b = total * slice / slices, e = total * (slice + 1) / slices;
  float s = 0.0f;
  for (int64_t i = b + threadIdx.x; i < e; i += CH_THREADS) {
    const int64_t n = i / P, p = i - n * P;
    s += grad[(n * C_out + co) * P + p];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = CH_THREADS / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) bpart[(int64_t)slice * C_out + co] = red[0];
}

// out[i] = sum over k < parts of part[k][i], in k order.
__global__ void reduce_partials_kernel(const float* __restrict__ part, int parts, int64_t len,
                                       float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= len) return;
  float s = 0.0f;
  for (int k = 0; k < parts; ++k) s += part[(int64_t)k * len + i];
  out[i] = s;
}

template <int WT>
int launch_flip(const void* w, void* wf, const BwdGeom& g, hipStream_t stream) {
  const int64_t total = (int64_t)g.C_out * g.C * g.KH * g.KW;
  const int64_t items = WT == E2M1 ? (total + 1) / 2 : total;
  const int64_t blocks = (items + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(flip_weights_kernel<WT>, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint8_t*>(w), static_cast<uint8_t*>(wf), g.C_out, g.C,
                     g.KH, g.KW);
  return check_launch();
}

template <int WT>
int launch_dinput(const float* grad, const void* w, const void* wf, const float* w_scale,
                  float* gi, const BwdGeom& g, hipStream_t stream) {
  // stride 1 and padding below the kernel size: the forward convolution of
  // grad with the flipped weights and zero padding (KH-1-ph, KW-1-pw)
  if (g.sh == 1 && g.sw == 1 && g.ph < g.KH && g.pw < g.KW) {
    int rc = launch_flip<WT>(w, const_cast<void*>(wf), g, stream);
    if (rc != NOVAQ_OK) return rc;
    rc = conv2d_launch(grad, g.N, g.C_out, g.OH, g.OW, wf, WT, w_scale, g.C, g.KH, g.KW, 1, 1,
                       g.KH - 1 - g.ph, g.KW - 1 - g.pw, NOVAQ_PAD_ZEROS, nullptr, gi, stream);
    if (rc != NOVAQ_ENOTSUP) return rc;
  }
  const int64_t total = (int64_t)g.N * g.C * g.H * g.W;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  hipLaunchKernelGGL(dinput_direct_kernel<WT>, dim3((unsigned)blocks), dim3(256), 0, stream,
                     grad, static_cast<const uint8_t*>(w), w_scale, gi, g);
  return check_launch();
}

}  // namespace

// Workspace layout of conv2d_backward (each part 256-byte aligned).
ConvBwdWs conv2d_bwd_workspace(int64_t N, int64_t C, int64_t C_out, int KH, int KW, int w_dtype,
                               int cus) {
  ConvBwdWs ws{};
  auto a256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const int64_t ckk = C * KH * KW;
  const int64_t co_blocks = (C_out + DW_M - 1) / DW_M, j_blocks = (ckk + DW_N - 1) / DW_N;
  // enough image chunks for about two workgroups per CU
  const int64_t want = std::max<int64_t>(1, (2LL * cus + co_blocks * j_blocks - 1) /
                                                (co_blocks * j_blocks));
  ws.chunks = (int)std::max<int64_t>(1, std::min<int64_t>(N, want));
  ws.slices = (int)std::max<int64_t>(1, std::min<int64_t>(N, 64));
  ws.wf = 0;
  ws.part = a256(((size_t)C_out * ckk * dtype_bits(w_dtype) + 7) / 8);
  ws.bpart = ws.part + a256((size_t)ws.chunks * C_out * ckk * 4);
  ws.total = ws.bpart + a256((size_t)ws.slices * C_out * 4);
  return ws;
}

int conv2d_backward_launch(const float* grad, const float* x, int64_t N, int64_t C, int64_t H,
                           int64_t W, const void* w_q, int w_dtype, const float* w_scale,
                           int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw,
                           int pad_mode, float* grad_input, float* grad_weight,
                           float* grad_bias, void* workspace, hipStream_t stream) {
  BwdGeom g{};
  g.N = (int)N; g.C = (int)C; g.H = (int)H; g.W = (int)W; g.C_out = (int)C_out;
  g.KH = KH; g.KW = KW; g.sh = sh; g.sw = sw; g.ph = ph; g.pw = pw; g.pad_mode = pad_mode;
  g.OH = (int)((H + 2 * (int64_t)ph - KH) / sh + 1);
  g.OW = (int)((W + 2 * (int64_t)pw - KW) / sw + 1);
  const ConvBwdWs ws = conv2d_bwd_workspace(N, C, C_out, KH, KW, w_dtype, device_cu_count());
  uint8_t* base = static_cast<uint8_t*>(workspace);
  int rc = NOVAQ_OK;
  if (grad_input && N > 0) {
    void* wf = base + ws.wf;
    switch (w_dtype) {
      case E4M3: rc = launch_dinput<E4M3>(grad, w_q, wf, w_scale, grad_input, g, stream); break;
      case E5M2: rc = launch_dinput<E5M2>(grad, w_q, wf, w_scale, grad_input, g, stream); break;
      case E2M1: rc = launch_dinput<E2M1>(grad, w_q, wf, w_scale, grad_input, g, stream); break;
      case BF16: rc = launch_dinput<BF16>(grad, w_q, wf, w_scale, grad_input, g, stream); break;
      case F16: rc = launch_dinput<F16>(grad, w_q, wf, w_scale, grad_input, g, stream); break;
      case F32: rc = launch_dinput<F32>(grad, w_q, wf, w_scale, grad_input, g, stream); break;
      default: return NOVAQ_EDTYPE;
    }
    if (rc != NOVAQ_OK) return rc;
  }
  const int64_t ckk = C * KH * KW;
  if (grad_weight) {
    float* part = reinterpret_cast<float*>(base + ws.part);
    const int64_t co_blocks = (C_out + DW_M - 1) / DW_M, j_blocks = (ckk + DW_N - 1) / DW_N;
    if (co_blocks > 65535 || j_blocks > 65535) return NOVAQ_EINVAL;
    hipLaunchKernelGGL(dweight_kernel, dim3((unsigned)ws.chunks, (unsigned)co_blocks,
                                            (unsigned)j_blocks),
                       dim3(DW_THREADS), 0, stream, grad, x, part, g, (int)ckk, ws.chunks);
    rc = check_launch();
    if (rc != NOVAQ_OK) return rc;
    const int64_t len = C_out * ckk;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3((unsigned)((len + 255) / 256)), dim3(256), 0,
                       stream, part, ws.chunks, len, grad_weight);
    rc = check_launch();
    if (rc != NOVAQ_OK) return rc;
  }
  if (grad_bias) {
    float* bpart = reinterpret_cast<float*>(base + ws.bpart);
    if (C_out > 0x7FFFFFFF) return NOVAQ_EINVAL;
    hipLaunchKernelGGL(chansum_partial_kernel, dim3((unsigned)C_out, (unsigned)ws.slices),
                       dim3(CH_THREADS), 0, stream, grad, g.N, g.C_out, g.OH * g.OW, ws.slices,
                       bpart);
    rc = check_launch();
    if (rc != NOVAQ_OK) return rc;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3((unsigned)((C_out + 255) / 256)), dim3(256),
                       0, stream, bpart, ws.slices, C_out, grad_bias);
    rc = check_launch();
  }
  return rc;
}

}  // namespace novaq
