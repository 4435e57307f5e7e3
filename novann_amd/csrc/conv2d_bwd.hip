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
//   - flip (in finish_kernel): Wf[c, co, kh, kw] = W[co, c, KH-1-kh, KW-1-kw],
//     codes permuted (exact).  With stride 1 and padding < kernel size,
//     grad_input is the forward convolution of grad with Wf and zero padding
//     (KH-1-ph, KW-1-pw), run by conv2d.hip's kernels;
//   - dinput_direct_kernel: the sum above element by element in fp32, for the
//     other strides and paddings;
//   - dweight_kernel: implicit GEMM on bf16 MFMA (v_mfma_f32_32x32x16_bf16):
//     M = output channels (64 per workgroup), N = (c, kh, kw) (64 per
//     workgroup), K = the output pixels of a run of images (a chunk), 64 per
//     LDS stage (grad rows staged with 16-byte loads, the padded-input
//     operand gathered element-wise with the padding mode resolved); each
//     workgroup writes one partial grad_weight tile to the workspace, and the
//     first j block also the per-channel grad sums of its chunk (grad_bias);
//   - finish_kernel: one launch that adds the chunk partials in a fixed order
//     (novaq_colsum.h's column sum, so results do not depend on scheduling;
//     16 columns a workgroup with one input channel, else 64); with one input
//     channel and grad_input on the one-output-channel kernel, c1_tail_kernel
//     instead: the same sums beside grad_input's bands, the weight read
//     flipped in place
//     for grad_weight and grad_bias, and flips the weights for grad_input;
//     grad_input's convolution runs after it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "conv2d_impl.h"
#include "novaq_colsum.h"
#include "novaq_convert.h"
#include "novaq_internal.h"

namespace novaq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2b __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int WT>
__device__ __forceinline__ uint32_t code_at(const uint8_t* __restrict__ w, int64_t e) {
  if constexpr (WT == E2M1) return (w[e >> 1] >> ((e & 1) * 4)) & 0xFu;
  else if constexpr (dtype_bits(WT) == 8) return w[e];
  else if constexpr (dtype_bits(WT) == 16) return reinterpret_cast<const uint16_t*>(w)[e];
  else return reinterpret_cast<const uint32_t*>(w)[e];
}

// Wf[c, co, kh, kw] = W[co, c, KH-1-kh, KW-1-kw]: output byte t (E2M1: two
// elements; an odd total leaves the last high nibble 0) or element t.
template <int WT>
__device__ __forceinline__ void flip_item(const uint8_t* __restrict__ w, uint8_t* __restrict__ wf,
                                          int64_t t, int C_out, int C, int KH, int KW) {
  constexpr int PER = WT == E2M1 ? 2 : 1;
  const int64_t total = (int64_t)C_out * C * KH * KW;
  uint32_t out = 0;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int64_t e = t * PER + q;  // index into Wf (c, co, kh, kw)
    if (e >= total) break;
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

// The backward's finishing launch (1024-lane workgroups): blocks [0, wb) sum
// grad_weight's columns over the chunk partials (permuted from (tap, co, c)
// to (co, c, tap) when pt > 0), [wb, wb + bb) grad_bias's, and the rest flip
// 1024 weight items each for grad_input.
struct FinishArgs {
  const float* part;
  float* gw;
  const float* bpart;
  float* gb;
  const uint8_t* w;
  uint8_t* wf;
  int64_t rows, wcols, bcols, flip_items;
  int pt, pco, pc;
  unsigned wb, bb;
};

// COLS: the column sums' block width (16 for the one-input-channel kernel's
// many short partials, else 64).
template <int WT, int COLS>
__global__ __launch_bounds__(1024) void finish_kernel(FinishArgs a, int C_out, int C, int KH,
                                                      int KW) {
  constexpr int SLICES = 1024 / COLS;
  __shared__ float part[SLICES][COLS];
  const unsigned b = blockIdx.x;
  if (b < a.wb) {
    colsum_block<COLS, SLICES>(a.part, a.rows, a.wcols, a.gw, a.pt, a.pco, a.pc, b, part);
  } else if (b < a.wb + a.bb) {
    colsum_block<COLS, SLICES>(a.bpart, a.rows, a.bcols, a.gb, 0, 0, 0, b - a.wb, part);
  } else {
    const int64_t t = (int64_t)(b - a.wb - a.bb) * 1024 + threadIdx.x;
    if (t < a.flip_items) flip_item<WT>(a.w, a.wf, t, C_out, C, KH, KW);
  }
}

struct BwdGeom {
  int N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, pad_mode, OH, OW;
};

// The last launch of a one-input-channel backward whose grad_input runs on
// the one-output-channel kernel: blocks [0, a.wb + a.bb) sum the partials
// (4 columns a 256-lane workgroup over the 64 row slices finish_kernel<WT,
// 16> uses: the same sums bit for bit), the rest are grad_input's bands --
// that kernel over grad with the weight read flipped in place, so no flip
// waits for the sums -- and the latency-bound sums hide under the bands.
template <int WT>
__global__ __launch_bounds__(256) void c1_tail_kernel(FinishArgs a, const float* __restrict__ grad,
                                                      const uint8_t* __restrict__ w,
                                                      const float* __restrict__ w_scale,
                                                      float* __restrict__ gi, Co1Geom cg) {
  extern __shared__ __attribute__((aligned(16))) uint8_t t_lds[];
  const unsigned b = blockIdx.x;
  if (b < a.wb + a.bb) {
    auto part = reinterpret_cast<float(*)[4]>(t_lds);  // 64 x 4 floats
    if (b < a.wb)
      colsum_block<4, 64>(a.part, a.rows, a.wcols, a.gw, a.pt, a.pco, a.pc, b, part);
    else
      colsum_block<4, 64>(a.bpart, a.rows, a.bcols, a.gb, 0, 0, 0, b - a.wb, part);
    return;
  }
  Epilogue ep{};
  ep.out_dtype = F32;
  co1_body<WT, F32, true>(reinterpret_cast<const uint8_t*>(grad), nullptr, w, w_scale, ep, gi,
                          cg, (int)(b - a.wb - a.bb), t_lds);
}

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
constexpr int DW_PER_CU = 8;        // target workgroups per CU
constexpr int DW_MAX_CHUNKS = 512;  // a multiple of 8
constexpr uint32_t DW_OOB = 0x80000000u;  // a buffer offset past any image (reads 0)

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
  f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Partial grad_weight of one (image chunk, co block, j block):
// part[chunk][co][j] fp32, j = (c, kh, kw) flattened (the weight's layout).
// The workgroups of j block 0 also write the partial grad_bias of their
// (chunk, co block) to bpart[chunk][co] when bpart is given: the fp32 sum of
// the grad values they stage (per lane in stage order, then a fixed butterfly
// over the 32 lanes that share a row).
//
// BIAS_ONLY: the same grid and grad reads, bias partials only (so a call
// that asks for grad_bias alone gets the same bits as one that also asks for
// grad_weight).
//
// Staging: lane l of wave w holds the two consecutive pixels 2*(l%32), +1 of
// the stage for the tile rows 2w + l/32 + 8i (i < 8): grad rows are read as
// 8-byte pairs, 256 contiguous bytes per half-wave.  The (c, kh, kw) of the
// B rows come from a 64-entry table built once per workgroup.
// BUF (P even, an image's grad and x under 1 GiB each): every stage load is a
// buffer load through per-image descriptors, a masked slot (a channel, tap
// or pixel past its end, or padding) carrying an offset past the buffer, so
// it reads 0 and no load sits behind a branch; all offsets are formed before
// the loads are issued back to back.  Same values staged, same results.
template <bool ZEROPAD, bool BIAS_ONLY, bool BUF>
__global__ __launch_bounds__(DW_THREADS, 2) void dweight_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, float* __restrict__ part,
    float* __restrict__ bpart, BwdGeom g, int ckk, int chunks, int co_blocks, int j_blocks) {
  __shared__ __attribute__((aligned(16))) __bf16 As[DW_M * DW_PITCH];  // [co][k]
  __shared__ __attribute__((aligned(16))) __bf16 Bs[DW_N * DW_PITCH];  // [j][k]
  // per B row: c*H*W + (kh - ph)*W + (kw - pw), kh - ph, kw - pw, j < ckk
  __shared__ int4 jtab[DW_N];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  // 1-D grid; the workgroups of one chunk (all its co and j blocks) share an
  // XCD (workgroup i runs on XCD i % 8) so its grad rows are fetched into
  // that XCD's L2 once: on XCD x, the k-th run of `per` workgroups is chunk
  // 8k + x (chunks is a multiple of 8 when it is at least 8)
  const int per = co_blocks * j_blocks;
  int chunk, member;
  if (chunks >= 8) {
    const int x8 = blockIdx.x & 7, i = blockIdx.x >> 3;
    chunk = (i / per) * 8 + x8;
    member = i % per;
  } else {
    chunk = blockIdx.x / per;
    member = blockIdx.x % per;
  }
  const int jb = member % j_blocks, cb = member / j_blocks;
  const int co0 = cb * DW_M, j0 = jb * DW_N;
  const int P = g.OH * g.OW;
  const int SP = (P + DW_K - 1) / DW_K;  // stages per image
  // this chunk's run of (image, stage) pairs
  const int64_t T = (int64_t)g.N * SP;
  const int64_t t_begin = T * chunk / chunks, t_end = T * (chunk + 1) / chunks;
  const int HW = g.H * g.W;  // C*H*W < 2^31 (checked by the entry point)
  const int wm = (wave & 1) * 32, wn = (wave >> 1) * 32;
  const bool want_bias = bpart != nullptr && jb == 0;

  if (!BIAS_ONLY && tid < DW_N) {
    const int j = j0 + tid;
    const int kw = j % g.KW, ckh = j / g.KW;
    const int kh = ckh % g.KH, c = ckh / g.KH;
    const int dh = kh - g.ph, dw = kw - g.pw;
    jtab[tid] = make_int4(c * HW + dh * g.W + dw, dh, dw, j < ckk ? 1 : 0);
  }
  float bsum[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) bsum[i] = 0.0f;

  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  if (!BIAS_ONLY) __syncthreads();  // jtab

  // one stage = 64 pixels of one image; stage s + 1 is loaded into registers
  // while stage s is multiplied
  const int k = 2 * (lane & 31), rbase = 2 * wave + half;
  const bool pvec = (P & 1) == 0;
  float a[8][2], bv[8][2];
  auto load_stage = [&](int n, int p0) {
    const float* gn = grad + (int64_t)n * g.C_out * P;
    const float* xn = x + (int64_t)n * g.C * HW;
    const int p = p0 + k;
    const bool v0 = p < P, v1 = p + 1 < P;
    if constexpr (BUF) {
      // P even: a pair is whole or past the end
      const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(gn), (short)0, g.C_out * P * 4, 0x00020000);
      uint32_t aoff[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int co = co0 + rbase + 8 * i;
        aoff[i] = co < g.C_out && v0 ? (uint32_t)(co * P + p) * 4 : DW_OOB;
      }
      uint32_t boff[8][2];
      int hb[2], wb[2];
      if constexpr (!BIAS_ONLY) {
        const int oh = p / g.OW, ow = p - oh * g.OW;
        hb[0] = oh * g.sh;
        wb[0] = ow * g.sw;
        const bool wrap = ow + 1 == g.OW;
        hb[1] = wrap ? hb[0] + g.sh : hb[0];
        wb[1] = wrap ? 0 : wb[0] + g.sw;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int4 t = jtab[rbase + 8 * i];
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            int hi = hb[q] + t.y, wi = wb[q] + t.z;
            bool in;
            int e;
            if constexpr (ZEROPAD) {
              in = (unsigned)hi < (unsigned)g.H && (unsigned)wi < (unsigned)g.W;
              e = t.x + hb[q] * g.W + wb[q];
            } else {
              hi = pad_index(hi, g.H, g.pad_mode);
              wi = pad_index(wi, g.W, g.pad_mode);
              in = hi >= 0 && wi >= 0;
              e = t.x - t.y * g.W - t.z + hi * g.W + wi;
            }
            boff[i][q] = t.w && (q ? v1 : v0) && in ? (uint32_t)e * 4 : DW_OOB;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const u32x2b v = __builtin_amdgcn_raw_buffer_load_b64(grs, aoff[i], 0, 0);
        a[i][0] = u2f(v[0]);
        a[i][1] = u2f(v[1]);
      }
      if constexpr (!BIAS_ONLY) {
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(xn), (short)0, g.C * HW * 4, 0x00020000);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int q = 0; q < 2; ++q)
            bv[i][q] = u2f(__builtin_amdgcn_raw_buffer_load_b32(xrs, boff[i][q], 0, 0));
      }
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
    // A: grad rows co0 + rbase + 8i at pixels p, p+1
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int co = co0 + rbase + 8 * i;
      a[i][0] = a[i][1] = 0.0f;
      if (co < g.C_out) {
        const float* row = gn + (int64_t)co * P + p;
        if (pvec && v1) {
          const float2 f = *reinterpret_cast<const float2*>(row);
          a[i][0] = f.x; a[i][1] = f.y;
        } else {
          if (v0) a[i][0] = row[0];
          if (v1) a[i][1] = row[1];
        }
      }
    }
    if constexpr (!BIAS_ONLY) {
      // B: xpad[n, c, oh*sh + kh - ph, ow*sw + kw - pw] for the rows' (c, kh, kw)
      int hb[2], wb[2];
      const int oh = p / g.OW, ow = p - oh * g.OW;
      hb[0] = oh * g.sh;
      wb[0] = ow * g.sw;
      const bool wrap = ow + 1 == g.OW;
      hb[1] = wrap ? hb[0] + g.sh : hb[0];
      wb[1] = wrap ? 0 : wb[0] + g.sw;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int4 t = jtab[rbase + 8 * i];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          bv[i][q] = 0.0f;
          if (!(t.w && (q ? v1 : v0))) continue;
          int hi = hb[q] + t.y, wi = wb[q] + t.z;
          if constexpr (ZEROPAD) {
            if ((unsigned)hi < (unsigned)g.H && (unsigned)wi < (unsigned)g.W)
              bv[i][q] = xn[t.x + hb[q] * g.W + wb[q]];
          } else {
            hi = pad_index(hi, g.H, g.pad_mode);
            wi = pad_index(wi, g.W, g.pad_mode);
            if (hi >= 0 && wi >= 0) bv[i][q] = xn[t.x - t.y * g.W - t.z + hi * g.W + wi];
          }
        }
      }
    }
  };
  int64_t t = t_begin;
  int n = (int)(t / SP), p0 = (int)(t - (int64_t)n * SP) * DW_K;
  if (t < t_end) load_stage(n, p0);
  while (t < t_end) {
    if (want_bias) {
#pragma unroll
      for (int i = 0; i < 8; ++i) bsum[i] += a[i][0] + a[i][1];
    }
    if constexpr (!BIAS_ONLY) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = rbase + 8 * i;
        *reinterpret_cast<uint32_t*>(&As[r * DW_PITCH + k]) = bf16_pair(a[i][0], a[i][1]);
        *reinterpret_cast<uint32_t*>(&Bs[r * DW_PITCH + k]) = bf16_pair(bv[i][0], bv[i][1]);
      }
    }
    // next stage
    ++t;
    p0 += DW_K;
    if (p0 >= P) { p0 = 0; ++n; }
    if constexpr (BIAS_ONLY) {
      if (t < t_end) load_stage(n, p0);
      continue;
    }
    // barriers order only LDS traffic: wait for this wave's LDS operations,
    // not for the prefetch loads in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (t < t_end) load_stage(n, p0);
#pragma unroll
    for (int st = 0; st < DW_K / 16; ++st) {
      const int kk = st * 16 + half * 8;
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(&As[(wm + (lane & 31)) * DW_PITCH + kk]);
      const bf16x8 bw = *reinterpret_cast<const bf16x8*>(&Bs[(wn + (lane & 31)) * DW_PITCH + kk]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bw, acc, 0, 0, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
  if constexpr (!BIAS_ONLY) {
    // lane holds column wn + (lane & 31) and rows wm + 8*(r/4) + 4*half + r%4
    float* pc = part + (int64_t)chunk * g.C_out * ckk;
    const int j = j0 + wn + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int co = co0 + wm + 8 * (r >> 2) + 4 * half + (r & 3);
      if (co < g.C_out && j < ckk) pc[(int64_t)co * ckk + j] = acc[r];
    }
  }
  if (want_bias) {
    // the 32 lanes of a half share rows rbase + 8i
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float s = bsum[i];
      s += __shfl_xor(s, 16, 32);
      s += __shfl_xor(s, 8, 32);
      s += __shfl_xor(s, 4, 32);
      s += __shfl_xor(s, 2, 32);
      s += __shfl_xor(s, 1, 32);
      const int co = co0 + rbase + 8 * i;
      if ((lane & 31) == 0 && co < g.C_out) bpart[(int64_t)chunk * g.C_out + co] = s;
    }
  }
}

// grad_weight for stride 1 and output rows of at most 64 pixels, one wave
// per window tap.  A workgroup owns 64 output channels (two 32-row MFMA
// tiles) and 32 input channels, and walks a chunk of (image, band of R output
// rows) stages.  Per stage it stages in LDS, as bf16:
//   - Gs[co][k]: grad of the band, k = r * OWP + ow (rows padded to OWP, a
//     multiple of 16, with zeros; R * OWP = 128 = 8 MFMA k-steps);
//   - Xs[c][rr][col] = xpad[c][oh0 + rr - ph][col - xo]: the band's R + KH - 1
//     input rows, XW = OWP + 8 columns each, input column 0 at staged column
//     xo >= pw, the padding mode resolved (zero rows and columns past what
//     the band's outputs read),
// so wave t = (kh, kw) multiplies A = Gs (8 consecutive pixels of one channel,
// a 16-byte LDS read) by B = Xs[c][r + kh][ow + kw - pw + xo ..] (8
// consecutive columns; at an odd start the 16 bytes sit across 5 dwords and
// v_alignbit realigns them) with v_mfma_f32_32x32x16_bf16 into the (co, c)
// block of its tap.  The Xs channel pitch is an odd number of dwords, so the
// 32 channels of a fragment read fall in distinct banks.
//
// All DR_WAVES waves stage, so the staging work is the same on every SIMD
// whatever the tap count; the waves past the taps only stage.  The loads are
// buffer loads: a masked slot (padding, rows past the image, channels past
// the tensor) carries an offset beyond the buffer's size and reads 0, so no
// lane branches.  Per stage a lane forms only its slots' row offsets (the
// channel offsets are fixed, the image and band are stepped, not divided out
// of the stage index).  Two register sets: stage t + 2's loads are issued as
// soon as stage t's registers are in LDS, so they have two stages' products
// to arrive.  Staging, one of two forms:
//   - VEC (zero padding, W and OW multiples of 4, 16-byte aligned tensors):
//     16-byte loads of 4 consecutive grad pixels (one Gs row run, an 8-byte
//     LDS write) or 4 consecutive input columns (two 4-byte LDS writes; xo is
//     pw rounded up to even), items spread over all lanes (GU grad and XJ
//     input items per lane); the padding columns of Xs are zeroed once and
//     never written;
//   - otherwise one 4-byte slot at a time: a band's R * OW grad values and a
//     channel's rows_in * XW staged slots spread over the 64 lanes of a wave
//     (2 and XJ slots per lane), wave w taking channels w, w + DR_WAVES, ...
// Each workgroup writes its chunk's partial as [tap][co][c]; the column sum
// adds the chunks and permutes to [co][c][kh][kw].
constexpr int DR_K = 128;          // pixels per stage
constexpr int DR_WAVES = 12;       // waves per workgroup (at most 12 taps)
constexpr int DR_GC = 6, DR_XC = 3;  // grad / input channels a wave stages (12 x 6 >= 64, 12 x 3 >= 32)
constexpr int DR_GU = 3;           // VEC: grad quads per lane (64 channels x 32 quads <= 3 x 768)
constexpr uint32_t DR_OOB = 0x80000000u;  // byte offset past any buffer (reads 0)
constexpr uint32_t DR_BUF3 = 0x00020000u;  // buffer resource word 3 (raw, 32-bit data)
constexpr int DR_FAR = 1 << 30;    // a row index no band reaches (masked item)

struct RowsGeom {
  int OWP, R, XW, rows_in, taps, cp, spi;  // padded output row, rows per stage, staged row
                                           // width, staged rows, KH*KW, Xs channel pitch
                                           // (bf16), stages per image
  int xo;                                  // staged column of input column 0
};

// One stage's loads in registers.
template <bool VEC, int XJ>
struct RowsRegs {
  float g[2 * DR_GC];
  float x[DR_XC * XJ];
};
template <int XJ>
struct RowsRegs<true, XJ> {
  f32x4 g[DR_GU];
  f32x4 x[XJ];
};

// MODE 0: grad_weight; 1: grad_weight and grad_bias; 2: grad_bias only (no x,
// no products).  grad_bias, in a fixed order: VEC: each lane adds each of its
// grad quads ((v0 + v1) + (v2 + v3)) per stage in stage order, then the
// quads of a channel are added in band order through LDS; otherwise each
// lane adds the grad values it loads per channel in stage order and the wave
// adds its 64 lanes in a fixed butterfly.  c block 0 writes the chunk's
// per-channel sum to bpart.
template <int XJ, int MODE, bool VEC>
__global__ __launch_bounds__(DR_WAVES * 64) void dweight_rows_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, float* __restrict__ part,
    float* __restrict__ bpart, BwdGeom g, RowsGeom rg, int chunks, int co_blocks,
    int c_blocks) {
  constexpr bool WGT = MODE != 2, BIAS = MODE != 0;
  constexpr int NT = DR_WAVES * 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t dr_lds[];
  constexpr int GP = DR_K + 8;  // Gs row pitch (bf16); slot DR_K takes masked lanes
  __bf16* Gs = reinterpret_cast<__bf16*>(dr_lds);
  __bf16* Xs = Gs + 64 * GP;
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tap = wave;  // the product of waves below rg.taps
  const int kh = tap / g.KW, kw = tap - kh * g.KW;
  int bid = blockIdx.x;
  const int cb = bid % c_blocks;
  bid /= c_blocks;
  const int cob = bid % co_blocks;
  const int chunk = bid / co_blocks;
  const int co0 = cob * 64, c0 = cb * 32;
  const int64_t T = (int64_t)g.N * rg.spi;
  const int64_t t_begin = T * chunk / chunks, t_end = T * (chunk + 1) / chunks;
  const int HW = g.H * g.W;
  const int P = g.OH * g.OW;
  const int xslots = rg.rows_in * rg.XW;
  const int q4 = rg.R * g.OW / 4;  // VEC: grad quads of a band per channel
  const int W4 = g.W / 4;

  f32x16 acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;

  // Gs padding columns (ow >= OW), and with VEC the Xs slots no stage writes,
  // are zeroed once.
  if constexpr (WGT) {
    uint32_t* z = reinterpret_cast<uint32_t*>(dr_lds);
    const int words = VEC ? (64 * GP + 32 * rg.cp) / 2 : 64 * GP / 2;
    for (int i = tid; i < words; i += NT) z[i] = 0u;
  }
  float bsum[VEC ? DR_GU : DR_GC];
#pragma unroll
  for (int i = 0; i < (VEC ? DR_GU : DR_GC); ++i) bsum[i] = 0.0f;

  // VEC items of this lane: grad quad u = channel co_l = it / q4, pixels
  // 4 (it % q4) .. + 3 of the band (byte offset gbase before the band's,
  // band row grow, Gs element gdst; DR_FAR / -1 when masked); input quad u =
  // channel it / (rows_in W4), staged row xrr, input columns 4q .. 4q + 3
  // (byte offset xcb before the row's, Xs element xdst)
  uint32_t gbase[DR_GU], xcb[XJ];
  int grow[DR_GU], gdst[DR_GU], xrr[XJ], xdst[XJ];
  // scalar slots of this lane: Gs slot j = grad value m = lane + 64 j of the
  // band (row gr, Gs column gk: DR_K past the band); Xs slot j = staged row
  // xr, input column xw (-1: zero, also for columns no output of the band
  // reads), Xs element xk (the pitch's spare slot past xslots); the byte
  // offsets of this wave's channels (beyond the buffer past the tile or the
  // tensor)
  int gr[2], gk[2], xr[XJ], xw[XJ], xk[XJ];
  uint32_t gch[DR_GC], xch[DR_XC];
  if constexpr (VEC) {
#pragma unroll
    for (int u = 0; u < DR_GU; ++u) {
      const int it = tid + NT * u;
      const int co_l = it / q4, m = 4 * (it - co_l * q4);
      const int r = m / g.OW, col = m - r * g.OW;
      const bool live = co_l < 64 && co0 + co_l < g.C_out;
      gbase[u] = (uint32_t)((co0 + co_l) * P + m) * 4u;
      grow[u] = live ? r : DR_FAR;
      gdst[u] = co_l < 64 ? co_l * GP + r * rg.OWP + col : -1;
    }
#pragma unroll
    for (int u = 0; u < XJ; ++u) {
      const int it = tid + NT * u;
      const int per = rg.rows_in * W4;
      const int c_l = it / per, rest = it - c_l * per;
      const int rr = rest / W4, q = rest - rr * W4;
      const bool live = c_l < 32 && c0 + c_l < g.C;
      xcb[u] = (uint32_t)((c0 + c_l) * HW + 4 * q) * 4u;
      xrr[u] = live ? rr : DR_FAR;
      xdst[u] = c_l < 32 ? c_l * rg.cp + rr * rg.XW + 4 * q + rg.xo : -1;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = lane + 64 * j;
      gr[j] = m / g.OW;
      gk[j] = m < rg.R * g.OW ? gr[j] * rg.OWP + (m - gr[j] * g.OW) : DR_K;
    }
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
      const int e = lane + 64 * j;
      xr[j] = e / rg.XW;
      const int col = e - xr[j] * rg.XW;
      xw[j] = (e < xslots && col < g.OW + g.KW - 1) ? pad_index(col - rg.xo, g.W, g.pad_mode) : -1;
      xk[j] = e < xslots ? e : xslots;
    }
#pragma unroll
    for (int i = 0; i < DR_GC; ++i) {
      const int co_l = wave + DR_WAVES * i;
      gch[i] = (co_l < 64 && co0 + co_l < g.C_out) ? (uint32_t)(co0 + co_l) * (uint32_t)P * 4u
                                                   : 0x40000000u;
    }
#pragma unroll
    for (int i = 0; i < DR_XC; ++i) {
      const int c_l = wave + DR_WAVES * i;
      xch[i] = (c_l < 32 && c0 + c_l < g.C) ? (uint32_t)(c0 + c_l) * (uint32_t)HW * 4u : 0x40000000u;
    }
  }

  typedef RowsRegs<VEC, XJ> Regs;
  // The loads of the stage of band s of image n, all in flight together.
  auto load_stage = [&](Regs& rv, int n, int s) {
    const int oh0 = s * rg.R;
    const int rows_left = g.OH - oh0;
    const int rows_read = (rows_left < rg.R ? rows_left : rg.R) + g.KH - 1;
    const __amdgpu_buffer_rsrc_t gbuf = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(grad + (int64_t)n * g.C_out * P), (short)0, g.C_out * P * 4, DR_BUF3);
    const __amdgpu_buffer_rsrc_t xbuf = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + (int64_t)n * g.C * HW), (short)0, g.C * HW * 4, DR_BUF3);
    if constexpr (VEC) {
      const uint32_t band = (uint32_t)(oh0 * g.OW) * 4u;
#pragma unroll
      for (int u = 0; u < DR_GU; ++u) {
        const uint32_t off = grow[u] < rows_left ? gbase[u] + band : DR_OOB;
        rv.g[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gbuf, off, 0, 0));
      }
      if constexpr (WGT) {
#pragma unroll
        for (int u = 0; u < XJ; ++u) {
          const int hi = oh0 - g.ph + xrr[u];
          const uint32_t off = (xrr[u] < rows_read && hi >= 0 && hi < g.H)
                                   ? xcb[u] + (uint32_t)(hi * g.W) * 4u : DR_OOB;
          rv.x[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xbuf, off, 0, 0));
        }
      }
    } else {
      // byte offsets of this lane's slots within a channel
      uint32_t goff[2], xoff[XJ];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        goff[j] = (gk[j] < DR_K && gr[j] < rows_left)
                      ? (uint32_t)(oh0 * g.OW + lane + 64 * j) * 4u : DR_OOB;
#pragma unroll
      for (int j = 0; j < XJ; ++j) {
        const int hi = (xr[j] < rows_read && xw[j] >= 0)
                           ? pad_index(oh0 - g.ph + xr[j], g.H, g.pad_mode) : -1;
        xoff[j] = hi >= 0 ? (uint32_t)(hi * g.W + xw[j]) * 4u : DR_OOB;
      }
#pragma unroll
      for (int k = 0; k < 2 * DR_GC; ++k)
        rv.g[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                gbuf, goff[k & 1] + gch[k >> 1], 0, 0));
      if constexpr (WGT) {
#pragma unroll
        for (int k = 0; k < DR_XC * XJ; ++k)
          rv.x[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  xbuf, xoff[k % XJ] + xch[k / XJ], 0, 0));
      }
    }
  };
  // this lane's share of the stage's grad sums
  auto add_bias = [&](const Regs& rv) {
    if constexpr (VEC) {
#pragma unroll
      for (int u = 0; u < DR_GU; ++u) bsum[u] += (rv.g[u][0] + rv.g[u][1]) + (rv.g[u][2] + rv.g[u][3]);
    } else {
#pragma unroll
      for (int k = 0; k < 2 * DR_GC; ++k) bsum[k >> 1] += rv.g[k];
    }
  };
  // the next stage to load (image ln, band ls), stepped after each load
  int ln = (int)(t_begin / rg.spi), ls = (int)(t_begin - (int64_t)ln * rg.spi);
  auto load_next = [&](Regs& rv) {
    load_stage(rv, ln, ls);
    if (++ls == rg.spi) {
      ls = 0;
      ++ln;
    }
  };

  Regs rv0, rv1;
  if constexpr (!WGT) {
    // grad_bias only: the stages' grad values, no products
    for (int64_t t = t_begin; t < t_end; ++t) {
      load_next(rv0);
      add_bias(rv0);
    }
  }
  // stage t: its registers into LDS, stage t + 2's loads into the same
  // registers, the products
  auto run_stage = [&](Regs& rv, int64_t t) {
    __syncthreads();  // the previous stage's fragment reads are done
    if constexpr (BIAS) add_bias(rv);
    if constexpr (VEC) {
#pragma unroll
      for (int u = 0; u < DR_GU; ++u) {
        if (gdst[u] < 0) continue;
        const f32x2 lo = {rv.g[u][0], rv.g[u][1]}, hi = {rv.g[u][2], rv.g[u][3]};
        *reinterpret_cast<u32x2b*>(Gs + gdst[u]) =
            u32x2b{__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                   __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2))};
      }
#pragma unroll
      for (int u = 0; u < XJ; ++u) {
        if (xdst[u] < 0) continue;
        const f32x2 lo = {rv.x[u][0], rv.x[u][1]}, hi = {rv.x[u][2], rv.x[u][3]};
        uint32_t* d = reinterpret_cast<uint32_t*>(Xs + xdst[u]);
        d[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2));
        d[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2));
      }
    } else {
#pragma unroll
      for (int k = 0; k < 2 * DR_GC; ++k) {
        const int co_l = wave + DR_WAVES * (k >> 1);
        if (co_l < 64) Gs[co_l * GP + gk[k & 1]] = (__bf16)rv.g[k];
      }
#pragma unroll
      for (int k = 0; k < DR_XC * XJ; ++k) {
        const int c_l = wave + DR_WAVES * (k / XJ);
        if (c_l < 32) Xs[c_l * rg.cp + xk[k % XJ]] = (__bf16)rv.x[k];
      }
    }
    if (t + 2 < t_end) load_next(rv);
    __syncthreads();
    if (tap >= rg.taps) return;
    // wave `tap`: 8 k-steps of 16 pixels, both 32-channel co tiles; B starts
    // at staged column ow + sft
    const int sft = kw - g.pw + rg.xo;
    const uint32_t* xd = reinterpret_cast<const uint32_t*>(Xs) + (lane & 31) * (rg.cp >> 1) +
                         (sft >> 1);
#pragma unroll
    for (int st = 0; st < DR_K / 16; ++st) {
      const int k0 = st * 16 + half * 8;
      const int r = (st * 16) / rg.OWP, ow0 = st * 16 - r * rg.OWP + half * 8;
      const uint32_t* p = xd + (((r + kh) * rg.XW + ow0) >> 1);
      uint32_t d[5];
#pragma unroll
      for (int i = 0; i < 5; ++i) d[i] = p[i];
      uint32_t bw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) bw[i] = (sft & 1) ? __builtin_amdgcn_alignbit(d[i + 1], d[i], 16) : d[i];
      const bf16x8 b = __builtin_bit_cast(bf16x8, bw);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(Gs + (i * 32 + (lane & 31)) * GP + k0);
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i], 0, 0, 0);
      }
    }
  };
  if constexpr (WGT) {
    if (t_begin < t_end) load_next(rv0);
    if (t_begin + 1 < t_end) load_next(rv1);
    for (int64_t t = t_begin; t < t_end; t += 2) {
      run_stage(rv0, t);
      if (t + 1 < t_end) run_stage(rv1, t + 1);
    }
  }
  if constexpr (BIAS && VEC) {
    // the quads of each channel added in band order
    float* red = reinterpret_cast<float*>(dr_lds);
    __syncthreads();  // the last stage's fragment reads are done
#pragma unroll
    for (int u = 0; u < DR_GU; ++u) {
      const int it = tid + NT * u;
      if (it < 64 * q4) red[it] = bsum[u];
    }
    __syncthreads();
    if (cb == 0 && tid < 64 && co0 + tid < g.C_out) {
      float v = 0.0f;
      for (int q = 0; q < q4; ++q) v += red[tid * q4 + q];
      bpart[(int64_t)chunk * g.C_out + co0 + tid] = v;
    }
  } else if constexpr (BIAS) {
    // channel co_l = wave + i * DR_WAVES: the wave's 64 lanes added
#pragma unroll
    for (int i = 0; i < DR_GC; ++i) {
      float v = bsum[i];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
      const int co_l = wave + DR_WAVES * i;
      if (cb == 0 && lane == 0 && co_l < 64 && co0 + co_l < g.C_out)
        bpart[(int64_t)chunk * g.C_out + co0 + co_l] = v;
    }
  }
  if (!WGT || tap >= rg.taps) return;
  // lane holds input channel c0 + (lane & 31), output channel rows
  // 8*(r/4) + 4*half + r%4 of tile i; the partial is stored as
  // [chunk][tap][co][c] (a half-wave writes 32 consecutive c), which the
  // column sum permutes into [co][c][kh][kw]
  float* pc = part + ((int64_t)chunk * rg.taps + tap) * g.C_out * g.C;
  const int c = c0 + (lane & 31);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int co = co0 + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
      if (co < g.C_out && c < g.C) pc[(int64_t)co * g.C + c] = acc[i][r];
    }
}

constexpr int DR_MAX_XJ = 5;

// grad_weight and grad_bias of a one-input-channel convolution (config [5]'s
// first layer), stride 1, at most 16 window taps: as a GEMM, M = the output
// channels, N = the taps, K = the output pixels, so v_mfma_f32_16x16x32_bf16
// tiles fill (the general kernel's N = (c, kh, kw) would hold 9 of 64
// columns).  A unit is a band of RB output rows of one image; a workgroup
// walks a chunk of units and writes one partial.  Per unit the band's grad
// (16-byte loads of 4 pixels, bf16 in Gs[co][r * OWP + ow], rows padded to
// OWP with zeros) and its RB + KH - 1 input rows (4-byte loads, the padding
// mode resolved, Xs[rr][col], input column 0 at staged column pw) go to LDS
// from registers loaded during the previous unit's products; wave w
// multiplies 16-channel tile w: A = Gs (8 pixels of a channel, one 16-byte
// read), B = Xs[r + kh][ow + kw ..] (8 columns of tap (kh, kw) read as 5
// dwords, realigned with v_alignbit for odd kw; taps past KH*KW are 0).
// grad_bias: each lane adds its grad quads ((v0 + v1) + (v2 + v3)) per unit
// in unit order, then a channel's quads are added in band order through
// LDS.  Masked loads (rows past the image, padding, channels past C_out)
// carry an offset past the buffer and read 0.
constexpr int D1_GQ = 8;   // grad quads per lane and unit, at most
constexpr int D1_CHUNKS = 1024;  // partials (workgroups), at most
constexpr int D1_XS = 2;   // staged input slots per lane and unit, at most

struct D1Geom {
  int RB, bands, OWP, XW, rows_in, taps, co_tiles, gitems, xslots;
};

template <int MODE>
__global__ __launch_bounds__(256) void dweight_c1_kernel(
    const float* __restrict__ grad, const float* __restrict__ x, float* __restrict__ part,
    float* __restrict__ bpart, BwdGeom g, D1Geom d, int chunks) {
  constexpr bool WGT = MODE != 2, BIAS = MODE != 0;
  extern __shared__ __attribute__((aligned(16))) uint8_t d1_lds[];
  const int GPW = d.RB * d.OWP + 8;  // Gs row pitch (bf16)
  __bf16* Gs = reinterpret_cast<__bf16*>(d1_lds);
  __bf16* Xs = Gs + d.co_tiles * 16 * GPW;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int P = g.OH * g.OW, HW = g.H * g.W, OW4 = g.OW / 4;
  const int per_co = d.RB * OW4;  // grad quads of one channel in a band
  const int64_t U = (int64_t)g.N * d.bands;
  const int64_t u_begin = U * blockIdx.x / chunks, u_end = U * (blockIdx.x + 1) / chunks;

  if constexpr (WGT) {  // Gs padding columns and rows past C_out stay 0
    uint32_t* z = reinterpret_cast<uint32_t*>(d1_lds);
    for (int i = tid; i < (d.co_tiles * 16 * GPW + d.rows_in * d.XW) / 2; i += 256) z[i] = 0u;
  }
  // this lane's grad quads: item it = (channel co, band row r, quad q)
  uint32_t gb[D1_GQ];
  int grow[D1_GQ], gdst[D1_GQ];
#pragma unroll
  for (int u = 0; u < D1_GQ; ++u) {
    const int it = tid + 256 * u;
    const int co = it / per_co, rest = it - co * per_co;
    const int r = rest / OW4, q = rest - r * OW4;
    const bool live = it < d.gitems;
    gb[u] = (uint32_t)(co * P + 4 * q) * 4u;
    grow[u] = live ? r : (1 << 30);
    gdst[u] = live ? co * GPW + r * d.OWP + 4 * q : -1;
  }
  // this lane's staged input slots: slot e = (staged row rr, column col)
  int xrr[D1_XS], xwi[D1_XS];
#pragma unroll
  for (int j = 0; j < D1_XS; ++j) {
    const int e = tid + 256 * j;
    const int rr = e / d.XW, col = e - rr * d.XW;
    xrr[j] = e < d.xslots ? rr : (1 << 30);
    xwi[j] = (e < d.xslots && col < g.OW + g.KW - 1) ? pad_index(col - g.pw, g.W, g.pad_mode) : -1;
  }
  f32x4 gv[D1_GQ];
  float xv[D1_XS];
  auto load = [&](int64_t unit) {
    const int n = (int)(unit / d.bands), b = (int)(unit - (int64_t)n * d.bands);
    const int oh0 = b * d.RB, rows_left = g.OH - oh0;
    const __amdgpu_buffer_rsrc_t gr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(grad + (int64_t)n * g.C_out * P), (short)0, g.C_out * P * 4, DR_BUF3);
    const uint32_t band = (uint32_t)(oh0 * g.OW) * 4u;
#pragma unroll
    for (int u = 0; u < D1_GQ; ++u) {
      const uint32_t off = grow[u] < rows_left ? gb[u] + band + (uint32_t)(grow[u] * g.OW) * 4u : DR_OOB;
      gv[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, off, 0, 0));
    }
    if constexpr (WGT) {
      const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float*>(x + (int64_t)n * HW), (short)0, HW * 4, DR_BUF3);
      const int rows_read = (rows_left < d.RB ? rows_left : d.RB) + g.KH - 1;
#pragma unroll
      for (int j = 0; j < D1_XS; ++j) {
        const int hi = (xrr[j] < rows_read && xwi[j] >= 0)
                           ? pad_index(oh0 - g.ph + xrr[j], g.H, g.pad_mode) : -1;
        const uint32_t off = hi >= 0 ? (uint32_t)(hi * g.W + xwi[j]) * 4u : DR_OOB;
        xv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, off, 0, 0));
      }
    }
  };

  float bq[D1_GQ];
#pragma unroll
  for (int u = 0; u < D1_GQ; ++u) bq[u] = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int tap = lane & 15, kq = lane >> 4;  // B: tap column, 8-pixel group of the k-step
  const int kh = tap / g.KW, kw = tap - kh * g.KW;
  const bool tap_live = tap < d.taps;
  const bf16x8 zero8 = __builtin_bit_cast(bf16x8, make_uint4(0u, 0u, 0u, 0u));
  const int ksteps = d.RB * d.OWP / 32;
  if (u_begin < u_end) load(u_begin);
  for (int64_t unit = u_begin; unit < u_end; ++unit) {
    __syncthreads();  // the previous unit's fragment reads are done
    if constexpr (BIAS) {
#pragma unroll
      for (int u = 0; u < D1_GQ; ++u) bq[u] += (gv[u][0] + gv[u][1]) + (gv[u][2] + gv[u][3]);
    }
    if constexpr (WGT) {
#pragma unroll
      for (int u = 0; u < D1_GQ; ++u) {
        if (gdst[u] < 0) continue;
        const f32x2 lo = {gv[u][0], gv[u][1]}, hi = {gv[u][2], gv[u][3]};
        *reinterpret_cast<u32x2b*>(Gs + gdst[u]) =
            u32x2b{__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                   __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2))};
      }
#pragma unroll
      for (int j = 0; j < D1_XS; ++j) {
        const int e = tid + 256 * j;
        if (e < d.xslots) Xs[e] = (__bf16)xv[j];
      }
    }
    if (unit + 1 < u_end) load(unit + 1);
    if constexpr (WGT) {
      __syncthreads();
      if (wave < d.co_tiles) {
        const __bf16* ga = Gs + (wave * 16 + (lane & 15)) * GPW + 8 * kq;
        for (int st = 0; st < ksteps; ++st) {
          const int k0 = st * 32;
          const int r = k0 / d.OWP, ow0 = k0 - r * d.OWP + 8 * kq;
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(ga + k0);
          bf16x8 bfr = zero8;
          if (tap_live) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(Xs) +
                                (((r + kh) * d.XW + ow0 + kw) >> 1);
            uint32_t dd[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) dd[i] = p[i];
            uint32_t bw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) bw[i] = (kw & 1) ? __builtin_amdgcn_alignbit(dd[i + 1], dd[i], 16) : dd[i];
            bfr = __builtin_bit_cast(bf16x8, bw);
          }
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bfr, acc, 0, 0, 0);
        }
      }
    }
  }
  if constexpr (BIAS) {
    // a channel's quads added in band order
    float* red = reinterpret_cast<float*>(d1_lds);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < D1_GQ; ++u) {
      const int it = tid + 256 * u;
      if (it < d.gitems) red[it] = bq[u];
    }
    __syncthreads();
    if (tid < g.C_out) {
      float v = 0.0f;
      for (int i = 0; i < per_co; ++i) v += red[tid * per_co + i];
      bpart[(int64_t)blockIdx.x * g.C_out + tid] = v;
    }
  }
  if constexpr (WGT) {
    // lane holds channels 16 w + 4 kq + i (i < 4) of tap `tap`: the partial
    // is [chunk][co][tap], grad_weight's own layout (one input channel)
    if (wave < d.co_tiles && tap_live) {
      float* pc = part + (int64_t)blockIdx.x * g.C_out * d.taps;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int co = wave * 16 + 4 * kq + i;
        if (co < g.C_out) pc[co * d.taps + tap] = acc[i];
      }
    }
  }
}

// The one-input-channel path applies (its LDS bytes), or 0.
size_t c1_geometry(const BwdGeom& g, D1Geom& d) {
  const int taps = g.KH * g.KW;
  if (g.C != 1 || g.sh != 1 || g.sw != 1 || taps > 16 || g.KW > 8 || g.OW % 4 != 0 ||
      g.OW > 64 || g.C_out > 64 || g.OH < 1)
    return 0;
  if ((int64_t)g.C_out * g.OH * g.OW * 4 >= ((int64_t)1 << 30)) return 0;
  d = D1Geom{};
  d.OWP = g.OW <= 32 ? 32 : 64;
  d.taps = taps;
  d.co_tiles = (g.C_out + 15) / 16;
  // band rows: a multiple of 32 pixels per channel row, the band's grad quads
  // within D1_GQ per lane and its input slots within D1_XS per lane
  d.RB = std::min(g.OH, 8);
  d.XW = d.OWP + 8;
  for (;; --d.RB) {
    if (d.RB < 1) return 0;
    d.rows_in = d.RB + g.KH - 1;
    d.gitems = g.C_out * d.RB * (g.OW / 4);
    d.xslots = d.rows_in * d.XW;
    if (d.gitems <= 256 * D1_GQ && d.xslots <= 256 * D1_XS) break;
  }
  d.bands = (g.OH + d.RB - 1) / d.RB;
  // (+16 bytes: a fragment read of the last staged row's last columns runs
  // one dword past them)
  const size_t bytes = ((size_t)d.co_tiles * 16 * (d.RB * d.OWP + 8) + (size_t)d.rows_in * d.XW) * 2 + 16;
  return std::max(bytes, (size_t)d.gitems * 4);
}


// The stride-1 rows path applies (its LDS bytes, input items or slots per
// lane XJ, and whether its staging is VEC), or 0.  aligned: grad and x start
// on 16 bytes (always through the C ABI, which requires it).
size_t rows_geometry(const BwdGeom& g, bool aligned, RowsGeom& rg, int& xj, bool& vec) {
  const int taps = g.KH * g.KW;
  // (fewer than 16 input channels leave most of the 32-channel tile idle: a
  // 1-channel 28x28 batch of 256 takes ~33 us here against 16.5 on dweight_kernel)
  // (at most DR_WAVES taps, one wave each)
  if (g.sh != 1 || g.sw != 1 || taps < 8 || taps > DR_WAVES || g.KW > 8 || g.OW > 64 || g.C < 16)
    return 0;
  // 32-bit buffer offsets: an image's grad and input stay below 1 GiB
  if ((int64_t)g.C_out * g.OH * g.OW * 4 >= (1 << 30) || (int64_t)g.C * g.H * g.W * 4 >= (1 << 30))
    return 0;
  rg.OWP = g.OW <= 16 ? 16 : g.OW <= 32 ? 32 : 64;
  rg.R = DR_K / rg.OWP;
  rg.XW = rg.OWP + 8;
  rg.rows_in = rg.R + g.KH - 1;
  rg.taps = taps;
  const int xslots = rg.rows_in * rg.XW;
  rg.cp = xslots + 2;  // odd dword pitch; slot xslots is the spare
  rg.spi = (g.OH + rg.R - 1) / rg.R;
  // VEC: input quads per lane; xo even (4-byte LDS writes), so xo + W and
  // the columns the products read stay within XW (stride 1, KW <= 8)
  const int vitems = 32 * rg.rows_in * (g.W / 4);
  const int vj = std::max(2, (vitems + DR_WAVES * 64 - 1) / (DR_WAVES * 64));
  vec = aligned && g.pad_mode == NOVAQ_PAD_ZEROS && g.W % 4 == 0 && g.OW % 4 == 0 &&
        vj <= DR_MAX_XJ;
  rg.xo = vec ? (g.pw + 1) & ~1 : g.pw;
  xj = vec ? vj : (xslots + 63) / 64;
  if (xj < 2 || xj > DR_MAX_XJ) return 0;  // (more slots per lane spill registers)
  const size_t bytes = (size_t)64 * (DR_K + 8) * 2 + (size_t)32 * rg.cp * 2;
  return bytes <= 150 * 1024 ? bytes : 0;
}

// grad_input as the forward convolution of grad with the flipped weights
bool flip_path(const BwdGeom& g) { return g.sh == 1 && g.sw == 1 && g.ph < g.KH && g.pw < g.KW; }

int64_t flip_items(const BwdGeom& g, int wt) {
  const int64_t total = (int64_t)g.C_out * g.C * g.KH * g.KW;
  return wt == E2M1 ? (total + 1) / 2 : total;
}

template <int COLS>
int launch_finish_cols(FinishArgs a, int wt, const BwdGeom& g, hipStream_t stream) {
  const int64_t wb = (a.wcols + COLS - 1) / COLS, bb = (a.bcols + COLS - 1) / COLS;
  const int64_t fb = (a.flip_items + 1023) / 1024;
  const int64_t blocks = wb + bb + fb;
  if (blocks == 0) return NOVAQ_OK;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  a.wb = (unsigned)wb;
  a.bb = (unsigned)bb;
  const dim3 grid((unsigned)blocks), block(1024);
  switch (wt) {
    case E4M3: hipLaunchKernelGGL((finish_kernel<E4M3, COLS>), grid, block, 0, stream, a, g.C_out, g.C, g.KH, g.KW); break;
    case E5M2: hipLaunchKernelGGL((finish_kernel<E5M2, COLS>), grid, block, 0, stream, a, g.C_out, g.C, g.KH, g.KW); break;
    case E2M1: hipLaunchKernelGGL((finish_kernel<E2M1, COLS>), grid, block, 0, stream, a, g.C_out, g.C, g.KH, g.KW); break;
    case BF16: hipLaunchKernelGGL((finish_kernel<BF16, COLS>), grid, block, 0, stream, a, g.C_out, g.C, g.KH, g.KW); break;
    case F16: hipLaunchKernelGGL((finish_kernel<F16, COLS>), grid, block, 0, stream, a, g.C_out, g.C, g.KH, g.KW); break;
    case F32: hipLaunchKernelGGL((finish_kernel<F32, COLS>), grid, block, 0, stream, a, g.C_out, g.C, g.KH, g.KW); break;
    default: return NOVAQ_EDTYPE;
  }
  return check_launch();
}

// With one input channel (C == 1: the one-input-channel kernel's up to
// D1_CHUNKS partials of C_out x taps columns) the sums take 16 columns a
// workgroup, otherwise 64.
int launch_finish(FinishArgs a, int wt, const BwdGeom& g, hipStream_t stream) {
  return g.C == 1 ? launch_finish_cols<16>(a, wt, g, stream) : launch_finish_cols<64>(a, wt, g, stream);
}

// grad_input of a one-input-channel convolution as the one-output-channel
// kernel's convolution of grad (N, C_out, OH, OW) -> (N, 1, H, W) with the
// flipped weight and zero padding (KH-1-ph, KW-1-pw): its band geometry, or
// false when that convolution would run on another kernel (a few output
// channels of the layer, C_out <= SC_MAX_C, take the small-channel kernel).
bool c1_tail_geometry(const BwdGeom& g, Co1Geom& cg, size_t& lds) {
  if (g.C != 1 || !flip_path(g) || g.C_out <= SC_MAX_C) return false;
  ConvGeom fg{};
  fg.N = g.N; fg.C = g.C_out; fg.H = g.OH; fg.W = g.OW; fg.C_out = 1;
  fg.KH = g.KH; fg.KW = g.KW; fg.sh = 1; fg.sw = 1;
  fg.ph = g.KH - 1 - g.ph; fg.pw = g.KW - 1 - g.pw; fg.pad_mode = NOVAQ_PAD_ZEROS;
  fg.OH = g.H; fg.OW = g.W;
  return co1_geometry(fg, cg, lds);
}

template <int WT>
int launch_c1_tail(FinishArgs a, const float* grad, const void* w, const float* w_scale,
                   float* gi, const BwdGeom& g, const Co1Geom& cg, size_t lds,
                   hipStream_t stream) {
  const int64_t wb = (a.wcols + 3) / 4, bb = (a.bcols + 3) / 4;
  const int64_t blocks = wb + bb + (int64_t)g.N * cg.bands;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  a.wb = (unsigned)wb;
  a.bb = (unsigned)bb;
  hipLaunchKernelGGL(c1_tail_kernel<WT>, dim3((unsigned)blocks), dim3(256),
                     std::max(lds, (size_t)(64 * 4 * sizeof(float))), stream, a, grad,
                     static_cast<const uint8_t*>(w), w_scale, gi, cg);
  return check_launch();
}

// wf holds the flipped weights when flip_path(g) (the finishing launch wrote
// them); the direct kernel covers the rest.
template <int WT>
int launch_dinput(const float* grad, const void* w, const void* wf, const float* w_scale,
                  float* gi, const BwdGeom& g, hipStream_t stream) {
  if (flip_path(g)) {
    const int rc = conv2d_launch(grad, g.N, g.C_out, g.OH, g.OW, wf, WT, w_scale, g.C, g.KH, g.KW,
                                 1, 1, g.KH - 1 - g.ph, g.KW - 1 - g.pw, NOVAQ_PAD_ZEROS, nullptr,
                                 gi, stream);
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

// Workspace layout of conv2d_backward (each part 256-byte aligned), sized
// for the largest chunk count a launch uses.
ConvBwdWs conv2d_bwd_workspace(int64_t N, int64_t C, int64_t C_out, int KH, int KW, int w_dtype,
                               int cus) {
  ConvBwdWs ws{};
  auto a256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const int64_t ckk = C * KH * KW;
  const int64_t co_blocks = (C_out + DW_M - 1) / DW_M, j_blocks = (ckk + DW_N - 1) / DW_N;
  // enough chunks of (image, 64-pixel stage) pairs for about DW_PER_CU
  // workgroups per CU (resident waves hide the gathers' latency), a multiple
  // of 8 for the XCD mapping; a launch uses fewer when there are fewer stages
  // (at most DW_MAX_CHUNKS: the partials are summed by a column sum whose
  // cost grows with their number)
  int64_t want = std::max<int64_t>(1, ((int64_t)DW_PER_CU * cus + co_blocks * j_blocks - 1) /
                                          (co_blocks * j_blocks));
  want = std::min<int64_t>(want, DW_MAX_CHUNKS);
  if (want >= 8) want = (want + 7) / 8 * 8;
  (void)N;
  // one input channel: room for up to D1_CHUNKS partials of C_out x taps
  // (the one-input-channel kernel's units, one per workgroup)
  if (C == 1) want = std::max<int64_t>(want, D1_CHUNKS);
  ws.chunks = (int)want;
  ws.wf = 0;
  ws.part = a256(((size_t)C_out * ckk * dtype_bits(w_dtype) + 7) / 8);
  ws.bpart = ws.part + a256((size_t)ws.chunks * C_out * ckk * 4);
  ws.total = ws.bpart + a256((size_t)ws.chunks * C_out * 4);
  return ws;
}

// grad_weight and grad_bias partials: the stride-1 rows kernel or the general
// implicit GEMM, one partial per chunk; fa receives what the finishing
// launch sums.
static int dweight_launch(const float* grad, const float* x, const BwdGeom& g, int64_t chunks,
                          const ConvBwdWs& ws, uint8_t* base, float* grad_weight,
                          float* grad_bias, FinishArgs& fa, hipStream_t stream) {
  if (!grad_weight && !grad_bias) return NOVAQ_OK;
  const int64_t C = g.C, C_out = g.C_out;
  const int64_t ckk = C * g.KH * g.KW;
  // one input channel: the taps as the GEMM's N (a bias-only call runs the
  // bias-only mode over the same chunks, so its bits match a full call's)
  D1Geom d1{};
  const size_t c1_lds = c1_geometry(g, d1);
  if (c1_lds) {
    float* part = reinterpret_cast<float*>(base + ws.part);
    float* bpart = reinterpret_cast<float*>(base + ws.bpart);
    const int64_t units = (int64_t)g.N * d1.bands;
    const int64_t rchunks = std::max<int64_t>(1, std::min<int64_t>(ws.chunks, units));
    if (rchunks > 0x7FFFFFFF) return NOVAQ_EINVAL;
    const int mode = grad_weight ? (grad_bias ? 1 : 0) : 2;
    const dim3 grid((unsigned)rchunks);
    if (mode == 0)
      hipLaunchKernelGGL((dweight_c1_kernel<0>), grid, dim3(256), c1_lds, stream, grad, x, part, bpart, g, d1, (int)rchunks);
    else if (mode == 1)
      hipLaunchKernelGGL((dweight_c1_kernel<1>), grid, dim3(256), c1_lds, stream, grad, x, part, bpart, g, d1, (int)rchunks);
    else
      hipLaunchKernelGGL((dweight_c1_kernel<2>), grid, dim3(256), c1_lds, stream, grad, x, part, bpart, g, d1, (int)rchunks);
    fa.rows = rchunks;
    if (grad_weight) {
      fa.part = part;
      fa.gw = grad_weight;
      fa.wcols = C_out * ckk;
    }
    if (grad_bias) {
      fa.bpart = bpart;
      fa.gb = grad_bias;
      fa.bcols = C_out;
    }
    return check_launch();
  }
  // stride-1 convolutions with short rows: grad_weight and grad_bias on the
  // rows kernel (a bias-only call runs its bias-only mode over the same
  // chunks, so its bits match a full call's)
  RowsGeom rg{};
  int xj = 0;
  bool vec = false;
  const bool aligned = ((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(x)) & 15) == 0;
  const size_t rows_lds = rows_geometry(g, aligned, rg, xj, vec);
  if (rows_lds) {
    float* part = reinterpret_cast<float*>(base + ws.part);
    float* bpart = reinterpret_cast<float*>(base + ws.bpart);
    const int64_t co_blocks = (C_out + 63) / 64, c_blocks = (C + 31) / 32;
    const int64_t units = (int64_t)g.N * rg.spi;
    // about one workgroup per CU: the chunk partials cost HBM traffic
    int64_t rchunks = std::max<int64_t>(1, device_cu_count() / (co_blocks * c_blocks));
    rchunks = std::min<int64_t>(std::min<int64_t>(rchunks, ws.chunks), std::max<int64_t>(units, 1));
    const int mode = grad_weight ? (grad_bias ? 1 : 0) : 2;
    const int64_t blocks = rchunks * co_blocks * (mode == 2 ? 1 : c_blocks);
    if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
    using RowsKernel = void (*)(const float*, const float*, float*, float*, BwdGeom, RowsGeom,
                                int, int, int);
    static const RowsKernel kerns[2][2][DR_MAX_XJ + 1] = {
        {{nullptr, nullptr, dweight_rows_kernel<2, 0, false>, dweight_rows_kernel<3, 0, false>,
          dweight_rows_kernel<4, 0, false>, dweight_rows_kernel<5, 0, false>},
         {nullptr, nullptr, dweight_rows_kernel<2, 1, false>, dweight_rows_kernel<3, 1, false>,
          dweight_rows_kernel<4, 1, false>, dweight_rows_kernel<5, 1, false>}},
        {{nullptr, nullptr, dweight_rows_kernel<2, 0, true>, dweight_rows_kernel<3, 0, true>,
          dweight_rows_kernel<4, 0, true>, dweight_rows_kernel<5, 0, true>},
         {nullptr, nullptr, dweight_rows_kernel<2, 1, true>, dweight_rows_kernel<3, 1, true>,
          dweight_rows_kernel<4, 1, true>, dweight_rows_kernel<5, 1, true>}}};
    static bool lds_raised[2][2][DR_MAX_XJ + 1] = {};
    if (mode == 2) {
      // the same grad reads and sums as a full call (VEC: the quads' sums
      // meet in LDS)
      const size_t red = vec ? (size_t)64 * (rg.R * g.OW / 4) * 4 : 0;
      if (vec)
        hipLaunchKernelGGL((dweight_rows_kernel<2, 2, true>), dim3((unsigned)blocks),
                           dim3(DR_WAVES * 64), red, stream, grad, x, part, bpart, g, rg,
                           (int)rchunks, (int)co_blocks, 1);
      else
        hipLaunchKernelGGL((dweight_rows_kernel<2, 2, false>), dim3((unsigned)blocks),
                           dim3(DR_WAVES * 64), 0, stream, grad, x, part, bpart, g, rg,
                           (int)rchunks, (int)co_blocks, 1);
    } else {
      const RowsKernel kern = kerns[vec][mode][xj];
      if (!lds_raised[vec][mode][xj]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 150 * 1024);
        if (e != hipSuccess) return hip_fail(e);
        lds_raised[vec][mode][xj] = true;
      }
      hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(DR_WAVES * 64), rows_lds, stream, grad,
                         x, part, bpart, g, rg, (int)rchunks, (int)co_blocks, (int)c_blocks);
    }
    fa.rows = rchunks;
    if (grad_weight) {
      fa.part = part;
      fa.gw = grad_weight;
      fa.wcols = C_out * ckk;
      fa.pt = (int)rg.taps;
      fa.pco = (int)C_out;
      fa.pc = (int)C;
    }
    if (grad_bias) {
      fa.bpart = bpart;
      fa.gb = grad_bias;
      fa.bcols = C_out;
    }
    return check_launch();
  }
  float* part = reinterpret_cast<float*>(base + ws.part);
  float* bpart = grad_bias ? reinterpret_cast<float*>(base + ws.bpart) : nullptr;
  const int64_t co_blocks = (C_out + DW_M - 1) / DW_M;
  const int64_t j_blocks = grad_weight ? (ckk + DW_N - 1) / DW_N : 1;
  if (co_blocks > 65535 || j_blocks > 65535) return NOVAQ_EINVAL;
  const int64_t blocks = chunks * co_blocks * j_blocks;
  if (blocks > 0x7FFFFFFF) return NOVAQ_EINVAL;
  const dim3 grid((unsigned)blocks);
  const bool zp = g.pad_mode == NOVAQ_PAD_ZEROS;
  // buffer loads: pairs whole (P even), per-image offsets within 31 bits
  const bool buf = (g.OH * g.OW) % 2 == 0 && C_out * g.OH * g.OW * 4 < ((int64_t)1 << 30) &&
                   C * g.H * g.W * 4 < ((int64_t)1 << 30);
  auto kern = grad_weight
                  ? (zp ? (buf ? dweight_kernel<true, false, true> : dweight_kernel<true, false, false>)
                        : (buf ? dweight_kernel<false, false, true> : dweight_kernel<false, false, false>))
                  : (buf ? dweight_kernel<true, true, true> : dweight_kernel<true, true, false>);
  hipLaunchKernelGGL(kern, grid, dim3(DW_THREADS), 0, stream, grad, x, part, bpart, g, (int)ckk,
                     (int)chunks, (int)co_blocks, (int)j_blocks);
  // partials added over the chunks in a fixed order by the finishing launch
  fa.rows = chunks;
  if (grad_weight) {
    fa.part = part;
    fa.gw = grad_weight;
    fa.wcols = C_out * ckk;
  }
  if (grad_bias) {
    fa.bpart = bpart;
    fa.gb = grad_bias;
    fa.bcols = C_out;
  }
  return check_launch();
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
  // chunks for this launch: at most one per (image, stage) pair, rounded up to
  // a multiple of 8 when at least 8 (never above ws.chunks, itself such a
  // multiple); chunks past the last stage add zeros
  const int64_t T = N * (((int64_t)g.OH * g.OW + DW_K - 1) / DW_K);
  int64_t chunks = std::min<int64_t>(std::min<int64_t>(ws.chunks, DW_MAX_CHUNKS), std::max<int64_t>(T, 1));
  if (chunks >= 8) chunks = (chunks + 7) / 8 * 8;
  switch (w_dtype) {
    case E4M3: case E5M2: case E2M1: case BF16: case F16: case F32: break;
    default: return NOVAQ_EDTYPE;
  }
  uint8_t* base = static_cast<uint8_t*>(workspace);
  void* wf = base + ws.wf;
  int rc = NOVAQ_OK;
  // order: the weight-gradient kernel, one finishing launch (its column sums
  // and the weight flip), then grad_input's convolution
  FinishArgs fa{};
  fa.w = static_cast<const uint8_t*>(w_q);
  fa.wf = static_cast<uint8_t*>(wf);
  // one input channel: the sums and grad_input in one last launch (no flip)
  Co1Geom cg{};
  size_t co1_lds = 0;
  const bool tail = grad_input && N > 0 && c1_tail_geometry(g, cg, co1_lds);
  fa.flip_items = grad_input && N > 0 && flip_path(g) && !tail ? flip_items(g, w_dtype) : 0;
  rc = dweight_launch(grad, x, g, chunks, ws, base, grad_weight, grad_bias, fa, stream);
  if (rc != NOVAQ_OK) return rc;
  if (tail) {
    switch (w_dtype) {
      case E4M3: return launch_c1_tail<E4M3>(fa, grad, w_q, w_scale, grad_input, g, cg, co1_lds, stream);
      case E5M2: return launch_c1_tail<E5M2>(fa, grad, w_q, w_scale, grad_input, g, cg, co1_lds, stream);
      case E2M1: return launch_c1_tail<E2M1>(fa, grad, w_q, w_scale, grad_input, g, cg, co1_lds, stream);
      case BF16: return launch_c1_tail<BF16>(fa, grad, w_q, w_scale, grad_input, g, cg, co1_lds, stream);
      case F16: return launch_c1_tail<F16>(fa, grad, w_q, w_scale, grad_input, g, cg, co1_lds, stream);
      default: return launch_c1_tail<F32>(fa, grad, w_q, w_scale, grad_input, g, cg, co1_lds, stream);
    }
  }
  rc = launch_finish(fa, w_dtype, g, stream);
  if (rc != NOVAQ_OK || !grad_input || N == 0) return rc;
  switch (w_dtype) {
    case E4M3: return launch_dinput<E4M3>(grad, w_q, wf, w_scale, grad_input, g, stream);
    case E5M2: return launch_dinput<E5M2>(grad, w_q, wf, w_scale, grad_input, g, stream);
    case E2M1: return launch_dinput<E2M1>(grad, w_q, wf, w_scale, grad_input, g, stream);
    case BF16: return launch_dinput<BF16>(grad, w_q, wf, w_scale, grad_input, g, stream);
    case F16: return launch_dinput<F16>(grad, w_q, wf, w_scale, grad_input, g, stream);
    default: return launch_dinput<F32>(grad, w_q, wf, w_scale, grad_input, g, stream);
  }
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free backward (novaq_conv2d_backward_noalloc): a
// file-scope device array, so every GPU the library runs on holds its own
// copy from module load until the process ends.  In host code `scratch` only
// names the symbol; its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and used from then on.  Every
// call on a GPU shares that GPU's array: calls that overlap on one GPU (on
// different streams) race; calls in one stream's order do not.  Nothing in it
// must start at zero: the weight-gradient kernels write every partial the
// finishing launch reads, and the flip writes every flipped weight.
static __device__ __align__(256) uint8_t scratch[CONV_BWD_SCRATCH_BYTES];

int conv2d_bwd_scratch(void** ptr) {
  static std::mutex lock;
  static void* per_device[64] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  if (dev < 0 || dev >= 64) return NOVAQ_EINVAL;
  std::lock_guard<std::mutex> guard(lock);
  if (!per_device[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e);
    if (!p) return NOVAQ_EHIP;
    per_device[dev] = p;
  }
  *ptr = per_device[dev];
  return NOVAQ_OK;
}

}  // namespace novaq
