// C ABI of libnovaq.so (declared in include/novaq.h): argument validation,
// status codes and dispatch to the kernel launchers.  No entry point
// allocates device memory or synchronises the stream.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "novaq_convert.h"
#include "novaq_epilogue.h"
#include "novaq_internal.h"

namespace novaq {

static thread_local int g_last_hip_error = 0;

int hip_fail(hipError_t e) {
  g_last_hip_error = (int)e;
  return NOVAQ_EHIP;
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of novaq_linear_backward: none when grad_input reads W's codes in
// place (and the fp32 grad, rounding it while staging); otherwise W^T in W's
// format, then grad in bf16 (at gyt) where the in-place weight-gradient
// product takes the shape, else grad^T (bf16, at gyt) and x^T (bf16, at xt);
// each part 256-byte aligned.
struct LinearBwdWs {
  size_t wt, gyt, xt, total;
  bool tn, wn;
};
static LinearBwdWs linear_bwd_ws(int64_t N, int64_t D_in, int64_t D_out, int w_dtype) {
  LinearBwdWs w;
  w.tn = linear_tn_supported(D_out, D_in, N);
  w.wn = w.tn && linear_wn_supported(N, D_out, D_in, w_dtype);
  w.wt = 0;
  w.gyt = align256(((size_t)D_in * (size_t)D_out * dtype_bits(w_dtype) + 7) / 8);
  w.xt = w.gyt + align256((size_t)D_out * (size_t)N * 2);
  w.total = w.wn ? 0 : w.xt + (w.tn ? 0 : align256((size_t)D_in * (size_t)N * 2));
  return w;
}
static bool valid_dtype(int dt) { return dt >= F32 && dt <= E2M1; }

}  // namespace novaq

using namespace novaq;

extern "C" {

int novaq_version(void) { return 100; }

const char* novaq_status_string(int status) {
  switch (status) {
    case NOVAQ_OK: return "ok";
    case NOVAQ_EINVAL: return "invalid argument";
    case NOVAQ_EDTYPE: return "unsupported dtype";
    case NOVAQ_ESHAPE: return "inconsistent shapes";
    case NOVAQ_EPADMODE: return "unknown padding mode";
    case NOVAQ_EALIGN: return "buffer not 16-byte aligned";
    case NOVAQ_EHIP: return "HIP runtime error";
    case NOVAQ_ENOTSUP: return "not supported";
    case NOVAQ_ESCRATCH: return "request exceeds the static scratch of an allocation-free entry point";
    default: return "unknown status";
  }
}

int novaq_last_hip_error(void) { return g_last_hip_error; }

int novaq_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
               const float* scale, void* stream) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return NOVAQ_EDTYPE;
  if (is_quant(src_dtype) && is_quant(dst_dtype)) return NOVAQ_EDTYPE;
  if (n < 0) return NOVAQ_EINVAL;
  if (scale && !is_quant(src_dtype) && !is_quant(dst_dtype)) return NOVAQ_EINVAL;
  if (n == 0) return NOVAQ_OK;
  if (!src || !dst) return NOVAQ_EINVAL;
  if (!aligned16(src) || !aligned16(dst)) return NOVAQ_EALIGN;
  return cast_launch(src, src_dtype, dst, dst_dtype, n, scale ? 1 : 0, scale, nullptr,
                     static_cast<hipStream_t>(stream));
}

int novaq_amax(const void* x, int dtype, int64_t n, float* amax, void* stream) {
  if (dtype != F32 && dtype != F16 && dtype != BF16) return NOVAQ_EDTYPE;
  if (n < 0 || !amax || (n > 0 && !x)) return NOVAQ_EINVAL;
  if (n > 0 && !aligned16(x)) return NOVAQ_EALIGN;
  return amax_launch(x, dtype, n, amax, static_cast<hipStream_t>(stream));
}

int novaq_scale_from_amax(const float* amax, int dst_dtype, float* scale, void* stream) {
  if (!is_quant(dst_dtype)) return NOVAQ_EDTYPE;
  if (!amax || !scale) return NOVAQ_EINVAL;
  return scale_from_amax_launch(amax, dst_dtype, scale, static_cast<hipStream_t>(stream));
}

int novaq_quantize(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
                   float* amax_scale, void* stream) {
  if (src_dtype != F32 && src_dtype != F16 && src_dtype != BF16) return NOVAQ_EDTYPE;
  if (!is_quant(dst_dtype)) return NOVAQ_EDTYPE;
  if (n < 0 || !amax_scale || (n > 0 && (!src || !dst))) return NOVAQ_EINVAL;
  if (n > 0 && (!aligned16(src) || !aligned16(dst))) return NOVAQ_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = amax_launch(src, src_dtype, n, amax_scale, s);
  if (rc != NOVAQ_OK) return rc;
  if (n == 0) return scale_from_amax_launch(amax_scale, dst_dtype, amax_scale + 1, s);
  return cast_launch(src, src_dtype, dst, dst_dtype, n, 2, amax_scale, amax_scale + 1, s);
}

int novaq_pack_fp4(const float* x, int64_t n, const float* scale, uint8_t* packed,
                   void* stream) {
  return novaq_cast(x, F32, packed, E2M1, n, scale, stream);
}

int novaq_unpack_fp4(const uint8_t* packed, int64_t n, const float* scale, float* y,
                     void* stream) {
  return novaq_cast(packed, E2M1, y, F32, n, scale, stream);
}

int novaq_linear_forward(const float* x, int64_t N, int64_t D_in, const void* w_q,
                         int w_dtype, const float* w_scale, const float* bias,
                         int64_t D_out, float* y, void* stream) {
  if (!valid_dtype(w_dtype)) return NOVAQ_EDTYPE;
  if (N < 0 || D_in < 0 || D_out < 0) return NOVAQ_EINVAL;
  if (N == 0 || D_out == 0) return NOVAQ_OK;
  if (!x || !w_q || !y) return NOVAQ_EINVAL;
  if (!aligned16(x) || !aligned16(w_q) || !aligned16(y) || (bias && !aligned16(bias)))
    return NOVAQ_EALIGN;
  return linear_launch(x, N, D_in, w_q, w_dtype, w_scale, bias, D_out, y,
                       static_cast<hipStream_t>(stream));
}

int novaq_conv2d_forward(const float* x, int64_t N, int64_t C, int64_t H, int64_t W,
                         const void* w_q, int w_dtype, const float* w_scale, int64_t C_out,
                         int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode,
                         const float* bias, float* y, void* stream) {
  if (!valid_dtype(w_dtype)) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || C_out <= 0 || KH <= 0 || KW <= 0 || sh <= 0 ||
      sw <= 0 || ph < 0 || pw < 0)
    return NOVAQ_EINVAL;
  if (H + 2 * (int64_t)ph < KH || W + 2 * (int64_t)pw < KW) return NOVAQ_ESHAPE;
  if (N == 0) return NOVAQ_OK;
  if (!x || !w_q || !y) return NOVAQ_EINVAL;
  if (!aligned16(x) || !aligned16(w_q) || !aligned16(y)) return NOVAQ_EALIGN;
  return conv2d_launch(x, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh, sw, ph, pw,
                       pad_mode, bias, y, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Argument checks shared by the two Conv2d backward entry points; *need gets
// the workspace bytes the call uses (0: nothing to compute).
int conv_bwd_check(const float* grad, const float* x, int64_t N, int64_t C, int64_t H,
                   int64_t W, const void* w_q, int w_dtype, int64_t C_out, int KH, int KW,
                   int sh, int sw, int ph, int pw, int pad_mode, const float* grad_input,
                   const float* grad_weight, const float* grad_bias, size_t* need) {
  *need = 0;
  if (!valid_dtype(w_dtype)) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || C_out <= 0 || KH <= 0 || KW <= 0 || sh <= 0 ||
      sw <= 0 || ph < 0 || pw < 0)
    return NOVAQ_EINVAL;
  if (H + 2 * (int64_t)ph < KH || W + 2 * (int64_t)pw < KW) return NOVAQ_ESHAPE;
  if (N > 0x7FFFFFFF || C * H * W > 0x7FFFFFFF || C_out * C * KH * KW > 0x7FFFFFFF ||
      C_out > 0x7FFFFFFF)
    return NOVAQ_EINVAL;
  if (!grad_input && !grad_weight && !grad_bias) return NOVAQ_OK;
  if (N > 0 && !grad) return NOVAQ_EINVAL;
  if (grad_input && N > 0 && !w_q) return NOVAQ_EINVAL;
  if (grad_weight && N > 0 && !x) return NOVAQ_EINVAL;
  for (const void* p : {(const void*)grad, (const void*)x, w_q, (const void*)grad_input,
                        (const void*)grad_weight, (const void*)grad_bias})
    if (p && !aligned16(p)) return NOVAQ_EALIGN;
  *need = conv2d_bwd_workspace(N, C, C_out, KH, KW, w_dtype, device_cu_count()).total;
  return NOVAQ_OK;
}

// Device-side epilogue from the C struct (NULL: bias only, fp32 output);
// zeroes the amax output first.  Returns a status.
int make_epilogue(const float* bias, const novaq_epilogue* epi, Epilogue* ep, hipStream_t stream) {
  *ep = Epilogue{};
  ep->bias = bias;
  ep->out_dtype = F32;
  if (!epi) return NOVAQ_OK;
  switch (epi->out_dtype) {
    case F32: case F16: case BF16: case E4M3: case E5M2: break;
    default: return NOVAQ_EDTYPE;
  }
  ep->mul = epi->channel_mul;
  ep->add = epi->channel_add;
  ep->out_scale = epi->out_scale;
  ep->amax = reinterpret_cast<uint32_t*>(epi->out_amax);
  ep->relu = epi->relu != 0;
  ep->out_dtype = epi->out_dtype;
  for (const void* p : {(const void*)ep->mul, (const void*)ep->add, (const void*)ep->out_scale,
                        (const void*)ep->amax})
    if (p && (reinterpret_cast<uintptr_t>(p) & 3)) return NOVAQ_EALIGN;
  if (ep->amax) return fill_u32_launch(ep->amax, 0u, 1, stream);
  return NOVAQ_OK;
}

}  // namespace

extern "C" {

int novaq_linear_forward_ex(const void* x, int x_dtype, const float* x_scale, int64_t N,
                            int64_t D_in, const void* w_q, int w_dtype, const float* w_scale,
                            const float* bias, int64_t D_out, const novaq_epilogue* epi,
                            void* y, void* stream) {
  if (!valid_dtype(w_dtype) || !valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (N < 0 || D_in < 0 || D_out < 0) return NOVAQ_EINVAL;
  if (epi && (epi->out_dtype == E2M1 || !valid_dtype(epi->out_dtype))) return NOVAQ_EDTYPE;
  if (N == 0 || D_out == 0) return NOVAQ_OK;
  if (!x || !w_q || !y) return NOVAQ_EINVAL;
  if (!aligned16(x) || !aligned16(w_q) || !aligned16(y) || (bias && !aligned16(bias)))
    return NOVAQ_EALIGN;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  Epilogue ep;
  const int rc = make_epilogue(bias, epi, &ep, st);
  if (rc != NOVAQ_OK) return rc;
  return linear_launch(x, x_dtype, x_scale, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, st);
}

int novaq_conv2d_forward_ex(const void* x, int x_dtype, const float* x_scale, int64_t N,
                            int64_t C, int64_t H, int64_t W, const void* w_q, int w_dtype,
                            const float* w_scale, int64_t C_out, int KH, int KW, int sh, int sw,
                            int ph, int pw, int pad_mode, const float* bias,
                            const novaq_epilogue* epi, void* y, void* stream) {
  if (!valid_dtype(w_dtype) || !valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || C_out <= 0 || KH <= 0 || KW <= 0 || sh <= 0 ||
      sw <= 0 || ph < 0 || pw < 0)
    return NOVAQ_EINVAL;
  if (epi && (epi->out_dtype == E2M1 || !valid_dtype(epi->out_dtype))) return NOVAQ_EDTYPE;
  if (H + 2 * (int64_t)ph < KH || W + 2 * (int64_t)pw < KW) return NOVAQ_ESHAPE;
  if (N == 0) return NOVAQ_OK;
  if (!x || !w_q || !y) return NOVAQ_EINVAL;
  if (!aligned16(x) || !aligned16(w_q) || !aligned16(y)) return NOVAQ_EALIGN;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  Epilogue ep;
  const int rc = make_epilogue(bias, epi, &ep, st);
  if (rc != NOVAQ_OK) return rc;
  return conv2d_launch(x, x_dtype, x_scale, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh,
                       sw, ph, pw, pad_mode, ep, y, st);
}

int novaq_max_pool2d(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W,
                     int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode, void* y,
                     void* stream) {
  if (!valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || sh <= 0 || sw <= 0 ||
      ph < 0 || pw < 0)
    return NOVAQ_EINVAL;
  if (H + 2 * (int64_t)ph < KH || W + 2 * (int64_t)pw < KW) return NOVAQ_ESHAPE;
  if (H > 0x7FFFFFFF || W > 0x7FFFFFFF) return NOVAQ_EINVAL;
  if (N == 0) return NOVAQ_OK;
  if (!x || !y) return NOVAQ_EINVAL;
  const uintptr_t eb = (uintptr_t)dtype_bits(x_dtype) / 8;  // element-aligned views only
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % eb) return NOVAQ_EALIGN;
  return max_pool2d_launch(x, x_dtype, N, C, H, W, KH, KW, sh, sw, ph, pw, pad_mode, y,
                           static_cast<hipStream_t>(stream));
}

int novaq_global_avg_pool2d(const void* x, int x_dtype, const float* x_scale, int64_t N,
                            int64_t C, int64_t H, int64_t W, float* y, void* stream) {
  if (!valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (x_scale && !is_quant(x_dtype)) return NOVAQ_EDTYPE;  // a scale belongs to FP8 codes
  if (N < 0 || C <= 0 || H <= 0 || W <= 0) return NOVAQ_EINVAL;
  if (N == 0) return NOVAQ_OK;
  if (!x || !y) return NOVAQ_EINVAL;
  // the plane loads are 4-element vectors wherever the plane offset allows
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(y) & 3) ||
      (x_scale && (reinterpret_cast<uintptr_t>(x_scale) & 3)))
    return NOVAQ_EALIGN;
  return global_avg_pool2d_launch(x, x_dtype, x_scale, N * C, H * W, y,
                                  static_cast<hipStream_t>(stream));
}

int novaq_max_pool2d_backward(const float* grad, const void* x, int x_dtype, int64_t N,
                              int64_t C, int64_t H, int64_t W, int KH, int KW, int sh, int sw,
                              int ph, int pw, int pad_mode, float* grad_input, void* stream) {
  if (!valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || sh <= 0 || sw <= 0 ||
      ph < 0 || pw < 0)
    return NOVAQ_EINVAL;
  if (H + 2 * (int64_t)ph < KH || W + 2 * (int64_t)pw < KW) return NOVAQ_ESHAPE;
  if (H > 0x7FFFFFFF || W > 0x7FFFFFFF) return NOVAQ_EINVAL;
  if (N == 0) return NOVAQ_OK;
  if (!grad || !x || !grad_input) return NOVAQ_EINVAL;
  const uintptr_t eb = (uintptr_t)dtype_bits(x_dtype) / 8;  // element-aligned views only
  if (reinterpret_cast<uintptr_t>(x) % eb ||
      ((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(grad_input)) & 3))
    return NOVAQ_EALIGN;
  return max_pool2d_backward_launch(grad, x, x_dtype, N, C, H, W, KH, KW, sh, sw, ph, pw,
                                    pad_mode, grad_input, static_cast<hipStream_t>(stream));
}

int novaq_global_avg_pool2d_backward(const float* grad, int64_t N, int64_t C, int64_t H,
                                     int64_t W, float* grad_input, void* stream) {
  if (N < 0 || C <= 0 || H <= 0 || W <= 0) return NOVAQ_EINVAL;
  if (N == 0) return NOVAQ_OK;
  if (!grad || !grad_input) return NOVAQ_EINVAL;
  if ((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(grad_input)) & 3)
    return NOVAQ_EALIGN;
  // the reference's factor 1.0 / (H * W): a double, made float32 by its
  // product with the float32 grad
  const float factor = (float)(1.0 / ((double)H * (double)W));
  return global_avg_pool2d_backward_launch(grad, N * C, H * W, factor, grad_input,
                                           static_cast<hipStream_t>(stream));
}

int novaq_im2col(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t C,
                 int64_t H, int64_t W, int KH, int KW, int sh, int sw, int ph, int pw,
                 int pad_mode, float* col, void* stream) {
  if (!valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (x_scale && !is_quant(x_dtype)) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || sh <= 0 || sw <= 0 ||
      ph < 0 || pw < 0)
    return NOVAQ_EINVAL;
  if (H + 2 * (int64_t)ph < KH || W + 2 * (int64_t)pw < KW) return NOVAQ_ESHAPE;
  if (H > 0x7FFFFFFF || W > 0x7FFFFFFF || C > 0x7FFFFFFF || N > 0x7FFFFFFF) return NOVAQ_EINVAL;
  if (N == 0) return NOVAQ_OK;
  if (!x || !col) return NOVAQ_EINVAL;
  const uintptr_t eb = (uintptr_t)dtype_bits(x_dtype) / 8;  // element-aligned x views work
  if (reinterpret_cast<uintptr_t>(x) % eb || !aligned16(col) ||
      (x_scale && (reinterpret_cast<uintptr_t>(x_scale) & 3)))
    return NOVAQ_EALIGN;
  return im2col_launch(x, x_dtype, x_scale, N, C, H, W, KH, KW, sh, sw, ph, pw, pad_mode, col,
                       static_cast<hipStream_t>(stream));
}

int novaq_pad2d(const void* x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int ph,
                int pw, int pad_mode, void* y, void* stream) {
  if (!valid_dtype(x_dtype) || x_dtype == E2M1) return NOVAQ_EDTYPE;
  if (pad_mode < NOVAQ_PAD_ZEROS || pad_mode > NOVAQ_PAD_CIRCULAR) return NOVAQ_EPADMODE;
  if (N < 0 || C <= 0 || H <= 0 || W <= 0 || ph < 0 || pw < 0) return NOVAQ_EINVAL;
  if (H > 0x7FFFFFFF || W > 0x7FFFFFFF || ph > 0x3FFFFFFF || pw > 0x3FFFFFFF) return NOVAQ_EINVAL;
  if (N == 0) return NOVAQ_OK;
  if (!x || !y) return NOVAQ_EINVAL;
  const uintptr_t eb = (uintptr_t)dtype_bits(x_dtype) / 8;
  if (reinterpret_cast<uintptr_t>(x) % eb || !aligned16(y)) return NOVAQ_EALIGN;
  return pad2d_launch(x, x_dtype, N, C, H, W, ph, pw, pad_mode, y,
                      static_cast<hipStream_t>(stream));
}

int novaq_adamw_step(float* w, const float* grad, float* m, float* v, int64_t n,
                     const novaq_adamw* hp, float* w_amax, void* stream) {
  if (!hp || n < 0 || hp->step < 1) return NOVAQ_EINVAL;
  if (n > 0 && (!w || !grad || !m || !v)) return NOVAQ_EINVAL;
  for (const void* p : {(const void*)w, (const void*)grad, (const void*)m, (const void*)v})
    if (p && !aligned16(p)) return NOVAQ_EALIGN;
  if (w_amax && (reinterpret_cast<uintptr_t>(w_amax) & 3)) return NOVAQ_EALIGN;
  return adamw_launch(w, grad, m, v, n, hp->lr, hp->beta1, hp->beta2, hp->eps, hp->weight_decay,
                      hp->step, hp->decay, w_amax, static_cast<hipStream_t>(stream));
}

int novaq_adamw_step_f64(double* w, const void* grad, int grad_f32, double* m, double* v,
                         int64_t n, const novaq_adamw* hp, void* stream) {
  if (!hp || n < 0 || hp->step < 1) return NOVAQ_EINVAL;
  if (n > 0 && (!w || !grad || !m || !v)) return NOVAQ_EINVAL;
  for (const void* p : {(const void*)w, (const void*)m, (const void*)v})
    if (p && (reinterpret_cast<uintptr_t>(p) & 7)) return NOVAQ_EALIGN;
  if (grad && (reinterpret_cast<uintptr_t>(grad) & (grad_f32 ? 3 : 7))) return NOVAQ_EALIGN;
  return adamw_f64_launch(w, grad, grad_f32 != 0, m, v, n, hp->lr, hp->beta1, hp->beta2, hp->eps,
                          hp->weight_decay, hp->step, hp->decay,
                          static_cast<hipStream_t>(stream));
}

int novaq_adamw_requantize(float* w, const float* grad, float* m, float* v, int64_t n,
                           const novaq_adamw* hp, void* codes, int q_dtype, float* amax_scale,
                           void* stream) {
  if (q_dtype != E4M3 && q_dtype != E5M2 && q_dtype != E2M1) return NOVAQ_EDTYPE;
  if (!amax_scale || (n > 0 && !codes)) return NOVAQ_EINVAL;
  if ((codes && !aligned16(codes)) || (reinterpret_cast<uintptr_t>(amax_scale) & 3))
    return NOVAQ_EALIGN;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = novaq_adamw_step(w, grad, m, v, n, hp, amax_scale, stream);
  if (rc != NOVAQ_OK) return rc;
  // the amax-scaled cast: s = amax / fmt_max (block 0 writes it), codes = enc(w * (1/s))
  return cast_launch(w, F32, codes, q_dtype, n, 2, amax_scale, amax_scale + 1, st);
}

int novaq_transpose(const void* src, int src_dtype, int64_t rows, int64_t cols, void* dst,
                    int dst_dtype, void* stream) {
  if (!valid_dtype(src_dtype) || !valid_dtype(dst_dtype)) return NOVAQ_EDTYPE;
  if (rows < 0 || cols < 0) return NOVAQ_EINVAL;
  if (rows == 0 || cols == 0) return NOVAQ_OK;
  if (!src || !dst) return NOVAQ_EINVAL;
  if (!aligned16(src) || !aligned16(dst)) return NOVAQ_EALIGN;
  return transpose_launch(src, src_dtype, rows, cols, dst, dst_dtype,
                          static_cast<hipStream_t>(stream));
}

int novaq_colsum(const float* x, int64_t rows, int64_t cols, float* out, void* stream) {
  if (rows < 0 || cols < 0) return NOVAQ_EINVAL;
  if (cols == 0) return NOVAQ_OK;
  if (!out || (rows > 0 && !x)) return NOVAQ_EINVAL;
  if ((rows > 0 && !aligned16(x)) || !aligned16(out)) return NOVAQ_EALIGN;
  return colsum_launch(x, rows, cols, out, static_cast<hipStream_t>(stream));
}

size_t novaq_linear_backward_workspace(int64_t N, int64_t D_in, int64_t D_out, int w_dtype) {
  if (!valid_dtype(w_dtype) || N < 0 || D_in < 0 || D_out < 0) return 0;
  return linear_bwd_ws(N, D_in, D_out, w_dtype).total;
}

int novaq_linear_backward(const float* grad, const float* x, int64_t N, int64_t D_in,
                          const void* w_q, int w_dtype, const float* w_scale, int64_t D_out,
                          float* grad_input, float* grad_weight, float* grad_bias,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(w_dtype)) return NOVAQ_EDTYPE;
  if (N < 0 || D_in < 0 || D_out < 0) return NOVAQ_EINVAL;
  if (w_dtype == E2M1 && ((D_in | D_out) & 1)) return NOVAQ_ESHAPE;  // whole bytes both ways
  const LinearBwdWs ws = linear_bwd_ws(N, D_in, D_out, w_dtype);
  if ((grad_input || grad_weight) && ws.total > 0 && (!workspace || workspace_bytes < ws.total))
    return NOVAQ_EINVAL;
  if (N > 0 && D_out > 0 && !grad) return NOVAQ_EINVAL;
  if (grad_input && N > 0 && D_in > 0 && D_out > 0 && !w_q) return NOVAQ_EINVAL;
  if (grad_weight && N > 0 && D_in > 0 && !x) return NOVAQ_EINVAL;
  for (const void* p : {(const void*)grad, (const void*)x, w_q, (const void*)grad_input,
                        (const void*)grad_weight, (const void*)grad_bias, (const void*)workspace})
    if (p && !aligned16(p)) return NOVAQ_EALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* base = static_cast<uint8_t*>(workspace);
  int rc = NOVAQ_OK;
  // grad_weight = grad^T @ x: where the shape allows, the product that reads
  // grad and x in place; it runs first, as it also leaves grad rounded to
  // bf16 for grad_input's product (the rounding that product's staging would
  // apply) and sums grad's columns into grad_bias
  const bool tn = grad_weight && D_out > 0 && D_in > 0 && ws.tn;
  uint16_t* g16 =
      tn && grad_input && !ws.wn ? reinterpret_cast<uint16_t*>(base + ws.gyt) : nullptr;
  bool bias_done = false;
  if (tn) {
    rc = linear_tn_launch(grad, x, D_out, D_in, N, grad_weight, grad_bias, g16, s);
    if (rc != NOVAQ_OK) return rc;
    bias_done = true;
  }
  // grad_input = grad @ (s * dec(W)): where the shape allows, on W's FP8 codes
  // read in place (transposing LDS reads) and the fp32 grad, rounded to bf16
  // while staged; else the forward product on W^T (codes permuted) and the
  // bf16 grad the weight-gradient product left
  if (grad_input && N > 0 && D_in > 0) {
    Epilogue ep{};
    ep.out_dtype = F32;
    if (ws.wn) {
      rc = linear_wn_launch(grad, F32, N, D_out, w_q, w_dtype, w_scale, ep, D_in, grad_input, s);
    } else {
      void* wt = base + ws.wt;
      rc = transpose_launch(w_q, w_dtype, D_out, D_in, wt, w_dtype, s);
      if (rc != NOVAQ_OK) return rc;
      if (g16)
        rc = linear_launch(g16, BF16, nullptr, N, D_out, wt, w_dtype, w_scale, ep, D_in,
                           grad_input, s);
      else
        rc = linear_launch(grad, N, D_out, wt, w_dtype, w_scale, nullptr, D_in, grad_input, s);
    }
    if (rc != NOVAQ_OK) return rc;
  }
  // otherwise the forward product of grad^T and x^T, both transposed straight
  // to bf16 (the same round-to-nearest-even)
  if (grad_weight && D_out > 0 && D_in > 0 && !tn) {
    void* gyt = base + ws.gyt;
    void* xt = base + ws.xt;
    rc = transpose_launch(grad, F32, N, D_out, gyt, BF16, s);
    if (rc != NOVAQ_OK) return rc;
    rc = transpose_launch(x, F32, N, D_in, xt, BF16, s);
    if (rc != NOVAQ_OK) return rc;
    Epilogue ep{};
    ep.out_dtype = F32;
    rc = linear_launch(gyt, BF16, nullptr, D_out, N, xt, BF16, nullptr, ep, D_in, grad_weight, s);
    if (rc != NOVAQ_OK) return rc;
  }
  // grad_bias = grad summed over the batch
  if (grad_bias && D_out > 0 && !bias_done) rc = colsum_launch(grad, N, D_out, grad_bias, s);
  return rc;
}

size_t novaq_conv2d_backward_workspace(int64_t N, int64_t C, int64_t C_out, int KH, int KW,
                                       int w_dtype) {
  if (!valid_dtype(w_dtype) || N < 0 || C <= 0 || C_out <= 0 || KH <= 0 || KW <= 0) return 0;
  return conv2d_bwd_workspace(N, C, C_out, KH, KW, w_dtype, device_cu_count()).total;
}

int novaq_conv2d_backward(const float* grad, const float* x, int64_t N, int64_t C, int64_t H,
                          int64_t W, const void* w_q, int w_dtype, const float* w_scale,
                          int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw,
                          int pad_mode, float* grad_input, float* grad_weight,
                          float* grad_bias, void* workspace, size_t workspace_bytes,
                          void* stream) {
  size_t need = 0;
  int rc = conv_bwd_check(grad, x, N, C, H, W, w_q, w_dtype, C_out, KH, KW, sh, sw, ph, pw,
                          pad_mode, grad_input, grad_weight, grad_bias, &need);
  if (rc != NOVAQ_OK || need == 0) return rc;
  if (!workspace || workspace_bytes < need) return NOVAQ_EINVAL;
  if (!aligned16(workspace)) return NOVAQ_EALIGN;
  return conv2d_backward_launch(grad, x, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh,
                                sw, ph, pw, pad_mode, grad_input, grad_weight, grad_bias,
                                workspace, static_cast<hipStream_t>(stream));
}

int novaq_conv2d_backward_noalloc(const float* grad, const float* x, int64_t N, int64_t C,
                                  int64_t H, int64_t W, const void* w_q, int w_dtype,
                                  const float* w_scale, int64_t C_out, int KH, int KW, int sh,
                                  int sw, int ph, int pw, int pad_mode, float* grad_input,
                                  float* grad_weight, float* grad_bias, void* stream) {
  size_t need = 0;
  int rc = conv_bwd_check(grad, x, N, C, H, W, w_q, w_dtype, C_out, KH, KW, sh, sw, ph, pw,
                          pad_mode, grad_input, grad_weight, grad_bias, &need);
  if (rc != NOVAQ_OK || need == 0) return rc;
  if (need > CONV_BWD_SCRATCH_BYTES) return NOVAQ_ESCRATCH;
  void* work = nullptr;
  rc = conv2d_bwd_scratch(&work);
  if (rc != NOVAQ_OK) return rc;
  return conv2d_backward_launch(grad, x, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh,
                                sw, ph, pw, pad_mode, grad_input, grad_weight, grad_bias, work,
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"
