/*
 * novaq -- MI355X (gfx950) quantized-dtype hot path for NovaNN-style layers.
 *
 * C ABI of libnovaq.so.  Plain pointers and sizes only: every tensor argument
 * is a DEVICE pointer owned by the caller, every entry point takes the HIP
 * stream to run on as `void *stream` (NULL = the default stream) and returns
 * an int status (NOVAQ_OK = 0, negative = error).  Nothing is synchronised:
 * results are ready once the stream has drained.  Calls on different streams
 * may run concurrently; a call never allocates device memory.
 *
 * Dtype codes and element storage:
 *   NOVAQ_F32   4 B   IEEE binary32
 *   NOVAQ_F16   2 B   IEEE binary16
 *   NOVAQ_BF16  2 B   bfloat16
 *   NOVAQ_E4M3  1 B   OCP FP8 E4M3 (bias 7, max 448, NaN 0x7F/0xFF, no Inf)
 *   NOVAQ_E5M2  1 B   OCP FP8 E5M2 (bias 15, max 57344, Inf 0x7C, NaN 0x7D-0x7F)
 *   NOVAQ_E2M1  1/2 B OCP MX FP4 E2M1 {0,.5,1,1.5,2,3,4,6}, two per byte:
 *                     element 2i in bits 3..0, element 2i+1 in bits 7..4; a
 *                     buffer of n elements holds ceil(n/2) bytes, an odd tail
 *                     is padded with +0.
 *
 * Rounding and specials (identical on every entry point):
 *   - narrowing is round-to-nearest-even; widening is exact;
 *   - fp16: overflow -> +-Inf; NaN -> 0x7C00 + (mantissa >> 13), +1 if that
 *     reads as Inf (numpy's float32->float16 rule); fp16 -> fp32 keeps the
 *     NaN payload;
 *   - bf16: overflow -> +-Inf; NaN -> top 16 bits with bit 6 (quiet) set;
 *   - E4M3 / E5M2 are saturating: finite overflow and +-Inf go to +-max;
 *     NaN -> 0x7F | sign; decoded NaN is 0x7FC00000 | sign;
 *   - E2M1 saturates to +-6 (Inf too); NaN -> +0;
 *   - -0 and negative values that round to zero keep the sign bit.
 *
 * Scaling (per tensor): `scale` points to one fp32 s on the device.  Casting
 * to E4M3/E5M2/E2M1 encodes x * (1/s); casting from them decodes q * s; each
 * is one correctly rounded fp32 multiply, and 1/s is a correctly rounded fp32
 * division.  scale == NULL means unscaled.  Scaling a cast that involves no
 * quantized type is an error.
 *
 * Buffers must be 16-byte aligned (NOVAQ_EALIGN otherwise).
 */
#ifndef NOVAQ_H
#define NOVAQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum novaq_dtype {
  NOVAQ_F32 = 0,
  NOVAQ_F16 = 1,
  NOVAQ_BF16 = 2,
  NOVAQ_E4M3 = 3,
  NOVAQ_E5M2 = 4,
  NOVAQ_E2M1 = 5
};

/* Padding modes of NovaNN's conv2d (novann/functional.py:325-344): numpy.pad's
 * constant(0) / reflect / edge / wrap. */
enum novaq_pad_mode {
  NOVAQ_PAD_ZEROS = 0,
  NOVAQ_PAD_REFLECT = 1,
  NOVAQ_PAD_REPLICATE = 2,
  NOVAQ_PAD_CIRCULAR = 3
};

enum novaq_status {
  NOVAQ_OK = 0,
  NOVAQ_EINVAL = -1,   /* null pointer, negative size, bad geometry */
  NOVAQ_EDTYPE = -2,   /* dtype code unknown or not allowed here */
  NOVAQ_ESHAPE = -3,   /* shapes inconsistent (e.g. output size <= 0) */
  NOVAQ_EPADMODE = -4, /* padding mode unknown (NovaNN raises ValueError) */
  NOVAQ_EALIGN = -5,   /* a buffer is not 16-byte aligned */
  NOVAQ_EHIP = -6,     /* the HIP runtime reported an error */
  NOVAQ_ENOTSUP = -7,  /* valid request this build does not implement */
  NOVAQ_ESCRATCH = -8  /* request needs more than an allocation-free entry point's
                          static scratch holds */
};

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int novaq_version(void);
/* Static text for a status code. */
const char *novaq_status_string(int status);
/* HIP error code (hipError_t value) behind the last NOVAQ_EHIP on this thread. */
int novaq_last_hip_error(void);

/* Element-wise cast of n elements from src (src_dtype) to dst (dst_dtype).
 * Replaces: NovaNN has no cast entry point; its only dtype conversions are
 * x.astype(np.float32, copy=False) at layer entry (novann/layers/linear/
 * linear.py:81, novann/layers/convolutional/conv2d.py:159) and
 * np.asarray(w, dtype=np.float32) at weight init (linear.py:59,
 * conv2d.py:65).  This generalises them to every pair of
 * {F32, F16, BF16} x {F32, F16, BF16, E4M3, E5M2, E2M1} and back; a cast
 * between two quantized types returns NOVAQ_EDTYPE. */
int novaq_cast(const void *src, int src_dtype, void *dst, int dst_dtype, int64_t n,
               const float *scale, void *stream);

/* NaN-ignoring max |x| of n F32/F16/BF16 elements, written to *amax (device).
 * No reference counterpart (per-tensor scaling is new on this path). */
int novaq_amax(const void *x, int dtype, int64_t n, float *amax, void *stream);

/* *scale = *amax / fmt_max (448 for E4M3, 57344 for E5M2, 6 for E2M1), or 1
 * when *amax is 0 or not finite.  Both pointers are device pointers. */
int novaq_scale_from_amax(const float *amax, int dst_dtype, float *scale, void *stream);

/* Per-tensor scaled quantization in one call: amax, scale, then the scaled
 * cast.  amax_scale points to two device floats; on completion
 * amax_scale[0] = amax of src and amax_scale[1] = s.  dst_dtype must be
 * E4M3, E5M2 or E2M1. */
int novaq_quantize(const void *src, int src_dtype, void *dst, int dst_dtype, int64_t n,
                   float *amax_scale, void *stream);

/* FP4 E2M1 pack / unpack of n fp32 elements (equivalent to novaq_cast
 * F32 <-> E2M1); packed holds ceil(n/2) bytes in the nibble order above. */
int novaq_pack_fp4(const float *x, int64_t n, const float *scale, uint8_t *packed,
                   void *stream);
int novaq_unpack_fp4(const uint8_t *packed, int64_t n, const float *scale, float *y,
                     void *stream);

/* y[N, D_out] = x[N, D_in] @ (s * dec(w_q))^T + bias.
 * Replaces: novann.functional.linear(input, weight, bias)
 * (novann/functional.py:147-163), called by Linear.forward
 * (novann/layers/linear/linear.py:70-83).  w_q is (D_out, D_in) row-major in
 * w_dtype (E4M3, E5M2, E2M1 packed along D_in, BF16, F16 or F32; an E2M1 row
 * holds ceil(D_in / 2) bytes, so with odd D_in each row ends with a pad
 * nibble, which is never read); w_scale is
 * the per-tensor s (NULL = 1); bias is D_out fp32 values or NULL (the
 * reference's (1, D_out) bias); y is (N, D_out) fp32, freshly written.
 * Products run on bf16 MFMA with fp32 accumulation; the scale and the bias are
 * applied in fp32 after accumulation. */
int novaq_linear_forward(const float *x, int64_t N, int64_t D_in, const void *w_q,
                         int w_dtype, const float *w_scale, const float *bias,
                         int64_t D_out, float *y, void *stream);

/* 2-D cross-correlation of x (N, C, H, W) fp32 with s * dec(w_q)
 * (C_out, C, KH, KW), stride (sh, sw), padding (ph, pw) in pad_mode, plus
 * bias (C_out values or NULL).  y is contiguous (N, C_out, OH, OW) fp32 with
 * OH = (H + 2ph - KH)/sh + 1, OW = (W + 2pw - KW)/sw + 1.
 * Replaces: novann.functional.conv2d(input, weight, kernel_size, stride,
 * padding, bias=, padding_mode=) (novann/functional.py:275-385), called by
 * Conv2d.forward (novann/layers/convolutional/conv2d.py:150-177).  The
 * reference materialises im2col (functional.py:346-368) and returns a
 * transposed view (:382); this computes the same values with implicit im2col
 * and writes NCHW directly.  Every padding mode takes any padding width, with
 * numpy.pad's index rules (reflect repeats with period 2(n-1)). */
int novaq_conv2d_forward(const float *x, int64_t N, int64_t C, int64_t H, int64_t W,
                         const void *w_q, int w_dtype, const float *w_scale,
                         int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw,
                         int pad_mode, const float *bias, float *y, void *stream);

/* Fused epilogue of the forward products: what the layers that follow a
 * Linear / Conv2d on NovaNN's main path (main.py:24-46: BatchNorm, ReLU)
 * do to its output, applied before the output is stored.  For output channel
 * c (Linear: output feature; Conv2d: output channel) each element becomes
 *   v = acc * s + bias[c]                the product, as novaq_*_forward
 *   v = v * channel_mul[c]               if channel_mul != NULL
 *   v = v + channel_add[c]               if channel_add != NULL
 *   v = v * (v > 0 ? 1 : 0)              if relu (novann functional.relu,
 *                                        functional.py:8-22: -0 for negative
 *                                        v, NaN stays NaN, -Inf gives NaN)
 * each step one fp32 operation rounded to nearest even, then v is stored as
 * out_dtype: F32; F16 / BF16 (the casts' rounding); E4M3 / E5M2 as
 * enc(v * (1 / *out_scale)) exactly as novaq_cast of the fp32 v with that scale
 * (out_scale NULL = 1).  Eval-mode BatchNorm (batchnorm2d.py:98-102,
 * gamma * (x - mean) / sqrt(var + eps) + beta) is the affine step with
 * channel_mul = gamma / sqrt(var + eps), channel_add = beta - mean *
 * channel_mul.  out_amax (optional, device fp32) receives max |v| over the
 * whole output before the store's cast (NaN ignored): the amax a delayed-
 * scaling caller turns into the next call's out_scale with
 * novaq_scale_from_amax.  All pointers are device pointers. */
typedef struct novaq_epilogue {
  const float *channel_mul;
  const float *channel_add;
  const float *out_scale;
  float *out_amax;
  int relu;
  int out_dtype;
} novaq_epilogue;

/* novaq_linear_forward with a fused epilogue (epi NULL: none, fp32 output).
 * x is (N, D_in) in x_dtype: F32, or BF16 / F16 / E4M3 / E5M2 as a previous
 * epilogue stored it, x_scale its per-tensor scale for FP8 (NULL = 1; the
 * product uses s_x * dec(x)).  y is (N, D_out) in epi->out_dtype.  With
 * FP8 x and FP8 / FP4 weights (N % 128, D_out % 256, D_in % 128) both
 * operands' codes go to the FP8 MFMA: exact products whose sums are not
 * rounded as fp32 additions are (about 1e-5 normwise against fp64).
 * No reference counterpart as one call: it replaces F.linear followed by the
 * BatchNorm / ReLU layers' forward (see novaq_epilogue). */
int novaq_linear_forward_ex(const void *x, int x_dtype, const float *x_scale, int64_t N,
                            int64_t D_in, const void *w_q, int w_dtype, const float *w_scale,
                            const float *bias, int64_t D_out, const novaq_epilogue *epi,
                            void *y, void *stream);

/* novaq_conv2d_forward with a fused epilogue and an x in x_dtype (as
 * novaq_linear_forward_ex); y is (N, C_out, OH, OW) in epi->out_dtype.
 * Replaces Conv2d.forward followed by BatchNorm2d (eval) and ReLU forward. */
int novaq_conv2d_forward_ex(const void *x, int x_dtype, const float *x_scale, int64_t N,
                            int64_t C, int64_t H, int64_t W, const void *w_q, int w_dtype,
                            const float *w_scale, int64_t C_out, int KH, int KW, int sh, int sw,
                            int ph, int pw, int pad_mode, const float *bias,
                            const novaq_epilogue *epi, void *y, void *stream);

/* y (N, C, OH, OW) = the max of each KH x KW window of x (N, C, H, W) padded
 * (ph, pw) in pad_mode with numpy.pad's rules (zeros pads +0), stride
 * (sh, sw); OH = (H + 2ph - KH)/sh + 1.  x and y in x_dtype (F32, or BF16 /
 * F16 / E4M3 / E5M2 as an epilogue stores activations; FP8 codes keep their
 * scale): the result is one of the window's values, the later one in
 * row-major window order when two are equal (the sign of a zero maximum),
 * NaN when the window holds one.  x and y need only be aligned to their
 * element size (NOVAQ_EALIGN otherwise): views into a larger tensor work.
 * Replaces: novann.functional.max_pool2d (novann/functional.py:450-532),
 * called by MaxPool2d.forward (layers/pooling/maxpool/maxpool2d.py:51-79). */
int novaq_max_pool2d(const void *x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W,
                     int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode, void *y,
                     void *stream);

/* y[n, c] = mean over H, W of x[n, c] (x_dtype as above, times x_scale for
 * FP8 when given; a scale with another dtype is NOVAQ_EDTYPE), fp32, evaluated as numpy's np.mean does on float32: 0 plus
 * numpy's pairwise sums of the plane's 8192-element blocks (its ufunc buffer
 * size), divided by H*W, so bit for bit equal.
 * Replaces: novann.functional.avg_pool2d (novann/functional.py:548-559),
 * called by GlobalAvgPool2d.forward (layers/pooling/gap/global_avg_pool2d.py:19-32);
 * y is the reference's (N, C, 1, 1) output. */
int novaq_global_avg_pool2d(const void *x, int x_dtype, const float *x_scale, int64_t N,
                            int64_t C, int64_t H, int64_t W, float *y, void *stream);

/* grad_input (N, C, H, W) fp32 = MaxPool2d's input gradient for grad (N, C,
 * OH, OW) fp32 and the forward's x (N, C, H, W) in x_dtype (as
 * novaq_max_pool2d; same kernel, stride, padding and pad_mode): over each
 * window of x padded in pad_mode, the elements equal to the window's maximum
 * (none when it holds a NaN) share grad / count (count = how many, 1 when
 * none), each other element gets 0 * (grad / count) (NaN for a non-finite
 * grad); an input element sums its windows' shares in (oh, ow) order from +0,
 * and shares that land on the padding are dropped.  fp32, IEEE divide: bit
 * for bit the reference's result.  grad and grad_input 4-byte aligned, x
 * element-aligned (NOVAQ_EALIGN otherwise).
 * Replaces: MaxPool2d.backward (novann/layers/pooling/maxpool/maxpool2d.py:79-129). */
int novaq_max_pool2d_backward(const float *grad, const void *x, int x_dtype, int64_t N,
                              int64_t C, int64_t H, int64_t W, int KH, int KW, int sh, int sw,
                              int ph, int pw, int pad_mode, float *grad_input, void *stream);

/* grad_input (N, C, H, W) fp32 = grad[n, c] * (float)(1.0 / (H * W)) over
 * each plane, grad (N, C) fp32 (the reference's (N, C, 1, 1)): its
 * ones * (grad * factor), the double factor made float32 by the product.
 * grad and grad_input 4-byte aligned (NOVAQ_EALIGN otherwise).
 * Replaces: GlobalAvgPool2d.backward
 * (novann/layers/pooling/gap/global_avg_pool2d.py:35-57). */
int novaq_global_avg_pool2d_backward(const float *grad, int64_t N, int64_t C, int64_t H,
                                     int64_t W, float *grad_input, void *stream);

/* col (C*KH*KW, N*OH*OW) fp32, row-major = the column matrix of NovaNN's
 * conv2d: col[(c*KH + kh)*KW + kw][(n*OH + oh)*OW + ow] = x padded (ph, pw) in
 * pad_mode with numpy.pad's rules, at [n][c][oh*sh + kh][ow*sw + kw]; rows
 * ordered (c, kh, kw) and columns (n, oh, ow) as the reference's
 * windows.transpose(1, 4, 5, 0, 2, 3).reshape(C*KH*KW, -1).  x (N, C, H, W)
 * is in x_dtype (F32, F16, BF16, E4M3, E5M2), decoded exactly; FP8 values are
 * multiplied by *x_scale when x_scale is given (one fp32 multiply, as
 * novaq_cast's dequantize).  x needs element alignment only; col 16 bytes.
 * Replaces: conv2d's _im2col (novann/functional.py:346-368), the `col` that
 * conv2d(..., extras=True) returns (:383-384) and Conv2d.forward caches for
 * its backward (novann/layers/convolutional/conv2d.py:162-175).  The forward
 * products never materialise it. */
int novaq_im2col(const void *x, int x_dtype, const float *x_scale, int64_t N, int64_t C,
                 int64_t H, int64_t W, int KH, int KW, int sh, int sw, int ph, int pw,
                 int pad_mode, float *col, void *stream);

/* y (N, C, H + 2ph, W + 2pw) = x (N, C, H, W) padded in pad_mode with
 * numpy.pad's rules (zeros pads +0; reflect, edge, wrap with any width), in
 * x's own storage (x_dtype F32, F16, BF16, E4M3 or E5M2; codes copied as
 * stored, so FP8 keeps its scale).  x needs element alignment only; y 16
 * bytes.  Replaces: max_pool2d's _add_padding (novann/functional.py:495-514),
 * the padded array behind the window view that max_pool2d(..., extras=True)
 * returns with its padded shape (:516-534) and MaxPool2d.forward caches
 * (novann/layers/pooling/maxpool/maxpool2d.py:63-75); the caller takes the
 * (N, C, OH, OW, KH, KW) window view of y with strides. */
int novaq_pad2d(const void *x, int x_dtype, int64_t N, int64_t C, int64_t H, int64_t W, int ph,
                int pw, int pad_mode, void *y, void *stream);

/* Hyper-parameters of one AdamW step (novann AdamW, adamw.py:17-38): Python
 * floats there, doubles here; step is the 1-based step count t; decay = 0
 * marks a parameter the reference never decays (BatchNorm gamma / beta,
 * adamw.py:50). */
typedef struct novaq_adamw {
  double lr, beta1, beta2, eps, weight_decay;
  int64_t step;
  int decay;
} novaq_adamw;

/* One AdamW step on n fp32 weights w with gradient grad and moment buffers
 * m, v (all device, updated in place):
 *   m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2
 *   w -= lr (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps)
 *   w -= (lr wd) w                      (if weight_decay > 0 and decay)
 * each a float32 operation with the hyper-parameter rounded to float32, as
 * numpy evaluates the reference's statements on its float32 arrays, so the
 * result equals the reference's bit for bit.  w_amax (optional, device)
 * receives max |w| of the updated weights (NaN ignored).
 * Replaces: AdamW.step for one parameter (novann/optim/adamw.py:41-65). */
int novaq_adamw_step(float *w, const float *grad, float *m, float *v, int64_t n,
                     const novaq_adamw *hp, float *w_amax, void *stream);

/* novaq_adamw_step on n float64 weights w with float64 moments m, v (all
 * device, updated in place; 8-byte aligned): the reference's statements on
 * its float64 parameters (BatchNorm gamma / beta, batchnorm2d.py:33-55, whose
 * moments np.zeros_like makes float64), evaluated as numpy does: in float64,
 * except that with grad_f32 != 0 (grad holds float32 values) the products
 * (1 - b1) * g and (1 - b2) * g^2 are float32 operations, widened for the
 * float64 sums; with grad_f32 == 0 grad holds float64 values.  Equal to the
 * reference bit for bit.
 * Replaces: AdamW.step for one float64 parameter (novann/optim/adamw.py:41-65). */
int novaq_adamw_step_f64(double *w, const void *grad, int grad_f32, double *m, double *v,
                         int64_t n, const novaq_adamw *hp, void *stream);

/* novaq_adamw_step on fp32 master weights, then their re-quantization into
 * codes (q_dtype E4M3, E5M2 or E2M1) with a fresh per-tensor scale:
 * amax_scale[0] = max |w|, amax_scale[1] = s = amax / fmt_max, codes =
 * enc(w * (1/s)), exactly as novaq_quantize of the updated w.  The packed
 * weight a quantized layer multiplies with follows each optimizer step.
 * No reference counterpart as one call: the reference steps float32 weights
 * (adamw.py:41-65) and has no quantized storage (module.py:20-23). */
int novaq_adamw_requantize(float *w, const float *grad, float *m, float *v, int64_t n,
                           const novaq_adamw *hp, void *codes, int q_dtype, float *amax_scale,
                           void *stream);

/* dst (cols x rows, dst_dtype) = src (rows x cols, src_dtype) transposed, both
 * row-major.  src_dtype == dst_dtype permutes the stored values (quantized
 * codes are never re-encoded; E2M1 needs even rows and cols, both sides
 * nibble-packed along their rows); F32 -> BF16 / F16 rounds to nearest even.
 * No reference counterpart: it stands in for the strided `.T` views NovaNN's
 * backward passes multiply with (novann/layers/linear/linear.py:101,107). */
int novaq_transpose(const void *src, int src_dtype, int64_t rows, int64_t cols, void *dst,
                    int dst_dtype, void *stream);

/* out[c] = sum over r of x[r][c] (rows x cols fp32, fp32 sums in a fixed
 * order).  Replaces: np.sum(grad, axis=0, keepdims=True), the bias gradient of
 * Linear.backward (novann/layers/linear/linear.py:103-104). */
int novaq_colsum(const float *x, int64_t rows, int64_t cols, float *out, void *stream);

/* Bytes of device workspace novaq_linear_backward needs for these shapes. */
size_t novaq_linear_backward_workspace(int64_t N, int64_t D_in, int64_t D_out, int w_dtype);

/* Gradients of y = x @ (s * dec(w_q))^T + bias with respect to x, the
 * dequantized weight and the bias, given grad = dL/dy (N, D_out) fp32 and the
 * forward input x (N, D_in) fp32:
 *   grad_input  (N, D_in)     = grad @ (s * dec(w_q))
 *   grad_weight (D_out, D_in) = grad^T @ x
 *   grad_bias   (D_out)       = grad summed over the N rows
 * Replaces: Linear.backward (novann/layers/linear/linear.py:85-108).  Any of
 * the three outputs may be NULL (not computed).  The products run on bf16
 * MFMA with fp32 accumulation on grad and x rounded to bf16.  For FP8 w_q at
 * whole-tile shapes (among other limits D_out % 128, D_in % 256 and N % 128
 * are 0) grad_input reads w_q's codes and the fp32 grad in place and
 * grad_weight reads grad and x in place; other shapes go through transposed
 * copies in the workspace (w_q's codes, exact; grad and x in bf16).  The
 * whole condition is the one novaq_linear_backward_workspace() evaluates:
 * when it returns 0, no workspace is needed, whichever gradients are asked
 * for.  grad_bias sums in a fixed order that depends on the shape and on the
 * device's CU count (the tile size the weight-gradient product picks), so it
 * is bit-reproducible per device and shape, not across them.  workspace:
 * device memory of novaq_linear_backward_workspace() bytes (16-byte aligned;
 * may be NULL when that is 0) the call may overwrite; it is not used after
 * the call's kernels complete. */
int novaq_linear_backward(const float *grad, const float *x, int64_t N, int64_t D_in,
                          const void *w_q, int w_dtype, const float *w_scale, int64_t D_out,
                          float *grad_input, float *grad_weight, float *grad_bias,
                          void *workspace, size_t workspace_bytes, void *stream);

/* Bytes of device workspace novaq_conv2d_backward needs for these shapes. */
size_t novaq_conv2d_backward_workspace(int64_t N, int64_t C, int64_t C_out, int KH, int KW,
                                       int w_dtype);

/* Gradients of the convolution novaq_conv2d_forward computes, given grad =
 * dL/dy (N, C_out, OH, OW) fp32 and the forward input x (N, C, H, W) fp32:
 *   grad_weight (C_out, C, KH, KW) = sum over (n, oh, ow) of grad times the
 *       input window padded in pad_mode (the reference's column matrix);
 *   grad_bias   (C_out)            = grad summed over (n, oh, ow);
 *   grad_input  (N, C, H, W)       = the transposed convolution of grad with
 *       s * dec(w_q), accumulated into a zero-padded image whose border is
 *       then cropped -- for every pad_mode, as the reference's col2im does.
 * Replaces: Conv2d.backward and Conv2d._col2im
 * (novann/layers/convolutional/conv2d.py:117-148, 179-207).  Any output may
 * be NULL.  grad_weight runs on bf16 MFMA (grad and the input rounded to
 * bf16, fp32 accumulation) with per-chunk partial sums added in a fixed
 * order; grad_input runs the forward kernels on the flipped weight codes when
 * the stride is 1 and the padding is below the kernel size, fp32 element
 * sums otherwise.  workspace: novaq_conv2d_backward_workspace() bytes. */
int novaq_conv2d_backward(const float *grad, const float *x, int64_t N, int64_t C, int64_t H,
                          int64_t W, const void *w_q, int w_dtype, const float *w_scale,
                          int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw,
                          int pad_mode, float *grad_input, float *grad_weight,
                          float *grad_bias, void *workspace, size_t workspace_bytes,
                          void *stream);

/* novaq_conv2d_backward without a workspace argument and without allocating:
 * no counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving or training
 * loops, harnesses that forbid hipMalloc).  Same arguments (less the
 * workspace), same kernels and the same results as novaq_conv2d_backward.
 * The workspace is a static device array in the library of 32 MiB per GPU
 * (held from the library's load until the process ends); a call whose
 * novaq_conv2d_backward_workspace() exceeds it returns NOVAQ_ESCRATCH (config
 * [5]'s conv2 at batch 256 needs 30.8 MB).  Every call on one GPU shares that
 * GPU's array: calls that overlap on one GPU (different streams, or threads)
 * race; calls ordered on one stream do not. */
int novaq_conv2d_backward_noalloc(const float *grad, const float *x, int64_t N, int64_t C,
                                  int64_t H, int64_t W, const void *w_q, int w_dtype,
                                  const float *w_scale, int64_t C_out, int KH, int KW, int sh,
                                  int sw, int ph, int pw, int pad_mode, float *grad_input,
                                  float *grad_weight, float *grad_bias, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* NOVAQ_H */
