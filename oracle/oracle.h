/*
 * novaq CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker for the HIP product path in novann_amd/.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path never links or calls it.
 *
 * What it restates:
 *   - The reference (JOSE-MDG/NovaNN v3.0.0) has no cast / FP8 / FP4 code at
 *     all.  Its only numeric backend is numpy; the fp16 rules here follow
 *     numpy's float32<->float16 astype bit for bit (that is what a NovaNN user
 *     gets from x.astype(np.float16)), including NaN payload handling.
 *   - bf16, FP8 E4M3 / E5M2 and FP4 E2M1 follow the public specs (bf16 RNE,
 *     OCP OFP8 v1.0, OCP MX v1.0 section 5.3.3) with the semantic decisions
 *     written next to each function.
 *   - linear / conv2d restate novann/functional.py:147-163 and :275-385 with
 *     fp64 accumulation.
 *
 * Two independent encoders exist for every narrowing format: the fast integer
 * rounding path (novaq_ref_encode) and a brute-force path (novaq_bf_encode)
 * that decodes every candidate code from the spec formula with ldexp and picks
 * the nearest one by exact midpoint comparison.  Tests check one against the
 * other.
 */
#ifndef NOVAQ_ORACLE_H
#define NOVAQ_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same numbering as include/novaq.h. */
enum {
  ORC_F32 = 0,
  ORC_F16 = 1,
  ORC_BF16 = 2,
  ORC_E4M3 = 3,
  ORC_E5M2 = 4,
  ORC_E2M1 = 5
};

enum { ORC_PAD_ZEROS = 0, ORC_PAD_REFLECT = 1, ORC_PAD_REPLICATE = 2, ORC_PAD_CIRCULAR = 3 };

/* ---- scalar conversions (bits in, bits out) ---- */
uint32_t novaq_ref_encode(uint32_t f32_bits, int dtype);   /* f32 -> code of dtype */
uint32_t novaq_ref_decode(uint32_t code, int dtype);       /* code of dtype -> f32 bits */
uint32_t novaq_bf_encode(uint32_t f32_bits, int dtype);    /* brute force, same contract */
uint32_t novaq_bf_decode(uint32_t code, int dtype);        /* ldexp formula, same contract */
uint32_t novaq_ref_quantize_scaled(uint32_t f32_bits, float inv_s, int dtype);
uint32_t novaq_ref_dequantize_scaled(uint32_t code, float s, int dtype);

/* ---- array operations (OpenMP over nthreads; nthreads<=0 means all) ---- */
/* Generic cast.  n counts elements; E2M1 buffers hold ceil(n/2) packed bytes
 * (element 2i in bits 3..0, element 2i+1 in bits 7..4, odd tail padded with +0).
 * scale == NULL: unscaled.  Otherwise *scale is s: quantizing multiplies by
 * 1/s, dequantizing multiplies by s.  Returns 0, or -1 for an unsupported pair. */
int novaq_ref_cast(const void *src, int src_dtype, void *dst, int dst_dtype,
                   int64_t n, const float *scale, int nthreads);
/* NaN-ignoring max |x| over f32/f16/bf16 input; 0 for n == 0. */
float novaq_ref_amax(const void *x, int dtype, int64_t n, int nthreads);
/* s = amax / fmt_max (448, 57344, 6); 1 when amax is 0 or not finite. */
float novaq_ref_scale_from_amax(float amax, int dtype);
/* Round-trip sweep over [begin, begin+count) of the 2^32 fp32 bit patterns:
 * counts (and reports the first) pattern where fast and brute-force encoders
 * disagree.  Used by the exhaustive tests. */
int64_t novaq_ref_sweep_encode(int dtype, uint64_t begin, uint64_t count,
                               uint32_t *first_bad, int nthreads);
/* Brute-force encode of n fp32 bit patterns into out (one uint32 code each). */
void novaq_bf_encode_array(const uint32_t *x, int64_t n, int dtype, uint32_t *out,
                           int nthreads);
/* Encodes [begin, begin+count) of the fp32 bit patterns with the fast encoder
 * into out (one code per pattern, packed as uint8/uint16 by dtype width). */
void novaq_ref_encode_range(int dtype, uint64_t begin, uint64_t count, void *out,
                            int nthreads);

/* ---- products (fp64 accumulation, fp32 result) ---- */
/* y[N, D_out] = x[N, D_in] @ w[D_out, D_in]^T (+ bias[D_out]);
 * restates novann/functional.py:160-162. */
void novaq_ref_linear_f64(const float *x, const float *w, const float *bias,
                          int64_t N, int64_t D_in, int64_t D_out, float *y,
                          int nthreads);
/* Direct cross-correlation, y contiguous NCHW; padding per pad_mode with
 * numpy.pad's constant / reflect / edge / wrap index rules
 * (novann/functional.py:325-344).  Returns 0 or -1 on a bad argument. */
int novaq_ref_conv2d_f64(const float *x, int64_t N, int64_t C, int64_t H, int64_t W,
                         const float *w, int64_t C_out, int KH, int KW, int sh,
                         int sw, int ph, int pw, int pad_mode, const float *bias,
                         float *y, int nthreads);
/* Source index along one axis of length n for padded coordinate i (may be
 * negative or >= n); -1 means "zero" (constant padding). */
int64_t novaq_ref_pad_index(int64_t i, int64_t n, int pad_mode);

#ifdef __cplusplus
}
#endif
#endif
