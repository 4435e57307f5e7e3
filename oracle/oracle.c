/*
 * novaq CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Semantic decisions (the reference leaves all of them open, it has no cast
 * code; the numbering matches the design notes):
 *   D1  E4M3: RNE, finite overflow and +-Inf saturate to +-448 (0x7E);
 *       NaN -> 0x7F | sign.
 *   D2  E5M2: RNE, finite overflow and +-Inf saturate to +-57344 (0x7B);
 *       NaN -> 0x7F | sign.  Decoding 0x7C / 0xFC gives +-Inf.
 *   D3  bf16: RNE on the top 16 bits; overflow -> +-Inf; NaN -> top 16 bits
 *       with the quiet bit (0x0040) set, sign and payload kept.
 *       bf16 -> f32 is the exact shift (bits << 16).
 *   fp16: numpy's float32 <-> float16 rules (numpy is the reference's
 *       numeric backend): RNE, overflow -> +-Inf, NaN -> 0x7C00 + (mantissa
 *       >> 13) (+1 if that would read as Inf); widening is exact and keeps
 *       NaN payloads.
 *   D4  E2M1: RNE, |x| > 6 and +-Inf saturate to +-6; NaN -> +0 (code 0).
 *   D5  scaling: quantize q = enc(x * (1/s)), dequantize y = dec(q) * s, one
 *       fp32 multiply each; the sign is computed separately (sign(x) xor
 *       sign(scale)) so NaN results do not depend on how a machine propagates
 *       NaN signs; a NaN product decodes to the canonical 0x7FC00000 | sign.
 *   D6  amax ignores NaN.  D7  s = amax / fmt_max, s = 1 if amax is 0 or not
 *       finite.  D8  element 2i in the low nibble, odd tail padded with +0.
 *   D9  -0 (and every negative value that rounds to zero) keeps its sign in
 *       every format.  FP8 NaN codes decode to 0x7FC00000 | sign.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

typedef struct {
  int mbits;          /* stored mantissa bits */
  int bias;           /* exponent bias */
  uint32_t max_code;  /* largest finite magnitude code */
} mini_fmt;

static const mini_fmt FMT_F16 = {10, 15, 0x7BFFu};
static const mini_fmt FMT_E4M3 = {3, 7, 0x7Eu};
static const mini_fmt FMT_E5M2 = {2, 15, 0x7Bu};
static const mini_fmt FMT_E2M1 = {1, 1, 0x7u};

static const mini_fmt *fmt_of(int dtype) {
  switch (dtype) {
    case ORC_F16: return &FMT_F16;
    case ORC_E4M3: return &FMT_E4M3;
    case ORC_E5M2: return &FMT_E5M2;
    case ORC_E2M1: return &FMT_E2M1;
    default: return NULL;
  }
}

static int is_quant(int dtype) {
  return dtype == ORC_E4M3 || dtype == ORC_E5M2 || dtype == ORC_E2M1;
}

/* Round the finite magnitude a (fp32 bits, sign clear) to a magnitude code,
 * RNE.  The returned code may exceed f->max_code (overflow); callers apply the
 * format's overflow rule. */
static uint32_t round_mag(uint32_t a, const mini_fmt *f) {
  int e = (int)(a >> 23);
  if (e == 0) return 0; /* fp32 zero/subnormal: < half the smallest target subnormal */
  int E = e - 127;
  int emin = 1 - f->bias;
  uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
  int s = (23 - f->mbits) + (E < emin ? (emin - E) : 0);
  if (s >= 25) return 0;
  uint32_t q = sig >> s;
  uint32_t rem = sig & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  uint32_t code = q + (E >= emin ? ((uint32_t)(E - emin) << f->mbits) : 0u);
  if (rem > half || (rem == half && (code & 1u))) code++;
  return code;
}

uint32_t novaq_ref_encode(uint32_t x, int dtype) {
  uint32_t a = x & 0x7FFFFFFFu;
  switch (dtype) {
    case ORC_F32:
      return x;
    case ORC_BF16:
      if (a > 0x7F800000u) return (x >> 16) | 0x0040u;
      return (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
    case ORC_F16: {
      uint32_t sign = (x >> 16) & 0x8000u;
      if (a >= 0x7F800000u) {
        if (a == 0x7F800000u) return sign | 0x7C00u;
        uint32_t r = 0x7C00u + ((a & 0x7FFFFFu) >> 13);
        if (r == 0x7C00u) r++;
        return sign | r;
      }
      uint32_t c = round_mag(a, &FMT_F16);
      if (c > FMT_F16.max_code) c = 0x7C00u;
      return sign | c;
    }
    case ORC_E4M3:
    case ORC_E5M2: {
      const mini_fmt *f = fmt_of(dtype);
      uint32_t sign = (x >> 24) & 0x80u;
      if (a > 0x7F800000u) return sign | 0x7Fu;
      if (a == 0x7F800000u) return sign | f->max_code;
      uint32_t c = round_mag(a, f);
      if (c > f->max_code) c = f->max_code;
      return sign | c;
    }
    case ORC_E2M1: {
      uint32_t sign = (x >> 28) & 0x8u;
      if (a > 0x7F800000u) return 0u;
      if (a == 0x7F800000u) return sign | 0x7u;
      uint32_t c = round_mag(a, &FMT_E2M1);
      if (c > 0x7u) c = 0x7u;
      return sign | c;
    }
    default:
      return 0;
  }
}

/* Exact decode of a finite magnitude code with mbits / bias to fp32 bits. */
static uint32_t decode_mag(uint32_t c, const mini_fmt *f) {
  uint32_t e = c >> f->mbits;
  uint32_t m = c & ((1u << f->mbits) - 1u);
  if (e == 0) {
    if (m == 0) return 0;
    int p = 31 - __builtin_clz(m); /* leading bit position, < mbits */
    int E = p + 1 - f->bias - f->mbits;
    return ((uint32_t)(E + 127) << 23) | ((m - (1u << p)) << (23 - p));
  }
  return ((uint32_t)((int)e - f->bias + 127) << 23) | (m << (23 - f->mbits));
}

uint32_t novaq_ref_decode(uint32_t c, int dtype) {
  switch (dtype) {
    case ORC_F32:
      return c;
    case ORC_BF16:
      return (c & 0xFFFFu) << 16;
    case ORC_F16: {
      uint32_t sign = (c & 0x8000u) << 16;
      uint32_t a = c & 0x7FFFu;
      if (a >= 0x7C00u) return sign | 0x7F800000u | ((a & 0x3FFu) << 13);
      return sign | decode_mag(a, &FMT_F16);
    }
    case ORC_E4M3: {
      uint32_t sign = (c & 0x80u) << 24;
      uint32_t a = c & 0x7Fu;
      if (a == 0x7Fu) return sign | 0x7FC00000u;
      return sign | decode_mag(a, &FMT_E4M3);
    }
    case ORC_E5M2: {
      uint32_t sign = (c & 0x80u) << 24;
      uint32_t a = c & 0x7Fu;
      if (a == 0x7Cu) return sign | 0x7F800000u;
      if (a > 0x7Cu) return sign | 0x7FC00000u;
      return sign | decode_mag(a, &FMT_E5M2);
    }
    case ORC_E2M1: {
      uint32_t sign = (c & 0x8u) << 28;
      return sign | decode_mag(c & 0x7u, &FMT_E2M1);
    }
    default:
      return 0;
  }
}

/* ---------------- brute force (independent of the bit tricks) ---------------- */

/* Value of a finite magnitude code straight from the spec formula. */
static double bf_value(uint32_t c, const mini_fmt *f) {
  uint32_t e = c >> f->mbits;
  uint32_t m = c & ((1u << f->mbits) - 1u);
  double frac = (double)m / (double)(1u << f->mbits);
  if (e == 0) return ldexp(frac, 1 - f->bias);
  return ldexp(1.0 + frac, (int)e - f->bias);
}

uint32_t novaq_bf_decode(uint32_t c, int dtype) {
  const mini_fmt *f = fmt_of(dtype);
  if (dtype == ORC_F32) return c;
  if (dtype == ORC_BF16) {
    /* bf16 is fp32 with the low 16 mantissa bits removed. */
    return (c & 0xFFFFu) << 16;
  }
  int sbit = dtype == ORC_F16 ? 15 : (dtype == ORC_E2M1 ? 3 : 7);
  uint32_t neg = (c >> sbit) & 1u;
  uint32_t a = c & ((1u << sbit) - 1u);
  uint32_t sign = neg << 31;
  if (dtype == ORC_F16 && a >= 0x7C00u) return sign | 0x7F800000u | ((a & 0x3FFu) << 13);
  if (dtype == ORC_E4M3 && a == 0x7Fu) return sign | 0x7FC00000u;
  if (dtype == ORC_E5M2 && a == 0x7Cu) return sign | 0x7F800000u;
  if (dtype == ORC_E5M2 && a > 0x7Cu) return sign | 0x7FC00000u;
  float v = (float)bf_value(a, f); /* exact: every code value fits fp32 */
  return sign | f2u(v);
}

/* Nearest finite magnitude code to |x| (x finite), ties to the even code, by
 * binary search over the monotone code values.  Overflow handled by caller. */
static uint32_t bf_nearest(double ax, const mini_fmt *f) {
  uint32_t lo = 0, hi = f->max_code;
  if (ax >= bf_value(hi, f)) return hi;
  while (hi - lo > 1) { /* invariant: value(lo) <= ax < value(hi) */
    uint32_t mid = lo + (hi - lo) / 2;
    if (bf_value(mid, f) <= ax) lo = mid; else hi = mid;
  }
  double mp = 0.5 * (bf_value(lo, f) + bf_value(hi, f)); /* exact in double */
  if (ax < mp) return lo;
  if (ax > mp) return hi;
  return (lo & 1u) ? hi : lo;
}

uint32_t novaq_bf_encode(uint32_t x, int dtype) {
  uint32_t neg = x >> 31;
  uint32_t a = x & 0x7FFFFFFFu;
  int isnan_ = a > 0x7F800000u, isinf_ = a == 0x7F800000u;
  double ax = fabs((double)u2f(x));
  switch (dtype) {
    case ORC_F32:
      return x;
    case ORC_BF16: {
      if (isnan_) return (x >> 16) | 0x0040u;
      if (isinf_) return (neg << 15) | 0x7F80u;
      /* candidates: truncation and truncation + 1 ulp (exact in double) */
      uint32_t t = a >> 16;
      double lo = (double)u2f(t << 16);
      double hi = t == 0x7F7Fu ? ldexp(1.0, 128) : (double)u2f((t + 1) << 16);
      double mp = 0.5 * (lo + hi);
      uint32_t r = ax < mp ? t : ax > mp ? t + 1 : ((t & 1u) ? t + 1 : t);
      return (neg << 15) | r; /* t + 1 == 0x7F80 is +Inf */
    }
    case ORC_F16: {
      uint32_t sign = neg << 15;
      if (isnan_) {
        uint32_t r = 0x7C00u + ((a & 0x7FFFFFu) >> 13);
        return sign | (r == 0x7C00u ? r + 1 : r);
      }
      if (isinf_ || ax >= 65520.0) return sign | 0x7C00u; /* 65520 ties to even 0x7C00 */
      return sign | bf_nearest(ax, &FMT_F16);
    }
    case ORC_E4M3:
    case ORC_E5M2: {
      const mini_fmt *f = fmt_of(dtype);
      uint32_t sign = neg << 7;
      if (isnan_) return sign | 0x7Fu;
      if (isinf_) return sign | f->max_code;
      return sign | bf_nearest(ax, f);
    }
    case ORC_E2M1: {
      uint32_t sign = neg << 3;
      if (isnan_) return 0u;
      if (isinf_) return sign | 0x7u;
      return sign | bf_nearest(ax, &FMT_E2M1);
    }
    default:
      return 0;
  }
}

/* ---------------- scaling (D5) ---------------- */

uint32_t novaq_ref_quantize_scaled(uint32_t x, float inv_s, int dtype) {
  uint32_t ib = f2u(inv_s);
  uint32_t sign = (x ^ ib) & 0x80000000u;
  float mag = fabsf(u2f(x)) * fabsf(inv_s);
  uint32_t mb = f2u(mag);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u || mb > 0x7F800000u) mb = 0x7FC00000u;
  return novaq_ref_encode(sign | mb, dtype);
}

static uint32_t scale_bits(uint32_t v, float s) {
  uint32_t sign = (v ^ f2u(s)) & 0x80000000u;
  float mag = fabsf(u2f(v)) * fabsf(s);
  uint32_t mb = f2u(mag);
  if ((v & 0x7FFFFFFFu) > 0x7F800000u || mb > 0x7F800000u) mb = 0x7FC00000u;
  return sign | mb;
}

uint32_t novaq_ref_dequantize_scaled(uint32_t code, float s, int dtype) {
  return scale_bits(novaq_ref_decode(code, dtype), s);
}

/* ---------------- arrays ---------------- */

static int threads_or_all(int nthreads) {
#ifdef _OPENMP
  return nthreads > 0 ? nthreads : omp_get_max_threads();
#else
  (void)nthreads;
  return 1;
#endif
}

static inline uint32_t load_elem(const void *p, int dtype, int64_t i) {
  switch (dtype) {
    case ORC_F32: return ((const uint32_t *)p)[i];
    case ORC_F16:
    case ORC_BF16: return ((const uint16_t *)p)[i];
    case ORC_E4M3:
    case ORC_E5M2: return ((const uint8_t *)p)[i];
    case ORC_E2M1: {
      uint8_t b = ((const uint8_t *)p)[i >> 1];
      return (i & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0xFu);
    }
    default: return 0;
  }
}

static inline void store_elem(void *p, int dtype, int64_t i, uint32_t c) {
  switch (dtype) {
    case ORC_F32: ((uint32_t *)p)[i] = c; break;
    case ORC_F16:
    case ORC_BF16: ((uint16_t *)p)[i] = (uint16_t)c; break;
    case ORC_E4M3:
    case ORC_E5M2: ((uint8_t *)p)[i] = (uint8_t)c; break;
    default: break; /* E2M1 stored by pairs in novaq_ref_cast */
  }
}

static inline uint32_t convert_one(uint32_t code, int st, int dt, int scaled, float s,
                                   float inv_s) {
  uint32_t v = novaq_ref_decode(code, st);
  if (scaled && is_quant(st)) v = scale_bits(v, s);
  if (scaled && is_quant(dt)) return novaq_ref_quantize_scaled(v, inv_s, dt);
  return novaq_ref_encode(v, dt);
}

int novaq_ref_cast(const void *src, int st, void *dst, int dt, int64_t n,
                   const float *scale, int nthreads) {
  if (st < ORC_F32 || st > ORC_E2M1 || dt < ORC_F32 || dt > ORC_E2M1) return -1;
  if (is_quant(st) && is_quant(dt)) return -1;
  if (scale && !is_quant(st) && !is_quant(dt)) return -1;
  if (n < 0) return -1;
  int scaled = scale != NULL;
  float s = scaled ? *scale : 1.0f;
  float inv_s = 1.0f / s;
  int nt = threads_or_all(nthreads);
  if (dt == ORC_E2M1) {
    int64_t nb = (n + 1) / 2;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t b = 0; b < nb; b++) {
      uint32_t lo = convert_one(load_elem(src, st, 2 * b), st, dt, scaled, s, inv_s);
      uint32_t hi = 2 * b + 1 < n
                        ? convert_one(load_elem(src, st, 2 * b + 1), st, dt, scaled, s, inv_s)
                        : 0u;
      ((uint8_t *)dst)[b] = (uint8_t)((lo & 0xFu) | ((hi & 0xFu) << 4));
    }
    return 0;
  }
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t i = 0; i < n; i++)
    store_elem(dst, dt, i, convert_one(load_elem(src, st, i), st, dt, scaled, s, inv_s));
  return 0;
}

float novaq_ref_amax(const void *x, int dtype, int64_t n, int nthreads) {
  int nt = threads_or_all(nthreads);
  uint32_t best = 0;
#pragma omp parallel for num_threads(nt) reduction(max : best) schedule(static)
  for (int64_t i = 0; i < n; i++) {
    uint32_t a = novaq_ref_decode(load_elem(x, dtype, i), dtype) & 0x7FFFFFFFu;
    if (a <= 0x7F800000u && a > best) best = a;
  }
  return u2f(best);
}

float novaq_ref_scale_from_amax(float amax, int dtype) {
  float fmax = dtype == ORC_E4M3 ? 448.0f
               : dtype == ORC_E5M2 ? 57344.0f
               : dtype == ORC_E2M1 ? 6.0f
                                    : 1.0f;
  if (!(amax > 0.0f) || !isfinite(amax)) return 1.0f;
  return amax / fmax;
}

int64_t novaq_ref_sweep_encode(int dtype, uint64_t begin, uint64_t count,
                               uint32_t *first_bad, int nthreads) {
  int nt = threads_or_all(nthreads);
  int64_t bad = 0;
  uint64_t first = UINT64_MAX;
#pragma omp parallel for num_threads(nt) reduction(+ : bad) reduction(min : first) schedule(static)
  for (uint64_t k = 0; k < count; k++) {
    uint32_t x = (uint32_t)(begin + k);
    if (novaq_ref_encode(x, dtype) != novaq_bf_encode(x, dtype)) {
      bad++;
      if (begin + k < first) first = begin + k;
    }
  }
  if (first_bad) *first_bad = (uint32_t)first;
  return bad;
}

void novaq_bf_encode_array(const uint32_t *x, int64_t n, int dtype, uint32_t *out,
                           int nthreads) {
  int nt = threads_or_all(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t i = 0; i < n; i++) out[i] = novaq_bf_encode(x[i], dtype);
}

void novaq_ref_encode_range(int dtype, uint64_t begin, uint64_t count, void *out,
                            int nthreads) {
  int nt = threads_or_all(nthreads);
  int wide = dtype == ORC_F16 || dtype == ORC_BF16;
#pragma omp parallel for num_threads(nt) schedule(static)
  for (uint64_t k = 0; k < count; k++) {
    uint32_t c = novaq_ref_encode((uint32_t)(begin + k), dtype);
    if (wide) ((uint16_t *)out)[k] = (uint16_t)c;
    else ((uint8_t *)out)[k] = (uint8_t)c;
  }
}

/* ---------------- products ---------------- */

void novaq_ref_linear_f64(const float *x, const float *w, const float *bias,
                          int64_t N, int64_t D_in, int64_t D_out, float *y,
                          int nthreads) {
  int nt = threads_or_all(nthreads);
#pragma omp parallel for num_threads(nt) collapse(2) schedule(static)
  for (int64_t i = 0; i < N; i++) {
    for (int64_t j = 0; j < D_out; j++) {
      const float *xr = x + i * D_in;
      const float *wr = w + j * D_in;
      double acc = 0.0;
      for (int64_t k = 0; k < D_in; k++) acc += (double)xr[k] * (double)wr[k];
      if (bias) acc += (double)bias[j];
      y[i * D_out + j] = (float)acc;
    }
  }
}

int64_t novaq_ref_pad_index(int64_t i, int64_t n, int pad_mode) {
  if (i >= 0 && i < n) return i;
  switch (pad_mode) {
    case ORC_PAD_ZEROS: return -1;
    case ORC_PAD_REPLICATE: return i < 0 ? 0 : n - 1;
    case ORC_PAD_CIRCULAR: {
      int64_t r = i % n;
      return r < 0 ? r + n : r;
    }
    case ORC_PAD_REFLECT: {
      if (n == 1) return 0;
      int64_t p = 2 * (n - 1);
      int64_t r = i % p;
      if (r < 0) r += p;
      return r >= n ? p - r : r;
    }
    default: return -1;
  }
}

int novaq_ref_conv2d_f64(const float *x, int64_t N, int64_t C, int64_t H, int64_t W,
                         const float *w, int64_t C_out, int KH, int KW, int sh,
                         int sw, int ph, int pw, int pad_mode, const float *bias,
                         float *y, int nthreads) {
  if (pad_mode < ORC_PAD_ZEROS || pad_mode > ORC_PAD_CIRCULAR) return -1;
  if (KH <= 0 || KW <= 0 || sh <= 0 || sw <= 0 || ph < 0 || pw < 0) return -1;
  int64_t OH = (H + 2 * ph - KH) / sh + 1;
  int64_t OW = (W + 2 * pw - KW) / sw + 1;
  if (H + 2 * ph < KH || W + 2 * pw < KW || OH <= 0 || OW <= 0) return -1;
  int nt = threads_or_all(nthreads);
#pragma omp parallel for num_threads(nt) collapse(2) schedule(static)
  for (int64_t n = 0; n < N; n++) {
    for (int64_t co = 0; co < C_out; co++) {
      for (int64_t oh = 0; oh < OH; oh++) {
        for (int64_t ow = 0; ow < OW; ow++) {
          double acc = bias ? (double)bias[co] : 0.0;
          for (int64_t c = 0; c < C; c++) {
            for (int kh = 0; kh < KH; kh++) {
              int64_t ih = novaq_ref_pad_index(oh * sh + kh - ph, H, pad_mode);
              if (ih < 0) continue;
              for (int kw = 0; kw < KW; kw++) {
                int64_t iw = novaq_ref_pad_index(ow * sw + kw - pw, W, pad_mode);
                if (iw < 0) continue;
                acc += (double)w[((co * C + c) * KH + kh) * KW + kw] *
                       (double)x[((n * C + c) * H + ih) * W + iw];
              }
            }
          }
          y[((n * C_out + co) * OH + oh) * OW + ow] = (float)acc;
        }
      }
    }
  }
  return 0;
}
