// Conv2d forward: fp32 x kernels and the dispatch over the stored dtype of x
// (the other x dtypes are instantiated in conv2d_x*.hip).
#include "conv2d_impl.h"

namespace novaq {

template int conv2d_launch_xt<F32>(const uint8_t*, const float*, int64_t, int64_t, int64_t,
                                   int64_t, const void*, int, const float*, int64_t, int, int, int,
                                   int, int, int, int, const Epilogue&, void*, hipStream_t);
extern template int conv2d_launch_xt<BF16>(const uint8_t*, const float*, int64_t, int64_t, int64_t,
                                           int64_t, const void*, int, const float*, int64_t, int,
                                           int, int, int, int, int, int, const Epilogue&, void*,
                                           hipStream_t);
extern template int conv2d_launch_xt<F16>(const uint8_t*, const float*, int64_t, int64_t, int64_t,
                                          int64_t, const void*, int, const float*, int64_t, int,
                                          int, int, int, int, int, int, const Epilogue&, void*,
                                          hipStream_t);
extern template int conv2d_launch_xt<E4M3>(const uint8_t*, const float*, int64_t, int64_t, int64_t,
                                           int64_t, const void*, int, const float*, int64_t, int,
                                           int, int, int, int, int, int, const Epilogue&, void*,
                                           hipStream_t);
extern template int conv2d_launch_xt<E5M2>(const uint8_t*, const float*, int64_t, int64_t, int64_t,
                                           int64_t, const void*, int, const float*, int64_t, int,
                                           int, int, int, int, int, int, const Epilogue&, void*,
                                           hipStream_t);

int conv2d_launch(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t C,
                  int64_t H, int64_t W, const void* w_q, int w_dtype, const float* w_scale,
                  int64_t C_out, int KH, int KW, int sh, int sw, int ph, int pw, int pad_mode,
                  const Epilogue& ep, void* y, hipStream_t stream) {
  const auto* xb = static_cast<const uint8_t*>(x);
#define NOVAQ_CONV_XT(T)                                                                    \
  conv2d_launch_xt<T>(xb, x_scale, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh, sw, \
                      ph, pw, pad_mode, ep, y, stream)
  switch (x_dtype) {
    case F32: return NOVAQ_CONV_XT(F32);
    case BF16: return NOVAQ_CONV_XT(BF16);
    case F16: return NOVAQ_CONV_XT(F16);
    case E4M3: return NOVAQ_CONV_XT(E4M3);
    case E5M2: return NOVAQ_CONV_XT(E5M2);
    default: return NOVAQ_EDTYPE;
  }
#undef NOVAQ_CONV_XT
}

int conv2d_launch(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const void* w_q,
                  int w_dtype, const float* w_scale, int64_t C_out, int KH, int KW, int sh,
                  int sw, int ph, int pw, int pad_mode, const Epilogue& ep, void* y,
                  hipStream_t stream) {
  return conv2d_launch(x, F32, nullptr, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh, sw,
                       ph, pw, pad_mode, ep, y, stream);
}

int conv2d_launch(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, const void* w_q,
                  int w_dtype, const float* w_scale, int64_t C_out, int KH, int KW, int sh,
                  int sw, int ph, int pw, int pad_mode, const float* bias, float* y,
                  hipStream_t stream) {
  Epilogue ep{};
  ep.bias = bias;
  ep.out_dtype = F32;
  return conv2d_launch(x, F32, nullptr, N, C, H, W, w_q, w_dtype, w_scale, C_out, KH, KW, sh, sw,
                       ph, pw, pad_mode, ep, y, stream);
}

}  // namespace novaq
