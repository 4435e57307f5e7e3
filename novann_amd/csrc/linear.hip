// Linear forward: fp32 x kernels and the dispatch over the stored dtype of x
// (the other x dtypes are instantiated in linear_x*.hip).
#include "linear_impl.h"

namespace novaq {

template int linear_launch_xt<F32>(const uint8_t*, const float*, int64_t, int64_t, const void*,
                                   int, const float*, const Epilogue&, int64_t, void*,
                                   hipStream_t);
extern template int linear_launch_xt<BF16>(const uint8_t*, const float*, int64_t, int64_t,
                                           const void*, int, const float*, const Epilogue&,
                                           int64_t, void*, hipStream_t);
extern template int linear_launch_xt<F16>(const uint8_t*, const float*, int64_t, int64_t,
                                          const void*, int, const float*, const Epilogue&,
                                          int64_t, void*, hipStream_t);
extern template int linear_launch_xt<E4M3>(const uint8_t*, const float*, int64_t, int64_t,
                                           const void*, int, const float*, const Epilogue&,
                                           int64_t, void*, hipStream_t);
extern template int linear_launch_xt<E5M2>(const uint8_t*, const float*, int64_t, int64_t,
                                           const void*, int, const float*, const Epilogue&,
                                           int64_t, void*, hipStream_t);
template int linear_wn_launch_xt<F32>(const uint8_t*, int64_t, int64_t, const void*, int,
                                      const float*, const Epilogue&, int64_t, void*, hipStream_t);
extern template int linear_wn_launch_xt<BF16>(const uint8_t*, int64_t, int64_t, const void*, int,
                                              const float*, const Epilogue&, int64_t, void*,
                                              hipStream_t);

int linear_wn_launch(const void* x, int x_dtype, int64_t M, int64_t K, const void* w_q,
                     int w_dtype, const float* w_scale, const Epilogue& ep, int64_t N, void* y,
                     hipStream_t stream) {
  const auto* xb = static_cast<const uint8_t*>(x);
  switch (x_dtype) {
    case F32: return linear_wn_launch_xt<F32>(xb, M, K, w_q, w_dtype, w_scale, ep, N, y, stream);
    case BF16: return linear_wn_launch_xt<BF16>(xb, M, K, w_q, w_dtype, w_scale, ep, N, y, stream);
    default: return NOVAQ_ENOTSUP;
  }
}

int linear_launch(const void* x, int x_dtype, const float* x_scale, int64_t N, int64_t D_in,
                  const void* w_q, int w_dtype, const float* w_scale, const Epilogue& ep,
                  int64_t D_out, void* y, hipStream_t stream) {
  const auto* xb = static_cast<const uint8_t*>(x);
  switch (x_dtype) {
    case F32: return linear_launch_xt<F32>(xb, x_scale, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
    case BF16: return linear_launch_xt<BF16>(xb, x_scale, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
    case F16: return linear_launch_xt<F16>(xb, x_scale, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
    case E4M3: return linear_launch_xt<E4M3>(xb, x_scale, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
    case E5M2: return linear_launch_xt<E5M2>(xb, x_scale, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
    default: return NOVAQ_EDTYPE;
  }
}

int linear_launch(const float* x, int64_t N, int64_t D_in, const void* w_q, int w_dtype,
                  const float* w_scale, const Epilogue& ep, int64_t D_out, void* y,
                  hipStream_t stream) {
  return linear_launch(x, F32, nullptr, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
}

int linear_launch(const float* x, int64_t N, int64_t D_in, const void* w_q, int w_dtype,
                  const float* w_scale, const float* bias, int64_t D_out, float* y,
                  hipStream_t stream) {
  Epilogue ep{};
  ep.bias = bias;
  ep.out_dtype = F32;
  return linear_launch(x, F32, nullptr, N, D_in, w_q, w_dtype, w_scale, ep, D_out, y, stream);
}

}  // namespace novaq
