// Conv2d forward kernels for x stored as e4m3 (a fused epilogue's output).
#include "conv2d_impl.h"

namespace novaq {

template int conv2d_launch_xt<E4M3>(const uint8_t*, const float*, int64_t, int64_t, int64_t,
                                    int64_t, const void*, int, const float*, int64_t, int, int,
                                    int, int, int, int, int, const Epilogue&, void*, hipStream_t);

}  // namespace novaq
