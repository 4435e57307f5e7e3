// Linear forward kernels for x stored as bf16 (a fused epilogue's output).
#include "linear_impl.h"

namespace novaq {

template int linear_launch_xt<BF16>(const uint8_t*, const float*, int64_t, int64_t, const void*,
                                  int, const float*, const Epilogue&, int64_t, void*,
                                  hipStream_t);
template int linear_wn_launch_xt<BF16>(const uint8_t*, int64_t, int64_t, const void*, int,
                                     const float*, const Epilogue&, int64_t, void*, hipStream_t);

}  // namespace novaq
