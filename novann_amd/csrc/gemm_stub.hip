#include "novaq_internal.h"
namespace novaq {
int linear_launch(const float*, int64_t, int64_t, const void*, int, const float*, const float*, int64_t, float*, hipStream_t) { return NOVAQ_ENOTSUP; }
int conv2d_launch(const float*, int64_t, int64_t, int64_t, int64_t, const void*, int, const float*, int64_t, int, int, int, int, int, int, int, const float*, float*, hipStream_t) { return NOVAQ_ENOTSUP; }
}
