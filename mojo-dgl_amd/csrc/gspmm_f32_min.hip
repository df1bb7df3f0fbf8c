// gspmm / segment_reduce kernels, float, reducer min.
#include "gspmm_impl.h"
MDGL_INSTANTIATE_GSPMM(float, mdgl::RED_MIN)
