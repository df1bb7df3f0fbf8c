// gspmm / segment_reduce kernels, float, reducer max.
#include "gspmm_impl.h"
MDGL_INSTANTIATE_GSPMM(float, mdgl::RED_MAX)
