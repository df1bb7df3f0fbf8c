// gspmm / segment_reduce kernels, float, reducer sum.
#include "gspmm_impl.h"
MDGL_INSTANTIATE_GSPMM(float, mdgl::RED_SUM)
