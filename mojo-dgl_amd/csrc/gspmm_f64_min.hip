// gspmm / segment_reduce kernels, double, reducer min.
#include "gspmm_impl.h"
MDGL_INSTANTIATE_GSPMM(double, mdgl::RED_MIN)
