// gspmm / segment_reduce kernels, double, reducer max.
#include "gspmm_impl.h"
MDGL_INSTANTIATE_GSPMM(double, mdgl::RED_MAX)
