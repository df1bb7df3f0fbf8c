// gsddmm kernels, double.
#include "gsddmm_impl.h"
MDGL_INSTANTIATE_GSDDMM(double)
