// gsddmm kernels, float.
#include "gsddmm_impl.h"
MDGL_INSTANTIATE_GSDDMM(float)
