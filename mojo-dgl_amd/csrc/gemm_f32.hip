// Grouped GEMM (segment_mm / gather_mm), float.
#include "gemm_impl.h"
MDGL_INSTANTIATE_GEMM(float)
