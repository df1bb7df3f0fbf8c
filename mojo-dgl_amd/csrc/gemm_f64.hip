// Grouped GEMM (segment_mm / gather_mm), double.
#include "gemm_impl.h"
MDGL_INSTANTIATE_GEMM(double)
