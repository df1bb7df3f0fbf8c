// segment_reduce kernels, double.
#include "segment_impl.h"
MDGL_INSTANTIATE_SEGMENT(double)
