// segment_reduce kernels, float.
#include "segment_impl.h"
MDGL_INSTANTIATE_SEGMENT(float)
