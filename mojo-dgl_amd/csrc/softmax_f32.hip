// CSR softmax kernels, float.
#include "softmax_impl.h"
MDGL_INSTANTIATE_SOFTMAX(float)
