// CSR softmax kernels, double.
#include "softmax_impl.h"
MDGL_INSTANTIATE_SOFTMAX(double)
