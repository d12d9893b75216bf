// The bf16 compile of the K-quarter 3x3x3 conv kernel (see elem.h).
#define LDX_ELEM_BF16 1
#include "conv3d_quad.hip"
