// The bf16 compile of the conv3d kernels and planner (see elem.h).
#define LDX_ELEM_BF16 1
#include "conv3d.hip"
