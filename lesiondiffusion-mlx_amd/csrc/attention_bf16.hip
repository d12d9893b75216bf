// The bf16 compile of the attention kernels (see elem.h).
#define LDX_ELEM_BF16 1
#include "attention.hip"
