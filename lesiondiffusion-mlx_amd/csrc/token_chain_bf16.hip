// The bf16 compile of the token-chain kernel (see elem.h).
#define LDX_ELEM_BF16 1
#include "token_chain.hip"
