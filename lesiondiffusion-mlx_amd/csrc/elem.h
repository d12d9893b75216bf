// Element type of a translation unit's activations and weights. The dense-path kernels
// (conv3d, its streamed variant, attention) are compiled once per type: as they stand for
// fp16, and from the *_bf16.hip units, which define LDX_ELEM_BF16 and include the same
// source, for bf16. Storage is 16 bits either way; the element type decides the float
// conversions (round to nearest even) and the MFMA instruction. Each compile keeps its
// kernels, parameter blocks and host planners in its own namespace, so both link into one
// library; the C entry points (compiled with the fp16 unit) dispatch on the dtype.
#pragma once

#include "common.h"

#if defined(LDX_ELEM_BF16)
#define LDX_ELEM_NS bf16_path
#else
#define LDX_ELEM_NS f16_path
#endif

namespace ldx {
namespace LDX_ELEM_NS {

#if defined(LDX_ELEM_BF16)
typedef bf16 E;
typedef bf16x2 E2;
typedef bf16x4 E4;
typedef bf16x8 E8;
constexpr int kDtype = LDX_DTYPE_BF16;
// D(32x32) += A(32x16) B(16x32), bf16 operands, fp32 accumulation.
__device__ __forceinline__ f32x16 mfma_e(E8 a, E8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// Dot product of two element pairs accumulated into an fp32 sum.
__device__ __forceinline__ float dot2_e(E2 a, E2 b, float c) { return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false); }
#else
typedef f16 E;
typedef f16x2 E2;
typedef f16x4 E4;
typedef f16x8 E8;
constexpr int kDtype = LDX_DTYPE_F16;
__device__ __forceinline__ f32x16 mfma_e(E8 a, E8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float dot2_e(E2 a, E2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
#endif

// The 16 bytes of a raw 16-byte load as eight elements.
__device__ __forceinline__ E8 as_e8(f16x8 v) { return __builtin_bit_cast(E8, v); }

}  // namespace LDX_ELEM_NS
}  // namespace ldx
