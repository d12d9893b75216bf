// K-quarter 3x3x3 stride-1 convolution (conv3d_quad.hip): parameters and the entry used
// by ldx_conv3d.
#pragma once

#include "elem.h"

namespace ldx {
namespace LDX_ELEM_NS {

struct QuadParams {
  int B, D, H, W;
  int C0, C1, C, O;
  int nchunk;               // 64-channel chunks of C0 + C1
  int NKC;                  // 16-channel k-steps of the packed weight's row
  int TD, TH, TW;           // brick
  int NBD, NBH, NBW, nob, nbr;
  UDiv dv_nob, dv_nbr, dv_nbw, dv_nbh;
  const E* x0; int64_t x0p;
  const E* x1; int64_t x1p;
  const E* w;
  const float* bias; int bias_batched;
  const E* shift; int64_t shiftp;
  const float* affine; int silu;   // GroupNorm affine (B, C, 2) and SiLU of the input, or none
  const E* res; int64_t resp;
  float scale;
  E* y; int64_t yp;
  float* stats;             // GroupNorm partial moments [B][schunks][O / 2][3], or null
  int schunks;              // moment blocks per batch item: one per brick
};

// True (and *p planned, bricks counted) when the K-quarter kernel takes this conv: a 3x3x3
// stride-1 conv with 64-channel input chunks and 64-channel output tiles, whose modelled
// time beats the streamed kernel's (LDX_CONV_QUAD=1 takes every eligible shape, =0 none).
bool conv3d_quad_plan(const ldx_conv3d_args* a, QuadParams* p);
int conv3d_quad_launch(QuadParams& p, hipStream_t st);

}  // namespace LDX_ELEM_NS
}  // namespace ldx
