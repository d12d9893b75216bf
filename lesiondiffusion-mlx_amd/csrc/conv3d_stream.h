// Streamed 3x3x3 stride-1 convolution (conv3d_stream.hip): parameters and the entry used
// by ldx_conv3d.
#pragma once

#include "elem.h"

namespace ldx {
namespace LDX_ELEM_NS {

struct StreamParams {
  int B, D, H, W;
  int C0, C1, C, O;
  int nchunk;               // 32-channel chunks of C0 + C1
  int NKC;                  // 16-channel k-steps of the packed weight's row
  int bo, TD, TH, TW;       // output tile and brick
  int NBD, NBH, NBW, nob, nbr;
  UDiv dv_nob, dv_nbr, dv_nbw, dv_nbh, dv_g1;
  int split, cps;           // split-K: workgroup ranges of cps channel chunks (split > 1)
  int g1;                   // workgroups per split: bricks x output blocks x batch items
  float* part;              // split > 1: fp32 partial sums [split][B * D * H * W][O]
  const E* x0; int64_t x0p;
  const E* x1; int64_t x1p;
  const E* w;
  const float* bias; int bias_batched;
  const E* shift; int64_t shiftp;
  const float* affine; int silu;
  const E* res; int64_t resp;
  float scale;
  E* y; int64_t yp;
  float* stats;             // GroupNorm partial moments [B][schunks][O / 2][3], or null
  int schunks;              // moment blocks per batch item: one per brick
};

// True (and *p planned) when the streamed kernel takes this conv. A plan that splits the
// reduction over channel chunks (p->split > 1) needs split * voxels * O floats of
// workspace: with check_ws, a conv whose caller passed less is not taken.
bool conv3d_stream_plan(const ldx_conv3d_args* a, StreamParams* p, bool check_ws = true);
int conv3d_stream_launch(StreamParams& p, hipStream_t st);

}  // namespace LDX_ELEM_NS
}  // namespace ldx
