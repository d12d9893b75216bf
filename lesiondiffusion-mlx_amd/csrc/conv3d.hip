// Implicit-GEMM 3-D convolution on gfx950 MFMA (v_mfma_f32_16x16x32_f16).
//
// GEMM view: rows = output channels (A operand = packed weights, K-contiguous per
// output channel), columns = output voxels (B operand = input channels of the
// voxel's tap window, K-contiguous in NDHWC), K = taps x input channels.
//
// A workgroup (4 waves) owns BO output channels x one brick of BV = TD*TH*TW
// voxels of the "row grid" (output grid; source grid for the upsample fold). For
// each chunk of CC input channels it stages the brick's halo -- the input voxels
// every tap of every brick voxel reads -- into LDS once, applying the fused
// GroupNorm affine + SiLU prologue and zero padding on the way. The tap loop then
// reads B fragments from LDS at a per-lane base plus a workgroup-uniform tap offset
// (no im2col buffer), while A fragments stream from L2 into registers one K-step
// ahead. Epilogue: bias (per batch item optional), output scale, residual, one fp16
// rounding, optional GELU, NDHWC store with a voxel pitch.
//
// Reference semantics: nax_conv3d (src/lesiondiffusion_mlx/_nax_conv.py:451-619):
// prologue _nax_conv.py:128-136, epilogue :265-270 (+ scaled variant :418-421),
// stride-2 / upsample window rule :185-189, 251-253.

#include "common.h"

namespace ldx {

struct ConvParams {
  int B, D, H, W;          // input / source grid
  int C0, C1, C, O;
  int RD, RH, RW;          // row grid tiled by bricks
  int OD, OH, OW;          // output grid
  int stride, upsample, taps;
  int TD, TH, TW;          // brick
  int NBD, NBH, NBW;       // bricks per axis
  int HD, HH, HW;          // halo dims
  int ID0, IH0, IW0;       // halo origin offset: origin = brick_start * s - pad
  const f16* x0; int64_t x0p;
  const f16* x1; int64_t x1p;
  const f16* w;
  const float* bias; int bias_batched;
  const float* affine; int silu;
  const f16* res; int64_t resp;
  float scale; int act;
  f16* y; int64_t yp; int yvec;
};

__device__ __forceinline__ float gelu_erf(float v) {
  return v * (1.0f + erff(v * 0.70710678118654752f)) * 0.5f;
}

template <int CC, bool VEC>
__device__ __forceinline__ void load_halo(const ConvParams& p, f16* halo, int b, int c0,
                                          int gd0, int gh0, int gw0) {
  constexpr int PITCH = CC + 8;
  const int hvox = p.HD * p.HH * p.HW;
  const float* aff = p.affine ? p.affine + (int64_t)b * p.C * 2 : nullptr;
  const int64_t vol = (int64_t)p.D * p.H * p.W;
  if constexpr (VEC) {
    constexpr int G = CC / 8;
    for (int idx = threadIdx.x; idx < hvox * G; idx += blockDim.x) {
      const int vox = idx / G, cg = idx - vox * G;
      const int hw = vox % p.HW, t = vox / p.HW, hh = t % p.HH, hd = t / p.HH;
      const int id = gd0 + hd, ih = gh0 + hh, iw = gw0 + hw;
      const int c = c0 + cg * 8;
      f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (c < p.C && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
        const int64_t vi = (int64_t)b * vol + ((int64_t)id * p.H + ih) * p.W + iw;
        const f16* src = c < p.C0 ? p.x0 + vi * p.x0p + c : p.x1 + vi * p.x1p + (c - p.C0);
        v = *reinterpret_cast<const f16x8*>(src);
        if (aff) {
#pragma unroll
          for (int e = 0; e < 8; e++) {
            const float2 sc = *reinterpret_cast<const float2*>(aff + 2 * (c + e));
            float yv = (float)v[e] * sc.x + sc.y;
            if (p.silu) yv = silu_f(yv);
            v[e] = (f16)yv;
          }
        } else if (p.silu) {
#pragma unroll
          for (int e = 0; e < 8; e++) v[e] = (f16)silu_f((float)v[e]);
        }
      }
      *reinterpret_cast<f16x8*>(halo + vox * PITCH + cg * 8) = v;
    }
  } else {
    for (int idx = threadIdx.x; idx < hvox * CC; idx += blockDim.x) {
      const int vox = idx / CC, cc = idx - vox * CC;
      const int hw = vox % p.HW, t = vox / p.HW, hh = t % p.HH, hd = t / p.HH;
      const int id = gd0 + hd, ih = gh0 + hh, iw = gw0 + hw;
      const int c = c0 + cc;
      f16 v = 0;
      if (c < p.C && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
        const int64_t vi = (int64_t)b * vol + ((int64_t)id * p.H + ih) * p.W + iw;
        const f16* src = c < p.C0 ? p.x0 + vi * p.x0p + c : p.x1 + vi * p.x1p + (c - p.C0);
        float yv = (float)*src;
        if (aff || p.silu) {
          if (aff) yv = yv * aff[2 * c] + aff[2 * c + 1];
          if (p.silu) yv = silu_f(yv);
          v = (f16)yv;
        } else {
          v = *src;
        }
      }
      halo[vox * PITCH + cc] = v;
    }
  }
}

template <int FO, bool VEC>
__device__ __forceinline__ void load_a(const ConvParams& p, f16x8 (&a)[FO], const f16* wbase,
                                       int o_lane, int k, int tap) {
  // wbase already offset by parity; row o: wbase + (o*taps + tap)*C + k
#pragma unroll
  for (int fo = 0; fo < FO; fo++) {
    const int o = o_lane + fo * 16;
    f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (o < p.O) {
      const f16* src = wbase + ((int64_t)o * p.taps + tap) * p.C + k;
      if constexpr (VEC) {
        if (k < p.C) v = *reinterpret_cast<const f16x8*>(src);
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++)
          if (k + e < p.C) v[e] = src[e];
      }
    }
    a[fo] = v;
  }
}

template <int WO, int WV, int FO, int FV, int CC, bool VEC>
__global__ __launch_bounds__(256) void conv3d_kernel(ConvParams p) {
  constexpr int BO = WO * FO * 16;
  constexpr int PITCH = CC + 8;
  constexpr int KSTEPS = CC / 32;
  extern __shared__ __attribute__((aligned(16))) f16 halo[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wo = wave / WV, wv = wave - wo * WV;
  const int z = blockIdx.z;
  const int b = p.upsample ? z >> 3 : z;
  const int parity = p.upsample ? z & 7 : 0;
  const int pd = parity >> 2, ph = (parity >> 1) & 1, pw = parity & 1;

  const int brick = blockIdx.x;
  const int bw_i = brick % p.NBW, bt = brick / p.NBW, bh_i = bt % p.NBH, bd_i = bt / p.NBH;
  const int d0 = bd_i * p.TD, h0 = bh_i * p.TH, w0 = bw_i * p.TW;
  const int s = p.stride;
  const int gd0 = d0 * s + p.ID0, gh0 = h0 * s + p.IH0, gw0 = w0 * s + p.IW0;

  const int o_lane = blockIdx.y * BO + wo * FO * 16 + (lane & 15);
  const int kq = 8 * (lane >> 4);

  // Per-lane column (voxel) bases.
  int lbase[FV];
  int rv[FV][3];
  bool valid[FV];
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    const int vloc = (wv * FV + fv) * 16 + (lane & 15);
    const int vw = vloc % p.TW, vt = vloc / p.TW, vh = vt % p.TH, vd = vt / p.TH;
    rv[fv][0] = d0 + vd; rv[fv][1] = h0 + vh; rv[fv][2] = w0 + vw;
    valid[fv] = vd < p.TD && rv[fv][0] < p.RD && rv[fv][1] < p.RH && rv[fv][2] < p.RW;
    const int hd = vd * s + pd, hh = vh * s + ph, hw = vw * s + pw;
    lbase[fv] = ((hd * p.HH + hh) * p.HW + hw) * PITCH + kq;
  }

  const f16* wbase = p.w + (int64_t)parity * p.O * p.taps * p.C;
  f32x4 acc[FO][FV];
#pragma unroll
  for (int i = 0; i < FO; i++)
#pragma unroll
    for (int j = 0; j < FV; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int ksz = p.taps == 27 ? 3 : (p.taps == 8 ? 2 : 1);
  const int nsteps = p.taps * KSTEPS;
  for (int c0 = 0; c0 < p.C; c0 += CC) {
    __syncthreads();
    load_halo<CC, VEC>(p, halo, b, c0, gd0, gh0, gw0);
    __syncthreads();
    f16x8 a_cur[FO], a_nxt[FO];
    load_a<FO, VEC>(p, a_cur, wbase, o_lane, c0 + kq, 0);
    for (int st = 0; st < nsteps; st++) {
      const int tap = st / KSTEPS, ks = st - tap * KSTEPS;
      if (st + 1 < nsteps) {
        const int tap1 = (st + 1) / KSTEPS, ks1 = (st + 1) - tap1 * KSTEPS;
        load_a<FO, VEC>(p, a_nxt, wbase, o_lane, c0 + ks1 * 32 + kq, tap1);
      }
      const int kd = tap / (ksz * ksz), kh = (tap / ksz) % ksz, kw = tap % ksz;
      const int toff = ((kd * p.HH + kh) * p.HW + kw) * PITCH + ks * 32;
      f16x8 bf[FV];
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
        bf[fv] = *reinterpret_cast<const f16x8*>(halo + lbase[fv] + toff);
#pragma unroll
      for (int fo = 0; fo < FO; fo++)
#pragma unroll
        for (int fv = 0; fv < FV; fv++) acc[fo][fv] = mfma16(a_cur[fo], bf[fv], acc[fo][fv]);
#pragma unroll
      for (int fo = 0; fo < FO; fo++) a_cur[fo] = a_nxt[fo];
    }
  }

  // Epilogue.
  const int64_t ovol = (int64_t)p.OD * p.OH * p.OW;
  const float* bias = p.bias ? p.bias + (p.bias_batched ? (int64_t)b * p.O : 0) : nullptr;
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    if (!valid[fv]) continue;
    int64_t ov;
    if (p.upsample)
      ov = ((int64_t)(2 * rv[fv][0] + pd) * p.OH + (2 * rv[fv][1] + ph)) * p.OW + 2 * rv[fv][2] + pw;
    else
      ov = ((int64_t)rv[fv][0] * p.OH + rv[fv][1]) * p.OW + rv[fv][2];
    ov += (int64_t)b * ovol;
    f16* yrow = p.y + ov * p.yp;
    const f16* rrow = p.res ? p.res + ov * p.resp : nullptr;
#pragma unroll
    for (int fo = 0; fo < FO; fo++) {
      const int o4 = blockIdx.y * BO + wo * FO * 16 + fo * 16 + 4 * (lane >> 4);
      if (o4 >= p.O) continue;
      f16x4 outv;
      float vals[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int o = o4 + r;
        float v = acc[fo][fv][r];
        if (o < p.O) {
          if (bias) v += bias[o];
          v *= p.scale;
          if (rrow) v += (float)rrow[o];
        }
        vals[r] = v;
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        f16 h = (f16)vals[r];
        if (p.act == LDX_ACT_GELU) h = (f16)gelu_erf((float)h);
        outv[r] = h;
      }
      const bool full = p.yvec && o4 + 4 <= p.O;
      if (full) {
        *reinterpret_cast<f16x4*>(yrow + o4) = outv;
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (o4 + r < p.O) yrow[o4 + r] = outv[r];
      }
    }
  }
}

// --------------------------------------------------------------------- host side

struct Tile {
  int WO, WV, FO, FV, CC;
  int BO() const { return WO * FO * 16; }
  int BV() const { return WV * FV * 16; }
};

static void pick_brick(const ConvParams& p, int BV, int s, int ks, int& TD, int& TH, int& TW) {
  // Minimise launched voxel slots (partial-brick waste), then the halo volume.
  int64_t best_slots = INT64_MAX, best_halo = INT64_MAX;
  for (int td = 1; td <= BV; td *= 2)
    for (int th = 1; td * th <= BV; th *= 2) {
      const int tw = BV / (td * th);
      if (td * th * tw != BV) continue;
      const int64_t nb = ceil_div64(p.RD, td) * ceil_div64(p.RH, th) * ceil_div64(p.RW, tw);
      const int64_t slots = nb * BV;
      const int hd = ks == 1 ? td : (s == 2 ? 2 * td + 1 : td + 2);
      const int hh = ks == 1 ? th : (s == 2 ? 2 * th + 1 : th + 2);
      const int hw = ks == 1 ? tw : (s == 2 ? 2 * tw + 1 : tw + 2);
      const int64_t halo = (int64_t)hd * hh * hw;
      if (slots < best_slots || (slots == best_slots && halo < best_halo)) {
        best_slots = slots; best_halo = halo; TD = td; TH = th; TW = tw;
      }
    }
}

template <int WO, int WV, int FO, int FV, int CC, bool VEC>
static int launch(ConvParams& p, int grid_z, hipStream_t stream, size_t lds) {
  constexpr int BO = WO * FO * 16;
  dim3 grid((unsigned)(p.NBD * p.NBH * p.NBW), (unsigned)((p.O + BO - 1) / BO), (unsigned)grid_z);
  auto kern = conv3d_kernel<WO, WV, FO, FV, CC, VEC>;
  if (lds > 65536) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return check_launch("conv3d: set LDS size");
  }
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, stream, p);
  return check_launch("conv3d");
}

template <int WO, int WV, int FO, int FV>
static int dispatch_cc(ConvParams& p, int cc, bool vec, int grid_z, hipStream_t stream, size_t lds) {
  if (cc == 64)
    return vec ? launch<WO, WV, FO, FV, 64, true>(p, grid_z, stream, lds)
               : launch<WO, WV, FO, FV, 64, false>(p, grid_z, stream, lds);
  return vec ? launch<WO, WV, FO, FV, 32, true>(p, grid_z, stream, lds)
             : launch<WO, WV, FO, FV, 32, false>(p, grid_z, stream, lds);
}

}  // namespace ldx

using namespace ldx;

extern "C" int ldx_conv3d(const ldx_conv3d_args* a, void* stream) {
  if (!a) return fail("conv3d: null args");
  if (a->batch < 1 || a->in_d < 1 || a->in_h < 1 || a->in_w < 1)
    return fail("conv3d: empty input grid (%d, %d, %d, %d)", a->batch, a->in_d, a->in_h, a->in_w);
  if (a->c0 < 1 || a->c1 < 0 || a->out_c < 1) return fail("conv3d: bad channel counts");
  if (a->ksize != 1 && a->ksize != 3) return fail("conv3d: ksize must be 1 or 3, got %d", a->ksize);
  if (a->stride != 1 && a->stride != 2) return fail("conv3d: stride must be 1 or 2, got %d", a->stride);
  if (a->ksize == 1 && (a->stride != 1 || a->upsample))
    return fail("conv3d: pointwise conv supports stride 1 without upsampling only");
  if (a->upsample && a->stride != 1) return fail("conv3d: upsample requires stride 1");
  if (!a->x0 || !a->weight || !a->y) return fail("conv3d: null x0/weight/y");
  if (a->c1 > 0 && !a->x1) return fail("conv3d: c1 > 0 but x1 is null");
  if (a->x0_pitch < a->c0 || (a->c1 > 0 && a->x1_pitch < a->c1) || a->y_pitch < a->out_c)
    return fail("conv3d: pitch smaller than channel count");
  if (a->residual && a->residual_pitch < a->out_c) return fail("conv3d: residual pitch < out_c");
  if (a->act != LDX_ACT_NONE && a->act != LDX_ACT_GELU) return fail("conv3d: unknown act %d", a->act);

  ConvParams p{};
  p.B = a->batch; p.D = a->in_d; p.H = a->in_h; p.W = a->in_w;
  p.C0 = a->c0; p.C1 = a->c1; p.C = a->c0 + a->c1; p.O = a->out_c;
  p.stride = a->ksize == 3 ? a->stride : 1;
  p.upsample = a->upsample ? 1 : 0;
  p.taps = a->ksize == 1 ? 1 : (p.upsample ? 8 : 27);
  if (p.upsample) {
    p.RD = p.D; p.RH = p.H; p.RW = p.W;
    p.OD = 2 * p.D; p.OH = 2 * p.H; p.OW = 2 * p.W;
  } else if (p.stride == 2) {
    p.OD = (p.D - 1) / 2 + 1; p.OH = (p.H - 1) / 2 + 1; p.OW = (p.W - 1) / 2 + 1;
    p.RD = p.OD; p.RH = p.OH; p.RW = p.OW;
  } else {
    p.OD = p.D; p.OH = p.H; p.OW = p.W;
    p.RD = p.D; p.RH = p.H; p.RW = p.W;
  }
  p.x0 = (const f16*)a->x0; p.x0p = a->x0_pitch;
  p.x1 = (const f16*)a->x1; p.x1p = a->x1_pitch;
  p.w = (const f16*)a->weight;
  p.bias = a->bias; p.bias_batched = a->bias_batched ? 1 : 0;
  p.affine = a->affine; p.silu = a->silu ? 1 : 0;
  p.res = (const f16*)a->residual; p.resp = a->residual_pitch;
  p.scale = a->output_scale; p.act = a->act;
  p.y = (f16*)a->y; p.yp = a->y_pitch;
  p.yvec = (p.yp % 4 == 0) && ((uintptr_t)a->y % 8 == 0);

  const bool vec = (p.C0 % 8 == 0) && (p.x0p % 8 == 0) && (p.C1 == 0 || (p.C1 % 8 == 0 && p.x1p % 8 == 0)) &&
                   ((uintptr_t)a->x0 % 16 == 0) && (p.C1 == 0 || (uintptr_t)a->x1 % 16 == 0) &&
                   ((uintptr_t)a->weight % 16 == 0);

  Tile t;
  if (p.O <= 16) t = {1, 4, 1, 2, 32};
  else if (p.O <= 32) t = {1, 4, 2, 2, 32};
  else if (p.O <= 64) t = {2, 2, 2, 4, 32};
  else t = {2, 2, 4, 4, 32};
  if (p.C >= 64 && p.stride == 1) t.CC = 64;

  const int ks = a->ksize;
  const int s = p.stride;
  int TD = 1, TH = 1, TW = 1;
  size_t lds = 0;
  for (;;) {
    pick_brick(p, t.BV(), s, ks, TD, TH, TW);
    p.TD = TD; p.TH = TH; p.TW = TW;
    p.HD = ks == 1 ? TD : (s == 2 ? 2 * TD + 1 : TD + 2);
    p.HH = ks == 1 ? TH : (s == 2 ? 2 * TH + 1 : TH + 2);
    p.HW = ks == 1 ? TW : (s == 2 ? 2 * TW + 1 : TW + 2);
    lds = (size_t)p.HD * p.HH * p.HW * (t.CC + 8) * sizeof(f16);
    if (lds <= 65536 || (t.CC == 32 && t.FV == 2)) break;
    if (t.CC == 64) t.CC = 32;
    else t.FV = 2;
  }
  if (lds > 160 * 1024) return fail("conv3d: halo of %zu bytes exceeds LDS", lds);
  p.NBD = (p.RD + TD - 1) / TD; p.NBH = (p.RH + TH - 1) / TH; p.NBW = (p.RW + TW - 1) / TW;
  p.ID0 = ks == 1 ? 0 : -1; p.IH0 = p.ID0; p.IW0 = p.ID0;
  const int64_t bricks = (int64_t)p.NBD * p.NBH * p.NBW;
  if (bricks > 0x7fffffff) return fail("conv3d: too many bricks");
  const int grid_z = p.B * (p.upsample ? 8 : 1);
  if (grid_z > 65535) return fail("conv3d: batch too large");
  hipStream_t st = as_stream(stream);

#define LDX_TILE(WO_, WV_, FO_, FV_) \
  if (t.WO == WO_ && t.WV == WV_ && t.FO == FO_ && t.FV == FV_) return dispatch_cc<WO_, WV_, FO_, FV_>(p, t.CC, vec, grid_z, st, lds);
  LDX_TILE(1, 4, 1, 2)
  LDX_TILE(1, 4, 1, 1)
  LDX_TILE(1, 4, 2, 2)
  LDX_TILE(1, 4, 2, 1)
  LDX_TILE(2, 2, 2, 4)
  LDX_TILE(2, 2, 2, 2)
  LDX_TILE(2, 2, 4, 4)
  LDX_TILE(2, 2, 4, 2)
#undef LDX_TILE
  return fail("conv3d: no kernel for tile");
}
