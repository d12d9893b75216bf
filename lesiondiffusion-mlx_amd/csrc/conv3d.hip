// Implicit-GEMM 3-D convolution on gfx950 MFMA (v_mfma_f32_32x32x16_f16).
//
// GEMM view: rows = output channels (A operand = packed weights, fragment-major: one
// 1 KB block per 32 output channels x 16 input channels, already in MFMA lane order),
// columns = output voxels (B operand = input channels of the voxel's tap window,
// K-contiguous in NDHWC), K = taps x input channels.
//
// A workgroup (4 waves) owns BO output channels x one brick of BV = TD*TH*TW voxels
// of the "row grid" (output grid; source grid for the upsample fold). For each chunk
// of CC input channels it stages the brick's halo -- the input voxels every tap of
// every brick voxel reads -- into LDS once, applying the fused GroupNorm affine + SiLU
// prologue and zero padding on the way (no im2col buffer). The weight fragments of
// one tap are staged through a two-slot LDS ring, the next tap's loaded into registers
// while the current tap's MFMAs run. B fragments are read from the halo at a per-lane
// base plus a workgroup-uniform tap offset. Epilogue: bias (per batch item optional),
// fp16 shift, output scale, residual, one fp16 rounding, optional GELU / SiLU, NDHWC
// store with a voxel pitch; or, split over channel chunks, fp32 partial planes that a
// reduce kernel sums in a fixed order.
//
// Reference semantics: nax_conv3d (src/lesiondiffusion_mlx/_nax_conv.py:451-619):
// prologue _nax_conv.py:128-136, epilogue :265-270 (+ scaled variant :418-421),
// stride-2 / upsample window rule :185-189, 251-253.

#include "common.h"

#include <cstdlib>

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
  float rHW, rHH;          // 1 / HW, 1 / HH (host-rounded)
  int RS;                  // halo row stride (halves): HW * (CC + 8) + row padding
  int NKC;                 // 16-channel K fragments of the packed weight
  int NOB;                 // 32-row output blocks of the packed weight
  int split, cps;          // split-K: channel-chunk ranges of cps chunks each
  float* part;             // split > 1: fp32 partial sums [split][B * output voxels][O]
  const f16* x0; int64_t x0p;
  const f16* x1; int64_t x1p;
  const f16* w;
  const float* bias; int bias_batched;
  const f16* shift; int64_t shiftp;
  const float* affine; int silu;
  const f16* res; int64_t resp;
  float scale; int act;
  f16* y; int64_t yp; int yvec;
};

__device__ __forceinline__ float gelu_erf(float v) {
  return v * (1.0f + erff(v * 0.70710678118654752f)) * 0.5f;
}

// Epilogue activation applied to the stored half value (a second rounding).
__device__ __forceinline__ f16 post_act(f16 h, int act) {
  if (act == LDX_ACT_GELU) return (f16)gelu_erf((float)h);
  if (act == LDX_ACT_SILU) return (f16)silu_f((float)h);
  return h;
}

// q = t / d for 0 <= t < 2^21 and small d, from a host-rounded reciprocal: (t + 0.5) / d
// lies at least 0.5 / d from an integer, far beyond the float error of the product.
__device__ __forceinline__ int fdiv(int t, float rcp) { return (int)(((float)t + 0.5f) * rcp); }

// Stage the halo of one brick for channels [c0, c0 + CC) into LDS, applying the
// affine + SiLU prologue and zero padding. Global loads are issued NB at a time before
// any of them is consumed, so their latencies overlap.
template <int CC, bool VEC>
__device__ __forceinline__ void load_halo(const ConvParams& p, f16* halo, int b, int c0,
                                          int gd0, int gh0, int gw0) {
  constexpr int PITCH = CC + 8;
  const int hvox = p.HD * p.HH * p.HW;
  const int64_t vol = (int64_t)p.D * p.H * p.W;
  const int64_t bvox = (int64_t)b * vol;
  if constexpr (VEC) {
    constexpr int G = CC / 8;          // 16-byte channel groups per voxel (divides 256)
    constexpr int VPI = 256 / G;       // voxels per pass of the workgroup
    constexpr int NB = 12;
    const int cg = threadIdx.x % G;
    const int c = c0 + cg * 8;
    const bool cval = c < p.C;
    const bool from0 = c < p.C0;
    const f16* src_base = from0 ? p.x0 + c : p.x1 + (c - p.C0);
    const int64_t pitch = from0 ? p.x0p : p.x1p;
    float sc[8], of[8];
    const bool aff = p.affine != nullptr;
    if (aff && cval) {
      const float* ap = p.affine + ((int64_t)b * p.C + c) * 2;
#pragma unroll
      for (int e = 0; e < 8; e++) { sc[e] = ap[2 * e]; of[e] = ap[2 * e + 1]; }
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) { sc[e] = 1.f; of[e] = 0.f; }
    }
    const int silu = p.silu;
    for (int v0 = threadIdx.x / G; v0 < hvox; v0 += VPI * NB) {
      f16x8 val[NB];
      bool ok[NB];
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int vox = v0 + j * VPI;
        const int t = fdiv(vox, p.rHW);
        const int hw = vox - t * p.HW;
        const int hd = fdiv(t, p.rHH);
        const int hh = t - hd * p.HH;
        const int id = gd0 + hd, ih = gh0 + hh, iw = gw0 + hw;
        ok[j] = vox < hvox && cval && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
        val[j] = (f16x8){0, 0, 0, 0, 0, 0, 0, 0};
        if (ok[j]) {
          const int64_t vi = bvox + ((int64_t)id * p.H + ih) * p.W + iw;
          val[j] = *reinterpret_cast<const f16x8*>(src_base + vi * pitch);
        }
      }
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int vox = v0 + j * VPI;
        if (vox >= hvox) break;
        f16x8 v = val[j];
        if (ok[j] && (aff || silu)) {
#pragma unroll
          for (int e = 0; e < 8; e++) {
            float yv = (float)v[e] * sc[e] + of[e];
            if (silu) yv = silu_f(yv);
            v[e] = (f16)yv;
          }
        }
        const int t2 = fdiv(vox, p.rHW);
        *reinterpret_cast<f16x8*>(halo + t2 * p.RS + (vox - t2 * p.HW) * PITCH + cg * 8) = v;
      }
    }
  } else {
    for (int idx = threadIdx.x; idx < hvox * CC; idx += blockDim.x) {
      const int vox = idx / CC, cc = idx - vox * CC;
      const int t = fdiv(vox, p.rHW);
      const int hw = vox - t * p.HW;
      const int hd = fdiv(t, p.rHH);
      const int hh = t - hd * p.HH;
      const int id = gd0 + hd, ih = gh0 + hh, iw = gw0 + hw;
      const int c = c0 + cc;
      f16 v = 0;
      if (c < p.C && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
        const int64_t vi = bvox + ((int64_t)id * p.H + ih) * p.W + iw;
        const f16* src = c < p.C0 ? p.x0 + vi * p.x0p + c : p.x1 + vi * p.x1p + (c - p.C0);
        if (p.affine || p.silu) {
          float yv = (float)*src;
          if (p.affine) yv = yv * p.affine[((int64_t)b * p.C + c) * 2] + p.affine[((int64_t)b * p.C + c) * 2 + 1];
          if (p.silu) yv = silu_f(yv);
          v = (f16)yv;
        } else {
          v = *src;
        }
      }
      halo[t * p.RS + hw * PITCH + cc] = v;
    }
  }
}

// One 32x32x16 f16 MFMA, D(32x32) += A(32x16) * B(16x32). Lane l: A row l%32 and
// B column l%32, k = 8*(l/32) + e; D column l%32, rows (e/4)*8 + 4*(l/32) + e%4.
// On gfx950 this shape sustains twice the throughput of 16x16x32 in a dense loop.
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int WO, int WV, int FO, int FV, int CC, int KSZ, bool VEC>
__global__ __launch_bounds__(256) void conv3d_kernel(ConvParams p) {
  constexpr int BO = WO * FO * 32;
  constexpr int PITCH = CC + 8;
  constexpr int KS = CC / 16;                 // MFMA k-steps per tap and chunk
  constexpr int TAPS = KSZ * KSZ * KSZ;
  constexpr int NFRAG = (BO / 32) * KS;       // 1 KB weight fragments per tap stage
  constexpr int WSTAGE = NFRAG * 512;         // halves per stage
  constexpr int WL = (NFRAG * 64 + 255) / 256;  // 16-byte loads per thread per stage
  extern __shared__ __attribute__((aligned(16))) f16 smem[];
  f16* wring = smem;                          // 2 stages of weights
  f16* halo = smem + 2 * WSTAGE;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wo = wave / WV, wv = wave - wo * WV;
  const int sidx = blockIdx.z % p.split;
  const int z = blockIdx.z / p.split;
  const int b = p.upsample ? z >> 3 : z;
  const int parity = p.upsample ? z & 7 : 0;
  const int pd = parity >> 2, ph = (parity >> 1) & 1, pw = parity & 1;

  const int brick = blockIdx.x;
  const int bw_i = brick % p.NBW, bt = brick / p.NBW, bh_i = bt % p.NBH, bd_i = bt / p.NBH;
  const int d0 = bd_i * p.TD, h0 = bh_i * p.TH, w0 = bw_i * p.TW;
  const int s = p.stride;
  const int gd0 = d0 * s + p.ID0, gh0 = h0 * s + p.IH0, gw0 = w0 * s + p.IW0;
  const int kq = 8 * (lane >> 5);

  // Per-lane B-operand (voxel) bases in the halo.
  int lbase[FV];
  int rv[FV][3];
  bool valid[FV];
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    const int vloc = (wv * FV + fv) * 32 + (lane & 31);
    const int vw = vloc % p.TW, vt = vloc / p.TW, vh = vt % p.TH, vd = vt / p.TH;
    rv[fv][0] = d0 + vd; rv[fv][1] = h0 + vh; rv[fv][2] = w0 + vw;
    valid[fv] = rv[fv][0] < p.RD && rv[fv][1] < p.RH && rv[fv][2] < p.RW;
    const int hd = vd * s + pd, hh = vh * s + ph, hw = vw * s + pw;
    lbase[fv] = (hd * p.HH + hh) * p.RS + hw * PITCH + kq;
  }
  const int sd = p.HH * p.RS, sh = p.RS;

  // Weight staging: thread t loads 16 bytes of fragment f = t/64 (+ 4 per extra load) of
  // the stage -- (ob, kc) = (f / KS, f % KS) -- contiguous 1 KB per wave-wide load.
  const int ob0 = blockIdx.y * (BO / 32);
  const f16* wsrc[WL];
  bool wok[WL];
#pragma unroll
  for (int i = 0; i < WL; i++) {
    const int e = tid + i * 256;
    wok[i] = e < NFRAG * 64;
    const int f = wok[i] ? e / 64 : 0, l = e % 64;
    const int ob = ob0 + f / KS, kc = f % KS;
    wsrc[i] = p.w + (((int64_t)parity * p.NOB + ob) * TAPS * p.NKC + kc) * 512 + l * 8;
  }
  auto wload = [&](f16x8 (&r)[WL], int tap, int kc0) {
#pragma unroll
    for (int i = 0; i < WL; i++)
      if (wok[i]) r[i] = *reinterpret_cast<const f16x8*>(wsrc[i] + ((int64_t)tap * p.NKC + kc0) * 512);
  };
  auto wstore = [&](const f16x8 (&r)[WL], int slot) {
#pragma unroll
    for (int i = 0; i < WL; i++)
      if (wok[i]) *reinterpret_cast<f16x8*>(wring + slot * WSTAGE + (tid + i * 256) * 8) = r[i];
  };

  f32x16 acc[FO][FV];
#pragma unroll
  for (int i = 0; i < FO; i++)
#pragma unroll
    for (int j = 0; j < FV; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  const int c_end = min(p.C, (sidx + 1) * p.cps * CC);
  for (int c0 = sidx * p.cps * CC; c0 < c_end; c0 += CC) {
    const int kc0 = c0 / 16;
    f16x8 r1[WL], r2[WL];
    wload(r1, 0, kc0);
    __syncthreads();  // previous chunk done with the LDS
    wstore(r1, 0);
    if (TAPS > 1) wload(r1, 1, kc0);
    load_halo<CC, VEC>(p, halo, b, c0, gd0, gh0, gw0);
    __syncthreads();
    for (int tap = 0; tap < TAPS; tap++) {
      if (tap + 2 < TAPS) wload(r2, tap + 2, kc0);
      const int kd = tap / (KSZ * KSZ), kh = (tap / KSZ) % KSZ, kw = tap % KSZ;
      const int toff = kd * sd + kh * sh + kw * PITCH;
      const f16* wst = wring + (tap & 1) * WSTAGE + lane * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        f16x8 a[FO], bf[FV];
#pragma unroll
        for (int fo = 0; fo < FO; fo++)
          a[fo] = *reinterpret_cast<const f16x8*>(wst + ((wo * FO + fo) * KS + ks) * 512);
#pragma unroll
        for (int fv = 0; fv < FV; fv++)
          bf[fv] = *reinterpret_cast<const f16x8*>(halo + lbase[fv] + toff + ks * 16);
#pragma unroll
        for (int fo = 0; fo < FO; fo++)
#pragma unroll
          for (int fv = 0; fv < FV; fv++) acc[fo][fv] = mfma32(a[fo], bf[fv], acc[fo][fv]);
      }
      if (tap + 1 < TAPS) wstore(r1, (tap + 1) & 1);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < WL; i++) r1[i] = r2[i];
    }
  }

  // Epilogue: lane holds voxel lane%32 of each column block and, per group j of four
  // accumulator elements, output channels (ob)*32 + j*8 + 4*(lane/32) + r.
  const int64_t ovol = (int64_t)p.OD * p.OH * p.OW;
  const float* bias = p.bias ? p.bias + (p.bias_batched ? (int64_t)b * p.O : 0) : nullptr;
  const f16* shb = p.shift ? p.shift + (int64_t)b * p.shiftp : nullptr;
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
    if (p.split > 1) {
      // Raw fp32 sums of this channel range; the reduce kernel finishes the epilogue.
      float* prow = p.part + ((int64_t)sidx * p.B * ovol + ov) * p.O;
#pragma unroll
      for (int fo = 0; fo < FO; fo++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int o4 = (ob0 + wo * FO + fo) * 32 + j * 8 + 4 * (lane >> 5);
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (o4 + r < p.O) prow[o4 + r] = acc[fo][fv][j * 4 + r];
        }
      continue;
    }
#pragma unroll
    for (int fo = 0; fo < FO; fo++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int o4 = (ob0 + wo * FO + fo) * 32 + j * 8 + 4 * (lane >> 5);
        if (o4 >= p.O) continue;
        f16x4 outv;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int o = o4 + r;
          float v = acc[fo][fv][j * 4 + r];
          if (o < p.O) {
            if (bias) v += bias[o];
            if (shb) v += (float)shb[o];
            v *= p.scale;
            if (rrow) v += (float)rrow[o];
          }
          outv[r] = post_act((f16)v, p.act);
        }
        if (p.yvec && o4 + 4 <= p.O) {
          *reinterpret_cast<f16x4*>(yrow + o4) = outv;
        } else {
#pragma unroll
          for (int r = 0; r < 4; r++)
            if (o4 + r < p.O) yrow[o4 + r] = outv[r];
        }
      }
    }
  }
}

// Split-K finish: sum the fp32 partial planes in split order, then the same epilogue
// as the single-pass kernel (bias, scale, residual, one rounding, optional GELU).
__global__ __launch_bounds__(256) void conv_reduce_kernel(ConvParams p, int64_t nvox) {
  const int64_t n = nvox * p.O;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ov = i / p.O;
    const int o = (int)(i - ov * p.O);
    float v = 0.f;
    for (int s2 = 0; s2 < p.split; s2++) v += p.part[(int64_t)s2 * n + i];
    const int64_t vol = nvox / p.B;
    const int b = (int)(ov / vol);
    if (p.bias) v += p.bias[(p.bias_batched ? (int64_t)b * p.O : 0) + o];
    if (p.shift) v += (float)p.shift[(int64_t)b * p.shiftp + o];
    v *= p.scale;
    if (p.res) v += (float)p.res[ov * p.resp + o];
    p.y[ov * p.yp + o] = post_act((f16)v, p.act);
  }
}

// --------------------------------------------------------------------- host side

struct Tile {
  int WO, WV, FO, FV, CC;
  int BO() const { return WO * FO * 32; }
  int BV() const { return WV * FV * 32; }
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

template <int WO, int WV, int FO, int FV, int CC, int KSZ, bool VEC>
static int launch(ConvParams& p, int grid_z, hipStream_t stream, size_t lds) {
  constexpr int BO = WO * FO * 32;
  lds += (size_t)2 * (BO / 32) * (CC / 16) * 512 * sizeof(f16);  // weight double buffer
  dim3 grid((unsigned)(p.NBD * p.NBH * p.NBW), (unsigned)((p.O + BO - 1) / BO), (unsigned)grid_z);
  auto kern = conv3d_kernel<WO, WV, FO, FV, CC, KSZ, VEC>;
  if (lds > 65536) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return check_launch("conv3d: set LDS size");
  }
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, stream, p);
  return check_launch("conv3d");
}

template <int WO, int WV, int FO, int FV, int KSZ>
static int dispatch_cc(ConvParams& p, int cc, bool vec, int grid_z, hipStream_t stream, size_t lds) {
  if (!vec) return launch<WO, WV, FO, FV, 32, KSZ, false>(p, grid_z, stream, lds);
  if (cc == 64) return launch<WO, WV, FO, FV, 64, KSZ, true>(p, grid_z, stream, lds);
  return launch<WO, WV, FO, FV, 32, KSZ, true>(p, grid_z, stream, lds);
}

template <int WO, int WV, int FO, int FV>
static int dispatch_k(ConvParams& p, int cc, bool vec, int grid_z, hipStream_t stream, size_t lds) {
  if (p.taps == 27) return dispatch_cc<WO, WV, FO, FV, 3>(p, cc, vec, grid_z, stream, lds);
  if (p.taps == 8) return dispatch_cc<WO, WV, FO, FV, 2>(p, cc, vec, grid_z, stream, lds);
  return dispatch_cc<WO, WV, FO, FV, 1>(p, cc, vec, grid_z, stream, lds);
}

}  // namespace ldx

using namespace ldx;

// Validate the arguments and choose tile, brick, channel chunk and split for them.
static int plan_conv(const ldx_conv3d_args* a, ConvParams& p, Tile& t, size_t& lds, bool& vec,
                     int64_t& ws_bytes) {
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
  if (a->act != LDX_ACT_NONE && a->act != LDX_ACT_GELU && a->act != LDX_ACT_SILU)
    return fail("conv3d: unknown act %d", a->act);
  if (a->shift && a->shift_pitch < a->out_c) return fail("conv3d: shift pitch < out_c");

  p = ConvParams{};
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
  p.shift = (const f16*)a->shift; p.shiftp = a->shift_pitch;
  p.affine = a->affine; p.silu = a->silu ? 1 : 0;
  p.res = (const f16*)a->residual; p.resp = a->residual_pitch;
  p.scale = a->output_scale; p.act = a->act;
  p.y = (f16*)a->y; p.yp = a->y_pitch;
  p.yvec = (p.yp % 4 == 0) && ((uintptr_t)a->y % 8 == 0);

  vec = (p.C0 % 8 == 0) && (p.x0p % 8 == 0) && (p.C1 == 0 || (p.C1 % 8 == 0 && p.x1p % 8 == 0)) &&
        ((uintptr_t)a->x0 % 16 == 0) && (p.C1 == 0 || (uintptr_t)a->x1 % 16 == 0);

  // Tiles: (waves over O) x (waves over voxels), 32x32 MFMA blocks per wave; chosen
  // from measured sweeps on MI355X: 64x64 wave tiles when the volume fills the GPU,
  // smaller tiles (plus split-K below) for the coarse UNet levels.
  const int64_t rows = (int64_t)p.B * p.RD * p.RH * p.RW * (p.upsample ? 8 : 1);
  if (p.O <= 32) t = {1, 4, 1, 2, 32};
  else if (p.O <= 64) t = {1, 4, 2, 1, 32};
  else if (rows / 256 * ((p.O + 63) / 64) >= 512) t = {1, 4, 2, 2, 32};
  else t = {2, 2, 1, 1, 32};
  // LDX_CONV_TILE="WO,WV,FO,FV,CC" overrides the tile heuristic (tuning sweeps).
  bool forced = false;
  if (const char* env = getenv("LDX_CONV_TILE")) {
    Tile o{};
    if (sscanf(env, "%d,%d,%d,%d,%d", &o.WO, &o.WV, &o.FO, &o.FV, &o.CC) == 5 && o.WO * o.WV == 4 &&
        (o.CC == 32 || (o.CC == 64 && p.C % 64 == 0 && vec))) {
      t = o;
      forced = true;
    }
  }

  const int ks = a->ksize;
  const int s = p.stride;
  int TD = 1, TH = 1, TW = 1;
  for (;;) {
    pick_brick(p, t.BV(), s, ks, TD, TH, TW);
    p.TD = TD; p.TH = TH; p.TW = TW;
    p.HD = ks == 1 ? TD : (s == 2 ? 2 * TD + 1 : TD + 2);
    p.HH = ks == 1 ? TH : (s == 2 ? 2 * TH + 1 : TH + 2);
    p.HW = ks == 1 ? TW : (s == 2 ? 2 * TW + 1 : TW + 2);
    {
      // Row stride: pad each halo row so that consecutive 8-voxel rows (TW = 8) or
      // 4-voxel rows (TW = 4) of a B fragment start TW 16-byte bank groups apart
      // (mod 16): each 16-lane group of a 128-bit LDS read then hits 16 distinct bank
      // groups.
      const int pitch_units = (t.CC + 8) / 8;
      const int base_units = p.HW * pitch_units;
      const int target = TW < 16 ? TW % 16 : base_units % 16;
      const int pad_units = ((target - base_units) % 16 + 16) % 16;
      p.RS = (base_units + pad_units) * 8;
    }
    lds = (size_t)p.HD * p.HH * p.RS * sizeof(f16);
    const size_t wbytes = (size_t)2 * (t.BO() / 32) * (t.CC / 16) * 1024;
    if (lds + wbytes <= (forced ? 160u * 1024 : 80u * 1024) || (t.CC == 32 && t.FV == 1)) break;
    if (t.CC == 64) t.CC = 32;
    else t.FV = 1;
  }
  if (lds + (size_t)2 * (t.BO() / 32) * (t.CC / 16) * 1024 > 160 * 1024)
    return fail("conv3d: halo of %zu bytes exceeds LDS", lds);
  p.NBD = (p.RD + TD - 1) / TD; p.NBH = (p.RH + TH - 1) / TH; p.NBW = (p.RW + TW - 1) / TW;
  p.ID0 = ks == 1 ? 0 : -1; p.IH0 = p.ID0; p.IW0 = p.ID0;
  p.rHW = 1.0f / (float)p.HW; p.rHH = 1.0f / (float)p.HH;
  p.NOB = (p.O + 127) / 128 * 4; p.NKC = (p.C + 63) / 64 * 4;
  if ((int64_t)p.HD * p.HH * p.HW >= (1 << 20)) return fail("conv3d: halo too large");
  const int64_t bricks = (int64_t)p.NBD * p.NBH * p.NBW;
  if (bricks > 0x7fffffff) return fail("conv3d: too many bricks");

  // Split-K over channel chunks when the grid would leave most CUs idle: fp32
  // partial planes summed in a fixed order by conv_reduce_kernel (deterministic).
  const int64_t wgs = bricks * ((p.O + t.BO() - 1) / t.BO()) * p.B * (p.upsample ? 8 : 1);
  const int nchunks = (p.C + t.CC - 1) / t.CC;
  p.split = 1;
  p.cps = nchunks;
  if (wgs < 192 && nchunks > 1 && p.taps > 1 && p.C >= 128) {
    int want = (int)((512 + wgs - 1) / wgs);
    if (want > nchunks) want = nchunks;
    p.cps = (nchunks + want - 1) / want;
    p.split = (nchunks + p.cps - 1) / p.cps;
  }
  const int64_t nvox = (int64_t)p.B * p.OD * p.OH * p.OW;
  ws_bytes = p.split > 1 ? (int64_t)p.split * nvox * p.O * (int64_t)sizeof(float) : 0;
  if ((int64_t)p.B * (p.upsample ? 8 : 1) * p.split > 65535) return fail("conv3d: batch too large");
  return LDX_OK;
}

extern "C" size_t ldx_conv3d_workspace_bytes(const ldx_conv3d_args* a) {
  ConvParams p;
  Tile t;
  size_t lds;
  bool vec;
  int64_t ws = 0;
  if (plan_conv(a, p, t, lds, vec, ws) != LDX_OK) return 0;
  return (size_t)ws;
}

extern "C" int ldx_conv3d(const ldx_conv3d_args* a, void* stream) {
  ConvParams p;
  Tile t;
  size_t lds;
  bool vec;
  int64_t ws = 0;
  int rc = plan_conv(a, p, t, lds, vec, ws);
  if (rc != LDX_OK) return rc;
  if (p.split > 1 && (!a->workspace || a->workspace_bytes < (size_t)ws)) {
    // No (or too small a) workspace: one pass over all channels.
    p.split = 1;
    p.cps = (p.C + t.CC - 1) / t.CC;
  }
  p.part = p.split > 1 ? (float*)a->workspace : nullptr;
  const int grid_z = p.B * (p.upsample ? 8 : 1) * p.split;
  hipStream_t st = as_stream(stream);

#define LDX_TILE(WO_, WV_, FO_, FV_) \
  if (t.WO == WO_ && t.WV == WV_ && t.FO == FO_ && t.FV == FV_) rc = dispatch_k<WO_, WV_, FO_, FV_>(p, t.CC, vec, grid_z, st, lds); else
  LDX_TILE(1, 4, 1, 2)
  LDX_TILE(1, 4, 1, 1)
  LDX_TILE(1, 4, 2, 2)
  LDX_TILE(1, 4, 2, 1)
  LDX_TILE(2, 2, 2, 2)
  LDX_TILE(2, 2, 1, 2)
  LDX_TILE(2, 2, 2, 1)
  LDX_TILE(2, 2, 1, 1)
  return fail("conv3d: no kernel for tile");
#undef LDX_TILE
  if (rc != LDX_OK || p.split == 1) return rc;
  const int64_t nvox = (int64_t)p.B * p.OD * p.OH * p.OW;
  const int64_t n = nvox * p.O;
  const unsigned blocks = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
  hipLaunchKernelGGL(conv_reduce_kernel, dim3(blocks), dim3(256), 0, st, p, nvox);
  return check_launch("conv3d: split reduce");
}
