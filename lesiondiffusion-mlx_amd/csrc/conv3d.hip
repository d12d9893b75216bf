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
// each tap arrive in a 4-slot LDS ring by direct global->LDS loads issued three taps
// ahead; the next tap's A and B fragments are read into registers while the current
// tap's MFMAs run. B fragments are read from the halo at a per-lane base plus a
// workgroup-uniform tap offset. Epilogue: bias (per batch item optional), fp16 shift,
// output scale, residual, one fp16 rounding, optional GELU / SiLU, NDHWC store with a
// voxel pitch; or, split over channel chunks, fp32 partial planes that a reduce kernel
// sums in a fixed order. Pointwise convs (and dense layers) run as a direct-load GEMM
// over the flattened volume instead (dense_kernel, dense_ksplit_kernel).
//
// Reference semantics: nax_conv3d (src/lesiondiffusion_mlx/_nax_conv.py:451-619):
// prologue _nax_conv.py:128-136, epilogue :265-270 (+ scaled variant :418-421),
// stride-2 / upsample window rule :185-189, 251-253.

#include "elem.h"
#include "conv3d_quad.h"
#include "conv3d_stream.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace ldx {
namespace LDX_ELEM_NS {

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
  float rTW, rTH;          // 1 / TW, 1 / TH
  int RS;                  // halo row stride (halves): HW * (CC + 8) + row padding
  int NKC;                 // 16-channel K fragments of the packed weight
  int NOB;                 // 32-row output blocks of the packed weight
  int split, cps;          // split-K: channel-chunk ranges of cps chunks each
  float* part;             // split > 1: fp32 partial sums [split][B * output voxels][O]
  const E* x0; int64_t x0p;
  const E* x1; int64_t x1p;
  const E* w;
  const float* bias; int bias_batched;
  const E* shift; int64_t shiftp;
  const float* affine; int silu;
  const E* res; int64_t resp;
  float scale; int act;
  E* y; int64_t yp; int yvec;
  int ep_vec;              // 16-byte epilogue accesses: y, residual, shift, bias, partials aligned
  int nh;                  // planned halo: register slots per thread (0: generic staging loop)
  int stg_off;             // > 0: LDS offset (floats) of the epilogue staging, past the halo
  int tps;                 // host only: > 1 asks for whole kw rows per weight stage
  int nob, nbr;            // output-channel blocks of the workgroup tile; bricks per batch item
  const float* ln_g;       // dense_ksplit with LayerNorm: per-channel gamma, beta and eps
  const float* ln_b;
  float ln_eps;
  float* stats;            // GroupNorm partial moments [B][schunks][O / 2][3], or null
  int schunks;             // voxel blocks per batch item the moments are kept for
  UDiv dv_nob, dv_nbr, dv_split, dv_nbw, dv_nbh;  // division by nob, nbr, split, NBW, NBH
};

__device__ __forceinline__ float gelu_erf(float v) {
  return v * (1.0f + erff(v * 0.70710678118654752f)) * 0.5f;
}

// Epilogue activation applied to the stored half value (a second rounding).
__device__ __forceinline__ E post_act(E h, int act) {
  if (act == LDX_ACT_GELU) return (E)gelu_erf((float)h);
  if (act == LDX_ACT_SILU) return (E)silu_f((float)h);
  return h;
}
template <int ACT>
__device__ __forceinline__ E post_act_t(E h) {
  if constexpr (ACT == LDX_ACT_GELU) return (E)gelu_erf((float)h);
  else if constexpr (ACT == LDX_ACT_SILU) return (E)silu_f((float)h);
  else return h;
}

// q = t / d for 0 <= t < 2^21 and small d, from a host-rounded reciprocal: (t + 0.5) / d
// lies at least 0.5 / d from an integer, far beyond the float error of the product.
__device__ __forceinline__ int fdiv(int t, float rcp) { return (int)(((float)t + 0.5f) * rcp); }


// Stage the halo of one brick for channels [c0, c0 + CC) into LDS, applying the
// affine + SiLU prologue and zero padding. Global loads are issued NB at a time before
// any of them is consumed, so their latencies overlap.
template <int CC, bool VEC, int NT>
__device__ __forceinline__ void load_halo(const ConvParams& p, E* halo, int b, int c0,
                                          int gd0, int gh0, int gw0) {
  constexpr int PITCH = CC + 8;
  const int hvox = p.HD * p.HH * p.HW;
  const int64_t vol = (int64_t)p.D * p.H * p.W;
  const int64_t bvox = (int64_t)b * vol;
  if constexpr (VEC) {
    constexpr int G = CC / 8;          // 16-byte channel groups per voxel (divides NT)
    constexpr int VPI = NT / G;        // voxels per pass of the workgroup
    constexpr int NB = 12;
    const int cg = threadIdx.x % G;
    const int c = c0 + cg * 8;
    const bool cval = c < p.C;
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
    const bool xf = aff || p.silu;
    const int silu = p.silu;
    // Source of this chunk: all of it in x0, or all in x1 (the host sends chunks that
    // straddle the split, or a batch item past 2 GiB, down the generic path). Reads go
    // through a buffer resource over the batch item, so padding voxels and channels
    // past C read as zero without a branch.
    const bool in0 = c0 < p.C0;
    const E* base = in0 ? p.x0 + bvox * p.x0p : p.x1 + bvox * p.x1p;
    const int64_t pitch = in0 ? p.x0p : p.x1p;
    const auto rs = make_rsrc(base, (unsigned)(vol * pitch * 2));
    const unsigned cofs = (unsigned)((in0 ? c : c - p.C0) * 2);
    for (int v0 = threadIdx.x / G; v0 < hvox; v0 += VPI * NB) {
      E8 val[NB];
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
        const unsigned off = ok[j] ? (unsigned)(((id * p.H + ih) * p.W + iw) * (unsigned)pitch * 2u) + cofs
                                   : 0xfffffff0u;
        val[j] = buffer_load16<E8>(rs, off);
      }
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int vox = v0 + j * VPI;
        if (vox >= hvox) break;
        E8 v = val[j];
        if (xf) {
#pragma unroll
          for (int e = 0; e < 8; e++) {
            float yv = (float)v[e] * sc[e] + of[e];
            if (silu) yv = silu_f(yv);
            v[e] = ok[j] ? (E)yv : (E)0;
          }
        }
        const int t2 = fdiv(vox, p.rHW);
        *reinterpret_cast<E8*>(halo + t2 * p.RS + (vox - t2 * p.HW) * PITCH + cg * 8) = v;
      }
    }
  } else {
    for (int idx = threadIdx.x; idx < hvox * CC; idx += NT) {
      const int vox = idx / CC, cc = idx - vox * CC;
      const int t = fdiv(vox, p.rHW);
      const int hw = vox - t * p.HW;
      const int hd = fdiv(t, p.rHH);
      const int hh = t - hd * p.HH;
      const int id = gd0 + hd, ih = gh0 + hh, iw = gw0 + hw;
      const int c = c0 + cc;
      E v = 0;
      if (c < p.C && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) {
        const int64_t vi = bvox + ((int64_t)id * p.H + ih) * p.W + iw;
        const E* src = c < p.C0 ? p.x0 + vi * p.x0p + c : p.x1 + vi * p.x1p + (c - p.C0);
        if (p.affine || p.silu) {
          float yv = (float)*src;
          if (p.affine) yv = yv * p.affine[((int64_t)b * p.C + c) * 2] + p.affine[((int64_t)b * p.C + c) * 2 + 1];
          if (p.silu) yv = silu_f(yv);
          v = (E)yv;
        } else {
          v = *src;
        }
      }
      halo[t * p.RS + hw * PITCH + cc] = v;
    }
  }
}

// One 32x32x16 E MFMA, D(32x32) += A(32x16) * B(16x32). Lane l: A row l%32 and
// B column l%32, k = 8*(l/32) + e; D column l%32, rows (e/4)*8 + 4*(l/32) + e%4.
// On gfx950 this shape sustains twice the throughput of 16x16x32 in a dense loop.
__device__ __forceinline__ f32x16 mfma32(E8 a, E8 b, f32x16 c) {
  return mfma_e(a, b, c);
}

// Weight ring: WRING slots, loads issued WPF = WRING - 1 stages ahead.
constexpr int WRING = 4;
constexpr int WPF = WRING - 1;

// Per-lane epilogue constants. In the epilogue each lane finishes one group of 8 output
// channels (from 32 * ob_first + 8 * (lane % (4 * FO))) for several voxels; the group's
// bias and shift are summed here, so a caller can load them before its main loop and
// keep their latency out of the epilogue.
struct EpiConst {
  int o;          // first channel of the lane's group
  int nch;        // channels of the group inside O (<= 0: none)
  bool vec8;      // whole group with 16-byte accesses
  float add8[8];  // bias + shift of the group's channels
};

template <int FO>
__device__ __forceinline__ EpiConst epi_const(const ConvParams& p, int lane, int ob_first, int b) {
  EpiConst e;
  constexpr int G8 = FO * 4;
  e.o = ob_first * 32 + (lane % G8) * 8;
  e.nch = min(8, p.O - e.o);
  e.vec8 = e.nch == 8 && p.ep_vec;
#pragma unroll
  for (int r = 0; r < 8; r++) e.add8[r] = 0.f;
  const float* bias = p.bias ? p.bias + (p.bias_batched ? (int64_t)b * p.O : 0) : nullptr;
  const E* shb = p.shift ? p.shift + (int64_t)b * p.shiftp : nullptr;
  if (e.nch > 0) {
    if (e.vec8) {
      if (bias) {
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(bias + e.o);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(bias + e.o + 4);
#pragma unroll
        for (int r = 0; r < 4; r++) { e.add8[r] = b0[r]; e.add8[r + 4] = b1[r]; }
      }
      if (shb) {
        const E8 s8 = *reinterpret_cast<const E8*>(shb + e.o);
#pragma unroll
        for (int r = 0; r < 8; r++) e.add8[r] += (float)s8[r];
      }
    } else {
      // Branch-free: indices clamped into the group (every load in bounds), values past it
      // dropped; a runtime index would put add8 in scratch memory.
#pragma unroll
      for (int r = 0; r < 8; r++) {
        const int rr = e.o + min(r, e.nch - 1);
        const float v = (bias ? bias[rr] : 0.f) + (shb ? (float)shb[rr] : 0.f);
        e.add8[r] = r < e.nch ? v : 0.f;
      }
    }
  }
  return e;
}

// Epilogue of one wave's FO x FV block of 32 x 32 accumulator tiles, through its LDS
// staging area `stg` (32 x (FO * 32 + 4) floats): voxels of the brick at (d0, h0, w0)
// (slot (wv * FV + fv) * 32 + v), output channels from 32 * ob_first. Each wave stages
// one 32-voxel column block at a time (its FO * 32 channels in fp32, voxel-major), then
// each lane finishes its 8-channel group for 32 * G8 / 64 voxels -- bias and shift (from
// `ec`), scale, residual, one rounding, activation -- and writes each as one 16-byte
// store, the lanes of a voxel covering its channels contiguously. Voxel indices are
// 32-bit (the host bounds B * output voxels below 2^31); the residual rows are all
// requested before the first is used. With p.stats and schunk >= 0, each column block
// also leaves the GroupNorm partial moments of its stored values (pair_moments) as voxel
// block schunk + fv of batch item b.
template <int FO, int FV>
__device__ __forceinline__ void conv_epilogue(const ConvParams& p, const EpiConst& ec, f32x16 (&acc)[FO][FV],
                                              float* stg, int lane, int wv, int b, int sidx, int pd, int ph,
                                              int pw, int d0, int h0, int w0, int schunk = -1) {
  constexpr int EPW = FO * 32 + 4;   // staging pitch (floats): conflict-free both ways
  constexpr int G8 = FO * 4;         // 8-channel groups per voxel (divides 64)
  constexpr int NI = 32 * G8 / 64;   // voxels per lane per column block
  const int col = lane & 31, hf = lane >> 5;
  const int g = lane % G8;
  const int o = ec.o, nch = ec.nch;
  const bool vec8 = ec.vec8;
  const int ovol = p.OD * p.OH * p.OW;
  const bool partial = p.split > 1;
  const bool pref_res = p.res && vec8 && !partial;
  // One copy of the store loop per activation: no per-element branch on it.
  auto finish = [&](auto act_c) {
  constexpr int ACT = decltype(act_c)::value;
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    // Lane (hf, col) holds voxel col, channels fo * 32 + j * 8 + 4 * hf + r.
#pragma unroll
    for (int fo = 0; fo < FO; fo++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const f32x4 q = {acc[fo][fv][j * 4], acc[fo][fv][j * 4 + 1], acc[fo][fv][j * 4 + 2], acc[fo][fv][j * 4 + 3]};
        *reinterpret_cast<f32x4*>(stg + col * EPW + fo * 32 + j * 8 + 4 * hf) = q;
      }
    __builtin_amdgcn_wave_barrier();  // (LDS operations of a wave complete in order)
    int ov[NI];
    bool ok[NI];
    E8 re8[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int v = lane / G8 + i * (64 / G8);
      const int vloc = (wv * FV + fv) * 32 + v;
      const int vt = fdiv(vloc, p.rTW), vw = vloc - vt * p.TW;
      const int vd = fdiv(vt, p.rTH), vh = vt - vd * p.TH;
      const int rd = d0 + vd, rh = h0 + vh, rw = w0 + vw;
      ok[i] = nch > 0 && vd < p.TD && rd < p.RD && rh < p.RH && rw < p.RW;
      if (p.upsample)
        ov[i] = ((2 * rd + pd) * p.OH + (2 * rh + ph)) * p.OW + 2 * rw + pw;
      else
        ov[i] = (rd * p.OH + rh) * p.OW + rw;
      ov[i] += b * ovol;
    }
    if (pref_res) {
#pragma unroll
      for (int i = 0; i < NI; i++)
        re8[i] = ok[i] ? *reinterpret_cast<const E8*>(p.res + (int64_t)ov[i] * p.resp + o)
                       : (E8){0, 0, 0, 0, 0, 0, 0, 0};
    } else {
#pragma unroll
      for (int i = 0; i < NI; i++) re8[i] = (E8){0, 0, 0, 0, 0, 0, 0, 0};
    }
    f32x4 lo[NI], hi[NI];
    E8 outv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
      outv[i] = (E8){0, 0, 0, 0, 0, 0, 0, 0};
      const int v = lane / G8 + i * (64 / G8);
      lo[i] = *reinterpret_cast<const f32x4*>(stg + v * EPW + g * 8);
      hi[i] = *reinterpret_cast<const f32x4*>(stg + v * EPW + g * 8 + 4);
    }
#pragma unroll
    for (int i = 0; i < NI; i++) {
      if (!ok[i]) continue;
      const float r8[8] = {lo[i][0], lo[i][1], lo[i][2], lo[i][3], hi[i][0], hi[i][1], hi[i][2], hi[i][3]};
      if (partial) {
        // Raw fp32 sums of this channel range; the reduce kernel finishes the epilogue.
        float* prow = p.part + ((int64_t)sidx * p.B * ovol + ov[i]) * p.O + o;
        if (vec8) {
          *reinterpret_cast<f32x4*>(prow) = lo[i];
          *reinterpret_cast<f32x4*>(prow + 4) = hi[i];
        } else {
#pragma unroll
          for (int r = 0; r < 8; r++)
            if (r < nch) prow[r] = r8[r];
        }
        continue;
      }
      E* yrow = p.y + (int64_t)ov[i] * p.yp + o;
      if (vec8) {
        E8& out = outv[i];
#pragma unroll
        for (int r = 0; r < 8; r++) out[r] = post_act_t<ACT>((E)((r8[r] + ec.add8[r]) * p.scale + (float)re8[i][r]));
        *reinterpret_cast<E8*>(yrow) = out;
      } else {
        const E* rrow = p.res ? p.res + (int64_t)ov[i] * p.resp + o : nullptr;
#pragma unroll
        for (int r = 0; r < 8; r++) {
          if (r >= nch) break;
          float t = (r8[r] + ec.add8[r]) * p.scale;
          if (rrow) t += (float)rrow[r];
          yrow[r] = post_act_t<ACT>((E)t);
        }
      }
    }
    // GroupNorm partial moments of the stored values (16-byte epilogue only; the host
    // admits stats with O a multiple of 8 and aligned rows): block schunk + fv of batch
    // item b; lanes g, g + G8, ... hold the same 8 channels.
    if (p.stats && schunk >= 0 && !partial) {
      bool okv[NI];
#pragma unroll
      for (int i = 0; i < NI; i++) okv[i] = ok[i] && vec8;
      pair_moments<NI, G8>(outv, okv, p.stats + (((int64_t)b * p.schunks + schunk + fv) * (p.O / 2) + o / 2) * 3,
                           lane < G8 && vec8);
    }
    __builtin_amdgcn_wave_barrier();
  }
  };
  if (p.act == LDX_ACT_GELU) finish(std::integral_constant<int, LDX_ACT_GELU>());
  else if (p.act == LDX_ACT_SILU) finish(std::integral_constant<int, LDX_ACT_SILU>());
  else finish(std::integral_constant<int, LDX_ACT_NONE>());
}

// Scheduling hint: spread NR LDS reads between NM MFMAs (one MFMA, then its share of
// the reads) so the next tap's operands stream in while the current tap's MFMAs run.
template <int NR, int NM, int I = 0>
__device__ __forceinline__ void interleave_reads_mfma() {
  if constexpr (I < NM) {
    constexpr int per = (NR + NM - 1) / NM;
    constexpr int left = NR - I * per;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
    if constexpr (left > 0) __builtin_amdgcn_sched_group_barrier(0x100, left < per ? left : per, 0);
    interleave_reads_mfma<NR, NM, I + 1>();
  }
}

// Halo slots per thread held in registers on the planned halo path: a thread's halo
// voxels (tid / G + j * VPI) are the same for every channel chunk, so their source voxel
// indices and LDS offsets are computed once per workgroup, and the next chunk's halo can
// be loaded into registers while the current chunk's taps run.
constexpr int NHMAX = 8;
constexpr int NHL = NHMAX + 4;   // loads per thread of one planned halo request (+ affine)

// PLAN: the planned halo path (VEC only; register slots per thread fixed per workgroup);
// otherwise the generic staging loop of load_halo.
// TPS: taps per weight stage. A stage is one ring slot, one barrier and one batch of DMAs;
// TPS = KSZ (a whole kw row per stage) takes two thirds of the barriers out of the tap loop
// for a ring three times the size, which pays where one workgroup per CU is all the grid
// has (the coarse UNet levels).
template <int WO, int WV, int FO, int FV, int CC, int KSZ, bool VEC, bool PLAN, int TPS>
__global__ __launch_bounds__(256) void conv3d_kernel(ConvParams p) {
  touch_args(p);
  // One K-group of four waves takes every k-step of a tap (the indexing below keeps the
  // group variables: a two-group variant, two waves per SIMD on one output tile, measured
  // no faster and was taken out).
  constexpr int KSPL = 1;
  static_assert(!PLAN || VEC, "the planned halo needs 16-byte channel groups");
  constexpr int NT = 256 * KSPL;
  constexpr int BO = WO * FO * 32;
  constexpr int PITCH = CC + 8;
  constexpr int KS = CC / 16;                 // MFMA k-steps per tap and chunk
  constexpr int KSG = KS / KSPL;              // k-steps per tap of one K-group
  static_assert(KSG * KSPL == KS && KSG >= 1, "K-groups must split the chunk's k-steps");
  constexpr int TAPS = KSZ * KSZ * KSZ;
  constexpr int NFRAG = (BO / 32) * KSG;      // 1 KB weight fragments per group stage
  static_assert((KSZ * KSZ * KSZ) % TPS == 0, "a stage holds whole taps of one chunk");
  constexpr int WSTAGE = NFRAG * 512 * TPS;   // halves per group stage
  constexpr int LW = (NFRAG + 3) / 4;         // weight DMAs per wave per stage
  constexpr int G = CC / 8;                   // 16-byte channel groups per voxel
  constexpr int VPI = NT / G;                 // halo voxels per pass of the workgroup
  constexpr int SPC = TAPS / TPS;             // stages per chunk
  // Stage of each chunk after whose weight load the next chunk's halo is requested: the
  // loads then have the last WPF - 1 stages of the chunk to land.
  constexpr int TPF = SPC - WPF;
  extern __shared__ __attribute__((aligned(16))) E smem[];
  E* halo = smem + KSPL * WRING * WSTAGE;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave >> 2, w4 = wave & 3;
  const int wo = w4 / WV, wv = w4 - wo * WV;
  E* wring = smem + kg * WRING * WSTAGE;    // this K-group's weight ring
  // Workgroup -> (output block, brick, z) with the output blocks of a brick adjacent and
  // the bricks each XCD receives (workgroups are dealt to the 8 XCDs round-robin)
  // contiguous, so neighbouring halos meet in the same L2.
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
  }
  // Divisions by host-made multipliers (scalar multiply-shift, no division sequence).
  const int q1 = udiv(wg, p.dv_nob);
  const int oblk = wg - q1 * p.nob;
  const int zz = udiv(q1, p.dv_nbr);
  const int brick = q1 - zz * p.nbr;
  const int z = udiv(zz, p.dv_split);
  const int sidx = zz - z * p.split;
  const int b = p.upsample ? z >> 3 : z;
  const int parity = p.upsample ? z & 7 : 0;
  const int pd = parity >> 2, ph = (parity >> 1) & 1, pw = parity & 1;

  const int bt = udiv(brick, p.dv_nbw), bw_i = brick - bt * p.NBW;
  const int bd_i = udiv(bt, p.dv_nbh), bh_i = bt - bd_i * p.NBH;
  const int d0 = bd_i * p.TD, h0 = bh_i * p.TH, w0 = bw_i * p.TW;
  const int s = p.stride;
  const int gd0 = d0 * s + p.ID0, gh0 = h0 * s + p.IH0, gw0 = w0 * s + p.IW0;
  const int kq = 8 * (lane >> 5) + kg * KSG * 16;
  const int ob0 = oblk * (BO / 32);
  // The epilogue's bias and shift, requested now so the main loop hides their latency.
  const EpiConst ec = epi_const<FO>(p, lane, ob0 + wo * FO, b);

  // Per-lane B-operand (voxel) bases in the halo.
  int lbase[FV];
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    const int vloc = (wv * FV + fv) * 32 + (lane & 31);
    const int vt = fdiv(vloc, p.rTW), vw = vloc - vt * p.TW;
    const int vd = fdiv(vt, p.rTH), vh = vt - vd * p.TH;
    const int hd = vd * s + pd, hh = vh * s + ph, hw = vw * s + pw;
    lbase[fv] = (hd * p.HH + hh) * p.RS + hw * PITCH + kq;
  }
  const int sd = p.HH * p.RS, sh = p.RS;

  // Weight staging: stage st = (channel chunk, TPS taps) of this workgroup's sequence goes
  // to ring slot st % WRING of each K-group by direct global->LDS loads, WPF stages ahead
  // of its use. Wave w4 of group g moves the group's fragments f = w4 + 4 i ((ob, k) =
  // (f / KSG, f % KSG)): one 1 KB fragment is one 16-byte-per-lane load, already in MFMA
  // lane order. A wave with fewer real fragments repeats one (same data to the same
  // place), so every wave issues LW loads per stage and the vmcnt wait is uniform.
  const int c_begin = sidx * p.cps * CC;
  const int c_end = min(p.C, (sidx + 1) * p.cps * CC);
  const int nst = (c_end - c_begin + CC - 1) / CC * SPC;
  const unsigned ring_lds = lds_offset(wring);
  // This wave's fragment sources at (tap 0, chunk 0); a stage adds (tap * NKC + kc0) * 512.
  const E* wsrc[LW];
#pragma unroll
  for (int i = 0; i < LW; i++) {
    const int f = (w4 + 4 * i) % NFRAG;
    wsrc[i] = p.w + (((int64_t)parity * p.NOB + ob0 + f / KSG) * TAPS * p.NKC + kg * KSG + f % KSG) * 512 +
              lane * 8;
  }
  // Next stage to load: (ntap, nkc); it stops advancing at the last stage.
  int ntap = 0, nkc = c_begin / 16, nleft = nst - 1;
  auto issue_stage = [&](int slot) {
#pragma unroll
    for (int j = 0; j < TPS; j++) {
      const int64_t off = ((int64_t)(ntap + j) * p.NKC + nkc) * 512;
#pragma unroll
      for (int i = 0; i < LW; i++)
        dma_b128(wsrc[i] + off, ring_lds + (unsigned)(((slot * TPS + j) * NFRAG + (w4 + 4 * i) % NFRAG) * 1024));
    }
    if (nleft > 0) {
      nleft--;
      ntap += TPS;
      if (ntap == TAPS) { ntap = 0; nkc += KS; }
    }
  };

  // Planned halo (16-byte channel groups and at most NHMAX slots per thread): per slot
  // the source voxel index within the batch item (~0u outside the volume) and the LDS
  // offset in halves (-1 past the halo).
  const bool xf = p.affine != nullptr || p.silu;
  const int cg = tid % G;
  unsigned hvi[NHMAX];
  int hlo[NHMAX];
  E8 hval[NHMAX];
  f32x4 haff[4];   // the chunk's (scale, offset) pairs of this thread's 8 channels
  if constexpr (PLAN) {
    const int hvox = p.HD * p.HH * p.HW;
#pragma unroll
    for (int j = 0; j < NHMAX; j++) {
      const int vox = tid / G + j * VPI;
      const int t = fdiv(vox, p.rHW);
      const int hw = vox - t * p.HW;
      const int hd = fdiv(t, p.rHH);
      const int hh = t - hd * p.HH;
      const int id = gd0 + hd, ih = gh0 + hh, iw = gw0 + hw;
      const bool in = vox < hvox && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
      hvi[j] = in ? (unsigned)((id * p.H + ih) * p.W + iw) : ~0u;
      hlo[j] = vox < hvox ? t * p.RS + hw * PITCH + cg * 8 : -1;
    }
  }
  // Request the halo of channels [c0, c0 + CC) into hval and the affine of this thread's
  // channel group into haff: exactly NHL loads per thread (padding voxels, channels past
  // C, unused slots and an absent affine read zeros through the buffer resources' range
  // checks).
  auto halo_issue = [&](int c0) {
    if constexpr (PLAN) {
      const bool in0 = c0 < p.C0;
      const int64_t vol = (int64_t)p.D * p.H * p.W;
      const E* base = in0 ? p.x0 + (int64_t)b * vol * p.x0p : p.x1 + (int64_t)b * vol * p.x1p;
      const unsigned pitch2 = (unsigned)((in0 ? p.x0p : p.x1p) * 2);
      const auto rs = make_rsrc(base, (unsigned)(vol * pitch2));
      const int c = c0 + cg * 8;
      const bool cval = c < p.C;
      const unsigned cofs = (unsigned)((in0 ? c : c - p.C0) * 2);
#pragma unroll
      for (int j = 0; j < NHMAX; j++) {
        const unsigned off = (hvi[j] != ~0u && cval) ? hvi[j] * pitch2 + cofs : 0xfffffff0u;
        hval[j] = buffer_load16<E8>(rs, off);
      }
      const auto ra = make_rsrc(p.affine ? p.affine + (int64_t)b * p.C * 2 : nullptr,
                                p.affine ? (unsigned)(p.C * 8) : 0u);
#pragma unroll
      for (int q = 0; q < 4; q++)
        haff[q] = __builtin_bit_cast(f32x4, buffer_load16<E8>(ra, (unsigned)(c * 8 + q * 16)));
    }
  };
  // Write hval to the halo, with the affine + SiLU prologue and one fp16 rounding;
  // padding voxels and channels past C stay zero.
  auto halo_store = [&](int c0) {
    if constexpr (PLAN) {
      const int c = c0 + cg * 8;
      const bool cval = c < p.C;
      float sc[8], of[8];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        sc[2 * q] = p.affine ? haff[q][0] : 1.f;
        of[2 * q] = p.affine ? haff[q][1] : 0.f;
        sc[2 * q + 1] = p.affine ? haff[q][2] : 1.f;
        of[2 * q + 1] = p.affine ? haff[q][3] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < NHMAX; j++) {
        if (hlo[j] < 0) continue;
        E8 v = hval[j];
        if (xf) {
          const bool ok = cval && hvi[j] != ~0u;
#pragma unroll
          for (int e = 0; e < 8; e++) {
            float yv = (float)v[e] * sc[e] + of[e];
            if (p.silu) yv = silu_f(yv);
            v[e] = ok ? (E)yv : (E)0;
          }
        }
        *reinterpret_cast<E8*>(halo + hlo[j]) = v;
      }
    }
  };

  f32x16 acc[FO][FV];
#pragma unroll
  for (int i = 0; i < FO; i++)
#pragma unroll
    for (int j = 0; j < FV; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // Prologue: the first chunk's halo, then the first WPF weight stages (the last stage
  // repeats past the end: repeats land in slots no stage uses before they are
  // rewritten), all requested before the first wait.
  if constexpr (PLAN) halo_issue(c_begin);
#pragma unroll
  for (int st = 0; st < WPF; st++) issue_stage(st);

  // Operand fragments double-buffered in registers: while the MFMAs of tap t run, the
  // A (weight ring) and B (halo) fragments of tap t + 1 are read from LDS.
  E8 ra[2][FO][KSG], rb[2][FV][KSG];
  auto load_frags = [&](int set, int stage, int tap) {
    const int kd = tap / (KSZ * KSZ), kh = (tap / KSZ) % KSZ, kw = tap % KSZ;
    const int toff = kd * sd + kh * sh + kw * PITCH;
    const E* wst = wring + (stage % WRING) * WSTAGE + (tap % TPS) * (NFRAG * 512) + lane * 8;
#pragma unroll
    for (int kk = 0; kk < KSG; kk++) {
#pragma unroll
      for (int fo = 0; fo < FO; fo++)
        ra[set][fo][kk] = *reinterpret_cast<const E8*>(wst + ((wo * FO + fo) * KSG + kk) * 512);
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
        rb[set][fv][kk] = *reinterpret_cast<const E8*>(halo + lbase[fv] + toff + kk * 16);
    }
  };
  auto mfma_frags = [&](int set) {
#pragma unroll
    for (int kk = 0; kk < KSG; kk++)
#pragma unroll
      for (int fo = 0; fo < FO; fo++)
#pragma unroll
        for (int fv = 0; fv < FV; fv++) acc[fo][fv] = mfma32(ra[set][fo][kk], rb[set][fv][kk], acc[fo][fv]);
  };

  int st = 0;
  bool pf = true;   // the current chunk's halo is in hval (planned path)
  // Every split owns at least one channel chunk (do-while: no zero-trip branch, before
  // which the compiler would drain the loads just issued).
  int c0 = c_begin;
  do {
    if constexpr (PLAN) {
      if (c0 == c_begin) {
        // The first halo and the weight stages behind it have landed; saying so also
        // clears the compiler's view of pending loads, which would otherwise drain the
        // weight prefetch at every tap.
        vmcnt_wait<0>();
      } else if (pf) {
        // Requested during the previous chunk's last stages; younger than them are only
        // the weight stages of its last WPF - 1 stages.
        vmcnt_wait<(WPF - 1) * LW * TPS>();
        __syncthreads();  // previous chunk done with the halo
      } else {
        __syncthreads();  // previous chunk done with the halo
        halo_issue(c0);
        vmcnt_wait<0>();
      }
      halo_store(c0);
    } else {
      __syncthreads();  // previous chunk done with the halo
      load_halo<CC, VEC, NT>(p, halo, b, c0, gd0, gh0, gw0);
      vmcnt_wait<0>();
    }
    __syncthreads();
    // Prefetch the next chunk's halo during this chunk's last taps.
    const bool pf_next = PLAN && TPF > 0 && c0 + CC < c_end;
    load_frags(0, st, 0);
#pragma unroll
    for (int tap = 0; tap < TAPS; tap++) {
      const int sc = tap / TPS;   // stage of this tap within the chunk
      if (tap % TPS == 0) {
        // Stage st + sc + 1 has landed once only the WPF - 2 stages after it (and, after
        // TPF, the next chunk's halo loads) may be pending; the barrier publishes every
        // wave's part of it and retires stage st + sc - 1 (its last tap was read into
        // registers before this stage began), whose slot the next load reuses.
        if (sc > TPF && pf_next) vmcnt_wait<(WPF - 2) * LW * TPS + NHL>();
        else vmcnt_wait<(WPF - 2) * LW * TPS>();
        __syncthreads();
        issue_stage((st + sc + WPF) % WRING);
        if (sc == TPF && pf_next) halo_issue(c0 + CC);
      }
      if (tap + 1 < TAPS) load_frags((tap + 1) & 1, st + (tap + 1) / TPS, tap + 1);
      mfma_frags(tap & 1);
      if (tap + 1 < TAPS) interleave_reads_mfma<(FO + FV) * KSG, FO * FV * KSG>();
    }
    st += SPC;
    pf = pf_next;
    c0 += CC;
  } while (c0 < c_end);
  // Drain the trailing (repeated) weight loads before the LDS is reused or released.
  vmcnt_wait<0>();

  constexpr int EPW = FO * 32 + 4;   // epilogue staging pitch (floats)
  float* stg;
  if (p.stg_off > 0) {
    // A staging area of its own past the halo: no wait for the other waves.
    stg = reinterpret_cast<float*>(smem) + p.stg_off + w4 * 32 * EPW;
  } else {
    __syncthreads();  // every wave is done with the halo and the weight rings
    stg = reinterpret_cast<float*>(smem) + w4 * 32 * EPW;
  }
  conv_epilogue<FO, FV>(p, ec, acc, stg, lane, wv, b, sidx, pd, ph, pw, d0, h0, w0,
                        (parity * p.nbr + brick) * (WV * FV) + wv * FV);
}

// Pointwise conv / dense layer: a GEMM whose operands both come straight from global
// memory in MFMA lane order -- A is one 1 KB packed-weight fragment per 16-byte-per-lane
// load, B is 16 bytes of one voxel row per lane -- PD k-steps in flight in registers, no
// LDS in the main loop (a 1 x 1 x 1 tap has no halo to share). The optional per-(b, c)
// affine + SiLU prologue is applied to B in registers. The host presents the volume
// flattened (D = H = 1, W = voxels) so the conv epilogue maps voxel slots directly.
template <int WO, int WV, int FO, int FV>
__global__ __launch_bounds__(256) void dense_kernel(ConvParams p) {
  touch_args(p);
  constexpr int BO = WO * FO * 32, BV = WV * FV * 32;
  constexpr int PD = 4;                       // k-steps of operands in flight
  constexpr int EPW = FO * 32 + 4;
  extern __shared__ __attribute__((aligned(16))) E smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wo = wave / WV, wv = wave - wo * WV;
  const int hf = lane >> 5;
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
  }
  const int nob = (p.O + BO - 1) / BO, nvb = p.NBW;
  const int oblk = wg % nob, vb = (wg / nob) % nvb, b = wg / nob / nvb;
  const int NV = p.W;                          // voxels per batch item
  const int ob0 = oblk * (BO / 32) + wo * FO;  // first 32-row output block of this wave
  const int nk = (p.C + 15) / 16;              // k-steps
  const int nk0 = p.C1 > 0 ? p.C0 / 16 : nk;   // k-steps read from x0 (C0 % 16 == 0 with x1)

  // B rows: voxel (vb * BV + (wv * FV + fv) * 32 + lane % 32), clamped into the volume
  // (slots past it compute on the last voxel and are not stored).
  const int64_t bvox = (int64_t)b * NV;
  const auto r0 = make_rsrc(p.x0 + bvox * p.x0p, (unsigned)((int64_t)NV * p.x0p * 2));
  const auto r1 = p.C1 > 0 ? make_rsrc(p.x1 + bvox * p.x1p, (unsigned)((int64_t)NV * p.x1p * 2)) : r0;
  unsigned boff0[FV], boff1[FV];
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    const int v = min(vb * BV + (wv * FV + fv) * 32 + (lane & 31), NV - 1);
    boff0[fv] = (unsigned)(v * p.x0p * 2 + hf * 16);
    boff1[fv] = (unsigned)(v * p.x1p * 2 + hf * 16);
  }
  const auto rw = make_rsrc(p.w, (unsigned)((size_t)p.NOB * p.NKC * 1024));
  const unsigned aoff = (unsigned)lane * 16u;
  const float* aff = p.affine ? p.affine + (int64_t)b * p.C * 2 : nullptr;
  const EpiConst ec = epi_const<FO>(p, lane, ob0, b);

  E8 ra[PD][FO], rb[PD][FV];
  auto load = [&](int set, int kc) {
#pragma unroll
    for (int fo = 0; fo < FO; fo++)
      ra[set][fo] = buffer_load16<E8>(rw, aoff, (unsigned)((ob0 + fo) * p.NKC + kc) * 1024u);
    const bool in0 = kc < nk0;
#pragma unroll
    for (int fv = 0; fv < FV; fv++)
      rb[set][fv] = in0 ? buffer_load16<E8>(r0, boff0[fv], (unsigned)kc * 32u)
                        : buffer_load16<E8>(r1, boff1[fv], (unsigned)(kc - nk0) * 32u);
  };
  auto prep = [&](int set, int kc) {
    // Channels past C (C % 16 != 0) meet zero weights; zero them so stray values cannot
    // turn into NaN. Then the optional affine + SiLU, one fp16 rounding.
    const int c = kc * 16 + hf * 8;
    if (c + 8 > p.C) {
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
#pragma unroll
        for (int e = 0; e < 8; e++)
          if (c + e >= p.C) rb[set][fv][e] = (E)0;
    }
    if (aff || p.silu) {
      float sc[8], of[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const bool ok = aff && c + e < p.C;
        sc[e] = ok ? aff[(c + e) * 2] : 1.f;
        of[e] = ok ? aff[(c + e) * 2 + 1] : 0.f;
      }
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          float y = (float)rb[set][fv][e] * sc[e] + of[e];
          if (p.silu) y = silu_f(y);
          rb[set][fv][e] = c + e < p.C ? (E)y : (E)0;
        }
    }
  };

  f32x16 acc[FO][FV];
#pragma unroll
  for (int i = 0; i < FO; i++)
#pragma unroll
    for (int j = 0; j < FV; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

#pragma unroll
  for (int j = 0; j < PD - 1; j++)
    if (j < nk) load(j, j);
  for (int kc0 = 0; kc0 < nk; kc0 += PD) {
#pragma unroll
    for (int j = 0; j < PD; j++) {
      const int kc = kc0 + j;
      if (kc < nk) {
        if (kc + PD - 1 < nk) load((j + PD - 1) % PD, kc + PD - 1);
        prep(j, kc);
#pragma unroll
        for (int fo = 0; fo < FO; fo++)
#pragma unroll
          for (int fv = 0; fv < FV; fv++) acc[fo][fv] = mfma32(ra[j][fo], rb[j][fv], acc[fo][fv]);
      }
    }
  }
  conv_epilogue<FO, FV>(p, ec, acc, reinterpret_cast<float*>(smem) + wave * 32 * EPW, lane, wv, b, 0, 0, 0,
                        0, 0, 0, vb * BV);
}

// Pointwise conv / dense layer for few output tiles: the 4 waves of a workgroup share
// one FO x FV block of 32 x 32 output tiles and split its k-steps four ways (a short
// dependent chain per wave, all of its operands requested up front), then add their
// partial sums through LDS in a fixed order (waves 1, 2, 3 into wave 0), which finishes
// the epilogue.
// LN: the input rows are layer-normalized first (ldx_dense_ln; one 32 x 32 tile, C <= 512
// so that every k-step of a wave is in registers at once): row mean, then the mean squared
// deviation (two passes, as the standalone LayerNorm kernel), summed per lane, lane pair
// and wave, then fp16((x - mean) * rstd * gamma + beta) as the B operand.
template <int FO, int FV, bool LN = false>
__global__ __launch_bounds__(256) void dense_ksplit_kernel(ConvParams p) {
  touch_args(p);
  constexpr int BO = FO * 32, BV = FV * 32;
  constexpr int PD = 8;                       // k-steps of operands in flight per wave
  constexpr int EPW = FO * 32 + 4;
  constexpr int PART = FO * FV * 1024;        // floats of one wave's partial block
  extern __shared__ __attribute__((aligned(16))) E smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hf = lane >> 5;
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
  }
  const int nob = (p.O + BO - 1) / BO, nvb = p.NBW;
  const int oblk = wg % nob, vb = (wg / nob) % nvb, b = wg / nob / nvb;
  const int NV = p.W;
  const int ob0 = oblk * FO;
  const int nk = (p.C + 15) / 16;
  const int nk0 = p.C1 > 0 ? p.C0 / 16 : nk;
  const int kb = wave * nk / 4, ke = (wave + 1) * nk / 4;   // this wave's k-steps

  const int64_t bvox = (int64_t)b * NV;
  const auto r0 = make_rsrc(p.x0 + bvox * p.x0p, (unsigned)((int64_t)NV * p.x0p * 2));
  const auto r1 = p.C1 > 0 ? make_rsrc(p.x1 + bvox * p.x1p, (unsigned)((int64_t)NV * p.x1p * 2)) : r0;
  unsigned boff0[FV], boff1[FV];
#pragma unroll
  for (int fv = 0; fv < FV; fv++) {
    const int v = min(vb * BV + fv * 32 + (lane & 31), NV - 1);
    boff0[fv] = (unsigned)(v * p.x0p * 2 + hf * 16);
    boff1[fv] = (unsigned)(v * p.x1p * 2 + hf * 16);
  }
  const auto rw = make_rsrc(p.w, (unsigned)((size_t)p.NOB * p.NKC * 1024));
  const unsigned aoff = (unsigned)lane * 16u;
  const float* aff = p.affine ? p.affine + (int64_t)b * p.C * 2 : nullptr;
  const EpiConst ec = epi_const<FO>(p, lane, ob0, b);

  E8 ra[PD][FO], rb[PD][FV];
  auto load = [&](int set, int kc) {
#pragma unroll
    for (int fo = 0; fo < FO; fo++)
      ra[set][fo] = buffer_load16<E8>(rw, aoff, (unsigned)((ob0 + fo) * p.NKC + kc) * 1024u);
    const bool in0 = kc < nk0;
#pragma unroll
    for (int fv = 0; fv < FV; fv++)
      rb[set][fv] = in0 ? buffer_load16<E8>(r0, boff0[fv], (unsigned)kc * 32u)
                        : buffer_load16<E8>(r1, boff1[fv], (unsigned)(kc - nk0) * 32u);
  };
  auto prep = [&](int set, int kc) {
    const int c = kc * 16 + hf * 8;
    if (c + 8 > p.C) {
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
#pragma unroll
        for (int e = 0; e < 8; e++)
          if (c + e >= p.C) rb[set][fv][e] = (E)0;
    }
    if (aff || p.silu) {
      float sc[8], of[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const bool ok = aff && c + e < p.C;
        sc[e] = ok ? aff[(c + e) * 2] : 1.f;
        of[e] = ok ? aff[(c + e) * 2 + 1] : 0.f;
      }
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          float y = (float)rb[set][fv][e] * sc[e] + of[e];
          if (p.silu) y = silu_f(y);
          rb[set][fv][e] = c + e < p.C ? (E)y : (E)0;
        }
    }
  };

  f32x16 acc[FO][FV];
#pragma unroll
  for (int i = 0; i < FO; i++)
#pragma unroll
    for (int j = 0; j < FV; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  float* red = reinterpret_cast<float*>(smem);
  if constexpr (LN) {
    static_assert(FO == 1 && FV == 1, "LayerNorm dense: one 32 x 32 tile");
    const int nks = ke - kb;   // <= PD (the host bounds C)
#pragma unroll
    for (int j = 0; j < PD; j++)
      if (j < nks) load(j, kb + j);
    // gamma and beta of the whole row into LDS (read back after the first barrier): kept
    // out of registers, so that four waves per SIMD still fit.
    float* lnr = red + 3 * PART + 32 * EPW;   // [2][4 waves][32 rows], then gamma, beta
    float* lng = lnr + 256;
    for (int i = threadIdx.x; i < p.C / 4; i += 256) {
      *reinterpret_cast<f32x4*>(lng + 4 * i) = *reinterpret_cast<const f32x4*>(p.ln_g + 4 * i);
      *reinterpret_cast<f32x4*>(lng + 512 + 4 * i) = *reinterpret_cast<const f32x4*>(p.ln_b + 4 * i);
    }
    const int col = lane & 31;
    float sm = 0.f;
#pragma unroll
    for (int j = 0; j < PD; j++)
      if (j < nks)
#pragma unroll
        for (int e = 0; e < 8; e++) sm += (float)rb[j][0][e];
    sm += __shfl_xor(sm, 32);
    if (hf == 0) lnr[wave * 32 + col] = sm;
    __syncthreads();
    const float mean = (((lnr[col] + lnr[32 + col]) + lnr[64 + col]) + lnr[96 + col]) / (float)p.C;
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < PD; j++)
      if (j < nks)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float dv = (float)rb[j][0][e] - mean;
          sq += dv * dv;
        }
    sq += __shfl_xor(sq, 32);
    if (hf == 0) lnr[128 + wave * 32 + col] = sq;
    __syncthreads();
    const float var = (((lnr[128 + col] + lnr[160 + col]) + lnr[192 + col]) + lnr[224 + col]) / (float)p.C;
    const float rstd = 1.0f / sqrtf(var + p.ln_eps);
#pragma unroll
    for (int j = 0; j < PD; j++)
      if (j < nks) {
        const int c = (kb + j) * 16 + hf * 8;
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(lng + c), g1 = *reinterpret_cast<const f32x4*>(lng + c + 4);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(lng + 512 + c);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(lng + 512 + c + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          rb[j][0][e] = (E)(((float)rb[j][0][e] - mean) * rstd * g0[e] + b0[e]);
          rb[j][0][e + 4] = (E)(((float)rb[j][0][e + 4] - mean) * rstd * g1[e] + b1[e]);
        }
        acc[0][0] = mfma32(ra[j][0], rb[j][0], acc[0][0]);
      }
  } else {
#pragma unroll
    for (int j = 0; j < PD - 1; j++)
      if (kb + j < ke) load(j, kb + j);
    for (int kc0 = kb; kc0 < ke; kc0 += PD) {
#pragma unroll
      for (int j = 0; j < PD; j++) {
        const int kc = kc0 + j;
        if (kc < ke) {
          if (kc + PD - 1 < ke) load((j + PD - 1) % PD, kc + PD - 1);
          prep(j, kc);
#pragma unroll
          for (int fo = 0; fo < FO; fo++)
#pragma unroll
            for (int fv = 0; fv < FV; fv++) acc[fo][fv] = mfma32(ra[j][fo], rb[j][fv], acc[fo][fv]);
        }
      }
    }
  }

  // Partial sums of waves 1..3 -> LDS (lane-major), then wave 0 adds them in order.
  if (wave > 0) {
#pragma unroll
    for (int fo = 0; fo < FO; fo++)
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
          const f32x4 q = {acc[fo][fv][e4 * 4], acc[fo][fv][e4 * 4 + 1], acc[fo][fv][e4 * 4 + 2],
                           acc[fo][fv][e4 * 4 + 3]};
          *reinterpret_cast<f32x4*>(red + (wave - 1) * PART + ((fo * FV + fv) * 4 + e4) * 256 + lane * 4) = q;
        }
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int w = 0; w < 3; w++)
#pragma unroll
    for (int fo = 0; fo < FO; fo++)
#pragma unroll
      for (int fv = 0; fv < FV; fv++)
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
          const f32x4 q = *reinterpret_cast<const f32x4*>(red + w * PART + ((fo * FV + fv) * 4 + e4) * 256 + lane * 4);
#pragma unroll
          for (int r = 0; r < 4; r++) acc[fo][fv][e4 * 4 + r] += q[r];
        }
  conv_epilogue<FO, FV>(p, ec, acc, red + 3 * PART, lane, 0, b, 0, 0, 0, 0, 0, 0, vb * BV);
}

// Split-K finish: sum the fp32 partial planes in split order, then the same epilogue
// as the single-pass kernel (bias, scale, residual, one rounding, optional GELU).
__global__ __launch_bounds__(256) void conv_reduce_kernel(ConvParams p, int64_t nvox) {
  touch_args(p);
  const int64_t n = nvox * p.O;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ov = i / p.O;
    const int o = (int)(i - ov * p.O);
    float v = 0.f;
    for (int s2 = 0; s2 < p.split; s2++) v += p.part[(int64_t)s2 * n + i];
    const int64_t vol = nvox / p.B;
    const int b = (int)(ov / vol);
    float add = p.bias ? p.bias[(p.bias_batched ? (int64_t)b * p.O : 0) + o] : 0.f;
    if (p.shift) add += (float)p.shift[(int64_t)b * p.shiftp + o];
    v = (v + add) * p.scale;
    if (p.res) v += (float)p.res[ov * p.resp + o];
    p.y[ov * p.yp + o] = post_act((E)v, p.act);
  }
}

// Split-K finish with 16-byte accesses (O a multiple of 8, aligned rows; B x voxels x O / 8
// below 2^31): thread per (voxel, 8 channels), partial planes summed in split order, then
// conv_reduce_kernel's epilogue.
__global__ __launch_bounds__(256) void conv_reduce8_kernel(ConvParams p, int nvox) {
  touch_args(p);
  const int G8 = p.O >> 3;
  const int n8 = nvox * G8;
  const int vol = nvox / p.B;
  const int64_t plane = (int64_t)nvox * p.O;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n8; i += gridDim.x * 256) {
    const int ov = i / G8;
    const int o = (i - ov * G8) * 8;
    const int b = ov / vol;
    const float* src = p.part + (int64_t)ov * p.O + o;
    f32x4 lo = *reinterpret_cast<const f32x4*>(src), hi = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll 4
    for (int s2 = 1; s2 < p.split; s2++) {
      lo += *reinterpret_cast<const f32x4*>(src + s2 * plane);
      hi += *reinterpret_cast<const f32x4*>(src + s2 * plane + 4);
    }
    float add[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
      const float* bb = p.bias + (p.bias_batched ? (int64_t)b * p.O : 0) + o;
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(bb), b1 = *reinterpret_cast<const f32x4*>(bb + 4);
#pragma unroll
      for (int r = 0; r < 4; r++) { add[r] = b0[r]; add[r + 4] = b1[r]; }
    }
    if (p.shift) {
      const E8 sh = *reinterpret_cast<const E8*>(p.shift + (int64_t)b * p.shiftp + o);
#pragma unroll
      for (int r = 0; r < 8; r++) add[r] += (float)sh[r];
    }
    E8 rs = {};
    if (p.res) rs = *reinterpret_cast<const E8*>(p.res + (int64_t)ov * p.resp + o);
    E8 out;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float v = (lo[r] + add[r]) * p.scale;
      if (p.res) v += (float)rs[r];
      out[r] = post_act((E)v, p.act);
      float w = (hi[r] + add[r + 4]) * p.scale;
      if (p.res) w += (float)rs[r + 4];
      out[r + 4] = post_act((E)w, p.act);
    }
    *reinterpret_cast<E8*>(p.y + (int64_t)ov * p.yp + o) = out;
  }
}

// Split-K finish that also leaves GroupNorm partial moments: workgroup (k, b) of 1024
// threads finishes output voxels [32 k, 32 k + 32) of batch item b, thread t the 8
// channels 8 (t % G8) .. (G8 = O / 8 <= 64) of voxels t / G8 + j * VP (VP = 1024 / G8 per
// pass, at most two passes) -- partial planes summed in split order, then the
// conv_reduce_kernel epilogue, 16-byte accesses. Per channel pair, the block's (count,
// mean, M2): per-thread sums added through LDS in voxel order, the mean first, then the
// squared deviations of the values the thread kept.
constexpr int RS_THREADS = 1024;
constexpr int RS_PASSES = 2;   // 32 / VP passes: VP >= 16 for O <= 512
__global__ __launch_bounds__(RS_THREADS) void conv_reduce_stats_kernel(ConvParams p, int ovol) {
  touch_args(p);
  __shared__ float part4[RS_THREADS * 4];
  __shared__ float pmean[256];
  const int G8 = p.O >> 3, VP = RS_THREADS / G8;
  const int t = threadIdx.x, g = t % G8, vs = t / G8, o = g * 8;
  const int k = blockIdx.x, b = blockIdx.y;
  const int nv = min(32, ovol - k * 32);
  const int64_t plane = (int64_t)p.B * ovol * p.O;
  E8 keep[RS_PASSES];
  bool okj[RS_PASSES];
  f32x4 lo[RS_PASSES], hi[RS_PASSES];
  E8 rs[RS_PASSES];
  int64_t ov[RS_PASSES];
  // Every pass's operands requested before any is summed.
#pragma unroll
  for (int j = 0; j < RS_PASSES; j++) {
    const int v = vs + j * VP;
    okj[j] = vs < VP && v < nv;
    ov[j] = (int64_t)b * ovol + k * 32 + (okj[j] ? v : 0);
    lo[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    hi[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    rs[j] = (E8){0, 0, 0, 0, 0, 0, 0, 0};
    if (okj[j] && p.res) rs[j] = *reinterpret_cast<const E8*>(p.res + ov[j] * p.resp + o);
  }
#pragma unroll 4
  for (int s2 = 0; s2 < p.split; s2++)
#pragma unroll
    for (int j = 0; j < RS_PASSES; j++)
      if (okj[j]) {
        const float* src = p.part + s2 * plane + ov[j] * p.O + o;
        lo[j] += *reinterpret_cast<const f32x4*>(src);
        hi[j] += *reinterpret_cast<const f32x4*>(src + 4);
      }
  float add[8];
  {
    const float* bias = p.bias ? p.bias + (p.bias_batched ? (int64_t)b * p.O : 0) + o : nullptr;
    f32x4 b0 = {0.f, 0.f, 0.f, 0.f}, b1 = {0.f, 0.f, 0.f, 0.f};
    if (bias && vs < VP) { b0 = *reinterpret_cast<const f32x4*>(bias); b1 = *reinterpret_cast<const f32x4*>(bias + 4); }
    E8 sh = {};
    if (p.shift && vs < VP) sh = *reinterpret_cast<const E8*>(p.shift + (int64_t)b * p.shiftp + o);
#pragma unroll
    for (int r = 0; r < 4; r++) { add[r] = b0[r] + (float)sh[r]; add[r + 4] = b1[r] + (float)sh[r + 4]; }
  }
  float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < RS_PASSES; j++) {
    keep[j] = (E8){0, 0, 0, 0, 0, 0, 0, 0};
    if (!okj[j]) continue;
    E8 out;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      out[r] = post_act((E)((lo[j][r] + add[r]) * p.scale + (float)rs[j][r]), p.act);
      out[r + 4] = post_act((E)((hi[j][r] + add[r + 4]) * p.scale + (float)rs[j][r + 4]), p.act);
    }
    *reinterpret_cast<E8*>(p.y + ov[j] * p.yp + o) = out;
    keep[j] = out;
#pragma unroll
    for (int q = 0; q < 4; q++) s4[q] += (float)out[2 * q] + (float)out[2 * q + 1];
  }
  const float n = 2.0f * (float)nv;
  const int npair = p.O >> 1;
#pragma unroll
  for (int q = 0; q < 4; q++) part4[t * 4 + q] = s4[q];
  __syncthreads();
  if (t < npair) {
    float a = 0.f;
    for (int u = 0; u < VP; u++) a += part4[(u * G8 + t / 4) * 4 + t % 4];
    pmean[t] = a / n;
  }
  __syncthreads();
  float m4[4] = {0.f, 0.f, 0.f, 0.f};
  if (vs < VP) {
    float mu[4];
#pragma unroll
    for (int q = 0; q < 4; q++) mu[q] = pmean[g * 4 + q];
#pragma unroll
    for (int j = 0; j < RS_PASSES; j++)
      if (okj[j])
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float d0 = (float)keep[j][2 * q] - mu[q], d1 = (float)keep[j][2 * q + 1] - mu[q];
          m4[q] += d0 * d0 + d1 * d1;
        }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; q++) part4[t * 4 + q] = m4[q];
  __syncthreads();
  if (t < npair) {
    float m2 = 0.f;
    for (int u = 0; u < VP; u++) m2 += part4[(u * G8 + t / 4) * 4 + t % 4];
    float* dst = p.stats + (((int64_t)b * p.schunks + k) * npair + t) * 3;
    dst[0] = n; dst[1] = pmean[t]; dst[2] = m2;
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
static int launch(ConvParams& p, int grid_z, hipStream_t stream, size_t halo_bytes) {
  constexpr int BO = WO * FO * 32;
  constexpr int NT = 256, VPI = NT / (CC / 8);
  auto al16 = [](size_t n) { return (n + 15) & ~(size_t)15; };
  const int hvox = p.HD * p.HH * p.HW;
  p.nh = VEC ? (hvox + VPI - 1) / VPI : 0;
  if (p.nh > NHMAX) p.nh = 0;
  // Whole kw rows per weight stage on the planned halo path when the planner asks.
  const int tps = VEC && p.nh > 0 && p.tps > 1 ? KSZ : 1;
  // LDS: the weight ring and the halo; then the epilogue staging.
  const size_t ring = (size_t)WRING * tps * (BO / 32) * (CC / 16) * 1024;
  const size_t main_bytes = ring + al16(halo_bytes);
  const size_t stg = (size_t)4 * 32 * (FO * 32 + 4) * sizeof(float);
  size_t lds;
  p.stg_off = 0;
  {
    // The staging gets an area of its own (no barrier before the epilogue) unless that
    // costs a workgroup per CU.
    const size_t overlap = std::max(main_bytes, stg), sep = main_bytes + stg;
    if (sep <= 160 * 1024 && (160 * 1024) / sep >= (160 * 1024) / overlap) {
      p.stg_off = (int)(main_bytes / sizeof(float));
      lds = sep;
    } else {
      lds = overlap;
    }
  }
  if (lds > 160 * 1024) return fail("conv3d: %zu bytes of LDS needed", lds);
  p.nob = (p.O + BO - 1) / BO;
  const int64_t nbr = (int64_t)p.NBD * p.NBH * p.NBW;
  const int64_t nwg = nbr * p.nob * grid_z;
  if (nwg > 0x7fffffff) return fail("conv3d: grid too large");
  p.nbr = (int)nbr;
  p.dv_nob = make_udiv((unsigned)p.nob);
  p.dv_nbr = make_udiv((unsigned)p.nbr);
  p.dv_split = make_udiv((unsigned)p.split);
  p.dv_nbw = make_udiv((unsigned)p.NBW);
  p.dv_nbh = make_udiv((unsigned)p.NBH);
  dim3 grid((unsigned)nwg);
  void (*kern)(ConvParams);
  if constexpr (VEC) {
    kern = p.nh == 0   ? conv3d_kernel<WO, WV, FO, FV, CC, KSZ, true, false, 1>
           : tps > 1 ? conv3d_kernel<WO, WV, FO, FV, CC, KSZ, true, true, KSZ>
                     : conv3d_kernel<WO, WV, FO, FV, CC, KSZ, true, true, 1>;
  } else {
    kern = conv3d_kernel<WO, WV, FO, FV, CC, KSZ, false, false, 1>;
  }
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
  if constexpr (KSZ == 1) {
    // Pointwise convs with 16-byte channel groups run as dense_kernel; this path only
    // serves the remaining ones, through the scalar staging loop.
    return fail("conv3d: vectorised pointwise conv belongs to the dense path");
  } else {
    if (cc == 64) return launch<WO, WV, FO, FV, 64, KSZ, true>(p, grid_z, stream, lds);
    return launch<WO, WV, FO, FV, 32, KSZ, true>(p, grid_z, stream, lds);
  }
}
template <int WO, int WV, int FO, int FV>
static int dispatch_k(ConvParams& p, int cc, bool vec, int grid_z, hipStream_t stream, size_t lds) {
  if (p.taps == 27) return dispatch_cc<WO, WV, FO, FV, 3>(p, cc, vec, grid_z, stream, lds);
  if (p.taps == 8) return dispatch_cc<WO, WV, FO, FV, 2>(p, cc, vec, grid_z, stream, lds);
  return dispatch_cc<WO, WV, FO, FV, 1>(p, cc, false, grid_z, stream, lds);
}


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
  p.x0 = (const E*)a->x0; p.x0p = a->x0_pitch;
  p.x1 = (const E*)a->x1; p.x1p = a->x1_pitch;
  p.w = (const E*)a->weight;
  p.bias = a->bias; p.bias_batched = a->bias_batched ? 1 : 0;
  p.shift = (const E*)a->shift; p.shiftp = a->shift_pitch;
  p.affine = a->affine; p.silu = a->silu ? 1 : 0;
  p.res = (const E*)a->residual; p.resp = a->residual_pitch;
  p.scale = a->output_scale; p.act = a->act;
  p.y = (E*)a->y; p.yp = a->y_pitch;
  p.yvec = (p.yp % 4 == 0) && ((uintptr_t)a->y % 8 == 0);
  p.ep_vec = p.yp % 8 == 0 && (uintptr_t)a->y % 16 == 0 &&
             (!a->residual || (p.resp % 8 == 0 && (uintptr_t)a->residual % 16 == 0)) &&
             (!a->shift || (p.shiftp % 8 == 0 && (uintptr_t)a->shift % 16 == 0)) &&
             (!a->bias || ((uintptr_t)a->bias % 16 == 0 && (!a->bias_batched || p.O % 4 == 0))) &&
             p.O % 4 == 0 && (!a->workspace || (uintptr_t)a->workspace % 16 == 0);

  // 16-byte halo reads through a buffer resource per batch item (byte offsets < 2 GiB).
  const int64_t in_vol = (int64_t)p.D * p.H * p.W;
  vec = (p.C0 % 8 == 0) && (p.x0p % 8 == 0) && (p.C1 == 0 || (p.C1 % 8 == 0 && p.x1p % 8 == 0)) &&
        ((uintptr_t)a->x0 % 16 == 0) && (p.C1 == 0 || (uintptr_t)a->x1 % 16 == 0) &&
        in_vol * p.x0p * 2 < ((int64_t)1 << 31) && (p.C1 == 0 || in_vol * p.x1p * 2 < ((int64_t)1 << 31));

  // Tiles: (waves over O) x (waves over voxels), 32x32 MFMA blocks per wave; chosen
  // from measured sweeps on MI355X: 64x64 wave tiles when the volume fills the GPU,
  // smaller tiles (plus split-K below) for the coarse UNet levels.
  const int64_t rows = (int64_t)p.B * p.RD * p.RH * p.RW * (p.upsample ? 8 : 1);
  // At most 32 outputs: 32 x 256 tiles, 32 x 128 below 64k voxels (measured: 32x40x40,
  // 64 -> 4 channels 19.3 -> 16.0 us).
  if (p.O <= 32) t = rows >= 65536 ? Tile{1, 4, 1, 2, 32} : Tile{1, 4, 1, 1, 32};
  // 64 outputs: 128-voxel tiles, or 64-voxel ones (twice the workgroups) for grids of
  // fewer than 128 such tiles and for the scalar-staged inputs (measured: the 16x20x20
  // stride-2 output 20.4 -> 15.0 us, the 9-channel conv_in at 32x40x40 20.9 -> 18.8 us).
  else if (p.O <= 64) t = vec && rows / 128 >= 128 ? Tile{1, 4, 2, 1, 32} : Tile{2, 2, 1, 1, 32};
  // Upsampling convs whose 128 x 128 tiles make 256 workgroups or more (measured:
  // 16x20x20 -> 32x40x40 at 128 channels 36.5 -> 24.3 us against 64 x 64 tiles; the VQ
  // decoder's 32x40x40 -> 64x80x80 at 256 channels 624 -> 545 us and 64x80x80 ->
  // 128x160x160 at 128 channels 1268 -> 1106 us against 64 x 256 tiles; 8x10x10 ->
  // 16x20x20 at 256 channels, 100 such tiles, stays below: 17.2 us there against 34.7).
  else if (p.upsample && rows / 128 * ((p.O + 127) / 128) >= 256) t = {2, 2, 2, 2, 32};
  else if (rows / 256 * ((p.O + 63) / 64) >= 512) t = {1, 4, 2, 2, 32};
  // Small volumes: 64-channel chunks, but 32-channel ones below 256 voxels, where the split
  // over channel chunks then spreads the weights over twice the workgroups (measured:
  // 4x5x5, 256 -> 256 channels 13.4 -> 12.0 us).
  else t = {2, 2, 1, 1, vec && p.taps > 1 && p.C % 64 == 0 && rows > 256 ? 64 : 32};
  // LDX_CONV_TILE="WO,WV,FO,FV,CC" overrides the tile heuristic (tuning sweeps).
  bool forced = false;
  if (const char* env = getenv("LDX_CONV_TILE")) {
    Tile o{};
    const int got = sscanf(env, "%d,%d,%d,%d,%d", &o.WO, &o.WV, &o.FO, &o.FV, &o.CC);
    if (got == 5 && o.WO * o.WV == 4 && (o.CC == 32 || (o.CC == 64 && p.C % 64 == 0 && vec))) {
      t = o;
      forced = true;
    }
  }

  // A channel chunk of the vectorised halo path comes from x0 or from x1, never both.
  if (vec && p.C1 > 0 && p.C0 % t.CC != 0) {
    if (p.C0 % 32 == 0) t.CC = 32;
    else vec = false;
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
    lds = (size_t)p.HD * p.HH * p.RS * sizeof(E);
    const size_t wbytes = (size_t)WRING * (t.BO() / 32) * (t.CC / 16) * 1024;
    if (lds + wbytes <= (forced ? 160u * 1024 : 80u * 1024) || (t.CC == 32 && t.FV == 1)) break;
    if (t.CC == 64) t.CC = 32;
    else t.FV = 1;
  }
  if (lds + (size_t)WRING * (t.BO() / 32) * (t.CC / 16) * 1024 > 160 * 1024)
    return fail("conv3d: halo of %zu bytes exceeds LDS", lds);
  p.NBD = (p.RD + TD - 1) / TD; p.NBH = (p.RH + TH - 1) / TH; p.NBW = (p.RW + TW - 1) / TW;
  p.ID0 = ks == 1 ? 0 : -1; p.IH0 = p.ID0; p.IW0 = p.ID0;
  p.rHW = 1.0f / (float)p.HW; p.rHH = 1.0f / (float)p.HH;
  p.rTW = 1.0f / (float)TW; p.rTH = 1.0f / (float)TH;
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
  // LDX_CONV_SPLIT_WG moves the grid size below which the reduction splits (tuning sweeps).
  int64_t split_below = 192;
  if (const char* env = getenv("LDX_CONV_SPLIT_WG")) split_below = atoll(env);
  if (wgs < split_below && nchunks > 1 && p.taps > 1 && p.C >= 128) {
    int want = (int)((512 + wgs - 1) / wgs);
    if (want > nchunks) want = nchunks;
    p.cps = (nchunks + want - 1) / want;
    p.split = (nchunks + p.cps - 1) / p.cps;
  }
  // Whole kw rows per weight stage (a third of the tap loop's barriers; half for the
  // folded 2 x 2 x 2 upsample taps) when the larger ring still keeps the whole grid
  // resident at once. LDX_CONV_TPS=1 / 3 forces one tap / whole rows (tuning sweeps).
  {
    const int kz = p.upsample ? 2 : ks;
    const size_t ring_row = (size_t)WRING * kz * (t.BO() / 32) * (t.CC / 16) * 1024;
    const size_t lds_row = ring_row + lds + (size_t)4 * 32 * (t.FO * 32 + 4) * sizeof(float);
    const int64_t grid = wgs * p.split;
    p.tps = lds_row <= 160 * 1024 && grid <= (int64_t)256 * (int64_t)((160 * 1024) / lds_row) ? 2 : 1;
    if (const char* env = getenv("LDX_CONV_TPS")) p.tps = atoi(env) > 1 ? 2 : 1;
    if (p.tps > 1 && lds_row > 160 * 1024) p.tps = 1;
  }
  const int64_t nvox = (int64_t)p.B * p.OD * p.OH * p.OW;
  ws_bytes = p.split > 1 ? (int64_t)p.split * nvox * p.O * (int64_t)sizeof(float) : 0;
  if ((int64_t)p.B * (p.upsample ? 8 : 1) * p.split > 65535) return fail("conv3d: batch too large");
  if ((int64_t)p.B * p.OD * p.OH * p.OW >= ((int64_t)1 << 31)) return fail("conv3d: output too large");
  return LDX_OK;
}

// Pointwise convs with 16-byte-aligned channel groups run as a direct-load GEMM over
// the flattened volume (dense_kernel).
static bool use_dense(const ldx_conv3d_args* a, bool vec) {
  return a->ksize == 1 && vec && (a->c1 == 0 || a->c0 % 16 == 0);
}

size_t conv3d_workspace_bytes(const ldx_conv3d_args* a) {
  ConvParams p;
  Tile t;
  size_t lds;
  bool vec;
  int64_t ws = 0;
  if (plan_conv(a, p, t, lds, vec, ws) != LDX_OK) return 0;
  if (use_dense(a, vec)) return 0;
  QuadParams qp;
  if (conv3d_quad_plan(a, &qp)) return 0;
  StreamParams sp;
  if (conv3d_stream_plan(a, &sp, false))
    return sp.split > 1 ? (size_t)sp.split * (size_t)p.B * p.OD * p.OH * p.OW * p.O * sizeof(float) : 0;
  return (size_t)ws;
}

template <int WO, int WV, int FO, int FV>
static int launch_dense(ConvParams p, hipStream_t st) {
  constexpr int BO = WO * FO * 32, BV = WV * FV * 32;
  const int NV = p.D * p.H * p.W;
  p.D = 1; p.H = 1; p.W = NV;
  p.RD = 1; p.RH = 1; p.RW = NV;
  p.OD = 1; p.OH = 1; p.OW = NV;
  p.TD = 1; p.TH = 1; p.TW = BV;
  p.rTW = 1.0f / (float)BV; p.rTH = 1.0f;
  p.NBD = 1; p.NBH = 1; p.NBW = (NV + BV - 1) / BV;
  p.split = 1;
  p.part = nullptr;
  const int64_t nwg = (int64_t)p.NBW * ((p.O + BO - 1) / BO) * p.B;
  if (nwg > 0x7fffffff) return fail("conv3d: grid too large");
  const size_t lds = (size_t)4 * 32 * (FO * 32 + 4) * sizeof(float);
  hipLaunchKernelGGL((dense_kernel<WO, WV, FO, FV>), dim3((unsigned)nwg), dim3(256), lds, st, p);
  return check_launch("conv3d: pointwise");
}

template <int FO, int FV, bool LN = false>
static int launch_dense_ksplit(ConvParams p, hipStream_t st) {
  constexpr int BO = FO * 32, BV = FV * 32;
  const int NV = p.D * p.H * p.W;
  p.D = 1; p.H = 1; p.W = NV;
  p.RD = 1; p.RH = 1; p.RW = NV;
  p.OD = 1; p.OH = 1; p.OW = NV;
  p.TD = 1; p.TH = 1; p.TW = BV;
  p.rTW = 1.0f / (float)BV; p.rTH = 1.0f;
  p.NBD = 1; p.NBH = 1; p.NBW = (NV + BV - 1) / BV;
  p.split = 1;
  p.part = nullptr;
  const int64_t nwg = (int64_t)p.NBW * ((p.O + BO - 1) / BO) * p.B;
  if (nwg > 0x7fffffff) return fail("conv3d: grid too large");
  const size_t lds = (size_t)(3 * FO * FV * 1024 + 32 * (FO * 32 + 4) + (LN ? 256 + 1024 : 0)) * sizeof(float);
  hipLaunchKernelGGL((dense_ksplit_kernel<FO, FV, LN>), dim3((unsigned)nwg), dim3(256), lds, st, p);
  return check_launch("conv3d: pointwise (k-split)");
}

static int run_dense(const ConvParams& p, hipStream_t st) {
  const int64_t nv = (int64_t)p.B * p.D * p.H * p.W;
  // Few 64 x 128 output tiles and a long reduction (>= 16 k-steps): one 32 x 32 tile per
  // workgroup with its k-steps split over the 4 waves (measured on MI355X: 800 x 1024 ->
  // 256 in 6.7 us instead of 13.9 us).
  const int64_t tiles64 = (nv + 127) / 128 * ((p.O + 63) / 64);
  const char* ks_env = getenv("LDX_DENSE_KSPLIT");
  if (ks_env ? atoi(ks_env) != 0 : (tiles64 < 256 && p.C >= 256)) {
    int fo = 1, fv = 1;
    if (const char* env = getenv("LDX_DENSE_KS_TILE")) sscanf(env, "%d,%d", &fo, &fv);
    if (fo == 1 && fv == 1) return launch_dense_ksplit<1, 1>(p, st);
    if (fo == 1 && fv == 2) return launch_dense_ksplit<1, 2>(p, st);
    if (fo == 2 && fv == 1) return launch_dense_ksplit<2, 1>(p, st);
    return launch_dense_ksplit<2, 2>(p, st);
  }
  int wo = 2, wv = 2, fo = 1, fv = 1;
  if (p.O <= 32) { wo = 1; wv = 4; fo = 1; fv = 1; }
  else if (p.O <= 64) { wo = 1; wv = 4; fo = 2; fv = 1; }
  else if ((nv + 127) / 128 * ((p.O + 127) / 128) >= 256) { fo = 2; fv = 2; }
  // LDX_DENSE_TILE="WO,WV,FO,FV" overrides the choice (tuning sweeps).
  if (const char* env = getenv("LDX_DENSE_TILE")) {
    int a0, a1, a2, a3;
    if (sscanf(env, "%d,%d,%d,%d", &a0, &a1, &a2, &a3) == 4) { wo = a0; wv = a1; fo = a2; fv = a3; }
  }
  if (wo == 1 && wv == 4 && fo == 1 && fv == 1) return launch_dense<1, 4, 1, 1>(p, st);
  if (wo == 1 && wv == 4 && fo == 2 && fv == 1) return launch_dense<1, 4, 2, 1>(p, st);
  if (wo == 2 && wv == 2 && fo == 2 && fv == 2) return launch_dense<2, 2, 2, 2>(p, st);
  if (wo == 1 && wv == 4 && fo == 1 && fv == 2) return launch_dense<1, 4, 1, 2>(p, st);
  return launch_dense<2, 2, 1, 1>(p, st);
}

// Split-K finish: the plain reduce, or (stats) the reduce that also leaves the
// GroupNorm moments of 32-voxel blocks.
static int launch_reduce(ConvParams& p, hipStream_t st, const char* what) {
  const int64_t ovol = (int64_t)p.OD * p.OH * p.OW;
  const int64_t nvox = (int64_t)p.B * ovol;
  if (p.stats) {
    hipLaunchKernelGGL(conv_reduce_stats_kernel, dim3((unsigned)((ovol + 31) / 32), (unsigned)p.B), dim3(RS_THREADS), 0,
                       st, p, (int)ovol);
    return check_launch(what);
  }
  const int64_t n = nvox * p.O;
  if (p.ep_vec && p.O % 8 == 0 && n / 8 < ((int64_t)1 << 31)) {
    const int64_t n8 = n / 8;
    const unsigned blocks = (unsigned)((n8 + 255) / 256 < 8192 ? (n8 + 255) / 256 : 8192);
    hipLaunchKernelGGL(conv_reduce8_kernel, dim3(blocks), dim3(256), 0, st, p, (int)nvox);
    return check_launch(what);
  }
  const unsigned blocks = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
  hipLaunchKernelGGL(conv_reduce_kernel, dim3(blocks), dim3(256), 0, st, p, nvox);
  return check_launch(what);
}

// One conv, as planned for these arguments. stats: also the GroupNorm partial moments of
// the output (null: none). With dry, nothing is launched: *chunks receives the voxel
// blocks per batch item the moments are kept for (0: this plan keeps none).
static int conv3d_run(const ldx_conv3d_args* a, float* stats, bool dry, int64_t* chunks, void* stream) {
  ConvParams p;
  Tile t;
  size_t lds;
  bool vec;
  int64_t ws = 0;
  if (chunks) *chunks = 0;
  int rc = plan_conv(a, p, t, lds, vec, ws);
  if (rc != LDX_OK) return rc;
  hipStream_t st = as_stream(stream);
  const int64_t ovol = (int64_t)p.OD * p.OH * p.OW;
  // Moments need the 16-byte epilogue; the split-K reduce keeps them for O <= 512.
  const bool can_stats = p.O % 8 == 0 && p.ep_vec;
  const int64_t reduce_chunks = can_stats && p.O <= 512 ? (ovol + 31) / 32 : 0;
  if (use_dense(a, vec)) {
    if (dry) return LDX_OK;
    if (stats) return fail("conv3d_stats: pointwise convs keep no moments");
    return run_dense(p, st);
  }
  {
    QuadParams qp;
    if (conv3d_quad_plan(a, &qp)) {
      const int64_t ch = can_stats ? qp.schunks : 0;
      if (chunks) *chunks = ch;
      if (dry) return LDX_OK;
      if (stats && ch == 0) return fail("conv3d_stats: this conv keeps no moments");
      qp.stats = stats;
      return conv3d_quad_launch(qp, st);
    }
  }
  {
    StreamParams sp;
    if (conv3d_stream_plan(a, &sp)) {
      const int64_t ch = sp.split == 1 ? (can_stats ? sp.schunks : 0) : reduce_chunks;
      if (chunks) *chunks = ch;
      if (dry) return LDX_OK;
      if (stats && ch == 0) return fail("conv3d_stats: this conv keeps no moments");
      sp.stats = stats;
      rc = conv3d_stream_launch(sp, st);
      if (rc != LDX_OK || sp.split == 1) return rc;
      // Split over channel chunks: the same fixed-order reduce and epilogue as the general
      // kernel's split-K.
      p.split = sp.split;
      p.part = sp.part;
      p.stats = stats;
      p.schunks = (int)ch;
      return launch_reduce(p, st, "conv3d (streamed): split reduce");
    }
  }
  if (p.split > 1 && (!a->workspace || a->workspace_bytes < (size_t)ws)) {
    // No (or too small a) workspace: one pass over all channels.
    p.split = 1;
    p.cps = (p.C + t.CC - 1) / t.CC;
  }
  p.part = p.split > 1 ? (float*)a->workspace : nullptr;
  {
    const int64_t ch = p.split == 1 ? (can_stats ? (int64_t)(p.upsample ? 8 : 1) * p.NBD * p.NBH * p.NBW * t.WV * t.FV : 0)
                                    : reduce_chunks;
    if (chunks) *chunks = ch;
    if (dry) return LDX_OK;
    if (stats && ch == 0) return fail("conv3d_stats: this conv keeps no moments");
    p.stats = stats;
    p.schunks = (int)ch;
  }
  const int grid_z = p.B * (p.upsample ? 8 : 1) * p.split;

#define LDX_TILE(WO_, WV_, FO_, FV_)                                      \
  if (t.WO == WO_ && t.WV == WV_ && t.FO == FO_ && t.FV == FV_)           \
    rc = dispatch_k<WO_, WV_, FO_, FV_>(p, t.CC, vec, grid_z, st, lds);   \
  else
  LDX_TILE(1, 4, 1, 2)
  LDX_TILE(1, 4, 1, 1)
  LDX_TILE(1, 4, 2, 2)
  LDX_TILE(1, 4, 2, 1)
  LDX_TILE(2, 2, 2, 2)
  LDX_TILE(2, 2, 1, 1)
  return fail("conv3d: no kernel for tile");
#undef LDX_TILE
  if (rc != LDX_OK || p.split == 1) return rc;
  return launch_reduce(p, st, "conv3d: split reduce");
}

int conv3d_entry(const ldx_conv3d_args* a, void* stream) {
  return conv3d_run(a, nullptr, false, nullptr, stream);
}

int64_t conv3d_stats_chunks(const ldx_conv3d_args* a) {
  int64_t ch = 0;
  if (!a || conv3d_run(a, nullptr, true, &ch, nullptr) != LDX_OK) return 0;
  return ch;
}

int conv3d_stats(const ldx_conv3d_args* a, float* stats, void* stream) {
  if (!stats) return fail("conv3d_stats: null moments buffer");
  if ((uintptr_t)stats % 16) return fail("conv3d_stats: moments buffer must be 16-byte aligned");
  return conv3d_run(a, stats, false, nullptr, stream);
}

int dense_ln(const ldx_conv3d_args* a, const float* gamma, const float* beta, float eps,
                            void* stream) {
  if (!a || !gamma || !beta) return fail("dense_ln: null pointer");
  if (a->ksize != 1 || a->c1 != 0 || a->affine || a->silu || a->stride != 1 || a->upsample)
    return fail("dense_ln: a pointwise conv of one input without affine or SiLU");
  if (a->c0 % 16 || a->c0 > 512) return fail("dense_ln: C = %d must be a multiple of 16, at most 512", a->c0);
  if ((uintptr_t)gamma % 16 || (uintptr_t)beta % 16) return fail("dense_ln: gamma and beta must be 16-byte aligned");
  if (!(eps > 0.f)) return fail("dense_ln: eps must be positive");
  ConvParams p;
  Tile t;
  size_t lds;
  bool vec;
  int64_t ws = 0;
  int rc = plan_conv(a, p, t, lds, vec, ws);
  if (rc != LDX_OK) return rc;
  if (!use_dense(a, vec)) return fail("dense_ln: input rows must be 16-byte aligned channel groups");
  p.ln_g = gamma;
  p.ln_b = beta;
  p.ln_eps = eps;
  return launch_dense_ksplit<1, 1, true>(p, as_stream(stream));
}

}  // namespace LDX_ELEM_NS
}  // namespace ldx

#if !defined(LDX_ELEM_BF16)
// The C entry points (in the fp16 unit only): argument checks shared by both element
// types, then the planner and kernels of the args' dtype.
namespace ldx {
namespace bf16_path {
size_t conv3d_workspace_bytes(const ldx_conv3d_args* a);
int conv3d_entry(const ldx_conv3d_args* a, void* stream);
int64_t conv3d_stats_chunks(const ldx_conv3d_args* a);
int conv3d_stats(const ldx_conv3d_args* a, float* stats, void* stream);
int dense_ln(const ldx_conv3d_args* a, const float* gamma, const float* beta, float eps, void* stream);
}  // namespace bf16_path
// exact.hip: the FP32 (split-FP16) conv.
size_t conv3d_exact_workspace_bytes(const ldx_conv3d_args* a);
int conv3d_exact(const ldx_conv3d_args* a, void* stream);
}  // namespace ldx

static bool conv_is_bf16(const ldx_conv3d_args* a) { return a && a->dtype == LDX_DTYPE_BF16; }
static bool conv_is_f32(const ldx_conv3d_args* a) { return a && a->dtype == LDX_DTYPE_F32; }
static int conv_dtype_ok(const ldx_conv3d_args* a, bool f32_ok = false) {
  if (a && a->dtype != LDX_DTYPE_F16 && a->dtype != LDX_DTYPE_BF16 && !(f32_ok && a->dtype == LDX_DTYPE_F32))
    return ldx::fail("conv3d: dtype %d is not %s", a->dtype,
                     f32_ok ? "LDX_DTYPE_F16, LDX_DTYPE_BF16 or LDX_DTYPE_F32" : "LDX_DTYPE_F16 or LDX_DTYPE_BF16");
  return LDX_OK;
}

extern "C" size_t ldx_conv3d_workspace_bytes(const ldx_conv3d_args* a) {
  if (conv_dtype_ok(a, true) != LDX_OK) return 0;
  if (conv_is_f32(a)) return ldx::conv3d_exact_workspace_bytes(a);
  return conv_is_bf16(a) ? ldx::bf16_path::conv3d_workspace_bytes(a) : ldx::f16_path::conv3d_workspace_bytes(a);
}

extern "C" int ldx_conv3d(const ldx_conv3d_args* a, void* stream) {
  if (int rc = conv_dtype_ok(a, true)) return rc;
  if (conv_is_f32(a)) return ldx::conv3d_exact(a, stream);
  return conv_is_bf16(a) ? ldx::bf16_path::conv3d_entry(a, stream) : ldx::f16_path::conv3d_entry(a, stream);
}

extern "C" int64_t ldx_conv3d_stats_chunks(const ldx_conv3d_args* a) {
  if (conv_dtype_ok(a) != LDX_OK) return 0;
  return conv_is_bf16(a) ? ldx::bf16_path::conv3d_stats_chunks(a) : ldx::f16_path::conv3d_stats_chunks(a);
}

extern "C" int ldx_conv3d_stats(const ldx_conv3d_args* a, float* stats, void* stream) {
  if (int rc = conv_dtype_ok(a)) return rc;
  return conv_is_bf16(a) ? ldx::bf16_path::conv3d_stats(a, stats, stream)
                         : ldx::f16_path::conv3d_stats(a, stats, stream);
}

extern "C" int ldx_dense_ln(const ldx_conv3d_args* a, const float* gamma, const float* beta, float eps,
                            void* stream) {
  if (int rc = conv_dtype_ok(a)) return rc;
  return conv_is_bf16(a) ? ldx::bf16_path::dense_ln(a, gamma, beta, eps, stream)
                         : ldx::f16_path::dense_ln(a, gamma, beta, eps, stream);
}
#endif
