// Source-order half-precision conv3d and GroupNorm: the reference's "source" arithmetic,
// which reproduces Torch-CPU's reduction order bit for bit
// (src/lesiondiffusion_mlx/_source_half.py).
//
// conv3d (_source_half.py:19-104). Output (n, o, position) is the dot product over
// k = c * taps + (kd * KH + kh) * KW + kw of the im2col column with weight row o. A
// product of two fp16 values is exact in fp32, so fused or not it is the same number;
// the products go into four fp32 partials by k % 4 for k < K - K % 4 in increasing k,
// the last K % 4 products into partial 0, then ((p0 + p1) + p2) + p3 + float(bias),
// rounded once to fp16. The order fixes the result; the tiling does not. One workgroup
// computes 64 positions x 64 output channels; each thread owns 4 positions x 4 channels
// x 4 partials in registers. Per 32-k step the workgroup gathers its im2col tile and
// weight tile into LDS as fp32; a thread's inner step is two 16-byte LDS reads and 16
// FMAs. It runs on the VALU: the MFMA's internal summation order is not Torch's.
//
// GroupNorm (_source_half.py:120-300, host 387-544). Per (batch item, group) the
// SIZE = C/G * voxels values in NCDHW order: vectors of 8, chunks of 16 vectors, Welford
// moments per vector lane within a chunk (src_gn_partial_kernel, a thread per lane), the
// binary-counter cascade of each 128-chunk block evaluated as the merge tree it is
// (src_gn_cascade_kernel, a wave per block), then per group one thread carries the
// blocks, the leftover chunks, the scalar tail and the four lanes in the reference's
// order from LDS and the workgroup writes the per-channel affine (src_gn_final_kernel);
// finally y = fp16(scale * x + offset) with two fp32 roundings (src_gn_apply_kernel).
// rstd = fp32(1 / sqrt(var + eps)) taken in fp64, the value Torch stores and the
// reference's compensated reciprocal root (:244-252) reproduces.
//
// Tensors are addressed by (batch, channel, voxel) strides in elements, so NCDHW
// (voxel stride 1) and channels-last NDHWC (channel stride 1) both work; the summation
// order is that of the logical NCDHW tensor either way.

#include "common.h"

#include <cmath>

// Every rounding point is explicit: no multiply and add may be contracted behind the
// code's back.
#pragma clang fp contract(off)

namespace ldx {

// ------------------------------------------------------------------------- conv3d

constexpr int SC_THREADS = 256;
constexpr int SC_P = 64;   // positions per workgroup
constexpr int SC_O = 64;   // output channels per workgroup
constexpr int SC_K = 32;   // k per LDS step
constexpr int SC_TP = 4;   // positions per thread
constexpr int SC_TO = 4;   // channels per thread

struct SrcConvParams {
  int B, C, D, H, W, O, KD, KH, KW, S, P, OD, OH, OW;
  int K, complete, taps, khw;
  int npos;                       // B * OD * OH * OW
  UDiv dv_taps, dv_khw, dv_kw, dv_ow, dv_oh, dv_od;
  const f16* x;
  int64_t xsN, xsC, xsV;
  const f16* w;                   // (O, K)
  const f16* bias;                // (O,) or null
  f16* y;
  int64_t ysN, ysC, ysV;
};

// Output position p -> batch item and voxel coordinates.
__device__ __forceinline__ void src_pos(const SrcConvParams& p, int pos, int& n, int& od, int& oh, int& ow) {
  const int q1 = udiv(pos, p.dv_ow);
  ow = pos - q1 * p.OW;
  const int q2 = udiv(q1, p.dv_oh);
  oh = q1 - q2 * p.OH;
  n = udiv(q2, p.dv_od);
  od = q2 - n * p.OD;
}

// im2col column k -> (channel offset in elements, kd, kh, kw). Called with wave-uniform k
// in the main loop, so it runs on the scalar unit.
struct SrcTap {
  int64_t coff;
  int kd, kh, kw;
};
__device__ __forceinline__ SrcTap src_tap(const SrcConvParams& p, int k) {
  const int c = udiv(k, p.dv_taps);
  const int tap = k - c * p.taps;
  const int kd = udiv(tap, p.dv_khw);
  const int r = tap - kd * p.khw;
  const int kh = udiv(r, p.dv_kw);
  return SrcTap{(int64_t)c * p.xsC, kd, kh, r - kh * p.KW};
}

// Input value at tap `tp` of the output position whose window starts at (zb, yb, xb) of
// batch item n, as fp32; zero outside the volume (the reference's padding,
// _source_half.py:38-46).
__device__ __forceinline__ float src_x(const SrcConvParams& p, const SrcTap& tp, int n, int zb, int yb, int xb) {
  const int z = zb + tp.kd, yy = yb + tp.kh, xx = xb + tp.kw;
  if ((unsigned)z >= (unsigned)p.D || (unsigned)yy >= (unsigned)p.H || (unsigned)xx >= (unsigned)p.W) return 0.f;
  const int64_t v = ((int64_t)z * p.H + yy) * p.W + xx;
  return (float)p.x[(int64_t)n * p.xsN + tp.coff + v * p.xsV];
}

__global__ __launch_bounds__(SC_THREADS) void src_conv_kernel(SrcConvParams p) {
  touch_args(p);
  __shared__ float4 xs[SC_K][SC_P / 4];   // im2col tile, k-major: 16-byte reads of 4 positions
  __shared__ float4 ws[SC_K][SC_O / 4];   // weight tile, k-major: 16-byte reads of 4 channels
  float* xsf = reinterpret_cast<float*>(&xs[0][0]);
  float* wsf = reinterpret_cast<float*>(&ws[0][0]);
  const int t = threadIdx.x;
  const int p0 = blockIdx.x * SC_P;
  const int o0 = blockIdx.y * SC_O;

  // Loader roles. Input: position t % 64 of the tile, k rows t / 64 + 4 r (r < 8).
  // Weight: channel t % 64, the same k rows. Each k row is wave-uniform.
  const int lp = t & (SC_P - 1);
  const int lkx = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lo = t & (SC_O - 1);
  const int lkw = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lpos = p0 + lp;
  const bool lpos_ok = lpos < p.npos;
  int ln = 0, lzb = 0, lyb = 0, lxb = 0;
  if (lpos_ok) {
    int od, oh, ow;
    src_pos(p, lpos, ln, od, oh, ow);
    lzb = od * p.S - p.P;
    lyb = oh * p.S - p.P;
    lxb = ow * p.S - p.P;
  }
  const bool lo_ok = o0 + lo < p.O;
  const f16* wrow = p.w + (int64_t)(lo_ok ? o0 + lo : 0) * p.K;

  // Compute role: positions 4 * ty + i, channels 4 * tx + j of the tile.
  const int tx = t & 15;
  const int ty = t >> 4;
  float acc[4][SC_TP][SC_TO];   // [partial][position i][channel j]
#pragma unroll
  for (int q = 0; q < 4; q++)
#pragma unroll
    for (int i = 0; i < SC_TP; i++)
#pragma unroll
      for (int j = 0; j < SC_TO; j++) acc[q][i][j] = 0.f;

  for (int base = 0; base < p.complete; base += SC_K) {
    __syncthreads();   // the previous step's tiles are no longer read
#pragma unroll
    for (int r = 0; r < SC_K / 4; r++) {
      const int kk = lkx + 4 * r;
      const int k = base + kk;
      float xv = 0.f;
      if (k < p.complete && lpos_ok) xv = src_x(p, src_tap(p, k), ln, lzb, lyb, lxb);
      xsf[kk * SC_P + lp] = xv;   // past the last whole group of four: zero (adds nothing)
    }
#pragma unroll
    for (int r = 0; r < SC_K / 4; r++) {
      const int kk = lkw + 4 * r;
      const int k = base + kk;
      wsf[kk * SC_O + lo] = (k < p.complete && lo_ok) ? (float)wrow[k] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < SC_K; kk += 4) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 xa0 = xs[kk + q][ty];
        const float4 wv = ws[kk + q][tx];
        const float xa[SC_TP] = {xa0.x, xa0.y, xa0.z, xa0.w};
        const float wa[SC_TO] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int i = 0; i < SC_TP; i++)
#pragma unroll
          for (int j = 0; j < SC_TO; j++) acc[q][i][j] = __builtin_fmaf(xa[i], wa[j], acc[q][i][j]);
      }
    }
  }

  // The last K % 4 products go to partial 0, in k order (_source_half.py:76-95).
  int cn[SC_TP], czb[SC_TP], cyb[SC_TP], cxb[SC_TP];
  bool cok[SC_TP];
#pragma unroll
  for (int i = 0; i < SC_TP; i++) {
    const int pos = p0 + SC_TP * ty + i;
    cok[i] = pos < p.npos;
    int od = 0, oh = 0, ow = 0, n = 0;
    if (cok[i]) src_pos(p, pos, n, od, oh, ow);
    cn[i] = n;
    czb[i] = od * p.S - p.P;
    cyb[i] = oh * p.S - p.P;
    cxb[i] = ow * p.S - p.P;
  }
  for (int k = p.complete; k < p.K; k++) {
    const SrcTap tp = src_tap(p, k);
    float wa[SC_TO], xa[SC_TP];
#pragma unroll
    for (int j = 0; j < SC_TO; j++) {
      const int o = o0 + SC_TO * tx + j;
      wa[j] = o < p.O ? (float)p.w[(int64_t)o * p.K + k] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < SC_TP; i++) xa[i] = cok[i] ? src_x(p, tp, cn[i], czb[i], cyb[i], cxb[i]) : 0.f;
#pragma unroll
    for (int i = 0; i < SC_TP; i++)
#pragma unroll
      for (int j = 0; j < SC_TO; j++) acc[0][i][j] = __builtin_fmaf(xa[i], wa[j], acc[0][i][j]);
  }

#pragma unroll
  for (int j = 0; j < SC_TO; j++) {
    const int o = o0 + SC_TO * tx + j;
    if (o >= p.O) continue;
    const float b = p.bias ? (float)p.bias[o] : 0.f;
#pragma unroll
    for (int i = 0; i < SC_TP; i++) {
      if (!cok[i]) continue;
      float s = ((acc[0][i][j] + acc[1][i][j]) + acc[2][i][j]) + acc[3][i][j];
      if (p.bias) s = s + b;
      const int64_t v = (((int64_t)(czb[i] + p.P) / p.S) * p.OH + (cyb[i] + p.P) / p.S) * p.OW + (cxb[i] + p.P) / p.S;
      p.y[(int64_t)cn[i] * p.ysN + (int64_t)o * p.ysC + v * p.ysV] = (f16)s;
    }
  }
}

// ---------------------------------------------------------------------- GroupNorm

constexpr int GN_VEC = 8;            // halves per vector
constexpr int GN_CHUNK = 16;         // vectors per chunk
constexpr int GN_BLOCK_DEPTH = 7;    // 128-chunk blocks
constexpr int GN_BLOCK_CHUNKS = 1 << GN_BLOCK_DEPTH;
constexpr int GN_MAX_DEPTH = 40;

struct SrcMoments {
  unsigned count;
  float4 mean, m2;
};

__device__ __forceinline__ float4 f4(float v) { return make_float4(v, v, v, v); }

// b folded into a (_source_half.py:121-132).
__device__ __forceinline__ void gn_merge(SrcMoments& a, const SrcMoments& b) {
  const unsigned count = a.count + b.count;
  const float ratio = count == 0 ? 0.f : (float)b.count / (float)count;
  const float ac = (float)a.count;
  float* am = &a.mean.x;
  float* am2 = &a.m2.x;
  const float* bm = &b.mean.x;
  const float* bm2 = &b.m2.x;
#pragma unroll
  for (int l = 0; l < 4; l++) {
    const float delta = bm[l] - am[l];
    const float correction = ratio * delta;
    const float prior = delta * ac;
    am[l] = am[l] + correction;
    am2[l] = __builtin_fmaf(prior, correction, am2[l] + bm2[l]);
  }
  a.count = count;
}

__device__ __forceinline__ SrcMoments gn_zero() { return SrcMoments{0u, f4(0.f), f4(0.f)}; }

struct SrcGnParams {
  int B, C, G, cpg;
  int64_t S, size, vectors, chunks, blocks;
  const f16* x;
  int64_t xsN, xsC, xsV;
  const f16* gamma;
  const f16* beta;
  float eps;
  float* partials;                // [B * G * chunks][16]
  float* cascades;                // [B * G * blocks][8]
  float* affine;                  // [B][C][2]
  f16* y;
  int64_t ysN, ysC, ysV;
};

// Group element i of group (n, g) -> its address.
__device__ __forceinline__ float gn_value(const SrcGnParams& p, int n, int g, int64_t i) {
  const int64_t cl = i / p.S;
  const int64_t v = i - cl * p.S;
  return (float)p.x[(int64_t)n * p.xsN + ((int64_t)g * p.cpg + cl) * p.xsC + v * p.xsV];
}

// One thread per (group, chunk, vector lane): lane l of chunk k reads group elements
// (16 k + j) * 8 + l for j < count, the reference's per-lane Welford chain
// (_source_half.py:135-162); neighbouring lanes read neighbouring values.
__global__ __launch_bounds__(256) void src_gn_partial_kernel(SrcGnParams p) {
  touch_args(p);
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.B * p.G * p.chunks * GN_VEC) return;
  const int lane = (int)(idx & (GN_VEC - 1));
  const int64_t cg = idx >> 3;   // group * chunks + chunk
  const int64_t group = cg / p.chunks;
  const int64_t chunk = cg - group * p.chunks;
  const int n = (int)(group / p.G), g = (int)(group - (int64_t)n * p.G);
  const int64_t left = p.vectors - chunk * GN_CHUNK;
  const int count = left < GN_CHUNK ? (int)(left > 0 ? left : 0) : GN_CHUNK;
  const f16* gx = p.x + (int64_t)n * p.xsN + (int64_t)g * p.cpg * p.xsC;
  const int64_t i0 = (chunk * GN_CHUNK) * GN_VEC + lane;
  float xv[GN_CHUNK];
  if (p.xsV == 1 && p.xsC == p.S) {   // the group's values are contiguous (NCDHW)
#pragma unroll
    for (int j = 0; j < GN_CHUNK; j++) xv[j] = j < count ? (float)gx[i0 + j * GN_VEC] : 0.f;
  } else {
    int64_t cl = i0 / p.S;
    int64_t v = i0 - cl * p.S;
#pragma unroll
    for (int j = 0; j < GN_CHUNK; j++) {
      xv[j] = j < count ? (float)gx[cl * p.xsC + v * p.xsV] : 0.f;
      v += GN_VEC;
      while (v >= p.S) {
        v -= p.S;
        ++cl;
      }
    }
  }
  float mean = 0.f, m2 = 0.f;
#pragma unroll
  for (int j = 0; j < GN_CHUNK; j++) {
    if (j < count) {
      const float ratio = 1.0f / (float)(j + 1);
      const float delta = xv[j] - mean;
      mean = __builtin_fmaf(delta, ratio, mean);
      m2 = __builtin_fmaf(delta, xv[j] - mean, m2);
    }
  }
  // [mean lanes 0-3, m2 lanes 0-3, mean lanes 4-7, m2 lanes 4-7] per chunk
  const int mi = lane < 4 ? lane : lane + 4;
  p.partials[cg * 16 + mi] = mean;
  p.partials[cg * 16 + mi + 4] = m2;
}

__device__ __forceinline__ unsigned gn_chunk_count(const SrcGnParams& p, int64_t chunk) {
  const int64_t left = p.vectors - chunk * GN_CHUNK;
  return (unsigned)(left < GN_CHUNK ? (left > 0 ? left : 0) : GN_CHUNK);
}

// Fold both lane halves of a chunk's partial moments into s0.
__device__ __forceinline__ void gn_take_chunk(const float4* part, unsigned count, SrcMoments& s0) {
  gn_merge(s0, SrcMoments{count, part[0], part[1]});
  gn_merge(s0, SrcMoments{count, part[2], part[3]});
}

// One wave per (group, 128-chunk block). The reference's binary-counter cascade over the
// block (_source_half.py:164-199) merges, at every level, a node into an empty slot and then
// its right neighbour into it: leaf t = chunks 2t and 2t + 1 folded in order into an empty
// set, node(L, i) = merge(merge(empty, node(L-1, 2i)), node(L-1, 2i+1)). The same merges,
// done level by level across the wave, give the reference's level-6 result bit for bit.
__global__ __launch_bounds__(64) void src_gn_cascade_kernel(SrcGnParams p) {
  touch_args(p);
  __shared__ SrcMoments nodes[64];
  const int t = threadIdx.x;
  const int64_t blk = blockIdx.x;   // group * blocks + block
  const int64_t group = blk / p.blocks;
  const int64_t first = (blk - group * p.blocks) * GN_BLOCK_CHUNKS;
  SrcMoments leaf = gn_zero();
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int64_t chunk = first + 2 * t + c;
    gn_take_chunk(reinterpret_cast<const float4*>(p.partials + (group * p.chunks + chunk) * 16),
                  gn_chunk_count(p, chunk), leaf);
  }
  nodes[t] = leaf;
  __syncthreads();
#pragma unroll
  for (int width = 32; width >= 1; width >>= 1) {
    SrcMoments m = gn_zero();
    if (t < width) {
      gn_merge(m, nodes[2 * t]);
      gn_merge(m, nodes[2 * t + 1]);
    }
    __syncthreads();
    if (t < width) nodes[t] = m;
    __syncthreads();
  }
  if (t == 0) {
    float4* out = reinterpret_cast<float4*>(p.cascades + blk * 8);
    out[0] = nodes[0].mean;
    out[1] = nodes[0].m2;
  }
}

constexpr int GN_STAGE = 512;   // block cascades or chunk partials staged in LDS per round

// One workgroup per (batch item, group): the group-wide cascade over the block results and
// the leftover chunks, the scalar tail and the four lanes, in the reference's order
// (_source_half.py:201-260), by one thread from LDS (the staging is cooperative); then the
// channel affines (:263-278).
__global__ __launch_bounds__(256) void src_gn_final_kernel(SrcGnParams p, int depth) {
  touch_args(p);
  __shared__ float4 stage[GN_STAGE * 4];
  __shared__ SrcMoments stack[GN_MAX_DEPTH];   // the cascade's levels (thread 0's; in LDS, not scratch)
  __shared__ float red[2];
  const int t = threadIdx.x;
  const int64_t group = blockIdx.x;
  const int n = (int)(group / p.G), g = (int)(group - (int64_t)n * p.G);
  if (t == 0)
    for (int l = 0; l < depth; l++) stack[l] = gn_zero();
  // block results: two float4 each
  for (int64_t b0 = 0; b0 < p.blocks; b0 += GN_STAGE) {
    const int nb = (int)(p.blocks - b0 < GN_STAGE ? p.blocks - b0 : GN_STAGE);
    __syncthreads();
    const float4* src = reinterpret_cast<const float4*>(p.cascades + (group * p.blocks + b0) * 8);
    for (int i = t; i < 2 * nb; i += 256) stage[i] = src[i];
    __syncthreads();
    if (t == 0) {
      for (int i = 0; i < nb; i++) {
        const int64_t b = b0 + i;
        const int64_t left = p.vectors - b * GN_BLOCK_CHUNKS * GN_CHUNK;
        const unsigned count =
            2u * (unsigned)(left < GN_BLOCK_CHUNKS * GN_CHUNK ? left : (int64_t)GN_BLOCK_CHUNKS * GN_CHUNK);
        gn_merge(stack[GN_BLOCK_DEPTH], SrcMoments{count, stage[2 * i], stage[2 * i + 1]});
        uint64_t mask = (uint64_t)b + 1;
        for (int l = GN_BLOCK_DEPTH + 1; l < depth && (mask & 1) == 0; l++) {
          gn_merge(stack[l], stack[l - 1]);
          stack[l - 1] = gn_zero();
          mask >>= 1;
        }
      }
    }
  }
  // leftover chunks (fewer than 128 when there are blocks): four float4 each
  for (int64_t c0 = p.blocks * GN_BLOCK_CHUNKS; c0 < p.chunks; c0 += GN_STAGE) {
    const int nc = (int)(p.chunks - c0 < GN_STAGE ? p.chunks - c0 : GN_STAGE);
    __syncthreads();
    const float4* src = reinterpret_cast<const float4*>(p.partials + (group * p.chunks + c0) * 16);
    for (int i = t; i < 4 * nc; i += 256) stage[i] = src[i];
    __syncthreads();
    if (t == 0) {
      for (int i = 0; i < nc; i++) {
        const int64_t ch = c0 + i;
        gn_take_chunk(&stage[4 * i], gn_chunk_count(p, ch), stack[0]);
        uint64_t mask = (uint64_t)ch + 1;
        for (int l = 1; l < depth && (mask & 1) == 0; l++) {
          gn_merge(stack[l], stack[l - 1]);
          stack[l - 1] = gn_zero();
          mask >>= 1;
        }
      }
    }
  }
  if (t == 0) {
    for (int l = 1; l < depth; l++) gn_merge(stack[0], stack[l]);
    // The scalar tail past the last whole vector, then the four lanes (:240-260).
    unsigned count = 0;
    float mean = 0.f, m2 = 0.f;
    for (int64_t i = p.vectors * GN_VEC; i < p.size; i++) {
      const float xv = gn_value(p, n, g, i);
      const float delta = xv - mean;
      ++count;
      mean = mean + delta / (float)count;
      m2 = __builtin_fmaf(delta, xv - mean, m2);
    }
    const unsigned added = (unsigned)(p.vectors * 2);
    const float* lm = &stack[0].mean.x;
    const float* lm2 = &stack[0].m2.x;
    for (int l = 0; l < 4; l++) {
      const unsigned nn = count + added;
      const float ratio = nn == 0 ? 0.f : (float)added / (float)nn;
      const float delta = lm[l] - mean;
      mean = __builtin_fmaf(ratio, delta, mean);
      m2 = m2 + __builtin_fmaf((delta * delta) * ratio, (float)count, lm2[l]);
      count = nn;
    }
    const float var = fmaxf(m2 / (float)p.size, 0.f);
    red[0] = mean;
    red[1] = (float)(1.0 / sqrt((double)var + (double)p.eps));
  }
  __syncthreads();
  const float mean = red[0], rstd = red[1];
  for (int c = t; c < p.cpg; c += 256) {
    const int ch = g * p.cpg + c;
    const float scale = rstd * (float)p.gamma[ch];
    const float offset = __builtin_fmaf(-scale, mean, (float)p.beta[ch]);
    p.affine[((int64_t)n * p.C + ch) * 2] = scale;
    p.affine[((int64_t)n * p.C + ch) * 2 + 1] = offset;
  }
}

// y = fp16(scale * x + offset), two fp32 roundings (_source_half.py:253-254, 292-299). Grid:
// (voxel blocks, channel, batch item); a thread takes 8 consecutive voxels of one channel.
__device__ __forceinline__ f16 gn_apply1(float scale, float offset, f16 x) {
  const float prod = scale * (float)x;
  return (f16)(prod + offset);
}

__global__ __launch_bounds__(256) void src_gn_apply_kernel(SrcGnParams p, int vec16) {
  touch_args(p);
  const int c = blockIdx.y, n = blockIdx.z;
  const int64_t v0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (v0 >= p.S) return;
  const float scale = p.affine[((int64_t)n * p.C + c) * 2];
  const float offset = p.affine[((int64_t)n * p.C + c) * 2 + 1];
  const f16* xp = p.x + (int64_t)n * p.xsN + (int64_t)c * p.xsC;
  f16* yp = p.y + (int64_t)n * p.ysN + (int64_t)c * p.ysC;
  if (vec16 && v0 + 8 <= p.S) {   // unit voxel strides, 16-byte aligned rows
    const f16x8 xv = *reinterpret_cast<const f16x8*>(xp + v0);
    f16x8 yv;
#pragma unroll
    for (int e = 0; e < 8; e++) yv[e] = gn_apply1(scale, offset, xv[e]);
    *reinterpret_cast<f16x8*>(yp + v0) = yv;
    return;
  }
  const int64_t v1 = v0 + 8 < p.S ? v0 + 8 : p.S;
  for (int64_t v = v0; v < v1; v++) yp[v * p.ysV] = gn_apply1(scale, offset, xp[v * p.xsV]);
}

// Workspace layout: partials, then block cascades (each 256-byte aligned).
static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

static void gn_geometry(int64_t voxels, int32_t channels, int32_t groups, int64_t& size, int64_t& vectors,
                        int64_t& chunks, int64_t& blocks) {
  size = (int64_t)(channels / groups) * voxels;
  vectors = size / GN_VEC;
  chunks = (vectors + GN_CHUNK - 1) / GN_CHUNK;   // max(1, ...) (_source_half.py:484)
  if (chunks < 1) chunks = 1;
  blocks = chunks > GN_BLOCK_CHUNKS ? chunks / GN_BLOCK_CHUNKS : 0;
}

}  // namespace ldx

using namespace ldx;

extern "C" int ldx_conv3d_source_half(const ldx_conv3d_source_args* a, void* stream) {
  if (!a) return fail("conv3d_source_half: null arguments");
  if (!a->x || !a->weight || !a->y) return fail("conv3d_source_half: null tensor pointer");
  if (a->batch < 1 || a->in_c < 1 || a->out_c < 1 || a->in_d < 1 || a->in_h < 1 || a->in_w < 1)
    return fail("conv3d_source_half: empty tensor (batch %d, channels %d -> %d, grid %dx%dx%d)", a->batch, a->in_c,
                a->out_c, a->in_d, a->in_h, a->in_w);
  if (a->kd < 1 || a->kh < 1 || a->kw < 1 || a->stride < 1 || a->padding < 0)
    return fail("conv3d_source_half: kernel %dx%dx%d, stride %d, padding %d", a->kd, a->kh, a->kw, a->stride,
                a->padding);
  SrcConvParams p{};
  p.B = a->batch;
  p.C = a->in_c;
  p.D = a->in_d;
  p.H = a->in_h;
  p.W = a->in_w;
  p.O = a->out_c;
  p.KD = a->kd;
  p.KH = a->kh;
  p.KW = a->kw;
  p.S = a->stride;
  p.P = a->padding;
  p.OD = (p.D + 2 * p.P - p.KD) / p.S + 1;
  p.OH = (p.H + 2 * p.P - p.KH) / p.S + 1;
  p.OW = (p.W + 2 * p.P - p.KW) / p.S + 1;
  if (p.D + 2 * p.P < p.KD || p.H + 2 * p.P < p.KH || p.W + 2 * p.P < p.KW)
    return fail("conv3d_source_half: conv3d kernel exceeds the padded input");
  const int64_t taps = (int64_t)p.KD * p.KH * p.KW;
  const int64_t K = taps * p.C;
  const int64_t npos = (int64_t)p.B * p.OD * p.OH * p.OW;
  if (K >= ((int64_t)1 << 30) || npos >= ((int64_t)1 << 30) || (int64_t)p.O * K >= ((int64_t)1 << 40))
    return fail("conv3d_source_half: too large (%lld reduction terms, %lld output positions)", (long long)K,
                (long long)npos);
  if ((int64_t)p.D * p.H * p.W >= ((int64_t)1 << 31)) return fail("conv3d_source_half: input grid too large");
  p.taps = (int)taps;
  p.khw = p.KH * p.KW;
  p.K = (int)K;
  p.complete = p.K - p.K % 4;
  p.npos = (int)npos;
  p.dv_taps = make_udiv((unsigned)p.taps);
  p.dv_khw = make_udiv((unsigned)p.khw);
  p.dv_kw = make_udiv((unsigned)p.KW);
  p.dv_ow = make_udiv((unsigned)p.OW);
  p.dv_oh = make_udiv((unsigned)p.OH);
  p.dv_od = make_udiv((unsigned)p.OD);
  p.x = (const f16*)a->x;
  p.xsN = a->x_batch_stride;
  p.xsC = a->x_channel_stride;
  p.xsV = a->x_voxel_stride;
  p.w = (const f16*)a->weight;
  p.bias = (const f16*)a->bias;
  p.y = (f16*)a->y;
  p.ysN = a->y_batch_stride;
  p.ysC = a->y_channel_stride;
  p.ysV = a->y_voxel_stride;
  const dim3 grid((unsigned)((npos + SC_P - 1) / SC_P), (unsigned)((p.O + SC_O - 1) / SC_O));
  if (grid.y > 65535) return fail("conv3d_source_half: %d output channels is too many", p.O);
  hipLaunchKernelGGL(src_conv_kernel, grid, dim3(SC_THREADS), 0, as_stream(stream), p);
  return check_launch("conv3d_source_half");
}

extern "C" size_t ldx_group_norm_source_workspace_bytes(int32_t batch, int32_t channels, int64_t voxels,
                                                        int32_t groups) {
  if (batch < 1 || channels < 1 || voxels < 1 || groups < 1 || channels % groups) return 0;
  int64_t size, vectors, chunks, blocks;
  gn_geometry(voxels, channels, groups, size, vectors, chunks, blocks);
  const int64_t bg = (int64_t)batch * groups;
  return al256((size_t)(bg * chunks * 16) * sizeof(float)) + al256((size_t)(bg * blocks * 8) * sizeof(float));
}

extern "C" int ldx_group_norm_source_half(const void* x, int64_t x_batch_stride, int64_t x_channel_stride,
                                          int64_t x_voxel_stride, int32_t batch, int32_t channels, int64_t voxels,
                                          int32_t groups, const void* weight, const void* bias, float eps,
                                          float* affine, void* y, int64_t y_batch_stride, int64_t y_channel_stride,
                                          int64_t y_voxel_stride, void* workspace, size_t workspace_bytes,
                                          void* stream) {
  if (!x || !weight || !bias || !affine) return fail("group_norm_source_half: null pointer");
  if (batch < 1 || channels < 1 || voxels < 1 || groups < 1)
    return fail("group_norm_source_half: empty tensor (batch %d, channels %d, %lld voxels, %d groups)", batch,
                channels, (long long)voxels, groups);
  if (channels % groups)
    return fail("group_norm channels %d must be divisible by num_groups %d", channels, groups);
  if (batch > 65535 || channels > 65535)
    return fail("group_norm_source_half: batch %d or channels %d above 65535", batch, channels);
  if (!(eps >= 0.f)) return fail("group_norm_source_half: eps must be >= 0");
  SrcGnParams p{};
  p.B = batch;
  p.C = channels;
  p.G = groups;
  p.cpg = channels / groups;
  p.S = voxels;
  gn_geometry(voxels, channels, groups, p.size, p.vectors, p.chunks, p.blocks);
  if (p.vectors >= ((int64_t)1 << 31))   // moment counts reach 2 * vectors in 32 bits
    return fail("group_norm_source_half: groups of 2^34 values or more");
  const size_t need = ldx_group_norm_source_workspace_bytes(batch, channels, voxels, groups);
  if (!workspace || workspace_bytes < need)
    return fail("group_norm_source_half: needs %zu bytes of workspace (ldx_group_norm_source_workspace_bytes)",
                need);
  const int64_t bg = (int64_t)batch * groups;
  int depth = 1;
  while (depth < GN_MAX_DEPTH && ((int64_t)1 << depth) < p.chunks) depth++;   // max(1, bit_length(chunks - 1))
  p.x = (const f16*)x;
  p.xsN = x_batch_stride;
  p.xsC = x_channel_stride;
  p.xsV = x_voxel_stride;
  p.gamma = (const f16*)weight;
  p.beta = (const f16*)bias;
  p.eps = eps;
  p.partials = (float*)workspace;
  p.cascades = (float*)((char*)workspace + al256((size_t)(bg * p.chunks * 16) * sizeof(float)));
  p.affine = affine;
  p.y = (f16*)y;
  p.ysN = y_batch_stride;
  p.ysC = y_channel_stride;
  p.ysV = y_voxel_stride;
  hipStream_t st = as_stream(stream);
  const int64_t np = bg * p.chunks * GN_VEC;
  hipLaunchKernelGGL(src_gn_partial_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, st, p);
  if (p.blocks)
    hipLaunchKernelGGL(src_gn_cascade_kernel, dim3((unsigned)(bg * p.blocks)), dim3(64), 0, st, p);
  hipLaunchKernelGGL(src_gn_final_kernel, dim3((unsigned)bg), dim3(256), 0, st, p, depth);
  if (y) {
    const int vec16 = x_voxel_stride == 1 && y_voxel_stride == 1 && x_channel_stride % 8 == 0 &&
                      y_channel_stride % 8 == 0 && x_batch_stride % 8 == 0 && y_batch_stride % 8 == 0 &&
                      ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0;
    const dim3 grid((unsigned)((voxels + 2047) / 2048), (unsigned)channels, (unsigned)batch);
    hipLaunchKernelGGL(src_gn_apply_kernel, grid, dim3(256), 0, st, p, vec16);
  }
  return check_launch("group_norm_source_half");
}
