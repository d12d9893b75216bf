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
// moments per vector lane within a chunk (src_gn_partial_kernel), a binary-counter
// cascade of each 128-chunk block (src_gn_cascade_kernel), then one thread per group
// carries the blocks, the leftover chunks, the scalar tail and the four lanes in the
// reference's order and writes the per-channel affine (src_gn_final_kernel); finally
// y = fp16(scale * x + offset) with two fp32 roundings (src_gn_apply_kernel).
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

// Input value of im2col column k at output position (n, zb + kd, yb + kh, xb + kw) as
// fp32; zero outside the volume (the reference's padding, _source_half.py:38-46).
__device__ __forceinline__ float src_x(const SrcConvParams& p, int k, int n, int zb, int yb, int xb) {
  const int c = udiv(k, p.dv_taps);
  const int tap = k - c * p.taps;
  const int kd = udiv(tap, p.dv_khw);
  const int r = tap - kd * p.khw;
  const int kh = udiv(r, p.dv_kw);
  const int kw = r - kh * p.KW;
  const int z = zb + kd, yy = yb + kh, xx = xb + kw;
  if ((unsigned)z >= (unsigned)p.D || (unsigned)yy >= (unsigned)p.H || (unsigned)xx >= (unsigned)p.W) return 0.f;
  const int64_t v = ((int64_t)z * p.H + yy) * p.W + xx;
  return (float)p.x[(int64_t)n * p.xsN + (int64_t)c * p.xsC + v * p.xsV];
}

__global__ __launch_bounds__(SC_THREADS) void src_conv_kernel(SrcConvParams p) {
  __shared__ float4 xs[SC_K][SC_P / 4];   // im2col tile, k-major: 16-byte reads of 4 positions
  __shared__ float4 ws[SC_K][SC_O / 4];   // weight tile, k-major: 16-byte reads of 4 channels
  float* xsf = reinterpret_cast<float*>(&xs[0][0]);
  float* wsf = reinterpret_cast<float*>(&ws[0][0]);
  const int t = threadIdx.x;
  const int p0 = blockIdx.x * SC_P;
  const int o0 = blockIdx.y * SC_O;

  // Loader role: position / channel t % 64 of the tile, k rows t / 64 + 4 r (r < 8).
  const int lp = t & 63;
  const int lk = t >> 6;
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
  const int lo = o0 + lp;
  const bool lo_ok = lo < p.O;
  const f16* wrow = p.w + (int64_t)(lo_ok ? lo : 0) * p.K;

  // Compute role: positions 4 * ty + i, channels 4 * tx + j of the tile.
  const int tx = t & 15;
  const int ty = t >> 4;
  float acc[4][4][4];   // [partial][position i][channel j]
#pragma unroll
  for (int q = 0; q < 4; q++)
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[q][i][j] = 0.f;

  for (int base = 0; base < p.complete; base += SC_K) {
    __syncthreads();   // the previous step's tiles are no longer read
#pragma unroll
    for (int r = 0; r < SC_K / 4; r++) {
      const int kk = lk + 4 * r;
      const int k = base + kk;
      float xv = 0.f, wv = 0.f;
      if (k < p.complete) {   // past the last whole group of four: zero (adds nothing)
        if (lpos_ok) xv = src_x(p, k, ln, lzb, lyb, lxb);
        if (lo_ok) wv = (float)wrow[k];
      }
      xsf[kk * SC_P + lp] = xv;
      wsf[kk * SC_O + lp] = wv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < SC_K; kk += 4) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 xv = xs[kk + q][ty];
        const float4 wv = ws[kk + q][tx];
        const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
        const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) acc[q][i][j] = __builtin_fmaf(xa[i], wa[j], acc[q][i][j]);
      }
    }
  }

  // The last K % 4 products go to partial 0, in k order (_source_half.py:76-95).
  int cn[4], czb[4], cyb[4], cxb[4];
  int64_t cv[4];
  bool cok[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int pos = p0 + 4 * ty + i;
    cok[i] = pos < p.npos;
    int od = 0, oh = 0, ow = 0, n = 0;
    if (cok[i]) src_pos(p, pos, n, od, oh, ow);
    cn[i] = n;
    czb[i] = od * p.S - p.P;
    cyb[i] = oh * p.S - p.P;
    cxb[i] = ow * p.S - p.P;
    cv[i] = ((int64_t)od * p.OH + oh) * p.OW + ow;
  }
  for (int k = p.complete; k < p.K; k++) {
    float wa[4], xa[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int o = o0 + 4 * tx + j;
      wa[j] = o < p.O ? (float)p.w[(int64_t)o * p.K + k] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) xa[i] = cok[i] ? src_x(p, k, cn[i], czb[i], cyb[i], cxb[i]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[0][i][j] = __builtin_fmaf(xa[i], wa[j], acc[0][i][j]);
  }

#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int o = o0 + 4 * tx + j;
    if (o >= p.O) continue;
    const float b = p.bias ? (float)p.bias[o] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (!cok[i]) continue;
      float s = ((acc[0][i][j] + acc[1][i][j]) + acc[2][i][j]) + acc[3][i][j];
      if (p.bias) s = s + b;
      p.y[(int64_t)cn[i] * p.ysN + (int64_t)o * p.ysC + cv[i] * p.ysV] = (f16)s;
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

__global__ __launch_bounds__(256) void src_gn_partial_kernel(SrcGnParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.B * p.G * p.chunks) return;
  const int64_t group = idx / p.chunks;
  const int64_t chunk = idx - group * p.chunks;
  const int n = (int)(group / p.G), g = (int)(group - (int64_t)n * p.G);
  const int64_t left = p.vectors - chunk * GN_CHUNK;
  const int count = left < GN_CHUNK ? (int)(left > 0 ? left : 0) : GN_CHUNK;
  float mean[GN_VEC], m2[GN_VEC];
#pragma unroll
  for (int l = 0; l < GN_VEC; l++) mean[l] = m2[l] = 0.f;
  // Walk (channel, voxel) of the chunk's first element forward one element at a time.
  int64_t i0 = chunk * GN_CHUNK * GN_VEC;
  int64_t cl = i0 / p.S;
  int64_t v = i0 - cl * p.S;
  const f16* gx = p.x + (int64_t)n * p.xsN + (int64_t)g * p.cpg * p.xsC;
  for (int j = 0; j < count; j++) {
    const float ratio = 1.0f / (float)(j + 1);
#pragma unroll
    for (int l = 0; l < GN_VEC; l++) {
      const float xv = (float)gx[cl * p.xsC + v * p.xsV];
      if (++v == p.S) {
        v = 0;
        ++cl;
      }
      const float delta = xv - mean[l];
      mean[l] = __builtin_fmaf(delta, ratio, mean[l]);
      m2[l] = __builtin_fmaf(delta, xv - mean[l], m2[l]);
    }
  }
  float4* out = reinterpret_cast<float4*>(p.partials + idx * 16);
  out[0] = make_float4(mean[0], mean[1], mean[2], mean[3]);
  out[1] = make_float4(m2[0], m2[1], m2[2], m2[3]);
  out[2] = make_float4(mean[4], mean[5], mean[6], mean[7]);
  out[3] = make_float4(m2[4], m2[5], m2[6], m2[7]);
}

__device__ __forceinline__ unsigned gn_chunk_count(const SrcGnParams& p, int64_t chunk) {
  const int64_t left = p.vectors - chunk * GN_CHUNK;
  return (unsigned)(left < GN_CHUNK ? (left > 0 ? left : 0) : GN_CHUNK);
}

// Fold chunk `chunk` of `group` (both lane halves) into stack[0].
__device__ __forceinline__ void gn_take_chunk(const SrcGnParams& p, int64_t group, int64_t chunk, SrcMoments& s0) {
  const float4* part = reinterpret_cast<const float4*>(p.partials + (group * p.chunks + chunk) * 16);
  const unsigned c = gn_chunk_count(p, chunk);
  gn_merge(s0, SrcMoments{c, part[0], part[1]});
  gn_merge(s0, SrcMoments{c, part[2], part[3]});
}

__global__ __launch_bounds__(256) void src_gn_cascade_kernel(SrcGnParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.B * p.G * p.blocks) return;
  const int64_t group = idx / p.blocks;
  const int64_t first = (idx - group * p.blocks) * GN_BLOCK_CHUNKS;
  SrcMoments stack[GN_BLOCK_DEPTH];
#pragma unroll
  for (int l = 0; l < GN_BLOCK_DEPTH; l++) stack[l] = gn_zero();
  for (int c = 0; c < GN_BLOCK_CHUNKS; c++) {
    gn_take_chunk(p, group, first + c, stack[0]);
    unsigned mask = (unsigned)c + 1;
#pragma unroll
    for (int l = 1; l < GN_BLOCK_DEPTH; l++) {
      if (mask & 1) break;
      gn_merge(stack[l], stack[l - 1]);
      stack[l - 1] = gn_zero();
      mask >>= 1;
    }
  }
  float4* out = reinterpret_cast<float4*>(p.cascades + idx * 8);
  out[0] = stack[GN_BLOCK_DEPTH - 1].mean;
  out[1] = stack[GN_BLOCK_DEPTH - 1].m2;
}

// One thread per (batch item, group): the group-wide cascade, tail and lane fold, then the
// channel affines (_source_half.py:201-278).
__global__ __launch_bounds__(64) void src_gn_final_kernel(SrcGnParams p, int depth) {
  const int64_t group = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (group >= (int64_t)p.B * p.G) return;
  const int n = (int)(group / p.G), g = (int)(group - (int64_t)n * p.G);
  SrcMoments stack[GN_MAX_DEPTH];
  for (int l = 0; l < depth; l++) stack[l] = gn_zero();
  for (int64_t b = 0; b < p.blocks; b++) {
    const int64_t left = p.vectors - b * GN_BLOCK_CHUNKS * GN_CHUNK;
    const unsigned count =
        2u * (unsigned)(left < GN_BLOCK_CHUNKS * GN_CHUNK ? left : (int64_t)GN_BLOCK_CHUNKS * GN_CHUNK);
    const float4* c = reinterpret_cast<const float4*>(p.cascades + (group * p.blocks + b) * 8);
    gn_merge(stack[GN_BLOCK_DEPTH], SrcMoments{count, c[0], c[1]});
    uint64_t mask = (uint64_t)b + 1;
    for (int l = GN_BLOCK_DEPTH + 1; l < depth && (mask & 1) == 0; l++) {
      gn_merge(stack[l], stack[l - 1]);
      stack[l - 1] = gn_zero();
      mask >>= 1;
    }
  }
  for (int64_t ch = p.blocks * GN_BLOCK_CHUNKS; ch < p.chunks; ch++) {
    gn_take_chunk(p, group, ch, stack[0]);
    uint64_t mask = (uint64_t)ch + 1;
    for (int l = 1; l < depth && (mask & 1) == 0; l++) {
      gn_merge(stack[l], stack[l - 1]);
      stack[l - 1] = gn_zero();
      mask >>= 1;
    }
  }
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
  const float rstd = (float)(1.0 / sqrt((double)var + (double)p.eps));
  for (int c = 0; c < p.cpg; c++) {
    const int ch = g * p.cpg + c;
    const float scale = rstd * (float)p.gamma[ch];
    const float offset = __builtin_fmaf(-scale, mean, (float)p.beta[ch]);
    p.affine[((int64_t)n * p.C + ch) * 2] = scale;
    p.affine[((int64_t)n * p.C + ch) * 2 + 1] = offset;
  }
}

// y = fp16(scale * x + offset), two fp32 roundings (_source_half.py:253-254, 292-299).
// Elements are enumerated channel-fastest when the channel stride is 1 (NDHWC), else
// voxel-fastest (NCDHW), so that neighbouring lanes touch neighbouring memory.
__global__ __launch_bounds__(256) void src_gn_apply_kernel(SrcGnParams p, int channel_fastest) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.C * p.S;
  if (e >= total) return;
  int64_t n, c, v;
  if (channel_fastest) {
    c = e % p.C;
    const int64_t q = e / p.C;
    v = q % p.S;
    n = q / p.S;
  } else {
    v = e % p.S;
    const int64_t q = e / p.S;
    c = q % p.C;
    n = q / p.C;
  }
  const float scale = p.affine[(n * p.C + c) * 2];
  const float offset = p.affine[(n * p.C + c) * 2 + 1];
  const float xv = (float)p.x[n * p.xsN + c * p.xsC + v * p.xsV];
  const float prod = scale * xv;
  p.y[n * p.ysN + c * p.ysC + v * p.ysV] = (f16)(prod + offset);
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
  const int64_t np = bg * p.chunks;
  hipLaunchKernelGGL(src_gn_partial_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, st, p);
  if (p.blocks) {
    const int64_t nc = bg * p.blocks;
    hipLaunchKernelGGL(src_gn_cascade_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, p);
  }
  hipLaunchKernelGGL(src_gn_final_kernel, dim3((unsigned)((bg + 63) / 64)), dim3(64), 0, st, p, depth);
  if (y) {
    const int64_t total = (int64_t)batch * channels * voxels;
    const int channel_fastest = x_channel_stride == 1 && y_channel_stride == 1;
    hipLaunchKernelGGL(src_gn_apply_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p,
                       channel_fastest);
  }
  return check_launch("group_norm_source_half");
}
