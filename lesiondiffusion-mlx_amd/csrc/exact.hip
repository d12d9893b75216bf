// FP32 networks ("exact" mode): the reference keeps LMNet, and the conditioned VQ decode, in
// FP32 (src/lesiondiffusion_mlx/_nax_conv.py:26-34; medmlx.py:1362-1366). Here:
//
// * conv3d / dense layers in the split-FP16 form of _nax_conv.py:26-34, 210-237: each FP32
//   value v becomes hi = half(v) and lo = half((v - hi) * 2^11); hi x hi products go to one
//   FP32 sum, hi x lo + lo x hi to another, scaled back by 2^-11 (only lo x lo is dropped:
//   about 2^-22 relative). The products run on this library's fp16 conv kernels -- the
//   input as 2C fp16 channels [hi | lo], the weights stacked into 2O rows [[W_hi, 0],
//   [W_lo, W_hi]] (one block of zero products: four fp16 products per FP32 product
//   instead of three, for reuse of the tuned kernels), their FP32 sums left raw -- and
//   exact_combine_kernel finishes y = ((S_hh + S_x * 2^-11) + (bias + shift)) * scale +
//   residual in FP32. The input split applies the GroupNorm affine and SiLU in FP32 first
//   (_nax_conv.py:128-136) and, for a conv of a nearest-2x upsampling, the upsampling (the
//   conv then runs on the upsampled grid with the unfolded weights, so no folded weight is
//   re-split: the reference folds in FP32 before splitting, the same sums in another order).
// * GroupNorm statistics and LayerNorm of FP32 tensors, FP32 timestep features.
// * attention in FP32 for head widths 16 / 32 / 64: a flash kernel on the VALU (the
//   reference's FP32 SIMD kernel, _attention.py:52-145): one query per lane, 64-key K/V
//   tiles in LDS shared by the workgroup's four waves, scores and P V as FP32 fused
//   multiply-adds, online softmax with exp2 of log2(e)-scaled scores.

#include "common.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace ldx {

// ------------------------------------------------------------------ weights
// The stacked split weight in the fragment-major layout of ldx_pack_weight for 2O rows and
// 2C channels: row o < O holds [hi(W[o, c]) (c < C), 0]; row O + o holds [lo(W[o, c]),
// hi(W[o, c])].
__device__ __forceinline__ f16 split_hi(float v) { return (f16)v; }
__device__ __forceinline__ f16 split_lo(float v) { return (f16)((v - (float)(f16)v) * 2048.0f); }

__global__ void pack_weight_exact_kernel(const float* __restrict__ w, int O, int C, int taps, f16* __restrict__ out) {
  const int O2 = 2 * O, C2 = 2 * C;
  const int NOB = (O2 + 127) / 128 * 4, NKC = (C2 + 63) / 64 * 4;
  const int64_t n = (int64_t)NOB * taps * NKC * 512;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int e = (int)(i & 7), l = (int)((i >> 3) & 63);
    const int64_t frag = i >> 9;
    const int kc = (int)(frag % NKC), tap = (int)((frag / NKC) % taps);
    const int64_t ob = frag / ((int64_t)NKC * taps);
    const int o2 = (int)ob * 32 + (l & 31);
    const int c2 = kc * 16 + 8 * (l >> 5) + e;
    f16 v = (f16)0.f;
    if (o2 < O2 && c2 < C2) {
      const int o = o2 < O ? o2 : o2 - O, c = c2 < C ? c2 : c2 - C;
      const float wv = w[((int64_t)o * C + c) * taps + tap];
      if (o2 < O) v = c2 < C ? split_hi(wv) : (f16)0.f;
      else v = c2 < C ? split_lo(wv) : split_hi(wv);
    }
    out[i] = v;
  }
}

// ------------------------------------------------------------------ input split
// out (fp16, NDHWC of the row grid, 2C channels, pitch 2C): [hi | lo] of the prepared input
// prep(x) = silu(x * scale + offset) (as set), read from x0 (channels [0, C0)) and x1 (the
// rest); with up, grid voxel (d, h, w) reads source voxel (d / 2, h / 2, w / 2).
__global__ void split_exact_kernel(const float* __restrict__ x0, int64_t p0, int C0, const float* __restrict__ x1,
                                   int64_t p1, int C, int B, int D, int H, int W, int up, const float* __restrict__ affine,
                                   int silu, f16* __restrict__ out) {
  const int RD = up ? 2 * D : D, RH = up ? 2 * H : H, RW = up ? 2 * W : W;
  const int64_t n = (int64_t)B * RD * RH * RW * C;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % C);
    int64_t r = i / C;
    const int w = (int)(r % RW); r /= RW;
    const int h = (int)(r % RH); r /= RH;
    const int d = (int)(r % RD);
    const int b = (int)(r / RD);
    const int sd = up ? d >> 1 : d, sh = up ? h >> 1 : h, sw = up ? w >> 1 : w;
    const int64_t sv = (((int64_t)b * D + sd) * H + sh) * W + sw;
    float v = c < C0 ? x0[sv * p0 + c] : x1[sv * p1 + (c - C0)];
    if (affine) v = v * affine[((int64_t)b * C + c) * 2] + affine[((int64_t)b * C + c) * 2 + 1];
    if (silu) v = v / (1.0f + expf(-v));
    const int64_t ov = (((int64_t)b * RD + d) * RH + h) * RW + w;
    out[ov * 2 * C + c] = split_hi(v);
    out[ov * 2 * C + C + c] = split_lo(v);
  }
}

__device__ __forceinline__ float gelu_erf32(float v) { return v * (1.0f + erff(v * 0.70710678118654752f)) * 0.5f; }

// y[b, v, o] = act(((S[v, o] + S[v, O + o] * 2^-11) + (bias + shift)) * scale + res), FP32.
__global__ void exact_combine_kernel(const float* __restrict__ part, int64_t nvox_b, int B, int O,
                                     const float* __restrict__ bias, int bias_batched, const float* __restrict__ shift,
                                     int64_t shiftp, float scale, const float* __restrict__ res, int64_t resp, int act,
                                     float* __restrict__ y, int64_t yp) {
  const int64_t n = (int64_t)B * nvox_b * O;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int o = (int)(i % O);
    const int64_t v = i / O;
    const int b = (int)(v / nvox_b);
    const float* s = part + v * 2 * O;
    const float sum = s[o] + s[O + o] * (1.0f / 2048.0f);
    float add = bias ? bias[(bias_batched ? (int64_t)b * O : 0) + o] : 0.f;
    if (shift) add += shift[(int64_t)b * shiftp + o];
    float t = (sum + add) * scale;
    if (res) t += res[v * resp + o];
    if (act == LDX_ACT_GELU) t = gelu_erf32(t);
    else if (act == LDX_ACT_SILU) t = t / (1.0f + expf(-t));
    y[v * yp + o] = t;
  }
}

// ------------------------------------------------------------------ GroupNorm / LayerNorm
// Per (group, batch item): Welford (count, mean, M2) per thread over its strided elements,
// merged in a fixed order (block_merge256), folded with gamma / beta into (scale, offset).
__device__ __forceinline__ Moments welford(Moments m, float x) {
  const float n = m.n + 1.f, d = x - m.mean, mean = m.mean + d / n;
  return {n, mean, m.m2 + d * (x - mean)};
}

__global__ __launch_bounds__(256) void gn_f32_kernel(const float* __restrict__ x0, int64_t p0, int C0,
                                                     const float* __restrict__ x1, int64_t p1, int C, int G,
                                                     int64_t voxels, const float* __restrict__ gamma,
                                                     const float* __restrict__ beta, float eps, float* __restrict__ affine) {
  __shared__ float red[12];
  const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int gs = C / G, c0 = g * gs;
  const int64_t items = voxels * gs;
  Moments m = {0.f, 0.f, 0.f};
  for (int64_t i = t; i < items; i += 256) {
    const int64_t v = i / gs;
    const int c = c0 + (int)(i - v * gs);
    const int64_t bv = (int64_t)b * voxels + v;
    m = welford(m, c < C0 ? x0[bv * p0 + c] : x1[bv * p1 + (c - C0)]);
  }
  const Moments tot = block_merge256(m, red);
  const float var = tot.n > 0.f ? tot.m2 / tot.n : 0.f;
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int c = c0 + t; c < c0 + gs; c += 256) {
    const float sc = gamma[c] * rstd;
    affine[((int64_t)b * C + c) * 2] = sc;
    affine[((int64_t)b * C + c) * 2 + 1] = beta[c] - sc * tot.mean;
  }
}

// One wave per row: mean, then the mean squared deviation, in FP32; the lanes' partial sums
// added in a fixed butterfly order.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ __launch_bounds__(256) void layer_norm_f32_kernel(const float* __restrict__ x, int64_t xp, int64_t rows,
                                                             int F, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float eps,
                                                             float* __restrict__ y, int64_t yp) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * xp;
  float s = 0.f;
  for (int c = lane; c < F; c += 64) s += xr[c];
  const float mean = wave_sum(s) / (float)F;
  float q = 0.f;
  for (int c = lane; c < F; c += 64) {
    const float d = xr[c] - mean;
    q += d * d;
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)F + eps);
  for (int c = lane; c < F; c += 64) y[row * yp + c] = (xr[c] - mean) * rstd * gamma[c] + beta[c];
}

__global__ void timestep_f32_kernel(const int32_t* __restrict__ t, int B, int channels, float* __restrict__ out) {
  const int half = channels / 2;
  const int64_t n = (int64_t)B * half;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int b = (int)(i / half), k = (int)(i % half);
    const float f = expf(-9.210340371976184f * (float)k / (float)half);   // ln(1e4) = 9.2103...
    const float ph = (float)t[b] * f;
    out[(int64_t)b * channels + k] = cosf(ph);
    out[(int64_t)b * channels + half + k] = sinf(ph);
  }
}

// ------------------------------------------------------------------ attention
// Workgroup: 4 waves x 64 queries of one (batch, head); 64-key tiles of K and V in LDS.
template <int D>
__global__ __launch_bounds__(256) void attention_f32_kernel(const float* __restrict__ q, int64_t qs0, int64_t qs1,
                                                            int64_t qs2, const float* __restrict__ k, int64_t ks0,
                                                            int64_t ks1, int64_t ks2, const float* __restrict__ v,
                                                            int64_t vs0, int64_t vs1, int64_t vs2, float* __restrict__ o,
                                                            int64_t os0, int64_t os1, int64_t os2, int H, int L, int LK,
                                                            float c) {
  constexpr int TK = 64;
  __shared__ float kt[TK][D];
  __shared__ float vt[TK][D];
  const int bh = blockIdx.y, b = bh / H, h = bh % H;
  const int qi = blockIdx.x * 256 + threadIdx.x;
  const bool live = qi < L;
  float qr[D], acc[D];
  const float* qp = q + (int64_t)b * qs0 + (int64_t)h * qs2 + (int64_t)(live ? qi : 0) * qs1;
#pragma unroll
  for (int d = 0; d < D; d++) { qr[d] = qp[d]; acc[d] = 0.f; }
  float m = -INFINITY, l = 0.f;
  const float* kb = k + (int64_t)b * ks0 + (int64_t)h * ks2;
  const float* vb = v + (int64_t)b * vs0 + (int64_t)h * vs2;
  for (int k0 = 0; k0 < LK; k0 += TK) {
    const int nk = min(TK, LK - k0);
    __syncthreads();
    for (int i = threadIdx.x; i < TK * D; i += 256) {
      const int r = i / D, d = i % D;
      kt[r][d] = r < nk ? kb[(int64_t)(k0 + r) * ks1 + d] : 0.f;
      vt[r][d] = r < nk ? vb[(int64_t)(k0 + r) * vs1 + d] : 0.f;
    }
    __syncthreads();
    float s[TK];
    float top = -INFINITY;
#pragma unroll
    for (int j = 0; j < TK; j++) {
      float a = 0.f;
#pragma unroll
      for (int d = 0; d < D; d++) a = fmaf(qr[d], kt[j][d], a);
      s[j] = j < nk ? a * c : -INFINITY;
      top = fmaxf(top, s[j]);
    }
    const float mn = fmaxf(m, top);
    const float alpha = exp2f(m - mn);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < TK; j++) {
      s[j] = exp2f(s[j] - mn);
      sum += s[j];
    }
    l = l * alpha + sum;
#pragma unroll
    for (int d = 0; d < D; d++) {
      float a = acc[d] * alpha;
#pragma unroll
      for (int j = 0; j < TK; j++) a = fmaf(s[j], vt[j][d], a);
      acc[d] = a;
    }
    m = mn;
  }
  if (!live) return;
  float* op = o + (int64_t)b * os0 + (int64_t)h * os2 + (int64_t)qi * os1;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int d = 0; d < D; d++) op[d] = acc[d] * inv;
}

// ------------------------------------------------------------------ attention (MFMA)
// FP32 attention on the fp16 matrix units in the reference's split form
// (_attention.py:19-28, 217-280): Q (scaled by scale * log2(e) in FP32), K, V and every
// probability p become hi = half(x) and lo = half((x - hi) * 2^11); S = Qh Kh +
// 2^-11 (Qh Kl + Ql Kh) and O = Ph Vh + 2^-11 (Ph Vl + Pl Vh), each in two FP32
// accumulators -- three fp16 products per FP32 product, only lo x lo dropped (about
// 2^-22 relative). The online softmax is FP32: running maximum (the exact base, moved
// every block it rises), exp2 of the log2-scaled scores, the row sum over the unrounded
// probabilities.
//
// Workgroup: 4 waves x 32 queries of one (batch, head); each wave computes S^T = K Q^T
// for a 32-key block (rows = keys permuted by split_key_row, columns = queries), so the
// lane's 16 scores are the B operand of O^T = V^T P^T as they lie, as in the fp16 kernels.
// 32-key tiles of K and V are loaded as FP32 into registers one block ahead, split, and
// stored as four fp16 planes (Kh, Kl rows permuted; Vh, Vl) in LDS, double-buffered with
// one barrier per block; the V^T operands are read with the transposing LDS read.
struct SplitAttnParams {
  int B, H, L, LK;
  const float* q; int64_t qs0, qs1, qs2;
  const float* k; int64_t ks0, ks1, ks2;
  const float* v; int64_t vs0, vs1, vs2;
  float* o; int64_t os0, os1, os2;
  float c;  // scale * log2(e)
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// The key permutation of the fp16 kernels: bits 2 and 3 of the row swapped, so that a
// lane's eight probabilities of one PV k-step are eight consecutive keys.
__device__ __forceinline__ int split_key_row(int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); }
__device__ __forceinline__ float split_halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float split_halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ f32x16 mfma_h(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int D>
__global__ __launch_bounds__(256) void attention_split_kernel(SplitAttnParams p) {
  constexpr int KB = 32;                 // keys per block
  constexpr int DK = D / 16, DB = D / 32;
  constexpr int KP = D + 8;              // plane pitch (halves)
  constexpr int PL = KB * KP;            // halves per plane
  constexpr int CH = KB * D / 4;         // 4-float chunks of an FP32 tile
  constexpr int CPT = CH / 256;          // of them per thread, for K and for V
  static_assert(D == 32 || D == 64, "head widths 32 and 64");
  static_assert(CH % 256 == 0, "whole chunks per thread");
  __shared__ __attribute__((aligned(16))) f16 smem[2 * 4 * PL];   // [buffer][Kh, Kl, Vh, Vl]

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hf = lane >> 5, col = lane & 31;
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
  }
  const int nqb = (p.L + 127) / 128;
  const int qblk = wg % nqb, h = (wg / nqb) % p.H, b = wg / nqb / p.H;
  const int q0 = qblk * 128 + wave * 32;
  const float* qb = p.q + (int64_t)b * p.qs0 + (int64_t)h * p.qs2;
  const float* kb_ = p.k + (int64_t)b * p.ks0 + (int64_t)h * p.ks2;
  const float* vb_ = p.v + (int64_t)b * p.vs0 + (int64_t)h * p.vs2;

  // Q^T fragments, scaled and split: lane holds query q0 + col, dims 16 dk + 8 hf .. + 7.
  const int qi = min(q0 + col, p.L - 1);
  f16x8 qh[DK], ql[DK];
#pragma unroll
  for (int dk = 0; dk < DK; dk++) {
    const float* src = qb + (int64_t)qi * p.qs1 + dk * 16 + 8 * hf;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src), c4 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      // The product is pinned as one fp32 value: left to contraction, the compiler rounds
      // q * c to fp16 once for one use (v_fma_mix) and via fp32 for the other, and where
      // the two roundings differ, hi and lo no longer split the same value.
      float x = (e < 4 ? a[e] : c4[e - 4]) * p.c;
      asm volatile("" : "+v"(x));
      const f16 hi = (f16)x;
      qh[dk][e] = hi;
      ql[dk][e] = (f16)((x - (float)hi) * 2048.0f);
    }
  }

  // The thread's chunks of a tile: chunk i covers key (tid + 256 i) / (D / 4), dims
  // 4 ((tid + 256 i) % (D / 4)) .. + 3; loads through buffer resources ending at the last
  // key, so rows past the sequence read zeros.
  f32x4 kst[CPT], vst[CPT];
  auto load_tile = [&](int kbase) {
    const int rows = min(KB, p.LK - kbase);
    const auto kr = make_rsrc(kb_ + (int64_t)kbase * p.ks1, (unsigned)(((rows - 1) * p.ks1 + D) * 4));
    const auto vr = make_rsrc(vb_ + (int64_t)kbase * p.vs1, (unsigned)(((rows - 1) * p.vs1 + D) * 4));
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int ch = threadIdx.x + 256 * i, key = ch / (D / 4), d0 = (ch % (D / 4)) * 4;
      kst[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, (int)((key * p.ks1 + d0) * 4), 0, 0));
      vst[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, (int)((key * p.vs1 + d0) * 4), 0, 0));
    }
  };
  auto store_tile = [&](int buf) {
    f16* base = smem + buf * 4 * PL;
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int ch = threadIdx.x + 256 * i, key = ch / (D / 4), d0 = (ch % (D / 4)) * 4;
      f16x4 kh, kl, vh, vl;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        kh[e] = (f16)kst[i][e];
        kl[e] = (f16)((kst[i][e] - (float)kh[e]) * 2048.0f);
        vh[e] = (f16)vst[i][e];
        vl[e] = (f16)((vst[i][e] - (float)vh[e]) * 2048.0f);
      }
      const int kr = split_key_row(key) * KP + d0, vrow = key * KP + d0;
      *reinterpret_cast<f16x4*>(base + kr) = kh;
      *reinterpret_cast<f16x4*>(base + PL + kr) = kl;
      *reinterpret_cast<f16x4*>(base + 2 * PL + vrow) = vh;
      *reinterpret_cast<f16x4*>(base + 3 * PL + vrow) = vl;
    }
  };
  // V^T operand of a PV k-step (rows = dims): in each 16-lane group g, lane i reads row
  // 8 (g / 2) + i / 4 (+ 4 for the second half, + 16 per k-step) at dims 16 (g % 2) +
  // 4 (i % 4) (+ 32 per block of O^T rows).
  const int vtr0 = (8 * (lane >> 5) + ((lane & 15) >> 2)) * KP + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  auto read_vt = [&](const f16* plane, int ks, int db) {
    const f16* va = plane + vtr0 + ks * 16 * KP + db * 32;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)((__attribute__((address_space(3))) char*)(va)));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)((__attribute__((address_space(3))) char*)(va + 4 * KP)));
    return __builtin_bit_cast(f16x8, (s16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
  };

  f32x16 oh[DB], ox[DB];
#pragma unroll
  for (int i = 0; i < DB; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) { oh[i][e] = 0.f; ox[i][e] = 0.f; }
  float m = -INFINITY, l = 0.f;
  const int nblk = (p.LK + KB - 1) / KB;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int it = 0; it < nblk; it++) {
    const int kbase = it * KB;
    if (it + 1 < nblk) load_tile(kbase + KB);
    const f16* Kh = smem + (it & 1) * 4 * PL;
    const f16* Kl = Kh + PL;
    const f16* Vh = Kh + 2 * PL;
    const f16* Vl = Kh + 3 * PL;
    f32x16 sh = {}, sx = {};
#pragma unroll
    for (int dk = 0; dk < DK; dk++) {
      const int d = dk * 16 + 8 * hf;
      const f16x8 kh = *reinterpret_cast<const f16x8*>(Kh + col * KP + d);
      const f16x8 kl = *reinterpret_cast<const f16x8*>(Kl + col * KP + d);
      sh = mfma_h(kh, qh[dk], sh);
      sx = mfma_h(kh, ql[dk], sx);
      sx = mfma_h(kl, qh[dk], sx);
    }
    // Lane holds keys kbase + 16 (e / 8) + 8 hf + e % 8 of query q0 + col (log2-scaled).
    float s[16], top = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int key = kbase + 16 * (e >> 3) + 8 * hf + (e & 7);
      s[e] = key < p.LK ? sh[e] + sx[e] * (1.0f / 2048.0f) : -INFINITY;
      top = fmaxf(top, s[e]);
    }
    const float mn = fmaxf(m, split_halves_max(top));
    const float alpha = exp2f(m - mn);
    m = mn;
    f16x8 ph[2], plo[2];
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const float pv = exp2f(s[e] - mn);
      sum += pv;
      const f16 hi = (f16)pv;
      ph[e >> 3][e & 7] = hi;
      plo[e >> 3][e & 7] = (f16)((pv - (float)hi) * 2048.0f);
    }
    l = l * alpha + sum;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int db = 0; db < DB; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) { oh[db][e] *= alpha; ox[db][e] *= alpha; }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int db = 0; db < DB; db++) {
        const f16x8 vh = read_vt(Vh, ks, db), vl = read_vt(Vl, ks, db);
        oh[db] = mfma_h(vh, ph[ks], oh[db]);
        ox[db] = mfma_h(vh, plo[ks], ox[db]);
        ox[db] = mfma_h(vl, ph[ks], ox[db]);
      }
    if (it + 1 < nblk) store_tile((it + 1) & 1);
    __syncthreads();
  }
  l = split_halves_sum(l);
  const int qo = q0 + col;
  if (qo < p.L) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    float* orow = p.o + (int64_t)b * p.os0 + (int64_t)h * p.os2 + (int64_t)qo * p.os1;
#pragma unroll
    for (int db = 0; db < DB; db++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f32x4 out;
#pragma unroll
        for (int r = 0; r < 4; r++) out[r] = (oh[db][j * 4 + r] + ox[db][j * 4 + r] * (1.0f / 2048.0f)) * inv;
        *reinterpret_cast<f32x4*>(orow + db * 32 + j * 8 + 4 * hf) = out;
      }
  }
}

static unsigned grid_for(int64_t n) {
  const int64_t g = (n + 255) / 256;
  return (unsigned)(g < 8192 ? g : 8192);
}

}  // namespace ldx

using namespace ldx;

// ------------------------------------------------------------------ entry points

extern "C" int ldx_pack_weight_exact(const float* weight, int32_t O, int32_t C, int32_t k, void* packed, void* stream) {
  if (!weight || !packed) return fail("pack_weight_exact: null pointer");
  if (O < 1 || C < 1 || (k != 1 && k != 3)) return fail("pack_weight_exact: bad shape O=%d C=%d k=%d", O, C, k);
  const int64_t n = (int64_t)ldx_packed_weight_elems(2 * O, 2 * C, k, 0);
  hipLaunchKernelGGL(pack_weight_exact_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), weight, O, C,
                     k * k * k, (f16*)packed);
  return check_launch("pack_weight_exact");
}

namespace ldx {
namespace f16_path {
int conv3d_raw(const ldx_conv3d_args* a, float* part, void* stream);
}  // namespace f16_path

// Geometry of an exact-mode conv: the row grid the fp16 conv reads and its output voxels.
static int exact_geometry(const ldx_conv3d_args* a, int64_t& row_vox, int64_t& out_vox) {
  if (!a) return fail("conv3d (fp32): null args");
  if (a->batch < 1 || a->in_d < 1 || a->in_h < 1 || a->in_w < 1 || a->c0 < 1 || a->c1 < 0 || a->out_c < 1)
    return fail("conv3d (fp32): bad shape");
  if (a->ksize != 1 && a->ksize != 3) return fail("conv3d (fp32): ksize must be 1 or 3");
  if (a->stride != 1 && a->stride != 2) return fail("conv3d (fp32): stride must be 1 or 2");
  if ((a->ksize == 1 || a->upsample) && a->stride != 1) return fail("conv3d (fp32): stride 2 needs a 3x3x3 conv");
  if (a->ksize == 1 && a->upsample) return fail("conv3d (fp32): upsampling needs a 3x3x3 conv");
  const int f = a->upsample ? 2 : 1;
  const int64_t rd = (int64_t)a->in_d * f, rh = (int64_t)a->in_h * f, rw = (int64_t)a->in_w * f;
  row_vox = rd * rh * rw;
  const int s = a->stride;
  auto ext = [&](int64_t n) { return s == 1 ? n : (n - 1) / 2 + 1; };
  out_vox = ext(rd) * ext(rh) * ext(rw);
  return LDX_OK;
}

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

size_t conv3d_exact_workspace_bytes(const ldx_conv3d_args* a) {
  int64_t rv, ov;
  if (exact_geometry(a, rv, ov) != LDX_OK) return 0;
  const int C = a->c0 + a->c1;
  return al256((size_t)a->batch * rv * 2 * C * sizeof(f16)) + (size_t)a->batch * ov * 2 * a->out_c * sizeof(float);
}

int conv3d_exact(const ldx_conv3d_args* a, void* stream) {
  int64_t rv, ov;
  if (int rc = exact_geometry(a, rv, ov)) return rc;
  if (!a->x0 || !a->weight || !a->y) return fail("conv3d (fp32): null x0 / weight / y");
  if (a->c1 > 0 && !a->x1) return fail("conv3d (fp32): c1 > 0 but x1 is null");
  if (a->x0_pitch < a->c0 || (a->c1 > 0 && a->x1_pitch < a->c1) || a->y_pitch < a->out_c)
    return fail("conv3d (fp32): pitch < channels");
  if (a->residual && a->residual_pitch < a->out_c) return fail("conv3d (fp32): residual pitch < out_c");
  if (a->act != LDX_ACT_NONE && a->act != LDX_ACT_GELU && a->act != LDX_ACT_SILU)
    return fail("conv3d (fp32): unknown act %d", a->act);
  const size_t need = conv3d_exact_workspace_bytes(a);
  if (!a->workspace || a->workspace_bytes < need)
    return fail("conv3d (fp32): needs %zu bytes of workspace (ldx_conv3d_workspace_bytes)", need);
  const int C = a->c0 + a->c1, O = a->out_c, B = a->batch;
  f16* xs = (f16*)a->workspace;
  float* part = (float*)((char*)a->workspace + al256((size_t)B * rv * 2 * C * sizeof(f16)));
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(split_exact_kernel, dim3(grid_for((int64_t)B * rv * C)), dim3(256), 0, st, (const float*)a->x0,
                     a->x0_pitch, a->c0, a->c1 > 0 ? (const float*)a->x1 : (const float*)a->x0,
                     a->c1 > 0 ? a->x1_pitch : a->x0_pitch, C, B, a->in_d, a->in_h, a->in_w, a->upsample, a->affine,
                     a->silu, xs);
  if (int rc = check_launch("conv3d (fp32): split")) return rc;
  // The products: an fp16 conv of the 2C split channels with the 2O stacked weight rows.
  ldx_conv3d_args ia{};
  const int f = a->upsample ? 2 : 1;
  ia.batch = B; ia.in_d = a->in_d * f; ia.in_h = a->in_h * f; ia.in_w = a->in_w * f;
  ia.c0 = 2 * C; ia.c1 = 0; ia.out_c = 2 * O; ia.ksize = a->ksize; ia.stride = a->stride; ia.upsample = 0;
  ia.x0 = xs; ia.x0_pitch = 2 * C;
  ia.weight = a->weight;
  ia.output_scale = 1.0f;
  ia.act = LDX_ACT_NONE;
  ia.y = part; ia.y_pitch = 2 * O;   // not written: the raw sums go to part
  ia.dtype = LDX_DTYPE_F16;
  if (int rc = f16_path::conv3d_raw(&ia, part, stream)) return rc;
  hipLaunchKernelGGL(exact_combine_kernel, dim3(grid_for((int64_t)B * ov * O)), dim3(256), 0, st, part, ov, B, O,
                     a->bias, a->bias_batched, (const float*)a->shift, a->shift_pitch, a->output_scale,
                     (const float*)a->residual, a->residual_pitch, a->act, (float*)a->y, a->y_pitch);
  return check_launch("conv3d (fp32): combine");
}

int attention_f32(const ldx_attention_args* a, void* stream) {
  if (!a || !a->q || !a->k || !a->v || !a->o) return fail("attention (fp32): null pointer");
  if (a->batch < 1 || a->heads < 1 || a->q_len < 1 || a->kv_len < 1) return fail("attention (fp32): empty input");
  if (a->mask) return fail("attention (fp32): masks are not supported");
  if ((int64_t)a->batch * a->heads > 65535) return fail("attention (fp32): too many (batch, head) pairs");
  const float c = a->scale * 1.44269504088896341f;
  hipStream_t st = as_stream(stream);
  // Head widths 32 and 64 with 16-byte rows run on the matrix units in the split form
  // (LDX_ATTN_F32=valu keeps the VALU kernel, for comparison); width 16 and other
  // layouts on the VALU kernel.
  const int D = a->head_dim;
  bool aligned = true;
  const int64_t* ss[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
  const void* ps[4] = {a->q, a->k, a->v, a->o};
  for (int i = 0; i < 4; i++) {
    if ((uintptr_t)ps[i] % 16) aligned = false;
    for (int j = 0; j < 3; j++)
      if (ss[i][j] % 4) aligned = false;
  }
  const char* env = getenv("LDX_ATTN_F32");
  if ((D == 32 || D == 64) && aligned && !(env && strcmp(env, "valu") == 0)) {
    // In-tile offsets are 32-bit: 32 key rows of K and of V.
    for (int i = 1; i < 3; i++)
      if (ss[i][1] < 0 || ss[i][1] > (1 << 24)) return fail("attention (fp32): key stride out of range");
    const int64_t n = (int64_t)((a->q_len + 127) / 128) * a->heads * a->batch;
    if (n > 0x7fffffff) return fail("attention (fp32): grid too large");
    SplitAttnParams sp{};
    sp.B = a->batch; sp.H = a->heads; sp.L = a->q_len; sp.LK = a->kv_len;
    sp.q = (const float*)a->q; sp.qs0 = a->q_stride[0]; sp.qs1 = a->q_stride[1]; sp.qs2 = a->q_stride[2];
    sp.k = (const float*)a->k; sp.ks0 = a->k_stride[0]; sp.ks1 = a->k_stride[1]; sp.ks2 = a->k_stride[2];
    sp.v = (const float*)a->v; sp.vs0 = a->v_stride[0]; sp.vs1 = a->v_stride[1]; sp.vs2 = a->v_stride[2];
    sp.o = (float*)a->o; sp.os0 = a->o_stride[0]; sp.os1 = a->o_stride[1]; sp.os2 = a->o_stride[2];
    sp.c = c;
    if (D == 32) hipLaunchKernelGGL(attention_split_kernel<32>, dim3((unsigned)n), dim3(256), 0, st, sp);
    else hipLaunchKernelGGL(attention_split_kernel<64>, dim3((unsigned)n), dim3(256), 0, st, sp);
    return check_launch("attention (fp32, split)");
  }
  const dim3 grid((unsigned)((a->q_len + 255) / 256), (unsigned)(a->batch * a->heads));
#define LDX_ATT32(D_)                                                                                           \
  hipLaunchKernelGGL(attention_f32_kernel<D_>, grid, dim3(256), 0, st, (const float*)a->q, a->q_stride[0],     \
                     a->q_stride[1], a->q_stride[2], (const float*)a->k, a->k_stride[0], a->k_stride[1],       \
                     a->k_stride[2], (const float*)a->v, a->v_stride[0], a->v_stride[1], a->v_stride[2],       \
                     (float*)a->o, a->o_stride[0], a->o_stride[1], a->o_stride[2], a->heads, a->q_len, a->kv_len, c)
  switch (a->head_dim) {
    case 16: LDX_ATT32(16); break;
    case 32: LDX_ATT32(32); break;
    case 64: LDX_ATT32(64); break;
    default: return fail("attention (fp32): head_dim %d not in {16, 32, 64}", a->head_dim);
  }
#undef LDX_ATT32
  return check_launch("attention (fp32)");
}
}  // namespace ldx

extern "C" int ldx_group_norm_affine_f32(const float* x0, int64_t x0_pitch, int32_t c0, const float* x1, int64_t x1_pitch,
                                         int32_t c1, int32_t batch, int64_t voxels, int32_t groups, const float* gamma,
                                         const float* beta, float eps, float* affine, void* stream) {
  if (!x0 || !gamma || !beta || !affine) return fail("group_norm_affine_f32: null pointer");
  if (c1 > 0 && !x1) return fail("group_norm_affine_f32: c1 > 0 but x1 is null");
  const int C = c0 + (c1 > 0 ? c1 : 0);
  if (batch < 1 || voxels < 1 || c0 < 1 || groups < 1 || C % groups || batch > 65535 || groups > 65535)
    return fail("group_norm_affine_f32: bad shape (batch %d voxels %lld C %d groups %d)", batch, (long long)voxels, C,
                groups);
  if (x0_pitch < c0 || (c1 > 0 && x1_pitch < c1)) return fail("group_norm_affine_f32: pitch < channels");
  hipLaunchKernelGGL(gn_f32_kernel, dim3(groups, batch), dim3(256), 0, as_stream(stream), x0, x0_pitch, c0,
                     c1 > 0 ? x1 : x0, c1 > 0 ? x1_pitch : x0_pitch, C, groups, voxels, gamma, beta, eps, affine);
  return check_launch("group_norm_affine_f32");
}

extern "C" int ldx_layer_norm_f32(const float* x, int64_t x_pitch, int64_t rows, int32_t features, const float* gamma,
                                  const float* beta, float eps, float* y, int64_t y_pitch, void* stream) {
  if (!x || !y || !gamma || !beta) return fail("layer_norm_f32: null pointer");
  if (rows < 1 || features < 1 || x_pitch < features || y_pitch < features) return fail("layer_norm_f32: bad shape");
  hipLaunchKernelGGL(layer_norm_f32_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, as_stream(stream), x,
                     x_pitch, rows, features, gamma, beta, eps, y, y_pitch);
  return check_launch("layer_norm_f32");
}

extern "C" int ldx_timestep_embedding_f32(const int32_t* timesteps, int32_t batch, int32_t channels, float* out,
                                          void* stream) {
  if (!timesteps || !out) return fail("timestep_embedding_f32: null pointer");
  if (batch < 1 || channels < 2 || channels % 2) return fail("timestep_embedding_f32: bad shape");
  hipLaunchKernelGGL(timestep_f32_kernel, dim3(grid_for((int64_t)batch * channels / 2)), dim3(256), 0,
                     as_stream(stream), timesteps, batch, channels, out);
  return check_launch("timestep_embedding_f32");
}
