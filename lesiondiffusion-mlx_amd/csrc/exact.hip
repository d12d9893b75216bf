// FP32 networks ("exact" mode): the reference keeps LMNet, and the conditioned VQ decode, in
// FP32 (src/lesiondiffusion_mlx/_nax_conv.py:26-34; medmlx.py:1362-1366). Here:
//
// * conv3d / dense layers in the split-FP16 form of _nax_conv.py:26-34, 210-237: each FP32
//   value v becomes hi = half(v) and lo = half((v - hi) * 2^11); hi x hi products go to one
//   FP32 sum, hi x lo + lo x hi to another, scaled back by 2^-11 (only lo x lo is dropped:
//   about 2^-22 relative). conv3d_exact_kernel does it in one launch: the FP32 input is
//   prepared (GroupNorm affine and SiLU in FP32, _nax_conv.py:128-136; a second input;
//   for a conv of a nearest-2x upsampling the upsampling, so that the conv runs on the
//   upsampled grid with the unfolded weights and no folded weight is re-split -- the
//   reference folds in FP32 before splitting, the same sums in another order), split into
//   hi / lo planes in LDS, three MFMAs per fragment pair accumulate the two sums, and the
//   epilogue y = ((S_hh + S_x * 2^-11) + (bias + shift)) * scale + residual (then GELU or
//   SiLU) runs in FP32 on the accumulators.
// * GroupNorm statistics and LayerNorm of FP32 tensors, FP32 timestep features.
// * attention in FP32: for head widths 32 / 64 on the matrix units in the reference's split
//   form (_attention.py:19-28, 217-280; attention_split_kernel), else (width 16, unaligned
//   tensors) a flash kernel on the VALU (the reference's FP32 SIMD kernel,
//   _attention.py:52-145): one query per lane, 64-key K/V tiles in LDS shared by the
//   workgroup's four waves, scores and P V as FP32 fused multiply-adds, online softmax
//   with exp2 of log2(e)-scaled scores.

#include "common.h"

#include <cmath>
#include <cstdlib>
#include <cstring>

namespace ldx {

// ------------------------------------------------------------------ weights
// The split weight as two fp16 planes, hi(W) then lo(W), each [NRB][NKC][taps][64][8]:
// row block rb (32 output channels), 16-channel chunk kc and tap t hold one MFMA A
// fragment -- lane l has row rb * 32 + l % 32, channels kc * 16 + 8 * (l / 32) + e -- so a
// wave reads a fragment as one 1 KiB run and a chunk's taps lie one after another.
// NRB = 2 * ceil(O / 64) (whole 64-row tiles), NKC = 4 * ceil(C / 64) (whole chunks of
// every k-grouping); zero outside O x C.
__host__ __device__ inline int64_t exact_plane_elems(int O, int C, int taps) {
  return (int64_t)((O + 63) / 64 * 2) * ((C + 63) / 64 * 4) * taps * 512;
}

__global__ void pack_weight_exact_kernel(const float* __restrict__ w, int O, int C, int taps, f16* __restrict__ out) {
  const int NKC = (C + 63) / 64 * 4;
  const int64_t plane = exact_plane_elems(O, C, taps);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < plane; i += (int64_t)gridDim.x * blockDim.x) {
    const int e = (int)(i & 7), l = (int)((i >> 3) & 63);
    const int64_t frag = i >> 9;
    const int tap = (int)(frag % taps), kc = (int)((frag / taps) % NKC);
    const int rb = (int)(frag / ((int64_t)taps * NKC));
    const int o = rb * 32 + (l & 31), c = kc * 16 + 8 * (l >> 5) + e;
    f16 hi = (f16)0.f, lo = (f16)0.f;
    if (o < O && c < C) {
      float wv = w[((int64_t)o * C + c) * taps + tap];
      asm volatile("" : "+v"(wv));  // one rounding of wv feeds both halves
      hi = (f16)wv;
      lo = (f16)((wv - (float)hi) * 2048.0f);
    }
    out[i] = hi;
    out[plane + i] = lo;
  }
}

__device__ __forceinline__ float gelu_erf32(float v) { return v * (1.0f + erff(v * 0.70710678118654752f)) * 0.5f; }

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
  touch_args(p);
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

// ------------------------------------------------------------------ conv (one pass)
// y = act(((W_h x_h + (W_h x_l + W_l x_h) 2^-11) + (bias + shift)) * scale + residual) in one
// launch: the FP32 input is read, prepared (GroupNorm affine, SiLU, nearest-2x upsampling,
// concatenation of x1) and split into hi / lo planes in LDS; three MFMAs per fragment pair
// (hi x hi into one FP32 accumulator, hi x lo and lo x hi into the other) and the FP32
// epilogue on the accumulators. No workspace, no intermediate tensor.
//
// Workgroup: a brick of BD x BH x BW output voxels (whole 32-voxel MFMA columns) of one
// batch item by 64 output channels, in KG k-groups (1, 2 or 4) of 2 x NCOL / NCW waves.
// Wave (kg, w) owns row block w % 2 and NCW columns from w / 2 on, for the 16 channels kg
// of each chunk of 16 KG channels. The brick's input halo, a chunk at a time, is staged as
// hi / lo fp16 sub-planes ([k-group][halo voxel][16], 32 B per voxel), double-buffered:
// the FP32 loads of the next chunk are issued at the chunk's first tap, and prepared and
// stored one item every other tap from tap 4 on, beside the MFMAs; one barrier per
// chunk. Weight fragments stream from the two-plane packing two taps ahead through a ring
// of three register slots (27 taps: the slot of a tap is fixed). At the end the k-groups'
// partial sums meet in LDS: with two groups of two columns per wave each wave hands one
// column to its partner and finishes the other; otherwise groups 1.. hand over and group
// 0 finishes. A sum over groups is S_g0 + S_g1 (+ S_g2 + S_g3), in that order. ksize 1
// (FLAT) treats the voxels of all batch items as one row of 128-voxel bricks.
struct ExactConvParams {
  const float* x0; const float* x1;
  int64_t p0, p1;
  int C0, C, O;
  int NCH;          // chunks of 16 KG channels
  int NKC;          // 16-channel chunks of the packed weight (a multiple of 4)
  int RD, RH, RW;   // row grid (the upsampled grid with up)
  int ID, IH, IW;   // source grid
  int OD, OH, OW;   // output grid
  int up, vec_in, vec_out;
  int nbd, nbh, nbw;  // bricks per output dimension (FLAT: nbw over all voxels)
  int64_t nvox;       // FLAT: batch * voxels
  const f16* w; int64_t wplane;  // two-plane weight, plane stride in halves
  const float* affine; int silu;
  const float* bias; int bias_batched;
  const float* shift; int64_t shiftp;
  float scale;
  const float* res; int64_t resp;
  int act;
  float* y; int64_t yp;
};

template <int KS, int S, int BD, int BH, int BW, int KG, int NCW>
struct ExactConvShape {
  static constexpr bool FLAT = KS == 1;
  static constexpr int PAD = KS / 2, TAPS = KS * KS * KS;
  static constexpr int HD = (BD - 1) * S + KS, HH = (BH - 1) * S + KS, HW = (BW - 1) * S + KS;
  static constexpr int NHV = HD * HH * HW;   // halo voxels
  static constexpr int NCOL = BD * BH * BW / 32;
  static constexpr int WPG = 2 * NCOL / NCW;  // waves per k-group: 2 row blocks x column sets
  static constexpr int NT = 64 * WPG * KG;    // threads
  static constexpr int GPV = 4 * KG;         // 4-channel groups per halo voxel and chunk
  static constexpr int PL = NHV * 16;        // halves per sub-plane
  static constexpr int BUF = 2 * KG * PL;    // halves per buffer (hi, lo x k-groups)
  static constexpr int NIT = (NHV * GPV + NT - 1) / NT;  // staging items per thread
  static constexpr int XCH = KG > 1 ? (KG == 2 ? NCW : KG - 1) * WPG * 2 * 16 * 64 * 4 : 0;  // exchange bytes
  static constexpr int LDS = 2 * BUF * 2 > XCH ? 2 * BUF * 2 : XCH;
  static_assert(BD * BH * BW % 32 == 0 && NCOL % NCW == 0, "whole columns per wave");
  static_assert(NT <= 1024, "workgroup size");
  static_assert(TAPS % 3 == 0 || TAPS == 1, "weight ring");
  static_assert(KG == 1 || (KG == 2 && NCW <= 2 && !FLAT) || (KG == 4 && NCW == 1 && !FLAT), "k-group exchange");
  static_assert(NT % GPV == 0, "a thread's channel group is fixed");
};

template <int KS, int S, int BD, int BH, int BW, int KG, int NCW>
__global__ __launch_bounds__((ExactConvShape<KS, S, BD, BH, BW, KG, NCW>::NT)) void conv3d_exact_kernel(
    ExactConvParams p) {
  touch_args(p);
  using SH = ExactConvShape<KS, S, BD, BH, BW, KG, NCW>;
  constexpr int TAPS = SH::TAPS, NIT = SH::NIT, PL = SH::PL, GPV = SH::GPV, WPG = SH::WPG;
  constexpr int CSETS = WPG / 2;   // column sets: wave w has columns w / 2 + CSETS j
  extern __shared__ __align__(16) f16 smem[];   // [2 buffers][hi, lo][k-group][PL]
  const int tid = threadIdx.x, lane = tid & 63;
  const int kg = tid / (64 * WPG), wave = (tid >> 6) % WPG;
  const int rb = wave & 1;
  const int oblk = blockIdx.y;

  // Brick origin (output grid) and batch item.
  int b = 0, od0 = 0, oh0 = 0, ow0 = 0;
  int64_t v0 = 0;   // FLAT: first voxel of the brick
  if constexpr (SH::FLAT) {
    v0 = (int64_t)blockIdx.x * 128;
  } else {
    int r = blockIdx.x;
    const int bw = r % p.nbw; r /= p.nbw;
    const int bh = r % p.nbh; r /= p.nbh;
    const int bd = r % p.nbd;
    b = r / p.nbd;
    od0 = bd * BD; oh0 = bh * BH; ow0 = bw * BW;
  }

  // Staging: item i = tid + NT k covers halo voxel i / GPV, channels 4 (i % GPV) .. + 3 of
  // the chunk (sub-plane (i % GPV) / 4); i % GPV is the same for all of a thread's items.
  const int g = tid % GPV;
  f32x4 pre[NIT];
  f32x4 aff_s = {1.f, 1.f, 1.f, 1.f}, aff_o = {0.f, 0.f, 0.f, 0.f};
  // Source voxel of each item's halo voxel, or -1 in the padding (or past the last FLAT
  // voxel); the same for every chunk.
  int sv[NIT];
#pragma unroll
  for (int k = 0; k < NIT; k++) {
    const int i = tid + SH::NT * k, hv = i / GPV;
    sv[k] = -1;
    if (i >= SH::NHV * GPV) continue;
    if constexpr (SH::FLAT) {
      if (v0 + hv < p.nvox) sv[k] = (int)(v0 + hv);
    } else {
      const int hd = hv / (SH::HH * SH::HW), hh = (hv / SH::HW) % SH::HH, hw = hv % SH::HW;
      const int rd = od0 * S - SH::PAD + hd, rh = oh0 * S - SH::PAD + hh, rw = ow0 * S - SH::PAD + hw;
      if (rd < 0 || rd >= p.RD || rh < 0 || rh >= p.RH || rw < 0 || rw >= p.RW) continue;
      const int sd = p.up ? rd >> 1 : rd, sh = p.up ? rh >> 1 : rh, sw = p.up ? rw >> 1 : rw;
      sv[k] = ((b * p.ID + sd) * p.IH + sh) * p.IW + sw;
    }
  }
  auto load_affine = [&](int bi, int c) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const bool in = c + e < p.C;
      const float* af = p.affine + ((int64_t)bi * p.C + (in ? c + e : 0)) * 2;
      aff_s[e] = in ? af[0] : 1.f;
      aff_o[e] = in ? af[1] : 0.f;
    }
  };
  auto load_chunk = [&](int kc) {
    const int c = kc * 16 * KG + g * 4;
    if (!SH::FLAT && p.affine) load_affine(b, c);
    const bool in0 = c < p.C0;
    const float* base = in0 ? p.x0 + c : p.x1 + (c - p.C0);
    const int64_t pitch = in0 ? p.p0 : p.p1;
#pragma unroll
    for (int k = 0; k < NIT; k++) {
      pre[k] = (f32x4){0.f, 0.f, 0.f, 0.f};
      if (sv[k] < 0 || c >= p.C) continue;
      if (p.vec_in) {
        pre[k] = *reinterpret_cast<const f32x4*>(base + sv[k] * pitch);
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (c + e < p.C) pre[k][e] = c + e < p.C0 ? p.x0[sv[k] * p.p0 + c + e] : p.x1[sv[k] * p.p1 + (c + e - p.C0)];
      }
    }
  };
  // Prepare (affine, SiLU), split and store item k of the loaded chunk into buffer buf.
  // Padding and channels past C stay zero (the conv pads the prepared input).
  auto store_item = [&](int k, int kc, int buf) {
    const int i = tid + SH::NT * k;
    if (i >= SH::NHV * GPV) return;
    const int hv = i / GPV;
    const int c = kc * 16 * KG + g * 4;
    const bool ok = sv[k] >= 0 && c < p.C;
    if (SH::FLAT && ok && p.affine) load_affine((int)(sv[k] / ((int64_t)p.OD * p.OH * p.OW)), c);
    f16x4 h4, l4;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float v = pre[k][e];
      if (p.affine) v = v * aff_s[e] + aff_o[e];
      if (p.silu) v = v / (1.0f + expf(-v));
      if (!ok || c + e >= p.C) v = 0.f;
      asm volatile("" : "+v"(v));  // one value feeds both halves
      const f16 vh = (f16)v;
      h4[e] = vh;
      l4[e] = (f16)((v - (float)vh) * 2048.0f);
    }
    f16* dst = smem + buf * SH::BUF + (g >> 2) * PL + hv * 16 + (g & 3) * 4;
    *reinterpret_cast<f16x4*>(dst) = h4;
    *reinterpret_cast<f16x4*>(dst + KG * PL) = l4;
  };

  // Columns of this wave: brick-local voxel of the lane and its halo voxel.
  int hb[NCW];
#pragma unroll
  for (int j = 0; j < NCW; j++) {
    const int v = ((wave >> 1) + CSETS * j) * 32 + (lane & 31);
    if constexpr (SH::FLAT) {
      hb[j] = v;
    } else {
      const int ld = v / (BH * BW), lh = (v / BW) % BH, lw = v % BW;
      hb[j] = (ld * S * SH::HH + lh * S) * SH::HW + lw * S;
    }
  }

  // Weight fragments: row block 2 * oblk + rb, 16-channel chunk KG kc + kg; (chunk, tap)
  // runs consecutively.
  const f16* wrow = p.w + ((int64_t)(2 * oblk + rb) * p.NKC + kg) * TAPS * 512 + lane * 8;
  constexpr int R = TAPS == 1 ? 2 : 3;
  f16x8 ah[R], al[R];
  auto load_w = [&](int kc, int t, int slot) {
    const f16* q = wrow + ((int64_t)kc * KG * TAPS + t) * 512;
    ah[slot] = *reinterpret_cast<const f16x8*>(q);
    al[slot] = *reinterpret_cast<const f16x8*>(q + p.wplane);
  };

  f32x16 acc_h[NCW], acc_x[NCW];
#pragma unroll
  for (int j = 0; j < NCW; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) acc_h[j][e] = acc_x[j][e] = 0.f;

  // Prologue: chunk 0 staged, the first weight fragments in flight.
  load_chunk(0);
  load_w(0, 0, 0);
  if constexpr (TAPS > 1) load_w(0, 1, 1);
#pragma unroll
  for (int k = 0; k < NIT; k++) store_item(k, 0, 0);
  __syncthreads();

  // First tap that stores a staged item of the next chunk (one every other tap).
  constexpr int T0 = 4 + 2 * (NIT - 1) < TAPS ? 4 : TAPS - 1 - 2 * (NIT - 1);
  static_assert(TAPS == 1 || T0 >= 1, "staging fits the tap loop");
  const int half = 8 * (lane >> 5);
  for (int kc = 0; kc < p.NCH; kc++) {
    const int buf = kc & 1;
    const bool more = kc + 1 < p.NCH;
    const f16* xb = smem + buf * SH::BUF + kg * PL + half;
    if constexpr (TAPS == 1) {
      if (more) load_w(kc + 1, 0, 1);
      if (more) load_chunk(kc + 1);
      f16x8 xh[NCW], xl[NCW];
#pragma unroll
      for (int j = 0; j < NCW; j++) {
        xh[j] = *reinterpret_cast<const f16x8*>(xb + hb[j] * 16);
        xl[j] = *reinterpret_cast<const f16x8*>(xb + KG * PL + hb[j] * 16);
      }
#pragma unroll
      for (int j = 0; j < NCW; j++) acc_h[j] = mfma_h(ah[0], xh[j], acc_h[j]);
#pragma unroll
      for (int j = 0; j < NCW; j++) acc_x[j] = mfma_h(ah[0], xl[j], acc_x[j]);
#pragma unroll
      for (int j = 0; j < NCW; j++) acc_x[j] = mfma_h(al[0], xh[j], acc_x[j]);
      ah[0] = ah[1];
      al[0] = al[1];
      if (more) {
#pragma unroll
        for (int k = 0; k < NIT; k++) store_item(k, kc + 1, buf ^ 1);
      }
    } else {
#pragma unroll
      for (int t = 0; t < TAPS; t++) {
        // Weights two taps ahead (into the slot tap t - 1 used), the next chunk's input
        // after the first of them.
        if (t + 2 < TAPS) load_w(kc, t + 2, (t + 2) % 3);
        else if (more) load_w(kc + 1, t + 2 - TAPS, (t + 2) % 3);
        if (t == 0 && more) load_chunk(kc + 1);
        const int toff = ((t / 9) * SH::HH + (t / 3) % 3) * SH::HW + t % 3;
        f16x8 xh[NCW], xl[NCW];
#pragma unroll
        for (int j = 0; j < NCW; j++) {
          xh[j] = *reinterpret_cast<const f16x8*>(xb + (hb[j] + toff) * 16);
          xl[j] = *reinterpret_cast<const f16x8*>(xb + KG * PL + (hb[j] + toff) * 16);
        }
        const int s = t % 3;
#pragma unroll
        for (int j = 0; j < NCW; j++) acc_h[j] = mfma_h(ah[s], xh[j], acc_h[j]);
#pragma unroll
        for (int j = 0; j < NCW; j++) acc_x[j] = mfma_h(ah[s], xl[j], acc_x[j]);
#pragma unroll
        for (int j = 0; j < NCW; j++) acc_x[j] = mfma_h(al[s], xh[j], acc_x[j]);
        if (more && t >= T0 && (t - T0) % 2 == 0 && (t - T0) / 2 < NIT) store_item((t - T0) / 2, kc + 1, buf ^ 1);
      }
    }
    __syncthreads();
  }

  // Two k-groups: with two columns per wave, wave (kg, w) leaves its partial sums of
  // column 1 - kg in LDS (the halo buffers are free after the loop's last barrier) and
  // finishes column kg with its partner's; with one, group 1 hands over and group 0
  // finishes. Either way a sum is S_g0 + S_g1, in that order.
  if constexpr (KG == 4) {
    // Groups 1-3 hand over; group 0 adds ((S_g0 + S_g1) + S_g2) + S_g3.
    float* xs = reinterpret_cast<float*>(smem);
    auto slot = [&](int g1, int acc, int e) { return ((((g1 * WPG + wave) * 2 + acc) * 16 + e) * 64) + lane; };
    if (kg > 0) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        xs[slot(kg - 1, 0, e)] = acc_h[0][e];
        xs[slot(kg - 1, 1, e)] = acc_x[0][e];
      }
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g1 = 0; g1 < 3; g1++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        acc_h[0][e] = acc_h[0][e] + xs[slot(g1, 0, e)];
        acc_x[0][e] = acc_x[0][e] + xs[slot(g1, 1, e)];
      }
  }
  if constexpr (KG == 2) {
    float* xs = reinterpret_cast<float*>(smem);
    auto slot = [&](int j, int acc, int e) { return ((((j * WPG + wave) * 2 + acc) * 16 + e) * 64) + lane; };
    if constexpr (NCW == 2) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        xs[slot(1 - kg, 0, e)] = kg ? acc_h[0][e] : acc_h[1][e];
        xs[slot(1 - kg, 1, e)] = kg ? acc_x[0][e] : acc_x[1][e];
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float ph = xs[slot(kg, 0, e)], px = xs[slot(kg, 1, e)];
        if (kg == 0) {
          acc_h[0][e] = acc_h[0][e] + ph;
          acc_x[0][e] = acc_x[0][e] + px;
        } else {
          acc_h[0][e] = ph + acc_h[1][e];
          acc_x[0][e] = px + acc_x[1][e];
        }
      }
    } else {
      if (kg == 1) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
          xs[slot(0, 0, e)] = acc_h[0][e];
          xs[slot(0, 1, e)] = acc_x[0][e];
        }
      }
      __syncthreads();
      if (kg == 1) return;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        acc_h[0][e] = acc_h[0][e] + xs[slot(0, 0, e)];
        acc_x[0][e] = acc_x[0][e] + xs[slot(0, 1, e)];
      }
    }
  }

  // Epilogue: lane (half, col) holds voxel col of each of its columns, channels
  // 64 oblk + 32 rb + 8 q + 4 (lane / 32) + r in element 4 q + r.
  const int64_t ovol = (int64_t)p.OD * p.OH * p.OW;
  constexpr int NFIN = KG > 1 ? 1 : NCW;   // columns this wave finishes
#pragma unroll
  for (int j = 0; j < NFIN; j++) {
    const int col = (wave >> 1) + CSETS * (KG == 2 && NCW == 2 ? kg : j);
    const int v = col * 32 + (lane & 31);
    int64_t ov;
    int bi = b;
    bool ok;
    if constexpr (SH::FLAT) {
      ov = v0 + v;
      ok = ov < p.nvox;
      bi = ok ? (int)(ov / ovol) : 0;
    } else {
      const int od = od0 + v / (BH * BW), oh = oh0 + (v / BW) % BH, ow = ow0 + v % BW;
      ok = od < p.OD && oh < p.OH && ow < p.OW;
      ov = (((int64_t)b * p.OD + od) * p.OH + oh) * p.OW + ow;
    }
    if (!ok) continue;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int o0 = oblk * 64 + rb * 32 + 8 * q + 4 * (lane >> 5);
      if (o0 >= p.O) continue;
      f32x4 t;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int o = o0 + r < p.O ? o0 + r : p.O - 1;
        const float sum = acc_h[j][4 * q + r] + acc_x[j][4 * q + r] * (1.0f / 2048.0f);
        float add = p.bias ? p.bias[(p.bias_batched ? (int64_t)bi * p.O : 0) + o] : 0.f;
        if (p.shift) add += p.shift[(int64_t)bi * p.shiftp + o];
        float u = (sum + add) * p.scale;
        if (p.res) u += p.res[ov * p.resp + o];
        if (p.act == LDX_ACT_GELU) u = gelu_erf32(u);
        else if (p.act == LDX_ACT_SILU) u = u / (1.0f + expf(-u));
        t[r] = u;
      }
      float* yo = p.y + ov * p.yp + o0;
      if (p.vec_out && o0 + 3 < p.O) {
        *reinterpret_cast<f32x4*>(yo) = t;
      } else {
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (o0 + r < p.O) yo[r] = t[r];
      }
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

extern "C" size_t ldx_packed_weight_exact_elems(int32_t O, int32_t C, int32_t k) {
  if (O < 1 || C < 1 || (k != 1 && k != 3)) return 0;
  return (size_t)(2 * exact_plane_elems(O, C, k * k * k));
}

extern "C" int ldx_pack_weight_exact(const float* weight, int32_t O, int32_t C, int32_t k, void* packed, void* stream) {
  if (!weight || !packed) return fail("pack_weight_exact: null pointer");
  if (O < 1 || C < 1 || (k != 1 && k != 3)) return fail("pack_weight_exact: bad shape O=%d C=%d k=%d", O, C, k);
  const int64_t n = exact_plane_elems(O, C, k * k * k);
  hipLaunchKernelGGL(pack_weight_exact_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), weight, O, C,
                     k * k * k, (f16*)packed);
  return check_launch("pack_weight_exact");
}

namespace ldx {

// Geometry of an exact-mode conv: its row grid (the upsampled grid with upsample) and
// output grid.
static int exact_geometry(const ldx_conv3d_args* a, int64_t rg[3], int64_t og[3]) {
  if (!a) return fail("conv3d (fp32): null args");
  if (a->batch < 1 || a->in_d < 1 || a->in_h < 1 || a->in_w < 1 || a->c0 < 1 || a->c1 < 0 || a->out_c < 1)
    return fail("conv3d (fp32): bad shape");
  if (a->ksize != 1 && a->ksize != 3) return fail("conv3d (fp32): ksize must be 1 or 3");
  if (a->stride != 1 && a->stride != 2) return fail("conv3d (fp32): stride must be 1 or 2");
  if ((a->ksize == 1 || a->upsample) && a->stride != 1) return fail("conv3d (fp32): stride 2 needs a 3x3x3 conv");
  if (a->ksize == 1 && a->upsample) return fail("conv3d (fp32): upsampling needs a 3x3x3 conv");
  const int f = a->upsample ? 2 : 1;
  rg[0] = (int64_t)a->in_d * f; rg[1] = (int64_t)a->in_h * f; rg[2] = (int64_t)a->in_w * f;
  for (int i = 0; i < 3; i++) og[i] = a->stride == 1 ? rg[i] : (rg[i] - 1) / 2 + 1;
  if (rg[0] * rg[1] * rg[2] * a->batch >= (1ll << 31) || (int64_t)a->c0 + a->c1 >= (1 << 24))
    return fail("conv3d (fp32): tensor too large");
  return LDX_OK;
}

size_t conv3d_exact_workspace_bytes(const ldx_conv3d_args*) { return 0; }

template <int KS, int S, int BD, int BH, int BW, int KG, int NCW>
static int launch_exact(ExactConvParams p, int64_t bricks, hipStream_t st) {
  using SH = ExactConvShape<KS, S, BD, BH, BW, KG, NCW>;
  auto kern = conv3d_exact_kernel<KS, S, BD, BH, BW, KG, NCW>;
  const int lds = SH::LDS;
  p.NCH = (p.C + 16 * KG - 1) / (16 * KG);
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
    return fail("conv3d (fp32): cannot reserve %d bytes of LDS", lds);
  if (bricks >= (1ll << 31) || (p.O + 63) / 64 > 65535) return fail("conv3d (fp32): grid too large");
  hipLaunchKernelGGL(kern, dim3((unsigned)bricks, (unsigned)((p.O + 63) / 64)), dim3(SH::NT), lds, st, p);
  return check_launch("conv3d (fp32)");
}

static bool al16(const void* q) { return ((uintptr_t)q & 15) == 0; }

int conv3d_exact(const ldx_conv3d_args* a, void* stream) {
  int64_t rg[3], og[3];
  if (int rc = exact_geometry(a, rg, og)) return rc;
  if (!a->x0 || !a->weight || !a->y) return fail("conv3d (fp32): null x0 / weight / y");
  if (a->c1 > 0 && !a->x1) return fail("conv3d (fp32): c1 > 0 but x1 is null");
  if (a->x0_pitch < a->c0 || (a->c1 > 0 && a->x1_pitch < a->c1) || a->y_pitch < a->out_c)
    return fail("conv3d (fp32): pitch < channels");
  if (a->residual && a->residual_pitch < a->out_c) return fail("conv3d (fp32): residual pitch < out_c");
  if (a->act != LDX_ACT_NONE && a->act != LDX_ACT_GELU && a->act != LDX_ACT_SILU)
    return fail("conv3d (fp32): unknown act %d", a->act);
  const int C = a->c0 + a->c1, O = a->out_c, K = a->ksize;
  ExactConvParams p{};
  p.x0 = (const float*)a->x0; p.p0 = a->x0_pitch; p.C0 = a->c0;
  p.x1 = a->c1 > 0 ? (const float*)a->x1 : p.x0; p.p1 = a->c1 > 0 ? a->x1_pitch : a->x0_pitch;
  p.C = C; p.O = O; p.NKC = (C + 63) / 64 * 4;
  p.RD = (int)rg[0]; p.RH = (int)rg[1]; p.RW = (int)rg[2];
  p.ID = a->in_d; p.IH = a->in_h; p.IW = a->in_w;
  p.OD = (int)og[0]; p.OH = (int)og[1]; p.OW = (int)og[2];
  p.up = a->upsample;
  p.vec_in = C % 4 == 0 && a->c0 % 4 == 0 && a->x0_pitch % 4 == 0 && al16(p.x0) &&
             (a->c1 == 0 || (a->x1_pitch % 4 == 0 && al16(p.x1)));
  p.vec_out = a->y_pitch % 4 == 0 && al16(a->y);
  p.w = (const f16*)a->weight; p.wplane = exact_plane_elems(O, C, K * K * K);
  p.affine = a->affine; p.silu = a->silu;
  p.bias = a->bias; p.bias_batched = a->bias_batched;
  p.shift = (const float*)a->shift; p.shiftp = a->shift_pitch;
  p.scale = a->output_scale;
  p.res = (const float*)a->residual; p.resp = a->residual_pitch;
  p.act = a->act;
  p.y = (float*)a->y; p.yp = a->y_pitch;
  hipStream_t st = as_stream(stream);
  if (K == 1) {
    p.nvox = (int64_t)a->batch * og[0] * og[1] * og[2];
    return launch_exact<1, 1, 1, 1, 128, 1, 2>(p, ceil_div64(p.nvox, 128), st);
  }
  auto bricks = [&](int bd, int bh, int bw) {
    p.nbd = (int)ceil_div64(og[0], bd); p.nbh = (int)ceil_div64(og[1], bh); p.nbw = (int)ceil_div64(og[2], bw);
    return (int64_t)a->batch * p.nbd * p.nbh * p.nbw;
  };
  // Tile choice (measured on MI355X at LMNet's grids): the 128-voxel brick with two
  // k-groups while it gives at least 128 workgroups (half
  // the CUs); below that the 32-voxel brick with four k-groups (3,040 voxels x 128
  // channels: 21.7 us against 50.5 us); stride 2 the 32-voxel brick with two k-groups
  // (its 5x9x9 halo leaves no room for four).
  const int64_t oblocks = (O + 63) / 64;
  int64_t nb;   // (the brick counts go into p before p is passed on)
  if (a->stride == 2) {
    nb = bricks(2, 4, 4);
    return launch_exact<3, 2, 2, 4, 4, 2, 1>(p, nb, st);
  }
  nb = bricks(4, 4, 8);
  if (nb * oblocks >= 128) return launch_exact<3, 1, 4, 4, 8, 2, 2>(p, nb, st);
  nb = bricks(2, 4, 4);
  return launch_exact<3, 1, 2, 4, 4, 4, 1>(p, nb, st);
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
