// Small kernels of the hot path: weight packing, GroupNorm statistics, LayerNorm,
// timestep features, SiLU, channel-slice copies and the DDIM step; plus the
// library's error plumbing.

#include "common.h"

#include <cmath>
#include <mutex>

namespace ldx {

static thread_local std::string g_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return LDX_EINVAL;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return LDX_EHIP;
  }
  return LDX_OK;
}

static inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }
static inline unsigned grid_cap(int64_t n, int per, unsigned cap) {
  const int64_t g = (n + per - 1) / per;
  return g < (int64_t)cap ? (unsigned)g : cap;
}

// ------------------------------------------------------------------ packing
// Fragment-major layout of the 32x32x16 MFMA A operand (32 output rows x 16 reduction
// values per fragment, 1 KB): fragment (ob, tap, kc) holds, at lane l's 16 bytes
// (offset l * 8 halves), W[o = ob*32 + l%32][tap][c = kc*16 + 8*(l/32) + e], e < 8,
// zero past O or C. NOB = ceil(O/128)*4 and NKC = ceil(C/64)*4, so any 128-row x
// 64-channel tile of fragments exists. Upsample weights prefix the parity:
// ((parity*NOB + ob)*8 + tap).
__device__ __forceinline__ void frag_coords(int64_t i, int NKC, int taps, int& e, int& l, int& kc,
                                            int& tap, int64_t& obp) {
  e = (int)(i & 7);
  l = (int)((i >> 3) & 63);
  const int64_t frag = i >> 9;
  kc = (int)(frag % NKC);
  tap = (int)((frag / NKC) % taps);
  obp = frag / ((int64_t)NKC * taps);
}

__global__ void pack_weight_kernel(const f16* __restrict__ w, int O, int C, int taps,
                                   f16* __restrict__ out) {
  const int NOB = (O + 127) / 128 * 4, NKC = (C + 63) / 64 * 4;
  const int64_t n = (int64_t)NOB * taps * NKC * 512;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int e, l, kc, tap; int64_t ob;
    frag_coords(i, NKC, taps, e, l, kc, tap, ob);
    const int o = (int)ob * 32 + (l & 31);
    const int c = kc * 16 + 8 * (l >> 5) + e;
    out[i] = (o < O && c < C) ? w[((int64_t)o * C + c) * taps + tap] : (f16)0;
  }
}

// Fold one axis: parity p, tap t -> the original taps it merges.
__device__ __forceinline__ void fold_set(int p, int t, int& k_lo, int& k_hi) {
  // p = 0: t = 0 -> {0}, t = 1 -> {1, 2};  p = 1: t = 0 -> {0, 1}, t = 1 -> {2}
  if (p == 0) { k_lo = t == 0 ? 0 : 1; k_hi = t == 0 ? 0 : 2; }
  else { k_lo = t == 0 ? 0 : 2; k_hi = t == 0 ? 1 : 2; }
}

// parity = pd*4+ph*2+pw, tap = td*4+th*2+tw. Sums are float32 and nest d (innermost),
// then h, then w, each left to right -- the order of the reference's per-axis folds
// (_nax_conv.py:394-405) -- and are rounded to fp16 once.
template <typename T>
__global__ void pack_upsample_kernel(const T* __restrict__ w, int O, int C, T* __restrict__ out) {
  const int NOB = (O + 127) / 128 * 4, NKC = (C + 63) / 64 * 4;
  const int64_t n = (int64_t)8 * NOB * 8 * NKC * 512;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int e, l, kc, tap; int64_t pob;
    frag_coords(i, NKC, 8, e, l, kc, tap, pob);
    const int parity = (int)(pob / NOB), ob = (int)(pob % NOB);
    const int o = ob * 32 + (l & 31);
    const int c = kc * 16 + 8 * (l >> 5) + e;
    if (o >= O || c >= C) { out[i] = (T)0.f; continue; }
    const int pd = parity >> 2, ph = (parity >> 1) & 1, pw = parity & 1;
    const int td = tap >> 2, th = (tap >> 1) & 1, tw = tap & 1;
    int d_lo, d_hi, h_lo, h_hi, w_lo, w_hi;
    fold_set(pd, td, d_lo, d_hi);
    fold_set(ph, th, h_lo, h_hi);
    fold_set(pw, tw, w_lo, w_hi);
    const T* base = w + ((int64_t)o * C + c) * 27;
    float tot = 0.0f;
    for (int kw = w_lo; kw <= w_hi; kw++) {
      float hs = 0.0f;
      for (int kh = h_lo; kh <= h_hi; kh++) {
        float ds = 0.0f;
        for (int kd = d_lo; kd <= d_hi; kd++) ds += (float)base[kd * 9 + kh * 3 + kw];
        hs += ds;
      }
      tot += hs;
    }
    out[i] = (T)tot;
  }
}

// ------------------------------------------------------------ group norm
// Pass 1: each workgroup reduces `chunk` voxels of one batch item to per-group
// (count, mean, M2) partials; per-thread sums over a few voxels, converted to
// (n, mean, M2) and merged (Chan et al.) in a fixed order, so results are
// deterministic run to run.
template <int V>
__global__ __launch_bounds__(256) void gn_partial_kernel(
    const f16* __restrict__ x0, int64_t p0, int C0, const f16* __restrict__ x1, int64_t p1,
    int C, int G, int64_t S, int64_t chunk, float* __restrict__ partial, int nchunks) {
  // Thread t owns channels [lane_c, lane_c + V) of voxels vsub, vsub + vpi, ... of the
  // chunk and sums (x - K_c) and (x - K_c)^2 with K_c the channel's value at the chunk's
  // first voxel (a shift that keeps the variance free of cancellation).
  __shared__ float s_sum[256 * V];
  __shared__ float s_sq[256 * V];
  __shared__ float c_n[2048], c_mean[2048], c_m2[2048];
  const int b = blockIdx.y;
  const int ch = blockIdx.x;
  const int tpv = C / V;
  const int vpi = 256 / tpv;
  const int t = threadIdx.x;
  const int lane_c = (t % tpv) * V;
  const int vsub = t / tpv;
  const bool active = vsub < vpi;
  const int64_t v_begin = (int64_t)ch * chunk;
  const int64_t v_end = min(S, v_begin + chunk);
  auto src_of = [&](int64_t v) {
    const int64_t vi = (int64_t)b * S + v;
    return lane_c < C0 ? x0 + vi * p0 + lane_c : x1 + vi * p1 + (lane_c - C0);
  };
  float k[V], sum[V], sq[V];
  {
    const f16* s0 = src_of(v_begin);
#pragma unroll
    for (int e = 0; e < V; e++) { k[e] = (float)s0[e]; sum[e] = 0.f; sq[e] = 0.f; }
  }
  if (active) {
    int64_t v = v_begin + vsub;
    if constexpr (V == 8) {
      // Eight voxels' loads in flight per thread (one wave per SIMD would otherwise wait
      // out each load's latency), summed in the same voxel order as one at a time.
      for (; v + 7 * vpi < v_end; v += 8 * vpi) {
        f16x8 h[8];
#pragma unroll
        for (int u = 0; u < 8; u++) h[u] = *reinterpret_cast<const f16x8*>(src_of(v + u * vpi));
#pragma unroll
        for (int u = 0; u < 8; u++)
#pragma unroll
          for (int e = 0; e < 8; e++) { const float f = (float)h[u][e] - k[e]; sum[e] += f; sq[e] += f * f; }
      }
    }
    for (; v < v_end; v += vpi) {
      const f16* src = src_of(v);
      if constexpr (V == 8) {
        const f16x8 h = *reinterpret_cast<const f16x8*>(src);
#pragma unroll
        for (int e = 0; e < 8; e++) { const float f = (float)h[e] - k[e]; sum[e] += f; sq[e] += f * f; }
      } else {
#pragma unroll
        for (int e = 0; e < V; e++) { const float f = (float)src[e] - k[e]; sum[e] += f; sq[e] += f * f; }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < V; e++) {
    s_sum[t * V + e] = active ? sum[e] : 0.f;
    s_sq[t * V + e] = active ? sq[e] : 0.f;
  }
  __syncthreads();
  // Per channel: add the vpi thread partials (same shift), then (n, mean, M2).
  const float n_c = (float)(v_end - v_begin);
  for (int c = t; c < C; c += 256) {
    const int tc = c / V, e = c % V;
    float a = 0.f, q = 0.f;
    for (int vs = 0; vs < vpi; vs++) { a += s_sum[(vs * tpv + tc) * V + e]; q += s_sq[(vs * tpv + tc) * V + e]; }
    const f16* s0 = c < C0 ? x0 + ((int64_t)b * S + v_begin) * p0 + c
                           : x1 + ((int64_t)b * S + v_begin) * p1 + (c - C0);
    const float kc = (float)*s0;
    const float m = a / n_c;
    c_n[c] = n_c;
    c_mean[c] = kc + m;
    c_m2[c] = fmaxf(q - a * m, 0.f);
  }
  __syncthreads();
  const int gs = C / G;
  for (int g = t; g < G; g += 256) {
    Moments m = {0.f, 0.f, 0.f};
    for (int c = g * gs; c < (g + 1) * gs; c++) m = merge(m, Moments{c_n[c], c_mean[c], c_m2[c]});
    float* out = partial + (((int64_t)b * nchunks + ch) * G + g) * 3;
    out[0] = m.n; out[1] = m.mean; out[2] = m.m2;
  }
}

// Pass 2: one workgroup per (group, batch item) merges the chunk partials in a
// fixed tree order and writes the (scale, offset) pairs of the group's channels.
__global__ __launch_bounds__(256) void gn_finalize_kernel(
    const float* __restrict__ partial, int nchunks, int C, int G, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, float* __restrict__ affine) {
  __shared__ float red[12];
  const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  Moments m = {0.f, 0.f, 0.f};
  for (int j = t; j < nchunks; j += 256) {
    const float* pp = partial + (((int64_t)b * nchunks + j) * G + g) * 3;
    m = merge(m, Moments{pp[0], pp[1], pp[2]});
  }
  const Moments tot = block_merge256(m, red);
  const float mean = tot.mean;
  const float var = tot.n > 0.f ? tot.m2 / tot.n : 0.f;
  const float rstd = 1.0f / sqrtf(var + eps);
  const int gs = C / G;
  for (int c = g * gs + t; c < (g + 1) * gs; c += 256) {
    const float sc = gamma[c] * rstd;
    affine[((int64_t)b * C + c) * 2] = sc;
    affine[((int64_t)b * C + c) * 2 + 1] = beta[c] - sc * mean;
  }
}

// Small tensors (coarse UNet levels): one launch, one workgroup per (group, batch item).
// Thread t sums (x - K) and (x - K)^2 over the group's channels of voxels t, t + 256, ...
// with K the group's first value (a shift against cancellation), converts them to
// (n, mean, M2) and the 256 threads merge in a fixed tree, so results repeat bit for bit.
__global__ __launch_bounds__(256) void gn_small_kernel(
    const f16* __restrict__ x0, int64_t p0, int C0, const f16* __restrict__ x1, int64_t p1,
    int C, int G, int64_t S, const float* __restrict__ gamma, const float* __restrict__ beta,
    float eps, float* __restrict__ affine) {
  __shared__ float red[12];
  const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int gs = C / G, c0 = g * gs;
  auto at = [&](int64_t v, int c) -> float {
    const int64_t vi = (int64_t)b * S + v;
    return (float)(c < C0 ? x0[vi * p0 + c] : x1[vi * p1 + (c - C0)]);
  };
  const float K = at(0, c0);
  float sum = 0.f, sq = 0.f;
  int64_t cnt = 0;
  const bool vec = gs % 8 == 0 && (c0 + gs <= C0 || c0 >= C0) && p0 % 8 == 0 && p1 % 8 == 0 &&
                   C0 % 8 == 0;
  for (int64_t v = t; v < S; v += 256) {
    if (vec) {
      const int64_t vi = (int64_t)b * S + v;
      const f16* row = c0 < C0 ? x0 + vi * p0 + c0 : x1 + vi * p1 + (c0 - C0);
      for (int c = 0; c < gs; c += 8) {
        const f16x8 h = *reinterpret_cast<const f16x8*>(row + c);
#pragma unroll
        for (int e = 0; e < 8; e++) { const float f = (float)h[e] - K; sum += f; sq += f * f; }
      }
    } else {
      for (int c = c0; c < c0 + gs; c++) { const float f = at(v, c) - K; sum += f; sq += f * f; }
    }
    cnt += gs;
  }
  Moments mt;
  {
    const float n = (float)cnt;
    const float m = n > 0.f ? sum / n : 0.f;
    mt = {n, K + m, n > 0.f ? fmaxf(sq - sum * m, 0.f) : 0.f};
  }
  const Moments tot = block_merge256(mt, red);
  const float mean = tot.mean;
  const float var = tot.n > 0.f ? tot.m2 / tot.n : 0.f;
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int c = c0 + t; c < c0 + gs; c += 256) {
    const float sc = gamma[c] * rstd;
    affine[((int64_t)b * C + c) * 2] = sc;
    affine[((int64_t)b * C + c) * 2 + 1] = beta[c] - sc * mean;
  }
}

// GroupNorm from moments a producer left (ldx_conv3d_stats): per channel pair and voxel
// block, (count, mean, M2) in [batch][chunks][pairs][3]. One workgroup per (group, batch
// item) merges its pairs' blocks -- pairs [0, c0 / 2) from m0, the rest from m1 (the
// decoder's concat) -- in a fixed order (thread t takes items t, t + 256, ... of the
// group's list, then a fixed tree), and writes the group's (scale, offset) pairs.
__global__ __launch_bounds__(256) void gn_moments_kernel(
    const float* __restrict__ m0, int64_t n0, int P0, const float* __restrict__ m1, int64_t n1, int P1,
    int C, int G, const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    float* __restrict__ affine) {
  __shared__ float red[12];
  const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int gs = C / G, u0 = g * gs / 2, nu = gs / 2;
  Moments m = {0.f, 0.f, 0.f};
  // The group's (pair, block) items in one list -- x0's pairs first, block-minor -- dealt
  // to the threads round-robin; four items' moments requested before any is merged.
  const int na = max(0, min(nu, P0 - u0));   // pairs of the group in x0
  const unsigned items0 = (unsigned)(na * n0), items = items0 + (unsigned)((nu - na) * n1);
  for (unsigned i0 = t; i0 < items; i0 += 4 * 256) {
    float3 r[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const unsigned i = i0 + e * 256;
      r[e] = make_float3(0.f, 0.f, 0.f);
      if (i < items0) {
        const unsigned u = u0 + i / (unsigned)n0, j = i % (unsigned)n0;
        r[e] = *reinterpret_cast<const float3*>(m0 + (((int64_t)b * n0 + j) * P0 + u) * 3);
      } else if (i < items) {
        const unsigned ii = i - items0;
        const unsigned u = u0 + na - P0 + ii / (unsigned)n1, j = ii % (unsigned)n1;
        r[e] = *reinterpret_cast<const float3*>(m1 + (((int64_t)b * n1 + j) * P1 + u) * 3);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (i0 + e * 256 < items) m = merge(m, Moments{r[e].x, r[e].y, r[e].z});
  }
  const Moments tot = block_merge256(m, red);
  const float mean = tot.mean;
  const float var = tot.n > 0.f ? tot.m2 / tot.n : 0.f;
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int c = g * gs + t; c < (g + 1) * gs; c += 256) {
    const float sc = gamma[c] * rstd;
    affine[((int64_t)b * C + c) * 2] = sc;
    affine[((int64_t)b * C + c) * 2 + 1] = beta[c] - sc * mean;
  }
}

// First pass of the moments merge for outputs with many moment blocks: workgroup (k, b)
// folds blocks [k per, min(n, (k + 1) per)) of every pair of m ([batch][n][P][3]) into
// block k of part ([batch][K][P][3]). Pairs go to consecutive threads (a block's pairs are
// one contiguous row: whole cache lines), S = 256 / np threads per pair take its blocks
// j0 + s, j0 + s + S, ... (at most GN_FOLD_ITEMS each, requested before any is merged),
// and the pair's S threads are merged in order. gn_moments_kernel then merges the K folded
// blocks: one workgroup per group reading its pairs out of every block would fetch a
// whole cache line per 12-byte block.
constexpr int GN_FOLD_ITEMS = 8;
__global__ __launch_bounds__(256) void gn_moments_fold_kernel(const float* __restrict__ m, int64_t n, int P,
                                                              int64_t per, float* __restrict__ part, int K) {
  __shared__ float sh[256 * 3];
  const int k = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int64_t j0 = (int64_t)k * per, j1 = j0 + per < n ? j0 + per : n;
  for (int p0 = 0; p0 < P; p0 += 256) {
    const int np = P - p0 < 256 ? P - p0 : 256;
    const int S = 256 / np, u = t % np, s = t / np;
    Moments acc = {0.f, 0.f, 0.f};
    if (s < S) {
      float3 r[GN_FOLD_ITEMS];
#pragma unroll
      for (int i = 0; i < GN_FOLD_ITEMS; i++) {
        const int64_t j = j0 + s + (int64_t)S * i;
        r[i] = j < j1 ? *reinterpret_cast<const float3*>(m + (((int64_t)b * n + j) * P + p0 + u) * 3)
                      : make_float3(0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < GN_FOLD_ITEMS; i++)
        if (j0 + s + (int64_t)S * i < j1) acc = merge(acc, Moments{r[i].x, r[i].y, r[i].z});
    }
    __syncthreads();   // the previous round's reads of sh are done
    sh[t * 3] = acc.n; sh[t * 3 + 1] = acc.mean; sh[t * 3 + 2] = acc.m2;
    __syncthreads();
    if (t < np) {
      Moments r = {sh[t * 3], sh[t * 3 + 1], sh[t * 3 + 2]};
      for (int s2 = 1; s2 < S; s2++) {
        const int q = s2 * np + t;
        r = merge(r, Moments{sh[q * 3], sh[q * 3 + 1], sh[q * 3 + 2]});
      }
      float* d = part + (((int64_t)b * K + k) * P + p0 + t) * 3;
      d[0] = r.n; d[1] = r.mean; d[2] = r.m2;
    }
  }
}

// Folded blocks of a moments tensor with n blocks of P pairs: K = 0 when one workgroup per
// group merges them directly (few items per group).
static int64_t gn_fold_blocks(int64_t n, int P, int nu) {
  if ((int64_t)nu * n <= 4096) return 0;
  const int np = P < 256 ? P : 256;
  const int64_t per = (int64_t)(256 / np) * GN_FOLD_ITEMS;
  return (n + per - 1) / per;
}

static int64_t gn_chunk(int64_t S, int batch) {
  // about 256 workgroups in pass 1 (one per CU), chunks of 64 .. 8192 voxels
  int64_t per = (S * batch + 255) / 256;
  if (per < 64) per = 64;
  if (per > 8192) per = 8192;
  return per;
}

// ------------------------------------------------------------- layer norm
// One wave per row; statistics in fp32 (two passes over registers).
template <int MAXV>
__global__ __launch_bounds__(256) void layer_norm_kernel(const f16* __restrict__ x, int64_t xp,
                                                         int64_t rows, int F,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float eps,
                                                         f16* __restrict__ y, int64_t yp) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const f16* xr = x + row * xp;
  float v[MAXV];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; i++) {
    const int c = lane + i * 64;
    v[i] = c < F ? (float)xr[c] : 0.f;
    s += v[i];
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  const float mean = s / F;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; i++) {
    const int c = lane + i * 64;
    const float d = c < F ? v[i] - mean : 0.f;
    q += d * d;
  }
  for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off);
  const float rstd = 1.0f / sqrtf(q / F + eps);
  f16* yr = y + row * yp;
#pragma unroll
  for (int i = 0; i < MAXV; i++) {
    const int c = lane + i * 64;
    if (c < F) yr[c] = (f16)((v[i] - mean) * rstd * gamma[c] + beta[c]);
  }
}

// --------------------------------------------------------------- small ops
__global__ void timestep_kernel(const int32_t* __restrict__ t, int B, int channels,
                                f16* __restrict__ out) {
  const int half = channels / 2;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * half) return;
  const int b = i / half, k = i % half;
  const float freq = expf(-9.21034037197618273607f * (float)k / (float)half);
  const float ph = (float)t[b] * freq;
  out[(int64_t)b * channels + k] = (f16)cosf(ph);
  out[(int64_t)b * channels + half + k] = (f16)sinf(ph);
}

__global__ void silu_kernel(const f16* __restrict__ x, int64_t n, f16* __restrict__ y) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = (float)x[i];
    y[i] = (f16)(v / (1.0f + expf(-v)));
  }
}


__global__ void copy_channels_kernel(const f16* __restrict__ src, int64_t sp, int so,
                                     f16* __restrict__ dst, int64_t dp, int dof, int64_t V, int C) {
  const int64_t n = V * C;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = i / C;
    const int c = (int)(i % C);
    dst[v * dp + dof + c] = src[v * sp + so + c];
  }
}

// Nearest 2x upsampling, NDHWC: out[2d+i, 2h+j, 2w+k] = in[d, h, w] (floor(i / 2) rule,
// src/lesiondiffusion_mlx/_spatial.py:12-26).
__global__ void upsample2_kernel(const f16* __restrict__ x, int64_t xp, int B, int D, int H, int W,
                                 int C, f16* __restrict__ y, int64_t yp) {
  const int64_t n = (int64_t)B * 8 * D * H * W * C;
  const int OH = 2 * H, OW = 2 * W, OD = 2 * D;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % C);
    int64_t r = i / C;
    const int ow = (int)(r % OW); r /= OW;
    const int oh = (int)(r % OH); r /= OH;
    const int od = (int)(r % OD);
    const int64_t b = r / OD;
    const int64_t src = ((b * D + od / 2) * H + oh / 2) * W + ow / 2;
    const int64_t dst = ((b * OD + od) * OH + oh) * (int64_t)OW + ow;
    y[dst * yp + c] = x[src * xp + c];
  }
}

__global__ void ddim_prepare_kernel(float* __restrict__ x, const float* __restrict__ cond,
                                    const float* __restrict__ mask, int64_t V, int C, int CC,
                                    f16* __restrict__ net, int64_t np) {
  for (int64_t v = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; v < V;
       v += (int64_t)gridDim.x * blockDim.x) {
    f16* row = net + v * np;
    if (mask) {
      const float m = mask[v];
      for (int c = 0; c < C; c++) {
        const float cv = cond[v * C + c];
        const float xm = x[v * C + c] * m + (1.0f - m) * cv;
        x[v * C + c] = xm;
        row[c] = (f16)xm;
        if (CC) row[C + c] = (f16)(cv * (1.0f - m));
      }
      row[C + CC] = (f16)m;
    } else {
      for (int c = 0; c < C; c++) row[c] = (f16)x[v * C + c];
      for (int c = 0; c < CC; c++) row[C + c] = (f16)cond[v * CC + c];
    }
  }
}

__global__ void ddim_update_kernel(float* __restrict__ x, const f16* __restrict__ net, int64_t np,
                                   const float* __restrict__ noise, const float* __restrict__ coef,
                                   const int32_t* __restrict__ step, int64_t V, int C) {
  const int si = step ? *step : 0;
  coef += 4 * si;
  noise += (int64_t)si * V * C;
  const float a = coef[0], prev = coef[1], sig = coef[2], s1m = coef[3];
  const float c_dir = sqrtf(1.0f - prev - sig * sig);
  const int64_t n = V * C;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t v = i / C;
    const int c = (int)(i % C);
    const float eps = (float)net[v * np + c];
    const float pred = (x[i] - s1m * eps) / sqrtf(a);
    x[i] = sqrtf(prev) * pred + c_dir * eps + sig * noise[i];
  }
}

}  // namespace ldx

using namespace ldx;

extern "C" const char* ldx_last_error(void) { return g_error.c_str(); }
extern "C" int ldx_abi_version(void) { return 12; }

extern "C" size_t ldx_packed_weight_elems(int32_t O, int32_t C, int32_t k, int32_t upsample) {
  if (O < 1 || C < 1 || (k != 1 && k != 3) || (upsample && k != 3)) return 0;
  const int taps = upsample ? 8 : k * k * k;
  return (size_t)(upsample ? 8 : 1) * ((O + 127) / 128 * 4) * taps * ((C + 63) / 64 * 4) * 512;
}

extern "C" int ldx_pack_weight(const void* weight, int32_t O, int32_t C, int32_t k, void* packed,
                               void* stream) {
  if (!weight || !packed) return fail("pack_weight: null pointer");
  if (O < 1 || C < 1 || (k != 1 && k != 3)) return fail("pack_weight: bad shape O=%d C=%d k=%d", O, C, k);
  const int taps = k * k * k;
  const int64_t n = (int64_t)ldx_packed_weight_elems(O, C, k, 0);
  hipLaunchKernelGGL(pack_weight_kernel, dim3(grid_cap(n, 256, 4096)), dim3(256), 0,
                     as_stream(stream), (const f16*)weight, O, C, taps, (f16*)packed);
  return check_launch("pack_weight");
}

extern "C" int ldx_pack_upsample_weight(const void* weight, int32_t O, int32_t C, int32_t dtype, void* packed,
                                        void* stream) {
  if (!weight || !packed) return fail("pack_upsample_weight: null pointer");
  if (O < 1 || C < 1) return fail("pack_upsample_weight: bad shape O=%d C=%d", O, C);
  if (dtype != LDX_DTYPE_F16 && dtype != LDX_DTYPE_BF16)
    return fail("pack_upsample_weight: dtype %d is not LDX_DTYPE_F16 or LDX_DTYPE_BF16", dtype);
  const int64_t n = (int64_t)ldx_packed_weight_elems(O, C, 3, 1);
  if (dtype == LDX_DTYPE_BF16)
    hipLaunchKernelGGL(pack_upsample_kernel<bf16>, dim3(grid_cap(n, 256, 4096)), dim3(256), 0,
                       as_stream(stream), (const bf16*)weight, O, C, (bf16*)packed);
  else
    hipLaunchKernelGGL(pack_upsample_kernel<f16>, dim3(grid_cap(n, 256, 4096)), dim3(256), 0,
                       as_stream(stream), (const f16*)weight, O, C, (f16*)packed);
  return check_launch("pack_upsample_weight");
}

extern "C" size_t ldx_group_norm_workspace_bytes(int32_t batch, int64_t voxels, int32_t channels,
                                                 int32_t groups) {
  if (batch < 1 || voxels < 1 || groups < 1) return 0;
  (void)channels;
  const int64_t chunk = gn_chunk(voxels, batch);
  const int64_t nchunks = (voxels + chunk - 1) / chunk;
  return (size_t)(batch * nchunks * groups * 3) * sizeof(float);
}

// Both GroupNorm entry points: statistics of x0 (and x1) into affine, the per-chunk partials
// of the two-pass path in `workspace` (every entry is written before it is read).
static int group_norm_affine_impl(const void* x0, int64_t p0, int32_t c0, const void* x1, int64_t p1,
                                  int32_t c1, int32_t batch, int64_t voxels, int32_t groups,
                                  const float* gamma, const float* beta, float eps, float* affine,
                                  void* workspace, hipStream_t st) {
  if (c1 > 0 && !x1) return fail("group_norm_affine: c1 > 0 but x1 is null");
  const int C = c0 + (c1 > 0 ? c1 : 0);
  if (batch < 1 || voxels < 1 || c0 < 1 || groups < 1 || C % groups)
    return fail("group_norm_affine: bad shape (batch %d voxels %lld C %d groups %d)", batch,
                (long long)voxels, C, groups);
  if (p0 < c0 || (c1 > 0 && p1 < c1)) return fail("group_norm_affine: pitch < channels");
  const bool vec = C % 8 == 0 && c0 % 8 == 0 && p0 % 8 == 0 && (c1 <= 0 || p1 % 8 == 0) &&
                   (uintptr_t)x0 % 16 == 0 && (c1 <= 0 || (uintptr_t)x1 % 16 == 0) && C / 8 <= 256;
  if (!vec && C > 256) return fail("group_norm_affine: unaligned input with more than 256 channels");
  if (C > 2048) return fail("group_norm_affine: more than 2048 channels");
  const int64_t chunk = gn_chunk(voxels, batch);
  const int64_t nchunks = (voxels + chunk - 1) / chunk;
  if (nchunks > 0x7fffffff || batch > 65535 || groups > 65535) return fail("group_norm_affine: too large");
  if (nchunks * batch <= 16) {
    // Few chunks: the one-launch per-group kernel.
    hipLaunchKernelGGL(gn_small_kernel, dim3(groups, batch), dim3(256), 0, st, (const f16*)x0, p0, c0,
                       (const f16*)x1, p1, C, groups, voxels, gamma, beta, eps, affine);
    return check_launch("group_norm_affine: small");
  }
  float* part = (float*)workspace;
  if (vec)
    hipLaunchKernelGGL(gn_partial_kernel<8>, dim3((unsigned)nchunks, batch), dim3(256), 0, st,
                       (const f16*)x0, p0, c0, (const f16*)x1, p1, C, groups, voxels, chunk, part,
                       (int)nchunks);
  else
    hipLaunchKernelGGL(gn_partial_kernel<1>, dim3((unsigned)nchunks, batch), dim3(256), 0, st,
                       (const f16*)x0, p0, c0, (const f16*)x1, p1, C, groups, voxels, chunk, part,
                       (int)nchunks);
  int rc = check_launch("group_norm_affine: partial");
  if (rc) return rc;
  hipLaunchKernelGGL(gn_finalize_kernel, dim3(groups, batch), dim3(256), 0, st, part, (int)nchunks, C,
                     groups, gamma, beta, eps, affine);
  return check_launch("group_norm_affine: finalize");
}

extern "C" int ldx_group_norm_affine(const void* x0, int64_t p0, int32_t c0, const void* x1,
                                     int64_t p1, int32_t c1, int32_t batch, int64_t voxels,
                                     int32_t groups, const float* gamma, const float* beta,
                                     float eps, float* affine, void* workspace, void* stream) {
  if (!x0 || !gamma || !beta || !affine || !workspace) return fail("group_norm_affine: null pointer");
  return group_norm_affine_impl(x0, p0, c0, x1, p1, c1, batch, voxels, groups, gamma, beta, eps, affine,
                                workspace, as_stream(stream));
}

// ------------------------------------------- GroupNorm without a caller workspace
// The partials of ldx_group_norm_affine_noalloc live in this file-scope device array, one
// copy per GPU for the life of the process. Host code never passes `gn_scratch` itself to
// a kernel (on the host it names a stand-in, not device memory): it passes the device
// address hipGetSymbolAddress returns, looked up once per device with that device current.
static __device__ __align__(256) float gn_scratch[LDX_GROUP_NORM_SCRATCH_BYTES / sizeof(float)];

static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[64];

// Device address of this device's gn_scratch (looked up on the first call per device).
static int scratch_for_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("group_norm_affine_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return LDX_EHIP;
  }
  if (dev < 0 || dev >= 64) return fail("group_norm_affine_noalloc: device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(gn_scratch));
    if (e != hipSuccess || !p) {
      set_error("group_norm_affine_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return LDX_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LDX_OK;
}

extern "C" int ldx_group_norm_affine_noalloc(const void* x0, int64_t p0, int32_t c0, const void* x1,
                                             int64_t p1, int32_t c1, int32_t batch, int64_t voxels,
                                             int32_t groups, const float* gamma, const float* beta,
                                             float eps, float* affine, void* stream) {
  if (!x0 || !gamma || !beta || !affine) return fail("group_norm_affine_noalloc: null pointer");
  const size_t need = ldx_group_norm_workspace_bytes(batch, voxels, c0 + (c1 > 0 ? c1 : 0), groups);
  if (need > LDX_GROUP_NORM_SCRATCH_BYTES)
    return fail("group_norm_affine_noalloc: %zu bytes of partials (batch %d, %lld voxels, %d groups) exceed "
                "the %d-byte device scratch; use ldx_group_norm_affine with a workspace",
                need, batch, (long long)voxels, groups, (int)LDX_GROUP_NORM_SCRATCH_BYTES);
  void* scratch = nullptr;
  const int rc = scratch_for_current_device(&scratch);
  if (rc) return rc;
  return group_norm_affine_impl(x0, p0, c0, x1, p1, c1, batch, voxels, groups, gamma, beta, eps, affine,
                                scratch, as_stream(stream));
}

extern "C" int ldx_group_norm_affine_moments(const float* m0, int64_t chunks0, int32_t c0, const float* m1,
                                             int64_t chunks1, int32_t c1, int32_t batch, int32_t groups,
                                             const float* gamma, const float* beta, float eps, float* affine,
                                             void* stream) {
  if (!m0 || !gamma || !beta || !affine) return fail("group_norm_affine_moments: null pointer");
  if (c1 > 0 && (!m1 || chunks1 < 1)) return fail("group_norm_affine_moments: c1 > 0 without moments");
  const int C = c0 + (c1 > 0 ? c1 : 0);
  if (batch < 1 || chunks0 < 1 || c0 < 2 || groups < 1 || C % groups || c0 % 2 || (c1 > 0 && c1 % 2) ||
      (C / groups) % 2)
    return fail("group_norm_affine_moments: bad shape (batch %d C %d (c0 %d) groups %d): moments are kept "
                "per channel pair, so c0, c1 and C / groups must be even", batch, C, c0, groups);
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(gn_moments_kernel, dim3(groups, batch), dim3(256), 0, st, m0, chunks0, c0 / 2,
                     c1 > 0 ? m1 : m0, c1 > 0 ? chunks1 : chunks0, c1 > 0 ? c1 / 2 : 1, C, groups, gamma, beta,
                     eps, affine);
  return check_launch("group_norm_affine_moments");
}

extern "C" size_t ldx_group_norm_moments_workspace_bytes(int64_t chunks0, int32_t c0, int64_t chunks1, int32_t c1,
                                                         int32_t batch, int32_t groups) {
  const int C = c0 + (c1 > 0 ? c1 : 0);
  if (batch < 1 || chunks0 < 1 || c0 < 2 || groups < 1 || C % groups || (C / groups) % 2) return 0;
  const int nu = C / groups / 2;
  const int64_t k0 = gn_fold_blocks(chunks0, c0 / 2, nu);
  const int64_t k1 = c1 > 0 ? gn_fold_blocks(chunks1, c1 / 2, nu) : 0;
  if (k0 == 0 && k1 == 0) return 0;
  return (size_t)batch * (size_t)(k0 * (c0 / 2) + k1 * (c1 > 0 ? c1 / 2 : 0)) * 3 * sizeof(float);
}

extern "C" int ldx_group_norm_affine_moments_ws(const float* m0, int64_t chunks0, int32_t c0, const float* m1,
                                                int64_t chunks1, int32_t c1, int32_t batch, int32_t groups,
                                                const float* gamma, const float* beta, float eps, float* affine,
                                                void* workspace, size_t workspace_bytes, void* stream) {
  const size_t need = ldx_group_norm_moments_workspace_bytes(chunks0, c0, chunks1, c1, batch, groups);
  if (need == 0)
    return ldx_group_norm_affine_moments(m0, chunks0, c0, m1, chunks1, c1, batch, groups, gamma, beta, eps,
                                         affine, stream);
  if (!m0 || !gamma || !beta || !affine || !workspace) return fail("group_norm_affine_moments: null pointer");
  if (c1 > 0 && (!m1 || chunks1 < 1)) return fail("group_norm_affine_moments: c1 > 0 without moments");
  if (workspace_bytes < need)
    return fail("group_norm_affine_moments: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (c0 % 2 || (c1 > 0 && c1 % 2)) return fail("group_norm_affine_moments: c0 and c1 must be even");
  const int C = c0 + (c1 > 0 ? c1 : 0), nu = C / groups / 2;
  hipStream_t st = as_stream(stream);
  float* part = (float*)workspace;
  // Each input's blocks folded (or taken as they are when few), then the per-group merge.
  const float* f[2] = {m0, c1 > 0 ? m1 : m0};
  int64_t nf[2] = {chunks0, c1 > 0 ? chunks1 : chunks0};
  const int64_t ns[2] = {chunks0, c1 > 0 ? chunks1 : 0};
  const int P[2] = {c0 / 2, c1 > 0 ? c1 / 2 : 1};
  for (int i = 0; i < (c1 > 0 ? 2 : 1); i++) {
    const int64_t K = gn_fold_blocks(ns[i], P[i], nu);
    if (K == 0) continue;
    if (K > 65535 || batch > 65535) return fail("group_norm_affine_moments: too many blocks");
    const int np = P[i] < 256 ? P[i] : 256;
    const int64_t per = (int64_t)(256 / np) * GN_FOLD_ITEMS;
    hipLaunchKernelGGL(gn_moments_fold_kernel, dim3((unsigned)K, batch), dim3(256), 0, st, f[i], ns[i], P[i], per,
                       part, (int)K);
    if (int rc = check_launch("group_norm_affine_moments: fold")) return rc;
    f[i] = part;
    nf[i] = K;
    part += (size_t)batch * K * P[i] * 3;
  }
  hipLaunchKernelGGL(gn_moments_kernel, dim3(groups, batch), dim3(256), 0, st, f[0], nf[0], P[0], f[1], nf[1],
                     P[1], C, groups, gamma, beta, eps, affine);
  return check_launch("group_norm_affine_moments");
}

extern "C" int ldx_layer_norm(const void* x, int64_t xp, int64_t rows, int32_t F, const float* gamma,
                              const float* beta, float eps, void* y, int64_t yp, void* stream) {
  if (!x || !y || !gamma || !beta) return fail("layer_norm: null pointer");
  if (rows < 1 || F < 1 || xp < F || yp < F) return fail("layer_norm: bad shape");
  if (F > 1024) return fail("layer_norm: features %d > 1024", F);
  const unsigned grid = (unsigned)((rows + 3) / 4);
  hipStream_t st = as_stream(stream);
  if (F <= 256)
    hipLaunchKernelGGL(layer_norm_kernel<4>, dim3(grid), dim3(256), 0, st, (const f16*)x, xp, rows, F,
                       gamma, beta, eps, (f16*)y, yp);
  else
    hipLaunchKernelGGL(layer_norm_kernel<16>, dim3(grid), dim3(256), 0, st, (const f16*)x, xp, rows, F,
                       gamma, beta, eps, (f16*)y, yp);
  return check_launch("layer_norm");
}

extern "C" int ldx_timestep_embedding(const int32_t* t, int32_t B, int32_t channels, void* out,
                                      void* stream) {
  if (!t || !out) return fail("timestep_embedding: null pointer");
  if (B < 1 || channels < 2 || channels % 2) return fail("timestep_embedding: bad shape");
  hipLaunchKernelGGL(timestep_kernel, dim3(blocks_for((int64_t)B * channels / 2, 256)), dim3(256), 0,
                     as_stream(stream), t, B, channels, (f16*)out);
  return check_launch("timestep_embedding");
}

extern "C" int ldx_silu(const void* x, int64_t n, void* y, void* stream) {
  if (!x || !y) return fail("silu: null pointer");
  if (n < 1) return fail("silu: empty");
  hipLaunchKernelGGL(silu_kernel, dim3(grid_cap(n, 256, 4096)), dim3(256), 0,
                     as_stream(stream), (const f16*)x, n, (f16*)y);
  return check_launch("silu");
}

extern "C" int ldx_copy_channels(const void* src, int64_t sp, int32_t so, void* dst, int64_t dp,
                                 int32_t dof, int64_t V, int32_t C, void* stream) {
  if (!src || !dst) return fail("copy_channels: null pointer");
  if (V < 1 || C < 1 || so < 0 || dof < 0 || so + C > sp || dof + C > dp)
    return fail("copy_channels: bad shape");
  const int64_t n = V * C;
  hipLaunchKernelGGL(copy_channels_kernel, dim3(grid_cap(n, 256, 8192)), dim3(256), 0,
                     as_stream(stream), (const f16*)src, sp, so, (f16*)dst, dp, dof, V, C);
  return check_launch("copy_channels");
}

extern "C" int ldx_upsample_nearest2(const void* x, int64_t xp, int32_t B, int32_t D, int32_t H,
                                     int32_t W, int32_t C, void* y, int64_t yp, void* stream) {
  if (!x || !y) return fail("upsample_nearest2: null pointer");
  if (B < 1 || D < 1 || H < 1 || W < 1 || C < 1 || xp < C || yp < C)
    return fail("upsample_nearest2: bad shape");
  const int64_t n = (int64_t)B * 8 * D * H * W * C;
  hipLaunchKernelGGL(upsample2_kernel, dim3(grid_cap(n, 256, 16384)), dim3(256), 0,
                     as_stream(stream), (const f16*)x, xp, B, D, H, W, C, (f16*)y, yp);
  return check_launch("upsample_nearest2");
}

extern "C" int ldx_ddim_prepare(float* x, const float* cond, const float* mask, int64_t V, int32_t C,
                                int32_t CC, void* net, int64_t np, void* stream) {
  if (!x || !cond || !net) return fail("ddim_prepare: null pointer");
  if (V < 1 || C < 1 || CC < 0) return fail("ddim_prepare: bad shape");
  if (mask && CC != 0 && CC != C) return fail("ddim_prepare: masked cond channels must be 0 or C");
  const int64_t need = mask ? (int64_t)C + CC + 1 : (int64_t)C + CC;
  if (np < need) return fail("ddim_prepare: pitch %lld < %lld", (long long)np, (long long)need);
  hipLaunchKernelGGL(ddim_prepare_kernel, dim3(grid_cap(V, 256, 4096)), dim3(256), 0,
                     as_stream(stream), x, cond, mask, V, C, CC, (f16*)net, np);
  return check_launch("ddim_prepare");
}

extern "C" int ldx_ddim_update(float* x, const void* net, int64_t np, const float* noise,
                               const float* coef, const int32_t* step, int64_t V, int32_t C,
                               void* stream) {
  if (!x || !net || !noise || !coef) return fail("ddim_update: null pointer");
  if (V < 1 || C < 1 || np < C) return fail("ddim_update: bad shape");
  const int64_t n = V * C;
  hipLaunchKernelGGL(ddim_update_kernel, dim3(grid_cap(n, 256, 4096)), dim3(256), 0,
                     as_stream(stream), x, (const f16*)net, np, noise, coef, step, V, C);
  return check_launch("ddim_update");
}

__global__ void ddim_timestep_kernel(const int32_t* step, const int32_t* table, int B, int32_t* out) {
  const int i = threadIdx.x;
  if (i < B) out[i] = table[*step];
}

__global__ void step_advance_kernel(int32_t* step) {
  if (threadIdx.x == 0) *step += 1;
}

extern "C" int ldx_ddim_timestep(const int32_t* step, const int32_t* table, int32_t B, int32_t* out,
                                 void* stream) {
  if (!step || !table || !out) return fail("ddim_timestep: null pointer");
  if (B < 1 || B > 1024) return fail("ddim_timestep: batch %d out of range", B);
  hipLaunchKernelGGL(ddim_timestep_kernel, dim3(1), dim3(1024), 0, as_stream(stream), step, table, B, out);
  return check_launch("ddim_timestep");
}

extern "C" int ldx_step_advance(int32_t* step, void* stream) {
  if (!step) return fail("step_advance: null pointer");
  hipLaunchKernelGGL(step_advance_kernel, dim3(1), dim3(64), 0, as_stream(stream), step);
  return check_launch("step_advance");
}
