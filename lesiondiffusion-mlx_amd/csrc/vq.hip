// Nearest-codebook search of the VQ autoencoder's four-channel latent (the native search of
// src/lesiondiffusion_mlx/_vq.py:12-82 and VqAutoencoder.quantize, mlx_model.py:742-803).
//
// Distance of latent vector z to code c, with the reference's rounding points in the element
// type T (fp16 or fp32): dot = fma chain of the four products in fp32 (first product plain,
// then three fmas); summed = T(|z|^2 + |c|^2); doubled = T(2 * T(dot)); distance =
// T(summed - doubled). The squared norms are the T-rounded squares summed in fp32 and
// rounded to T once. Selection: the lowest index whose distance is NaN if any is NaN, else
// the lowest index of the smallest distance (argmin's order) -- a function of the distance
// list alone, so any scan order gives the same index.
//
// One lane owns one latent vector and scans every code in increasing order; the codebook
// moves through LDS in chunks, read by all lanes of a wave at the same address (a
// broadcast). Integer/index results are bit-exact; nothing is accumulated across lanes.

#include "common.h"

#include <cmath>

// Every rounding point above is explicit; no multiply-add may be fused behind the code's back
// (the reference compiles its search with contraction off as well).
#pragma clang fp contract(off)

namespace ldx {

constexpr int VQ_THREADS = 256;
constexpr int VQ_CHUNK = 2048;   // codes staged per round: 2048 x (4 + 1) x 4 B = 40 KB

// fp32 squared norm of one four-vector as the reference forms it: each square rounded to T,
// the four summed in fp32 in index order, the sum rounded to T once.
template <typename T>
__device__ __forceinline__ T squared_norm4(const T* v) {
  float s = (float)(T)(v[0] * v[0]);
  s += (float)(T)(v[1] * v[1]);
  s += (float)(T)(v[2] * v[2]);
  s += (float)(T)(v[3] * v[3]);
  return (T)s;
}

template <typename T>
__global__ __launch_bounds__(VQ_THREADS) void vq_norms4_kernel(const T* __restrict__ x, int64_t n,
                                                               T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * VQ_THREADS + threadIdx.x;
  if (i >= n) return;
  T v[4];
#pragma unroll
  for (int c = 0; c < 4; c++) v[c] = x[i * 4 + c];
  out[i] = squared_norm4<T>(v);
}

// Replace (best, best_index) by (d, code) under the selection rule, for codes visited in
// increasing order: the first code is always taken; then a NaN only while best is not NaN,
// and otherwise only a strictly smaller distance (an equal one keeps the lower index).
template <typename T>
__device__ __forceinline__ void vq_take(T d, int code, T& best, int& best_index) {
  const bool dn = d != d, bn = best != best;
  if (best_index < 0 || (dn && !bn) || (!bn && !dn && d < best)) {
    best = d;
    best_index = code;
  }
}

template <typename T>
__global__ __launch_bounds__(VQ_THREADS) void vq_nearest4_kernel(
    const T* __restrict__ z, const T* __restrict__ z_norm, const T* __restrict__ codebook,
    const T* __restrict__ cb_norm, int64_t P, int E, int32_t* __restrict__ indices, T* __restrict__ quantized) {
  __shared__ float4 cb[VQ_CHUNK];
  __shared__ T cbn[VQ_CHUNK];
  const int64_t pos = (int64_t)blockIdx.x * VQ_THREADS + threadIdx.x;
  const bool live = pos < P;
  float zf[4] = {0.f, 0.f, 0.f, 0.f};
  T zt[4] = {};
  T zn = (T)0.f;
  if (live) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      zt[c] = z[pos * 4 + c];
      zf[c] = (float)zt[c];
    }
    zn = z_norm ? z_norm[pos] : squared_norm4<T>(zt);
  }
  T best = (T)0.f;
  int best_index = -1;   // no code taken yet
  for (int base = 0; base < E; base += VQ_CHUNK) {
    const int n = min(VQ_CHUNK, E - base);
    __syncthreads();   // the previous chunk is no longer read
    for (int i = threadIdx.x; i < n; i += VQ_THREADS) {
      const T* e = codebook + (int64_t)(base + i) * 4;
      cb[i] = make_float4((float)e[0], (float)e[1], (float)e[2], (float)e[3]);
      cbn[i] = cb_norm[base + i];
    }
    __syncthreads();
    if (!live) continue;
    for (int i = 0; i < n; i++) {
      const float4 e = cb[i];
      float dot = zf[0] * e.x;
      dot = __builtin_fmaf(zf[1], e.y, dot);
      dot = __builtin_fmaf(zf[2], e.z, dot);
      dot = __builtin_fmaf(zf[3], e.w, dot);
      const T summed = (T)(zn + cbn[i]);
      const T doubled = (T)((T)2.f * (T)dot);
      vq_take<T>((T)(summed - doubled), base + i, best, best_index);
    }
  }
  if (!live) return;
  indices[pos] = best_index;
  if (quantized) {
    const T* e = codebook + (int64_t)best_index * 4;
    // The straight-through form z + (selected - z), each operation rounded to T
    // (mlx_model.py:788-789).
#pragma unroll
    for (int c = 0; c < 4; c++) quantized[pos * 4 + c] = (T)(zt[c] + (T)(e[c] - zt[c]));
  }
}

}  // namespace ldx

using namespace ldx;

extern "C" int ldx_vq_squared_norms4(const void* x, int64_t n, int32_t dtype, void* out, void* stream) {
  if (!x || !out) return fail("vq_squared_norms4: null pointer");
  if (n < 1) return fail("vq_squared_norms4: n = %lld < 1", (long long)n);
  const unsigned grid = (unsigned)((n + VQ_THREADS - 1) / VQ_THREADS);
  hipStream_t st = as_stream(stream);
  if (dtype == LDX_DTYPE_F16)
    hipLaunchKernelGGL(vq_norms4_kernel<f16>, dim3(grid), dim3(VQ_THREADS), 0, st, (const f16*)x, n, (f16*)out);
  else if (dtype == LDX_DTYPE_F32)
    hipLaunchKernelGGL(vq_norms4_kernel<float>, dim3(grid), dim3(VQ_THREADS), 0, st, (const float*)x, n,
                       (float*)out);
  else
    return fail("vq_squared_norms4: dtype %d is not LDX_DTYPE_F16 or LDX_DTYPE_F32", dtype);
  return check_launch("vq_squared_norms4");
}

extern "C" int ldx_vq_nearest4(const void* z, const void* z_norm, const void* codebook, const void* codebook_norm,
                               int64_t positions, int32_t entries, int32_t dtype, int32_t* indices,
                               void* quantized, void* stream) {
  if (!z || !codebook || !codebook_norm || !indices) return fail("vq_nearest4: null pointer");
  if (positions < 1 || entries < 1)
    return fail("vq_nearest4: empty input (%lld positions, %d codes)", (long long)positions, entries);
  if (positions > ((int64_t)1 << 31)) return fail("vq_nearest4: more than 2^31 positions");
  const unsigned grid = (unsigned)((positions + VQ_THREADS - 1) / VQ_THREADS);
  hipStream_t st = as_stream(stream);
  if (dtype == LDX_DTYPE_F16)
    hipLaunchKernelGGL(vq_nearest4_kernel<f16>, dim3(grid), dim3(VQ_THREADS), 0, st, (const f16*)z,
                       (const f16*)z_norm, (const f16*)codebook, (const f16*)codebook_norm, positions, entries,
                       indices, (f16*)quantized);
  else if (dtype == LDX_DTYPE_F32)
    hipLaunchKernelGGL(vq_nearest4_kernel<float>, dim3(grid), dim3(VQ_THREADS), 0, st, (const float*)z,
                       (const float*)z_norm, (const float*)codebook, (const float*)codebook_norm, positions,
                       entries, indices, (float*)quantized);
  else
    return fail("vq_nearest4: dtype %d is not LDX_DTYPE_F16 or LDX_DTYPE_F32", dtype);
  return check_launch("vq_nearest4");
}
