// Shared device/host helpers for libldx (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "ldx.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace ldx {

// ---------------------------------------------------------------- errors (host)
void set_error(const char* fmt, ...);
int fail(const char* fmt, ...);  // set_error + return LDX_EINVAL
int check_launch(const char* what);  // hipGetLastError -> LDX_EHIP / LDX_OK

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------- device math
// SiLU in fp32 from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about 2 ulp of
// fp32, against ~15 instructions for an IEEE divide). Every caller rounds the result to
// fp16, 2^13 fp32 ulps apart. Large negative y gives rcp(inf) = 0, i.e. -0.
__device__ __forceinline__ float silu_f(float y) {
  return y * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y * -1.4426950408889634f));
}

// q = n / d for 0 <= n < 2^31 and 1 <= d < 2^31 from a host-made multiplier: with
// l = ceil(log2 d), s = 31 + l and m = ceil(2^s / d) < 2^32, n * m / 2^s exceeds n / d by
// less than n / 2^s <= 1 / d, which never reaches the next integer.
struct UDiv {
  unsigned m, s;
};
__device__ __forceinline__ int udiv(int n, UDiv d) {
  return (int)(((unsigned long long)(unsigned)n * d.m) >> d.s);
}
inline UDiv make_udiv(unsigned d) {
  unsigned l = 0;
  while ((1ull << l) < d) l++;
  const unsigned s = 31 + l;
  return UDiv{(unsigned)(((1ull << s) + d - 1) / d), s};
}

// One 16x16x32 f16 MFMA: D(16x16) += A(16x32) * B(32x16).
// Lane l: A row l%16, k = 8*(l/16)+e; B col l%16, k = 8*(l/16)+e;
// D col l%16, rows 4*(l/16)+r.
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__host__ __device__ __forceinline__ int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Raw buffer resource over `bytes` bytes from `base` (gfx9 descriptor word 3): loads at
// offsets past the extent return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// 16 bytes at byte offset off + soff (soff wave-uniform) of a buffer resource.
template <typename V8 = f16x8>
__device__ __forceinline__ V8 buffer_load16(__amdgpu_buffer_rsrc_t r, unsigned off, unsigned soff = 0) {
  return __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0));
}

// ---------------------------------------------------------------- LDS DMA

// Byte offset of an LDS pointer within the workgroup's LDS (the low 32 bits of its
// flat address).
__device__ __forceinline__ unsigned lds_offset(const void* p) { return (unsigned)(uintptr_t)p; }

// The two LDS-DMA helpers below write M0. M0 is a reserved register on gfx9: the
// compiler keeps no value of its own in it across code it did not generate (it sets M0
// right before each instruction of its own that reads it), and clang rejects M0 in a
// clobber list (a reserved register there is undefined behaviour), so none is given.
//
// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (global_load_lds_dwordx4). Issued as asm so that the compiler's wait insertion,
// which cannot tell these writes from the halo, does not drain all of them before
// every LDS read; completion is awaited explicitly with vmcnt_wait (+ a barrier when
// other waves read the data).
__device__ __forceinline__ void dma_b128(const void* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory");
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer resource (gfx9 descriptor: base, stride 0, num_records = bytes, the raw-buffer
// flags of make_rsrc) as four scalars, for the asm DMA below.
__device__ __forceinline__ i32x4 dma_rsrc(const void* base, unsigned bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(unsigned)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)(unsigned)(a >> 32) & 0xffff);
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane from a buffer (byte offset voff + soff; out of range reads zeros)
// straight into LDS at lds + 16 * lane. Asm for the same reason as dma_b128: completion
// is awaited with explicit vmcnt waits.
__device__ __forceinline__ void dma_buffer_b128(i32x4 rs, unsigned voff, unsigned soff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rs),
               "s"(soff), "s"(lds)
               : "memory");
}

// 16 bytes per lane from a buffer (byte offset voff + soff; out of range reads zeros) into
// registers, by asm: the compiler's wait insertion does not see it (and so drains nothing
// on its account). The caller awaits it with vmcnt_wait and then passes the value through
// pin_value before its first use.
template <typename V8 = f16x8>
__device__ __forceinline__ V8 buffer_load16_asm(i32x4 rs, unsigned voff, unsigned soff = 0) {
  V8 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rs), "s"(soff) : "memory");
  return v;
}
// Orders every later use of v after this point (after the wait that made it valid).
template <typename T>
__device__ __forceinline__ void pin_value(T& v) {
  asm volatile("" : "+v"(v));
}

// Reads one word of every 64-byte line of a kernel's argument block in one batch of
// scalar loads, awaited together at kernel entry. Argument reads the compiler places after
// branches on earlier arguments then hit the scalar cache; left alone, each new line is a
// miss awaited on its own (up to a dozen round trips in series before the first request).
template <typename P>
__device__ __forceinline__ void touch_args(const P& p) {
  const int* w = reinterpret_cast<const int*>(&p);
  constexpr int N = (int)((sizeof(P) + 63) / 64);
  static_assert(N <= 8, "argument block above 512 bytes");
  const unsigned g = gridDim.x;   // the dispatch's own line (hidden arguments)
  if constexpr (N == 1) asm volatile("" :: "s"(g), "s"(w[0]));
  if constexpr (N == 2) asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]));
  if constexpr (N == 3) asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]), "s"(w[32]));
  if constexpr (N == 4) asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]), "s"(w[32]), "s"(w[48]));
  if constexpr (N == 5) asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]), "s"(w[32]), "s"(w[48]), "s"(w[64]));
  if constexpr (N == 6)
    asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]), "s"(w[32]), "s"(w[48]), "s"(w[64]), "s"(w[80]));
  if constexpr (N == 7)
    asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]), "s"(w[32]), "s"(w[48]), "s"(w[64]), "s"(w[80]),
                 "s"(w[96]));
  if constexpr (N == 8)
    asm volatile("" :: "s"(g), "s"(w[0]), "s"(w[16]), "s"(w[32]), "s"(w[48]), "s"(w[64]), "s"(w[80]),
                 "s"(w[96]), "s"(w[112]));
}

// (count, mean, M2) of a set of values, merged pairwise (Chan et al.): no cancellation.
struct Moments { float n, mean, m2; };

__device__ __forceinline__ Moments merge(Moments a, Moments b) {
  const float n = a.n + b.n;
  if (n == 0.0f) return a;
  const float d = b.mean - a.mean;
  const float fb = b.n / n;
  return {n, a.mean + d * fb, a.m2 + b.m2 + d * d * a.n * fb};
}

// merge with the weight b.n / n from the hardware reciprocal (within 1 ulp; no IEEE
// division sequence) -- for the short epilogue folds of a brick's partial moments.
__device__ __forceinline__ Moments merge_rcp(Moments a, Moments b) {
  const float n = a.n + b.n;
  if (n == 0.0f) return a;
  const float d = b.mean - a.mean;
  const float fb = b.n * __builtin_amdgcn_rcpf(n);
  return {n, a.mean + d * fb, a.m2 + b.m2 + d * d * a.n * fb};
}

// Fold of N (2, 4 or 8) partial moments e[0..N-1] held at stride `stride` floats from q:
// all loaded first, then merged as a fixed balanced tree ((0, 1), (2, 3)), ((4, 5), (6, 7)).
template <int N>
__device__ __forceinline__ Moments fold_moments(const float* q, int stride) {
  static_assert(N == 2 || N == 4 || N == 8, "2, 4 or 8 partial moments");
  Moments e[N];
#pragma unroll
  for (int i = 0; i < N; i++) e[i] = Moments{q[i * stride], q[i * stride + 1], q[i * stride + 2]};
#pragma unroll
  for (int w = 1; w < N; w *= 2)
#pragma unroll
    for (int i = 0; i < N; i += 2 * w) e[i] = merge_rcp(e[i], e[i + w]);
  return e[0];
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ Moments merge_dpp(Moments m) {
  return merge(m, Moments{dpp_f<CTRL>(m.n), dpp_f<CTRL>(m.mean), dpp_f<CTRL>(m.m2)});
}
// Lane l merges its moments with those of the lane one row (permlane16) or one half
// (permlane32) away: each swap of v with itself gives a lane its own value and its partner's.
__device__ __forceinline__ Moments merge_swap16(Moments m) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_int(m.n), __float_as_int(m.n), false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_int(m.mean), __float_as_int(m.mean), false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(__float_as_int(m.m2), __float_as_int(m.m2), false, false);
  return merge(Moments{__int_as_float(a[0]), __int_as_float(b[0]), __int_as_float(c[0])},
               Moments{__int_as_float(a[1]), __int_as_float(b[1]), __int_as_float(c[1])});
}
__device__ __forceinline__ Moments merge_swap32(Moments m) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_int(m.n), __float_as_int(m.n), false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_int(m.mean), __float_as_int(m.mean), false, false);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_int(m.m2), __float_as_int(m.m2), false, false);
  return merge(Moments{__int_as_float(a[0]), __int_as_float(b[0]), __int_as_float(c[0])},
               Moments{__int_as_float(a[1]), __int_as_float(b[1]), __int_as_float(c[1])});
}

// Merge of a workgroup's 256 per-thread moments in a fixed order: in each wave, lane l
// merges with the lanes 8, 4, 2, 1 places round its 16-lane row (DPP row rotations), then
// across rows and halves (v_permlane16/32_swap); lane 0 holds the wave's total. Then the
// four waves' totals in wave order through LDS (red: 12 floats). Every thread returns the
// same total; results repeat bit for bit.
__device__ __forceinline__ Moments block_merge256(Moments m, float* red) {
  m = merge_dpp<0x128>(m);   // row_ror:8
  m = merge_dpp<0x124>(m);   // row_ror:4
  m = merge_dpp<0x122>(m);   // row_ror:2
  m = merge_dpp<0x121>(m);   // row_ror:1
  m = merge_swap16(m);
  m = merge_swap32(m);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { red[w * 3] = m.n; red[w * 3 + 1] = m.mean; red[w * 3 + 2] = m.m2; }
  __syncthreads();
  Moments r = {red[0], red[1], red[2]};
#pragma unroll
  for (int i = 1; i < 4; i++) r = merge(r, Moments{red[3 * i], red[3 * i + 1], red[3 * i + 2]});
  return r;
}

// Sum of v over the lanes that share lane % L (L = 4 or 8): rotations by 8 (and 4) inside
// each 16-lane row (DPP), then v_permlane16_swap and v_permlane32_swap of v with itself
// (each lane gets its own value and its partner's one row / half away). No LDS traffic;
// the additions run in a fixed order on every lane.
template <int L>
__device__ __forceinline__ float lane_group_sum(float v) {
  static_assert(L == 4 || L == 8, "lane groups of 4 or 8");
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));  // row_ror:8
  if constexpr (L == 4)
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false));  // row_ror:4
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  v = __int_as_float(r16[0]) + __int_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r32[0]) + __int_as_float(r32[1]);
}

// GroupNorm partial moments of one wave's block of finished outputs, per channel pair.
// Each lane holds 8 consecutive channels (4 pairs) of NI voxels (ok[i]: the voxel is an
// output); the lanes holding the same channels are L apart (L = 4 or 8).
// Two passes over the values -- the pair's mean, then its squared deviations -- each
// summed over those lanes (lane_group_sum: every lane ends with the same sums), so the
// block's (count, mean, M2) carry no cancellation. With `store`, the lane writes its four
// pairs' moments as 12 consecutive floats at dst (16-byte aligned).
template <int NI, int L, typename V8>
__device__ __forceinline__ void pair_moments(const V8 (&v)[NI], const bool (&ok)[NI], float* dst,
                                             bool store) {
  float cnt = 0.f, s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NI; i++)
    if (ok[i]) {
      cnt += 2.f;
#pragma unroll
      for (int q = 0; q < 4; q++) s[q] += (float)v[i][2 * q] + (float)v[i][2 * q + 1];
    }
  cnt = lane_group_sum<L>(cnt);
#pragma unroll
  for (int q = 0; q < 4; q++) s[q] = lane_group_sum<L>(s[q]);
  float mean[4], m2[4];
  const float inv = cnt > 0.f ? 1.0f / cnt : 0.f;   // one division for the four pairs
#pragma unroll
  for (int q = 0; q < 4; q++) { mean[q] = s[q] * inv; m2[q] = 0.f; }
#pragma unroll
  for (int i = 0; i < NI; i++)
    if (ok[i]) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float d0 = (float)v[i][2 * q] - mean[q], d1 = (float)v[i][2 * q + 1] - mean[q];
        m2[q] += d0 * d0 + d1 * d1;
      }
    }
#pragma unroll
  for (int q = 0; q < 4; q++) m2[q] = lane_group_sum<L>(m2[q]);
  if (store) {
    f32x4* d = reinterpret_cast<f32x4*>(dst);
    d[0] = (f32x4){cnt, mean[0], m2[0], cnt};
    d[1] = (f32x4){mean[1], m2[1], cnt, mean[2]};
    d[2] = (f32x4){m2[2], cnt, mean[3], m2[3]};
  }
}

// Wait until at most N vector-memory loads of this wave are outstanding.
// (s_waitcnt immediate for gfx9: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt
// 11:8 left at their no-wait maxima.)
template <int N>
__device__ __forceinline__ void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

}  // namespace ldx
