// Token-row chains of the spatial transformer in one launch: dense layers and LayerNorms
// applied row by row to a 32-token tile kept in LDS, so that the tile never returns to
// memory between them (the transformer block of mlx_model.py:522-552).
//
// One workgroup owns 32 token rows (of every batch item's token sequence laid end to
// end) and runs, in order:
//
//   [x' = half(x * affine[b, c, 0] + affine[b, c, 1])]      GroupNorm affine (optional)
//   y1  = half(W1 x' + b1 [+ res1])                        G1 (stored if y1 is set)
//   z   = half(LN(y1) * gamma + beta)                      LayerNorm
//   h   = act(half(W2 z + b2))                             G2
//   [y3 = half(W3 h + b3 + y1)]                            G3 (optional)
//   [out = half(W4 y3 + b4 + res4)]                        G4 (optional)
//
// and stores the last stage's output. The transformer block uses it three times:
// proj_in -> norm1 -> attn1 q/k/v; attn1 to_out (+ x) -> norm2 -> attn2 to_q; attn2 to_out
// (+ x) -> norm3 -> ff.net.0 (GELU) -> ff.net.2 (+ x) -> proj_out (+ the block input).
// Every stage rounds where the separate dense launches round (one rounding of the fp32
// sum with bias and residual; GELU of the rounded value), so the fused chain and the
// separate launches agree to the order of fp32 summation.
//
// GEMM stages: rows = output channels (A = the packed weight, 1 KB fragments in MFMA lane
// order, loaded from global memory through a buffer resource), columns = the tile's 32
// tokens (B = 16-byte reads of the LDS tile, rows padded by 16 bytes). Each of the 8 waves
// owns every 8th 32-channel output tile and sums its whole reduction in one
// v_mfma_f32_32x32x16 accumulator; its tiles' weight fragments are one stream with up to
// 16 fragments in flight, across tile boundaries. A workgroup streams every weight of its
// chain, so the number of loads in flight per CU, not the MFMA rate, sets the time.
// Biases and residual rows are staged in LDS first, so no global load sits between the
// weight loads. The LayerNorm: 16 lanes per row, two passes (mean, then squared
// deviations) in fp32.

#include "elem.h"

#include <cmath>

namespace ldx {
namespace LDX_ELEM_NS {

constexpr int TC_ROWS = 32;
constexpr int TC_NW = 8;            // waves per workgroup (two per SIMD)
constexpr int TC_THREADS = 64 * TC_NW;

struct ChainGemm {
  const E* w;          // packed fragments (ldx_pack_weight, ksize 1)
  const float* bias;   // fp32 (O), or null
  int O, NKC;          // output channels; 16-channel fragments per packed row
  int act;             // LDX_ACT_*
  int bias_lds;        // float offset of this GEMM's bias in the LDS bias table
};

struct ChainParams {
  int rows, T, C;                    // token rows (batch * T), tokens per batch item, width of x
  const E* x; int64_t xp;
  const float* affine;               // (batch, C, 2) or null
  const E* res1; int64_t res1p;      // residual of G1, or null
  E* y1; int64_t y1p;                // G1's output, or null
  const float* ln_g; const float* ln_b; float ln_eps;
  ChainGemm g1, g2, g3, g4;
  int has_g3, has_g4;
  const E* res4; int64_t res4p;
  E* out; int64_t outp;
  int pitch_c, pitch_h;              // LDS row pitches (halves) of C-wide and G2-wide tiles
  int nbias;                         // floats of the LDS bias table
};

__device__ __forceinline__ float gelu_erf_tc(float v) { return v * (1.0f + erff(v * 0.70710678118654752f)) * 0.5f; }

// One GEMM stage: the tile (32 tokens x g.O) from the LDS tile `in` (32 x K, pitch ip). A
// wave owns output tiles wave, wave + NW, ...; their weight fragments form one stream in
// groups of PD (PD divides K / 16), held in two register sets that alternate: while one
// group's MFMAs run, the other set's loads are in flight, and a set is reloaded with the
// group after next as soon as its MFMAs are issued -- 2 PD fragments in flight, across tile
// boundaries. The group count is padded to even with loads past the buffer's end (zeros,
// no fetch) whose MFMAs land in an accumulator that is dropped. The epilogue adds the bias
// (LDS table `bl`) and the residual (LDS rows `rl`, pitch rlp, when given), rounds, applies
// the activation and writes the LDS tile `ol` (pitch olp; may be rl).
template <int PD>
__device__ __forceinline__ void chain_gemm(const ChainGemm& g, int K, const E* in, int ip, const float* bl,
                                           const E* rl, int rlp, E* ol, int olp, int lane, int wave) {
  const int col = lane & 31, hf = lane >> 5;
  const int nk = K / 16;
  const int ntiles = g.O / 32;
  if (wave >= ntiles) return;
  const int ntw = (ntiles - wave + TC_NW - 1) / TC_NW;   // this wave's output tiles
  const int F = ntw * nk;                                  // its weight fragments, in order
  const int G = F / PD;                                    // groups
  const unsigned wbytes = (unsigned)((size_t)((g.O + 127) / 128 * 4) * g.NKC * 1024);
  const auto rw = make_rsrc(g.w, wbytes);
  const unsigned aoff = (unsigned)lane * 16u;
  const E* brow = in + col * ip + hf * 8;
  auto goff = [&](int gi) {   // byte offset of group gi's first fragment; past the stream: out of range
    const int f = gi * PD, t = f / nk;
    return gi < G ? (unsigned)((wave + TC_NW * t) * g.NKC + (f - t * nk)) * 1024u : wbytes;
  };
  E8 ra[2][PD];
#pragma unroll
  for (int s2 = 0; s2 < 2; s2++) {
    const unsigned o = goff(s2);
#pragma unroll
    for (int j = 0; j < PD; j++) ra[s2][j] = buffer_load16<E8>(rw, aoff, o + j * 1024u);
  }
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; e++) acc[e] = 0.f;
  auto epilogue = [&](int t) {
    // Lane (hf, col) holds token col, channels ob * 32 + 8 i + 4 hf + r (acc[4 i + r]).
    const int ob = wave + TC_NW * t;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int oc = ob * 32 + 8 * i + 4 * hf;
      const f32x4 bias = *reinterpret_cast<const f32x4*>(bl + oc);
      float res[4] = {0.f, 0.f, 0.f, 0.f};
      if (rl) {
        const E4 r4 = *reinterpret_cast<const E4*>(rl + col * rlp + oc);
#pragma unroll
        for (int r = 0; r < 4; r++) res[r] = (float)r4[r];
      }
      E4 v;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const E h = (E)((acc[4 * i + r] + bias[r]) * 1.0f + res[r]);
        v[r] = g.act == LDX_ACT_GELU ? (E)gelu_erf_tc((float)h) : (g.act == LDX_ACT_SILU ? (E)silu_f((float)h) : h);
      }
      *reinterpret_cast<E4*>(ol + col * olp + oc) = v;
    }
#pragma unroll
    for (int e = 0; e < 16; e++) acc[e] = 0.f;
  };
  for (int g0 = 0; g0 < G; g0 += 2) {
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
      const int gi = g0 + s2;
      const int f = gi * PD, t = f / nk, k0 = f - t * nk;
      const E* bk = brow + (gi < G ? k0 : 0) * 16;   // a padding group reads valid rows
      const unsigned on = goff(gi + 2);
#pragma unroll
      for (int j = 0; j < PD; j++) {
        const E8 b = *reinterpret_cast<const E8*>(bk + j * 16);
        acc = mfma_e(ra[s2][j], b, acc);
        ra[s2][j] = buffer_load16<E8>(rw, aoff, on + j * 1024u);
      }
      if (gi < G && k0 + PD == nk) epilogue(t);
    }
  }
}

// PD: 16, 8, 4, 2 or 1 fragments per group, the largest that divides the k-steps.
__device__ __forceinline__ void chain_gemm_any(const ChainGemm& g, int K, const E* in, int ip, const float* bl,
                                               const E* rl, int rlp, E* ol, int olp, int lane, int wave) {
  const int nk = K / 16;
  if (nk % 16 == 0) chain_gemm<16>(g, K, in, ip, bl, rl, rlp, ol, olp, lane, wave);
  else if (nk % 8 == 0) chain_gemm<8>(g, K, in, ip, bl, rl, rlp, ol, olp, lane, wave);
  else if (nk % 4 == 0) chain_gemm<4>(g, K, in, ip, bl, rl, rlp, ol, olp, lane, wave);
  else chain_gemm<2>(g, K, in, ip, bl, rl, rlp, ol, olp, lane, wave);
}

// The tile's valid rows (cols channels) from LDS rows (pitch lp) to global rows (pitch gp).
__device__ __forceinline__ void store_rows(E* dst, int64_t gp, const E* src, int lp, int cols, int row0, int nrows) {
  const int cpr = cols / 4;
  for (int i = threadIdx.x; i < nrows * cpr; i += TC_THREADS) {
    const int r = i / cpr, c4 = (i - r * cpr) * 4;
    *reinterpret_cast<E4*>(dst + (int64_t)(row0 + r) * gp + c4) = *reinterpret_cast<const E4*>(src + r * lp + c4);
  }
}

// 32 rows of `cols` channels from global rows (pitch gp) into LDS rows (pitch lp), zero
// past the valid rows.
__device__ __forceinline__ void stage_rows(E* dst, int lp, const E* src, int64_t gp, int cols, int row0, int nrows) {
  const int cpr = cols / 4;
  for (int i = threadIdx.x; i < TC_ROWS * cpr; i += TC_THREADS) {
    const int r = i / cpr, c4 = (i - r * cpr) * 4;
    E4 v = (E4){};
    if (r < nrows) v = *reinterpret_cast<const E4*>(src + (int64_t)(row0 + r) * gp + c4);
    *reinterpret_cast<E4*>(dst + r * lp + c4) = v;
  }
}

__global__ __launch_bounds__(TC_THREADS) void token_chain_kernel(ChainParams p) {
  extern __shared__ __attribute__((aligned(16))) E tsm[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = blockIdx.x * TC_ROWS;
  const int nrows = min(TC_ROWS, p.rows - row0);
  const int pc = p.pitch_c, ph = p.pitch_h;
  E* X = tsm;                          // x' ; then LN(y1) ; then G3's output
  E* Y1 = X + TC_ROWS * pc;            // res1, then G1's output in place (G3's residual); then res4
  E* H = Y1 + TC_ROWS * pc;            // G2's output; G4's
  float* BL = reinterpret_cast<float*>(H + TC_ROWS * ph);   // the biases

  for (int i = threadIdx.x; i < p.nbias; i += TC_THREADS) BL[i] = 0.f;
  __syncthreads();
  for (const ChainGemm* g : {&p.g1, &p.g2, &p.g3, &p.g4})
    if (g->bias)
      for (int i = threadIdx.x; i < g->O; i += TC_THREADS) BL[g->bias_lds + i] = g->bias[i];
  // x (16-byte chunks) -> LDS, through the GroupNorm affine when given.
  const int cpr = p.C / 8;
  for (int i = threadIdx.x; i < TC_ROWS * cpr; i += TC_THREADS) {
    const int r = i / cpr, c8 = (i - r * cpr) * 8;
    E8 v = (E8){};
    if (r < nrows) {
      v = *reinterpret_cast<const E8*>(p.x + (int64_t)(row0 + r) * p.xp + c8);
      if (p.affine) {
        const float* a = p.affine + ((int64_t)((row0 + r) / p.T) * p.C + c8) * 2;
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (E)((float)v[e] * a[2 * e] + a[2 * e + 1]);
      }
    }
    *reinterpret_cast<E8*>(X + r * pc + c8) = v;
  }
  if (p.res1) stage_rows(Y1, pc, p.res1, p.res1p, p.g1.O, row0, nrows);
  __syncthreads();
  chain_gemm_any(p.g1, p.C, X, pc, BL + p.g1.bias_lds, p.res1 ? Y1 : nullptr, pc, Y1, pc, lane, wave);
  __syncthreads();
  if (p.y1) store_rows(p.y1, p.y1p, Y1, pc, p.g1.O, row0, nrows);

  // LayerNorm of y1 -> X: 16 lanes per row, each wave 4 rows at once.
  {
    const int C1 = p.g1.O;
    const int r = wave * 4 + (lane >> 4), l16 = lane & 15;
    const E* yr = Y1 + r * pc;
    float s = 0.f;
    for (int c = l16 * 8; c < C1; c += 128) {
      const E8 v = *reinterpret_cast<const E8*>(yr + c);
#pragma unroll
      for (int e = 0; e < 8; e++) s += (float)v[e];
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 8);
    const float mean = s / (float)C1;
    float q = 0.f;
    for (int c = l16 * 8; c < C1; c += 128) {
      const E8 v = *reinterpret_cast<const E8*>(yr + c);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = (float)v[e] - mean;
        q += d * d;
      }
    }
    q += __shfl_xor(q, 1);
    q += __shfl_xor(q, 2);
    q += __shfl_xor(q, 4);
    q += __shfl_xor(q, 8);
    const float rstd = 1.0f / sqrtf(q / (float)C1 + p.ln_eps);
    for (int c = l16 * 8; c < C1; c += 128) {
      const E8 v = *reinterpret_cast<const E8*>(yr + c);
      const f32x4 g0 = *reinterpret_cast<const f32x4*>(p.ln_g + c), g1 = *reinterpret_cast<const f32x4*>(p.ln_g + c + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(p.ln_b + c), b1 = *reinterpret_cast<const f32x4*>(p.ln_b + c + 4);
      E8 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        o[e] = (E)(((float)v[e] - mean) * rstd * g0[e] + b0[e]);
        o[e + 4] = (E)(((float)v[e + 4] - mean) * rstd * g1[e] + b1[e]);
      }
      *reinterpret_cast<E8*>(X + r * pc + c) = o;
    }
  }
  __syncthreads();
  // G2 -> H; then G3 (+ y1) -> X; then res4 -> Y1 and G4 (+ res4) -> H. The last GEMM's
  // tile goes to global memory from LDS.
  chain_gemm_any(p.g2, p.g1.O, X, pc, BL + p.g2.bias_lds, nullptr, 0, H, ph, lane, wave);
  __syncthreads();
  if (!p.has_g3) {
    store_rows(p.out, p.outp, H, ph, p.g2.O, row0, nrows);
    return;
  }
  chain_gemm_any(p.g3, p.g2.O, H, ph, BL + p.g3.bias_lds, Y1, pc, X, pc, lane, wave);
  __syncthreads();
  if (!p.has_g4) {
    store_rows(p.out, p.outp, X, pc, p.g3.O, row0, nrows);
    return;
  }
  if (p.res4) stage_rows(Y1, pc, p.res4, p.res4p, p.g4.O, row0, nrows);
  __syncthreads();
  chain_gemm_any(p.g4, p.g3.O, X, pc, BL + p.g4.bias_lds, p.res4 ? Y1 : nullptr, pc, H, ph, lane, wave);
  __syncthreads();
  store_rows(p.out, p.outp, H, ph, p.g4.O, row0, nrows);
}

static ChainGemm chain_gemm_of(const ldx_chain_gemm& g, int in_c) {
  return ChainGemm{(const E*)g.weight, g.bias, g.out_c, (in_c + 63) / 64 * 4, g.act, 0};
}

// Validate and launch; the LDS footprint is 32 rows x (2 C-wide tiles + the G2 tile).
int token_chain_entry(const ldx_token_chain_args* a, void* stream) {
  if (!a) return fail("token_chain: null arguments");
  if (!a->x || !a->out || !a->ln_gamma || !a->ln_beta || !a->g1.weight || !a->g2.weight)
    return fail("token_chain: null x, out, LayerNorm or G1/G2 weight");
  if (a->rows < 1 || a->tokens < 1 || a->channels < 1)
    return fail("token_chain: empty input (%d rows, %d tokens, %d channels)", a->rows, a->tokens, a->channels);
  const int C = a->channels, C1 = a->g1.out_c, C2 = a->g2.out_c;
  const int C3 = a->has_g3 ? a->g3.out_c : 0, C4 = a->has_g4 ? a->g4.out_c : 0;
  auto bad = [](int c) { return c < 32 || c % 32 != 0; };
  if (bad(C) || bad(C1) || bad(C2) || (a->has_g3 && bad(C3)) || (a->has_g4 && bad(C4)))
    return fail("token_chain: channel counts must be positive multiples of 32 (%d, %d, %d, %d, %d)", C, C1, C2, C3, C4);
  if (a->has_g4 && !a->has_g3) return fail("token_chain: G4 needs G3");
  if ((a->has_g3 && (!a->g3.weight || C3 != C1)) || (a->has_g4 && (!a->g4.weight || C4 > C)))
    return fail("token_chain: G3 must map back to G1's width and G4 to at most x's");
  if (a->has_g4 && C3 > C) return fail("token_chain: G3's output must fit the x tile");
  if (C1 > C) return fail("token_chain: G1 wider than its input tile");
  for (int act : {a->g1.act, a->g2.act, a->g3.act, a->g4.act})
    if (act != LDX_ACT_NONE && act != LDX_ACT_GELU && act != LDX_ACT_SILU)
      return fail("token_chain: unknown act %d", act);
  if (a->x_pitch < C || (a->res1 && a->res1_pitch < C1) || (a->y1 && a->y1_pitch < C1) ||
      (a->res4 && a->res4_pitch < C4) || a->out_pitch < (a->has_g4 ? C4 : a->has_g3 ? C3 : C2))
    return fail("token_chain: pitch smaller than its row");
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  auto a8 = [](const void* p) { return ((uintptr_t)p & 7) == 0; };
  if (!a16(a->x) || a->x_pitch % 8 || !a8(a->out) || a->out_pitch % 4 || (a->res1 && (!a8(a->res1) || a->res1_pitch % 4)) ||
      (a->y1 && (!a8(a->y1) || a->y1_pitch % 4)) || (a->res4 && (!a8(a->res4) || a->res4_pitch % 4)) ||
      !a16(a->ln_gamma) || !a16(a->ln_beta) || (a->affine && !a8(a->affine)))
    return fail("token_chain: rows must be 16-byte (x) / 8-byte aligned");
  for (const ldx_chain_gemm* g : {&a->g1, &a->g2, &a->g3, &a->g4})
    if (g->bias && !a16(g->bias)) return fail("token_chain: bias must be 16-byte aligned");
  ChainParams p{};
  p.rows = a->rows; p.T = a->tokens; p.C = C;
  p.x = (const E*)a->x; p.xp = a->x_pitch;
  p.affine = a->affine;
  p.res1 = (const E*)a->res1; p.res1p = a->res1_pitch;
  p.y1 = (E*)a->y1; p.y1p = a->y1_pitch;
  p.ln_g = a->ln_gamma; p.ln_b = a->ln_beta; p.ln_eps = a->ln_eps;
  p.g1 = chain_gemm_of(a->g1, C);
  p.g2 = chain_gemm_of(a->g2, C1);
  p.g3 = a->has_g3 ? chain_gemm_of(a->g3, C2) : ChainGemm{};
  p.g4 = a->has_g4 ? chain_gemm_of(a->g4, C3) : ChainGemm{};
  p.has_g3 = a->has_g3 ? 1 : 0; p.has_g4 = a->has_g4 ? 1 : 0;
  p.res4 = (const E*)a->res4; p.res4p = a->res4_pitch;
  p.out = (E*)a->out; p.outp = a->out_pitch;
  p.pitch_c = C + 8;
  p.pitch_h = (C2 > C4 ? C2 : C4) + 8;
  p.g1.bias_lds = 0;
  p.g2.bias_lds = C1;
  p.g3.bias_lds = C1 + C2;
  p.g4.bias_lds = C1 + C2 + C3;
  p.nbias = C1 + C2 + C3 + C4;
  const size_t lds = (size_t)TC_ROWS * (2 * p.pitch_c + p.pitch_h) * sizeof(E) + (size_t)p.nbias * sizeof(float);
  if (lds > 160 * 1024) return fail("token_chain: %zu bytes of LDS tiles exceed 160 KiB", lds);
  auto kern = token_chain_kernel;
  if (lds > 65536 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return check_launch("token_chain: set LDS size");
  const unsigned grid = (unsigned)((a->rows + TC_ROWS - 1) / TC_ROWS);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(TC_THREADS), lds, as_stream(stream), p);
  return check_launch("token_chain");
}

}  // namespace LDX_ELEM_NS
}  // namespace ldx

#if !defined(LDX_ELEM_BF16)
namespace ldx {
namespace bf16_path {
int token_chain_entry(const ldx_token_chain_args* a, void* stream);
}
}  // namespace ldx

extern "C" int ldx_token_chain(const ldx_token_chain_args* a, void* stream) {
  if (a && a->dtype == LDX_DTYPE_BF16) return ldx::bf16_path::token_chain_entry(a, stream);
  if (a && a->dtype != LDX_DTYPE_F16)
    return ldx::fail("token_chain: dtype %d is not LDX_DTYPE_F16 or LDX_DTYPE_BF16", a->dtype);
  return ldx::f16_path::token_chain_entry(a, stream);
}
#endif
