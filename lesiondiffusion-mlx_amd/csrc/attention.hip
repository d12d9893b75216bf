// Flash attention on gfx950 MFMA (v_mfma_f32_16x16x32_f16), fp16 in/out, fp32
// scores, online softmax and accumulation.
//
// Orientation: each wave computes S^T = K Q^T (rows = keys, columns = its 16*FQ
// queries) so a lane's score registers -- four consecutive keys of one query -- are
// already the B-operand layout of O^T = V^T P^T: probabilities never leave
// registers, and every per-query quantity (running max, alpha, partial row sum)
// is lane-local. Q^T fragments stay in registers for the whole key loop; K tiles
// (row-major) and V^T tiles (transposed on the LDS store) stream through LDS, the
// next tile's global loads in flight while the current one is computed.
//
// Reference semantics: flash_attention_half (src/lesiondiffusion_mlx/_attention_half.py:
// 23-114): scores scaled by scale*log2(e) in fp32 (:70-72), exp2 online softmax
// (:74-92), probabilities rounded to fp16 for the PV product (:86), output
// half(o / l) (:105-113); plus the additive mask of mx.fast.scaled_dot_product_attention
// (mlx_model.py:843-847, 860-862).

#include "common.h"

namespace ldx {

struct AttnParams {
  int B, H, L, LK;
  const f16* q; int64_t qs0, qs1, qs2;
  const f16* k; int64_t ks0, ks1, ks2;
  const f16* v; int64_t vs0, vs1, vs2;
  f16* o; int64_t os0, os1, os2;
  float c;  // scale * log2(e)
  const float* mask; int64_t ms0, ms1, ms2, ms3;
};

template <int D, int FQ, int KB>
__global__ __launch_bounds__(256) void attention_kernel(AttnParams p) {
  constexpr int DK = D >= 32 ? D / 32 : 1;   // K-steps of the QK^T product
  constexpr int DB = D / 16;                 // 16-row blocks of O^T
  constexpr int KR = KB / 16;                // 16-key row blocks of S^T
  constexpr int KJ = KB / 32;                // 32-key K-steps of the PV product
  constexpr int KP = D + 8;                  // K tile pitch (halves)
  constexpr int VP = KB + 8;                 // V^T tile pitch (halves)
  constexpr int CPR = D / 8;                 // 16-byte chunks per key row
  constexpr int NCH = KB * CPR;              // chunks per tile
  constexpr int CPT = (NCH + 255) / 256;     // chunks per thread
  __shared__ __attribute__((aligned(16))) f16 Ks[KB * KP];
  __shared__ __attribute__((aligned(16))) f16 Vt[D * VP];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, col = lane & 15;
  const int h = blockIdx.y, b = blockIdx.z;
  const int q0 = blockIdx.x * (64 * FQ) + wave * 16 * FQ;
  const f16* qb = p.q + (int64_t)b * p.qs0 + (int64_t)h * p.qs2;
  const f16* kb_ = p.k + (int64_t)b * p.ks0 + (int64_t)h * p.ks2;
  const f16* vb = p.v + (int64_t)b * p.vs0 + (int64_t)h * p.vs2;

  // Q^T fragments: lane holds query q0+fq*16+col, dims dk*32 + 8g .. +7.
  f16x8 qf[FQ][DK];
#pragma unroll
  for (int fq = 0; fq < FQ; fq++) {
    const int qi = min(q0 + fq * 16 + col, p.L - 1);
#pragma unroll
    for (int dk = 0; dk < DK; dk++) {
      const int d = dk * 32 + 8 * g;
      f16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (d < D) v = *reinterpret_cast<const f16x8*>(qb + (int64_t)qi * p.qs1 + d);
      qf[fq][dk] = v;
    }
  }

  f32x4 o[DB][FQ];
#pragma unroll
  for (int i = 0; i < DB; i++)
#pragma unroll
    for (int j = 0; j < FQ; j++) o[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m[FQ], l[FQ];
#pragma unroll
  for (int j = 0; j < FQ; j++) { m[j] = -INFINITY; l[j] = 0.f; }

  const float* mrow[FQ];
#pragma unroll
  for (int fq = 0; fq < FQ; fq++) {
    const int qi = min(q0 + fq * 16 + col, p.L - 1);
    mrow[fq] = p.mask ? p.mask + (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)qi * p.ms2 : nullptr;
  }

  // Register staging of the next tile.
  f16x8 kst[CPT], vst[CPT];
  auto load_tile = [&](int kbase) {
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int ch = threadIdx.x + i * 256;
      const int key = ch / CPR, dc = ch - key * CPR;
      f16x8 kv = {0, 0, 0, 0, 0, 0, 0, 0}, vv = kv;
      if (ch < NCH && kbase + key < p.LK) {
        kv = *reinterpret_cast<const f16x8*>(kb_ + (int64_t)(kbase + key) * p.ks1 + dc * 8);
        vv = *reinterpret_cast<const f16x8*>(vb + (int64_t)(kbase + key) * p.vs1 + dc * 8);
      }
      kst[i] = kv; vst[i] = vv;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < CPT; i++) {
      const int ch = threadIdx.x + i * 256;
      if (ch < NCH) {
        const int key = ch / CPR, dc = ch - key * CPR;
        *reinterpret_cast<f16x8*>(Ks + key * KP + dc * 8) = kst[i];
#pragma unroll
        for (int e = 0; e < 8; e++) Vt[(dc * 8 + e) * VP + key] = vst[i][e];
      }
    }
  };

  const int nblk = (p.LK + KB - 1) / KB;
  load_tile(0);
  for (int blk = 0; blk < nblk; blk++) {
    const int kbase = blk * KB;
    __syncthreads();
    store_tile();
    __syncthreads();
    if (blk + 1 < nblk) load_tile(kbase + KB);

    // S^T = K Q^T
    f32x4 s[KR][FQ];
#pragma unroll
    for (int kr = 0; kr < KR; kr++)
#pragma unroll
      for (int fq = 0; fq < FQ; fq++) s[kr][fq] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kr = 0; kr < KR; kr++) {
#pragma unroll
      for (int dk = 0; dk < DK; dk++) {
        const int d = dk * 32 + 8 * g;
        f16x8 kf = {0, 0, 0, 0, 0, 0, 0, 0};
        if (d < D) kf = *reinterpret_cast<const f16x8*>(Ks + (kr * 16 + col) * KP + d);
#pragma unroll
        for (int fq = 0; fq < FQ; fq++) s[kr][fq] = mfma16(kf, qf[fq][dk], s[kr][fq]);
      }
    }

    // Online softmax per query column.
    f16x8 pf[KJ][FQ];
#pragma unroll
    for (int fq = 0; fq < FQ; fq++) {
      float top = -INFINITY;
#pragma unroll
      for (int kr = 0; kr < KR; kr++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int key = kbase + kr * 16 + 4 * g + r;
          float t = s[kr][fq][r] * p.c;
          if (mrow[fq] && key < p.LK) t += mrow[fq][(int64_t)key * p.ms3] * 1.44269504088896341f;
          if (key >= p.LK) t = -INFINITY;
          s[kr][fq][r] = t;
          top = fmaxf(top, t);
        }
      top = fmaxf(top, __shfl_xor(top, 16));
      top = fmaxf(top, __shfl_xor(top, 32));
      const float mn = fmaxf(m[fq], top);
      // A row with every key so far removed keeps m = -inf: contribute nothing.
      const float base = mn == -INFINITY ? 0.f : mn;
      const float alpha = exp2f(m[fq] - base);
      m[fq] = mn;
      float sum = 0.f;
#pragma unroll
      for (int kr = 0; kr < KR; kr++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float e = exp2f(s[kr][fq][r] - base);
          sum += e;
          pf[kr >> 1][fq][(kr & 1) * 4 + r] = (f16)e;
        }
      l[fq] = l[fq] * alpha + sum;
#pragma unroll
      for (int db = 0; db < DB; db++) o[db][fq] *= alpha;
    }

    // O^T += V^T P^T
#pragma unroll
    for (int kj = 0; kj < KJ; kj++) {
#pragma unroll
      for (int db = 0; db < DB; db++) {
        const f16* vr = Vt + (db * 16 + col) * VP + kj * 32 + 4 * g;
        const f16x4 lo = *reinterpret_cast<const f16x4*>(vr);
        const f16x4 hi = *reinterpret_cast<const f16x4*>(vr + 16);
        const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
        for (int fq = 0; fq < FQ; fq++) o[db][fq] = mfma16(vf, pf[kj][fq], o[db][fq]);
      }
    }
  }

  // Normalise and store: lane holds dims db*16 + 4g + r of query q0+fq*16+col.
  f16* ob = p.o + (int64_t)b * p.os0 + (int64_t)h * p.os2;
#pragma unroll
  for (int fq = 0; fq < FQ; fq++) {
    float tot = l[fq];
    tot += __shfl_xor(tot, 16);
    tot += __shfl_xor(tot, 32);
    const int qi = q0 + fq * 16 + col;
    if (qi >= p.L) continue;
    const float inv = tot > 0.f ? 1.0f / tot : 0.f;
    f16* orow = ob + (int64_t)qi * p.os1;
#pragma unroll
    for (int db = 0; db < DB; db++) {
      f16x4 out;
#pragma unroll
      for (int r = 0; r < 4; r++) out[r] = (f16)(o[db][fq][r] * inv);
      *reinterpret_cast<f16x4*>(orow + db * 16 + 4 * g) = out;
    }
  }
}

template <int D, int FQ, int KB>
static int launch_attn(const AttnParams& p, hipStream_t st) {
  dim3 grid((unsigned)((p.L + 64 * FQ - 1) / (64 * FQ)), (unsigned)p.H, (unsigned)p.B);
  hipLaunchKernelGGL((attention_kernel<D, FQ, KB>), grid, dim3(256), 0, st, p);
  return check_launch("attention");
}

}  // namespace ldx

using namespace ldx;

extern "C" int ldx_attention(const ldx_attention_args* a, void* stream) {
  if (!a) return fail("attention: null args");
  if (a->batch < 1 || a->heads < 1 || a->q_len < 1 || a->kv_len < 1)
    return fail("attention: empty shape (B %d H %d L %d LK %d)", a->batch, a->heads, a->q_len, a->kv_len);
  const int D = a->head_dim;
  if (D != 16 && D != 32 && D != 64 && D != 128 && D != 256)
    return fail("attention: head_dim %d not in {16, 32, 64, 128, 256}", D);
  if (!a->q || !a->k || !a->v || !a->o) return fail("attention: null tensor");
  if (a->batch > 65535 || a->heads > 65535) return fail("attention: batch/heads too large");
  const int64_t* ss[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
  const void* ps[4] = {a->q, a->k, a->v, a->o};
  for (int i = 0; i < 4; i++) {
    for (int j = 0; j < 3; j++)
      if (ss[i][j] % 8 != 0) return fail("attention: strides must be multiples of 8 elements");
    if ((uintptr_t)ps[i] % 16 != 0) return fail("attention: tensors must be 16-byte aligned");
  }
  AttnParams p{};
  p.B = a->batch; p.H = a->heads; p.L = a->q_len; p.LK = a->kv_len;
  p.q = (const f16*)a->q; p.qs0 = a->q_stride[0]; p.qs1 = a->q_stride[1]; p.qs2 = a->q_stride[2];
  p.k = (const f16*)a->k; p.ks0 = a->k_stride[0]; p.ks1 = a->k_stride[1]; p.ks2 = a->k_stride[2];
  p.v = (const f16*)a->v; p.vs0 = a->v_stride[0]; p.vs1 = a->v_stride[1]; p.vs2 = a->v_stride[2];
  p.o = (f16*)a->o; p.os0 = a->o_stride[0]; p.os1 = a->o_stride[1]; p.os2 = a->o_stride[2];
  p.c = a->scale * 1.44269504088896341f;
  p.mask = a->mask;
  p.ms0 = a->mask_stride[0]; p.ms1 = a->mask_stride[1]; p.ms2 = a->mask_stride[2]; p.ms3 = a->mask_stride[3];
  hipStream_t st = as_stream(stream);
  switch (D) {
    case 16: return launch_attn<16, 1, 64>(p, st);
    case 32: return launch_attn<32, 1, 64>(p, st);
    case 64: return launch_attn<64, 1, 64>(p, st);
    case 128: return launch_attn<128, 1, 32>(p, st);
    default: return launch_attn<256, 1, 32>(p, st);
  }
}
