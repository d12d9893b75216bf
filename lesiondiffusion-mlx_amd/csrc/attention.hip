// Flash attention on gfx950 MFMA (v_mfma_f32_32x32x16_f16), fp16 in/out, fp32
// scores, online softmax and accumulation.
//
// Orientation: a wave computes S^T = K Q^T for a 32-key block and its 32 queries (rows
// = keys, columns = queries), so the lane's score registers -- 16 of the block's keys
// for one query -- are already the B operand of O^T = V^T P^T: probabilities never
// leave registers, and the running max / rescale / partial row sum of a query are
// lane-local (its other 16 keys sit in lane ^ 32, one lane swap away). Q^T stays in
// registers. K and V tiles (rows = keys, as they lie in memory) stream through LDS with
// 16-byte stores, loaded one or two blocks ahead through buffer resources; the V^T
// operand is read back with gfx950's transposing LDS read (ds_read_b64_tr_b16), so V is
// never transposed in memory. Masking and key bounds are applied only on blocks that
// need them. Row sums add the fp32 probabilities before their rounding, as the
// reference's total does; fp32 adds issue beside the MFMAs, v_dot2 does not (measured).
//
// SPLIT = 1: a workgroup's 4 waves own 4 x 32 queries and share each K/V tile.
// SPLIT = 4 / 8: the waves own the same 32 queries and take interleaved key blocks with
// private tiles; their (max, sum, O) states merge through LDS at the end -- more waves
// for short sequences (1,600 tokens x 8 heads is only 400 query blocks).
// attention_pipe_kernel (long key sequences, head width 32 or 64): the four-way split
// with tiles moved global->LDS by DMA and the S^T MFMAs of the next block issued ahead
// of the current block's softmax. Its exponent base moves only when a block raises a
// query's maximum by more than 8 (log2 units), so probabilities lie in [0, 2^8] rather
// than [0, 1]: the same fp16 relative rounding, with the accumulator rescale skipped on
// most blocks.
//
// Reference semantics: flash_attention_half (src/lesiondiffusion_mlx/_attention_half.py:
// 23-114): scores scaled by scale*log2(e) in fp32 (:70-72), exp2 online softmax
// (:74-92), probabilities rounded to fp16 for the PV product (:86), output half(o / l)
// (:105-113); plus the additive mask of mx.fast.scaled_dot_product_attention
// (mlx_model.py:843-847, 860-862).

#include "elem.h"

#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace ldx {
namespace LDX_ELEM_NS {

struct AttnParams {
  int B, H, L, LK;
  const E* q; int64_t qs0, qs1, qs2;
  const E* k; int64_t ks0, ks1, ks2;
  const E* v; int64_t vs0, vs1, vs2;
  E* o; int64_t os0, os1, os2;
  float c;  // scale * log2(e)
  const float* mask; int64_t ms0, ms1, ms2, ms3;
  // Split wide-head schedule (attention_wide_kernel): part != null gives each query tile
  // pmax workgroups, one per equal piece of its key blocks; each leaves its partial
  // state in part ([tile][piece]) for attention_wide_merge_kernel.
  float* part; int pmax;
  size_t part_bytes;   // host only: the caller's workspace size
  // Key shares of attention_pipe_kernel: the key blocks repeat in periods of kper; share w
  // takes kcnt[w] of each period, at the positions held in the bytes of kslot[w] (in
  // increasing order), knit[w] blocks in all.
  int kper, kcnt[8], knit[8];
  unsigned kslot[8][4];
};

__device__ __forceinline__ f32x16 mfma32x(E8 a, E8 b, f32x16 c) {
  return mfma_e(a, b, c);
}



// acc *= a with tied operands, so the branch that rescales leaves the accumulator in
// the registers the other branch keeps it in (no copies across the loop). The compiler
// does not see the asm's register reads and writes for MFMA hazards, so it waits out
// the longest MFMA-result latency first (18 wait states for a 32x32 result read by
// VALU) and the VALU-write-to-MFMA-read gap after.
__device__ __forceinline__ void scale_in_place(f32x16& acc, float a) {
  asm volatile(
      "s_nop 7\n s_nop 7\n s_nop 3\n"
      "v_mul_f32 %0, %16, %0\n v_mul_f32 %1, %16, %1\n v_mul_f32 %2, %16, %2\n v_mul_f32 %3, %16, %3\n"
      "v_mul_f32 %4, %16, %4\n v_mul_f32 %5, %16, %5\n v_mul_f32 %6, %16, %6\n v_mul_f32 %7, %16, %7\n"
      "v_mul_f32 %8, %16, %8\n v_mul_f32 %9, %16, %9\n v_mul_f32 %10, %16, %10\n v_mul_f32 %11, %16, %11\n"
      "v_mul_f32 %12, %16, %12\n v_mul_f32 %13, %16, %13\n v_mul_f32 %14, %16, %14\n v_mul_f32 %15, %16, %15\n"
      "s_nop 4"
      : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(acc[4]), "+v"(acc[5]), "+v"(acc[6]),
        "+v"(acc[7]), "+v"(acc[8]), "+v"(acc[9]), "+v"(acc[10]), "+v"(acc[11]), "+v"(acc[12]), "+v"(acc[13]),
        "+v"(acc[14]), "+v"(acc[15])
      : "v"(a));
}

// Max / sum of a value over lanes l and l ^ 32. v_permlane32_swap of v with itself
// leaves each lane holding its own value and its partner's, one in each result.
__device__ __forceinline__ float halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
// Maximum of a lane's 16 scores: a tree of three-input maxima.
__device__ __forceinline__ float max16(const f32x16& s) {
  const float t0 = fmaxf(fmaxf(s[0], s[1]), s[2]), t1 = fmaxf(fmaxf(s[3], s[4]), s[5]);
  const float t2 = fmaxf(fmaxf(s[6], s[7]), s[8]), t3 = fmaxf(fmaxf(s[9], s[10]), s[11]);
  const float t4 = fmaxf(fmaxf(s[12], s[13]), s[14]);
  return fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, s[15]));
}
__device__ __forceinline__ float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Pointer into this workgroup's LDS as the address-space-3 pointer that the transposing
// read takes.
__device__ __forceinline__ lds_s16x4* lds_v4(const E* p) {
  return (lds_s16x4*)((__attribute__((address_space(3))) char*)(p));
}

// The keys of a 32-key block are stored in LDS K-tile rows permuted by pi (bits 2 and 3
// of the row swapped; pi is its own inverse). MFMA row r of S^T then holds key pi(r), so
// a lane's score register e is key 16 * (e / 8) + 8 * hf + e % 8: the eight
// probabilities of one PV k-step are eight consecutive keys, and the matching V^T
// operand is one 16-byte read.
__device__ __forceinline__ int key_row(int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); }

// Waves per SIMD >= 2 keeps the register budget at 256 VGPRs, so the MFMA accumulators
// live in ordinary VGPRs (no accumulator-register copies around the softmax); the
// eight-wave key split asks for four (128 VGPRs) so that two of its workgroups share a
// CU.
template <int D, int SPLIT>
struct AttnOcc { static constexpr int waves = SPLIT == 8 ? 4 : (D <= 64 ? 2 : 1); };

// SPLIT = 1: a workgroup's 4 waves own 4 x 32 queries and share each K/V tile (double-
// buffered in LDS, one barrier per tile). SPLIT = 4 or 8: SPLIT waves own the same 32
// queries and take interleaved key blocks with private tiles; their (max, sum, O)
// states merge through LDS at the end.
template <int D, int SPLIT>
__global__ __launch_bounds__(SPLIT == 1 ? 256 : 64 * SPLIT)
__attribute__((amdgpu_waves_per_eu(AttnOcc<D, SPLIT>::waves, 8)))
void attention_kernel(AttnParams p) {
  touch_args(p);
  constexpr int NT = SPLIT == 1 ? 256 : 64 * SPLIT;
  constexpr int KB = 32;                      // keys per block
  constexpr int DK = D >= 16 ? D / 16 : 1;    // 16-wide k-steps of Q K^T
  constexpr int DB = D >= 32 ? D / 32 : 1;    // 32-row blocks of O^T
  constexpr int KP = D + 8;                   // K tile pitch (halves)
  constexpr int KG = D / 8;                   // 16-byte chunks per key row
  constexpr int KCH = KB * KG;                // 16-byte chunks of a K tile
  constexpr int TPT = SPLIT == 1 ? 256 : 64;  // threads loading one tile
  constexpr int KPT = (KCH + TPT - 1) / TPT;
  constexpr bool KALL = KCH % TPT == 0;
  constexpr int TILE = 2 * KB * KP;           // halves per (K, V) tile pair, rows = keys
  constexpr int NTILE = SPLIT == 1 ? 2 : SPLIT;
  constexpr int MERGE = SPLIT == 1 ? 0 : SPLIT * (D * 32 + 64);  // floats for the merge
  constexpr int LDS_H = NTILE * TILE > MERGE * 2 ? NTILE * TILE : MERGE * 2;
  // (+64 halves: for D = 16 the transposing V reads of the unused O^T rows 16..31 run
  // up to 8 halves past the last tile.)
  __shared__ __attribute__((aligned(16))) E smem[LDS_H + 64];

  // The wave index is uniform; readfirstlane lets the compiler keep block indices,
  // tile bases and loop conditions in scalar registers.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hf = lane >> 5, col = lane & 31;
  // Workgroup -> (query block, head, batch item), query blocks fastest, with the range of
  // workgroups each XCD receives (they are dealt to the 8 XCDs round-robin) contiguous:
  // the query blocks of one head then share its K and V in one L2.
  constexpr int QPW = SPLIT == 1 ? 128 : 32;   // queries per workgroup
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
  }
  const int nqb = (p.L + QPW - 1) / QPW;
  const int qblk = wg % nqb, h = (wg / nqb) % p.H, b = wg / nqb / p.H;
  const int q0 = SPLIT == 1 ? qblk * 128 + wave * 32 : qblk * 32;
  E* Ks = smem + (SPLIT == 1 ? 0 : wave) * TILE;  // SPLIT > 1: this wave's tile
  const int ltid = SPLIT == 1 ? threadIdx.x : lane;

  const E* qb = p.q + (int64_t)b * p.qs0 + (int64_t)h * p.qs2;
  const E* kb_ = p.k + (int64_t)b * p.ks0 + (int64_t)h * p.ks2;
  const E* vb_ = p.v + (int64_t)b * p.vs0 + (int64_t)h * p.vs2;

  // Q^T fragments: lane holds query q0 + col, dims 16*dk + 8*hf .. +7.
  const int qi = min(q0 + col, p.L - 1);
  E8 qf[DK];
#pragma unroll
  for (int dk = 0; dk < DK; dk++) {
    const int d = dk * 16 + 8 * hf;
    E8 v = {0, 0, 0, 0, 0, 0, 0, 0};
    if (d < D) v = *reinterpret_cast<const E8*>(qb + (int64_t)qi * p.qs1 + d);
    qf[dk] = v;
  }
  const float* mrow = p.mask ? p.mask + (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)qi * p.ms2 : nullptr;

  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[i][e] = 0.f;
  float m = -INFINITY, l = 0.f;

  // This thread's 16-byte chunks of a tile: chunk i = key k0 + i * KST, dims
  // (ltid % KG) * 8, of K (stored at LDS row key_row(key)) and of V (stored at row key).
  // Only the i = 0 offsets live in registers: the others add a uniform byte stride
  // (global side) or a constant (LDS side, since key_row acts bitwise on the disjoint
  // bits of k0 and i * KST). Byte offsets from the tile base fit in 32 bits (the host
  // bounds the key strides).
  constexpr int KST = TPT / KG;               // keys between a thread's chunks
  const int k0 = ltid / KG, dc = ltid % KG;
  const unsigned koff0 = (unsigned)(k0 * p.ks1 + dc * 8) * 2u;
  const unsigned kstep = (unsigned)(KST * p.ks1) * 2u;
  const unsigned voff0 = (unsigned)(k0 * p.vs1 + dc * 8) * 2u;
  const unsigned vstep = (unsigned)(KST * p.vs1) * 2u;
  const int kst0 = key_row(k0) * KP + dc * 8;
  const int vst0 = k0 * KP + dc * 8;
  // V^T operand of a PV k-step through transposing LDS reads: in each 16-lane group g,
  // lane i addresses row 8 * (g / 2) + i / 4 (+ 4 for the second half, + 16 per k-step)
  // at dims 16 * (g % 2) + 4 * (i % 4) (+ 32 per block of O^T rows), and receives dim
  // 16 * (g % 2) + i of that row group's four keys.
  const int vtr0 = (8 * (lane >> 5) + ((lane & 15) >> 2)) * KP + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // PF register sets of tile chunks. PF = 2: the tile two blocks ahead loads while the
  // next one is stored and the current one is multiplied. PF = 1 (eight-wave key split,
  // where the register budget must allow four waves per SIMD): the next tile loads
  // while the current one is multiplied.
  constexpr int PF = (SPLIT == 8 || D >= 128) ? 1 : 2;
  E8 kst[PF][KPT], vst[PF][KPT];
  // Tile loads through buffer resources whose extent ends at the last valid key:
  // addresses need no per-lane arithmetic and rows past the key length read as zero.
  // (V^T reads past a row's padded end wrap into the next row: finite values whose
  // probabilities are zero.)
  auto load_tile = [&](auto set_c, int kbase) {
    constexpr int S = decltype(set_c)::value;
    const int rows = min(KB, p.LK - kbase);
    const auto kr = make_rsrc(kb_ + (int64_t)kbase * p.ks1, (unsigned)(((rows - 1) * p.ks1 + D) * 2));
    const auto vr = make_rsrc(vb_ + (int64_t)kbase * p.vs1, (unsigned)(((rows - 1) * p.vs1 + D) * 2));
#pragma unroll
    for (int i = 0; i < KPT; i++)
      if (KALL || ltid + i * TPT < KCH) kst[S][i] = buffer_load16<E8>(kr, koff0, i * kstep);
#pragma unroll
    for (int i = 0; i < KPT; i++)
      if (KALL || ltid + i * TPT < KCH) vst[S][i] = buffer_load16<E8>(vr, voff0, i * vstep);
  };
  auto store_tile = [&](auto set_c, E* kd) {
    constexpr int S = decltype(set_c)::value;
    E* vd = kd + KB * KP;
#pragma unroll
    for (int i = 0; i < KPT; i++)
      if (KALL || ltid + i * TPT < KCH)
        *reinterpret_cast<E8*>(kd + kst0 + key_row((i * KST) & 31) * KP) = kst[S][i];
#pragma unroll
    for (int i = 0; i < KPT; i++)
      if (KALL || ltid + i * TPT < KCH) *reinterpret_cast<E8*>(vd + vst0 + ((i * KST) & 31) * KP) = vst[S][i];
  };

  const int nblk = (p.LK + KB - 1) / KB;
  const int nit = SPLIT == 1 ? nblk : (nblk - wave + SPLIT - 1) / SPLIT;   // this wave's blocks
  auto blk_of = [&](int it) { return SPLIT == 1 ? it : it * SPLIT + wave; };
  auto tile_k = [&](int it) { return SPLIT == 1 ? smem + (it & 1) * TILE : Ks; };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  if (nit > 0) load_tile(S0(), blk_of(0) * KB);
  if (nit > 0) store_tile(S0(), tile_k(0));
  if constexpr (PF == 2) {
    if (nit > 1) load_tile(S1(), blk_of(1) * KB);
  }
  if constexpr (SPLIT == 1) __syncthreads();

  // One key block: block it is in LDS, block it + 1 in register set NEXT (stored after
  // the multiply), block it + 2 is loaded into the other set.
  auto block = [&](int it, auto next_c) {
    constexpr int NX = PF == 2 ? decltype(next_c)::value : 0;
    using NXC = std::integral_constant<int, NX>;
    const int kbase = blk_of(it) * KB;
    if constexpr (PF == 2) {
      if (it + 2 < nit) load_tile(std::integral_constant<int, 1 - NX>(), blk_of(it + 2) * KB);
    } else {
      if (it + 1 < nit) load_tile(NXC(), blk_of(it + 1) * KB);
    }
    const E* Kc = tile_k(it);
    const E* Vc = Kc + KB * KP;

    // S^T = K Q^T: rows = keys (permuted by key_row), columns = queries.
    f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; e++) s[e] = 0.f;
#pragma unroll
    for (int dk = 0; dk < DK; dk++) {
      const int d = dk * 16 + 8 * hf;
      E8 kf = {0, 0, 0, 0, 0, 0, 0, 0};
      if (d < D) kf = *reinterpret_cast<const E8*>(Kc + col * KP + d);
      s = mfma32x(kf, qf[dk], s);
    }
    // Lane holds keys kbase + 16*(e/8) + 8*hf + e%8 of query q0 + col. Exponents are
    // log2-scaled: t = s * scale * log2(e) (+ mask * log2(e)).
    float mn, base;
    if (kbase + KB <= p.LK && !mrow) {
      // med3(a, b, +inf) = max(a, b) without the operand canonicalisation fmaxf needs.
      float top = __builtin_amdgcn_fmed3f(s[0], s[1], INFINITY);
#pragma unroll
      for (int e = 2; e < 16; e++) top = __builtin_amdgcn_fmed3f(top, s[e], INFINITY);
      top = halves_max(top);
      mn = fmaxf(m, top * p.c);
      base = mn;
#pragma unroll
      for (int e = 0; e < 16; e++) s[e] = s[e] * p.c - base;
    } else {
      float top = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int key = kbase + 16 * (e >> 3) + 8 * hf + (e & 7);
        float t = s[e] * p.c;
        if (key >= p.LK) t = -INFINITY;
        else if (mrow) t += mrow[(int64_t)key * p.ms3] * 1.44269504088896341f;
        s[e] = t;
        top = fmaxf(top, t);
      }
      top = halves_max(top);
      mn = fmaxf(m, top);
      // A query with every key so far removed keeps m = -inf and contributes nothing.
      base = mn == -INFINITY ? 0.f : mn;
#pragma unroll
      for (int e = 0; e < 16; e++) s[e] -= base;
    }
    const float alpha = __builtin_amdgcn_exp2f(m - base);
    m = mn;
    E8 pf[2];
    float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(s[e]), p1 = __builtin_amdgcn_exp2f(s[e + 1]);
      const E2 pr = __builtin_convertvector((f32x2){p0, p1}, E2);
      pf[e >> 3][e & 7] = pr[0];
      pf[e >> 3][(e & 7) + 1] = pr[1];
      sum0 += p0;
      sum1 += p1;
    }
    l = l * alpha + (sum0 + sum1);
    // Rescale only when some query's running max moved (wave-uniform test).
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int db = 0; db < DB; db++) scale_in_place(o[db], alpha);
    }
    // O^T += V^T P^T over two 16-key k-steps: lane (hf, d) supplies keys 16*ks + 8*hf ..
    // + 7 of dim d, the keys pf[ks] holds.
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int db = 0; db < DB; db++) {
        const E* va = Vc + vtr0 + ks * 16 * KP + db * 32;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4(va));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4(va + 4 * KP));
        const E8 vf = __builtin_bit_cast(E8, (s16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        o[db] = mfma32x(vf, pf[ks], o[db]);
      }
    }
    if constexpr (SPLIT == 1) {
      if (it + 1 < nit) store_tile(NXC(), tile_k(it + 1));
      __syncthreads();
    } else {
      // Wave-private tile: LDS operations of one wave complete in order, so only the
      // compiler must keep the stores after this block's reads.
      __builtin_amdgcn_wave_barrier();
      if (it + 1 < nit) store_tile(NXC(), Ks);
      __builtin_amdgcn_wave_barrier();
    }
  };
  // Wait once for every vector-memory load so far (Q fragments, the first tiles): the
  // compiler then sees nothing outstanding that the loop's MFMAs read, and no longer
  // drains the tile prefetch in front of them.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  for (int it = 0; it < nit; it += 2) {
    block(it, S1());
    if (it + 1 < nit) block(it + 1, S0());
  }
  l = halves_sum(l);

  E* ob = p.o + (int64_t)b * p.os0 + (int64_t)h * p.os2;
  const int qo = q0 + col;
  if constexpr (SPLIT == 1) {
    if (qo < p.L) {
      const float inv = l > 0.f ? 1.0f / l : 0.f;
      E* orow = ob + (int64_t)qo * p.os1;
#pragma unroll
      for (int db = 0; db < DB; db++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int d = db * 32 + j * 8 + 4 * hf;
          if (d < D) {
            E4 out;
#pragma unroll
            for (int r = 0; r < 4; r++) out[r] = (E)(o[db][j * 4 + r] * inv);
            *reinterpret_cast<E4*>(orow + d) = out;
          }
        }
    }
  } else {
    // Merge the waves' states: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w.
    float* mo = reinterpret_cast<float*>(smem);            // [SPLIT][D][32] partial O^T
    float* ml = mo + SPLIT * D * 32;                        // [SPLIT][32] m, then [SPLIT][32] l
    __syncthreads();
#pragma unroll
    for (int db = 0; db < DB; db++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int d = db * 32 + (e >> 2) * 8 + 4 * hf + (e & 3);
        if (d < D) mo[(wave * D + d) * 32 + col] = o[db][e];
      }
    if (hf == 0) { ml[wave * 32 + col] = m; ml[SPLIT * 32 + wave * 32 + col] = l; }
    __syncthreads();
    // Thread t finishes query t % 32 for dims (t / 32) * 4 .. + 4.
    for (int idx = threadIdx.x; idx < 32 * (D / 4); idx += NT) {
      const int qq = idx & 31, d4 = (idx >> 5) * 4;
      float mw[SPLIT], M = -INFINITY;
#pragma unroll
      for (int w = 0; w < SPLIT; w++) { mw[w] = ml[w * 32 + qq]; M = fmaxf(M, mw[w]); }
      const float bse = M == -INFINITY ? 0.f : M;
      float den = 0.f, f[SPLIT];
#pragma unroll
      for (int w = 0; w < SPLIT; w++) { f[w] = exp2f(mw[w] - bse); den += f[w] * ml[SPLIT * 32 + w * 32 + qq]; }
      const float inv = den > 0.f ? 1.0f / den : 0.f;
      const int qg = q0 + qq;
      if (qg < p.L) {
        E4 out;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          float acc = 0.f;
#pragma unroll
          for (int w = 0; w < SPLIT; w++) acc += f[w] * mo[(w * D + d4 + r) * 32 + qq];
          out[r] = (E)(acc * inv);
        }
        *reinterpret_cast<E4*>(ob + (int64_t)qg * p.os1 + d4) = out;
      }
    }
  }
}

// Key-split kernel with tiles moved by DMA and a software-pipelined block loop: a
// workgroup's SPLIT waves own the same 32 queries and take interleaved 32-key blocks
// (block SPLIT * i + wave). Each wave has private tile buffers in LDS -- K three deep, V
// two deep -- that direct global->LDS loads fill, so no register holds a tile in transit.
// Tile rows are D halves without padding; 16-byte chunk c of row r sits at chunk position
// c ^ (r mod KG) (KG = D / 8 chunks per row), which spreads both the K-fragment reads and
// the transposing V reads over the banks. K rows are permuted by key_row as in
// attention_kernel; the loads go through buffer resources that end at the last key, so
// rows past the sequence read zeros (probability zero).
//
// Step it of the loop issues eight MFMAs whose operands are already in registers -- S^T
// of block it + 1 (K fragments read during step it - 1) and O^T += V^T P^T of block it - 1
// (probabilities and V^T fragments from step it - 1), the S chain and the two O chains
// alternating -- then reads the K fragments of block it + 2 and the V^T fragments of
// block it, whose latency the softmax of block it covers. No MFMA waits on an LDS read or
// on the softmax it runs beside; two register sets alternate with the step's parity.
template <int D, int SPLIT, int QG>
struct AttnPipeLds {
  static constexpr int HT = 32 * D;                              // halves per K or V tile
  static constexpr int MERGE = QG * (SPLIT * 32 * (D + 4) + 2 * 32 * SPLIT);   // floats for the merge
  static constexpr int RING = QG * SPLIT * 5 * HT * 2;                          // bytes of the tile rings
  static constexpr size_t bytes = (size_t)(RING > MERGE * 4 ? RING : MERGE * 4);
};

template <int D, int SPLIT, int QG>
__global__ __launch_bounds__(64 * SPLIT * QG) __attribute__((amdgpu_waves_per_eu(2, 8)))
void attention_pipe_kernel(AttnParams p) {
  touch_args(p);
  constexpr int NT = 64 * SPLIT * QG;
  constexpr int KB = 32;
  constexpr int DK = D / 16, DB = D / 32, KG = D / 8;
  constexpr int HT = AttnPipeLds<D, SPLIT, QG>::HT;
  constexpr int NH = HT * 2 / 1024;           // 1 KB DMA instructions per K or V tile
  constexpr int RPD = 1024 / (D * 2);
  static_assert(D == 32 || D == 64, "DMA tiles for head widths 32 and 64");
  static_assert(DK == 2 * DB, "one PV (k-step, dims block) pair per S k-step");
  extern __shared__ __attribute__((aligned(16))) E smem[];

  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hf = lane >> 5, col = lane & 31;
  // Wave wv takes query block qg of the workgroup's QG and key share `wave`: the QG waves
  // of a key share (neighbours, on different SIMDs) stream the same tiles together.
  const int qg = wv % QG, wave = wv / QG;
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x < rem ? x * (per + 1) + k : rem * (per + 1) + (x - rem) * per + k;
  }
  const int nqb = (p.L + 32 * QG - 1) / (32 * QG);
  const int qblk = wg % nqb, h = (wg / nqb) % p.H, b = wg / nqb / p.H;
  const int q0 = (qblk * QG + qg) * 32;
  E* kbuf = smem + wv * 5 * HT;             // three K tiles, then two V tiles
  E* vbuf = kbuf + 3 * HT;
  const unsigned kbuf_lds = lds_offset(kbuf), vbuf_lds = lds_offset(vbuf);

  const E* qb_ = p.q + (int64_t)b * p.qs0 + (int64_t)h * p.qs2;
  const E* kb_ = p.k + (int64_t)b * p.ks0 + (int64_t)h * p.ks2;
  const E* vb_ = p.v + (int64_t)b * p.vs0 + (int64_t)h * p.vs2;

  const int qi = min(q0 + col, p.L - 1);
  const float* mrow = p.mask ? p.mask + (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)qi * p.ms2 : nullptr;
  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[i][e] = 0.f;
  float l = 0.f;
  float m = -INFINITY;   // exponent base of the lane's query (log2 units), -inf before its first key

  unsigned koff[NH], voff[NH];
#pragma unroll
  for (int j = 0; j < NH; j++) {
    const int R = j * RPD + lane / KG, c = (lane % KG) ^ (R % KG);
    koff[j] = (unsigned)(key_row(R) * p.ks1 + c * 8) * 2u;
    voff[j] = (unsigned)(R * p.vs1 + c * 8) * 2u;
  }
  const i32x4 krs = dma_rsrc(kb_, (unsigned)(((int64_t)(p.LK - 1) * p.ks1 + D) * 2));
  const i32x4 vrs = dma_rsrc(vb_, (unsigned)(((int64_t)(p.LK - 1) * p.vs1 + D) * 2));
  const int nblk = (p.LK + KB - 1) / KB;
  // This wave's key blocks: the share's positions of each period, period after period.
  // (Selected with constant indices: a kernel argument indexed at run time would be
  // copied to scratch memory.)
  int kcnt = p.kcnt[0], nit = p.knit[0];
  unsigned ksl0 = p.kslot[0][0], ksl1 = p.kslot[0][1], ksl2 = p.kslot[0][2], ksl3 = p.kslot[0][3];
#pragma unroll
  for (int w = 1; w < SPLIT; w++)
    if (wave == w) {
      kcnt = p.kcnt[w]; nit = p.knit[w];
      ksl0 = p.kslot[w][0]; ksl1 = p.kslot[w][1]; ksl2 = p.kslot[w][2]; ksl3 = p.kslot[w][3];
    }
  const int kper = p.kper;
  const uint64_t kslo = ((uint64_t)ksl1 << 32) | ksl0, kshi = ((uint64_t)ksl3 << 32) | ksl2;
  auto slot = [&](int r) {   // position r of the share's period (two shifts, no table)
    return (int)(((r < 8 ? kslo : kshi) >> ((r & 7) * 8)) & 0xffu);
  };
  auto block_of = [&](int it) { const int q = it / kcnt; return q * kper + slot(it - q * kcnt); };
  // The K and V requests walk the blocks in order: one (period, position) cursor each.
  int kq = 0, kr = 0, vq = 0, vr = 0;
  // Tiles past this wave's blocks are loaded too (their rows lie past the sequence and
  // read zeros), so every pipeline step issues the same number of loads.
  auto issue_k = [&](int it) {
    const unsigned ks = __builtin_amdgcn_readfirstlane((unsigned)((kq * kper + slot(kr)) * KB * p.ks1) * 2u);
    if (++kr == kcnt) { kr = 0; kq++; }
    const unsigned dst = __builtin_amdgcn_readfirstlane(kbuf_lds + (unsigned)((it % 3) * HT * 2));
#pragma unroll
    for (int j = 0; j < NH; j++) dma_buffer_b128(krs, koff[j], ks, dst + j * 1024);
  };
  auto issue_v = [&](int it) {
    const unsigned vs = __builtin_amdgcn_readfirstlane((unsigned)((vq * kper + slot(vr)) * KB * p.vs1) * 2u);
    if (++vr == kcnt) { vr = 0; vq++; }
    const unsigned dst = __builtin_amdgcn_readfirstlane(vbuf_lds + (unsigned)((it & 1) * HT * 2));
#pragma unroll
    for (int j = 0; j < NH; j++) dma_buffer_b128(vrs, voff[j], vs, dst + j * 1024);
  };
  const int vr0 = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int vd0 = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  auto vaddr = [&](int r, int d) { return r * D + (((d >> 3) ^ (r % KG)) << 3) + (d & 7); };
  // V^T read addresses (halves, in the first V buffer; the second is HT further).
  int va[2][DB][2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++)
#pragma unroll
    for (int db = 0; db < DB; db++) {
      va[ks][db][0] = vaddr(vr0 + ks * 16, vd0 + db * 32);
      va[ks][db][1] = vaddr(vr0 + ks * 16 + 4, vd0 + db * 32);
    }
  // K fragment (k-step dk) of the block in K slot `slot`, V^T fragment (ks, db) of the
  // block in V slot `slot`.
  auto read_k = [&](int slot, int dk) {
    const int c = 2 * dk + hf;
    return *reinterpret_cast<const E8*>(kbuf + slot * HT + col * D + ((c ^ (col % KG)) << 3));
  };
  auto read_v = [&](int slot, int ks, int db) {
    const E* Vc = vbuf + slot * HT;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4(Vc + va[ks][db][0]));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4(Vc + va[ks][db][1]));
    return __builtin_bit_cast(E8, (s16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
  };

  // Pipeline state, two register sets alternating with the parity of the step.
  E8 qf[DK];
  E8 kf[2][DK];        // K fragments of the block whose S^T the step issues
  E8 pf[2][2];         // probabilities of a block (the B operands of its two PV k-steps)
  E8 vf[2][2][DB];     // V^T fragments of a block
  f32x16 sacc[2];      // S^T of the block in softmax / of the next block
#pragma unroll
  for (int x = 0; x < 2; x++) {
#pragma unroll
    for (int y = 0; y < 2; y++) {
      pf[x][y] = (E8){};
#pragma unroll
      for (int db = 0; db < DB; db++) vf[x][y][db] = (E8){};
    }
  }

  // Q^T fragments by asm loads, issued before the tile DMAs: the compiler's own wait for a
  // load it could see would drain every DMA issued after it.
#pragma unroll
  for (int dk = 0; dk < DK; dk++)
    asm volatile("global_load_dwordx4 %0, %1, off"
                 : "=v"(qf[dk])
                 : "v"(qb_ + (int64_t)qi * p.qs1 + dk * 16 + 8 * hf)
                 : "memory");
  issue_k(0); issue_k(1); issue_k(2); issue_v(0); issue_v(1);
  vmcnt_wait<4 * NH>();   // Q and K(0) have landed
#pragma unroll
  for (int dk = 0; dk < DK; dk++) asm volatile("" : "+v"(qf[dk]));
  sacc[0] = (f32x16){};
#pragma unroll
  for (int dk = 0; dk < DK; dk++) sacc[0] = mfma32x(read_k(0, dk), qf[dk], sacc[0]);
  vmcnt_wait<3 * NH>();   // K(1) has landed
#pragma unroll
  for (int dk = 0; dk < DK; dk++) kf[0][dk] = read_k(1, dk);
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): K slots 0 and 1 are read
  issue_k(3); issue_k(4);
  // In flight now: K(2), V(0), V(1), K(3), K(4); step it awaits all but the last 3 * NH.

  constexpr float RB = 8.f;
  // Probabilities of exponent arguments sc rounded to the element type in pairs (one
  // packed conversion each) for the PV product; the row sum adds the unrounded fp32
  // values, as the reference's total does (_attention_half.py:84-86).
  auto probs = [&](const f32x16& sc, E8 (&pc)[2]) {
    float sum0, sum1;
    unsigned pk[8];
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(sc[e]), p1 = __builtin_amdgcn_exp2f(sc[e + 1]);
      pk[e >> 1] = __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2){p0, p1}, E2));
      sum0 = e == 0 ? p0 : sum0 + p0;
      sum1 = e == 0 ? p1 : sum1 + p1;
    }
    pc[0] = __builtin_bit_cast(E8, (u32x4){pk[0], pk[1], pk[2], pk[3]});
    pc[1] = __builtin_bit_cast(E8, (u32x4){pk[4], pk[5], pk[6], pk[7]});
    return sum0 + sum1;
  };
  // Softmax of block it (scores sc) into probabilities pc; returns alpha, the factor for
  // the accumulator (1 unless the base moved). The base moves only when the block's
  // maximum exceeds it by more than RB (log2 units): probabilities stay small enough for
  // the element type, and the accumulator rescale is skipped for all but the few blocks
  // that raise the maximum that much.
  // FULL (every key lies in the sequence, no mask, the base is finite): the
  // probabilities are formed against the current base first, with no block maximum --
  // each is at most its lane's sum of 16, so a sum of at most 16 * 2^RB (inf and NaN
  // fail the test) keeps every one within 2^12, far inside the element type. Only a wave
  // with a larger sum takes the block maximum (over the exponent arguments s * c - m,
  // canonical FMA results), moves the base of each query whose maximum exceeds RB, and
  // forms its probabilities again.
  // Otherwise the block maximum comes first; a query with every key so far removed keeps
  // m = -inf and contributes nothing.
  auto softmax = [&](int it, auto full_c, f32x16& sc, E8 (&pc)[2]) {
    constexpr bool FULL = decltype(full_c)::value;
    float alpha = 1.f, sum;
    if constexpr (FULL) {
#pragma unroll
      for (int e = 0; e < 16; e++) sc[e] = sc[e] * p.c - m;
      sum = probs(sc, pc);
      if (__builtin_expect(__ballot(!(sum <= 16.f * 256.f)) != 0, 0)) {
        const float top = halves_max(max16(sc));
        const float dlt = top > RB ? top : 0.f;
#pragma unroll
        for (int e = 0; e < 16; e++) sc[e] -= dlt;
        alpha = __builtin_amdgcn_exp2f(-dlt);
        m += dlt;
        sum = probs(sc, pc);
      }
    } else {
      const int kbase = block_of(it) * KB;
      float top = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int key = kbase + 16 * (e >> 3) + 8 * hf + (e & 7);
        float t = sc[e] * p.c;
        if (key >= p.LK) t = -INFINITY;
        else if (mrow) t += mrow[(int64_t)key * p.ms3] * 1.44269504088896341f;
        sc[e] = t;
        top = fmaxf(top, t);
      }
      top = halves_max(top);
      const float mn = top > m + RB ? top : m;
      const float base = mn == -INFINITY ? 0.f : mn;
      alpha = __builtin_amdgcn_exp2f(m - base);
      m = mn;
#pragma unroll
      for (int e = 0; e < 16; e++) sc[e] -= base;
      sum = probs(sc, pc);
    }
    l = l * alpha + sum;
    return alpha;
  };

  // One pipeline step; X = it % 2 picks the register sets (the loop runs two steps per
  // iteration): kf[X] holds K(it + 1), pf[1 - X] / vf[1 - X] block it - 1, sacc[X] S(it).
  auto step = [&](int it, auto x_c, auto full_c) {
    constexpr int X = decltype(x_c)::value;
    vmcnt_wait<3 * NH>();   // K(it + 2) and V(it) have landed
    // S^T of block it + 1 and O^T += V^T P^T of block it - 1, the chains alternating (the
    // PV pairs (ks, db) in the order that revisits a dims block two issues later); both
    // are harmless when their block lies past this wave's last (tiles of zeros, zero
    // probabilities before the first block).
    sacc[1 - X] = (f32x16){};
#pragma unroll
    for (int i = 0; i < DK; i++) {
      sacc[1 - X] = mfma32x(kf[X][i], qf[i], sacc[1 - X]);
      o[i % DB] = mfma32x(vf[1 - X][i / DB][i % DB], pf[1 - X][i / DB], o[i % DB]);
    }
    // K fragments of block it + 2 and V^T fragments of block it, for the next step: read
    // before the softmax, whose VALU work covers their latency.
#pragma unroll
    for (int dk = 0; dk < DK; dk++) kf[1 - X][dk] = read_k((it + 2) % 3, dk);
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int db = 0; db < DB; db++) vf[X][ks][db] = read_v(it & 1, ks, db);
    const float alpha = softmax(it, full_c, sacc[X], pf[X]);
    // Rescale after this step's P V (the asm waits out the MFMA results first).
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int db = 0; db < DB; db++) scale_in_place(o[db], alpha);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this step's fragment reads have returned
    issue_v(it + 2);
    issue_k(it + 5);
  };

  // Blocks before nfull are whole and unmasked (only the sequence's last block can be
  // partial, and only the wave that owns it has it as its last). A wave whose first block
  // is whole seeds its queries' bases with that block's maximum, so whole blocks always
  // meet a finite base.
  const int nfull = p.mask ? 0 : (p.LK % KB == 0 || nit == 0 || block_of(nit - 1) != nblk - 1 ? nit : nit - 1);
  if (nfull > 0) m = halves_max(max16(sacc[0])) * p.c;
  using T = std::integral_constant<bool, true>;
  using F = std::integral_constant<bool, false>;
  using V0 = std::integral_constant<int, 0>;
  using V1 = std::integral_constant<int, 1>;
  int it = 0;
  for (; it + 1 < nfull; it += 2) {
    step(it, V0(), T());
    step(it + 1, V1(), T());
  }
  for (; it < nit; it += 2) {
    if (it < nfull) step(it, V0(), T());
    else step(it, V0(), F());
    if (it + 1 < nit) step(it + 1, V1(), F());
  }
  // P V of the wave's last block (its probabilities and V^T are in set (nit - 1) % 2).
  auto last_pv = [&](auto x_c) {
    constexpr int X = decltype(x_c)::value;
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int db = 0; db < DB; db++) o[db] = mfma32x(vf[X][ks][db], pf[X][ks], o[db]);
  };
  if (nit > 0) {
    if (((nit - 1) & 1) == 0) last_pv(V0());
    else last_pv(V1());
  }

  // Merge: every wave publishes its (base, sum) per query; then each scales its O^T by
  // exp2(m_w - M) / den (M and den over the waves) and stores it as [wave][query][d] fp32
  // rows padded to D + 4 (16-byte writes free of bank conflicts); each thread then sums
  // the SPLIT partials of 8 consecutive d of one query into one 16-byte store.
  E* ob = p.o + (int64_t)b * p.os0 + (int64_t)h * p.os2;
  constexpr int RP = D + 4;
  constexpr int MG = SPLIT * 32 * RP + 2 * 32 * SPLIT;   // floats of one query block's merge
  float* mo = reinterpret_cast<float*>(smem) + qg * MG;  // [SPLIT][32][RP] scaled partial O
  float* ml = mo + SPLIT * 32 * RP;                       // [32][SPLIT] m, then the same for l
  vmcnt_wait<0>();
  __syncthreads();   // every wave done with its tiles (the merge area overlaps them)
  {
    const float lj = halves_sum(l);
    if (hf == 0) {
      ml[col * SPLIT + wave] = m;
      ml[32 * SPLIT + col * SPLIT + wave] = lj;
    }
  }
  __syncthreads();
  {
    float M = -INFINITY, mw[SPLIT];
#pragma unroll
    for (int w = 0; w < SPLIT; w++) { mw[w] = ml[col * SPLIT + w]; M = fmaxf(M, mw[w]); }
    const float bse = M == -INFINITY ? 0.f : M;
    float den = 0.f;
#pragma unroll
    for (int w = 0; w < SPLIT; w++) den += __builtin_amdgcn_exp2f(mw[w] - bse) * ml[32 * SPLIT + col * SPLIT + w];
    const float f = den > 0.f ? __builtin_amdgcn_exp2f(m - bse) / den : 0.f;
    float* row = mo + (wave * 32 + col) * RP + 4 * hf;
#pragma unroll
    for (int db = 0; db < DB; db++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const f32x4 v = {o[db][4 * g] * f, o[db][4 * g + 1] * f, o[db][4 * g + 2] * f, o[db][4 * g + 3] * f};
        *reinterpret_cast<f32x4*>(row + db * 32 + g * 8) = v;
      }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < QG * 32 * (D / 8); idx += NT) {
    const int d8 = (idx % (D / 8)) * 8, qq = (idx / (D / 8)) % 32, g = idx / (32 * (D / 8));
    const int qr = (qblk * QG + g) * 32 + qq;
    if (qr >= p.L) continue;
    const float* mg = reinterpret_cast<const float*>(smem) + g * MG;
    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < SPLIT; w++) {
      const float* r = mg + (w * 32 + qq) * RP + d8;
      a0 += *reinterpret_cast<const f32x4*>(r);
      a1 += *reinterpret_cast<const f32x4*>(r + 4);
    }
    const E8 out = {(E)a0[0], (E)a0[1], (E)a0[2], (E)a0[3], (E)a1[0], (E)a1[1], (E)a1[2], (E)a1[3]};
    *reinterpret_cast<E8*>(ob + (int64_t)qr * p.os1 + d8) = out;
  }
}

// The key-share pattern of attention_pipe_kernel for cnt[w] blocks of share w per period:
// the period's positions go to the shares in the order of their due times (k + 1/2) /
// cnt[w], so that every share's blocks spread evenly over the period and all shares
// sweep the key range together.
static int share_pattern(AttnParams& q, int split, const int* cnt) {
  int per = 0;
  for (int w = 0; w < split; w++) {
    if (cnt[w] < 1 || cnt[w] > 16) return fail("attention: key share counts must lie in 1..16");
    per += cnt[w];
  }
  if (per > 64) return fail("attention: key share period above 64 blocks");
  int order[64], n = 0;
  for (int w = 0; w < split; w++)
    for (int k = 0; k < cnt[w]; k++) order[n++] = w * 16 + k;
  // insertion sort by due time, ties by share
  auto due_lt = [&](int a, int b) {
    const int wa = a / 16, ka = a % 16, wb = b / 16, kb = b % 16;
    const long l = (long)(2 * ka + 1) * cnt[wb], r = (long)(2 * kb + 1) * cnt[wa];
    return l < r || (l == r && wa < wb);
  };
  for (int i = 1; i < n; i++)
    for (int j = i; j > 0 && due_lt(order[j], order[j - 1]); j--) std::swap(order[j], order[j - 1]);
  const int nblk = (q.LK + 31) / 32, full = nblk / per, rem = nblk % per;
  q.kper = per;
  for (int w = 0; w < 8; w++) {
    q.kcnt[w] = w < split ? cnt[w] : 1;
    q.knit[w] = 0;
    for (int r = 0; r < 4; r++) q.kslot[w][r] = 0;
  }
  for (int i = 0; i < n; i++) {
    const int w = order[i] / 16, k = order[i] % 16;
    q.kslot[w][k / 4] |= (unsigned)i << (8 * (k % 4));
  }
  for (int w = 0; w < split; w++) {
    q.knit[w] = full * cnt[w];
    for (int k = 0; k < cnt[w]; k++)
      if ((int)((q.kslot[w][k / 4] >> (8 * (k % 4))) & 0xffu) < rem) q.knit[w]++;
  }
  return 0;
}

template <int D, int SPLIT, int QG = 1>
static int launch_attn_pipe(const AttnParams& p0, hipStream_t st) {
  AttnParams p = p0;
  // Blocks per period of each key share: with two query blocks per workgroup a SIMD holds
  // two waves, and the one of the lower key share (the older wave) issues first whenever
  // both are ready, so with equal shares it ends well before the other, which then runs
  // alone; the lower shares take two blocks per period to the upper shares' one (config 2:
  // 12.96 -> 12.46 us; 3:2 the same, 7:3 12.6, 3:1 13.2). LDX_ATTN_SHARES="c0,c1,..."
  // overrides (sweeps).
  int cnt[SPLIT];
  for (int w = 0; w < SPLIT; w++) cnt[w] = QG == 2 ? (w < SPLIT / 2 ? 2 : 1) : 1;
  if (const char* e = getenv("LDX_ATTN_SHARES")) {
    for (int w = 0; w < SPLIT; w++) {
      char* end = nullptr;
      cnt[w] = (int)strtol(e, &end, 10);
      e = *end == ',' ? end + 1 : end;
    }
  }
  if (int rc = share_pattern(p, SPLIT, cnt)) return rc;
  // Tile byte offsets within a (batch, head), up to six periods past the last block, are
  // 32-bit.
  if (((int64_t)p.LK + 32 * 6 * p.kper + 64) * (p.ks1 > p.vs1 ? p.ks1 : p.vs1) * 2 >= ((int64_t)1 << 31))
    return fail("attention: key range too large for the DMA kernel");
  const int64_t n = (int64_t)((p.L + 32 * QG - 1) / (32 * QG)) * p.H * p.B;
  if (n > 0x7fffffff) return fail("attention: grid too large");
  constexpr size_t lds = AttnPipeLds<D, SPLIT, QG>::bytes;
  static_assert(lds <= 160 * 1024, "LDS");
  auto kern = attention_pipe_kernel<D, SPLIT, QG>;
  if (lds > 65536 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return check_launch("attention: set LDS size");
  hipLaunchKernelGGL(kern, dim3((unsigned)n), dim3(64 * SPLIT * QG), lds, st, p);
  return check_launch("attention");
}

template <int D, int SPLIT>
static int launch_attn(const AttnParams& p, hipStream_t st) {
  const int per = SPLIT == 1 ? 128 : 32;
  const int64_t n = (int64_t)((p.L + per - 1) / per) * p.H * p.B;
  if (n > 0x7fffffff) return fail("attention: grid too large");
  dim3 grid((unsigned)n);
  hipLaunchKernelGGL((attention_kernel<D, SPLIT>), grid, dim3(SPLIT == 1 ? 256 : 64 * SPLIT), 0, st, p);
  return check_launch("attention");
}

// Wide heads (D = 128, 256; the VQ decoder's single 256-wide head over 51,200 tokens): a
// workgroup's 4 waves own 4 x 32 queries and share every K/V tile. Tiles move global->LDS
// by DMA (rows of D halves, 16-byte chunk c of row r at chunk position c ^ (r mod D/8);
// K rows permuted by key_row), three deep for K and for V, each wave moving a quarter of
// each tile; one barrier per key block, after which the slots the previous block freed
// are refilled. The S^T MFMAs of block it + 1 are issued before block it's softmax, so its
// VALU work runs under them; the exponent base moves only past a 2^8 margin (as in
// attention_pipe_kernel).
template <int D>
struct AttnWideLds {
  static constexpr int TB = 32 * D * 2;          // bytes per K or V tile (and per wave's Q block)
  static constexpr bool QL = D == 256;           // Q fragments read from LDS (registers too few)
  static constexpr size_t bytes = (QL ? 10 : 6) * (size_t)TB;
};

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 ? 2 : 1, D == 128 ? 2 : 1)))
void attention_wide_kernel(AttnParams p) {
  touch_args(p);
  constexpr int KB = 32;
  constexpr int DK = D / 16, DB = D / 32, KG = D / 8;
  constexpr int TB = AttnWideLds<D>::TB;
  constexpr int NHW = TB / 1024 / 4;          // 1 KB DMA instructions per wave per tile
  constexpr int RPD = 1024 / (D * 2);         // tile rows per DMA instruction
  constexpr bool QL = AttnWideLds<D>::QL;
  static_assert(D == 128 || D == 256, "wide heads");
  extern __shared__ __attribute__((aligned(16))) E smem[];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hf = lane >> 5, col = lane & 31;
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x * per + min(x, rem) + k;
  }
  const int nqb = (p.L + 127) / 128;
  const int nblk_all = (p.LK + KB - 1) / KB;
  E* kbuf = smem;                 // K tiles 0..2, then V tiles 0..2
  E* vbuf = smem + 3 * (TB / 2);
  const unsigned kbuf_lds = lds_offset(kbuf), vbuf_lds = lds_offset(vbuf);
  E* qbuf = smem + 6 * (TB / 2) + wave * (TB / 2);

  // This workgroup's query tile and key blocks [kb0, kb0 + nblk): all of them, or under
  // the split schedule piece `piece` of pmax equal pieces.
  const int S = p.part ? p.pmax : 1;
  const int t = wg / S, piece = wg - t * S;
  const int kb0 = (int)((unsigned)(piece * nblk_all) / (unsigned)S);   // < 2^31: S <= 8
  const int nblk = (int)((unsigned)((piece + 1) * nblk_all) / (unsigned)S) - kb0;
  const int qblk = t % nqb, h = (t / nqb) % p.H, b = t / nqb / p.H;
  const int q0 = qblk * 128 + wave * 32;
  const E* qb_ = p.q + (int64_t)b * p.qs0 + (int64_t)h * p.qs2;
  const E* kb_ = p.k + (int64_t)b * p.ks0 + (int64_t)h * p.ks2;
  const E* vb_ = p.v + (int64_t)b * p.vs0 + (int64_t)h * p.vs2;
  const int qi = min(q0 + col, p.L - 1);
  const float* mrow = p.mask ? p.mask + (int64_t)b * p.ms0 + (int64_t)h * p.ms1 + (int64_t)qi * p.ms2 : nullptr;

  // Q^T fragments: in registers (D = 128), or (D = 256, where O^T alone takes 128
  // registers) in this wave's LDS block, laid out like a K tile without the row
  // permutation and read with the K fragments.
  E8 qf[QL ? 1 : DK];
  if constexpr (!QL) {
#pragma unroll
    for (int dk = 0; dk < DK; dk++) qf[dk] = *reinterpret_cast<const E8*>(qb_ + (int64_t)qi * p.qs1 + dk * 16 + 8 * hf);
  }
  f32x16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[i][e] = 0.f;
  float m = -INFINITY, l = 0.f;

  // This wave's DMA instructions of a tile: j = wave * NHW + jj covers rows RPD j ..
  // + RPD - 1; lane -> row RPD j + lane / KG, chunk position lane % KG.
  unsigned koff[NHW], voff[NHW];
#pragma unroll
  for (int jj = 0; jj < NHW; jj++) {
    const int R = (wave * NHW + jj) * RPD + lane / KG, c = (lane % KG) ^ (R % KG);
    koff[jj] = (unsigned)(key_row(R) * p.ks1 + c * 8) * 2u;
    voff[jj] = (unsigned)(R * p.vs1 + c * 8) * 2u;
  }
  // Block it's tile through a buffer resource that ends at the sequence's last key (none
  // past it: a block beyond the last reads zeros).
  auto issue = [&](const E* base, int64_t rs1, const unsigned (&off)[NHW], unsigned dst_base, int it) {
    const int kbase = (kb0 + it) * KB;
    const int rows = min(KB, p.LK - kbase);
    const i32x4 rs = dma_rsrc(rows > 0 ? base + (int64_t)kbase * rs1 : base,
                              rows > 0 ? (unsigned)(((rows - 1) * rs1 + D) * 2) : 0u);
    const unsigned dst = dst_base + (unsigned)((it % 3) * TB + wave * NHW * 1024);
#pragma unroll
    for (int jj = 0; jj < NHW; jj++) dma_buffer_b128(rs, off[jj], 0, dst + jj * 1024);
  };
  auto issue_k = [&](int it) { issue(kb_, p.ks1, koff, kbuf_lds, it); };
  auto issue_v = [&](int it) { issue(vb_, p.vs1, voff, vbuf_lds, it); };

  // Fragment read addresses, in bytes from the tile base: (lane part + slot base) ^ (a
  // compile-time constant per k-step, row group and block of dims). K: row col, chunk
  // position (2 dk + hf) ^ (col mod KG) = (hf ^ col mod KG) ^ 2 dk. V^T (transposing
  // reads): row vr0 + 16 ks + 4 hi and dims vd0 + 32 db, whose bits are disjoint, so that
  // row and chunk position each split into a lane part and a constant part by XOR. The lane
  // parts pass through an empty asm once per block, so that the compiler forms the
  // addresses at each read instead of keeping every one of them in a register.
  const int vr0 = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int vd0 = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const unsigned ka_lane = (unsigned)(col * D * 2 + ((hf ^ (col % KG)) << 4));
  const unsigned va_lane = (unsigned)(2 * D * vr0 + (((vd0 >> 3) ^ (vr0 % KG)) << 4) + 2 * (vd0 & 7));
  auto kconst = [](int dk) { return (unsigned)(dk << 5); };
  auto vconst = [](int ks, int hi, int db) {
    const int rc = 16 * ks + 4 * hi;                         // row bits added to vr0
    const int cc = (4 * db) ^ (rc % KG);                     // chunk bits added to vd0 / 8
    return (unsigned)(2 * D * rc) ^ (unsigned)(cc << 4);
  };
  const char* kbase_p = reinterpret_cast<const char*>(kbuf);
  const char* qbase_p = reinterpret_cast<const char*>(qbuf);
  const char* vbase_p = reinterpret_cast<const char*>(vbuf);
  // S^T = K Q^T of block it (rows = keys permuted by key_row, columns = queries).
  // (Operands are read four k-steps at a time, fenced from the scheduler, so that the
  // fragments in flight stay within the register budget.)
  auto compute_s = [&](int it, f32x16& s) {
    unsigned ka = ka_lane + (unsigned)((it % 3) * TB);
    asm volatile("" : "+v"(ka));
    s = (f32x16){};
#pragma unroll
    for (int g = 0; g < DK; g += 4) {
      E8 kf[4];
#pragma unroll
      for (int u = 0; u < 4; u++) kf[u] = *reinterpret_cast<const E8*>(kbase_p + (ka ^ kconst(g + u)));
      if constexpr (QL) {
        E8 qg[4];
#pragma unroll
        for (int u = 0; u < 4; u++) qg[u] = *reinterpret_cast<const E8*>(qbase_p + (ka_lane ^ kconst(g + u)));
#pragma unroll
        for (int u = 0; u < 4; u++) s = mfma32x(kf[u], qg[u], s);
      } else {
#pragma unroll
        for (int u = 0; u < 4; u++) s = mfma32x(kf[u], qf[g + u], s);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  constexpr float RB = 8.f;
  auto softmax_pv = [&](int it, auto full_c, f32x16& s) {
    constexpr bool FULL = decltype(full_c)::value;
    unsigned va = va_lane + (unsigned)((it % 3) * TB);
    float top;
    if constexpr (FULL) {
      const float t0 = fmaxf(fmaxf(s[0], s[1]), s[2]), t1 = fmaxf(fmaxf(s[3], s[4]), s[5]);
      const float t2 = fmaxf(fmaxf(s[6], s[7]), s[8]), t3 = fmaxf(fmaxf(s[9], s[10]), s[11]);
      const float t4 = fmaxf(fmaxf(s[12], s[13]), s[14]);
      top = halves_max(fmaxf(fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)), fmaxf(t4, s[15]))) * p.c;
    } else {
      const int kbase = (kb0 + it) * KB;
      top = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int key = kbase + 16 * (e >> 3) + 8 * hf + (e & 7);
        float t = s[e] * p.c;
        if (key >= p.LK) t = -INFINITY;
        else if (mrow) t += mrow[(int64_t)key * p.ms3] * 1.44269504088896341f;
        s[e] = t;
        top = fmaxf(top, t);
      }
      top = halves_max(top);
    }
    // The exponent base moves only when the block raises the query's maximum by more than
    // RB (log2 units); a query with every key so far removed keeps m = -inf.
    const float mn = top > m + RB ? top : m;
    const float base = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - base);
    m = mn;
    if constexpr (FULL) {
#pragma unroll
      for (int e = 0; e < 16; e++) s[e] = s[e] * p.c - base;
    } else {
#pragma unroll
      for (int e = 0; e < 16; e++) s[e] -= base;
    }
    E8 pf[2];
    float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float p0 = __builtin_amdgcn_exp2f(s[e]), p1 = __builtin_amdgcn_exp2f(s[e + 1]);
      const E2 pr = __builtin_convertvector((f32x2){p0, p1}, E2);
      pf[e >> 3][e & 7] = pr[0];
      pf[e >> 3][(e & 7) + 1] = pr[1];
      sum0 += p0;
      sum1 += p1;
    }
    l = l * alpha + (sum0 + sum1);
    // (Plain multiplies: the accumulators may live in AGPRs, which the rescale reaches
    // through the compiler's own moves.)
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int db = 0; db < DB; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] *= alpha;
    }
    asm volatile("" : "+v"(va));
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int g = 0; g < DB; g += 4) {
        E8 vf[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const E* a0 = reinterpret_cast<const E*>(vbase_p + (va ^ vconst(ks, 0, g + u)));
          const E* a1 = reinterpret_cast<const E*>(vbase_p + (va ^ vconst(ks, 1, g + u)));
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4(a0));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_v4(a1));
          vf[u] = __builtin_bit_cast(E8, (s16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
        }
#pragma unroll
        for (int u = 0; u < 4; u++) o[g + u] = mfma32x(vf[u], pf[ks], o[g + u]);
        __builtin_amdgcn_sched_barrier(0);
      }
  };
  // One step: K(it + 1) and V(it) landed in every wave (own wait, then the barrier, which
  // also retires every read of block it - 1); refill the slots block it - 1 freed, issue
  // S of block it + 1, then block it's softmax and P V.
  auto step = [&](int it, auto full_c, f32x16& cur, f32x16& nxt) {
    vmcnt_wait<2 * NHW>();
    __syncthreads();
    issue_k(it + 3);
    issue_v(it + 2);
    if (it + 1 < nblk) compute_s(it + 1, nxt);
    softmax_pv(it, full_c, cur);
  };

  if constexpr (QL) {
    // This wave's 32 query rows (rows past the sequence read zeros), 16 DMA instructions.
    const int rows = min(32, p.L - q0);
    const i32x4 rs = dma_rsrc(qb_ + (int64_t)q0 * p.qs1, rows > 0 ? (unsigned)(((rows - 1) * p.qs1 + D) * 2) : 0u);
    const unsigned dst = lds_offset(qbuf);
#pragma unroll
    for (int j = 0; j < TB / 1024; j++) {
      const int R = j * RPD + lane / KG, c = (lane % KG) ^ (R % KG);
      dma_buffer_b128(rs, (unsigned)(R * p.qs1 + c * 8) * 2u, 0, dst + j * 1024);
    }
  }
  issue_k(0); issue_v(0); issue_k(1); issue_v(1); issue_k(2);
  vmcnt_wait<0>();
  __syncthreads();
  f32x16 sa, sb;
  if (nblk > 0) compute_s(0, sa);
  const int nfull_all = p.mask ? 0 : (p.LK % KB == 0 ? nblk_all : nblk_all - 1);
  const int nfull = min(max(nfull_all - kb0, 0), nblk);
  using T = std::integral_constant<bool, true>;
  using F = std::integral_constant<bool, false>;
  // Pairs of whole blocks, then the rest (at most a whole block and the partial one, or
  // every block under a mask) through the general softmax, which is exact for whole
  // blocks too. (A tail that mixed the two instantiations per iteration doubled the live
  // registers.)
  int it = 0;
  for (; it + 1 < nfull; it += 2) {
    step(it, T(), sa, sb);
    step(it + 1, T(), sb, sa);
  }
  for (; it + 1 < nblk; it += 2) {
    step(it, F(), sa, sb);
    step(it + 1, F(), sb, sa);
  }
  if (it < nblk) step(it, F(), sa, sb);
  vmcnt_wait<0>();   // trailing DMAs land before the workgroup's LDS is released
  l = halves_sum(l);
  if (S > 1) {
    // A piece of the tile's key range: O^T unnormalized in register order, four registers
    // per lane and row, then (base, row sum): [tile][piece][wave][DB * 4 + 1][64 lanes][4].
    f32x4* dst = reinterpret_cast<f32x4*>(p.part) + (((int64_t)t * S + piece) * 4 + wave) * (DB * 4 + 1) * 64 + lane;
#pragma unroll
    for (int db = 0; db < DB; db++)
#pragma unroll
      for (int e4 = 0; e4 < 4; e4++)
        dst[(db * 4 + e4) * 64] = (f32x4){o[db][4 * e4], o[db][4 * e4 + 1], o[db][4 * e4 + 2], o[db][4 * e4 + 3]};
    dst[(DB * 4) * 64] = (f32x4){m, l, 0.f, 0.f};
    return;
  }
  const int qo = q0 + col;
  if (qo < p.L) {
    E* orow = p.o + (int64_t)b * p.os0 + (int64_t)h * p.os2 + (int64_t)qo * p.os1;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int db = 0; db < DB; db++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        E4 out;
#pragma unroll
        for (int r = 0; r < 4; r++) out[r] = (E)(o[db][j * 4 + r] * inv);
        *reinterpret_cast<E4*>(orow + db * 32 + j * 8 + 4 * hf) = out;
      }
  }
}

// The pieces of each split query tile, combined in piece order (deterministic): with M
// the largest base, o = sum_j 2^(m_j - M) O_j / sum_j 2^(m_j - M) l_j. One workgroup per
// tile, a wave per 32 of its queries.
template <int D, int S>
__global__ __launch_bounds__(256) void attention_wide_merge_kernel(AttnParams p) {
  touch_args(p);
  constexpr int DB = D / 32, R4 = DB * 4 + 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hf = lane >> 5, col = lane & 31;
  const int nqb = (p.L + 127) / 128;
  const int t = blockIdx.x;
  const f32x4* src = reinterpret_cast<const f32x4*>(p.part) + ((int64_t)t * S * 4 + wave) * R4 * 64 + lane;
  constexpr int64_t pstride = (int64_t)4 * R4 * 64;   // float4 rows per piece
  float mj[S], f[S];
  float M = -INFINITY, den = 0.f;
#pragma unroll
  for (int j = 0; j < S; j++) {
    const f32x4 ml = src[j * pstride + (DB * 4) * 64];
    mj[j] = ml[0];
    f[j] = ml[1];   // the row sum, until it becomes the weight below
    M = fmaxf(M, mj[j]);
  }
  const float bse = M == -INFINITY ? 0.f : M;
#pragma unroll
  for (int j = 0; j < S; j++) {
    const float w = __builtin_amdgcn_exp2f(mj[j] - bse);
    den += w * f[j];
    f[j] = w;
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  const int qblk = t % nqb, h = (t / nqb) % p.H, b = t / nqb / p.H;
  const int qo = qblk * 128 + wave * 32 + col;
  if (qo >= p.L) return;
  E* orow = p.o + (int64_t)b * p.os0 + (int64_t)h * p.os2 + (int64_t)qo * p.os1;
  // Two tiles of 32 dims (8 rows of every piece) requested before any is summed.
#pragma unroll
  for (int db = 0; db < DB; db += 2) {
    f32x4 v[2][4][S];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
#pragma unroll
        for (int j = 0; j < S; j++) v[u][jj][j] = src[j * pstride + ((db + u) * 4 + jj) * 64];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        f32x4 acc = f[0] * v[u][jj][0];
#pragma unroll
        for (int j = 1; j < S; j++) acc += f[j] * v[u][jj][j];
        E4 out;
#pragma unroll
        for (int r = 0; r < 4; r++) out[r] = (E)(acc[r] * inv);
        *reinterpret_cast<E4*>(orow + (db + u) * 32 + jj * 8 + 4 * hf) = out;
      }
  }
}

// Split schedule of the wide-head kernel: when the query tiles spread unevenly over the
// CUs (config 4: 400 tiles of 128 queries on 256 CUs, so 144 CUs take two), each tile's
// key blocks are cut into S equal pieces, one workgroup each, S chosen to minimise the
// busiest CU's work -- ceil(tiles S / CUs) x (blocks per piece + a piece's start-up) --
// plus the merge's traffic, in key-block units. S = 1: no split.
template <int D>
static void wide_split(const AttnParams& p, int& S, size_t& bytes) {
  S = 1; bytes = 0;
  const int64_t ntile = (int64_t)((p.L + 127) / 128) * p.H * p.B;
  const int nblk = (p.LK + 31) / 32;
  if (nblk < 64 || getenv("LDX_ATTN_NO_BALANCE")) return;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return;
  const double startup = 4.0, merge = 0.04;   // key-block units (measured scale, D = 256)
  double best = 0.0;
  for (int s = 1; s <= 8; s++) {
    if (nblk / s < 32 || ntile * s > 0x7fffffff) break;
    const double per_cu = std::ceil((double)(ntile * s) / cus);
    const double cost = per_cu * ((double)nblk / s + startup) + (s > 1 ? merge * (double)(ntile * s) : 0.0);
    if (s == 1 || cost < best * 0.99) { best = cost; S = s; }
  }
  if (S > 1) bytes = (size_t)ntile * S * 4 * (D / 32 * 4 + 1) * 64 * 4 * sizeof(float);
}

template <int D>
static int launch_attn_wide(AttnParams p, hipStream_t st) {
  const int64_t n = (int64_t)((p.L + 127) / 128) * p.H * p.B;
  if (n > 0x7fffffff) return fail("attention: grid too large");
  constexpr size_t lds = AttnWideLds<D>::bytes;
  static_assert(lds <= 160 * 1024, "LDS");
  auto kern = attention_wide_kernel<D>;
  if (lds > 65536 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return check_launch("attention: set LDS size");
  int S = 1;
  size_t bytes = 0;
  wide_split<D>(p, S, bytes);
  // Without a workspace of that size (none given, or a caller sized for another plan):
  // one workgroup per tile.
  if (S == 1 || !p.part || p.part_bytes < bytes || ((uintptr_t)p.part & 15)) {
    p.part = nullptr;
    p.pmax = 1;
    hipLaunchKernelGGL(kern, dim3((unsigned)n), dim3(256), lds, st, p);
    return check_launch("attention (wide heads)");
  }
  p.pmax = S;
  hipLaunchKernelGGL(kern, dim3((unsigned)(n * S)), dim3(256), lds, st, p);
  const int rc = check_launch("attention (wide heads, split)");
  if (rc != LDX_OK) return rc;
  switch (S) {
#define LDX_MERGE(S_) \
  case S_: hipLaunchKernelGGL((attention_wide_merge_kernel<D, S_>), dim3((unsigned)n), dim3(256), 0, st, p); break;
    LDX_MERGE(2) LDX_MERGE(3) LDX_MERGE(4) LDX_MERGE(5) LDX_MERGE(6) LDX_MERGE(7) LDX_MERGE(8)
#undef LDX_MERGE
    default: return fail("attention: %d key pieces", S);
  }
  return check_launch("attention (wide heads, merge)");
}

// The kernel family launch_d picks: 1 / 4 / 8 (register-staged, key split), -4 / -8
// (pipelined DMA key split) or -1 (wide heads).
template <int D>
static int attn_split(const AttnParams& p) {
  // Key-split workgroups when 128-query workgroups would leave most CUs idle: for long
  // key sequences the pipelined DMA kernel (head widths 32, 64) or eight waves per 32
  // queries (16), else four.
  const int64_t wgs = (int64_t)((p.L + 127) / 128) * p.H * p.B;
  int split = 1;
  if (const char* env = getenv("LDX_ATTN_SPLIT")) split = atoi(env);
  else if (D == 128 && wgs >= 256) split = -1;   // enough 128-query workgroups to fill the CUs
  else if (D <= 128 && wgs < 512 && p.LK > 64)
    split = (D == 32 || D == 64) && p.LK >= 512 ? -4 : (D <= 64 && p.LK >= 512) ? 8 : 4;
  return split;
}

// Whether launch_d runs the wide-head kernel.
template <int D>
static bool attn_wide(const AttnParams& p) {
  const int split = attn_split<D>(p);
  return (D == 128 || D == 256) && (split == -1 || (split == 1 && getenv("LDX_ATTN_SPLIT") == nullptr));
}

// Whether the four-way key split pairs query blocks in eight-wave workgroups: when there
// are more 32-query workgroups than CUs, a CU would hold two, each streaming its head's K
// and V through L2 separately (the per-CU L2 rate bounds those CUs); a pair's two waves
// of a key share request the same tiles back to back, the second mostly from L1.
static bool pipe_pairs(const AttnParams& p) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return false;
  return (int64_t)((p.L + 31) / 32) * p.H * p.B > cus;
}

template <int D>
static int launch_d(const AttnParams& p, hipStream_t st) {
  const int split = attn_split<D>(p);
  if constexpr (D == 32 || D == 64) {
    // Long key sequences: the DMA-fed, software-pipelined four-way key split
    // (LDX_ATTN_SPLIT=-4 selects it for any length, -42 with query-block pairs; -8 the
    // eight-way split).
    if (split == -4 && !getenv("LDX_ATTN_SPLIT") && pipe_pairs(p)) return launch_attn_pipe<D, 4, 2>(p, st);
    if (split == -4) return launch_attn_pipe<D, 4>(p, st);
    if (split == -42) return launch_attn_pipe<D, 4, 2>(p, st);
    if (split == -8) return launch_attn_pipe<D, 8>(p, st);
  }
  if constexpr (D <= 64) {
    if (split == 8) return launch_attn<D, 8>(p, st);
  }
  if constexpr (D <= 128) {
    if (split == 4 || split == 8) return launch_attn<D, 4>(p, st);
  }
  if constexpr (D == 128 || D == 256) {
    // Wide heads with 128-query workgroups: the DMA-fed pipelined kernel by default
    // (LDX_ATTN_SPLIT=-1 forces it, =1 keeps the register-staged one).
    if (split == -1 || (split == 1 && getenv("LDX_ATTN_SPLIT") == nullptr)) return launch_attn_wide<D>(p, st);
  }
  return launch_attn<D, 1>(p, st);
}


static int check_attention_args(const ldx_attention_args* a) {
  if (!a) return fail("attention: null args");
  if (a->batch < 1 || a->heads < 1 || a->q_len < 1 || a->kv_len < 1)
    return fail("attention: empty shape (B %d H %d L %d LK %d)", a->batch, a->heads, a->q_len, a->kv_len);
  const int D = a->head_dim;
  if (D != 16 && D != 32 && D != 64 && D != 128 && D != 256)
    return fail("attention: head_dim %d not in {16, 32, 64, 128, 256}", D);
  if (!a->q || !a->k || !a->v || !a->o) return fail("attention: null tensor");
  if (a->batch > 65535 || a->heads > 65535 || (int64_t)a->batch * a->heads > 65535)
    return fail("attention: batch x heads too large");
  const int64_t* ss[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
  const void* ps[4] = {a->q, a->k, a->v, a->o};
  for (int i = 0; i < 4; i++) {
    for (int j = 0; j < 3; j++)
      if (ss[i][j] % 8 != 0) return fail("attention: strides must be multiples of 8 elements");
    if ((uintptr_t)ps[i] % 16 != 0) return fail("attention: tensors must be 16-byte aligned");
  }
  // In-tile offsets are 32-bit: 32 key rows of K and of V.
  for (int i = 1; i < 3; i++)
    if (ss[i][1] < 0 || ss[i][1] > (1 << 25))
      return fail("attention: key stride %lld out of range", (long long)ss[i][1]);
  return LDX_OK;
}

static AttnParams make_params(const ldx_attention_args* a) {
  AttnParams p{};
  p.B = a->batch; p.H = a->heads; p.L = a->q_len; p.LK = a->kv_len;
  p.q = (const E*)a->q; p.qs0 = a->q_stride[0]; p.qs1 = a->q_stride[1]; p.qs2 = a->q_stride[2];
  p.k = (const E*)a->k; p.ks0 = a->k_stride[0]; p.ks1 = a->k_stride[1]; p.ks2 = a->k_stride[2];
  p.v = (const E*)a->v; p.vs0 = a->v_stride[0]; p.vs1 = a->v_stride[1]; p.vs2 = a->v_stride[2];
  p.o = (E*)a->o; p.os0 = a->o_stride[0]; p.os1 = a->o_stride[1]; p.os2 = a->o_stride[2];
  p.c = a->scale * 1.44269504088896341f;
  p.mask = a->mask;
  p.ms0 = a->mask_stride[0]; p.ms1 = a->mask_stride[1]; p.ms2 = a->mask_stride[2]; p.ms3 = a->mask_stride[3];
  p.part = (float*)a->workspace;
  p.part_bytes = a->workspace ? a->workspace_bytes : 0;
  return p;
}

// Scratch memory: only the balanced wide-head schedule uses it (the partial states of
// the query tiles it splits); V needs none, being transposed by the LDS reads.
size_t attention_workspace_bytes(const ldx_attention_args* a) {
  if (check_attention_args(a) != LDX_OK) return 0;
  const AttnParams p = make_params(a);
  int S = 1;
  size_t bytes = 0;
  if (a->head_dim == 128 && attn_wide<128>(p)) wide_split<128>(p, S, bytes);
  if (a->head_dim == 256 && attn_wide<256>(p)) wide_split<256>(p, S, bytes);
  return bytes;
}

int attention_entry(const ldx_attention_args* a, void* stream) {
  int rc = check_attention_args(a);
  if (rc != LDX_OK) return rc;
  const int D = a->head_dim;
  const AttnParams p = make_params(a);
  hipStream_t st = as_stream(stream);
  switch (D) {
    case 16: return launch_d<16>(p, st);
    case 32: return launch_d<32>(p, st);
    case 64: return launch_d<64>(p, st);
    case 128: return launch_d<128>(p, st);
    default: return launch_d<256>(p, st);
  }
}

}  // namespace LDX_ELEM_NS
}  // namespace ldx

#if !defined(LDX_ELEM_BF16)
namespace ldx {
namespace bf16_path {
size_t attention_workspace_bytes(const ldx_attention_args* a);
int attention_entry(const ldx_attention_args* a, void* stream);
}  // namespace bf16_path
int attention_f32(const ldx_attention_args* a, void* stream);   // exact.hip
}  // namespace ldx

// The C entry points (in the fp16 unit only): the kernels of the args' dtype.
extern "C" size_t ldx_attention_workspace_bytes(const ldx_attention_args* a) {
  if (a && a->dtype == LDX_DTYPE_BF16) return ldx::bf16_path::attention_workspace_bytes(a);
  if (a && a->dtype == LDX_DTYPE_F16) return ldx::f16_path::attention_workspace_bytes(a);
  return 0;
}

extern "C" int ldx_attention(const ldx_attention_args* a, void* stream) {
  if (a && a->dtype == LDX_DTYPE_BF16) return ldx::bf16_path::attention_entry(a, stream);
  if (a && a->dtype == LDX_DTYPE_F32) return ldx::attention_f32(a, stream);
  if (a && a->dtype != LDX_DTYPE_F16)
    return ldx::fail("attention: dtype %d is not LDX_DTYPE_F16, LDX_DTYPE_BF16 or LDX_DTYPE_F32", a->dtype);
  return ldx::f16_path::attention_entry(a, stream);
}
#endif
