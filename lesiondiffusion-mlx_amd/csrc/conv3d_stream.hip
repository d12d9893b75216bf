// Streamed implicit-GEMM 3x3x3 stride-1 convolution on gfx950 MFMA (v_mfma_f32_32x32x16_f16)
// for the common shapes: input channels in 32-channel chunks (C0, C1 multiples of 32),
// output channels a multiple of the 64- or 128-channel workgroup tile, 16-byte aligned
// NDHWC rows, no output activation, enough bricks to fill the GPU. Everything else runs
// through conv3d_kernel.
//
// Workgroup: 8 waves = 2 K-groups x 4 waves. Each wave owns a 64-channel x 64-voxel block
// (2 x 2 MFMA tiles: every A and every B fragment read from LDS feeds two MFMAs, 1 KB of
// LDS reads per MFMA); the two K-groups take the two 16-channel k-steps of every tap of
// a 32-channel chunk, so each SIMD runs two waves of the same output tile.
//
// Per chunk the weights stream through a 4-slot LDS ring in 9 stages of 3 taps (one
// (kd, kh) pair, kw = 0..2), filled by direct global->LDS loads. One barrier per stage,
// placed between its second and third tap: after it the next stage's slot is readable,
// so the next stage's operands are read from LDS while the third tap's MFMAs run, and
// the slot two stages back is refilled (three stages ahead of its use). Operands sit
// in three register sets (one per kw); every tap's offset in the halo is a compile-time
// constant, so all operand reads are ds_read_b128 at a base register plus an immediate.
// The brick's halo is double-buffered in LDS: the next chunk's halo is requested into
// registers at stage 3 and written (with the fused GroupNorm affine + SiLU prologue, one
// fp16 rounding) into the other buffer during the last stage.
//
// Epilogue: both K-groups leave their partial sums as fp32 voxel rows in LDS; each wave
// then finishes one 64-channel x 32-voxel half of its block, a lane 8 consecutive channels
// of a voxel: (group 0 + group 1), bias (+ per-batch-item bias) plus fp16 shift, output
// scale, fp16 residual, one fp16 rounding, 16-byte stores.
//
// Reference semantics: nax_conv3d (src/lesiondiffusion_mlx/_nax_conv.py:451-619), prologue
// _nax_conv.py:128-136, epilogue :265-270 (+ scaled variant :418-421).

#include "elem.h"
#include "conv3d_stream.h"

#include <type_traits>

namespace ldx {
namespace LDX_ELEM_NS {
namespace cs {

constexpr int CC = 32;            // channels per chunk (two k-steps, one per K-group)
constexpr int PITCH = CC + 8;     // halves per halo voxel
constexpr int NSTG = 9;           // stages per chunk: (kd, kh); a stage is kw = 0..2
constexpr int NSLOT = 4;          // weight ring slots
constexpr int NT = 512;           // 8 waves
constexpr int G = CC / 8;         // 16-byte channel groups per halo voxel
constexpr int VPI = NT / G;       // halo voxels per pass of the workgroup
constexpr int HS = 3;             // stage at which the next chunk's halo is requested

// Halo row stride in halves: each row of TW + 2 voxels padded so that consecutive rows of
// a B fragment (TW voxels apart in the fragment) start TW 16-byte bank groups apart
// (mod 16), which keeps the 16-byte reads of a wave free of bank conflicts.
template <int TW>
constexpr int row_stride() {
  constexpr int pu = PITCH / 8, base = (TW + 2) * pu, target = TW % 16;
  constexpr int pad = ((target - base) % 16 + 16) % 16;
  return (base + pad) * 8;
}

template <int BO, int TD, int TH, int TW>
struct Shape {
  static constexpr int NOBT = BO / 32;              // 32-row output blocks of the tile
  static constexpr int WO = BO / 64, WV = 4 / WO;   // waves over O, over voxels (per K-group)
  static constexpr int BV = WV * 64;                // voxels per brick
  static_assert(TD * TH * TW == BV, "the brick must hold the tile's voxels");
  static constexpr int HD = TD + 2, HH = TH + 2, HW = TW + 2;
  static constexpr int HVOX = HD * HH * HW;
  static constexpr int NHS = (HVOX + VPI - 1) / VPI;  // halo slots per thread
  static constexpr int NHL = NHS + 4;                 // loads of one halo request (+ affine)
  static constexpr int RS = row_stride<TW>();
  static constexpr int HALO = HD * HH * RS * 2;       // bytes of one halo
  static constexpr int HALOP = (HALO + 8191) / 8192 * 8192;  // halo buffer: whole 8 KB rounds
  static constexpr int NR = HALOP / 8192;             // halo DMAs per thread (direct halo)
  static constexpr int NF = 3 * 2 * NOBT;             // 1 KB weight fragments per stage
  static constexpr int LW = (NF + 7) / 8;             // DMAs per wave per stage
  static constexpr int STAGE = NF * 1024;             // bytes per ring slot
  static constexpr int RING = 2 * HALOP;              // byte offset of the ring
  static constexpr int RP = 64 + 4;                   // floats per epilogue row (padded)
  static constexpr int EPI = 16 * 32 * RP * 4;        // epilogue rows: [w4][fv][group] x 32 voxels
  static constexpr int LDS_MAIN = RING + NSLOT * STAGE;
  static constexpr int MST = 8 * 32 * 3 * 4;           // per-wave GroupNorm moments, past the rows
  static constexpr int LDS = LDS_MAIN > EPI + MST ? LDS_MAIN : EPI + MST;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(HALO % 16 == 0 && STAGE % 1024 == 0, "alignment");
};

__device__ __forceinline__ f32x16 mfma(E8 a, E8 b, f32x16 c) {
  return mfma_e(a, b, c);
}

template <int I>
using ic = std::integral_constant<int, I>;

// XF: the GroupNorm affine + SiLU prologue applies (halo staged through registers and
// transformed); otherwise the halo is copied global -> LDS by DMA in its padded layout,
// each lane loading the 16 bytes that belong at its position (padding positions and
// voxels outside the volume read zeros).
template <int BO, int TD, int TH, int TW, bool XF>
__global__ __launch_bounds__(NT) void conv3s1_kernel(StreamParams p) {
  touch_args(p);
  using S = Shape<BO, TD, TH, TW>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave >> 2, w4 = wave & 3;
  const int wo = w4 / S::WV, wv = w4 - wo * S::WV;
  // Every kernel argument the prologue needs, fetched in one batch: left to itself the
  // compiler requests them where first used, one scalar-cache round trip after another.
  asm volatile("" ::"s"(p.x0), "s"(p.x1), "s"(p.x0p), "s"(p.x1p), "s"(p.w), "s"(p.C0), "s"(p.C), "s"(p.NKC),
               "s"(p.nchunk), "s"(p.D), "s"(p.H), "s"(p.W), "s"(gridDim.x), "s"(p.nob), "s"(p.nbr), "s"(p.NBW),
               "s"(p.NBH), "s"(p.dv_nob.m), "s"(p.dv_nob.s), "s"(p.dv_nbr.m), "s"(p.dv_nbr.s), "s"(p.dv_nbw.m),
               "s"(p.dv_nbw.s), "s"(p.dv_nbh.m), "s"(p.dv_nbh.s));

  // Workgroup -> (output tile, brick, batch item); the bricks each XCD receives
  // (workgroups are dealt to the 8 XCDs round-robin) are contiguous, so neighbouring
  // halos meet in the same L2.
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x * per + min(x, rem) + k;   // XCD x's range starts at x * per + min(x, rem)
  }
  // Split-K (the slowest index, so that each XCD's contiguous range shares one chunk range):
  // workgroup ranges of cps channel chunks.
  const int sk = p.split > 1 ? udiv(wg, p.dv_g1) : 0;
  wg -= sk * p.g1;
  const int cb = sk * p.cps;
  const int ce = min(p.nchunk, cb + p.cps);
  const int q1 = udiv(wg, p.dv_nob);
  const int oblk = wg - q1 * p.nob;
  const int b = udiv(q1, p.dv_nbr);
  const int brick = q1 - b * p.nbr;
  const int bt = udiv(brick, p.dv_nbw), bw_i = brick - bt * p.NBW;
  const int bd_i = udiv(bt, p.dv_nbh), bh_i = bt - bd_i * p.NBH;
  const int d0 = bd_i * TD, h0 = bh_i * TH, w0 = bw_i * TW;

  // ---- halo slots of this thread: halo voxel tid / G + j * VPI, channel group cg.
  const int cg = tid % G;
  unsigned hvi[S::NHS];   // source voxel within the batch item, ~0u outside the volume
  int hlo[S::NHS];        // byte offset in a halo buffer, -1 past the halo
#pragma unroll
  for (int j = 0; j < S::NHS; j++) {
    const int vox = tid / G + j * VPI;
    const int hw = vox % S::HW, t = vox / S::HW, hh = t % S::HH, hd = t / S::HH;
    const int id = d0 - 1 + hd, ih = h0 - 1 + hh, iw = w0 - 1 + hw;
    const bool in = vox < S::HVOX && id >= 0 && id < p.D && ih >= 0 && ih < p.H && iw >= 0 && iw < p.W;
    hvi[j] = in ? (unsigned)((id * p.H + ih) * p.W + iw) : ~0u;
    hlo[j] = vox < S::HVOX ? ((hd * S::HH + hh) * S::RS + hw * PITCH + cg * 8) * 2 : -1;
  }
  const int64_t vol = (int64_t)p.D * p.H * p.W;
  E8 hval[S::NHS];
  f32x4 haff[4];
  // Request chunk ch's halo (NHS 16-byte loads) and the affine of this thread's 8
  // channels (4 loads): exactly NHL loads, zeros where a buffer range ends (padding
  // voxels, no affine, a chunk past the last). The loads are asm, so that the compiler
  // inserts no wait of its own for them (its count would ignore the weight DMAs issued
  // after them and drain those too); halo_store runs after an explicit wait.
  auto halo_issue = [&](int ch) {
    const int c0 = ch * CC;
    const bool live = ch < ce;
    const bool in0 = c0 < p.C0;
    const E* base = in0 ? p.x0 + b * vol * p.x0p : p.x1 + b * vol * p.x1p;
    const unsigned pitch2 = (unsigned)((in0 ? p.x0p : p.x1p) * 2);
    const i32x4 rs = dma_rsrc(base, live ? (unsigned)(vol * pitch2) : 0u);
    const unsigned cofs = (unsigned)(((in0 ? c0 : c0 - p.C0) + cg * 8) * 2);
#pragma unroll
    for (int j = 0; j < S::NHS; j++)
      hval[j] = buffer_load16_asm<E8>(rs, hvi[j] != ~0u ? hvi[j] * pitch2 + cofs : 0xfffffff0u);
    const i32x4 ra = dma_rsrc(p.affine ? p.affine + (int64_t)b * p.C * 2 : p.affine,
                              p.affine && live ? (unsigned)(p.C * 8) : 0u);
#pragma unroll
    for (int q = 0; q < 4; q++)
      haff[q] = __builtin_bit_cast(f32x4, buffer_load16_asm(ra, (unsigned)((c0 + cg * 8) * 8 + q * 16)));
  };
  // Write the requested halo into buffer `buf`: affine + SiLU in fp32, one fp16 rounding;
  // padding voxels stay zero. Called after the wait that covers halo_issue's loads.
  auto halo_store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < S::NHS; j++) pin_value(hval[j]);
#pragma unroll
    for (int q = 0; q < 4; q++) pin_value(haff[q]);
    char* hb = smem + buf * S::HALOP;
    const bool xf = p.affine != nullptr || p.silu;
#pragma unroll
    for (int j = 0; j < S::NHS; j++) {
      if (hlo[j] < 0) continue;
      E8 v = hval[j];
      if (xf) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float sc = p.affine ? haff[e >> 1][(e & 1) * 2] : 1.f;
          const float of = p.affine ? haff[e >> 1][(e & 1) * 2 + 1] : 0.f;
          float yv = (float)v[e] * sc + of;
          if (p.silu) yv = silu_f(yv);
          v[e] = hvi[j] != ~0u ? (E)yv : (E)0;
        }
      }
      *reinterpret_cast<E8*>(hb + hlo[j]) = v;
    }
  };

  // ---- direct halo: this thread's NR positions, 16-byte unit (r * 8 + wave) * 64 + lane
  // of a buffer; per position the source voxel (~0u for padding and for voxels outside the
  // volume) and the 8-channel group within the chunk.
  unsigned dvi[S::NR];
  unsigned dq[S::NR];
  {
    // Unsigned arithmetic throughout: the divisions by constants become multiply-shifts
    // without sign fix-ups.
    const unsigned u = (unsigned)(wave * 64 + lane) * 16u;
    const unsigned dd = (unsigned)p.D, hh_ = (unsigned)p.H, ww = (unsigned)p.W;
#pragma unroll
    for (int r = 0; r < S::NR; r++) {
      const unsigned pb = (unsigned)r * 8192u + u;
      const unsigned row = pb / (unsigned)(S::RS * 2), o = pb - row * (unsigned)(S::RS * 2);
      const unsigned hw = o / (unsigned)(PITCH * 2), q = (o - hw * (unsigned)(PITCH * 2)) / 16u;
      const unsigned hd = row / (unsigned)S::HH, hh = row - hd * (unsigned)S::HH;
      const unsigned id = (unsigned)(d0 - 1) + hd, ih = (unsigned)(h0 - 1) + hh, iw = (unsigned)(w0 - 1) + hw;
      // Bitwise tests, one unsigned compare per axis (id = -1 wraps past the bound), so the
      // selection compiles to masks rather than branches.
      const bool in = (row < (unsigned)(S::HD * S::HH)) & (hw < (unsigned)S::HW) & (q < (unsigned)G) & (id < dd) &
                      (ih < hh_) & (iw < ww);
      dvi[r] = in ? (id * hh_ + ih) * ww + iw : ~0u;
      dq[r] = q * 16u;
    }
  }
  // Chunk ch's halo into buffer buf: NR DMAs per thread (a chunk past this workgroup's
  // range reads zeros).
  auto halo_dma = [&](int ch, int buf) {
    const int c0 = ch * CC;
    const bool live = ch < ce;
    const bool in0 = c0 < p.C0;
    const E* base = in0 ? p.x0 + b * vol * p.x0p : p.x1 + b * vol * p.x1p;
    const unsigned pitch2 = (unsigned)((in0 ? p.x0p : p.x1p) * 2);
    const i32x4 rs = dma_rsrc(base, live ? (unsigned)(vol * pitch2) : 0u);
    const unsigned cb = (unsigned)((in0 ? c0 : c0 - p.C0) * 2);
    const unsigned dst = lds_offset(smem) + (unsigned)(buf * S::HALOP + wave * 1024);
#pragma unroll
    for (int r = 0; r < S::NR; r++)
      dma_buffer_b128(rs, dvi[r] != ~0u ? dvi[r] * pitch2 + cb + dq[r] : 0xfffffff0u, 0,
                      dst + (unsigned)(r * 8192));
  };

  // ---- weight ring: stage g = NSTG * chunk + (kd * 3 + kh) holds, at fragment
  // f = (kw * 2 + k) * NOBT + ob, the packed fragment of output block oblk * NOBT + ob, tap
  // (kd, kh, kw) and k-step 2 * chunk + k. Wave w moves fragments (w + 8 i) % NF (a repeat
  // moves the same data to the same place, so every wave issues LW loads per stage).
  const E* wsrc[S::LW];
  unsigned wdst[S::LW];
#pragma unroll
  for (int i = 0; i < S::LW; i++) {
    const int f = (wave + 8 * i) % S::NF;
    const int kw = f / (2 * S::NOBT), r = f % (2 * S::NOBT), k = r / S::NOBT, ob = r % S::NOBT;
    wsrc[i] = p.w + ((int64_t)((oblk * S::NOBT + ob) * 27 + kw) * p.NKC + k) * 512 + lane * 8;
    wdst[i] = lds_offset(smem) + (unsigned)(S::RING + f * 1024);
  }
  const int nst = p.nchunk * NSTG, gend = ce * NSTG;
  auto issue_stage = [&](int g) {
    // (Stages past the workgroup's last are not requested; the clamp keeps any index in
    // range.)
    const int gg = g < nst ? g : nst - 1;
    const int ch = gg / NSTG, t = gg - ch * NSTG;
    const int64_t off = ((int64_t)(t * 3) * p.NKC + 2 * ch) * 512;   // tap (kd, kh, 0) = 3 t
    const unsigned slot = (unsigned)((g % NSLOT) * S::STAGE);
#pragma unroll
    for (int i = 0; i < S::LW; i++) dma_b128(wsrc[i] + off, wdst[i] + slot);
  };

  // ---- operand bases: B at the lane's voxel, k-half and K-group in halo buffer 0; A at
  // the lane's 16 bytes of fragment (kw = 0, k = kg, ob = 2 wo) in ring slot 0.
  int bofs[2];
#pragma unroll
  for (int fv = 0; fv < 2; fv++) {
    const int vloc = (wv * 2 + fv) * 32 + (lane & 31);
    const int vw = vloc % TW, vh = (vloc / TW) % TH, vd = vloc / (TW * TH);
    bofs[fv] = ((vd * S::HH + vh) * S::RS + vw * PITCH + 8 * (lane >> 5) + kg * 16) * 2;
  }
  const char* aptr = smem + S::RING + (kg * S::NOBT + wo * 2) * 1024 + lane * 16;

  const int hf = lane >> 5;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  E8 ra[3][2], rb[3][2];   // operands of taps kw = 0, 1, 2: [kw][fo], [kw][fv]
  auto tap_off = [&](int kd, int kh, int kw) { return ((kd * S::HH + kh) * S::RS + kw * PITCH) * 2; };
  // A of tap kw of the stage at ring position `as`.
  auto load_a = [&](int kw, const char* as) {
#pragma unroll
    for (int fo = 0; fo < 2; fo++)
      ra[kw][fo] = *reinterpret_cast<const E8*>(as + (kw * 2 * S::NOBT + fo) * 1024);
  };
  // B of tap (kd, kh, kw) from halo buffer hb.
  auto load_b = [&](int kw, int kd, int kh, const char* hb) {
#pragma unroll
    for (int fv = 0; fv < 2; fv++) rb[kw][fv] = *reinterpret_cast<const E8*>(hb + bofs[fv] + tap_off(kd, kh, kw));
  };
  auto mfma_tap = [&](int kw) {
#pragma unroll
    for (int fo = 0; fo < 2; fo++)
#pragma unroll
      for (int fv = 0; fv < 2; fv++) acc[fo][fv] = mfma(ra[kw][fo], rb[kw][fv], acc[fo][fv]);
  };

  // Prologue: chunk 0's halo and the first three weight stages, one wait, then stage 0's
  // first operands.
  const int g0 = cb * NSTG;
  if constexpr (XF) halo_issue(cb);
  else halo_dma(cb, cb & 1);
  issue_stage(g0);
  issue_stage(g0 + 1);
  issue_stage(g0 + 2);
  vmcnt_wait<2 * S::LW>();   // the first halo and stage landed (the next two may be pending)
  if constexpr (XF) halo_store(cb & 1);
  __syncthreads();
#pragma unroll
  for (int kw = 0; kw < 3; kw++) {
    load_a(kw, aptr + (g0 % NSLOT) * S::STAGE);
    load_b(kw, 0, 0, smem + (cb & 1) * S::HALOP);
  }

  for (int ch = cb; ch < ce; ch++) {
    const char* hb = smem + (ch & 1) * S::HALOP;
    const char* hb_next = smem + ((ch + 1) & 1) * S::HALOP;
#pragma unroll
    for (int t = 0; t < NSTG; t++) {
      const int g = ch * NSTG + t;
      const int kd = t / 3, kh = t % 3;
      (void)kd; (void)kh;
      // taps 0 and 1 (operands read after the previous barrier)
      mfma_tap(0);
      mfma_tap(1);
      if constexpr (XF) {
        if (t == NSTG - 1 && ch + 1 < ce) {
          // The next chunk's halo, requested at stage HS, into the other buffer (last read
          // in chunk ch - 1); younger than it are the stages issued since.
          vmcnt_wait<(NSTG - 2 - HS) * S::LW>();
          halo_store((ch + 1) & 1);
        }
      }
      // Stage g + 1 has landed once only the loads issued after it may be pending: stage
      // g + 2's (none past this workgroup's last stage), and the next chunk's halo when it
      // was requested in between (none after the last chunk). (A directly copied halo has
      // landed with the stage after it, before this barrier.)
      const bool sp = g + 2 < gend, hp = (t == HS + 1 || t == HS + 2) && ch + 1 < ce;
      if (sp && hp) vmcnt_wait<S::LW + (XF ? S::NHL : S::NR)>();
      else if (sp) vmcnt_wait<S::LW>();
      else if (hp) vmcnt_wait<(XF ? S::NHL : S::NR)>();
      else vmcnt_wait<0>();
      __syncthreads();   // stage g + 1 visible; every wave done with stage g - 1's slot
      // Nothing is requested past the last stage and chunk: the epilogue would wait for it.
      if (g + 3 < gend) issue_stage(g + 3);
      if (t == HS && ch + 1 < ce) {
        // The next chunk's halo, into the buffer chunk ch - 1 used.
        if constexpr (XF) halo_issue(ch + 1);
        else halo_dma(ch + 1, (ch + 1) & 1);
      }
      // stage g + 1's operands (the next chunk's halo after the last stage): taps 0 and 1
      // while tap 2 of stage g runs, then tap 2 behind it
      const char* an = aptr + ((g + 1) % NSLOT) * S::STAGE;
      const char* hn = t + 1 < NSTG ? hb : hb_next;
      const int kdn = t + 1 < NSTG ? (t + 1) / 3 : 0, khn = t + 1 < NSTG ? (t + 1) % 3 : 0;
      load_a(0, an);
      load_b(0, kdn, khn, hn);
      load_a(1, an);
      load_b(1, kdn, khn, hn);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      mfma_tap(2);
      load_a(2, an);
      load_b(2, kdn, khn, hn);
    }
  }
  // Every request has landed before the LDS is reused or released.
  vmcnt_wait<0>();
  __syncthreads();   // every wave done with the halo buffers

  // ---- Epilogue rows. The wave's kept block is column block fv = kg: 32 voxels x 64
  // channels, summed (group 0 + group 1) from both K-groups' partial rows; lane l finishes
  // channels 8 (l % 8) .. + 7 of voxels l / 8 + 8 i, i < 4 (128 contiguous bytes per voxel,
  // 1 KB per store instruction when the 64 channels are the whole row). In the MFMA layout
  // lane (hf, col) holds voxel col, channels 32 fo + 8 j + 4 hf + r.
  const int col = lane & 31, g8 = lane & 7;
  const int o8 = oblk * BO + wo * 64 + g8 * 8;
  int64_t ovr[4];
  bool okr[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int vloc = (wv * 2 + kg) * 32 + (lane >> 3) + 8 * i;
    const int vw = vloc % TW, vh = (vloc / TW) % TH, vd = vloc / (TW * TH);
    const int od = d0 + vd, oh = h0 + vh, ow = w0 + vw;
    okr[i] = od < p.D && oh < p.H && ow < p.W;
    ovr[i] = (int64_t)b * vol + ((int64_t)od * p.H + oh) * p.W + ow;
  }
  // The epilogue operands of these rows -- bias (+ per-batch-item bias), fp16 shift and
  // residual -- requested before the partial rows are written, which hides their latency
  // (and none of these loads delays the prologue's DMA).
  const bool partial = p.split > 1;
  f32x4 bv0 = {0.f, 0.f, 0.f, 0.f}, bv1 = {0.f, 0.f, 0.f, 0.f};
  E8 sv = {};
  E8 res[4];
  if (p.bias && !partial) {
    const float* bias = p.bias + (p.bias_batched ? (int64_t)b * p.O : 0) + o8;
    bv0 = *reinterpret_cast<const f32x4*>(bias);
    bv1 = *reinterpret_cast<const f32x4*>(bias + 4);
  }
  if (p.shift && !partial) sv = *reinterpret_cast<const E8*>(p.shift + (int64_t)b * p.shiftp + o8);
#pragma unroll
  for (int i = 0; i < 4; i++)
    res[i] = p.res && !partial && okr[i] ? *reinterpret_cast<const E8*>(p.res + ovr[i] * p.resp + o8)
                                             : (E8){};
  // Both K-groups leave their partial sums as fp32 rows, [w4][fv][group][voxel][channel]
  // (rows padded to RP floats: 16-byte writes free of bank conflicts).
  float* rowsb = reinterpret_cast<float*>(smem);
  auto rowp = [&](int fv, int grp) { return rowsb + ((w4 * 2 + fv) * 2 + grp) * (32 * S::RP); };
#pragma unroll
  for (int fo = 0; fo < 2; fo++)
#pragma unroll
    for (int fv = 0; fv < 2; fv++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const f32x4 v = {acc[fo][fv][4 * j], acc[fo][fv][4 * j + 1], acc[fo][fv][4 * j + 2], acc[fo][fv][4 * j + 3]};
        *reinterpret_cast<f32x4*>(rowp(fv, kg) + col * S::RP + fo * 32 + 8 * j + 4 * hf) = v;
      }
  __syncthreads();
  // Rows fv = kg: (group 0 + group 1), then bias + shift, scale, residual, one rounding --
  // or, split over channel chunks, the fp32 sums of this range (the reduce finishes them).
  E8 outv[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int ro = ((lane >> 3) + 8 * i) * S::RP + g8 * 8;
    const float* r0 = rowp(kg, 0) + ro;
    const float* r1 = rowp(kg, 1) + ro;
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(r0) + *reinterpret_cast<const f32x4*>(r1);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(r0 + 4) + *reinterpret_cast<const f32x4*>(r1 + 4);
    if (partial) {
      if (okr[i]) {
        float* prow = p.part + ((int64_t)sk * p.B * vol + ovr[i]) * p.O + o8;
        *reinterpret_cast<f32x4*>(prow) = s0;
        *reinterpret_cast<f32x4*>(prow + 4) = s1;
      }
      continue;
    }
    E8& out = outv[i];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      out[e] = (E)((s0[e] + (bv0[e] + (float)sv[e])) * p.scale + (float)res[i][e]);
      out[e + 4] = (E)((s1[e] + (bv1[e] + (float)sv[e + 4])) * p.scale + (float)res[i][e + 4]);
    }
    if (okr[i]) *reinterpret_cast<E8*>(p.y + ovr[i] * p.yp + o8) = out;
  }
  // GroupNorm partial moments of the stored values, one block per brick: each wave's
  // 32 voxels x 32 channel pairs (lanes l, l + 8, ... hold the same 8 channels) into LDS
  // past the epilogue rows, then thread pp < BO / 2 merges pair pp over the waves of its
  // 64-channel half as a fixed tree.
  if (p.stats && !partial) {
    float* mst = reinterpret_cast<float*>(smem + S::EPI);   // [8 waves][32 pairs][3]
    pair_moments<4, 8>(outv, okr, mst + (wave * 32 + g8 * 4) * 3, lane < 8);
    __syncthreads();
    if (tid < BO / 2) {
      const int wo_p = tid >> 5, pp = tid & 31;
      // The waves of this 64-channel half, (K-group, voxel block), folded as a fixed tree.
      Moments m;
      if constexpr (S::WV == 4) {
        m = fold_moments<8>(mst + pp * 3, 32 * 3);
      } else {
        static_assert(S::WV == 2, "two or four voxel blocks per K-group");
        const Moments m0 = fold_moments<2>(mst + ((wo_p * 2) * 32 + pp) * 3, 32 * 3);
        const Moments m1 = fold_moments<2>(mst + ((4 + wo_p * 2) * 32 + pp) * 3, 32 * 3);
        m = merge_rcp(m0, m1);
      }
      float* dst = p.stats + (((int64_t)b * p.schunks + brick) * (p.O / 2) + oblk * (BO / 2) + tid) * 3;
      dst[0] = m.n; dst[1] = m.mean; dst[2] = m.m2;
    }
  }
}

template <int BO, int TD, int TH, int TW>
static int launch(StreamParams& p, hipStream_t st) {
  using S = Shape<BO, TD, TH, TW>;
  p.nob = p.O / BO;
  p.NBD = (p.D + TD - 1) / TD;
  p.NBH = (p.H + TH - 1) / TH;
  p.NBW = (p.W + TW - 1) / TW;
  const int64_t nbr = (int64_t)p.NBD * p.NBH * p.NBW;
  const int64_t nwg = nbr * p.nob * p.B;
  if (nwg * p.split > 0x7fffffff) return fail("conv3d: grid too large");
  p.nbr = (int)nbr;
  p.g1 = (int)nwg;
  p.dv_g1 = make_udiv((unsigned)p.g1);
  p.dv_nob = make_udiv((unsigned)p.nob);
  p.dv_nbr = make_udiv((unsigned)p.nbr);
  p.dv_nbw = make_udiv((unsigned)p.NBW);
  p.dv_nbh = make_udiv((unsigned)p.NBH);
  auto kern = p.affine || p.silu ? conv3s1_kernel<BO, TD, TH, TW, true> : conv3s1_kernel<BO, TD, TH, TW, false>;
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS) !=
      hipSuccess)
    return check_launch("conv3d (streamed): set LDS size");
  hipLaunchKernelGGL(kern, dim3((unsigned)(nwg * p.split)), dim3(NT), S::LDS, st, p);
  return check_launch("conv3d (streamed)");
}

struct Brick {
  int TD, TH, TW;
};

// Instantiated bricks per tile width (256 voxels for 64-channel tiles, 128 for 128-channel
// tiles; two halo buffers and the 4-slot ring must fit in 160 KB of LDS).
static const Brick kBricks64[] = {{4, 8, 8}, {8, 4, 8}};
static const Brick kBricks128[] = {{4, 4, 8}};

// Bricks launched (with partial-brick waste) for a volume; the halo volume breaks ties.
static int64_t brick_cost(const StreamParams& p, const Brick& k, int64_t* halo) {
  *halo = (int64_t)(k.TD + 2) * (k.TH + 2) * (k.TW + 2);
  return ceil_div64(p.D, k.TD) * ceil_div64(p.H, k.TH) * ceil_div64(p.W, k.TW);
}

}  // namespace cs

// Eligibility, tile and brick choice: false leaves the conv to conv3d_kernel.
bool conv3d_stream_plan(const ldx_conv3d_args* a, StreamParams* out, bool check_ws) {
  using namespace cs;
  if (const char* env = getenv("LDX_CONV_STREAM"))
    if (atoi(env) == 0) return false;
  if (a->ksize != 3 || a->stride != 1 || a->upsample || a->act != LDX_ACT_NONE) return false;
  if (a->c0 % CC || a->c1 % CC || a->out_c % 64) return false;
  if (a->c1 > 0 && !a->x1) return false;
  if (a->x0_pitch % 8 || (a->c1 > 0 && a->x1_pitch % 8)) return false;
  if ((uintptr_t)a->x0 % 16 || (a->c1 > 0 && (uintptr_t)a->x1 % 16)) return false;
  if (a->y_pitch % 8 || (uintptr_t)a->y % 16) return false;
  if (a->residual && (a->residual_pitch % 8 || (uintptr_t)a->residual % 16)) return false;
  if (a->shift && (a->shift_pitch % 8 || (uintptr_t)a->shift % 16)) return false;
  if (a->bias && (uintptr_t)a->bias % 16) return false;
  const int64_t vol = (int64_t)a->in_d * a->in_h * a->in_w;
  if (vol * a->x0_pitch * 2 >= ((int64_t)1 << 31)) return false;
  if (a->c1 > 0 && vol * a->x1_pitch * 2 >= ((int64_t)1 << 31)) return false;
  if ((int64_t)a->batch * vol >= ((int64_t)1 << 31)) return false;

  StreamParams& p = *out;
  p = StreamParams{};
  p.B = a->batch; p.D = a->in_d; p.H = a->in_h; p.W = a->in_w;
  p.C0 = a->c0; p.C1 = a->c1; p.C = a->c0 + a->c1; p.O = a->out_c;
  p.nchunk = p.C / CC;
  p.NKC = (p.C + 63) / 64 * 4;
  p.x0 = (const E*)a->x0; p.x0p = a->x0_pitch;
  p.x1 = a->c1 > 0 ? (const E*)a->x1 : p.x0; p.x1p = a->c1 > 0 ? a->x1_pitch : a->x0_pitch;
  p.w = (const E*)a->weight;
  p.bias = a->bias; p.bias_batched = a->bias_batched ? 1 : 0;
  p.shift = (const E*)a->shift; p.shiftp = a->shift_pitch;
  p.affine = a->affine; p.silu = a->silu ? 1 : 0;
  p.res = (const E*)a->residual; p.resp = a->residual_pitch;
  p.scale = a->output_scale;
  p.y = (E*)a->y; p.yp = a->y_pitch;

  // Among the tiles that launch at least 200 workgroups: the fewest launched voxel slots
  // (partial-brick waste), then the fewest halo voxels per output, then 128-channel tiles
  // (half the halo traffic per output channel).
  // LDX_CONV_STREAM_MIN_WG sets the fill threshold (tests use it to run small shapes
  // through this kernel) and, when set, also admits tiles whose workgroups, split over
  // ranges of channel chunks, reach about that many -- provided their bricks waste at
  // most a quarter of the launched voxels. (Split-K is not the default: on the UNet's
  // 16x20x20 level, 128 -> 128 channels, it measured 23.9 us with its reduce against
  // 16.2 us for the general kernel; every workgroup repays the fixed prologue and
  // epilogue for one or two chunks, and the fp32 partials cost a second pass.)
  int64_t min_wg = 200;
  int passes = 1;
  if (const char* env = getenv("LDX_CONV_STREAM_MIN_WG")) { min_wg = atoll(env); passes = 2; }
  const int64_t nvox = (int64_t)p.B * vol;
  for (int pass = 0; pass < passes && p.bo == 0; pass++) {
    int64_t best_slots = INT64_MAX, best_halo = INT64_MAX;
    for (int bo : {128, 64}) {
      if (p.O % bo) continue;
      const Brick* list = bo == 128 ? kBricks128 : kBricks64;
      const int bv = bo == 128 ? 128 : 256;
      for (int i = 0; i < (bo == 128 ? 1 : 2); i++) {
        int64_t halo;
        const int64_t nb = brick_cost(p, list[i], &halo);
        const int64_t g1 = nb * p.B * (p.O / bo);
        int split = 1, cps = p.nchunk;
        if (pass == 0) {
          if (g1 < min_wg) continue;
        } else {
          if (p.nchunk < 2 || nb * bv * 4 > nvox * 5) continue;
          const int64_t want = (min_wg + g1 - 1) / g1;
          cps = (int)((p.nchunk + want - 1) / want);
          split = (p.nchunk + cps - 1) / cps;
          if (split < 2 || g1 * split * 4 < min_wg * 3) continue;
        }
        const int64_t slots = nb * bv;
        const int64_t hpo = halo * 4096 / ((int64_t)bv * bo);
        if (slots < best_slots || (slots == best_slots && hpo < best_halo)) {
          best_slots = slots; best_halo = hpo; p.bo = bo;
          p.TD = list[i].TD; p.TH = list[i].TH; p.TW = list[i].TW;
          p.split = split; p.cps = cps;
        }
      }
    }
  }
  if (p.bo != 0 && p.split > 1) {
    const size_t need = (size_t)p.split * (size_t)nvox * (size_t)p.O * sizeof(float);
    if (check_ws && (!a->workspace || a->workspace_bytes < need)) return false;
    p.part = (float*)a->workspace;
  }
  if (p.bo != 0)
    p.schunks = (int)(ceil_div64(p.D, p.TD) * ceil_div64(p.H, p.TH) * ceil_div64(p.W, p.TW));
  return p.bo != 0;
}

int conv3d_stream_launch(StreamParams& p, hipStream_t st) {
  if (p.bo == 64) {
    if (p.TD == 4 && p.TH == 8 && p.TW == 8) return cs::launch<64, 4, 8, 8>(p, st);
    if (p.TD == 8 && p.TH == 4 && p.TW == 8) return cs::launch<64, 8, 4, 8>(p, st);
  } else if (p.bo == 128) {
    if (p.TD == 4 && p.TH == 4 && p.TW == 8) return cs::launch<128, 4, 4, 8>(p, st);
  }
  return fail("conv3d (streamed): no kernel for tile %d, brick %dx%dx%d", p.bo, p.TD, p.TH, p.TW);
}

}  // namespace LDX_ELEM_NS
}  // namespace ldx
