// K-quarter implicit-GEMM 3x3x3 stride-1 convolution on gfx950 MFMA
// (v_mfma_f32_32x32x16_f16 / _bf16) for volumes whose bricks of at most 224 voxels fill the
// GPU: input channels in 64-channel chunks, output channels in 64-channel tiles, 16-byte
// aligned NDHWC rows, with or without the GroupNorm affine + SiLU input transform.
//
// Workgroup: 8 waves, two per SIMD (one workgroup per CU). The workgroup owns one brick of
// V <= 224 voxels (NCOL = ceil(V / 32) MFMA columns) x 64 output channels. The two waves
// of SIMD s take the same quarter of the reduction -- channels 16 s .. 16 s + 15 of every
// 64-channel chunk, all 27 taps -- one for column group 0 (columns 0 .. NC0 - 1, NC0 =
// NCOL / 2), the other for group 1 (the rest), in 2 x NC accumulator tiles: per tap a wave
// reads 2 weight fragments and NC halo fragments for 2 NC MFMAs (a SIMD at NCOL = 7: 7 halo
// fragments from LDS and 4 weight fragments from L2 per 14 MFMAs, against one LDS fragment
// per MFMA for a 2 x 2 register block).
//
// Operands: the brick's halo (64 channels) is copied global -> LDS by DMA once per chunk
// (with the input transform: loaded into registers, transformed -- fp32 affine, SiLU, one
// fp16 rounding -- and written), in rows along W of 9 16-byte units per voxel (8 of
// channels, 1 of padding) with row and plane strides padded so that the halo unit of the
// brick's raster voxel v is 9 v (mod 16): any 16 consecutive voxels of a column hit 16
// distinct bank groups at every tap offset. Each tap's offset is a compile-time constant,
// so a halo fragment is one ds_read_b128 at a base register plus an immediate. The weight
// fragments come straight from global memory (L2) into registers, three taps ahead; the
// tap loop writes no LDS. The DMA path awaits the halo's first TD planes (all that the
// taps kd = 0 read) before the tap loop and the last two at tap TB.
//
// Epilogue: group 0 has fewer columns and leaves the tap loop first. Its waves reduce their
// columns while group 1 still runs MFMAs: quarter c owns column c, the other three leave
// their partial sums in LDS slots past the halo and count themselves in on an LDS counter;
// the owner adds the four quarters in order and finishes the column through LDS rows of
// its own. After the barrier that ends every tap loop, group 1's waves write their partial
// sums as fp32 voxel rows and every thread takes 8 consecutive channels of a voxel, adds
// the quarters in order and finishes it. Finishing: bias (+ per-batch-item bias) plus fp16
// shift, output scale, fp16 residual, one rounding, one 16-byte store (whole 128-byte rows
// per 8 lanes); optionally the GroupNorm moments of the stored values, one block per brick.
//
// Reference semantics: nax_conv3d (src/lesiondiffusion_mlx/_nax_conv.py:451-619), epilogue
// _nax_conv.py:265-270 (+ scaled variant :418-421).

#include "elem.h"
#include "conv3d_quad.h"

#include <cstdlib>

namespace ldx {
namespace LDX_ELEM_NS {
namespace cq {

constexpr int NT = 512;                 // 8 waves, two per SIMD
constexpr int KC = 64;                  // input channels per halo chunk
constexpr int PU = 9;                   // 16-byte units per halo voxel (8 + 1 of padding)
constexpr int RP = 68;                  // floats per epilogue row: 64 channels + 4 of padding
constexpr int NA = 4;                   // weight operand sets in flight (three taps ahead)
constexpr unsigned OOB = 0xfffffff0u;   // a buffer offset past every extent: reads zeros
constexpr int TB = 4;                   // tap at whose start the halo's last planes are awaited

// Smallest x >= base with x = r (mod 16).
constexpr int up16(int base, int r) { return base + ((r - base) % 16 + 16) % 16; }

template <int TD, int TH, int TW>
struct QShape {
  static constexpr int V = TD * TH * TW;            // voxels per brick
  static constexpr int NCOL = (V + 31) / 32;        // 32-voxel MFMA columns
  static_assert(NCOL <= 7, "at most seven columns (224 voxels) per brick");
  // Column groups: group 0 takes columns [0, NC0), group 1 [NC0, NCOL). Group 0 is the
  // smaller: its waves finish the tap loop first and reduce their columns while group 1
  // still runs MFMAs.
  static constexpr int NC0 = NCOL / 2, NC1 = NCOL - NC0;
  static_assert(NC1 <= 4, "at most four columns per group");
  static constexpr int HD = TD + 2, HH = TH + 2, HW = TW + 2;
  // Unit of brick voxel (vd, vh, vw) in the halo: vd PSU + vh RSU + vw PU, which is 9 v
  // (mod 16) for the voxel's raster index v = (vd TH + vh) TW + vw.
  static constexpr int RU = HW * PU;                // units of a row holding voxels
  static constexpr int RDMA = (RU + 63) / 64;       // 64-lane DMAs per row
  static constexpr int RLAST = RU - 64 * (RDMA - 1);   // lanes of a row's last DMA
  static constexpr int RSU = up16(RU, (9 * TW) % 16);
  static constexpr int PSU = up16(HH * RSU, (9 * TW * TH) % 16);
  static constexpr int HALO = HD * PSU * 16;
  static constexpr int NROW = HD * HH;              // halo rows (along W)
  static constexpr int RPW = (NROW + 7) / 8;        // rows per wave
  static constexpr int NXU = NROW * HW * 8;          // 16-byte data units of a halo
  static constexpr int XPT = (NXU + NT - 1) / NT;    // of them per thread (input transform)
  // Group 0's exchange, past the halo: for each of its columns, the partial sums of the
  // three quarters that do not own it (8 KB each, in the MFMA lane layout), then a counter.
  static constexpr int G0X = HALO;
  static constexpr int CNT = G0X + NC0 * 3 * 8192;
  // Group 1's epilogue rows (after the barrier that ends the tap loops): [quarter][column]
  // [voxel] rows of RP floats; the GroupNorm moments past them.
  static constexpr int EPI = 4 * 4 * 32 * RP * 4;
  static constexpr int MST = EPI;
  static constexpr int LDS = CNT + 16 > MST + 8 * 32 * 3 * 4 ? CNT + 16 : MST + 8 * 32 * 3 * 4;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert((2 * PSU + 2 * RSU + 2 * PU) * 16 < 65536, "tap offsets fit the ds_read immediate");
};

__device__ __forceinline__ f32x16 mfma(E8 a, E8 b, f32x16 c) { return mfma_e(a, b, c); }

template <int TD, int TH, int TW, bool XF>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void conv3q_kernel(QuadParams p) {
  touch_args(p);
  using S = QShape<TD, TH, TW>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int sq = wave & 3, grp = wave >> 2;   // reduction quarter, column group

  // Workgroup -> (output tile, brick, batch item); each XCD (workgroups are dealt to the 8
  // XCDs round-robin) receives a contiguous range, so neighbouring halos meet in its L2.
  int wg;
  {
    const int n = gridDim.x, l = blockIdx.x, per = n >> 3, rem = n & 7, x = l & 7, k = l >> 3;
    wg = x * per + min(x, rem) + k;
  }
  const int q1 = udiv(wg, p.dv_nob);
  const int oblk = wg - q1 * p.nob;
  const int b = udiv(q1, p.dv_nbr);
  const int brick = q1 - b * p.nbr;
  const int bt = udiv(brick, p.dv_nbw), bw_i = brick - bt * p.NBW;
  const int bd_i = udiv(bt, p.dv_nbh), bh_i = bt - bd_i * p.NBH;
  const int d0 = bd_i * TD, h0 = bh_i * TH, w0 = bw_i * TW;
  const int vol = p.D * p.H * p.W;

  // ---- halo DMA lanes: unit u = 64 h + lane of a halo row is voxel hw = u / PU, 16-byte
  // channel group q = u % PU. The padding unit q = 8 loads zeros (it is never read); so do
  // voxels outside the volume, which are the conv's zero padding. A row's last DMA runs on
  // its first RLAST lanes only, so that no DMA writes past its row.
  bool lok[S::RDMA];
  unsigned lpos[S::RDMA];
#pragma unroll
  for (int h = 0; h < S::RDMA; h++) {
    const int u = 64 * h + lane, hw = u / PU, q = u - hw * PU;
    const int iw = w0 - 1 + hw;
    lok[h] = q < 8 && (unsigned)iw < (unsigned)p.W;
    lpos[h] = (unsigned)(iw * 65536 + q * 16);   // voxel along W, byte of its channel group
  }
  // Chunk j's halo: the wave's rows r = wave + 8 i, RDMA DMAs of 1 KB each; first the rows
  // of planes 0 .. TD - 1 (all the taps kd = 0 read), then the last two planes. Returns the
  // number of DMAs of the second part.
  auto halo_dma = [&](int j) {
    const int c0 = j * KC;
    const bool in0 = c0 < p.C0;
    const E* base = in0 ? p.x0 + (int64_t)b * vol * p.x0p : p.x1 + (int64_t)b * vol * p.x1p;
    const unsigned pitch2 = (unsigned)((in0 ? p.x0p : p.x1p) * 2);
    const i32x4 rs = dma_rsrc(base, (unsigned)vol * pitch2);
    const unsigned cb = (unsigned)((in0 ? c0 : c0 - p.C0) * 2);
    unsigned lo[S::RDMA];
#pragma unroll
    for (int h = 0; h < S::RDMA; h++) lo[h] = (lpos[h] >> 16) * pitch2 + (lpos[h] & 0xffffu) + cb;
    unsigned m0[S::RPW], roff[S::RPW];
    bool rowok[S::RPW];
    {
      int hd = wave / S::HH, hh = wave % S::HH;
#pragma unroll
      for (int i = 0; i < S::RPW; i++) {
        const int id = d0 - 1 + hd, ih = h0 - 1 + hh;
        rowok[i] = wave + 8 * i < S::NROW && (unsigned)id < (unsigned)p.D && (unsigned)ih < (unsigned)p.H;
        roff[i] = (unsigned)((id * p.H + ih) * p.W) * pitch2;
        m0[i] = lds_offset(smem) + (unsigned)(hd * S::PSU + hh * S::RSU) * 16u;
        hh += 8;
#pragma unroll
        for (int k = 0; k < 8 / S::HH + 1; k++)
          if (hh >= S::HH) { hh -= S::HH; hd += 1; }
      }
    }
    int late = 0;
#pragma unroll
    for (int part = 0; part < 2; part++) {
#pragma unroll
      for (int h = 0; h < S::RDMA - 1; h++)
#pragma unroll
        for (int i = 0; i < S::RPW; i++) {
          const int r = wave + 8 * i;
          if (r < S::NROW && (r < TD * S::HH) == (part == 0))
            dma_buffer_b128(rs, rowok[i] && lok[h] ? lo[h] + roff[i] : OOB, 0, m0[i] + 1024u * h);
        }
      if (lane < S::RLAST) {
        constexpr int h = S::RDMA - 1;
#pragma unroll
        for (int i = 0; i < S::RPW; i++) {
          const int r = wave + 8 * i;
          if (r < S::NROW && (r < TD * S::HH) == (part == 0))
            dma_buffer_b128(rs, rowok[i] && lok[h] ? lo[h] + roff[i] : OOB, 0, m0[i] + 1024u * h);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < S::RPW; i++) {
      const int r = wave + 8 * i;
      if (r < S::NROW && r >= TD * S::HH) late += S::RDMA;
    }
    return late;
  };

  // Chunk j's halo through registers with the GroupNorm affine + SiLU prologue: unit
  // u = i * NT + tid is halo row u / (HW * 8), voxel (u / 8) % HW, channel group u % 8 =
  // tid % 8 (one affine per thread). The arithmetic is the streamed kernel's (fp32 multiply-
  // add, silu_f, one rounding); voxels outside the volume are zero after the transform
  // (the conv pads the normalised input). The loads are asm, awaited explicitly. Units
  // below XNA are the first TD planes (all that the taps kd = 0 read): they are staged
  // before the tap loop; the last two planes' units are loaded with them and transformed
  // at tap TB, beside the MFMAs, as the DMA path awaits its last planes there.
  constexpr int XNA = TD * S::HH * S::HW * 8;            // units of the first TD planes
  constexpr int XA = (XNA + NT - 1) / NT;                // of them per thread
  constexpr int XL = (S::NXU - XNA + NT - 1) / NT;       // late units per thread
  f32x4 xaf[4];
  auto xf_affine = [&](int j) {
    const int c0 = j * KC, q = tid & 7;
    const i32x4 ra = dma_rsrc(p.affine ? p.affine + (int64_t)b * p.C * 2 : p.affine, p.affine ? (unsigned)(p.C * 8) : 0u);
#pragma unroll
    for (int k = 0; k < 4; k++) xaf[k] = __builtin_bit_cast(f32x4, buffer_load16_asm(ra, (unsigned)((c0 + q * 8) * 8 + k * 16)));
  };
  // Load unit u (u >= NXU: none) of chunk j: its value, LDS destination (-1: none) and
  // whether it lies inside the volume.
  auto xf_load = [&](int j, int u, E8& v, int& dst, bool& in) {
    const int c0 = j * KC;
    const bool in0 = c0 < p.C0;
    const E* base = in0 ? p.x0 + (int64_t)b * vol * p.x0p : p.x1 + (int64_t)b * vol * p.x1p;
    const unsigned pitch2 = (unsigned)((in0 ? p.x0p : p.x1p) * 2);
    const i32x4 rs = dma_rsrc(base, (unsigned)vol * pitch2);
    const unsigned cb = (unsigned)((in0 ? c0 : c0 - p.C0) * 2);
    const int q = tid & 7;
    const int r = u / (S::HW * 8), hw = (u / 8) % S::HW;
    const int hd = r / S::HH, hh = r - hd * S::HH;
    const int id = d0 - 1 + hd, ih = h0 - 1 + hh, iw = w0 - 1 + hw;
    in = u < S::NXU && (unsigned)id < (unsigned)p.D && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
    dst = u < S::NXU ? (hd * S::PSU + hh * S::RSU + hw * PU + q) * 16 : -1;
    v = buffer_load16_asm<E8>(rs, in ? (unsigned)((id * p.H + ih) * p.W + iw) * pitch2 + cb + q * 16 : OOB);
  };
  // Transform a loaded unit and write it to the halo.
  auto xf_store = [&](E8 v, int dst, bool in) {
    pin_value(v);
    if (dst < 0) return;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float sc = p.affine ? xaf[e >> 1][(e & 1) * 2] : 1.f;
      const float of = p.affine ? xaf[e >> 1][(e & 1) * 2 + 1] : 0.f;
      float yv = (float)v[e] * sc + of;
      if (p.silu) yv = silu_f(yv);
      v[e] = in ? (E)yv : (E)0;
    }
    *reinterpret_cast<E8*>(smem + dst) = v;
  };
  // The first TD planes of chunk j: all at once when no accumulator is live (chunk 0),
  // else in two batches, so that the staging fits beside the live accumulators.
  auto xf_early = [&](int j, bool batched) __attribute__((always_inline)) {
    constexpr int XB1 = (XA + 1) / 2;
    if (!batched) {
      E8 xv[XA];
      int dst[XA];
      bool in[XA];
#pragma unroll
      for (int i = 0; i < XA; i++) xf_load(j, i * NT + tid < XNA ? i * NT + tid : S::NXU, xv[i], dst[i], in[i]);
      vmcnt_wait<0>();
#pragma unroll
      for (int k = 0; k < 4; k++) pin_value(xaf[k]);
#pragma unroll
      for (int i = 0; i < XA; i++) xf_store(xv[i], dst[i], in[i]);
    } else {
#pragma unroll
      for (int b0 = 0; b0 < XA; b0 += XB1) {
        E8 xv[XB1];
        int dst[XB1];
        bool in[XB1];
#pragma unroll
        for (int ii = 0; ii < XB1; ii++) {
          const int u = (b0 + ii) * NT + tid;
          xf_load(j, b0 + ii < XA && u < XNA ? u : S::NXU, xv[ii], dst[ii], in[ii]);
        }
        vmcnt_wait<0>();
#pragma unroll
        for (int k = 0; k < 4; k++) pin_value(xaf[k]);
#pragma unroll
        for (int ii = 0; ii < XB1; ii++) xf_store(xv[ii], dst[ii], in[ii]);
      }
    }
  };
  // The late units travel raw by DMA into a staging area over group 0's exchange slots
  // (unused until the last chunk's tap loop ends), unit i * NT + tid of the late range at
  // 16 (i * NT + tid): each thread reads back exactly what its own DMA wrote.
  static_assert(S::G0X + XL * NT * 16 <= S::CNT || S::NC0 == 0, "late staging within the exchange slots");
  auto xf_unit = [&](int u, unsigned& off, int& dst, bool& in) {
    const int q = tid & 7;
    const int r = u / (S::HW * 8), hw = (u / 8) % S::HW;
    const int hd = r / S::HH, hh = r - hd * S::HH;
    const int id = d0 - 1 + hd, ih = h0 - 1 + hh, iw = w0 - 1 + hw;
    in = u < S::NXU && (unsigned)id < (unsigned)p.D && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
    dst = u < S::NXU ? (hd * S::PSU + hh * S::RSU + hw * PU + q) * 16 : -1;
    off = (unsigned)((id * p.H + ih) * p.W + iw);
  };
  auto xf_late_load = [&](int j) {
    const int c0 = j * KC;
    const bool in0 = c0 < p.C0;
    const E* base = in0 ? p.x0 + (int64_t)b * vol * p.x0p : p.x1 + (int64_t)b * vol * p.x1p;
    const unsigned pitch2 = (unsigned)((in0 ? p.x0p : p.x1p) * 2);
    const i32x4 rs = dma_rsrc(base, (unsigned)vol * pitch2);
    const unsigned cb = (unsigned)((in0 ? c0 : c0 - p.C0) * 2);
#pragma unroll
    for (int i = 0; i < XL; i++) {
      unsigned off;
      int dst;
      bool in;
      xf_unit(XNA + i * NT + tid, off, dst, in);
      dma_buffer_b128(rs, in ? off * pitch2 + cb + (tid & 7) * 16 : OOB, 0,
                      lds_offset(smem) + (unsigned)(S::G0X + (i * NT + wave * 64) * 16));
    }
  };
  auto xf_late_store = [&]() {
#pragma unroll
    for (int i = 0; i < XL; i++) {
      unsigned off;
      int dst;
      bool in;
      xf_unit(XNA + i * NT + tid, off, dst, in);
      xf_store(*reinterpret_cast<const E8*>(smem + S::G0X + (i * NT + tid) * 16), dst, in);
    }
  };

  // ---- weight fragments: (tile o, tap t, k-step 4 j + sq) of output block 2 oblk + o,
  // 1 KB each, the lane's 16 bytes at lane * 16. wa walks the taps of a chunk.
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, (unsigned)(p.O * 27 * p.NKC * 32));
  const unsigned voffa = (unsigned)(lane * 16 + sq * 1024);
  E8 aq[NA][2];
  unsigned wa = 0, wstep = 0, wob = 0;
  auto load_a = [&](E8(&dst)[2]) {
    dst[0] = as_e8(buffer_load16(wr, voffa, wa));
    dst[1] = as_e8(buffer_load16(wr, voffa, wa + wob));
    wa += wstep;
  };

  f32x16 acc[4][2];
  int* cnt = reinterpret_cast<int*>(smem + S::CNT);
  if (tid == 0) *cnt = 0;   // ordered before its use by the barrier of the first chunk

  // The wave's column group G (NC columns from CB), all chunks.
  auto body = [&](auto gc) {
    constexpr int G = decltype(gc)::value;
    constexpr int NC = G == 0 ? S::NC0 : S::NC1, CB = G == 0 ? 0 : S::NC0;
    // ---- halo fragments: column CB + c's lane reads voxel min(32 (CB + c) + lane % 32,
    // V - 1), channels 16 sq + 8 (lane / 32) .. + 7.
    int bb[NC > 0 ? NC : 1];
#pragma unroll
    for (int c = 0; c < NC; c++) {
      int v = 32 * (CB + c) + (lane & 31);
      if (v > S::V - 1) v = S::V - 1;
      const int vw = v % TW, vh = (v / TW) % TH, vd = v / (TW * TH);
      bb[c] = ((vd * S::PSU + vh * S::RSU + vw * PU) + 2 * sq + (lane >> 5)) * 16;
    }
    E8 bq[2][NC > 0 ? NC : 1];

    // One 64-channel chunk: its halo by DMA and the first three taps' weights, one wait and
    // barrier, then the 27 taps. FIRST: the accumulators start from the first MFMA (C = 0).
    auto run_chunk = [&](int j, auto first) {
      constexpr bool FIRST = decltype(first)::value;
      // With the input transform the first TD planes are staged through registers first,
      // while no weight operands are held (a later chunk's staging runs beside live
      // accumulators); the last two planes' loads follow the first taps' weights and stay
      // in flight into the tap loop.
      if constexpr (XF) {
        xf_affine(j);
        xf_early(j, !FIRST);
      }
      const int late = XF ? 0 : halo_dma(j);
      if constexpr (NC > 0) {
        // Per-chunk weight walk; the asm keeps the step opaque, so that no tap's offset is
        // computed once outside the chunk loop and held for the whole kernel.
        wstep = (unsigned)__builtin_amdgcn_readfirstlane(p.NKC * 1024);
        asm volatile("" : "+s"(wstep));
        wob = 27u * wstep;
        wa = (unsigned)(oblk * 2) * wob + (unsigned)(4 * j * 1024);
#pragma unroll
        for (int t = 0; t < NA - 1; t++) load_a(aq[t]);
      }
      if constexpr (XF) xf_late_load(j);
      if constexpr (XF) {
        // The early planes are written (their loads awaited above); the late ones and the
        // weight requests stay in flight.
      } else if constexpr (NC > 0) {
        // The first TD planes of the halo have landed once at most the last planes' DMAs
        // and the weight requests are in flight (the count is wave-uniform).
        static_assert(2 * S::RDMA <= 8, "late DMA counts handled below");
        if (late == 0) vmcnt_wait<(NA - 1) * 2>();
        else if (late == S::RDMA) vmcnt_wait<(NA - 1) * 2 + S::RDMA>();
        else vmcnt_wait<(NA - 1) * 2 + 2 * S::RDMA>();
      } else {
        vmcnt_wait<0>();
      }
      __syncthreads();
      if constexpr (NC == 0) {
        if constexpr (XF) {
          vmcnt_wait<0>();
          xf_late_store();
        }
        __syncthreads();   // the tap loop's barrier
      }
      if constexpr (NC > 0) {
#pragma unroll
        for (int c = 0; c < NC; c++) bq[0][c] = *reinterpret_cast<const E8*>(smem + bb[c]);
#pragma unroll
        for (int t = 0; t < 27; t++) {
          if (t == TB) {
            // The last planes, first read by the taps kd = 1 (whose fragments are requested
            // from tap 8 on): every wave's DMAs (or late loads) have landed once its weight
            // requests older than tap TB's have; with the input transform each thread then
            // writes its late units.
            vmcnt_wait<(NA - 1) * 2>();
            if constexpr (XF) xf_late_store();
            __syncthreads();
          }
          // Issue order, pinned by scheduling barriers: per column the MFMA pair of this
          // tap, then that column's halo fragment of the next tap (it has a tap of MFMAs to
          // land in); the weight requests after the first pair.
          const int kd = (t + 1) / 9, kh = ((t + 1) / 3) % 3, kw = (t + 1) % 3;
          const int toff = (kd * S::PSU + kh * S::RSU + kw * PU) * 16;
#pragma unroll
          for (int c = 0; c < NC; c++) {
#pragma unroll
            for (int o = 0; o < 2; o++) {
              if (FIRST && t == 0) acc[c][o] = mfma(aq[0][o], bq[0][c], (f32x16){});
              else acc[c][o] = mfma(aq[t % NA][o], bq[t & 1][c], acc[c][o]);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (t + 1 < 27) bq[(t + 1) & 1][c] = *reinterpret_cast<const E8*>(smem + bb[c] + toff);
            if (c == 0 && t + NA - 1 < 27) load_a(aq[(t + NA - 1) % NA]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    };
    run_chunk(0, std::true_type{});
    for (int j = 1; j < p.nchunk; j++) {
      __syncthreads();   // every wave done with the previous chunk's halo
      run_chunk(j, std::false_type{});
    }
  };
  if (grp == 0) body(std::integral_constant<int, 0>{});
  else body(std::integral_constant<int, 1>{});

  // ---- epilogue operands: bias (+ per-batch-item bias) + fp16 shift of the thread's 8
  // channels (channels 8 (lane % 8) .. + 7 of the tile in every row layout below)
  const int col = lane & 31, hf = lane >> 5, g8 = tid & 7;
  const int o8 = oblk * 64 + g8 * 8;
  float bs[8];
  {
    f32x4 bv0 = {0.f, 0.f, 0.f, 0.f}, bv1 = {0.f, 0.f, 0.f, 0.f};
    E8 sv = {};
    if (p.bias) {
      const float* bias = p.bias + (p.bias_batched ? b * p.O : 0) + o8;
      bv0 = *reinterpret_cast<const f32x4*>(bias);
      bv1 = *reinterpret_cast<const f32x4*>(bias + 4);
    }
    if (p.shift) sv = *reinterpret_cast<const E8*>(p.shift + (int64_t)b * p.shiftp + o8);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      bs[e] = bv0[e] + (float)sv[e];
      bs[e + 4] = bv1[e] + (float)sv[e + 4];
    }
  }
  // Outputs and residual rows through buffer resources (32-bit byte offsets).
  const __amdgpu_buffer_rsrc_t yr = make_rsrc(p.y, (unsigned)(p.B * vol) * (unsigned)p.yp * 2u);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(p.res, p.res ? (unsigned)(p.B * vol) * (unsigned)p.resp * 2u : 0u);
  const bool has_res = p.res != nullptr, scaled = p.scale != 1.0f;
  // The stored values and their validity, kept for the GroupNorm moments: units 0..3 of a
  // group-0 owner, units 4..5 of the final round.
  E8 outv[6] = {};
  bool okv[6] = {false, false, false, false, false, false};
  // Output voxel of brick voxel v (okv: inside the volume), and its residual row.
  auto locate = [&](int v, bool valid, unsigned& ovr, E8& res) {
    const int vd = v / (TW * TH), rv = v - vd * (TW * TH), vh = rv / TW, vw = rv - vh * TW;
    const int od = d0 + vd, oh = h0 + vh, ow = w0 + vw;
    const bool ok = valid && v < S::V && od < p.D && oh < p.H && ow < p.W;
    ovr = (unsigned)(b * vol + (od * p.H + oh) * p.W + ow);
    res = (E8){};
    if (has_res && ok) res = buffer_load16<E8>(rr, (ovr * (unsigned)p.resp + o8) * 2u);
    return ok;
  };
  // One row of summed partials (8 channels at r0, 8 at r0 + 4): bias, shift, scale,
  // residual, one rounding, one 16-byte store.
  auto finish = [&](f32x4 s0, f32x4 s1, const E8& res, unsigned ovr, E8& out) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      f[e] = s0[e] + bs[e];
      f[e + 4] = s1[e] + bs[e + 4];
    }
    if (scaled) {
#pragma unroll
      for (int e = 0; e < 8; e++) f[e] *= p.scale;
    }
    if (has_res) {
#pragma unroll
      for (int e = 0; e < 8; e++) f[e] += (float)res[e];
    }
#pragma unroll
    for (int e = 0; e < 8; e++) out[e] = (E)f[e];
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, out), yr, (int)((ovr * (unsigned)p.yp + o8) * 2u),
                                           0, 0);
  };
  // Partial sums of column c's tile o as four 16-byte pieces per lane (MFMA layout) at
  // slot base sb: piece jj of lane l at sb + ((o * 4 + jj) * 64 + l) * 16.
  float* rows = reinterpret_cast<float*>(smem);

  // ---- group 0: reduce its columns while group 1 still runs its tap loop. Column c's
  // owner is quarter c; the other three quarters leave their sums in the owner's slots,
  // count themselves in, and the owner waits for all four, adds the quarters in order, and
  // finishes the column through rows of its own (the slots it has read).
  if constexpr (S::NC0 > 0) {
    if (grp == 0) {
      char* g0x = smem + S::G0X;
#pragma unroll
      for (int c = 0; c < S::NC0; c++) {
        if (c == sq) continue;
        const int k = sq < c ? sq : sq - 1;
        char* sb = g0x + (c * 3 + k) * 8192;
#pragma unroll
        for (int o = 0; o < 2; o++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const f32x4 v = {acc[c][o][4 * jj], acc[c][o][4 * jj + 1], acc[c][o][4 * jj + 2], acc[c][o][4 * jj + 3]};
            *reinterpret_cast<f32x4*>(sb + ((o * 4 + jj) * 64 + lane) * 16) = v;
          }
      }
      // The writes above are performed before the count (LDS requests of a wave complete
      // in order); the owner reads the slots only after all four quarters counted in.
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
      if (lane == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      while (__hip_atomic_load(cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < 4) __builtin_amdgcn_s_sleep(1);
      auto owner = [&](auto cc) {
        constexpr int C = decltype(cc)::value;
        char* sb = g0x + C * 3 * 8192;
        f32x16 sum[2];
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
          for (int o = 0; o < 2; o++) {
            f32x16 v;
            if (q == C) {
              v = acc[C][o];
            } else {
              const char* src = sb + (q < C ? q : q - 1) * 8192;
#pragma unroll
              for (int jj = 0; jj < 4; jj++) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(src + ((o * 4 + jj) * 64 + lane) * 16);
                v[4 * jj] = x[0]; v[4 * jj + 1] = x[1]; v[4 * jj + 2] = x[2]; v[4 * jj + 3] = x[3];
              }
            }
            sum[o] = q == 0 ? v : sum[o] + v;
          }
        // The column's 32 voxels, transposed into rows over the slots just read.
        float* tr = reinterpret_cast<float*>(sb);
#pragma unroll
        for (int o = 0; o < 2; o++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const f32x4 v = {sum[o][4 * jj], sum[o][4 * jj + 1], sum[o][4 * jj + 2], sum[o][4 * jj + 3]};
            *reinterpret_cast<f32x4*>(tr + col * RP + 32 * o + 8 * jj + 4 * hf) = v;
          }
        unsigned ovr[4];
        E8 res[4];
#pragma unroll
        for (int i = 0; i < 4; i++) okv[i] = locate(32 * C + (lane >> 3) + 8 * i, true, ovr[i], res[i]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          if (!okv[i]) continue;
          const float* r0 = tr + ((lane >> 3) + 8 * i) * RP + g8 * 8;
          finish(*reinterpret_cast<const f32x4*>(r0), *reinterpret_cast<const f32x4*>(r0 + 4), res[i], ovr[i],
                 outv[i]);
        }
      };
      if (sq == 0) owner(std::integral_constant<int, 0>{});
      if constexpr (S::NC0 > 1) if (sq == 1) owner(std::integral_constant<int, 1>{});
      if constexpr (S::NC0 > 2) if (sq == 2) owner(std::integral_constant<int, 2>{});
    }
  }

  // ---- group 1's columns, after every tap loop: the four group-1 waves write their
  // partial sums as rows [quarter][column][voxel]; any thread then takes 8 channels of a
  // voxel (units i = 0, 1: row 64 i + tid / 8), adds the quarters in order and finishes.
  {
    unsigned ovr[2];
    E8 res[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int r = 64 * i + (tid >> 3);
      okv[4 + i] = locate(32 * S::NC0 + r, (r >> 5) < S::NC1, ovr[i], res[i]);
    }
    __syncthreads();   // every wave done with the halo and the group-0 exchange
    if (grp == 1) {
#pragma unroll
      for (int cl = 0; cl < S::NC1; cl++)
#pragma unroll
        for (int o = 0; o < 2; o++)
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const f32x4 v = {acc[cl][o][4 * jj], acc[cl][o][4 * jj + 1], acc[cl][o][4 * jj + 2], acc[cl][o][4 * jj + 3]};
            *reinterpret_cast<f32x4*>(rows + ((sq * 4 + cl) * 32 + col) * RP + 32 * o + 8 * jj + 4 * hf) = v;
          }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; i++) {
      if (!okv[4 + i]) continue;
      const float* r0 = rows + (64 * i + (tid >> 3)) * RP + g8 * 8;
      f32x4 s0 = *reinterpret_cast<const f32x4*>(r0);
      f32x4 s1 = *reinterpret_cast<const f32x4*>(r0 + 4);
#pragma unroll
      for (int w = 1; w < 4; w++) {
        const float* rw = r0 + w * 4 * 32 * RP;
        s0 += *reinterpret_cast<const f32x4*>(rw);
        s1 += *reinterpret_cast<const f32x4*>(rw + 4);
      }
      finish(s0, s1, res[i], ovr[i], outv[4 + i]);
    }
  }

  // GroupNorm partial moments of the stored values, one block per brick: each wave's
  // channel pairs over its voxels (lanes l, l + 8, ... hold the same 8 channels) into LDS
  // past the epilogue rows, then thread pp < 32 merges pair pp over the eight waves (a fixed tree).
  if (p.stats) {
    float* mst = reinterpret_cast<float*>(smem + S::MST);   // [8 waves][32 pairs][3]
    pair_moments<6, 8>(outv, okv, mst + (wave * 32 + g8 * 4) * 3, lane < 8);
    __syncthreads();
    if (tid < 32) {
      const Moments m = fold_moments<8>(mst + tid * 3, 32 * 3);   // the eight waves, a fixed tree
      float* dst = p.stats + (((int64_t)b * p.schunks + brick) * (p.O / 2) + oblk * 32 + tid) * 3;
      dst[0] = m.n; dst[1] = m.mean; dst[2] = m.m2;
    }
  }
}

template <int TD, int TH, int TW>
static int launch(QuadParams& p, hipStream_t st) {
  using S = QShape<TD, TH, TW>;
  p.dv_nob = make_udiv((unsigned)p.nob);
  p.dv_nbr = make_udiv((unsigned)p.nbr);
  p.dv_nbw = make_udiv((unsigned)p.NBW);
  p.dv_nbh = make_udiv((unsigned)p.NBH);
  auto kern = p.affine || p.silu ? conv3q_kernel<TD, TH, TW, true> : conv3q_kernel<TD, TH, TW, false>;
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS) != hipSuccess)
    return check_launch("conv3d (K-quarter): set LDS size");
  const int64_t nwg = (int64_t)p.nbr * p.nob * p.B;
  hipLaunchKernelGGL(kern, dim3((unsigned)nwg), dim3(NT), S::LDS, st, p);
  return check_launch("conv3d (K-quarter)");
}

struct QBrick {
  int TD, TH, TW;
};
static const QBrick kQBricks[] = {{4, 5, 10}};

}  // namespace cq

bool conv3d_quad_plan(const ldx_conv3d_args* a, QuadParams* out) {
  using namespace cq;
  int force = -1;
  if (const char* env = getenv("LDX_CONV_QUAD")) force = atoi(env);
  if (force == 0) return false;
  if (a->ksize != 3 || a->stride != 1 || a->upsample || a->act != LDX_ACT_NONE) return false;
  if (a->c0 % KC || a->c1 % KC || a->out_c % 64) return false;
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
  if ((int64_t)a->batch * vol * a->y_pitch * 2 >= ((int64_t)1 << 32)) return false;
  if (a->residual && (int64_t)a->batch * vol * a->residual_pitch * 2 >= ((int64_t)1 << 32)) return false;
  if ((int64_t)a->out_c * 27 * ((a->c0 + a->c1 + 63) / 64 * 4) * 32 >= ((int64_t)1 << 31)) return false;

  const QBrick& k = kQBricks[0];
  const int64_t nb = ceil_div64(a->in_d, k.TD) * ceil_div64(a->in_h, k.TH) * ceil_div64(a->in_w, k.TW);
  const int64_t nwg = nb * (a->out_c / 64) * a->batch;
  if (nwg > 0x7fffffff) return false;
  if (force != 1) {
    // Grids that leave CUs idle go to the kernels built for them.
    if (nwg < 200) return false;
    // Modelled workgroup time (cycles per 64 input channels): MFMA cycles of the busiest
    // SIMD at the measured main-loop efficiency of each kernel, plus the per-workgroup
    // fixed cost, times the rounds of workgroups over 256 CUs (a partial last round counts
    // whole). The streamed kernel's brick is 256 voxels. With the input transform this
    // kernel stages every chunk's halo through registers before its taps (≈7k cycles a
    // chunk), while the streamed kernel's double-buffered halo hides all but the first
    // (≈3k). Same-box timings with the transform, µs, streamed / this kernel: 64x80x80
    // 128 -> 128 415 / 460, 256 -> 128 783 / 859, 128x160x160 64 -> 64 1004 / 1128 (the
    // streamed kernel), 32x40x40 256 -> 256 237 / 215, 256 -> 128 116 / 110 (this kernel:
    // the streamed kernel's 800 or 400 workgroups leave its last round part-empty).
    const int ncol = (k.TD * k.TH * k.TW + 31) / 32;
    const int64_t nchunk = (a->c0 + a->c1) / KC;
    const bool xf = a->affine || a->silu;
    const double quad = (double)ceil_div64(nwg, 256) *
                        (nchunk * ncol * 54 * 32 / 0.95 + 6000.0 + (xf ? 7000.0 * nchunk : 0.0));
    const int64_t snb = ceil_div64(a->in_d, 4) * ceil_div64(a->in_h, 8) * ceil_div64(a->in_w, 8);
    const int64_t swg = snb * (a->out_c / 64) * a->batch;
    const double stream = (double)ceil_div64(swg, 256) * (nchunk * 432 * 32 / 0.7 + 9000.0 + (xf ? 3000.0 : 0.0));
    if (!(quad < stream)) return false;
  }
  QuadParams& p = *out;
  p = QuadParams{};
  p.B = a->batch; p.D = a->in_d; p.H = a->in_h; p.W = a->in_w;
  p.C0 = a->c0; p.C1 = a->c1; p.C = a->c0 + a->c1; p.O = a->out_c;
  p.nchunk = p.C / KC;
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
  p.TD = k.TD; p.TH = k.TH; p.TW = k.TW;
  p.nob = p.O / 64;
  p.NBD = (int)ceil_div64(p.D, k.TD);
  p.NBH = (int)ceil_div64(p.H, k.TH);
  p.NBW = (int)ceil_div64(p.W, k.TW);
  p.nbr = (int)nb;
  p.schunks = p.nbr;
  return true;
}

int conv3d_quad_launch(QuadParams& p, hipStream_t st) {
  if (p.TD == 4 && p.TH == 5 && p.TW == 10) return cq::launch<4, 5, 10>(p, st);
  return fail("conv3d (K-quarter): no kernel for brick %dx%dx%d", p.TD, p.TH, p.TW);
}

}  // namespace LDX_ELEM_NS
}  // namespace ldx
