/* ldx.h -- C ABI of libldx.so, the MI355X (gfx950) dense hot path of 3-D latent
 * diffusion: implicit-GEMM conv3d with fused GroupNorm/SiLU prologue and
 * bias/shift/residual/scale epilogue, flash attention, GroupNorm statistics,
 * LayerNorm, weight packing and the DDIM step.
 *
 * Conventions
 *  - Activations are channels-last NDHWC float16 ("voxels x channels"), or bfloat16 where
 *    an entry point takes a dtype (conv3d, attention, the weight packers); every
 *    activation pointer comes with a voxel pitch in elements (>= channels), so a
 *    kernel can read or write a channel slice of a wider tensor (zero-copy concat).
 *  - All pointers are device pointers owned by the caller; no entry point allocates
 *    device memory. Work is enqueued on `stream` (a hipStream_t, passed as void*;
 *    NULL = the default stream) and is stream-ordered; nothing synchronises the host.
 *  - Return 0 on success, LDX_EINVAL for an argument the kernels do not accept
 *    (nothing is launched), LDX_EHIP for a HIP launch error. ldx_last_error() gives
 *    the message of the calling thread's last failure.
 *
 * Reference correspondence (MedMLX/lesiondiffusion-mlx v0.3.0; the reference binds
 * its kernels through mx.fast.metal_kernel, src/lesiondiffusion_mlx/_typing.py:35-66,
 * and exposes the op-level functions cited at each entry point below).
 */
#ifndef LDX_H
#define LDX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LDX_OK 0
#define LDX_EINVAL (-1)
#define LDX_EHIP (-2)

/* Element types of the entry points that take a `dtype` argument. */
#define LDX_DTYPE_F16 0
#define LDX_DTYPE_F32 1
#define LDX_DTYPE_BF16 2

/* Message of the calling thread's most recent failure ("" if none). */
const char* ldx_last_error(void);
/* ABI version (12); bumped on any change to the structs below or the entry points. */
int ldx_abi_version(void);

/* ---------------------------------------------------------------- conv3d -------
 * Replaces nax_conv3d (src/lesiondiffusion_mlx/_nax_conv.py:451-619) and the
 * pointwise/dense paths of SourceLayers.conv/dense (mlx_model.py:159-220).
 *
 * y[b, v, o] = half( (sum_{tap,c} W[o, tap, c] * xin[b, v@tap, c] + bias[(b,) o]
 *                     + shift[b, o]) * output_scale + residual[b, v, o] )
 * xin = half(silu(x * affine[b, c, 0] + affine[b, c, 1])) when affine/silu are set
 * (rounded once, zero padding applied after it), else x. One rounding of the FP32
 * sum. act = LDX_ACT_GELU / LDX_ACT_SILU further stores half(gelu_erf(float(y))) /
 * half(silu(float(y))) (the dense -> GELU pair of mlx_model.py:549 and the
 * dense -> SiLU pairs of the time embedding, mlx_model.py:434, 614). shift is the
 * ResBlock's projected time embedding (fp16, batch pitch in elements), added with
 * the bias (mlx_model.py:340-341).
 *
 * Geometry: ksize 3 (padding 1) with stride 1 or 2, or with upsample = 1 (conv of
 * the nearest 2x upsampling of x, weights from ldx_pack_upsample_weight); ksize 1
 * (padding 0, stride 1) covers pointwise convs and dense layers (a dense layer over
 * L tokens is a 1 x 1 x L volume). Output extents: n (stride 1), (n-1)/2+1
 * (stride 2), 2n (upsample).
 *
 * x may be split over two tensors along channels (x1 may be NULL): channels
 * [0, c0) come from x0 and [c0, c0 + c1) from x1 -- the UNet decoder's
 * concat([x, skip]) without a copy.
 */
#define LDX_ACT_NONE 0
#define LDX_ACT_GELU 1
#define LDX_ACT_SILU 2

typedef struct ldx_conv3d_args {
  int32_t batch, in_d, in_h, in_w;   /* input (source) grid */
  int32_t c0, c1;                    /* channels of x0 and x1 (c1 = 0 without x1) */
  int32_t out_c;                     /* output channels O */
  int32_t ksize;                     /* 3 or 1 */
  int32_t stride;                    /* 1 or 2 */
  int32_t upsample;                  /* 0 or 1 */
  const void* x0; int64_t x0_pitch;  /* fp16 NDHWC, voxel pitch in elements */
  const void* x1; int64_t x1_pitch;
  const void* weight;                /* packed fp16, ldx_pack_weight layout */
  const float* bias;                 /* fp32 (O) or (batch, O) if bias_batched; may be NULL */
  int32_t bias_batched;
  const void* shift; int64_t shift_pitch;  /* fp16 (batch, O) with batch pitch, or NULL */
  const float* affine;               /* fp32 (batch, c0 + c1, 2) scale/offset pairs or NULL */
  int32_t silu;                      /* apply SiLU to the prepared input */
  const void* residual; int64_t residual_pitch;  /* fp16 NDHWC of the output grid or NULL */
  float output_scale;                /* 1.0 = plain */
  int32_t act;                       /* LDX_ACT_* */
  void* y; int64_t y_pitch;          /* fp16 NDHWC output */
  void* workspace;                   /* optional device scratch for split-K partial sums */
  size_t workspace_bytes;
  int32_t dtype;                     /* LDX_DTYPE_F16 (0), LDX_DTYPE_BF16 or LDX_DTYPE_F32: the type
                                        of x0, x1, shift, residual and y (bias and affine stay
                                        fp32); see the FP32 mode below for the weight */
} ldx_conv3d_args;

/* Bytes of workspace with which ldx_conv3d splits the reduction over channel chunks
 * across workgroups (small grids); 0 when it would not split. Without it the conv
 * runs in one pass -- same results up to fp32 summation order. */
size_t ldx_conv3d_workspace_bytes(const ldx_conv3d_args* args);
int ldx_conv3d(const ldx_conv3d_args* args, void* stream);

/* ldx_conv3d that also leaves the GroupNorm partial moments of its stored output -- the
 * fused GroupNorm-statistics epilogue of the conv that feeds a norm_silu_conv
 * (mlx_model.py:290-342 normalises what the previous conv wrote; here that conv's
 * epilogue reduces it while it is still in registers). moments: fp32
 * [batch][chunks][out_c / 2][3], per channel pair and block of output voxels
 * (count, mean, M2), 16-byte aligned; chunks = ldx_conv3d_stats_chunks(args) for the
 * same args (workspace included: it decides split-K). Returns 0 chunks (and
 * ldx_conv3d_stats LDX_EINVAL) for convs whose plan keeps no moments: pointwise and
 * dense layers, out_c not a multiple of 8, unaligned rows. Same y as ldx_conv3d. */
int64_t ldx_conv3d_stats_chunks(const ldx_conv3d_args* args);
int ldx_conv3d_stats(const ldx_conv3d_args* args, float* moments, void* stream);

/* A pointwise conv (dense layer: ksize 1, one input, no affine / SiLU, c0 a multiple of 16
 * and at most 512) whose input rows are first layer-normalized over their c0 channels:
 * x' = half((x - mean) * rsqrt(var + eps) * gamma[c] + beta[c]) with fp32 row statistics
 * (mean, then the mean squared deviation), then ldx_conv3d's product and epilogue on x'.
 * One launch for the reference's LayerNorm followed by its dense layer
 * (mlx_model.py:541-548: norm1 -> attn1 q/k/v, norm2 -> attn2 to_q, norm3 -> ff); gamma
 * and beta are fp32 (c0), 16-byte aligned. */
int ldx_dense_ln(const ldx_conv3d_args* args, const float* gamma, const float* beta, float eps,
                 void* stream);

/* FP32 mode (dtype LDX_DTYPE_F32) -- the reference's exact split-FP16 mode for FP32 networks
 * (_nax_conv.py:26-34, 210-237, 343-364): every FP32 value v is split into hi = half(v) and
 * lo = half((v - hi) * 2^11), and y = hi x hi + (hi x lo + lo x hi) * 2^-11 with FP32 sums
 * (only lo x lo is dropped, about 2^-22 relative; |v| < 65504). The weight is the two-plane
 * split of ldx_pack_weight_exact; the prologue (affine, SiLU), the epilogue (bias + shift,
 * scale, residual, GELU / SiLU) and y are FP32, with no rounding to 16 bits. upsample = 1
 * takes the unfolded 3x3x3 weight (the conv runs on the upsampled grid). One launch, no
 * workspace (ldx_conv3d_workspace_bytes() is 0). ldx_conv3d_stats and ldx_dense_ln take
 * fp16 / bf16 only. */
int ldx_pack_weight_exact(const float* weight, int32_t out_c, int32_t in_c, int32_t ksize, void* packed,
                          void* stream);
/* ldx_pack_weight_exact: a Torch-layout FP32 (O, C, K, K, K) (or dense (O, C), K = 1) weight
 * (_nax_conv.py:343-364 splits the same values) as two fp16 planes, hi(W) then
 * lo(W) = half((W - hi(W)) * 2^11), each [NRB][NKC][K^3][64][8] with NRB = 2*ceil(O/64),
 * NKC = 4*ceil(C/64): fragment ((rb*NKC + kc)*K^3 + tap) holds lane l's eight values
 * W[rb*32 + l%32, kc*16 + 8*(l/32) + e, tap] at l*8 (zero past O or C).
 * ldx_packed_weight_exact_elems(O, C, K) halves in all (0 for a bad shape). */
size_t ldx_packed_weight_exact_elems(int32_t out_c, int32_t in_c, int32_t ksize);

/* Pack a Torch-layout fp16 or bf16 weight (O, C, K, K, K) (K = 3 or 1; a dense (O, C)
 * weight is K = 1; a pure rearrangement of 16-bit values, the same for both types) into
 * the kernel's fragment-major layout of
 * ldx_packed_weight_elems(O, C, K, 0) halves: with NOB = 4*ceil(O/128), NKC =
 * 4*ceil(C/64), tap = kd*9 + kh*3 + kw, fragment ((ob*K^3 + tap)*NKC + kc) holds 512
 * halves, lane l's eight at offset l*8 being W[ob*32 + l%32, kc*16 + 8*(l/32) + e,
 * kd, kh, kw] (zero past O or C) -- the A operand of v_mfma_f32_32x32x16_f16. The reference's pack_weight
 * (_nax_conv.py:350-364) stores the same values as (27*C', O') with row tap*C' + c;
 * this order makes every MFMA A-operand load one contiguous 1 KB wave read. */
size_t ldx_packed_weight_elems(int32_t out_c, int32_t in_c, int32_t ksize, int32_t upsample);
int ldx_pack_weight(const void* weight, int32_t out_c, int32_t in_c, int32_t ksize,
                    void* packed, void* stream);

/* Fold a Torch-layout (O, C, 3, 3, 3) weight of type dtype (LDX_DTYPE_F16 or
 * LDX_DTYPE_BF16) into the 8 parity 2x2x2 filters of a nearest-2x-upsampled conv
 * (pack_upsample_weight, _nax_conv.py:367-405): merged taps summed in fp32 in the
 * reference's order and rounded to dtype once,
 * stored fragment-major as above with parity = pd*4+ph*2+pw leading and tap =
 * td*4+th*2+tw: fragment (((parity*NOB + ob)*8 + tap)*NKC + kc). */
int ldx_pack_upsample_weight(const void* weight, int32_t out_c, int32_t in_c, int32_t dtype,
                             void* packed, void* stream);

/* ------------------------------------------------------------- group norm -------
 * Replaces medmlx_core group_norm_affine (call sites mlx_model.py:328-335,
 * _scaled_vq.py:93-100): per-(b, group) mean / biased variance of x (optionally the
 * channel concat of x0 and x1), folded with gamma/beta into fp32 (batch, C, 2)
 * (scale = gamma * rsqrt(var + eps), offset = beta - scale * mean). Two
 * deterministic passes (no float atomics) through a caller-provided workspace of
 * ldx_group_norm_workspace_bytes() bytes. gamma/beta are fp32 (C). */
size_t ldx_group_norm_workspace_bytes(int32_t batch, int64_t voxels, int32_t channels,
                                      int32_t groups);
int ldx_group_norm_affine(const void* x0, int64_t x0_pitch, int32_t c0,
                          const void* x1, int64_t x1_pitch, int32_t c1,
                          int32_t batch, int64_t voxels, int32_t groups,
                          const float* gamma, const float* beta, float eps,
                          float* affine, void* workspace, void* stream);

/* ldx_group_norm_affine without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference (its kernels allocate their outputs through
 * MLX). Same kernels and same results as ldx_group_norm_affine; the two-pass path's
 * partials go to a device array of LDX_GROUP_NORM_SCRATCH_BYTES that the library holds on
 * each GPU it runs on until the process ends. Nothing is allocated. Returns LDX_EINVAL when
 * ldx_group_norm_workspace_bytes() of the same shape exceeds that size (at 32 groups: up
 * to batch * ceil(voxels / 8192) <= 10922, e.g. 4 volumes of 256^3). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race
 * and must be ordered by the caller. */
#define LDX_GROUP_NORM_SCRATCH_BYTES (4u << 20)
int ldx_group_norm_affine_noalloc(const void* x0, int64_t x0_pitch, int32_t c0,
                                  const void* x1, int64_t x1_pitch, int32_t c1,
                                  int32_t batch, int64_t voxels, int32_t groups,
                                  const float* gamma, const float* beta, float eps,
                                  float* affine, void* stream);

/* group_norm_affine from moments a conv left (ldx_conv3d_stats) instead of a pass over x:
 * m0 holds x0's (chunks0 blocks, c0 / 2 pairs), m1 x1's for the concat (c1 = 0: none).
 * Merged per group in a fixed order (Chan's pairwise update); c0, c1 and C / groups
 * must be even. Same (batch, C, 2) output as ldx_group_norm_affine. */
int ldx_group_norm_affine_moments(const float* m0, int64_t chunks0, int32_t c0,
                                  const float* m1, int64_t chunks1, int32_t c1,
                                  int32_t batch, int32_t groups,
                                  const float* gamma, const float* beta, float eps,
                                  float* affine, void* stream);
/* The same for moments of many blocks (more than 4,096 (pair, block) items per group): each
 * input's blocks are first folded, a pass over whole block rows on many workgroups, into
 * at most 65,535 blocks in the caller's workspace, then merged per group as above (a fixed
 * order; it differs from the one-pass order, so the pairs agree with
 * ldx_group_norm_affine_moments to fp32 rounding, not bit for bit). The workspace size is
 * ldx_group_norm_moments_workspace_bytes(); with 0 (few items) the call is
 * ldx_group_norm_affine_moments and the workspace is not used. Same output. */
size_t ldx_group_norm_moments_workspace_bytes(int64_t chunks0, int32_t c0, int64_t chunks1, int32_t c1,
                                              int32_t batch, int32_t groups);
int ldx_group_norm_affine_moments_ws(const float* m0, int64_t chunks0, int32_t c0,
                                     const float* m1, int64_t chunks1, int32_t c1,
                                     int32_t batch, int32_t groups,
                                     const float* gamma, const float* beta, float eps,
                                     float* affine, void* workspace, size_t workspace_bytes, void* stream);

/* GroupNorm statistics (as ldx_group_norm_affine) and LayerNorm (as ldx_layer_norm) of FP32
 * tensors, statistics in FP32 (per-thread Welford moments merged in a fixed order; the row
 * mean, then the mean squared deviation), FP32 output -- the FP32 networks' norms
 * (mlx_model.py:328-335, 360-367). No workspace. */
int ldx_group_norm_affine_f32(const float* x0, int64_t x0_pitch, int32_t c0, const float* x1, int64_t x1_pitch,
                              int32_t c1, int32_t batch, int64_t voxels, int32_t groups, const float* gamma,
                              const float* beta, float eps, float* affine, void* stream);
int ldx_layer_norm_f32(const float* x, int64_t x_pitch, int64_t rows, int32_t features, const float* gamma,
                       const float* beta, float eps, float* y, int64_t y_pitch, void* stream);

/* LayerNorm over the last axis of fp16 (rows, features) (mx.fast.layer_norm,
 * mlx_model.py:360-367): y = half((x - mean) * rsqrt(var + eps) * gamma + beta),
 * statistics in fp32. gamma/beta fp32. */
int ldx_layer_norm(const void* x, int64_t x_pitch, int64_t rows, int32_t features,
                   const float* gamma, const float* beta, float eps,
                   void* y, int64_t y_pitch, void* stream);

/* -------------------------------------------------------------- attention -------
 * Replaces flash_attention_half (_attention_half.py:129-147) and the fused
 * mx.fast.scaled_dot_product_attention routes of LdmUnet.attention
 * (mlx_model.py:443-493): o = softmax(q k^T * scale + mask) v per (batch, head),
 * fp16 inputs/outputs, fp32 scores, online softmax and accumulation.
 * Tensors are 4-D (batch, len, heads, head_dim) with arbitrary element strides
 * (head_dim stride must be 1); both the projection layout (B, L, H*D) and
 * (B, H, L, D) are views of this. head_dim in {16, 32, 64, 128, 256}.
 * mask (optional) is additive fp32 with strides (batch, head, query, key), 0 for a
 * broadcast axis; -inf removes a key; a query row with every key removed gives 0.
 * LDX_DTYPE_F32 (the FP32 networks; the reference's FP32 attention, _attention.py:52-145):
 * head_dim 16, 32 or 64, no mask, FP32 scores, probabilities and products throughout.
 * V is read as it lies and transposed by the LDS reads. Scratch memory serves one plan
 * only: wide heads (128, 256) whose 128-query tiles spread unevenly over the CUs (the VQ
 * decoder's 51,200-token mid attention: 400 tiles on 256 CUs) split each tile's keys into
 * equal pieces, one workgroup each, and merge the pieces' partial states in a second
 * launch; ldx_attention_workspace_bytes returns their size (0 for every other plan). A
 * NULL or smaller workspace runs one workgroup per tile instead (same results within
 * fp32 summation order). */
typedef struct ldx_attention_args {
  int32_t batch, heads, q_len, kv_len, head_dim;
  const void* q; int64_t q_stride[3];   /* batch, len, head strides (elements) */
  const void* k; int64_t k_stride[3];
  const void* v; int64_t v_stride[3];
  void* o; int64_t o_stride[3];
  float scale;
  const float* mask; int64_t mask_stride[4];
  void* workspace; size_t workspace_bytes;   /* see ldx_attention_workspace_bytes; may be NULL / 0 */
  int32_t dtype;                        /* LDX_DTYPE_F16 (0), LDX_DTYPE_BF16 or LDX_DTYPE_F32: q, k, v, o */
} ldx_attention_args;

size_t ldx_attention_workspace_bytes(const ldx_attention_args* args);
int ldx_attention(const ldx_attention_args* args, void* stream);

/* ------------------------------------------------------------ small ops ---------
 * Sinusoidal timestep features [cos(t f_i), sin(t f_i)], f_i = exp(-ln(1e4) i/half)
 * (mlx_model.py:609-612), written as fp16 (batch, channels). timesteps int32. */
int ldx_timestep_embedding(const int32_t* timesteps, int32_t batch, int32_t channels,
                           void* out, void* stream);
/* The same features in FP32 (the FP32 networks). */
int ldx_timestep_embedding_f32(const int32_t* timesteps, int32_t batch, int32_t channels, float* out, void* stream);

/* y = half(silu(float(x))) elementwise over n fp16 values (LdmUnet.silu,
 * mlx_model.py:409-413). */
int ldx_silu(const void* x, int64_t n, void* y, void* stream);

/* Copy a channel slice: dst[v, dst_off + c] = src[v, src_off + c], c < channels,
 * for `voxels` voxels of fp16 NDHWC tensors (concat / split without torch). */
int ldx_copy_channels(const void* src, int64_t src_pitch, int32_t src_off,
                      void* dst, int64_t dst_pitch, int32_t dst_off,
                      int64_t voxels, int32_t channels, void* stream);

/* Nearest 2x upsampling of fp16 NDHWC (B, D, H, W, C) into (B, 2D, 2H, 2W, C): output
 * index i of each axis reads input floor(i / 2) (upsample_nearest2 / resize_nearest,
 * src/lesiondiffusion_mlx/_spatial.py:41-69). The fused conv path (upsample = 1 in
 * ldx_conv3d) never forms this tensor; this entry point serves callers that need it. */
int ldx_upsample_nearest2(const void* x, int64_t x_pitch, int32_t batch, int32_t d, int32_t h,
                          int32_t w, int32_t channels, void* y, int64_t y_pitch, void* stream);

/* One masked DDIM step of the conditioned sampler (mlx_sampling.py:172-185) on
 * NDHWC latents with `channels` channels (fp32 state x, fp16 network in/out):
 *   prepare: with a mask, xm = x*m + (1-m)*cond, x = xm, and net_in[v] =
 *       [half(xm) (C), half(cond*(1-m)) (cond_channels = C, or absent when 0),
 *       half(m) (1)]; without a mask net_in[v] = [half(x) (C), half(cond)
 *       (cond_channels)] (the mask-free form of mlx_sampling.py:177-178).
 *   update: x = sqrt(prev)*(x - s1m*eps)/sqrt(a) + sqrt(1-prev-sig^2)*eps
 *       + sig*noise, eps = float(net_out[v, 0:C))
 * coef = {alpha, previous, sigma, sqrt_one_minus} (fp32 device array of 4). x, cond,
 * noise are fp32 NDHWC with `channels` (cond: cond_channels without a mask)
 * channels; mask is fp32 (voxels). */
int ldx_ddim_prepare(float* x, const float* cond, const float* mask, int64_t voxels,
                     int32_t channels, int32_t cond_channels, void* net_in,
                     int64_t net_pitch, void* stream);
int ldx_ddim_update(float* x, const void* net_out, int64_t net_pitch, const float* noise,
                    const float* coef, const int32_t* step, int64_t voxels, int32_t channels,
                    void* stream);

/* Device-side step indexing for a captured (graph-replayed) sampler step: with
 * step != NULL, ldx_ddim_update reads coef + 4 * (*step) and noise + (*step) * voxels
 * * channels (tables of all steps); ldx_ddim_timestep writes t_out[0..batch) =
 * t_table[*step]; ldx_step_advance increments *step (one thread). */
int ldx_ddim_timestep(const int32_t* step, const int32_t* t_table, int32_t batch,
                      int32_t* t_out, void* stream);
int ldx_step_advance(int32_t* step, void* stream);

/* ------------------------------------------------------- VQ codebook search -------
 * Replaces the native four-channel nearest-codebook search nearest_codebook4
 * (src/lesiondiffusion_mlx/_vq.py:12-82) and the quantize step of VqAutoencoder
 * (mlx_model.py:742-803). Element type T = dtype (LDX_DTYPE_F16 or LDX_DTYPE_F32) for
 * every array but the int32 indices; vectors are rows of 4 contiguous values.
 *
 * ldx_vq_squared_norms4: out[i] = T(sum_c float(T(x[i,c] * x[i,c]))), the four squares
 * rounded to T, summed in fp32 in channel order, the sum rounded to T.
 *
 * ldx_vq_nearest4: for each of `positions` latent vectors z[p], the code index chosen over
 * the `entries` codebook rows with the reference's distance and rounding points:
 *   dot = fma(z3, c3, fma(z2, c2, fma(z1, c1, z0 * c0)))            (fp32)
 *   distance = T(T(z_norm[p] + codebook_norm[c]) - T(2 * T(dot)))
 * the lowest index with a NaN distance if there is one, else the lowest index of the
 * smallest distance (MLX argmin's order; exact, independent of the scan). z_norm may be
 * NULL (computed as in ldx_vq_squared_norms4); codebook_norm is required (computed once per
 * codebook by the caller). quantized (may be NULL) receives the straight-through value
 * z + (selected - z), each operation rounded to T. */
int ldx_vq_squared_norms4(const void* x, int64_t n, int32_t dtype, void* out, void* stream);
int ldx_vq_nearest4(const void* z, const void* z_norm, const void* codebook, const void* codebook_norm,
                    int64_t positions, int32_t entries, int32_t dtype, int32_t* indices,
                    void* quantized, void* stream);

/* ------------------------------------------------- source-order fp16 arithmetic -------
 * The reference's "source" arithmetic, which reproduces Torch-CPU's reduction order bit
 * for bit (src/lesiondiffusion_mlx/_source_half.py). Tensors are fp16, addressed by
 * (batch, channel, voxel) strides in elements -- NCDHW (voxel stride 1, the reference's
 * layout) or channels-last -- with voxel index (z * H + y) * W + x; the arithmetic follows
 * the logical NCDHW order either way.
 *
 * ldx_conv3d_source_half replaces conv3d_half (_source_half.py:19-104, 327-384):
 *   y[n, o, v] = half( ((p0 + p1) + p2) + p3 + float(bias[o]) )
 * over k = c * KD*KH*KW + (kd * KH + kh) * KW + kw of the zero-padded im2col column,
 * partial k % 4 for k < K - K % 4 in increasing k, the remaining k into p0, every product
 * of two fp16 values (exact in fp32) added in fp32. Any kernel size, stride >= 1,
 * padding >= 0; weight (out_c, in_c, kd, kh, kw) contiguous fp16; bias fp16 or NULL.
 * Output extents (n + 2 * padding - k) / stride + 1; a kernel larger than the padded
 * input is rejected ("conv3d kernel exceeds the padded input").
 *
 * ldx_group_norm_source_half replaces group_norm_half (_source_half.py:120-300, 387-544):
 * per (batch item, group) Welford moments of vectors of 8 values in chunks of 16 vectors,
 * merged by the reference's binary-counter cascade (128-chunk blocks in parallel, then
 * group-wide), the scalar tail and the four lanes last; var = max(m2 / SIZE, 0),
 * rstd = float(1 / sqrt(double(var) + double(eps))), scale = rstd * weight[c],
 * offset = fma(-scale, mean, bias[c]) into affine[b, c, 0..1] (fp32, required); then, if
 * y is not NULL, y = half(float(scale * x) + offset). weight and bias are fp16 (C,). The
 * workspace holds the chunk and block moments: ldx_group_norm_source_workspace_bytes. */
typedef struct ldx_conv3d_source_args {
  int32_t batch, in_c, in_d, in_h, in_w;
  int32_t out_c, kd, kh, kw;
  int32_t stride, padding;
  const void* x;
  int64_t x_batch_stride, x_channel_stride, x_voxel_stride;
  const void* weight;
  const void* bias;
  void* y;
  int64_t y_batch_stride, y_channel_stride, y_voxel_stride;
} ldx_conv3d_source_args;

int ldx_conv3d_source_half(const ldx_conv3d_source_args* args, void* stream);
size_t ldx_group_norm_source_workspace_bytes(int32_t batch, int32_t channels, int64_t voxels, int32_t groups);
int ldx_group_norm_source_half(const void* x, int64_t x_batch_stride, int64_t x_channel_stride,
                               int64_t x_voxel_stride, int32_t batch, int32_t channels, int64_t voxels,
                               int32_t groups, const void* weight, const void* bias, float eps,
                               float* affine, void* y, int64_t y_batch_stride, int64_t y_channel_stride,
                               int64_t y_voxel_stride, void* workspace, size_t workspace_bytes,
                               void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LDX_H */
