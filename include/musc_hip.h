/*
 * musc_hip.h -- C-ABI of libmusc_hip.so, the MI355X (gfx950) implementation of
 * MuSc's data-parallel hot path: mutual scoring (MSM), LNAMD neighbourhood
 * aggregation, the score-map epilogue and ViT block attention.
 *
 * Conventions shared by every entry point
 *   - All array pointers are DEVICE pointers unless a parameter says "host".
 *   - Every launch is asynchronous on the given hipStream_t (0 = null stream);
 *     nothing synchronises the host.
 *   - The caller owns every buffer, including the workspace; the library keeps
 *     no device state between calls.  Calls on different streams with
 *     different workspaces may overlap.
 *   - Return value: 0 on success, a hipError_t value (1..999) when the HIP
 *     runtime reports an error, or a library code >= 1000 for argument errors
 *     (see MUSC_ERR_*).  musc_strerror() turns any of them into text.
 *
 * The reference (DylanMartinLSC/musc-gpu) reaches its kernels through a ctypes
 * bridge to NVRTC and the CUDA driver (models/modules/_cuda_runtime.py:58-100):
 * it compiles CUDA C strings at first use and launches raw CUfunctions with
 * data_ptr()/int arguments on torch's current stream.  This header replaces
 * that bridge with fixed, typed entry points; each one names the reference
 * function whose contract it serves.
 */
#ifndef MUSC_HIP_H
#define MUSC_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Error codes (library-defined, >= 1000).                                   */
/* ------------------------------------------------------------------------ */
#define MUSC_OK                 0
#define MUSC_ERR_INVALID_ARG    1001  /* bad shape, rank window, null pointer */
#define MUSC_ERR_WORKSPACE      1002  /* workspace smaller than required      */
#define MUSC_ERR_UNSUPPORTED    1003  /* shape outside the implemented range  */
#define MUSC_ERR_SCRATCH_LIMIT  1004  /* needs more than the no-allocation scratch */

/* Text for any return code of this library (never NULL). */
const char* musc_strerror(int code);

/* Library version, as MAJOR*10000 + MINOR*100 + PATCH. */
int musc_version(void);

/* The GPU architecture the kernels are compiled for ("gfx950").  A device whose
 * architecture name (hipDeviceProp_t.gcnArchName up to the first ':') differs cannot
 * run them; the backend selector then falls back to the original path, as the
 * reference's selector does when its accelerated runtime cannot run
 * (models/modules/_backend.py:10-13).  The reference's NVRTC bridge compiles for the
 * device at first use instead (models/modules/_cuda_runtime.py:58-92). */
const char* musc_target_arch(void);

/* ------------------------------------------------------------------------ */
/* Mutual scoring module (MSM).                                              */
/* ------------------------------------------------------------------------ */

/* Workspace needed by musc_msm_scores_f32 / musc_msm_nearest_f32 for a pool of
 * n images x p patches x c channels.  Writes the byte count to *out.
 * Replaces the scratch tensors the reference allocates inside
 * models/modules/_MSM_gpu.py:717-748.  Every MSM entry point taking a workspace
 * requires it to start at a 256-byte-aligned address (MUSC_ERR_INVALID_ARG
 * otherwise); hipMalloc and torch's allocator return such addresses. */
int musc_msm_workspace_bytes(int n, int p, int c, size_t* out);

/* Mutual scores of a pool.
 *   z       (n, p, c) fp32, row-major, contiguous.
 *   rank_lo, rank_hi   trimmed rank window [rank_lo, rank_hi) over the n-1
 *           per-reference-image minima, 0 <= rank_lo < rank_hi <= n-1.
 *           The reference call site uses topmin_min=0, topmin_max=0.3, i.e.
 *           rank_lo = int((n-1)*0), rank_hi = int((n-1)*0.3).
 *   scores  (n, p) float64 out: for patch q of image i, the mean of ascending
 *           ranks [rank_lo, rank_hi) of { min_r ||z[i,q]-z[j,r]||_2 : j != i },
 *           the mean rounded to fp32 and widened to float64.
 * Same contract as the reference's scoring plugin
 * models/modules/_MSM_gpu.py:701-830 and the original
 * models/modules/_MSM.py:10-30,53-59 (called at models/musc.py:254). */
int musc_msm_scores_f32(const float* z, int n, int p, int c,
                        int rank_lo, int rank_hi, double* scores,
                        void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* musc_msm_scores_f32 without a workspace argument and without allocating: no
 * counterpart in the reference.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The workspace is a device array inside the library, one per GPU,
 * of MUSC_NOALLOC_SCRATCH_BYTES (256 MiB, the reference's own scratch cap
 * (models/modules/_MSM_gpu.py:11); held by every GPU the library runs on
 * until the process ends), so pools whose musc_msm_workspace_bytes exceeds it are
 * rejected with MUSC_ERR_SCRATCH_LIMIT (at P = 1369: N = 83 needs 37 MiB, N = 160
 * 136 MiB; N = 225 does not fit).  Runs on the current device; `stream` must belong to it.
 * Every call on one GPU uses that GPU's array: calls that overlap on one GPU (other
 * streams or threads) race and must be serialised by the caller.  Same arguments
 * (minus the workspace), results and errors as musc_msm_scores_f32. */
#define MUSC_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int musc_msm_scores_f32_noalloc(const float* z, int n, int p, int c, int rank_lo, int rank_hi,
                                double* scores, hipStream_t stream);

/* Per-reference-image nearest distances, the intermediate of the scoring:
 *   nearest (n*p, n) fp32 out, nearest[i*p+q][j] = min_r ||z[i,q]-z[j,r]||_2
 *           for j != i, and +inf for j == i.
 * Matches `torch.min(torch.cdist(...), -1)[0]` of models/modules/_MSM.py:16-17
 * and the `nearest` tensor of models/modules/_MSM_gpu.py:717. */
int musc_msm_nearest_f32(const float* z, int n, int p, int c, float* nearest,
                         void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

/* Flags for musc_msm_prepare_f32. */
#define MUSC_MSM_NORMALIZE_ROWS 1  /* score z_row / ||z_row|| instead of z_row: the L2
                                      normalisation of models/musc.py:238 applied
                                      inside MSM, so an aggregation that writes
                                      unnormalised features needs no extra pass   */

/* The four stages of musc_msm_scores_f32, for callers that time or overlap
 * them separately (same arguments and workspace):
 *   prepare      row norms ||z||^2 (and, with MUSC_MSM_NORMALIZE_ROWS, the row
 *                scales 1/||z||) and the +inf fill of the minima buffer;
 *   pair_minima  fp32-MFMA pairwise distances of every unordered patch pair of
 *                different images, reduced along rows and columns into the
 *                per-(patch, image) minima (the hot kernel);
 *   refine       exact minima where ||a||^2 + ||b||^2 - 2 a.b cancels: every
 *                (patch, image) minimum with d^2 <= max(32 c, 4096) FLT_EPSILON
 *                (||q||^2 + the image's largest ||r||^2) is recomputed over that
 *                image's p patches by explicit differences, as the reference
 *                recomputes such pairs (models/modules/_MSM_gpu.py:219-228, bound
 *                32 FLT_EPSILON c (||q||^2 + ||r||^2); the floor of 4096 covers the
 *                norm roundings that bound misses for small c); with nothing to
 *                recompute it reads the minima once.  Works on the workspace of
 *                either engine (the split engine's included) after its
 *                pair_minima, with the same z;
 *   rank         trimmed rank means of the minima into scores.
 * prepare, pair_minima, refine and rank run in that order on one stream
 * (musc_msm_scores_f32, musc_msm_nearest_f32 and musc_msm_split_scores_f32 run
 * all four). */
int musc_msm_prepare_f32(const float* z, int n, int p, int c, int flags,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);
int musc_msm_pair_minima_f32(const float* z, int n, int p, int c,
                             void* workspace, size_t workspace_bytes, hipStream_t stream);
int musc_msm_refine_f32(const float* z, int n, int p, int c,
                        void* workspace, size_t workspace_bytes, hipStream_t stream);
int musc_msm_rank_f32(int n, int p, int rank_lo, int rank_hi, double* scores,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Split engine: the same scores, with each fp32 dot product formed from three
 * fp16 MFMA products.  Rows are L2-normalised and scaled by 2^10 (v in fp64), split
 * as hi = fp16(fp32(v)), lo = fp16(fp32(v - hi)) with every narrowing rounded to
 * nearest even, and a.b is accumulated in fp32 as
 * hi.hi + hi.lo + lo.hi (error below 2^-22 |a||b|, the order of fp32's own
 * accumulation error); a per-row scale restores the units, so MUSC_MSM_NORMALIZE_ROWS
 * and unnormalised inputs both work.  Same contract, arguments and stage order as
 * the fp32 engine above (replaces the same reference interface,
 * models/modules/_MSM_gpu.py:701-830), with a larger workspace (the split rows) and
 * p >= 256 (MUSC_ERR_UNSUPPORTED otherwise).  musc_msm_rank_f32 accepts this
 * workspace.  Choose the engine by shape and accuracy need: the fp32 engine is the
 * reference-faithful default. */
int musc_msm_split_workspace_bytes(int n, int p, int c, size_t* out);
int musc_msm_split_prepare_f32(const float* z, int n, int p, int c, int flags,
                               void* workspace, size_t workspace_bytes, hipStream_t stream);
int musc_msm_split_pair_minima(int n, int p, int c, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);
int musc_msm_split_scores_f32(const float* z, int n, int p, int c, int rank_lo, int rank_hi,
                              int flags, double* scores, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* LNAMD: per-image LayerNorm over (C,H,W) + r x r zero-padded box mean.     */
/* ------------------------------------------------------------------------ */
#define MUSC_DTYPE_F32 0
#define MUSC_DTYPE_F16 1

/* Output layouts of musc_lnamd_f32 (R radii, L layers, B images, P patches). */
#define MUSC_LAYOUT_RBPLC 0  /* out[r][b][p][l][c]: one (B,P,L,C) block per radius,
                                the aggregation plugin's return layout           */
#define MUSC_LAYOUT_RLBPC 1  /* out[r][l][b][p][c]: one contiguous (B,P,C) pool
                                per (radius, layer), the MSM input layout        */

/* Flags for musc_lnamd_f32. */
#define MUSC_LNAMD_L2NORM 1  /* also divide every output patch by its L2 norm over C
                                (models/musc.py:238, fused)                        */
#define MUSC_LNAMD_STATS_READY 2  /* the workspace already holds the LayerNorm
                                statistics of these same tokens from an earlier
                                call (e.g. another radius): skip the stats pass.
                                Serves the per-division reuse of
                                models/modules/_aggregation_cache.py:15-58.     */
#define MUSC_LNAMD_RAW_SUMS 4  /* write the r x r window sums of (x - mean) without
                                the 1/sqrt(var+eps) and 1/r^2 factors: the input
                                of an L2-normalising consumer (musc_msm_prepare_f32
                                with MUSC_MSM_NORMALIZE_ROWS), for which those
                                factors cancel.  Not combinable with L2NORM.     */

int musc_lnamd_workspace_bytes(int batch, int n_layers, size_t* out);

/* tokens   host array of n_layers device pointers, each (batch, tokens_per_image, c)
 *          of dtype in_dtype, contiguous.  When has_cls != 0 token 0 of each image
 *          is the class token and is skipped; the remaining tokens form a
 *          side x side grid (side*side == tokens_per_image - has_cls).
 * radii    host array of n_radii odd radii (1, 3, 5, 7 or 9, in any order; a window
 *          may exceed the grid); the output keeps the caller's order.
 * Limits: n_radii <= 4, n_layers <= 16, 4 <= c <= 4096 with c % 4 == 0, a grid side
 *          of at most 1024, and 32 * n_radii * side bytes of LDS (48 * n_radii * side
 *          with pooling) within 64 KB: side <= 1024 for one or two radii, 682 for
 *          three, 512 for four (341 pooled); MUSC_ERR_UNSUPPORTED beyond.
 * eps      LayerNorm epsilon (torch default 1e-5).
 * out      fp32, layout out_layout, batch*P*n_layers*c*n_radii floats.
 * Semantics per radius r and layer l (models/modules/_LNAMD.py:72-129 and the
 * identity used by models/modules/_encoder_gpu.py:14-42,
 * models/modules/_aggregation_cache.py:15-58):
 *   y = (x - mean) / sqrt(var + eps) over all C*H*W values of one image (biased var,
 *       unit weight, zero bias), then out = avg_pool2d(y, r, stride 1, pad r//2,
 *       count_include_pad=True); with MUSC_LNAMD_L2NORM, out /= ||out||_2 over C. */
int musc_lnamd_f32(const void* const* tokens, int n_layers, int in_dtype,
                   int batch, int tokens_per_image, int c, int has_cls,
                   const int* radii, int n_radii, float eps, int flags,
                   float* out, int out_layout,
                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/* musc_lnamd_f32 with the side x side grid of outputs adaptively average-pooled to
 * pool_side x pool_side in the same pass (F.adaptive_avg_pool2d windows, the
 * super_fast 37 -> 28 step of models/modules/_super_fast.py:17-27 applied after
 * LNAMD): out holds pool_side^2 patches per (radius, image, layer) in out_layout.
 * 1 <= pool_side <= side (pool_side == side: no pooling); not with
 * MUSC_LNAMD_L2NORM.  With MUSC_LNAMD_RAW_SUMS the pooled values are plain sums
 * (no 1/r^2, no division by the window count: scales an L2-normalising consumer
 * removes); otherwise LayerNorm + box mean + adaptive mean exactly. */
int musc_lnamd_pooled_f32(const void* const* tokens, int n_layers, int in_dtype, int batch,
                          int tokens_per_image, int c, int has_cls, const int* radii, int n_radii,
                          float eps, int flags, int pool_side, float* out, int out_layout,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Adaptive average pooling of patch grids, F.adaptive_avg_pool2d semantics:
 *   in   (batch, side_in*side_in, ch) fp32, out (batch, side_out*side_out, ch) fp32.
 * The super_fast aggregation pools the r=3 LNAMD grid 37x37 -> 28x28
 * (models/modules/_super_fast.py:17-27); a (B, P, L, C) block is pooled as
 * batch = B, ch = L*C, an (R, L, N, P, C) pool as batch = R*L*N, ch = C. */
int musc_adaptive_pool_f32(const float* in, int batch, int side_in, int ch, int side_out,
                           float* out, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Epilogue: layer/radius averaging, bilinear upsampling, image scores.      */
/* ------------------------------------------------------------------------ */

/* scores    (n_radii, n_layers, n, side*side) float64 per-(radius, layer) MSM maps.
 * maps      (n, out_size, out_size) float64 out: mean over layers, then over radii
 *           (models/musc.py:259,263), upsampled bilinearly with align_corners=True
 *           (models/musc.py:269-272).
 * image_scores (n,) float64 out: max over each upsampled map (models/musc.py:288).
 *           May be NULL.  maps may be NULL when only image_scores are wanted.
 * Any out_size >= 1 (upsampling or downsampling); side <= 128 (MUSC_ERR_UNSUPPORTED
 * beyond: a grid row is staged whole in LDS). */
int musc_maps_f64(const double* scores, int n_radii, int n_layers, int n, int side,
                  int out_size, double* maps, double* image_scores,
                  hipStream_t stream);

/* RsCIN refinement of image scores (models/modules/_RsCIN.py:5-32):
 *   cls_tokens   (n, d) fp32 L2-normalised class tokens (models/musc.py:215,218);
 *   image_scores (n,) float64 raw image scores (map maxima, models/musc.py:288);
 *   k_list       host array of n_k neighbourhood sizes (1 <= k <= n; MVTec uses 1,2,3);
 *   out          (n,) fp32: mean over k of sum_{j in top-k(i)} W_ij s_j / sum W_ij with
 *                W = X X^T and s the min-max normalised scores.
 * The reference returns the scores unchanged when k_list contains 0; callers do that
 * check (the entry point rejects k < 1).  Limits: n <= 4096, n_k <= 16
 * (MUSC_ERR_UNSUPPORTED beyond). */
int musc_rscin_f32(const float* cls_tokens, const double* image_scores, int n, int d,
                   const int* k_list, int n_k, float* out, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* Image preprocessing of the data path (decoded uint8 RGB -> encoder input). */
/* ------------------------------------------------------------------------ */

/* images  (batch, in_h, in_w, 3) uint8 RGB, interleaved (as decoded by PIL after
 *         .convert("RGB"), datasets/mvtec.py:101);
 * out     (batch, 3, out_h, out_w) float32: Resize((out_h, out_w), BICUBIC) with
 *         Pillow's 8-bit fixed-point resampling, CenterCrop (identity at that size),
 *         ToTensor (u8 / 255) and Normalize ((x - mean[c]) / std[c]), bit-identical to
 *         the reference's evaluation transform run on the CPU
 *         (models/backbone/open_clip/transform.py:118-133, Pillow==11.1.0);
 * mean3, std3  host arrays of 3 floats (OPENAI_DATASET_MEAN / _STD for CLIP).
 * Workspace: musc_preprocess_workspace_bytes (coefficient tables, plus the uint8 output
 * of the horizontal pass when both axes are resampled and the band of source rows does
 * not fit the fused kernel's LDS, or in_w % 4 != 0).  When the fused kernel runs,
 * images must be 4-byte aligned (MUSC_ERR_INVALID_ARG otherwise).  Reduction factors up
 * to 15.5 per axis (64 taps); MUSC_ERR_UNSUPPORTED beyond, or for batch, in_h or out_h
 * above 65535. */
int musc_preprocess_workspace_bytes(int batch, int in_h, int in_w, int out_h, int out_w, size_t* out);
int musc_preprocess_u8(const uint8_t* images, int batch, int in_h, int in_w, int out_h, int out_w,
                       const float* mean3, const float* std3, float* out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* ViT block attention: out = softmax(q k^T * scale) v per (batch*head).      */
/* ------------------------------------------------------------------------ */

/* q, k, v, out  (bh, t, d) contiguous, dtype MUSC_DTYPE_F32 or MUSC_DTYPE_F16
 *               (fp16 storage, fp32 softmax and accumulation).
 * Replaces the bmm -> softmax -> bmm of nn.MultiheadAttention inside
 * models/backbone/open_clip/transformer.py:232-234 and the fused softmax
 * models/modules/_attention_gpu.py:41-81,115-146.  d must be 64. */
int musc_attention_fwd(const void* q, const void* k, const void* v, void* out,
                       int dtype, int bh, int t, int d, float scale,
                       hipStream_t stream);

/* Head-averaged attention probabilities:
 *   weights (batch, t, t) fp32 out, weights[b][i][j] = mean over heads h of
 *   softmax_j(q[b*heads+h][i] . k[b*heads+h][j] * scale); q, k (batch*heads, t, d),
 *   fp32 or fp16 (dtype), logits and probabilities in fp32.
 * Serves the one block whose weights the encoder reads (need_weights=True,
 * models/backbone/open_clip/transformer.py:232-234,331-333; the fp32 softmax the
 * reference keeps for that block, models/modules/_attention_gpu.py:41-81).
 * Workspace: musc_attention_weights_workspace_bytes (per-(head, query) softmax
 * statistics), 8-byte aligned.  d = 64, batch*heads <= 65535. */
int musc_attention_weights_workspace_bytes(int batch, int heads, int t, size_t* out);
int musc_attention_weights(const void* q, const void* k, int dtype, int batch, int heads,
                           int t, int d, float scale, float* weights,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Strided variants: head bh = b*heads + h of q, k, v lives at element
 * b*in_sb + h*in_sh + row*in_st (+ d); the output at b*out_sb + h*out_sh + row*out_st.
 * This reads nn.MultiheadAttention's packed in-projection output (t, batch, 3,
 * heads, 64) in place (q, k, v = base, base + heads*64, base + 2*heads*64;
 * in_st = batch*3*heads*64, in_sb = 3*heads*64, in_sh = 64) and writes the
 * (t, batch, heads*64) layout the out-projection takes, so the head transposes of
 * the reference's math path (torch/nn/functional.py multi_head_attention_forward,
 * called at models/backbone/open_clip/transformer.py:232-234) are not made.
 * Strides in elements, >= 0, multiples of 16 bytes; in_st, out_st >= d; the forward
 * pass reads 32-row K/V blocks through 32-bit buffer extents, so (31*in_st + d) times
 * the element size must stay below 2^31 (else MUSC_ERR_UNSUPPORTED). */
int musc_attention_fwd_strided(const void* q, const void* k, const void* v, void* out,
                               int dtype, int batch, int heads, int t, int d,
                               long long in_sb, long long in_sh, long long in_st,
                               long long out_sb, long long out_sh, long long out_st,
                               float scale, hipStream_t stream);
int musc_attention_weights_strided(const void* q, const void* k, int dtype, int batch, int heads,
                                   int t, int d, long long in_sb, long long in_sh, long long in_st,
                                   float scale, float* weights,
                                   void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Row LayerNorm over the last dimension `width` of (rows, width) x, dtype
 * MUSC_DTYPE_F32 or MUSC_DTYPE_F16, fp32 statistics and affine (weight, bias fp32,
 * either may be NULL for 1 / 0), output y in the input dtype: the cast-back
 * LayerNorm of models/backbone/open_clip/transformer.py:23-29 (under fp16 autocast:
 * fp32 layer_norm then .to(fp16)).  With residual != NULL it first forms
 * sum_out = x + residual rounded to the dtype (the residual add of
 * transformer.py:247) and normalises that (ln_2 of :248).  sum_out may alias x or
 * residual.  width % (16 bytes / element size) == 0, width <= 2048 (fp16) / 1024
 * (fp32); 16-byte aligned buffers (weight and bias included). */
int musc_layernorm_rows(const void* x, const void* residual, void* sum_out,
                        const float* weight, const float* bias, int dtype, int rows, int width,
                        float eps, void* y, hipStream_t stream);

#define MUSC_ACT_QUICK_GELU 0  /* x * sigmoid(1.702 x), transformer.py:32-35 (fp16: the
                                  three torch ops' roundings: 1.702 x, sigmoid, product) */
#define MUSC_ACT_GELU 1        /* nn.GELU (erf form), model.py:87 for non-OpenAI weights */
/* y = act(x) elementwise over n values (y may alias x); n a multiple of 16 bytes. */
int musc_activation(const void* x, void* y, int dtype, int mode, long long n, hipStream_t stream);

/* Calibration (no counterpart in the reference; a measurement aid): `blocks`
 * workgroups of 4 waves each issue iters*64 independent v_mfma_f32_32x32x2f32
 * with no memory traffic, then write one float per thread to out (blocks*256
 * floats).  *flop (host, may be NULL) receives the FLOP count of the launch, so
 * flop / time is the sustained fp32 MFMA rate of the device. */
int musc_calibrate_mfma_f32(float* out, int blocks, int iters, double* flop, hipStream_t stream);
/* The same with independent v_mfma_f32_32x32x16_f16 (the split MSM engine's
 * instruction): the sustained fp16 MFMA rate of the device. */
int musc_calibrate_mfma_f16(float* out, int blocks, int iters, double* flop, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MUSC_HIP_H */
