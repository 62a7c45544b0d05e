/*
 * ttsplat.h -- C ABI of the MI355X (gfx950) poly-splat / WSR 3DGS hot path.
 *
 * Every entry point takes device pointers allocated by the caller, plain sizes and a
 * hipStream_t; it only enqueues work on that stream (no allocation, no synchronisation),
 * so every call can be captured into a hipGraph.  (A kernel that needs more than 64 KB of LDS --
 * the step seam always, the binning's count pass on grids whose count histogram passes 64 KB --
 * raises its limit once per device with hipFuncSetAttribute on its first call: make that first
 * call outside stream capture.)  Return value: 0 on success, a negative
 * TTS_E* domain code for bad arguments (nothing is launched), or a positive hipError_t from
 * the launch.  tts_strerror() names a code.
 *
 * The reference (tt-splat) is pure Python; each entry point below replaces the Python/ttnn
 * function cited beside it (paths relative to the reference checkout).
 *
 * Shared layouts
 *   params [G,14] fp32 row-major, columns mx,my,mz, qw,qx,qy,qz, lx,ly,lz, cr,cg,cb, op
 *                 (tools/resident_traced.py:91, the fused-Adam [G,14] block :233-235)
 *   camera [16]   fp32: R_v row-major (9), t_v (3), fx, fy, cx, cy  (world->camera, OpenCV)
 *   proj   [G,12] fp32 per-gaussian record written by tts_geom_fwd, 16-byte aligned:
 *                 0 mu_x, 1 mu_y, 2 a, 3 b, 4 c (conic = Sigma2d^-1), 5 depth,
 *                 6..8 color_o = keep*sigmoid(op)*color, 9 o_col = keep*sigmoid(op),
 *                 10 sigmoid(op), 11 zero
 *   keep   [G]    uint8, depth > near
 *   bins   idx[T,K] int32 (0 in empty slots), valid[T,K] uint8; tiles row-major, T = (H/S)*(W/S)
 *   inv    [G,9]  int32 inverse bin table: inv[g][j] = t*K + slot of gaussian g in the tile it
 *                 reaches through stencil index j, or -1 (the slot table of
 *                 tools/m9_scatter_oracle.py:20-32, indexed by stencil position)
 *   image  [H,W,3] fp32 row-major; den [H,W] fp32 (WSR denominator sum(w*oc) + w_b)
 *   bg     [4]    fp32: w_b (already softplus'ed), c_b r, g, b
 *   gslot  [T,K,9] fp32 per-slot gradient of (a, b, c, mu_x, mu_y, col_o r,g,b, o_col): the
 *                 concatenated per-slot outputs [gct|gmt|gcol|goc] of tools/resident_traced.py:387-388
 *   grad9  [G,9]  fp32 per-gaussian sum of gslot over the gaussian's slots
 *                 (the scatter output of tools/resident_traced.py:383-395 / :718-727)
 *   theta  [T,6,K] fp32 monomial-major theta_u, col [T,K,3], oc [T,K] (tools/m4_train_binned.py:130-143)
 */
#ifndef TTSPLAT_H
#define TTSPLAT_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTS_OK 0
#define TTS_EINVAL (-1)     /* null pointer, non-positive size, or a size over an entry's limit */
#define TTS_ETILE (-2)      /* S not in {16,32}, H/W not a multiple of S, or over 38912 tiles */
#define TTS_EK (-3)         /* K outside [1, 512] */
#define TTS_EWORKSPACE (-4) /* workspace missing or too small */
#define TTS_ESPAN (-5)      /* quantised-distance span outside [1, 8192] */
#define TTS_EG (-6)         /* G above 2^30 (2^28 for binning) */
#define TTS_ERADIUS (-7)    /* stencil radius other than 1 */
#define TTS_ESH (-8)        /* SH degree outside [0, 3], or rest coefficients missing */
#define TTS_ESCRATCH (-9)   /* sizes beyond the fixed scratch of an allocation-free entry point */

/* Library version, (major << 16) | minor. */
int tts_version(void);

/* Static description of a return code. */
const char* tts_strerror(int code);

/* ---------------------------------------------------------------- geometry ---------- */

/* Geometry forward + activations for one camera.
 * Replaces spike/geometry.py:28-57 (project_ewa, with quat_to_rotmat :10-19 and cov3d
 * :22-25 on exp(log_scales)), spike/forward.py:69-71 (color_from_dc) and the activations of
 * tools/m4_train_binned.py:194-202; device form tools/geom_device.py:44-94.
 * Writes proj[G,12] and keep[G].  near = 0.2, blur = 0.3 in the reference. */
int tts_geom_fwd(const float* params, int G, const float* camera, float near_z, float blur,
                 float* proj, uint8_t* keep, hipStream_t stream);

/* Geometry + activation backward: grad9[G,9] -> gparams[G,14] (overwritten).
 * Replaces tools/geom_bwd.py:67-152 (bwd) and the activation part of
 * tools/operands_manual.py:83-111 (bwd_manual); device form tools/geom_device.py:106-198,
 * tools/resident_traced.py:397-427. */
int tts_geom_bwd(const float* params, int G, const float* camera, float near_z, float blur,
                 const float* grad9, float* gparams, hipStream_t stream);

/* ------------------------------------------------------------------ binning --------- */

/* Bytes of scratch tts_assign_bins needs for G gaussians on an H x W image with S x S tiles.
 * It needs no initialisation: every pass writes what the next one reads. */
size_t tts_bin_workspace_bytes(int G, int H, int W, int S);

/* Fixed-budget spatial-hash binning, R = 1: each gaussian is hashed to one S x S cell, offered
 * to the 3x3 tiles around it, and each tile keeps the K candidates nearest its centre.
 * Replaces tools/m4_train_binned.py:75-127 (assign_bins) and the dense device binning of
 * tools/bin_device.py:140-187 (with its inverse table, :219-276).  mu2d[g*mu_stride + {0,1}],
 * keep[g*keep_stride].  Order inside a tile is by (clamp(int64(dist2), 0, span-1), stencil
 * index j, gaussian id), i.e. the reference's sort key with ties in its concatenation order;
 * span = 2048 at S = 16.  Writes idx[T,K], valid[T,K]; count[T] (kept per tile), ncand[T]
 * (candidates per tile), inv[G,9] and order[T] are optional (may be NULL).  order receives the
 * tile ids sorted by kept count, heaviest first (what tts_tile_order computes, here without a
 * pass of its own).  Grids of up to 38912 tiles (T rounded up to 64; TTS_ETILE beyond). */
int tts_assign_bins(const float* mu2d, int mu_stride, const uint8_t* keep, int keep_stride,
                    int G, int H, int W, int S, int R, int K, int span,
                    int32_t* idx, uint8_t* valid, int32_t* count, int32_t* ncand, int32_t* inv,
                    int32_t* order, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Size of the fixed device scratch behind tts_assign_bins_noalloc (40 MiB per GPU: enough for
 * G = 2^20 gaussians on 1920 x 1072 at S = 16, which needs 36.4 MiB). */
#define TTS_BIN_SCRATCH_BYTES ((size_t)40 << 20)

/* tts_assign_bins without a caller workspace and without any allocation: the binning scratch
 * lives in a file-scope device array of TTS_BIN_SCRATCH_BYTES in the library (each GPU the
 * library runs on holds its own copy until the process ends; its address is looked up on the
 * first call on a device).  Same arguments, checks and results as tts_assign_bins; returns
 * TTS_ESCRATCH when tts_bin_workspace_bytes(G, H, W, S) exceeds TTS_BIN_SCRATCH_BYTES.
 * Nothing in the scratch has to start at zero, so a call does not depend on what an earlier
 * one left.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap on one GPU (different streams or threads without ordering) race.
 * No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int tts_assign_bins_noalloc(const float* mu2d, int mu_stride, const uint8_t* keep,
                            int keep_stride, int G, int H, int W, int S, int R, int K, int span,
                            int32_t* idx, uint8_t* valid, int32_t* count, int32_t* ncand,
                            int32_t* inv, int32_t* order, hipStream_t stream);

/* Tile ids ordered by kept count, heaviest first (counting sort of count[T], values in [0,K]).
 * Handing it to tts_splat_fwd / tts_splat_bwd makes the expensive tiles start first.  No
 * counterpart in the reference (whose tiles are batched matmuls of equal shape). */
int tts_tile_order(const int32_t* count, int T, int K, int32_t* order, hipStream_t stream);

/* ------------------------------------------------------------------- splat ---------- */

/* Per-tile gather + theta_u build: proj + bins -> theta[T,6,K], col[T,K,3], oc[T,K]
 * (zero in invalid slots).  Replaces tools/m4_train_binned.py:130-143 (theta_u_gathered) with
 * the gathers of :207-211 (_operands); device form tools/traced_fwd.py:63-82.  k = poly cutoff. */
int tts_theta_u_gathered(const float* proj, const int32_t* idx, const uint8_t* valid,
                         int H, int W, int S, int K, float k,
                         float* theta, float* col, float* oc, hipStream_t stream);

/* Fused binned splat forward from the per-gaussian records: gather, tile-local theta_u,
 * u = Phi.theta_u, w = relu(u)^2, C = (sum w col + w_b c_b) / (sum w oc + w_b), written
 * straight into the image.  Replaces tools/bh_views.py:65-71 on _operands
 * (tools/m4_train_binned.py:189-212) and the device chain tools/resident_traced.py:358-370.
 * den may be NULL (it is needed by tts_splat_bwd).  order (tts_tile_order) may be NULL.
 * For S = 16 each wave walks the whole tile for a quarter of the slots, u factored per pixel
 * column (images within the fp32 contract, 1e-4 of the reference; they round differently from
 * tts_splat_fwd_theta). */
int tts_splat_fwd(const float* proj, const int32_t* idx, const uint8_t* valid,
                  const int32_t* order, int H, int W, int S, int K, float k, const float* bg,
                  float* image, float* den, hipStream_t stream);

/* tts_splat_fwd on the matrix cores (S = 16 only): per 32-slot chunk, u = Phi.theta_u as one
 * bf16 MFMA whose spare contraction depth carries split-precision terms (theta in three bf16
 * parts, Phi in two), then [num|den] = w.[col_o|o_col] as a second MFMA.  bf16 = 0: w and the
 * colours split hi+lo as well (fp32-level accuracy); bf16 = 1: the bf16 render variant (w and the
 * colours rounded to bf16, fp32 accumulation; tools/resident_traced.py:265-274).
 * Same operands, outputs and tile order as tts_splat_fwd. */
int tts_splat_fwd_mx(const float* proj, const int32_t* idx, const uint8_t* valid,
                     const int32_t* order, int H, int W, int S, int K, float k, const float* bg,
                     float* image, float* den, int bf16, hipStream_t stream);

/* Splat forward from pre-gathered operands theta[T,6,K], col[T,K,3], oc[T,K].
 * Replaces _DevRenderBinned.forward, tools/m4_train_binned.py:154-166 (ops :146-151). */
int tts_splat_fwd_theta(const float* theta, const float* col, const float* oc,
                        int H, int W, int S, int K, const float* bg,
                        float* image, float* den, hipStream_t stream);

/* tts_splat_fwd_theta on bf16 operands: theta[T,6,K], col[T,K,3], oc[T,K] as bfloat16 (raw
 * 16-bit patterns), the reference's device upload (`up`, tools/m4_train_binned.py:42-43, used by
 * _DevRenderBinned.forward :154-166); arithmetic and outputs fp32. */
int tts_splat_fwd_theta_bf16(const uint16_t* theta, const uint16_t* col, const uint16_t* oc,
                             int H, int W, int S, int K, const float* bg, float* image,
                             float* den, hipStream_t stream);

/* Fused binned splat backward: given dL/dimage, recompute w per (pixel, slot), contract over
 * the tile's pixels per slot and apply the theta backward; each valid slot's 9 gradients are
 * stored to gslot[T,K,9] (entries of invalid slots are left untouched).  gwb, if not NULL,
 * receives per-tile partials of dL/dw_b ([T], the caller sums them).  Replaces
 * WSRPolySplatHot.backward (spike/backward.py:42-58) and render_bwd + theta_bwd
 * (tools/resident_traced.py:60-88).  order (tts_tile_order) may be NULL. */
int tts_splat_bwd(const float* proj, const int32_t* idx, const uint8_t* valid,
                  const int32_t* order, int H, int W, int S, int K, float k, const float* bg,
                  const float* image, const float* den, const float* gimage,
                  float* gslot, float* gwb, hipStream_t stream);

/* tts_splat_fwd (S = 16) on the slot records of tts_geom_fwd_assign_bins: tile order[p] is
 * rendered from slot_rec[p][0 .. pos_count[p]) -- the same image and den as tts_splat_fwd on
 * those bins in that order, with one read of contiguous records per tile in place of the
 * order -> idx -> proj chain.  Replaces tools/bh_views.py:65-71 and the device chain
 * tools/resident_traced.py:358-370 on the operands of the θ gather
 * (tools/m4_train_binned.py:130-143, 207-211). */
int tts_splat_fwd_rec(const float* slot_rec, const int32_t* pos_count, const int32_t* order,
                      int H, int W, int S, int K, float k, const float* bg, float* image,
                      float* den, hipStream_t stream);

/* tts_splat_fwd_mx on the slot records (S = 16; bf16 as there): the same image and den as
 * tts_splat_fwd_mx on those bins in that order, without its compaction scan and with one read
 * of contiguous records per tile. */
int tts_splat_fwd_mx_rec(const float* slot_rec, const int32_t* pos_count,
                         const int32_t* order, int H, int W, int S, int K, float k,
                         const float* bg, float* image, float* den, int bf16,
                         hipStream_t stream);

/* tts_splat_bwd (S = 16) on the slot records: the same gslot (at slot t*K + s of tile
 * t = order[p]) and gwb.  Replaces WSRPolySplatHot.backward (spike/backward.py:42-58) and
 * render_bwd + theta_bwd (tools/resident_traced.py:60-88) on the gathered operands. */
int tts_splat_bwd_rec(const float* slot_rec, const int32_t* pos_count, const int32_t* order,
                      int H, int W, int S, int K, float k, const float* bg, const float* image,
                      const float* den, const float* gimage, float* gslot, float* gwb,
                      hipStream_t stream);

/* Splat backward on pre-gathered operands: writes per-slot gtheta[T,6,K], gcol[T,K,3],
 * goc[T,K] (overwritten) and per-tile dL/dw_b partials gwb[T] (may be NULL).  Replaces
 * _DevRenderBinned.backward, tools/m4_train_binned.py:168-186. */
int tts_splat_bwd_theta(const float* theta, const float* col, const float* oc,
                        int H, int W, int S, int K, const float* bg,
                        const float* image, const float* den, const float* gimage,
                        float* gtheta, float* gcol, float* goc, float* gwb,
                        hipStream_t stream);

/* tts_splat_bwd_theta on bf16 operands (as tts_splat_fwd_theta_bf16): the backward of
 * _DevRenderBinned (tools/m4_train_binned.py:168-186) on the reference's bf16 upload; fp32
 * gradients out. */
int tts_splat_bwd_theta_bf16(const uint16_t* theta, const uint16_t* col, const uint16_t* oc,
                             int H, int W, int S, int K, const float* bg, const float* image,
                             const float* den, const float* gimage, float* gtheta, float* gcol,
                             float* goc, float* gwb, hipStream_t stream);

/* Slot -> gaussian reduce: grad9[g] = sum over the gaussian's slots of gslot, gathered through
 * inv in stencil order (deterministic, no atomics).  Replaces the device gather-reduce
 * tools/resident_traced.py:383-395 (gather_reduce, tools/m9_scatter_oracle.py:35-42). */
int tts_slot_reduce(const float* gslot, const int32_t* inv, int G, float* grad9,
                    hipStream_t stream);

/* Slot -> gaussian reduce for bins without an inverse table: grad9 (zeroed by the caller)
 * += gslot of every valid slot, with float atomics.  Replaces the host index_add of
 * tools/resident_traced.py:718-727. */
int tts_slot_scatter(const float* gslot, const int32_t* idx, const uint8_t* valid, int T, int K,
                     float* grad9, hipStream_t stream);

/* -------------------------------------------------------------------- loss ---------- */

/* Bytes of the target statistics of an H x W target: mu_y and s_y = G*y^2 - mu_y^2 of each
 * channel on the (H-10) x (W-10) valid SSIM map (six planes of floats), then the target itself
 * channel-planar (three H x W planes), which the gradient kernel reads instead of the
 * interleaved image. */
size_t tts_loss_stats_bytes(int H, int W);

/* Bytes of scratch tts_loss_grad needs: the target statistics (tts_loss_stats_bytes). */
size_t tts_loss_workspace_bytes(int H, int W);

/* Number of fp32 partial sums tts_loss_grad / tts_loss_grad_stats write.  The first *n_ssim are
 * sums of the SSIM map, the rest are sums of |x-y|:
 *   loss = (1-l) * sum|x-y| / (3HW) + l * (1 - sumS / (3 (H-10)(W-10))). */
int tts_loss_partials_count(int H, int W, int* n_ssim);

/* The target's SSIM statistics (stats: tts_loss_stats_bytes bytes, written whole), computed
 * whenever the target changes: the target maps muy/sy that tools/resident_traced.py:305-325
 * builds and recompute_gt_stats refreshes on each view switch (:677-678).  Size limits as
 * tts_loss_grad. */
int tts_loss_target_stats(const float* target, int H, int W, float* stats, hipStream_t stream);

/* A training target composited over a random background (the --random-bg mode of
 * tools/resident_traced.py:182-185,671-674, whose background is torch.rand(3) on the host):
 * bg = three uniforms in (0,1), ((w >> 8) + 0.5) * 2^-24 of words 0..2 of Philox4x32-10 with
 * counter (view, step[0], 4, 0) and key (seed, 0), step read on the device (a replayed graph
 * draws anew each step); target[H,W,3] = rgba_pm[..., c] + rgba_pm[..., 3] * bg[c], where
 * rgba_pm [H,W,4] (16-byte aligned) holds (alpha r, alpha g, alpha b, 1 - alpha); bg4[1..3] = bg
 * (the splat kernels' numerator background colour; bg4[0] = w_b is not written). */
int tts_composite_random_bg(const float* rgba_pm, int H, int W, const int32_t* step, int view,
                            unsigned seed, float* bg4, float* target, hipStream_t stream);

/* dL/dimage of L = (1-lambda)*mean|x-y| + lambda*(1 - mean SSIM(clamp(x,0,1), clamp(y,0,1))),
 * 11-tap gaussian window (sigma 1.5), valid borders, C1 = 1e-4, C2 = 9e-4, with the target's
 * statistics from tts_loss_target_stats (target must be the image they were computed from;
 * the kernel reads the planar copy inside stats): one kernel, no workspace.  Replaces the
 * device loss of tools/resident_traced.py:431-464 (its filt/filt_T banded matmuls over
 * precomputed target maps).  image, target, gimage: [H,W,3]; H, W >= 11 and H*W*24 <= 2^31-17 (TTS_EINVAL
 * otherwise: the kernels address with 32-bit buffer offsets; 7680x4320 fits).  partials (NULL
 * or tts_loss_partials_count floats) receives the partial sums. */
int tts_loss_grad_stats(const float* image, const float* target, const float* stats, int H,
                        int W, float lambda, float* gimage, float* partials, hipStream_t stream);

/* tts_loss_target_stats into the workspace, then tts_loss_grad_stats.  Replaces
 * spike/metrics.py:26-28 (loss_fn, differentiated by autograd) and the manual gradient
 * tools/loss_manual.py:76-103. */
int tts_loss_grad(const float* image, const float* target, int H, int W, float lambda,
                  float* gimage, float* partials, void* workspace, size_t workspace_bytes,
                  hipStream_t stream);

/* -------------------------------------------------------------------- adam ---------- */

/* Advance the device step counter (int32, step[0] += 1) and derive the bias corrections the
 * following tts_adam / tts_geom_bwd_adam read.  step must point at 4 int32 words (the last
 * three hold the derived fp32 factors).  Replaces the host bias-correction of
 * tools/resident_traced.py:478-481. */
int tts_adam_advance(int32_t* step, float beta1, float beta2, hipStream_t stream);

/* Adam over n = G*14 fp32 values with a per-column learning rate lr[14]; reads the factors
 * tts_adam_advance stored.  Replaces adam_fused, tools/resident_traced.py:478-490
 * (and torch.optim.Adam in spike/train.py:19). */
int tts_adam(float* params, float* m, float* v, const float* grad, const float* lr, int G,
             const int32_t* step, float beta1, float beta2, float eps, hipStream_t stream);

/* Fused slot reduce + geometry backward + Adam for one step: gslot gathered through inv ->
 * 14 gradients -> Adam update of params/m/v.  gparams (the 14 gradients) may be NULL.
 * Replaces tools/resident_traced.py:383-427 (scatter_dev + geom_bwd) + :739-740 (adam_fused). */
int tts_geom_bwd_adam(float* params, int G, const float* camera, float near_z, float blur,
                      const float* gslot, const int32_t* inv, float* gparams, float* m, float* v,
                      const float* lr, const int32_t* step, float beta1, float beta2, float eps,
                      hipStream_t stream);

/* Gradient accumulation over a batch of views: gacc[G,14] += scale * dL/dparams, with the
 * slot gradients gathered through inv and pushed through the geometry backward (as in
 * tts_geom_bwd_adam, without the Adam update).  A batch of views accumulates one view at a time;
 * tts_adam then applies the update and tts_zero clears gacc.  Replaces the reference's
 * full-batch accumulation (spike/train.py:25-31; gacc accumulation of
 * tools/resident_traced.py:718-727). */
int tts_geom_bwd_accum(const float* params, int G, const float* camera, float near_z,
                       float blur, const float* gslot, const int32_t* inv, float scale,
                       float* gacc, hipStream_t stream);

/* ---- extended geometry: view-dependent SH colour and the depth weight ----
 *
 * SH colour, degree sh_degree in [0, 3].  sh_rest holds the rest coefficients (SH indices
 * 1..15) coefficient-major:
 *   sh_rest[(l * 3 + c) * G + g], l = 0..14, channel c   (spike's color_rest[G,15,3] permuted)
 * Only the first (sh_degree+1)^2 - 1 rows are read.  colour = max(0.5 + C0*dc + sum_l b_l(dir)
 * rest_l, 0) with dir = means3d - camera centre (spike/sh.py:54-72 as used by the device step,
 * tools/resident_traced.py:246-264,339-341).  In the backward the direction is a constant
 * (tools/resident_traced.py:405-410): dL/drest_l = b_l(dir) * dL/dcolour through the clamp gate.
 *
 * Depth weight (arm B's occlusion lever, spike/arms.py:34-37; device step
 * tools/resident_traced.py:333-337,418-426): depth_bt = device (beta, tau) or NULL;
 * keo = keep * sigmoid(op) * sigmoid(beta (tau - z_cam)).  gdepth [G,2] receives each gaussian's
 * dL/d(beta, tau); tts_depth_weight_adam reduces it and updates (beta, tau).  As in the device
 * step no gradient reaches the means through z_cam, unless depth_zgrad (tts_geom_bwd_ex only) asks
 * for it (the dense arm-B autograd of spike/render.py).
 *
 * depth_zgrad of tts_geom_bwd_ex is a set of flags for the dense render's autograd
 * (spike/render.py:14-49, where nothing is detached): TTS_GRAD_DEPTH_Z adds the gradient through
 * z_cam in the depth weight, TTS_GRAD_SH_DIR the gradient of the SH colour through its view
 * direction mean - centre (both into the means). */
#define TTS_GRAD_DEPTH_Z 1
#define TTS_GRAD_SH_DIR 2

/* Geometry forward with SH colour and/or the depth weight.  Replaces the SHD > 0 and
 * --depth-weight branches of tools/resident_traced.py:327-346 (geom_fwd).
 * step_adv (optional, the training step's Adam step block): also advanced in this launch, as
 * tts_adam_advance(step_adv, beta1, beta2) would (the first kernel of a training step carries
 * the advance instead of a launch of its own).  NULL: beta1, beta2 are ignored. */
int tts_geom_fwd_ex(const float* params, const float* sh_rest, int sh_degree,
                    const float* depth_bt, int G, const float* camera, float near_z, float blur,
                    float* proj, uint8_t* keep, int32_t* step_adv, float beta1, float beta2,
                    hipStream_t stream);

/* tts_geom_fwd_ex followed by tts_assign_bins on its output (mu2d = proj, mu_stride 12, keep
 * stride 1), as one call with the results of the two: the geometry trace and the rebin that
 * follows it in the reference trainer (tools/resident_traced.py:682-686, geom_fwd :327-346,
 * do_bin :519-539 on the projected means cache["mu2d_x/y"] and keep).  The binning's count
 * pass runs inside the geometry launch, on the means it has just projected (one launch and one
 * read of proj fewer), in blocks of 512 gaussians up to G = 131072 and of 4096 above; grids whose
 * count histogram would not fit the launch's LDS take the two launches.
 * Arguments and errors as the two entry points'.
 * slot_rec [T][K][12] and pos_count [T] (optional, together, and only with order): the slot
 * records of the bins -- the projection record proj[idx[t][s]] of every kept slot s, stored at
 * slot_rec[p][s] where p is the tile's place in order (order[p] = t), and pos_count[p] =
 * count[t].  They are the per-(tile, slot) operands of the reference's θ gather
 * (tools/m4_train_binned.py:130-143, 207-211) in the order the splat kernels take their tiles;
 * tts_splat_fwd_rec / tts_splat_bwd_rec read them instead of order -> idx -> proj.  Slots at or
 * past pos_count[p] are not written. */
int tts_geom_fwd_assign_bins(const float* params, const float* sh_rest, int sh_degree,
                             const float* depth_bt, int G, const float* camera, float near_z,
                             float blur, float* proj, uint8_t* keep, int32_t* step_adv,
                             float beta1, float beta2, int H, int W, int S, int R, int K,
                             int span, int32_t* idx, uint8_t* valid, int32_t* count,
                             int32_t* ncand, int32_t* inv, int32_t* order, float* slot_rec,
                             int32_t* pos_count, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* The seam between two training steps in one launch: tts_geom_bwd_adam of step i (camera_bwd,
 * its slot gradients gslot through inv; gparams may be NULL) followed by the geometry forward
 * of step i+1 (camera_fwd, into proj and keep) and the count pass of its binning into the
 * workspace -- the first kernel of tts_geom_fwd_assign_bins for that view.  Finish the binning
 * with tts_assign_bins_counted on the same workspace.  The results equal tts_geom_bwd_adam
 * followed by tts_geom_fwd_assign_bins.  Supports the plain step only (no SH rest
 * coefficients, depth weight or MCMC terms: those take the two calls) and G <= 131072
 * (TTS_EG otherwise); no step advance (tts_assign_bins_counted carries step i+1's).  Replaces
 * the reference trainer's adam_fused of one iteration (tools/resident_traced.py:383-427,
 * 739-740) and the geom_fwd + do_bin count of the next (:682-686, geom_fwd :327-346, do_bin
 * :519-539).  The first call on a device raises the kernel's LDS limit
 * (hipFuncSetAttribute): make it outside stream capture. */
int tts_geom_bwd_adam_fwd_count(float* params, int G, const float* camera_bwd,
                                const float* camera_fwd, float near_z, float blur,
                                const float* gslot, const int32_t* inv, float* gparams, float* m,
                                float* v, const float* lr, const int32_t* step, float beta1,
                                float beta2, float eps, float* proj, uint8_t* keep, int H, int W,
                                int S, int R, int K, int span, void* workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* The rest of tts_geom_fwd_assign_bins after tts_geom_bwd_adam_fwd_count ran its count pass
 * into the workspace: the binning's column scan, scatter and select on proj / keep, with the
 * same outputs (idx, valid, count, ncand, inv, order, slot records) as that call.  step_adv
 * (optional): the training step's Adam step block, advanced by the column scan as
 * tts_adam_advance would (step i+1's advance; tools/resident_traced.py:478-481).  Replaces
 * do_bin (tools/resident_traced.py:519-539) after its count. */
int tts_assign_bins_counted(const float* proj, const uint8_t* keep, int G, int H, int W, int S,
                            int R, int K, int span, int32_t* idx, uint8_t* valid, int32_t* count,
                            int32_t* ncand, int32_t* inv, int32_t* order, float* slot_rec,
                            int32_t* pos_count, int32_t* step_adv, float beta1, float beta2,
                            void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Geometry backward with SH colour and/or the depth weight: grad9 -> gparams[G,14], gsh_rest
 * (rest layout; rows beyond the degree written as zero; needed when sh_degree > 0), gdepth [G,2]
 * (optional).  Replaces tools/resident_traced.py:397-427 (geom_bwd) with its SH and depth-weight
 * branches. */
int tts_geom_bwd_ex(const float* params, const float* sh_rest, int sh_degree,
                    const float* depth_bt, int depth_zgrad, int G, const float* camera,
                    float near_z, float blur, const float* grad9, float* gparams,
                    float* gsh_rest, float* gdepth, hipStream_t stream);

/* tts_geom_bwd_adam with the optional extensions of the device step, in one kernel:
 *  - SH colour (sh_degree > 0): the rest coefficients and their Adam moments sh_m, sh_v (rest
 *    layout) take the same Adam step with learning rate lr_sh[0] (device scalar; the reference
 *    uses the colour rate / 20).  Replaces adam_crest, tools/resident_traced.py:492-501.
 *  - depth weight (depth_bt): rho in keo, per-gaussian dL/d(beta, tau) into gdepth [G,2]
 *    (then tts_depth_weight_adam).
 *  - MCMC regulariser (lambda_o, lambda_s > 0): the gradient of lambda_o mean(sigmoid(op)) +
 *    lambda_s mean(exp(log_scales)) is added before Adam (spike/mcmc.py:18-22; device form
 *    tools/resident_traced.py:732-738).
 *  - SGLD (noise_lr > 0): after Adam, means += R(q) diag(exp(ls)) eps * sigmoid(100 ((1 - o) -
 *    0.995)) * noise_lr * lr[0] with eps three Philox4x32-10 normals for counter (g, step[0],
 *    1, 0) and key (seed, 0) (spike/mcmc.py:25-34; the reference draws eps on the host,
 *    tools/resident_traced.py:620-629).
 * sh_rest, sh_m, sh_v, lr_sh may be NULL when sh_degree is 0; depth_bt and gdepth may be NULL. */
int tts_geom_bwd_adam_ex(float* params, float* sh_rest, float* sh_m, float* sh_v, int sh_degree,
                         const float* depth_bt, float* gdepth, int G, const float* camera,
                         float near_z, float blur, const float* gslot, const int32_t* inv,
                         float* gparams, float* m, float* v, const float* lr, const float* lr_sh,
                         const int32_t* step, float beta1, float beta2, float eps,
                         float lambda_o, float lambda_s, float noise_lr, uint32_t seed,
                         hipStream_t stream);

/* tts_geom_bwd_accum with the extensions: also gacc_sh += scale * dL/drest (rest layout, when
 * sh_degree > 0) and gacc_depth[G,2] += scale * dL/d(beta, tau) (when depth_bt). */
int tts_geom_bwd_accum_ex(const float* params, const float* sh_rest, int sh_degree,
                          const float* depth_bt, int G, const float* camera, float near_z,
                          float blur, const float* gslot, const int32_t* inv, float scale,
                          float* gacc, float* gacc_sh, float* gacc_depth, hipStream_t stream);

/* Workspace of tts_depth_weight_adam for G gaussians. */
size_t tts_depth_weight_workspace_bytes(int G);

/* Sum of gdepth[G,2] over the gaussians (deterministic, fixed order) and one Adam step on the
 * device scalars depth_bt = (beta, tau) with bt_state = (m_beta, m_tau, v_beta, v_tau) and
 * learning rate lr1[0], bias factors from `step`.  Replaces adam_bt,
 * tools/resident_traced.py:503-512 (host sum + host Adam). */
int tts_depth_weight_adam(const float* gdepth, int G, float* depth_bt, float* bt_state,
                          const float* lr1, const int32_t* step, float beta1, float beta2,
                          float eps, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

/* Adam over n values with one learning rate lr1[0] (device scalar), bias factors from `step`
 * (tts_adam_advance): the SH rest block's update in batch mode (torch.optim.Adam's step for
 * one parameter group, spike/train.py:19; tools/resident_traced.py:492-501). */
int tts_adam_flat(float* params, float* m, float* v, const float* grad, const float* lr1,
                  int64_t n, const int32_t* step, float beta1, float beta2, float eps,
                  hipStream_t stream);

/* ---- fixed-count MCMC density control (spike/mcmc.py) ---- */

/* Batch form of the MCMC regulariser: grad[G,14] += d/dparams of lambda_o mean(sigmoid(op)) +
 * lambda_s mean(exp(log_scales)) (spike/mcmc.py:18-22). */
int tts_mcmc_reg_grad(const float* params, int G, float lambda_o, float lambda_s, float* grad,
                      hipStream_t stream);

/* Batch form of the SGLD step on the means (see tts_geom_bwd_adam_ex; noise scale
 * noise_lr * lr[0]).  Replaces add_sgld_noise, spike/mcmc.py:25-34. */
int tts_sgld_noise(float* params, int G, const float* lr, float noise_lr, uint32_t seed,
                   const int32_t* step, hipStream_t stream);

/* Workspace for tts_relocate (G gaussians). */
size_t tts_relocate_workspace_bytes(int G);

/* Relocation (spike/mcmc.py:41-93; host code in the reference, tools/resident_traced.py:631-663):
 * dead slots (sigmoid(op) < dead_thr), in ascending index order, each copy a live gaussian drawn
 * with probability proportional to its opacity (inverse CDF over the live gaussians in index
 * order, uniform from Philox counter (i, step[0], 2, 0), key (seed, 0)); the copy's means are
 * offset by offset * N(0,1) (Philox counter (i, step[0], 3, 0)); a target drawn n times and its
 * copies get opacity clamp(o / (n + 1), 1e-6, 1 - 1e-6); the Adam moments of dead slots and
 * targets are zeroed (m, v [G,14]; sh_m, sh_v when sh_rest is given, whose 15 rest rows are
 * copied too).  moved (optional, device int32) receives the number of relocated slots (0 when no
 * gaussian is live).  Six kernels with fixed grids: no host synchronisation, graph-capturable. */
int tts_relocate(float* params, float* m, float* v, float* sh_rest, float* sh_m, float* sh_v,
                 int G, float dead_thr, float offset, uint32_t seed, const int32_t* step,
                 int32_t* moved, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Fill n fp32 values with zero (a kernel, so graph captures hold no memset node). */
int tts_zero(float* buf, int64_t n, hipStream_t stream);

/* ---- dense (unbinned) forms, O(H*W*G): every gaussian against every pixel ---- */

/* Dense blend arms of tts_render_dense_arm (spike/arms.py). */
#define TTS_ARM_A 0   /* depth-free WSR (:22-31); arm B = A with the depth weight of tts_geom_fwd_ex */
#define TTS_ARM_SZ 1  /* soft-Z visibility prepass (:50-68) */
#define TTS_ARM_RV 2  /* revealage compositing (:71-83) */

/* Workspace for the dense backward entry points (G gaussians, P pixels). */
size_t tts_dense_workspace_bytes(int G, int P);

/* Dense arm-A render from proj[G,12]: Q = a dx^2 + 2b dx dy + c dy^2 at pixel centres
 * (col+0.5, row+0.5), w = max(0, 1 - Q/k)^2, WSR blend with bg = (w_b, c_b).  Any H, W.
 * image [H,W,3]; den [H,W] (may be NULL) = sum w*o_col + w_b.
 * Replaces spike/render.py:14-49 (arm "A": forward.quad_form + poly_splat_wgeo + arms.blend_A). */
int tts_render_dense(const float* proj, int G, int H, int W, float k, const float* bg,
                     float* image, float* den, hipStream_t stream);

/* Backward of tts_render_dense: grad9 [G,9] = dL/d(a, b, c, mu_x, mu_y, col_o rgb, o_col) (the
 * geometry backward's input), gwb[0] = dL/dw_b (gwb may be NULL).  Deterministic (band partials
 * summed in a fixed order).  Replaces autograd through spike/render.py:14-49. */
int tts_render_dense_bwd(const float* proj, int G, int H, int W, float k, const float* bg,
                         const float* image, const float* den, const float* gimage, float* grad9,
                         float* gwb, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Dense render with the per-pixel occlusion arms (arm = TTS_ARM_*): SZ computes the visible
 * front depth z* = sum W0 z / (sum W0 + 1e-6) per pixel (W0 = o w_geo, z = camera depth proj[5])
 * and blends W0 sigmoid(-softz_beta (z - z*)) by WSR (spike/arms.py:50-68); RV blends
 * C_avg (1 - R) + c_b R with revealage R = exp(sum log(1 - min(W0, 1 - 1e-4))) and no w_b
 * (:71-83).  aux [P,4] receives the per-pixel state the backward needs (SZ: z*, den0; RV: R,
 * C_avg); softz_beta is a device scalar (SZ only).  den: the WSR denominator (RV: sum W0 + 1e-6).
 * TTS_ARM_A behaves as tts_render_dense. */
int tts_render_dense_arm(const float* proj, int G, int H, int W, float k, const float* bg,
                         int arm, const float* softz_beta, float* image, float* den, float* aux,
                         hipStream_t stream);

/* Backward of tts_render_dense_arm: grad10 [G,10] = the 9 per-gaussian gradients of
 * tts_render_dense_bwd, plus (SZ) column 9 = this gaussian's share of dL/dsoftz_beta (sum over
 * the gaussians for the scalar's gradient; row stride 10 for SZ, 9 otherwise).  z enters as a
 * constant, z* does not (its gradient is a pixel pre-pass).  gwb = dL/dw_b (0 for RV). */
int tts_render_dense_arm_bwd(const float* proj, int G, int H, int W, float k, const float* bg,
                             int arm, const float* softz_beta, const float* image,
                             const float* den, const float* aux, const float* gimage,
                             float* grad10, float* gwb, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* WSR poly-splat over an explicit basis: u[p,g] = phi[p,:6] . theta[g,:6],
 * w = o[g]*keep[g]*max(u,0)^2, C [P,3] = (w@color + w_b c_b)/(sum w + w_b); den [P] may be NULL;
 * keep (u8) may be NULL (all kept).  Replaces spike/backward.py:11-20 / :23-39 (forward). */
int tts_wsr_dense(const float* theta, const float* o, const float* color, const uint8_t* keep,
                  const float* phi, int G, int P, const float* bg, float* C, float* den,
                  hipStream_t stream);

/* Backward of tts_wsr_dense: gtheta10 [G,10] = (dL/dtheta 0..5, dL/do, dL/dcolor rgb);
 * gwb[0] = dL/dw_b (may be NULL).  Replaces WSRPolySplatHot.backward, spike/backward.py:41-58. */
int tts_wsr_dense_bwd(const float* theta, const float* o, const float* color,
                      const uint8_t* keep, const float* phi, int G, int P, const float* bg,
                      const float* C, const float* den, const float* gC, float* gtheta10,
                      float* gwb, void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TTSPLAT_H */
