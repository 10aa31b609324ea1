/*
 * g2v.h -- C ABI of the MI355X (gfx950) Gaussian-to-Voxel splatting library (libg2v_hip.so).
 *
 * Drop-in boundary for the reference's pybind11 module CudaGaussianVoxelizer._C
 * (src/bindings.cpp:7-64 of lunarlab-gatech/ShelfGaussian-CudaGaussianVoxelizer).
 * Every entry point takes plain device pointers, sizes and an explicit HIP stream (passed as
 * void*, a hipStream_t); nothing allocates device memory: outputs and workspaces belong to the
 * caller, whose sizes come from the *_workspace queries.  Entry points return G2V_OK or an
 * error code; g2v_last_error() gives the message (thread-local).  Nothing calls exit().
 *
 * Conventions (reference include/utils.cuh:50-80, src/cuda_gaussian_voxelizer.cu:1511-1519):
 *   dims  X = (int)((r[3]-r[0])/s[0]) in float32 (likewise Y, Z); grid tensors are C-contiguous
 *         (X, Y, Z[, C]);  tiles 4x4x4, Tx = ceil(X/4);  tile id (tx*Ty + ty)*Tz + tz.
 *   means (N,3), opacity (N,), covariances (N,9 row-major 3x3), features (N,C): float32.
 *   cov_inv (N,9) float32; lb, ub (N,3) int32 inclusive voxel box (0,-1 when empty);
 *   nvox (N,) int32; g2t_offsets (N+1,) int32; g2t_tile_ids (M,) int32.
 */
#ifndef G2V_H
#define G2V_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G2V_OK 0
#define G2V_ERR_INVALID 1   /* bad argument (shape, null pointer, workspace too small) */
#define G2V_ERR_HIP 2       /* a HIP runtime call failed */
#define G2V_ERR_LIMIT 3     /* problem exceeds a 32-bit index (pairs, grid cells) */

/* Element type of the feature tensors (features, grid_feats, grad_features): float32, or
 * bfloat16 (grid_feats and grad_features are then rounded to nearest even from float32 sums).
 * Everything else (means, opacity, covariances, density, upstream gradients) is float32. */
#define G2V_DTYPE_F32 0
#define G2V_DTYPE_BF16 1

/* Message of the last failed call on this thread ("" if none). */
const char* g2v_last_error(void);

/* ABI version of this library. */
int g2v_abi_version(void);

/* Voxel and tile grid of a (voxel_size, voxel_range) pair, host only.
 * Reference: src/cuda_gaussian_voxelizer.cu:1511-1519. */
int g2v_grid_dims(const float voxel_size[3], const float voxel_range[6], int dims[3], int tiles[3]);

/* ---- forward ------------------------------------------------------------------------------
 * The reference forward (cuda_gaussian_voxelizer_forward, src/cuda_gaussian_voxelizer.cu:1484-1918,
 * bound at src/bindings.cpp:8-28) is split in two calls because the length M of the
 * Gaussian->Tile CSR is data dependent and the caller allocates g2t_tile_ids:
 *
 * g2v_forward_plan: per-Gaussian box, inverse covariance, voxel count and G->T row offsets
 * (reference .cu:1575-1631).  Synchronises the stream once to return M in *num_pairs.  When
 * bwd_plan_workspace is non-NULL (g2v_backward_plan_workspace(n) bytes) it also does the work of
 * g2v_backward_plan into it and returns that pair count in *num_region_pairs on the same
 * synchronisation, so that the backward needs no plan call of its own. */
size_t g2v_forward_plan_workspace(int n);
int g2v_forward_plan(int n, const float* means3D, const float* covariances,
                     const float voxel_size[3], const float voxel_range[6],
                     float* cov_inv, int* valid_voxel_lb, int* valid_voxel_ub,
                     int* num_voxels_per_gaussian, int* g2t_offsets,
                     void* workspace, size_t workspace_bytes, long long* num_pairs,
                     void* bwd_plan_workspace, size_t bwd_plan_workspace_bytes,
                     long long* num_region_pairs, void* stream);

/* g2v_forward_plan_async: the same work without the synchronisation, for callers that plan
 * several scenes and wait once: the pair counts land in counts[0] (M) and counts[1] (the
 * (region, Gaussian) pair count when bwd_plan_workspace is given, else 0) when the stream
 * reaches them.  counts is device memory or pinned host memory (hipHostMalloc, or a pinned
 * allocation of a framework's host allocator); for the latter the kernels write through the
 * device address hipHostGetDevicePointer gives, and pageable host memory is rejected.  No counterpart in the
 * reference, which handles one scene per call. */
int g2v_forward_plan_async(int n, const float* means3D, const float* covariances, const float voxel_size[3],
                           const float voxel_range[6], float* cov_inv, int* valid_voxel_lb, int* valid_voxel_ub,
                           int* num_voxels_per_gaussian, int* g2t_offsets, void* workspace, size_t workspace_bytes,
                           void* bwd_plan_workspace, size_t bwd_plan_workspace_bytes, long long* counts,
                           void* stream);

/* g2v_forward_pack_features: the features as the matrix-core splat gathers them (bfloat16
 * (hi, lo) pairs of float32 values, bfloat16 values as they are; rows padded, plus a zero row)
 * into packed (g2v_forward_packed_bytes(n, feat_dim) bytes).  It depends on the features alone,
 * so a caller queues it before waiting for the plan's pair count (g2v_forward_plan_async), and
 * it runs while the host waits.  Part of the reference's forward (.cu:1634-1904), which gathers
 * the float32 rows directly.  Asynchronous. */
size_t g2v_forward_packed_bytes(int n, int feat_dim);
int g2v_forward_pack_features(int n, int feat_dim, const void* features, int feat_dtype, void* packed,
                              size_t packed_bytes, void* stream);

/* g2v_forward_splat: G->T fill, radix sort into the Tile->Gaussian CSR, per-tile splat of the
 * density and, when feat_dim > 0, of the density-weighted feature average (reference
 * .cu:1634-1904).  density (X,Y,Z) and grid_feats (X,Y,Z,feat_dim) are written completely;
 * features and packed_features may be NULL when feat_dim == 0; otherwise packed_features holds
 * g2v_forward_pack_features's output for the same features, queued before on the same stream,
 * in packed_bytes >= g2v_forward_packed_bytes(n, feat_dim) bytes (a smaller buffer, one packed
 * for fewer Gaussians or channels, is rejected with G2V_ERR_INVALID).
 * When t2g_tiles, t2g_gauss (M each) and t2g_offsets (T+1) are all non-NULL the
 * Tile->Gaussian CSR is built there (and can be handed to g2v_backward, which then skips
 * rebuilding it); otherwise it lives in the workspace.  The workspace also holds a 64-byte
 * packed record per Gaussian that the splat's tile kernels gather (included in the size
 * g2v_forward_splat_workspace returns).  Asynchronous. */
size_t g2v_forward_splat_workspace(int n, int feat_dim, long long num_pairs, const float voxel_size[3],
                                   const float voxel_range[6]);
int g2v_forward_splat(int n, int feat_dim, const float* means3D, const float* opacity,
                      const void* features, int feat_dtype, const void* packed_features, size_t packed_bytes,
                      const float voxel_size[3], const float voxel_range[6], const float* cov_inv,
                      const int* valid_voxel_lb, const int* valid_voxel_ub, const int* g2t_offsets,
                      long long num_pairs, int* g2t_tile_ids, float* density, void* grid_feats, int* t2g_tiles,
                      int* t2g_gauss, int* t2g_offsets, void* workspace, size_t workspace_bytes, void* stream);

/* ---- backward -----------------------------------------------------------------------------
 * Replaces cuda_gaussian_voxelizer_backward (src/cuda_gaussian_voxelizer.cu:1920-2057, bound at
 * src/bindings.cpp:30-64), in two calls like the forward:
 *
 * g2v_backward_plan: with features, counts the (region, Gaussian) pairs of the feature-gradient
 * phase (regions of 2x2x4 tiles) into plan_workspace and synchronises the stream once to return
 * their number; without features it does nothing and returns 0. */
size_t g2v_backward_plan_workspace(int n);
int g2v_backward_plan(int n, int feat_dim, const float voxel_size[3], const float voxel_range[6],
                      const int* valid_voxel_lb, const int* valid_voxel_ub, void* plan_workspace,
                      size_t plan_workspace_bytes, long long* num_region_pairs, void* stream);

/* g2v_backward: writes grad_means (N,3), grad_cov (N,9, symmetric), grad_opacity (N,) and, when
 * feat_dim > 0, grad_features (N,feat_dim).  grad_feats (X,Y,Z,feat_dim), grid_feats, features
 * and grad_features are all of feat_dtype (float32 or bfloat16; a bfloat16 grad_feats is
 * multiplied as it is, with float32 accumulation).  grad_feats/grid_feats/features may be NULL when
 * feat_dim == 0.  plan_workspace is the one given to g2v_backward_plan.  t2g_tiles, t2g_gauss
 * and t2g_offsets may carry the Tile->Gaussian CSR written by g2v_forward_splat for the same
 * Gaussians (all three non-NULL); with NULL it is rebuilt from g2t_offsets/g2t_tile_ids, as the
 * reference's backward signature provides only those.  Asynchronous; atomic-free and
 * deterministic. */
size_t g2v_backward_workspace(int n, int feat_dim, long long num_pairs, long long num_region_pairs,
                              const float voxel_size[3], const float voxel_range[6]);
int g2v_backward(int n, int feat_dim, const float* grad_density, const void* grad_feats,
                 const float* means3D, const float* opacity, const float* cov_inv,
                 const float voxel_size[3], const float voxel_range[6],
                 const int* valid_voxel_lb, const int* valid_voxel_ub,
                 const int* num_voxels_per_gaussian, const int* g2t_offsets,
                 const int* g2t_tile_ids, long long num_pairs, long long num_region_pairs,
                 const float* density, const void* grid_feats, const void* features, int feat_dtype,
                 float* grad_means, float* grad_cov, float* grad_opacity, void* grad_features,
                 const int* t2g_tiles, const int* t2g_gauss, const int* t2g_offsets,
                 const void* plan_workspace, void* workspace, size_t workspace_bytes, void* stream);

/* g2v_backward_prepare: the part of g2v_backward that needs no upstream gradient, for the
 * feature case (feat_dim > 0): the bf16 split of the features, the (region, Gaussian) CSR and the
 * row table of the feature-gradient phase, written into workspace (g2v_backward_workspace bytes).
 * It needs the forward's Tile->Gaussian CSR (t2g_tiles, t2g_gauss from g2v_forward_splat) and the
 * backward plan.  No counterpart in the reference, whose backward starts with the upstream
 * gradients: a caller that blocks between forward and backward (the reference's module waits for
 * the forward to finish, to report its time) can queue this behind the forward so that it runs
 * while the host hands over to the backward.  Asynchronous.
 *
 * g2v_backward_prepared: g2v_backward, for a workspace that g2v_backward_prepare has filled for the
 * same Gaussians, features, CSR and plan (and that nothing has written since); it skips those
 * kernels.  Requires the Tile->Gaussian CSR arguments. */
int g2v_backward_prepare(int n, int feat_dim, const float voxel_size[3], const float voxel_range[6],
                         const int* valid_voxel_lb, const int* valid_voxel_ub, const void* features,
                         int feat_dtype, long long num_pairs, long long num_region_pairs, const int* t2g_tiles,
                         const int* t2g_gauss, const void* plan_workspace, void* workspace,
                         size_t workspace_bytes, void* stream);
int g2v_backward_prepared(int n, int feat_dim, const float* grad_density, const void* grad_feats,
                          const float* means3D, const float* opacity, const float* cov_inv,
                          const float voxel_size[3], const float voxel_range[6],
                          const int* valid_voxel_lb, const int* valid_voxel_ub,
                          const int* num_voxels_per_gaussian, const int* g2t_offsets,
                          const int* g2t_tile_ids, long long num_pairs, long long num_region_pairs,
                          const float* density, const void* grid_feats, const void* features, int feat_dtype,
                          float* grad_means, float* grad_cov, float* grad_opacity, void* grad_features,
                          const int* t2g_tiles, const int* t2g_gauss, const int* t2g_offsets,
                          const void* plan_workspace, void* workspace, size_t workspace_bytes, void* stream);

/* g2v_backward_cosine: g2v_backward when the upstream gradient of grid_feats is that of the
 * feature cosine loss (g2v_cosine_loss_forward_coef on this grid_feats and pseudo_gt), fused into
 * the feature backward.  The reference chains the two through autograd (CudaGaussianVoxelizer/
 * __init__.py:36-67): src/cuda_feats_loss.cu:233-366 writes the gradient of grid_feats and
 * src/cuda_gaussian_voxelizer.cu:1920-2057 reads it.  Instead of reading an (X,Y,Z,feat_dim)
 * grad_feats, the kernels form it per voxel on chip as
 *     k1 pseudo_gt + k2 grid_feats,  (k1, k2) = coef[2v .. 2v+1] * grad_loss[0] / num_valid_voxel
 * (0 when num_valid_voxel == 0), the expression of g2v_cosine_loss_backward, so the gradient is
 * never written to or read from memory.  grad_loss is the device float upstream gradient of the
 * loss.  float32 features (feat_dtype G2V_DTYPE_F32) with feat_dim % 4 == 0; pseudo_gt and
 * grid_feats 16-byte aligned.  prepared != 0: the workspace was filled by g2v_backward_prepare
 * (as for g2v_backward_prepared; the Tile->Gaussian CSR arguments are then required).  The other
 * arguments are g2v_backward's.  Asynchronous. */
int g2v_backward_cosine(int n, int feat_dim, const float* grad_density, const float* grad_loss,
                        const void* pseudo_gt, const float* coef, int num_valid_voxel,
                        const float* means3D, const float* opacity, const float* cov_inv,
                        const float voxel_size[3], const float voxel_range[6],
                        const int* valid_voxel_lb, const int* valid_voxel_ub,
                        const int* num_voxels_per_gaussian, const int* g2t_offsets,
                        const int* g2t_tile_ids, long long num_pairs, long long num_region_pairs,
                        const float* density, const void* grid_feats, const void* features, int feat_dtype,
                        float* grad_means, float* grad_cov, float* grad_opacity, void* grad_features,
                        const int* t2g_tiles, const int* t2g_gauss, const int* t2g_offsets,
                        const void* plan_workspace, void* workspace, size_t workspace_bytes, int prepared,
                        void* stream);

/* ---- Tile->Gaussian CSR (inspection) -------------------------------------------------------
 * The internal Tile->Gaussian CSR of the forward, for parity tests: the stable sort of the G->T
 * pairs by tile (sorted_tiles, sorted_gauss: M each; reference .cu:1673-1691), the list bounds of
 * every tile (tile_offsets: T+1), and the run-length encoding of the sorted tiles (unique_tiles,
 * counts: T each, runs_offsets: T+1, *num_runs on the device; reference .cu:1708-1772). */
size_t g2v_t2g_workspace(int n, long long num_pairs, const float voxel_size[3],
                         const float voxel_range[6]);
int g2v_build_t2g(int n, const float voxel_size[3], const float voxel_range[6],
                  const int* valid_voxel_lb, const int* valid_voxel_ub, const int* g2t_offsets,
                  const int* g2t_tile_ids, long long num_pairs, int* sorted_tiles,
                  int* sorted_gauss, int* tile_offsets, int* unique_tiles, int* counts,
                  int* runs_offsets, int* num_runs, void* workspace, size_t workspace_bytes,
                  void* stream);

/* ---- batches of scenes on one grid -------------------------------------------------------------
 * No counterpart in the reference, which takes one scene per call; ShelfGaussian batches B scenes
 * (its recorded batch holds (1, 6, 300) Gaussians).  B scenes of n Gaussians each on one
 * (voxel_size, voxel_range) grid run as one problem of B n Gaussians on B T tiles: one launch per
 * kernel for the whole batch instead of one per scene.  Inputs are scene-major (B, n, ...) arrays,
 * outputs (B, X, Y, Z) and (B, X, Y, Z, feat_dim); cov_inv, lb, ub and nvox are (B, n, ...) with the
 * values of single-scene calls, and every per-scene output equals that of g2v_forward_plan /
 * g2v_forward_splat / g2v_backward on the scene alone, bit for bit.
 *
 * g2v_batch_forward_plan: boxes, inverse covariances and the per-scene G->T row offsets
 * g2t_offsets (B, n+1) of every scene, scene-local as g2v_forward_plan writes them; the batch's own
 * offsets stay in plan_workspace (g2v_batch_plan_workspace bytes), which the caller keeps until the
 * batch's backward.  counts (B + 1 long longs, device-accessible: device or pinned host memory)
 * receives each scene's pair count M_b and, last, the batch's (region, Gaussian) pair count when
 * want_backward != 0 (else 0).  Asynchronous: the caller waits once for the whole batch.
 *
 * g2v_batch_forward_splat: the splat of the batch, num_pairs = sum of M_b.  g2t_tile_ids (num_pairs,
 * optional) receives the scene-local tile ids of scene 0's pairs, then scene 1's, ...; density and
 * grid_feats are written completely; t2g_tiles, t2g_gauss (num_pairs) and t2g_offsets (B T + 1),
 * when all non-NULL, receive the batch's Tile->Gaussian CSR (batch tile ids b T + t, batch
 * Gaussian ids b n + g) for the backward.
 *
 * g2v_batch_backward_prepare / g2v_batch_backward: g2v_backward_prepare and g2v_backward
 * (prepared != 0: as g2v_backward_prepared) for the batch, with num_pairs and num_region_pairs the
 * batch's totals, plan_workspace the batch plan's (planned with want_backward != 0 when
 * feat_dim > 0) and the batch's Tile->Gaussian CSR from g2v_batch_forward_splat (optional without
 * prepared: rebuilt from the boxes).  Gradients are (B, n, ...).  Asynchronous. */
size_t g2v_batch_plan_workspace(int num_scenes, int n);
int g2v_batch_forward_plan(int num_scenes, int n, const float* means3D, const float* covariances,
                           const float voxel_size[3], const float voxel_range[6], float* cov_inv, int* valid_voxel_lb,
                           int* valid_voxel_ub, int* num_voxels_per_gaussian, int* g2t_offsets, void* plan_workspace,
                           size_t plan_workspace_bytes, int want_backward, long long* counts, void* stream);
size_t g2v_batch_forward_splat_workspace(int num_scenes, int n, int feat_dim, long long num_pairs,
                                         const float voxel_size[3], const float voxel_range[6]);
int g2v_batch_forward_splat(int num_scenes, int n, int feat_dim, const float* means3D, const float* opacity,
                            const void* features, int feat_dtype, const float voxel_size[3],
                            const float voxel_range[6], const float* cov_inv, const int* valid_voxel_lb,
                            const int* valid_voxel_ub, const void* plan_workspace, size_t plan_workspace_bytes,
                            long long num_pairs, int* g2t_tile_ids, float* density, void* grid_feats, int* t2g_tiles,
                            int* t2g_gauss, int* t2g_offsets, void* workspace, size_t workspace_bytes, void* stream);
size_t g2v_batch_backward_workspace(int num_scenes, int n, int feat_dim, long long num_pairs,
                                    long long num_region_pairs, const float voxel_size[3], const float voxel_range[6]);
int g2v_batch_backward_prepare(int num_scenes, int n, int feat_dim, const float voxel_size[3],
                               const float voxel_range[6], const int* valid_voxel_lb, const int* valid_voxel_ub,
                               const void* features, int feat_dtype, long long num_pairs, long long num_region_pairs,
                               const int* t2g_tiles, const int* t2g_gauss, const void* plan_workspace,
                               size_t plan_workspace_bytes, void* workspace, size_t workspace_bytes, void* stream);
int g2v_batch_backward(int num_scenes, int n, int feat_dim, const float* grad_density, const void* grad_feats,
                       const float* means3D, const float* opacity, const float* cov_inv, const float voxel_size[3],
                       const float voxel_range[6], const int* valid_voxel_lb, const int* valid_voxel_ub,
                       long long num_pairs, long long num_region_pairs, const float* density, const void* grid_feats,
                       const void* features, int feat_dtype, float* grad_means, float* grad_cov, float* grad_opacity,
                       void* grad_features, const int* t2g_tiles, const int* t2g_gauss, const int* t2g_offsets,
                       const void* plan_workspace, size_t plan_workspace_bytes, void* workspace,
                       size_t workspace_bytes, int prepared, void* stream);

/* ---- feature cosine loss --------------------------------------------------------------------
 * Replaces CudaFeatsCosinelossForward / CudaFeatsCosinelossBackward (src/cuda_feats_loss.cu:154-231
 * and :311-366, bound at src/bindings.cpp:67-104).  Over num_voxels = X*Y*Z voxels with
 * voxel_label (X,Y,Z) float32, occ_mask (X,Y,Z) bool (one byte, 0 or 1), grid_feats and pseudo_gt
 * (X,Y,Z,feat_dim) of feat_dtype (G2V_DTYPE_F32, as the reference, or G2V_DTYPE_BF16: both tensors,
 * and grad_grid_feats, then hold bfloat16; the sums are float32), a voxel is valid when
 * occ_mask != 0 and voxel_label > 0, and
 *     loss = mean over valid voxels of 1 - p.g / (sqrt(max(|p|^2,1e-6)) sqrt(max(|g|^2,1e-6)) + 1e-6)
 * (0 when no voxel is valid).
 *
 * g2v_cosine_loss_forward writes the loss (a device float) and the valid-voxel count (a device
 * int); when num_valid_host is non-NULL it also synchronises the stream once and returns the count
 * there (the reference returns it to Python as an int).  Deterministic: fixed summation order.
 * The workspace (g2v_cosine_loss_workspace bytes) holds per-block partial sums. */
size_t g2v_cosine_loss_workspace(long long num_voxels, int feat_dim);
int g2v_cosine_loss_forward(long long num_voxels, int feat_dim, const float* voxel_label,
                            const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                            int feat_dtype, float* loss, int* num_valid, int* num_valid_host, void* workspace,
                            size_t workspace_bytes, void* stream);

/* g2v_cosine_loss_forward_coef: g2v_cosine_loss_forward that also writes, for g2v_backward_cosine,
 * the unscaled gradient coefficients of every voxel into coef (num_voxels x 2 floats, 8-byte
 * aligned): (c1, c2) with d loss / d grid_feats = (c1 pseudo_gt + c2 grid_feats) grad / count on a
 * valid voxel (reference src/cuda_feats_loss.cu:278-291), (0, 0) on the others. */
int g2v_cosine_loss_forward_coef(long long num_voxels, int feat_dim, const float* voxel_label,
                                 const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                                 int feat_dtype, float* loss, int* num_valid, int* num_valid_host, float* coef,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* g2v_cosine_loss_forward_noalloc: g2v_cosine_loss_forward without a workspace and without the
 * host count, for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  No counterpart in the reference.  The block
 * partial sums live in a 32 KiB device array of the library (one per GPU, held until the process
 * ends), which fits the partials of any num_voxels up to INT32_MAX (larger counts are rejected with
 * G2V_ERR_LIMIT); calls that overlap on one GPU share it and race.  Same kernels, so the same
 * results, bit for bit.  Asynchronous; allocates nothing. */
int g2v_cosine_loss_forward_noalloc(long long num_voxels, int feat_dim, const float* voxel_label,
                                    const unsigned char* occ_mask, const void* grid_feats, const void* pseudo_gt,
                                    int feat_dtype, float* loss, int* num_valid, void* stream);

/* g2v_cosine_loss_backward writes d loss / d grid_feats (X,Y,Z,feat_dim) for the upstream scalar
 * gradient grad_output (a device float: no host read, where the reference calls .item()) and the
 * forward's valid-voxel count; zero on invalid voxels.  Asynchronous, needs no workspace. */
int g2v_cosine_loss_backward(long long num_voxels, int feat_dim, const float* grad_output,
                             const float* voxel_label, const unsigned char* occ_mask, const void* grid_feats,
                             const void* pseudo_gt, int feat_dtype, int num_valid_voxel, void* grad_grid_feats,
                             void* stream);

/* ---- covariances from scales and rotations -------------------------------------------------
 * The covariance construction that ShelfGaussian runs before the voxelizer (reference
 * test/gaussian_voxelizer.py:14-37 quat_to_rotmat / get_covariance, called at :168-169), for
 * callers that hold scales (N,3) and rotation quaternions (N,4, real part first, not necessarily
 * normalised) instead of covariances: covariances (N,9) = R diag(s) (R diag(s))^T row-major, R the
 * rotation of q/|q|.  The backward maps grad_covariances (N,9, e.g. g2v_backward's grad_cov) to
 * grad_scales (N,3) and grad_rotations (N,4).  Asynchronous. */
int g2v_covariance_from_scale_rotation(int n, const float* scales, const float* rotations, float* covariances,
                                       void* stream);
int g2v_covariance_from_scale_rotation_backward(int n, const float* scales, const float* rotations,
                                                const float* grad_covariances, float* grad_scales,
                                                float* grad_rotations, void* stream);

/* ---- per-kernel timing (benchmarks) --------------------------------------------------------
 * No counterpart in the reference (which times the whole forward/backward with one CUDA event
 * pair, src/cuda_gaussian_voxelizer.cu:1549-1555, :1905-1913).  While enabled, every kernel launch
 * of the library is bracketed by two HIP events on its stream.  g2v_profile_collect() waits for
 * the recorded events and returns the number of distinct kernels; g2v_profile_entry(i, ...) gives
 * the name, launch count and total milliseconds of kernel i since the last reset. */
int g2v_profile_enable(int on);
int g2v_profile_reset(void);
int g2v_profile_collect(void);
int g2v_profile_entry(int i, char* name, int name_len, long long* launches, double* total_ms);

#ifdef __cplusplus
}
#endif

#endif /* G2V_H */
