/*
 * gs_rasterizer.h — C ABI of the MI355X (gfx950) Gaussian-splatting rasterizer.
 *
 * Every entry point takes raw device pointers, element counts and the caller's
 * HIP stream, enqueues its kernels on that stream and returns an int status:
 *   0            success
 *   > 0          a hipError_t reported by the HIP runtime (launch or API failure)
 *   < 0          one of the GS_ERR_* argument errors below (nothing was launched)
 * No entry point allocates device memory; scratch space is passed in by the
 * caller (query its size with the *_workspace_size functions), except in
 * gs_ssim_forward_noalloc, which keeps it in a static device array.  No entry point
 * synchronises the stream.  Outputs are written in full (culled / masked
 * entries are written as zero), so callers need not pre-clear them, except
 * where an entry point documents accumulation.
 *
 * Layouts follow the reference extension module `cuda_rasterizer`
 * (src/cuda/rasterizer.cpp:442-464): fp32 row-major AoS tensors, quaternions
 * in (x, y, z, w) order, world_to_camera a row-major 4x4 world->camera matrix
 * (OpenCV axes, u = fx*x/z + cx), intrinsic a row-major 3x3 matrix, masks one
 * byte per Gaussian (0/1), ids and tile offsets int32.
 */
#ifndef GS_RASTERIZER_H
#define GS_RASTERIZER_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    GS_OK = 0,
    GS_ERR_INVALID_ARGUMENT = -1,   /* negative size, null required pointer, bad tile size */
    GS_ERR_WORKSPACE_TOO_SMALL = -2,/* workspace_bytes below the *_workspace_size result */
    GS_ERR_TOO_MANY_KEYS = -3,      /* more than INT32_MAX (tile, Gaussian) keys */
    GS_ERR_UNSUPPORTED = -4,        /* argument combination this build does not implement */
};

/* Human-readable text for a status returned by any gs_* function. */
const char *gs_status_string(int status);

/* Version of this ABI (incremented on any signature change). */
int gs_abi_version(void);

/* The device address of pinned host memory (hipHostMalloc) for the current
 * device, for entries that write a few values straight to the host (e.g. the
 * totals of gs_bin_count).  Non-zero status (and *device = NULL) when the
 * memory is not mapped for the device.  No counterpart in the reference. */
int gs_host_device_pointer(void *host, void **device);

/* ---------------------------------------------------------------- preprocess */

/*
 * Projection of N Gaussians into the image plane.
 * Replaces cuda_rasterizer.project_points (src/cuda/rasterizer.cpp:140-191,
 * kernel src/cuda/kernel.cu:411-500); culling follows the Torch rasterizer
 * (src/torch_rasterizer.py:47-144): keep iff opacity >= min_opacity,
 * near < z < far, the 2D covariance is finite, min_radius <= r <= max_radius
 * and -r_u < u < W + r_u, -r_v < v < H + r_v.
 * Outputs (N rows each): points_image (u,v), depths (z), cov_image (a,b,c),
 * cov_inv_image (conic A,B,C), radii (r_u,r_v), mask (1 = kept).
 */
int gs_project_points(const float *means, const float *scales, const float *quaternions,
                      const float *opacities, const float *world_to_camera,
                      const float *intrinsic, int64_t n, float near_plane, float far_plane,
                      float min_opacity, float min_radius, float max_radius, int32_t width,
                      int32_t height, float *points_image, float *depths, float *cov_image,
                      float *cov_inv_image, float *radii, uint8_t *mask, hipStream_t stream);

/*
 * Gradient of project_points w.r.t. means, scales and quaternions.
 * Replaces cuda_rasterizer.project_points_backward
 * (src/cuda/rasterizer.cpp:193-232, kernel src/cuda/kernel.cu:502-543); the
 * Jacobian term is the exact derivative of the forward (the reference's
 * kernel.cu:381-394 doubles the off-diagonal term; this one does not).
 */
int gs_project_points_backward(const float *grad_points_image, const float *grad_cov_inv_image,
                               const float *means, const float *scales,
                               const float *quaternions, const float *opacities,
                               const float *world_to_camera, const float *intrinsic, int64_t n,
                               int32_t width, int32_t height, const float *cov_image,
                               const uint8_t *mask, float *grad_means, float *grad_scales,
                               float *grad_quaternions, hipStream_t stream);

/*
 * Degree-3 real spherical harmonics -> RGB along the view direction
 * normalize(mean - camera_pos).  Replaces
 * cuda_rasterizer.evaluate_spherical_harmonics (src/cuda/rasterizer.cpp:234-257,
 * kernel src/cuda/kernel.cu:545-617).  sh_rest is (N,15,3).  Masked rows are 0.
 * sh_sigmoid != 0 applies a sigmoid to the result.
 */
int gs_evaluate_sh(const float *camera_pos, const float *means, const float *sh_dc,
                   const float *sh_rest, const uint8_t *mask, int64_t n, int32_t sh_sigmoid,
                   float *colors, hipStream_t stream);

/*
 * Gradient of gs_evaluate_sh.  Replaces
 * cuda_rasterizer.evaluate_spherical_harmonics_backward
 * (src/cuda/rasterizer.cpp:259-290, kernel src/cuda/kernel.cu:619-782).
 */
int gs_evaluate_sh_backward(const float *grad_colors, const float *camera_pos,
                            const float *means, const float *sh_dc, const float *sh_rest,
                            const float *colors, const uint8_t *mask, int64_t n,
                            int32_t sh_sigmoid, float *grad_means, float *grad_sh_dc,
                            float *grad_sh_rest, hipStream_t stream);

/* ------------------------------------------------------------------- binning */

/*
 * compute_tile_intersection (src/cuda/rasterizer.cpp:292-359) in two phases
 * around the one host read of the entry counts:
 *
 *   gs_bin_count: the tile rectangle of every Gaussian (tiles_touched,
 *     kernel.cu:784-818 semantics), a stable sort of the Gaussians with tiles
 *     by depth bits, and the placement of their supertile entries (a supertile
 *     is 8 x 8 tiles): per-supertile counts and positions when the grid has at
 *     most 256 supertiles, else an exclusive scan.  Writes two int64:
 *     totals[0] = K, the number of (tile, Gaussian) keys, and totals[1] = M,
 *     the number of (supertile, Gaussian) entries (M <= K).  Keeps its state in
 *     `workspace`, which gs_bin_sort reads.
 *   gs_bin_sort: sorts the M entries by supertile (depth order kept), then
 *     expands every supertile list to its tiles and writes each Gaussian id
 *     once, at its final position.  The result equals a stable sort of the
 *     reference's 64-bit keys (tile_id << 32 | depth_bits) emitted in Gaussian
 *     order (kernel.cu:820-914): entries ordered by (tile, depth bits,
 *     Gaussian index).  indexing_offset[t] = number of entries with tile < t
 *     (one int32 per tile).  Optional outputs (may be NULL): sorted_keys (K
 *     uint64, the 64-bit keys in sorted order) and tiles_touched (N int32).
 *     The workspace size depends on M and the image/tile geometry only.
 *
 * gs_bin_count = gs_bin_count_begin followed by gs_bin_count_finish (same
 * arguments).  totals is final once the work gs_bin_count_begin launched has
 * run, and nothing writes it after that, so a caller can queue its copy of
 * totals between the two calls and wait for that copy after queueing
 * gs_bin_count_finish: the host read of K and M then overlaps the second phase
 * instead of idling the GPU (the reference reads num_rendered with .item()
 * after all of its counting, rasterizer.cpp:322).  totals may also be pinned
 * host memory the device can write (hipHostMalloc): the host then reads it
 * directly after an event recorded between the two calls, with no copy.
 */
int gs_bin_count_workspace_size(int64_t n, size_t *bytes);
int gs_bin_count(const float *points_image, const float *radii, const float *depths,
                 const uint8_t *mask, int64_t n, int32_t width, int32_t height,
                 int32_t tile_size, void *workspace, size_t workspace_bytes, int64_t *totals,
                 hipStream_t stream);
int gs_bin_count_begin(const float *points_image, const float *radii, const float *depths,
                       const uint8_t *mask, int64_t n, int32_t width, int32_t height,
                       int32_t tile_size, void *workspace, size_t workspace_bytes,
                       int64_t *totals, hipStream_t stream);
int gs_bin_count_finish(const float *points_image, const float *radii, const float *depths,
                        const uint8_t *mask, int64_t n, int32_t width, int32_t height,
                        int32_t tile_size, void *workspace, size_t workspace_bytes,
                        int64_t *totals, hipStream_t stream);

/*
 * gs_bin_count_begin with a depth hint and four totals.  The depth sort orders
 * the keys (depth bits) by a 16-bit bucket and then by the whole key; its
 * transform {kmin, shift} maps key -> (key - kmin) >> shift clamped to
 * [0, 0xFFFF], which keeps the order of any keys.  gs_bin_count_begin derives
 * it from the least and greatest key with tiles, which costs a launch; here the
 * caller supplies it (hint_kmin, hint_shift in 0..16; hint_shift < 0: derived
 * as in gs_bin_count_begin), e.g. from the previous call's totals, and the count
 * kernel histograms the first depth pass itself.  The outputs are the same
 * for every hint; a hint far from the keys' range only puts many keys in one
 * bucket, which the segment sort then sorts more slowly.  totals: 4 entries --
 * K, M, the least and the greatest depth key (bits) of the Gaussians with
 * tiles (0xFFFFFFFF and 0 when there is none).  Follow it with
 * gs_bin_count_finish as after gs_bin_count_begin.  No counterpart in the
 * reference extension (which sorts 64-bit keys and needs no transform).
 */
int gs_bin_count_begin_hinted(const float *points_image, const float *radii,
                              const float *depths, const uint8_t *mask, int64_t n,
                              int32_t width, int32_t height, int32_t tile_size,
                              void *workspace, size_t workspace_bytes, uint32_t hint_kmin,
                              int32_t hint_shift, int64_t *totals, hipStream_t stream);
int gs_bin_sort_workspace_size(int64_t n, int64_t k, int64_t m, int32_t width, int32_t height,
                               int32_t tile_size, size_t *bytes);
int gs_bin_sort(const float *points_image, const float *radii, const float *depths, int64_t n,
                int32_t width, int32_t height, int32_t tile_size, int64_t k, int64_t m,
                const void *count_workspace, void *workspace, size_t workspace_bytes,
                int32_t *indexing_offset, int32_t *gaussian_ids_sorted, uint64_t *sorted_keys,
                int32_t *tiles_touched, hipStream_t stream);

/*
 * gs_bin_sort that also writes launch_order (n_tiles int32, required): a launch
 * order for gs_rasterize_display_l1's forward_order, computed from the tile
 * lists alone.  Within each XCD's tile range (the ranges the blend kernels use:
 * with base = n_tiles / 8 and rem = n_tiles % 8, range x starts at
 * x * base + min(x, rem) and holds base + (x < rem) tiles), the range's tiles by
 * ascending bit length of their list length (0, 1, 2-3, 4-7, ...), in tile
 * order within each of those buckets.  Measured at 1920x1080 it shortens the
 * forward by 10-20 us against tile order (the tiles with the longest lists,
 * which start after the first wave of tiles, are not the slowest); it changes
 * no result.  The order comes from extra workgroups of the last binning launch.
 * No counterpart in the reference extension.
 */
int gs_bin_sort_ordered(const float *points_image, const float *radii, const float *depths,
                        int64_t n, int32_t width, int32_t height, int32_t tile_size, int64_t k,
                        int64_t m, const void *count_workspace, void *workspace,
                        size_t workspace_bytes, int32_t *indexing_offset,
                        int32_t *gaussian_ids_sorted, uint64_t *sorted_keys,
                        int32_t *tiles_touched, int32_t *launch_order, hipStream_t stream);

/*
 * gs_bin_sort_ordered sized by capacities instead of K and M, so that it can be
 * queued before the host has read them: K and M come from count_workspace on
 * the device (written by the gs_bin_count_begin* call that filled it).  The
 * workspace is sized by gs_bin_sort_workspace_size(n, k_capacity, m_capacity,
 * ...); gaussian_ids_sorted holds k_capacity ids.  With K <= k_capacity and
 * M <= m_capacity the lists are the exact ones, shifted by k_capacity - K:
 * indexing_offset[t] is K's offset plus that shift, so the lists end at
 * k_capacity and (indexing_offset, gaussian_ids_sorted, k_capacity) is a valid
 * input of every blend entry (ids[0 .. k_capacity - K) belong to no tile).
 * Otherwise nothing is written but indexing_offset, all k_capacity (every tile
 * empty), and launch_order; the caller reads K and M (the totals of the count)
 * and redoes the binning with exact sizes.  Grids of at most 256 supertiles of
 * 8x8 tiles (16384 tiles; e.g. up to 2048x2048 at tile size 16), else
 * GS_ERR_UNSUPPORTED.  No counterpart in the reference extension (its
 * rasterizer.cpp:322 reads num_rendered with .item() before sizing the sort).
 */
int gs_bin_sort_capped(const float *points_image, const float *radii, const float *depths,
                       int64_t n, int32_t width, int32_t height, int32_t tile_size,
                       int64_t k_capacity, int64_t m_capacity, const void *count_workspace,
                       void *workspace, size_t workspace_bytes, int32_t *indexing_offset,
                       int32_t *gaussian_ids_sorted, int32_t *launch_order,
                       hipStream_t stream);

/* --------------------------------------------------------------------- blend */

/*
 * Waves per 16x16 tile of the blend kernels (every gs_rasterize* entry with
 * tile_size 16): 0, the default, picks by the tile count (4 waves for grids of
 * at most 1024 tiles; above that 1, except the forward entries, which take 2
 * up to 6144 tiles); 1, 2 or 4 force that count.  With
 * W waves, wave w composites strips w * 4/W .. of the tile's four 16x4 strips
 * and the waves share each staged batch.  Images are bit-equal for every
 * setting; gradients and the per-tile loss sums differ only in float summation
 * order.  Process-wide; not synchronised with launches in flight.  No
 * counterpart in the reference extension.
 */
int gs_set_blend_waves(int32_t waves);

/*
 * Front-to-back alpha compositing of each tile's sorted Gaussian list.
 * Replaces cuda_rasterizer.rasterize (src/cuda/rasterizer.cpp:361-395, kernel
 * src/cuda/kernel.cu:916-987) with the Torch rasterizer's inclusion rules
 * (src/torch_rasterizer.py:262-282): a Gaussian contributes to pixel (x,y)
 * (integer coordinates) iff E < chi_squared_threshold, alpha >= alpha_threshold
 * and the transmittance before it is >= transmittance_threshold.
 * image is (H,W,3), un-clamped, no background.  n_tiles = length of
 * indexing_offset, k = length of gaussian_ids_sorted.  NaN thresholds are
 * rejected with GS_ERR_INVALID_ARGUMENT (here and in the blend entries below).
 */
int gs_rasterize(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                 int32_t n_tiles, int64_t k, const float *points_image,
                 const float *cov_inv_image, const float *opacities, const float *colors,
                 int64_t n, int32_t width, int32_t height, int32_t tile_size,
                 float alpha_threshold, float transmittance_threshold,
                 float chi_squared_threshold, float *image, hipStream_t stream);

/*
 * Gradient of gs_rasterize w.r.t. points_image, cov_inv_image, opacities and
 * colors.  Replaces cuda_rasterizer.rasterize_backward
 * (src/cuda/rasterizer.cpp:397-440, kernel src/cuda/kernel.cu:989-1111).
 * `image` is the forward output for the same inputs, or NULL (the kernel then
 * recomputes it).  accumulate == 0: the four gradient outputs are overwritten;
 * accumulate != 0: the gradients are added to their current contents (e.g. to
 * sum over cameras into buffers the caller zeroed once).
 */
int gs_rasterize_backward(const float *grad_image, const float *image,
                          const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                          int32_t n_tiles, int64_t k, const float *points_image,
                          const float *cov_inv_image, const float *opacities,
                          const float *colors, int64_t n, int32_t width, int32_t height,
                          int32_t tile_size, float alpha_threshold,
                          float transmittance_threshold, float chi_squared_threshold,
                          float *grad_points_image, float *grad_cov_inv_image,
                          float *grad_opacities, float *grad_colors, int32_t accumulate,
                          hipStream_t stream);

/* ------------------------------------------------------- render() fusions */

/*
 * Fused forms of what render() does around the seven functions
 * (src/cuda/wrapper.py:223-294); each equals the unfused sequence.  No
 * counterpart in the reference extension.
 *
 * gs_evaluate_sh_render: colors = max(gs_evaluate_sh(camera_pos, ...) + 0.5, 0)
 *   with camera_pos = -R^T t taken from world_to_camera
 *   (src/cuda/wrapper.py:260-265); masked rows are 0.5.
 * gs_evaluate_sh_render_beside: gs_evaluate_sh_render (the same values) for a
 *   stream that runs beside other work, such as binning's chain of small
 *   launches: one workgroup per compute unit (more beyond 32 Gaussians per
 *   thread) walks the Gaussians, leaving the rest of each unit's slots to the
 *   other stream.
 * gs_evaluate_sh_render_cache: gs_evaluate_sh_render (beside = 0) or
 *   gs_evaluate_sh_render_beside (beside != 0) that also writes the colour-
 *   gradient cache sh_cache: 10 floats per Gaussian (8-byte aligned), the
 *   rows d raw_c / d mean (c = 0..2, through the view direction) and, in the
 *   tenth, the clamp's pass bits as a uint32 (bit c where raw_c + 0.5 >= 0);
 *   rows outside the mask are not written.  gs_render_preprocess_backward and
 *   gs_preprocess_backward take it in place of sh_dc and sh_rest, which they
 *   then do not read (the same results, bit for bit).  No counterpart in the
 *   reference extension.
 * gs_evaluate_sh_render_backward: its gradient (the clamp passes the gradient
 *   where raw + 0.5 >= 0, as torch.clamp_min does); accumulate_means != 0 adds
 *   the means gradient to grad_means instead of overwriting it.
 * gs_rasterize_display: gs_rasterize that also writes
 *   display = clamp(image, 0, 1) * 255 (src/cuda/wrapper.py:294); tile_size 16.
 *   tile_schedule: null, or gs_tile_schedule_size(n_tiles) int32 that receive
 *   the work per tile, the backward's launch order and the walk's checkpoints
 *   (as in gs_rasterize_display_l1).
 *   forward_order: null or a launch order of the tiles, as in
 *   gs_rasterize_display_l1 (e.g. gs_bin_sort_ordered's).
 * gs_rasterize_display_backward: gs_rasterize_backward given the gradient of
 *   display (image required): the image gradient is grad_display * 255 where
 *   0 <= image <= 1, else 0.  tile_schedule: null, or the buffer that
 *   gs_rasterize_display filled for the same tile layout (the tiles then start
 *   heaviest first; the results do not depend on it).
 */
int gs_evaluate_sh_render(const float *world_to_camera, const float *means, const float *sh_dc,
                          const float *sh_rest, const uint8_t *mask, int64_t n, float *colors,
                          hipStream_t stream);
int gs_evaluate_sh_render_beside(const float *world_to_camera, const float *means,
                                 const float *sh_dc, const float *sh_rest, const uint8_t *mask,
                                 int64_t n, float *colors, hipStream_t stream);
int gs_evaluate_sh_render_cache(const float *world_to_camera, const float *means,
                                const float *sh_dc, const float *sh_rest, const uint8_t *mask,
                                int64_t n, int32_t beside, float *colors, float *sh_cache,
                                hipStream_t stream);
int gs_evaluate_sh_render_backward(const float *grad_colors, const float *world_to_camera,
                                   const float *means, const float *sh_dc, const float *sh_rest,
                                   const uint8_t *mask, int64_t n, int32_t accumulate_means,
                                   float *grad_means, float *grad_sh_dc, float *grad_sh_rest,
                                   hipStream_t stream);
int gs_rasterize_display(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                         int32_t n_tiles, int64_t k, const float *points_image,
                         const float *cov_inv_image, const float *opacities, const float *colors,
                         int64_t n, int32_t width, int32_t height, int32_t tile_size,
                         float alpha_threshold, float transmittance_threshold,
                         float chi_squared_threshold, float *image, float *display,
                         int32_t *tile_schedule, const int32_t *forward_order,
                         hipStream_t stream);
int gs_rasterize_display_backward(const float *grad_display, const float *image,
                                  const int32_t *indexing_offset,
                                  const int32_t *gaussian_ids_sorted, int32_t n_tiles, int64_t k,
                                  const float *points_image, const float *cov_inv_image,
                                  const float *opacities, const float *colors, int64_t n,
                                  int32_t width, int32_t height, int32_t tile_size,
                                  float alpha_threshold, float transmittance_threshold,
                                  float chi_squared_threshold, float *grad_points_image,
                                  float *grad_cov_inv_image, float *grad_opacities,
                                  float *grad_colors, int32_t accumulate,
                                  const int32_t *tile_schedule, hipStream_t stream);

/* ----------------------------------------------- fused training step */

/*
 * Fused preprocess of the library training step: activations
 * (scripts/train.py:135-143), projection (as gs_project_points) and the
 * render() colour max(SH + 0.5, 0) (as gs_evaluate_sh_render) in one pass over
 * each Gaussian's raw parameters; opacities receives sigmoid(logits) for the
 * blend.  gs_preprocess_backward takes the gradients of points_image,
 * cov_inv_image, opacities and colors and writes those of the raw parameters
 * (means, log-scales, raw quaternions, logits, SH dc and rest), recomputing the
 * activations.  Each equals the unfused sequence of the entries it replaces.
 * No counterpart in the reference extension (it leaves activations to PyTorch).
 * quats_raw and grad_quats_raw must be 16-byte aligned.  With colors NULL the
 * forward skips the colours (sh_dc and sh_rest may then be NULL): a caller can
 * compute them with gs_evaluate_sh_render_beside on another stream, beside
 * binning.  sh_cache: NULL, or (with colors) the colour-gradient cache that
 * gs_evaluate_sh_render_cache describes, written beside the colours; given to
 * gs_preprocess_backward (sh_dc and sh_rest may then be NULL) it replaces the
 * backward's read of the 180-byte SH rows with 40 bytes per Gaussian.
 */
int gs_preprocess_forward(const float *means, const float *log_scales, const float *quats_raw,
                          const float *opacity_logits, const float *sh_dc, const float *sh_rest,
                          const float *world_to_camera, const float *intrinsic, int64_t n,
                          float near_plane, float far_plane, float min_opacity, float min_radius,
                          float max_radius, int32_t width, int32_t height, float *points_image,
                          float *depths, float *cov_image, float *cov_inv_image, float *radii,
                          uint8_t *mask, float *opacities, float *colors, float *sh_cache,
                          hipStream_t stream);
int gs_preprocess_backward(const float *grad_points_image, const float *grad_cov_inv_image,
                           const float *grad_opacities, const float *grad_colors,
                           const float *means, const float *log_scales, const float *quats_raw,
                           const float *opacity_logits, const float *sh_dc, const float *sh_rest,
                           const float *cov_image, const uint8_t *mask,
                           const float *world_to_camera, const float *intrinsic, int64_t n,
                           int32_t width, int32_t height, float *grad_means,
                           float *grad_log_scales, float *grad_quats_raw,
                           float *grad_opacity_logits, float *grad_sh_dc, float *grad_sh_rest,
                           const float *sh_cache, hipStream_t stream);

/*
 * The drop-in render()'s backward of projection and colours in one pass:
 * gs_project_points_backward (src/cuda/rasterizer.cpp:193-232) and
 * gs_evaluate_sh_render_backward (the colour max(SH + 0.5, 0) of
 * src/cuda/wrapper.py:260-265, backward of rasterizer.cpp:259-290), with
 * grad_means the sum of the two means gradients.  Inputs as those entries take
 * them: scales and quaternions as rendered (no activation), cov_image and mask
 * from gs_project_points, sh_rest (N, 15, 3).  Each output equals the
 * corresponding output of the two entries (the means: their sum).  No
 * counterpart in the reference extension, whose wrapper runs the two
 * backwards as separate autograd nodes.  sh_cache: NULL, or the cache
 * gs_evaluate_sh_render_cache wrote for the same inputs (sh_dc and sh_rest may
 * then be NULL).
 */
int gs_render_preprocess_backward(const float *grad_points_image,
                                  const float *grad_cov_inv_image, const float *grad_colors,
                                  const float *means, const float *scales,
                                  const float *quaternions, const float *sh_dc,
                                  const float *sh_rest, const float *cov_image,
                                  const uint8_t *mask, const float *world_to_camera,
                                  const float *intrinsic, int64_t n, int32_t width,
                                  int32_t height, float *grad_means, float *grad_scales,
                                  float *grad_quaternions, float *grad_sh_dc, float *grad_sh_rest,
                                  const float *sh_cache, hipStream_t stream);

/*
 * The caller-side glue of a training step (scripts/train.py:135-143,187-191),
 * fused: no counterpart in the reference extension.
 *
 * gs_activate: scales = exp(log_scales), quaternions = q / max(|q|, 1e-12),
 *   opacities = sigmoid(logits) (N rows; quaternion rows 16-byte aligned).
 * gs_activate_backward: maps gradients of those outputs (any may be NULL =
 *   zero) to log_scales, raw quaternions and logits.
 * gs_rasterize_display_l1: gs_rasterize_display that also writes, per tile,
 *   the sum over its pixels of |display / 255 - target| (tile_loss, one float
 *   per tile; n_tiles must cover the image; tile_size 16).  When clear is set,
 *   it also writes clear_count zeros there (in the blend kernel when clear is
 *   16-byte aligned and clear_count a multiple of 4): the accumulators that
 *   gs_rasterize_l1_backward then adds into with accumulate = 1, without a
 *   separate fill.  When loss is set, loss = sum(tile_loss) / (H * W * 3) is
 *   written as well (the gs_l1_finish result).  When tile_schedule is set
 *   (gs_tile_schedule_size(n_tiles) int32), the forward's work per tile goes to
 *   elements [0, n_tiles) and the backward's launch order to [n_tiles,
 *   2 n_tiles): per XCD's tile range, the tiles by descending work, so that
 *   gs_rasterize_l1_backward, given the same buffer, starts the heaviest tiles
 *   first.  The rest receives checkpoints of each tile's walk: every 128 list
 *   entries (every batch of 256 with 4 waves per tile), at most 3 times, each
 *   pixel's transmittance and accumulated colour, from which the backward walks
 *   the tile in up to 4 segments on as many workgroups (the results do not
 *   depend on either, up to float rounding).
 *   forward_order: null (each XCD's range in tile order), or elements
 *   [n_tiles, 2 n_tiles) of a tile_schedule buffer that an earlier call filled
 *   for the same tile grid, e.g. the last render of the same view in a training
 *   loop that visits
 *   a fixed set of views: this forward then also starts its heaviest tiles (as
 *   they were then) first.  It must be a permutation of every XCD range (such a
 *   buffer is); the results do not depend on it.
 * gs_l1_finish: loss = sum(tile_loss) / count (count = H * W * 3), one float.
 * gs_rasterize_l1_backward: gs_rasterize_backward seeded by
 *   loss = mean(|clamp(image, 0, 1) * 255 / 255 - target|) with upstream
 *   gradient *grad_loss (device float): the image gradient is computed per
 *   pixel from image and target (image required; tile_size 16), the L1 term
 *   weighted by loss_scale (1 for the plain L1 loss; 1 - lambda in the
 *   reference's L1 + SSIM loss).  When grad_display01 is set (an (H, W, 3)
 *   image), it is a further gradient with respect to display / 255 (e.g. of an
 *   SSIM term on the same image, scripts/train.py:185-205), added to the L1
 *   one at that node.  tile_schedule: null, or the buffer that
 *   gs_rasterize_display_l1 filled for the same tile layout and image (its
 *   order is a permutation of the tiles and its checkpoints belong to that
 *   forward; other contents give wrong gradients, never an access outside the
 *   lists: segment bounds are clamped into each tile's list).  With it the
 *   tiles that have checkpoints run in segments.
 * gs_tile_schedule_size: the int32 elements of a tile_schedule buffer for
 *   n_tiles tiles: 2 n_tiles (work, order), n_tiles checkpoint counts,
 *   3 n_tiles checkpoint positions, 3 n_tiles work counts, 4 n_tiles
 *   segment-list entries, 8 list lengths (the forward's launch of the order
 *   writes the lists: per XCD tile range, the segments of its tiles by
 *   descending work), padded to 16 bytes, then
 *   3 * 256 * 4 floats per tile (2 for n_tiles = 0).  Grids of more than 6144
 *   tiles take no checkpoints (the backward starts one workgroup per tile, more
 *   than the GPU holds at once, which balances them already): 2 n_tiles.  No counterpart in the reference (its
 *   backward is one thread per pixel over the whole list,
 *   src/cuda/kernel.cu:989-1111).
 */
int gs_activate(const float *log_scales, const float *quats_raw, const float *opacity_logits,
                int64_t n, float *scales, float *quats, float *opacities, hipStream_t stream);
int gs_activate_backward(const float *grad_scales, const float *grad_quats,
                         const float *grad_opacities, const float *scales,
                         const float *quats_raw, const float *opacities, int64_t n,
                         float *grad_log_scales, float *grad_quats_raw,
                         float *grad_opacity_logits, hipStream_t stream);
int gs_rasterize_display_l1(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                            int32_t n_tiles, int64_t k, const float *points_image,
                            const float *cov_inv_image, const float *opacities,
                            const float *colors, int64_t n, int32_t width, int32_t height,
                            int32_t tile_size, float alpha_threshold,
                            float transmittance_threshold, float chi_squared_threshold,
                            const float *target, float *image, float *display, float *tile_loss,
                            float *loss, int32_t *tile_schedule, float *clear,
                            int64_t clear_count, const int32_t *forward_order,
                            hipStream_t stream);
int gs_l1_finish(const float *tile_loss, int32_t n_tiles, int64_t count, float *loss,
                 hipStream_t stream);
int gs_rasterize_l1_backward(const float *target, const float *grad_loss, const float *image,
                             const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                             int32_t n_tiles, int64_t k, const float *points_image,
                             const float *cov_inv_image, const float *opacities,
                             const float *colors, int64_t n, int32_t width, int32_t height,
                             int32_t tile_size, float alpha_threshold,
                             float transmittance_threshold, float chi_squared_threshold,
                             float *grad_points_image, float *grad_cov_inv_image,
                             float *grad_opacities, float *grad_colors, int32_t accumulate,
                             float loss_scale, const float *grad_display01,
                             const int32_t *tile_schedule, hipStream_t stream);
int gs_tile_schedule_size(int32_t n_tiles, size_t *elements);

/* ------------------------------------------------------------ training loop */

/*
 * Kernels for the optimizer and densification steps of the training loop
 * (scripts/train.py:17-44,211-222; src/strategy.py:47-229).  No counterpart
 * in the reference extension (it leaves these to PyTorch).
 *
 * gs_adam_step: one launch updates every tensor of the list (torch.optim.Adam
 *   without weight decay / amsgrad): m = b1 m + (1-b1) g, v = b2 v + (1-b2) g^2,
 *   p -= step_size * m / (sqrt(v) / bias_correction2_sqrt + eps), with
 *   step_size = lr / (1 - b1^t) and bias_correction2_sqrt = sqrt(1 - b2^t)
 *   given per tensor.  grad may be NULL (a zero gradient).  The betas and eps
 *   are doubles, as the Python scalars of torch.optim.Adam are: 1 - beta is
 *   formed in double and rounded once to float, as PyTorch does.
 * gs_accumulate_grad2d: src/strategy.py:47-68 -- for Gaussians whose two radii
 *   are > 0, grads += |(du * W/2, dv * H/2)| and count += 1.
 * gs_gather_rows: dst row r = src row src_rows[r] (+ delta row r when delta is
 *   set) for every tensor of the list, or zeros where fresh_rows[r] != 0 and
 *   the tensor has zero_fresh (optimizer state of new Gaussians).  Rebuilds
 *   parameters and optimizer state after prune / clone / split in one launch.
 */
typedef struct {
    float *param;
    const float *grad;
    float *exp_avg;
    float *exp_avg_sq;
    int64_t count;
    float step_size;
    float bias_correction2_sqrt;
} GsAdamTensor;

typedef struct {
    const float *src;
    float *dst;
    const float *delta;
    int32_t width;
    int32_t zero_fresh;
} GsGatherTensor;

int gs_adam_step(const GsAdamTensor *tensors, int32_t n_tensors, double beta1, double beta2,
                 double eps, hipStream_t stream);
int gs_accumulate_grad2d(const float *grad_points_image, const float *radii, int64_t n,
                         int32_t width, int32_t height, float *grads, float *count,
                         hipStream_t stream);
int gs_gather_rows(int64_t n_out, const int32_t *src_rows, const uint8_t *fresh_rows,
                   const GsGatherTensor *tensors, int32_t n_tensors, hipStream_t stream);

/* -------------------------------------------------------------- SSIM loss */

/*
 * Replace fused_ssim(img1, img2, padding, train) of the third-party package
 * fused-ssim (fused-ssim==0.0.0, environment.yml:56; not vendored), which the
 * reference's loss calls at scripts/train.py:193-197 (also
 * scripts/check_cuda_gradients.py:976-980 and scripts/evaluate.py:57-61).
 * Images are float32 (batch, channels, height, width) with element strides
 * strides[0..3] (host arrays of 4; any layout -- the reference passes (H, W, C)
 * images permuted to (1, C, H, W)).  SSIM per pixel: 11x11 Gaussian window of
 * standard deviation 1.5 per plane, zero padding, C1 = 0.01^2, C2 = 0.03^2.
 *
 * The SSIM sees img1's elements times 1 / img1_divisor, the reciprocal rounded
 *   to float (1: as stored; 255 for a [0, 255] display image: the values equal
 *   PyTorch's GPU rendered_image / 255.0, which multiplies by that reciprocal).
 * gs_ssim_forward: *ssim_mean (device float) = mean of the SSIM map over every
 *   pixel (valid_padding = 0) or over the pixels at least 5 from the border
 *   (valid_padding = 1; NaN when that region is empty).  The three map pointers
 *   are all NULL or all set; when set, each receives a planar
 *   (batch * channels, height, width) map -- d mean / d E[x], d mean / d E[x^2]
 *   and d mean / d E[xy] per pixel, with mu1 = E[x], E[x^2] and E[xy] taken as
 *   the independent local statistics (zero outside the region) -- for
 *   gs_ssim_backward.  The mean is reduced in a fixed order (deterministic).
 *   When loss is set, also *loss = (1 - lambda) * *other_loss + lambda *
 *   (1 - mean): the reference's training loss (scripts/train.py:205).
 * gs_ssim_backward: grad_img1 (element strides grad_strides) = grad_scale *
 *   *grad_mean (device float) times d(mean SSIM)/d x, x = img1 / img1_divisor.
 *   img2 gets no gradient.
 * batch * channels must be <= 65535.  Strides must be >= 0, a plane's last
 * element lie less than 2^31 elements past its first and a row's last less
 * than 2^30 past its first (GS_ERR_UNSUPPORTED otherwise).
 */
int gs_ssim_workspace_size(int32_t batch, int32_t channels, int32_t height, int32_t width,
                           size_t *bytes);
int gs_ssim_forward(const float *img1, const int64_t *strides1, const float *img2,
                    const int64_t *strides2, int32_t batch, int32_t channels, int32_t height,
                    int32_t width, int32_t valid_padding, float img1_divisor, float *ssim_mean,
                    float *dm_dmu1, float *dm_dsigma1_sq, float *dm_dsigma12,
                    const float *other_loss, float lambda, float *loss, void *workspace,
                    size_t workspace_bytes, hipStream_t stream);
/*
 * gs_ssim_forward_noalloc: gs_ssim_forward without a workspace argument; it
 *   allocates nothing and keeps its per-workgroup partials in a static device
 *   array of 1024 doubles (8 KiB) that each GPU the library runs on holds until
 *   the process ends.  No counterpart in the reference: it is for callers that
 *   cannot allocate (code under HIP graph capture, tight serving loops).  The
 *   current device must be the device of `stream`.  Every call on one GPU uses
 *   the same array: calls that overlap on that GPU (on different streams) race.
 *   Geometries beyond the array are rejected with GS_ERR_WORKSPACE_TOO_SMALL
 *   (none exist: the forward runs at most 1024 workgroups).
 */
int gs_ssim_forward_noalloc(const float *img1, const int64_t *strides1, const float *img2,
                            const int64_t *strides2, int32_t batch, int32_t channels,
                            int32_t height, int32_t width, int32_t valid_padding,
                            float img1_divisor, float *ssim_mean, float *dm_dmu1,
                            float *dm_dsigma1_sq, float *dm_dsigma12, const float *other_loss,
                            float lambda, float *loss, hipStream_t stream);
int gs_ssim_backward(const float *grad_mean, const float *img1, const int64_t *strides1,
                     const float *img2, const int64_t *strides2, int32_t batch, int32_t channels,
                     int32_t height, int32_t width, float img1_divisor, const float *dm_dmu1,
                     const float *dm_dsigma1_sq, const float *dm_dsigma12, float grad_scale,
                     float *grad_img1, const int64_t *grad_strides, hipStream_t stream);

/*
 * Measurement entry (no counterpart in the reference): the work of the
 * reference blend loop (src/cuda/kernel.cu:954-982) for the same inputs as
 * gs_rasterize.  *visited = sum over pixels of the list entries walked until
 * the transmittance test stops the pixel; *composited = entries that passed
 * the chi-square and alpha tests and were blended.  Both are device uint64
 * counters (overwritten).  Used to express blend throughput in flop/s.
 */
int gs_rasterize_work(const int32_t *indexing_offset, const int32_t *gaussian_ids_sorted,
                      int32_t n_tiles, int64_t k, const float *points_image,
                      const float *cov_inv_image, const float *opacities, int64_t n,
                      int32_t width, int32_t height, int32_t tile_size, float alpha_threshold,
                      float transmittance_threshold, float chi_squared_threshold,
                      uint64_t *visited, uint64_t *composited, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GS_RASTERIZER_H */
