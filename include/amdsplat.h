/*
 * amdsplat: C ABI of the MI355X (gfx950) Gaussian-splat rasterizer.
 *
 * Calling model (every entry point):
 *   - All array arguments are DEVICE pointers owned by the caller, except the gs_camera
 *     struct and the background colour, which are host memory read during the call.
 *   - `stream` is a hipStream_t (NULL = default stream). Work is only enqueued; nothing
 *     synchronises, allocates or copies between host and device.
 *   - Return value: 0 on success, otherwise a GS_ERR_* code; gs_last_error() then returns
 *     a message (thread-local). A failed call enqueues nothing.
 *   - Sizes are element counts. Layouts are C-contiguous.
 *
 * The 3D path replaces Faster-GS's _C.forward / _C.backward (called at
 * phase1/tests/test_parity.py:90,97-98 and cluster/patches/fastergs_lean_adam.patch:328-345):
 *   gs_preprocess_fwd -> gs_bin_prepare_3d -> [host reads M, the sum of the preprocess's
 *   wave_counts] -> gs_bin_fill_3d -> gs_blend_fwd_3d;   backward: gs_blend_bwd_3d ->
 *   gs_preprocess_bwd.
 * The 2D entry points replace the extension functions of toy2d/csrc/rasterize.cu:366-448
 * and phase0/csrc/macrotile/bindings.cpp:156-239.
 */
#ifndef AMDSPLAT_H
#define AMDSPLAT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  GS_OK = 0,
  GS_ERR_ARG = 1,        /* invalid argument (null pointer, negative size, bad enum) */
  GS_ERR_WORKSPACE = 2,  /* workspace smaller than the size query returned */
  GS_ERR_LAUNCH = 3,     /* the HIP runtime rejected a launch */
  GS_ERR_ALIGN = 4       /* a pointer does not have the required alignment */
};

/* Rule sets (the three operator surfaces) and floating types of the 2D entry points. */
enum {
  GS_RULES_3D = 0,      /* 3D rasterize: Faster-GS rules (phase1/fastergs_macro.patch:181-205) */
  GS_RULES_TOY2D = 1,   /* gs2d.rasterize: toy2d/csrc/rasterize.cu:37-101, toy2d/gs2d/reference.py:3-8 */
  GS_RULES_PHASE0 = 2   /* splat2d.render: phase0/csrc/macrotile/splat2d_common.h:7-11 */
};
enum { GS_FLOAT32 = 0, GS_FLOAT64 = 1, GS_BFLOAT16 = 2 };

/* Pinhole camera. viewmat is the row-major 4x4 world-to-camera matrix with OpenCV axes
 * (x right, y down, z forward); pixel (i, j) covers [i, i+1) x [j, j+1), so its centre is
 * at (i + 0.5, j + 0.5). flags: GS_CAM_* bits (0 = the plain rules). */
typedef struct gs_camera {
  float viewmat[16];
  float fx, fy, cx, cy;
  int32_t width, height;
  float near_plane, far_plane; /* near_plane must be > 0 */
  int32_t flags;
} gs_camera;

/* Faster-GS's proper_antialiasing setting (phase1/tests/test_parity.py:82, consumed at
 * phase1/fastergs_macro.patch:215): the blended opacity is o * sqrt(max(det S / det S', 0)),
 * S the projected 2D covariance and S' = S + 0.3 I the dilated one (the Mip-Splatting 2D
 * filter), and its gradient flows through the compensation factor into the covariance. */
#define GS_CAM_PROPER_ANTIALIASING 1

/* Binning path (gs_camera.flags for the 3D entry points, the flags argument of
 * gs_bin_fill_rect): by default the span binning is taken from GS_BIN_SPAN_MIN_GAUSSIANS
 * Gaussians on canvases of at most GS_BIN_SPAN_MAX_TILES tiles per side, otherwise the radix
 * path; these bits force one of them (GS_BIN_SPANS only where the canvas allows it). Both give
 * the same lists, ranges and bucket offsets. */
#define GS_BIN_SPANS 2
#define GS_BIN_RADIX 4
#define GS_BIN_SPAN_MIN_GAUSSIANS 2000000
/* gs_bin_path values: the 3D fill's path for a camera and Gaussian count */
enum { GS_BIN_PATH_RADIX = 0, GS_BIN_PATH_SPANS = 1 };

/* Thread-local message of the last failed call. */
const char* gs_last_error(void);

/* Library version and the number of bytes of a splat record / screen-gradient record. */
int gs_version(void);
int gs_splat_record_floats(void);  /* 16: mean2d, conic, opacity, depth, threshold, rgb, mask, bounds */
int gs_grad2d_floats(void);        /* 12 */

/* ---------------------------------------------------------------------------------------
 * Exclusive prefix sum of n uint32 values: out[0] = 0, out[i] = in[0] + ... + in[i-1],
 * out[n] = total. `out` holds n + 1 values. Workspace from gs_scan_workspace_size(n).
 * Replaces torch.cumsum in toy2d/gs2d/binning.py:76-85 and cub DeviceScan in Faster-GS.
 * ------------------------------------------------------------------------------------- */
size_t gs_scan_workspace_size(int64_t n);
int gs_scan_u32(const uint32_t* in, uint32_t* out, int64_t n, void* workspace,
                size_t workspace_bytes, void* stream);

/* out[0] = in[0] + ... + in[n-1] as a uint64 (one workgroup, no workspace). With the
 * preprocess's wave_counts it gives the instance count m as one value to copy to the host
 * (Faster-GS reads the count back after its scan, phase2/fastergs_readback.patch:46-85). */
int gs_sum_u32(const uint32_t* in, int64_t n, uint64_t* out, void* stream);

/* The instance count read back to the host without draining `stream`: gs_count_begin enqueues
 * the sum of wave_counts[0 .. n_waves), stored by its kernel straight into pinned host memory,
 * on `stream` itself (on_side_stream 0: the work enqueued after it waits for the 3-5 us sum, and
 * the call costs the host one launch) or on a side stream of the library's (default priority)
 * that waits for the work enqueued so far on `stream` (on_side_stream 1: nothing on `stream`
 * waits, at the cost of an event record and a stream wait on the host); gs_count_end (same
 * thread, same current device) waits for that kernel only and returns the sum in *m. The two are the exceptions to "nothing synchronises or copies": per
 * host thread and device, the side stream, two events and an 8-byte pinned, coherent host word
 * are created on first use and kept until the process ends. A second gs_count_begin before gs_count_end on the same thread and device is an
 * error. (Faster-GS reads the count after its tiles_touched scan, with the stream drained,
 * phase2/fastergs_readback.patch:46-85.) */
int gs_count_begin(const uint32_t* wave_counts, int64_t n_waves, int on_side_stream, void* stream);
int gs_count_end(uint64_t* m);

/* ---------------------------------------------------------------------------------------
 * 3D preprocess forward (replaces Faster-GS preprocess_cu; signature evidence
 * results/phase1/garden_main_4475452_5k_cuda_gpu_kern_sum.csv:7). Per Gaussian: view
 * transform, near/far culling, opacity = sigmoid(logit), covariance from exp(log_scales)
 * and the normalised quaternion (w, x, y, z), EWA projection with a 0.3 px^2 dilation,
 * conic, SH colour of degree sh_degree (+0.5, clamped at 0), the alpha >= 1/255 ellipse
 * bounds, and the number of 16x16 tiles the ellipse reaches (0 = culled).
 *   means, log_scales [n,3]; quats [n,4]; opacity_logits [n]; sh [n, sh_coeffs, 3] with
 *   sh_coeffs in {1,4,9,16} and (sh_degree+1)^2 <= sh_coeffs; or, with sh_rest not NULL, the
 *   DC coefficients sh [n, 1, 3] and the rest sh_rest [n, sh_coeffs - 1, 3] as two arrays (the
 *   sh_coefficients_0 / sh_coefficients_rest split of Faster-GS's model).
 *   out: splat_rec [n,16] floats (16-byte aligned; a culled Gaussian's record gets only the
 *   empty bounds (0, -1, 0, -1) in its last 4 words), tiles_touched [n] uint32, and (may be
 *   NULL) depth_keys [n] uint32: the orderable bits of the view depth of a Gaussian with
 *   tiles, 0xffffffff for a culled one (the keys gs_bin_prepare_3d sorts by).
 *   wave_counts (may be NULL): [ceil(n / 64)] uint32, the tiles touched by each group of 64
 *   consecutive Gaussians. Their total is the instance count m (= offsets[n] of
 *   gs_bin_prepare_3d): the caller can copy these few bytes to host memory right after the
 *   preprocess, while the depth sort runs, instead of reading offsets[n] after it (Faster-GS
 *   reads the count back after its tiles_touched scan, phase2/fastergs_readback.patch:46-85).
 * ------------------------------------------------------------------------------------- */
int gs_preprocess_fwd(const float* means, const float* log_scales, const float* quats,
                      const float* opacity_logits, const float* sh, const float* sh_rest, int64_t n,
                      int sh_coeffs, int sh_degree, const gs_camera* cam, float* splat_rec,
                      uint32_t* tiles_touched, uint32_t* depth_keys, uint32_t* wave_counts,
                      void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D binning (replaces the cub DeviceScan of tiles_touched, create_instances_cu, the two cub
 * Onesweep sorts, extract_instance_ranges_cu and extract_bucket_counts; the call sequence is
 * visible in results/phase1/garden_main_4475452_5k_cuda_gpu_kern_sum.csv:10-31).
 * Produces the stable order of instances by (tile, depth, Gaussian index) -- the order of a
 * stable sort of 64-bit keys (tile << 32 | orderable depth bits) over instances emitted in
 * Gaussian-index order, by one of two paths (gs_bin_path):
 *   GS_BIN_PATH_RADIX (default below GS_BIN_SPAN_MIN_GAUSSIANS): a stable radix sort of the
 *     Gaussians by depth, then the instances emitted in that order and stably radix-sorted by tile;
 *   GS_BIN_PATH_SPANS: the depth sort, then two counting passes over the Gaussians' row spans
 *     (the run of tiles a Gaussian touches in one tile row): by tile row over the Gaussians in
 *     depth order, then by column within each row, which writes every instance once.
 * The caller runs gs_bin_prepare_3d (the order and, except on the span path, the instance
 * offsets), then gs_bin_fill_3d.
 *
 * gs_bin_prepare_3d: depth ordering (radix and span paths).
 *   depth_keys [n] from gs_preprocess_fwd with the same camera (order keys of the view depth
 *   relative to the near plane's, culled Gaussians after every visible one, so the sort reads
 *   only as many bits as the near/far range needs), or NULL (then computed from splat_rec and
 *   tiles_touched).
 *   out: order [n]        Gaussian indices by depth key, stable (culled Gaussians last)
 *        offsets [n + 1]  (may be NULL: gs_bin_fill_3d needs them in depth order only on the
 *                         radix path) exclusive scan of tiles_touched[order[j]]; offsets[n] = m,
 *                         the number of instances
 *   tiles_touched may be NULL when offsets is NULL and depth_keys is given.
 *   Workspace from gs_bin_prepare_workspace_size(n).
 * gs_bin_fill_3d: tile lists, ranges, bucket offsets. splat_rec as gs_preprocess_fwd wrote it
 *   (a culled Gaussian's record holds the empty bounds (0, -1, 0, -1)); m = the sum of the
 *   preprocess's wave_counts. Writes
 *   point_list [m]        Gaussian index per instance, tile-major, front to back
 *   sorted_keys [m]       the 64-bit keys in that order (may be NULL: not needed downstream;
 *                         needs depth_keys)
 *   ranges [T,2]          [start, end) of each tile in point_list
 *   bucket_offsets [T+1]  exclusive scan of ceil(len/32); bucket_offsets[T] = number of buckets
 *   bucket_list (may be NULL): the list gs_blend_fwd_3d appends to; its header is cleared
 *                         here, so that call can take GS_BLEND_LIST_CLEARED
 *   order, offsets: as gs_bin_prepare_3d wrote them for the same path (offsets NULL on the span
 *   path).
 *   Workspace from gs_bin_fill_3d_workspace_size(n, m, cam): this fill's own path only (the
 *   larger gs_bin_workspace_size(n, m, tiles_x, tiles_y, cam->flags) also covers it). The
 *   workspace holds nothing the blends read: it can be released once the fill has run.
 * ------------------------------------------------------------------------------------- */
#define GS_BIN_SPAN_MAX_TILES 512
size_t gs_bin_prepare_workspace_size(int64_t n);
int gs_bin_prepare_3d(const float* splat_rec, const uint32_t* tiles_touched, const uint32_t* depth_keys,
                      int64_t n, const gs_camera* cam, uint32_t* order, uint32_t* offsets,
                      void* workspace, size_t workspace_bytes, void* stream);
size_t gs_bin_workspace_size(int64_t n, int64_t m, int tiles_x, int tiles_y, int flags);
size_t gs_bin_fill_3d_workspace_size(int64_t n, int64_t m, const gs_camera* cam);
int gs_bin_path(int64_t n, const gs_camera* cam); /* GS_BIN_PATH_* the fill takes for n Gaussians */
int gs_bin_fill_3d(const float* splat_rec, const uint32_t* depth_keys, const uint32_t* order,
                   const uint32_t* offsets, int64_t n, const gs_camera* cam, int64_t m,
                   uint64_t* sorted_keys, uint32_t* point_list, uint32_t* ranges,
                   uint32_t* bucket_offsets, uint32_t* bucket_list, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Rectangle binning for the 2D operators (replaces toy2d/gs2d/binning.py:34-88, whose
 * per-tile lists are ordered by a stable depth rank, and phase0/splat2d/ops.py:206-255, whose
 * lists are in index order). rects [n,4] int32 = (tx0, ty0, tx1, ty1) tile rectangle, max
 * exclusive, 16-byte aligned (clipped to the grid); depth [n] of depth_dtype (NULL = index
 * order); counts from gs2d_rects_toy / gs2d_rects_phase0 / gs_rect_counts. Outputs as
 * gs_bin_fill_3d, plus (each may be NULL) tile_offsets [T+1] (CSR form of ranges) and
 * order [n] = the stable argsort of depth (toy2d Bins.order). sorted_keys needs a float32
 * depth. Ranges of empty tiles are empty ranges at their CSR position. flags: GS_BIN_* bits.
 * Workspace from gs_bin_workspace_size(n, m, tiles_x, tiles_y, flags). */
int gs_rect_counts(const int32_t* rects, int64_t n, int tiles_x, int tiles_y, uint32_t* counts,
                   void* stream);
int gs_bin_fill_rect(const int32_t* rects, const void* depth, int depth_dtype, const uint32_t* counts,
                     int64_t n, int tiles_x, int tiles_y, int64_t m, uint64_t* sorted_keys,
                     uint32_t* point_list, uint32_t* ranges, uint32_t* tile_offsets,
                     uint32_t* bucket_offsets, uint32_t* order, int flags, void* workspace,
                     size_t workspace_bytes, void* stream);

/* bucket_to_tile[b] = tile of bucket b, for b < bucket_offsets[n_tiles] (read on device);
 * entries up to n_buckets_max are written, unused ones with 0xffffffff. */
int gs_bucket_fill(const uint32_t* bucket_offsets, int n_tiles, uint32_t* bucket_to_tile,
                   int64_t n_buckets_max, void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D forward blend (replaces Faster-GS blend_cu, csv:5). One 16x16 tile per workgroup.
 *   image [3,H,W] = C + T_final * bg; final_T [H,W]; n_contrib [H,W] = 1 + list position of
 *   the last splat blended into the pixel (0 if none); tile_max [T] = max n_contrib of the
 *   tile; ckpt [n_buckets, 256, 4] = (C.r, C.g, C.b, T) at the start of every 32-entry
 *   bucket. bg is host memory (3 floats) or NULL for black. splat_rec, point_list and ckpt
 *   may be NULL when there are no instances (every tile range empty). alpha [H,W] (may be
 *   NULL) = 1 - final_T, the rasterizer's alpha output.
 *   bucket_list (NULL, or 16-byte aligned uint32 [4 + n_buckets_max] with the bound of
 *   gs_bucket_fill; needs ckpt): receives the buckets the backward reads (those starting before
 *   their tile's tile_max) for gs_blend_bwd_3d: [0] their number, [4 ...] their indices in any
 *   order. Its header is cleared by this call, unless flags has GS_BLEND_LIST_CLEARED (the
 *   caller passed the list to gs_bin_fill_3d, which cleared it).
 *   bucket_to_tile (may be NULL; needs bucket_offsets): receives the tile of every bucket
 *   b < bucket_offsets[T], as gs_bucket_fill would write it.
 *   clear (may be NULL): 16-byte aligned float buffer of clear_floats (a multiple of 4) that
 *   the call sets to zero while it blends -- the grad2d that gs_blend_bwd_3d with
 *   GS_ACCUMULATE adds to.
 *   Inference (Faster-GS's inference blend, upstream/upstream_main_kernels.patch:131-150):
 *   ckpt NULL, and then bucket_offsets, n_contrib, tile_max and bucket_list may be NULL too;
 *   image and final_T are the same bits as with them.
 * ------------------------------------------------------------------------------------- */
int gs_blend_fwd_3d(const float* splat_rec, const uint32_t* ranges, const uint32_t* point_list,
                    const uint32_t* bucket_offsets, int width, int height, const float* bg,
                    float* image, float* final_T, float* alpha, int32_t* n_contrib, uint32_t* tile_max,
                    float* ckpt, uint32_t* bucket_list, uint32_t* bucket_to_tile, float* clear,
                    int64_t clear_floats, int flags, void* stream);
enum { GS_BLEND_LIST_CLEARED = 1 };

/* ---------------------------------------------------------------------------------------
 * Pruning scores (replaces Faster-GS's pruning-score blend, kernels_pruning_scores.cuh, seen
 * at upstream/upstream_main_kernels.patch:152-198): for every splat g,
 *   scores[g] += sum over the pixels it is blended into of its blending weight alpha * T,
 * with the forward's rules decision for decision (same list walk, skip and stop). Accumulates
 * (zero scores before the first view). n = length of scores.
 * ------------------------------------------------------------------------------------- */
int gs_blend_scores_3d(const float* splat_rec, const uint32_t* ranges, const uint32_t* point_list,
                       int width, int height, int64_t n, float* scores, void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D bucketed blend backward (replaces blend_backward_cu / blend_backward_macro_cu,
 * phase1/fastergs_macro.patch:40-314). One wavefront per bucket; grad2d [n,12] receives
 * dL/d(mean2d, conic A B C), opacity x dL/dopacity (sum over pixels of alpha dL/dalpha; the
 * preprocess backward divides by the opacity), dL/dcolour and, with GS_ABS_GRAD in flags, |dL/dmean2d|
 * (slots 9-10; Faster-GS's compute_abs_grad instantiation, phase1/fastergs_macro.patch:206-209).
 * It is zeroed by the call unless flags has GS_ACCUMULATE (then the call adds to it, e.g. over
 * views).
 * n_buckets is read on device from bucket_offsets[T]; n_buckets_max bounds the grid.
 * grad_alpha [H,W] (may be NULL) is the gradient of the alpha = 1 - final_T output.
 * bucket_list: the forward's (or NULL): only the listed buckets are processed (the others
 * have no blended entry); NULL: every bucket of the table is examined.
 * counters: NULL or 3 device uint64 that receive the atomic adds issued (9 per reduced
 * bucket-splat, 11 with GS_ABS_GRAD) and, in [2], the (pixel, splat) pairs evaluated.
 * grad_conic64 (may be NULL; 8-byte aligned [n, 4] double, zeroed or accumulated like grad2d):
 * the conic-gradient sums of the elongated splats in float64. A splat whose 2D covariance has a
 * condition number of at least 256 (from its record's conic) has its three conic sums reduced and
 * added over the buckets in float64 into grad_conic64[g, 0..2] instead of grad2d[g, 2..4], and
 * grad2d[g, 11] set to 1: gs_preprocess_bwd, whose conic -> covariance step divides by det^2,
 * then takes them unrounded. With NULL every splat takes the float32 sums of grad2d.
 * ------------------------------------------------------------------------------------- */
enum { GS_ACCUMULATE = 1, GS_ABS_GRAD = 2 };
int gs_blend_bwd_3d(const float* splat_rec, const uint32_t* ranges, const uint32_t* point_list,
                    const uint32_t* bucket_offsets, const uint32_t* bucket_to_tile,
                    int64_t n_buckets_max, int64_t n, int width, int height, const float* image,
                    const float* grad_image, const float* final_T, const float* grad_alpha,
                    const int32_t* n_contrib, const uint32_t* tile_max, const float* ckpt,
                    uint32_t* bucket_list, float* grad2d, double* grad_conic64, int flags,
                    unsigned long long* counters, void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D preprocess backward (replaces Faster-GS preprocess_backward_cu, csv:4): chains grad2d
 * into the parameters. Every output row is written (zeros for culled Gaussians).
 *   grad_means, grad_log_scales [n,3]; grad_quats [n,4]; grad_opacity_logits [n];
 *   grad_sh [n, sh_coeffs, 3] (coefficients above the active degree get 0); with the split
 *   layout (sh_rest not NULL) grad_sh [n, 1, 3] and grad_sh_rest [n, sh_coeffs - 1, 3].
 *   The colour clamp of the forward is recomputed from the SH rows it reads anyway (the same
 *   operations, so the same bits), so the splat records are not needed.
 *   grad_conic64 (may be NULL): gs_blend_bwd_3d's float64 conic sums; for a row with grad2d[g, 11]
 *   set, the conic gradient is grad2d[g, 2..4] + grad_conic64[g, 0..2] (in float64).
 * ------------------------------------------------------------------------------------- */
int gs_preprocess_bwd(const float* means, const float* log_scales, const float* quats,
                      const float* opacity_logits, const float* sh, const float* sh_rest, int64_t n,
                      int sh_coeffs, int sh_degree, const gs_camera* cam,
                      const uint32_t* tiles_touched, const float* grad2d, const double* grad_conic64,
                      float* grad_means,
                      float* grad_log_scales, float* grad_quats, float* grad_opacity_logits,
                      float* grad_sh, float* grad_sh_rest, void* stream);

/* Densification statistics of one backward, accumulated into info [rows, n] (rows 2 or 3) for
 * the visible Gaussians (tiles_touched > 0): info[0] += 1; info[1] += |(W/2 g_x, H/2 g_y)|, the
 * norm of the mean2d gradient in NDC units (grad2d[:, 0:2]); info[2] (rows == 3) += the same
 * norm of the summed per-pixel |dL/dmean2d| (grad2d[:, 9:11]). The densification_info rows of
 * Faster-GS's backward (phase1/tests/test_parity.py:93-106, fastergs_macro.patch:59,206-209);
 * the NDC scaling is the one of the original 3DGS rasterizer's mean2D gradient. */
int gs_densification_stats(const float* grad2d, const uint32_t* tiles_touched, int64_t n, int width,
                           int height, int rows, float* info, void* stream);

/* =======================================================================================
 * 2D surfaces (rules GS_RULES_TOY2D / GS_RULES_PHASE0; dtype GS_FLOAT32 / GS_FLOAT64)
 * ===================================================================================== */

/* The toy2d activation in one launch (the caller-side toy2d/gs2d/params.py:36-56, activate and
 * radii_from_cov, for fit loops that would otherwise run a dozen small tensor operations and their
 * backwards per step; no kernel of the reference): log_scale [n,2], theta [n], rgb_logit [n,3],
 * opacity_logit [n] -> conic [n,3] = (cyy, -cxy, cxx) / det of cov = R diag(exp(2 log_scale))
 * R^T, color [n,3] and opacity [n] (sigmoids), cov [n,3] = (cxx, cxy, cyy) and radii [n] (the
 * integer 3-sigma radius, 0 where det <= 0; cov and radii may be NULL). The reference's operation
 * order, float32; exp, cos and sin from the device math library. gs2d_activate_bwd: the
 * gradients of log_scale, theta, rgb_logit and opacity_logit from those of conic, color and
 * opacity (each may be NULL: zero); the means pass through. */
int gs2d_activate_fwd(const float* log_scale, const float* theta, const float* rgb_logit,
                      const float* opacity_logit, int64_t n, float* conic, float* color, float* opacity,
                      float* cov, int32_t* radii, void* stream);
int gs2d_activate_bwd(const float* log_scale, const float* theta, const float* rgb_logit,
                      const float* opacity_logit, int64_t n, const float* grad_conic, const float* grad_color,
                      const float* grad_opacity, float* grad_log_scale, float* grad_theta,
                      float* grad_rgb_logit, float* grad_opacity_logit, void* stream);

/* toy2d tile rectangles from the 3-sigma radius (replaces the getRect part of
 * toy2d/gs2d/binning.py:44-57): means [n,2] float32 (8-byte aligned), radii [n] int32 ->
 * rects [n,4] (xmin, ymin, xmax, ymax in tiles, max exclusive, empty = collapsed to
 * (xmin, ymin)), counts [n] = tiles covered. */
int gs2d_rects_toy(const float* means, const int32_t* radii, int64_t n, int width, int height,
                   int32_t* rects, uint32_t* counts, void* stream);

/* phase0 tile rectangles of the alpha >= 1/255 ellipse bounding box with one pixel of slack,
 * evaluated in float64 (replaces phase0/splat2d/ops.py:206-235): means [n,2], chol [n,3],
 * opacity_logit [n] of dtype -> rects [n,4] (tx0, ty0, tx1+1, ty1+1), counts [n]. */
int gs2d_rects_phase0(int dtype, const void* means, const void* chol, const void* opacity_logit,
                      int64_t n, int width, int height, int32_t* rects, uint32_t* counts, void* stream);

/* Splat records rec [n,16] of dtype (16-byte aligned) from the 2D parameters: toy2d
 * (means [n,2], conic [n,3], color [n,3], opacity [n]); phase0 (means [n,2], chol [n,3],
 * colors [n,3], opacity_logit [n]; the record holds sigmoid(logit)). */
int gs2d_pack(int rules, int dtype, const void* means, const void* shape, const void* color,
              const void* opacity, int64_t n, void* rec, void* stream);

/* Splits a 2D gradient record grad_rec [n,12] of dtype into dmeans [n,2], dshape [n,3],
 * dopacity [n] and dcolor [n,3] (slots 0-1, 2-4, 5, 6-8), the four tensors the reference's
 * backward functions return (toy2d/csrc/rasterize.cu:405-406, phase0/csrc/macrotile/
 * bindings.cpp:111-114), in one launch. */
int gs2d_unpack_grads(int dtype, const void* grad_rec, int64_t n, void* dmeans, void* dshape, void* dopacity,
                      void* dcolor, void* stream);

/* 2D forward blend (replaces toy2d rasterize_forward, toy2d/csrc/rasterize.cu:366-394, and
 * phase0 forward, phase0/csrc/macrotile/bindings.cpp:156-178). Tile t's list is
 * point_list[ranges[t*range_stride] .. ranges[t*range_stride+1]) (range_stride 2 for (T,2)
 * ranges, 1 for (T+1) CSR offsets). Outputs: image ([3,H,W] toy2d, [H,W,3] phase0) of dtype,
 * final_T [H,W], n_contrib [H,W] (toy2d: last list position + 1; phase0: number of splats),
 * last_contrib [H,W] (phase0, may be NULL), tile_max [T] (may be NULL), ckpt [B,256,4]
 * (toy2d (T, C); phase0 (C, T); NULL = not saved; bucket_offsets [T], each tile's first bucket,
 * needed with it). Every output is written whole: ckpt slots of buckets after a tile stopped hold
 * zeros (toy2d) or the tile's final state (phase0).
 * bg: 3 host doubles (toy2d) or NULL. counters: NULL or 3 device uint64 (atomic adds,
 * checkpoint bytes, splat-pixel evaluations) that the kernels add to
 * (phase0/csrc/macrotile/splat2d_common.h:260-266). */
int gs2d_blend_fwd(int rules, int dtype, const void* rec, const uint32_t* ranges, int range_stride,
                   const uint32_t* point_list, const uint32_t* bucket_offsets, int width, int height,
                   const double* bg, void* image, void* final_T, int32_t* n_contrib,
                   int32_t* last_contrib, uint32_t* tile_max, void* ckpt,
                   unsigned long long* counters, void* stream);

/* 2D bucketed backward (replaces toy2d rasterize_backward_splat, toy2d/csrc/rasterize.cu:
 * 419-448, and phase0 backward_splat, phase0/csrc/macrotile/bindings.cpp:201-220). One
 * wavefront per 32-entry bucket; limit [H,W] = list position + 1 of each pixel's last splat
 * (toy2d n_contrib, phase0 last_contrib); tile_max may be NULL. grad_rec [n,12] of dtype is
 * zeroed by the call and receives dL/d(mean 2, shape 3, opacity, colour 3) in slots 0..8
 * (phase0: the opacity slot holds dL/dlogit). */
int gs2d_blend_bwd_bucket(int rules, int dtype, const void* rec, const uint32_t* ranges,
                          int range_stride, const uint32_t* point_list,
                          const uint32_t* bucket_offsets, const uint32_t* bucket_to_tile,
                          int64_t n_buckets, int64_t n, int width, int height, const void* image,
                          const void* grad_image, const int32_t* limit, const uint32_t* tile_max,
                          const void* ckpt, void* grad_rec, unsigned long long* counters,
                          void* stream);

/* 2D per-pixel backward (replaces toy2d rasterize_backward_pixel, toy2d/csrc/rasterize.cu:
 * 396-417, and phase0 backward_pixel, phase0/csrc/macrotile/bindings.cpp:180-199): back to
 * front, T recovered by division. phase0 rules: one atomic per parameter per (pixel, splat) pair
 * (backward A, counted in counters[0]); toy2d rules: a wavefront's pixels' gradients of a splat
 * summed first, then one atomic per parameter. */
int gs2d_blend_bwd_pixel(int rules, int dtype, const void* rec, const uint32_t* ranges,
                         int range_stride, const uint32_t* point_list, int64_t n, int width,
                         int height, const double* bg, const void* final_T, const int32_t* limit,
                         const void* grad_image, void* grad_rec, unsigned long long* counters,
                         void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused Adam over several parameter groups in one launch (replaces Faster-GS adam_step and
 * adam_step_sparse, cluster/patches/fastergs_lean_adam.patch:80-186, called per group by
 * FusedAdam.step, :65-81). Per element, with g the gradient and m, v the moments:
 *   m' = fma(beta1, m - g, g);  v' = fma(beta2, v - g*g, g*g)
 *   p' = p - (step_size * m') / (sqrt(v') * bc2 + eps)
 * with step_size = lr / (1 - beta1^step) and bc2 = 1 / sqrt(1 - beta2^step), both computed in
 * double and rounded to float. visibility [n_primitives] int32 (may be NULL = dense): rows of a
 * primitive with visibility 0 are not touched (parameters and moments). Moments are float32, or
 * bfloat16 (moment_dtype GS_BFLOAT16) written with stochastic rounding: the 16 dropped bits get
 * uniform noise from an integer hash of (element index ^ seed), seed = 0x9E3779B9 * step +
 * 0x85EBCA6B (uint32). Each group is [n_primitives, ...] contiguous; at most GS_ADAM_MAX_GROUPS.
 * ------------------------------------------------------------------------------------- */
#define GS_ADAM_MAX_GROUPS 8
typedef struct gs_adam_group {
  const float* grad;
  float* param;
  void* exp_avg;      /* float32 or bfloat16 (uint16 bits), n_elements each */
  void* exp_avg_sq;
  int64_t n_elements; /* n_primitives * features per primitive */
  int32_t moment_dtype; /* GS_FLOAT32 or GS_BFLOAT16 */
  int32_t step;       /* the group's step count after this update (>= 1) */
  double lr, beta1, beta2, eps;
} gs_adam_group;
int gs_adam_step(const gs_adam_group* groups, int n_groups, int64_t n_primitives,
                 const int32_t* visibility, void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused L1 + D-SSIM loss on [C, H, W] float32 images (replaces the fused-ssim extension's
 * fusedssimCUDA / fusedssim_backwardCUDA, results/phase1/README.md:46-47, with the trainers'
 * L1 term; LAMBDA_DSSIM of phase2/logs/run_4559238/runs/b_room_up_s10/training_config.yaml:100):
 *   L = (1 - lambda) mean|x - y| + lambda (1 - mean SSIM(x, y)),
 * SSIM with an 11x11 Gaussian window (sigma 1.5), C1 = 0.01^2, C2 = 0.03^2, zero padding.
 * gs_l1_ssim_fwd writes loss[3] = (L, mean|x - y|, mean SSIM) on the device and, if dmap is not
 * NULL, dmap [C, 3, H, W] = (dS/dmu_x, dS/dE[x^2], dS/dE[xy]) per pixel for the backward.
 * Workspace from gs_l1_ssim_workspace_size. gs_l1_ssim_bwd writes grad_image [C, H, W] =
 * dL/dx, scaled by grad_loss[0] (a device float; NULL = 1).
 * ------------------------------------------------------------------------------------- */
size_t gs_l1_ssim_workspace_size(int channels, int height, int width);
int gs_l1_ssim_fwd(const float* image, const float* target, int channels, int height, int width,
                   float lambda_dssim, float* dmap, float* loss, void* workspace, size_t workspace_bytes,
                   void* stream);
int gs_l1_ssim_bwd(const float* image, const float* target, const float* dmap, int channels, int height,
                   int width, float lambda_dssim, const float* grad_loss, float* grad_image, void* stream);

/* ---------------------------------------------------------------------------------------
 * Measurement probes: the achievable ceilings of the GPU the library runs on, against which
 * bench.py quotes its roofline fractions besides the published peaks (the reference measured
 * its copy and read-only bandwidth the same way, results/phase1/README.md:10-16).
 *   gs_probe_copy   out[i] = in[i] for n floats (n a multiple of 4, 16-byte aligned): 8n bytes
 *   gs_probe_read   reads n floats (n a multiple of 4, 16-byte aligned) once and writes
 *                   gs_probe_read_sums(n) partial sums (one per wavefront; that many floats
 *                   in `sums`)
 *   gs_probe_fma    `threads` threads (a multiple of 256) each run 64 * iters dependent-free
 *                   FP32 FMAs (16 chains) and write one float to out[threads]
 * ------------------------------------------------------------------------------------- */
int gs_probe_copy(const float* in, float* out, int64_t n, void* stream);
int64_t gs_probe_read_sums(int64_t n);
int gs_probe_read(const float* in, int64_t n, float* sums, void* stream);
int gs_probe_fma(float* out, int64_t threads, int iters, void* stream);

/* ---------------------------------------------------------------------------------------
 * Stage marks (measurement only; bench.py's per-stage split of the binning chain). After
 * gs_stage_marks(1), the calls made on this thread record a HIP event on their stream at each
 * internal stage boundary (the event is named after the stage that ends there; the first mark of
 * a call is its start). gs_stage_marks_read waits for the last mark and writes, for up to `max`
 * marks in order, names[i] and ms[i] = the time from mark i - 1 to mark i (ms[0] = 0); it returns
 * the number written, or -GS_ERR_* on failure. gs_stage_marks(0) stops recording (and both calls forget earlier marks).
 * The events are created on first use and kept; with marks off (the default) nothing is recorded.
 * ------------------------------------------------------------------------------------- */
int gs_stage_marks(int enable);
int gs_stage_marks_read(float* ms, const char** names, int max);

/* ---------------------------------------------------------------------------------------
 * Allocation-free gs_l1_ssim_fwd. It has no counterpart in the reference. It is for callers
 * that cannot allocate device memory: code under HIP graph capture, tight serving loops, and
 * harnesses that forbid hipMalloc.
 * Same arguments and results as gs_l1_ssim_fwd (the same kernels, so the same bits), without
 * the workspace: the per-tile partial sums go to a static device buffer of the library of
 * 2 * GS_L1_SSIM_NOALLOC_MAX_TILES floats (1 MiB), one per GPU, held until the process ends.
 * channels * ceil(height/16) * ceil(width/16) must not exceed GS_L1_SSIM_NOALLOC_MAX_TILES
 * (e.g. 3 x 2048 x 2048 fits); larger images return GS_ERR_ARG. The call allocates nothing.
 * Every call on one GPU shares that GPU's buffer and leaves its partial sums there (nothing
 * in it has to start at zero): calls that can overlap on one GPU (on streams not ordered
 * with each other) race, so order them.
 * ------------------------------------------------------------------------------------- */
#define GS_L1_SSIM_NOALLOC_MAX_TILES 131072
int gs_l1_ssim_fwd_noalloc(const float* image, const float* target, int channels, int height, int width,
                           float lambda_dssim, float* dmap, float* loss, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMDSPLAT_H */
