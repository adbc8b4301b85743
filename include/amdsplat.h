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
 *   gs_preprocess_fwd -> gs_scan_u32 (tiles touched) -> [host reads M] -> gs_bin_fill_3d
 *   -> gs_bucket_fill -> gs_blend_fwd_3d;   backward: gs_blend_bwd_3d -> gs_preprocess_bwd.
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

/* Pinhole camera. viewmat is the row-major 4x4 world-to-camera matrix with OpenCV axes
 * (x right, y down, z forward); pixel (i, j) covers [i, i+1) x [j, j+1), so its centre is
 * at (i + 0.5, j + 0.5). */
typedef struct gs_camera {
  float viewmat[16];
  float fx, fy, cx, cy;
  int32_t width, height;
  float near_plane, far_plane; /* near_plane must be > 0 */
} gs_camera;

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

/* ---------------------------------------------------------------------------------------
 * 3D preprocess forward (replaces Faster-GS preprocess_cu; signature evidence
 * results/phase1/garden_main_4475452_5k_cuda_gpu_kern_sum.csv:7). Per Gaussian: view
 * transform, near/far culling, opacity = sigmoid(logit), covariance from exp(log_scales)
 * and the normalised quaternion (w, x, y, z), EWA projection with a 0.3 px^2 dilation,
 * conic, SH colour of degree sh_degree (+0.5, clamped at 0), the alpha >= 1/255 ellipse
 * bounds, and the number of 16x16 tiles the ellipse reaches (0 = culled).
 *   means, log_scales [n,3]; quats [n,4]; opacity_logits [n]; sh [n, sh_coeffs, 3] with
 *   sh_coeffs in {1,4,9,16} and (sh_degree+1)^2 <= sh_coeffs.
 *   out: splat_rec [n,16] floats (16-byte aligned), tiles_touched [n] uint32.
 * ------------------------------------------------------------------------------------- */
int gs_preprocess_fwd(const float* means, const float* log_scales, const float* quats,
                      const float* opacity_logits, const float* sh, int64_t n, int sh_coeffs,
                      int sh_degree, const gs_camera* cam, float* splat_rec,
                      uint32_t* tiles_touched, void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D binning (replaces create_instances_cu, the two cub Onesweep sorts,
 * extract_instance_ranges_cu and extract_bucket_counts; the call sequence is visible in
 * results/phase1/garden_main_4475452_5k_cuda_gpu_kern_sum.csv:10-31).
 * m = sum of tiles_touched (the caller reads it, e.g. from gs_scan_u32's out[n]).
 * Produces the stable order of instances by (tile, depth, Gaussian index) -- the order of a
 * stable sort of 64-bit keys (tile << 32 | orderable depth bits) over instances emitted in
 * Gaussian-index order -- with two stable LSD radix sorts: the Gaussians by depth, then the
 * instances (emitted in depth order) by tile. Writes
 *   point_list [m]        Gaussian index per instance, tile-major, front to back
 *   sorted_keys [m]       the 64-bit keys in that order (may be NULL: not needed downstream)
 *   ranges [T,2]          [start, end) of each tile in point_list
 *   bucket_offsets [T+1]  exclusive scan of ceil(len/32); bucket_offsets[T] = number of buckets
 * Workspace from gs_bin_workspace_size(n, m, T).
 * ------------------------------------------------------------------------------------- */
size_t gs_bin_workspace_size(int64_t n, int64_t m, int n_tiles);
int gs_bin_fill_3d(const float* splat_rec, const uint32_t* tiles_touched, int64_t n,
                   const gs_camera* cam, int64_t m, uint64_t* sorted_keys, uint32_t* point_list,
                   uint32_t* ranges, uint32_t* bucket_offsets, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Rectangle binning for the 2D operators (replaces toy2d/gs2d/binning.py:34-88, whose
 * per-tile lists are ordered by a stable depth rank, and phase0/splat2d/ops.py:206-255, whose
 * lists are in index order). rects [n,4] int32 = (tx0, ty0, tx1, ty1) tile rectangle, max
 * exclusive, 16-byte aligned; depth [n] (NULL = index order). counts from gs_rect_counts.
 * Outputs as gs_bin_fill_3d; the depth key is the orderable image of the float depth. */
int gs_rect_counts(const int32_t* rects, int64_t n, int tiles_x, int tiles_y, uint32_t* counts,
                   void* stream);
int gs_bin_fill_rect(const int32_t* rects, const float* depth, const uint32_t* counts, int64_t n,
                     int tiles_x, int tiles_y, int64_t m, uint64_t* sorted_keys,
                     uint32_t* point_list, uint32_t* ranges, uint32_t* bucket_offsets,
                     void* workspace, size_t workspace_bytes, void* stream);

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
 *   may be NULL when there are no instances (every tile range empty).
 * ------------------------------------------------------------------------------------- */
int gs_blend_fwd_3d(const float* splat_rec, const uint32_t* ranges, const uint32_t* point_list,
                    const uint32_t* bucket_offsets, int width, int height, const float* bg,
                    float* image, float* final_T, int32_t* n_contrib, uint32_t* tile_max,
                    float* ckpt, void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D bucketed blend backward (replaces blend_backward_cu / blend_backward_macro_cu,
 * phase1/fastergs_macro.patch:40-314). One wavefront per bucket; grad2d [n,12] is zeroed
 * by the call and receives dL/d(mean2d, conic A B C, opacity, colour) and |dL/dmean2d|.
 * n_buckets is read on device from bucket_offsets[T]; n_buckets_max bounds the grid.
 * grad_alpha [H,W] (may be NULL) is the gradient of the alpha = 1 - final_T output.
 * ------------------------------------------------------------------------------------- */
int gs_blend_bwd_3d(const float* splat_rec, const uint32_t* ranges, const uint32_t* point_list,
                    const uint32_t* bucket_offsets, const uint32_t* bucket_to_tile,
                    int64_t n_buckets_max, int64_t n, int width, int height, const float* image,
                    const float* grad_image, const float* final_T, const float* grad_alpha,
                    const int32_t* n_contrib, const uint32_t* tile_max, const float* ckpt,
                    float* grad2d, void* stream);

/* ---------------------------------------------------------------------------------------
 * 3D preprocess backward (replaces Faster-GS preprocess_backward_cu, csv:4): chains grad2d
 * into the parameters. Every output row is written (zeros for culled Gaussians).
 *   grad_means, grad_log_scales [n,3]; grad_quats [n,4]; grad_opacity_logits [n];
 *   grad_sh [n, sh_coeffs, 3] (coefficients above the active degree get 0).
 * ------------------------------------------------------------------------------------- */
int gs_preprocess_bwd(const float* means, const float* log_scales, const float* quats,
                      const float* opacity_logits, const float* sh, int64_t n, int sh_coeffs,
                      int sh_degree, const gs_camera* cam, const float* splat_rec,
                      const uint32_t* tiles_touched, const float* grad2d, float* grad_means,
                      float* grad_log_scales, float* grad_quats, float* grad_opacity_logits,
                      float* grad_sh, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMDSPLAT_H */
