// C entry points over the reference's own phase0 CPU twin (phase0/csrc/macrotile/
// splat2d_cpu.cpp + splat2d_common.h, compiled from where they lie in the reference tree by
// oracle/ref.mk into oracle/_ref/). TEST INFRASTRUCTURE ONLY: the tests use it to pin the
// phase0 restatement in oracle2d.c; the product never loads it.
#include <stdint.h>

#include "splat2d_common.h"

namespace {

template <typename S>
splat2d::SceneView<S> view(const S* means, const S* chol, const S* logit, const S* colors, const int32_t* tile_off,
                           const int32_t* tile_ids, const int32_t* bucket_off, const int32_t* bucket_tile,
                           int num_tiles, int num_buckets, int height, int width) {
  splat2d::SceneView<S> v;
  v.means = means;
  v.chol = chol;
  v.opacity_logit = logit;
  v.colors = colors;
  v.tile_off = tile_off;
  v.tile_ids = tile_ids;
  v.bucket_off = bucket_off;
  v.bucket_tile = bucket_tile;
  v.height = height;
  v.width = width;
  v.tiles_x = (width + splat2d::kTile - 1) / splat2d::kTile;
  v.num_tiles = num_tiles;
  v.num_buckets = num_buckets;
  return v;
}

}  // namespace

#define REF_ENTRY(S, SFX)                                                                                        \
  extern "C" void ref2d_forward_##SFX(const S* means, const S* chol, const S* logit, const S* colors,           \
                                      const int32_t* tile_off, const int32_t* tile_ids, const int32_t* boff,    \
                                      const int32_t* btile, int num_tiles, int num_buckets, int height,         \
                                      int width, S* image, S* t_final, int32_t* n_contrib,                      \
                                      int32_t* last_contrib, S* ckpt) {                                         \
    const auto v = view<S>(means, chol, logit, colors, tile_off, tile_ids, boff, btile, num_tiles, num_buckets, \
                           height, width);                                                                      \
    splat2d::FwdOut<S> out{image, t_final, n_contrib, last_contrib, ckpt};                                     \
    splat2d::forward_cpu<S>(v, out);                                                                            \
  }                                                                                                             \
  extern "C" void ref2d_backward_##SFX(int splat_mode, const S* means, const S* chol, const S* logit,           \
                                       const S* colors, const int32_t* tile_off, const int32_t* tile_ids,       \
                                       const int32_t* boff, const int32_t* btile, int num_tiles,                \
                                       int num_buckets, int height, int width, const S* grad_image,            \
                                       const S* image, const S* t_final, const int32_t* last_contrib,          \
                                       const S* ckpt, S* g_means, S* g_chol, S* g_logit, S* g_colors) {        \
    const auto v = view<S>(means, chol, logit, colors, tile_off, tile_ids, boff, btile, num_tiles, num_buckets, \
                           height, width);                                                                      \
    splat2d::Grads<S> g{g_means, g_chol, g_logit, g_colors};                                                    \
    if (splat_mode) splat2d::backward_splat_cpu<S>(v, grad_image, image, ckpt, g);                              \
    else splat2d::backward_pixel_cpu<S>(v, grad_image, t_final, last_contrib, g);                               \
  }

REF_ENTRY(float, f32)
REF_ENTRY(double, f64)

extern "C" void ref2d_counters(int64_t* out) {
  out[0] = splat2d::counters().atomic_adds;
  out[1] = splat2d::counters().checkpoint_bytes;
  out[2] = splat2d::counters().splat_pixel_evals;
}

extern "C" void ref2d_reset_counters(void) { splat2d::counters() = splat2d::Counters{}; }
