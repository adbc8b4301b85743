/*
 * Body of the 2D oracle, included twice by oracle2d.c: once with S = float (suffix _f32) and
 * once with S = double (suffix _f64). Forward decisions (alpha >= 1/255, the 0.99 clamp,
 * termination) are evaluated in S with the operation order of the GPU kernels, so integer
 * outputs match bit for bit; gradients are accumulated in double from the replayed S state.
 *
 * Rules: toy2d/csrc/rasterize.cu:37-101,106-177,182-350 and toy2d/gs2d/reference.py:3-8
 * (rules = 1); phase0/csrc/macrotile/splat2d_common.h:7-254 and splat2d_cpu.cpp:31-181
 * (rules = 2).
 */

typedef struct {
  S mx, my, s0, s1, s2, o, cr, cg, cb;
} SFX(Sp);

typedef struct {
  S dx, dy, G, alpha, a, b;
  int clamped;
} SFX(Ev);

static SFX(Sp) SFX(load)(int rules, const S* means, const S* shape, const S* color, const S* opac, int64_t g) {
  SFX(Sp) s;
  s.mx = means[2 * g];
  s.my = means[2 * g + 1];
  s.s0 = shape[3 * g];
  s.s1 = shape[3 * g + 1];
  s.s2 = shape[3 * g + 2];
  s.o = rules == 2 ? SFX(sigmoid)(opac[g]) : opac[g];
  s.cr = color[3 * g];
  s.cg = color[3 * g + 1];
  s.cb = color[3 * g + 2];
  return s;
}

static int SFX(eval)(int rules, const SFX(Sp) * s, S px, S py, SFX(Ev) * e) {
  if (rules == 1) {
    e->dx = s->mx - px;
    e->dy = s->my - py;
    S t1 = (s->s0 * e->dx) * e->dx;
    S t2 = (s->s2 * e->dy) * e->dy;
    S power = (S)(-0.5) * (t1 + t2) - (s->s1 * e->dx) * e->dy;
    if (power > (S)0) return 0;
    e->G = SFX(exp)(power);
    S raw = s->o * e->G;
    e->clamped = raw > (S)0.99;
    e->alpha = e->clamped ? (S)0.99 : raw;
    return e->alpha >= (S)1 / (S)255;
  }
  e->dx = px - s->mx;
  e->dy = py - s->my;
  e->a = s->s0 * e->dx + s->s1 * e->dy;
  e->b = s->s2 * e->dy;
  S q = e->a * e->a + e->b * e->b;
  e->G = SFX(exp)((S)(-0.5) * q);
  S raw = s->o * e->G;
  e->clamped = raw > (S)0.99;
  e->alpha = e->clamped ? (S)0.99 : raw;
  return e->alpha >= (S)(1.0 / 255.0);
}

/* Gradient of one pair w.r.t. (mean 2, shape 3, opacity, -, -, -), in double. */
static void SFX(shape_grads)(int rules, const SFX(Sp) * s, const SFX(Ev) * e, double dLda, double* acc) {
  if (e->clamped) return;
  acc[5] += (double)e->G * dLda;
  double hp = (double)e->alpha * dLda;
  double dx = e->dx, dy = e->dy;
  if (rules == 2) {
    double a = e->a, b = e->b;
    acc[0] += hp * a * s->s0;
    acc[1] += hp * (a * s->s1 + b * s->s2);
    acc[2] -= hp * a * dx;
    acc[3] -= hp * a * dy;
    acc[4] -= hp * b * dy;
  } else {
    acc[2] += -0.5 * hp * dx * dx;
    acc[3] += -hp * dx * dy;
    acc[4] += -0.5 * hp * dy * dy;
    acc[0] += -hp * ((double)s->s0 * dx + (double)s->s1 * dy);
    acc[1] += -hp * ((double)s->s1 * dx + (double)s->s2 * dy);
  }
}

/* Forward. Tile t's list is point_list[ranges[2t] .. ranges[2t+1]); bucket_offsets [T+1]
 * (may be NULL when ckpt is NULL). image: rules 1 [3,H,W] with bg, rules 2 [H,W,3]. Returns
 * the number of splat-pixel evaluations. */
int64_t SFX(or2d_forward)(int rules, const S* means, const S* shape, const S* color, const S* opac,
                          const uint32_t* ranges, const uint32_t* point_list, const uint32_t* bucket_offsets,
                          int W, int H, const double* bg, S* image, S* final_T, int32_t* n_contrib,
                          int32_t* last_contrib, S* ckpt) {
  int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
  int64_t HW = (int64_t)W * H, evals = 0;
  S pix_off = rules == 1 ? (S)0 : (S)0.5;
  S t_stop = (S)1e-4;
  for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t s0 = ranges[2 * tile], len = ranges[2 * tile + 1] - s0;
    for (int t = 0; t < 256; ++t) {
      int px = tx * 16 + (t & 15), py = ty * 16 + (t >> 4);
      int inside = px < W && py < H;
      S pxf = (S)px + pix_off, pyf = (S)py + pix_off;
      S T = (S)1, Cr = (S)0, Cg = (S)0, Cb = (S)0;
      int last = 0, count = 0, done = !inside;
      for (uint32_t idx = 0; idx < len; ++idx) {
        if (ckpt && (idx % 32) == 0) {
          S* c = ckpt + ((int64_t)(bucket_offsets[tile] + idx / 32) * 256 + t) * 4;
          if (rules == 1) {
            c[0] = T; c[1] = Cr; c[2] = Cg; c[3] = Cb;
          } else {
            c[0] = Cr; c[1] = Cg; c[2] = Cb; c[3] = T;
          }
        }
        if (done) continue;
        SFX(Sp) sp = SFX(load)(rules, means, shape, color, opac, point_list[s0 + idx]);
        SFX(Ev) e;
        ++evals;
        if (!SFX(eval)(rules, &sp, pxf, pyf, &e)) continue;
        if (rules == 1) {
          if (T * ((S)1 - e.alpha) < t_stop) {
            done = 1;
            continue;
          }
          S w = e.alpha * T;
          Cr = SFX(fma)(sp.cr, w, Cr);
          Cg = SFX(fma)(sp.cg, w, Cg);
          Cb = SFX(fma)(sp.cb, w, Cb);
        } else {
          Cr = Cr + (sp.cr * e.alpha) * T;
          Cg = Cg + (sp.cg * e.alpha) * T;
          Cb = Cb + (sp.cb * e.alpha) * T;
        }
        T = T * ((S)1 - e.alpha);
        ++count;
        last = (int)idx + 1;
        if (rules == 2 && T < t_stop) done = 1;
      }
      if (!inside) continue;
      int64_t pix = (int64_t)py * W + px;
      if (rules == 1) {
        S b0 = bg ? (S)bg[0] : (S)0, b1 = bg ? (S)bg[1] : (S)0, b2 = bg ? (S)bg[2] : (S)0;
        image[pix] = SFX(fma)(T, b0, Cr);
        image[HW + pix] = SFX(fma)(T, b1, Cg);
        image[2 * HW + pix] = SFX(fma)(T, b2, Cb);
      } else {
        image[3 * pix] = Cr;
        image[3 * pix + 1] = Cg;
        image[3 * pix + 2] = Cb;
      }
      final_T[pix] = T;
      n_contrib[pix] = rules == 2 ? count : last;
      if (last_contrib) last_contrib[pix] = last;
    }
  }
  return evals;
}

/* Bucketed backward replaying (C, T) checkpoints (every bucket of the tables; pixels beyond
 * `limit` are skipped). grad_rec [n,12] (double) is overwritten; slot 5 holds dL/dopacity
 * (rules 1) or dL/dlogit (rules 2). Returns the number of atomics the kernel issues. */
int64_t SFX(or2d_backward_bucket)(int rules, const S* means, const S* shape, const S* color, const S* opac,
                                  int64_t n, const uint32_t* ranges, const uint32_t* point_list,
                                  const uint32_t* bucket_offsets, int W, int H, const S* image,
                                  const S* grad_image, const int32_t* limit, const S* ckpt, double* grad_rec) {
  int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
  int64_t HW = (int64_t)W * H, atomics = 0;
  S pix_off = rules == 1 ? (S)0 : (S)0.5;
  memset(grad_rec, 0, (size_t)n * 12 * sizeof(double));
  for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t s0 = ranges[2 * tile], len = ranges[2 * tile + 1] - s0;
    for (uint32_t b = bucket_offsets[tile]; b < bucket_offsets[tile + 1]; ++b) {
      int bstart = (int)(b - bucket_offsets[tile]) * 32;
      int bsize = (int)len - bstart < 32 ? (int)len - bstart : 32;
      /* per-pixel replay state */
      S T[256];
      double rho[256], G[256][3];
      int lim[256];
      for (int t = 0; t < 256; ++t) {
        int px = tx * 16 + (t & 15), py = ty * 16 + (t >> 4);
        lim[t] = 0;
        if (px >= W || py >= H) continue;
        int64_t pix = (int64_t)py * W + px;
        lim[t] = limit[pix] - bstart;
        if (lim[t] <= 0) continue;
        const S* c = ckpt + ((int64_t)b * 256 + t) * 4;
        S c0, c1, c2;
        if (rules == 1) {
          T[t] = c[0]; c0 = c[1]; c1 = c[2]; c2 = c[3];
        } else {
          c0 = c[0]; c1 = c[1]; c2 = c[2]; T[t] = c[3];
        }
        double im[3];
        for (int ch = 0; ch < 3; ++ch) {
          G[t][ch] = rules == 1 ? grad_image[ch * HW + pix] : grad_image[3 * pix + ch];
          im[ch] = rules == 1 ? image[ch * HW + pix] : image[3 * pix + ch];
        }
        rho[t] = G[t][0] * (im[0] - c0) + G[t][1] * (im[1] - c1) + G[t][2] * (im[2] - c2);
      }
      for (int j = 0; j < bsize; ++j) {
        uint32_t id = point_list[s0 + bstart + j];
        SFX(Sp) sp = SFX(load)(rules, means, shape, color, opac, id);
        double acc[11] = {0};
        int used = 0;
        for (int t = 0; t < 256; ++t) {
          if (j >= lim[t]) continue;
          if (rules == 2 && T[t] < (S)1e-4) continue;
          S pxf = (S)(tx * 16 + (t & 15)) + pix_off, pyf = (S)(ty * 16 + (t >> 4)) + pix_off;
          SFX(Ev) e;
          if (!SFX(eval)(rules, &sp, pxf, pyf, &e)) continue;
          used = 1;
          double w = (double)T[t] * e.alpha;
          double dot = G[t][0] * sp.cr + G[t][1] * sp.cg + G[t][2] * sp.cb;
          acc[6] += w * G[t][0];
          acc[7] += w * G[t][1];
          acc[8] += w * G[t][2];
          rho[t] -= w * dot;
          double dLda = (double)T[t] * dot - rho[t] / (1.0 - (double)e.alpha);
          SFX(shape_grads)(rules, &sp, &e, dLda, acc);
          T[t] = T[t] * ((S)1 - e.alpha);
        }
        if (!used) continue;
        if (rules == 2) acc[5] *= (double)sp.o * (1.0 - (double)sp.o);
        for (int k = 0; k < 9; ++k) grad_rec[12 * (int64_t)id + k] += acc[k];
        atomics += 9;
      }
    }
  }
  return atomics;
}

/* Per-pixel backward, back to front with T recovered by division (double arithmetic on the
 * S forward values). Returns the number of atomics the kernel issues. */
int64_t SFX(or2d_backward_pixel)(int rules, const S* means, const S* shape, const S* color, const S* opac,
                                 int64_t n, const uint32_t* ranges, const uint32_t* point_list, int W, int H,
                                 const double* bg, const S* final_T, const int32_t* limit, const S* grad_image,
                                 double* grad_rec) {
  int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
  int64_t HW = (int64_t)W * H, atomics = 0;
  S pix_off = rules == 1 ? (S)0 : (S)0.5;
  memset(grad_rec, 0, (size_t)n * 12 * sizeof(double));
  for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t s0 = ranges[2 * tile];
    for (int t = 0; t < 256; ++t) {
      int px = tx * 16 + (t & 15), py = ty * 16 + (t >> 4);
      if (px >= W || py >= H) continue;
      int64_t pix = (int64_t)py * W + px;
      double Gp[3], acc_c[3] = {0, 0, 0};
      for (int ch = 0; ch < 3; ++ch) Gp[ch] = rules == 1 ? grad_image[ch * HW + pix] : grad_image[3 * pix + ch];
      double bg_dot = (rules == 1 && bg) ? bg[0] * Gp[0] + bg[1] * Gp[1] + bg[2] * Gp[2] : 0.0;
      double Tf = final_T[pix], Tcur = Tf;
      S pxf = (S)px + pix_off, pyf = (S)py + pix_off;
      for (int pos = limit[pix] - 1; pos >= 0; --pos) {
        uint32_t id = point_list[s0 + pos];
        SFX(Sp) sp = SFX(load)(rules, means, shape, color, opac, id);
        SFX(Ev) e;
        if (!SFX(eval)(rules, &sp, pxf, pyf, &e)) continue;
        double a = e.alpha, oma = 1.0 - a;
        double Tb = Tcur / oma;
        double c[3] = {sp.cr, sp.cg, sp.cb};
        double dot = 0;
        for (int ch = 0; ch < 3; ++ch) dot += Gp[ch] * (c[ch] - acc_c[ch]);
        for (int ch = 0; ch < 3; ++ch) acc_c[ch] = a * c[ch] + oma * acc_c[ch];
        Tcur = Tb;
        double dLda = Tb * dot + (rules == 1 ? (-Tf / oma) * bg_dot : 0.0);
        double g[11] = {0};
        for (int ch = 0; ch < 3; ++ch) g[6 + ch] = a * Tb * Gp[ch];
        SFX(shape_grads)(rules, &sp, &e, dLda, g);
        if (rules == 2) g[5] *= (double)sp.o * (1.0 - (double)sp.o);
        for (int k = 0; k < 9; ++k) grad_rec[12 * (int64_t)id + k] += g[k];
        atomics += 9;
      }
    }
  }
  return atomics;
}

/* phase0 tile rectangles (float64 evaluation of the ellipse bounding box). */
void SFX(or2d_rects_phase0)(const S* means, const S* chol, const S* logit, int64_t n, int W, int H,
                            int32_t* rects, uint32_t* counts) {
  for (int64_t i = 0; i < n; ++i) {
    double mx = means[2 * i], my = means[2 * i + 1];
    double l0 = chol[3 * i], l1 = chol[3 * i + 1], l2 = chol[3 * i + 2];
    double o = or_sigmoid_f64((double)logit[i]);
    double r2 = 2.0 * or_log_f64(255.0 * o);
    double r = sqrt(fmax(r2, 0.0));
    double q = l1 / (l0 * l2);
    double ex = r * sqrt(1.0 / (l0 * l0) + q * q);
    double ey = r / fabs(l2);
    double x0 = floor((mx - ex) - 0.5) - 1.0, x1 = ceil((mx + ex) - 0.5) + 1.0;
    double y0 = floor((my - ey) - 0.5) - 1.0, y1 = ceil((my + ey) - 0.5) + 1.0;
    double wm = W - 1, hm = H - 1;
    int32_t* rr = rects + 4 * i;
    if (!((r2 > 0.0) && (x1 >= 0.0) && (x0 <= wm) && (y1 >= 0.0) && (y0 <= hm))) {
      rr[0] = rr[1] = rr[2] = rr[3] = 0;
      counts[i] = 0;
      continue;
    }
    int tx0 = (int)floor(fmin(fmax(x0, 0.0), wm) / 16), tx1 = (int)floor(fmin(fmax(x1, 0.0), wm) / 16);
    int ty0 = (int)floor(fmin(fmax(y0, 0.0), hm) / 16), ty1 = (int)floor(fmin(fmax(y1, 0.0), hm) / 16);
    rr[0] = tx0; rr[1] = ty0; rr[2] = tx1 + 1; rr[3] = ty1 + 1;
    counts[i] = (uint32_t)((tx1 - tx0 + 1) * (ty1 - ty0 + 1));
  }
}
