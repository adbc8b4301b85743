/*
 * CPU oracle for the 3D Gaussian-splat rasterizer path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load this library, and only as the checker / CPU baseline; the product path never
 * calls it.
 *
 * This is a plain-C restatement of the rules the rasterizer implements, evaluated in float32
 * with the same operation order as the GPU kernels for every decision (tile membership,
 * alpha >= 1/255, termination), so integer outputs must match bit for bit and the forward
 * image to rounding. Backward sums are accumulated in double.
 *
 * Rules and where they come from (the 3D rasterizer itself is Faster-GS, an external
 * dependency not present in the reference tree; its rules are taken from the in-tree patches):
 *   - pixel centre (x + 0.5, y + 0.5)                 upstream/upstream_main_kernels.patch:98
 *   - G = exp(min(power, 0)), alpha = o G, no clamp  phase1/fastergs_macro.patch:181-185, PLAN.md:53
 *     (the kernels take 2^x from the hardware exp2, this restatement from its own polynomial:
 *     forward decisions within a few ulp of a threshold are reported as ambiguous)
 *   - skip alpha < 1/255; stop after T < 1e-4        phase2/blend_stats.patch:132,246
 *   - (C, T) checkpoint every 32 list entries         phase1/fastergs_macro.patch:131,150-152
 *   - dL/dalpha = T (G.c) - rho_after / max(1-alpha, 1e-6), rho = G.(image - C)
 *                                                     phase1/fastergs_macro.patch:186-205
 *   - colour clamped at 0 with a gradient mask        phase1/fastergs_macro.patch:105-107
 *   - exp2-folded conic                               upstream/upstream_main_kernels.patch:9-13
 *   - SH basis and its backward                       phase2/sh_coalesce.patch:80-170
 *   - tile assignment: exact ellipse test per tile row against the alpha >= 1/255 ellipse (the
 *     role of create_instances_cu, phase2/ellipse_cull.patch:66-68); depth-sorted
 *     per-tile lists with ties in Gaussian-index order (phase2/tests/test_readback_equiv.py:57-59)
 *   - EWA projection with a 0.3 px^2 dilation and the 1.3x frustum clamp of the Jacobian
 *     (the published 3DGS preprocess; not pinned by any in-tree file).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define TILE 16
#define TILE_PIX 256
#define BUCKET 32
#define STRIP_ROWS 4
#define N_STRIPS 4

static const float ALPHA_MIN = 1.0f / 255.0f;
static const float T_STOP = 1e-4f;
static const float OMA_EPS = 1e-6f;
static const float DILATION = 0.3f;
static const float LOG2E = 1.44269504f;
static const float NEG_HALF_LOG2E = -0.72134752f;
static const float NEG_LOG2E = -1.44269504f;
static const float LN2 = 0.693147182f;
static const float SQRT2F = 1.41421354f;

/* ---- float32 elementary functions built from correctly rounded operations ---- */
static float poly2(float f) {
  float p = 0.00015469732170458883f;
  p = fmaf(p, f, 0.0013400432653725147f);
  p = fmaf(p, f, 0.00961802527308464f);
  p = fmaf(p, f, 0.05550327152013779f);
  p = fmaf(p, f, 0.24022650718688965f);
  p = fmaf(p, f, 0.6931471824645996f);
  p = fmaf(p, f, 1.0f);
  return p;
}

float or_exp2_neg(float x) {
  x = fmaxf(x, -64.0f);
  float k = rintf(x);
  return ldexpf(poly2(x - k), (int)k);
}

float or_exp2_any(float x) {
  x = fminf(fmaxf(x, -126.0f), 126.0f);
  float k = rintf(x);
  return ldexpf(poly2(x - k), (int)k);
}

static float exp_any(float x) { return or_exp2_any(x * LOG2E); }
float or_sigmoid(float z) { return 1.0f / (1.0f + exp_any(-z)); }

float or_log_pos(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  int e = (int)((bits >> 23) & 0xffu) - 127;
  uint32_t mb = (bits & 0x007fffffu) | 0x3f800000u;
  float m;
  memcpy(&m, &mb, 4);
  if (m > SQRT2F) {
    m = m * 0.5f;
    e = e + 1;
  }
  float s = (m - 1.0f) / (m + 1.0f);
  float s2 = s * s;
  float p = 1.0f / 9.0f;
  p = fmaf(p, s2, 1.0f / 7.0f);
  p = fmaf(p, s2, 1.0f / 5.0f);
  p = fmaf(p, s2, 1.0f / 3.0f);
  p = fmaf(p, s2, 1.0f);
  float t = s * p;
  t = t + t;
  return fmaf((float)e, LN2, t);
}

static uint32_t fbits(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return u;
}
static float bitsf(uint32_t u) {
  float v;
  memcpy(&v, &u, 4);
  return v;
}
static uint32_t order_key(float v) {
  uint32_t u = fbits(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* ---- camera ---- */
typedef struct {
  float viewmat[16];
  float fx, fy, cx, cy;
  int32_t width, height;
  float near_plane, far_plane;
  int32_t flags;
} or_camera;

#define CAM_PROPER_ANTIALIASING 1

typedef struct {
  float r[9], t[3];
  float fx, fy, cx, cy;
  int W, H;
  float znear, zfar;
  int flags;
  float campos[3];
  float lxlo, lxhi, lylo, lyhi;
  int tiles_x, tiles_y;
} Cam;

static Cam make_cam(const or_camera* c) {
  Cam k;
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 3; ++j) k.r[3 * i + j] = c->viewmat[4 * i + j];
    k.t[i] = c->viewmat[4 * i + 3];
  }
  k.fx = c->fx; k.fy = c->fy; k.cx = c->cx; k.cy = c->cy;
  k.W = c->width; k.H = c->height;
  k.znear = c->near_plane; k.zfar = c->far_plane;
  k.flags = c->flags;
  for (int j = 0; j < 3; ++j) {
    double s = 0.0;
    for (int i = 0; i < 3; ++i) s -= (double)c->viewmat[4 * i + j] * c->viewmat[4 * i + 3];
    k.campos[j] = (float)s;
  }
  k.lxlo = (float)(-1.3 * (double)c->cx / c->fx);
  k.lxhi = (float)(1.3 * ((double)c->width - c->cx) / c->fx);
  k.lylo = (float)(-1.3 * (double)c->cy / c->fy);
  k.lyhi = (float)(1.3 * ((double)c->height - c->cy) / c->fy);
  k.tiles_x = (c->width + TILE - 1) / TILE;
  k.tiles_y = (c->height + TILE - 1) / TILE;
  return k;
}

/* ---- real SH basis, degree <= 3 ---- */
static const float SH0 = 0.28209479177387814f, SH1 = 0.4886025119029199f;
static const float SH2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                             -1.0925484305920792f, 0.5462742152960396f};
static const float SH3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                             0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                             -0.5900435899266435f};

void or_sh_basis(float x, float y, float z, int n, float* b) {
  b[0] = SH0;
  if (n <= 1) return;
  b[1] = -SH1 * y;
  b[2] = SH1 * z;
  b[3] = -SH1 * x;
  if (n <= 4) return;
  float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
  b[4] = SH2[0] * xy;
  b[5] = SH2[1] * yz;
  {
    float t = zz + zz;
    t = t - xx;
    t = t - yy;
    b[6] = SH2[2] * t;
  }
  b[7] = SH2[3] * xz;
  b[8] = SH2[4] * (xx - yy);
  if (n <= 9) return;
  b[9] = (SH3[0] * y) * fmaf(3.0f, xx, -yy);
  b[10] = (SH3[1] * xy) * z;
  b[11] = (SH3[2] * y) * (fmaf(4.0f, zz, -xx) - yy);
  {
    float t = zz + zz;
    t = fmaf(-3.0f, xx, t);
    t = fmaf(-3.0f, yy, t);
    b[12] = (SH3[3] * z) * t;
  }
  b[13] = (SH3[4] * x) * (fmaf(4.0f, zz, -xx) - yy);
  b[14] = (SH3[5] * z) * (xx - yy);
  b[15] = (SH3[6] * x) * fmaf(-3.0f, yy, xx);
}

/* gradient of sum_k g[k] b_k(x,y,z), in double */
static void sh_basis_grad(double x, double y, double z, int n, const double* g, double* out) {
  double gx = 0, gy = 0, gz = 0;
  if (n > 1) {
    gy += -(double)SH1 * g[1];
    gz += (double)SH1 * g[2];
    gx += -(double)SH1 * g[3];
  }
  if (n > 4) {
    gx += SH2[0] * y * g[4]; gy += SH2[0] * x * g[4];
    gy += SH2[1] * z * g[5]; gz += SH2[1] * y * g[5];
    gx += -2.0 * SH2[2] * x * g[6]; gy += -2.0 * SH2[2] * y * g[6]; gz += 4.0 * SH2[2] * z * g[6];
    gx += SH2[3] * z * g[7]; gz += SH2[3] * x * g[7];
    gx += 2.0 * SH2[4] * x * g[8]; gy += -2.0 * SH2[4] * y * g[8];
  }
  if (n > 9) {
    double xx = x * x, yy = y * y, zz = z * z;
    gx += SH3[0] * 6.0 * x * y * g[9]; gy += SH3[0] * 3.0 * (xx - yy) * g[9];
    gx += SH3[1] * y * z * g[10]; gy += SH3[1] * x * z * g[10]; gz += SH3[1] * x * y * g[10];
    gx += SH3[2] * -2.0 * x * y * g[11]; gy += SH3[2] * (4.0 * zz - xx - 3.0 * yy) * g[11];
    gz += SH3[2] * 8.0 * y * z * g[11];
    gx += SH3[3] * -6.0 * x * z * g[12]; gy += SH3[3] * -6.0 * y * z * g[12];
    gz += SH3[3] * (6.0 * zz - 3.0 * xx - 3.0 * yy) * g[12];
    gx += SH3[4] * (4.0 * zz - 3.0 * xx - yy) * g[13]; gy += SH3[4] * -2.0 * x * y * g[13];
    gz += SH3[4] * 8.0 * x * z * g[13];
    gx += SH3[5] * 2.0 * x * z * g[14]; gy += SH3[5] * -2.0 * y * z * g[14]; gz += SH3[5] * (xx - yy) * g[14];
    gx += SH3[6] * 3.0 * (xx - yy) * g[15]; gy += SH3[6] * -6.0 * x * y * g[15];
  }
  out[0] = gx; out[1] = gy; out[2] = gz;
}

/* ---- forward geometry (float32, kernel operation order) ---- */
typedef struct {
  int vis;
  float vx, vy, vz, iz, tx, ty, txc, tyc, o;
  float os, rho, ratio, ar, cr; /* sigmoid, antialiasing factor sqrt(ratio), undilated diagonal */
  float qw, qx, qy, qz, qinv;
  float R[9], s[3], M[9], S[6], T[6];
  float a, b, c, det, A, B, C, mx, my;
} Geom;

static void geom(const float* means, const float* ls, const float* quats, const float* op, int64_t i,
                 const Cam* cam, Geom* g) {
  float px = means[3 * i], py = means[3 * i + 1], pz = means[3 * i + 2];
  g->vx = fmaf(cam->r[0], px, fmaf(cam->r[1], py, fmaf(cam->r[2], pz, cam->t[0])));
  g->vy = fmaf(cam->r[3], px, fmaf(cam->r[4], py, fmaf(cam->r[5], pz, cam->t[1])));
  g->vz = fmaf(cam->r[6], px, fmaf(cam->r[7], py, fmaf(cam->r[8], pz, cam->t[2])));
  int vis = (g->vz > cam->znear) && (g->vz < cam->zfar);
  g->o = or_sigmoid(op[i]);
  vis = vis && (g->o >= ALPHA_MIN);
  const float* q = quats + 4 * i;
  float n2 = fmaf(q[0], q[0], fmaf(q[1], q[1], fmaf(q[2], q[2], q[3] * q[3])));
  vis = vis && (n2 > 0.0f);
  g->qinv = 1.0f / sqrtf(n2);
  float w = q[0] * g->qinv, x = q[1] * g->qinv, y = q[2] * g->qinv, z = q[3] * g->qinv;
  g->qw = w; g->qx = x; g->qy = y; g->qz = z;
  float xx = x * x, yy = y * y, zz = z * z, xy = x * y, xz = x * z, yz = y * z;
  float wx = w * x, wy = w * y, wz = w * z, t;
  t = yy + zz; t = t + t; g->R[0] = 1.0f - t;
  t = xy - wz; g->R[1] = t + t;
  t = xz + wy; g->R[2] = t + t;
  t = xy + wz; g->R[3] = t + t;
  t = xx + zz; t = t + t; g->R[4] = 1.0f - t;
  t = yz - wx; g->R[5] = t + t;
  t = xz - wy; g->R[6] = t + t;
  t = yz + wx; g->R[7] = t + t;
  t = xx + yy; t = t + t; g->R[8] = 1.0f - t;
  for (int k = 0; k < 3; ++k) g->s[k] = exp_any(ls[3 * i + k]);
  for (int r = 0; r < 3; ++r)
    for (int k = 0; k < 3; ++k) g->M[3 * r + k] = g->R[3 * r + k] * g->s[k];
  const float* M = g->M;
  g->S[0] = fmaf(M[0], M[0], fmaf(M[1], M[1], M[2] * M[2]));
  g->S[1] = fmaf(M[0], M[3], fmaf(M[1], M[4], M[2] * M[5]));
  g->S[2] = fmaf(M[0], M[6], fmaf(M[1], M[7], M[2] * M[8]));
  g->S[3] = fmaf(M[3], M[3], fmaf(M[4], M[4], M[5] * M[5]));
  g->S[4] = fmaf(M[3], M[6], fmaf(M[4], M[7], M[5] * M[8]));
  g->S[5] = fmaf(M[6], M[6], fmaf(M[7], M[7], M[8] * M[8]));
  g->iz = 1.0f / g->vz;
  g->tx = g->vx * g->iz;
  g->ty = g->vy * g->iz;
  g->txc = fminf(fmaxf(g->tx, cam->lxlo), cam->lxhi);
  g->tyc = fminf(fmaxf(g->ty, cam->lylo), cam->lyhi);
  float j00 = cam->fx * g->iz, j11 = cam->fy * g->iz;
  float j02 = -(j00 * g->txc), j12 = -(j11 * g->tyc);
  for (int k = 0; k < 3; ++k) {
    g->T[k] = fmaf(j00, cam->r[k], j02 * cam->r[6 + k]);
    g->T[3 + k] = fmaf(j11, cam->r[3 + k], j12 * cam->r[6 + k]);
  }
  const float* S = g->S;
  const float* T = g->T;
  float u00 = fmaf(T[0], S[0], fmaf(T[1], S[1], T[2] * S[2]));
  float u01 = fmaf(T[0], S[1], fmaf(T[1], S[3], T[2] * S[4]));
  float u02 = fmaf(T[0], S[2], fmaf(T[1], S[4], T[2] * S[5]));
  float u10 = fmaf(T[3], S[0], fmaf(T[4], S[1], T[5] * S[2]));
  float u11 = fmaf(T[3], S[1], fmaf(T[4], S[3], T[5] * S[4]));
  float u12 = fmaf(T[3], S[2], fmaf(T[4], S[4], T[5] * S[5]));
  g->ar = fmaf(u00, T[0], fmaf(u01, T[1], u02 * T[2]));
  g->b = fmaf(u00, T[3], fmaf(u01, T[4], u02 * T[5]));
  g->cr = fmaf(u10, T[3], fmaf(u11, T[4], u12 * T[5]));
  g->a = g->ar + DILATION;
  g->c = g->cr + DILATION;
  g->det = fmaf(g->a, g->c, -(g->b * g->b));
  vis = vis && (g->det > 0.0f);
  /* proper antialiasing: the 0.3 px^2 low-pass keeps the splat's integral, o sqrt(det S / det S')
   * (Mip-Splatting's 2D filter; Faster-GS's flag, phase1/fastergs_macro.patch:215) */
  g->os = g->o;
  g->rho = 1.0f;
  g->ratio = 1.0f;
  if (cam->flags & CAM_PROPER_ANTIALIASING) {
    float det_raw = fmaf(g->ar, g->cr, -(g->b * g->b));
    g->ratio = fmaxf(det_raw / g->det, 0.0f);
    g->rho = sqrtf(g->ratio);
    g->o = g->os * g->rho;
    vis = vis && (g->o >= ALPHA_MIN);
  }
  float idet = 1.0f / g->det;
  g->A = g->c * idet;
  g->B = -g->b * idet;
  g->C = g->a * idet;
  g->mx = fmaf(cam->fx, g->tx, cam->cx);
  g->my = fmaf(cam->fy, g->ty, cam->cy);
  g->vis = vis;
}

/* Tile assignment (row-band rule): for each tile row, the pixel-centre band [Y0, Y1] (tile
 * rows clipped to the pixel bounds) meets the ellipse 1/2 d^T Q d <= thr in a convex set with
 * x-extent [xl, xr]; the splat touches the tiles owning a column c of its bounds with
 * c + 0.5 in [xl, xr]. Outputs the column range; returns 0 if the band misses. */
int or_band_columns(float mx, float my, float A, float B, float C, float thr, float Y0, float Y1,
                    int bx0, int bx1, int* c0, int* c1) {
  float t2 = thr + thr;
  float det = fmaf(A, C, -(B * B));
  if (!(det > 0.0f)) return 0;
  float tA = t2 * A;
  float idet = 1.0f / det, invA = 1.0f / A;
  float vmax = sqrtf(tA * idet);
  float ur = sqrtf((t2 * C) * idet);
  float vr = -((B / C) * ur);
  float v0 = fmaxf(Y0 - my, -vmax);
  float v1 = fminf(Y1 - my, vmax);
  if (!(v0 <= v1)) return 0;
  float vc = fminf(fmaxf(vr, v0), v1);
  float dr = fmaxf(fmaf(-det, vc * vc, tA), 0.0f);
  float br = B * vc;
  float xr = mx + (sqrtf(dr) - br) * invA;
  float vl = fminf(fmaxf(-vr, v0), v1);
  float dl = fmaxf(fmaf(-det, vl * vl, tA), 0.0f);
  float bl = B * vl;
  float xl = mx + (-bl - sqrtf(dl)) * invA;
  float f0 = fmaxf(ceilf(xl - 0.5f), (float)bx0);
  float f1 = fminf(floorf(xr - 0.5f), (float)bx1);
  if (!(f0 <= f1)) return 0;
  *c0 = (int)f0;
  *c1 = (int)f1;
  return 1;
}

/* record layout: a = (mx, my, A, B), b = (C, o, depth, thr), c = (r, g, b, mask), d = (x0, x1, y0, y1) */
static int touched_tiles(const float* rec, int tiles_x, uint32_t* tiles_out) {
  const int32_t* d = (const int32_t*)(rec + 12);
  int cnt = 0;
  for (int ty = d[2] / TILE; ty <= d[3] / TILE; ++ty) {
    int py0 = ty * TILE > d[2] ? ty * TILE : d[2];
    int py1 = ty * TILE + TILE - 1 < d[3] ? ty * TILE + TILE - 1 : d[3];
    int c0, c1;
    if (!or_band_columns(rec[0], rec[1], rec[2], rec[3], rec[4], rec[7], (float)py0 + 0.5f,
                         (float)py1 + 0.5f, d[0], d[1], &c0, &c1))
      continue;
    for (int tx = c0 / TILE; tx <= c1 / TILE; ++tx) {
      if (tiles_out) tiles_out[cnt] = (uint32_t)(ty * tiles_x + tx);
      ++cnt;
    }
  }
  return cnt;
}

int or_preprocess_fwd(const float* means, const float* ls, const float* quats, const float* op,
                      const float* sh, int64_t n, int K, int sh_degree, const or_camera* camera,
                      float* rec, uint32_t* touched) {
  Cam cam = make_cam(camera);
  int active = (sh_degree + 1) * (sh_degree + 1);
#pragma omp parallel for schedule(dynamic, 1024)
  for (int64_t i = 0; i < n; ++i) {
    Geom g;
    geom(means, ls, quats, op, i, &cam, &g);
    touched[i] = 0;
    if (!g.vis) continue;
    float thr = or_log_pos(255.0f * g.o);
    float t2 = thr + thr;
    float ex = sqrtf(t2 * g.a), ey = sqrtf(t2 * g.c);
    float xf0 = ceilf((g.mx - ex) - 0.5f), xf1 = floorf((g.mx + ex) - 0.5f);
    float yf0 = ceilf((g.my - ey) - 0.5f), yf1 = floorf((g.my + ey) - 0.5f);
    int ok = (thr > 0.0f) && isfinite(xf0) && isfinite(xf1) && isfinite(yf0) && isfinite(yf1);
    xf0 = fmaxf(xf0, 0.0f);
    yf0 = fmaxf(yf0, 0.0f);
    xf1 = fminf(xf1, (float)(cam.W - 1));
    yf1 = fminf(yf1, (float)(cam.H - 1));
    ok = ok && (xf0 <= xf1) && (yf0 <= yf1);
    if (!ok) continue;
    float* r = rec + 16 * i;
    r[0] = g.mx; r[1] = g.my; r[2] = g.A; r[3] = g.B;
    r[4] = g.C; r[5] = g.o; r[6] = g.vz; r[7] = thr;
    int32_t* d = (int32_t*)(r + 12);
    d[0] = (int32_t)xf0; d[1] = (int32_t)xf1; d[2] = (int32_t)yf0; d[3] = (int32_t)yf1;
    int cnt = touched_tiles(r, cam.tiles_x, NULL);
    if (cnt == 0) continue;
    /* colour */
    float dx = means[3 * i] - cam.campos[0];
    float dy = means[3 * i + 1] - cam.campos[1];
    float dz = means[3 * i + 2] - cam.campos[2];
    float len = sqrtf(fmaf(dx, dx, fmaf(dy, dy, dz * dz)));
    float il = 1.0f / len;
    float basis[16];
    or_sh_basis(dx * il, dy * il, dz * il, active, basis);
    const float* row = sh + (int64_t)i * 3 * K;
    uint32_t mask = 0;
    for (int ch = 0; ch < 3; ++ch) {
      float acc = basis[0] * row[ch];
      for (int k = 1; k < active; ++k) acc = fmaf(basis[k], row[3 * k + ch], acc);
      acc = acc + 0.5f;
      if (acc < 0.0f) mask |= 1u << ch;
      r[8 + ch] = fmaxf(acc, 0.0f);
    }
    r[11] = bitsf(mask);
    touched[i] = (uint32_t)cnt;
  }
  return 0;
}

/* ---- binning ---- */
typedef struct {
  uint64_t key;
  uint32_t val;
  uint32_t seq;
} Inst;

static int inst_cmp(const void* a, const void* b) {
  const Inst* x = (const Inst*)a;
  const Inst* y = (const Inst*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  return x->seq < y->seq ? -1 : (x->seq > y->seq ? 1 : 0);
}

/* Emits instances in Gaussian-index order and sorts them stably by key. */
int64_t or_bin(const float* rec, const uint32_t* touched, int64_t n, const or_camera* camera,
               uint64_t* keys_out, uint32_t* point_list, uint32_t* ranges, uint32_t* bucket_offsets) {
  Cam cam = make_cam(camera);
  int n_tiles = cam.tiles_x * cam.tiles_y;
  int64_t m = 0;
  for (int64_t i = 0; i < n; ++i) m += touched[i];
  Inst* inst = (Inst*)malloc((size_t)(m > 0 ? m : 1) * sizeof(Inst));
  uint32_t* tl = (uint32_t*)malloc((size_t)n_tiles * sizeof(uint32_t));
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (!touched[i]) continue;
    const float* r = rec + 16 * i;
    int cnt = touched_tiles(r, cam.tiles_x, tl);
    uint64_t dk = order_key(r[6]);
    for (int c = 0; c < cnt; ++c) {
      inst[k].key = ((uint64_t)tl[c] << 32) | dk;
      inst[k].val = (uint32_t)i;
      inst[k].seq = (uint32_t)k;
      ++k;
    }
  }
  free(tl);
  if (k != m) {
    free(inst);
    return -1;
  }
  qsort(inst, (size_t)m, sizeof(Inst), inst_cmp);
  /* CSR ranges: tile t holds [start, end); an empty tile has an empty range at its position */
  for (int t = 0; t < 2 * n_tiles; ++t) ranges[t] = 0;
  for (int64_t p = 0; p < m; ++p) {
    keys_out[p] = inst[p].key;
    point_list[p] = inst[p].val;
    ranges[2 * (inst[p].key >> 32) + 1]++;
  }
  uint32_t run = 0;
  for (int t = 0; t < n_tiles; ++t) {
    ranges[2 * t] = run;
    run += ranges[2 * t + 1];
    ranges[2 * t + 1] = run;
  }
  free(inst);
  bucket_offsets[0] = 0;
  for (int t = 0; t < n_tiles; ++t) {
    uint32_t len = ranges[2 * t + 1] - ranges[2 * t];
    bucket_offsets[t + 1] = bucket_offsets[t] + (len + BUCKET - 1) / BUCKET;
  }
  return m;
}

/* ---- blending ---- */
/* qa dx^2 + qb dx dy + qc dy^2 as a0 + dy (qc dy + b1), a0 = (qa dx) dx, b1 = qb dx (the
 * column terms a lane owning several pixels of one column shares), clamped to <= 0. */
static float power2(float qa, float qb, float qc, float dx, float dy) {
  float a0 = (qa * dx) * dx;
  float b1 = qb * dx;
  float e = fmaf(dy, fmaf(qc, dy, b1), a0);
  return fminf(e, 0.0f);
}

static int strip_hit(const float* r, int tile_y0, int strip) {
  const int32_t* d = (const int32_t*)(r + 12);
  int r0 = tile_y0 + STRIP_ROWS * strip, r1 = r0 + STRIP_ROWS - 1;
  return d[2] <= r1 && d[3] >= r0;
}

/* A forward decision is ambiguous between this restatement's polynomial exp2 and the
 * kernels' hardware exp2 (each within about 1 ulp) when it falls inside the error the two can
 * accumulate: alpha >= 1/255 within AMB_ALPHA (relative; the two alphas are at most ~3 ulp
 * apart), and T < 1e-4 within a running relative bound on T that every composite grows by
 * AMB_ALPHA * alpha / (1 - alpha) (the alpha error carried through 1 - alpha) plus one
 * rounding of the product. */
#define AMB_ALPHA 4e-7f
#define AMB_ROUND 1.2e-7f

/* ckpt and amb may be NULL. Checkpoints are written for every bucket the pixel loop reaches.
 * amb [H, W] = 1 where some decision of the pixel fell within the margins above (its
 * n_contrib, and the image from that point on, may then legitimately differ).
 * scores (may be NULL): scores[g] += the blending weight alpha T of splat g at every pixel it is
 * blended into (the pruning-score blend). */
int or_blend_fwd(const float* rec, const uint32_t* ranges, const uint32_t* point_list,
                 const uint32_t* bucket_offsets, int W, int H, const float* bg, float* image,
                 float* final_T, int32_t* n_contrib, uint32_t* tile_max, float* ckpt, uint8_t* amb,
                 double* scores) {
  int tiles_x = (W + TILE - 1) / TILE, tiles_y = (H + TILE - 1) / TILE;
  int64_t HW = (int64_t)W * H;
  float bgc[3] = {bg ? bg[0] : 0.0f, bg ? bg[1] : 0.0f, bg ? bg[2] : 0.0f};
#pragma omp parallel for schedule(dynamic, 1)
  for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t s = ranges[2 * tile], e = ranges[2 * tile + 1];
    uint32_t tmax = 0;
    for (int t = 0; t < TILE_PIX; ++t) {
      int px = tx * TILE + (t & 15), py = ty * TILE + (t >> 4);
      int inside = px < W && py < H;
      float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
      int strip = (t >> 4) / STRIP_ROWS;
      float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f};
      int last = 0, done = !inside, near = 0;
      float tbound = 0.0f; /* relative error bound of T between the two exp2s */
      for (uint32_t idx = 0; idx < e - s; ++idx) {
        if (done) break; /* later checkpoints of this pixel keep (C, T) */
        if ((idx % BUCKET) == 0 && ckpt) {
          float* c = ckpt + ((int64_t)(bucket_offsets[tile] + idx / BUCKET) * TILE_PIX + t) * 4;
          c[0] = C[0]; c[1] = C[1]; c[2] = C[2]; c[3] = T;
        }
        const float* r = rec + 16 * (int64_t)point_list[s + idx];
        if (!strip_hit(r, ty * TILE, strip)) continue;
        float qa = r[2] * NEG_HALF_LOG2E, qb = r[3] * NEG_LOG2E, qc = r[4] * NEG_HALF_LOG2E;
        float dx = r[0] - pxf, dy = r[1] - pyf;
        float G = or_exp2_neg(power2(qa, qb, qc, dx, dy));
        float alpha = r[5] * G;
        if (fabsf(alpha - ALPHA_MIN) <= AMB_ALPHA * ALPHA_MIN) near = 1;
        if (alpha < ALPHA_MIN) continue;
        float w = alpha * T;
        if (scores) {
#pragma omp atomic
          scores[point_list[s + idx]] += (double)w;
        }
        C[0] = fmaf(r[8], w, C[0]);
        C[1] = fmaf(r[9], w, C[1]);
        C[2] = fmaf(r[10], w, C[2]);
        T = T * (1.0f - alpha);
        tbound += AMB_ALPHA * alpha / (1.0f - alpha) + AMB_ROUND;
        last = (int)idx + 1;
        if (fabsf(T - T_STOP) <= tbound * T_STOP) near = 1;
        if (T < T_STOP) done = 1;
      }
      if (ckpt) { /* checkpoints past the termination point keep the final state */
        for (uint32_t idx = ((uint32_t)last + BUCKET - 1) / BUCKET * BUCKET; idx < e - s; idx += BUCKET) {
          float* c = ckpt + ((int64_t)(bucket_offsets[tile] + idx / BUCKET) * TILE_PIX + t) * 4;
          c[0] = C[0]; c[1] = C[1]; c[2] = C[2]; c[3] = T;
        }
      }
      if (inside) {
        int64_t pix = (int64_t)py * W + px;
        image[pix] = fmaf(T, bgc[0], C[0]);
        image[HW + pix] = fmaf(T, bgc[1], C[1]);
        image[2 * HW + pix] = fmaf(T, bgc[2], C[2]);
        final_T[pix] = T;
        n_contrib[pix] = last;
        if (amb) amb[pix] = (uint8_t)near;
        if ((uint32_t)last > tmax) tmax = (uint32_t)last;
      }
    }
    tile_max[tile] = tmax;
  }
  return 0;
}

/* Discrete structure of the forward, for a float64 reference: mask[p][t] = 1 iff list entry p
 * (of its tile) was blended into pixel t of that tile (t = 16 * row + column): the pixel is
 * inside the image, p precedes the pixel's termination (position < n_contrib), the splat's
 * bounds reach the pixel's strip and alpha (float32, as in the kernels) is >= 1/255. */
int or_contrib_mask(const float* rec, const uint32_t* ranges, const uint32_t* point_list, int W, int H,
                    const int32_t* n_contrib, uint8_t* mask) {
  int tiles_x = (W + TILE - 1) / TILE, tiles_y = (H + TILE - 1) / TILE;
  for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t s = ranges[2 * tile], e = ranges[2 * tile + 1];
    for (uint32_t p = s; p < e; ++p) {
      const float* r = rec + 16 * (int64_t)point_list[p];
      float qa = r[2] * NEG_HALF_LOG2E, qb = r[3] * NEG_LOG2E, qc = r[4] * NEG_HALF_LOG2E;
      for (int t = 0; t < TILE_PIX; ++t) {
        int px = tx * TILE + (t & 15), py = ty * TILE + (t >> 4);
        uint8_t v = 0;
        if (px < W && py < H && (int)(p - s) < n_contrib[(int64_t)py * W + px] &&
            strip_hit(r, ty * TILE, (t >> 4) / STRIP_ROWS)) {
          float dx = r[0] - ((float)px + 0.5f), dy = r[1] - ((float)py + 0.5f);
          float alpha = r[5] * or_exp2_neg(power2(qa, qb, qc, dx, dy));
          v = alpha >= ALPHA_MIN;
        }
        mask[(int64_t)p * TILE_PIX + t] = v;
      }
    }
  }
  return 0;
}

/* Bucketed backward in double, replaying each bucket from its checkpoint.
 * grad2d [n,12] is overwritten (the double sums rounded to float); conic64 [n,4] (may be NULL)
 * receives the conic-gradient sums (columns 2-4) unrounded. */
int or_blend_bwd(const float* rec, const uint32_t* ranges, const uint32_t* point_list,
                 const uint32_t* bucket_offsets, int W, int H, const float* image,
                 const float* grad_image, const float* final_T, const float* grad_alpha,
                 const int32_t* n_contrib, const uint32_t* tile_max, const float* ckpt, int64_t n,
                 float* grad2d, double* conic64) {
  int tiles_x = (W + TILE - 1) / TILE, tiles_y = (H + TILE - 1) / TILE;
  int64_t HW = (int64_t)W * H;
  double* acc = (double*)calloc((size_t)n * 12, sizeof(double));
  /* tiles in parallel; each bucket's per-splat sums are formed over its pixels in double, then
   * added to the shared totals (one atomic add per value and splat of the bucket) */
#pragma omp parallel for schedule(dynamic, 1)
  for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
    int tx = tile % tiles_x, ty = tile / tiles_x;
    uint32_t s = ranges[2 * tile];
    double loc[BUCKET][12];
    for (uint32_t b = bucket_offsets[tile]; b < bucket_offsets[tile + 1]; ++b) {
      int bstart = (int)(b - bucket_offsets[tile]) * BUCKET;
      if (bstart >= (int)tile_max[tile]) break;
      int bsize = (int)tile_max[tile] - bstart;
      if (bsize > BUCKET) bsize = BUCKET;
      memset(loc, 0, sizeof(loc));
      for (int t = 0; t < TILE_PIX; ++t) {
        int px = tx * TILE + (t & 15), py = ty * TILE + (t >> 4);
        if (px >= W || py >= H) continue;
        int64_t pix = (int64_t)py * W + px;
        int lim = n_contrib[pix] - bstart;
        if (lim <= 0) continue;
        float pxf = (float)px + 0.5f, pyf = (float)py + 0.5f;
        int strip = (t >> 4) / STRIP_ROWS;
        const float* ck = ckpt + ((int64_t)b * TILE_PIX + t) * 4;
        float T = ck[3];
        double G[3] = {grad_image[pix], grad_image[HW + pix], grad_image[2 * HW + pix]};
        double rho = G[0] * ((double)image[pix] - ck[0]) + G[1] * ((double)image[HW + pix] - ck[1]) +
                     G[2] * ((double)image[2 * HW + pix] - ck[2]);
        if (grad_alpha) rho -= (double)grad_alpha[pix] * final_T[pix];
        for (int j = 0; j < bsize && j < lim; ++j) {
          uint32_t id = point_list[s + bstart + j];
          const float* r = rec + 16 * (int64_t)id;
          if (!strip_hit(r, ty * TILE, strip)) continue;
          float qa = r[2] * NEG_HALF_LOG2E, qb = r[3] * NEG_LOG2E, qc = r[4] * NEG_HALF_LOG2E;
          float dx = r[0] - pxf, dy = r[1] - pyf;
          float Gs = or_exp2_neg(power2(qa, qb, qc, dx, dy));
          float alpha = r[5] * Gs;
          if (alpha < ALPHA_MIN) continue;
          double w = (double)T * alpha;
          double dot = G[0] * r[8] + G[1] * r[9] + G[2] * r[10];
          double* a = loc[j];
          a[6] += w * G[0]; a[7] += w * G[1]; a[8] += w * G[2];
          rho -= w * dot;
          float oma = 1.0f - alpha;
          double dLda = (double)T * dot - rho / (double)fmaxf(oma, OMA_EPS);
          a[5] += (double)alpha * dLda; /* opacity times dL/dopacity (sum alpha dL/dalpha) */
          double hp = (double)alpha * dLda;
          a[2] += -0.5 * hp * dx * dx;
          a[3] += -hp * dx * dy;
          a[4] += -0.5 * hp * dy * dy;
          double gmx = -hp * ((double)r[2] * dx + (double)r[3] * dy);
          double gmy = -hp * ((double)r[3] * dx + (double)r[4] * dy);
          a[0] += gmx; a[1] += gmy;
          a[9] += fabs(gmx); a[10] += fabs(gmy);
          T = T * oma;
        }
      }
      for (int j = 0; j < bsize; ++j) {
        double* dst = acc + 12 * (int64_t)point_list[s + bstart + j];
        for (int k = 0; k < 11; ++k) {
          if (loc[j][k] == 0.0) continue;
#pragma omp atomic
          dst[k] += loc[j][k];
        }
      }
    }
  }
  for (int64_t i = 0; i < n * 12; ++i) grad2d[i] = (float)acc[i];
  if (conic64)
    for (int64_t i = 0; i < n; ++i) {
      for (int k = 0; k < 3; ++k) conic64[4 * i + k] = acc[12 * i + 2 + k];
      conic64[4 * i + 3] = 0.0;
    }
  free(acc);
  return 0;
}

/* ---- preprocess backward (double arithmetic on the float32 forward quantities) ---- */
int or_preprocess_bwd(const float* means, const float* ls, const float* quats, const float* op,
                      const float* sh, int64_t n, int K, int sh_degree, const or_camera* camera,
                      const float* rec, const uint32_t* touched, const float* grad2d,
                      const double* conic64, float* g_means, float* g_ls, float* g_quats, float* g_op,
                      float* g_sh) {
  Cam cam = make_cam(camera);
  int active = (sh_degree + 1) * (sh_degree + 1);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    for (int k = 0; k < 3; ++k) g_means[3 * i + k] = g_ls[3 * i + k] = 0.0f;
    for (int k = 0; k < 4; ++k) g_quats[4 * i + k] = 0.0f;
    g_op[i] = 0.0f;
    for (int k = 0; k < 3 * K; ++k) g_sh[3 * K * i + k] = 0.0f;
    if (!touched[i]) continue;
    const float* g2 = grad2d + 12 * i;
    const float* r = rec + 16 * i;
    uint32_t mask = fbits(r[11]);
    double gcol[3];
    for (int ch = 0; ch < 3; ++ch) gcol[ch] = (mask & (1u << ch)) ? 0.0 : g2[6 + ch];
    double gm[3] = {0, 0, 0};
    /* SH */
    float dxw = means[3 * i] - cam.campos[0], dyw = means[3 * i + 1] - cam.campos[1],
          dzw = means[3 * i + 2] - cam.campos[2];
    double len = sqrt((double)dxw * dxw + (double)dyw * dyw + (double)dzw * dzw);
    double d[3] = {dxw / len, dyw / len, dzw / len};
    float basis[16];
    or_sh_basis((float)d[0], (float)d[1], (float)d[2], active, basis);
    const float* row = sh + (int64_t)i * 3 * K;
    double gb[16];
    for (int k = 0; k < 16; ++k) gb[k] = 0.0;
    for (int k = 0; k < active; ++k) {
      gb[k] = row[3 * k] * gcol[0] + row[3 * k + 1] * gcol[1] + row[3 * k + 2] * gcol[2];
      for (int ch = 0; ch < 3; ++ch) g_sh[3 * K * i + 3 * k + ch] = (float)(basis[k] * gcol[ch]);
    }
    double gd[3];
    sh_basis_grad(d[0], d[1], d[2], active, gb, gd);
    double dd = d[0] * gd[0] + d[1] * gd[1] + d[2] * gd[2];
    for (int k = 0; k < 3; ++k) gm[k] = (gd[k] - d[k] * dd) / len;
    /* geometry */
    Geom g;
    geom(means, ls, quats, op, i, &cam, &g);
    int aa = cam.flags & CAM_PROPER_ANTIALIASING;
    /* g2[5] = o dL/do for the blended opacity o = os rho: dL/dlogit = g2[5] (1 - os) */
    g_op[i] = (float)((double)g2[5] * (1.0 - (aa ? g.os : g.o)));
    double iz = 1.0 / g.vz;
    double gvx = g2[0] * (double)cam.fx * iz, gvy = g2[1] * (double)cam.fy * iz;
    double gvz = -((double)g2[0] * cam.fx * g.vx + (double)g2[1] * cam.fy * g.vy) * iz * iz;
    double a = g.a, b = g.b, c = g.c, det = a * c - b * b;
    /* the conic gradient: grad2d's float columns, or conic64's unrounded sums when given */
    double gA = g2[2], gB = g2[3], gC = g2[4], id2 = 1.0 / (det * det);
    if (conic64) {
      gA = conic64[4 * i];
      gB = conic64[4 * i + 1];
      gC = conic64[4 * i + 2];
    }
    double ga = (-c * c * gA + b * c * gB - b * b * gC) * id2;
    double gbb = (2 * b * c * gA - (a * c + b * b) * gB + 2 * a * b * gC) * id2;
    double gc = (-b * b * gA + a * b * gB - a * a * gC) * id2;
    if (aa) { /* d/d(a, b, c) of rho = sqrt((ar cr - b^2) / (a c - b^2)), ar = a - 0.3, cr = c - 0.3 */
      double ar = g.ar, cr = g.cr, ratio = (ar * cr - b * b) / det, rho = sqrt(ratio);
      double k = (double)g2[5] / (2.0 * (double)g.rho * rho * det);
      ga += k * (cr - ratio * c);
      gc += k * (ar - ratio * a);
      gbb += -2.0 * k * b * (1.0 - ratio);
    }
    double Gc[2][2] = {{ga, 0.5 * gbb}, {0.5 * gbb, gc}};
    double T[2][3], Sm[3][3];
    for (int k = 0; k < 3; ++k) { T[0][k] = g.T[k]; T[1][k] = g.T[3 + k]; }
    Sm[0][0] = g.S[0]; Sm[0][1] = Sm[1][0] = g.S[1]; Sm[0][2] = Sm[2][0] = g.S[2];
    Sm[1][1] = g.S[3]; Sm[1][2] = Sm[2][1] = g.S[4]; Sm[2][2] = g.S[5];
    double GT[2][3], dS[3][3], dT[2][3];
    for (int r0 = 0; r0 < 2; ++r0)
      for (int k = 0; k < 3; ++k) GT[r0][k] = Gc[r0][0] * T[0][k] + Gc[r0][1] * T[1][k];
    for (int r0 = 0; r0 < 3; ++r0)
      for (int c0 = 0; c0 < 3; ++c0) dS[r0][c0] = T[0][r0] * GT[0][c0] + T[1][r0] * GT[1][c0];
    for (int r0 = 0; r0 < 2; ++r0)
      for (int c0 = 0; c0 < 3; ++c0) {
        double s = 0;
        for (int k = 0; k < 3; ++k) s += GT[r0][k] * Sm[k][c0];
        dT[r0][c0] = 2 * s;
      }
    double gj00 = 0, gj02 = 0, gj11 = 0, gj12 = 0;
    for (int k = 0; k < 3; ++k) {
      gj00 += dT[0][k] * cam.r[k];
      gj02 += dT[0][k] * cam.r[6 + k];
      gj11 += dT[1][k] * cam.r[3 + k];
      gj12 += dT[1][k] * cam.r[6 + k];
    }
    double iz2 = iz * iz;
    gvz += -cam.fx * iz2 * gj00 - cam.fy * iz2 * gj11;
    gvz += cam.fx * (double)g.txc * iz2 * gj02 + cam.fy * (double)g.tyc * iz2 * gj12;
    if (g.tx >= cam.lxlo && g.tx <= cam.lxhi) {
      gvx += -cam.fx * iz2 * gj02;
      gvz += cam.fx * (double)g.vx * iz2 * iz * gj02;
    }
    if (g.ty >= cam.lylo && g.ty <= cam.lyhi) {
      gvy += -cam.fy * iz2 * gj12;
      gvz += cam.fy * (double)g.vy * iz2 * iz * gj12;
    }
    gm[0] += cam.r[0] * gvx + cam.r[3] * gvy + cam.r[6] * gvz;
    gm[1] += cam.r[1] * gvx + cam.r[4] * gvy + cam.r[7] * gvz;
    gm[2] += cam.r[2] * gvx + cam.r[5] * gvy + cam.r[8] * gvz;
    double dM[3][3], dR[3][3];
    for (int r0 = 0; r0 < 3; ++r0)
      for (int c0 = 0; c0 < 3; ++c0) {
        double s = 0;
        for (int k = 0; k < 3; ++k) s += dS[r0][k] * g.M[3 * k + c0];
        dM[r0][c0] = 2 * s;
      }
    for (int k = 0; k < 3; ++k) {
      double ds = 0;
      for (int r0 = 0; r0 < 3; ++r0) {
        ds += dM[r0][k] * g.R[3 * r0 + k];
        dR[r0][k] = dM[r0][k] * g.s[k];
      }
      g_ls[3 * i + k] = (float)(ds * g.s[k]);
    }
    double w = g.qw, x = g.qx, y = g.qy, z = g.qz;
    double gw = 2 * (-z * dR[0][1] + y * dR[0][2] + z * dR[1][0] - x * dR[1][2] - y * dR[2][0] + x * dR[2][1]);
    double gx = 2 * (y * dR[0][1] + z * dR[0][2] + y * dR[1][0] - 2 * x * dR[1][1] - w * dR[1][2] + z * dR[2][0] +
                     w * dR[2][1] - 2 * x * dR[2][2]);
    double gy = 2 * (-2 * y * dR[0][0] + x * dR[0][1] + w * dR[0][2] + x * dR[1][0] + z * dR[1][2] - w * dR[2][0] +
                     z * dR[2][1] - 2 * y * dR[2][2]);
    double gz = 2 * (-2 * z * dR[0][0] - w * dR[0][1] + x * dR[0][2] + w * dR[1][0] - 2 * z * dR[1][1] +
                     y * dR[1][2] + x * dR[2][0] + y * dR[2][1]);
    double qd = w * gw + x * gx + y * gy + z * gz;
    g_quats[4 * i + 0] = (float)((gw - w * qd) * g.qinv);
    g_quats[4 * i + 1] = (float)((gx - x * qd) * g.qinv);
    g_quats[4 * i + 2] = (float)((gy - y * qd) * g.qinv);
    g_quats[4 * i + 3] = (float)((gz - z * qd) * g.qinv);
    for (int k = 0; k < 3; ++k) g_means[3 * i + k] = (float)gm[k];
  }
  return 0;
}
