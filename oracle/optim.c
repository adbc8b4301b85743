/* CPU restatement of the fused Adam update (TEST INFRASTRUCTURE: used by tests/ only).
 *
 * Follows cluster/patches/fastergs_lean_adam.patch:96-139 (the per-element update and the
 * bfloat16 stochastic rounding) and :165-169 (step size and bias corrections in double, the
 * seed of the rounding noise), with the same float32 rounding steps as the kernel. */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* 32-bit "lowbias32" hash finaliser (patch :84-87). */
uint32_t or_sr_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

static float bits_to_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* bfloat16 bits of f with stochastic rounding: noise in the 16 dropped bits, then truncation
 * (patch :94-97). */
uint16_t or_bf16_sr(float f, uint32_t rnd) { return (uint16_t)((f_to_bits(f) + (rnd & 0xffffu)) >> 16); }

/* One Adam step over n elements of a [n_prim, n / n_prim] group. lowp: moments are bfloat16
 * bits (uint16). vis: per-primitive visibility or NULL. */
void or_adam_step(const float* grad, float* param, void* m_raw, void* v_raw, int lowp, int64_t n, int64_t n_prim,
                  const int32_t* vis, int step, double lr, double beta1, double beta2, double eps) {
  const int64_t feat = n_prim > 0 ? n / n_prim : 1;
  const double bc1 = 1.0 / (1.0 - pow(beta1, step));
  const double bc2 = 1.0 / sqrt(1.0 - pow(beta2, step));
  const float step_size = (float)(lr * bc1), b1 = (float)beta1, b2 = (float)beta2, e = (float)eps, c2 = (float)bc2;
  const uint32_t seed = 0x9E3779B9u * (uint32_t)step + 0x85EBCA6Bu;
  for (int64_t i = 0; i < n; ++i) {
    if (vis && vis[i / feat] == 0) continue;
    const float g = grad[i];
    float m, v;
    if (lowp) {
      m = bits_to_f((uint32_t)((const uint16_t*)m_raw)[i] << 16);
      v = bits_to_f((uint32_t)((const uint16_t*)v_raw)[i] << 16);
    } else {
      m = ((const float*)m_raw)[i];
      v = ((const float*)v_raw)[i];
    }
    const float gsq = g * g;
    m = fmaf(b1, m - g, g);
    v = fmaf(b2, v - gsq, gsq);
    const float denom = sqrtf(v) * c2 + e;
    param[i] = param[i] - (step_size * m) / denom;
    if (lowp) {
      const uint32_t r1 = or_sr_hash((uint32_t)i ^ seed), r2 = or_sr_hash(r1);
      ((uint16_t*)m_raw)[i] = or_bf16_sr(m, r1);
      ((uint16_t*)v_raw)[i] = or_bf16_sr(v, r2);
    } else {
      ((float*)m_raw)[i] = m;
      ((float*)v_raw)[i] = v;
    }
  }
}
