/*
 * tm_oracle.c -- CPU restatement of the optimizer-step arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP path is compared
 * against; it is never linked into, loaded by, or called from the product
 * (torchure_amd/). Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it.
 *
 * Built with -ffp-contract=off so that every rounding point is the one written
 * here. The fused multiply-adds are explicit fma() calls (C99, correctly rounded).
 *
 * What each function restates:
 *   orc_adamw_scalars  bias corrections and step size of torch's fused AdamW
 *                      functor, torch/include/ATen/native/hip/fused_adam_utils.cuh:128-139,
 *                      :71 (step_size = lr / float(bias_correction1)); the step is
 *                      incremented before the math (torch/optim/adam.py:877).
 *   orc_adamw_update   per-element AdamW (ADAMW mode, no amsgrad, no maximize),
 *                      fused_adam_utils.cuh:43-92 -- the same math the reference
 *                      calls through torch.optim.AdamW(fused=True)
 *                      (torchure/optimizer/builder.py:46).
 *   orc_bf16_rne       fp32 -> bf16 round-to-nearest-even, NaN -> 0x7FC0,
 *                      torch/include/torch/headeronly/util/BFloat16.h:100-114.
 *   orc_sumsq          brute-force fp64 sum of squares (the global norm of
 *                      torchure/core/grad_helper.py:17-18 is its square root).
 *   orc_clip_coef      clamp(max_norm / (total + 1e-6), max=1.0), grad_helper.py:32,
 *                      evaluated as reciprocal-then-multiply in fp32
 *                      (torch/_tensor.py:1119-1122).
 * The element loops carry OpenMP pragmas: the liborc_mt.so build splits them over
 * threads (same per-element results), liborc.so runs them serially.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_bf16_rne1(float f) {
  if (f != f) return 0x7FC0u;
  uint32_t u;
  memcpy(&u, &f, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

void orc_bf16_rne(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_bf16_rne1(src[i]);
}

void orc_bf16_to_f32(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = bf16_to_f32(src[i]);
}

/* step_after = step + 1 (fp32), then
 *   bc1 = 1 - beta1^step (double), bc2s = sqrt(1 - beta2^step) (double)
 *   out[0] = step_size = float(lr / double(float(bc1)))
 *   out[1] = float(bc2s)                                                   */
void orc_adamw_scalars(float step_after, double lr, double beta1, double beta2, float* out) {
  double bc1 = 1.0 - pow(beta1, (double)step_after);
  double bc2 = 1.0 - pow(beta2, (double)step_after);
  float bc1f = (float)bc1;
  out[0] = (float)(lr / (double)bc1f);
  out[1] = (float)sqrt(bc2);
}

static inline void adamw_elem(float* pp, float* mp, float* vp, float g, double neg_lrwd, int decay,
                              double beta1, double beta2, double eps, float step_size, float bc2s) {
  float p = *pp, m = *mp, v = *vp;
  if (decay) {
    double pd = (double)p;
    p = (float)fma(neg_lrwd, pd, pd);
  }
  double gd = (double)g;
  m = (float)fma(beta1, (double)m, (1.0 - beta1) * gd);
  v = (float)fma(beta2, (double)v, ((1.0 - beta2) * gd) * gd);
  float q = sqrtf(v) / bc2s;
  float denom = (float)((double)q + eps);
  p = p - (step_size * m) / denom;
  *pp = p;
  *mp = m;
  *vp = v;
}

/* In-place AdamW over n elements. g is the fp32 grad after any clip scaling.
 * step_after is the already-incremented step counter. */
void orc_adamw_update(float* p, float* m, float* v, const float* g, int64_t n, float step_after,
                      double lr, double beta1, double beta2, double weight_decay, double eps) {
  float sc[2];
  orc_adamw_scalars(step_after, lr, beta1, beta2, sc);
  const double neg_lrwd = -(lr * weight_decay);
  const int decay = weight_decay != 0.0;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    adamw_elem(p + i, m + i, v + i, g[i], neg_lrwd, decay, beta1, beta2, eps, sc[0], sc[1]);
}

/* Same update reading a bf16 grad and applying the clip coefficient in fp32
 * (g = float(bf16) * coef, one rounding, as torch._foreach_mul_ on fp32 grads),
 * optionally writing the bf16 working copy. Threaded with OpenMP when built so. */
void orc_adamw_update_bf16(float* p, float* m, float* v, const uint16_t* g, uint16_t* out_bf16,
                           int64_t n, float coef, int clip, float step_after, double lr,
                           double beta1, double beta2, double weight_decay, double eps) {
  float sc[2];
  orc_adamw_scalars(step_after, lr, beta1, beta2, sc);
  const double neg_lrwd = -(lr * weight_decay);
  const int decay = weight_decay != 0.0;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    float gi = bf16_to_f32(g[i]);
    if (clip) gi = gi * coef;
    adamw_elem(p + i, m + i, v + i, gi, neg_lrwd, decay, beta1, beta2, eps, sc[0], sc[1]);
    if (out_bf16) out_bf16[i] = orc_bf16_rne1(p[i]);
  }
}

double orc_sumsq_f32(const float* g, int64_t n) {
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) s += (double)g[i] * (double)g[i];
  return s;
}

double orc_sumsq_bf16(const uint16_t* g, int64_t n) {
  double s = 0.0;
#pragma omp parallel for reduction(+ : s) schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    double x = (double)bf16_to_f32(g[i]);
    s += x * x;
  }
  return s;
}

float orc_clip_coef(float total, float max_norm) {
  float t = total + 1e-6f;
  float r = 1.0f / t;
  float c = r * max_norm;
  return (c > 1.0f) ? 1.0f : c;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
