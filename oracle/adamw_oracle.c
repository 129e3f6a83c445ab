/*
 * adamw_oracle.c -- CPU restatement of the AdamW optimizer step and the global
 * gradient-norm clip, used ONLY as test infrastructure (the checker).
 *
 * Nothing in the product links or calls this file.  The pytest suite and the
 * smoke check load it through oracle.py.
 *
 * What it restates (torch 2.10.0+rocm7.0, the third-party code mini-megatron's
 * training loop calls; the reference itself contains no optimizer arithmetic):
 *   - torch/optim/adam.py:396-547  `_single_tensor_adam`, the path that
 *     mini-megatron's main.py:177 (AdamW(..., fused=False)) takes, as the
 *     per-element op chain of the 7 ATen kernels it launches per tensor:
 *       adam.py:419  p  = p * f32(1 - lr*wd)                       (mul_)
 *       adam.py:457  m  = lerp(m, g, f32(1 - beta1))                 (lerp_)
 *       adam.py:476  v  = v * f32(beta2); v = v + f32(1-beta2)*g*g   (mul_, addcmul_)
 *       adam.py:545  d  = sqrt(v) / bc2_sqrt; d = d + f32(eps)       (sqrt, div, add_)
 *       (amsgrad, adam.py:538-543: vmax = maximum(vmax, v), NaN-propagating,
 *        and d is computed from vmax instead of v)
 *       adam.py:547  p  = p + f32(-step_size) * (m / d)              (addcdiv_)
 *   - torch/optim/adam.py:480-527  the same loop with capturable=True: the step
 *     counts are device tensors and the per-step values are 0-d fp32 tensor ops,
 *       adam.py:488,497  bc1 = 1 - beta1**step, bc2 = 1 - beta2**step
 *       adam.py:499-502  step_size = lr / bc1, neg = -step_size, bc2_sqrt = sqrt(bc2)
 *       adam.py:520-522  d = sqrt(v) / (bc2_sqrt * neg) + eps / neg
 *       adam.py:527      p = p + m / d                                  (addcdiv_)
 *   - torch/optim/adam.py:803-895  the fused=True path (_fused_adam ->
 *     torch._fused_adamw_), per element adam_math of
 *     ATen/native/hip/fused_adam_utils.cuh: float64 scalars and moment sums, one
 *     rounding to fp32 each (see oracle_fused_scalars below).
 *   - torch/include/ATen/native/Lerp.h:21-35  the two-branch lerp formula.
 *   - torch/nn/utils/clip_grad.py:50-117,121-183  global L2 norm, then
 *     coef = clamp(max_norm * reciprocal(norm + 1e-6), max=1), g *= coef.
 *
 * Every ATen kernel rounds its result to fp32, so each step above is one fp32
 * rounding.  Whether the compiler that built a given torch binary contracted
 * `a + b*c` into one fused multiply-add, and whether division by a host scalar
 * runs as a true division or as a multiply by an fp32 reciprocal, differs
 * between torch's CPU and GPU builds.  Those choices are the fields of
 * `oracle_opmodel`; the tests pin one op model against torch on the CPU
 * (golden fixtures) and one against torch on the GPU (per-op probes).
 *
 * Build: gcc -O2 -ffp-contract=off (Makefile beside this file).  Contraction
 * must stay off so that every fused multiply-add here is an explicit fmaf().
 * Declarations: adamw_oracle.h.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "adamw_oracle.h"

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* fp32 -> bf16, round to nearest even; every NaN becomes 0x7FC0, the value
 * torch's Tensor.to(torch.bfloat16) produces for NaN. */
uint16_t oracle_f32_to_bf16(float x)
{
    uint32_t u = f2u(x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu))
        return (uint16_t)0x7fc0u;
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Lerp.h:21-35 with fp32 opmath. */
static inline float lerp_f32(float self, float end, float w, int use_fma)
{
    float diff = end - self;
    if (fabsf(w) < 0.5f)
        return use_fma ? fmaf(w, diff, self) : self + w * diff;
    float omw = 1.0f - w;
    return use_fma ? fmaf(-diff, omw, end) : end - diff * omw;
}

static inline float addcmul_f32(float v, float s, float g, int mode)
{
    switch (mode) {
    case 1: return fmaf(s, g * g, v);
    case 2: return fmaf(s * g, g, v);
    case 3: { float sg = s * g; float t = sg * g; return v + t; }
    default: { float gg = g * g; float t = s * gg; return v + t; }
    }
}

/* torch.maximum: NaN if either operand is NaN (a first), else the larger, a on
 * ties. */
static inline float maximum_nan(float a, float b)
{
    if (isnan(a)) return a;
    if (isnan(b)) return b;
    return a < b ? b : a;
}

/* The ops both chains share (adam.py:419-476, amsgrad's maximum at :538-540 or,
 * capturable, :510-512): p, m, v (and vmax with amsgrad, when non-NULL) updated
 * in place.  Returns the value whose square root the denominator takes. */
static inline float shared_ops(float *p, float g, float *m, float *v, float *vmax,
                               float wd_factor, float lerp_w, float beta2, float omb2,
                               const oracle_opmodel *om)
{
    float pp = *p * wd_factor;                              /* adam.py:419 */
    float mm = lerp_f32(*m, g, lerp_w, om->lerp_fma);       /* adam.py:457 */
    float vv = *v * beta2;                                  /* adam.py:476 */
    vv = addcmul_f32(vv, omb2, g, om->addcmul_mode);
    float dv = vv;
    if (vmax) {
        *vmax = maximum_nan(*vmax, vv);
        dv = *vmax;
    }
    *p = pp; *m = mm; *v = vv;
    return dv;
}

/* One element of the default chain. */
static inline void adamw_elem(float *p, float g, float *m, float *v, float *vmax,
                              const oracle_hyper *h, const oracle_opmodel *om,
                              float inv_bc2, float bc2f)
{
    float dv = shared_ops(p, g, m, v, vmax, h->wd_factor, h->lerp_w, h->beta2,
                          h->one_minus_beta2, om);
    float pp = *p, mm = *m;
    float d = sqrtf(dv);                                    /* adam.py:543,545 */
    d = om->div_recip ? d * inv_bc2 : d / bc2f;
    d = d + h->eps;
                                                            /* adam.py:547 */
    if (om->addcdiv_mode == 2) {
        float sm = h->neg_step_size * mm;
        pp = pp + sm / d;
    } else {
        float q = mm / d;
        pp = om->addcdiv_mode == 1 ? fmaf(h->neg_step_size, q, pp) : pp + h->neg_step_size * q;
    }
    *p = pp;
}

/* fp32 state: p, g, m, v (and vmax, or NULL without amsgrad) are n contiguous
 * floats.  grad_scale multiplies the gradient first (clip_grad.py:174,
 * g *= coef), then grad_sign applies `maximize` (adam.py:397). */
void oracle_adamw_f32(float *p, const float *g, float *m, float *v, float *vmax, int64_t n,
                      const oracle_hyper *h, const oracle_opmodel *om, float grad_scale,
                      int apply_scale)
{
    float bc2f = (float)h->bc2_sqrt;
    float inv_bc2 = (float)(1.0 / h->bc2_sqrt);
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (apply_scale) gi = gi * grad_scale;
        gi = gi * h->grad_sign;
        adamw_elem(&p[i], gi, &m[i], &v[i], vmax ? &vmax[i] : NULL, h, om, inv_bc2, bc2f);
    }
}

/* bf16 state variant: m, v (and vmax) are stored as bf16, widened to fp32,
 * updated with the same fp32 op chain, and stored back rounded to nearest even. */
void oracle_adamw_bf16state(float *p, const float *g, uint16_t *m, uint16_t *v,
                            uint16_t *vmax, int64_t n, const oracle_hyper *h,
                            const oracle_opmodel *om, float grad_scale, int apply_scale)
{
    float bc2f = (float)h->bc2_sqrt;
    float inv_bc2 = (float)(1.0 / h->bc2_sqrt);
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (apply_scale) gi = gi * grad_scale;
        gi = gi * h->grad_sign;
        float mm = oracle_bf16_to_f32(m[i]);
        float vv = oracle_bf16_to_f32(v[i]);
        float mx = vmax ? oracle_bf16_to_f32(vmax[i]) : 0.0f;
        adamw_elem(&p[i], gi, &mm, &vv, vmax ? &mx : NULL, h, om, inv_bc2, bc2f);
        m[i] = oracle_f32_to_bf16(mm);
        v[i] = oracle_f32_to_bf16(vv);
        if (vmax) vmax[i] = oracle_f32_to_bf16(mx);
    }
}

/* adam.py:480-502 in fp32, one rounding per 0-d tensor op.  A float lr reaches
 * `lr / bc1` as bc1.reciprocal() * lr (Tensor.__rtruediv__); a tensor lr as a
 * true division.  eps / neg is likewise reciprocal(neg) * eps.  powf is this C
 * library's; torch's device pow may differ from it in the last bit for some
 * steps, so bit-level comparisons with the GPU pass torch's own values. */
void oracle_capt_scalars(float beta1, float beta2, float lr, float eps, float step,
                         int lr_is_tensor, float *den_scale, float *den_add)
{
    float bc1 = 1.0f - powf(beta1, step);
    float bc2 = 1.0f - powf(beta2, step);
    float step_size = lr_is_tensor ? lr / bc1 : (1.0f / bc1) * lr;
    float neg = -step_size;
    float bc2_sqrt = sqrtf(bc2);
    *den_scale = bc2_sqrt * neg;
    *den_add = (1.0f / neg) * eps;
}

/* One element of the capturable chain (adam.py:419-527, capturable=True). */
static inline void adamw_capt_elem(float *p, float g, float *m, float *v, float *vmax,
                                   const oracle_capt *h, const oracle_opmodel *om)
{
    float dv = shared_ops(p, g, m, v, vmax, h->wd_factor, h->lerp_w, h->beta2,
                          h->one_minus_beta2, om);
    float d = sqrtf(dv);                                    /* adam.py:516-522 */
    d = d / h->den_scale;
    d = d + h->den_add;
    *p = *p + *m / d;                                       /* adam.py:527, value 1 */
}

void oracle_adamw_capt_f32(float *p, const float *g, float *m, float *v, float *vmax,
                           int64_t n, const oracle_capt *h, const oracle_opmodel *om,
                           float grad_scale, int apply_scale)
{
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (apply_scale) gi = gi * grad_scale;
        gi = gi * h->grad_sign;
        adamw_capt_elem(&p[i], gi, &m[i], &v[i], vmax ? &vmax[i] : NULL, h, om);
    }
}

void oracle_adamw_capt_bf16state(float *p, const float *g, uint16_t *m, uint16_t *v,
                                 uint16_t *vmax, int64_t n, const oracle_capt *h,
                                 const oracle_opmodel *om, float grad_scale, int apply_scale)
{
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (apply_scale) gi = gi * grad_scale;
        gi = gi * h->grad_sign;
        float mm = oracle_bf16_to_f32(m[i]);
        float vv = oracle_bf16_to_f32(v[i]);
        float mx = vmax ? oracle_bf16_to_f32(vmax[i]) : 0.0f;
        adamw_capt_elem(&p[i], gi, &mm, &vv, vmax ? &mx : NULL, h, om);
        m[i] = oracle_f32_to_bf16(mm);
        v[i] = oracle_f32_to_bf16(vv);
        if (vmax) vmax[i] = oracle_f32_to_bf16(mx);
    }
}

/* torch's fused=True chain: torch.optim.AdamW(fused=True) -> adam.py:803-895
 * (_fused_adam: step counts += 1 on the device, then torch._fused_adamw_), whose
 * per-element math is adam_math in ATen/native/hip/fused_adam_utils.cuh (ADAMW
 * mode).  lr, the betas, weight decay and eps stay float64 there, so m, v and the
 * decayed p are formed in float64 from the fp32 values and rounded once to fp32:
 *   p  = f32(p - (lr*wd) * p)                       (only when wd != 0)
 *   m  = f32(beta1*m + (1-beta1)*g)
 *   v  = f32(beta2*v + ((1-beta2)*g)*g)
 *   d  = f32((double)(sqrtf(v) / bc2_sqrt) + eps)   (amsgrad: from max(vmax, v))
 *   p  = p - (step_size * m) / d                    (fp32 ops)
 * The per-step values are float64 on the device and reach adam_math as fp32:
 *   bc1 = f32(1 - pow(beta1, step)), bc2_sqrt = f32(sqrt(1 - pow(beta2, step))),
 *   step_size = f32(lr / (double)bc1).
 * Which float64 `a*b + c*d` torch-ROCm's compiler contracted into one fused
 * multiply-add is the model's choice (oracle_fused_model); the pinned model is the
 * one torch's own GPU results select on inputs where the candidates round apart. */
void oracle_fused_scalars(double lr, double beta1, double beta2, float step, float *bc1,
                          float *bc2_sqrt, float *step_size)
{
    double b1c = 1.0 - pow(beta1, (double)step);
    double b2c = 1.0 - pow(beta2, (double)step);
    *bc1 = (float)b1c;
    *bc2_sqrt = (float)sqrt(b2c);
    *step_size = (float)(lr / (double)*bc1);
}

/* oracle_fused_scalars' bc1 and bc2_sqrt for n step counts (beta1 for bc1, beta2 for
 * bc2_sqrt). */
void oracle_fused_scalars_many(double beta1, double beta2, const float *steps, int64_t n,
                               float *bc1, float *bc2_sqrt)
{
    for (int64_t i = 0; i < n; ++i) {
        float ss;
        oracle_fused_scalars(1.0, beta1, beta2, steps[i], &bc1[i], &bc2_sqrt[i], &ss);
    }
}

static inline void fused_elem(float *p, float g, float *m, float *v, float *vmax,
                              const oracle_fused *h, const oracle_fused_model *fm)
{
    const double omb1 = 1.0 - h->beta1, omb2 = 1.0 - h->beta2;
    float pp = *p;
    if (h->weight_decay != 0.0) {
        const double t = h->lr * h->weight_decay;
        pp = fm->wd_fma ? (float)fma(-t, (double)pp, (double)pp)
                        : (float)((double)pp - t * (double)pp);
    }
    const double dm = (double)*m, dg = (double)g, dvv = (double)*v;
    float mm, vv;
    switch (fm->m_mode) {
    case 1: mm = (float)fma(h->beta1, dm, omb1 * dg); break;
    case 2: mm = (float)fma(omb1, dg, h->beta1 * dm); break;
    default: mm = (float)(h->beta1 * dm + omb1 * dg); break;
    }
    const double q = omb2 * dg;
    switch (fm->v_mode) {
    case 1: vv = (float)fma(h->beta2, dvv, q * dg); break;
    case 2: vv = (float)fma(q, dg, h->beta2 * dvv); break;
    default: vv = (float)(h->beta2 * dvv + q * dg); break;
    }
    /* amsgrad: ::max on the device is fmaxf (the number if one operand is NaN) */
    const float dv = vmax ? (*vmax = fmaxf(*vmax, vv)) : vv;
    const float d = (float)((double)(sqrtf(dv) / h->bc2_sqrt) + h->eps);
    pp = pp - (h->step_size * mm) / d;
    *p = pp; *m = mm; *v = vv;
}

void oracle_adamw_fused_f32(float *p, const float *g, float *m, float *v, float *vmax,
                            int64_t n, const oracle_fused *h, const oracle_fused_model *fm,
                            float grad_scale, int apply_scale)
{
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (apply_scale) gi = gi * grad_scale;
        gi = gi * h->grad_sign;
        fused_elem(&p[i], gi, &m[i], &v[i], vmax ? &vmax[i] : NULL, h, fm);
    }
}

void oracle_adamw_fused_bf16state(float *p, const float *g, uint16_t *m, uint16_t *v,
                                  uint16_t *vmax, int64_t n, const oracle_fused *h,
                                  const oracle_fused_model *fm, float grad_scale,
                                  int apply_scale)
{
    for (int64_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (apply_scale) gi = gi * grad_scale;
        gi = gi * h->grad_sign;
        float mm = oracle_bf16_to_f32(m[i]);
        float vv = oracle_bf16_to_f32(v[i]);
        float mx = vmax ? oracle_bf16_to_f32(vmax[i]) : 0.0f;
        fused_elem(&p[i], gi, &mm, &vv, vmax ? &mx : NULL, h, fm);
        m[i] = oracle_f32_to_bf16(mm);
        v[i] = oracle_f32_to_bf16(vv);
        if (vmax) vmax[i] = oracle_f32_to_bf16(mx);
    }
}

void oracle_to_bf16(const float *x, uint16_t *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(x[i]);
}

/* Sum of squares in float64.  Each square of an fp32 value is exact in
 * float64; blocks of 4096 are summed first so the rounding error stays far
 * below fp32 resolution even for 1e10 terms. */
double oracle_sumsq_f64(const float *g, int64_t n)
{
    double total = 0.0;
    for (int64_t b = 0; b < n; b += 4096) {
        int64_t e = b + 4096 < n ? b + 4096 : n;
        double s = 0.0;
        for (int64_t i = b; i < e; ++i) { double x = (double)g[i]; s += x * x; }
        total += s;
    }
    return total;
}

/* clip_grad.py:165-169 on a 0-d fp32 tensor `norm`:
 *   t = norm + f32(1e-6); r = 1/t (Tensor.__rtruediv__ = reciprocal * other);
 *   coef = r * f32(max_norm); clamp(max=1.0) keeps NaN. */
float oracle_clip_coef(float total_norm, double max_norm)
{
    float t = total_norm + (float)1e-6;
    float r = 1.0f / t;
    float c = r * (float)max_norm;
    return (c > 1.0f) ? 1.0f : c;
}

/* ulp distance between two fp32 arrays, as the number of representable floats
 * between them (sign-magnitude mapped to a monotone integer line).  NaN vs NaN
 * counts as 0, NaN vs number as INT64_MAX. */
int64_t oracle_max_ulp(const float *a, const float *b, int64_t n, int64_t *argmax)
{
    int64_t worst = 0, where = -1;
    for (int64_t i = 0; i < n; ++i) {
        int an = isnan(a[i]), bn = isnan(b[i]);
        int64_t d;
        if (an || bn) d = (an && bn) ? 0 : INT64_MAX;
        else {
            int32_t ia = (int32_t)f2u(a[i]), ib = (int32_t)f2u(b[i]);
            int64_t la = ia < 0 ? (int64_t)INT32_MIN - ia : ia;
            int64_t lb = ib < 0 ? (int64_t)INT32_MIN - ib : ib;
            d = la > lb ? la - lb : lb - la;
        }
        if (d > worst) { worst = d; where = i; }
    }
    if (argmax) *argmax = where;
    return worst;
}
