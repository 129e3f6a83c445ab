/*
 * adamw_oracle.h -- declarations of the CPU oracle (adamw_oracle.c), test
 * infrastructure only: the Python tests bind it through oracle.py, the C ABI
 * test (tests/c/abi_check.c) links it directly.  Nothing in the product
 * includes this header.
 */
#ifndef ADAMW_ORACLE_H
#define ADAMW_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct oracle_opmodel {
    int lerp_fma;     /* 1: self + w*(end-self) evaluated as fmaf(w, end-self, self)    */
    int addcmul_mode; /* v + s*g*g:  0 = v + (s*(g*g)) rounded per op,
                                      1 = fmaf(s, g*g, v),
                                      2 = fmaf(s*g, g, v),
                                      3 = v + ((s*g)*g) rounded per op               */
    int addcdiv_mode; /* p + s*m/d:  0 = p + (s*(m/d)) rounded per op,
                                      1 = fmaf(s, m/d, p),
                                      2 = p + ((s*m)/d) rounded per op               */
    int div_recip;    /* 1: x / c evaluated as x * f32(1.0 / c), the reciprocal taken
                            in float64 on the host (host scalar c); 0: x / f32(c)      */
} oracle_opmodel;

/* Host scalars of one AdamW step, already reduced the way adam.py:414-536 and
 * ATen's scalar handling reduce them (float64 on the host, then cast to fp32). */
typedef struct oracle_hyper {
    float wd_factor;       /* f32(1 - lr*wd); 1.0f when weight_decay == 0 (adam.py:417-419) */
    float lerp_w;          /* f32(1 - beta1)                         (adam.py:457)          */
    float beta2;           /* f32(beta2)                             (adam.py:476)          */
    float one_minus_beta2; /* f32(1 - beta2)                         (adam.py:476)          */
    double bc2_sqrt;       /* (1 - beta2**step) ** 0.5 in float64    (adam.py:532,536)      */
    float eps;             /* f32(eps)                               (adam.py:545)          */
    float neg_step_size;   /* f32(-(lr / (1 - beta1**step)))         (adam.py:534,547)      */
    float grad_sign;       /* -1.0f when maximize (adam.py:397), else 1.0f                  */
} oracle_hyper;

/* Scalars of the capturable chain (adam.py:480-527, capturable=True): the
 * first four and grad_sign as in oracle_hyper; the two per-step values are
 * fp32 results of 0-d tensor ops (oracle_capt_scalars, or torch's own). */
typedef struct oracle_capt {
    float wd_factor;
    float lerp_w;
    float beta2;
    float one_minus_beta2;
    float den_scale;       /* sqrt(bc2) * -step_size                (adam.py:521)          */
    float den_add;         /* eps / -step_size                      (adam.py:522)          */
    float grad_sign;
} oracle_capt;

/* torch's fused=True chain (ATen/native/hip/fused_adam_utils.cuh adam_math): which
 * float64 `a*b + c*d` forms one fused multiply-add. */
typedef struct oracle_fused_model {
    int wd_fma;       /* 1: p - (lr*wd)*p as fma(-(lr*wd), p, p); 0: two roundings       */
    int m_mode;       /* beta1*m + (1-beta1)*g: 0 = no fma, 1 = fma(beta1, m, (1-beta1)*g),
                                                2 = fma(1-beta1, g, beta1*m)            */
    int v_mode;       /* beta2*v + ((1-beta2)*g)*g: 0 = no fma, 1 = fma(beta2, v, .),
                                                2 = fma((1-beta2)*g, g, beta2*v)        */
} oracle_fused_model;

/* Scalars of the fused chain: the float64 hyperparameters as _fused_adamw_ receives
 * them and the per-step values it forms (oracle_fused_scalars). */
typedef struct oracle_fused {
    double lr;
    double beta1;
    double beta2;
    double weight_decay;
    double eps;
    float step_size;       /* f32(lr / (double)bc1)                                      */
    float bc2_sqrt;        /* f32(sqrt(1 - pow(beta2, step)))                           */
    float grad_sign;       /* -1.0f when maximize, else 1.0f                             */
} oracle_fused;

uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t h);

/* fp32 state: p, g, m, v (and vmax, or NULL without amsgrad) are n contiguous
 * floats, updated in place; grad_scale multiplies g first when apply_scale. */
void oracle_adamw_f32(float *p, const float *g, float *m, float *v, float *vmax, int64_t n,
                      const oracle_hyper *h, const oracle_opmodel *om, float grad_scale,
                      int apply_scale);

/* bf16-stored moments (bit patterns), fp32 math, stores rounded to nearest even. */
void oracle_adamw_bf16state(float *p, const float *g, uint16_t *m, uint16_t *v,
                            uint16_t *vmax, int64_t n, const oracle_hyper *h,
                            const oracle_opmodel *om, float grad_scale, int apply_scale);

/* adam.py:480-502: den_scale and den_add of step `step` in fp32 (libm powf). */
void oracle_capt_scalars(float beta1, float beta2, float lr, float eps, float step,
                         int lr_is_tensor, float *den_scale, float *den_add);

/* The capturable chain: d = sqrt(v) / den_scale + den_add, p = p + m / d. */
void oracle_adamw_capt_f32(float *p, const float *g, float *m, float *v, float *vmax,
                           int64_t n, const oracle_capt *h, const oracle_opmodel *om,
                           float grad_scale, int apply_scale);
void oracle_adamw_capt_bf16state(float *p, const float *g, uint16_t *m, uint16_t *v,
                                 uint16_t *vmax, int64_t n, const oracle_capt *h,
                                 const oracle_opmodel *om, float grad_scale, int apply_scale);

/* The fused=True chain's per-step values (libm pow in float64). */
void oracle_fused_scalars(double lr, double beta1, double beta2, float step, float *bc1,
                          float *bc2_sqrt, float *step_size);

/* bc1 and bc2_sqrt of oracle_fused_scalars for n step counts. */
void oracle_fused_scalars_many(double beta1, double beta2, const float *steps, int64_t n,
                               float *bc1, float *bc2_sqrt);

/* torch's fused=True chain, fp32 and bf16-stored moments. */
void oracle_adamw_fused_f32(float *p, const float *g, float *m, float *v, float *vmax,
                            int64_t n, const oracle_fused *h, const oracle_fused_model *fm,
                            float grad_scale, int apply_scale);
void oracle_adamw_fused_bf16state(float *p, const float *g, uint16_t *m, uint16_t *v,
                                  uint16_t *vmax, int64_t n, const oracle_fused *h,
                                  const oracle_fused_model *fm, float grad_scale,
                                  int apply_scale);

void oracle_to_bf16(const float *x, uint16_t *out, int64_t n);

/* Sum of squares in float64 (per 4096-element block, then across blocks). */
double oracle_sumsq_f64(const float *g, int64_t n);

/* clip_grad.py:165-169: min(max_norm * (1 / (norm + 1e-6)), 1) in fp32, NaN kept. */
float oracle_clip_coef(float total_norm, double max_norm);

/* Largest ulp distance between two fp32 arrays (NaN vs NaN counts 0). */
int64_t oracle_max_ulp(const float *a, const float *b, int64_t n, int64_t *argmax);

#ifdef __cplusplus
}
#endif

#endif /* ADAMW_ORACLE_H */
