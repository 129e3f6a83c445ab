/*
 * abi_check.c -- libmi_adamw's C ABI (include/mi_adamw.h) driven from plain C:
 * no Python, no torch, only the HIP runtime API for device memory.  It shows
 * that the boundary works for any host that can call C, the way a cgo / JNI /
 * N-API binding would call it.
 *
 *   abi_check cpu   host-side checks only, no device needed: version, error
 *                   text, the chunk-table helper, and argument rejections that
 *                   return before any launch.
 *   abi_check gpu   parity on the device against the CPU oracle
 *                   (oracle/adamw_oracle.h, test infrastructure):
 *                   - flat range, fp32 state, fused clip: norm within 1e-6,
 *                     coefficient and p, m, v bit-exact;
 *                   - tensor/chunk tables, three tensors, two hyperparameter
 *                     sets, bf16 moments and bf16 model copy: bit-exact;
 *                   - flat range with amsgrad: p, m, v, max_exp_avg_sq bit-exact;
 *                   - capturable chain through tables: two tensors at different
 *                     device step counts, a float lr, then a device lr: bit-exact;
 *                   - torch's fused=True chain: a flat range with the clip, then
 *                     tables with two sets (one without weight decay, with
 *                     maximize), then tables at device step counts with a device
 *                     lr: bit-exact.
 *
 * The per-step scalars are computed here as the header documents (float64 on
 * the host, as torch/optim/adam.py:529-536 does, then cast to fp32), with
 * floating-point contraction off so that no step fuses.
 * Exit status 0 on success; the first failed check prints and exits 1.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "adamw_oracle.h"
#include "mi_adamw.h"

#define CHECK(cond, ...)                                                      \
    do {                                                                      \
        if (!(cond)) {                                                        \
            fprintf(stderr, "abi_check: FAILED %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                                     \
            fprintf(stderr, "\n");                                            \
            exit(1);                                                          \
        }                                                                     \
    } while (0)
#define HIP(x) CHECK((x) == hipSuccess, "%s", #x)

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static float urand(void) /* uniform in [-1, 1) */
{
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (float)((double)(rng_state >> 11) * (2.0 / 9007199254740992.0) - 1.0);
}

static const oracle_opmodel ROCM_OPS = {1, 1, 1, 1};

/* One (group, step) of AdamW, for the library and for the oracle. */
static void scalars(double lr, double b1, double b2, double eps, double wd, double step,
                    int maximize, mi_adamw_hyper *h, oracle_hyper *o)
{
    const double bc1 = 1.0 - pow(b1, step);
    const double bc2 = 1.0 - pow(b2, step);
    const double bc2_sqrt = pow(bc2, 0.5);
    h->wd_factor = wd != 0.0 ? (float)(1.0 - lr * wd) : 1.0f;
    h->lerp_w = (float)(1.0 - b1);
    h->beta2 = (float)b2;
    h->one_minus_beta2 = (float)(1.0 - b2);
    h->inv_bc2_sqrt = (float)(1.0 / bc2_sqrt);
    h->eps = (float)eps;
    h->neg_step_size = (float)(-(lr / bc1));
    h->grad_sign = maximize ? -1.0f : 1.0f;
    o->wd_factor = h->wd_factor;
    o->lerp_w = h->lerp_w;
    o->beta2 = h->beta2;
    o->one_minus_beta2 = h->one_minus_beta2;
    o->bc2_sqrt = bc2_sqrt;
    o->eps = h->eps;
    o->neg_step_size = h->neg_step_size;
    o->grad_sign = h->grad_sign;
}

static void fill(float *x, int64_t n, float scale, int absolute)
{
    for (int64_t i = 0; i < n; ++i) {
        float u = urand() * scale;
        x[i] = absolute ? fabsf(u) : u;
    }
}

static void *dev_copy(const void *host, size_t bytes)
{
    void *d = NULL;
    HIP(hipMalloc(&d, bytes));
    HIP(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
    return d;
}

static void back(void *host, const void *dev, size_t bytes)
{
    HIP(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
}

static void same_f32(const float *a, const float *b, int64_t n, const char *what)
{
    int64_t where = -1;
    const int64_t ulp = oracle_max_ulp(a, b, n, &where);
    CHECK(ulp == 0, "%s differs from the oracle by %lld ulp at %lld", what, (long long)ulp,
          (long long)where);
}

static void same_u16(const uint16_t *a, const uint16_t *b, int64_t n, const char *what)
{
    for (int64_t i = 0; i < n; ++i)
        CHECK(a[i] == b[i], "%s differs from the oracle at %lld: %04x vs %04x", what,
              (long long)i, a[i], b[i]);
}

/* ------------------------------------------------------------------ CPU */

static int cpu_checks(void)
{
    char want[32];
    snprintf(want, sizeof want, "mi_adamw %d gfx950", MI_ADAMW_ABI_VERSION);
    CHECK(strncmp(mi_adamw_version(), want, strlen(want)) == 0, "version %s", mi_adamw_version());
    CHECK(strstr(mi_adamw_strerror(MI_ADAMW_E_INVALID), "invalid") != NULL, "strerror");

    const int64_t numels[5] = {0, 1, 4096, 4097, 3 * 4096 - 5};
    const int64_t n = mi_adamw_build_chunks(numels, 5, 4096, NULL, 0);
    CHECK(n == 7, "chunk count %lld", (long long)n);
    mi_adamw_chunk chunks[7];
    CHECK(mi_adamw_build_chunks(numels, 5, 4096, chunks, 7) == 7, "chunk fill");
    const int32_t want_rows[7][2] = {{1, 0}, {2, 0}, {3, 0}, {3, 1}, {4, 0}, {4, 1}, {4, 2}};
    for (int i = 0; i < 7; ++i)
        CHECK(chunks[i].tensor == want_rows[i][0] && chunks[i].index == want_rows[i][1],
              "chunk %d", i);
    CHECK(mi_adamw_build_chunks(numels, 5, 1000, NULL, 0) == MI_ADAMW_E_INVALID, "chunk size");
    CHECK(mi_adamw_build_chunks(numels, 5, 4096, chunks, 6) == MI_ADAMW_E_INVALID, "capacity");

    /* Every call below is refused on the host before anything is launched. */
    mi_adamw_hyper h[1];
    memset(h, 0, sizeof h);
    const void *fake = (const void *)(uintptr_t)4096;
    CHECK(mi_adamw_step(NULL, NULL, 1, 4096, h, 1, NULL, 0, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "null tables");
    CHECK(mi_adamw_step(fake, fake, 1, 4096, h, MI_ADAMW_MAX_HYPER + 1, NULL, 0, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "too many hyper sets");
    CHECK(mi_adamw_step(fake, fake, 1, 1000, h, 1, NULL, 0, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "chunk size");
    CHECK(mi_adamw_step(fake, fake, 1, 4096, h, 1, NULL, 0, MI_ADAMW_F_CLIP, 0, NULL) ==
              MI_ADAMW_E_INVALID, "clip without a scale");
    mi_adamw_tensor t;
    memset(&t, 0, sizeof t);
    t.param = (float *)(uintptr_t)4096;
    t.grad = (float *)(uintptr_t)(8192 + 4); /* flagged aligned, but not 16-byte aligned */
    t.exp_avg = (void *)(uintptr_t)12288;
    t.exp_avg_sq = (void *)(uintptr_t)16384;
    t.numel = 10;
    t.flags = MI_ADAMW_T_VEC;
    CHECK(mi_adamw_step_flat(&t, h, NULL, 4096, MI_ADAMW_STATE_F32, 0, 0, NULL) ==
              MI_ADAMW_E_ALIGN, "misaligned flat range");
    t.grad = (float *)(uintptr_t)8192;
    CHECK(mi_adamw_step_flat(&t, h, NULL, 4096, MI_ADAMW_STATE_F32, MI_ADAMW_F_AMSGRAD, 0,
                             NULL) == MI_ADAMW_E_INVALID, "amsgrad without max_exp_avg_sq");
    CHECK(mi_adamw_grad_norm_flat(NULL, 10, 4096, 1.0f, NULL, NULL, NULL, NULL) ==
              MI_ADAMW_E_INVALID, "null gradient");
    mi_adamw_capt_hyper ch;
    memset(&ch, 0, sizeof ch);
    CHECK(mi_adamw_step_capturable(fake, fake, 1, 4096, &ch, 1, NULL, fake, NULL, 0, 0, 0,
                                   NULL) == MI_ADAMW_E_INVALID, "capturable without steps");
    ch.lr_mode = 7;
    CHECK(mi_adamw_step_capturable(fake, fake, 1, 4096, &ch, 1, fake, fake, NULL, 0, 0, 0,
                                   NULL) == MI_ADAMW_E_INVALID, "unknown lr mode");
    ch.lr_mode = MI_ADAMW_LR_DEVICE;
    CHECK(mi_adamw_step_capturable(fake, fake, 1, 4096, &ch, 1, fake, fake, NULL, 0, 0, 0,
                                   NULL) == MI_ADAMW_E_INVALID, "device lr without a pointer");
    ch.lr_mode = MI_ADAMW_LR_FLOAT;
    CHECK(mi_adamw_step_capturable_rows(fake, 1, fake, 1, 4096, &ch, 1, fake, fake, NULL, NULL,
                                        0, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "capturable rows without row scalars");
    CHECK(mi_adamw_step_capturable_rows(fake, 1, fake, 1, 4096, &ch, 1, fake, fake,
                                        (void *)(uintptr_t)8, NULL, 0, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "misaligned row scalars");
    CHECK(mi_adamw_step_capturable_rows(fake, 0, fake, 1, 4096, &ch, 1, fake, fake,
                                        (void *)(uintptr_t)4096, NULL, 0, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "capturable rows with no rows");
    CHECK(mi_adamw_widen_bf16(NULL, fake, 1, 4096, NULL) == MI_ADAMW_E_INVALID,
          "widen without tensors");
    CHECK(mi_adamw_widen_bf16(fake, fake, 0, 4096, NULL) == MI_ADAMW_E_INVALID,
          "widen with no chunks");
    CHECK(mi_adamw_widen_bf16(fake, fake, 1, 1000, NULL) == MI_ADAMW_E_INVALID,
          "widen chunk size");
    CHECK(mi_adamw_probe(NULL, fake, 1, 4096, MI_ADAMW_STATE_F32, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "probe without tensors");
    CHECK(mi_adamw_probe(fake, fake, 1, 4096, 7, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "probe state dtype");
    CHECK(mi_adamw_probe(fake, fake, 1, 4096, MI_ADAMW_STATE_F32, 1 << 9, 0, NULL) ==
              MI_ADAMW_E_INVALID, "probe unknown flag");
    CHECK(mi_adamw_probe_flat(NULL, 4096, MI_ADAMW_STATE_F32, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "flat probe without a range");
    CHECK(mi_adamw_probe_flat(&t, 1000, MI_ADAMW_STATE_F32, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "flat probe chunk size");
    /* the clip split at the all-reduce, the pre-scaled steps, the gradient patch, the no-alloc
       norm: argument checks */
    double *fake_d = (double *)(uintptr_t)4096;
    float *fake_f = (float *)(uintptr_t)4096;
    CHECK(mi_adamw_grad_sumsq_flat(NULL, 10, 4096, 1.0f, fake_d, fake_d, NULL) ==
              MI_ADAMW_E_INVALID, "sumsq without a gradient");
    CHECK(mi_adamw_grad_sumsq_flat(fake_f, 0, 4096, 1.0f, fake_d, fake_d, NULL) ==
              MI_ADAMW_E_INVALID, "sumsq of nothing");
    CHECK(mi_adamw_grad_sumsq_flat(fake_f, 10, 4096, INFINITY, fake_d, fake_d, NULL) ==
              MI_ADAMW_E_INVALID, "sumsq with a non-finite pre-scale");
    CHECK(mi_adamw_grad_sumsq(NULL, fake, 1, 4096, 1.0f, fake_d, fake_d, NULL) ==
              MI_ADAMW_E_INVALID, "sumsq without tables");
    CHECK(mi_adamw_norm_from_sumsq(NULL, 1, 1.0f, fake_f, fake_f, NULL) == MI_ADAMW_E_INVALID,
          "finalize without sums");
    CHECK(mi_adamw_norm_from_sumsq(fake_d, 0, 1.0f, fake_f, fake_f, NULL) == MI_ADAMW_E_INVALID,
          "finalize of no sums");
    CHECK(mi_adamw_norm_from_sumsq(fake_d, MI_ADAMW_MAX_NORM_BLOCKS + 1, 1.0f, fake_f, fake_f,
                                   NULL) == MI_ADAMW_E_INVALID, "finalize of too many sums");
    CHECK(mi_adamw_step_flat_prescaled(&t, h, NULL, NAN, 4096, MI_ADAMW_STATE_F32, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "flat step with a NaN pre-scale");
    CHECK(mi_adamw_step_prescaled(fake, fake, 1, 4096, h, 1, NULL, INFINITY, 0, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "table step with an infinite pre-scale");
    const int32_t bad_row[1] = {2};
    const uint64_t some_grad[1] = {4096};
    const uint8_t vec0[1] = {0};
    CHECK(mi_adamw_set_grads((mi_adamw_tensor *)fake, 2, 1, bad_row, some_grad, vec0, NULL) ==
              MI_ADAMW_E_INVALID, "gradient patch of a row outside the table");
    CHECK(mi_adamw_set_grads(NULL, 2, 1, bad_row, some_grad, vec0, NULL) == MI_ADAMW_E_INVALID,
          "gradient patch without a table");
    const int32_t twice[3] = {0, 1, 0};
    const uint64_t three_grads[3] = {4096, 8192, 12288};
    const uint8_t vec3[3] = {1, 1, 0};
    CHECK(mi_adamw_set_grads((mi_adamw_tensor *)fake, 2, 3, twice, three_grads, vec3, NULL) ==
              MI_ADAMW_E_INVALID, "gradient patch naming one row twice");
    CHECK(mi_adamw_grad_norm_flat_noalloc(NULL, 10, 4096, 1.0f, fake_f, fake_f, NULL) ==
              MI_ADAMW_E_INVALID, "no-alloc norm without a gradient");
    CHECK(strstr(mi_adamw_strerror(MI_ADAMW_E_SCRATCH), "scratch") != NULL, "scratch error text");
    mi_adamw_fused_hyper fh[1];
    memset(fh, 0, sizeof fh);
    CHECK(mi_adamw_step_fused_chain(NULL, fake, 1, 4096, fh, 1, NULL, NULL, NULL, 1.0f, 0, 0, 0,
                                    NULL) == MI_ADAMW_E_INVALID, "fused chain without tables");
    CHECK(mi_adamw_step_fused_chain(fake, fake, 1, 4096, fh, MI_ADAMW_MAX_HYPER + 1, NULL, NULL,
                                    NULL, 1.0f, 0, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "fused chain with too many sets");
    CHECK(mi_adamw_step_fused_chain(fake, fake, 1, 4096, fh, 1, fake_f, NULL, NULL, 1.0f, 0, 0, 0,
                                    NULL) == MI_ADAMW_E_INVALID,
          "fused chain with device steps but no step index");
    CHECK(mi_adamw_step_fused_chain(fake, fake, 1, 4096, fh, 1, NULL, NULL, NULL, NAN, 0, 0, 0,
                                    NULL) == MI_ADAMW_E_INVALID, "fused chain with a NaN pre-scale");
    CHECK(mi_adamw_step_fused_chain(fake, fake, 1, 4096, fh, 1, NULL, NULL, NULL, 1.0f, 0,
                                    MI_ADAMW_F_CLIP, 0, NULL) == MI_ADAMW_E_INVALID,
          "fused chain clip without a scale");
    CHECK(mi_adamw_step_fused_chain_rows(fake, 1, fake, 1, 4096, fh, 1, NULL, NULL,
                                         (void *)(uintptr_t)4096, NULL, 1.0f, 0, 0, 0, NULL) ==
              MI_ADAMW_E_INVALID, "fused chain rows without device steps");
    CHECK(mi_adamw_step_fused_chain_rows(fake, 1, fake, 1, 4096, fh, 1, fake_f, fake, NULL, NULL,
                                         1.0f, 0, 0, 0, NULL) == MI_ADAMW_E_INVALID,
          "fused chain rows without row scalars");
    t.grad = (float *)(uintptr_t)(8192 + 4);
    CHECK(mi_adamw_step_flat_fused_chain(&t, fh, NULL, 1.0f, 4096, MI_ADAMW_STATE_F32, 0, 0,
                                         NULL) == MI_ADAMW_E_ALIGN, "misaligned fused flat range");
    CHECK(mi_adamw_step_flat_fused_chain(&t, NULL, NULL, 1.0f, 4096, MI_ADAMW_STATE_F32, 0, 0,
                                         NULL) == MI_ADAMW_E_INVALID, "fused flat without a set");
    printf("abi_check cpu: ok (%s)\n", mi_adamw_version());
    return 0;
}

/* ------------------------------------------------------------------ GPU */

/* Flat range, fp32 state, fused clip (optionally amsgrad). */
static void flat_case(int64_t n, int amsgrad)
{
    const size_t fb = (size_t)n * sizeof(float);
    float *p = malloc(fb), *g = malloc(fb), *m = malloc(fb), *v = malloc(fb), *x = malloc(fb);
    float *pr = malloc(fb), *mr = malloc(fb), *vr = malloc(fb), *xr = malloc(fb);
    CHECK(p && g && m && v && x && pr && mr && vr && xr, "host allocation");
    fill(p, n, 0.02f, 0);
    fill(g, n, 1e-2f, 0); /* norm ~ 1e-2 sqrt(n/3) >> 1: the clip scales */
    fill(m, n, 1e-3f, 0);
    fill(v, n, 1e-6f, 1);
    fill(x, n, 2e-6f, 1); /* running maximum above v on part of the elements */
    memcpy(pr, p, fb);
    memcpy(mr, m, fb);
    memcpy(vr, v, fb);
    memcpy(xr, x, fb);

    float *dp = dev_copy(p, fb), *dg = dev_copy(g, fb), *dm = dev_copy(m, fb);
    float *dv = dev_copy(v, fb), *dx = amsgrad ? dev_copy(x, fb) : NULL;
    double *dpart = NULL;
    float *dnorm = NULL, *dcoef = NULL;
    HIP(hipMalloc((void **)&dpart, MI_ADAMW_MAX_NORM_BLOCKS * sizeof(double)));
    HIP(hipMalloc((void **)&dnorm, sizeof(float)));
    HIP(hipMalloc((void **)&dcoef, sizeof(float)));

    mi_adamw_hyper h;
    oracle_hyper oh;
    scalars(3e-4, 0.9, 0.95, 1e-8, 0.1, 1001.0, 0, &h, &oh);
    int rc = mi_adamw_grad_norm_flat(dg, n, 4096, 1.0f, dpart, dnorm, dcoef, NULL);
    CHECK(rc == 0, "mi_adamw_grad_norm_flat: %s", mi_adamw_strerror(rc));
    mi_adamw_tensor t;
    memset(&t, 0, sizeof t);
    t.param = dp;
    t.grad = dg;
    t.exp_avg = dm;
    t.exp_avg_sq = dv;
    t.max_exp_avg_sq = dx;
    t.numel = n;
    t.flags = MI_ADAMW_T_VEC; /* hipMalloc pointers are 256-byte aligned */
    const int32_t flags = MI_ADAMW_F_CLIP | (amsgrad ? MI_ADAMW_F_AMSGRAD : 0);
    rc = mi_adamw_step_flat(&t, &h, dcoef, 4096, MI_ADAMW_STATE_F32, flags, 0, NULL);
    CHECK(rc == 0, "mi_adamw_step_flat: %s", mi_adamw_strerror(rc));
    HIP(hipDeviceSynchronize());

    float norm, coef;
    back(&norm, dnorm, sizeof norm);
    back(&coef, dcoef, sizeof coef);
    const double ref = sqrt(oracle_sumsq_f64(g, n));
    CHECK(fabs((double)norm - ref) <= 1e-6 * ref, "norm %.9g vs %.9g", norm, ref);
    const float coef_ref = oracle_clip_coef(norm, 1.0);
    CHECK(memcmp(&coef, &coef_ref, sizeof coef) == 0 && coef < 1.0f, "coef %.9g vs %.9g", coef,
          coef_ref);
    oracle_adamw_f32(pr, g, mr, vr, amsgrad ? xr : NULL, n, &oh, &ROCM_OPS, coef, 1);
    back(p, dp, fb);
    back(m, dm, fb);
    back(v, dv, fb);
    same_f32(p, pr, n, "param");
    same_f32(m, mr, n, "exp_avg");
    same_f32(v, vr, n, "exp_avg_sq");
    if (amsgrad) {
        back(x, dx, fb);
        same_f32(x, xr, n, "max_exp_avg_sq");
    }
    printf("abi_check gpu: flat fp32 %s n=%lld: norm %.7g coef %.7g, bit-exact\n",
           amsgrad ? "amsgrad + clip" : "clip", (long long)n, norm, coef);
    HIP(hipFree(dp)); HIP(hipFree(dg)); HIP(hipFree(dm)); HIP(hipFree(dv));
    if (dx) HIP(hipFree(dx));
    HIP(hipFree(dpart)); HIP(hipFree(dnorm)); HIP(hipFree(dcoef));
    free(p); free(g); free(m); free(v); free(x); free(pr); free(mr); free(vr); free(xr);
}

/* Tensor and chunk tables: three tensors, two hyper sets, bf16 moments, bf16 copy. */
static void table_case(void)
{
    enum { NT = 3 };
    const int64_t numel[NT] = {5, 3 * 4096 + 7, 70001};
    mi_adamw_hyper h[2];
    oracle_hyper oh[2];
    scalars(3e-4, 0.9, 0.95, 1e-8, 0.1, 11.0, 0, &h[0], &oh[0]);
    scalars(1e-3, 0.9, 0.999, 1e-8, 0.0, 3.0, 1, &h[1], &oh[1]); /* no decay, maximize */
    const int32_t hyper_of[NT] = {1, 0, 0};

    mi_adamw_tensor rows[NT];
    float *p[NT], *g[NT], *pr[NT];
    uint16_t *m[NT], *v[NT], *mr[NT], *vr[NT], *c[NT];
    void *dp[NT], *dg[NT], *dm[NT], *dv[NT], *dc[NT];
    for (int k = 0; k < NT; ++k) {
        const int64_t n = numel[k];
        p[k] = malloc(n * 4); g[k] = malloc(n * 4); pr[k] = malloc(n * 4);
        m[k] = malloc(n * 2); v[k] = malloc(n * 2); mr[k] = malloc(n * 2); vr[k] = malloc(n * 2);
        c[k] = malloc(n * 2);
        CHECK(p[k] && g[k] && pr[k] && m[k] && v[k] && mr[k] && vr[k] && c[k], "host allocation");
        fill(p[k], n, 0.02f, 0);
        fill(g[k], n, 1e-3f, 0);
        for (int64_t i = 0; i < n; ++i) {
            m[k][i] = oracle_f32_to_bf16(urand() * 1e-3f);
            v[k][i] = oracle_f32_to_bf16(fabsf(urand()) * 1e-6f);
        }
        memcpy(pr[k], p[k], n * 4);
        memcpy(mr[k], m[k], n * 2);
        memcpy(vr[k], v[k], n * 2);
        dp[k] = dev_copy(p[k], n * 4);
        dg[k] = dev_copy(g[k], n * 4);
        dm[k] = dev_copy(m[k], n * 2);
        dv[k] = dev_copy(v[k], n * 2);
        HIP(hipMalloc(&dc[k], n * 2));
        memset(&rows[k], 0, sizeof rows[k]);
        rows[k].param = dp[k];
        rows[k].grad = dg[k];
        rows[k].exp_avg = dm[k];
        rows[k].exp_avg_sq = dv[k];
        rows[k].param_copy = dc[k];
        rows[k].numel = n;
        rows[k].hyper = hyper_of[k];
        rows[k].flags = MI_ADAMW_T_VEC;
    }
    const int64_t n_chunks = mi_adamw_build_chunks(numel, NT, 4096, NULL, 0);
    CHECK(n_chunks == 1 + 4 + 18, "chunk count %lld", (long long)n_chunks);
    mi_adamw_chunk *chunks = malloc(n_chunks * sizeof *chunks);
    CHECK(chunks && mi_adamw_build_chunks(numel, NT, 4096, chunks, n_chunks) == n_chunks,
          "chunk table");
    void *d_rows = dev_copy(rows, sizeof rows);
    void *d_chunks = dev_copy(chunks, n_chunks * sizeof *chunks);
    const int rc = mi_adamw_step(d_rows, d_chunks, n_chunks, 4096, h, 2, NULL,
                                 MI_ADAMW_STATE_BF16, MI_ADAMW_F_BF16_COPY, 0, NULL);
    CHECK(rc == 0, "mi_adamw_step: %s", mi_adamw_strerror(rc));
    HIP(hipDeviceSynchronize());
    for (int k = 0; k < NT; ++k) {
        const int64_t n = numel[k];
        oracle_adamw_bf16state(pr[k], g[k], mr[k], vr[k], NULL, n, &oh[hyper_of[k]], &ROCM_OPS,
                               1.0f, 0);
        back(p[k], dp[k], n * 4);
        back(m[k], dm[k], n * 2);
        back(v[k], dv[k], n * 2);
        back(c[k], dc[k], n * 2);
        same_f32(p[k], pr[k], n, "param (tables)");
        same_u16(m[k], mr[k], n, "bf16 exp_avg");
        same_u16(v[k], vr[k], n, "bf16 exp_avg_sq");
        for (int64_t i = 0; i < n; ++i)
            CHECK(c[k][i] == oracle_f32_to_bf16(pr[k][i]), "bf16 copy at %lld", (long long)i);
        HIP(hipFree(dp[k])); HIP(hipFree(dg[k])); HIP(hipFree(dm[k])); HIP(hipFree(dv[k]));
        HIP(hipFree(dc[k]));
        free(p[k]); free(g[k]); free(pr[k]); free(m[k]); free(v[k]); free(mr[k]); free(vr[k]);
        free(c[k]);
    }
    HIP(hipFree(d_rows));
    HIP(hipFree(d_chunks));
    free(chunks);
    printf("abi_check gpu: tables, %d tensors, %lld chunks, bf16 state + copy: bit-exact\n", NT,
           (long long)n_chunks);
}

/* The capturable chain through tables: two tensors at different device step
 * counts (3 and 1), first with a float lr, then with a device lr.  beta1 = 0.5
 * and beta2 = 0.75 make beta**step exact at these steps, so the oracle's libm
 * powf and the device's powf agree by construction. */
static void capt_case(void)
{
    enum { NT = 2 };
    const int64_t numel[NT] = {2 * 4096 + 3, 70001};
    const float steps[3] = {7.0f, 1.0f, 3.0f};  /* the device step buffer */
    const int32_t step_index[NT] = {2, 1};      /* row -> index into steps */
    float *p[NT], *g[NT], *m[NT], *v[NT], *pr[NT], *mr[NT], *vr[NT];
    void *dp[NT], *dg[NT], *dm[NT], *dv[NT];
    mi_adamw_tensor rows[NT];
    for (int k = 0; k < NT; ++k) {
        const int64_t n = numel[k];
        p[k] = malloc(n * 4); g[k] = malloc(n * 4); m[k] = malloc(n * 4); v[k] = malloc(n * 4);
        pr[k] = malloc(n * 4); mr[k] = malloc(n * 4); vr[k] = malloc(n * 4);
        CHECK(p[k] && g[k] && m[k] && v[k] && pr[k] && mr[k] && vr[k], "host allocation");
        fill(p[k], n, 0.02f, 0);
        fill(g[k], n, 1e-3f, 0);
        fill(m[k], n, 1e-3f, 0);
        fill(v[k], n, 1e-6f, 1);
        memcpy(pr[k], p[k], n * 4);
        memcpy(mr[k], m[k], n * 4);
        memcpy(vr[k], v[k], n * 4);
        dp[k] = dev_copy(p[k], n * 4);
        dg[k] = dev_copy(g[k], n * 4);
        dm[k] = dev_copy(m[k], n * 4);
        dv[k] = dev_copy(v[k], n * 4);
        memset(&rows[k], 0, sizeof rows[k]);
        rows[k].param = dp[k];
        rows[k].grad = dg[k];
        rows[k].exp_avg = dm[k];
        rows[k].exp_avg_sq = dv[k];
        rows[k].numel = n;
        rows[k].flags = MI_ADAMW_T_VEC;
    }
    const int64_t n_chunks = mi_adamw_build_chunks(numel, NT, 4096, NULL, 0);
    mi_adamw_chunk *chunks = malloc(n_chunks * sizeof *chunks);
    CHECK(chunks && mi_adamw_build_chunks(numel, NT, 4096, chunks, n_chunks) == n_chunks,
          "chunk table");
    void *d_rows = dev_copy(rows, sizeof rows);
    void *d_chunks = dev_copy(chunks, n_chunks * sizeof *chunks);
    float *d_steps = dev_copy(steps, sizeof steps);
    int32_t *d_index = dev_copy(step_index, sizeof step_index);
    const float lr_dev = 2e-3f;
    float *d_lr = dev_copy(&lr_dev, sizeof lr_dev);
    void *d_row_scalars = NULL;
    HIP(hipMalloc(&d_row_scalars, NT * MI_ADAMW_ROW_SCALAR_BYTES));
    /* passes 0, 1: mi_adamw_step_capturable; 2, 3: mi_adamw_step_capturable_rows; even
     * passes a float lr, odd ones a device lr; the state carries over from pass to pass */
    for (int pass = 0; pass < 4; ++pass) {
        const int dev_lr = pass & 1, rows_entry = pass >= 2;
        mi_adamw_capt_hyper ch;
        memset(&ch, 0, sizeof ch);
        ch.beta1 = 0.5f;
        ch.beta2 = 0.75f;
        ch.lerp_w = (float)(1.0 - 0.5);
        ch.one_minus_beta2 = (float)(1.0 - 0.75);
        ch.eps = 1e-8f;
        ch.grad_sign = 1.0f;
        float lr, wd_factor;
        if (!dev_lr) {
            ch.lr_mode = MI_ADAMW_LR_FLOAT;
            ch.lr = lr = (float)1e-3;
            ch.wd_factor = wd_factor = (float)(1.0 - 1e-3 * 0.1);
        } else {
            ch.lr_mode = MI_ADAMW_LR_DEVICE;
            ch.lr_ptr = d_lr;
            ch.weight_decay = 0.1f;
            lr = lr_dev;
            wd_factor = 1.0f - lr_dev * 0.1f;   /* two fp32 ops, as on the device */
        }
        const int rc =
            rows_entry
                ? mi_adamw_step_capturable_rows(d_rows, NT, d_chunks, n_chunks, 4096, &ch, 1,
                                                d_steps, d_index, d_row_scalars, NULL,
                                                MI_ADAMW_STATE_F32, 0, 0, NULL)
                : mi_adamw_step_capturable(d_rows, d_chunks, n_chunks, 4096, &ch, 1, d_steps,
                                           d_index, NULL, MI_ADAMW_STATE_F32, 0, 0, NULL);
        CHECK(rc == 0, "mi_adamw_step_capturable%s: %s", rows_entry ? "_rows" : "",
              mi_adamw_strerror(rc));
        HIP(hipDeviceSynchronize());
        for (int k = 0; k < NT; ++k) {
            const int64_t n = numel[k];
            oracle_capt oc;
            oc.wd_factor = wd_factor;
            oc.lerp_w = ch.lerp_w;
            oc.beta2 = ch.beta2;
            oc.one_minus_beta2 = ch.one_minus_beta2;
            oc.grad_sign = 1.0f;
            oracle_capt_scalars(ch.beta1, ch.beta2, lr, ch.eps, steps[step_index[k]], dev_lr,
                                &oc.den_scale, &oc.den_add);
            oracle_adamw_capt_f32(pr[k], g[k], mr[k], vr[k], NULL, n, &oc, &ROCM_OPS, 1.0f, 0);
            back(p[k], dp[k], n * 4);
            back(m[k], dm[k], n * 4);
            back(v[k], dv[k], n * 4);
            same_f32(p[k], pr[k], n, "param (capturable)");
            same_f32(m[k], mr[k], n, "exp_avg (capturable)");
            same_f32(v[k], vr[k], n, "exp_avg_sq (capturable)");
        }
    }
    for (int k = 0; k < NT; ++k) {
        HIP(hipFree(dp[k])); HIP(hipFree(dg[k])); HIP(hipFree(dm[k])); HIP(hipFree(dv[k]));
        free(p[k]); free(g[k]); free(m[k]); free(v[k]); free(pr[k]); free(mr[k]); free(vr[k]);
    }
    HIP(hipFree(d_rows)); HIP(hipFree(d_chunks)); HIP(hipFree(d_steps)); HIP(hipFree(d_index));
    HIP(hipFree(d_lr));
    HIP(hipFree(d_row_scalars));
    free(chunks);
    printf("abi_check gpu: capturable tables, steps 3 and 1, float then device lr, both entry "
           "points: bit-exact\n");
}

/* The clip split at the all-reduce over `world` slices of one flat range, with the
 * data-parallel pre-scale f32(1/world): each slice's float64 sum, the finalize over the
 * sums, each slice's pre-scaled update; against the oracle stepping the pre-scaled
 * gradients.  Then the no-alloc norm against the workspace one. */
static void split_case(int64_t n, int world)
{
    const size_t fb = (size_t)n * sizeof(float);
    float *p = malloc(fb), *g = malloc(fb), *m = malloc(fb), *v = malloc(fb), *gp = malloc(fb);
    float *pr = malloc(fb), *mr = malloc(fb), *vr = malloc(fb);
    CHECK(p && g && m && v && gp && pr && mr && vr, "host allocation");
    fill(p, n, 0.02f, 0);
    fill(g, n, 3e-2f, 0);
    fill(m, n, 1e-3f, 0);
    fill(v, n, 1e-6f, 1);
    const float pre = (float)(1.0 / world);
    for (int64_t i = 0; i < n; ++i) gp[i] = g[i] * pre; /* what grad.div_(world) stores */
    memcpy(pr, p, fb);
    memcpy(mr, m, fb);
    memcpy(vr, v, fb);
    float *dp = dev_copy(p, fb), *dg = dev_copy(g, fb), *dm = dev_copy(m, fb);
    float *dv = dev_copy(v, fb);
    double *dpart = NULL, *dsum = NULL;
    float *dnorm = NULL, *dcoef = NULL;
    HIP(hipMalloc((void **)&dpart, MI_ADAMW_MAX_NORM_BLOCKS * sizeof(double)));
    HIP(hipMalloc((void **)&dsum, world * sizeof(double)));
    HIP(hipMalloc((void **)&dnorm, 4 * sizeof(float)));
    HIP(hipMalloc((void **)&dcoef, 4 * sizeof(float)));
    mi_adamw_hyper h;
    oracle_hyper oh;
    scalars(3e-4, 0.9, 0.95, 1e-8, 0.1, 1001.0, 0, &h, &oh);
    const int64_t units = n / 32;
    int rc;
    for (int r = 0; r < world; ++r) {
        const int64_t lo = (r * units / world) * 32;
        const int64_t hi = r + 1 == world ? n : ((r + 1) * units / world) * 32;
        rc = mi_adamw_grad_sumsq_flat(dg + lo, hi - lo, 4096, pre, dpart, dsum + r, NULL);
        CHECK(rc == 0, "mi_adamw_grad_sumsq_flat: %s", mi_adamw_strerror(rc));
    }
    rc = mi_adamw_norm_from_sumsq(dsum, world, 1.0f, dnorm, dcoef, NULL);
    CHECK(rc == 0, "mi_adamw_norm_from_sumsq: %s", mi_adamw_strerror(rc));
    for (int r = 0; r < world; ++r) {
        const int64_t lo = (r * units / world) * 32;
        const int64_t hi = r + 1 == world ? n : ((r + 1) * units / world) * 32;
        mi_adamw_tensor t;
        memset(&t, 0, sizeof t);
        t.param = dp + lo;
        t.grad = dg + lo;
        t.exp_avg = dm + lo;
        t.exp_avg_sq = dv + lo;
        t.numel = hi - lo;
        t.flags = MI_ADAMW_T_VEC; /* 32-element (128-byte) slice boundaries */
        rc = mi_adamw_step_flat_prescaled(&t, &h, dcoef, pre, 4096, MI_ADAMW_STATE_F32,
                                          MI_ADAMW_F_CLIP, 0, NULL);
        CHECK(rc == 0, "mi_adamw_step_flat_prescaled: %s", mi_adamw_strerror(rc));
    }
    /* the no-alloc norm against the workspace norm, on the raw gradients */
    rc = mi_adamw_grad_norm_flat(dg, n, 4096, 1.0f, dpart, dnorm + 1, dcoef + 1, NULL);
    CHECK(rc == 0, "mi_adamw_grad_norm_flat: %s", mi_adamw_strerror(rc));
    rc = mi_adamw_grad_norm_flat_noalloc(dg, n, 4096, 1.0f, dnorm + 2, dcoef + 2, NULL);
    CHECK(rc == 0, "mi_adamw_grad_norm_flat_noalloc: %s", mi_adamw_strerror(rc));
    HIP(hipDeviceSynchronize());
    float norm[4], coef[4];
    back(norm, dnorm, sizeof norm);
    back(coef, dcoef, sizeof coef);
    const double ref = sqrt(oracle_sumsq_f64(gp, n));
    CHECK(fabs((double)norm[0] - ref) <= 1e-6 * ref, "split norm %.9g vs %.9g", norm[0], ref);
    const float coef_ref = oracle_clip_coef(norm[0], 1.0);
    CHECK(memcmp(&coef[0], &coef_ref, sizeof coef_ref) == 0 && coef[0] < 1.0f,
          "split coef %.9g vs %.9g", coef[0], coef_ref);
    CHECK(memcmp(&norm[1], &norm[2], 4) == 0 && memcmp(&coef[1], &coef[2], 4) == 0,
          "no-alloc norm %.9g / %.9g vs workspace %.9g / %.9g", norm[2], coef[2], norm[1], coef[1]);
    oracle_adamw_f32(pr, gp, mr, vr, NULL, n, &oh, &ROCM_OPS, coef[0], 1);
    back(p, dp, fb);
    back(m, dm, fb);
    back(v, dv, fb);
    same_f32(p, pr, n, "param (split clip)");
    same_f32(m, mr, n, "exp_avg (split clip)");
    same_f32(v, vr, n, "exp_avg_sq (split clip)");
    printf("abi_check gpu: split clip over %d slices, pre-scale 1/%d, n=%lld: norm %.7g, "
           "no-alloc norm equal, bit-exact\n", world, world, (long long)n, norm[0]);
    HIP(hipFree(dp)); HIP(hipFree(dg)); HIP(hipFree(dm)); HIP(hipFree(dv));
    HIP(hipFree(dpart)); HIP(hipFree(dsum)); HIP(hipFree(dnorm)); HIP(hipFree(dcoef));
    free(p); free(g); free(m); free(v); free(gp); free(pr); free(mr); free(vr);
}

/* Tables of two tensors, two chained steps: the second step's gradients are new
 * buffers written into the device table by mi_adamw_set_grads (one of them misaligned,
 * so its row leaves the vector path). */
static void set_grads_case(void)
{
    enum { NT = 2 };
    const int64_t numel[NT] = {70001, 4099};
    float *p[NT], *pr[NT], *m[NT], *mr[NT], *v[NT], *vr[NT], *g1[NT], *g2[NT];
    void *dp[NT], *dm[NT], *dv[NT], *dg1[NT], *dg2[NT];
    mi_adamw_tensor rows[NT];
    for (int k = 0; k < NT; ++k) {
        const int64_t n = numel[k];
        p[k] = malloc(n * 4); pr[k] = malloc(n * 4); m[k] = malloc(n * 4); mr[k] = malloc(n * 4);
        v[k] = malloc(n * 4); vr[k] = malloc(n * 4); g1[k] = malloc(n * 4); g2[k] = malloc(n * 4);
        CHECK(p[k] && pr[k] && m[k] && mr[k] && v[k] && vr[k] && g1[k] && g2[k], "host allocation");
        fill(p[k], n, 0.02f, 0);
        fill(m[k], n, 1e-3f, 0);
        fill(v[k], n, 1e-6f, 1);
        fill(g1[k], n, 1e-3f, 0);
        fill(g2[k], n, 1e-3f, 0);
        memcpy(pr[k], p[k], n * 4);
        memcpy(mr[k], m[k], n * 4);
        memcpy(vr[k], v[k], n * 4);
        dp[k] = dev_copy(p[k], n * 4);
        dm[k] = dev_copy(m[k], n * 4);
        dv[k] = dev_copy(v[k], n * 4);
        dg1[k] = dev_copy(g1[k], n * 4);
        /* the second gradient of tensor 1 sits one element into its buffer: misaligned */
        HIP(hipMalloc(&dg2[k], (n + 1) * 4));
        HIP(hipMemcpy((float *)dg2[k] + k, g2[k], n * 4, hipMemcpyHostToDevice));
        memset(&rows[k], 0, sizeof rows[k]);
        rows[k].param = dp[k];
        rows[k].grad = dg1[k];
        rows[k].exp_avg = dm[k];
        rows[k].exp_avg_sq = dv[k];
        rows[k].numel = n;
        rows[k].hyper = 0;
        rows[k].flags = MI_ADAMW_T_VEC;
    }
    const int64_t nc = mi_adamw_build_chunks(numel, NT, 4096, NULL, 0);
    mi_adamw_chunk *chunks = malloc(nc * sizeof *chunks);
    CHECK(chunks && mi_adamw_build_chunks(numel, NT, 4096, chunks, nc) == nc, "chunks");
    void *d_rows = dev_copy(rows, sizeof rows), *d_chunks = dev_copy(chunks, nc * sizeof *chunks);
    for (int step = 1; step <= 2; ++step) {
        if (step == 2) {
            const int32_t which[NT] = {0, 1};
            const uint64_t ptrs[NT] = {(uint64_t)(uintptr_t)dg2[0],
                                       (uint64_t)(uintptr_t)((float *)dg2[1] + 1)};
            const uint8_t vec[NT] = {1, 0};
            const int rc = mi_adamw_set_grads((mi_adamw_tensor *)d_rows, NT, NT, which, ptrs, vec,
                                              NULL);
            CHECK(rc == 0, "mi_adamw_set_grads: %s", mi_adamw_strerror(rc));
        }
        mi_adamw_hyper h;
        oracle_hyper oh;
        scalars(3e-4, 0.9, 0.95, 1e-8, 0.1, 10.0 + step, 0, &h, &oh);
        const int rc = mi_adamw_step(d_rows, d_chunks, nc, 4096, &h, 1, NULL, MI_ADAMW_STATE_F32,
                                     0, 0, NULL);
        CHECK(rc == 0, "mi_adamw_step: %s", mi_adamw_strerror(rc));
        for (int k = 0; k < NT; ++k)
            oracle_adamw_f32(pr[k], step == 1 ? g1[k] : g2[k], mr[k], vr[k], NULL, numel[k], &oh,
                             &ROCM_OPS, 1.0f, 0);
    }
    HIP(hipDeviceSynchronize());
    mi_adamw_tensor after[NT];
    back(after, d_rows, sizeof after);
    CHECK(after[0].grad == dg2[0] && (after[0].flags & MI_ADAMW_T_VEC), "row 0 after the patch");
    CHECK(after[1].grad == (float *)dg2[1] + 1 && !(after[1].flags & MI_ADAMW_T_VEC),
          "row 1 after the patch");
    for (int k = 0; k < NT; ++k) {
        back(p[k], dp[k], numel[k] * 4);
        back(m[k], dm[k], numel[k] * 4);
        back(v[k], dv[k], numel[k] * 4);
        same_f32(p[k], pr[k], numel[k], "param (patched gradients)");
        same_f32(m[k], mr[k], numel[k], "exp_avg (patched gradients)");
        same_f32(v[k], vr[k], numel[k], "exp_avg_sq (patched gradients)");
        HIP(hipFree(dp[k])); HIP(hipFree(dm[k])); HIP(hipFree(dv[k]));
        HIP(hipFree(dg1[k])); HIP(hipFree(dg2[k]));
        free(p[k]); free(pr[k]); free(m[k]); free(mr[k]); free(v[k]); free(vr[k]);
        free(g1[k]); free(g2[k]);
    }
    HIP(hipFree(d_rows)); HIP(hipFree(d_chunks));
    free(chunks);
    printf("abi_check gpu: gradients moved between two table steps (one misaligned), patched by "
           "mi_adamw_set_grads: bit-exact\n");
}

/* One set of torch's fused=True chain (mi_adamw_fused_hyper) and the oracle's scalars for
 * it: the float64 hyperparameters, and the per-step values formed from the step count with
 * libm pow, as the library forms them on the host. */
static void fused_set(mi_adamw_fused_hyper *h, oracle_fused *o, double lr, double b1, double b2,
                      double wd, float step, int maximize)
{
    memset(h, 0, sizeof *h);
    h->lr = lr;
    h->beta1 = b1;
    h->beta2 = b2;
    h->weight_decay = wd;
    h->eps = 1e-8;
    h->step = step;
    h->grad_sign = maximize ? -1.0f : 1.0f;
    memset(o, 0, sizeof *o);
    o->lr = lr;
    o->beta1 = b1;
    o->beta2 = b2;
    o->weight_decay = wd;
    o->eps = 1e-8;
    float bc1;
    oracle_fused_scalars(lr, b1, b2, step, &bc1, &o->bc2_sqrt, &o->step_size);
    o->grad_sign = h->grad_sign;
}

/* torch's fused=True chain: tensor 0 as a flat range with the clip; both tensors through
 * tables with two sets (the second without weight decay, with maximize); then the tables
 * at device step counts (3 and 1) with a device lr, where beta1 = 0.5 and beta2 = 0.75 make
 * pow exact at those steps on the host and the device alike. */
static void fused_case(void)
{
    static const oracle_fused_model TORCH_FUSED = {1, 1, 1};
    enum { NT = 2 };
    const int64_t numel[NT] = {3 * 4096 + 1, 50003};
    float *p[NT], *g[NT], *m[NT], *v[NT], *pr[NT], *mr[NT], *vr[NT];
    void *dp[NT], *dg[NT], *dm[NT], *dv[NT];
    mi_adamw_tensor rows[NT];
    for (int k = 0; k < NT; ++k) {
        const int64_t n = numel[k];
        p[k] = malloc(n * 4); g[k] = malloc(n * 4); m[k] = malloc(n * 4); v[k] = malloc(n * 4);
        pr[k] = malloc(n * 4); mr[k] = malloc(n * 4); vr[k] = malloc(n * 4);
        CHECK(p[k] && g[k] && m[k] && v[k] && pr[k] && mr[k] && vr[k], "host allocation");
        fill(p[k], n, 0.02f, 0);
        fill(g[k], n, 2e-2f, 0);
        fill(m[k], n, 1e-3f, 0);
        fill(v[k], n, 1e-6f, 1);
        memcpy(pr[k], p[k], n * 4);
        memcpy(mr[k], m[k], n * 4);
        memcpy(vr[k], v[k], n * 4);
        dp[k] = dev_copy(p[k], n * 4);
        dg[k] = dev_copy(g[k], n * 4);
        dm[k] = dev_copy(m[k], n * 4);
        dv[k] = dev_copy(v[k], n * 4);
        memset(&rows[k], 0, sizeof rows[k]);
        rows[k].param = dp[k];
        rows[k].grad = dg[k];
        rows[k].exp_avg = dm[k];
        rows[k].exp_avg_sq = dv[k];
        rows[k].numel = n;
        rows[k].hyper = k;
        rows[k].flags = MI_ADAMW_T_VEC;
    }
    {
        const int64_t n = numel[0];
        double *d_partials;
        float *d_norm, *d_coef;
        HIP(hipMalloc((void **)&d_partials, MI_ADAMW_MAX_NORM_BLOCKS * sizeof(double)));
        HIP(hipMalloc((void **)&d_norm, 4));
        HIP(hipMalloc((void **)&d_coef, 4));
        int rc = mi_adamw_grad_norm_flat(dg[0], n, 4096, 1.0f, d_partials, d_norm, d_coef, NULL);
        CHECK(rc == 0, "mi_adamw_grad_norm_flat: %s", mi_adamw_strerror(rc));
        mi_adamw_fused_hyper h;
        oracle_fused o;
        fused_set(&h, &o, 3e-4, 0.9, 0.95, 0.1, 1000.0f, 0);
        rc = mi_adamw_step_flat_fused_chain(&rows[0], &h, d_coef, 1.0f, 4096, MI_ADAMW_STATE_F32,
                                            MI_ADAMW_F_CLIP, 0, NULL);
        CHECK(rc == 0, "mi_adamw_step_flat_fused_chain: %s", mi_adamw_strerror(rc));
        HIP(hipDeviceSynchronize());
        float coef;
        back(&coef, d_coef, 4);
        CHECK(coef < 1.0f, "the clip triggers (coef %g)", coef);
        oracle_adamw_fused_f32(pr[0], g[0], mr[0], vr[0], NULL, n, &o, &TORCH_FUSED, coef, 1);
        back(p[0], dp[0], n * 4);
        back(m[0], dm[0], n * 4);
        back(v[0], dv[0], n * 4);
        same_f32(p[0], pr[0], n, "param (fused chain, flat, clip)");
        same_f32(m[0], mr[0], n, "exp_avg (fused chain, flat, clip)");
        same_f32(v[0], vr[0], n, "exp_avg_sq (fused chain, flat, clip)");
        HIP(hipFree(d_partials)); HIP(hipFree(d_norm)); HIP(hipFree(d_coef));
    }
    const int64_t n_chunks = mi_adamw_build_chunks(numel, NT, 4096, NULL, 0);
    mi_adamw_chunk *chunks = malloc(n_chunks * sizeof *chunks);
    CHECK(chunks && mi_adamw_build_chunks(numel, NT, 4096, chunks, n_chunks) == n_chunks,
          "chunk table");
    void *d_rows = dev_copy(rows, sizeof rows);
    void *d_chunks = dev_copy(chunks, n_chunks * sizeof *chunks);
    const float steps[3] = {9.0f, 1.0f, 3.0f};      /* the device step buffer */
    const int32_t step_index[NT] = {2, 1};          /* row -> index into steps */
    float *d_steps = dev_copy(steps, sizeof steps);
    int32_t *d_index = dev_copy(step_index, sizeof step_index);
    const float lr_dev = 2e-3f;
    float *d_lr = dev_copy(&lr_dev, sizeof lr_dev);
    void *d_row_scalars = NULL;
    HIP(hipMalloc(&d_row_scalars, NT * MI_ADAMW_ROW_SCALAR_BYTES));
    /* pass 0: host steps; 1: device steps and lr, mi_adamw_step_fused_chain; 2: the same
     * through mi_adamw_step_fused_chain_rows; the state carries over */
    for (int pass = 0; pass < 3; ++pass) {
        mi_adamw_fused_hyper h[NT];
        oracle_fused o[NT];
        int rc;
        if (pass == 0) {
            fused_set(&h[0], &o[0], 3e-4, 0.9, 0.95, 0.1, 1001.0f, 0);
            fused_set(&h[1], &o[1], 1e-3, 0.9, 0.999, 0.0, 7.0f, 1);
            rc = mi_adamw_step_fused_chain(d_rows, d_chunks, n_chunks, 4096, h, NT, NULL, NULL,
                                           NULL, 1.0f, MI_ADAMW_STATE_F32, 0, 0, NULL);
        } else {
            for (int k = 0; k < NT; ++k) {
                fused_set(&h[k], &o[k], (double)lr_dev, 0.5, 0.75, 0.1,
                          steps[step_index[k]], 0);
                h[k].lr = 0.0;           /* the kernel reads the device lr */
                h[k].lr_ptr = d_lr;
                h[k].step = 0.0f;        /* and the device step counts */
            }
            rc = pass == 1
                     ? mi_adamw_step_fused_chain(d_rows, d_chunks, n_chunks, 4096, h, NT,
                                                 d_steps, d_index, NULL, 1.0f,
                                                 MI_ADAMW_STATE_F32, 0, 0, NULL)
                     : mi_adamw_step_fused_chain_rows(d_rows, NT, d_chunks, n_chunks, 4096, h,
                                                      NT, d_steps, d_index, d_row_scalars, NULL,
                                                      1.0f, MI_ADAMW_STATE_F32, 0, 0, NULL);
        }
        CHECK(rc == 0, "mi_adamw_step_fused_chain (pass %d): %s", pass, mi_adamw_strerror(rc));
        HIP(hipDeviceSynchronize());
        for (int k = 0; k < NT; ++k) {
            const int64_t n = numel[k];
            oracle_adamw_fused_f32(pr[k], g[k], mr[k], vr[k], NULL, n, &o[k], &TORCH_FUSED, 1.0f,
                                   0);
            back(p[k], dp[k], n * 4);
            back(m[k], dm[k], n * 4);
            back(v[k], dv[k], n * 4);
            same_f32(p[k], pr[k], n, pass ? "param (fused chain, device steps)"
                                          : "param (fused chain, tables)");
            same_f32(m[k], mr[k], n, "exp_avg (fused chain)");
            same_f32(v[k], vr[k], n, "exp_avg_sq (fused chain)");
        }
    }
    for (int k = 0; k < NT; ++k) {
        HIP(hipFree(dp[k])); HIP(hipFree(dg[k])); HIP(hipFree(dm[k])); HIP(hipFree(dv[k]));
        free(p[k]); free(g[k]); free(m[k]); free(v[k]); free(pr[k]); free(mr[k]); free(vr[k]);
    }
    HIP(hipFree(d_rows)); HIP(hipFree(d_chunks)); HIP(hipFree(d_steps)); HIP(hipFree(d_index));
    HIP(hipFree(d_lr));
    HIP(hipFree(d_row_scalars));
    free(chunks);
    printf("abi_check gpu: fused=True chain, flat with clip, tables with two sets, device steps "
           "and lr (both entry points): bit-exact\n");
}

static int gpu_checks(void)
{
    int count = 0;
    HIP(hipGetDeviceCount(&count));
    CHECK(count > 0, "no GPU");
    HIP(hipSetDevice(0));
    flat_case(1000003, 0);
    table_case();
    flat_case(262147, 1);
    capt_case();
    split_case(3000000 + 96, 3);
    set_grads_case();
    fused_case();
    printf("abi_check gpu: ok (%s)\n", mi_adamw_version());
    return 0;
}

int main(int argc, char **argv)
{
    if (argc == 2 && strcmp(argv[1], "cpu") == 0) return cpu_checks();
    if (argc == 2 && strcmp(argv[1], "gpu") == 0) return gpu_checks();
    fprintf(stderr, "usage: abi_check cpu|gpu\n");
    return 2;
}
