/*
 * mi_adamw.h -- C ABI of the MI355X (gfx950) fused clip + AdamW optimizer step.
 *
 * One shared library, libmi_adamw.so, exports these symbols.  They take plain
 * device pointers, sizes, host structs and a hipStream_t (passed as void*), and
 * never throw: every entry point returns MI_ADAMW_OK (0), a negative
 * MI_ADAMW_E_* code for a rejected argument, or a positive hipError_t value.
 * All work is enqueued on the given stream; nothing synchronises the host.
 *
 * What the entry points replace.  mini-megatron steps `torch.optim.AdamW(...,
 * fused=False)` once per iteration (main.py:177 builds it, main.py:209 and
 * parallel/pipeline_parallel.py:260 call step()).  That runs torch's
 * `_single_tensor_adam` (torch/optim/adam.py:396-547): 8 elementwise kernels
 * per parameter tensor.  The gradient clip that config.py:16 names
 * (MAX_GRAD_NORM) is torch's clip_grad_norm_ (torch/nn/utils/clip_grad.py:186).
 * The Python class mi_adamw.FusedAdamW (a torch.optim.Optimizer) is the only
 * caller; it is the drop-in for the reference's optimizer object.
 *
 * Layout.  A launch covers many tensors through two device-resident tables:
 *   - a tensor table (mi_adamw_tensor[]): the pointers and size of each tensor;
 *   - a chunk table (mi_adamw_chunk[]): (tensor, chunk index) pairs, one per
 *     `chunk_elems`-element slice of a tensor.  Chunk i of tensor t covers
 *     elements [i*chunk_elems, min((i+1)*chunk_elems, numel)).
 * The "flat" entry points take one contiguous range instead of the tables
 * (the flat-buffer layout: every tensor packed at a 128-byte-aligned offset).
 *
 * Numerics.  Each element follows the fp32 op chain of adam.py:419-547, with
 * one fp32 rounding per ATen op, in the contraction pattern torch-ROCm's kernels
 * use (lerp, addcmul and addcdiv as fused multiply-adds; division by the host
 * scalar bc2_sqrt as a multiply by its reciprocal rounded to fp32).  The caller computes
 * the per-step scalars on the host in float64 (adam.py:529-536) and passes them
 * rounded to fp32 in mi_adamw_hyper.  The *_fused_chain entry points follow torch's
 * fused=True chain instead (torch._fused_adamw_, see mi_adamw_fused_hyper); the
 * capturable entry point follows torch's capturable chain.
 */
#ifndef MI_ADAMW_H
#define MI_ADAMW_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_ADAMW_ABI_VERSION 9
#define MI_ADAMW_MAX_HYPER 16      /* hyperparameter sets per launch */
#define MI_ADAMW_MAX_NORM_BLOCKS 4096 /* partial sums per grad-norm launch */

/* Return codes (positive values are hipError_t). */
#define MI_ADAMW_OK 0
#define MI_ADAMW_E_INVALID (-1)    /* a size, count or pointer argument is out of range */
#define MI_ADAMW_E_ALIGN (-2)      /* a tensor flagged aligned has a misaligned pointer */
#define MI_ADAMW_E_SCRATCH (-3)    /* a no-alloc launch needs more than the static scratch holds */

/* Storage dtype of exp_avg / exp_avg_sq. */
#define MI_ADAMW_STATE_F32 0
#define MI_ADAMW_STATE_BF16 1

/* mi_adamw_step* flags. */
#define MI_ADAMW_F_CLIP (1 << 0)       /* multiply every gradient by *grad_scale first */
#define MI_ADAMW_F_BF16_COPY (1 << 1)  /* write the updated parameter to param_copy as bf16 */
#define MI_ADAMW_F_WRITE_GRAD (1 << 2) /* store the scaled gradient back into grad */
#define MI_ADAMW_F_AMSGRAD (1 << 3)    /* amsgrad: max_exp_avg_sq = maximum(max_exp_avg_sq,
                                          exp_avg_sq), and the denominator is taken from it
                                          (adam.py:538-543); every row needs max_exp_avg_sq */

/* mi_adamw_tensor.flags */
#define MI_ADAMW_T_VEC (1 << 0) /* fp32 pointers 16-byte aligned and bf16 pointers 8-byte
                                   aligned: the dwordx4 path may be used */

typedef struct mi_adamw_tensor {
    float *param;          /* fp32 master parameter, updated in place                */
    float *grad;           /* fp32 gradient (written only with MI_ADAMW_F_WRITE_GRAD) */
    void *exp_avg;         /* first moment, fp32 or bf16 (state dtype of the launch)  */
    void *exp_avg_sq;      /* second moment, fp32 or bf16                             */
    uint16_t *param_copy;  /* bf16 model copy, or NULL without MI_ADAMW_F_BF16_COPY   */
    void *max_exp_avg_sq;  /* running maximum of exp_avg_sq (state dtype), or NULL
                              without MI_ADAMW_F_AMSGRAD                               */
    int64_t numel;         /* elements (a complex64 tensor counts 2 per value)        */
    int32_t hyper;         /* index of this tensor's mi_adamw_hyper in the launch     */
    int32_t flags;         /* MI_ADAMW_T_*                                            */
} mi_adamw_tensor;

typedef struct mi_adamw_chunk {
    int32_t tensor;        /* row of the tensor table            */
    int32_t index;         /* chunk number within that tensor    */
} mi_adamw_chunk;

/* Per-step scalars of one parameter group at one step count, as the ATen
 * kernels of adam.py see them (each a float64 host value cast to fp32). */
typedef struct mi_adamw_hyper {
    float wd_factor;       /* 1 - lr*weight_decay; 1 when weight_decay == 0  (adam.py:419) */
    float lerp_w;          /* 1 - beta1                                      (adam.py:457) */
    float beta2;           /* beta2                                          (adam.py:476) */
    float one_minus_beta2; /* 1 - beta2                                      (adam.py:476) */
    float inv_bc2_sqrt;    /* (float)(1.0 / (1 - beta2**step) ** 0.5): the reciprocal taken in
                              float64, as torch-ROCm divides a tensor by a host scalar
                              (adam.py:536,545)                                              */
    float eps;             /* eps                                            (adam.py:545) */
    float neg_step_size;   /* -(lr / (1 - beta1**step))                      (adam.py:534,547) */
    float grad_sign;       /* -1 with maximize=True, else 1                  (adam.py:397) */
} mi_adamw_hyper;

/* How a capturable launch gets the learning rate (mi_adamw_capt_hyper.lr_mode). */
#define MI_ADAMW_LR_FLOAT 0   /* lr is a Python float: step_size = (1/bc1) * lr, the way
                                 torch evaluates `float / tensor` (Tensor.__rtruediv__)      */
#define MI_ADAMW_LR_VALUE 1   /* lr is a tensor whose value the host passes in `lr`:
                                 step_size = lr / bc1, a true division                       */
#define MI_ADAMW_LR_DEVICE 2  /* lr is a device fp32 scalar at lr_ptr, read by the kernel:
                                 step_size = lr / bc1, and the weight-decay factor
                                 1 - lr*weight_decay is formed on the device                 */

/* One parameter group of a capturable step (torch.optim.AdamW(capturable=True):
 * adam.py:396-527, the per-step scalars at adam.py:480-522).  Nothing here
 * depends on the step count: the kernel reads each tensor's step from device
 * memory and forms
 *   bc1 = 1 - beta1**step, bc2 = 1 - beta2**step, step_size (see lr_mode),
 *   a = sqrt(bc2) * -step_size, e = eps * (1 / -step_size)
 * in fp32, op for op, so that a launch recorded into a HIP graph stays right as
 * the steps advance.  The element chain is then
 *   p = p*wd_factor; m = lerp(m, g, lerp_w); v = v*beta2 + (1-beta2)*g*g;
 *   p = p + m / (sqrt(v) / a + e). */
typedef struct mi_adamw_capt_hyper {
    float beta1;           /* base of beta1**step                              (adam.py:488) */
    float beta2;           /* v *= beta2, and the base of beta2**step          (adam.py:476,497) */
    float lerp_w;          /* 1 - beta1                                        (adam.py:457) */
    float one_minus_beta2; /* 1 - beta2                                        (adam.py:476) */
    float eps;             /* eps                                              (adam.py:522) */
    float grad_sign;       /* -1 with maximize=True, else 1                    (adam.py:397) */
    float lr;              /* LR_FLOAT, LR_VALUE: the learning rate                          */
    float wd_factor;       /* LR_FLOAT, LR_VALUE: 1 - lr*weight_decay, 1 when wd == 0 (:419) */
    float weight_decay;    /* LR_DEVICE: the weight decay, 0 for none                        */
    int32_t lr_mode;       /* MI_ADAMW_LR_*                                                  */
    const float *lr_ptr;   /* LR_DEVICE: device fp32 learning rate                           */
} mi_adamw_capt_hyper;

/* One parameter group of a step in torch's fused=True chain.  The reference builds
 * its optimizer as torch.optim.AdamW(..., fused=args.fused) (main.py:80,144,177); with
 * --fused that runs adam.py:803-895 (_fused_adam): the step counts += 1 on the device,
 * then torch._fused_adamw_, whose per-element math is adam_math in
 * ATen/native/hip/fused_adam_utils.cuh (ADAMW mode).  The hyperparameters stay float64
 * there, and each workgroup forms the per-step values from the fp32 step count:
 *   bc1 = f32(1 - pow(beta1, step)), bc2_sqrt = f32(sqrt(1 - pow(beta2, step))),
 *   step_size = f32(lr / (double)bc1)          (pow, sqrt, division in float64)
 * Each element, from fp32 p, g, m, v (g after the clip scale and the maximize sign):
 *   p = f32(fma(-(lr*wd), p, p))      when weight_decay != 0   (float64)
 *   m = f32(fma(beta1, m, (1-beta1)*g))                        (float64)
 *   v = f32(fma(beta2, v, ((1-beta2)*g)*g))                    (float64)
 *   d = f32((double)(sqrtf(v) / bc2_sqrt) + eps)   (amsgrad: from fmaxf(vmax, v))
 *   p = p - (step_size * m) / d                                (fp32)
 * the fused multiply-adds where torch-ROCm's build of that kernel has them. */
typedef struct mi_adamw_fused_hyper {
    double lr;             /* the learning rate (a host tensor lr: its value)            */
    double beta1;
    double beta2;
    double weight_decay;
    double eps;
    float step;            /* the step count after this step's increment; unused when the
                              launch reads device step counts (d_steps)                   */
    float grad_sign;       /* -1 with maximize=True, else 1                               */
    const float *lr_ptr;   /* non-NULL: a device fp32 learning rate (a device tensor lr),
                              read by the kernel in place of lr                           */
} mi_adamw_fused_hyper;

/* Library identification: "mi_adamw <abi> gfx950 ...". */
const char *mi_adamw_version(void);

/* Text for a return code (MI_ADAMW_E_* or hipError_t). */
const char *mi_adamw_strerror(int code);

/* Chunk sizes (chunk_elems) must be positive multiples of this (one update tile). */
#define MI_ADAMW_CHUNK_QUANTUM 4096

/* Host-side helper: fill `out` (capacity `cap` entries, host memory) with the
 * chunk table of `n_tensors` tensors of the given sizes.  Returns the number of
 * chunks written, or MI_ADAMW_E_INVALID if it would exceed `cap` or if
 * chunk_elems is not a positive multiple of MI_ADAMW_CHUNK_QUANTUM.  With
 * out == NULL only counts. */
int64_t mi_adamw_build_chunks(const int64_t *numels, int32_t n_tensors, int64_t chunk_elems,
                              mi_adamw_chunk *out, int64_t cap);

/* Global gradient L2 norm and clip coefficient (two launches: the float64
 * sum-of-squares pass over a fixed grid, then a one-workgroup reduction).
 * Replaces clip_grad.py:50-117 (_get_total_norm, norm_type 2) and :165-169.
 *   d_norm  <- fp32(sqrt(sum of g*g over every grad)), summed in float64;
 *   d_coef  <- min(max_norm * (1 / (norm + 1e-6)), 1) in fp32 (NaN propagates).
 * `d_partials` holds MI_ADAMW_MAX_NORM_BLOCKS doubles of scratch.  The
 * partial-sum assignment is fixed, so the result is bitwise reproducible. */
int mi_adamw_grad_norm(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                       int64_t n_chunks, int64_t chunk_elems, float max_norm,
                       double *d_partials, float *d_norm, float *d_coef, void *stream);

/* Same over one contiguous fp32 gradient range of n elements. */
int mi_adamw_grad_norm_flat(const float *d_grad, int64_t n, int64_t chunk_elems, float max_norm,
                            double *d_partials, float *d_norm, float *d_coef, void *stream);

/* Bytes of device scratch that mi_adamw_grad_norm_flat_noalloc uses on each GPU: one
 * float64 partial sum per workgroup of the norm pass, which never runs more than 512. */
#define MI_ADAMW_NOALLOC_SCRATCH_BYTES 4096

/* mi_adamw_grad_norm_flat without the d_partials workspace: allocates nothing, and
 * calls no hipMalloc, hipFree or allocating library routine.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * results as mi_adamw_grad_norm_flat, bit for bit.
 * The partial sums live in a static device array of MI_ADAMW_NOALLOC_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends; its device
 * address is looked up on the first call on each device.  Every call on one GPU
 * shares that array: calls that may overlap on one GPU (on different streams) race
 * and must be ordered by the caller.  Each call writes every partial it reads, so
 * nothing needs clearing between calls.  Any n is accepted (the pass runs at most
 * 512 workgroups); a launch needing more partials than the scratch holds would
 * return MI_ADAMW_E_SCRATCH.  The stream must belong to the current device
 * (MI_ADAMW_E_INVALID otherwise). */
int mi_adamw_grad_norm_flat_noalloc(const float *d_grad, int64_t n, int64_t chunk_elems,
                                    float max_norm, float *d_norm, float *d_coef, void *stream);

/* The clip split at the all-reduce, for ZeRO-1 range sharding (the flat layout cut into
 * one contiguous range per data-parallel rank).  Each rank sums the squares of its own
 * range's gradients into one float64 (8 bytes); the ranks' sums are all-reduced (or, on
 * one GPU, gathered) and every rank forms the same norm and coefficient from them.  This
 * replaces the per-tensor all-reduce + div_(world) of parallel/data_parallel.py:14-15
 * followed by clip_grad.py:50-117 and :165-169, with the world-size division folded in
 * as a gradient pre-scale.
 *
 * grad_prescale: every gradient is first multiplied by this fp32 factor, rounding once,
 * which is what `grad.div_(world)` stores on the GPU (torch divides a tensor by a host
 * scalar as a multiply by f32(1 / world)); 1 leaves the gradients as they are.
 *
 * mi_adamw_grad_sumsq / _flat: *d_sumsq <- float64 sum of (grad_prescale * g)^2 over the
 * tables' chunks or the range, reduced from MI_ADAMW_MAX_NORM_BLOCKS doubles of scratch at
 * d_partials in a fixed order (bitwise reproducible).
 * mi_adamw_norm_from_sumsq: d_sumsq[0..n) summed in a fixed order (1 <= n <=
 * MI_ADAMW_MAX_NORM_BLOCKS), then the norm and coefficient exactly as mi_adamw_grad_norm
 * forms them.  With n == 1 and the sum of one range, the result equals mi_adamw_grad_norm
 * over that range bit for bit. */
int mi_adamw_grad_sumsq(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                        int64_t n_chunks, int64_t chunk_elems, float grad_prescale,
                        double *d_partials, double *d_sumsq, void *stream);
int mi_adamw_grad_sumsq_flat(const float *d_grad, int64_t n, int64_t chunk_elems,
                             float grad_prescale, double *d_partials, double *d_sumsq,
                             void *stream);
int mi_adamw_norm_from_sumsq(const double *d_sumsq, int32_t n, float max_norm, float *d_norm,
                             float *d_coef, void *stream);

/* New gradient pointers for rows of a device tensor table of n_rows rows: row rows[i]
 * gets grads[i], and its MI_ADAMW_T_VEC flag set if vec[i] is non-zero, cleared if not
 * (the caller sets vec[i] when every pointer of the row, the new gradient included, is
 * aligned for the vector path).  For the step after zero_grad() freed the gradients and
 * backward allocated new ones (main.py:204-209): only the gradient column of the table
 * changes.  rows, grads and vec are host arrays of n entries, carried to the device as
 * kernel arguments, so they may be reused as soon as the call returns.  Each row may
 * appear at most once (MI_ADAMW_E_INVALID otherwise, as for a row outside [0, n_rows)).
 * Ordered on the stream like every other call: launches queued earlier on it still see
 * the old rows. */
int mi_adamw_set_grads(mi_adamw_tensor *d_tensors, int32_t n_rows, int32_t n, const int32_t *rows,
                       const uint64_t *grads, const uint8_t *vec, void *stream);

/* Multiply every gradient of the tables by *d_coef in place.
 * Replaces clip_grad.py:170-183 (_clip_grads_with_norm_'s foreach mul). */
int mi_adamw_scale_grads(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                         int64_t n_chunks, int64_t chunk_elems, const float *d_coef,
                         void *stream);

/* bf16 -> fp32 of every tensor of the tables in one launch: for each row,
 * param[i] = (float)param_copy[i] (param_copy holds the bf16 source, param the fp32
 * destination), exact.  Replaces one Tensor.to(torch.float32) per weight: the
 * backward of the bf16 cast that autocast applies to every linear weight in
 * mini-megatron's --amp forward (main.py:93; F.linear at
 * parallel/tensor_parallel.py:55,79), which widens each bf16 weight gradient for its
 * fp32 master.  mi_adamw.bf16_weights, which replaces the forward cast, widens all
 * of them with this one launch.  MI_ADAMW_T_VEC: param 16-byte and param_copy 8-byte
 * aligned. */
int mi_adamw_widen_bf16(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                        int64_t n_chunks, int64_t chunk_elems, void *stream);

/* The fused AdamW update over every chunk of the tables (one launch).
 * Replaces the per-tensor loop body of adam.py:396-547.
 * hypers: host array of n_hyper (<= MI_ADAMW_MAX_HYPER) sets, indexed by
 * mi_adamw_tensor.hyper.  d_grad_scale: device fp32 scalar, read with
 * MI_ADAMW_F_CLIP (normally d_coef of mi_adamw_grad_norm on the same stream).
 * state_dtype: MI_ADAMW_STATE_*.  flags: MI_ADAMW_F_*.
 * max_blocks: upper bound on workgroups (0 = one per chunk). */
int mi_adamw_step(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                  int64_t n_chunks, int64_t chunk_elems, const mi_adamw_hyper *hypers,
                  int32_t n_hyper, const float *d_grad_scale, int32_t state_dtype,
                  int32_t flags, int32_t max_blocks, void *stream);

/* The fused AdamW update over one contiguous range of n elements (the
 * flat-buffer layout; replaces the owned-parameter step of
 * parallel/distributed_optimizer.py:36-37).  `t` is a host struct whose
 * pointers are device pointers; t->hyper is ignored (hyper is the one set). */
int mi_adamw_step_flat(const mi_adamw_tensor *t, const mi_adamw_hyper *hyper,
                       const float *d_grad_scale, int64_t chunk_elems, int32_t state_dtype,
                       int32_t flags, int32_t max_blocks, void *stream);

/* mi_adamw_step and mi_adamw_step_flat with the gradient pre-scale of
 * mi_adamw_grad_sumsq: every gradient is multiplied by grad_prescale (one fp32 rounding),
 * then by *d_grad_scale with MI_ADAMW_F_CLIP, as torch's div_(world), clip and AdamW do in
 * turn.  With MI_ADAMW_F_WRITE_GRAD the stored gradient is the pre-scaled, clipped one.
 * The flat variant is the owned-range step of a ZeRO-1 rank: its range may cut through
 * tensors (the element chain does not depend on tensor boundaries). */
int mi_adamw_step_prescaled(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                            int64_t n_chunks, int64_t chunk_elems, const mi_adamw_hyper *hypers,
                            int32_t n_hyper, const float *d_grad_scale, float grad_prescale,
                            int32_t state_dtype, int32_t flags, int32_t max_blocks,
                            void *stream);
int mi_adamw_step_flat_prescaled(const mi_adamw_tensor *t, const mi_adamw_hyper *hyper,
                                 const float *d_grad_scale, float grad_prescale,
                                 int64_t chunk_elems, int32_t state_dtype, int32_t flags,
                                 int32_t max_blocks, void *stream);

/* The fused AdamW update of torch's capturable chain (adam.py:480-527) over
 * every chunk of the tables, for a step that may be recorded into a HIP graph:
 * no argument depends on the step count.  hypers: host array of n_hyper
 * (<= MI_ADAMW_MAX_HYPER) groups, indexed by mi_adamw_tensor.hyper.
 * d_steps: device fp32 step counts, already incremented for this step
 * (adam.py:414); d_step_index: device int32 array, one entry per row of the
 * tensor table, giving the row's index into d_steps.  The other arguments are
 * those of mi_adamw_step. */
int mi_adamw_step_capturable(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                             int64_t n_chunks, int64_t chunk_elems,
                             const mi_adamw_capt_hyper *hypers, int32_t n_hyper,
                             const float *d_steps, const int32_t *d_step_index,
                             const float *d_grad_scale, int32_t state_dtype, int32_t flags,
                             int32_t max_blocks, void *stream);

/* The same step as mi_adamw_step_capturable (torch's capturable chain, adam.py:480-527,
 * for a step recorded into a HIP graph), with the per-step values formed once per table
 * row instead of in every workgroup: a first launch forms each row's values (two powf,
 * three divisions, from the row's device step count, by the code the update would run)
 * into d_row_scalars, and the update reads them there.  Both launches go on `stream`, so
 * a graph that records the call records both.  Same results bit for bit; the update no
 * longer waits on that prologue, which bounds mi_adamw_step_capturable's update when the
 * moments are bf16.  d_row_scalars: device memory of n_rows * MI_ADAMW_ROW_SCALAR_BYTES
 * bytes, 16-byte aligned, provided by the caller and overwritten by every call (calls
 * that overlap on one buffer race); n_rows: the rows of d_tensors, above every chunk's
 * `tensor` (the update reads the slot of that row).  The other arguments are those of
 * mi_adamw_step_capturable. */
#define MI_ADAMW_ROW_SCALAR_BYTES 64
int mi_adamw_step_capturable_rows(const mi_adamw_tensor *d_tensors, int32_t n_rows,
                                  const mi_adamw_chunk *d_chunks, int64_t n_chunks,
                                  int64_t chunk_elems, const mi_adamw_capt_hyper *hypers,
                                  int32_t n_hyper, const float *d_steps,
                                  const int32_t *d_step_index, void *d_row_scalars,
                                  const float *d_grad_scale, int32_t state_dtype, int32_t flags,
                                  int32_t max_blocks, void *stream);

/* The fused AdamW update in torch's fused=True chain (mi_adamw_fused_hyper) over
 * every chunk of the tables, or over one contiguous range (_flat).  Replaces
 * torch._fused_adamw_ (adam.py:878-895) for torch.optim.AdamW(fused=True), which the
 * reference builds with --fused (main.py:144,177).  hypers: host array of n_hyper
 * (<= MI_ADAMW_MAX_HYPER) sets, indexed by mi_adamw_tensor.hyper.  d_steps and
 * d_step_index: both NULL (each set's step count is hypers[i].step), or, as in
 * mi_adamw_step_capturable, device fp32 step counts already incremented for this step
 * and one int32 index into them per row of the tensor table (the launch may then be
 * recorded into a HIP graph).  grad_prescale, d_grad_scale, state_dtype, flags and
 * max_blocks are those of mi_adamw_step_prescaled; amsgrad's running maximum is
 * fmaxf(max_exp_avg_sq, exp_avg_sq), as ::max in that kernel.  In the flat variant
 * `t` is a host struct of device pointers, t->hyper is ignored and the step count is
 * hyper->step. */
int mi_adamw_step_fused_chain(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                              int64_t n_chunks, int64_t chunk_elems,
                              const mi_adamw_fused_hyper *hypers, int32_t n_hyper,
                              const float *d_steps, const int32_t *d_step_index,
                              const float *d_grad_scale, float grad_prescale,
                              int32_t state_dtype, int32_t flags, int32_t max_blocks,
                              void *stream);
int mi_adamw_step_flat_fused_chain(const mi_adamw_tensor *t, const mi_adamw_fused_hyper *hyper,
                                   const float *d_grad_scale, float grad_prescale,
                                   int64_t chunk_elems, int32_t state_dtype, int32_t flags,
                                   int32_t max_blocks, void *stream);

/* mi_adamw_step_fused_chain with device step counts (d_steps, d_step_index required),
 * the per-step values formed once per table row instead of in every workgroup, as
 * mi_adamw_step_capturable_rows does for the capturable chain: a first launch forms each
 * row's values (two float64 pow and the divisions, by the code the update would run) into
 * d_row_scalars (n_rows * MI_ADAMW_ROW_SCALAR_BYTES bytes, 16-byte aligned, overwritten by
 * every call), and the update reads them there.  Same results bit for bit.  Replaces, as
 * mi_adamw_step_fused_chain does, torch._fused_adamw_ (adam.py:878-895) for
 * torch.optim.AdamW(fused=True, capturable=True). */
int mi_adamw_step_fused_chain_rows(const mi_adamw_tensor *d_tensors, int32_t n_rows,
                                   const mi_adamw_chunk *d_chunks, int64_t n_chunks,
                                   int64_t chunk_elems, const mi_adamw_fused_hyper *hypers,
                                   int32_t n_hyper, const float *d_steps,
                                   const int32_t *d_step_index, void *d_row_scalars,
                                   const float *d_grad_scale, float grad_prescale,
                                   int32_t state_dtype, int32_t flags, int32_t max_blocks,
                                   void *stream);

/* Measurement helper with no counterpart in the reference, for benchmarks that want
 * the memory ceiling of the update on the tensors it actually runs on: the same
 * launch as mi_adamw_step / mi_adamw_step_flat (tables or one flat range, launch
 * shape, access widths, cache hints, software pipelining) with the arithmetic left
 * out.  Every loaded value is stored back unchanged and the bf16 copy is written as
 * the bf16 of its master (equal to what the step leaves there), so the bytes moved
 * are exactly the step's and the tensors keep their values.  MI_ADAMW_F_CLIP is
 * accepted and ignored (the gradient is read either way); the other flags select
 * the same streams as in the step. */
int mi_adamw_probe(const mi_adamw_tensor *d_tensors, const mi_adamw_chunk *d_chunks,
                   int64_t n_chunks, int64_t chunk_elems, int32_t state_dtype, int32_t flags,
                   int32_t max_blocks, void *stream);
int mi_adamw_probe_flat(const mi_adamw_tensor *t, int64_t chunk_elems, int32_t state_dtype,
                        int32_t flags, int32_t max_blocks, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_ADAMW_H */
