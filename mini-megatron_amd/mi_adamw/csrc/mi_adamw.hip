// mi_adamw.hip -- fused clip + AdamW optimizer step for MI355X (gfx950).
//
// Kernels (all HBM-streaming, no MFMA: the step is ~15 fp32 ops per 22-34 bytes):
//   mi_adamw_sumsq_kernel  pass 1 of the clip: float64 sum of g*g over every
//                          gradient, reduced wave (shuffle) -> LDS -> one
//                          partial per workgroup; it walks the chunks last to
//                          first, and the last 256 MB it reads (the first the
//                          update reads) stay in the Infinity Cache for pass 2;
//   mi_adamw_norm_finalize_kernel  one workgroup reduces the partials in a fixed
//                          order and writes the norm and the clip coefficient
//                          to device memory (no host sync).
//   mi_adamw_update_kernel pass 2: p, g, m, v streamed with dwordx4 loads and
//                          stores, the AdamW op chain in fp32 registers, optional
//                          bf16 moments, bf16 model copy, gradient write-back and
//                          amsgrad's running maximum of v.  Three chains: torch's
//                          default one (per-step scalars from the host), its
//                          capturable one (per-step scalars formed per workgroup
//                          from a device step count, for HIP graph capture) and
//                          its fused=True one (_fused_adamw_: float64 scalars and
//                          float64 moment updates, per-step values formed per
//                          workgroup from the step count).
//   mi_adamw_scale_kernel  g *= coef in place (clip_grad_norm_'s write-back).
//   mi_adamw_widen_kernel  bf16 -> fp32 of many tensors in one launch (the backward of
//                          the bf16 weight copies the forward runs on), exact.
//   mi_adamw_update_kernel<..., ProbeHyper, ...>  the update's memory traffic without its
//                          arithmetic, values stored back unchanged (a measurement twin).
//
// Every launch walks a chunk table (one entry per `chunk_elems` slice of a
// tensor) so that all parameter tensors go through one launch, or one
// contiguous range in the flat-buffer layout.
//
// The default element math follows torch's per-op chain (torch/optim/adam.py:419-547)
// with one fp32 rounding per ATen op; the fused=True chain follows adam_math of
// ATen/native/hip/fused_adam_utils.cuh.  The file is compiled with
// -ffp-contract=off; each fused multiply-add below is explicit and sits where
// torch-ROCm's own kernels fuse (lerp, addcmul, addcdiv; in the fused chain the
// float64 moment sums and the weight decay).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string.h>

#include <atomic>
#include <cmath>
#include <mutex>
#include <vector>

#include "mi_adamw.h"
#include "fp32_math.h"   // bf16x2_bits, bf16_bits, div_by_recip

namespace {

constexpr int kVec = 4;                       // fp32 elements per lane per access (dwordx4)
// Norm pass: 256-thread workgroups (4 wave64), four 1024-element tiles per
// 4096-element chunk, so a workgroup has four dwordx4 loads per lane in flight.
constexpr int kNormThreads = 256;
constexpr int kNormTile = kNormThreads * kVec;
// Update: 1024-thread workgroups (16 wave64), one 4096-element tile per chunk.
// Measured on MI355X: a whole chunk per tile (each workgroup issues all its
// loads at once and retires) streams 3-4% faster than 256-thread workgroups
// looping over four tiles.
constexpr int kUpdThreads = 1024;
constexpr int kUpdTile = kUpdThreads * kVec;
constexpr int kChunkQuantum = kUpdTile;       // chunk sizes are multiples of this
static_assert(kChunkQuantum == MI_ADAMW_CHUNK_QUANTUM, "header and kernels agree");

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct HyperPack {
    mi_adamw_hyper h[MI_ADAMW_MAX_HYPER];
};

static_assert(sizeof(mi_adamw_tensor) == 64, "mi_adamw_tensor is read as 8 words");
static_assert(offsetof(mi_adamw_tensor, max_exp_avg_sq) == 40 &&
              offsetof(mi_adamw_tensor, numel) == 48, "pointer words, then numel");
static_assert(offsetof(mi_adamw_tensor, hyper) == 56 && offsetof(mi_adamw_tensor, flags) == 60,
              "hyper and flags share the last word");
static_assert(sizeof(mi_adamw_chunk) == 8, "mi_adamw_chunk is two int32");
static_assert(sizeof(mi_adamw_capt_hyper) == 48 && offsetof(mi_adamw_capt_hyper, lr_ptr) == 40,
              "mi_adamw_capt_hyper: ten 4-byte fields, then the lr pointer");
static_assert(sizeof(mi_adamw_fused_hyper) == 56 && offsetof(mi_adamw_fused_hyper, step) == 40 &&
                  offsetof(mi_adamw_fused_hyper, lr_ptr) == 48,
              "mi_adamw_fused_hyper: five doubles, two floats, then the lr pointer");

// ---------------------------------------------------------------------------
// Element math

__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// Lerp.h:21-35, fp32 opmath, fused the way torch-ROCm compiles it.
__device__ __forceinline__ float lerp_fused(float self, float end, float w) {
    float diff = end - self;
    if (__builtin_fabsf(w) < 0.5f) return __builtin_fmaf(w, diff, self);
    return __builtin_fmaf(-diff, 1.0f - w, end);
}

// torch.maximum(a, b): NaN if either operand is NaN (a first), else the larger,
// a on ties.
__device__ __forceinline__ float maximum_nan(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    return a < b ? b : a;
}

// The scalars one workgroup's element chain uses.  Default chain: the host's
// per-step values (mi_adamw_hyper).  Capturable chain (kCapt): den_scale is
// sqrt(bc2) * -step_size, divided by, and den_add is eps / -step_size.
struct ElemScalars {
    float wd_factor;
    float lerp_w;
    float beta2;
    float one_minus_beta2;
    float den_scale;       // 1 / bc2_sqrt (multiplied), or sqrt(bc2) * -step_size (divided by)
    float den_add;         // eps, or eps / -step_size
    float neg_step_size;   // default chain only
    float grad_sign;
    float inv_den_scale;   // capturable chain: 1.0f / den_scale, when den_recip
    int32_t den_recip;     // capturable chain: den_scale in div_by_neg_recip's range
};

// One element of adam.py:419-547.  g already carries the clip scale and sign.
// With kAms, x is amsgrad's running maximum of v and the denominator uses it.
template <bool kAms, bool kCapt>
__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float& x,
                                           const ElemScalars& h) {
    p = p * h.wd_factor;                                   // adam.py:419 mul_
    m = lerp_fused(m, g, h.lerp_w);                        // adam.py:457 lerp_
    v = v * h.beta2;                                       // adam.py:476 mul_
    v = __builtin_fmaf(h.one_minus_beta2, g * g, v);       // adam.py:476 addcmul_
    float dv = v;
    if (kAms) {
        x = maximum_nan(x, v);                             // adam.py:512/540 maximum
        dv = x;
    }
    float d = __builtin_sqrtf(dv);                         // adam.py:520/545 sqrt
    if (kCapt) {
        // adam.py:520-521 / (bc2_sqrt * -step_size): the correctly rounded quotient, from the
        // workgroup's reciprocal when den_scale is in range (fp32_math.h), else divided
        d = h.den_recip ? div_by_neg_recip(d, h.den_scale, h.inv_den_scale) : d / h.den_scale;
        d = d + h.den_add;                                 // adam.py:522 add_(eps / -step_size)
        p = p + m / d;                                     // adam.py:527 addcdiv_, value 1
    } else {
        d = d * h.den_scale;                               //   / bc2_sqrt (reciprocal mul)
        d = d + h.den_add;                                 //   add_(eps)
        p = __builtin_fmaf(h.neg_step_size, m / d, p);     // adam.py:547 addcdiv_
    }
}

// The scalars of torch's fused=True chain for one workgroup (FusedHyper): the float64
// hyperparameters as _fused_adamw_ receives them, and the per-step values it forms.
// kRecip: the quotient by bc2_sqrt is formed from its reciprocal (div_by_recip), which
// gives the division's bits; without it, by the division itself.  The host-step chain
// and the per-row chain (FusedRowsHyper) take kRecip: their per-step values are kernel
// arguments or scalar loads, so the reciprocal costs no vector register.  The device-step
// chain that forms them in every workgroup does so after two out-of-line pow calls with
// the first tile's loads in flight, where one more value spills, so it divides.
template <bool kRecip>
struct FusedScalarsT {
    double beta1, one_minus_beta1;
    double beta2, one_minus_beta2;
    double lr_wd;          // lr * weight_decay
    double eps;
    float step_size;       // f32(lr / (double)f32(1 - beta1^step))
    float bc2_sqrt;        // f32(sqrt(1 - beta2^step))
    float inv_bc2_sqrt;    // kRecip: 1.0f / bc2_sqrt, correctly rounded
    float grad_sign;
    bool decay;            // weight_decay != 0
};

// One element of adam_math (fused_adam_utils.cuh, ADAMW mode): m, v and the decayed
// p are float64 expressions of fp32 values, each rounded once to fp32; the contractions
// are those of torch-ROCm's build of that kernel (the left product of each sum fused).
// ::max there is fmaxf.  g already carries the clip scale and sign.
template <bool kAms, bool kCapt, bool kRecip>
__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float& x,
                                           const FusedScalarsT<kRecip>& h) {
    if (h.decay)                                           // param -= lr * wd * param
        p = static_cast<float>(__builtin_fma(-h.lr_wd, double(p), double(p)));
    const double dg = g;
    m = static_cast<float>(__builtin_fma(h.beta1, double(m), h.one_minus_beta1 * dg));
    v = static_cast<float>(__builtin_fma(h.beta2, double(v), (h.one_minus_beta2 * dg) * dg));
    float dv = v;
    if (kAms) {
        x = __builtin_fmaxf(x, v);
        dv = x;
    }
    // fp32 sqrt, then the correctly rounded fp32 quotient by bc2_sqrt (div_by_recip gives
    // the division's bits for every value sqrtf can give here, fp32_math.h)
    const float s = __builtin_sqrtf(dv);
    float q;
    if constexpr (kRecip) q = div_by_recip(s, h.bc2_sqrt, h.inv_bc2_sqrt);
    else q = s / h.bc2_sqrt;
    const float d = static_cast<float>(double(q) + h.eps); // + eps in float64
    p = p - (h.step_size * m) / d;                         // fp32
}

// ---------------------------------------------------------------------------
// Streaming loads and stores.  The update touches every value once per step, so
// its loads and stores carry the nontemporal hint (measured: ordinary ones make
// the update 6-15% slower).  Only the gradients are read twice, by the norm pass
// and then by the update; see ld4_norm.  Tensor pointers come out of the tensor
// table, so the compiler cannot tell they are global memory; the casts to
// address space 1 make it emit global_load/global_store (vmcnt only) instead of
// flat accesses.

#define GLOBAL __attribute__((address_space(1)))

__device__ __forceinline__ f32x4 ld4(const float* p) {
    return __builtin_nontemporal_load((const GLOBAL f32x4*)(p));
}
// Norm-pass loads.  kKeep: an ordinary load, which allocates the line in the
// memory-side cache (MI355X Infinity Cache), so that the update pass right after
// finds it there; otherwise a streaming (nontemporal) load.
template <bool kKeep>
__device__ __forceinline__ f32x4 ld4_norm(const float* p) {
    if (kKeep) return *(const GLOBAL f32x4*)(p);
    return __builtin_nontemporal_load((const GLOBAL f32x4*)(p));
}
__device__ __forceinline__ void st4(float* p, f32x4 v) {
    __builtin_nontemporal_store(v, (GLOBAL f32x4*)(p));
}
__device__ __forceinline__ float ld1(const float* p) { return *(const GLOBAL float*)(p); }
__device__ __forceinline__ void st1(float* p, float v) { *(GLOBAL float*)(p) = v; }
__device__ __forceinline__ uint32_t ld1_u16(const uint16_t* p) {
    return *(const GLOBAL uint16_t*)(p);
}
__device__ __forceinline__ void st1_u16(uint16_t* p, uint32_t v) {
    *(GLOBAL uint16_t*)(p) = static_cast<uint16_t>(v);
}
__device__ __forceinline__ f32x4 ld4_bf16(const uint16_t* p) {
    u32x2 w = __builtin_nontemporal_load((const GLOBAL u32x2*)(p));
    f32x4 r;
    r.x = __uint_as_float(w.x << 16);
    r.y = __uint_as_float(w.x & 0xffff0000u);
    r.z = __uint_as_float(w.y << 16);
    r.w = __uint_as_float(w.y & 0xffff0000u);
    return r;
}
__device__ __forceinline__ void st4_bf16(uint16_t* p, f32x4 v) {
    u32x2 w;
    w.x = bf16x2_bits(v.x, v.y);
    w.y = bf16x2_bits(v.z, v.w);
    __builtin_nontemporal_store(w, (GLOBAL u32x2*)(p));
}

// adamw_elem on the four lanes of a dwordx4 group (H: ElemScalars or FusedScalarsT).
template <bool kAms, bool kCapt, class H>
__device__ __forceinline__ void adamw_vec(f32x4& p, f32x4 g, f32x4& m, f32x4& v, f32x4& x,
                                          const H& h) {
    float p0 = p.x, p1 = p.y, p2 = p.z, p3 = p.w;
    float m0 = m.x, m1 = m.y, m2 = m.z, m3 = m.w;
    float v0 = v.x, v1 = v.y, v2 = v.z, v3 = v.w;
    float x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
    adamw_elem<kAms, kCapt>(p0, g.x, m0, v0, x0, h);
    adamw_elem<kAms, kCapt>(p1, g.y, m1, v1, x1, h);
    adamw_elem<kAms, kCapt>(p2, g.z, m2, v2, x2, h);
    adamw_elem<kAms, kCapt>(p3, g.w, m3, v3, x3, h);
    p = f32x4{p0, p1, p2, p3};
    m = f32x4{m0, m1, m2, m3};
    v = f32x4{v0, v1, v2, v3};
    if (kAms) x = f32x4{x0, x1, x2, x3};
}

template <typename S> struct StateIO;
template <> struct StateIO<float> {
    static __device__ __forceinline__ f32x4 ld(const void* b, int64_t i) {
        return ld4(static_cast<const float*>(b) + i);
    }
    static __device__ __forceinline__ void st(void* b, int64_t i, f32x4 v) {
        st4(static_cast<float*>(b) + i, v);
    }
    static __device__ __forceinline__ float ld1(const void* b, int64_t i) {
        return ::ld1(static_cast<const float*>(b) + i);
    }
    static __device__ __forceinline__ void st1(void* b, int64_t i, float v) {
        ::st1(static_cast<float*>(b) + i, v);
    }
};
template <> struct StateIO<uint16_t> {
    static __device__ __forceinline__ f32x4 ld(const void* b, int64_t i) {
        return ld4_bf16(static_cast<const uint16_t*>(b) + i);
    }
    static __device__ __forceinline__ void st(void* b, int64_t i, f32x4 v) {
        st4_bf16(static_cast<uint16_t*>(b) + i, v);
    }
    static __device__ __forceinline__ float ld1(const void* b, int64_t i) {
        return bf16_to_f32(ld1_u16(static_cast<const uint16_t*>(b) + i));
    }
    static __device__ __forceinline__ void st1(void* b, int64_t i, float v) {
        st1_u16(static_cast<uint16_t*>(b) + i, bf16_bits(v));
    }
};

// ---------------------------------------------------------------------------
// Work sources: where chunk c of a launch lives.

#define CONSTANT __attribute__((address_space(4)))

// The tables do not change while a launch runs, so they are read through the
// constant address space: the compiler then fetches a chunk entry and its
// tensor row with scalar loads (s_load), keeps the tensor's base pointers in
// SGPRs and addresses the streams as SGPR base + VGPR offset.
struct TableSource {
    const mi_adamw_tensor* tensors;
    const mi_adamw_chunk* chunks;
    __device__ __forceinline__ void get(int64_t c, int64_t chunk_elems, mi_adamw_tensor& t,
                                        int64_t& begin, int64_t& end, int32_t& row) const {
        const CONSTANT int32_t* ck = (const CONSTANT int32_t*)(chunks + c);
        row = ck[0];
        const int32_t index = ck[1];
        // mi_adamw_tensor is 8 eight-byte words: 6 pointers, numel, (hyper, flags).
        const CONSTANT uint64_t* w = (const CONSTANT uint64_t*)(tensors + row);
        t.param = reinterpret_cast<float*>(w[0]);
        t.grad = reinterpret_cast<float*>(w[1]);
        t.exp_avg = reinterpret_cast<void*>(w[2]);
        t.exp_avg_sq = reinterpret_cast<void*>(w[3]);
        t.param_copy = reinterpret_cast<uint16_t*>(w[4]);
        t.max_exp_avg_sq = reinterpret_cast<void*>(w[5]);
        t.numel = static_cast<int64_t>(w[6]);
        t.hyper = static_cast<int32_t>(w[7] & 0xffffffffu);
        t.flags = static_cast<int32_t>(w[7] >> 32);
        begin = static_cast<int64_t>(index) * chunk_elems;
        end = begin + chunk_elems < t.numel ? begin + chunk_elems : t.numel;
    }
};

struct FlatSource {
    mi_adamw_tensor t;
    __device__ __forceinline__ void get(int64_t c, int64_t chunk_elems, mi_adamw_tensor& out,
                                        int64_t& begin, int64_t& end, int32_t& row) const {
        out = t;
        row = 0;
        begin = c * chunk_elems;
        end = begin + chunk_elems < t.numel ? begin + chunk_elems : t.numel;
    }
};

// ---------------------------------------------------------------------------
// Per-step scalars: where a workgroup's ElemScalars come from.

// Default chain: the host formed every per-step value (adam.py:529-536).
struct StaticHyper {
    using Scalars = ElemScalars;
    static constexpr bool kCapt = false;
    static constexpr bool kLate = false;
    static constexpr bool kProbe = false;
    static constexpr bool kShare = false;
    HyperPack hp;
    __device__ __forceinline__ ElemScalars get(const mi_adamw_tensor& t, int32_t) const {
        const mi_adamw_hyper& x = hp.h[t.hyper];
        return ElemScalars{x.wd_factor, x.lerp_w, x.beta2, x.one_minus_beta2,
                           x.inv_bc2_sqrt, x.eps, x.neg_step_size, x.grad_sign};
    }
};

struct CaptPack {
    mi_adamw_capt_hyper h[MI_ADAMW_MAX_HYPER];
};

// Capturable chain: adam.py:480-522 from the tensor's device step count, in
// fp32 with one rounding per ATen op (powf is the device pow torch-ROCm's pow
// kernel calls; `float / tensor` is a reciprocal times the float).  The step
// counts and a device lr were written by earlier work on the stream and do not
// change during the launch, so they are read through the constant address
// space (scalar loads).
struct CaptHyper {
    using Scalars = ElemScalars;
    static constexpr bool kCapt = true;
    static constexpr bool kLate = true;
    static constexpr bool kProbe = false;
    static constexpr bool kShare = true;
    CaptPack cp;
    const float* steps;
    const int32_t* step_index;
    __device__ __forceinline__ ElemScalars get(const mi_adamw_tensor& t, int32_t row) const {
        const mi_adamw_capt_hyper& c = cp.h[t.hyper];
        const int32_t slot = *((const CONSTANT int32_t*)(step_index) + row);
        const float step = *((const CONSTANT float*)(steps) + slot);
        const float bc1 = 1.0f - powf(c.beta1, step);                 // adam.py:488
        const float bc2 = 1.0f - powf(c.beta2, step);                 // adam.py:497
        float lr = c.lr;
        float wd_factor = c.wd_factor;
        if (c.lr_mode == MI_ADAMW_LR_DEVICE) {
            lr = *(const CONSTANT float*)(c.lr_ptr);
            // adam.py:419 with a tensor lr: 1 - lr * weight_decay, two fp32 ops
            wd_factor = c.weight_decay != 0.0f ? 1.0f - lr * c.weight_decay : 1.0f;
        }
        // adam.py:499: lr / bc1; a float lr divides as (1 / bc1) * lr
        const float step_size = c.lr_mode == MI_ADAMW_LR_FLOAT ? (1.0f / bc1) * lr : lr / bc1;
        const float neg = -step_size;                                 // adam.py:500
        const float bc2_sqrt = __builtin_sqrtf(bc2);                  // adam.py:502
        ElemScalars h;
        h.wd_factor = wd_factor;
        h.lerp_w = c.lerp_w;
        h.beta2 = c.beta2;
        h.one_minus_beta2 = c.one_minus_beta2;
        h.den_scale = bc2_sqrt * neg;                                 // adam.py:521
        h.den_add = (1.0f / neg) * c.eps;                             // adam.py:522 eps / neg
        h.neg_step_size = 0.0f;
        h.grad_sign = c.grad_sign;
        h.den_recip = neg_recip_in_range(h.den_scale);
        h.inv_den_scale = h.den_recip ? 1.0f / h.den_scale : 0.0f;
        return h;
    }
};

// The capturable chain's per-step values formed once per table row
// (mi_adamw_step_capturable_rows): a first launch runs CaptHyper::get for every row, one
// thread per row, and the update reads its row's values with scalar loads, as the default
// chain reads its kernel arguments, instead of forming them in every workgroup.
struct alignas(16) RowScalars {
    ElemScalars s;
    uint8_t pad[MI_ADAMW_ROW_SCALAR_BYTES - sizeof(ElemScalars)];
};
static_assert(sizeof(RowScalars) == MI_ADAMW_ROW_SCALAR_BYTES, "one row's values per slot");

__global__ __launch_bounds__(256) void mi_adamw_capt_rows_kernel(
    const mi_adamw_tensor* __restrict__ rows, int32_t n_rows, CaptHyper hs,
    RowScalars* __restrict__ out) {
    const int32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= n_rows) return;
    out[r].s = hs.get(rows[r], r);
}

struct CaptRowsHyper {
    using Scalars = ElemScalars;
    static constexpr bool kCapt = true;
    static constexpr bool kLate = true;
    static constexpr bool kProbe = false;
    static constexpr bool kShare = false;
    const RowScalars* rows;
    __device__ __forceinline__ ElemScalars get(const mi_adamw_tensor&, int32_t row) const {
        // written by the launch before this one on the stream: read word by word through
        // the constant address space, so the loads are scalar
        static_assert(sizeof(ElemScalars) % 4 == 0, "read as 32-bit words");
        const CONSTANT uint32_t* w = (const CONSTANT uint32_t*)(rows + row);
        uint32_t v[sizeof(ElemScalars) / 4];
#pragma unroll
        for (unsigned k = 0; k < sizeof(ElemScalars) / 4; ++k) v[k] = w[k];
        ElemScalars s;
        memcpy(&s, v, sizeof(s));
        return s;
    }
};

// One set of the fused=True chain as the kernel takes it: the float64 hyperparameters
// and, with host step counts, the per-step values the library formed on the host from
// them (fused_set_from): both bias corrections, and with a host lr also lr_wd,
// step_size and inv_bc2_sqrt.
struct FusedSet {
    double beta1, one_minus_beta1;
    double beta2, one_minus_beta2;
    double lr, weight_decay, eps;
    float bc1;                   // f32(1 - pow(beta1, step))
    float bc2_sqrt;              // f32(sqrt(1 - pow(beta2, step)))
    float grad_sign;
    int32_t decay;               // weight_decay != 0
    const float* lr_ptr;         // device fp32 lr, or NULL
    // host step counts and a host lr: the per-step values of the workgroup prologue,
    // formed once on the host with the same correctly rounded IEEE operations
    double lr_wd;                // lr * weight_decay
    float step_size;             // f32(lr / (double)bc1)
    float inv_bc2_sqrt;          // 1.0f / bc2_sqrt
};

struct FusedPack {
    FusedSet h[MI_ADAMW_MAX_HYPER];
};

// pow in float64, out of line: inlined into the update it adds 10-15 VGPRs to every
// instance of the device-step chain.
__device__ __attribute__((noinline)) double pow_f64(double x, double y) { return pow(x, y); }

// torch's fused=True chain: the per-step values of fused_adam_utils.cuh
// FusedAdamMathFunctor, as adam_math's fp32 (opmath_t) parameters take them.
// bc1 and bc2_sqrt come from the set (host step counts) or, with kDevSteps, are formed
// here from the row's device step count with the device pow and sqrt, as that functor
// does; step_size = f32(lr / bc1) and lr * weight_decay are formed here in float64 in
// both cases, from the host lr or a device lr.  Device step counts and a device lr
// were written by earlier work on the stream and do not change during the launch, so
// they are read through the constant address space.
template <bool kDevSteps>
struct FusedHyper {
    using Scalars = FusedScalarsT<!kDevSteps>;
    static constexpr bool kCapt = false;
    static constexpr bool kLate = true;
    static constexpr bool kProbe = false;
    // every wave forms its own: with device step counts the two out-of-line float64 pow
    // calls in one wave's branch spill under this chain's 64-VGPR cap, and with host step
    // counts the prologue is a few loads
    static constexpr bool kShare = false;
    FusedPack fp;
    const float* steps;
    const int32_t* step_index;
    __device__ __forceinline__ Scalars get(const mi_adamw_tensor& t, int32_t row) const {
        const FusedSet& c = fp.h[t.hyper];
        float bc1 = c.bc1, bc2_sqrt = c.bc2_sqrt;
        if (kDevSteps) {
            const int32_t slot = *((const CONSTANT int32_t*)(step_index) + row);
            const double step = *((const CONSTANT float*)(steps) + slot);
            bc1 = static_cast<float>(1.0 - pow_f64(c.beta1, step));
            bc2_sqrt = static_cast<float>(sqrt(1.0 - pow_f64(c.beta2, step)));
        }
        Scalars s;
        s.beta1 = c.beta1;
        s.one_minus_beta1 = c.one_minus_beta1;
        s.beta2 = c.beta2;
        s.one_minus_beta2 = c.one_minus_beta2;
        s.eps = c.eps;
        s.bc2_sqrt = bc2_sqrt;
        s.grad_sign = c.grad_sign;
        s.decay = c.decay != 0;
        if (!kDevSteps && !c.lr_ptr) {
            // formed on the host (fused_set_from)
            s.lr_wd = c.lr_wd;
            s.step_size = c.step_size;
            s.inv_bc2_sqrt = c.inv_bc2_sqrt;
        } else {
            const double lr = c.lr_ptr ? double(*(const CONSTANT float*)(c.lr_ptr)) : c.lr;
            s.lr_wd = lr * c.weight_decay;
            s.step_size = static_cast<float>(lr / double(bc1));
            if (!kDevSteps) s.inv_bc2_sqrt = 1.0f / bc2_sqrt;
        }
        return s;
    }
};

// The fused=True chain's per-step values with device step counts formed once per table
// row (mi_adamw_step_fused_chain_rows): a first launch runs FusedHyper<true>::get for
// every row, one thread per row (two float64 pow, divisions), and keeps what depends on
// the step in the row's slot; the update reads it with scalar loads and takes the rest
// from the group's set, as with host step counts, and forms the quotient by bc2_sqrt from
// the reciprocal formed here (div_by_recip).
struct FusedRow {
    double lr_wd;              // lr * weight_decay
    float step_size;           // f32(lr / (double)bc1)
    float bc2_sqrt;            // f32(sqrt(1 - pow(beta2, step)))
    float inv_bc2_sqrt;        // 1.0f / bc2_sqrt
    float unused;
};
static_assert(sizeof(FusedRow) <= MI_ADAMW_ROW_SCALAR_BYTES, "one row's values per slot");

__global__ __launch_bounds__(256) void mi_adamw_fused_rows_kernel(
    const mi_adamw_tensor* __restrict__ rows, int32_t n_rows, FusedHyper<true> hs,
    RowScalars* __restrict__ out) {
    const int32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= n_rows) return;
    const FusedScalarsT<false> s = hs.get(rows[r], r);
    FusedRow f;
    f.lr_wd = s.lr_wd;
    f.step_size = s.step_size;
    f.bc2_sqrt = s.bc2_sqrt;
    f.inv_bc2_sqrt = 1.0f / s.bc2_sqrt;
    f.unused = 0.0f;
    memcpy(&out[r], &f, sizeof(f));
}

struct FusedRowsHyper {
    using Scalars = FusedScalarsT<true>;
    static constexpr bool kCapt = false;
    static constexpr bool kLate = true;
    static constexpr bool kProbe = false;
    static constexpr bool kShare = false;
    FusedPack fp;
    const RowScalars* rows;
    __device__ __forceinline__ Scalars get(const mi_adamw_tensor& t, int32_t row) const {
        const FusedSet& c = fp.h[t.hyper];
        // written by the launch before this one on the stream: read word by word through
        // the constant address space, so the loads are scalar
        static_assert(sizeof(FusedRow) % 4 == 0, "read as 32-bit words");
        const CONSTANT uint32_t* w = (const CONSTANT uint32_t*)(rows + row);
        uint32_t v[sizeof(FusedRow) / 4];
#pragma unroll
        for (unsigned k = 0; k < sizeof(FusedRow) / 4; ++k) v[k] = w[k];
        FusedRow f;
        memcpy(&f, v, sizeof(f));
        Scalars s;
        s.beta1 = c.beta1;
        s.one_minus_beta1 = c.one_minus_beta1;
        s.beta2 = c.beta2;
        s.one_minus_beta2 = c.one_minus_beta2;
        s.eps = c.eps;
        s.grad_sign = c.grad_sign;
        s.decay = c.decay != 0;
        s.lr_wd = f.lr_wd;
        s.step_size = f.step_size;
        s.bc2_sqrt = f.bc2_sqrt;
        s.inv_bc2_sqrt = f.inv_bc2_sqrt;
        return s;
    }
};

// Memory-only twin of the update, for measurement (mi_adamw_probe): the same
// loads and stores, launch shape and cache hints, with the arithmetic left out.
// Every value is stored back as it was read (the bf16 copy as the bf16 of the
// master, which the step keeps it equal to), so running it leaves the tensors
// unchanged.
struct ProbeHyper {
    using Scalars = ElemScalars;
    static constexpr bool kCapt = false;
    static constexpr bool kLate = false;
    static constexpr bool kProbe = true;
    static constexpr bool kShare = false;
    __device__ __forceinline__ ElemScalars get(const mi_adamw_tensor&, int32_t) const {
        return ElemScalars{};
    }
};

// Keeps a loaded value live without using it, so its load stays in the code.
__device__ __forceinline__ void keep(f32x4 v) {
    asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
}
__device__ __forceinline__ void keep(float v) { asm volatile("" ::"v"(v)); }

// ---------------------------------------------------------------------------
// Reductions

__device__ __forceinline__ double wave_sum(double x) {
    // wave64 butterfly; __shfl_xor moves the two 32-bit halves.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

// Sum over the workgroup; the result is valid in every lane of wave 0.
template <int kThreads>
__device__ __forceinline__ double block_sum(double x) {
    __shared__ double lds[kThreads / 64];
    x = wave_sum(x);
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if (lane == 0) lds[wave] = x;
    __syncthreads();
    double r = 0.0;
    if (wave == 0) {
        r = lane < kThreads / 64 ? lds[lane] : 0.0;
        r = wave_sum(r);
    }
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// Pass 1: float64 sum of squares and the clip coefficient.
//
// A fixed grid of at most kNormBlocks workgroups strides over the chunks:
// workgroup b sums chunks b, b + grid, b + 2*grid, ...  Small chunks (4096
// elements by default) keep every workgroup's share within one chunk of the
// others, and the fixed assignment makes the sum bitwise reproducible.  The
// next chunk's table entry is fetched before the current chunk's loads are
// consumed, so the scalar-load latency of the lookup overlaps the stream.

// The squares of pre*g, each product rounded to fp32 first: the value a caller's
// `grad.div_(world)` (parallel/data_parallel.py:15) would have stored.  pre == 1 leaves
// every gradient as it is (x * 1 == x).
__device__ __forceinline__ void sumsq4(f32x4 a, float pre, double& acc0, double& acc1) {
    const float x = a.x * pre, y = a.y * pre, z = a.z * pre, w = a.w * pre;
    acc0 += (double)x * x + (double)y * y;
    acc1 += (double)z * z + (double)w * w;
}

// Sum of squares over chunks c, c + stride, ... below c_end.  The next chunk's
// table entry is fetched while the current chunk's loads are in flight.  Returns
// the first chunk of the sequence at or past c_end.
template <bool kKeep, class Src>
__device__ __forceinline__ int64_t sumsq_chunks(const Src& src, int64_t c, int64_t c_end,
                                                int64_t stride, int64_t chunk_elems, float pre,
                                                double& acc0, double& acc1) {
    mi_adamw_tensor t;
    int64_t begin = 0, end = 0;
    int32_t row;
    if (c < c_end) src.get(c, chunk_elems, t, begin, end, row);
    for (; c < c_end; c += stride) {
        const float* __restrict__ g = t.grad;
        const bool vec = t.flags & MI_ADAMW_T_VEC;
        const int64_t vend = vec ? begin + ((end - begin) & ~static_cast<int64_t>(kVec - 1)) : begin;
        int64_t i = begin + threadIdx.x * kVec;
        // Issue the first four tiles of this chunk (a whole 4096-element chunk)...
        f32x4 a{}, b{}, d{}, e{};
        const bool full = i + 3 * kNormTile < vend;
        if (full) {
            a = ld4_norm<kKeep>(g + i);
            b = ld4_norm<kKeep>(g + i + kNormTile);
            d = ld4_norm<kKeep>(g + i + 2 * kNormTile);
            e = ld4_norm<kKeep>(g + i + 3 * kNormTile);
        }
        // ...then look up the next chunk while those loads are in flight; the
        // barrier keeps the scheduler from hoisting the lookup (and its waits)
        // above the vector loads.
        __builtin_amdgcn_sched_barrier(0);
        mi_adamw_tensor tn;
        int64_t bn = 0, en = 0;
        const bool more = c + stride < c_end;
        if (more) src.get(c + stride, chunk_elems, tn, bn, en, row);
        __builtin_amdgcn_sched_barrier(0);
        if (full) {
            sumsq4(a, pre, acc0, acc1);
            sumsq4(b, pre, acc0, acc1);
            sumsq4(d, pre, acc0, acc1);
            sumsq4(e, pre, acc0, acc1);
            i += 4 * kNormTile;
            for (; i + 3 * kNormTile < vend; i += 4 * kNormTile) {
                a = ld4_norm<kKeep>(g + i);
                b = ld4_norm<kKeep>(g + i + kNormTile);
                d = ld4_norm<kKeep>(g + i + 2 * kNormTile);
                e = ld4_norm<kKeep>(g + i + 3 * kNormTile);
                sumsq4(a, pre, acc0, acc1);
                sumsq4(b, pre, acc0, acc1);
                sumsq4(d, pre, acc0, acc1);
                sumsq4(e, pre, acc0, acc1);
            }
        }
        for (; i < vend; i += kNormTile) sumsq4(ld4_norm<kKeep>(g + i), pre, acc0, acc1);
        for (int64_t j = vend + threadIdx.x; j < end; j += kNormThreads) {
            const double x = ld1(g + j) * pre;
            acc0 += x * x;
        }
        if (more) {
            t = tn;
            begin = bn;
            end = en;
        }
    }
    return c;
}

// The chunks of a work source in reverse order: the norm pass walks the gradients from the
// last chunk to the first, so the chunks it reads last (kept in the memory-side cache) are
// the ones the update, which walks them from the first, reads first.
template <class Src>
struct ReverseSource {
    Src src;
    int64_t n_chunks;
    __device__ __forceinline__ void get(int64_t c, int64_t chunk_elems, mi_adamw_tensor& t,
                                        int64_t& begin, int64_t& end, int32_t& row) const {
        src.get(n_chunks - 1 - c, chunk_elems, t, begin, end, row);
    }
};

// Workgroup b sums chunks b, b + grid, b + 2*grid, ... of the reversed order: streaming
// loads below keep_from, ordinary loads from keep_from on (the last chunks the pass reads,
// the first ones the update reads, which then come from the memory-side cache: measured
// 0.2-0.6% off the update against keeping the chunks the update reads last, which its own
// traffic evicts first).  Two loops, not one with a per-chunk choice: the compiler would
// fold the two loads into one.
template <class Src>
__global__ __launch_bounds__(kNormThreads) void mi_adamw_sumsq_kernel(
    Src src, int64_t n_chunks, int64_t chunk_elems, double* __restrict__ partials,
    int64_t keep_from, float pre) {
    double acc0 = 0.0, acc1 = 0.0;
    int64_t c = blockIdx.x;
    const ReverseSource<Src> rev{src, n_chunks};
    c = sumsq_chunks<false>(rev, c, keep_from, gridDim.x, chunk_elems, pre, acc0, acc1);
    sumsq_chunks<true>(rev, c, n_chunks, gridDim.x, chunk_elems, pre, acc0, acc1);
    const double total = block_sum<kNormThreads>(acc0 + acc1);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// One workgroup: reduce the partial sums in a fixed order, then the norm and
// the clip coefficient.  Running as its own launch, it sees every partial
// through the kernel boundary; no fence or completion counter is needed.
__global__ __launch_bounds__(kNormThreads) void mi_adamw_norm_finalize_kernel(
    const double* __restrict__ partials, int n_partials, float max_norm,
    float* __restrict__ norm_out, float* __restrict__ coef_out) {
    double s = 0.0;
    for (int i = threadIdx.x; i < n_partials; i += kNormThreads) s += partials[i];
    s = block_sum<kNormThreads>(s);
    if (threadIdx.x == 0) {
        const float norm = static_cast<float>(__builtin_sqrt(s));
        // clip_grad.py:165-169: t = norm + 1e-6; coef = max_norm * (1/t); clamp(max=1)
        const float tt = norm + 1e-6f;
        const float r = 1.0f / tt;
        const float coef = r * max_norm;
        *norm_out = norm;
        *coef_out = coef > 1.0f ? 1.0f : coef;  // NaN stays NaN, as torch.clamp
    }
}

// One workgroup: the partial sums of one range reduced to its float64 sum of squares,
// in the same fixed order as the finalize above.  Fed back to the finalize as a
// one-element array, the sum gives the same norm, bit for bit, as the finalize over
// the partials themselves (0 + s == s, and s + 0 == s for s >= 0).
__global__ __launch_bounds__(kNormThreads) void mi_adamw_sumsq_reduce_kernel(
    const double* __restrict__ partials, int n_partials, double* __restrict__ sumsq_out) {
    double s = 0.0;
    for (int i = threadIdx.x; i < n_partials; i += kNormThreads) s += partials[i];
    s = block_sum<kNormThreads>(s);
    if (threadIdx.x == 0) *sumsq_out = s;
}

// ---------------------------------------------------------------------------
// Pass 2: the AdamW update.
//
// One chunk per workgroup (grid = number of chunks): the hardware dispatcher
// hands the next chunk to whichever CU frees a slot, which balances ragged
// tensors.  With the default 4096-element chunk a workgroup covers its chunk in
// one tile.  Larger chunks are walked tile by tile, software-pipelined: the
// loads of tile k+1 are issued before tile k is computed and stored.

template <typename StateT, bool kAms>
struct Tile {
    f32x4 p, g, m, v, x;
    __device__ __forceinline__ void load(const float* P, const float* G, const void* M,
                                         const void* V, const void* X, int64_t k) {
        g = ld4(G + k);
        p = ld4(P + k);
        m = StateIO<StateT>::ld(M, k);
        v = StateIO<StateT>::ld(V, k);
        if (kAms) x = StateIO<StateT>::ld(X, k);
    }
};

// Waves per SIMD each instance must allow: 8 (two workgroups per CU, at most 64 VGPRs)
// for the fused=True chain's instances without amsgrad, whose float64 math would
// otherwise take 65-70 VGPRs and halve the workgroups in flight; 4 (one workgroup,
// what 1024-thread workgroups need anyway) for the rest.
template <class HS, bool kAms>
constexpr int update_waves_per_eu() {
    return (HS::kLate && !HS::kCapt && !kAms) ? 8 : 4;
}

// The scalars of a chunk formed by the workgroup's first wave and read by every wave
// from LDS: they are the same in every lane, and forming them takes a few hundred
// instructions (two pow, divisions), which every wave would otherwise issue.  Called
// by every thread of the workgroup, once per chunk, with parity alternating: wave 0
// writes buffer `parity` only after all threads have passed the previous chunk's
// barrier, so no thread still reads the buffer it overwrites (that buffer was last
// read two chunks back, before that barrier).
template <class HS>
__device__ __forceinline__ typename HS::Scalars shared_scalars(const HS& hs,
                                                               const mi_adamw_tensor& t,
                                                               int32_t row, int parity) {
    using S = typename HS::Scalars;
    __shared__ S buf[2];
    if (threadIdx.x < 64) {
        const S h = hs.get(t, row);
        if (threadIdx.x == 0) buf[parity] = h;
    }
    __syncthreads();
    // the same words in every lane: into scalar registers, so that branches on them are
    // scalar and the element loop keeps its vector registers
    static_assert(sizeof(S) % 4 == 0, "shared scalars are read as 32-bit words");
    uint32_t w[sizeof(S) / 4];
    memcpy(w, &buf[parity], sizeof(S));
#pragma unroll
    for (unsigned k = 0; k < sizeof(S) / 4; ++k) w[k] = __builtin_amdgcn_readfirstlane(w[k]);
    S r;
    memcpy(&r, w, sizeof(S));
    return r;
}

template <class Src, class HS, typename StateT, bool kClip, bool kCopy, bool kWriteGrad, bool kAms>
__global__ __launch_bounds__(kUpdThreads)
__attribute__((amdgpu_waves_per_eu(update_waves_per_eu<HS, kAms>())))
void mi_adamw_update_kernel(
    Src src, int64_t n_chunks, int64_t chunk_elems, HS hs,
    const float* __restrict__ grad_scale, float pre) {
    using IO = StateIO<StateT>;
    using T = Tile<StateT, kAms>;
    constexpr bool kCapt = HS::kCapt;
    constexpr bool kLate = HS::kLate;
    constexpr bool kProbe = HS::kProbe;
    const float scale = kClip ? *grad_scale : 1.0f;
    int parity = 0;   // shared_scalars' buffer of this chunk
    for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
        mi_adamw_tensor t;
        int64_t begin, end;
        int32_t row;
        src.get(c, chunk_elems, t, begin, end, row);
        // Default chain: the scalars are kernel arguments.  Capturable and fused
        // chains: they are formed once the first tile's loads are in flight; in the
        // capturable chain (two powf, three divisions: a few hundred instructions) by
        // the first wave alone and shared through LDS (kShare).
        typename HS::Scalars h;
        if (!kLate) h = hs.get(t, row);
        float* __restrict__ P = t.param;
        float* __restrict__ G = t.grad;
        void* __restrict__ M = t.exp_avg;
        void* __restrict__ V = t.exp_avg_sq;
        uint16_t* __restrict__ C = t.param_copy;
        void* __restrict__ X = t.max_exp_avg_sq;

        int64_t vend = begin;
        int64_t i = begin + threadIdx.x * kVec;
        T cur;
        bool have = false;
        if (t.flags & MI_ADAMW_T_VEC) {
            vend = begin + ((end - begin) & ~static_cast<int64_t>(kVec - 1));
            have = i < vend;
            if (have) cur.load(P, G, M, V, X, i);
        }
        if (kLate) {
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (HS::kShare) {
                h = shared_scalars(hs, t, row, parity);
                parity ^= 1;
            } else {
                h = hs.get(t, row);
            }
        }
        if (have) {
            const float gmul = h.grad_sign;
            while (true) {
                const int64_t j = i + kUpdTile;
                const bool more = j < vend;
                T nxt = cur;
                if (more) nxt.load(P, G, M, V, X, j);
                // the stored value of div_(world), then of the clip, then -g with maximize
                f32x4 gs = f32x4{cur.g.x * pre, cur.g.y * pre, cur.g.z * pre, cur.g.w * pre};
                if (kClip) gs = f32x4{gs.x * scale, gs.y * scale, gs.z * scale, gs.w * scale};
                if (kWriteGrad) st4(G + i, gs);
                if (kProbe) {
                    keep(gs);
                } else {
                    gs = f32x4{gs.x * gmul, gs.y * gmul, gs.z * gmul, gs.w * gmul};
                    adamw_vec<kAms, kCapt>(cur.p, gs, cur.m, cur.v, cur.x, h);
                }
                st4(P + i, cur.p);
                IO::st(M, i, cur.m);
                IO::st(V, i, cur.v);
                if (kAms) IO::st(X, i, cur.x);
                if (kCopy) st4_bf16(C + i, cur.p);
                if (!more) break;
                cur = nxt;
                i = j;
            }
        }
        // Scalar path: the ragged tail of a vector tensor, or a whole tensor
        // whose pointers are not aligned for dwordx4.
        const float gmul = h.grad_sign;
        for (int64_t j = vend + threadIdx.x; j < end; j += kUpdThreads) {
            float g1 = ld1(G + j) * pre;
            if (kClip) g1 = g1 * scale;
            if (kWriteGrad) st1(G + j, g1);
            g1 = g1 * gmul;
            float p1 = ld1(P + j), m1 = IO::ld1(M, j), v1 = IO::ld1(V, j);
            float x1 = kAms ? IO::ld1(X, j) : 0.0f;
            if (kProbe)
                keep(g1);
            else
                adamw_elem<kAms, kCapt>(p1, g1, m1, v1, x1, h);
            st1(P + j, p1);
            IO::st1(M, j, m1);
            IO::st1(V, j, v1);
            if (kAms) IO::st1(X, j, x1);
            if (kCopy) st1_u16(C + j, bf16_bits(p1));
        }
    }
}

// ---------------------------------------------------------------------------
// g *= coef (clip write-back on its own).

__global__ __launch_bounds__(kUpdThreads) void mi_adamw_scale_kernel(
    TableSource src, int64_t n_chunks, int64_t chunk_elems, const float* __restrict__ coef) {
    const float s = *coef;
    for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
        mi_adamw_tensor t;
        int64_t begin, end;
        int32_t row;
        src.get(c, chunk_elems, t, begin, end, row);
        float* __restrict__ G = t.grad;
        int64_t vend = begin;
        if (t.flags & MI_ADAMW_T_VEC) {
            vend = begin + ((end - begin) & ~static_cast<int64_t>(kVec - 1));
            for (int64_t i = begin + threadIdx.x * kVec; i < vend; i += kUpdTile) {
                f32x4 g = ld4(G + i);
                st4(G + i, f32x4{g.x * s, g.y * s, g.z * s, g.w * s});
            }
        }
        for (int64_t j = vend + threadIdx.x; j < end; j += kUpdThreads) st1(G + j, ld1(G + j) * s);
    }
}

// ---------------------------------------------------------------------------
// bf16 -> fp32 of every tensor of the tables: param = (float)param_copy, exact (the bf16
// bits are the upper half of the fp32 value, NaN payloads included).

__global__ __launch_bounds__(kUpdThreads) void mi_adamw_widen_kernel(
    TableSource src, int64_t n_chunks, int64_t chunk_elems) {
    for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
        mi_adamw_tensor t;
        int64_t begin, end;
        int32_t row;
        src.get(c, chunk_elems, t, begin, end, row);
        const uint16_t* __restrict__ S = t.param_copy;
        float* __restrict__ D = t.param;
        int64_t vend = begin;
        if (t.flags & MI_ADAMW_T_VEC) {
            vend = begin + ((end - begin) & ~static_cast<int64_t>(kVec - 1));
            for (int64_t i = begin + threadIdx.x * kVec; i < vend; i += kUpdTile)
                st4(D + i, ld4_bf16(S + i));
        }
        for (int64_t j = vend + threadIdx.x; j < end; j += kUpdThreads)
            st1(D + j, bf16_to_f32(ld1_u16(S + j)));
    }
}

// ---------------------------------------------------------------------------
// New gradient addresses for rows of a tensor table, for when only the gradients moved
// (zero_grad freed them and backward allocated new ones).  The values travel as kernel
// arguments, so the host needs no staging buffer and may reuse its arrays at once.

constexpr int kPatchRows = 128;
struct GradPatch {
    uint64_t grad[kPatchRows];
    int32_t row[kPatchRows];
    uint32_t vec[kPatchRows / 32];   // bit i: row[i] may take the dwordx4 path
    int32_t count;
};

__global__ __launch_bounds__(kPatchRows) void mi_adamw_set_grads_kernel(
    mi_adamw_tensor* __restrict__ tensors, GradPatch patch) {
    const int i = threadIdx.x;
    if (i < patch.count) {
        mi_adamw_tensor* t = tensors + patch.row[i];
        t->grad = reinterpret_cast<float*>(patch.grad[i]);
        const bool vec = (patch.vec[i >> 5] >> (i & 31)) & 1u;
        t->flags = (t->flags & ~MI_ADAMW_T_VEC) | (vec ? MI_ADAMW_T_VEC : 0);
    }
}

// ---------------------------------------------------------------------------
// Host side

// Workgroups (and partial sums) of the norm pass: two 256-thread workgroups per CU.
// Measured on MI355X over 163M-2G gradients: 512 reads at 6.9-7.3 TB/s, 1024 at
// 6.6-7.0, 2048-4096 and non-multiples of the CU count lower.
constexpr int kNormBlocks = 512;
// Gradient bytes the norm pass reads with cache-allocating loads (its last chunks):
// the update pass, whose own streaming accesses do not displace them, then reads
// them from the 256 MB Infinity Cache instead of HBM.
#ifndef MI_ADAMW_NORM_KEEP_MB
#define MI_ADAMW_NORM_KEEP_MB 256
#endif
constexpr int64_t kNormKeepBytes = int64_t(MI_ADAMW_NORM_KEEP_MB) << 20;

bool chunk_elems_ok(int64_t chunk_elems) {
    return chunk_elems > 0 && (chunk_elems % kChunkQuantum) == 0 &&
           chunk_elems <= (int64_t(1) << 30);
}

int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? MI_ADAMW_OK : static_cast<int>(e);
}

unsigned grid_for(int64_t n_chunks, int32_t max_blocks, int threads) {
    int64_t g = n_chunks;
    if (max_blocks > 0 && g > max_blocks) g = max_blocks;
    if (g > 0x7fffffff / threads) g = 0x7fffffff / threads;
    return static_cast<unsigned>(g);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool finite(float x) { return x - x == 0.0f; }

// Pass 1 alone: one float64 partial sum of (pre*g)^2 per workgroup into `partials`
// (partials_cap doubles available).  Sets *grid_out to the number of partials written.
template <class Src>
int launch_sumsq(const Src& src, int64_t n_chunks, int64_t chunk_elems, float pre,
                 double* partials, int64_t partials_cap, unsigned* grid_out, hipStream_t s) {
    if (n_chunks <= 0 || !chunk_elems_ok(chunk_elems) || !partials) return MI_ADAMW_E_INVALID;
    const unsigned grid = grid_for(n_chunks, kNormBlocks, kNormThreads);
    if (grid > partials_cap) return MI_ADAMW_E_SCRATCH;
    const int64_t keep_chunks = kNormKeepBytes / (chunk_elems * static_cast<int64_t>(sizeof(float)));
    const int64_t keep_from = n_chunks > keep_chunks ? n_chunks - keep_chunks : 0;
    hipLaunchKernelGGL(mi_adamw_sumsq_kernel<Src>, dim3(grid), dim3(kNormThreads), 0, s, src,
                       n_chunks, chunk_elems, partials, keep_from, pre);
    *grid_out = grid;
    return launch_status();
}

// Pass 1 and the finalize: norm and clip coefficient of one range.
template <class Src>
int launch_norm(const Src& src, int64_t n_chunks, int64_t chunk_elems, float max_norm,
                double* partials, float* norm, float* coef, hipStream_t s,
                int64_t partials_cap = MI_ADAMW_MAX_NORM_BLOCKS, float pre = 1.0f) {
    if (!norm || !coef) return MI_ADAMW_E_INVALID;
    unsigned grid = 0;
    int rc = launch_sumsq(src, n_chunks, chunk_elems, pre, partials, partials_cap, &grid, s);
    if (rc != MI_ADAMW_OK) return rc;
    hipLaunchKernelGGL(mi_adamw_norm_finalize_kernel, dim3(1), dim3(kNormThreads), 0, s, partials,
                       static_cast<int>(grid), max_norm, norm, coef);
    return launch_status();
}

// Pass 1 and the reduction of its partials to one float64 sum of squares.
template <class Src>
int launch_sumsq_total(const Src& src, int64_t n_chunks, int64_t chunk_elems, float pre,
                       double* partials, double* sumsq, hipStream_t s) {
    if (!sumsq) return MI_ADAMW_E_INVALID;
    unsigned grid = 0;
    int rc = launch_sumsq(src, n_chunks, chunk_elems, pre, partials, MI_ADAMW_MAX_NORM_BLOCKS,
                          &grid, s);
    if (rc != MI_ADAMW_OK) return rc;
    hipLaunchKernelGGL(mi_adamw_sumsq_reduce_kernel, dim3(1), dim3(kNormThreads), 0, s, partials,
                       static_cast<int>(grid), sumsq);
    return launch_status();
}

template <class Src, class HS, typename StateT, bool kClip, bool kCopy, bool kWriteGrad,
          bool kAms>
int launch_update_k(const Src& src, int64_t n_chunks, int64_t chunk_elems, const HS& hs,
                    const float* scale, float pre, unsigned grid, hipStream_t s) {
    hipLaunchKernelGGL((mi_adamw_update_kernel<Src, HS, StateT, kClip, kCopy, kWriteGrad, kAms>),
                       dim3(grid), dim3(kUpdThreads), 0, s, src, n_chunks, chunk_elems, hs, scale,
                       pre);
    return launch_status();
}

// Runtime flags -> kernel template: one instantiation per (copy, write-grad, amsgrad).
template <class Src, class HS, typename StateT, bool kClip>
int launch_update_cw(const Src& src, int64_t n_chunks, int64_t chunk_elems, const HS& hs,
                     const float* scale, float pre, int32_t flags, unsigned grid,
                     hipStream_t s) {
    const int sel = ((flags & MI_ADAMW_F_BF16_COPY) ? 1 : 0) |
                    ((flags & MI_ADAMW_F_WRITE_GRAD) ? 2 : 0) |
                    ((flags & MI_ADAMW_F_AMSGRAD) ? 4 : 0);
#define MI_ADAMW_SEL(k, C, W, A)                                                              \
    case k:                                                                                   \
        return launch_update_k<Src, HS, StateT, kClip, C, W, A>(src, n_chunks, chunk_elems,  \
                                                                 hs, scale, pre, grid, s);
    switch (sel) {
        MI_ADAMW_SEL(0, false, false, false)
        MI_ADAMW_SEL(1, true, false, false)
        MI_ADAMW_SEL(2, false, true, false)
        MI_ADAMW_SEL(3, true, true, false)
        MI_ADAMW_SEL(4, false, false, true)
        MI_ADAMW_SEL(5, true, false, true)
        MI_ADAMW_SEL(6, false, true, true)
        MI_ADAMW_SEL(7, true, true, true)
    }
#undef MI_ADAMW_SEL
    return MI_ADAMW_E_INVALID;
}

template <class Src, class HS>
int launch_update(const Src& src, int64_t n_chunks, int64_t chunk_elems, const HS& hs,
                  const float* scale, int32_t state_dtype, int32_t flags, int32_t max_blocks,
                  hipStream_t s, float pre = 1.0f) {
    if (n_chunks <= 0 || !chunk_elems_ok(chunk_elems)) return MI_ADAMW_E_INVALID;
    if (state_dtype != MI_ADAMW_STATE_F32 && state_dtype != MI_ADAMW_STATE_BF16)
        return MI_ADAMW_E_INVALID;
    if (flags & ~(MI_ADAMW_F_CLIP | MI_ADAMW_F_BF16_COPY | MI_ADAMW_F_WRITE_GRAD |
                  MI_ADAMW_F_AMSGRAD))
        return MI_ADAMW_E_INVALID;
    const bool clip = flags & MI_ADAMW_F_CLIP;
    if (clip && !scale) return MI_ADAMW_E_INVALID;
    const unsigned grid = grid_for(n_chunks, max_blocks, kUpdThreads);
    if (state_dtype == MI_ADAMW_STATE_F32)
        return clip ? launch_update_cw<Src, HS, float, true>(src, n_chunks, chunk_elems, hs,
                                                              scale, pre, flags, grid, s)
                    : launch_update_cw<Src, HS, float, false>(src, n_chunks, chunk_elems, hs,
                                                               scale, pre, flags, grid, s);
    return clip ? launch_update_cw<Src, HS, uint16_t, true>(src, n_chunks, chunk_elems, hs, scale,
                                                             pre, flags, grid, s)
                : launch_update_cw<Src, HS, uint16_t, false>(src, n_chunks, chunk_elems, hs,
                                                              scale, pre, flags, grid, s);
}

// The memory-only twin of launch_update (no clip: the gradient is read either way).
template <class Src>
int launch_probe(const Src& src, int64_t n_chunks, int64_t chunk_elems, int32_t state_dtype,
                 int32_t flags, int32_t max_blocks, hipStream_t s) {
    if (n_chunks <= 0 || !chunk_elems_ok(chunk_elems)) return MI_ADAMW_E_INVALID;
    if (state_dtype != MI_ADAMW_STATE_F32 && state_dtype != MI_ADAMW_STATE_BF16)
        return MI_ADAMW_E_INVALID;
    flags &= ~MI_ADAMW_F_CLIP;
    if (flags & ~(MI_ADAMW_F_BF16_COPY | MI_ADAMW_F_WRITE_GRAD | MI_ADAMW_F_AMSGRAD))
        return MI_ADAMW_E_INVALID;
    const unsigned grid = grid_for(n_chunks, max_blocks, kUpdThreads);
    const ProbeHyper hs;
    if (state_dtype == MI_ADAMW_STATE_F32)
        return launch_update_cw<Src, ProbeHyper, float, false>(src, n_chunks, chunk_elems, hs,
                                                               nullptr, 1.0f, flags, grid, s);
    return launch_update_cw<Src, ProbeHyper, uint16_t, false>(src, n_chunks, chunk_elems, hs,
                                                              nullptr, 1.0f, flags, grid, s);
}

// The kernel's form of one mi_adamw_fused_hyper.  With host step counts the per-step
// values torch's kernel forms in float64 on the device are formed here with the host
// libm pow and sqrt, then rounded to fp32 as adam_math takes them.  (The device pow and
// libm pow can differ in the last float64 bit; for the betas tested over steps 1-1e6
// that never moves the fp32 values.)
FusedSet fused_set_from(const mi_adamw_fused_hyper& h, bool host_steps) {
    FusedSet f;
    memset(&f, 0, sizeof(f));
    f.beta1 = h.beta1;
    f.one_minus_beta1 = 1.0 - h.beta1;
    f.beta2 = h.beta2;
    f.one_minus_beta2 = 1.0 - h.beta2;
    f.lr = h.lr;
    f.weight_decay = h.weight_decay;
    f.eps = h.eps;
    if (host_steps) {
        f.bc1 = static_cast<float>(1.0 - std::pow(h.beta1, double(h.step)));
        f.bc2_sqrt = static_cast<float>(std::sqrt(1.0 - std::pow(h.beta2, double(h.step))));
        if (!h.lr_ptr) {
            f.lr_wd = h.lr * h.weight_decay;
            f.step_size = static_cast<float>(h.lr / double(f.bc1));
            f.inv_bc2_sqrt = 1.0f / f.bc2_sqrt;
        }
    }
    f.grad_sign = h.grad_sign;
    f.decay = h.weight_decay != 0.0;
    f.lr_ptr = h.lr_ptr;
    return f;
}

// Validate one host-visible tensor descriptor for the flat entry points.
int check_flat(const mi_adamw_tensor* t, int32_t state_dtype, int32_t flags) {
    if (!t || t->numel <= 0 || !t->param || !t->grad || !t->exp_avg || !t->exp_avg_sq)
        return MI_ADAMW_E_INVALID;
    if ((flags & MI_ADAMW_F_BF16_COPY) && !t->param_copy) return MI_ADAMW_E_INVALID;
    if ((flags & MI_ADAMW_F_AMSGRAD) && !t->max_exp_avg_sq) return MI_ADAMW_E_INVALID;
    if (t->flags & MI_ADAMW_T_VEC) {
        const uintptr_t sa = state_dtype == MI_ADAMW_STATE_BF16 ? 8 : 16;
        if (!aligned(t->param, 16) || !aligned(t->grad, 16) || !aligned(t->exp_avg, sa) ||
            !aligned(t->exp_avg_sq, sa) ||
            ((flags & MI_ADAMW_F_BF16_COPY) && !aligned(t->param_copy, 8)) ||
            ((flags & MI_ADAMW_F_AMSGRAD) && !aligned(t->max_exp_avg_sq, sa)))
            return MI_ADAMW_E_ALIGN;
    }
    return MI_ADAMW_OK;
}

// The capturable entry points' host checks and kernel argument: MI_ADAMW_E_INVALID or 0.
int capt_hyper_from(const mi_adamw_capt_hyper* hypers, int32_t n_hyper, const float* d_steps,
                    const int32_t* d_step_index, CaptHyper& hs) {
    if (!hypers || n_hyper <= 0 || n_hyper > MI_ADAMW_MAX_HYPER || !d_steps || !d_step_index)
        return MI_ADAMW_E_INVALID;
    for (int32_t i = 0; i < n_hyper; ++i) {
        const int32_t mode = hypers[i].lr_mode;
        if (mode != MI_ADAMW_LR_FLOAT && mode != MI_ADAMW_LR_VALUE && mode != MI_ADAMW_LR_DEVICE)
            return MI_ADAMW_E_INVALID;
        if (mode == MI_ADAMW_LR_DEVICE && !hypers[i].lr_ptr) return MI_ADAMW_E_INVALID;
    }
    memset(&hs, 0, sizeof(hs));
    memcpy(hs.cp.h, hypers, sizeof(mi_adamw_capt_hyper) * n_hyper);
    hs.steps = d_steps;
    hs.step_index = d_step_index;
    return 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// Library-owned scratch of mi_adamw_grad_norm_flat_noalloc: the norm pass's partial
// sums, one float64 per workgroup.  Each GPU holds its own copy from module load until
// the process ends.  Host code never names the array in a launch or a copy: it looks
// up each device's address once (scratch_on) and passes that pointer.

constexpr int kScratchDoubles = MI_ADAMW_NOALLOC_SCRATCH_BYTES / sizeof(double);
static_assert(kScratchDoubles >= kNormBlocks, "the scratch holds one partial per norm workgroup");

static __device__ __align__(256) double scratch[kScratchDoubles];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<double*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of `scratch` on the stream's device, looked up on that device's
// first call (with the device current) and kept.  The stream must belong to the current
// device; the null stream is the current device's.
int scratch_on(hipStream_t s, double** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (s) {
        hipDevice_t sdev = -1;
        e = hipStreamGetDevice(s, &sdev);
        if (e != hipSuccess) return static_cast<int>(e);
        if (sdev != dev) return MI_ADAMW_E_INVALID;
    }
    if (dev < 0 || dev >= kMaxDevices) return MI_ADAMW_E_INVALID;
    double* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* addr = nullptr;
            e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return static_cast<int>(e);
            if (!addr) return MI_ADAMW_E_INVALID;
            p = static_cast<double*>(addr);
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MI_ADAMW_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI

extern "C" {

const char* mi_adamw_version(void) {
    return "mi_adamw 9 gfx950 fused clip+adamw (fp32/bf16 state, bf16 copy, amsgrad, flat, "
           "capturable, fused=True chain, bf16 widen, memory probe, no-alloc norm, range norm, "
           "grad prescale, grad patch)";
}

const char* mi_adamw_strerror(int code) {
    if (code == MI_ADAMW_OK) return "success";
    if (code == MI_ADAMW_E_INVALID) return "mi_adamw: invalid argument (size, count or pointer)";
    if (code == MI_ADAMW_E_ALIGN) return "mi_adamw: pointer not aligned for the vector path";
    if (code == MI_ADAMW_E_SCRATCH)
        return "mi_adamw: the launch needs more partial sums than the library's static scratch holds";
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "mi_adamw: unknown error";
}

int64_t mi_adamw_build_chunks(const int64_t* numels, int32_t n_tensors, int64_t chunk_elems,
                              mi_adamw_chunk* out, int64_t cap) {
    if (!numels || n_tensors < 0 || !chunk_elems_ok(chunk_elems)) return MI_ADAMW_E_INVALID;
    int64_t n = 0;
    for (int32_t t = 0; t < n_tensors; ++t) {
        if (numels[t] < 0) return MI_ADAMW_E_INVALID;
        const int64_t k = (numels[t] + chunk_elems - 1) / chunk_elems;
        if (k > 0x7fffffff) return MI_ADAMW_E_INVALID;
        for (int64_t i = 0; i < k; ++i, ++n) {
            if (out) {
                if (n >= cap) return MI_ADAMW_E_INVALID;
                out[n].tensor = t;
                out[n].index = static_cast<int32_t>(i);
            }
        }
    }
    return n;
}

int mi_adamw_grad_norm(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                       int64_t n_chunks, int64_t chunk_elems, float max_norm, double* d_partials,
                       float* d_norm, float* d_coef, void* stream) {
    if (!d_tensors || !d_chunks) return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    return launch_norm(src, n_chunks, chunk_elems, max_norm, d_partials, d_norm, d_coef,
                       static_cast<hipStream_t>(stream));
}

int mi_adamw_grad_norm_flat(const float* d_grad, int64_t n, int64_t chunk_elems, float max_norm,
                            double* d_partials, float* d_norm, float* d_coef, void* stream) {
    if (!d_grad || n <= 0 || !chunk_elems_ok(chunk_elems)) return MI_ADAMW_E_INVALID;
    FlatSource src;
    memset(&src.t, 0, sizeof(src.t));
    src.t.grad = const_cast<float*>(d_grad);
    src.t.numel = n;
    src.t.flags = aligned(d_grad, 16) ? MI_ADAMW_T_VEC : 0;
    const int64_t n_chunks = (n + chunk_elems - 1) / chunk_elems;
    return launch_norm(src, n_chunks, chunk_elems, max_norm, d_partials, d_norm, d_coef,
                       static_cast<hipStream_t>(stream));
}

int mi_adamw_grad_norm_flat_noalloc(const float* d_grad, int64_t n, int64_t chunk_elems,
                                    float max_norm, float* d_norm, float* d_coef, void* stream) {
    if (!d_grad || n <= 0 || !chunk_elems_ok(chunk_elems) || !d_norm || !d_coef)
        return MI_ADAMW_E_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    double* partials = nullptr;
    const int rc = scratch_on(s, &partials);
    if (rc != MI_ADAMW_OK) return rc;
    FlatSource src;
    memset(&src.t, 0, sizeof(src.t));
    src.t.grad = const_cast<float*>(d_grad);
    src.t.numel = n;
    src.t.flags = aligned(d_grad, 16) ? MI_ADAMW_T_VEC : 0;
    const int64_t n_chunks = (n + chunk_elems - 1) / chunk_elems;
    return launch_norm(src, n_chunks, chunk_elems, max_norm, partials, d_norm, d_coef, s,
                       kScratchDoubles);
}

int mi_adamw_grad_sumsq(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                        int64_t n_chunks, int64_t chunk_elems, float grad_prescale,
                        double* d_partials, double* d_sumsq, void* stream) {
    if (!d_tensors || !d_chunks || !finite(grad_prescale)) return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    return launch_sumsq_total(src, n_chunks, chunk_elems, grad_prescale, d_partials, d_sumsq,
                              static_cast<hipStream_t>(stream));
}

int mi_adamw_grad_sumsq_flat(const float* d_grad, int64_t n, int64_t chunk_elems,
                             float grad_prescale, double* d_partials, double* d_sumsq,
                             void* stream) {
    if (!d_grad || n <= 0 || !chunk_elems_ok(chunk_elems) || !finite(grad_prescale))
        return MI_ADAMW_E_INVALID;
    FlatSource src;
    memset(&src.t, 0, sizeof(src.t));
    src.t.grad = const_cast<float*>(d_grad);
    src.t.numel = n;
    src.t.flags = aligned(d_grad, 16) ? MI_ADAMW_T_VEC : 0;
    const int64_t n_chunks = (n + chunk_elems - 1) / chunk_elems;
    return launch_sumsq_total(src, n_chunks, chunk_elems, grad_prescale, d_partials, d_sumsq,
                              static_cast<hipStream_t>(stream));
}

int mi_adamw_norm_from_sumsq(const double* d_sumsq, int32_t n, float max_norm, float* d_norm,
                             float* d_coef, void* stream) {
    if (!d_sumsq || n <= 0 || n > MI_ADAMW_MAX_NORM_BLOCKS || !d_norm || !d_coef)
        return MI_ADAMW_E_INVALID;
    hipLaunchKernelGGL(mi_adamw_norm_finalize_kernel, dim3(1), dim3(kNormThreads), 0,
                       static_cast<hipStream_t>(stream), d_sumsq, static_cast<int>(n), max_norm,
                       d_norm, d_coef);
    return launch_status();
}

int mi_adamw_set_grads(mi_adamw_tensor* d_tensors, int32_t n_rows, int32_t n,
                       const int32_t* rows, const uint64_t* grads, const uint8_t* vec,
                       void* stream) {
    if (!d_tensors || n_rows <= 0 || n < 0 || (n > 0 && (!rows || !grads || !vec)))
        return MI_ADAMW_E_INVALID;
    // each row at most once: two patch lanes writing one row would race on its pointer
    // and its alignment flag
    std::vector<uint8_t> seen(static_cast<size_t>(n_rows), 0);
    for (int32_t i = 0; i < n; ++i) {
        if (rows[i] < 0 || rows[i] >= n_rows || seen[rows[i]]) return MI_ADAMW_E_INVALID;
        seen[rows[i]] = 1;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int32_t base = 0; base < n; base += kPatchRows) {
        GradPatch patch;
        memset(&patch, 0, sizeof(patch));
        patch.count = n - base < kPatchRows ? n - base : kPatchRows;
        for (int32_t i = 0; i < patch.count; ++i) {
            patch.grad[i] = grads[base + i];
            patch.row[i] = rows[base + i];
            if (vec[base + i]) patch.vec[i >> 5] |= 1u << (i & 31);
        }
        hipLaunchKernelGGL(mi_adamw_set_grads_kernel, dim3(1), dim3(kPatchRows), 0, s, d_tensors,
                           patch);
        const int rc = launch_status();
        if (rc != MI_ADAMW_OK) return rc;
    }
    return MI_ADAMW_OK;
}

int mi_adamw_scale_grads(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                         int64_t n_chunks, int64_t chunk_elems, const float* d_coef,
                         void* stream) {
    if (!d_tensors || !d_chunks || !d_coef || n_chunks <= 0 || !chunk_elems_ok(chunk_elems))
        return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    hipLaunchKernelGGL(mi_adamw_scale_kernel, dim3(grid_for(n_chunks, 0, kUpdThreads)),
                       dim3(kUpdThreads), 0,
                       static_cast<hipStream_t>(stream), src, n_chunks, chunk_elems, d_coef);
    return launch_status();
}

int mi_adamw_widen_bf16(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                        int64_t n_chunks, int64_t chunk_elems, void* stream) {
    if (!d_tensors || !d_chunks || n_chunks <= 0 || !chunk_elems_ok(chunk_elems))
        return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    hipLaunchKernelGGL(mi_adamw_widen_kernel, dim3(grid_for(n_chunks, 0, kUpdThreads)),
                       dim3(kUpdThreads), 0, static_cast<hipStream_t>(stream), src, n_chunks,
                       chunk_elems);
    return launch_status();
}

int mi_adamw_step_prescaled(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                            int64_t n_chunks, int64_t chunk_elems, const mi_adamw_hyper* hypers,
                            int32_t n_hyper, const float* d_grad_scale, float grad_prescale,
                            int32_t state_dtype, int32_t flags, int32_t max_blocks,
                            void* stream) {
    if (!d_tensors || !d_chunks || !hypers || n_hyper <= 0 || n_hyper > MI_ADAMW_MAX_HYPER ||
        !finite(grad_prescale))
        return MI_ADAMW_E_INVALID;
    StaticHyper hs;
    memset(&hs, 0, sizeof(hs));
    memcpy(hs.hp.h, hypers, sizeof(mi_adamw_hyper) * n_hyper);
    TableSource src{d_tensors, d_chunks};
    return launch_update(src, n_chunks, chunk_elems, hs, d_grad_scale, state_dtype, flags,
                         max_blocks, static_cast<hipStream_t>(stream), grad_prescale);
}

int mi_adamw_step(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                  int64_t n_chunks, int64_t chunk_elems, const mi_adamw_hyper* hypers,
                  int32_t n_hyper, const float* d_grad_scale, int32_t state_dtype, int32_t flags,
                  int32_t max_blocks, void* stream) {
    return mi_adamw_step_prescaled(d_tensors, d_chunks, n_chunks, chunk_elems, hypers, n_hyper,
                                   d_grad_scale, 1.0f, state_dtype, flags, max_blocks, stream);
}

int mi_adamw_step_flat_prescaled(const mi_adamw_tensor* t, const mi_adamw_hyper* hyper,
                                 const float* d_grad_scale, float grad_prescale,
                                 int64_t chunk_elems, int32_t state_dtype, int32_t flags,
                                 int32_t max_blocks, void* stream) {
    if (!hyper || !chunk_elems_ok(chunk_elems) || !finite(grad_prescale))
        return MI_ADAMW_E_INVALID;
    int rc = check_flat(t, state_dtype, flags);
    if (rc != MI_ADAMW_OK) return rc;
    StaticHyper hs;
    memset(&hs, 0, sizeof(hs));
    hs.hp.h[0] = *hyper;
    FlatSource src;
    src.t = *t;
    src.t.hyper = 0;
    const int64_t n_chunks = (t->numel + chunk_elems - 1) / chunk_elems;
    return launch_update(src, n_chunks, chunk_elems, hs, d_grad_scale, state_dtype, flags,
                         max_blocks, static_cast<hipStream_t>(stream), grad_prescale);
}

int mi_adamw_step_flat(const mi_adamw_tensor* t, const mi_adamw_hyper* hyper,
                       const float* d_grad_scale, int64_t chunk_elems, int32_t state_dtype,
                       int32_t flags, int32_t max_blocks, void* stream) {
    return mi_adamw_step_flat_prescaled(t, hyper, d_grad_scale, 1.0f, chunk_elems, state_dtype,
                                        flags, max_blocks, stream);
}

int mi_adamw_step_capturable(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                             int64_t n_chunks, int64_t chunk_elems,
                             const mi_adamw_capt_hyper* hypers, int32_t n_hyper,
                             const float* d_steps, const int32_t* d_step_index,
                             const float* d_grad_scale, int32_t state_dtype, int32_t flags,
                             int32_t max_blocks, void* stream) {
    CaptHyper hs;
    if (!d_tensors || !d_chunks || capt_hyper_from(hypers, n_hyper, d_steps, d_step_index, hs))
        return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    return launch_update(src, n_chunks, chunk_elems, hs, d_grad_scale, state_dtype, flags,
                         max_blocks, static_cast<hipStream_t>(stream));
}

int mi_adamw_step_capturable_rows(const mi_adamw_tensor* d_tensors, int32_t n_rows,
                                  const mi_adamw_chunk* d_chunks, int64_t n_chunks,
                                  int64_t chunk_elems, const mi_adamw_capt_hyper* hypers,
                                  int32_t n_hyper, const float* d_steps,
                                  const int32_t* d_step_index, void* d_row_scalars,
                                  const float* d_grad_scale, int32_t state_dtype, int32_t flags,
                                  int32_t max_blocks, void* stream) {
    CaptHyper hs;
    if (!d_tensors || n_rows <= 0 || !d_chunks || !d_row_scalars || !aligned(d_row_scalars, 16) ||
        capt_hyper_from(hypers, n_hyper, d_steps, d_step_index, hs))
        return MI_ADAMW_E_INVALID;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    RowScalars* rows = static_cast<RowScalars*>(d_row_scalars);
    hipLaunchKernelGGL(mi_adamw_capt_rows_kernel, dim3((n_rows + 255) / 256), dim3(256), 0, s,
                       d_tensors, n_rows, hs, rows);
    const int rc = launch_status();
    if (rc) return rc;
    TableSource src{d_tensors, d_chunks};
    return launch_update(src, n_chunks, chunk_elems, CaptRowsHyper{rows}, d_grad_scale,
                         state_dtype, flags, max_blocks, s);
}

int mi_adamw_step_fused_chain(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                              int64_t n_chunks, int64_t chunk_elems,
                              const mi_adamw_fused_hyper* hypers, int32_t n_hyper,
                              const float* d_steps, const int32_t* d_step_index,
                              const float* d_grad_scale, float grad_prescale,
                              int32_t state_dtype, int32_t flags, int32_t max_blocks,
                              void* stream) {
    if (!d_tensors || !d_chunks || !hypers || n_hyper <= 0 || n_hyper > MI_ADAMW_MAX_HYPER ||
        !finite(grad_prescale) || (d_steps == nullptr) != (d_step_index == nullptr))
        return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (d_steps) {
        FusedHyper<true> hs;
        memset(&hs, 0, sizeof(hs));
        for (int32_t i = 0; i < n_hyper; ++i) hs.fp.h[i] = fused_set_from(hypers[i], false);
        hs.steps = d_steps;
        hs.step_index = d_step_index;
        return launch_update(src, n_chunks, chunk_elems, hs, d_grad_scale, state_dtype, flags,
                             max_blocks, s, grad_prescale);
    }
    FusedHyper<false> hs;
    memset(&hs, 0, sizeof(hs));
    for (int32_t i = 0; i < n_hyper; ++i) hs.fp.h[i] = fused_set_from(hypers[i], true);
    return launch_update(src, n_chunks, chunk_elems, hs, d_grad_scale, state_dtype, flags,
                         max_blocks, s, grad_prescale);
}

int mi_adamw_step_fused_chain_rows(const mi_adamw_tensor* d_tensors, int32_t n_rows,
                                   const mi_adamw_chunk* d_chunks, int64_t n_chunks,
                                   int64_t chunk_elems, const mi_adamw_fused_hyper* hypers,
                                   int32_t n_hyper, const float* d_steps,
                                   const int32_t* d_step_index, void* d_row_scalars,
                                   const float* d_grad_scale, float grad_prescale,
                                   int32_t state_dtype, int32_t flags, int32_t max_blocks,
                                   void* stream) {
    if (!d_tensors || n_rows <= 0 || !d_chunks || !hypers || n_hyper <= 0 ||
        n_hyper > MI_ADAMW_MAX_HYPER || !finite(grad_prescale) || !d_steps || !d_step_index ||
        !d_row_scalars || !aligned(d_row_scalars, 16))
        return MI_ADAMW_E_INVALID;
    FusedHyper<true> hs;
    memset(&hs, 0, sizeof(hs));
    for (int32_t i = 0; i < n_hyper; ++i) hs.fp.h[i] = fused_set_from(hypers[i], false);
    hs.steps = d_steps;
    hs.step_index = d_step_index;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    RowScalars* rows = static_cast<RowScalars*>(d_row_scalars);
    hipLaunchKernelGGL(mi_adamw_fused_rows_kernel, dim3((n_rows + 255) / 256), dim3(256), 0, s,
                       d_tensors, n_rows, hs, rows);
    const int rc = launch_status();
    if (rc) return rc;
    FusedRowsHyper rh;
    memset(&rh, 0, sizeof(rh));
    rh.fp = hs.fp;
    rh.rows = rows;
    TableSource src{d_tensors, d_chunks};
    return launch_update(src, n_chunks, chunk_elems, rh, d_grad_scale, state_dtype, flags,
                         max_blocks, s, grad_prescale);
}

int mi_adamw_step_flat_fused_chain(const mi_adamw_tensor* t, const mi_adamw_fused_hyper* hyper,
                                   const float* d_grad_scale, float grad_prescale,
                                   int64_t chunk_elems, int32_t state_dtype, int32_t flags,
                                   int32_t max_blocks, void* stream) {
    if (!hyper || !chunk_elems_ok(chunk_elems) || !finite(grad_prescale))
        return MI_ADAMW_E_INVALID;
    int rc = check_flat(t, state_dtype, flags);
    if (rc != MI_ADAMW_OK) return rc;
    FusedHyper<false> hs;
    memset(&hs, 0, sizeof(hs));
    hs.fp.h[0] = fused_set_from(*hyper, true);
    FlatSource src;
    src.t = *t;
    src.t.hyper = 0;
    const int64_t n_chunks = (t->numel + chunk_elems - 1) / chunk_elems;
    return launch_update(src, n_chunks, chunk_elems, hs, d_grad_scale, state_dtype, flags,
                         max_blocks, static_cast<hipStream_t>(stream), grad_prescale);
}

int mi_adamw_probe(const mi_adamw_tensor* d_tensors, const mi_adamw_chunk* d_chunks,
                   int64_t n_chunks, int64_t chunk_elems, int32_t state_dtype, int32_t flags,
                   int32_t max_blocks, void* stream) {
    if (!d_tensors || !d_chunks) return MI_ADAMW_E_INVALID;
    TableSource src{d_tensors, d_chunks};
    return launch_probe(src, n_chunks, chunk_elems, state_dtype, flags, max_blocks,
                        static_cast<hipStream_t>(stream));
}

int mi_adamw_probe_flat(const mi_adamw_tensor* t, int64_t chunk_elems, int32_t state_dtype,
                        int32_t flags, int32_t max_blocks, void* stream) {
    if (!chunk_elems_ok(chunk_elems)) return MI_ADAMW_E_INVALID;
    int rc = check_flat(t, state_dtype, flags);
    if (rc != MI_ADAMW_OK) return rc;
    FlatSource src;
    src.t = *t;
    src.t.hyper = 0;
    const int64_t n_chunks = (t->numel + chunk_elems - 1) / chunk_elems;
    return launch_probe(src, n_chunks, chunk_elems, state_dtype, flags, max_blocks,
                        static_cast<hipStream_t>(stream));
}

}  // extern "C"
