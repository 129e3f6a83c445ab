// Checks the fp32 helpers of the update kernels (mini-megatron_amd/mi_adamw/csrc/
// fp32_math.h), compiled from that header, against the forms they replace, on the GPU:
//
// 1. bf16x2_bits against round-to-nearest-even on the integers, (u + 0x7fff +
//    ((u >> 16) & 1)) >> 16 with every NaN -> 0x7FC0, for all 2^32 fp32 patterns;
// 2. the reference of 3: the device's fp32 division (s / b as the compiler emits it, the
//    division torch's fused AdamW kernel performs) against the host's IEEE division on
//    random pairs over the ranges below;
// 3. div_by_recip(s, b, 1.0f / b) against s / b, bit for bit:
//    - s and b at every exponent pairing the fused=True chain can give (s = sqrtf(v) in
//      [2^-75, 2^64] and +-0, inf, NaN; b = bc2_sqrt in [2^-27, 1]), sampled;
//    - every pair of significands (s, b in [1, 2), 2^46 pairs), unless a smaller number of
//      the 128 launches of 2^39 pairs is asked for;
// 4. div_by_neg_recip(s, b, 1.0f / b), the capturable chain's quotient by a negative b,
//    against s / b: s as in 3, b in -[2^-62, 2^50] at every exponent (sampled), and the
//    significand pairs of 16 of the 128 launches with b negated (its nonzero results are
//    the exact negations of div_by_recip's, which 3 covers in full).
//
// Usage: fp32_math_check [launches]   (default 128: all pairs; about 35 s on an MI355X)
// Prints one line per step and "fp32_math_check: ok" when nothing differs.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "fp32_math.h"

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
            return 2;                                                                  \
        }                                                                              \
    } while (0)

constexpr int kKeep = 16;   // mismatches recorded per kernel: 4 words each

__device__ void record(unsigned long long* bad, uint32_t* first, uint32_t a, uint32_t b,
                       uint32_t want, uint32_t got) {
    const unsigned long long n = atomicAdd(bad, 1ull);
    if (n < kKeep) {
        first[4 * n] = a;
        first[4 * n + 1] = b;
        first[4 * n + 2] = want;
        first[4 * n + 3] = got;
    }
}

__device__ __forceinline__ uint32_t rne_bits(uint32_t u) {
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return 0x7fc0u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// pair i: the patterns 2i and 2i + 1
__global__ void check_bf16(unsigned long long* bad, uint32_t* first) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (1ull << 31);
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t ua = (uint32_t)(2 * i), ub = ua + 1;
        const uint32_t want = rne_bits(ua) | (rne_bits(ub) << 16);
        const uint32_t got = bf16x2_bits(__uint_as_float(ua), __uint_as_float(ub));
        if (got != want) record(bad, first, ua, ub, want, got);
    }
}

__global__ void divide(const float* s, const float* b, float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = s[i] / b[i];
}

__device__ __forceinline__ bool same(float x, float y) {
    return (x != x && y != y) || __float_as_uint(x) == __float_as_uint(y);
}

template <bool kNeg>
__global__ void check_div_sampled(const float* s, const float* b, int ns, int nb,
                                  unsigned long long* bad, uint32_t* first) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ns * nb) return;
    const float sv = s[i / nb], bv = kNeg ? -b[i % nb] : b[i % nb];
    const float want = sv / bv;
    const float got = kNeg ? div_by_neg_recip(sv, bv, 1.0f / bv) : div_by_recip(sv, bv, 1.0f / bv);
    if (!same(want, got))
        record(bad, first, __float_as_uint(sv), __float_as_uint(bv), __float_as_uint(want),
               __float_as_uint(got));
}

// thread t: b significand b_base + (t >> 6); s significands [(t & 63) << 17, + 2^17)
template <bool kNeg>
__global__ __launch_bounds__(256) void check_div_all(uint32_t b_base, unsigned long long* bad,
                                                     uint32_t* first) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    const float b = __uint_as_float((kNeg ? 0xbf800000u : 0x3f800000u) | (b_base + (t >> 6)));
    const float r = 1.0f / b;
    const uint32_t s0 = (t & 63u) << 17;
    for (uint32_t k = 0; k < (1u << 17); ++k) {
        const float s = __uint_as_float(0x3f800000u | (s0 + k));
        const float want = s / b;
        const float got = kNeg ? div_by_neg_recip(s, b, r) : div_by_recip(s, b, r);
        if (__float_as_uint(want) != __float_as_uint(got))
            record(bad, first, __float_as_uint(s), __float_as_uint(b), __float_as_uint(want),
                   __float_as_uint(got));
    }
}

static float rand_sig() { return 1.0f + (float)(rand() & 0x7fffff) / 8388608.0f; }

static int report(const char* what, unsigned long long* d_bad, uint32_t* d_first,
                  unsigned long long* total) {
    unsigned long long n;
    uint32_t f[4 * kKeep];
    CK(hipMemcpy(&n, d_bad, sizeof n, hipMemcpyDeviceToHost));
    CK(hipMemcpy(f, d_first, sizeof f, hipMemcpyDeviceToHost));
    printf("%s: %llu differ\n", what, n);
    for (unsigned long long k = 0; k < n && k < 4; ++k)
        printf("    in %08x %08x  want %08x  got %08x\n", f[4 * k], f[4 * k + 1], f[4 * k + 2],
               f[4 * k + 3]);
    fflush(stdout);
    *total += n;
    CK(hipMemset(d_bad, 0, sizeof n));
    return 0;
}

int main(int argc, char** argv) {
    const int launches = argc > 1 ? atoi(argv[1]) : 128;
    if (launches < 0 || launches > 128) {
        printf("launches must be 0..128\n");
        return 2;
    }
    unsigned long long* bad;
    uint32_t* first;
    unsigned long long total = 0;
    CK(hipMalloc(&bad, sizeof *bad));
    CK(hipMalloc(&first, 4 * kKeep * sizeof *first));
    CK(hipMemset(bad, 0, sizeof *bad));

    // 1. the bf16 pack, every pattern
    check_bf16<<<8192, 256>>>(bad, first);
    CK(hipDeviceSynchronize());
    if (report("bf16x2_bits, all 2^32 fp32 patterns", bad, first, &total)) return 2;

    // 2. the device division against the host's IEEE division
    srand(20261202);
    const int n = 1 << 20;
    std::vector<float> hs(n), hb(n), ho(n);
    for (int i = 0; i < n; ++i) {
        hs[i] = ldexpf(rand_sig(), rand() % 140 - 75);
        hb[i] = ldexpf(rand_sig(), -(rand() % 28));
    }
    float *ds, *db, *dq;
    CK(hipMalloc(&ds, n * sizeof(float)));
    CK(hipMalloc(&db, n * sizeof(float)));
    CK(hipMalloc(&dq, n * sizeof(float)));
    CK(hipMemcpy(ds, hs.data(), n * sizeof(float), hipMemcpyHostToDevice));
    CK(hipMemcpy(db, hb.data(), n * sizeof(float), hipMemcpyHostToDevice));
    divide<<<n / 256, 256>>>(ds, db, dq, n);
    CK(hipMemcpy(ho.data(), dq, n * sizeof(float), hipMemcpyDeviceToHost));
    unsigned long long host_bad = 0;
    for (int i = 0; i < n; ++i) {
        volatile float q = hs[i] / hb[i];
        if (q != ho[i]) ++host_bad;
    }
    printf("device fp32 division against the host's, %d random pairs: %llu differ\n", n,
           host_bad);
    total += host_bad;

    // 3a. every exponent pairing, sampled, and the special values of s
    const int ns = 140 * 64 + 4, nb = 28 * 64;
    std::vector<float> ss(ns), bb(nb);
    for (int e = 0; e < 140; ++e)
        for (int j = 0; j < 64; ++j) ss[e * 64 + j] = ldexpf(j ? rand_sig() : 1.0f, e - 75);
    ss[140 * 64] = 0.0f;
    ss[140 * 64 + 1] = -0.0f;
    ss[140 * 64 + 2] = INFINITY;
    ss[140 * 64 + 3] = NAN;
    for (int e = 0; e < 28; ++e)
        for (int j = 0; j < 64; ++j) bb[e * 64 + j] = ldexpf(j ? rand_sig() : 1.0f, -e);
    float *dss, *dbb;
    CK(hipMalloc(&dss, ns * sizeof(float)));
    CK(hipMalloc(&dbb, nb * sizeof(float)));
    CK(hipMemcpy(dss, ss.data(), ns * sizeof(float), hipMemcpyHostToDevice));
    CK(hipMemcpy(dbb, bb.data(), nb * sizeof(float), hipMemcpyHostToDevice));
    check_div_sampled<false><<<(ns * nb + 255) / 256, 256>>>(dss, dbb, ns, nb, bad, first);
    CK(hipDeviceSynchronize());
    char what[128];
    snprintf(what, sizeof what, "div_by_recip, %d sampled and special pairs", ns * nb);
    if (report(what, bad, first, &total)) return 2;

    // 4a. the negative divisor over its whole range, sampled (b negated in the kernel)
    const int nbn = 113 * 64;
    std::vector<float> bneg(nbn);
    for (int e = 0; e < 113; ++e)
        for (int j = 0; j < 64; ++j) bneg[e * 64 + j] = ldexpf(j ? rand_sig() : 1.0f, e - 62);
    float* dbn;
    CK(hipMalloc(&dbn, nbn * sizeof(float)));
    CK(hipMemcpy(dbn, bneg.data(), nbn * sizeof(float), hipMemcpyHostToDevice));
    check_div_sampled<true><<<(ns * nbn + 255) / 256, 256>>>(dss, dbn, ns, nbn, bad, first);
    CK(hipDeviceSynchronize());
    snprintf(what, sizeof what, "div_by_neg_recip, %d sampled and special pairs", ns * nbn);
    if (report(what, bad, first, &total)) return 2;

    // 3b. every pair of significands
    for (int L = 0; L < launches; ++L) {
        check_div_all<false><<<(1u << 22) / 256, 256>>>((uint32_t)L << 16, bad, first);
        CK(hipDeviceSynchronize());
        unsigned long long sofar;
        CK(hipMemcpy(&sofar, bad, sizeof sofar, hipMemcpyDeviceToHost));
        if ((L + 1) % 16 == 0 || L + 1 == launches || sofar) {
            printf("div_by_recip, significand pairs: %d of 128 launches, %llu differ so far\n",
                   L + 1, sofar);
            fflush(stdout);
        }
    }
    snprintf(what, sizeof what, "div_by_recip, significand pairs (%d of 128 launches)", launches);
    if (report(what, bad, first, &total)) return 2;

    // 4b. b negated: 16 launches spread over the significands of b
    const int neg_launches = launches < 16 ? launches : 16;
    for (int L = 0; L < neg_launches; ++L)
        check_div_all<true><<<(1u << 22) / 256, 256>>>((uint32_t)(L * 8) << 16, bad, first);
    CK(hipDeviceSynchronize());
    snprintf(what, sizeof what, "div_by_neg_recip, significand pairs (%d launches)", neg_launches);
    if (report(what, bad, first, &total)) return 2;

    CK(hipFree(bad));
    CK(hipFree(first));
    CK(hipFree(ds));
    CK(hipFree(db));
    CK(hipFree(dq));
    CK(hipFree(dss));
    CK(hipFree(dbb));
    CK(hipFree(dbn));
    if (total) {
        printf("fp32_math_check: FAILED (%llu differ)\n", total);
        return 1;
    }
    printf("fp32_math_check: ok\n");
    return 0;
}
