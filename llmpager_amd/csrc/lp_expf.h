// The single-precision exponential that llmpager's routing runs through.
//
// Routing in the reference is host Rust: `(v - m).exp()` in top_k_softmax
// (crates/llmpager-run/src/decode.rs:736) and `(-v).exp()` in sigmoid_topk
// (crates/llmpager-run/src/kimi.rs:1163).  Rust's f32::exp lowers to the
// platform libm `expf`, i.e. glibc.  Bit-exact routing on the GPU therefore
// needs the GPU to produce glibc's expf bits, not merely an accurate exp.
//
// glibc (>= 2.28, here 2.35 on x86_64) implements expf with the published
// method of ARM's Optimized Routines: scale x by N/ln2 (N = 32), round to an
// integer k with the 1.5*2^52 shift trick, take 2^(k/N) from a 32-entry table
// of 2^(i/32) (each entry pre-biased by -(i << 47) so that adding k << 47
// yields the scaled power), and evaluate a degree-3 polynomial for 2^(r/N),
// all in double, rounding once to float at the end.  On x86_64 hosts with
// FMA (every MI355X host) glibc selects its FMA build, in which the compiler
// has fused the range reduction and the polynomial Horner steps; the fusions
// below are exactly those.  This restatement was checked bit-for-bit against
// glibc 2.35's expf over every non-NaN float (4,278,190,082 inputs, 0
// differences); the table entries are 2^(i/32) rounded to nearest double.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define LP_HD __host__ __device__
#else
#define LP_HD
#endif

namespace lp {

LP_HD inline double expf_bits_to_double(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}

LP_HD inline uint64_t expf_double_to_bits(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}

LP_HD inline uint32_t expf_float_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// 2^(i/32) to nearest double, minus (i << 47).
#if defined(__HIPCC__)
__device__ __constant__
#endif
static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

#if defined(__HIPCC__)
__device__ inline uint64_t exp2tab(uint32_t i) { return kExp2Tab[i]; }
#endif

// The normal-range arithmetic of expf_glibc, with the table read through
// tab(i).  Specials (|x| >= ~88, inf, nan) are the callers' business.
template <typename Tab>
LP_HD inline float expf_glibc_core(float x, Tab tab) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;  // 32 / ln 2
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = expf_double_to_bits(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = tab((uint32_t)(ki % 32)) + (ki << 47);
    const double s = expf_bits_to_double(t);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

LP_HD inline float expf_glibc(float x) {
    const uint32_t ux = expf_float_to_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                      // |x| >= 88 or x is inf/nan
        if (ux == 0xff800000u) return 0.0f;      // -inf
        if (abstop >= 0x7f8u) return x + x;      // +inf or nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;              // underflow
    }
#if defined(__HIP_DEVICE_COMPILE__)
    return expf_glibc_core(x, [](uint32_t i) { return exp2tab(i); });
#else
    return expf_glibc_core(x, [](uint32_t i) { return kExp2Tab[i]; });
#endif
}

#if defined(__HIPCC__)
// Wave form of expf_glibc: the table lives in registers (lanes 0..31 hold
// entry `lane`, from exp2tab_lane()) and is read with cross-lane shuffles,
// so no lookup waits on memory.  Every lane of the wave must call it
// together (no lane may sit out under a branch); specials are selected after
// the normal-range arithmetic, which is harmless for them.  Bit-identical
// to expf_glibc.
__device__ inline uint64_t exp2tab_lane() {
    const uint32_t l = __lane_id();
    return l < 32 ? exp2tab(l) : 0ull;
}

__device__ inline float expf_glibc_wave(float x, uint64_t tabv) {
    const int lo = (int)(uint32_t)tabv, hi = (int)(uint32_t)(tabv >> 32);
    const float y = expf_glibc_core(x, [&](uint32_t i) {
        return (uint64_t)(uint32_t)__shfl(lo, (int)i, 64) | ((uint64_t)(uint32_t)__shfl(hi, (int)i, 64) << 32);
    });
    const uint32_t ux = expf_float_to_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    float r = y;
    if (abstop >= 0x42bu) {
        if (x < -0x1.9fe368p6f) r = 0.0f;
        if (x > 0x1.62e42ep6f) r = __builtin_inff();
        if (abstop >= 0x7f8u) r = x + x;
        if (ux == 0xff800000u) r = 0.0f;
    }
    return r;
}
#endif

}  // namespace lp
