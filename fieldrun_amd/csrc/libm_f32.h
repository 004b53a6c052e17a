// libm_f32.h — the f32 math the reference's layers call, bit for bit.
//
// The reference computes exp and tanh with Rust's f32::exp / f32::tanh,
// which call the platform libm's expf / tanhf (glibc on the x86-64 Linux
// hosts it runs on).  These restate the published algorithms glibc 2.35
// ships, so the device computes the same f32 results:
//   frq_expf    ARM optimized-routines expf (glibc's e_expf.c since 2.27):
//               x * 32/ln2 = k + r, 2^(k/32) from a 32-entry table, a cubic in
//               r in double, one rounding to f32.  On hosts with FMA glibc's
//               ifunc picks the build with contracted multiply-adds (kd, r
//               and the three polynomial steps as fused multiply-adds); that
//               is the form here.
//   frq_expm1f  fdlibm's expm1f (Sun Microsystems 1993, in glibc as
//               s_expm1f.c): reduction by ln2 in hi/lo parts and the Q1..Q5
//               rational form.
//   frq_tanhf   fdlibm's tanhf over expm1f.
// Both were checked against glibc 2.35's expf / tanhf on every one of the
// 2^32 f32 inputs (identical results, NaNs as NaN).  Only IEEE add, mul,
// div, sqrt and fma appear, so host and device builds agree with each other.
#pragma once

#include <stdint.h>
#include <string.h>

#ifndef __HIPCC__
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif

namespace frq {
namespace libm {

__host__ __device__ inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
__host__ __device__ inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
__host__ __device__ inline uint64_t d2u(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
__host__ __device__ inline double u2d(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }


// tab[i] = bits(RN(2^(i/32))) - (i << 47): the double nearest 2^(i/32) with
// its exponent field pre-subtracted, so adding k << 47 scales it by 2^(k/32).
constexpr uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// frq_expf's arithmetic away from the special cases, for any x (inputs the
// special cases take give an unused value; the table index stays in range),
// with the table read from tab (kExp2Tab's 32 entries, e.g. a copy in LDS).
__host__ __device__ inline float frq_expf_core_t(float x, const uint64_t* tab) {
    constexpr double shift = 0x1.8p+52, invln2n = 0x1.71547652b82fep+0 * 32;
    constexpr double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                     c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(invln2n, xd, shift);
    const uint64_t ki = d2u(kd);
    kd -= shift;
    const double r = __builtin_fma(invln2n, xd, -kd);
    const double s = u2d(tab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

__host__ __device__ inline float frq_expf_core(float x) { return frq_expf_core_t(x, kExp2Tab); }

__host__ __device__ inline float frq_expf(float x) {
    const uint32_t abstop = (f2u(x) >> 20) & 0x7ff;
    if (abstop >= (0x42b00000u >> 20)) {          // |x| >= 88 or NaN
        if (f2u(x) == 0xff800000u) return 0.0f;  // -inf
        if (abstop >= (0x7f800000u >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;              // underflow
    }
    return frq_expf_core(x);
}

// frq_expf without branches: the core always runs and the special cases
// replace its value by selects, so a run of these in one thread keeps all
// their table loads in flight together.  Same value as frq_expf for every x.
__host__ __device__ inline float frq_expf_sel_t(float x, const uint64_t* tab) {
    // every special input has |x| >= 88, so the selects need no outer test;
    // applied lowest precedence first
    const uint32_t ux = f2u(x);
    float r = frq_expf_core_t(x, tab);
    r = x < -0x1.9fe368p6f ? 0.0f : r;              // underflow
    r = x > 0x1.62e42ep6f ? u2f(0x7f800000u) : r;   // overflow
    r = (ux & 0x7fffffffu) >= 0x7f800000u ? x + x : r;  // inf, NaN
    r = ux == 0xff800000u ? 0.0f : r;               // -inf
    return r;
}
__host__ __device__ inline float frq_expf_sel(float x) { return frq_expf_sel_t(x, kExp2Tab); }

__host__ __device__ inline float frq_expm1f(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = 8.8721679688e+01f,
                ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f,
                q1 = -3.3333335072e-02f, q2 = 1.5873016091e-03f, q3 = -7.9365076090e-05f,
                q4 = 4.0082177293e-06f, q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = f2u(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {                 // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {             // |x| >= 88.72
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - one;     // -1
    }
    if (hx > 0x3eb17218u) {                  // |x| > ln2 / 2: reduce
        if (hx < 0x3f851592u) {              // and |x| < 3 ln2 / 2
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {          // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (q1 + hxs * (q2 + hxs * (q3 + hxs * (q4 + hxs * q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : one + 2.0f * (x - e);
    if (k <= -2 || k > 56) {                 // exp(x) - 1 ~ exp(x)
        y = one - (e - x);
        if (k == 128) y = y * 2.0f * 0x1p127f;
        else y = u2f(f2u(y) + ((uint32_t)k << 23));
        return y - one;
    }
    if (k < 23) {
        t = u2f(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
    } else {
        t = u2f((uint32_t)(0x7f - k) << 23);        // 2^-k
        y = x - (e + t);
        y += one;
    }
    return u2f(f2u(y) + ((uint32_t)k << 23));
}

__host__ __device__ inline float frq_tanhf(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const int32_t jx = (int32_t)f2u(x), ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;  // inf, NaN
    if (ix < 0x41b00000) {                   // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x);  // |x| < 2^-55
        if (ix >= 0x3f800000) {              // |x| >= 1
            t = frq_expm1f(two * (jx < 0 ? -x : x));
            z = one - two / (t + two);
        } else {
            t = frq_expm1f(-two * (jx < 0 ? -x : x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;                      // |x| >= 22: +-1
    }
    return jx >= 0 ? z : -z;
}

}  // namespace libm
}  // namespace frq
