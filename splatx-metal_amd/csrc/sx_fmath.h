// sx_fmath.h — deterministic transcendental functions shared by the gfx950 kernels and the CPU
// oracle.
//
// Why this exists: integer outputs of the step (radii, AccuTile tile sets, isect keys, raster
// last_ids) are functions of log/exp results. Device libm and glibc may differ by an ulp, which
// can flip an integer boundary. Every function here is written with IEEE-754 basic operations
// only (+ - * /, sqrt, rint, fma, integer bit manipulation), evaluated in a fixed order, so the
// host compiler (g++ -ffp-contract=off) and hipcc (-ffp-contract=off, correctly rounded
// div/sqrt) produce identical bits. The double-based float functions (sx_logf, sx_expf,
// sx_powf, sx_sincosf) carry ~2^-50 relative error before the final rounding to float, so they
// return the correctly rounded float for all but astronomically rare inputs; the tests compare
// them with glibc and with long-double references.
//
// Methods (textbook, no library code reproduced):
//   log:  x = m·2^e, m in [1/sqrt2, sqrt2); log m = 2·atanh(s), s = (m-1)/(m+1), odd series.
//   exp:  Cody–Waite reduction z = k·ln2 + r with ln2 split hi/lo, Taylor series of e^r, 2^k by
//         exponent-field construction.
//   sin/cos: reduction by pi/2 (hi/lo split) to |r| <= pi/4, Taylor series, quadrant table.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define SX_HD __host__ __device__
#else
#define SX_HD
#endif

#if defined(__HIP_DEVICE_COMPILE__)
#define SX_SQRTF(x) __builtin_sqrtf(x)
#define SX_SQRT(x) __builtin_sqrt(x)
#else
#include <cmath>
#define SX_SQRTF(x) std::sqrt(static_cast<float>(x))
#define SX_SQRT(x) std::sqrt(static_cast<double>(x))
#endif

namespace sxm {

SX_HD inline uint64_t bits_of(double x) {
    uint64_t u;
    __builtin_memcpy(&u, &x, 8);
    return u;
}
SX_HD inline double double_of(uint64_t u) {
    double x;
    __builtin_memcpy(&x, &u, 8);
    return x;
}
SX_HD inline uint32_t bits_of(float x) {
    uint32_t u;
    __builtin_memcpy(&u, &x, 4);
    return u;
}
SX_HD inline float float_of(uint32_t u) {
    float x;
    __builtin_memcpy(&x, &u, 4);
    return x;
}

SX_HD inline bool isnan_f(float x) { return x != x; }
SX_HD inline bool isnan_d(double x) { return x != x; }

// ---------------------------------------------------------------------------------------------
// double log for finite x > 0 (callers handle the special values).
// ---------------------------------------------------------------------------------------------
SX_HD inline double log_pos_d(double x) {
    uint64_t b = bits_of(x);
    int e = static_cast<int>((b >> 52) & 0x7ff);
    if (e == 0) { // subnormal double: scale by 2^54 (exact)
        x = x * 18014398509481984.0;
        b = bits_of(x);
        e = static_cast<int>((b >> 52) & 0x7ff) - 54;
    }
    e -= 1023;
    double m = double_of((b & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL); // [1,2)
    if (m > 1.4142135623730951) {
        m = m * 0.5; // exact
        e += 1;
    }
    const double f = m - 1.0;  // exact (m within a factor 2 of 1)
    const double s = f / (2.0 + f);
    const double s2 = s * s;
    // atanh(s)/s - 1 = s2/3 + s2^2/5 + ... (11 terms: s2 <= 0.0295, truncation < 2^-56)
    double p = 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    const double two_s = s + s;
    const double logm = two_s + two_s * (s2 * p);
    // ln2 = hi + lo, hi has 32 trailing zero bits so e*hi is exact for |e| < 2^20
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    const double ed = static_cast<double>(e);
    return (ed * ln2_hi) + (ed * ln2_lo + logm);
}

// ---------------------------------------------------------------------------------------------
// double exp with a finite result range; saturates to 0 / +inf outside it.
// ---------------------------------------------------------------------------------------------
SX_HD inline double exp_d(double z) {
    if (isnan_d(z)) return z;
    if (z > 709.78) return double_of(0x7ff0000000000000ULL);
    if (z < -745.2) return 0.0;
    const double kd = __builtin_rint(z * 1.4426950408889634);
    const double ln2_hi = 6.93147180369123816490e-01;
    const double ln2_lo = 1.90821492927058770002e-10;
    double r = z - kd * ln2_hi; // exact product (hi has 32 trailing zeros, |k| < 1100)
    r = r - kd * ln2_lo;        // |r| <= 0.3466
    // e^r Taylor to degree 13: truncation r^14/14! < 5e-18
    double p = 1.0 / 6227020800.0;       // 1/13!
    p = p * r + 1.0 / 479001600.0;       // 1/12!
    p = p * r + 1.0 / 39916800.0;        // 1/11!
    p = p * r + 1.0 / 3628800.0;         // 1/10!
    p = p * r + 1.0 / 362880.0;          // 1/9!
    p = p * r + 1.0 / 40320.0;           // 1/8!
    p = p * r + 1.0 / 5040.0;            // 1/7!
    p = p * r + 1.0 / 720.0;             // 1/6!
    p = p * r + 1.0 / 120.0;             // 1/5!
    p = p * r + 1.0 / 24.0;              // 1/4!
    p = p * r + 1.0 / 6.0;               // 1/3!
    p = p * r + 0.5;                     // 1/2!
    p = p * r;                           // r/2 + ...
    const double er = 1.0 + (r + r * p); // e^r = 1 + r + r^2/2 + ...
    int k = static_cast<int>(kd);
    double scale = 1.0;
    if (k < -1000) { // keep 2^k in the normal range, result may become subnormal
        scale = double_of(static_cast<uint64_t>(1023 - 600) << 52); // 2^-600
        k += 600;
    } else if (k > 1000) {
        scale = double_of(static_cast<uint64_t>(1023 + 600) << 52); // 2^600
        k -= 600;
    }
    const double two_k = double_of(static_cast<uint64_t>(k + 1023) << 52);
    return (er * two_k) * scale;
}

// ---------------------------------------------------------------------------------------------
// float log / exp / pow computed through the double kernels and rounded once.
// ---------------------------------------------------------------------------------------------
SX_HD inline float logf_(float x) {
    if (isnan_f(x)) return x;
    if (x < 0.0f) return float_of(0x7fc00000u);          // NaN
    if (x == 0.0f) return float_of(0xff800000u);         // -inf
    if (bits_of(x) == 0x7f800000u) return x;             // +inf
    return static_cast<float>(log_pos_d(static_cast<double>(x)));
}

SX_HD inline float expf_(float x) {
    if (isnan_f(x)) return x;
    return static_cast<float>(exp_d(static_cast<double>(x)));
}

// x^y for x >= 0 (the only domain used: relocation opacities and their complements).
SX_HD inline float powf_(float x, float y) {
    if (isnan_f(x) || isnan_f(y)) return float_of(0x7fc00000u);
    if (y == 0.0f || x == 1.0f) return 1.0f;
    if (x == 0.0f) return y > 0.0f ? 0.0f : float_of(0x7f800000u);
    if (x < 0.0f) return float_of(0x7fc00000u);
    if (bits_of(x) == 0x7f800000u) return y > 0.0f ? x : 0.0f;
    return static_cast<float>(exp_d(static_cast<double>(y) * log_pos_d(static_cast<double>(x))));
}

// ---------------------------------------------------------------------------------------------
// sin and cos of a float argument (|x| well below 2^20; Box-Muller uses (0, 2pi]).
// ---------------------------------------------------------------------------------------------
SX_HD inline void sincos_reduced_d(double r, double* s, double* c) {
    const double r2 = r * r;
    // sin r = r - r^3/3! + ... (to r^17), cos r = 1 - r^2/2! + ... (to r^18); |r| <= pi/4
    double ps = -1.0 / 355687428096000.0;  // -1/17!
    ps = ps * r2 + 1.0 / 1307674368000.0;  //  1/15!
    ps = ps * r2 - 1.0 / 6227020800.0;     // -1/13!
    ps = ps * r2 + 1.0 / 39916800.0;       //  1/11!
    ps = ps * r2 - 1.0 / 362880.0;         // -1/9!
    ps = ps * r2 + 1.0 / 5040.0;           //  1/7!
    ps = ps * r2 - 1.0 / 120.0;            // -1/5!
    ps = ps * r2 + 1.0 / 6.0;              //  1/3! (sign applied below)
    *s = r - r * (r2 * ps);
    double pc = 1.0 / 6402373705728000.0;  //  1/18!
    pc = pc * r2 - 1.0 / 20922789888000.0; // -1/16!
    pc = pc * r2 + 1.0 / 87178291200.0;    //  1/14!
    pc = pc * r2 - 1.0 / 479001600.0;      // -1/12!
    pc = pc * r2 + 1.0 / 3628800.0;        //  1/10!
    pc = pc * r2 - 1.0 / 40320.0;          // -1/8!
    pc = pc * r2 + 1.0 / 720.0;            //  1/6!
    pc = pc * r2 - 1.0 / 24.0;             // -1/4!
    pc = pc * r2 + 0.5;                    //  1/2! (sign applied below)
    *c = 1.0 - r2 * pc;
}

SX_HD inline void sincosf_(float x, float* sout, float* cout) {
    const double xd = static_cast<double>(x);
    const double q = __builtin_rint(xd * 0.63661977236758134308); // 2/pi
    // pi/2 = hi + lo; hi has 33 significant bits so q*hi is exact for |q| < 2^20
    const double pio2_hi = 1.57079632673412561417e+00;
    const double pio2_lo = 6.07710050650619224932e-11;
    const double r = (xd - q * pio2_hi) - q * pio2_lo;
    double s, c;
    sincos_reduced_d(r, &s, &c);
    const int quad = static_cast<int>(q) & 3;
    double so, co;
    if (quad == 0) { so = s; co = c; }
    else if (quad == 1) { so = c; co = -s; }
    else if (quad == 2) { so = -s; co = -c; }
    else { so = -c; co = s; }
    *sout = static_cast<float>(so);
    *cout = static_cast<float>(co);
}

// ---------------------------------------------------------------------------------------------
// Fast float exp for the rasterizer inner loop: float arithmetic with explicit fma, <= ~1 ulp,
// bit-identical on host and device (fma is exactly rounded on both).
// ---------------------------------------------------------------------------------------------
SX_HD inline float expf_fast(float x) {
    if (isnan_f(x)) return x;
    if (x > 88.72283f) return float_of(0x7f800000u);
    if (x < -103.97208f) return 0.0f;
    const float kf = __builtin_rintf(x * 1.44269502f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);   // ln2 hi (15 significant bits)
    r = __builtin_fmaf(kf, -1.42860677e-06f, r);             // ln2 lo
    float p = 2.48015873e-05f;                               // 1/8!
    p = __builtin_fmaf(p, r, 1.98412698e-04f);               // 1/7!
    p = __builtin_fmaf(p, r, 1.38888889e-03f);               // 1/6!
    p = __builtin_fmaf(p, r, 8.33333377e-03f);               // 1/5!
    p = __builtin_fmaf(p, r, 4.16666679e-02f);               // 1/4!
    p = __builtin_fmaf(p, r, 1.66666672e-01f);               // 1/3!
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int k = static_cast<int>(kf);
    float scale = 1.0f;
    if (k < -125) {
        scale = float_of(static_cast<uint32_t>(127 - 64) << 23); // 2^-64
        k += 64;
    } else if (k > 127) {
        scale = 2.0f;
        k -= 1;
    }
    const float two_k = float_of(static_cast<uint32_t>(k + 127) << 23);
    return (p * two_k) * scale;
}

// Saturating float -> int32 truncation (NaN -> 0). Used where the reference casts a float that is
// in range for all valid inputs; the defined behavior keeps host and device identical otherwise.
SX_HD inline int32_t f2i_trunc(float x) {
    if (isnan_f(x)) return 0;
    if (x >= 2147483648.0f) return 2147483647;
    if (x <= -2147483648.0f) return static_cast<int32_t>(0x80000000u);
    return static_cast<int32_t>(x);
}

} // namespace sxm
