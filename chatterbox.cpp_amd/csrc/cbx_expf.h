// cbx_expf.h -- binary32 exp with the exact results of the host libm expf
// that the reference's std::exp(float) calls (src/main.cpp:759, :789).
//
// Published method: the table-driven expf of ARM optimized-routines
// (Szabolcs Nagy, 2017), shipped as glibc >= 2.27's expf
// (sysdeps/ieee754/flt-32/e_expf.c, data in e_exp2f_data.c).  x*32/ln2 is split
// as k + r with |r| <= 1/2; exp(x) = 2^(k/32) * P(r) with a 2^(i/32) table
// entry (i = k mod 32) and a degree-3 polynomial P, all in binary64, rounded
// once to binary32 at the end.
//
// The x86-64 glibc picks its FMA build of this routine on CPUs with FMA+AVX2.
// That build contracts the range reduction (kd = fma(InvLn2N, x, SHIFT),
// r = fma(InvLn2N, x, -kd)) and the three polynomial steps into FMAs; the
// same contractions are written out here with explicit fma calls, so host and
// device evaluate identical binary64 operations.
//
//  * tab[i] = bits(RN64(2^(i/32))) - (i << 47): derived from the mathematics
//    (tests check every entry against a 200-bit evaluation).
//  * The polynomial coefficients are the routine's minimax constants.
//  * Checked exhaustively against libm for every binary32 x in [-104, 89]
//    (2.24e9 inputs): identical bits.
#pragma once

#include <stdint.h>

// In a HIP translation unit the routine is device code reading a __constant__
// table; a plain C++ compile (the CPU test) gets the same code on the host.
#if defined(__HIPCC__)
#define CBX_HD __device__ __forceinline__
#else
#define CBX_HD inline
#include <math.h>
#include <string.h>
#endif

namespace cbx {

struct Exp2Table {
    uint64_t t[32];
};

#if defined(__HIPCC__)
static __device__ __constant__ const Exp2Table kExp2TabDev = {{
#else
static const Exp2Table kExp2TabHost = {{
#endif
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
}};

namespace expf_detail {
constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;  // 32 / ln 2
constexpr double kShift = 0x1.8p+52;                     // round-to-int shifter
constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;

CBX_HD uint32_t f2u(float x) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint32_t, x);
#else
    uint32_t u; memcpy(&u, &x, 4); return u;
#endif
}
CBX_HD uint64_t d2u(double x) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint64_t, x);
#else
    uint64_t u; memcpy(&u, &x, 8); return u;
#endif
}
CBX_HD double u2d(uint64_t u) {
#if defined(__HIPCC__)
    return __builtin_bit_cast(double, u);
#else
    double d; memcpy(&d, &u, 8); return d;
#endif
}
CBX_HD double fma64(double a, double b, double c) {
#if defined(__HIPCC__)
    return __builtin_fma(a, b, c);
#else
    return fma(a, b, c);
#endif
}
}  // namespace expf_detail

// The special-case thresholds are binary32 constants: 88.0f (0x42b00000),
// log(2^128) ~ 88.72 (0x42b17217), log(2^-150) ~ -103.97 (0xc2cff1b4).
CBX_HD float expf_libm(float x) {
    using namespace expf_detail;
    const uint32_t ux = f2u(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= (0x42b00000u >> 20)) {           // |x| >= 88 or NaN
        if (ux == 0xff800000u) return 0.0f;         // -inf
        if (abstop >= (0x7f800000u >> 20)) return x + x;  // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = fma64(kInvLn2N, xd, kShift);
    const uint64_t ki = d2u(kd);
    kd -= kShift;
    const double r = fma64(kInvLn2N, xd, -kd);
#if defined(__HIPCC__)
    uint64_t t = kExp2TabDev.t[ki % 32];
#else
    uint64_t t = kExp2TabHost.t[ki % 32];
#endif
    t += ki << (52 - 5);
    const double s = u2d(t);
    const double z = fma64(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma64(kC2, r, 1.0);
    y = fma64(z, r2, y);
    y = y * s;
    return (float)y;
}

// The same function without branches: the main path runs on an argument
// replaced by 0 where a special case applies, and the special value is
// selected afterwards.  `tab` points at the 32 table words (on the device an
// LDS copy, so the lookup is a local read).  Bit-identical to expf_libm for
// every input (checked exhaustively on the host).
CBX_HD float expf_libm_branchless(float x, const uint64_t* tab) {
    using namespace expf_detail;
    const uint32_t ux = f2u(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    const bool minus_inf = ux == 0xff800000u;
    const bool inf_nan = abstop >= (0x7f800000u >> 20);
    const bool over = x > 0x1.62e42ep6f;
    const bool under = x < -0x1.9fe368p6f;
    const bool special = minus_inf || inf_nan || over || under;
    const double xd = (double)(special ? 0.0f : x);
    double kd = fma64(kInvLn2N, xd, kShift);
    const uint64_t ki = d2u(kd);
    kd -= kShift;
    const double r = fma64(kInvLn2N, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << (52 - 5);
    const double s = u2d(t);
    const double z = fma64(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma64(kC2, r, 1.0);
    y = fma64(z, r2, y);
    y = y * s;
    const float main = (float)y;
    const float sp = minus_inf ? 0.0f
                   : inf_nan   ? x + x
                   : over      ? __builtin_huge_valf()
                               : 0.0f;
    return special ? sp : main;
}

// The branch-free form for arguments x <= 0 (including -inf, not NaN): the
// only special case left is the underflow to 0 below log(2^-150).  Equal to
// expf_libm on that domain (checked exhaustively on the host).
CBX_HD float expf_nonpos(float x, const uint64_t* tab) {
    using namespace expf_detail;
    const bool under = x < -0x1.9fe368p6f;
    const double xd = (double)(under ? 0.0f : x);
    double kd = fma64(kInvLn2N, xd, kShift);
    const uint64_t ki = d2u(kd);
    kd -= kShift;
    const double r = fma64(kInvLn2N, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << (52 - 5);
    const double s = u2d(t);
    const double z = fma64(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma64(kC2, r, 1.0);
    y = fma64(z, r2, y);
    y = y * s;
    return under ? 0.0f : (float)y;
}

#if !defined(__HIPCC__)
inline float expf_libm_branchless(float x) { return expf_libm_branchless(x, kExp2TabHost.t); }
inline float expf_nonpos(float x) { return expf_nonpos(x, kExp2TabHost.t); }
#endif

}  // namespace cbx
