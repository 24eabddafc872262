// Host sincosf for the rotation table: glibc 2.28's generic sincosf
// (sysdeps/ieee754/flt-32/s_sincosf.c, s_sincosf.h), which the reference
// ports bit for bit (libm::sincosf, src/libm.rs:350-497) so that its RoPE
// angles give the same (sin, cos) on every platform. A newer C library rounds
// some results differently in the last bit, so the table does not call it.
//
// |x| is reduced by k*pi/2 (a table of multiples below 9pi/4, two pi/2
// pieces below 2^23, 28-bit pieces of 4/pi above), then evaluated in f64 with
// Chebyshev forms on [-pi/4, pi/4] and rounded to binary32. Multiply-adds are
// fused exactly where the reference fuses them (its mul_add calls: glibc
// built with FMA contraction); every other operation is unfused, so this file
// is compiled with -ffp-contract=off like the rest of the library.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

namespace pcl {

namespace sincosf_detail {

constexpr double kCos[5] = {-0x1.ffffffffe98aep-2, 0x1.55555545c50c7p-5,
                            -0x1.6c16b348b6874p-10, 0x1.a00eb9ac43ccp-16,
                            -0x1.23c97dd8844d7p-22};
constexpr double kSin[5] = {-0x1.5555555551cd9p-3, 0x1.1111110c2688bp-7,
                            -0x1.a019f8b4bd1f9p-13, 0x1.71d7264e6b5b4p-19,
                            -0x1.a947e1674b58ap-26};
// k * pi/2, k = 0..5
constexpr double kPio2[6] = {0.0,
                             0x1.921fb54442d18p+0,
                             0x1.921fb54442d18p+1,
                             0x1.2d97c7f3321d2p+2,
                             0x1.921fb54442d18p+2,
                             0x1.f6a7a2955385ep+2};
// 4/pi in 28-bit pieces
constexpr double kInvPio4[8] = {0.0,
                                0x1.45f306cp+0,
                                0x1.c9c882ap-28,
                                0x1.4fe13a8p-58,
                                0x1.f47d4d0p-85,
                                0x1.bb81b6cp-112,
                                0x1.4acc9e0p-142,
                                0x1.0e4107cp-169};
constexpr double kPi4 = 0x1.921fb54442d18p-1;
constexpr double kInvPi4 = 0x1.45f306dc9c883p+0;
constexpr double kNinePi4 = 0x1.c463abeccb2bbp+2;
constexpr double kPi2Hi = 0x1.921fb544p+0;
constexpr double kPi2Lo = 0x1.0b4611a626332p-34;

inline double sin_form(double t, double t2)
{
    double p = std::fma(kSin[4], t2, kSin[3]);
    for (int k = 2; k >= 0; --k)
        p = std::fma(t2, p, kSin[k]);
    return std::fma(t * t2, p, t);
}

inline double cos_form(double t2)
{
    double p = std::fma(kCos[4], t2, kCos[3]);
    for (int k = 2; k >= 0; --k)
        p = std::fma(t2, p, kCos[k]);
    return std::fma(t2, p, 1.0);
}

// t: reduced |x|; n = trunc(|x| / (pi/4)) + 1 picks the form and the sign.
inline void from_reduced(double t, uint32_t n, bool negative, float *s, float *c)
{
    const double t2 = t * t;
    const double sv = (n & 2) == 0 ? sin_form(t, t2) : cos_form(t2);
    const uint32_t m = n + 2;
    const double cv = (m & 2) == 0 ? sin_form(t, t2) : cos_form(t2);
    *s = (float)((((n >> 2) & 1) != 0) != negative ? -sv : sv);
    *c = (float)(((m >> 2) & 1) != 0 ? -cv : cv);
}

} // namespace sincosf_detail

inline void sincosf_glibc228(float x, float *s, float *c)
{
    using namespace sincosf_detail;
    const double t = (double)x;
    const double at = std::fabs(t);
    if (at < kPi4) {
        if (at >= 0x1p-5) {
            const double t2 = t * t;
            *s = (float)sin_form(t, t2);
            *c = (float)cos_form(t2);
        } else if (at >= 0x1p-27) {
            const double t2 = t * t, t3 = t * t2;
            *s = (float)std::fma(t3, std::fma(t2, 0x1.110f475cec8c5p-7, -0x1.555555543d49dp-3), t);
            *c = (float)std::fma(t2, std::fma(t3, 0x1.55514b178dac5p-5, -0x1.fffffff5cc6fdp-2),
                                 1.0);
        } else {
            *s = (float)(t != 0.0 ? std::fma(-t, 0x1p-50, t) : t);
            *c = (float)(1.0 - at);
        }
        return;
    }
    const bool negative = x < 0.0f;
    if (at < kNinePi4) {
        const uint32_t n = (uint32_t)std::fma(at, kInvPi4, 1.0);
        from_reduced(at - kPio2[n / 2], n, negative, s, c);
        return;
    }
    if (!std::isfinite(at)) {
        *s = *c = x - x;
        return;
    }
    if (at < 0x1p23) {
        const uint32_t n = (uint32_t)(at * kInvPi4) + 1;
        const double k = (double)(n / 2);
        from_reduced(std::fma(-k, kPi2Lo, std::fma(-k, kPi2Hi, at)), n, negative, s, c);
        return;
    }
    // |x| >= 2^23: |x| times four pieces of 4/pi, starting at the piece that
    // keeps the integer part of the product exact
    uint32_t bits;
    const float ax = std::fabs(x);
    std::memcpy(&bits, &ax, sizeof bits);
    const int e = ((int)(bits >> 23) - 127 + 3) / 28;
    double a = kInvPio4[e] * at;
    const double b = kInvPio4[e + 1] * at, cc = kInvPio4[e + 2] * at, d = kInvPio4[e + 3] * at;
    uint64_t l = (uint64_t)a & ~(uint64_t)7;
    a -= (double)l;
    double f = a + b;
    l = (uint64_t)f;
    f = a - (double)l;
    if (l & 1) {
        f -= 1.0;
        f = d + (cc + (b + f));
    } else {
        f = d + (cc + (b + f));
        if (f > 1.0) {
            l += 1;
            f -= 2.0;
        }
    }
    from_reduced(f * kPi4, (uint32_t)l + 1, negative, s, c);
}

} // namespace pcl
