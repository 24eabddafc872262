// Sine and cosine of a rotary angle, as the head transform's rotation table
// holds them.
//
// The angle is an f32, so its double is exact; the C library's double sin
// and cos of it are within about an ulp of double, and a single rounding to
// f32 then gives the float nearest the true value unless the true value lies
// within a few double ulps of the midpoint between two floats, where the
// result may be the other neighbour: at most one f32 ulp from the correctly
// rounded result. The engine's own table (p9_ref_rope's sincosf,
// src/kernels/portable/reference.rs:294-305) is also within an ulp of it, so
// the two tables agree to an ulp and almost always bit for bit.
#pragma once

#include <cmath>

namespace pcl {

inline void rotation_sincos(float angle, float *s, float *c)
{
    const double a = (double)angle;
    *s = (float)std::sin(a);
    *c = (float)std::cos(a);
}

} // namespace pcl
