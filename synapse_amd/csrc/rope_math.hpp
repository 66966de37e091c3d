// rope_math.hpp -- sin and cos of a RoPE angle, for the device kernels and
// (with __host__ and __device__ defined away) the CPU test that pins them.
#pragma once

#include <cmath>

namespace syn {

// sin and cos of an f32 angle t, rounded to f32 from a double evaluation
// (Cody-Waite reduction and Taylor series): t - k pi/2 with pi/2 held as two
// doubles (exact enough for |t| < 2^32), then the series of sin and cos
// about 0 on the remainder (|r| <= pi/4, to the r^17 and r^18 terms: the
// first term left out is below 1e-19) in nested form, and the quadrant k mod
// 4 picks and signs the pair. The f32 math library's large-angle reduction
// (angles reach pos radians) cost registers and time in the decode kernel;
// this is a few dozen fp64 operations, accurate to about 1e-16, so the f32
// result is the correctly rounded one but in the rarest ties.
__host__ __device__ inline void sincos_of(float t, float& sn, float& cs) {
    constexpr double half_pi_hi = 1.5707963267948966;     // pi/2 rounded to double
    constexpr double half_pi_lo = 6.123233995736766e-17;  // pi/2 - half_pi_hi
    constexpr double two_over_pi = 0.6366197723675814;
    const double x = t;
    const double k = rint(x * two_over_pi);
    const double r = fma(-k, half_pi_lo, fma(-k, half_pi_hi, x));
    const double r2 = r * r;
    // sin r = r (1 - r^2/(2*3) (1 - r^2/(4*5) (... (1 - r^2/(16*17))))),
    // cos r = 1 - r^2/(1*2) (1 - r^2/(3*4) (... (1 - r^2/(17*18)))).
    double s = 1.0;
    double c = 1.0;
#pragma unroll
    for (int j = 9; j >= 1; --j) {
        c = 1.0 - r2 * (1.0 / ((2.0 * j - 1.0) * (2.0 * j))) * c;
        if (j <= 8) {
            s = 1.0 - r2 * (1.0 / ((2.0 * j) * (2.0 * j + 1.0))) * s;
        }
    }
    s *= r;
    const auto q = static_cast<unsigned>(static_cast<long long>(k) & 3);
    const double sv = q == 0 ? s : q == 1 ? c : q == 2 ? -s : -c;
    const double cv = q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
    sn = static_cast<float>(sv);
    cs = static_cast<float>(cv);
}

}  // namespace syn
