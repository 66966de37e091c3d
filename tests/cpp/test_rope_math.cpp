// The RoPE kernels' sin and cos (syn::sincos_of, a Cody-Waite reduction and
// Taylor series in double) against long double sinl / cosl rounded to float:
// every angle's result must be the correctly rounded one, from tiny angles
// to the 2^32 radians a position can reach (RoPE pair 0's angle is the
// position itself). The host build of the same inline function the device
// kernels use.
#define __host__
#define __device__
#include "rope_math.hpp"

#include "check.hpp"

#include <cmath>
#include <cstdint>
#include <random>

int main() {
    std::mt19937_64 g(20261202);
    std::uniform_real_distribution<double> mant(1.0, 2.0);
    long n = 0, wrong = 0;
    const auto one = [&](float t) {
        float s = 0.0f, c = 0.0f;
        syn::sincos_of(t, s, c);
        const auto ws = static_cast<float>(sinl(static_cast<long double>(t)));
        const auto wc = static_cast<float>(cosl(static_cast<long double>(t)));
        ++n;
        if (s != ws || c != wc) {
            ++wrong;
        }
    };
    for (int e = -12; e <= 32; ++e) {
        for (int i = 0; i < 20000; ++i) {
            const auto t = static_cast<float>(std::ldexp(mant(g), e));
            one(t);
            one(-t);
        }
    }
    // Exact multiples of pi/2's neighbours and the positions themselves.
    for (std::uint32_t p = 0; p < 70000; ++p) {
        one(static_cast<float>(p));
    }
    for (std::uint32_t p = 4294900000u; p != 0; ++p) {
        one(static_cast<float>(p));
        if (p > 4294967000u) {
            break;
        }
    }
    std::printf("%ld angles, %ld not correctly rounded\n", n, wrong);
    CHECK(wrong == 0);
    CHECK_DONE();
}
