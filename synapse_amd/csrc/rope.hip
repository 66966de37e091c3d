// rope.hip — rotary position embedding of n rows (op_rope,
// S/graph/session.hpp:337-342; rope, S/kernels/attention.hpp:89-129).
//
// One block per row; thread p owns pair p of every head. theta_p is built as
// the reference builds it, pos times theta_scale p times in f32 (repeated
// multiplication, not pow), so the angle is the reference's to the last bit;
// cos and sin then come from the device math library.

#include "kernels.hpp"

namespace syn {

namespace {

__global__ __launch_bounds__(128) void rope_kernel(const rope_args a) {
    // Every product and sum rounds on its own, as the reference's
    // -ffp-contract=off build does.
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x;
    const uint32_t half = a.hd / 2;
    const float* x = a.in + static_cast<std::size_t>(i) * a.size;
    float* y = a.out + static_cast<std::size_t>(i) * a.size;
    const uint32_t stride = a.mode == 0 ? 2 : 1;
    const uint32_t offset = a.mode == 0 ? 1 : half;
    for (uint32_t p = threadIdx.x; p < half; p += blockDim.x) {
        float theta = static_cast<float>(a.pos + i);
        for (uint32_t j = 0; j < p; ++j) {
            theta *= a.theta_scale;
        }
        const float ff = a.freq_factors ? a.freq_factors[p] : 1.0f;
        const float theta_extrap = theta / ff;
        const float theta_interp = a.freq_scale * theta_extrap;
        float t = theta_interp;
        float mscale = a.attn_factor;
        if (a.ext_factor != 0.0f) {
            const float yv = (static_cast<float>(p) - a.corr_low) / fmaxf(0.001f, a.corr_high - a.corr_low);
            const float ramp_mix = (1 - fminf(1.0f, fmaxf(0.0f, yv))) * a.ext_factor;
            t = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / a.freq_scale);
        }
        const float cs = cosf(t) * mscale;
        const float sn = sinf(t) * mscale;
        const uint32_t e = stride * p;
        for (uint32_t hb = 0; hb < a.size; hb += a.hd) {
            const float x0 = x[hb + e];
            const float x1 = x[hb + e + offset];
            y[hb + e] = x0 * cs - x1 * sn;
            y[hb + e + offset] = x0 * sn + x1 * cs;
        }
    }
}

}  // namespace

hipError_t launch_rope(const rope_args& a, hipStream_t stream) {
    rope_kernel<<<a.n, 128, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace syn
