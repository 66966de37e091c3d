// rope.hip — rotary position embedding of n rows (op_rope,
// S/graph/session.hpp:337-342; rope, S/kernels/attention.hpp:89-129).
//
// One block per row: its first wave builds the row's cos / sin table
// (rope_table, which the decode kernel's fused RoPE uses too), then every
// thread rotates pairs of the row's heads.

#include "kernels.hpp"

namespace syn {

namespace {

__global__ __launch_bounds__(256) void rope_kernel(const rope_args a) {
    // Every product and sum rounds on its own, as the reference's
    // -ffp-contract=off build does.
#pragma clang fp contract(off)
    __shared__ float tab[2 * rope_max_pairs];  // cos, then sin, of each pair
    __shared__ float th[rope_max_pairs];        // the pairs' angles
    const uint32_t i = blockIdx.x;
    const uint32_t half = a.hd / 2;
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0) {
            rope_angles(a.pos + (a.period != 0 ? i % a.period : i), a.theta_scale, half, th);
        }
        rope_table(a, th, half, a.freq_factors, tab, threadIdx.x);
    }
    __syncthreads();
    // in and out do not overlap (the C ABI checks): every pair's loads are
    // independent, one memory round trip for the row.
    const float* __restrict__ x = a.in + static_cast<std::size_t>(i) * a.size;
    float* __restrict__ y = a.out + static_cast<std::size_t>(i) * a.size;
    const uint32_t stride = a.mode == 0 ? 2 : 1;
    const uint32_t offset = a.mode == 0 ? 1 : half;
    for (uint32_t u = threadIdx.x; u < a.size / 2; u += 256) {
        const uint32_t p = u % half;
        const uint32_t e = (u / half) * a.hd + stride * p;
        const float x0 = x[e];
        const float x1 = x[e + offset];
        y[e] = rope_first(x0, x1, tab[p], tab[half + p]);
        y[e + offset] = rope_second(x0, x1, tab[p], tab[half + p]);
    }
}

}  // namespace

hipError_t launch_rope(const rope_args& a, hipStream_t stream) {
    rope_kernel<<<a.n, 256, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace syn
