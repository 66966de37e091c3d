// softmax.hpp — the online softmax step of the bidirectional matrix-core
// attention kernel (flash.hip).
//
// Layout: a 32x32x16 score product S^T = K . Q^T leaves, for E 32-key slices,
// 16 scores per lane: lane (H, qi) holds keys 16(i/8) + 8H + i%8 of each
// slice for query qi, so a query's keys are split over lanes qi and qi + 32.
// The probabilities are written as binary16 P^T operands of the following
// P.V product: pv[2e + i/8][i%8].
//
// Scores stay raw q.k; the scale and log2(e) fold into one multiply-add
// before exp2 (c = scale * log2 e, which must be positive). The running max
// m is lazy: probabilities are first taken against the current m, and only
// a query whose slice sum then exceeds 2^8 (or that has no max yet) takes
// the rescale path -- it raises m to the true running max, rescales its sum
// and O, and recomputes its probabilities. Every probability is therefore
// at most 2^8 (f16 holds it) and O and the sum always share one m, so the
// quotient O / sum is the softmax-weighted average. The decision is the
// query's own: lanes that do not grow keep their values bit for bit
// (a scale by 1), so a query's result never depends on another query's
// scores; the wave only skips the rescale work when no query needs it.
#pragma once

#include "kernels.hpp"

namespace syn {

// Probabilities of the E slices against m (binary16 P^T operands) and the
// query's sum of them (the same in both of its lanes).
template <int E>
__device__ __forceinline__ float softmax_probs(const f16v (&sc)[E], float c, float m, h8 (&pv)[2 * E]) {
    const float mc = (m == -INFINITY ? 0.0f : m) * c;
#pragma unroll
    for (int e = 0; e < E; ++e) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pv[2 * e + (i >> 3)][i & 7] = to_h(fast_exp2(sc[e][i] * c - mc));
        }
    }
    float ps = 0.0f;
#pragma unroll
    for (int s = 0; s < 2 * E; ++s) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            ps = add_pair(h2{pv[s][i], pv[s][i + 1]}, ps);
        }
    }
    return sum32(ps);
}

// A sweep's first step: no query of the wave has a max yet, so the max is
// taken first (the optimistic pass would send every query to the rescale
// path and compute its probabilities twice).
template <int E>
__device__ __forceinline__ void first_softmax(const f16v (&sc)[E], float c, float& m_run, float& l_run,
                                              h8 (&pv)[2 * E]) {
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < E; ++e) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            tmax = fmaxf(tmax, sc[e][i]);
        }
    }
    m_run = max32(tmax);
    l_run += softmax_probs<E>(sc, c, m_run, pv);
}

// The later steps. The caller takes the first step with first_softmax, out
// of its loop: with both forms in the loop body, the compiler kept the
// output accumulators in two register ranges and copied them across on
// every step (48 moves per step at hd 64).
template <int E, int NT>
__device__ __forceinline__ void online_softmax(const f16v (&sc)[E], float c, float& m_run, float& l_run,
                                               f16v (&o)[NT], h8 (&pv)[2 * E]) {
    float psum = softmax_probs<E>(sc, c, m_run, pv);
    const bool grow = m_run == -INFINITY || !(psum <= 256.0f);
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        float tmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < E; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                // Opaque to the optimiser: otherwise it hoists this max out of
                // the rare branch and every step pays for it.
                float x = sc[e][i];
                asm volatile("" : "+v"(x));
                tmax = fmaxf(tmax, x);
            }
        }
        tmax = max32(tmax);
        const float m_new = grow ? fmaxf(m_run, tmax) : m_run;
        // m_run -inf, m_new finite: alpha 0 (O and the sum are still 0).
        const float alpha = grow && m_new != -INFINITY ? fast_exp2((m_run - m_new) * c) : 1.0f;
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                o[n][i] *= alpha;
            }
        }
        // A query that did not grow recomputes the same values bit for bit.
        psum = softmax_probs<E>(sc, c, m_run, pv);
    }
    l_run += psum;
}

}  // namespace syn
