// generic.hip — plain f32 attention kernels for the shapes the matrix-core
// kernels do not take: head_dim not a multiple of 8 (the reference accepts
// any head_dim <= 256, S/graph/graph.hpp:698-719) and more than 16 query
// heads per KV head. One wave per (row, head); each lane owns head dims
// lane, lane+64, ...; online softmax over the keys. Same rounding points as
// the fast kernels: q and k operands in f16 (exactly the reference's for the
// causal path), p rounded to f16.

#include "kernels.hpp"

namespace syn {

namespace {

template <bool CAUSAL, bool F16>
__global__ __launch_bounds__(64) void generic_kernel(const flash_args a) {
    const int ln = threadIdx.x;
    const uint32_t i = blockIdx.x;  // query row inside the image
    const uint32_t h = blockIdx.y;
    const uint32_t img = blockIdx.z;
    const uint32_t g = h / a.group;
    const uint32_t hd = a.hd;
    const std::size_t row_base = static_cast<std::size_t>(img) * a.n;
    const float c = a.scale_log2e;

    const auto load = [&](const void* p, std::size_t idx) -> float {
        if constexpr (F16) {
            return static_cast<float>(static_cast<const _Float16*>(p)[idx]);
        } else {
            return static_cast<const float*>(p)[idx];
        }
    };

    float q[4], o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = ln + 64 * j;
        q[j] = d < hd ? static_cast<float>(to_h(load(a.q, (row_base + i) * a.q_row + h * hd + d))) : 0.0f;
        o[j] = 0.0f;
    }
    const uint32_t n_keys = CAUSAL ? a.pos + i + 1 : a.kv_len;
    float m_run = -INFINITY, l_run = 0.0f;
    for (uint32_t t = 0; t < n_keys; ++t) {
        float dot = 0.0f;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = ln + 64 * j;
            float kd = 0.0f, vd = 0.0f;
            if (d < hd) {
                if constexpr (CAUSAL) {
                    kd = static_cast<float>(a.k[static_cast<std::size_t>(t) * a.row + g * hd + d]);
                    vd = static_cast<float>(a.vt[static_cast<std::size_t>(g * hd + d) * a.ctx_stride + t]);
                } else {
                    kd = static_cast<float>(to_h(load(a.k_rows, (row_base + t) * a.row + g * hd + d)));
                    vd = static_cast<float>(to_h(load(a.v_rows, (row_base + t) * a.row + g * hd + d)));
                }
            }
            dot += q[j] * kd;
            v[j] = vd;
        }
#pragma unroll
        for (int mask = 32; mask >= 1; mask >>= 1) {
            dot = xor_sum(dot, mask);
        }
        const float m_new = fmaxf(m_run, dot);
        const float alpha = fast_exp2((m_run - m_new) * c);
        const float p = static_cast<float>(to_h(fast_exp2((dot - m_new) * c)));
        l_run = l_run * alpha + p;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            o[j] = o[j] * alpha + p * v[j];
        }
        m_run = m_new;
    }
    float* out = a.out + (row_base + i) * a.q_row + h * hd;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = ln + 64 * j;
        if (d < hd) {
            out[d] = o[j] / l_run;
        }
    }
}

// Image-encoder attention on f32 rows, close to the reference's arithmetic
// (self_attend_head, S/kernels/attention.hpp:324-486). What follows the
// reference's order: a score is acc = fma(q_d, k_d, acc) over d from 0,
// times scale; the max is subtracted (exact in any order); each probability
// is e_j * float(1 / sum); an output element is acc = fma(p_j, v_j, acc) over
// j from 0. What does not: the exponential is the device's expf, not the
// host libm's std::exp, and the double sum of the exponentials is taken per
// lane over keys l, l + 64, ... and then across the lanes by an xor tree,
// where the reference adds them in key order (S/kernels/elementwise.hpp:
// 190-194). Both differ from the reference in the last bits only, and no
// binary16 rounding happens anywhere, so f32 inputs keep f32 precision end to
// end (the tests hold it within 2e-6 of the largest output). One wave per
// (query row, head, image): lane l scores keys l, l + 64, ... (each chain in
// order), the probabilities sit in LDS, and lane l then sums output dims
// l, l + 64, ... over the keys in order. The f16-input and long-image shapes
// take the matrix-core kernel.
__global__ __launch_bounds__(64) void self_f32_kernel(const flash_args a) {
    extern __shared__ float probs[];  // n
    const int ln = threadIdx.x;
    const uint32_t i = blockIdx.x;
    const uint32_t h = blockIdx.y;
    const uint32_t img = blockIdx.z;
    const uint32_t hd = a.hd;
    const uint32_t n = a.n;
    const std::size_t row_base = static_cast<std::size_t>(img) * n;
    const float* q = static_cast<const float*>(a.q) + (row_base + i) * a.q_row + static_cast<std::size_t>(h) * hd;
    const float* kb = static_cast<const float*>(a.k_rows) + row_base * a.row + static_cast<std::size_t>(h) * hd;
    const float* vb = static_cast<const float*>(a.v_rows) + row_base * a.row + static_cast<std::size_t>(h) * hd;

    float mx = -INFINITY;
    for (uint32_t j = ln; j < n; j += 64) {
        const float* kj = kb + static_cast<std::size_t>(j) * a.row;
        float acc = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) {
            acc = fmaf(q[d], kj[d], acc);
        }
        const float sj = acc * a.scale;
        probs[j] = sj;
        mx = fmaxf(mx, sj);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        mx = xor_max(mx, m);
    }
    double sum = 0.0;
    for (uint32_t j = ln; j < n; j += 64) {
        const float e = expf(probs[j] - mx);
        probs[j] = e;
        sum += e;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        sum += __shfl_xor(sum, m, wave);
    }
    const auto inv = static_cast<float>(1.0 / sum);
    for (uint32_t j = ln; j < n; j += 64) {
        probs[j] *= inv;
    }
    __syncthreads();  // every lane reads every probability below
    float* out = a.out + (row_base + i) * a.q_row + static_cast<std::size_t>(h) * hd;
    for (uint32_t e = ln; e < hd; e += 64) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < n; ++j) {
            acc = fmaf(probs[j], vb[static_cast<std::size_t>(j) * a.row + e], acc);
        }
        out[e] = acc;
    }
}

}  // namespace

bool self_f32_fits(uint32_t n) {
    return n <= self_f32_max_keys;
}

hipError_t launch_self_f32(const flash_args& a, hipStream_t stream) {
    const dim3 grid(a.n, a.n_heads, a.batch);
    self_f32_kernel<<<grid, 64, a.n * sizeof(float), stream>>>(a);
    return hipGetLastError();
}

hipError_t launch_generic_causal(const flash_args& a, uint32_t q_dtype, hipStream_t stream) {
    const dim3 grid(a.n, a.n_heads, 1);
    if (q_dtype == 1) {
        generic_kernel<true, true><<<grid, 64, 0, stream>>>(a);
    } else {
        generic_kernel<true, false><<<grid, 64, 0, stream>>>(a);
    }
    return hipGetLastError();
}

hipError_t launch_generic_bidirectional(const flash_args& a, uint32_t in_dtype, hipStream_t stream) {
    const dim3 grid(a.n, a.n_heads, a.batch);
    if (in_dtype == 1) {
        generic_kernel<false, true><<<grid, 64, 0, stream>>>(a);
    } else {
        generic_kernel<false, false><<<grid, 64, 0, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace syn
