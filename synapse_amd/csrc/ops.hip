// ops.hip — the rest of a Llama-family decode graph on the device: embedding
// rows, RMSNorm, F32 matrix products, and the element-wise ops between them.
// With rope.hip and the attention kernels, a whole layer stack runs on the
// GPU from one arena. These follow the reference's session executors
// (S/graph/session.hpp:287-336, :375-378) and kernels
// (S/kernels/elementwise.hpp:28-81, :208-235); they are small and
// latency-bound at decode sizes and are written plainly, one row or one
// output per wave.

#include "kernels.hpp"

namespace syn {

namespace {

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        v += __shfl_xor(v, m, wave);
    }
    return v;
}

// out row i = table row tokens[i] (session::execute(op_embed), :331-336).
__global__ __launch_bounds__(256) void embed_kernel(const float* table, float* out, embed_tokens t, uint32_t size) {
    const uint32_t i = blockIdx.y;
    const float* src = table + static_cast<std::size_t>(t.token[i]) * size;
    float* dst = out + static_cast<std::size_t>(i) * size;
    for (uint32_t e = blockIdx.x * 256 + threadIdx.x; e < size; e += gridDim.x * 256) {
        dst[e] = src[e];
    }
}

// out = (x * (1 / sqrt(mean(x^2) + eps))) * gamma per row, the squares summed
// in double as the reference sums them (S/kernels/elementwise.hpp:208-235).
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* in, const float* gamma, float* out, uint32_t size,
                                                       float eps) {
    __shared__ double part[256];
    __shared__ float scale_s;
    const float* x = in + static_cast<std::size_t>(blockIdx.x) * size;
    float* y = out + static_cast<std::size_t>(blockIdx.x) * size;
    double s = 0.0;
    for (uint32_t e = threadIdx.x; e < size; e += 256) {
        const float v = x[e];
        s += static_cast<double>(v * v);
    }
    part[threadIdx.x] = s;
    __syncthreads();
    for (uint32_t k = 128; k > 0; k >>= 1) {
        if (threadIdx.x < k) {
            part[threadIdx.x] += part[threadIdx.x + k];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float mean = static_cast<float>(part[0] / static_cast<double>(size));
        scale_s = 1.0f / sqrtf(mean + eps);
    }
    __syncthreads();
    const float sc = scale_s;
    for (uint32_t e = threadIdx.x; e < size; e += 256) {
        y[e] = (x[e] * sc) * gamma[e];
    }
}

// out[r][o] = sum_c w[o][c] x[r][c] (+ bias[o]): one wave per output element,
// lanes striding over the columns (session::execute(op_matmul), :287-302;
// op_add_bias, :306-312).
__global__ __launch_bounds__(256) void matmul_kernel(const float* w, const float* x, const float* bias, float* out,
                                                     uint32_t rows, uint32_t cols) {
    const uint32_t o = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t r = blockIdx.y;
    if (o >= rows) {
        return;  // wave-uniform
    }
    const uint32_t ln = threadIdx.x & 63;
    const float* wr = w + static_cast<std::size_t>(o) * cols;
    const float* xr = x + static_cast<std::size_t>(r) * cols;
    float acc = 0.0f;
    for (uint32_t c = ln; c < cols; c += 64) {
        acc += wr[c] * xr[c];
    }
    acc = wave_sum_f(acc);
    if (ln == 0) {
        out[static_cast<std::size_t>(r) * rows + o] = bias != nullptr ? acc + bias[o] : acc;
    }
}

// Element-wise ops (S/kernels/elementwise.hpp:28-81).
__global__ __launch_bounds__(256) void elementwise_kernel(const float* a, const float* b, float* out, uint64_t count,
                                                          uint32_t op, float scalar) {
    for (uint64_t e = blockIdx.x * 256ull + threadIdx.x; e < count; e += gridDim.x * 256ull) {
        const float x = a[e];
        float y;
        switch (op) {
        case elementwise_add:
            y = x + b[e];
            break;
        case elementwise_mul:
            y = x * b[e];
            break;
        case elementwise_silu_mul:
            // silu(x) = x / (1 + exp(-x)) rounded to float, then the product,
            // as op_silu followed by op_mul computes it.
            y = (x / (1.0f + expf(-x))) * b[e];
            break;
        default:  // elementwise_scale
            y = x * scalar;
            break;
        }
        out[e] = y;
    }
}

uint32_t grid_for(uint64_t count) {
    const uint64_t blocks = (count + 255) / 256;
    return static_cast<uint32_t>(blocks < 4096 ? (blocks == 0 ? 1 : blocks) : 4096);
}

}  // namespace

hipError_t launch_embed(const float* table, float* out, const embed_tokens& t, uint32_t n, uint32_t size,
                        hipStream_t stream) {
    const dim3 grid(grid_for(size), n);
    embed_kernel<<<grid, 256, 0, stream>>>(table, out, t, size);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float* in, const float* gamma, float* out, uint32_t n, uint32_t size, float eps,
                           hipStream_t stream) {
    rms_norm_kernel<<<n, 256, 0, stream>>>(in, gamma, out, size, eps);
    return hipGetLastError();
}

hipError_t launch_matmul(const float* w, const float* x, const float* bias, float* out, uint32_t n, uint32_t rows,
                         uint32_t cols, hipStream_t stream) {
    const dim3 grid((rows + 3) / 4, n);
    matmul_kernel<<<grid, 256, 0, stream>>>(w, x, bias, out, rows, cols);
    return hipGetLastError();
}

hipError_t launch_elementwise(const float* a, const float* b, float* out, uint64_t count, uint32_t op, float scalar,
                              hipStream_t stream) {
    elementwise_kernel<<<grid_for(count), 256, 0, stream>>>(a, b, out, count, op, scalar);
    return hipGetLastError();
}

}  // namespace syn
