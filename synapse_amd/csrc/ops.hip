// ops.hip — the rest of the reference's model graphs on the device: embedding
// rows, RMSNorm and layer norm, F32 matrix products, the element-wise ops
// between them (GELU included) and the pixel shuffle of the CLIP projector.
// With rope.hip and the attention kernels, a whole layer stack runs on the
// GPU from one arena. These follow the reference's session executors
// (S/graph/session.hpp:287-336, :375-378) and kernels
// (S/kernels/elementwise.hpp:28-81, :208-235); they are small and
// latency-bound at decode sizes and are written plainly, one row or one
// output per wave.

#include "kernels.hpp"

#include <atomic>

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

// GELU as ggml's CPU op computes it (S/kernels/elementwise.hpp:115-167):
// x <= -10 gives 0, x >= 10 gives x; otherwise x is rounded to binary16 and
// the tanh approximation of that half, rounded to binary16, is returned --
// the value ggml's 65536-entry table holds, computed here per element.
__device__ __forceinline__ float gelu_f16_table(float x) {
    const float h = static_cast<float>(static_cast<_Float16>(x));
    const float g = 0.5f * h * (1.0f + tanhf(0.79788456080286535587989211986876f * h * (1.0f + 0.044715f * h * h)));
    const float t = static_cast<float>(static_cast<_Float16>(g));
    return x <= -10.0f ? 0.0f : (x >= 10.0f ? x : t);
}

// Element-wise ops (S/kernels/elementwise.hpp:28-81).
__global__ __launch_bounds__(256) void elementwise_kernel(const float* a, const float* b, float* out, uint64_t count,
                                                          uint32_t op, float scalar, uint32_t period) {
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
        case elementwise_gelu:
            y = gelu_f16_table(x);
            break;
        case elementwise_silu:  // kernels::silu
            y = x / (1.0f + expf(-x));
            break;
        case elementwise_add_bias:  // kernels::add_bias on every row
            y = x + b[e % period];
            break;
        default:  // elementwise_scale
            y = x * scalar;
            break;
        }
        out[e] = y;
    }
}

// Row softmax (kernels::softmax, S/kernels/elementwise.hpp:169-199): the row
// maximum subtracted before expf, the exponentials summed in double, and
// every one multiplied by the float of 1 / sum. One block per row; out may
// alias in (each element is read before it is written, by the same thread).
// op_attn_temperature (S/graph/session.hpp:343-347): block i scales row i
// by its position's temperature, each element one f32 multiply
// (kernels::scale).
__global__ __launch_bounds__(256) void temperature_kernel(const float* in, float* out, uint32_t size, uint32_t pos,
                                                          uint32_t floor_len, float scale) {
    const uint32_t i = blockIdx.x;
    const float t = attn_temperature(pos + i, scale, floor_len);
    const std::size_t base = static_cast<std::size_t>(i) * size;
    for (uint32_t e = threadIdx.x; e < size; e += 256) {
        out[base + e] = in[base + e] * t;
    }
}

__global__ __launch_bounds__(256) void softmax_kernel(const float* in, float* out, uint32_t size) {
    __shared__ float wmax[4];
    __shared__ double wsum[4];
    const float* x = in + static_cast<std::size_t>(blockIdx.x) * size;
    float* y = out + static_cast<std::size_t>(blockIdx.x) * size;
    const int w = threadIdx.x >> 6;
    float m = -INFINITY;
    for (uint32_t i = threadIdx.x; i < size; i += 256) {
        m = fmaxf(m, x[i]);
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        m = fmaxf(m, __shfl_xor(m, k, wave));
    }
    if ((threadIdx.x & 63) == 0) {
        wmax[w] = m;
    }
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    double s = 0.0;
    for (uint32_t i = threadIdx.x; i < size; i += 256) {
        const float e = expf(x[i] - m);
        y[i] = e;
        s += e;
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        s += __shfl_xor(s, k, wave);
    }
    if ((threadIdx.x & 63) == 0) {
        wsum[w] = s;
    }
    __syncthreads();
    const float scale = static_cast<float>(1.0 / (((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]));
    for (uint32_t i = threadIdx.x; i < size; i += 256) {
        y[i] *= scale;
    }
}

// out = ((x - mean) * (1 / sqrt(var + eps))) * gamma + beta per row, with the
// reference's accumulation: the mean from a double sum divided in float, the
// variance from a double sum of the float squared deviations
// (S/kernels/elementwise.hpp:240-305).
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* in, const float* gamma, const float* beta,
                                                         float* out, uint32_t size, float eps) {
    __shared__ double part[256];
    __shared__ float stat;
    const float* x = in + static_cast<std::size_t>(blockIdx.x) * size;
    float* y = out + static_cast<std::size_t>(blockIdx.x) * size;
    const auto block_sum = [&](double s) {
        part[threadIdx.x] = s;
        __syncthreads();
        for (uint32_t k = 128; k > 0; k >>= 1) {
            if (threadIdx.x < k) {
                part[threadIdx.x] += part[threadIdx.x + k];
            }
            __syncthreads();
        }
        const double r = part[0];
        __syncthreads();
        return r;
    };
    double s = 0.0;
    for (uint32_t e = threadIdx.x; e < size; e += 256) {
        s += static_cast<double>(x[e]);
    }
    const double sum = block_sum(s);
    if (threadIdx.x == 0) {
        stat = static_cast<float>(sum) / static_cast<float>(size);
    }
    __syncthreads();
    const float mean = stat;
    double q = 0.0;
    for (uint32_t e = threadIdx.x; e < size; e += 256) {
        const float d = x[e] - mean;
        q += static_cast<double>(d * d);
    }
    const double sq = block_sum(q);
    const float scale = 1.0f / sqrtf(static_cast<float>(sq / static_cast<double>(size)) + eps);
    for (uint32_t e = threadIdx.x; e < size; e += 256) {
        const float v = ((x[e] - mean) * scale) * gamma[e];
        y[e] = beta != nullptr ? v + beta[e] : v;
    }
}

// Merge each s x s block of a grid_w x grid_h grid of patch rows (n floats
// each, patch x + grid_w * y) into one row of s^2 n floats: out row
// bx + (grid_w / s) by holds patch (bx s + dx, by s + dy) at offset
// (dy s + dx) n (kernels::pixel_shuffle, S/kernels/elementwise.hpp:307-333).
__global__ __launch_bounds__(256) void pixel_shuffle_kernel(const float* in, float* out, uint32_t n, uint32_t grid_w,
                                                            uint32_t s, uint64_t count) {
    const uint32_t bw = grid_w / s;
    const uint64_t merged = uint64_t{s} * s * n;
    for (uint64_t e = blockIdx.x * 256ull + threadIdx.x; e < count; e += gridDim.x * 256ull) {
        const uint64_t orow = e / merged;
        const uint32_t within = static_cast<uint32_t>(e % merged);
        const uint32_t sub = within / n, k = within % n;
        const uint32_t bx = static_cast<uint32_t>(orow % bw), by = static_cast<uint32_t>(orow / bw);
        const uint32_t dy = sub / s, dx = sub % s;
        out[e] = in[(static_cast<uint64_t>(bx * s + dx) + uint64_t{grid_w} * (by * s + dy)) * n + k];
    }
}

uint32_t grid_for(uint64_t count) {
    const uint64_t blocks = (count + 255) / 256;
    return static_cast<uint32_t>(blocks < 4096 ? (blocks == 0 ? 1 : blocks) : 4096);
}

}  // namespace

uint32_t device_cu_count() {
    constexpr int max_devices = 64;
    static std::atomic<int> cus[max_devices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= max_devices) {
        return 0;
    }
    int v = cus[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) {
            return 0;
        }
        cus[dev].store(v, std::memory_order_relaxed);
    }
    return static_cast<uint32_t>(v);
}

hipError_t launch_embed(const float* table, float* out, const embed_tokens& t, uint32_t n, uint32_t size,
                        hipStream_t stream) {
    const dim3 grid(grid_for(size), n);
    embed_kernel<<<grid, 256, 0, stream>>>(table, out, t, size);
    return hipGetLastError();
}

hipError_t launch_softmax(const float* in, float* out, uint32_t n, uint32_t size, hipStream_t stream) {
    softmax_kernel<<<n, 256, 0, stream>>>(in, out, size);
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

hipError_t launch_layer_norm(const float* in, const float* gamma, const float* beta, float* out, uint32_t n,
                             uint32_t size, float eps, hipStream_t stream) {
    layer_norm_kernel<<<n, 256, 0, stream>>>(in, gamma, beta, out, size, eps);
    return hipGetLastError();
}

hipError_t launch_pixel_shuffle(const float* in, float* out, uint32_t n, uint32_t grid_w, uint32_t grid_h, uint32_t s,
                                hipStream_t stream) {
    const uint64_t count = uint64_t{grid_w} * grid_h * n;
    pixel_shuffle_kernel<<<grid_for(count), 256, 0, stream>>>(in, out, n, grid_w, s, count);
    return hipGetLastError();
}

hipError_t launch_attn_temperature(const float* in, float* out, uint32_t n, uint32_t size, uint32_t pos,
                                   uint32_t floor_len, float scale, hipStream_t stream) {
    temperature_kernel<<<n, 256, 0, stream>>>(in, out, size, pos, floor_len, scale);
    return hipGetLastError();
}

hipError_t launch_elementwise(const float* a, const float* b, float* out, uint64_t count, uint32_t op, float scalar,
                              uint32_t period, hipStream_t stream) {
    elementwise_kernel<<<grid_for(count), 256, 0, stream>>>(a, b, out, count, op, scalar, period);
    return hipGetLastError();
}

}  // namespace syn
