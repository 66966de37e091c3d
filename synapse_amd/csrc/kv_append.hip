// kv_append.hip — store a run's K and V rows into the binary16 KV state.
//
// kv_append (S/kernels/attention.hpp:165-175) for rows pos0..pos0+n-1, as
// session::execute(op_attention) calls it for every token of a run before any
// attention (S/graph/session.hpp:354-356). K keeps the reference's row-major
// layout; V is written transposed (V^T[feature][position]), so each block
// stages a 32-position x 64-feature tile in LDS and writes it out along
// positions.

#include "kernels.hpp"

namespace syn {

namespace {

constexpr int tile_pos = 32;
constexpr int tile_feat = 64;

template <typename T>
__device__ __forceinline__ float load_elem(const T* p);
template <>
__device__ __forceinline__ float load_elem<float>(const float* p) {
    return *p;
}
template <>
__device__ __forceinline__ float load_elem<_Float16>(const _Float16* p) {
    return static_cast<float>(*p);
}

// grid: (ceil(row / 64), ceil(n / 32)), block 256.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(const T* __restrict__ k_rows, const T* __restrict__ v_rows,
                                                        _Float16* __restrict__ k_cache,
                                                        _Float16* __restrict__ vt_cache, uint32_t row, uint32_t n,
                                                        uint32_t pos0, uint32_t ctx_stride) {
    __shared__ _Float16 tile[tile_feat][tile_pos + 2];
    const int t = threadIdx.x;
    const uint32_t f0 = blockIdx.x * tile_feat;
    const uint32_t p0 = blockIdx.y * tile_pos;
    // Load: features fastest, so each wave reads whole row segments.
    for (int e = t; e < tile_pos * tile_feat; e += 256) {
        const uint32_t p = e / tile_feat;
        const uint32_t f = e % tile_feat;
        const uint32_t gp = p0 + p, gf = f0 + f;
        _Float16 vh = 0;
        if (gp < n && gf < row) {
            const std::size_t src = static_cast<std::size_t>(gp) * row + gf;
            k_cache[static_cast<std::size_t>(pos0 + gp) * row + gf] = to_h(load_elem(k_rows + src));
            vh = to_h(load_elem(v_rows + src));
        }
        tile[f][p] = vh;
    }
    __syncthreads();
    // Store V^T: positions fastest.
    for (int e = t; e < tile_pos * tile_feat; e += 256) {
        const uint32_t f = e / tile_pos;
        const uint32_t p = e % tile_pos;
        const uint32_t gp = p0 + p, gf = f0 + f;
        if (gp < n && gf < row) {
            vt_cache[static_cast<std::size_t>(gf) * ctx_stride + pos0 + gp] = tile[f][p];
        }
    }
}

}  // namespace

hipError_t launch_kv_append(const kv_layout& c, const void* k_rows, const void* v_rows, uint32_t n, uint32_t pos0,
                            uint32_t dtype, hipStream_t stream) {
    const uint32_t row = c.n_kv * c.hd;
    const dim3 grid((row + tile_feat - 1) / tile_feat, (n + tile_pos - 1) / tile_pos);
    if (dtype == 0) {
        kv_append_kernel<float><<<grid, 256, 0, stream>>>(static_cast<const float*>(k_rows),
                                                          static_cast<const float*>(v_rows), c.k, c.vt, row, n, pos0,
                                                          c.ctx_stride);
    } else {
        kv_append_kernel<_Float16><<<grid, 256, 0, stream>>>(static_cast<const _Float16*>(k_rows),
                                                             static_cast<const _Float16*>(v_rows), c.k, c.vt, row, n,
                                                             pos0, c.ctx_stride);
    }
    return hipGetLastError();
}

}  // namespace syn
