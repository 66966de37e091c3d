// kv_append.hip — store a run's K and V rows into the binary16 KV state, and
// for a RoPE'd run rotate its q and K rows on the way (one launch).
//
// kv_append (S/kernels/attention.hpp:165-175) for rows pos0..pos0+n-1, as
// session::execute(op_attention) calls it for every token of a run before any
// attention (S/graph/session.hpp:354-356). K keeps the reference's row-major
// layout, so a run's K rows are one contiguous stretch of the cache; V is
// written transposed (V^T[feature][position]).
//
// One grid, two kinds of block:
//  - V blocks: a 64-position x 64-feature tile, read along features with
//    16-byte loads, turned in LDS, written along positions with 16-byte
//    stores. Tiles sit on the cache's 64-position grid, so every full group
//    of 8 positions is one aligned store; the run's ragged ends are written
//    element by element.
//  - K blocks: without RoPE, 4096 consecutive elements of the run's K rows
//    converted to binary16, 16 per thread. With RoPE, one block per
//    position: its first wave builds the position's cos / sin table
//    (rope_angles and rope_table, as the rope kernel does), then the block
//    rotates the position's q row (times the attention temperature) into
//    binary16 q rows and its K row into the cache. The rotated values are the rope kernel's and the
//    temperature kernel's to the bit, and rounding them to binary16 here is
//    the rounding the attention kernels apply to f32 q and the append to f32
//    K, so the fused run equals the separate calls bit for bit.

#include "kernels.hpp"

namespace syn {

namespace {

constexpr uint32_t vt_pos = 64;     // positions per V tile
constexpr uint32_t vt_feat = 64;    // features per V tile
constexpr uint32_t k_chunk = 4096;  // K elements per block without RoPE (2 x 8 per thread)

template <typename T>
__device__ __forceinline__ float load_elem(const T* p) {
    return static_cast<float>(*p);
}

// 8 consecutive elements at p (16-byte aligned) as binary16.
__device__ __forceinline__ h8 load8_h(const float* p) {
    const f4 lo = *reinterpret_cast<const f4*>(p);
    const f4 hi = *reinterpret_cast<const f4*>(p + 4);
    return h8{to_h(lo[0]), to_h(lo[1]), to_h(lo[2]), to_h(lo[3]), to_h(hi[0]), to_h(hi[1]), to_h(hi[2]), to_h(hi[3])};
}
__device__ __forceinline__ h8 load8_h(const _Float16* p) {
    return *reinterpret_cast<const h8*>(p);
}

template <typename T>
__device__ void v_tile(const append_run_args& a, uint32_t tile, _Float16 (*lds)[vt_pos + 8]) {
    const T* v = static_cast<const T*>(a.v_rows);
    const uint32_t f0 = (tile % a.v_feat_tiles) * vt_feat;
    const uint32_t c0 = (a.pos0 & ~(vt_pos - 1)) + (tile / a.v_feat_tiles) * vt_pos;  // first cache position
    const uint32_t end = a.pos0 + a.n;
    const uint32_t t = threadIdx.x;
    // Rows in: 8 features per thread, 8 threads per row, 32 rows per pass;
    // both passes' loads go out before either is written to LDS.
    const uint32_t fl = (t % 8) * 8;
    constexpr uint32_t passes = vt_pos / 32;
    h8 h[passes];
    if (a.vec && c0 >= a.pos0 && c0 + vt_pos <= end && f0 + vt_feat <= a.row) {  // the whole tile: uniform
#pragma unroll
        for (uint32_t q = 0; q < passes; ++q) {
            h[q] = load8_h(v + static_cast<std::size_t>(c0 + t / 8 + 32 * q - a.pos0) * a.row + f0 + fl);
        }
    } else {
#pragma unroll
        for (uint32_t q = 0; q < passes; ++q) {
            const uint32_t c = c0 + t / 8 + 32 * q;
            const bool in = c >= a.pos0 && c < end;
            const std::size_t src = static_cast<std::size_t>(c - a.pos0) * a.row + f0 + fl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                h[q][e] = in && f0 + fl + e < a.row ? to_h(load_elem(v + src + e)) : _Float16(0);
            }
        }
    }
#pragma unroll
    for (uint32_t q = 0; q < passes; ++q) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            lds[fl + e][t / 8 + 32 * q] = h[q][e];
        }
    }
    __syncthreads();
    // V^T out: a feature's 64 positions per 4 threads, 16 each.
    const uint32_t f = t / 4;
    if (f0 + f >= a.row) {
        return;
    }
    _Float16* dst = a.vt_cache + static_cast<std::size_t>(f0 + f) * a.ctx_stride;
#pragma unroll
    for (uint32_t s = 0; s < 2; ++s) {
        const uint32_t pl = (t % 4) * 16 + 8 * s;
        const uint32_t c = c0 + pl;
        const h8 h = *reinterpret_cast<const h8*>(&lds[f][pl]);
        if (c >= a.pos0 && c + 8 <= end) {
            *reinterpret_cast<h8*>(dst + c) = h;
        } else {
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e) {
                if (c + e >= a.pos0 && c + e < end) {
                    dst[c + e] = h[e];
                }
            }
        }
    }
}

template <typename T>
__device__ void k_chunk_of(const append_run_args& a, uint32_t chunk) {
    const T* k = static_cast<const T*>(a.k_rows);
    const std::size_t total = static_cast<std::size_t>(a.n) * a.row;
    const std::size_t i = static_cast<std::size_t>(chunk) * k_chunk + threadIdx.x * 8;
    _Float16* dst = a.k_cache + static_cast<std::size_t>(a.pos0) * a.row;
    constexpr uint32_t parts = k_chunk / 2048;
    if (a.vec && a.pos0 * a.row % 8 == 0 && i + 2048 * (parts - 1) + 8 <= total) {
        h8 h[parts];
#pragma unroll
        for (uint32_t q = 0; q < parts; ++q) {
            h[q] = load8_h(k + i + 2048 * q);
        }
#pragma unroll
        for (uint32_t q = 0; q < parts; ++q) {
            *reinterpret_cast<h8*>(dst + i + 2048 * q) = h[q];
        }
        return;
    }
    for (uint32_t q = 0; q < parts; ++q) {
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            const std::size_t j = i + 2048 * q + e;
            if (j < total) {
                dst[j] = to_h(load_elem(k + j));
            }
        }
    }
}

// Rotates the size / 2 pairs of one row: x (f32) to y (binary16), times mul
// when scaled (the temperature, applied to the rotated values). The block's
// 256 threads; each loads 8 pairs before it computes and stores any, so
// config 3's q row (2048 pairs) is one round trip.
__device__ __forceinline__ void rotate_row(const float* __restrict__ x, _Float16* __restrict__ y, uint32_t size,
                                           uint32_t hd, uint32_t mode, const float* tab, bool scaled, float mul) {
#pragma clang fp contract(off)
    constexpr uint32_t B = 8;
    const uint32_t half = hd / 2;
    const uint32_t pairs = size / 2;
    for (uint32_t u0 = threadIdx.x; u0 < pairs; u0 += 256 * B) {
        float x0[B], x1[B];
#pragma unroll
        for (uint32_t b = 0; b < B; ++b) {
            const uint32_t u = u0 + 256 * b;
            if (u < pairs) {
                if (mode == 0) {
                    // Pair (2u, 2u + 1): u = head * half + p.
                    const float2 xv = *reinterpret_cast<const float2*>(x + 2 * u);
                    x0[b] = xv.x;
                    x1[b] = xv.y;
                } else {
                    const uint32_t e = (u / half) * hd + u % half;
                    x0[b] = x[e];
                    x1[b] = x[e + half];
                }
            }
        }
#pragma unroll
        for (uint32_t b = 0; b < B; ++b) {
            const uint32_t u = u0 + 256 * b;
            if (u < pairs) {
                const uint32_t p = u % half;
                const float cs = tab[p], sn = tab[half + p];
                float y0 = rope_first(x0[b], x1[b], cs, sn);
                float y1 = rope_second(x0[b], x1[b], cs, sn);
                if (scaled) {
                    y0 = y0 * mul;
                    y1 = y1 * mul;
                }
                if (mode == 0) {
                    *reinterpret_cast<h2*>(y + 2 * u) = h2{to_h(y0), to_h(y1)};
                } else {
                    const uint32_t e = (u / half) * hd + p;
                    y[e] = to_h(y0);
                    y[e + half] = to_h(y1);
                }
            }
        }
    }
}

__device__ void rope_position(const append_run_args& a, uint32_t i, float* th, float* tab) {
    const uint32_t half = a.hd / 2;
    const uint32_t pos = a.pos0 + i;
    if (threadIdx.x < 64) {
        if (threadIdx.x == 0) {
            rope_angles(pos, a.r.theta_scale, half, th);
        }
        // The wave's LDS operations complete in order: th is there to read.
        rope_table(a.r, th, half, a.r.freq_factors, tab, threadIdx.x);
    }
    __syncthreads();
    const bool scaled = a.r.temp_floor_len != 0;
    const float t = scaled ? attn_temperature(pos, a.r.temp_scale, a.r.temp_floor_len) : 1.0f;
    rotate_row(a.q + static_cast<std::size_t>(i) * a.q_size, a.q16 + static_cast<std::size_t>(i) * a.q_size,
               a.q_size, a.hd, a.r.mode, tab, scaled, t);
    rotate_row(static_cast<const float*>(a.k_rows) + static_cast<std::size_t>(i) * a.row,
               a.k_cache + static_cast<std::size_t>(pos) * a.row, a.row, a.hd, a.r.mode, tab, false, 1.0f);
}

// grid: v_tiles V blocks, then the K blocks; block 256.
template <typename T, bool ROPE>
__global__ __launch_bounds__(256) void append_run_kernel(const append_run_args a) {
    __shared__ _Float16 tile[vt_feat][vt_pos + 8];  // rows of 144 bytes: 16-byte aligned reads
    __shared__ float th[rope_max_pairs];
    __shared__ float tab[2 * rope_max_pairs];
    const uint32_t b = blockIdx.x;
    if (b < a.v_tiles) {
        v_tile<T>(a, b, tile);
        return;
    }
    if constexpr (ROPE) {
        rope_position(a, b - a.v_tiles, th, tab);
    } else {
        k_chunk_of<T>(a, b - a.v_tiles);
    }
}

}  // namespace

hipError_t launch_append_run(append_run_args a, uint32_t dtype, bool rope, hipStream_t stream) {
    if (a.n == 0) {
        return hipSuccess;
    }
    a.v_feat_tiles = (a.row + vt_feat - 1) / vt_feat;
    a.v_tiles = (a.pos0 % vt_pos + a.n + vt_pos - 1) / vt_pos * a.v_feat_tiles;
    const uint32_t size = dtype == 0 ? 4 : 2;
    a.vec = reinterpret_cast<uintptr_t>(a.k_rows) % 16 == 0 && reinterpret_cast<uintptr_t>(a.v_rows) % 16 == 0 &&
            a.row * size % 16 == 0;
    const uint64_t k_blocks = rope ? a.n : (uint64_t{a.n} * a.row + k_chunk - 1) / k_chunk;
    const uint64_t blocks = a.v_tiles + k_blocks;
    if (blocks > 0x7fffffffu) {
        return hipErrorInvalidValue;
    }
    if (rope) {
        if (dtype != 0) {
            return hipErrorInvalidValue;
        }
        append_run_kernel<float, true><<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(a);
    } else if (dtype == 0) {
        append_run_kernel<float, false><<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(a);
    } else {
        append_run_kernel<_Float16, false><<<static_cast<uint32_t>(blocks), 256, 0, stream>>>(a);
    }
    return hipGetLastError();
}

hipError_t launch_kv_append(const kv_layout& c, const void* k_rows, const void* v_rows, uint32_t n, uint32_t pos0,
                            uint32_t dtype, hipStream_t stream) {
    append_run_args a{};
    a.k_rows = k_rows;
    a.v_rows = v_rows;
    a.k_cache = c.k;
    a.vt_cache = c.vt;
    a.row = c.n_kv * c.hd;
    a.hd = c.hd;
    a.n = n;
    a.pos0 = pos0;
    a.ctx_stride = c.ctx_stride;
    return launch_append_run(a, dtype, false, stream);
}

}  // namespace syn
