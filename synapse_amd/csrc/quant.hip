// quant.hip — products with quantized weights, as ggml computes them: the
// activations are quantized to the format ggml pairs with the weights
// (Q8_0 for Q4_0 / Q5_0 / Q8_0, Q8_K for Q4_K / Q6_K), then every weight
// block meets its activation block in an exact integer dot, and the block
// scales combine the integers in float. The reference restates the same
// (S/quant/*.hpp, S/kernels/dot.hpp, gemv.hpp:148-166); the block layouts
// are ggml's published ones (ggml-common.h), the quantizers ggml's
// reference quantizers (quantize_row_q8_0_ref, quantize_row_q8_K_ref).
//
// The GEMV is HBM-bound: one wave streams one weight row, each lane a unit
// of 32 weights; a unit's integers are exact whatever the lane order, so
// results differ from ggml's only by float re-association.

#include "kernels.hpp"

// Arithmetic as written (no fused multiply-adds): the dequantized values are
// then bit-identical to ggml's, and the float combines follow its order.
#pragma clang fp contract(off)

namespace syn {

namespace {

__device__ __forceinline__ float half_at(const uint8_t* p) {
    const uint16_t bits = static_cast<uint16_t>(p[0] | (p[1] << 8));
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ float wave_sum_q(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        v += __shfl_xor(v, m, wave);
    }
    return v;
}

// (scale, min) of sub-block j of a Q4_K super-block's 12 packed bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& sc, int& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// ---- activation quantizers -------------------------------------------------------

// Q8_0, one 32-lane half-wave per block: d = amax / 127 stored as binary16,
// q = round-half-away-from-zero(x / d).
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* x, uint8_t* out, uint64_t n_blocks) {
    const uint64_t blk = (static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x) / 32;
    const int l = threadIdx.x & 31;
    if (blk >= n_blocks) {
        return;  // whole half-waves
    }
    const float v = x[blk * 32 + l];
    float amax = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* b = out + blk * 34;
    b[2 + l] = static_cast<uint8_t>(static_cast<int8_t>(roundf(v * id)));
    if (l == 0) {
        const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(d));
        b[0] = static_cast<uint8_t>(h & 0xFF);
        b[1] = static_cast<uint8_t>(h >> 8);
    }
}

// Q8_K, one wave per 256-block: max = the first element of largest
// magnitude, iscale = -127 / max, q = min(127, nearest-even(iscale x)),
// d = 1 / iscale (f32), and the 16 sums of 16.
__global__ __launch_bounds__(256) void quantize_q8_k_kernel(const float* x, uint8_t* out, uint64_t n_blocks) {
    const uint64_t blk = static_cast<uint64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int ln = threadIdx.x & 63;
    if (blk >= n_blocks) {
        return;  // wave-uniform
    }
    const float* src = x + blk * 256;
    float v[4];
    float amax = 0.0f;
    int at = 256;  // index of the first element with the largest magnitude
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = src[4 * ln + i];
        const float a = fabsf(v[i]);
        if (a > amax) {
            amax = a;
            at = 4 * ln + i;
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float oa = __shfl_xor(amax, m, wave);
        const int oi = __shfl_xor(at, m, wave);
        if (oa > amax || (oa == amax && oi < at)) {
            amax = oa;
            at = oi;
        }
    }
    uint8_t* b = out + blk * 292;
    int8_t q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (amax != 0.0f) {
        const float mx = src[at];
        const float iscale = -127.0f / mx;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = static_cast<int8_t>(min(127, static_cast<int>(rintf(iscale * v[i]))));
        }
        d = 1.0f / iscale;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b[4 + 4 * ln + i] = static_cast<uint8_t>(q[i]);
    }
    // Sum of 16 = 4 lanes of 4.
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, wave);
    s += __shfl_xor(s, 2, wave);
    if ((ln & 3) == 0) {
        const uint16_t u = static_cast<uint16_t>(static_cast<int16_t>(s));
        b[260 + 2 * (ln >> 2)] = static_cast<uint8_t>(u & 0xFF);
        b[261 + 2 * (ln >> 2)] = static_cast<uint8_t>(u >> 8);
    }
    if (ln == 0) {
        const uint32_t u = __builtin_bit_cast(uint32_t, d);
        b[0] = static_cast<uint8_t>(u);
        b[1] = static_cast<uint8_t>(u >> 8);
        b[2] = static_cast<uint8_t>(u >> 16);
        b[3] = static_cast<uint8_t>(u >> 24);
    }
}

// ---- the GEMV: one wave per weight row, one lane per 32 weights ------------------
//
// A lane's unit is 32 consecutive weights -- a Q4_0 / Q5_0 / Q8_0 block, or
// one 32-weight slice of a Q4_K / Q6_K super-block -- decoded to 8 dwords of
// non-negative (or, for Q8_0, signed) int8 values, dotted with the matching
// 32 activation int8 by v_dot4, and the format's offset (8, 16, 32) taken
// out through the activation sums. Every integer is exact, so a unit's sum
// is ggml's; the float combination differs only by association. The wave's
// loads of one row are contiguous across its lanes; rows are read through a
// buffer resource of the row's bytes, so the unaligned windows below can
// over-read the last block and see zeros.

__device__ __forceinline__ uint32_t ld32(rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ uint32_t ld16(rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// N dwords of the byte stream at a 2-byte aligned offset: N + 1 aligned
// dwords realigned with v_alignbyte.
template <int N>
__device__ __forceinline__ void window(rsrc r, uint32_t off, uint32_t (&d)[N]) {
    const uint32_t base = off & ~3u, sh = off & 3u;
    uint32_t w[N + 1];
#pragma unroll
    for (int k = 0; k <= N; ++k) {
        w[k] = ld32(r, base + 4 * k);
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
        d[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], sh);
    }
}

__device__ __forceinline__ int dot8(const uint32_t (&a)[8], const uint32_t (&b)[8], int first, int last) {
    int s = 0;
#pragma unroll
    for (int k = first; k < last; ++k) {
        s = __builtin_amdgcn_sdot4(static_cast<int>(a[k]), static_cast<int>(b[k]), s, false);
    }
    return s;
}

// Bits 0..3 of x to bit 4 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
    return ((x & 1u) << 4) | ((x & 2u) << 11) | ((x & 4u) << 18) | ((x & 8u) << 25);
}

template <uint32_t T>
constexpr uint32_t block_bytes = T == qtype_q4_0 ? 18 : T == qtype_q5_0 ? 22 : T == qtype_q8_0 ? 34 : T == qtype_q4_k ? 144 : 210;

template <uint32_t T>
constexpr bool k_quant = T == qtype_q4_k || T == qtype_q6_k;

template <uint32_t T, int NR>
__global__ __launch_bounds__(256) void gemv_q_kernel(const uint8_t* w, const uint8_t* act, const float* bias,
                                                     float* out, uint32_t n, uint32_t rows, uint32_t cols) {
    const uint32_t o = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (o >= rows) {
        return;  // wave-uniform
    }
    const uint32_t ln = threadIdx.x & 63;
    const uint32_t r0 = blockIdx.y * NR;
    const uint32_t units = cols / 32;
    const uint32_t wrow = cols / (k_quant<T> ? 256 : 32) * block_bytes<T>;
    const uint32_t arow = k_quant<T> ? cols / 256 * 292 : cols / 32 * 34;
    const rsrc wr = make_rsrc(w + static_cast<std::size_t>(o) * wrow, wrow);
    rsrc ar[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        // Rows past n (the last group's tail) read row n - 1; never stored.
        ar[i] = make_rsrc(act + static_cast<std::size_t>(min(r0 + i, n - 1)) * arow, arow);
    }
    float acc[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        acc[i] = 0.0f;
    }
    constexpr uint32_t nib = 0x0F0F0F0Fu, ones = 0x01010101u;
#pragma unroll 2
    for (uint32_t u = ln; u < units; u += 64) {
        uint32_t q[8];
        if constexpr (k_quant<T>) {
            const uint32_t sb = u / 8, s = u % 8;
            if constexpr (T == qtype_q4_k) {
                const uint32_t b = sb * 144;
                const u4 h = buffer_load16(wr, b);  // d, dmin, 12 scale bytes
                const u4 q0 = buffer_load16(wr, b + 16 + 32 * (s / 2));
                const u4 q1 = buffer_load16(wr, b + 32 + 32 * (s / 2));
                const uint32_t shift = (s & 1) * 4;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    q[k] = (q0[k] >> shift) & nib;
                    q[4 + k] = (q1[k] >> shift) & nib;
                }
                const auto byte = [&](uint32_t j) { return (h[1 + j / 4] >> (8 * (j % 4))) & 0xFFu; };
                int sc, m;
                if (s < 4) {
                    sc = static_cast<int>(byte(s) & 63);
                    m = static_cast<int>(byte(s + 4) & 63);
                } else {
                    sc = static_cast<int>((byte(s + 4) & 0xF) | ((byte(s - 4) >> 6) << 4));
                    m = static_cast<int>((byte(s + 4) >> 4) | ((byte(s) >> 6) << 4));
                }
                const float d = half_bits(h[0]), dmin = half_bits(h[0] >> 16);
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    const uint32_t a = sb * 292;
                    const float yd = __builtin_bit_cast(float, ld32(ar[i], a));
                    const u4 y0 = buffer_load16(ar[i], a + 4 + 32 * s);
                    const u4 y1 = buffer_load16(ar[i], a + 20 + 32 * s);
                    const uint32_t bs = ld32(ar[i], a + 260 + 4 * s);
                    const uint32_t y[8] = {y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
                    const int isum = sc * dot8(q, y, 0, 8);
                    const int imin = m * (static_cast<int16_t>(bs & 0xFFFF) + static_cast<int16_t>(bs >> 16));
                    acc[i] += (d * yd) * static_cast<float>(isum) - (dmin * yd) * static_cast<float>(imin);
                }
            } else {  // Q6_K: slice s is quarter s % 4 of half s / 4
                const uint32_t b = sb * 210, hf = s / 4, k4 = s % 4;
                uint32_t lo[8], hi[8];
                window(wr, b + 64 * hf + 32 * (k4 & 1), lo);
                window(wr, b + 128 + 32 * hf, hi);
                const uint32_t scp = ld16(wr, b + 192 + 8 * hf + 2 * k4);
                const float d = half_bits(ld16(wr, b + 208));
                const uint32_t lshift = (k4 >> 1) * 4;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    q[k] = ((lo[k] >> lshift) & nib) | (((hi[k] >> (2 * k4)) & 0x03030303u) << 4);
                }
                const int sc0 = static_cast<int8_t>(scp & 0xFF), sc1 = static_cast<int8_t>(scp >> 8);
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    const uint32_t a = sb * 292;
                    const float yd = __builtin_bit_cast(float, ld32(ar[i], a));
                    const u4 y0 = buffer_load16(ar[i], a + 4 + 32 * s);
                    const u4 y1 = buffer_load16(ar[i], a + 20 + 32 * s);
                    const uint32_t bs = ld32(ar[i], a + 260 + 4 * s);
                    const uint32_t y[8] = {y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
                    const int s0 = dot8(q, y, 0, 4) - 32 * static_cast<int16_t>(bs & 0xFFFF);
                    const int s1 = dot8(q, y, 4, 8) - 32 * static_cast<int16_t>(bs >> 16);
                    acc[i] += (d * yd) * static_cast<float>(sc0 * s0 + sc1 * s1);
                }
            }
        } else {
            const uint32_t b = u * block_bytes<T>;
            const float d = half_bits(ld16(wr, b));
            int offset = 0;  // the format's zero point, taken out through the activation sum
            if constexpr (T == qtype_q8_0) {
                window(wr, b + 2, q);
            } else if constexpr (T == qtype_q4_0) {
                uint32_t qs[4];
                window(wr, b + 2, qs);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    q[k] = qs[k] & nib;
                    q[4 + k] = (qs[k] >> 4) & nib;
                }
                offset = 8;
            } else {  // Q5_0
                uint32_t qh[1], qs[4];
                window(wr, b + 2, qh);
                window(wr, b + 6, qs);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    q[k] = (qs[k] & nib) | spread4((qh[0] >> (4 * k)) & 0xF);
                    q[4 + k] = ((qs[k] >> 4) & nib) | spread4((qh[0] >> (16 + 4 * k)) & 0xF);
                }
                offset = 16;
            }
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const uint32_t a = u * 34;
                const float da = half_bits(ld16(ar[i], a));
                uint32_t y[8];
                window(ar[i], a + 2, y);
                int sumi = dot8(q, y, 0, 8);
                if (offset != 0) {
                    const uint32_t one8[8] = {ones, ones, ones, ones, ones, ones, ones, ones};
                    sumi -= offset * dot8(one8, y, 0, 8);
                }
                acc[i] += static_cast<float>(sumi) * (d * da);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const float s = wave_sum_q(acc[i]);
        if (ln == 0 && r0 + i < n) {
            out[static_cast<std::size_t>(r0 + i) * rows + o] = bias != nullptr ? s + bias[o] : s;
        }
    }
}

// ---- dequantized rows (embedding lookups) ------------------------------------------

template <uint32_t T>
__device__ __forceinline__ float dequant_at(const uint8_t* row, uint32_t e) {
    if constexpr (T == qtype_q4_0 || T == qtype_q5_0 || T == qtype_q8_0) {
        const uint32_t wbytes = T == qtype_q8_0 ? 34 : (T == qtype_q4_0 ? 18 : 22);
        const uint8_t* b = row + std::size_t{e / 32} * wbytes;
        const uint32_t j = e % 32;
        const float d = half_at(b);
        if constexpr (T == qtype_q8_0) {
            return static_cast<float>(reinterpret_cast<const int8_t*>(b + 2)[j]) * d;
        } else if constexpr (T == qtype_q4_0) {
            const int q = j < 16 ? (b[2 + j] & 0xF) : (b[2 + j - 16] >> 4);
            return static_cast<float>(q - 8) * d;
        } else {
            const uint32_t qh = b[2] | (b[3] << 8) | (b[4] << 16) | (static_cast<uint32_t>(b[5]) << 24);
            const uint32_t jj = j % 16;
            const int q = j < 16 ? ((b[6 + jj] & 0xF) | (((qh >> jj) << 4) & 0x10))
                                 : ((b[6 + jj] >> 4) | ((qh >> (jj + 12)) & 0x10));
            return static_cast<float>(q - 16) * d;
        }
    } else if constexpr (T == qtype_q4_k) {
        const uint8_t* b = row + std::size_t{e / 256} * 144;
        const uint32_t k = e % 256, sub = k / 32, l = k % 32;
        int sc, m;
        scale_min_k4(static_cast<int>(sub), b + 4, sc, m);
        const uint8_t q = b[16 + 32 * (sub / 2) + l];
        const int v = (sub & 1) ? (q >> 4) : (q & 0xF);
        return (half_at(b) * static_cast<float>(sc)) * static_cast<float>(v) - half_at(b + 2) * static_cast<float>(m);
    } else {  // Q6_K
        const uint8_t* b = row + std::size_t{e / 256} * 210;
        const uint32_t k = e % 256, n = k / 128, kk = k % 128, quarter = kk / 32, l = kk % 32;
        const int QL = b[64 * n + l + (quarter & 1) * 32], QH = b[128 + 32 * n + l];
        const int lowbits = quarter < 2 ? (QL & 0xF) : (QL >> 4);
        const int q = (lowbits | (((QH >> (2 * quarter)) & 3) << 4)) - 32;
        const int8_t sc = reinterpret_cast<const int8_t*>(b + 192)[8 * n + l / 16 + 2 * quarter];
        return (half_at(b + 208) * static_cast<float>(sc)) * static_cast<float>(q);
    }
}

template <uint32_t T>
__global__ __launch_bounds__(256) void embed_q_kernel(const uint8_t* table, float* out, embed_tokens t, uint32_t size,
                                                      uint64_t row_bytes) {
    const uint32_t i = blockIdx.y;
    const uint8_t* row = table + static_cast<std::size_t>(t.token[i]) * row_bytes;
    float* dst = out + static_cast<std::size_t>(i) * size;
    for (uint32_t e = blockIdx.x * 256 + threadIdx.x; e < size; e += gridDim.x * 256) {
        dst[e] = dequant_at<T>(row, e);
    }
}

uint32_t q_grid(uint64_t count) {
    const uint64_t blocks = (count + 255) / 256;
    return static_cast<uint32_t>(blocks < 4096 ? (blocks == 0 ? 1 : blocks) : 4096);
}

}  // namespace

bool qtype_known(uint32_t t) {
    return t == qtype_q4_0 || t == qtype_q5_0 || t == qtype_q8_0 || t == qtype_q4_k || t == qtype_q6_k;
}

uint32_t qtype_block(uint32_t t) {
    return t == qtype_q4_k || t == qtype_q6_k ? 256 : 32;
}

uint64_t qtype_row_bytes(uint32_t t, uint32_t cols) {
    const uint64_t per = t == qtype_q4_0 ? 18 : t == qtype_q5_0 ? 22 : t == qtype_q8_0 ? 34 : t == qtype_q4_k ? 144 : 210;
    return uint64_t{cols} / qtype_block(t) * per;
}

uint64_t qtype_act_bytes(uint32_t t, uint32_t n, uint32_t cols) {
    return t == qtype_q4_k || t == qtype_q6_k ? uint64_t{n} * (cols / 256) * 292 : uint64_t{n} * (cols / 32) * 34;
}

hipError_t launch_matmul_q(uint32_t t, const uint8_t* w, const float* x, uint8_t* act, const float* bias, float* out,
                           uint32_t n, uint32_t rows, uint32_t cols, hipStream_t stream) {
    if (t == qtype_q4_k || t == qtype_q6_k) {
        const uint64_t nb = uint64_t{n} * (cols / 256);
        quantize_q8_k_kernel<<<static_cast<uint32_t>((nb + 3) / 4), 256, 0, stream>>>(x, act, nb);
    } else {
        const uint64_t nb = uint64_t{n} * (cols / 32);
        quantize_q8_0_kernel<<<static_cast<uint32_t>((nb + 7) / 8), 256, 0, stream>>>(x, act, nb);
    }
    const uint32_t nr = n >= 4 ? 4 : (n >= 2 ? 2 : 1);
    const dim3 grid((rows + 3) / 4, (n + nr - 1) / nr);
    const auto go = [&]<uint32_t T>() {
        if (nr == 4) {
            gemv_q_kernel<T, 4><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        } else if (nr == 2) {
            gemv_q_kernel<T, 2><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        } else {
            gemv_q_kernel<T, 1><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        }
    };
    switch (t) {
    case qtype_q4_0:
        go.template operator()<qtype_q4_0>();
        break;
    case qtype_q5_0:
        go.template operator()<qtype_q5_0>();
        break;
    case qtype_q8_0:
        go.template operator()<qtype_q8_0>();
        break;
    case qtype_q4_k:
        go.template operator()<qtype_q4_k>();
        break;
    default:
        go.template operator()<qtype_q6_k>();
        break;
    }
    return hipGetLastError();
}

hipError_t launch_embed_q(uint32_t t, const uint8_t* table, float* out, const embed_tokens& tk, uint32_t n,
                          uint32_t size, hipStream_t stream) {
    const dim3 grid(q_grid(size), n);
    const uint64_t rb = qtype_row_bytes(t, size);
    switch (t) {
    case qtype_q4_0:
        embed_q_kernel<qtype_q4_0><<<grid, 256, 0, stream>>>(table, out, tk, size, rb);
        break;
    case qtype_q5_0:
        embed_q_kernel<qtype_q5_0><<<grid, 256, 0, stream>>>(table, out, tk, size, rb);
        break;
    case qtype_q8_0:
        embed_q_kernel<qtype_q8_0><<<grid, 256, 0, stream>>>(table, out, tk, size, rb);
        break;
    case qtype_q4_k:
        embed_q_kernel<qtype_q4_k><<<grid, 256, 0, stream>>>(table, out, tk, size, rb);
        break;
    default:
        embed_q_kernel<qtype_q6_k><<<grid, 256, 0, stream>>>(table, out, tk, size, rb);
        break;
    }
    return hipGetLastError();
}

}  // namespace syn
