// quant.hpp -- pieces shared by the quantized GEMV and GEMM (quant.hip,
// quant_gemm.hip): ggml's block formats, buffer loads of 2-byte aligned
// streams, and ggml's reference activation quantizers (Q8_0, Q8_K), one lane
// per 32 values. Included by one translation unit each, inside an anonymous
// namespace.
#pragma once

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

// ---- buffer loads ------------------------------------------------------------------

__device__ __forceinline__ uint32_t ld32(rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ uint32_t ld16(rsrc r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

__device__ __forceinline__ float half_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
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

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xFF) | ((static_cast<uint32_t>(b) & 0xFF) << 8) |
           ((static_cast<uint32_t>(c) & 0xFF) << 16) | (static_cast<uint32_t>(d) << 24);
}

template <uint32_t T>
constexpr uint32_t block_bytes = T == qtype_q4_0   ? 18
                                 : T == qtype_q5_0 ? 22
                                 : T == qtype_q8_0 ? 34
                                 : T == qtype_q4_k ? 144
                                                   : 210;

template <uint32_t T>
constexpr bool k_quant = T == qtype_q4_k || T == qtype_q6_k;

// ---- activations: ggml's reference quantizers, one lane per 32 values -----------

// A lane's 32 quantized activations: the int8 values (4 per dword), the
// block scale as the dot reads it, and sums of the values (Q8_K: the two
// sums of 16 it stores; Q8_0: the sum of all 32).
struct act_unit {
    uint32_t q[8];
    float d;
    int s0, s1;
};

// x[32u, 32u + 32), loaded apart from its quantization so that the loads
// can be issued ahead of others.
struct x_unit {
    f4 v[8];
};

__device__ __forceinline__ x_unit load_x(const float* x, uint32_t u) {
    const f4* src = reinterpret_cast<const f4*>(x + 32 * static_cast<std::size_t>(u));
    x_unit r;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        r.v[k] = src[k];
    }
    return r;
}

// Q8_0 of one unit: d = amax / 127 stored as binary16,
// q = round-half-away-from-zero(x / d) (quantize_row_q8_0_ref).
__device__ __forceinline__ act_unit quantize_q8_0(const x_unit& xu, uint16_t& d_bits) {
    const f4 (&v)[8] = xu.v;
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            amax = fmaxf(amax, fabsf(v[k][i]));
        }
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    act_unit a;
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        int q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = static_cast<int>(roundf(v[k][i] * id));
            sum += q[i];
        }
        a.q[k] = pack4(q[0], q[1], q[2], q[3]);
    }
    d_bits = __builtin_bit_cast(uint16_t, static_cast<_Float16>(d));
    a.d = half_bits(d_bits);
    a.s0 = sum;
    a.s1 = 0;
    return a;
}

// Q8_K slice u % 8 of super-block u / 8, the super-block's 8 slices on 8
// consecutive lanes: max = the first element of largest magnitude,
// iscale = -127 / max, q = min(127, nearest-even(iscale x)), d = 1 / iscale
// (quantize_row_q8_K_ref).
__device__ __forceinline__ act_unit quantize_q8_k(const x_unit& xu, uint32_t u) {
    const f4 (&v)[8] = xu.v;
    float amax = 0.0f, mx = 0.0f;
    int at = 1 << 20;  // block index of the first element with the largest magnitude
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = fabsf(v[k][i]);
            if (a > amax) {
                amax = a;
                mx = v[k][i];
                at = static_cast<int>(32 * (u % 8)) + 4 * k + i;
            }
        }
    }
#pragma unroll
    for (int m = 1; m <= 4; m <<= 1) {
        const float oa = __shfl_xor(amax, m, wave);
        const float om = __shfl_xor(mx, m, wave);
        const int oi = __shfl_xor(at, m, wave);
        if (oa > amax || (oa == amax && oi < at)) {
            amax = oa;
            mx = om;
            at = oi;
        }
    }
    act_unit a;
    if (amax == 0.0f) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            a.q[k] = 0;
        }
        a.d = 0.0f;
        a.s0 = a.s1 = 0;
        return a;
    }
    const float iscale = -127.0f / mx;
    int s[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        int q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = min(127, static_cast<int>(rintf(iscale * v[k][i])));
            s[k / 4] += q[i];
        }
        a.q[k] = pack4(q[0], q[1], q[2], q[3]);
    }
    a.d = 1.0f / iscale;
    a.s0 = s[0];
    a.s1 = s[1];
    return a;
}

// ---- 2-byte aligned streams ------------------------------------------------------

template <int N>
__device__ __forceinline__ void fetch_window(rsrc r, uint32_t off, uint32_t (&w)[N]) {
    const uint32_t base = off & ~3u;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        w[k] = ld32(r, base + 4 * k);
    }
}

template <int N>
__device__ __forceinline__ void realign(const uint32_t (&w)[N + 1], uint32_t off, uint32_t (&d)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        d[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], off & 3u);
    }
}

// The quantized activation unit u of row r, in ggml's layout, into act (rows
// of units / 8 Q8_K blocks, or of units Q8_0 blocks).
template <bool KQ>
__device__ __forceinline__ void store_act_unit(uint8_t* act, uint32_t r, uint32_t units, uint32_t u,
                                               const act_unit& a, uint16_t d_bits) {
    if constexpr (KQ) {
        uint8_t* blk = act + static_cast<std::size_t>(r) * (units / 8) * 292 + std::size_t{u / 8} * 292;
        const uint32_t s = u % 8;
        uint32_t* qd = reinterpret_cast<uint32_t*>(blk + 4 + 32 * s);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            qd[k] = a.q[k];
        }
        *reinterpret_cast<uint32_t*>(blk + 260 + 4 * s) =
            (static_cast<uint32_t>(a.s0) & 0xFFFF) | (static_cast<uint32_t>(a.s1) << 16);
        if (s == 0) {
            *reinterpret_cast<float*>(blk) = a.d;
        }
    } else {
        uint16_t* blk = reinterpret_cast<uint16_t*>(act + (static_cast<std::size_t>(r) * units + u) * 34);
        blk[0] = d_bits;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            blk[1 + 2 * k] = static_cast<uint16_t>(a.q[k]);
            blk[2 + 2 * k] = static_cast<uint16_t>(a.q[k] >> 16);
        }
    }
}

}  // namespace

}  // namespace syn
