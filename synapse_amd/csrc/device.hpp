// device.hpp — gfx950 building blocks shared by the attention kernels:
// binary16 vectors, the two f16 matrix-core shapes, wave64 reductions and the
// exp2 the online softmax uses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace syn {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr int wave = 64;
constexpr float log2e = 1.4426950408889634f;

// 16 bytes <-> 8 halves, bit for bit.
__device__ __forceinline__ h8 as_h8(u4 v) {
    return __builtin_bit_cast(h8, v);
}
__device__ __forceinline__ u4 as_u4(h8 v) {
    return __builtin_bit_cast(u4, v);
}

__device__ __forceinline__ u4 zero_u4() {
    return u4{0u, 0u, 0u, 0u};
}

// 16-byte global load; the pointer must be 16-B aligned.
__device__ __forceinline__ u4 load16(const void* p) {
    return *reinterpret_cast<const u4*>(p);
}
__device__ __forceinline__ void store16(void* p, u4 v) {
    *reinterpret_cast<u4*>(p) = v;
}

// f32 -> binary16, round to nearest even (v_cvt_f16_f32 in the default mode),
// the rounding kv_append and attend_group apply (S/numeric/half.hpp:46-82).
__device__ __forceinline__ _Float16 to_h(float x) {
    return static_cast<_Float16>(x);
}

// D(16x16) += A(16x32) B(32x16), f16 operands, f32 accumulate. Lane l holds
// A[l%16][k-group l/16], B[k-group l/16][l%16] (8 k values each) and
// D[4*(l/16) + i][l%16], i = 0..3.
__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D(32x32) += A(32x16) B(16x32). Lane l holds A[l%32][k-group l/32],
// B[k-group l/32][l%32] and D[8*(i/4) + 4*(l/32) + i%4][l%32], i = 0..15.
__device__ __forceinline__ f16v mfma32(h8 a, h8 b, f16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 2^x on the transcendental unit (v_exp_f32). exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float xor_max(float v, int mask) {
    return fmaxf(v, __shfl_xor(v, mask, wave));
}
__device__ __forceinline__ float xor_sum(float v, int mask) {
    return v + __shfl_xor(v, mask, wave);
}

__device__ __forceinline__ int lane_id() {
    return static_cast<int>(__lane_id());
}

}  // namespace syn
