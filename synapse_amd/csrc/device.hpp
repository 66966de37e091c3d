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

// Byte address of an LDS location (what M0 and ds_* addresses take): the low
// 32 bits of its generic address (the shared aperture sits above 4 GiB and
// starts on a 4 GiB boundary). Unlike an address-space cast this has no null
// check, so a kernel keeps each LDS address in one scalar register instead
// of a 64-bit pointer plus a compare and select per use.
__device__ __forceinline__ uint32_t lds_address(const void* lds) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
}

// Raw buffer access: a 128-bit resource (base, byte limit) in scalar
// registers and a 32-bit per-lane byte offset. A load at or past the limit
// returns zeros, so a lane with nothing to read just gets an out-of-range
// offset (buffer_oob). 0x00020000 is the raw-buffer format word on CDNA.
typedef __amdgpu_buffer_rsrc_t rsrc;
constexpr uint32_t buffer_oob = 0x80000000u;
__device__ __forceinline__ rsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}
__device__ __forceinline__ u4 buffer_load16(rsrc r, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
}

// Direct global -> LDS copies: lane l's 16 bytes land at lds + 16 * l; lds
// must be the same for every lane of the wave. Counted by vmcnt like any
// vector load, and they take no registers.
//
// They are issued through asm on purpose. The compiler cannot tell which LDS
// bytes a copy writes, so after a copy it issued itself it waits for every
// outstanding vector load (s_waitcnt vmcnt(0)) before the next LDS read of
// any buffer: a pipeline's prefetch into one stage would then be waited for
// before the other stage is read, and a decode block would wait for all its
// K/V loads before reading q. Callers of these wait for their own copies
// (s_waitcnt vmcnt(n), then an LDS-only barrier when other waves read them).
// M0 holds the LDS address; one wait state separates its write from the copy.
__device__ __forceinline__ void load16_lds(const void* g, void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_address(lds));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(m0) : "memory");
}
// Lane l's 16 bytes at byte `offset` of r (zeros at or past its limit).
__device__ __forceinline__ void buffer_load16_lds(rsrc r, void* lds, uint32_t offset) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_address(lds));
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(offset), "s"(r), "{m0}"(m0) : "memory");
}

// Workgroup barrier that waits only for this wave's LDS operations.
// __syncthreads() carries a release fence that also waits for every
// outstanding vector load, prefetches meant to stay in flight across the
// barrier included. The memory clobber keeps LDS accesses on their side.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// f32 -> binary16, round to nearest even (v_cvt_f16_f32 in the default mode),
// the rounding kv_append and attend_group apply (S/numeric/half.hpp:46-82).
__device__ __forceinline__ _Float16 to_h(float x) {
    return static_cast<_Float16>(x);
}

// acc + x.x + x.y in f32 (v_dot2_f32_f16 against (1, 1)): sums binary16
// pairs with no conversions.
__device__ __forceinline__ float add_pair(h2 x, float acc) {
    typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(fp16x2, x), __builtin_bit_cast(fp16x2, h2{1, 1}), acc, false);
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

// Partner exchange across the wave's 16-lane rows on the VALU (gfx950's
// v_permlane16_swap / v_permlane32_swap), with no LDS traffic:
// partner16(v)[l] = v[l ^ 16], partner32(v)[l] = v[l ^ 32].
// swap16(a, b) returns {a.row0, b.row0, a.row2, b.row2} and
// {a.row1, b.row1, a.row3, b.row3}; swap32 does the same with 32-lane
// halves. Each partner is built from two swaps against zero: with the same
// value in both operands this compiler folds the second result into the
// first, so the operands are always different.
__device__ __forceinline__ float partner16(float v) {
    const unsigned x = __builtin_bit_cast(unsigned, v);
    const auto lo = __builtin_amdgcn_permlane16_swap(x, 0u, false, false);  // [1] = row above, in even rows
    const auto hi = __builtin_amdgcn_permlane16_swap(0u, x, false, false);  // [0] = row below, in odd rows
    return __builtin_bit_cast(float, (__lane_id() & 16) ? hi[0] : lo[1]);
}
__device__ __forceinline__ float partner32(float v) {
    const unsigned x = __builtin_bit_cast(unsigned, v);
    const auto lo = __builtin_amdgcn_permlane32_swap(x, 0u, false, false);  // [1] = upper half, in the lower
    const auto hi = __builtin_amdgcn_permlane32_swap(0u, x, false, false);  // [0] = lower half, in the upper
    return __builtin_bit_cast(float, (__lane_id() & 32) ? hi[0] : lo[1]);
}
__device__ __forceinline__ float max16(float v) {
    return fmaxf(v, partner16(v));
}
__device__ __forceinline__ float max32(float v) {
    return fmaxf(v, partner32(v));
}
__device__ __forceinline__ float sum16(float v) {
    return v + partner16(v);
}
__device__ __forceinline__ float sum32(float v) {
    return v + partner32(v);
}

// Reductions over the whole wave on the VALU, the result the same in every
// lane: within each quad by DPP (lane ^ 1, lane ^ 2), across the quads of a
// row by DPP mirrors (lane l with 7 - l, then with 15 - l), then across rows
// and halves by the permlane swaps above. Every step combines two lanes'
// values in both of them, and max and addition commute, so all lanes agree
// bit for bit. (A shuffle per step goes through the LDS crossbar and waits
// out its latency: six round trips for one reduction.)
template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int dpp_quad_xor1 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int dpp_quad_xor2 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int dpp_row_half_mirror = 0x141;
constexpr int dpp_row_mirror = 0x140;
__device__ __forceinline__ float wave_reduce_max(float v) {
    v = fmaxf(v, dpp_read<dpp_quad_xor1>(v));
    v = fmaxf(v, dpp_read<dpp_quad_xor2>(v));
    v = fmaxf(v, dpp_read<dpp_row_half_mirror>(v));
    v = fmaxf(v, dpp_read<dpp_row_mirror>(v));
    return max32(max16(v));
}
__device__ __forceinline__ float wave_reduce_sum(float v) {
    v += dpp_read<dpp_quad_xor1>(v);
    v += dpp_read<dpp_quad_xor2>(v);
    v += dpp_read<dpp_row_half_mirror>(v);
    v += dpp_read<dpp_row_mirror>(v);
    return sum32(sum16(v));
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
