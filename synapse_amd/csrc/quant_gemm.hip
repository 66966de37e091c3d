// quant_gemm.hip — products with quantized weights for many activation rows
// (a prompt), on the int8 matrix cores, with ggml's arithmetic.
//
// The reference's gemm_rows (S/kernels/gemm.hpp:142-236) computes, for each
// weight row and each activation row, the same block dots as its gemv: the
// activations quantized to the paired format (Q8_0 for Q4_0 / Q5_0 / Q8_0,
// Q8_K for Q4_K / Q6_K), exact integer sums per block, float combines. Here
// the integer sums come out of v_mfma_i32_32x32x32_i8 (Q6_K, whose scales
// change every 16 weights: v_mfma_i32_32x32x16_i8), 32 activation rows x 32
// weight rows per product, and the block scales combine them in float:
//
//   Q4_0, Q5_0, Q8_0   per 32-block:  float(sumi) * (d_w * d_a)
//   Q4_K               per 256-block: yd (d float(sum_s sc_s sumi_s) - dmin float(sum_k m_k bsum_k))
//   Q6_K               per 256-block: (d yd) (float(sum_k sc_k sumi_k) - 32 sum_k sc_k bsum_k)
//
// so each block's integers are ggml's and results differ from its gemv only
// by float association. Three kernels:
// - gemm_q4k_kernel (Q4_K): a workgroup (4 waves) owns 128 weight rows x 64
//   activation rows; a wave 32 weight rows (one per lane, the product's B
//   operand) against the 64 activation rows (two A operands). Each
//   256-block's weight and activation bytes reach LDS through whole-line
//   direct copies, two stages deep; the sub-block scales are folded into two
//   int8 weight planes and the mins take one f16 product per block.
// - gemm_q6k_kernel (Q6_K): 64 x 64 per workgroup, 32 x 32 per wave, the
//   same LDS staging; unsigned quants, the offset through the activation
//   sums on one f16 product per block.
// - gemm_qb32_kernel (Q4_0, Q5_0, Q8_0): the Q4_K tile, stages of two
//   32-blocks read at compile-time shifts.
// - gemm_q_kernel (the same three when cols is not a multiple of 64): the
//   same tile, every lane loading its own weight row's and activation rows'
//   bytes into registers, two batches of steps in flight.
// Details at each kernel.

#include "quant.hpp"

// The quantizers above keep ggml's rounding (no contraction); the GEMM's
// float combines below may fuse: they differ from ggml's gemv by float
// association in any case.
#pragma clang fp contract(fast)

namespace syn {

namespace {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));

constexpr uint32_t gq_m = 128;  // weight rows per workgroup
constexpr uint32_t gq_n = 64;   // activation rows per workgroup
constexpr uint32_t gq_k = 128;  // 32-wide steps per staged chunk of activation scales

// Signed bytes from 4- and 5-bit fields: x - 8, x - 16 per byte
// (flip the top bit, then extend it; no carries cross bytes).
__device__ __forceinline__ uint32_t sext4(uint32_t nib) {
    const uint32_t t = nib ^ 0x08080808u;
    return t | ((t & 0x08080808u) * 0x1Eu);
}
__device__ __forceinline__ uint32_t sext5(uint32_t x) {
    const uint32_t t = x ^ 0x10101010u;
    return t | ((t & 0x10101010u) * 0x0Eu);
}

// Activations to ggml's layout, one lane per 32 values (the 8 lanes of a
// Q8_K block on consecutive lanes: units is a multiple of 8 there).
template <bool KQ>
__global__ __launch_bounds__(256) void quantize_act_kernel(const float* x, uint8_t* act, uint32_t n, uint32_t cols) {
    const uint32_t units = cols / 32;
    const uint64_t id = blockIdx.x * 256ull + threadIdx.x;
    if (id >= uint64_t{n} * units) {
        return;  // whole 8-lane groups
    }
    const uint32_t r = static_cast<uint32_t>(id / units), u = static_cast<uint32_t>(id % units);
    const x_unit xv = load_x(x + static_cast<std::size_t>(r) * cols, u);
    uint16_t d_bits = 0;
    act_unit a;
    if constexpr (KQ) {
        a = quantize_q8_k(xv, u);
    } else {
        a = quantize_q8_0(xv, d_bits);
    }
    store_act_unit<KQ>(act, r, units, u, a, d_bits);
}

// One step's loads (32 weights of this lane's row, k-half H; the 16
// activation bytes of each of the lane's two activation rows), issued
// together ahead of the step's products. Windows are aligned dwords of a
// 2-byte aligned stream, realigned when the step is computed.
template <uint32_t T>
struct raw_step;
template <>
struct raw_step<qtype_q8_0> {
    uint32_t d, qw[5], aw[2][5];
};
template <>
struct raw_step<qtype_q4_0> {
    uint32_t d, qw[5], aw[2][5];
};
template <>
struct raw_step<qtype_q5_0> {
    uint32_t d, hw[2], qw[5], aw[2][5];
};

template <uint32_t T>
__device__ __forceinline__ raw_step<T> fetch_step(rsrc wr, rsrc ar, uint32_t wlane, uint32_t arow, uint32_t li,
                                                  uint32_t H, uint32_t k) {
    raw_step<T> x;
    {
        const uint32_t b0 = wlane + k * block_bytes<T>;
        x.d = ld16(wr, b0);
        if constexpr (T == qtype_q8_0) {
            fetch_window(wr, b0 + 2 + 16 * H, x.qw);
        } else if constexpr (T == qtype_q4_0) {
            fetch_window(wr, b0 + 2, x.qw);
        } else {
            fetch_window(wr, b0 + 2, x.hw);
            fetch_window(wr, b0 + 6, x.qw);
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            fetch_window(ar, (32 * g + li) * arow + k * 34 + 2 + 16 * H, x.aw[g]);
        }
    }
    return x;
}

// A batch of BS steps' loads.
template <uint32_t T, int BS>
struct raw_batch {
    raw_step<T> s[BS];
};

template <uint32_t T>
__global__ __launch_bounds__(256) void gemm_q_kernel(const uint8_t* w, const uint8_t* act, const float* bias,
                                                     float* out, uint32_t n, uint32_t rows, uint32_t cols) {
    // The activation scales d_a per (step, row).
    __shared__ __attribute__((aligned(16))) float lds_d[gq_k][gq_n];

    const uint32_t tid = threadIdx.x;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ln = tid & 63, H = ln >> 5, li = ln & 31;
    const uint32_t units = cols / 32;
    const uint32_t wrow = units * block_bytes<T>;
    const uint32_t arow = units * 34;
    const uint32_t o0 = blockIdx.x * gq_m + wv * 32;  // the wave's first weight row
    const uint32_t t0 = blockIdx.y * gq_n;            // the block's first activation row

    // The wave's 32 weight rows through one resource starting at the dword at
    // or before its first row; rows past `rows` read zeros.
    const uint32_t wave_rows = o0 < rows ? min(32u, rows - o0) : 0;
    const uint8_t* wp = w + static_cast<std::size_t>(min(o0, rows - 1)) * wrow;
    const uint32_t delta = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(wp) & 3);
    const rsrc wr = make_rsrc(wp - delta, wave_rows * wrow + delta);
    const uint32_t wlane = li * wrow + delta;  // this lane's row inside the resource
    // The block's 64 activation rows; rows past n read zeros.
    const rsrc ar = make_rsrc(act + static_cast<std::size_t>(t0) * arow, min(gq_n, n - t0) * arow);

    float acc[2][16];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[g][i] = 0.0f;
        }
    }
    const i16v zero16 = {};
    constexpr int BS = 4;  // steps per batch of loads
    using batch_t = raw_batch<T, BS>;

    for (uint32_t kc = 0; kc < units; kc += gq_k) {
        const uint32_t steps = min(gq_k, units - kc);
        // ---- stage the chunk's activation scales ----
        __syncthreads();  // the previous chunk's reads are done
        for (uint32_t e = tid; e < steps * gq_n; e += 256) {
            const uint32_t st = e / gq_n, r = e % gq_n;
            lds_d[st][r] = half_bits(ld16(ar, r * arow + (kc + st) * 34));
        }
        __syncthreads();

        // Steps go in batches of BS, two batches in flight: batch i + 1's
        // loads are issued before batch i's products, so a wave's memory
        // waits overlap its own work. Loads past the chunk's last step read a
        // valid step whose products are dropped.
        const auto fetch_batch = [&](batch_t& bt, uint32_t sb) __attribute__((always_inline)) {
#pragma unroll
            for (int b = 0; b < BS; ++b) {
                bt.s[b] = fetch_step<T>(wr, ar, wlane, arow, li, H, kc + min(sb + b, steps - 1));
            }
        };
        const auto compute_batch = [&](const batch_t& bt, uint32_t sb) __attribute__((always_inline)) {
            // Keep the batch's loads ahead of its products, and each step's
            // products next to their scaling (no instruction is emitted): else
            // the scheduler hoists every product of the batch and holds all
            // their results at once.
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = 0; b < BS; ++b) {
                const uint32_t st = min(sb + b, steps - 1);
                const uint32_t k = kc + st;  // 32-wide step
                {  // block k: 16 signed weights for this lane half
                    const uint32_t b0 = wlane + k * block_bytes<T>;
                    // A step past the chunk's last (the batch's tail) adds zeros.
                    const float dw = sb + b < steps ? half_bits(bt.s[b].d) : 0.0f;
                    uint32_t q[4];
                    if constexpr (T == qtype_q8_0) {
                        realign(bt.s[b].qw, b0 + 2 + 16 * H, q);
                    } else if constexpr (T == qtype_q4_0) {
                        uint32_t qs[4];
                        realign(bt.s[b].qw, b0 + 2, qs);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            q[j] = sext4((qs[j] >> (4 * H)) & 0x0F0F0F0Fu);
                        }
                    } else {  // Q5_0
                        uint32_t qhv[1], qs[4];
                        realign(bt.s[b].hw, b0 + 2, qhv);
                        realign(bt.s[b].qw, b0 + 6, qs);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            q[j] = sext5(((qs[j] >> (4 * H)) & 0x0F0F0F0Fu) |
                                         spread4((qhv[0] >> (16 * H + 4 * j)) & 0xF));
                        }
                    }
                    const i4v bw = {static_cast<int>(q[0]), static_cast<int>(q[1]), static_cast<int>(q[2]),
                                    static_cast<int>(q[3])};
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        uint32_t av[4];
                        realign(bt.s[b].aw[g], (32 * g + li) * arow + k * 34 + 2 + 16 * H, av);
                        const i4v a = {static_cast<int>(av[0]), static_cast<int>(av[1]), static_cast<int>(av[2]),
                                       static_cast<int>(av[3])};
                        const i16v cm = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bw, zero16, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const uint32_t r = 32 * g + 8 * (i / 4) + 4 * H + i % 4;
                            acc[g][i] += static_cast<float>(cm[i]) * (dw * lds_d[st][r]);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        batch_t ba, bb;
        fetch_batch(ba, 0);
        for (uint32_t sb = 0; sb < steps; sb += 2 * BS) {
            fetch_batch(bb, sb + BS);
            compute_batch(ba, sb);
            fetch_batch(ba, sb + 2 * BS);
            compute_batch(bb, sb + BS);
        }
    }

    // ---- out[row][o]: lane li's weight row, the 32 activation rows it holds ----
    const uint32_t o = o0 + li;
    if (o < rows) {
        const float bo = bias != nullptr ? bias[o] : 0.0f;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t r = t0 + 32 * g + 8 * (i / 4) + 4 * H + i % 4;
                if (r < n) {
                    out[static_cast<std::size_t>(r) * rows + o] = bias != nullptr ? acc[g][i] + bo : acc[g][i];
                }
            }
        }
    }
}

// ---- Q4_K through LDS ------------------------------------------------------------------
//
// The same tile (4 waves, 128 weight rows x 64 activation rows, a wave's 32
// weight rows against all 64), but every 256-block reaches the matrix cores
// through LDS: each wave copies its rows' 144-byte blocks and a quarter of
// the activation blocks with whole-line direct copies (buffer_load ... lds,
// 1 KiB per instruction), two stages deep, one barrier per block. The block
// dots are the reference's integers (S/kernels/dot.hpp:166-201): per
// 256-block
//   isum = sum_s sc_s sum_{j in s} q_j a_j,   mins = sum_k m_{k/2} bsum_k
// over the 16 activation sums of 16, and the float combine
// yd (d isum - dmin mins). The sub-block scale is
// folded into the weights so the products accumulate in place: sc = 8 sh + sl
// (sh, sl < 8), planes q sl and q sh (each below 128, so int8), and isum =
// sum(a . q sl) + 8 sum(a . q sh). The mins take one f16 product per block:
// the 16 activation sums of 16 (|b| <= 2032, exact in binary16) against m of
// their sub-block (each product and the sum of 16 exact in f32).

constexpr uint32_t k4_wave = 32 * 144;                                // one wave's weight rows, one block
constexpr uint32_t k4_stage = 4 * k4_wave + 64 * 256 + 4 * 512 + 4 * 256;  // weights, qs, bsums, d
constexpr uint32_t k4_a = 4 * k4_wave, k4_bs = k4_a + 64 * 256, k4_d = k4_bs + 4 * 512;

// Direct copies into LDS at M0 + 16 lane (M0 + 4 lane for the dword form).
__device__ __forceinline__ void copy16_lds(rsrc r, uint32_t m0, uint32_t voff) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(r), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void copy4_lds(rsrc r, uint32_t m0, uint32_t voff) {
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" : : "v"(voff), "s"(r), "{m0}"(m0) : "memory");
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Byte k of x in both 16-bit halves (the other bytes zero).
__device__ __forceinline__ uint32_t byte_pair(uint32_t x, uint32_t k) {
    return __builtin_amdgcn_perm(0u, x, 0x0C000C00u | (k << 16) | k);
}
__device__ __forceinline__ uint32_t mul_u16x2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}

__global__ __launch_bounds__(256, 2) void gemm_q4k_kernel(const uint8_t* w, const uint8_t* act, const float* bias,
                                                          float* out, uint32_t n, uint32_t rows, uint32_t cols) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][k4_stage];

    const uint32_t tid = threadIdx.x;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ln = tid & 63, H = ln >> 5, li = ln & 31;
    const uint32_t nb = cols / 256;
    const uint32_t wrow = nb * 144, arow = nb * 292;
    const uint32_t o0 = blockIdx.x * gq_m + wv * 32;
    const uint32_t t0 = blockIdx.y * gq_n;

    // The wave's weight rows and the block's activation rows; each copy
    // reads through a resource rebased to its 256-block, so rows past the
    // last read zeros.
    const uint32_t wave_rows = o0 < rows ? min(32u, rows - o0) : 0;
    const uint8_t* wp = w + static_cast<std::size_t>(min(o0, rows - 1)) * wrow;
    const uint32_t delta = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(wp) & 3);
    const uint8_t* wbase = wp - delta;
    // Whole dwords: a copy's range check is per dword, and the last row may
    // end inside one (which never crosses a page).
    const uint32_t wbytes = (wave_rows * wrow + delta + 3) & ~3u;
    const uint8_t* abase = act + static_cast<std::size_t>(t0) * arow;
    const uint32_t abytes = min(gq_n, n - t0) * arow;

    // Per-lane source offsets inside a block. Weights: byte b of the wave's
    // 32 x 144 image is row b / 144, byte b % 144. Activation qs: row
    // 16 wv + 4 i + ln / 16, its 16-byte chunk (ln % 16) ^ (row % 16), so a
    // row's chunks rotate across the LDS banks. bsums: row 16 wv + ln / 2,
    // half ln % 2 (lanes 0..31). d: row 16 wv + ln (lanes 0..15).
    uint32_t wo[5], ao[4];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const uint32_t b = 1024 * i + 16 * ln;
        wo[i] = delta + b / 144 * wrow + b % 144;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = 16 * wv + 4 * i + (ln >> 4);
        ao[i] = row * arow + 4 + 16 * ((ln & 15) ^ (row & 15));
    }
    const uint32_t bo = (16 * wv + (ln >> 1)) * arow + 260 + 16 * (ln & 1);
    const uint32_t dof = ln < 16 ? (16 * wv + ln) * arow : buffer_oob;

    const uint32_t L0 = lds_address(&lds[0][0]);
    const auto issue = [&](uint32_t U) __attribute__((always_inline)) {
        const uint32_t S = L0 + (U & 1) * k4_stage;
        const rsrc wr = make_rsrc(wbase + U * 144, wave_rows != 0 ? wbytes - U * 144 : 0);
        const rsrc ar = make_rsrc(abase + U * 292, abytes - U * 292);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            copy16_lds(wr, S + wv * k4_wave + 1024 * i, wo[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            copy16_lds(ar, S + k4_a + (16 * wv + 4 * i) * 256, ao[i]);
        }
        copy4_lds(ar, S + k4_d + 256 * wv, dof);
        if (ln < 32) {
            copy16_lds(wr, S + wv * k4_wave + 4096, wo[4]);
            copy16_lds(ar, S + k4_bs + 512 * wv, bo);
        }
    };

    float acc[2][16];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[g][i] = 0.0f;
        }
    }
    const i16v zi = {};
    const f16v zf = {};

    issue(0);
    for (uint32_t U = 0; U < nb; ++U) {
        // Block U landed in every wave; every wave is done with block U - 1,
        // whose stage block U + 1 now takes.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        if (U + 1 < nb) {
            issue(U + 1);
        }
        const uint8_t* S = lds[U & 1];
        const uint8_t* Wl = S + wv * k4_wave + li * 144;

        // d, dmin and the 8 (scale, min) pairs of this lane's weight row, as
        // bytes: sc 0..3, sc 4..7, m 0..3, m 4..7 (ggml's get_scale_min_k4).
        const u4 hdr = *reinterpret_cast<const u4*>(Wl);
        const float wd = half_bits(hdr[0] & 0xFFFF), wdmin = half_bits(hdr[0] >> 16);
        const uint32_t sc[2] = {hdr[1] & 0x3F3F3F3Fu, (hdr[3] & 0x0F0F0F0Fu) | ((hdr[1] >> 2) & 0x30303030u)};
        const uint32_t mn[2] = {hdr[2] & 0x3F3F3F3Fu, ((hdr[3] >> 4) & 0x0F0F0F0Fu) | ((hdr[2] >> 2) & 0x30303030u)};

        i16v a1[2], a2[2];
#pragma unroll
        for (int t = 0; t < 4; ++t) {  // sub-blocks 2t (low nibbles) and 2t + 1 (high)
            const u4 qw = *reinterpret_cast<const u4*>(Wl + 16 + 32 * t + 16 * H);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t s = 2 * t + e;
                const uint32_t sl = byte_pair(sc[s / 4] & 0x07070707u, s % 4);
                const uint32_t sh = byte_pair((sc[s / 4] >> 3) & 0x07070707u, s % 4);
                i4v p1, p2;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t nib = (qw[j] >> (4 * e)) & 0x0F0F0F0Fu;
                    p1[j] = static_cast<int>(mul_u16x2(nib, sl));
                    p2[j] = static_cast<int>(mul_u16x2(nib, sh));
                }
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    const uint32_t row = 32 * g + li;
                    const u4 av = *reinterpret_cast<const u4*>(S + k4_a + row * 256 + 16 * ((2 * s + H) ^ (li & 15)));
                    const i4v a = {static_cast<int>(av[0]), static_cast<int>(av[1]), static_cast<int>(av[2]),
                                   static_cast<int>(av[3])};
                    a1[g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, p1, s == 0 ? zi : a1[g], 0, 0, 0);
                    a2[g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, p2, s == 0 ? zi : a2[g], 0, 0, 0);
                }
            }
        }

        // mins: B = m of sub-blocks 4H .. 4H + 3, each for its two sums of 16.
        const uint32_t mh = mn[H];
        h8 mb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const _Float16 m = static_cast<_Float16>(static_cast<float>((mh >> (8 * j)) & 0xFF));
            mb[2 * j] = m;
            mb[2 * j + 1] = m;
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t row = 32 * g + li;
            const u4 bv = *reinterpret_cast<const u4*>(S + k4_bs + 512 * (row / 16) + 32 * (row % 16) + 16 * H);
            h8 ab;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ab[2 * j] = static_cast<_Float16>(static_cast<int16_t>(bv[j] & 0xFFFF));
                ab[2 * j + 1] = static_cast<_Float16>(static_cast<int16_t>(bv[j] >> 16));
            }
            const f16v fm = mfma32(ab, mb, zf);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t r0 = 32 * g + 8 * q + 4 * H;
                const f4 yd = *reinterpret_cast<const f4*>(S + k4_d + 256 * (r0 / 16) + 4 * (r0 % 16));
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int i = 4 * q + k;
                    const int isum = a1[g][i] + (a2[g][i] << 3);
                    acc[g][i] += yd[k] * (wd * static_cast<float>(isum) - wdmin * fm[i]);
                }
            }
        }
    }

    const uint32_t o = o0 + li;
    if (o < rows) {
        const float bo2 = bias != nullptr ? bias[o] : 0.0f;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t r = t0 + 32 * g + 8 * (i / 4) + 4 * H + i % 4;
                if (r < n) {
                    out[static_cast<std::size_t>(r) * rows + o] = acc[g][i] + bo2;
                }
            }
        }
    }
}

// ---- Q6_K through LDS ------------------------------------------------------------------
//
// A workgroup (4 waves) owns 64 weight rows x 64 activation rows; a wave 32
// x 32 (weight half wv % 2, activation half wv / 2), so a shape like
// ffn_down (4096 rows) still fills every SIMD twice. Each 256-block reaches
// LDS through direct copies: a weight row's 210-byte block as the 240-byte
// window from the dword at or before it (read back realigned by
// v_alignbyte), the activation blocks as in the Q4_K kernel. The block dot
// is the reference's (S/kernels/dot.hpp:203-236): per sub-block of 16,
// sc_k sum (q - 32) a. The quants are used unsigned (q, 0..63, on the int8
// matrix cores; each sub-block's sum scaled by sc_k in 24-bit integer
// multiply-adds) and the offset comes out through the activation sums of 16:
//   isum = sum_k sc_k sum_{j in k} q_j a_j - 32 sum_k sc_k bsum_k
// the second sum on one f16 product per block (|sc| <= 128, |bsum| <= 2032:
// exact in binary16, each product and the sum of 16 exact in f32).

// A row's window: 15 chunks, 210 bytes from any dword start plus one chunk
// of padding, so that rows 60 dwords apart hit distinct LDS banks.
constexpr uint32_t k6_win = 240;
constexpr uint32_t k6_a = 64 * k6_win, k6_bs = k6_a + 64 * 256, k6_d = k6_bs + 4 * 512;
constexpr uint32_t k6_stage = k6_d + 4 * 256;

// 8 bytes at byte o (0..3) of the 12 at p (p 4-aligned).
__device__ __forceinline__ uint64_t lds_bytes8(const uint8_t* p, uint32_t o) {
    const uint32_t* d = reinterpret_cast<const uint32_t*>(p);
    const uint32_t a = d[0], b = d[1], c = d[2];
    return (static_cast<uint64_t>(__builtin_amdgcn_alignbyte(c, b, o)) << 32) | __builtin_amdgcn_alignbyte(b, a, o);
}

__global__ __launch_bounds__(256, 2) void gemm_q6k_kernel(const uint8_t* w, const uint8_t* act, const float* bias,
                                                          float* out, uint32_t n, uint32_t rows, uint32_t cols) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][k6_stage];

    const uint32_t tid = threadIdx.x;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ln = tid & 63, H = ln >> 5, li = ln & 31;
    const uint32_t wh = wv & 1, ag = wv >> 1;
    const uint32_t nb = cols / 256;
    const uint32_t wrow = nb * 210, arow = nb * 292;
    const uint32_t r0 = blockIdx.x * 64;  // the block's first weight row (< rows)
    const uint32_t t0 = blockIdx.y * gq_n;

    const uint8_t* wp = w + static_cast<std::size_t>(r0) * wrow;
    const uint32_t delta = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(wp) & 3);
    const uint8_t* wbase = wp - delta;
    // Whole dwords: a copy's range check is per dword, and the last row's
    // block may end inside one (which never crosses a page).
    const uint32_t wbytes = (min(64u, rows - r0) * wrow + delta + 3) & ~3u;
    const uint8_t* abase = act + static_cast<std::size_t>(t0) * arow;
    const uint32_t abytes = min(gq_n, n - t0) * arow;

    // Block U of row r starts at byte X_r + 210 U of the weight resource, X_r
    // = delta + r wrow. Its window starts at the dword at or before that,
    // (X_r + 2 (U % 2)) rounded down plus 210 U - 2 (U % 2) (a multiple of
    // 4), so each copy reads through a resource rebased by the latter, from
    // one of two per-lane offsets by the parity of U. Wave wv copies rows
    // 16 wv .. 16 wv + 15: chunk ch = 64 i + ln of its 240, row 16 wv + ch /
    // 15, chunk ch % 15 (lanes 0..47 of the fourth copy).
    uint32_t wo[2][4], ao[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t ch = 64 * i + ln;
        const uint32_t x = delta + (16 * wv + ch / 15) * wrow;
        wo[0][i] = (x & ~3u) + 16 * (ch % 15);
        wo[1][i] = ((x + 2) & ~3u) + 16 * (ch % 15);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t row = 16 * wv + 4 * i + (ln >> 4);
        ao[i] = row * arow + 4 + 16 * ((ln & 15) ^ (row & 15));
    }
    const uint32_t bo = (16 * wv + (ln >> 1)) * arow + 260 + 16 * (ln & 1);
    const uint32_t dof = ln < 16 ? (16 * wv + ln) * arow : buffer_oob;

    const uint32_t L0 = lds_address(&lds[0][0]);
    const auto issue = [&](uint32_t U) __attribute__((always_inline)) {
        const uint32_t S = L0 + (U & 1) * k6_stage;
        const uint32_t shift = 210 * U - 2 * (U & 1);
        const rsrc wr = make_rsrc(wbase + shift, wbytes - shift);
        const rsrc ar = make_rsrc(abase + U * 292, abytes - U * 292);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            copy16_lds(wr, S + 16 * k6_win * wv + 1024 * i, (U & 1) ? wo[1][i] : wo[0][i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            copy16_lds(ar, S + k6_a + (16 * wv + 4 * i) * 256, ao[i]);
        }
        copy4_lds(ar, S + k6_d + 256 * wv, dof);
        if (ln < 48) {
            copy16_lds(wr, S + 16 * k6_win * wv + 3072, (U & 1) ? wo[1][3] : wo[0][3]);
        }
        if (ln < 32) {
            copy16_lds(ar, S + k6_bs + 512 * wv, bo);
        }
    };

    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        acc[i] = 0.0f;
    }
    const f16v zf = {};
    const uint32_t wrow_l = 32 * wh + li;  // this lane's weight row in the block
    const uint32_t arow_l = 32 * ag + li;  // this lane's activation row (A operand)
    const uint32_t xl = delta + wrow_l * wrow;

    issue(0);
    for (uint32_t U = 0; U < nb; ++U) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        if (U + 1 < nb) {
            issue(U + 1);
        }
        const uint8_t* S = lds[U & 1];
        const uint8_t* RB = S + wrow_l * k6_win;  // the window; the block starts at byte o
        const uint32_t o = (xl + 2 * (U & 1)) & 3;

        // 16 signed scales and d.
        const u4 s4 = *reinterpret_cast<const u4*>(RB + 192);
        const uint32_t s5 = *reinterpret_cast<const uint32_t*>(RB + 208);
        const uint32_t s6 = *reinterpret_cast<const uint32_t*>(RB + 212);
        const uint32_t sc[4] = {__builtin_amdgcn_alignbyte(s4[1], s4[0], o), __builtin_amdgcn_alignbyte(s4[2], s4[1], o),
                                __builtin_amdgcn_alignbyte(s4[3], s4[2], o), __builtin_amdgcn_alignbyte(s5, s4[3], o)};
        const float wd = half_bits(__builtin_amdgcn_alignbyte(s6, s5, o) & 0xFFFF);

        // Four groups (hf, kq) of four products (kh, e) each: a group's
        // products are issued before the previous group's results are scaled,
        // so the matrix cores run under the integer multiply-adds.
        int isum[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            isum[i] = 0;
        }
        i16v cm[2][4];
        int sck[2][4];
        const auto scale_group = [&](int t) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    // |sums| < 2^17 and |sc| <= 128: 24-bit multiplies are
                    // exact. The empty asm keeps one multiply-add per product
                    // (else the adds are regrouped into separate multiplies
                    // and three-input adds).
                    int v = __mul24(sck[t & 1][j], cm[t & 1][j][i]) + isum[i];
                    asm volatile("" : "+v"(v));
                    isum[i] = v;
                }
            }
        };
        uint64_t qh[2];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int hf = t / 2, kq = t % 2;
            if (kq == 0) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    qh[e] = lds_bytes8(RB + 128 + 32 * hf + 16 * e + 8 * H, o);
                }
            }
            uint64_t ql[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                ql[e] = lds_bytes8(RB + 64 * hf + 32 * kq + 16 * e + 8 * H, o);
            }
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const int k4 = 2 * kh + kq, s = 4 * hf + k4;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint64_t lo = (ql[e] >> (4 * kh)) & 0x0F0F0F0F0F0F0F0Full;
                    const uint64_t hi = k4 < 3 ? (qh[e] << (4 - 2 * k4)) & 0x3030303030303030ull
                                               : (qh[e] >> 2) & 0x3030303030303030ull;
                    const long bw = static_cast<long>(lo | hi);
                    const long a = *reinterpret_cast<const long*>(S + k6_a + arow_l * 256 +
                                                                  16 * ((2 * s + e) ^ (li & 15)) + 8 * H);
                    cm[t & 1][2 * kh + e] = __builtin_amdgcn_mfma_i32_32x32x16_i8(a, bw, i16v{}, 0, 0, 0);
                    const uint32_t k = 2 * s + e;  // sub-block of 16
                    sck[t & 1][2 * kh + e] = static_cast<int8_t>((sc[k / 4] >> (8 * (k % 4))) & 0xFF);
                }
            }
            if (t > 0) {
                scale_group(t - 1);
            }
        }
        scale_group(3);

        // The offset term: A = the activation sums of 16, B = sc, both for
        // k = 8H .. 8H + 7.
        const u4 bv = *reinterpret_cast<const u4*>(S + k6_bs + 512 * (arow_l / 16) + 32 * (arow_l % 16) + 16 * H);
        h8 ab, sb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ab[2 * j] = static_cast<_Float16>(static_cast<int16_t>(bv[j] & 0xFFFF));
            ab[2 * j + 1] = static_cast<_Float16>(static_cast<int16_t>(bv[j] >> 16));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sb[j] = static_cast<_Float16>(static_cast<int8_t>((sc[2 * H + j / 4] >> (8 * (j % 4))) & 0xFF));
        }
        const f16v cf = mfma32(ab, sb, zf);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t rq = 32 * ag + 8 * q + 4 * H;
            const f4 yd = *reinterpret_cast<const f4*>(S + k6_d + 256 * (rq / 16) + 4 * (rq % 16));
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = 4 * q + k;
                acc[i] += (wd * yd[k]) * (static_cast<float>(isum[i]) - 32.0f * cf[i]);
            }
        }
    }

    const uint32_t o = r0 + wrow_l;
    if (o < rows) {
        const float bo2 = bias != nullptr ? bias[o] : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = t0 + 32 * ag + 8 * (i / 4) + 4 * H + i % 4;
            if (r < n) {
                out[static_cast<std::size_t>(r) * rows + o] = acc[i] + bo2;
            }
        }
    }
}


// ---- Q4_0, Q5_0, Q8_0 through LDS ------------------------------------------------------
//
// The Q4_K tile (4 waves, 128 weight rows x 64 activation rows, a wave's 32
// against all 64) over stages of two 32-blocks (64 weights): 20-32 KB of
// LDS, so the whole grid of a 14336-row product is resident at once (stages
// of four Q8_0 blocks measured 4-5 % slower). The interface keeps w and act
// 4-byte aligned and this kernel runs when cols is a multiple of 64, so
// every row, and each row's two blocks of a stage (36, 44 or 68 bytes;
// activations always Q8_0's 68), start on a dword: a row is copied as the
// window of whole 16-byte chunks from there (48 or 80 bytes: rows 12 or 20
// dwords apart in LDS, distinct banks), and each block's bytes sit at a
// shift known at compile time, so the operands are read as two whole chunks
// (conflict-free) and realigned in registers by v_alignbyte (Q8_0 read in
// dwords at a run-time shift measured 205 against 152 us: all lanes at the
// same byte of their chunk hit a quarter of the banks). The stage's
// activation scales (64 rows x 2 blocks, one per thread) are loaded into
// registers with the copies and written to LDS as f32 before the stage's
// barrier. Per block, the reference's block kernels (S/kernels/dot.hpp:
// 102-163): sum (q - z) a with z = 8, 16, 0, as float(sumi) (d_w d_a); the
// weights are decoded to their signed values.

template <uint32_t T>
constexpr uint32_t k32_wwin = T == qtype_q8_0 ? 80 : 48;  // a weight row's window over 2 blocks
constexpr uint32_t k32_awin = 80;                          // an activation row's (Q8_0 blocks)
template <uint32_t T>
constexpr uint32_t k32_a = 128 * k32_wwin<T>;
template <uint32_t T>
constexpr uint32_t k32_da = k32_a<T> + 64 * k32_awin;
template <uint32_t T>
constexpr uint32_t k32_stage = k32_da<T> + 2 * 64 * 4;  // d_a [block][row] as f32

// N dwords from byte M of the two 16-byte chunks at p (p 16-aligned).
template <uint32_t M, int N>
__device__ __forceinline__ void lds_chunk_words(const uint8_t* p, uint32_t (&d)[N]) {
    const u4 c0 = *reinterpret_cast<const u4*>(p), c1 = *reinterpret_cast<const u4*>(p + 16);
    const uint32_t w8[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    constexpr uint32_t k = M / 4, sh = M % 4;
    static_assert(k + N < 8 || (k + N == 8 && sh == 0), "past the two chunks");
#pragma unroll
    for (int j = 0; j < N; ++j) {
        d[j] = __builtin_amdgcn_alignbyte(w8[(k + j + 1) & 7], w8[k + j], sh);
    }
}

template <uint32_t T>
__global__ __launch_bounds__(256, 4) void gemm_qb32_kernel(const uint8_t* w, const uint8_t* act, const float* bias,
                                                           float* out, uint32_t n, uint32_t rows, uint32_t cols) {
    constexpr uint32_t BB = block_bytes<T>, WWIN = k32_wwin<T>, WCH = WWIN / 16;
    constexpr uint32_t KA = k32_a<T>, KD = k32_da<T>, KS = k32_stage<T>;
    constexpr int NW = (32 * WCH + 63) / 64, NA = (16 * 5 + 63) / 64;  // copies per wave
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][KS];

    const uint32_t tid = threadIdx.x;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ln = tid & 63, H = ln >> 5, li = ln & 31;
    const uint32_t nst = cols / 64;
    const uint32_t wrow = cols / 32 * BB, arow = cols / 32 * 34;  // multiples of 4
    const uint32_t o0 = blockIdx.x * gq_m + wv * 32;
    const uint32_t t0 = blockIdx.y * gq_n;

    // The wave's weight rows and the block's activation rows, each through a
    // resource rebased per stage (rows past the last read zeros).
    const uint32_t wave_rows = o0 < rows ? min(32u, rows - o0) : 0;
    const uint8_t* wbase = w + static_cast<std::size_t>(min(o0, rows - 1)) * wrow;
    const uint32_t wbytes = wave_rows * wrow;
    const uint8_t* abase = act + static_cast<std::size_t>(t0) * arow;
    const uint32_t abytes = min(gq_n, n - t0) * arow;

    // Copies: wave wv's 32 weight rows, chunk ch = 64 i + ln of their 32 WCH
    // (row ch / WCH, chunk ch % WCH), and activation rows 16 wv .. 16 wv +
    // 15, chunk ch of their 80 (row ch / 5); the last copy of each with the
    // lanes that remain. The d_a of row tid % 64, block tid / 64 (threads
    // 0..127).
    uint32_t wo[NW], ao[NA];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const uint32_t ch = 64 * i + ln;
        wo[i] = ch / WCH * wrow + 16 * (ch % WCH);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const uint32_t ch = 64 * i + ln;
        ao[i] = (16 * wv + ch / 5) * arow + 16 * (ch % 5);
    }
    const uint32_t dao = (tid & 63) * arow + (tid >> 6) * 34;

    const uint32_t L0 = lds_address(&lds[0][0]);
    uint32_t dah = 0;
    const auto issue = [&](uint32_t U) __attribute__((always_inline)) {
        const uint32_t S = L0 + (U & 1) * KS;
        const rsrc wr = make_rsrc(wbase + U * 2 * BB, wave_rows != 0 ? wbytes - U * 2 * BB : 0);
        const rsrc ar = make_rsrc(abase + U * 68, abytes - U * 68);
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            if (64 * i + 64 <= 32 * WCH || ln < 32 * WCH - 64 * i) {
                copy16_lds(wr, S + 32 * WWIN * wv + 1024 * i, wo[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            if (64 * i + 64 <= 80 || ln < 80 - 64 * i) {
                copy16_lds(ar, S + KA + 16 * k32_awin * wv + 1024 * i, ao[i]);
            }
        }
        if (tid < 128) {
            dah = ld16(ar, dao);
        }
    };

    float acc[2][16];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[g][i] = 0.0f;
        }
    }

    issue(0);
    for (uint32_t U = 0; U < nst; ++U) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (tid < 128) {
            reinterpret_cast<float*>(lds[U & 1] + KD)[tid] = half_bits(dah);
        }
        lds_barrier();
        if (U + 1 < nst) {
            issue(U + 1);
        }
        const uint8_t* S = lds[U & 1];
        const uint8_t* WR = S + (32 * wv + li) * WWIN;
        const float* da = reinterpret_cast<const float*>(S + KD);
        const auto block = [&]<int b>() __attribute__((always_inline)) {
            // d_w at byte BB b of the row, then the block's quants.
            const float dw = half_bits(*reinterpret_cast<const uint16_t*>(WR + BB * b));
            uint32_t q[4];
            if constexpr (T == qtype_q8_0) {  // this lane half's 16 bytes at 34 b + 2 + 16 H
                constexpr uint32_t C = (34 * b + 2) / 16 * 16, M = (34 * b + 2) % 16;
                lds_chunk_words<M>(WR + C + 16 * H, q);
            } else if constexpr (T == qtype_q4_0) {  // 16 bytes at 18 b + 2, this lane half's nibbles
                constexpr uint32_t C = (18 * b + 2) / 16 * 16, M = (18 * b + 2) % 16;
                uint32_t qs[4];
                lds_chunk_words<M>(WR + C, qs);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    q[j] = sext4((qs[j] >> (4 * H)) & 0x0F0F0F0Fu);
                }
            } else {  // Q5_0: the 32 high bits at 22 b + 2, then 16 bytes
                constexpr uint32_t C = (22 * b + 2) / 16 * 16, M = (22 * b + 2) % 16;
                uint32_t hq[5];
                lds_chunk_words<M>(WR + C, hq);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    q[j] = sext5(((hq[1 + j] >> (4 * H)) & 0x0F0F0F0Fu) | spread4((hq[0] >> (16 * H + 4 * j)) & 0xF));
                }
            }
            const i4v qv = {static_cast<int>(q[0]), static_cast<int>(q[1]), static_cast<int>(q[2]),
                            static_cast<int>(q[3])};
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                constexpr uint32_t CA = (34 * b + 2) / 16 * 16, MA = (34 * b + 2) % 16;
                uint32_t av[4];
                lds_chunk_words<MA>(S + KA + (32 * g + li) * k32_awin + CA + 16 * H, av);
                const i4v a = {static_cast<int>(av[0]), static_cast<int>(av[1]), static_cast<int>(av[2]),
                               static_cast<int>(av[3])};
                const i16v cm = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qv, i16v{}, 0, 0, 0);
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const f4 d4 = *reinterpret_cast<const f4*>(da + 64 * b + 32 * g + 8 * qd + 4 * H);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        acc[g][4 * qd + k] += static_cast<float>(cm[4 * qd + k]) * (dw * d4[k]);
                    }
                }
            }
        };
        block.template operator()<0>();
        block.template operator()<1>();
    }

    const uint32_t o = o0 + li;
    if (o < rows) {
        const float bo = bias != nullptr ? bias[o] : 0.0f;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t r = t0 + 32 * g + 8 * (i / 4) + 4 * H + i % 4;
                if (r < n) {
                    out[static_cast<std::size_t>(r) * rows + o] = acc[g][i] + bo;
                }
            }
        }
    }
}
}  // namespace

hipError_t launch_gemm_q(uint32_t t, const uint8_t* w, const float* x, uint8_t* act, const float* bias, float* out,
                         uint32_t n, uint32_t rows, uint32_t cols, hipStream_t stream) {
    const bool kq = t == qtype_q4_k || t == qtype_q6_k;
    const uint64_t total = uint64_t{n} * (cols / 32);
    const uint32_t qblocks = static_cast<uint32_t>((total + 255) / 256);
    if (kq) {
        quantize_act_kernel<true><<<qblocks, 256, 0, stream>>>(x, act, n, cols);
    } else {
        quantize_act_kernel<false><<<qblocks, 256, 0, stream>>>(x, act, n, cols);
    }
    const dim3 grid((rows + gq_m - 1) / gq_m, (n + gq_n - 1) / gq_n);
    // The 32-block formats through LDS when every row's stage starts on a
    // dword (whole stages of two blocks; w and act 4-byte aligned, as the
    // interface keeps them); else the register kernel.
    const bool staged = cols % 64 == 0 && (reinterpret_cast<uintptr_t>(w) & 3) == 0 &&
                        (reinterpret_cast<uintptr_t>(act) & 3) == 0;
    switch (t) {
    case qtype_q4_0:
        if (staged) {
            gemm_qb32_kernel<qtype_q4_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        } else {
            gemm_q_kernel<qtype_q4_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        }
        break;
    case qtype_q5_0:
        if (staged) {
            gemm_qb32_kernel<qtype_q5_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        } else {
            gemm_q_kernel<qtype_q5_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        }
        break;
    case qtype_q8_0:
        if (staged) {
            gemm_qb32_kernel<qtype_q8_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        } else {
            gemm_q_kernel<qtype_q8_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        }
        break;
    case qtype_q4_k:
        gemm_q4k_kernel<<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    default:
        gemm_q6k_kernel<<<dim3((rows + 63) / 64, grid.y), 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    }
    return hipGetLastError();
}

}  // namespace syn
