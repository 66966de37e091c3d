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
//   Q4_K               per 256-block: (d yd) float(sum_s sc_s sumi_s) - (dmin yd) float(sum_s m_s bsum_s)
//   Q6_K               per 256-block: (d yd) float(sum_h sc_h sumi_h)
//
// so each block's integers are ggml's and results differ from its gemv only
// by float association. The weights are decoded to int8 in registers (Q4_0
// and Q5_0 to their signed values, Q6_K to q - 32, Q4_K to its unsigned
// nibbles with the mins through the activation sums).
//
// A workgroup (4 waves) owns 128 weight rows x 64 activation rows; a wave 32
// weight rows (one per lane, the product's B operand) against the 64
// activation rows (two A operands), so each decoded weight feeds two
// products. The activation scales of the block's 64 rows (and, for Q4_K,
// their sums of 32) are staged in LDS for 128 steps of 32 at a time.

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

// Signed bytes from 4-, 5- and 6-bit fields: x - 8, x - 16, x - 32 per byte
// (flip the top bit, then extend it; no carries cross bytes).
__device__ __forceinline__ uint32_t sext4(uint32_t nib) {
    const uint32_t t = nib ^ 0x08080808u;
    return t | ((t & 0x08080808u) * 0x1Eu);
}
__device__ __forceinline__ uint32_t sext5(uint32_t x) {
    const uint32_t t = x ^ 0x10101010u;
    return t | ((t & 0x10101010u) * 0x0Eu);
}
__device__ __forceinline__ uint32_t sext6(uint32_t x) {
    const uint32_t t = x ^ 0x20202020u;
    return t | ((t & 0x20202020u) * 0x06u);
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
struct raw_step<qtype_q4_k> {
    u4 q, a[2];
};
template <>
struct raw_step<qtype_q6_k> {
    uint32_t lw[2][3], hw[2][3], a[2][2][2];  // [half e], [half e][row group][dword]
};
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
    if constexpr (T == qtype_q4_k) {
        const uint32_t U = k / 8, s = k % 8;
        x.q = buffer_load16(wr, wlane + U * 144 + 16 + 32 * (s / 2) + 16 * H);
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            x.a[g] = buffer_load16(ar, (32 * g + li) * arow + U * 292 + 4 + 32 * s + 16 * H);
        }
    } else if constexpr (T == qtype_q6_k) {
        const uint32_t U = k / 8, s = k % 8, hf = s / 4, k4 = s % 4;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            fetch_window(wr, wlane + U * 210 + 64 * hf + 32 * (k4 & 1) + 16 * e + 8 * H, x.lw[e]);
            fetch_window(wr, wlane + U * 210 + 128 + 32 * hf + 16 * e + 8 * H, x.hw[e]);
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const uint32_t aoff = (32 * g + li) * arow + U * 292 + 4 + 32 * s + 16 * e + 8 * H;
                x.a[e][g][0] = ld32(ar, aoff);
                x.a[e][g][1] = ld32(ar, aoff + 4);
            }
        }
    } else {
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

// A batch of BS steps' loads and, for the K-quants, its 256-block header
// (Q4_K: d, dmin, 12 scale bytes; Q6_K: the window of its 16 scales, and d).
template <uint32_t T, int BS>
struct raw_batch {
    raw_step<T> s[BS];
    u4 hdr;
    uint32_t sw[5], d6;
};

template <uint32_t T>
__global__ __launch_bounds__(256) void gemm_q_kernel(const uint8_t* w, const uint8_t* act, const float* bias,
                                                     float* out, uint32_t n, uint32_t rows, uint32_t cols) {
    constexpr bool KQ = k_quant<T>;
    // Q8_0 pairs: d_a per (step, row); K-quants: yd per (256-block, row), and
    // for Q4_K the activation sum of each 32-step per (step, row).
    __shared__ __attribute__((aligned(16))) float lds_d[KQ ? gq_k / 8 : gq_k][gq_n];
    __shared__ __attribute__((aligned(16))) int lds_s[T == qtype_q4_k ? gq_k : 1][gq_n];

    const uint32_t tid = threadIdx.x;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t ln = tid & 63, H = ln >> 5, li = ln & 31;
    const uint32_t units = cols / 32;
    const uint32_t wrow = cols / (KQ ? 256 : 32) * block_bytes<T>;
    const uint32_t arow = KQ ? units / 8 * 292 : units * 34;
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
    int isum[2][16];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[g][i] = 0.0f;
            isum[g][i] = 0;
        }
    }
    const i16v zero16 = {};
    // Steps per batch of loads (a Q4_K / Q6_K 256-block is 8 steps).
    constexpr int BS = KQ ? 2 : 4;
    using batch_t = raw_batch<T, BS>;
    // Per 256-block weight data of this lane's row (K-quants).
    u4 hdr = {};          // Q4_K: d, dmin, 12 scale bytes; Q6_K: 16 scales
    float wd = 0.0f, wdmin = 0.0f;

    for (uint32_t kc = 0; kc < units; kc += gq_k) {
        const uint32_t steps = min(gq_k, units - kc);
        // ---- stage the chunk's activation scales (and Q4_K sums) ----
        __syncthreads();  // the previous chunk's reads are done
        if constexpr (KQ) {
            for (uint32_t e = tid; e < steps / 8 * gq_n; e += 256) {
                const uint32_t b = e / gq_n, r = e % gq_n;
                lds_d[b][r] = __builtin_bit_cast(float, ld32(ar, r * arow + (kc / 8 + b) * 292));
            }
            if constexpr (T == qtype_q4_k) {
                for (uint32_t e = tid; e < steps * gq_n; e += 256) {
                    const uint32_t st = e / gq_n, r = e % gq_n;
                    const uint32_t k = kc + st;
                    const uint32_t bs = ld32(ar, r * arow + k / 8 * 292 + 260 + 4 * (k % 8));
                    lds_s[st][r] = static_cast<int16_t>(bs & 0xFFFF) + static_cast<int16_t>(bs >> 16);
                }
            }
        } else {
            for (uint32_t e = tid; e < steps * gq_n; e += 256) {
                const uint32_t st = e / gq_n, r = e % gq_n;
                lds_d[st][r] = half_bits(ld16(ar, r * arow + (kc + st) * 34));
            }
        }
        __syncthreads();

        // Steps go in batches of BS, two batches in flight: batch i + 1's
        // loads are issued before batch i's products, so a wave's memory
        // waits overlap its own work. Loads past the chunk's last step read a
        // valid step whose products are dropped (Q4_0 / Q5_0 / Q8_0; the
        // K-quant chunks are whole 256-blocks).
        const auto fetch_batch = [&](batch_t& bt, uint32_t sb) __attribute__((always_inline)) {
#pragma unroll
            for (int b = 0; b < BS; ++b) {
                bt.s[b] = fetch_step<T>(wr, ar, wlane, arow, li, H, kc + min(sb + b, steps - 1));
            }
            if constexpr (KQ) {
                // The 256-block's header (a block spans several batches and each loads it).
                const uint32_t U = (kc + min(sb, steps - 1)) / 8;
                if constexpr (T == qtype_q4_k) {
                    bt.hdr = buffer_load16(wr, wlane + U * 144);
                } else {
                    fetch_window(wr, wlane + U * 210 + 192, bt.sw);
                    bt.d6 = ld16(wr, wlane + U * 210 + 208);
                }
            }
        };
        const auto compute_batch = [&](const batch_t& bt, uint32_t sb) __attribute__((always_inline)) {
            // Keep the batch's loads ahead of its products, and each step's
            // products next to their scaling (no instruction is emitted): else
            // the scheduler hoists every product of the batch and holds all
            // their results at once.
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (T == qtype_q4_k) {
                hdr = bt.hdr;
                wd = half_bits(hdr[0]);
                wdmin = half_bits(hdr[0] >> 16);
            } else if constexpr (T == qtype_q6_k) {
                uint32_t scw[4];
                realign(bt.sw, wlane + (kc + sb) / 8 * 210 + 192, scw);
                hdr = u4{scw[0], scw[1], scw[2], scw[3]};
                wd = half_bits(bt.d6);
            }
#pragma unroll
            for (int b = 0; b < BS; ++b) {
                const uint32_t st = min(sb + b, steps - 1);
                const uint32_t k = kc + st;  // 32-wide step
                if constexpr (T == qtype_q4_k) {
                    const uint32_t s = k % 8, sh = (s & 1) * 4;
                    const u4 q = bt.s[b].q;
                    const i4v bw = {static_cast<int>((q[0] >> sh) & 0x0F0F0F0Fu),
                                    static_cast<int>((q[1] >> sh) & 0x0F0F0F0Fu),
                                    static_cast<int>((q[2] >> sh) & 0x0F0F0F0Fu),
                                    static_cast<int>((q[3] >> sh) & 0x0F0F0F0Fu)};
                    const auto byte = [&](uint32_t j) { return (hdr[1 + j / 4] >> (8 * (j % 4))) & 0xFFu; };
                    const int sc = s < 4 ? static_cast<int>(byte(s) & 63)
                                         : static_cast<int>((byte(s + 4) & 0xF) | ((byte(s - 4) >> 6) << 4));
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        const u4 av = bt.s[b].a[g];
                        const i4v a = {static_cast<int>(av[0]), static_cast<int>(av[1]), static_cast<int>(av[2]),
                                       static_cast<int>(av[3])};
                        const i16v cm = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bw, zero16, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            // |sums| < 2^23: 24-bit multiplies are exact.
                            isum[g][i] += __mul24(sc, cm[i]);
                        }
                    }
                } else if constexpr (T == qtype_q6_k) {  // two 16-wide halves with their own scales
                    const uint32_t s = k % 8, hf = s / 4, k4 = s % 4;
                    const uint32_t U = k / 8;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        uint32_t lo[2], hi[2];
                        realign(bt.s[b].lw[e], wlane + U * 210 + 64 * hf + 32 * (k4 & 1) + 16 * e + 8 * H, lo);
                        realign(bt.s[b].hw[e], wlane + U * 210 + 128 + 32 * hf + 16 * e + 8 * H, hi);
                        uint32_t q[2];
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            q[j] = sext6(((lo[j] >> (4 * (k4 >> 1))) & 0x0F0F0F0Fu) |
                                         (((hi[j] >> (2 * k4)) & 0x03030303u) << 4));
                        }
                        const long bw = static_cast<long>((static_cast<uint64_t>(q[1]) << 32) | q[0]);
                        const uint32_t si = 8 * hf + 2 * k4 + e;  // this half's scale
                        const int sc = static_cast<int8_t>((hdr[si / 4] >> (8 * (si % 4))) & 0xFF);
#pragma unroll
                        for (int g = 0; g < 2; ++g) {
                            const long a = static_cast<long>((static_cast<uint64_t>(bt.s[b].a[e][g][1]) << 32) |
                                                             bt.s[b].a[e][g][0]);
                            const i16v cm = __builtin_amdgcn_mfma_i32_32x32x16_i8(a, bw, zero16, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 16; ++i) {
                                isum[g][i] += __mul24(sc, cm[i]);
                            }
                        }
                    }
                } else {
                    // Q4_0 / Q5_0 / Q8_0 block k: 16 signed weights for this lane half.
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
                if constexpr (KQ) {
                    // Batches of BS steps tile each 8-step 256-block: the batch
                    // that ends one has sb % 8 == 8 - BS.
                    if (b == BS - 1 && sb % 8 == 8 - BS) {
                        // Q4_K mins: sum_s m_s bsum_s per (activation row, weight
                        // row) on the f32 matrix cores, K = the 8 sub-blocks;
                        // every product and sum is an integer below 2^24, so
                        // exact. A: the activation sums of 32 (lane: row l % 32,
                        // sub-block 2j + H); B: this lane's weight row's mins.
                        f16v fmin[2];
                        if constexpr (T == qtype_q4_k) {
                            const auto byte = [&](uint32_t j) { return (hdr[1 + j / 4] >> (8 * (j % 4))) & 0xFFu; };
#pragma unroll
                            for (int g = 0; g < 2; ++g) {
#pragma unroll
                                for (int i = 0; i < 16; ++i) {
                                    fmin[g][i] = 0.0f;
                                }
                            }
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const uint32_t sub = 2 * j + H;
                                const int m = sub < 4 ? static_cast<int>(byte(sub + 4) & 63)
                                                      : static_cast<int>((byte(sub + 4) >> 4) | ((byte(sub) >> 6) << 4));
#pragma unroll
                                for (int g = 0; g < 2; ++g) {
                                    const float am = static_cast<float>(lds_s[st - 7 + sub][32 * g + li]);
                                    fmin[g] = __builtin_amdgcn_mfma_f32_32x32x2f32(am, static_cast<float>(m), fmin[g],
                                                                                   0, 0, 0);
                                }
                            }
                        }
                        // The 256-block's float combine.
#pragma unroll
                        for (int g = 0; g < 2; ++g) {
#pragma unroll
                            for (int i = 0; i < 16; ++i) {
                                const uint32_t r = 32 * g + 8 * (i / 4) + 4 * H + i % 4;
                                const float yd = lds_d[st / 8][r];
                                if constexpr (T == qtype_q4_k) {
                                    acc[g][i] += (wd * yd) * static_cast<float>(isum[g][i]) -
                                                 (wdmin * yd) * fmin[g][i];
                                } else {
                                    acc[g][i] += (wd * yd) * static_cast<float>(isum[g][i]);
                                }
                                isum[g][i] = 0;
                            }
                        }
                    }
                }
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
    switch (t) {
    case qtype_q4_0:
        gemm_q_kernel<qtype_q4_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    case qtype_q5_0:
        gemm_q_kernel<qtype_q5_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    case qtype_q8_0:
        gemm_q_kernel<qtype_q8_0><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    case qtype_q4_k:
        gemm_q_kernel<qtype_q4_k><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    default:
        gemm_q_kernel<qtype_q6_k><<<grid, 256, 0, stream>>>(w, act, bias, out, n, rows, cols);
        break;
    }
    return hipGetLastError();
}

}  // namespace syn
