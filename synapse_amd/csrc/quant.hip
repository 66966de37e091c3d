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

#include "quant.hpp"

#include <atomic>
#include <mutex>

namespace syn {

namespace {

// ---- weights: a lane's 32 weights, fetched, then decoded for v_dot4 -------------
//
// fetch<T> issues the unit's loads and nothing else, so a wave can hold the
// next batch's loads in flight while it decodes and dots the current one.
// The 2-byte aligned formats fetch aligned dword windows (one dword more than
// the stream) that decode realigns with v_alignbyte.

template <uint32_t T>
struct raw_unit;
template <>
struct raw_unit<qtype_q4_k> {
    u4 h, q0, q1;  // d, dmin, 12 scale bytes; the slice's 32 quant bytes
};
template <>
struct raw_unit<qtype_q6_k> {
    uint32_t lo[9], hi[9], scp, d;
};
template <>
struct raw_unit<qtype_q8_0> {
    uint32_t q[9], d;
};
template <>
struct raw_unit<qtype_q4_0> {
    uint32_t q[5], d;
};
template <>
struct raw_unit<qtype_q5_0> {
    uint32_t qh[2], q[5], d;
};

// Unit u of a row whose resource starts delta (0 or 2) bytes before it.
template <uint32_t T>
__device__ __forceinline__ raw_unit<T> fetch(rsrc wr, uint32_t delta, uint32_t u) {
    raw_unit<T> x;
    if constexpr (T == qtype_q4_k) {
        const uint32_t b = u / 8 * 144 + delta, s = u % 8;
        x.h = buffer_load16(wr, b);
        x.q0 = buffer_load16(wr, b + 16 + 32 * (s / 2));
        x.q1 = buffer_load16(wr, b + 32 + 32 * (s / 2));
    } else if constexpr (T == qtype_q6_k) {  // slice s is quarter s % 4 of half s / 4
        const uint32_t b = u / 8 * 210 + delta, s = u % 8, hf = s / 4, k4 = s % 4;
        fetch_window(wr, b + 64 * hf + 32 * (k4 & 1), x.lo);
        fetch_window(wr, b + 128 + 32 * hf, x.hi);
        x.scp = ld16(wr, b + 192 + 8 * hf + 2 * k4);
        x.d = ld16(wr, b + 208);
    } else {
        const uint32_t b = u * block_bytes<T> + delta;
        x.d = ld16(wr, b);
        if constexpr (T == qtype_q5_0) {
            fetch_window(wr, b + 2, x.qh);
            fetch_window(wr, b + 6, x.q);
        } else {
            fetch_window(wr, b + 2, x.q);
        }
    }
    return x;
}

// q: 8 dwords of int8 (non-negative, except Q8_0's signed values); the dot
// is then combined with the scales below.
struct weight_unit {
    uint32_t q[8];
    float d, dmin;
    int sc0, sc1;  // Q4_K: scale and min; Q6_K: the two 16-weight scales
};

template <uint32_t T>
__device__ __forceinline__ weight_unit decode(const raw_unit<T>& r, uint32_t delta, uint32_t u) {
    constexpr uint32_t nib = 0x0F0F0F0Fu;
    weight_unit x;
    x.dmin = 0.0f;
    x.sc0 = x.sc1 = 0;
    if constexpr (T == qtype_q4_k) {
        const uint32_t s = u % 8, shift = (s & 1) * 4;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x.q[k] = (r.q0[k] >> shift) & nib;
            x.q[4 + k] = (r.q1[k] >> shift) & nib;
        }
        const auto byte = [&](uint32_t j) { return (r.h[1 + j / 4] >> (8 * (j % 4))) & 0xFFu; };
        if (s < 4) {
            x.sc0 = static_cast<int>(byte(s) & 63);
            x.sc1 = static_cast<int>(byte(s + 4) & 63);
        } else {
            x.sc0 = static_cast<int>((byte(s + 4) & 0xF) | ((byte(s - 4) >> 6) << 4));
            x.sc1 = static_cast<int>((byte(s + 4) >> 4) | ((byte(s) >> 6) << 4));
        }
        x.d = half_bits(r.h[0]);
        x.dmin = half_bits(r.h[0] >> 16);
    } else if constexpr (T == qtype_q6_k) {
        const uint32_t b = u / 8 * 210 + delta, s = u % 8, hf = s / 4, k4 = s % 4;
        uint32_t lo[8], hi[8];
        realign(r.lo, b + 64 * hf + 32 * (k4 & 1), lo);
        realign(r.hi, b + 128 + 32 * hf, hi);
        const uint32_t lshift = (k4 >> 1) * 4;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            x.q[k] = ((lo[k] >> lshift) & nib) | (((hi[k] >> (2 * k4)) & 0x03030303u) << 4);
        }
        x.d = half_bits(r.d);
        x.sc0 = static_cast<int8_t>(r.scp & 0xFF);
        x.sc1 = static_cast<int8_t>(r.scp >> 8);
    } else {
        const uint32_t b = u * block_bytes<T> + delta;
        x.d = half_bits(r.d);
        if constexpr (T == qtype_q8_0) {
            realign(r.q, b + 2, x.q);
        } else if constexpr (T == qtype_q4_0) {
            uint32_t qs[4];
            realign(r.q, b + 2, qs);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x.q[k] = qs[k] & nib;
                x.q[4 + k] = (qs[k] >> 4) & nib;
            }
        } else {  // Q5_0
            uint32_t qh[1], qs[4];
            realign(r.qh, b + 2, qh);
            realign(r.q, b + 6, qs);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x.q[k] = (qs[k] & nib) | spread4((qh[0] >> (4 * k)) & 0xF);
                x.q[4 + k] = ((qs[k] >> 4) & nib) | spread4((qh[0] >> (16 + 4 * k)) & 0xF);
            }
        }
    }
    return x;
}

// One unit's contribution: exact integers, then the scales in float as ggml
// combines a block.
template <uint32_t T>
__device__ __forceinline__ float unit_dot(const weight_unit& w, const act_unit& a) {
    if constexpr (T == qtype_q4_k) {
        const int isum = w.sc0 * dot8(w.q, a.q, 0, 8);
        const int imin = w.sc1 * (a.s0 + a.s1);
        return (w.d * a.d) * static_cast<float>(isum) - (w.dmin * a.d) * static_cast<float>(imin);
    } else if constexpr (T == qtype_q6_k) {
        const int s0 = dot8(w.q, a.q, 0, 4) - 32 * a.s0;
        const int s1 = dot8(w.q, a.q, 4, 8) - 32 * a.s1;
        return (w.d * a.d) * static_cast<float>(w.sc0 * s0 + w.sc1 * s1);
    } else {
        // The zero point (8 for Q4_0, 16 for Q5_0) comes out through the sum.
        constexpr int zero = T == qtype_q4_0 ? 8 : (T == qtype_q5_0 ? 16 : 0);
        const int sumi = dot8(w.q, a.q, 0, 8) - zero * a.s0;
        return static_cast<float>(sumi) * (w.d * a.d);
    }
}

// ---- the fused GEMV -----------------------------------------------------------------
//
// out[r][o] = sum_c W[o][c] x[r][c] (+ bias[o]) with ggml's arithmetic: x
// quantized to the paired activation format (Q8_0 for Q4_0 / Q5_0 / Q8_0,
// Q8_K for Q4_K / Q6_K), integer block dots, float block combines.
//
// One launch. A workgroup of 8 waves first quantizes the NR activation rows
// into LDS, one lane per 32 values (the 8 lanes of a Q8_K super-block agree
// on its scale by shuffles); workgroup 0 also stores those blocks, in ggml's
// layout, into act -- the C ABI's scratch, as the reference's op_matmul
// leaves them in its scratch. Then each wave streams whole weight rows, one
// lane per 32 weights (a Q4_0/Q5_0/Q8_0 block or a 32-weight slice of a
// Q4_K/Q6_K super-block), taking rows blockIdx * 8 + wave, then every
// gridDim * 8: the grid is sized to stay resident, so the activations are
// quantized once per workgroup, not once per row. Rows are read through a
// buffer resource of the row's bytes: the 2-byte aligned formats load
// aligned dword windows realigned by v_alignbyte, and the last window's
// over-read sees zeros.

// LDS bytes of NR quantized activation rows: per unit 32 int8, a float
// scale and two int sums.
inline __host__ __device__ uint32_t gemv_lds_bytes(uint32_t nr, uint32_t units) {
    return nr * units * (32 + 4 + 8);
}

template <uint32_t T, int NR>
__global__ __launch_bounds__(512) void gemv_q_kernel(const uint8_t* w, const float* x, uint8_t* act,
                                                      const float* bias, float* out, uint32_t n, uint32_t rows,
                                                      uint32_t cols) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const uint32_t units = cols / 32;
    u4* lds_q = reinterpret_cast<u4*>(lds);                                   // [NR][units][2] x 16 B
    float* lds_d = reinterpret_cast<float*>(lds + NR * units * 32);           // [NR][units]
    int2* lds_s = reinterpret_cast<int2*>(lds + NR * units * 36);             // [NR][units]
    const uint32_t r0 = blockIdx.y * NR;

    // ---- whole weight rows, one per wave at a time ----------------------------------------
    // A wave's work is a sequence of items -- B units per lane of one row --
    // over its rows (blockIdx * 8 + wave, then every gridDim * 8). Loads run
    // two items ahead of the one being decoded, and the first two go out
    // before the activations are quantized. Every load is unconditional:
    // units past the row, and items past the wave's last, read zeros through
    // the resource without touching memory, and their products are dropped.
    constexpr int B = T == qtype_q6_k ? 1 : (T == qtype_q8_0 || T == qtype_q4_k || T == qtype_q5_0 ? 2 : 4);
    // Wave-uniform (scalar) so that the row resources live in SGPRs.
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ln = threadIdx.x & 63;
    const uint32_t wrow = cols / (k_quant<T> ? 256 : 32) * block_bytes<T>;
    const uint32_t nb = (units + 64 * B - 1) / (64 * B);  // items per row
    const uint32_t o_step = gridDim.x * 8;
    const uint32_t o0 = blockIdx.x * 8 + wv;
    const uint32_t n_items = o0 < rows ? (rows - o0 + o_step - 1) / o_step * nb : 0;
    struct item_src {
        rsrc r;
        uint32_t delta, k;
    };
    const auto item = [&](uint32_t t) {
        item_src x{make_rsrc(w, 0), 0, 0};
        if (t < n_items) {
            // Rows of an odd number of 22- or 210-byte blocks start 2 bytes
            // into a dword: the resource starts at the dword.
            const uint8_t* rp = w + static_cast<std::size_t>(o0 + t / nb * o_step) * wrow;
            x.delta = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(rp) & 3);
            x.r = make_rsrc(rp - x.delta, wrow + x.delta);
            x.k = t % nb;
        }
        return x;
    };
    raw_unit<T> buf[3][B];
    item_src src[3];
    const auto fetch_item = [&](int slot, uint32_t t) {
        src[slot] = item(t);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            buf[slot][b] = fetch<T>(src[slot].r, src[slot].delta, ln + 64 * (B * src[slot].k + b));
        }
    };
    // ---- the activations, into LDS --------------------------------------------------
    const auto quantize_store = [&](uint32_t u, int j, const x_unit& xv) __attribute__((always_inline)) {
        const uint32_t r = min(r0 + j, n - 1);
        act_unit a;
        uint16_t d_bits = 0;
        if constexpr (k_quant<T>) {
            a = quantize_q8_k(xv, u);
        } else {
            a = quantize_q8_0(xv, d_bits);
        }
        lds_q[2 * (j * units + u)] = u4{a.q[0], a.q[1], a.q[2], a.q[3]};
        lds_q[2 * (j * units + u) + 1] = u4{a.q[4], a.q[5], a.q[6], a.q[7]};
        lds_d[j * units + u] = a.d;
        lds_s[j * units + u] = int2{a.s0, a.s1};
        if (blockIdx.x == 0 && r0 + j < n) {
            store_act_unit<k_quant<T>>(act, r, units, u, a, d_bits);
        }
    };
    const auto x_row = [&](int j) { return x + static_cast<std::size_t>(min(r0 + j, n - 1)) * cols; };
    if constexpr (NR <= 2) {
        // The thread's first activation unit is loaded before the first two
        // weight items, so waiting for it does not wait for them (memory
        // operations complete in issue order as the wait counter sees them).
        x_unit xf[NR];
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            xf[j] = load_x(x_row(j), min(threadIdx.x, units - 1));
        }
        fetch_item(0, 0);
        fetch_item(1, 1);
        if (threadIdx.x < units) {
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                quantize_store(threadIdx.x, j, xf[j]);
            }
        }
        for (uint32_t u = threadIdx.x + 512; u < units; u += 512) {
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                quantize_store(u, j, load_x(x_row(j), u));
            }
        }
    } else {
        for (uint32_t u = threadIdx.x; u < units; u += 512) {
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                quantize_store(u, j, load_x(x_row(j), u));
            }
        }
        fetch_item(0, 0);
        fetch_item(1, 1);
    }
    // LDS complete; the weight loads stay in flight.
    lds_barrier();

    float acc[NR];
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        acc[j] = 0.0f;
    }
    // Item t decodes from slot C = t % 3 while item t + 2 loads into slot
    // (C + 2) % 3. Slots are compile-time (three steps per trip) so the
    // buffers stay in registers; a trip's steps past the last item run on
    // zeros and store nothing.
    const auto step = [&]<int C>(uint32_t t) __attribute__((always_inline)) {
        fetch_item((C + 2) % 3, t + 2);
        const bool live = t < n_items;
        const uint32_t k = src[C].k;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const uint32_t u = ln + 64 * (B * k + b);
            const uint32_t ua = min(u, units - 1);  // a valid LDS slot; dropped below
            const weight_unit wu = decode<T>(buf[C][b], src[C].delta, u);
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                act_unit a;
                const u4 q0 = lds_q[2 * (j * units + ua)], q1 = lds_q[2 * (j * units + ua) + 1];
                a.q[0] = q0[0], a.q[1] = q0[1], a.q[2] = q0[2], a.q[3] = q0[3];
                a.q[4] = q1[0], a.q[5] = q1[1], a.q[6] = q1[2], a.q[7] = q1[3];
                a.d = lds_d[j * units + ua];
                const int2 sm = lds_s[j * units + ua];
                a.s0 = sm.x;
                a.s1 = sm.y;
                const float c = unit_dot<T>(wu, a);
                acc[j] += live && u < units ? c : 0.0f;
            }
        }
        if (live && k + 1 == nb) {
            const uint32_t o = o0 + t / nb * o_step;
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                const float s = wave_reduce_sum(acc[j]);
                if (ln == 0 && r0 + j < n) {
                    out[static_cast<std::size_t>(r0 + j) * rows + o] = bias != nullptr ? s + bias[o] : s;
                }
                acc[j] = 0.0f;
            }
        }
    };
    for (uint32_t t = 0; t < n_items; t += 3) {
        step.template operator()<0>(t);
        step.template operator()<1>(t + 1);
        step.template operator()<2>(t + 2);
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
    const uint64_t per = t == qtype_q4_0   ? 18
                         : t == qtype_q5_0 ? 22
                         : t == qtype_q8_0 ? 34
                         : t == qtype_q4_k ? 144
                                           : 210;
    return uint64_t{cols} / qtype_block(t) * per;
}

uint64_t qtype_act_bytes(uint32_t t, uint32_t n, uint32_t cols) {
    return t == qtype_q4_k || t == qtype_q6_k ? uint64_t{n} * (cols / 256) * 292 : uint64_t{n} * (cols / 32) * 34;
}

uint32_t matmul_q_rows_per_pass(uint32_t n, uint32_t cols) {
    // Up to 4 activation rows share a pass over the weights, as LDS allows.
    for (uint32_t nr = n >= 4 ? 4 : (n >= 2 ? 2 : 1); nr >= 1; nr /= 2) {
        if (gemv_lds_bytes(nr, cols / 32) <= matmul_q_max_lds) {
            return nr;
        }
    }
    return 0;
}

namespace {

// The resident workgroups per CU of each GEMV (kernel, LDS size) per device,
// asked of the runtime once: a small fixed table (no allocation); past its
// end the runtime is asked each call.
constexpr int gemv_max_devices = 64;

struct gemv_occupancy {
    std::atomic<const void*> kernel{nullptr};
    std::atomic<uint32_t> lds{0};
    std::atomic<int> per_cu{0};
};
constexpr int gemv_occupancy_slots = 64;
gemv_occupancy gemv_occupancy_table[gemv_max_devices][gemv_occupancy_slots];

// The slot of (kernel, lds) on dev, claimed if new; null when the row is full.
gemv_occupancy* gemv_occupancy_of(int dev, const void* kernel, uint32_t lds) {
    static std::mutex claim;
    auto& row = gemv_occupancy_table[dev];
    for (auto& e : row) {
        if (e.kernel.load(std::memory_order_acquire) == kernel && e.lds.load(std::memory_order_relaxed) == lds) {
            return &e;
        }
    }
    std::lock_guard<std::mutex> lock(claim);
    for (auto& e : row) {
        const void* k = e.kernel.load(std::memory_order_relaxed);
        if (k == kernel && e.lds.load(std::memory_order_relaxed) == lds) {
            return &e;
        }
        if (k == nullptr) {
            e.lds.store(lds, std::memory_order_relaxed);
            e.kernel.store(kernel, std::memory_order_release);
            return &e;
        }
    }
    return nullptr;
}

}  // namespace

hipError_t launch_matmul_q(uint32_t t, const uint8_t* w, const float* x, uint8_t* act, const float* bias, float* out,
                           uint32_t n, uint32_t rows, uint32_t cols, hipStream_t stream) {
    if (n >= matmul_q_gemm_rows) {
        return launch_gemm_q(t, w, x, act, bias, out, n, rows, cols, stream);
    }
    const uint32_t nr = matmul_q_rows_per_pass(n, cols);
    if (nr == 0) {
        return hipErrorInvalidValue;
    }
    const uint32_t lds = gemv_lds_bytes(nr, cols / 32);
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) {
        return e;
    }
    if (dev < 0 || dev >= gemv_max_devices) {
        return hipErrorInvalidDevice;
    }
    const uint32_t cus = device_cu_count();
    if (cus == 0) {
        return hipErrorInvalidDevice;
    }
    const auto go = [&]<uint32_t T>() {
        const auto run = [&](auto kernel) {
            // A resident grid: as many 8-wave workgroups as the CUs hold at
            // once with this kernel's registers and this LDS. The occupancy
            // query runs once per (device, kernel, LDS size) and is kept.
            gemv_occupancy* slot = gemv_occupancy_of(dev, reinterpret_cast<const void*>(kernel), lds);
            int per_cu = slot ? slot->per_cu.load(std::memory_order_relaxed) : 0;
            if (per_cu < 1) {
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 512, lds) != hipSuccess ||
                    per_cu < 1) {
                    per_cu = 1;
                }
                if (slot) {
                    slot->per_cu.store(per_cu, std::memory_order_relaxed);
                }
            }
            const uint32_t resident = cus * static_cast<uint32_t>(per_cu);
            const dim3 grid(std::min((rows + 7) / 8, resident), (n + nr - 1) / nr);
            kernel<<<grid, 512, lds, stream>>>(w, x, act, bias, out, n, rows, cols);
        };
        if (nr == 4) {
            run(gemv_q_kernel<T, 4>);
        } else if (nr == 2) {
            run(gemv_q_kernel<T, 2>);
        } else {
            run(gemv_q_kernel<T, 1>);
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
