// flash.hip — bidirectional (image encoder) attention over rows on the f16
// matrix cores: session::execute(op_self_attention) (S/graph/session.hpp:
// 409-449) with self_attend_head's math (S/kernels/attention.hpp:460-486),
// for `batch` independent images of n rows each.
//
// A block (4 waves) owns 128 queries of one head of one image; wave w owns 32
// of them. Key tiles of 64 keys are staged in LDS (K rows as given; V rows
// transposed on the way in) and shared by the 4 waves. Per 32-key slice a
// wave computes
//   S^T (32 keys x 32 queries) = K (32 x hd) . Q^T          hd/16 MFMA 32x32x16
//   O^T (32 dims x 32 queries) += V^T (32 x 16 keys) . P^T   per 16 keys and 32 dims
// With S^T, a query's scores sit in one lane (two, across the lane halves),
// so the softmax row max and sum are in-lane plus one exchange, and the
// output rescale is a per-lane multiply. The K rows of a slice are loaded in
// a permuted order so that the S^T accumulator registers are, unchanged, the
// P^T operand of the second product (lane half H holds keys 8H..8H+7 of each
// 16-key step). Scores stay raw q.k; scale and log2(e) fold into one
// multiply before exp2. Operands and P are binary16 for the matrix cores
// (the reference keeps f32 here; the difference is within the parity bound).

#include "kernels.hpp"

namespace syn {

namespace {

constexpr int bq = 128;   // queries per block
constexpr int bk = 64;    // keys per LDS tile
constexpr int kpad = 8;   // halves of padding per LDS row (bank spread)

// Key offset (inside a 32-key slice) that S^T accumulator row m holds.
__device__ __forceinline__ int slice_key(int m) {
    return 16 * (m >> 4) + 8 * ((m >> 2) & 1) + 4 * ((m >> 3) & 1) + (m & 3);
}

template <bool F16>
__device__ __forceinline__ u4 load8_as_h(const void* base, std::size_t index) {
    if constexpr (F16) {
        return load16(static_cast<const _Float16*>(base) + index);
    } else {
        const float* p = static_cast<const float*>(base) + index;
        const f4 lo = *reinterpret_cast<const f4*>(p);
        const f4 hi = *reinterpret_cast<const f4*>(p + 4);
        h8 r;
        r[0] = to_h(lo[0]);
        r[1] = to_h(lo[1]);
        r[2] = to_h(lo[2]);
        r[3] = to_h(lo[3]);
        r[4] = to_h(hi[0]);
        r[5] = to_h(hi[1]);
        r[6] = to_h(hi[2]);
        r[7] = to_h(hi[3]);
        return as_u4(r);
    }
}

// K and V rows of type QF16 ? f16 : f32.
template <int HD, bool QF16>
__global__ __launch_bounds__(256) void flash_kernel(const flash_args a) {
    constexpr int NS = HD / 16;       // k-steps of the score product
    constexpr int NT = HD / 32;       // 32-dim tiles of the output
    constexpr int HSPAN = HD / 2;     // dims a lane half holds across the k-steps
    constexpr int KROW = HD + kpad;   // LDS K row (halves)
    constexpr int VROW = bk + kpad;   // LDS V^T row (halves)
    __shared__ __attribute__((aligned(16))) _Float16 lk[bk * KROW];
    __shared__ __attribute__((aligned(16))) _Float16 lv[HD * VROW];

    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int ln = tid & 63;
    const int H = ln >> 5;   // lane half
    const int qi = ln & 31;  // query column of this lane
    const uint32_t hd = a.hd;
    const uint32_t qt = blockIdx.x;
    const uint32_t h = blockIdx.y;
    const uint32_t img = blockIdx.z;
    const uint32_t g = h / a.group;
    const float c = a.scale_log2e;

    const uint32_t q_first = qt * bq;                    // first query of the block
    const uint32_t q_row0 = q_first + 32 * w;            // first query of the wave
    const uint32_t my_q = q_row0 + qi;                   // this lane's query
    const std::size_t row_base = static_cast<std::size_t>(img) * a.n;

    // Q^T operand, kept for the whole block: lane (H, qi) holds query my_q,
    // dims H*HSPAN + 8*st + [0, 8).
    h8 qv[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const uint32_t d0 = H * HSPAN + 8 * st;
        if (my_q < a.n && d0 < hd) {
            qv[st] = as_h8(load8_as_h<QF16>(a.q, (row_base + my_q) * a.q_row + h * hd + d0));
        } else {
            qv[st] = as_h8(zero_u4());
        }
    }

    f16v o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            o[n][i] = 0.0f;
        }
    }
    float m_run = -INFINITY, l_run = 0.0f;

    const uint32_t kv_end = a.kv_len;

    for (uint32_t t0 = 0; t0 < kv_end; t0 += bk) {
        __syncthreads();  // the previous tile is no longer read
        // ---- stage K (rows) and V^T into LDS ----
        constexpr int kchunks = bk * (HD / 8);
#pragma unroll
        for (int cidx = tid; cidx < kchunks; cidx += 256) {
            const int kr = cidx / (HD / 8);
            const int k8 = cidx % (HD / 8);
            const uint32_t key = t0 + kr;
            u4 v = zero_u4();
            if (key < kv_end && k8 * 8 < static_cast<int>(hd)) {
                v = load8_as_h<QF16>(a.k_rows, (row_base + key) * a.row + g * hd + k8 * 8);
            }
            *reinterpret_cast<u4*>(lk + kr * KROW + k8 * 8) = v;
        }
        {
            // V rows -> V^T: each thread reads 8 dims of one key and scatters them.
            constexpr int vchunks = bk * (HD / 8);
#pragma unroll
            for (int cidx = tid; cidx < vchunks; cidx += 256) {
                const int kr = cidx % bk;
                const int d8 = cidx / bk;
                const uint32_t key = t0 + kr;
                u4 v = zero_u4();
                if (key < kv_end && d8 * 8 < static_cast<int>(hd)) {
                    v = load8_as_h<QF16>(a.v_rows, (row_base + key) * a.row + g * hd + d8 * 8);
                }
                const h8 hv = as_h8(v);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    lv[(d8 * 8 + j) * VROW + kr] = hv[j];
                }
            }
        }
        __syncthreads();

        if (q_row0 >= a.n) {
            continue;  // a wave past the last query
        }

        // ---- scores for the two 32-key slices ----
        f16v sc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sc[e][i] = 0.0f;
            }
            const _Float16* krow = lk + (32 * e + slice_key(qi)) * KROW + H * HSPAN;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const h8 kv = *reinterpret_cast<const h8*>(krow + 8 * st);
                sc[e] = mfma32(kv, qv[st], sc[e]);
            }
        }
        // Register i of slice e holds key t0 + 32e + 16(i/8) + 8H + i%8.
        float tmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t key = t0 + 32 * e + 16 * (i >> 3) + 8 * H + (i & 7);
                const bool masked = key >= kv_end;
                if (masked) {
                    sc[e][i] = -INFINITY;
                }
                tmax = fmaxf(tmax, sc[e][i]);
            }
        }
        tmax = xor_max(tmax, 32);
        const float m_new = fmaxf(m_run, tmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = fast_exp2((m_run - m_use) * c);
        m_run = m_new;
        h8 pv[4];  // P^T operands: 16-key steps 0..3 of the tile
        float psum = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const _Float16 ph = to_h(fast_exp2((sc[e][i] - m_use) * c));
                pv[2 * e + (i >> 3)][i & 7] = ph;
                psum += static_cast<float>(ph);
            }
        }
        psum = xor_sum(psum, 32);
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                o[n][i] *= alpha;
            }
        }
        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const _Float16* vrow = lv + (32 * n + qi) * VROW + 8 * H;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const h8 vv = *reinterpret_cast<const h8*>(vrow + 16 * s);
                o[n] = mfma32(vv, pv[s], o[n]);
            }
        }
    }

    if (my_q >= a.n) {
        return;
    }
    const float inv = 1.0f / l_run;
    float* out = a.out + (row_base + my_q) * a.q_row + h * hd;
    // Register i of tile n holds dim 32n + 8(i/4) + 4H + i%4.
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t d = 32 * n + 8 * b + 4 * H;
            if (d < hd) {
                const f4 v{o[n][4 * b] * inv, o[n][4 * b + 1] * inv, o[n][4 * b + 2] * inv, o[n][4 * b + 3] * inv};
                *reinterpret_cast<f4*>(out + d) = v;
            }
        }
    }
}

template <int HD>
hipError_t launch_hd(const flash_args& a, uint32_t dtype, hipStream_t stream) {
    const dim3 grid((a.n + bq - 1) / bq, a.n_heads, a.batch);
    if (dtype == 1) {
        flash_kernel<HD, true><<<grid, 256, 0, stream>>>(a);
    } else {
        flash_kernel<HD, false><<<grid, 256, 0, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_bidirectional(const flash_args& a, uint32_t in_dtype, hipStream_t stream) {
    switch ((a.hd + 31) / 32 * 32) {
    case 32:
        return launch_hd<32>(a, in_dtype, stream);
    case 64:
        return launch_hd<64>(a, in_dtype, stream);
    case 96:
        return launch_hd<96>(a, in_dtype, stream);
    case 128:
        return launch_hd<128>(a, in_dtype, stream);
    case 160:
        return launch_hd<160>(a, in_dtype, stream);
    case 192:
        return launch_hd<192>(a, in_dtype, stream);
    case 224:
        return launch_hd<224>(a, in_dtype, stream);
    case 256:
        return launch_hd<256>(a, in_dtype, stream);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace syn
