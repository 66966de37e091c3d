// decode.hip — split-KV decode attention (one query row per sequence).
//
// The GPU form of attend_group for every KV group at once
// (S/kernels/attention.hpp:185-244): out_h = softmax_t(scale q_h . K_t) V_t
// over cached rows t = 0..len-1, query head h reading KV head h / group.
//
// Memory-bound design. A block (4 waves) owns one (sequence, KV head, split
// of `chunk` positions), so every K and V byte of the split is read exactly
// once, for all `group` query heads that share it. A wave takes 32 positions
// at a time and does both products on the f16 matrix cores:
//   S^T (16 positions x 16 heads) = K (16 x hd) . q^T       2 tiles, hd/32 MFMAs each
//   O   (16 heads x 16 dims)     += P (16 x 32 positions) . V   hd/16 MFMAs
// K rows and V^T rows are the MFMA operands exactly as they sit in memory
// (one 16-byte load per lane and k-step), and the S^T tiles are laid out so
// their accumulator registers ARE the P operand of the second product: the
// position order inside a tile is permuted so that lane group G holds the 8
// consecutive positions 8G..8G+7 of the block. No LDS, no shuffles on the
// path from K to O. Softmax is online (running max and sum per head), q is
// rounded to f16 as the reference rounds it (:204-206), and p is rounded to
// f16 as the reference rounds it (:225-227) -- before normalisation here,
// which the online form needs.
//
// The 4 waves merge their (max, sum, O) through LDS; splits then merge in the
// same launch: each block publishes its partial, and the last block of a
// (sequence, KV head) to finish (an agent-scope counter) combines all splits
// in split order, so the result is deterministic, and resets the counter.

#include "kernels.hpp"

namespace syn {

namespace {

template <int HDP, bool QF16>
__device__ __forceinline__ h8 load_q8(const void* q, std::size_t index) {
    if constexpr (QF16) {
        return as_h8(load16(static_cast<const _Float16*>(q) + index));
    } else {
        const float* p = static_cast<const float*>(q) + index;
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
        return r;
    }
}

template <int HDP, bool QF16>
__global__ __launch_bounds__(256) void decode_kernel(const decode_args a) {
    constexpr int NS = HDP / 32;   // k-steps of the score product
    constexpr int NT = HDP / 16;   // 16-dim tiles of the output
    constexpr int SPAN = HDP / 4;  // dims a lane group holds across the k-steps
    extern __shared__ float lds[];  // [4][16][2] (max, sum), then [2][group][hd]

    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int ln = tid & 63;
    const int G = ln >> 4;  // lane group
    const int r = ln & 15;  // row / column inside the group
    const uint32_t hd = a.hd;
    const uint32_t group = a.group;

    // Block -> (sequence, split, KV head). Splits of one KV head are n_kv
    // blocks apart, so with n_kv a multiple of 8 they share an XCD (and its L2).
    const uint32_t b = blockIdx.x;
    const uint32_t g = b % a.n_kv;
    const uint32_t sb = b / a.n_kv;
    uint32_t si = 0;
    while (si + 1 < a.n_seqs && sb >= a.seq[si + 1].block0) {
        ++si;
    }
    const decode_seq s = a.seq[si];
    const uint32_t split = sb - s.block0;
    const uint32_t t_begin = split * a.chunk;
    const uint32_t t_end = min(s.len, t_begin + a.chunk);
    const uint32_t h0 = g * group;
    const float c = a.scale_log2e;

    // q^T operand: lane (G, r) holds head h0 + r, dims G*SPAN + 8*st + [0, 8).
    h8 qv[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const uint32_t d0 = G * SPAN + 8 * st;
        if (static_cast<uint32_t>(r) < group && d0 < hd) {
            qv[st] = load_q8<HDP, QF16>(s.q, static_cast<std::size_t>(h0 + r) * hd + d0);
        } else {
            qv[st] = as_h8(zero_u4());
        }
    }

    float m_run = -INFINITY;  // running max of raw q.k for head r
    float l_run = 0.0f;       // running sum of f16-rounded p for head r
    f4 o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        o[n] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const _Float16* kbase = s.k + g * hd + G * SPAN;
    for (uint32_t tb = t_begin + decode_positions_per_wave * w; tb < t_end;
         tb += decode_positions_per_wave * decode_waves) {
        // K rows for the two S^T tiles: row r of tile e is position
        // tb + 8*(r/4) + 4*e + r%4, so accumulator row 4G+i of tile e is
        // position tb + 8G + 4e + i.
        u4 kr[2][NS];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t t = tb + 8 * (r >> 2) + 4 * e + (r & 3);
            const _Float16* kp = kbase + static_cast<std::size_t>(t) * a.row;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const bool ok = t < s.len && G * SPAN + 8 * st < hd;
                kr[e][st] = ok ? load16(kp + 8 * st) : zero_u4();
            }
        }
        // V^T rows: lane (G, r) of tile n holds dim 16n + r at positions tb + 8G + [0, 8).
        const uint32_t tv = tb + 8 * G;
        u4 vr[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const uint32_t dim = 16 * n + r;
            const bool ok = dim < hd && tv < s.len;
            vr[n] = ok ? load16(s.vt + static_cast<std::size_t>(g * hd + dim) * s.ctx_stride + tv) : zero_u4();
        }

        f4 sc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            sc[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                sc[e] = mfma16(as_h8(kr[e][st]), qv[st], sc[e]);
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (tv + 4 * e + i >= t_end) {
                    sc[e][i] = -INFINITY;
                }
                bm = fmaxf(bm, sc[e][i]);
            }
        }
        bm = xor_max(bm, 16);
        bm = xor_max(bm, 32);
        const float m_new = fmaxf(m_run, bm);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = fast_exp2((m_run - m_use) * c);
        h8 pa;
        float ps = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const _Float16 ph = to_h(fast_exp2((sc[e][i] - m_use) * c));
                pa[4 * e + i] = ph;
                ps += static_cast<float>(ph);
            }
        }
        ps = xor_sum(ps, 16);
        ps = xor_sum(ps, 32);
        l_run = l_run * alpha + ps;
        m_run = m_new;

        // Output rows are heads 4G + i: fetch their rescale factors.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * G + i, wave);
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                o[n][i] *= ai;
            }
        }
        // Positions past the split end carry p = 0; zero their V too, so a
        // stale non-finite half past the cache's length cannot reach O.
        if (tv + 8 > t_end) {
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                h8 v = as_h8(vr[n]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (tv + j >= t_end) {
                        v[j] = 0;
                    }
                }
                vr[n] = as_u4(v);
            }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            o[n] = mfma16(pa, as_h8(vr[n]), o[n]);
        }
    }

    // ---- merge the 4 waves ---------------------------------------------------
    float* lds_ml = lds;
    float* lds_o = lds + 4 * 16 * 2;
    if (G == 0) {
        lds_ml[(w * 16 + r) * 2] = m_run;
        lds_ml[(w * 16 + r) * 2 + 1] = l_run;
    }
    __syncthreads();
    float fac[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * G + i;
        float mx = lds_ml[h * 2];
#pragma unroll
        for (int v = 1; v < 4; ++v) {
            mx = fmaxf(mx, lds_ml[(v * 16 + h) * 2]);
        }
        fac[i] = fast_exp2((lds_ml[(w * 16 + h) * 2] - mx) * c);
    }
    // Waves 0, 1 store their scaled O; waves 2, 3 then add theirs on top.
    const int slot = w & 1;
    for (int phase = 0; phase < 2; ++phase) {
        if ((w >> 1) == phase) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t h = 4 * G + i;
                if (h < group) {
#pragma unroll
                    for (int n = 0; n < NT; ++n) {
                        const uint32_t d = 16 * n + r;
                        if (d < hd) {
                            float* dst = lds_o + (slot * group + h) * hd + d;
                            const float v = o[n][i] * fac[i];
                            *dst = phase == 0 ? v : *dst + v;
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    const uint32_t nout = group * hd;
    if (s.n_splits == 1) {
        float* out = s.out + static_cast<std::size_t>(h0) * hd;
        for (uint32_t e = tid; e < nout; e += 256) {
            const uint32_t h = e / hd;
            float mx = lds_ml[h * 2];
            for (int v = 1; v < 4; ++v) {
                mx = fmaxf(mx, lds_ml[(v * 16 + h) * 2]);
            }
            float sum = 0.0f;
            for (int v = 0; v < 4; ++v) {
                sum += lds_ml[(v * 16 + h) * 2 + 1] * fast_exp2((lds_ml[(v * 16 + h) * 2] - mx) * c);
            }
            out[e] = (lds_o[e] + lds_o[nout + e]) / sum;
        }
        return;
    }

    // ---- publish this split's partial ------------------------------------------
    for (uint32_t e = tid; e < nout; e += 256) {
        const uint32_t h = e / hd;
        const uint32_t d = e % hd;
        a.part_o[static_cast<std::size_t>(b) * nout + e] = lds_o[e] + lds_o[nout + e];
        if (d == 0) {
            float mx = lds_ml[h * 2];
            for (int v = 1; v < 4; ++v) {
                mx = fmaxf(mx, lds_ml[(v * 16 + h) * 2]);
            }
            float sum = 0.0f;
            for (int v = 0; v < 4; ++v) {
                sum += lds_ml[(v * 16 + h) * 2 + 1] * fast_exp2((lds_ml[(v * 16 + h) * 2] - mx) * c);
            }
            a.part_ml[(static_cast<std::size_t>(b) * group + h) * 2] = mx;
            a.part_ml[(static_cast<std::size_t>(b) * group + h) * 2 + 1] = sum;
        }
    }
    __threadfence();  // this thread's partial stores, visible device-wide
    __syncthreads();
    __shared__ uint32_t last;
    uint32_t* counter = a.counters + a.counter0 + si * a.n_kv + g;
    if (tid == 0) {
        last = atomicAdd(counter, 1u) == s.n_splits - 1 ? 1u : 0u;
    }
    __syncthreads();
    if (!last) {
        return;
    }
    __threadfence();  // acquire every other split's partial

    // ---- last block: combine the splits in split order -------------------------
    float* out = s.out + static_cast<std::size_t>(h0) * hd;
    for (uint32_t e = tid; e < nout; e += 256) {
        const uint32_t h = e / hd;
        float mx = -INFINITY, sum = 0.0f, acc = 0.0f;
        for (uint32_t j = 0; j < s.n_splits; ++j) {
            const std::size_t pb = static_cast<std::size_t>(s.block0 + j) * a.n_kv + g;
            const float mj = a.part_ml[(pb * group + h) * 2];
            const float lj = a.part_ml[(pb * group + h) * 2 + 1];
            const float oj = a.part_o[pb * nout + e];
            const float m_new = fmaxf(mx, mj);
            const float sa = fast_exp2((mx - m_new) * c);
            const float sj = fast_exp2((mj - m_new) * c);
            sum = sum * sa + lj * sj;
            acc = acc * sa + oj * sj;
            mx = m_new;
        }
        out[e] = acc / sum;
    }
    if (tid == 0) {
        *counter = 0u;  // ready for the next launch
    }
}

template <int HDP>
hipError_t launch_hdp(const decode_args& a, uint32_t total_splits, uint32_t q_dtype, hipStream_t stream) {
    const std::size_t lds = (4 * 16 * 2 + 2 * static_cast<std::size_t>(a.group) * a.hd) * sizeof(float);
    const dim3 grid(total_splits * a.n_kv);
    if (q_dtype == 1) {
        decode_kernel<HDP, true><<<grid, 256, lds, stream>>>(a);
    } else {
        decode_kernel<HDP, false><<<grid, 256, lds, stream>>>(a);
    }
    return hipGetLastError();
}

}  // namespace

uint32_t decode_choose_chunk(uint64_t total_positions, uint32_t n_kv) {
    // Enough splits to give every CU about one block of 128 positions per
    // KV-head pass; longer runs take longer chunks, which keeps the partials
    // (and the last block's merge) small against the KV bytes.
    const uint64_t work = total_positions * n_kv;
    uint32_t chunk = decode_chunk_unit;
    while (chunk < 1024 && work / chunk > 2048) {
        chunk *= 2;
    }
    return chunk;
}

hipError_t launch_decode(const decode_args& a, uint32_t total_splits, uint32_t q_dtype, hipStream_t stream) {
    const uint32_t hdp = (a.hd + 31) / 32 * 32;
    switch (hdp) {
    case 32:
        return launch_hdp<32>(a, total_splits, q_dtype, stream);
    case 64:
        return launch_hdp<64>(a, total_splits, q_dtype, stream);
    case 96:
        return launch_hdp<96>(a, total_splits, q_dtype, stream);
    case 128:
        return launch_hdp<128>(a, total_splits, q_dtype, stream);
    case 160:
        return launch_hdp<160>(a, total_splits, q_dtype, stream);
    case 192:
        return launch_hdp<192>(a, total_splits, q_dtype, stream);
    case 224:
        return launch_hdp<224>(a, total_splits, q_dtype, stream);
    case 256:
        return launch_hdp<256>(a, total_splits, q_dtype, stream);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace syn
