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

#include "softmax.hpp"

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

// ---- head-resident form -------------------------------------------------------
// When an image's K and V^T for one head fit in LDS (short rows, as a ViT's
// 257 tokens), a block owns one (image, head): it stages all n keys once --
// K rows padded by one 16-byte chunk, V transposed to V^T rows -- and then
// its waves sweep their 32-query tiles over the resident keys in 32-key
// slices, with no further barriers or global loads besides q. Keys past n
// are zero rows and masked.

// LDS bytes of the resident form for n keys (keys padded to a multiple of 32).
__host__ __device__ constexpr uint32_t resident_lds_bytes(uint32_t n, uint32_t hdp) {
    const uint32_t np = (n + 31) / 32 * 32;
    return np * (hdp / 8 + 1) * 16 + hdp * (np / 8 + 1) * 16;
}
// Two blocks per CU: at most 80 KB each.
constexpr uint32_t resident_lds_limit = 80 * 1024;
// The most keys (a multiple of 32) the resident form holds at head size hdp.
__host__ __device__ constexpr uint32_t resident_max_keys(uint32_t hdp) {
    uint32_t np = 32;
    while (resident_lds_bytes(np + 32, hdp) <= resident_lds_limit) {
        np += 32;
    }
    return np;
}
// Keys of the first staging half for np (padded) keys: about half, a
// multiple of 64 (the compute steps' size), all of them up to 64.
__host__ __device__ constexpr uint32_t resident_half1(uint32_t np) {
    return np <= 64 ? np : (np / 128 > 0 ? np / 128 * 64 : 64);
}
// The most keys either half holds for up to npmax keys.
__host__ __device__ constexpr uint32_t resident_half1_max(uint32_t npmax) {
    uint32_t m = 0;
    for (uint32_t np = 32; np <= npmax; np += 32) {
        m = resident_half1(np) > m ? resident_half1(np) : m;
    }
    return m;
}
__host__ __device__ constexpr uint32_t resident_half2_max(uint32_t npmax) {
    uint32_t m = 0;
    for (uint32_t np = 32; np <= npmax; np += 32) {
        m = np - resident_half1(np) > m ? np - resident_half1(np) : m;
    }
    return m;
}

template <int HD, bool F16>
__global__ __launch_bounds__(256, 2) void resident_kernel(const flash_args a) {
    constexpr int NS = HD / 16;      // k-steps of the score product
    constexpr int NT = HD / 32;      // 32-dim tiles of the output
    constexpr int KCPR = HD / 8;     // 16-byte chunks of a K row
    constexpr int KROWC = KCPR + 1;  // LDS K row in chunks (one of padding)
    extern __shared__ __attribute__((aligned(16))) char lds[];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = tid & 63;
    const int H = ln >> 5;
    const int qi = ln & 31;
    const uint32_t n = a.n;
    const uint32_t hd = a.hd;
    const uint32_t np = (n + 31) / 32 * 32;
    const uint32_t vrowc = np / 8 + 1;  // LDS V^T row in chunks (one of padding)
    const uint32_t h = blockIdx.x % a.n_heads;
    const uint32_t img = blockIdx.x / a.n_heads;
    const std::size_t row_base = static_cast<std::size_t>(img) * n;
    const float c = a.scale_log2e;
    char* lk = lds;
    char* lv = lds + np * KROWC * 16;

    // ---- stage K rows and V^T in two halves of the keys ----
    // Keys [0, kh) are the first half and [kh, np) the second. Every load of
    // the block is issued at once, q and the first half first; the waves then
    // run all their query tiles over the first half while the second half
    // lands, and finish over the second. Zeros past n and past hd.
    // f32 rows take twice the staging registers: they stage all keys at
    // once (the first half is everything).
    constexpr uint32_t NPMAX = resident_max_keys(HD);
    constexpr uint32_t CH1 = ((F16 ? resident_half1_max(NPMAX) : NPMAX) * KCPR + 255) / 256;  // chunks per thread
    constexpr uint32_t CH2 = F16 ? (resident_half2_max(NPMAX) * KCPR + 255) / 256 : 1;
    constexpr uint32_t ESZ = F16 ? 2 : 4;
    const uint32_t kh = F16 ? resident_half1(np) : np;
    // The image's rows through buffer resources: chunks past n or past hd
    // take an out-of-range offset and read as zeros, so every load is
    // unconditional.
    const uint32_t img_bytes = n * a.row * ESZ;
    const rsrc k_res = make_rsrc(static_cast<const char*>(a.k_rows) + row_base * a.row * ESZ, img_bytes);
    const rsrc v_res = make_rsrc(static_cast<const char*>(a.v_rows) + row_base * a.row * ESZ, img_bytes);
    const auto chunk = [&](rsrc r, uint32_t off) {
        if constexpr (F16) {
            return buffer_load16(r, off);
        } else {
            const f4 lo = __builtin_bit_cast(f4, buffer_load16(r, off));
            const f4 hi = __builtin_bit_cast(f4, buffer_load16(r, off == buffer_oob ? off : off + 16));
            return as_u4(h8{to_h(lo[0]), to_h(lo[1]), to_h(lo[2]), to_h(lo[3]), to_h(hi[0]), to_h(hi[1]),
                            to_h(hi[2]), to_h(hi[3])});
        }
    };
    // The wave's q tiles (wave (w + block) % 4 takes tiles w', w' + 4, ..., so
    // the extra tiles of co-resident blocks land on different SIMDs) go out
    // first.
    constexpr uint32_t TPW = (NPMAX / 32 + 3) / 4;  // q tiles per wave, at most
    const uint32_t n_qt = np / 32;
    const uint32_t w0 = (static_cast<uint32_t>(w) + blockIdx.x) % 4;
    const rsrc q_res = make_rsrc(static_cast<const char*>(a.q) + row_base * a.q_row * ESZ, n * a.q_row * ESZ);
    u4 qc[TPW][NS];
#pragma unroll
    for (uint32_t t = 0; t < TPW; ++t) {
        const uint32_t my_q = 32 * (w0 + 4 * t) + qi;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const uint32_t d0 = H * (HD / 2) + 8 * st;
            qc[t][st] = chunk(q_res, my_q < n && d0 < hd ? (my_q * a.q_row + h * hd + d0) * ESZ : buffer_oob);
        }
    }
    // Chunk i of a half [k0, k1): K takes row-major chunks (consecutive lanes
    // read consecutive 16 bytes of a row), V takes consecutive keys of one
    // 8-dim chunk (each of the 8 half-word writes of a wave then covers 128
    // contiguous bytes of a V^T row).
    const auto load_half = [&]<uint32_t C>(uint32_t k0, uint32_t k1, u4 (&kc)[C], u4 (&vc)[C])
                               __attribute__((always_inline)) {
        const uint32_t count = (k1 - k0) * KCPR, span = max(k1 - k0, 1u);  // an empty half loads nothing
#pragma unroll
        for (uint32_t i = 0; i < C; ++i) {
            const uint32_t idx = tid + 256 * i;
            const uint32_t key = k0 + idx / KCPR, cc = idx % KCPR;
            kc[i] = chunk(k_res, idx < count && key < n && 8 * cc < hd ? (key * a.row + h * hd + 8 * cc) * ESZ
                                                                       : buffer_oob);
            const uint32_t vkey = k0 + idx % span, vcc = idx / span;
            vc[i] = chunk(v_res, idx < count && vkey < n && 8 * vcc < hd
                                     ? (vkey * a.row + h * hd + 8 * vcc) * ESZ
                                     : buffer_oob);
        }
    };
    const auto store_half = [&]<uint32_t C>(uint32_t k0, uint32_t k1, const u4 (&kc)[C], const u4 (&vc)[C])
                                __attribute__((always_inline)) {
        const uint32_t count = (k1 - k0) * KCPR, span = max(k1 - k0, 1u);
#pragma unroll
        for (uint32_t i = 0; i < C; ++i) {
            const uint32_t idx = tid + 256 * i;
            if (idx < count) {
                const uint32_t key = k0 + idx / KCPR, cc = idx % KCPR;
                *reinterpret_cast<u4*>(lk + (key * KROWC + cc) * 16) = kc[i];
                const uint32_t vkey = k0 + idx % span, vcc = idx / span;
                const h8 hv = as_h8(vc[i]);
                _Float16* col = reinterpret_cast<_Float16*>(lv) + (8 * vcc * vrowc * 8 + vkey);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    col[j * vrowc * 8] = hv[j];
                }
            }
        }
    };
    u4 kc1[CH1], vc1[CH1], kc2[CH2], vc2[CH2];
    load_half(0, kh, kc1, vc1);
    if constexpr (F16) {
        load_half(kh, np, kc2, vc2);
    }

    // ---- the wave's query tiles over the resident keys ----
    // The first tile runs over the first half while the second half lands;
    // the other tiles start once all keys are resident.
    f16v o[NT];
    float m_run = -INFINITY, l_run = 0.0f;
    h8 qv[NS];
    // E 32-key slices from key t0 (keys past n masked).
    const auto step = [&]<int E>(uint32_t t0) __attribute__((always_inline)) {
        f16v sc[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sc[e][i] = 0.0f;
            }
            const char* krow = lk + ((t0 + 32 * e + slice_key(qi)) * KROWC + H * (KCPR / 2)) * 16;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                sc[e] = mfma32(*reinterpret_cast<const h8*>(krow + 16 * st), qv[st], sc[e]);
            }
        }
        // Register i of slice e holds key t0 + 32e + 16(i/8) + 8H + i%8:
        // masked unless ck = 32e + 16(i/8) + i%8 < n - t0 - 8H.
        if (t0 + 32 * E > n) {
            const int dk = static_cast<int>(n - t0) - 8 * H;
#pragma unroll
            for (int e = 0; e < E; ++e) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int ck = 32 * e + 16 * (i >> 3) + (i & 7);
                    sc[e][i] = ck < dk ? sc[e][i] : -INFINITY;
                }
            }
        }
        h8 pv[2 * E];
        online_softmax<E, NT>(sc, c, m_run, l_run, o, pv);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            // V^T row 32t + qi, keys t0 + 8H + 16 s ..
            const char* vrow = lv + ((32 * t + qi) * vrowc + t0 / 8 + H) * 16;
#pragma unroll
            for (int s2 = 0; s2 < 2 * E; ++s2) {
                o[t] = mfma32(*reinterpret_cast<const h8*>(vrow + 32 * s2), pv[s2], o[t]);
            }
        }
    };
    // Keys [k0, k1) of the current tile (k0 a multiple of 64).
    const auto sweep = [&](uint32_t k0, uint32_t k1) __attribute__((always_inline)) {
        uint32_t t0 = k0;
        for (; t0 + 64 <= k1; t0 += 64) {
            step.template operator()<2>(t0);
        }
        if (t0 < k1) {
            step.template operator()<1>(t0);
        }
    };
    const auto begin_tile = [&](uint32_t tq) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            qv[st] = as_h8(qc[tq][st]);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                o[t][i] = 0.0f;
            }
        }
        m_run = -INFINITY;
        l_run = 0.0f;
    };
    const auto end_tile = [&](uint32_t tq) __attribute__((always_inline)) {
        const uint32_t my_q = 32 * (w0 + 4 * tq) + qi;
        if (my_q >= n) {
            return;
        }
        const float inv = 1.0f / l_run;
        float* out = a.out + (row_base + my_q) * a.q_row + h * hd;
        // Register i of tile t holds dim 32t + 8(i/4) + 4H + i%4.
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t d = 32 * t + 8 * b + 4 * H;
                if (d < hd) {
                    *reinterpret_cast<f4*>(out + d) =
                        f4{o[t][4 * b] * inv, o[t][4 * b + 1] * inv, o[t][4 * b + 2] * inv, o[t][4 * b + 3] * inv};
                }
            }
        }
    };
    // LDS-only barriers: the second half's loads stay in flight across the
    // first. No wave still reads the first half's rows when another writes
    // the second half's: the halves are disjoint in LDS.
    const bool first = w0 < n_qt;  // this wave has a tile at all
    store_half(0, kh, kc1, vc1);
    lds_barrier();
    if (first) {
        begin_tile(0);
        sweep(0, kh);
    }
    if constexpr (F16) {
        store_half(kh, np, kc2, vc2);
        lds_barrier();
    }
    if (first) {
        sweep(kh, np);
        end_tile(0);
    }
#pragma unroll
    for (uint32_t tq = 1; tq < TPW; ++tq) {
        if (w0 + 4 * tq >= n_qt) {
            break;
        }
        begin_tile(tq);
        sweep(0, np);
        end_tile(tq);
    }
}

// f16 rows only: f32 rows of images this short take the f32 kernel
// (generic.hip), which keeps the reference's f32 arithmetic.
template <int HD>
hipError_t launch_resident(const flash_args& a, uint32_t lds_bytes, hipStream_t stream) {
    const dim3 grid(a.n_heads * a.batch);
    resident_kernel<HD, true><<<grid, 256, lds_bytes, stream>>>(a);
    return hipGetLastError();
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
    const uint32_t hdp = (a.hd + 31) / 32 * 32;
    // Resident form while two blocks fit a CU's LDS (160 KB).
    // (An image's rows are addressed through one buffer resource: < 2^31 bytes.)
    if (in_dtype == 1 && hdp <= 128 && uint64_t{a.n_heads} * a.batch <= 0x7fffffffu &&
        uint64_t{a.n} * a.row * 2 < (uint64_t{1} << 31)) {
        const uint32_t bytes = resident_lds_bytes(a.n, hdp);
        if (bytes <= resident_lds_limit) {
            switch (hdp) {
            case 32:
                return launch_resident<32>(a, bytes, stream);
            case 64:
                return launch_resident<64>(a, bytes, stream);
            case 96:
                return launch_resident<96>(a, bytes, stream);
            default:
                return launch_resident<128>(a, bytes, stream);
            }
        }
    }
    switch (hdp) {
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
