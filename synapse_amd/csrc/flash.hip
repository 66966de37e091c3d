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
// When one head of one image (a unit: its K rows and V^T) fits in half a
// CU's LDS (short rows, as a ViT's 257 tokens), a block of 4 waves keeps it
// resident, two blocks per CU. Every load of the block goes out at the
// start (K rows, V rows and each wave's q tiles, into registers); the K rows
// then go to padded LDS rows and V is transposed to V^T rows, and after one
// barrier wave w0 sweeps query tiles w0, w0 + 4, ... over the unit's keys in
// 32-key slices, with no further barriers or K/V loads. Keys past n are zero
// rows and masked.

// LDS bytes of one unit's K rows and V^T for n keys (padded to 32).
__host__ __device__ constexpr uint32_t resident_lds_bytes(uint32_t n, uint32_t hdp) {
    const uint32_t np = (n + 31) / 32 * 32;
    return np * (hdp / 8 + 1) * 16 + hdp * (np / 8 + 1) * 16;
}
// A last query tile of at most this many rows that would be a third tile on
// one wave (query tiles = 1 mod 4, as 257 rows make 9) is computed on the
// vector units instead, by all four waves after their tiles, so every wave
// sweeps the same number of tiles. Its LDS: the rows' q and one row of
// scores (then probabilities).
constexpr uint32_t resident_tail_rows = 2;
__host__ __device__ constexpr uint32_t resident_tail_bytes(uint32_t n, uint32_t hdp) {
    return resident_tail_rows * hdp * 2 + (n + 31) / 32 * 32 * 4;
}
__host__ __device__ constexpr bool resident_has_tail(uint32_t n) {
    const uint32_t n_qt = (n + 31) / 32;
    return n_qt % 4 == 1 && n - 32 * (n_qt - 1) <= resident_tail_rows;
}
__host__ __device__ constexpr uint32_t resident_unit_bytes(uint32_t n, uint32_t hdp) {
    return resident_lds_bytes(n, hdp) + (resident_has_tail(n) ? resident_tail_bytes(n, hdp) : 0u);
}
// Two blocks per CU: at most 80 KB each.
constexpr uint32_t resident_lds_limit = 80 * 1024;
// The most keys (a multiple of 32) the resident form holds at head size hdp.
__host__ __device__ constexpr uint32_t resident_max_keys(uint32_t hdp) {
    uint32_t np = 32;
    while (resident_lds_bytes(np + 32, hdp) + resident_tail_bytes(np + 32, hdp) <= resident_lds_limit) {
        np += 32;
    }
    return np;
}

// Staggered staging. Two blocks share each CU, and a block computes nothing
// until its whole unit has landed; when both stage at once, both land late.
// Blocks from..to-1 -- the second block on their CU, with the grid dealt to
// the CUs in order -- wait `ticks` of the 100 MHz constant clock first: the
// time the first block's bytes take at peak HBM bandwidth shared over the
// CUs. The first block then computes while the second's bytes land.
struct resident_stagger {
    uint32_t from, to, ticks;
};

template <int HD>
__global__ __launch_bounds__(256, 2) void resident_kernel(const flash_args a, const resident_stagger st) {
    constexpr int NS = HD / 16;      // k-steps of the score product
    constexpr int NT = HD / 32;      // 32-dim tiles of the output
    constexpr int KCPR = HD / 8;     // 16-byte chunks of a K row
    constexpr int KROWC = KCPR + 1;  // LDS K row in chunks (one of padding)
    constexpr uint32_t WAVES = 4;
    constexpr uint32_t THREADS = 64 * WAVES;
    constexpr uint32_t NPMAX = resident_max_keys(HD);
    constexpr uint32_t KC = (NPMAX * KCPR + THREADS - 1) / THREADS;      // K chunks per thread and unit
    constexpr uint32_t VC = (NPMAX / 2 * KCPR + THREADS - 1) / THREADS;  // V key pairs per thread and unit
    // Up to head dim 64 a wave stages only its first query tile's q and
    // loads each later tile's during the tile before (the staging, which
    // every wave waits for, is then ~16 % smaller); above, the registers are
    // not there, and the first QT tiles are staged.
    constexpr bool QPRE = HD <= 64;
    constexpr uint32_t QT = QPRE ? 1 : (NPMAX / 32 + WAVES - 1) / WAVES;  // q tiles staged per wave
    extern __shared__ __attribute__((aligned(16))) char lds[];

    const int tid = threadIdx.x;
    const int ln = tid & 63;
    const int H = ln >> 5;
    const int qi = ln & 31;
    // Wave w0 takes tiles w0, w0 + WAVES, ...; rotated by the block so that
    // the extra tiles of co-resident blocks land on different SIMDs.
    const uint32_t w0 = (static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(tid >> 6)) + blockIdx.x) % WAVES;
    const uint32_t n = a.n;
    const uint32_t hd = a.hd;
    const uint32_t np = (n + 31) / 32 * 32;
    const uint32_t vrowc = np / 8 + 1;  // LDS V^T row in chunks (one of padding)
    const uint32_t n_qt = np / 32;
    const bool tail = resident_has_tail(n);
    const uint32_t n_mq = tail ? n_qt - 1 : n_qt;  // tiles on the matrix cores
    const float c = a.scale_log2e;

    // The unit's head, rows and LDS; its rows through buffer resources:
    // chunks past n or past hd take an out-of-range offset and read as
    // zeros, so every load is unconditional.
    struct unit {
        uint32_t h;
        std::size_t row_base;
        char* lk;
        char* lv;
        rsrc k_res, v_res, q_res;
    };
    unit U;
    U.h = blockIdx.x % a.n_heads;
    U.row_base = static_cast<std::size_t>(blockIdx.x / a.n_heads) * n;
    U.lk = lds;
    U.lv = lds + np * KROWC * 16;
    const uint32_t img_bytes = n * a.row * 2;
    U.k_res = make_rsrc(static_cast<const _Float16*>(a.k_rows) + U.row_base * a.row, img_bytes);
    U.v_res = make_rsrc(static_cast<const _Float16*>(a.v_rows) + U.row_base * a.row, img_bytes);
    U.q_res = make_rsrc(static_cast<const _Float16*>(a.q) + U.row_base * a.q_row, n * a.q_row * 2);

    // Staging. K: chunk idx is chunk idx % KCPR of key idx / KCPR
    // (consecutive lanes read consecutive 16 bytes of a row). V: the same
    // over key pairs, a lane reading one 8-dim chunk of two consecutive
    // keys, so each of its 8 dword writes to LDS puts one dim of both keys
    // into a V^T row.
    const auto load_unit = [&](u4 (&kc)[KC], u4 (&vc)[VC][2], u4 (&qc)[QT][NS], u4& tq)
                               __attribute__((always_inline)) {
        const uint32_t count = np * KCPR;
#pragma unroll
        for (uint32_t i = 0; i < KC; ++i) {
            const uint32_t idx = tid + THREADS * i;
            const uint32_t key = idx / KCPR, cc = idx % KCPR;
            kc[i] = buffer_load16(U.k_res, idx < count && key < n && 8 * cc < hd ? (key * a.row + U.h * hd + 8 * cc) * 2
                                                                               : buffer_oob);
        }
#pragma unroll
        for (uint32_t i = 0; i < VC; ++i) {
            const uint32_t idx = tid + THREADS * i;
            const uint32_t key = 2 * (idx / KCPR), cc = idx % KCPR;
            const bool in = 2 * idx < count && 8 * cc < hd;
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                vc[i][e] = buffer_load16(U.v_res, in && key + e < n ? ((key + e) * a.row + U.h * hd + 8 * cc) * 2
                                                                    : buffer_oob);
            }
        }
        // The wave's first QT query tiles (tile w0 + WAVES t): lane (qi, H)
        // holds dims H * HD / 2 + 8 st of row 32 tile + qi, the score
        // product's operand.
#pragma unroll
        for (uint32_t t = 0; t < QT; ++t) {
            const uint32_t tile = w0 + WAVES * t;
            const uint32_t my_q = 32 * tile + qi;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const uint32_t d0 = H * (HD / 2) + 8 * st;
                qc[t][st] = buffer_load16(U.q_res, tile < n_mq && my_q < n && d0 < hd
                                                       ? (my_q * a.q_row + U.h * hd + d0) * 2
                                                       : buffer_oob);
            }
        }
        // The tail rows' q, chunk ln (row ln / KCPR); wave 0's copy goes to
        // LDS for the block.
        const uint32_t tr = 32 * n_mq + ln / KCPR, tc = ln % KCPR;
        tq = buffer_load16(U.q_res, tail && tr < n && 8 * tc < hd ? (tr * a.q_row + U.h * hd + 8 * tc) * 2
                                                                  : buffer_oob);
    };
    const auto store_unit = [&](const u4 (&kc)[KC], const u4 (&vc)[VC][2]) __attribute__((always_inline)) {
        const uint32_t count = np * KCPR;
#pragma unroll
        for (uint32_t i = 0; i < KC; ++i) {
            const uint32_t idx = tid + THREADS * i;
            if (idx < count) {
                *reinterpret_cast<u4*>(U.lk + ((idx / KCPR) * KROWC + idx % KCPR) * 16) = kc[i];
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < VC; ++i) {
            const uint32_t idx = tid + THREADS * i;
            if (2 * idx < count) {
                // The key count np is even, so a key pair is a dword of
                // every V^T row.
                const uint32_t key = 2 * (idx / KCPR), cc = idx % KCPR;
                const h8 v0 = as_h8(vc[i][0]), v1 = as_h8(vc[i][1]);
                _Float16* col = reinterpret_cast<_Float16*>(U.lv) + (8 * cc * vrowc * 8 + key);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    *reinterpret_cast<h2*>(col + j * vrowc * 8) = h2{v0[j], v1[j]};
                }
            }
        }
    };

    // ---- a wave's query tiles over a unit's resident keys ----
    f16v o[NT];
    float m_run = -INFINITY, l_run = 0.0f;
    h8 qv[NS];
    // E 32-key slices from key t0 (keys past n masked).
    const auto step = [&]<int E, bool FIRST>(uint32_t t0) __attribute__((always_inline)) {
        f16v sc[E];
        // All K operands are read before the first product, and (up to head
        // dim 64, where the registers are there) the V^T operands right after
        // the score products: their LDS latency then runs under the products
        // and the softmax instead of before each product.
        h8 kop[E][NS];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const char* krow = U.lk + ((t0 + 32 * e + slice_key(qi)) * KROWC + H * (KCPR / 2)) * 16;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                kop[e][st] = *reinterpret_cast<const h8*>(krow + 16 * st);
            }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sc[e][i] = 0.0f;
            }
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                sc[e] = mfma32(kop[e][st], qv[st], sc[e]);
            }
        }
        constexpr bool VPRE = HD <= 64;
        h8 vop[VPRE ? NT : 1][VPRE ? 2 * E : 1];
        if constexpr (VPRE) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const char* vrow = U.lv + ((32 * t + qi) * vrowc + t0 / 8 + H) * 16;
#pragma unroll
                for (int s2 = 0; s2 < 2 * E; ++s2) {
                    vop[t][s2] = *reinterpret_cast<const h8*>(vrow + 32 * s2);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
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
        if constexpr (FIRST) {
            first_softmax<E>(sc, c, m_run, l_run, pv);
        } else {
            online_softmax<E, NT>(sc, c, m_run, l_run, o, pv);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            // V^T row 32t + qi, keys t0 + 8H + 16 s ..
            const char* vrow = U.lv + ((32 * t + qi) * vrowc + t0 / 8 + H) * 16;
#pragma unroll
            for (int s2 = 0; s2 < 2 * E; ++s2) {
                if constexpr (VPRE) {
                    o[t] = mfma32(vop[t][s2], pv[s2], o[t]);
                } else {
                    o[t] = mfma32(*reinterpret_cast<const h8*>(vrow + 32 * s2), pv[s2], o[t]);
                }
            }
        }
    };
    const auto run_unit = [&](const u4 (&qc)[QT][NS]) __attribute__((always_inline)) {
        u4 qn[QPRE ? NS : 1];  // the next tile's q, loaded while this tile computes
        for (uint32_t t = 0; w0 + WAVES * t < n_mq; ++t) {
            const uint32_t tq = w0 + WAVES * t;
            const uint32_t my_q = 32 * tq + qi;
            // The first QT tiles' q came with the staging; later ones were
            // loaded during the tile before (QPRE) or load here.
            if (t < QT) {
#pragma unroll
                for (uint32_t tt = 0; tt < QT; ++tt) {
                    if (tt == t) {
#pragma unroll
                        for (int st = 0; st < NS; ++st) {
                            qv[st] = as_h8(qc[tt][st]);
                        }
                    }
                }
            } else if constexpr (QPRE) {
#pragma unroll
                for (int st = 0; st < NS; ++st) {
                    qv[st] = as_h8(qn[st]);
                }
            } else {
#pragma unroll
                for (int st = 0; st < NS; ++st) {
                    const uint32_t d0 = H * (HD / 2) + 8 * st;
                    qv[st] = as_h8(buffer_load16(U.q_res, my_q < n && d0 < hd ? (my_q * a.q_row + U.h * hd + d0) * 2
                                                                              : buffer_oob));
                }
            }
            if constexpr (QPRE) {
                const uint32_t my_q1 = my_q + 32 * WAVES;
#pragma unroll
                for (int st = 0; st < NS; ++st) {
                    const uint32_t d0 = H * (HD / 2) + 8 * st;
                    qn[st] = buffer_load16(U.q_res, tq + WAVES < n_mq && my_q1 < n && d0 < hd
                                                        ? (my_q1 * a.q_row + U.h * hd + d0) * 2
                                                        : buffer_oob);
                }
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
            // The first step apart (first_softmax), then the rest.
            uint32_t t0;
            if (np >= 64) {
                step.template operator()<2, true>(0);
                t0 = 64;
            } else {
                step.template operator()<1, true>(0);
                t0 = np;
            }
            for (; t0 + 64 <= np; t0 += 64) {
                step.template operator()<2, false>(t0);
            }
            if (t0 < np) {
                step.template operator()<1, false>(t0);
            }
            if (my_q < n) {
                const float inv = 1.0f / l_run;
                float* out = a.out + (U.row_base + my_q) * a.q_row + U.h * hd;
                // Register i of tile t holds dim 32t + 8(i/4) + 4H + i%4.
#pragma unroll
                for (int t = 0; t < NT; ++t) {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const uint32_t d = 32 * t + 8 * b + 4 * H;
                        if (d < hd) {
                            *reinterpret_cast<f4*>(out + d) = f4{o[t][4 * b] * inv, o[t][4 * b + 1] * inv,
                                                                 o[t][4 * b + 2] * inv, o[t][4 * b + 3] * inv};
                        }
                    }
                }
            }
        }
    };

    // ---- the tail rows on the vector units, all four waves ----
    // Per row: the block scores the keys into s_lds (thread t keys t,
    // t + 256, ...; f32 sums of binary16 products over the dims in order).
    // Every wave then takes the softmax whole over all keys (max, sum,
    // p = e / sum, kept in f32; the waves compute the same values), and wave
    // v writes back the p of the 64-key blocks u with u % 4 == v. Wave v sums
    // output dims 64 c + 16 v + l % 16: each 16-lane row of the wave takes a
    // quarter of the keys (8 partial sums by key mod 8, added in order), and
    // the four quarters are added across the rows.
    const auto tail_rows = [&](u4 tq) __attribute__((always_inline)) {
        const uint32_t r0 = 32 * n_mq;
        const uint32_t rows = n - r0;
        char* ltail = U.lv + HD * vrowc * 16;
        _Float16* q_lds = reinterpret_cast<_Float16*>(ltail);                        // [tail rows][HD]
        float* s_lds = reinterpret_cast<float*>(ltail + resident_tail_rows * HD * 2);  // [np]
        const uint32_t wv = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(tid >> 6));
        if (static_cast<uint32_t>(tid) < rows * KCPR) {  // wave 0's lanes: rows * KCPR <= 32
            *reinterpret_cast<u4*>(q_lds + (tid / KCPR) * HD + 8 * (tid % KCPR)) = tq;
        }
        lds_barrier();
        constexpr uint32_t KPL = (NPMAX + 63) / 64;            // keys per lane in a wave, at most
        constexpr uint32_t KPB = (NPMAX + THREADS - 1) / THREADS;  // keys per thread in the block
        typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
        const uint32_t quarter = np / 4;  // a multiple of 8
        const uint32_t kg = static_cast<uint32_t>(ln) >> 4;
        for (uint32_t i = 0; i < rows; ++i) {
            h8 qr[KCPR];
#pragma unroll
            for (int ch = 0; ch < KCPR; ++ch) {
                qr[ch] = *reinterpret_cast<const h8*>(q_lds + i * HD + 8 * ch);
            }
            // Chunk-major over the thread's keys, so each chunk's reads of
            // all its keys are in flight together. Rows n..np-1 are zero
            // rows; threads past np read the last one and store nothing.
            float sj[KPB];
#pragma unroll
            for (uint32_t u = 0; u < KPB; ++u) {
                sj[u] = 0.0f;
            }
#pragma unroll
            for (int ch = 0; ch < KCPR; ++ch) {
                h8 kk[KPB];
#pragma unroll
                for (uint32_t u = 0; u < KPB; ++u) {
                    kk[u] = *reinterpret_cast<const h8*>(U.lk + (min(tid + THREADS * u, np - 1) * KROWC + ch) * 16);
                }
#pragma unroll
                for (uint32_t u = 0; u < KPB; ++u) {
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        sj[u] = __builtin_amdgcn_fdot2(__builtin_bit_cast(fp16x2, h2{qr[ch][e], qr[ch][e + 1]}),
                                                       __builtin_bit_cast(fp16x2, h2{kk[u][e], kk[u][e + 1]}), sj[u],
                                                       false);
                    }
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < KPB; ++u) {
                const uint32_t j = tid + THREADS * u;
                if (j < np) {
                    s_lds[j] = sj[u];
                }
            }
            lds_barrier();
            float ej[KPL];
            float mx = -INFINITY;
#pragma unroll
            for (uint32_t u = 0; u < KPL; ++u) {
                const uint32_t j = ln + 64 * u;
                ej[u] = j < n ? s_lds[j] : -INFINITY;
                mx = fmaxf(mx, ej[u]);
            }
            mx = wave_reduce_max(mx);
            float sum = 0.0f;
#pragma unroll
            for (uint32_t u = 0; u < KPL; ++u) {
                ej[u] = fast_exp2((ej[u] - mx) * c);  // 0 past n
                sum += ej[u];
            }
            sum = wave_reduce_sum(sum);
            const float inv = 1.0f / sum;
            lds_barrier();  // every wave has read the scores
#pragma unroll
            for (uint32_t u = 0; u < KPL; ++u) {
                const uint32_t j = ln + 64 * u;
                if (u % WAVES == wv && j < np) {
                    s_lds[j] = ej[u] * inv;
                }
            }
            lds_barrier();
            float* out = a.out + (U.row_base + r0 + i) * a.q_row + U.h * hd;
#pragma unroll
            for (uint32_t d0 = 0; d0 < HD; d0 += 64) {
                const uint32_t d = d0 + 16 * wv + (ln & 15);
                float r = 0.0f;
                if (d < hd) {
                    // V^T row d: keys 0..np-1 in order (zeros past n).
                    const char* vrow = U.lv + d * vrowc * 16;
                    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
                    const uint32_t jb = kg * quarter;
#pragma unroll 3
                    for (uint32_t j8 = 0; j8 < quarter; j8 += 8) {
                        const h8 vv = *reinterpret_cast<const h8*>(vrow + 2 * (jb + j8));
                        const f4 p0 = *reinterpret_cast<const f4*>(s_lds + jb + j8);
                        const f4 p1 = *reinterpret_cast<const f4*>(s_lds + jb + j8 + 4);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            acc[e] = fmaf(p0[e], static_cast<float>(vv[e]), acc[e]);
                            acc[4 + e] = fmaf(p1[e], static_cast<float>(vv[4 + e]), acc[4 + e]);
                        }
                    }
                    r = acc[0];
#pragma unroll
                    for (int e = 1; e < 8; ++e) {
                        r += acc[e];
                    }
                }
                r = sum32(sum16(r));  // quarters (0 + 1) + (2 + 3)
                if (kg == 0 && d < hd) {
                    out[d] = r;
                }
            }
            if (i + 1 < rows) {
                lds_barrier();  // the next row rewrites s_lds
            }
        }
    };

    u4 kc[KC], vc[VC][2], qc[QT][NS], tq;
    if (blockIdx.x >= st.from && blockIdx.x < st.to) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__builtin_amdgcn_s_memrealtime() - t0 < st.ticks) {
            __builtin_amdgcn_s_sleep(2);
        }
    }
    load_unit(kc, vc, qc, tq);
    store_unit(kc, vc);
    lds_barrier();
    run_unit(qc);
    if (tail) {
        tail_rows(tq);
    }
}

// f16 rows only: f32 rows of images this short take the f32 kernel
// (generic.hip), which keeps the reference's f32 arithmetic.
template <int HD>
hipError_t launch_resident(const flash_args& a, hipStream_t stream) {
    const dim3 grid(a.n_heads * a.batch);
    resident_stagger st{0, 0, 0};
    const uint32_t cus = device_cu_count();
    if (cus > 0 && grid.x > cus) {
        // A unit's staged bytes: its K, V and q rows in binary16.
        const double bytes = 3.0 * a.n * a.hd * 2;
        st = {cus, std::min(grid.x, 2 * cus), static_cast<uint32_t>(bytes * cus / 8e12 * 1e8)};
    }
    resident_kernel<HD><<<grid, 256, resident_unit_bytes(a.n, HD), stream>>>(a, st);
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
        if (resident_unit_bytes(a.n, hdp) <= resident_lds_limit) {
            switch (hdp) {
            case 32:
                return launch_resident<32>(a, stream);
            case 64:
                return launch_resident<64>(a, stream);
            case 96:
                return launch_resident<96>(a, stream);
            default:
                return launch_resident<128>(a, stream);
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
