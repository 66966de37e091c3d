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
// (one 16-byte load per lane and k-step; the score contraction visits the
// dims in the order 32*st + 8*G, so one load instruction reads 64
// contiguous bytes of each of its 16 rows), and the S^T tiles are laid out so
// their accumulator registers ARE the P operand of the second product: the
// position order inside a tile is permuted so that lane group G holds the 8
// consecutive positions 8G..8G+7 of the block. No LDS, no shuffles on the
// path from K to O. Softmax is online (running max and sum per head), q is
// rounded to f16 as the reference rounds it (:204-206), and p is rounded to
// f16 as the reference rounds it (:225-227) -- before normalisation here,
// which the online form needs.
//
// The 4 waves merge their (max, sum, O) through LDS. A sequence with more
// than one split then needs its splits combined: each block writes its
// unnormalised partial (max, sum, O) to scratch, and a second small kernel on
// the same stream merges them, one block per (sequence, query head). The
// kernel boundary is what makes the partials visible. Merging inside this
// kernel was built and measured slower: the partials must be stored
// write-through or read with agent-scope loads (plain loads on another CU
// never see them), and the handoff -- store acknowledged, arrival counter,
// poll, partial loads -- costs three or four loaded memory round trips,
// more than the second launch. The merge needs no LDS and no barrier: each
// wave of a merge block owns a quarter of the head's output and turns all
// the splits' (max, sum) into weights itself (wave-wide max and sum by DPP
// and permlane swaps), then streams the partial outputs with independent
// 16-byte loads. Each output sums its splits in a fixed order, so results
// are deterministic.
//
// A single-token step passes its new K, V row (k_new, v_new). The waves'
// steps cover the cached rows only; the block of the last split also rounds
// the new row to binary16, stores it into the cache and attends it as a
// fifth partial of its 4-wave merge (its score computed while the K, V loads
// are in flight), so there is no separate append launch and the row never
// makes a split of its own: config 2's 4096 cached rows are 32 splits per KV
// head, 256 blocks, one per CU. (As its own one-row split the grid was 264
// blocks, and the 8 CUs holding two blocks finished 1-1.5 us after the rest.)

#include "kernels.hpp"

namespace syn {

#ifdef SYN_DECODE_STAMPS
// Timing build only (python -m synapse_amd.build --stamps): every wave of the
// split kernel's first decode_stamp_blocks blocks keeps s_memrealtime stamps
// (100 MHz, one clock for the whole device) at decode_stamp_points phase
// points; every merge block its entry and end. Block 0 of a split launch
// first copies the previous launch's merge stamps aside, so one read after a
// run of steps shows a whole step: previous merge, split, merge.
constexpr uint32_t decode_stamp_blocks = 512;
constexpr uint32_t decode_stamp_points = 12;
constexpr uint32_t decode_stamp_merges = 64;
__device__ unsigned long long decode_stamp_split[decode_stamp_blocks * 4 * decode_stamp_points];
__device__ unsigned long long decode_stamp_merge[decode_stamp_merges * 2];
__device__ unsigned long long decode_stamp_prev[decode_stamp_merges * 2];
#define DECODE_STAMP(k) stamp_[k] = __builtin_amdgcn_s_memrealtime()
#else
#define DECODE_STAMP(k) (void)0
#endif

namespace {

// The sequence a block belongs to: starts[] is non-decreasing, and sequence
// i owns blocks [starts[i], starts[i+1]). All loads are independent, so they
// go out as one batch.
__device__ __forceinline__ uint32_t find_seq(const uint32_t* starts, uint32_t n, uint32_t x) {
    uint32_t si = 0;
#pragma unroll
    for (uint32_t i = 1; i < decode_max_seqs; ++i) {
        si += (i < n && x >= starts[i]) ? 1u : 0u;
    }
    return si;
}

// One sequence per launch (a decode step) or a table of them (ragged batch):
// the kernels see either through these.
template <class A>
struct decode_traits;
template <>
struct decode_traits<decode_one_args> {
    static constexpr bool multi = false;
    __host__ __device__ static const decode_seq& seq(const decode_one_args& a, uint32_t) { return a.s; }
    __device__ static uint32_t find(const decode_one_args&, uint32_t) { return 0; }
    __device__ static uint32_t find_merge(const decode_one_args&, uint32_t) { return 0; }
};
template <>
struct decode_traits<decode_rope_args> {
    static constexpr bool multi = false;
    __host__ __device__ static const decode_seq& seq(const decode_rope_args& a, uint32_t) { return a.s; }
    __device__ static uint32_t find(const decode_rope_args&, uint32_t) { return 0; }
    __device__ static uint32_t find_merge(const decode_rope_args&, uint32_t) { return 0; }
};
template <>
struct decode_traits<decode_batch_args> {
    static constexpr bool multi = true;
    __host__ __device__ static const decode_seq& seq(const decode_batch_args& a, uint32_t i) { return a.seq[i]; }
    __device__ static uint32_t find(const decode_batch_args& a, uint32_t sb) {
        return find_seq(a.block0s, a.p.n_seqs, sb);
    }
    __device__ static uint32_t find_merge(const decode_batch_args& a, uint32_t u) {
        return find_seq(a.merge0s, a.p.n_seqs, u);
    }
};

// LDS of the split kernel: the group's q as given (f32 size, the larger),
// the new K and V row of one head (likewise), per-wave (max, sum), the
// waves' unscaled outputs (head rows padded by 4 floats), then a fused
// step's RoPE table (hd/2 cos, hd/2 sin), frequency factors (a 1 KB copy)
// and the pairs' angles.
inline __host__ __device__ uint32_t q_lds_bytes(uint32_t group, uint32_t hd) {
    return (group * hd * 4 + 15) / 16 * 16;
}
inline __host__ __device__ uint32_t new_lds_bytes(uint32_t hd) {
    return (2 * hd * 4 + 15) / 16 * 16;
}
// (max, sum) slots: 4 waves and the new row, 16 heads each; then the 4
// waves' parts of the new row's scores, 16 heads each.
constexpr uint32_t decode_ml_floats = 5 * 16 * 2 + 4 * 16;
inline __host__ __device__ uint32_t rope_lds_offset(uint32_t group, uint32_t hd) {
    return q_lds_bytes(group, hd) + new_lds_bytes(hd) + (decode_ml_floats + 4 * group * (hd + 4)) * 4;
}
inline std::size_t decode_lds_bytes(uint32_t group, uint32_t hd) {
    return rope_lds_offset(group, hd) + std::size_t{hd} * sizeof(float) + 1024 + rope_max_pairs * sizeof(float);
}

// s_waitcnt immediate that waits until at most n vector memory operations
// are outstanding (gfx9 encoding: vmcnt split over bits 3:0 and 15:14;
// expcnt and lgkmcnt left at their no-wait maxima).
constexpr int vmcnt_imm(int n) {
    return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

// The fused step's RoPE fields (other launches have none and never use them).
template <class A>
__device__ __forceinline__ const rope_params& a_rope(const A& a) {
    if constexpr (std::is_same_v<A, decode_rope_args>) {
        return a.r;
    } else {
        __builtin_unreachable();
    }
}

// SHORT: some sequence of the launch has at most decode_chunk_unit rows and
// takes the whole-softmax path below; launches without one compile it out
// (it costs the online path about 60 registers).
template <int HDP, bool QF16, bool SHORT, class A>
__global__ __launch_bounds__(256, SHORT && HDP <= 128 ? 2 : 1) void decode_kernel(const A a) {
    using T = decode_traits<A>;
    constexpr bool MULTI = T::multi;
    constexpr bool ROPE = std::is_same_v<A, decode_rope_args>;
    static_assert(!(ROPE && QF16), "a fused RoPE step takes f32 q");
    const decode_params& p = a.p;
    constexpr int NS = HDP / 32;   // k-steps of the score product
    constexpr int NT = HDP / 16;   // 16-dim tiles of the output

#ifdef SYN_DECODE_STAMPS
    unsigned long long stamp_[decode_stamp_points] = {};
    if (blockIdx.x == 0 && threadIdx.x < 64) {
        for (uint32_t i = threadIdx.x; i < decode_stamp_merges * 2; i += 64) {
            decode_stamp_prev[i] = decode_stamp_merge[i];
        }
    }
#endif
    DECODE_STAMP(0);
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int ln = tid & 63;
    const int G = ln >> 4;  // lane group
    const int r = ln & 15;  // row / column inside the group
    const uint32_t hd = p.hd;
    const uint32_t group = p.group;

    // Block -> (sequence, split, KV head). Splits of one KV head are n_kv
    // blocks apart, so with n_kv a multiple of 8 they share an XCD (and its L2).
    // A sequence's splits go out last first: the last split is the short one
    // and holds the step's new row, and blocks dispatched last get their
    // loads served last, so it must not be among them (measured: 0.9 us per
    // config-2 step). Partials sit at the split's own slot.
    const uint32_t b = blockIdx.x;
    const uint32_t g = b % p.n_kv;
    const uint32_t sb = b / p.n_kv;
    const uint32_t si = T::find(a, sb);
    const decode_seq& s = T::seq(a, si);
    const uint32_t split = s.n_splits - 1 - (sb - s.block0);
    const std::size_t slot = static_cast<std::size_t>(s.block0 + split) * p.n_kv + g;
    // The waves attend the split's cached rows [t_begin, t_end); a step's
    // new row (position len - 1, from k_new / v_new) is not among them: the
    // last split's block attends it apart (new_here).
    // The arguments the K, V loads need, materialised here: the compiler
    // otherwise fetches them after the q copy below, a second dependent
    // round trip to the kernel arguments (about half a microsecond) before
    // any wave's first K, V load.
    asm volatile("" : : "s"(s.len), "s"(s.n_splits), "s"(s.ctx_stride), "s"(p.scale_log2e));
    DECODE_STAMP(9);
    const uint32_t cached = s.len - (s.k_new != nullptr ? 1u : 0u);
    const uint32_t t_begin = split * p.chunk;
    const uint32_t t_end = min(cached, t_begin + p.chunk);
    const uint32_t h0 = g * group;
    const float c = p.scale_log2e;
    const uint32_t new_t = s.len - 1;
    const bool new_here = s.k_new != nullptr && split == s.n_splits - 1;
    const bool kv_f16 = !ROPE && p.kv_dtype == 1;  // a fused RoPE step takes f32 rows

    // Every K, V load below is unconditional, so a wave issues all of them
    // back to back: a lane with nothing to read points at valid data and
    // zeroes what it got afterwards.
    //
    // The group's q rows are copied once per block into LDS, 1 KB per wave
    // instruction, straight from global memory (no registers): every wave of
    // every split reading q itself would pile thousands of requests onto the
    // same few lines.
    extern __shared__ __attribute__((aligned(16))) char lds_bytes[];
    const uint32_t q_bytes = group * hd * (QF16 ? 2 : 4);
    const char* q_src = static_cast<const char*>(s.q) + static_cast<std::size_t>(h0) * hd * (QF16 ? 2 : 4);
    for (uint32_t c0 = 1024 * w; c0 < q_bytes; c0 += 4096) {
        // q_bytes is a multiple of 16; a lane past its end re-reads chunk 0.
        const uint32_t off = c0 + 16 * ln < q_bytes ? c0 + 16 * ln : 0;
        load16_lds(q_src + off, lds_bytes + c0);
    }
    // The block holding the step's new row stages that row of KV head g the
    // same way (K then V, as given), for the step that appends it.
    char* new_lds = lds_bytes + q_lds_bytes(group, hd);
    const uint32_t new_bytes = hd * (kv_f16 ? 2 : 4);
    // Dims d .. d + 7 (K) or d .. d + 3 (V) of the new row from its LDS
    // copy, rounded to binary16 as the cache stores them; d is a multiple of
    // 8 (4), so each is one or two vector reads.
    const auto new_k8 = [&](uint32_t d) -> h8 {
        if (kv_f16) {
            return *reinterpret_cast<const h8*>(new_lds + 2 * d);
        }
        const f4 lo = *reinterpret_cast<const f4*>(new_lds + 4 * d);
        const f4 hi = *reinterpret_cast<const f4*>(new_lds + 4 * d + 16);
        return h8{to_h(lo[0]), to_h(lo[1]), to_h(lo[2]), to_h(lo[3]), to_h(hi[0]), to_h(hi[1]), to_h(hi[2]), to_h(hi[3])};
    };
    const auto new_v4 = [&](uint32_t d) -> f4 {
        if (kv_f16) {
            const h4 x = *reinterpret_cast<const h4*>(new_lds + new_bytes + 2 * d);
            return f4{static_cast<float>(x[0]), static_cast<float>(x[1]), static_cast<float>(x[2]),
                      static_cast<float>(x[3])};
        }
        const f4 x = *reinterpret_cast<const f4*>(new_lds + new_bytes + 4 * d);
        return f4{static_cast<float>(to_h(x[0])), static_cast<float>(to_h(x[1])), static_cast<float>(to_h(x[2])),
                  static_cast<float>(to_h(x[3]))};
    };
    if (new_here) {
        const std::size_t row_off = static_cast<std::size_t>(g) * new_bytes;
        for (uint32_t c0 = 1024 * w; c0 < 2 * new_bytes; c0 += 4096) {
            const uint32_t c = c0 + 16 * ln < 2 * new_bytes ? c0 + 16 * ln : 0;
            const char* src = c < new_bytes ? static_cast<const char*>(s.k_new) + row_off + c
                                            : static_cast<const char*>(s.v_new) + row_off + (c - new_bytes);
            load16_lds(src, new_lds + c0);
        }
    }

    // K rows for the two S^T tiles: row r of tile e is position
    // tb + 8*(r/4) + 4*e + r%4, so accumulator row 4G+i of tile e is position
    // tb + 8G + 4e + i. V^T rows: lane (G, r) of tile n holds dim 16n + r at
    // positions tb + 8G + [0, 8). Both through buffer resources based at the
    // split: K past the split and dims past the head read as zeros.
    const uint32_t row2 = p.row * 2;
    const uint32_t vstride2 = s.ctx_stride * 2;
    // k_rows counts the split's rows. K past them reads zeros through the
    // resource's limit; V columns that start at or past them take an
    // out-of-range offset (zeros, no request). The new row's cache slot is
    // never read: the step writes it.
    // (readfirstlane: without it the batched kernel cannot tell the limit is
    // uniform and wraps every K load in a loop over lanes.)
    const uint32_t k_rows = __builtin_amdgcn_readfirstlane(t_end - t_begin);
    const rsrc k_res = make_rsrc(s.k + static_cast<std::size_t>(t_begin) * p.row + g * hd,
                                 k_rows ? k_rows * row2 - g * hd * 2 : 0u);
    const rsrc v_res = make_rsrc(s.vt + static_cast<std::size_t>(g) * hd * s.ctx_stride + t_begin,
                                 hd * vstride2 - t_begin * 2);
    const auto load_kv = [&](uint32_t tb, u4 (&kr)[2][NS], u4 (&vr)[NT]) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t rel = tb - t_begin + 8 * (r >> 2) + 4 * e + (r & 3);
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const uint32_t d0 = 8 * G + 32 * st;
                kr[e][st] = buffer_load16(k_res, d0 < hd ? rel * row2 + d0 * 2 : buffer_oob);
            }
        }
        const uint32_t rel_t = tb - t_begin + 8 * G;
        const uint32_t rel_v = rel_t < k_rows ? rel_t * 2 : buffer_oob;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const uint32_t dim = 16 * n + r;
            vr[n] = buffer_load16(v_res, dim < hd ? dim * vstride2 + rel_v : buffer_oob);
        }
    };

    float m_run = -INFINITY;  // running max of raw q.k for head r
    float l_run = 0.0f;       // running sum of f16-rounded p for head r
    f4 o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        o[n] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // q^T operand: lane (G, r) holds head h0 + r, dims 32*st + 8*G + [0, 8),
    // rounded to binary16 as attend_group rounds q (S/kernels/attention.hpp:204-206).
    h8 qv[NS];
    // A fused RoPE step rotates the q rows and the new K row in LDS, once per
    // block, after they have landed: wave 0 has built every pair's cos and
    // sin into a table (here, when frequency factors had to land first),
    // then the pairs of every row are rotated in place
    // (q also times the temperature factor), and the staging below reads the
    // rotated f32 rows as it reads unrotated ones.
    float* rope_tab = reinterpret_cast<float*>(lds_bytes + rope_lds_offset(group, hd));
    char* ff_lds = lds_bytes + rope_lds_offset(group, hd) + hd * 4;
    float* rope_th = reinterpret_cast<float*>(ff_lds + 1024);  // the pairs' angles
    const auto rope_rows = [&]() {
        const uint32_t half = hd / 2;
        if (w == 0 && a_rope(a).freq_factors != nullptr) {  // (without factors: built before the loads)
            rope_table(a_rope(a), rope_th, half, reinterpret_cast<const float*>(ff_lds), rope_tab,
                       static_cast<uint32_t>(ln));
        }
        DECODE_STAMP(10);
        lds_barrier();
        const bool normal = a_rope(a).mode == 0;
        const float q_scale = a_rope(a).temp_floor_len != 0
                                  ? attn_temperature(new_t, a_rope(a).temp_scale, a_rope(a).temp_floor_len)
                                  : 1.0f;
        const uint32_t rows = group + (new_here ? 1u : 0u);  // q heads, then the new K row
        for (uint32_t u = tid; u < rows * half; u += 256) {
            const uint32_t row = u / half;
            const uint32_t pr = u % half;
            float* x = row < group ? reinterpret_cast<float*>(lds_bytes) + row * hd : reinterpret_cast<float*>(new_lds);
            const float f = row < group ? q_scale : 1.0f;
            const uint32_t i0 = normal ? 2 * pr : pr;
            const uint32_t i1 = normal ? i0 + 1 : pr + half;
            const float cs = rope_tab[pr], sn = rope_tab[half + pr];
            const float x0 = x[i0], x1 = x[i1];
            x[i0] = rope_first(x0, x1, cs, sn) * f;
            x[i1] = rope_second(x0, x1, cs, sn) * f;
        }
        DECODE_STAMP(11);
    };
    const auto convert_q = [&](bool kv_issued) {
        // Wait for this wave's copies (q, the new row) only: the K, V loads
        // issued after them stay in flight. A wave with no positions issued
        // none, so it waits for everything it has. Every wave has waited for
        // its own copies, so the barrier needs no more than the LDS counter
        // (__syncthreads() would also wait for the K, V loads). A batched
        // launch waits for its first K, V too: it runs many blocks per CU,
        // which hide the wait, and the schedule the early q then allows needs
        // more registers than two waves per SIMD leave.
        if (kv_issued && !MULTI) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * NS + NT));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        if constexpr (ROPE) {
            rope_rows();
        }
        lds_barrier();
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const uint32_t d0 = 8 * G + 32 * st;
            const uint32_t e0 = static_cast<uint32_t>(r) * hd + d0;
            if (static_cast<uint32_t>(r) < group && d0 < hd) {
                if constexpr (QF16) {
                    qv[st] = *reinterpret_cast<const h8*>(lds_bytes + 2 * e0);
                } else {
                    const f4 lo = *reinterpret_cast<const f4*>(lds_bytes + 4 * e0);
                    const f4 hi = *reinterpret_cast<const f4*>(lds_bytes + 4 * e0 + 16);
                    qv[st] = h8{to_h(lo[0]), to_h(lo[1]), to_h(lo[2]), to_h(lo[3]),
                                to_h(hi[0]), to_h(hi[1]), to_h(hi[2]), to_h(hi[3])};
                }
            } else {
                qv[st] = as_h8(zero_u4());
            }
        }
    };

    // scores: raw q.k of head r at positions tv + 4e + i in sc[e][i], -inf
    // past the split end; returns their max over the wave's 32 positions.
    const auto scores = [&](uint32_t tv, u4 (&kr)[2][NS], f4 (&sc)[2]) {
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
        return max32(max16(bm));
    };
    // accumulate: O^T += V^T . P^T for the step's probabilities pa.
    const auto accumulate = [&](uint32_t tv, u4 (&vr)[NT], h8 pa) {
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
        // O^T (16 dims x 16 heads) += V^T (16 dims x 32 positions) . P^T: the
        // V^T rows and the score registers are the operands as they stand.
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            o[n] = mfma16(as_h8(vr[n]), pa, o[n]);
        }
    };

    // One online-softmax step: p = exp(s - running max) rounded to f16. The
    // running max is lazy: a head's max is raised only when the step's rises
    // more than 8 above it in the exp2 domain (its p then stay below 2^8,
    // which binary16 holds), and only then are its sum and O rescaled --
    // never on a wave's first step, whose O is still zero. O lives in the
    // accumulation registers: rescaled on every step, all of it was read out
    // and written back each time.
    bool o_zero = true;
    const auto step = [&](uint32_t tb, u4 (&kr)[2][NS], u4 (&vr)[NT]) {
        const uint32_t tv = tb + 8 * G;
        f4 sc[2];
        const float bm = scores(tv, kr, sc);
        DECODE_STAMP(3);
        const bool grow = (bm - m_run) * c > 8.0f;  // false for bm = -inf
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float alpha = grow ? fast_exp2((m_run - bm) * c) : 1.0f;  // 0 from m_run = -inf
            m_run = grow ? bm : m_run;
            l_run *= alpha;
            if (!o_zero) {
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    o[n] *= alpha;
                }
            }
        }
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
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
        l_run += sum32(sum16(ps));
        DECODE_STAMP(4);
        accumulate(tv, vr, pa);
        o_zero = false;
        DECODE_STAMP(5);
    };

    // The wave's first K, V loads go out with q's; later steps load their
    // 32 positions at the top of the step.
    constexpr uint32_t stride = decode_positions_per_wave * decode_waves;
    u4 kr[2][NS], vr[NT];
    uint32_t tb = t_begin + decode_positions_per_wave * w;
    if constexpr (ROPE) {
        // A fused step's frequency factors (hd/2 floats, at most 512 bytes)
        // land in LDS with q, in wave 0's copy, which builds the table: its
        // wait for q covers them. Lanes past the end re-read byte 0 into the
        // area's slack.
        if (w == 0 && a.r.freq_factors != nullptr) {
            const uint32_t off = 16 * ln < 2 * hd ? 16 * ln : 0;
            load16_lds(reinterpret_cast<const char*>(a.r.freq_factors) + off, ff_lds);
        }
    }
    if constexpr (ROPE) {
        // The angles need neither q nor the factors, and without factors
        // neither does the cos / sin table: wave 0 builds them before its
        // K, V loads go out. (After the loads, the chain and the table took
        // wave 0 ~1.2 us past the moment q had landed, on every block's
        // critical path: a wave's loads take ~1.5 us to issue, and the
        // other waves waited at the barrier for the table.) With factors
        // the table waits for their copy, with q.
        if (w == 0) {
            if (ln == 0) {
                rope_angles(new_t, a.r.theta_scale, hd / 2, rope_th);
            }
            if (a.r.freq_factors == nullptr) {
                rope_table(a.r, rope_th, hd / 2, static_cast<const float*>(nullptr), rope_tab,
                           static_cast<uint32_t>(ln));
            }
        }
    }
    // A fused RoPE step loads unconditionally: a wave with no positions
    // reads past the resources' limits and gets zeros without memory
    // traffic. (Guarded, the results met zero-initialised registers at the
    // join, the compiler moved each as soon as it landed, waiting for it
    // between the loads.)
    if (ROPE || tb < t_end) {
        load_kv(tb, kr, vr);
    }
    DECODE_STAMP(1);
    convert_q(ROPE || tb < t_end);
    DECODE_STAMP(2);
    float* lds_ml = reinterpret_cast<float*>(lds_bytes + q_lds_bytes(group, hd) + new_lds_bytes(hd));
    // The new row, from its LDS copy (rotated there by a fused RoPE step),
    // while the K, V loads are in flight: wave w takes the
    // part of its raw score q.k over the dims of k-step w (mod 4) for every
    // head of the group, and the merge adds the 4 parts in wave order. As a
    // split of one row it has p = 1 at its own max: the fifth (max, sum)
    // slot is (score, 1). (One wave taking the whole score held its own
    // step, and the block, back by 0.5 us.)
    float* lds_snew = lds_ml + 5 * 16 * 2;
    const auto new_score = [&](uint32_t h) {
        return ((lds_snew[h] + lds_snew[16 + h]) + lds_snew[32 + h]) + lds_snew[48 + h];
    };
    if (new_here) {
        // Lane (G, r) holds head r's q at dims 32 st + 8 G + [0, 8): the
        // products of two binary16 values are exact in f32, summed in f32
        // over the lane's dims, then over the 4 lane groups.
        float part = 0.0f;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const uint32_t d0 = 8 * G + 32 * st;
            if (st % 4 == w && d0 < hd) {
                const h8 kn = new_k8(d0);
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) {
                    part = fmaf(static_cast<float>(qv[st][j]), static_cast<float>(kn[j]), part);
                }
            }
        }
        part = sum32(sum16(part));
        if (G == 0) {
            lds_snew[16 * w + r] = part;
        }
    }
    // A sequence of at most 128 rows is one split in which every wave takes
    // at most one step. Its softmax is then taken whole, as attend_group
    // takes it (S/kernels/attention.hpp:222-227): max and sum over all the
    // sequence's positions first (exchanged through LDS), then
    // p = exp(s - max) * (1 / sum) rounded to binary16, so the rounding falls
    // on the normalised probability, as the reference's does, and O needs no
    // final division. Longer sequences round the unnormalised p of the
    // online softmax and divide at the end.
    const bool whole = SHORT && s.len <= decode_chunk_unit;
    if (whole) {
        const bool have = tb < t_end;  // wave-uniform
        const uint32_t tv = tb + 8 * G;
        f4 sc[2];
        float bm = -INFINITY;
        if (have) {
            bm = scores(tv, kr, sc);
        } else {
            sc[0] = sc[1] = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        }
        if (G == 0) {
            lds_ml[(w * 16 + r) * 2] = bm;
        }
        lds_barrier();
        float mx = lds_ml[r * 2];
#pragma unroll
        for (int v = 1; v < 4; ++v) {
            mx = fmaxf(mx, lds_ml[(v * 16 + r) * 2]);
        }
        const float s_new = new_here ? new_score(r) : -INFINITY;
        mx = fmaxf(mx, s_new);
        const float m_use = mx == -INFINITY ? 0.0f : mx;
        float ex[8];
        float es = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ex[4 * e + i] = fast_exp2((sc[e][i] - m_use) * c);  // 0 past the end
                es += ex[4 * e + i];
            }
        }
        es = sum32(sum16(es));
        if (G == 0) {
            lds_ml[(w * 16 + r) * 2 + 1] = es;
        }
        lds_barrier();
        float total = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            total += lds_ml[(v * 16 + r) * 2 + 1];
        }
        const float ex_new = fast_exp2((s_new - m_use) * c);  // 0 without a new row
        total += ex_new;
        const float inv = 1.0f / total;
        // The new row's normalised p, rounded as the others, for the merge
        // below (no wave reads this slot before the barrier there).
        if (new_here && w == 0 && G == 0 && static_cast<uint32_t>(r) < group) {
            lds_ml[(64 + r) * 2 + 1] = static_cast<float>(to_h(ex_new * inv));
        }
        h8 pa;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            pa[j] = to_h(ex[j] * inv);
        }
        if (have) {
            accumulate(tv, vr, pa);
        }
    } else {
        while (tb < t_end) {
            step(tb, kr, vr);
            tb += stride;
            if (tb < t_end) {
                load_kv(tb, kr, vr);
            }
        }
    }

    // ---- merge the 4 waves (one barrier) -----------------------------------------
    // Each wave leaves its per-head (max, sum) and its unscaled O^T in its own
    // LDS slot (head rows padded by 4 floats against bank conflicts); then
    // every thread combines the 4 slots for its output elements. Lane (G, r)
    // holds O^T[16n + 4G + i][head r] in o[n][i]. A whole-softmax sequence's
    // waves hold normalised parts of one sum (and other waves may still be
    // reading the (max, sum) slots), so they write O only.
    const uint32_t orow = hd + 4;
    float* lds_o = lds_ml + decode_ml_floats;
    if (G == 0 && !whole) {
        lds_ml[(w * 16 + r) * 2] = m_run;
        lds_ml[(w * 16 + r) * 2 + 1] = l_run;
    }
    if (static_cast<uint32_t>(r) < group) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const uint32_t d0 = 16 * n + 4 * G;
            if (d0 < hd) {
                *reinterpret_cast<f4*>(lds_o + (w * group + r) * orow + d0) = o[n];
            }
        }
    }
    // LDS only: the block appending the step's row must not wait here for
    // its scattered cache stores, as __syncthreads() would.
    DECODE_STAMP(6);
    lds_barrier();
    DECODE_STAMP(7);

    // Every thread combines the waves for 4 consecutive elements of one head:
    // the output for a sequence of one split, else this split's partial,
    // which the merge kernel reads after the kernel boundary.
    const uint32_t nout = group * hd;
    // The new row into the cache as binary16 (kv_append, S/kernels/
    // attention.hpp:165-175), by the threads the merge below leaves idle
    // (the last wave when it has work for every thread): K 16 bytes per
    // lane, V^T one binary16 per dim, a column. Here its scattered stores
    // delay no load or product of the block.
    if (new_here) {
        const uint32_t t0 = nout / 4 < 256 - 64 ? (nout / 4 + 63) / 64 * 64 : 192;
        for (uint32_t i = tid - t0; tid >= t0 && i < hd / 4; i += 256 - t0) {
            const uint32_t d = 4 * i;
            if (d % 8 == 0) {
                store16(s.k + static_cast<std::size_t>(new_t) * p.row + g * hd + d, as_u4(new_k8(d)));
            }
            const f4 x = new_v4(d);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s.vt[static_cast<std::size_t>(g * hd + d + j) * s.ctx_stride + new_t] = static_cast<_Float16>(x[j]);
            }
        }
    }
    float* part_o = p.part + slot * nout;
    float* part_ml = p.part + static_cast<std::size_t>(p.total_slots) * nout + slot * group * 2;
    for (uint32_t e = 4 * tid; e < nout; e += 4 * 256) {
        const uint32_t h = e / hd;
        const uint32_t d = e % hd;
        // The new row's V at dims d .. d + 3 (binary16 values).
        const f4 vnew = new_here ? new_v4(d) : f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (whole) {
            f4 acc = *reinterpret_cast<const f4*>(lds_o + h * orow + d);
#pragma unroll
            for (int v = 1; v < 4; ++v) {
                acc += *reinterpret_cast<const f4*>(lds_o + (v * group + h) * orow + d);
            }
            if (new_here) {
                acc += lds_ml[(64 + h) * 2 + 1] * vnew;
            }
            *reinterpret_cast<f4*>(s.out + static_cast<std::size_t>(h0) * hd + e) = acc;
            continue;
        }
        float mw[5];
        float mx = -INFINITY;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            mw[v] = lds_ml[(v * 16 + h) * 2];
            mx = fmaxf(mx, mw[v]);
        }
        mw[4] = new_here ? new_score(h) : -INFINITY;
        mx = fmaxf(mx, mw[4]);
        float sum = 0.0f;
        f4 acc{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float f = fast_exp2((mw[v] - mx) * c);  // 0 for a wave with no positions
            sum += lds_ml[(v * 16 + h) * 2 + 1] * f;
            acc += f * *reinterpret_cast<const f4*>(lds_o + (v * group + h) * orow + d);
        }
        if (new_here) {
            const float f = fast_exp2((mw[4] - mx) * c);
            sum += f;
            acc += f * vnew;
        }
        if (s.n_splits == 1) {
            *reinterpret_cast<f4*>(s.out + static_cast<std::size_t>(h0) * hd + e) = acc / sum;
        } else {
            *reinterpret_cast<f4*>(part_o + e) = acc;
            if (d == 0) {
                part_ml[2 * h] = mx;
                part_ml[2 * h + 1] = sum;
            }
        }
    }
#ifdef SYN_DECODE_STAMPS
    DECODE_STAMP(8);
    if (ln == 0 && b < decode_stamp_blocks) {
        for (uint32_t k = 0; k < decode_stamp_points; ++k) {
            decode_stamp_split[(b * 4 + w) * decode_stamp_points + k] = stamp_[k];
        }
    }
#endif
}

// One block per (sequence with splits, query head): out = sum_j w_j O_j with
// w_j = exp2((m_j - max) c) / sum_i l_i exp2((m_i - max) c), splits in a
// fixed order, so results are deterministic.
//
// Every load is unconditional and issued before any is used: lanes with
// nothing to read take an out-of-range buffer offset and get zeros. (Loads
// guarded by a condition into an array were issued one at a time, each
// waited for before the next: eight round trips instead of one.)
template <class A>
__global__ __launch_bounds__(256) void decode_merge_kernel(const A a) {
    using T = decode_traits<A>;
    const decode_params& p = a.p;
#ifdef SYN_DECODE_STAMPS
    unsigned long long stamp_[1];
    DECODE_STAMP(0);
    const unsigned long long entry_ = stamp_[0];
#endif
    const int tid = threadIdx.x;
    const int ln = tid & 63;
    const uint32_t u = blockIdx.x;
    const uint32_t si = T::find_merge(a, u);
    const decode_seq& s = T::seq(a, si);
    // Heads of one KV head go n_kv blocks apart, as the split kernel's
    // blocks do, so with n_kv a multiple of 8 a merge block runs on the XCD
    // whose L2 took its KV head's partials.
    const uint32_t k = u - s.merge0;
    const uint32_t g = k % p.n_kv;
    const uint32_t h = k / p.n_kv;
    const uint32_t hd = p.hd;
    const uint32_t group = p.group;
    const uint32_t nout = group * hd;
    const uint32_t S = s.n_splits;
    const float c = p.scale_log2e;
    // Partials of this (sequence, KV head): split j's O at slot (block0 + j) * n_kv + g.
    const uint32_t o_stride = p.n_kv * nout * 4;   // bytes between consecutive splits' O
    const uint32_t ml_stride = p.n_kv * group * 8;  // and (max, sum) pairs
    const std::size_t slot0 = static_cast<std::size_t>(s.block0) * p.n_kv + g;
    const rsrc o_r = make_rsrc(p.part + slot0 * nout + static_cast<std::size_t>(h) * hd, (S - 1) * o_stride + hd * 4);
    const rsrc ml_r = make_rsrc(p.part + static_cast<std::size_t>(p.total_slots) * nout + (slot0 * group + h) * 2,
                                (S - 1) * ml_stride + 8);
    // Every argument fetched in the first batch of scalar loads (the
    // compiler otherwise fetches these after the first loads, a second
    // dependent round trip).
    asm volatile("" : : "s"(p.total_slots), "s"(c), "s"(s.out));

    // Each wave owns qw of the head's nq output quads and does its whole
    // merge alone, with no barrier: lane (part, quad) sums the splits
    // part, part + pw, ... of its quad in that order, then the pw parts meet
    // in a fixed xor tree of shuffles. Every wave computes the weights
    // itself from all the (max, sum) pairs (at most 256, 4 per lane). The
    // first 8 partial outputs of every lane go out with those loads.
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nq = hd / 4;
    const uint32_t qw = (nq + 3) / 4;
    const uint32_t qwp = qw <= 1 ? 1 : qw <= 2 ? 2 : qw <= 4 ? 4 : qw <= 8 ? 8 : 16;  // a power of two
    const uint32_t pw = 64 / qwp;
    const uint32_t ql = ln % qwp;
    const uint32_t part = ln / qwp;
    const uint32_t quad = w * qw + ql;
    const bool mine = ql < qw && quad < nq;
    const auto o_off = [&](uint32_t j) { return mine && j < S ? j * o_stride + 16 * quad : buffer_oob; };
    f4 ov[8];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        ov[i] = __builtin_bit_cast(f4, buffer_load16(o_r, o_off(part + i * pw)));
    }
    constexpr uint32_t per_lane = decode_max_splits / 64;
    float mj[per_lane], lj[per_lane];
#pragma unroll
    for (uint32_t i = 0; i < per_lane; ++i) {
        const uint32_t j = ln + 64 * i;
        const uint32_t off = j < S ? j * ml_stride : buffer_oob;
        mj[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ml_r, off, 0, 0));
        lj[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ml_r, off == buffer_oob ? off : off + 4, 0, 0));
    }
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t i = 0; i < per_lane; ++i) {
        mj[i] = ln + 64 * i < S ? mj[i] : -INFINITY;
        mx = fmaxf(mx, mj[i]);
    }
    mx = wave_reduce_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < per_lane; ++i) {
        mj[i] = fast_exp2((mj[i] - mx) * c);  // 0 for absent splits
        sum += lj[i] * mj[i];
    }
    sum = wave_reduce_sum(sum);
    const float inv = 1.0f / sum;
#pragma unroll
    for (uint32_t i = 0; i < per_lane; ++i) {
        mj[i] *= inv;  // the weight of split ln + 64 i
    }
    // The weights of splits j0 + i pw + part, j0 a multiple of 8 pw: split j
    // is lane j % 64 of slot j / 64 (uniform: pw divides 64). Every lane
    // takes part in the shuffles, all 8 issued before any is used.
    const auto weights = [&](uint32_t j0, float (&wt)[8]) {
        if (S <= 64) {  // one slot
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) {
                wt[i] = __shfl(mj[0], static_cast<int>((j0 + i * pw + part) % 64), 64);
            }
            return;
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t slot = (j0 + i * pw) / 64;
            const float src = slot == 0 ? mj[0] : slot == 1 ? mj[1] : slot == 2 ? mj[2] : mj[3];
            wt[i] = __shfl(src, static_cast<int>((j0 + i * pw + part) % 64), 64);
        }
    };
    f4 acc{0.0f, 0.0f, 0.0f, 0.0f};
    float wt[8];
    weights(0, wt);
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        acc += wt[i] * ov[i];  // 0 * 0 past the splits
    }
    for (uint32_t j0 = 8 * pw; j0 < S; j0 += 8 * pw) {
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            ov[i] = __builtin_bit_cast(f4, buffer_load16(o_r, o_off(j0 + i * pw + part)));
        }
        weights(j0, wt);
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            acc += wt[i] * ov[i];
        }
    }
    for (uint32_t m = qwp; m < 64; m <<= 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc[e] += __shfl_xor(acc[e], static_cast<int>(m), 64);
        }
    }
    if (part == 0 && mine) {
        *reinterpret_cast<f4*>(s.out + (static_cast<std::size_t>(g) * group + h) * hd + 4 * quad) = acc;
    }
#ifdef SYN_DECODE_STAMPS
    DECODE_STAMP(0);
    if (tid == 0 && u < decode_stamp_merges) {
        decode_stamp_merge[2 * u] = entry_;
        decode_stamp_merge[2 * u + 1] = stamp_[0];
    }
#endif
}

template <int HDP, class A>
hipError_t launch_hdp(const A& a, uint32_t q_dtype, hipStream_t stream) {
    const std::size_t lds = decode_lds_bytes(a.p.group, a.p.hd);
    const dim3 grid(a.p.total_slots);
    bool any_short = false;
    for (uint32_t i = 0; i < a.p.n_seqs; ++i) {
        any_short = any_short || decode_traits<A>::seq(a, i).len <= decode_chunk_unit;
    }
    if constexpr (std::is_same_v<A, decode_rope_args>) {
        if (q_dtype != 0) {
            return hipErrorInvalidValue;
        }
        const auto kernel = any_short ? decode_kernel<HDP, false, true, A> : decode_kernel<HDP, false, false, A>;
        kernel<<<grid, 256, lds, stream>>>(a);
    } else {
        const auto kernel = q_dtype == 1
                                ? (any_short ? decode_kernel<HDP, true, true, A> : decode_kernel<HDP, true, false, A>)
                                : (any_short ? decode_kernel<HDP, false, true, A> : decode_kernel<HDP, false, false, A>);
        kernel<<<grid, 256, lds, stream>>>(a);
    }
    if (a.p.merge_blocks > 0) {
        decode_merge_kernel<A><<<a.p.merge_blocks, 256, 0, stream>>>(a);
    }
    return hipGetLastError();
}

template <class A>
hipError_t launch_any(const A& a, uint32_t q_dtype, hipStream_t stream) {
    switch ((a.p.hd + 31) / 32 * 32) {
    case 32:
        return launch_hdp<32>(a, q_dtype, stream);
    case 64:
        return launch_hdp<64>(a, q_dtype, stream);
    case 96:
        return launch_hdp<96>(a, q_dtype, stream);
    case 128:
        return launch_hdp<128>(a, q_dtype, stream);
    case 160:
        return launch_hdp<160>(a, q_dtype, stream);
    case 192:
        return launch_hdp<192>(a, q_dtype, stream);
    case 224:
        return launch_hdp<224>(a, q_dtype, stream);
    case 256:
        return launch_hdp<256>(a, q_dtype, stream);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace

uint32_t decode_choose_chunk(uint64_t total_positions, uint32_t n_kv, uint32_t max_len) {
    // Enough splits to give every CU about one block of 128 positions per
    // KV-head pass; longer runs take longer chunks, which keeps the partials
    // (and their merge) small against the KV bytes. No sequence
    // may have more than decode_max_splits splits.
    const uint64_t work = total_positions * n_kv;
    uint64_t chunk = decode_chunk_unit;
    while ((chunk < 1024 && work / chunk > 2048) || (uint64_t{max_len} + chunk - 1) / chunk > decode_max_splits) {
        chunk *= 2;
    }
    return static_cast<uint32_t>(chunk);
}

hipError_t launch_decode(const decode_one_args& a, uint32_t q_dtype, hipStream_t stream) {
    return launch_any(a, q_dtype, stream);
}

hipError_t launch_decode(const decode_batch_args& a, uint32_t q_dtype, hipStream_t stream) {
    return launch_any(a, q_dtype, stream);
}

hipError_t launch_decode(const decode_rope_args& a, uint32_t q_dtype, hipStream_t stream) {
    return launch_any(a, q_dtype, stream);
}

}  // namespace syn

#ifdef SYN_DECODE_STAMPS
// The timing build's stamps of the last decode launches, copied to the host
// (synchronous): split[decode_stamp_blocks][4 waves][decode_stamp_points],
// merge[decode_stamp_merges][entry, end] and the previous launch's merge
// stamps in the same layout. 0 = not written.
extern "C" int syn_hip_decode_stamps(unsigned long long* split, unsigned long long* merge,
                                     unsigned long long* prev_merge) {
    hipError_t e = hipMemcpyFromSymbol(split, HIP_SYMBOL(syn::decode_stamp_split), sizeof(syn::decode_stamp_split));
    if (e == hipSuccess) {
        e = hipMemcpyFromSymbol(merge, HIP_SYMBOL(syn::decode_stamp_merge), sizeof(syn::decode_stamp_merge));
    }
    if (e == hipSuccess) {
        e = hipMemcpyFromSymbol(prev_merge, HIP_SYMBOL(syn::decode_stamp_prev), sizeof(syn::decode_stamp_prev));
    }
    return static_cast<int>(e);
}
#endif

