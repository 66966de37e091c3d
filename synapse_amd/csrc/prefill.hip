// prefill.hip — causal attention of a run of n tokens over the KV cache, on
// the f16 matrix cores.
//
// session::execute(op_attention) for tokens at positions pos..pos+n-1
// (S/graph/session.hpp:348-374): token i attends cache rows 0..pos+i with
// attend_group's math (S/kernels/attention.hpp:185-244), the run's own rows
// already appended.
//
// A block (4 waves) owns 128 queries of one head, a wave 32 of them. Key
// tiles of 64 keys pass through LDS in two stages, copied straight from
// global memory (buffer_load ... lds, no registers): while the waves compute
// tile t from one stage, tile t+1's copy is landing in the other. Per 32-key
// slice a wave computes
//   S^T (32 keys x 32 queries) = K (32 x hd) . Q^T          hd/16 MFMA 32x32x16
//   O^T (32 dims x 32 queries) += V^T (32 x 16 keys) . P^T   per 16 keys and 32 dims
// K rows are loaded in a permuted order so the S^T accumulators are, as they
// stand, the P^T operand; a query's scores sit in one lane (two across the
// lane halves), so the row max and sum are in-lane plus one exchange. Only
// tiles that cross a wave's diagonal (or the end) are masked.

#include "kernels.hpp"

namespace syn {

namespace {

constexpr int pf_bq = 128;  // queries per block
constexpr int pf_bk = 64;   // keys per LDS tile

// Key offset (inside a 32-key slice) that S^T accumulator row m holds.
__device__ __forceinline__ int pf_slice_key(int m) {
    return 16 * (m >> 4) + 8 * ((m >> 2) & 1) + 4 * ((m >> 3) & 1) + (m & 3);
}

// s_waitcnt immediate: at most n vector memory operations outstanding
// (vmcnt split over bits 3:0 and 15:14; expcnt, lgkmcnt not waited on).
constexpr int pf_vmcnt(int n) {
    return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}

// Workgroup barrier for the tile pipeline: each wave waits for its own
// copies with s_waitcnt vmcnt before it, so the barrier only needs the LDS
// operations (reads of the stage about to be refilled, the tail fix-up
// writes) complete, and the copy just issued for the other stage stays in
// flight.
__device__ __forceinline__ void pf_barrier() {
    lds_barrier();
}

// One 1 KB tile copy: lane l's 16 bytes at byte `offset` of r land at LDS
// byte address at + 16 l (offsets at or past r's limit land as zeros).
__device__ __forceinline__ void pf_copy(rsrc r, uint32_t at, uint32_t offset) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(offset), "s"(r), "{m0}"(at) : "memory");
}

// v, which the compiler must treat as unknown here: keeps a value computed
// from it next to its use instead of hoisted and held across a loop.
__device__ __forceinline__ uint32_t pf_opaque(uint32_t v) {
    asm volatile("" : "+s"(v));
    return v;
}

// The LDS byte address of a wave's first copy into a stage, in one scalar
// register that the compiler must treat as new on every item: it then adds
// each copy's constant offset as it sets M0, instead of keeping every copy's
// address live in a register of its own across the loop (register pressure
// that spilled scalar registers).
__device__ __forceinline__ uint32_t pf_copy_base(const char* lds, uint32_t first) {
    uint32_t at = lds_address(lds) + 1024 * first;
    asm volatile("" : "+s"(at));
    return at;
}

// Block j of a row of n_heads blocks -> its query head. Consecutive blocks
// go to the 8 XCDs in turn, so with n_heads a multiple of 8 block j takes
// head (j % 8) * (n_heads / 8) + j / 8: XCD x holds heads x * n_heads / 8
// onwards, and since the query heads of one KV head are consecutive, each
// XCD's L2 holds the K and V of whole KV heads (for Llama-3-8B's 32 heads
// over 8 KV heads, one KV head per XCD) instead of parts of four.
__device__ __forceinline__ uint32_t pf_head(uint32_t j, uint32_t n_heads) {
    return n_heads % 8 == 0 ? (j % 8) * (n_heads / 8) + j / 8 : j;
}

template <bool F16>
__device__ __forceinline__ h8 pf_load_q(const void* base, std::size_t index) {
    if constexpr (F16) {
        return as_h8(load16(static_cast<const _Float16*>(base) + index));
    } else {
        const float* p = static_cast<const float*>(base) + index;
        const f4 lo = *reinterpret_cast<const f4*>(p);
        const f4 hi = *reinterpret_cast<const f4*>(p + 4);
        return h8{to_h(lo[0]), to_h(lo[1]), to_h(lo[2]), to_h(lo[3]), to_h(hi[0]), to_h(hi[1]), to_h(hi[2]),
                  to_h(hi[3])};
    }
}

// The P^T operands of one 64-key tile from its raw scores: p = exp2(s c - mc)
// rounded to binary16. A query whose keys all lie in the first key tile
// (position < pf_bk) takes its softmax whole there, as attend_group takes it
// (S/kernels/attention.hpp:222-227): its max is the tile's, its sum the
// tile's unrounded sum, and it rounds the normalised p = exp(s - max) / sum.
// Returns true for such a query (its O is then complete and normalised, its
// sum 1); later tiles hold none of its keys. Other queries keep the online
// form: unnormalised p rounded, O divided by the sum of the rounded p at the
// end. Only a wave whose first query sits in the first tile pays for the sum.
__device__ __forceinline__ bool probabilities(uint32_t t0, uint32_t pos_row0, uint32_t my_pos, float mc,
                                              f16v (&sc)[2], h8 (&pv)[4], float c) {
    if (t0 == 0 && pos_row0 < pf_bk) {  // wave-uniform
        float es = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sc[e][i] = fast_exp2(sc[e][i] * c - mc);  // the scores are not needed again
                es += sc[e][i];
            }
        }
        es = sum32(es);
        const bool whole = my_pos < pf_bk;
        const float f = whole ? 1.0f / es : 1.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                pv[2 * e + (i >> 3)][i & 7] = to_h(sc[e][i] * f);
            }
        }
        return whole;
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pv[2 * e + (i >> 3)][i & 7] = to_h(fast_exp2(sc[e][i] * c - mc));
        }
    }
    return false;
}

template <int HD, bool QF16>
__global__ __launch_bounds__(256, HD <= 128 ? 2 : 1) void prefill_kernel(const flash_args a) {
    constexpr int NS = HD / 16;     // k-steps of the score product
    constexpr int NT = HD / 32;     // 32-dim tiles of the output
    constexpr int HSPAN = HD / 2;   // dims a lane half holds across the k-steps
    constexpr int KCPR = HD / 8;               // 16-byte chunks of a K row
    constexpr int KROWC = KCPR + 1;            // LDS K row: one chunk of padding
    constexpr int VROWC = pf_bk / 8 + 1;       // LDS V^T row: 8 chunks of keys + padding
    constexpr int TK = pf_bk * KROWC / 64;     // 1 KB copies per K tile (exact)
    constexpr int TV = (HD * VROWC + 63) / 64; // 1 KB copies per V^T tile (last one partly slack)
    constexpr int TT = TK + TV;
    // Two LDS stages, separate objects so the compiler can tell a copy into
    // one from reads of the other.
    __shared__ __attribute__((aligned(16))) char lk0[TK * 1024];
    __shared__ __attribute__((aligned(16))) char lk1[TK * 1024];
    __shared__ __attribute__((aligned(16))) char lv0[TV * 1024];
    __shared__ __attribute__((aligned(16))) char lv1[TV * 1024];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int ln = tid & 63;
    const int H = ln >> 5;   // lane half
    const int qi = ln & 31;  // query column of this lane
    const uint32_t hd = a.hd;
    // Block -> (query tile, head): heads fastest; the first half of the grid
    // takes the latest (heaviest) query tiles in descending order, the second
    // half the earliest in ascending order, so the blocks resident together
    // on a CU carry about equal causal work.
    const uint32_t n_qt = (a.n + pf_bq - 1) / pf_bq;
    const uint32_t rank = blockIdx.x / a.n_heads;
    const uint32_t h = pf_head(blockIdx.x % a.n_heads, a.n_heads);
    const uint32_t heavy = (n_qt + 1) / 2;
    const uint32_t qt = rank < heavy ? n_qt - 1 - rank : rank - heavy;
    const uint32_t g = h / a.group;
    const float c = a.scale_log2e;

    const uint32_t q_first = qt * pf_bq;
    const uint32_t q_row0 = q_first + 32 * w;
    const uint32_t my_q = q_row0 + qi;
    const uint32_t my_pos = a.pos + my_q;
    const uint32_t q_last_block = min(a.n, q_first + pf_bq) - 1;
    const uint32_t kv_end = min(a.kv_len, a.pos + q_last_block + 1);  // keys this block needs
    const uint32_t wave_last_pos = a.pos + min(a.n - 1, q_row0 + 31);  // causal horizon of the wave
    const uint32_t n_tiles = (kv_end + pf_bk - 1) / pf_bk;

    // Q^T operand for the whole block: lane (H, qi) holds query my_q, dims
    // H*HSPAN + 8*st + [0, 8), rounded to binary16 (S/kernels/attention.hpp:204-206).
    h8 qv[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st) {
        const uint32_t d0 = H * HSPAN + 8 * st;
        qv[st] = my_q < a.n && d0 < hd ? pf_load_q<QF16>(a.q, static_cast<std::size_t>(my_q) * a.q_row + h * hd + d0)
                                       : as_h8(zero_u4());
    }

    // Tile copies, global -> LDS through buffer resources, 1 KB per wave
    // instruction (buffer_load ... lds writes lane l's 16 bytes at +16 l).
    // LDS rows carry one 16-byte chunk of padding (K: 64 rows of KCPR + 1
    // chunks; V^T: HD rows of 8 + 1), so the operand reads below spread over
    // the banks. Copy j of a tile goes to wave j % 4. A lane's byte offset
    // inside a tile is fixed, so it is computed once; the tile moves the
    // resource base. Padding slots, dims past hd and slack past the V^T rows
    // take an out-of-range offset and arrive as zeros; so do K rows at or past
    // kv_end (the K resource ends there) and, in the last tile, V^T chunks
    // that start at or past it.
    constexpr int CPW = (TT + 3) / 4;  // copies per wave and tile, at most
    uint32_t coff[CPW];
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const uint32_t j = w + 4 * i;
        coff[i] = buffer_oob;
        if (j < TK) {
            const uint32_t L = 64 * j + ln;
            const uint32_t r = L / KROWC, cc = L % KROWC;
            if (cc < KCPR && 8 * cc < hd) {
                coff[i] = r * a.row * 2 + cc * 16;
            }
        } else if (j < TT) {
            const uint32_t L = 64 * (j - TK) + ln;
            const uint32_t d = L / VROWC, cc = L % VROWC;
            if (cc < 8 && d < hd) {
                coff[i] = d * a.ctx_stride * 2 + cc * 16;
            }
        }
    }
    const _Float16* k_head = a.k + g * hd;
    const _Float16* v_head = a.vt + static_cast<std::size_t>(g) * hd * a.ctx_stride;
    const uint32_t k_bytes = kv_end * a.row * 2 - g * hd * 2;  // through K row kv_end - 1 of head g
    const uint32_t v_bytes = hd * a.ctx_stride * 2;
    const auto issue = [&](uint32_t t0, char* sk, char* sv) {
        const rsrc k_res = make_rsrc(k_head + static_cast<std::size_t>(t0) * a.row, k_bytes - t0 * a.row * 2);
        const rsrc v_res = make_rsrc(v_head + t0, v_bytes - t0 * 2);
        const bool last = t0 + pf_bk > kv_end;
        const uint32_t kb = pf_copy_base(sk, w);
        const uint32_t vb = pf_copy_base(sv - 1024 * TK, w);
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const uint32_t j = w + 4 * i;
            if (j < TK) {
                pf_copy(k_res, kb + 4096 * i, coff[i]);
            } else if (j < TT) {
                uint32_t off = coff[i];
                if (last && 8 * ((64 * (j - TK) + ln) % VROWC) >= kv_end - t0) {
                    off = buffer_oob;
                }
                pf_copy(v_res, vb + 4096 * i, off);
            }
        }
    };
    // The last tile's V^T chunk that straddles kv_end holds stale halves past
    // it (a zero probability times a stale non-finite half would be NaN): zero them.
    const auto fixup = [&](uint32_t t0, char* sv) {
        if (kv_end % 8 != 0 && tid < HD) {
            _Float16* chunk = reinterpret_cast<_Float16*>(sv + (tid * VROWC + (kv_end - t0) / 8) * 16);
            for (uint32_t j = kv_end % 8; j < 8; ++j) {
                chunk[j] = 0;
            }
        }
    };

    f16v o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            o[n][i] = 0.0f;
        }
    }
    // Running max (raw q.k units) and sum of this lane's query. The max moves
    // lazily: only when some query of the wave sees scores more than
    // 8 / c above it (exp2 argument > 8), so most tiles skip the rescale of O;
    // probabilities then stay <= 2^8, and O and the sum share the same max,
    // so the quotient is unchanged.
    float m_run = -INFINITY, l_run = 0.0f;

    // One 64-key tile from one LDS stage.
    const auto compute = [&](uint32_t t0, const char* sk, const char* sv) {
        if (q_row0 >= a.n || t0 > wave_last_pos) {
            return;  // every key of the tile is after every query of this wave
        }
        f16v sc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sc[e][i] = 0.0f;
            }
            const char* krow = sk + ((32 * e + pf_slice_key(qi)) * KROWC + H * (KCPR / 2)) * 16;
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                sc[e] = mfma32(*reinterpret_cast<const h8*>(krow + 16 * st), qv[st], sc[e]);
            }
        }
        // Register i of slice e holds key t0 + 32e + 16(i/8) + 8H + i%8.
        if (t0 + pf_bk - 1 > a.pos + q_row0 || t0 + pf_bk > kv_end) {  // the tile crosses the diagonal or the end
            const uint32_t lim = max(min(my_pos + 1, kv_end), t0) - t0;  // keys t0 + [0, lim) are visible
#pragma unroll
            for (int e = 0; e < 2; ++e) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t kk = 32 * e + 16 * (i >> 3) + 8 * H + (i & 7);
                    sc[e][i] = kk < lim ? sc[e][i] : -INFINITY;
                }
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                tmax = fmaxf(tmax, sc[e][i]);
            }
        }
        tmax = max32(tmax);
        // (both -inf: NaN, no growth; m_run -inf and tmax finite: +inf, growth.)
        // The decision is the lane's own, so a query's result never depends
        // on other queries' scores; the wave skips the work when no lane grows.
        const bool grow = (tmax - m_run) * c > 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = grow ? tmax : m_run;
            const float alpha = grow ? fast_exp2((m_run - m_new) * c) : 1.0f;
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    o[n][i] *= alpha;
                }
            }
        }
        const float mc = (m_run == -INFINITY ? 0.0f : m_run) * c;
        h8 pv[4];  // P^T operands: 16-key steps 0..3 of the tile
        const bool whole = probabilities(t0, a.pos + q_row0, my_pos, mc, sc, pv, c);
        float psum = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                psum = add_pair(h2{pv[s2][i], pv[s2][i + 1]}, psum);
            }
        }
        psum = sum32(psum);
        l_run = whole ? 1.0f : l_run + psum;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const char* vrow = sv + ((32 * n + qi) * VROWC + H) * 16;  // V^T row 32n + qi, keys 8H..
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                o[n] = mfma32(*reinterpret_cast<const h8*>(vrow + 32 * s2), pv[s2], o[n]);
            }
        }
    };

    // Pipeline over tiles, two stages: tile t computes from one stage while
    // tile t+1's copy lands in the other; a stage is refilled (tile t+2)
    // once every wave has finished reading it.
    // This wave's copies per tile: TT / 4 or one more.
    const uint32_t per_tile = (TT - w + 3) / 4;
    const auto wait_tile = [&](uint32_t next_issued) {
        if (!next_issued) {
            __builtin_amdgcn_s_waitcnt(pf_vmcnt(0));
        } else if (per_tile == (TT + 3) / 4) {
            __builtin_amdgcn_s_waitcnt(pf_vmcnt((TT + 3) / 4));
        } else {
            __builtin_amdgcn_s_waitcnt(pf_vmcnt(TT / 4));
        }
    };
    issue(0, lk0, lv0);
    if (n_tiles > 1) {
        issue(pf_bk, lk1, lv1);
    }
    wait_tile(n_tiles > 1);
    pf_barrier();
    if (n_tiles == 1) {
        fixup(0, lv0);
        pf_barrier();
    }
    for (uint32_t t = 0; t < n_tiles; t += 2) {
        compute(t * pf_bk, lk0, lv0);
        if (t + 1 >= n_tiles) {
            break;
        }
        pf_barrier();
        if (t + 2 < n_tiles) {
            issue((t + 2) * pf_bk, lk0, lv0);
        }
        wait_tile(t + 2 < n_tiles);
        pf_barrier();
        if (t + 2 == n_tiles) {
            fixup((t + 1) * pf_bk, lv1);
            pf_barrier();
        }
        compute((t + 1) * pf_bk, lk1, lv1);
        if (t + 2 >= n_tiles) {
            break;
        }
        pf_barrier();
        if (t + 3 < n_tiles) {
            issue((t + 3) * pf_bk, lk1, lv1);
        }
        wait_tile(t + 3 < n_tiles);
        pf_barrier();
        if (t + 3 == n_tiles) {
            fixup((t + 2) * pf_bk, lv0);
            pf_barrier();
        }
    }

    if (my_q >= a.n) {
        return;
    }
    const float inv = 1.0f / l_run;
    float* out = a.out + static_cast<std::size_t>(my_q) * a.q_row + h * hd;
    // Register i of tile n holds dim 32n + 8(i/4) + 4H + i%4.
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t d = 32 * n + 8 * b + 4 * H;
            if (d < hd) {
                *reinterpret_cast<f4*>(out + d) =
                    f4{o[n][4 * b] * inv, o[n][4 * b + 1] * inv, o[n][4 * b + 2] * inv, o[n][4 * b + 3] * inv};
            }
        }
    }
}

// ---- balanced causal prefill: pairs of query tiles ----------------------------------
//
// Under the causal cut query tile t needs t + 1 key spans, so with one block
// per tile the latest tile's block runs long after its co-resident partner
// has finished. Here a block of 8 waves takes a pair of query tiles
// (r, n_qt - 1 - r) of one head. Wave group 1 (waves 4-7) takes the later
// tile's last key tiles; wave group 0 (waves 0-3) the earlier tile whole,
// then the later tile's first key tiles, so the groups do the same number of
// key tiles (within one). Each group runs the 4-wave kernel's two-stage LDS
// pipeline on its own stages, 128 queries, a wave 32 of them; both run the
// same number of steps, so the block-wide barriers pair up. The two partial
// (max, sum, O) of the later tile's queries meet in LDS at the end, in a
// fixed order. The tail of the last V^T chunk past kv_end is zeroed by the
// lane that copied it, right after its copy lands.
template <int HD, bool QF16>
__global__ __launch_bounds__(512, 2) void prefill_pair_kernel(const flash_args a) {
    constexpr int NS = HD / 16;
    constexpr int NT = HD / 32;
    constexpr int HSPAN = HD / 2;
    constexpr int KCPR = HD / 8;
    constexpr int KROWC = KCPR + 1;
    constexpr int VROWC = pf_bk / 8 + 1;
    constexpr int TK = pf_bk * KROWC / 64;
    constexpr int TV = (HD * VROWC + 63) / 64;
    constexpr int TT = TK + TV;
    // The merge of the two partials takes NT * 16 + 2 floats per lane, 1 KB
    // each for the group's 256 lanes, from group 0's four stage buffers.
    static_assert(2 * TK + 2 * TV >= NT * 16 + 2, "merge does not fit the stage buffers");
    __shared__ __attribute__((aligned(16))) char lk00[TK * 1024];
    __shared__ __attribute__((aligned(16))) char lk01[TK * 1024];
    __shared__ __attribute__((aligned(16))) char lv00[TV * 1024];
    __shared__ __attribute__((aligned(16))) char lv01[TV * 1024];
    __shared__ __attribute__((aligned(16))) char lk10[TK * 1024];
    __shared__ __attribute__((aligned(16))) char lk11[TK * 1024];
    __shared__ __attribute__((aligned(16))) char lv10[TV * 1024];
    __shared__ __attribute__((aligned(16))) char lv11[TV * 1024];

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int grp = w >> 2;                                   // wave group
    const int wg = w & 3;                                     // wave inside the group
    const int ln = tid & 63;
    const int H = ln >> 5;
    const int qi = ln & 31;
    const uint32_t hd = a.hd;
    const uint32_t n_qt = (a.n + pf_bq - 1) / pf_bq;
    const uint32_t pr = blockIdx.x / a.n_heads;
    const uint32_t h = pf_head(blockIdx.x % a.n_heads, a.n_heads);
    const uint32_t tA = pr, tB = n_qt - 1 - pr;  // tA == tB: the middle tile of an odd count
    const uint32_t g = h / a.group;
    const float c = a.scale_log2e;

    const auto kv_end_of = [&](uint32_t qt) __attribute__((always_inline)) {
        return min(a.kv_len, a.pos + min(a.n, qt * pf_bq + pf_bq));
    };
    const uint32_t nA = tA == tB ? 0 : (kv_end_of(tA) + pf_bk - 1) / pf_bk;
    const uint32_t nB = (kv_end_of(tB) + pf_bk - 1) / pf_bk;
    const uint32_t half = (nA + nB + 1) / 2;  // group 0's items; nA <= half
    const uint32_t split = half - nA;         // the later tile's key tiles group 0 takes
    const uint32_t cnt = grp == 0 ? half : nB - split;
    // Item j of this group: (query tile, key tile).
    const auto item_qt = [&](uint32_t j) __attribute__((always_inline)) { return grp == 0 && j < nA ? tA : tB; };
    const auto item_kt = [&](uint32_t j) __attribute__((always_inline)) {
        return grp == 0 ? (j < nA ? j : j - nA) : split + j;
    };

    // The query tile being computed and what follows from it.
    uint32_t q_row0 = 0, my_q = 0, my_pos = 0, kv_end = 0, wave_last_pos = 0;
    h8 qv[NS];
    const auto enter = [&](uint32_t qt) __attribute__((always_inline)) {
        q_row0 = qt * pf_bq + 32 * wg;
        my_q = q_row0 + qi;
        my_pos = a.pos + my_q;
        kv_end = kv_end_of(qt);
        wave_last_pos = a.pos + min(a.n - 1, q_row0 + 31);
        const uint32_t hd_here = pf_opaque(hd);  // (as in store)
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const uint32_t d0 = H * HSPAN + 8 * st;
            qv[st] = my_q < a.n && d0 < hd_here
                         ? pf_load_q<QF16>(a.q, static_cast<std::size_t>(my_q) * a.q_row + h * hd + d0)
                         : as_h8(zero_u4());
        }
        // Wait for q here, once per query tile: left to the compiler, the
        // wait would sit before every tile's first product (it cannot tell
        // whether this ran) and hold each tile until the next tile's copy
        // had landed too.
        __builtin_amdgcn_s_waitcnt(pf_vmcnt(0));
    };

    // Copy offsets as in the 4-wave kernel, over the group's 4 waves; vc[i]
    // is the key chunk of a V^T copy (8 keys), or 8 for none.
    constexpr int CPW = (TT + 3) / 4;
    uint32_t coff[CPW], vc[CPW];
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const uint32_t j = wg + 4 * i;
        coff[i] = buffer_oob;
        vc[i] = 8;
        if (j < TK) {
            const uint32_t L = 64 * j + ln;
            const uint32_t r = L / KROWC, cc = L % KROWC;
            if (cc < KCPR && 8 * cc < hd) {
                coff[i] = r * a.row * 2 + cc * 16;
            }
        } else if (j < TT) {
            const uint32_t L = 64 * (j - TK) + ln;
            const uint32_t d = L / VROWC, cc = L % VROWC;
            if (cc < 8 && d < hd) {
                coff[i] = d * a.ctx_stride * 2 + cc * 16;
                vc[i] = cc;
            }
        }
    }
    const _Float16* k_head = a.k + g * hd;
    const _Float16* v_head = a.vt + static_cast<std::size_t>(g) * hd * a.ctx_stride;
    const uint32_t v_bytes = hd * a.ctx_stride * 2;
    const auto issue = [&](uint32_t j, char* sk, char* sv) __attribute__((always_inline)) {
        const uint32_t ke = kv_end_of(item_qt(j));
        const uint32_t t0 = item_kt(j) * pf_bk;
        const rsrc k_res = make_rsrc(k_head + static_cast<std::size_t>(t0) * a.row, (ke - t0) * a.row * 2 - g * hd * 2);
        const rsrc v_res = make_rsrc(v_head + t0, v_bytes - t0 * 2);
        const bool last = t0 + pf_bk > ke;
        const uint32_t kb = pf_copy_base(sk, wg);
        const uint32_t vb = pf_copy_base(sv - 1024 * TK, wg);
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const uint32_t jj = wg + 4 * i;
            if (jj < TK) {
                pf_copy(k_res, kb + 4096 * i, coff[i]);
            } else if (jj < TT) {
                pf_copy(v_res, vb + 4096 * i, last && 8 * vc[i] >= ke - t0 ? buffer_oob : coff[i]);
            }
        }
    };
    // After item j's copies landed: the V^T chunk straddling kv_end holds
    // stale halves past it (a zero probability times a stale non-finite half
    // would be NaN); the lane that copied it zeroes them.
    const auto tail = [&](uint32_t j, char* sv) __attribute__((always_inline)) {
        const uint32_t ke = kv_end_of(item_qt(j));
        const uint32_t t0 = item_kt(j) * pf_bk;
        if (t0 + pf_bk <= ke || ke % 8 == 0) {
            return;
        }
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const uint32_t jj = wg + 4 * i;
            if (jj >= TK && jj < TT && vc[i] == (ke - t0) / 8) {
                _Float16* chunk = reinterpret_cast<_Float16*>(sv + 1024 * (jj - TK) + 16 * ln);
                for (uint32_t k = ke % 8; k < 8; ++k) {
                    chunk[k] = 0;
                }
            }
        }
    };

    f16v o[NT];
    float m_run = -INFINITY, l_run = 0.0f;
    const auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                o[n][i] = 0.0f;
            }
        }
        m_run = -INFINITY;
        l_run = 0.0f;
    };
    // The normalised rows of the current query tile, to out.
    const auto store = [&]() __attribute__((always_inline)) {
        if (my_q >= a.n) {
            return;
        }
        const float inv = 1.0f / l_run;
        float* out = a.out + static_cast<std::size_t>(my_q) * a.q_row + h * hd;
        // The dims' bounds compared here, where they are used: hoisted out of
        // the item loop, their lane masks took 32 scalar registers for the
        // whole kernel and spilled.
        const uint32_t hd_here = pf_opaque(hd);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t d = 32 * n + 8 * b + 4 * H;
                if (d < hd_here) {
                    *reinterpret_cast<f4*>(out + d) =
                        f4{o[n][4 * b] * inv, o[n][4 * b + 1] * inv, o[n][4 * b + 2] * inv, o[n][4 * b + 3] * inv};
                }
            }
        }
    };

    // One 64-key tile from one LDS stage (the 4-wave kernel's step).
    // W: this item may hold queries that take their softmax whole (the first
    // key tile of the first query tile); only the group's first item can.
    const auto compute = [&]<bool W>(uint32_t t0, const char* sk, const char* sv) __attribute__((always_inline)) {
        if (q_row0 >= a.n || t0 > wave_last_pos) {
            return;
        }
        f16v sc[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sc[e][i] = 0.0f;
            }
            const char* krow = sk + ((32 * e + pf_slice_key(qi)) * KROWC + H * (KCPR / 2)) * 16;
            // The slice's K operands read in one batch ahead of its products
            // (left to itself, the scheduler reused one register and waited
            // out each read's latency before its product).
            h8 kop[NS];
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                kop[st] = *reinterpret_cast<const h8*>(krow + 16 * st);
            }
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                sc[e] = mfma32(kop[st], qv[st], sc[e]);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, NS, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, NS, 0);
        }
        if (t0 + pf_bk - 1 > a.pos + q_row0 || t0 + pf_bk > kv_end) {
            // Key 32 e + 16 (i / 8) + 8 H + i % 8 of the tile is kept when it
            // is below the bound; the lane's half moved to the bound, each
            // compare is against a constant and no key index is held in a
            // register (that took 20 VGPRs for the whole kernel).
            const int lim = static_cast<int>(max(min(my_pos + 1, kv_end), t0) - t0) - 8 * H;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    sc[e][i] = 32 * e + 16 * (i >> 3) + (i & 7) < lim ? sc[e][i] : -INFINITY;
                }
            }
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                tmax = fmaxf(tmax, sc[e][i]);
            }
        }
        tmax = max32(tmax);
        const bool grow = (tmax - m_run) * c > 8.0f;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = grow ? tmax : m_run;
            const float alpha = grow ? fast_exp2((m_run - m_new) * c) : 1.0f;
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    o[n][i] *= alpha;
                }
            }
        }
        const float mc = (m_run == -INFINITY ? 0.0f : m_run) * c;
        h8 pv[4];
        bool whole = false;
        if constexpr (W) {
            whole = probabilities(t0, a.pos + q_row0, my_pos, mc, sc, pv, c);
        } else {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    pv[2 * e + (i >> 3)][i & 7] = to_h(fast_exp2(sc[e][i] * c - mc));
                }
            }
        }
        float psum = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                psum = add_pair(h2{pv[s2][i], pv[s2][i + 1]}, psum);
            }
        }
        psum = sum32(psum);
        l_run = whole ? 1.0f : l_run + psum;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const char* vrow = sv + ((32 * n + qi) * VROWC + H) * 16;
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                o[n] = mfma32(*reinterpret_cast<const h8*>(vrow + 32 * s2), pv[s2], o[n]);
            }
        }
    };

    // This wave's copies per item: TT / 4 or one more.
    const uint32_t per_tile = (TT - wg + 3) / 4;
    const auto wait_item = [&](bool next_issued) __attribute__((always_inline)) {
        if (!next_issued) {
            __builtin_amdgcn_s_waitcnt(pf_vmcnt(0));
        } else if (per_tile == (TT + 3) / 4) {
            __builtin_amdgcn_s_waitcnt(pf_vmcnt((TT + 3) / 4));
        } else {
            __builtin_amdgcn_s_waitcnt(pf_vmcnt(TT / 4));
        }
    };

    // Item j: switch query tile when it changes (group 0 after the earlier
    // tile: its rows go out, the later tile's queries come in), then compute.
    uint32_t cur_qt = item_qt(0);
    const auto run = [&](uint32_t j, const char* sk, const char* sv) __attribute__((always_inline)) {
        if (j >= cnt) {
            return;
        }
        const uint32_t qt = item_qt(j);
        if (qt != cur_qt) {
            store();
            reset();
            enter(qt);
            cur_qt = qt;
        }
        compute.template operator()<false>(item_kt(j) * pf_bk, sk, sv);
    };
    // The group's pipeline over its items; both groups take `half` steps
    // (two barriers each), so every barrier has all 8 waves.
    // The first query tile's q loads go out after the first two items'
    // copies, and enter's wait covers all of them.
    const auto pipeline = [&](char* k0, char* v0, char* k1, char* v1) __attribute__((always_inline)) {
        if (cnt > 0) {
            issue(0, k0, v0);
        }
        if (cnt > 1) {
            issue(1, k1, v1);
        }
        enter(cur_qt);
        if (cnt > 0) {
            tail(0, v0);
        }
        pf_barrier();
        // Item 0 apart, the only one that can hold whole-softmax queries, so
        // the loop's items keep the plain form's registers. The loop is the
        // same sequence rotated: each item, then its two barriers.
        if (cnt > 0) {
            compute.template operator()<true>(item_kt(0) * pf_bk, k0, v0);
        }
        for (uint32_t j = 0; j < half; j += 2) {
            pf_barrier();
            if (j + 2 < cnt) {
                issue(j + 2, k0, v0);
            }
            wait_item(j + 2 < cnt);
            if (j + 1 < cnt) {
                tail(j + 1, v1);
            }
            pf_barrier();
            if (j + 1 >= half) {
                break;
            }
            run(j + 1, k1, v1);
            pf_barrier();
            if (j + 3 < cnt) {
                issue(j + 3, k1, v1);
            }
            wait_item(j + 3 < cnt);
            if (j + 2 < cnt) {
                tail(j + 2, v0);
            }
            pf_barrier();
            if (j + 2 >= half) {
                break;
            }
            run(j + 2, k0, v0);
        }
    };
    reset();
    if (grp == 0) {
        pipeline(lk00, lv00, lk01, lv01);
    } else {
        pipeline(lk10, lv10, lk11, lv11);
    }
    // Group 0 may have ended on the earlier tile (it took none of the later
    // tile's keys): its rows go out and its partial of the later tile is empty.
    if (grp == 0 && cur_qt != tB) {
        store();
        reset();
        enter(tB);
    }

    // ---- merge the later tile's two partials: group 0 -> LDS -> group 1 --------------
    // Float f of lane (wg, ln) sits at index (f * 256 + 64 wg + ln) of group
    // 0's stage buffers taken in order (lk00, lk01, lv00, lv01): o[n][i] is
    // f = 16 n + i, then the max and the sum.
    const auto slot = [&](int f) __attribute__((always_inline)) -> float* {
        const uint32_t lane = 64 * wg + ln;
        if (f < TK) {
            return reinterpret_cast<float*>(lk00) + f * 256 + lane;
        }
        if (f < 2 * TK) {
            return reinterpret_cast<float*>(lk01) + (f - TK) * 256 + lane;
        }
        if (f < 2 * TK + TV) {
            return reinterpret_cast<float*>(lv00) + (f - 2 * TK) * 256 + lane;
        }
        return reinterpret_cast<float*>(lv01) + (f - 2 * TK - TV) * 256 + lane;
    };
    if (grp == 0) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                *slot(16 * n + i) = o[n][i];
            }
        }
        *slot(16 * NT) = m_run;
        *slot(16 * NT + 1) = l_run;
    }
    pf_barrier();
    if (grp == 1) {
        const float m0 = *slot(16 * NT), l0 = *slot(16 * NT + 1);
        const float m = fmaxf(m0, m_run);
        const float a0 = m0 == -INFINITY ? 0.0f : fast_exp2((m0 - m) * c);
        const float a1 = m_run == -INFINITY ? 0.0f : fast_exp2((m_run - m) * c);
        l_run = l0 * a0 + l_run * a1;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                o[n][i] = *slot(16 * n + i) * a0 + o[n][i] * a1;
            }
        }
        store();
    }
}

template <int HD>
hipError_t launch_hd(const flash_args& a, uint32_t dtype, hipStream_t stream) {
    if constexpr (HD <= 128) {
        // Two wave groups' stages fit LDS up to hd 128.
        const dim3 grid(a.n_heads * ((a.n + 2 * pf_bq - 1) / (2 * pf_bq)));
        if (dtype == 1) {
            prefill_pair_kernel<HD, true><<<grid, 512, 0, stream>>>(a);
        } else {
            prefill_pair_kernel<HD, false><<<grid, 512, 0, stream>>>(a);
        }
    } else {
        const dim3 grid(a.n_heads * ((a.n + pf_bq - 1) / pf_bq));
        if (dtype == 1) {
            prefill_kernel<HD, true><<<grid, 256, 0, stream>>>(a);
        } else {
            prefill_kernel<HD, false><<<grid, 256, 0, stream>>>(a);
        }
    }
    return hipGetLastError();
}

}  // namespace

bool prefill_fits(uint32_t kv_len, uint32_t row, uint32_t hd, uint32_t ctx_stride) {
    return uint64_t{kv_len} * row * 2 < (uint64_t{1} << 31) && uint64_t{hd} * ctx_stride * 2 < (uint64_t{1} << 31);
}

hipError_t launch_prefill(const flash_args& a, uint32_t q_dtype, hipStream_t stream) {
    switch ((a.hd + 31) / 32 * 32) {
    case 32:
        return launch_hd<32>(a, q_dtype, stream);
    case 64:
        return launch_hd<64>(a, q_dtype, stream);
    case 96:
        return launch_hd<96>(a, q_dtype, stream);
    case 128:
        return launch_hd<128>(a, q_dtype, stream);
    case 160:
        return launch_hd<160>(a, q_dtype, stream);
    case 192:
        return launch_hd<192>(a, q_dtype, stream);
    case 224:
        return launch_hd<224>(a, q_dtype, stream);
    case 256:
        return launch_hd<256>(a, q_dtype, stream);
    default:
        return hipErrorInvalidValue;
    }
}

}  // namespace syn
