// oracle.cpp — CPU restatement of synapse's KV-cache attention semantics.
//
// TEST INFRASTRUCTURE ONLY: the checker for the HIP path (see oracle.h). Only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
//
// Each function restates the reference function cited above it
// (branes-ai/synapse v0.15.12; S/ = sdk/include/branes/synapse/). The float
// operations are kept in the reference's order, because the point of this
// file is to round where the reference rounds: -ffp-contract=off
// (cmake/numerics.cmake:13-15) and no reassociation.
//
// Parity of every function here is pinned by tests/test_oracle_*.py against
// numpy's IEEE binary16 conversion, double-precision closed forms, brute force
// on tiny inputs and the reference's own known-answer checks.

#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <bit>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <span>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// binary16 <-> binary32 (S/numeric/half.hpp:18-41, :46-82)

float widen(std::uint16_t h) {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t e = (h >> 10) & 0x1fu;
    const std::uint32_t f = h & 0x3ffu;
    if (e == 0x1fu) {  // inf / NaN, payload kept
        return std::bit_cast<float>(sign | 0x7f800000u | (f << 13));
    }
    if (e != 0) {
        return std::bit_cast<float>(sign | ((e + 112u) << 23) | (f << 13));
    }
    // zero or subnormal: f * 2^-24, exact in float.
    const float mag = std::ldexp(static_cast<float>(f), -24);
    return std::bit_cast<float>(sign | std::bit_cast<std::uint32_t>(mag));
}

std::uint16_t narrow(float x) {
    const std::uint32_t bits = std::bit_cast<std::uint32_t>(x);
    const auto sign = static_cast<std::uint16_t>((bits >> 16) & 0x8000u);
    const std::uint32_t mag = bits & 0x7fffffffu;
    if (mag > 0x7f800000u) {  // NaN: quiet, top payload bits kept
        return static_cast<std::uint16_t>(sign | 0x7c00u | 0x200u | ((mag >> 13) & 0x3ffu));
    }
    if (mag >= 0x477ff000u) {  // inf, or rounds past 65504
        return static_cast<std::uint16_t>(sign | 0x7c00u);
    }
    if (mag < 0x38800000u) {  // below 2^-14: a subnormal count of 2^-24
        // |x| * 2^24 is exact in double; nearbyint rounds half to even.
        const double units = std::nearbyint(static_cast<double>(std::bit_cast<float>(mag)) * 16777216.0);
        return static_cast<std::uint16_t>(sign | static_cast<std::uint16_t>(units));
    }
    const std::uint32_t r = mag - (112u << 23);  // rebias 127 -> 15
    std::uint32_t h = r >> 13;
    const std::uint32_t rest = r & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) {
        ++h;  // a carry out of the fraction bumps the exponent, as it should
    }
    return static_cast<std::uint16_t>(sign | h);
}

float round16(float x) {
    return widen(narrow(x));
}

// ---------------------------------------------------------------------------
// softmax (S/kernels/elementwise.hpp:174-201): exact max, float exp, a double
// sum in element order, then a multiply by float(1/sum).

void softmax_inplace(float* x, std::size_t n) {
    float mx = x[0];
    for (std::size_t i = 1; i < n; ++i) {
        mx = std::max(mx, x[i]);
    }
    for (std::size_t i = 0; i < n; ++i) {
        x[i] = std::exp(x[i] - mx);
    }
    double sum = 0.0;
    for (std::size_t i = 0; i < n; ++i) {
        sum += x[i];
    }
    const auto inv = static_cast<float>(1.0 / sum);
    for (std::size_t i = 0; i < n; ++i) {
        x[i] *= inv;
    }
}

struct cache_view {
    std::uint16_t* k;
    std::uint16_t* v;
    std::size_t max_ctx, n_kv, hd;
    std::size_t row() const {
        return n_kv * hd;
    }
};

// kv_append (S/kernels/attention.hpp:165-175)
void append_row(const float* k, const float* v, const cache_view& c, std::uint32_t pos) {
    const std::size_t row = c.row();
    std::uint16_t* kr = c.k + std::size_t{pos} * row;
    std::uint16_t* vr = c.v + std::size_t{pos} * row;
    for (std::size_t i = 0; i < row; ++i) {
        kr[i] = narrow(k[i]);
        vr[i] = narrow(v[i]);
    }
}

// attend_group (S/kernels/attention.hpp:185-244). scores holds, for each of
// the group's heads, a row over the positions (laid out j * n_pos + t), then
// the group's q rounded to F16 at offset group * max_ctx.
void attend(const float* q, const cache_view& c, std::uint32_t pos, std::size_t n_heads, float scale, float* out,
            float* scores, std::size_t g) {
    const std::size_t hd = c.hd, row = c.row();
    const std::size_t group = n_heads / c.n_kv;
    const std::size_t n_pos = std::size_t{pos} + 1;
    float* qg = scores + group * c.max_ctx;
    for (std::size_t i = 0; i < group * hd; ++i) {
        qg[i] = round16(q[g * group * hd + i]);  // :204-206
    }
    float kv[256];
    for (std::size_t t = 0; t < n_pos; ++t) {  // :208-221
        const std::uint16_t* kt = c.k + t * row + g * hd;
        for (std::size_t d = 0; d < hd; ++d) {
            kv[d] = widen(kt[d]);
        }
        for (std::size_t j = 0; j < group; ++j) {
            const float* qj = qg + j * hd;
            float dot = 0.0f;
            for (std::size_t d = 0; d < hd; ++d) {
                dot += qj[d] * kv[d];
            }
            scores[j * n_pos + t] = dot * scale;
        }
    }
    for (std::size_t j = 0; j < group; ++j) {  // :222-229
        float* s = scores + j * n_pos;
        softmax_inplace(s, n_pos);
        for (std::size_t t = 0; t < n_pos; ++t) {
            s[t] = round16(s[t]);
        }
        std::fill_n(out + (g * group + j) * hd, hd, 0.0f);
    }
    for (std::size_t t = 0; t < n_pos; ++t) {  // :231-243
        const std::uint16_t* vt = c.v + t * row + g * hd;
        for (std::size_t d = 0; d < hd; ++d) {
            kv[d] = widen(vt[d]);
        }
        for (std::size_t j = 0; j < group; ++j) {
            const float p = scores[j * n_pos + t];
            float* oj = out + (g * group + j) * hd;
            for (std::size_t d = 0; d < hd; ++d) {
                oj[d] += p * kv[d];
            }
        }
    }
}

std::size_t group_floats(std::size_t n_heads, std::size_t n_kv, std::size_t hd, std::size_t max_ctx) {
    return n_heads / n_kv * (max_ctx + hd);  // S/kernels/attention.hpp:147-152
}

// body(i) for i in [0, n) on `threads` std::threads taking items off one
// counter, standing in for session::parallel (S/graph/session.hpp:259-278):
// each item is computed by one call whatever the split, so the result does
// not depend on the thread count.
template <typename Body>
void parallel_items(std::size_t n, unsigned threads, Body&& body) {
    const std::size_t team = std::min<std::size_t>(std::max(1u, threads), n);
    if (team <= 1) {
        for (std::size_t i = 0; i < n; ++i) {
            body(i);
        }
        return;
    }
    std::atomic<std::size_t> next{0};
    std::vector<std::thread> pool;
    pool.reserve(team);
    for (std::size_t w = 0; w < team; ++w) {
        pool.emplace_back([&] {
            for (;;) {
                const std::size_t i = next.fetch_add(1, std::memory_order_relaxed);
                if (i >= n) {
                    return;
                }
                body(i);
            }
        });
    }
    for (auto& t : pool) {
        t.join();
    }
}

void attend_rows(const float* q, std::size_t n, std::uint32_t pos, const cache_view& c, std::size_t n_heads,
                 float scale, float* out, float* scores, unsigned threads) {
    const std::size_t slot = group_floats(n_heads, c.n_kv, c.hd, c.max_ctx);
    const std::size_t qsize = n_heads * c.hd;
    // session.hpp:360-373: the KV groups in parallel, each over every token.
    parallel_items(c.n_kv, threads, [&](std::size_t g) {
        for (std::size_t i = 0; i < n; ++i) {
            attend(q + i * qsize, c, pos + static_cast<std::uint32_t>(i), n_heads, scale, out + i * qsize,
                   scores + g * slot, g);
        }
    });
}

}  // namespace

extern "C" {

float orc_fp16_to_float(uint16_t h) {
    return widen(h);
}
uint16_t orc_float_to_fp16(float f) {
    return narrow(f);
}
void orc_fp16_to_float_n(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = widen(h[i]);
    }
}
void orc_float_to_fp16_n(const float* f, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        out[i] = narrow(f[i]);
    }
}

// rope_theta_scale (S/kernels/attention.hpp:47-49)
float orc_rope_theta_scale(float base, size_t head_dim) {
    return std::pow(base, -2.0f / static_cast<float>(head_dim));
}

// rope_yarn_corr_dims (S/kernels/attention.hpp:71-81), in float.
void orc_rope_yarn_corr_dims(size_t n_dims, size_t n_ctx_orig, float base, float beta_fast, float beta_slow,
                             float out[2]) {
    const float pi = 3.14159265358979323846f;
    const auto dim = [&](float n_rot) {
        return static_cast<float>(n_dims) * std::log(static_cast<float>(n_ctx_orig) / (n_rot * 2 * pi)) /
               (2 * std::log(base));
    };
    out[0] = std::max(0.0f, std::floor(dim(beta_fast)));
    out[1] = std::min(static_cast<float>(n_dims) - 1, std::ceil(dim(beta_slow)));
}

// rope (S/kernels/attention.hpp:89-129): theta for pair i is pos *
// theta_scale^i, built by repeated float multiplication; YaRN as rope_yarn.
void orc_rope(const float* x, float* out, size_t size, size_t head_dim, uint32_t pos, float theta_scale,
              const float* freq_factors, int mode, const float* scaling) {
    const float freq_scale = scaling ? scaling[0] : 1.0f;
    const float ext_factor = scaling ? scaling[1] : 0.0f;
    const float attn_factor = scaling ? scaling[2] : 1.0f;
    const float corr_low = scaling ? scaling[3] : 0.0f;
    const float corr_high = scaling ? scaling[4] : 0.0f;
    const size_t stride = mode == 0 ? 2 : 1;
    const size_t offset = mode == 0 ? 1 : head_dim / 2;
    float theta = static_cast<float>(pos);
    for (size_t i = 0; i < head_dim / 2; ++i) {
        const float ff = freq_factors ? freq_factors[i] : 1.0f;
        const float theta_extrap = theta / ff;
        const float theta_interp = freq_scale * theta_extrap;
        float t = theta_interp;
        float mscale = attn_factor;
        if (ext_factor != 0.0f) {
            const float y = (static_cast<float>(i) - corr_low) / std::max(0.001f, corr_high - corr_low);
            const float ramp_mix = (1 - std::min(1.0f, std::max(0.0f, y))) * ext_factor;
            t = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
            mscale *= 1.0f + 0.1f * std::log(1.0f / freq_scale);
        }
        const float c = std::cos(t) * mscale;
        const float s = std::sin(t) * mscale;
        const size_t a = stride * i;
        for (size_t h = 0; h < size; h += head_dim) {
            const float x0 = x[h + a];
            const float x1 = x[h + a + offset];
            out[h + a] = x0 * c - x1 * s;
            out[h + a + offset] = x0 * s + x1 * c;
        }
        theta *= theta_scale;
    }
}

void orc_softmax(const float* x, float* out, size_t n) {
    if (out != x) {
        std::memcpy(out, x, n * sizeof(float));
    }
    softmax_inplace(out, n);
}

size_t orc_attention_group_floats(size_t n_heads, size_t n_kv, size_t hd, size_t max_ctx) {
    return group_floats(n_heads, n_kv, hd, max_ctx);
}
size_t orc_attention_scratch_floats(size_t n_heads, size_t n_kv, size_t hd, size_t max_ctx) {
    return n_kv * group_floats(n_heads, n_kv, hd, max_ctx);  // S/kernels/attention.hpp:156-161
}

void orc_kv_append(const float* k, const float* v, uint16_t* k_cache, uint16_t* v_cache, size_t max_ctx,
                   size_t n_kv, size_t hd, uint32_t pos) {
    append_row(k, v, cache_view{k_cache, v_cache, max_ctx, n_kv, hd}, pos);
}

void orc_attend_group(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, size_t max_ctx,
                      size_t n_kv, size_t hd, uint32_t pos, size_t n_heads, float scale, float* out,
                      float* scores, size_t g) {
    const cache_view c{const_cast<uint16_t*>(k_cache), const_cast<uint16_t*>(v_cache), max_ctx, n_kv, hd};
    attend(q, c, pos, n_heads, scale, out, scores, g);
}

// attention (S/kernels/attention.hpp:254-269)
void orc_attention(const float* q, const float* k, const float* v, uint16_t* k_cache, uint16_t* v_cache,
                   size_t max_ctx, size_t n_kv, size_t hd, uint32_t pos, size_t n_heads, float scale, float* out,
                   float* scores) {
    const cache_view c{k_cache, v_cache, max_ctx, n_kv, hd};
    append_row(k, v, c, pos);
    const size_t slot = group_floats(n_heads, n_kv, hd, max_ctx);
    for (size_t g = 0; g < n_kv; ++g) {
        attend(q, c, pos, n_heads, scale, out, scores + g * slot, g);
    }
}

// session::execute(op_attention) (S/graph/session.hpp:348-374)
void orc_attention_rows(const float* q, const float* k, const float* v, size_t n, uint32_t pos,
                        uint16_t* k_cache, uint16_t* v_cache, size_t max_ctx, size_t n_kv, size_t hd,
                        size_t n_heads, float scale, float* out, float* scores, unsigned threads) {
    const cache_view c{k_cache, v_cache, max_ctx, n_kv, hd};
    const size_t row = c.row();
    for (size_t i = 0; i < n; ++i) {  // :354-356, every token appended first
        append_row(k + i * row, v + i * row, c, pos + static_cast<uint32_t>(i));
    }
    attend_rows(q, n, pos, c, n_heads, scale, out, scores, threads);
}

void orc_attend_rows(const float* q, size_t n, uint32_t pos, const uint16_t* k_cache, const uint16_t* v_cache,
                     size_t max_ctx, size_t n_kv, size_t hd, size_t n_heads, float scale, float* out,
                     float* scores, unsigned threads) {
    const cache_view c{const_cast<uint16_t*>(k_cache), const_cast<uint16_t*>(v_cache), max_ctx, n_kv, hd};
    attend_rows(q, n, pos, c, n_heads, scale, out, scores, threads);
}

// session::execute(op_self_attention) (S/graph/session.hpp:409-449) with
// self_attend_head's arithmetic (S/kernels/attention.hpp:324-486): a score is
// acc = fma(q_d, k_d, acc) over d in order from 0, times scale; softmax in
// float; an output element is acc = fma(p_j, v_j, acc) over j in order. The
// transposed-K scratch and the register tiles only reorder loads, not these
// chains (the reference's D1 property), so they are not restated. The work
// units are (head, query block), 16 blocks per head (graph.hpp:132).
void orc_self_attention(const float* q, const float* k, const float* v, size_t n, size_t row_size,
                        size_t n_heads, float scale, float* out, unsigned threads) {
    const size_t hd = row_size / n_heads;
    const size_t blocks = 16;
    const size_t per_block = (n + blocks - 1) / blocks;
    parallel_items(n_heads * blocks, threads, [&](size_t u) {
        const size_t h = u / blocks;
        const size_t i0 = std::min(n, (u % blocks) * per_block);
        const size_t i1 = std::min(n, i0 + per_block);
        std::vector<float> s(n);
        const size_t off = h * hd;
        for (size_t i = i0; i < i1; ++i) {
            const float* qi = q + i * row_size + off;
            for (size_t j = 0; j < n; ++j) {
                const float* kj = k + j * row_size + off;
                float acc = 0.0f;
                for (size_t d = 0; d < hd; ++d) {
                    acc = std::fma(qi[d], kj[d], acc);
                }
                s[j] = acc * scale;
            }
            softmax_inplace(s.data(), n);
            float* oi = out + i * row_size + off;
            for (size_t e = 0; e < hd; ++e) {
                float acc = 0.0f;
                for (size_t j = 0; j < n; ++j) {
                    acc = std::fma(s[j], v[j * row_size + off + e], acc);
                }
                oi[e] = acc;
            }
        }
    });
}

}  // extern "C"
