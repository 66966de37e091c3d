// GPU test of the host session (synapse_amd/host/session.hpp) against the CPU
// oracle: graphs built with the reference's builder API, run through the C
// ABI, compared with the oracle's restatement of the same graph (rope, then
// session::execute(op_attention) / op_self_attention). Covers config 1's
// prefill-then-decode sequence, a Llama-3-8B-shaped GQA layer, the run()
// argument checks (S/graph/session.hpp:143-177), reset() reproducibility
// (tests/sdk/graph_session.cpp:256-291) and an image encoder's
// self-attention, one image per run_rows and several per run_images.
#include "check.hpp"
#include "oracle.h"
#include "session.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

using namespace syn::graph;

namespace {

std::vector<float> normal(std::size_t n, std::uint32_t seed) {
    std::mt19937 rng(seed);
    std::vector<float> v(n);
    for (std::size_t i = 0; i < n; i += 2) {  // Box-Muller on the 32-bit engine: portable
        const double u1 = (rng() + 1.0) / 4294967297.0, u2 = rng() / 4294967296.0;
        const double r = std::sqrt(-2.0 * std::log(u1));
        v[i] = static_cast<float>(r * std::cos(6.283185307179586 * u2));
        if (i + 1 < n) {
            v[i + 1] = static_cast<float>(r * std::sin(6.283185307179586 * u2));
        }
    }
    return v;
}

float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    float m = 0.0f;
    for (std::size_t i = 0; i < a.size(); ++i) {
        m = std::fmax(m, std::fabs(a[i] - b[i]));
    }
    return m;
}

struct layer_case {
    std::size_t n_heads, n_kv, hd, max_ctx, max_batch;
    float base;
};

// rope(q), rope(k), attention: the Llama layer's attention wiring
// (S/models/llama.hpp:455-463).
struct attention_layer {
    compute_graph g;
    tensor_id q, k, v, out;
};

attention_layer build(const layer_case& c) {
    graph_builder b(c.max_batch);
    const tensor_id q = b.input(c.n_heads * c.hd), k = b.input(c.n_kv * c.hd), v = b.input(c.n_kv * c.hd);
    const state_id cache = b.kv_cache(c.max_ctx, c.n_kv, c.hd);
    const tensor_id out = b.attention(b.rope(q, c.hd, c.base), b.rope(k, c.hd, c.base), v, cache, c.n_heads,
                                      1.0f / std::sqrt(static_cast<float>(c.hd)));
    b.output(out);
    auto r = std::move(b).finalize();
    CHECK(r.has_value());
    return attention_layer{std::move(r).value(), q, k, v, out};
}

// Runs `runs` (n tokens each, consecutive positions) through a session and
// the oracle; returns the worst max-abs difference.
float compare_sequence(const layer_case& c, const std::vector<std::size_t>& runs, std::uint32_t seed) {
    attention_layer L = build(c);
    session s(L.g);
    CHECK(s.status() == SYN_HIP_OK);
    const std::size_t qs = c.n_heads * c.hd, ks = c.n_kv * c.hd;
    std::vector<std::uint16_t> kc(c.max_ctx * ks, 0), vc(c.max_ctx * ks, 0);
    std::vector<float> scores(orc_attention_scratch_floats(c.n_heads, c.n_kv, c.hd, c.max_ctx));
    const float ts = orc_rope_theta_scale(c.base, c.hd);
    const float scale = 1.0f / std::sqrt(static_cast<float>(c.hd));
    float worst = 0.0f;
    std::uint32_t pos = 0;
    for (std::size_t n : runs) {
        const auto q = normal(n * qs, seed++), k = normal(n * ks, seed++), v = normal(n * ks, seed++);
        CHECK(s.write(L.q, q) && s.write(L.k, k) && s.write(L.v, v));
        std::vector<std::uint32_t> tokens(n, 0);
        CHECK(s.run(batch{tokens, pos}));
        std::vector<float> got(n * qs);
        CHECK(s.read(L.out, got));
        std::vector<float> qr(n * qs), kr(n * ks), want(n * qs);
        for (std::size_t i = 0; i < n; ++i) {
            orc_rope(q.data() + i * qs, qr.data() + i * qs, qs, c.hd, pos + static_cast<std::uint32_t>(i), ts,
                     nullptr, 0, nullptr);
            orc_rope(k.data() + i * ks, kr.data() + i * ks, ks, c.hd, pos + static_cast<std::uint32_t>(i), ts,
                     nullptr, 0, nullptr);
        }
        orc_attention_rows(qr.data(), kr.data(), v.data(), n, pos, kc.data(), vc.data(), c.max_ctx, c.n_kv, c.hd,
                           c.n_heads, scale, want.data(), scores.data(), 8);
        worst = std::fmax(worst, max_abs_diff(got, want));
        pos += static_cast<std::uint32_t>(n);
    }
    CHECK(s.status() == SYN_HIP_OK);
    return worst;
}

void config1_prefill_then_decode() {
    const layer_case c{8, 8, 32, 64, 32, 10000.0f};
    std::vector<std::size_t> runs{32};
    runs.insert(runs.end(), 32, 1);
    const float d = compare_sequence(c, runs, 100);
    std::printf("config 1 (32-token prefill + 32 decode steps): max-abs %.3g\n", d);
    CHECK(d <= 2e-3f);
}

void llama3_8b_layer() {
    const layer_case c{32, 8, 128, 600, 256, 500000.0f};
    const float d = compare_sequence(c, {256, 200, 1, 1, 7, 1}, 200);
    std::printf("8B layer (256 + 200 prefill, decode steps): max-abs %.3g\n", d);
    CHECK(d <= 2e-3f);
}

void run_arguments_and_reset() {
    const layer_case c{4, 2, 16, 12, 4, 10000.0f};
    attention_layer L = build(c);
    session s(L.g);
    CHECK(s.status() == SYN_HIP_OK);
    CHECK(L.g.position_limit() == 12);
    std::vector<std::uint32_t> five(5, 0), four(4, 0);
    CHECK(!s.run(batch{{}, 0}));           // empty
    CHECK(!s.run(batch{five, 0}));         // above max_batch
    CHECK(!s.run(batch{four, 9}));         // 9 + 4 > position_limit
    CHECK(!s.run(step{0, 12}));            // position 12 of 12
    const auto q = normal(4 * 64, 1), k = normal(4 * 32, 2), v = normal(4 * 32, 3);
    std::vector<float> a(4 * 64), b2(4 * 64);
    CHECK(s.write(L.q, q) && s.write(L.k, k) && s.write(L.v, v) && s.run(batch{four, 0}) && s.read(L.out, a));
    // run the same prompt again on a reset cache: identical, bit for bit
    s.reset();
    CHECK(s.write(L.q, q) && s.write(L.k, k) && s.write(L.v, v) && s.run(batch{four, 0}) && s.read(L.out, b2));
    CHECK(a == b2);
    // at position 0 the output is V's binary16 value, head h from KV head h / 2
    for (std::size_t h = 0; h < 4; ++h) {
        for (std::size_t d = 0; d < 16; ++d) {
            const float want = orc_fp16_to_float(orc_float_to_fp16(v[(h / 2) * 16 + d]));
            CHECK(a[h * 16 + d] == want);
        }
    }
    CHECK(s.state_bytes() >= 2u * 2 * 12 * 2 * 16);
}

void image_encoder() {
    const std::size_t H = 16, hd = 64, n = 257, images = 3;
    graph_builder b(n * images);
    const tensor_id q = b.input(H * hd), k = b.input(H * hd), v = b.input(H * hd);
    const tensor_id out = b.self_attention(q, k, v, H, 0.125f);
    b.output(out);
    auto r = std::move(b).finalize();
    CHECK(r.has_value());
    session s(r.value());
    CHECK(s.status() == SYN_HIP_OK);
    const std::size_t rows = n * images, size = H * hd;
    auto qv = normal(rows * size, 7), kv = normal(rows * size, 8), vv = normal(rows * size, 9);
    for (auto* x : {&qv, &kv, &vv}) {
        for (float& f : *x) {
            f = orc_fp16_to_float(orc_float_to_fp16(0.5f * f));  // config 5: f16 values ~ N(0, 0.5^2)
        }
    }
    CHECK(s.write(q, qv) && s.write(k, kv) && s.write(v, vv));
    std::vector<float> got(rows * size), want(n * size);
    CHECK(s.run_images(n, images) && s.read(out, got));
    float worst = 0.0f;
    for (std::size_t img = 0; img < images; ++img) {
        orc_self_attention(qv.data() + img * n * size, kv.data() + img * n * size, vv.data() + img * n * size, n,
                           size, H, 0.125f, want.data(), 8);
        for (std::size_t i = 0; i < n * size; ++i) {
            worst = std::fmax(worst, std::fabs(got[img * n * size + i] - want[i]));
        }
    }
    std::printf("image encoder (3 images x 257 rows, 16 heads of 64): max-abs %.3g\n", worst);
    CHECK(worst <= 2e-3f);
    // one image per run_rows, as the reference encodes
    std::vector<float> one(n * size);
    CHECK(s.write(q, std::span(qv).first(n * size)) && s.write(k, std::span(kv).first(n * size)) &&
          s.write(v, std::span(vv).first(n * size)) && s.run_rows(n) && s.read(out, one));
    CHECK(std::equal(one.begin(), one.end(), got.begin()));
    CHECK(!s.run_images(n, images + 1));  // more rows than max_batch
}

}  // namespace

int main() {
    config1_prefill_then_decode();
    llama3_8b_layer();
    run_arguments_and_reset();
    image_encoder();
    CHECK_DONE();
}
