// GPU test of the host session with every op of a Llama-family model: the
// decode graph built through graph_builder the way the reference's model
// builder builds it (S/models/llama.hpp:454-481: embed, rms_norm, matmul and
// add_bias, rope, attn_temperature, kv_cache, attention, add, silu, mul,
// last_row), run through the session, and checked against the logits
// llama.cpp computed for the reference's tiny models
// (tests/sdk/llama_golden.cpp:58-83).
//
// The same program checks the image encoder's graph (layer_norm, gelu,
// add_rows, self_attention, pixel_shuffle) against clip_tiny's golden
// embeddings when the dump's config says "model clip".
//
// Usage: test_model_session <dump dir> <max|rms|rowrms> <bound>. The directory
// holds what tests/test_host_cpp.py extracts from a fixture: config.txt
// (key value), manifest.txt (name type rows cols offset bytes) over
// weights.bin, tokens.txt and logits.bin (tokens x n_vocab f32). Each token
// is decoded as its own run(step), then the whole sequence as one
// run(batch), whose last row must give the last position's logits.
#include "check.hpp"
#include "session.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iterator>
#include <map>
#include <sstream>
#include <string>
#include <vector>

using namespace syn::graph;

namespace {

struct model_dump {
    std::map<std::string, std::string> cfg;
    std::vector<char> blob;
    std::map<std::string, weight_view> weights;
    std::vector<std::uint32_t> tokens;
    std::vector<float> logits;

    double num(const std::string& k) const {
        return std::strtod(cfg.at(k).c_str(), nullptr);
    }
    float f32(const std::string& k) const {
        return std::strtof(cfg.at(k).c_str(), nullptr);
    }
    std::size_t count(const std::string& k) const {
        return static_cast<std::size_t>(std::strtoull(cfg.at(k).c_str(), nullptr, 10));
    }
    bool has(const std::string& name) const {
        return weights.count(name) != 0;
    }
    matrix_ref w(const std::string& name) const {
        return weights.at(name);
    }
};

std::vector<char> slurp(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return {std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>()};
}

model_dump load(const std::string& dir) {
    model_dump d;
    std::ifstream cfg(dir + "/config.txt");
    for (std::string k, v; cfg >> k >> v;) {
        d.cfg[k] = v;
    }
    d.blob = slurp(dir + "/weights.bin");
    std::ifstream man(dir + "/manifest.txt");
    std::string name;
    std::uint32_t type;
    std::size_t rows, cols, offset, bytes;
    while (man >> name >> type >> rows >> cols >> offset >> bytes) {
        CHECK(offset + bytes <= d.blob.size());
        d.weights[name] = weight_view{type, rows, cols, d.blob.data() + offset};
    }
    std::ifstream tok(dir + "/tokens.txt");
    for (std::uint32_t t; tok >> t;) {
        d.tokens.push_back(t);
    }
    const std::vector<char> lg = slurp(dir + "/logits.bin");
    d.logits.resize(lg.size() / sizeof(float));
    std::copy(lg.begin(), lg.end(), reinterpret_cast<char*>(d.logits.data()));
    return d;
}

struct llama_graph {
    compute_graph g;
    tensor_id logits;
};

// S/models/llama.hpp:454-481, with linear(w, b, x) = matmul, then add_bias
// when the file has the bias.
llama_graph build(const model_dump& m, std::size_t max_batch, std::size_t max_ctx) {
    graph_builder b(max_batch);
    const std::size_t n_layer = m.count("n_layer"), hd = m.count("head_dim");
    const std::size_t n_head = m.count("n_head"), n_head_kv = m.count("n_head_kv");
    const float eps = m.f32("rms_eps"), base = m.f32("rope_base"), temp = m.f32("attn_temp_scale");
    const rope_mode mode = m.count("rope_mode") == 1 ? rope_mode::neox : rope_mode::normal;
    const rope_scaling scaling{m.f32("freq_scale"), m.f32("ext_factor"), m.f32("attn_factor"), m.f32("corr_low"),
                               m.f32("corr_high")};
    std::span<const float> freq_factors;
    if (m.has("rope_freqs.weight")) {
        const weight_view& ff = m.weights.at("rope_freqs.weight");
        freq_factors = {static_cast<const float*>(ff.data), ff.cols};
    }
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    const auto linear = [&](const std::string& w, const std::string& bias, tensor_id x) {
        const tensor_id y = b.matmul(m.w(w), x);
        return m.has(bias) ? b.add_bias(y, m.w(bias)) : y;
    };
    const matrix_ref embd = m.w("token_embd.weight");
    tensor_id x = b.embed(embd);
    for (std::size_t l = 0; l < n_layer; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        const tensor_id h = b.rms_norm(x, m.w(p + "attn_norm.weight"), eps);
        tensor_id q = b.rope(linear(p + "attn_q.weight", p + "attn_q.bias", h), hd, base, freq_factors, mode, scaling);
        const tensor_id k =
            b.rope(linear(p + "attn_k.weight", p + "attn_k.bias", h), hd, base, freq_factors, mode, scaling);
        const tensor_id v = linear(p + "attn_v.weight", p + "attn_v.bias", h);
        if (temp != 0.0f) {
            q = b.attn_temperature(q, temp, m.count("n_ctx_orig"));
        }
        const state_id cache = b.kv_cache(max_ctx, n_head_kv, hd);
        const tensor_id attn = b.attention(q, k, v, cache, n_head, scale);
        x = b.add(linear(p + "attn_output.weight", p + "attn_output.bias", attn), x);
        const tensor_id h2 = b.rms_norm(x, m.w(p + "ffn_norm.weight"), eps);
        const tensor_id act = b.mul(b.silu(linear(p + "ffn_gate.weight", p + "ffn_gate.bias", h2)),
                                    linear(p + "ffn_up.weight", p + "ffn_up.bias", h2));
        x = b.add(linear(p + "ffn_down.weight", p + "ffn_down.bias", act), x);
    }
    const std::string out = m.has("output.weight") ? "output.weight" : "token_embd.weight";
    const tensor_id logits =
        linear(out, "output.bias", b.rms_norm(b.last_row(x), m.w("output_norm.weight"), eps));
    b.output(logits);
    auto r = std::move(b).finalize();
    CHECK(r.has_value());
    if (!r.has_value()) {
        std::fprintf(stderr, "graph error %s at node %zu\n", std::string(to_string(r.error().code)).c_str(),
                     r.error().node);
        std::exit(1);
    }
    return {std::move(r).value(), logits};
}

// max |got - ref| / max |ref| ("max", the F32 fixtures' bound) or the
// relative rms error ("rms", the quantized fixtures'), and the argmax.
bool close(const float* got, const float* ref, std::size_t n, const std::string& metric, double bound, double* err) {
    double dmax = 0, rmax = 0, d2 = 0, r2 = 0;
    for (std::size_t i = 0; i < n; ++i) {
        const double d = static_cast<double>(got[i]) - ref[i];
        dmax = std::max(dmax, std::fabs(d));
        rmax = std::max(rmax, std::fabs(static_cast<double>(ref[i])));
        d2 += d * d;
        r2 += static_cast<double>(ref[i]) * ref[i];
    }
    *err = metric == "rms" ? std::sqrt(d2 / r2) : dmax / rmax;
    const bool same_argmax = std::max_element(got, got + n) - got == std::max_element(ref, ref + n) - ref;
    return std::isfinite(*err) && *err < bound && same_argmax;
}

// The image encoder, as S/models/clip.hpp:300-380 builds it: patch
// projection with add_bias and add_rows (position embeddings), per layer
// layer_norm, q/k/v, self_attention, the output projection and the GELU
// MLP with residual adds, then post layer_norm (when the file has it),
// pixel_shuffle and the projector matmul.
struct clip_graph {
    compute_graph g;
    tensor_id patches, embeddings;
};

clip_graph build_clip(const model_dump& m) {
    const std::size_t P = m.count("n_patches"), E = m.count("n_embd"), H = m.count("n_head");
    graph_builder b(P);
    const float eps = m.f32("eps");
    const auto linear = [&](const std::string& w, const std::string& bias, tensor_id x) {
        const tensor_id y = b.matmul(m.w(w), x);
        return m.has(bias) ? b.add_bias(y, m.w(bias)) : y;
    };
    const tensor_id patches = b.input(m.count("patch_floats"));
    tensor_id x = b.add_rows(linear("patch.w", "patch.b", patches), m.w("pos"));
    for (std::size_t l = 0; l < m.count("n_layer"); ++l) {
        const std::string p = "v.blk." + std::to_string(l) + ".";
        const tensor_id h = b.layer_norm(x, m.w(p + "ln1.weight"), m.w(p + "ln1.bias"), eps);
        const tensor_id a = b.self_attention(linear(p + "attn_q.weight", p + "attn_q.bias", h),
                                             linear(p + "attn_k.weight", p + "attn_k.bias", h),
                                             linear(p + "attn_v.weight", p + "attn_v.bias", h), H,
                                             1.0f / std::sqrt(static_cast<float>(E / H)));
        x = b.add(linear(p + "attn_out.weight", p + "attn_out.bias", a), x);
        const tensor_id h2 = b.layer_norm(x, m.w(p + "ln2.weight"), m.w(p + "ln2.bias"), eps);
        x = b.add(x, linear(p + "down.w", p + "down.b", b.gelu(linear(p + "up.w", p + "up.b", h2))));
    }
    if (m.has("post.w")) {
        x = b.layer_norm(x, m.w("post.w"), m.w("post.b"), eps);
    }
    const tensor_id emb = b.matmul(m.w("fc"), b.pixel_shuffle(x, m.count("grid"), m.count("scale_factor")));
    b.output(emb);
    auto r = std::move(b).finalize();
    CHECK(r.has_value());
    if (!r.has_value()) {
        std::fprintf(stderr, "graph error %s at node %zu\n", std::string(to_string(r.error().code)).c_str(),
                     r.error().node);
        std::exit(1);
    }
    return {std::move(r).value(), patches, emb};
}

// Per output row, rms(got - ref) / rms(ref) (tests/sdk/clip_golden.cpp:22-35).
int run_clip(const model_dump& m, const std::string& dir, double bound) {
    const clip_graph cg = build_clip(m);
    session s(cg.g);
    CHECK(s.status() == SYN_HIP_OK);
    const std::vector<char> raw = slurp(dir + "/patches.bin");
    std::vector<float> patches(raw.size() / sizeof(float));
    std::copy(raw.begin(), raw.end(), reinterpret_cast<char*>(patches.data()));
    const std::size_t rows = m.count("n_tokens"), width = m.count("n_embd_text");
    std::vector<float> got(rows * width);
    CHECK(s.write(cg.patches, patches));
    CHECK(s.run_rows(m.count("n_patches")));
    CHECK(!s.run_rows(m.count("n_patches") - 1));  // a pixel-shuffle graph takes full batches only
    CHECK(s.read(cg.embeddings, got));
    CHECK(m.logits.size() == got.size());
    double worst = 0;
    for (std::size_t r = 0; r < rows; ++r) {
        double d2 = 0, r2 = 0;
        for (std::size_t i = 0; i < width; ++i) {
            const double d = static_cast<double>(got[r * width + i]) - m.logits[r * width + i];
            d2 += d * d;
            r2 += static_cast<double>(m.logits[r * width + i]) * m.logits[r * width + i];
        }
        worst = std::max(worst, std::sqrt(d2 / r2));
    }
    std::printf("%s, image encoder: worst per-token rel rms %.3g (bound %g)\n", dir.c_str(), worst, bound);
    CHECK(std::isfinite(worst) && worst < bound);
    CHECK_DONE();
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 4) {
        std::fprintf(stderr, "usage: %s <dump dir> <max|rms> <bound>\n", argv[0]);
        return 2;
    }
    const model_dump m = load(argv[1]);
    const std::string metric = argv[2];
    const double bound = std::strtod(argv[3], nullptr);
    if (m.cfg.count("model") != 0 && m.cfg.at("model") == "clip") {
        return run_clip(m, argv[1], bound);
    }
    const std::size_t n_vocab = m.count("n_vocab"), n_tok = m.tokens.size();
    CHECK(n_tok > 0 && m.logits.size() == n_tok * n_vocab);

    // One token per run, as the reference's golden test decodes.
    {
        const llama_graph lg = build(m, 1, n_tok);
        session s(lg.g);
        CHECK(s.status() == SYN_HIP_OK);
        std::vector<float> got(n_vocab);
        double worst = 0;
        for (std::size_t pos = 0; pos < n_tok; ++pos) {
            CHECK(s.run(step{m.tokens[pos], static_cast<std::uint32_t>(pos)}));
            CHECK(s.read(lg.logits, got));
            double err = 0;
            CHECK(close(got.data(), m.logits.data() + pos * n_vocab, n_vocab, metric, bound, &err));
            worst = std::max(worst, err);
        }
        std::printf("%s, one token per run: worst %s error %.3g (bound %g)\n", argv[1], metric.c_str(), worst, bound);
        // run() rejects what the reference rejects
        CHECK(!s.run(step{static_cast<std::uint32_t>(lg.g.token_limit()), 0}));  // token past the table
        CHECK(!s.run(step{m.tokens[0], static_cast<std::uint32_t>(n_tok)}));    // position past the caches
        CHECK(!s.run_rows(1));                                                   // the graph embeds
    }
    // The whole sequence as one batch: last_row carries the last position.
    {
        const llama_graph lg = build(m, n_tok, n_tok);
        session s(lg.g);
        CHECK(s.status() == SYN_HIP_OK);
        std::vector<float> got(n_vocab);
        CHECK(s.run(batch{m.tokens, 0}));
        CHECK(s.read(lg.logits, got));
        double err = 0;
        CHECK(close(got.data(), m.logits.data() + (n_tok - 1) * n_vocab, n_vocab, metric, bound, &err));
        std::printf("%s, %zu tokens in one run: last position's %s error %.3g\n", argv[1], n_tok, metric.c_str(), err);
    }
    CHECK_DONE();
}
