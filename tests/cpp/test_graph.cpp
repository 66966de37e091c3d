// Host-only tests of the graph builder and the planner (no GPU): the
// reference's builder checks (tests/sdk/graph_builder.cpp:158-284) and
// planner invariants over random graphs (tests/sdk/graph_planner.cpp:18-118),
// restated for the attention path's operations.
#include "check.hpp"
#include "graph.hpp"
#include "planner.hpp"

#include <cmath>
#include <limits>
#include <random>
#include <vector>

using namespace syn::graph;

namespace {

graph_errc error_of(graph_builder&& b) {
    auto r = std::move(b).finalize();
    return r ? graph_errc{} : r.error().code;
}

void llama_attention_wiring() {
    graph_builder b(4);
    const tensor_id q = b.input(32 * 128), k = b.input(8 * 128), v = b.input(8 * 128);
    const tensor_id qr = b.rope(q, 128, 500000.0f), kr = b.rope(k, 128, 500000.0f);
    const state_id c = b.kv_cache(4097, 8, 128);
    const tensor_id out = b.attention(qr, kr, v, c, 32, 1.0f / std::sqrt(128.0f));
    b.output(out);
    auto r = std::move(b).finalize();
    CHECK(r.has_value());
    const compute_graph& g = r.value();
    CHECK(g.nodes().size() == 3);
    CHECK(g.position_limit() == 4097);
    CHECK(g.states().size() == 1 && g.states()[0].bytes == 2u * 2 * 4097 * 8 * 128);
    const auto& a = std::get<op_attention>(g.nodes()[2]);
    CHECK(g.tensors()[a.scratch].role == tensor_role::scratch);
    CHECK(g.tensors()[a.scratch].bytes == syn_hip_attention_scratch_bytes(32, 8, 128, 4097, 4));
    CHECK(g.tensors()[out].size == 32 * 128 && g.rows(out) == 4);
    const memory_plan p = plan(g);
    CHECK(plan_is_valid(g, p));
    CHECK(p.arena_bytes <= p.naive_bytes);
}

void kv_cache_errors() {
    {
        graph_builder b;
        CHECK(b.kv_cache(0, 8, 128) == invalid_state);
        CHECK(error_of(std::move(b)) == graph_errc::bad_shape);
    }
    {
        graph_builder b;
        CHECK(b.kv_cache(16, 8, 258) == invalid_state);  // head_dim > 256
        CHECK(error_of(std::move(b)) == graph_errc::bad_shape);
    }
    {
        // a position count of at most 2^32 (S/graph/graph.hpp:703): 2^32 is
        // accepted, one more is not
        graph_builder b;
        CHECK(b.kv_cache((std::size_t{1} << 32) + 1, 1, 2) == invalid_state);
        CHECK(error_of(std::move(b)) == graph_errc::bad_shape);
        graph_builder ok;
        const state_id c = ok.kv_cache(std::size_t{1} << 32, 1, 2);
        CHECK(c == 0);
        const tensor_id kv = ok.input(2);
        ok.output(ok.attention(kv, kv, kv, c, 1, 0.5f));
        auto r = std::move(ok).finalize();
        CHECK(r.has_value() && r.value().position_limit() == (std::size_t{1} << 32));
    }
    {
        graph_builder b;
        CHECK(b.kv_cache(std::size_t{1} << 31, std::size_t{1} << 40, 256) == invalid_state);
        CHECK(error_of(std::move(b)) == graph_errc::too_large);
    }
}

void attention_errors() {
    const auto base = [](auto&& body) {
        graph_builder b(2);
        const tensor_id q = b.input(4 * 16), k = b.input(2 * 16), v = b.input(2 * 16);
        const state_id c = b.kv_cache(12, 2, 16);
        body(b, q, k, v, c);
        return error_of(std::move(b));
    };
    CHECK(base([](graph_builder& b, tensor_id q, tensor_id k, tensor_id v, state_id c) {
              b.output(b.attention(q, k, v, c, 4, 0.25f));
          }) == graph_errc{});
    CHECK(base([](graph_builder& b, tensor_id q, tensor_id k, tensor_id v, state_id) {
              b.attention(q, k, v, 7, 4, 0.25f);
          }) == graph_errc::bad_state);
    CHECK(base([](graph_builder& b, tensor_id q, tensor_id k, tensor_id v, state_id c) {
              b.output(b.attention(q, k, v, c, 4, 0.25f));
              b.attention(q, k, v, c, 4, 0.25f);  // the cache is already used (I7)
          }) == graph_errc::bad_state);
    CHECK(base([](graph_builder& b, tensor_id q, tensor_id k, tensor_id v, state_id c) {
              b.attention(q, k, v, c, 3, 0.25f);  // 3 heads on 2 KV heads
          }) == graph_errc::bad_shape);
    CHECK(base([](graph_builder& b, tensor_id, tensor_id k, tensor_id v, state_id c) {
              b.attention(k, k, v, c, 4, 0.25f);  // q is not 4 heads
          }) == graph_errc::bad_shape);
    for (float s : {0.0f, -1.0f, NAN, INFINITY}) {
        CHECK(base([s](graph_builder& b, tensor_id q, tensor_id k, tensor_id v, state_id c) {
                  b.attention(q, k, v, c, 4, s);
              }) == graph_errc::bad_parameter);
    }
    CHECK(base([](graph_builder& b, tensor_id q, tensor_id k, tensor_id v, state_id c) {
              b.attention(q, k, v + 100, c, 4, 0.25f);
          }) == graph_errc::invalid_operand);
}

void first_error_wins() {
    graph_builder b;
    const tensor_id q = b.input(64);
    b.rope(q, 3, 0.5f);  // odd head_dim: bad_shape at node 0
    CHECK(b.kv_cache(0, 1, 1) == invalid_state);
    auto r = std::move(b).finalize();
    CHECK(!r.has_value() && r.error().code == graph_errc::bad_shape && r.error().node == 0);
    graph_builder none;
    none.input(4);
    auto r2 = std::move(none).finalize();
    CHECK(!r2.has_value() && r2.error().code == graph_errc::no_outputs);
    graph_builder zero(0);
    CHECK(error_of(std::move(zero)) == graph_errc::bad_shape);
}

// Zero-filled weights of a given format and shape, for the builder's checks
// (it reads shapes and formats, never values).
struct zero_weights {
    std::vector<unsigned char> bytes;
    weight_view view;
    zero_weights(std::uint32_t type, std::size_t rows_, std::size_t cols_)
        : bytes(rows_ * cols_ / block_values(type) * block_bytes(type)),
          view{type, rows_, cols_, bytes.data()} {}
    matrix_ref ref() const { return matrix_ref{view}; }
};

// The reference's builder cases (tests/sdk/graph_builder.cpp:21-284), restated
// for this builder: the same graphs, the same codes at the same nodes.
// Scratch sizes are this build's (the GPU kernels' buffers).
void reference_builder_cases() {
    // builds a valid graph in topological order (:21-58)
    {
        const zero_weights w(SYN_TYPE_Q4_K, 512, 256), gamma(SYN_TYPE_F32, 1, 256);
        graph_builder b;
        const tensor_id x = b.input(256);
        const tensor_id h = b.rms_norm(x, gamma.ref(), 1e-5f);
        const tensor_id y = b.matmul(w.ref(), h);
        const tensor_id z = b.silu(y);
        b.output(z);
        auto r = std::move(b).finalize();
        CHECK(r.has_value());
        const compute_graph& g = r.value();
        CHECK(g.inputs().size() == 1 && g.outputs().size() == 1 && g.nodes().size() == 3);
        CHECK(g.tensors()[y].size == 512 && g.tensors()[z].role == tensor_role::output);
        const auto& mm = std::get<op_matmul>(g.nodes()[1]);
        CHECK(g.tensors()[mm.scratch].role == tensor_role::scratch);
        CHECK(g.tensors()[mm.scratch].bytes == syn_hip_matmul_q_act_bytes(SYN_TYPE_Q4_K, 1, 256));
        for (std::size_t i = 0; i < g.nodes().size(); ++i) {  // I1
            for (tensor_id t : operands(g.nodes()[i])) {
                bool earlier = g.tensors()[t].role == tensor_role::input;
                for (std::size_t j = 0; j < i; ++j) {
                    for (tensor_id res : results(g.nodes()[j])) {
                        earlier = earlier || res == t;
                    }
                }
                CHECK(earlier);
            }
        }
    }
    // rejects mismatched sizes and reports the node (:60-73)
    {
        const zero_weights w(SYN_TYPE_Q8_0, 64, 128);
        graph_builder b;
        const tensor_id y = b.silu(b.input(256));
        CHECK(b.matmul(w.ref(), y) == invalid_tensor);
        b.output(y);
        auto r = std::move(b).finalize();
        CHECK(!r.has_value() && r.error().code == graph_errc::size_mismatch && r.error().node == 1);
    }
    // the first error wins and later calls are no-ops (:75-85)
    {
        graph_builder b;
        const tensor_id a = b.input(8), c = b.input(16);
        CHECK(b.add(a, c) == invalid_tensor);
        CHECK(b.silu(a) == invalid_tensor);
        CHECK(b.input(4) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::size_mismatch);
    }
    // invalid operands, empty inputs, bad outputs (:87-128)
    {
        graph_builder b;
        CHECK(b.silu(42) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::invalid_operand);
    }
    {
        graph_builder b;
        CHECK(b.input(0) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::empty_tensor);
    }
    {
        graph_builder b;
        b.input(8);
        CHECK(error_of(std::move(b)) == graph_errc::no_outputs);
    }
    {
        graph_builder b;
        const tensor_id y = b.silu(b.input(8));
        b.output(y);
        b.output(y);
        CHECK(error_of(std::move(b)) == graph_errc::bad_output);
    }
    {
        const zero_weights w(SYN_TYPE_Q8_0, 32, 32);
        graph_builder b;
        const tensor_id y = b.matmul(w.ref(), b.input(32));
        b.output(y + 1);  // the matmul's scratch tensor
        CHECK(error_of(std::move(b)) == graph_errc::bad_output);
    }
    {
        const zero_weights gamma(SYN_TYPE_F32, 2, 8);  // not a row vector
        graph_builder b;
        CHECK(b.rms_norm(b.input(8), gamma.ref(), 1e-5f) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::size_mismatch);
    }
    // sizes whose byte counts would overflow (:130-156)
    {
        graph_builder b;
        CHECK(b.input(std::numeric_limits<std::size_t>::max() / 2) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::too_large);
    }
    {
        graph_builder b;
        const std::size_t quarter = (max_graph_bytes / 4 - plan_alignment) / sizeof(float);
        for (int i = 0; i < 4; ++i) {
            CHECK(b.input(quarter) != invalid_tensor);
        }
        CHECK(b.input(quarter) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::too_large);
    }
    {
        graph_builder b;
        const tensor_id x = b.input(max_graph_bytes / sizeof(float) / 2);
        CHECK(x != invalid_tensor);
        CHECK(b.silu(x) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::too_large);
    }
    // embed, rope, and attention over a KV cache (:158-185)
    {
        const zero_weights table(SYN_TYPE_Q8_0, 100, 64);
        graph_builder b;
        const tensor_id x = b.embed(table.ref());
        const tensor_id q = b.rope(x, 16, 10000.0f);
        const tensor_id k = b.rope(b.silu(x), 16, 10000.0f);
        const tensor_id v = b.silu(x);
        const state_id small = b.kv_cache(32, 4, 16);
        const state_id large = b.kv_cache(64, 4, 16);
        const tensor_id a = b.attention(q, k, v, small, 4, 0.25f);
        const tensor_id a2 = b.attention(q, k, v, large, 4, 0.25f);
        b.output(b.add(a, a2));
        auto r = std::move(b).finalize();
        CHECK(r.has_value());
        const compute_graph& g = r.value();
        CHECK(g.inputs().empty() && g.token_limit() == 100 && g.position_limit() == 32);
        CHECK(g.states().size() == 2 && g.states()[small].bytes == 2 * 32 * 4 * 16 * sizeof(std::uint16_t));
        const auto& op = std::get<op_attention>(g.nodes()[5]);
        CHECK((operands(g.nodes()[5]) == std::vector<tensor_id>{q, k, v}));
        CHECK((results(g.nodes()[5]) == std::vector<tensor_id>{a, op.scratch}));
        CHECK(g.tensors()[op.scratch].role == tensor_role::scratch);
        CHECK(g.tensors()[op.scratch].bytes == std::max<std::uint64_t>(syn_hip_attention_scratch_bytes(4, 4, 16, 32, 1), 1));
    }
    // head layouts and parameters that do not fit (:187-234)
    const auto code = [](auto build) {
        graph_builder b;
        build(b);
        return error_of(std::move(b));
    };
    CHECK(code([](graph_builder& b) { b.rope(b.input(30), 15, 1e4f); }) == graph_errc::bad_shape);
    CHECK(code([](graph_builder& b) { b.rope(b.input(30), 4, 1e4f); }) == graph_errc::bad_shape);
    CHECK(code([](graph_builder& b) {
              const float f[3] = {1, 1, 1};
              b.rope(b.input(32), 8, 1e4f, f);
          }) == graph_errc::bad_shape);
    CHECK(code([](graph_builder& b) { b.rope(b.input(32), 8, std::nanf("")); }) == graph_errc::bad_parameter);
    CHECK(code([](graph_builder& b) {
              const float f[4] = {1, 0, 1, 1};
              b.rope(b.input(32), 8, 1e4f, f);
          }) == graph_errc::bad_parameter);
    CHECK(code([](graph_builder& b) { b.kv_cache(0, 2, 8); }) == graph_errc::bad_shape);
    CHECK(code([](graph_builder& b) { b.kv_cache(8, 2, max_head_dim + 2); }) == graph_errc::bad_shape);
    CHECK(code([](graph_builder& b) { b.kv_cache(std::size_t{1} << 30, std::size_t{1} << 28, 64); }) ==
          graph_errc::too_large);
    const auto attend = [](std::size_t q_size, std::size_t n_heads, float scale) {
        return [=](graph_builder& b) {
            const tensor_id q = b.input(q_size);
            const tensor_id kv = b.input(16);  // 2 KV heads of 8
            b.attention(q, kv, kv, b.kv_cache(8, 2, 8), n_heads, scale);
        };
    };
    CHECK(code(attend(24, 3, 1.0f)) == graph_errc::bad_shape);
    CHECK(code(attend(24, 4, 1.0f)) == graph_errc::bad_shape);
    CHECK(code(attend(32, 4, 0.0f)) == graph_errc::bad_parameter);
    CHECK(code([](graph_builder& b) {
              const tensor_id t = b.input(16);
              b.attention(t, t, t, 0, 2, 1.0f);
          }) == graph_errc::bad_state);
    CHECK(code([](graph_builder& b) {
              const tensor_id t = b.input(16);
              const state_id c = b.kv_cache(8, 2, 8);
              b.attention(t, t, t, c, 2, 1.0f);
              b.attention(t, t, t, c, 2, 1.0f);
          }) == graph_errc::bad_state);
    CHECK(code([](graph_builder& b) { b.embed(matrix_ref{}); }) == graph_errc::empty_tensor);
    // batched graphs size tensors for max_batch rows (:236-255)
    {
        const zero_weights w(SYN_TYPE_Q8_0, 64, 32);
        graph_builder b(8);
        const tensor_id x = b.input(32);
        const tensor_id y = b.matmul(w.ref(), x);
        const tensor_id last = b.last_row(y);
        const tensor_id z = b.silu(last);
        b.output(z);
        auto r = std::move(b).finalize();
        CHECK(r.has_value());
        const compute_graph& g = r.value();
        CHECK(g.max_batch() == 8 && g.rows(x) == 8 && g.tensors()[x].bytes == 8 * 32 * sizeof(float));
        CHECK(g.rows(y) == 8 && g.rows(last) == 1 && g.rows(z) == 1);
        const auto& mm = std::get<op_matmul>(g.nodes()[0]);
        CHECK(g.tensors()[mm.scratch].bytes == syn_hip_matmul_q_act_bytes(SYN_TYPE_Q8_0, 8, 32));
    }
    // ops that mix batched and single-row tensors (I8) (:257-284)
    const auto code4 = [](auto build) {
        graph_builder b(4);
        build(b);
        return error_of(std::move(b));
    };
    CHECK(code4([](graph_builder& b) {
              const tensor_id x = b.input(16);
              b.add(x, b.last_row(x));
          }) == graph_errc::size_mismatch);
    CHECK(code4([](graph_builder& b) { b.rope(b.last_row(b.input(16)), 8, 1e4f); }) == graph_errc::bad_shape);
    CHECK(code4([](graph_builder& b) { b.last_row(b.last_row(b.input(16))); }) == graph_errc::bad_shape);
    CHECK(code4([](graph_builder& b) {
              const tensor_id x = b.input(16);
              b.attention(b.last_row(x), x, x, b.kv_cache(8, 2, 8), 2, 1.0f);
          }) == graph_errc::bad_shape);
    {
        graph_builder b(0);
        CHECK(b.input(4) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::bad_shape);
    }
    {
        graph_builder b(std::numeric_limits<std::size_t>::max() / 8);  // max_batch * size * 4 wraps
        CHECK(b.input(64) == invalid_tensor);
        CHECK(error_of(std::move(b)) == graph_errc::too_large);
    }
}

void self_attention_errors() {
    graph_builder b(257);
    const tensor_id q = b.input(16 * 64), k = b.input(16 * 64), v = b.input(16 * 64);
    b.output(b.self_attention(q, k, v, 16, 0.125f));
    CHECK(error_of(std::move(b)) == graph_errc{});
    graph_builder c(8);
    const tensor_id x = c.input(30);
    c.self_attention(x, x, x, 4, 0.5f);  // 30 is not whole heads
    CHECK(error_of(std::move(c)) == graph_errc::bad_shape);
}

void planner_random_graphs() {
    std::mt19937 rng(11);
    int planned = 0;
    for (int trial = 0; trial < 200; ++trial) {
        graph_builder b(1 + rng() % 8);
        std::vector<std::pair<tensor_id, std::size_t>> live;  // (tensor, floats per row)
        for (int i = 0; i < 1 + static_cast<int>(rng() % 4); ++i) {
            const std::size_t size = 64 * (1 + rng() % 8);
            live.emplace_back(b.input(size), size);
        }
        const int n_ops = 1 + static_cast<int>(rng() % 12);
        for (int i = 0; i < n_ops; ++i) {
            const auto [x, size] = live[rng() % live.size()];
            switch (rng() % 3) {
            case 0:
                live.emplace_back(b.rope(x, 32, 0.9f), size);
                break;
            case 1:
                live.emplace_back(b.self_attention(x, x, x, 2, 0.5f), size);
                break;
            default: {
                const state_id c = b.kv_cache(16 + rng() % 64, 1, 32);
                const tensor_id kv = b.input(32);
                live.emplace_back(b.attention(x, kv, kv, c, size / 32, 0.5f), size);
            }
            }
        }
        // a few random outputs
        b.output(live.back().first);
        if (live.size() > 3 && rng() % 2) {
            b.output(live[1].first);
        }
        auto r = std::move(b).finalize();
        CHECK(r.has_value());
        if (!r) {
            continue;
        }
        const memory_plan p = plan(r.value());
        CHECK(plan_is_valid(r.value(), p));
        CHECK(p.arena_bytes <= p.naive_bytes);
        ++planned;
    }
    CHECK(planned == 200);
}

void planner_reuses_dead_tensors() {
    // a chain of ropes: each result dies once the next reads it, so the
    // arena holds two rows of tensors, not the whole chain
    graph_builder b(4);
    tensor_id x = b.input(4096);
    for (int i = 0; i < 10; ++i) {
        x = b.rope(x, 128, 0.9f);
    }
    b.output(x);
    auto r = std::move(b).finalize();
    CHECK(r.has_value());
    const memory_plan p = plan(r.value());
    CHECK(plan_is_valid(r.value(), p));
    CHECK(p.arena_bytes == 2 * align_up(4096 * 4 * 4));
    CHECK(p.naive_bytes == 11 * align_up(4096 * 4 * 4));
}

// The builder checks of the model ops (S/graph/graph.hpp:536-896): each
// misuse fails with the reference's code at the node being added.
void model_op_errors() {
    static const float w64x16[64 * 16] = {}, v16[16] = {}, table[8 * 16] = {};
    static const unsigned char q8[4 * 34] = {};
    const matrix_ref w{weight_view{SYN_TYPE_F32, 64, 16, w64x16}};
    const matrix_ref g16{weight_view{SYN_TYPE_F32, 1, 16, v16}};
    const matrix_ref rows8{weight_view{SYN_TYPE_F32, 8, 16, table}};
    const matrix_ref q8_row{weight_view{SYN_TYPE_Q8_0, 1, 128, q8}};
    const auto err = [](auto&& build) {
        graph_builder b(4);
        const tensor_id x = b.input(16);
        build(b, x);
        return error_of(std::move(b));
    };
    const auto ok = [&](auto&& build) {
        graph_builder b(4);
        const tensor_id x = b.input(16);
        b.output(build(b, x));
        return error_of(std::move(b)) == graph_errc{};
    };
    CHECK(ok([&](graph_builder& b, tensor_id x) { return b.matmul(w, x); }));
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.matmul(w, b.matmul(w, x))); }) ==
          graph_errc::size_mismatch);  // 64 values into a 16-column matrix
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.matmul(matrix_ref{}, x)); }) ==
          graph_errc::size_mismatch);  // the empty matrix
    CHECK(err([&](graph_builder& b, tensor_id x) {
              b.output(b.matmul(matrix_ref{weight_view{SYN_TYPE_F32, 64, 16, nullptr}}, x));
          }) == graph_errc::bad_parameter);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.add(x, b.matmul(w, x))); }) ==
          graph_errc::size_mismatch);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.mul(x, b.last_row(x))); }) ==
          graph_errc::size_mismatch);  // batched against one row (I8)
    CHECK(ok([&](graph_builder& b, tensor_id x) { return b.add_bias(x, g16); }));
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.add_bias(x, rows8)); }) == graph_errc::size_mismatch);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.add_bias(b.matmul(w, x), q8_row)); }) ==
          graph_errc::size_mismatch);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.rms_norm(x, w, 1e-5f)); }) ==
          graph_errc::size_mismatch);
    CHECK(ok([&](graph_builder& b, tensor_id x) { return b.softmax(b.silu(b.gelu(b.rms_norm(x, g16, 1e-5f)))); }));
    CHECK(err([&](graph_builder& b, tensor_id) { b.output(b.embed(matrix_ref{})); }) == graph_errc::empty_tensor);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.attn_temperature(x, 0.5f, 0)); }) ==
          graph_errc::bad_parameter);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.attn_temperature(x, NAN, 4)); }) ==
          graph_errc::bad_parameter);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.attn_temperature(b.last_row(x), 0.5f, 4)); }) ==
          graph_errc::bad_shape);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.last_row(b.last_row(x))); }) == graph_errc::bad_shape);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.layer_norm(x, g16, matrix_ref{}, -1.0f)); }) ==
          graph_errc::bad_parameter);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.layer_norm(x, g16, rows8, 1e-5f)); }) ==
          graph_errc::size_mismatch);
    CHECK(ok([&](graph_builder& b, tensor_id x) { return b.layer_norm(x, g16, g16, 0.0f); }));
    CHECK(ok([&](graph_builder& b, tensor_id x) { return b.add_rows(x, rows8); }));
    CHECK(err([&](graph_builder& b, tensor_id x) {
              b.output(b.add_rows(x, matrix_ref{weight_view{SYN_TYPE_F32, 3, 16, table}}));
          }) == graph_errc::size_mismatch);  // fewer rows than max_batch
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.pixel_shuffle(x, 3, 2)); }) == graph_errc::bad_shape);
    CHECK(err([&](graph_builder& b, tensor_id x) { b.output(b.pixel_shuffle(x, 2, 1)); }) == graph_errc::bad_shape);
    CHECK(err([&](graph_builder& b, tensor_id x) {
              b.output(b.pixel_shuffle(b.pixel_shuffle(x, 2, 2), 1, 2));
          }) == graph_errc::bad_shape);  // its result is not per-token (I8)
    CHECK(err([&](graph_builder& b, tensor_id x) {
              const tensor_id y = b.silu(x);
              b.output(y);
              b.output(y);
          }) == graph_errc::bad_output);
    {
        // a 2 x 2 grid of 4 patches merged into one row of 4 * 16; the graph
        // then takes full batches only (I9)
        graph_builder b(4);
        const tensor_id x = b.input(16);
        const tensor_id y = b.pixel_shuffle(x, 2, 2);
        b.output(b.matmul(matrix_ref{weight_view{SYN_TYPE_F32, 8, 64, w64x16}}, y));
        auto r = std::move(b).finalize();
        CHECK(r.has_value());
        if (r) {
            const compute_graph& g = r.value();
            CHECK(g.full_batch_only() && !g.embeds());
            CHECK(g.rows(y) == 1 && g.tensors()[y].size == 64 && g.tensors()[y].row_div == 4);
            CHECK(plan_is_valid(g, plan(g)));
        }
    }
    {
        // embed bounds the tokens a run accepts; matmul on quantized
        // weights sizes its activation scratch through the library
        graph_builder b(2);
        const tensor_id x = b.embed(rows8);
        const tensor_id y = b.matmul(matrix_ref{weight_view{SYN_TYPE_Q8_0, 4, 16 * 2, q8}}, b.add(x, x));
        b.output(y);
        auto r = std::move(b).finalize();
        CHECK(!r.has_value() && r.error().code == graph_errc::size_mismatch);  // 16 values, 32 columns
        graph_builder b2(2);
        const tensor_id x2 = b2.embed(rows8);
        const tensor_id h = b2.matmul(matrix_ref{weight_view{SYN_TYPE_F32, 2, 16, w64x16}}, x2);
        const tensor_id y2 = b2.matmul(matrix_ref{weight_view{SYN_TYPE_Q8_0, 4, 32, q8}},
                                       b2.matmul(matrix_ref{weight_view{SYN_TYPE_F32, 32, 2, w64x16}}, h));
        b2.output(y2);
        auto r2 = std::move(b2).finalize();
        CHECK(r2.has_value());
        if (r2) {
            const compute_graph& g = r2.value();
            CHECK(g.embeds() && g.token_limit() == 8 && !g.full_batch_only());
            const auto& mm = std::get<op_matmul>(g.nodes().back());
            CHECK(g.tensors()[mm.scratch].bytes == syn_hip_matmul_q_act_bytes(SYN_TYPE_Q8_0, 2, 32));
            CHECK(plan_is_valid(g, plan(g)));
        }
    }
}

}  // namespace

int main() {
    reference_builder_cases();
    model_op_errors();
    llama_attention_wiring();
    kv_cache_errors();
    attention_errors();
    first_error_wins();
    self_attention_errors();
    planner_random_graphs();
    planner_reuses_dead_tensors();
    CHECK_DONE();
}
