// Host-only tests of the graph builder and the planner (no GPU): the
// reference's builder checks (tests/sdk/graph_builder.cpp:158-284) and
// planner invariants over random graphs (tests/sdk/graph_planner.cpp:18-118),
// restated for the attention path's operations.
#include "check.hpp"
#include "graph.hpp"
#include "planner.hpp"

#include <cmath>
#include <random>

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
        graph_builder b;
        CHECK(b.kv_cache(std::size_t{1} << 33, 8, 128) == invalid_state);  // not a 32-bit position
        CHECK(error_of(std::move(b)) == graph_errc::bad_shape);
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

}  // namespace

int main() {
    llama_attention_wiring();
    kv_cache_errors();
    attention_errors();
    first_error_wins();
    self_attention_errors();
    planner_random_graphs();
    planner_reuses_dead_tensors();
    CHECK_DONE();
}
