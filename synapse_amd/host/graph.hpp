// graph.hpp — C++20 host side of the attention path: the graph IR and its
// checked builder, mirroring branes-ai/synapse's graph API for the operations
// on this path (S/ = sdk/include/branes/synapse/):
//   graph_builder::kv_cache        S/graph/graph.hpp:698-719
//   graph_builder::attention       S/graph/graph.hpp:727-761
//   graph_builder::self_attention  S/graph/graph.hpp:831-863
//   graph_builder::rope            S/graph/graph.hpp (op_rope; executed as S/graph/session.hpp:337-342)
//   op_attention / op_self_attention / op_rope node payloads, graph_errc codes,
//   "first error wins" with the node index (S/graph/graph.hpp:388-428, :919-928).
// Names, argument meanings and error codes are the reference's, so a model
// builder written against it (S/models/llama.hpp:455-463,
// S/models/clip.hpp:348-349) builds unchanged. What differs is what the
// scratch tensors hold: the GPU kernels need split-KV partials for decode
// and nothing for self-attention, not the CPU kernels' score rows.
//
// Invariants of a finalized graph (numbered as the reference's):
//   I1 node order is a topological order (operands exist before use);
//   I3 every tensor is an input or the result (or scratch) of one node;
//   I4 at least one output, outputs distinct and not scratch;
//   I5 the sum of tensor bytes and of state bytes are each <= max_graph_bytes;
//   I6 head layouts fit: whole heads, even head_dim <= 256 for rope and
//      attention, query heads divide evenly among the KV heads;
//   I7 every KV state is read and written by at most one attention node;
//   I8 rope, attention and self_attention take batched (per-token) tensors.
#pragma once

#include "synapse_hip.h"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <optional>
#include <string_view>
#include <utility>
#include <variant>
#include <vector>

namespace syn::graph {

using tensor_id = std::uint32_t;
using state_id = std::uint32_t;

inline constexpr tensor_id invalid_tensor = std::numeric_limits<tensor_id>::max();
inline constexpr state_id invalid_state = std::numeric_limits<state_id>::max();

// Alignment of every tensor and state in the device arena: the reference uses
// a 64-byte cache line (S/graph/graph.hpp:122); 256 bytes keeps every row a
// kernel reads with 16-byte vector or buffer loads aligned.
inline constexpr std::size_t plan_alignment = 256;
inline constexpr std::size_t max_graph_bytes = std::numeric_limits<std::size_t>::max() / 2;
inline constexpr std::size_t max_head_dim = 256;  // S/kernels/attention.hpp:44

enum class tensor_role : std::uint8_t { input, intermediate, scratch };

struct tensor_desc {
    std::size_t bytes = 0;
    std::size_t size = 0;  // floats per row; 0 for scratch
    tensor_role role = tensor_role::intermediate;
    bool batched = true;   // max_batch rows, or one
};

// A KV cache layer kept across runs. bytes is the reference's unpadded size
// (S/graph/graph.hpp:707-716); the session places the device layout
// (syn_hip_kv_state_bytes) of each state after the planned arena.
struct state_desc {
    std::size_t bytes = 0;
    std::size_t max_ctx = 0;
    std::size_t n_kv_heads = 0;
    std::size_t head_dim = 0;
};

enum class rope_mode : std::uint8_t { normal, neox };  // S/kernels/attention.hpp:51-55

struct rope_scaling {  // S/kernels/attention.hpp:57-66
    float freq_scale = 1.0f;
    float ext_factor = 0.0f;
    float attn_factor = 1.0f;
    float corr_low = 0.0f;
    float corr_high = 0.0f;
};

struct op_rope {
    tensor_id in, out;
    std::size_t head_dim;
    float theta_scale;
    std::vector<float> freq_factors;  // empty, or head_dim / 2
    rope_mode mode;
    rope_scaling scaling;
};
struct op_attention {
    tensor_id q, k, v, out, scratch;
    state_id cache;
    std::size_t n_heads;
    float scale;
};
struct op_self_attention {
    tensor_id q, k, v, out;
    std::size_t n_heads;
    float scale;
};

using node = std::variant<op_rope, op_attention, op_self_attention>;

inline std::vector<tensor_id> operands(const node& n) {
    if (const auto* r = std::get_if<op_rope>(&n)) {
        return {r->in};
    }
    if (const auto* a = std::get_if<op_attention>(&n)) {
        return {a->q, a->k, a->v};
    }
    const auto& s = std::get<op_self_attention>(n);
    return {s.q, s.k, s.v};
}

inline std::vector<tensor_id> results(const node& n) {
    if (const auto* a = std::get_if<op_attention>(&n)) {
        return {a->out, a->scratch};
    }
    return {std::visit([](const auto& o) { return o.out; }, n)};
}

enum class graph_errc : std::uint32_t {  // S/graph/graph.hpp:388-398
    invalid_operand = 1,
    size_mismatch,
    empty_tensor,
    bad_output,
    no_outputs,
    too_large,
    bad_shape,
    bad_parameter,
    bad_state,
};

constexpr std::string_view to_string(graph_errc code) noexcept {
    switch (code) {
    case graph_errc::invalid_operand:
        return "invalid operand";
    case graph_errc::size_mismatch:
        return "operand sizes do not match";
    case graph_errc::empty_tensor:
        return "empty tensor";
    case graph_errc::bad_output:
        return "invalid graph output";
    case graph_errc::no_outputs:
        return "graph has no outputs";
    case graph_errc::too_large:
        return "graph tensors too large";
    case graph_errc::bad_shape:
        return "head layout does not fit the operation";
    case graph_errc::bad_parameter:
        return "invalid scalar parameter";
    case graph_errc::bad_state:
        return "invalid or reused state";
    }
    return "unknown error";
}

struct graph_error {
    graph_errc code;
    std::size_t node = 0;  // index of the node being added when the error occurred
};

// Value or error, no exceptions (the reference's result<T, E>, S/result.hpp:20-69).
template <typename T, typename E>
class result {
public:
    result(T value) : v_(std::in_place_index<0>, std::move(value)) {}
    result(E error) : v_(std::in_place_index<1>, std::move(error)) {}
    bool has_value() const noexcept {
        return v_.index() == 0;
    }
    explicit operator bool() const noexcept {
        return has_value();
    }
    T& value() & {
        return std::get<0>(v_);
    }
    const T& value() const& {
        return std::get<0>(v_);
    }
    T&& value() && {
        return std::get<0>(std::move(v_));
    }
    const E& error() const {
        return std::get<1>(v_);
    }

private:
    std::variant<T, E> v_;
};

class graph_builder;

class compute_graph {
public:
    const std::vector<tensor_desc>& tensors() const noexcept {
        return tensors_;
    }
    const std::vector<state_desc>& states() const noexcept {
        return states_;
    }
    const std::vector<node>& nodes() const noexcept {
        return nodes_;
    }
    const std::vector<tensor_id>& inputs() const noexcept {
        return inputs_;
    }
    const std::vector<tensor_id>& outputs() const noexcept {
        return outputs_;
    }
    // Positions a run accepts are < position_limit(): the smallest KV cache's max_ctx.
    std::size_t position_limit() const noexcept {
        return position_limit_;
    }
    std::size_t max_batch() const noexcept {
        return max_batch_;
    }
    std::size_t rows(tensor_id t) const noexcept {
        return tensors_[t].batched ? max_batch_ : 1;
    }

private:
    friend class graph_builder;
    compute_graph() = default;
    std::vector<tensor_desc> tensors_;
    std::vector<state_desc> states_;
    std::vector<node> nodes_;
    std::vector<tensor_id> inputs_;
    std::vector<tensor_id> outputs_;
    std::size_t position_limit_ = std::numeric_limits<std::size_t>::max();
    std::size_t max_batch_ = 1;
};

// Builds a graph one operation at a time; after the first error every call
// returns the invalid id and finalize() reports that error.
class graph_builder {
public:
    explicit graph_builder(std::size_t max_batch = 1) {
        if (max_batch == 0 || max_batch > std::numeric_limits<std::uint32_t>::max()) {
            fail(graph_errc::bad_shape);
        } else {
            g_.max_batch_ = max_batch;
        }
    }

    // A graph input of `size` floats per token (batched).
    tensor_id input(std::size_t size) {
        if (failed()) {
            return invalid_tensor;
        }
        if (size == 0) {
            return fail(graph_errc::empty_tensor);
        }
        const tensor_id t = add_floats(size, tensor_role::input);
        if (t != invalid_tensor) {
            g_.inputs_.push_back(t);
        }
        return t;
    }

    // Every head of x rotated by its token's position (S/kernels/attention.hpp:89-129).
    tensor_id rope(tensor_id x, std::size_t head_dim, float theta_scale, std::vector<float> freq_factors = {},
                   rope_mode mode = rope_mode::normal, rope_scaling scaling = {}) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (head_dim == 0 || head_dim % 2 != 0 || head_dim > max_head_dim || size_of(x) % head_dim != 0 ||
            !g_.tensors_[x].batched || (!freq_factors.empty() && freq_factors.size() != head_dim / 2)) {
            return fail(graph_errc::bad_shape);  // I6, I8
        }
        if (!std::isfinite(theta_scale) || theta_scale <= 0.0f || !std::isfinite(scaling.freq_scale) ||
            scaling.freq_scale <= 0.0f) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate);
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_rope{x, out, head_dim, theta_scale, std::move(freq_factors), mode, scaling});
        }
        return out;
    }

    // A KV cache layer of max_ctx positions (S/graph/graph.hpp:698-719).
    state_id kv_cache(std::size_t max_ctx, std::size_t n_kv_heads, std::size_t head_dim) {
        if (failed()) {
            return invalid_state;
        }
        if (max_ctx == 0 || n_kv_heads == 0 || head_dim == 0 || head_dim > max_head_dim ||
            max_ctx > std::size_t{std::numeric_limits<std::uint32_t>::max()}) {
            fail(graph_errc::bad_shape);
            return invalid_state;
        }
        constexpr std::size_t half = 2;
        const std::size_t limit = max_graph_bytes - state_bytes_;
        if (n_kv_heads > limit / head_dim || max_ctx > limit / (n_kv_heads * head_dim) / (2 * half)) {
            fail(graph_errc::too_large);  // I5
            return invalid_state;
        }
        const std::size_t bytes = 2 * half * max_ctx * n_kv_heads * head_dim;
        state_bytes_ += bytes;
        g_.states_.push_back(state_desc{bytes, max_ctx, n_kv_heads, head_dim});
        state_used_.push_back(false);
        return static_cast<state_id>(g_.states_.size() - 1);
    }

    // Append (k, v) to cache at the run's positions, then attend q, as
    // n_heads query heads, causally over the cache (S/graph/graph.hpp:727-761).
    tensor_id attention(tensor_id q, tensor_id k, tensor_id v, state_id cache, std::size_t n_heads, float scale) {
        if (!operand_ok(q) || !operand_ok(k) || !operand_ok(v)) {
            return invalid_tensor;
        }
        if (cache >= g_.states_.size() || state_used_[cache]) {
            return fail(graph_errc::bad_state);  // I7
        }
        const state_desc& c = g_.states_[cache];
        const std::size_t row = c.n_kv_heads * c.head_dim;
        if (n_heads == 0 || n_heads % c.n_kv_heads != 0 || n_heads > max_graph_bytes / c.head_dim ||
            size_of(q) != n_heads * c.head_dim || size_of(k) != row || size_of(v) != row || !batched(q) ||
            !batched(k) || !batched(v) || c.head_dim % 2 != 0) {
            return fail(graph_errc::bad_shape);  // I6, I8
        }
        if (!std::isfinite(scale) || scale <= 0.0f) {
            return fail(graph_errc::bad_parameter);
        }
        // The GPU decode kernel's split-KV partials (the reference sizes a
        // score row per head here, S/kernels/attention.hpp:147-161).
        const std::size_t scratch_bytes = syn_hip_attention_scratch_bytes(
            static_cast<uint32_t>(n_heads), static_cast<uint32_t>(c.n_kv_heads), static_cast<uint32_t>(c.head_dim),
            static_cast<uint32_t>(c.max_ctx), static_cast<uint32_t>(g_.max_batch_));
        const tensor_id out = add_floats(size_of(q), tensor_role::intermediate);
        const tensor_id scratch = add_tensor(std::max<std::size_t>(scratch_bytes, 1), 0, tensor_role::scratch, false);
        if (out == invalid_tensor || scratch == invalid_tensor) {
            return invalid_tensor;
        }
        state_used_[cache] = true;
        g_.position_limit_ = std::min(g_.position_limit_, c.max_ctx);
        g_.nodes_.emplace_back(op_attention{q, k, v, out, scratch, cache, n_heads, scale});
        return out;
    }

    // Bidirectional attention over the run's rows (S/graph/graph.hpp:831-863).
    tensor_id self_attention(tensor_id q, tensor_id k, tensor_id v, std::size_t n_heads, float scale) {
        if (!operand_ok(q) || !operand_ok(k) || !operand_ok(v)) {
            return invalid_tensor;
        }
        if (n_heads == 0 || size_of(q) % n_heads != 0 || size_of(k) != size_of(q) || size_of(v) != size_of(q) ||
            !batched(q) || !batched(k) || !batched(v) || size_of(q) / n_heads > max_head_dim) {
            return fail(graph_errc::bad_shape);  // I6, I8
        }
        if (!std::isfinite(scale) || scale <= 0.0f) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(q), tensor_role::intermediate);
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_self_attention{q, k, v, out, n_heads, scale});
        }
        return out;
    }

    // Marks t as a graph output (I4).
    void output(tensor_id t) {
        if (failed()) {
            return;
        }
        if (t >= g_.tensors_.size() || g_.tensors_[t].role == tensor_role::scratch ||
            std::find(g_.outputs_.begin(), g_.outputs_.end(), t) != g_.outputs_.end()) {
            fail(graph_errc::bad_output);
            return;
        }
        g_.outputs_.push_back(t);
    }

    result<compute_graph, graph_error> finalize() && {
        if (error_) {
            return graph_error{error_->first, error_->second};
        }
        if (g_.outputs_.empty()) {
            return graph_error{graph_errc::no_outputs, g_.nodes_.size()};
        }
        return std::move(g_);
    }

private:
    bool failed() const noexcept {
        return error_.has_value();
    }

    tensor_id fail(graph_errc code) {
        if (!error_) {
            error_ = std::pair{code, g_.nodes_.size()};
        }
        return invalid_tensor;
    }

    bool operand_ok(tensor_id t) {
        if (failed()) {
            return false;
        }
        if (t >= g_.tensors_.size() || g_.tensors_[t].role == tensor_role::scratch) {
            fail(graph_errc::invalid_operand);
            return false;
        }
        return true;
    }

    std::size_t size_of(tensor_id t) const noexcept {
        return g_.tensors_[t].size;
    }
    bool batched(tensor_id t) const noexcept {
        return g_.tensors_[t].batched;
    }

    tensor_id add_floats(std::size_t size, tensor_role role) {
        if (size > max_graph_bytes / sizeof(float) / g_.max_batch_) {
            return fail(graph_errc::too_large);
        }
        return add_tensor(size * sizeof(float) * g_.max_batch_, size, role, true);
    }

    tensor_id add_tensor(std::size_t bytes, std::size_t size, tensor_role role, bool batched) {
        const std::size_t aligned = (bytes + plan_alignment - 1) / plan_alignment * plan_alignment;
        if (bytes > max_graph_bytes || aligned > max_graph_bytes - tensor_bytes_) {
            return fail(graph_errc::too_large);  // I5
        }
        tensor_bytes_ += aligned;
        g_.tensors_.push_back(tensor_desc{bytes, size, role, batched});
        return static_cast<tensor_id>(g_.tensors_.size() - 1);
    }

    compute_graph g_;
    std::vector<bool> state_used_;
    std::size_t tensor_bytes_ = 0;
    std::size_t state_bytes_ = 0;
    std::optional<std::pair<graph_errc, std::size_t>> error_;
};

}  // namespace syn::graph
