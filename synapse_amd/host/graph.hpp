// graph.hpp — C++20 host side of the attention path: the graph IR and its
// checked builder, mirroring branes-ai/synapse's graph API
// (S/ = sdk/include/branes/synapse/, S/graph/graph.hpp):
//   the node payloads (:215-295), operands/results (:316-385), graph_errc
//   codes (:388-398), compute_graph (:424-490) and graph_builder (:506-1010)
//   with every builder method the model builders call: input, matmul, add,
//   mul, add_bias, silu, softmax, rms_norm, embed, rope, attn_temperature,
//   kv_cache, attention, last_row, layer_norm, gelu, add_rows,
//   self_attention, pixel_shuffle, output, finalize; "first error wins" with
//   the node index (:919-928).
// Names, argument meanings and error codes are the reference's, so a model
// builder written against it (S/models/llama.hpp:454-481,
// S/models/clip.hpp:348-349) builds the same graph. What differs:
//   - matrix_ref is a view of host memory in GGUF layout (weight_view: a
//     ggml type, rows, cols, data) in place of the reference's mtl block
//     views; the session uploads what the graph binds once, at construction.
//     Formats: F32, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K for matmul and embed; F32
//     for the 1 x size vectors (bias, gamma, beta) and add_rows' table, which
//     the device kernels read as floats (bad_parameter otherwise).
//   - the scratch tensors hold what the GPU kernels need: split-KV partials
//     for decode, quantized activations for matmul, nothing for
//     self-attention.
//
// Invariants of a finalized graph (numbered as the reference's):
//   I1 node order is a topological order (operands exist before use);
//   I2 operand sizes fit their operation;
//   I3 every tensor is an input or the result (or scratch) of one node;
//   I4 at least one output, outputs distinct and not scratch;
//   I5 the sum of tensor bytes and of state bytes are each <= max_graph_bytes;
//   I6 head layouts fit: whole heads, even head_dim <= 256 for rope and
//      attention, query heads divide evenly among the KV heads;
//   I7 every KV state is read and written by at most one attention node;
//   I8 per-token ops (rope, attention, self_attention, attn_temperature,
//      last_row, add_rows, pixel_shuffle) take batched tensors of one row
//      per run row;
//   I9 a pixel_shuffle's grid is the whole batch: its result has one row per
//      s*s run rows (row_div), and the graph then runs full batches only.
#pragma once

#include "synapse_hip.h"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <optional>
#include <span>
#include <string_view>
#include <type_traits>
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

enum class tensor_role : std::uint8_t { input, intermediate, output, scratch };

struct tensor_desc {
    std::size_t bytes = 0;
    std::size_t size = 0;  // floats per row; 0 for scratch
    tensor_role role = tensor_role::intermediate;
    bool batched = true;      // max_batch / row_div rows, or one
    std::size_t row_div = 1;  // run rows per row: 1, or s*s below a pixel_shuffle (I9)
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

// A weight matrix in host memory: rows rows of cols values of a ggml type
// (SYN_TYPE_*), each row in that type's blocks, as a GGUF file stores it.
// The data must stay valid until a session has been constructed from the
// graph (the session copies it to the device then).
struct weight_view {
    std::uint32_t type = SYN_TYPE_F32;
    std::size_t rows = 0;
    std::size_t cols = 0;
    const void* data = nullptr;
};

// A weight matrix, or no matrix (monostate, the default: 0 x 0, which every
// builder check rejects), as S/graph/graph.hpp:141-151.
using matrix_ref = std::variant<std::monostate, weight_view>;

// Values and bytes per block of a format the device computes with; 0 for
// any other type.
constexpr std::size_t block_values(std::uint32_t type) noexcept {
    switch (type) {
    case SYN_TYPE_F32:
        return 1;
    case SYN_TYPE_Q4_0:
    case SYN_TYPE_Q5_0:
    case SYN_TYPE_Q8_0:
        return 32;
    case SYN_TYPE_Q4_K:
    case SYN_TYPE_Q6_K:
        return 256;
    default:
        return 0;
    }
}
constexpr std::size_t block_bytes(std::uint32_t type) noexcept {
    switch (type) {
    case SYN_TYPE_F32:
        return 4;
    case SYN_TYPE_Q4_0:
        return 18;
    case SYN_TYPE_Q5_0:
        return 22;
    case SYN_TYPE_Q8_0:
        return 34;
    case SYN_TYPE_Q4_K:
        return 144;
    case SYN_TYPE_Q6_K:
        return 210;
    default:
        return 0;
    }
}

// Rows and columns of m; 0 for the empty matrix.
inline std::size_t rows(const matrix_ref& m) noexcept {
    const auto* w = std::get_if<weight_view>(&m);
    return w ? w->rows : 0;
}
inline std::size_t cols(const matrix_ref& m) noexcept {
    const auto* w = std::get_if<weight_view>(&m);
    return w ? w->cols : 0;
}
// Bytes of one row and of the whole matrix; 0 for the empty matrix.
inline std::size_t row_bytes(const matrix_ref& m) noexcept {
    const auto* w = std::get_if<weight_view>(&m);
    return w && block_values(w->type) ? w->cols / block_values(w->type) * block_bytes(w->type) : 0;
}
inline std::size_t matrix_bytes(const matrix_ref& m) noexcept {
    return rows(m) * row_bytes(m);
}
inline std::uint32_t type_of(const matrix_ref& m) noexcept {
    const auto* w = std::get_if<weight_view>(&m);
    return w ? w->type : std::uint32_t{SYN_TYPE_F32};
}

enum class rope_mode : std::uint8_t { normal, neox };  // S/kernels/attention.hpp:51-55

struct rope_scaling {  // S/kernels/attention.hpp:57-66
    float freq_scale = 1.0f;
    float ext_factor = 0.0f;
    float attn_factor = 1.0f;
    float corr_low = 0.0f;
    float corr_high = 0.0f;
};

// base^(-2 / head_dim) in float (kernels::rope_theta_scale, S/kernels/attention.hpp:47-49).
inline float rope_theta_scale(float base, std::size_t head_dim) noexcept {
    return std::pow(base, -2.0f / static_cast<float>(head_dim));
}

// The node payloads (S/graph/graph.hpp:215-295).
struct op_matmul {  // out = w * in
    matrix_ref w;
    tensor_id in, out, scratch;
};
struct op_add {
    tensor_id a, b, out;
};
struct op_add_bias {  // bias (1 x size) added to every row
    tensor_id in;
    matrix_ref bias;
    tensor_id out;
};
struct op_mul {
    tensor_id a, b, out;
};
struct op_silu {
    tensor_id in, out;
};
struct op_softmax {
    tensor_id in, out;
};
struct op_rms_norm {
    tensor_id in;
    matrix_ref gamma;
    float eps;
    tensor_id out;
};
struct op_embed {  // out row i = table row tokens[i]
    matrix_ref table;
    tensor_id out;
};
struct op_rope {
    tensor_id in, out;
    std::size_t head_dim;
    float theta_scale;                // base^(-2 / head_dim)
    std::vector<float> freq_factors;  // empty, or head_dim / 2
    rope_mode mode;
    rope_scaling scaling;
};
struct op_attn_temperature {  // row i times 1 + scale * ln(floor(pos_i / floor_len) + 1)
    tensor_id in, out;
    float scale;
    std::size_t floor_len;
};
struct op_attention {
    tensor_id q, k, v, out, scratch;
    state_id cache;
    std::size_t n_heads;
    float scale;
};
struct op_last_row {
    tensor_id in, out;
};
struct op_layer_norm {
    tensor_id in;
    matrix_ref gamma;
    matrix_ref beta;  // or empty
    float eps;
    tensor_id out;
};
struct op_gelu {
    tensor_id in, out;
};
struct op_add_rows {  // out row i = in row i + table row i
    tensor_id in;
    matrix_ref table;
    tensor_id out;
};
struct op_self_attention {
    tensor_id q, k, v, out;
    std::size_t n_heads;
    float scale;
};
struct op_pixel_shuffle {
    tensor_id in, out;
    std::size_t grid_w;
    std::size_t scale;
};

using node = std::variant<op_matmul, op_add, op_add_bias, op_mul, op_silu, op_softmax, op_rms_norm, op_embed, op_rope,
                          op_attn_temperature, op_attention, op_last_row, op_layer_norm, op_gelu, op_add_rows,
                          op_self_attention, op_pixel_shuffle>;

// Operand (read) tensors of a node.
inline std::vector<tensor_id> operands(const node& n) {
    return std::visit(
        [](const auto& o) -> std::vector<tensor_id> {
            using T = std::decay_t<decltype(o)>;
            if constexpr (std::is_same_v<T, op_add> || std::is_same_v<T, op_mul>) {
                return {o.a, o.b};
            } else if constexpr (std::is_same_v<T, op_attention> || std::is_same_v<T, op_self_attention>) {
                return {o.q, o.k, o.v};
            } else if constexpr (std::is_same_v<T, op_embed>) {
                return {};
            } else {
                return {o.in};
            }
        },
        n);
}

// Tensors a node writes: its result, and its scratch if it has one.
inline std::vector<tensor_id> results(const node& n) {
    if (const auto* m = std::get_if<op_matmul>(&n)) {
        return {m->out, m->scratch};
    }
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

// A tensor's row layout: floats per row, whether it has a row per run row
// (batched) or a single row, and how many run rows share one of its rows
// (row_div: 1, or s*s below a pixel_shuffle).
struct row_layout {
    std::size_t size = 0;
    bool batched = true;
    std::size_t row_div = 1;

    static constexpr row_layout per_run_row(std::size_t size) noexcept {
        return {size, true, 1};
    }
    static constexpr row_layout one_row(std::size_t size) noexcept {
        return {size, false, 1};
    }
    constexpr row_layout with_size(std::size_t s) const noexcept {
        return {s, batched, row_div};
    }
    // What per-token operations take (I8).
    constexpr bool per_token() const noexcept {
        return batched && row_div == 1;
    }
    constexpr bool operator==(const row_layout&) const = default;
};

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
    // A run's positions stay below this: the smallest KV cache's max_ctx.
    std::size_t position_limit() const noexcept {
        return limits_.positions;
    }
    std::size_t max_batch() const noexcept {
        return limits_.batch;
    }
    // A run's tokens stay below this: the smallest embedding table's row
    // count (unbounded without an embed node).
    std::size_t token_limit() const noexcept {
        return limits_.tokens;
    }
    // Every run processes exactly max_batch() rows (the graph has a pixel_shuffle, I9).
    bool full_batch_only() const noexcept {
        return limits_.whole_batches;
    }
    // A run needs tokens (the graph has an embed node).
    bool embeds() const noexcept {
        return limits_.takes_tokens;
    }
    // Rows of tensor t: max_batch() / row_div when batched, else one.
    std::size_t rows(tensor_id t) const noexcept {
        const tensor_desc& d = tensors_[t];
        return d.batched ? limits_.batch / d.row_div : 1;
    }

private:
    friend class graph_builder;
    struct run_limits {
        std::size_t batch = 1;
        std::size_t positions = std::numeric_limits<std::size_t>::max();
        std::size_t tokens = std::numeric_limits<std::size_t>::max();
        bool whole_batches = false;
        bool takes_tokens = false;
    };
    compute_graph() = default;
    std::vector<tensor_desc> tensors_;
    std::vector<state_desc> states_;
    std::vector<node> nodes_;
    std::vector<tensor_id> inputs_;
    std::vector<tensor_id> outputs_;
    run_limits limits_;
};

// Builds a graph one operation at a time. Each operation validates its
// operand ids, then applies its own shape and parameter rules in a fixed
// order (so a misuse reports the reference's code), then sizes its result
// (and scratch) against the byte budget (I5). The first failure latches:
// every later call returns the invalid id, and finalize() reports the code
// with the index of the node that was being added.
class graph_builder {
public:
    // Rule: max_batch >= 1 (bad_shape). A batch too large for any tensor
    // fails later, at the first tensor (too_large).
    explicit graph_builder(std::size_t max_batch = 1) {
        if (max_batch == 0) {
            latch_.set(graph_errc::bad_shape, 0);
        } else {
            graph_.limits_.batch = max_batch;
        }
    }

    // A graph input of `size` floats per run row.
    tensor_id input(std::size_t size) {
        if (latch_.set_already()) {
            return invalid_tensor;
        }
        if (size == 0) {
            return reject(graph_errc::empty_tensor);
        }
        const tensor_id t = new_rows(row_layout::per_run_row(size), tensor_role::input);
        if (t != invalid_tensor) {
            graph_.inputs_.push_back(t);
        }
        return t;
    }

    // w * x for every row of x (S/graph/graph.hpp:536-572). Rules: x has
    // cols(w) floats; w is in a format the device computes with. Block-format
    // weights take their activations quantized once per run, into a scratch
    // the library sizes (syn_hip_matmul_q_act_bytes).
    tensor_id matmul(const matrix_ref& w, tensor_id x) {
        return emit(
            {x},
            [&]() -> finding {
                if (shape(x).size != cols(w)) {
                    return graph_errc::size_mismatch;
                }
                return device_matrix(w) ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return shape(x).with_size(rows(w)); },
            [&](tensor_id out, tensor_id scratch) { return op_matmul{w, x, out, scratch}; },
            [&]() -> std::optional<std::size_t> {
                if (type_of(w) == SYN_TYPE_F32) {
                    return std::size_t{1};
                }
                const std::size_t n = graph_.rows(x);
                if (n > std::numeric_limits<std::uint32_t>::max() || cols(w) > std::numeric_limits<std::uint32_t>::max()) {
                    return std::nullopt;
                }
                return static_cast<std::size_t>(syn_hip_matmul_q_act_bytes(
                    type_of(w), static_cast<std::uint32_t>(n), static_cast<std::uint32_t>(cols(w))));
            });
    }

    tensor_id add(tensor_id a, tensor_id b) {
        return elementwise2(a, b, [](tensor_id x, tensor_id y, tensor_id out) { return op_add{x, y, out}; });
    }
    tensor_id mul(tensor_id a, tensor_id b) {
        return elementwise2(a, b, [](tensor_id x, tensor_id y, tensor_id out) { return op_mul{x, y, out}; });
    }

    // x + bias on every row. Rule: bias is a 1 x size float vector (I2).
    tensor_id add_bias(tensor_id x, const matrix_ref& bias) {
        return emit(
            {x}, [&] { return vector_rule(bias, shape(x).size); }, [&] { return shape(x); },
            [&](tensor_id out) { return op_add_bias{x, bias, out}; });
    }
    tensor_id silu(tensor_id x) {
        return elementwise1(x, [](tensor_id in, tensor_id out) { return op_silu{in, out}; });
    }
    tensor_id softmax(tensor_id x) {
        return elementwise1(x, [](tensor_id in, tensor_id out) { return op_softmax{in, out}; });
    }
    tensor_id gelu(tensor_id x) {
        return elementwise1(x, [](tensor_id in, tensor_id out) { return op_gelu{in, out}; });
    }

    // x / rms(x) * gamma. Rule: gamma is a 1 x size float vector.
    tensor_id rms_norm(tensor_id x, const matrix_ref& gamma, float eps) {
        return emit(
            {x}, [&] { return vector_rule(gamma, shape(x).size); }, [&] { return shape(x); },
            [&](tensor_id out) { return op_rms_norm{x, gamma, eps, out}; });
    }

    // Row `token` of table for each token of a run. Rule: the table is
    // non-empty, in a device format, with at most 2^32 - 1 rows.
    tensor_id embed(const matrix_ref& table) {
        return emit(
            {},
            [&]() -> finding {
                if (rows(table) == 0 || cols(table) == 0) {
                    return graph_errc::empty_tensor;
                }
                if (!device_matrix(table) || rows(table) > std::numeric_limits<std::uint32_t>::max()) {
                    return graph_errc::bad_parameter;
                }
                return ok;
            },
            [&] { return row_layout::per_run_row(cols(table)); },
            [&](tensor_id out) {
                graph_.limits_.tokens = std::min(graph_.limits_.tokens, rows(table));
                graph_.limits_.takes_tokens = true;
                return op_embed{table, out};
            });
    }

    // Every head of x rotated by its token's position, theta_i = pos *
    // base^(-2i / head_dim) / freq_factors[i] (S/graph/graph.hpp:642-676,
    // S/kernels/attention.hpp:89-129). Rules: whole even heads of at most 256
    // on a per-token x, freq_factors empty or head_dim / 2 long (I6, I8);
    // then base, the factors, freq_scale and attn_factor finite and positive,
    // ext_factor and the correction dims finite.
    tensor_id rope(tensor_id x, std::size_t head_dim, float base, std::span<const float> freq_factors = {},
                   rope_mode mode = rope_mode::normal, const rope_scaling& scaling = {}) {
        return emit(
            {x},
            [&]() -> finding {
                const row_layout l = shape(x);
                const bool heads_fit = head_dim != 0 && head_dim % 2 == 0 && head_dim <= max_head_dim &&
                                       l.size % head_dim == 0;
                const bool factors_fit = freq_factors.empty() || freq_factors.size() == head_dim / 2;
                if (!heads_fit || !l.per_token() || !factors_fit) {
                    return graph_errc::bad_shape;
                }
                const bool params_ok = positive(base) && std::all_of(freq_factors.begin(), freq_factors.end(), positive) &&
                                       positive(scaling.freq_scale) && positive(scaling.attn_factor) &&
                                       std::isfinite(scaling.ext_factor) && std::isfinite(scaling.corr_low) &&
                                       std::isfinite(scaling.corr_high);
                return params_ok ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return row_layout::per_run_row(shape(x).size); },
            [&](tensor_id out) {
                return op_rope{x, out, head_dim, rope_theta_scale(base, head_dim),
                               std::vector<float>(freq_factors.begin(), freq_factors.end()), mode, scaling};
            });
    }

    // x with each row scaled by its position's attention temperature,
    // 1 + scale * ln(floor(pos / floor_len) + 1) (S/graph/graph.hpp:678-696).
    // Rules: per-token x (I8); then scale finite, floor_len >= 1.
    tensor_id attn_temperature(tensor_id x, float scale, std::size_t floor_len) {
        return emit(
            {x},
            [&]() -> finding {
                if (!shape(x).per_token()) {
                    return graph_errc::bad_shape;
                }
                return std::isfinite(scale) && floor_len != 0 ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return row_layout::per_run_row(shape(x).size); },
            [&](tensor_id out) { return op_attn_temperature{x, out, scale, floor_len}; });
    }

    // A KV cache layer of max_ctx positions (S/graph/graph.hpp:698-719).
    // Rules: non-zero sizes, head_dim <= 256, max_ctx at most 2^32 (a 32-bit
    // position count); then its K and V halves within the state budget (I5).
    state_id kv_cache(std::size_t max_ctx, std::size_t n_kv_heads, std::size_t head_dim) {
        if (latch_.set_already()) {
            return invalid_state;
        }
        constexpr std::size_t positions = std::size_t{1} << 32;
        if (max_ctx == 0 || n_kv_heads == 0 || head_dim == 0 || head_dim > max_head_dim || max_ctx > positions) {
            reject(graph_errc::bad_shape);
            return invalid_state;
        }
        // K and V, each max_ctx x n_kv_heads x head_dim binary16 values.
        const wide bytes = wide{2} * sizeof(std::uint16_t) * max_ctx * n_kv_heads * head_dim;
        if (bytes > max_graph_bytes - state_budget_used_) {
            reject(graph_errc::too_large);
            return invalid_state;
        }
        state_budget_used_ += static_cast<std::size_t>(bytes);
        graph_.states_.push_back(state_desc{static_cast<std::size_t>(bytes), max_ctx, n_kv_heads, head_dim});
        cache_taken_.push_back(0);
        return static_cast<state_id>(graph_.states_.size() - 1);
    }

    // Append (k, v) to the cache at the run's positions, then attend q, as
    // n_heads query heads, causally over it (S/graph/graph.hpp:727-761).
    // Rules: the cache exists and no other attention uses it (I7); whole heads
    // -- q n_heads x head_dim, k and v n_kv_heads x head_dim, n_heads a
    // multiple of n_kv_heads, an even head_dim -- on per-token tensors (I6,
    // I8); a finite, positive scale. The scratch holds the GPU decode's
    // split-KV partials (the reference sizes a score row per head here,
    // S/kernels/attention.hpp:147-161).
    tensor_id attention(tensor_id q, tensor_id k, tensor_id v, state_id cache, std::size_t n_heads, float scale) {
        return emit(
            {q, k, v},
            [&]() -> finding {
                if (cache >= graph_.states_.size() || cache_taken_[cache]) {
                    return graph_errc::bad_state;
                }
                const state_desc& c = graph_.states_[cache];
                const std::size_t kv_size = c.n_kv_heads * c.head_dim;
                const bool heads_fit = n_heads != 0 && n_heads % c.n_kv_heads == 0 &&
                                       n_heads <= max_graph_bytes / c.head_dim && c.head_dim % 2 == 0 &&
                                       shape(q).size == n_heads * c.head_dim && shape(k).size == kv_size &&
                                       shape(v).size == kv_size;
                if (!heads_fit || !shape(q).per_token() || !shape(k).per_token() || !shape(v).per_token()) {
                    return graph_errc::bad_shape;
                }
                return positive(scale) ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return row_layout::per_run_row(shape(q).size); },
            [&](tensor_id out, tensor_id scratch) {
                cache_taken_[cache] = 1;
                graph_.limits_.positions = std::min(graph_.limits_.positions, graph_.states_[cache].max_ctx);
                return op_attention{q, k, v, out, scratch, cache, n_heads, scale};
            },
            [&]() -> std::optional<std::size_t> {
                const state_desc& c = graph_.states_[cache];
                const auto u32 = [](std::size_t x) { return static_cast<std::uint32_t>(x); };
                return std::max<std::size_t>(
                    syn_hip_attention_scratch_bytes(u32(n_heads), u32(c.n_kv_heads), u32(c.head_dim),
                                                    u32(std::min<std::size_t>(c.max_ctx, 0xFFFFFFFFu)),
                                                    u32(graph_.limits_.batch)),
                    1);
            });
    }

    // Bidirectional attention over the run's rows (S/graph/graph.hpp:831-863).
    // Rules: q, k, v of one size, whole heads of at most 256, per-token
    // (I6, I8); a finite, positive scale.
    tensor_id self_attention(tensor_id q, tensor_id k, tensor_id v, std::size_t n_heads, float scale) {
        return emit(
            {q, k, v},
            [&]() -> finding {
                const std::size_t size = shape(q).size;
                const bool heads_fit = n_heads != 0 && size % n_heads == 0 && size / n_heads <= max_head_dim &&
                                       shape(k).size == size && shape(v).size == size;
                if (!heads_fit || !shape(q).per_token() || !shape(k).per_token() || !shape(v).per_token()) {
                    return graph_errc::bad_shape;
                }
                return positive(scale) ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return row_layout::per_run_row(shape(q).size); },
            [&](tensor_id out) { return op_self_attention{q, k, v, out, n_heads, scale}; });
    }

    // Row n-1 of x for a run of n rows (S/graph/graph.hpp:765-781). Rule: per-token x (I8).
    tensor_id last_row(tensor_id x) {
        return emit(
            {x}, [&] { return shape(x).per_token() ? ok : finding{graph_errc::bad_shape}; },
            [&] { return row_layout::one_row(shape(x).size); },
            [&](tensor_id out) { return op_last_row{x, out}; });
    }

    // (x - mean) / sqrt(var + eps) * gamma (+ beta unless empty)
    // (S/graph/graph.hpp:783-800). Rules: gamma (and beta) 1 x size; then eps
    // finite and non-negative, both float vectors.
    tensor_id layer_norm(tensor_id x, const matrix_ref& gamma, const matrix_ref& beta, float eps) {
        return emit(
            {x},
            [&]() -> finding {
                const std::size_t size = shape(x).size;
                const bool has_beta = !std::holds_alternative<std::monostate>(beta);
                const auto is_row = [&](const matrix_ref& m) { return rows(m) == 1 && cols(m) == size; };
                if (!is_row(gamma) || (has_beta && !is_row(beta))) {
                    return graph_errc::size_mismatch;
                }
                const bool ok_params = std::isfinite(eps) && eps >= 0.0f && float_vector(gamma) &&
                                       (!has_beta || float_vector(beta));
                return ok_params ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return shape(x); }, [&](tensor_id out) { return op_layer_norm{x, gamma, beta, eps, out}; });
    }

    // x with row i of table added to its row i (S/graph/graph.hpp:809-829).
    // Rules: per-token x (I8); the table x.size wide with at least max_batch
    // rows; a float table.
    tensor_id add_rows(tensor_id x, const matrix_ref& table) {
        return emit(
            {x},
            [&]() -> finding {
                if (!shape(x).per_token()) {
                    return graph_errc::bad_shape;
                }
                if (cols(table) != shape(x).size || rows(table) < graph_.limits_.batch) {
                    return graph_errc::size_mismatch;
                }
                return float_vector(table) ? ok : finding{graph_errc::bad_parameter};
            },
            [&] { return row_layout::per_run_row(shape(x).size); },
            [&](tensor_id out) { return op_add_rows{x, table, out}; });
    }

    // x's rows as a grid_w-wide patch grid, each s x s block of patches merged
    // into one row of s*s*x.size floats (S/graph/graph.hpp:872-896). Rules:
    // per-token x, s >= 2, a grid of max_batch patches whose sides are
    // multiples of s (I8, I9); the merged row within the budget.
    tensor_id pixel_shuffle(tensor_id x, std::size_t grid_w, std::size_t s) {
        return emit(
            {x},
            [&]() -> finding {
                const std::size_t n = graph_.limits_.batch;
                const bool grid_fits = s >= 2 && grid_w != 0 && n % grid_w == 0 && grid_w % s == 0 &&
                                       (n / grid_w) % s == 0;
                if (!shape(x).per_token() || !grid_fits) {
                    return graph_errc::bad_shape;
                }
                return wide{shape(x).size} * s * s > max_graph_bytes ? finding{graph_errc::too_large} : ok;
            },
            [&] { return row_layout{shape(x).size * s * s, true, s * s}; },
            [&](tensor_id out) {
                graph_.limits_.whole_batches = true;
                return op_pixel_shuffle{x, out, grid_w, s};
            });
    }

    // Marks t as a graph output, kept until the end of a run (I4). Rule: an
    // existing, non-scratch tensor not already an output.
    void output(tensor_id t) {
        if (latch_.set_already()) {
            return;
        }
        const auto& outs = graph_.outputs_;
        if (t >= graph_.tensors_.size() || graph_.tensors_[t].role == tensor_role::scratch ||
            std::find(outs.begin(), outs.end(), t) != outs.end()) {
            reject(graph_errc::bad_output);
            return;
        }
        tensor_desc& d = graph_.tensors_[t];
        if (d.role == tensor_role::intermediate) {
            d.role = tensor_role::output;
        }
        graph_.outputs_.push_back(t);
    }

    result<compute_graph, graph_error> finalize() && {
        if (latch_.set_already()) {
            return latch_.error();
        }
        if (graph_.outputs_.empty()) {
            return graph_error{graph_errc::no_outputs, graph_.nodes_.size()};
        }
        return std::move(graph_);
    }

private:
    using wide = unsigned __int128;
    // A rule's finding: no error, or the code the operation fails with.
    using finding = std::optional<graph_errc>;
    static constexpr finding ok{};

    // The first error and the node it happened at; later calls are no-ops.
    class latch {
    public:
        void set(graph_errc code, std::size_t node) {
            if (!first_) {
                first_ = graph_error{code, node};
            }
        }
        bool set_already() const noexcept {
            return first_.has_value();
        }
        graph_error error() const {
            return *first_;
        }

    private:
        std::optional<graph_error> first_;
    };

    static bool positive(float f) noexcept {
        return std::isfinite(f) && f > 0.0f;
    }
    // A matrix in a device format, whole blocks per row, with data.
    static bool device_matrix(const matrix_ref& m) noexcept {
        const auto* w = std::get_if<weight_view>(&m);
        return w != nullptr && w->data != nullptr && block_values(w->type) != 0 && w->cols % block_values(w->type) == 0;
    }
    // A matrix the device reads as floats (biases, gammas, position tables).
    static bool float_vector(const matrix_ref& m) noexcept {
        return device_matrix(m) && type_of(m) == SYN_TYPE_F32;
    }
    // A 1 x size float vector: size_mismatch first, then bad_parameter.
    static finding vector_rule(const matrix_ref& m, std::size_t size) noexcept {
        if (rows(m) != 1 || cols(m) != size) {
            return graph_errc::size_mismatch;
        }
        return float_vector(m) ? ok : finding{graph_errc::bad_parameter};
    }

    tensor_id reject(graph_errc code) {
        latch_.set(code, graph_.nodes_.size());
        return invalid_tensor;
    }

    row_layout shape(tensor_id t) const noexcept {
        const tensor_desc& d = graph_.tensors_[t];
        return row_layout{d.size, d.batched, d.row_div};
    }

    // Operand ids: each an existing tensor that is not a node's scratch.
    bool usable(std::initializer_list<tensor_id> ids) {
        if (latch_.set_already()) {
            return false;
        }
        for (const tensor_id t : ids) {
            if (t >= graph_.tensors_.size() || graph_.tensors_[t].role == tensor_role::scratch) {
                reject(graph_errc::invalid_operand);
                return false;
            }
        }
        return true;
    }

    // A tensor within the budget (I5): `bytes` (a float tensor's, or a
    // scratch's) rounded up to plan_alignment; too_large past it.
    tensor_id new_tensor(wide bytes, std::size_t size, tensor_role role, bool batched, std::size_t row_div) {
        const wide rounded = (bytes + plan_alignment - 1) / plan_alignment * plan_alignment;
        if (bytes > max_graph_bytes || rounded > max_graph_bytes - tensor_budget_used_) {
            return reject(graph_errc::too_large);
        }
        tensor_budget_used_ += static_cast<std::size_t>(rounded);
        graph_.tensors_.push_back(tensor_desc{static_cast<std::size_t>(bytes), size, role, batched, row_div});
        return static_cast<tensor_id>(graph_.tensors_.size() - 1);
    }
    tensor_id new_rows(const row_layout& l, tensor_role role) {
        const std::size_t n = l.batched ? graph_.limits_.batch / l.row_div : 1;
        return new_tensor(wide{l.size} * sizeof(float) * n, l.size, role, l.batched, l.batched ? l.row_div : 1);
    }

    // One operation: operand ids, its rules, then its result (and scratch,
    // when `scratch_bytes` is given; nullopt from it is too_large) and node.
    struct no_scratch {};
    template <class Rule, class Layout, class Make, class Scratch = no_scratch>
    tensor_id emit(std::initializer_list<tensor_id> ids, Rule&& rule, Layout&& layout, Make&& make,
                   Scratch&& scratch_bytes = {}) {
        if (!usable(ids)) {
            return invalid_tensor;
        }
        if (const finding f = rule()) {
            return reject(*f);
        }
        const tensor_id out = new_rows(layout(), tensor_role::intermediate);
        if (out == invalid_tensor) {
            return invalid_tensor;
        }
        if constexpr (std::is_same_v<std::decay_t<Scratch>, no_scratch>) {
            graph_.nodes_.emplace_back(make(out));
        } else {
            const std::optional<std::size_t> bytes = scratch_bytes();
            if (!bytes) {
                return reject(graph_errc::too_large);
            }
            const tensor_id scratch = new_tensor(*bytes, 0, tensor_role::scratch, false, 1);
            if (scratch == invalid_tensor) {
                return invalid_tensor;
            }
            graph_.nodes_.emplace_back(make(out, scratch));
        }
        return out;
    }

    // Same-layout element-wise operations (I2, I8: batching must agree).
    template <class Make>
    tensor_id elementwise2(tensor_id a, tensor_id b, Make&& make) {
        return emit(
            {a, b}, [&] { return shape(a) == shape(b) ? ok : finding{graph_errc::size_mismatch}; },
            [&] { return shape(a); }, [&](tensor_id out) { return make(a, b, out); });
    }
    template <class Make>
    tensor_id elementwise1(tensor_id x, Make&& make) {
        return emit({x}, [] { return ok; }, [&] { return shape(x); }, [&](tensor_id out) { return make(x, out); });
    }

    compute_graph graph_;
    latch latch_;
    std::vector<unsigned char> cache_taken_;  // per state: used by an attention node (I7)
    std::size_t tensor_budget_used_ = 0;      // rounded tensor bytes so far (I5)
    std::size_t state_budget_used_ = 0;       // state bytes so far (I5)
};

}  // namespace syn::graph
