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
    // Tokens a run accepts are < token_limit(): the smallest embedding
    // table's row count (unbounded without an embed node).
    std::size_t token_limit() const noexcept {
        return token_limit_;
    }
    // True if every run must process exactly max_batch() rows (a pixel_shuffle, I9).
    bool full_batch_only() const noexcept {
        return full_batch_only_;
    }
    // True if the graph has an embed node, so a run needs tokens.
    bool embeds() const noexcept {
        return embeds_;
    }
    // Rows a tensor holds: max_batch() / row_div if batched, else 1.
    std::size_t rows(tensor_id t) const noexcept {
        return tensors_[t].batched ? max_batch_ / tensors_[t].row_div : 1;
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
    std::size_t token_limit_ = std::numeric_limits<std::size_t>::max();
    std::size_t max_batch_ = 1;
    bool full_batch_only_ = false;
    bool embeds_ = false;
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

    // w * x (S/graph/graph.hpp:536-572). Pre (checked): x.size == cols(w);
    // w in a format the device computes with.
    tensor_id matmul(const matrix_ref& w, tensor_id x) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (size_of(x) != cols(w)) {
            return fail(graph_errc::size_mismatch);
        }
        if (!matrix_ok(w)) {
            return fail(graph_errc::bad_parameter);
        }
        // Quantized weights take their activations quantized once per run,
        // into this scratch (syn_hip_matmul_q_act_bytes for every row of x).
        const std::size_t n = g_.rows(x);
        std::size_t scratch_bytes = 1;
        if (type_of(w) != SYN_TYPE_F32) {
            if (n > std::numeric_limits<std::uint32_t>::max() || cols(w) > std::numeric_limits<std::uint32_t>::max()) {
                return fail(graph_errc::too_large);
            }
            scratch_bytes = syn_hip_matmul_q_act_bytes(type_of(w), static_cast<std::uint32_t>(n),
                                                       static_cast<std::uint32_t>(cols(w)));
        }
        const tensor_id out = add_floats(rows(w), tensor_role::intermediate, batched(x), row_div(x));
        const tensor_id scratch = add_tensor(scratch_bytes, 0, tensor_role::scratch, false);
        if (out == invalid_tensor || scratch == invalid_tensor) {
            return invalid_tensor;
        }
        g_.nodes_.emplace_back(op_matmul{w, x, out, scratch});
        return out;
    }

    tensor_id add(tensor_id a, tensor_id b) {
        return binary<op_add>(a, b);
    }
    tensor_id mul(tensor_id a, tensor_id b) {
        return binary<op_mul>(a, b);
    }

    // x + bias on every row. Pre (checked): bias is 1 x x.size (I2).
    tensor_id add_bias(tensor_id x, const matrix_ref& bias) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (rows(bias) != 1 || cols(bias) != size_of(x)) {
            return fail(graph_errc::size_mismatch);
        }
        if (!vector_ok(bias)) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, batched(x), row_div(x));
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_add_bias{x, bias, out});
        }
        return out;
    }
    tensor_id silu(tensor_id x) {
        return unary<op_silu>(x);
    }
    tensor_id softmax(tensor_id x) {
        return unary<op_softmax>(x);
    }

    // x / rms(x) * gamma. Pre (checked): gamma is 1 x x.size.
    tensor_id rms_norm(tensor_id x, const matrix_ref& gamma, float eps) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (rows(gamma) != 1 || cols(gamma) != size_of(x)) {
            return fail(graph_errc::size_mismatch);
        }
        if (!vector_ok(gamma)) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, batched(x), row_div(x));
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_rms_norm{x, gamma, eps, out});
        }
        return out;
    }

    // Row `token` of table for each token of a run. Pre (checked): table non-empty.
    tensor_id embed(const matrix_ref& table) {
        if (failed()) {
            return invalid_tensor;
        }
        if (rows(table) == 0 || cols(table) == 0) {
            return fail(graph_errc::empty_tensor);
        }
        if (!matrix_ok(table) || rows(table) > std::numeric_limits<std::uint32_t>::max()) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(cols(table), tensor_role::intermediate, true);
        if (out != invalid_tensor) {
            g_.token_limit_ = std::min(g_.token_limit_, rows(table));
            g_.embeds_ = true;
            g_.nodes_.emplace_back(op_embed{table, out});
        }
        return out;
    }

    // Every head of x rotated by its token's position, theta_i = pos *
    // base^(-2i / head_dim) / freq_factors[i] (S/graph/graph.hpp:642-676,
    // S/kernels/attention.hpp:89-129). Pre (checked): I6, I8; base and every
    // freq factor finite and positive; scaling's freq_scale and attn_factor
    // finite and positive, its ext_factor and correction dims finite.
    tensor_id rope(tensor_id x, std::size_t head_dim, float base, std::span<const float> freq_factors = {},
                   rope_mode mode = rope_mode::normal, const rope_scaling& scaling = {}) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (head_dim == 0 || head_dim % 2 != 0 || head_dim > max_head_dim || size_of(x) % head_dim != 0 ||
            !per_token(x) || (!freq_factors.empty() && freq_factors.size() != head_dim / 2)) {
            return fail(graph_errc::bad_shape);  // I6, I8
        }
        const auto positive = [](float f) { return std::isfinite(f) && f > 0.0f; };
        if (!positive(base) || !std::all_of(freq_factors.begin(), freq_factors.end(), positive) ||
            !positive(scaling.freq_scale) || !positive(scaling.attn_factor) || !std::isfinite(scaling.ext_factor) ||
            !std::isfinite(scaling.corr_low) || !std::isfinite(scaling.corr_high)) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, true);
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_rope{x, out, head_dim, rope_theta_scale(base, head_dim),
                                           std::vector<float>(freq_factors.begin(), freq_factors.end()), mode,
                                           scaling});
        }
        return out;
    }

    // x with each row scaled by its position's attention temperature,
    // 1 + scale * ln(floor(pos / floor_len) + 1) (S/graph/graph.hpp:678-696).
    // Pre (checked): I8; scale finite; floor_len >= 1.
    tensor_id attn_temperature(tensor_id x, float scale, std::size_t floor_len) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (!per_token(x)) {
            return fail(graph_errc::bad_shape);  // I8
        }
        if (!std::isfinite(scale) || floor_len == 0) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, true);
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_attn_temperature{x, out, scale, floor_len});
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
            size_of(q) != n_heads * c.head_dim || size_of(k) != row || size_of(v) != row || !per_token(q) ||
            !per_token(k) || !per_token(v) || c.head_dim % 2 != 0) {
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
            !per_token(q) || !per_token(k) || !per_token(v) || size_of(q) / n_heads > max_head_dim) {
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

    // Row n-1 of x for a run of n rows (S/graph/graph.hpp:765-781). Pre (checked): I8.
    tensor_id last_row(tensor_id x) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (!per_token(x)) {
            return fail(graph_errc::bad_shape);  // I8
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, false);
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_last_row{x, out});
        }
        return out;
    }

    // (x - mean) / sqrt(var + eps) * gamma (+ beta unless empty)
    // (S/graph/graph.hpp:783-800). Pre (checked): gamma, beta 1 x x.size;
    // eps finite and non-negative.
    tensor_id layer_norm(tensor_id x, const matrix_ref& gamma, const matrix_ref& beta, float eps) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        const bool has_beta = !std::holds_alternative<std::monostate>(beta);
        if (rows(gamma) != 1 || cols(gamma) != size_of(x) ||
            (has_beta && (rows(beta) != 1 || cols(beta) != size_of(x)))) {
            return fail(graph_errc::size_mismatch);
        }
        if (!std::isfinite(eps) || eps < 0.0f || !vector_ok(gamma) || (has_beta && !vector_ok(beta))) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, batched(x), row_div(x));
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_layer_norm{x, gamma, beta, eps, out});
        }
        return out;
    }

    tensor_id gelu(tensor_id x) {
        return unary<op_gelu>(x);
    }

    // x with row i of table added to its row i (S/graph/graph.hpp:809-829).
    // Pre (checked): I8; table has x.size columns and >= max_batch rows.
    tensor_id add_rows(tensor_id x, const matrix_ref& table) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (!per_token(x)) {
            return fail(graph_errc::bad_shape);  // I8
        }
        if (cols(table) != size_of(x) || rows(table) < g_.max_batch_) {
            return fail(graph_errc::size_mismatch);
        }
        if (!vector_ok(table)) {
            return fail(graph_errc::bad_parameter);
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, true);
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(op_add_rows{x, table, out});
        }
        return out;
    }

    // x's rows as a grid_w-wide patch grid, each s x s block of patches merged
    // into one row of s*s*x.size floats (S/graph/graph.hpp:872-896). Pre
    // (checked): I8, I9 (grid_w * grid_h == max_batch, both multiples of s >= 2).
    tensor_id pixel_shuffle(tensor_id x, std::size_t grid_w, std::size_t s) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        if (!per_token(x) || s < 2 || grid_w == 0 || g_.max_batch_ % grid_w != 0 || grid_w % s != 0 ||
            (g_.max_batch_ / grid_w) % s != 0) {
            return fail(graph_errc::bad_shape);  // I8, I9
        }
        if (size_of(x) > max_graph_bytes / (s * s)) {
            return fail(graph_errc::too_large);
        }
        const tensor_id out = add_floats(size_of(x) * s * s, tensor_role::intermediate, true, s * s);
        if (out != invalid_tensor) {
            g_.full_batch_only_ = true;
            g_.nodes_.emplace_back(op_pixel_shuffle{x, out, grid_w, s});
        }
        return out;
    }

    // Marks t as a graph output: kept until the end of a run (I4).
    void output(tensor_id t) {
        if (failed()) {
            return;
        }
        if (t >= g_.tensors_.size() || g_.tensors_[t].role == tensor_role::scratch ||
            g_.tensors_[t].role == tensor_role::output ||
            std::find(g_.outputs_.begin(), g_.outputs_.end(), t) != g_.outputs_.end()) {
            fail(graph_errc::bad_output);
            return;
        }
        if (g_.tensors_[t].role == tensor_role::intermediate) {
            g_.tensors_[t].role = tensor_role::output;
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
    std::size_t row_div(tensor_id t) const noexcept {
        return g_.tensors_[t].row_div;
    }
    // Batched with one row per run row: what per-token ops take (I8).
    bool per_token(tensor_id t) const noexcept {
        return batched(t) && row_div(t) == 1;
    }
    // A matrix in a device format, whole blocks per row, with data.
    static bool matrix_ok(const matrix_ref& m) noexcept {
        const auto* w = std::get_if<weight_view>(&m);
        return w != nullptr && w->data != nullptr && block_values(w->type) != 0 && w->cols % block_values(w->type) == 0;
    }
    // A 1 x size vector or table the device reads as floats.
    static bool vector_ok(const matrix_ref& m) noexcept {
        return matrix_ok(m) && type_of(m) == SYN_TYPE_F32;
    }

    template <typename Op>
    tensor_id binary(tensor_id a, tensor_id b) {
        if (!operand_ok(a) || !operand_ok(b)) {
            return invalid_tensor;
        }
        if (size_of(a) != size_of(b) || batched(a) != batched(b) || row_div(a) != row_div(b)) {
            return fail(graph_errc::size_mismatch);  // I2, I8
        }
        const tensor_id out = add_floats(size_of(a), tensor_role::intermediate, batched(a), row_div(a));
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(Op{a, b, out});
        }
        return out;
    }

    template <typename Op>
    tensor_id unary(tensor_id x) {
        if (!operand_ok(x)) {
            return invalid_tensor;
        }
        const tensor_id out = add_floats(size_of(x), tensor_role::intermediate, batched(x), row_div(x));
        if (out != invalid_tensor) {
            g_.nodes_.emplace_back(Op{x, out});
        }
        return out;
    }

    // A float tensor of `size` per row, max_batch / div rows if batched;
    // the one place a float tensor's byte count is computed (checked, I5).
    tensor_id add_floats(std::size_t size, tensor_role role, bool is_batched = true, std::size_t div = 1) {
        const std::size_t n = is_batched ? g_.max_batch_ / div : 1;
        if (size > max_graph_bytes / sizeof(float) / n) {
            return fail(graph_errc::too_large);
        }
        const tensor_id t = add_tensor(n * size * sizeof(float), size, role, is_batched);
        if (t != invalid_tensor) {
            g_.tensors_[t].row_div = is_batched ? div : 1;
        }
        return t;
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
