// session.hpp — executes a compute_graph on one MI355X through the C ABI
// (include/synapse_hip.h). The reference's session (S/graph/session.hpp:
// 82-467) owns a host arena laid out by the static plan plus the KV states;
// this one owns a device arena laid out the same way:
//
//   [ planned tensors: plan(g), 256-byte aligned ][ bound weights ]
//   [ RoPE frequency tables ][ KV state 0 ][ KV state 1 ] ...
//
// one syn_hip_arena_create at construction, which also copies every matrix
// the graph binds (each distinct host matrix once), and nothing allocated
// afterwards. run(batch) keeps the reference's contract (:143-177): it
// returns false and runs nothing unless 1 <= n <= max_batch (n == max_batch
// for a pixel-shuffle graph), pos + n <= position_limit and every token <
// token_limit; otherwise it executes every node in graph order on the
// arena's stream, each through its C-ABI call (execute(op_*), :287-453).
// Inputs are written and outputs read with write()/read(), the device
// counterparts of tensor(t) (:107-110). A HIP failure during a run stops
// it, returns false and is kept in status().
//
// One fusion: a layer's op_rope(q), op_rope(k), op_attn_temperature(q) and
// op_attention run as one syn_hip_attention_rope call, which a decode step
// makes one kernel (the RoPE and temperature nodes are skipped; the RoPE
// inputs stay live in the memory plan up to the attention).
#pragma once

#include "graph.hpp"
#include "planner.hpp"

#include <array>
#include <cmath>
#include <limits>
#include <optional>
#include <span>
#include <unordered_map>

namespace syn::graph {

struct step {  // S/graph/session.hpp: one token at a position
    std::uint32_t token = 0;
    std::uint32_t pos = 0;
};

struct batch {  // tokens.size() consecutive tokens, the first at pos
    std::span<const std::uint32_t> tokens;
    std::uint32_t pos = 0;
};

// An op_attention whose q is op_rope's result (directly, or through
// op_attn_temperature) and whose k is op_rope's result, with those results
// read by nothing else and not graph outputs, both rotations alike and of
// the cache's head size: the nodes folded into it.
struct rope_fold {
    static constexpr std::size_t none = ~std::size_t{0};
    std::size_t rope_q = none;
    std::size_t rope_k = none;
    std::size_t temperature = none;
};

inline bool same_rotation(const op_rope& a, const op_rope& b) noexcept {
    return a.head_dim == b.head_dim && a.theta_scale == b.theta_scale && a.mode == b.mode &&
           a.freq_factors == b.freq_factors && a.scaling.freq_scale == b.scaling.freq_scale &&
           a.scaling.ext_factor == b.scaling.ext_factor && a.scaling.attn_factor == b.scaling.attn_factor &&
           a.scaling.corr_low == b.scaling.corr_low && a.scaling.corr_high == b.scaling.corr_high;
}

// Per node: its fold if it is such an attention.
inline std::vector<std::optional<rope_fold>> find_rope_folds(const compute_graph& g) {
    const auto& nodes = g.nodes();
    const std::size_t n_t = g.tensors().size();
    std::vector<std::size_t> producer(n_t, rope_fold::none);
    std::vector<std::size_t> readers(n_t, 0);
    for (std::size_t i = 0; i < nodes.size(); ++i) {
        for (tensor_id t : results(nodes[i])) {
            producer[t] = i;
        }
        for (tensor_id t : operands(nodes[i])) {
            ++readers[t];
        }
    }
    for (tensor_id t : g.outputs()) {
        ++readers[t];  // an output is read by the caller
    }
    const auto only_for = [&](tensor_id t) { return t < n_t && readers[t] == 1 && producer[t] != rope_fold::none; };
    std::vector<std::optional<rope_fold>> folds(nodes.size());
    for (std::size_t i = 0; i < nodes.size(); ++i) {
        const auto* a = std::get_if<op_attention>(&nodes[i]);
        if (a == nullptr || !only_for(a->q) || !only_for(a->k)) {
            continue;
        }
        rope_fold f;
        std::size_t q_src = producer[a->q];
        if (const auto* t = std::get_if<op_attn_temperature>(&nodes[q_src])) {
            if (!only_for(t->in) || t->floor_len == 0 || t->floor_len > std::numeric_limits<std::uint32_t>::max()) {
                continue;
            }
            f.temperature = q_src;
            q_src = producer[t->in];
        }
        const auto* rq = std::get_if<op_rope>(&nodes[q_src]);
        const auto* rk = std::get_if<op_rope>(&nodes[producer[a->k]]);
        if (rq == nullptr || rk == nullptr || !same_rotation(*rq, *rk) ||
            rq->head_dim != g.states()[a->cache].head_dim) {
            continue;
        }
        f.rope_q = q_src;
        f.rope_k = producer[a->k];
        folds[i] = f;
    }
    return folds;
}

// liveness(g) with each folded RoPE input kept up to its attention.
inline std::vector<live_interval> liveness_with_folds(const compute_graph& g,
                                                      const std::vector<std::optional<rope_fold>>& folds) {
    auto live = liveness(g);
    for (std::size_t i = 0; i < folds.size(); ++i) {
        if (folds[i]) {
            for (std::size_t r : {folds[i]->rope_q, folds[i]->rope_k}) {
                const tensor_id in = std::get<op_rope>(g.nodes()[r]).in;
                live[in].last = std::max(live[in].last, i);
            }
        }
    }
    return live;
}

class session {
public:
    explicit session(const compute_graph& g)
        : graph_(&g), folds_(find_rope_folds(g)), plan_(plan(g, liveness_with_folds(g, folds_))) {
        folded_.assign(g.nodes().size(), false);
        for (const auto& f : folds_) {
            if (f) {
                folded_[f->rope_q] = folded_[f->rope_k] = true;
                if (f->temperature != rope_fold::none) {
                    folded_[f->temperature] = true;
                }
            }
        }
        // Run sizes go to the device as 32-bit counts.
        if (g.max_batch() > std::numeric_limits<std::uint32_t>::max()) {
            status_ = SYN_HIP_EUNSUPPORTED;
            return;
        }
        std::size_t top = plan_.arena_bytes;
        const auto& nodes = g.nodes();
        // Every bound matrix once, keyed by its host data.
        std::unordered_map<const void*, std::uint64_t> placed;
        std::vector<std::pair<std::uint64_t, const matrix_ref*>> uploads;
        weight_offset_.assign(nodes.size(), {no_offset, no_offset});
        for (std::size_t i = 0; i < nodes.size(); ++i) {
            const auto bound = bound_matrices(nodes[i]);
            for (std::size_t j = 0; j < bound.size(); ++j) {
                const matrix_ref* m = bound[j];
                if (m == nullptr || std::holds_alternative<std::monostate>(*m)) {
                    continue;
                }
                const void* key = std::get<weight_view>(*m).data;
                auto [it, fresh] = placed.try_emplace(key, top);
                if (fresh) {
                    uploads.emplace_back(top, m);
                    top = align_up(top + matrix_bytes(*m));
                }
                weight_offset_[i][j] = it->second;
            }
        }
        const_offset_.assign(nodes.size(), ~std::uint64_t{0});
        for (std::size_t i = 0; i < nodes.size(); ++i) {
            if (const auto* r = std::get_if<op_rope>(&nodes[i]); r && !r->freq_factors.empty()) {
                const_offset_[i] = top;
                top = align_up(top + r->freq_factors.size() * sizeof(float));
            }
        }
        const std::size_t states_begin = top;
        for (const state_desc& s : g.states()) {
            // The device KV descriptor counts positions in 32 bits; the
            // builder accepts caches of up to 2^32 positions, as the
            // reference's does (S/graph/graph.hpp:698-719).
            if (s.max_ctx > std::numeric_limits<std::uint32_t>::max()) {
                status_ = SYN_HIP_EUNSUPPORTED;
                return;
            }
            const auto max_ctx = static_cast<std::uint32_t>(s.max_ctx);
            const auto n_kv = static_cast<std::uint32_t>(s.n_kv_heads);
            const auto hd = static_cast<std::uint32_t>(s.head_dim);
            const std::uint64_t k_bytes = align_up(std::size_t{max_ctx} * n_kv * hd * 2);
            kv_.push_back(syn_kv_desc{top, top + k_bytes, max_ctx, n_kv, hd, syn_hip_kv_ctx_stride(max_ctx)});
            top = align_up(top + syn_hip_kv_state_bytes(max_ctx, n_kv, hd));
        }
        state_bytes_ = top - states_begin;
        status_ = syn_hip_arena_create(std::max<std::size_t>(top, plan_alignment), &arena_);
        if (status_ != SYN_HIP_OK) {
            arena_ = nullptr;
            return;
        }
        for (const auto& [offset, m] : uploads) {
            if (status_ == SYN_HIP_OK) {
                status_ = syn_hip_upload(arena_, offset, std::get<weight_view>(*m).data, matrix_bytes(*m));
            }
        }
        for (std::size_t i = 0; i < nodes.size() && status_ == SYN_HIP_OK; ++i) {
            if (const_offset_[i] != ~std::uint64_t{0}) {
                const auto& ff = std::get<op_rope>(nodes[i]).freq_factors;
                status_ = syn_hip_upload(arena_, const_offset_[i], ff.data(), ff.size() * sizeof(float));
            }
        }
        reset();
    }
    session(const compute_graph&&) = delete;  // the graph must outlive the session
    session(const session&) = delete;
    session& operator=(const session&) = delete;
    ~session() {
        (void)syn_hip_arena_destroy(arena_);
    }

    // SYN_HIP_OK, or why construction or the last run failed.
    int status() const noexcept {
        return status_;
    }
    const memory_plan& memory() const noexcept {
        return plan_;
    }
    // Device bytes held by the KV states.
    std::size_t state_bytes() const noexcept {
        return state_bytes_;
    }
    syn_arena* arena() noexcept {
        return arena_;
    }
    std::uint64_t offset(tensor_id t) const noexcept {
        return plan_.offset[t];
    }
    const syn_kv_desc& state(state_id s) const noexcept {
        return kv_[s];
    }

    // Writes the first rows of tensor t (an input) from host floats.
    bool write(tensor_id t, std::span<const float> rows) noexcept {
        if (!usable(t, rows.size())) {
            return false;
        }
        return keep(syn_hip_upload(arena_, plan_.offset[t], rows.data(), rows.size_bytes()));
    }
    // Reads the first rows of tensor t (after the run that wrote them).
    bool read(tensor_id t, std::span<float> rows) noexcept {
        if (!usable(t, rows.size())) {
            return false;
        }
        return keep(syn_hip_download(arena_, plan_.offset[t], rows.data(), rows.size_bytes()));
    }

    // Zeroes every state, as before a new sequence (S/graph/session.hpp:127-129).
    void reset() noexcept {
        if (arena_ != nullptr && state_bytes_ > 0) {
            keep(syn_hip_fill(arena_, kv_.front().k_offset, 0, state_bytes_));
        }
    }

    [[nodiscard]] bool run(step s = {}) noexcept {
        return run(batch{std::span<const std::uint32_t>(&s.token, 1), s.pos});
    }

    [[nodiscard]] bool run(batch b) noexcept {
        const std::size_t n = b.tokens.size();
        if (!accepts(n, b.pos)) {
            return false;
        }
        for (std::uint32_t t : b.tokens) {
            if (t >= graph_->token_limit()) {
                return false;
            }
        }
        tokens_ = b.tokens.data();
        return execute_all(n, 1, b.pos);
    }

    // n rows at position 0, one image, for a graph that embeds nothing
    // (S/graph/session.hpp:164-171).
    [[nodiscard]] bool run_rows(std::size_t n) noexcept {
        if (graph_->embeds() || !accepts(n, 0)) {
            return false;
        }
        return execute_all(n, 1, 0);
    }

    // GPU extension: `images` independent images of `rows` rows each in one
    // run (rows * images <= max_batch); self-attention stays within an image.
    // The reference encodes one image per run_rows call (S/models/clip.hpp:410).
    // Graphs that embed, keep KV states or pixel-shuffle run one image per call.
    [[nodiscard]] bool run_images(std::size_t rows, std::size_t images) noexcept {
        if (images == 0 || rows > graph_->max_batch() / std::max<std::size_t>(images, 1) || !accepts(rows * images, 0) ||
            graph_->embeds() ||
            (images > 1 && (!graph_->states().empty() || graph_->full_batch_only()))) {
            return false;
        }
        return execute_all(rows, images, 0);
    }

private:
    static constexpr std::uint64_t no_offset = ~std::uint64_t{0};

    bool accepts(std::size_t n, std::uint32_t pos) const noexcept {
        return arena_ != nullptr && n != 0 && n <= graph_->max_batch() &&
               (!graph_->full_batch_only() || n == graph_->max_batch()) &&
               std::size_t{pos} + n <= graph_->position_limit();
    }

    // The matrices a node binds, in a fixed order (weight_offset_'s slots).
    static std::array<const matrix_ref*, 2> bound_matrices(const node& n) noexcept {
        return std::visit(
            [](const auto& o) -> std::array<const matrix_ref*, 2> {
                using T = std::decay_t<decltype(o)>;
                if constexpr (std::is_same_v<T, op_matmul>) {
                    return {&o.w, nullptr};
                } else if constexpr (std::is_same_v<T, op_add_bias>) {
                    return {&o.bias, nullptr};
                } else if constexpr (std::is_same_v<T, op_rms_norm>) {
                    return {&o.gamma, nullptr};
                } else if constexpr (std::is_same_v<T, op_embed> || std::is_same_v<T, op_add_rows>) {
                    return {&o.table, nullptr};
                } else if constexpr (std::is_same_v<T, op_layer_norm>) {
                    return {&o.gamma, &o.beta};
                } else {
                    return {nullptr, nullptr};
                }
            },
            n);
    }

    // Rows of t a run of n rows (per image) uses.
    std::size_t active_rows(tensor_id t, std::size_t n) const noexcept {
        const tensor_desc& d = graph_->tensors()[t];
        return d.batched ? n / d.row_div : 1;
    }
    std::size_t size_of(tensor_id t) const noexcept {
        return graph_->tensors()[t].size;
    }
    int elementwise(std::uint32_t op, std::uint64_t a, std::uint64_t b, std::uint64_t out, std::uint64_t count,
                    float scalar = 0.0f, std::uint32_t period = 0) noexcept {
        syn_elementwise_desc d{};
        d.a_offset = a;
        d.b_offset = b;
        d.out_offset = out;
        d.count = count;
        d.op = op;
        d.scalar = scalar;
        d.period = period;
        return syn_hip_elementwise(arena_, &d);
    }

    bool usable(tensor_id t, std::size_t floats) const noexcept {
        return arena_ != nullptr && t < graph_->tensors().size() &&
               graph_->tensors()[t].role != tensor_role::scratch &&
               floats <= graph_->rows(t) * graph_->tensors()[t].size;
    }

    bool keep(int status) noexcept {
        if (status != SYN_HIP_OK) {
            status_ = status;
        }
        return status == SYN_HIP_OK;
    }

    bool execute_all(std::size_t rows, std::size_t images, std::uint32_t pos) noexcept {
        const auto& nodes = graph_->nodes();
        for (std::size_t i = 0; i < nodes.size(); ++i) {
            if (folded_[i]) {
                continue;  // done by its attention's syn_hip_attention_rope
            }
            const int e = std::visit([&](const auto& op) { return execute(op, i, rows, images, pos); }, nodes[i]);
            if (!keep(e)) {
                return false;
            }
        }
        return true;
    }

    int execute(const op_matmul& o, std::size_t i, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        const std::size_t n = active_rows(o.in, rows * images);
        if (type_of(o.w) == SYN_TYPE_F32) {
            syn_matmul_desc d{};
            d.w_offset = weight_offset_[i][0];
            d.x_offset = plan_.offset[o.in];
            d.bias_offset = no_offset;
            d.out_offset = plan_.offset[o.out];
            d.n = static_cast<std::uint32_t>(n);
            d.rows = static_cast<std::uint32_t>(graph::rows(o.w));
            d.cols = static_cast<std::uint32_t>(cols(o.w));
            return syn_hip_matmul(arena_, &d);
        }
        syn_matmul_q_desc d{};
        d.w_offset = weight_offset_[i][0];
        d.x_offset = plan_.offset[o.in];
        d.act_offset = plan_.offset[o.scratch];
        d.bias_offset = no_offset;
        d.out_offset = plan_.offset[o.out];
        d.w_type = type_of(o.w);
        d.n = static_cast<std::uint32_t>(n);
        d.rows = static_cast<std::uint32_t>(graph::rows(o.w));
        d.cols = static_cast<std::uint32_t>(cols(o.w));
        return syn_hip_matmul_q(arena_, &d);
    }
    int execute(const op_add& o, std::size_t, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        return elementwise(SYN_ADD, plan_.offset[o.a], plan_.offset[o.b], plan_.offset[o.out],
                           std::uint64_t{active_rows(o.a, rows * images)} * size_of(o.a));
    }
    int execute(const op_mul& o, std::size_t, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        return elementwise(SYN_MUL, plan_.offset[o.a], plan_.offset[o.b], plan_.offset[o.out],
                           std::uint64_t{active_rows(o.a, rows * images)} * size_of(o.a));
    }
    int execute(const op_add_bias& o, std::size_t i, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        return elementwise(SYN_ADD_BIAS, plan_.offset[o.in], weight_offset_[i][0], plan_.offset[o.out],
                           std::uint64_t{active_rows(o.in, rows * images)} * size_of(o.in), 0.0f,
                           static_cast<std::uint32_t>(size_of(o.in)));
    }
    int execute(const op_silu& o, std::size_t, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        return elementwise(SYN_SILU, plan_.offset[o.in], no_offset, plan_.offset[o.out],
                           std::uint64_t{active_rows(o.in, rows * images)} * size_of(o.in));
    }
    int execute(const op_gelu& o, std::size_t, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        return elementwise(SYN_GELU, plan_.offset[o.in], no_offset, plan_.offset[o.out],
                           std::uint64_t{active_rows(o.in, rows * images)} * size_of(o.in));
    }
    int execute(const op_softmax& o, std::size_t, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        syn_softmax_desc d{};
        d.in_offset = plan_.offset[o.in];
        d.out_offset = plan_.offset[o.out];
        d.n = static_cast<std::uint32_t>(active_rows(o.in, rows * images));
        d.size = static_cast<std::uint32_t>(size_of(o.in));
        return syn_hip_softmax(arena_, &d);
    }
    int execute(const op_rms_norm& o, std::size_t i, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        syn_norm_desc d{};
        d.in_offset = plan_.offset[o.in];
        d.weight_offset = weight_offset_[i][0];
        d.out_offset = plan_.offset[o.out];
        d.n = static_cast<std::uint32_t>(active_rows(o.in, rows * images));
        d.size = static_cast<std::uint32_t>(size_of(o.in));
        d.eps = o.eps;
        return syn_hip_rms_norm(arena_, &d);
    }
    int execute(const op_layer_norm& o, std::size_t i, std::size_t rows, std::size_t images,
                std::uint32_t) noexcept {
        syn_layer_norm_desc d{};
        d.in_offset = plan_.offset[o.in];
        d.weight_offset = weight_offset_[i][0];
        d.bias_offset = weight_offset_[i][1];
        d.out_offset = plan_.offset[o.out];
        d.n = static_cast<std::uint32_t>(active_rows(o.in, rows * images));
        d.size = static_cast<std::uint32_t>(size_of(o.in));
        d.eps = o.eps;
        return syn_hip_layer_norm(arena_, &d);
    }
    int execute(const op_embed& o, std::size_t i, std::size_t rows, std::size_t, std::uint32_t) noexcept {
        syn_embed_desc d{};
        d.table_offset = weight_offset_[i][0];
        d.out_offset = plan_.offset[o.out];
        d.n_table_rows = static_cast<std::uint32_t>(graph::rows(o.table));
        d.size = static_cast<std::uint32_t>(cols(o.table));
        d.table_type = type_of(o.table);
        return syn_hip_embed(arena_, &d, tokens_, static_cast<std::uint32_t>(rows));
    }
    // Each row times its position's temperature: a float quotient, the log
    // in double, rounded to float (kernels::attn_temperature,
    // S/kernels/elementwise.hpp:66-71).
    // One launch per image; the device computes each row's factor from its
    // position (syn_hip_attn_temperature).
    int execute(const op_attn_temperature& o, std::size_t, std::size_t rows, std::size_t images,
                std::uint32_t pos) noexcept {
        if (o.floor_len == 0 || o.floor_len > std::numeric_limits<std::uint32_t>::max()) {
            return SYN_HIP_EINVAL;
        }
        const std::uint64_t image = std::uint64_t{rows} * size_of(o.in) * sizeof(float);
        for (std::size_t img = 0; img < images; ++img) {
            syn_temperature_desc d{};
            d.in_offset = plan_.offset[o.in] + img * image;
            d.out_offset = plan_.offset[o.out] + img * image;
            d.n = static_cast<std::uint32_t>(rows);
            d.size = static_cast<std::uint32_t>(size_of(o.in));
            d.pos = pos;
            d.floor_len = static_cast<std::uint32_t>(o.floor_len);
            d.scale = o.scale;
            if (const int e = syn_hip_attn_temperature(arena_, &d)) {
                return e;
            }
        }
        return SYN_HIP_OK;
    }
    int execute(const op_last_row& o, std::size_t, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        const std::uint64_t row = size_of(o.in) * sizeof(float);
        return syn_hip_copy(arena_, plan_.offset[o.out], plan_.offset[o.in] + (rows * images - 1) * row, row);
    }
    // Table row i added to row i of each image (rows start again per image).
    // One launch for every image: the table's rows*size floats repeat over
    // the images (SYN_ADD_BIAS with the image as its period).
    int execute(const op_add_rows& o, std::size_t i, std::size_t rows, std::size_t images, std::uint32_t) noexcept {
        const std::uint64_t image = std::uint64_t{rows} * size_of(o.in);
        if (image > std::numeric_limits<std::uint32_t>::max()) {
            return SYN_HIP_EUNSUPPORTED;
        }
        return elementwise(SYN_ADD_BIAS, plan_.offset[o.in], weight_offset_[i][0], plan_.offset[o.out],
                           image * images, 0.0f, static_cast<std::uint32_t>(image));
    }
    int execute(const op_pixel_shuffle& o, std::size_t, std::size_t rows, std::size_t, std::uint32_t) noexcept {
        syn_pixel_shuffle_desc d{};
        d.in_offset = plan_.offset[o.in];
        d.out_offset = plan_.offset[o.out];
        d.n = static_cast<std::uint32_t>(size_of(o.in));
        d.grid_w = static_cast<std::uint32_t>(o.grid_w);
        d.grid_h = static_cast<std::uint32_t>(rows / o.grid_w);
        d.scale = static_cast<std::uint32_t>(o.scale);
        return syn_hip_pixel_shuffle(arena_, &d);
    }

    // One launch for every image, positions restarting per image.
    int execute(const op_rope& r, std::size_t i, std::size_t rows, std::size_t images, std::uint32_t pos) noexcept {
        syn_rope_desc d{};
        d.in_offset = plan_.offset[r.in];
        d.out_offset = plan_.offset[r.out];
        d.freq_factors_offset = const_offset_[i];
        d.n = static_cast<std::uint32_t>(rows * images);
        d.period = static_cast<std::uint32_t>(rows);
        d.size = static_cast<std::uint32_t>(graph_->tensors()[r.in].size);
        d.head_dim = static_cast<std::uint32_t>(r.head_dim);
        d.pos = pos;
        d.theta_scale = r.theta_scale;
        d.mode = r.mode == rope_mode::neox ? 1u : 0u;
        d.freq_scale = r.scaling.freq_scale;
        d.ext_factor = r.scaling.ext_factor;
        d.attn_factor = r.scaling.attn_factor;
        d.corr_low = r.scaling.corr_low;
        d.corr_high = r.scaling.corr_high;
        return syn_hip_rope(arena_, &d);
    }

    int execute(const op_attention& a, std::size_t i, std::size_t rows, std::size_t, std::uint32_t pos) noexcept {
        syn_attn_desc d{};
        d.cache = kv_[a.cache];
        d.q_offset = plan_.offset[a.q];
        d.k_offset = plan_.offset[a.k];
        d.v_offset = plan_.offset[a.v];
        d.out_offset = plan_.offset[a.out];
        d.scratch_offset = plan_.offset[a.scratch];
        d.scratch_bytes = graph_->tensors()[a.scratch].bytes;
        d.n_heads = static_cast<std::uint32_t>(a.n_heads);
        d.pos = pos;
        d.n = static_cast<std::uint32_t>(rows);
        d.scale = a.scale;
        d.q_dtype = SYN_F32;
        d.kv_dtype = SYN_F32;
        if (!folds_[i]) {
            return syn_hip_attention(arena_, &d);
        }
        const rope_fold& f = *folds_[i];
        const auto& rq = std::get<op_rope>(graph_->nodes()[f.rope_q]);
        const auto& rk = std::get<op_rope>(graph_->nodes()[f.rope_k]);
        syn_attn_rope_desc r{};
        d.q_offset = plan_.offset[rq.in];
        d.k_offset = plan_.offset[rk.in];
        r.q_out_offset = plan_.offset[a.q];
        r.k_out_offset = plan_.offset[a.k];
        r.freq_factors_offset = const_offset_[f.rope_q];
        r.theta_scale = rq.theta_scale;
        r.mode = rq.mode == rope_mode::neox ? 1u : 0u;
        r.freq_scale = rq.scaling.freq_scale;
        r.ext_factor = rq.scaling.ext_factor;
        r.attn_factor = rq.scaling.attn_factor;
        r.corr_low = rq.scaling.corr_low;
        r.corr_high = rq.scaling.corr_high;
        if (f.temperature != rope_fold::none) {
            const auto& t = std::get<op_attn_temperature>(graph_->nodes()[f.temperature]);
            r.temp_scale = t.scale;
            r.temp_floor_len = static_cast<std::uint32_t>(t.floor_len);
        }
        return syn_hip_attention_rope(arena_, &d, &r);
    }

    int execute(const op_self_attention& s, std::size_t, std::size_t rows, std::size_t images,
                std::uint32_t) noexcept {
        const std::size_t size = graph_->tensors()[s.q].size;
        syn_self_desc d{};
        d.q_offset = plan_.offset[s.q];
        d.k_offset = plan_.offset[s.k];
        d.v_offset = plan_.offset[s.v];
        d.out_offset = plan_.offset[s.out];
        d.n = static_cast<std::uint32_t>(rows);
        d.batch = static_cast<std::uint32_t>(images);
        d.n_heads = static_cast<std::uint32_t>(s.n_heads);
        d.head_dim = static_cast<std::uint32_t>(size / s.n_heads);
        d.scale = s.scale;
        d.in_dtype = SYN_F32;
        return syn_hip_self_attention(arena_, &d);
    }

    const compute_graph* graph_;
    std::vector<std::optional<rope_fold>> folds_;  // per node: the RoPE folded into this attention
    std::vector<bool> folded_;                     // per node: run inside a later attention
    memory_plan plan_;
    std::vector<std::uint64_t> const_offset_;                  // per node: its RoPE table, or ~0
    std::vector<std::array<std::uint64_t, 2>> weight_offset_;  // per node: its bound matrices
    const std::uint32_t* tokens_ = nullptr;                    // the running batch's tokens
    std::vector<syn_kv_desc> kv_;
    std::size_t state_bytes_ = 0;
    syn_arena* arena_ = nullptr;
    int status_ = SYN_HIP_OK;
};

}  // namespace syn::graph
