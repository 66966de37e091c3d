// session::run allocates nothing: the reference's graph_no_alloc test
// (tests/sdk/graph_no_alloc.cpp:199-263) restated for this session. Global
// operator new / delete are replaced and counted while armed; the session is
// built first (its construction allocates: the plan, the arena), then decode
// steps, a batched prefill and image-encoder runs execute with the counter
// armed. Linked against stub_abi.cpp, so the count is the session's own host
// code (the device side makes its one hipMalloc at arena creation).
#include "check.hpp"
#include "graph.hpp"
#include "session.hpp"

#include <cstdio>
#include <cstdlib>
#include <new>
#include <vector>

namespace stub {
extern long calls;
extern long rope, temperature, attention, attention_rope;
}

namespace {
bool armed = false;
long allocations = 0;

void* counted(std::size_t n) {
    if (armed) {
        ++allocations;
    }
    if (void* p = std::malloc(n ? n : 1)) {
        return p;
    }
    throw std::bad_alloc{};
}
void* counted_aligned(std::size_t n, std::size_t align) {
    if (armed) {
        ++allocations;
    }
    const std::size_t rounded = (n + align - 1) / align * align;
    if (void* p = std::aligned_alloc(align, rounded ? rounded : align)) {
        return p;
    }
    throw std::bad_alloc{};
}
}  // namespace

void* operator new(std::size_t n) { return counted(n); }
void* operator new[](std::size_t n) { return counted(n); }
void* operator new(std::size_t n, const std::nothrow_t&) noexcept {
    try {
        return counted(n);
    } catch (...) {
        return nullptr;
    }
}
void* operator new[](std::size_t n, const std::nothrow_t&) noexcept {
    try {
        return counted(n);
    } catch (...) {
        return nullptr;
    }
}
void* operator new(std::size_t n, std::align_val_t a) { return counted_aligned(n, static_cast<std::size_t>(a)); }
void* operator new[](std::size_t n, std::align_val_t a) { return counted_aligned(n, static_cast<std::size_t>(a)); }
void operator delete(void* p) noexcept { std::free(p); }
void operator delete[](void* p) noexcept { std::free(p); }
void operator delete(void* p, std::size_t) noexcept { std::free(p); }
void operator delete[](void* p, std::size_t) noexcept { std::free(p); }
void operator delete(void* p, std::align_val_t) noexcept { std::free(p); }
void operator delete[](void* p, std::align_val_t) noexcept { std::free(p); }
void operator delete(void* p, std::size_t, std::align_val_t) noexcept { std::free(p); }
void operator delete[](void* p, std::size_t, std::align_val_t) noexcept { std::free(p); }

using namespace syn::graph;

namespace {

struct zeros {
    std::vector<unsigned char> bytes;
    weight_view view;
    zeros(std::uint32_t type, std::size_t rows_, std::size_t cols_)
        : bytes(rows_ * cols_ / block_values(type) * block_bytes(type)), view{type, rows_, cols_, bytes.data()} {}
    matrix_ref ref() const { return matrix_ref{view}; }
};

// A two-layer Llama-family decode graph (S/models/llama.hpp:405-473): embed,
// RMSNorm, q/k/v projections (one block-format), RoPE, attention temperature,
// attention over a KV cache, output projection, SwiGLU MLP, last row, logits.
void llama_runs() {
    constexpr std::size_t embd = 64, heads = 4, kv_heads = 2, hd = 16, ff = 128, vocab = 100, ctx = 32, n_batch = 8;
    const zeros table(SYN_TYPE_F32, vocab, embd), norm(SYN_TYPE_F32, 1, embd), wq(SYN_TYPE_Q8_0, heads * hd, embd),
        wk(SYN_TYPE_F32, kv_heads * hd, embd), wv(SYN_TYPE_F32, kv_heads * hd, embd), wo(SYN_TYPE_F32, embd, heads * hd),
        wg(SYN_TYPE_F32, ff, embd), wu(SYN_TYPE_F32, ff, embd), wd(SYN_TYPE_F32, embd, ff), out(SYN_TYPE_F32, vocab, embd),
        bias(SYN_TYPE_F32, 1, heads * hd);
    graph_builder b(n_batch);
    tensor_id h = b.embed(table.ref());
    for (int layer = 0; layer < 2; ++layer) {
        const tensor_id x = b.rms_norm(h, norm.ref(), 1e-5f);
        const tensor_id q = b.attn_temperature(b.rope(b.add_bias(b.matmul(wq.ref(), x), bias.ref()), hd, 1e4f), 0.1f, 8);
        const tensor_id k = b.rope(b.matmul(wk.ref(), x), hd, 1e4f);
        const tensor_id v = b.matmul(wv.ref(), x);
        const tensor_id a = b.attention(q, k, v, b.kv_cache(ctx, kv_heads, hd), heads, 0.25f);
        h = b.add(h, b.matmul(wo.ref(), a));
        const tensor_id y = b.rms_norm(h, norm.ref(), 1e-5f);
        h = b.add(h, b.matmul(wd.ref(), b.mul(b.silu(b.matmul(wg.ref(), y)), b.matmul(wu.ref(), y))));
    }
    b.output(b.matmul(out.ref(), b.rms_norm(b.last_row(h), norm.ref(), 1e-5f)));
    auto g = std::move(b).finalize();
    CHECK(g.has_value());
    if (!g) {
        return;
    }
    session s{g.value()};
    CHECK(s.status() == SYN_HIP_OK);
    const std::uint32_t tokens[n_batch] = {1, 2, 3, 4, 5, 6, 7, 8};
    const long before = stub::calls;
    allocations = 0;
    armed = true;
    bool ran = s.run(batch{std::span<const std::uint32_t>(tokens, n_batch), 0});  // batched prefill
    ran = s.run(batch{std::span<const std::uint32_t>(tokens, 5), 8}) && ran;   // a shorter batch after it
    for (std::uint32_t pos = 13; pos < 24; ++pos) {   // decode steps
        ran = s.run(step{static_cast<std::uint32_t>(pos * 7 % vocab), pos}) && ran;
    }
    armed = false;
    CHECK(ran);
    CHECK(allocations == 0);
    CHECK(stub::calls - before > 13 * 20);  // the runs did ask for device work

    // A decode step's layer: RoPE of q and k, the temperature and the
    // attention fold into one syn_hip_attention_rope call (one kernel on the
    // device) -- 1 call per layer where the graph has 4 nodes.
    const long rope0 = stub::rope, temp0 = stub::temperature, attn0 = stub::attention, fused0 = stub::attention_rope;
    const long calls0 = stub::calls;
    CHECK(s.run(step{5, 24}));
    CHECK(stub::attention_rope - fused0 == 2);
    CHECK(stub::rope == rope0 && stub::temperature == temp0 && stub::attention == attn0);
    const long per_step = stub::calls - calls0;

    // The same graph with q's rotation also read elsewhere cannot fold: the
    // separate calls, the temperature one launch per run.
    graph_builder b2(n_batch);
    tensor_id h2 = b2.embed(table.ref());
    const tensor_id x2 = b2.rms_norm(h2, norm.ref(), 1e-5f);
    const tensor_id qr = b2.rope(b2.matmul(wq.ref(), x2), hd, 1e4f);
    const tensor_id q2 = b2.attn_temperature(qr, 0.1f, 8);
    const tensor_id k2 = b2.rope(b2.matmul(wk.ref(), x2), hd, 1e4f);
    const tensor_id a2 = b2.attention(q2, k2, b2.matmul(wv.ref(), x2), b2.kv_cache(ctx, kv_heads, hd), heads, 0.25f);
    b2.output(b2.add(b2.matmul(wo.ref(), a2), qr));
    auto g2 = std::move(b2).finalize();
    CHECK(g2.has_value());
    if (g2) {
        session s2{g2.value()};
        const long r1 = stub::rope, t1 = stub::temperature, a1 = stub::attention, f1 = stub::attention_rope;
        CHECK(s2.run(batch{std::span<const std::uint32_t>(tokens, 6), 0}));
        CHECK(stub::rope - r1 == 2 && stub::temperature - t1 == 1 && stub::attention - a1 == 1);
        CHECK(stub::attention_rope == f1);
    }
    std::printf("decode step: %ld C-ABI calls for 2 layers\n", per_step);
}

// An image encoder (S/models/clip.hpp:300-417): layer norm, projection,
// self-attention, position table, GELU, pixel shuffle.
void vision_runs() {
    constexpr std::size_t rows = 16, size = 64, heads = 4;
    const zeros gamma(SYN_TYPE_F32, 1, size), w(SYN_TYPE_F32, size, size), pos(SYN_TYPE_F32, rows, size),
        proj(SYN_TYPE_F32, 32, size * 4);
    graph_builder b(rows);
    const tensor_id x = b.input(size);
    const tensor_id e = b.add_rows(x, pos.ref());
    const tensor_id n = b.layer_norm(e, gamma.ref(), gamma.ref(), 1e-6f);
    const tensor_id a = b.self_attention(b.matmul(w.ref(), n), b.matmul(w.ref(), n), b.matmul(w.ref(), n), heads, 0.25f);
    const tensor_id y = b.add(e, b.gelu(b.matmul(w.ref(), a)));
    b.output(b.matmul(proj.ref(), b.pixel_shuffle(y, 4, 2)));
    auto g = std::move(b).finalize();
    CHECK(g.has_value());
    if (!g) {
        return;
    }
    session s{g.value()};
    CHECK(s.status() == SYN_HIP_OK);
    const long before = stub::calls;
    allocations = 0;
    armed = true;
    bool ran = s.run_rows(rows);
    ran = s.run_rows(rows) && ran;
    armed = false;
    CHECK(ran);
    CHECK(allocations == 0);
    CHECK(stub::calls - before >= 2 * 10);

    // Several images per run (no pixel shuffle): run_images.
    graph_builder b2(4 * rows);
    const tensor_id x2 = b2.input(size);
    b2.output(b2.self_attention(x2, x2, x2, heads, 0.25f));
    auto g2 = std::move(b2).finalize();
    CHECK(g2.has_value());
    if (!g2) {
        return;
    }
    session s2{g2.value()};
    allocations = 0;
    armed = true;
    const bool ran2 = s2.run_images(rows, 4);
    armed = false;
    CHECK(ran2);
    CHECK(allocations == 0);
}

}  // namespace

int main() {
    llama_runs();
    vision_runs();
    CHECK_DONE();
}
