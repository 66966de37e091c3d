// A stand-in for libsynapse_hip.so that launches nothing: every entry point
// the host session calls succeeds and counts the call. Linked only into the
// no-allocation test, so that test counts the session's own allocations on
// the CPU, not the HIP runtime's (which allocates host objects per launch).
#include "synapse_hip.h"

#include <cstdint>

struct syn_arena {
    size_t bytes;
};

namespace stub {
long calls = 0;  // device work the session asked for
// Calls by entry point, for the launch counts of a decode layer.
long rope = 0, temperature = 0, attention = 0, attention_rope = 0;
}

namespace {
int ok() {
    ++stub::calls;
    return SYN_HIP_OK;
}
uint64_t align256(uint64_t x) {
    return (x + 255) / 256 * 256;
}
}  // namespace

extern "C" {
int syn_hip_arena_create(size_t bytes, syn_arena** out) {
    *out = new syn_arena{bytes};
    return SYN_HIP_OK;
}
int syn_hip_arena_destroy(syn_arena* a) {
    delete a;
    return SYN_HIP_OK;
}
int syn_hip_upload(syn_arena*, uint64_t, const void*, size_t) { return ok(); }
int syn_hip_download(syn_arena*, uint64_t, void*, size_t) { return ok(); }
int syn_hip_fill(syn_arena*, uint64_t, int, size_t) { return ok(); }
int syn_hip_copy(syn_arena*, uint64_t, uint64_t, size_t) { return ok(); }
uint32_t syn_hip_kv_ctx_stride(uint32_t max_ctx) { return (max_ctx + 63) / 64 * 64; }
uint64_t syn_hip_kv_state_bytes(uint32_t max_ctx, uint32_t n_kv, uint32_t hd) {
    const uint64_t row = uint64_t{n_kv} * hd;
    return align256(uint64_t{max_ctx} * row * 2) + align256(row * syn_hip_kv_ctx_stride(max_ctx) * 2);
}
uint64_t syn_hip_attention_scratch_bytes(uint32_t n_heads, uint32_t n_kv, uint32_t hd, uint32_t max_ctx, uint32_t) {
    return n_kv == 0 || n_heads % n_kv ? 0 : align256(uint64_t{(max_ctx + 127) / 128} * n_heads * (hd + 2) * 4);
}
uint64_t syn_hip_matmul_q_act_bytes(uint32_t, uint32_t n, uint32_t cols) { return uint64_t{n} * cols + 1024; }
int syn_hip_attention(syn_arena*, const syn_attn_desc*) {
    ++stub::attention;
    return ok();
}
int syn_hip_attention_rope(syn_arena*, const syn_attn_desc*, const syn_attn_rope_desc*) {
    ++stub::attention_rope;
    return ok();
}
int syn_hip_attn_temperature(syn_arena*, const syn_temperature_desc*) {
    ++stub::temperature;
    return ok();
}
int syn_hip_self_attention(syn_arena*, const syn_self_desc*) { return ok(); }
int syn_hip_rope(syn_arena*, const syn_rope_desc*) {
    ++stub::rope;
    return ok();
}
int syn_hip_embed(syn_arena*, const syn_embed_desc*, const uint32_t*, uint32_t) { return ok(); }
int syn_hip_rms_norm(syn_arena*, const syn_norm_desc*) { return ok(); }
int syn_hip_matmul(syn_arena*, const syn_matmul_desc*) { return ok(); }
int syn_hip_matmul_q(syn_arena*, const syn_matmul_q_desc*) { return ok(); }
int syn_hip_elementwise(syn_arena*, const syn_elementwise_desc*) { return ok(); }
int syn_hip_softmax(syn_arena*, const syn_softmax_desc*) { return ok(); }
int syn_hip_layer_norm(syn_arena*, const syn_layer_norm_desc*) { return ok(); }
int syn_hip_pixel_shuffle(syn_arena*, const syn_pixel_shuffle_desc*) { return ok(); }
}
