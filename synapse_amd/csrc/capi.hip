// capi.hip — the extern "C" boundary (include/synapse_hip.h).
//
// Every entry point checks its descriptor on the host -- shapes, alignment,
// and that every byte a kernel may touch lies inside the arena -- before it
// queues anything, so a bad descriptor is an error code, never a GPU fault.
// Nothing here throws; nothing here allocates after syn_hip_arena_create.

#include "../../include/synapse_hip.h"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

struct syn_arena {
    char* base = nullptr;   // device bytes
    std::size_t bytes = 0;  // usable bytes (the allocation is rounded up to 256)
    hipStream_t stream = nullptr;
    int device = 0;
};

// ---- the allocation-free entry point's scratch ------------------------------
// syn_hip_attention_noalloc keeps the split-KV decode's partials here instead
// of in caller scratch: 4 MiB per device, held until the process ends (e.g.
// config 2, 33 splits x 8 KV heads x 4 heads x 130 floats, takes 549 KB).
// In host code `scratch` names a host-side stand-in; kernels get the device
// address that hipGetSymbolAddress returns for the current device.
constexpr std::size_t noalloc_scratch_bytes = std::size_t{4} << 20;
static __device__ __align__(256) float scratch[noalloc_scratch_bytes / sizeof(float)];

namespace {

constexpr uint64_t no_offset = ~uint64_t{0};

// Device address of `scratch`, one per device (each device holds its own copy
// of the array at its own address), looked up with that device current.
constexpr int max_devices = 64;
std::mutex scratch_mutex;
float* scratch_device[max_devices] = {};

thread_local char last_error[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(last_error, sizeof last_error, fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) {
        return SYN_HIP_OK;
    }
    return fail(static_cast<int>(e), "%s: %s", what, hipGetErrorString(e));
}

// Looks up (once per device) the static scratch's address on `device`, which
// must be the current device.
int lookup_scratch(int device) {
    if (device < 0 || device >= max_devices) {
        return fail(SYN_HIP_ENODEV, "device %d: no static scratch slot", device);
    }
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_device[device] == nullptr) {
        void* ptr = nullptr;
        if (int e = hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) {
            return e;
        }
        scratch_device[device] = static_cast<float*>(ptr);
    }
    return SYN_HIP_OK;
}

// [offset, offset + bytes) inside the arena, without wrapping.
bool in_arena(const syn_arena* a, uint64_t offset, uint64_t bytes) {
    return offset <= a->bytes && bytes <= a->bytes - offset;
}

bool aligned(uint64_t offset, uint64_t to) {
    return offset % to == 0;
}

std::size_t dtype_size(uint32_t t) {
    return t == SYN_F16 ? 2 : 4;
}

bool dtype_ok(uint32_t t) {
    return t == SYN_F32 || t == SYN_F16;
}

int check_arena(const syn_arena* a) {
    if (a == nullptr || a->base == nullptr) {
        return fail(SYN_HIP_EINVAL, "null arena");
    }
    return SYN_HIP_OK;
}

int check_range(const syn_arena* a, uint64_t offset, uint64_t bytes, uint64_t align, const char* what) {
    if (!in_arena(a, offset, bytes)) {
        return fail(SYN_HIP_ERANGE, "%s: [%llu, +%llu) outside the arena of %zu bytes", what,
                    static_cast<unsigned long long>(offset), static_cast<unsigned long long>(bytes), a->bytes);
    }
    if (!aligned(offset, align)) {
        return fail(SYN_HIP_EINVAL, "%s: offset %llu not %llu-byte aligned", what,
                    static_cast<unsigned long long>(offset), static_cast<unsigned long long>(align));
    }
    return SYN_HIP_OK;
}

uint32_t ctx_stride_of(uint32_t max_ctx) {
    return (max_ctx + 63u) / 64u * 64u;
}

uint64_t align256(uint64_t x) {
    return (x + 255u) / 256u * 256u;
}

// A KV state: shape limits of kv_cache (S/graph/graph.hpp:698-719) and the
// byte ranges of both blocks.
int check_cache(const syn_arena* a, const syn_kv_desc& c) {
    if (c.max_ctx == 0 || c.n_kv_heads == 0 || c.head_dim == 0 || c.head_dim > 256 || c.head_dim % 2 != 0) {
        return fail(SYN_HIP_EINVAL, "kv cache: max_ctx %u, n_kv_heads %u, head_dim %u", c.max_ctx, c.n_kv_heads,
                    c.head_dim);
    }
    if (c.ctx_stride < c.max_ctx || c.ctx_stride % 8 != 0) {
        return fail(SYN_HIP_EINVAL, "kv cache: ctx_stride %u for max_ctx %u (want a multiple of 8 >= max_ctx)",
                    c.ctx_stride, c.max_ctx);
    }
    const uint64_t row = uint64_t{c.n_kv_heads} * c.head_dim;
    if (int e = check_range(a, c.k_offset, uint64_t{c.max_ctx} * row * 2, 16, "kv cache K")) {
        return e;
    }
    if (int e = check_range(a, c.v_offset, row * c.ctx_stride * 2, 16, "kv cache V^T")) {
        return e;
    }
    return SYN_HIP_OK;
}

syn::kv_layout layout_of(syn_arena* a, const syn_kv_desc& c) {
    return syn::kv_layout{reinterpret_cast<_Float16*>(a->base + c.k_offset),
                          reinterpret_cast<_Float16*>(a->base + c.v_offset), c.max_ctx, c.n_kv_heads, c.head_dim,
                          c.ctx_stride};
}

// Matrix-core kernels need 16-byte operand chunks: head_dim a multiple of 8.
bool fast_shape(uint32_t hd) {
    return hd % 8 == 0;
}

uint64_t decode_scratch_bytes(uint32_t splits, uint32_t n_kv, uint32_t group, uint32_t hd) {
    return uint64_t{splits} * n_kv * syn::decode_split_floats(group, hd) * sizeof(float);
}

// Where a decode launch keeps its split partials: caller scratch in the arena
// (checked against it), or the library's static array (`device` non-null).
struct partial_area {
    uint64_t arena_offset;
    uint64_t bytes;
    float* device;
};

// One decode launch over seqs[0..n): fills the argument block, checks the
// scratch, launches. kv_dtype types the sequences' k_new / v_new rows.
int run_decode(syn_arena* a, const syn::decode_seq* seqs, uint32_t n, uint32_t n_kv, uint32_t hd, uint32_t group,
               float scale, uint32_t q_dtype, uint32_t kv_dtype, const partial_area& pa,
               const syn::rope_params* rope = nullptr) {
    if (n == 0 || n > syn::decode_max_seqs) {
        return fail(SYN_HIP_EINVAL, "decode: %u sequences in one launch", n);
    }
    uint64_t positions = 0;
    uint32_t max_len = 0;
    for (uint32_t i = 0; i < n; ++i) {
        positions += seqs[i].len;
        max_len = std::max(max_len, seqs[i].len);
    }
    const uint32_t chunk = syn::decode_choose_chunk(positions, n_kv, max_len);
    for (uint32_t i = 0; i < n; ++i) {
        if (!syn::decode_fits(chunk, n_kv * hd, hd, seqs[i].ctx_stride)) {
            return fail(SYN_HIP_EUNSUPPORTED, "decode: a split or V^T row span exceeds 2^31 bytes");
        }
    }
    syn::decode_params prm{};
    uint32_t splits = 0;
    uint32_t merge_blocks = 0;
    syn::decode_seq table[syn::decode_max_seqs];
    for (uint32_t i = 0; i < n; ++i) {
        table[i] = seqs[i];
        table[i].block0 = splits;
        // A step's new row is attended apart by the last split's block, so
        // the splits cover the cached rows (at least one split).
        const uint32_t cached = seqs[i].len - (seqs[i].k_new != nullptr ? 1u : 0u);
        table[i].n_splits = std::max(1u, (cached + chunk - 1) / chunk);
        table[i].merge0 = merge_blocks;
        splits += table[i].n_splits;
        if (table[i].n_splits > 1) {
            merge_blocks += n_kv * group;
        }
    }
    prm.n_kv = n_kv;
    prm.hd = hd;
    prm.group = group;
    prm.row = n_kv * hd;
    prm.chunk = chunk;
    prm.kv_dtype = kv_dtype;
    prm.total_slots = splits * n_kv;
    prm.merge_blocks = merge_blocks;
    prm.n_seqs = n;
    prm.scale_log2e = scale * syn::log2e;
    if (merge_blocks > 0) {
        const uint64_t need = decode_scratch_bytes(splits, n_kv, group, hd);
        if (need > pa.bytes) {
            if (pa.device != nullptr) {
                return fail(SYN_HIP_EINVAL, "decode: the allocation-free entry point's static scratch holds %llu "
                            "bytes; this step's split partials need %llu",
                            static_cast<unsigned long long>(pa.bytes), static_cast<unsigned long long>(need));
            }
            return fail(SYN_HIP_EINVAL, "decode: scratch of %llu bytes, %llu needed",
                        static_cast<unsigned long long>(pa.bytes), static_cast<unsigned long long>(need));
        }
        if (pa.device != nullptr) {
            prm.part = pa.device;
        } else {
            if (int e = check_range(a, pa.arena_offset, need, 16, "decode scratch")) {
                return e;
            }
            prm.part = reinterpret_cast<float*>(a->base + pa.arena_offset);
        }
    }
    if (n == 1 && rope != nullptr) {
        syn::decode_rope_args one{prm, table[0], *rope};
        return hip_status(syn::launch_decode(one, q_dtype, a->stream), "decode launch");
    }
    if (n == 1) {
        syn::decode_one_args one{prm, table[0]};
        return hip_status(syn::launch_decode(one, q_dtype, a->stream), "decode launch");
    }
    syn::decode_batch_args batch{};
    batch.p = prm;
    for (uint32_t i = 0; i < n; ++i) {
        batch.seq[i] = table[i];
        batch.block0s[i] = table[i].block0;
        batch.merge0s[i] = table[i].merge0;
    }
    return hip_status(syn::launch_decode(batch, q_dtype, a->stream), "decode launch");
}

int check_attn(const syn_arena* a, const syn_attn_desc* d, bool with_new_rows) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (int e = check_cache(a, d->cache)) {
        return e;
    }
    const syn_kv_desc& c = d->cache;
    if (d->n_heads == 0 || d->n_heads % c.n_kv_heads != 0) {
        return fail(SYN_HIP_EINVAL, "attention: %u query heads on %u KV heads", d->n_heads, c.n_kv_heads);
    }
    if (!(std::isfinite(d->scale) && d->scale > 0.0f)) {
        return fail(SYN_HIP_EINVAL, "attention: scale %g (want finite and > 0)", static_cast<double>(d->scale));
    }
    if (d->n == 0 || uint64_t{d->pos} + d->n > c.max_ctx) {
        return fail(SYN_HIP_EINVAL, "attention: run of %u at position %u on a cache of %u", d->n, d->pos, c.max_ctx);
    }
    if (!dtype_ok(d->q_dtype) || !dtype_ok(d->kv_dtype)) {
        return fail(SYN_HIP_EINVAL, "attention: dtypes %u, %u", d->q_dtype, d->kv_dtype);
    }
    const uint64_t qsize = uint64_t{d->n_heads} * c.head_dim;
    const uint64_t row = uint64_t{c.n_kv_heads} * c.head_dim;
    if (int e = check_range(a, d->q_offset, d->n * qsize * dtype_size(d->q_dtype), 16, "attention q")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, d->n * qsize * 4, 16, "attention out")) {
        return e;
    }
    if (with_new_rows) {
        if (int e = check_range(a, d->k_offset, d->n * row * dtype_size(d->kv_dtype), 16, "attention k")) {
            return e;
        }
        if (int e = check_range(a, d->v_offset, d->n * row * dtype_size(d->kv_dtype), 16, "attention v")) {
            return e;
        }
    }
    return SYN_HIP_OK;
}

syn::flash_args flash_of(syn_arena* a, const syn_attn_desc* d) {
    const syn_kv_desc& c = d->cache;
    syn::flash_args f{};
    f.q = a->base + d->q_offset;
    f.out = reinterpret_cast<float*>(a->base + d->out_offset);
    f.k = reinterpret_cast<const _Float16*>(a->base + c.k_offset);
    f.vt = reinterpret_cast<const _Float16*>(a->base + c.v_offset);
    f.n = d->n;
    f.batch = 1;
    f.pos = d->pos;
    f.kv_len = d->pos + d->n;
    f.n_heads = d->n_heads;
    f.n_kv = c.n_kv_heads;
    f.hd = c.head_dim;
    f.group = d->n_heads / c.n_kv_heads;
    f.q_row = d->n_heads * c.head_dim;
    f.row = c.n_kv_heads * c.head_dim;
    f.ctx_stride = c.ctx_stride;
    f.scale_log2e = d->scale * syn::log2e;
    return f;
}

bool decode_shape(const syn_attn_desc* d) {
    const syn_kv_desc& c = d->cache;
    const uint32_t len = d->pos + 1;
    return d->n == 1 && fast_shape(c.head_dim) && d->n_heads / c.n_kv_heads <= 16 &&

           syn::decode_fits(syn::decode_choose_chunk(len, c.n_kv_heads, len), c.n_kv_heads * c.head_dim, c.head_dim,
                            c.ctx_stride);
}

// Attends the run; with_new_rows, a single-token step's K, V row is appended
// by the decode kernel itself (one launch), longer runs were appended before.
int attend_checked(syn_arena* a, const syn_attn_desc* d, bool with_new_rows, const partial_area* static_area = nullptr,
                   const syn::rope_params* rope = nullptr) {
    const syn_kv_desc& c = d->cache;
    const uint32_t group = d->n_heads / c.n_kv_heads;
    if (decode_shape(d)) {
        syn::decode_seq s{};
        s.q = a->base + d->q_offset;
        s.out = reinterpret_cast<float*>(a->base + d->out_offset);
        s.k = reinterpret_cast<_Float16*>(a->base + c.k_offset);
        s.vt = reinterpret_cast<_Float16*>(a->base + c.v_offset);
        if (with_new_rows) {
            s.k_new = a->base + d->k_offset;
            s.v_new = a->base + d->v_offset;
        }
        s.len = d->pos + 1;
        s.ctx_stride = c.ctx_stride;
        const partial_area arena_area{d->scratch_offset, d->scratch_bytes, nullptr};
        return run_decode(a, &s, 1, c.n_kv_heads, c.head_dim, group, d->scale, d->q_dtype, d->kv_dtype,
                          static_area != nullptr ? *static_area : arena_area, rope);
    }
    const syn::flash_args f = flash_of(a, d);
    if (fast_shape(c.head_dim) && (uint64_t{d->n} + 127) / 128 <= 65535 &&
        syn::prefill_fits(d->pos + d->n, c.n_kv_heads * c.head_dim, c.head_dim, c.ctx_stride)) {
        return hip_status(syn::launch_prefill(f, d->q_dtype, a->stream), "prefill launch");
    }
    return hip_status(syn::launch_generic_causal(f, d->q_dtype, a->stream), "generic causal launch");
}

}  // namespace

extern "C" {

const char* syn_hip_error_string(int status) {
    switch (status) {
    case SYN_HIP_OK:
        return "ok";
    case SYN_HIP_EINVAL:
        return "invalid argument";
    case SYN_HIP_ERANGE:
        return "offset outside the arena";
    case SYN_HIP_EUNSUPPORTED:
        return "unsupported shape";
    case SYN_HIP_ENOMEM:
        return "device allocation failed";
    case SYN_HIP_ENODEV:
        return "no gfx950 device";
    default:
        return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown error";
    }
}

const char* syn_hip_last_error(void) {
    return last_error;
}

int syn_hip_arena_create(size_t bytes, syn_arena** out) {
    if (out == nullptr) {
        return fail(SYN_HIP_EINVAL, "null output pointer");
    }
    *out = nullptr;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        return fail(SYN_HIP_ENODEV, "no HIP device");
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        return fail(SYN_HIP_ENODEV, "hipGetDeviceProperties failed");
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return fail(SYN_HIP_ENODEV, "device %d is %s, this library is built for gfx950", device, prop.gcnArchName);
    }
    const std::size_t user = align256(bytes);
    if (bytes == 0 || user < bytes) {
        return fail(SYN_HIP_EINVAL, "arena of %zu bytes", bytes);
    }
    auto* a = new (std::nothrow) syn_arena;
    if (a == nullptr) {
        return fail(SYN_HIP_ENOMEM, "host allocation failed");
    }
    void* p = nullptr;
    if (hipMalloc(&p, user) != hipSuccess) {
        delete a;
        return fail(SYN_HIP_ENOMEM, "hipMalloc of %zu bytes failed", user);
    }
    a->base = static_cast<char*>(p);
    a->bytes = bytes;
    a->device = device;
    if (int e = lookup_scratch(device)) {
        (void)hipFree(p);
        delete a;
        return e;
    }
    if (hipStreamCreateWithFlags(&a->stream, hipStreamNonBlocking) != hipSuccess) {
        (void)hipFree(p);
        delete a;
        return fail(SYN_HIP_ENOMEM, "hipStreamCreate failed");
    }
    *out = a;
    return SYN_HIP_OK;
}

int syn_hip_arena_destroy(syn_arena* a) {
    if (a == nullptr) {
        return SYN_HIP_OK;
    }
    int e = hip_status(hipStreamSynchronize(a->stream), "destroy sync");
    (void)hipStreamDestroy(a->stream);
    (void)hipFree(a->base);
    delete a;
    return e;
}

size_t syn_hip_arena_bytes(const syn_arena* a) {
    return a ? a->bytes : 0;
}

void* syn_hip_arena_stream(syn_arena* a) {
    return a ? static_cast<void*>(a->stream) : nullptr;
}

int syn_hip_upload(syn_arena* a, uint64_t offset, const void* host, size_t bytes) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (int e = check_range(a, offset, bytes, 1, "upload")) {
        return e;
    }
    if (bytes == 0) {
        return SYN_HIP_OK;
    }
    if (host == nullptr) {
        return fail(SYN_HIP_EINVAL, "upload: null host pointer");
    }
    return hip_status(hipMemcpyAsync(a->base + offset, host, bytes, hipMemcpyHostToDevice, a->stream), "upload");
}

int syn_hip_download(syn_arena* a, uint64_t offset, void* host, size_t bytes) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (int e = check_range(a, offset, bytes, 1, "download")) {
        return e;
    }
    if (bytes == 0) {
        return SYN_HIP_OK;
    }
    if (host == nullptr) {
        return fail(SYN_HIP_EINVAL, "download: null host pointer");
    }
    if (int e = hip_status(hipMemcpyAsync(host, a->base + offset, bytes, hipMemcpyDeviceToHost, a->stream),
                           "download")) {
        return e;
    }
    return hip_status(hipStreamSynchronize(a->stream), "download sync");
}

int syn_hip_fill(syn_arena* a, uint64_t offset, int value, size_t bytes) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (int e = check_range(a, offset, bytes, 1, "fill")) {
        return e;
    }
    if (bytes == 0) {
        return SYN_HIP_OK;
    }
    return hip_status(hipMemsetAsync(a->base + offset, value, bytes, a->stream), "fill");
}

int syn_hip_copy(syn_arena* a, uint64_t dst, uint64_t src, size_t bytes) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (int e = check_range(a, dst, bytes, 1, "copy dst")) {
        return e;
    }
    if (int e = check_range(a, src, bytes, 1, "copy src")) {
        return e;
    }
    if (bytes == 0) {
        return SYN_HIP_OK;
    }
    return hip_status(hipMemcpyAsync(a->base + dst, a->base + src, bytes, hipMemcpyDeviceToDevice, a->stream),
                      "copy");
}

int syn_hip_synchronize(syn_arena* a) {
    if (int e = check_arena(a)) {
        return e;
    }
    return hip_status(hipStreamSynchronize(a->stream), "synchronize");
}

uint32_t syn_hip_kv_ctx_stride(uint32_t max_ctx) {
    return ctx_stride_of(max_ctx);
}

uint64_t syn_hip_kv_state_bytes(uint32_t max_ctx, uint32_t n_kv_heads, uint32_t head_dim) {
    const uint64_t row = uint64_t{n_kv_heads} * head_dim;
    return align256(uint64_t{max_ctx} * row * 2) + align256(row * ctx_stride_of(max_ctx) * 2);
}

uint64_t syn_hip_attention_scratch_bytes(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_ctx,
                                         uint32_t max_batch) {
    (void)max_batch;  // runs of more than one token use the flash kernel, which needs none
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0) {
        return 0;
    }
    const uint32_t splits = (max_ctx + syn::decode_chunk_unit - 1) / syn::decode_chunk_unit;
    return align256(decode_scratch_bytes(splits, n_kv_heads, n_heads / n_kv_heads, head_dim));
}

int syn_hip_kv_append(syn_arena* a, const syn_kv_desc* cache, uint64_t k_rows, uint64_t v_rows, uint32_t n,
                      uint32_t pos0, uint32_t kv_dtype) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (cache == nullptr) {
        return fail(SYN_HIP_EINVAL, "null cache descriptor");
    }
    if (int e = check_cache(a, *cache)) {
        return e;
    }
    if (!dtype_ok(kv_dtype)) {
        return fail(SYN_HIP_EINVAL, "kv_append: dtype %u", kv_dtype);
    }
    if (n == 0) {
        return SYN_HIP_OK;
    }
    if (uint64_t{pos0} + n > cache->max_ctx) {
        return fail(SYN_HIP_EINVAL, "kv_append: rows %u..%u on a cache of %u", pos0, pos0 + n - 1, cache->max_ctx);
    }
    const uint64_t bytes = uint64_t{n} * cache->n_kv_heads * cache->head_dim * dtype_size(kv_dtype);
    if (int e = check_range(a, k_rows, bytes, dtype_size(kv_dtype), "kv_append k")) {
        return e;
    }
    if (int e = check_range(a, v_rows, bytes, dtype_size(kv_dtype), "kv_append v")) {
        return e;
    }
    return hip_status(syn::launch_kv_append(layout_of(a, *cache), a->base + k_rows, a->base + v_rows, n, pos0,
                                            kv_dtype, a->stream),
                      "kv_append launch");
}

int syn_hip_attention(syn_arena* a, const syn_attn_desc* d) {
    if (int e = check_attn(a, d, true)) {
        return e;
    }
    if (decode_shape(d)) {
        return attend_checked(a, d, true);  // the decode kernel appends the row itself
    }
    if (int e = syn_hip_kv_append(a, &d->cache, d->k_offset, d->v_offset, d->n, d->pos, d->kv_dtype)) {
        return e;
    }
    return attend_checked(a, d, false);
}

int syn_hip_attention_noalloc(syn_arena* a, const syn_attn_desc* d) {
    if (int e = check_attn(a, d, true)) {
        return e;
    }
    if (!decode_shape(d)) {
        // Runs of more than one token (and shapes outside the split-KV
        // kernel) use no scratch: the same launches as syn_hip_attention.
        return syn_hip_attention(a, d);
    }
    float* dev = scratch_device[a->device];
    if (dev == nullptr) {
        return fail(SYN_HIP_ENODEV, "static scratch of device %d was not looked up", a->device);
    }
    const partial_area area{0, noalloc_scratch_bytes, dev};
    return attend_checked(a, d, true, &area);
}

int syn_hip_attn_temperature(syn_arena* a, const syn_temperature_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->floor_len == 0 || d->size == 0) {
        return fail(SYN_HIP_EINVAL, "attn_temperature: size %u, floor_len %u", d->size, d->floor_len);
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t bytes = uint64_t{d->n} * d->size * 4;
    if (int e = check_range(a, d->in_offset, bytes, 4, "attn_temperature in")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "attn_temperature out")) {
        return e;
    }
    return hip_status(syn::launch_attn_temperature(reinterpret_cast<const float*>(a->base + d->in_offset),
                                                   reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->size,
                                                   d->pos, d->floor_len, d->scale, a->stream),
                      "attn_temperature launch");
}

int syn_hip_attention_rope(syn_arena* a, const syn_attn_desc* d, const syn_attn_rope_desc* r) {
    if (int e = check_attn(a, d, true)) {
        return e;
    }
    if (r == nullptr) {
        return fail(SYN_HIP_EINVAL, "null RoPE descriptor");
    }
    const syn_kv_desc& c = d->cache;
    if (d->q_dtype != SYN_F32 || d->kv_dtype != SYN_F32 || c.head_dim % 2 != 0 || r->mode > 1 ||
        c.head_dim > 2 * syn::rope_max_pairs) {
        return fail(SYN_HIP_EINVAL, "attention_rope: q dtype %u, k dtype %u (want f32), head_dim %u, mode %u",
                    d->q_dtype, d->kv_dtype, c.head_dim, r->mode);
    }
    const float* ff = nullptr;
    if (r->freq_factors_offset != no_offset) {
        if (int e = check_range(a, r->freq_factors_offset, uint64_t{c.head_dim} / 2 * 4, 16, "rope freq_factors")) {
            return e;
        }
        ff = reinterpret_cast<const float*>(a->base + r->freq_factors_offset);
    }
    if (decode_shape(d)) {
        // One kernel: q and the new K row rotated in LDS, the K row appended.
        syn::rope_params rp{};
        rp.freq_factors = ff;
        rp.mode = r->mode;
        rp.theta_scale = r->theta_scale;
        rp.freq_scale = r->freq_scale;
        rp.ext_factor = r->ext_factor;
        rp.attn_factor = r->attn_factor;
        rp.corr_low = r->corr_low;
        rp.corr_high = r->corr_high;
        rp.temp_scale = r->temp_scale;
        rp.temp_floor_len = r->temp_floor_len;
        return attend_checked(a, d, true, nullptr, &rp);
    }
    // A run (or a head size the split-KV kernel does not take): one launch
    // rotates q (times the temperature) into binary16 rows at q_out_offset,
    // rotates and appends the K rows and appends the V rows; then the
    // attention kernel reads those q rows. binary16 is the rounding every
    // attention kernel applies to f32 q, so this equals the separate calls.
    const uint64_t q_bytes = uint64_t{d->n} * d->n_heads * c.head_dim * 4;
    const uint64_t kv_bytes = uint64_t{d->n} * c.n_kv_heads * c.head_dim * 4;
    if (int e = check_range(a, r->q_out_offset, q_bytes, 16, "attention_rope q_out")) {
        return e;
    }
    const auto overlap = [](uint64_t p, uint64_t pn, uint64_t q, uint64_t qn) { return p < q + qn && q < p + pn; };
    if (overlap(r->q_out_offset, q_bytes, d->q_offset, q_bytes) ||
        overlap(r->q_out_offset, q_bytes, d->k_offset, kv_bytes) ||
        overlap(r->q_out_offset, q_bytes, d->v_offset, kv_bytes)) {
        return fail(SYN_HIP_EINVAL, "attention_rope: q_out overlaps the q, k or v rows");
    }
    syn::append_run_args ar{};
    ar.k_rows = a->base + d->k_offset;
    ar.v_rows = a->base + d->v_offset;
    ar.k_cache = reinterpret_cast<_Float16*>(a->base + c.k_offset);
    ar.vt_cache = reinterpret_cast<_Float16*>(a->base + c.v_offset);
    ar.row = c.n_kv_heads * c.head_dim;
    ar.hd = c.head_dim;
    ar.n = d->n;
    ar.pos0 = d->pos;
    ar.ctx_stride = c.ctx_stride;
    ar.q = reinterpret_cast<const float*>(a->base + d->q_offset);
    ar.q16 = reinterpret_cast<_Float16*>(a->base + r->q_out_offset);
    ar.q_size = d->n_heads * c.head_dim;
    ar.r.freq_factors = ff;
    ar.r.mode = r->mode;
    ar.r.theta_scale = r->theta_scale;
    ar.r.freq_scale = r->freq_scale;
    ar.r.ext_factor = r->ext_factor;
    ar.r.attn_factor = r->attn_factor;
    ar.r.corr_low = r->corr_low;
    ar.r.corr_high = r->corr_high;
    ar.r.temp_scale = r->temp_scale;
    ar.r.temp_floor_len = r->temp_floor_len;
    if (int e = hip_status(syn::launch_append_run(ar, 0, true, a->stream), "rope append launch")) {
        return e;
    }
    syn_attn_desc rotated = *d;
    rotated.q_offset = r->q_out_offset;
    rotated.q_dtype = SYN_F16;
    return attend_checked(a, &rotated, false);
}

uint64_t syn_hip_attention_noalloc_scratch_limit(void) {
    return noalloc_scratch_bytes;
}

int syn_hip_attend(syn_arena* a, const syn_attn_desc* d) {
    if (int e = check_attn(a, d, false)) {
        return e;
    }
    return attend_checked(a, d, false);
}

uint64_t syn_hip_attend_batch_scratch_bytes(const syn_seq_desc* seqs, uint32_t n_seqs, uint32_t n_heads) {
    if (seqs == nullptr || n_seqs == 0 || seqs[0].cache.n_kv_heads == 0) {
        return 0;
    }
    const uint32_t n_kv = seqs[0].cache.n_kv_heads;
    const uint32_t hd = seqs[0].cache.head_dim;
    const uint32_t per = syn::decode_max_seqs;
    uint64_t worst = 0;
    for (uint32_t b0 = 0; b0 < n_seqs; b0 += per) {
        const uint32_t nb = std::min(n_seqs - b0, per);
        uint64_t positions = 0;
        uint32_t max_len = 0;
        for (uint32_t i = 0; i < nb; ++i) {
            positions += uint64_t{seqs[b0 + i].pos} + 1;
            max_len = std::max(max_len, seqs[b0 + i].pos + 1);
        }
        const uint32_t chunk = syn::decode_choose_chunk(positions, n_kv, max_len);
        uint64_t splits = 0;
        for (uint32_t i = 0; i < nb; ++i) {
            splits += (uint64_t{seqs[b0 + i].pos} + chunk) / chunk;
        }
        worst = std::max(worst, splits * n_kv * syn::decode_split_floats(n_heads / n_kv, hd) * sizeof(float));
    }
    return align256(worst);
}

int syn_hip_attend_batch(syn_arena* a, const syn_seq_desc* seqs, uint32_t n_seqs, uint32_t n_heads, float scale,
                         uint32_t q_dtype, uint64_t scratch_offset, uint64_t scratch_bytes) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (seqs == nullptr || n_seqs == 0) {
        return fail(SYN_HIP_EINVAL, "attend_batch: no sequences");
    }
    if (!(std::isfinite(scale) && scale > 0.0f) || !dtype_ok(q_dtype)) {
        return fail(SYN_HIP_EINVAL, "attend_batch: scale %g, dtype %u", static_cast<double>(scale), q_dtype);
    }
    const uint32_t n_kv = seqs[0].cache.n_kv_heads;
    const uint32_t hd = seqs[0].cache.head_dim;
    for (uint32_t i = 0; i < n_seqs; ++i) {
        const syn_seq_desc& s = seqs[i];
        if (int e = check_cache(a, s.cache)) {
            return e;
        }
        if (s.cache.n_kv_heads != n_kv || s.cache.head_dim != hd) {
            return fail(SYN_HIP_EINVAL, "attend_batch: sequence %u has a different head layout", i);
        }
        if (s.pos >= s.cache.max_ctx) {
            return fail(SYN_HIP_EINVAL, "attend_batch: sequence %u at position %u of %u", i, s.pos,
                        s.cache.max_ctx);
        }
        const uint64_t qsize = uint64_t{n_heads} * hd;
        if (int e = check_range(a, s.q_offset, qsize * dtype_size(q_dtype), 16, "attend_batch q")) {
            return e;
        }
        if (int e = check_range(a, s.out_offset, qsize * 4, 16, "attend_batch out")) {
            return e;
        }
    }
    if (n_heads == 0 || n_heads % n_kv != 0) {
        return fail(SYN_HIP_EINVAL, "attend_batch: %u query heads on %u KV heads", n_heads, n_kv);
    }
    const uint32_t group = n_heads / n_kv;
    const uint32_t per = syn::decode_max_seqs;
    bool fits = true;
    for (uint32_t b0 = 0; fits && b0 < n_seqs; b0 += per) {
        const uint32_t nb = std::min(n_seqs - b0, per);
        uint64_t positions = 0;
        uint32_t max_len = 0;
        for (uint32_t i = 0; i < nb; ++i) {
            positions += uint64_t{seqs[b0 + i].pos} + 1;
            max_len = std::max(max_len, seqs[b0 + i].pos + 1);
        }
        const uint32_t chunk = syn::decode_choose_chunk(positions, n_kv, max_len);
        for (uint32_t i = 0; i < nb; ++i) {
            fits = fits && syn::decode_fits(chunk, n_kv * hd, hd, seqs[b0 + i].cache.ctx_stride);
        }
    }
    if (!fast_shape(hd) || group > 16 || !fits) {
        // Shapes outside the split-KV kernel: one causal launch per sequence.
        for (uint32_t i = 0; i < n_seqs; ++i) {
            syn_attn_desc d{};
            d.cache = seqs[i].cache;
            d.q_offset = seqs[i].q_offset;
            d.out_offset = seqs[i].out_offset;
            d.n_heads = n_heads;
            d.pos = seqs[i].pos;
            d.n = 1;
            d.scale = scale;
            d.q_dtype = q_dtype;
            const syn::flash_args f = flash_of(a, &d);
            if (int e = hip_status(syn::launch_generic_causal(f, q_dtype, a->stream), "generic launch")) {
                return e;
            }
        }
        return SYN_HIP_OK;
    }
    for (uint32_t b0 = 0; b0 < n_seqs; b0 += per) {
        const uint32_t nb = std::min(n_seqs - b0, per);
        syn::decode_seq ds[syn::decode_max_seqs];
        for (uint32_t i = 0; i < nb; ++i) {
            const syn_seq_desc& s = seqs[b0 + i];
            ds[i] = syn::decode_seq{};
            ds[i].q = a->base + s.q_offset;
            ds[i].out = reinterpret_cast<float*>(a->base + s.out_offset);
            ds[i].k = reinterpret_cast<_Float16*>(a->base + s.cache.k_offset);
            ds[i].vt = reinterpret_cast<_Float16*>(a->base + s.cache.v_offset);
            ds[i].len = s.pos + 1;
            ds[i].ctx_stride = s.cache.ctx_stride;
        }
        if (int e = run_decode(a, ds, nb, n_kv, hd, group, scale, q_dtype, SYN_F32,
                               partial_area{scratch_offset, scratch_bytes, nullptr})) {
            return e;
        }
    }
    return SYN_HIP_OK;
}

int syn_hip_self_attention(syn_arena* a, const syn_self_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->n == 0 || d->batch == 0 || d->n_heads == 0 || d->head_dim == 0 || d->head_dim > 256 ||
        !dtype_ok(d->in_dtype)) {
        return fail(SYN_HIP_EINVAL, "self_attention: n %u, batch %u, heads %u, head_dim %u, dtype %u", d->n,
                    d->batch, d->n_heads, d->head_dim, d->in_dtype);
    }
    if (!(std::isfinite(d->scale) && d->scale > 0.0f)) {
        return fail(SYN_HIP_EINVAL, "self_attention: scale %g", static_cast<double>(d->scale));
    }
    const uint64_t rows = uint64_t{d->n} * d->batch;
    const uint64_t size = uint64_t{d->n_heads} * d->head_dim;
    const uint64_t in_bytes = rows * size * dtype_size(d->in_dtype);
    const uint64_t align = fast_shape(d->head_dim) ? 16 : dtype_size(d->in_dtype);
    if (int e = check_range(a, d->q_offset, in_bytes, align, "self_attention q")) {
        return e;
    }
    if (int e = check_range(a, d->k_offset, in_bytes, align, "self_attention k")) {
        return e;
    }
    if (int e = check_range(a, d->v_offset, in_bytes, align, "self_attention v")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, rows * size * 4, fast_shape(d->head_dim) ? 16 : 4,
                            "self_attention out")) {
        return e;
    }
    syn::flash_args f{};
    f.q = a->base + d->q_offset;
    f.out = reinterpret_cast<float*>(a->base + d->out_offset);
    f.k_rows = a->base + d->k_offset;
    f.v_rows = a->base + d->v_offset;
    f.n = d->n;
    f.batch = d->batch;
    f.pos = 0;
    f.kv_len = d->n;
    f.n_heads = d->n_heads;
    f.n_kv = d->n_heads;
    f.hd = d->head_dim;
    f.group = 1;
    f.q_row = static_cast<uint32_t>(size);
    f.row = static_cast<uint32_t>(size);
    f.scale_log2e = d->scale * syn::log2e;
    f.scale = d->scale;
    if (d->in_dtype == SYN_F32 && syn::self_f32_fits(d->n)) {
        return hip_status(syn::launch_self_f32(f, a->stream), "self_attention launch");
    }
    if (fast_shape(d->head_dim)) {
        return hip_status(syn::launch_bidirectional(f, d->in_dtype, a->stream), "self_attention launch");
    }
    return hip_status(syn::launch_generic_bidirectional(f, d->in_dtype, a->stream), "self_attention launch");
}

int syn_hip_rope(syn_arena* a, const syn_rope_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->head_dim == 0 || d->head_dim % 2 != 0 || d->head_dim > 2 * syn::rope_max_pairs || d->size == 0 ||
        d->size % d->head_dim != 0 || d->mode > 1) {
        return fail(SYN_HIP_EINVAL, "rope: size %u, head_dim %u (even, <= 256), mode %u", d->size, d->head_dim,
                    d->mode);
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t bytes = uint64_t{d->n} * d->size * 4;
    if (int e = check_range(a, d->in_offset, bytes, 4, "rope in")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "rope out")) {
        return e;
    }
    if (d->in_offset < d->out_offset + bytes && d->out_offset < d->in_offset + bytes) {
        return fail(SYN_HIP_EINVAL, "rope: out aliases in");
    }
    syn::rope_args r{};
    r.in = reinterpret_cast<const float*>(a->base + d->in_offset);
    r.out = reinterpret_cast<float*>(a->base + d->out_offset);
    if (d->freq_factors_offset != no_offset) {
        if (int e = check_range(a, d->freq_factors_offset, uint64_t{d->head_dim} / 2 * 4, 4, "rope freq_factors")) {
            return e;
        }
        r.freq_factors = reinterpret_cast<const float*>(a->base + d->freq_factors_offset);
    }
    r.n = d->n;
    r.size = d->size;
    r.hd = d->head_dim;
    r.pos = d->pos;
    r.mode = d->mode;
    r.theta_scale = d->theta_scale;
    r.freq_scale = d->freq_scale;
    r.ext_factor = d->ext_factor;
    r.attn_factor = d->attn_factor;
    r.corr_low = d->corr_low;
    r.corr_high = d->corr_high;
    r.period = d->period;
    return hip_status(syn::launch_rope(r, a->stream), "rope launch");
}

int syn_hip_embed(syn_arena* a, const syn_embed_desc* d, const uint32_t* tokens, uint32_t n) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr || (tokens == nullptr && n > 0)) {
        return fail(SYN_HIP_EINVAL, "null descriptor or tokens");
    }
    if (d->size == 0 || d->n_table_rows == 0) {
        return fail(SYN_HIP_EINVAL, "embed: %u rows of size %u", d->n_table_rows, d->size);
    }
    const bool quantized = d->table_type != SYN_TYPE_F32;
    if (quantized && (!syn::qtype_known(d->table_type) || d->size % syn::qtype_block(d->table_type) != 0)) {
        return fail(SYN_HIP_EINVAL, "embed: table type %u with rows of %u", d->table_type, d->size);
    }
    if (n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t row_bytes = quantized ? syn::qtype_row_bytes(d->table_type, d->size) : uint64_t{d->size} * 4;
    if (int e = check_range(a, d->table_offset, uint64_t{d->n_table_rows} * row_bytes, quantized ? 1 : 4,
                            "embed table")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, uint64_t{n} * d->size * 4, 4, "embed out")) {
        return e;
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (tokens[i] >= d->n_table_rows) {
            return fail(SYN_HIP_EINVAL, "embed: token %u at %u, table has %u rows", tokens[i], i, d->n_table_rows);
        }
    }
    auto* out = reinterpret_cast<float*>(a->base + d->out_offset);
    for (uint32_t i0 = 0; i0 < n; i0 += syn::embed_max_tokens) {
        const uint32_t m = std::min(n - i0, syn::embed_max_tokens);
        syn::embed_tokens t{};
        std::copy(tokens + i0, tokens + i0 + m, t.token);
        float* dst = out + uint64_t{i0} * d->size;
        const char* table = a->base + d->table_offset;
        const hipError_t err =
            quantized ? syn::launch_embed_q(d->table_type, reinterpret_cast<const uint8_t*>(table), dst, t, m, d->size,
                                            a->stream)
                      : syn::launch_embed(reinterpret_cast<const float*>(table), dst, t, m, d->size, a->stream);
        if (int e = hip_status(err, "embed launch")) {
            return e;
        }
    }
    return SYN_HIP_OK;
}

int syn_hip_rms_norm(syn_arena* a, const syn_norm_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->size == 0 || !(std::isfinite(d->eps) && d->eps >= 0.0f)) {
        return fail(SYN_HIP_EINVAL, "rms_norm: size %u, eps %g", d->size, static_cast<double>(d->eps));
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t bytes = uint64_t{d->n} * d->size * 4;
    if (int e = check_range(a, d->in_offset, bytes, 4, "rms_norm in")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "rms_norm out")) {
        return e;
    }
    if (int e = check_range(a, d->weight_offset, uint64_t{d->size} * 4, 4, "rms_norm weight")) {
        return e;
    }
    return hip_status(syn::launch_rms_norm(reinterpret_cast<const float*>(a->base + d->in_offset),
                                           reinterpret_cast<const float*>(a->base + d->weight_offset),
                                           reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->size, d->eps,
                                           a->stream),
                      "rms_norm launch");
}

int syn_hip_matmul(syn_arena* a, const syn_matmul_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->rows == 0 || d->cols == 0 || d->n > 65535) {
        return fail(SYN_HIP_EINVAL, "matmul: %u x %u weights, %u rows", d->rows, d->cols, d->n);
    }
    if (syn::matmul_q_rows_per_pass(1, d->cols) == 0) {
        return fail(SYN_HIP_EUNSUPPORTED, "matmul_q: %u columns exceed the activation LDS", d->cols);
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t x_bytes = uint64_t{d->n} * d->cols * 4;
    const uint64_t out_bytes = uint64_t{d->n} * d->rows * 4;
    if (int e = check_range(a, d->w_offset, uint64_t{d->rows} * d->cols * 4, 4, "matmul w")) {
        return e;
    }
    if (int e = check_range(a, d->x_offset, x_bytes, 4, "matmul x")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, out_bytes, 4, "matmul out")) {
        return e;
    }
    if (d->x_offset < d->out_offset + out_bytes && d->out_offset < d->x_offset + x_bytes) {
        return fail(SYN_HIP_EINVAL, "matmul: out aliases x");
    }
    const float* bias = nullptr;
    if (d->bias_offset != no_offset) {
        if (int e = check_range(a, d->bias_offset, uint64_t{d->rows} * 4, 4, "matmul bias")) {
            return e;
        }
        bias = reinterpret_cast<const float*>(a->base + d->bias_offset);
    }
    return hip_status(syn::launch_matmul(reinterpret_cast<const float*>(a->base + d->w_offset),
                                         reinterpret_cast<const float*>(a->base + d->x_offset), bias,
                                         reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->rows, d->cols,
                                         a->stream),
                      "matmul launch");
}

uint64_t syn_hip_matmul_q_act_bytes(uint32_t w_type, uint32_t n, uint32_t cols) {
    if (!syn::qtype_known(w_type) || cols % syn::qtype_block(w_type) != 0) {
        return 0;
    }
    return syn::qtype_act_bytes(w_type, n, cols);
}

int syn_hip_matmul_q(syn_arena* a, const syn_matmul_q_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (!syn::qtype_known(d->w_type)) {
        return fail(SYN_HIP_EUNSUPPORTED, "matmul_q: weight type %u", d->w_type);
    }
    if (d->rows == 0 || d->cols == 0 || d->cols % syn::qtype_block(d->w_type) != 0 || d->n > 65535 ||
        syn::qtype_row_bytes(d->w_type, d->cols) >= (uint64_t{1} << 31)) {
        return fail(SYN_HIP_EINVAL, "matmul_q: %u x %u weights of type %u, %u rows", d->rows, d->cols, d->w_type,
                    d->n);
    }
    if (syn::matmul_q_rows_per_pass(1, d->cols) == 0) {
        return fail(SYN_HIP_EUNSUPPORTED, "matmul_q: %u columns exceed the activation LDS", d->cols);
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t x_bytes = uint64_t{d->n} * d->cols * 4;
    const uint64_t out_bytes = uint64_t{d->n} * d->rows * 4;
    const uint64_t act_bytes = syn::qtype_act_bytes(d->w_type, d->n, d->cols);
    if (int e = check_range(a, d->w_offset, uint64_t{d->rows} * syn::qtype_row_bytes(d->w_type, d->cols), 4,
                            "matmul_q w")) {
        return e;
    }
    if (int e = check_range(a, d->x_offset, x_bytes, 16, "matmul_q x")) {
        return e;
    }
    if (int e = check_range(a, d->act_offset, act_bytes, 4, "matmul_q act")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, out_bytes, 4, "matmul_q out")) {
        return e;
    }
    const auto overlap = [](uint64_t p, uint64_t pn, uint64_t q, uint64_t qn) { return p < q + qn && q < p + pn; };
    if (overlap(d->act_offset, act_bytes, d->x_offset, x_bytes) ||
        overlap(d->act_offset, act_bytes, d->out_offset, out_bytes) ||
        overlap(d->act_offset, act_bytes, d->w_offset, uint64_t{d->rows} * syn::qtype_row_bytes(d->w_type, d->cols))) {
        return fail(SYN_HIP_EINVAL, "matmul_q: act overlaps an operand");
    }
    const float* bias = nullptr;
    if (d->bias_offset != no_offset) {
        if (int e = check_range(a, d->bias_offset, uint64_t{d->rows} * 4, 4, "matmul_q bias")) {
            return e;
        }
        bias = reinterpret_cast<const float*>(a->base + d->bias_offset);
    }
    return hip_status(syn::launch_matmul_q(d->w_type, reinterpret_cast<const uint8_t*>(a->base + d->w_offset),
                                           reinterpret_cast<const float*>(a->base + d->x_offset),
                                           reinterpret_cast<uint8_t*>(a->base + d->act_offset), bias,
                                           reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->rows, d->cols,
                                           a->stream),
                      "matmul_q launch");
}

int syn_hip_elementwise(syn_arena* a, const syn_elementwise_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->op > SYN_ADD_BIAS) {
        return fail(SYN_HIP_EINVAL, "elementwise: op %u", d->op);
    }
    if (d->count == 0) {
        return SYN_HIP_OK;
    }
    if (d->count > (uint64_t{1} << 40)) {
        return fail(SYN_HIP_EINVAL, "elementwise: count %llu", static_cast<unsigned long long>(d->count));
    }
    const uint64_t bytes = d->count * 4;
    if (int e = check_range(a, d->a_offset, bytes, 4, "elementwise a")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "elementwise out")) {
        return e;
    }
    const float* b = nullptr;
    if (d->op == SYN_ADD_BIAS) {
        if (d->period == 0 || d->count % d->period != 0) {
            return fail(SYN_HIP_EINVAL, "elementwise: period %u for count %llu", d->period,
                        static_cast<unsigned long long>(d->count));
        }
        if (int e = check_range(a, d->b_offset, uint64_t{d->period} * 4, 4, "elementwise bias")) {
            return e;
        }
        b = reinterpret_cast<const float*>(a->base + d->b_offset);
    } else if (d->op != SYN_SCALE && d->op != SYN_GELU && d->op != SYN_SILU) {
        if (int e = check_range(a, d->b_offset, bytes, 4, "elementwise b")) {
            return e;
        }
        b = reinterpret_cast<const float*>(a->base + d->b_offset);
    }
    return hip_status(syn::launch_elementwise(reinterpret_cast<const float*>(a->base + d->a_offset), b,
                                              reinterpret_cast<float*>(a->base + d->out_offset), d->count, d->op,
                                              d->scalar, d->period, a->stream),
                      "elementwise launch");
}

int syn_hip_softmax(syn_arena* a, const syn_softmax_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->size == 0) {
        return fail(SYN_HIP_EINVAL, "softmax: size 0");
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t bytes = uint64_t{d->n} * d->size * 4;
    if (int e = check_range(a, d->in_offset, bytes, 4, "softmax in")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "softmax out")) {
        return e;
    }
    if (d->in_offset != d->out_offset && d->in_offset < d->out_offset + bytes && d->out_offset < d->in_offset + bytes) {
        return fail(SYN_HIP_EINVAL, "softmax: out overlaps in without being it");
    }
    return hip_status(syn::launch_softmax(reinterpret_cast<const float*>(a->base + d->in_offset),
                                          reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->size,
                                          a->stream),
                      "softmax launch");
}

int syn_hip_layer_norm(syn_arena* a, const syn_layer_norm_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->size == 0 || !(std::isfinite(d->eps) && d->eps >= 0.0f)) {
        return fail(SYN_HIP_EINVAL, "layer_norm: size %u, eps %g", d->size, static_cast<double>(d->eps));
    }
    if (d->n == 0) {
        return SYN_HIP_OK;
    }
    const uint64_t bytes = uint64_t{d->n} * d->size * 4;
    if (int e = check_range(a, d->in_offset, bytes, 4, "layer_norm in")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "layer_norm out")) {
        return e;
    }
    if (int e = check_range(a, d->weight_offset, uint64_t{d->size} * 4, 4, "layer_norm weight")) {
        return e;
    }
    const float* beta = nullptr;
    if (d->bias_offset != no_offset) {
        if (int e = check_range(a, d->bias_offset, uint64_t{d->size} * 4, 4, "layer_norm bias")) {
            return e;
        }
        beta = reinterpret_cast<const float*>(a->base + d->bias_offset);
    }
    return hip_status(syn::launch_layer_norm(reinterpret_cast<const float*>(a->base + d->in_offset),
                                             reinterpret_cast<const float*>(a->base + d->weight_offset), beta,
                                             reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->size, d->eps,
                                             a->stream),
                      "layer_norm launch");
}

int syn_hip_pixel_shuffle(syn_arena* a, const syn_pixel_shuffle_desc* d) {
    if (int e = check_arena(a)) {
        return e;
    }
    if (d == nullptr) {
        return fail(SYN_HIP_EINVAL, "null descriptor");
    }
    if (d->n == 0 || d->scale == 0 || d->grid_w == 0 || d->grid_h == 0 || d->grid_w % d->scale != 0 ||
        d->grid_h % d->scale != 0) {
        return fail(SYN_HIP_EINVAL, "pixel_shuffle: %u x %u grid of %u, scale %u", d->grid_w, d->grid_h, d->n,
                    d->scale);
    }
    const uint64_t bytes = uint64_t{d->grid_w} * d->grid_h * d->n * 4;
    if (int e = check_range(a, d->in_offset, bytes, 4, "pixel_shuffle in")) {
        return e;
    }
    if (int e = check_range(a, d->out_offset, bytes, 4, "pixel_shuffle out")) {
        return e;
    }
    if (d->in_offset < d->out_offset + bytes && d->out_offset < d->in_offset + bytes) {
        return fail(SYN_HIP_EINVAL, "pixel_shuffle: out aliases in");
    }
    return hip_status(syn::launch_pixel_shuffle(reinterpret_cast<const float*>(a->base + d->in_offset),
                                                reinterpret_cast<float*>(a->base + d->out_offset), d->n, d->grid_w,
                                                d->grid_h, d->scale, a->stream),
                      "pixel_shuffle launch");
}

}  // extern "C"
