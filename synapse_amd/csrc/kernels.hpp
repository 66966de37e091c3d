// kernels.hpp — host-side launch interface of the attention kernels. Each
// launcher queues its kernels on `stream` and returns hipGetLastError(); the
// C ABI (capi.hip) validates every shape and offset before calling one.
#pragma once

#include "device.hpp"
#include "rope_math.hpp"

#include <cstddef>
#include <cstdint>

namespace syn {

// One KV state resolved to device pointers. K: [max_ctx][n_kv][hd];
// V^T: [n_kv][hd][ctx_stride].
struct kv_layout {
    _Float16* k;
    _Float16* vt;
    uint32_t max_ctx, n_kv, hd, ctx_stride;
};

hipError_t launch_kv_append(const kv_layout& c, const void* k_rows, const void* v_rows, uint32_t n, uint32_t pos0,
                            uint32_t dtype, hipStream_t stream);

// ---- split-KV decode --------------------------------------------------------
// One query row attending cache rows 0..len-1.
struct decode_seq {
    const void* q;        // n_heads * hd, f32 or f16
    float* out;           // n_heads * hd
    _Float16* k;          // K block
    _Float16* vt;         // V^T block
    const void* k_new;    // the step's new K row (position len-1, n_kv * hd of kv_dtype), or nullptr:
    const void* v_new;    //   the kernel then stores it into the cache (kv_append) and attends it
    uint32_t len;         // attended positions
    uint32_t ctx_stride;  // V^T row length
    uint32_t block0;      // first split of this sequence in the launch's split numbering
    uint32_t n_splits;    // ceil(len / chunk), <= decode_max_splits
    uint32_t merge0;      // first merge block of this sequence (sequences with one split have none)
};

constexpr uint32_t decode_max_seqs = 32;  // sequences per batched launch (kernel-argument table)
constexpr uint32_t decode_positions_per_wave = 32;
constexpr uint32_t decode_waves = 4;
constexpr uint32_t decode_chunk_unit = decode_positions_per_wave * decode_waves;  // 128
constexpr uint32_t decode_max_splits = 256;  // splits of one sequence

// The splits of a sequence are combined by a second, small kernel on the same
// stream: one block per (sequence with splits, query head). (Merging inside
// the split kernel, through arrival counters and agent-scope loads, measured
// slower: each cross-block hop costs a loaded memory round trip, and the
// merge needs three or four of them.)
struct decode_params {
    float* part;           // partial O [slots][group][hd], then (max, sum) [slots][group][2]; slot = split * n_kv + g
    uint32_t n_kv;
    uint32_t hd;
    uint32_t group;        // query heads per KV head, <= 16
    uint32_t row;          // n_kv * hd: K row length in halves
    uint32_t chunk;        // positions per split, a multiple of decode_chunk_unit
    uint32_t kv_dtype;     // type of k_new / v_new: 0 f32, 1 f16
    uint32_t total_slots;  // split blocks of the launch: splits * n_kv
    uint32_t merge_blocks; // blocks of the merge kernel: n_kv * group per sequence with splits
    uint32_t n_seqs;
    float scale_log2e;     // scale * log2(e)
};

// One sequence: the argument block a decode step carries (~120 bytes; a
// kernel-argument block of kilobytes costs a microsecond per launch).
struct decode_one_args {
    decode_params p;
    decode_seq s;
};

// Up to decode_max_seqs sequences in one launch (ragged batched decode).
struct decode_batch_args {
    decode_params p;
    decode_seq seq[decode_max_seqs];
    uint32_t block0s[decode_max_seqs];  // seq[i].block0, contiguous: a block finds its sequence in one load batch
    uint32_t merge0s[decode_max_seqs];  // seq[i].merge0, likewise for the merge kernel
};

// RoPE and the attention temperature inside a single-sequence decode step:
// the step's q row and new K row are rotated as op_rope rotates them
// (S/kernels/attention.hpp:89-129), then q is multiplied by the
// op_attn_temperature factor of the step's position (S/kernels/
// elementwise.hpp:66-72; none when temp_floor_len is 0), computed on the
// device by attn_temperature, before q's rounding to binary16. The same
// arithmetic as the rope and temperature kernels, so the fused step equals
// the unfused one bit for bit. q and the new rows are f32.
struct rope_params {
    const float* freq_factors;  // head_dim / 2 floats, or nullptr
    uint32_t mode;              // 0 normal (pairs 2i, 2i + 1), 1 neox (pairs i, i + hd/2)
    float theta_scale, freq_scale, ext_factor, attn_factor, corr_low, corr_high;
    float temp_scale;           // attention temperature: 1 + temp_scale ln(floor(pos / temp_floor_len) + 1)
    uint32_t temp_floor_len;    //   0: no temperature
};

struct decode_rope_args {
    decode_params p;
    decode_seq s;
    rope_params r;
};
hipError_t launch_decode(const decode_rope_args& a, uint32_t q_dtype, hipStream_t stream);


constexpr uint32_t rope_max_pairs = 128;  // head_dim <= 256, as attention's

// The angles of RoPE pairs 0 .. n_pairs-1 at position pos, as rope() builds
// them (S/kernels/attention.hpp:101-127): pos times theta_scale p times over
// by repeated f32 multiplication (not pow), so each angle is the reference's
// to the last bit. One lane runs the chain and stores every angle to th (LDS)
// as it goes: the chain is the only dependency. (Every lane running it and
// keeping the values at its own pairs by compare and select per step cost
// 1.9 us per fused decode step; a chain per lane of its own length was a
// divergent loop.) The calling wave may read th right after: its LDS
// operations complete in order.
__device__ inline void rope_angles(uint32_t pos, float theta_scale, uint32_t n_pairs, float* th) {
#pragma clang fp contract(off)
    float t = static_cast<float>(pos);
    th[0] = t;
#pragma unroll 8
    for (uint32_t j = 1; j < n_pairs; ++j) {
        t *= theta_scale;
        th[j] = t;
    }
}

// cos and sin of RoPE pair p with angle theta (rope_angles), times the YaRN
// magnitude, as rope() computes them (S/kernels/attention.hpp:101-121): every
// product and sum rounds on its own; cos and sin of the f32 angle from
// sincos_of. R has the fields of rope_params (theta_scale .. corr_high).
template <class R>
__device__ inline void rope_coeffs(const R& r, float theta, uint32_t p, float ff, float& cs, float& sn) {
#pragma clang fp contract(off)
    const float theta_extrap = theta / ff;
    const float theta_interp = r.freq_scale * theta_extrap;
    float t = theta_interp;
    float mscale = r.attn_factor;
    if (r.ext_factor != 0.0f) {
        const float yv = (static_cast<float>(p) - r.corr_low) / fmaxf(0.001f, r.corr_high - r.corr_low);
        const float ramp_mix = (1 - fminf(1.0f, fmaxf(0.0f, yv))) * r.ext_factor;
        t = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / r.freq_scale);
    }
    float c1, s1;
    sincos_of(t, s1, c1);
    cs = c1 * mscale;
    sn = s1 * mscale;
}

// One wave builds the cos / sin table of every pair (n_pairs <= 128) into
// tab[0 .. n_pairs) / tab[n_pairs .. 2 n_pairs) from the angles rope_angles
// left in th; ff, if not null, holds the pairs' frequency factors.
template <class R>
__device__ inline void rope_table(const R& r, const float* th, uint32_t n_pairs, const float* ff, float* tab,
                                  uint32_t lane) {
    if (lane < n_pairs) {
        rope_coeffs(r, th[lane], lane, ff ? ff[lane] : 1.0f, tab[lane], tab[n_pairs + lane]);
    }
    if (lane + 64 < n_pairs) {
        rope_coeffs(r, th[lane + 64], lane + 64, ff ? ff[lane + 64] : 1.0f, tab[lane + 64], tab[n_pairs + lane + 64]);
    }
}

// The rotated pair: (x0 cs - x1 sn, x0 sn + x1 cs), each product and sum
// rounded on its own (S/kernels/attention.hpp:122-125).
__device__ __forceinline__ float rope_first(float x0, float x1, float cs, float sn) {
#pragma clang fp contract(off)
    return x0 * cs - x1 * sn;
}
__device__ __forceinline__ float rope_second(float x0, float x1, float cs, float sn) {
#pragma clang fp contract(off)
    return x0 * sn + x1 * cs;
}

// The attention temperature of position pos (kernels::attn_temperature,
// S/kernels/elementwise.hpp:66-72): a float quotient floored, the logarithm
// in double, the result rounded to float; the double multiply and add round
// on their own, as the reference's -ffp-contract=off build computes them.
// Only device code calls it (the row kernel and the fused decode step), so
// both use the same logarithm and agree bit for bit.
__device__ inline float attn_temperature(uint32_t pos, float scale, uint32_t floor_len) {
#pragma clang fp contract(off)
    const float q = floorf(static_cast<float>(pos) / static_cast<float>(floor_len));
    return static_cast<float>(log(static_cast<double>(q) + 1.0) * static_cast<double>(scale) + 1.0);
}

// A run's append (kv_append.hip): K rows to the cache, V rows to V^T, both
// rounded to binary16 (rows f32 or binary16). With RoPE (f32 rows only) the
// run's q and K rows are rotated on the way, as op_rope rotates them, and q
// is multiplied by the attention temperature (none when
// r.temp_floor_len is 0): q goes to q16 as binary16 rows, K to the cache.
struct append_run_args {
    const void* k_rows;      // n rows of `row` elements
    const void* v_rows;
    _Float16* k_cache;       // K rows of the cache (row 0)
    _Float16* vt_cache;      // V^T of the cache
    uint32_t row, hd, n, pos0, ctx_stride;
    const float* q;          // RoPE: n rows of q_size f32
    _Float16* q16;           // RoPE: n rows of q_size binary16 out
    uint32_t q_size;
    rope_params r;           // RoPE parameters and the temperature
    // set by launch_append_run
    uint32_t v_tiles, v_feat_tiles;
    bool vec;                // rows 16-byte aligned: vector loads
};
hipError_t launch_append_run(append_run_args a, uint32_t dtype, bool rope, hipStream_t stream);

// Scratch floats one split contributes: (max, sum, output) for each head.
inline std::size_t decode_split_floats(uint32_t group, uint32_t hd) {
    return static_cast<std::size_t>(group) * (hd + 2);
}

// Picks the chunk (positions per split) for a launch whose sequences attend
// `total_positions` positions across n_kv heads, the longest `max_len`.
uint32_t decode_choose_chunk(uint64_t total_positions, uint32_t n_kv, uint32_t max_len);

// The split kernel addresses a split's K rows and a head's V^T rows through
// 32-bit buffer offsets: both spans must stay below 2^31 bytes.
inline bool decode_fits(uint32_t chunk, uint32_t row, uint32_t hd, uint32_t ctx_stride) {
    return uint64_t{chunk} * row * 2 < (uint64_t{1} << 31) && uint64_t{hd} * ctx_stride * 2 < (uint64_t{1} << 31);
}

hipError_t launch_decode(const decode_one_args& a, uint32_t q_dtype, hipStream_t stream);
hipError_t launch_decode(const decode_batch_args& a, uint32_t q_dtype, hipStream_t stream);

// ---- flash prefill / bidirectional -----------------------------------------
struct flash_args {
    const void* q;         // rows [n][q_row], head h at h * hd
    float* out;            // rows [n][q_row]
    // causal over a cache:
    const _Float16* k;     // K block [max_ctx][row]
    const _Float16* vt;    // V^T block [row][ctx_stride]
    // bidirectional over rows:
    const void* k_rows;    // [n][row]
    const void* v_rows;
    uint32_t n;            // query rows (per image)
    uint32_t batch;        // images (bidirectional), 1 for causal
    uint32_t pos;          // causal: absolute position of query 0
    uint32_t kv_len;       // keys attended at most (causal: pos + n; bidirectional: n)
    uint32_t n_heads, n_kv, hd, group;
    uint32_t q_row;        // n_heads * hd
    uint32_t row;          // n_kv * hd
    uint32_t ctx_stride;
    float scale_log2e;
    float scale;           // the f32 image kernel's own multiply
};

// Causal prefill over the cache (prefill.hip). Its buffer resources span the
// K rows up to kv_len and a head's V^T rows: both must stay below 2^31 bytes.
bool prefill_fits(uint32_t kv_len, uint32_t row, uint32_t hd, uint32_t ctx_stride);
hipError_t launch_prefill(const flash_args& a, uint32_t q_dtype, hipStream_t stream);
hipError_t launch_bidirectional(const flash_args& a, uint32_t in_dtype, hipStream_t stream);

// ---- any-shape fallback -----------------------------------------------------
// A plain f32 kernel for shapes the matrix-core kernels do not take
// (head_dim not a multiple of 8, more than 16 query heads per KV head):
// causal over a cache, one query row per (token, head).
hipError_t launch_generic_causal(const flash_args& a, uint32_t q_dtype, hipStream_t stream);
hipError_t launch_generic_bidirectional(const flash_args& a, uint32_t in_dtype, hipStream_t stream);

// Image-encoder attention on f32 rows in the reference's own f32 arithmetic
// (no binary16 operands); images of up to self_f32_max_keys rows (the
// probabilities of one query row sit in 64 KiB of LDS).
constexpr uint32_t self_f32_max_keys = 16384;
bool self_f32_fits(uint32_t n);
hipError_t launch_self_f32(const flash_args& a, hipStream_t stream);

// ---- RoPE -------------------------------------------------------------------
struct rope_args {
    const float* in;
    float* out;
    const float* freq_factors;  // or nullptr
    uint32_t n, size, hd, pos, mode;
    float theta_scale, freq_scale, ext_factor, attn_factor, corr_low, corr_high;
    uint32_t period;  // rows per image (positions restart), or 0
};
hipError_t launch_rope(const rope_args& a, hipStream_t stream);

// The current device's compute units, asked of the runtime once per device
// (0 if the runtime cannot say).
uint32_t device_cu_count();

// ---- the rest of a decode graph (ops.hip) -----------------------------------
constexpr uint32_t embed_max_tokens = 256;  // tokens per embed launch (kernel argument)
struct embed_tokens {
    uint32_t token[embed_max_tokens];
};
enum elementwise_op : uint32_t {
    elementwise_add = 0,       // a + b
    elementwise_mul = 1,       // a * b
    elementwise_silu_mul = 2,  // silu(a) * b
    elementwise_scale = 3,     // a * scalar
    elementwise_gelu = 4,      // gelu(a), ggml's binary16-rounded tanh form
    elementwise_silu = 5,      // silu(a)
    elementwise_add_bias = 6,  // a + b[e % period]
};
hipError_t launch_embed(const float* table, float* out, const embed_tokens& t, uint32_t n, uint32_t size,
                        hipStream_t stream);
hipError_t launch_softmax(const float* in, float* out, uint32_t n, uint32_t size, hipStream_t stream);
hipError_t launch_rms_norm(const float* in, const float* gamma, float* out, uint32_t n, uint32_t size, float eps,
                           hipStream_t stream);
hipError_t launch_matmul(const float* w, const float* x, const float* bias, float* out, uint32_t n, uint32_t rows,
                         uint32_t cols, hipStream_t stream);
// op_attn_temperature over n rows at positions pos.. in one launch.
hipError_t launch_attn_temperature(const float* in, float* out, uint32_t n, uint32_t size, uint32_t pos,
                                   uint32_t floor_len, float scale, hipStream_t stream);
hipError_t launch_elementwise(const float* a, const float* b, float* out, uint64_t count, uint32_t op, float scalar,
                              uint32_t period,
                              hipStream_t stream);
// Quantized weights (quant.hip), ggml type numbers.
constexpr uint32_t qtype_q4_0 = 2, qtype_q5_0 = 6, qtype_q8_0 = 8, qtype_q4_k = 12, qtype_q6_k = 14;
bool qtype_known(uint32_t t);
uint32_t qtype_block(uint32_t t);                                   // elements per block
uint64_t qtype_row_bytes(uint32_t t, uint32_t cols);                // bytes of one row of cols
uint64_t qtype_act_bytes(uint32_t t, uint32_t n, uint32_t cols);    // quantized activations of n rows
// LDS a quantized matmul may take for its activation rows (an 8-wave
// workgroup), and the activation rows one pass can carry (0: cols too long).
constexpr uint32_t matmul_q_max_lds = 160 * 1024;
// From this many activation rows on, the quantized product runs as a GEMM
// on the int8 matrix cores instead of passes of the GEMV.
constexpr uint32_t matmul_q_gemm_rows = 32;
uint32_t matmul_q_rows_per_pass(uint32_t n, uint32_t cols);
// The same product for many activation rows on the int8 matrix cores
// (quantizes x into act first).
hipError_t launch_gemm_q(uint32_t t, const uint8_t* w, const float* x, uint8_t* act, const float* bias, float* out,
                         uint32_t n, uint32_t rows, uint32_t cols, hipStream_t stream);
hipError_t launch_matmul_q(uint32_t t, const uint8_t* w, const float* x, uint8_t* act, const float* bias, float* out,
                           uint32_t n, uint32_t rows, uint32_t cols, hipStream_t stream);
hipError_t launch_embed_q(uint32_t t, const uint8_t* table, float* out, const embed_tokens& tk, uint32_t n,
                          uint32_t size, hipStream_t stream);
hipError_t launch_layer_norm(const float* in, const float* gamma, const float* beta, float* out, uint32_t n,
                             uint32_t size, float eps, hipStream_t stream);
hipError_t launch_pixel_shuffle(const float* in, float* out, uint32_t n, uint32_t grid_w, uint32_t grid_h, uint32_t s,
                                hipStream_t stream);

}  // namespace syn
