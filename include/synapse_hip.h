/* synapse_hip.h — C ABI of the MI355X (gfx950) KV-cache attention library.
 *
 * The drop-in boundary for synapse's attention path (branes-ai/synapse
 * v0.15.12; S/ = sdk/include/branes/synapse/). A host session calls these
 * from its two attention executor hooks, session::execute(op_attention)
 * (S/graph/session.hpp:348-374) and session::execute(op_self_attention)
 * (S/graph/session.hpp:409-449). Plain pointers, sizes and POD descriptors
 * only; no C++ or framework types cross this interface, and no exception
 * does: every call returns SYN_HIP_OK (0) or an error code.
 *
 * Memory model. The library owns one device arena per session (one
 * hipMalloc at creation). Every tensor, scratch buffer and KV state a call
 * touches is named by its byte offset into that arena, so the library can
 * bounds-check every descriptor on the host before it launches anything.
 * All work of one arena runs in order on the arena's own HIP stream.
 *
 * KV state layout (one layer, all halves = IEEE binary16):
 *   K   at k_offset: [max_ctx][n_kv_heads][head_dim]   row-major, as the
 *       reference stores K (S/kernels/attention.hpp:131-143);
 *   V^T at v_offset: [n_kv_heads][head_dim][ctx_stride] — V is stored
 *       TRANSPOSED (position fastest), ctx_stride = syn_hip_kv_ctx_stride().
 *       The reference keeps V row-major; the transposed layout lets the
 *       P.V matrix-core step read its operand straight from memory.
 * Row tensors are [n][size] floats (or halves where a dtype says so).
 */
#ifndef SYNAPSE_HIP_H
#define SYNAPSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
    SYN_HIP_OK = 0,
    SYN_HIP_EINVAL = -1,       /* bad argument or descriptor (shape, scale, dtype) */
    SYN_HIP_ERANGE = -2,       /* an offset + extent falls outside the arena */
    SYN_HIP_EUNSUPPORTED = -3, /* a shape this build has no kernel for */
    SYN_HIP_ENOMEM = -4,       /* device allocation failed */
    SYN_HIP_ENODEV = -5        /* no gfx950 device, or the HIP runtime failed to start */
    /* positive values: a hipError_t returned by the HIP runtime */
};

/* Element types of row tensors. */
enum { SYN_F32 = 0, SYN_F16 = 1 };

typedef struct syn_arena syn_arena;

/* Text for a status code; never NULL. */
const char* syn_hip_error_string(int status);
/* The last error's detail on this thread ("" if none). */
const char* syn_hip_last_error(void);

/* ---- arena (session construction / destruction) ------------------------
 * Replaces session's arena + states allocation (S/graph/session.hpp:90-95,
 * :193-197) with one device allocation of `bytes` (> 0) bytes, 256-B
 * aligned, on the current HIP device, and one HIP stream. */
int syn_hip_arena_create(size_t bytes, syn_arena** out);
int syn_hip_arena_destroy(syn_arena* arena);
size_t syn_hip_arena_bytes(const syn_arena* arena);
/* The arena's hipStream_t, for callers that record events on it. */
void* syn_hip_arena_stream(syn_arena* arena);

/* Host <-> arena copies, in stream order; download waits for completion.
 * Stand-ins for reading and writing session::tensor() (S/graph/session.hpp:107-110). */
int syn_hip_upload(syn_arena* arena, uint64_t offset, const void* host, size_t bytes);
int syn_hip_download(syn_arena* arena, uint64_t offset, void* host, size_t bytes);
/* Byte fill, as session::reset() zeroes the states (S/graph/session.hpp:127-129). */
int syn_hip_fill(syn_arena* arena, uint64_t offset, int value, size_t bytes);
/* Copy within the arena. */
int syn_hip_copy(syn_arena* arena, uint64_t dst, uint64_t src, size_t bytes);
/* Wait for all work queued on the arena. */
int syn_hip_synchronize(syn_arena* arena);

/* ---- KV state sizing ----------------------------------------------------
 * V^T row length in halves for a cache of max_ctx positions (padded so every
 * row starts 128-B aligned). */
uint32_t syn_hip_kv_ctx_stride(uint32_t max_ctx);
/* Device bytes of one KV state: K block (256-B aligned) then V^T block. The
 * reference's state_desc::bytes (2*2*max_ctx*n_kv*hd, S/graph/graph.hpp:707-716)
 * is the unpadded size of the same data. */
uint64_t syn_hip_kv_state_bytes(uint32_t max_ctx, uint32_t n_kv_heads, uint32_t head_dim);

typedef struct syn_kv_desc {
    uint64_t k_offset;   /* K block */
    uint64_t v_offset;   /* V^T block */
    uint32_t max_ctx;
    uint32_t n_kv_heads;
    uint32_t head_dim;   /* even, <= 256 (S/kernels/attention.hpp:44) */
    uint32_t ctx_stride; /* = syn_hip_kv_ctx_stride(max_ctx) */
} syn_kv_desc;

/* ---- causal attention over a KV cache ----------------------------------- */
typedef struct syn_attn_desc {
    syn_kv_desc cache;
    uint64_t q_offset;       /* n rows of n_heads*head_dim, type q_dtype */
    uint64_t k_offset;       /* n rows of n_kv_heads*head_dim, type kv_dtype: the run's new K */
    uint64_t v_offset;       /* n rows of n_kv_heads*head_dim, type kv_dtype: the run's new V */
    uint64_t out_offset;     /* n rows of n_heads*head_dim f32 */
    uint64_t scratch_offset; /* split-KV partials; see syn_hip_attention_scratch_bytes */
    uint64_t scratch_bytes;
    uint32_t n_heads;        /* a multiple of cache.n_kv_heads */
    uint32_t pos;            /* position of the run's first token */
    uint32_t n;              /* tokens in the run, >= 1; pos + n <= cache.max_ctx */
    float scale;             /* finite, > 0 */
    uint32_t q_dtype;        /* SYN_F32 or SYN_F16 */
    uint32_t kv_dtype;       /* SYN_F32 or SYN_F16 */
} syn_attn_desc;

/* Scratch bytes syn_hip_attention needs for runs of up to max_batch tokens
 * against a cache of max_ctx positions. The GPU counterpart of
 * attention_scratch_floats (S/kernels/attention.hpp:147-161): per-split
 * (max, sum, output) partials instead of a whole score row per head. */
uint64_t syn_hip_attention_scratch_bytes(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                         uint32_t max_ctx, uint32_t max_batch);

/* session::execute(op_attention) (S/graph/session.hpp:348-374): store the
 * run's n K, V rows at positions pos..pos+n-1, rounded to binary16 (kv_append,
 * S/kernels/attention.hpp:165-175), then for every token i and query head h,
 * out_i,h = softmax_t(scale * fp16(q_i,h) . K_t,g) V_t,g over t = 0..pos+i,
 * g = h / (n_heads / n_kv_heads) (attend_group, S/kernels/attention.hpp:185-244;
 * attention, :254-269). Softmax and accumulation in f32, f32 output. */
int syn_hip_attention(syn_arena* arena, const syn_attn_desc* desc);

/* No reference counterpart: syn_hip_attention for callers that cannot let a
 * call allocate or take caller scratch -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation. Same inputs,
 * outputs and results; desc's scratch_offset / scratch_bytes are ignored.
 * The split-KV decode's partials go to a file-scope device array of
 * syn_hip_attention_noalloc_scratch_limit() bytes (4 MiB) that each GPU holds
 * until the process ends; a step whose partials need more returns
 * SYN_HIP_EINVAL without launching. Every call on one GPU shares that array:
 * calls that overlap on one GPU (different streams or arenas) race. Nothing
 * in the array needs to start at zero. */
int syn_hip_attention_noalloc(syn_arena* arena, const syn_attn_desc* desc);
uint64_t syn_hip_attention_noalloc_scratch_limit(void);

/* The attend half only: the cache already holds rows 0..pos+n-1 (desc's
 * k_offset and v_offset are ignored). */
int syn_hip_attend(syn_arena* arena, const syn_attn_desc* desc);

/* kv_append for n rows (S/kernels/attention.hpp:165-175, driven as
 * S/graph/session.hpp:354-356): rows pos0..pos0+n-1 of K and V^T <- fp16 of
 * the n rows at k_rows / v_rows (type kv_dtype). */
int syn_hip_kv_append(syn_arena* arena, const syn_kv_desc* cache, uint64_t k_rows, uint64_t v_rows, uint32_t n,
                      uint32_t pos0, uint32_t kv_dtype);

/* ---- ragged batched decode ----------------------------------------------
 * No reference counterpart: the reference decodes one sequence per session
 * (S/graph/session.hpp:34-43), so a batch is n_seqs separate attention()
 * calls. Here each sequence has its own KV state in the arena and attends
 * its one query row to its cached rows 0..pos (already appended). */
typedef struct syn_seq_desc {
    syn_kv_desc cache;
    uint64_t q_offset;   /* one row of n_heads*head_dim, type q_dtype */
    uint64_t out_offset; /* one row of n_heads*head_dim f32 */
    uint32_t pos;        /* attends rows 0..pos */
    uint32_t reserved;
} syn_seq_desc;

uint64_t syn_hip_attend_batch_scratch_bytes(const syn_seq_desc* seqs, uint32_t n_seqs, uint32_t n_heads);
int syn_hip_attend_batch(syn_arena* arena, const syn_seq_desc* seqs, uint32_t n_seqs, uint32_t n_heads,
                         float scale, uint32_t q_dtype, uint64_t scratch_offset, uint64_t scratch_bytes);

/* ---- bidirectional self-attention (image encoders) ----------------------
 * session::execute(op_self_attention) (S/graph/session.hpp:409-449) with
 * self_attend_head's math (S/kernels/attention.hpp:460-486): for every row i
 * and head h, out_i,h = softmax_j(scale * q_i,h . k_j,h) v_j,h over j = 0..n-1.
 * Rows are grouped into `batch` independent images of n rows each (the
 * reference runs one image per run_rows call, S/models/clip.hpp:405-416).
 * f32 rows of images up to 16384 rows keep the reference's f32 arithmetic
 * (its fma chains, in its order); f16 rows, and longer f32 images, go to the
 * matrix cores as binary16 operands with binary16 probabilities. Softmax
 * and accumulation in f32, f32 output. */
typedef struct syn_self_desc {
    uint64_t q_offset;   /* batch*n rows of n_heads*head_dim, type in_dtype */
    uint64_t k_offset;
    uint64_t v_offset;
    uint64_t out_offset; /* batch*n rows, f32 */
    uint32_t n;          /* rows per image, >= 1 */
    uint32_t batch;      /* images, >= 1 */
    uint32_t n_heads;
    uint32_t head_dim;
    float scale;
    uint32_t in_dtype;   /* SYN_F32 or SYN_F16 */
} syn_self_desc;

int syn_hip_self_attention(syn_arena* arena, const syn_self_desc* desc);

/* ---- RoPE ---------------------------------------------------------------
 * op_rope (S/graph/session.hpp:337-342) with rope's math
 * (S/kernels/attention.hpp:89-129): row i of n rows of `size` floats is
 * rotated by position pos+i, theta_i = pos * theta_scale^i / freq_factor[i]
 * built by repeated f32 multiplication; mode 0 pairs (x[2i], x[2i+1]),
 * mode 1 (neox) pairs (x[i], x[i+hd/2]). YaRN scaling when ext_factor != 0. */
typedef struct syn_rope_desc {
    uint64_t in_offset;           /* n rows of size f32 */
    uint64_t out_offset;          /* n rows of size f32; may not alias in */
    uint64_t freq_factors_offset; /* head_dim/2 f32, or UINT64_MAX for none */
    uint32_t n;
    uint32_t size;                /* a multiple of head_dim */
    uint32_t head_dim;            /* even, <= 256 */
    uint32_t pos;
    float theta_scale;            /* base^(-2/head_dim) */
    uint32_t mode;                /* 0 normal, 1 neox */
    float freq_scale, ext_factor, attn_factor, corr_low, corr_high;
    uint32_t period;              /* rows per image: row i at pos + i % period (images restart); 0: pos + i */
} syn_rope_desc;

int syn_hip_rope(syn_arena* arena, const syn_rope_desc* desc);

/* op_attn_temperature over n rows in one launch (S/graph/session.hpp:343-347):
 * row i times t(pos + i), t(p) = float(log(floor(float(p) / floor_len) + 1)
 * * scale + 1) with the logarithm in double (kernels::attn_temperature,
 * S/kernels/elementwise.hpp:66-72), computed on the device per row. */
typedef struct syn_temperature_desc {
    uint64_t in_offset;  /* n rows of size f32 */
    uint64_t out_offset; /* n rows of size f32; may alias in */
    uint32_t n;
    uint32_t size;
    uint32_t pos;        /* position of row 0 */
    uint32_t floor_len;  /* >= 1 */
    float scale;
    uint32_t reserved;
} syn_temperature_desc;

int syn_hip_attn_temperature(syn_arena* arena, const syn_temperature_desc* desc);

/* One layer's op_rope on q, op_rope on k, op_attn_temperature on q (when
 * temp_floor_len != 0) and op_attention (S/graph/session.hpp:337-374, four
 * ops in the reference) as one call; desc's q_offset and k_offset hold the
 * rows before RoPE, f32. A single-token step that the split-KV decode
 * kernel takes is that one kernel: it rotates q and the new K row in LDS
 * with syn_hip_rope's arithmetic, multiplies q by the temperature, stores
 * the rotated K row into the cache, and writes no rotated rows. Any other
 * run (several tokens, or head sizes that kernel does not take) is two
 * launches: one rotates q (and multiplies it by the temperature) into
 * binary16 rows at q_out_offset, rotates the K rows into the cache and
 * appends the V rows; then the attention kernel reads those q rows. Both
 * are equal, bit for bit, to the separate calls (binary16 is the rounding
 * the attention kernels give f32 q). q_out must not overlap the q, k or v
 * rows. */
typedef struct syn_attn_rope_desc {
    uint64_t q_out_offset;        /* room for n rows of n_heads*head_dim f32, 16-byte aligned; runs write
                                     binary16 rows into its first half, the single-token step nothing */
    uint64_t k_out_offset;        /* unused (rotated K rows go straight to the cache) */
    uint64_t freq_factors_offset; /* head_dim/2 f32 (16-byte aligned), or UINT64_MAX for none */
    float theta_scale;
    uint32_t mode;                /* 0 normal, 1 neox */
    float freq_scale, ext_factor, attn_factor, corr_low, corr_high;
    float temp_scale;             /* op_attn_temperature's scale */
    uint32_t temp_floor_len;      /* its floor length; 0: no temperature */
} syn_attn_rope_desc;

int syn_hip_attention_rope(syn_arena* arena, const syn_attn_desc* desc, const syn_attn_rope_desc* rope);

/* ---- the rest of a Llama-family decode graph ---------------------------------
 * With syn_hip_rope and syn_hip_attention these run a whole layer stack from
 * one arena (all rows f32). */

/* Weight formats, by their GGUF (ggml) type numbers and block layouts. */
enum {
    SYN_TYPE_F32 = 0,
    SYN_TYPE_Q4_0 = 2,  /* 32 per 18-byte block */
    SYN_TYPE_Q5_0 = 6,  /* 32 per 22-byte block */
    SYN_TYPE_Q8_0 = 8,  /* 32 per 34-byte block */
    SYN_TYPE_Q4_K = 12, /* 256 per 144-byte block */
    SYN_TYPE_Q6_K = 14  /* 256 per 210-byte block */
};

/* Embedding rows: out row i = table row tokens[i] (tokens from host memory,
 * each checked < n_table_rows; quantized rows dequantized as ggml does). Replaces session::execute(const op_embed&),
 * S/graph/session.hpp:331-336. */
typedef struct syn_embed_desc {
    uint64_t table_offset; /* n_table_rows rows of size elements of table_type */
    uint64_t out_offset;   /* n rows of size f32 */
    uint32_t n_table_rows;
    uint32_t size;
    uint32_t table_type;   /* SYN_TYPE_F32, or a quantized SYN_TYPE_* (rows dequantized) */
    uint32_t reserved;
} syn_embed_desc;

int syn_hip_embed(syn_arena* arena, const syn_embed_desc* desc, const uint32_t* tokens, uint32_t n);

/* RMSNorm per row: out = (x * (1 / sqrt(mean(x^2) + eps))) * gamma, squares
 * summed in double. Replaces execute(const op_rms_norm&), :324-330
 * (kernels::rms_norm, S/kernels/elementwise.hpp:208-235). */
typedef struct syn_norm_desc {
    uint64_t in_offset;     /* n rows of size f32 */
    uint64_t weight_offset; /* size f32 (gamma) */
    uint64_t out_offset;    /* n rows of size f32; may alias in */
    uint32_t n;
    uint32_t size;
    float eps;              /* >= 0 */
    uint32_t reserved;
} syn_norm_desc;

int syn_hip_rms_norm(syn_arena* arena, const syn_norm_desc* desc);

/* F32 matrix product: out[r][o] = sum_c w[o][c] x[r][c] (+ bias[o]).
 * Replaces execute(const op_matmul&) for F32 weights, :287-302, and
 * execute(const op_add_bias&), :306-312. */
typedef struct syn_matmul_desc {
    uint64_t w_offset;    /* rows x cols f32, row-major (GGUF ne = {cols, rows}) */
    uint64_t x_offset;    /* n rows of cols f32 */
    uint64_t bias_offset; /* rows f32, or UINT64_MAX for none */
    uint64_t out_offset;  /* n rows of rows f32; may not alias x */
    uint32_t n;
    uint32_t rows;
    uint32_t cols;
    uint32_t reserved;
} syn_matmul_desc;

int syn_hip_matmul(syn_arena* arena, const syn_matmul_desc* desc);

/* Product with quantized weights, as ggml computes it: x is quantized to the
 * format ggml pairs with w_type (Q8_0 for Q4_0 / Q5_0 / Q8_0, Q8_K for Q4_K /
 * Q6_K; ggml's reference quantizers, into act), then each weight block meets
 * its activation block in an exact integer dot, combined in float with the
 * block scales. Replaces execute(const op_matmul&) for quantized weights,
 * S/graph/session.hpp:287-302 (S/kernels/gemm.hpp, dot.hpp). */
typedef struct syn_matmul_q_desc {
    uint64_t w_offset;    /* rows rows of cols in w_type blocks */
    uint64_t x_offset;    /* n rows of cols f32 */
    uint64_t act_offset;  /* scratch of syn_hip_matmul_q_act_bytes(w_type, n, cols) */
    uint64_t bias_offset; /* rows f32, or UINT64_MAX for none */
    uint64_t out_offset;  /* n rows of rows f32 */
    uint32_t w_type;      /* SYN_TYPE_Q* */
    uint32_t n;
    uint32_t rows;
    uint32_t cols;        /* a multiple of the format's block */
} syn_matmul_q_desc;

uint64_t syn_hip_matmul_q_act_bytes(uint32_t w_type, uint32_t n, uint32_t cols);
int syn_hip_matmul_q(syn_arena* arena, const syn_matmul_q_desc* desc);

/* Element-wise over count floats (S/kernels/elementwise.hpp:28-81, :115-167):
 * SYN_ADD a + b (op_add, and op_add_rows over whole tables), SYN_MUL a * b
 * (op_mul), SYN_SILU_MUL silu(a) * b (op_silu then op_mul), SYN_SCALE
 * a * scalar (kernels::scale, as op_attn_temperature applies it), SYN_GELU
 * gelu(a) in ggml's binary16-rounded form (op_gelu), SYN_SILU
 * a / (1 + exp(-a)) (op_silu), SYN_ADD_BIAS a + b[e % period], the
 * period floats of b added to every row (op_add_bias,
 * S/graph/session.hpp:306-312). out may alias a or b. */
enum { SYN_ADD = 0, SYN_MUL = 1, SYN_SILU_MUL = 2, SYN_SCALE = 3, SYN_GELU = 4, SYN_SILU = 5, SYN_ADD_BIAS = 6 };

typedef struct syn_elementwise_desc {
    uint64_t a_offset;
    uint64_t b_offset;   /* unused by SYN_SCALE */
    uint64_t out_offset;
    uint64_t count;
    uint32_t op;
    float scalar;
    uint32_t period;     /* SYN_ADD_BIAS: floats of b, dividing count */
    uint32_t reserved;
} syn_elementwise_desc;

int syn_hip_elementwise(syn_arena* arena, const syn_elementwise_desc* desc);

/* Softmax per row: out = exp(x - max) * float(1 / sum), the sum in double.
 * Replaces execute(const op_softmax&), S/graph/session.hpp:319-323
 * (kernels::softmax, S/kernels/elementwise.hpp:169-199). */
typedef struct syn_softmax_desc {
    uint64_t in_offset;  /* n rows of size f32 */
    uint64_t out_offset; /* n rows of size f32; may alias in */
    uint32_t n;
    uint32_t size;       /* >= 1 */
} syn_softmax_desc;

int syn_hip_softmax(syn_arena* arena, const syn_softmax_desc* desc);

/* Layer norm per row: ((x - mean) / sqrt(var + eps)) * gamma + beta, sums in
 * double. Replaces execute(const op_layer_norm&), S/graph/session.hpp:380-392
 * (kernels::layer_norm, S/kernels/elementwise.hpp:240-305). */
typedef struct syn_layer_norm_desc {
    uint64_t in_offset;     /* n rows of size f32 */
    uint64_t weight_offset; /* size f32 (gamma) */
    uint64_t bias_offset;   /* size f32 (beta), or UINT64_MAX for none */
    uint64_t out_offset;    /* n rows of size f32; may alias in */
    uint32_t n;
    uint32_t size;
    float eps;              /* >= 0 */
    uint32_t reserved;
} syn_layer_norm_desc;

int syn_hip_layer_norm(syn_arena* arena, const syn_layer_norm_desc* desc);

/* Pixel shuffle of a grid_w x grid_h grid of patch rows (n f32 each) into
 * (grid_w/s)(grid_h/s) rows of s*s*n. Replaces execute(const
 * op_pixel_shuffle&), :450-453 (kernels::pixel_shuffle,
 * S/kernels/elementwise.hpp:307-333). */
typedef struct syn_pixel_shuffle_desc {
    uint64_t in_offset;
    uint64_t out_offset; /* may not alias in */
    uint32_t n;
    uint32_t grid_w;
    uint32_t grid_h;
    uint32_t scale;      /* >= 1, divides grid_w and grid_h */
} syn_pixel_shuffle_desc;

int syn_hip_pixel_shuffle(syn_arena* arena, const syn_pixel_shuffle_desc* desc);

#ifdef __cplusplus
}
#endif

#endif /* SYNAPSE_HIP_H */
