/* oracle.h — CPU restatement of synapse's KV-cache attention semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. Nothing in synapse_amd/ links, loads or calls it.
 *
 * Every function restates one function of branes-ai/synapse v0.15.12
 * (sdk/include/branes/synapse/...), cited at its definition in oracle.cpp.
 * Built with -ffp-contract=off, as the reference builds
 * (cmake/numerics.cmake:13-15), so every float operation rounds where the
 * reference's does.
 *
 * KV cache layout here is the REFERENCE layout (kernels/attention.hpp:131-143):
 * K[max_ctx][n_kv*hd] halves, then V[max_ctx][n_kv*hd] halves, V not
 * transposed. Row tensors are float [n][size].
 */
#ifndef SYNAPSE_ORACLE_H
#define SYNAPSE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* numeric/half.hpp:18-41 and :46-82 */
float orc_fp16_to_float(uint16_t h);
uint16_t orc_float_to_fp16(float f);
void orc_fp16_to_float_n(const uint16_t* h, float* out, size_t n);
void orc_float_to_fp16_n(const float* f, uint16_t* out, size_t n);

/* kernels/attention.hpp:47-49, :71-81, :89-129.
 * scaling: NULL, or 5 floats {freq_scale, ext_factor, attn_factor, corr_low, corr_high}.
 * freq_factors: NULL or head_dim/2 floats. mode: 0 normal, 1 neox. */
float orc_rope_theta_scale(float base, size_t head_dim);
void orc_rope_yarn_corr_dims(size_t n_dims, size_t n_ctx_orig, float base, float beta_fast, float beta_slow,
                             float out[2]);
void orc_rope(const float* x, float* out, size_t size, size_t head_dim, uint32_t pos, float theta_scale,
              const float* freq_factors, int mode, const float* scaling);

/* kernels/elementwise.hpp:174-201 */
void orc_softmax(const float* x, float* out, size_t n);

/* kernels/attention.hpp:147-161 */
size_t orc_attention_group_floats(size_t n_heads, size_t n_kv, size_t hd, size_t max_ctx);
size_t orc_attention_scratch_floats(size_t n_heads, size_t n_kv, size_t hd, size_t max_ctx);

/* kernels/attention.hpp:165-175: row pos of K, V <- fp16(k), fp16(v). */
void orc_kv_append(const float* k, const float* v, uint16_t* k_cache, uint16_t* v_cache, size_t max_ctx,
                   size_t n_kv, size_t hd, uint32_t pos);

/* kernels/attention.hpp:185-244: the query heads of KV group g over rows 0..pos. */
void orc_attend_group(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, size_t max_ctx,
                      size_t n_kv, size_t hd, uint32_t pos, size_t n_heads, float scale, float* out,
                      float* scores, size_t g);

/* kernels/attention.hpp:254-269: kv_append, then attend_group for every group. */
void orc_attention(const float* q, const float* k, const float* v, uint16_t* k_cache, uint16_t* v_cache,
                   size_t max_ctx, size_t n_kv, size_t hd, uint32_t pos, size_t n_heads, float scale, float* out,
                   float* scores);

/* graph/session.hpp:348-374: append all n tokens' K, V at positions pos..pos+n-1,
 * then for each KV group and each token i, attend_group at position pos+i.
 * threads: >= 1; groups are split over std::threads the way session::parallel
 * splits them (results do not depend on it). scores: n_kv slots of
 * orc_attention_group_floats. */
void orc_attention_rows(const float* q, const float* k, const float* v, size_t n, uint32_t pos,
                        uint16_t* k_cache, uint16_t* v_cache, size_t max_ctx, size_t n_kv, size_t hd,
                        size_t n_heads, float scale, float* out, float* scores, unsigned threads);

/* Only the attend half of orc_attention_rows (the cache already holds rows
 * 0..pos+n-1): what the CPU baseline times against the GPU attention kernel. */
void orc_attend_rows(const float* q, size_t n, uint32_t pos, const uint16_t* k_cache, const uint16_t* v_cache,
                     size_t max_ctx, size_t n_kv, size_t hd, size_t n_heads, float scale, float* out,
                     float* scores, unsigned threads);

/* kernels/attention.hpp:273-315, :324-486 and graph/session.hpp:409-449:
 * bidirectional self-attention of n rows, float operands, every score one
 * fma chain over d then times scale, softmax, every output one fma chain
 * over j. q, k, v, out: [n][row_size] with n_heads heads of row_size/n_heads. */
void orc_self_attention(const float* q, const float* k, const float* v, size_t n, size_t row_size,
                        size_t n_heads, float scale, float* out, unsigned threads);

#ifdef __cplusplus
}
#endif

#endif
