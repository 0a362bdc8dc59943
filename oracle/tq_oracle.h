/* tq_oracle.h — CPU restatement of the reference's scalar Q8 attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product (libtqhip.so, libtqattn.so) never
 * links, loads or calls it.
 *
 * Every function restates one reference function (cited file:line) from its
 * arithmetic, in the same floating-point operation order, and is compiled
 * without FMA contraction (-ffp-contract=off), as the reference's scalar
 * sources are (no -mfma for them).  Cache layout is the reference's flat one:
 * [n_kv_heads][max_tokens][head_dim/32] block_q8 for K and for V, with
 * slot(h, pos) = h*max_tokens + pos (model/attention_layer.c:62-64).
 */
#ifndef TQ_ORACLE_H
#define TQ_ORACLE_H

#include <stddef.h>
#include "../include/tq/block_q8.h"

#ifdef __cplusplus
extern "C" {
#endif

/* kernel/quant_x.c:12-33 */
void oracle_quantize_row_q8(const float *x, block_q8 *out, int n);

/* model/rope.c:4-12 and :14-22 */
void oracle_rope_table(float *cos_t, float *sin_t, int head_dim, int pos, float theta);
void oracle_rope_apply(float *x, int head_dim, const float *cos_t, const float *sin_t);

/* model/softmax.c:4-23 */
void oracle_softmax(float *x, int n);

/* model/attn_q8.c:17-34 */
void oracle_attn_scores_q8(const block_q8 *q, int g, const block_q8 *k, int n, int nb,
                           float scale, float *scores, size_t stride);

/* model/attn_q8.c:36-54 */
void oracle_attn_accum_q8(const float *w, size_t w_stride, int g, const block_q8 *v,
                          int n, int nb, float *out, size_t out_stride);

/* model/attn_q8.c:78-90 */
void oracle_attention_head_q8(const float *q, block_q8 *q_q8, const block_q8 *k_cache,
                              const block_q8 *v_cache, int n, int head_dim,
                              float *scores, float *out);

/* model/attention_layer.c:66-90, TQ_KV_Q8 branch: k is post-RoPE. */
int oracle_store_kv_q8(block_q8 *k_cache, block_q8 *v_cache, int n_kv_heads, int head_dim,
                       int max_tokens, int pos, const float *k, const float *v);

/* model/attention_layer.c:125-150 (attend_q8), serial over kv heads.
 * scores: n_q_heads * max_tokens floats, as the reference's ctx->scores. */
int oracle_attend_q8(const block_q8 *k_cache, const block_q8 *v_cache, int n_q_heads,
                     int n_kv_heads, int head_dim, int max_tokens, const float *q, int pos,
                     float *scores, float *out);

/* The attention core of attention_layer (model/attention_layer.c:172,186-191):
 * pos range check, rope_table(pos), RoPE on q and k, store_kv, attend_q8.
 * q and k are post-norm and pre-RoPE; q is rotated in place.  Returns -1 for a
 * bad pos before any write, else 0. */
int oracle_attention_qkv(block_q8 *k_cache, block_q8 *v_cache, int n_q_heads, int n_kv_heads,
                         int head_dim, int max_tokens, float rope_theta, int pos,
                         float *q, float *k, const float *v, float *scores, float *out);

/* The attention loop of attention_layer_batch (model/attention_layer.c:203-204,
 * 221-236): n tokens at pos0..pos0+n-1, token-major q/k/v/out. */
int oracle_prefill_qkv(block_q8 *k_cache, block_q8 *v_cache, int n_q_heads, int n_kv_heads,
                       int head_dim, int max_tokens, float rope_theta, int pos0, int n,
                       float *q, float *k, const float *v, float *scores, float *out);

/* model/rmsnorm.c:4-19 (in place allowed). */
void oracle_rmsnorm(const float *x, const float *weight, float *out, int n, float eps);

/* model/attention_layer.c:169-194: the whole attention layer for one token
 * (projections, q/k RMSNorm, RoPE, store_kv, attend_q8, output projection). */
int oracle_attention_layer(const block_q8 *wq, const block_q8 *wk, const block_q8 *wv,
                           const block_q8 *wo, const float *q_norm, const float *k_norm,
                           int n_q_heads, int n_kv_heads, int head_dim, int hidden,
                           float rope_theta, float rms_eps, block_q8 *k_cache,
                           block_q8 *v_cache, int max_tokens, int pos, const float *xn,
                           float *scores, float *out);

/* model/silu.c:6-18 */
void oracle_silu_mul(const float *gate, const float *up, float *out, int n);

/* model/mlp.c:3-17 */
int oracle_mlp_layer(const block_q8 *wgate, const block_q8 *wup, const block_q8 *wdown, int hidden,
                     int inter, const float *xn, float *out);

/* model/embedding.c:4-17 (Q8) */
int oracle_embed_lookup_q8(const block_q8 *embed, int rows, int cols, int token, float *out);

/* model/sampler.c:3-13 */
int oracle_sample_greedy(const float *logits, int n);

/* A Q8 or Q4 model as tq_model holds it (model/model_ops.h:50-73), per-layer
 * pointers in arrays of n_layers; embed is vocab x hidden (tied lm_head). */
struct oracle_model {
    int n_layers, n_q_heads, n_kv_heads, head_dim, hidden, inter, vocab;
    float rope_theta, rms_eps;
    const void *embed;               /* block_q8 or block_q4 rows (embed_format) */
    const float *final_norm;
    const float *const *input_norm;
    const float *const *post_norm;
    const void *const *wq, *const *wk, *const *wv, *const *wo;   /* block_q8 or block_q4 (format) */
    const float *const *q_norm, *const *k_norm;
    const void *const *wgate, *const *wup, *const *wdown;
    int format;                      /* the layers' matrices: 0 Q8, 1 Q4 */
    int embed_format;                /* the embedding / lm_head: 0 Q8, 1 Q4 */
};

/* model/context.c:104-126 (tq_forward_token) on flat Q8 caches. */
int oracle_forward_token(const struct oracle_model *m, block_q8 *const *k_caches,
                         block_q8 *const *v_caches, int max_tokens, int pos, int token, float *logits);

/* packer/packer.c:4-31 (pack_row_q8 over every row): weights -> block_q8. */
void oracle_pack_matrix_q8(const float *W, int rows, int cols, block_q8 *out);

/* packer/packer.c:40-52 (pack_row_q4 over every row, block_scale with qmax 7,
 * :11-19): weights -> block_q4. */
void oracle_pack_matrix_q4(const float *W, int rows, int cols, block_q4 *out);

/* packer/packer.c:54-61 (unpack_row_q4 over every row). */
void oracle_unpack_matrix_q4(const block_q4 *in, int rows, int cols, float *out);

/* kernel/q4_scalar.c:3-24 (and :27-32 for n_tok rows of input). */
void oracle_matmul_q4_batch(const block_q4 *W, const block_q8 *xq, float *y, int rows, int cols, int n_tok);

/* model/embedding.c:20-27 (Q4) */
int oracle_embed_lookup_q4(const block_q4 *embed, int rows, int cols, int token, float *out);

/* kernel/q8_scalar.c:3-22 */
void oracle_matmul_q8(const block_q8 *W, const block_q8 *xq, float *y, int rows, int cols);

/* kernel/q8_scalar.c:25-30 */
void oracle_matmul_q8_batch(const block_q8 *W, const block_q8 *xq, float *y, int rows, int cols,
                            int n_tok);

/* quantize_row_q8 per input row, then the Q8 matmul: project_qkv for one
 * matrix and project_output (model/attention_layer.c:38-46,161-167). */
void oracle_project_q8(const block_q8 *W, int rows, int cols, const float *x, int n_tok,
                       float *y);

#ifdef __cplusplus
}
#endif

#endif /* TQ_ORACLE_H */
