/* tq_model.h — a Q8 model's token forward on one MI355X: the device
 * counterpart of tq_ctx_init / tq_forward_token (model/context.c:6-52,
 * 104-126), in libtqattn.so over libtqhip.so.
 *
 * Weights live on the device (tiled Q8 matrices made by tq_hip_q8_pack, fp32
 * norm rows); the context owns one TQ_KV_Q8_DEVICE cache per layer, the
 * activations, a RoPE table for every position (computed on the host with the
 * reference's rope_table arithmetic) and one workspace.  tq_dev_forward_token
 * only enqueues work on the context's stream; tq_dev_logits and
 * tq_dev_sample_greedy wait for it.
 */
#ifndef TQ_MODEL_H
#define TQ_MODEL_H

#include "tq_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* tq_layer_weights (model/model_ops.h:57-62), device pointers. */
typedef struct {
    const float *input_norm;      /* [hidden] */
    tq_hip_attn_weights attn;     /* wq, wk, wv, wo, q_norm, k_norm, hidden, rms_eps */
    const float *post_norm;       /* [hidden] */
    tq_hip_mlp_weights mlp;       /* wgate, wup, wdown, hidden, inter */
} tq_dev_layer_weights;

/* tq_model (model/model_ops.h:50-73), device pointers; `layers` is a host
 * array of n_layers.  embed (vocab x hidden, tiled Q8, or tiled Q4 with
 * embed_format TQ_HIP_FORMAT_Q4) is also the lm_head
 * (model/embedding.c:35-40).  Each layer's attn.format and mlp.format say the
 * format of its matrices, as each tq_matrix carries its own. */
typedef struct {
    tq_attn_config attn;
    int n_layers;
    int intermediate_size;
    int vocab_size;
    const void *embed;
    const float *final_norm;
    const tq_dev_layer_weights *layers;
    int embed_format;             /* TQ_HIP_FORMAT_Q8 (0) or TQ_HIP_FORMAT_Q4 */
} tq_dev_model;

/* tq_ctx (model/model_ops.h:75-95) for the device.  The struct tag lets a
 * host tq_ctx point at one (struct tq_dev_ctx *) before this header. */
typedef struct tq_dev_ctx {
    const tq_dev_model *model;
    tq_kv_cache *caches;          /* n_layers TQ_KV_Q8_DEVICE caches */
    int pos;
    int max_tokens;
    void *stream;                 /* every launch goes here */
    float *x, *xn, *y, *logits;   /* device: residual, normalized, block output, [vocab] */
    float *cos_t, *sin_t;         /* device [max_tokens][head_dim/2] */
    int32_t *positions;           /* device [max_tokens]: 0, 1, 2, ... */
    void *ws;                     /* device workspace of the attention and MLP calls */
    size_t ws_bytes;
    int32_t *sampled;             /* device: tq_dev_sample_greedy's result */
} tq_dev_ctx;

/* model/context.c:6-52: -1 for a NULL model, max_tokens <= 0, hidden or
 * intermediate size not a multiple of 32, n_layers or vocab_size <= 0, a
 * missing weight pointer, or a device or allocation failure (everything
 * allocated so far is freed). */
int tq_dev_ctx_init(tq_dev_ctx *ctx, const tq_dev_model *m, int max_tokens);
/* model/context.c:55-77; idempotent. */
void tq_dev_ctx_free(tq_dev_ctx *ctx);

/* model/context.c:104-126: embed_lookup, per layer rmsnorm -> attention_layer
 * -> residual add -> rmsnorm -> mlp_layer -> residual add, then the final
 * rmsnorm and lm_head into ctx->logits; pos advances.  -1 for pos >=
 * max_tokens or a token outside [0, vocab_size) before any launch. */
int tq_dev_forward_token(tq_dev_ctx *ctx, int token);
/* tq_batch_ws (model/model_ops.h:146-154) for the device: activations of up
 * to cap tokens, their token ids, and the workspace of the batched attention
 * and MLP calls (sized on the first tq_dev_forward_batch, which knows the
 * cache). */
typedef struct {
    int cap;
    float *x, *xn, *y;            /* device [cap][hidden] */
    int32_t *tokens;              /* device [cap] */
    void *ws;
    size_t ws_bytes;
} tq_dev_batch_ws;

/* model/context.c:141-172: -1 for a NULL model or cap <= 0 or an allocation
 * failure (everything allocated so far is freed). */
int tq_dev_batch_ws_init(tq_dev_batch_ws *ws, const tq_dev_model *m, int cap);
/* model/context.c:131-139; idempotent. */
void tq_dev_batch_ws_free(tq_dev_batch_ws *ws);

/* model/context.c:174-213: n tokens at positions pos .. pos+n-1 in one pass:
 * embed_lookup of each, then per layer the rows' rmsnorm ->
 * attention_layer_batch -> residual add -> rmsnorm -> mlp_layer_batch ->
 * residual add; with want_logits the last token's final rmsnorm and lm_head
 * into ctx->logits.  pos advances by n.  -1, before any launch, for n <= 0, n
 * > ws->cap, pos + n > max_tokens or a token outside [0, vocab_size).  The
 * token ids are copied to the device through the stream, which is waited for
 * once after that copy; everything else is only enqueued. */
int tq_dev_forward_batch(tq_dev_ctx *ctx, tq_dev_batch_ws *ws, const int *tokens, int n, int want_logits);

/* Tokens per tq_dev_forward_batch call of tq_dev_prefill.  The reference
 * uses 16 (model/model_ops.h:144), sized for its CPU; the device's GEMM
 * tiles are 128 rows x 128 tokens, and at the 8B shape a 512-token call
 * leaves the q/k/v and output projections half the CUs (128-192 tiles for
 * 256 CUs).  The chunk changes only rounding: every token attends to all
 * tokens before it. */
#define TQ_DEV_PREFILL_BATCH 2048

/* model/context.c:215-229: the whole prompt in chunks of
 * TQ_DEV_PREFILL_BATCH, logits of the last token in ctx->logits.  -1 for n
 * <= 0 or pos + n > max_tokens. */
int tq_dev_prefill(tq_dev_ctx *ctx, const int *tokens, int n);

/* Wait for the stream and copy the last token's logits to host[vocab]. */
int tq_dev_logits(tq_dev_ctx *ctx, float *host);
/* sample_greedy (model/sampler.c:3-13) of the last token's logits on the
 * device; waits and returns the token (or < 0 on failure). */
int tq_dev_sample_greedy(tq_dev_ctx *ctx);

#ifdef __cplusplus
}
#endif

#endif /* TQ_MODEL_H */
