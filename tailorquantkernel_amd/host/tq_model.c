/* tq_model.c — tq_ctx_init / tq_forward_token for a Q8 model on the device
 * (model/context.c:6-126), composed from libtqhip's kernels.  See
 * include/tq/tq_model.h.  Built with -ffp-contract=off: the RoPE table is
 * tq_attn_rope_table, the reference's rope_table arithmetic. */
#include "tq/tq_model.h"

#include <stdlib.h>
#include <string.h>

static int check_model(const tq_dev_model *m) {
    if (!m || !m->embed || !m->final_norm || !m->layers) return -1;
    const tq_attn_config *a = &m->attn;
    if (a->hidden_size <= 0 || a->hidden_size % QK != 0 || m->intermediate_size <= 0 ||
        m->intermediate_size % QK != 0)
        return -1;
    if (m->n_layers <= 0 || m->vocab_size <= 0) return -1;
    if (m->embed_format != TQ_HIP_FORMAT_Q8 && m->embed_format != TQ_HIP_FORMAT_Q4) return -1;
    if (a->n_q_heads <= 0 || a->n_kv_heads <= 0 || a->head_dim <= 0 || a->head_dim % 2 != 0) return -1;
    for (int l = 0; l < m->n_layers; l++) {
        const tq_dev_layer_weights *L = &m->layers[l];
        if (!L->input_norm || !L->post_norm || !L->attn.wq || !L->attn.wk || !L->attn.wv || !L->attn.wo ||
            !L->attn.q_norm || !L->attn.k_norm || !L->mlp.wgate || !L->mlp.wup || !L->mlp.wdown)
            return -1;
        if (L->attn.hidden != a->hidden_size || L->mlp.hidden != a->hidden_size ||
            L->mlp.inter != m->intermediate_size)
            return -1;
        if ((L->attn.format != TQ_HIP_FORMAT_Q8 && L->attn.format != TQ_HIP_FORMAT_Q4) ||
            (L->mlp.format != TQ_HIP_FORMAT_Q8 && L->mlp.format != TQ_HIP_FORMAT_Q4))
            return -1;
    }
    return 0;
}

static int dmalloc(void **p, size_t bytes) { return tq_hip_malloc(p, bytes) == TQ_HIP_OK ? 0 : -1; }

/* lm_head (model/embedding.c:35-40) in the embedding's format. */
static int lm_head(const tq_dev_model *m, const float *xn, void *ws, float *logits, void *s) {
    const int hidden = m->attn.hidden_size;
    return m->embed_format == TQ_HIP_FORMAT_Q4
               ? tq_hip_project_output_q4(m->embed, m->vocab_size, hidden, xn, 1, (block_q8 *)ws, logits, s)
               : tq_hip_project_output(m->embed, m->vocab_size, hidden, xn, 1, (block_q8 *)ws, logits, s);
}

int tq_dev_ctx_init(tq_dev_ctx *ctx, const tq_dev_model *m, int max_tokens) {
    memset(ctx, 0, sizeof *ctx);
    if (check_model(m) != 0 || max_tokens <= 0) return -1;
    const tq_attn_config *a = &m->attn;
    const int hidden = a->hidden_size, vocab = m->vocab_size, half = a->head_dim / 2;
    ctx->model = m;
    ctx->max_tokens = max_tokens;
    ctx->caches = calloc((size_t)m->n_layers, sizeof(tq_kv_cache));
    if (!ctx->caches) return -1;
    for (int l = 0; l < m->n_layers; l++) {
        if (tq_kv_cache_init(&ctx->caches[l], TQ_KV_Q8_DEVICE, a, max_tokens) != 0) {
            tq_dev_ctx_free(ctx);
            return -1;
        }
    }
    ctx->stream = tq_hip_kv_stream(ctx->caches[0].dev);
    size_t ws = tq_hip_attention_layer_ws_bytes(ctx->caches[0].dev, &m->layers[0].attn, 1);
    const size_t ws_mlp = tq_hip_mlp_ws_bytes(&m->layers[0].mlp, 1);
    if (ws_mlp > ws) ws = ws_mlp;
    if (ws == 0) {
        tq_dev_ctx_free(ctx);
        return -1;
    }
    ctx->ws_bytes = ws;
    const size_t tb = (size_t)max_tokens * half * sizeof(float);
    if (dmalloc((void **)&ctx->x, (size_t)hidden * 4) || dmalloc((void **)&ctx->xn, (size_t)hidden * 4) ||
        dmalloc((void **)&ctx->y, (size_t)hidden * 4) || dmalloc((void **)&ctx->logits, (size_t)vocab * 4) ||
        dmalloc((void **)&ctx->cos_t, tb) || dmalloc((void **)&ctx->sin_t, tb) ||
        dmalloc((void **)&ctx->positions, (size_t)max_tokens * sizeof(int32_t)) || dmalloc(&ctx->ws, ws) ||
        dmalloc((void **)&ctx->sampled, sizeof(int32_t))) {
        tq_dev_ctx_free(ctx);
        return -1;
    }
    /* RoPE table for every position and the position list, once */
    float *hc = malloc(tb), *hs = malloc(tb);
    int32_t *hp = malloc((size_t)max_tokens * sizeof(int32_t));
    int rc = (hc && hs && hp) ? 0 : -1;
    for (int p = 0; rc == 0 && p < max_tokens; p++) {
        tq_attn_rope_table(hc + (size_t)p * half, hs + (size_t)p * half, a->head_dim, p, a->rope_theta);
        hp[p] = p;
    }
    if (rc == 0 && (tq_hip_memcpy_h2d(ctx->cos_t, hc, tb, NULL) != TQ_HIP_OK ||
                    tq_hip_memcpy_h2d(ctx->sin_t, hs, tb, NULL) != TQ_HIP_OK ||
                    tq_hip_memcpy_h2d(ctx->positions, hp, (size_t)max_tokens * sizeof(int32_t), NULL) !=
                        TQ_HIP_OK))
        rc = -1;
    free(hc);
    free(hs);
    free(hp);
    if (rc != 0) tq_dev_ctx_free(ctx);
    return rc;
}

void tq_dev_ctx_free(tq_dev_ctx *ctx) {
    if (!ctx) return;
    if (ctx->stream) tq_hip_stream_synchronize(ctx->stream);
    if (ctx->caches && ctx->model)
        for (int l = 0; l < ctx->model->n_layers; l++) tq_kv_cache_free(&ctx->caches[l]);
    free(ctx->caches);
    tq_hip_free(ctx->x);
    tq_hip_free(ctx->xn);
    tq_hip_free(ctx->y);
    tq_hip_free(ctx->logits);
    tq_hip_free(ctx->cos_t);
    tq_hip_free(ctx->sin_t);
    tq_hip_free(ctx->positions);
    tq_hip_free(ctx->ws);
    tq_hip_free(ctx->sampled);
    memset(ctx, 0, sizeof *ctx);
}

#define TRY(expr)                      \
    do {                               \
        const int rc_ = (expr);        \
        if (rc_ != TQ_HIP_OK) return rc_; \
    } while (0)

int tq_dev_forward_token(tq_dev_ctx *ctx, int token) {
    if (!ctx || !ctx->model) return -1;
    if (ctx->pos >= ctx->max_tokens) return -1;
    const tq_dev_model *m = ctx->model;
    const tq_attn_config *a = &m->attn;
    const int hidden = a->hidden_size, half = a->head_dim / 2, pos = ctx->pos;
    void *s = ctx->stream;
    if (token < 0 || token >= m->vocab_size) return -1;
    /* :113 embed_lookup */
    TRY(m->embed_format == TQ_HIP_FORMAT_Q4 ? tq_hip_embed_lookup_q4(m->embed, m->vocab_size, hidden, token, ctx->x, s)
                                            : tq_hip_embed_lookup_q8(m->embed, m->vocab_size, hidden, token, ctx->x, s));
    const float *pending = NULL;   /* the previous block's output, added in the next norm */
    for (int l = 0; l < m->n_layers; l++) {
        const tq_dev_layer_weights *L = &m->layers[l];
        /* :100 (x += mlp of the previous layer), :83 rmsnorm(input_norm) */
        TRY(tq_hip_add_rmsnorm(ctx->x, pending, L->input_norm, ctx->xn, 1, hidden, a->rms_eps, s));
        /* :85-86 attention_layer */
        TRY(tq_hip_attention_layer_async(ctx->caches[l].dev, &L->attn, 1, NULL, ctx->positions + pos, pos,
                                         ctx->xn, ctx->cos_t + (size_t)pos * half,
                                         ctx->sin_t + (size_t)pos * half, ctx->y, ctx->ws, ctx->ws_bytes, s));
        /* :88 x += attn, :95 rmsnorm(post_norm) */
        TRY(tq_hip_add_rmsnorm(ctx->x, ctx->y, L->post_norm, ctx->xn, 1, hidden, a->rms_eps, s));
        /* :97-98 mlp_layer */
        TRY(tq_hip_mlp_layer_async(&L->mlp, 1, ctx->xn, ctx->y, ctx->ws, ctx->ws_bytes, s));
        pending = ctx->y;
    }
    /* :100 x += mlp, :121 rmsnorm(final_norm), :122 lm_head */
    TRY(tq_hip_add_rmsnorm(ctx->x, pending, m->final_norm, ctx->xn, 1, hidden, a->rms_eps, s));
    TRY(lm_head(m, ctx->xn, ctx->ws, ctx->logits, s));
    ctx->pos++;
    return 0;
}

int tq_dev_batch_ws_init(tq_dev_batch_ws *ws, const tq_dev_model *m, int cap) {
    memset(ws, 0, sizeof *ws);
    if (check_model(m) != 0 || cap <= 0) return -1;
    const size_t rows = (size_t)cap * m->attn.hidden_size * sizeof(float);
    ws->cap = cap;
    if (dmalloc((void **)&ws->x, rows) || dmalloc((void **)&ws->xn, rows) || dmalloc((void **)&ws->y, rows) ||
        dmalloc((void **)&ws->tokens, (size_t)cap * sizeof(int32_t))) {
        tq_dev_batch_ws_free(ws);
        return -1;
    }
    return 0;
}

void tq_dev_batch_ws_free(tq_dev_batch_ws *ws) {
    if (!ws) return;
    tq_hip_free(ws->x);
    tq_hip_free(ws->xn);
    tq_hip_free(ws->y);
    tq_hip_free(ws->tokens);
    tq_hip_free(ws->ws);
    memset(ws, 0, sizeof *ws);
}

int tq_dev_forward_batch(tq_dev_ctx *ctx, tq_dev_batch_ws *ws, const int *tokens, int n, int want_logits) {
    /* :175-177 */
    if (!ctx || !ctx->model || !ws || !tokens) return -1;
    if (n <= 0 || n > ws->cap) return -1;
    if (ctx->pos + n > ctx->max_tokens) return -1;
    const tq_dev_model *m = ctx->model;
    const tq_attn_config *a = &m->attn;
    const int hidden = a->hidden_size, half = a->head_dim / 2, pos0 = ctx->pos;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->vocab_size) return -1;   /* :185 */
    if (!ws->ws) {
        /* the workspace of the widest call, for cap tokens */
        size_t b = tq_hip_attention_layer_ws_bytes(ctx->caches[0].dev, &m->layers[0].attn, ws->cap);
        const size_t bm = tq_hip_mlp_ws_bytes(&m->layers[0].mlp, ws->cap);
        if (bm > b) b = bm;
        if (b == 0 || dmalloc(&ws->ws, b)) return -1;
        ws->ws_bytes = b;
    }
    void *s = ctx->stream;
    /* the ids go through the stream; waiting once here lets the caller reuse
     * `tokens` on return whatever the copy path */
    TRY(tq_hip_memcpy_h2d(ws->tokens, tokens, (size_t)n * sizeof(int32_t), s));
    TRY(tq_hip_stream_synchronize(s));
    /* :184-187 embed_lookup of every token */
    TRY(m->embed_format == TQ_HIP_FORMAT_Q4
            ? tq_hip_embed_lookup_q4_batch(m->embed, m->vocab_size, hidden, ws->tokens, n, ws->x, s)
            : tq_hip_embed_lookup_q8_batch(m->embed, m->vocab_size, hidden, ws->tokens, n, ws->x, s));
    const float *pending = NULL;   /* the previous block's rows, added in the next norm */
    for (int l = 0; l < m->n_layers; l++) {
        const tq_dev_layer_weights *L = &m->layers[l];
        /* :202 (x += mlp of the previous layer), :192-194 rmsnorm of every row */
        TRY(tq_hip_add_rmsnorm(ws->x, pending, L->input_norm, ws->xn, n, hidden, a->rms_eps, s));
        /* :195-196 attention_layer_batch */
        TRY(tq_hip_attention_layer_batch_async(ctx->caches[l].dev, &L->attn, 0, pos0, n, ws->xn,
                                               ctx->cos_t + (size_t)pos0 * half, ctx->sin_t + (size_t)pos0 * half,
                                               ws->y, ws->ws, ws->ws_bytes, s));
        /* :197 x += attn, :199-201 rmsnorm(post_norm) of every row */
        TRY(tq_hip_add_rmsnorm(ws->x, ws->y, L->post_norm, ws->xn, n, hidden, a->rms_eps, s));
        /* :202 mlp_layer_batch */
        TRY(tq_hip_mlp_layer_async(&L->mlp, n, ws->xn, ws->y, ws->ws, ws->ws_bytes, s));
        pending = ws->y;
    }
    if (want_logits) {
        /* :203 x += mlp (the last row is the one read), :206-208 rmsnorm(final_norm) + lm_head */
        const size_t last = (size_t)(n - 1) * hidden;
        TRY(tq_hip_add_rmsnorm(ws->x + last, pending + last, m->final_norm, ctx->xn, 1, hidden, a->rms_eps, s));
        TRY(lm_head(m, ctx->xn, ctx->ws, ctx->logits, s));
    }
    ctx->pos += n;
    return 0;
}

int tq_dev_prefill(tq_dev_ctx *ctx, const int *tokens, int n) {
    /* :216-217 */
    if (!ctx || !ctx->model || !tokens || n <= 0) return -1;
    if (ctx->pos + n > ctx->max_tokens) return -1;
    const int cap = n < TQ_DEV_PREFILL_BATCH ? n : TQ_DEV_PREFILL_BATCH;
    tq_dev_batch_ws ws;
    if (tq_dev_batch_ws_init(&ws, ctx->model, cap) != 0) return -1;
    int rc = 0;
    for (int i = 0; i < n && rc == 0; i += cap) {
        const int c = n - i < cap ? n - i : cap;
        rc = tq_dev_forward_batch(ctx, &ws, tokens + i, c, i + c == n);
    }
    /* the workspace is freed only after the stream has used it */
    if (ctx->stream) tq_hip_stream_synchronize(ctx->stream);
    tq_dev_batch_ws_free(&ws);
    return rc;
}

int tq_dev_logits(tq_dev_ctx *ctx, float *host) {
    if (!ctx || !ctx->model || !host) return -1;
    TRY(tq_hip_memcpy_d2h(host, ctx->logits, (size_t)ctx->model->vocab_size * sizeof(float), ctx->stream));
    return tq_hip_stream_synchronize(ctx->stream);
}

int tq_dev_sample_greedy(tq_dev_ctx *ctx) {
    if (!ctx || !ctx->model) return -1;
    TRY(tq_hip_sample_greedy(ctx->logits, ctx->model->vocab_size, ctx->sampled, ctx->stream));
    int32_t tok = -1;
    TRY(tq_hip_memcpy_d2h(&tok, ctx->sampled, sizeof tok, ctx->stream));
    TRY(tq_hip_stream_synchronize(ctx->stream));
    return tok;
}
