/* ref_driver.c — flat-argument entry points into the compiled reference.
 *
 * TEST INFRASTRUCTURE ONLY.  Linked into oracle/_ref/libtqref*.so together
 * with the reference's own sources (compiled where they lie under
 * /root/reference by oracle/Makefile).  It lets ctypes drive the reference's
 * public API without mirroring its structs in Python:
 *
 *   tqref_layer_run / tqref_layer_batch_run   call the reference's own
 *       attention_layer / attention_layer_batch (model/attention_layer.c:169-194,
 *       200-243), which run its static store_kv and attend_q8;
 *   tqref_project_qkv / tqref_project_out     reproduce the projections and
 *       per-head norms around the attention core from public functions
 *       (quantize_row_q8, get_matmul, rmsnorm), so the oracle's attention core
 *       can be slotted between them and the whole layer compared;
 *   tqref_attention_qkv                       the attention core alone (RoPE,
 *       store_kv, attend_q8) composed from the reference's public kernels with
 *       attend_q8's OpenMP policy; bench.py times it as the CPU baseline.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "kernel/kernel.h"
#include "model/model_ops.h"

/* Parallelise over kv heads only from this many tokens on, as
 * model/attention_layer.c:8,134 does. */
#define TQREF_PARALLEL_MIN_TOKENS 256

static void bind(tq_matrix *m, const block_q8 *data, int rows, int cols) {
    m->data = data;
    m->format = TQ_FORMAT_Q8;
    m->rows = rows;
    m->cols = cols;
}

static void make_layer(tq_attn_weights *w, tq_attn_config *cfg, int nq, int nkv, int hd,
                       int hidden, float theta, float eps, const block_q8 *wq,
                       const block_q8 *wk, const block_q8 *wv, const block_q8 *wo,
                       const float *qn, const float *kn) {
    memset(w, 0, sizeof *w);
    memset(cfg, 0, sizeof *cfg);
    cfg->n_q_heads = nq;
    cfg->n_kv_heads = nkv;
    cfg->head_dim = hd;
    cfg->hidden_size = hidden;
    cfg->rope_theta = theta;
    cfg->rms_eps = eps;
    bind(&w->wq, wq, nq * hd, hidden);
    bind(&w->wk, wk, nkv * hd, hidden);
    bind(&w->wv, wv, nkv * hd, hidden);
    bind(&w->wo, wo, hidden, nq * hd);
    w->q_norm = qn;
    w->k_norm = kn;
}

static void make_cache(tq_kv_cache *c, block_q8 *k, block_q8 *v, int max_tokens) {
    memset(c, 0, sizeof *c);
    c->type = TQ_KV_Q8;
    c->k_q8 = k;
    c->v_q8 = v;
    c->max_tokens = max_tokens;
}

int tqref_layer_run(int nq, int nkv, int hd, int hidden, float theta, float eps,
                    const block_q8 *wq, const block_q8 *wk, const block_q8 *wv,
                    const block_q8 *wo, const float *qn, const float *kn,
                    block_q8 *k_cache, block_q8 *v_cache, int max_tokens, int pos,
                    const float *xn, float *scores, float *out) {
    tq_attn_weights w;
    tq_attn_config cfg;
    tq_kv_cache cache;
    make_layer(&w, &cfg, nq, nkv, hd, hidden, theta, eps, wq, wk, wv, wo, qn, kn);
    make_cache(&cache, k_cache, v_cache, max_tokens);
    int rc = tq_attn_validate(&w, &cfg);
    if (rc != 0) return rc;
    return attention_layer(&w, &cfg, &cache, pos, xn, scores, out);
}

int tqref_layer_batch_run(int nq, int nkv, int hd, int hidden, float theta, float eps,
                          const block_q8 *wq, const block_q8 *wk, const block_q8 *wv,
                          const block_q8 *wo, const float *qn, const float *kn,
                          block_q8 *k_cache, block_q8 *v_cache, int max_tokens, int pos0,
                          int n, const float *xn, float *scores, float *out) {
    tq_attn_weights w;
    tq_attn_config cfg;
    tq_kv_cache cache;
    make_layer(&w, &cfg, nq, nkv, hd, hidden, theta, eps, wq, wk, wv, wo, qn, kn);
    make_cache(&cache, k_cache, v_cache, max_tokens);
    int rc = tq_attn_validate(&w, &cfg);
    if (rc != 0) return rc;

    /* attention_layer_batch touches only cap, q, k, v, attn and xq of the
     * workspace (model/attention_layer.c:203-241). */
    const int cap = n > 0 ? n : 1;
    const int qdim = nq * hd, kvdim = nkv * hd;
    const int widest = hidden > qdim ? hidden : qdim;
    tq_batch_ws ws;
    memset(&ws, 0, sizeof ws);
    ws.cap = cap;
    ws.q = calloc((size_t)cap * qdim, sizeof(float));
    ws.attn = calloc((size_t)cap * qdim, sizeof(float));
    ws.k = calloc((size_t)cap * kvdim, sizeof(float));
    ws.v = calloc((size_t)cap * kvdim, sizeof(float));
    ws.xq = calloc((size_t)cap * widest / QK, sizeof(block_q8));
    if (!ws.q || !ws.attn || !ws.k || !ws.v || !ws.xq) {
        rc = -100;
    } else {
        rc = attention_layer_batch(&w, &cfg, &cache, pos0, n, xn, scores, out, &ws);
    }
    free(ws.q);
    free(ws.attn);
    free(ws.k);
    free(ws.v);
    free(ws.xq);
    return rc;
}

/* Projections and per-head RMSNorm as attention_layer performs them before
 * RoPE (model/attention_layer.c:38-53,181-184). Outputs post-norm, pre-RoPE
 * q [nq*hd], k [nkv*hd] and raw v [nkv*hd]. */
int tqref_project_qkv(int nq, int nkv, int hd, int hidden, float eps, const block_q8 *wq,
                      const block_q8 *wk, const block_q8 *wv, const float *qn,
                      const float *kn, const float *xn, float *q, float *k, float *v) {
    block_q8 *xq = malloc((size_t)(hidden / QK) * sizeof(block_q8));
    if (!xq) return -100;
    quantize_row_q8(xn, xq, hidden);
    MatmulFn mm = get_matmul(TQ_FORMAT_Q8);
    mm(wq, xq, q, nq * hd, hidden);
    mm(wk, xq, k, nkv * hd, hidden);
    mm(wv, xq, v, nkv * hd, hidden);
    for (int h = 0; h < nq; h++) rmsnorm(q + (size_t)h * hd, qn, q + (size_t)h * hd, hd, eps);
    for (int h = 0; h < nkv; h++) rmsnorm(k + (size_t)h * hd, kn, k + (size_t)h * hd, hd, eps);
    free(xq);
    return 0;
}

/* Output projection (model/attention_layer.c:161-167). */
int tqref_project_out(int nq, int hd, int hidden, const block_q8 *wo, const float *attn,
                      float *out) {
    const int in_dim = nq * hd;
    block_q8 *aq = malloc((size_t)(in_dim / QK) * sizeof(block_q8));
    if (!aq) return -100;
    quantize_row_q8(attn, aq, in_dim);
    get_matmul(TQ_FORMAT_Q8)(wo, aq, out, hidden, in_dim);
    free(aq);
    return 0;
}

/* The attention core on the reference's kernels: rope_table + rope_apply on
 * q and k heads, quantize_row_q8 of K and V into slot h*max_tokens+pos, then
 * per kv head (OpenMP over kv heads from 256 tokens on) quantize the group's q
 * rows, attn_scores_q8, softmax per head, attn_accum_q8.  q and k are
 * post-norm, pre-RoPE and rotated in place.  scores: nq * max_tokens. */
int tqref_attention_qkv(int nq, int nkv, int hd, int max_tokens, float theta,
                        block_q8 *k_cache, block_q8 *v_cache, int pos, float *q, float *k,
                        const float *v, float *scores, float *out) {
    if (pos < 0 || pos >= max_tokens) return -1;
    const int nb = hd / QK;
    const int n = pos + 1;
    const int group = nq / nkv;
    const float scale = 1.0f / sqrtf((float)hd);
    const size_t stride = (size_t)max_tokens;
    float cos_t[hd / 2], sin_t[hd / 2];

    rope_table(cos_t, sin_t, hd, pos, theta);
    for (int h = 0; h < nq; h++) rope_apply(q + (size_t)h * hd, hd, cos_t, sin_t);
    for (int h = 0; h < nkv; h++) rope_apply(k + (size_t)h * hd, hd, cos_t, sin_t);

    for (int h = 0; h < nkv; h++) {
        const size_t at = ((size_t)h * max_tokens + pos) * nb;
        quantize_row_q8(k + (size_t)h * hd, k_cache + at, hd);
        quantize_row_q8(v + (size_t)h * hd, v_cache + at, hd);
    }

#pragma omp parallel for schedule(static) if (n >= TQREF_PARALLEL_MIN_TOKENS)
    for (int kvh = 0; kvh < nkv; kvh++) {
        block_q8 qq[group * nb];
        const size_t first = (size_t)kvh * max_tokens * nb;
        for (int g = 0; g < group; g++)
            quantize_row_q8(q + ((size_t)kvh * group + g) * hd, qq + (size_t)g * nb, hd);
        float *sc = scores + (size_t)kvh * group * stride;
        attn_scores_q8(qq, group, k_cache + first, n, nb, scale, sc, stride);
        for (int g = 0; g < group; g++) softmax(sc + (size_t)g * stride, n);
        attn_accum_q8(sc, stride, group, v_cache + first, n, nb,
                      out + (size_t)kvh * group * hd, (size_t)hd);
    }
    return 0;
}

/* The reference's own mlp_layer (model/mlp.c:3-17) on Q8 matrices. */
int tqref_mlp_run(int hidden, int inter, const block_q8 *wgate, const block_q8 *wup,
                  const block_q8 *wdown, const float *xn, float *out) {
    tq_mlp_weights w;
    bind(&w.wgate, wgate, inter, hidden);
    bind(&w.wup, wup, inter, hidden);
    bind(&w.wdown, wdown, hidden, inter);
    block_q8 *xq = malloc((size_t)hidden / QK * sizeof(block_q8));
    block_q8 *hq = malloc((size_t)inter / QK * sizeof(block_q8));
    float *gate = malloc((size_t)inter * sizeof(float)), *up = malloc((size_t)inter * sizeof(float));
    int rc = (xq && hq && gate && up) ? mlp_layer(&w, xn, xq, gate, up, hq, out) : -100;
    free(xq); free(hq); free(gate); free(up);
    return rc;
}

/* A tq_model over flat per-layer pointer arrays; *layers_out is the layer
 * array to free. */
#define TQREF_MODEL_ARGS                                                                                 \
    int n_layers, int nq, int nkv, int hd, int hidden, int inter, int vocab, float theta, float eps,     \
        const block_q8 *embed, const float *final_norm, const float *const *input_norm,                  \
        const float *const *post_norm, const block_q8 *const *wq, const block_q8 *const *wk,             \
        const block_q8 *const *wv, const block_q8 *const *wo, const float *const *qn,                   \
        const float *const *kn, const block_q8 *const *wgate, const block_q8 *const *wup,                \
        const block_q8 *const *wdown, int fmt, int embed_fmt

static int build_model(tq_model *m, tq_layer_weights **layers_out, TQREF_MODEL_ARGS) {
    tq_layer_weights *layers = calloc((size_t)n_layers, sizeof *layers);
    if (!layers) return -100;
    memset(m, 0, sizeof *m);
    for (int l = 0; l < n_layers; l++) {
        make_layer(&layers[l].attn, &m->cfg.attn, nq, nkv, hd, hidden, theta, eps, wq[l], wk[l], wv[l],
                   wo[l], qn[l], kn[l]);
        layers[l].input_norm = input_norm[l];
        layers[l].post_norm = post_norm[l];
        bind(&layers[l].mlp.wgate, wgate[l], inter, hidden);
        bind(&layers[l].mlp.wup, wup[l], inter, hidden);
        bind(&layers[l].mlp.wdown, wdown[l], hidden, inter);
        /* fmt 1: the arrays hold block_q4 rows (get_matmul(TQ_FORMAT_Q4)) */
        tq_matrix *all[7] = {&layers[l].attn.wq, &layers[l].attn.wk, &layers[l].attn.wv, &layers[l].attn.wo,
                             &layers[l].mlp.wgate, &layers[l].mlp.wup, &layers[l].mlp.wdown};
        for (int i = 0; i < 7; i++) all[i]->format = fmt == 1 ? TQ_FORMAT_Q4 : TQ_FORMAT_Q8;
    }
    m->cfg.n_layers = n_layers;
    m->cfg.intermediate_size = inter;
    m->cfg.vocab_size = vocab;
    bind(&m->w.embed, embed, vocab, hidden);
    m->w.embed.format = embed_fmt == 1 ? TQ_FORMAT_Q4 : TQ_FORMAT_Q8;
    m->w.final_norm = final_norm;
    m->w.layers = layers;
    *layers_out = layers;
    return 0;
}

#define TQREF_MODEL_PASS                                                                                \
    n_layers, nq, nkv, hd, hidden, inter, vocab, theta, eps, embed, final_norm, input_norm, post_norm, wq, \
        wk, wv, wo, qn, kn, wgate, wup, wdown, fmt, embed_fmt

/* The reference's own tq_ctx_init + tq_forward_token (model/context.c:6-52,
 * 104-126) over n_tok tokens on a Q8 model given as flat per-layer pointer
 * arrays, with TQ_KV_Q8 caches; logits [n_tok][vocab].  Returns the first
 * nonzero code, or 0. */
int tqref_forward_run(TQREF_MODEL_ARGS, int max_tokens, int n_tok, const int *tokens, float *logits) {
    tq_model m;
    tq_layer_weights *layers = NULL;
    int rc = build_model(&m, &layers, TQREF_MODEL_PASS);
    if (rc != 0) return rc;
    tq_ctx ctx;
    rc = tq_ctx_init(&ctx, &m, TQ_KV_Q8, max_tokens);
    for (int i = 0; rc == 0 && i < n_tok; i++) {
        rc = tq_forward_token(&ctx, tokens[i]);
        if (rc == 0) memcpy(logits + (size_t)i * vocab, ctx.logits, (size_t)vocab * sizeof(float));
    }
    tq_ctx_free(&ctx);
    free(layers);
    return rc;
}

/* The reference's own tq_prefill (model/context.c:215-229: tq_forward_batch
 * in chunks of TQ_PREFILL_BATCH) over n_tok tokens on fresh TQ_KV_Q8 caches:
 * the last token's logits [vocab], and each layer's K and V caches
 * ([n_kv][max_tokens][hd/32] block_q8) into k_out[l] / v_out[l] when given. */
int tqref_prefill_run(TQREF_MODEL_ARGS, int max_tokens, int n_tok, const int *tokens, float *logits,
                      block_q8 *const *k_out, block_q8 *const *v_out) {
    tq_model m;
    tq_layer_weights *layers = NULL;
    int rc = build_model(&m, &layers, TQREF_MODEL_PASS);
    if (rc != 0) return rc;
    tq_ctx ctx;
    rc = tq_ctx_init(&ctx, &m, TQ_KV_Q8, max_tokens);
    if (rc == 0) rc = tq_prefill(&ctx, tokens, n_tok);
    if (rc == 0) {
        memcpy(logits, ctx.logits, (size_t)vocab * sizeof(float));
        const size_t cache = (size_t)nkv * max_tokens * (hd / QK) * sizeof(block_q8);
        for (int l = 0; k_out && v_out && l < n_layers; l++) {
            memcpy(k_out[l], ctx.caches[l].k_q8, cache);
            memcpy(v_out[l], ctx.caches[l].v_q8, cache);
        }
    }
    tq_ctx_free(&ctx);
    free(layers);
    return rc;
}

/* Which matmul/attention ISA the build dispatches to ("AVX2" or "scalar"). */
const char *tqref_isa(void) { return kernel_isa_name(); }
