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
 *
 * Built with -DTQ_DROPIN against the reference's attention_layer.c,
 * context.c and model_ops.h as edited by dropin_patch.sh (the MI355X
 * library's drop-in edits) and linked with libtqattn.so, the same entry
 * points run the reference's own callers on either cache type
 * (tqref_set_kv_type): TQ_KV_Q8 host arrays or the TQ_KV_Q8_DEVICE HBM cache,
 * whose contents are uploaded from and downloaded into the caller's arrays
 * around each call.  tqref_layer_steps runs attention_layer over a run of
 * positions on one cache, and tqref_forward_devmodel_run runs
 * tq_forward_token through the edited context.c's device-model branch.
 */
#include <math.h>
#include <omp.h>
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

/* When set, tqref_layer_batch_run copies the attention rows it computed
 * (the workspace's attn, [n][nq*hd], before the output projection) here. */
static float *g_attn_rows = NULL;
void tqref_capture_attn(float *dst) { g_attn_rows = dst; }

static void make_cache(tq_kv_cache *c, block_q8 *k, block_q8 *v, int max_tokens) {
    memset(c, 0, sizeof *c);
    c->type = TQ_KV_Q8;
    c->k_q8 = k;
    c->v_q8 = v;
    c->max_tokens = max_tokens;
}

#ifdef TQ_DROPIN
static tq_kv_type g_kv_type = TQ_KV_Q8;
static int g_cache_q_heads = 0;

/* Device caches are created for this many query heads instead of the
 * layer's (0: the layer's), so a call whose config does not match its cache
 * can be made on purpose. */
void tqref_set_cache_q_heads(int nq) { g_cache_q_heads = nq; }

/* The cache type the drivers build: TQ_KV_Q8 (the reference's host arrays,
 * the default) or TQ_KV_Q8_DEVICE. */
void tqref_set_kv_type(int type) { g_kv_type = (tq_kv_type)type; }
#endif

/* A cache over the caller's [nkv][max_tokens][nb] arrays: the arrays
 * themselves (TQ_KV_Q8), or a device cache initialised from them. */
static int open_cache(tq_kv_cache *c, const tq_attn_config *cfg, block_q8 *k, block_q8 *v, int max_tokens) {
#ifdef TQ_DROPIN
    if (g_kv_type == TQ_KV_Q8_DEVICE) {
        tq_attn_config dc = *cfg;
        if (g_cache_q_heads > 0) dc.n_q_heads = g_cache_q_heads;
        if (tq_kv_cache_init(c, TQ_KV_Q8_DEVICE, &dc, max_tokens) != 0) return -100;
        if (tq_kv_cache_upload(c, k, v) != 0) {
            tq_kv_cache_free(c);
            return -101;
        }
        return 0;
    }
#endif
    (void)cfg;
    make_cache(c, k, v, max_tokens);
    return 0;
}

/* Leaves the cache's contents in the caller's arrays and releases it. */
static int close_cache(tq_kv_cache *c, block_q8 *k, block_q8 *v) {
#ifdef TQ_DROPIN
    if (c->type == TQ_KV_Q8_DEVICE) {
        const int rc = tq_kv_cache_download(c, k, v);
        tq_kv_cache_free(c);
        return rc != 0 ? -102 : 0;
    }
#endif
    (void)c;
    (void)k;
    (void)v;
    return 0;
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
    int rc = tq_attn_validate(&w, &cfg);
    if (rc != 0) return rc;
    rc = open_cache(&cache, &cfg, k_cache, v_cache, max_tokens);
    if (rc != 0) return rc;
    rc = attention_layer(&w, &cfg, &cache, pos, xn, scores, out);
    const int rc2 = close_cache(&cache, k_cache, v_cache);
    return rc != 0 ? rc : rc2;
}

/* attention_layer for positions pos0 .. pos0+n-1 on one cache (xn and out:
 * [n][hidden]).  Returns the first nonzero code. */
int tqref_layer_steps(int nq, int nkv, int hd, int hidden, float theta, float eps, const block_q8 *wq,
                      const block_q8 *wk, const block_q8 *wv, const block_q8 *wo, const float *qn,
                      const float *kn, block_q8 *k_cache, block_q8 *v_cache, int max_tokens, int pos0, int n,
                      const float *xn, float *scores, float *out) {
    tq_attn_weights w;
    tq_attn_config cfg;
    tq_kv_cache cache;
    make_layer(&w, &cfg, nq, nkv, hd, hidden, theta, eps, wq, wk, wv, wo, qn, kn);
    int rc = tq_attn_validate(&w, &cfg);
    if (rc != 0) return rc;
    rc = open_cache(&cache, &cfg, k_cache, v_cache, max_tokens);
    if (rc != 0) return rc;
    rc = tq_attn_validate_cache(&cache);
    for (int i = 0; rc == 0 && i < n; i++)
        rc = attention_layer(&w, &cfg, &cache, pos0 + i, xn + (size_t)i * hidden, scores, out + (size_t)i * hidden);
    const int rc2 = close_cache(&cache, k_cache, v_cache);
    return rc != 0 ? rc : rc2;
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
    int rc = tq_attn_validate(&w, &cfg);
    if (rc != 0) return rc;
    rc = open_cache(&cache, &cfg, k_cache, v_cache, max_tokens);
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
        if (rc == 0 && g_attn_rows) memcpy(g_attn_rows, ws.attn, (size_t)n * qdim * sizeof(float));
    }
    free(ws.q);
    free(ws.attn);
    free(ws.k);
    free(ws.v);
    free(ws.xq);
    const int rc2 = close_cache(&cache, k_cache, v_cache);
    return rc != 0 ? rc : rc2;
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

/* A batch of independent sequences, each one attention core (RoPE, store_kv
 * of its new token at lens[s]-1, attend over [0, lens[s])) on its own flat
 * cache kc[s] / vc[s] of lens[s] positions.  The reference has no batch API:
 * policy 0 loops over the sequences, each call with attend_q8's own OpenMP
 * over kv heads (the reference's policy); policy 1 runs the sequences in
 * parallel (OpenMP over sequences, each single-threaded).  q [nseq][nq*hd],
 * k, v [nseq][nkv*hd] (k, q pre-RoPE; copied, not modified); out
 * [nseq][nq*hd].  Returns the first nonzero code. */
int tqref_attention_batch(int policy, int nseq, int nq, int nkv, int hd, float theta, const int *lens,
                          block_q8 *const *kc, block_q8 *const *vc, const float *q, const float *k,
                          const float *v, float *out) {
    int rc = 0;
    const int levels = omp_get_max_active_levels();
    if (policy == 1) omp_set_max_active_levels(1);   /* each sequence's attend_q8 on one thread */
#pragma omp parallel for schedule(dynamic, 1) if (policy == 1) reduction(min : rc)
    for (int s = 0; s < nseq; s++) {
        const int L = lens[s];
        float *qs = malloc((size_t)nq * hd * sizeof(float));
        float *ks = malloc((size_t)nkv * hd * sizeof(float));
        float *sc = malloc((size_t)nq * L * sizeof(float));
        int r = -100;
        if (qs && ks && sc) {
            memcpy(qs, q + (size_t)s * nq * hd, (size_t)nq * hd * sizeof(float));
            memcpy(ks, k + (size_t)s * nkv * hd, (size_t)nkv * hd * sizeof(float));
            r = tqref_attention_qkv(nq, nkv, hd, L, theta, kc[s], vc[s], L - 1, qs, ks, v + (size_t)s * nkv * hd, sc,
                                    out + (size_t)s * nq * hd);
        }
        free(qs);
        free(ks);
        free(sc);
        if (r < rc) rc = r;
    }
    omp_set_max_active_levels(levels);
    return rc;
}

/* The attention loop of attention_layer_batch (model/attention_layer.c:
 * 221-236) for tokens pos0 .. pos0+n-1 of one flat cache: for each token,
 * the attention core (RoPE, store_kv, attend over [0, pos]) with attend_q8's
 * OpenMP over kv heads.  q [n][nq*hd], k, v [n][nkv*hd] (post-norm, pre-RoPE;
 * copied, not modified); out [n][nq*hd]. */
int tqref_prefill_core(int nq, int nkv, int hd, int max_tokens, float theta, block_q8 *kc, block_q8 *vc, int pos0,
                       int n, const float *q, const float *k, const float *v, float *out) {
    float *qs = malloc((size_t)nq * hd * sizeof(float));
    float *ks = malloc((size_t)nkv * hd * sizeof(float));
    float *sc = malloc((size_t)nq * max_tokens * sizeof(float));
    int rc = (qs && ks && sc) ? 0 : -100;
    for (int i = 0; rc == 0 && i < n; i++) {
        memcpy(qs, q + (size_t)i * nq * hd, (size_t)nq * hd * sizeof(float));
        memcpy(ks, k + (size_t)i * nkv * hd, (size_t)nkv * hd * sizeof(float));
        rc = tqref_attention_qkv(nq, nkv, hd, max_tokens, theta, kc, vc, pos0 + i, qs, ks, v + (size_t)i * nkv * hd,
                                 sc, out + (size_t)i * nq * hd);
    }
    free(qs);
    free(ks);
    free(sc);
    return rc;
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
#ifdef TQ_DROPIN
    rc = tq_ctx_init(&ctx, &m, g_kv_type, max_tokens);
#else
    rc = tq_ctx_init(&ctx, &m, TQ_KV_Q8, max_tokens);
#endif
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
#ifdef TQ_DROPIN
    rc = tq_ctx_init(&ctx, &m, g_kv_type, max_tokens);
#else
    rc = tq_ctx_init(&ctx, &m, TQ_KV_Q8, max_tokens);
#endif
    if (rc == 0) rc = tq_prefill(&ctx, tokens, n_tok);
    if (rc == 0) {
        memcpy(logits, ctx.logits, (size_t)vocab * sizeof(float));
        const size_t cache = (size_t)nkv * max_tokens * (hd / QK) * sizeof(block_q8);
        for (int l = 0; k_out && v_out && l < n_layers; l++) {
#ifdef TQ_DROPIN
            if (ctx.caches[l].type == TQ_KV_Q8_DEVICE) {
                if (tq_kv_cache_download(&ctx.caches[l], k_out[l], v_out[l]) != 0) rc = -102;
                continue;
            }
#endif
            memcpy(k_out[l], ctx.caches[l].k_q8, cache);
            memcpy(v_out[l], ctx.caches[l].v_q8, cache);
        }
    }
    tq_ctx_free(&ctx);
    free(layers);
    return rc;
}

#ifdef TQ_DROPIN
/* One host matrix (block_q8 or block_q4 rows) on the device in the tiled
 * layout of the MI355X library; NULL on failure. */
static void *upload_matrix(const void *host, int rows, int cols, int q4) {
    const size_t bytes = q4 ? tq_hip_q4_matrix_bytes(rows, cols) : tq_hip_q8_matrix_bytes(rows, cols);
    void *staging = NULL, *dev = NULL;
    int rc = tq_hip_malloc(&staging, bytes);
    if (rc == 0) rc = tq_hip_malloc(&dev, bytes);
    if (rc == 0) rc = tq_hip_memcpy_h2d(staging, host, bytes, NULL);
    if (rc == 0)
        rc = q4 ? tq_hip_q4_pack(dev, (const block_q4 *)staging, rows, cols, NULL)
                : tq_hip_q8_pack(dev, (const block_q8 *)staging, rows, cols, NULL);
    if (rc == 0) rc = tq_hip_device_synchronize();
    tq_hip_free(staging);
    if (rc != 0) {
        tq_hip_free(dev);
        return NULL;
    }
    return dev;
}

static float *upload_floats(const float *host, int n) {
    void *dev = NULL;
    if (tq_hip_malloc(&dev, (size_t)n * sizeof(float)) != 0) return NULL;
    if (tq_hip_memcpy_h2d(dev, host, (size_t)n * sizeof(float), NULL) != 0) {
        tq_hip_free(dev);
        return NULL;
    }
    return (float *)dev;
}

/* The reference's tq_ctx_init + tq_forward_token with ctx.dev pointing at a
 * device model built from the same host weights (tq_dev_ctx_init): the
 * edited tq_forward_token runs each token there and copies the logits into
 * ctx.logits, which land in logits [n_tok][vocab]. */
int tqref_forward_devmodel_run(TQREF_MODEL_ARGS, int max_tokens, int n_tok, const int *tokens, float *logits) {
    tq_model m;
    tq_layer_weights *layers = NULL;
    int rc = build_model(&m, &layers, TQREF_MODEL_PASS);
    if (rc != 0) return rc;
    const int q4 = fmt == 1;
    tq_dev_layer_weights *dl = calloc((size_t)n_layers, sizeof *dl);
    void **owned = calloc((size_t)n_layers * 11 + 2, sizeof(void *));
    int n_owned = 0;
#define KEEP(p) (owned[n_owned++] = (void *)(p), (p))
    if (!dl || !owned) rc = -100;
    for (int l = 0; rc == 0 && l < n_layers; l++) {
        dl[l].input_norm = KEEP(upload_floats(input_norm[l], hidden));
        dl[l].post_norm = KEEP(upload_floats(post_norm[l], hidden));
        dl[l].attn.wq = KEEP(upload_matrix(wq[l], nq * hd, hidden, q4));
        dl[l].attn.wk = KEEP(upload_matrix(wk[l], nkv * hd, hidden, q4));
        dl[l].attn.wv = KEEP(upload_matrix(wv[l], nkv * hd, hidden, q4));
        dl[l].attn.wo = KEEP(upload_matrix(wo[l], hidden, nq * hd, q4));
        dl[l].attn.q_norm = KEEP(upload_floats(qn[l], hd));
        dl[l].attn.k_norm = KEEP(upload_floats(kn[l], hd));
        dl[l].attn.hidden = hidden;
        dl[l].attn.rms_eps = eps;
        dl[l].attn.format = q4 ? TQ_HIP_FORMAT_Q4 : TQ_HIP_FORMAT_Q8;
        dl[l].mlp.wgate = KEEP(upload_matrix(wgate[l], inter, hidden, q4));
        dl[l].mlp.wup = KEEP(upload_matrix(wup[l], inter, hidden, q4));
        dl[l].mlp.wdown = KEEP(upload_matrix(wdown[l], hidden, inter, q4));
        dl[l].mlp.hidden = hidden;
        dl[l].mlp.inter = inter;
        dl[l].mlp.format = dl[l].attn.format;
        for (int i = n_owned - 11; i < n_owned; i++)
            if (!owned[i]) rc = -103;
    }
    tq_dev_model dm;
    memset(&dm, 0, sizeof dm);
    if (rc == 0) {
        dm.attn = m.cfg.attn;
        dm.n_layers = n_layers;
        dm.intermediate_size = inter;
        dm.vocab_size = vocab;
        dm.embed = KEEP(upload_matrix(embed, vocab, hidden, embed_fmt == 1));
        dm.final_norm = KEEP(upload_floats(final_norm, hidden));
        dm.layers = dl;
        dm.embed_format = embed_fmt == 1 ? TQ_HIP_FORMAT_Q4 : TQ_HIP_FORMAT_Q8;
        if (!dm.embed || !dm.final_norm) rc = -103;
    }
#undef KEEP
    tq_dev_ctx dctx;
    memset(&dctx, 0, sizeof dctx);
    tq_ctx ctx;
    memset(&ctx, 0, sizeof ctx);
    if (rc == 0) rc = tq_dev_ctx_init(&dctx, &dm, max_tokens);
    if (rc == 0) rc = tq_ctx_init(&ctx, &m, TQ_KV_Q8, max_tokens);
    if (rc == 0) ctx.dev = &dctx;
    for (int i = 0; rc == 0 && i < n_tok; i++) {
        rc = tq_forward_token(&ctx, tokens[i]);
        if (rc == 0) memcpy(logits + (size_t)i * vocab, ctx.logits, (size_t)vocab * sizeof(float));
    }
    ctx.dev = NULL;
    tq_ctx_free(&ctx);
    tq_dev_ctx_free(&dctx);
    for (int i = 0; owned && i < n_owned; i++) tq_hip_free(owned[i]);
    free(owned);
    free(dl);
    free(layers);
    return rc;
}
#endif

/* Which matmul/attention ISA the build dispatches to ("AVX2" or "scalar"). */
const char *tqref_isa(void) { return kernel_isa_name(); }
