/* tq_attn.c — host side of the Q8 GQA attention path: the kv_cache and
 * attention entry points of the reference's model_ops.h for a device-resident
 * Q8 cache, on top of libtqhip.so.  Every compute call goes to the GPU; there
 * is no host compute path in this file (the host cache types are allocated
 * and validated with the reference's semantics, never computed on).
 *
 * Built with -ffp-contract=off: tq_attn_rope_table must round like the
 * reference's rope_table, which is compiled without FMA contraction.
 */
#include "tq/tq_attn.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define TQ_ATTN_EPOS (-1)   /* bad position, count or shape */
#define TQ_ATTN_ESTORE (-2) /* cache holds no storage */
#define TQ_ATTN_ETYPE (-3)  /* cache type not computed here */

static void clear_cache(tq_kv_cache *cache) {
    cache->k_f32 = NULL;
    cache->v_f32 = NULL;
    cache->k_q8 = NULL;
    cache->v_q8 = NULL;
    cache->dev = NULL;
}

void tq_kv_cache_free(tq_kv_cache *cache) {
    if (!cache) return;
    free(cache->k_f32);
    free(cache->v_f32);
    free(cache->k_q8);
    free(cache->v_q8);
    tq_hip_kv_destroy(cache->dev);
    clear_cache(cache);
    cache->max_tokens = 0;
}

static int device_is_gfx950(void) {
    char arch[64];
    if (tq_hip_device_arch(arch, sizeof arch) != TQ_HIP_OK) return 0;
    return strncmp(arch, "gfx950", 6) == 0;
}

/* One sequence of max_tokens positions: ceil(max_tokens / 16) pages mapped in
 * order, so slot (kvh, pos) of the reference's layout is row pos % 16 of page
 * pos / 16, kv head kvh. */
static int device_cache_init(tq_kv_cache *cache, const tq_attn_config *cfg, int max_tokens) {
    if (!cfg || cfg->n_q_heads <= 0 || cfg->n_kv_heads <= 0 || cfg->head_dim <= 0) return -1;
    if (!device_is_gfx950()) return -1;
    const int pages = (max_tokens + TQ_HIP_PAGE_TOKENS - 1) / TQ_HIP_PAGE_TOKENS;
    tq_hip_kv_desc desc = {cfg->n_q_heads, cfg->n_kv_heads, cfg->head_dim, pages, 1, pages};
    tq_hip_kv *kv = NULL;
    if (tq_hip_kv_create(&kv, &desc) != TQ_HIP_OK) return -1;
    int32_t *table = malloc((size_t)pages * sizeof *table);
    if (!table) {
        tq_hip_kv_destroy(kv);
        return -1;
    }
    for (int p = 0; p < pages; p++) table[p] = p;
    const int rc = tq_hip_kv_set_pages(kv, 0, table, pages);
    free(table);
    if (rc != TQ_HIP_OK) {
        tq_hip_kv_destroy(kv);
        return -1;
    }
    cache->dev = kv;
    return 0;
}

int tq_kv_cache_init(tq_kv_cache *cache, tq_kv_type type, const tq_attn_config *cfg,
                     int max_tokens) {
    cache->type = type;
    cache->max_tokens = max_tokens;
    clear_cache(cache);
    if (max_tokens <= 0) return -1;

    switch (type) {
        case TQ_KV_F32: {
            const size_t n = (size_t)cfg->n_kv_heads * max_tokens * cfg->head_dim;
            cache->k_f32 = malloc(n * sizeof(float));
            cache->v_f32 = malloc(n * sizeof(float));
            if (!cache->k_f32 || !cache->v_f32) break;
            return 0;
        }
        case TQ_KV_Q8: {
            const size_t n = (size_t)cfg->n_kv_heads * max_tokens * (cfg->head_dim / QK);
            cache->k_q8 = malloc(n * sizeof(block_q8));
            cache->v_q8 = malloc(n * sizeof(block_q8));
            if (!cache->k_q8 || !cache->v_q8) break;
            return 0;
        }
        case TQ_KV_Q8_DEVICE:
            if (device_cache_init(cache, cfg, max_tokens) == 0) return 0;
            break;
        default:
            return -1;
    }
    tq_kv_cache_free(cache);
    return -1;
}

int tq_attn_validate_cache(const tq_kv_cache *cache) {
    if (cache->max_tokens <= 0) return -1;
    switch (cache->type) {
        case TQ_KV_F32:
            if (cache->k_f32 == NULL || cache->v_f32 == NULL) return -2;
            break;
        case TQ_KV_Q8:
            if (cache->k_q8 == NULL || cache->v_q8 == NULL) return -2;
            break;
        case TQ_KV_Q8_DEVICE:
            if (cache->dev == NULL) return -2;
            break;
        default:
            return -3;
    }
    return 0;
}

void tq_attn_rope_table(float *cos_t, float *sin_t, int head_dim, int pos, float theta) {
    const float inv_hd = 1.0f / (float)head_dim;
    for (int i = 0; i < head_dim / 2; i++) {
        const float exponent = -2.0f * (float)i * inv_hd;
        const float angle = (float)pos * powf(theta, exponent);
        cos_t[i] = cosf(angle);
        sin_t[i] = sinf(angle);
    }
}

/* Checks shared by the compute entry points, in the reference's order: the
 * position range first (model/attention_layer.c:172,204), then the cache. */
static int check_call(const tq_kv_cache *cache, const tq_attn_config *cfg, int pos0, int n) {
    if (!cache || !cfg) return TQ_ATTN_EPOS;
    if (n <= 0 || pos0 < 0 || pos0 > cache->max_tokens - n) return TQ_ATTN_EPOS;
    if (cache->type != TQ_KV_Q8_DEVICE) return TQ_ATTN_ETYPE;
    if (cache->dev == NULL) return TQ_ATTN_ESTORE;
    tq_hip_kv_desc d;
    const int rc = tq_hip_kv_get_desc(cache->dev, &d);
    if (rc != TQ_HIP_OK) return rc;
    if (d.n_q_heads != cfg->n_q_heads || d.n_kv_heads != cfg->n_kv_heads ||
        d.head_dim != cfg->head_dim)
        return TQ_ATTN_EPOS;
    return 0;
}

int tq_store_kv_device(tq_kv_cache *cache, const tq_attn_config *cfg, int pos, const float *k,
                       const float *v) {
    const int rc = check_call(cache, cfg, pos, 1);
    if (rc != 0) return rc;
    if (!k || !v) return TQ_ATTN_EPOS;
    return tq_hip_kv_append(cache->dev, 0, pos, k, v, NULL, NULL);
}

int tq_attend_device(const tq_kv_cache *cache, const tq_attn_config *cfg, const float *q, int pos,
                     float *out) {
    const int rc = check_call(cache, cfg, pos, 1);
    if (rc != 0) return rc;
    if (!q || !out) return TQ_ATTN_EPOS;
    return tq_hip_attend(cache->dev, 0, pos, q, NULL, NULL, out);
}

int tq_attention_core_batch(const tq_attn_config *cfg, tq_kv_cache *cache, int pos0, int n,
                            const float *q, const float *k, const float *v, float *out) {
    int rc = check_call(cache, cfg, pos0, n);
    if (rc != 0) return rc;
    if (!q || !k || !v || !out) return TQ_ATTN_EPOS;
    const int half = cfg->head_dim / 2;
    float *tab = malloc(2 * (size_t)n * half * sizeof *tab);
    if (!tab) return TQ_HIP_ENOMEM;
    float *cos_t = tab, *sin_t = tab + (size_t)n * half;
    for (int i = 0; i < n; i++)
        tq_attn_rope_table(cos_t + (size_t)i * half, sin_t + (size_t)i * half, cfg->head_dim,
                           pos0 + i, cfg->rope_theta);
    rc = tq_hip_prefill(cache->dev, 0, pos0, n, q, k, v, cos_t, sin_t, out);
    free(tab);
    return rc;
}

int tq_attention_core(const tq_attn_config *cfg, tq_kv_cache *cache, int pos, const float *q,
                      const float *k, const float *v, float *out) {
    return tq_attention_core_batch(cfg, cache, pos, 1, q, k, v, out);
}

static int device_rows(const tq_kv_cache *cache, block_q8 *k_q8, block_q8 *v_q8, int to_device) {
    if (!cache) return TQ_ATTN_EPOS;
    if (cache->type != TQ_KV_Q8_DEVICE) return TQ_ATTN_ETYPE;
    if (cache->dev == NULL) return TQ_ATTN_ESTORE;
    if (cache->max_tokens <= 0) return TQ_ATTN_EPOS;
    return to_device ? tq_hip_kv_write(cache->dev, 0, 0, cache->max_tokens, k_q8, v_q8)
                     : tq_hip_kv_read(cache->dev, 0, 0, cache->max_tokens, k_q8, v_q8);
}

int tq_kv_cache_upload(tq_kv_cache *cache, const block_q8 *k_q8, const block_q8 *v_q8) {
    return device_rows(cache, (block_q8 *)k_q8, (block_q8 *)v_q8, 1);
}

int tq_kv_cache_download(const tq_kv_cache *cache, block_q8 *k_q8, block_q8 *v_q8) {
    return device_rows(cache, k_q8, v_q8, 0);
}
