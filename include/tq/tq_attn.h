/* tq_attn.h — C host interface of the Q8 GQA attention path (libtqattn.so, C11).
 *
 * Keeps the reference's kv_cache and attention entry points
 * (model/model_ops.h:95-97,124) and adds one cache type, TQ_KV_Q8_DEVICE, whose
 * K/V live in an HBM-resident paged cache on the current HIP device.  The
 * reference's attention_layer.c reaches it through the two switches on
 * cache->type it already has (store_kv, model/attention_layer.c:75, and
 * attend_all_heads, :154), which call tq_store_kv_device / tq_attend_device.
 * Compute for the device type runs on the GPU only (libtqhip.so); the host
 * cache types keep their reference semantics for allocation and validation,
 * and the compute entry points here reject them (-3).
 *
 * Types: when the reference's model_ops.h has been included first (its guard
 * TAILORQUANT_MODEL_OPS_H is defined) its tq_attn_config / tq_kv_type /
 * tq_kv_cache are used, and they must carry the additions below (the enum
 * value TQ_KV_Q8_DEVICE and the trailing `dev` field).
 *
 * Return codes follow the reference: 0 ok, negative error.  -1 is a bad
 * position / count / shape (checked before anything is written), -2 a cache
 * without storage, -3 a cache type this library does not compute; device
 * failures pass through libtqhip's codes (TQ_HIP_E*, <= -1000 for HIP
 * runtime errors).  Every call is synchronous: outputs are valid on return.
 */
#ifndef TQ_ATTN_H
#define TQ_ATTN_H

#include "block_q8.h"
#include "tq_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef TAILORQUANT_MODEL_OPS_H
/* model/model_ops.h:12-19 */
typedef struct {
    int n_q_heads;
    int n_kv_heads;
    int head_dim;
    int hidden_size;
    float rope_theta;
    float rms_eps;
} tq_attn_config;

/* model/model_ops.h:39, plus the device type. */
typedef enum { TQ_KV_F32, TQ_KV_Q8, TQ_KV_Q8_DEVICE } tq_kv_type;

/* model/model_ops.h:41-48, plus `dev` (NULL unless type is TQ_KV_Q8_DEVICE).
 * The host fields keep their offsets. */
typedef struct {
    tq_kv_type type;
    float *k_f32;
    float *v_f32;
    block_q8 *k_q8;
    block_q8 *v_q8;
    int max_tokens;
    struct tq_hip_kv *dev;
} tq_kv_cache;
#endif

/* model/kv_cache.c:17-48.  TQ_KV_F32 / TQ_KV_Q8: host buffers of the
 * reference's flat layout [n_kv_heads][max_tokens][...].  TQ_KV_Q8_DEVICE: a
 * zero-filled paged HBM cache holding one sequence of max_tokens positions
 * (16-token pages, identity page table) on the current device, which must be a
 * gfx950.  Returns -1 for max_tokens <= 0, a bad type, a shape the device
 * kernels do not cover, no device, or out of memory; every pointer is NULL
 * after a failure. */
int tq_kv_cache_init(tq_kv_cache *cache, tq_kv_type type, const tq_attn_config *cfg,
                     int max_tokens);

/* model/kv_cache.c:5-15.  Frees whatever the cache holds; idempotent. */
void tq_kv_cache_free(tq_kv_cache *cache);

/* model/attention_layer.c:23-36: -1 max_tokens <= 0, -2 missing storage,
 * -3 unknown type. */
int tq_attn_validate_cache(const tq_kv_cache *cache);

/* model/rope.c:4-12 rope_table: cos/sin of pos * theta^(-2i/head_dim) for
 * i < head_dim/2, with the reference's fp32 expression order and libm. */
void tq_attn_rope_table(float *cos_t, float *sin_t, int head_dim, int pos, float theta);

/* store_kv for TQ_KV_Q8_DEVICE (model/attention_layer.c:66-90, Q8 branch):
 * k (post-RoPE) and v, [n_kv_heads * head_dim] each, quantized with
 * quantize_row_q8 into slot pos.  -1 when pos is outside [0, max_tokens). */
int tq_store_kv_device(tq_kv_cache *cache, const tq_attn_config *cfg, int pos, const float *k,
                       const float *v);

/* attend_q8 for TQ_KV_Q8_DEVICE (model/attention_layer.c:125-150): q
 * (post-RoPE, [n_q_heads * head_dim]) against positions [0, pos]; out
 * [n_q_heads * head_dim].  The reference's `scores` scratch is not written. */
int tq_attend_device(const tq_kv_cache *cache, const tq_attn_config *cfg, const float *q, int pos,
                     float *out);

/* The attention core of attention_layer (model/attention_layer.c:172,
 * 186-191) in one device round trip: rope_table(pos, cfg->rope_theta), RoPE
 * on q and k (post-norm, pre-RoPE here), store_kv, attend.  -1 for pos outside
 * [0, max_tokens) before anything is written. */
int tq_attention_core(const tq_attn_config *cfg, tq_kv_cache *cache, int pos, const float *q,
                      const float *k, const float *v, float *out);

/* The per-token loop of attention_layer_batch (model/attention_layer.c:
 * 203-204,220-236) for tokens pos0..pos0+n-1: q [n][n_q_heads*hd], k/v
 * [n][n_kv_heads*hd] (k pre-RoPE), out [n][n_q_heads*hd]; token i sees
 * positions <= pos0+i.  -1 for n <= 0 or a range outside [0, max_tokens). */
int tq_attention_core_batch(const tq_attn_config *cfg, tq_kv_cache *cache, int pos0, int n,
                            const float *q, const float *k, const float *v, float *out);

/* Whole-cache copies between a TQ_KV_Q8_DEVICE cache and host arrays in the
 * reference's TQ_KV_Q8 layout [n_kv_heads][max_tokens][head_dim/32]
 * (model/attention_layer.c:62-64): the host view that tests and benches build
 * by hand (tools/test_model.c:842-850) or read back (:1118-1126).  Either
 * array may be NULL. */
int tq_kv_cache_upload(tq_kv_cache *cache, const block_q8 *k_q8, const block_q8 *v_q8);
int tq_kv_cache_download(const tq_kv_cache *cache, block_q8 *k_q8, block_q8 *v_q8);

#ifdef __cplusplus
}
#endif

#endif /* TQ_ATTN_H */
