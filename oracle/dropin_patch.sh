#!/bin/sh
# dropin_patch.sh REF OUT — TEST INFRASTRUCTURE ONLY.
#
# Writes edited copies of three of the reference's files under OUT (never
# into the repository's history: OUT is under oracle/_ref/), applying the
# reference-side edits that make the MI355X library a drop-in for the Q8
# attention path:
#
#   model/model_ops.h        tq_kv_type gains TQ_KV_Q8_DEVICE (:39); tq_kv_cache
#                            gains `struct tq_hip_kv *dev` after its host fields
#                            (:47); tq_ctx gains `struct tq_dev_ctx *dev` (:95);
#                            the library's header tq/tq_model.h is included last.
#   model/attention_layer.c  tq_attn_validate_cache accepts the device type
#                            (:29-31); store_kv (:68) and attend_all_heads (:154)
#                            route the device type to tq_store_kv_device /
#                            tq_attend_device and abort on a device error (they
#                            return void); attention_layer (:186) and
#                            attention_layer_batch (:218) take the fused device
#                            calls, tq_attention_core / tq_attention_core_batch,
#                            and return their codes — unless built with
#                            -DTQ_DROPIN_ROUTE_ONLY, which leaves only the two
#                            routing points.
#   model/context.c          tq_forward_token (:104-107) runs the whole token on
#                            the device model when ctx->dev is set.
#
# Every edit is anchored on an exact line of the reference; the script fails
# if an anchor is missing, so a changed reference cannot build silently
# without the edit.
set -eu
REF=$1
OUT=$2
mkdir -p "$OUT/model"

need() {   # need FILE COUNT PATTERN: the edited file holds PATTERN exactly COUNT times
    n=$(grep -c -F -- "$3" "$1" || true)
    if [ "$n" != "$2" ]; then
        echo "dropin_patch: $1: expected $2 x '$3', found $n" >&2
        exit 1
    fi
}

# ---- model/model_ops.h ----
sed -e 's/^typedef enum { TQ_KV_F32, TQ_KV_Q8 } tq_kv_type;$/typedef enum { TQ_KV_F32, TQ_KV_Q8, TQ_KV_Q8_DEVICE } tq_kv_type;/' \
    -e '/^    int max_tokens;$/{N;s/^    int max_tokens;\n} tq_kv_cache;$/    int max_tokens;\n    struct tq_hip_kv *dev;   \/* TQ_KV_Q8_DEVICE: paged HBM cache, else NULL *\/\n} tq_kv_cache;/}' \
    -e 's/^} tq_ctx;$/    struct tq_dev_ctx *dev;      \/* the device model, when the token runs there *\/\n} tq_ctx;/' \
    -e '$ s/^#endif$/#include "tq\/tq_model.h"\n#endif/' \
    "$REF/model/model_ops.h" > "$OUT/model/model_ops.h"
H="$OUT/model/model_ops.h"
need "$H" 1 "TQ_KV_Q8_DEVICE } tq_kv_type;"
need "$H" 1 "struct tq_hip_kv *dev;"
need "$H" 1 "struct tq_dev_ctx *dev;"
need "$H" 1 '#include "tq/tq_model.h"'

# ---- model/attention_layer.c ----
sed -e 's/^#include <string.h>$/&\n#include <stdlib.h>/' \
    -e '/^            if (cache->k_q8 == NULL || cache->v_q8 == NULL) return -2;$/{n;s/^            break;$/&\n        case TQ_KV_Q8_DEVICE:\n            if (cache->dev == NULL) return -2;\n            break;/}' \
    -e 's/^    assert(pos >= 0 \&\& pos < cache->max_tokens);$/&\n    if (cache->type == TQ_KV_Q8_DEVICE) {   \/* k is post-RoPE here *\/\n        if (tq_store_kv_device(cache, cfg, pos, k, v) != 0) abort();\n        return;\n    }/' \
    -e '/^static void attend_all_heads(/{n;s/$/\n    if (cache->type == TQ_KV_Q8_DEVICE) {   \/* scores are not written *\/\n        if (tq_attend_device(cache, cfg, q, pos, out) != 0) abort();\n        return;\n    }/}' \
    -e 's/^    rope_table(rope_cos, rope_sin, hd, pos, cfg->rope_theta);$/#ifndef TQ_DROPIN_ROUTE_ONLY\n    if (cache->type == TQ_KV_Q8_DEVICE) {   \/* q, k post-norm, pre-RoPE: one device round trip *\/\n        int rc_dev = tq_attention_core(cfg, cache, pos, q, k, v, attn);\n        if (rc_dev != 0) return rc_dev;\n        project_output(w, cfg, attn, out);\n        return 0;\n    }\n#endif\n&/' \
    -e 's/^    get_matmul_batch(w->wv.format)(w->wv.data, ws->xq, ws->v, w->wv.rows, w->wv.cols, n);$/&\n#ifndef TQ_DROPIN_ROUTE_ONLY\n    if (cache->type == TQ_KV_Q8_DEVICE) {   \/* the per-token loop as one device call *\/\n        for (int i = 0; i < n; i++) {\n            norm_heads(ws->q + (size_t)i * q_dim, cfg->n_q_heads,  hd, w->q_norm, cfg->rms_eps);\n            norm_heads(ws->k + (size_t)i * kv_dim, cfg->n_kv_heads, hd, w->k_norm, cfg->rms_eps);\n        }\n        int rc_dev = tq_attention_core_batch(cfg, cache, pos0, n, ws->q, ws->k, ws->v, ws->attn);\n        if (rc_dev != 0) return rc_dev;\n        for (int i = 0; i < n; i++)\n            quantize_row_q8(ws->attn + (size_t)i * q_dim, ws->xq + (size_t)i * nbq, q_dim);\n        get_matmul_batch(w->wo.format)(w->wo.data, ws->xq, out, w->wo.rows, w->wo.cols, n);\n        return 0;\n    }\n#endif/' \
    "$REF/model/attention_layer.c" > "$OUT/model/attention_layer.c"
A="$OUT/model/attention_layer.c"
need "$A" 1 "#include <stdlib.h>"
need "$A" 1 "case TQ_KV_Q8_DEVICE:"
need "$A" 1 "tq_store_kv_device(cache, cfg, pos, k, v)"
need "$A" 1 "tq_attend_device(cache, cfg, q, pos, out)"
need "$A" 1 "tq_attention_core(cfg, cache, pos, q, k, v, attn)"
need "$A" 1 "tq_attention_core_batch(cfg, cache, pos0, n, ws->q, ws->k, ws->v, ws->attn)"

# ---- model/context.c ----
sed -e 's/^    if (ctx->pos >= ctx->max_tokens) return -1;$/&\n    if (ctx->dev != NULL) {   \/* the whole token on the device model built beside this one *\/\n        if (token < 0 || token >= ctx->model->cfg.vocab_size) return -1;\n        if (tq_dev_forward_token(ctx->dev, token) != 0) return -1;\n        if (tq_dev_logits(ctx->dev, ctx->logits) != 0) return -1;\n        ctx->pos++;\n        return 0;\n    }/' \
    "$REF/model/context.c" > "$OUT/model/context.c"
need "$OUT/model/context.c" 1 "tq_dev_forward_token(ctx->dev, token)"
