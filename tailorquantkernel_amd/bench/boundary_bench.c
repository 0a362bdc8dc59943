/* boundary_bench.c — the synchronous drop-in boundary timed from C.
 *
 * attention_layer (model/attention_layer.c:169-194) in the drop-in mode calls
 * tq_attention_core once per layer per token: host q, k, v in, host
 * attention rows out.  This program times that call on a device cache at the
 * Llama-3-8B shape (32 q / 8 kv heads, head_dim 128, RoPE theta 5e5) at
 * position `pos` of a cache holding `pos` earlier tokens, and, beside it, the
 * pieces it is made of: the host RoPE table, the append (store_kv) alone and
 * the attend alone, each through the same synchronous entry points.
 *
 *   boundary_bench [pos] [calls]      (defaults 4095, 2000)
 *
 * Prints one JSON line; every figure is microseconds per call, the median of
 * 20 batches of calls / 20.
 */
#define _POSIX_C_SOURCE 199309L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "tq/tq_attn.h"

static double now_us(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e6 + t.tv_nsec * 1e-3;
}

static int cmp_double(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

#define BATCHES 20

typedef int (*call_fn)(void *ctx);

/* Median over BATCHES batches of calls/BATCHES calls each, after 50 warm-up calls. */
static double time_calls(call_fn fn, void *ctx, int calls, int *rc_out) {
    double per[BATCHES];
    int rc = 0;
    for (int i = 0; i < 50 && rc == 0; i++) rc = fn(ctx);
    const int each = calls / BATCHES > 0 ? calls / BATCHES : 1;
    for (int b = 0; b < BATCHES && rc == 0; b++) {
        const double t0 = now_us();
        for (int i = 0; i < each && rc == 0; i++) rc = fn(ctx);
        per[b] = (now_us() - t0) / each;
    }
    *rc_out = rc;
    if (rc != 0) return -1.0;
    qsort(per, BATCHES, sizeof per[0], cmp_double);
    return per[BATCHES / 2];
}

typedef struct {
    tq_attn_config cfg;
    tq_kv_cache cache;
    int pos;
    float *q, *k, *v, *out, *cos_t, *sin_t;
} bench_ctx;

static int call_core(void *p) {
    bench_ctx *c = p;
    return tq_attention_core(&c->cfg, &c->cache, c->pos, c->q, c->k, c->v, c->out);
}
static int call_rope(void *p) {
    bench_ctx *c = p;
    tq_attn_rope_table(c->cos_t, c->sin_t, c->cfg.head_dim, c->pos, c->cfg.rope_theta);
    return 0;
}
static int call_store(void *p) {
    bench_ctx *c = p;
    return tq_store_kv_device(&c->cache, &c->cfg, c->pos, c->k, c->v);
}
static int call_attend(void *p) {
    bench_ctx *c = p;
    return tq_attend_device(&c->cache, &c->cfg, c->q, c->pos, c->out);
}

static float urand(unsigned *s) {
    *s = *s * 1664525u + 1013904223u;
    return (float)(*s >> 8) / 16777216.0f * 2.0f - 1.0f;
}

int main(int argc, char **argv) {
    bench_ctx c;
    memset(&c, 0, sizeof c);
    c.pos = argc > 1 ? atoi(argv[1]) : 4095;
    const int calls = argc > 2 ? atoi(argv[2]) : 2000;
    c.cfg = (tq_attn_config){32, 8, 128, 4096, 500000.0f, 1e-5f};
    const int max_tokens = c.pos + 1;
    if (c.pos < 0 || calls <= 0) {
        fprintf(stderr, "usage: boundary_bench [pos >= 0] [calls > 0]\n");
        return 2;
    }
    if (tq_hip_init(0) != TQ_HIP_OK || tq_kv_cache_init(&c.cache, TQ_KV_Q8_DEVICE, &c.cfg, max_tokens) != 0) {
        fprintf(stderr, "boundary_bench: no gfx950 device cache\n");
        return 1;
    }
    const int nb = c.cfg.head_dim / QK;
    const size_t rows = (size_t)c.cfg.n_kv_heads * max_tokens * nb;
    block_q8 *kq = malloc(rows * sizeof *kq), *vq = malloc(rows * sizeof *vq);
    const size_t qn = (size_t)c.cfg.n_q_heads * c.cfg.head_dim, kn = (size_t)c.cfg.n_kv_heads * c.cfg.head_dim;
    c.q = malloc(qn * sizeof(float));
    c.out = malloc(qn * sizeof(float));
    c.k = malloc(kn * sizeof(float));
    c.v = malloc(kn * sizeof(float));
    c.cos_t = malloc(c.cfg.head_dim / 2 * sizeof(float));
    c.sin_t = malloc(c.cfg.head_dim / 2 * sizeof(float));
    if (!kq || !vq || !c.q || !c.out || !c.k || !c.v || !c.cos_t || !c.sin_t) return 1;
    unsigned seed = 2024;
    for (size_t i = 0; i < rows; i++) {
        kq[i].d = 0.01f + 0.01f * (urand(&seed) + 1.0f);
        vq[i].d = 0.01f + 0.01f * (urand(&seed) + 1.0f);
        for (int j = 0; j < QK; j++) {
            kq[i].q[j] = (int8_t)(127.0f * urand(&seed));
            vq[i].q[j] = (int8_t)(127.0f * urand(&seed));
        }
    }
    for (size_t i = 0; i < qn; i++) c.q[i] = urand(&seed);
    for (size_t i = 0; i < kn; i++) {
        c.k[i] = urand(&seed);
        c.v[i] = urand(&seed);
    }
    if (tq_kv_cache_upload(&c.cache, kq, vq) != 0) {
        fprintf(stderr, "boundary_bench: upload failed\n");
        return 1;
    }
    int rc_core, rc_rope, rc_store, rc_attend;
    const double core = time_calls(call_core, &c, calls, &rc_core);
    const double rope = time_calls(call_rope, &c, calls, &rc_rope);
    const double store = time_calls(call_store, &c, calls, &rc_store);
    const double attend = time_calls(call_attend, &c, calls, &rc_attend);
    if (rc_core || rc_rope || rc_store || rc_attend) {
        fprintf(stderr, "boundary_bench: call failed (%d %d %d %d)\n", rc_core, rc_rope, rc_store, rc_attend);
        return 1;
    }
    double sum = 0.0;
    for (size_t i = 0; i < qn; i++) sum += c.out[i];
    printf("{\"pos\": %d, \"calls\": %d, \"attention_core_us\": %.3f, \"rope_table_us\": %.3f, "
           "\"store_kv_device_us\": %.3f, \"attend_device_us\": %.3f, \"out_checksum\": %.6e}\n",
           c.pos, calls, core, rope, store, attend, sum);
    tq_kv_cache_free(&c.cache);
    free(kq);
    free(vq);
    free(c.q);
    free(c.out);
    free(c.k);
    free(c.v);
    free(c.cos_t);
    free(c.sin_t);
    return 0;
}
