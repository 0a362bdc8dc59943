/* tq_oracle.c — CPU restatement of the reference's scalar Q8 attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle): loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product libraries.  Built with gcc -O2 -ffp-contract=off (see Makefile) so
 * that every a*b+c below is a rounded multiply followed by a rounded add, the
 * same operation sequence the reference's scalar code executes on x86-64
 * without -mfma.
 *
 * Pinning (tests/test_oracle.py): every function here is checked bit for bit
 * against the compiled reference (oracle/_ref, when built) and against the
 * committed golden vectors in tests/golden/ made from it, and also against
 * closed forms: fp64 brute force for scores/accum/softmax/attention, RoPE
 * identities, and quantizer invariants (max|q| = 127, ties to even).
 */
#include "tq_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* kernel/quant_x.c:5-10.  Adding 1.5*2^23 moves v into the binade where the
 * fp32 ulp is 1, so the add itself rounds v to the nearest integer with ties
 * to even; the low mantissa bits then hold that integer (two's complement
 * relative to the constant's bit pattern).  The int8 result is the low byte
 * of the difference, which is also what a NaN or out-of-range input yields. */
static int8_t rne_code(float v) {
    const float shifted = v + 12582912.0f;
    uint32_t bits;
    memcpy(&bits, &shifted, sizeof bits);
    return (int8_t)(uint8_t)((bits - 0x4B400000u) & 0xFFu);
}

/* kernel/quant_x.c:12-33: per 32 values, scale = amax/127, inverse 0 for an
 * all-zero block, codes = RNE(x * inverse). */
void oracle_quantize_row_q8(const float *x, block_q8 *out, int n) {
    const int nblocks = n / QK;
    for (int b = 0; b < nblocks; b++) {
        const float *xb = x + (size_t)b * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) {
            float a = xb[j];
            if (a < 0) a = -a;
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float inv = (d != 0.0f) ? 1.0f / d : 0.0f;
        out[b].d = d;
        for (int j = 0; j < QK; j++) out[b].q[j] = rne_code(xb[j] * inv);
    }
}

/* model/rope.c:4-12: freq_i = theta^(-2 i / hd), angle = pos * freq_i, with
 * the exponent evaluated as (-2.0f * i) * (1.0f / hd) in fp32. */
void oracle_rope_table(float *cos_t, float *sin_t, int head_dim, int pos, float theta) {
    const float inv_hd = 1.0f / (float)head_dim;
    for (int i = 0; i < head_dim / 2; i++) {
        const float e = (-2.0f * (float)i) * inv_hd;
        const float freq = powf(theta, e);
        const float angle = (float)pos * freq;
        cos_t[i] = cosf(angle);
        sin_t[i] = sinf(angle);
    }
}

/* model/rope.c:14-22: rotate-half pairing of i with i + hd/2. */
void oracle_rope_apply(float *x, int head_dim, const float *cos_t, const float *sin_t) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; i++) {
        const float a = x[i], b = x[i + half];
        x[i] = a * cos_t[i] - b * sin_t[i];
        x[i + half] = a * sin_t[i] + b * cos_t[i];
    }
}

/* model/softmax.c:4-23: max-subtracted expf, serial sum, scale by 1/sum. */
void oracle_softmax(float *x, int n) {
    if (n <= 0) return;
    float m = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > m) m = x[i];
    float total = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        total += x[i];
    }
    const float r = 1.0f / total;
    for (int i = 0; i < n; i++) x[i] *= r;
}

/* model/attn_q8.c:17-34: per (token, head) an exact int32 dot per block,
 * scaled by (qd * kd) and summed over blocks in order in fp32, times scale. */
void oracle_attn_scores_q8(const block_q8 *q, int g, const block_q8 *k, int n, int nb,
                           float scale, float *scores, size_t stride) {
    for (int t = 0; t < n; t++) {
        const block_q8 *krow = k + (size_t)t * nb;
        for (int h = 0; h < g; h++) {
            const block_q8 *qrow = q + (size_t)h * nb;
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) {
                int32_t dot = 0;
                for (int j = 0; j < QK; j++)
                    dot += (int32_t)qrow[b].q[j] * (int32_t)krow[b].q[j];
                const float dd = qrow[b].d * krow[b].d;
                acc += (float)dot * dd;
            }
            scores[(size_t)h * stride + t] = acc * scale;
        }
    }
}

/* model/attn_q8.c:36-54: out[h][j] = sum_t (w[h][t] * vd[t][b]) * code[t][j],
 * zeroed first, tokens in order. */
void oracle_attn_accum_q8(const float *w, size_t w_stride, int g, const block_q8 *v,
                          int n, int nb, float *out, size_t out_stride) {
    const int hd = nb * QK;
    for (int h = 0; h < g; h++) {
        float *o = out + (size_t)h * out_stride;
        for (int j = 0; j < hd; j++) o[j] = 0.0f;
        for (int t = 0; t < n; t++) {
            const float wt = w[(size_t)h * w_stride + t];
            const block_q8 *vrow = v + (size_t)t * nb;
            for (int b = 0; b < nb; b++) {
                const float a = wt * vrow[b].d;
                for (int j = 0; j < QK; j++) o[b * QK + j] += a * (float)vrow[b].q[j];
            }
        }
    }
}

/* model/attn_q8.c:78-90: one head (g = 1); q_q8 is an output. */
void oracle_attention_head_q8(const float *q, block_q8 *q_q8, const block_q8 *k_cache,
                              const block_q8 *v_cache, int n, int head_dim,
                              float *scores, float *out) {
    const int nb = head_dim / QK;
    const float scale = 1.0f / sqrtf((float)head_dim);
    oracle_quantize_row_q8(q, q_q8, head_dim);
    oracle_attn_scores_q8(q_q8, 1, k_cache, n, nb, scale, scores, (size_t)n);
    oracle_softmax(scores, n);
    oracle_attn_accum_q8(scores, (size_t)n, 1, v_cache, n, nb, out, (size_t)head_dim);
}

/* model/attention_layer.c:62-64 */
static size_t slot_of(int max_tokens, int h, int pos) {
    return (size_t)h * (size_t)max_tokens + (size_t)pos;
}

/* model/attention_layer.c:66-90, Q8 branch. */
int oracle_store_kv_q8(block_q8 *k_cache, block_q8 *v_cache, int n_kv_heads, int head_dim,
                       int max_tokens, int pos, const float *k, const float *v) {
    if (pos < 0 || pos >= max_tokens) return -1;
    const int nb = head_dim / QK;
    for (int h = 0; h < n_kv_heads; h++) {
        const size_t base = slot_of(max_tokens, h, pos) * (size_t)nb;
        oracle_quantize_row_q8(k + (size_t)h * head_dim, k_cache + base, head_dim);
        oracle_quantize_row_q8(v + (size_t)h * head_dim, v_cache + base, head_dim);
    }
    return 0;
}

/* model/attention_layer.c:125-150.  The group's q rows are quantized, scored
 * against tokens 0..pos of their kv head, softmaxed per head and accumulated
 * against V.  q head h reads kv head h / (n_q_heads / n_kv_heads). */
int oracle_attend_q8(const block_q8 *k_cache, const block_q8 *v_cache, int n_q_heads,
                     int n_kv_heads, int head_dim, int max_tokens, const float *q, int pos,
                     float *scores, float *out) {
    if (pos < 0 || pos >= max_tokens) return -1;
    const int nb = head_dim / QK;
    const int n = pos + 1;
    const int group = n_q_heads / n_kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t stride = (size_t)max_tokens;
    block_q8 qq[group * nb];

    for (int kvh = 0; kvh < n_kv_heads; kvh++) {
        const float *qg = q + (size_t)kvh * group * head_dim;
        float *og = out + (size_t)kvh * group * head_dim;
        float *sg = scores + (size_t)kvh * group * stride;
        const size_t base = slot_of(max_tokens, kvh, 0) * (size_t)nb;
        for (int h = 0; h < group; h++)
            oracle_quantize_row_q8(qg + (size_t)h * head_dim, qq + (size_t)h * nb, head_dim);
        oracle_attn_scores_q8(qq, group, k_cache + base, n, nb, scale, sg, stride);
        for (int h = 0; h < group; h++) oracle_softmax(sg + (size_t)h * stride, n);
        oracle_attn_accum_q8(sg, stride, group, v_cache + base, n, nb, og, (size_t)head_dim);
    }
    return 0;
}

int oracle_attention_qkv(block_q8 *k_cache, block_q8 *v_cache, int n_q_heads, int n_kv_heads,
                         int head_dim, int max_tokens, float rope_theta, int pos,
                         float *q, float *k, const float *v, float *scores, float *out) {
    if (pos < 0 || pos >= max_tokens) return -1;
    float cos_t[head_dim / 2], sin_t[head_dim / 2];
    oracle_rope_table(cos_t, sin_t, head_dim, pos, rope_theta);
    for (int h = 0; h < n_q_heads; h++)
        oracle_rope_apply(q + (size_t)h * head_dim, head_dim, cos_t, sin_t);
    for (int h = 0; h < n_kv_heads; h++)
        oracle_rope_apply(k + (size_t)h * head_dim, head_dim, cos_t, sin_t);
    oracle_store_kv_q8(k_cache, v_cache, n_kv_heads, head_dim, max_tokens, pos, k, v);
    return oracle_attend_q8(k_cache, v_cache, n_q_heads, n_kv_heads, head_dim, max_tokens,
                            q, pos, scores, out);
}

int oracle_prefill_qkv(block_q8 *k_cache, block_q8 *v_cache, int n_q_heads, int n_kv_heads,
                       int head_dim, int max_tokens, float rope_theta, int pos0, int n,
                       float *q, float *k, const float *v, float *scores, float *out) {
    if (n <= 0) return -1;
    if (pos0 < 0 || pos0 + n > max_tokens) return -1;
    const size_t qdim = (size_t)n_q_heads * head_dim;
    const size_t kvdim = (size_t)n_kv_heads * head_dim;
    for (int i = 0; i < n; i++) {
        int rc = oracle_attention_qkv(k_cache, v_cache, n_q_heads, n_kv_heads, head_dim,
                                      max_tokens, rope_theta, pos0 + i, q + i * qdim,
                                      k + i * kvdim, v + i * kvdim, scores, out + i * qdim);
        if (rc != 0) return rc;
    }
    return 0;
}

/* ---- weight side: packing and the Q8 weight x Q8 activation matmul ------ */

/* packer/packer.c:4-9,11-19,22-31 (quantize, block_scale, pack_row_q8):
 * per 32 weights, d = amax/127 with 1 in place of 0 for an all-zero block,
 * inverse 1/d, code = lroundf(w * inverse) (half away from zero) clamped to
 * [-127, 127].  This differs from quantize_row_q8 on purpose: the activation
 * quantizer rounds half to even and keeps d = 0. */
void oracle_pack_matrix_q8(const float *W, int rows, int cols, block_q8 *out) {
    const int nb = cols / QK;
    for (int r = 0; r < rows; r++) {
        for (int b = 0; b < nb; b++) {
            const float *w = W + (size_t)r * cols + (size_t)b * QK;
            block_q8 *o = out + (size_t)r * nb + b;
            float amax = 0.0f;
            for (int j = 0; j < QK; j++) {
                const float v = fabsf(w[j]);
                if (v > amax) amax = v;
            }
            float d = amax / 127.0f;
            if (d == 0.0f) d = 1.0f;
            const float id = 1.0f / d;
            o->d = d;
            for (int j = 0; j < QK; j++) {
                long q = lroundf(w[j] * id);
                if (q > 127) q = 127;
                if (q < -127) q = -127;
                o->q[j] = (int8_t)q;
            }
        }
    }
}

/* packer/packer.c:40-52: block_scale (:11-19) with qmax 7 (d = amax / 7, 1
 * for an all-zero block), codes lroundf(w * (1/d)) clamped to [-7, 7] (:4-9),
 * stored + 8 with code j in the low nibble of byte j and code j + 16 in the
 * high nibble. */
void oracle_pack_matrix_q4(const float *W, int rows, int cols, block_q4 *out) {
    const int nb = cols / QK;
    for (int r = 0; r < rows; r++) {
        for (int b = 0; b < nb; b++) {
            const float *w = W + (size_t)r * cols + (size_t)b * QK;
            block_q4 *o = out + (size_t)r * nb + b;
            float amax = 0.0f;
            for (int j = 0; j < QK; j++) {
                const float v = fabsf(w[j]);
                if (v > amax) amax = v;
            }
            float d = amax / 7.0f;
            if (d == 0.0f) d = 1.0f;
            const float id = 1.0f / d;
            o->d = d;
            for (int j = 0; j < QK / 2; j++) {
                long lo = lroundf(w[j] * id), hi = lroundf(w[j + QK / 2] * id);
                lo = lo > 7 ? 7 : (lo < -7 ? -7 : lo);
                hi = hi > 7 ? 7 : (hi < -7 ? -7 : hi);
                o->q[j] = (uint8_t)(((hi + 8) << 4) | (lo + 8));
            }
        }
    }
}

/* packer/packer.c:54-61: ((nibble) - 8) * d. */
void oracle_unpack_matrix_q4(const block_q4 *in, int rows, int cols, float *out) {
    const int nb = cols / QK;
    for (int r = 0; r < rows; r++) {
        for (int b = 0; b < nb; b++) {
            const block_q4 *k = in + (size_t)r * nb + b;
            float *o = out + (size_t)r * cols + (size_t)b * QK;
            for (int j = 0; j < QK / 2; j++) {
                o[j] = (float)((k->q[j] & 0x0F) - 8) * k->d;
                o[j + QK / 2] = (float)((k->q[j] >> 4) - 8) * k->d;
            }
        }
    }
}

/* kernel/q4_scalar.c:3-15: per block the exact int32 sum of (nibble - 8) *
 * x code over the 16 low and 16 high codes, then ((float)s * w.d) * x.d added
 * to one serial fp32 sum in block order. */
static float dot_q4(const block_q4 *w, const block_q8 *x, int nb) {
    float sum = 0.0f;
    for (int b = 0; b < nb; b++) {
        int32_t s = 0;
        for (int j = 0; j < QK / 2; j++) {
            const int lo = (w[b].q[j] & 0x0F) - 8;
            const int hi = (w[b].q[j] >> 4) - 8;
            s += lo * x[b].q[j] + hi * x[b].q[j + QK / 2];
        }
        sum += (float)s * w[b].d * x[b].d;
    }
    return sum;
}

void oracle_matmul_q4_batch(const block_q4 *W, const block_q8 *xq, float *y, int rows, int cols, int n_tok) {
    const int nb = cols / QK;
    for (int t = 0; t < n_tok; t++)
        for (int r = 0; r < rows; r++)
            y[(size_t)t * rows + r] = dot_q4(W + (size_t)r * nb, xq + (size_t)t * nb, nb);
}

/* model/embedding.c:20-27: the unpacked row `token`. */
int oracle_embed_lookup_q4(const block_q4 *embed, int rows, int cols, int token, float *out) {
    if (token < 0 || token >= rows || cols % QK != 0) return -1;
    oracle_unpack_matrix_q4(embed + (size_t)token * (cols / QK), 1, cols, out);
    return 0;
}

/* kernel/q8_scalar.c:3-13: exact int32 dot of each block's codes, then
 * ((float)s * w.d) * x.d added to one serial fp32 sum in block order. */
static float dot_q8(const block_q8 *w, const block_q8 *x, int nb) {
    float sum = 0.0f;
    for (int b = 0; b < nb; b++) {
        int32_t s = 0;
        for (int j = 0; j < QK; j++) s += (int32_t)w[b].q[j] * (int32_t)x[b].q[j];
        sum += (float)s * w[b].d * x[b].d;
    }
    return sum;
}

/* kernel/q8_scalar.c:15-22: y[r] = dot(W row r, xq). */
void oracle_matmul_q8(const block_q8 *W, const block_q8 *xq, float *y, int rows, int cols) {
    const int nb = cols / QK;
    for (int r = 0; r < rows; r++) y[r] = dot_q8(W + (size_t)r * nb, xq, nb);
}

/* kernel/q8_scalar.c:25-30: token t reads xq + t*nb and writes y + t*rows. */
void oracle_matmul_q8_batch(const block_q8 *W, const block_q8 *xq, float *y, int rows, int cols,
                            int n_tok) {
    const int nb = cols / QK;
    for (int t = 0; t < n_tok; t++)
        oracle_matmul_q8(W, xq + (size_t)t * nb, y + (size_t)t * rows, rows, cols);
}

/* A projection as attention_layer makes it: quantize_row_q8 of each input
 * row, then the Q8 matmul (project_qkv for one matrix,
 * model/attention_layer.c:38-46; project_output, :161-167; the batched
 * versions quantize every token row first, :213-218 and :238-241).
 * x: n_tok rows of cols floats; y: n_tok rows of rows floats. */
void oracle_project_q8(const block_q8 *W, int rows, int cols, const float *x, int n_tok,
                       float *y) {
    const int nb = cols / QK;
    block_q8 xq[nb > 0 ? nb : 1];
    for (int t = 0; t < n_tok; t++) {
        oracle_quantize_row_q8(x + (size_t)t * cols, xq, cols);
        oracle_matmul_q8(W, xq, y + (size_t)t * rows, rows, cols);
    }
}

/* model/rmsnorm.c:4-19: sum of squares in one serial fp32 pass, rms =
 * sqrtf(eps + sum / n), inverse 1/rms, out = (x * inverse) * weight.  In place
 * (out == x) is allowed, as norm_heads uses it (model/attention_layer.c:48-53). */
void oracle_rmsnorm(const float *x, const float *weight, float *out, int n, float eps) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += x[i] * x[i];
    const float inv = 1.0f / sqrtf(eps + sum / (float)n);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * weight[i];
}

/* One matmul / projection in a weight format: 0 Q8 (kernel/q8_scalar.c), 1 Q4
 * (kernel/q4_scalar.c), as get_matmul(format) picks (kernel/dispatch.c). */
static void matmul_fmt(int fmt, const void *W, const block_q8 *xq, float *y, int rows, int cols) {
    if (fmt == 1)
        oracle_matmul_q4_batch((const block_q4 *)W, xq, y, rows, cols, 1);
    else
        oracle_matmul_q8((const block_q8 *)W, xq, y, rows, cols);
}

static void project_fmt(int fmt, const void *W, int rows, int cols, const float *x, float *y) {
    const int nb = cols / QK;
    block_q8 xq[nb > 0 ? nb : 1];
    oracle_quantize_row_q8(x, xq, cols);
    matmul_fmt(fmt, W, xq, y, rows, cols);
}

static int attention_layer_fmt(int fmt, const void *wq, const void *wk, const void *wv, const void *wo,
                               const float *q_norm, const float *k_norm, int n_q_heads, int n_kv_heads,
                               int head_dim, int hidden, float rope_theta, float rms_eps, block_q8 *k_cache,
                               block_q8 *v_cache, int max_tokens, int pos, const float *xn, float *scores,
                               float *out);
static int mlp_layer_fmt(int fmt, const void *wgate, const void *wup, const void *wdown, int hidden, int inter,
                         const float *xn, float *out);

/* model/attention_layer.c:169-194 (attention_layer) on the flat Q8 cache:
 * project_qkv (quantize_row_q8 of xn, then wq, wk, wv), per-head RMSNorm of q
 * and k (:48-53), RoPE + store_kv + attend_q8 (oracle_attention_qkv), then
 * project_output (quantize the attention output, then wo).  Returns -1 for a
 * bad pos before any write. */
int oracle_attention_layer(const block_q8 *wq, const block_q8 *wk, const block_q8 *wv,
                           const block_q8 *wo, const float *q_norm, const float *k_norm,
                           int n_q_heads, int n_kv_heads, int head_dim, int hidden,
                           float rope_theta, float rms_eps, block_q8 *k_cache,
                           block_q8 *v_cache, int max_tokens, int pos, const float *xn,
                           float *scores, float *out) {
    return attention_layer_fmt(0, wq, wk, wv, wo, q_norm, k_norm, n_q_heads, n_kv_heads, head_dim, hidden,
                               rope_theta, rms_eps, k_cache, v_cache, max_tokens, pos, xn, scores, out);
}

static int attention_layer_fmt(int fmt, const void *wq, const void *wk, const void *wv, const void *wo,
                               const float *q_norm, const float *k_norm, int n_q_heads, int n_kv_heads,
                               int head_dim, int hidden, float rope_theta, float rms_eps, block_q8 *k_cache,
                               block_q8 *v_cache, int max_tokens, int pos, const float *xn, float *scores,
                               float *out) {
    if (pos < 0 || pos >= max_tokens) return -1;
    const int qdim = n_q_heads * head_dim, kvdim = n_kv_heads * head_dim;
    float q[qdim], k[kvdim], v[kvdim], attn[qdim];
    project_fmt(fmt, wq, qdim, hidden, xn, q);
    project_fmt(fmt, wk, kvdim, hidden, xn, k);
    project_fmt(fmt, wv, kvdim, hidden, xn, v);
    for (int h = 0; h < n_q_heads; h++)
        oracle_rmsnorm(q + (size_t)h * head_dim, q_norm, q + (size_t)h * head_dim, head_dim, rms_eps);
    for (int h = 0; h < n_kv_heads; h++)
        oracle_rmsnorm(k + (size_t)h * head_dim, k_norm, k + (size_t)h * head_dim, head_dim, rms_eps);
    int rc = oracle_attention_qkv(k_cache, v_cache, n_q_heads, n_kv_heads, head_dim, max_tokens,
                                  rope_theta, pos, q, k, v, scores, attn);
    if (rc != 0) return rc;
    project_fmt(fmt, wo, hidden, qdim, attn, out);
    return 0;
}

/* ---- the rest of the block: MLP, embedding, lm_head, sampler, forward ---- */

/* model/silu.c:6-18: out = silu(g) * u, silu(x) = x * (1 / (1 + expf(-x))). */
void oracle_silu_mul(const float *gate, const float *up, float *out, int n) {
    for (int i = 0; i < n; i++) {
        const float g = gate[i];
        const float sig = 1.0f / (1.0f + expf(-g));
        out[i] = g * sig * up[i];
    }
}

/* model/mlp.c:3-17 (mlp_layer): quantize xn, gate and up matmuls, silu_mul,
 * quantize, down matmul.  wgate/wup: inter x hidden; wdown: hidden x inter. */
int oracle_mlp_layer(const block_q8 *wgate, const block_q8 *wup, const block_q8 *wdown, int hidden,
                     int inter, const float *xn, float *out) {
    return mlp_layer_fmt(0, wgate, wup, wdown, hidden, inter, xn, out);
}

static int mlp_layer_fmt(int fmt, const void *wgate, const void *wup, const void *wdown, int hidden, int inter,
                         const float *xn, float *out) {
    if (hidden % QK != 0 || inter % QK != 0) return -1;
    float *gate = (float *)malloc((size_t)inter * sizeof(float));
    float *up = (float *)malloc((size_t)inter * sizeof(float));
    block_q8 *q = (block_q8 *)malloc((size_t)(inter > hidden ? inter : hidden) / QK * sizeof(block_q8));
    if (!gate || !up || !q) {
        free(gate); free(up); free(q);
        return -100;
    }
    oracle_quantize_row_q8(xn, q, hidden);
    matmul_fmt(fmt, wgate, q, gate, inter, hidden);
    matmul_fmt(fmt, wup, q, up, inter, hidden);
    oracle_silu_mul(gate, up, gate, inter);
    oracle_quantize_row_q8(gate, q, inter);
    matmul_fmt(fmt, wdown, q, out, hidden, inter);
    free(gate); free(up); free(q);
    return 0;
}

/* model/embedding.c:4-17, Q8 branch: out[b*32+j] = d * q[j] of row `token`. */
int oracle_embed_lookup_q8(const block_q8 *embed, int rows, int cols, int token, float *out) {
    if (token < 0 || token >= rows || cols % QK != 0) return -1;
    const int nb = cols / QK;
    const block_q8 *row = embed + (size_t)token * nb;
    for (int b = 0; b < nb; b++)
        for (int j = 0; j < QK; j++) out[b * QK + j] = row[b].d * (float)row[b].q[j];
    return 0;
}

/* model/sampler.c:3-13: the first index of the largest logit (strict >). */
int oracle_sample_greedy(const float *logits, int n) {
    if (n <= 0) return -1;
    float m = logits[0];
    int idx = 0;
    for (int i = 1; i < n; i++)
        if (logits[i] > m) {
            m = logits[i];
            idx = i;
        }
    return idx;
}

/* model/context.c:104-126 (tq_forward_token) with Q8 weights and the flat Q8
 * caches: embed_lookup, per layer rmsnorm(input_norm) -> attention_layer ->
 * x += attn (vec_add, model/vec.c:3-6) -> rmsnorm(post_norm) -> mlp_layer ->
 * x += mlp, then rmsnorm(final_norm) and lm_head (model/embedding.c:35-40:
 * quantize + matmul against the embedding).  Per-layer pointers come in arrays
 * of n_layers; caches[l] are [n_kv][max_tokens][nb] K then V arrays. */
int oracle_forward_token(const struct oracle_model *m, block_q8 *const *k_caches,
                         block_q8 *const *v_caches, int max_tokens, int pos, int token, float *logits) {
    const int hidden = m->hidden;
    if (pos < 0 || pos >= max_tokens || token < 0 || token >= m->vocab) return -1;
    float *x = (float *)malloc((size_t)hidden * sizeof(float));
    float *xn = (float *)malloc((size_t)hidden * sizeof(float));
    float *y = (float *)malloc((size_t)hidden * sizeof(float));
    float *scores = (float *)malloc((size_t)m->n_q_heads * max_tokens * sizeof(float));
    int rc = (x && xn && y && scores) ? 0 : -100;
    if (rc == 0)
        rc = m->embed_format == 1 ? oracle_embed_lookup_q4((const block_q4 *)m->embed, m->vocab, hidden, token, x)
                                  : oracle_embed_lookup_q8((const block_q8 *)m->embed, m->vocab, hidden, token, x);
    for (int l = 0; rc == 0 && l < m->n_layers; l++) {
        oracle_rmsnorm(x, m->input_norm[l], xn, hidden, m->rms_eps);
        rc = attention_layer_fmt(m->format, m->wq[l], m->wk[l], m->wv[l], m->wo[l], m->q_norm[l], m->k_norm[l],
                                 m->n_q_heads, m->n_kv_heads, m->head_dim, hidden, m->rope_theta,
                                 m->rms_eps, k_caches[l], v_caches[l], max_tokens, pos, xn, scores, y);
        if (rc != 0) break;
        for (int i = 0; i < hidden; i++) x[i] += y[i];
        oracle_rmsnorm(x, m->post_norm[l], xn, hidden, m->rms_eps);
        rc = mlp_layer_fmt(m->format, m->wgate[l], m->wup[l], m->wdown[l], hidden, m->inter, xn, y);
        if (rc != 0) break;
        for (int i = 0; i < hidden; i++) x[i] += y[i];
    }
    if (rc == 0) {
        oracle_rmsnorm(x, m->final_norm, xn, hidden, m->rms_eps);
        project_fmt(m->embed_format, m->embed, m->vocab, hidden, xn, logits);
    }
    free(x); free(xn); free(y); free(scores);
    return rc;
}
