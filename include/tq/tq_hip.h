/* tq_hip.h — C-ABI of libtqhip.so, the MI355X (gfx950) Q8 GQA attention path.
 *
 * Plain pointers and sizes only.  Every call returns 0 on success or a
 * negative code (TQ_HIP_E*); HIP runtime errors come back as
 * TQ_HIP_EHIP_BASE - hipError_t.  No call aborts the process.
 *
 * Two kinds of entry point:
 *   - synchronous ones take HOST buffers, copy them in, run, copy results out
 *     and return with the results valid (the boundary of attention_layer).
 *     A call that waits on completion flags returns as soon as its outputs are
 *     visible in host memory, which may be before the cache's stream has
 *     drained (the kernel's last waves may still be retiring); work enqueued
 *     next on that stream is still ordered after it.  The host thread spins
 *     (with a pause hint, not a yield) while it waits, and asks the stream
 *     for its status only once the flags are 25 us late, so that a device
 *     error still ends the wait;
 *   - *_async ones take DEVICE buffers and a stream (hipStream_t as void*,
 *     NULL = the cache's own stream) and only enqueue work.
 *
 * Environment variables named TQ_HIP_* are for tests and plan sweeps only:
 * each forces one launch plan or code path for A/B comparisons, and
 * production callers leave them unset.  Results stay within the documented
 * tolerances under every setting.  Decode: TQ_HIP_DECODE_WG_TARGET,
 * TQ_HIP_DECODE_MAX_SPLITS, TQ_HIP_DECODE_SPLIT_CAP, TQ_HIP_DECODE_WAVES,
 * TQ_HIP_DECODE_KERNEL; prefill: TQ_HIP_PREFILL_DENSE, TQ_HIP_PREFILL_ROWS,
 * TQ_HIP_PREFILL_WHOLE, TQ_HIP_PREFILL_FUSED_NORM, TQ_HIP_PREFILL_QUANT_OUT; weight matmuls:
 * TQ_HIP_GEMV_RW, TQ_HIP_GEMV_GC, TQ_HIP_GEMM_MIN_TOKENS, TQ_HIP_GEMM_SPLIT,
 * TQ_HIP_GEMM_XS, TQ_HIP_MLP_FUSED.
 *
 * KV storage is an HBM-resident paged cache.  A page holds TQ_HIP_PAGE_TOKENS
 * consecutive positions of one sequence for every kv head, K then V:
 *   page[kvh][0=K,1=V][16 tokens][head_dim/32] block_q8
 * so one (page, kv head) is a contiguous 2 * 16 * head_dim/32 * 36 byte run
 * (4,608 B at head_dim 128).  Each sequence owns a page table (logical page ->
 * physical page).  Within a token row the bytes are exactly the reference's
 * block_q8 row (model/attention_layer.c:62-64, packer/packer.h:7-11).
 */
#ifndef TQ_HIP_H
#define TQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "block_q8.h"

#ifdef __cplusplus
extern "C" {
#endif

#define TQ_HIP_PAGE_TOKENS 16

#define TQ_HIP_OK 0
#define TQ_HIP_EINVAL (-1)     /* argument out of range: pos, n, seq, shape     */
#define TQ_HIP_ENOMEM (-2)     /* device or host allocation failed              */
#define TQ_HIP_ETYPE (-3)      /* unsupported head_dim / group size             */
#define TQ_HIP_ENODEV (-4)     /* no usable gfx950 device                        */
#define TQ_HIP_ENOTREADY (-5)  /* sequence has no page for a requested position  */
#define TQ_HIP_ESCRATCH (-6)   /* beyond the allocation-free call's fixed scratch */
#define TQ_HIP_EHIP_BASE (-1000)

/* ---- device and plumbing ------------------------------------------------ */

/* Select the device for this thread and check it is gfx950.  Idempotent. */
int tq_hip_init(int device);
const char *tq_hip_strerror(int code);
/* Name of the current device's architecture (e.g. "gfx950:sramecc+:xnack-"). */
int tq_hip_device_arch(char *buf, size_t len);

int tq_hip_malloc(void **ptr, size_t bytes);
int tq_hip_free(void *ptr);
/* stream NULL: synchronous copy. */
int tq_hip_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int tq_hip_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int tq_hip_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
int tq_hip_stream_synchronize(void *stream);
int tq_hip_device_synchronize(void);

/* ---- kernel-level ops on flat block_q8 arrays (device pointers) --------- */

/* kernel/quant_x.c:12-33 quantize_row_q8: x[n] -> out[n/32], bit-exact.  x and out
 * must be 4-byte aligned (a float array, a block_q8 array), else -1. */
int tq_hip_quantize_row_q8(const float *x, block_q8 *out, int n, void *stream);

/* model/rope.c:14-22 rope_apply on n_heads consecutive heads of x, in place,
 * with a host-computed cos/sin table of head_dim/2 entries (bit-exact). */
int tq_hip_rope_apply(float *x, int n_heads, int head_dim, const float *cos_t,
                      const float *sin_t, void *stream);

/* model/attn_q8.c:17-34 attn_scores_q8(_scalar): scores[gi*stride + t] for
 * t < n, gi < g; nothing at or past n is written.  Bit-exact vs the scalar. */
int tq_hip_attn_scores_q8(const block_q8 *q, int g, const block_q8 *k, int n, int nb,
                          float scale, float *scores, size_t stride, void *stream);

/* model/attn_q8.c:36-54 attn_accum_q8(_scalar): out[gi*out_stride + j], j < nb*32,
 * zeroed first; nothing past nb*32 is written.  Bit-exact vs the scalar. */
int tq_hip_attn_accum_q8(const float *w, size_t w_stride, int g, const block_q8 *v, int n,
                         int nb, float *out, size_t out_stride, void *stream);

/* model/softmax.c:4-23 softmax on `rows` rows of n values, row r at x + r*stride. */
int tq_hip_softmax(float *x, int n, int rows, size_t stride, void *stream);

/* rmsnorm (model/rmsnorm.c:4-19) of n_rows rows of n floats with one weight
 * row, as norm_heads applies it per head (model/attention_layer.c:48-53);
 * the squares are summed serially in element order, so the result is the
 * reference's bit for bit.  out may equal x.  n <= 8191. */
int tq_hip_rmsnorm_rows(const float *x, const float *weight, float *out, int n_rows, int n, float eps,
                        void *stream);

/* model/attn_q8.c:78-90 attention_head_q8: writes q_q8 (head_dim/32 blocks),
 * scores[n] (the softmax weights) and out[head_dim]. */
int tq_hip_attention_head_q8(const float *q, block_q8 *q_q8, const block_q8 *k_cache,
                             const block_q8 *v_cache, int n, int head_dim, float *scores,
                             float *out, void *stream);

/* ---- paged KV cache -------------------------------------------------------
 * Replaces tq_kv_cache_init / tq_kv_cache_free (model/kv_cache.c:17-48) for a
 * device-resident Q8 cache; the reference's flat layout becomes one sequence
 * whose page table is the identity. */

typedef struct tq_hip_kv tq_hip_kv;

typedef struct {
    int n_q_heads;          /* query heads (sizes decode scratch)        */
    int n_kv_heads;
    int head_dim;           /* 32, 64, 128 or 256                        */
    int n_pages;            /* physical pages in the pool                */
    int max_seqs;           /* sequences (page tables)                   */
    int max_pages_per_seq;  /* logical pages per sequence                */
} tq_hip_kv_desc;

/* Allocate the pool (zero-filled), page tables (all -1) and a stream on the
 * current device.  Returns TQ_HIP_EINVAL for a bad shape (same conditions as
 * tq_attn_validate: model/attention_layer.c:11,16-17), TQ_HIP_ETYPE for a
 * head_dim or group size the kernels do not cover, TQ_HIP_ENOMEM on OOM. */
int tq_hip_kv_create(tq_hip_kv **kv, const tq_hip_kv_desc *desc);
/* Idempotent; NULL is fine. */
void tq_hip_kv_destroy(tq_hip_kv *kv);
/* Map logical pages 0..n_pages-1 of `seq` to the given physical pages (host
 * array); entries of -1 unmap.  Pages past n_pages are unmapped. */
int tq_hip_kv_set_pages(tq_hip_kv *kv, int seq, const int32_t *pages, int n_pages);
/* Tokens addressable in `seq` (mapped logical pages * 16), or < 0. */
int tq_hip_kv_capacity(const tq_hip_kv *kv, int seq);
/* The shape the cache was created with. */
int tq_hip_kv_get_desc(const tq_hip_kv *kv, tq_hip_kv_desc *desc);
void *tq_hip_kv_stream(tq_hip_kv *kv);
/* Device base and size of the pool; device pointer of the page tables
 * ([max_seqs][max_pages_per_seq] int32). */
int tq_hip_kv_pool(tq_hip_kv *kv, void **base, size_t *bytes, int32_t **page_table);

/* Copy rows [pos0, pos0+n) of `seq` between the cache and host block_q8
 * arrays laid out [n_kv_heads][n][head_dim/32] (the reference's flat layout
 * when pos0 = 0 and n = max_tokens).  Either of k/v may be NULL. */
int tq_hip_kv_write(tq_hip_kv *kv, int seq, int pos0, int n, const block_q8 *k, const block_q8 *v);
int tq_hip_kv_read(tq_hip_kv *kv, int seq, int pos0, int n, block_q8 *k, block_q8 *v);

/* ---- append: store_kv, Q8 branch (model/attention_layer.c:66-90) fused with
 * rope_heads on k (:188).  k, v: [n_kv_heads * head_dim] fp32; with cos/sin
 * (head_dim/2 each) k is post-norm and pre-RoPE, with NULL it is already
 * rotated.  K and V codes and scales are bit-exact with quantize_row_q8. */
int tq_hip_kv_append(tq_hip_kv *kv, int seq, int pos, const float *k, const float *v,
                     const float *cos_t, const float *sin_t);
/* Device form for n_rows rows: row r goes to sequence d_seq[r] at position
 * d_pos[r]; k/v rows at r * n_kv_heads * head_dim; cos/sin rows at r *
 * head_dim/2 (or NULL).  Rows whose position has no mapped page are skipped. */
int tq_hip_kv_append_async(tq_hip_kv *kv, int n_rows, const int32_t *d_seq,
                           const int32_t *d_pos, const float *d_k, const float *d_v,
                           const float *d_cos, const float *d_sin, void *stream);

/* ---- decode: attend_q8 (model/attention_layer.c:125-150) -----------------
 * For query i: q heads at q + i*n_q_heads*head_dim (post-RoPE, or pre-RoPE
 * with a cos/sin row), quantized with quantize_row_q8; q head h attends kv
 * head h / (n_q_heads/n_kv_heads) over tokens [0, len) of its sequence;
 * out[i][h][head_dim] fp32.  Split-K over the context with an online softmax;
 * partials are combined in a fixed order, so results do not depend on timing. */
int tq_hip_attend(tq_hip_kv *kv, int seq, int pos, const float *q, const float *cos_t,
                  const float *sin_t, float *out);
/* d_seq may be NULL: query i then reads sequence i.  max_len: an upper bound
 * of every d_len[i] (sizes the grid); at most 64 * 8192 tokens. */
int tq_hip_decode_async(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_len,
                        int max_len, const float *d_q, const float *d_cos, const float *d_sin,
                        float *d_out, void *stream);

/* ---- decode step: the attention core of attention_layer
 * (model/attention_layer.c:186-191): RoPE on q and k, store_kv of token
 * d_pos[i] of sequence d_seq[i], then attend over [0, d_pos[i]].  The new
 * token's K/V are quantized once, written to the cache and used by the same
 * launch.  max_pos: an upper bound of every d_pos[i].  d_seq may be NULL
 * (query i is sequence i); a sequence appears at most once per call. */
int tq_hip_decode_step_async(tq_hip_kv *kv, int n_q, const int32_t *d_seq,
                             const int32_t *d_pos, int max_pos, const float *d_q,
                             const float *d_k, const float *d_v, const float *d_cos,
                             const float *d_sin, float *d_out, void *stream);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tq_hip_decode_step_async with its split-K scratch (the
 * partial rows and arrival counters) taken from one fixed array of
 * TQ_HIP_NOALLOC_SCRATCH_BYTES that the library holds on each GPU until the
 * process ends, instead of buffers the cache grows with hipMalloc.  Same
 * kernels, same results bit for bit; it allocates nothing.  A call whose
 * scratch would not fit — split-K over more than 1024 (query, kv head)
 * pairs, or more partial rows than the rest of the array holds (it holds 64
 * queries of up to 16k tokens or one of up to 512k at the 8B shape, 16 of
 * 32k at the 70B shape) — returns TQ_HIP_ESCRATCH before launching.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (several
 * streams at once) race.  tq_hip_init sets the array up on its device
 * (counters cleared); without it the first call on a device does, and must
 * then not be inside a graph capture. */
#define TQ_HIP_NOALLOC_SCRATCH_BYTES (8u << 20)
int tq_hip_decode_step_noalloc(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_pos,
                               int max_pos, const float *d_q, const float *d_k, const float *d_v,
                               const float *d_cos, const float *d_sin, float *d_out, void *stream);
/* The same step with the per-head RMSNorm of q and of the new K in front of
 * RoPE (norm_heads, model/attention_layer.c:48-53,183-184; model/rmsnorm.c:4-19):
 * d_q and d_k are the projections' raw outputs, d_q_norm / d_k_norm the
 * head_dim weights (16-byte aligned).  The norm keeps the reference's serial
 * sum of squares, so the cached K codes equal those of attention_layer bit for
 * bit.  Head dims 32/64/128 with groups 1..8 (the MFMA decode kernel);
 * TQ_HIP_ETYPE otherwise. */
int tq_hip_decode_step_norm_async(tq_hip_kv *kv, int n_q, const int32_t *d_seq, const int32_t *d_pos,
                                  int max_pos, const float *d_q, const float *d_k, const float *d_v,
                                  const float *d_q_norm, const float *d_k_norm, float rms_eps,
                                  const float *d_cos, const float *d_sin, float *d_out, void *stream);

/* ---- prefill: the attention loop of attention_layer_batch
 * (model/attention_layer.c:203-204,221-236): tokens pos0..pos0+n-1 of `seq`,
 * each stored then attending causally to [0, pos0+i].  q [n][nq*hd], k/v
 * [n][nkv*hd] (k pre-RoPE), cos/sin [n][hd/2], out [n][nq*hd]. */
int tq_hip_prefill(tq_hip_kv *kv, int seq, int pos0, int n, const float *q, const float *k,
                   const float *v, const float *cos_t, const float *sin_t, float *out);
int tq_hip_prefill_async(tq_hip_kv *kv, int seq, int pos0, int n, const float *d_q,
                         const float *d_k, const float *d_v, const float *d_cos,
                         const float *d_sin, float *d_out, void *stream);

/* ---- the weight side: Q8 weight matrices and the projections -----------
 *
 * A weight matrix lives on the device in the "tiled Q8" layout, the same
 * byte count as the reference's rows x cols/32 block_q8 array
 * (packed_matrix_bytes, packer/packer.c:62-75):
 *   codes  [rows][cols] int8; each row in groups of up to 64 blocks, a group
 *          of n blocks holding the first 16 codes of each block (block order)
 *          and then the last 16 codes of each;
 *   scales [rows][cols/32] fp32 at byte offset rows*cols.
 * Matrices and the output are device memory; every call is asynchronous on
 * `stream` (hipStream_t as void*, NULL = the null stream).  cols must be a
 * multiple of 32; W 16-byte aligned; block_q8 and fp32 arrays 4-byte
 * aligned (16-byte aligned activations are copied in wider pieces).
 */

/* Bytes of a tiled rows x cols matrix (0 for a bad shape). */
size_t tq_hip_q8_matrix_bytes(int rows, int cols);
/* The reference's block_q8 rows (pack_matrix output, packer/packer.c:77-89,
 * already on the device) -> tiled; and back (as unpack_matrix reads them,
 * :91-103, the block_q8 bytes are restored exactly). */
int tq_hip_q8_pack(void *dst, const block_q8 *src, int rows, int cols, void *stream);
int tq_hip_q8_unpack(block_q8 *dst, const void *src, int rows, int cols, void *stream);

/* y[r] = sum over blocks of (int dot of codes) * w.d * x.d: the Q8 MatmulFn
 * (kernel/kernel.h:13, kernel/q8_scalar.c:15-22, kernel/q8_avx2.c:18-25). */
int tq_hip_matmul_q8(const void *W, const block_q8 *xq, float *y, int rows, int cols, void *stream);
/* n_tok activation rows xq[t*cols/32 ...] -> y[t*rows + r]: the Q8
 * MatmulBatchFn (kernel/kernel.h:17-20, kernel/q8_scalar.c:25-30,
 * kernel/avx2_util.h:26-66). */
int tq_hip_matmul_q8_batch(const void *W, const block_q8 *xq, float *y, int rows, int cols,
                           int n_tok, void *stream);

/* project_qkv for n_tok rows of xn [n_tok][hidden] (model/attention_layer.c:38-46,
 * batched :213-218): quantize_row_q8 of every row into xq_ws (n_tok*hidden/32
 * block_q8, the reference's xn_q8 / ws->xq), then q = wq.xq, k = wk.xq,
 * v = wv.xq in one launch over the concatenated rows; q [n_tok][q_rows],
 * k and v [n_tok][kv_rows].  wq is q_rows x hidden, wk and wv kv_rows x hidden. */
int tq_hip_project_qkv(const void *wq, const void *wk, const void *wv, int q_rows, int kv_rows,
                       int hidden, const float *xn, int n_tok, block_q8 *xq_ws, float *q, float *k,
                       float *v, void *stream);
/* project_output (model/attention_layer.c:161-167, batched :238-241):
 * quantize_row_q8 of attn [n_tok][cols] into xq_ws, then out = wo.xq,
 * out [n_tok][rows]. */
int tq_hip_project_output(const void *wo, int rows, int cols, const float *attn, int n_tok,
                          block_q8 *xq_ws, float *out, void *stream);

/* ---- Q4 weight matrices (packer/packer.h:9, kernel/q4_scalar.c,
 * kernel/q4_avx2.c) --------------------------------------------------------
 *
 * The "tiled Q4" layout, the same byte count as the reference's rows x
 * cols/32 block_q4 array (packer/packer.c:63-75):
 *   codes  [rows][cols/2]: each block's 16 nibble bytes exactly as block_q4.q
 *          holds them (code j + 8 in the low nibble of byte j, code j + 24 in
 *          the high nibble), blocks in row order;
 *   scales [rows][cols/32] fp32 at byte offset rows*cols/2.
 * The matmuls take the same block_q8 activations as the Q8 ones and compute
 * each block's exact int32 dot sum_j (nibble_j - 8) * x_j, then
 * ((float)s * w.d) * x.d (kernel/q4_scalar.c:3-15). */

/* The matrix format of a weight struct (tq_format, kernel/kernel.h:6-9). */
#define TQ_HIP_FORMAT_Q8 0
#define TQ_HIP_FORMAT_Q4 1

/* Bytes of a tiled Q4 rows x cols matrix (0 for a bad shape). */
size_t tq_hip_q4_matrix_bytes(int rows, int cols);
/* The reference's block_q4 rows (pack_matrix with bit_type '4',
 * packer/packer.c:40-52,77-89, on the device) -> tiled Q4; and back. */
int tq_hip_q4_pack(void *dst, const block_q4 *src, int rows, int cols, void *stream);
int tq_hip_q4_unpack(block_q4 *dst, const void *src, int rows, int cols, void *stream);
/* The Q4 MatmulFn / MatmulBatchFn (kernel/q4_scalar.c:17-32,
 * kernel/q4_avx2.c:27-36). */
int tq_hip_matmul_q4(const void *W, const block_q8 *xq, float *y, int rows, int cols, void *stream);
int tq_hip_matmul_q4_batch(const void *W, const block_q8 *xq, float *y, int rows, int cols,
                           int n_tok, void *stream);
/* tq_hip_project_qkv / tq_hip_project_output with tiled Q4 matrices. */
int tq_hip_project_qkv_q4(const void *wq, const void *wk, const void *wv, int q_rows, int kv_rows,
                          int hidden, const float *xn, int n_tok, block_q8 *xq_ws, float *q, float *k,
                          float *v, void *stream);
int tq_hip_project_output_q4(const void *wo, int rows, int cols, const float *attn, int n_tok,
                             block_q8 *xq_ws, float *out, void *stream);

/* ---- the rest of the block: MLP, residual norm, embedding, sampler ------- */

/* tq_mlp_weights (model/model_ops.h:29-31) with device pointers: wgate and wup
 * inter x hidden, wdown hidden x inter, all tiled Q8 (tq_hip_q8_pack) or, with
 * format TQ_HIP_FORMAT_Q4, all tiled Q4 (tq_hip_q4_pack). */
typedef struct {
    const void *wgate;
    const void *wup;
    const void *wdown;
    int hidden;
    int inter;
    int format;              /* TQ_HIP_FORMAT_Q8 (0) or TQ_HIP_FORMAT_Q4 */
} tq_hip_mlp_weights;

/* Device workspace bytes for tq_hip_mlp_layer_async over n rows (gate, up and
 * the quantized rows), or 0 for a bad shape. */
size_t tq_hip_mlp_ws_bytes(const tq_hip_mlp_weights *w, int n);
/* mlp_layer / mlp_layer_batch (model/mlp.c:3-43) for n rows of d_xn
 * [n][hidden] into d_out [n][hidden]: quantize_row_q8, the gate and up
 * matmuls in one launch, silu_mul (model/silu.c:6-18, device expf) fused with
 * the quantization of the hidden rows, the down matmul.  d_ws 16-byte aligned. */
int tq_hip_mlp_layer_async(const tq_hip_mlp_weights *w, int n, const float *d_xn, float *d_out, void *d_ws,
                           size_t ws_bytes, void *stream);

/* The residual add and RMSNorm of model/context.c:80-102 for n_rows rows of n:
 * x += y (model/vec.c:3-6; y may be NULL), then xn = rmsnorm(x, weight)
 * (model/rmsnorm.c:4-19) with the sum of squares taken in parallel (within
 * fp32 rounding of the reference's serial sum; the per-head norms in front
 * of the cache keep the serial order, tq_hip_rmsnorm_rows). */
int tq_hip_add_rmsnorm(float *x, const float *y, const float *weight, float *xn, int n_rows, int n, float eps,
                       void *stream);

/* embed_lookup, Q8 (model/embedding.c:4-17): row `token` of a tiled Q8
 * rows x cols matrix, dequantized into out[cols].  TQ_HIP_EINVAL for a token
 * outside [0, rows), as the reference returns -1. */
int tq_hip_embed_lookup_q8(const void *embed, int rows, int cols, int token, float *out, void *stream);
/* The embed_lookup loop of tq_forward_batch (model/context.c:184-187) for n
 * tokens held on the device: row i of out[n][cols] <- row d_tokens[i].  The
 * caller checks the tokens (the reference returns -1 for one outside [0,
 * rows)); the kernel writes zeros for such a row rather than read outside the
 * matrix.  n at most 65535. */
int tq_hip_embed_lookup_q8_batch(const void *embed, int rows, int cols, const int32_t *d_tokens, int n, float *out,
                                 void *stream);
/* The same for a tiled Q4 matrix (model/embedding.c:20-27: d * (nibble - 8)). */
int tq_hip_embed_lookup_q4(const void *embed, int rows, int cols, int token, float *out, void *stream);
int tq_hip_embed_lookup_q4_batch(const void *embed, int rows, int cols, const int32_t *d_tokens, int n, float *out,
                                 void *stream);

/* sample_greedy (model/sampler.c:3-13): the first index of the largest of n
 * logits (strict >, so NaN never wins and ties keep the lower index), written
 * to out[0] on the device. */
int tq_hip_sample_greedy(const float *logits, int n, int32_t *out, void *stream);

/* ---- the whole attention layer on the device --------------------------- */

/* tq_attn_weights (model/model_ops.h:27-37) with device pointers: the four
 * projection matrices in the tiled Q8 layout (tq_hip_q8_pack; tiled Q4 with
 * format TQ_HIP_FORMAT_Q4) and the
 * head_dim RMSNorm weights of q and k (16-byte aligned). */
typedef struct {
    const void *wq;          /* n_q_heads*head_dim x hidden   */
    const void *wk;          /* n_kv_heads*head_dim x hidden  */
    const void *wv;          /* n_kv_heads*head_dim x hidden  */
    const void *wo;          /* hidden x n_q_heads*head_dim   */
    const float *q_norm;
    const float *k_norm;
    int hidden;
    float rms_eps;
    int format;              /* TQ_HIP_FORMAT_Q8 (0) or TQ_HIP_FORMAT_Q4: the four matrices */
} tq_hip_attn_weights;

/* Device workspace bytes tq_hip_attention_layer_async needs for n_q tokens
 * (q, k, v and attention rows plus the quantized activations, the reference's
 * tq_batch_ws), or 0 for a bad shape. */
size_t tq_hip_attention_layer_ws_bytes(const tq_hip_kv *kv, const tq_hip_attn_weights *w, int n_q);

/* attention_layer (model/attention_layer.c:169-194) for n_q decode tokens,
 * each of sequence d_seq[i] (NULL: sequence i) at position d_pos[i] <= max_pos,
 * in three launches on `stream`: project_qkv over the n_q rows of d_xn
 * [n_q][hidden]; RMSNorm + RoPE (d_cos/d_sin [n_q][head_dim/2], or NULL) +
 * append + attend (tq_hip_decode_step_norm_async); project_output into
 * d_out [n_q][hidden].  d_ws: tq_hip_attention_layer_ws_bytes bytes, 16-byte
 * aligned.  Each token is the next token of its own sequence (batched
 * decode); with n_q = 1 this is attention_layer.  Several consecutive tokens
 * of one sequence are attention_layer_batch's work (prefill), not this call's. */
int tq_hip_attention_layer_async(tq_hip_kv *kv, const tq_hip_attn_weights *w, int n_q,
                                 const int32_t *d_seq, const int32_t *d_pos, int max_pos,
                                 const float *d_xn, const float *d_cos, const float *d_sin,
                                 float *d_out, void *d_ws, size_t ws_bytes, void *stream);

/* attention_layer_batch (model/attention_layer.c:200-243) for tokens
 * pos0..pos0+n-1 of sequence `seq`, all on the device: project_qkv over the n
 * rows of d_xn [n][hidden] (the MFMA GEMM from 16 rows on), the per-head
 * RMSNorm of q and k (tq_hip_rmsnorm_rows), RoPE + KV append + causal
 * attention (tq_hip_prefill_async; d_cos/d_sin [n][head_dim/2] or NULL),
 * project_output into d_out [n][hidden].  Where the prefill runs its dense
 * kernel, the q/k norm happens in its staging launch and, for a GEMM output
 * projection, the attention rows are quantized in its store (the same bytes;
 * the workspace then holds no fp32 attention rows).  d_ws: tq_hip_attention_layer_ws_bytes
 * bytes for n tokens, 16-byte aligned.  Returns -1 (TQ_HIP_EINVAL) for n <= 0
 * or a range past the sequence's pages before any launch, as
 * attention_layer_batch does (:203-204). */
int tq_hip_attention_layer_batch_async(tq_hip_kv *kv, const tq_hip_attn_weights *w, int seq, int pos0,
                                       int n, const float *d_xn, const float *d_cos, const float *d_sin,
                                       float *d_out, void *d_ws, size_t ws_bytes, void *stream);

/* ---- measurement: streaming-read bandwidth of device memory, the GPU
 * counterpart of the reference's host RAM probe (tools/membw.h:1-80).  Reads
 * `bytes` (a multiple of 16) of `buf` once with 16-byte loads; `sink` (device,
 * tq_hip_membw_sink_bytes() bytes) is written only if the XOR of the data
 * equals `never`.  Asynchronous on `stream`; the caller times it. */
size_t tq_hip_membw_sink_bytes(void);
int tq_hip_membw_read(const void *buf, size_t bytes, void *sink, unsigned int never, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TQ_HIP_H */
