// tq_common.hpp — shared device helpers and launch interfaces of libtqhip.so.
//
// Exactness rules (the quantized KV codes and scales must equal the
// reference's quantize_row_q8 bit for bit, kernel/quant_x.c:12-33):
//   * every helper that reproduces a reference expression disables FP
//   contraction for its body, so a*b+c stays a rounded multiply followed by a
//   rounded add, as on the reference's x86 build without -mfma;
//   * fp32 division uses hipcc's default correctly rounded division (no
//   fast-math anywhere in this library).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/tq/tq_hip.h"

namespace tq {

constexpr int kQK = 32;           // values per block
constexpr int kBlockBytes = 36;   // sizeof(block_q8)
constexpr int kPage = TQ_HIP_PAGE_TOKENS;
constexpr int kThreads = 256;     // work-group size of the attention kernels

// 16-byte vector as a native clang vector, which stays in registers where
// HIP's struct-wrapped uint4 can end up in scratch.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Cross-lane moves with DPP (a VALU modifier, a few cycles) instead of
// ds_bpermute (an LDS-pipe round trip).  Control words of the gfx9 DPP:
//   quad_perm [a,b,c,d] = a | b<<2 | c<<4 | d<<6;  row_shl:k = 0x100 + k;
//   row_mirror = 0x140 (lane i <- 15-i);  row_half_mirror = 0x141 (i <- 7-i).
constexpr int kDppQuadXor1 = 0xB1;   // [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float lane_f(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Max / sum over each row of 16 lanes, result in every lane of the row.
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f<kDppQuadXor1>(x));
    x = fmaxf(x, dpp_f<kDppQuadXor2>(x));
    x = fmaxf(x, dpp_f<kDppRowHalfMirror>(x));
    return fmaxf(x, dpp_f<kDppRowMirror>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f<kDppQuadXor1>(x);
    x += dpp_f<kDppQuadXor2>(x);
    x += dpp_f<kDppRowHalfMirror>(x);
    return x + dpp_f<kDppRowMirror>(x);
}
// Over the whole wave (64 lanes); the result is uniform.
__device__ __forceinline__ float wave_max(float x) {
    x = row16_max(x);
    return fmaxf(fmaxf(lane_f(x, 0), lane_f(x, 16)), fmaxf(lane_f(x, 32), lane_f(x, 48)));
}
__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    return (lane_f(x, 0) + lane_f(x, 16)) + (lane_f(x, 32) + lane_f(x, 48));
}

// ---------------------------------------------------------------------------
// Quantization of one 32-value block spread one value per lane over 32
// consecutive lanes of a wave (lanes 0-31 or 32-63).

// max(0, |x_j|) over the 32 lanes with the reference's strict "val > max"
// update (kernel/quant_x.c:18-22): NaN never wins, -0 counts as 0.  Only
// non-NaN values >= +0 enter the reduction and max is exact, so any
// reduction order gives the serial scan's value.
__device__ __forceinline__ float block_amax32(float x) {
    const float a = x < 0.0f ? -x : x;
    float m = a > 0.0f ? a : 0.0f;
    m = row16_max(m);
    const float lo = fmaxf(lane_f(m, 0), lane_f(m, 16));
    const float hi = fmaxf(lane_f(m, 32), lane_f(m, 48));
    return (threadIdx.x & 32) ? hi : lo;
}

// scale = amax / 127, inverse = 1/scale or 0 for an all-zero block
// (kernel/quant_x.c:24-27); both divisions correctly rounded.
__device__ __forceinline__ float quant_scale(float amax) { return amax / 127.0f; }
__device__ __forceinline__ float quant_inverse(float d) { return d != 0.0f ? 1.0f / d : 0.0f; }

// Code of x: x*inverse rounded to nearest, ties to even, by adding 1.5*2^23 so
// the fp32 add rounds, and reading the integer back out of the low mantissa
// bits; the low byte of that difference is the code (kernel/quant_x.c:5-10,31).
__device__ __forceinline__ uint32_t quant_code(float x, float inv) {
#pragma clang fp contract(off)
    const float scaled = x * inv;
    const float shifted = scaled + 12582912.0f;
    return (__float_as_uint(shifted) - 0x4B400000u) & 0xFFu;
}

// Gather the 32 codes of a block into dwords: lane j (j % 4 == 0 within the
// 32-lane group) gets codes j..j+3 little-endian, ready for a 4-byte store at
// block offset 4 + j.
__device__ __forceinline__ uint32_t pack_codes4(uint32_t code) {
    const uint32_t c1 = dpp_u<0x55>(code);  // quad_perm [1,1,1,1]
    const uint32_t c2 = dpp_u<0xAA>(code);  // quad_perm [2,2,2,2]
    const uint32_t c3 = dpp_u<0xFF>(code);  // quad_perm [3,3,3,3]
    return code | (c1 << 8) | (c2 << 16) | (c3 << 24);
}

// Quantize the block owned by this lane's 32-lane group and store it at
// `blk` (a 36-byte block_q8 in global or shared memory).
__device__ __forceinline__ void quantize_store32(float x, unsigned char *blk) {
    const int lane = threadIdx.x & 31;
    const float d = quant_scale(block_amax32(x));
    const uint32_t code = quant_code(x, quant_inverse(d));
    const uint32_t word = pack_codes4(code);
    if (lane == 0) *reinterpret_cast<float *>(blk) = d;
    if ((lane & 3) == 0) *reinterpret_cast<uint32_t *>(blk + 4 + lane) = word;
}

// Quantize a 32-value block held 4 values per lane over an aligned group of 8
// lanes (half a DPP row) and store its scale and this lane's 4 codes
// (quantize_row_q8, kernel/quant_x.c:12-33).  The absmax keeps the strict
// "val > max" scan's value as block_amax32 does: |x| with NaN and -0 mapped
// to 0, then an exact max in any order.
__device__ __forceinline__ void quantize8x4(const float (&x)[4], float *d_out, unsigned char *codes, bool leader) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = x[i] < 0.0f ? -x[i] : x[i];
        m = fmaxf(m, a > 0.0f ? a : 0.0f);
    }
    m = fmaxf(m, dpp_f<kDppQuadXor1>(m));
    m = fmaxf(m, dpp_f<kDppQuadXor2>(m));
    m = fmaxf(m, dpp_f<kDppRowHalfMirror>(m));
    const float d = quant_scale(m);
    const float inv = quant_inverse(d);
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) w |= quant_code(x[i], inv) << (8 * i);
    if (leader) *d_out = d;
    *reinterpret_cast<uint32_t *>(codes) = w;
}

// h = silu(g) * u with silu(x) = x * (1 / (1 + expf(-x))) (model/silu.c:6-18,
// model/mlp.c:12-13), evaluated left to right with no contraction: every
// kernel that forms the MLP's hidden rows uses this one definition.
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
    const float sig = 1.0f / (1.0f + expf(-g));
    return g * sig * u;
}

// ---------------------------------------------------------------------------
// RoPE, rotate-half pairing i <-> i + hd/2 (model/rope.c:14-22):
//   lower half: x0*c - x1*s      upper half: x0*s + x1*c
// with x0 = x[i], x1 = x[i + hd/2], c/s from the host table.
__device__ __forceinline__ float rope_lower(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    return x0 * c - x1 * s;
}
__device__ __forceinline__ float rope_upper(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    return x0 * s + x1 * c;
}

// Element e of a head after RoPE (cos_t == nullptr: no rotation).
__device__ __forceinline__ float rope_elem(const float *head, int e, int hd, const float *cos_t,
                                           const float *sin_t) {
    if (cos_t == nullptr) return head[e];
    const int half = hd >> 1;
    if (e < half) return rope_lower(head[e], head[e + half], cos_t[e], sin_t[e]);
    const int i = e - half;
    return rope_upper(head[i], head[e], cos_t[i], sin_t[i]);
}

// ---------------------------------------------------------------------------
// Paged cache view.  page[kvh][K|V][16][nb] block_q8.
struct PagedView {
    unsigned char *pool;
    const int32_t *page_table;  // [max_seqs][max_pages]
    int max_seqs;
    int max_pages;
    int n_pages;
    int n_kv_heads;
    int nb;
    size_t page_bytes;  // n_kv_heads * head_run
    size_t head_run;    // 2 * kv_chunk
    size_t kv_chunk;    // 16 * nb * 36
    size_t row_bytes;   // nb * 36
};

// Physical page holding logical page lp of seq, or -1.
__device__ __forceinline__ int phys_page(const PagedView &v, int seq, int lp) {
    if (seq < 0 || seq >= v.max_seqs || lp < 0 || lp >= v.max_pages) return -1;
    const int p = v.page_table[(size_t)seq * v.max_pages + lp];
    return (p >= 0 && p < v.n_pages) ? p : -1;
}

__device__ __forceinline__ unsigned char *head_run_ptr(const PagedView &v, int phys, int kvh) {
    return v.pool + (size_t)phys * v.page_bytes + (size_t)kvh * v.head_run;
}

}  // namespace tq

// ---------------------------------------------------------------------------
// Launchers (host side, implemented in the .hip files, used by shim.hip).

// Arrival counters of the MFMA decode are TQ_DECODE_COUNTER_STRIDE ints apart.
#define TQ_DECODE_COUNTER_STRIDE 64

struct TqDecodeArgs {
    tq::PagedView view;
    const int32_t *seq_of;   // [n_q], or null: query i reads seq_const + seq_stride*i
    const int32_t *len_of;   // [n_q] tokens to attend minus len_plus, or null:
                             // query i attends pos0 + i + 1 tokens
    const float *q;          // [n_q][n_q_heads][hd]
    const float *cos_t;      // [n_q][hd/2] or null
    const float *sin_t;
    const float *k_new;      // step mode: [n_q][n_kv_heads][hd] (pre-RoPE), else null
    const float *v_new;
    const float *q_norm;     // [hd] RMSNorm weights applied to q (and k_norm to the new
    const float *k_norm;     // K) before RoPE, or null: q and k are already normalized
    float rms_eps;
    float *out;              // [n_q][n_q_heads][hd]
    float *partials;         // [n_q][n_kv][n_splits][G*(hd+2)] when n_splits > 1
    int *counters;           // [n_q][n_kv] arrival counters, zero between launches
    int n_q;
    int n_q_heads;
    int n_kv_heads;
    int head_dim;
    int split_tokens;
    int n_splits;
    float scale;
    int seq_const;
    int seq_stride;
    int pos0;
    int len_plus;            // step mode passes positions and 1 here
    int contig_first;        // >= 0: every query reads one sequence whose logical
    int contig_pages;        // page lp < contig_pages is physical contig_first + lp
    // Completion flags for a host that waits on memory instead of the stream
    // (MFMA kernel only), or null: the rows of (query i, kv head h) are stored
    // at system scope and acknowledged, then done[i * n_kv_heads + h] = done_seq.
    unsigned *done;
    unsigned done_seq;
};

hipError_t tq_launch_quantize(const float *x, block_q8 *out, int n, hipStream_t s);
hipError_t tq_launch_rope(float *x, int n_heads, int hd, const float *c, const float *sn,
                          hipStream_t s);
hipError_t tq_launch_scores(const block_q8 *q, int g, const block_q8 *k, int n, int nb,
                            float scale, float *scores, size_t stride, hipStream_t s);
hipError_t tq_launch_accum(const float *w, size_t w_stride, int g, const block_q8 *v, int n,
                           int nb, float *out, size_t out_stride, hipStream_t s);
hipError_t tq_launch_softmax(float *x, int n, int rows, size_t stride, hipStream_t s);
// h = silu(g) * u of n floats (rows of whole blocks), quantized to hq.
hipError_t tq_launch_silu_quant(const float *gate, const float *up, block_q8 *hq, long n, hipStream_t s);
// The same quantizations of rows x cols values into the split layout the
// batched matmul reads, block-major: for block b of row t its codes 0-15 at
// out + ((2b) rows + t) 16 and 16-31 at out + ((2b + 1) rows + t) 16, then
// the fp32 scales at out + rows * cols as [b][t]; cols % 32 == 0, every
// pointer 16-byte aligned.
hipError_t tq_launch_quantize_split(const float *x, unsigned char *out, int rows, int cols, hipStream_t s);
hipError_t tq_launch_silu_quant_split(const float *gate, const float *up, unsigned char *hq, int rows, int cols,
                                      hipStream_t s);

// tq_hip_project_qkv / tq_hip_project_output over tiled Q8 (q4 false) or
// tiled Q4 (q4 true) matrices; TQ_HIP_* codes.
// part / part_floats: room for split-K partials (tq_gemm_partial_floats),
// or null: a few tokens then take GEMV launches or the unsplit GEMM.
int tq_project_qkv_fmt(bool q4, const void *wq, const void *wk, const void *wv, int q_rows, int kv_rows, int hidden,
                       const float *xn, int n_tok, block_q8 *xq_ws, float *q, float *k, float *v, void *stream,
                       float *part = nullptr, size_t part_floats = 0);
int tq_project_output_fmt(bool q4, const void *wo, int rows, int cols, const float *attn, int n_tok,
                          block_q8 *xq_ws, float *out, void *stream, float *part = nullptr, size_t part_floats = 0);
// Whether tq_project_output_fmt over n_tok rows (with this workspace and
// partials) quantizes its input into the split layout for a GEMM; then
// tq_project_output_xs runs the same projection from rows a producer already
// left in that layout at xq_ws.
bool tq_project_output_takes_xs(bool q4, const void *wo, int rows, int cols, int n_tok, const void *xq_ws,
                                float *part, size_t part_floats);
int tq_project_output_xs(bool q4, const void *wo, int rows, int cols, const void *xq_ws, int n_tok, float *out,
                         void *stream, float *part, size_t part_floats);
// Partial floats the split-K GEMM of a rows x cols matrix needs for up to n_cap tokens.
size_t tq_gemm_partial_floats(int rows, int cols, int n_cap);
// In place allowed (out == x); n <= 8191.
hipError_t tq_launch_rmsnorm_rows(const float *x, const float *w, float *out, int n_rows, int n, float eps,
                                  hipStream_t s);
// seq null: every row goes to seq_const; pos null: row r goes to pos0 + r.
// done non-null: each (row, kv head) work-group raises done[row * n_kv + kvh] =
// done_seq at system scope once its inputs are read and its stores acknowledged.
hipError_t tq_launch_append(const tq::PagedView &view, int n_rows, const int32_t *seq,
                            const int32_t *pos, int seq_const, int pos0, const float *k,
                            const float *v, const float *c, const float *sn, int hd,
                            hipStream_t s, unsigned *done = nullptr, unsigned done_seq = 0);
// Tokens per sub-chunk of the decode kernel for a head_dim.
int tq_decode_tsub(int head_dim);
// Upper bounds of n_splits (for a head_dim and group size) and of
// split_tokens that the decode kernel handles.
int tq_decode_max_splits(int head_dim, int group);
int tq_decode_max_split_tokens();
bool tq_decode_supported(int head_dim, int group);
hipError_t tq_launch_decode(const TqDecodeArgs &a, hipStream_t s);
// The MFMA decode kernel (decode3.hip): head_dim 32/64/128, groups 1..8;
// split_tokens a multiple of 32, at most tq_decode3_max_splits() splits of at
// most tq_decode3_max_split_tokens() tokens.
bool tq_decode3_supported(int head_dim, int group);
int tq_decode3_max_splits();
int tq_decode3_max_split_tokens();
// Floats per split partial row of the MFMA decode (16-byte aligned rows).
int tq_decode3_partial_floats(int head_dim, int group);
// waves: 4 or 8 per work-group; split_tokens a multiple of 32*waves keeps the
// waves' tile counts equal.
hipError_t tq_launch_decode3(const TqDecodeArgs &a, int waves, hipStream_t s);

struct TqPrefillArgs {
    tq::PagedView view;
    int seq;
    int pos0;
    int n;                 // tokens pos0 .. pos0+n-1
    const float *q;        // [n][n_q_heads][hd]
    const float *k_new;    // [n][n_kv_heads][hd] appended by the launch (K pre-RoPE if cos_t),
    const float *v_new;    //   or null: already appended
    const float *cos_t;    // [n][hd/2] or null (q already rotated)
    const float *sin_t;
    float *out;            // [n][n_q_heads][hd]
    int n_q_heads;
    int n_kv_heads;
    int head_dim;
    float scale;
    int contig_first;      // as in TqDecodeArgs
    int contig_pages;
    unsigned char *img;    // tq_prefill_image_bytes() of scratch: the staged key tiles and q blocks
    float *partials;       // split-K partials (tq_prefill_scratch bytes)
    int *counters;         // split-K arrival counters, zero between launches
    // RMSNorm weights [hd] of the q heads and of the new K rows, applied by the
    // staging launch before RoPE (model/attention_layer.c:227-228), or null: q
    // and k_new are already normalized.  k_norm needs k_new.
    const float *q_norm;
    const float *k_norm;
    float rms_eps;
    // Or null: the attention rows go to out as fp32.  Set, they are not stored
    // as fp32; each row's quantize_row_q8 goes here instead, in the split
    // layout tq_launch_quantize_split writes for n rows of n_q_heads * hd
    // values (the batched output projection's input).
    unsigned char *out_xs;
};
// Scratch the prefill of tokens [pos0, pos0+n) needs beyond the image: split-K
// partials (bytes) and arrival counters (ints, zero-initialised by the caller).
void tq_prefill_scratch(int head_dim, int group, int n_kv_heads, int pos0, int n, size_t *partial_bytes,
                        size_t *counter_ints);
// The MFMA causal prefill covers head_dim 64/128, groups 1/2/4/8 and keys
// [0, kend) up to 65536.
bool tq_prefill_mfma_supported(int head_dim, int group, int kend);
size_t tq_prefill_image_bytes(int head_dim, int group, int n_kv_heads, int pos0, int n);
hipError_t tq_launch_prefill(const TqPrefillArgs &a, hipStream_t s);
