// prefill.hip — the causal attention of attention_layer_batch's token loop
// (model/attention_layer.c:221-236) as one dense MFMA contraction.
//
// The reference runs token i as store_kv(pos0+i) then attend(pos0+i), so
// token i sees positions [0, pos0+i].  Here the n new K/V rows are appended
// first (append_kernel, same bytes as store_kv), then every token's attention
// is computed at once with a causal mask: the same keys per token, the same
// quantized operands.  Two kernels follow the append:
//
// prefill_stage_kernel — once per (key tile of 32, kv head) over [0, kend):
//   reads the tile's K and V rows from the paged cache and writes one
//   contiguous tile image laid out as the MFMA operands want them (and, in
//   the same launch, once per (query block, kv head): the block's q rows
//   after RoPE, quantized exactly as quantize_row_q8 does, as int8 codes and
//   fp32 scales in the layout prefill_kernel keeps them in LDS, so every
//   segment of the block copies them instead of re-deriving them):
//     K codes [key half][block][lane][8 bf16]     (A of the score product)
//     K scales [key half][block][lane group][4]   (kd of a lane's four keys)
//     V' hi|lo [column tile][lane][8 bf16]        (A of the P.V product)
//   The int8 K codes are exact in bf16.  V' = code * vd is rounded once to
//   fp32 and split into bf16 hi + lo (hi + lo = x to 2^-18 relative).  Every
//   query block then streams these images instead of re-deriving them.
//
// The attention — per 4 waves, one kv head, 64*NJ
//   (query, head) rows = QB = 64*NJ/G consecutive query tokens x the G heads
//   of the group, in row tiles of 16 queries of one head; wave w owns NJ row
//   tiles.  The block's staged q codes go to registers as bf16 (exact), its
//   scales times scale * log2(e) beside them.
//   Key tiles are copied straight into two LDS buffers (global_load_lds), one
//   tile ahead, one barrier per tile:
//     S^T = sum over blocks b of (kd_b * qd_b) * D_b, D_b = Kcodes_b .
//       qcodes_b^T on v_mfma_f32_16x16x32_bf16: products of integers below
//       2^14, summed 32 at a time, stay below 2^24, so D_b is the exact int32
//       block dot of attn_scores_q8 (model/attn_q8.c:24-30) in any
//       accumulation order; each block's dot is scaled and added in block
//       order (one multiply, one fma per score and block), exp2 domain;
//     online softmax per query with a causal mask; scores are accumulated
//       against the running max, which moves only when a tile exceeds it by
//       more than 2^8: a tile that needs no mask and stays under that for
//       every row of the wave takes a fast path with no cross-lane reduction;
//     O^T += V'^T . P^T on the same bf16 product, P split into hi + lo.
//   The S^T orientation leaves each lane with 8 keys of one query: exactly a
//   B operand of the P.V product (keys permuted identically in A and B), so P
//   never goes through LDS.
//
// Balance: under the causal mask query block b reads b + 1 key tiles.  Two
// attention kernels share the per-tile code:
//
// prefill_block_kernel — with at least two query blocks per CU (the 2048-
//   token prefill: 64 blocks x 8 kv heads), one work-group of 8 waves per
//   (query block, kv head), dealt longest block first, so the CUs pair long
//   blocks with short ones by themselves.  Its two 4-wave halves cover the
//   same 128 rows and split the block's key tiles (half h: tiles h, h+2, ...);
//   half 1 leaves its (o, m, l) in LDS and half 0 merges the two in half
//   order.  Nothing leaves the work-group but the output rows.
// prefill_kernel — with fewer blocks, query blocks are paired last with first
//   (p with nb-1-p), so every pair reads about the same number of tiles, and a
//   pair's tile sequence (the later block's tiles, then the earlier block's)
//   is cut into nsp equal chunks, one 4-wave work-group each.  A block covered
//   by several segments: every segment writes its partial (o, m, l per row)
//   with agent-coherent 16-byte stores, waits for them and arrives on a
//   counter; the last to arrive merges the partials and its own registers in
//   segment order, so the result does not depend on which finished last.  No
//   work-group waits on another.
//
// Grid: one dimension, work-group w serves kv head w % n_kv, so with 8 kv
// heads each XCD (work-groups go round-robin over the 8 XCDs) works on one
// head and keeps that head's tile image in its own L2.
#include <algorithm>

#include "tq_common.hpp"

namespace {

using namespace tq;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

constexpr int kKT = 32;                  // keys per tile
constexpr int kMaxPrefillKeys = 65536;   // keys [0, kend) the dense path serves
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;            // log2 headroom before the running max moves
constexpr int kMaxSplitsP = 8;           // chunks of one query-block pair
constexpr int kItemOverheadTiles = 3;    // prologue + merge of a work item, in tile times
constexpr int kCounterStrideP = 64;      // ints: one 256-byte line per counter
constexpr int kCoherentP = 16;           // cache policy sc1: agent-coherent access

// Layout of one tile image (bytes), shared by both kernels.
template <int HD>
struct TileImg {
    static constexpr int NB = HD / kQK;
    static constexpr int MT = HD / 16;
    static constexpr int ROW = NB * kBlockBytes;
    static constexpr int KC_OFF = 0;                           // [2][NB][64] x 16 B: 8 bf16 codes
    static constexpr int KD_OFF = KC_OFF + 2 * NB * 64 * 16;   // [2][NB][4][4] fp32 scales,
    static constexpr int VH_OFF = KD_OFF + 1024;               //   padded to 1 KB; [MT][64] x 16 B
    static constexpr int VL_OFF = VH_OFF + MT * 64 * 16;
    static constexpr int BYTES = VL_OFF + MT * 64 * 16;
    static constexpr int CHUNKS = BYTES / 16;
    static constexpr int ROUNDS = CHUNKS / kThreads;           // whole rounds of 16-byte copies
    static constexpr int REM = CHUNKS % kThreads;              // copies of the last, partial round
    static_assert(BYTES % 16 == 0 && KD_OFF % 16 == 0 && VH_OFF % 16 == 0, "16-byte chunks");
    static_assert(2 * NB * 16 * 4 <= 1024, "K scales fit their 1 KB");
    static_assert(REM % 64 == 0, "the partial round is whole waves");
};

// Key slot i (0..7) of lane group g in the MFMA k order used for P.V:
// keys 4g..4g+3 then 16+4g..16+4g+3 (the rows a lane holds of S^T).
__device__ __forceinline__ int perm_key(int g, int i) { return i < 4 ? 4 * g + i : 12 + 4 * g + i; }

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    v2bf v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
// bf16 hi | lo parts of four pairs of values.
__device__ __forceinline__ void split_bf16(const float (&x)[8], u32x4 &hi, u32x4 &lo) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t h = bf16_pair(x[2 * i], x[2 * i + 1]);
        hi[i] = h;
        lo[i] = bf16_pair(x[2 * i] - __uint_as_float(h << 16), x[2 * i + 1] - __uint_as_float(h & 0xFFFF0000u));
    }
}

__device__ __forceinline__ v8bf as_v8bf(u32x4 w) { return __builtin_bit_cast(v8bf, w); }

// Max / sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows), the same
// value in all four: permlane32_swap pairs rows (0,2) and (1,3),
// permlane16_swap rows (0,1) and (2,3); VALU only, lower row first in adds.
__device__ __forceinline__ float xrow_max(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xrow_sum(float x) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

typedef __attribute__((address_space(3))) unsigned char lds_u8;

// 16 bytes from each lane's global address into LDS at dst + 16*lane
// (global_load_lds_dwordx4, M0 = LDS byte address, restored after).  Inline
// assembly keeps the compiler from following the copy with a full vmcnt(0)
// wait before every LDS access; the kernel waits for its copies itself.
__device__ __forceinline__ void dma16(const void *src, unsigned char *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8 *)dst;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(lds));
}

// Wait until at most N vector memory operations of this wave are outstanding
// (the copies above are counted in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

struct StageArgs {
    PagedView view;
    int seq;
    int kend;            // keys [0, kend)
    int n_tiles;         // tiles per kv head in the image buffer
    unsigned char *img;  // [n_kv][n_tiles][TileImg::BYTES]
    int contig_first;
    int contig_pages;
    // the q blocks: tokens [pos0, pos0 + n), blocks of QB queries
    int pos0;
    int n;
    int qblocks;
    int n_q_heads;
    const float *q;      // [n][n_q_heads][hd], pre-RoPE if cos_t
    const float *cos_t;  // [n][hd/2] or null
    const float *sin_t;
    unsigned char *qimg; // [n_kv][qblocks][PShape::Q_BYTES]
    // the new K, V rows [n][n_kv][hd] (K pre-RoPE if cos_t), appended here;
    // null: rows [pos0, pos0 + n) are already in the cache
    const float *k_new;
    const float *v_new;
    // RMSNorm weights of q and of the new K rows (applied before RoPE), or null
    const float *q_norm;
    const float *k_norm;
    float rms_eps;
};

// 1 / rms of an hd-value row, as model/rmsnorm.c:4-12 computes it: the
// squares summed serially in element order, then a correctly rounded sqrt and
// divide; eight 16-byte loads in flight at a time.
template <int HD>
__device__ __forceinline__ float row_inv_rms(const float *row, float eps) {
#pragma clang fp contract(off)
    float sum = 0.0f;
    for (int i0 = 0; i0 < HD; i0 += 32) {
        v4f v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = *reinterpret_cast<const v4f *>(row + i0 + 4 * j);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            sum += v[j].x * v[j].x;
            sum += v[j].y * v[j].y;
            sum += v[j].z * v[j].z;
            sum += v[j].w * v[j].w;
        }
    }
    return 1.0f / sqrtf(eps + sum / (float)HD);
}

// (x * inv) * w, rounded as model/rmsnorm.c:14-18 does, on four values.
__device__ __forceinline__ v4f norm4(v4f x, float inv, v4f w) {
#pragma clang fp contract(off)
    return v4f{x.x * inv * w.x, x.y * inv * w.y, x.z * inv * w.z, x.w * inv * w.w};
}

template <int HD, int G, int NJ>
struct PShape {
    using I = TileImg<HD>;
    static constexpr int NB = I::NB;
    static constexpr int RW = 64 * NJ;             // (query, head) rows per work-group
    static constexpr int QB = RW / G;              // query tokens per work-group
    static constexpr int QT = QB / 16;             // query tiles per head
    static constexpr int MT = I::MT;               // output column tiles
    static constexpr int QCS = HD + 8;             // LDS stride of a q code row
    static constexpr int Q_BYTES = RW * QCS + RW * NB * 4;   // staged q: codes | scales
    static_assert(RW % G == 0 && QB % 16 == 0, "whole query tiles");
    static_assert(Q_BYTES <= I::BYTES, "q staging fits one tile buffer");
};

// The q rows of query block blk (QB tokens x the G heads of kv head kvh) after
// RoPE, quantized as quantize_row_q8 does (kernel/quant_x.c:12-33), into the
// block's staged image: codes [RW][QCS] (row r = 16 nt + query, head nt / QT)
// then scales [RW][NB].  Task (row r, c) covers q[4c..4c+3] and its
// rotate-half partner q[HD/2+4c..+3]; every load of the thread's tasks is
// issued before the first is used.  Rows of tokens past n are zero.
template <int HD, int G, int NJ>
__device__ __forceinline__ void stage_q(const StageArgs &a, int kvh, int blk) {
    using S = PShape<HD, G, NJ>;
    constexpr int NB = S::NB;
    constexpr int HALF = HD / 2;
    constexpr int CPR = HD / 8;                      // tasks per row; 8 | CPR
    constexpr int TASKS = S::RW * CPR / kThreads;    // per thread
    static_assert(S::RW * CPR % kThreads == 0, "whole tasks");
    const int tid = threadIdx.x;
    const int i0 = blk * S::QB;
    unsigned char *qc = a.qimg + ((size_t)kvh * a.qblocks + blk) * S::Q_BYTES;
    float *qd = reinterpret_cast<float *>(qc + S::RW * S::QCS);
    constexpr int TB = TASKS > 4 ? 4 : TASKS;       // tasks whose loads are in flight together
    static_assert(TASKS % TB == 0, "whole task batches");
    static_assert(kThreads % CPR == 0, "a thread's tasks share their columns");
    v4f xl[TB], xu[TB], cs[TB], sn[TB];
    auto load_batch = [&](int t0) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const int k = tid + kThreads * (t0 + t);
            const int r = k / CPR, c = k % CPR;
            const int nt = r >> 4;
            const int qi = i0 + (nt % S::QT) * 16 + (r & 15);
            xl[t] = xu[t] = cs[t] = sn[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (qi < a.n) {
                const float *head = a.q + ((size_t)qi * a.n_q_heads + (size_t)kvh * G + nt / S::QT) * HD;
                xl[t] = *reinterpret_cast<const v4f *>(head + 4 * c);
                xu[t] = *reinterpret_cast<const v4f *>(head + HALF + 4 * c);
                if (a.cos_t) {
                    cs[t] = *reinterpret_cast<const v4f *>(a.cos_t + (size_t)qi * HALF + 4 * c);
                    sn[t] = *reinterpret_cast<const v4f *>(a.sin_t + (size_t)qi * HALF + 4 * c);
                }
            }
        }
    };
    // the first batch's loads and this thread's norm weights (every task of a
    // thread has the same columns) are in flight while the norms are taken
    load_batch(0);
    // with q_norm: 1/rms of each of the RW rows, one row per thread
    __shared__ float inv_s[S::RW];
    v4f wlo = v4f{0.0f, 0.0f, 0.0f, 0.0f}, whi = wlo;
    if (a.q_norm) {
        static_assert(S::RW <= kThreads, "one row per thread");
        const int c = tid % CPR;
        wlo = *reinterpret_cast<const v4f *>(a.q_norm + 4 * c);
        whi = *reinterpret_cast<const v4f *>(a.q_norm + HALF + 4 * c);
        if (tid < S::RW) {
            const int r = tid, nt = r >> 4;
            const int qi = i0 + (nt % S::QT) * 16 + (r & 15);
            inv_s[r] = qi < a.n ? row_inv_rms<HD>(a.q + ((size_t)qi * a.n_q_heads + (size_t)kvh * G + nt / S::QT) * HD,
                                                  a.rms_eps)
                                : 0.0f;
        }
        __syncthreads();
    }
#pragma unroll
    for (int t0 = 0; t0 < TASKS; t0 += TB) {
    if (t0 > 0) load_batch(t0);
    if (a.q_norm) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const int k = tid + kThreads * (t0 + t);
            const float inv = inv_s[k / CPR];
            xl[t] = norm4(xl[t], inv, wlo);
            xu[t] = norm4(xu[t], inv, whi);
        }
    }
#pragma unroll
    for (int t = 0; t < TB; t++) {
        const int k = tid + kThreads * (t0 + t);
        const int r = k / CPR, c = k % CPR;
        float lo[4], up[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (a.cos_t) {
                lo[i] = rope_lower(xl[t][i], xu[t][i], cs[t][i], sn[t][i]);
                up[i] = rope_upper(xl[t][i], xu[t][i], cs[t][i], sn[t][i]);
            } else {
                lo[i] = xl[t][i];
                up[i] = xu[t][i];
            }
        }
        const bool leader = (c & 7) == 0;
        quantize8x4(lo, qd + r * NB + c / 8, qc + r * S::QCS + 4 * c, leader);
        quantize8x4(up, qd + r * NB + (HALF + 4 * c) / kQK, qc + r * S::QCS + HALF + 4 * c, leader);
    }
    }
}

// Grid (n_tiles + qblocks, n_kv): x < n_tiles stages key tile x, the rest
// stage q block x - n_tiles.
template <int HD, int G, int NJ>
__global__ __launch_bounds__(kThreads) void prefill_stage_kernel(StageArgs a) {
    if ((int)blockIdx.x >= a.n_tiles) {
        stage_q<HD, G, NJ>(a, blockIdx.y, (int)blockIdx.x - a.n_tiles);
        return;
    }
    using I = TileImg<HD>;
    constexpr int ROW = I::ROW;
    constexpr int RDW = kKT * ROW / 4;   // dwords of one tile's K (or V) rows
    __shared__ __align__(16) uint32_t raw[2][RDW];
    __shared__ int page[2];
    const int tid = threadIdx.x;
    const int kt = blockIdx.x;
    const int kvh = blockIdx.y;
    const PagedView &v = a.view;
    if (tid < 2) {
        const int lp = 2 * kt + tid;
        int p = -1;
        if (lp * kPage < a.kend) {
            if (a.contig_first >= 0 && lp < a.contig_pages)
                p = a.contig_first + lp;
            else
                p = phys_page(v, a.seq, lp);
        }
        page[tid] = p;
    }
    __syncthreads();
    // Rows of the tile: a new row (position in [pos0, kend) on a mapped page,
    // with k_new given) is computed here and appended; an older one is read
    // from the cache; every other row (past the keys, unmapped) is zero so that
    // no stale scale reaches P.V.
    const int t0 = kt * kKT;
    auto fresh = [&](int p, int phys) { return a.k_new && p >= a.pos0 && p < a.kend && phys >= 0; };
    // a page's K (or V) rows are one contiguous run: copy them in CB-byte
    // pieces, whole rows per piece
    constexpr int CB = ROW % 16 == 0 ? 16 : 8;
    constexpr int PR = kPage * ROW / CB;   // pieces per page run
    typedef uint32_t piece_t __attribute__((ext_vector_type(CB / 4)));
    for (int i = tid; i < 2 * 2 * PR; i += kThreads) {
        const int kv = i / (2 * PR), pg = (i / PR) & 1, ch = i % PR;
        const int p = t0 + pg * kPage + (ch * CB) / ROW;
        const int phys = page[pg];
        if (fresh(p, phys)) continue;
        piece_t x = piece_t(0u);
        if (p < a.kend && phys >= 0)
            x = *reinterpret_cast<const piece_t *>(head_run_ptr(v, phys, kvh) + kv * v.kv_chunk + ch * CB);
        *reinterpret_cast<piece_t *>(reinterpret_cast<unsigned char *>(raw[kv]) + pg * kPage * ROW + ch * CB) = x;
    }
    // the new rows: store_kv's Q8 branch (model/attention_layer.c:66-90) with
    // RoPE on K (:188), quantized exactly as quantize_row_q8 into the tile's
    // LDS rows.  Task (row r, K|V, c) covers x[4c..4c+3] and its rotate-half
    // partner x[HD/2+4c..+3]; the 8 lanes of a 32-value block share their row,
    // so a whole block is computed or skipped together.
    const bool has_new = a.k_new && t0 + kKT > a.pos0 && t0 < a.kend;
    // with k_norm: 1/rms of each new K row of the tile, one row per thread;
    // the tasks' own loads below are issued first, so the two overlap
    __shared__ float kinv_s[kKT];
    if (has_new) {
        constexpr int HALF = HD / 2;
        constexpr int CPR = HD / 8;
        constexpr int TPT = kKT * 2 * CPR / kThreads;
        static_assert(kKT * 2 * CPR % kThreads == 0 && CPR % 8 == 0, "whole tasks, whole blocks");
        const bool rot = a.cos_t != nullptr;
        v4f xl[TPT], xu[TPT], cs[TPT], sn[TPT];
        bool mine[TPT];
#pragma unroll
        for (int t = 0; t < TPT; t++) {
            const int task = tid + kThreads * t;
            const int r = task / (2 * CPR), kv = (task / CPR) & 1, c = task % CPR;
            const int p = t0 + r;
            mine[t] = fresh(p, page[r / kPage]);
            xl[t] = xu[t] = cs[t] = sn[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (mine[t]) {
                const size_t row = (size_t)(p - a.pos0);
                const float *src = (kv ? a.v_new : a.k_new) + (row * v.n_kv_heads + kvh) * HD;
                xl[t] = *reinterpret_cast<const v4f *>(src + 4 * c);
                xu[t] = *reinterpret_cast<const v4f *>(src + HALF + 4 * c);
                if (!kv && rot) {
                    cs[t] = *reinterpret_cast<const v4f *>(a.cos_t + row * HALF + 4 * c);
                    sn[t] = *reinterpret_cast<const v4f *>(a.sin_t + row * HALF + 4 * c);
                }
            }
        }
        if (a.k_norm) {
            // every task of a thread has the same columns: its weights once
            const int cw = tid % CPR;
            const v4f wlo = *reinterpret_cast<const v4f *>(a.k_norm + 4 * cw);
            const v4f whi = *reinterpret_cast<const v4f *>(a.k_norm + HALF + 4 * cw);
            if (tid < kKT) {
                const int p = t0 + tid;
                kinv_s[tid] = fresh(p, page[tid / kPage])
                                  ? row_inv_rms<HD>(a.k_new + ((size_t)(p - a.pos0) * v.n_kv_heads + kvh) * HD,
                                                    a.rms_eps)
                                  : 0.0f;
            }
            __syncthreads();
#pragma unroll
            for (int t = 0; t < TPT; t++) {
                const int task = tid + kThreads * t;
                const int r = task / (2 * CPR), kv = (task / CPR) & 1;
                if (mine[t] && !kv) {
                    xl[t] = norm4(xl[t], kinv_s[r], wlo);
                    xu[t] = norm4(xu[t], kinv_s[r], whi);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TPT; t++) {
            if (!mine[t]) continue;
            const int task = tid + kThreads * t;
            const int r = task / (2 * CPR), kv = (task / CPR) & 1, c = task % CPR;
            float lo[4], up[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (!kv && rot) {
                    lo[i] = rope_lower(xl[t][i], xu[t][i], cs[t][i], sn[t][i]);
                    up[i] = rope_upper(xl[t][i], xu[t][i], cs[t][i], sn[t][i]);
                } else {
                    lo[i] = xl[t][i];
                    up[i] = xu[t][i];
                }
            }
            unsigned char *row = reinterpret_cast<unsigned char *>(raw[kv]) + r * ROW;
            const bool leader = (c & 7) == 0;
            const int bl = (4 * c) / kQK, bu = (HALF + 4 * c) / kQK;
            quantize8x4(lo, reinterpret_cast<float *>(row + bl * kBlockBytes),
                        row + bl * kBlockBytes + 4 + (4 * c) % kQK, leader);
            quantize8x4(up, reinterpret_cast<float *>(row + bu * kBlockBytes),
                        row + bu * kBlockBytes + 4 + (4 * c) % kQK, leader);
        }
    }
    __syncthreads();
    if (has_new) {
        // the new rows into the cache, whole rows
        for (int i = tid; i < 2 * 2 * PR; i += kThreads) {
            const int kv = i / (2 * PR), pg = (i / PR) & 1, ch = i % PR;
            const int p = t0 + pg * kPage + (ch * CB) / ROW;
            const int phys = page[pg];
            if (!fresh(p, phys)) continue;
            *reinterpret_cast<piece_t *>(head_run_ptr(v, phys, kvh) + kv * v.kv_chunk + ch * CB) =
                *reinterpret_cast<const piece_t *>(reinterpret_cast<const unsigned char *>(raw[kv]) + pg * kPage * ROW +
                                                   ch * CB);
        }
    }
    const unsigned char *rk = reinterpret_cast<const unsigned char *>(raw[0]);
    const unsigned char *rv = reinterpret_cast<const unsigned char *>(raw[1]);
    unsigned char *out = a.img + ((size_t)a.n_tiles * kvh + kt) * I::BYTES;
    // K codes: entry (mt, b, lane) = key mt*16 + lane%16, block b, codes 8*(lane/16)..+7 as bf16
    for (int e = tid; e < 2 * I::NB * 64; e += kThreads) {
        const int mt = e / (I::NB * 64), b = (e / 64) % I::NB, ln = e % 64;
        const unsigned char *row = rk + (mt * 16 + (ln & 15)) * ROW + b * kBlockBytes + 4 + 8 * (ln >> 4);
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = bf16_pair((float)(int8_t)row[2 * i], (float)(int8_t)row[2 * i + 1]);
        *reinterpret_cast<u32x4 *>(out + I::KC_OFF + e * 16) = w;
    }
    // K scales: entry (mt, b, g, r) = kd of key mt*16 + 4g + r, block b (the
    // four keys a lane of group g holds of the score product)
    for (int e = tid; e < 2 * I::NB * 16; e += kThreads) {
        const int mt = e / (I::NB * 16), b = (e / 16) % I::NB, key = mt * 16 + (e & 15);
        *reinterpret_cast<float *>(out + I::KD_OFF + e * 4) =
            *reinterpret_cast<const float *>(rk + key * ROW + b * kBlockBytes);
    }
    // V' = code * vd: entry (m, lane) = column m*16 + lane%16, keys perm_key(lane/16, 0..7)
    for (int e = tid; e < I::MT * 64; e += kThreads) {
        const int m = e / 64, ln = e % 64;
        const int col = m * 16 + (ln & 15);
        const int blk = col / kQK, cb = col % kQK;
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const unsigned char *row = rv + perm_key(ln >> 4, i) * ROW + blk * kBlockBytes;
            x[i] = (float)(int8_t)row[4 + cb] * *reinterpret_cast<const float *>(row);
        }
        u32x4 hi, lo;
        split_bf16(x, hi, lo);
        *reinterpret_cast<u32x4 *>(out + I::VH_OFF + e * 16) = hi;
        *reinterpret_cast<u32x4 *>(out + I::VL_OFF + e * 16) = lo;
    }
}


struct PrefillArgs {
    int pos0;
    int n;
    int qblocks;         // query blocks of QB tokens
    int nsp;             // chunks per block pair = most segments of one block
    int n_kv;
    float *partials;     // [n_kv][qblocks][nsp][RW][HD + 4]
    int *counters;       // [n_kv][qblocks] x kCounterStrideP
    const unsigned char *qimg;   // [n_kv][qblocks][PShape::Q_BYTES] (prefill_stage_kernel)
    float *out;          // [n][n_q_heads][hd]
    unsigned char *out_xs;   // or, when set, the rows quantized in the split layout
    int n_q_heads;
    float scale;
    int n_tiles;         // tiles per kv head in the image buffer
    const unsigned char *img;
};


// Key tiles query block b reads: keys [0, pos0 + its last query + 1).
__host__ __device__ inline int block_tiles(int pos0, int n, int qb, int b) {
    const int last = (b + 1) * qb < n ? (b + 1) * qb : n;
    return (pos0 + last + kKT - 1) / kKT;
}

// Per-row state of one wave's NJ row tiles over a run of key tiles: o and
// lsum are taken against moff (mrow, or 0 before any key); mrow is the running
// max; thr the largest score - moff a tile may hold without moving the max
// (kLazy; -inf before any key, so the first visible key takes the slow path);
// lsum is this lane's share of the row sum, added over the row's lanes at the
// end.  The same in the row's four lanes.
template <int HD, int G, int NJ>
struct PRows {
    static constexpr int MT = PShape<HD, G, NJ>::MT;
    v4f o[MT][NJ];
    float mrow[NJ], moff[NJ], thr[NJ], lsum[NJ];
    __device__ __forceinline__ void init() {
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int j = 0; j < NJ; j++) o[m][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            mrow[j] = -INFINITY;
            moff[j] = 0.0f;
            thr[j] = -INFINITY;
            lsum[j] = 0.0f;
        }
    }
};

// The score product's B operands of one wave's rows: the q codes of query
// l16, values 32b + 8lg .. +7, as bf16 (exact), qd * scale * log2(e) per
// block, and each row's query position.
template <int HD, int G, int NJ>
struct PQ {
    static constexpr int NB = PShape<HD, G, NJ>::NB;
    v8bf qcb[NJ][NB];
    float qsc[NJ][NB];
    int qpos[NJ];
};

// From the block's staged q image in LDS (codes at qc, scales after them).
template <int HD, int G, int NJ>
__device__ __forceinline__ void load_q(const PrefillArgs &a, const unsigned char *qc, int i0, int wave, int lane,
                                       PQ<HD, G, NJ> &q) {
    using S = PShape<HD, G, NJ>;
    constexpr int NB = S::NB;
    const int l16 = lane & 15, lg = lane >> 4;
    const float *qd = reinterpret_cast<const float *>(qc + S::RW * S::QCS);
    const float qscale = a.scale * kLog2e;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int r = (wave * NJ + j) * 16 + l16;
        const int nt = r >> 4;
        int qi = i0 + (nt % S::QT) * 16 + l16;
        qi = qi < a.n ? qi : a.n - 1;
        q.qpos[j] = a.pos0 + qi;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            q.qsc[j][b] = qd[r * NB + b] * qscale;
            const unsigned char *c = qc + r * S::QCS + b * kQK + 8 * lg;
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = bf16_pair((float)(int8_t)c[2 * i], (float)(int8_t)c[2 * i + 1]);
            q.qcb[j][b] = as_v8bf(w);
        }
    }
}

// The P operands of one tile: P = exp2(S - moff) split into bf16 hi | lo.
template <int NJ>
struct PP {
    u32x4 hi[NJ], lo[NJ];
};

// One key tile kt (image T in LDS) against the wave's rows, first part:
// exact scores, the causal mask, the online softmax (o and lsum rescaled when
// the max moves) and this tile's P.
template <int HD, int G, int NJ>
__device__ __forceinline__ void tile_scores(const PrefillArgs &a, const unsigned char *T, int kt, int i0, int lane,
                                            const PQ<HD, G, NJ> &q, PRows<HD, G, NJ> &st, PP<NJ> &pp) {
    using S = PShape<HD, G, NJ>;
    using I = TileImg<HD>;
    constexpr int NB = S::NB;
    const int lg = lane >> 4;
    // S^T - moff for keys [32kt, 32kt+32) x the wave's queries: per block the
    // exact int32 dot on the matrix cores, then (kd * qd') * dot added in
    // block order onto -moff
    v4f s[2][NJ];
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const v8bf kc = as_v8bf(*reinterpret_cast<const u32x4 *>(T + I::KC_OFF + ((mt * NB + b) * 64 + lane) * 16));
            const v4f kd = *reinterpret_cast<const v4f *>(T + I::KD_OFF + ((mt * NB + b) * 4 + lg) * 16);
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const v4f d =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(kc, q.qcb[j][b], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    s[mt][j][r] = __builtin_fmaf(d[r], kd[r] * q.qsc[j][b], b == 0 ? -st.moff[j] : s[mt][j][r]);
            }
        }
    }

    // fast path: no row's tile max passes its threshold, and the tile needs
    // no causal mask (it ends at or before the block's first query); the lane
    // maxima are taken here, in the block that computes the scores
    auto max8 = [](const v4f &x, const v4f &y) {
        return fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3])));
    };
    const int k0 = kt * kKT;
    const bool diag = k0 + kKT - 1 > a.pos0 + i0;
    bool move = false;
#pragma unroll
    for (int j = 0; j < NJ; j++) move |= max8(s[0][j], s[1][j]) > st.thr[j];
    if (diag || __builtin_amdgcn_ballot_w64(move) != 0) {
        // slow path, for the whole wave: the causal mask, the row max over the
        // four lanes, the lazy move (only by more than kLazy), o and lsum
        // rescaled and the tile re-offset
        if (diag) {
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int kp = k0 + mt * 16 + 4 * lg + r;
                        s[mt][j][r] = kp > q.qpos[j] ? -INFINITY : s[mt][j][r];
                    }
        }
        bool rescale = false;
        float corr[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const float mx = xrow_max(max8(s[0][j], s[1][j])) + st.moff[j];
            const float mnew = mx > st.mrow[j] + kLazy ? mx : st.mrow[j];
            const float onew = mnew == -INFINITY ? 0.0f : mnew;
            // nothing is accumulated while mrow is -inf: corr 0, not exp2 of a difference
            corr[j] = st.mrow[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(st.moff[j] - onew);
            const float delta = st.moff[j] - onew;
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) s[mt][j][r] += delta;
            rescale |= corr[j] != 1.0f;
            st.lsum[j] *= corr[j];
            st.mrow[j] = mnew;
            st.moff[j] = onew;
            st.thr[j] = mnew == -INFINITY ? -INFINITY : kLazy;
        }
        if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
            for (int m = 0; m < S::MT; m++)
#pragma unroll
                for (int j = 0; j < NJ; j++) st.o[m][j] *= corr[j];
        }
    }
    // P = exp2(S - moff) <= 2^kLazy, split into bf16 hi | lo (B operands)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        float p[8];
        float ps = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[mt * 4 + r] = __builtin_amdgcn_exp2f(s[mt][j][r]);
                ps += p[mt * 4 + r];
            }
        st.lsum[j] += ps;
        split_bf16(p, pp.hi[j], pp.lo[j]);
    }
}

// Second part: O^T += V'^T . P^T with the tile's V' (image T) and its P.
template <int HD, int G, int NJ>
__device__ __forceinline__ void tile_pv(const unsigned char *T, int lane, const PP<NJ> &pp, PRows<HD, G, NJ> &st) {
    using S = PShape<HD, G, NJ>;
    using I = TileImg<HD>;
#pragma unroll
    for (int m = 0; m < S::MT; m++) {
        const v8bf ahi = as_v8bf(*reinterpret_cast<const u32x4 *>(T + I::VH_OFF + (m * 64 + lane) * 16));
        const v8bf alo = as_v8bf(*reinterpret_cast<const u32x4 *>(T + I::VL_OFF + (m * 64 + lane) * 16));
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            st.o[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, as_v8bf(pp.hi[j]), st.o[m][j], 0, 0, 0);
            st.o[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, as_v8bf(pp.lo[j]), st.o[m][j], 0, 0, 0);
            st.o[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, as_v8bf(pp.hi[j]), st.o[m][j], 0, 0, 0);
        }
    }
}

// Both parts of one tile.
template <int HD, int G, int NJ>
__device__ __forceinline__ void tile_update(const PrefillArgs &a, const unsigned char *T, int kt, int i0, int lane,
                                            const PQ<HD, G, NJ> &q, PRows<HD, G, NJ> &st) {
    PP<NJ> pp;
    tile_scores<HD, G, NJ>(a, T, kt, i0, lane, q, st, pp);
    tile_pv<HD, G, NJ>(T, lane, pp, st);
}

// Normalise and store the wave's rows: lane holds columns 16m + 4lg .. +3 of
// query l16.  Either fp32 rows into out, or (out_xs) each row quantized as
// quantize_row_q8 straight into the split layout the output GEMM reads.
template <int HD, int G, int NJ>
__device__ __forceinline__ void store_rows(const PrefillArgs &a, int kvh, int i0, int wave, int lane,
                                           const PRows<HD, G, NJ> &st, const float (&lrow)[NJ]) {
    using S = PShape<HD, G, NJ>;
    const int l16 = lane & 15, lg = lane >> 4;
    if (a.out_xs) {
        // block b of a head is columns 32b..32b+31, tiles m = 2b (codes 0-15)
        // and 2b+1 (codes 16-31), 8 values in each of the 4 lanes of the
        // query (lanes l16 + 16 lg); the absmax as quantize8x4 takes it (|x|,
        // NaN and -0 as 0, an exact max), then the same scale, inverse and
        // codes as a separate quantize launch over the stored rows
        const size_t nrows = (size_t)a.n, cols = (size_t)a.n_q_heads * HD;
        float *xd = reinterpret_cast<float *>(a.out_xs + nrows * cols);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const float inv = 1.0f / lrow[j];
            const int nt = wave * NJ + j;
            const int g = nt / S::QT;
            const int qi = i0 + (nt % S::QT) * 16 + l16;
#pragma unroll
            for (int b = 0; b < HD / kQK; b++) {
                const v4f x0 = st.o[2 * b][j] * inv, x1 = st.o[2 * b + 1][j] * inv;
                float m = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float a0 = x0[i] < 0.0f ? -x0[i] : x0[i];
                    const float a1 = x1[i] < 0.0f ? -x1[i] : x1[i];
                    m = fmaxf(m, a0 > 0.0f ? a0 : 0.0f);
                    m = fmaxf(m, a1 > 0.0f ? a1 : 0.0f);
                }
                m = fmaxf(m, __shfl_xor(m, 16));
                m = fmaxf(m, __shfl_xor(m, 32));
                const float d = quant_scale(m);
                const float qinv = quant_inverse(d);
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    w0 |= quant_code(x0[i], qinv) << (8 * i);
                    w1 |= quant_code(x1[i], qinv) << (8 * i);
                }
                if (qi < a.n) {
                    const size_t gb = (size_t)(kvh * G + g) * (HD / kQK) + b;
                    *reinterpret_cast<uint32_t *>(a.out_xs + ((2 * gb) * nrows + qi) * 16 + 4 * lg) = w0;
                    *reinterpret_cast<uint32_t *>(a.out_xs + ((2 * gb + 1) * nrows + qi) * 16 + 4 * lg) = w1;
                    if (lg == 0) xd[gb * nrows + qi] = d;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float inv = 1.0f / lrow[j];
        const int nt = wave * NJ + j;
        const int g = nt / S::QT;
        const int qi = i0 + (nt % S::QT) * 16 + l16;
        if (qi < a.n) {
            float *orow = a.out + ((size_t)qi * a.n_q_heads + (size_t)kvh * G + g) * HD;
#pragma unroll
            for (int m = 0; m < S::MT; m++) *reinterpret_cast<v4f *>(orow + m * 16 + 4 * lg) = st.o[m][j] * inv;
        }
    }
}

// Merge the partial (ms, ls, os) into the running (M, L, acc), in order.
template <int MT>
__device__ __forceinline__ void merge_part(float &M, float &L, v4f (&acc)[MT], float ms, float ls, const v4f (&os)[MT]) {
    const float Mn = fmaxf(M, ms);
    const float fo = __builtin_amdgcn_exp2f(M - Mn);   // 0 while M is -inf
    const float fs = __builtin_amdgcn_exp2f(ms - Mn);  // 0 for a partial with no key
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = acc[m] * fo + os[m] * fs;
    L = L * fo + ls * fs;
    M = Mn;
}

// Copy of key tile kt of img into an LDS buffer by the 256 threads of one
// 4-wave group (thread t's copy r is chunk t + 256 r; the partial last round:
// the first REM threads, whole waves).
template <int HD>
__device__ __forceinline__ void fetch_tile(const unsigned char *img, int kt, unsigned char *buf, int gtid, int gwave) {
    using I = TileImg<HD>;
    const unsigned char *src = img + (size_t)kt * I::BYTES;
    const int wu = __builtin_amdgcn_readfirstlane(gwave);
#pragma unroll
    for (int r = 0; r < I::ROUNDS; r++) dma16(src + 16 * (gtid + kThreads * r), buf + 16 * (kThreads * r + 64 * wu));
    if (I::REM > 0 && 64 * wu < I::REM)
        dma16(src + 16 * (gtid + kThreads * I::ROUNDS), buf + 16 * (kThreads * I::ROUNDS + 64 * wu));
}
// Copies of one tile a wave of the group issues.
template <int HD>
__device__ __forceinline__ bool tile_has_rem(int gwave) {
    using I = TileImg<HD>;
    return I::REM > 0 && 64 * gwave < I::REM;
}

// One segment: query block blk against key tiles [kt_begin, kt_end), the
// segment sp of the nsp that cover the block (4-wave work-group).
template <int HD, int G, int NJ>
__device__ __forceinline__ void prefill_segment(const PrefillArgs &a, int kvh, int blk, int kt_begin, int kt_end,
                                                int sp, int nsp, unsigned char *tile0, unsigned char *tile1) {
    using S = PShape<HD, G, NJ>;
    using I = TileImg<HD>;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l16 = lane & 15;
    const int lg = lane >> 4;
    const int i0 = blk * S::QB;
    const unsigned char *img = a.img + (size_t)kvh * a.n_tiles * I::BYTES;

    // ---- the block's staged q rows (prefill_stage_kernel) into tile1, then
    //      the first key tile into tile0; waiting for all but this wave's
    //      copies of the tile leaves only the tile in flight
    {
        constexpr int QCH = S::Q_BYTES / 16;
        const unsigned char *src = a.qimg + ((size_t)kvh * a.qblocks + blk) * S::Q_BYTES;
        const int wu = __builtin_amdgcn_readfirstlane(wave);
        for (int c0 = 64 * wu; c0 < QCH; c0 += kThreads)
            if (c0 + lane < QCH) dma16(src + 16 * (c0 + lane), tile1 + 16 * c0);
    }
    fetch_tile<HD>(img, kt_begin, tile0, tid, wave);
    if (tile_has_rem<HD>(wave))
        wait_vm<I::ROUNDS + 1>();
    else
        wait_vm<I::ROUNDS>();
    __syncthreads();

    PQ<HD, G, NJ> q;
    load_q<HD, G, NJ>(a, tile1, i0, wave, lane, q);
    PRows<HD, G, NJ> st;
    st.init();

    // ---- the key loop: two LDS buffers, one tile ahead, one barrier per tile
    for (int kt = kt_begin; kt < kt_end; kt++) {
        const bool odd = (kt - kt_begin) & 1;
        unsigned char *T = odd ? tile1 : tile0;
        // this thread's copies of tile kt have landed; the barrier makes every
        // thread's visible and frees the other buffer (tile kt-1, or the q
        // staging) for the next copy
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();
        if (kt + 1 < kt_end) fetch_tile<HD>(img, kt + 1, odd ? tile0 : tile1, tid, wave);
        tile_update<HD, G, NJ>(a, T, kt, i0, lane, q, st);
    }

    float lrow[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) lrow[j] = xrow_sum(st.lsum[j]);
    if (nsp == 1) {
        store_rows<HD, G, NJ>(a, kvh, i0, wave, lane, st, lrow);
        return;
    }

    // ---- split: every segment writes its partial rows [RW][HD + 4] (o
    //      unnormalised, m, l) with agent-coherent stores, waits for them,
    //      then arrives; the last to arrive merges all of them in segment
    //      order (its own from registers) and puts the counter back to 0.
    //      Nothing waits on another work-group.
    constexpr int PS = HD + 4;
    const size_t pblock = ((size_t)kvh * a.qblocks + blk) * a.nsp;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(a.partials + pblock * S::RW * PS, 0, nsp * S::RW * PS * 4, 0x00020000);
    int *counter = a.counters + ((size_t)kvh * a.qblocks + blk) * kCounterStrideP;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int r = (wave * NJ + j) * 16 + l16;
        const int base = (sp * S::RW + r) * PS;
#pragma unroll
        for (int m = 0; m < S::MT; m++)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, st.o[m][j]), prs,
                                                   (base + m * 16 + 4 * lg) * 4, 0, kCoherentP);
        if (lg == 0) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(st.mrow[j]), prs, (base + HD) * 4, 0, kCoherentP);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lrow[j]), prs, (base + HD + 1) * 4, 0, kCoherentP);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // this thread's partial is at the point of coherence
    int *flag = reinterpret_cast<int *>(tile0);
    __syncthreads();                 // every thread's partial; every wave done with the tile buffers
    if (tid == 0) *flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsp - 1;
    __syncthreads();
    if (!*flag) return;
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int r = (wave * NJ + j) * 16 + l16;
        float M = -INFINITY, L = 0.0f;
        v4f acc[S::MT];
#pragma unroll
        for (int m = 0; m < S::MT; m++) acc[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        for (int s2 = 0; s2 < nsp; s2++) {
            const int base = (s2 * S::RW + r) * PS;
            float ms, ls;
            v4f os[S::MT];
            if (s2 == sp) {
                ms = st.mrow[j];
                ls = lrow[j];
#pragma unroll
                for (int m = 0; m < S::MT; m++) os[m] = st.o[m][j];
            } else {
                ms = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(prs, (base + HD) * 4, 0, kCoherentP));
                ls = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(prs, (base + HD + 1) * 4, 0, kCoherentP));
#pragma unroll
                for (int m = 0; m < S::MT; m++)
                    os[m] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                        prs, (base + m * 16 + 4 * lg) * 4, 0, kCoherentP));
            }
            merge_part<S::MT>(M, L, acc, ms, ls, os);
        }
#pragma unroll
        for (int m = 0; m < S::MT; m++) st.o[m][j] = acc[m];
        lrow[j] = L;
    }
    store_rows<HD, G, NJ>(a, kvh, i0, wave, lane, st, lrow);
}

template <int HD, int G, int NJ>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(PrefillArgs a) {
    using I = TileImg<HD>;
    using S = PShape<HD, G, NJ>;
    __shared__ __attribute__((aligned(16))) unsigned char tile0[I::BYTES];
    __shared__ __attribute__((aligned(16))) unsigned char tile1[I::BYTES];
    const int kvh = (int)blockIdx.x % a.n_kv;
    const int item = (int)blockIdx.x / a.n_kv;
    const int p = item / a.nsp, c = item % a.nsp;
    // pair p: the later block bh, then the earlier bl (none for the middle block)
    const int bh = a.qblocks - 1 - p, bl = p;
    const int th = block_tiles(a.pos0, a.n, S::QB, bh);
    const int tp = th + (bl < bh ? block_tiles(a.pos0, a.n, S::QB, bl) : 0);
    const int C = (tp + a.nsp - 1) / a.nsp;             // tiles per chunk
    const int c0 = c * C, c1 = min(tp, c0 + C);          // this chunk of the pair's sequence
    if (c0 < min(c1, th))
        prefill_segment<HD, G, NJ>(a, kvh, bh, c0, min(c1, th), c, (th + C - 1) / C, tile0, tile1);
    if (c1 > max(c0, th)) {
        __syncthreads();   // the LDS buffers are free again
        prefill_segment<HD, G, NJ>(a, kvh, bl, max(c0, th) - th, c1 - th, c - th / C, (tp + C - 1) / C - th / C,
                                   tile0, tile1);
    }
}

// Whole query blocks: one work-group of 8 waves per (query block, kv head),
// longest block first.  The two 4-wave halves cover the same 128 rows and
// split the block's key tiles, half h taking tiles h, h + 2, h + 4, ...; they
// step together (one barrier per pair of tiles, each half with its own two
// LDS buffers, one tile ahead), then half 1 leaves its (o, m, l) in LDS and
// half 0 merges the two in half order and stores the rows.  No partial leaves
// the work-group and no work-group waits on another.
template <int HD, int G, int NJ>
__global__ __launch_bounds__(2 * kThreads, 1) void prefill_block_kernel(PrefillArgs a) {
    using S = PShape<HD, G, NJ>;
    using I = TileImg<HD>;
    constexpr int MT = S::MT;
    // tile buffers: half 0 uses 0, 1; half 1 uses 2, 3
    __shared__ __attribute__((aligned(16))) unsigned char tiles[4][I::BYTES];
    static_assert(4 * 64 * (MT * NJ * 16 + NJ * 8) <= 4 * I::BYTES, "half 1's rows fit the tile buffers");
    const int kvh = (int)blockIdx.x % a.n_kv;
    const int blk = a.qblocks - 1 - (int)blockIdx.x / a.n_kv;
    const int tid = threadIdx.x;
    const int half = __builtin_amdgcn_readfirstlane(tid >> 8);
    const int htid = tid & (kThreads - 1);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);   // wave within the half
    const int i0 = blk * S::QB;
    const unsigned char *img = a.img + (size_t)kvh * a.n_tiles * I::BYTES;
    const int nt = block_tiles(a.pos0, a.n, S::QB, blk);
    const int mine = (nt - half + 1) / 2;   // tiles of this half
    const int steps = (nt + 1) / 2;         // half 0 has the most

    // buffer of this half's step s
    auto buf = [&](int st_) -> unsigned char * { return tiles[2 * half + (st_ & 1)]; };
    // ---- the block's staged q rows into buffer 1 (half 0's second; all 8
    //      waves copy), then each half's first tile into its first buffer;
    //      waiting for all but this wave's copies of its tile leaves only the
    //      tile in flight
    {
        constexpr int QCH = S::Q_BYTES / 16;
        const unsigned char *src = a.qimg + ((size_t)kvh * a.qblocks + blk) * S::Q_BYTES;
        const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);
        for (int c0 = 64 * wu; c0 < QCH; c0 += 2 * kThreads)
            if (c0 + lane < QCH) dma16(src + 16 * (c0 + lane), tiles[1] + 16 * c0);
    }
    if (mine > 0) {
        fetch_tile<HD>(img, half, buf(0), htid, wave);
        if (tile_has_rem<HD>(wave))
            wait_vm<I::ROUNDS + 1>();
        else
            wait_vm<I::ROUNDS>();
    } else {
        wait_vm<0>();
    }
    __syncthreads();

    PQ<HD, G, NJ> q;
    load_q<HD, G, NJ>(a, tiles[1], i0, wave, lane, q);
    PRows<HD, G, NJ> st;
    st.init();

    // Both halves step together, one barrier per step, each tile's scores
    // and P.V in its step.  (Running half 1 one part behind, so that each
    // SIMD's two waves would meet matrix products with vector work, measured
    // slower: 256 registers, and no overlap gained.)
    for (int s = 0; s < steps; s++) {
        // this thread's copies of its half's tile have landed; the barrier
        // makes every thread's visible and frees the other buffers (the
        // previous step's tiles, or the q staging) for the next copies
        asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
        __syncthreads();
        if (s + 1 < mine) fetch_tile<HD>(img, 2 * (s + 1) + half, buf(s + 1), htid, wave);
        if (s < mine) tile_update<HD, G, NJ>(a, buf(s), 2 * s + half, i0, lane, q, st);
    }

    float lrow[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) lrow[j] = xrow_sum(st.lsum[j]);
    // half 1's rows, lane by lane (the waves of both halves hold the same
    // rows and columns in the same lanes), into the free tile buffers
    v4f *ob = reinterpret_cast<v4f *>(&tiles[0][0]);              // [wave][MT][NJ][64]
    float *mb = reinterpret_cast<float *>(ob + 4 * MT * NJ * 64);  // [wave][NJ][64] x (m, l)
    __syncthreads();   // every wave is done with the tile buffers
    if (half == 1) {
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int j = 0; j < NJ; j++) ob[((wave * MT + m) * NJ + j) * 64 + lane] = st.o[m][j];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            mb[((wave * NJ + j) * 64 + lane) * 2] = st.mrow[j];
            mb[((wave * NJ + j) * 64 + lane) * 2 + 1] = lrow[j];
        }
    }
    __syncthreads();
    if (half == 1) return;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        float M = -INFINITY, L = 0.0f;
        v4f acc[MT], os[MT];
#pragma unroll
        for (int m = 0; m < MT; m++) {
            acc[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            os[m] = st.o[m][j];
        }
        merge_part<MT>(M, L, acc, st.mrow[j], lrow[j], os);
#pragma unroll
        for (int m = 0; m < MT; m++) os[m] = ob[((wave * MT + m) * NJ + j) * 64 + lane];
        merge_part<MT>(M, L, acc, mb[((wave * NJ + j) * 64 + lane) * 2], mb[((wave * NJ + j) * 64 + lane) * 2 + 1], os);
#pragma unroll
        for (int m = 0; m < MT; m++) st.o[m][j] = acc[m];
        lrow[j] = L;
    }
    store_rows<HD, G, NJ>(a, kvh, i0, wave, lane, st, lrow);
}

// Rows per work-group: 128 (two row tiles per wave) by default;
// TQ_HIP_PREFILL_ROWS=64 selects one row tile per wave where G allows.
int prefill_rows(int g) {
    static int forced = [] {
        const char *s = getenv("TQ_HIP_PREFILL_ROWS");
        return s ? atoi(s) : 0;
    }();
    if (g == 8) return 128;
    return forced == 64 ? 64 : 128;
}

// Query tokens per work-group for a shape (the kernel's QB).
int prefill_qb(int g) { return 64 * (prefill_rows(g) == 128 ? 2 : 1) / g; }

// With at least two query blocks per CU, every (query block, kv head) is one
// work-group of prefill_block_kernel (no partials): dealt longest first, the
// blocks pair up on the CUs by themselves.  With fewer, query blocks are
// paired last with first and cut into nsp chunks, the count that minimises
// the time of the item waves (items of ceil(tp/nsp) tiles each,
// kItemOverheadTiles extra, resident work-groups at once per wave), run by
// prefill_kernel with split partials.
constexpr int kCUs = 256;                // compute units of an MI355X
// TQ_HIP_PREFILL_WHOLE=1|0 forces the whole-block kernel or the paired split
// one (tests of both at any size); read on every call.  -1: the plan decides.
int prefill_whole_env() {
    const char *s = getenv("TQ_HIP_PREFILL_WHOLE");
    return (s && *s) ? (s[0] == '1' ? 1 : 0) : -1;
}
struct PrefillPlan {
    int qblocks, nsp, rows, items;
    bool whole;                          // prefill_block_kernel
};
PrefillPlan plan_prefill(int hd, int g, int n_kv_heads, int pos0, int n) {
    PrefillPlan p;
    const int qb = prefill_qb(g);
    p.rows = 64 * (prefill_rows(g) == 128 ? 2 : 1);
    p.qblocks = (n + qb - 1) / qb;
    const int forced = prefill_whole_env();
    p.whole = forced >= 0 ? forced == 1 : (long)p.qblocks * n_kv_heads >= 2L * kCUs;
    if (p.whole) {
        p.nsp = 1;
        p.items = p.qblocks;
        return p;
    }
    const int pairs = (p.qblocks + 1) / 2;
    int tp_max = 0;
    for (int q = 0; q < pairs; q++) {
        const int bh = p.qblocks - 1 - q;
        const int tp = block_tiles(pos0, n, qb, bh) + (q < bh ? block_tiles(pos0, n, qb, q) : 0);
        tp_max = std::max(tp_max, tp);
    }
    const long slots = 256L * (hd == 128 ? 2 : 4);   // resident work-groups: 2 or 4 per CU
    long best = -1;
    p.nsp = 1;
    for (int k = 1; k <= kMaxSplitsP; k++) {
        const int C = (tp_max + k - 1) / k;
        if (k > 1 && C < 4) break;
        const long waves = ((long)pairs * k * n_kv_heads + slots - 1) / slots;
        const long cost = waves * (C + kItemOverheadTiles);
        if (best < 0 || cost < best) {
            best = cost;
            p.nsp = k;
        }
    }
    p.items = pairs * p.nsp;
    return p;
}

// Byte offset of the staged q blocks in the image buffer (after the key
// tiles, 256-byte aligned).
size_t qimg_offset(int head_dim, int n_kv_heads, int kend) {
    const size_t tiles = (size_t)(kend + kKT - 1) / kKT;
    const size_t per = head_dim == 64 ? TileImg<64>::BYTES : TileImg<128>::BYTES;
    return (tiles * per * (size_t)n_kv_heads + 255) & ~(size_t)255;
}

// The staging launch (key tiles and q blocks), then the attention.
template <int HD, int G, int NJ>
hipError_t launch_hd_g(const TqPrefillArgs &t, const PrefillArgs &a, bool whole, hipStream_t s) {
    StageArgs st;
    st.view = t.view;
    st.seq = t.seq;
    st.kend = t.pos0 + t.n;
    st.n_tiles = a.n_tiles;
    st.img = t.img;
    st.contig_first = t.contig_first;
    st.contig_pages = t.contig_pages;
    st.pos0 = t.pos0;
    st.n = t.n;
    st.qblocks = a.qblocks;
    st.n_q_heads = t.n_q_heads;
    st.q = t.q;
    st.cos_t = t.cos_t;
    st.sin_t = t.sin_t;
    st.qimg = const_cast<unsigned char *>(a.qimg);
    st.k_new = t.k_new;
    st.v_new = t.v_new;
    st.q_norm = t.q_norm;
    st.k_norm = t.k_norm;
    st.rms_eps = t.rms_eps;
    hipLaunchKernelGGL((prefill_stage_kernel<HD, G, NJ>), dim3(a.n_tiles + a.qblocks, t.n_kv_heads), dim3(kThreads),
                       0, s, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (whole) {
        hipLaunchKernelGGL((prefill_block_kernel<HD, G, NJ>), dim3(a.qblocks * t.n_kv_heads), dim3(2 * kThreads), 0,
                           s, a);
    } else {
        const int items = (a.qblocks + 1) / 2 * a.nsp;
        hipLaunchKernelGGL((prefill_kernel<HD, G, NJ>), dim3(items * t.n_kv_heads), dim3(kThreads), 0, s, a);
    }
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const TqPrefillArgs &t, const PrefillArgs &a, int g, bool whole, hipStream_t s) {
    const bool wide = prefill_rows(g) == 128;
    switch (g) {
        case 1: return wide ? launch_hd_g<HD, 1, 2>(t, a, whole, s) : launch_hd_g<HD, 1, 1>(t, a, whole, s);
        case 2: return wide ? launch_hd_g<HD, 2, 2>(t, a, whole, s) : launch_hd_g<HD, 2, 1>(t, a, whole, s);
        case 4: return wide ? launch_hd_g<HD, 4, 2>(t, a, whole, s) : launch_hd_g<HD, 4, 1>(t, a, whole, s);
        case 8: return launch_hd_g<HD, 8, 2>(t, a, whole, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool tq_prefill_mfma_supported(int head_dim, int group, int kend) {
    const bool hd_ok = head_dim == 64 || head_dim == 128;
    const bool g_ok = group == 1 || group == 2 || group == 4 || group == 8;
    return hd_ok && g_ok && kend > 0 && kend <= kMaxPrefillKeys;
}

void tq_prefill_scratch(int head_dim, int group, int n_kv_heads, int pos0, int n, size_t *partial_bytes,
                        size_t *counter_ints) {
    const PrefillPlan p = plan_prefill(head_dim, group, n_kv_heads, pos0, n);
    if (p.whole || p.nsp == 1) {
        *partial_bytes = 0;
        *counter_ints = 0;
        return;
    }
    *partial_bytes = (size_t)n_kv_heads * p.qblocks * p.nsp * p.rows * (head_dim + 4) * sizeof(float);
    *counter_ints = (size_t)n_kv_heads * p.qblocks * kCounterStrideP;
}

size_t tq_prefill_image_bytes(int head_dim, int group, int n_kv_heads, int pos0, int n) {
    const PrefillPlan p = plan_prefill(head_dim, group, n_kv_heads, pos0, n);
    const size_t qrow = head_dim == 64 ? PShape<64, 1, 1>::QCS + 2 * 4 : PShape<128, 1, 1>::QCS + 4 * 4;
    return qimg_offset(head_dim, n_kv_heads, pos0 + n) + (size_t)n_kv_heads * p.qblocks * p.rows * qrow;
}

hipError_t tq_launch_prefill(const TqPrefillArgs &t, hipStream_t s) {
    const int g = t.n_q_heads / t.n_kv_heads;
    if (!tq_prefill_mfma_supported(t.head_dim, g, t.pos0 + t.n) || !t.img) return hipErrorInvalidValue;
    PrefillArgs a;
    a.pos0 = t.pos0;
    a.n = t.n;
    a.out = t.out;
    a.out_xs = t.out_xs;
    a.n_q_heads = t.n_q_heads;
    a.scale = t.scale;
    a.n_tiles = (t.pos0 + t.n + kKT - 1) / kKT;
    a.img = t.img;
    a.qimg = t.img + qimg_offset(t.head_dim, t.n_kv_heads, t.pos0 + t.n);
    const PrefillPlan p = plan_prefill(t.head_dim, g, t.n_kv_heads, t.pos0, t.n);
    a.qblocks = p.qblocks;
    a.nsp = p.nsp;
    a.n_kv = t.n_kv_heads;
    a.partials = t.partials;
    a.counters = t.counters;
    if (p.nsp > 1 && (!t.partials || !t.counters)) return hipErrorInvalidValue;
    return t.head_dim == 64 ? launch_hd<64>(t, a, g, p.whole, s) : launch_hd<128>(t, a, g, p.whole, s);
}
