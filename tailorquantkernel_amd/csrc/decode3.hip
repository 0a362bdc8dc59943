// decode3.hip — attend_q8 (model/attention_layer.c:125-150) on the paged cache,
// with both contractions on the matrix cores.
//
// Grid (split, kv head, query); a work-group of W waves (4, or 8 for short
// splits) owns the tokens [split*split_tokens, +split_tokens) of one kv head
// and all G query heads that read it, so every K/V byte is fetched once per
// step.  The range is cut into tiles of 32 keys (two pages); wave w takes tiles
// w, w+W, w+2W, ... and runs its own online softmax over them, so the key loop
// has no barrier at all.  Each wave quantizes the group's q rows itself, from
// its own staged copy, straight into the lanes of its score operand.
// Tiles are copied straight from HBM into the wave's LDS slots by
// global_load_lds_dwordx4 (no staging registers), two tiles ahead, then:
//
//   scores  S[key][(h,b)] on v_mfma_i32_16x16x32_i8.  The N columns of the
//           product are the (query head h, block b) pairs of the group and the
//           K dimension one 32-value block: the product for block b' has the q
//           codes of block b' in the columns with b == b' and zeros elsewhere,
//           so accumulating the NB products leaves the exact int32 block dot
//           sum_j q[h][b][j]*k[key][b][j] in column (h,b), every lane useful at
//           G*NB = 16.  Each lane scales its dots by qd*kd (qd pre-multiplied
//           by the softmax scale and log2 e) and the NB lanes of a head add
//           them with two DPP butterflies: the score of attn_scores_q8_scalar
//           (model/attn_q8.c:17-34) up to fp32 rounding order, in the exp2
//           domain.
//   softmax online, per lane, exp2 domain, the scores taken against the
//           running max, which moves only when a tile exceeds it by more
//           than 2^8 (p <= 256 in between).  A tile with no key past the
//           split's end and no lane over that threshold takes a fast path:
//           no cross-lane work at all.  Otherwise the max over the four
//           16-lane rows holding the tile's keys comes from permlane32/16
//           swaps and the accumulators are rescaled when it moves.  Each lane
//           keeps its own share of the row sum; the rows are added once, at
//           the end.
//   P.V     O[col][(h,b)] += V[key][col] * W[key][(h,b)] on
//           v_mfma_f32_16x16x32_bf16, K = 32 keys.  W = p * vd (the weight of
//           attn_accum_q8's ws = wt * vb[b].d, model/attn_q8.c:48) lies in
//           exactly the lanes and key order the score product left it in, split
//           into bf16 hi + lo (exact to 2^-18 relative); the int8 V codes are
//           exact in bf16, so hi.V + lo.V in fp32 carries W's precision.
//           Column (h,b) of the output is kept for the columns of block b.
//
// The W waves merge (m, l, o) through LDS in wave order.  With several
// splits each work-group writes its partial (o, m, l) with 16-byte stores at
// agent coherence (sc1: through to the point all XCDs share) and bumps an
// arrival counter; the last one merges the partials in split order, so results
// do not depend on arrival order.
//
// Step mode (k_new != null): the work-group owning position len-1 quantizes the
// new token's K (after RoPE) and V exactly as store_kv does, writes them to the
// cache and patches them into the staged tile: append + attend in one launch.
//
// With q_norm (and k_norm in step mode) the q rows and the new K row are the
// projections' raw outputs: each wave first takes every head's RMSNorm
// (model/rmsnorm.c:4-19, norm_heads at model/attention_layer.c:48-53,183-184)
// in the reference's order — one lane per head sums the squares serially —
// and applies (x * inverse) * weight before RoPE, so the K codes stay
// bit-exact with the whole attention_layer.
#include "tq_common.hpp"

namespace {

using namespace tq;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

constexpr int kTK = 32;                  // keys per tile
constexpr int kMaxSplits3 = 64;
constexpr int kMaxSplitPages3 = 512;     // page ids a work-group stages (8,192 tokens)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;            // log2 headroom before the running max moves
constexpr int kCoherent = 16;            // cache policy sc1: agent-coherent access
constexpr int kSystem = 17;              // sc0 sc1: written through to memory, acknowledged at system scope
constexpr int kBufWord3 = 0x00020000;    // raw buffer descriptor, 32-bit data
constexpr int kCounterStride = TQ_DECODE_COUNTER_STRIDE;   // ints: one 256-byte line per counter
constexpr int kSortQ = 128;              // ragged batches up to this many queries go longest first

template <int HD, int G>
struct L3 {
    static constexpr int NB = HD / kQK;
    static constexpr int ROW = NB * kBlockBytes;        // bytes per token row
    static constexpr int NCOL = G * NB;                 // (head, block) columns
    static constexpr int NT = (NCOL + 15) / 16;         // 16-column tiles of them
    static constexpr int CT = HD / 16;                  // 16-column tiles of the output
    static constexpr int TILE = 2 * kTK * ROW;          // K rows | V rows
    static constexpr int RUN = kPage * ROW;             // bytes of one page's K (or V) run
    static constexpr int RUN_FULL = RUN / 1024;         // whole-wave 16-byte copies per run
    static constexpr int RUN_TAIL = RUN % 1024 / 16;    // lanes of the run's last, partial copy
    static constexpr int CPL = 4 * (RUN_FULL + (RUN_TAIL > 0));   // copies per tile
    static constexpr int U = G * HD / 4;                // float4 units of a head group's output
    static constexpr int PSTRIDE = (G * (HD + 2) + 3) / 4 * 4;   // floats per partial row
    static constexpr int MERGE = G * (HD + 2) * 4;      // one wave's share of the merge
    static_assert(NB == 1 || NB == 2 || NB == 4, "a head's blocks share one DPP quad");
    static_assert(16 % NB == 0, "column tiles hold whole heads");
    static_assert(kTK * ROW % 16 == 0 && RUN % 16 == 0, "16-byte chunks");
    static_assert(TILE == 4 * RUN, "a tile is four page runs");
    static_assert(MERGE <= TILE, "the merge reuses the tile slots");
    static_assert(U % 1 == 0 && HD % 4 == 0, "float4 units");
};

template <int HD, int G>
struct Smem3 {
    using L = L3<HD, G>;
    unsigned char newrow[2 * L::ROW];        // step mode: the new token's K, V
    int pages[kMaxSplitPages3];              // physical page of each page of the split
    int qlen[kSortQ];                        // the batch's lengths and sequences, for the
    int qseq[kSortQ];                        // longest-first order
    int qsel;
    float wts[G * kMaxSplits3];              // combine weights
    int last;
};

__device__ __forceinline__ long lds_ld8(const unsigned char *p) {
    const uint32_t lo = *reinterpret_cast<const uint32_t *>(p);
    const uint32_t hi = *reinterpret_cast<const uint32_t *>(p + 4);
    return (long)(((unsigned long)hi << 32) | lo);
}
__device__ __forceinline__ float lds_f(const unsigned char *p) { return *reinterpret_cast<const float *>(p); }

// Key held in slot i (0..7) of lane group g: the rows 4g..4g+3 of the two
// 16-key halves of the tile, as the score product leaves them.
__device__ __forceinline__ int slot_key(int g, int i) { return 16 * (i >> 2) + 4 * g + (i & 3); }

// Sum over the NB lanes (h, 0..NB-1) of a head, (x0 + x1) + (x2 + x3): the
// same value in each of them (fp32 add commutes).
template <int NB>
__device__ __forceinline__ float head_block_sum(float x) {
    if constexpr (NB >= 2) x += dpp_f<kDppQuadXor1>(x);
    if constexpr (NB == 4) x += dpp_f<kDppQuadXor2>(x);
    return x;
}

// Max / sum over lanes l, l^16, l^32, l^48 (the four 16-lane rows), the same
// value in all four: permlane32_swap pairs rows (0,2) and (1,3),
// permlane16_swap rows (0,1) and (2,3); lower row first in every add.
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

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    v2bf v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
// x = hi + lo with hi = bf16(x), lo = bf16(x - hi), four pairs.
__device__ __forceinline__ void split_bf16(const float (&x)[8], v8bf &hi, v8bf &lo) {
    u32x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w = bf16_pair(x[2 * i], x[2 * i + 1]);
        h[i] = w;
        l[i] = bf16_pair(x[2 * i] - __uint_as_float(w << 16), x[2 * i + 1] - __uint_as_float(w & 0xFFFF0000u));
    }
    hi = __builtin_bit_cast(v8bf, h);
    lo = __builtin_bit_cast(v8bf, l);
}

typedef __attribute__((address_space(3))) unsigned char lds_u8;

// 16 bytes from each lane's global address into LDS at dst + 16*lane
// (global_load_lds_dwordx4; M0 holds the LDS byte address and is restored).
// Issued as inline assembly so that the compiler does not follow every such
// copy with a full vmcnt(0) wait before LDS accesses: the kernel waits for
// exactly the copies it needs (wait_copies), counting them in issue order.
// No memory clobber: LDS reads of a slot are ordered before a refill by
// wait_lds() (a compiler barrier plus lgkmcnt(0)) and after its copies by
// wait_copies(); leaving memory unclobbered keeps the uniform loads that
// precede the copies scalar.
__device__ __forceinline__ void dma16(const void *src, unsigned char *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8 *)dst;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(lds));
}
// The same copy from a scalar base address plus each lane's 32-bit offset
// (the saddr form): a uniform base costs no vector address arithmetic.
__device__ __forceinline__ void dma16s(const unsigned char *base, uint32_t off, unsigned char *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8 *)dst;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
        "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds));
}
// 4 bytes per lane, the same way (into LDS at dst + 4*lane).
__device__ __forceinline__ void dma4s(const unsigned char *base, uint32_t off, unsigned char *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8 *)dst;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
        "global_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds));
}
// Wait until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_copies() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
// Every LDS access issued so far has completed (before a copy may land on
// memory those accesses touch).
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory"); }

// RMSNorm's last step, out = (x * inverse) * weight, rounded as
// model/rmsnorm.c:17 rounds it.
__device__ __forceinline__ float norm1(float x, float inv, float w) {
#pragma clang fp contract(off)
    return x * inv * w;
}
__device__ __forceinline__ void norm8(float (&x)[8], float inv, const float *w) {
    float ww[8];
    *reinterpret_cast<v4f *>(&ww[0]) = *reinterpret_cast<const v4f *>(w);
    *reinterpret_cast<v4f *>(&ww[4]) = *reinterpret_cast<const v4f *>(w + 4);
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = norm1(x[i], inv, ww[i]);
}

// W waves per work-group (4, or 8 when each wave has only a tile or two).
template <int HD, int G, int W>
__global__ __launch_bounds__(64 * W) void decode3_kernel(TqDecodeArgs a) {
    using L = L3<HD, G>;
    constexpr int kWaves = W;
    constexpr int kThreads = 64 * W;
    constexpr int NB = L::NB, ROW = L::ROW, NT = L::NT, CT = L::CT, CPL = L::CPL;
    __shared__ __align__(16) Smem3<HD, G> sm;
    // two tile slots per wave, separate objects so the wait for one slot's
    // copies does not wait for the other's
    __shared__ __align__(16) unsigned char slot0[kWaves][L::TILE];
    __shared__ __align__(16) unsigned char slot1[kWaves][L::TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lg = lane >> 4, l16 = lane & 15;
    const int split = blockIdx.x, kvh = blockIdx.y;
    // The query this work-group serves.  A ragged batch goes longest first:
    // grid z is the rank of the query's length (ties by index), so the
    // work-groups of the longest sequences are dispatched first and the
    // short ones fill the gaps at the end (longest-processing-time order).
    // Each query's result does not depend on the order.
    int qi = blockIdx.z;
    // (the query's raw length and sequence, when the ranking below reads them)
    bool ranked = false;
    int len_rk = 0, seq_rk = 0;
    if (a.n_q > 1) {
        if (!a.len_of) {
            qi = a.n_q - 1 - (int)blockIdx.z;   // query i attends pos0 + i + 1 keys
        } else if (a.n_q <= kSortQ) {
            // the batch's lengths (and sequences) through LDS, ranked by one
            // thread per query; the chosen query's length and sequence are
            // then read from LDS, not loaded again
            // both loads issued before either is waited for (a missing
            // sequence array reads the lengths again and stores 0)
            for (int i = tid; i < a.n_q; i += kThreads) {
                const int li = a.len_of[i];
                const int si = (a.seq_of ? a.seq_of : a.len_of)[i];
                sm.qlen[i] = li;
                sm.qseq[i] = a.seq_of ? si : 0;
            }
            __syncthreads();
            for (int i = tid; i < a.n_q; i += kThreads) {
                const int li = sm.qlen[i];
                int r = 0;
                for (int u = 0; u < a.n_q; u++) {
                    const int lu = sm.qlen[u];
                    r += (lu > li) || (lu == li && u < i);
                }
                if (r == (int)blockIdx.z) sm.qsel = i;
            }
            __syncthreads();
            qi = sm.qsel;
            ranked = true;
        }
    }
    qi = __builtin_amdgcn_readfirstlane(qi);
    if (ranked) {
        len_rk = __builtin_amdgcn_readfirstlane(sm.qlen[qi]);
        seq_rk = __builtin_amdgcn_readfirstlane(sm.qseq[qi]);
    }
    const int t_begin = split * a.split_tokens;
    const int split_end = t_begin + a.split_tokens;
    const PagedView &view = a.view;
    const bool contig = a.contig_first >= 0;
    const bool rot = a.cos_t != nullptr;
    const bool step = a.k_new != nullptr;
    unsigned char *tb0 = slot0[wave];
    unsigned char *tb1 = slot1[wave];
    // Uniform inputs: issued first as unconditional scalar loads (a dummy
    // address when absent), used only after the copies below are issued, so
    // the copies do not wait for them.
    const int len_raw = ranked ? len_rk : *(a.len_of ? a.len_of + qi : reinterpret_cast<const int32_t *>(a.q));
    const int seq_raw = ranked ? seq_rk : *(a.seq_of ? a.seq_of + qi : reinterpret_cast<const int32_t *>(a.q));

    // ---- 1. this wave's copy of the inputs it quantizes, into the tail-free
    //      front of its second slot: q rows of the group | cos | sin | new K | new V
    //      (fp32).  These copies go first so that waiting for them lets every
    //      later K/V copy stay in flight.
    const bool nrm = a.q_norm != nullptr;
    float *stq = reinterpret_cast<float *>(tb1);
    float *stc = stq + G * HD;
    float *sts = stc + HD / 2;
    float *stk = sts + HD / 2;
    float *stv = stk + HD;
    float *stqn = stv + HD;          // RMSNorm weights of q | of k
    float *stkn = stqn + HD;
    float *stinv = stkn + HD;        // 1/rms of the G q heads, then of the new K row
    static_assert((G + 5) * HD * 4 + 4 * (G + 1) <= L::TILE, "staged inputs fit the slot");
    {
        // 16-byte chunks per part; the cos/sin slots are always there (without
        // RoPE they repeat q) so every part sits at a fixed offset; with the
        // norm weights the K and V slots are too (without a step they repeat q)
        constexpr int QC = G * HD / 4, RC = HD / 8, NC = HD / 4;
        const int nch = QC + 2 * RC + (nrm ? 4 * NC : (step ? 2 * NC : 0));
        const float *qg = a.q + ((size_t)qi * a.n_q_heads + (size_t)kvh * G) * HD;
        const size_t nrow = ((size_t)qi * a.n_kv_heads + kvh) * HD;
        for (int c0 = 0; c0 < nch; c0 += 64) {
            const int c = c0 + lane;
            const float *src = qg;
            if (c < QC) {
                src = qg + 4 * c;
            } else if (c < QC + 2 * RC) {
                const int r = c - QC;
                if (rot) src = (r < RC ? a.cos_t : a.sin_t) + (size_t)qi * (HD / 2) + 4 * (r < RC ? r : r - RC);
            } else if (c < QC + 2 * RC + 2 * NC) {
                const int r = c - QC - 2 * RC;
                if (step) src = (r < NC ? a.k_new : a.v_new) + nrow + 4 * (r < NC ? r : r - NC);
            } else if (c < nch) {
                const int r = c - QC - 2 * RC - 2 * NC;
                src = r < NC ? a.q_norm + 4 * r : (step ? a.k_norm : a.q_norm) + 4 * (r - NC);
            }
            if (c0 + 64 <= nch || c < nch) dma16(src, tb1 + 16 * c0);
        }
    }

    // Each lane's byte offset inside a page run for each copy of the run.
    // (a 256-byte tail goes as one whole-wave 4-byte copy)
    constexpr bool kTail4 = L::RUN_TAIL == 16;
    uint32_t roff[L::RUN_FULL + 1];
#pragma unroll
    for (int j = 0; j <= L::RUN_FULL; j++) roff[j] = (uint32_t)(1024 * j + (kTail4 && j == L::RUN_FULL ? 4 : 16) * lane);
    const unsigned char *head0 = view.pool + (size_t)kvh * view.head_run;
    int load_end;   // keys below this are mapped; pages past it are not fetched

    // Physical page of logical page lp of this sequence, or -1.
    auto page_of = [&](int lp) -> int {
        if (contig) return lp < a.contig_pages ? a.contig_first + lp : -1;
        return sm.pages[min(max(lp - t_begin / kPage, 0), kMaxSplitPages3 - 1)];
    };
    // Copy the tile with keys [k0, k0+32) into an LDS slot (CPL copies): the
    // image [K page 0 | K page 1 | V page 0 | V page 1] is four contiguous
    // page runs, each copied from its own scalar base (RUN_FULL whole-wave
    // copies and one of RUN_TAIL lanes).  A page that is unmapped (or past
    // load_end) is read from physical page 0 instead: those keys are masked out.
    auto fetch = [&](unsigned char *dst, int k0) {
        int p0 = page_of(k0 / kPage), p1 = page_of(k0 / kPage + 1);
        p0 = __builtin_amdgcn_readfirstlane((p0 >= 0 && k0 < load_end) ? p0 : 0);
        p1 = __builtin_amdgcn_readfirstlane((p1 >= 0 && k0 + kPage < load_end) ? p1 : 0);
        const unsigned char *b0 = head0 + (size_t)p0 * view.page_bytes;
        const unsigned char *b1 = head0 + (size_t)p1 * view.page_bytes;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const unsigned char *base = ((r & 1) ? b1 : b0) + (r >> 1) * view.kv_chunk;
            unsigned char *d = dst + r * L::RUN;
#pragma unroll
            for (int j = 0; j < L::RUN_FULL; j++) dma16s(base, roff[j], d + 1024 * j);
            if constexpr (kTail4) {
                dma4s(base, roff[L::RUN_FULL], d + 1024 * L::RUN_FULL);
            } else if constexpr (L::RUN_TAIL > 0) {
                if (lane < L::RUN_TAIL) dma16s(base, roff[L::RUN_FULL], d + 1024 * L::RUN_FULL);
            }
        }
    };

    // ---- 2. the first tile (contiguous sequence: before len is known) ----
    const int k_first = t_begin + kTK * wave;
    bool first_issued = false;
    if (contig) {
        load_end = min(split_end, a.contig_pages * kPage);
        if (k_first < load_end) {
            fetch(tb0, k_first);
            first_issued = true;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int len = a.len_of ? len_raw + a.len_plus : a.pos0 + qi + 1;
    const int seq = a.seq_of ? seq_raw : a.seq_const + a.seq_stride * qi;
    int t_end;
    if (contig) {
        if (len <= 0 || t_begin >= len) return;
        t_end = min(len, split_end);
        load_end = min(load_end, t_end);
    } else {
        // paged: the split's page ids through LDS (the only barrier before the merge)
        const int split_pages = a.split_tokens / kPage;
        int page_id[(kMaxSplitPages3 + kThreads - 1) / kThreads];
#pragma unroll
        for (int i = 0; i < (kMaxSplitPages3 + kThreads - 1) / kThreads; i++) {
            const int p = tid + i * kThreads;
            if (p < split_pages) page_id[i] = phys_page(view, seq, t_begin / kPage + p);
        }
        if (len <= 0 || t_begin >= len) return;
#pragma unroll
        for (int i = 0; i < (kMaxSplitPages3 + kThreads - 1) / kThreads; i++) {
            const int p = tid + i * kThreads;
            if (p < split_pages) sm.pages[p] = page_id[i];
        }
        t_end = min(len, split_end);
        load_end = t_end;
        __syncthreads();
        if (k_first < load_end) {
            fetch(tb0, k_first);
            first_issued = true;
        }
    }
    // the staged inputs have landed; the first tile may still be in flight
    if (first_issued)
        wait_copies<CPL>();
    else
        wait_copies<0>();
    if (nrm) {
        // 1/rms of each q head (lanes 0..G-1) and of the new K row (lane G):
        // the squares summed serially in element order, as model/rmsnorm.c:4-12
        if (lane <= G) {
#pragma clang fp contract(off)
            const float *src = lane < G ? stq + lane * HD : stk;
            float sum = 0.0f;
            // eight loads in flight, then their adds in element order: the
            // chain waits on LDS HD / 32 times, not HD / 4
            for (int i0 = 0; i0 < HD; i0 += 32) {
                v4f v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = *reinterpret_cast<const v4f *>(src + i0 + 4 * j);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    sum += v[j].x * v[j].x;
                    sum += v[j].y * v[j].y;
                    sum += v[j].z * v[j].z;
                    sum += v[j].w * v[j].w;
                }
            }
            stinv[lane] = 1.0f / sqrtf(a.rms_eps + sum / (float)HD);
        }
    }
    const int pos_new = len - 1;
    const bool owns_new = step && pos_new >= t_begin && pos_new < t_end;
    // the one wave whose tiles hold pos_new appends the new token
    const bool wave_new = owns_new && ((pos_new - t_begin) / kTK) % kWaves == wave;

    // ---- 3. the B operand of the score product, per wave from its own staged
    //      copy (no barrier): lane (l16, lg) holds column (h, b) = 16 nt + l16,
    //      values 8 lg .. 8 lg + 7 of q block b of head h after RoPE, quantized
    //      exactly as quantize_row_q8 does (kernel/quant_x.c:12-33): the block's
    //      absmax is the max over its four lanes (l16 + 16 lg) ----
    const int bl = l16 % NB;                  // block of this lane's columns (same in every nt)
    long qb[NT][NB];                          // B operand of the score product for block b'
    float qdl[NT];                            // qd[h][b] * scale * log2 e
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int h = (16 * nt + l16) / NB;
        const bool real = h < G;
        const float *row = stq + min(h, G - 1) * HD;
        const int e0 = kQK * bl + 8 * lg;
        float x[8];
        *reinterpret_cast<v4f *>(&x[0]) = *reinterpret_cast<const v4f *>(row + e0);
        *reinterpret_cast<v4f *>(&x[4]) = *reinterpret_cast<const v4f *>(row + e0 + 4);
        const float inv_h = nrm ? stinv[min(h, G - 1)] : 1.0f;
        if (nrm) norm8(x, inv_h, stqn + e0);
        if (rot) {
            constexpr int HALF = HD / 2;
            const bool lower = e0 < HALF;
            const int pi = lower ? e0 : e0 - HALF;
            const float *pr = row + (lower ? e0 + HALF : e0 - HALF);
            float y[8], c[8], sn[8];
            *reinterpret_cast<v4f *>(&y[0]) = *reinterpret_cast<const v4f *>(pr);
            *reinterpret_cast<v4f *>(&y[4]) = *reinterpret_cast<const v4f *>(pr + 4);
            if (nrm) norm8(y, inv_h, stqn + (lower ? e0 + HALF : e0 - HALF));
            *reinterpret_cast<v4f *>(&c[0]) = *reinterpret_cast<const v4f *>(stc + pi);
            *reinterpret_cast<v4f *>(&c[4]) = *reinterpret_cast<const v4f *>(stc + pi + 4);
            *reinterpret_cast<v4f *>(&sn[0]) = *reinterpret_cast<const v4f *>(sts + pi);
            *reinterpret_cast<v4f *>(&sn[4]) = *reinterpret_cast<const v4f *>(sts + pi + 4);
#pragma unroll
            for (int i = 0; i < 8; i++)
                x[i] = lower ? rope_lower(x[i], y[i], c[i], sn[i]) : rope_upper(y[i], x[i], c[i], sn[i]);
        }
        // |x| with NaN and -0 as 0, the strict "val > max" scan's value in any order
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float av = x[i] < 0.0f ? -x[i] : x[i];
            m = fmaxf(m, av > 0.0f ? av : 0.0f);
        }
        m = xrow_max(m);
        const float d = quant_scale(m);
        const float inv = quant_inverse(d);
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w0 |= quant_code(x[i], inv) << (8 * i);
            w1 |= quant_code(x[4 + i], inv) << (8 * i);
        }
        const long codes = (long)(((unsigned long)w1 << 32) | w0);
        qdl[nt] = real ? d * (a.scale * kLog2e) : 0.0f;
#pragma unroll
        for (int bb = 0; bb < NB; bb++) qb[nt][bb] = (real && bb == bl) ? codes : 0;
    }

    // ---- the work-group that appends: RoPE + exact quantize_row_q8 of the
    //      new K (after RoPE) and V rows, one 32-value block per half-wave,
    //      written to the cache and kept for the staged tile ----
    if (owns_new) {
        constexpr int NNB = 2 * NB;
        for (int j0 = 2 * wave; j0 < NNB; j0 += 2 * kWaves) {
            const int j = j0 + (lane >> 5);
            if (j < NNB) {   // a whole 32-lane block is in or out
                const int b = j % NB;
                const int col = 32 * b + (lane & 31);
                const bool is_v = j >= NB;
                const float *row = is_v ? stv : stk;
                // the K row's values through its RMSNorm when there is one
                auto kval = [&](int e) { return nrm && !is_v ? norm1(row[e], stinv[G], stkn[e]) : row[e]; };
                float x = kval(col);
                if (rot && !is_v) {
                    const int half = HD / 2;
                    const int pi = col < half ? col : col - half;
                    x = col < half ? rope_lower(kval(col), kval(col + half), stc[pi], sts[pi])
                                   : rope_upper(kval(col - half), kval(col), stc[pi], sts[pi]);
                }
                quantize_store32(x, sm.newrow + (is_v ? ROW : 0) + b * kBlockBytes);
            }
        }
        __syncthreads();
        const int phys = page_of(pos_new / kPage);
        if (phys >= 0 && tid < 2 * (ROW / 4)) {
            const bool is_v = tid >= ROW / 4;
            const int ww = is_v ? tid - ROW / 4 : tid;
            unsigned char *dst = head_run_ptr(view, phys, kvh) + (is_v ? view.kv_chunk : 0) +
                                 (pos_new % kPage) * ROW + 4 * ww;
            *reinterpret_cast<uint32_t *>(dst) =
                *reinterpret_cast<const uint32_t *>(sm.newrow + (is_v ? ROW : 0) + 4 * ww);
        }
    }

    // ---- 4. the second tile goes into the slot the staging used ----
    const int n_tiles = (t_end - t_begin + kTK - 1) / kTK;
    const int my_tiles = wave < n_tiles ? (n_tiles - wave + kWaves - 1) / kWaves : 0;
    if (k_first + kTK * kWaves < load_end) {
        wait_lds();   // the reads of the staging area are done
        fetch(tb1, k_first + kTK * kWaves);
    }
    (void)seq;

    v4f o[CT][NT];
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) o[c][nt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // per column (the same in the head's lanes and over the four 16-lane
    // rows): m_run the running max, moff the offset o and l_part are taken
    // against (m_run, or 0 before any key), thr the largest score - moff a
    // tile may hold without moving the max (kLazy; -inf before any key);
    // l_part is this lane's share of the row sum, added over the rows once
    // at the end
    float m_run[NT], moff[NT], thr[NT], l_part[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        m_run[nt] = -INFINITY;
        moff[nt] = 0.0f;
        thr[nt] = -INFINITY;
        l_part[nt] = 0.0f;
    }
    const int pr_new = wave_new ? pos_new : -1;

    // One staged tile with keys [k0, k0 + 32) in tb.
    auto process = [&](const unsigned char *tb, int k0) {
        const unsigned char *Kt = tb;
        const unsigned char *Vt = tb + kTK * ROW;
        // only a split's last tile can hold keys past its end (wave-uniform)
        const bool edge = k0 + kTK > t_end;

        // scores: exact int32 block dots, column (h, b) keeps block b
        v4i acc[2][NT];
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) acc[st][nt] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int st = 0; st < 2; st++) {
#pragma unroll
            for (int bb = 0; bb < NB; bb++) {
                const long ka = lds_ld8(Kt + (16 * st + l16) * ROW + bb * kBlockBytes + 4 + 8 * lg);
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    acc[st][nt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka, qb[nt][bb], acc[st][nt], 0, 0, 0);
            }
        }
        float kd[8], vd[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            kd[i] = lds_f(Kt + slot_key(lg, i) * ROW + bl * kBlockBytes);
            vd[i] = lds_f(Vt + slot_key(lg, i) * ROW + bl * kBlockBytes);
        }

        // scores - moff: each of the head's NB lanes adds -moff/NB (exact) to
        // its scaled block dot before the butterfly sums them
        float sc[NT][8];
        bool move = false;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const float mq = moff[nt] * (1.0f / NB);
#pragma unroll
            for (int i = 0; i < 8; i++)
                sc[nt][i] = head_block_sum<NB>(__builtin_fmaf((float)acc[i >> 2][nt][i & 3], qdl[nt] * kd[i], -mq));
            const float lmax = fmaxf(fmaxf(fmaxf(sc[nt][0], sc[nt][1]), fmaxf(sc[nt][2], sc[nt][3])),
                                     fmaxf(fmaxf(sc[nt][4], sc[nt][5]), fmaxf(sc[nt][6], sc[nt][7])));
            move |= lmax > thr[nt];
        }
        // slow path, for the whole wave when the tile holds keys past the
        // split's end or any column's tile max passes its threshold: the mask,
        // the max over the four rows, the lazy move (only by more than kLazy),
        // o and l_part rescaled and the tile re-offset
        if (edge || __builtin_amdgcn_ballot_w64(move) != 0) {
            bool rescale = false;
            float corr[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                if (edge) {
#pragma unroll
                    for (int i = 0; i < 8; i++) sc[nt][i] = k0 + slot_key(lg, i) < t_end ? sc[nt][i] : -INFINITY;
                }
                float mx = fmaxf(fmaxf(fmaxf(sc[nt][0], sc[nt][1]), fmaxf(sc[nt][2], sc[nt][3])),
                                 fmaxf(fmaxf(sc[nt][4], sc[nt][5]), fmaxf(sc[nt][6], sc[nt][7])));
                mx = xrow_max(mx) + moff[nt];
                const float m_new = mx > m_run[nt] + kLazy ? mx : m_run[nt];
                const float onew = m_new == -INFINITY ? 0.0f : m_new;
                // nothing is accumulated while m_run is -inf: corr 0, not exp2 of a difference
                corr[nt] = m_run[nt] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(moff[nt] - onew);
                const float delta = moff[nt] - onew;
#pragma unroll
                for (int i = 0; i < 8; i++) sc[nt][i] += delta;
                rescale |= corr[nt] != 1.0f;
                l_part[nt] *= corr[nt];
                m_run[nt] = m_new;
                moff[nt] = onew;
                thr[nt] = m_new == -INFINITY ? -INFINITY : kLazy;
            }
            if (__builtin_amdgcn_ballot_w64(rescale) != 0) {
#pragma unroll
                for (int c = 0; c < CT; c++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) o[c][nt] *= corr[nt];
            }
        }

        // W = exp2(S - moff) * vd <= 2^kLazy * vd, split into bf16 hi | lo
        v8bf whi[NT], wlo[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            float w[8];
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float p = __builtin_amdgcn_exp2f(sc[nt][i]);
                ps += p;
                w[i] = p * vd[i];
            }
            if (edge) {
                // keys past the end: p is 0, and their slot's scale may be
                // anything the copy saw (an unmapped page reads page 0)
#pragma unroll
                for (int i = 0; i < 8; i++) w[i] = k0 + slot_key(lg, i) < t_end ? w[i] : 0.0f;
            }
            l_part[nt] += ps;
            split_bf16(w, whi[nt], wlo[nt]);
        }

        // P.V: A = V codes of 16 columns x the 32 keys in slot order
#pragma unroll
        for (int c = 0; c < CT; c++) {
            const int col = 16 * c + l16;
            const unsigned char *vcol = Vt + (col >> 5) * kBlockBytes + 4 + (col & 31);
            float vf[8];
#pragma unroll
            for (int i = 0; i < 8; i++) vf[i] = (float)(int)(int8_t)vcol[slot_key(lg, i) * ROW];
            u32x4 pk;
#pragma unroll
            for (int i = 0; i < 4; i++) pk[i] = bf16_pair(vf[2 * i], vf[2 * i + 1]);
            const v8bf av = __builtin_bit_cast(v8bf, pk);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                o[c][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, whi[nt], o[c][nt], 0, 0, 0);
                o[c][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, wlo[nt], o[c][nt], 0, 0, 0);
            }
        }
    };

    // The new row replaces what the copy saw at pos_new.
    auto patch = [&](unsigned char *tb, int k0) {
        if (pr_new >= k0 && pr_new < k0 + kTK) {
            const int r = pr_new - k0;
            for (int w = lane; w < 2 * (ROW / 4); w += 64) {
                const bool is_v = w >= ROW / 4;
                const int ww = is_v ? w - ROW / 4 : w;
                *reinterpret_cast<uint32_t *>(tb + (is_v ? kTK * ROW : 0) + r * ROW + 4 * ww) =
                    *reinterpret_cast<const uint32_t *>(sm.newrow + (is_v ? ROW : 0) + 4 * ww);
            }
        }
    };

    // ---- the key loop: process a slot, refill it eight tiles on ----
    // Before tile j is read, its copies are done: the copies of tile j+1 (if it
    // is one of ours, already issued after tile j's) may stay in flight.
    auto wait_tile = [&](int j) {
        if (j + 1 < my_tiles)
            wait_copies<CPL>();
        else
            wait_copies<0>();
    };
    for (int it = 0; it < my_tiles; it += 2) {
        {
            const int k0 = t_begin + kTK * (wave + kWaves * it);
            wait_tile(it);
            patch(tb0, k0);
            process(tb0, k0);
            const int kn = k0 + 2 * kTK * kWaves;
            if (kn < load_end) {
                wait_lds();   // every read of the slot has completed
                fetch(tb0, kn);
            }
        }
        if (it + 1 < my_tiles) {
            const int k0 = t_begin + kTK * (wave + kWaves * (it + 1));
            wait_tile(it + 1);
            patch(tb1, k0);
            process(tb1, k0);
            const int kn = k0 + 2 * kTK * kWaves;
            if (kn < load_end) {
                wait_lds();
                fetch(tb1, kn);
            }
        }
    }

    // ---- merge the four waves in wave order ----
    __builtin_amdgcn_s_waitcnt(0);   // no copy into a slot is still in flight
    __syncthreads();                 // every wave is done with its slots
    float *mw = reinterpret_cast<float *>(&slot0[0][0]);     // [W][G]
    float *lw = mw + kWaves * G;                               // [W][G]
    float *ow = lw + kWaves * G;                               // [W][G][HD]
    float l_row[NT];   // every lane takes part in the cross-row sums
#pragma unroll
    for (int nt = 0; nt < NT; nt++) l_row[nt] = xrow_sum(l_part[nt]);
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int h = (16 * nt + l16) / NB;
        if (h < G) {
            if (lg == 0 && bl == 0) {
                mw[wave * G + h] = m_run[nt];
                lw[wave * G + h] = l_row[nt];
            }
#pragma unroll
            for (int c = 0; c < CT; c++) {
                if ((c >> 1) == bl)
                    *reinterpret_cast<v4f *>(ow + (wave * G + h) * HD + 16 * c + 4 * lg) = o[c][nt];
            }
        }
    }
    __syncthreads();

    const size_t out_row = (size_t)qi * a.n_q_heads + (size_t)kvh * G;
    const size_t pbase = ((size_t)qi * a.n_kv_heads + kvh) * a.n_splits;
    const bool single = a.n_splits == 1;
    // Float4 f4 / 4 of this (query, kv head)'s G output rows.  With completion
    // flags the rows are stored through to system scope, every wave waits for
    // its acknowledgements, and then one lane raises the flag: a host that sees
    // the flag finds the rows in its memory (and the kernel writes nothing after).
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(a.out + out_row * HD, 0, G * HD * 4, kBufWord3);
    auto put_out = [&](int f4, v4f val) {
        if (a.done)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, val), ors, 4 * f4, 0, kSystem);
        else
            *reinterpret_cast<v4f *>(a.out + out_row * HD + f4) = val;
    };
    auto signal_done = [&]() {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            __hip_atomic_store(a.done + (size_t)qi * a.n_kv_heads + kvh, a.done_seq, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
    };
    // partial rows of this (query, kv head); accesses past n_splits rows read 0
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        single ? a.out : a.partials + pbase * L::PSTRIDE, 0, single ? 0 : a.n_splits * L::PSTRIDE * 4, kBufWord3);
    for (int u = tid; u < L::U; u += kThreads) {
        const int h = (4 * u) / HD, j = 4 * u - h * HD;
        // every wave's (m, l, o) read at once: one LDS round trip
        float mws[kWaves], lws[kWaves];
        v4f ows[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            mws[w] = mw[w * G + h];
            lws[w] = lw[w * G + h];
            ows[w] = *reinterpret_cast<const v4f *>(ow + (w * G + h) * HD + j);
        }
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, mws[w]);
        v4f O = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        float Lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float f = __builtin_amdgcn_exp2f(mws[w] - M);
            O += f * ows[w];
            Lsum += f * lws[w];
        }
        if (single) {
            put_out(4 * u, O / Lsum);
        } else {
            // (the buffer intrinsics move raw 32-bit words: floats go through bit casts)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, O), prs, (split * L::PSTRIDE + 4 * u) * 4,
                                                   0, kCoherent);
            if (j == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M), prs, (split * L::PSTRIDE + G * HD + h) * 4, 0,
                                                      kCoherent);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Lsum), prs,
                                                      (split * L::PSTRIDE + G * HD + G + h) * 4, 0, kCoherent);
            }
        }
    }
    if (single) {
        if (a.done) signal_done();
        return;
    }
    __builtin_amdgcn_s_waitcnt(0);   // the partial is at the point of coherence
    __syncthreads();

    // ---- the last work-group of this (query, kv head) to arrive combines ----
    const int nvalid = (len + a.split_tokens - 1) / a.split_tokens;
    // one counter per (query, kv head), each on its own line: the splits of
    // one head serialize on it, other heads do not add to that
    int *counter = a.counters + ((size_t)qi * a.n_kv_heads + kvh) * kCounterStride;
    if (tid == 0)
        sm.last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nvalid - 1;
    __syncthreads();
    if (!sm.last) return;
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // Thread (unit u, split subset sg) sums splits sg, sg + NSG, ... of float4
    // unit u.  The first CL rows are requested together with (m, l), before
    // the weights are known; only the rows of real splits are requested (the
    // others stay 0), the weights of a pass are read together and the sum has
    // no branch, so one wait covers a pass's loads.
    constexpr int NSG = L::U >= kThreads ? 1 : kThreads / L::U;
    constexpr int TPS = L::U >= kThreads ? kThreads : L::U;
    constexpr int CL = 16;
    const int sg = tid / TPS;
    const bool active = sg < NSG;   // TPS * NSG can fall short of the 256 threads
    constexpr int HR = (G + kWaves - 1) / kWaves;   // heads per wave for the weights
    float mv[HR], lv[HR];
#pragma unroll
    for (int r = 0; r < HR; r++) {
        const int h = min(wave + kWaves * r, G - 1);
        mv[r] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(prs, (lane * L::PSTRIDE + G * HD + h) * 4, 0, kCoherent));
        lv[r] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(prs, (lane * L::PSTRIDE + G * HD + G + h) * 4, 0, kCoherent));
    }
    float *red = reinterpret_cast<float *>(&slot1[0][0]);     // [NSG][TPS][4]
    for (int u0 = 0; u0 < L::U; u0 += TPS) {
        const int u = u0 + tid % TPS;
        const float *wt = sm.wts + ((4 * u) / HD) * kMaxSplits3;
        v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < nvalid; s0 += NSG * CL) {
            v4f rows[CL];
#pragma unroll
            for (int i = 0; i < CL; i++) {
                const int s = s0 + sg + NSG * i;
                rows[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                if (s < nvalid)
                    rows[i] = __builtin_bit_cast(
                        v4f, __builtin_amdgcn_raw_buffer_load_b128(prs, (s * L::PSTRIDE + 4 * u) * 4, 0, kCoherent));
            }
            if (u0 == 0 && s0 == 0) {
#pragma unroll
                for (int r = 0; r < HR; r++) {
                    const int h = wave + kWaves * r;
                    if (h < G) {
                        const bool ok = lane < nvalid;
                        const float m = ok ? mv[r] : -INFINITY;
                        const float M = wave_max(m);
                        const float f = ok ? __builtin_amdgcn_exp2f(m - M) : 0.0f;
                        sm.wts[h * kMaxSplits3 + lane] = f / wave_sum(ok ? lv[r] * f : 0.0f);
                    }
                }
                __syncthreads();
            }
            float w[CL];
#pragma unroll
            for (int i = 0; i < CL; i++) w[i] = wt[min(s0 + sg + NSG * i, kMaxSplits3 - 1)];
#pragma unroll
            for (int i = 0; i < CL; i++) acc += (s0 + sg + NSG * i < nvalid ? w[i] : 0.0f) * rows[i];
        }
        if constexpr (NSG == 1) {
            if (active) put_out(4 * u, acc);
        } else {
            *reinterpret_cast<v4f *>(red + 4 * tid) = acc;
            __syncthreads();
            if (tid < TPS) {
                v4f r = *reinterpret_cast<const v4f *>(red + 4 * tid);
                for (int g = 1; g < NSG; g++) r += *reinterpret_cast<const v4f *>(red + 4 * (g * TPS + tid));
                put_out(4 * (u0 + tid), r);
            }
            __syncthreads();
        }
    }
    if (a.done) signal_done();
}

template <int HD, int G>
hipError_t launch3_hd_g(const TqDecodeArgs &a, int waves, hipStream_t s) {
    if (waves == 8)
        hipLaunchKernelGGL((decode3_kernel<HD, G, 8>), dim3(a.n_splits, a.n_kv_heads, a.n_q), dim3(512), 0, s, a);
    else
        hipLaunchKernelGGL((decode3_kernel<HD, G, 4>), dim3(a.n_splits, a.n_kv_heads, a.n_q), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int HD>
hipError_t launch3_hd(const TqDecodeArgs &a, int g, int waves, hipStream_t s) {
    switch (g) {
        case 1: return launch3_hd_g<HD, 1>(a, waves, s);
        case 2: return launch3_hd_g<HD, 2>(a, waves, s);
        case 3: return launch3_hd_g<HD, 3>(a, waves, s);
        case 4: return launch3_hd_g<HD, 4>(a, waves, s);
        case 5: return launch3_hd_g<HD, 5>(a, waves, s);
        case 6: return launch3_hd_g<HD, 6>(a, waves, s);
        case 7: return launch3_hd_g<HD, 7>(a, waves, s);
        case 8: return launch3_hd_g<HD, 8>(a, waves, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool tq_decode3_supported(int head_dim, int group) {
    const bool hd_ok = head_dim == 32 || head_dim == 64 || head_dim == 128;
    return hd_ok && group >= 1 && group <= 8;
}

int tq_decode3_max_splits() { return kMaxSplits3; }
int tq_decode3_max_split_tokens() { return kMaxSplitPages3 * kPage; }
int tq_decode3_partial_floats(int head_dim, int group) { return (group * (head_dim + 2) + 3) / 4 * 4; }

hipError_t tq_launch_decode3(const TqDecodeArgs &a, int waves, hipStream_t s) {
    if (a.n_q <= 0) return hipSuccess;
    if (waves != 4 && waves != 8) return hipErrorInvalidValue;
    if (a.n_splits < 1 || a.n_splits > kMaxSplits3 || a.split_tokens <= 0 || a.split_tokens % kTK != 0 ||
        a.split_tokens > kMaxSplitPages3 * kPage)
        return hipErrorInvalidValue;
    if (a.n_splits > 1 && (a.partials == nullptr || a.counters == nullptr)) return hipErrorInvalidValue;
    const int g = a.n_q_heads / a.n_kv_heads;
    if (!tq_decode3_supported(a.head_dim, g)) return hipErrorInvalidValue;
    switch (a.head_dim) {
        case 32: return launch3_hd<32>(a, g, waves, s);
        case 64: return launch3_hd<64>(a, g, waves, s);
        case 128: return launch3_hd<128>(a, g, waves, s);
        default: return hipErrorInvalidValue;
    }
}
