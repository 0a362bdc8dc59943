// decode.hip — attend_q8 (model/attention_layer.c:125-150) on the paged cache.
//
// decode_kernel, grid (split, kv head, query): a 256-thread work-group owns
// tokens [split*split_tokens, min(len, (split+1)*split_tokens)) of one kv head
// and all G = n_q_heads/n_kv_heads query heads reading it, so each K/V byte is
// fetched once per step.  The range is walked in sub-chunks of TSUB = 256/nb
// tokens (18,432 bytes of K+V at any head_dim).
//
// At batch 1 a decode step is a ~9 MB read, so latency, not bandwidth, sets
// its time; the work-group keeps dependent round trips and barriers few:
//   1. one round trip brings len, the group's q rows (and in step mode the new
//      K/V rows) into registers and the split's physical page ids into LDS;
//   2. the K/V pages of the first two sub-chunks are requested (16-byte
//      coalesced loads into registers) with no global load between them, so
//      the in-order vmcnt never makes one prefetch wait on another;
//   3. while they fly, q gets RoPE and quantize_row_q8 (exact) into LDS;
//   4. each sub-chunk is processed from one of two LDS buffers while the loads
//      of sub-chunk i+2 fly, with three barriers:
//        scores: thread (token, block) computes the exact int32 block dot for
//        all G heads off one K block (v_dot4_i32_i8), scales by qd*kd and
//        sums a token's blocks in block order with DPP lane moves — scores
//        bit-identical to attn_scores_q8_scalar (model/attn_q8.c:17-34);
//        online softmax: one wave per head, DPP reductions;
//        P.V: thread (4 columns, token subset) accumulates all G heads over
//        8 tokens, fully unrolled and branch-free (masked tokens weigh 0).
//
// Several splits: each work-group writes its (o, m, l) partial with
// agent-scope atomic stores (written through to the point of coherence of all
// XCDs), waits for their acknowledgement and bumps an integer arrival counter;
// the last work-group of a (query, kv head) merges all partials in split order
// with weights exp(m_s - M)/L.  One launch per step, no float atomics, a result
// independent of which work-group arrived last, and no cache write-back or
// invalidation fence (an L2 write-back per work-group, serialised per XCD,
// costs ~24 us here; an L2 invalidation ~2 us): the combining work-group reads
// the partials back with agent-scope atomic loads, all in one round trip.
//
// Step mode (k_new != null): the work-group owning position len-1 quantizes
// the new token's K (after RoPE) and V exactly as store_kv does, writes them to
// the cache and patches them into its LDS copy: append + attend in one launch.
#include "tq_common.hpp"

namespace {

using namespace tq;

constexpr int kMaxSplits = 64;
constexpr int kMaxSplitPages = 512;  // page ids a work-group stages (8,192 tokens)

// A load that observes stores made coherent at agent scope by other XCDs.
__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lane t of a token's NB consecutive lanes gets the value of lane t + J (row_shl:J).
template <int J>
__device__ __forceinline__ float from_lane_plus(float x) {
    return dpp_f<0x100 + J>(x);
}

// Ordered sum over the NB lanes of a token, valid in its first lane:
// ((0 + x0) + x1) + ... as attn_scores_q8_scalar sums its blocks.
template <int NB>
__device__ __forceinline__ float token_block_sum(float x) {
#pragma clang fp contract(off)
    float acc = 0.0f;
    acc += x;
    if constexpr (NB >= 2) acc += from_lane_plus<1>(x);
    if constexpr (NB >= 4) {
        acc += from_lane_plus<2>(x);
        acc += from_lane_plus<3>(x);
    }
    if constexpr (NB >= 8) {
        acc += from_lane_plus<4>(x);
        acc += from_lane_plus<5>(x);
        acc += from_lane_plus<6>(x);
        acc += from_lane_plus<7>(x);
    }
    return acc;
}

template <int HD, int G>
struct Shape {
    static constexpr int NB = HD / kQK;
    static constexpr int ROW = NB * kBlockBytes;           // bytes per token row
    static constexpr int TSUB = kThreads / NB;             // tokens per sub-chunk
    static constexpr int NPG = TSUB / kPage;               // pages per sub-chunk
    static constexpr int CHUNK = kPage * ROW;              // one page of K (or V), one head
    static constexpr int VEC_PER_PAGE = 2 * CHUNK / 16;    // K+V run in 16-byte vectors
    static constexpr int NVEC = NPG * VEC_PER_PAGE;
    static constexpr int VPT = (NVEC + kThreads - 1) / kThreads;
    static constexpr int NCG = HD / 4;                     // 4-column groups
    static constexpr int NTS = kThreads / NCG;             // token subsets in P.V
    static constexpr int TPT = TSUB / NTS;                 // tokens per thread in P.V (8)
    static constexpr int KV_BYTES = 2 * TSUB * ROW;        // one buffer: K rows | V rows
    static constexpr int RED_BYTES = NTS * G * HD * 4;
    static constexpr int SMEM = 2 * KV_BYTES > RED_BYTES ? 2 * KV_BYTES : RED_BYTES;
    static constexpr int QE = (G * HD + kThreads - 1) / kThreads;   // q values per thread
    static constexpr int NE = (2 * HD + kThreads - 1) / kThreads;   // new K/V values per thread
    // P.V tokens whose LDS reads are batched (register budget at large G)
    static constexpr int PV_UNROLL = G <= 4 ? 8 : 4;
    // combine: U float4 outputs, NSG split subsets of TPS threads, CL partial
    // rows requested per thread in one round
    static constexpr int U = G * HD / 4;
    static constexpr int NSG = kThreads / U > 0 ? kThreads / U : 1;
    static constexpr int TPS = kThreads / NSG;
    static constexpr int CL = U <= 128 ? 16 : 8;
    static constexpr int MAX_SPLITS = NSG * CL < kMaxSplits ? NSG * CL : kMaxSplits;
    static_assert(NB * TSUB == kThreads, "one (token, block) pair per thread");
    static_assert(TSUB % kPage == 0, "sub-chunks are whole pages");
    static_assert(NTS * NCG == kThreads, "one (column group, subset) per thread");
};

template <int HD, int G>
struct Smem {
    using S = Shape<HD, G>;
    unsigned char kv[S::SMEM];              // two K|V buffers; later the P.V reduction
    unsigned char qblk[G * S::ROW];         // quantized q rows of the group
    unsigned char newrow[2 * S::ROW];       // step mode: the new token's K, V
    float sp[2][S::TSUB * G];               // scores, then probabilities, [token][head]
    float corr[2][G];                       // exp(m_old - m_new) of the sub-chunk
    float mfin[G], lfin[G];
    int pages[kMaxSplitPages];              // physical page of each page of the split
    float wts[G * kMaxSplits];              // combine weights exp(m_s - M) / L
    int last;                               // this work-group combines
};

// A value of a head row after RoPE, from registers: own value, partner
// (i +- hd/2) and the table entry of the pair.
struct RopeIn {
    float x, partner, c, s;
};

__device__ __forceinline__ RopeIn rope_fetch(const float *head, int col, int hd, const float *ct,
                                             const float *st) {
    RopeIn r;
    r.x = head[col];
    if (ct) {
        const int half = hd >> 1;
        const int i = col < half ? col : col - half;
        r.partner = head[col < half ? col + half : col - half];
        r.c = ct[i];
        r.s = st[i];
    }
    return r;
}

__device__ __forceinline__ float rope_value(const RopeIn &r, int col, int hd, bool rotate) {
    if (!rotate) return r.x;
    return col < (hd >> 1) ? rope_lower(r.x, r.partner, r.c, r.s) : rope_upper(r.partner, r.x, r.c, r.s);
}

// Per-work-group state; members are indexed statically after inlining, so
// they all live in registers.
template <int HD, int G>
struct Decoder {
    using S = Shape<HD, G>;
    static constexpr int NB = S::NB, ROW = S::ROW, TSUB = S::TSUB;

    Smem<HD, G> &sm;
    const PagedView &view;
    int tid, lane, wave, kvh, t_begin, t_end, pos_new;
    int load_end;                // loads cover tokens below this
    int contig_first, contig_pages;  // contiguous sequence: page = first + lp
    bool owns_new;
    float scale;
    // scores role: (token my_t, block my_b)
    int my_t, my_b;
    int32_t qreg[G][8];
    float qd[G];
    // P.V role: (column group cg, token subset ts)
    int cg, ts;
    float o[G][4];
    // softmax role: wave owns heads wave, wave + 4
    float m_run[2], l_run[2];

    __device__ __forceinline__ Decoder(Smem<HD, G> &s, const PagedView &v, int kvh_, int t_begin_, int load_end_,
                                       int contig_first_, int contig_pages_, float scale_)
        : sm(s), view(v), kvh(kvh_), t_begin(t_begin_), t_end(load_end_), pos_new(-1), load_end(load_end_),
          contig_first(contig_first_), contig_pages(contig_pages_), owns_new(false), scale(scale_) {
        tid = threadIdx.x;
        lane = tid & 63;
        wave = tid >> 6;
        my_t = tid / NB;
        my_b = tid % NB;
        cg = tid % S::NCG;
        ts = tid / S::NCG;
#pragma unroll
        for (int gi = 0; gi < G; gi++)
#pragma unroll
            for (int c = 0; c < 4; c++) o[gi][c] = 0.0f;
        m_run[0] = m_run[1] = -INFINITY;
        l_run[0] = l_run[1] = 0.0f;
    }

    // 16-byte loads of sub-chunk [c0, c0+TSUB): vector vi is page vi / VEC_PER_PAGE,
    // byte 16*(vi % VEC_PER_PAGE) of that page's K+V run.  Page ids come from LDS,
    // or, for a contiguous sequence, from contig_first without any memory access.
    __device__ __forceinline__ void load(u32x4 (&pf)[S::VPT], int c0) const {
#pragma unroll
        for (int i = 0; i < S::VPT; i++) {
            const int vi = tid + i * kThreads;
            if (vi < S::NVEC) {
                const int p = vi / S::VEC_PER_PAGE;
                const int w = vi - p * S::VEC_PER_PAGE;
                const int tok0 = c0 + p * kPage;
                int phys;
                if (contig_first >= 0) {
                    const int lp = tok0 / kPage;
                    phys = lp < contig_pages ? contig_first + lp : -1;
                } else {
                    // page id read unconditionally (index clamped into the array)
                    phys = sm.pages[min((tok0 - t_begin) / kPage, kMaxSplitPages - 1)];
                }
                if (tok0 < load_end && phys >= 0)
                    pf[i] = *reinterpret_cast<const u32x4 *>(head_run_ptr(view, phys, kvh) + 16 * w);
            }
        }
    }

    // Prefetched vectors -> LDS buffer: K rows contiguous, then V rows ([TSUB][nb] each).
    __device__ __forceinline__ void store(const u32x4 (&pf)[S::VPT], unsigned char *kbuf) {
#pragma unroll
        for (int i = 0; i < S::VPT; i++) {
            const int vi = tid + i * kThreads;
            if (vi < S::NVEC) {
                const int p = vi / S::VEC_PER_PAGE;
                const int byte = 16 * (vi - p * S::VEC_PER_PAGE);
                unsigned char *dst = byte < S::CHUNK ? kbuf + p * S::CHUNK + byte
                                                     : kbuf + TSUB * ROW + p * S::CHUNK + (byte - S::CHUNK);
                *reinterpret_cast<u32x4 *>(dst) = pf[i];
            }
        }
    }

    __device__ __forceinline__ void load_q_regs() {
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            const unsigned char *qb = sm.qblk + gi * ROW + my_b * kBlockBytes;
            qd[gi] = *reinterpret_cast<const float *>(qb);
#pragma unroll
            for (int w = 0; w < 8; w++) qreg[gi][w] = *reinterpret_cast<const int32_t *>(qb + 4 + 4 * w);
        }
    }

    // One sub-chunk starting at token c0 whose loads sit in pf, processed in
    // LDS buffer BUF; pf is then refilled with sub-chunk c_next if c_next < t_end.
    // Buffers alternate, so no barrier is needed after P.V: the next sub-chunk
    // writes the other buffer, and the one after passes this one's barriers.
    template <int BUF>
    __device__ __forceinline__ void run(u32x4 (&pf)[S::VPT], int c0, int c_next) {
        unsigned char *kbuf = sm.kv + BUF * S::KV_BYTES;
        unsigned char *vbuf = kbuf + TSUB * ROW;
        float *sp = sm.sp[BUF];
        float *corr = sm.corr[BUF];
        store(pf, kbuf);
        __syncthreads();
        if (owns_new && pos_new >= c0 && pos_new < c0 + TSUB) {
            const int r = pos_new - c0;
            if (tid < 2 * (ROW / 4)) {
                const bool is_v = tid >= ROW / 4;
                const int w = is_v ? tid - ROW / 4 : tid;
                *reinterpret_cast<uint32_t *>((is_v ? vbuf : kbuf) + r * ROW + 4 * w) =
                    *reinterpret_cast<const uint32_t *>(sm.newrow + (is_v ? ROW : 0) + 4 * w);
            }
            __syncthreads();
        }
        if (c_next < load_end) load(pf, c_next);

        // ---- scores -------------------------------------------------------------
        {
            // Same rounding sequence as attn_scores_q8_scalar: no contraction.
#pragma clang fp contract(off)
            const unsigned char *kb = kbuf + my_t * ROW + my_b * kBlockBytes;
            const float kd = *reinterpret_cast<const float *>(kb);
            int32_t kc[8];
#pragma unroll
            for (int w = 0; w < 8; w++) kc[w] = *reinterpret_cast<const int32_t *>(kb + 4 + 4 * w);
            const bool valid = c0 + my_t < t_end;
#pragma unroll
            for (int gi = 0; gi < G; gi++) {
                int32_t dot = 0;
#pragma unroll
                for (int w = 0; w < 8; w++) dot = __builtin_amdgcn_sdot4(qreg[gi][w], kc[w], dot, false);
                const float x = (float)dot * (qd[gi] * kd);
                const float acc = token_block_sum<NB>(x);
                if (my_b == 0) sp[my_t * G + gi] = valid ? acc * scale : -INFINITY;
            }
        }
        __syncthreads();

        // ---- online softmax, one wave per head ------------------------------------
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int gi = wave + 4 * r;
            if (gi < G) {
                float sv[(TSUB + 63) / 64];
                float mloc = -INFINITY;
#pragma unroll
                for (int i = 0; i < (TSUB + 63) / 64; i++) {
                    const int t = lane + 64 * i;
                    const float x = sp[min(t, TSUB - 1) * G + gi];  // unconditional LDS read
                    sv[i] = t < TSUB ? x : -INFINITY;
                    mloc = fmaxf(mloc, sv[i]);
                }
                mloc = wave_max(mloc);
                const float m_new = fmaxf(m_run[r], mloc);
                const float c = expf(m_run[r] - m_new);
                float lsum = 0.0f;
#pragma unroll
                for (int i = 0; i < (TSUB + 63) / 64; i++) {
                    const int t = lane + 64 * i;
                    const float p = expf(sv[i] - m_new);
                    if (t < TSUB) sp[t * G + gi] = p;
                    lsum += p;
                }
                lsum = wave_sum(lsum);
                l_run[r] = l_run[r] * c + lsum;
                m_run[r] = m_new;
                if (lane == 0) corr[gi] = c;
            }
        }
        __syncthreads();

        // ---- P.V: 8 tokens, unrolled, masked tokens weigh 0 ------------------------
        {
#pragma unroll
            for (int gi = 0; gi < G; gi++) {
                const float c = corr[gi];
#pragma unroll
                for (int k = 0; k < 4; k++) o[gi][k] *= c;
            }
            const int pv_b = cg >> 3, pv_w = cg & 7;
            // Every LDS read is unconditional (a read under a condition becomes a
            // branch with its own wait); masking is a select on the V scale, so a
            // stale scale of a masked token never reaches the sum (p is 0 there).
#pragma unroll S::PV_UNROLL
            for (int k = 0; k < S::TPT; k++) {
                const int t = ts + k * S::NTS;
                const unsigned char *vb = vbuf + t * ROW + pv_b * kBlockBytes;
                const float vd_raw = *reinterpret_cast<const float *>(vb);
                const uint32_t codes = *reinterpret_cast<const uint32_t *>(vb + 4 + 4 * pv_w);
                float pt[G];
#pragma unroll
                for (int gi = 0; gi < G; gi++) pt[gi] = sp[t * G + gi];
                const float vd = c0 + t < t_end ? vd_raw : 0.0f;
                const float f0 = (float)(int8_t)(codes & 0xFF);
                const float f1 = (float)(int8_t)((codes >> 8) & 0xFF);
                const float f2 = (float)(int8_t)((codes >> 16) & 0xFF);
                const float f3 = (float)(int8_t)(codes >> 24);
#pragma unroll
                for (int gi = 0; gi < G; gi++) {
                    const float av = pt[gi] * vd;
                    o[gi][0] += av * f0;
                    o[gi][1] += av * f1;
                    o[gi][2] += av * f2;
                    o[gi][3] += av * f3;
                }
            }
        }
    }

    // Sum the token subsets in a fixed order into red[gi*HD + j] (LDS).
    __device__ __forceinline__ float *reduce() {
        __syncthreads();  // the last P.V has read the LDS buffers
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int gi = wave + 4 * r;
            if (gi < G && lane == 0) {
                sm.mfin[gi] = m_run[r];
                sm.lfin[gi] = l_run[r];
            }
        }
        float *red = reinterpret_cast<float *>(sm.kv);
#pragma unroll
        for (int gi = 0; gi < G; gi++)
            *reinterpret_cast<float4 *>(red + ((size_t)ts * G + gi) * HD + cg * 4) =
                make_float4(o[gi][0], o[gi][1], o[gi][2], o[gi][3]);
        __syncthreads();
        return red;
    }
};

template <int HD, int G>
__global__ __launch_bounds__(256) void decode_kernel(TqDecodeArgs a) {
    using S = Shape<HD, G>;
    constexpr int ROW = S::ROW, TSUB = S::TSUB;
    __shared__ __align__(16) Smem<HD, G> sm;

    const int tid = threadIdx.x;
    const int split = blockIdx.x, kvh = blockIdx.y, qi = blockIdx.z;
    const int seq = a.seq_of ? a.seq_of[qi] : a.seq_const + a.seq_stride * qi;
    const int t_begin = split * a.split_tokens;

    // ---- 1. one round trip: len, q rows, new K/V rows, the split's page ids ----
    // None of these loads waits for another; len is consulted only afterwards.
    const int len = a.len_of ? a.len_of[qi] + a.len_plus : a.pos0 + qi + 1;
    const bool rot = a.cos_t != nullptr;
    const float *ct = rot ? a.cos_t + (size_t)qi * (HD / 2) : nullptr;
    const float *st = rot ? a.sin_t + (size_t)qi * (HD / 2) : nullptr;
    const float *qg = a.q + ((size_t)qi * a.n_q_heads + (size_t)kvh * G) * HD;
    RopeIn qin[S::QE];
#pragma unroll
    for (int i = 0; i < S::QE; i++) {
        const int e = tid + i * kThreads;
        if (e < G * HD) qin[i] = rope_fetch(qg + (e / HD) * HD, e % HD, HD, ct, st);
    }
    RopeIn nin[S::NE];
    if (a.k_new != nullptr) {
        const size_t off = ((size_t)qi * a.n_kv_heads + kvh) * HD;
#pragma unroll
        for (int i = 0; i < S::NE; i++) {
            const int e = tid + i * kThreads;
            if (e < HD) nin[i] = rope_fetch(a.k_new + off, e, HD, ct, st);
            else if (e < 2 * HD) nin[i].x = a.v_new[off + e - HD];
        }
    }
    const bool contig = a.contig_first >= 0;
    Decoder<HD, G> d(sm, a.view, kvh, t_begin, t_begin + a.split_tokens, a.contig_first, a.contig_pages, a.scale);
    u32x4 pfa[S::VPT], pfb[S::VPT];
    int len_known;
    if (contig) {
        // ---- 2a. contiguous sequence: K/V requested at once, before len is known;
        //      only pages the sequence maps are touched ------------------------------
        d.load_end = min(t_begin + a.split_tokens, a.contig_pages * kPage);
        d.load(pfa, t_begin);
        if (d.load_end > t_begin + TSUB) d.load(pfb, t_begin + TSUB);
        len_known = len;
        if (len_known <= 0 || t_begin >= len_known) return;
    } else {
        // ---- 2b. paged: the split's page ids into LDS, then K/V ---------------------
        const int split_pages = a.split_tokens / kPage;
        int page_id[(kMaxSplitPages + kThreads - 1) / kThreads];
#pragma unroll
        for (int i = 0; i < (kMaxSplitPages + kThreads - 1) / kThreads; i++) {
            const int p = tid + i * kThreads;
            if (p < split_pages) page_id[i] = phys_page(a.view, seq, t_begin / kPage + p);
        }
        len_known = len;
        if (len_known <= 0 || t_begin >= len_known) return;
#pragma unroll
        for (int i = 0; i < (kMaxSplitPages + kThreads - 1) / kThreads; i++) {
            const int p = tid + i * kThreads;
            if (p < split_pages) sm.pages[p] = page_id[i];
        }
        __syncthreads();
        d.load_end = min(len_known, t_begin + a.split_tokens);
        d.load(pfa, t_begin);
        if (d.load_end > t_begin + TSUB) d.load(pfb, t_begin + TSUB);
    }
    const int t_end = min(len_known, t_begin + a.split_tokens);
    const int pos_new = len_known - 1;
    const bool owns_new = a.k_new != nullptr && pos_new >= t_begin && pos_new < t_end;
    d.t_end = t_end;
    d.load_end = min(d.load_end, t_end);
    d.pos_new = pos_new;
    d.owns_new = owns_new;
    const int n_sub = (t_end - t_begin + TSUB - 1) / TSUB;

    // ---- 3. RoPE + exact quantize of q (and the new row) into LDS ---------------------
#pragma unroll
    for (int i = 0; i < S::QE; i++) {
        const int e = tid + i * kThreads;
        if (e < G * HD) {
            const int gi = e / HD, col = e % HD;
            quantize_store32(rope_value(qin[i], col, HD, rot), sm.qblk + gi * ROW + (col >> 5) * kBlockBytes);
        }
    }
    if (owns_new) {
#pragma unroll
        for (int i = 0; i < S::NE; i++) {
            const int e = tid + i * kThreads;
            if (e < 2 * HD) {
                const bool is_v = e >= HD;
                const int col = is_v ? e - HD : e;
                const float x = is_v ? nin[i].x : rope_value(nin[i], col, HD, rot);
                quantize_store32(x, sm.newrow + (is_v ? ROW : 0) + (col >> 5) * kBlockBytes);
            }
        }
    }
    __syncthreads();
    if (owns_new) {
        const int lp = pos_new / kPage;
        const int phys = contig ? (lp < a.contig_pages ? a.contig_first + lp : -1) : sm.pages[(pos_new - t_begin) / kPage];
        if (phys >= 0 && tid < 2 * (ROW / 4)) {
            const bool is_v = tid >= ROW / 4;
            const int w = is_v ? tid - ROW / 4 : tid;
            unsigned char *dst = head_run_ptr(a.view, phys, kvh) + (is_v ? S::CHUNK : 0) +
                                 (pos_new % kPage) * ROW + 4 * w;
            *reinterpret_cast<uint32_t *>(dst) = *reinterpret_cast<const uint32_t *>(sm.newrow + (is_v ? ROW : 0) + 4 * w);
        }
    }
    d.load_q_regs();

    // ---- 4. sub-chunks: prefetch buffers and LDS buffers in turn ---------------------------
    for (int sub = 0; sub < n_sub; sub += 2) {
        const int c0 = t_begin + sub * TSUB;
        d.template run<0>(pfa, c0, c0 + 2 * TSUB);
        if (sub + 1 < n_sub) d.template run<1>(pfb, c0 + TSUB, c0 + 3 * TSUB);
    }
    float *red = d.reduce();

    if (a.n_splits == 1) {
        const size_t out_row = (size_t)qi * a.n_q_heads + (size_t)kvh * G;
        for (int idx = tid; idx < G * HD; idx += kThreads) {
            const int gi = idx / HD, j = idx - gi * HD;
            float acc = 0.0f;
            for (int s = 0; s < S::NTS; s++) acc += red[((size_t)s * G + gi) * HD + j];
            a.out[(out_row + gi) * HD + j] = acc / sm.lfin[gi];
        }
        return;
    }

    // ---- 5. partial (o[G][HD], m[G], l[G]) of this split ------------------------------------
    // Agent-scope atomic stores go through to the point of coherence of all
    // XCDs; once they are acknowledged (s_waitcnt) the arrival counter is bumped.
    const size_t pstride = (size_t)G * (HD + 2);
    const size_t pbase = ((size_t)qi * a.n_kv_heads + kvh) * a.n_splits;
    float *part = a.partials + (pbase + split) * pstride;
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int gi = idx / HD, j = idx - gi * HD;
        float acc = 0.0f;
        for (int s = 0; s < S::NTS; s++) acc += red[((size_t)s * G + gi) * HD + j];
        __hip_atomic_store(part + idx, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < G) {
        __hip_atomic_store(part + G * HD + tid, sm.mfin[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part + G * HD + G + tid, sm.lfin[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // ---- 6. the last work-group of this (query, kv head) to arrive combines ----------------
    const int nvalid = (len + a.split_tokens - 1) / a.split_tokens;
    int *counter = a.counters + (size_t)qi * a.n_kv_heads + kvh;
    if (tid == 0)
        sm.last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nvalid - 1;
    __syncthreads();
    if (!sm.last) return;
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // The partials are read back with agent-scope atomic loads, coherent across
    // XCDs like the stores that wrote them, so no cache invalidation (an
    // acquire fence costs ~2 us here) is needed.  One round trip: (m, l) of
    // every split for the wave's heads, then thread (float4 output u, split
    // subset sg) requests its CL partial rows.
    const float *parts = a.partials + pbase * pstride;
    const int wv = tid >> 6, ln = tid & 63;
    float mv[2], lv[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int gi = wv + 4 * r;
        const bool ok = gi < G && ln < nvalid;
        mv[r] = ok ? coherent_load(parts + ln * pstride + G * HD + gi) : -INFINITY;
        lv[r] = ok ? coherent_load(parts + ln * pstride + G * HD + G + gi) : 0.0f;
    }
    float4 *fred = reinterpret_cast<float4 *>(sm.kv);
    for (int u0 = 0; u0 < S::U; u0 += S::TPS) {
        const int u = u0 + tid % S::TPS, sg = tid / S::TPS;
        const bool act = u < S::U && sg < S::NSG;
        float4 ov[S::CL];
#pragma unroll
        for (int i = 0; i < S::CL; i++) {
            const int s = sg + S::NSG * i;
            ov[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (act && s < nvalid) {
                const float *src = parts + s * pstride + 4 * u;
                ov[i] = make_float4(coherent_load(src), coherent_load(src + 1), coherent_load(src + 2),
                                    coherent_load(src + 3));
            }
        }
        if (u0 == 0) {
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int gi = wv + 4 * r;
                if (gi < G) {
                    const float M = wave_max(mv[r]);
                    const float w = ln < nvalid ? expf(mv[r] - M) : 0.0f;
                    sm.wts[gi * kMaxSplits + ln] = w / wave_sum(lv[r] * w);
                }
            }
            __syncthreads();
        }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        {
            // weights of splits past nvalid are 0 and their rows were zeroed
            const float *wt = sm.wts + (min(4 * u, G * HD - 4) / HD) * kMaxSplits;
#pragma unroll
            for (int i = 0; i < S::CL; i++) {
                const float w = wt[min(sg + S::NSG * i, kMaxSplits - 1)];
                acc.x += ov[i].x * w;
                acc.y += ov[i].y * w;
                acc.z += ov[i].z * w;
                acc.w += ov[i].w * w;
            }
        }
        fred[tid] = acc;
        __syncthreads();
        if (tid < S::TPS && u0 + tid < S::U) {
            float4 r = fred[tid];
            for (int g = 1; g < S::NSG; g++) {
                const float4 x = fred[g * S::TPS + tid];
                r.x += x.x;
                r.y += x.y;
                r.z += x.z;
                r.w += x.w;
            }
            const int uu = u0 + tid;
            const int gi = (4 * uu) / HD, j = 4 * uu - gi * HD;
            *reinterpret_cast<float4 *>(a.out + ((size_t)qi * a.n_q_heads + (size_t)kvh * G + gi) * HD + j) = r;
        }
        __syncthreads();
    }
}

template <int HD, int G>
hipError_t launch_hd_g(const TqDecodeArgs &a, hipStream_t s) {
    if (a.n_splits > Shape<HD, G>::MAX_SPLITS) return hipErrorInvalidValue;
    hipLaunchKernelGGL((decode_kernel<HD, G>), dim3(a.n_splits, a.n_kv_heads, a.n_q), dim3(kThreads), 0,
                       s, a);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const TqDecodeArgs &a, int g, hipStream_t s) {
    switch (g) {
        case 1: return launch_hd_g<HD, 1>(a, s);
        case 2: return launch_hd_g<HD, 2>(a, s);
        case 3: return launch_hd_g<HD, 3>(a, s);
        case 4: return launch_hd_g<HD, 4>(a, s);
        case 5: return launch_hd_g<HD, 5>(a, s);
        case 6: return launch_hd_g<HD, 6>(a, s);
        case 7: return launch_hd_g<HD, 7>(a, s);
        case 8: return launch_hd_g<HD, 8>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

int tq_decode_tsub(int head_dim) { return kThreads / (head_dim / kQK); }
int tq_decode_max_split_tokens() { return kMaxSplitPages * kPage; }

// Splits the in-kernel combine takes: its one round of partial loads covers
// CL splits per thread subset (Shape::MAX_SPLITS).
int tq_decode_max_splits(int head_dim, int group) {
    const int u = group * head_dim / 4;
    const int nsg = kThreads / u > 0 ? kThreads / u : 1;
    const int cl = u <= 128 ? 16 : 8;
    return nsg * cl < kMaxSplits ? nsg * cl : kMaxSplits;
}

bool tq_decode_supported(int head_dim, int group) {
    const bool hd_ok = head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
    return hd_ok && group >= 1 && group <= 8;
}

hipError_t tq_launch_decode(const TqDecodeArgs &a, hipStream_t s) {
    if (a.n_q <= 0) return hipSuccess;
    if (a.n_splits < 1 || a.split_tokens <= 0 || a.split_tokens > kMaxSplitPages * kPage) return hipErrorInvalidValue;
    if (a.n_splits > 1 && (a.partials == nullptr || a.counters == nullptr)) return hipErrorInvalidValue;
    const int g = a.n_q_heads / a.n_kv_heads;
    switch (a.head_dim) {
        case 32: return launch_hd<32>(a, g, s);
        case 64: return launch_hd<64>(a, g, s);
        case 128: return launch_hd<128>(a, g, s);
        case 256: return launch_hd<256>(a, g, s);
        default: return hipErrorInvalidValue;
    }
}
