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
//   contiguous tile image laid out as the MFMA operands want it:
//     K codes  [2 key tiles][block][lane][8 bytes]  (A of the i8 product)
//     K scales [block][key]
//     V' hi|lo [column tile][lane][8 bf16]          (A of the bf16 product)
//   with V' = code * vd rounded once to fp32 and split into bf16 hi + lo.
//   Every query block then streams these images instead of re-deriving them.
//
// prefill_kernel — work-group of 256 threads (4 waves), one kv head, 64*NJ
//   (query, head) rows = QB = 64*NJ/G consecutive query tokens x the G heads
//   of the group, in row tiles of 16 queries of one head; wave w owns NJ row
//   tiles.  Key tiles stream through two LDS buffers (16-byte loads into
//   registers one tile ahead), one barrier per tile:
//     S^T = K . Q^T per 32-element block on v_mfma_i32_16x16x32_i8 — exact
//       int32 block dots, as attn_scores_q8 forms them (model/attn_q8.c:24-30)
//       — scaled by qd*kd per block in fp32 (FMA: scores match within
//       rounding, not bit for bit);
//     online softmax per query (exp2 domain), causal mask;
//     O^T += V'^T . P^T on v_mfma_f32_16x16x32_bf16, P split into bf16 hi + lo
//       like V': hi.hi + hi.lo + lo.hi carries ~16 significant bits per
//       product, fp32 accumulation.
//   The S^T orientation leaves each lane with 8 keys of one query: exactly a
//   B operand of the P.V product (keys permuted identically in A and B), so P
//   never goes through LDS.  Grid x runs the heaviest (latest) query blocks
//   first.
#include "tq_common.hpp"

namespace {

using namespace tq;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kKT = 32;                  // keys per tile
constexpr int kMaxPrefillKeys = 65536;   // keys [0, kend) the dense path serves
constexpr float kLog2e = 1.4426950408889634f;

// Layout of one tile image (bytes), shared by both kernels.
template <int HD>
struct TileImg {
    static constexpr int NB = HD / kQK;
    static constexpr int MT = HD / 16;
    static constexpr int ROW = NB * kBlockBytes;
    static constexpr int KC_OFF = 0;
    static constexpr int KD_OFF = KC_OFF + 2 * NB * 64 * 8;
    static constexpr int VH_OFF = KD_OFF + NB * kKT * 4;
    static constexpr int VL_OFF = VH_OFF + MT * 64 * 16;
    static constexpr int BYTES = VL_OFF + MT * 64 * 16;
    static constexpr int CHUNKS = BYTES / 16;
    static_assert(BYTES % 16 == 0, "16-byte chunks");
};

// Key slot i (0..7) of lane group g in the MFMA k order used for P.V:
// keys 4g..4g+3 then 16+4g..16+4g+3 (the rows a lane holds of S^T).
__device__ __forceinline__ int perm_key(int g, int i) { return i < 4 ? 4 * g + i : 12 + 4 * g + i; }

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    v2bf v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
// fp32 values of the two bf16 halves of a pair (exact).
__device__ __forceinline__ float bf16_lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi_f(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
// bf16 hi | lo parts of four pairs of values.
__device__ __forceinline__ void split_bf16(const float (&x)[8], u32x4 &hi, u32x4 &lo) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t h = bf16_pair(x[2 * i], x[2 * i + 1]);
        hi[i] = h;
        lo[i] = bf16_pair(x[2 * i] - bf16_lo_f(h), x[2 * i + 1] - bf16_hi_f(h));
    }
}

__device__ __forceinline__ v8bf as_v8bf(u32x4 w) { return __builtin_bit_cast(v8bf, w); }

struct StageArgs {
    PagedView view;
    int seq;
    int kend;            // keys [0, kend)
    int n_tiles;         // tiles per kv head in the image buffer
    unsigned char *img;  // [n_kv][n_tiles][TileImg::BYTES]
    int contig_first;
    int contig_pages;
};

template <int HD>
__global__ __launch_bounds__(kThreads) void prefill_stage_kernel(StageArgs a) {
    using I = TileImg<HD>;
    constexpr int ROW = I::ROW;
    constexpr int RDW = kKT * ROW / 4;   // dwords of one tile's K (or V) rows
    __shared__ uint32_t raw[2][RDW];
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
    for (int i = tid; i < 2 * RDW; i += kThreads) {
        const int kv = i / RDW, rem = i % RDW;
        const int t = rem / (ROW / 4), w = rem % (ROW / 4);
        const int p = kt * kKT + t;
        const int pg = page[t / kPage];
        uint32_t x = 0;
        if (p < a.kend && pg >= 0)
            x = *reinterpret_cast<const uint32_t *>(head_run_ptr(v, pg, kvh) + kv * v.kv_chunk +
                                                    (p % kPage) * ROW + w * 4);
        raw[kv][rem] = x;
    }
    __syncthreads();
    const unsigned char *rk = reinterpret_cast<const unsigned char *>(raw[0]);
    const unsigned char *rv = reinterpret_cast<const unsigned char *>(raw[1]);
    unsigned char *out = a.img + ((size_t)kvh * a.n_tiles + kt) * I::BYTES;
    // K codes: entry (mt, b, lane) = key mt*16 + lane%16, block b, bytes 8*(lane/16)..
    for (int e = tid; e < 2 * I::NB * 64; e += kThreads) {
        const int mt = e / (I::NB * 64), b = (e / 64) % I::NB, ln = e % 64;
        const int off = (mt * 16 + (ln & 15)) * ROW + b * kBlockBytes + 4 + 8 * (ln >> 4);
        const u32x2 c = {*reinterpret_cast<const uint32_t *>(rk + off),
                         *reinterpret_cast<const uint32_t *>(rk + off + 4)};
        *reinterpret_cast<u32x2 *>(out + I::KC_OFF + e * 8) = c;
    }
    // K scales [block][key]
    for (int e = tid; e < I::NB * kKT; e += kThreads) {
        const int b = e / kKT, key = e % kKT;
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

template <int HD, int G, int NJ>
struct PShape {
    using I = TileImg<HD>;
    static constexpr int NB = I::NB;
    static constexpr int RW = 64 * NJ;             // (query, head) rows per work-group
    static constexpr int QB = RW / G;              // query tokens per work-group
    static constexpr int QT = QB / 16;             // query tiles per head
    static constexpr int MT = I::MT;               // output column tiles
    static constexpr int QCS = HD + 8;             // LDS stride of a q code row
    static constexpr int LOADS = (I::CHUNKS + kThreads - 1) / kThreads;
    static constexpr int Q_BYTES = RW * QCS + RW * NB * 4;
    static_assert(RW % G == 0 && QB % 16 == 0, "whole query tiles");
    static_assert(Q_BYTES <= 2 * I::BYTES, "q staging fits the tile buffers");
};

struct PrefillArgs {
    int pos0;
    int n;
    const float *q;      // [n][n_q_heads][hd], pre-RoPE if cos_t
    const float *cos_t;  // [n][hd/2] or null
    const float *sin_t;
    float *out;          // [n][n_q_heads][hd]
    int n_q_heads;
    float scale;
    int n_tiles;         // tiles per kv head in the image buffer
    const unsigned char *img;
};

// Quantize the 32-value block spread over this lane's 32-lane group and
// store its scale and codes separately (quantize_row_q8, kernel/quant_x.c:12-33).
__device__ __forceinline__ void quantize_split32(float x, float *d_out, unsigned char *codes) {
    const int lane = threadIdx.x & 31;
    const float d = quant_scale(block_amax32(x));
    const uint32_t word = pack_codes4(quant_code(x, quant_inverse(d)));
    if (lane == 0) *d_out = d;
    if ((lane & 3) == 0) *reinterpret_cast<uint32_t *>(codes + lane) = word;
}

template <int HD, int G, int NJ>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(PrefillArgs a) {
    using S = PShape<HD, G, NJ>;
    using I = TileImg<HD>;
    constexpr int NB = S::NB;
    __shared__ __attribute__((aligned(16))) unsigned char tile[2][I::BYTES];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l16 = lane & 15;
    const int lg = lane >> 4;
    const int kvh = blockIdx.y;
    const int qblocks = (a.n + S::QB - 1) / S::QB;
    const int i0 = (qblocks - 1 - (int)blockIdx.x) * S::QB;   // heaviest blocks first
    const int i_end = min(i0 + S::QB, a.n);
    const int kend = a.pos0 + i_end;                          // keys [0, kend)
    const int n_tiles = (kend + kKT - 1) / kKT;

    // ---- q rows of this wave: RoPE + quantize_row_q8 into LDS
    unsigned char *qc = tile[0];
    float *qd = reinterpret_cast<float *>(tile[0] + S::RW * S::QCS);
    for (int pass = 0; pass < 8 * NJ * NB; pass++) {
        const int blk = pass * 2 + (lane >> 5);          // block of the wave's rows
        const int r = wave * 16 * NJ + blk / NB;         // row: tile r/16, query r%16
        const int b = blk % NB;
        const int nt = r >> 4;
        const int g = nt / S::QT;
        const int qi = i0 + (nt % S::QT) * 16 + (r & 15);
        float x = 0.0f;
        if (qi < a.n) {
            const float *head = a.q + ((size_t)qi * a.n_q_heads + (size_t)kvh * G + g) * HD;
            const float *ct = a.cos_t ? a.cos_t + (size_t)qi * (HD / 2) : nullptr;
            const float *st = a.sin_t ? a.sin_t + (size_t)qi * (HD / 2) : nullptr;
            x = rope_elem(head, b * kQK + (lane & 31), HD, ct, st);
        }
        quantize_split32(x, qd + r * NB + b, qc + r * S::QCS + b * kQK);
    }
    __syncthreads();

    // ---- per-lane operands of the wave's query tiles
    long qb[NJ][NB];      // B operand: 8 codes of query l16, block b, k 8*lg..
    float qdp[NJ][NB];    // its scale * softmax scale * log2(e)
    int qpos[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int r = (wave * NJ + j) * 16 + l16;
        const int nt = r >> 4;
        int qi = i0 + (nt % S::QT) * 16 + l16;
        qi = qi < a.n ? qi : a.n - 1;
        qpos[j] = a.pos0 + qi;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            qb[j][b] = *reinterpret_cast<const long *>(qc + r * S::QCS + b * kQK + 8 * lg);
            qdp[j][b] = qd[r * NB + b] * (a.scale * kLog2e);
        }
    }
    __syncthreads();   // the q area is reused by the tile buffers below

    // ---- tile streaming: 16-byte chunks, one tile ahead in registers
    const unsigned char *img = a.img + (size_t)kvh * a.n_tiles * I::BYTES;
    u32x4 stg[S::LOADS];
    auto load_tile = [&](int kt) {
        const unsigned char *src = img + (size_t)kt * I::BYTES;
#pragma unroll
        for (int i = 0; i < S::LOADS; i++) {
            const int c = tid + kThreads * i;
            if (c < I::CHUNKS) stg[i] = *reinterpret_cast<const u32x4 *>(src + c * 16);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < S::LOADS; i++) {
            const int c = tid + kThreads * i;
            if (c < I::CHUNKS) *reinterpret_cast<u32x4 *>(tile[buf] + c * 16) = stg[i];
        }
    };

    // ---- the key loop
    v4f o[S::MT][NJ];
#pragma unroll
    for (int m = 0; m < S::MT; m++)
#pragma unroll
        for (int j = 0; j < NJ; j++) o[m][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float mrow[NJ], lsum[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        mrow[j] = -INFINITY;
        lsum[j] = 0.0f;
    }

    load_tile(0);
    for (int kt = 0; kt < n_tiles; kt++) {
        const int buf = kt & 1;
        store_tile(buf);
        if (kt + 1 < n_tiles) load_tile(kt + 1);
        __syncthreads();
        const unsigned char *T = tile[buf];

        // S^T = K . Q^T for keys [32kt, 32kt+32) x the wave's queries
        v4f s[2][NJ];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int j = 0; j < NJ; j++) s[mt][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < NB; b++) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const long ka = *reinterpret_cast<const long *>(T + I::KC_OFF + ((mt * NB + b) * 64 + lane) * 8);
                const v4f kdv = *reinterpret_cast<const v4f *>(T + I::KD_OFF + (b * kKT + mt * 16 + 4 * lg) * 4);
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    const v4i acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka, qb[j][b], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) s[mt][j][r] = fmaf((float)acc[r], qdp[j][b] * kdv[r], s[mt][j][r]);
                }
            }
        }

        // causal mask, online softmax, P split into bf16 hi | lo (B operands)
        const int k0 = kt * kKT;
        u32x4 phi[NJ], plo[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (k0 + kKT - 1 > a.pos0 + i0) {   // tiles past the block's first query need the mask
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int kp = k0 + mt * 16 + 4 * lg + r;
                        s[mt][j][r] = kp > qpos[j] ? -INFINITY : s[mt][j][r];
                    }
            }
            float mx = fmaxf(fmaxf(fmaxf(s[0][j][0], s[0][j][1]), fmaxf(s[0][j][2], s[0][j][3])),
                             fmaxf(fmaxf(s[1][j][0], s[1][j][1]), fmaxf(s[1][j][2], s[1][j][3])));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mnew = fmaxf(mrow[j], mx);
            const float corr = __builtin_amdgcn_exp2f(mrow[j] - mnew);
            mrow[j] = mnew;
            float p[8];
            float ps = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    p[mt * 4 + r] = __builtin_amdgcn_exp2f(s[mt][j][r] - mnew);
                    ps += p[mt * 4 + r];
                }
            lsum[j] = lsum[j] * corr + ps;
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f) != 0) {
#pragma unroll
                for (int m = 0; m < S::MT; m++) o[m][j] *= corr;
            }
            split_bf16(p, phi[j], plo[j]);
        }

        // O^T += V'^T . P^T
#pragma unroll
        for (int m = 0; m < S::MT; m++) {
            const v8bf ahi = as_v8bf(*reinterpret_cast<const u32x4 *>(T + I::VH_OFF + (m * 64 + lane) * 16));
            const v8bf alo = as_v8bf(*reinterpret_cast<const u32x4 *>(T + I::VL_OFF + (m * 64 + lane) * 16));
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                o[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, as_v8bf(phi[j]), o[m][j], 0, 0, 0);
                o[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, as_v8bf(plo[j]), o[m][j], 0, 0, 0);
                o[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, as_v8bf(phi[j]), o[m][j], 0, 0, 0);
            }
        }
    }

    // ---- normalise and store: lane holds columns 16m + 4lg .. +3 of query l16
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        float l = lsum[j];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const float inv = 1.0f / l;
        const int nt = wave * NJ + j;
        const int g = nt / S::QT;
        const int qi = i0 + (nt % S::QT) * 16 + l16;
        if (qi < a.n) {
            float *orow = a.out + ((size_t)qi * a.n_q_heads + (size_t)kvh * G + g) * HD;
#pragma unroll
            for (int m = 0; m < S::MT; m++)
                *reinterpret_cast<v4f *>(orow + m * 16 + 4 * lg) = o[m][j] * inv;
        }
    }
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

template <int HD, int G, int NJ>
hipError_t launch_hd_g(const PrefillArgs &a, int n_kv_heads, hipStream_t s) {
    using S = PShape<HD, G, NJ>;
    const int qblocks = (a.n + S::QB - 1) / S::QB;
    hipLaunchKernelGGL((prefill_kernel<HD, G, NJ>), dim3(qblocks, n_kv_heads), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const TqPrefillArgs &t, const PrefillArgs &a, int g, hipStream_t s) {
    StageArgs st;
    st.view = t.view;
    st.seq = t.seq;
    st.kend = t.pos0 + t.n;
    st.n_tiles = a.n_tiles;
    st.img = t.img;
    st.contig_first = t.contig_first;
    st.contig_pages = t.contig_pages;
    hipLaunchKernelGGL((prefill_stage_kernel<HD>), dim3(a.n_tiles, t.n_kv_heads), dim3(kThreads), 0, s, st);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const bool wide = prefill_rows(g) == 128;
    switch (g) {
        case 1: return wide ? launch_hd_g<HD, 1, 2>(a, t.n_kv_heads, s) : launch_hd_g<HD, 1, 1>(a, t.n_kv_heads, s);
        case 2: return wide ? launch_hd_g<HD, 2, 2>(a, t.n_kv_heads, s) : launch_hd_g<HD, 2, 1>(a, t.n_kv_heads, s);
        case 4: return wide ? launch_hd_g<HD, 4, 2>(a, t.n_kv_heads, s) : launch_hd_g<HD, 4, 1>(a, t.n_kv_heads, s);
        case 8: return launch_hd_g<HD, 8, 2>(a, t.n_kv_heads, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool tq_prefill_mfma_supported(int head_dim, int group, int kend) {
    const bool hd_ok = head_dim == 64 || head_dim == 128;
    const bool g_ok = group == 1 || group == 2 || group == 4 || group == 8;
    return hd_ok && g_ok && kend > 0 && kend <= kMaxPrefillKeys;
}

size_t tq_prefill_image_bytes(int head_dim, int n_kv_heads, int kend) {
    const size_t tiles = (size_t)(kend + kKT - 1) / kKT;
    const size_t per = head_dim == 64 ? TileImg<64>::BYTES : TileImg<128>::BYTES;
    return tiles * per * (size_t)n_kv_heads;
}

hipError_t tq_launch_prefill(const TqPrefillArgs &t, hipStream_t s) {
    const int g = t.n_q_heads / t.n_kv_heads;
    if (!tq_prefill_mfma_supported(t.head_dim, g, t.pos0 + t.n) || !t.img) return hipErrorInvalidValue;
    PrefillArgs a;
    a.pos0 = t.pos0;
    a.n = t.n;
    a.q = t.q;
    a.cos_t = t.cos_t;
    a.sin_t = t.sin_t;
    a.out = t.out;
    a.n_q_heads = t.n_q_heads;
    a.scale = t.scale;
    a.n_tiles = (t.pos0 + t.n + kKT - 1) / kKT;
    a.img = t.img;
    return t.head_dim == 64 ? launch_hd<64>(t, a, g, s) : launch_hd<128>(t, a, g, s);
}
