// decode.hip — attend_q8 (model/attention_layer.c:125-150) on the paged cache.
//
// Grid (split, kv head, query).  A 256-thread work-group owns tokens
// [split*split_tokens, min(len, (split+1)*split_tokens)) of one kv head and
// all G = n_q_heads/n_kv_heads query heads reading it, so every K/V byte is
// fetched once per step.  It walks its range in sub-chunks of TSUB = 256/nb
// tokens (18,432 bytes of K+V per sub-chunk at any head_dim):
//
//   * the next sub-chunk's pages are loaded into registers with 16-byte
//     coalesced loads while the current one is processed from LDS;
//   * scores: thread (token, block) computes the exact int32 block dot for all
//     G heads off one K block (v_dot4_i32_i8), scales by qd*kd and the
//     token's blocks are summed in block order, giving scores bit-identical
//     to attn_scores_q8_scalar (model/attn_q8.c:17-34);
//   * online softmax per head: one wave per head, running max/sum in
//     registers, wave shuffles for the reductions;
//   * P.V: thread (4 columns, token subset) accumulates all G heads, with
//     o *= exp(m_old - m_new) at each sub-chunk.
//
// With more than one split the work-group writes (o, m, l) partials and a
// second kernel combines them in split order, so the result never depends on
// scheduling.  In step mode (k_new != null) the work-group owning position
// len-1 first quantizes the new token's K (after RoPE) and V exactly as
// store_kv does, writes them to the cache and patches them into its LDS copy,
// so the append and the attention over it are one launch.
#include "tq_common.hpp"

namespace {

using namespace tq;

__device__ __forceinline__ float wmax64(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ float wsum64(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int HD, int G>
struct DecodeShape {
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
    static constexpr int KV_BYTES = 2 * TSUB * ROW;
    static constexpr int RED_BYTES = NTS * G * HD * 4;
    static constexpr int SMEM = KV_BYTES > RED_BYTES ? KV_BYTES : RED_BYTES;
    static_assert(NB * TSUB == kThreads, "one (token, block) pair per thread");
    static_assert(TSUB % kPage == 0, "sub-chunks are whole pages");
    static_assert(NTS * NCG == kThreads, "one (column group, subset) per thread");
};

// Issue the 16-byte loads of sub-chunk [c0, c0+TSUB): vector vi of the
// sub-chunk is page vi / VEC_PER_PAGE, byte 16*(vi % VEC_PER_PAGE) of that
// page's K+V run for kv head kvh.  Pages at or past t_end are not touched.
template <typename S>
__device__ __forceinline__ void load_sub(u32x4 (&pf)[S::VPT], const PagedView &view, int seq, int kvh,
                                         int c0, int t_end, int tid) {
#pragma unroll
    for (int i = 0; i < S::VPT; i++) {
        const int vi = tid + i * kThreads;
        if (vi < S::NVEC) {
            const int p = vi / S::VEC_PER_PAGE;
            const int w = vi - p * S::VEC_PER_PAGE;
            const int tok0 = c0 + p * kPage;
            if (tok0 < t_end) {
                const int phys = phys_page(view, seq, tok0 / kPage);
                if (phys >= 0) pf[i] = *reinterpret_cast<const u32x4 *>(head_run_ptr(view, phys, kvh) + 16 * w);
            }
        }
    }
}

// Scatter the prefetched vectors into LDS: K rows of the sub-chunk contiguous
// in kbuf, V rows in vbuf ([TSUB][nb] block_q8 each).
template <typename S>
__device__ __forceinline__ void store_sub(const u32x4 (&pf)[S::VPT], unsigned char *kbuf, unsigned char *vbuf,
                                          int tid) {
#pragma unroll
    for (int i = 0; i < S::VPT; i++) {
        const int vi = tid + i * kThreads;
        if (vi < S::NVEC) {
            const int p = vi / S::VEC_PER_PAGE;
            const int byte = 16 * (vi - p * S::VEC_PER_PAGE);
            unsigned char *dst = byte < S::CHUNK ? kbuf + p * S::CHUNK + byte : vbuf + p * S::CHUNK + (byte - S::CHUNK);
            *reinterpret_cast<u32x4 *>(dst) = pf[i];
        }
    }
}

template <int HD, int G>
__global__ __launch_bounds__(256) void decode_kernel(TqDecodeArgs a) {
    using S = DecodeShape<HD, G>;
    constexpr int NB = S::NB, ROW = S::ROW, TSUB = S::TSUB, CHUNK = S::CHUNK;

    __shared__ __align__(16) unsigned char smem[S::SMEM];
    __shared__ __align__(16) unsigned char qblk[G * ROW];
    __shared__ __align__(16) unsigned char newrow[2 * ROW];
    __shared__ __align__(16) float sp[TSUB * G];
    __shared__ float corr[G];
    __shared__ float mfin[G];
    __shared__ float lfin[G];
    unsigned char *kbuf = smem;
    unsigned char *vbuf = smem + TSUB * ROW;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, kvh = blockIdx.y, qi = blockIdx.z;
    const PagedView &view = a.view;
    const int seq = a.seq_of ? a.seq_of[qi] : a.seq_const;
    const int len = a.len_of ? a.len_of[qi] + a.len_plus : a.pos0 + qi + 1;
    const int t_begin = split * a.split_tokens;
    if (len <= 0 || t_begin >= len) return;
    const int t_end = min(len, t_begin + a.split_tokens);
    const int pos_new = len - 1;
    const bool owns_new = a.k_new != nullptr && pos_new >= t_begin && pos_new < t_end;

    const float *ct = a.cos_t ? a.cos_t + (size_t)qi * (HD / 2) : nullptr;
    const float *st = a.sin_t ? a.sin_t + (size_t)qi * (HD / 2) : nullptr;

    // ---- q rows of this kv group: RoPE, quantize (exact) into LDS ----------
    {
        const float *qg = a.q + ((size_t)qi * a.n_q_heads + (size_t)kvh * G) * HD;
        for (int e = tid; e < G * HD; e += kThreads) {
            const int gi = e / HD, col = e - gi * HD;
            const float x = rope_elem(qg + (size_t)gi * HD, col, HD, ct, st);
            quantize_store32(x, qblk + gi * ROW + (col >> 5) * kBlockBytes);
        }
    }
    // ---- step mode: the new token's K (RoPE) and V rows ----------------------
    if (owns_new) {
        const size_t off = ((size_t)qi * a.n_kv_heads + kvh) * HD;
        for (int e = tid; e < 2 * HD; e += kThreads) {
            const bool is_v = e >= HD;
            const int col = is_v ? e - HD : e;
            const float x = is_v ? a.v_new[off + col] : rope_elem(a.k_new + off, col, HD, ct, st);
            quantize_store32(x, newrow + (is_v ? ROW : 0) + (col >> 5) * kBlockBytes);
        }
    }
    __syncthreads();
    if (owns_new) {
        const int phys = phys_page(view, seq, pos_new / kPage);
        if (phys >= 0 && tid < 2 * (ROW / 4)) {
            const bool is_v = tid >= ROW / 4;
            const int w = is_v ? tid - ROW / 4 : tid;
            unsigned char *dst = head_run_ptr(view, phys, kvh) + (is_v ? CHUNK : 0) +
                                 (pos_new % kPage) * ROW + 4 * w;
            *reinterpret_cast<uint32_t *>(dst) =
                *reinterpret_cast<const uint32_t *>(newrow + (is_v ? ROW : 0) + 4 * w);
        }
    }

    // ---- this thread's q blocks in registers (scores phase role) -------------
    const int my_t = tid / NB, my_b = tid % NB;
    int32_t qreg[G][8];
    float qd[G];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        const unsigned char *qb = qblk + gi * ROW + my_b * kBlockBytes;
        qd[gi] = *reinterpret_cast<const float *>(qb);
#pragma unroll
        for (int w = 0; w < 8; w++) qreg[gi][w] = *reinterpret_cast<const int32_t *>(qb + 4 + 4 * w);
    }

    // P.V role
    const int cg = tid % S::NCG, ts = tid / S::NCG;
    const int pv_b = cg >> 3, pv_w = cg & 7;
    float o[G][4];
#pragma unroll
    for (int gi = 0; gi < G; gi++)
#pragma unroll
        for (int c = 0; c < 4; c++) o[gi][c] = 0.0f;

    // softmax role: wave w owns heads w, w+4
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.0f, 0.0f};

    u32x4 pf[S::VPT];
    const int n_sub = (t_end - t_begin + TSUB - 1) / TSUB;
    load_sub<S>(pf, view, seq, kvh, t_begin, t_end, tid);
    for (int sub = 0; sub < n_sub; sub++) {
        const int c0 = t_begin + sub * TSUB;
        store_sub<S>(pf, kbuf, vbuf, tid);
        __syncthreads();
        if (owns_new && pos_new >= c0 && pos_new < c0 + TSUB) {
            const int r = pos_new - c0;
            if (tid < 2 * (ROW / 4)) {
                const bool is_v = tid >= ROW / 4;
                const int w = is_v ? tid - ROW / 4 : tid;
                unsigned char *dst = (is_v ? vbuf : kbuf) + r * ROW + 4 * w;
                *reinterpret_cast<uint32_t *>(dst) =
                    *reinterpret_cast<const uint32_t *>(newrow + (is_v ? ROW : 0) + 4 * w);
            }
            __syncthreads();
        }
        if (sub + 1 < n_sub) load_sub<S>(pf, view, seq, kvh, c0 + TSUB, t_end, tid);

        // ---- scores ---------------------------------------------------------
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
                float acc = 0.0f;
                if constexpr (NB == 1) {
                    acc += x;
                } else {
                    const int base = lane - my_b;
#pragma unroll
                    for (int j = 0; j < NB; j++) acc += __shfl(x, base + j, 64);
                }
                if (my_b == 0) sp[my_t * G + gi] = valid ? acc * a.scale : -INFINITY;
            }
        }
        __syncthreads();

        // ---- online softmax, one wave per head --------------------------------
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int gi = wave + 4 * r;
            if (gi < G) {
                float mloc = -INFINITY;
                for (int t = lane; t < TSUB; t += 64) mloc = fmaxf(mloc, sp[t * G + gi]);
                mloc = wmax64(mloc);
                const float m_new = fmaxf(m_run[r], mloc);
                const float c = expf(m_run[r] - m_new);
                float lsum = 0.0f;
                for (int t = lane; t < TSUB; t += 64) {
                    const float p = expf(sp[t * G + gi] - m_new);
                    sp[t * G + gi] = p;
                    lsum += p;
                }
                lsum = wsum64(lsum);
                l_run[r] = l_run[r] * c + lsum;
                m_run[r] = m_new;
                if (lane == 0) corr[gi] = c;
            }
        }
        __syncthreads();

        // ---- P.V ----------------------------------------------------------------
        {
#pragma unroll
            for (int gi = 0; gi < G; gi++) {
                const float c = corr[gi];
#pragma unroll
                for (int k = 0; k < 4; k++) o[gi][k] *= c;
            }
            for (int t = ts; t < TSUB; t += S::NTS) {
                if (c0 + t < t_end) {
                    const unsigned char *vb = vbuf + t * ROW + pv_b * kBlockBytes;
                    const float vd = *reinterpret_cast<const float *>(vb);
                    const uint32_t codes = *reinterpret_cast<const uint32_t *>(vb + 4 + 4 * pv_w);
                    const float f0 = (float)(int8_t)(codes & 0xFF);
                    const float f1 = (float)(int8_t)((codes >> 8) & 0xFF);
                    const float f2 = (float)(int8_t)((codes >> 16) & 0xFF);
                    const float f3 = (float)(int8_t)(codes >> 24);
#pragma unroll
                    for (int gi = 0; gi < G; gi++) {
                        const float av = sp[t * G + gi] * vd;
                        o[gi][0] += av * f0;
                        o[gi][1] += av * f1;
                        o[gi][2] += av * f2;
                        o[gi][3] += av * f3;
                    }
                }
            }
        }
        __syncthreads();
    }

    // ---- reduce the token subsets in a fixed order ------------------------------
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int gi = wave + 4 * r;
        if (gi < G && lane == 0) {
            mfin[gi] = m_run[r];
            lfin[gi] = l_run[r];
        }
    }
    float *red = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int gi = 0; gi < G; gi++)
        *reinterpret_cast<float4 *>(red + ((size_t)ts * G + gi) * HD + cg * 4) =
            make_float4(o[gi][0], o[gi][1], o[gi][2], o[gi][3]);
    __syncthreads();

    const bool direct = a.n_splits == 1;
    const size_t pstride = (size_t)G * (HD + 2);
    float *part = direct ? nullptr
                         : a.partials + (((size_t)qi * a.n_kv_heads + kvh) * a.n_splits + split) * pstride;
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int gi = idx / HD, j = idx - gi * HD;
        float acc = 0.0f;
        for (int s = 0; s < S::NTS; s++) acc += red[((size_t)s * G + gi) * HD + j];
        if (direct)
            a.out[((size_t)qi * a.n_q_heads + (size_t)kvh * G + gi) * HD + j] = acc / lfin[gi];
        else
            part[idx] = acc;
    }
    if (!direct && tid < G) {
        part[G * HD + tid] = mfin[tid];
        part[G * HD + G + tid] = lfin[tid];
    }
}

// One work-group per (q head, query): weights exp(m_s - M) over the valid
// splits, summed in split order.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ partials,
                                                      const int32_t *__restrict__ len_of,
                                                      int len_plus, int pos0,
                                                      float *__restrict__ out, int n_q_heads,
                                                      int n_kv_heads, int G, int HD,
                                                      int split_tokens, int n_splits) {
    const int h = blockIdx.x, qi = blockIdx.y;
    const int kvh = h / G, gi = h - kvh * G;
    const int len = len_of ? len_of[qi] + len_plus : pos0 + qi + 1;
    float *dst = out + ((size_t)qi * n_q_heads + h) * HD;
    if (len <= 0) {
        for (int j = threadIdx.x; j < HD; j += 256) dst[j] = 0.0f;
        return;
    }
    const int nvalid = min(n_splits, (len + split_tokens - 1) / split_tokens);
    const size_t pstride = (size_t)G * (HD + 2);
    const float *base = partials + ((size_t)qi * n_kv_heads + kvh) * n_splits * pstride;
    float M = -INFINITY;
    for (int s = 0; s < nvalid; s++) M = fmaxf(M, base[s * pstride + G * HD + gi]);
    float L = 0.0f;
    for (int s = 0; s < nvalid; s++)
        L += base[s * pstride + G * HD + G + gi] * expf(base[s * pstride + G * HD + gi] - M);
    for (int j = threadIdx.x; j < HD; j += 256) {
        float acc = 0.0f;
        for (int s = 0; s < nvalid; s++)
            acc += base[s * pstride + gi * HD + j] * expf(base[s * pstride + G * HD + gi] - M);
        dst[j] = acc / L;
    }
}

template <int HD, int G>
hipError_t launch_hd_g(const TqDecodeArgs &a, hipStream_t s) {
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

bool tq_decode_supported(int head_dim, int group) {
    const bool hd_ok = head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
    return hd_ok && group >= 1 && group <= 8;
}

hipError_t tq_launch_decode(const TqDecodeArgs &a, hipStream_t s) {
    if (a.n_q <= 0) return hipSuccess;
    const int g = a.n_q_heads / a.n_kv_heads;
    hipError_t e;
    switch (a.head_dim) {
        case 32: e = launch_hd<32>(a, g, s); break;
        case 64: e = launch_hd<64>(a, g, s); break;
        case 128: e = launch_hd<128>(a, g, s); break;
        case 256: e = launch_hd<256>(a, g, s); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || a.n_splits == 1) return e;
    hipLaunchKernelGGL(combine_kernel, dim3(a.n_q_heads, a.n_q), dim3(256), 0, s, a.partials, a.len_of,
                       a.len_plus, a.pos0, a.out, a.n_q_heads, a.n_kv_heads, g, a.head_dim, a.split_tokens, a.n_splits);
    return hipGetLastError();
}
