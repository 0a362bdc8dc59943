// kv_append.hip — store_kv, Q8 branch (model/attention_layer.c:66-90), fused
// with RoPE on K (rope_heads, :188), into the paged HBM cache.
//
// Two kernels, one result:
//   append_kernel      rows with their own (sequence, position) each: one
//                      work-group per (row, kv head), 2*head_dim threads, one
//                      value per thread, a 32-lane group per block.
//   append_run_kernel  a run of consecutive positions of one sequence (the
//                      prefill and bulk case): one work-group per (logical
//                      page, kv head).  Every thread issues all its 16-byte
//                      loads first, a 32-value block is quantized over 8
//                      lanes of 4 values, and the page's rows are assembled in
//                      LDS and written whole, only the rows of the run.
// Both quantize exactly as quantize_row_q8 does.  Rows whose position has no
// mapped page are skipped whole.
#include "tq_common.hpp"

namespace {

using namespace tq;

// One value per thread of row `row`, kv head kvh: K (after RoPE) then V,
// quantized by 32-lane groups into the cache at position pos.
__device__ __forceinline__ void append_row(const PagedView &view, int phys, int pos, int row, int kvh,
                                           const float *__restrict__ k, const float *__restrict__ v,
                                           const float *__restrict__ cos_t, const float *__restrict__ sin_t,
                                           int hd) {
    const int e = threadIdx.x;
    const bool is_v = e >= hd;
    const int col = is_v ? e - hd : e;
    const size_t head_off = ((size_t)row * view.n_kv_heads + kvh) * hd;
    float x;
    if (is_v) {
        x = v[head_off + col];
    } else {
        const float *c = cos_t ? cos_t + (size_t)row * (hd / 2) : nullptr;
        const float *s = sin_t ? sin_t + (size_t)row * (hd / 2) : nullptr;
        x = rope_elem(k + head_off, col, hd, c, s);
    }
    unsigned char *dst = head_run_ptr(view, phys, kvh) + (is_v ? view.kv_chunk : 0) +
                         (size_t)(pos % kPage) * view.row_bytes + (size_t)(col >> 5) * kBlockBytes;
    quantize_store32(x, dst);
}

__global__ __launch_bounds__(512) void append_kernel(PagedView view, const int32_t *__restrict__ seq_of,
                                                     const int32_t *__restrict__ pos_of,
                                                     const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     const float *__restrict__ cos_t,
                                                     const float *__restrict__ sin_t, int hd,
                                                     int seq_const, int pos0, unsigned *done,
                                                     unsigned done_seq) {
    const int row = blockIdx.x, kvh = blockIdx.y;
    const int seq = seq_of ? seq_of[row] : seq_const;
    const int pos = pos_of ? pos_of[row] : pos0 + row;
    const int phys = pos < 0 ? -1 : phys_page(view, seq, pos / kPage);
    if (phys >= 0) append_row(view, phys, pos, row, kvh, k, v, cos_t, sin_t, hd);
    if (done) {
        // completion flag of (row, kv head) for a host that waits on memory: the
        // inputs are read and every store of the work-group is acknowledged
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_store(done + (size_t)row * view.n_kv_heads + kvh, done_seq, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int HD>
__global__ __launch_bounds__(kThreads) void append_run_kernel(PagedView view, int seq, int pos0, int n,
                                                             const float *__restrict__ k,
                                                             const float *__restrict__ v,
                                                             const float *__restrict__ cos_t,
                                                             const float *__restrict__ sin_t) {
    constexpr int HALF = HD / 2;
    constexpr int CPR = HD / 8;                          // tasks per (row, K|V): float4 c of each half
    constexpr int ROW = HD / kQK * kBlockBytes;          // bytes of a row
    constexpr int TASKS = kPage * 2 * CPR;
    constexpr int TPT = (TASKS + kThreads - 1) / kThreads;
    constexpr int CB = ROW % 16 == 0 ? 16 : 8;           // bytes per copy of a row
    static_assert(CPR % 8 == 0 && ROW % CB == 0, "whole blocks per half, whole copies per row");
    __shared__ __align__(16) unsigned char run[2][kPage][ROW];   // the page's K rows | V rows
    const int lp = pos0 / kPage + (int)blockIdx.x, kvh = blockIdx.y;
    const int p_lo = max(pos0, lp * kPage), p_hi = min(pos0 + n, lp * kPage + kPage);
    const int phys = phys_page(view, seq, lp);
    if (phys < 0) return;
    const int tid = threadIdx.x;
    const bool rot = cos_t != nullptr;

    v4f xl[TPT], xu[TPT], cs[TPT], sn[TPT];
#pragma unroll
    for (int t = 0; t < TPT; t++) {
        const int task = tid + kThreads * t;
        const int r = task / (2 * CPR), kv = (task / CPR) & 1, c = task % CPR;
        const int pos = lp * kPage + r;
        xl[t] = xu[t] = cs[t] = sn[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (task < TASKS && pos >= p_lo && pos < p_hi) {
            const size_t row = (size_t)(pos - pos0);
            const float *src = (kv ? v : k) + (row * view.n_kv_heads + kvh) * HD;
            xl[t] = *reinterpret_cast<const v4f *>(src + 4 * c);
            xu[t] = *reinterpret_cast<const v4f *>(src + HALF + 4 * c);
            if (!kv && rot) {
                cs[t] = *reinterpret_cast<const v4f *>(cos_t + row * HALF + 4 * c);
                sn[t] = *reinterpret_cast<const v4f *>(sin_t + row * HALF + 4 * c);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TPT; t++) {
        const int task = tid + kThreads * t;
        if (TPT * kThreads > TASKS && task >= TASKS) break;   // whole 8-lane groups
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
        unsigned char *row = run[kv][r];
        const bool leader = (c & 7) == 0;
        const int bl = (4 * c) / kQK, bu = (HALF + 4 * c) / kQK;
        quantize8x4(lo, reinterpret_cast<float *>(row + bl * kBlockBytes), row + bl * kBlockBytes + 4 + (4 * c) % kQK,
                    leader);
        quantize8x4(up, reinterpret_cast<float *>(row + bu * kBlockBytes), row + bu * kBlockBytes + 4 + (4 * c) % kQK,
                    leader);
    }
    __syncthreads();
    // the run's rows of this page, whole rows in CB-byte copies
    unsigned char *dst = head_run_ptr(view, phys, kvh);
    constexpr int PER_ROW = ROW / CB;
    for (int ch = tid; ch < 2 * kPage * PER_ROW; ch += kThreads) {
        const int kv = ch / (kPage * PER_ROW), r = (ch / PER_ROW) % kPage, j = ch % PER_ROW;
        const int pos = lp * kPage + r;
        if (pos < p_lo || pos >= p_hi) continue;
        unsigned char *g = dst + (kv ? view.kv_chunk : 0) + (size_t)r * ROW + CB * j;
        if constexpr (CB == 16)
            *reinterpret_cast<u32x4 *>(g) = *reinterpret_cast<const u32x4 *>(run[kv][r] + CB * j);
        else
            *reinterpret_cast<u32x2 *>(g) = *reinterpret_cast<const u32x2 *>(run[kv][r] + CB * j);
    }
}

}  // namespace

hipError_t tq_launch_append(const PagedView &view, int n_rows, const int32_t *seq,
                            const int32_t *pos, int seq_const, int pos0, const float *k,
                            const float *v, const float *c, const float *sn, int hd,
                            hipStream_t s, unsigned *done, unsigned done_seq) {
    if (n_rows <= 0) return hipSuccess;
    // a run of one sequence with 16-byte aligned inputs: a work-group per page
    // (completion flags: one work-group per row)
    const bool aligned = (((uintptr_t)k | (uintptr_t)v | (uintptr_t)c | (uintptr_t)sn) & 15) == 0;
    if (!done && !seq && !pos && aligned && (hd == 64 || hd == 128 || hd == 256) && pos0 >= 0) {
        const int pages = (pos0 + n_rows - 1) / kPage - pos0 / kPage + 1;
        const dim3 grid(pages, view.n_kv_heads);
        switch (hd) {
            case 64: hipLaunchKernelGGL(append_run_kernel<64>, grid, dim3(kThreads), 0, s, view, seq_const, pos0, n_rows, k, v, c, sn); break;
            case 128: hipLaunchKernelGGL(append_run_kernel<128>, grid, dim3(kThreads), 0, s, view, seq_const, pos0, n_rows, k, v, c, sn); break;
            default: hipLaunchKernelGGL(append_run_kernel<256>, grid, dim3(kThreads), 0, s, view, seq_const, pos0, n_rows, k, v, c, sn); break;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(append_kernel, dim3(n_rows, view.n_kv_heads), dim3(2 * hd), 0, s, view, seq,
                       pos, k, v, c, sn, hd, seq_const, pos0, done, done_seq);
    return hipGetLastError();
}
