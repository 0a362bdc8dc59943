// kv_append.hip — store_kv, Q8 branch (model/attention_layer.c:66-90), fused
// with RoPE on K (rope_heads, :188), into the paged HBM cache.
//
// One work-group per (row, kv head), 2*head_dim threads: threads [0, hd) own
// the K row, [hd, 2hd) the V row, one value each; each 32-lane group
// quantizes one block (exact quantize_row_q8) and writes it as a 36-byte
// block_q8 with dword stores.  Rows whose position has no mapped page are
// skipped whole.
#include "tq_common.hpp"

namespace {

using namespace tq;

__global__ __launch_bounds__(512) void append_kernel(PagedView view, const int32_t *__restrict__ seq_of,
                                                     const int32_t *__restrict__ pos_of,
                                                     const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     const float *__restrict__ cos_t,
                                                     const float *__restrict__ sin_t, int hd,
                                                     int seq_const, int pos0) {
    const int row = blockIdx.x, kvh = blockIdx.y;
    const int seq = seq_of ? seq_of[row] : seq_const;
    const int pos = pos_of ? pos_of[row] : pos0 + row;
    if (pos < 0) return;
    const int phys = phys_page(view, seq, pos / kPage);
    if (phys < 0) return;

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

}  // namespace

hipError_t tq_launch_append(const PagedView &view, int n_rows, const int32_t *seq,
                            const int32_t *pos, int seq_const, int pos0, const float *k,
                            const float *v, const float *c, const float *sn, int hd,
                            hipStream_t s) {
    if (n_rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(append_kernel, dim3(n_rows, view.n_kv_heads), dim3(2 * hd), 0, s, view, seq,
                       pos, k, v, c, sn, hd, seq_const, pos0);
    return hipGetLastError();
}
