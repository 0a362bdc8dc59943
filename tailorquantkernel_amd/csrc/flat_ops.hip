// flat_ops.hip — the reference's kernel-level Q8 attention ops on flat
// block_q8 arrays in device memory: quantize_row_q8, rope_apply,
// attn_scores_q8, attn_accum_q8, softmax.
//
// These keep the reference's per-element operation order, so quantize, RoPE,
// scores and accum are bit-exact with the scalar code (model/attn_q8.c:17-54,
// kernel/quant_x.c:12-33, model/rope.c:14-22); softmax uses a parallel sum and
// the device expf, within tolerance of model/softmax.c:4-23.
#include "tq_common.hpp"

namespace {

using namespace tq;

// One 32-lane group per block; 8 blocks per 256-thread work-group.
__global__ __launch_bounds__(256) void quantize_kernel(const float *__restrict__ x,
                                                       unsigned char *__restrict__ out,
                                                       int nblocks) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int blk = e >> 5;
    if (blk >= nblocks) return;  // whole 32-lane groups leave together
    quantize_store32(x[e], out + (size_t)blk * kBlockBytes);
}

// The same with 8 lanes x 4 values per block: one float4 load and one dword
// of codes per lane (16-byte aligned x).  Whole 8-lane groups stay together
// (256 is a multiple of 8), as quantize8x4's DPP steps need.
// scales null: block_q8 blocks at out.  Else the split layout the batched
// matmul reads, block-major over the n = nblocks / nb rows: for block b of
// row t, codes 0-15 at out + ((2b) n + t) 16, codes 16-31 at
// out + ((2b + 1) n + t) 16, the scale at scales[b n + t].
__global__ __launch_bounds__(256) void quantize8_kernel(const float *__restrict__ x, unsigned char *__restrict__ out,
                                                        long nblocks, float *__restrict__ scales, int nb) {
    const long k = (long)blockIdx.x * 256 + threadIdx.x;
    const long g = k >> 3;
    if (g >= nblocks) return;
    const int e = (int)(k & 7);
    if (scales) {
        // block-major: consecutive 8-lane groups take consecutive rows of one
        // block, so a wave's code stores are two contiguous 128-byte runs
        const long n = nblocks / nb, b = g / n, t = g - b * n;
        const float4 v = *reinterpret_cast<const float4 *>(x + (t * nb + b) * kQK + 4 * e);
        const float xv[4] = {v.x, v.y, v.z, v.w};
        quantize8x4(xv, scales + b * n + t, out + ((2 * b + (e >> 2)) * n + t) * 16 + 4 * (e & 3), e == 0);
        return;
    }
    const long tb = g;
    const float4 v = *reinterpret_cast<const float4 *>(x + tb * kQK + 4 * e);
    const float xv[4] = {v.x, v.y, v.z, v.w};
    {
        unsigned char *blk = out + tb * kBlockBytes;
        quantize8x4(xv, reinterpret_cast<float *>(blk), blk + 4 + 4 * e, e == 0);
    }
}

// One thread per (head, pair i < hd/2): reads both halves, writes both.
__global__ __launch_bounds__(256) void rope_kernel(float *__restrict__ x, int n_heads, int hd,
                                                   const float *__restrict__ c,
                                                   const float *__restrict__ s) {
    const int half = hd >> 1;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_heads * half) return;
    const int h = idx / half, i = idx - h * half;
    float *head = x + (size_t)h * hd;
    const float x0 = head[i], x1 = head[i + half];
    head[i] = rope_lower(x0, x1, c[i], s[i]);
    head[i + half] = rope_upper(x0, x1, c[i], s[i]);
}

__device__ __forceinline__ int32_t dot32(const unsigned char *a, const unsigned char *b) {
    const int32_t *qa = reinterpret_cast<const int32_t *>(a + 4);
    const int32_t *qb = reinterpret_cast<const int32_t *>(b + 4);
    int32_t acc = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) acc = __builtin_amdgcn_sdot4(qa[w], qb[w], acc, false);
    return acc;
}

// One thread per (token t, head gi): model/attn_q8.c:17-34 order.
__global__ __launch_bounds__(256) void scores_kernel(const unsigned char *__restrict__ q, int g,
                                                     const unsigned char *__restrict__ k, int n,
                                                     int nb, float scale,
                                                     float *__restrict__ scores,
                                                     size_t stride) {
#pragma clang fp contract(off)
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)n * g) return;
    const int t = (int)(idx / g), gi = (int)(idx - (long)t * g);
    const unsigned char *kr = k + (size_t)t * nb * kBlockBytes;
    const unsigned char *qr = q + (size_t)gi * nb * kBlockBytes;
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const unsigned char *kb = kr + b * kBlockBytes;
        const unsigned char *qb = qr + b * kBlockBytes;
        const int32_t dot = dot32(qb, kb);
        const float dd = *reinterpret_cast<const float *>(qb) * *reinterpret_cast<const float *>(kb);
        acc += (float)dot * dd;
    }
    scores[(size_t)gi * stride + t] = acc * scale;
}

// One thread per (head gi, column j), tokens in order: model/attn_q8.c:36-54.
__global__ __launch_bounds__(256) void accum_kernel(const float *__restrict__ w, size_t w_stride,
                                                    int g, const unsigned char *__restrict__ v,
                                                    int n, int nb, float *__restrict__ out,
                                                    size_t out_stride) {
#pragma clang fp contract(off)
    const int hd = nb * kQK;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= g * hd) return;
    const int gi = idx / hd, j = idx - gi * hd;
    const int b = j >> 5, jj = j & 31;
    const float *wr = w + (size_t)gi * w_stride;
    float o = 0.0f;
    for (int t = 0; t < n; t++) {
        const unsigned char *blk = v + ((size_t)t * nb + b) * kBlockBytes;
        const float a = wr[t] * *reinterpret_cast<const float *>(blk);
        o += a * (float)(int8_t)blk[4 + jj];
    }
    out[(size_t)gi * out_stride + j] = o;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// One 256-thread work-group per row.
__global__ __launch_bounds__(256) void softmax_kernel(float *__restrict__ x, int n,
                                                      size_t stride) {
    __shared__ float red[4];
    float *row = x + (size_t)blockIdx.x * stride;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    float m = -INFINITY;
    for (int i = tid; i < n; i += 256) m = row[i] > m ? row[i] : m;
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < 4; w++) m = red[w] > m ? red[w] : m;
    __syncthreads();

    float sum = 0.0f;
    for (int i = tid; i < n; i += 256) {
        const float e = expf(row[i] - m);
        row[i] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    const float inv = 1.0f / (red[0] + red[1] + red[2] + red[3]);
    for (int i = tid; i < n; i += 256) row[i] *= inv;
}

inline unsigned grid_for(long items) { return (unsigned)((items + 255) / 256); }

}  // namespace

hipError_t tq_launch_quantize(const float *x, block_q8 *out, int n, hipStream_t s) {
    const int nblocks = n / kQK;
    if (nblocks <= 0) return hipSuccess;
    if ((((uintptr_t)x & 15) | ((uintptr_t)out & 3)) == 0)
        hipLaunchKernelGGL(quantize8_kernel, dim3(grid_for((long)nblocks * 8)), dim3(256), 0, s, x,
                           reinterpret_cast<unsigned char *>(out), (long)nblocks, (float *)nullptr, 1);
    else
        hipLaunchKernelGGL(quantize_kernel, dim3(grid_for((long)nblocks * kQK)), dim3(256), 0, s, x,
                           reinterpret_cast<unsigned char *>(out), nblocks);
    return hipGetLastError();
}

hipError_t tq_launch_quantize_split(const float *x, unsigned char *out, int rows, int cols, hipStream_t s) {
    const long nblocks = (long)rows * (cols / kQK);
    if (nblocks <= 0) return hipSuccess;
    if (cols % kQK || (((uintptr_t)x | (uintptr_t)out) & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize8_kernel, dim3(grid_for(nblocks * 8)), dim3(256), 0, s, x, out, nblocks,
                       reinterpret_cast<float *>(out + nblocks * kQK), cols / kQK);
    return hipGetLastError();
}

hipError_t tq_launch_rope(float *x, int n_heads, int hd, const float *c, const float *sn,
                          hipStream_t s) {
    const long items = (long)n_heads * (hd / 2);
    if (items <= 0) return hipSuccess;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(items)), dim3(256), 0, s, x, n_heads, hd, c, sn);
    return hipGetLastError();
}

hipError_t tq_launch_scores(const block_q8 *q, int g, const block_q8 *k, int n, int nb,
                            float scale, float *scores, size_t stride, hipStream_t s) {
    const long items = (long)n * g;
    if (items <= 0 || nb <= 0) return hipSuccess;
    hipLaunchKernelGGL(scores_kernel, dim3(grid_for(items)), dim3(256), 0, s,
                       reinterpret_cast<const unsigned char *>(q), g,
                       reinterpret_cast<const unsigned char *>(k), n, nb, scale, scores, stride);
    return hipGetLastError();
}

hipError_t tq_launch_accum(const float *w, size_t w_stride, int g, const block_q8 *v, int n,
                           int nb, float *out, size_t out_stride, hipStream_t s) {
    const long items = (long)g * nb * kQK;
    if (items <= 0) return hipSuccess;
    hipLaunchKernelGGL(accum_kernel, dim3(grid_for(items)), dim3(256), 0, s, w, w_stride, g,
                       reinterpret_cast<const unsigned char *>(v), n, nb, out, out_stride);
    return hipGetLastError();
}

// RMSNorm of rows of n floats (model/rmsnorm.c:4-19; norm_heads,
// model/attention_layer.c:48-53): a work-group copies R rows into LDS with
// coalesced loads (row stride n+1, so the lanes' serial walks below fall in
// distinct banks); lane r sums row r's squares serially in element order, as
// the reference does; then every thread writes (x * inverse) * weight.  out
// may be x.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float *__restrict__ x,
                                                           const float *__restrict__ w, float *out,
                                                           int n_rows, int n, int rows_per_wg, float eps) {
#pragma clang fp contract(off)
    extern __shared__ float rows_s[];
    const int r0 = blockIdx.x * rows_per_wg;
    const int nr = min(rows_per_wg, n_rows - r0);
    const int stride = n + 1;
    float *inv_s = rows_s + rows_per_wg * stride;
    for (int e = threadIdx.x; e < nr * n; e += 256) {
        const int r = e / n, j = e - r * n;
        rows_s[r * stride + j] = x[(size_t)r0 * n + e];
    }
    __syncthreads();
    if ((int)threadIdx.x < nr) {
        const float *row = rows_s + threadIdx.x * stride;
        float sum = 0.0f;
        for (int j = 0; j < n; j++) sum += row[j] * row[j];
        inv_s[threadIdx.x] = 1.0f / sqrtf(eps + sum / (float)n);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nr * n; e += 256) {
        const int r = e / n, j = e - r * n;
        out[(size_t)r0 * n + e] = rows_s[r * stride + j] * inv_s[r] * w[j];
    }
}

// The same with 16-byte accesses (n a multiple of 4, x, w and out 16-byte
// aligned): every thread issues its float4 loads of the staged rows eight at
// a time before writing any of them to LDS, so the staging is a few memory
// round trips rather than one per element.  The per-row serial sum is the
// same.
__global__ __launch_bounds__(256) void rmsnorm_rows4_kernel(const float *__restrict__ x,
                                                            const float *__restrict__ w, float *out,
                                                            int n_rows, int n, int rows_per_wg, float eps) {
#pragma clang fp contract(off)
    extern __shared__ float rows_s[];
    const int r0 = blockIdx.x * rows_per_wg;
    const int nr = min(rows_per_wg, n_rows - r0);
    const int stride = n + 1, n4 = n >> 2, tot4 = nr * n4;
    float *inv_s = rows_s + rows_per_wg * stride;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)r0 * n);
    constexpr int U = 8;
    for (int base = 0; base < tot4; base += 256 * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * 256 + (int)threadIdx.x;
            v[u] = x4[i < tot4 ? i : tot4 - 1];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * 256 + (int)threadIdx.x;
            if (i < tot4) {
                const int r = i / n4, j = 4 * (i - r * n4);
                float *d = rows_s + r * stride + j;
                d[0] = v[u].x;
                d[1] = v[u].y;
                d[2] = v[u].z;
                d[3] = v[u].w;
            }
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < nr) {
        const float *row = rows_s + threadIdx.x * stride;
        float sum = 0.0f;
        for (int j = 0; j < n; j++) sum += row[j] * row[j];
        inv_s[threadIdx.x] = 1.0f / sqrtf(eps + sum / (float)n);
    }
    __syncthreads();
    float4 *o4 = reinterpret_cast<float4 *>(out + (size_t)r0 * n);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    for (int i = threadIdx.x; i < tot4; i += 256) {
        const int r = i / n4, j4 = i - r * n4;
        const float *src = rows_s + r * stride + 4 * j4;
        const float inv = inv_s[r];
        const float4 wv = w4[j4];
        o4[i] = make_float4(src[0] * inv * wv.x, src[1] * inv * wv.y, src[2] * inv * wv.z, src[3] * inv * wv.w);
    }
}

hipError_t tq_launch_rmsnorm_rows(const float *x, const float *w, float *out, int n_rows, int n, float eps,
                                  hipStream_t s) {
    if (n_rows <= 0) return hipSuccess;
    int per = 8192 / (n + 1);
    per = per < 1 ? 1 : (per > 64 ? 64 : per);
    const size_t lds = ((size_t)per * (n + 1) + per) * sizeof(float);
    const dim3 grid((unsigned)((n_rows + per - 1) / per));
    if (n % 4 == 0 && (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0)
        hipLaunchKernelGGL(rmsnorm_rows4_kernel, grid, dim3(256), lds, s, x, w, out, n_rows, n, per, eps);
    else
        hipLaunchKernelGGL(rmsnorm_rows_kernel, grid, dim3(256), lds, s, x, w, out, n_rows, n, per, eps);
    return hipGetLastError();
}

hipError_t tq_launch_softmax(float *x, int n, int rows, size_t stride, hipStream_t s) {
    if (n <= 0 || rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(256), 0, s, x, n, stride);
    return hipGetLastError();
}
