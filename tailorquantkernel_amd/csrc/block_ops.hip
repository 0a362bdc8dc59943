// block_ops.hip — the rest of a transformer block on gfx950, around the
// attention layer and the projections: the MLP's silu_mul + quantize
// (model/silu.c:6-18, model/mlp.c:3-17), the residual add + RMSNorm
// (model/vec.c:3-6, model/rmsnorm.c:4-19, model/context.c:83-105), the Q8
// embedding lookup (model/embedding.c:4-17) and the greedy sampler
// (model/sampler.c:3-13).
#include "tq_common.hpp"

namespace {

using namespace tq;

// h = silu(g) * u (silu(x) = x * (1 / (1 + expf(-x)))), then quantize_row_q8
// of h: one 32-lane group per block, 8 blocks per work-group.  Rows are
// contiguous, so blocks never straddle two of them.
__global__ __launch_bounds__(256) void silu_quant_kernel(const float *__restrict__ gate,
                                                         const float *__restrict__ up,
                                                         unsigned char *__restrict__ hq, long nblocks) {
#pragma clang fp contract(off)
    const long e = (long)blockIdx.x * 256 + threadIdx.x;
    if ((e >> 5) >= nblocks) return;   // whole 32-lane groups leave together
    const float g = gate[e];
    const float sig = 1.0f / (1.0f + expf(-g));
    const float h = g * sig * up[e];
    quantize_store32(h, hq + (e >> 5) * kBlockBytes);
}

// x += y (when y is given), then xn = rmsnorm(x) with `weight`: one
// work-group per row.  The sum of squares is a parallel sum (per-thread
// serial over a strided slice, then a wave tree and the four waves in
// order), so xn agrees with the reference's serial sum within fp32 rounding.
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(float *__restrict__ x, const float *__restrict__ y,
                                                          const float *__restrict__ w, float *__restrict__ xn,
                                                          int n, float eps) {
#pragma clang fp contract(off)
    __shared__ float part[4];
    float *xr = x + (size_t)blockIdx.x * n;
    const float *yr = y ? y + (size_t)blockIdx.x * n : nullptr;
    float *xnr = xn + (size_t)blockIdx.x * n;
    float sum = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        float v = xr[i];
        if (yr) {
            v += yr[i];
            xr[i] = v;
        }
        sum += v * v;
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
    __syncthreads();
    const float total = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = 1.0f / sqrtf(eps + total / (float)n);
    for (int i = threadIdx.x; i < n; i += 256) xnr[i] = xr[i] * inv * w[i];
}

// One row of a tiled Q8 matrix to fp32: out[b*32 + j] = d_b * code_j.
__global__ __launch_bounds__(256) void embed_q8_kernel(const unsigned char *__restrict__ E, int rows, int cols,
                                                       int token, float *__restrict__ out) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= cols) return;
    const int nb = cols / kQK;
    const int b = e / kQK, j = e - b * kQK;
    const int g = b / 64, rest = nb - 64 * g, n = rest < 64 ? rest : 64, i = b - 64 * g;
    const int off = g * 2048 + (j < 16 ? 16 * i + j : 16 * n + 16 * i + (j - 16));
    const signed char code = (signed char)E[(size_t)token * cols + off];
    const float d = reinterpret_cast<const float *>(E + (size_t)rows * cols)[(size_t)token * nb + b];
    out[e] = d * (float)code;
}

// The first index of the largest logit, as the serial scan with a strict ">"
// finds it (NaN never wins; a NaN at index 0 keeps index 0): thread t scans
// its contiguous slice in order (slice 0 from logits[0], the others from
// -inf with no index), then thread 0 merges the 256 slices in order.
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ logits, int n,
                                                     int32_t *__restrict__ out) {
    __shared__ float sm[256];
    __shared__ int si[256];
    const int per = (n + 255) / 256;
    const int i0 = threadIdx.x * per, i1 = min(n, i0 + per);
    float m = threadIdx.x == 0 ? logits[0] : -__builtin_inff();
    int idx = threadIdx.x == 0 ? 0 : -1;
    for (int i = (threadIdx.x == 0 ? 1 : i0); i < i1; i++) {
        const float v = logits[i];
        if (v > m) {
            m = v;
            idx = i;
        }
    }
    sm[threadIdx.x] = m;
    si[threadIdx.x] = idx;
    __syncthreads();
    if (threadIdx.x == 0) {
        float bm = sm[0];
        int bi = si[0];
        for (int t = 1; t < 256; t++)
            if (si[t] >= 0 && sm[t] > bm) {
                bm = sm[t];
                bi = si[t];
            }
        *out = bi;
    }
}

int herr(hipError_t e) { return e == hipSuccess ? TQ_HIP_OK : TQ_HIP_EHIP_BASE - (int)e; }

}  // namespace

hipError_t tq_launch_silu_quant(const float *gate, const float *up, block_q8 *hq, long n, hipStream_t s) {
    const long nblocks = n / kQK;
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(silu_quant_kernel, dim3((unsigned)((nblocks * kQK + 255) / 256)), dim3(256), 0, s, gate, up,
                       reinterpret_cast<unsigned char *>(hq), nblocks);
    return hipGetLastError();
}

extern "C" {

int tq_hip_add_rmsnorm(float *x, const float *y, const float *weight, float *xn, int n_rows, int n, float eps,
                       void *stream) {
    if (n_rows < 0 || n <= 0 || (n_rows > 0 && (!x || !weight || !xn))) return TQ_HIP_EINVAL;
    if (n_rows == 0) return TQ_HIP_OK;
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, x, y, weight,
                       xn, n, eps);
    return herr(hipGetLastError());
}

int tq_hip_embed_lookup_q8(const void *embed, int rows, int cols, int token, float *out, void *stream) {
    if (!embed || !out || rows <= 0 || cols <= 0 || cols % kQK != 0 || ((uintptr_t)embed & 15)) return TQ_HIP_EINVAL;
    if (token < 0 || token >= rows) return TQ_HIP_EINVAL;   // model/embedding.c:5
    hipLaunchKernelGGL(embed_q8_kernel, dim3((unsigned)((cols + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const unsigned char *)embed, rows, cols, token, out);
    return herr(hipGetLastError());
}

int tq_hip_sample_greedy(const float *logits, int n, int32_t *out, void *stream) {
    if (n <= 0 || !logits || !out) return TQ_HIP_EINVAL;   // model/sampler.c:4
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, logits, n, out);
    return herr(hipGetLastError());
}

}  // extern "C"
