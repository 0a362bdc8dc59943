// block_ops.hip — the rest of a transformer block on gfx950, around the
// attention layer and the projections: the MLP's silu_mul + quantize
// (model/silu.c:6-18, model/mlp.c:3-17), the residual add + RMSNorm
// (model/vec.c:3-6, model/rmsnorm.c:4-19, model/context.c:80-102), the Q8
// embedding lookup (model/embedding.c:4-17) and the greedy sampler
// (model/sampler.c:3-13).
#include "tq_common.hpp"

namespace {

using namespace tq;

typedef float v4f __attribute__((ext_vector_type(4)));

// h = silu(g) * u (silu(x) = x * (1 / (1 + expf(-x))), model/silu.c:6-18),
// then quantize_row_q8 of h, 8 lanes x 4 values per block: float4 loads of
// gate and up, one dword of codes per lane.  Rows are contiguous, so blocks
// never straddle two of them; whole 8-lane groups stay together, as
// quantize8x4's DPP steps need.
// scales non-null: the block-major split layout of quantize8_kernel over
// rows of nb blocks.
__global__ __launch_bounds__(256) void silu_quant8_kernel(const float *__restrict__ gate,
                                                          const float *__restrict__ up,
                                                          unsigned char *__restrict__ hq, long nblocks,
                                                          float *__restrict__ scales, int nb) {
#pragma clang fp contract(off)
    const long k = (long)blockIdx.x * 256 + threadIdx.x;
    const long gi = k >> 3;
    if (gi >= nblocks) return;
    const int e = (int)(k & 7);
    // split layout: block-major order (consecutive groups, consecutive rows of
    // one block), so the code stores coalesce
    const long n = scales ? nblocks / nb : 1, bq = scales ? gi / n : 0, tq = scales ? gi - bq * n : 0;
    const long tb = scales ? tq * nb + bq : gi;
    const float4 g4 = *reinterpret_cast<const float4 *>(gate + tb * kQK + 4 * e);
    const float4 u4 = *reinterpret_cast<const float4 *>(up + tb * kQK + 4 * e);
    const float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w};
    float h[4];
#pragma unroll
    for (int i = 0; i < 4; i++) h[i] = silu_mul(g[i], u[i]);
    if (scales) {
        quantize8x4(h, scales + bq * n + tq, hq + ((2 * bq + (e >> 2)) * n + tq) * 16 + 4 * (e & 3), e == 0);
    } else {
        unsigned char *blk = hq + tb * kBlockBytes;
        quantize8x4(h, reinterpret_cast<float *>(blk), blk + 4 + 4 * e, e == 0);
    }
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

// The same with 16-byte accesses and every load of a row issued up front:
// 1024 threads, K float4 of the row per thread held in registers, so the row
// costs one round trip to memory instead of one per strided slice.  The sum
// of squares is per thread (its K float4 in order), then a wave tree, then the
// 16 waves in order.
template <int K>
__global__ __launch_bounds__(1024) void add_rmsnorm4_kernel(float *__restrict__ x, const float *__restrict__ y,
                                                            const float *__restrict__ w, float *__restrict__ xn,
                                                            int n, float eps) {
#pragma clang fp contract(off)
    __shared__ float part[16];
    const int n4 = n >> 2;
    v4f *xr = reinterpret_cast<v4f *>(x + (size_t)blockIdx.x * n);
    const v4f *yr = y ? reinterpret_cast<const v4f *>(y + (size_t)blockIdx.x * n) : nullptr;
    const v4f *wr = reinterpret_cast<const v4f *>(w);
    v4f *xnr = reinterpret_cast<v4f *>(xn + (size_t)blockIdx.x * n);
    v4f v[K], wv[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = threadIdx.x + 1024 * k;
        const int ic = i < n4 ? i : n4 - 1;   // clamped: every load is issued unconditionally
        v[k] = xr[ic];
        wv[k] = wr[ic];
    }
    if (yr) {
        v4f yv[K];
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + 1024 * k;
            yv[k] = yr[i < n4 ? i : n4 - 1];
        }
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int i = threadIdx.x + 1024 * k;
            v[k] += yv[k];
            if (i < n4) xr[i] = v[k];
        }
    }
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        if (threadIdx.x + 1024 * k < n4) {
            sum += v[k].x * v[k].x;
            sum += v[k].y * v[k].y;
            sum += v[k].z * v[k].z;
            sum += v[k].w * v[k].w;
        }
    }
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) total += part[i];
    const float inv = 1.0f / sqrtf(eps + total / (float)n);
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int i = threadIdx.x + 1024 * k;
        if (i < n4) xnr[i] = v[k] * inv * wv[k];
    }
}

// One row of a tiled Q8 matrix to fp32: out[b*32 + j] = d_b * code_j.  With
// `tokens`, grid row y looks up tokens[y] into out + y*cols (a token outside
// [0, rows) writes zeros).
// Q4: a tiled Q4 row, out[b*32 + j] = d_b * (nibble - 8) (model/embedding.c:20-27).
template <bool Q4>
__global__ __launch_bounds__(256) void embed_q8_kernel(const unsigned char *__restrict__ E, int rows, int cols,
                                                       int token, const int32_t *__restrict__ tokens,
                                                       float *__restrict__ out) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= cols) return;
    if (tokens) {
        token = tokens[blockIdx.y];
        out += (size_t)blockIdx.y * cols;
        if (token < 0 || token >= rows) {
            out[e] = 0.0f;
            return;
        }
    }
    const int nb = cols / kQK;
    const int b = e / kQK, j = e - b * kQK;
    if (Q4) {
        const unsigned char byte = E[(size_t)token * (cols / 2) + 16 * b + (j & 15)];
        const int code = (j < 16 ? (byte & 0x0F) : (byte >> 4)) - 8;
        const float d = reinterpret_cast<const float *>(E + (size_t)rows * (cols / 2))[(size_t)token * nb + b];
        out[e] = d * (float)code;
        return;
    }
    const int g = b / 64, rest = nb - 64 * g, n = rest < 64 ? rest : 64, i = b - 64 * g;
    const int off = g * 2048 + (j < 16 ? 16 * i + j : 16 * n + 16 * i + (j - 16));
    const signed char code = (signed char)E[(size_t)token * cols + off];
    const float d = reinterpret_cast<const float *>(E + (size_t)rows * cols)[(size_t)token * nb + b];
    out[e] = d * (float)code;
}

// The first index of the largest logit, as the serial scan with a strict ">"
// from logits[0] finds it: NaN never wins, and a NaN at index 0 keeps index 0.
// Every other NaN is skipped, so the answer is the smallest index holding the
// largest non-NaN value — an order-free reduction of (value, index) pairs with
// "larger value, then smaller index" wins.  1024 threads; each loads its
// share in batches of 8 independent float4 (or float) loads.
__device__ __forceinline__ void arg_better(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

template <bool VEC>
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ logits, int n,
                                                      int32_t *__restrict__ out) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float bv = -__builtin_inff();
    int bi = n;   // none yet
    constexpr int B = 8;
    if constexpr (VEC) {
        const v4f *l4 = reinterpret_cast<const v4f *>(logits);
        const int n4 = n >> 2;
        for (int u0 = 0; u0 < n4; u0 += 1024 * B) {
            v4f x[B];
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int u = u0 + 1024 * b + (int)threadIdx.x;
                x[b] = l4[u < n4 ? u : n4 - 1];
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int u = u0 + 1024 * b + (int)threadIdx.x;
                if (u < n4) {
                    arg_better(x[b].x, 4 * u, bv, bi);
                    arg_better(x[b].y, 4 * u + 1, bv, bi);
                    arg_better(x[b].z, 4 * u + 2, bv, bi);
                    arg_better(x[b].w, 4 * u + 3, bv, bi);
                }
            }
        }
    } else {
        for (int e0 = 0; e0 < n; e0 += 1024 * B) {
            float x[B];
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int e = e0 + 1024 * b + (int)threadIdx.x;
                x[b] = logits[e < n ? e : n - 1];
            }
#pragma unroll
            for (int b = 0; b < B; b++) {
                const int e = e0 + 1024 * b + (int)threadIdx.x;
                if (e < n) arg_better(x[b], e, bv, bi);
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        arg_better(ov, oi, bv, bi);
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++) arg_better(sv[w], si[w], bv, bi);
        const float first = logits[0];
        *out = (first != first || bi >= n) ? 0 : bi;
    }
}

int herr(hipError_t e) { return e == hipSuccess ? TQ_HIP_OK : TQ_HIP_EHIP_BASE - (int)e; }

int embed_lookup(bool q4, const void *embed, int rows, int cols, int token, const int32_t *d_tokens, int n,
                 float *out, void *stream) {
    if (!embed || !out || rows <= 0 || cols <= 0 || cols % kQK != 0 || ((uintptr_t)embed & 15)) return TQ_HIP_EINVAL;
    if (!d_tokens && (token < 0 || token >= rows)) return TQ_HIP_EINVAL;   // model/embedding.c:5
    if (d_tokens && (n < 0 || n > 65535)) return TQ_HIP_EINVAL;
    if (d_tokens && n == 0) return TQ_HIP_OK;
    const dim3 grid((unsigned)((cols + 255) / 256), d_tokens ? (unsigned)n : 1u);
    if (q4)
        hipLaunchKernelGGL(embed_q8_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream,
                           (const unsigned char *)embed, rows, cols, token, d_tokens, out);
    else
        hipLaunchKernelGGL(embed_q8_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream,
                           (const unsigned char *)embed, rows, cols, token, d_tokens, out);
    return herr(hipGetLastError());
}

}  // namespace

hipError_t tq_launch_silu_quant(const float *gate, const float *up, block_q8 *hq, long n, hipStream_t s) {
    const long nblocks = n / kQK;
    if (nblocks <= 0) return hipSuccess;
    // gate, up and hq are workspace rows at 256-byte offsets of a 16-byte
    // aligned workspace (tq_hip_mlp_layer_async checks it)
    if ((((uintptr_t)gate | (uintptr_t)up) & 15) || ((uintptr_t)hq & 3)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(silu_quant8_kernel, dim3((unsigned)((nblocks * 8 + 255) / 256)), dim3(256), 0, s, gate, up,
                       reinterpret_cast<unsigned char *>(hq), nblocks, (float *)nullptr, 1);
    return hipGetLastError();
}

hipError_t tq_launch_silu_quant_split(const float *gate, const float *up, unsigned char *hq, int rows, int cols,
                                      hipStream_t s) {
    const long nblocks = (long)rows * (cols / kQK);
    if (nblocks <= 0) return hipSuccess;
    if (cols % kQK || (((uintptr_t)gate | (uintptr_t)up | (uintptr_t)hq) & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(silu_quant8_kernel, dim3((unsigned)((nblocks * 8 + 255) / 256)), dim3(256), 0, s, gate, up, hq,
                       nblocks, reinterpret_cast<float *>(hq + nblocks * kQK), cols / kQK);
    return hipGetLastError();
}

extern "C" {

int tq_hip_add_rmsnorm(float *x, const float *y, const float *weight, float *xn, int n_rows, int n, float eps,
                       void *stream) {
    if (n_rows < 0 || n <= 0 || (n_rows > 0 && (!x || !weight || !xn))) return TQ_HIP_EINVAL;
    if (n_rows == 0) return TQ_HIP_OK;
    const hipStream_t s = (hipStream_t)stream;
    const bool vec = n % 4 == 0 && (((uintptr_t)x | (uintptr_t)y | (uintptr_t)weight | (uintptr_t)xn) & 15) == 0;
    const int k = (n / 4 + 1023) / 1024;
    const dim3 grid((unsigned)n_rows);
    if (vec && k == 1)
        hipLaunchKernelGGL(add_rmsnorm4_kernel<1>, grid, dim3(1024), 0, s, x, y, weight, xn, n, eps);
    else if (vec && k == 2)
        hipLaunchKernelGGL(add_rmsnorm4_kernel<2>, grid, dim3(1024), 0, s, x, y, weight, xn, n, eps);
    else if (vec && k <= 4)
        hipLaunchKernelGGL(add_rmsnorm4_kernel<4>, grid, dim3(1024), 0, s, x, y, weight, xn, n, eps);
    else if (vec && k <= 8)
        hipLaunchKernelGGL(add_rmsnorm4_kernel<8>, grid, dim3(1024), 0, s, x, y, weight, xn, n, eps);
    else
        hipLaunchKernelGGL(add_rmsnorm_kernel, grid, dim3(256), 0, s, x, y, weight, xn, n, eps);
    return herr(hipGetLastError());
}

int tq_hip_embed_lookup_q8(const void *embed, int rows, int cols, int token, float *out, void *stream) {
    return embed_lookup(false, embed, rows, cols, token, nullptr, 0, out, stream);
}

int tq_hip_embed_lookup_q8_batch(const void *embed, int rows, int cols, const int32_t *d_tokens, int n, float *out,
                                 void *stream) {
    if (!d_tokens) return TQ_HIP_EINVAL;
    return embed_lookup(false, embed, rows, cols, 0, d_tokens, n, out, stream);
}

int tq_hip_embed_lookup_q4(const void *embed, int rows, int cols, int token, float *out, void *stream) {
    return embed_lookup(true, embed, rows, cols, token, nullptr, 0, out, stream);
}

int tq_hip_embed_lookup_q4_batch(const void *embed, int rows, int cols, const int32_t *d_tokens, int n, float *out,
                                 void *stream) {
    if (!d_tokens) return TQ_HIP_EINVAL;
    return embed_lookup(true, embed, rows, cols, 0, d_tokens, n, out, stream);
}

int tq_hip_sample_greedy(const float *logits, int n, int32_t *out, void *stream) {
    if (n <= 0 || !logits || !out) return TQ_HIP_EINVAL;   // model/sampler.c:4
    if (n % 4 == 0 && ((uintptr_t)logits & 15) == 0)
        hipLaunchKernelGGL(argmax_kernel<true>, dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, n, out);
    else
        hipLaunchKernelGGL(argmax_kernel<false>, dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, n, out);
    return herr(hipGetLastError());
}

}  // extern "C"
