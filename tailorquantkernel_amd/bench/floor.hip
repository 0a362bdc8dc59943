// floor.hip — bench-only measurement kernel (libtqbench.so, loaded by bench.py;
// not part of the attention library): the floor of one split-K decode step on
// this GPU, the same grid and synchronisation with no attention math.
#include "../csrc/tq_common.hpp"
#include "tq_bench.h"

namespace {

using namespace tq;

// Work-group w (of n_heads * n_splits, head = w / n_splits)
// reads its 1/n_wg chunk of the buffer with every 16-byte load in flight.
// mode 0 returns at once (the launch alone), mode 1 stops after the read,
// mode 2 then writes a PF-float partial row with agent-coherent stores, waits
// for them, bumps its head's arrival counter, and the last work-group of the
// head pulls the head's n_splits rows and writes their sum: the decode's
// store -> counter -> pull chain.
constexpr int kFloorPF = 520;            // one split's partial at the 8B shape: 4 heads x (128 + 2)
constexpr int kFloorCounterStride = 64;  // ints: one 256-byte line per counter
constexpr int kFloorLoads = 16;          // 16-byte loads per thread per round

__global__ __launch_bounds__(256) void floor_step_kernel(const u32x4 *buf, size_t n16, int n_splits, int mode,
                                                         float *partials, int *counters, float *out, uint32_t never) {
    if (mode == 0) return;
    const int head = blockIdx.x / n_splits, split = blockIdx.x % n_splits;
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t begin = per * blockIdx.x;
    const size_t end = begin + per < n16 ? begin + per : n16;
    u32x4 acc = u32x4{0u, 0u, 0u, 0u};
    for (size_t i0 = begin; i0 < end; i0 += (size_t)kFloorLoads * 256) {
        u32x4 v[kFloorLoads];
#pragma unroll
        for (int u = 0; u < kFloorLoads; u++) {
            const size_t i = i0 + threadIdx.x + (size_t)u * 256;
            v[u] = i < end ? buf[i] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kFloorLoads; u++) acc ^= v[u];
    }
    const uint32_t fold = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (mode == 1) {
        if (fold == never) out[blockIdx.x] = 1.0f;
        return;
    }
    // the partial row: its split index, plus 0 unless the fold hit `never`
    const float val = (float)split + (fold == never ? 1.0f : 0.0f);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        partials + (size_t)head * n_splits * kFloorPF, 0, n_splits * kFloorPF * 4, 0x00020000);
    for (int u = threadIdx.x; u < kFloorPF / 4; u += 256)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(val), __float_as_uint(val), __float_as_uint(val),
                                                     __float_as_uint(val)},
                                               pr, (split * kFloorPF + 4 * u) * 4, 0, 16);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int last;
    int *counter = counters + (size_t)head * kFloorCounterStride;
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_splits - 1;
    __syncthreads();
    if (!last) return;
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // one batch of loads per thread for up to 32 splits, as the decode's
    // combine requests all of a pass's rows before it sums any
    if (threadIdx.x < kFloorPF / 4) {
        float f[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < n_splits; s0 += 32) {
            u32x4 rows[32];
#pragma unroll
            for (int i = 0; i < 32; i++)
                rows[i] = s0 + i < n_splits ? __builtin_amdgcn_raw_buffer_load_b128(
                                                  pr, ((s0 + i) * kFloorPF + 4 * threadIdx.x) * 4, 0, 16)
                                            : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < 32; i++)
#pragma unroll
                for (int c = 0; c < 4; c++) f[c] += __uint_as_float(rows[i][c]);
        }
        *reinterpret_cast<float4 *>(out + (size_t)head * kFloorPF + 4 * threadIdx.x) = float4{f[0], f[1], f[2], f[3]};
    }
}

}  // namespace

extern "C" size_t tq_hip_floor_scratch_bytes(int n_heads, int n_splits) {
    if (n_heads <= 0 || n_splits <= 0) return 0;
    return (size_t)n_heads * kFloorCounterStride * sizeof(int) + (size_t)n_heads * n_splits * kFloorPF * sizeof(float);
}

extern "C" size_t tq_hip_floor_out_bytes(int n_heads, int n_splits) {
    if (n_heads <= 0 || n_splits <= 0) return 0;
    const size_t a = (size_t)n_heads * kFloorPF, b = (size_t)n_heads * n_splits;
    return (a > b ? a : b) * sizeof(float);
}

extern "C" int tq_hip_floor_step(const void *buf, size_t bytes, int n_heads, int n_splits, int mode, void *scratch,
                                 void *out, void *stream) {
    if (!buf || !scratch || !out || bytes < 16 || bytes % 16 != 0 || n_heads <= 0 || n_splits <= 0 ||
        (size_t)n_heads * n_splits > 65535 || mode < 0 || mode > 2 || ((uintptr_t)scratch & 255) ||
        ((uintptr_t)out & 15))
        return TQ_HIP_EINVAL;
    int *counters = static_cast<int *>(scratch);
    float *partials = reinterpret_cast<float *>(counters + (size_t)n_heads * kFloorCounterStride);
    hipLaunchKernelGGL(floor_step_kernel, dim3(n_heads * n_splits), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const u32x4 *>(buf), bytes / 16, n_splits, mode, partials, counters,
                       static_cast<float *>(out), 0x9E3779B9u);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_HIP_OK : TQ_HIP_EHIP_BASE - (int)e;
}

