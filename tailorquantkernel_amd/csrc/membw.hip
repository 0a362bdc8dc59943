// membw.hip — streaming-read bandwidth of the GPU's HBM: the device-side
// counterpart of the reference's host probe (tools/membw.h:1-80, best of
// several timed reads of a buffer far larger than the last-level cache).
//
// Each work-group reads one contiguous chunk of the buffer, every lane 16-byte
// vectors, sixteen in flight per loop trip (measured on MI355X: contiguous
// chunks reach 6.2-6.4 TB/s where a grid-stride walk of the same buffer stays
// at 5.3-6.1).  The loaded words are folded with XOR and written out only when
// the fold hits a value the caller chose, so the loads stay live but the
// kernel writes (almost) nothing.  The caller times it.
#include "tq_common.hpp"

namespace {

using namespace tq;

constexpr int kMembwThreads = 256;
constexpr int kMembwGroups = 4096;       // 16 per CU
constexpr int kMembwUnroll = 16;

__global__ __launch_bounds__(kMembwThreads) void membw_read_kernel(const u32x4 *p, size_t n16, u32x4 *sink,
                                                                   uint32_t never) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t begin = per * blockIdx.x;
    const size_t end = begin + per < n16 ? begin + per : n16;
    size_t i = begin + threadIdx.x;
    u32x4 acc = u32x4{0u, 0u, 0u, 0u};
    for (; i + (kMembwUnroll - 1) * kMembwThreads < end; i += kMembwUnroll * kMembwThreads) {
        u32x4 v[kMembwUnroll];
#pragma unroll
        for (int u = 0; u < kMembwUnroll; u++) v[u] = p[i + u * kMembwThreads];
#pragma unroll
        for (int u = 0; u < kMembwUnroll; u++) acc ^= v[u];
    }
    for (; i < end; i += kMembwThreads) acc ^= p[i];
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == never) sink[blockIdx.x * kMembwThreads + threadIdx.x] = acc;
}

}  // namespace

extern "C" size_t tq_hip_membw_sink_bytes(void) { return (size_t)kMembwGroups * kMembwThreads * sizeof(u32x4); }

extern "C" int tq_hip_membw_read(const void *buf, size_t bytes, void *sink, unsigned int never, void *stream) {
    if (!buf || !sink || bytes < 16 || bytes % 16 != 0) return TQ_HIP_EINVAL;
    hipLaunchKernelGGL(membw_read_kernel, dim3(kMembwGroups), dim3(kMembwThreads), 0, (hipStream_t)stream,
                       static_cast<const u32x4 *>(buf), bytes / 16, static_cast<u32x4 *>(sink), never);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_HIP_OK : TQ_HIP_EHIP_BASE - (int)e;
}
