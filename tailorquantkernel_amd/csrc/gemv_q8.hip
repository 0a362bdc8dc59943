// gemv_q8.hip — the Q8 weight side of the attention layer on gfx950: the
// weight x Q8-activation matmul (kernel/q8_scalar.c:3-30, kernel/kernel.h:13-20)
// and the projections around attention that use it (project_qkv and
// project_output, model/attention_layer.c:38-46,161-167, and their batched
// forms, :213-218,238-241).
//
// Device weight layout ("tiled Q8"), exactly the byte count of the
// reference's rows x cols/32 block_q8 array:
//   codes  [rows][cols] int8.  A row is cut into groups of up to 64 blocks
//          (2048 codes); a group of n blocks holds the first 16 codes of each
//          of its n blocks (16 B per block, in block order), then the last 16
//          codes of each.  Lane l of a wave reads block 64g+l of a row as two
//          16-byte loads, each wave-wide load one contiguous 1 KiB.
//   scales [rows][cols/32] fp32 at byte offset rows*cols, one coalesced
//          dword per lane per group.
// tq_hip_q8_pack turns the reference's block_q8 rows into this layout on the
// device; tq_hip_q8_unpack turns it back.
//
// "Tiled Q4" (packer/packer.h:9, the reference's 20-byte block_q4), the same
// byte count as its rows x cols/32 block_q4 array:
//   codes  [rows][cols/2]: each block's 16 nibble bytes as the reference
//          stores them (byte j: code j + 8 in the low nibble, code j + 24 in
//          the high nibble), blocks in order, so lane l of a wave reads block
//          64g+l as one 16-byte load and a wave-wide load is 1 KiB.
//   scales [rows][cols/32] fp32 at byte offset rows*cols/2.
// A Q4 dword w is turned into two dwords of signed bytes 16*code with
// x = w ^ 0x88888888 (the nibble n becomes n - 8 in 4-bit two's complement):
// (x << 4) & 0xF0F0F0F0 holds the low codes, x & 0xF0F0F0F0 the high codes.
// The int32 dot of those with the activation codes is 16 times the block's
// exact dot sum_j (n_j - 8) * x_j of kernel/q4_scalar.c:6-11, and an
// arithmetic shift by 4 gives it back exactly.
//
// Matmul: the work is one pass over the weight bytes (HBM-bound).  A
// 256-thread work-group runs 4 waves; a wave owns RW consecutive rows.  The
// work-group first copies the activation rows (up to T tokens of block_q8,
// the reference's activation format) straight into LDS with
// global_load_lds_dwordx4, then every wave issues the loads of its first 8
// (row, group) units, and only then waits: the copies, issued first, are
// complete once no more than those 3*8 weight loads are outstanding, so the
// activation copy hides under the weight latency.
// Per block: int32 dot of the 32 code pairs (8 v_dot4_i32_i8), then
// ((float)s * w_d) * x_d as the scalar reference rounds it; the per-lane sums
// over groups and the 64-lane sum replace the reference's serial block-order
// sum (the reference's own SIMD kernels reorder that sum as well).
//
// The projections (project_qkv: wq, wk and wv in one launch over their
// concatenated rows; project_output) take fp32 input rows.  For one or two
// rows the matmul launch copies them into LDS and quantizes them there
// (bit-exact quantize_row_q8), and work-group 0 leaves the blocks in the
// caller's workspace; for more rows quantize_row_q8 runs into the workspace
// first, as the reference quantizes into xn_q8 / ws->xq, and the matmul
// reads the blocks from there.
#include "tq_common.hpp"

#include <stdlib.h>

namespace {

using namespace tq;

constexpr int kGemvWaves = 4;
constexpr int kGroupBlocks = 64;
constexpr int kGroupBytes = kGroupBlocks * kQK;   // 2048
constexpr int kGroupBytes4 = kGroupBlocks * 16;   // 1024: a Q4 group
constexpr int kBlockBytes4 = 20;                  // sizeof(block_q4)
constexpr int kMaxSegs = 3;
// Activation rows in LDS per work-group: 8 rows of 8192 (73,728 bytes) fit,
// two work-groups per CU's 160 KiB.
constexpr size_t kMaxStageBytes = 80 * 1024;
constexpr size_t kDefaultLdsLimit = 64 * 1024;    // beyond this a kernel must opt in

int herr(hipError_t e) { return e == hipSuccess ? TQ_HIP_OK : TQ_HIP_EHIP_BASE - (int)e; }

// Byte offset inside a tiled row of code j (0..31) of block b.
__host__ __device__ __forceinline__ int tiled_offset(int nb, int b, int j) {
    const int g = b / kGroupBlocks;
    const int rest = nb - g * kGroupBlocks;
    const int n = rest < kGroupBlocks ? rest : kGroupBlocks;
    const int i = b - g * kGroupBlocks;
    return g * kGroupBytes + (j < 16 ? 16 * i + j : 16 * n + 16 * i + (j - 16));
}

// ---------------------------------------------------------------------------
// block_q8 rows <-> tiled layout.  One thread per block.
__global__ __launch_bounds__(256) void pack_kernel(unsigned char *__restrict__ dst,
                                                   const unsigned char *__restrict__ src,
                                                   int rows, int nb) {
    const long long k = (long long)blockIdx.x * 256 + threadIdx.x;
    if (k >= (long long)rows * nb) return;
    const int r = (int)(k / nb), b = (int)(k - (long long)r * nb);
    const uint32_t *blk = reinterpret_cast<const uint32_t *>(src + (size_t)k * kBlockBytes);
    u32x4 lo, hi;
    lo.x = blk[1]; lo.y = blk[2]; lo.z = blk[3]; lo.w = blk[4];
    hi.x = blk[5]; hi.y = blk[6]; hi.z = blk[7]; hi.w = blk[8];
    const int cols = nb * kQK;
    unsigned char *row = dst + (size_t)r * cols;
    *reinterpret_cast<u32x4 *>(row + tiled_offset(nb, b, 0)) = lo;
    *reinterpret_cast<u32x4 *>(row + tiled_offset(nb, b, 16)) = hi;
    reinterpret_cast<uint32_t *>(dst + (size_t)rows * cols)[k] = blk[0];
}

__global__ __launch_bounds__(256) void unpack_kernel(unsigned char *__restrict__ dst,
                                                     const unsigned char *__restrict__ src,
                                                     int rows, int nb) {
    const long long k = (long long)blockIdx.x * 256 + threadIdx.x;
    if (k >= (long long)rows * nb) return;
    const int r = (int)(k / nb), b = (int)(k - (long long)r * nb);
    const int cols = nb * kQK;
    const unsigned char *row = src + (size_t)r * cols;
    const u32x4 lo = *reinterpret_cast<const u32x4 *>(row + tiled_offset(nb, b, 0));
    const u32x4 hi = *reinterpret_cast<const u32x4 *>(row + tiled_offset(nb, b, 16));
    uint32_t *blk = reinterpret_cast<uint32_t *>(dst + (size_t)k * kBlockBytes);
    blk[0] = reinterpret_cast<const uint32_t *>(src + (size_t)rows * cols)[k];
    blk[1] = lo.x; blk[2] = lo.y; blk[3] = lo.z; blk[4] = lo.w;
    blk[5] = hi.x; blk[6] = hi.y; blk[7] = hi.z; blk[8] = hi.w;
}

// block_q4 rows <-> tiled Q4.  One thread per block.
__global__ __launch_bounds__(256) void pack4_kernel(unsigned char *__restrict__ dst,
                                                    const unsigned char *__restrict__ src, long long n) {
    const long long k = (long long)blockIdx.x * 256 + threadIdx.x;
    if (k >= n) return;
    const uint32_t *blk = reinterpret_cast<const uint32_t *>(src + (size_t)k * kBlockBytes4);
    u32x4 q;
    q.x = blk[1]; q.y = blk[2]; q.z = blk[3]; q.w = blk[4];
    *reinterpret_cast<u32x4 *>(dst + (size_t)k * 16) = q;
    reinterpret_cast<uint32_t *>(dst + (size_t)n * 16)[k] = blk[0];
}

__global__ __launch_bounds__(256) void unpack4_kernel(unsigned char *__restrict__ dst,
                                                      const unsigned char *__restrict__ src, long long n) {
    const long long k = (long long)blockIdx.x * 256 + threadIdx.x;
    if (k >= n) return;
    const u32x4 q = *reinterpret_cast<const u32x4 *>(src + (size_t)k * 16);
    uint32_t *blk = reinterpret_cast<uint32_t *>(dst + (size_t)k * kBlockBytes4);
    blk[0] = reinterpret_cast<const uint32_t *>(src + (size_t)n * 16)[k];
    blk[1] = q.x; blk[2] = q.y; blk[3] = q.z; blk[4] = q.w;
}

// Signed bytes 16 * code from a dword of Q4 nibbles: low nibbles, high nibbles.
__device__ __forceinline__ uint32_t q4_lo16(uint32_t w) { return ((w ^ 0x88888888u) << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t q4_hi16(uint32_t w) { return (w ^ 0x88888888u) & 0xF0F0F0F0u; }

// ---------------------------------------------------------------------------
// Matmul over up to three row-concatenated matrices sharing one input
// (project_qkv runs wq, wk and wv in one launch).

struct GemvSeg {
    const unsigned char *w;   // tiled matrix
    float *y;                 // y[t * rows + r]
    int rows;
};

struct GemvArgs {
    GemvSeg seg[kMaxSegs];
    int seg_end[kMaxSegs];    // cumulative row ends
    int rows_total;
    int cols, nb, ng;
    const unsigned char *xq;  // block_q8 [n_tok][nb] (when x is null)
    const float *x;           // fp32 [n_tok][cols], 16-byte aligned, quantized in LDS
    unsigned char *xq_out;    // where work-group 0 leaves quantize_row_q8(x), or null
    int n_tok;                // rows of input in this launch (<= T)
    bool q4;                  // the matrices are tiled Q4 (else tiled Q8)
    bool uni_tiles;           // GEMM: every 128-row tile lies in one segment and every
                              // segment's codes and scales are under 2 GiB
    float *part;              // GEMM split-K partial tiles [ksplit][n_tok][rows_total], or null
    size_t part_floats;       // their capacity
    int ksplit;               // GEMM: K splits of this launch (1: none)
    bool xs;                  // GEMM: xq holds the block-major split layout of
                              // tq_launch_quantize_split instead of block_q8 rows
    unsigned char *hq;        // GEMM over the MLP's gate (segment 0) and up (segment 1)
                              // matrices: each tile pairs 64 rows of both, and the
                              // epilogue writes silu_mul + quantize_row_q8 of the
                              // hidden rows in the split layout here instead of y
};

typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef int v4i __attribute__((ext_vector_type(4)));

// 16 bytes from each active lane's global address into LDS at dst + 16*lane
// (global_load_lds_dwordx4; M0 holds the LDS byte address and is restored;
// dst must be the same for the whole wave).
// The memory clobber keeps every later load after it in program order, which
// the vmcnt arithmetic below relies on.
__device__ __forceinline__ void dma16(const void *src, unsigned char *dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8 *)dst);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(lds)
        : "memory");
}

// Wait until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// 4 bytes from each active lane's global address into LDS at dst + 4*lane
// (global_load_lds_dword).
__device__ __forceinline__ void dma4(const void *src, unsigned char *dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8 *)dst);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\t"
        "global_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(lds)
        : "memory");
}

// The same copies from a uniform base plus a 32-bit lane offset (the saddr
// form): no per-lane 64-bit address arithmetic.  base and dst are uniform.
__device__ __forceinline__ void dma16s(const unsigned char *base, uint32_t off, unsigned char *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8 *)dst;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
        "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds)
        : "memory");
}
__device__ __forceinline__ void dma4s(const unsigned char *base, uint32_t off, unsigned char *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_u8 *)dst;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
        "global_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds)
        : "memory");
}

// `bytes` (a multiple of 4) from src into LDS at dst, all by DMA: whole
// 16-byte chunks when src is 16-byte aligned, the rest (and everything
// otherwise) as dwords.  The caller's wait_vm covers the copies.
__device__ __forceinline__ void stage_bytes(const unsigned char *src, int bytes, unsigned char *dst) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunks = ((uintptr_t)src & 15) ? 0 : bytes >> 4;
    for (int c0 = wave * 64; c0 < chunks; c0 += kThreads) {
        if (c0 + lane < chunks) dma16(src + 16 * (c0 + lane), dst + 16 * c0);
    }
    const int words = (bytes - (chunks << 4)) >> 2;
    const int base = chunks << 4;
    for (int w0 = wave * 64; w0 < words; w0 += kThreads) {
        if (w0 + lane < words) dma4(src + base + 4 * (w0 + lane), dst + base + 4 * w0);
    }
}

// quantize_row_q8 (kernel/quant_x.c:12-33) of the n_tok fp32 rows staged at
// xf into block_q8 rows at xs: 8 lanes x 4 values per block.  The task count
// and the stride are multiples of 8, so a block's 8 lanes are active
// together.  Work-group 0 also leaves the blocks at a.xq_out.
__device__ __forceinline__ void quantize_lds(const GemvArgs &a, const unsigned char *xf, unsigned char *xs) {
    const int blocks = a.n_tok * a.nb;
    for (int k = threadIdx.x; k < blocks * 8; k += kThreads) {
        const int e = k & 7, tb = k >> 3;
        const float4 v = *reinterpret_cast<const float4 *>(xf + (size_t)(tb * kQK + 4 * e) * 4);
        const float xv[4] = {v.x, v.y, v.z, v.w};
        unsigned char *blk = xs + (size_t)tb * kBlockBytes;
        quantize8x4(xv, reinterpret_cast<float *>(blk), blk + 4 + 4 * e, e == 0);
    }
    if (a.xq_out && blockIdx.x == 0) {
        __syncthreads();
        const uint32_t *src = reinterpret_cast<const uint32_t *>(xs);
        uint32_t *dst = reinterpret_cast<uint32_t *>(a.xq_out);
        for (int w = threadIdx.x; w < blocks * (kBlockBytes / 4); w += kThreads) dst[w] = src[w];
    }
}

// Every load is unconditional (rows past the end and groups past the last
// one are clamped to real data and masked out of the sums), so no load
// result is left unread on any path and the compiler never has to wait for
// one in-flight load before issuing the next.
// XF: the input is fp32 rows, staged raw and quantized in LDS (T <= 2).
// Q4: the matrices are tiled Q4: one 16-byte load per (row, block) instead of
// two, turned into the two code halves before the dot products.
template <int T, int RW, int GC, bool XF, bool Q4>
__global__ __launch_bounds__(256) void gemv_q8_kernel(GemvArgs a) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kGemvWaves + wave) * RW;
    const int cols = a.cols, nb = a.nb, ng = a.ng;
    // xs: [T][nb] block_q8, as in global memory; with XF the fp32 rows come
    // first in LDS and the blocks after them.
    unsigned char *xs = XF ? smem + (size_t)T * cols * 4 : smem;
    if (XF) stage_bytes(reinterpret_cast<const unsigned char *>(a.x), a.n_tok * cols * 4, smem);
    else stage_bytes(a.xq, a.n_tok * nb * kBlockBytes, smem);

    const unsigned char *wrow[RW];
    const float *drow[RW];
    float *yrow[RW];
    int ldy[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) {
        const int r = row0 + i < a.rows_total ? row0 + i : a.rows_total - 1;
        // Field-wise selects keep the segment in scalar registers (an indexed
        // a.seg[s] would be a vector load of the kernel arguments).
        const bool s0 = r < a.seg_end[0], s1 = !s0 && r < a.seg_end[1];
        const unsigned char *w = s0 ? a.seg[0].w : (s1 ? a.seg[1].w : a.seg[2].w);
        float *y = s0 ? a.seg[0].y : (s1 ? a.seg[1].y : a.seg[2].y);
        const int rows = s0 ? a.seg[0].rows : (s1 ? a.seg[1].rows : a.seg[2].rows);
        const int lr = r - (s0 ? 0 : (s1 ? a.seg_end[0] : a.seg_end[1]));
        const size_t rowb = Q4 ? (size_t)cols / 2 : (size_t)cols;   // code bytes per row
        wrow[i] = w + (size_t)lr * rowb;
        drow[i] = reinterpret_cast<const float *>(w + (size_t)rows * rowb) + (size_t)lr * nb;
        yrow[i] = y + lr;
        ldy[i] = rows;
    }

    float acc[RW][T];
#pragma unroll
    for (int i = 0; i < RW; i++)
#pragma unroll
        for (int t = 0; t < T; t++) acc[i][t] = 0.0f;

    for (int g0 = 0; g0 < ng; g0 += GC) {
        u32x4 wlo[GC][RW], whi[GC][RW];
        float wd[GC][RW];
#pragma unroll
        for (int u = 0; u < GC; u++) {
            const int g = g0 + u < ng ? g0 + u : ng - 1;
            const int rest = nb - g * kGroupBlocks;
            const int n = rest < kGroupBlocks ? rest : kGroupBlocks;
            const int bl = lane < n ? lane : n - 1;
#pragma unroll
            for (int i = 0; i < RW; i++) {
                if (Q4) {
                    wlo[u][i] = *reinterpret_cast<const u32x4 *>(wrow[i] + g * kGroupBytes4 + 16 * bl);
                } else {
                    const unsigned char *p = wrow[i] + g * kGroupBytes + 16 * bl;
                    wlo[u][i] = *reinterpret_cast<const u32x4 *>(p);
                    whi[u][i] = *reinterpret_cast<const u32x4 *>(p + 16 * n);
                }
                wd[u][i] = drow[i][g * kGroupBlocks + bl];
            }
        }
        if (g0 == 0) {
            // the activation copies, issued first, have landed once no more
            // than this wave's weight loads (2 or 3 per unit) are in flight
            wait_vm<(Q4 ? 2 : 3) * GC * RW>();
            __syncthreads();
            if (XF) {
                quantize_lds(a, smem, xs);
                __syncthreads();
            }
        }
#pragma unroll
        for (int u = 0; u < GC; u++) {
            const int g = g0 + u < ng ? g0 + u : ng - 1;
            const int rest = nb - g * kGroupBlocks;
            const int n = rest < kGroupBlocks ? rest : kGroupBlocks;
            const bool valid = lane < n && g0 + u < ng;
            const int bl = lane < n ? lane : n - 1;
            if (Q4) {
#pragma unroll
                for (int i = 0; i < RW; i++) {
                    const u32x4 w = wlo[u][i];
                    wlo[u][i] = u32x4{q4_lo16(w.x), q4_lo16(w.y), q4_lo16(w.z), q4_lo16(w.w)};
                    whi[u][i] = u32x4{q4_hi16(w.x), q4_hi16(w.y), q4_hi16(w.z), q4_hi16(w.w)};
                }
            }
            int s[T][RW];
            float xd[T];
#pragma unroll
            for (int t = 0; t < T; t++) {
                // Block 64g+bl of token t: d, then 8 dwords of codes (a 36-byte
                // lane stride is 9 banks apart: conflict-free).
                const uint32_t *xb = reinterpret_cast<const uint32_t *>(
                    xs + (size_t)(t * nb + g * kGroupBlocks + bl) * kBlockBytes);
                xd[t] = __uint_as_float(xb[0]);
#pragma unroll
                for (int i = 0; i < RW; i++) {
                    int d = 0;
                    d = __builtin_amdgcn_sdot4(wlo[u][i].x, xb[1], d, false);
                    d = __builtin_amdgcn_sdot4(wlo[u][i].y, xb[2], d, false);
                    d = __builtin_amdgcn_sdot4(wlo[u][i].z, xb[3], d, false);
                    d = __builtin_amdgcn_sdot4(wlo[u][i].w, xb[4], d, false);
                    d = __builtin_amdgcn_sdot4(whi[u][i].x, xb[5], d, false);
                    d = __builtin_amdgcn_sdot4(whi[u][i].y, xb[6], d, false);
                    d = __builtin_amdgcn_sdot4(whi[u][i].z, xb[7], d, false);
                    d = __builtin_amdgcn_sdot4(whi[u][i].w, xb[8], d, false);
                    s[t][i] = Q4 ? d >> 4 : d;
                }
            }
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int i = 0; i < RW; i++) {
                    const float p = ((float)s[t][i] * wd[u][i]) * xd[t];
                    acc[i][t] += valid ? p : 0.0f;
                }
        }
    }

#pragma unroll
    for (int i = 0; i < RW; i++) {
        if (row0 + i >= a.rows_total) continue;
#pragma unroll
        for (int t = 0; t < T; t++) {
            if (t < a.n_tok) {
                const float v = wave_sum(acc[i][t]);
                if (lane == 0) yrow[i][(size_t)t * ldy[i]] = v;
            }
        }
    }
}

// LDS of a launch: t block_q8 rows, plus the t fp32 rows they are quantized
// from when the input is fp32.
size_t lds_bytes(int t, int nb, bool xf) {
    return (size_t)t * nb * kBlockBytes + (xf ? (size_t)t * nb * kQK * 4 : 0);
}

// ---------------------------------------------------------------------------
// Many tokens: int8 MFMA GEMM.  A work-group of 8 waves computes a 128-row x
// 128-token tile; wave w owns rows 32(w%4)..+31 (two 16-row tiles) of tokens
// 64(w/4)..+63 (four 16-token tiles).  The K dimension goes 4 blocks (128
// codes) per stage through two LDS buffers filled by direct-to-LDS copies, one
// stage ahead of the one being multiplied; at 73.7 KB two work-groups share a
// CU, so one's scaling overlaps the other's products.  Per block,
// v_mfma_i32_16x16x32_i8 gives the exact int32 block dot for a 16 x 16 tile,
// and each lane folds its four into fp32 with fma(s, w_d * x_d, acc): one
// fp32 scaling per (row, token, block), the reference's per-block product
// (kernel/q8_scalar.c:9-11) with one rounding fewer, summed over blocks in
// order.
//
// Tile order: work-groups are dealt to the 8 XCDs round-robin, so the grid is
// laid out so that every token tile of one row tile runs on the same XCD
// (work-group w: XCD w % 8, row tile 8 (w/8 / n_tt) + w % 8) and the tile's
// 128 weight rows are read from HBM once into that XCD's L2.
//
// LDS per stage (36,864 B):
//   A   [4 blocks][2 halves][128 rows][16 B]   weight codes, one copy per 16 B
//   WD  [4 blocks][128 rows] fp32             weight scales
//   B   [128 tokens][4 blocks x 36 B]         the tokens' block_q8, as stored:
//       with 16-byte aligned rows and a block count that is a multiple of 4,
//       a token's 144 bytes are nine 16-byte copies (three rounds of 512, the
//       last round's surplus lanes, whole waves, issue none); otherwise 36
//       dword copies per token.
constexpr int kGemmThreads = 512;
constexpr int kGemmRows = 128, kGemmToks = 128, kGemmKB = 4, kGemmBufs = 2;
constexpr int kGemmA = kGemmKB * 2 * kGemmRows * 16;            // 16,384
constexpr int kGemmWD = kGemmKB * kGemmRows * 4;                // 2,048
constexpr int kGemmBRow = kGemmKB * kBlockBytes;                // 144 bytes per token
constexpr int kGemmB = kGemmToks * kGemmBRow;                   // 18,432
constexpr int kGemmBChunks = kGemmB / 16;                       // 1,152 16-byte copies
constexpr int kGemmBRounds = (kGemmBChunks + kGemmThreads - 1) / kGemmThreads;   // 3
constexpr int kGemmStage = kGemmA + kGemmWD + kGemmB;           // 36,864 (16-byte multiple)
constexpr int kGemmBWords = kGemmB / 4;                         // 4,608 dword copies
constexpr int kGemmXsCodes = kGemmKB * kQK * kGemmToks;          // 16,384: split-layout codes, then scales
static_assert(kGemmXsCodes + kGemmKB * kGemmToks * 4 == kGemmB, "the split layout fills the token stage");
static_assert(kGemmBChunks % 64 == 0 && (kGemmBRounds - 1) * kGemmThreads < kGemmBChunks,
              "the last B round's copies past the tile are whole waves");
static_assert(kGemmA / 16 % kGemmThreads == 0 && kGemmWD / 4 % kGemmThreads == 0 &&
              kGemmBWords % kGemmThreads == 0, "whole copy rounds per stage");

__device__ __forceinline__ long lds_pair(const unsigned char *p) {
    const uint32_t lo = *reinterpret_cast<const uint32_t *>(p);
    const uint32_t hi = *reinterpret_cast<const uint32_t *>(p + 4);
    return (long)(((unsigned long)hi << 32) | lo);
}

// BX4: the activation rows are 16-byte aligned and nb % 4 == 0.
// Q4: tiled Q4 matrices.  A holds [4 blocks][128 rows][16 B] nibble bytes (one
// copy per thread instead of two); each lane turns its 8 bytes into 16 x its
// 8 codes (low nibbles for k < 16, high for k >= 16), and the int32 products
// are shifted back by 4 before scaling.
template <bool BX4, bool Q4, bool UNI, bool XS>
__global__ __launch_bounds__(512) void gemm_q8_kernel(GemvArgs a) {
    static_assert(!UNI || BX4, "uniform copies need whole 16-byte stages");
    static_assert(!XS || UNI, "the split layout is copied from uniform bases");
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lg = lane >> 4;
    const int cols = a.cols, nb = a.nb;
    const int n_tt = (a.n_tok + kGemmToks - 1) / kGemmToks;
    const int n_rt = (a.rows_total + kGemmRows - 1) / kGemmRows;
    // split ks of ksplit takes the ks-th run of stages; the grid repeats the
    // tile order once per split (a multiple of 8 work-groups each, so the XCD
    // of a tile is the same in every split)
    const int g0 = gridDim.x / a.ksplit;
    const int bx = blockIdx.x % g0, ks = blockIdx.x / g0;
    const int k = bx >> 3;
    const int rt = (k / n_tt) * 8 + (bx & 7), tt = k % n_tt;
    if (rt >= n_rt) return;   // the padding of the last row of XCD groups
    const int row0 = rt * kGemmRows, tok0 = tt * kGemmToks;
    const int stages = (nb + kGemmKB - 1) / kGemmKB;
    const int st_begin = ks * stages / a.ksplit, st_end = (ks + 1) * stages / a.ksplit;
    const int wr = 32 * (wave & 3), wt = 64 * (wave >> 2);

    // A chunk c = tid + 512 j -> (block c / 256, half (c / 128) & 1, row c % 128):
    // row = tid % 128 for every j; WD dword c = tid -> (block c / 128, row c % 128).
    const int my_row = tid & 127;
    const unsigned char *wrow;
    const float *drow;
    {
        const int r = row0 + my_row < a.rows_total ? row0 + my_row : a.rows_total - 1;
        const bool s0 = r < a.seg_end[0], s1 = !s0 && r < a.seg_end[1];
        const unsigned char *w = s0 ? a.seg[0].w : (s1 ? a.seg[1].w : a.seg[2].w);
        const int rows = s0 ? a.seg[0].rows : (s1 ? a.seg[1].rows : a.seg[2].rows);
        const int lr = r - (s0 ? 0 : (s1 ? a.seg_end[0] : a.seg_end[1]));
        const size_t rowb = Q4 ? (size_t)cols / 2 : (size_t)cols;
        wrow = w + (size_t)lr * rowb;
        drow = reinterpret_cast<const float *>(w + (size_t)rows * rowb) + (size_t)lr * nb;
    }

    // Copies from uniform bases, when every tile lies in one segment (the
    // host checks that segment ends fall on tile boundaries and that offsets
    // fit 32 bits) and every stage is whole (16-byte token rows, nb % 4 == 0):
    // a stage's four blocks then lie in one 64-block group, the block and
    // half of each copy are the same for the whole wave, and a copy is a
    // scalar base (segment, group, block, half) plus this lane's fixed row
    // offset, with no vector address arithmetic per stage.
    constexpr bool uni = UNI;
    const unsigned char *useg = nullptr;   // the tile's segment: codes, then scales at uscale
    size_t uscale = 0;
    uint32_t vrow = 0, vdrow = 0, vb[kGemmBRounds];
    if constexpr (uni) {
        const bool s0 = row0 < a.seg_end[0], s1 = !s0 && row0 < a.seg_end[1];
        useg = s0 ? a.seg[0].w : (s1 ? a.seg[1].w : a.seg[2].w);
        int rows = s0 ? a.seg[0].rows : (s1 ? a.seg[1].rows : a.seg[2].rows);
        int start = s0 ? 0 : (s1 ? a.seg_end[0] : a.seg_end[1]);
        int r = row0 + my_row < a.rows_total ? row0 + my_row : a.rows_total - 1;
        if (a.hq) {
            // paired tile rt: rows 64 rt.. of the gate matrix, then the same
            // rows of the up matrix.  A wave's copies all lie in one half
            // (row tid % 128 = 64 (wave & 1) + lane), so its base stays uniform.
            useg = (wave & 1) ? a.seg[1].w : a.seg[0].w;
            rows = a.seg[0].rows;
            start = 0;
            r = 64 * rt + lane;
        }
        const uint32_t rowb = Q4 ? (uint32_t)cols / 2 : (uint32_t)cols;
        uscale = (size_t)rows * rowb;
        vrow = (uint32_t)(r - start) * rowb;
        vdrow = (uint32_t)(r - start) * (uint32_t)nb * 4u;
        if constexpr (XS) {
            // every copy of this lane is for token 64 (wave & 1) + lane of the
            // tile: its 16-byte half-block and its scale in the block-major runs
            const int tk = 64 * (wave & 1) + lane;
            const int t = tok0 + tk < a.n_tok ? tok0 + tk : a.n_tok - 1;
            vb[0] = 16u * (uint32_t)t;
            vb[1] = 4u * (uint32_t)t;
        } else {
#pragma unroll
            for (int j = 0; j < kGemmBRounds; j++) {
                const int c = tid + kGemmThreads * j;
                const int cc = c < kGemmBChunks ? c : kGemmBChunks - 1;
                const int tk = cc / 9, piece = cc - 9 * tk;
                const int t = tok0 + tk < a.n_tok ? tok0 + tk : a.n_tok - 1;
                vb[j] = (uint32_t)t * (uint32_t)nb * (uint32_t)kBlockBytes + 16u * (uint32_t)piece;
            }
        }
    }

    // The token rows' sources of this thread's B copies, fixed over the stages
    // (a stage only adds 36 bytes per block to each).
    const unsigned char *bsrc[kGemmBRounds];
    if (BX4) {
#pragma unroll
        for (int j = 0; j < kGemmBRounds; j++) {
            const int c = tid + kGemmThreads * j;
            const int cc = c < kGemmBChunks ? c : kGemmBChunks - 1;
            const int tk = cc / 9, piece = cc - 9 * tk;
            const int t = tok0 + tk < a.n_tok ? tok0 + tk : a.n_tok - 1;
            bsrc[j] = a.xq + (size_t)t * nb * kBlockBytes + 16 * piece;
        }
    }

    // the same copies from uniform bases (whole stages only)
    auto issue_uni = [&](int st, unsigned char *buf) {
        const int b0 = st * kGemmKB;
        const int g = b0 / kGroupBlocks, i0 = b0 - g * kGroupBlocks;
        const int n = nb - g * kGroupBlocks < kGroupBlocks ? nb - g * kGroupBlocks : kGroupBlocks;
        if (Q4) {
            // chunk tid -> (block tid / 128, row tid % 128): the block is the wave's
            dma16s(useg + 16 * (b0 + (wave >> 1)), vrow, buf + 16 * 64 * wave);
        } else {
#pragma unroll
            for (int j = 0; j < kGemmA / 16 / kGemmThreads; j++) {
                const int c = 64 * wave + kGemmThreads * j;   // the wave's first chunk
                const int blk = c >> 8, half = (c >> 7) & 1;
                dma16s(useg + g * kGroupBytes + 16 * (i0 + blk) + (half ? 16 * n : 0), vrow, buf + 16 * c);
            }
        }
        dma4s(useg + uscale + 4 * (b0 + (wave >> 1)), vdrow, buf + kGemmA + 4 * 64 * wave);
        if constexpr (XS) {
            // codes: chunk c -> (block c / 256, half (c / 128) & 1, token c % 128),
            // the same [block][half][row] 16-byte layout as the weights, one
            // contiguous KiB per wave; scales: dword c -> (block c / 128, token c % 128)
            const size_t n16 = 16 * (size_t)a.n_tok;
#pragma unroll
            for (int j = 0; j < kGemmA / 16 / kGemmThreads; j++) {
                const int c = 64 * wave + kGemmThreads * j;
                const int blk = c >> 8, half = (c >> 7) & 1;
                dma16s(a.xq + (size_t)(2 * (b0 + blk) + half) * n16 + 16 * tok0, vb[0] - 16u * (uint32_t)tok0,
                       buf + kGemmA + kGemmWD + 16 * c);
            }
            dma4s(a.xq + (size_t)a.n_tok * cols + 4 * ((size_t)(b0 + (wave >> 1)) * a.n_tok + tok0),
                  vb[1] - 4u * (uint32_t)tok0, buf + kGemmA + kGemmWD + kGemmXsCodes + 4 * 64 * wave);
        } else {
#pragma unroll
            for (int j = 0; j < kGemmBRounds; j++) {
                const int c = 64 * wave + kGemmThreads * j;
                if (c < kGemmBChunks)
                    dma16s(a.xq + (size_t)b0 * kBlockBytes, vb[j], buf + kGemmA + kGemmWD + 16 * c);
            }
        }
    };

    // kGemmCopies direct-to-LDS copies per thread per stage, nothing else
    auto issue = [&](int st, unsigned char *buf) {
        if constexpr (uni) {
            issue_uni(st, buf);
            return;
        }
        const int b0 = st * kGemmKB;
        if (Q4) {
            // chunk tid -> (block tid / 128, row tid % 128)
            const int blk = tid >> 7;
            const int b = b0 + blk < nb ? b0 + blk : nb - 1;
            dma16(wrow + 16 * b, buf + 16 * (tid - lane));
        } else {
#pragma unroll
            for (int j = 0; j < kGemmA / 16 / kGemmThreads; j++) {
                const int c = tid + kGemmThreads * j;
                const int blk = c >> 8, half = (c >> 7) & 1;
                const int b = b0 + blk < nb ? b0 + blk : nb - 1;
                dma16(wrow + tiled_offset(nb, b, 16 * half), buf + 16 * (c - lane));
            }
        }
        {
            const int blk = tid >> 7;
            const int b = b0 + blk < nb ? b0 + blk : nb - 1;
            dma4(drow + b, buf + kGemmA + 4 * (tid - lane));
        }
        if (BX4) {
            // the last round's copies past the tile are left out (whole waves)
#pragma unroll
            for (int j = 0; j < kGemmBRounds; j++)
                if (tid + kGemmThreads * j < kGemmBChunks)
                    dma16(bsrc[j] + b0 * kBlockBytes, buf + kGemmA + kGemmWD + 16 * (tid + kGemmThreads * j - lane));
        } else {
#pragma unroll
            for (int j = 0; j < kGemmBWords / kGemmThreads; j++) {
                const int c = tid + kGemmThreads * j;
                const int tk = c / (kGemmBRow / 4), w = c - tk * (kGemmBRow / 4);
                const int blk = w / 9;
                const int t = tok0 + tk < a.n_tok ? tok0 + tk : a.n_tok - 1;
                const int b = b0 + blk < nb ? b0 + blk : nb - 1;
                dma4(a.xq + ((size_t)t * nb + b) * kBlockBytes + 4 * (w - 9 * blk),
                     buf + kGemmA + kGemmWD + 4 * (c - lane));
            }
        }
    };

    float acc[2][4][4];
#pragma unroll
    for (int r2 = 0; r2 < 2; r2++)
#pragma unroll
        for (int t4 = 0; t4 < 4; t4++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[r2][t4][i] = 0.0f;

    // Two buffers (73.7 KB, so two work-groups share a CU): stage st+1 is
    // copied while stage st is multiplied.
    issue(st_begin, smem);
    for (int st = st_begin; st < st_end; st++) {
        unsigned char *buf = smem + ((st - st_begin) & 1) * kGemmStage;
        wait_vm<0>();      // this wave's copies of stage st have landed
        __syncthreads();   // stage st is in LDS everywhere; stage st-1's buffer is free
        if (st + 1 < st_end) issue(st + 1, smem + ((st + 1 - st_begin) & 1) * kGemmStage);
        const unsigned char *A = buf, *WD = buf + kGemmA, *B = buf + kGemmA + kGemmWD;
        // two blocks at a time: the second block's LDS reads and products
        // overlap the first one's scaling
#pragma unroll 2
        for (int blk = 0; blk < kGemmKB; blk++) {
            // (with 16-byte token rows every stage is whole)
            const bool valid = BX4 || st * kGemmKB + blk < nb;
            long av[2], bv[4];
            float wd[2][4], xd[4];
#pragma unroll
            for (int r2 = 0; r2 < 2; r2++) {
                const int row = wr + 16 * r2;
                if (Q4) {
                    const long raw = lds_pair(A + ((blk * kGemmRows) + row + l16) * 16 + 8 * (lg & 1));
                    const uint32_t w0 = (uint32_t)raw, w1 = (uint32_t)((unsigned long)raw >> 32);
                    const uint32_t c0 = lg < 2 ? q4_lo16(w0) : q4_hi16(w0);
                    const uint32_t c1 = lg < 2 ? q4_lo16(w1) : q4_hi16(w1);
                    av[r2] = (long)(((unsigned long)c1 << 32) | c0);
                } else {
                    av[r2] = lds_pair(A + (((blk * 2 + (lg >> 1)) * kGemmRows) + row + l16) * 16 + 8 * (lg & 1));
                }
                const float4 w4 = *reinterpret_cast<const float4 *>(WD + (blk * kGemmRows + row + 4 * lg) * 4);
                wd[r2][0] = w4.x; wd[r2][1] = w4.y; wd[r2][2] = w4.z; wd[r2][3] = w4.w;
            }
#pragma unroll
            for (int t4 = 0; t4 < 4; t4++) {
                if constexpr (XS) {
                    // 8-byte reads of 16-byte rows: no bank conflicts, as for A
                    bv[t4] = lds_pair(B + ((blk * 2 + (lg >> 1)) * kGemmToks + wt + 16 * t4 + l16) * 16 + 8 * (lg & 1));
                    xd[t4] = *reinterpret_cast<const float *>(B + kGemmXsCodes + (blk * kGemmToks + wt + 16 * t4 + l16) * 4);
                } else {
                    const unsigned char *tb = B + (wt + 16 * t4 + l16) * kGemmBRow + blk * kBlockBytes;
                    bv[t4] = lds_pair(tb + 4 + 8 * lg);
                    // the staged scale is always a real block's (past nb the copies
                    // repeat block nb-1): load it unconditionally and select, so no
                    // branch splits the block's LDS reads from its products
                    const float xv = *reinterpret_cast<const float *>(tb);
                    xd[t4] = valid ? xv : 0.0f;
                }
            }
            // all eight products first, so that each one's latency hides
            // under the others before its results are read
            v4i c[2][4];
#pragma unroll
            for (int r2 = 0; r2 < 2; r2++)
#pragma unroll
                for (int t4 = 0; t4 < 4; t4++)
                    c[r2][t4] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[r2], bv[t4], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int r2 = 0; r2 < 2; r2++)
#pragma unroll
                for (int t4 = 0; t4 < 4; t4++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[r2][t4][i] = fmaf((float)(Q4 ? c[r2][t4][i] >> 4 : c[r2][t4][i]), wd[r2][i] * xd[t4],
                                              acc[r2][t4][i]);
        }
    }

    // y[t][r]: lane (l16, lg) holds rows 4lg..4lg+3 of each 16-row tile for
    // token l16 of each 16-token tile.  A split writes its partial instead.
    if (UNI && XS && a.hq) {
        // the paired tile's gate (rows 0-63) and up (rows 64-127) values meet
        // in LDS as [token][row] with 132-float token rows (a float4 store of
        // 16 tokens then covers all 64 banks); then h = silu(g) * u of the
        // tile's two 32-row blocks, quantized as silu_quant8_kernel does, 8
        // lanes x 4 values per (block, token), written in the split layout
        // (codes of block b, token t at ((2b + half) n + t) 16, scales [b][t]
        // after the n * inter code bytes)
        constexpr int kHs = kGemmRows + 4;
        static_assert(kGemmToks * kHs * 4 <= kGemmBufs * kGemmStage, "the fp32 tile fits the stage buffers");
        float *hs = reinterpret_cast<float *>(smem);
        __syncthreads();   // every wave is done with the last stage
#pragma unroll
        for (int r2 = 0; r2 < 2; r2++)
#pragma unroll
            for (int t4 = 0; t4 < 4; t4++)
                *reinterpret_cast<float4 *>(hs + (wt + 16 * t4 + l16) * kHs + wr + 16 * r2 + 4 * lg) =
                    make_float4(acc[r2][t4][0], acc[r2][t4][1], acc[r2][t4][2], acc[r2][t4][3]);
        __syncthreads();
        const int n = a.n_tok, inter = a.seg[0].rows;
        float *scales = reinterpret_cast<float *>(a.hq + (size_t)n * inter);
        // (block, token) units in block-major order: consecutive units are
        // consecutive tokens, so a wave's code stores are 128 contiguous bytes
#pragma unroll
        for (int j = 0; j < 2 * kGemmToks * 8 / kGemmThreads; j++) {
            const int q = tid + kGemmThreads * j;
            const int e = q & 7, bl = q >> 10, tk = (q >> 3) & (kGemmToks - 1);
            const int t = tok0 + tk;
            if (t >= n) continue;   // whole 8-lane groups share t
            const float4 g4 = *reinterpret_cast<const float4 *>(hs + tk * kHs + 32 * bl + 4 * e);
            const float4 u4 = *reinterpret_cast<const float4 *>(hs + tk * kHs + 64 + 32 * bl + 4 * e);
            const float h[4] = {silu_mul(g4.x, u4.x), silu_mul(g4.y, u4.y), silu_mul(g4.z, u4.z),
                                silu_mul(g4.w, u4.w)};
            const size_t gb = 2 * (size_t)rt + bl;
            quantize8x4(h, scales + gb * n + t, a.hq + ((2 * gb + (e >> 2)) * n + t) * 16 + 4 * (e & 3), e == 0);
        }
        return;
    }
    if (a.ksplit > 1) {
        float *p = a.part + (size_t)ks * a.n_tok * a.rows_total;
#pragma unroll
        for (int r2 = 0; r2 < 2; r2++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = row0 + wr + 16 * r2 + 4 * lg + i;
#pragma unroll
                for (int t4 = 0; t4 < 4; t4++) {
                    const int t = tok0 + wt + 16 * t4 + l16;
                    if (r < a.rows_total && t < a.n_tok) p[(size_t)t * a.rows_total + r] = acc[r2][t4][i];
                }
            }
        return;
    }
#pragma unroll
    for (int r2 = 0; r2 < 2; r2++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = row0 + wr + 16 * r2 + 4 * lg + i;
            if (r >= a.rows_total) continue;
            const bool s0 = r < a.seg_end[0], s1 = !s0 && r < a.seg_end[1];
            float *y = s0 ? a.seg[0].y : (s1 ? a.seg[1].y : a.seg[2].y);
            const int rows = s0 ? a.seg[0].rows : (s1 ? a.seg[1].rows : a.seg[2].rows);
            const int lr = r - (s0 ? 0 : (s1 ? a.seg_end[0] : a.seg_end[1]));
#pragma unroll
            for (int t4 = 0; t4 < 4; t4++) {
                const int t = tok0 + wt + 16 * t4 + l16;
                if (t < a.n_tok) y[(size_t)t * rows + lr] = acc[r2][t4][i];
            }
        }
    }
}

// The split-K sum: y of (token t, row r) is the splits' partials added in
// split order (the same order on every launch).
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemvArgs a) {
    const size_t total = (size_t)a.n_tok * a.rows_total;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        float acc = a.part[i];
        for (int s = 1; s < a.ksplit; s++) acc += a.part[(size_t)s * total + i];
        const int t = (int)(i / a.rows_total), r = (int)(i - (size_t)t * a.rows_total);
        const bool s0 = r < a.seg_end[0], s1 = !s0 && r < a.seg_end[1];
        float *y = s0 ? a.seg[0].y : (s1 ? a.seg[1].y : a.seg[2].y);
        const int rows = s0 ? a.seg[0].rows : (s1 ? a.seg[1].rows : a.seg[2].rows);
        const int lr = r - (s0 ? 0 : (s1 ? a.seg_end[0] : a.seg_end[1]));
        y[(size_t)t * rows + lr] = acc;
    }
}

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    return (s && *s) ? atoi(s) : dflt;
}

// Rows per wave: enough work-groups to put two on every CU where the row
// count allows (TQ_HIP_GEMV_RW=1|2|4 overrides).  Four rows only where a row
// has 4 or more 64-block groups, or for Q4: Q8 rows of 4096 columns (two
// groups) keep more waves streaming at two rows (8B gate/up, 28672 x 4096:
// model forward 437 -> 449 tokens/s), while 10240 x 8192 is faster at four
// (36.1 against 38.2 us).
int pick_rw(int rows_total, int ng, bool q4) {
    const int forced = env_int("TQ_HIP_GEMV_RW", 0);
    if (forced == 1 || forced == 2 || forced == 4) return forced;
    if (rows_total >= 4 * kGemvWaves * 512 && (q4 || ng >= 4)) return 4;
    if (rows_total >= 2 * kGemvWaves * 512) return 2;
    return 1;
}

// Groups per row per pass: up to 8 (row, group) units in flight per wave (16
// for Q4, whose units are half the bytes), never more groups than a row has
// (TQ_HIP_GEMV_GC=1|2|4 overrides).
int pick_gc(int ng, int rw, bool q4) {
    const int forced = env_int("TQ_HIP_GEMV_GC", 0);
    int gc = (forced == 1 || forced == 2 || forced == 4) ? forced : (q4 ? 16 : 8) / rw;
    if (gc > 4) gc = 4;
    while (gc > 1 && gc / 2 >= ng) gc /= 2;
    return gc;
}

// Largest token count per launch whose staged rows fit the LDS budget
// (fp32 input: 1 or 2 rows, quantized in LDS).
int pick_tokens(int nb, bool xf) {
    for (int t : {8, 4, 2, 1})
        if ((!xf || t <= 2) && lds_bytes(t, nb, xf) <= kMaxStageBytes) return t;
    return 0;
}

template <int T, int RW, int GC, bool XF, bool Q4>
hipError_t launch_t(const GemvArgs &a, hipStream_t s) {
    const int waves = (a.rows_total + RW - 1) / RW;
    const int grid = (waves + kGemvWaves - 1) / kGemvWaves;
    const size_t lds = (lds_bytes(T, a.nb, XF) + 15) & ~(size_t)15;
    if (lds > kDefaultLdsLimit) {
        static bool opted = false;   // once per instantiation (and process)
        if (!opted) {
            const hipError_t e = hipFuncSetAttribute((const void *)gemv_q8_kernel<T, RW, GC, XF, Q4>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)kMaxStageBytes);
            if (e != hipSuccess) return e;
            opted = true;
        }
    }
    hipLaunchKernelGGL((gemv_q8_kernel<T, RW, GC, XF, Q4>), dim3(grid), dim3(kThreads), lds, s, a);
    return hipGetLastError();
}

template <int RW, int GC, bool Q4>
hipError_t launch_tok_f(const GemvArgs &a, int tmax, bool xf, hipStream_t s) {
    if (xf) return tmax == 2 ? launch_t<2, RW, GC, true, Q4>(a, s) : launch_t<1, RW, GC, true, Q4>(a, s);
    switch (tmax) {
        case 8: return launch_t<8, RW, GC, false, Q4>(a, s);
        case 4: return launch_t<4, RW, GC, false, Q4>(a, s);
        case 2: return launch_t<2, RW, GC, false, Q4>(a, s);
        default: return launch_t<1, RW, GC, false, Q4>(a, s);
    }
}

template <int RW, int GC>
hipError_t launch_tok(const GemvArgs &a, int tmax, bool xf, hipStream_t s) {
    return a.q4 ? launch_tok_f<RW, GC, true>(a, tmax, xf, s) : launch_tok_f<RW, GC, false>(a, tmax, xf, s);
}

hipError_t launch_gemv(const GemvArgs &a, int tcap, bool xf, int rw, int gc, hipStream_t s) {
    switch (rw * 16 + gc) {
        case 0x11: return launch_tok<1, 1>(a, tcap, xf, s);
        case 0x12: return launch_tok<1, 2>(a, tcap, xf, s);
        case 0x14: return launch_tok<1, 4>(a, tcap, xf, s);
        case 0x21: return launch_tok<2, 1>(a, tcap, xf, s);
        case 0x22: return launch_tok<2, 2>(a, tcap, xf, s);
        case 0x24: return launch_tok<2, 4>(a, tcap, xf, s);
        case 0x41: return launch_tok<4, 1>(a, tcap, xf, s);
        case 0x44: return launch_tok<4, 4>(a, tcap, xf, s);
        default: return launch_tok<4, 2>(a, tcap, xf, s);
    }
}

// From how many tokens on (block_q8 input) the MFMA GEMM runs instead of GEMV
// launches of tmax tokens each (TQ_HIP_GEMM_MIN_TOKENS overrides).  A GEMV
// launch streams the weights once (about 5 TB/s, plus 2 us of launch), so
// its cost grows with the token count; the GEMM's first round of 128-row
// tiles costs its K loop, about 0.0183 us per column on MI355X, whatever the
// token count.  Measured crossovers: 6144 x 4096 between 64 and 96 tokens
// (77 against 62 us at 64), 28672 x 4096 between 16 and 32, 4096 x 14336
// between 64 and 96; the model below puts them at 80, 22 and 70.
int gemm_min_tokens(int rows, int cols, int tmax) {
    const int v = env_int("TQ_HIP_GEMM_MIN_TOKENS", 0);
    if (v > 0) return v;
    const double chunk_us = (double)rows * cols * (kBlockBytes / (double)kQK) / 5.0e6 + 2.0;
    const double gemm_us = 0.0183 * cols + 2.0;
    const int n = (int)(tmax * gemm_us / chunk_us) + 1;
    return n < 16 ? 16 : (n > 256 ? 256 : n);
}

// Every 128-row tile inside one segment (segment ends on tile boundaries) and
// 32-bit copy offsets: the uniform-base copies apply.
bool gemm_uniform(const GemvArgs &a) {
    for (int i = 0; i < kMaxSegs; i++) {
        if (a.seg_end[i] < a.rows_total && a.seg_end[i] % kGemmRows != 0) return false;
        const size_t rowb = a.q4 ? (size_t)a.cols / 2 : (size_t)a.cols;
        if ((size_t)a.seg[i].rows * (rowb + 4 * (size_t)a.nb) >= ((size_t)1 << 31)) return false;
    }
    return (size_t)a.n_tok * a.nb * kBlockBytes < ((size_t)1 << 31);
}

hipError_t launch_gemm(const GemvArgs &a, int ksplit, hipStream_t s) {
    const int n_rt = (a.rows_total + kGemmRows - 1) / kGemmRows;
    const int n_tt = (a.n_tok + kGemmToks - 1) / kGemmToks;
    const long groups = ((long)n_rt + 7) / 8;   // row tiles per XCD, rounded up
    const long grid = groups * 8 * n_tt * ksplit;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    const size_t lds = (size_t)kGemmBufs * kGemmStage;
    static bool opted = false;
    if (!opted) {
        for (const void *f : {(const void *)gemm_q8_kernel<true, false, false, false>,
                              (const void *)gemm_q8_kernel<false, false, false, false>,
                              (const void *)gemm_q8_kernel<true, true, false, false>,
                              (const void *)gemm_q8_kernel<false, true, false, false>,
                              (const void *)gemm_q8_kernel<true, false, true, false>,
                              (const void *)gemm_q8_kernel<true, true, true, false>,
                              (const void *)gemm_q8_kernel<true, false, true, true>,
                              (const void *)gemm_q8_kernel<true, true, true, true>}) {
            const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        opted = true;
    }
    const bool bx4 = (((uintptr_t)a.xq & 15) == 0) && a.nb % kGemmKB == 0;
    GemvArgs u = a;
    u.ksplit = ksplit;
    u.uni_tiles = gemm_uniform(a);
    if (a.xs && !(bx4 && u.uni_tiles)) return hipErrorInvalidValue;   // the caller's plan and this disagree
    // paired gate/up tiles: one unsplit split-layout GEMM over two segments
    // of equal rows, a multiple of 64
    if (a.hq && (ksplit != 1 || !a.xs || a.seg[0].rows != a.seg[1].rows || a.seg[0].rows % 64 != 0 ||
                 a.rows_total != 2 * a.seg[0].rows))
        return hipErrorInvalidValue;
    const dim3 g((unsigned)grid), b(kGemmThreads);
    if (a.q4) {
        if (a.xs)
            hipLaunchKernelGGL((gemm_q8_kernel<true, true, true, true>), g, b, lds, s, u);
        else if (bx4 && u.uni_tiles)
            hipLaunchKernelGGL((gemm_q8_kernel<true, true, true, false>), g, b, lds, s, u);
        else if (bx4)
            hipLaunchKernelGGL((gemm_q8_kernel<true, true, false, false>), g, b, lds, s, u);
        else
            hipLaunchKernelGGL((gemm_q8_kernel<false, true, false, false>), g, b, lds, s, u);
    } else {
        if (a.xs)
            hipLaunchKernelGGL((gemm_q8_kernel<true, false, true, true>), g, b, lds, s, u);
        else if (bx4 && u.uni_tiles)
            hipLaunchKernelGGL((gemm_q8_kernel<true, false, true, false>), g, b, lds, s, u);
        else if (bx4)
            hipLaunchKernelGGL((gemm_q8_kernel<true, false, false, false>), g, b, lds, s, u);
        else
            hipLaunchKernelGGL((gemm_q8_kernel<false, false, false, false>), g, b, lds, s, u);
    }
    if (ksplit > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const size_t total = (size_t)a.n_tok * a.rows_total;
        const size_t blocks = (total + 255) / 256 < 2048 ? (total + 255) / 256 : 2048;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, s, u);
    }
    return hipGetLastError();
}

// Split-K GEMM while the tiles alone leave CUs of the 256 idle (each tile
// then runs the whole K loop): K is cut into S runs of stages, as many as
// keep the grid within one round of 512 work-groups (two per CU), each split
// writing a partial tile that one more launch sums in split order.  The 8B
// MLP over 16 / 64 / 256 / 512 rows: 130 / 141 / 272 / 481 us against
// 134 / 325 / 427 / 570 without.
constexpr int kSplitWgs = 512;

int gemm_ksplit(int rows, int cols, int n_tok) {
    if (n_tok < 16) return 1;
    const long wgs = ((long)(rows + kGemmRows - 1) / kGemmRows + 7) / 8 * 8 * ((n_tok + kGemmToks - 1) / kGemmToks);
    // once every CU holds a tile, splitting adds occupancy but not CUs, and
    // the partials' traffic outweighs it (4,096 x 14,336 at 1,024 tokens)
    if (wgs >= kSplitWgs / 2) return 1;
    const int stages = (cols / kQK + kGemmKB - 1) / kGemmKB;
    long sp = kSplitWgs / wgs;
    if (sp > stages) sp = stages;
    return sp < 2 ? 1 : (int)sp;
}

// The GEMM launch run_gemv makes over n_tok rows of block_q8 input (its K
// split count), or 0 for GEMV launches.  With a workspace for the partials a
// few tokens take the split-K GEMM; otherwise the cost model decides.
int gemm_plan(const GemvArgs &a, int n_tok) {
    if (a.x != nullptr) return 0;
    const int ksplit = a.part ? gemm_ksplit(a.rows_total, a.cols, n_tok) : 1;
    const bool split = ksplit > 1 && (size_t)ksplit * n_tok * a.rows_total <= a.part_floats &&
                       env_int("TQ_HIP_GEMM_SPLIT", 1) != 0;
    if (split) return ksplit;
    return n_tok >= gemm_min_tokens(a.rows_total, a.cols, pick_tokens(a.nb, false)) ? 1 : 0;
}

// Whether the matmul's input should be quantized into the split layout:
// internal callers (a partials workspace) whose launch is a GEMM with
// uniform-base copies over whole stages, xq 16-byte aligned
// (TQ_HIP_GEMM_XS=0 keeps block_q8 rows).
bool xs_layout(const GemvArgs &a, int n_tok, const void *xq) {
    if (!a.part || a.x || ((uintptr_t)xq & 15) || a.nb % kGemmKB || env_int("TQ_HIP_GEMM_XS", 1) == 0) return false;
    GemvArgs t = a;
    t.n_tok = n_tok;
    return gemm_plan(a, n_tok) > 0 && gemm_uniform(t);
}

// Runs the matmul over all tokens: one GEMM launch for many block_q8 rows,
// else GEMV launches of up to tmax tokens.  With fp32 input (a.x) each GEMV
// launch quantizes its rows in LDS.
int run_gemv(GemvArgs a, int n_tok, hipStream_t s) {
    const bool xf = a.x != nullptr;
    const int plan = gemm_plan(a, n_tok);
    if (plan > 0) {
        if ((size_t)n_tok * a.nb > (size_t)INT32_MAX / kBlockBytes) return TQ_HIP_EINVAL;
        a.n_tok = n_tok;
        return herr(launch_gemm(a, plan, s));
    }
    if (a.xs) return TQ_HIP_EINVAL;   // the split layout is for the GEMM only
    const int tmax = pick_tokens(a.nb, xf);
    if (tmax == 0) return TQ_HIP_EINVAL;
    const int rw = pick_rw(a.rows_total, a.ng, a.q4);
    const int gc = pick_gc(a.ng, rw, a.q4);
    const unsigned char *xq0 = a.xq;
    const float *x0 = a.x;
    unsigned char *out0 = a.xq_out;
    GemvSeg seg0[kMaxSegs];
    for (int i = 0; i < kMaxSegs; i++) seg0[i] = a.seg[i];
    for (int t0 = 0; t0 < n_tok; t0 += tmax) {
        const int nt = n_tok - t0 < tmax ? n_tok - t0 : tmax;
        int tcap = 1;
        while (tcap < nt) tcap *= 2;
        a.n_tok = nt;
        const size_t blk_off = (size_t)t0 * a.nb * kBlockBytes;
        a.xq = xq0 ? xq0 + blk_off : nullptr;
        a.x = x0 ? x0 + (size_t)t0 * a.cols : nullptr;
        a.xq_out = out0 ? out0 + blk_off : nullptr;
        for (int i = 0; i < kMaxSegs; i++)
            a.seg[i].y = seg0[i].y ? seg0[i].y + (size_t)t0 * seg0[i].rows : nullptr;
        const hipError_t e = launch_gemv(a, tcap, xf, rw, gc, s);
        if (e != hipSuccess) return herr(e);
    }
    return TQ_HIP_OK;
}

// fp32 input is quantized inside the matmul launch for one or two rows (one
// launch instead of two); more rows go through quantize_row_q8 into the
// workspace first, so that a launch still covers up to 8 of them.
bool fuse_quantize(const float *x, int n_tok, int nb) {
    return n_tok <= 2 && ((uintptr_t)x & 15) == 0 && lds_bytes(n_tok, nb, true) <= kMaxStageBytes;
}

bool aligned(const void *p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

bool shape_ok(int rows, int cols) { return rows > 0 && cols > 0 && cols % kQK == 0; }

void init_args(GemvArgs &a, int cols) {
    a = GemvArgs{};
    a.cols = cols;
    a.nb = cols / kQK;
    a.ng = (a.nb + kGroupBlocks - 1) / kGroupBlocks;
}

int matmul_fmt(bool q4, const void *W, const block_q8 *xq, float *y, int rows, int cols, int n_tok,
               void *stream) {
    if (!shape_ok(rows, cols) || n_tok <= 0 || !W || !xq || !y || !aligned(W, 16) || !aligned(xq, 4) ||
        !aligned(y, 4))
        return TQ_HIP_EINVAL;
    GemvArgs a;
    init_args(a, cols);
    a.q4 = q4;
    a.seg[0] = GemvSeg{(const unsigned char *)W, y, rows};
    a.seg_end[0] = a.seg_end[1] = a.seg_end[2] = rows;
    a.rows_total = rows;
    a.xq = (const unsigned char *)xq;
    return run_gemv(a, n_tok, (hipStream_t)stream);
}

}  // namespace

extern "C" {

size_t tq_hip_q8_matrix_bytes(int rows, int cols) {
    if (!shape_ok(rows, cols)) return 0;
    return (size_t)rows * (size_t)(cols / kQK) * kBlockBytes;
}

int tq_hip_q8_pack(void *dst, const block_q8 *src, int rows, int cols, void *stream) {
    if (!shape_ok(rows, cols) || !dst || !src || !aligned(dst, 16) || !aligned(src, 4))
        return TQ_HIP_EINVAL;
    const long long n = (long long)rows * (cols / kQK);
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (unsigned char *)dst, (const unsigned char *)src, rows, cols / kQK);
    return herr(hipGetLastError());
}

int tq_hip_q8_unpack(block_q8 *dst, const void *src, int rows, int cols, void *stream) {
    if (!shape_ok(rows, cols) || !dst || !src || !aligned(src, 16) || !aligned(dst, 4))
        return TQ_HIP_EINVAL;
    const long long n = (long long)rows * (cols / kQK);
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (unsigned char *)dst, (const unsigned char *)src, rows, cols / kQK);
    return herr(hipGetLastError());
}

int tq_hip_matmul_q8_batch(const void *W, const block_q8 *xq, float *y, int rows, int cols, int n_tok,
                           void *stream) {
    return matmul_fmt(false, W, xq, y, rows, cols, n_tok, stream);
}

int tq_hip_matmul_q8(const void *W, const block_q8 *xq, float *y, int rows, int cols, void *stream) {
    return matmul_fmt(false, W, xq, y, rows, cols, 1, stream);
}

size_t tq_hip_q4_matrix_bytes(int rows, int cols) {
    if (!shape_ok(rows, cols)) return 0;
    return (size_t)rows * (size_t)(cols / kQK) * kBlockBytes4;
}

int tq_hip_q4_pack(void *dst, const block_q4 *src, int rows, int cols, void *stream) {
    if (!shape_ok(rows, cols) || !dst || !src || !aligned(dst, 16) || !aligned(src, 4)) return TQ_HIP_EINVAL;
    const long long n = (long long)rows * (cols / kQK);
    hipLaunchKernelGGL(pack4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (unsigned char *)dst, (const unsigned char *)src, n);
    return herr(hipGetLastError());
}

int tq_hip_q4_unpack(block_q4 *dst, const void *src, int rows, int cols, void *stream) {
    if (!shape_ok(rows, cols) || !dst || !src || !aligned(src, 16) || !aligned(dst, 4)) return TQ_HIP_EINVAL;
    const long long n = (long long)rows * (cols / kQK);
    hipLaunchKernelGGL(unpack4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (unsigned char *)dst, (const unsigned char *)src, n);
    return herr(hipGetLastError());
}

int tq_hip_matmul_q4_batch(const void *W, const block_q8 *xq, float *y, int rows, int cols, int n_tok,
                           void *stream) {
    return matmul_fmt(true, W, xq, y, rows, cols, n_tok, stream);
}

int tq_hip_matmul_q4(const void *W, const block_q8 *xq, float *y, int rows, int cols, void *stream) {
    return matmul_fmt(true, W, xq, y, rows, cols, 1, stream);
}

int tq_hip_project_qkv(const void *wq, const void *wk, const void *wv, int q_rows, int kv_rows,
                       int hidden, const float *xn, int n_tok, block_q8 *xq_ws, float *q, float *k,
                       float *v, void *stream) {
    return tq_project_qkv_fmt(false, wq, wk, wv, q_rows, kv_rows, hidden, xn, n_tok, xq_ws, q, k, v, stream);
}

int tq_hip_project_qkv_q4(const void *wq, const void *wk, const void *wv, int q_rows, int kv_rows,
                          int hidden, const float *xn, int n_tok, block_q8 *xq_ws, float *q, float *k,
                          float *v, void *stream) {
    return tq_project_qkv_fmt(true, wq, wk, wv, q_rows, kv_rows, hidden, xn, n_tok, xq_ws, q, k, v, stream);
}

int tq_hip_project_output(const void *wo, int rows, int cols, const float *attn, int n_tok,
                          block_q8 *xq_ws, float *out, void *stream) {
    return tq_project_output_fmt(false, wo, rows, cols, attn, n_tok, xq_ws, out, stream);
}

int tq_hip_project_output_q4(const void *wo, int rows, int cols, const float *attn, int n_tok,
                             block_q8 *xq_ws, float *out, void *stream) {
    return tq_project_output_fmt(true, wo, rows, cols, attn, n_tok, xq_ws, out, stream);
}

}  // extern "C"

// The matmul input of a (segments, workspace set): one or two rows quantized
// inside the GEMV launch; else quantize_row_q8 of every row into the
// workspace first, as block_q8 rows or, for a GEMM that reads it, in the
// split layout.
int quantize_input(GemvArgs &a, const float *x, int n_tok, int cols, void *xq_ws, hipStream_t s) {
    if (fuse_quantize(x, n_tok, a.nb)) {
        a.x = x;
        a.xq_out = (unsigned char *)xq_ws;
        return TQ_HIP_OK;
    }
    a.xs = xs_layout(a, n_tok, xq_ws);
    const hipError_t e = a.xs ? tq_launch_quantize_split(x, (unsigned char *)xq_ws, n_tok, cols, s)
                              : tq_launch_quantize(x, (block_q8 *)xq_ws, n_tok * cols, s);
    if (e != hipSuccess) return herr(e);
    a.xq = (const unsigned char *)xq_ws;
    return TQ_HIP_OK;
}

int tq_project_qkv_fmt(bool q4, const void *wq, const void *wk, const void *wv, int q_rows, int kv_rows, int hidden,
                    const float *xn, int n_tok, block_q8 *xq_ws, float *q, float *k, float *v, void *stream,
                    float *part, size_t part_floats) {
    if (!shape_ok(q_rows, hidden) || kv_rows <= 0 || n_tok <= 0 || !wq || !wk || !wv || !xn ||
        !xq_ws || !q || !k || !v || !aligned(wq, 16) || !aligned(wk, 16) || !aligned(wv, 16) ||
        !aligned(xn, 4) || !aligned(xq_ws, 4) || !aligned(q, 4) || !aligned(k, 4) || !aligned(v, 4))
        return TQ_HIP_EINVAL;
    const hipStream_t s = (hipStream_t)stream;
    GemvArgs a;
    init_args(a, hidden);
    a.q4 = q4;
    a.seg[0] = GemvSeg{(const unsigned char *)wq, q, q_rows};
    a.seg[1] = GemvSeg{(const unsigned char *)wk, k, kv_rows};
    a.seg[2] = GemvSeg{(const unsigned char *)wv, v, kv_rows};
    a.seg_end[0] = q_rows;
    a.seg_end[1] = q_rows + kv_rows;
    a.seg_end[2] = q_rows + 2 * kv_rows;
    a.rows_total = a.seg_end[2];
    a.part = part;
    a.part_floats = part_floats;
    const int rc = quantize_input(a, xn, n_tok, hidden, xq_ws, s);
    return rc != TQ_HIP_OK ? rc : run_gemv(a, n_tok, s);
}

int tq_project_output_fmt(bool q4, const void *wo, int rows, int cols, const float *attn, int n_tok,
                       block_q8 *xq_ws, float *out, void *stream, float *part, size_t part_floats) {
    if (!shape_ok(rows, cols) || n_tok <= 0 || !wo || !attn || !xq_ws || !out || !aligned(wo, 16) ||
        !aligned(attn, 4) || !aligned(xq_ws, 4) || !aligned(out, 4))
        return TQ_HIP_EINVAL;
    const hipStream_t s = (hipStream_t)stream;
    GemvArgs a;
    init_args(a, cols);
    a.q4 = q4;
    a.seg[0] = GemvSeg{(const unsigned char *)wo, out, rows};
    a.seg_end[0] = a.seg_end[1] = a.seg_end[2] = rows;
    a.rows_total = rows;
    a.part = part;
    a.part_floats = part_floats;
    const int rc = quantize_input(a, attn, n_tok, cols, xq_ws, s);
    return rc != TQ_HIP_OK ? rc : run_gemv(a, n_tok, s);
}

static void output_args(GemvArgs &a, bool q4, const void *wo, int rows, int cols, float *out, float *part,
                        size_t part_floats) {
    init_args(a, cols);
    a.q4 = q4;
    a.seg[0] = GemvSeg{(const unsigned char *)wo, out, rows};
    a.seg_end[0] = a.seg_end[1] = a.seg_end[2] = rows;
    a.rows_total = rows;
    a.part = part;
    a.part_floats = part_floats;
}

bool tq_project_output_takes_xs(bool q4, const void *wo, int rows, int cols, int n_tok, const void *xq_ws,
                                float *part, size_t part_floats) {
    if (!shape_ok(rows, cols) || n_tok <= 2 || !wo || !xq_ws || !aligned(wo, 16)) return false;
    GemvArgs a;
    output_args(a, q4, wo, rows, cols, nullptr, part, part_floats);
    return xs_layout(a, n_tok, xq_ws);
}

int tq_project_output_xs(bool q4, const void *wo, int rows, int cols, const void *xq_ws, int n_tok, float *out,
                         void *stream, float *part, size_t part_floats) {
    if (!out || !aligned(out, 4) || !tq_project_output_takes_xs(q4, wo, rows, cols, n_tok, xq_ws, part, part_floats))
        return TQ_HIP_EINVAL;
    GemvArgs a;
    output_args(a, q4, wo, rows, cols, out, part, part_floats);
    a.xs = true;
    a.xq = (const unsigned char *)xq_ws;
    return run_gemv(a, n_tok, (hipStream_t)stream);
}

// Partial floats a split-K GEMM of rows x cols needs for any token count up
// to n_cap: the largest S * n over the token-tile counts that still split.
size_t tq_gemm_partial_floats(int rows, int cols, int n_cap) {
    if (rows <= 0 || cols <= 0 || n_cap < 16) return 0;
    size_t most = 0;
    for (int tiles = 1; (long)(tiles - 1) * kGemmToks < n_cap; tiles++) {
        const int n = n_cap < tiles * kGemmToks ? n_cap : tiles * kGemmToks;
        const int sp = gemm_ksplit(rows, cols, n);
        if (sp < 2) break;
        const size_t need = (size_t)sp * n * rows;
        if (need > most) most = need;
    }
    return most;
}

extern "C" {

static size_t mlp_ws(int hidden, int inter, int n, size_t *off_gate, size_t *off_up, size_t *off_xq,
                     size_t *off_part, size_t *part_floats) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    size_t o = 0;
    *off_gate = o;
    o += al((size_t)n * inter * 4);
    *off_up = o;
    o += al((size_t)n * inter * 4);
    *off_xq = o;
    o += al((size_t)n * (size_t)(hidden > inter ? hidden : inter) / kQK * kBlockBytes);
    // split-K partials of the gate/up and the down matmuls (one at a time)
    const size_t pg = tq_gemm_partial_floats(2 * inter, hidden, n), pd = tq_gemm_partial_floats(hidden, inter, n);
    *part_floats = pg > pd ? pg : pd;
    *off_part = o;
    o += al(*part_floats * 4);
    return o;
}

static bool mlp_ok(const tq_hip_mlp_weights *w, int n) {
    return w && n > 0 && w->wgate && w->wup && w->wdown && shape_ok(w->inter, w->hidden) &&
           shape_ok(w->hidden, w->inter) && aligned(w->wgate, 16) && aligned(w->wup, 16) &&
           aligned(w->wdown, 16) && (w->format == TQ_HIP_FORMAT_Q8 || w->format == TQ_HIP_FORMAT_Q4);
}

size_t tq_hip_mlp_ws_bytes(const tq_hip_mlp_weights *w, int n) {
    if (!mlp_ok(w, n)) return 0;
    size_t a, b, c, d, e;
    return mlp_ws(w->hidden, w->inter, n, &a, &b, &c, &d, &e);
}

int tq_hip_mlp_layer_async(const tq_hip_mlp_weights *w, int n, const float *d_xn, float *d_out, void *d_ws,
                           size_t ws_bytes, void *stream) {
    if (!mlp_ok(w, n) || !d_xn || !d_out || !d_ws || !aligned(d_ws, 16) || !aligned(d_xn, 4) ||
        !aligned(d_out, 4))
        return TQ_HIP_EINVAL;
    size_t og, ou, ox, op, pf;
    if (ws_bytes < mlp_ws(w->hidden, w->inter, n, &og, &ou, &ox, &op, &pf)) return TQ_HIP_EINVAL;
    unsigned char *ws = (unsigned char *)d_ws;
    float *gate = (float *)(ws + og), *up = (float *)(ws + ou);
    float *part = (float *)(ws + op);
    block_q8 *xq = (block_q8 *)(ws + ox);
    const hipStream_t s = (hipStream_t)stream;
    // model/mlp.c:9-11: quantize xn, then the gate and up matmuls in one launch
    const bool q4 = w->format == TQ_HIP_FORMAT_Q4;
    GemvArgs a;
    init_args(a, w->hidden);
    a.q4 = q4;
    a.seg[0] = GemvSeg{(const unsigned char *)w->wgate, gate, w->inter};
    a.seg[1] = GemvSeg{(const unsigned char *)w->wup, up, w->inter};
    a.seg_end[0] = w->inter;
    a.seg_end[1] = a.seg_end[2] = 2 * w->inter;
    a.rows_total = 2 * w->inter;
    a.part = part;
    a.part_floats = pf;
    int rc = quantize_input(a, d_xn, n, w->hidden, xq, s);
    if (rc != TQ_HIP_OK) return rc;
    // :14 the down matmul, over :12-13 silu_mul with the hidden rows quantized
    GemvArgs d;
    init_args(d, w->inter);
    d.q4 = q4;
    d.seg[0] = GemvSeg{(const unsigned char *)w->wdown, d_out, w->hidden};
    d.seg_end[0] = d.seg_end[1] = d.seg_end[2] = w->hidden;
    d.rows_total = w->hidden;
    d.part = part;
    d.part_floats = pf;
    // When the gate/up matmul is one unsplit GEMM over the split layout and
    // the down matmul reads the split layout too, the gate/up tiles pair 64
    // rows of both matrices and their epilogue writes the quantized hidden
    // rows (into the gate rows' space, which they then no longer need);
    // otherwise gate and up rows go to the workspace and one more launch
    // forms them (block_q8 rows, or the split layout).  TQ_HIP_MLP_FUSED=0
    // keeps the separate launch.
    const bool fused = a.xs && gemm_plan(a, n) == 1 && xs_layout(d, n, gate) &&
                       env_int("TQ_HIP_MLP_FUSED", 1) != 0;
    if (fused) a.hq = (unsigned char *)gate;
    rc = run_gemv(a, n, s);
    if (rc != TQ_HIP_OK) return rc;
    if (fused) {
        d.xs = true;
        d.xq = (const unsigned char *)gate;
        return run_gemv(d, n, s);
    }
    d.xs = xs_layout(d, n, xq);
    const hipError_t e = d.xs ? tq_launch_silu_quant_split(gate, up, (unsigned char *)xq, n, w->inter, s)
                              : tq_launch_silu_quant(gate, up, xq, (long)n * w->inter, s);
    if (e != hipSuccess) return herr(e);
    d.xq = (const unsigned char *)xq;
    return run_gemv(d, n, s);
}

}  // extern "C"
