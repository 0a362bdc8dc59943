/* tq_bench.h — bench-only measurement entry points (libtqbench.so), used by
 * bench.py beside the attention library; no counterpart in the reference and
 * not part of the drop-in boundary.
 *
 * The floor of one split-K decode step on this GPU.  n_heads * n_splits
 * work-groups of 256 threads; work-group w reads its 1/(n_heads*n_splits)
 * chunk of buf (bytes, a multiple of 16) with every 16-byte load in flight.
 * mode 0: the launch alone; 1: the read; 2: the read, then the decode's
 * combine chain with no math — a 520-float partial row stored agent-coherent,
 * an arrival counter per head, and the head's last work-group pulling its
 * n_splits rows and writing their sum to out[head][520].  scratch:
 * tq_hip_floor_scratch_bytes bytes, 256-byte aligned, its first n_heads*256
 * bytes (the counters) zeroed once; out: tq_hip_floor_out_bytes bytes,
 * 16-byte aligned.  Asynchronous on stream; TQ_HIP_* return codes. */
#ifndef TQ_BENCH_H
#define TQ_BENCH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

size_t tq_hip_floor_scratch_bytes(int n_heads, int n_splits);
size_t tq_hip_floor_out_bytes(int n_heads, int n_splits);
int tq_hip_floor_step(const void *buf, size_t bytes, int n_heads, int n_splits, int mode, void *scratch,
                      void *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TQ_BENCH_H */
