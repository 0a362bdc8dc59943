"""Q8 GQA decode benchmark on one MI355X.

Workload (default, --config c2): Llama-3-8B-shaped attention, 32 q heads / 8 kv
heads / head_dim 128, batch 1, context 4096.  One step = the attention core of
one layer for one new token: RoPE (theta 5e5) on q and k, quantize and append
the token's K/V into that layer's paged HBM cache, and attend over all 4096
tokens — one call of tq_hip_decode_step_async.  Steps rotate over 32 layer
caches (32 x 9.44 MB = 302 MB > the 256 MB MALL) so every step streams its KV
from HBM.  The timed steps are replayed from a HIP graph of 32 steps; inputs
are resident in HBM before the timed region.

value = tokens/s of one layer step (batch / step time).  KV bytes per step =
n_tokens * n_kv_heads * 2 * (head_dim/32) * 36 = 9,437,184 (the reference's KV
accounting, tools/bench_forward.c:153-159).

Other workloads: --config c3 (64 sequences, ragged 512..8192, paged),
c5 (64q/8kv, batch 16, context 32768, 1 % outliers), c4 (causal prefill of
2048 tokens).  They print the same JSON fields for their own shape.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q8 GQA decode tokens/sec + achieved HBM GB/s (KV bytes) at 8B shape, 1 GPU"
HBM_PEAK_GBS = 8000.0
QK, BLOCK_BYTES, PAGE = 32, 36, 16


# ---------------------------------------------------------------------------
# HIP runtime pieces used for timing and graphs (events on the launch stream)

class Hip:
    def __init__(self):
        path = None
        for cand in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                self.lib = C.CDLL(cand)
                path = cand
                break
            except OSError:
                continue
        if path is None:
            raise RuntimeError("libamdhip64.so not found")
        L = self.lib
        vp = C.c_void_p
        L.hipEventCreate.argtypes = [C.POINTER(vp)]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        L.hipEventDestroy.argtypes = [vp]
        L.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        L.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        L.hipDeviceSynchronize.argtypes = []

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def event(self):
        e = C.c_void_p()
        self.ok(self.lib.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e.value

    def record(self, e, stream):
        self.ok(self.lib.hipEventRecord(e, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self.ok(self.lib.hipEventSynchronize(b), "hipEventSynchronize")
        ms = C.c_float()
        self.ok(self.lib.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return float(ms.value)

    def sync(self):
        self.ok(self.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def capture(self, stream, fn):
        """Capture fn()'s launches on `stream` into an instantiated graph."""
        self.ok(self.lib.hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = self.lib.hipStreamEndCapture(stream, C.byref(g))
        self.ok(rc, "hipStreamEndCapture")
        ex = C.c_void_p()
        self.ok(self.lib.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return ex.value, g.value

    def launch_graph(self, ex, stream):
        self.ok(self.lib.hipGraphLaunch(ex, stream), "hipGraphLaunch")


# ---------------------------------------------------------------------------
# cache content

def paged_pool_bytes(kflat: np.ndarray, vflat: np.ndarray, nkv: int, T: int, nb: int,
                     page_ids: np.ndarray, n_pages_pool: int) -> np.ndarray:
    """Flat block_q8 caches [nkv][T][nb] -> pool bytes [page][kvh][K|V][16][nb]."""
    row = nb * BLOCK_BYTES
    npg = T // PAGE
    k = kflat.view(np.uint8).reshape(nkv, npg, PAGE * row)
    v = vflat.view(np.uint8).reshape(nkv, npg, PAGE * row)
    runs = np.stack([k, v], axis=2).transpose(1, 0, 2, 3)  # [page][kvh][2][16*row]
    pool = np.zeros((n_pages_pool, nkv, 2, PAGE * row), np.uint8)
    pool[page_ids] = runs
    return pool.reshape(-1)


def quantized_normal(oracle, n_values: int, seed: int, outliers: float = 0.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n_values, dtype=np.float32)
    if outliers > 0:
        idx = rng.choice(n_values, int(n_values * outliers), replace=False)
        x[idx] = np.where(rng.random(idx.size) < 0.5, -8.0, 8.0).astype(np.float32)
    return oracle.quantize_row_q8(x)


# ---------------------------------------------------------------------------
# CPU baseline: the reference's kernels (oracle/_ref), AVX2 dispatch, OpenMP
# over kv heads from 256 tokens on, as the reference runs them.

def cpu_baseline_c2(nq, nkv, hd, T, theta, budget_s: float = 10.0):
    from oracle.binding import Oracle, Ref, ptr
    oracle = Oracle()
    nb = hd // QK
    layers = 8  # 8 x 9.44 MB = 75 MB of host cache rotated, beyond the L3
    kind = "reference" if Ref.available() else "port"
    caches = [(quantized_normal(oracle, nkv * T * hd, 10 + l), quantized_normal(oracle, nkv * T * hd, 50 + l))
              for l in range(layers)]
    rng = np.random.default_rng(1)
    q0 = rng.standard_normal(nq * hd, dtype=np.float32)
    k0 = rng.standard_normal(nkv * hd, dtype=np.float32)
    v0 = rng.standard_normal(nkv * hd, dtype=np.float32)
    scores = np.zeros(nq * T, np.float32)
    out = np.zeros(nq * hd, np.float32)
    pos = T - 1
    if kind == "reference":
        ref = Ref()
        fn = lambda kc, vc, q, k: ref.lib.tqref_attention_qkv(nq, nkv, hd, T, theta, ptr(kc), ptr(vc), pos,
                                                              ptr(q), ptr(k), ptr(v0), ptr(scores), ptr(out))
        isa = ref.isa()
    else:
        fn = lambda kc, vc, q, k: oracle.lib.oracle_attention_qkv(ptr(kc), ptr(vc), nq, nkv, hd, T, theta, pos,
                                                                  ptr(q), ptr(k), ptr(v0), ptr(scores), ptr(out))
        isa = "scalar"
    for l in range(2):  # warm up
        fn(caches[l][0], caches[l][1], q0.copy(), k0.copy())
    times = []
    t_start = time.perf_counter()
    i = 0
    while (time.perf_counter() - t_start < budget_s and i < 100000) or i < 5:
        kc, vc = caches[i % layers]
        q, k = q0.copy(), k0.copy()
        t0 = time.perf_counter()
        rc = fn(kc, vc, q, k)
        times.append(time.perf_counter() - t0)
        assert rc == 0
        i += 1
    med = float(np.median(times))
    omp = int(os.environ.get("OMP_NUM_THREADS", str(os.cpu_count() or 1)))
    cores = min(nkv, omp, os.cpu_count() or 1) if kind == "reference" else 1
    try:
        cpu_model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:
        cpu_model = "unknown"
    return {"value": 1.0 / med, "unit": "tokens/s", "cores": cores, "kind": kind,
            "sample": (f"{len(times)} single-token layer steps (RoPE+store_kv+attend_q8, ctx {T}, "
                       f"{nq}q/{nkv}kv/hd{hd}) rotating {layers} host caches, median; {isa} kernels, "
                       f"OMP over kv heads (OMP_NUM_THREADS={omp}, nproc={os.cpu_count()}, {cpu_model})"),
            "ms_per_step": med * 1e3}


# ---------------------------------------------------------------------------

def bench_c2(args, nat, hip):
    from oracle.binding import Oracle
    oracle = Oracle()
    nq, nkv, hd, T, theta = 32, 8, 128, 4096, 500000.0
    nb = hd // QK
    layers = args.layers
    npg = T // PAGE
    kv_bytes = T * nkv * 2 * nb * BLOCK_BYTES
    lib = nat.load()

    # one layer's cache content, quantized N(0,1), written to every layer pool
    kflat = quantized_normal(oracle, nkv * T * hd, 1)
    vflat = quantized_normal(oracle, nkv * T * hd, 2)
    pool_bytes = paged_pool_bytes(kflat, vflat, nkv, T, nb, np.arange(npg), npg)
    kvs = []
    for l in range(layers):
        kv = nat.PagedKV.single(nq, nkv, hd, T)
        base, nbytes, _ = kv.pool()
        assert nbytes == pool_bytes.nbytes
        nat.check(lib.tq_hip_memcpy_h2d(base, pool_bytes.ctypes.data, nbytes, None), "pool upload")
        kvs.append(kv)
    stream = kvs[0].stream

    rng = np.random.default_rng(3)
    pos = T - 1
    q = rng.standard_normal(nq * hd, dtype=np.float32)
    k = rng.standard_normal(nkv * hd, dtype=np.float32)
    v = rng.standard_normal(nkv * hd, dtype=np.float32)
    c, s = oracle.rope_table(hd, pos, theta)
    D = nat.DeviceBuffer.from_numpy
    dq, dk, dv, dc, ds = D(q), D(k), D(v), D(c), D(s)
    dseq, dpos = D(np.zeros(1, np.int32)), D(np.array([pos], np.int32))
    outs = [nat.DeviceBuffer(nq * hd * 4) for _ in range(layers)]

    def step(l):
        nat.check(lib.tq_hip_decode_step_async(kvs[l].h, 1, None, dpos.ptr, pos, dq.ptr, dk.ptr, dv.ptr,
                                               dc.ptr, ds.ptr, outs[l].ptr, stream), "decode_step")

    # eager warm-up (allocates split-K scratch before capture)
    for i in range(max(args.warmup, layers)):
        step(i % layers)
    hip.sync()

    # parity of the measured path against the oracle on this layer shape
    rc, ref = oracle.attention_qkv(kflat.copy(), vflat.copy(), nq, nkv, hd, T, theta, pos, q, k, v)
    got = outs[0].download((nq * hd,), np.float32)
    err = np.abs(got.astype(np.float64) - ref)
    parity_ok = bool(rc == 0 and (err <= 1e-4 + 1e-3 * np.abs(ref)).all())

    graph, g = hip.capture(stream, lambda: [step(l) for l in range(layers)])
    for _ in range(2):
        hip.launch_graph(graph, stream)
    hip.sync()
    got_graph = outs[0].download((nq * hd,), np.float32)
    parity_ok = parity_ok and got_graph.tobytes() == got.tobytes()

    reps = max(1, args.steps // layers)
    steps = reps * layers
    e0, e1 = hip.event(), hip.event()
    hip.sync()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for _ in range(reps):
        hip.launch_graph(graph, stream)
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1)
    hip.sync()
    wall = time.perf_counter() - t0
    ms_per_step = ms / steps

    # per-launch duration of the step (events around each launch, eager)
    n_k = min(256, 8 * layers)
    ev = [(hip.event(), hip.event()) for _ in range(n_k)]
    for i in range(n_k):
        hip.record(ev[i][0], stream)
        step(i % layers)
        hip.record(ev[i][1], stream)
    hip.sync()
    per = np.array([hip.elapsed_ms(a, b) for a, b in ev])
    kern_ms = float(per.mean())
    achieved = kv_bytes / (kern_ms * 1e-3) / 1e9

    line = {
        "metric": METRIC,
        "value": 1e3 / ms_per_step,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": ("Q8 GQA decode, 32q/8kv/hd128, batch 1, context 4096, fused RoPE(theta 5e5)"
                                f" + KV append + attend per layer step, {layers} layer caches rotated "
                                f"({layers * kv_bytes / 1e6:.0f} MB), HIP graph of {layers} steps"),
                   "batch": 1, "context": T, "n_q_heads": nq, "n_kv_heads": nkv, "head_dim": hd,
                   "kv_bytes_per_step": kv_bytes, "layers_rotated": layers},
        "kv_gbps": kv_bytes / (ms_per_step * 1e-3) / 1e9,
        "tokens_per_s_32_layers": 1e3 / ms_per_step / 32,
        "wall_s": wall,
        "parity": {"ok": parity_ok, "max_abs_err": float(err.max()), "bar": "1e-4 + 1e-3*|ref|"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "decode_step (decode_kernel<128,4> + combine)",
                     "kernel_ms": kern_ms, "algorithmic_bytes": kv_bytes},
    }
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3200)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--config", default="c2", choices=["c2"])
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline sampling")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): this path has no multi-GPU "
              "collective; see the sharding note in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    from tailorquantkernel_amd import native as nat
    nat.init(0)
    hip = Hip()
    line = bench_c2(args, nat, hip)
    if not args.no_cpu:
        cb = cpu_baseline_c2(32, 8, 128, 4096, 500000.0, args.cpu_budget)
        line["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
