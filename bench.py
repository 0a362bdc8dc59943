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


# ---------------------------------------------------------------------------
# batched / long-context decode (C3, C5) and prefill (C4)

def fill_pool_tiled(nat, kv, pattern: np.ndarray, n_pages: int, page_bytes: int):
    """Write valid quantized pages into the whole pool by tiling a pattern of
    whole pages (the content only has to be valid block_q8 data)."""
    lib = nat.load()
    base, nbytes, _ = kv.pool()
    assert nbytes == n_pages * page_bytes and pattern.nbytes % page_bytes == 0
    pat_pages = pattern.nbytes // page_bytes
    for p0 in range(0, n_pages, pat_pages):
        n = min(pat_pages, n_pages - p0)
        nat.check(lib.tq_hip_memcpy_h2d(base + p0 * page_bytes, pattern.ctypes.data, n * page_bytes, None), "fill")


def bench_batched(args, nat, hip, *, nq, nkv, hd, lens, theta, outliers, workload, metric):
    from oracle.binding import Oracle, dequant
    oracle = Oracle()
    lib = nat.load()
    nb = hd // QK
    nseq = len(lens)
    pages_per = (lens + PAGE - 1) // PAGE
    total = int(pages_per.sum())
    maxp = int(pages_per.max())
    page_bytes = nkv * 2 * PAGE * nb * BLOCK_BYTES
    kv = nat.PagedKV(nq, nkv, hd, n_pages=total, max_seqs=nseq, max_pages_per_seq=maxp)
    rng = np.random.default_rng(7)
    perm = rng.permutation(total).astype(np.int32)    # physical pages scattered over the pool
    at = 0
    for i in range(nseq):
        kv.set_pages(i, perm[at:at + pages_per[i]])
        at += pages_per[i]
    pat_pages = min(total, 512)
    pk = quantized_normal(oracle, pat_pages * PAGE * nkv * hd, 11, outliers)
    pv = quantized_normal(oracle, pat_pages * PAGE * nkv * hd, 12, outliers)
    pattern = paged_pool_bytes(pk, pv, nkv, pat_pages * PAGE, nb, np.arange(pat_pages), pat_pages)
    fill_pool_tiled(nat, kv, pattern, total, page_bytes)
    stream = kv.stream
    kv_bytes = int(lens.sum()) * nkv * 2 * nb * BLOCK_BYTES

    pos = (lens - 1).astype(np.int32)
    q = rng.standard_normal(nseq * nq * hd, dtype=np.float32)
    k = rng.standard_normal(nseq * nkv * hd, dtype=np.float32)
    v = rng.standard_normal(nseq * nkv * hd, dtype=np.float32)
    tabs = [oracle.rope_table(hd, int(p), theta) for p in pos]
    cos = np.concatenate([c for c, _ in tabs]); sin = np.concatenate([s_ for _, s_ in tabs])
    D = nat.DeviceBuffer.from_numpy
    dq, dk, dv, dc, ds, dpos = D(q), D(k), D(v), D(cos), D(sin), D(pos)
    dseq = D(np.arange(nseq, dtype=np.int32))
    out = nat.DeviceBuffer(nseq * nq * hd * 4)
    max_pos = int(pos.max())

    def step():
        nat.check(lib.tq_hip_decode_step_async(kv.h, nseq, dseq.ptr, dpos.ptr, max_pos, dq.ptr, dk.ptr, dv.ptr,
                                               dc.ptr, ds.ptr, out.ptr, stream), "decode_step")

    for _ in range(max(args.warmup // 8, 2)):
        step()
    hip.sync()
    # parity on two sequences: the cache after the step (with the appended row)
    got = out.download((nseq, nq * hd), np.float32)
    errs, ok = [], True
    for i in (0, nseq - 1):
        L = int(lens[i])
        kb, vb = kv.read(i, 0, L)
        c, s_ = tabs[i]
        qr = np.concatenate([oracle.rope_apply(q[(i * nq + h) * hd:(i * nq + h + 1) * hd], c, s_) for h in range(nq)])
        rc, ref = oracle.attend_q8(kb.reshape(-1), vb.reshape(-1), nq, nkv, hd, L, qr, L - 1)
        e = np.abs(got[i].astype(np.float64) - ref)
        errs.append(float(e.max()))
        ok = ok and rc == 0 and bool((e <= 1e-4 + 1e-3 * np.abs(ref)).all())

    steps = max(4, args.steps // 64)
    e0, e1 = hip.event(), hip.event()
    hip.sync()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for _ in range(steps):
        step()
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1) / steps
    hip.sync()
    wall = time.perf_counter() - t0
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    return {
        "metric": metric, "value": nseq * 1e3 / ms, "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": max(args.warmup // 8, 2), "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": workload, "batch": nseq, "n_q_heads": nq, "n_kv_heads": nkv, "head_dim": hd,
                   "context_sum": int(lens.sum()), "context_max": int(lens.max()), "kv_bytes_per_step": kv_bytes,
                   "pool_mb": total * page_bytes / 1e6},
        "kv_gbps": gbs, "wall_s": wall,
        "parity": {"ok": ok, "max_abs_err": max(errs), "bar": "1e-4 + 1e-3*|ref|", "checked_seqs": 2},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None, "kernel": f"decode_kernel<{hd},{nq // nkv}>",
                     "kernel_ms": ms, "algorithmic_bytes": kv_bytes},
    }


def bench_c3(args, nat, hip):
    lens = np.random.default_rng(2024).integers(512, 8193, size=64).astype(np.int32)
    return bench_batched(args, nat, hip, nq=32, nkv=8, hd=128, lens=lens, theta=500000.0, outliers=0.0,
                         workload="Q8 GQA batched decode, 64 sequences, context U[512,8192] (seeded), 16-token "
                                  "pages scattered over the pool, 32q/8kv/hd128, fused RoPE + append + attend",
                         metric="Q8 GQA batched decode tokens/sec + achieved HBM GB/s (KV bytes), 1 GPU")


def bench_c5(args, nat, hip):
    lens = np.full(16, 32768, np.int32)
    return bench_batched(args, nat, hip, nq=64, nkv=8, hd=128, lens=lens, theta=500000.0, outliers=0.01,
                         workload="Q8 GQA long-context decode, 64q/8kv/hd128 (70B layer), batch 16, context 32768, "
                                  "1% K/V outliers at +-8 sigma, split-K, fused RoPE + append + attend",
                         metric="Q8 GQA long-context decode tokens/sec + achieved HBM GB/s (KV bytes), 1 GPU")


def bench_c4(args, nat, hip):
    from oracle.binding import Oracle
    oracle = Oracle()
    lib = nat.load()
    nq, nkv, hd, n, theta = 32, 8, 128, 2048, 500000.0
    kv = nat.PagedKV.single(nq, nkv, hd, n)
    rng = np.random.default_rng(5)
    q = rng.standard_normal(n * nq * hd, dtype=np.float32)
    k = rng.standard_normal(n * nkv * hd, dtype=np.float32)
    v = rng.standard_normal(n * nkv * hd, dtype=np.float32)
    tabs = [oracle.rope_table(hd, p, theta) for p in range(n)]
    cos = np.stack([c for c, _ in tabs]); sin = np.stack([s_ for _, s_ in tabs])
    D = nat.DeviceBuffer.from_numpy
    dq, dk, dv, dc, ds = D(q), D(k), D(v), D(cos), D(sin)
    out = nat.DeviceBuffer(n * nq * hd * 4)
    stream = kv.stream

    def step():
        nat.check(lib.tq_hip_prefill_async(kv.h, 0, 0, n, dq.ptr, dk.ptr, dv.ptr, dc.ptr, ds.ptr, out.ptr, stream),
                  "prefill")

    step()
    hip.sync()
    # parity: the oracle prefill on the first 256 tokens (a causal prefix is unchanged by later tokens)
    m = 256
    from oracle.binding import blocks
    kc, vc = blocks(nkv * n * (hd // QK)), blocks(nkv * n * (hd // QK))
    rc, ref = oracle.prefill_qkv(kc, vc, nq, nkv, hd, n, theta, 0, m, q[:m * nq * hd], k[:m * nkv * hd], v[:m * nkv * hd])
    got = out.download((n, nq * hd), np.float32)[:m]
    e = np.abs(got.astype(np.float64) - ref)
    ok = bool(rc == 0 and (e <= 1e-4 + 1e-3 * np.abs(ref)).all())
    steps = max(3, args.steps // 400)
    e0, e1 = hip.event(), hip.event()
    hip.sync()
    hip.record(e0, stream)
    for _ in range(steps):
        step()
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1) / steps
    useful_ops = 2.0 * nq * (n * (n + 1) / 2) * hd * 2      # Q.K^T and P.V over the causal triangle
    tflops = useful_ops / (ms * 1e-3) / 1e12
    return {
        "metric": "Q8 GQA causal prefill tokens/sec + MFMA utilisation, 2048 tokens at 8B shape, 1 GPU",
        "value": n * 1e3 / ms, "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": 1, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Q8 GQA causal prefill, 2048 tokens, 32q/8kv/hd128, RoPE theta 5e5, KV append + "
                               "causal attention", "tokens": n, "useful_ops": useful_ops},
        "parity": {"ok": ok, "max_abs_err": float(e.max()), "bar": "1e-4 + 1e-3*|ref|", "checked_tokens": m},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 5000.0, "unit": "TFLOP/s",
                     "frac": tflops / 5000.0, "traffic": None, "kernel": "prefill", "kernel_ms": ms},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3200)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--config", default="c2", choices=["c2", "c3", "c4", "c5"])
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
    line = {"c2": bench_c2, "c3": bench_c3, "c4": bench_c4, "c5": bench_c5}[args.config](args, nat, hip)
    if not args.no_cpu and args.config == "c2":
        cb = cpu_baseline_c2(32, 8, 128, 4096, 500000.0, args.cpu_budget)
        line["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
