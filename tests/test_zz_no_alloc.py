"""The allocation-free decode step, tq_hip_decode_step_noalloc, through the
C-ABI: the same launch as tq_hip_decode_step_async with its split-K scratch
in the library's fixed per-GPU array instead of buffers grown with hipMalloc.

Two calls in a row, the second smaller (fewer queries, shorter contexts, so
another split plan), each against tq_hip_decode_step_async on the same inputs
(bit for bit: same kernel, same plan) and sampled sequences against the
oracle (|gpu - oracle| <= 1e-4 + 1e-3|oracle|, K/V codes bit-exact); then a
call too large for the array is refused with TQ_HIP_ESCRATCH before any
launch, and a call after it still matches (the counters stay zero).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import QK
from tests.test_gpu_workloads import assert_close, fill_from_pattern, quantize_heads, rope_rows, rows_of

pytestmark = pytest.mark.gpu

PAGE = 16


@pytest.fixture(scope="module")
def nat():
    from tailorquantkernel_amd import native
    native.init(0)
    assert native.device_arch().startswith("gfx950")
    return native


def dev(nat, a):
    return nat.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def batch_case(nat, oracle, lens, seed, sample):
    lib = nat.load()
    nq, nkv, hd, theta = 32, 8, 128, 5e5
    nb = hd // QK
    nseq = lens.size
    pages_per = (lens + PAGE - 1) // PAGE
    total = int(pages_per.sum())
    kv = nat.PagedKV(nq, nkv, hd, n_pages=total, max_seqs=nseq, max_pages_per_seq=int(pages_per.max()))
    rng = np.random.default_rng(seed)
    perm = rng.permutation(total).astype(np.int32)
    page_lists, at = [], 0
    for i in range(nseq):
        page_lists.append(perm[at:at + pages_per[i]])
        kv.set_pages(i, page_lists[-1])
        at += pages_per[i]
    pat = int(lens.max())
    krows = rng.standard_normal((pat, nkv * hd), dtype=np.float32)
    vrows = rng.standard_normal((pat, nkv * hd), dtype=np.float32)
    dk_rows, dv_rows = dev(nat, krows), dev(nat, vrows)
    for i in range(nseq):
        fill_from_pattern(nat, kv, i, int(lens[i]), dk_rows, dv_rows, pat)
    pos = (lens - 1).astype(np.int32)
    q = rng.standard_normal(nseq * nq * hd, dtype=np.float32)
    k = rng.standard_normal(nseq * nkv * hd, dtype=np.float32)
    v = rng.standard_normal(nseq * nkv * hd, dtype=np.float32)
    cos, sin = rope_rows(oracle, hd, pos, theta)
    bufs = [dev(nat, a) for a in (q, k, v, cos, sin, pos, np.arange(nseq, dtype=np.int32))]
    dq, dk, dv, dc, ds, dpos, dseq = (b.ptr for b in bufs)
    outs = {}
    for name in ("tq_hip_decode_step_async", "tq_hip_decode_step_noalloc"):
        dout = nat.DeviceBuffer(nseq * nq * hd * 4)
        nat.check(getattr(lib, name)(kv.h, nseq, dseq, dpos, int(pos.max()), dq, dk, dv, dc, ds, dout.ptr,
                                     kv.stream), name)
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        outs[name] = dout.download((nseq, nq * hd), np.float32)
    assert outs["tq_hip_decode_step_noalloc"].tobytes() == outs["tq_hip_decode_step_async"].tobytes()
    base, nbytes, _ = kv.pool()
    raw = np.empty(nbytes, np.uint8)
    nat.check(lib.tq_hip_memcpy_d2h(raw.ctypes.data, base, nbytes, None), "pool download")
    kpat, vpat = quantize_heads(oracle, krows, nkv, hd), quantize_heads(oracle, vrows, nkv, hd)
    for i in sample:
        L = int(lens[i])
        kc, vc = np.ascontiguousarray(kpat[:, :L]), np.ascontiguousarray(vpat[:, :L])
        rc, ref = oracle.attention_qkv(kc.reshape(-1), vc.reshape(-1), nq, nkv, hd, L, theta, L - 1,
                                       q[i * nq * hd:(i + 1) * nq * hd], k[i * nkv * hd:(i + 1) * nkv * hd],
                                       v[i * nkv * hd:(i + 1) * nkv * hd])
        assert rc == 0
        gk, gv = rows_of(raw, nkv, nb, page_lists[i], L)
        assert gk.tobytes() == kc.tobytes() and gv.tobytes() == vc.tobytes(), f"cache of sequence {i}"
        assert_close(outs["tq_hip_decode_step_noalloc"][i], ref, f"no-alloc step, sequence {i} len {L}")
    kv.close()


def test_noalloc_matches_step(nat, oracle):
    lens = np.random.default_rng(5).integers(600, 5001, size=24).astype(np.int32)
    batch_case(nat, oracle, lens, 1, [int(np.argmax(lens)), int(np.argmin(lens)), 7])
    # the second call is smaller: 3 queries of at most 2000 keys (16 splits of 128)
    batch_case(nat, oracle, np.array([2000, 130, 1500], np.int32), 2, [0, 1, 2])


def test_noalloc_refuses_oversized_call(nat, oracle):
    """129 queries x 8 kv heads with split-K (16384 keys: two splits of 8192,
    the most one work-group stages) need more arrival counters than the array
    holds: TQ_HIP_ESCRATCH, nothing launched."""
    lib = nat.load()
    nq, nkv, hd, T, nseq = 32, 8, 128, 16384, 129
    kv = nat.PagedKV(nq, nkv, hd, n_pages=T // PAGE, max_seqs=1, max_pages_per_seq=T // PAGE)
    kv.set_pages(0, np.arange(T // PAGE, dtype=np.int32))
    pos = np.full(nseq, T - 1, np.int32)
    bufs = [dev(nat, np.zeros(nseq * nq * hd, np.float32)), dev(nat, np.zeros(nseq * nkv * hd, np.float32)),
            dev(nat, pos), dev(nat, np.zeros(nseq, np.int32))]
    out = nat.DeviceBuffer(nseq * nq * hd * 4)
    rc = lib.tq_hip_decode_step_noalloc(kv.h, nseq, bufs[3].ptr, bufs[2].ptr, T - 1, bufs[0].ptr, bufs[1].ptr,
                                        bufs[1].ptr, None, None, out.ptr, kv.stream)
    assert rc == nat.ESCRATCH, rc
    assert "scratch" in nat.strerror(rc)
    kv.close()
    # the array is intact: another call still matches the grown-buffer entry point
    batch_case(nat, oracle, np.array([4200, 700], np.int32), 3, [0, 1])
