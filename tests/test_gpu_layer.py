"""GPU parity of the attention layer around the cache: the per-head q/k RMSNorm
fused into the decode step (model/attention_layer.c:48-53,183-191), checked
through libtqhip.so's C-ABI against the oracle (oracle_rmsnorm then the
attention core; the oracle's whole layer is bit-exact with the reference's
attention_layer, tests/test_oracle_norm.py).

Bar: the cached K/V codes and scales bit-exact (the norm keeps the reference's
serial sum of squares, so a 1-ulp slip in 1/rms would change K scales), the
attention output within 1e-4 + 1e-3|ref|.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import QK, blocks
from tests.golden.gen import normal

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-3


def assert_close(gpu, ref, what=""):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside tolerance, max err {err.max()}"


@pytest.fixture(scope="module")
def nat():
    from tailorquantkernel_amd import native
    native.init(0)
    assert native.device_arch().startswith("gfx950")
    return native


def dev(nat, a):
    return nat.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def norm_weights(hd, seed):
    rng = np.random.default_rng(seed)
    return (rng.uniform(0.3, 1.7, hd) * rng.choice([-1.0, 1.0], hd)).astype(np.float32)


def run_norm_steps(nat, oracle, nq, nkv, hd, T, theta, eps, nseq, steps, scattered):
    lib = nat.load()
    nb = hd // QK
    pages = (T + 15) // 16
    kv = nat.PagedKV(nq, nkv, hd, n_pages=nseq * pages, max_seqs=nseq, max_pages_per_seq=pages)
    perm = (np.random.default_rng(3).permutation(nseq * pages) if scattered
            else np.arange(nseq * pages)).astype(np.int32)
    for i in range(nseq):
        kv.set_pages(i, perm[i * pages:(i + 1) * pages])
    caches = [(blocks(nkv * T * nb), blocks(nkv * T * nb)) for _ in range(nseq)]
    qn, kn = norm_weights(hd, 1), norm_weights(hd, 2)
    dqn, dkn = dev(nat, qn), dev(nat, kn)
    dseq = dev(nat, np.arange(nseq, dtype=np.int32)) if nseq > 1 else None
    for step in steps:
        pos = np.array([min(T - 1, step + 3 * i) for i in range(nseq)], np.int32)
        # raw projections: scaled and shifted so that the norm matters
        q = normal(nseq * nq * hd, step) * 7.0 + 0.5
        k = normal(nseq * nkv * hd, step + 1) * 0.05 - 0.01
        v = normal(nseq * nkv * hd, step + 2)
        cs = [oracle.rope_table(hd, int(p), theta) for p in pos]
        cos = np.concatenate([c for c, _ in cs])
        sin = np.concatenate([s for _, s in cs])
        dq, dk, dv, dc, ds = dev(nat, q), dev(nat, k), dev(nat, v), dev(nat, cos), dev(nat, sin)
        dpos, dout = dev(nat, pos), nat.DeviceBuffer(nseq * nq * hd * 4)
        nat.check(lib.tq_hip_decode_step_norm_async(kv.h, nseq, dseq.ptr if dseq else None, dpos.ptr,
                                                    int(pos.max()), dq.ptr, dk.ptr, dv.ptr, dqn.ptr, dkn.ptr,
                                                    eps, dc.ptr, ds.ptr, dout.ptr, None), "decode_step_norm")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        out = dout.download((nseq, nq * hd), np.float32)
        for i in range(nseq):
            kc, vc = caches[i]
            qi = oracle.rmsnorm(q[i * nq * hd:(i + 1) * nq * hd], qn, eps)
            ki = oracle.rmsnorm(k[i * nkv * hd:(i + 1) * nkv * hd], kn, eps)
            rc, ref = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, int(pos[i]), qi, ki,
                                           v[i * nkv * hd:(i + 1) * nkv * hd])
            assert rc == 0
            assert_close(out[i], ref, f"seq {i} pos {pos[i]}")
    for i in range(nseq):
        gk, gv = kv.read(i, 0, T)
        kc, vc = caches[i]
        assert gk.reshape(-1).tobytes() == kc.tobytes(), f"K codes/scales of seq {i}"
        assert gv.reshape(-1).tobytes() == vc.tobytes(), f"V codes/scales of seq {i}"
    kv.close()


def test_norm_step_8b_two_sequences(nat, oracle):
    run_norm_steps(nat, oracle, 32, 8, 128, 400, 5e5, 1e-6, 2, range(0, 400, 23), scattered=True)


@pytest.mark.parametrize("shape", [(8, 2, 64, 1e4, 1e-5), (4, 4, 32, 1e6, 1e-6), (8, 1, 128, 5e5, 1e-6),
                                   (6, 2, 64, 1e4, 1e-6), (16, 2, 128, 5e5, 1e-5)])
def test_norm_step_group_sizes(nat, oracle, shape):
    nq, nkv, hd, theta, eps = shape
    run_norm_steps(nat, oracle, nq, nkv, hd, 150, theta, eps, 1, list(range(0, 150, 7)) + [149], scattered=False)


def test_norm_step_errors(nat):
    lib = nat.load()
    from tailorquantkernel_amd import native
    kv = nat.PagedKV.single(8, 2, 64, 64)
    q, k, v = dev(nat, np.ones(8 * 64, np.float32)), dev(nat, np.ones(2 * 64, np.float32)), dev(nat, np.ones(128, np.float32))
    w = dev(nat, np.ones(64 + 4, np.float32))
    pos = dev(nat, np.array([3], np.int32))
    out = nat.DeviceBuffer(8 * 64 * 4)
    # a norm weight pointer that is not 16-byte aligned
    assert lib.tq_hip_decode_step_norm_async(kv.h, 1, None, pos.ptr, 3, q.ptr, k.ptr, v.ptr, w.ptr + 4, w.ptr,
                                             1e-6, None, None, out.ptr, None) == native.EINVAL
    assert lib.tq_hip_decode_step_norm_async(kv.h, 1, None, pos.ptr, 3, q.ptr, k.ptr, v.ptr, None, w.ptr,
                                             1e-6, None, None, out.ptr, None) == native.EINVAL
    kv.close()
    # head_dim 256 runs on the VALU decode kernel, which has no fused norm
    kv = nat.PagedKV.single(4, 2, 256, 32)
    q, k, v = dev(nat, np.ones(4 * 256, np.float32)), dev(nat, np.ones(512, np.float32)), dev(nat, np.ones(512, np.float32))
    w = dev(nat, np.ones(256, np.float32))
    out = nat.DeviceBuffer(4 * 256 * 4)
    assert lib.tq_hip_decode_step_norm_async(kv.h, 1, None, pos.ptr, 3, q.ptr, k.ptr, v.ptr, w.ptr, w.ptr,
                                             1e-6, None, None, out.ptr, None) == native.ETYPE
    kv.close()
