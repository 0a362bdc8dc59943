"""GPU parity at the full sizes of the measured workloads, through the C-ABI.

Each test runs the launch the benchmark times — the same entry point, the
same batch, the same lengths, so the same split-K plan — and checks it against
the oracle (the C restatement of the reference's scalar Q8 path):

* batch-1 decode at the Llama-3-8B shape, context 4096: the fused step
  (RoPE + append + attend, 32 splits of 128 keys);
* 64 ragged sequences, lengths U[512, 8192] drawn with seed 2024, 16-token
  pages scattered over the pool, the fused step (one split per sequence and
  kv head, eight-wave work-groups, longest first);
* the 70B per-layer shape (64 q / 8 kv heads), batch 16 x 32768 keys, 1 % of
  the K/V values at +-8 sigma, the fused step (4 splits of 8192 keys);
* the causal prefill of 2048 tokens: the whole cache against the oracle's own
  quantize_row_q8 of the rotated k and v rows, and sampled outputs against
  attend_q8 over that independent cache;
* the reference's large-score case (tools/test_model.c:725-728: q and k x30,
  head_dim 128, 16 keys), a near-tie variant of it, and the same data through
  the paged decode and the dense prefill.

Bars: K/V codes and scales bit-exact; outputs |gpu - oracle| <= 1e-4 +
1e-3*|oracle| (fp32).  Batched runs are repeated and must match bit for bit,
and queries that read the same sequence with the same q give identical rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import BLOCK_Q8, QK, dequant
from tests.golden.gen import fill_random, normal

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-3
PAGE = 16


def assert_close(gpu, ref, what=""):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    if bad.any():
        i = int(np.argmax(err - (ATOL + RTOL * np.abs(ref))))
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside 1e-4 + 1e-3|ref|; "
                             f"worst at {i}: gpu {gpu.flat[i]!r} ref {ref.flat[i]!r}")


def assert_close_x30(gpu, ref, what=""):
    """The reference's own bar for its large-score case: is_close(actual,
    expected, 1e-3), |a - e| <= 1e-3 * (1 + |e|) (tools/test_model.c:12-14,727).
    Near ties at this scale are ill-conditioned in fp32: the reference's AVX2
    build differs from its scalar build by up to 3e-4 on the tie data here
    (2 values of 1024 outside 1e-4 + 1e-3|ref| at g=4, 300 keys), so they are
    held to this bar, and the cases without a tie to the strict one."""
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    bad = err > 1e-3 * (1.0 + np.abs(ref))
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside 1e-3(1+|ref|), max {err.max():.3e}"


@pytest.fixture(scope="module")
def nat():
    from tailorquantkernel_amd import native
    native.init(0)
    assert native.device_arch().startswith("gfx950")
    return native


def dev(nat, a):
    return nat.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def rope_rows(oracle, hd, positions, theta):
    cos = np.zeros((len(positions), hd // 2), np.float32)
    sin = np.zeros((len(positions), hd // 2), np.float32)
    for i, p in enumerate(positions):
        cos[i], sin[i] = oracle.rope_table(hd, int(p), theta)
    return cos, sin


def quantize_heads(oracle, rows, nkv, hd):
    """rows [T][nkv*hd] fp32 -> the reference's flat cache layout [nkv][T][nb]."""
    T = rows.shape[0]
    per_head = np.ascontiguousarray(rows.reshape(T, nkv, hd).transpose(1, 0, 2))
    return oracle.quantize_row_q8(per_head.reshape(-1)).reshape(nkv, T, hd // QK)


def fill_from_pattern(nat, kv, seq, length, dk_rows, dv_rows, pattern_rows):
    """Positions [0, length) of `seq` <- pattern row (p mod pattern_rows),
    quantized on the device by tq_hip_kv_append_async (no RoPE)."""
    lib = nat.load()
    dseq = dev(nat, np.full(pattern_rows, seq, np.int32))
    keep = []
    for p0 in range(0, length, pattern_rows):
        n = min(pattern_rows, length - p0)
        dpos = dev(nat, np.arange(p0, p0 + n, dtype=np.int32))
        nat.check(lib.tq_hip_kv_append_async(kv.h, n, dseq.ptr, dpos.ptr, dk_rows.ptr, dv_rows.ptr, None, None,
                                             kv.stream), "tq_hip_kv_append_async")
        keep.append(dpos)
    nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")


def pool_rows(nat, kv, pages, length):
    """Rows [0, length) of a sequence whose logical pages are `pages`, read
    from one download of the whole pool: K and V as [nkv][length][nb]."""
    base, nbytes, _ = kv.pool()
    raw = np.empty(nbytes, np.uint8)
    nat.check(nat.load().tq_hip_memcpy_d2h(raw.ctypes.data, base, nbytes, None), "pool download")
    return rows_of(raw, kv.nkv, kv.nb, pages, length)


def rows_of(raw, nkv, nb, pages, length):
    row = nb * 36
    p = raw.reshape(-1, nkv, 2, PAGE, row)
    sel = p[np.asarray(pages)[: (length + PAGE - 1) // PAGE]]          # [np][nkv][2][16][row]
    sel = sel.transpose(1, 2, 0, 3, 4).reshape(nkv, 2, -1, row)[:, :, :length]
    k = np.ascontiguousarray(sel[:, 0]).view(BLOCK_Q8).reshape(nkv, length, nb)
    v = np.ascontiguousarray(sel[:, 1]).view(BLOCK_Q8).reshape(nkv, length, nb)
    return k, v


def outlier_rows(rng, n_rows, width, frac):
    x = rng.standard_normal((n_rows, width), dtype=np.float32)
    flat = x.reshape(-1)
    idx = rng.choice(flat.size, int(flat.size * frac), replace=False)
    flat[idx] = np.where(rng.random(idx.size) < 0.5, -8.0, 8.0).astype(np.float32)
    return x


def run_batched_step(nat, oracle, *, nq, nkv, hd, lens, theta, outliers, sample, seed):
    """The batched fused step exactly as the benchmark launches it, then the
    sampled sequences against the oracle and the batch-wide properties."""
    lib = nat.load()
    nb = hd // QK
    nseq = lens.size
    pages_per = (lens + PAGE - 1) // PAGE
    total = int(pages_per.sum())
    kv = nat.PagedKV(nq, nkv, hd, n_pages=total, max_seqs=nseq, max_pages_per_seq=int(pages_per.max()))
    rng = np.random.default_rng(seed)
    perm = rng.permutation(total).astype(np.int32)     # pages scattered over the pool
    page_lists, at = [], 0
    for i in range(nseq):
        page_lists.append(perm[at:at + pages_per[i]])
        kv.set_pages(i, page_lists[-1])
        at += pages_per[i]
    pat = 8192
    krows = outlier_rows(rng, pat, nkv * hd, outliers)
    vrows = outlier_rows(rng, pat, nkv * hd, outliers)
    dk_rows, dv_rows = dev(nat, krows), dev(nat, vrows)
    for i in range(nseq):
        fill_from_pattern(nat, kv, i, int(lens[i]), dk_rows, dv_rows, pat)
    del dk_rows, dv_rows
    kpat, vpat = quantize_heads(oracle, krows, nkv, hd), quantize_heads(oracle, vrows, nkv, hd)

    pos = (lens - 1).astype(np.int32)
    q = rng.standard_normal(nseq * nq * hd, dtype=np.float32)
    k = rng.standard_normal(nseq * nkv * hd, dtype=np.float32)
    v = rng.standard_normal(nseq * nkv * hd, dtype=np.float32)
    cos, sin = rope_rows(oracle, hd, pos, theta)
    dq, dk, dv, dc, ds, dpos = dev(nat, q), dev(nat, k), dev(nat, v), dev(nat, cos), dev(nat, sin), dev(nat, pos)
    dseq = dev(nat, np.arange(nseq, dtype=np.int32))
    dout = nat.DeviceBuffer(nseq * nq * hd * 4)
    outs = []
    for _ in range(2):   # the step is idempotent: the same token lands in the same slot
        nat.check(lib.tq_hip_decode_step_async(kv.h, nseq, dseq.ptr, dpos.ptr, int(pos.max()), dq.ptr, dk.ptr,
                                               dv.ptr, dc.ptr, ds.ptr, dout.ptr, kv.stream), "decode_step")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        outs.append(dout.download((nseq, nq * hd), np.float32))
    assert outs[0].tobytes() == outs[1].tobytes(), "repeated launch differs"
    out = outs[0]

    base, nbytes, _ = kv.pool()
    raw = np.empty(nbytes, np.uint8)
    nat.check(lib.tq_hip_memcpy_d2h(raw.ctypes.data, base, nbytes, None), "pool download")
    for i in sample:
        L = int(lens[i])
        # the oracle's cache: the pattern rows, then store_kv of the step's token
        kc = np.ascontiguousarray(np.tile(kpat, (1, (L + pat - 1) // pat, 1))[:, :L])
        vc = np.ascontiguousarray(np.tile(vpat, (1, (L + pat - 1) // pat, 1))[:, :L])
        rc, ref = oracle.attention_qkv(kc.reshape(-1), vc.reshape(-1), nq, nkv, hd, L, theta, L - 1,
                                       q[i * nq * hd:(i + 1) * nq * hd], k[i * nkv * hd:(i + 1) * nkv * hd],
                                       v[i * nkv * hd:(i + 1) * nkv * hd])
        assert rc == 0
        gk, gv = rows_of(raw, nkv, nb, page_lists[i], L)
        assert gk.tobytes() == kc.tobytes(), f"K cache of sequence {i} (len {L})"
        assert gv.tobytes() == vc.tobytes(), f"V cache of sequence {i} (len {L})"
        assert_close(out[i], ref, f"sequence {i} len {L}")

    # identical (sequence, q) pairs give identical rows, wherever they sit in
    # the batch: every sampled sequence twice, same q, through the attend-only
    # entry with the benchmark's batch size and longest length
    order = np.array([sample[j % len(sample)] for j in range(nseq)], np.int32)
    q2 = np.concatenate([q[s * nq * hd:(s + 1) * nq * hd] for s in order])
    dq2, dseq2, dlen2 = dev(nat, q2), dev(nat, order), dev(nat, lens[order])
    dc2, ds2 = dev(nat, cos[order]), dev(nat, sin[order])
    nat.check(lib.tq_hip_decode_async(kv.h, nseq, dseq2.ptr, dlen2.ptr, int(lens.max()), dq2.ptr, dc2.ptr, ds2.ptr,
                                      dout.ptr, kv.stream), "decode_async")
    nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
    out2 = dout.download((nseq, nq * hd), np.float32)
    for j in range(len(sample), nseq):
        assert out2[j].tobytes() == out2[j % len(sample)].tobytes(), f"row {j} differs from its twin"
    kv.close()
    return out


def test_step_8b_ctx4096(nat, oracle):
    """Batch-1 fused step at the 8B shape, context 4096: the launch the
    headline benchmark times (one sequence on consecutive pages, 32 splits)."""
    lib = nat.load()
    nq, nkv, hd, T, theta = 32, 8, 128, 4096, 5e5
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    rng = np.random.default_rng(41)
    rows_k = rng.standard_normal((T, nkv * hd), dtype=np.float32)
    rows_v = rng.standard_normal((T, nkv * hd), dtype=np.float32)
    dk_rows, dv_rows = dev(nat, rows_k), dev(nat, rows_v)
    fill_from_pattern(nat, kv, 0, T, dk_rows, dv_rows, T)
    kc, vc = quantize_heads(oracle, rows_k, nkv, hd), quantize_heads(oracle, rows_v, nkv, hd)
    for pos in (T - 1, T - 130, 2047):
        q = rng.standard_normal(nq * hd, dtype=np.float32)
        k = rng.standard_normal(nkv * hd, dtype=np.float32)
        v = rng.standard_normal(nkv * hd, dtype=np.float32)
        cos, sin = rope_rows(oracle, hd, [pos], theta)
        dq, dk, dv, dc, ds = dev(nat, q), dev(nat, k), dev(nat, v), dev(nat, cos), dev(nat, sin)
        dpos = dev(nat, np.array([pos], np.int32))
        dout = nat.DeviceBuffer(nq * hd * 4)
        nat.check(lib.tq_hip_decode_step_async(kv.h, 1, None, dpos.ptr, pos, dq.ptr, dk.ptr, dv.ptr, dc.ptr, ds.ptr,
                                               dout.ptr, kv.stream), "decode_step")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        got = dout.download((nq * hd,), np.float32)
        kf, vf = kc.reshape(-1).copy(), vc.reshape(-1).copy()
        rc, ref = oracle.attention_qkv(kf, vf, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0
        assert_close(got, ref, f"8B step at pos {pos}")
        gk, gv = pool_rows(nat, kv, np.arange(T // PAGE), T)
        assert gk.tobytes() == kf.tobytes() and gv.tobytes() == vf.tobytes(), f"cache after the step at {pos}"
        kc, vc = kf.reshape(nkv, T, hd // QK), vf.reshape(nkv, T, hd // QK)
    kv.close()


def test_batched_64_ragged(nat, oracle):
    """64 sequences, lengths U[512, 8192] (seed 2024), 8B shape, scattered
    pages, fused step.  Sampled: the longest, the shortest and six more."""
    lens = np.random.default_rng(2024).integers(512, 8193, size=64).astype(np.int32)
    by_len = np.argsort(lens, kind="stable")
    sample = sorted({int(by_len[-1]), int(by_len[0]), 0, 7, 21, 33, 50, 63})
    run_batched_step(nat, oracle, nq=32, nkv=8, hd=128, lens=lens, theta=5e5, outliers=0.0, sample=sample, seed=7)


def test_long_context_70b_batch16(nat, oracle):
    """The 70B per-layer shape, batch 16 x 32768 keys, 1 % of K/V values at
    +-8 sigma, fused step.  Sampled: the first, the last and two more."""
    lens = np.full(16, 32768, np.int32)
    run_batched_step(nat, oracle, nq=64, nkv=8, hd=128, lens=lens, theta=5e5, outliers=0.01, sample=[0, 5, 10, 15],
                     seed=8)


def test_prefill_2048_whole_cache(nat, oracle):
    """The 8B-shape causal prefill of 2048 tokens: every K row equals the
    oracle's quantize_row_q8 of the rotated k, every V row that of v, and
    sampled outputs equal attend_q8 over that independently built cache
    (token i reads rows [0, i])."""
    nq, nkv, hd, n, theta = 32, 8, 128, 2048, 5e5
    kv = nat.PagedKV.single(nq, nkv, hd, n)
    q, k, v = normal(n * nq * hd, 31), normal(n * nkv * hd, 32), normal(n * nkv * hd, 33)
    cos, sin = rope_rows(oracle, hd, range(n), theta)
    rc, out = kv.prefill(0, 0, n, q, k, v, cos, sin)
    assert rc == 0
    kr = np.concatenate([oracle.rope_apply(k[(t * nkv + h) * hd:(t * nkv + h + 1) * hd], cos[t], sin[t])
                         for t in range(n) for h in range(nkv)]).reshape(n, nkv * hd)
    kc = quantize_heads(oracle, kr, nkv, hd)
    vc = quantize_heads(oracle, v.reshape(n, nkv * hd), nkv, hd)
    gk, gv = pool_rows(nat, kv, np.arange(n // PAGE), n)
    assert gk.tobytes() == kc.tobytes(), "K cache after prefill"
    assert gv.tobytes() == vc.tobytes(), "V cache after prefill"
    for i in (0, 1, 31, 32, 100, 511, 1024, 1500, 2046, 2047):
        qi = q[i * nq * hd:(i + 1) * nq * hd]
        qr = np.concatenate([oracle.rope_apply(qi[h * hd:(h + 1) * hd], cos[i], sin[i]) for h in range(nq)])
        rc, ref = oracle.attend_q8(kc.reshape(-1), vc.reshape(-1), nq, nkv, hd, n, qr, i)
        assert rc == 0
        assert_close(out[i], ref, f"prefill token {i}")
    kv.close()


# ---------------------------------------------------------------------------
# large scores (tools/test_model.c:725-728) and near ties

def large_score_data(hd, n, seed, scale=30.0):
    """q and k x scale, v x1, from the reference test generator (attn_q8_case:
    fill_random(q, seed), k seed+1000, v seed+2000)."""
    return fill_random(hd, seed, scale), fill_random(n * hd, seed + 1000, scale), fill_random(n * hd, seed + 2000)


def near_tie(oracle, q, kf, hd, n, gap=(0.2, 0.8)):
    """k rows with the runner-up key moved next to the best one: the two top
    scores of attend_q8 (over the quantized q and k) end up `gap` apart."""
    qb = oracle.quantize_row_q8(q)
    qd = dequant(qb).astype(np.float64)
    scale = 1.0 / np.sqrt(hd)
    rng = np.random.default_rng(99)
    kf = kf.copy()
    for _ in range(2000):
        s = dequant(oracle.quantize_row_q8(kf)).reshape(n, hd).astype(np.float64) @ qd * scale
        a, b = np.argsort(s)[-2:][::-1]
        d = s[a] - s[b]
        if gap[0] <= d <= gap[1]:
            return kf
        # move key b toward key a (or away) by a random fraction
        t = rng.uniform(0.0, 1.0) if d > gap[1] else -rng.uniform(0.0, 0.05)
        kf[b * hd:(b + 1) * hd] = (1 - t) * kf[b * hd:(b + 1) * hd] + t * kf[a * hd:(a + 1) * hd] \
            + rng.standard_normal(hd).astype(np.float32) * 0.05
    raise AssertionError("no near tie found")


@pytest.mark.parametrize("tie", [False, True])
def test_large_scores_head(nat, oracle, tie):
    """attention_head_q8 on the reference's large-score case: head_dim 128, 16
    keys, q and k x30 (seed 90); also against the fp32 attention on the
    dequantized data within the reference's own 1e-3."""
    lib = nat.load()
    hd, n = 128, 16
    nb = hd // QK
    q, kf, vf = large_score_data(hd, n, 90)
    if tie:
        kf = near_tie(oracle, q, kf, hd, n)
    kb, vb = oracle.quantize_row_q8(kf), oracle.quantize_row_q8(vf)
    out_ref, qq_ref, _ = oracle.attention_head_q8(q, kb, vb, n, hd)
    dq, dk, dv = dev(nat, q), dev(nat, kb), dev(nat, vb)
    dqq, dsc, dout = nat.DeviceBuffer(nb * 36), nat.DeviceBuffer(n * 4), nat.DeviceBuffer(hd * 4)
    nat.check(lib.tq_hip_attention_head_q8(dq.ptr, dqq.ptr, dk.ptr, dv.ptr, n, hd, dsc.ptr, dout.ptr, None),
              "attention_head_q8")
    nat.check(lib.tq_hip_device_synchronize(), "sync")
    got = dout.download((hd,), np.float32)
    assert dqq.download((nb,), BLOCK_Q8).tobytes() == qq_ref.tobytes()
    assert_close(got, out_ref, f"large scores head (tie={tie})")
    # tools/test_model.c:639-653: against the float path on dequantized data, 1e-3
    qd, kd, vd = (dequant(x).astype(np.float64) for x in (qq_ref, kb, vb))
    s = kd.reshape(n, hd) @ qd / np.sqrt(hd)
    p = np.exp(s - s.max())
    deq = (p / p.sum()) @ vd.reshape(n, hd)
    assert np.all(np.abs(got - deq) <= 1e-3 * (1 + np.abs(deq)))


@pytest.mark.parametrize("g,T", [(1, 16), (4, 16), (8, 16), (4, 300), (4, 4096), (8, 2000)])
@pytest.mark.parametrize("tie", [False, True])
def test_large_scores_decode(nat, oracle, g, T, tie):
    """The paged MFMA decode on x30 q and k (scores of order 1e3, so the
    running max moves by far more than the lazy-rescale headroom), with and
    without a near tie between the two best keys of every query head."""
    lib = nat.load()
    nkv, hd = 2, 128
    nq = g * nkv
    nb = hd // QK
    kflat = np.zeros((nkv, T, hd), np.float32)
    q = np.zeros(nq * hd, np.float32)
    for h in range(nkv):
        qh, kh, _ = large_score_data(hd, T if T <= 300 else 16, 90 + h)
        if T > 300:   # long contexts: x30 keys from numpy, the reference generator's q
            kh = (normal(T * hd, 500 + h) * 30.0).astype(np.float32)
        for j in range(g):
            qj = fill_random(hd, 190 + 10 * h + j, 30.0) if j else qh
            q[(h * g + j) * hd:(h * g + j + 1) * hd] = qj
        if tie:
            kh = near_tie(oracle, q[h * g * hd:(h * g + 1) * hd], kh, hd, T)
        kflat[h] = kh.reshape(T, hd)
    vflat = normal(nkv * T * hd, 77).reshape(nkv, T, hd)
    kc = oracle.quantize_row_q8(kflat.reshape(-1)).reshape(nkv, T, nb)
    vc = oracle.quantize_row_q8(vflat.reshape(-1)).reshape(nkv, T, nb)
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    kv.write(0, 0, kc, vc)
    dq, dout = dev(nat, q), nat.DeviceBuffer(nq * hd * 4)
    dlen = dev(nat, np.array([T], np.int32))
    nat.check(lib.tq_hip_decode_async(kv.h, 1, None, dlen.ptr, T, dq.ptr, None, None, dout.ptr, None), "decode")
    nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
    got = dout.download((nq * hd,), np.float32)
    rc, ref = oracle.attend_q8(kc.reshape(-1), vc.reshape(-1), nq, nkv, hd, T, q, T - 1)
    assert rc == 0
    (assert_close_x30 if tie else assert_close)(got, ref, f"x30 decode g={g} T={T} tie={tie}")
    kv.close()


def exact_prefill(oracle, kc, vc, nq, nkv, hd, n, q, cos, sin):
    """attention_layer_batch's outputs evaluated in fp64 on the operands the
    reference quantizes (its rotated, quantize_row_q8'd q rows and the cache
    its store_kv wrote): the value both fp32 evaluations approximate."""
    nb, g = hd // QK, nq // nkv
    kc, vc = kc.reshape(nkv, n, nb), vc.reshape(nkv, n, nb)
    kd, kq = kc["d"].astype(np.float64), kc["q"].astype(np.float64)
    V = (vc["q"].astype(np.float64) * vc["d"].astype(np.float64)[..., None]).reshape(nkv, n, hd)
    out = np.zeros((n, nq * hd))
    for t in range(n):
        for h in range(nq):
            qb = oracle.quantize_row_q8(oracle.rope_apply(q[(t * nq + h) * hd:(t * nq + h + 1) * hd], cos[t], sin[t]))
            dots = np.einsum("kbj,bj->kb", kq[h // g, :t + 1], qb["q"].astype(np.float64))
            s = (dots * kd[h // g, :t + 1] * qb["d"].astype(np.float64)[None]).sum(1) / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ V[h // g, :t + 1]
    return out


@pytest.mark.parametrize("whole", ["", "1"])
@pytest.mark.parametrize("tie", [False, True])
def test_large_scores_prefill(nat, oracle, tie, whole, monkeypatch):
    """The dense MFMA prefill on x30 q and k (128 tokens at the 8B shape),
    with and without near ties between each token's two best keys; by the
    plan's choice (the paired kernel at this size) and forced through the
    whole-block kernel.

    Scores here reach ~10^3, so every fp32 evaluation carries ~1e-4 relative
    error in its softmax weights: the oracle (the reference's scalar order)
    is itself 1.7e-4 to 4.1e-4 away from the fp64 value of the same quantized
    operands over seeds 0-7, beyond 1e-4 + 1e-3|ref|.  So the outputs are held
    to the reference's own bar for this case against the oracle, and to the
    exact value: no further from it than twice the oracle's own distance
    (measured 0.4-1.2x over seeds 0-7, both kernels)."""
    if whole:
        monkeypatch.setenv("TQ_HIP_PREFILL_WHOLE", whole)
    nq, nkv, hd, n, theta = 32, 8, 128, 128, 1e4
    rng = np.random.default_rng(5)
    q = (rng.standard_normal(n * nq * hd, dtype=np.float32) * 30.0).astype(np.float32)
    k = (rng.standard_normal(n * nkv * hd, dtype=np.float32) * 30.0).astype(np.float32)
    v = rng.standard_normal(n * nkv * hd, dtype=np.float32)
    if tie:
        # key t+1 repeats key t (before RoPE): query t+1's two best candidates
        # include two rows a rotation apart, and exact repeats tie exactly
        kk = k.reshape(n, nkv * hd)
        kk[1::2] = kk[0::2] + rng.standard_normal(kk[1::2].shape).astype(np.float32) * 0.3
    cos, sin = rope_rows(oracle, hd, range(n), theta)
    kv = nat.PagedKV.single(nq, nkv, hd, n)
    rc, out = kv.prefill(0, 0, n, q, k, v, cos, sin)
    assert rc == 0
    from oracle.binding import blocks
    kc, vc = blocks(nkv * n * (hd // QK)), blocks(nkv * n * (hd // QK))
    rc, ref = oracle.prefill_qkv(kc, vc, nq, nkv, hd, n, theta, 0, n, q, k, v)
    assert rc == 0
    assert_close_x30(out, ref, f"x30 prefill tie={tie}")
    exact = exact_prefill(oracle, kc, vc, nq, nkv, hd, n, q, cos, sin)
    e_gpu, e_ref = np.abs(out - exact).max(), np.abs(ref - exact).max()
    assert e_gpu <= 2.0 * e_ref, f"x30 prefill tie={tie}: {e_gpu:.3e} from the fp64 value, the oracle {e_ref:.3e}"
    kv.close()
