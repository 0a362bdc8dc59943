"""GPU parity of the Q4 weight format: the tiled Q4 layout, the Q4 matmul
(GEMV and MFMA GEMM), the Q4 projections and the Q4 embedding lookup.

Compared through libtqhip.so's C-ABI with the oracle (oracle_matmul_q4_batch
restates kernel/q4_scalar.c:3-32, bit-exact with the reference's scalar
build) and with the golden vectors the reference wrote on its own kernel-test
shapes (tools/test_kernel.c:178-190).  Bar, as for Q8 (tools/test_kernel.c:15):
relative L2 error <= 1e-5 and element-wise |gpu - oracle| <= 2 (nb + 2) 2^-24
sum_b |s_b w_d x_d|; pack/unpack and the embedding rows bit-exact.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.binding import QK, blocks4
from tests.golden.gen import fill_random

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden_matmul_q8.npz")


@pytest.fixture(scope="module")
def nat():
    from tailorquantkernel_amd import native
    native.init(0)
    assert native.device_arch().startswith("gfx950")
    return native


def dev(nat, a):
    return nat.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def sync(nat):
    nat.check(nat.load().tq_hip_device_synchronize(), "sync")


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    den = float((b * b).sum())
    num = float(((a - b) ** 2).sum())
    return float(np.sqrt(num / den)) if den > 0 else float(np.sqrt(num))


def codes_q4(Wq):
    q = Wq["q"].astype(np.int16)
    return np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=-1)


def check_matmul(gpu, ref, Wq, xq, rows, cols, n_tok, what):
    nb = cols // QK
    gpu = np.asarray(gpu, np.float64).reshape(n_tok, rows)
    ref = np.asarray(ref, np.float64).reshape(n_tok, rows)
    assert rel_err(gpu, ref) <= 1e-5, what
    wq = codes_q4(Wq.reshape(rows, nb)).astype(np.float32)
    xqq = xq["q"].reshape(n_tok, nb, QK).astype(np.float32)
    wd = np.abs(Wq["d"].reshape(rows, nb).astype(np.float64))
    xd = np.abs(xq["d"].reshape(n_tok, nb).astype(np.float64))
    step = max(1, (1 << 24) // (rows * nb))
    for t0 in range(0, n_tok, step):
        s = np.einsum("rbj,tbj->trb", wq, xqq[t0:t0 + step]).astype(np.float64)
        terms = (np.abs(s) * wd[None] * xd[t0:t0 + step, None, :]).sum(-1)
        bound = 2 * (nb + 2) * 2.0 ** -24 * terms + 1e-37
        bad = np.abs(gpu[t0:t0 + step] - ref[t0:t0 + step]) > bound
        assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond the summation-order bound"


class Matrix4:
    """A tiled Q4 matrix on the device, made from block_q4 rows by tq_hip_q4_pack."""

    def __init__(self, nat, Wq, rows, cols):
        lib = nat.load()
        self.rows, self.cols = rows, cols
        nbytes = lib.tq_hip_q4_matrix_bytes(rows, cols)
        assert nbytes == Wq.nbytes == rows * (cols // QK) * 20
        src = dev(nat, Wq)
        self.buf = nat.DeviceBuffer(nbytes)
        nat.check(lib.tq_hip_q4_pack(self.buf.ptr, src.ptr, rows, cols, None), "q4_pack")
        sync(nat)

    @property
    def ptr(self):
        return self.buf.ptr


def gpu_matmul4(nat, M, xq, n_tok):
    lib = nat.load()
    dx = dev(nat, xq)
    dy = nat.DeviceBuffer(n_tok * M.rows * 4)
    if n_tok == 1:
        nat.check(lib.tq_hip_matmul_q4(M.ptr, dx.ptr, dy.ptr, M.rows, M.cols, None), "matmul_q4")
    else:
        nat.check(lib.tq_hip_matmul_q4_batch(M.ptr, dx.ptr, dy.ptr, M.rows, M.cols, n_tok, None),
                  "matmul_q4_batch")
    sync(nat)
    return dy.download((n_tok, M.rows), np.float32)


def quantize_tokens(oracle, x, n_tok, cols):
    x = np.asarray(x, np.float32).reshape(n_tok, cols)
    return np.concatenate([oracle.quantize_row_q8(x[t]) for t in range(n_tok)])


def test_q4_layout_pack_unpack(nat, oracle):
    lib = nat.load()
    rows, cols = 37, 2080          # 65 blocks: a second, one-block group
    W = fill_random(rows * cols, 71, 1.0).reshape(rows, cols)
    Wq = oracle.pack_matrix_q4(W)
    M = Matrix4(nat, Wq, rows, cols)
    raw = M.buf.download((Wq.nbytes,), np.uint8)
    nb = cols // QK
    # the documented layout: block_q4.q of every block in row order, then the scales
    assert raw[:rows * nb * 16].tobytes() == np.ascontiguousarray(Wq["q"]).tobytes()
    assert raw[rows * nb * 16:].tobytes() == np.ascontiguousarray(Wq["d"]).tobytes()
    back = nat.DeviceBuffer(Wq.nbytes)
    nat.check(lib.tq_hip_q4_unpack(back.ptr, M.ptr, rows, cols, None), "q4_unpack")
    sync(nat)
    assert back.download((Wq.nbytes,), np.uint8).tobytes() == Wq.tobytes()
    assert lib.tq_hip_q4_matrix_bytes(rows, 33) == 0
    assert lib.tq_hip_q4_pack(M.ptr + 4, back.ptr, rows, cols, None) != 0   # unaligned tiled matrix


@pytest.mark.parametrize("rows,cols,n_tok", [(256, 512, 1), (7, 64, 1), (10, 32, 1), (1027, 96, 1), (3072, 1024, 1),
                                             (6144, 4096, 1), (4096, 14336, 1), (28672, 4096, 1), (33, 160, 7),
                                             (64, 2048, 4), (300, 4096, 2), (256, 512, 16), (1000, 1024, 40),
                                             (130, 96, 17), (4096, 4096, 130)])
def test_q4_matmul(nat, oracle, rows, cols, n_tok, monkeypatch):
    """From 16 tokens on the GEMM is forced (the default may pick GEMV launches)."""
    monkeypatch.setenv("TQ_HIP_GEMM_MIN_TOKENS", "16")
    rng = np.random.default_rng(rows + 7 * cols + n_tok)
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    W[rows // 2, :QK] = 0.0
    x = rng.standard_normal((n_tok, cols)).astype(np.float32) * 2
    Wq = oracle.pack_matrix_q4(W)
    xq = quantize_tokens(oracle, x, n_tok, cols)
    ref = oracle.matmul_q4(Wq, xq, rows, cols, n_tok)
    got = gpu_matmul4(nat, Matrix4(nat, Wq, rows, cols), xq, n_tok)
    check_matmul(got, ref, Wq, xq, rows, cols, n_tok, (rows, cols, n_tok))
    # an all-zero input gives exactly zero
    zq = quantize_tokens(oracle, np.zeros((n_tok, cols), np.float32), n_tok, cols)
    z = gpu_matmul4(nat, Matrix4(nat, Wq, rows, cols), zq, n_tok)
    assert np.abs(z).max() == 0.0


def test_q4_golden(nat, oracle):
    g = np.load(GOLDEN, allow_pickle=False)
    for i, (rows, cols, n_tok, kind) in enumerate(g["cases"]):
        rows, cols, n_tok, kind = int(rows), int(cols), int(n_tok), int(kind)
        W = fill_random(rows * cols, 3000 + 17 * i, 1.0).reshape(rows, cols)
        if kind == 0:
            x = fill_random(n_tok * cols, 4000 + 17 * i, 1.0)
        elif kind == 1:
            x = np.ones(n_tok * cols, np.float32)
        else:
            x = np.zeros(n_tok * cols, np.float32)
        Wq = oracle.pack_matrix_q4(W)
        xq = quantize_tokens(oracle, x, n_tok, cols)
        got = gpu_matmul4(nat, Matrix4(nat, Wq, rows, cols), xq, n_tok)
        check_matmul(got, g[f"y4_{i}"], Wq, xq, rows, cols, n_tok, ("golden", i))


@pytest.mark.parametrize("n_tok", [1, 2, 5, 20])
def test_q4_projections(nat, oracle, n_tok):
    lib = nat.load()
    hidden, qr, kr = 1024, 1024, 256
    rng = np.random.default_rng(40 + n_tok)
    mats = {k: oracle.pack_matrix_q4(rng.standard_normal((r, c)).astype(np.float32) * 0.05)
            for k, (r, c) in dict(wq=(qr, hidden), wk=(kr, hidden), wv=(kr, hidden), wo=(hidden, qr)).items()}
    dims = dict(wq=(qr, hidden), wk=(kr, hidden), wv=(kr, hidden), wo=(hidden, qr))
    D = {k: Matrix4(nat, mats[k], *dims[k]) for k in mats}
    xn = rng.standard_normal((n_tok, hidden)).astype(np.float32)
    attn = rng.standard_normal((n_tok, qr)).astype(np.float32)
    dxn, dattn = dev(nat, xn), dev(nat, attn)
    ws = nat.DeviceBuffer(n_tok * max(hidden, qr) // QK * 36)
    dq, dk, dv = (nat.DeviceBuffer(n_tok * r * 4) for r in (qr, kr, kr))
    dout = nat.DeviceBuffer(n_tok * hidden * 4)
    nat.check(lib.tq_hip_project_qkv_q4(D["wq"].ptr, D["wk"].ptr, D["wv"].ptr, qr, kr, hidden, dxn.ptr, n_tok,
                                        ws.ptr, dq.ptr, dk.ptr, dv.ptr, None), "project_qkv_q4")
    sync(nat)
    xq = quantize_tokens(oracle, xn, n_tok, hidden)
    for name, buf, r in (("wq", dq, qr), ("wk", dk, kr), ("wv", dv, kr)):
        got = buf.download((n_tok, r), np.float32)
        check_matmul(got, oracle.matmul_q4(mats[name], xq, r, hidden, n_tok), mats[name], xq, r, hidden, n_tok,
                     name)
    nat.check(lib.tq_hip_project_output_q4(D["wo"].ptr, hidden, qr, dattn.ptr, n_tok, ws.ptr, dout.ptr, None),
              "project_output_q4")
    sync(nat)
    aq = quantize_tokens(oracle, attn, n_tok, qr)
    check_matmul(dout.download((n_tok, hidden), np.float32), oracle.matmul_q4(mats["wo"], aq, hidden, qr, n_tok),
                 mats["wo"], aq, hidden, qr, n_tok, "wo")


def test_q4_embed_lookup(nat, oracle):
    lib = nat.load()
    from tailorquantkernel_amd import native
    rng = np.random.default_rng(8)
    vocab, hidden = 1000, 2080
    E = oracle.pack_matrix_q4(rng.standard_normal((vocab, hidden)).astype(np.float32))
    dE = Matrix4(nat, E, vocab, hidden)
    out = nat.DeviceBuffer(hidden * 4)
    for tok in (0, 1, 517, vocab - 1):
        nat.check(lib.tq_hip_embed_lookup_q4(dE.ptr, vocab, hidden, tok, out.ptr, None), "embed_q4")
        sync(nat)
        rc, exp = oracle.embed_lookup_q4(E, vocab, hidden, tok)
        assert rc == 0 and out.download((hidden,), np.float32).tobytes() == exp.tobytes()
    assert lib.tq_hip_embed_lookup_q4(dE.ptr, vocab, hidden, vocab, out.ptr, None) == native.EINVAL
    toks = np.array([5, 999, 0, 5, 321], np.int32)
    dt = dev(nat, toks)
    outb = nat.DeviceBuffer(toks.size * hidden * 4)
    nat.check(lib.tq_hip_embed_lookup_q4_batch(dE.ptr, vocab, hidden, dt.ptr, toks.size, outb.ptr, None), "batch")
    sync(nat)
    got = outb.download((toks.size, hidden), np.float32)
    for i, t in enumerate(toks):
        assert got[i].tobytes() == oracle.embed_lookup_q4(E, vocab, hidden, int(t))[1].tobytes()
    assert blocks4(1).itemsize == 20


@pytest.mark.parametrize("split", ["1", "0"])
def test_q4_mlp_split_k(nat, oracle, split, monkeypatch):
    """A Q4 MLP over 20 rows: with split-K on, the gate/up and down matmuls
    take the split GEMM (partials in the workspace, summed in split order);
    off, the unsplit launches.  gate/up against the oracle's Q4 matmul of the
    quantized rows, down against the oracle's Q4 matmul of the GPU's own
    hidden rows, both within the matmul bar."""
    monkeypatch.setenv("TQ_HIP_GEMM_SPLIT", split)
    monkeypatch.setenv("TQ_HIP_GEMM_XS", "0")   # the hidden rows are read back as block_q8 rows
    import ctypes as C
    from oracle.binding import BLOCK_Q8
    lib = nat.load()
    hidden, inter, n = 512, 1024, 20
    rng = np.random.default_rng(20)
    wg = oracle.pack_matrix_q4(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wu = oracle.pack_matrix_q4(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wd = oracle.pack_matrix_q4(rng.standard_normal((hidden, inter)).astype(np.float32) * 0.1)
    G, U, D = Matrix4(nat, wg, inter, hidden), Matrix4(nat, wu, inter, hidden), Matrix4(nat, wd, hidden, inter)
    w = nat.MlpWeights(G.buf.ptr, U.buf.ptr, D.buf.ptr, hidden, inter, nat.FORMAT_Q4)
    wsb = lib.tq_hip_mlp_ws_bytes(C.byref(w), n)
    ws = nat.DeviceBuffer(wsb)
    xn = (rng.standard_normal(n * hidden) * 2).astype(np.float32)
    dx, dout = dev(nat, xn), nat.DeviceBuffer(n * hidden * 4)
    nat.check(lib.tq_hip_mlp_layer_async(C.byref(w), n, dx.ptr, dout.ptr, ws.ptr, wsb, None), "mlp")
    sync(nat)
    out = dout.download((n, hidden), np.float32)
    raw = ws.download((wsb,), np.uint8)
    al = lambda b: (b + 255) & ~255
    gate = raw[:n * inter * 4].view(np.float32).reshape(n, inter)
    up = raw[al(n * inter * 4):al(n * inter * 4) + n * inter * 4].view(np.float32).reshape(n, inter)
    hq = raw[2 * al(n * inter * 4):2 * al(n * inter * 4) + n * inter // QK * 36].view(BLOCK_Q8)
    xq = quantize_tokens(oracle, xn, n, hidden)
    check_matmul(gate, oracle.matmul_q4(wg, xq, inter, hidden, n), wg, xq, inter, hidden, n, "gate")
    check_matmul(up, oracle.matmul_q4(wu, xq, inter, hidden, n), wu, xq, inter, hidden, n, "up")
    check_matmul(out, oracle.matmul_q4(wd, hq, hidden, inter, n), wd, hq, hidden, inter, n, "down")
