"""GPU parity of the weight side: pack/unpack, the Q8 matmul and the projections.

Compared through libtqhip.so's C-ABI with the oracle (oracle_matmul_q8 is the
restatement of kernel/q8_scalar.c:3-30) and with the golden vectors the
reference wrote on its own kernel-test shapes (tools/test_kernel.c:178-190).

Bar (the reference's own, tools/test_kernel.c:15,104): the GPU may sum the
per-block terms in another order than the scalar loop, so
* relative L2 error against the oracle <= 1e-5, and element-wise
  |gpu - oracle| <= 2 (nb + 2) 2^-24 sum_b |s_b w_d x_d| (both sums are within
  (nb + 2) 2^-24 sum_b |term| of the exact block sum);
* an all-zero input gives exactly zero (:107-117);
* pack/unpack and the workspace quantization are bit-exact.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.binding import BLOCK_Q8, QK, blocks, f32
from tests.golden.gen import checksum, fill_random

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


def abs_terms(Wq, xq, rows, cols, n_tok):
    """sum_b |s_b * w_d * x_d| in fp64, shape [n_tok, rows] (a few tokens at a time)."""
    nb = cols // QK
    wq = Wq["q"].reshape(rows, nb, QK).astype(np.float32)
    xqq = xq["q"].reshape(n_tok, nb, QK).astype(np.float32)
    wd = np.abs(Wq["d"].reshape(rows, nb).astype(np.float64))
    xd = np.abs(xq["d"].reshape(n_tok, nb).astype(np.float64))
    out = np.empty((n_tok, rows))
    step = max(1, (1 << 24) // (rows * nb))
    for t0 in range(0, n_tok, step):
        # int8 x int8 block dots are exact in fp32 (|s| <= 32 * 127^2 < 2^24)
        s = np.einsum("rbj,tbj->trb", wq, xqq[t0:t0 + step]).astype(np.float64)
        out[t0:t0 + step] = (np.abs(s) * wd[None] * xd[t0:t0 + step, None, :]).sum(-1)
    return out


def check_matmul(gpu, ref, Wq, xq, rows, cols, n_tok, what):
    gpu = np.asarray(gpu, np.float64).reshape(n_tok, rows)
    ref = np.asarray(ref, np.float64).reshape(n_tok, rows)
    assert rel_err(gpu, ref) <= 1e-5, what
    bound = 2 * (cols // QK + 2) * 2.0 ** -24 * abs_terms(Wq, xq, rows, cols, n_tok) + 1e-37
    bad = np.abs(gpu - ref) > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond the summation-order bound"


class Matrix:
    """A tiled weight matrix on the device, made from block_q8 rows by tq_hip_q8_pack."""

    def __init__(self, nat, Wq, rows, cols):
        lib = nat.load()
        self.rows, self.cols = rows, cols
        nbytes = lib.tq_hip_q8_matrix_bytes(rows, cols)
        assert nbytes == Wq.nbytes
        src = dev(nat, Wq)
        self.buf = nat.DeviceBuffer(nbytes)
        nat.check(lib.tq_hip_q8_pack(self.buf.ptr, src.ptr, rows, cols, None), "q8_pack")
        sync(nat)

    @property
    def ptr(self):
        return self.buf.ptr


def gpu_matmul(nat, M, xq, n_tok):
    lib = nat.load()
    dx = dev(nat, xq)
    dy = nat.DeviceBuffer(n_tok * M.rows * 4)
    if n_tok == 1:
        nat.check(lib.tq_hip_matmul_q8(M.ptr, dx.ptr, dy.ptr, M.rows, M.cols, None), "matmul_q8")
    else:
        nat.check(lib.tq_hip_matmul_q8_batch(M.ptr, dx.ptr, dy.ptr, M.rows, M.cols, n_tok, None),
                  "matmul_q8_batch")
    sync(nat)
    return dy.download((n_tok, M.rows), np.float32)


def tiled_layout(Wq, rows, cols):
    """The documented device layout, restated in numpy."""
    nb = cols // QK
    codes = np.zeros((rows, cols), np.int8)
    q = Wq["q"].reshape(rows, nb, QK)
    for g0 in range(0, nb, 64):
        n = min(64, nb - g0)
        grp = q[:, g0:g0 + n, :]
        base = g0 * QK
        codes[:, base:base + 16 * n] = grp[:, :, :16].reshape(rows, 16 * n)
        codes[:, base + 16 * n:base + 32 * n] = grp[:, :, 16:].reshape(rows, 16 * n)
    return codes.tobytes() + np.ascontiguousarray(Wq["d"].reshape(rows, nb)).tobytes()


def random_weights(oracle, rows, cols, seed):
    rng = np.random.default_rng(seed)
    W = (rng.random((rows, cols), dtype=np.float32) - 0.5) * 2
    return oracle.pack_matrix_q8(W)


def quantize_tokens(oracle, x, n_tok, cols):
    x = f32(x).reshape(n_tok, cols)
    return np.concatenate([oracle.quantize_row_q8(x[t]) for t in range(n_tok)])


# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(7, 64), (10, 32), (1027, 96), (33, 160), (16, 4096), (3, 2080),
                                       (5, 6144)])
def test_pack_layout_and_roundtrip(nat, oracle, rows, cols):
    lib = nat.load()
    Wq = random_weights(oracle, rows, cols, rows + cols)
    M = Matrix(nat, Wq, rows, cols)
    got = M.buf.download((Wq.nbytes,), np.uint8).tobytes()
    assert got == tiled_layout(Wq, rows, cols)
    back = nat.DeviceBuffer(Wq.nbytes)
    nat.check(lib.tq_hip_q8_unpack(back.ptr, M.ptr, rows, cols, None), "q8_unpack")
    sync(nat)
    assert back.download((Wq.size,), BLOCK_Q8).tobytes() == Wq.reshape(-1).tobytes()


def test_golden_matmul_on_gpu(nat, oracle):
    """The reference's matmul_q8_scalar outputs, reproduced within the summation-order bound."""
    g = np.load(GOLDEN, allow_pickle=False)
    for i, (rows, cols, n_tok, kind) in enumerate(g["cases"]):
        rows, cols, n_tok, kind = int(rows), int(cols), int(n_tok), int(kind)
        W = fill_random(rows * cols, 3000 + 17 * i, 1.0)
        x = (fill_random(n_tok * cols, 4000 + 17 * i, 1.0) if kind == 0 else
             np.full(n_tok * cols, 1.0 if kind == 1 else 0.0, np.float32))
        Wq = oracle.pack_matrix_q8(W.reshape(rows, cols))
        xq = quantize_tokens(oracle, x, n_tok, cols)
        assert [checksum(Wq), checksum(xq)] == list(g[f"packed_sum_{i}"])
        y = gpu_matmul(nat, Matrix(nat, Wq, rows, cols), xq, n_tok)
        ref = g[f"y_{i}"].reshape(n_tok, rows)
        if kind == 2:
            assert np.abs(y).max() == 0.0
        else:
            check_matmul(y, ref, Wq, xq, rows, cols, n_tok, f"golden case {i}")


@pytest.mark.parametrize("rows,cols", [(256, 512), (7, 64), (10, 32), (1027, 96), (1024, 1024), (3072, 1024),
                                       (1024, 3072), (4096, 4096), (1024, 8192), (100, 2080)])
@pytest.mark.parametrize("n_tok", [1, 3, 8, 13])
def test_matmul_vs_oracle(nat, oracle, rows, cols, n_tok):
    Wq = random_weights(oracle, rows, cols, 11 * rows + cols)
    rng = np.random.default_rng(rows + 7 * cols + n_tok)
    x = rng.standard_normal((n_tok, cols)).astype(np.float32)
    xq = quantize_tokens(oracle, x, n_tok, cols)
    M = Matrix(nat, Wq, rows, cols)
    y = gpu_matmul(nat, M, xq, n_tok)
    ref = oracle.matmul_q8(Wq, xq, rows, cols, n_tok)
    check_matmul(y, ref, Wq, xq, rows, cols, n_tok, f"{rows}x{cols} n_tok={n_tok}")
    if 1 < n_tok < 16:
        # a token's row does not depend on the rest of the batch
        nb = cols // QK
        for t in (0, n_tok - 1):
            y1 = gpu_matmul(nat, M, xq[t * nb:(t + 1) * nb], 1)
            assert y1.tobytes() == y[t:t + 1].tobytes()


@pytest.mark.parametrize("rows,cols,n_tok", [(256, 512, 16), (1027, 96, 17), (7, 64, 64), (10, 32, 65),
                                             (4096, 4096, 256), (100, 2080, 100), (1024, 8192, 300),
                                             (6144, 4096, 192), (300, 2176, 48)])
def test_gemm_vs_oracle(nat, oracle, rows, cols, n_tok, monkeypatch):
    """The MFMA GEMM (forced from 16 tokens on): ragged row, token and block
    tails (2176 columns: a last 64-block group of 4 blocks in the tiled
    layout); then the default choice between the GEMM and GEMV launches."""
    Wq = random_weights(oracle, rows, cols, 3 * rows + cols)
    rng = np.random.default_rng(rows + cols + n_tok)
    x = rng.standard_normal((n_tok, cols)).astype(np.float32)
    xq = quantize_tokens(oracle, x, n_tok, cols)
    M = Matrix(nat, Wq, rows, cols)
    ref = oracle.matmul_q8(Wq, xq, rows, cols, n_tok)
    monkeypatch.setenv("TQ_HIP_GEMM_MIN_TOKENS", "16")
    y = gpu_matmul(nat, M, xq, n_tok)
    check_matmul(y, ref, Wq, xq, rows, cols, n_tok, f"gemm {rows}x{cols} n_tok={n_tok}")
    # a token's row does not depend on the rest of the batch
    nb = cols // QK
    y16 = gpu_matmul(nat, M, xq[:16 * nb], 16)
    assert y16.tobytes() == y[:16].tobytes()
    monkeypatch.delenv("TQ_HIP_GEMM_MIN_TOKENS")
    check_matmul(gpu_matmul(nat, M, xq, n_tok), ref, Wq, xq, rows, cols, n_tok, f"default {rows}x{cols} n_tok={n_tok}")


@pytest.mark.parametrize("rw", ["1", "2", "4"])
def test_rows_per_wave_identical(nat, oracle, rw, monkeypatch):
    """The rows-per-wave choice changes the launch shape, not one bit of the result."""
    rows, cols, n_tok = 1000, 2048, 5
    Wq = random_weights(oracle, rows, cols, 5)
    xq = quantize_tokens(oracle, fill_random(n_tok * cols, 9, 2.0), n_tok, cols)
    M = Matrix(nat, Wq, rows, cols)
    base = gpu_matmul(nat, M, xq, n_tok)
    monkeypatch.setenv("TQ_HIP_GEMV_RW", rw)
    assert gpu_matmul(nat, M, xq, n_tok).tobytes() == base.tobytes()


@pytest.mark.parametrize("cols,n_tok", [(96, 3), (128, 20), (4096, 40)])
def test_unaligned_activation_rows(nat, oracle, cols, n_tok, monkeypatch):
    """block_q8 activations at a 4-byte (not 16-byte) aligned address (GEMV and GEMM)."""
    monkeypatch.setenv("TQ_HIP_GEMM_MIN_TOKENS", "16")
    rows = 300
    Wq = random_weights(oracle, rows, cols, 77)
    xq = quantize_tokens(oracle, fill_random(n_tok * cols, 78, 1.0), n_tok, cols)
    M = Matrix(nat, Wq, rows, cols)
    lib = nat.load()
    raw = np.zeros(xq.nbytes + 16, np.uint8)
    raw[4:4 + xq.nbytes] = np.frombuffer(xq.tobytes(), np.uint8)
    dx = dev(nat, raw)
    dy = nat.DeviceBuffer(n_tok * rows * 4)
    nat.check(lib.tq_hip_matmul_q8_batch(M.ptr, dx.ptr + 4, dy.ptr, rows, cols, n_tok, None), "matmul")
    sync(nat)
    y = dy.download((n_tok, rows), np.float32)
    check_matmul(y, oracle.matmul_q8(Wq, xq, rows, cols, n_tok), Wq, xq, rows, cols, n_tok, "unaligned")


@pytest.mark.parametrize("nq,nkv,hd,hidden,n_tok", [(32, 8, 128, 4096, 1), (32, 8, 128, 4096, 4),
                                                    (8, 2, 64, 256, 3), (6, 2, 32, 160, 1),
                                                    (64, 8, 128, 8192, 1), (32, 8, 128, 4096, 40),
                                                    (8, 2, 64, 256, 130), (8, 2, 32, 256, 40)])
def test_project_qkv_and_output(nat, oracle, nq, nkv, hd, hidden, n_tok):
    """(8, 2, 32, 256, 40): q/k/v segments end at rows 256, 320 and 384, so a
    128-row GEMM tile spans two segments (the per-row copy addressing)."""
    lib = nat.load()
    qr, kr = nq * hd, nkv * hd
    wq = random_weights(oracle, qr, hidden, 1)
    wk = random_weights(oracle, kr, hidden, 2)
    wv = random_weights(oracle, kr, hidden, 3)
    wo = random_weights(oracle, hidden, qr, 4)
    xn = fill_random(n_tok * hidden, 5, 2.0)
    Mq, Mk, Mv, Mo = (Matrix(nat, wq, qr, hidden), Matrix(nat, wk, kr, hidden), Matrix(nat, wv, kr, hidden),
                      Matrix(nat, wo, hidden, qr))
    dx = dev(nat, xn)
    ws = nat.DeviceBuffer(n_tok * max(hidden, qr) // QK * 36)
    dq, dk, dv = (nat.DeviceBuffer(n_tok * qr * 4), nat.DeviceBuffer(n_tok * kr * 4),
                  nat.DeviceBuffer(n_tok * kr * 4))
    nat.check(lib.tq_hip_project_qkv(Mq.ptr, Mk.ptr, Mv.ptr, qr, kr, hidden, dx.ptr, n_tok, ws.ptr,
                                     dq.ptr, dk.ptr, dv.ptr, None), "project_qkv")
    sync(nat)
    xq = quantize_tokens(oracle, xn, n_tok, hidden)
    assert ws.download((xq.size,), BLOCK_Q8).tobytes() == xq.tobytes()
    for name, M, W, d in (("q", Mq, wq, dq), ("k", Mk, wk, dk), ("v", Mv, wv, dv)):
        got = d.download((n_tok, M.rows), np.float32)
        ref = oracle.project_q8(W, M.rows, hidden, xn)
        check_matmul(got, ref, W, xq, M.rows, hidden, n_tok, f"project_qkv {name}")

    attn = fill_random(n_tok * qr, 6, 1.5)
    da = dev(nat, attn)
    dout = nat.DeviceBuffer(n_tok * hidden * 4)
    nat.check(lib.tq_hip_project_output(Mo.ptr, hidden, qr, da.ptr, n_tok, ws.ptr, dout.ptr, None),
              "project_output")
    sync(nat)
    aq = quantize_tokens(oracle, attn, n_tok, qr)
    got = dout.download((n_tok, hidden), np.float32)
    check_matmul(got, oracle.project_q8(wo, hidden, qr, attn), wo, aq, hidden, qr, n_tok, "project_output")


def test_zero_and_constant_input(nat, oracle):
    lib = nat.load()
    rows, cols = 256, 512
    Wq = random_weights(oracle, rows, cols, 3)
    M = Matrix(nat, Wq, rows, cols)
    ws = nat.DeviceBuffer(2 * cols // QK * 36)
    for x in (np.zeros(2 * cols, np.float32), np.ones(2 * cols, np.float32)):
        dx = dev(nat, x)
        dy = nat.DeviceBuffer(2 * rows * 4)
        nat.check(lib.tq_hip_project_output(M.ptr, rows, cols, dx.ptr, 2, ws.ptr, dy.ptr, None), "project")
        sync(nat)
        y = dy.download((2, rows), np.float32)
        ref = oracle.project_q8(Wq, rows, cols, x)
        if not x.any():
            assert np.abs(y).max() == 0.0
        else:
            xq = quantize_tokens(oracle, x, 2, cols)
            check_matmul(y, ref, Wq, xq, rows, cols, 2, "constant x")
