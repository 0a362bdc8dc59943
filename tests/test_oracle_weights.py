"""Pins the oracle's weight side: pack_matrix and the Q8 matmul.

oracle/tq_oracle.c restates packer/packer.c:4-31 (oracle_pack_matrix_q8) and
kernel/q8_scalar.c:3-30 (oracle_matmul_q8, oracle_matmul_q8_batch), plus the
quantize-then-matmul projection of model/attention_layer.c:38-46,161-167
(oracle_project_q8).  Anchors:

1. golden vectors (tests/golden/golden_matmul_q8.npz) written by the reference
   compiled from its own sources, on the shapes of its own kernel test
   (tools/test_kernel.c:178-190) — bit-exact;
2. the compiled reference (oracle/_ref) when built: bit-exact against
   matmul_q8_scalar, within the reference's SIMD-vs-scalar limit (relative L2
   error 1e-5, tools/test_kernel.c:15,22-30,104) against matmul_q8_avx2 and
   its token-tiled batch;
3. the mathematics: the exact block sum sum_b s_b*w_d*x_d in fp64 (a dropped
   scale, a transposed operand or a wrong block index fails it), the fp64
   product with the unquantized weights within the reference's 1.5 %
   (tools/test_kernel.c:13,101), an all-zero input giving exactly zero
   (:107-117), and the packer's own rules (scale 1 for a zero block, ties away
   from zero, |code| <= 127).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.binding import QK, blocks, f32
from tests.golden.gen import checksum, fill_random

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden_matmul_q8.npz")


def rel_err(a, b) -> float:
    """tools/test_kernel.c:22-30: ||a - b||_2 / ||b||_2 (||a - b|| when b = 0)."""
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    num = float(((a - b) ** 2).sum())
    den = float((b * b).sum())
    return float(np.sqrt(num / den)) if den > 0 else float(np.sqrt(num))


def quantize_tokens(oracle, x, n_tok, cols):
    x = f32(x).reshape(n_tok, cols)
    return np.concatenate([oracle.quantize_row_q8(x[t]) for t in range(n_tok)])


def exact_terms(Wq, xq, rows, cols, n_tok):
    """fp64 per-block terms s_b * w_d * x_d, shape [n_tok, rows, nb]."""
    nb = cols // QK
    wq = Wq["q"].reshape(rows, nb, QK).astype(np.int64)
    wd = Wq["d"].reshape(rows, nb).astype(np.float64)
    xqq = xq["q"].reshape(n_tok, nb, QK).astype(np.int64)
    xd = xq["d"].reshape(n_tok, nb).astype(np.float64)
    s = np.einsum("rbj,tbj->trb", wq, xqq)
    return s.astype(np.float64) * wd[None] * xd[:, None, :]


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def _golden_inputs(i, rows, cols, n_tok, kind):
    W = fill_random(rows * cols, 3000 + 17 * i, 1.0)
    if kind == 0:
        x = fill_random(n_tok * cols, 4000 + 17 * i, 1.0)
    elif kind == 1:
        x = np.ones(n_tok * cols, np.float32)
    else:
        x = np.zeros(n_tok * cols, np.float32)
    return W, x


# --------------------------------------------------------------------------
# 1. golden vectors
# --------------------------------------------------------------------------

def test_golden_pack_and_matmul(oracle, golden):
    for i, (rows, cols, n_tok, kind) in enumerate(golden["cases"]):
        rows, cols, n_tok, kind = int(rows), int(cols), int(n_tok), int(kind)
        W, x = _golden_inputs(i, rows, cols, n_tok, kind)
        assert [checksum(W), checksum(x)] == list(golden[f"in_sum_{i}"])
        Wq = oracle.pack_matrix_q8(W.reshape(rows, cols))
        xq = quantize_tokens(oracle, x, n_tok, cols)
        assert [checksum(Wq), checksum(xq)] == list(golden[f"packed_sum_{i}"])
        y = oracle.matmul_q8(Wq, xq, rows, cols, n_tok)
        assert y.reshape(-1).tobytes() == golden[f"y_{i}"].tobytes(), (rows, cols, n_tok, kind)
        yp = oracle.project_q8(Wq, rows, cols, x)
        assert yp.tobytes() == y.tobytes()


# --------------------------------------------------------------------------
# 2. the compiled reference
# --------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols,n_tok", [(256, 512, 1), (7, 64, 1), (10, 32, 1), (1027, 96, 1),
                                             (3072, 1024, 1), (1024, 3072, 1), (33, 160, 7),
                                             (64, 2048, 4)])
def test_ref_matmul(oracle, ref_scalar, ref_avx2, rows, cols, n_tok):
    rng = np.random.default_rng(rows * 31 + cols + n_tok)
    W = (rng.random((rows, cols), dtype=np.float32) - 0.5) * 2
    x = (rng.random((n_tok, cols), dtype=np.float32) - 0.5) * 2
    Wq = oracle.pack_matrix_q8(W)
    assert Wq.tobytes() == ref_scalar.pack_matrix_q8(W).tobytes()
    xq = quantize_tokens(oracle, x, n_tok, cols)
    y = oracle.matmul_q8(Wq, xq, rows, cols, n_tok)
    assert y.tobytes() == ref_scalar.matmul_q8(Wq, xq, rows, cols, n_tok).tobytes()
    y_simd = ref_avx2.matmul_q8(Wq, xq, rows, cols, n_tok, simd=True)
    assert rel_err(y_simd, y) <= 1e-5


# --------------------------------------------------------------------------
# 3. the mathematics
# --------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols,n_tok", [(256, 512, 1), (10, 32, 1), (1027, 96, 1), (48, 1024, 3)])
def test_matmul_vs_exact_block_sum(oracle, rows, cols, n_tok):
    rng = np.random.default_rng(cols + rows)
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal((n_tok, cols)).astype(np.float32) * 3
    Wq = oracle.pack_matrix_q8(W)
    xq = quantize_tokens(oracle, x, n_tok, cols)
    y = oracle.matmul_q8(Wq, xq, rows, cols, n_tok).astype(np.float64)
    terms = exact_terms(Wq, xq, rows, cols, n_tok)
    exact = terms.sum(-1)
    # Each term is rounded twice and each of the nb serial adds once.
    nb = cols // QK
    bound = (nb + 2) * 2.0 ** -24 * np.abs(terms).sum(-1) + 1e-30
    assert (np.abs(y - exact) <= bound).all()
    # Against the unquantized product: the reference's 1.5 % relative L2 limit.
    dense = x.astype(np.float64) @ W.astype(np.float64).T
    assert rel_err(y, dense) <= 0.015


def test_matmul_zero_and_constant_input(oracle):
    rows, cols = 256, 512
    W = fill_random(rows * cols, 11, 1.0).reshape(rows, cols)
    Wq = oracle.pack_matrix_q8(W)
    y0 = oracle.project_q8(Wq, rows, cols, np.zeros(cols, np.float32))
    assert np.abs(y0).max() == 0.0
    y1 = oracle.project_q8(Wq, rows, cols, np.ones(cols, np.float32))
    # x = 1 quantizes to d = 1/127, codes 127: y_r = sum_b (127 * sum_j q_j) * d_b / 127.
    nb = cols // QK
    exact = (Wq["q"].reshape(rows, nb, QK).astype(np.int64).sum(-1) * 127).astype(np.float64)
    exact = (exact * Wq["d"].reshape(rows, nb) * np.float64(np.float32(1.0) / np.float32(127.0))).sum(-1)
    assert np.allclose(y1[0], exact, rtol=1e-5, atol=1e-6)


def test_pack_rules(oracle):
    W = np.zeros((2, 64), np.float32)
    # block 0: all zero -> d = 1, codes 0
    # block 1: amax 127 -> d = 1, ties away from zero
    W[0, 32:] = [127.0, 0.5, -0.5, 2.5, -2.5, 1.5, 126.5, -126.5] + [0.0] * 24
    W[1, :] = np.linspace(-3.0, 5.0, 64, dtype=np.float32)
    Wq = oracle.pack_matrix_q8(W)
    assert Wq["d"][0, 0] == 1.0 and (Wq["q"][0, 0] == 0).all()
    assert Wq["d"][0, 1] == 1.0
    assert list(Wq["q"][0, 1, :8]) == [127, 1, -1, 3, -3, 2, 127, -127]
    # the activation quantizer rounds the same ties to even and keeps d = 0
    xq = oracle.quantize_row_q8(W[0])
    assert xq["d"][0] == 0.0 and list(xq["q"][1, :8]) == [127, 0, 0, 2, -2, 2, 126, -126]
    assert np.abs(Wq["q"].astype(np.int32)).max() == 127
    # the reference's pack/unpack round trip limit (tools/test_kernel.c:13,144-157)
    rows, cols = 16, 512
    Wr = fill_random(rows * cols, 99, 1.0).reshape(rows, cols)
    Wrq = oracle.pack_matrix_q8(Wr)
    back = Wrq["q"].astype(np.float32) * Wrq["d"][..., None]
    assert rel_err(back.reshape(rows, cols), Wr) <= 0.015


def test_batch_is_per_token(oracle):
    rows, cols, n_tok = 40, 256, 6
    W = fill_random(rows * cols, 5, 1.0).reshape(rows, cols)
    x = fill_random(n_tok * cols, 6, 2.0)
    Wq = oracle.pack_matrix_q8(W)
    xq = quantize_tokens(oracle, x, n_tok, cols)
    yb = oracle.matmul_q8(Wq, xq, rows, cols, n_tok)
    nb = cols // QK
    for t in range(n_tok):
        yt = oracle.matmul_q8(Wq, xq[t * nb:(t + 1) * nb], rows, cols, 1)
        assert yt.tobytes() == yb[t].tobytes()
    assert blocks(1).itemsize == 36
