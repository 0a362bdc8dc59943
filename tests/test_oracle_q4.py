"""Pins the oracle's Q4 weight format: pack_row_q4 / unpack_row_q4 and the Q4
matmul.

oracle/tq_oracle.c restates packer/packer.c:40-61 (oracle_pack_matrix_q4,
oracle_unpack_matrix_q4, with block_scale :11-19 at qmax 7), kernel/q4_scalar.c
:3-32 (oracle_matmul_q4_batch) and the Q4 branch of model/embedding.c:20-27
(oracle_embed_lookup_q4).  Anchors:

1. golden vectors (tests/golden/golden_matmul_q8.npz, the Q4 entries) written
   by the reference compiled from its own sources, on the shapes of its own
   kernel test (tools/test_kernel.c:178-190) — bit-exact;
2. the compiled reference (oracle/_ref) when built: pack and unpack byte for
   byte, matmul_q4_scalar bit-exact, matmul_q4_avx2 within the reference's
   SIMD-vs-scalar limit (relative L2 1e-5, tools/test_kernel.c:15);
3. the mathematics: the exact fp64 block sum of (nibble - 8) * x codes (a
   swapped nibble, a missing -8 or a transposed operand fails it), the fp64
   product with the unquantized weights within the reference's 10 %
   (tools/test_kernel.c:14), the pack round trip within half a step per
   value, and the packer's rules (scale 1 for a zero block, ties away from
   zero, codes in [-7, 7], code j in the low nibble of byte j).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.binding import QK, blocks4, f32
from tests.golden.gen import checksum, fill_random

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden_matmul_q8.npz")


def rel_err(a, b) -> float:
    """tools/test_kernel.c:22-30."""
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    den = float((b * b).sum())
    num = float(((a - b) ** 2).sum())
    return float(np.sqrt(num / den)) if den > 0 else float(np.sqrt(num))


def quantize_tokens(oracle, x, n_tok, cols):
    x = f32(x).reshape(n_tok, cols)
    return np.concatenate([oracle.quantize_row_q8(x[t]) for t in range(n_tok)])


def codes_q4(Wq):
    """block_q4 -> signed codes [..., 32] (low nibbles first, then high)."""
    q = Wq["q"].astype(np.int64)
    return np.concatenate([(q & 15) - 8, (q >> 4) - 8], axis=-1)


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_golden_pack_and_matmul_q4(oracle, golden):
    for i, (rows, cols, n_tok, kind) in enumerate(golden["cases"]):
        rows, cols, n_tok = int(rows), int(cols), int(n_tok)
        W = fill_random(rows * cols, 3000 + 17 * i, 1.0)
        if kind == 0:
            x = fill_random(n_tok * cols, 4000 + 17 * i, 1.0)
        elif kind == 1:
            x = np.ones(n_tok * cols, np.float32)
        else:
            x = np.zeros(n_tok * cols, np.float32)
        W4 = oracle.pack_matrix_q4(W.reshape(rows, cols))
        assert [checksum(W4)] == list(golden[f"packed4_sum_{i}"]), (rows, cols)
        xq = quantize_tokens(oracle, x, n_tok, cols)
        y = oracle.matmul_q4(W4, xq, rows, cols, n_tok)
        assert y.reshape(-1).tobytes() == golden[f"y4_{i}"].tobytes(), (rows, cols, n_tok, kind)


@pytest.mark.parametrize("rows,cols,n_tok", [(256, 512, 1), (7, 64, 1), (10, 32, 1), (1027, 96, 1),
                                             (3072, 1024, 1), (33, 160, 7), (64, 2048, 4)])
def test_ref_q4(oracle, ref_scalar, ref_avx2, rows, cols, n_tok):
    rng = np.random.default_rng(rows * 37 + cols + n_tok)
    W = (rng.random((rows, cols), dtype=np.float32) - 0.5) * 2
    W[0, :QK] = 0.0                                  # a zero block
    x = (rng.random((n_tok, cols), dtype=np.float32) - 0.5) * 2
    Wq = oracle.pack_matrix_q4(W)
    assert Wq.tobytes() == ref_scalar.pack_matrix_q4(W).tobytes()
    assert oracle.unpack_matrix_q4(Wq, rows, cols).tobytes() == \
        ref_scalar.unpack_matrix_q4(Wq, rows, cols).tobytes()
    xq = quantize_tokens(oracle, x, n_tok, cols)
    y = oracle.matmul_q4(Wq, xq, rows, cols, n_tok)
    assert y.tobytes() == ref_scalar.matmul_q4(Wq, xq, rows, cols, n_tok).tobytes()
    y_simd = ref_avx2.matmul_q4(Wq, xq, rows, cols, n_tok, simd=True)
    assert rel_err(y_simd, y) <= 1e-5
    # the Q4 embedding row is the unpacked row (model/embedding.c:20-27)
    for tok in (0, rows - 1):
        rc, e = oracle.embed_lookup_q4(Wq, rows, cols, tok)
        assert rc == 0 and e.tobytes() == ref_scalar.unpack_matrix_q4(Wq[tok], 1, cols).reshape(-1).tobytes()
    assert oracle.embed_lookup_q4(Wq, rows, cols, rows)[0] == -1


@pytest.mark.parametrize("rows,cols,n_tok", [(256, 512, 1), (10, 32, 1), (1027, 96, 1), (48, 1024, 3)])
def test_q4_matmul_vs_exact_block_sum(oracle, rows, cols, n_tok):
    rng = np.random.default_rng(cols + rows + 7)
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal((n_tok, cols)).astype(np.float32) * 3
    Wq = oracle.pack_matrix_q4(W)
    xq = quantize_tokens(oracle, x, n_tok, cols)
    y = oracle.matmul_q4(Wq, xq, rows, cols, n_tok).astype(np.float64)
    nb = cols // QK
    wq = codes_q4(Wq).reshape(rows, nb, QK)
    xqq = xq["q"].reshape(n_tok, nb, QK).astype(np.int64)
    s = np.einsum("rbj,tbj->trb", wq, xqq).astype(np.float64)
    terms = s * Wq["d"].reshape(rows, nb).astype(np.float64)[None] * \
        xq["d"].reshape(n_tok, nb).astype(np.float64)[:, None, :]
    bound = (nb + 2) * 2.0 ** -24 * np.abs(terms).sum(-1) + 1e-30
    assert (np.abs(y - terms.sum(-1)) <= bound).all()
    dense = x.astype(np.float64) @ W.astype(np.float64).T
    assert rel_err(y, dense) <= 0.10


def test_q4_pack_rules(oracle):
    W = np.zeros((1, 64), np.float32)
    # block 0 all zero -> d = 1, every nibble 8; block 1: amax 7 -> d = 1
    W[0, 32:] = [7.0, 0.5, -0.5, 2.5, -2.5, 1.5, 6.5, -6.5] + [0.0] * 8 + [-7.0, 3.0] + [0.0] * 14
    Wq = oracle.pack_matrix_q4(W)
    assert Wq["d"][0, 0] == 1.0 and (Wq["q"][0, 0] == 0x88).all()
    assert Wq["d"][0, 1] == 1.0
    codes = codes_q4(Wq)[0, 1]
    assert list(codes[:8]) == [7, 1, -1, 3, -3, 2, 7, -7]
    assert list(codes[16:18]) == [-7, 3]
    # code j in the low nibble of byte j, code j + 16 in the high nibble
    assert Wq["q"][0, 1, 0] == ((-7 + 8) << 4) | (7 + 8)
    assert blocks4(1).itemsize == 20
    # round trip: every value within half a step d/2 (plus fp32 rounding)
    rows, cols = 16, 512
    Wr = fill_random(rows * cols, 98, 1.0).reshape(rows, cols)
    Wrq = oracle.pack_matrix_q4(Wr)
    back = oracle.unpack_matrix_q4(Wrq, rows, cols)
    step = np.repeat(Wrq["d"].reshape(rows, cols // QK), QK, axis=1)
    assert (np.abs(back - Wr) <= step * (0.5 + 1e-6)).all()
    assert np.abs(codes_q4(Wrq)).max() == 7
    assert rel_err(back, Wr) <= 0.10
