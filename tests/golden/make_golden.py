"""Write the golden vectors of the Q8 attention path from the compiled reference.

Run in a container that has the reference sources, after ``make -C oracle ref``:

    python tests/golden/make_golden.py

It loads oracle/_ref/libtqref_scalar.so (the reference built from its own
sources without TQ_HAVE_AVX2, i.e. its scalar kernels) and records, for inputs
rebuilt from seeds by tests/golden/gen.py, the reference's outputs:

* quantize_row_q8 codes and scales (kernel/quant_x.c:12-33), random and
  hand-built edge rows (zeros, exact ties, tiny, huge, inf/nan);
* rope_table cos/sin (model/rope.c:4-12) for several (head_dim, pos, theta);
* attn_scores_q8_scalar, softmax, attn_accum_q8_scalar (model/attn_q8.c:17-54,
  model/softmax.c:4-23) over g x n x head_dim;
* attention_head_q8 (model/attn_q8.c:78-90), output and q_q8;
* the attention core (RoPE, store_kv, attend_q8) at 8q/2kv/hd64/theta 1e4 over
  256 positions and one step at 32q/8kv/hd128/theta 5e5, pos 4095: the stored
  K/V rows and the attention output.

Output: tests/golden/golden_q8.npz (inputs by seed + checksum, outputs in full).

    python tests/golden/make_golden.py weights

writes tests/golden/golden_matmul_q8.npz instead: the weight side of the
path, on the shapes the reference's own kernel test runs
(tools/test_kernel.c:178-180,187-190) — pack_matrix (packer/packer.c:22-31)
of seeded weights, quantize_row_q8 of seeded activations and
matmul_q8_scalar / matmul_q8_scalar_batch (kernel/q8_scalar.c:15-30); and
the same weights packed as Q4 (packer/packer.c:40-52) with
matmul_q4_scalar / matmul_q4_scalar_batch (kernel/q4_scalar.c:17-32).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.binding import BLOCK_Q8, QK, Ref, blocks, blocks4, f32, ptr  # noqa: E402
from tests.golden.gen import checksum, fill_random  # noqa: E402

OUT = os.path.join(HERE, "golden_q8.npz")

# Edge rows for the quantizer, 32 values each.
def edge_rows() -> np.ndarray:
    rows = []
    rows.append(np.zeros(32, np.float32))                                     # all zero -> d = 0
    r = np.zeros(32, np.float32); r[0] = 127.0                                 # d = 1 exactly
    r[1:9] = [2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5]                    # exact ties -> even
    rows.append(r)
    r = np.full(32, -1.0, np.float32); r[5] = 1.0                              # sign pattern, amax from a negative
    rows.append(r)
    r = np.linspace(-1e-38, 1e-38, 32).astype(np.float32)                      # subnormal-range values
    rows.append(r)
    r = np.linspace(-3e38, 3e38, 32).astype(np.float32)                        # huge values
    rows.append(r)
    r = fill_random(32, 77, 1.0); r[3] = np.inf                                # inf: scale inf, inverse 0
    rows.append(r)
    r = fill_random(32, 78, 1.0); r[7] = np.nan                                # nan: skipped by the max
    rows.append(r)
    r = np.zeros(32, np.float32); r[31] = -1e-3                                # one nonzero
    rows.append(r)
    return np.stack(rows)


def main() -> None:
    ref = Ref(scalar=True)
    L = ref.lib
    data: dict[str, np.ndarray] = {}

    # ---- quantize_row_q8 --------------------------------------------------
    rnd = np.concatenate([fill_random(64 * 128, 1234 + i, 3.0) for i in range(1)])
    edges = edge_rows()
    x = np.concatenate([rnd, edges.reshape(-1)]).astype(np.float32)
    qb = blocks(x.size // QK)
    L.quantize_row_q8(ptr(x), ptr(qb), x.size)
    data["quant_edges"] = edges
    data["quant_x_seed"] = np.array([1234, 64 * 128], np.int64)
    data["quant_x_sum"] = np.array([checksum(x)], np.int64)
    data["quant_d"] = qb["d"].copy()
    data["quant_q"] = qb["q"].copy()

    # ---- rope_table ---------------------------------------------------------
    rope_cases = [(2, 1, 10000.0), (64, 0, 10000.0), (64, 255, 10000.0), (64, 17, 10000.0),
                  (128, 4095, 500000.0), (128, 100, 1000000.0), (128, 32767, 500000.0),
                  (128, 2047, 500000.0), (32, 7, 1000000.0)]
    data["rope_cases"] = np.array(rope_cases, np.float64)
    for i, (hd, pos, th) in enumerate(rope_cases):
        c = np.zeros(int(hd) // 2, np.float32)
        s = np.zeros(int(hd) // 2, np.float32)
        L.rope_table(ptr(c), ptr(s), int(hd), int(pos), float(th))
        data[f"rope_cos_{i}"] = c
        data[f"rope_sin_{i}"] = s

    # ---- scores / softmax / accum kernels -------------------------------
    kcases = []
    for g in (4, 8):
        for n in (1, 129, 300):
            for hd in (64, 128):
                kcases.append((g, n, hd))
    data["kern_cases"] = np.array(kcases, np.int64)
    for i, (g, n, hd) in enumerate(kcases):
        nb = hd // QK
        seed = 900 + 7 * i
        qf = fill_random(g * hd, seed, 1.0)
        kf = fill_random(n * hd, seed + 1, 1.0)
        vf = fill_random(n * hd, seed + 2, 1.0)
        w = fill_random(g * n, seed + 3, 1.0)
        qbk, kbk, vbk = blocks(g * nb), blocks(n * nb), blocks(n * nb)
        L.quantize_row_q8(ptr(qf), ptr(qbk), qf.size)
        L.quantize_row_q8(ptr(kf), ptr(kbk), kf.size)
        L.quantize_row_q8(ptr(vf), ptr(vbk), vf.size)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        sc = np.zeros(g * n, np.float32)
        L.attn_scores_q8_scalar(ptr(qbk), g, ptr(kbk), n, nb, float(scale), ptr(sc), n)
        sm = sc.copy()
        for h in range(g):
            row = np.ascontiguousarray(sm[h * n:(h + 1) * n])
            L.softmax(ptr(row), n)
            sm[h * n:(h + 1) * n] = row
        out = np.zeros(g * hd, np.float32)
        L.attn_accum_q8_scalar(ptr(w), n, g, ptr(vbk), n, nb, ptr(out), hd)
        data[f"kern_in_sum_{i}"] = np.array([checksum(qbk), checksum(kbk), checksum(vbk), checksum(w)], np.int64)
        data[f"kern_scores_{i}"] = sc
        data[f"kern_softmax_{i}"] = sm
        data[f"kern_accum_{i}"] = out

    # ---- attention_head_q8 --------------------------------------------------
    hcases = [(32, 1), (32, 7), (128, 100), (128, 16), (64, 300)]
    data["head_cases"] = np.array(hcases, np.int64)
    for i, (hd, n) in enumerate(hcases):
        nb = hd // QK
        seed = 70 + 11 * i
        q = fill_random(hd, seed, 1.0)
        kf = fill_random(n * hd, seed + 1000, 1.0)
        vf = fill_random(n * hd, seed + 2000, 1.0)
        kbk, vbk = blocks(n * nb), blocks(n * nb)
        L.quantize_row_q8(ptr(kf), ptr(kbk), kf.size)
        L.quantize_row_q8(ptr(vf), ptr(vbk), vf.size)
        qq = blocks(nb)
        sc = np.zeros(n, np.float32)
        out = np.zeros(hd, np.float32)
        L.attention_head_q8(ptr(q), ptr(qq), ptr(kbk), ptr(vbk), n, hd, ptr(sc), ptr(out))
        data[f"head_out_{i}"] = out
        data[f"head_qd_{i}"] = qq["d"].copy()
        data[f"head_qq_{i}"] = qq["q"].copy()

    # ---- attention core, 8q/2kv/hd64/theta 1e4, positions 0..255 ---------
    nq, nkv, hd, T, theta = 8, 2, 64, 256, 10000.0
    nb = hd // QK
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc["d"] = 999.0
    vc["d"] = 999.0
    keep = (0, 1, 100, 255)
    for pos in range(T):
        q = fill_random(nq * hd, 5000 + pos, 1.0)
        k = fill_random(nkv * hd, 6000 + pos, 1.0)
        v = fill_random(nkv * hd, 7000 + pos, 1.0)
        sc = np.zeros(nq * T, np.float32)
        out = np.zeros(nq * hd, np.float32)
        rc = L.tqref_attention_qkv(nq, nkv, hd, T, theta, ptr(kc), ptr(vc), pos, ptr(q), ptr(k),
                                   ptr(v), ptr(sc), ptr(out))
        assert rc == 0
        if pos in keep:
            data[f"core1_out_{pos}"] = out
    data["core1_keep"] = np.array(keep, np.int64)
    data["core1_kc"] = kc.view(np.uint8).reshape(-1).copy()
    data["core1_vc"] = vc.view(np.uint8).reshape(-1).copy()

    # ---- attention core, 32q/8kv/hd128/theta 5e5, one step at pos 4095 ----
    nq, nkv, hd, T, theta = 32, 8, 128, 4096, 500000.0
    nb = hd // QK
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    pos = T - 1
    q = fill_random(nq * hd, 8100, 1.0)
    k = fill_random(nkv * hd, 8200, 1.0)
    v = fill_random(nkv * hd, 8300, 1.0)
    sc = np.zeros(nq * T, np.float32)
    out = np.zeros(nq * hd, np.float32)
    rc = L.tqref_attention_qkv(nq, nkv, hd, T, theta, ptr(kc), ptr(vc), pos, ptr(q), ptr(k),
                               ptr(v), ptr(sc), ptr(out))
    assert rc == 0
    rows_k = np.stack([kc[(h * T + pos) * nb:(h * T + pos + 1) * nb] for h in range(nkv)])
    rows_v = np.stack([vc[(h * T + pos) * nb:(h * T + pos + 1) * nb] for h in range(nkv)])
    data["core2_k_rows"] = rows_k.view(np.uint8).reshape(-1).copy()
    data["core2_v_rows"] = rows_v.view(np.uint8).reshape(-1).copy()
    data["core2_out"] = out

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(data)} arrays)")


WEIGHTS_OUT = os.path.join(HERE, "golden_matmul_q8.npz")


def weights() -> None:
    ref = Ref(scalar=True)
    L = ref.lib
    data: dict[str, np.ndarray] = {}
    # (rows, cols, n_tok, x kind): the reference test's shapes (random x),
    # its constant-x and zero-x cases, and two token batches.
    cases = [(256, 512, 1, 0), (7, 64, 1, 0), (10, 32, 1, 0), (1027, 96, 1, 0),
             (1024, 1024, 1, 0), (256, 512, 1, 1), (256, 512, 1, 2), (64, 256, 5, 0),
             (96, 160, 9, 0)]
    data["cases"] = np.array(cases, np.int64)
    for i, (rows, cols, n_tok, kind) in enumerate(cases):
        nb = cols // QK
        W = fill_random(rows * cols, 3000 + 17 * i, 1.0)
        if kind == 0:
            x = fill_random(n_tok * cols, 4000 + 17 * i, 1.0)
        elif kind == 1:
            x = np.ones(n_tok * cols, np.float32)
        else:
            x = np.zeros(n_tok * cols, np.float32)
        Wq = blocks(rows * nb)
        assert L.pack_matrix(ptr(W), rows, cols, ptr(Wq), b"8") == 0
        xq = blocks(n_tok * nb)
        for t in range(n_tok):
            xt = np.ascontiguousarray(x[t * cols:(t + 1) * cols])
            xb = blocks(nb)
            L.quantize_row_q8(ptr(xt), ptr(xb), cols)
            xq[t * nb:(t + 1) * nb] = xb
        y = np.zeros(n_tok * rows, np.float32)
        if n_tok == 1:
            L.matmul_q8_scalar(ptr(Wq), ptr(xq), ptr(y), rows, cols)
        else:
            L.matmul_q8_scalar_batch(ptr(Wq), ptr(xq), ptr(y), rows, cols, n_tok)
        data[f"in_sum_{i}"] = np.array([checksum(W), checksum(x)], np.int64)
        data[f"packed_sum_{i}"] = np.array([checksum(Wq), checksum(xq)], np.int64)
        data[f"y_{i}"] = y
        # the same weights as Q4 (pack_matrix '4', matmul_q4_scalar)
        W4 = blocks4(rows * nb)
        assert L.pack_matrix(ptr(W), rows, cols, ptr(W4), b"4") == 0
        y4 = np.zeros(n_tok * rows, np.float32)
        if n_tok == 1:
            L.matmul_q4_scalar(ptr(W4), ptr(xq), ptr(y4), rows, cols)
        else:
            L.matmul_q4_scalar_batch(ptr(W4), ptr(xq), ptr(y4), rows, cols, n_tok)
        data[f"packed4_sum_{i}"] = np.array([checksum(W4)], np.int64)
        data[f"y4_{i}"] = y4
    np.savez_compressed(WEIGHTS_OUT, **data)
    print(f"wrote {WEIGHTS_OUT} ({os.path.getsize(WEIGHTS_OUT)} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    if sys.argv[1:] == ["weights"]:
        weights()
    else:
        main()
