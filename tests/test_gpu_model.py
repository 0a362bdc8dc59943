"""GPU parity of the rest of the block and the token forward: the MLP, the
residual add + RMSNorm, the Q8 embedding lookup, the greedy sampler and
tq_dev_forward_token (libtqattn.so over libtqhip.so), against the oracle
(oracle_mlp_layer, oracle_forward_token: bit-exact with the reference's own
mlp_layer and tq_forward_token, tests/test_oracle_model.py).

Bars:
* the embedding lookup and the sampler: exact;
* the residual add: exact; the residual norm (a parallel sum of squares):
  within 2e-6 relative of the reference's serial one;
* the MLP link by link from its workspace: gate and up within the matmul bar
  (relative L2 1e-5) of the oracle's projections; the quantized hidden rows
  equal the oracle's quantization of silu(gate) * up computed from the GPU's
  own gate/up, except for codes at a rounding boundary that the device expf
  (within an ulp of glibc's) moves by one (under 0.1 % of them); the output
  within the matmul bar of the oracle's down projection of those rows;
* the token forward, per token: the first token (one key, attention output =
  V exactly) within relative L2 1e-4 of the reference's logits; every token,
  against the reference's forward started from the caches the GPU holds at
  that step and against an independent run, within 3e-2; the greedy token
  equal wherever the reference's top two logits are more than 2 % of the
  logit scale apart.  The links are each checked closely elsewhere (the
  attention output is within about 3e-6 of the oracle's from the same
  q/k/v); what reaches the logits is their amplification by quantization:
  a 3e-6 difference in the attention rows moves about one of the 4096 codes
  quantized for wo per token, which moves the layer output by about 3e-4,
  enough to move a few percent of the MLP's hidden codes, and the logits by
  up to about 1e-2 at hidden 4096 with these random weights.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle.binding import BLOCK_Q8, QK, Model, blocks
from tests.golden.gen import normal

pytestmark = pytest.mark.gpu


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


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    return float(np.sqrt(((a - b) ** 2).sum() / max((b * b).sum(), 1e-300)))


def tiled(nat, Wq, rows, cols):
    """block_q8 (or block_q4) rows -> a tiled matrix on the device."""
    lib = nat.load()
    src = dev(nat, Wq)
    q4 = Wq.dtype.itemsize == 20
    b = nat.DeviceBuffer((lib.tq_hip_q4_matrix_bytes if q4 else lib.tq_hip_q8_matrix_bytes)(rows, cols))
    nat.check((lib.tq_hip_q4_pack if q4 else lib.tq_hip_q8_pack)(b.ptr, src.ptr, rows, cols, None), "pack")
    sync(nat)
    return b


@pytest.mark.parametrize("hidden,inter,n,skew", [(256, 640, 1, 0), (256, 640, 2, 0), (128, 320, 3, 0),
                                                 (512, 1024, 20, 0), (256, 640, 1, 4), (128, 320, 3, 4),
                                                 (512, 1024, 20, 4)])
def test_mlp_layer(nat, oracle, hidden, inter, n, skew, monkeypatch):
    """skew=4: xn sits 4 bytes past a 16-byte boundary, so its rows are
    quantized by the one-value-per-lane kernel before the matmuls.  The
    quantized rows are read back from the workspace as block_q8 rows, so the
    split layout a GEMM would read is switched off here (test_mlp_layer_xs
    checks that it changes no bit of the output)."""
    monkeypatch.setenv("TQ_HIP_GEMM_XS", "0")
    lib = nat.load()
    rng = np.random.default_rng(hidden + n)
    wg = oracle.pack_matrix_q8(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wu = oracle.pack_matrix_q8(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wd = oracle.pack_matrix_q8(rng.standard_normal((hidden, inter)).astype(np.float32) * 0.1)
    G, U, Dn = tiled(nat, wg, inter, hidden), tiled(nat, wu, inter, hidden), tiled(nat, wd, hidden, inter)
    w = nat.MlpWeights(G.ptr, U.ptr, Dn.ptr, hidden, inter)
    wsb = lib.tq_hip_mlp_ws_bytes(C.byref(w), n)
    ws = nat.DeviceBuffer(wsb)
    xn = normal(n * hidden, 7) * 2
    dx, dout = dev(nat, np.concatenate([np.zeros(skew // 4, np.float32), xn])), nat.DeviceBuffer(n * hidden * 4)
    nat.check(lib.tq_hip_mlp_layer_async(C.byref(w), n, dx.ptr + skew, dout.ptr, ws.ptr, wsb, None), "mlp")
    sync(nat)
    out = dout.download((n, hidden), np.float32)
    raw = ws.download((wsb,), np.uint8)
    al = lambda b: (b + 255) & ~255
    gate = raw[:n * inter * 4].view(np.float32)
    up = raw[al(n * inter * 4):al(n * inter * 4) + n * inter * 4].view(np.float32)
    hq = raw[2 * al(n * inter * 4):2 * al(n * inter * 4) + n * inter // QK * 36].view(BLOCK_Q8)
    # gate / up: the matmul bar against the oracle's projections of quantized xn
    for t in range(n):
        xt = xn[t * hidden:(t + 1) * hidden]
        assert rel_l2(gate[t * inter:(t + 1) * inter], oracle.project_q8(wg, inter, hidden, xt)) <= 1e-5
        assert rel_l2(up[t * inter:(t + 1) * inter], oracle.project_q8(wu, inter, hidden, xt)) <= 1e-5
    # the hidden rows: silu(g) * u of the GPU's own gate/up, quantized
    hq_ref = oracle.quantize_row_q8(oracle.silu_mul(gate, up))
    moved = hq["q"].astype(np.int32) - hq_ref["q"].astype(np.int32)
    assert np.abs(moved).max() <= 1 and (moved != 0).mean() < 1e-3
    assert np.allclose(hq["d"], hq_ref["d"], rtol=1e-6, atol=0)
    # down: the matmul bar against the oracle's down projection of the GPU's rows
    nbi = inter // QK
    for t in range(n):
        ref = oracle.matmul_q8(wd, hq[t * nbi:(t + 1) * nbi], hidden, inter, 1)[0]
        assert rel_l2(out[t], ref) <= 1e-5


def test_mlp_layer_split_k_off(nat, oracle, monkeypatch):
    """20 rows take the split-K GEMM (partials in the workspace, summed in
    split order); with it switched off they take the unsplit launches, under
    the same bars."""
    monkeypatch.setenv("TQ_HIP_GEMM_SPLIT", "0")
    test_mlp_layer(nat, oracle, 512, 1024, 20, 0, monkeypatch)


@pytest.mark.parametrize("fmt,n", [("q8", 20), ("q8", 130), ("q4", 20), ("q8", 300)])
def test_mlp_layer_xs(nat, oracle, fmt, n, monkeypatch):
    """The GEMM reads the quantized rows either as block_q8 rows or in the
    split layout (codes apart from scales, conflict-free LDS reads): the same
    codes, scales and products in the same order, so the MLP output is
    bit-identical either way (split-K and unsplit GEMMs, Q8 and Q4)."""
    lib = nat.load()
    hidden, inter = 512, 1024
    rng = np.random.default_rng(n)
    pack = oracle.pack_matrix_q4 if fmt == "q4" else oracle.pack_matrix_q8
    wg = pack(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wu = pack(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wd = pack(rng.standard_normal((hidden, inter)).astype(np.float32) * 0.1)
    q4 = fmt == "q4"
    G, U, Dn = tiled(nat, wg, inter, hidden), tiled(nat, wu, inter, hidden), tiled(nat, wd, hidden, inter)
    w = nat.MlpWeights(G.ptr, U.ptr, Dn.ptr, hidden, inter, nat.FORMAT_Q4 if q4 else nat.FORMAT_Q8)
    wsb = lib.tq_hip_mlp_ws_bytes(C.byref(w), n)
    ws = nat.DeviceBuffer(wsb)
    dx, dout = dev(nat, normal(n * hidden, 9) * 2), nat.DeviceBuffer(n * hidden * 4)
    outs = []
    for xs in ("1", "0"):
        monkeypatch.setenv("TQ_HIP_GEMM_XS", xs)
        nat.check(lib.tq_hip_mlp_layer_async(C.byref(w), n, dx.ptr, dout.ptr, ws.ptr, wsb, None), "mlp")
        sync(nat)
        outs.append(dout.download((n, hidden), np.float32))
    assert outs[0].tobytes() == outs[1].tobytes()


@pytest.mark.parametrize("fmt,hidden,inter,n,split", [("q8", 512, 1024, 130, "0"), ("q8", 512, 1024, 300, "0"),
                                                     ("q4", 512, 1024, 300, "0"), ("q8", 512, 4096, 520, "1")])
def test_mlp_layer_fused(nat, oracle, fmt, hidden, inter, n, split, monkeypatch):
    """An unsplit gate/up GEMM pairs 64 rows of both matrices per tile and
    its epilogue forms the down matmul's input itself: silu_mul of the same
    fp32 gate and up values, quantized as the separate launch does.  The
    hidden rows it leaves in the workspace (the gate rows' space) equal byte
    for byte the separate launch's (TQ_HIP_MLP_FUSED=0), which also proves
    that the fused path ran; the output is bit-identical; and the output of
    the first and last token is within the matmul bar of the oracle's down
    projection of those rows.  Ragged token counts (130, 300, 520), Q8 and
    Q4; split "0" forces the unsplit GEMM at small counts, at 520 tokens over
    4096 rows it is the default plan (the down matmul still splits K)."""
    lib = nat.load()
    monkeypatch.setenv("TQ_HIP_GEMM_SPLIT", split)
    rng = np.random.default_rng(inter + n)
    q4 = fmt == "q4"
    pack = oracle.pack_matrix_q4 if q4 else oracle.pack_matrix_q8
    wg = pack(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wu = pack(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
    wd = pack(rng.standard_normal((hidden, inter)).astype(np.float32) * 0.1)
    G, U, Dn = tiled(nat, wg, inter, hidden), tiled(nat, wu, inter, hidden), tiled(nat, wd, hidden, inter)
    w = nat.MlpWeights(G.ptr, U.ptr, Dn.ptr, hidden, inter, nat.FORMAT_Q4 if q4 else nat.FORMAT_Q8)
    wsb = lib.tq_hip_mlp_ws_bytes(C.byref(w), n)
    ws = nat.DeviceBuffer(wsb)
    dx, dout = dev(nat, normal(n * hidden, 11) * 2), nat.DeviceBuffer(n * hidden * 4)
    al = lambda b: (b + 255) & ~255
    hq_bytes = n * inter + n * (inter // QK) * 4
    outs, hqs = [], []
    for fused in ("1", "0"):
        monkeypatch.setenv("TQ_HIP_MLP_FUSED", fused)
        nat.check(lib.tq_hip_mlp_layer_async(C.byref(w), n, dx.ptr, dout.ptr, ws.ptr, wsb, None), "mlp")
        sync(nat)
        outs.append(dout.download((n, hidden), np.float32))
        raw = ws.download((wsb,), np.uint8)
        off = 0 if fused == "1" else 2 * al(n * inter * 4)
        hqs.append(raw[off:off + hq_bytes].copy())
    assert hqs[0].tobytes() == hqs[1].tobytes()
    assert outs[0].tobytes() == outs[1].tobytes()
    # the split layout back to block_q8 rows: codes of block b, token t at
    # ((2b + half) n + t) 16, scales [b][t] after the n * inter code bytes
    nbi = inter // QK
    codes = hqs[0][:n * inter].view(np.int8).reshape(nbi, 2, n, 16)
    scales = hqs[0][n * inter:].view(np.float32).reshape(nbi, n)
    for t in (0, n - 1):
        rows = np.zeros(nbi, BLOCK_Q8)
        rows["d"] = scales[:, t]
        rows["q"] = codes[:, :, t, :].reshape(nbi, QK)
        mm = oracle.matmul_q4 if q4 else oracle.matmul_q8
        ref = mm(wd, rows, hidden, inter, 1)[0]
        assert rel_l2(outs[0][t], ref) <= 1e-5


def test_add_rmsnorm(nat, oracle):
    lib = nat.load()
    # 1024-thread kernel holding 1, 2, 4 and 8 float4 per thread, and the
    # strided kernel past that
    for n, rows in ((4096, 1), (256, 5), (8192, 2), (14336, 1), (32768, 1), (40000, 2)):
        x = normal(rows * n, n) * 3
        y = normal(rows * n, n + 1)
        w = np.random.default_rng(n).uniform(0.5, 1.5, n).astype(np.float32)
        dx, dy, dw, dxn = dev(nat, x), dev(nat, y), dev(nat, w), nat.DeviceBuffer(x.nbytes)
        nat.check(lib.tq_hip_add_rmsnorm(dx.ptr, dy.ptr, dw.ptr, dxn.ptr, rows, n, 1e-6, None), "add_rmsnorm")
        sync(nat)
        xs = (x + y).astype(np.float32)
        assert dx.download((x.size,), np.float32).tobytes() == xs.tobytes()
        got = dxn.download((x.size,), np.float32)
        ref = oracle.rmsnorm(xs, w, 1e-6)
        # the reference sums the squares serially: its own rounding error grows
        # up to n * 2^-24 relative, halved by the inverse square root; the
        # parallel sum here stays within 1e-6 of the fp64 norm
        assert np.allclose(got, ref, rtol=2e-6 + n * 2.0 ** -25, atol=0)
        x64 = xs.astype(np.float64).reshape(rows, n)
        ref64 = x64 / np.sqrt(1e-6 + (x64 * x64).mean(axis=1, keepdims=True)) * w
        assert np.allclose(got.reshape(rows, n), ref64, rtol=1e-6, atol=0)
        # without y: norm only, x untouched
        nat.check(lib.tq_hip_add_rmsnorm(dx.ptr, None, dw.ptr, dxn.ptr, rows, n, 1e-6, None), "rmsnorm")
        sync(nat)
        assert dx.download((x.size,), np.float32).tobytes() == xs.tobytes()
    # rows not 16-byte aligned take the strided kernel
    n = 4096
    x = normal(n + 1, 5) * 3
    y = normal(n + 1, 6)
    w = np.random.default_rng(1).uniform(0.5, 1.5, n + 1).astype(np.float32)
    dx, dy, dw, dxn = dev(nat, x), dev(nat, y), dev(nat, w), nat.DeviceBuffer(x.nbytes)
    nat.check(lib.tq_hip_add_rmsnorm(dx.ptr + 4, dy.ptr + 4, dw.ptr + 4, dxn.ptr + 4, 1, n, 1e-6, None), "unaligned")
    sync(nat)
    xs = (x[1:] + y[1:]).astype(np.float32)
    assert dx.download((n + 1,), np.float32)[1:].tobytes() == xs.tobytes()
    assert np.allclose(dxn.download((n + 1,), np.float32)[1:], oracle.rmsnorm(xs, w[1:], 1e-6), rtol=2e-6, atol=0)


def test_embed_lookup_and_sampler(nat, oracle):
    lib = nat.load()
    from tailorquantkernel_amd import native
    rng = np.random.default_rng(4)
    vocab, hidden = 1000, 2080
    E = oracle.pack_matrix_q8(rng.standard_normal((vocab, hidden)).astype(np.float32))
    dE = tiled(nat, E, vocab, hidden)
    out = nat.DeviceBuffer(hidden * 4)
    for tok in (0, 1, 517, vocab - 1):
        nat.check(lib.tq_hip_embed_lookup_q8(dE.ptr, vocab, hidden, tok, out.ptr, None), "embed")
        sync(nat)
        exp = np.zeros(hidden, np.float32)
        assert oracle.lib.oracle_embed_lookup_q8(E.ctypes.data, vocab, hidden, tok, exp.ctypes.data) == 0
        assert out.download((hidden,), np.float32).tobytes() == exp.tobytes()
    assert lib.tq_hip_embed_lookup_q8(dE.ptr, vocab, hidden, vocab, out.ptr, None) == native.EINVAL
    assert lib.tq_hip_embed_lookup_q8(dE.ptr, vocab, hidden, -1, out.ptr, None) == native.EINVAL
    # greedy sampler: exact, including ties, NaN and -inf
    cases = [normal(128256, 3), np.array([0.5, 2.0, 2.0, -1.0], np.float32), np.array([np.nan, 5.0], np.float32),
             np.array([1.0, np.nan, 3.0], np.float32), np.full(300, -np.inf, np.float32)]
    big = normal(50000, 9)
    big[[100, 30000, 49999]] = 7.5
    cases.append(big)
    # ties spread over threads and batches; +inf twice; odd lengths (scalar loads)
    tie = normal(128256, 10)
    tie[[70000, 5, 128000]] = 9.0
    cases.append(tie)
    inf2 = normal(4000, 11)
    inf2[[3001, 17]] = np.inf
    cases.append(inf2)
    odd = normal(1027, 12)
    odd[[1026, 1000]] = 6.0
    cases += [odd, np.array([-3.0], np.float32), np.array([1.0, 2.0, np.nan], np.float32),
              np.array([np.nan] * 5 + [1.0], np.float32), np.array([-np.inf, np.nan, -np.inf, -1.0], np.float32)]
    dt = nat.DeviceBuffer(4)
    for lg in cases:
        d = dev(nat, lg)
        nat.check(lib.tq_hip_sample_greedy(d.ptr, lg.size, dt.ptr, None), "sample")
        sync(nat)
        assert int(dt.download((1,), np.int32)[0]) == oracle.lib.oracle_sample_greedy(lg.ctypes.data, lg.size)
    assert lib.tq_hip_sample_greedy(dt.ptr, 0, dt.ptr, None) == native.EINVAL


class DeviceModel:
    """A Model's weights on the device and the tq_dev_model that points at them."""

    def __init__(self, nat, m: Model):
        from tailorquantkernel_amd import attn
        self.bufs = []

        def mat(a, r, c):
            b = tiled(nat, a, r, c)
            self.bufs.append(b)
            return b.ptr

        def vec(a):
            b = dev(nat, a)
            self.bufs.append(b)
            return b.ptr

        hd, qd, kd = m.hd, m.nq * m.hd, m.nkv * m.hd
        layers = (attn.DevLayerWeights * m.n_layers)()
        for i, L in enumerate(m.layers):
            layers[i].input_norm = vec(L["input_norm"])
            layers[i].post_norm = vec(L["post_norm"])
            layers[i].attn = nat.AttnWeights(mat(L["wq"], qd, m.hidden), mat(L["wk"], kd, m.hidden),
                                             mat(L["wv"], kd, m.hidden), mat(L["wo"], m.hidden, qd),
                                             vec(L["q_norm"]), vec(L["k_norm"]), m.hidden, m.eps, m.format)
            layers[i].mlp = nat.MlpWeights(mat(L["wgate"], m.inter, m.hidden), mat(L["wup"], m.inter, m.hidden),
                                           mat(L["wdown"], m.hidden, m.inter), m.hidden, m.inter, m.format)
        self.layers = layers
        cfg = attn.AttnConfig(m.nq, m.nkv, hd, m.hidden, m.theta, m.eps)
        self.model = attn.DevModel(cfg, m.n_layers, m.inter, m.vocab, mat(m.embed, m.vocab, m.hidden),
                                   vec(m.final_norm), layers, m.embed_format)


@pytest.mark.parametrize("shape", [(2, 4, 2, 32, 128, 256, 300), (3, 8, 2, 64, 256, 512, 1000),
                                   (1, 32, 8, 128, 4096, 1024, 512)])
def test_forward_tokens(nat, oracle, shape):
    from tailorquantkernel_amd import attn
    L = attn.load()
    m = Model(oracle, *shape, seed=shape[0] + 10)
    dm = DeviceModel(nat, m)
    tokens = [3, 77 % m.vocab, 12, 3, 96 % m.vocab, 0, 255 % m.vocab, 11]
    T = 16
    ref, _, _ = oracle.forward(m, tokens, T)
    ctx = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(dm.model), T) == 0
    caches = C.cast(ctx.caches, C.POINTER(attn.KVCache))
    st, keep = m.struct()
    nb = m.hd // QK
    errs, errs_state = [], []
    for i, t in enumerate(tokens):
        # the reference's forward for this token from the caches the GPU holds now
        kc = [blocks(m.nkv * T * nb) for _ in range(m.n_layers)]
        vc = [blocks(m.nkv * T * nb) for _ in range(m.n_layers)]
        for l in range(m.n_layers):
            assert L.tq_kv_cache_download(C.byref(caches[l]), kc[l].ctypes.data, vc[l].ctypes.data) == 0
        karr = (C.c_void_p * m.n_layers)(*[c.ctypes.data for c in kc])
        varr = (C.c_void_p * m.n_layers)(*[c.ctypes.data for c in vc])
        ref_state = np.zeros(m.vocab, np.float32)
        assert oracle.lib.oracle_forward_token(C.byref(st), karr, varr, T, i, t, ref_state.ctypes.data) == 0
        assert L.tq_dev_forward_token(C.byref(ctx), t) == 0
        got = np.zeros(m.vocab, np.float32)
        assert L.tq_dev_logits(C.byref(ctx), got.ctypes.data) == 0
        errs.append(rel_l2(got, ref[i]))
        errs_state.append(rel_l2(got, ref_state))
        top = np.sort(ref[i])[-2:]
        if top[1] - top[0] > 2e-2 * np.abs(ref[i]).max():
            assert L.tq_dev_sample_greedy(C.byref(ctx)) == int(np.argmax(ref[i])), (i, t)
    print(f"logits relative L2 per token, from the GPU's caches: {['%.1e' % e for e in errs_state]}; "
          f"independent run: {['%.1e' % e for e in errs]}")
    assert errs[0] <= 1e-4
    assert max(errs_state) <= 3e-2 and max(errs) <= 3e-2
    # the reference's checks (tools/test_model.c:1488-1507): a token outside the
    # vocabulary leaves pos as it was, then a full context
    pos = ctx.pos
    assert L.tq_dev_forward_token(C.byref(ctx), m.vocab) == -1
    assert L.tq_dev_forward_token(C.byref(ctx), -1) == -1
    assert ctx.pos == pos
    ctx2 = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx2), C.byref(dm.model), 1) == 0
    assert L.tq_dev_forward_token(C.byref(ctx2), 1) == 0
    assert L.tq_dev_forward_token(C.byref(ctx2), 1) == -1
    L.tq_dev_ctx_free(C.byref(ctx2))
    L.tq_dev_ctx_free(C.byref(ctx))
    L.tq_dev_ctx_free(C.byref(ctx))   # idempotent


@pytest.mark.parametrize("shape", [(3, 8, 2, 64, 256, 512, 1000), (2, 32, 8, 128, 4096, 1024, 512)])
def test_forward_layers_state_fed(nat, oracle, shape):
    """Every layer of the token forward, fed the device's own input: the op
    sequence of tq_dev_forward_token (host/tq_model.c; model/context.c:83-100)
    run launch by launch through the C-ABI, and after each attention layer and
    each MLP the oracle's attention_layer / mlp_layer (bit-exact with the
    reference's, tests/test_oracle_model.py) run on the same input, the
    attention from the cache the device holds at that step.  Per layer output
    element, |device - oracle| / rms(oracle row): median <= 1e-4 and max <=
    1e-2 over all layers and tokens (the reference's own forward check is
    1e-5 on its logits, tools/test_model.c:1538-1578; here a quantization code
    at a rounding boundary may move, which the max allows and the median does
    not).  The appended K/V rows: codes within one of the oracle's, at most
    1 % moved, scales within 1e-5.  The end-to-end logits bar (3e-2) stays in
    test_forward_tokens; this one sees a regression of any single layer."""
    lib = nat.load()
    m = Model(oracle, *shape, seed=shape[0] + 70)
    dm = DeviceModel(nat, m)
    T = 8
    nb = m.hd // QK
    kvs = [nat.PagedKV.single(m.nq, m.nkv, m.hd, T) for _ in range(m.n_layers)]
    s = kvs[0].stream
    wsb = max(lib.tq_hip_attention_layer_ws_bytes(kvs[0].h, C.byref(dm.layers[0].attn), 1),
              lib.tq_hip_mlp_ws_bytes(C.byref(dm.layers[0].mlp), 1))
    ws = nat.DeviceBuffer(wsb)
    x, xn, ya, ym = (nat.DeviceBuffer(m.hidden * 4) for _ in range(4))
    errs = []
    moved_codes, n_codes = 0, 0

    def err(dev_out, ref):
        ref = np.asarray(ref, np.float64)
        e = np.abs(np.asarray(dev_out, np.float64) - ref) / max(np.sqrt((ref * ref).mean()), 1e-30)
        errs.append(e)

    for pos, tok in enumerate([3, 77 % m.vocab, 12, 3, 96 % m.vocab, 0]):
        c, sn = oracle.rope_table(m.hd, pos, m.theta)
        dpos, dc, ds = dev(nat, np.array([pos], np.int32)), dev(nat, c), dev(nat, sn)
        nat.check(lib.tq_hip_embed_lookup_q8(dm.model.embed, m.vocab, m.hidden, tok, x.ptr, s), "embed")
        pending = None
        for l, L in enumerate(m.layers):
            DL = dm.layers[l]
            nat.check(lib.tq_hip_add_rmsnorm(x.ptr, pending, DL.input_norm, xn.ptr, 1, m.hidden, m.eps, s), "norm")
            sync(nat)
            xin = xn.download((m.hidden,), np.float32)
            kc, vc = (a.reshape(-1).copy() for a in kvs[l].read(0, 0, T))
            nat.check(lib.tq_hip_attention_layer_async(kvs[l].h, C.byref(DL.attn), 1, None, dpos.ptr, pos, xn.ptr,
                                                       dc.ptr, ds.ptr, ya.ptr, ws.ptr, wsb, s), "attention_layer")
            sync(nat)
            rc, ref = oracle.attention_layer((L["wq"], L["wk"], L["wv"], L["wo"], L["q_norm"], L["k_norm"]),
                                             m.nq, m.nkv, m.hd, m.hidden, m.theta, m.eps, kc, vc, T, pos, xin)
            assert rc == 0
            err(ya.download((m.hidden,), np.float32), ref)
            gk, gv = kvs[l].read(0, 0, T)
            for g, r in ((gk, kc), (gv, vc)):
                g, r = g.reshape(m.nkv, T, nb)[:, pos], r.reshape(m.nkv, T, nb)[:, pos]
                d = g["q"].astype(np.int32) - r["q"].astype(np.int32)
                assert np.abs(d).max() <= 1, f"layer {l} pos {pos}: a K/V code moved by more than one"
                moved_codes += int((d != 0).sum())
                n_codes += d.size
                assert np.allclose(g["d"], r["d"], rtol=1e-5, atol=0), f"layer {l} pos {pos}: K/V scales"
            nat.check(lib.tq_hip_add_rmsnorm(x.ptr, ya.ptr, DL.post_norm, xn.ptr, 1, m.hidden, m.eps, s), "norm")
            sync(nat)
            xin = xn.download((m.hidden,), np.float32)
            nat.check(lib.tq_hip_mlp_layer_async(C.byref(DL.mlp), 1, xn.ptr, ym.ptr, ws.ptr, wsb, s), "mlp")
            sync(nat)
            err(ym.download((m.hidden,), np.float32),
                oracle.mlp_layer(L["wgate"], L["wup"], L["wdown"], m.hidden, m.inter, xin))
            pending = ym.ptr
    e = np.concatenate(errs)
    print(f"per-layer outputs from the device's inputs: median {np.median(e):.1e}, max {e.max():.1e} of the row "
          f"RMS; K/V codes moved {moved_codes} of {n_codes}")
    assert np.median(e) <= 1e-4 and e.max() <= 1e-2
    assert moved_codes <= 0.01 * n_codes
    for kv in kvs:
        kv.close()


@pytest.mark.parametrize("shape,n,chunks", [((2, 4, 2, 32, 128, 256, 300), 40, (16, 24)),
                                            ((3, 8, 2, 64, 256, 512, 1000), 40, (7, 33)),
                                            ((1, 32, 8, 128, 4096, 1024, 512), 64, (64,))])
def test_forward_batch_and_prefill(nat, oracle, shape, n, chunks):
    """tq_dev_forward_batch over chunks and tq_dev_prefill (model/context.c:174-229)
    against the reference's tq_prefill (its logits equal its own token loop's
    bit for bit; the oracle's token loop where the reference is not built):
    last-token logits within relative L2 3e-2 (the bar of the token forward:
    a moved code is amplified through the layers), and within the same bar of
    the oracle's forward of the last token from the caches the GPU filled.
    Layer 0's K/V codes move by at most one, in under 1 % of the codes."""
    from tailorquantkernel_amd import attn
    from oracle.binding import Ref
    L = attn.load()
    m = Model(oracle, *shape, seed=shape[0] + 20)
    dm = DeviceModel(nat, m)
    toks = np.random.default_rng(n + shape[4]).integers(0, m.vocab, n).astype(np.int32)
    T = n + 8
    nb = m.hd // QK
    if Ref.available():
        ref_last, rk, rv = Ref().prefill(m, toks, T)
    else:
        lg, rk, rv = oracle.forward(m, toks, T)
        ref_last = lg[-1]
    ctx = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(dm.model), T) == 0
    ws = attn.DevBatchWs()
    assert L.tq_dev_batch_ws_init(C.byref(ws), C.byref(dm.model), max(chunks)) == 0
    # the reference's checks, before any launch
    assert L.tq_dev_forward_batch(C.byref(ctx), C.byref(ws), toks.ctypes.data, max(chunks) + 1, 1) == -1
    assert L.tq_dev_forward_batch(C.byref(ctx), C.byref(ws), toks.ctypes.data, 0, 1) == -1
    bad = toks.copy()
    bad[1] = m.vocab
    assert L.tq_dev_forward_batch(C.byref(ctx), C.byref(ws), bad.ctypes.data, 2, 1) == -1
    assert ctx.pos == 0
    i = 0
    for c in chunks:
        assert L.tq_dev_forward_batch(C.byref(ctx), C.byref(ws), toks[i:].ctypes.data, c, int(i + c == n)) == 0
        i += c
    assert ctx.pos == n
    got = np.zeros(m.vocab, np.float32)
    assert L.tq_dev_logits(C.byref(ctx), got.ctypes.data) == 0
    caches = C.cast(ctx.caches, C.POINTER(attn.KVCache))
    kc = [blocks(m.nkv * T * nb) for _ in range(m.n_layers)]
    vc = [blocks(m.nkv * T * nb) for _ in range(m.n_layers)]
    for l in range(m.n_layers):
        assert L.tq_kv_cache_download(C.byref(caches[l]), kc[l].ctypes.data, vc[l].ctypes.data) == 0
    # the oracle's forward of the last token from the GPU's caches
    st, keep = m.struct()
    karr = (C.c_void_p * m.n_layers)(*[c.ctypes.data for c in kc])
    varr = (C.c_void_p * m.n_layers)(*[c.ctypes.data for c in vc])
    from_state = np.zeros(m.vocab, np.float32)
    assert oracle.lib.oracle_forward_token(C.byref(st), karr, varr, T, n - 1, int(toks[-1]),
                                           from_state.ctypes.data) == 0
    e_ref, e_state = rel_l2(got, ref_last), rel_l2(got, from_state)
    # layer 0's codes of the n positions, against the reference's
    filled = lambda c: c.reshape(m.nkv, T, nb)[:, :n]
    moved = [(filled(a)["q"].astype(np.int32) - filled(b)["q"].astype(np.int32)) for a, b in
             ((kc[0], rk[0]), (vc[0], rv[0]))]
    frac = max(float((d != 0).mean()) for d in moved)
    print(f"prefill last-token logits relative L2: {e_ref:.1e} (reference), {e_state:.1e} (from the GPU's caches); "
          f"layer-0 codes moved: {frac:.1e}")
    assert e_ref <= 3e-2 and e_state <= 3e-2
    assert max(int(np.abs(d).max()) for d in moved) <= 1 and frac < 1e-2
    # a full context, then tq_dev_prefill in one call on a fresh context
    assert L.tq_dev_forward_batch(C.byref(ctx), C.byref(ws), toks.ctypes.data, 9, 1) == -1
    L.tq_dev_batch_ws_free(C.byref(ws))
    L.tq_dev_batch_ws_free(C.byref(ws))   # idempotent
    ctx2 = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx2), C.byref(dm.model), T) == 0
    assert L.tq_dev_prefill(C.byref(ctx2), toks.ctypes.data, n) == 0
    assert ctx2.pos == n
    got2 = np.zeros(m.vocab, np.float32)
    assert L.tq_dev_logits(C.byref(ctx2), got2.ctypes.data) == 0
    assert rel_l2(got2, ref_last) <= 3e-2
    assert L.tq_dev_prefill(C.byref(ctx2), toks.ctypes.data, T - n + 1) == -1
    # the next token after the prompt, through the token forward
    assert L.tq_dev_forward_token(C.byref(ctx2), int(toks[0])) == 0
    L.tq_dev_ctx_free(C.byref(ctx2))
    L.tq_dev_ctx_free(C.byref(ctx))


@pytest.mark.parametrize("shape,fmt,embed_fmt", [((2, 4, 2, 32, 128, 256, 300), "q4", "q4"),
                                                 ((1, 32, 8, 128, 4096, 1024, 512), "q4", "q8"),
                                                 ((2, 8, 2, 64, 256, 512, 1000), "q8", "q4")])
def test_forward_q4(nat, oracle, shape, fmt, embed_fmt):
    """A model with Q4 layer matrices and/or a Q4 embedding (each tq_matrix's
    format, kernel/q4_scalar.c, model/embedding.c:20-27) through
    tq_dev_forward_token and tq_dev_prefill: the token forward against the
    oracle's (bit-exact with the reference's scalar build) with the bars of
    test_forward_tokens; the prefill's last logits against the token loop's."""
    from tailorquantkernel_amd import attn
    L = attn.load()
    m = Model(oracle, *shape, seed=shape[0] + 40, fmt=fmt, embed_fmt=embed_fmt)
    dm = DeviceModel(nat, m)
    tokens = [3, 77 % m.vocab, 12, 3, 96 % m.vocab, 0]
    T = 8
    ref, _, _ = oracle.forward(m, tokens, T)
    ctx = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(dm.model), T) == 0
    errs = []
    for i, t in enumerate(tokens):
        assert L.tq_dev_forward_token(C.byref(ctx), t) == 0
        got = np.zeros(m.vocab, np.float32)
        assert L.tq_dev_logits(C.byref(ctx), got.ctypes.data) == 0
        errs.append(rel_l2(got, ref[i]))
    print(f"{fmt}/{embed_fmt} logits relative L2 per token: {['%.1e' % e for e in errs]}")
    assert errs[0] <= 1e-4 and max(errs) <= 3e-2
    L.tq_dev_ctx_free(C.byref(ctx))
    ctx2 = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx2), C.byref(dm.model), T) == 0
    toks = np.array(tokens, np.int32)
    assert L.tq_dev_prefill(C.byref(ctx2), toks.ctypes.data, len(tokens)) == 0
    got = np.zeros(m.vocab, np.float32)
    assert L.tq_dev_logits(C.byref(ctx2), got.ctypes.data) == 0
    assert rel_l2(got, ref[-1]) <= 3e-2
    L.tq_dev_ctx_free(C.byref(ctx2))
    # a format outside Q8/Q4 is refused
    bad = attn.DevModel(dm.model.attn, m.n_layers, m.inter, m.vocab, dm.model.embed, dm.model.final_norm,
                        dm.layers, 7)
    ctx3 = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx3), C.byref(bad), T) == -1
