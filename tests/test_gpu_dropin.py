"""The drop-in, run as the reference's own code.

oracle/_ref/libtqref_dropin*.so is the reference compiled from its own
sources with the three edits the MI355X library asks of it applied at build
time (oracle/dropin_patch.sh: the TQ_KV_Q8_DEVICE cache type and handle in
model_ops.h, the routing in attention_layer.c, the device-model branch of
tq_forward_token in context.c), linked against libtqattn.so.  Each test runs
one of the reference's entry points twice in that same library — once on
its host TQ_KV_Q8 cache, once on a TQ_KV_Q8_DEVICE cache — and compares:

* the caches bit for bit (the projections, norms and RoPE tables are the same
  host code on both sides, so the rows handed to store_kv are identical);
* attention_layer outputs: the per-token relative L2 error has median <= 1e-4
  and max <= 1e-2 (the device attention agrees with attend_q8 within 1e-4 +
  1e-3|ref|; a last-bit difference can move one code of the quantized
  attention row before the output projection);
* attention_layer_batch: its attention rows (before the output projection)
  within 1e-4 + 1e-3|ref|, its outputs at median <= 1e-3, max <= 1e-2;
* tq_forward_token / tq_prefill logits within relative L2 3e-2 per token, the
  first token within 1e-4, and the greedy token equal where the top two
  logits are more than 2 % of the scale apart; after tq_prefill, layer 0's
  cache rows bit for bit and deeper layers' within relative L2 1e-2.

"fused" is the primary route (tq_attention_core in attention_layer, returning
its code); "route" builds only the two routing points (store_kv /
attend_all_heads), which abort on a device error.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import QK, Model, Ref, blocks
from tests.golden.gen import normal

pytestmark = pytest.mark.gpu


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    return float(np.sqrt(((a - b) ** 2).sum() / max((b * b).sum(), 1e-300)))


@pytest.fixture(scope="module")
def nat():
    from tailorquantkernel_amd import native
    native.init(0)
    assert native.device_arch().startswith("gfx950")
    return native


def dropin(variant):
    if not Ref.available(dropin=variant):
        pytest.fail(f"oracle/_ref/{Ref._name(True, variant)} is missing: build it with `make -C oracle dropin`")
    return Ref(dropin=variant)


def layer_weights(oracle, nq, nkv, hd, hidden, seed):
    rng = np.random.default_rng(seed)

    def mat(rows, cols):
        return oracle.pack_matrix_q8(rng.standard_normal((rows, cols)).astype(np.float32) * 0.05)

    return (mat(nq * hd, hidden), mat(nkv * hd, hidden), mat(nkv * hd, hidden), mat(hidden, nq * hd),
            rng.uniform(0.5, 1.5, hd).astype(np.float32), rng.uniform(0.5, 1.5, hd).astype(np.float32))


def run_steps(ref, kv_type, w, shape, T, pos0, n, xn, kc, vc):
    from oracle.binding import ptr
    nq, nkv, hd, hidden, theta, eps = shape
    ref.set_kv_type(kv_type)
    out = np.zeros((n, hidden), np.float32)
    scores = np.zeros(nq * T, np.float32)
    rc = ref.lib.tqref_layer_steps(nq, nkv, hd, hidden, theta, eps, *[ptr(a) for a in w], ptr(kc), ptr(vc), T,
                                   pos0, n, ptr(xn), ptr(scores), ptr(out))
    return rc, out


def run_batch(ref, kv_type, w, shape, T, pos0, n, xn, kc, vc, attn=None):
    """attention_layer_batch; with `attn` ([n][nq*hd]) its attention rows
    before the output projection are copied there."""
    from oracle.binding import ptr
    nq, nkv, hd, hidden, theta, eps = shape
    ref.set_kv_type(kv_type)
    out = np.zeros((n, hidden), np.float32)
    scores = np.zeros(nq * T, np.float32)
    ref.lib.tqref_capture_attn(ptr(attn) if attn is not None else None)
    try:
        rc = ref.lib.tqref_layer_batch_run(nq, nkv, hd, hidden, theta, eps, *[ptr(a) for a in w], ptr(kc), ptr(vc),
                                           T, pos0, n, ptr(xn), ptr(scores), ptr(out))
    finally:
        ref.lib.tqref_capture_attn(None)
    return rc, out


def check_outputs(dev_out, host_out, what, median=1e-4):
    errs = [rel_l2(a, b) for a, b in zip(dev_out, host_out)]
    assert max(errs) <= 1e-2, f"{what}: worst token relative L2 {max(errs):.3e}"
    assert np.median(errs) <= median, f"{what}: median relative L2 {np.median(errs):.3e}"


def assert_close(gpu, ref, what):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    bad = err > 1e-4 + 1e-3 * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside 1e-4 + 1e-3|ref|, max {err.max():.3e}"


SHAPES = [(8, 2, 64, 256, 1e4, 1e-6), (32, 8, 128, 1024, 5e5, 1e-6), (4, 4, 128, 512, 1e6, 1e-5)]


@pytest.mark.parametrize("variant", ["fused", "route"])
@pytest.mark.parametrize("shape", SHAPES)
def test_attention_layer(nat, oracle, variant, shape):
    """The reference's attention_layer over 40 positions on one cache, host
    TQ_KV_Q8 against TQ_KV_Q8_DEVICE."""
    ref = dropin(variant)
    nq, nkv, hd, hidden = shape[:4]
    T, n = 48, 40
    w = layer_weights(oracle, nq, nkv, hd, hidden, 3)
    xn = normal(n * hidden, 11)
    kc_h, vc_h = blocks(nkv * T * (hd // QK)), blocks(nkv * T * (hd // QK))
    kc_d, vc_d = kc_h.copy(), vc_h.copy()
    rc, out_h = run_steps(ref, Ref.TQ_KV_Q8, w, shape, T, 0, n, xn, kc_h, vc_h)
    assert rc == 0
    rc, out_d = run_steps(ref, Ref.TQ_KV_Q8_DEVICE, w, shape, T, 0, n, xn, kc_d, vc_d)
    assert rc == 0
    assert kc_d.tobytes() == kc_h.tobytes() and vc_d.tobytes() == vc_h.tobytes(), "caches differ"
    check_outputs(out_d, out_h, f"attention_layer {variant} {shape}")
    # a position outside [0, max_tokens) is -1 before anything is written
    before = kc_d.tobytes()
    rc, _ = run_steps(ref, Ref.TQ_KV_Q8_DEVICE, w, shape, T, T, 1, xn[:hidden], kc_d, vc_d)
    assert rc == -1 and kc_d.tobytes() == before


@pytest.mark.parametrize("variant", ["fused", "route"])
@pytest.mark.parametrize("chunks", [[(0, 40), (40, 8)], [(0, 1), (1, 33), (34, 5)]])
def test_attention_layer_batch(nat, oracle, variant, chunks):
    """The reference's attention_layer_batch in chunks (the fused route is one
    tq_attention_core_batch per chunk: the MFMA prefill from 32 tokens on)."""
    ref = dropin(variant)
    shape = (32, 8, 128, 1024, 5e5, 1e-6)
    nq, nkv, hd, hidden = shape[:4]
    T = 48
    w = layer_weights(oracle, nq, nkv, hd, hidden, 5)
    kc_h, vc_h = blocks(nkv * T * (hd // QK)), blocks(nkv * T * (hd // QK))
    kc_d, vc_d = kc_h.copy(), vc_h.copy()
    for pos0, n in chunks:
        xn = normal(n * hidden, 100 + pos0)
        attn_h, attn_d = np.zeros((n, nq * hd), np.float32), np.zeros((n, nq * hd), np.float32)
        rc, out_h = run_batch(ref, Ref.TQ_KV_Q8, w, shape, T, pos0, n, xn, kc_h, vc_h, attn_h)
        assert rc == 0
        rc, out_d = run_batch(ref, Ref.TQ_KV_Q8_DEVICE, w, shape, T, pos0, n, xn, kc_d, vc_d, attn_d)
        assert rc == 0
        assert kc_d.tobytes() == kc_h.tobytes() and vc_d.tobytes() == vc_h.tobytes(), f"caches after {pos0}+{n}"
        # the attention rows themselves to the attention bar; the outputs
        # after the output projection carry the odd moved activation code
        assert_close(attn_d, attn_h, f"attention rows {variant} {pos0}+{n}")
        check_outputs(out_d, out_h, f"attention_layer_batch {variant} {pos0}+{n}", median=1e-3)
    # n past the cache is -1 before any launch
    rc, _ = run_batch(ref, Ref.TQ_KV_Q8_DEVICE, w, shape, T, T - 2, 3, normal(3 * hidden, 9), kc_d, vc_d)
    assert rc == -1


def test_config_mismatch_fails(nat, oracle):
    """A device cache made for another head count: the fused route returns the
    library's -1 from attention_layer instead of attending garbage."""
    ref = dropin("fused")
    shape = (8, 2, 64, 256, 1e4, 1e-6)
    w = layer_weights(oracle, 8, 2, 64, 256, 1)
    kc, vc = blocks(2 * 16 * 2), blocks(2 * 16 * 2)
    ref.lib.tqref_set_cache_q_heads(4)
    try:
        rc, _ = run_steps(ref, Ref.TQ_KV_Q8_DEVICE, w, shape, 16, 0, 1, normal(256, 1), kc, vc)
        assert rc == -1
        rc, _ = run_batch(ref, Ref.TQ_KV_Q8_DEVICE, w, shape, 16, 0, 4, normal(4 * 256, 2), kc, vc)
        assert rc == -1
    finally:
        ref.lib.tqref_set_cache_q_heads(0)


def logits_close(got, want, what, first_bar=1e-4):
    for t in range(got.shape[0]):
        err = rel_l2(got[t], want[t])
        assert err <= (first_bar if t == 0 else 3e-2), f"{what}: token {t} relative L2 {err:.3e}"
        top = np.sort(want[t])[-2:]
        if top[1] - top[0] > 0.02 * np.abs(want[t]).max():
            assert int(np.argmax(got[t])) == int(np.argmax(want[t])), f"{what}: greedy token {t}"


@pytest.mark.parametrize("variant", ["fused", "route"])
def test_forward_token_device_caches(nat, oracle, variant):
    """tq_ctx_init(..., TQ_KV_Q8_DEVICE) + the reference's tq_forward_token:
    every layer's attention through the edited attention_layer."""
    ref = dropin(variant)
    m = Model(oracle, 2, 8, 2, 64, 256, 512, 300, seed=21)
    tokens = np.random.default_rng(2).integers(0, 300, 24)
    ref.set_kv_type(Ref.TQ_KV_Q8)
    host = ref.forward(m, tokens, 32)
    ref.set_kv_type(Ref.TQ_KV_Q8_DEVICE)
    devl = ref.forward(m, tokens, 32)
    logits_close(devl, host, f"tq_forward_token on device caches ({variant})")


def test_prefill_device_caches(nat, oracle):
    """The reference's tq_prefill (tq_forward_batch in chunks of 16 through
    attention_layer_batch) on TQ_KV_Q8_DEVICE caches: last logits and every
    layer's cache against the host run (layer 0 bit for bit)."""
    ref = dropin("fused")
    m = Model(oracle, 2, 8, 2, 64, 256, 512, 300, seed=22)
    tokens = np.random.default_rng(3).integers(0, 300, 50)
    ref.set_kv_type(Ref.TQ_KV_Q8)
    lh, kh, vh = ref.prefill(m, tokens, 64)
    ref.set_kv_type(Ref.TQ_KV_Q8_DEVICE)
    ld, kd, vd = ref.prefill(m, tokens, 64)
    assert rel_l2(ld, lh) <= 3e-2
    # rows [0, 50) only: the host cache, like the reference's (model/kv_cache.c:29-34), is uninitialised past them
    nb = m.hd // QK
    rows = lambda c: c.reshape(m.nkv, 64, nb)[:, :len(tokens)]
    assert rows(kd[0]).tobytes() == rows(kh[0]).tobytes(), "layer 0 K cache"
    assert rows(vd[0]).tobytes() == rows(vh[0]).tobytes(), "layer 0 V cache"
    # deeper layers see the previous layers' outputs, which carry the device
    # attention's rounding (and the odd moved activation code) forward
    from oracle.binding import dequant
    for l in range(1, m.n_layers):
        for d_, h_, what in ((kd[l], kh[l], "K"), (vd[l], vh[l], "V")):
            assert rel_l2(dequant(rows(d_).reshape(-1)), dequant(rows(h_).reshape(-1))) <= 1e-2, f"layer {l} {what}"


def test_forward_token_device_model(nat, oracle):
    """The edited tq_forward_token's device-model branch (ctx->dev set: the
    whole token on the device, logits copied into ctx->logits) against the
    reference's own host forward of the same weights."""
    ref = dropin("fused")
    m = Model(oracle, 2, 8, 2, 64, 256, 512, 300, seed=23)
    tokens = np.random.default_rng(4).integers(0, 300, 16)
    ref.set_kv_type(Ref.TQ_KV_Q8)
    host = ref.forward(m, tokens, 32)
    devl = ref.forward_devmodel(m, tokens, 32)
    logits_close(devl, host, "tq_forward_token with ctx->dev")
