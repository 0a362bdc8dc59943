"""CPU checks of the C host interface (libtqattn.so, include/tq/tq_attn.h).

No compute runs here: these pin the header/binding ABI, the kv_cache
allocation and validation semantics of model/kv_cache.c:5-48 and
model/attention_layer.c:23-36, the argument checks the compute entry points
make before touching a device, and rope_table bit for bit.
"""
from __future__ import annotations

import ctypes as C
import os
import shutil
import subprocess

import numpy as np
import pytest

from tests.test_abi import ROOT, declared


@pytest.fixture(scope="module")
def attn():
    from tailorquantkernel_amd import attn
    attn.load()
    return attn


def cfg_of(attn, nq=8, nkv=2, hd=64, theta=10000.0):
    return attn.AttnConfig(nq, nkv, hd, nq * hd, theta, 1e-6)


def test_exports_every_declared_symbol(attn):
    names = declared("tq_attn.h", "tq_") | declared("tq_model.h", "tq_")
    names = {n for n in names if not n.startswith("tq_hip_")}
    assert len(names) == 19
    assert names == set(attn.EXPORTS), "ctypes prototypes out of step with tq_attn.h / tq_model.h"
    for n in names:
        assert hasattr(attn.load(), n)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_struct_layout_matches_header(attn, tmp_path):
    """The binding's tq_kv_cache / tq_attn_config match the C header's layout."""
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "tq/tq_attn.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu\\n\", sizeof(tq_kv_cache),"
        " offsetof(tq_kv_cache, k_q8), offsetof(tq_kv_cache, max_tokens),"
        " offsetof(tq_kv_cache, dev), sizeof(tq_attn_config), sizeof(tq_kv_type));"
        " return TQ_KV_Q8_DEVICE == 2 ? 0 : 1;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    K = attn.KVCache
    want = [C.sizeof(K), K.k_q8.offset, K.max_tokens.offset, K.dev.offset,
            C.sizeof(attn.AttnConfig), C.sizeof(C.c_int)]
    assert [int(x) for x in got] == want


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_model_struct_layout_matches_header(attn, tmp_path):
    """tq_dev_layer_weights / tq_dev_model / tq_dev_ctx and the tq_hip weight
    structs: the binding's layout is the header's."""
    src = tmp_path / "layout2.c"
    fields = [("tq_hip_attn_weights", "rms_eps"), ("tq_hip_mlp_weights", "inter"),
              ("tq_dev_layer_weights", "post_norm"), ("tq_dev_layer_weights", "mlp"),
              ("tq_dev_model", "vocab_size"), ("tq_dev_model", "layers"), ("tq_dev_ctx", "ws_bytes"),
              ("tq_dev_ctx", "sampled"), ("tq_dev_batch_ws", "tokens"), ("tq_dev_batch_ws", "ws_bytes"),
              ("tq_hip_attn_weights", "format"), ("tq_hip_mlp_weights", "format"), ("tq_dev_model", "embed_format")]
    body = " ".join(f'printf("%zu %zu ", sizeof({t}), offsetof({t}, {f}));' for t, f in fields)
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "tq/tq_model.h"\n'
                   f"int main(void){{{body} return 0;}}\n")
    exe = tmp_path / "layout2"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    from tailorquantkernel_amd import native
    py = {"tq_hip_attn_weights": native.AttnWeights, "tq_hip_mlp_weights": native.MlpWeights,
          "tq_dev_layer_weights": attn.DevLayerWeights, "tq_dev_model": attn.DevModel, "tq_dev_ctx": attn.DevCtx,
          "tq_dev_batch_ws": attn.DevBatchWs}
    want = []
    for t, f in fields:
        want += [C.sizeof(py[t]), getattr(py[t], f).offset]
    assert got == want


@pytest.mark.parametrize("kv_type", [0, 1])
def test_host_cache_init_free(attn, kv_type):
    """model/kv_cache.c:17-48: host types allocate, validate, free idempotently."""
    c = attn.Cache(kv_type, cfg_of(attn), 64)
    assert c.rc == 0
    assert c.c.max_tokens == 64 and c.c.type == kv_type and not c.c.dev
    if kv_type == 0:
        assert c.c.k_f32 and c.c.v_f32 and not c.c.k_q8
    else:
        assert c.c.k_q8 and c.c.v_q8 and not c.c.k_f32
    assert c.validate() == 0
    c.free()
    assert not (c.c.k_f32 or c.c.v_f32 or c.c.k_q8 or c.c.v_q8 or c.c.dev)
    assert c.c.max_tokens == 0
    assert c.validate() == -1
    c.free()


@pytest.mark.parametrize("kv_type", [0, 1, 2, 7])
def test_cache_init_rejects(attn, kv_type):
    c = attn.Cache(kv_type, cfg_of(attn), 0)
    assert c.rc == -1
    assert not (c.c.k_f32 or c.c.v_f32 or c.c.k_q8 or c.c.v_q8 or c.c.dev)
    if kv_type == 7:
        assert attn.Cache(7, cfg_of(attn), 16).rc == -1


def test_device_cache_needs_device(attn):
    from tailorquantkernel_amd import native
    if native.load().tq_hip_init(0) == 0:
        pytest.skip("a GPU is present; covered by the GPU tests")
    c = attn.Cache(attn.TQ_KV_Q8_DEVICE, cfg_of(attn), 64)
    assert c.rc == -1 and not c.c.dev
    # like an allocation failure in model/kv_cache.c:39-44: freed, max_tokens 0
    assert c.c.type == attn.TQ_KV_Q8_DEVICE and c.c.max_tokens == 0 and c.validate() == -1


def hand_cache(attn, kv_type, max_tokens, k_q8=None):
    c = attn.KVCache()
    c.type, c.max_tokens = kv_type, max_tokens
    if k_q8 is not None:
        c.k_q8 = c.v_q8 = k_q8.ctypes.data
    return c


def test_validate_codes(attn):
    """model/attention_layer.c:23-36, plus the device type."""
    lib = attn.load()
    v = lambda c: lib.tq_attn_validate_cache(C.byref(c))  # noqa: E731
    buf = np.zeros(16, np.uint8)
    assert v(hand_cache(attn, 1, 0, buf)) == -1
    assert v(hand_cache(attn, 1, 16)) == -2
    assert v(hand_cache(attn, 1, 16, buf)) == 0
    assert v(hand_cache(attn, 0, 16)) == -2
    assert v(hand_cache(attn, 2, 16)) == -2
    assert v(hand_cache(attn, 9, 16)) == -3


def test_compute_argument_order(attn):
    """Position range first (-1, model/attention_layer.c:172,203-204), then
    the cache type (-3) and storage (-2), all before any device call."""
    lib = attn.load()
    cfg = cfg_of(attn)
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    host = hand_cache(attn, 1, 16, np.zeros(16, np.uint8))
    dev = hand_cache(attn, 2, 16)
    for c, code in ((host, -3), (dev, -2)):
        for pos in (-1, 16, 1 << 30):
            assert lib.tq_attention_core(C.byref(cfg), C.byref(c), pos, p, p, p, p) == -1
            assert lib.tq_store_kv_device(C.byref(c), C.byref(cfg), pos, p, p) == -1
            assert lib.tq_attend_device(C.byref(c), C.byref(cfg), p, pos, p) == -1
        assert lib.tq_attention_core(C.byref(cfg), C.byref(c), 15, p, p, p, p) == code
        assert lib.tq_store_kv_device(C.byref(c), C.byref(cfg), 0, p, p) == code
        assert lib.tq_attend_device(C.byref(c), C.byref(cfg), p, 0, p) == code
        for pos0, n in ((0, 0), (0, -1), (10, 7), (-1, 2), (2147483000, 1000)):
            assert lib.tq_attention_core_batch(C.byref(cfg), C.byref(c), pos0, n, p, p, p, p) == -1
        assert lib.tq_attention_core_batch(C.byref(cfg), C.byref(c), 0, 16, p, p, p, p) == code
        assert lib.tq_kv_cache_upload(C.byref(c), p, p) == code
        assert lib.tq_kv_cache_download(C.byref(c), p, p) == code


@pytest.mark.parametrize("hd", [32, 64, 128, 256])
def test_rope_table_bit_exact(attn, oracle, hd):
    """tq_attn_rope_table == the oracle's rope_table (model/rope.c:4-12), bit for bit."""
    for theta in (1e4, 5e5, 1e6):
        for pos in (0, 1, 2, 255, 4095, 32767, 131071):
            c, s = attn.rope_table(hd, pos, theta)
            oc, os_ = oracle.rope_table(hd, pos, theta)
            assert c.tobytes() == oc.tobytes() and s.tobytes() == os_.tobytes(), (hd, pos, theta)


def test_rope_table_matches_reference_build(attn, ref_scalar):
    for hd in (64, 128):
        for pos in (0, 7, 4095):
            c, s = attn.rope_table(hd, pos, 5e5)
            rc = np.zeros(hd // 2, np.float32)
            rs = np.zeros(hd // 2, np.float32)
            ref_scalar.lib.rope_table(rc.ctypes.data, rs.ctypes.data, hd, pos, 5e5)
            assert c.tobytes() == rc.tobytes() and s.tobytes() == rs.tobytes()


def test_dev_model_guards(attn):
    """model/context.c:6-54 and :104-229's guards on the device model, checked
    before any device call (tools/test_model.c:1455-1480,1488-1510): NULL model
    or context, max_tokens 0, hidden not a multiple of 32, no layers, a missing
    weight in the last layer, a layer whose sizes disagree with the model, an
    unknown matrix format; a failed init leaves the context zeroed; free is
    idempotent."""
    from tailorquantkernel_amd import native
    L = attn.load()
    fake = 1 << 20        # never dereferenced: every call below fails validation first
    n_layers = 2
    layers = (attn.DevLayerWeights * n_layers)()
    for l in range(n_layers):
        layers[l].input_norm = layers[l].post_norm = fake
        layers[l].attn = native.AttnWeights(fake, fake, fake, fake, fake, fake, 256, 1e-6)
        layers[l].mlp = native.MlpWeights(fake, fake, fake, 256, 512)
    cfg = attn.AttnConfig(4, 2, 64, 256, 1e4, 1e-6)

    def model(**kw):
        m = attn.DevModel(cfg, n_layers, 512, 300, fake, fake, layers)
        for k, v in kw.items():
            setattr(m, k, v)
        return m

    ctx = attn.DevCtx()
    assert L.tq_dev_ctx_init(C.byref(ctx), None, 8) == -1
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model()), 0) == -1
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model(n_layers=0)), 8) == -1
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model(vocab_size=0)), 8) == -1
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model(embed_format=2)), 8) == -1
    bad_cfg = attn.AttnConfig(4, 2, 64, 257, 1e4, 1e-6)
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model(attn=bad_cfg)), 8) == -1
    layers[1].attn.wq = None                       # the last layer's weights are checked too
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model()), 8) == -1
    layers[1].attn.wq = fake
    layers[1].mlp.inter = 1024                     # disagrees with intermediate_size
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model()), 8) == -1
    layers[1].mlp.inter = 512
    layers[0].mlp.format = 5
    assert L.tq_dev_ctx_init(C.byref(ctx), C.byref(model()), 8) == -1
    layers[0].mlp.format = 0
    assert bytes(ctx) == bytes(attn.DevCtx())      # a failed init leaves the context zeroed
    L.tq_dev_ctx_free(C.byref(ctx))
    L.tq_dev_ctx_free(None)
    # the token calls on a context with no model, and NULL pointers
    assert L.tq_dev_forward_token(None, 0) == -1
    assert L.tq_dev_forward_token(C.byref(ctx), 0) == -1
    assert L.tq_dev_logits(C.byref(ctx), None) == -1
    assert L.tq_dev_sample_greedy(C.byref(ctx)) == -1
    ws = attn.DevBatchWs()
    assert L.tq_dev_batch_ws_init(C.byref(ws), None, 4) == -1
    assert L.tq_dev_batch_ws_init(C.byref(ws), C.byref(model()), 0) == -1
    L.tq_dev_batch_ws_free(C.byref(ws))
    toks = (C.c_int * 2)(1, 2)
    assert L.tq_dev_forward_batch(None, C.byref(ws), toks, 2, 1) == -1
    assert L.tq_dev_forward_batch(C.byref(ctx), C.byref(ws), toks, 2, 1) == -1
    assert L.tq_dev_prefill(None, toks, 2) == -1
    assert L.tq_dev_prefill(C.byref(ctx), toks, 2) == -1
