"""GPU parity through the C host interface (libtqattn.so): the kv_cache and
attention entry points a patched attention_layer.c calls for a
TQ_KV_Q8_DEVICE cache, against the oracle's restatement of the same calls.

Bar as everywhere: K/V codes and scales bit-exact, outputs within
1e-4 + 1e-3*|oracle| in fp32.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import BLOCK_Q8, QK, blocks
from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def attn():
    from tailorquantkernel_amd import attn, native
    native.init(0)
    attn.load()
    return attn


def make(attn, nq, nkv, hd, T, theta):
    cfg = attn.AttnConfig(nq, nkv, hd, nq * hd, theta, 1e-6)
    c = attn.Cache(attn.TQ_KV_Q8_DEVICE, cfg, T)
    assert c.rc == 0 and c.validate() == 0 and c.c.dev
    return cfg, c


def flat_caches(nkv, T, nb):
    return blocks(nkv * T * nb).reshape(nkv, T, nb), blocks(nkv * T * nb).reshape(nkv, T, nb)


def assert_same_blocks(a, b, what):
    assert a.tobytes() == b.tobytes(), what


@pytest.mark.parametrize("shape", [(8, 2, 64, 70, 1e4), (32, 8, 128, 40, 5e5), (16, 2, 128, 33, 1e6)])
def test_attention_core_steps(attn, oracle, shape):
    """attention_layer's core (rope_table, RoPE, store_kv, attend) token by
    token, as attn_block drives it (model/context.c:85)."""
    nq, nkv, hd, T, theta = shape
    nb = hd // QK
    cfg, c = make(attn, nq, nkv, hd, T, theta)
    kc, vc = flat_caches(nkv, T, nb)
    rng = np.random.default_rng(17)
    for pos in range(T):
        q = rng.standard_normal(nq * hd, dtype=np.float32)
        k = rng.standard_normal(nkv * hd, dtype=np.float32)
        v = rng.standard_normal(nkv * hd, dtype=np.float32)
        rc, out = c.attention_core(pos, q, k, v)
        orc, ref = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0 and orc == 0
        assert_close(out, ref, f"pos {pos}")
    rc, gk, gv = c.download()
    assert rc == 0
    assert_same_blocks(gk, kc, "K cache")
    assert_same_blocks(gv, vc, "V cache")
    c.free()
    assert c.validate() == -1


def test_store_then_attend_routing(attn, oracle):
    """The two routing targets of attention_layer.c's switches: the host
    applies RoPE (model/attention_layer.c:186-188), then store_kv and
    attend_all_heads go to the device."""
    nq, nkv, hd, T, theta = 8, 2, 64, 48, 1e4
    nb = hd // QK
    cfg, c = make(attn, nq, nkv, hd, T, theta)
    kc, vc = flat_caches(nkv, T, nb)
    rng = np.random.default_rng(5)
    for pos in range(T):
        q = rng.standard_normal(nq * hd, dtype=np.float32)
        k = rng.standard_normal(nkv * hd, dtype=np.float32)
        v = rng.standard_normal(nkv * hd, dtype=np.float32)
        cs, sn = attn.rope_table(hd, pos, theta)
        qr = np.concatenate([oracle.rope_apply(q[h * hd:(h + 1) * hd], cs, sn) for h in range(nq)])
        kr = np.concatenate([oracle.rope_apply(k[h * hd:(h + 1) * hd], cs, sn) for h in range(nkv)])
        assert c.store_kv(pos, kr, v) == 0
        rc, out = c.attend(pos, qr)
        assert rc == 0
        orc, ref = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, q, k, v)
        assert orc == 0
        assert_close(out, ref, f"pos {pos}")
    rc, gk, gv = c.download()
    assert rc == 0
    assert_same_blocks(gk, kc, "K cache")
    assert_same_blocks(gv, vc, "V cache")


@pytest.mark.parametrize("shape", [(8, 2, 64, 300, 1e4, 0, 300), (32, 8, 128, 640, 5e5, 21, 600)])
def test_attention_core_batch(attn, oracle, shape):
    """attention_layer_batch's token loop (model/attention_layer.c:221-236)
    over a cache that already holds pos0 tokens."""
    nq, nkv, hd, T, theta, pos0, n = shape
    nb = hd // QK
    cfg, c = make(attn, nq, nkv, hd, T, theta)
    kc, vc = flat_caches(nkv, T, nb)
    rng = np.random.default_rng(99)
    if pos0:
        for arr in (kc, vc):
            pre = oracle.quantize_row_q8(rng.standard_normal(nkv * pos0 * hd, dtype=np.float32))
            arr[:, :pos0, :] = pre.reshape(nkv, pos0, nb)
        assert c.upload(kc, vc) == 0
    q = rng.standard_normal((n, nq * hd), dtype=np.float32)
    k = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    v = rng.standard_normal((n, nkv * hd), dtype=np.float32)
    rc, out = c.attention_core_batch(pos0, n, q, k, v)
    orc, ref = oracle.prefill_qkv(kc, vc, nq, nkv, hd, T, theta, pos0, n, q, k, v)
    assert rc == 0 and orc == 0
    assert_close(out, ref, "batch")
    rc, gk, gv = c.download()
    assert_same_blocks(gk, kc, "K cache")
    assert_same_blocks(gv, vc, "V cache")


def test_device_cache_errors_write_nothing(attn):
    """Bad positions and a config that does not match the cache return -1
    and leave the cache as it was (tools/test_model.c:1015-1049)."""
    nq, nkv, hd, T = 8, 2, 64, 32
    cfg, c = make(attn, nq, nkv, hd, T, 1e4)
    rng = np.random.default_rng(3)
    k = np.frombuffer(rng.integers(0, 256, nkv * T * 2 * 36, dtype=np.uint8).tobytes(), BLOCK_Q8)
    k = k.copy().reshape(nkv, T, 2)
    k["d"] = np.abs(k["d"]) % 4  # finite scales
    assert c.upload(k, k) == 0
    x = np.ones(nq * hd, np.float32)
    for pos in (-1, T, T + 100):
        assert c.attention_core(pos, x, x[:nkv * hd], x[:nkv * hd])[0] == -1
        assert c.store_kv(pos, x[:nkv * hd], x[:nkv * hd]) == -1
        assert c.attend(pos, x)[0] == -1
    assert c.attention_core_batch(T - 3, 4, np.ones((4, nq * hd)), np.ones((4, nkv * hd)),
                                  np.ones((4, nkv * hd)))[0] == -1
    other = attn.AttnConfig(nq, nkv, 128, nq * 128, 1e4, 1e-6)
    saved, c.cfg = c.cfg, other
    assert c.store_kv(0, np.ones(nkv * 128), np.ones(nkv * 128)) == -1
    c.cfg = saved
    rc, gk, gv = c.download()
    assert rc == 0
    assert_same_blocks(gk, k, "K after rejected calls")
    assert_same_blocks(gv, k, "V after rejected calls")
    c.free()
    c.free()
    assert c.validate() == -1
