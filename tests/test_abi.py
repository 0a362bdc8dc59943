"""CPU checks of the C-ABI: the libraries load, export every symbol the
headers declare, and reject bad arguments before touching a device."""
from __future__ import annotations

import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header: str, prefix: str) -> set[str]:
    text = open(os.path.join(ROOT, "include", "tq", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(" + prefix + r"\w*)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    from tailorquantkernel_amd import native
    return native.load()


def test_tq_hip_exports_every_declared_symbol(lib):
    from tailorquantkernel_amd import native
    names = declared("tq_hip.h", "tq_hip_")
    assert len(names) >= 25
    for n in sorted(names):
        assert hasattr(lib, n), f"libtqhip.so does not export {n}"
    assert names == set(native.EXPORTS), "ctypes prototypes out of step with tq_hip.h"


def test_host_validation_without_device(lib):
    from tailorquantkernel_amd import native
    h = C.c_void_p()
    bad = [(0, 2, 64, 4, 1, 4), (8, 0, 64, 4, 1, 4), (8, 3, 64, 4, 1, 4), (8, 2, 48, 4, 1, 4),
           (8, 2, 64, 0, 1, 4), (8, 2, 64, 4, 0, 4), (8, 2, 64, 4, 1, 0)]
    for d in bad:
        desc = native.KVDesc(*d)
        assert lib.tq_hip_kv_create(C.byref(h), C.byref(desc)) == native.EINVAL, d
        assert h.value is None
    assert lib.tq_hip_kv_create(None, None) == native.EINVAL
    for d in [(8, 2, 96, 4, 1, 4), (40, 2, 64, 4, 1, 4)]:
        desc = native.KVDesc(*d)
        assert lib.tq_hip_kv_create(C.byref(h), C.byref(desc)) == native.ETYPE, d
    lib.tq_hip_kv_destroy(None)
    assert lib.tq_hip_kv_capacity(None, 0) == native.EINVAL
    assert lib.tq_hip_kv_set_pages(None, 0, None, 0) == native.EINVAL
    assert lib.tq_hip_kv_append(None, 0, 0, None, None, None, None) == native.EINVAL
    assert lib.tq_hip_attend(None, 0, 0, None, None, None, None) == native.EINVAL
    assert lib.tq_hip_prefill(None, 0, 0, 1, None, None, None, None, None, None) == native.EINVAL
    assert lib.tq_hip_quantize_row_q8(None, None, -1, None) == native.EINVAL
    assert lib.tq_hip_attn_scores_q8(None, 0, None, 1, 1, 1.0, None, 1, None) == native.EINVAL
    assert lib.tq_hip_attn_accum_q8(None, 1, 1, None, 1, 1, None, 8, None) == native.EINVAL
    assert lib.tq_hip_softmax(None, -1, 1, 1, None) == native.EINVAL
    assert lib.tq_hip_membw_read(None, 1 << 20, None, 0, None) == native.EINVAL
    assert lib.tq_hip_membw_read(C.c_void_p(16), 100, C.c_void_p(16), 0, None) == native.EINVAL   # not whole 16 B
    assert lib.tq_hip_membw_sink_bytes() > 0
    # weight side: shapes, nulls and alignment are refused before any device call
    assert lib.tq_hip_q8_matrix_bytes(4096, 4096) == 4096 * 128 * 36
    assert lib.tq_hip_q8_matrix_bytes(7, 48) == 0 and lib.tq_hip_q8_matrix_bytes(0, 64) == 0
    p16 = C.c_void_p(4096)
    assert lib.tq_hip_q8_pack(p16, p16, 4, 48, None) == native.EINVAL
    assert lib.tq_hip_q8_pack(C.c_void_p(4100), p16, 4, 64, None) == native.EINVAL   # dst not 16 B aligned
    assert lib.tq_hip_q8_unpack(None, p16, 4, 64, None) == native.EINVAL
    assert lib.tq_hip_matmul_q8(p16, p16, p16, 0, 64, None) == native.EINVAL
    assert lib.tq_hip_matmul_q8(p16, p16, p16, 4, 33, None) == native.EINVAL
    assert lib.tq_hip_matmul_q8(C.c_void_p(4104), p16, p16, 4, 64, None) == native.EINVAL
    assert lib.tq_hip_matmul_q8_batch(p16, p16, p16, 4, 64, 0, None) == native.EINVAL
    assert lib.tq_hip_matmul_q8_batch(p16, None, p16, 4, 64, 1, None) == native.EINVAL
    assert lib.tq_hip_project_qkv(p16, p16, p16, 64, 16, 64, p16, 1, None, p16, p16, p16, None) == native.EINVAL
    assert lib.tq_hip_project_qkv(p16, p16, p16, 64, 0, 64, p16, 1, p16, p16, p16, p16, None) == native.EINVAL
    assert lib.tq_hip_project_output(p16, 64, 48, p16, 1, p16, p16, None) == native.EINVAL
    assert lib.tq_hip_project_output(p16, 64, 64, p16, 0, p16, p16, None) == native.EINVAL
    for code, text in ((0, "ok"), (-1, "argument out of range"), (-3, "unsupported head_dim or group size")):
        assert native.strerror(code) == text


def test_init_reports_missing_device(lib):
    """Without a GPU (this CPU suite) tq_hip_init returns an error, never aborts."""
    from tailorquantkernel_amd import native
    rc = lib.tq_hip_init(0)
    if rc == 0:
        pytest.skip("a gfx950 device is present")
    assert rc == native.ENODEV or rc <= native.EHIP_BASE


def test_missing_library_fails_loudly(tmp_path):
    from tailorquantkernel_amd import native
    saved = native._lib
    native._lib = None
    try:
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            native.load(str(tmp_path / "libtqhip.so"))
    finally:
        native._lib = saved


def test_bench_library_exports_its_header():
    """libtqbench.so (bench.py's step floor, not part of the attention
    library) exports what tailorquantkernel_amd/bench/tq_bench.h declares, and
    the attention library exports none of it."""
    text = open(os.path.join(ROOT, "tailorquantkernel_amd", "bench", "tq_bench.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(tq_hip_\w*)\s*\(", text))
    assert names == {"tq_hip_floor_scratch_bytes", "tq_hip_floor_out_bytes", "tq_hip_floor_step"}
    bench = C.CDLL(os.path.join(ROOT, "tailorquantkernel_amd", "libtqbench.so"))
    from tailorquantkernel_amd import native
    attn = native.load()
    for n in names:
        assert hasattr(bench, n), n
        assert not hasattr(attn, n), f"{n} still exported by libtqhip.so"
    f = bench.tq_hip_floor_step
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    assert f(None, 1 << 20, 8, 32, 2, None, None, None) == native.EINVAL
