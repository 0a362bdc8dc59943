"""The drop-in's reference-side edits, checked on the CPU (no GPU calls).

oracle/dropin_patch.sh edits the reference's model_ops.h, attention_layer.c
and context.c at build time.  Here:

* the reference's own model_ops.h, the edited one (which includes
  tq/tq_model.h, hence tq/tq_attn.h, after its types) and tq/tq_attn.h alone
  are compiled side by side: tq_kv_cache keeps every host field at the
  reference's offset (caches built by hand, tools/test_model.c:842-850, still
  work), the edited struct and the library's own definition agree field for
  field, and the enum values of the reference's cache types are unchanged;
* the edited attention_layer.c and context.c compile against the library's
  headers with implicit declarations as errors;
* the script refuses a reference whose anchor lines have moved.

Needs the reference's sources (skipped where they are absent).
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
PATCH = os.path.join(ROOT, "oracle", "dropin_patch.sh")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "model")),
                                reason="the reference's sources are not here")

PROBE = r"""
#include <stddef.h>
#include <stdio.h>
%s
int main(void) {
    printf("size %%zu\n", sizeof(tq_kv_cache));
    printf("type %%zu\n", offsetof(tq_kv_cache, type));
    printf("k_f32 %%zu\n", offsetof(tq_kv_cache, k_f32));
    printf("v_f32 %%zu\n", offsetof(tq_kv_cache, v_f32));
    printf("k_q8 %%zu\n", offsetof(tq_kv_cache, k_q8));
    printf("v_q8 %%zu\n", offsetof(tq_kv_cache, v_q8));
    printf("max_tokens %%zu\n", offsetof(tq_kv_cache, max_tokens));
    %s
    printf("cfg %%zu %%zu %%zu %%zu %%zu %%zu\n", offsetof(tq_attn_config, n_q_heads),
           offsetof(tq_attn_config, n_kv_heads), offsetof(tq_attn_config, head_dim),
           offsetof(tq_attn_config, hidden_size), offsetof(tq_attn_config, rope_theta),
           offsetof(tq_attn_config, rms_eps));
    printf("enum %%d %%d\n", (int)TQ_KV_F32, (int)TQ_KV_Q8);
    %s
    return 0;
}
"""


def probe(tmp, name, include, extra="", incdirs=()):
    src = os.path.join(tmp, name + ".c")
    exe = os.path.join(tmp, name)
    dev_lines = ('printf("dev %zu\\n", offsetof(tq_kv_cache, dev));', 'printf("device %d\\n", (int)TQ_KV_Q8_DEVICE);')
    with open(src, "w") as f:
        f.write(PROBE % (include, dev_lines[0] if extra else "", dev_lines[1] if extra else ""))
    cmd = ["gcc", "-std=gnu11", "-Werror=implicit-function-declaration", "-o", exe, src]
    for d in incdirs:
        cmd += ["-I", d]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return dict(line.split(" ", 1) for line in out.strip().splitlines())


def test_layouts_agree(tmp_path):
    tmp = str(tmp_path)
    edited = os.path.join(tmp, "edited")
    subprocess.run(["sh", PATCH, REF, edited], check=True, capture_output=True, text=True)
    inc = os.path.join(ROOT, "include")
    ref = probe(tmp, "probe_ref", '#include "model/model_ops.h"', incdirs=(REF, os.path.join(REF, "model")))
    ed = probe(tmp, "probe_edited", '#include "model/model_ops.h"', extra=True,
               incdirs=(edited, REF, os.path.join(REF, "model"), inc))
    lib = probe(tmp, "probe_lib", '#include "tq/tq_attn.h"', extra=True, incdirs=(inc,))
    for key in ("type", "k_f32", "v_f32", "k_q8", "v_q8", "max_tokens", "cfg", "enum"):
        assert ed[key] == ref[key], (key, ed[key], ref[key])
    assert ed == lib, (ed, lib)
    assert int(ed["dev"]) >= int(ref["size"]) - 8 and int(ed["size"]) > int(ref["size"])
    assert ed["device"] == "2"


def test_edited_sources_compile(tmp_path):
    tmp = str(tmp_path)
    edited = os.path.join(tmp, "edited")
    subprocess.run(["sh", PATCH, REF, edited], check=True, capture_output=True, text=True)
    for name in ("attention_layer.c", "context.c"):
        for route in ((), ("-DTQ_DROPIN_ROUTE_ONLY",)):
            subprocess.run(["gcc", "-std=gnu11", "-fopenmp", "-Werror=implicit-function-declaration", *route,
                            "-I", edited, "-I", REF, "-I", os.path.join(REF, "model"),
                            "-I", os.path.join(ROOT, "include"), "-c", os.path.join(edited, "model", name),
                            "-o", os.path.join(tmp, name + ".o")], check=True, capture_output=True, text=True)


def test_patch_refuses_moved_anchor(tmp_path):
    """A reference whose attend_all_heads routing anchor changed: the script
    fails instead of building without the edit."""
    fake = tmp_path / "ref"
    shutil.copytree(os.path.join(REF, "model"), fake / "model")
    p = fake / "model" / "attention_layer.c"
    p.write_text(p.read_text().replace("static void attend_all_heads(", "static void attend_every_head("))
    r = subprocess.run(["sh", PATCH, str(fake), str(tmp_path / "out")], capture_output=True, text=True)
    assert r.returncode != 0 and "tq_attend_device" in r.stderr
