"""MI355X (gfx950) Q8 grouped-query attention path of TailorQuantKernel.

Native pieces (built in-tree):
  * libtqhip.so  — HIP kernels + C-ABI shim (include/tq/tq_hip.h)
  * libtqattn.so — C11 host library with the reference's model_ops.h attention
                   and KV-cache entry points for a device-resident cache
                   (include/tq/tq_attn.h)

``native`` is the ctypes binding of libtqhip.so used by tests and bench.py.
"""
from . import native  # noqa: F401

__all__ = ["native"]
