"""wush_int4_kernel_amd -- MI355X (gfx950) WUSH INT4 W4A4 inference path.

Native pieces (built in place by ``wush_int4_kernel_amd._build`` /
``__graft_entry__.build()``):

* ``libwush_int4.so`` -- the hand-written HIP kernels and their C ABI
  (``include/wush_int4.h``);
* ``_C`` -- a torch module with the reference's ``my_int4._C`` op names and
  signatures (reference ``csrc/bindings.cpp:28-68``), calling that C ABI.

Importing this package imports torch first (the reference does the same,
``my_int4/__init__.py:4-6``), then ``_C``.  There is no fallback: if the
native module is missing the import fails.
"""
import torch  # noqa: F401  (loads torch's HIP runtime before _C links against it)

try:
    from . import _C  # noqa: F401
except ImportError as e:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        "wush_int4_kernel_amd._C is not built; run `python -m wush_int4_kernel_amd._build` "
        "(or __graft_entry__.build()) first"
    ) from e

from ._C import quant_int4  # noqa: F401,E402

__all__ = ["_C", "quant_int4"]
