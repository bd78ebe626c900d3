"""Drop-in ``my_int4`` package: the reference's package name and ``_C`` op
surface (reference ``my_int4/__init__.py:4-6``), served by the MI355X build in
``wush_int4_kernel_amd``.  Like the reference, importing it imports torch first
and then ``_C``; ``from my_int4._C import ...`` and ``from my_int4 import _C``
both work."""
import torch  # noqa: F401

from my_int4._C import quant_int4  # noqa: F401,E402
