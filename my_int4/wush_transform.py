"""``my_int4.wush_transform`` with the reference's names and signatures
(reference my_int4/wush_transform.py:27-58): the offline WUSH transform
solve, the weight transform W' = W T^-1 and the fp64 activation transform
X' = X T^T, all per 32-column block in fp64.

The reference delegates the solve to the un-vendored IST-DASLab WUSH module;
this build's own closed form is in wush_int4_kernel_amd.wush_transform (the
transform T makes T Gx T^T = T^-T Gw T^-1 and carries a Hadamard rotation).
These are offline set-up steps, not the inference path."""
from wush_int4_kernel_amd.wush_transform import (  # noqa: F401
    compute_wush_transform,
    transform_activations_reference,
    transform_weights,
)

__all__ = ["compute_wush_transform", "transform_weights", "transform_activations_reference"]
