"""Alias of ``ops3d_amd.flash_deform_attn`` under the reference's module path."""
from ops3d_amd.flash_deform_attn import (  # noqa: F401
    FlashDeformAttnFunction,
    _C,
    factors,
    findspec,
    findspec_bwd,
    ms_deform_attn_core_pytorch_3d,
)
