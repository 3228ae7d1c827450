"""Drop-in alias: ``import ops3d`` resolves to the gfx950 implementation in ``ops3d_amd``.

Code written against the reference (``from ops3d import FlashDeformAttnFunction``,
``from ops3d.flash_deform_attn import findspec``, ``ops3d._C``) runs unchanged.  Only the
flash-deform-attn path exists here; DCNv4-3D, NMS-3D and ROI-Align-3D are not provided.
"""
from ops3d_amd import _C, FlashDeformAttnFunction, ms_deform_attn_core_pytorch_3d
from . import flash_deform_attn

__all__ = ["FlashDeformAttnFunction", "ms_deform_attn_core_pytorch_3d", "_C"]
