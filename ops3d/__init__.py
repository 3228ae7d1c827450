"""Drop-in alias: ``import ops3d`` resolves to the gfx950 implementation in ``ops3d_amd``.

Code written against the reference (``from ops3d import FlashDeformAttnFunction``,
``from ops3d.flash_deform_attn import findspec``, ``ops3d._C``, ``from ops3d.nms_nd import
nms_nd``, ``from ops3d.roi_align_nd import RoIAlign``) runs unchanged; ``_C`` also carries
``nms_3d``, ``roi_align_3d_forward/backward`` and ``dcnv4_forward/backward``
(reference csrc/vision.cpp:14-25).
"""
from ops3d_amd import _C, FlashDeformAttnFunction, ms_deform_attn_core_pytorch_3d
from . import flash_deform_attn, nms_nd, roi_align_nd

__all__ = ["FlashDeformAttnFunction", "ms_deform_attn_core_pytorch_3d", "_C"]
