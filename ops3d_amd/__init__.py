"""ops3d_amd -- MI355X-native (gfx950) Flash Deformable 3D Attention and the reference's other
3-D ops on the same library.

Exports the reference's flash-deform-attn API (reference ops3d/__init__.py:3-25):
``FlashDeformAttnFunction`` and ``ms_deform_attn_core_pytorch_3d``; the offset-mode op and
module (``FlashDeformAttnFromOffsets``, ``FlashDeformAttn3D``); ``_C`` is the native extension
object (None when libops3d_fda.so is not built), which also carries nms_3d,
roi_align_3d_forward/backward and dcnv4_forward/backward.  Submodules: ``nms`` (nms_nd),
``roi_align`` (RoIAlign3DFunction, RoIAlign), ``dcnv4`` (DCNv4Function).
"""
from ._extension import _C
from .flash_deform_attn import FlashDeformAttnFromOffsets, FlashDeformAttnFunction, ms_deform_attn_core_pytorch_3d
from .modules import FlashDeformAttn3D

__all__ = ["FlashDeformAttnFunction", "FlashDeformAttnFromOffsets", "FlashDeformAttn3D",
           "ms_deform_attn_core_pytorch_3d", "_C"]
