"""ops3d_amd -- MI355X-native (gfx950) Flash Deformable 3D Attention.

Exports the reference's flash-deform-attn API (reference ops3d/__init__.py:3-25):
``FlashDeformAttnFunction`` and ``ms_deform_attn_core_pytorch_3d``; ``_C`` is the native
extension object (None when libops3d_fda.so is not built).
"""
from ._extension import _C
from .flash_deform_attn import FlashDeformAttnFromOffsets, FlashDeformAttnFunction, ms_deform_attn_core_pytorch_3d
from .modules import FlashDeformAttn3D

__all__ = ["FlashDeformAttnFunction", "FlashDeformAttnFromOffsets", "FlashDeformAttn3D",
           "ms_deform_attn_core_pytorch_3d", "_C"]
