"""DCNv4-3D: deformable 3-D convolution, version 4 (reference csrc/dcnv4.h:7-60, kernels
csrc/cuda/dcnv4_im2col_cuda.cuh / dcnv4_col2im_cuda.cuh; the reference binds them as
_C.dcnv4_forward / _C.dcnv4_backward and ships no Python wrapper).

``DCNv4Function.apply(value, p_offset, kernel, stride, pad, dilation, group, group_channels,
offset_scale, im2col_step, remove_center, softmax)`` wraps the two entry points for autograd
(kernel, stride, pad and dilation are (d, h, w) triples).  value [B, Din, Hin, Win, G*D];
p_offset [B, Dout, Hout, Wout, padded_offset_dim] with, per group, K (x, y, z) offsets and K mask
values (K = taps of the kernel, minus the centre when remove_center).  The gfx950 kernels are the
flash-deform-attn kernels in DCN mode: pixel coordinates formed from the output voxel, tap,
dilation, padding and offset_scale; grad_value gathered by tiles (no atomics).
"""
from __future__ import annotations

from torch.autograd import Function
from torch.autograd.function import once_differentiable

from ._extension import _C


class DCNv4Function(Function):
    @staticmethod
    def forward(ctx, value, p_offset, kernel, stride, pad, dilation, group, group_channels, offset_scale,
                im2col_step=64, remove_center=0, softmax=False):
        if _C is None:
            raise RuntimeError("ops3d_amd native library (libops3d_fda.so) not built; DCNv4Function requires it.")
        ctx.args = (*kernel, *stride, *pad, *dilation, group, group_channels, offset_scale, im2col_step)
        ctx.remove_center, ctx.softmax = remove_center, softmax
        ctx.save_for_backward(value, p_offset)
        return _C.dcnv4_forward(value, p_offset, *ctx.args, remove_center, 8, 0, softmax)

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        value, p_offset = ctx.saved_tensors
        grad_value, grad_offset = _C.dcnv4_backward(value, p_offset, *ctx.args, grad_output.contiguous(),
                                                    ctx.remove_center, 8, 0, ctx.softmax)
        return grad_value, grad_offset, None, None, None, None, None, None, None, None, None, None


dcnv4_3d = DCNv4Function.apply
