"""3-D RoI Align (reference ops3d/roi_align_nd.py:26-117; kernels in csrc/roi_align3d.hip).

The Function / module interface (names, arguments, the order-0 sampling rule and two error
messages) follows the reference's ops3d/roi_align_nd.py, which comes from MedVision
(https://github.com/TimothyZero/MedVision, medvision/ops/roi_align_nd.py) under the Apache
License 2.0; the bodies here are this package's own.

Same API: ``RoIAlign3DFunction`` / ``roi_align_3d(features, rois, output_size, spatial_scale,
sampling_ratio=0, order=1)`` and the ``RoIAlign`` module.  features [N, C, D, H, W]; rois
[R, 7] (batch index, x1, y1, z1, x2, y2, z2); output [R, C, d, h, w].  Gradients flow to the
features (none to the rois, as in the reference).
"""
from __future__ import annotations

from torch import nn
from torch.autograd import Function

from ._extension import _C


class RoIAlign3DFunction(Function):
    @staticmethod
    def forward(ctx, features, rois, output_size, spatial_scale, sampling_ratio=0, order=1):
        if _C is None:
            raise RuntimeError("ops3d_amd native library (libops3d_fda.so) not built; RoIAlign requires it.")
        if isinstance(output_size, int):
            out_d = out_h = out_w = output_size
        elif isinstance(output_size, tuple):
            if len(output_size) != 3 or not all(isinstance(v, int) for v in output_size):
                raise TypeError('"output_size" must be an integer or a tuple of 3 integers')
            out_d, out_h, out_w = output_size
        else:
            raise TypeError('"output_size" must be an integer or tuple of integers')
        ctx.spatial_scale = spatial_scale
        ctx.sampling_ratio = sampling_ratio
        ctx.order = order
        ctx.save_for_backward(rois)
        ctx.feature_size = features.size()
        num_rois, num_channels = rois.size(0), features.size(1)
        output = features.new_empty(num_rois, num_channels, out_d, out_h, out_w)   # written in full
        _C.roi_align_3d_forward(features, rois, output, out_d, out_h, out_w, spatial_scale, sampling_ratio, order)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        rois = ctx.saved_tensors[0]
        grad_input = None
        if ctx.needs_input_grad[0]:
            out_d, out_h, out_w = grad_output.shape[2:]
            grad_input = grad_output.new_empty(ctx.feature_size)   # written in full
            _C.roi_align_3d_backward(grad_output.contiguous(), rois, grad_input, out_d, out_h, out_w,
                                     ctx.spatial_scale, ctx.sampling_ratio, ctx.order)
        return grad_input, None, None, None, None, None


roi_align_3d = RoIAlign3DFunction.apply


class RoIAlign(nn.Module):
    """RoI Align over (N, C, D, H, W) features for rois (n, 7) = (batch index, x1, y1, z1, x2,
    y2, z2).  output_size (d, h, w); spatial_scale scales the boxes; sampling_ratio samples per
    bin and axis (<= 0: adaptive).  forward(features, rois, order=1): order 0 nearest, 1 linear."""

    def __init__(self, output_size: tuple, spatial_scale: float, sampling_ratio: int = -1):
        super().__init__()
        self.output_size = tuple(output_size)
        self.spatial_scale = float(spatial_scale)
        self.sampling_ratio = int(sampling_ratio)
        self.dim = len(self.output_size)
        if self.dim != 3:
            raise ValueError(f"Tried to init RoIAlign module with incorrect output size: {self.output_size}")
        self.roi_align = roi_align_3d

    def forward(self, features, rois, order=1):
        if order not in (0, 1):
            raise ValueError("only support order = 0 (nearest) or 1 (linear)")
        sampling_ratio = 1 if order == 0 else self.sampling_ratio
        return self.roi_align(features, rois, self.output_size, self.spatial_scale, sampling_ratio, order)
