"""3-D non-maximum suppression (reference ops3d/nms_nd.py:28-53, csrc/nms_3d.h:27-44).

``nms_nd(dets, iou_threshold)`` takes dets [N, 7] (x1, y1, z1, x2, y2, z2, score) and returns
``(keep, dets)`` as the reference does: keep holds the int64 indices of the kept boxes in
decreasing score order.  The work runs in libops3d_fda.so (csrc/nms3d.hip): the IoU bitmask
and the greedy pass both on the GPU.
"""
from __future__ import annotations

import torch

from ._extension import _C


def nms_nd(dets: torch.Tensor, iou_threshold: float):
    """Greedy NMS: a box is dropped when its IoU with a kept higher-scoring box exceeds
    iou_threshold.  Returns (keep, dets)."""
    if _C is None:
        raise RuntimeError("ops3d_amd native library (libops3d_fda.so) not built; nms_nd requires it.")
    boxes = dets[:, :-1]
    scores = dets[:, -1]
    return _C.nms_3d(boxes, scores, iou_threshold), dets
