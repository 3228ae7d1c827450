"""CPU restatement of 3-D NMS -- TEST INFRASTRUCTURE / CPU BASELINE ONLY.

Follows the reference's nms_3d_cuda (csrc/cuda/nms_3d_cuda.cu:36-47 IoU, :105-162 sort and
greedy pass): boxes (x1, y1, z1, x2, y2, z2) sorted by decreasing score, a box removed when its
IoU with a kept higher-scoring box exceeds the threshold.  IoU in float32, each step rounded
(numpy float32 arithmetic does not contract), in the kernel's order:
    extents max(min(hi) - max(lo), 0); inter = (w * h) * d; S = ((x2-x1) * (y2-y1)) * (z2-z1);
    iou = inter / ((Sa + Sb) - inter).
The sort is stable (equal scores keep index order), as the gfx950 build's.
"""
from __future__ import annotations

import numpy as np


def iou3d(a, b):
    """IoU of box a [6] against boxes b [M, 6], float32 step by step -> [M] float32."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32).reshape(-1, 6)
    with np.errstate(invalid="ignore", divide="ignore"):
        w = np.maximum(np.minimum(a[3], b[:, 3]) - np.maximum(a[0], b[:, 0]), np.float32(0))
        h = np.maximum(np.minimum(a[4], b[:, 4]) - np.maximum(a[1], b[:, 1]), np.float32(0))
        d = np.maximum(np.minimum(a[5], b[:, 5]) - np.maximum(a[2], b[:, 2]), np.float32(0))
        inter = (w * h) * d
        sa = ((a[3] - a[0]) * (a[4] - a[1])) * (a[5] - a[2])
        sb = ((b[:, 3] - b[:, 0]) * (b[:, 4] - b[:, 1])) * (b[:, 5] - b[:, 2])
        return (inter / ((sa + sb) - inter)).astype(np.float32)


def nms3d(boxes, scores, iou_threshold):
    """-> int64 array of kept indices (original order numbers), in decreasing score order."""
    boxes = np.asarray(boxes, dtype=np.float32).reshape(-1, 6)
    scores = np.asarray(scores)
    order = np.argsort(-scores.astype(np.float64), kind="stable")
    b = boxes[order]
    n = len(order)
    removed = np.zeros(n, dtype=bool)
    keep = []
    thr = np.float32(iou_threshold)
    for i in range(n):
        if removed[i]:
            continue
        keep.append(order[i])
        if i + 1 < n:
            removed[i + 1:] |= iou3d(b[i], b[i + 1:]) > thr
    return np.asarray(keep, dtype=np.int64)
