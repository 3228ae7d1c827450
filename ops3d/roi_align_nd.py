"""Alias of ``ops3d_amd.roi_align`` under the reference's module path (ops3d/roi_align_nd.py)."""
from ops3d_amd.roi_align import RoIAlign, RoIAlign3DFunction, roi_align_3d  # noqa: F401
