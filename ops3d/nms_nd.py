"""Alias of ``ops3d_amd.nms`` under the reference's module path (ops3d/nms_nd.py)."""
from ops3d_amd.nms import nms_nd  # noqa: F401
