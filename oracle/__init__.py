"""CPU oracle of Flash Deformable 3D Attention -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the timed CPU baseline; the product package
``ops3d_amd`` never imports it.

* ``forward`` / ``backward``: numpy wrappers of the float64 C restatement ``fda_oracle.c``
  (reference algorithm: ops3d/flash_deform_attn.py:139-165 for semantics,
  csrc/cuda/common.h:52-353 and flash_deform_{im2col,col2im}_cuda.cuh for the softmax, the
  sampling range test and the gradients -- file:line details are in fda_oracle.c).
* ``torch_port``: a PyTorch restatement of the reference's naive path (grid_sample +
  softmax + autograd), used as the CPU baseline and as a second, library-based check.

Parity pinning (tests/test_oracle.py): every function here is checked against torch's
``F.grid_sample`` (a library routine) and its autograd, against an independent pure-Python
brute-force loop on tiny volumes, against central finite differences of the forward, and
against closed-form special cases (voxel centres, constant fields, uniform logits,
out-of-volume samples, zero upstream gradient).  None is left unpinned.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "libfda_oracle.so")
_lib = None


def build() -> str:
    """Compile libfda_oracle.so with gcc (via the Makefile recipe in this directory)."""
    subprocess.run(["make", "-s", "-C", _DIR, "libfda_oracle.so"], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(
            os.path.join(_DIR, "fda_oracle.c")
        ):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        dp = ctypes.POINTER(ctypes.c_double)
        ip = ctypes.POINTER(ctypes.c_int64)
        ci = ctypes.c_int
        lib.fda_oracle_forward.argtypes = [dp, ip, ip, dp, dp] + [ci] * 8
        lib.fda_oracle_forward.restype = None
        lib.fda_oracle_backward.argtypes = [dp, ip, ip, dp, dp, dp, dp] + [ci] * 9
        lib.fda_oracle_backward.restype = None
        _lib = lib
    return _lib


def _d(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _p(a, t):
    return a.ctypes.data_as(ctypes.POINTER(t))


def _meta(shapes):
    shapes = np.ascontiguousarray(np.asarray(shapes, dtype=np.int64).reshape(-1, 3))
    sizes = shapes.prod(1)
    lsi = np.ascontiguousarray(np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64))
    return shapes, lsi


def forward(value, shapes, loc_attn, K, coord_mode=1):
    """value [B,S,G,D], shapes [L,3], loc_attn [B,Q,G,4LK] -> out [B,Q,G*D] (float64)."""
    lib = _load()
    value, loc_attn = _d(value), _d(loc_attn)
    shapes, lsi = _meta(shapes)
    B, S, G, D = value.shape
    L = shapes.shape[0]
    Q = loc_attn.shape[1]
    assert loc_attn.shape == (B, Q, G, 4 * L * K), loc_attn.shape
    assert int(shapes.prod(1).sum()) == S
    out = np.zeros((B, Q, G * D), dtype=np.float64)
    dp, ip = ctypes.c_double, ctypes.c_int64
    lib.fda_oracle_forward(_p(value, dp), _p(shapes, ip), _p(lsi, ip), _p(loc_attn, dp), _p(out, dp),
                           B, S, G, D, L, Q, K, coord_mode)
    return out


def backward(value, shapes, loc_attn, grad_out, K, coord_mode=1, abs_mode=0):
    """-> (grad_value [B,S,G,D], grad_loc_attn [B,Q,G,4LK]) in float64.  abs_mode=1 returns
    the per-element magnitude M (sum of |terms|) instead, for rounding-error bounds; abs_mode=2
    the same with grad_value holding each element's number of terms."""
    lib = _load()
    value, loc_attn, grad_out = _d(value), _d(loc_attn), _d(grad_out)
    shapes, lsi = _meta(shapes)
    B, S, G, D = value.shape
    L = shapes.shape[0]
    Q = loc_attn.shape[1]
    assert grad_out.size == B * Q * G * D
    gv = np.zeros_like(value)
    gla = np.zeros_like(loc_attn)
    dp, ip = ctypes.c_double, ctypes.c_int64
    lib.fda_oracle_backward(_p(value, dp), _p(shapes, ip), _p(lsi, ip), _p(loc_attn, dp), _p(grad_out, dp),
                            _p(gv, dp), _p(gla, dp), B, S, G, D, L, Q, K, coord_mode, abs_mode)
    return gv, gla


FP32_UNIT_ROUNDOFF = 2.0 ** -24

# Allowance factor of the fp32 location gradients, in units of sqrt(n) * u * M (below).  Sized
# on the fp32 PyTorch path (torch_port: grid_sample + autograd) against this float64 oracle on
# the benchmark inputs: it breaks the plain rtol 1e-5 / atol 1e-6 bar on up to 0.45 % of the
# location gradients (by up to 81x), and needs at most 0.14 sqrt(n) u M beyond that bar; the
# other outputs (forward, grad_value, logit gradients) stay inside the plain bar.
FP32_LOC_ALLOWANCE_K = 0.15


def fp32_loc_allowance(value, shapes, loc_attn, grad_out, K, k=FP32_LOC_ALLOWANCE_K):
    """Per-element rounding allowance for fp32 gradients of sampling_loc_attn, shaped like it:
    k * sqrt(n) * u * M on the 3*L*K location entries and 0 on the L*K logit entries.  M is the
    sum of |terms| of the element (backward(abs_mode=1)), u the fp32 unit roundoff and
    n = 8*D + 2*L*K + 8 the number of rounded operations in one element (8 corners x D channels,
    the softmax sums, the weight products).  A location gradient sums the value differences of
    corner pairs, which cancel: its magnitude can be far below M, so no fixed relative bar
    holds for it in fp32 whatever the summation order; rounding errors of independent operations
    add like a random walk, whose typical size is sqrt(n) * u * M."""
    value = np.asarray(value)
    D = value.shape[-1]
    L = len(shapes)
    _, m = backward(value, shapes, loc_attn, grad_out, K, coord_mode=1, abs_mode=1)
    n = 8 * D + 2 * L * K + 8
    allow = k * np.sqrt(n) * FP32_UNIT_ROUNDOFF * m
    allow[..., 3 * L * K:] = 0.0
    return allow
