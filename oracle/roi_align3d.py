"""CPU restatement of 3-D RoI Align -- TEST INFRASTRUCTURE / CPU BASELINE ONLY.

Follows the reference's roi_align_3d_{forward,backward}_cuda_kernel
(csrc/cuda/roi_align_3d_cuda_kernel.cuh:27-220) and its interpolation helpers
(csrc/cuda/interpolation_helpers_3d.h:25-260):
  roi start = coordinate * scale (no rounding), extents max(end - start, 1), bin = extent / pooled,
  samples per axis = sampling_ratio (> 0) or ceil(extent / pooled), sample i at
  start + p * bin + (i + 0.5) * bin / grid;
  a sample beyond [-1, size] on any axis reads 0; coordinates <= 0 clamp to 0; base corner
  floor(c), and a base corner >= size - 1 collapses both corners onto size - 1 (coordinate set to
  it); order 1: trilinear weights (hz hy hx, ... in the reference's corner order), order 0: weight
  1 on the first corner whose three weights are >= 0.5;
  output = sum of the samples / max(number of samples, 1); backward: the adjoint scatter.
Sample coordinates are computed in float32 step by step (what the kernels compute); weights,
interpolation and sums in float64.
"""
from __future__ import annotations

import math

import numpy as np

f32 = np.float32


def _roi(r, scale, sr, pooled):
    b = int(f32(r[0]))
    s = [f32(f32(r[1 + a]) * f32(scale)) for a in range(3)]       # x, y, z starts
    e = [f32(f32(r[4 + a]) * f32(scale)) for a in range(3)]
    ext = [max(f32(e[a] - s[a]), f32(1.0)) for a in range(3)]
    pw, ph, pd = pooled[2], pooled[1], pooled[0]
    pz = [pw, ph, pd]
    bins = [f32(ext[a] / f32(pz[a])) for a in range(3)]
    grid = [sr if sr > 0 else int(math.ceil(f32(ext[a] / f32(pz[a])))) for a in range(3)]
    count = max(grid[0] * grid[1] * grid[2], 1)
    return b, s, bins, grid, count


def _coord(start, p, bin_, i, grid):
    return f32(f32(start + f32(f32(p) * bin_)) + f32(f32(f32(f32(i) + f32(0.5)) * bin_) / f32(grid)))


def _corners(z, y, x, D, H, W, order):
    """-> list of (flat offset, weight) for one sample (empty if it reads nothing)."""
    if y < -1.0 or y > H or x < -1.0 or x > W or z < -1.0 or z > D:
        return []
    z = float(z) if z > 0 else 0.0
    y = float(y) if y > 0 else 0.0
    x = float(x) if x > 0 else 0.0
    z0, y0, x0 = int(z), int(y), int(x)
    if z0 >= D - 1:
        z0 = z1 = D - 1
        z = float(z0)
    else:
        z1 = z0 + 1
    if y0 >= H - 1:
        y0 = y1 = H - 1
        y = float(y0)
    else:
        y1 = y0 + 1
    if x0 >= W - 1:
        x0 = x1 = W - 1
        x = float(x0)
    else:
        x1 = x0 + 1
    lz, ly, lx = z - z0, y - y0, x - x0
    hz, hy, hx = 1 - lz, 1 - ly, 1 - lx
    zs, ys, xs = (z0, z1), (y0, y1), (x0, x1)
    wz, wy, wx = (hz, lz), (hy, ly), (hx, lx)
    out = []
    if order == 0:
        for c in range(8):
            dz, dy, dx = c >> 2, (c >> 1) & 1, c & 1
            if wz[dz] >= 0.5 and wy[dy] >= 0.5 and wx[dx] >= 0.5:
                return [((zs[dz] * H + ys[dy]) * W + xs[dx], 1.0)]
        return []
    for c in range(8):
        dz, dy, dx = c >> 2, (c >> 1) & 1, c & 1
        out.append(((zs[dz] * H + ys[dy]) * W + xs[dx], wz[dz] * wy[dy] * wx[dx]))
    return out


def _bin_taps(rois, shape, pooled, scale, sr, order):
    """For every (roi, pd, ph, pw): (batch, list of (offset, weight / count))."""
    N, C, D, H, W = shape
    PD, PH, PW = pooled
    taps = {}
    for r in range(len(rois)):
        b, s, bins, grid, count = _roi(rois[r], scale, sr, pooled)
        for pd in range(PD):
            for ph in range(PH):
                for pw in range(PW):
                    t = []
                    if 0 <= b < N:
                        for iz in range(grid[2]):
                            z = _coord(s[2], pd, bins[2], iz, grid[2])
                            for iy in range(grid[1]):
                                y = _coord(s[1], ph, bins[1], iy, grid[1])
                                for ix in range(grid[0]):
                                    x = _coord(s[0], pw, bins[0], ix, grid[0])
                                    t += [(o, w / count) for o, w in _corners(z, y, x, D, H, W, order)]
                    taps[(r, pd, ph, pw)] = (b, t)
    return taps


def forward(features, rois, pooled, scale, sampling_ratio, order=1):
    """features [N,C,D,H,W], rois [R,7] -> [R,C,PD,PH,PW] float64."""
    x = np.asarray(features, dtype=np.float64)
    N, C, D, H, W = x.shape
    flat = x.reshape(N, C, D * H * W)
    rois = np.asarray(rois, dtype=np.float64)
    PD, PH, PW = pooled
    out = np.zeros((len(rois), C, PD, PH, PW))
    for (r, pd, ph, pw), (b, t) in _bin_taps(rois, x.shape, pooled, scale, sampling_ratio, order).items():
        if t:
            o = np.array([a for a, _ in t])
            w = np.array([v for _, v in t])
            out[r, :, pd, ph, pw] = flat[b][:, o] @ w
    return out


def backward(grad_output, rois, feature_shape, scale, sampling_ratio, order=1):
    """grad_output [R,C,PD,PH,PW] -> grad of the features [N,C,D,H,W] float64 (the adjoint)."""
    g = np.asarray(grad_output, dtype=np.float64)
    N, C, D, H, W = feature_shape
    pooled = g.shape[2:]
    out = np.zeros((N, C, D * H * W))
    for (r, pd, ph, pw), (b, t) in _bin_taps(np.asarray(rois, np.float64), feature_shape, pooled, scale,
                                             sampling_ratio, order).items():
        for o, w in t:
            out[b, :, o] += g[r, :, pd, ph, pw] * w
    return out.reshape(N, C, D, H, W)
