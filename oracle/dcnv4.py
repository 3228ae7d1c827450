"""CPU restatement of DCNv4-3D -- TEST INFRASTRUCTURE / CPU BASELINE ONLY.

Follows the reference's forward_kernel_dcn (csrc/cuda/dcnv4_im2col_cuda.cuh:20-205) and
backward_kernel_dcn (csrc/cuda/dcnv4_col2im_cuda.cuh:47-320), with the trilinear helpers of
csrc/cuda/common.h:52-353:
  value [B, Din, Hin, Win, G*D]; offset [B, Dout, Hout, Wout, padded]: per group K (x, y, z)
  offsets then K mask values; tap t runs over x (w) outermost, y, z innermost, skipping the
  centre when remove_center;
  pixel = p0' + (tap * dil + offset) * scale,  p0' = ((dil (k-1)) >> 1) - pad + pos * stride -
          ((dil (k-1)) >> 1) * scale   (float32, step by step -- what the kernels compute);
  a sample counts when every coordinate is in (-1, size); trilinear, zero outside the volume;
  out = sum over taps of mask * sample, the masks softmaxed over K when softmax.
Interpolation, softmax and sums in float64.  Backward: grad_value (scatter), offset gradients
mask * scale * sum_c g_c d(sample_c)/d(pixel), mask gradients (through the softmax).
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def geometry(size_in, kernel, stride, pad, dil, remove_center):
    """-> (output size (D, H, W), taps [K, 3] as (i_w, j_h, k_d))."""
    out = tuple((n + 2 * p - (d * (k - 1) + 1)) // s + 1 for n, k, s, p, d in zip(size_in, kernel, stride, pad, dil))
    kd, kh, kw = kernel
    taps = []
    for i in range(kw):
        for j in range(kh):
            for k in range(kd):
                if remove_center and i == kw // 2 and j == kh // 2 and k == kd // 2:
                    continue
                taps.append((i, j, k))
    return out, np.array(taps, dtype=np.int64)


def pixels(offsets, size_in, kernel, stride, pad, dil, scale, remove_center):
    """offsets [B, Dout, Hout, Wout, G, K, 3] (x, y, z) -> pixel coordinates (x, y, z), float32."""
    out, taps = geometry(size_in, kernel, stride, pad, dil, remove_center)
    Do, Ho, Wo = out
    zo, yo, xo = np.meshgrid(np.arange(Do), np.arange(Ho), np.arange(Wo), indexing="ij")
    pos = (xo, yo, zo)                                   # per axis x, y, z
    axes = [(2, 0, 0), (1, 1, 1), (0, 2, 2)]             # (kernel/stride/pad index, tap column, offset axis)
    res = []
    s = f32(scale)
    for a, (ki, tc, oa) in enumerate(axes):
        k, st, p, d = kernel[ki], stride[ki], pad[ki], dil[ki]
        half = (d * (k - 1)) >> 1
        p0 = (f32(half - p) + f32(0)) + (pos[a] * st).astype(f32)        # exact integers
        p0 = (p0.astype(f32) - f32(half) * s).astype(f32)
        t = (taps[:, tc] * d).astype(f32)
        o = offsets[..., oa].astype(f32)
        v = (p0[None, :, :, :, None, None] + ((t[None, None, None, None, None, :] + o) * s).astype(f32)).astype(f32)
        res.append(v)
    return res   # [x, y, z], each [B, Do, Ho, Wo, G, K]


def _split(offset, G, K):
    B, Do, Ho, Wo, _ = offset.shape
    o = np.asarray(offset, dtype=np.float64)[..., : G * 4 * K].reshape(B, Do, Ho, Wo, G, 4 * K)
    return o[..., : 3 * K].reshape(B, Do, Ho, Wo, G, K, 3), o[..., 3 * K:]


def _softmax(m):
    e = np.exp(m - m.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def _corners(px, py, pz, size):
    """Trilinear set-up: list of 8 (zi, yi, xi, weight, valid) arrays, plus the sample mask."""
    Di, Hi, Wi = size
    inside = (px > -1) & (py > -1) & (pz > -1) & (px < Wi) & (py < Hi) & (pz < Di)
    x0, y0, z0 = np.floor(px), np.floor(py), np.floor(pz)
    fx, fy, fz = px - x0, py - y0, pz - z0
    out = []
    for c in range(8):
        dz, dy, dx = c >> 2, (c >> 1) & 1, c & 1
        zi, yi, xi = (z0 + dz).astype(np.int64), (y0 + dy).astype(np.int64), (x0 + dx).astype(np.int64)
        w = (fz if dz else 1 - fz) * (fy if dy else 1 - fy) * (fx if dx else 1 - fx)
        ok = inside & (zi >= 0) & (zi < Di) & (yi >= 0) & (yi < Hi) & (xi >= 0) & (xi < Wi)
        out.append((np.where(ok, zi, 0), np.where(ok, yi, 0), np.where(ok, xi, 0), w, ok, dz, dy, dx))
    return out, inside


def forward(value, offset, kernel, stride, pad, dil, group, scale, remove_center=0, softmax=False, magnitude=False):
    """-> output [B, Dout, Hout, Wout, G*D] float64; magnitude=True: the sum of |terms| of each
    output element instead (for rounding-error bounds)."""
    v = np.asarray(value, dtype=np.float64)
    if magnitude:
        v = np.abs(v)
    B, Di, Hi, Wi, C = v.shape
    G = group
    D = C // G
    out_size, taps = geometry((Di, Hi, Wi), kernel, stride, pad, dil, remove_center)
    K = len(taps)
    off, m = _split(offset, G, K)
    attn = _softmax(m) if softmax else m
    if magnitude:
        attn = np.abs(attn)
    px, py, pz = pixels(off, (Di, Hi, Wi), kernel, stride, pad, dil, scale, remove_center)
    px, py, pz = px.astype(np.float64), py.astype(np.float64), pz.astype(np.float64)
    vg = v.reshape(B, Di, Hi, Wi, G, D)
    bi = np.arange(B).reshape(B, 1, 1, 1, 1, 1)
    gi = np.arange(G).reshape(1, 1, 1, 1, G, 1)
    corners, _ = _corners(px, py, pz, (Di, Hi, Wi))
    samp = 0.0
    for zi, yi, xi, w, ok, *_ in corners:
        samp = samp + (w * ok)[..., None] * vg[bi, zi, yi, xi, gi]        # [B,Do,Ho,Wo,G,K,D]
    out = (attn[..., None] * samp).sum(-2)
    return out.reshape(B, *out_size, G * D)


def backward(value, offset, grad_output, kernel, stride, pad, dil, group, scale, remove_center=0, softmax=False,
             magnitude=False):
    """-> (grad_value [B,Din,Hin,Win,G*D], grad_offset [B,Dout,Hout,Wout,padded]) float64;
    magnitude=True: the offset gradients' sums of |terms| instead (value gradient unchanged)."""
    v = np.asarray(value, dtype=np.float64)
    if magnitude:
        v = np.abs(v)
    B, Di, Hi, Wi, C = v.shape
    G = group
    D = C // G
    out_size, taps = geometry((Di, Hi, Wi), kernel, stride, pad, dil, remove_center)
    K = len(taps)
    off, m = _split(offset, G, K)
    attn = _softmax(m) if softmax else m
    px, py, pz = pixels(off, (Di, Hi, Wi), kernel, stride, pad, dil, scale, remove_center)
    px, py, pz = px.astype(np.float64), py.astype(np.float64), pz.astype(np.float64)
    g = np.asarray(grad_output, dtype=np.float64).reshape(B, *out_size, G, 1, D)
    if magnitude:
        g = np.abs(g)
        attn = np.abs(attn)
    vg = v.reshape(B, Di, Hi, Wi, G, D)
    bi = np.arange(B).reshape(B, 1, 1, 1, 1, 1)
    gi = np.arange(G).reshape(1, 1, 1, 1, G, 1)
    corners, _ = _corners(px, py, pz, (Di, Hi, Wi))
    fx, fy, fz = px - np.floor(px), py - np.floor(py), pz - np.floor(pz)
    gv = np.zeros((B, Di, Hi, Wi, G, D))
    gsamp = np.zeros(attn.shape)
    gpx = np.zeros(attn.shape)
    gpy = np.zeros(attn.shape)
    gpz = np.zeros(attn.shape)
    for zi, yi, xi, w, ok, dz, dy, dx in corners:
        val = vg[bi, zi, yi, xi, gi] * ok[..., None]                     # [B,Do,Ho,Wo,G,K,D]
        gd = (g * val).sum(-1)                                           # g . V_corner
        gsamp += w * gd
        sx = 1.0 if (dx or magnitude) else -1.0
        sy = 1.0 if (dy or magnitude) else -1.0
        sz = 1.0 if (dz or magnitude) else -1.0
        wz, wy, wx = (fz if dz else 1 - fz), (fy if dy else 1 - fy), (fx if dx else 1 - fx)
        gpx += sx * wz * wy * gd
        gpy += sy * wz * wx * gd
        gpz += sz * wy * wx * gd
        contrib = (attn * w * ok)[..., None] * g                         # into grad_value
        np.add.at(gv, (np.broadcast_to(bi, zi.shape), zi, yi, xi, np.broadcast_to(gi, zi.shape)), contrib)
    goff = np.stack([gpx, gpy, gpz], -1) * (attn * scale)[..., None]     # [..., K, 3]
    if softmax:
        gm = attn * (gsamp - (attn * gsamp).sum(-1, keepdims=True))
    else:
        gm = gsamp
    grad_offset = np.zeros(np.asarray(offset).shape)
    rows = np.concatenate([goff.reshape(*goff.shape[:-2], 3 * K), gm], -1)   # [B,Do,Ho,Wo,G,4K]
    grad_offset[..., : G * 4 * K] = rows.reshape(*rows.shape[:-2], G * 4 * K)
    return gv.reshape(B, Di, Hi, Wi, C), grad_offset
