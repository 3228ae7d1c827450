"""DCNv4-3D: the CPU oracle pinned (agreement with the independent flash-deform-attn C oracle,
identity and shift closed forms, finite differences) and the GPU kernels against it (marked
gpu).  The reference ships no DCNv4 tests; semantics from csrc/cuda/dcnv4_im2col_cuda.cuh and
dcnv4_col2im_cuda.cuh."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import dcnv4 as O


def _inputs(B, size, G, D, kernel, stride, pad, dil, remove_center, seed, off_std=1.0, pad_extra=4):
    r = np.random.default_rng(seed)
    out, taps = O.geometry(size, kernel, stride, pad, dil, remove_center)
    K = len(taps)
    padded = G * 4 * K + pad_extra
    value = r.normal(size=(B, *size, G * D))
    off = np.zeros((B, *out, padded))
    rows = np.concatenate([r.normal(0, off_std, size=(B, *out, G, 3 * K)), r.normal(size=(B, *out, G, K))], -1)
    off[..., : G * 4 * K] = rows.reshape(B, *out, G * 4 * K)
    gout = r.normal(size=(B, *out, G * D))
    return value.astype(np.float32), off.astype(np.float32), gout.astype(np.float32), K


# --- oracle pinning (CPU) --------------------------------------------------------------------
def test_agrees_with_fda_oracle():
    """DCN sample positions are pixel coordinates p; the flash-deform-attn C oracle (float64,
    exact coordinates, softmax over the masks) samples at loc * size - 0.5, so
    loc = (p + 0.5) / size reproduces them (the softmax-free path is pinned by the closed forms
    and finite differences below).
    Outputs, value gradients and mask gradients agree; offset gradients are the location
    gradients * scale / size."""
    size, G, D = (5, 6, 7), 2, 4
    kernel, stride, pad, dil, rc, scale = (3, 3, 3), (1, 2, 1), (1, 1, 1), (1, 1, 2), 1, 0.7
    value, off, gout, K = _inputs(1, size, G, D, kernel, stride, pad, dil, rc, seed=1)
    out = O.forward(value, off, kernel, stride, pad, dil, G, scale, rc, True)
    gv, go = O.backward(value, off, gout, kernel, stride, pad, dil, G, scale, rc, True)
    # the same problem in the flash-deform-attn layout: one level, Q = output voxels
    o, _ = O._split(off, G, K)
    px, py, pz = O.pixels(o, size, kernel, stride, pad, dil, scale, rc)
    Din, Hin, Win = size
    loc = np.stack([(px.astype(np.float64) + 0.5) / Win, (py.astype(np.float64) + 0.5) / Hin,
                    (pz.astype(np.float64) + 0.5) / Din], -1)                 # [B,Do,Ho,Wo,G,K,3]
    B, Q = 1, int(np.prod(out.shape[1:4]))
    m = off[..., : G * 4 * K].reshape(B, Q, G, 4 * K)[..., 3 * K:].astype(np.float64)
    sla = np.concatenate([loc.reshape(B, Q, G, 3 * K), m], -1)
    fo = oracle.forward(value.astype(np.float64).reshape(B, -1, G, D), [size], sla, K, coord_mode=0)
    fgv, fgs = oracle.backward(value.astype(np.float64).reshape(B, -1, G, D), [size], sla,
                               gout.astype(np.float64).reshape(B, Q, G * D), K, coord_mode=0)
    assert np.allclose(out.reshape(B, Q, G * D), fo, rtol=1e-9, atol=1e-10)
    assert np.allclose(gv.reshape(B, -1, G, D), fgv, rtol=1e-9, atol=1e-10)
    gor = go[..., : G * 4 * K].reshape(B, Q, G, 4 * K)
    sizes = np.array([Win, Hin, Din], np.float64)
    want_off = fgs[..., : 3 * K].reshape(B, Q, G, K, 3) * scale / sizes
    assert np.allclose(gor[..., : 3 * K].reshape(B, Q, G, K, 3), want_off, rtol=1e-8, atol=1e-10)
    assert np.allclose(gor[..., 3 * K:], fgs[..., 3 * K:], rtol=1e-9, atol=1e-10)
    assert np.all(go[..., G * 4 * K:] == 0)                                   # row padding


def test_identity_and_shift():
    size, G, D = (4, 5, 6), 2, 3
    r = np.random.default_rng(0)
    value = r.normal(size=(1, *size, G * D))
    # 1x1x1 kernel, zero offsets, mask 1, no softmax: the identity
    out, taps = O.geometry(size, (1, 1, 1), (1, 1, 1), (0, 0, 0), (1, 1, 1), 0)
    off = np.zeros((1, *out, G * 4))
    off[..., 3::4] = 1.0
    assert np.allclose(O.forward(value, off, (1, 1, 1), (1, 1, 1), (0, 0, 0), (1, 1, 1), G, 1.0), value)
    # 3x3x3 kernel, pad 1, zero offsets, a one-hot mask on tap (i, j, k): value shifted by (k-1, j-1, i-1)
    kernel = (3, 3, 3)
    out, taps = O.geometry(size, kernel, (1, 1, 1), (1, 1, 1), (1, 1, 1), 0)
    K = len(taps)
    t = 5
    i, j, k = taps[t]
    off = np.zeros((1, *out, G * 4 * K))
    for g in range(G):
        off[..., g * 4 * K + 3 * K + t] = 1.0
    got = O.forward(value, off, kernel, (1, 1, 1), (1, 1, 1), (1, 1, 1), G, 1.0)
    want = np.zeros_like(value)
    dz, dy, dx = k - 1, j - 1, i - 1
    Di, Hi, Wi = size
    for z in range(Di):
        for y in range(Hi):
            for x in range(Wi):
                zz, yy, xx = z + dz, y + dy, x + dx
                if 0 <= zz < Di and 0 <= yy < Hi and 0 <= xx < Wi:
                    want[0, z, y, x] = value[0, zz, yy, xx]
    assert np.allclose(got, want)


def test_finite_differences_without_softmax():
    size, G, D, kernel = (4, 4, 5), 1, 3, (2, 2, 2)
    stride, pad, dil, scale = (1, 1, 1), (0, 0, 0), (1, 1, 1), 0.5
    value, off, gout, K = _inputs(1, size, G, D, kernel, stride, pad, dil, 0, seed=3, off_std=0.3)
    value, off, gout = value.astype(np.float64), off.astype(np.float64), gout.astype(np.float64)
    _, go = O.backward(value, off, gout, kernel, stride, pad, dil, G, scale, 0, False)
    r = np.random.default_rng(7)
    for _ in range(12):
        idx = tuple(int(r.integers(0, n)) for n in off.shape[:-1]) + (int(r.integers(0, G * 4 * K)),)
        h = 1e-3
        a, b = off.copy(), off.copy()
        a[idx] += h
        b[idx] -= h
        fd = (np.sum(O.forward(value, a, kernel, stride, pad, dil, G, scale) * gout)
              - np.sum(O.forward(value, b, kernel, stride, pad, dil, G, scale) * gout)) / (2 * h)
        # offsets pass through float32 pixel coordinates: allow for that rounding
        assert abs(fd - go[idx]) < 2e-3 * max(1.0, abs(fd)), (idx, fd, go[idx])


# --- GPU ---------------------------------------------------------------------------------------
CASES = [
    # B, size, G, D, kernel, stride, pad, dil, remove_center, scale, softmax, dtype
    (2, (6, 8, 10), 4, 16, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), 0, 1.0, False, torch.float32),
    (1, (6, 8, 10), 4, 16, (3, 3, 3), (2, 1, 2), (1, 1, 1), (1, 2, 1), 1, 0.5, True, torch.float32),
    (2, (8, 8, 8), 8, 32, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), 0, 1.0, True, torch.bfloat16),
    (1, (5, 7, 9), 2, 32, (2, 3, 3), (1, 1, 1), (0, 1, 1), (1, 1, 1), 0, 1.0, False, torch.float16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_gpu_matches_oracle(gpu_device, case):
    from fda_helpers import TOL, assert_close, log

    from ops3d_amd.dcnv4 import dcnv4_3d

    B, size, G, D, kernel, stride, pad, dil, rc, scale, sm, dt = CASES[case]
    log(f"[case] dcnv4 #{case}: B={B} size={size} G={G} D={D} k={kernel} s={stride} p={pad} d={dil} rc={rc} "
        f"scale={scale} softmax={sm} {dt}")
    value, off, gout, K = _inputs(B, size, G, D, kernel, stride, pad, dil, rc, seed=10 + case)
    v = torch.from_numpy(value).to(dt)
    o = torch.from_numpy(off).to(dt)
    g = torch.from_numpy(gout).to(dt)
    vg = v.to(gpu_device).requires_grad_(True)
    og = o.to(gpu_device).requires_grad_(True)
    out = dcnv4_3d(vg, og, kernel, stride, pad, dil, G, D, scale, 64, rc, sm)
    out.backward(g.to(gpu_device))
    torch.cuda.synchronize()
    vd, od, gd = v.double().numpy(), o.double().numpy(), g.double().numpy()
    want = O.forward(vd, od, kernel, stride, pad, dil, G, scale, rc, sm)
    wgv, wgo = O.backward(vd, od, gd, kernel, stride, pad, dil, G, scale, rc, sm)
    rtol, atol = TOL[dt]
    fp32 = dt == torch.float32
    # fp32: the output and the value gradient without softmax (raw mask values of either sign)
    # and the offset gradients (cancelling corner differences) are cancelling sums: they get the
    # allowance of the flash-deform-attn location gradients, 0.15 sqrt(n) u sum|terms| (oracle
    # magnitude mode).  fp32 PyTorch needs about 0.5 of that unit on case 0's output and value
    # gradient (test_dcnv4_fp32_bar.py); the kernel uses at most 0.02 of it on these cases.
    u = 2.0 ** -24
    m_out = O.forward(vd, od, kernel, stride, pad, dil, G, scale, rc, sm, magnitude=True)
    m_gv, m_off = O.backward(vd, od, gd, kernel, stride, pad, dil, G, scale, rc, sm, magnitude=True)
    assert tuple(out.shape) == want.shape and out.dtype == dt
    assert_close("dcnv4 output", out.detach(), want, rtol, atol,
                 0.15 * np.sqrt(8 * K + 2) * u * m_out if fp32 else None)
    assert_close("dcnv4 grad_value", vg.grad, wgv, rtol, atol,
                 0.15 * np.sqrt(8 * K) * u * m_gv if fp32 else None)
    n = 3 * K
    go = og.grad.double().cpu().numpy()

    def rows(x):
        return x[..., : G * 4 * K].reshape(*x.shape[:-1], G, 4 * K)

    extra = 0.15 * np.sqrt(8 * D + 8) * u * rows(m_off)[..., :n] if fp32 else None
    assert_close("dcnv4 grad_offset", rows(go)[..., :n], rows(wgo)[..., :n], rtol, atol, extra)
    assert_close("dcnv4 grad_mask", rows(go)[..., n:], rows(wgo)[..., n:], rtol, atol)
    assert np.all(go[..., G * 4 * K:] == 0)   # the rows' padding
