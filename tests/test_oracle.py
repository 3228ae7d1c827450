"""Pins the CPU oracle (oracle/) before anything is compared against it.

Checks, each chosen so a plausible mistake (wrong axis order, dropped corner, sign error in a
location gradient, missing size factor, softmax over one level only, off-by-half pixel
convention) fails at least one of them:
  * torch's F.grid_sample + autograd (library routine; the reference's own PyTorch path,
    ops3d/flash_deform_attn.py:139-165) in float64, forward and all three gradients;
  * an independent pure-Python brute force (nested lerps) on tiny volumes;
  * central finite differences of the oracle forward vs the oracle backward;
  * closed forms: voxel centres return the voxel, constant fields return the constant,
    uniform logits give 1/(L*K), out-of-volume samples contribute nothing;
  * the committed golden fixture (tests/golden/).
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_port
from ops3d_amd.workloads import level_meta, pack

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "c1_small.npz")


def _inputs(shapes, B, Q, G, D, K, seed=0, lo=0.0, hi=1.0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    L = len(shapes)
    S = sum(a * b * c for a, b, c in shapes)
    v = torch.randn(B, S, G, D, generator=g, dtype=dtype)
    loc = torch.rand(B, Q, G, L, K, 3, generator=g, dtype=dtype) * (hi - lo) + lo
    lg = torch.randn(B, Q, G, L, K, generator=g, dtype=dtype)
    go = torch.randn(B, Q, G * D, generator=g, dtype=dtype)
    return v, pack(loc, lg), go


CASES = [
    # shapes, B, Q, G, D, K, lo, hi
    (((4, 8, 16), (2, 4, 8)), 1, 40, 3, 8, 4, 0.0, 1.0),          # c1 geometry
    (((3, 5, 7),), 2, 17, 2, 4, 8, -0.2, 1.2),                    # anisotropic, OOB
    (((1, 1, 1), (6, 6, 6)), 1, 9, 2, 5, 4, 0.0, 1.0),            # uneven levels incl. 1^3
    (((2, 3, 4), (4, 2, 3), (1, 2, 2)), 1, 11, 1, 3, 2, -0.5, 1.5),  # L=3, heavy OOB
]


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_grid_sample_float64(case):
    shapes, B, Q, G, D, K, lo, hi = case
    v, sla, go = _inputs(shapes, B, Q, G, D, K, lo=lo, hi=hi)
    out_t, gv_t, gs_t = torch_port.forward_backward(v, shapes, sla, go, K)
    out_o = oracle.forward(v.numpy(), shapes, sla.numpy(), K, coord_mode=0)
    gv_o, gs_o = oracle.backward(v.numpy(), shapes, sla.numpy(), go.numpy(), K, coord_mode=0)
    np.testing.assert_allclose(out_o, out_t.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gv_o, gv_t.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gs_o, gs_t.numpy(), rtol=1e-10, atol=1e-10)


def test_oracle_fp32_coordinates_match_fp32_grid_sample():
    shapes = ((4, 8, 16), (2, 4, 8))
    v, sla, go = _inputs(shapes, 1, 64, 2, 8, 4, dtype=torch.float32)
    out_t, gv_t, gs_t = torch_port.forward_backward(v, shapes, sla, go, 4)
    out_o = oracle.forward(v.numpy(), shapes, sla.numpy(), 4, coord_mode=1)
    gv_o, gs_o = oracle.backward(v.numpy(), shapes, sla.numpy(), go.numpy(), 4, coord_mode=1)
    np.testing.assert_allclose(out_o, out_t.double().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gv_o, gv_t.double().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gs_o, gs_t.double().numpy(), rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------------------------
def _lerp_sample(vol, x, y, z):
    """Trilinear sample of vol[D][H][W][C] at pixel (x,y,z) with zero padding, by nested
    lerps -- written independently of the oracle's 8-weight form."""
    Dl, Hl, Wl = len(vol), len(vol[0]), len(vol[0][0])
    C = len(vol[0][0][0])

    def at(zi, yi, xi, c):
        if 0 <= zi < Dl and 0 <= yi < Hl and 0 <= xi < Wl:
            return vol[zi][yi][xi][c]
        return 0.0

    x0, y0, z0 = math.floor(x), math.floor(y), math.floor(z)
    fx, fy, fz = x - x0, y - y0, z - z0
    res = []
    for c in range(C):
        plane = []
        for zi in (z0, z0 + 1):
            row = []
            for yi in (y0, y0 + 1):
                a, b = at(zi, yi, x0, c), at(zi, yi, x0 + 1, c)
                row.append(a + fx * (b - a))
            plane.append(row[0] + fy * (row[1] - row[0]))
        res.append(plane[0] + fz * (plane[1] - plane[0]))
    return res


def _brute_forward(v, shapes, sla, K):
    B, S, G, D = v.shape
    L = len(shapes)
    Q = sla.shape[1]
    out = np.zeros((B, Q, G * D))
    for b in range(B):
        for q in range(Q):
            for g in range(G):
                rec = sla[b, q, g]
                logits = rec[3 * L * K:]
                e = [math.exp(t - max(logits)) for t in logits]
                attn = [t / sum(e) for t in e]
                start = 0
                for l, (Dl, Hl, Wl) in enumerate(shapes):
                    vol = [[[[v[b, start + (zi * Hl + yi) * Wl + xi, g, c] for c in range(D)]
                             for xi in range(Wl)] for yi in range(Hl)] for zi in range(Dl)]
                    start += Dl * Hl * Wl
                    for k in range(K):
                        s = l * K + k
                        x = rec[3 * s] * Wl - 0.5
                        y = rec[3 * s + 1] * Hl - 0.5
                        z = rec[3 * s + 2] * Dl - 0.5
                        smp = _lerp_sample(vol, x, y, z)
                        for c in range(D):
                            out[b, q, g * D + c] += attn[s] * smp[c]
    return out


def test_oracle_matches_brute_force():
    shapes = ((2, 3, 4), (1, 2, 2))
    v, sla, _ = _inputs(shapes, 1, 5, 2, 3, 2, lo=-0.3, hi=1.3, seed=3)
    ref = _brute_forward(v.numpy(), shapes, sla.numpy(), 2)
    out = oracle.forward(v.numpy(), shapes, sla.numpy(), 2, coord_mode=0)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-13)


def test_oracle_backward_matches_finite_differences():
    shapes = ((3, 4, 5), (2, 2, 3))
    K = 2
    v, sla, go = _inputs(shapes, 1, 4, 2, 3, K, lo=0.05, hi=0.95, seed=7)
    vn, sn, gn = v.numpy(), sla.numpy(), go.numpy()
    gv, gs = oracle.backward(vn, shapes, sn, gn, K, coord_mode=0)

    def loss(vv, ss):
        return float((oracle.forward(vv, shapes, ss, K, coord_mode=0) * gn).sum())

    rng = np.random.default_rng(0)
    h = 1e-6
    for _ in range(12):
        idx = tuple(rng.integers(0, n) for n in vn.shape)
        vp, vm = vn.copy(), vn.copy()
        vp[idx] += h
        vm[idx] -= h
        fd = (loss(vp, sn) - loss(vm, sn)) / (2 * h)
        assert abs(fd - gv[idx]) < 1e-6 * max(1.0, abs(fd)), (idx, fd, gv[idx])
    for _ in range(24):   # locations and logits
        idx = tuple(rng.integers(0, n) for n in sn.shape)
        sp, sm = sn.copy(), sn.copy()
        sp[idx] += h
        sm[idx] -= h
        fd = (loss(vn, sp) - loss(vn, sm)) / (2 * h)
        assert abs(fd - gs[idx]) < 1e-5 * max(1.0, abs(fd)), (idx, fd, gs[idx])


def test_oracle_closed_forms():
    shapes = ((4, 5, 6), (2, 3, 2))
    L, K, G, D = 2, 4, 2, 3
    S = 4 * 5 * 6 + 2 * 3 * 2
    rng = np.random.default_rng(1)
    v = rng.standard_normal((1, S, G, D))
    # voxel centres (i + 0.5)/size on every sample, uniform logits -> mean of those voxels
    Q = 3
    locs = np.zeros((1, Q, G, L, K, 3))
    expect = np.zeros((1, Q, G * D))
    start = [0, 120]
    for q in range(Q):
        for g in range(G):
            for l, (Dl, Hl, Wl) in enumerate(shapes):
                for k in range(K):
                    xi, yi, zi = rng.integers(0, Wl), rng.integers(0, Hl), rng.integers(0, Dl)
                    locs[0, q, g, l, k] = [(xi + 0.5) / Wl, (yi + 0.5) / Hl, (zi + 0.5) / Dl]
                    vox = start[l] + (zi * Hl + yi) * Wl + xi
                    expect[0, q, g * D:(g + 1) * D] += v[0, vox, g] / (L * K)
    sla = pack(torch.from_numpy(locs), torch.zeros(1, Q, G, L, K, dtype=torch.float64)).numpy()
    np.testing.assert_allclose(oracle.forward(v, shapes, sla, K, coord_mode=0), expect, rtol=1e-12, atol=1e-12)
    # constant field c with all corners inside -> output c for any softmax weights
    vc = np.full_like(v, 2.5)
    inner = pack(torch.rand(1, Q, G, L, K, 3, dtype=torch.float64) * 0.4 + 0.3,
                 torch.randn(1, Q, G, L, K, dtype=torch.float64)).numpy()
    np.testing.assert_allclose(oracle.forward(vc, shapes, inner, K, coord_mode=0), 2.5, rtol=1e-12)
    # samples outside the volume contribute nothing and get zero location gradients
    far = pack(torch.full((1, Q, G, L, K, 3), 1.7, dtype=torch.float64),
               torch.randn(1, Q, G, L, K, dtype=torch.float64)).numpy()
    assert np.all(oracle.forward(v, shapes, far, K, coord_mode=0) == 0)
    gv, gs = oracle.backward(v, shapes, far, np.ones((1, Q, G * D)), K, coord_mode=0)
    assert np.all(gv == 0) and np.all(gs == 0)
    # zero upstream gradient -> exactly zero gradients
    gv, gs = oracle.backward(v, shapes, inner, np.zeros((1, Q, G * D)), K, coord_mode=0)
    assert np.all(gv == 0) and np.all(gs == 0)
    # grad_value mass: sum over voxels = sum over samples of attn * (sum of in-bounds weights) * g
    g_up = rng.standard_normal((1, Q, G * D))
    gv, _ = oracle.backward(v, shapes, inner, g_up, K, coord_mode=0)
    logits = inner[..., 3 * L * K:]
    attn = np.exp(logits - logits.max(-1, keepdims=True))
    attn /= attn.sum(-1, keepdims=True)
    mass = attn.sum(-1)  # all corners inside -> weights sum to 1 per sample
    expect_sum = (g_up.reshape(1, Q, G, D) * mass[..., None]).sum(1)  # [1,G,D]
    np.testing.assert_allclose(gv.sum(1), expect_sum, rtol=1e-12, atol=1e-12)


def test_oracle_golden_fixture():
    fx = np.load(GOLDEN)
    shapes = [tuple(int(t) for t in s) for s in fx["shapes"]]
    K = int(fx["K"])
    out = oracle.forward(fx["value"], shapes, fx["sampling_loc_attn"], K, coord_mode=0)
    gv, gs = oracle.backward(fx["value"], shapes, fx["sampling_loc_attn"], fx["grad_output"], K, coord_mode=0)
    np.testing.assert_allclose(out, fx["output"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gv, fx["grad_value"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(gs, fx["grad_sampling_loc_attn"], rtol=1e-9, atol=1e-11)


def test_level_meta():
    st, lsi = level_meta(((4, 8, 16), (2, 4, 8)), "cpu")
    assert st.tolist() == [[4, 8, 16], [2, 4, 8]]
    assert lsi.tolist() == [0, 512]


def test_oracle_term_counts():
    """abs_mode=2: grad_value holds each element's number of terms -- whole numbers, the same
    for every channel, summing to D x (in-volume corners of all samples), counted here
    independently from the fp32 pixel coordinates."""
    shapes = [(3, 4, 5), (2, 2, 3)]
    B, Q, G, D, K = 1, 17, 2, 4, 4
    L = len(shapes)
    v, sla, go = (t.numpy() for t in _inputs(shapes, B, Q, G, D, K, seed=7, lo=-0.2, hi=1.2))
    n, _ = oracle.backward(v, shapes, sla, go, K, coord_mode=1, abs_mode=2)
    assert np.all(n == np.round(n)) and np.all(n >= 0)
    assert np.all(n == n[..., :1])

    def pix(loc, size):   # torch grid_sample's fp32 rounding, as the oracle's coord_mode=1
        l = np.float32(loc)
        t = np.float32(np.float32(np.float32(np.float32(2.0) * l) - np.float32(1.0)) + np.float32(1.0))
        return float(np.float32(np.float32(np.float32(t * np.float32(size)) - np.float32(1.0)) * np.float32(0.5)))

    corners = 0
    for b in range(B):
        for q in range(Q):
            for g in range(G):
                rec = sla[b, q, g]
                for l, (dd, hh, ww) in enumerate(shapes):
                    for k in range(K):
                        s = l * K + k
                        x, y, z = pix(rec[3 * s], ww), pix(rec[3 * s + 1], hh), pix(rec[3 * s + 2], dd)
                        if not (-1 <= x < ww and -1 <= y < hh and -1 <= z < dd):
                            continue
                        x0, y0, z0 = math.floor(x), math.floor(y), math.floor(z)
                        for dz in (0, 1):
                            for dy in (0, 1):
                                for dx in (0, 1):
                                    corners += (0 <= x0 + dx < ww) and (0 <= y0 + dy < hh) and (0 <= z0 + dz < dd)
    assert n.sum() == D * corners
