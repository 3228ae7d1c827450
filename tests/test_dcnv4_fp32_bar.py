"""Evidence for the DCNv4-3D fp32 bar (CPU): a plain fp32 PyTorch DCNv4-3D (grid_sample over each
group's volume at the kernels' float32 pixel coordinates, masks softmaxed or raw, autograd for
the value gradient) against the float64 oracle, on the fp32 cases of the GPU test.

With raw mask values (no softmax) the output and the value gradient are sums of terms of both
signs, so they can be far smaller than their sum of |terms| M, and fp32 PyTorch misses the plain
bar rtol 1e-5 / atol 1e-6 on some of them (torch 2.10, case 0: 153 of 61440 outputs, 172 of
61440 value gradients, by up to 3.4x).  What it needs beyond the plain bar stays below the
random-walk rounding unit sqrt(n) u M (n = 8K + 2 operations per output, 8K per value-gradient
term, u = 2^-24): about half of it.  The GPU test grants the kernel 0.15 of that unit, less than
fp32 PyTorch uses.  Only the upper bound is asserted; the break counts are printed."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dcnv4 as O
from test_dcnv4 import CASES, _inputs

RTOL, ATOL = 1e-5, 1e-6
U = 2.0 ** -24


def _torch_dcn(value, off, kernel, stride, pad, dil, G, scale, rc, softmax):
    """fp32 DCNv4-3D through grid_sample: pixel p -> grid (2p + 1) / size - 1 (align_corners
    False), zero padding; returns the output [B, Do, Ho, Wo, G*D] and value (requires grad)."""
    B, Din, Hin, Win, GD = value.shape
    D = GD // G
    (Do, Ho, Wo), taps = O.geometry((Din, Hin, Win), kernel, stride, pad, dil, rc)
    K = len(taps)
    o, m = O._split(off, G, K)
    px, py, pz = O.pixels(o, (Din, Hin, Win), kernel, stride, pad, dil, scale, rc)
    v = torch.from_numpy(value).float().requires_grad_(True)
    mt = torch.from_numpy(np.asarray(m, np.float32))
    if softmax:
        mt = torch.softmax(mt, -1)
    vol = v.reshape(B, Din, Hin, Win, G, D).permute(0, 4, 5, 1, 2, 3).reshape(B * G, D, Din, Hin, Win)

    def norm(p, n):
        return torch.from_numpy((2 * p.astype(np.float32) + 1) / np.float32(n) - 1)

    grid = torch.stack([norm(px, Win), norm(py, Hin), norm(pz, Din)], -1)          # [B,Do,Ho,Wo,G,K,3]
    grid = grid.permute(0, 4, 1, 2, 3, 5, 6).reshape(B * G, Do * Ho * Wo, K, 1, 3)
    s = F.grid_sample(vol, grid, mode="bilinear", padding_mode="zeros", align_corners=False)[..., 0]
    w = mt.permute(0, 4, 1, 2, 3, 5).reshape(B * G, 1, Do * Ho * Wo, K)
    out = (s * w).sum(-1).reshape(B, G, D, Do, Ho, Wo).permute(0, 3, 4, 5, 1, 2).reshape(B, Do, Ho, Wo, G * D)
    return out, v


@pytest.mark.parametrize("case", [i for i, c in enumerate(CASES) if c[-1] == torch.float32])
def test_torch_fp32_dcn_within_the_rounding_unit(case):
    B, size, G, D, kernel, stride, pad, dil, rc, scale, sm, _ = CASES[case]
    value, off, gout, K = _inputs(B, size, G, D, kernel, stride, pad, dil, rc, seed=10 + case)
    out, v = _torch_dcn(value, off, kernel, stride, pad, dil, G, scale, rc, sm)
    out.backward(torch.from_numpy(gout))
    vd, od, gd = value.astype(np.float64), off.astype(np.float64), gout.astype(np.float64)
    want = O.forward(vd, od, kernel, stride, pad, dil, G, scale, rc, sm)
    wgv, _ = O.backward(vd, od, gd, kernel, stride, pad, dil, G, scale, rc, sm)
    m_out = O.forward(vd, od, kernel, stride, pad, dil, G, scale, rc, sm, magnitude=True)
    m_gv, _ = O.backward(vd, od, gd, kernel, stride, pad, dil, G, scale, rc, sm, magnitude=True)
    for name, got, exp, m, n in (("output", out.detach().double().numpy(), want, m_out, 8 * K + 2),
                                 ("grad_value", v.grad.double().numpy(), wgv, m_gv, 8 * K)):
        err = np.abs(got - exp)
        raw = ATOL + RTOL * np.abs(exp)
        unit = np.sqrt(n) * U * m
        use = float(((err - raw) / unit).max())
        print(f"[dcnv4 fp32 bar] case {case} {name}: {int((err > raw).sum())} of {err.size} beyond the plain "
              f"bar (up to {float((err / raw).max()):.1f}x), {max(use, 0.0):.2f} of the rounding unit used", flush=True)
        assert use <= 1.0, (name, use)
