"""Evidence for the fp32 gradient bar (CPU): the fp32 PyTorch path of the op (oracle.torch_port:
per-level grid_sample + softmax + autograd, the reference's own formulation) against the
float64 oracle on c1 and on a query slice of c4.

The plain bar rtol 1e-5 / atol 1e-6 holds for the fp32 forward output, grad_value and the
logit gradients, but not for the location gradients: they are sums of cancelling corner
differences, and fp32 PyTorch breaks the plain bar on some of them by several times.  What it
needs beyond the plain bar is a small fraction of the random-walk rounding size sqrt(n) u M;
the allowance oracle.fp32_loc_allowance grants (FP32_LOC_ALLOWANCE_K = 0.15 of it) was sized on
fp32 PyTorch (torch 2.10: on c1, 113 of 110592 location gradients beyond the plain bar, up to
4.8x), and the GPU tests hold the kernel to the same bar.  Only the upper bound is asserted:
how many elements another torch build puts beyond the plain bar is printed, not tested."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_port
from ops3d_amd.workloads import WORKLOADS, make_inputs

RTOL, ATOL = 1e-5, 1e-6


def _case(name, q_limit):
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=0, dtype=torch.float32, q_limit=q_limit)
    vd = inp["value"].double().numpy()
    sd = inp["sampling_loc_attn"].double().numpy()
    gd = inp["grad_output"].double().numpy()
    ro = oracle.forward(vd, w.shapes, sd, w.K, coord_mode=1)
    rgv, rgs = oracle.backward(vd, w.shapes, sd, gd, w.K, coord_mode=1)
    allow = oracle.fp32_loc_allowance(vd, w.shapes, sd, gd, w.K)
    v = inp["value"].clone().requires_grad_(True)
    s = inp["sampling_loc_attn"].clone().requires_grad_(True)
    out = torch_port.forward_packed(v, w.shapes, s, w.K)
    out.backward(inp["grad_output"])
    n = 3 * w.L * w.K
    return {
        "out": (out.detach().double().numpy().reshape(ro.shape), ro, None),
        "grad_value": (v.grad.double().numpy(), rgv, None),
        "grad_loc": (s.grad.double().numpy()[..., :n], rgs[..., :n], allow[..., :n]),
        "grad_logit": (s.grad.double().numpy()[..., n:], rgs[..., n:], None),
    }


@pytest.mark.parametrize("name,q_limit", [("c1", None), ("c4", 1024)])
def test_torch_fp32_within_the_loc_allowance(name, q_limit):
    res = _case(name, q_limit)
    for key in ("out", "grad_value", "grad_logit"):   # the plain bar holds
        got, exp, _ = res[key]
        raw = ATOL + RTOL * np.abs(exp)
        assert (np.abs(got - exp) <= raw).all(), key
    got, exp, allow = res["grad_loc"]
    err = np.abs(got - exp)
    raw = ATOL + RTOL * np.abs(exp)
    breaks = int((err > raw).sum())
    ratio = float((err / raw).max())
    use = float(((err - raw) / allow).max())
    print(f"[fp32 bar] {name}: {breaks} location gradients beyond the plain bar (up to {ratio:.1f}x), "
          f"{use:.2f} of the allowance used", flush=True)
    # fp32 PyTorch stays inside the plain bar plus the allowance
    assert use <= 1.0, use
