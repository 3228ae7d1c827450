"""Helpers shared by the GPU parity tests: run the op through the public API and compare
with the float64 C oracle on the same (dtype-rounded) inputs."""
from __future__ import annotations

import sys

import numpy as np
import torch

import oracle
from ops3d_amd import FlashDeformAttnFunction
from ops3d_amd.workloads import level_meta, pack

TOL = {
    # tolerances of the parity bar: fp32 rtol 1e-5 / atol 1e-6, bf16 (and fp16) 2e-2 / 2e-2
    torch.float32: (1e-5, 1e-6),
    torch.bfloat16: (2e-2, 2e-2),
    torch.float16: (2e-2, 2e-2),
}


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def random_inputs(shapes, B, Q, G, D, K, dtype, seed=0, lo=0.0, hi=1.0, value_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    L = len(shapes)
    S = sum(a * b * c for a, b, c in shapes)
    v = torch.randn(B, S, G, D, generator=g) * value_scale
    loc = torch.rand(B, Q, G, L, K, 3, generator=g) * (hi - lo) + lo
    lg = torch.randn(B, Q, G, L, K, generator=g)
    go = torch.randn(B, Q, G * D, generator=g)
    return {
        "value": v.to(dtype),
        "sampling_loc_attn": pack(loc, lg).to(dtype),
        "grad_output": go.to(dtype),
        "shapes": [tuple(s) for s in shapes],
        "K": K,
    }


def run_gpu(inp, device, backward=True, im2col_step=64):
    """Forward (+ backward with inp['grad_output']) through FlashDeformAttnFunction."""
    st, lsi = level_meta(inp["shapes"], device)
    v = inp["value"].to(device).contiguous().requires_grad_(backward)
    s = inp["sampling_loc_attn"].to(device).contiguous().requires_grad_(backward)
    out = FlashDeformAttnFunction.apply(v, st, lsi, s, im2col_step, inp["K"], True)
    if not backward:
        torch.cuda.synchronize()
        return out.detach(), None, None
    out.backward(inp["grad_output"].to(device))
    torch.cuda.synchronize()
    return out.detach(), v.grad, s.grad


def run_oracle(inp, backward=True):
    v = inp["value"].double().numpy()
    s = inp["sampling_loc_attn"].double().numpy()
    out = oracle.forward(v, inp["shapes"], s, inp["K"], coord_mode=1)
    if not backward:
        return out, None, None
    gv, gs = oracle.backward(v, inp["shapes"], s, inp["grad_output"].double().numpy(), inp["K"], coord_mode=1)
    return out, gv, gs


def assert_close(name, actual, expected, rtol, atol, extra=None):
    a = actual.detach().double().cpu().numpy() if isinstance(actual, torch.Tensor) else np.asarray(actual)
    e = np.asarray(expected, dtype=np.float64).reshape(a.shape)
    assert np.isfinite(a).all(), f"{name}: non-finite values"
    err = np.abs(a - e)
    allow = atol + rtol * np.abs(e)
    if extra is not None:
        allow = allow + np.asarray(extra).reshape(a.shape)
    bad = err > allow
    if bad.any():
        i = np.unravel_index(np.argmax(err - rtol * np.abs(e)), a.shape)
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{a.size} elements outside rtol={rtol} atol={atol}; "
            f"max abs err {err.max():.3e}; worst at {i}: got {a[i]!r} expected {e[i]!r}"
        )


def fp32_allowance(inp):
    """Rounding allowance of the fp32 location gradients (oracle.fp32_loc_allowance,
    0.15 sqrt(n) u M; zero on the logit entries), shaped like sampling_loc_attn.  The bar
    applied to them is rtol 1e-5 / atol 1e-6 plus this; everything else gets the plain bar."""
    return oracle.fp32_loc_allowance(
        inp["value"].double().numpy(), inp["shapes"], inp["sampling_loc_attn"].double().numpy(),
        inp["grad_output"].double().numpy(), inp["K"])


def compare_all(tag, got, ref, L, K, dtype, tol=None, inp=None):
    rtol, atol = tol or TOL[dtype]
    out, gv, gs = got
    ro, rgv, rgs = ref
    assert_close(f"{tag} output", out, ro, rtol, atol)
    if gv is not None:
        assert_close(f"{tag} grad_value", gv, rgv, rtol, atol)
        n = 3 * L * K
        extra = None
        if dtype == torch.float32 and inp is not None:
            extra = fp32_allowance(inp).reshape(gs.shape)[..., :n]
        assert_close(f"{tag} grad_loc", gs[..., :n], rgs[..., :n], rtol, atol, extra)
        assert_close(f"{tag} grad_logit", gs[..., n:], rgs[..., n:], rtol, atol)
