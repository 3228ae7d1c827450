"""GPU: the allocation-free backward (ops3d_fda_backward_noalloc, the library's static device
scratch as workspace) against the workspace backward (ops3d_fda_backward) on the same inputs,
for calls in a row on decreasing sizes -- each call finds the previous call's data in the
scratch, so whatever must start at zero has to be cleared by the call itself."""
from __future__ import annotations

import pytest
import torch

from fda_helpers import TOL, assert_close, log, run_oracle
from ops3d_amd import _C
from ops3d_amd.workloads import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu


def _backward_both(inp, device):
    args = [inp[k].to(device) for k in ("value", "spatial_shapes", "level_start_index", "sampling_loc_attn",
                                        "grad_output")]
    gv_ref, gs_ref = _C.flash_deform_attn_backward(*args, 64, inp["K"])
    gv, gs = _C.flash_deform_attn_backward_noalloc(*args, 64, inp["K"])
    torch.cuda.synchronize()
    return (gv, gs), (gv_ref, gs_ref)


def test_noalloc_matches_workspace_backward(gpu_device):
    # c2 (49 MiB of workspace), then c3 (18 MiB, two batch items, out-of-volume samples), then
    # c1 (fp32, 34 MiB of which the split scratch is the most), each in the same scratch
    for name, dt in (("c2", torch.bfloat16), ("c3", torch.bfloat16), ("c1", torch.float32)):
        w = WORKLOADS[name]
        inp = make_inputs(w, seed=3, dtype=dt)
        need = _C._lib.ops3d_fda_backward_workspace_bytes(
            {torch.float32: 0, torch.bfloat16: 2}[dt], w.B, w.S, w.G, w.D, w.L, w.nq, w.K)
        log(f"[case] noalloc {name} {dt}: workspace {need / 2**20:.1f} MiB")
        assert 0 < need <= 64 << 20
        (gv, gs), (gv_ref, gs_ref) = _backward_both(inp, gpu_device)
        # location/logit gradients are bitwise repeatable; grad_value sums may differ in order
        assert torch.equal(gs, gs_ref), f"{name}: grad_sampling_loc_attn differs"
        rtol, atol = TOL[dt]
        assert_close(f"{name} grad_value", gv, gv_ref.double().cpu().numpy(), rtol, atol)
        if name == "c1":   # and the smallest case against the float64 oracle as well
            _, rgv, _ = run_oracle(inp)
            assert_close("c1 grad_value vs oracle", gv, rgv, rtol, atol)


def test_noalloc_refuses_large_problems(gpu_device):
    w = WORKLOADS["c4"]   # 340 MiB of workspace: refused before any device work
    full = make_inputs(w, seed=0, dtype=torch.bfloat16)
    args = [full[k].to(gpu_device) for k in ("value", "spatial_shapes", "level_start_index",
                                             "sampling_loc_attn", "grad_output")]
    log("[case] noalloc c4 refused")
    with pytest.raises(ValueError, match="too large for the allocation-free backward"):
        _C.flash_deform_attn_backward_noalloc(*args, 64, w.K)
