"""Host-side API checks that need no GPU: the drop-in surface (ops3d / ops3d_amd exports,
findspec / findspec_bwd results, error contracts raised before any device work) and the
PyTorch path ms_deform_attn_core_pytorch_3d against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from ops3d_amd.workloads import WORKLOADS, level_meta, make_inputs, pack


def _ref_factors(N):
    return [i for i in range(1, N + 1) if N % i == 0]


def _ref_findspec(B, Q, G, C):
    # restatement of reference ops3d/flash_deform_attn.py:26-41 (full divisor scan)
    d_stride, multiplier = 8, 1
    for m in _ref_factors(B * Q):
        if m <= 64 and (m * G * C // d_stride) <= 512:
            multiplier = m
    return d_stride, multiplier * G * C // d_stride


def _ref_findspec_bwd(B, Q, G, C, max_tpb=256, max_mult=64):
    # restatement of reference ops3d/flash_deform_attn.py:44-62
    for d in (1, 2, 4, 8, 16, 32):
        if C % d == 0 and G * (C // d) <= max_tpb:
            d_stride = d
            break
    best = 1
    for m in _ref_factors(B * Q):
        if m <= max_mult and m * G * (C // d_stride) <= max_tpb:
            best = max(best, m)
    return d_stride, best * G * (C // d_stride)


def test_drop_in_imports():
    import ops3d
    import ops3d_amd
    from ops3d import FlashDeformAttnFunction, ms_deform_attn_core_pytorch_3d  # noqa: F401
    from ops3d.flash_deform_attn import findspec, findspec_bwd  # noqa: F401

    assert ops3d.FlashDeformAttnFunction is ops3d_amd.FlashDeformAttnFunction
    assert hasattr(ops3d, "_C")


@pytest.mark.parametrize("B,Q,G,C", [(1, 576, 8, 32), (1, 4608, 8, 32), (2, 200, 8, 32), (1, 73728, 8, 32),
                                     (1, 4096, 8, 64), (1, 294912, 8, 48), (5, 64, 4, 32), (1, 1, 4, 32),
                                     (3, 7, 6, 24), (1, 97, 16, 128)])
def test_findspec_matches_reference(B, Q, G, C):
    from ops3d.flash_deform_attn import factors, findspec, findspec_bwd

    assert factors(B * Q) == _ref_factors(B * Q)
    assert findspec(B, Q, G, C) == _ref_findspec(B, Q, G, C)
    assert findspec_bwd(B, Q, G, C) == _ref_findspec_bwd(B, Q, G, C)


def test_findspec_bwd_unfittable():
    from ops3d.flash_deform_attn import findspec_bwd

    with pytest.raises(RuntimeError, match="Cannot fit"):
        findspec_bwd(1, 8, 512, 1)


def test_cpu_tensors_raise():
    from ops3d import FlashDeformAttnFunction, _C

    if _C is None:
        pytest.skip("library not built")
    w = WORKLOADS["c1"]
    inp = make_inputs(w, seed=0, dtype=torch.float32)
    with pytest.raises(RuntimeError, match="CPU"):
        FlashDeformAttnFunction.apply(inp["value"], inp["spatial_shapes"], inp["level_start_index"],
                                      inp["sampling_loc_attn"], 1, 4, True)


def test_shape_mismatch_raises_value_error():
    from ops3d import FlashDeformAttnFunction, _C

    if _C is None:
        pytest.skip("library not built")
    st, lsi = level_meta(((4, 4, 4), (4, 4, 4)), "cpu")
    v = torch.rand(1, 128, 4, 32)
    bad = torch.rand(1, 64, 4, 16)  # L=1 packing for an L=2 value
    with pytest.raises(ValueError, match="does not match"):
        FlashDeformAttnFunction.apply(v, st, lsi, bad, 1, 4, True)


def test_missing_library_raises(monkeypatch):
    import ops3d_amd.flash_deform_attn as fda

    monkeypatch.setattr(fda, "_C", None)
    st, lsi = level_meta(((4, 4, 4),), "cpu")
    with pytest.raises(RuntimeError, match="not built"):
        fda.FlashDeformAttnFunction.apply(torch.rand(1, 64, 4, 32), st, lsi, torch.rand(1, 8, 4, 16), 1, 4, True)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_pytorch_path_matches_oracle(dtype):
    """ms_deform_attn_core_pytorch_3d with F.softmax'd logits == oracle (reference tests
    feed the PyTorch path post-softmax weights, tests/test_flash_deform_attn.py:38-40)."""
    from ops3d import ms_deform_attn_core_pytorch_3d

    shapes = ((4, 8, 16), (2, 4, 8))
    B, Q, G, D, L, K = 2, 50, 3, 8, 2, 4
    g = torch.Generator().manual_seed(0)
    S = sum(a * b * c for a, b, c in shapes)
    v = torch.randn(B, S, G, D, generator=g, dtype=dtype)
    loc = torch.rand(B, Q, G, L, K, 3, generator=g, dtype=dtype) * 1.2 - 0.1
    lg = torch.randn(B, Q, G, L, K, generator=g, dtype=dtype)
    attn = F.softmax(lg.flatten(-2), -1).unflatten(-1, (L, K))
    st, _ = level_meta(shapes, "cpu")
    out = ms_deform_attn_core_pytorch_3d(v, st, loc, attn)
    ref = oracle.forward(v.double().numpy(), shapes, pack(loc, lg).double().numpy(), K,
                         coord_mode=1 if dtype == torch.float32 else 0)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    np.testing.assert_allclose(out.double().numpy(), ref, rtol=tol, atol=tol)


def test_workload_byte_counts():
    # compulsory-traffic figures of the benchmark plan (MB): c4 113.2 / 188.7, c5 1071.6 / 1837.1
    c4 = WORKLOADS["c4"].algorithmic_bytes(2)
    assert round(c4["fwd"] / 1e6, 1) == 113.2 and round(c4["bwd"] / 1e6, 1) == 188.7
    c5 = WORKLOADS["c5"].algorithmic_bytes(2)
    assert round(c5["fwd"] / 1e6, 1) == 1071.6 and round(c5["bwd"] / 1e6, 1) == 1837.1
    assert WORKLOADS["c4"].S == 73728 and WORKLOADS["c5"].S == 598016 and WORKLOADS["c3"].S == 37376


def test_torch_extension_bound_and_checks():
    """The PyTorch extension module (C++ over the C ABI) is built and serves _C's tensor entry
    points, with the reference's error behaviour."""
    import ops3d_amd
    from ops3d_amd import _fda_torch

    C = ops3d_amd._C
    if C is None:
        pytest.skip("libops3d_fda.so not built")
    for name in ("flash_deform_attn_forward", "flash_deform_attn_backward", "forward_keep_head_major",
                 "backward_with_head_major"):
        assert getattr(C, name) is getattr(_fda_torch, name), name
    v = torch.zeros(1, 8, 1, 8)
    st = torch.tensor([[2, 2, 2]])
    lsi = torch.zeros(1, dtype=torch.long)
    with pytest.raises(RuntimeError, match="CPU"):
        C.flash_deform_attn_forward(v, st, lsi, torch.zeros(1, 2, 1, 16), 64, 4)
    with pytest.raises(TypeError):
        C.flash_deform_attn_forward(v.numpy(), st, lsi, torch.zeros(1, 2, 1, 16), 64, 4)
