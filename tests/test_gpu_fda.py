"""GPU parity of the gfx950 kernels against the float64 C oracle, through the public API
(FlashDeformAttnFunction -> ops3d_amd._C -> libops3d_fda.so).

Coverage follows the reference's tests (tests/test_flash_deform_attn.py,
tests/test_flash_deform_attn_stress.py): the benchmark configurations c1..c5, edge shapes
(1^3 volumes, anisotropic, uneven levels, B=64), K in {4, 8}, L up to 5, D in {32, 48, 64},
fp32/fp16/bf16, out-of-volume samples, value scales 0 / 1e-6 / 1e4, zero upstream gradient,
im2col_step invariance and the error contracts.  Tolerances: fp32 rtol 1e-5 / atol 1e-6,
bf16 and fp16 rtol 2e-2 / atol 2e-2 (fda_helpers.TOL).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fda_helpers import TOL, assert_close, compare_all, log, random_inputs, run_gpu, run_oracle
from ops3d_amd import FlashDeformAttnFunction
from ops3d_amd.workloads import WORKLOADS, level_meta, make_inputs

pytestmark = pytest.mark.gpu


def _check(tag, inp, device, dtype, backward=True, tol=None, im2col_step=64):
    log(f"[case] {tag}: shapes={inp['shapes']} value={tuple(inp['value'].shape)} "
        f"sla={tuple(inp['sampling_loc_attn'].shape)} dtype={dtype} bwd={backward}")
    got = run_gpu(inp, device, backward=backward, im2col_step=im2col_step)
    ref = run_oracle(inp, backward=backward)
    compare_all(tag, got, ref, len(inp["shapes"]), inp["K"], dtype, tol, inp=inp)


# --- benchmark configurations --------------------------------------------------------------
def test_c1_fp32(gpu_device):
    w = WORKLOADS["c1"]
    inp = make_inputs(w, seed=0, dtype=torch.float32)
    _check("c1 fp32", inp, gpu_device, torch.float32)


def test_golden_fixture_fp32(gpu_device):
    import os

    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_small.npz"))
    inp = {
        "value": torch.from_numpy(fx["value"]),
        "sampling_loc_attn": torch.from_numpy(fx["sampling_loc_attn"]),
        "grad_output": torch.from_numpy(fx["grad_output"]),
        "shapes": [tuple(int(t) for t in s) for s in fx["shapes"]],
        "K": int(fx["K"]),
    }
    log("[case] golden c1_small fp32")
    out, gv, gs = run_gpu(inp, gpu_device)
    # fixture inputs are exact in fp32; the fp32 bar: rtol 1e-5 / atol 1e-6, plus the rounding
    # allowance of the location gradients (oracle.fp32_loc_allowance)
    rtol, atol = TOL[torch.float32]
    assert_close("golden output", out, fx["output"], rtol, atol)
    assert_close("golden grad_value", gv, fx["grad_value"], rtol, atol)
    assert_close("golden grad_sla", gs, fx["grad_sampling_loc_attn"], rtol, atol,
                 __import__("fda_helpers").fp32_allowance(inp))


@pytest.mark.parametrize("name", ["c2", "c3"])
def test_bf16_configs(gpu_device, name):
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=0, dtype=torch.bfloat16)
    _check(f"{name} bf16", inp, gpu_device, torch.bfloat16)


def test_c4_bf16_full(gpu_device):
    w = WORKLOADS["c4"]
    inp = make_inputs(w, seed=0, dtype=torch.bfloat16)
    _check("c4 bf16", inp, gpu_device, torch.bfloat16)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_c5_query_slice(gpu_device, dt):
    """c5 at full size on the GPU.  Forward and location/logit gradients are per query, so a
    query slice is checked directly; grad_value is checked exactly by zeroing the upstream
    gradient outside the slice (the kernel still scatters from every query)."""
    w = WORKLOADS["c5"]
    inp = make_inputs(w, seed=0, dtype=dt)
    nq = 2048
    sel = torch.arange(0, w.nq, w.nq // nq)[:nq]
    mask = torch.zeros(w.nq, dtype=torch.bool)
    mask[sel] = True
    go = inp["grad_output"].clone()
    go[:, ~mask] = 0
    inp["grad_output"] = go
    backward = dt == torch.bfloat16
    log(f"[case] c5 {dt} full-size, oracle on {nq} queries, backward={backward}")
    out, gv, gs = run_gpu(inp, gpu_device, backward=backward)
    sub = dict(inp)
    sub["sampling_loc_attn"] = inp["sampling_loc_attn"][:, sel]
    sub["grad_output"] = go[:, sel]
    ref = run_oracle(sub, backward=backward)
    rtol, atol = TOL[dt]
    assert_close("c5 output", out[:, sel.to(out.device)], ref[0], rtol, atol)
    if backward:
        assert_close("c5 grad_value", gv, ref[1], rtol, atol)
        assert_close("c5 grad_sla", gs[:, sel.to(gs.device)], ref[2], rtol, atol)


def _paired_inputs(G, D, dt, Q=96, seed=7, B=1):
    """A 32x64x256 level (33.5 MB per head with 64-byte rows: stored as x-pair lines in the
    head-major copy) and a small one; queries 0..26 sample every corner, edge and face centre
    of the unit cube in both levels (pixel -0.5 / size-0.5: base corners at -1 and at the last
    voxel, so the level's first voxel is read through line -1 and the last voxel's x-neighbour
    is outside)."""
    from ops3d_amd.workloads import pack

    shapes = [(32, 64, 256), (4, 8, 16)]
    g = torch.Generator().manual_seed(seed)
    S = sum(a * b * c for a, b, c in shapes)
    v = torch.randn(B, S, G, D, generator=g)
    loc = torch.rand(B, Q, G, 2, 4, 3, generator=g)
    pts = torch.tensor([(x, y, z) for z in (0.0, 0.5, 1.0) for y in (0.0, 0.5, 1.0) for x in (0.0, 0.5, 1.0)])
    loc[:, : len(pts)] = pts[None, :, None, None, None, :]
    loc[:, len(pts): 2 * len(pts), :, :, 0] = pts[None, :, None, None, :] * 0.999   # just inside
    lg = torch.randn(B, Q, G, 2, 4, generator=g)
    go = torch.randn(B, Q, G * D, generator=g)
    return {"value": v.to(dt), "sampling_loc_attn": pack(loc, lg).to(dt), "grad_output": go.to(dt),
            "shapes": shapes, "K": 4}


@pytest.mark.parametrize("dt,D,G,B", [(torch.bfloat16, 32, 8, 1), (torch.float16, 32, 2, 1), (torch.float32, 16, 2, 1),
                                      (torch.bfloat16, 32, 2, 2)])
def test_paired_level(gpu_device, dt, D, G, B):
    inp = _paired_inputs(G, D, dt, B=B)
    _check(f"paired level {dt} D={D} G={G} B={B}", inp, gpu_device, dt)


def test_paired_level_backward_own_copy(gpu_device):
    """_C.flash_deform_attn_backward (no forward workspace): the backward makes the paired copy."""
    from ops3d_amd import _C

    inp = _paired_inputs(8, 32, torch.bfloat16)
    log("[case] paired level, _C backward with its own head-major copy")
    st, lsi = level_meta(inp["shapes"], gpu_device)
    v = inp["value"].to(gpu_device)
    s = inp["sampling_loc_attn"].to(gpu_device)
    go = inp["grad_output"].to(gpu_device)
    gv, gs = _C.flash_deform_attn_backward(v, st, lsi, s, go, 64, 4, 1, 256)
    torch.cuda.synchronize()
    _, rgv, rgs = run_oracle(inp)
    assert_close("grad_value", gv, rgv, *TOL[torch.bfloat16])
    assert_close("grad_sla", gs, rgs, *TOL[torch.bfloat16])


def test_reordered_levels_large(gpu_device):
    """value holding the levels in reverse order (level_start_index = [n1, 0]): not the layout
    whose large levels are paired, so every level stays at its own start; checked against the
    oracle on the same data in the usual order."""
    inp = _paired_inputs(8, 32, torch.bfloat16, Q=64)
    n0 = 32 * 64 * 256
    log("[case] reordered levels, large volume")
    v = inp["value"]
    v_rev = torch.cat([v[:, n0:], v[:, :n0]], dim=1).to(gpu_device).requires_grad_(True)
    st = torch.tensor(inp["shapes"], dtype=torch.int64, device=gpu_device)
    lsi = torch.tensor([v.shape[1] - n0, 0], dtype=torch.int64, device=gpu_device)
    s = inp["sampling_loc_attn"].to(gpu_device).requires_grad_(True)
    out = FlashDeformAttnFunction.apply(v_rev, st, lsi, s, 64, 4, True)
    out.backward(inp["grad_output"].to(gpu_device))
    torch.cuda.synchronize()
    ref_out, ref_gv, ref_gs = run_oracle(inp)
    gv = torch.cat([v_rev.grad[:, -n0:], v_rev.grad[:, :-n0]], dim=1)
    assert_close("output", out.detach(), ref_out, *TOL[torch.bfloat16])
    assert_close("grad_value", gv, ref_gv, *TOL[torch.bfloat16])
    assert_close("grad_sla", s.grad, ref_gs, *TOL[torch.bfloat16])


# --- reference stress shapes (tests/test_flash_deform_attn_stress.py:47-97) ------------------
EDGE_SHAPE_CASES = [
    (1, (1, 1, 1), 1), (1, (4, 4, 4), 1), (1, (7, 7, 7), 1), (1, (8, 8, 8), 1),
    (1, (16, 16, 16), 1), (2, (4, 4, 4), 1), (2, (8, 8, 8), 1), (3, (4, 4, 4), 1),
    (3, (16, 16, 16), 1), (4, (8, 8, 8), 2), (5, (4, 4, 4), 1), (1, (32, 16, 8), 1),
    (2, (16, 8, 4), 1), (1, (8, 4, 2), 1), (2, (32, 16, 8), 1), (1, (8, 8, 8), 64),
]


@pytest.mark.parametrize("L,spatial,B", EDGE_SHAPE_CASES)
@pytest.mark.parametrize("K", [4, 8])
def test_edge_shapes_fp32(gpu_device, L, spatial, B, K):
    d, h, w = spatial
    Q = max(1, min(64, d * h * w))
    inp = random_inputs([spatial] * L, B, Q, 4, 32, K, torch.float32, seed=42)
    _check(f"edge L={L} {spatial} B={B} K={K}", inp, gpu_device, torch.float32, im2col_step=B)


def test_uneven_levels(gpu_device):
    inp = random_inputs([(1, 1, 1), (64, 64, 64)], 1, 64, 4, 32, 4, torch.float32, seed=42)
    _check("uneven 1^3+64^3", inp, gpu_device, torch.float32)


def test_anisotropic_multilevel(gpu_device):
    inp = random_inputs([(32, 16, 8), (16, 8, 4)], 1, 64, 4, 32, 4, torch.float32, seed=42)
    _check("anisotropic", inp, gpu_device, torch.float32)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Q", [300, 1200])
def test_thin_levels_atomic_bucketing(gpu_device, dt, Q):
    """Levels one voxel thick and thousands long are cut into more tiles than the bucketing
    matrix holds (S/16 + 64 per head), so the backward buckets them with global atomics -- in
    the one-block-per-head launch (Q = 300: 2400 samples per head) and across blocks (Q = 1200)."""
    inp = random_inputs([(1, 1, 4096), (1, 2048, 1)], 1, Q, 8, 32, 4, dt, seed=8)
    _check(f"thin levels {dt} Q={Q}", inp, gpu_device, dt)


def test_out_of_volume_fp32(gpu_device):
    inp = random_inputs([(6, 5, 7), (3, 2, 4)], 2, 300, 8, 32, 4, torch.float32, seed=5, lo=-0.3, hi=1.3)
    _check("oob fp32", inp, gpu_device, torch.float32)


def test_all_samples_outside_volume(gpu_device):
    """Every sample outside [-1, size): all keys invalid, grad_value all zero."""
    inp = random_inputs([(6, 5, 7), (3, 2, 4)], 1, 200, 8, 32, 4, torch.float32, seed=6, lo=1.6, hi=2.5)
    _check("all outside fp32", inp, gpu_device, torch.float32)


# --- seeded random configurations ------------------------------------------------------------
def _random_config(seed):
    """A small random problem: 1-4 levels of 1-24 voxels per axis, B 1-3, Q 1-400, G in
    {1, 2, 4, 8, 16}, D in {16, 32, 48}, K 1-8, some samples outside the volume.  Across the
    seeds this mixes split and unsplit tile launches, both tile orders and all XCD mappings."""
    r = np.random.default_rng(1000 + seed)
    L = int(r.integers(1, 5))
    shapes = [tuple(int(x) for x in r.integers(1, 25, size=3)) for _ in range(L)]
    B = int(r.integers(1, 4))
    Q = int(r.integers(1, 401))
    G = int(r.choice([1, 2, 4, 8, 16]))
    D = int(r.choice([16, 32, 48]))
    K = int(r.integers(1, 9))
    dt = torch.float32 if seed % 2 == 0 else torch.bfloat16
    return shapes, B, Q, G, D, K, dt


@pytest.mark.parametrize("seed", range(12))
def test_random_configs(gpu_device, seed):
    shapes, B, Q, G, D, K, dt = _random_config(seed)
    inp = random_inputs(shapes, B, Q, G, D, K, dt, seed=seed, lo=-0.1, hi=1.1)
    _check(f"random #{seed}: L={len(shapes)} B={B} Q={Q} G={G} D={D} K={K}", inp, gpu_device, dt,
           im2col_step=B)


# --- head widths, head counts (XCD mappings), dtypes ---------------------------------------
@pytest.mark.parametrize("D", [8, 16, 24, 32, 48, 64, 96, 128])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_head_width(gpu_device, D, dt):
    inp = random_inputs([(5, 6, 7), (3, 3, 4)], 1, 150, 8, D, 4, dt, seed=D)
    _check(f"D={D} {dt}", inp, gpu_device, dt)


@pytest.mark.parametrize("G", [1, 2, 3, 4, 6, 8, 16, 24])
def test_head_count(gpu_device, G):
    inp = random_inputs([(6, 6, 6), (3, 3, 3)], 2, 333, G, 32, 4, torch.float32, seed=G)
    _check(f"G={G}", inp, gpu_device, torch.float32)


def test_reference_forward_params_fp16(gpu_device):
    """Reference default_forward_params (tests/conftest.py:27-57) with Lq reduced 4x:
    D=64, L=4, K=8, levels 64^3/32^3/16^3/8^3, fp16."""
    shapes = [(64, 64, 64), (32, 32, 32), (16, 16, 16), (8, 8, 8)]
    inp = random_inputs(shapes, 1, 1024, 8, 64, 8, torch.float16, seed=42)
    _check("ref fwd params fp16", inp, gpu_device, torch.float16, backward=False)


def test_reference_backward_params_fp16(gpu_device):
    """Reference default_backward_params (tests/conftest.py:60-87), D=48, L=2, K=4,
    levels 64^3/32^3, Lq reduced to 8192."""
    inp = random_inputs([(64, 64, 64), (32, 32, 32)], 1, 8192, 8, 48, 4, torch.float16, seed=42)
    _check("ref bwd params fp16", inp, gpu_device, torch.float16)


# --- numerics (stress :240-377, :385-405) -------------------------------------------------
def test_zero_values(gpu_device):
    inp = random_inputs([(4, 4, 4)], 1, 64, 4, 32, 4, torch.float32, value_scale=0.0)
    out, _, _ = run_gpu(inp, gpu_device, backward=False)
    assert torch.all(out == 0)


@pytest.mark.parametrize("scale", [1e-6, 1e4])
def test_value_scales_fp32(gpu_device, scale):
    inp = random_inputs([(4, 4, 4)], 1, 64, 4, 32, 4, torch.float32, value_scale=scale)
    rtol, atol = TOL[torch.float32]
    _check(f"scale {scale}", inp, gpu_device, torch.float32, tol=(rtol, atol * max(1.0, scale)))


def test_zero_upstream_grad_gives_zero_grads(gpu_device):
    inp = random_inputs([(4, 4, 4), (4, 4, 4)], 1, 64, 4, 32, 4, torch.float32)
    inp["grad_output"] = torch.zeros_like(inp["grad_output"])
    _, gv, gs = run_gpu(inp, gpu_device)
    assert gv.abs().max().item() == 0 and gs.abs().max().item() == 0


def test_im2col_step_invariance_and_determinism(gpu_device):
    inp = random_inputs([(5, 5, 5), (2, 3, 4)], 4, 77, 8, 32, 4, torch.bfloat16, seed=9)
    outs = [run_gpu(inp, gpu_device, backward=False, im2col_step=s)[0] for s in (1, 2, 4, 64)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_backward_repeatable(gpu_device):
    """grad_sampling_loc_attn is bitwise identical across runs.  grad_value rows are fp32 sums
    whose order follows the order in which blocks fill a tile's entry list, so runs may differ
    by fp32 rounding of the sums (relative to the sum of the terms' magnitudes, ~1 here), seen
    after the bf16 rounding as one bf16 ulp, or a few ulps of a row that nearly cancels."""
    inp = random_inputs([(8, 8, 8), (4, 4, 4)], 2, 500, 8, 32, 4, torch.bfloat16, seed=11)
    a = run_gpu(inp, gpu_device)
    b = run_gpu(inp, gpu_device)
    assert torch.equal(a[2], b[2])
    ga, gb = a[1].float(), b[1].float()
    tol = torch.maximum(ga.abs(), gb.abs()) * 2.0 ** -7 + 1e-5   # >= one bf16 ulp of either
    d = (ga - gb).abs()
    assert (d <= tol).all(), f"max diff {d.max().item():.3e} at |g| {ga.flatten()[d.argmax()].item():.3e}"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_backward_accumulate_f32(gpu_device, dt):
    """_C.flash_deform_attn_backward_accumulate adds the value gradient into an fp32 buffer."""
    from ops3d_amd import _C

    inp = random_inputs([(6, 5, 4), (3, 3, 2)], 1, 200, 8, 32, 4, dt, seed=3)
    st, lsi = level_meta(inp["shapes"], gpu_device)
    v = inp["value"].to(gpu_device)
    s = inp["sampling_loc_attn"].to(gpu_device)
    go = inp["grad_output"].to(gpu_device)
    acc = torch.full(v.shape, 0.25, dtype=torch.float32, device=gpu_device)
    g1 = _C.flash_deform_attn_backward_accumulate(v, st, lsi, s, go, acc, 64, 4)
    g2 = _C.flash_deform_attn_backward_accumulate(v, st, lsi, s, go, acc, 64, 4)
    torch.cuda.synchronize()
    _, rgv, rgs = run_oracle(inp)
    rtol, atol = TOL[torch.float32] if dt == torch.float32 else (1e-5, 1e-5)
    assert_close("accumulated grad_value", acc, 0.25 + 2 * rgv, rtol, 2 * atol)
    assert torch.equal(g1, g2)
    assert_close("grad_sla", g1, rgs, *TOL[dt], extra=None if dt != torch.float32 else
                 __import__("fda_helpers").fp32_allowance(inp))


@pytest.mark.parametrize("dt,G,D,lo,hi", [(torch.bfloat16, 8, 32, 0.0, 1.0), (torch.float32, 8, 32, -0.1, 1.1),
                                          (torch.float32, 3, 16, -0.1, 1.1), (torch.float16, 2, 64, 0.0, 1.0)])
def test_scatter_baseline(gpu_device, dt, G, D, lo, hi):
    """The measurement baseline (the reference's fp32 atomic scatter of grad_value at its own lane
    layout, libops3d_fda_bench.so) computes the same value gradient as the oracle, to fp32
    rounding of its sums."""
    from ops3d_amd import _bench_lib

    inp = random_inputs([(6, 5, 8), (3, 3, 4)], 2, 150, G, D, 4, dt, seed=5, lo=lo, hi=hi)
    st, lsi = level_meta(inp["shapes"], gpu_device)
    gv = _bench_lib.ref_scatter(inp["value"].to(gpu_device), st, lsi, inp["sampling_loc_attn"].to(gpu_device),
                                inp["grad_output"].to(gpu_device), 4)
    torch.cuda.synchronize()
    _, rgv, _ = run_oracle(inp)
    assert gv.dtype == torch.float32
    assert_close("scatter baseline grad_value", gv, rgv, 1e-5, 1e-5)


def test_empty_queries(gpu_device):
    inp = random_inputs([(4, 4, 4)], 1, 0, 4, 32, 4, torch.float32)
    out, gv, gs = run_gpu(inp, gpu_device)
    assert out.shape == (1, 0, 128) and gs.shape == (1, 0, 4, 16)
    assert torch.all(gv == 0)


# --- error contracts (stress :151-232) ----------------------------------------------------
def _apply(inp, device, step=1):
    st, lsi = level_meta(inp["shapes"], device)
    return FlashDeformAttnFunction.apply(
        inp["value"].to(device), st, lsi, inp["sampling_loc_attn"].to(device), step, inp["K"], True
    )


def test_error_batch_not_divisible(gpu_device):
    inp = random_inputs([(4, 4, 4), (4, 4, 4)], 5, 64, 4, 32, 4, torch.float32)
    with pytest.raises(RuntimeError, match="must divide"):
        _apply(inp, gpu_device, step=2)


def test_error_six_levels(gpu_device):
    inp = random_inputs([(4, 4, 4)] * 6, 1, 64, 4, 32, 4, torch.float32)
    with pytest.raises(ValueError, match="invalid number of scales"):
        _apply(inp, gpu_device)


def test_error_shape_mismatch(gpu_device):
    inp = random_inputs([(4, 4, 4), (4, 4, 4)], 1, 64, 4, 32, 4, torch.float32)
    inp["sampling_loc_attn"] = inp["sampling_loc_attn"][..., :16].contiguous()
    with pytest.raises(ValueError, match="does not match"):
        _apply(inp, gpu_device)


def test_error_non_contiguous(gpu_device):
    inp = random_inputs([(4, 4, 4)], 1, 64, 4, 32, 4, torch.float32)
    st, lsi = level_meta(inp["shapes"], gpu_device)
    v = inp["value"].to(gpu_device).transpose(1, 2).contiguous().transpose(1, 2)
    with pytest.raises(RuntimeError, match="contiguous"):
        FlashDeformAttnFunction.apply(v, st, lsi, inp["sampling_loc_attn"].to(gpu_device), 1, 4, True)


def test_error_unsupported_channels(gpu_device):
    inp = random_inputs([(4, 4, 4)], 1, 8, 2, 20, 4, torch.bfloat16)
    with pytest.raises(ValueError, match="unsupported channels"):
        _apply(inp, gpu_device)


@pytest.mark.gpu
def test_gather_ceiling_probe(gpu_device):
    """The measurement library's random-gather probe runs and folds what it loads: a buffer of
    ones gives every thread the fold of its loads (iters * (1 ^ 1 ^ 1 ^ 1) = 0)."""
    from ops3d_amd import _bench_lib

    src = torch.ones(1 << 18, dtype=torch.int32, device=gpu_device)
    out = torch.full((8 * 256,), 7, dtype=torch.int32, device=gpu_device)
    for g in (4, 8, 32, 64):
        _bench_lib.gather(src, g, 8, 16, out)
        torch.cuda.synchronize()
        assert bool((out == 0).all())
