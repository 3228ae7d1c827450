"""3-D RoI Align: the CPU oracle pinned (closed forms, nearest rounding, the adjoint identity,
batch-index guard) and the GPU kernels against it (marked gpu).

The reference ships no RoI Align tests; its semantics are those of
csrc/cuda/roi_align_3d_cuda_kernel.cuh:27-220 and csrc/cuda/interpolation_helpers_3d.h:25-260."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import roi_align3d as O


def _rois(R, N, size, seed, lo=-2.0, hi=None):
    r = np.random.default_rng(seed)
    D, H, W = size
    hi = hi if hi is not None else max(D, H, W) + 2.0
    p = r.uniform(lo, hi, size=(R, 2, 3))
    a, b = np.minimum(p[:, 0], p[:, 1]), np.maximum(p[:, 0], p[:, 1])
    bi = r.integers(0, N, size=(R, 1)).astype(np.float64)
    return np.concatenate([bi, a, b], 1).astype(np.float32)   # (b, x1, y1, z1, x2, y2, z2)


# --- oracle pinning (CPU) --------------------------------------------------------------------
def test_constant_and_linear_fields():
    N, C, D, H, W = 1, 2, 8, 9, 10
    z, y, x = np.meshgrid(np.arange(D), np.arange(H), np.arange(W), indexing="ij")
    lin = 0.5 * x + 0.25 * y - 0.75 * z + 3.0
    feat = np.stack([np.full((D, H, W), 2.5), lin])[None]
    # rois well inside [0, size-1] on every axis (x 1..8, y 1..7, z 1..6): every sample interpolates
    rois = np.array([[0, 1.0, 1.0, 1.0, 8.0, 7.0, 6.0], [0, 2.2, 1.5, 1.25, 5.0, 6.5, 4.75]], np.float32)
    for sr in (1, 2, 3):
        out = O.forward(feat, rois, (3, 2, 4), 1.0, sr)
        assert np.allclose(out[:, 0], 2.5)
        for r in range(2):
            x1, y1, z1, x2, y2, z2 = rois[r, 1:]
            for pd in range(3):
                for ph in range(2):
                    for pw in range(4):
                        cx = x1 + (pw + 0.5) * (x2 - x1) / 4
                        cy = y1 + (ph + 0.5) * (y2 - y1) / 2
                        cz = z1 + (pd + 0.5) * (z2 - z1) / 3
                        want = 0.5 * cx + 0.25 * cy - 0.75 * cz + 3.0   # linear: mean = value at the centre
                        assert abs(out[r, 1, pd, ph, pw] - want) < 1e-5


def test_nearest_rounds_half_down_and_clamps():
    D = H = W = 4
    feat = np.arange(D * H * W, dtype=np.float64).reshape(1, 1, D, H, W)
    # one sample per bin at the roi centre: roi [c - 0.5, c + 0.5] -> sample at c
    def at(x, y, z):
        roi = np.array([[0, x - 0.5, y - 0.5, z - 0.5, x + 0.5, y + 0.5, z + 0.5]], np.float32)
        return O.forward(feat, roi, (1, 1, 1), 1.0, 1, order=0)[0, 0, 0, 0, 0]
    assert at(1.3, 2.0, 0.0) == (0 * H + 2) * W + 1      # x frac .3 -> x0
    assert at(1.5, 2.0, 0.0) == (0 * H + 2) * W + 1      # .5 -> x0 (hx >= .5 is tested first)
    assert at(1.7, 2.0, 0.0) == (0 * H + 2) * W + 2      # .7 -> x1
    assert at(3.4, 3.9, 2.6) == (3 * H + 3) * W + 3      # beyond size-1: clamped to the last voxel
    assert at(-0.6, 0.0, 0.0) == 0                       # below 0 (but >= -1): clamped to 0


def test_out_of_range_samples_and_batch_guard():
    feat = np.ones((1, 1, 4, 4, 4))
    # a roi entirely beyond the volume (samples > size) reads nothing
    far = np.array([[0, 10, 10, 10, 12, 12, 12]], np.float32)
    assert np.all(O.forward(feat, far, (2, 2, 2), 1.0, 2) == 0)
    bad = np.array([[3, 0, 0, 0, 2, 2, 2]], np.float32)      # batch index 3 of 1
    assert np.all(O.forward(feat, bad, (2, 2, 2), 1.0, 2) == 0)


@pytest.mark.parametrize("order,sr", [(1, 0), (1, 2), (0, 1)])
def test_adjoint_identity(order, sr):
    """The backward is the adjoint of the (linear) forward: <F(x), g> == <x, B(g)>."""
    r = np.random.default_rng(order * 10 + sr)
    shape = (2, 3, 5, 6, 7)
    x = r.normal(size=shape)
    rois = _rois(6, 2, shape[2:], seed=5)
    pooled = (2, 3, 2)
    g = r.normal(size=(6, 3) + pooled)
    lhs = float(np.sum(O.forward(x, rois, pooled, 0.9, sr, order) * g))
    rhs = float(np.sum(x * O.backward(g, rois, shape, 0.9, sr, order)))
    assert abs(lhs - rhs) < 1e-9 * max(1.0, abs(lhs))


# --- GPU ---------------------------------------------------------------------------------------
CASES = [
    # N, C, (D, H, W), R, pooled, scale, sampling_ratio, order, dtype
    (2, 8, (8, 12, 16), 20, (3, 3, 3), 1.0, 2, 1, torch.float32),
    (2, 8, (8, 12, 16), 20, (2, 3, 4), 0.5, 0, 1, torch.float32),       # adaptive grid
    (1, 3, (5, 6, 7), 15, (2, 2, 2), 1.0, 1, 0, torch.float32),         # nearest, C % 4 != 0
    (2, 16, (10, 10, 10), 30, (4, 4, 4), 1.0, 2, 1, torch.bfloat16),
    (1, 4, (6, 8, 8), 12, (3, 2, 2), 2.0, 0, 1, torch.float16),
    (1, 70, (6, 7, 9), 10, (2, 2, 3), 1.0, 2, 1, torch.float32),       # a partial 64-channel group
    (2, 130, (5, 9, 11), 8, (3, 2, 2), 1.0, 3, 0, torch.bfloat16),     # nearest, 130 channels
    (1, 5, (6, 7, 9), 6, (9, 8, 8), 1.0, 1, 1, torch.float32),          # 576 bins: atomic backward
    (1, 3, (6, 7, 9), 6, (2, 65, 2), 1.0, 1, 0, torch.bfloat16),        # 65 bins on y: atomic backward
    (1, 6, (12, 14, 16), 10, (2, 3, 2), 1.0, 4, 1, torch.float32),      # 4 samples per axis: separable, 8 taps
    (1, 5, (12, 14, 16), 10, (1, 2, 1), 1.0, 0, 1, torch.float32),      # adaptive, wide bins: > 8 taps
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CASES)))
def test_gpu_matches_oracle(gpu_device, case):
    from fda_helpers import TOL, assert_close, log

    from ops3d_amd.roi_align import roi_align_3d

    N, C, size, R, pooled, scale, sr, order, dt = CASES[case]
    log(f"[case] roi_align3d #{case}: N={N} C={C} size={size} R={R} pooled={pooled} sr={sr} order={order} {dt}")
    r = np.random.default_rng(case)
    x = torch.from_numpy(r.normal(size=(N, C) + size).astype(np.float32)).to(dt)
    rois_np = _rois(R, N, tuple(int(v / scale) for v in size), seed=100 + case)
    rois = torch.from_numpy(rois_np).to(dt)
    xg = x.to(gpu_device).requires_grad_(True)
    out = roi_align_3d(xg, rois.to(gpu_device), pooled, scale, sr, order)
    g = torch.from_numpy(r.normal(size=tuple(out.shape)).astype(np.float32)).to(dt)
    out.backward(g.to(gpu_device))
    torch.cuda.synchronize()
    want = O.forward(x.double().numpy(), rois.double().numpy(), pooled, scale, sr, order)
    gwant = O.backward(g.double().numpy(), rois.double().numpy(), x.shape, scale, sr, order)
    rtol, atol = TOL[dt]
    assert out.dtype == dt and tuple(out.shape) == (R, C) + pooled
    assert_close("roi_align output", out.detach(), want, rtol, atol)
    # gradients: fp32 sums of up to count * 8 terms per voxel, added by atomics in any order
    assert_close("roi_align grad", xg.grad, gwant, rtol, atol * (10 if dt == torch.float32 else 1))


def test_backward_workspace_sizes():
    """The gather backward (at most 64 bins per axis and 384 in all) needs the per-roi axis
    weight tables, R * (D*PD + H*PH + W*PW + D + H + W) words rounded up to 16 bytes, and a
    channels-last copy of grad_output; the atomic one an fp32 buffer of grad_input's size (the
    C ABI, no GPU needed)."""
    from ops3d_amd import _extension

    lib = _extension.load_library()
    f = lib.ops3d_roi_align3d_backward_workspace_bytes

    def tables(R, D, H, W, PD, PH, PW):
        return (R * (D * PD + H * PH + W * PW + D + H + W) * 4 + 15) // 16 * 16

    assert f(2, 2, 256, 32, 64, 64, 512, 7, 7, 7) == tables(512, 32, 64, 64, 7, 7, 7) + 512 * 343 * 256 * 2
    assert f(0, 1, 5, 6, 7, 9, 6, 6, 8, 8) == tables(6, 6, 7, 9, 6, 8, 8) + 6 * 384 * 5 * 4
    assert f(1, 1, 3, 6, 7, 9, 5, 1, 1, 3) == tables(5, 6, 7, 9, 1, 1, 3) + 5 * 3 * 3 * 2
    assert f(0, 1, 5, 6, 7, 9, 0, 6, 8, 8) == 0                          # no rois: nothing
    assert f(0, 1, 5, 6, 7, 9, 6, 7, 8, 8) == 5 * 6 * 7 * 9 * 4          # 448 bins: atomic path
    assert f(2, 1, 3, 6, 7, 9, 2, 2, 65, 2) == 3 * 6 * 7 * 9 * 4
    assert f(2, 1, 3, 6, 7, 9, 0, 2, 65, 2) == 3 * 6 * 7 * 9 * 4          # atomic path, no rois


@pytest.mark.gpu
def test_gpu_backward_repeatable(gpu_device):
    """The gather backward sums each voxel's rois in roi order: the same bits on every run."""
    from ops3d_amd.roi_align import roi_align_3d

    r = np.random.default_rng(3)
    x = torch.from_numpy(r.normal(size=(2, 20, 8, 12, 16)).astype(np.float32)).to(gpu_device)
    rois = torch.from_numpy(_rois(40, 2, (8, 12, 16), seed=9)).to(gpu_device)
    g = torch.randn(40, 20, 3, 3, 3, device=gpu_device)
    grads = []
    for _ in range(3):
        xg = x.clone().requires_grad_(True)
        roi_align_3d(xg, rois, (3, 3, 3), 1.0, 2, 1).backward(g)
        grads.append(xg.grad)
    torch.cuda.synchronize()
    assert torch.equal(grads[0], grads[1]) and torch.equal(grads[0], grads[2])


@pytest.mark.gpu
def test_gpu_wide_bins(gpu_device):
    """Rows whose bins span more than 64 voxels on y (adaptive grid, one bin): the backward's
    per-sample path; and bins of one voxel or less (many samples per tap) on the same volume."""
    from fda_helpers import assert_close, log

    from ops3d_amd.roi_align import roi_align_3d

    log("[case] roi_align3d wide bins (per-sample path) and dense samples")
    r = np.random.default_rng(7)
    x = torch.from_numpy(r.normal(size=(1, 3, 4, 80, 6)).astype(np.float32))
    rois = torch.tensor([[0, 0.0, 0.0, 0.0, 5.0, 79.0, 3.0],      # y extent 79, one bin: 79 samples
                         [0, 1.0, -0.5, 0.5, 4.5, 78.5, 2.5],
                         [0, 2.0, 10.0, 1.0, 2.5, 10.8, 1.4]])     # sub-voxel roi, 8 samples per axis
    for pooled, sr in (((1, 1, 1), 0), ((2, 1, 2), 0), ((1, 2, 1), 8)):
        xg = x.to(gpu_device).requires_grad_(True)
        out = roi_align_3d(xg, rois.to(gpu_device), pooled, 1.0, sr, 1)
        g = torch.from_numpy(r.normal(size=tuple(out.shape)).astype(np.float32))
        out.backward(g.to(gpu_device))
        torch.cuda.synchronize()
        want = O.forward(x.double().numpy(), rois.double().numpy(), pooled, 1.0, sr, 1)
        gwant = O.backward(g.double().numpy(), rois.double().numpy(), x.shape, 1.0, sr, 1)
        assert_close(f"wide-bin output {pooled} sr={sr}", out.detach(), want, 1e-5, 1e-6)
        assert_close(f"wide-bin grad {pooled} sr={sr}", xg.grad, gwant, 1e-5, 1e-5)


@pytest.mark.gpu
def test_gpu_module_edges(gpu_device):
    from ops3d_amd import _C
    from ops3d_amd.roi_align import RoIAlign

    m = RoIAlign((2, 2, 2), 1.0, 2)
    x = torch.randn(1, 4, 4, 4, 4, device=gpu_device)
    rois = torch.tensor([[0, 0, 0, 0, 3, 3, 3], [5, 0, 0, 0, 3, 3, 3]], dtype=torch.float32, device=gpu_device)
    out = m(x, rois)
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0)                                    # batch index 5 of 1: nothing
    want = O.forward(x.cpu().double().numpy(), rois.cpu().numpy(), (2, 2, 2), 1.0, 2)
    assert np.allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6)
    empty = m(x, torch.zeros(0, 7, device=gpu_device))
    assert tuple(empty.shape) == (0, 4, 2, 2, 2)
    with pytest.raises(RuntimeError, match="CPU"):
        _C.roi_align_3d_forward(x.cpu(), rois.cpu(), torch.empty(2, 4, 2, 2, 2), 2, 2, 2, 1.0, 2, 1)
    with pytest.raises(RuntimeError, match="size_rois should be 7"):
        _C.roi_align_3d_forward(x, rois[:, :6], torch.empty(2, 4, 2, 2, 2, device=gpu_device), 2, 2, 2, 1.0, 2, 1)


@pytest.mark.gpu
def test_gpu_many_overlapping_rois(gpu_device):
    """The gather backward's grouping at the shape the benchmark times: more than 128 rois (one
    staging batch holds 128) with 7x7x7 bins, all overlapping one small volume, so every voxel is
    reached by many rois and the groups are cut by the 384-bin and weight-table limits."""
    from fda_helpers import assert_close, log

    from ops3d_amd.roi_align import roi_align_3d

    N, C, size, R, pooled = 1, 8, (9, 10, 12), 150, (7, 7, 7)
    log(f"[case] roi_align3d many overlapping rois: R={R} pooled={pooled} size={size}")
    r = np.random.default_rng(11)
    x = torch.from_numpy(r.normal(size=(N, C) + size).astype(np.float32))
    rois = torch.from_numpy(_rois(R, N, size, seed=12, lo=-1.0, hi=9.0))
    xg = x.to(gpu_device).requires_grad_(True)
    out = roi_align_3d(xg, rois.to(gpu_device), pooled, 1.0, 1, 1)
    g = torch.from_numpy(r.normal(size=tuple(out.shape)).astype(np.float32))
    out.backward(g.to(gpu_device))
    torch.cuda.synchronize()
    want = O.forward(x.double().numpy(), rois.double().numpy(), pooled, 1.0, 1, 1)
    gwant = O.backward(g.double().numpy(), rois.double().numpy(), x.shape, 1.0, 1, 1)
    assert_close("overlapping rois output", out.detach(), want, 1e-5, 1e-6)
    assert_close("overlapping rois grad", xg.grad, gwant, 1e-5, 1e-5)


# --- channels-last forward ----------------------------------------------------------------------
CL_CASES = [
    # N, C, (D, H, W), R, pooled, scale, sampling_ratio, order, dtype
    (2, 8, (8, 12, 16), 20, (3, 3, 3), 1.0, 2, 1, torch.float32),
    (2, 16, (8, 12, 16), 20, (2, 3, 4), 0.5, 0, 1, torch.bfloat16),     # adaptive grid
    (1, 24, (5, 6, 7), 15, (2, 2, 2), 1.0, 3, 0, torch.float16),        # per-sample path, nearest
    (1, 256, (6, 10, 12), 40, (7, 7, 7), 1.0, 2, 1, torch.bfloat16),    # the benchmark's bins
    (1, 256, (6, 10, 12), 12, (3, 5, 6), 1.0, 2, 1, torch.float32),
    (2, 2048, (4, 4, 4), 6, (2, 3, 4), 1.0, 2, 1, torch.bfloat16),      # one bin per block
    (1, 40, (9, 10, 12), 150, (7, 7, 7), 1.0, 1, 1, torch.float32),     # many overlapping rois
    (1, 16, (12, 14, 16), 30, (2, 3, 2), 1.0, 4, 1, torch.float32),     # 4 samples per axis (8-tap lists)
    (2, 32, (12, 14, 16), 30, (1, 2, 1), 0.5, 0, 0, torch.bfloat16),    # adaptive: 8-tap lists and wider
]


def test_channels_last_support_and_argument_errors():
    """Which shapes the channels-last forward takes, and its argument checks (no GPU needed)."""
    from ops3d_amd import _extension

    lib = _extension.load_library()
    ok = lib.ops3d_roi_align3d_channels_last_supported
    assert ok(2, 256, 32, 64, 64, 7) == 1 and ok(0, 8, 1, 1, 1, 1) == 1 and ok(1, 2048, 4, 4, 4, 4) == 1
    assert ok(2, 12, 4, 4, 4, 4) == 0                  # C % 8 != 0
    assert ok(2, 2056, 4, 4, 4, 4) == 0                # C > 2048
    assert ok(2, 256, 256, 256, 256, 7) == 0           # D*H*W*C >= 2^32
    assert ok(3, 256, 4, 4, 4, 4) == 0                 # dtype
    f = lib.ops3d_roi_align3d_forward_channels_last
    import ctypes
    a = (2, 1, 256, 4, 4, 4, 3, 2, 2, 2, ctypes.c_float(1.0), 2, 1, None)
    assert f(None, None, None, *a) == 1                # NULL pointers
    assert f(None, None, None, 2, 1, 12, 4, 4, 4, 3, 2, 2, 2, ctypes.c_float(1.0), 2, 1, None) == 1
    assert f(None, None, None, 2, 1, 256, 4, 4, 4, 0, 2, 2, 2, ctypes.c_float(1.0), 2, 1, None) == 0   # no rois
    t = lib.ops3d_roi_align3d_to_channels_last
    assert t(None, None, 2, 1, 8, 4, 4, 4, None) == 1
    assert t(None, None, 2, 0, 8, 4, 4, 4, None) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(CL_CASES)))
def test_gpu_channels_last_same_bits(gpu_device, case):
    """The channels-last forward computes the NCDHW kernel's terms in its order: the same bits,
    through the C ABI; and the copy into [N,D,H,W,C] is an exact permutation."""
    import ctypes

    from fda_helpers import log

    from ops3d_amd import _extension

    lib = _extension.load_library()
    N, C, size, R, pooled, scale, sr, order, dt = CL_CASES[case]
    log(f"[case] roi_align3d channels-last #{case}: N={N} C={C} size={size} R={R} pooled={pooled} sr={sr} {dt}")
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[dt]
    r = np.random.default_rng(50 + case)
    x = torch.from_numpy(r.normal(size=(N, C) + size).astype(np.float32)).to(dt).to(gpu_device)
    rois_np = _rois(R, N, tuple(int(v / scale) for v in size), seed=150 + case)
    rois_np[0, 0] = N + 3                              # a batch item that does not exist: zeros
    rois = torch.from_numpy(rois_np).to(dt).to(gpu_device)
    xc = torch.empty((N,) + size + (C,), dtype=dt, device=gpu_device)
    o1 = torch.empty((R, C) + pooled, dtype=dt, device=gpu_device)
    o2 = torch.full_like(o1, 7.0)
    st = torch.cuda.current_stream().cuda_stream
    args = (code, N, C, *size, R, *pooled, ctypes.c_float(scale), sr, order, st)
    assert lib.ops3d_roi_align3d_forward(x.data_ptr(), rois.data_ptr(), o1.data_ptr(), *args) == 0
    assert lib.ops3d_roi_align3d_to_channels_last(x.data_ptr(), xc.data_ptr(), code, N, C, *size, st) == 0
    assert lib.ops3d_roi_align3d_forward_channels_last(xc.data_ptr(), rois.data_ptr(), o2.data_ptr(), *args) == 0
    torch.cuda.synchronize()
    assert torch.equal(xc, x.permute(0, 2, 3, 4, 1))
    assert torch.equal(o1, o2)
    assert torch.all(o2[0] == 0)


@pytest.mark.gpu
def test_gpu_channels_last_through_the_op(gpu_device):
    """roi_align_3d takes the channels-last kernel for large outputs (here 40 x 64 x 7^3 elements)
    and for channels_last_3d input: checked against the oracle, and the channels_last_3d input
    gives the contiguous input's output and gradient bit for bit."""
    from fda_helpers import assert_close, log

    from ops3d_amd.roi_align import roi_align_3d

    N, C, size, R, pooled = 1, 64, (6, 8, 10), 40, (7, 7, 7)
    log(f"[case] roi_align3d channels-last op: N={N} C={C} size={size} R={R} pooled={pooled}")
    r = np.random.default_rng(11)
    x = torch.from_numpy(r.normal(size=(N, C) + size).astype(np.float32))
    rois = torch.from_numpy(_rois(R, N, size, seed=12))
    outs, grads = [], []
    g = torch.from_numpy(r.normal(size=(R, C) + pooled).astype(np.float32)).to(gpu_device)
    for fmt in (torch.contiguous_format, torch.channels_last_3d):
        xg = x.to(gpu_device).contiguous(memory_format=fmt).requires_grad_(True)
        out = roi_align_3d(xg, rois.to(gpu_device), pooled, 1.0, 2, 1)
        out.backward(g)
        outs.append(out.detach())
        grads.append(xg.grad.contiguous())
    torch.cuda.synchronize()
    want = O.forward(x.double().numpy(), rois.double().numpy(), pooled, 1.0, 2, 1)
    assert_close("channels-last op output", outs[0], want, 1e-5, 1e-6)
    assert torch.equal(outs[0], outs[1]) and torch.equal(grads[0], grads[1])


@pytest.mark.gpu
def test_gpu_backward_more_rois_than_one_grid_dimension(gpu_device):
    """More than 65535 rois: the gather backward's channels-last copy of grad_output is made in
    launches of at most 65535 rois.  Checked two ways: the adjoint identity <F(x), g> = <x, F^T g>
    (float64 sums of the GPU's fp32 results) and against the sum of the two halves' gradients."""
    from fda_helpers import log

    from ops3d_amd.roi_align import roi_align_3d

    N, C, size, R, pooled = 1, 8, (6, 7, 9), 70000, (1, 2, 1)
    log(f"[case] roi_align3d backward with R={R} rois")
    r = np.random.default_rng(21)
    x = torch.from_numpy(r.normal(size=(N, C) + size).astype(np.float32)).to(gpu_device)
    rois = torch.from_numpy(_rois(R, N, size, seed=22)).to(gpu_device)
    g = torch.from_numpy(r.normal(size=(R, C) + pooled).astype(np.float32)).to(gpu_device)

    def grad_of(rr, gg):
        xg = x.clone().requires_grad_(True)
        roi_align_3d(xg, rr, pooled, 1.0, 2, 1).backward(gg)
        return xg.grad

    full = grad_of(rois, g)
    h = 65535
    halves = grad_of(rois[:h], g[:h]) + grad_of(rois[h:], g[h:])
    with torch.no_grad():
        out = roi_align_3d(x, rois, pooled, 1.0, 2, 1)
    torch.cuda.synchronize()
    lhs = float((out.double() * g.double()).sum())
    rhs = float((x.double() * full.double()).sum())
    assert abs(lhs - rhs) <= 1e-4 * float((out.double().abs() * g.double().abs()).sum())
    assert torch.allclose(full, halves, rtol=1e-5, atol=1e-4)
