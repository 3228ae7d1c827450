"""3-D NMS: the CPU oracle pinned (closed-form IoUs, the reference's own test cases, an
independent pairwise formulation), and the GPU kernels against it (marked gpu).

Reference tests: tests/test_nms.py:17-49 (1000 duplicates of one box -> only the top box;
two disjoint boxes -> both kept)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import nms3d as O


def _clustered(n, seed, spread=30.0, size=(2.0, 12.0)):
    """Boxes in a few clusters (so suppression happens), random scores with some ties."""
    r = np.random.default_rng(seed)
    centres = r.uniform(0, 100, size=(max(1, n // 20), 3))
    c = centres[r.integers(0, len(centres), n)] + r.normal(0, spread / 10, size=(n, 3))
    e = r.uniform(*size, size=(n, 3))
    boxes = np.concatenate([c - e / 2, c + e / 2], 1).astype(np.float32)
    scores = np.round(r.uniform(0, 1, n), 2).astype(np.float32)   # two decimals: ties
    return boxes, scores


# --- oracle pinning (CPU) --------------------------------------------------------------------
def test_iou_closed_forms():
    a = [0, 0, 0, 2, 2, 2]
    assert O.iou3d(a, [a])[0] == 1.0
    assert O.iou3d(a, [[3, 3, 3, 4, 4, 4]])[0] == 0.0                      # disjoint
    assert O.iou3d(a, [[2, 0, 0, 4, 2, 2]])[0] == 0.0                      # touching faces
    assert np.isclose(O.iou3d(a, [[1, 0, 0, 3, 2, 2]])[0], 4 / 12)         # half shifted along x
    assert np.isclose(O.iou3d([0, 0, 0, 4, 4, 4], [[1, 1, 1, 3, 3, 3]])[0], 8 / 64)   # nested
    assert np.isclose(O.iou3d(a, [[1, 1, 1, 3, 3, 3]])[0], 1 / 15)        # corner overlap
    # zero-volume pair: 0/0 -> NaN, never above a threshold
    assert np.isnan(O.iou3d([1, 1, 1, 1, 1, 1], [[1, 1, 1, 1, 1, 1]])[0])


def test_oracle_reference_cases():
    box0 = [0, 0, 0, 100, 100, 100]
    boxes = np.tile(np.asarray(box0, np.float32), (1000, 1))
    scores = np.zeros(1000, np.float32)
    scores[0] = 0.9
    assert O.nms3d(boxes, scores, 0.1).tolist() == [0]
    two = np.asarray([[0, 0, 0, 10, 10, 10], [20, 20, 20, 30, 30, 30]], np.float32)
    assert O.nms3d(two, np.asarray([0.6, 0.7]), 0.5).tolist() == [1, 0]   # both, by score


def test_oracle_against_pairwise_definition():
    """The greedy pass restated from a full float64 IoU matrix: box i is kept iff no kept box
    before it (in score order) has IoU above the threshold with it.  Boxes whose IoU lies within
    1e-5 of the threshold are excluded so that fp32 and fp64 decide alike."""
    for seed in range(5):
        boxes, scores = _clustered(300, seed)
        order = np.argsort(-scores.astype(np.float64), kind="stable")
        b = boxes[order].astype(np.float64)
        lo, hi = np.maximum(b[:, None, :3], b[None, :, :3]), np.minimum(b[:, None, 3:], b[None, :, 3:])
        inter = np.prod(np.clip(hi - lo, 0, None), -1)
        vol = np.prod(b[:, 3:] - b[:, :3], -1)
        iou = inter / (vol[:, None] + vol[None, :] - inter)
        thr = 0.3
        if np.any(np.abs(iou - thr) < 1e-5):
            continue
        kept = []
        for i in range(len(b)):
            if all(iou[k, i] <= thr for k in kept):
                kept.append(i)
        assert O.nms3d(boxes, scores, thr).tolist() == order[kept].tolist()


# --- GPU ---------------------------------------------------------------------------------------
@pytest.mark.gpu
def test_gpu_reference_cases(gpu_device):
    from ops3d_amd import _C

    box0 = torch.tensor([0, 0, 0, 100, 100, 100], device=gpu_device, dtype=torch.float32)
    boxes = box0.unsqueeze(0).repeat(1000, 1)
    scores = torch.cat([torch.tensor([0.9], device=gpu_device), torch.zeros(999, device=gpu_device)])
    assert _C.nms_3d(boxes, scores, 0.1).cpu().tolist() == [0]
    two = torch.tensor([[0, 0, 0, 10, 10, 10], [20, 20, 20, 30, 30, 30]], device=gpu_device, dtype=torch.float32)
    assert set(_C.nms_3d(two, torch.tensor([0.6, 0.7], device=gpu_device), 0.5).cpu().tolist()) == {0, 1}
    empty = _C.nms_3d(torch.empty(0, 6, device=gpu_device), torch.empty(0, device=gpu_device), 0.5)
    assert empty.dtype == torch.long and empty.numel() == 0


@pytest.mark.gpu
@pytest.mark.parametrize("n,thr,seed", [(1, 0.5, 0), (63, 0.3, 1), (64, 0.3, 2), (65, 0.3, 3), (1000, 0.1, 4),
                                        (1000, 0.5, 5), (4097, 0.3, 6), (20000, 0.3, 7)])
def test_gpu_matches_oracle(gpu_device, n, thr, seed):
    from fda_helpers import log

    from ops3d_amd.nms import nms_nd

    log(f"[case] nms3d n={n} thr={thr} seed={seed}")
    boxes, scores = _clustered(n, seed)
    dets = torch.from_numpy(np.concatenate([boxes, scores[:, None]], 1)).to(gpu_device)
    keep, _ = nms_nd(dets, thr)
    want = O.nms3d(boxes, scores, thr)
    assert keep.dtype == torch.long
    assert keep.cpu().numpy().tolist() == want.tolist()


@pytest.mark.gpu
def test_gpu_degenerate_and_thresholds(gpu_device):
    from ops3d_amd import _C

    boxes, scores = _clustered(500, 9)
    boxes[::7, 3:] = boxes[::7, :3]     # zero-volume boxes: IoU NaN with each other
    b = torch.from_numpy(boxes).to(gpu_device)
    s = torch.from_numpy(scores).to(gpu_device)
    for thr in (0.0, 0.3, 1.0):
        got = _C.nms_3d(b, s, thr).cpu().numpy().tolist()
        assert got == O.nms3d(boxes, scores, thr).tolist(), thr
    with pytest.raises(RuntimeError, match="CPU"):
        _C.nms_3d(torch.from_numpy(boxes), torch.from_numpy(scores), 0.5)
