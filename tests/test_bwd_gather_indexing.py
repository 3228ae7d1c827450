"""CPU emulation of the backward gather's index arithmetic (no GPU): the bin keys of the query
kernel, the stable sort, the bin offsets and the value kernel's pair ranges, checked against
the float64 oracle's grad_value, with every bin_start read asserted to stay inside the entries
the bin-offset kernel writes ([0, real bins]).  Covers odd widths, 1-voxel rows and levels,
several heads and batch items -- the shapes where a pair has a single voxel."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from ops3d_amd.workloads import pack


def _level_bins(d, h, w):
    return 0 if (d == 0 or h == 0 or w == 0) else (d + 1) * (h + 1) * (w + 1)


def _pixel(loc, size):
    # the kernel's fp32 rounding of ((2*loc - 1 + 1) * size - 1) / 2
    l = np.float32(loc)
    grid = np.float32(np.float32(2.0) * l) - np.float32(1.0)
    t = np.float32(np.float32(grid + np.float32(1.0)) * np.float32(size))
    return float(np.float32(np.float32(t - np.float32(1.0)) * np.float32(0.5)))


def emulate_grad_value(value, shapes, sla, grad_out, K):
    B, S, G, D = value.shape
    Q = sla.shape[1]
    L = len(shapes)
    LK = L * K
    bins_bg = sum(_level_bins(*s) for s in shapes)
    nbins_real = B * G * bins_bg
    lsi = np.concatenate([[0], np.cumsum([d * h * w for d, h, w in shapes])[:-1]])
    keys, stash, rows = [], [], []
    invalid = B * G * 8 * S
    for b in range(B):
        for g in range(G):
            for q in range(Q):
                rec = sla[b, q, g]
                lg = rec[3 * LK:].astype(np.float64)
                e = np.exp(lg - lg.max())
                attn = e / e.sum()
                boff = (b * G + g) * bins_bg
                for l, (Dl, Hl, Wl) in enumerate(shapes):
                    for k in range(K):
                        s = l * K + k
                        x, y, z = (_pixel(rec[3 * s], Wl), _pixel(rec[3 * s + 1], Hl), _pixel(rec[3 * s + 2], Dl))
                        if not (x >= -1 and y >= -1 and z >= -1 and x < Wl and y < Hl and z < Dl):
                            keys.append(invalid)
                        else:
                            x0, y0, z0 = math.floor(x), math.floor(y), math.floor(z)
                            keys.append(boff + ((z0 + 1) * (Hl + 1) + (y0 + 1)) * (Wl + 1) + (x0 + 1))
                        stash.append((x - math.floor(x), y - math.floor(y), z - math.floor(z), attn[s]))
                        rows.append((b * Q + q) * G + g)
                    boff += _level_bins(Dl, Hl, Wl)
    keys = np.array(keys, dtype=np.int64)
    order = np.argsort(keys, kind="stable")
    skeys = keys[order]
    # bin offsets: written for bins [0, nbins_real]
    bin_start = np.searchsorted(skeys, np.arange(nbins_real + 1), side="left")

    def bs(i):
        assert 0 <= i <= nbins_real, f"bin_start[{i}] read outside [0, {nbins_real}]"
        return int(bin_start[i])

    gv = np.zeros_like(value, dtype=np.float64)
    for b in range(B):
        for g in range(G):
            bin_lvl = 0
            for l, (Dl, Hl, Wl) in enumerate(shapes):
                W1, HW1 = Wl + 1, (Hl + 1) * (Wl + 1)
                bin_lb = (b * G + g) * bins_bg + bin_lvl
                for z in range(Dl):
                    for y in range(Hl):
                        for x0 in range(0, Wl, 2):
                            two = x0 + 1 < Wl
                            bin_p = bin_lb + (z + 1) * HW1 + (y + 1) * W1 + x0
                            acc = np.zeros((2, D))
                            for r in range(4):
                                rb = bin_p - (r >> 1) * HW1 - (r & 1) * W1
                                s0, s1, s2 = bs(rb), bs(rb + 1), bs(rb + 2)
                                s3 = bs(rb + 3) if two else s2
                                for i in range(s0, s3):
                                    fx, fy, fz, at = stash[order[i]]
                                    wy = fy if (r & 1) else 1 - fy
                                    wz = fz if (r >> 1) else 1 - fz
                                    wx0 = fx if i < s1 else (1 - fx if i < s2 else 0.0)
                                    wx1 = 0.0 if i < s1 else (fx if i < s2 else 1 - fx)
                                    tg = grad_out.reshape(-1, D)[rows[order[i]]]
                                    acc[0] += at * wx0 * wy * wz * tg
                                    acc[1] += at * wx1 * wy * wz * tg
                            for dv in range(2 if two else 1):
                                gv[b, lsi[l] + (z * Hl + y) * Wl + x0 + dv, g] = acc[dv]
                bin_lvl += _level_bins(Dl, Hl, Wl)
    return gv


CASES = [
    ([(1, 1, 1)], 1, 7, 1, 4),
    ([(1, 1, 1), (2, 3, 5)], 2, 9, 2, 4),
    ([(3, 2, 7), (1, 1, 3)], 1, 11, 3, 2),
    ([(2, 2, 2), (4, 3, 1)], 2, 6, 1, 8),
]


@pytest.mark.parametrize("shapes,B,Q,G,K", CASES)
def test_gather_index_emulation_matches_oracle(shapes, B, Q, G, K):
    D, L = 4, len(shapes)
    S = sum(d * h * w for d, h, w in shapes)
    gen = torch.Generator().manual_seed(len(shapes) * 7 + Q)
    value = torch.randn(B, S, G, D, generator=gen).double()
    loc = torch.rand(B, Q, G, L, K, 3, generator=gen) * 1.3 - 0.15
    sla = pack(loc, torch.randn(B, Q, G, L, K, generator=gen)).float().double()
    go = torch.randn(B, Q, G * D, generator=gen).double()
    gv = emulate_grad_value(value.numpy(), shapes, sla.numpy(), go.numpy(), K)
    ref, _ = oracle.backward(value.numpy(), shapes, sla.numpy(), go.numpy(), K, coord_mode=1)
    np.testing.assert_allclose(gv, ref, rtol=1e-9, atol=1e-11)


def emulate_bin_start_fill(skeys, last, small_gap=4, wave=64):
    """The bin-offset kernel's boundary fill: element i starts every bin in (k[i-1], k[i]],
    clamped to [0, last]; wide gaps are filled wave-cooperatively (same values)."""
    n = len(skeys)
    out = np.full(last + 1, -1, dtype=np.int64)
    for i in range(n + 1):
        lo = 0 if i == 0 else int(skeys[i - 1]) + 1
        hi = last if i == n else min(int(skeys[i]), last)
        if lo > hi:
            continue
        if hi - lo < small_gap:
            out[lo:hi + 1] = i
        else:
            for lane in range(wave):
                out[lo + lane:hi + 1:wave] = i
    return out


@pytest.mark.parametrize("case", ["random", "all_invalid", "empty", "dense", "sparse_tail"])
def test_bin_start_fill_matches_lower_bound(case):
    rng = np.random.default_rng(3)
    last, invalid = 500, 800
    if case == "random":
        keys = rng.integers(0, last + 1, 300)
        keys[rng.random(300) < 0.1] = invalid
    elif case == "all_invalid":
        keys = np.full(50, invalid)
    elif case == "empty":
        keys = np.zeros(0, dtype=np.int64)
    elif case == "dense":
        keys = rng.integers(0, 20, 400)
    else:
        keys = rng.integers(0, 7, 30)
    skeys = np.sort(keys, kind="stable")
    got = emulate_bin_start_fill(skeys, last)
    want = np.searchsorted(skeys, np.arange(last + 1), side="left")
    np.testing.assert_array_equal(got, want)
