"""CPU emulation of the backward's tile index arithmetic (no GPU): the home tile and tile-local
word of the query kernel, the entry expansion of the bucketing kernels (entries are sample
indices), and the tile kernel's local bins (from the stashed pixel coordinates and the tile's
origin), counting sort and x-pair ranges, checked against the float64 oracle's grad_value.
Every LDS index the tile kernel would use is asserted to stay inside its array.  Covers odd
widths, 1-voxel rows and levels, levels smaller than a tile, partial last tiles, several heads
and batch items, and nominal tile sizes down to 2x1x1 (every sample then crosses tiles)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from ops3d_amd.workloads import pack


def _pixel(loc, size):
    # the kernel's fp32 rounding of ((2*loc - 1 + 1) * size - 1) / 2
    l = np.float32(loc)
    grid = np.float32(np.float32(2.0) * l) - np.float32(1.0)
    t = np.float32(np.float32(grid + np.float32(1.0)) * np.float32(size))
    return float(np.float32(np.float32(t - np.float32(1.0)) * np.float32(0.5)))


def level_tiles(shape, nominal):
    """(t, nt, count) per fda_device.h level_tiles: nominal (tz, ty, tx) clipped to the level."""
    t, nt = [], []
    for n, T in zip(shape, nominal):
        ta = (n if n > 0 else 1) if n < T else T
        t.append(ta)
        nt.append((n + ta - 1) // ta if n > 0 else 0)
    return t, nt, nt[0] * nt[1] * nt[2]


def tile_threads(lpu, big=False):
    """fda_device.h tile_threads."""
    if big and lpu == 4:
        return 512
    return 256 if lpu <= 4 else (1024 if lpu >= 16 else 64 * lpu)


def tile_dims(lpu, big=False):
    """fda_device.h tile_dims -> (tx, ty, tz)."""
    v, lg = 2 * tile_threads(lpu, big) // lpu, 0
    while (1 << lg) < v:
        lg += 1
    bz = lg // 3
    by = (lg - bz) // 2
    bx = lg - bz - by
    return 1 << bx, 1 << by, 1 << bz


def emulate_grad_value(value, shapes, sla, grad_out, K, TX, TY, TZ):
    B, S, G, D = value.shape
    Q = sla.shape[1]
    L = len(shapes)
    LK = L * K
    nominal = (TZ, TY, TX)
    lts = [level_tiles(s, nominal) for s in shapes]
    T_h = sum(lt[2] for lt in lts)
    lbase = np.concatenate([[0], np.cumsum([lt[2] for lt in lts])[:-1]]).astype(int)
    lsi = np.concatenate([[0], np.cumsum([d * h * w for d, h, w in shapes])[:-1]]).astype(int)
    # phase 1: per sample (head-major numbering) key, word, stash
    keys, words, stash = [], [], []
    for b in range(B):
        for g in range(G):
            for q in range(Q):
                rec = sla[b, q, g]
                lg = rec[3 * LK:].astype(np.float64)
                e = np.exp(lg - lg.max())
                attn = e / e.sum()
                for l, (Dl, Hl, Wl) in enumerate(shapes):
                    (tz, ty, tx), (ntz, nty, ntx), _ = lts[l]
                    for k in range(K):
                        s = l * K + k
                        x, y, z = (_pixel(rec[3 * s], Wl), _pixel(rec[3 * s + 1], Hl), _pixel(rec[3 * s + 2], Dl))
                        inside = x >= -1 and y >= -1 and z >= -1 and x < Wl and y < Hl and z < Dl
                        stash.append((x, y, z, attn[s]))   # pixel coordinates
                        if not inside:
                            keys.append(None)
                            words.append(0)
                            continue
                        x0, y0, z0 = math.floor(x), math.floor(y), math.floor(z)
                        hz, hy, hx = max(z0, 0) // tz, max(y0, 0) // ty, max(x0, 0) // tx
                        lz, ly, lx = z0 - hz * tz, y0 - hy * ty, x0 - hx * tx
                        assert -1 <= lx < tx and -1 <= ly < ty and -1 <= lz < tz
                        ex = int(lx == tx - 1 and (hx + 1) * tx < Wl)
                        ey = int(ly == ty - 1 and (hy + 1) * ty < Hl)
                        ez = int(lz == tz - 1 and (hz + 1) * tz < Dl)
                        keys.append((b * G + g) * T_h + lbase[l] + (hz * nty + hy) * ntx + hx)
                        w = (lx + 1) | ((ly + 1) << 5) | ((lz + 1) << 10)
                        words.append(w | (ex << 15) | (ey << 16) | (ez << 17) | (l << 18))
    # phase 2: entries grouped by tile (any order inside a tile)
    buckets = [[] for _ in range(B * G * T_h)]
    for sidx, (key, w) in enumerate(zip(keys, words)):
        if key is None:
            continue
        l = w >> 18
        (_, _, _), (ntz, nty, ntx), _ = lts[l]
        ex, ey, ez = (w >> 15) & 1, (w >> 16) & 1, (w >> 17) & 1
        for dz in range(ez + 1):
            for dy in range(ey + 1):
                for dx in range(ex + 1):
                    ww = w & 0x7FFF
                    if dx:
                        ww &= ~0x1F
                    if dy:
                        ww &= ~(0x1F << 5)
                    if dz:
                        ww &= ~(0x1F << 10)
                    tid = key + dx + dy * ntx + dz * ntx * nty
                    assert tid < B * G * T_h
                    buckets[tid].append(sidx)
    # phase 3: tile kernel
    gv = np.full_like(value, np.nan, dtype=np.float64)
    go_rows = grad_out.reshape(B, Q, G, D).transpose(0, 2, 1, 3).reshape(-1, D)   # head-major rows
    NBX = (TX + 1) * (TY + 1) * (TZ + 1)
    for b in range(B):
        for g in range(G):
            for l, (Dl, Hl, Wl) in enumerate(shapes):
                (tz, ty, tx), (ntz, nty, ntx), cnt = lts[l]
                TXp, TYp = tx + 1, ty + 1
                nb = TXp * TYp * (tz + 1)
                assert nb <= NBX
                for t in range(cnt):
                    itx, ity, itz = t % ntx, (t // ntx) % nty, t // (ntx * nty)
                    ent = buckets[(b * G + g) * T_h + lbase[l] + t]
                    ox, oy, oz = itx * tx - 1, ity * ty - 1, itz * tz - 1   # bin 0 = local -1
                    lb = []
                    for sidx in ent:
                        sx, sy, sz, _ = stash[sidx]
                        v = ((math.floor(sz) - oz) * TYp + (math.floor(sy) - oy)) * TXp + (math.floor(sx) - ox)
                        assert 0 <= v < nb
                        lb.append(v)
                    counts = np.bincount(np.array(lb, dtype=int), minlength=nb) if lb else np.zeros(nb, int)
                    start = np.concatenate([[0], np.cumsum(counts)])
                    order = np.argsort(np.array(lb, dtype=int), kind="stable") if lb else np.zeros(0, int)

                    def st(i):
                        assert 0 <= i <= nb, f"start[{i}] outside [0, {nb}]"
                        return int(start[i])

                    for pz in range(TZ):
                        for py in range(TY):
                            for px in range(TX // 2):
                                z, y, x0 = itz * tz + pz, ity * ty + py, itx * tx + 2 * px
                                live = 2 * px < tx and py < ty and pz < tz and z < Dl and y < Hl and x0 < Wl
                                two = 2 * px + 1 < tx and x0 + 1 < Wl
                                if not live:
                                    continue
                                acc = np.zeros((2, D))
                                for r in range(4):
                                    dz, dy = r >> 1, r & 1
                                    rb = ((pz - dz + 1) * TYp + (py - dy + 1)) * TXp + 2 * px
                                    s0, m1, m2 = st(rb), st(rb + 1), st(rb + 2)
                                    s3 = st(rb + 3) if two else m2
                                    for i in range(s0, s3):
                                        sidx = ent[order[i]]
                                        sx, sy, sz, at = stash[sidx]
                                        fx, fy, fz = sx - math.floor(sx), sy - math.floor(sy), sz - math.floor(sz)
                                        wy = fy if dy else 1 - fy
                                        wz = fz if dz else 1 - fz
                                        lft, ctr = i < m1, i < m2
                                        aw0 = fx if lft else (1 - fx if ctr else 0.0)
                                        aw1 = 0.0 if lft else (fx if ctr else 1 - fx)
                                        tg = go_rows[sidx // LK]
                                        acc[0] += at * wy * wz * aw0 * tg
                                        acc[1] += at * wy * wz * aw1 * tg
                                for dv in range(2 if two else 1):
                                    v = lsi[l] + (z * Hl + y) * Wl + x0 + dv
                                    assert np.isnan(gv[b, v, g, 0]), "grad_value row written twice"
                                    gv[b, v, g] = acc[dv]
    assert not np.isnan(gv).any(), "grad_value row never written"
    return gv


CASES = [
    ([(1, 1, 1)], 1, 7, 1, 4),
    ([(1, 1, 1), (2, 3, 5)], 2, 9, 2, 4),
    ([(3, 2, 7), (1, 1, 3)], 1, 11, 3, 2),
    ([(2, 2, 2), (4, 3, 1)], 2, 6, 1, 8),
    ([(5, 6, 9)], 1, 20, 2, 4),
]
TILES = [(2, 1, 1), (4, 2, 2), (8, 4, 4), (8, 8, 4), (8, 8, 8)]   # (8, 8, 4): the big tiles of LPU 4


@pytest.mark.parametrize("tiles", TILES)
@pytest.mark.parametrize("shapes,B,Q,G,K", CASES)
def test_tile_index_emulation_matches_oracle(shapes, B, Q, G, K, tiles):
    D, L = 4, len(shapes)
    S = sum(d * h * w for d, h, w in shapes)
    gen = torch.Generator().manual_seed(len(shapes) * 7 + Q)
    value = torch.randn(B, S, G, D, generator=gen).double()
    loc = torch.rand(B, Q, G, L, K, 3, generator=gen) * 1.3 - 0.15
    sla = pack(loc, torch.randn(B, Q, G, L, K, generator=gen)).float().double()
    go = torch.randn(B, Q, G * D, generator=gen).double()
    gv = emulate_grad_value(value.numpy(), shapes, sla.numpy(), go.numpy(), K, *tiles)
    ref, _ = oracle.backward(value.numpy(), shapes, sla.numpy(), go.numpy(), K, coord_mode=1)
    np.testing.assert_allclose(gv, ref, rtol=1e-9, atol=1e-11)


@pytest.mark.parametrize("lpu,big", [(1, False), (2, False), (4, False), (4, True), (8, False), (16, False),
                                     (32, False)])
def test_tile_dims_fill_the_block(lpu, big):
    tx, ty, tz = tile_dims(lpu, big)
    threads = tile_threads(lpu, big)
    assert threads % 64 == 0 and 256 <= threads <= 1024
    assert tx % 2 == 0
    assert (tx // 2) * ty * tz * lpu == threads   # one x-pair per LPU lanes
    assert tx <= 16 and ty <= 16 and tz <= 16     # 5-bit tile-local coordinates
    assert max(tx, ty, tz) <= 2 * min(tx, ty, tz)
