"""PyTorch restatement of the reference's naive path -- TEST INFRASTRUCTURE / CPU BASELINE ONLY.

Follows ops3d/flash_deform_attn.py:139-165 (per-level ``F.grid_sample``, trilinear on 5-D,
zero padding, align_corners=False, grid = 2*loc - 1, weighted sum over L*K samples) with the
softmax the reference's tests apply to the raw logits (tests/test_flash_deform_attn.py:38-40,
126-128).  Backward is torch autograd through it.  Used by bench.py as the CPU baseline and by
the tests as a library-based oracle.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def unpack(sampling_loc_attn: torch.Tensor, L: int, K: int):
    """[B,Q,G,4LK] -> locations [B,Q,G,L,K,3], logits [B,Q,G,L,K]."""
    B, Q, G, _ = sampling_loc_attn.shape
    locs = sampling_loc_attn[..., : 3 * L * K].reshape(B, Q, G, L, K, 3)
    logits = sampling_loc_attn[..., 3 * L * K :].reshape(B, Q, G, L, K)
    return locs, logits


def core(value, shapes, locs, attn):
    """value [B,S,G,D]; shapes list of (D,H,W); locs [B,Q,G,L,K,3]; attn [B,Q,G,L,K] -> [B,Q,G*D]."""
    B, S, G, D = value.shape
    Q, L, K = locs.shape[1], locs.shape[3], locs.shape[4]
    out = value.new_zeros(B * G, D, Q)
    start = 0
    for l, (d, h, w) in enumerate(shapes):
        n = d * h * w
        vol = value[:, start : start + n].permute(0, 2, 3, 1).reshape(B * G, D, d, h, w)
        start += n
        grid = (2 * locs[:, :, :, l] - 1).transpose(1, 2).reshape(B * G, 1, Q, K, 3)
        samp = F.grid_sample(vol, grid, mode="bilinear", padding_mode="zeros", align_corners=False)
        a = attn[:, :, :, l].transpose(1, 2).reshape(B * G, 1, Q, K)
        out = out + (samp[:, :, 0] * a).sum(-1)
    return out.reshape(B, G * D, Q).transpose(1, 2).contiguous()


def forward_packed(value, shapes, sampling_loc_attn, K):
    L = len(shapes)
    locs, logits = unpack(sampling_loc_attn, L, K)
    attn = F.softmax(logits.flatten(-2), dim=-1).unflatten(-1, (L, K))
    return core(value, shapes, locs, attn)


def forward_backward(value, shapes, sampling_loc_attn, grad_out, K):
    """fp32/fp64 CPU or GPU: returns (out, grad_value, grad_sampling_loc_attn)."""
    v = value.detach().clone().requires_grad_(True)
    sla = sampling_loc_attn.detach().clone().requires_grad_(True)
    out = forward_packed(v, shapes, sla, K)
    out.backward(grad_out)
    return out.detach(), v.grad, sla.grad
