"""Flash Deformable 3D Attention: Python API and autograd Function (MI355X / gfx950).

Drop-in for the reference's ``ops3d/flash_deform_attn.py``:
  * ``FlashDeformAttnFunction.apply(value, value_spatial_shapes, value_level_start_index,
    sampling_loc_attn, im2col_step, K=8, use_reg=True)`` -- same arguments, same
    ``ValueError`` on a wrong packed last dimension, same ``RuntimeError`` when the native
    library is missing, same backward return tuple (reference :65-136);
  * ``findspec`` / ``findspec_bwd`` -- same results as the reference's launch heuristics
    (:26-62), computed from a divisor walk up to sqrt(B*Q) instead of a scan of all B*Q
    integers.  Their values are passed to ``_C`` for interface fidelity only: the gfx950
    library chooses its own launch geometry;
  * ``ms_deform_attn_core_pytorch_3d`` -- the reference's PyTorch path (:139-165), written
    with ``F.grid_sample`` (trilinear on 5-D input, zero padding, align_corners=False).

Layout of ``sampling_loc_attn`` [B, Q, G, L*K*3 + L*K]: per (b, q, g), first the L*K (x, y, z)
locations in [0, 1] (level-major, point-minor; x indexes W, y H, z D), then the L*K raw
attention logits; the softmax over all L*K logits is applied inside the op.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.autograd import Function
from torch.autograd.function import once_differentiable

from ._extension import _C


def factors(N):
    """All positive divisors of N in increasing order (reference :17-23)."""
    small, large = [], []
    i = 1
    while i * i <= N:
        if N % i == 0:
            small.append(i)
            if i != N // i:
                large.append(N // i)
        i += 1
    return small + large[::-1]


def findspec(B, Q, G, C):
    """Forward launch spec of the reference (:26-41): d_stride 8 and
    threads = m*G*C//8 for the largest m | B*Q with m <= 64 and threads <= 512."""
    d_stride = 8
    multiplier = 1
    for m in factors(B * Q):
        if m <= 64 and (m * G * C // d_stride) <= 512:
            multiplier = m
    return d_stride, multiplier * G * C // d_stride


def findspec_bwd(B, Q, G, C, max_tpb=256, max_mult=64):
    """Backward launch spec of the reference (:44-62)."""
    for d in (1, 2, 4, 8, 16, 32):
        if C % d == 0 and G * (C // d) <= max_tpb:
            d_stride = d
            break
    else:
        raise RuntimeError(f"Cannot fit G={G}, C={C} into {max_tpb} threads")
    best_mult = 1
    for m in factors(B * Q):
        if m <= max_mult and m * G * (C // d_stride) <= max_tpb:
            best_mult = max(best_mult, m)
    return d_stride, best_mult * G * (C // d_stride)


class FlashDeformAttnFunction(Function):
    @staticmethod
    def forward(
        ctx,
        value,
        value_spatial_shapes,
        value_level_start_index,
        sampling_loc_attn,
        im2col_step,
        K=8,
        use_reg=True,
    ):
        if _C is None:
            raise RuntimeError(
                "ops3d_amd native library (libops3d_fda.so) not built; FlashDeformAttnFunction requires it."
            )
        ctx.K = K
        ctx.im2col_step = im2col_step

        L = value_spatial_shapes.shape[0]
        expected_last = L * K * 3 + L * K
        if sampling_loc_attn.shape[-1] != expected_last:
            raise ValueError(
                "sampling_loc_attn last dimension ({}) does not match "
                "value_spatial_shapes level count L={} and K={} (expected {})".format(
                    sampling_loc_attn.shape[-1], L, K, expected_last
                )
            )

        # The reference derives CUDA launch hints here (findspec / findspec_bwd, still exported);
        # the gfx950 library chooses its own geometry, so they are not computed.  The forward's
        # head-major copy of value is kept for the backward, which needs the same copy.
        output, value_hm = _C.forward_keep_head_major(
            value, value_spatial_shapes, value_level_start_index, sampling_loc_attn, ctx.im2col_step, K
        )
        ctx.save_for_backward(value, value_spatial_shapes, value_level_start_index, sampling_loc_attn, value_hm)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        value, value_spatial_shapes, value_level_start_index, sampling_loc_attn, value_hm = ctx.saved_tensors
        grad_value, grad_sampling_loc_attn = _C.backward_with_head_major(
            value,
            value_hm,
            value_spatial_shapes,
            value_level_start_index,
            sampling_loc_attn,
            grad_output.contiguous(),
            ctx.im2col_step,
            ctx.K,
        )
        return grad_value, None, None, grad_sampling_loc_attn, None, None, None


class FlashDeformAttnFromOffsets(Function):
    """Caller-side fusion of the op's producer and consumer (offset mode, no counterpart in the
    reference).  ``offset_attn`` [B,Q,G,4*L*K] has the packed planar layout of
    sampling_loc_attn, but its L*K (x,y,z) triples are offsets in voxels of their level: it is
    the output of one linear projection of the query, used as is.  The kernels form
    ``loc = reference_points + offset / (W, H, D)_level`` in fp32 (``reference_points``
    [B,Q,1 or L,3] float32, (x,y,z) in [0,1]), so the caller's add, divide and torch.cat passes
    (reference tests/test_flash_deform_attn.py:30-37) and their backward split disappear.
    Gradients: value, offset_attn (offsets and logits in its layout) and, when it requires
    grad, reference_points (the sum over heads and points of offset gradient * level size,
    added up in the kernels)."""

    @staticmethod
    def forward(ctx, value, value_spatial_shapes, value_level_start_index, offset_attn, reference_points,
                im2col_step, K=8):
        if _C is None:
            raise RuntimeError(
                "ops3d_amd native library (libops3d_fda.so) not built; FlashDeformAttnFromOffsets requires it."
            )
        ctx.K = K
        ctx.im2col_step = im2col_step
        output, value_hm = _C.forward_offsets(
            value, value_spatial_shapes, value_level_start_index, offset_attn, reference_points, im2col_step, K
        )
        ctx.save_for_backward(value, value_spatial_shapes, value_level_start_index, offset_attn, reference_points,
                              value_hm)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        value, shapes, lsi, offset_attn, ref, value_hm = ctx.saved_tensors
        grad_value, grad_oa, grad_ref = _C.backward_offsets(
            value, value_hm, shapes, lsi, offset_attn, ref, grad_output.contiguous(), ctx.im2col_step, ctx.K,
            bool(ctx.needs_input_grad[4]),
        )
        return grad_value, None, None, grad_oa, grad_ref, None, None


def ms_deform_attn_core_pytorch_3d(value, value_spatial_shapes, sampling_locations, attention_weights):
    """PyTorch path of 3-D deformable attention (reference ops3d/flash_deform_attn.py:139-165).

    value [N, S, M, E]; value_spatial_shapes [L, 3] rows (D, H, W); sampling_locations
    [N, Lq, M, L, P, 3] in [0, 1] (x, y, z); attention_weights [N, Lq, M, L, P], already
    normalised.  Returns [N, Lq, M*E].
    """
    N, S, M, E = value.shape
    _, Lq, _, L, P, _ = sampling_locations.shape
    sizes = [int(d) * int(h) * int(w) for d, h, w in value_spatial_shapes.tolist()]
    per_level = value.split(sizes, dim=1)
    grids = 2 * sampling_locations - 1
    sampled = []
    for lid, (d, h, w) in enumerate(value_spatial_shapes.tolist()):
        # [N, DHW, M, E] -> [N*M, E, D, H, W]
        vol = per_level[lid].permute(0, 2, 3, 1).reshape(N * M, E, int(d), int(h), int(w))
        # [N, Lq, M, P, 3] -> [N*M, 1, Lq, P, 3]
        grid = grids[:, :, :, lid].permute(0, 2, 1, 3, 4).reshape(N * M, 1, Lq, P, 3)
        s = F.grid_sample(vol, grid, mode="bilinear", padding_mode="zeros", align_corners=False)
        sampled.append(s.squeeze(2))  # [N*M, E, Lq, P]
    # [N*M, E, Lq, L*P] * [N*M, 1, Lq, L*P] -> sum -> [N*M, E, Lq]
    attn = attention_weights.permute(0, 2, 1, 3, 4).reshape(N * M, 1, Lq, L * P)
    out = (torch.stack(sampled, dim=-2).flatten(-2) * attn).sum(-1)
    return out.view(N, M * E, Lq).transpose(1, 2).contiguous()
