"""Multi-scale deformable attention over 3-D volumes, built on the offset-mode op.

The caller of the reference's op computes the sampling locations (reference points + offsets
scaled per level), the attention logits, and concatenates them into ``sampling_loc_attn``
(reference tests/test_flash_deform_attn.py:30-37); its backward splits the gradient again.
``FlashDeformAttn3D`` produces the packed planar layout with ONE linear projection of the query
(for each head: the L*K (x,y,z) offsets in voxels of their level, then the L*K logits) and hands
it to ``FlashDeformAttnFromOffsets``, which forms the locations inside the kernels: no add,
divide, cat or split pass on either side of the op.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .flash_deform_attn import FlashDeformAttnFromOffsets


class FlashDeformAttn3D(nn.Module):
    """value_proj -> deformable attention (FlashDeformAttnFromOffsets) -> output_proj.

    forward(query [B,Q,C], reference_points [B,Q,1 or L,3] float32 in [0,1], value [B,S,C],
    spatial_shapes [L,3] int64 (D,H,W), level_start_index [L] int64) -> [B,Q,C].
    """

    def __init__(self, embed_dim: int = 256, num_heads: int = 8, num_levels: int = 4, num_points: int = 4,
                 im2col_step: int = 64):
        super().__init__()
        if embed_dim % num_heads:
            raise ValueError(f"embed_dim ({embed_dim}) must be divisible by num_heads ({num_heads})")
        self.embed_dim, self.num_heads = embed_dim, num_heads
        self.num_levels, self.num_points = num_levels, num_points
        self.head_dim = embed_dim // num_heads
        self.im2col_step = im2col_step
        self.packed = 4 * num_levels * num_points   # per head: 3*L*K offsets, then L*K logits
        self.value_proj = nn.Linear(embed_dim, embed_dim)
        self.sampling = nn.Linear(embed_dim, num_heads * self.packed)
        self.output_proj = nn.Linear(embed_dim, embed_dim)
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self) -> None:
        nn.init.xavier_uniform_(self.value_proj.weight)
        nn.init.zeros_(self.value_proj.bias)
        nn.init.xavier_uniform_(self.output_proj.weight)
        nn.init.zeros_(self.output_proj.bias)
        # offsets start on a ring of directions per head, point k at k+1 voxels; logits at 0
        nn.init.zeros_(self.sampling.weight)
        G, L, K = self.num_heads, self.num_levels, self.num_points
        bias = torch.zeros(G, self.packed)
        golden = math.pi * (3.0 - math.sqrt(5.0))   # spread G directions over the sphere
        for g in range(G):
            zc = 1.0 - 2.0 * (g + 0.5) / G
            r = math.sqrt(max(0.0, 1.0 - zc * zc))
            d = torch.tensor([r * math.cos(golden * g), r * math.sin(golden * g), zc])
            d = d / d.abs().max()
            for l in range(L):
                for k in range(K):
                    s = l * K + k
                    bias[g, 3 * s: 3 * s + 3] = d * (k + 1)
        self.sampling.bias.copy_(bias.flatten())

    def forward(self, query, reference_points, value, spatial_shapes, level_start_index):
        B, Q, C = query.shape
        S = value.shape[1]
        v = self.value_proj(value).view(B, S, self.num_heads, self.head_dim)
        oa = self.sampling(query).view(B, Q, self.num_heads, self.packed)   # packed planar, as produced
        out = FlashDeformAttnFromOffsets.apply(v, spatial_shapes, level_start_index, oa,
                                               reference_points.to(torch.float32), self.im2col_step, self.num_points)
        return self.output_proj(out)
