"""Writes c1_small.npz: seeded inputs (stored as float32, so an fp32 kernel can consume them
exactly) and float64 outputs of the c1 geometry (levels (4,8,16), (2,4,8); L=2, K=4) with
G=2 heads, D=32 channels, Q=48 queries, B=1.

Expected values come from torch's F.grid_sample + softmax + autograd in float64
(oracle/torch_port.py: the reference's PyTorch path, ops3d/flash_deform_attn.py:139-165),
i.e. from the library routine, not from the C oracle the fixture is used to check.
Run from the repo root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import torch_port  # noqa: E402
from ops3d_amd.workloads import pack  # noqa: E402

shapes = ((4, 8, 16), (2, 4, 8))
B, Q, G, D, L, K = 1, 48, 2, 32, 2, 4
S = sum(a * b * c for a, b, c in shapes)
g = torch.Generator().manual_seed(1234)
value = torch.randn(B, S, G, D, generator=g).float()
locs = torch.rand(B, Q, G, L, K, 3, generator=g) * 1.1 - 0.05
logits = torch.randn(B, Q, G, L, K, generator=g)
sla = pack(locs, logits).float()
grad_out = torch.randn(B, Q, G * D, generator=g).float()
out, gv, gs = torch_port.forward_backward(value.double(), shapes, sla.double(), grad_out.double(), K)
np.savez_compressed(
    os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1_small.npz"),
    shapes=np.array(shapes, dtype=np.int64), K=np.int64(K),
    value=value.numpy(), sampling_loc_attn=sla.numpy(), grad_output=grad_out.numpy(),
    output=out.numpy(), grad_value=gv.numpy(), grad_sampling_loc_attn=gs.numpy(),
)
print("wrote c1_small.npz")
