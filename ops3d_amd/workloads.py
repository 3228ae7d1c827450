"""Synthetic workloads of the benchmark configurations (c1..c5) and an input builder.

Shapes follow the five configurations of the headline benchmark: self-attention over tiled
light-sheet volumes at strides 16/32 (and 8/16/32), cross-attention of 200 object queries.
All use G=8 heads, D=32 channels per head, K=4 points.  Inputs: value ~ N(0,1) [B,S,G,D];
locations ~ U(0,1) [B,Q,G,L,K,3] (c3: 10 % of the (x,y,z) triples ~ U(-0.1, 1.1) to exercise
out-of-volume masking); logits ~ N(0,1) [B,Q,G,L,K]; upstream grad ~ N(0,1) [B,Q,G*D].  They
are packed planar into sampling_loc_attn [B,Q,G,L*K*3 + L*K] as the reference's tests do
(tests/test_flash_deform_attn.py:31-37).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    mode: str               # "self" or "cross"
    shapes: tuple           # ((D,H,W), ...) per level
    B: int
    Q: int                  # 0 = self-attention, Q = S
    G: int = 8
    D: int = 32
    K: int = 4
    dtype: str = "bf16"
    oob_frac: float = 0.0   # fraction of location triples drawn from U(-0.1, 1.1)

    @property
    def L(self) -> int:
        return len(self.shapes)

    @property
    def S(self) -> int:
        return sum(d * h * w for d, h, w in self.shapes)

    @property
    def nq(self) -> int:
        return self.Q if self.Q else self.S

    @property
    def P(self) -> int:
        return 4 * self.L * self.K

    def algorithmic_bytes(self, esize: int) -> dict:
        """Compulsory HBM traffic, each tensor once at its API dtype.
        fwd: value + sampling_loc_attn read, output written.
        bwd: value + sampling_loc_attn + grad_output read, grad_value + grad_sampling_loc_attn
        written."""
        v = self.B * self.S * self.G * self.D
        r = self.B * self.nq * self.G * self.P
        o = self.B * self.nq * self.G * self.D
        fwd = esize * (v + r + o)
        bwd = esize * (2 * v + 2 * r + o)
        return {"fwd": fwd, "bwd": bwd, "total": fwd + bwd}

    def samples(self) -> int:
        """queries * heads * samples per launch: B*Q*G*L*K."""
        return self.B * self.nq * self.G * self.L * self.K


WORKLOADS = {
    "c1": Workload("c1", "self", ((4, 8, 16), (2, 4, 8)), B=1, Q=0, dtype="fp32"),
    "c2": Workload("c2", "self", ((8, 16, 32), (4, 8, 16)), B=1, Q=0),
    "c3": Workload("c3", "cross", ((16, 32, 64), (8, 16, 32), (4, 8, 16)), B=2, Q=200, oob_frac=0.1),
    "c4": Workload("c4", "self", ((16, 32, 128), (8, 16, 64)), B=1, Q=0),
    "c5": Workload("c5", "self", ((32, 64, 256), (16, 32, 128), (8, 16, 64)), B=1, Q=0),
}

DTYPES = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def level_meta(shapes, device):
    """spatial_shapes [L,3] int64 and level_start_index [L] int64 on `device`."""
    st = torch.tensor([list(s) for s in shapes], dtype=torch.int64)
    lsi = torch.cat([st.new_zeros(1), st.prod(1).cumsum(0)[:-1]])
    return st.to(device), lsi.to(device)


def pack(locs: torch.Tensor, logits: torch.Tensor) -> torch.Tensor:
    B, Q, G, L, K = locs.shape[:5]
    return torch.cat([locs.reshape(B, Q, G, 3 * L * K), logits.reshape(B, Q, G, L * K)], dim=-1).contiguous()


def make_inputs(w: Workload, seed: int = 0, dtype=None, device="cpu", q_limit: int | None = None):
    """Seeded synthetic inputs for workload `w`.  Generated in fp32 with a generator on
    `device`, then cast to `dtype` (default: the workload's).  q_limit truncates the query
    count (for oracle-sized slices).  Returns a dict of tensors plus shapes/K."""
    dt = DTYPES[dtype or w.dtype] if isinstance(dtype or w.dtype, str) else dtype
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    Q = w.nq if q_limit is None else min(q_limit, w.nq)
    value = torch.randn(w.B, w.S, w.G, w.D, generator=gen, device=dev)
    locs = torch.rand(w.B, Q, w.G, w.L, w.K, 3, generator=gen, device=dev)
    if w.oob_frac > 0:
        wide = torch.rand(w.B, Q, w.G, w.L, w.K, 3, generator=gen, device=dev) * 1.2 - 0.1
        pick = torch.rand(w.B, Q, w.G, w.L, w.K, 1, generator=gen, device=dev) < w.oob_frac
        locs = torch.where(pick, wide, locs)
    logits = torch.randn(w.B, Q, w.G, w.L, w.K, generator=gen, device=dev)
    grad_out = torch.randn(w.B, Q, w.G * w.D, generator=gen, device=dev)
    shapes_t, lsi = level_meta(w.shapes, dev)
    return {
        "value": value.to(dt).contiguous(),
        "sampling_loc_attn": pack(locs, logits).to(dt),
        "grad_output": grad_out.to(dt).contiguous(),
        "spatial_shapes": shapes_t,
        "level_start_index": lsi,
        "shapes": [tuple(s) for s in w.shapes],
        "K": w.K,
    }
