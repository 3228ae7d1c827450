"""GPU parity of offset mode (FlashDeformAttnFromOffsets / ops3d_fda_*_offsets, the caller-side
fusion of the op's producer and consumer) and of the FlashDeformAttn3D module.

The oracle is the float64 C oracle on the packed locations loc = ref + offset / size formed in
fp32 step by step (what the kernels form, and what a caller packing fp32 locations passes);
offset gradients are the oracle's location gradients divided by the level size, reference
point gradients their sums over heads and points.  Tolerances as in test_gpu_fda.py: fp32 rtol
1e-5 / atol 1e-6 (location gradients plus oracle.fp32_loc_allowance, divided by the level size
for offsets), bf16 rtol 2e-2 / atol 2e-2."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fda_helpers import TOL, assert_close, log
from ops3d_amd import FlashDeformAttn3D, FlashDeformAttnFromOffsets, FlashDeformAttnFunction
from ops3d_amd.workloads import level_meta, pack

pytestmark = pytest.mark.gpu


def _inputs(shapes, B, Q, G, D, K, R, dt, seed):
    g = torch.Generator().manual_seed(seed)
    L = len(shapes)
    S = sum(a * b * c for a, b, c in shapes)
    value = torch.randn(B, S, G, D, generator=g).to(dt)
    ref = torch.rand(B, Q, R, 3, generator=g) * 1.1 - 0.05                 # some near or past the edge
    off = (torch.randn(B, Q, G, L, K, 3, generator=g) * 2.0).to(dt)        # voxels of the level
    logits = torch.randn(B, Q, G, L, K, generator=g).to(dt)
    go = torch.randn(B, Q, G * D, generator=g).to(dt)
    oa = torch.cat([off.reshape(B, Q, G, 3 * L * K), logits.reshape(B, Q, G, L * K)], -1).contiguous()
    return value, ref, off, logits, oa, go


def _locations_fp32(shapes, ref, off, L, K):
    """loc = ref + offset / size per level and axis, each step rounded in fp32 (numpy)."""
    B, Q, G = off.shape[:3]
    R = ref.shape[2]
    size = np.array([[w, h, d] for d, h, w in shapes], dtype=np.float32)          # (W, H, D)
    o = off.to(torch.float32).numpy().reshape(B, Q, G, L, K, 3)
    r = ref.numpy().astype(np.float32)
    r = r.reshape(B, Q, 1, R, 1, 3) if R > 1 else r.reshape(B, Q, 1, 1, 1, 3)
    q = (o / size.reshape(1, 1, 1, L, 1, 3)).astype(np.float32)
    return (r + q).astype(np.float32)


def _oracle(shapes, value, ref, off, logits, go, K):
    B, Q, G, L = off.shape[0], off.shape[1], off.shape[2], len(shapes)
    loc = _locations_fp32(shapes, ref, off, L, K)
    sla = np.concatenate([loc.reshape(B, Q, G, 3 * L * K), logits.to(torch.float32).numpy().reshape(B, Q, G, L * K)],
                         -1).astype(np.float64)
    v = value.double().numpy()
    out = oracle.forward(v, shapes, sla, K, coord_mode=1)
    gv, gs = oracle.backward(v, shapes, sla, go.double().numpy(), K, coord_mode=1)
    allow = oracle.fp32_loc_allowance(v, shapes, sla, go.double().numpy(), K)
    size = np.array([[w, h, d] for d, h, w in shapes], dtype=np.float64).reshape(1, 1, 1, L, 1, 3)
    gl = gs[..., : 3 * L * K].reshape(B, Q, G, L, K, 3)
    goff = (gl / size).reshape(B, Q, G, 3 * L * K)
    aoff = (allow[..., : 3 * L * K].reshape(B, Q, G, L, K, 3) / size).reshape(B, Q, G, 3 * L * K)
    R = ref.shape[2]
    gref = gl.sum(axis=(2, 4))                                   # [B, Q, L, 3]
    aref = allow[..., : 3 * L * K].reshape(B, Q, G, L, K, 3).sum(axis=(2, 4))
    if R == 1:
        gref, aref = gref.sum(axis=2, keepdims=True), aref.sum(axis=2, keepdims=True)
    return out, gv, goff, gs[..., 3 * L * K:], gref, aoff, aref


CASES = [
    # shapes, B, Q, G, D, K, R, dtype
    ([(6, 8, 10), (3, 4, 5)], 2, 150, 8, 32, 4, 2, torch.float32),
    ([(6, 8, 10), (3, 4, 5)], 2, 150, 8, 32, 4, 1, torch.bfloat16),
    ([(16, 32, 64), (8, 16, 32), (4, 8, 16)], 1, 300, 8, 32, 4, 3, torch.bfloat16),
    ([(5, 6, 7)], 1, 64, 4, 16, 8, 1, torch.float32),
    ([(5, 6, 7), (3, 3, 4)], 1, 100, 3, 48, 4, 2, torch.float16),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_offsets_vs_oracle(gpu_device, case):
    shapes, B, Q, G, D, K, R, dt = CASES[case]
    L = len(shapes)
    log(f"[case] offsets #{case}: shapes={shapes} B={B} Q={Q} G={G} D={D} K={K} R={R} {dt}")
    value, ref, off, logits, oa, go = _inputs(shapes, B, Q, G, D, K, R, dt, seed=case)
    st, lsi = level_meta(shapes, gpu_device)
    v = value.to(gpu_device).requires_grad_(True)
    o = oa.to(gpu_device).requires_grad_(True)
    r = ref.to(gpu_device).requires_grad_(True)
    out = FlashDeformAttnFromOffsets.apply(v, st, lsi, o, r, 64, K)
    out.backward(go.to(gpu_device))
    torch.cuda.synchronize()
    ro, rgv, rgoff, rglog, rgref, aoff, aref = _oracle(shapes, value, ref, off, logits, go, K)
    rtol, atol = TOL[dt]
    fp32 = dt == torch.float32
    n = 3 * L * K
    assert_close("output", out.detach(), ro, rtol, atol)
    assert_close("grad_value", v.grad, rgv, rtol, atol)
    assert_close("grad_offset", o.grad[..., :n], rgoff, rtol, atol, aoff if fp32 else None)
    assert_close("grad_logit", o.grad[..., n:], rglog, rtol, atol)
    # reference points: fp32 sums of the offset gradients times the level size
    assert_close("grad_ref", r.grad, rgref, rtol, atol * n * G, (aref + 1e-6 * np.abs(rgref)) if fp32 else None)


def test_offsets_equal_packed_path_fp32(gpu_device):
    """fp32: the offset-mode forward is bitwise the packed forward on locations the caller forms
    in fp32 (ref + offset / size); logit gradients bitwise too, offset gradients are the location
    gradients divided by the size."""
    shapes, B, Q, G, D, K = [(6, 8, 10), (3, 4, 5)], 2, 200, 8, 32, 4
    L = len(shapes)
    log("[case] offsets == packed, fp32")
    value, ref, off, logits, oa, go = _inputs(shapes, B, Q, G, D, K, L, torch.float32, seed=11)
    dev = gpu_device
    st, lsi = level_meta(shapes, dev)
    size = torch.tensor([[w, h, d] for d, h, w in shapes], dtype=torch.float32, device=dev).view(1, 1, 1, L, 1, 3)
    r = ref.to(dev)
    loc = r.view(B, Q, 1, L, 1, 3) + off.to(dev).view(B, Q, G, L, K, 3) / size
    sla = pack(loc, logits.to(dev)).requires_grad_(True)
    v1 = value.to(dev).requires_grad_(True)
    out_p = FlashDeformAttnFunction.apply(v1, st, lsi, sla, 64, K, True)
    out_p.backward(go.to(dev))
    v2 = value.to(dev).requires_grad_(True)
    o2 = oa.to(dev).requires_grad_(True)
    out_o = FlashDeformAttnFromOffsets.apply(v2, st, lsi, o2, r, 64, K)
    out_o.backward(go.to(dev))
    torch.cuda.synchronize()
    n = 3 * L * K
    assert torch.equal(out_p, out_o)
    assert torch.equal(sla.grad[..., n:], o2.grad[..., n:])
    gl = sla.grad[..., :n].view(B, Q, G, L, K, 3)
    assert_close("grad_offset vs grad_loc / size", o2.grad[..., :n], (gl / size).reshape(B, Q, G, n).cpu().numpy(),
                 1e-6, 1e-7)
    assert_close("grad_value", v2.grad, v1.grad.double().cpu().numpy(), *TOL[torch.float32])


def test_module_matches_unfused_caller(gpu_device):
    """FlashDeformAttn3D (one projection, offset mode) against the same module written the way
    the reference's callers feed the op (locations computed and concatenated in torch, the
    packed op): outputs and the gradients of every parameter, the query, the value input and
    the reference points."""
    torch.manual_seed(0)
    dev = gpu_device
    shapes = [(8, 16, 32), (4, 8, 16)]
    L, G, K, C, B, Q = len(shapes), 8, 4, 256, 2, 500
    S = sum(a * b * c for a, b, c in shapes)
    log("[case] FlashDeformAttn3D vs unfused caller, fp32")
    m = FlashDeformAttn3D(C, G, L, K).to(dev)
    with torch.no_grad():
        m.sampling.weight.normal_(0.0, 0.05)
    query = torch.randn(B, Q, C, device=dev, requires_grad=True)
    value_in = torch.randn(B, S, C, device=dev, requires_grad=True)
    ref = torch.rand(B, Q, 1, 3, device=dev, requires_grad=True)
    st, lsi = level_meta(shapes, dev)
    out = m(query, ref, value_in, st, lsi)
    gout = torch.randn_like(out)
    out.backward(gout)
    grads = [p.grad.clone() for p in m.parameters()] + [query.grad.clone(), value_in.grad.clone(), ref.grad.clone()]
    for p in list(m.parameters()) + [query, value_in, ref]:
        p.grad = None
    # the unfused caller: split the projection, form locations, concatenate, packed op
    size = torch.tensor([[w, h, d] for d, h, w in shapes], dtype=torch.float32, device=dev).view(1, 1, 1, L, 1, 3)
    v = m.value_proj(value_in).view(B, S, G, C // G)
    proj = m.sampling(query).view(B, Q, G, 4 * L * K)
    off = proj[..., : 3 * L * K].reshape(B, Q, G, L, K, 3)
    loc = ref.view(B, Q, 1, 1, 1, 3) + off / size
    sla = torch.cat([loc.reshape(B, Q, G, 3 * L * K), proj[..., 3 * L * K:]], -1)
    out2 = m.output_proj(FlashDeformAttnFunction.apply(v, st, lsi, sla.contiguous(), 64, K, True))
    out2.backward(gout)
    grads2 = [p.grad for p in m.parameters()] + [query.grad, value_in.grad, ref.grad]
    torch.cuda.synchronize()
    assert_close("module output", out, out2.detach().double().cpu().numpy(), 1e-5, 1e-6)
    names = [n for n, _ in m.named_parameters()] + ["query", "value_input", "reference_points"]
    for name, a, b in zip(names, grads, grads2):
        # fp32 sums over up to Q*G*L*K terms in different orders: relative to the largest gradient
        scale = float(b.abs().max())
        assert_close(f"grad {name}", a, b.double().cpu().numpy(), 1e-4, 1e-5 * max(scale, 1.0))
