#!/usr/bin/env python3
"""Benchmark of Flash Deformable 3D Attention forward+backward on one MI355X.

Default workload: c4, the headline configuration -- bf16 self-attention over a 256x512x2048
volume at strides 16/32 (levels (16,32,128) and (8,16,64), S = Q = 73728), B=1, G=8, D=32,
L=2, K=4, synthetic seeded inputs (value N(0,1), locations U(0,1), logits N(0,1), upstream
grad N(0,1)), all resident in HBM before timing.

A step is one forward + backward through FlashDeformAttnFunction (autograd), over one batch.
W untimed warmup steps, then K timed steps bracketed by torch.cuda.synchronize(); HIP events
on the launch stream give per-step times (median / p10 / p90) and, in separate loops, the
average duration of each kernel launch (HIP events the library records between its launches,
ops3d_fda_profile_*).

  value    = fwd+bwd algorithmic bytes / ms_per_step (GB/s).  Algorithmic bytes count each
             tensor once at its API dtype: fwd reads value + sampling_loc_attn and writes the
             output; bwd reads value + sampling_loc_attn + grad_output and writes grad_value +
             grad_sampling_loc_attn.
  roofline = the same figure for the dominant kernel alone, against 8 TB/s HBM3E peak: its
             algorithmic bytes over its average duration in the committed rocprofv3 summary
             (profiles/kernel_stats_<cfg>_bf16.md), and the same from this run's HIP events
             (frac_live); traffic = its rocprofv3 FETCH_SIZE + WRITE_SIZE bytes per dispatch.
  cpu_baseline = the PyTorch restatement of the reference's naive path (oracle/torch_port.py:
             grid_sample + softmax + autograd) in fp32 on the host CPU, on all queries when
             that fits the time target, else on a query slice scaled linearly to the full
             query count (the sample field says which).
  memory   = the library's forward / backward workspace sizes and torch's peak allocation of
             a step above the resident inputs.

--all prints a per-configuration table (c1..c5, plus fp16 and fp32 forward at c5) to stderr,
and at c4 and c5 the offset-mode op (FlashDeformAttnFromOffsets: caller-side fusion of the
location producer) against the unfused caller.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "fwd+bwd ms & achieved HBM GB/s (% of peak), bf16 self-attn S=73728, 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pct(xs, p):
    xs = sorted(xs)
    k = (len(xs) - 1) * p / 100.0
    lo, hi = int(k), min(int(k) + 1, len(xs) - 1)
    return xs[lo] + (xs[hi] - xs[lo]) * (k - lo)


def _rocprof_avg_us(kernel: str, workload: str):
    """Average dispatch duration (us) of `kernel` in the committed rocprofv3 --stats summary
    profiles/kernel_stats_<workload>_bf16.md (a cross-check of the event timing)."""
    path = os.path.join(ROOT, "profiles", f"kernel_stats_{workload}_bf16.md")
    if not os.path.exists(path):
        return None
    stem = kernel.replace("fda_bwd_query_kernel", "fda_bwd_query_pair_kernel").replace(
        "fda_forward_kernel", "fda_forward_pair_kernel")
    for line in open(path):
        m = re.match(r"\|\s*`" + re.escape(stem) + r"[<`][^|]*\|\s*\d+\s*\|\s*([0-9.]+)", line)
        if m:
            return float(m.group(1))
    return None


def _traffic_from_profiles(kernel: str, workload: str):
    """HBM bytes per dispatch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled
    by a copy-kernel calibration), read from profiles/pmc_<kernel>_<workload>.md."""
    path = os.path.join(ROOT, "profiles", f"pmc_{kernel}_{workload}.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"hbm_bytes_per_dispatch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


class Bench:
    def __init__(self, w, dtype, device, seed=0):
        import torch

        from ops3d_amd.workloads import make_inputs

        self.torch = torch
        self.w = w
        self.dtype = dtype
        self.dev = device
        inp = make_inputs(w, seed=seed, dtype=dtype, device=device)
        self.inp = inp
        self.value = inp["value"].requires_grad_(True)
        self.sla = inp["sampling_loc_attn"].requires_grad_(True)
        self.go = inp["grad_output"]
        self.st = inp["spatial_shapes"]
        self.lsi = inp["level_start_index"]
        self.esize = self.value.element_size()

    def step(self):
        from ops3d_amd import FlashDeformAttnFunction

        self.value.grad = None
        self.sla.grad = None
        out = FlashDeformAttnFunction.apply(self.value, self.st, self.lsi, self.sla, 64, self.w.K, True)
        out.backward(self.go)

    def fwd(self):
        from ops3d_amd import FlashDeformAttnFunction

        with self.torch.no_grad():
            FlashDeformAttnFunction.apply(self.value, self.st, self.lsi, self.sla, 64, self.w.K, True)

    def memory(self, base, peak):
        """Device memory of a fwd+bwd step: the library's workspaces (from its size queries)
        and torch's peak allocation above the resident inputs (outputs, gradients, saved
        forward workspace, backward workspace)."""
        from ops3d_amd import _C

        w = self.w
        code = {self.torch.float32: 0, self.torch.float16: 1, self.torch.bfloat16: 2}[self.value.dtype]
        args = (code, w.B, w.S, w.G, w.D, w.L, w.nq, w.K)
        return {
            "inputs_bytes": int(base),
            "fwd_workspace_bytes": int(_C._lib.ops3d_fda_forward_workspace_bytes(*args)),
            "bwd_workspace_bytes": int(_C._lib.ops3d_fda_backward_workspace_bytes(*args)),
            "step_peak_above_inputs_bytes": int(peak - base),
        }

    def time_loop(self, fn, steps, warmup):
        """Two timed loops of `steps` calls after `warmup` untimed ones.
        back-to-back: the calls run as a training loop runs them, between one pair of HIP events
          (synchronized on both sides); total_ms / steps is ms_per_step, the headline;
        per-step: a HIP event pair around every call, for the median / p10 / p90.  Each event
          pair costs the stream about 10 us (the event's completion and the next launch), so
          these per-step times sit above the back-to-back mean."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        total = a.elapsed_time(b)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in evs:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        ms = [a.elapsed_time(b) for a, b in evs]
        return {"total_ms": total, "wall_ms": wall, "mean": total / steps, "median": statistics.median(ms),
                "p10": pct(ms, 10), "p90": pct(ms, 90), "per_step_mean": sum(ms) / len(ms)}

    def kernel_times(self, steps, warmup):
        """Average launch duration (ms) of the forward kernel (events around its one-kernel
        call) and of each backward phase (events the library records between its launches)."""
        from ops3d_amd import _C

        torch = self.torch
        v, s = self.value.detach(), self.sla.detach()

        def run(fn, which):
            phases = {}
            for i in range(warmup + steps):
                fn()
                r = _C.profile_read(which)
                if i >= warmup:
                    for k, t in r.items():
                        phases.setdefault(k, []).append(t)
            out = {k: {"mean": sum(t) / len(t), "median": statistics.median(t)} for k, t in phases.items()}
            out["total"] = {"mean": sum(x["mean"] for x in out.values())}
            return out

        _C.profile_enable(True)
        try:
            fwd = run(lambda: _C.flash_deform_attn_forward(v, self.st, self.lsi, s, 64, self.w.K), "forward")
            # as in FlashDeformAttnFunction: the backward reuses the forward's head-major value
            _, vhm = _C.forward_keep_head_major(v, self.st, self.lsi, s, 64, self.w.K)
            bwd = run(lambda: _C.backward_with_head_major(v, vhm, self.st, self.lsi, s, self.go, 64, self.w.K),
                      "backward")
        finally:
            _C.profile_enable(False)
        return fwd, bwd


def measure_offsets(w, steps, warmup, device):
    """Caller-side fusion at workload w: fwd+bwd of FlashDeformAttnFromOffsets (offsets from one
    projection, locations formed in the kernels) against the caller the reference's tests
    write -- locations ref + offset / size and torch.cat in torch, the packed op, autograd
    splitting the gradient -- on the same inputs (bf16 offsets/logits, fp32 reference points)."""
    import torch

    from ops3d_amd import FlashDeformAttnFromOffsets, FlashDeformAttnFunction
    from ops3d_amd.workloads import make_inputs

    inp = make_inputs(w, seed=0, dtype=w.dtype, device=device)
    B, Q, G, L, K = w.B, w.nq, w.G, w.L, w.K
    n = 3 * L * K
    gen = torch.Generator(device=device).manual_seed(1)
    value = inp["value"].requires_grad_(True)
    oa = inp["sampling_loc_attn"].clone()
    oa[..., :n] = (torch.randn(B, Q, G, n, generator=gen, device=device) * 2.0).to(oa.dtype)
    oa.requires_grad_(True)
    ref = torch.rand(B, Q, 1, 3, generator=gen, device=device, requires_grad=True)
    st, lsi, go = inp["spatial_shapes"], inp["level_start_index"], inp["grad_output"]
    size = st.flip(-1).to(torch.float32).view(1, 1, 1, L, 1, 3)

    def fused():
        value.grad = oa.grad = ref.grad = None
        FlashDeformAttnFromOffsets.apply(value, st, lsi, oa, ref, 64, K).backward(go)

    def unfused():
        value.grad = oa.grad = ref.grad = None
        off = oa[..., :n].view(B, Q, G, L, K, 3)
        loc = (ref.view(B, Q, 1, 1, 1, 3) + off.float() / size).to(oa.dtype)
        sla = torch.cat([loc.reshape(B, Q, G, n), oa[..., n:]], -1)
        FlashDeformAttnFunction.apply(value, st, lsi, sla, 64, K, True).backward(go)

    b = Bench.__new__(Bench)
    b.torch = torch
    return {"fused": b.time_loop(fused, steps, warmup), "unfused": b.time_loop(unfused, steps, warmup)}


def measure_nms(n, steps, warmup, device, threshold=0.3, cpu=True):
    """3-D NMS over n clustered boxes (a few hundred clusters, extents 2-12, scores with ties):
    the whole _C.nms_3d call (sort, IoU mask, greedy pass, the kept count read back), and the
    float32 CPU oracle on the same boxes."""
    import numpy as np
    import torch

    from ops3d_amd import _C

    r = np.random.default_rng(0)
    centres = r.uniform(0, 100, size=(max(1, n // 20), 3))
    c = centres[r.integers(0, len(centres), n)] + r.normal(0, 3.0, size=(n, 3))
    e = r.uniform(2.0, 12.0, size=(n, 3))
    boxes = np.concatenate([c - e / 2, c + e / 2], 1).astype(np.float32)
    scores = np.round(r.uniform(0, 1, n), 2).astype(np.float32)
    b = torch.from_numpy(boxes).to(device)
    s = torch.from_numpy(scores).to(device)
    kept = []

    def call():
        kept.append(_C.nms_3d(b, s, threshold).numel())

    bb = Bench.__new__(Bench)
    bb.torch = torch
    res = {"n": n, "gpu": bb.time_loop(call, steps, warmup), "kept": kept[-1]}
    if cpu:
        from oracle import nms3d as O

        t0 = time.perf_counter()
        O.nms3d(boxes, scores, threshold)
        res["cpu_ms"] = (time.perf_counter() - t0) * 1e3
    return res


def measure_roi_align(steps, warmup, device, dtype="bf16"):
    """3-D RoI Align fwd and bwd: features [2, 256, 32, 64, 64], 512 rois of 4-32 voxels per
    axis, 7x7x7 bins, sampling_ratio 2 (8 trilinear samples per bin), linear order."""
    import numpy as np
    import torch

    from ops3d_amd.roi_align import roi_align_3d

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    N, C, D, H, W, R = 2, 256, 32, 64, 64, 512
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(N, C, D, H, W, generator=g, device=device).to(dt).requires_grad_(True)
    r = np.random.default_rng(0)
    ext = r.uniform(4, 32, size=(R, 3))
    lo = r.uniform(0, 1, size=(R, 3)) * (np.array([W, H, D]) - ext)
    rois = torch.from_numpy(np.concatenate([r.integers(0, N, (R, 1)), lo, lo + ext], 1).astype(np.float32))
    rois = rois.to(device).to(dt)
    pooled = (7, 7, 7)
    gout = torch.randn(R, C, *pooled, generator=g, device=device).to(dt)

    def fwd():
        with torch.no_grad():
            roi_align_3d(x, rois, pooled, 1.0, 2, 1)

    def step():
        x.grad = None
        roi_align_3d(x, rois, pooled, 1.0, 2, 1).backward(gout)

    b = Bench.__new__(Bench)
    b.torch = torch
    out_bytes = R * C * 343 * x.element_size()
    # the same forward on features already in channels_last_3d memory (no transposed copy)
    xcl = x.detach().contiguous(memory_format=torch.channels_last_3d)

    def fwd_cl():
        with torch.no_grad():
            roi_align_3d(xcl, rois, pooled, 1.0, 2, 1)

    def fwd_adaptive():   # sampling_ratio 0: ceil(extent / 7) samples per axis, 1-5 here
        with torch.no_grad():
            roi_align_3d(x, rois, pooled, 1.0, 0, 1)

    return {"fwd": b.time_loop(fwd, steps, warmup), "step": b.time_loop(step, steps, warmup),
            "fwd_cl": b.time_loop(fwd_cl, steps, warmup), "fwd_adaptive": b.time_loop(fwd_adaptive, steps, warmup),
            "samples": R * C * 343 * 8, "out_bytes": out_bytes}


def measure_dcnv4(steps, warmup, device, dtype="bf16"):
    """DCNv4-3D fwd and fwd+bwd: value [2, 32, 64, 64, 256] (G 8 x D 32), 3x3x3 kernel, stride 1,
    pad 1, softmax over the 27 masks, offsets ~N(0, 1) voxels."""
    import torch

    from ops3d_amd.dcnv4 import dcnv4_3d

    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    B, D_, H_, W_, G, D = 2, 32, 64, 64, 8, 32
    K = 27
    padded = (G * 4 * K + 7) // 8 * 8
    g = torch.Generator(device=device).manual_seed(0)
    value = torch.randn(B, D_, H_, W_, G * D, generator=g, device=device).to(dt).requires_grad_(True)
    off = torch.randn(B, D_, H_, W_, padded, generator=g, device=device).to(dt).requires_grad_(True)
    gout = torch.randn(B, D_, H_, W_, G * D, generator=g, device=device).to(dt)
    args = ((3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), G, D, 1.0, 64, 0, True)

    def fwd():
        with torch.no_grad():
            dcnv4_3d(value, off, *args)

    def step():
        value.grad = off.grad = None
        dcnv4_3d(value, off, *args).backward(gout)

    b = Bench.__new__(Bench)
    b.torch = torch
    return {"fwd": b.time_loop(fwd, steps, warmup), "step": b.time_loop(step, steps, warmup),
            "samples": B * D_ * H_ * W_ * G * K}


def measure_atomic_baseline(w, steps, warmup, device):
    """grad_value by the reference's scheme at the reference's lane layout (one fp32 atomic add per
    sample, corner and channel, one lane per channel; libops3d_fda_bench.so, with its clearing of
    the fp32 buffer) against the library's whole backward (which also computes
    grad_sampling_loc_attn), both on device-resident inputs of `w`; and the LDS float-atomic rate
    (ds_add_f32), which bounds any scheme that pre-combines the same adds in LDS."""
    import torch

    from ops3d_amd import _C, _bench_lib
    from ops3d_amd.workloads import make_inputs

    x = make_inputs(w, seed=0, device=device)
    args = (x["value"], x["spatial_shapes"], x["level_start_index"], x["sampling_loc_attn"], x["grad_output"])

    def timed(fn):
        for _ in range(warmup):
            fn()
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in evs:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        return statistics.median(a.elapsed_time(b) for a, b in evs)

    atomic = timed(lambda: _bench_lib.ref_scatter(*args, w.K))
    gather = timed(lambda: _C.flash_deform_attn_backward(*args, 64, w.K))
    adds = w.samples() * 8 * w.D   # upper bound: corners outside the volume add nothing
    blocks, iters = 256 * 8, 4096
    out = torch.empty(blocks, dtype=torch.float32, device=device)
    lds = {}
    for pattern in (0, 1):
        lds[pattern] = timed(lambda: _bench_lib.lds_atomic(out, blocks, iters, pattern))
        torch.cuda.synchronize()
        assert bool((out == 256.0 * iters).all()), "LDS atomic probe lost adds"
    lds_rate = blocks * 256 * iters / (min(lds.values()) * 1e-3)
    return {"atomic_ms": atomic, "backward_ms": gather, "atomic_adds": adds, "lds_adds_per_s": lds_rate,
            "lds_ms": lds, "lds_bound_ms": adds / lds_rate * 1e3}


def measure_gather_ceiling(device, sizes_mib=(2, 32, 512), groups=(4, 8, 32), blocks=4096, iters=256):
    """Random-gather ceiling (libops3d_fda_bench.so): TB/s at which waves fetch randomly placed
    blocks of 16 * group bytes (group lanes, one 16-byte load each) from buffers inside L2 (2
    MiB), inside the MALL (32 MiB) and in HBM (512 MiB).  Group 8 is the sampling kernels'
    128-byte x-pair line, group 4 a 64-byte row.  Median of 5 timed launches after one untimed."""
    import torch

    from ops3d_amd import _bench_lib

    out = torch.empty(blocks * 256, dtype=torch.int32, device=device)
    res = {}
    for mib in sizes_mib:
        src = torch.ones(mib << 18, dtype=torch.int32, device=device)   # mib MiB
        for g in groups:
            _bench_lib.gather(src, g, blocks, iters, out)
            ts = []
            for k in range(5):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                _bench_lib.gather(src, g, blocks, iters, out, seed=k + 2)
                b.record()
                torch.cuda.synchronize()
                ts.append(a.elapsed_time(b))
            res[(mib, g)] = blocks * 256 * iters * 16 / (statistics.median(ts) * 1e-3) / 1e12
        del src
    return res


def measure(w, dtype, steps, warmup, device, with_kernels=True, fwd_only=False):
    b = Bench(w, dtype, device)
    res = {"workload": w.name, "dtype": dtype}
    by = w.algorithmic_bytes(b.esize)
    res["bytes"] = by
    res["fwd"] = b.time_loop(b.fwd, steps, warmup)
    if not fwd_only:
        import torch

        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        res["step"] = b.time_loop(b.step, steps, warmup)
        res["memory"] = b.memory(base, torch.cuda.max_memory_allocated())
    if with_kernels:
        fk, bk = b.kernel_times(steps, warmup)
        res["fwd_kernel"], res["bwd_kernel"] = fk, bk
    del b
    import torch

    torch.cuda.empty_cache()
    return res


def cpu_baseline(w, target_s=4.0, reps=5, warmup=2):
    """fp32 PyTorch naive path on the host CPU, fwd+bwd over a query slice of `w`."""
    import torch

    from oracle import torch_port
    from ops3d_amd.workloads import make_inputs

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(cores)
    nq = min(w.nq, 1024)
    while True:
        inp = make_inputs(w, seed=0, dtype="fp32", device="cpu", q_limit=nq)
        t0 = time.perf_counter()
        torch_port.forward_backward(inp["value"], inp["shapes"], inp["sampling_loc_attn"], inp["grad_output"], w.K)
        dt = time.perf_counter() - t0
        if dt >= target_s / 4 or nq >= w.nq:
            break
        nq = min(w.nq, nq * max(2, int(target_s / 4 / max(dt, 1e-3))))
    for _ in range(warmup):   # the sizing run above was the first
        torch_port.forward_backward(inp["value"], inp["shapes"], inp["sampling_loc_attn"], inp["grad_output"], w.K)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        torch_port.forward_backward(inp["value"], inp["shapes"], inp["sampling_loc_attn"], inp["grad_output"], w.K)
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    t_full = t * w.nq / nq
    scaled = nq < w.nq
    by = w.algorithmic_bytes(2 if w.dtype in ("bf16", "fp16") else 4)["total"]
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    if scaled:
        what = (f"on {nq} of {w.nq} queries of {w.name}, median of {reps} after {warmup + 1} untimed, {t:.2f} s per rep, scaled "
                f"linearly to the full query count ({t_full * 1e3:.0f} ms)")
    else:
        what = f"on all {w.nq} queries of {w.name}, median of {reps} after {warmup + 1} untimed, {t:.2f} s per rep"
    return {
        "value": round(by / t_full / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"oracle/torch_port fp32 fwd+bwd (grid_sample+softmax+autograd) {what}; CPU: {cpu}",
        "ms_full_workload": round(t_full * 1e3, 1),
        "queries_timed": nq,
    }


def config_entry(r, w, dt, steps):
    """One configuration's figures for the JSON line: back-to-back mean ms (and the per-step
    median) of the forward and of forward+backward, algorithmic GB/s and fraction of 8 TB/s,
    queries*heads*samples per second."""
    by = r["bytes"]
    f = r["fwd"]["mean"]
    e = {"dtype": dt, "steps": steps, "B": w.B, "Q": w.nq, "S": w.S, "L": w.L,
         "fwd_ms": round(f, 5), "fwd_ms_median": round(r["fwd"]["median"], 5),
         "fwd_gbs": round(by["fwd"] / f / 1e6, 1), "fwd_frac_of_hbm_peak": round(by["fwd"] / f / 1e6 / HBM_PEAK_GBS, 4),
         "fwd_qhs_per_s": round(w.samples() / (f * 1e-3), 1)}
    if "step" in r:
        t = r["step"]["mean"]
        e.update({"fwd_bwd_ms": round(t, 5), "fwd_bwd_ms_median": round(r["step"]["median"], 5),
                  "fwd_bwd_gbs": round(by["total"] / t / 1e6, 1),
                  "fwd_bwd_frac_of_hbm_peak": round(by["total"] / t / 1e6 / HBM_PEAK_GBS, 4),
                  "fwd_bwd_qhs_per_s": round(w.samples() / (t * 1e-3), 1)})
    return e


def summary_line(r):
    by = r["bytes"]
    f = r["fwd"]["mean"]
    s = r.get("step", {}).get("mean")
    fk = r.get("fwd_kernel", {}).get("total", {}).get("mean")
    bk = r.get("bwd_kernel", {}).get("total", {}).get("mean")
    samples = r["samples"]
    parts = [f"{r['workload']:>3} {r['dtype']:>4}", f"fwd {f * 1e3:8.1f} us ({by['fwd'] / f / 1e6:7.0f} GB/s, "
             f"{100 * by['fwd'] / f / 1e6 / HBM_PEAK_GBS:5.1f}%)"]
    if s:
        parts.append(f"fwd+bwd {s * 1e3:8.1f} us ({by['total'] / s / 1e6:7.0f} GB/s, "
                     f"{100 * by['total'] / s / 1e6 / HBM_PEAK_GBS:5.1f}%)")
    if fk:
        fp = r["fwd_kernel"]
        parts.append(f"fwd call {fk * 1e3:7.1f} us [copy {fp['head_major_copy']['mean'] * 1e3:.1f} "
                     f"k {fp['forward_kernel']['mean'] * 1e3:.1f}]")
    if bk:
        ph = r["bwd_kernel"]
        parts.append(f"bwd {bk * 1e3:7.1f} us [copy {ph['head_major_copies']['mean'] * 1e3:.1f} "
                     f"q {ph['query_kernel']['mean'] * 1e3:.1f} count {ph['tile_count']['mean'] * 1e3:.1f} "
                     f"scatter {ph['tile_scatter']['mean'] * 1e3:.1f} tile {ph['tile_kernel']['mean'] * 1e3:.1f}]")
    parts.append(f"{samples / (s or f) / 1e6:.3g} Gsamples/s" if (s or f) else "")
    if "memory" in r:
        m = r["memory"]
        parts.append(f"ws fwd {m['fwd_workspace_bytes'] / 2**20:.0f} MiB bwd {m['bwd_workspace_bytes'] / 2**20:.0f} MiB, "
                     f"step peak +{m['step_peak_above_inputs_bytes'] / 2**20:.0f} MiB")
    return " | ".join(parts)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c4")
    ap.add_argument("--all", action="store_true", help="also report every configuration (stderr)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true",
                    help="only the headline configuration (skip c1, c2, c3, c5 and the c5 fp16/fp32 forwards)")
    ap.add_argument("--json-out", default=None, help="write all results as JSON to this path")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the per-kernel loops of --config (for profilers); prints no JSON line")
    ap.add_argument("--nms", action="store_true", help="only 3-D NMS at 4k, 16k and 64k boxes (stderr)")
    ap.add_argument("--roi", action="store_true", help="only 3-D RoI Align fwd and fwd+bwd (stderr)")
    ap.add_argument("--dcn", action="store_true", help="only DCNv4-3D fwd and fwd+bwd (stderr)")
    ap.add_argument("--offsets", action="store_true",
                    help="only the offset-mode op against the unfused caller at --config (stderr)")
    ap.add_argument("--atomic-baseline", action="store_true",
                    help="only grad_value by the reference's fp32 atomic scatter against the library's "
                         "backward, at --config (stderr)")
    ap.add_argument("--gather-ceiling", action="store_true",
                    help="only the random-gather ceiling (TB/s for 64 to 512-byte blocks from L2, MALL, HBM)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB, 5 times (HBM counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs on one GPU only "
              f"(the flash-deform-attn path has no multi-GPU mode); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import ops3d_amd
    from ops3d_amd.workloads import WORKLOADS

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    if ops3d_amd._C is None:
        print("bench.py: libops3d_fda.so is not built (run __graft_entry__.build())", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    log(f"device: {torch.cuda.get_device_name(0)}; torch {torch.__version__}")
    if args.copy_calibration:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {args.copy_calibration} MiB 5 times")
        return
    if args.gather_ceiling:
        o = measure_gather_ceiling(dev)
        for mib in sorted({k[0] for k in o}):
            log(f" random gather from a {mib:4d} MiB buffer | " +
                " | ".join(f"{16 * g:4d}-byte blocks {o[(mib, g)]:6.2f} TB/s" for g in sorted({k[1] for k in o})))
        return
    if args.dcn or args.all:
        o = measure_dcnv4(args.steps, args.warmup, dev)
        f, st = o["fwd"]["mean"], o["step"]["mean"]
        log(f" dcnv4_3d bf16 [2,32,64,64,8x32] 3^3 taps, softmax | fwd {f * 1e3:8.1f} us "
            f"({o['samples'] / f / 1e6:.3g} G samples/s) | fwd+bwd {st * 1e3:8.1f} us")
        if args.dcn:
            return
    if args.roi or args.all:
        o = measure_roi_align(args.steps, args.warmup, dev)
        f, st = o["fwd"]["mean"], o["step"]["mean"]
        log(f" roi_align3d bf16 [2,256,32,64,64] x 512 rois, 7^3 bins, 8 samples | fwd {f * 1e3:8.1f} us "
            f"({o['samples'] / f / 1e6:.3g} G samples/s) | fwd+bwd {st * 1e3:8.1f} us | fwd on channels_last_3d "
            f"features {o['fwd_cl']['mean'] * 1e3:8.1f} us | fwd with sampling_ratio 0 (adaptive) "
            f"{o['fwd_adaptive']['mean'] * 1e3:8.1f} us")
        if args.roi:
            return
    if args.nms or args.all:
        for n in (4096, 16384, 65536):
            o = measure_nms(n, args.steps, args.warmup, dev, cpu=n <= 16384)
            cpu = f" | CPU oracle (numpy fp32, 1 core) {o['cpu_ms']:9.1f} ms" if "cpu_ms" in o else ""
            log(f" nms3d n={n:6d} | GPU {o['gpu']['median'] * 1e3:9.1f} us per call (sort + mask + greedy + count), "
                f"kept {o['kept']}{cpu}")
        if args.nms:
            return
    if args.offsets:
        o = measure_offsets(WORKLOADS[args.config], args.steps, args.warmup, dev)
        log(f" {args.config} offsets | fwd+bwd fused (FlashDeformAttnFromOffsets) {o['fused']['median'] * 1e3:8.1f} us"
            f" | unfused caller (ref + off/size, cat, packed op) {o['unfused']['median'] * 1e3:8.1f} us")
        return
    if args.atomic_baseline or args.all:
        name = args.config if args.atomic_baseline else "c4"
        o = measure_atomic_baseline(WORKLOADS[name], max(3, min(args.steps, 10)), 2, dev)
        log(f" {name} grad_value by fp32 atomics (reference scheme and lane layout) {o['atomic_ms'] * 1e3:9.1f} us "
            f"({o['atomic_adds'] / (o['atomic_ms'] * 1e-3) / 1e9:.0f} G adds/s) | library backward (all "
            f"gradients) {o['backward_ms'] * 1e3:8.1f} us | LDS ds_add_f32 {o['lds_adds_per_s'] / 1e9:.0f} G adds/s "
            f"(consecutive {o['lds_ms'][0]:.2f} ms, random {o['lds_ms'][1]:.2f} ms for {256 * 8 * 256 * 4096:d} adds): "
            f"the same adds pre-combined in LDS take at least {o['lds_bound_ms'] * 1e3:.0f} us")
        if args.atomic_baseline:
            return
    if args.kernels_only:
        w = WORKLOADS[args.config]
        b = Bench(w, w.dtype, dev)
        fk, bk = b.kernel_times(args.steps, args.warmup)
        log(f"{w.name}: forward " + ", ".join(f"{k} {v['mean'] * 1e3:.1f} us" for k, v in fk.items())
            + "; backward " + ", ".join(f"{k} {v['mean'] * 1e3:.1f} us" for k, v in bk.items()))
        return

    results = []
    configs = {}
    if not args.no_configs:
        # every BASELINE configuration (reference tests/benchmark_flash_deform_attn.py:105-116 is
        # where the grid comes from), plus the fp16 and fp32 forwards at c5; c4 is the headline
        # below and is filled in from it
        plan = [(n, WORKLOADS[n].dtype, False) for n in ("c1", "c2", "c3", "c5")]
        plan += [("c5", "fp16", True), ("c5", "fp32", True)]
        for name, dt, fo in plan:
            w = WORKLOADS[name]
            steps = min(args.steps, 20) if name == "c5" else min(args.steps, 30)
            log(f"[bench] {name} {dt} fwd_only={fo} steps={steps}")
            r = measure(w, dt, steps, min(args.warmup, 5), dev, with_kernels=args.all, fwd_only=fo)
            r["samples"] = w.samples()
            results.append(r)
            log(summary_line(r))
            configs[f"{name}_{dt}" + ("_fwd" if fo else "")] = config_entry(r, w, dt, steps)

    if args.all:
        for name in ("c4", "c5"):
            o = measure_offsets(WORKLOADS[name], args.steps, args.warmup, dev)
            log(f" {name} offsets | fwd+bwd fused (FlashDeformAttnFromOffsets) {o['fused']['mean'] * 1e3:8.1f} us"
                f" | unfused caller (ref + off/size, cat, packed op) {o['unfused']['mean'] * 1e3:8.1f} us")
            results.append({"workload": name, "offsets": o})
            torch.cuda.empty_cache()

    w = WORKLOADS[args.config]
    log(f"[bench] headline {w.name} {w.dtype} steps={args.steps} warmup={args.warmup}")
    r = measure(w, w.dtype, args.steps, args.warmup, dev)
    r["samples"] = w.samples()
    log(summary_line(r))
    by = r["bytes"]
    ms_step = r["step"]["mean"]   # back-to-back loop: total / steps
    ph = r["bwd_kernel"]
    e = 2 if w.dtype in ("bf16", "fp16") else 4
    V, R, O = w.B * w.S * w.G * w.D * e, w.B * w.nq * w.G * w.P * e, w.B * w.nq * w.G * w.D * e
    # per-kernel algorithmic bytes (each API tensor the kernel must touch, once):
    #   forward: read value + sampling_loc_attn, write output
    #   backward query kernel: read value + sampling_loc_attn + grad_output, write grad_sampling_loc_attn
    #   backward tile kernel: read grad_output, write grad_value
    kern = {
        "fda_forward_kernel": (r["fwd_kernel"]["forward_kernel"]["mean"], V + R + O),
        "fda_bwd_query_kernel": (ph["query_kernel"]["mean"], V + 2 * R + O),
        "fda_bwd_tile_kernel": (ph["tile_kernel"]["mean"], O + V),
        "tile_bucketing": (ph["tile_count"]["mean"] + ph["tile_scatter"]["mean"], None),
    }
    dominant = max(kern, key=lambda k: kern[k][0])
    kms, kbytes = kern[dominant]
    if kbytes is None:  # the bucketing moves only internal entries; report the backward as a whole
        dominant, kms, kbytes = "backward (all phases)", ph["total"]["mean"], by["bwd"]
    achieved = kbytes / (kms * 1e-3) / 1e9
    kf, kb = r["fwd_kernel"]["total"]["mean"], ph["total"]["mean"]
    traffic = _traffic_from_profiles(dominant, w.name)
    rp_us = _rocprof_avg_us(dominant, w.name)
    achieved_rp = kbytes / (rp_us * 1e-6) / 1e9 if rp_us else None
    line = {
        "metric": METRIC,
        "value": round(by["total"] / (ms_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w.dtype == "bf16" else w.dtype,
        "data": "synthetic (seeded: value N(0,1), locations U(0,1), logits N(0,1), grad N(0,1))",
        "config": {
            "workload": f"{w.name}: {w.mode}-attention, levels {list(w.shapes)}, S={w.S}, B={w.B}, "
                        f"Q={w.nq}, G={w.G}, D={w.D}, L={w.L}, K={w.K}, fwd+bwd",
            "B": w.B, "Q": w.nq, "S": w.S, "G": w.G, "D": w.D, "L": w.L, "K": w.K,
        },
        "timing": ("value, ms_per_step, fwd_ms: K back-to-back steps between one pair of HIP events "
                   "(synchronized on both sides), total / K; *_median, *_p10, *_p90: a second loop of K "
                   "steps with an event pair around each (each pair adds about 10 us per step)"),
        "fwd_bwd_ms_median": round(r["step"]["median"], 5),
        "fwd_bwd_ms_p10": round(r["step"]["p10"], 5),
        "fwd_bwd_ms_p90": round(r["step"]["p90"], 5),
        "fwd_ms": round(r["fwd"]["mean"], 5),
        "fwd_ms_median": round(r["fwd"]["median"], 5),
        "frac_of_hbm_peak": round(by["total"] / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "qhs_per_s": round(w.samples() / (ms_step * 1e-3), 1),
        "kernels_us": {**{k: round(v[0] * 1e3, 2) for k, v in kern.items()},
                       "head_major_copy_fwd": round(r["fwd_kernel"]["head_major_copy"]["mean"] * 1e3, 2),
                       "head_major_copies_bwd": round(ph["head_major_copies"]["mean"] * 1e3, 2),
                       "tile_count_scan": round(ph["tile_count"]["mean"] * 1e3, 2),
                       "tile_scatter": round(ph["tile_scatter"]["mean"] * 1e3, 2),
                       "forward_total": round(kf * 1e3, 2), "backward_total": round(kb * 1e3, 2)},
        "roofline": {
            "kernel": dominant,
            "bound": "hbm",
            "achieved": round(achieved_rp if rp_us else achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round((achieved_rp if rp_us else achieved) / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": kbytes,
            "duration_us": round(rp_us if rp_us else kms * 1e3, 2),
            "duration_source": (f"rocprofv3 --kernel-trace --stats average of the kernel in "
                                f"profiles/kernel_stats_{w.name}_bf16.md (frac = algorithmic_bytes / duration_us / "
                                f"peak, recomputable from that file)" if rp_us else
                                "HIP events the library records around the kernel on its launch stream (no committed "
                                "rocprof summary for this configuration)"),
            "duration_us_live": round(kms * 1e3, 2),
            "achieved_live": round(achieved, 2),
            "frac_live": round(achieved / HBM_PEAK_GBS, 4),
            "live_source": "HIP events the library records around the kernel on its launch stream, mean over "
                           "this run's timed calls",
            "graded": "frac",
            "traffic_ratio": round(traffic / kbytes, 2) if traffic else None,
            "traffic_source": (f"profiles/pmc_{dominant}_{w.name}.md: rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE per "
                               f"dispatch, scaled by the copy-kernel calibration" if traffic is not None else None),
        },
        "memory": r["memory"],
        "cpu_baseline": None,
    }
    if configs:
        configs[f"{w.name}_{w.dtype}"] = config_entry(r, w, w.dtype, args.steps)
        line["configs"] = dict(sorted(configs.items()))
    if not args.no_cpu:
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline(w)
    if args.json_out:
        with open(args.json_out, "w") as f:
            json.dump({"headline": line, "configs": results + [r]}, f, indent=1, default=str)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
