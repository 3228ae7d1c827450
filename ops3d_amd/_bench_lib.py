"""ctypes binding of libops3d_fda_bench.so (include/ops3d_fda_bench.h): measurement baselines (the
backward's value gradient by atomics, the LDS atomic rate, the random-gather ceiling), not part of
the op.  Used by bench.py --atomic-baseline / --gather-ceiling and their tests only."""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libops3d_fda_bench.so")
_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_lib = None


def load() -> ctypes.CDLL:
    """The measurement library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (python -m ops3d_amd._build)")
        lib = ctypes.CDLL(LIB_PATH)
        vp, i = ctypes.c_void_p, ctypes.c_int
        lib.ops3d_fda_bench_last_error.restype = ctypes.c_char_p
        lib.ops3d_fda_bench_ref_scatter.restype = i
        lib.ops3d_fda_bench_ref_scatter.argtypes = [vp] * 5 + [i] * 8 + [vp]
        lib.ops3d_fda_bench_lds_atomic.restype = i
        lib.ops3d_fda_bench_lds_atomic.argtypes = [vp, i, i, i, vp]
        lib.ops3d_fda_bench_gather.restype = i
        lib.ops3d_fda_bench_gather.argtypes = [vp, ctypes.c_size_t, i, i, i, vp, ctypes.c_uint, vp]
        _lib = lib
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        msg = load().ops3d_fda_bench_last_error().decode()
        raise (ValueError if rc == 1 else RuntimeError)(msg)


def ref_scatter(value, spatial_shapes, level_start_index, sampling_loc_attn, grad_output, K: int):
    """grad_value [B, S, G, D] (fp32) by the reference's atomic scheme and lane layout."""
    lib = load()
    B, S, G, D = value.shape
    L, Q = spatial_shapes.shape[0], sampling_loc_attn.shape[1]
    gv = torch.empty(value.shape, dtype=torch.float32, device=value.device)
    with torch.cuda.device(value.device):
        _check(lib.ops3d_fda_bench_ref_scatter(
            spatial_shapes.data_ptr(), level_start_index.data_ptr(), sampling_loc_attn.data_ptr(),
            grad_output.data_ptr(), gv.data_ptr(), _DT[value.dtype], B, S, G, D, L, Q, int(K),
            torch.cuda.current_stream(value.device).cuda_stream))
    return gv


def gather(src: torch.Tensor, group: int, blocks: int, iters: int, out: torch.Tensor, seed: int = 1) -> None:
    """Launch the random-gather probe over the bytes of `src` (out: int32 device tensor of at
    least blocks * 256 elements)."""
    lib = load()
    _check(lib.ops3d_fda_bench_gather(src.data_ptr(), src.numel() * src.element_size(), int(group), int(blocks),
                                      int(iters), out.data_ptr(), int(seed),
                                      torch.cuda.current_stream(src.device).cuda_stream))


def lds_atomic(out: torch.Tensor, blocks: int, iters: int, pattern: int) -> None:
    """Launch the LDS float-atomic probe (out: fp32 device tensor of at least `blocks` elements)."""
    lib = load()
    _check(lib.ops3d_fda_bench_lds_atomic(out.data_ptr(), int(blocks), int(iters), int(pattern),
                                          torch.cuda.current_stream(out.device).cuda_stream))
