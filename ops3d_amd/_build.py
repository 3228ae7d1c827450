"""Build libops3d_fda.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc, and the PyTorch
extension module over it (g++ against torch's headers).

gfx950 only, no hipify, no CUDA headers.  Sources are compiled in parallel, then linked with
hipcc.  Used by ``setup.py`` and ``__graft_entry__.build()``; also runnable as
``python -m ops3d_amd._build``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libops3d_fda.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
TORCH_EXT_NAME = "_fda_torch"
SOURCES = ["fda_capi.hip", "fda_tiles.hip", "fda_f32.hip", "fda_f16.hip", "fda_bf16.hip", "nms3d.hip", "roi_align3d.hip"]
# measurement baselines (not part of the op): a library of their own
BENCH_SOURCE = "bench_scatter.hip"
BENCH_LIB_PATH = os.path.join(PKG_DIR, "libops3d_fda_bench.so")
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
# -munsafe-fp-atomics: fp32 atomics lower to the hardware add (no CAS loop); all our atomics
# target coarse-grained device memory, where that is exact.
# atomic optimizer off: it turns a one-lane atomic with a uniform address (the tile kernel's work
# counter) into a wave-aggregated one that reads the result back at once, so the wave waits for
# the atomic's round trip where the kernel means to hide it; no kernel here has atomics that
# aggregation would help (their addresses vary per lane).
HIP_FLAGS = [
    "-std=c++17",
    "-O3",
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-fPIC",
    "-fvisibility=hidden",
    "-munsafe-fp-atomics",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def _hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; the ops3d_amd kernels need ROCm's hipcc")
    return cand


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def _torch_ext_cmds(build_dir: str) -> tuple[list[str], list[str], str]:
    """g++ compile and link commands of the PyTorch extension module (csrc/torch_ext.cpp: host
    code over the C ABI, linked against libops3d_fda.so next to it)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    obj = os.path.join(build_dir, "torch_ext.o")
    out = os.path.join(PKG_DIR, TORCH_EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in cpp_extension.include_paths()] + [
        f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include"]
    cc = ["g++", "-std=c++17", "-O2", "-fPIC", "-fvisibility=hidden", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          f"-DTORCH_EXTENSION_NAME={TORCH_EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H", "-DUSE_ROCM",
          "-D__HIP_PLATFORM_AMD__=1", *inc, "-c", os.path.join(CSRC, "torch_ext.cpp"), "-o", obj]
    libdirs = cpp_extension.library_paths()
    link = ["g++", "-shared", obj, "-o", out + ".tmp", *[f"-L{d}" for d in libdirs], f"-L{PKG_DIR}",
            "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lops3d_fda",
            "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs]]
    return cc, link, out


def build(out_path: str = LIB_PATH, build_dir: str | None = None) -> str:
    """Compile every source for gfx950 and link ``libops3d_fda.so``, then the PyTorch
    extension module over it and the measurement library ``libops3d_fda_bench.so``; return the
    library's path."""
    hipcc = _hipcc()
    build_dir = build_dir or os.path.join(PKG_DIR, "_build")
    os.makedirs(build_dir, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    ext_cc, ext_link, ext_out = _torch_ext_cmds(build_dir)
    cmds.append(ext_cc)
    main = out_path == LIB_PATH
    if main:
        cmds.append([hipcc, *HIP_FLAGS, "-shared", os.path.join(CSRC, BENCH_SOURCE), "-o", BENCH_LIB_PATH + ".tmp"])
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
        list(ex.map(_run, cmds))
    tmp = out_path + ".tmp"
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp])
    os.replace(tmp, out_path)
    if main:
        _run(ext_link)
        os.replace(ext_out + ".tmp", ext_out)
        os.replace(BENCH_LIB_PATH + ".tmp", BENCH_LIB_PATH)
    return out_path


if __name__ == "__main__":
    print(build())
