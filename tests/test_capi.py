"""The C ABI library loads, exports every function include/*.h declares, and rejects
bad arguments before touching the GPU (no compute calls here)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))]


def _declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"OPS3D_FDA_API\s+[\w\s\*]*?\b(ops3d_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from ops3d_amd import _extension

    if not os.path.exists(_extension.LIB_PATH):
        pytest.skip("libops3d_fda.so not built")
    return _extension.load_library()


def test_header_declares_all_bound_symbols():
    from ops3d_amd._extension import EXPORTED_SYMBOLS

    assert _declared() == sorted(EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_bench_library_exports_every_declared_symbol():
    """libops3d_fda_bench.so (measurement baselines, include/ops3d_fda_bench.h)."""
    from ops3d_amd import _bench_lib

    if not os.path.exists(_bench_lib.LIB_PATH):
        pytest.skip("libops3d_fda_bench.so not built")
    text = open(os.path.join(ROOT, "include", "ops3d_fda_bench.h")).read()
    names = sorted(set(re.findall(r"OPS3D_FDA_BENCH_API\s+[\w\s\*]*?\b(ops3d_\w+)\s*\(", text)))
    assert len(names) == 4
    blib = _bench_lib.load()
    for name in names:
        assert hasattr(blib, name), name


def test_abi_version_and_support_table(lib):
    assert lib.ops3d_fda_abi_version() == 7
    F32, F16, BF16 = 0, 1, 2
    for d in (8, 16, 24, 32, 48, 64, 96, 128, 192, 256):
        assert lib.ops3d_fda_supported(BF16, d) == 1, d
        assert lib.ops3d_fda_supported(F16, d) == 1, d
    for d in (8, 16, 24, 32, 48, 64, 96, 128, 192):
        assert lib.ops3d_fda_supported(F32, d) == 1, d
    for d in (0, 5, 20, 40, 7):
        assert lib.ops3d_fda_supported(BF16, d) == 0, d
    assert lib.ops3d_fda_supported(9, 32) == 0


def test_forward_workspace_bytes(lib):
    c4 = (1, 73728, 8, 32, 2, 73728, 4)   # B, S, G, D, L, Q, K

    def fw(dtype, B, S, G, D, L, Q, K):
        return lib.ops3d_fda_forward_workspace_bytes(dtype, B, S, G, D, L, Q, K)

    # 64-byte rows: head slices of 2*S + 10 rows (room for levels stored as x-pair lines)
    assert fw(2, *c4) == 8 * (2 * 73728 + 10) * 32 * 2
    # other row sizes: S rows
    assert fw(2, 1, 73728, 8, 64, 2, 73728, 4) == 73728 * 8 * 64 * 2
    assert fw(0, *c4) == 73728 * 8 * 32 * 4
    assert fw(2, 1, 73728, 1, 32, 2, 73728, 4) == 0   # G == 1: already head-major
    assert fw(7, *c4) == 0
    # no copy, so no workspace: value under 8 MiB per batch item (c1, c2) ...
    assert fw(0, 1, 576, 8, 32, 2, 576, 4) == 0       # c1 (fp32)
    assert fw(2, 1, 4608, 8, 32, 2, 4608, 4) == 0     # c2
    # ... or fewer corner reads than a head has rows (cross-attention with few queries)
    assert fw(2, 1, 73728, 8, 32, 2, 1000, 4) == 0
    assert fw(2, 1, 73728, 8, 32, 2, 1152, 4) > 0     # Q*L*K*8 == S
    assert fw(2, 1, 73728, 8, 32, 2, 0, 4) == 0


def test_workspace_bytes(lib):
    B, S, G, D, L, Q, K = 1, 73728, 8, 32, 2, 73728, 4   # c4
    n = B * Q * G * L * K

    def al(x):
        return (x + 255) // 256 * 256

    # keys, words, stash, <= 8 entries per sample, 3 tile arrays of B*G*S+1 words, the work
    # counters, the split scratch, the bucketing matrix (64 blocks x S/16+64 tiles per head),
    # head-major copies of value and grad_output; no split scratch at c4 (at least
    # B*G*S/128 = 4608 tiles)
    def want(B, S, G, D, L, Q, K, split_slots, value_copy=True):
        n = B * Q * G * L * K
        return (al(4 * n) + al(16 * n) + al(32 * n) + 3 * al(4 * (B * G * S + 1)) + 256
                + al(split_slots * 128 * D * 4)
                + al(4 * B * G * 64 * (S // 16 + 64)) + (al(B * G * (2 * S + 10) * D * 2) if value_copy else 0) + (al(B * Q * G * D * 2) if B * Q * G * D * 2 > 64 << 20 else 0))
    assert lib.ops3d_fda_backward_workspace_bytes(2, B, S, G, D, L, Q, K) == want(B, S, G, D, L, Q, K, 0)
    assert lib.ops3d_fda_backward_workspace_bytes(9, B, S, G, D, L, Q, K) == 0
    # c5: grad_output (306 MB) gets its head-major copy
    c5 = (1, 598016, 8, 32, 3, 598016, 4)
    assert lib.ops3d_fda_backward_workspace_bytes(2, *c5) == want(*c5, 0)
    # c2: at least 8 * 4608/128 = 288 tiles (< 2048): 2048 scratch tiles for split tiles; value
    # (2.4 MB) under 8 MiB: no head-major copy
    c2 = (1, 4608, 8, 32, 2, 4608, 4)
    assert lib.ops3d_fda_backward_workspace_bytes(2, *c2) == want(*c2, 2048, value_copy=False)


def _fwd(lib, ptr=None, ws=None, ws_bytes=0, **kw):
    a = dict(dtype=2, B=1, S=576, G=8, D=32, L=2, Q=576, K=4, step=64)
    a.update(kw)
    return lib.ops3d_fda_forward(ptr, ptr, ptr, ptr, ptr, ws, ws_bytes, a["dtype"], a["B"], a["S"], a["G"],
                                 a["D"], a["L"], a["Q"], a["K"], a["step"], None)


def test_argument_errors_before_device_work(lib):
    assert _fwd(lib, L=6) == 1 and b"invalid number of scales" in lib.ops3d_fda_last_error()
    assert _fwd(lib, L=0) == 1
    assert _fwd(lib, K=0) == 1 and _fwd(lib, K=17) == 1
    assert _fwd(lib, D=20) == 1 and b"unsupported channels" in lib.ops3d_fda_last_error()
    assert _fwd(lib, dtype=7) == 1
    assert _fwd(lib, B=5, step=2) == 2 and b"must divide" in lib.ops3d_fda_last_error()
    assert _fwd(lib, step=0) == 1
    assert _fwd(lib, S=1 << 26) == 1 and b"too large" in lib.ops3d_fda_last_error()
    # valid sizes but NULL pointers are rejected, not dereferenced
    assert _fwd(lib) == 1 and b"NULL" in lib.ops3d_fda_last_error()
    # nothing to do: B*Q == 0 succeeds without touching any pointer
    assert _fwd(lib, Q=0) == 0


def test_forward_workspace_too_small(lib):
    p = ctypes.c_void_p(256)
    c4 = dict(S=73728, Q=73728)
    need = lib.ops3d_fda_forward_workspace_bytes(2, 1, 73728, 8, 32, 2, 73728, 4)
    # a non-NULL workspace smaller than the forward needs is refused before any device work
    assert _fwd(lib, p, p, need - 256, **c4) == 1 and b"workspace too small" in lib.ops3d_fda_last_error()


def test_backward_workspace_check(lib):
    p = ctypes.c_void_p(256)
    rc = lib.ops3d_fda_backward(p, p, p, p, p, p, p, None, 0, 2, 1, 576, 8, 32, 2, 576, 4, 64, None)
    assert rc == 1 and b"workspace too small" in lib.ops3d_fda_last_error()
    # argument errors are still reported before anything else
    rc = lib.ops3d_fda_backward(p, p, p, p, p, p, p, None, 0, 2, 1, 576, 8, 32, 6, 576, 4, 64, None)
    assert rc == 1 and b"invalid number of scales" in lib.ops3d_fda_last_error()


def test_noalloc_refuses_large_problems_before_device_work(lib):
    p = ctypes.c_void_p(256)
    # c4 needs 340 MiB of workspace; the static scratch holds 64 MiB
    rc = lib.ops3d_fda_backward_noalloc(p, p, p, p, p, p, p, 2, 1, 73728, 8, 32, 2, 73728, 4, 64, None)
    assert rc == 1 and b"too large for the allocation-free backward" in lib.ops3d_fda_last_error()
    # argument errors first
    rc = lib.ops3d_fda_backward_noalloc(p, p, p, p, p, p, p, 2, 1, 576, 8, 32, 6, 576, 4, 64, None)
    assert rc == 1 and b"invalid number of scales" in lib.ops3d_fda_last_error()


def test_offsets_argument_errors_before_device_work(lib):
    p = ctypes.c_void_p(256)
    args = (2, 1, 576, 8, 32, 2, 576, 4, 64, None)   # dtype, B, S, G, D, L, Q, K, step, stream
    rc = lib.ops3d_fda_forward_offsets(p, p, p, p, None, 1, p, None, 0, *args)
    assert rc == 1 and b"reference_points is NULL" in lib.ops3d_fda_last_error()
    rc = lib.ops3d_fda_forward_offsets(p, p, p, p, p, 3, p, None, 0, *args)
    assert rc == 1 and b"ref_levels must be 1 or num_levels" in lib.ops3d_fda_last_error()
    rc = lib.ops3d_fda_backward_offsets(p, None, p, p, p, p, 3, p, p, p, None, None, 0, *args)
    assert rc == 1 and b"ref_levels must be 1 or num_levels" in lib.ops3d_fda_last_error()
    # nothing to do (Q = 0): no check of the reference points, success
    rc = lib.ops3d_fda_forward_offsets(p, p, p, p, None, 1, p, None, 0, 2, 1, 576, 8, 32, 2, 0, 4, 64, None)
    assert rc == 0


def test_bench_library_argument_errors_before_device_work():
    """The measurement library (libops3d_fda_bench.so, not part of the op) validates before any
    device work, and the op's library no longer exports the baseline."""
    from ops3d_amd import _bench_lib, _extension

    blib = _bench_lib.load()
    f = blib.ops3d_fda_bench_ref_scatter
    args = dict(dtype=2, B=1, S=576, G=8, D=32, L=2, Q=576, K=4)

    def call(**kw):
        a = {**args, **kw}
        return f(None, None, None, None, None, a["dtype"], a["B"], a["S"], a["G"], a["D"], a["L"], a["Q"],
                 a["K"], None)

    assert call(D=20) == 1 and b"unsupported channels" in blib.ops3d_fda_bench_last_error()
    assert call(L=6) == 1
    assert call(dtype=7) == 1
    assert call() == 1 and b"NULL" in blib.ops3d_fda_bench_last_error()
    assert blib.ops3d_fda_bench_lds_atomic(None, 1, 1, 0, None) == 1
    g = blib.ops3d_fda_bench_gather
    assert g(None, 1 << 20, 8, 1, 1, None, 1, None) == 1                      # NULL buffers
    # (the calls below pass stand-in pointers: each is refused before any launch)
    assert g(16, 1 << 20, 5, 1, 1, 16, 1, None) == 1 and b"group" in blib.ops3d_fda_bench_last_error()
    assert g(16, 8, 8, 1, 1, 16, 1, None) == 1 and b"size" in blib.ops3d_fda_bench_last_error()
    assert g(16, 1 << 20, 8, 0, 1, 16, 1, None) == 1
    assert not hasattr(_extension.load_library(), "ops3d_fda_scatter_baseline")
