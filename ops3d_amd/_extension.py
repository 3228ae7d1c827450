"""Load libops3d_fda.so and expose it as ``_C``, the extension-module object of the package.

Mirrors the reference's loader contract (ops3d/_extension.py:13-55): importing the package
never fails; when the native library cannot be loaded, ``_C`` is ``None`` and
``FlashDeformAttnFunction`` raises ``RuntimeError`` (reference ops3d/flash_deform_attn.py:78-79).
There is no fallback implementation.

``_C.flash_deform_attn_forward`` / ``_C.flash_deform_attn_backward`` keep the argument lists
of the reference's pybind entry points (csrc/vision.cpp:23-24, csrc/flash_deform_attn.h:7-52).
They check what only the tensors know (device, dtype, contiguity, ranks), allocate outputs and
the fp32 workspace with torch, and call the C ABI (include/ops3d_fda.h) on torch's current
HIP stream.  Everything else (L/K/D limits, im2col_step divisibility, launch geometry) is
checked by the C library.
"""
from __future__ import annotations

import ctypes
import os

import torch  # imported first: its HIP runtime is the one libops3d_fda.so binds to

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libops3d_fda.so")

OPS3D_FDA_OK, OPS3D_FDA_EINVAL, OPS3D_FDA_ERUNTIME = 0, 1, 2
# RoI Align forward: below this many output elements the NCDHW kernel is as fast as the
# transposed copy of the features plus the channels-last kernel
ROI_CL_MIN_OUTPUTS = 1 << 19
_DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_vp, _i, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t

EXPORTED_SYMBOLS = (
    "ops3d_fda_abi_version",
    "ops3d_fda_last_error",
    "ops3d_fda_supported",
    "ops3d_fda_forward_workspace_bytes",
    "ops3d_fda_forward",
    "ops3d_fda_backward_workspace_bytes",
    "ops3d_fda_backward",
    "ops3d_fda_backward_ex",
    "ops3d_fda_backward_accumulate_f32",
    "ops3d_fda_backward_noalloc",
    "ops3d_fda_forward_offsets",
    "ops3d_fda_backward_offsets",
    "ops3d_dcnv4_workspace_bytes",
    "ops3d_dcnv4_forward",
    "ops3d_dcnv4_backward",
    "ops3d_nms3d_workspace_bytes",
    "ops3d_nms3d",
    "ops3d_roi_align3d_forward",
    "ops3d_roi_align3d_backward_workspace_bytes",
    "ops3d_roi_align3d_backward",
    "ops3d_roi_align3d_channels_last_supported",
    "ops3d_roi_align3d_forward_channels_last",
    "ops3d_roi_align3d_to_channels_last",
    "ops3d_fda_profile_enable",
    "ops3d_fda_profile_read",
)


def _declare(lib: ctypes.CDLL) -> None:
    lib.ops3d_fda_abi_version.restype = _i
    lib.ops3d_fda_abi_version.argtypes = []
    lib.ops3d_fda_last_error.restype = ctypes.c_char_p
    lib.ops3d_fda_last_error.argtypes = []
    lib.ops3d_fda_supported.restype = _i
    lib.ops3d_fda_supported.argtypes = [_i, _i]
    lib.ops3d_fda_forward_workspace_bytes.restype = _sz
    lib.ops3d_fda_forward_workspace_bytes.argtypes = [_i] * 8
    lib.ops3d_fda_forward.restype = _i
    lib.ops3d_fda_forward.argtypes = [_vp] * 6 + [_sz] + [_i] * 9 + [_vp]
    lib.ops3d_fda_backward_workspace_bytes.restype = _sz
    lib.ops3d_fda_backward_workspace_bytes.argtypes = [_i] * 8
    lib.ops3d_fda_backward.restype = _i
    lib.ops3d_fda_backward.argtypes = [_vp] * 8 + [_sz] + [_i] * 9 + [_vp]
    lib.ops3d_fda_backward_ex.restype = _i
    lib.ops3d_fda_backward_ex.argtypes = [_vp] * 9 + [_sz] + [_i] * 9 + [_vp]
    lib.ops3d_fda_profile_enable.restype = _i
    lib.ops3d_fda_profile_enable.argtypes = [_i]
    lib.ops3d_fda_profile_read.restype = _i
    lib.ops3d_fda_profile_read.argtypes = [_i, ctypes.POINTER(ctypes.c_float), _i]
    lib.ops3d_fda_backward_accumulate_f32.restype = _i
    lib.ops3d_fda_backward_accumulate_f32.argtypes = [_vp] * 8 + [_sz] + [_i] * 9 + [_vp]
    lib.ops3d_fda_backward_noalloc.restype = _i
    lib.ops3d_fda_backward_noalloc.argtypes = [_vp] * 7 + [_i] * 9 + [_vp]
    lib.ops3d_fda_forward_offsets.restype = _i
    lib.ops3d_fda_forward_offsets.argtypes = [_vp] * 5 + [_i] + [_vp] * 2 + [_sz] + [_i] * 9 + [_vp]
    lib.ops3d_fda_backward_offsets.restype = _i
    lib.ops3d_dcnv4_workspace_bytes.restype = _sz
    lib.ops3d_dcnv4_workspace_bytes.argtypes = [_i] * 21
    lib.ops3d_dcnv4_forward.restype = _i
    lib.ops3d_dcnv4_forward.argtypes = [_vp] * 4 + [_sz] + [_i] * 19 + [ctypes.c_float] + [_i] * 4 + [_vp]
    lib.ops3d_dcnv4_backward.restype = _i
    lib.ops3d_dcnv4_backward.argtypes = [_vp] * 6 + [_sz] + [_i] * 19 + [ctypes.c_float] + [_i] * 4 + [_vp]
    lib.ops3d_nms3d_workspace_bytes.restype = _sz
    lib.ops3d_nms3d_workspace_bytes.argtypes = [_i]
    lib.ops3d_nms3d.restype = _i
    lib.ops3d_nms3d.argtypes = [_vp, _vp, _i, ctypes.c_float, _vp, _sz, _vp, _vp, _vp]
    lib.ops3d_roi_align3d_forward.restype = _i
    lib.ops3d_roi_align3d_forward.argtypes = [_vp] * 3 + [_i] * 10 + [ctypes.c_float, _i, _i, _vp]
    lib.ops3d_roi_align3d_backward_workspace_bytes.restype = _sz
    lib.ops3d_roi_align3d_backward_workspace_bytes.argtypes = [_i] * 10
    lib.ops3d_roi_align3d_backward.restype = _i
    lib.ops3d_roi_align3d_backward.argtypes = [_vp] * 4 + [_sz] + [_i] * 10 + [ctypes.c_float, _i, _i, _vp]
    lib.ops3d_roi_align3d_channels_last_supported.restype = _i
    lib.ops3d_roi_align3d_channels_last_supported.argtypes = [_i] * 6
    lib.ops3d_roi_align3d_forward_channels_last.restype = _i
    lib.ops3d_roi_align3d_forward_channels_last.argtypes = [_vp] * 3 + [_i] * 10 + [ctypes.c_float, _i, _i, _vp]
    lib.ops3d_roi_align3d_to_channels_last.restype = _i
    lib.ops3d_roi_align3d_to_channels_last.argtypes = [_vp] * 2 + [_i] * 6 + [_vp]
    lib.ops3d_fda_backward_offsets.argtypes = [_vp] * 6 + [_i] + [_vp] * 5 + [_sz] + [_i] * 9 + [_vp]


def _ptr(t: torch.Tensor | None) -> int | None:
    return t.data_ptr() if (t is not None and t.numel() > 0) else None


class _NativeFDA:
    """Host side of the flash-deform-attn extension, bound to libops3d_fda.so."""

    ABI_VERSION = 7

    def __init__(self, lib: ctypes.CDLL, path: str, ext=None):
        self._lib = lib
        self.__file__ = path
        ver = lib.ops3d_fda_abi_version()
        if ver != self.ABI_VERSION:
            raise ImportError(f"{path}: ABI version {ver}, expected {self.ABI_VERSION}")
        # The PyTorch extension module (csrc/torch_ext.cpp) does the same checks and calls of
        # the tensor entry points in C++, for a fraction of the host time: when it is built,
        # those methods are its functions.
        self._ext = ext
        if ext is not None:
            for name in ("flash_deform_attn_forward", "flash_deform_attn_backward",
                         "forward_keep_head_major", "backward_with_head_major",
                         "forward_offsets", "backward_offsets", "nms_3d", "roi_align_3d_forward",
                         "roi_align_3d_backward", "dcnv4_forward", "dcnv4_backward"):
                setattr(self, name, getattr(ext, name))

    # -- helpers ---------------------------------------------------------------------------
    def _raise(self, rc: int, what: str) -> None:
        msg = self._lib.ops3d_fda_last_error().decode(errors="replace") or what
        if rc == OPS3D_FDA_EINVAL:
            raise ValueError(msg)
        raise RuntimeError(msg)

    @staticmethod
    def _check_inputs(tensors: dict, value: torch.Tensor) -> None:
        for name, t in tensors.items():
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"{name} must be a torch.Tensor")
            if not t.is_cuda:
                # reference csrc/flash_deform_attn.h:24,51
                raise RuntimeError(f"Not implemented on the CPU ({name} is on {t.device})")
            if not t.is_contiguous():
                raise RuntimeError(f"{name} tensor has to be contiguous")
            if t.device != value.device:
                raise RuntimeError(f"{name} is on {t.device}, value on {value.device}")

    def _common(self, value, spatial_shapes, level_start_index, sampling_loc_attn, K, extra):
        tensors = {
            "value": value,
            "spatial_shapes": spatial_shapes,
            "level_start_index": level_start_index,
            "sampling_loc_attn": sampling_loc_attn,
            **extra,
        }
        self._check_inputs(tensors, value)
        if value.dtype not in _DTYPE_CODE:
            raise ValueError(f"unsupported value dtype {value.dtype}")
        for name in ("sampling_loc_attn", *extra):
            if tensors[name].dtype != value.dtype:
                raise ValueError(f"{name} dtype {tensors[name].dtype} differs from value dtype {value.dtype}")
        if spatial_shapes.dtype != torch.int64 or level_start_index.dtype != torch.int64:
            raise ValueError("spatial_shapes and level_start_index must be int64")
        if value.dim() != 4:
            raise ValueError(f"value must be [B, S, G, D], got shape {tuple(value.shape)}")
        B, S, G, D = value.shape
        L = spatial_shapes.shape[0]
        if spatial_shapes.dim() != 2 or spatial_shapes.shape[1] != 3:
            raise ValueError(f"spatial_shapes must be [L, 3], got {tuple(spatial_shapes.shape)}")
        if level_start_index.shape != (L,):
            raise ValueError(f"level_start_index must be [{L}], got {tuple(level_start_index.shape)}")
        if sampling_loc_attn.dim() != 4 or sampling_loc_attn.shape[0] != B or sampling_loc_attn.shape[2] != G:
            raise ValueError(
                f"sampling_loc_attn must be [B={B}, Q, G={G}, P], got {tuple(sampling_loc_attn.shape)}"
            )
        P = L * K * 4
        if sampling_loc_attn.shape[3] != P:
            raise ValueError(
                f"sampling_loc_attn last dimension ({sampling_loc_attn.shape[3]}) does not match "
                f"L={L}, K={K} (expected {P})"
            )
        Q = sampling_loc_attn.shape[1]
        return B, S, G, D, L, Q

    # -- entry points (reference csrc/flash_deform_attn.h) -----------------------------------
    def flash_deform_attn_forward(
        self, value, spatial_shapes, level_start_index, sampling_loc_attn, im2col_step, K,
        d_stride=8, block_thread=0, use_reg=True,
    ):
        """Forward; ``d_stride``, ``block_thread`` and ``use_reg`` are accepted and ignored
        (the gfx950 launch geometry is chosen by the library).  Returns [B, Q, G*D]."""
        return self.forward_keep_head_major(value, spatial_shapes, level_start_index, sampling_loc_attn,
                                            im2col_step, K)[0]

    def forward_keep_head_major(self, value, spatial_shapes, level_start_index, sampling_loc_attn, im2col_step, K):
        """Forward that also returns its workspace, which holds the head-major copy of value
        (None when the forward makes no copy), for backward_with_head_major."""
        B, S, G, D, L, Q = self._common(value, spatial_shapes, level_start_index, sampling_loc_attn, K, {})
        out = torch.empty((B, Q, G * D), dtype=value.dtype, device=value.device)
        code = _DTYPE_CODE[value.dtype]
        n = self._lib.ops3d_fda_forward_workspace_bytes(code, B, S, G, D, L, Q, int(K))
        ws = torch.empty(n, dtype=torch.uint8, device=value.device) if n else None
        stream = torch.cuda.current_stream(value.device).cuda_stream
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_fda_forward(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index), _ptr(sampling_loc_attn),
                _ptr(out), _ptr(ws), n, code, B, S, G, D, L, Q, int(K), int(im2col_step), stream,
            )
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "flash_deform_attn_forward failed")
        return out, ws

    def flash_deform_attn_backward(
        self, value, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
        im2col_step, K, d_stride=1, block_thread=0,
    ):
        """Backward; returns [grad_value, grad_sampling_loc_attn] in value's dtype."""
        return self.backward_with_head_major(value, None, spatial_shapes, level_start_index, sampling_loc_attn,
                                             grad_output, im2col_step, K)

    def backward_with_head_major(
        self, value, value_head_major, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
        im2col_step, K,
    ):
        """Backward reusing ``value_head_major``, the workspace forward_keep_head_major returned
        for this value (or None)."""
        B, S, G, D, L, Q = self._common(
            value, spatial_shapes, level_start_index, sampling_loc_attn, K, {"grad_output": grad_output}
        )
        if grad_output.numel() != B * Q * G * D:
            raise ValueError(f"grad_output must have B*Q*G*D = {B * Q * G * D} elements, got {grad_output.numel()}")
        code = _DTYPE_CODE[value.dtype]
        if value_head_major is not None:
            need = self._lib.ops3d_fda_forward_workspace_bytes(code, B, S, G, D, L, Q, int(K))
            if (value_head_major.device != value.device or value_head_major.dtype != torch.uint8
                    or value_head_major.numel() != need):
                raise ValueError("value_head_major is not a forward workspace of this value")
        grad_value = torch.empty_like(value)
        grad_sla = torch.empty_like(sampling_loc_attn)
        ws, ws_bytes = self._workspace(code, B, S, G, D, L, Q, K, value.device)
        stream = torch.cuda.current_stream(value.device).cuda_stream
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_fda_backward_ex(
                _ptr(value), _ptr(value_head_major), _ptr(spatial_shapes), _ptr(level_start_index),
                _ptr(sampling_loc_attn), _ptr(grad_output), _ptr(grad_value), _ptr(grad_sla), _ptr(ws), ws_bytes,
                code, B, S, G, D, L, Q, int(K), int(im2col_step), stream,
            )
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "flash_deform_attn_backward failed")
        return [grad_value, grad_sla]

    def _workspace(self, code, B, S, G, D, L, Q, K, device):
        n = self._lib.ops3d_fda_backward_workspace_bytes(code, B, S, G, D, L, Q, int(K))
        if n == 0:
            return None, 0
        return torch.empty(n, dtype=torch.uint8, device=device), n

    def flash_deform_attn_backward_accumulate(
        self, value, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
        grad_value_f32, im2col_step, K,
    ):
        """Backward that adds the value gradient into the fp32 tensor ``grad_value_f32``
        ([B,S,G,D], not cleared) and returns a new grad_sampling_loc_attn (value dtype)."""
        B, S, G, D, L, Q = self._common(
            value, spatial_shapes, level_start_index, sampling_loc_attn, K, {"grad_output": grad_output}
        )
        if grad_value_f32.dtype != torch.float32 or grad_value_f32.shape != value.shape:
            raise ValueError("grad_value_f32 must be an fp32 tensor shaped like value")
        self._check_inputs({"grad_value_f32": grad_value_f32}, value)
        grad_sla = torch.empty_like(sampling_loc_attn)
        code = _DTYPE_CODE[value.dtype]
        ws, ws_bytes = self._workspace(code, B, S, G, D, L, Q, K, value.device)
        stream = torch.cuda.current_stream(value.device).cuda_stream
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_fda_backward_accumulate_f32(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index), _ptr(sampling_loc_attn),
                _ptr(grad_output), _ptr(grad_value_f32), _ptr(grad_sla), _ptr(ws), ws_bytes,
                code, B, S, G, D, L, Q, int(K), int(im2col_step), stream,
            )
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "flash_deform_attn_backward_accumulate failed")
        return grad_sla

    def _ref_levels(self, reference_points, value, B, Q, L):
        self._check_inputs({"reference_points": reference_points}, value)
        if reference_points.dtype != torch.float32:
            raise ValueError(f"reference_points must be float32, got {reference_points.dtype}")
        if reference_points.dim() != 4 or tuple(reference_points.shape[:2]) != (B, Q) \
                or reference_points.shape[3] != 3 or reference_points.shape[2] not in (1, L):
            raise ValueError(f"reference_points must be [B={B}, Q={Q}, 1 or L={L}, 3], "
                             f"got {tuple(reference_points.shape)}")
        return int(reference_points.shape[2])

    def forward_offsets(self, value, spatial_shapes, level_start_index, offset_attn, reference_points,
                        im2col_step, K):
        """Offset-mode forward (ops3d_fda_forward_offsets): offset_attn holds offsets in voxels of
        their level instead of locations.  Returns the output and the forward workspace."""
        B, S, G, D, L, Q = self._common(value, spatial_shapes, level_start_index, offset_attn, K, {})
        R = self._ref_levels(reference_points, value, B, Q, L)
        out = torch.empty((B, Q, G * D), dtype=value.dtype, device=value.device)
        code = _DTYPE_CODE[value.dtype]
        n = self._lib.ops3d_fda_forward_workspace_bytes(code, B, S, G, D, L, Q, int(K))
        ws = torch.empty(n, dtype=torch.uint8, device=value.device) if n else None
        stream = torch.cuda.current_stream(value.device).cuda_stream
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_fda_forward_offsets(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index), _ptr(offset_attn),
                _ptr(reference_points), R, _ptr(out), _ptr(ws), n, code, B, S, G, D, L, Q, int(K),
                int(im2col_step), stream,
            )
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "flash_deform_attn_forward_offsets failed")
        return out, ws

    def backward_offsets(self, value, value_head_major, spatial_shapes, level_start_index, offset_attn,
                         reference_points, grad_output, im2col_step, K, want_ref_grad):
        """Offset-mode backward (ops3d_fda_backward_offsets): returns [grad_value,
        grad_offset_attn (offset and logit gradients, in offset_attn's layout),
        grad_reference_points (fp32, None unless want_ref_grad)]."""
        B, S, G, D, L, Q = self._common(
            value, spatial_shapes, level_start_index, offset_attn, K, {"grad_output": grad_output}
        )
        R = self._ref_levels(reference_points, value, B, Q, L)
        if grad_output.numel() != B * Q * G * D:
            raise ValueError(f"grad_output must have B*Q*G*D = {B * Q * G * D} elements, got {grad_output.numel()}")
        code = _DTYPE_CODE[value.dtype]
        if value_head_major is not None:
            need = self._lib.ops3d_fda_forward_workspace_bytes(code, B, S, G, D, L, Q, int(K))
            if (value_head_major.device != value.device or value_head_major.dtype != torch.uint8
                    or value_head_major.numel() != need):
                raise ValueError("value_head_major is not a forward workspace of this value")
        grad_value = torch.empty_like(value)
        grad_oa = torch.empty_like(offset_attn)
        grad_ref = torch.zeros_like(reference_points) if want_ref_grad else None
        ws, ws_bytes = self._workspace(code, B, S, G, D, L, Q, K, value.device)
        stream = torch.cuda.current_stream(value.device).cuda_stream
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_fda_backward_offsets(
                _ptr(value), _ptr(value_head_major), _ptr(spatial_shapes), _ptr(level_start_index),
                _ptr(offset_attn), _ptr(reference_points), R, _ptr(grad_output), _ptr(grad_value), _ptr(grad_oa),
                _ptr(grad_ref), _ptr(ws), ws_bytes, code, B, S, G, D, L, Q, int(K), int(im2col_step), stream,
            )
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "flash_deform_attn_backward_offsets failed")
        return [grad_value, grad_oa, grad_ref]

    def flash_deform_attn_backward_noalloc(
        self, value, spatial_shapes, level_start_index, sampling_loc_attn, grad_output, im2col_step, K,
    ):
        """Backward through the allocation-free entry point (the library's static device scratch,
        at most 64 MiB of workspace; calls overlapping on one device race).  The output tensors
        are allocated here by torch; a caller that cannot allocate calls
        ops3d_fda_backward_noalloc with its own output buffers."""
        B, S, G, D, L, Q = self._common(
            value, spatial_shapes, level_start_index, sampling_loc_attn, K, {"grad_output": grad_output}
        )
        if grad_output.numel() != B * Q * G * D:
            raise ValueError(f"grad_output must have B*Q*G*D = {B * Q * G * D} elements, got {grad_output.numel()}")
        code = _DTYPE_CODE[value.dtype]
        grad_value = torch.empty_like(value)
        grad_sla = torch.empty_like(sampling_loc_attn)
        stream = torch.cuda.current_stream(value.device).cuda_stream
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_fda_backward_noalloc(
                _ptr(value), _ptr(spatial_shapes), _ptr(level_start_index), _ptr(sampling_loc_attn),
                _ptr(grad_output), _ptr(grad_value), _ptr(grad_sla),
                code, B, S, G, D, L, Q, int(K), int(im2col_step), stream,
            )
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "flash_deform_attn_backward_noalloc failed")
        return [grad_value, grad_sla]

    def nms_3d(self, dets, scores, threshold):
        """3-D NMS (reference csrc/nms_3d.h:27-44): dets [N,6] (x1,y1,z1,x2,y2,z2), scores [N]
        -> int64 indices of the kept boxes, in decreasing score order (ties in index order)."""
        if not dets.is_cuda:
            raise RuntimeError("Not compiled with CPU support")
        if dets.numel() == 0:
            return torch.empty(0, dtype=torch.long, device=dets.device)
        if dets.dim() != 2 or dets.shape[1] != 6:
            raise ValueError("dets must be [N, 6] (x1,y1,z1,x2,y2,z2)")
        if scores.dim() != 1 or scores.shape[0] != dets.shape[0] or scores.device != dets.device:
            raise ValueError("scores must be [N] on the boxes' device")
        order = torch.sort(scores, stable=True, descending=True)[1]
        boxes = dets.index_select(0, order).to(torch.float32).contiguous()
        n = boxes.shape[0]
        wsb = self._lib.ops3d_nms3d_workspace_bytes(n)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dets.device)
        keep = torch.empty(n, dtype=torch.long, device=dets.device)
        num = torch.empty(1, dtype=torch.int32, device=dets.device)
        stream = torch.cuda.current_stream(dets.device).cuda_stream
        with torch.cuda.device(dets.device):
            rc = self._lib.ops3d_nms3d(_ptr(boxes), _ptr(order), n, float(threshold), _ptr(ws), wsb, _ptr(keep),
                                       _ptr(num), stream)
        if rc == OPS3D_FDA_EINVAL:
            raise ValueError("nms_3d: too many boxes (at most 2^19)")
        if rc != OPS3D_FDA_OK:
            raise RuntimeError("nms_3d: kernel launch failed")
        return keep[: int(num.item())]

    @staticmethod
    def _roi_checks(data, rois, other):
        if not data.is_cuda:
            raise RuntimeError("RoIAlign is not implemented on CPU")
        if rois.dim() != 2 or rois.shape[1] != 7:
            raise RuntimeError("wrong roi size! size_rois should be 7")
        for t in (rois, other):
            if t.device != data.device:
                raise RuntimeError("RoIAlign tensors must be on one device")
            if t.dtype != data.dtype:
                raise ValueError("RoIAlign tensors must share a dtype")
        if not other.is_contiguous():
            raise RuntimeError("RoIAlign output tensor has to be contiguous")
        if data.dtype not in _DTYPE_CODE:
            raise ValueError(f"unsupported dtype {data.dtype}")
        return _DTYPE_CODE[data.dtype]

    def roi_align_3d_forward(self, features, rois, output, out_d, out_h, out_w, spatial_scale, sampling_ratio, order):
        """RoI Align 3-D forward into `output` [R, C, out_d, out_h, out_w] (reference
        csrc/roi_align_3d.h:97-115)."""
        code = self._roi_checks(features, rois, output)
        r = rois.contiguous()
        N, C, D, H, W = features.shape
        R = r.shape[0]
        if tuple(output.shape) != (R, C, out_d, out_h, out_w):
            raise ValueError("output must be [R, C, out_d, out_h, out_w]")
        cl_in = (not features.is_contiguous() and features.is_contiguous(memory_format=torch.channels_last_3d)
                 and features.data_ptr() % 16 == 0)
        use_cl = (N <= 65535 and self._lib.ops3d_roi_align3d_channels_last_supported(code, C, D, H, W, out_w)
                  and (cl_in or R * C * out_d * out_h * out_w >= ROI_CL_MIN_OUTPUTS))
        with torch.cuda.device(features.device):
            st = torch.cuda.current_stream(features.device).cuda_stream
            args = (code, N, C, D, H, W, R, out_d, out_h, out_w, float(spatial_scale), int(sampling_ratio),
                    int(order), st)
            if use_cl:
                # the channels-last kernel, on the caller's channels_last_3d memory or a transposed copy
                fc = features
                if not cl_in:
                    f = features.contiguous()
                    fc = torch.empty((N, D, H, W, C), dtype=f.dtype, device=f.device)
                    rc = self._lib.ops3d_roi_align3d_to_channels_last(_ptr(f), _ptr(fc), code, N, C, D, H, W, st)
                    if rc != OPS3D_FDA_OK:
                        raise RuntimeError("roi_align_3d_forward: channels-last copy failed")
                rc = self._lib.ops3d_roi_align3d_forward_channels_last(_ptr(fc), _ptr(r), _ptr(output), *args)
            else:
                f = features.contiguous()
                rc = self._lib.ops3d_roi_align3d_forward(_ptr(f), _ptr(r), _ptr(output), *args)
        if rc == OPS3D_FDA_EINVAL:
            raise ValueError("roi_align_3d_forward: invalid sizes or order")
        if rc != OPS3D_FDA_OK:
            raise RuntimeError("roi_align_3d_forward: kernel launch failed")

    def roi_align_3d_backward(self, top_grad, rois, bottom_grad, out_d, out_h, out_w, spatial_scale, sampling_ratio,
                              order):
        """RoI Align 3-D backward into `bottom_grad` [N, C, D, H, W], every element written
        (reference csrc/roi_align_3d.h:117-136)."""
        code = self._roi_checks(top_grad, rois, bottom_grad)
        g, r = top_grad.contiguous(), rois.contiguous()
        N, C, D, H, W = bottom_grad.shape
        wsb = self._lib.ops3d_roi_align3d_backward_workspace_bytes(code, N, C, D, H, W, r.shape[0], out_d, out_h,
                                                                   out_w)
        ws = torch.empty((wsb + 3) // 4, dtype=torch.float32, device=g.device) if wsb else None
        with torch.cuda.device(g.device):
            rc = self._lib.ops3d_roi_align3d_backward(
                _ptr(g), _ptr(r), _ptr(bottom_grad), _ptr(ws), wsb, code, N, C, D, H, W, r.shape[0], out_d, out_h,
                out_w, float(spatial_scale), int(sampling_ratio), int(order),
                torch.cuda.current_stream(g.device).cuda_stream)
        if rc == OPS3D_FDA_EINVAL:
            raise ValueError("roi_align_3d_backward: invalid sizes or order")
        if rc != OPS3D_FDA_OK:
            raise RuntimeError("roi_align_3d_backward: kernel launch failed")

    def _dcn(self, value, p_offset, group, group_channels):
        if not value.is_cuda:
            raise RuntimeError("Not implemented on the CPU")
        if not p_offset.is_cuda:
            raise RuntimeError("offset must be a CUDA tensor")
        if not value.is_contiguous() or not p_offset.is_contiguous():
            raise RuntimeError("input tensor has to be contiguous")
        if value.dim() != 5 or p_offset.dim() != 5:
            raise ValueError("value and p_offset must be 5-D")
        if p_offset.dtype != value.dtype or value.dtype not in _DTYPE_CODE:
            raise ValueError("p_offset dtype differs from value (or unsupported dtype)")
        if value.shape[4] != group * group_channels:
            raise RuntimeError("Input channels and group times group channels dont match")
        return _DTYPE_CODE[value.dtype]

    def dcnv4_forward(self, value, p_offset, kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh, dw, group, group_channels,
                      offset_scale, im2col_step, remove_center, d_stride=8, block_thread=0, softmax=False):
        """DCNv4-3D forward (reference csrc/dcnv4.h:7-32): value [B,Din,Hin,Win,G*D], p_offset
        [B,Dout,Hout,Wout,padded] -> output [B,Dout,Hout,Wout,G*D]."""
        code = self._dcn(value, p_offset, group, group_channels)
        B, Din, Hin, Win, _ = value.shape
        geo = [int(v) for v in (kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh, dw)]
        outs = [(n + 2 * p - (d * (k - 1) + 1)) // s + 1 for n, k, s, p, d in
                zip((Din, Hin, Win), geo[0:3], geo[3:6], geo[6:9], geo[9:12])]
        out = torch.empty((B, *outs, group * group_channels), dtype=value.dtype, device=value.device)
        wsb = self._lib.ops3d_dcnv4_workspace_bytes(code, B, Din, Hin, Win, group, group_channels, *geo,
                                                   int(remove_center), 0)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=value.device)
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_dcnv4_forward(
                _ptr(value), _ptr(p_offset), _ptr(out), _ptr(ws), wsb, code, B, Din, Hin, Win, group,
                group_channels, *geo, float(offset_scale), int(remove_center), 1 if softmax else 0,
                p_offset.shape[4], int(im2col_step), torch.cuda.current_stream(value.device).cuda_stream)
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "dcnv4_forward failed")
        return out

    def dcnv4_backward(self, value, p_offset, kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh, dw, group,
                       group_channels, offset_scale, im2col_step, grad_output, remove_center, d_stride=8,
                       block_thread=0, softmax=False):
        """DCNv4-3D backward (reference csrc/dcnv4.h:34-60) -> [grad_value, grad_offset]."""
        code = self._dcn(value, p_offset, group, group_channels)
        B, Din, Hin, Win, _ = value.shape
        geo = [int(v) for v in (kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh, dw)]
        grad_value = torch.empty_like(value)
        grad_offset = torch.zeros_like(p_offset)
        wsb = self._lib.ops3d_dcnv4_workspace_bytes(code, B, Din, Hin, Win, group, group_channels, *geo,
                                                   int(remove_center), 1)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=value.device)
        go = grad_output.contiguous()
        with torch.cuda.device(value.device):
            rc = self._lib.ops3d_dcnv4_backward(
                _ptr(value), _ptr(p_offset), _ptr(go), _ptr(grad_value), _ptr(grad_offset), _ptr(ws), wsb, code, B,
                Din, Hin, Win, group, group_channels, *geo, float(offset_scale), int(remove_center),
                1 if softmax else 0, p_offset.shape[4], int(im2col_step),
                torch.cuda.current_stream(value.device).cuda_stream)
        if rc != OPS3D_FDA_OK:
            self._raise(rc, "dcnv4_backward failed")
        return [grad_value, grad_offset]

    def profile_enable(self, on: bool = True) -> None:
        """Record HIP events around the backward phases of every following call."""
        if self._lib.ops3d_fda_profile_enable(1 if on else 0) != OPS3D_FDA_OK:
            self._raise(OPS3D_FDA_ERUNTIME, "profile_enable failed")

    def profile_read(self, which: str = "backward") -> dict:
        """Phase durations (ms) of the last backward / forward call (waits for it to finish)."""
        buf = (ctypes.c_float * 8)()
        if which == "backward":
            n = self._lib.ops3d_fda_profile_read(0, buf, 8)
            names = ("head_major_copies", "query_kernel", "tile_count", "tile_scatter", "tile_kernel")
        else:
            n = self._lib.ops3d_fda_profile_read(1, buf, 8)
            names = ("head_major_copy", "forward_kernel")
        return {names[i]: buf[i] for i in range(n)}

    def supported(self, dtype: torch.dtype, channels: int) -> bool:
        return dtype in _DTYPE_CODE and bool(self._lib.ops3d_fda_supported(_DTYPE_CODE[dtype], int(channels)))


_HANDLES: list = []   # dlopen handles this module opened (closed by reload)


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """dlopen libops3d_fda.so and declare its C signatures (raises OSError if absent)."""
    lib = ctypes.CDLL(path)
    _HANDLES.append(lib._handle)
    _declare(lib)
    return lib


def _torch_ext(fresh_library: bool):
    """The PyTorch extension module, or None when it is not built (or, after a rebuild, when an
    earlier build of it is already loaded in this process: an extension module cannot be
    unloaded, and it would keep the old library)."""
    import sys

    name = __package__ + "._fda_torch"
    if fresh_library and name in sys.modules:
        return None
    try:
        import importlib

        return importlib.import_module(name)
    except ImportError:
        return None


def _load(fresh_library: bool = False):
    try:
        lib = load_library(LIB_PATH)
        return _NativeFDA(lib, LIB_PATH, _torch_ext(fresh_library))
    except (OSError, ImportError, AttributeError):
        return None


_C = _load()


def reload() -> None:
    """Re-resolve ``_C`` (after building the library in this process).  dlopen of a path this
    process has open returns the open library, so the handles opened so far (including one that
    failed the ABI check) are closed first and the rebuilt file is loaded afresh."""
    global _C
    import _ctypes

    _C = None
    while _HANDLES:
        try:
            _ctypes.dlclose(_HANDLES.pop())
        except OSError:
            pass
    _C = _load(fresh_library=True)
    import sys

    from . import flash_deform_attn as _fda

    _fda._C = _C
    for name in ("ops3d_amd", "ops3d", "ops3d.flash_deform_attn"):   # modules that re-export _C
        mod = sys.modules.get(name)
        if mod is not None:
            mod._C = _C
