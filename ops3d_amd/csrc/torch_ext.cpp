// PyTorch extension module over the C ABI of libops3d_fda.so: the tensor-level entry points of
// the reference's `_C` (csrc/vision.cpp:23-24 -> csrc/flash_deform_attn.h:7-52), plus the two
// calls FlashDeformAttnFunction makes (forward keeping the head-major copy of value, backward
// reusing it) and the offset-mode pair.  Host code only: argument checks, output allocation through torch's caching
// allocator, torch's current HIP stream, then one C ABI call.  It exists for host overhead --
// the same checks and calls through ctypes cost several times as much per call.
//
// Errors: a failed check or an OPS3D_FDA_EINVAL from the library raises ValueError
// (std::invalid_argument, as the reference's), OPS3D_FDA_ERUNTIME raises RuntimeError.
#include <torch/extension.h>

// torch's current HIP stream of a device (c10's native HIP API); the device is made current
// with HIP's own calls (DeviceGuard below)
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>
#include <tuple>

#include "../../include/ops3d_fda.h"
#include "../../include/ops3d_dcnv4.h"
#include "../../include/ops3d_nms3d.h"
#include "../../include/ops3d_roi_align3d.h"

namespace {

int dtype_code(const at::Tensor &t) {
  switch (t.scalar_type()) {
    case at::kFloat: return OPS3D_FDA_F32;
    case at::kHalf: return OPS3D_FDA_F16;
    case at::kBFloat16: return OPS3D_FDA_BF16;
    default: throw std::invalid_argument(std::string("unsupported value dtype ") + c10::toString(t.scalar_type()));
  }
}

void check_tensor(const at::Tensor &t, const char *name, const at::Tensor &value) {
  // reference csrc/flash_deform_attn.h:24,51 (CPU tensors are not implemented)
  if (!t.is_cuda()) throw std::runtime_error(std::string("Not implemented on the CPU (") + name + " is on the CPU)");
  if (!t.is_contiguous()) throw std::runtime_error(std::string(name) + " tensor has to be contiguous");
  if (t.device() != value.device()) throw std::runtime_error(std::string(name) + " is on another device than value");
}

struct Sizes {
  int code, B, S, G, D, L, Q, K;
};

// Shared checks of every entry point; returns the problem sizes.
Sizes common(const at::Tensor &value, const at::Tensor &shapes, const at::Tensor &lsi, const at::Tensor &sla,
             int64_t K) {
  check_tensor(value, "value", value);
  check_tensor(shapes, "spatial_shapes", value);
  check_tensor(lsi, "level_start_index", value);
  check_tensor(sla, "sampling_loc_attn", value);
  Sizes z{};
  z.code = dtype_code(value);
  if (sla.scalar_type() != value.scalar_type())
    throw std::invalid_argument("sampling_loc_attn dtype differs from value dtype");
  if (shapes.scalar_type() != at::kLong || lsi.scalar_type() != at::kLong)
    throw std::invalid_argument("spatial_shapes and level_start_index must be int64");
  if (value.dim() != 4) throw std::invalid_argument("value must be [B, S, G, D]");
  if (shapes.dim() != 2 || shapes.size(1) != 3) throw std::invalid_argument("spatial_shapes must be [L, 3]");
  const int64_t L = shapes.size(0);
  if (lsi.dim() != 1 || lsi.size(0) != L) throw std::invalid_argument("level_start_index must be [L]");
  if (sla.dim() != 4 || sla.size(0) != value.size(0) || sla.size(2) != value.size(2))
    throw std::invalid_argument("sampling_loc_attn must be [B, Q, G, P]");
  if (sla.size(3) != L * K * 4)
    throw std::invalid_argument("sampling_loc_attn last dimension (" + std::to_string(sla.size(3)) +
                                ") does not match L=" + std::to_string(L) + ", K=" + std::to_string(K) +
                                " (expected " + std::to_string(L * K * 4) + ")");
  z.B = (int)value.size(0);
  z.S = (int)value.size(1);
  z.G = (int)value.size(2);
  z.D = (int)value.size(3);
  z.L = (int)L;
  z.Q = (int)sla.size(1);
  z.K = (int)K;
  return z;
}

void raise(int rc, const char *what) {
  const char *msg = ops3d_fda_last_error();
  const std::string m = (msg && *msg) ? msg : what;
  if (rc == OPS3D_FDA_EINVAL) throw std::invalid_argument(m);
  throw std::runtime_error(m);
}

hipStream_t stream_of(const at::Tensor &value) {
  return c10::hip::getCurrentHIPStream(value.device().index()).stream();
}

// Makes value's device current for the call and restores the previous one (the reference's
// entry points rely on the current device; torch's own guard types for ROCm label HIP devices
// as cuda, so plain HIP calls are used here).
class DeviceGuard {
 public:
  explicit DeviceGuard(const c10::Device &d) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (d.has_index() && d.index() != prev_ && hipSetDevice(d.index()) == hipSuccess) set_ = true;
  }
  ~DeviceGuard() {
    if (set_ && prev_ >= 0) (void)hipSetDevice(prev_);
  }
  DeviceGuard(const DeviceGuard &) = delete;
  DeviceGuard &operator=(const DeviceGuard &) = delete;

 private:
  int prev_ = -1;
  bool set_ = false;
};

void *ptr(const at::Tensor &t) { return t.defined() && t.numel() > 0 ? t.data_ptr() : nullptr; }

void check_grad_output(const at::Tensor &grad_output, const at::Tensor &value, const Sizes &z) {
  check_tensor(grad_output, "grad_output", value);
  if (grad_output.scalar_type() != value.scalar_type())
    throw std::invalid_argument("grad_output dtype differs from value dtype");
  if (grad_output.numel() != (int64_t)z.B * z.Q * z.G * z.D)
    throw std::invalid_argument("grad_output must have B*Q*G*D elements");
}

// Forward; returns the output and the forward workspace (the head-major copy of value), which
// is undefined (None) when the library makes no copy.
std::tuple<at::Tensor, c10::optional<at::Tensor>> forward_keep_head_major(
    const at::Tensor &value, const at::Tensor &shapes, const at::Tensor &lsi, const at::Tensor &sla,
    int64_t im2col_step, int64_t K) {
  const Sizes z = common(value, shapes, lsi, sla, K);
  const DeviceGuard guard(value.device());
  at::Tensor out = at::empty({z.B, z.Q, (int64_t)z.G * z.D}, value.options());
  const size_t n = ops3d_fda_forward_workspace_bytes(z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K);
  c10::optional<at::Tensor> ws;
  if (n) ws = at::empty({(int64_t)n}, value.options().dtype(at::kByte));
  const int rc = ops3d_fda_forward(ptr(value), shapes.data_ptr<int64_t>(), lsi.data_ptr<int64_t>(), ptr(sla),
                                   ptr(out), ws ? ws->data_ptr() : nullptr, n, z.code, z.B, z.S, z.G, z.D, z.L, z.Q,
                                   z.K, (int)im2col_step, stream_of(value));
  if (rc != OPS3D_FDA_OK) raise(rc, "flash_deform_attn_forward failed");
  return {out, ws};
}

// Backward; value_head_major: the forward workspace for this value, or None.
std::vector<at::Tensor> backward_with_head_major(const at::Tensor &value,
                                                 const c10::optional<at::Tensor> &value_head_major,
                                                 const at::Tensor &shapes, const at::Tensor &lsi,
                                                 const at::Tensor &sla, const at::Tensor &grad_output,
                                                 int64_t im2col_step, int64_t K) {
  const Sizes z = common(value, shapes, lsi, sla, K);
  check_grad_output(grad_output, value, z);
  const void *vhm = nullptr;
  if (value_head_major && value_head_major->defined()) {
    const at::Tensor &h = *value_head_major;
    const size_t need = ops3d_fda_forward_workspace_bytes(z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K);
    if (h.device() != value.device() || h.scalar_type() != at::kByte || (size_t)h.numel() != need)
      throw std::invalid_argument("value_head_major is not a forward workspace of this value");
    vhm = h.data_ptr();
  }
  const DeviceGuard guard(value.device());
  at::Tensor grad_value = at::empty_like(value);
  at::Tensor grad_sla = at::empty_like(sla);
  const size_t n = ops3d_fda_backward_workspace_bytes(z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K);
  at::Tensor ws;
  if (n) ws = at::empty({(int64_t)n}, value.options().dtype(at::kByte));
  const int rc = ops3d_fda_backward_ex(ptr(value), vhm, shapes.data_ptr<int64_t>(), lsi.data_ptr<int64_t>(),
                                       ptr(sla), ptr(grad_output), ptr(grad_value), ptr(grad_sla), ptr(ws), n,
                                       z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K, (int)im2col_step,
                                       stream_of(value));
  if (rc != OPS3D_FDA_OK) raise(rc, "flash_deform_attn_backward failed");
  return {grad_value, grad_sla};
}

// Offset mode: reference_points [B,Q,1 or L,3] fp32; returns ref_levels.
int ref_levels_of(const at::Tensor &ref, const at::Tensor &value, const Sizes &z) {
  check_tensor(ref, "reference_points", value);
  if (ref.scalar_type() != at::kFloat) throw std::invalid_argument("reference_points must be float32");
  if (ref.dim() != 4 || ref.size(0) != z.B || ref.size(1) != z.Q || ref.size(3) != 3 ||
      (ref.size(2) != 1 && ref.size(2) != z.L))
    throw std::invalid_argument("reference_points must be [B, Q, 1 or L, 3]");
  return (int)ref.size(2);
}

// Forward with offsets in voxels of their level in place of locations (ops3d_fda_forward_offsets).
std::tuple<at::Tensor, c10::optional<at::Tensor>> forward_offsets(
    const at::Tensor &value, const at::Tensor &shapes, const at::Tensor &lsi, const at::Tensor &offset_attn,
    const at::Tensor &reference_points, int64_t im2col_step, int64_t K) {
  const Sizes z = common(value, shapes, lsi, offset_attn, K);
  const int R = ref_levels_of(reference_points, value, z);
  const DeviceGuard guard(value.device());
  at::Tensor out = at::empty({z.B, z.Q, (int64_t)z.G * z.D}, value.options());
  const size_t n = ops3d_fda_forward_workspace_bytes(z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K);
  c10::optional<at::Tensor> ws;
  if (n) ws = at::empty({(int64_t)n}, value.options().dtype(at::kByte));
  const int rc = ops3d_fda_forward_offsets(ptr(value), shapes.data_ptr<int64_t>(), lsi.data_ptr<int64_t>(),
                                           ptr(offset_attn), reference_points.data_ptr<float>(), R, ptr(out),
                                           ws ? ws->data_ptr() : nullptr, n, z.code, z.B, z.S, z.G, z.D, z.L, z.Q,
                                           z.K, (int)im2col_step, stream_of(value));
  if (rc != OPS3D_FDA_OK) raise(rc, "flash_deform_attn_forward_offsets failed");
  return {out, ws};
}

// Backward of forward_offsets (ops3d_fda_backward_offsets): [grad_value, grad_offset_attn,
// grad_reference_points] (the last undefined -- None -- unless want_ref_grad).
std::vector<at::Tensor> backward_offsets(const at::Tensor &value, const c10::optional<at::Tensor> &value_head_major,
                                         const at::Tensor &shapes, const at::Tensor &lsi,
                                         const at::Tensor &offset_attn, const at::Tensor &reference_points,
                                         const at::Tensor &grad_output, int64_t im2col_step, int64_t K,
                                         bool want_ref_grad) {
  const Sizes z = common(value, shapes, lsi, offset_attn, K);
  check_grad_output(grad_output, value, z);
  const int R = ref_levels_of(reference_points, value, z);
  const void *vhm = nullptr;
  if (value_head_major && value_head_major->defined()) {
    const at::Tensor &h = *value_head_major;
    const size_t need = ops3d_fda_forward_workspace_bytes(z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K);
    if (h.device() != value.device() || h.scalar_type() != at::kByte || (size_t)h.numel() != need)
      throw std::invalid_argument("value_head_major is not a forward workspace of this value");
    vhm = h.data_ptr();
  }
  const DeviceGuard guard(value.device());
  at::Tensor grad_value = at::empty_like(value);
  at::Tensor grad_oa = at::empty_like(offset_attn);
  at::Tensor grad_ref;
  if (want_ref_grad) grad_ref = at::zeros_like(reference_points);
  const size_t n = ops3d_fda_backward_workspace_bytes(z.code, z.B, z.S, z.G, z.D, z.L, z.Q, z.K);
  at::Tensor ws;
  if (n) ws = at::empty({(int64_t)n}, value.options().dtype(at::kByte));
  const int rc = ops3d_fda_backward_offsets(ptr(value), vhm, shapes.data_ptr<int64_t>(), lsi.data_ptr<int64_t>(),
                                            ptr(offset_attn), reference_points.data_ptr<float>(), R, ptr(grad_output),
                                            ptr(grad_value), ptr(grad_oa),
                                            want_ref_grad ? grad_ref.data_ptr<float>() : nullptr, ptr(ws), n, z.code, z.B, z.S, z.G, z.D,
                                            z.L, z.Q, z.K, (int)im2col_step, stream_of(value));
  if (rc != OPS3D_FDA_OK) raise(rc, "flash_deform_attn_backward_offsets failed");
  return {grad_value, grad_oa, grad_ref};
}

// reference csrc/flash_deform_attn.h:7-25 (d_stride, block_thread and use_reg are launch hints
// of the CUDA build; the gfx950 library chooses its own geometry)
at::Tensor flash_deform_attn_forward(const at::Tensor &value, const at::Tensor &shapes, const at::Tensor &lsi,
                                     const at::Tensor &sla, int64_t im2col_step, int64_t K, int64_t /*d_stride*/,
                                     int64_t /*block_thread*/, bool /*use_reg*/) {
  return std::get<0>(forward_keep_head_major(value, shapes, lsi, sla, im2col_step, K));
}

// reference csrc/flash_deform_attn.h:27-52
std::vector<at::Tensor> flash_deform_attn_backward(const at::Tensor &value, const at::Tensor &shapes,
                                                   const at::Tensor &lsi, const at::Tensor &sla,
                                                   const at::Tensor &grad_output, int64_t im2col_step, int64_t K,
                                                   int64_t /*d_stride*/, int64_t /*block_thread*/) {
  return backward_with_head_major(value, c10::nullopt, shapes, lsi, sla, grad_output, im2col_step, K);
}

// reference csrc/nms_3d.h:27-44 -> nms_3d_cuda (csrc/cuda/nms_3d_cuda.cu:105-162): boxes [N,6]
// (x1,y1,z1,x2,y2,z2) and scores [N] on the GPU -> int64 indices of the kept boxes in
// decreasing score order.  Ties in score keep index order (a stable sort).  The kept count is
// read back to size the result (the reference synchronises too).
at::Tensor nms_3d(const at::Tensor &dets, const at::Tensor &scores, double threshold) {
  if (!dets.is_cuda()) throw std::runtime_error("Not compiled with CPU support");
  if (dets.numel() == 0) return at::empty({0}, dets.options().dtype(at::kLong));
  if (dets.dim() != 2 || dets.size(1) != 6) throw std::invalid_argument("dets must be [N, 6] (x1,y1,z1,x2,y2,z2)");
  if (scores.dim() != 1 || scores.size(0) != dets.size(0) || scores.device() != dets.device())
    throw std::invalid_argument("scores must be [N] on the boxes' device");
  const DeviceGuard guard(dets.device());
  const at::Tensor order = std::get<1>(scores.sort(/*stable=*/true, /*dim=*/0, /*descending=*/true));
  const at::Tensor boxes = dets.index_select(0, order).to(at::kFloat).contiguous();
  const int n = (int)boxes.size(0);
  const size_t wsb = ops3d_nms3d_workspace_bytes(n);
  at::Tensor ws = at::empty({(int64_t)wsb}, dets.options().dtype(at::kByte));
  at::Tensor keep = at::empty({n}, dets.options().dtype(at::kLong));
  at::Tensor num = at::empty({1}, dets.options().dtype(at::kInt));
  const int rc = ops3d_nms3d(boxes.data_ptr<float>(), order.data_ptr<int64_t>(), n, (float)threshold, ws.data_ptr(),
                             wsb, keep.data_ptr<int64_t>(), num.data_ptr<int32_t>(), stream_of(dets));
  if (rc == OPS3D_FDA_EINVAL) throw std::invalid_argument("nms_3d: too many boxes (at most 2^19)");
  if (rc != OPS3D_FDA_OK) throw std::runtime_error("nms_3d: kernel launch failed");
  return keep.narrow(0, 0, num.item<int32_t>());
}

// RoI Align 3-D (reference csrc/roi_align_3d.h:35-136): shared checks; returns the dtype code.
int roi_checks(const at::Tensor &data, const at::Tensor &rois, const at::Tensor &other) {
  if (!data.is_cuda()) throw std::runtime_error("RoIAlign is not implemented on CPU");
  if (rois.dim() != 2 || rois.size(1) != 7) throw std::runtime_error("wrong roi size! size_rois should be 7");
  for (const at::Tensor *t : {&rois, &other}) {
    if (t->device() != data.device()) throw std::runtime_error("RoIAlign tensors must be on one device");
    if (t->scalar_type() != data.scalar_type()) throw std::invalid_argument("RoIAlign tensors must share a dtype");
  }
  if (!other.is_contiguous()) throw std::runtime_error("RoIAlign output tensor has to be contiguous");
  return dtype_code(data);
}

// Features already in channels_last_3d memory ([N,D,H,W,C] order, 16-byte aligned).
bool is_channels_last_input(const at::Tensor &input) {
  return !input.is_contiguous() && input.is_contiguous(at::MemoryFormat::ChannelsLast3d) &&
         (reinterpret_cast<uintptr_t>(input.data_ptr()) & 15u) == 0;
}

// Whether the forward runs the channels-last kernel: always on channels-last input it supports;
// on [N,C,D,H,W] input when the output has at least kRoiClMinOutputs elements, so that the
// transposed copy of the features is repaid (below that the NCDHW kernel is as fast).
constexpr int64_t kRoiClMinOutputs = (int64_t)1 << 19;
bool roi_channels_last(const at::Tensor &input, int code, int R, int pd, int ph, int pw) {
  const int C = (int)input.size(1);
  if (!ops3d_roi_align3d_channels_last_supported(code, C, (int)input.size(2), (int)input.size(3),
                                                 (int)input.size(4), pw) ||
      input.size(0) > 65535)
    return false;
  return is_channels_last_input(input) || (int64_t)R * C * pd * ph * pw >= kRoiClMinOutputs;
}

void roi_align_3d_forward(const at::Tensor &input, const at::Tensor &rois, at::Tensor output, int64_t pd, int64_t ph,
                          int64_t pw, double spatial_scale, int64_t sampling_ratio, int64_t order) {
  const int code = roi_checks(input, rois, output);
  if (input.dim() != 5) throw std::invalid_argument("features must be [N, C, D, H, W]");
  const at::Tensor r = rois.contiguous();
  if (output.dim() != 5 || output.size(0) != r.size(0) || output.size(1) != input.size(1) || output.size(2) != pd ||
      output.size(3) != ph || output.size(4) != pw)
    throw std::invalid_argument("output must be [R, C, out_d, out_h, out_w]");
  const DeviceGuard guard(input.device());
  const int N = (int)input.size(0), C = (int)input.size(1), D = (int)input.size(2), H = (int)input.size(3),
            W = (int)input.size(4), R = (int)r.size(0);
  int rc;
  if (roi_channels_last(input, code, R, (int)pd, (int)ph, (int)pw)) {
    // channels-last kernel: on the caller's channels_last_3d memory, or on a transposed copy
    at::Tensor fc = input;
    if (!is_channels_last_input(input)) {
      const at::Tensor f = input.contiguous();
      fc = at::empty({N, D, H, W, C}, input.options());
      rc = ops3d_roi_align3d_to_channels_last(ptr(f), ptr(fc), code, N, C, D, H, W, stream_of(input));
      if (rc != OPS3D_FDA_OK) throw std::runtime_error("roi_align_3d_forward: channels-last copy failed");
    }
    rc = ops3d_roi_align3d_forward_channels_last(ptr(fc), ptr(r), ptr(output), code, N, C, D, H, W, R, (int)pd,
                                                 (int)ph, (int)pw, (float)spatial_scale, (int)sampling_ratio,
                                                 (int)order, stream_of(input));
  } else {
    const at::Tensor f = input.contiguous();
    rc = ops3d_roi_align3d_forward(ptr(f), ptr(r), ptr(output), code, N, C, D, H, W, R, (int)pd, (int)ph, (int)pw,
                                   (float)spatial_scale, (int)sampling_ratio, (int)order, stream_of(input));
  }
  if (rc == OPS3D_FDA_EINVAL) throw std::invalid_argument("roi_align_3d_forward: invalid sizes or order");
  if (rc != OPS3D_FDA_OK) throw std::runtime_error("roi_align_3d_forward: kernel launch failed");
}

void roi_align_3d_backward(const at::Tensor &top_grad, const at::Tensor &rois, at::Tensor bottom_grad, int64_t pd,
                           int64_t ph, int64_t pw, double spatial_scale, int64_t sampling_ratio, int64_t order) {
  const int code = roi_checks(top_grad, rois, bottom_grad);
  if (bottom_grad.dim() != 5) throw std::invalid_argument("bottom_grad must be [N, C, D, H, W]");
  const at::Tensor g = top_grad.contiguous(), r = rois.contiguous();
  const int N = (int)bottom_grad.size(0), C = (int)bottom_grad.size(1), D = (int)bottom_grad.size(2),
            H = (int)bottom_grad.size(3), W = (int)bottom_grad.size(4);
  if (g.dim() != 5 || g.size(0) != r.size(0) || g.size(1) != C || g.size(2) != pd || g.size(3) != ph ||
      g.size(4) != pw)
    throw std::invalid_argument("top_grad must be [R, C, out_d, out_h, out_w]");
  const DeviceGuard guard(top_grad.device());
  const size_t wsb =
      ops3d_roi_align3d_backward_workspace_bytes(code, N, C, D, H, W, (int)r.size(0), (int)pd, (int)ph, (int)pw);
  at::Tensor ws;
  if (wsb) ws = at::empty({(int64_t)((wsb + 3) / 4)}, top_grad.options().dtype(at::kFloat));
  const int rc = ops3d_roi_align3d_backward(ptr(g), ptr(r), ptr(bottom_grad), ptr(ws), wsb, code, N, C, D, H, W,
                                            (int)r.size(0), (int)pd, (int)ph, (int)pw, (float)spatial_scale,
                                            (int)sampling_ratio, (int)order, stream_of(top_grad));
  if (rc == OPS3D_FDA_EINVAL) throw std::invalid_argument("roi_align_3d_backward: invalid sizes or order");
  if (rc != OPS3D_FDA_OK) throw std::runtime_error("roi_align_3d_backward: kernel launch failed");
}

// DCNv4-3D (reference csrc/dcnv4.h:7-60): value [B,Din,Hin,Win,G*D], p_offset
// [B,Dout,Hout,Wout,padded]; d_stride and block_thread are launch hints of the CUDA build
// (accepted, not used).
struct DcnArgs {
  int B, Din, Hin, Win, code;
};

DcnArgs dcn_check(const at::Tensor &value, const at::Tensor &p_offset, int64_t group, int64_t group_channels) {
  if (!value.is_cuda()) throw std::runtime_error("Not implemented on the CPU");
  if (!p_offset.is_cuda()) throw std::runtime_error("offset must be a CUDA tensor");
  if (!value.is_contiguous()) throw std::runtime_error("input tensor has to be contiguous");
  if (!p_offset.is_contiguous()) throw std::runtime_error("offset tensor has to be contiguous");
  if (value.dim() != 5 || p_offset.dim() != 5) throw std::invalid_argument("value and p_offset must be 5-D");
  if (p_offset.scalar_type() != value.scalar_type()) throw std::invalid_argument("p_offset dtype differs from value");
  if (value.size(4) != group * group_channels)
    throw std::runtime_error("Input channels and group times group channels dont match");
  return {(int)value.size(0), (int)value.size(1), (int)value.size(2), (int)value.size(3), dtype_code(value)};
}

at::Tensor dcnv4_forward(const at::Tensor &value, const at::Tensor &p_offset, int64_t kd, int64_t kh, int64_t kw,
                         int64_t sd, int64_t sh, int64_t sw, int64_t pd, int64_t ph, int64_t pw, int64_t dd,
                         int64_t dh, int64_t dw, int64_t group, int64_t group_channels, double offset_scale,
                         int64_t im2col_step, int64_t remove_center, int64_t /*d_stride*/, int64_t /*block_thread*/,
                         bool softmax) {
  const DcnArgs z = dcn_check(value, p_offset, group, group_channels);
  const int Dout = (z.Din + 2 * (int)pd - ((int)dd * ((int)kd - 1) + 1)) / (int)sd + 1;
  const int Hout = (z.Hin + 2 * (int)ph - ((int)dh * ((int)kh - 1) + 1)) / (int)sh + 1;
  const int Wout = (z.Win + 2 * (int)pw - ((int)dw * ((int)kw - 1) + 1)) / (int)sw + 1;
  if (p_offset.size(0) != z.B || p_offset.size(1) != Dout || p_offset.size(2) != Hout || p_offset.size(3) != Wout)
    throw std::invalid_argument("p_offset must be [B, Dout, Hout, Wout, padded_offset_dim]");
  const DeviceGuard guard(value.device());
  at::Tensor out = at::empty({z.B, Dout, Hout, Wout, group * group_channels}, value.options());
  const size_t wsb = ops3d_dcnv4_workspace_bytes(z.code, z.B, z.Din, z.Hin, z.Win, (int)group, (int)group_channels,
                                                 (int)kd, (int)kh, (int)kw, (int)sd, (int)sh, (int)sw, (int)pd,
                                                 (int)ph, (int)pw, (int)dd, (int)dh, (int)dw, (int)remove_center, 0);
  at::Tensor ws = at::empty({(int64_t)(wsb ? wsb : 256)}, value.options().dtype(at::kByte));
  const int rc = ops3d_dcnv4_forward(ptr(value), ptr(p_offset), ptr(out), ws.data_ptr(), wsb, z.code, z.B, z.Din,
                                     z.Hin, z.Win, (int)group, (int)group_channels, (int)kd, (int)kh, (int)kw,
                                     (int)sd, (int)sh, (int)sw, (int)pd, (int)ph, (int)pw, (int)dd, (int)dh, (int)dw,
                                     (float)offset_scale, (int)remove_center, softmax ? 1 : 0,
                                     (int)p_offset.size(4), (int)im2col_step, stream_of(value));
  if (rc != OPS3D_FDA_OK) raise(rc, "dcnv4_forward failed");
  return out;
}

std::vector<at::Tensor> dcnv4_backward(const at::Tensor &value, const at::Tensor &p_offset, int64_t kd, int64_t kh,
                                       int64_t kw, int64_t sd, int64_t sh, int64_t sw, int64_t pd, int64_t ph,
                                       int64_t pw, int64_t dd, int64_t dh, int64_t dw, int64_t group,
                                       int64_t group_channels, double offset_scale, int64_t im2col_step,
                                       const at::Tensor &grad_output, int64_t remove_center,
                                       int64_t /*d_stride*/, int64_t /*block_thread*/, bool softmax) {
  const DcnArgs z = dcn_check(value, p_offset, group, group_channels);
  if (!grad_output.is_cuda() || !grad_output.is_contiguous() || grad_output.scalar_type() != value.scalar_type())
    throw std::runtime_error("grad_output tensor has to be a contiguous CUDA tensor of the value dtype");
  const DeviceGuard guard(value.device());
  at::Tensor grad_value = at::empty_like(value);
  at::Tensor grad_offset = at::zeros_like(p_offset);   // the row padding stays zero
  const size_t wsb = ops3d_dcnv4_workspace_bytes(z.code, z.B, z.Din, z.Hin, z.Win, (int)group, (int)group_channels,
                                                 (int)kd, (int)kh, (int)kw, (int)sd, (int)sh, (int)sw, (int)pd,
                                                 (int)ph, (int)pw, (int)dd, (int)dh, (int)dw, (int)remove_center, 1);
  at::Tensor ws = at::empty({(int64_t)(wsb ? wsb : 256)}, value.options().dtype(at::kByte));
  const int rc = ops3d_dcnv4_backward(ptr(value), ptr(p_offset), ptr(grad_output), ptr(grad_value), ptr(grad_offset),
                                      ws.data_ptr(), wsb, z.code, z.B, z.Din, z.Hin, z.Win, (int)group,
                                      (int)group_channels, (int)kd, (int)kh, (int)kw, (int)sd, (int)sh, (int)sw,
                                      (int)pd, (int)ph, (int)pw, (int)dd, (int)dh, (int)dw, (float)offset_scale,
                                      (int)remove_center, softmax ? 1 : 0, (int)p_offset.size(4), (int)im2col_step,
                                      stream_of(value));
  if (rc != OPS3D_FDA_OK) raise(rc, "dcnv4_backward failed");
  return {grad_value, grad_offset};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("flash_deform_attn_forward", &flash_deform_attn_forward, "flash_deform_attn_forward",
        py::arg("value"), py::arg("spatial_shapes"), py::arg("level_start_index"), py::arg("sampling_loc_attn"),
        py::arg("im2col_step"), py::arg("K"), py::arg("d_stride") = 8, py::arg("block_thread") = 0,
        py::arg("use_reg") = true);
  m.def("flash_deform_attn_backward", &flash_deform_attn_backward, "flash_deform_attn_backward",
        py::arg("value"), py::arg("spatial_shapes"), py::arg("level_start_index"), py::arg("sampling_loc_attn"),
        py::arg("grad_output"), py::arg("im2col_step"), py::arg("K"), py::arg("d_stride") = 1,
        py::arg("block_thread") = 0);
  m.def("forward_keep_head_major", &forward_keep_head_major, "forward that also returns its workspace");
  m.def("backward_with_head_major", &backward_with_head_major, "backward reusing the forward workspace");
  m.def("forward_offsets", &forward_offsets, "forward from offsets and reference points");
  m.def("backward_offsets", &backward_offsets, "backward of forward_offsets");
  m.def("nms_3d", &nms_3d, "non-maximum suppression for 3d");
  m.def("dcnv4_forward", &dcnv4_forward, "dcnv4_forward");
  m.def("dcnv4_backward", &dcnv4_backward, "dcnv4_backward");
  m.def("roi_align_3d_forward", &roi_align_3d_forward, "roi_align_3d_forward");
  m.def("roi_align_3d_backward", &roi_align_3d_backward, "roi_align_3d_backward");
}
