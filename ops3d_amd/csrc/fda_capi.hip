// C ABI of libops3d_fda.so: argument validation, launch geometry and the two entry points.
//
// Replaces the ATen host code of the reference (csrc/cuda/flash_deform_attn_cuda.cu:20-179)
// and its template launchers (flash_deform_im2col_cuda.cuh:298-593,
// flash_deform_col2im_cuda.cuh:432-730).  Differences by design:
//   * the launch geometry is chosen here for gfx950 (wave64 units of LPU lanes, 256-thread
//     blocks of one head, XCD-aware block order); the reference's d_stride / block_thread
//     hints are accepted by the Python layer and ignored;
//   * the whole batch is one launch: im2col_step chunking gives identical results, so it is
//     only validated (min(B, step) must divide B, as flash_deform_attn_cuda.cu:56-58);
//   * outputs are written in full by the kernels (no zero-fill of output / grad_offset), and
//     only the fp32 grad_value accumulator is cleared and converted.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "../../include/ops3d_fda.h"
#include "fda_device.h"

namespace ops3d_fda {
hipError_t launch_f32(bool, int, int, const Args &, unsigned, size_t, hipStream_t);
hipError_t launch_f16(bool, int, int, const Args &, unsigned, size_t, hipStream_t);
hipError_t launch_bf16(bool, int, int, const Args &, unsigned, size_t, hipStream_t);
}  // namespace ops3d_fda

using namespace ops3d_fda;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int elem_size(int dtype) {
  switch (dtype) {
    case OPS3D_FDA_F32: return 4;
    case OPS3D_FDA_F16: return 2;
    case OPS3D_FDA_BF16: return 2;
    default: return 0;
  }
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Channels per lane (CPL) and lanes per unit (LPU) for head width D: one 16-byte vector per
// lane when possible (8 x 16-bit or 4 x fp32 channels), else 24 bytes (12 x 16-bit, 6 x fp32);
// LPU = D / CPL must be a power of two <= 32 so a unit never straddles a wave.
bool pick_config(int dtype, int D, int &cpl, int &lpu) {
  const int e = elem_size(dtype);
  if (e == 0 || D <= 0) return false;
  const int cands2[2] = {8, 12}, cands4[2] = {4, 6};
  const int *cands = (e == 2) ? cands2 : cands4;
  for (int i = 0; i < 2; ++i) {
    const int c = cands[i];
    if (D % c) continue;
    const int l = D / c;
    if (is_pow2(l) && l <= 32) {
      cpl = c;
      lpu = l;
      return true;
    }
  }
  return false;
}

struct Geometry {
  Args a;
  unsigned grid;
  size_t lds;
  int cpl, lpu;
};

int common_checks(int dtype, int B, int S, int G, int D, int L, int Q, int K, int step,
                  bool backward, Geometry &geo) {
  if (elem_size(dtype) == 0) return fail(OPS3D_FDA_EINVAL, "unsupported dtype code %d", dtype);
  if (B < 0 || S < 0 || G <= 0 || D <= 0 || Q < 0)
    return fail(OPS3D_FDA_EINVAL, "invalid sizes B=%d S=%d G=%d D=%d Q=%d", B, S, G, D, Q);
  if (L < 1 || L > 5) return fail(OPS3D_FDA_EINVAL, "invalid number of scales L=%d (supported 1..5)", L);
  if (K < 1 || K > 16) return fail(OPS3D_FDA_EINVAL, "invalid number of points K=%d (supported 1..16)", K);
  if (step <= 0) return fail(OPS3D_FDA_EINVAL, "im2col_step must be positive, got %d", step);
  const int step_ = B < step ? B : step;
  if (B > 0 && B % step_ != 0)
    return fail(OPS3D_FDA_ERUNTIME, "batch(%d) must divide im2col_step(%d)", B, step_);
  if (!pick_config(dtype, D, geo.cpl, geo.lpu))
    return fail(OPS3D_FDA_EINVAL,
                "unsupported channels per head D=%d for this dtype (need D = c * 2^k, c in %s, "
                "2^k <= 32)",
                D, elem_size(dtype) == 2 ? "{8,12}" : "{4,6}");
  if ((int64_t)S * G * D > kMaxLevelElems)
    return fail(OPS3D_FDA_EINVAL, "value too large: S*G*D = %lld exceeds %lld elements per batch item",
                (long long)S * G * D, (long long)kMaxLevelElems);
  const int LK = L * K, P = 4 * LK;
  const int UPB = kWavesPerBlock * (kWave / geo.lpu);
  const size_t lds = (size_t)UPB * (size_t)(P + (backward ? LK : 0) + 1) * sizeof(float);
  if (lds > 64 * 1024)
    return fail(OPS3D_FDA_EINVAL, "L*K=%d too large for D=%d (needs %zu bytes of LDS per block)", LK, D, lds);

  Args &a = geo.a;
  a = Args{};
  a.B = B; a.S = S; a.G = G; a.D = D; a.L = L; a.K = K; a.Q = Q; a.P = P;
  a.nqb = (Q + UPB - 1) / UPB;
  a.ncol = B * a.nqb;
  int64_t grid;
  if (G % 8 == 0) {
    a.xcd_mode = 0; a.hpx = G / 8;
    grid = (int64_t)G * a.ncol;
  } else if (8 % G == 0) {
    a.xcd_mode = 1; a.xpg = 8 / G;
    grid = 8 * (((int64_t)a.ncol + a.xpg - 1) / a.xpg);
  } else {
    a.xcd_mode = 2;
    grid = (int64_t)G * a.ncol;
  }
  if (grid > 0x7fffffff) return fail(OPS3D_FDA_EINVAL, "problem too large (%lld blocks)", (long long)grid);
  geo.grid = (unsigned)grid;
  geo.lds = lds;
  return OPS3D_FDA_OK;
}

bool misaligned(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) != 0; }

hipError_t launch(int dtype, bool backward, const Geometry &g, hipStream_t st) {
  switch (dtype) {
    case OPS3D_FDA_F32: return launch_f32(backward, g.cpl, g.lpu, g.a, g.grid, g.lds, st);
    case OPS3D_FDA_F16: return launch_f16(backward, g.cpl, g.lpu, g.a, g.grid, g.lds, st);
    default: return launch_bf16(backward, g.cpl, g.lpu, g.a, g.grid, g.lds, st);
  }
}

// Fill n floats with zero (a kernel, not hipMemsetAsync, so a captured graph replays correctly).
__global__ __launch_bounds__(256) void zero_f32_kernel(float *p, int64_t n) {
  const int64_t n4 = n >> 2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
    reinterpret_cast<float4 *>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < (n & 3)) p[(n4 << 2) + t] = 0.f;
}

// fp32 -> T, 4 elements per thread and step.
template <typename T>
__global__ __launch_bounds__(256) void convert_kernel(const float *src, T *dst, int64_t n) {
  const int64_t n4 = n >> 2;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4 *>(src)[i];
    const float f[4] = {v.x, v.y, v.z, v.w};
    const uint32_t w0 = Elem<T>::pack(f), w1 = Elem<T>::pack(f + 2);
    reinterpret_cast<u32x2 *>(dst)[i] = u32x2{w0, w1};
  }
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < (n & 3)) dst[(n4 << 2) + t] = (T)src[(n4 << 2) + t];
}

unsigned elementwise_grid(int64_t n) {
  int64_t blocks = ((n >> 2) + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  return (unsigned)blocks;
}

}  // namespace

extern "C" {

int ops3d_fda_abi_version(void) { return 1; }

const char *ops3d_fda_last_error(void) { return g_last_error.c_str(); }

int ops3d_fda_supported(int dtype, int channels) {
  int cpl, lpu;
  return pick_config(dtype, channels, cpl, lpu) ? 1 : 0;
}

int ops3d_fda_forward(const void *value, const int64_t *spatial_shapes,
                      const int64_t *level_start_index, const void *sampling_loc_attn,
                      void *output, int dtype, int batch, int spatial_size, int num_heads,
                      int channels, int num_levels, int num_query, int num_point,
                      int im2col_step, void *stream) {
  g_last_error.clear();
  Geometry geo;
  int rc = common_checks(dtype, batch, spatial_size, num_heads, channels, num_levels, num_query,
                         num_point, im2col_step, false, geo);
  if (rc) return rc;
  if ((int64_t)batch * num_query == 0) return OPS3D_FDA_OK;
  if (!value && spatial_size > 0) return fail(OPS3D_FDA_EINVAL, "value is NULL");
  if (!spatial_shapes || !level_start_index || !sampling_loc_attn || !output)
    return fail(OPS3D_FDA_EINVAL, "NULL pointer argument");
  if (misaligned(value) || misaligned(sampling_loc_attn) || misaligned(output))
    return fail(OPS3D_FDA_EINVAL, "tensor data pointers must be 4-byte aligned");
  geo.a.value = value;
  geo.a.shapes = spatial_shapes;
  geo.a.lsi = level_start_index;
  geo.a.loc_attn = sampling_loc_attn;
  geo.a.out = output;
  hipError_t e = launch(dtype, false, geo, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(OPS3D_FDA_ERUNTIME, "forward kernel launch failed: %s (grid=%u, lds=%zu)",
                hipGetErrorString(e), geo.grid, geo.lds);
  return OPS3D_FDA_OK;
}

size_t ops3d_fda_backward_workspace_bytes(int dtype, int batch, int spatial_size, int num_heads,
                                          int channels) {
  if (dtype == OPS3D_FDA_F32 || batch <= 0 || spatial_size <= 0 || num_heads <= 0 || channels <= 0)
    return 0;
  return (size_t)batch * spatial_size * num_heads * channels * sizeof(float);
}

static int backward_impl(const void *value, const int64_t *spatial_shapes,
                         const int64_t *level_start_index, const void *sampling_loc_attn,
                         const void *grad_output, float *acc, void *grad_sampling_loc_attn,
                         int dtype, int batch, int spatial_size, int num_heads, int channels,
                         int num_levels, int num_query, int num_point, int im2col_step,
                         hipStream_t st, bool zero_first, void *convert_to) {
  Geometry geo;
  int rc = common_checks(dtype, batch, spatial_size, num_heads, channels, num_levels, num_query,
                         num_point, im2col_step, true, geo);
  if (rc) return rc;
  const int64_t nval = (int64_t)batch * spatial_size * num_heads * channels;
  const bool work = (int64_t)batch * num_query > 0;
  if (nval > 0 && !acc) return fail(OPS3D_FDA_EINVAL, "grad_value is NULL");
  if (work && (!spatial_shapes || !level_start_index || !sampling_loc_attn || !grad_output ||
               !grad_sampling_loc_attn || (!value && spatial_size > 0)))
    return fail(OPS3D_FDA_EINVAL, "NULL pointer argument");
  if (misaligned(value) || misaligned(sampling_loc_attn) || misaligned(grad_output) ||
      misaligned(grad_sampling_loc_attn) || misaligned(acc) || misaligned(convert_to))
    return fail(OPS3D_FDA_EINVAL, "tensor data pointers must be 4-byte aligned");
  if (zero_first && nval > 0) {
    hipLaunchKernelGGL(zero_f32_kernel, dim3(elementwise_grid(nval)), dim3(256), 0, st, acc, nval);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "zero-fill launch failed: %s", hipGetErrorString(e));
  }
  if (work) {
    geo.a.value = value;
    geo.a.shapes = spatial_shapes;
    geo.a.lsi = level_start_index;
    geo.a.loc_attn = sampling_loc_attn;
    geo.a.grad_out = grad_output;
    geo.a.grad_value = acc;
    geo.a.grad_loc_attn = grad_sampling_loc_attn;
    hipError_t e = launch(dtype, true, geo, st);
    if (e != hipSuccess)
      return fail(OPS3D_FDA_ERUNTIME, "backward kernel launch failed: %s (grid=%u, lds=%zu)",
                  hipGetErrorString(e), geo.grid, geo.lds);
  }
  if (convert_to && nval > 0) {
    if (dtype == OPS3D_FDA_F16)
      hipLaunchKernelGGL(convert_kernel<_Float16>, dim3(elementwise_grid(nval)), dim3(256), 0, st,
                         acc, static_cast<_Float16 *>(convert_to), nval);
    else
      hipLaunchKernelGGL(convert_kernel<__bf16>, dim3(elementwise_grid(nval)), dim3(256), 0, st,
                         acc, static_cast<__bf16 *>(convert_to), nval);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "convert launch failed: %s", hipGetErrorString(e));
  }
  return OPS3D_FDA_OK;
}

int ops3d_fda_backward(const void *value, const int64_t *spatial_shapes,
                       const int64_t *level_start_index, const void *sampling_loc_attn,
                       const void *grad_output, void *grad_value,
                       void *grad_sampling_loc_attn, void *workspace, size_t workspace_bytes,
                       int dtype, int batch, int spatial_size, int num_heads, int channels,
                       int num_levels, int num_query, int num_point, int im2col_step,
                       void *stream) {
  g_last_error.clear();
  if (elem_size(dtype) == 0) return fail(OPS3D_FDA_EINVAL, "unsupported dtype code %d", dtype);
  const size_t need = ops3d_fda_backward_workspace_bytes(dtype, batch, spatial_size, num_heads, channels);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(OPS3D_FDA_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  const bool f32 = dtype == OPS3D_FDA_F32;
  float *acc = f32 ? static_cast<float *>(grad_value) : static_cast<float *>(workspace);
  if (!f32 && need > 0 && !grad_value) return fail(OPS3D_FDA_EINVAL, "grad_value is NULL");
  return backward_impl(value, spatial_shapes, level_start_index, sampling_loc_attn, grad_output, acc,
                       grad_sampling_loc_attn, dtype, batch, spatial_size, num_heads, channels,
                       num_levels, num_query, num_point, im2col_step, static_cast<hipStream_t>(stream),
                       true, f32 ? nullptr : grad_value);
}

int ops3d_fda_backward_accumulate_f32(const void *value, const int64_t *spatial_shapes,
                                      const int64_t *level_start_index,
                                      const void *sampling_loc_attn, const void *grad_output,
                                      float *grad_value_f32, void *grad_sampling_loc_attn,
                                      int dtype, int batch, int spatial_size, int num_heads,
                                      int channels, int num_levels, int num_query, int num_point,
                                      int im2col_step, void *stream) {
  g_last_error.clear();
  return backward_impl(value, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
                       grad_value_f32, grad_sampling_loc_attn, dtype, batch, spatial_size, num_heads,
                       channels, num_levels, num_query, num_point, im2col_step,
                       static_cast<hipStream_t>(stream), false, nullptr);
}

}  // extern "C"
