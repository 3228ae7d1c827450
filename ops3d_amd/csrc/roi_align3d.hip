// 3-D RoI Align on gfx950 (replaces the reference's roi_align_3d_{forward,backward}_cuda_kernel,
// csrc/cuda/roi_align_3d_cuda_kernel.cuh:27-220, with the interpolation helpers of
// csrc/cuda/interpolation_helpers_3d.h:25-260; bound as _C.roi_align_3d_forward/backward by
// csrc/roi_align_3d.h:97-136).
//
// features [N, C, D, H, W]; rois [R, 7] (batch index, x1, y1, z1, x2, y2, z2) in the features'
// dtype; output [R, C, PD, PH, PW].  Per output bin: the roi scaled by spatial_scale (no
// rounding), extents clamped to >= 1, the bin cut into a grid of samples (sampling_ratio per
// axis, or ceil(extent / pooled) when it is <= 0), each sample interpolated (order 1: trilinear
// with the reference's edge handling -- a sample beyond [-1, size] reads 0, coordinates below 0
// clamp to 0, a base corner at size-1 collapses both corners onto it; order 0: the nearest
// corner), and the samples averaged.  All arithmetic is fp32 (16-bit types are widened on load;
// the reference computes in the element type), rounded step by step (no contraction).
//
// Forward: a gather, one thread per (roi, group of CPT channels, bin), so each sample's
// set-up (8 offsets and weights) serves CPT channels.  Backward: the adjoint scatter of
// top_grad * w / count into the 8 corners with fp32 hardware atomics, into the fp32 gradient
// itself or, for 16-bit types, into an fp32 workspace cast afterwards; the call clears it first
// (a fill kernel) and writes every element of grad_input.  A roi whose batch index is outside
// [0, N) reads and writes nothing (its output is 0; the reference indexes out of bounds).
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/ops3d_roi_align3d.h"

namespace ops3d_roi {

template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

struct Roi {
  int b;
  float sw, sh, sd;      // roi start (x, y, z) in feature voxels
  float bw, bh, bd;      // bin sizes
  int gw, gh, gd;        // samples per bin and axis
  float count;
};

template <typename T>
__device__ __forceinline__ Roi roi_setup(const T *rois, int r, float scale, int sr, int PD, int PH, int PW) {
#pragma clang fp contract(off)
  const T *p = rois + (int64_t)r * 7;
  Roi o;
  o.b = (int)to_f(p[0]);
  o.sw = to_f(p[1]) * scale;
  o.sh = to_f(p[2]) * scale;
  o.sd = to_f(p[3]) * scale;
  const float ew = to_f(p[4]) * scale, eh = to_f(p[5]) * scale, ed = to_f(p[6]) * scale;
  const float rw = fmaxf(ew - o.sw, 1.f), rh = fmaxf(eh - o.sh, 1.f), rd = fmaxf(ed - o.sd, 1.f);
  o.bd = rd / (float)PD;
  o.bh = rh / (float)PH;
  o.bw = rw / (float)PW;
  o.gd = sr > 0 ? sr : (int)ceilf(rd / (float)PD);
  o.gh = sr > 0 ? sr : (int)ceilf(rh / (float)PH);
  o.gw = sr > 0 ? sr : (int)ceilf(rw / (float)PW);
  o.count = (float)max(o.gd * o.gh * o.gw, 1);
  return o;
}

// Sample coordinate along one axis: start + p * bin + (i + 0.5) * bin / grid.
__device__ __forceinline__ float sample_coord(float start, int p, float bin, int i, int grid) {
#pragma clang fp contract(off)
  return start + (float)p * bin + ((float)i + 0.5f) * bin / (float)grid;
}

// The 8 corner offsets (voxel index inside one (batch, channel) volume) and weights of a
// sample; false when the sample lies beyond [-1, size] on some axis (it contributes nothing).
// Corner order: (z0|z1) x (y0|y1) x (x0|x1), x fastest.
__device__ __forceinline__ bool corners(float z, float y, float x, int D, int H, int W, int order, int64_t off[8],
                                        float w[8]) {
#pragma clang fp contract(off)
  if (y < -1.f || y > (float)H || x < -1.f || x > (float)W || z < -1.f || z > (float)D) return false;
  if (z <= 0.f) z = 0.f;
  if (y <= 0.f) y = 0.f;
  if (x <= 0.f) x = 0.f;
  int z0 = (int)z, y0 = (int)y, x0 = (int)x, z1, y1, x1;
  if (z0 >= D - 1) { z1 = z0 = D - 1; z = (float)z0; } else { z1 = z0 + 1; }
  if (y0 >= H - 1) { y1 = y0 = H - 1; y = (float)y0; } else { y1 = y0 + 1; }
  if (x0 >= W - 1) { x1 = x0 = W - 1; x = (float)x0; } else { x1 = x0 + 1; }
  const float lz = z - (float)z0, ly = y - (float)y0, lx = x - (float)x0;
  const float hz = 1.f - lz, hy = 1.f - ly, hx = 1.f - lx;
  const int64_t zz[2] = {(int64_t)z0 * H * W, (int64_t)z1 * H * W}, yy[2] = {(int64_t)y0 * W, (int64_t)y1 * W};
  const int xx[2] = {x0, x1};
#pragma unroll
  for (int c = 0; c < 8; ++c) off[c] = zz[c >> 2] + yy[(c >> 1) & 1] + xx[c & 1];
  if (order == 0) {   // the first corner (in this order) whose three weights are all >= 0.5
    const bool zl = hz >= 0.5f, zh = lz >= 0.5f, yl = hy >= 0.5f, yh = ly >= 0.5f, xl = hx >= 0.5f, xh = lx >= 0.5f;
    const bool hit[8] = {zl && yl && xl, zl && yl && xh, zl && yh && xl, zl && yh && xh,
                         zh && yl && xl, zh && yl && xh, zh && yh && xl, zh && yh && xh};
    bool done = false;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      w[c] = (!done && hit[c]) ? 1.f : 0.f;
      done = done || hit[c];
    }
  } else {
    const float wz[2] = {hz, lz}, wy[2] = {hy, ly}, wx[2] = {hx, lx};
#pragma unroll
    for (int c = 0; c < 8; ++c) w[c] = wz[c >> 2] * wy[(c >> 1) & 1] * wx[c & 1];
  }
  return true;
}

template <typename T, int CPT>
__global__ __launch_bounds__(256) void roi_align3d_forward_kernel(const T *feat, const T *rois, T *out, int N, int C, int D,
                                                                  int H, int W, int R, int PD, int PH, int PW,
                                                                  float scale, int sr, int order) {
#pragma clang fp contract(off)
  const int CG = C / CPT;
  const int64_t total = (int64_t)R * CG * PD * PH * PW;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int pw = (int)(idx % PW), ph = (int)((idx / PW) % PH), pd = (int)((idx / ((int64_t)PW * PH)) % PD);
  const int cg = (int)((idx / ((int64_t)PW * PH * PD)) % CG);
  const int r = (int)(idx / ((int64_t)PW * PH * PD * CG));
  const Roi q = roi_setup(rois, r, scale, sr, PD, PH, PW);
  const int64_t vol = (int64_t)D * H * W;
  const bool inb = q.b >= 0 && q.b < N;   // a roi of a batch item that does not exist reads nothing
  const T *base = feat + ((int64_t)(inb ? q.b : 0) * C + (int64_t)cg * CPT) * vol;
  float acc[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) acc[c] = 0.f;
  for (int iz = 0; inb && iz < q.gd; ++iz) {
    const float z = sample_coord(q.sd, pd, q.bd, iz, q.gd);
    for (int iy = 0; iy < q.gh; ++iy) {
      const float y = sample_coord(q.sh, ph, q.bh, iy, q.gh);
      for (int ix = 0; ix < q.gw; ++ix) {
        const float x = sample_coord(q.sw, pw, q.bw, ix, q.gw);
        int64_t off[8];
        float w[8];
        if (!corners(z, y, x, D, H, W, order, off, w)) continue;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
          const T *v = base + (int64_t)c * vol;
          float s = w[0] * to_f(v[off[0]]);   // w1 v1 + w2 v2 + ... in order (the reference's sum)
#pragma unroll
          for (int k = 1; k < 8; ++k) s = s + w[k] * to_f(v[off[k]]);
          acc[c] = acc[c] + s;
        }
      }
    }
  }
  const int64_t o = ((((int64_t)r * C + (int64_t)cg * CPT) * PD + pd) * PH + ph) * PW + pw;
  const int64_t cs = (int64_t)PD * PH * PW;
#pragma unroll
  for (int c = 0; c < CPT; ++c) out[o + c * cs] = from_f<T>(acc[c] / q.count);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float *p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0.f;
}

template <typename T>
__global__ __launch_bounds__(256) void cast_kernel(const float *src, T *dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = from_f<T>(src[i]);
}

// One thread per (roi, channel, bin): the 8 corners of each sample get top * w / count.
template <typename T>
__global__ __launch_bounds__(256) void roi_align3d_backward_kernel(const T *top, const T *rois, float *grad, int N, int C,
                                                                   int D, int H, int W, int R, int PD, int PH, int PW,
                                                                   float scale, int sr, int order) {
#pragma clang fp contract(off)
  const int64_t total = (int64_t)R * C * PD * PH * PW;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int pw = (int)(idx % PW), ph = (int)((idx / PW) % PH), pd = (int)((idx / ((int64_t)PW * PH)) % PD);
  const int c = (int)((idx / ((int64_t)PW * PH * PD)) % C);
  const int r = (int)(idx / ((int64_t)PW * PH * PD * C));
  const float g = to_f(top[idx]);
  if (g == 0.f) return;   // adds zeros only
  const Roi q = roi_setup(rois, r, scale, sr, PD, PH, PW);
  if (q.b < 0 || q.b >= N) return;   // a roi of a batch item that does not exist
  const int64_t vol = (int64_t)D * H * W;
  float *base = grad + ((int64_t)q.b * C + c) * vol;
  for (int iz = 0; iz < q.gd; ++iz) {
    const float z = sample_coord(q.sd, pd, q.bd, iz, q.gd);
    for (int iy = 0; iy < q.gh; ++iy) {
      const float y = sample_coord(q.sh, ph, q.bh, iy, q.gh);
      for (int ix = 0; ix < q.gw; ++ix) {
        const float x = sample_coord(q.sw, pw, q.bw, ix, q.gw);
        int64_t off[8];
        float w[8];
        if (!corners(z, y, x, D, H, W, order, off, w)) continue;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (w[k] != 0.f) atomicAdd(base + off[k], g * w[k] / q.count);
      }
    }
  }
}

template <typename T>
int forward(const void *features, const void *rois, void *output, int N, int C, int D, int H, int W, int R, int PD,
            int PH, int PW, float scale, int sr, int order, hipStream_t st) {
  const T *f = static_cast<const T *>(features);
  const T *ro = static_cast<const T *>(rois);
  T *o = static_cast<T *>(output);
  const int cpt = C % 4 == 0 ? 4 : 1;
  const int64_t total = (int64_t)R * (C / cpt) * PD * PH * PW;
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (cpt == 4)
    hipLaunchKernelGGL((roi_align3d_forward_kernel<T, 4>), dim3(grid), dim3(256), 0, st, f, ro, o, N, C, D, H, W, R, PD,
                       PH, PW, scale, sr, order);
  else
    hipLaunchKernelGGL((roi_align3d_forward_kernel<T, 1>), dim3(grid), dim3(256), 0, st, f, ro, o, N, C, D, H, W, R, PD,
                       PH, PW, scale, sr, order);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

template <typename T>
int backward(const void *grad_output, const void *rois, void *grad_input, float *acc, int N, int C, int D, int H,
             int W, int R, int PD, int PH, int PW, float scale, int sr, int order, hipStream_t st) {
  const int64_t nin = (int64_t)N * C * D * H * W;
  const int64_t nout = (int64_t)R * C * PD * PH * PW;
  const int64_t fg = (nin + 255) / 256;
  const unsigned fill_grid = (unsigned)(fg < 65536 ? (fg > 0 ? fg : 1) : 65536);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(fill_grid), dim3(256), 0, st, acc, nin);
  if (nout > 0)
    hipLaunchKernelGGL((roi_align3d_backward_kernel<T>), dim3((unsigned)((nout + 255) / 256)), dim3(256), 0, st,
                       static_cast<const T *>(grad_output), static_cast<const T *>(rois), acc, N, C, D, H, W, R, PD, PH,
                       PW, scale, sr, order);
  if constexpr (!std::is_same<T, float>::value)
    hipLaunchKernelGGL((cast_kernel<T>), dim3(fill_grid), dim3(256), 0, st, acc, static_cast<T *>(grad_input), nin);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

bool valid(int dtype, int N, int C, int D, int H, int W, int R, int PD, int PH, int PW, int order) {
  return (dtype == OPS3D_FDA_F32 || dtype == OPS3D_FDA_F16 || dtype == OPS3D_FDA_BF16) && N >= 0 && C >= 0 &&
         D > 0 && H > 0 && W > 0 && R >= 0 && PD > 0 && PH > 0 && PW > 0 && (order == 0 || order == 1) &&
         (int64_t)N * C * D * H * W < ((int64_t)1 << 40);
}

}  // namespace ops3d_roi

using namespace ops3d_roi;

extern "C" {

int ops3d_roi_align3d_forward(const void *features, const void *rois, void *output, int dtype, int N, int C, int D,
                              int H, int W, int R, int PD, int PH, int PW, float spatial_scale, int sampling_ratio,
                              int order, void *stream) {
  if (!valid(dtype, N, C, D, H, W, R, PD, PH, PW, order)) return OPS3D_FDA_EINVAL;
  if ((int64_t)R * C == 0) return OPS3D_FDA_OK;
  if (!features || !rois || !output) return OPS3D_FDA_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case OPS3D_FDA_F32:
      return forward<float>(features, rois, output, N, C, D, H, W, R, PD, PH, PW, spatial_scale, sampling_ratio, order, st);
    case OPS3D_FDA_F16:
      return forward<__half>(features, rois, output, N, C, D, H, W, R, PD, PH, PW, spatial_scale, sampling_ratio, order, st);
    default:
      return forward<__hip_bfloat16>(features, rois, output, N, C, D, H, W, R, PD, PH, PW, spatial_scale, sampling_ratio,
                                     order, st);
  }
}

size_t ops3d_roi_align3d_backward_workspace_bytes(int dtype, int N, int C, int D, int H, int W) {
  if (dtype == OPS3D_FDA_F32 || N <= 0 || C <= 0 || D <= 0 || H <= 0 || W <= 0) return 0;
  return (size_t)N * C * D * H * W * sizeof(float);
}

int ops3d_roi_align3d_backward(const void *grad_output, const void *rois, void *grad_input, void *workspace,
                               size_t workspace_bytes, int dtype, int N, int C, int D, int H, int W, int R, int PD,
                               int PH, int PW, float spatial_scale, int sampling_ratio, int order, void *stream) {
  if (!valid(dtype, N, C, D, H, W, R, PD, PH, PW, order)) return OPS3D_FDA_EINVAL;
  if ((int64_t)N * C == 0) return OPS3D_FDA_OK;
  if (!grad_input || ((int64_t)R > 0 && (!grad_output || !rois))) return OPS3D_FDA_EINVAL;
  if (workspace_bytes < ops3d_roi_align3d_backward_workspace_bytes(dtype, N, C, D, H, W) ||
      (dtype != OPS3D_FDA_F32 && (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 3u))))
    return OPS3D_FDA_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case OPS3D_FDA_F32:
      return backward<float>(grad_output, rois, grad_input, static_cast<float *>(grad_input), N, C, D, H, W, R, PD, PH,
                             PW, spatial_scale, sampling_ratio, order, st);
    case OPS3D_FDA_F16:
      return backward<__half>(grad_output, rois, grad_input, static_cast<float *>(workspace), N, C, D, H, W, R, PD, PH,
                              PW, spatial_scale, sampling_ratio, order, st);
    default:
      return backward<__hip_bfloat16>(grad_output, rois, grad_input, static_cast<float *>(workspace), N, C, D, H, W, R,
                                      PD, PH, PW, spatial_scale, sampling_ratio, order, st);
  }
}

}  // extern "C"
