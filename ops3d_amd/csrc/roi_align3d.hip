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
// Forward: a gather, one thread per (roi, CPT = 4 channels, bin), or on channels-last features
// one lane per (bin, 8 channels) (the same bits).  With at most 2 samples per bin and axis it is
// separable: the bin's average is the sum over its distinct z, y and x taps (at most 4 each) of
// the per-axis weight sums times the value, fewer loads than 8 corners per sample; larger sample
// grids take the reference's per-sample loop.  Backward: the adjoint, as a gather when the
// output has at most 64 bins per axis and 384 in all (each voxel sums, in registers, the rois
// that reach it, in roi order: no atomics, the same bits on every run; the workspace holds the
// rois' axis weight tables and a channels-last copy of grad_output),
// otherwise by fp32 atomics into a channels-last workspace (64 lanes = 64 contiguous channels
// per atomic instruction) transposed into grad_input afterwards.  A roi whose batch index is
// outside [0, N) reads and writes nothing (its output is 0; the reference indexes out of
// bounds).
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

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

// The taps of one axis of a bin: up to NT distinct positions with their summed weights, in the
// order the samples first reach them (increasing position; weights of invalid samples and
// collapsed taps are left out); `over` when the samples reach more than NT positions.  Static
// register indices only (predicated), so nothing spills to scratch.
template <int NT>
struct AxisTaps {
  int n;
  bool over;
  int pos[NT];
  float w[NT];
  __device__ __forceinline__ void add(int p, float wt) {
    if (wt == 0.f) return;
    bool done = false;
#pragma unroll
    for (int k = 0; k < NT; ++k)
      if (!done && k < n && pos[k] == p) {
        w[k] += wt;
        done = true;
      }
    if (!done) {
      if (n == NT) {
        over = true;
        return;
      }
#pragma unroll
      for (int k = 0; k < NT; ++k)
        if (k == n) {
          pos[k] = p;
          w[k] = wt;
        }
      ++n;
    }
  }
  // drop the first tap (register moves, so a loop over the taps needs no dynamic index)
  __device__ __forceinline__ void shift() {
#pragma unroll
    for (int k = 0; k + 1 < NT; ++k) {
      pos[k] = pos[k + 1];
      w[k] = w[k + 1];
    }
    --n;
  }
};
using AxisTaps4 = AxisTaps<4>;
using AxisTaps8 = AxisTaps<8>;
// Grids of more than 2 samples per axis take the separable sum when every axis of the bin has
// at most kSepTaps distinct taps, the per-sample loop otherwise.
constexpr int kSepTaps = 8;

__device__ __forceinline__ AxisTaps4 bin_taps(float start, int p, float bin, int grid, int size, int order);
template <int NT>
__device__ __forceinline__ AxisTaps<NT> bin_taps_n(float start, int p, float bin, int grid, int size, int order);

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
  if (inb && q.gd <= 2 && q.gh <= 2 && q.gw <= 2) {
    // separable: the bin's average is sum over its distinct z, y, x taps of WZ * WY * WX * value
    // (the samples form a full grid and the corner weights are products, so the per-axis weight
    // sums factor), at most 4 taps per axis instead of 8 corners per sample
    const AxisTaps4 tz = bin_taps(q.sd, pd, q.bd, q.gd, D, order);
    const AxisTaps4 ty = bin_taps(q.sh, ph, q.bh, q.gh, H, order);
    const AxisTaps4 tx = bin_taps(q.sw, pw, q.bw, q.gw, W, order);
#pragma unroll
    for (int kz = 0; kz < 4; ++kz) {
      if (kz >= tz.n) break;
#pragma unroll
      for (int ky = 0; ky < 4; ++ky) {
        if (ky >= ty.n) break;
        const float wzy = tz.w[kz] * ty.w[ky];
        const int64_t rowo = ((int64_t)tz.pos[kz] * H + ty.pos[ky]) * W;
#pragma unroll
        for (int kx = 0; kx < 4; ++kx) {
          if (kx >= tx.n) break;
          const float wgt = wzy * tx.w[kx];
#pragma unroll
          for (int c = 0; c < CPT; ++c) acc[c] = acc[c] + wgt * to_f(base[(int64_t)c * vol + rowo + tx.pos[kx]]);
        }
      }
    }
  }
  bool wide = inb && (q.gd > 2 || q.gh > 2 || q.gw > 2);
  if (wide) {
    // larger grids: separable too when every axis has at most kSepTaps distinct taps (the same
    // loop over taps, z and y taps consumed by shifting the lists)
    AxisTaps8 tz = bin_taps_n<kSepTaps>(q.sd, pd, q.bd, q.gd, D, order);
    AxisTaps8 ty = bin_taps_n<kSepTaps>(q.sh, ph, q.bh, q.gh, H, order);
    const AxisTaps8 tx = bin_taps_n<kSepTaps>(q.sw, pw, q.bw, q.gw, W, order);
    if (!tz.over && !ty.over && !tx.over) {
      wide = false;
      for (; tz.n > 0; tz.shift()) {
        AxisTaps8 tyc = ty;
        for (; tyc.n > 0; tyc.shift()) {
          const float wzy = tz.w[0] * tyc.w[0];
          const int64_t rowo = ((int64_t)tz.pos[0] * H + tyc.pos[0]) * W;
#pragma unroll
          for (int kx = 0; kx < kSepTaps; ++kx) {
            if (kx >= tx.n) break;
            const float wgt = wzy * tx.w[kx];
#pragma unroll
            for (int c = 0; c < CPT; ++c) acc[c] = acc[c] + wgt * to_f(base[(int64_t)c * vol + rowo + tx.pos[kx]]);
          }
        }
      }
    }
  }
  for (int iz = 0; wide && iz < q.gd; ++iz) {
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

// Channels-last fp32 [N, V, C] -> [N, C, V] in T, through a 64 x 64 LDS tile (padded rows: the
// column reads are conflict-free).  grid (ceil(V/64), ceil(C/64), N), 256 threads.
template <typename T>
__global__ __launch_bounds__(256) void channels_last_to_ncdhw_kernel(const float *src, T *dst, int C, int64_t V) {
  __shared__ float t[64][65];
  const int tid = threadIdx.x, lane = tid & 63, row = tid >> 6;
  const int64_t v0 = (int64_t)blockIdx.x * 64;
  const int c0 = blockIdx.y * 64;
  const int64_t n = blockIdx.z;
  const float *s = src + n * V * C;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int vv = i * 4 + row;
    if (v0 + vv < V && c0 + lane < C) t[vv][lane] = s[(v0 + vv) * C + c0 + lane];
  }
  __syncthreads();
  T *d = dst + n * C * V;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int cc = i * 4 + row;
    if (c0 + cc < C && v0 + lane < V) d[(int64_t)(c0 + cc) * V + v0 + lane] = from_f<T>(t[lane][cc]);
  }
}

// One axis of a sample's interpolation, with the edge rules of corners(): valid unless beyond
// [-1, size]; below 0 clamps to 0; a base at size - 1 collapses both taps onto it (weights 1, 0).
// Order 0 keeps the nearest tap (the low one when its weight is >= 0.5), weight 1.  corners()'s
// eight weights are the products of the three axes' (its nearest-corner rule picks, axis by
// axis, the low tap whenever allowed, so it is this per-axis choice too).
struct AxisTap {
  bool ok;
  int i0, i1;
  float w0, w1;
};
__device__ __forceinline__ AxisTap axis_tap(float c, int size, int order) {
#pragma clang fp contract(off)
  AxisTap t;
  t.ok = !(c < -1.f || c > (float)size);
  if (c <= 0.f) c = 0.f;
  t.i0 = (int)c;
  if (t.i0 >= size - 1) {
    t.i1 = t.i0 = size - 1;
    c = (float)t.i0;
  } else {
    t.i1 = t.i0 + 1;
  }
  const float l = c - (float)t.i0, h = 1.f - l;
  if (order == 0) {
    t.w0 = h >= 0.5f ? 1.f : 0.f;
    t.w1 = h >= 0.5f ? 0.f : 1.f;
  } else {
    t.w0 = h;
    t.w1 = l;
  }
  return t;
}

// The taps of bin p on one axis (grid <= 2 samples), merged by position.
__device__ __forceinline__ AxisTaps4 bin_taps(float start, int p, float bin, int grid, int size, int order) {
  AxisTaps4 t;
  t.n = 0;
  t.over = false;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    t.pos[k] = 0;
    t.w[k] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (i >= grid) break;
    const AxisTap a = axis_tap(sample_coord(start, p, bin, i, grid), size, order);
    if (!a.ok) continue;
    t.add(a.i0, a.w0);
    if (a.i1 != a.i0) t.add(a.i1, a.w1);
  }
  return t;
}

// The taps of bin p on one axis for any grid, up to NT of them (t.over beyond that).
template <int NT>
__device__ __forceinline__ AxisTaps<NT> bin_taps_n(float start, int p, float bin, int grid, int size, int order) {
  AxisTaps<NT> t;
  t.n = 0;
  t.over = false;
#pragma unroll
  for (int k = 0; k < NT; ++k) {
    t.pos[k] = 0;
    t.w[k] = 0.f;
  }
  for (int i = 0; i < grid && !t.over; ++i) {
    const AxisTap a = axis_tap(sample_coord(start, p, bin, i, grid), size, order);
    if (!a.ok) continue;
    t.add(a.i0, a.w0);
    if (a.i1 != a.i0) t.add(a.i1, a.w1);
  }
  return t;
}

// Sum of the valid samples' weights on tap position `pos` of one axis (sample i at
// sample_coord(start, p, bin, i, grid)).
__device__ __forceinline__ float axis_weight_at(int pos, float start, int p, float bin, int grid, int size, int order) {
  float s = 0.f;
  for (int i = 0; i < grid; ++i) {
    const AxisTap t = axis_tap(sample_coord(start, p, bin, i, grid), size, order);
    if (!t.ok) continue;
    if (t.i0 == pos) s += t.w0;
    if (t.i1 == pos && t.i1 != t.i0) s += t.w1;
  }
  return s;
}

// Backward: one wave per (roi, 64 channels, output row (pd, ph)); lane = channel.  The weights
// are separable, so the row's contribution to voxel (z, y, x) is WZ[z] * WY[y] * X[x], with WZ
// and WY the row's summed z and y tap weights and X[x] = sum over the row's x samples of
// top[bin] * wx / count.  The wave walks the x samples in increasing x (they are sorted), keeps
// the running X of the two newest tap positions per lane and, once the walk has passed a
// position, adds WZ * WY * X to every (z, y) tap of it with one atomic instruction each: 64
// contiguous channels of the channels-last workspace.  Every voxel a row touches thus gets one
// atomic per (row, 64 channels) instead of one per sample corner.  WZ / WY sit in lanes
// (lane t: tap position min + t); rows with more than 64 tap positions on an axis (adaptive
// grids of huge bins) take the per-sample path.
constexpr int kBwdWaves = 4;
template <typename T>
__global__ __launch_bounds__(64 * kBwdWaves) void roi_align3d_backward_kernel(const T *top, const T *rois, float *acc,
                                                                            int N, int C, int D, int H, int W, int R,
                                                                            int PD, int PH, int PW, float scale, int sr,
                                                                            int order) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int CG = (C + 63) / 64;
  const int64_t wid = (int64_t)blockIdx.x * kBwdWaves + (threadIdx.x >> 6);
  if (wid >= (int64_t)R * CG * PD * PH) return;   // whole waves
  const int ph = (int)(wid % PH), pd = (int)((wid / PH) % PD);
  const int cg = (int)((wid / ((int64_t)PH * PD)) % CG);
  const int r = (int)(wid / ((int64_t)PH * PD * CG));
  const int c = cg * 64 + lane;
  const bool active = c < C;
  const Roi q = roi_setup(rois, r, scale, sr, PD, PH, PW);
  if (q.b < 0 || q.b >= N) return;   // a roi of a batch item that does not exist
  const int64_t vol = (int64_t)D * H * W;
  float *base = acc + (int64_t)q.b * vol * C + c;
  const T *tg = top + (((int64_t)r * C + (active ? c : 0)) * PD + pd) * PH * PW + (int64_t)ph * PW;
  // tap ranges of the row's z and y samples (coordinates increase with the sample index)
  int z_lo = 1 << 30, z_hi = -1, y_lo = 1 << 30, y_hi = -1;
  for (int i = 0; i < q.gd; ++i) {
    const AxisTap t = axis_tap(sample_coord(q.sd, pd, q.bd, i, q.gd), D, order);
    if (t.ok) { z_lo = min(z_lo, t.i0); z_hi = max(z_hi, t.i1); }
  }
  for (int i = 0; i < q.gh; ++i) {
    const AxisTap t = axis_tap(sample_coord(q.sh, ph, q.bh, i, q.gh), H, order);
    if (t.ok) { y_lo = min(y_lo, t.i0); y_hi = max(y_hi, t.i1); }
  }
  if (z_hi < 0 || y_hi < 0) return;   // no valid sample in z or y: the row adds nothing
  const int nz = z_hi - z_lo + 1, ny = y_hi - y_lo + 1;
  if (nz <= 64 && ny <= 64) {
    const float wz_l = lane < nz ? axis_weight_at(z_lo + lane, q.sd, pd, q.bd, q.gd, D, order) : 0.f;
    const float wy_l = lane < ny ? axis_weight_at(y_lo + lane, q.sh, ph, q.bh, q.gh, H, order) : 0.f;
    // X of the tap position px (a0) and px + 1 (a1); `open`: px holds a position
    int px = 0;
    bool open = false, used1 = false;
    float a0 = 0.f, a1 = 0.f;
    const auto flush = [&](int x, float v) {
      const float vc = v / q.count;
      for (int tz = 0; tz < nz; ++tz) {
        const float wz = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wz_l), tz));
        if (wz == 0.f) continue;
        for (int ty = 0; ty < ny; ++ty) {
          const float wy = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wy_l), ty));
          if (wy == 0.f) continue;
          if (active) atomicAdd(base + (((int64_t)(z_lo + tz) * H + (y_lo + ty)) * W + x) * C, (wz * wy) * vc);
        }
      }
    };
    for (int pw = 0; pw < PW; ++pw) {
      const float g = active ? to_f(tg[pw]) : 0.f;
      for (int ix = 0; ix < q.gw; ++ix) {
        const AxisTap t = axis_tap(sample_coord(q.sw, pw, q.bw, ix, q.gw), W, order);
        if (!t.ok) continue;
        if (!open) {
          px = t.i0;
          open = true;
        } else if (t.i0 == px + 1) {
          flush(px, a0);
          px = t.i0;
          a0 = a1;
          a1 = 0.f;
          used1 = false;
        } else if (t.i0 > px + 1) {
          flush(px, a0);
          if (used1) flush(px + 1, a1);
          px = t.i0;
          a0 = a1 = 0.f;
          used1 = false;
        }
        a0 += g * t.w0;
        if (t.i1 != t.i0) {
          a1 += g * t.w1;
          used1 = true;
        }
      }
    }
    if (open) {
      flush(px, a0);
      if (used1) flush(px + 1, a1);
    }
    return;
  }
  // per-sample path: the 8 corners of each sample, top * w / count each
  for (int pw = 0; pw < PW; ++pw) {
    const float g = active ? to_f(tg[pw]) : 0.f;
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
            if (w[k] != 0.f && active) atomicAdd(base + off[k] * C, g * w[k] / q.count);
        }
      }
    }
  }
}

// Backward as a gather (no atomics): a block owns a tile of 4 x 8 x 8 voxels of one batch item
// (a thread per voxel) and 16 channels, and sums into registers the contributions of every roi
// whose footprint reaches the tile, rois in index order, so the result is the same on every run.
// The weights are separable: voxel (z, y, x) gets, from roi r, the sum over bins (pd, ph, pw) of
// WZ[z][pd] * WY[y][ph] * WX[x][pw] * top[r, c, pd, ph, pw] / count, where WZ[z][pd] is the sum of
// bin pd's z-sample tap weights on z (and so on) -- the sum over the bin's samples of their
// corner weights.  The block takes its rois in groups, so that one round trip to memory serves
// several rois: for up to 8 rois it finds the bins that reach the tile on each axis (a thread
// per (roi, tile position, bin)), keeps the longest prefix whose bin boxes and weight tables fit
// the LDS arenas, writes their tables and stages top for their boxes and its 16 channels as
// fp32, and each thread then walks, roi by roi, the nonzero bins of its voxel.  Needs at most 64
// bins per axis and 384 in all (else the atomic path below is used).
constexpr int kGTZ = 4, kGTY = 8, kGTX = 8;   // tile: 256 voxels, a thread each
constexpr int kGPos = kGTZ + kGTY + kGTX;      // tile positions over the three axes
constexpr int kGCC = 16;                       // channels per block (registers per thread)
constexpr int kGMaxAxisBins = 64, kGMaxBins = 384;
constexpr int kGGroup = 8;                     // rois examined per group
constexpr int kGTab = 2048;                    // weight-table arena (floats)
constexpr int kGList = 128;                    // rois per compaction batch

__host__ __device__ inline bool gather_fits(int PD, int PH, int PW) {
  return PD <= kGMaxAxisBins && PH <= kGMaxAxisBins && PW <= kGMaxAxisBins && PD * PH * PW <= kGMaxBins;
}

// Whether a roi's taps on one axis can reach [t0, t0 + T): its samples lie in [start, end]
// (coordinates), their taps in [floor(max(start, 0)), floor(max(end, 0)) + 1], none if
// start > size.
__device__ __forceinline__ bool axis_reaches(float start, float end, int size, int t0, int T) {
  if (start > (float)size) return false;
  const float lo = floorf(fmaxf(start, 0.f)), hi = floorf(fmaxf(end, 0.f)) + 1.f;
  return !(hi < (float)t0 || lo > (float)(t0 + T - 1));
}

// A roi's parameters in LDS (the Roi fields the gather needs).
struct GatherRoi {
  float s[3], bin[3], inv_count;   // z, y, x
  int grid[3];
};
// Bin ranges of one roi of a group: [first, last] bin reaching the tile per axis, and per tile
// position (z positions, then y, then x).
struct GatherRanges {
  int box[3][2];
  int pos[kGPos][2];
};
constexpr int kGRangeInts = (int)(sizeof(GatherRanges) / sizeof(int));

// Per-roi axis tables of the gather backward, made once per call instead of in every tile block
// that the roi reaches (each of them recomputed them per 16-channel block): for roi r and axis a
// (size S_a, P_a bins), wt[r][a][x][p] = axis_weight_at(x, .., p, ..) for every position x of
// the axis, and ft[r][a][x] = the first and last bin with a nonzero weight at x (low and high
// 16 bits; first > last when none).  The gather kernel reads the same values it computed before.
// Layout per roi: floats D*PD (z), H*PH (y), W*PW (x); ints D, H, W.
template <typename T>
__global__ __launch_bounds__(256) void roi_axis_table_kernel(const T *rois, float *wt, uint32_t *ft, int D, int H,
                                                             int W, int PD, int PH, int PW, float scale, int sr,
                                                             int order) {
  const int r = blockIdx.x, ax = blockIdx.y;
  const Roi q = roi_setup(rois, r, scale, sr, PD, PH, PW);
  const int S = ax == 0 ? D : (ax == 1 ? H : W), P = ax == 0 ? PD : (ax == 1 ? PH : PW);
  const float st = ax == 0 ? q.sd : (ax == 1 ? q.sh : q.sw), bn = ax == 0 ? q.bd : (ax == 1 ? q.bh : q.bw);
  const int gr = ax == 0 ? q.gd : (ax == 1 ? q.gh : q.gw);
  const size_t wofs = (size_t)r * ((size_t)D * PD + (size_t)H * PH + (size_t)W * PW) +
                      (ax == 0 ? 0 : (ax == 1 ? (size_t)D * PD : (size_t)D * PD + (size_t)H * PH));
  const size_t fofs = (size_t)r * ((size_t)D + H + W) + (ax == 0 ? 0 : (ax == 1 ? (size_t)D : (size_t)D + H));
  for (int x = threadIdx.x; x < S; x += 256) {
    uint32_t first = 0xffffu, last = 0u;
    for (int p = 0; p < P; ++p) {
      const float w = axis_weight_at(x, st, p, bn, gr, S, order);
      wt[wofs + (size_t)x * P + p] = w;
      if (w != 0.f) {
        first = min(first, (uint32_t)p);
        last = (uint32_t)p;
      }
    }
    ft[fofs + x] = first | (last << 16);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void roi_align3d_backward_gather_kernel(const T *top_cl, const T *rois, T *grad,
                                                                          const float *wt, const uint32_t *ft, bool vec4,
                                                                          int N,
                                                                          int C, int D, int H, int W, int R, int PD,
                                                                          int PH, int PW, float scale, int sr,
                                                                          int order) {
#pragma clang fp contract(off)
  __shared__ float4 g_l[kGCC / 4][kGMaxBins];   // [channel quad][bin of the group's boxes]
  __shared__ float tab_l[kGTab];                // the group's weight tables
  __shared__ GatherRoi roi_l[kGList];
  __shared__ int rid_l[kGList];
  __shared__ GatherRanges rng_l[kGGroup];
  __shared__ int goff_l[kGGroup + 1][2];         // per group roi: first bin, first table entry
  __shared__ int cnt_l[4], gsize_l;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int ntx = (W + kGTX - 1) / kGTX, nty = (H + kGTY - 1) / kGTY, ntz = (D + kGTZ - 1) / kGTZ;
  const int ncc = (C + kGCC - 1) / kGCC;
  int64_t bid = blockIdx.x;
  const int txi = (int)(bid % ntx);
  bid /= ntx;
  const int tyi = (int)(bid % nty);
  bid /= nty;
  const int tzi = (int)(bid % ntz);
  bid /= ntz;
  const int cc = (int)(bid % ncc), n = (int)(bid / ncc);
  const int t0[3] = {tzi * kGTZ, tyi * kGTY, txi * kGTX};
  const int c0 = cc * kGCC;
  const int zl = tid / (kGTY * kGTX), yl = (tid / kGTX) % kGTY, xl = tid % kGTX;
  const int S[3] = {D, H, W}, TT[3] = {kGTZ, kGTY, kGTX};
  const int pos0[3] = {0, kGTZ, kGTZ + kGTY};     // first position of each axis in the ranges
  const int64_t pvol = (int64_t)PD * PH * PW;
  const size_t wroi = (size_t)D * PD + (size_t)H * PH + (size_t)W * PW, froi = (size_t)D + H + W;
  const size_t wax[3] = {0, (size_t)D * PD, (size_t)D * PD + (size_t)H * PH}, fax[3] = {0, (size_t)D, (size_t)D + H};
  const int PA[3] = {PD, PH, PW};

  float acc[kGCC];
#pragma unroll
  for (int k = 0; k < kGCC; ++k) acc[k] = 0.f;
  for (int rb = 0; rb < R; rb += kGList) {
    // the rois of batch item n whose taps can reach the tile, in index order, with their
    // parameters in LDS
    const int r = rb + tid;
    bool hit = false;
    Roi q;
    if (tid < kGList && r < R) {
      q = roi_setup(rois, r, scale, sr, PD, PH, PW);
      hit = q.b == n && axis_reaches(q.sd, q.sd + q.bd * (float)PD, D, t0[0], kGTZ) &&
            axis_reaches(q.sh, q.sh + q.bh * (float)PH, H, t0[1], kGTY) &&
            axis_reaches(q.sw, q.sw + q.bw * (float)PW, W, t0[2], kGTX);
    }
    const uint64_t m = __ballot(hit);
    if (lane == 0) cnt_l[wv] = __popcll(m);
    __syncthreads();
    int off = 0, tot = 0;
    for (int w = 0; w < 4; ++w) {
      off += w < wv ? cnt_l[w] : 0;
      tot += cnt_l[w];
    }
    if (hit) {
      const int i = off + __popcll(m & ((1ull << lane) - 1ull));
      rid_l[i] = r;
      GatherRoi g;
      g.s[0] = q.sd, g.s[1] = q.sh, g.s[2] = q.sw;
      g.bin[0] = q.bd, g.bin[1] = q.bh, g.bin[2] = q.bw;
      g.grid[0] = q.gd, g.grid[1] = q.gh, g.grid[2] = q.gw;
      g.inv_count = 1.f / q.count;
      roi_l[i] = g;
    }
    for (int li = 0; li < tot;) {
      const int gmax = min(kGGroup, tot - li);
      for (int i = tid; i < kGGroup * kGRangeInts; i += 256)
        reinterpret_cast<int *>(rng_l)[i] = (i & 1) ? -1 : (1 << 30);
      __syncthreads();   // (also: the previous group's sums are done with the LDS state)
      // 1. bin ranges of the next gmax rois, from the axis tables: a thread per (roi, position)
      for (int e = tid; e < gmax * kGPos; e += 256) {
        const int w = e / kGPos, k = e - w * kGPos;
        const int ax = k < kGTZ ? 0 : (k < kGTZ + kGTY ? 1 : 2), pos = k - pos0[ax];
        const int at = t0[ax] + pos;
        if (at < S[ax]) {
          const uint32_t fl = ft[(size_t)rid_l[li + w] * froi + fax[ax] + at];
          const int first = (int)(fl & 0xffffu), last = (int)(fl >> 16);
          if (first <= last) {
            atomicMin(&rng_l[w].box[ax][0], first);
            atomicMax(&rng_l[w].box[ax][1], last);
            rng_l[w].pos[k][0] = first;
            rng_l[w].pos[k][1] = last;
          }
        }
      }
      __syncthreads();
      // 2. the group: the longest prefix whose boxes and tables fit (at least one roi)
      if (tid == 0) {
        int nbin = 0, ntab = 0, gs = 0;
        for (; gs < gmax; ++gs) {
          const GatherRanges &rg = rng_l[gs];
          int b = 1, t = 0;
          for (int ax = 0; ax < 3; ++ax) {
            const int nb = rg.box[ax][1] < 0 ? 0 : rg.box[ax][1] - rg.box[ax][0] + 1;
            b *= nb;
            t += TT[ax] * nb;
          }
          if (b == 0) t = 0;   // reaches nothing: no table, no bins
          if (gs > 0 && (nbin + b > kGMaxBins || ntab + t > kGTab)) break;
          goff_l[gs][0] = nbin;
          goff_l[gs][1] = ntab;
          nbin += b;
          ntab += t;
        }
        goff_l[gs][0] = nbin;
        goff_l[gs][1] = ntab;
        gsize_l = gs;
      }
      __syncthreads();
      const int gs = gsize_l;
      // 3. the group's tables (weights of the box bins at the tile positions) ...
      const int ntab = goff_l[gs][1], nbin = goff_l[gs][0];
      for (int e = tid; e < ntab; e += 256) {
        int w = 0;
        while (goff_l[w + 1][1] <= e) ++w;
        const GatherRanges &rg = rng_l[w];
        int f = e - goff_l[w][1], ax = 0;
        for (; ax < 2; ++ax) {
          const int sz = TT[ax] * (rg.box[ax][1] - rg.box[ax][0] + 1);
          if (f < sz) break;
          f -= sz;
        }
        const int nb = rg.box[ax][1] - rg.box[ax][0] + 1;
        const int pos = f / nb, p = rg.box[ax][0] + (f - pos * nb);
        const int at = t0[ax] + pos;
        tab_l[e] = at < S[ax] ? wt[(size_t)rid_l[li + w] * wroi + wax[ax] + (size_t)at * PA[ax] + p] : 0.f;
      }
      // ... and top for their boxes of bins and the block's channels, as fp32, from the
      // channels-last copy [R, bins, C] (consecutive threads on consecutive channel quads of one
      // bin: the block's 16 channels of a bin are one contiguous run)
      for (int e = tid; e < nbin * (kGCC / 4); e += 256) {
        const int gb = e / (kGCC / 4), k4 = e - gb * (kGCC / 4);
        int w = 0;
        while (goff_l[w + 1][0] <= gb) ++w;
        const GatherRanges &rg = rng_l[w];
        const int lb = gb - goff_l[w][0];
        const int nby = rg.box[1][1] - rg.box[1][0] + 1, nbx = rg.box[2][1] - rg.box[2][0] + 1;
        const int bx = lb % nbx, bzy = lb / nbx, by = bzy % nby, bz = bzy / nby;
        const int c = c0 + 4 * k4;
        const T *src = top_cl + ((int64_t)rid_l[li + w] * pvol +
                                 ((int64_t)(rg.box[0][0] + bz) * PH + rg.box[1][0] + by) * PW + rg.box[2][0] + bx) *
                                    C + c;
        float4 v;
        if (vec4 && c < C) {   // 4 channels, one 8- or 16-byte load
          float f[4];
          if constexpr (sizeof(T) == 4) {
            const float4 u = *reinterpret_cast<const float4 *>(src);
            f[0] = u.x; f[1] = u.y; f[2] = u.z; f[3] = u.w;
          } else {
            const uint2 u = *reinterpret_cast<const uint2 *>(src);
            const uint32_t wd[2] = {u.x, u.y};
#pragma unroll
            for (int k = 0; k < 4; ++k)
              f[k] = to_f(__builtin_bit_cast(T, (unsigned short)((k & 1) ? (wd[k >> 1] >> 16) : (wd[k >> 1] & 0xffffu))));
          }
          v = make_float4(f[0], f[1], f[2], f[3]);
        } else {
          v.x = c + 0 < C ? to_f(src[0]) : 0.f;
          v.y = c + 1 < C ? to_f(src[1]) : 0.f;
          v.z = c + 2 < C ? to_f(src[2]) : 0.f;
          v.w = c + 3 < C ? to_f(src[3]) : 0.f;
        }
        g_l[k4][gb] = v;
      }
      __syncthreads();
      // 4. this voxel's sums, roi by roi: its bins are a contiguous range per axis
      for (int w = 0; w < gs; ++w) {
        const GatherRanges &rg = rng_l[w];
        if (rg.box[0][1] < 0 || rg.box[1][1] < 0 || rg.box[2][1] < 0) continue;
        const int pz0 = rg.box[0][0], py0 = rg.box[1][0], px0 = rg.box[2][0];
        const int nbz = rg.box[0][1] - pz0 + 1, nby = rg.box[1][1] - py0 + 1, nbx = rg.box[2][1] - px0 + 1;
        const float *tz = tab_l + goff_l[w][1] + zl * nbz - pz0;
        const float *ty = tab_l + goff_l[w][1] + kGTZ * nbz + yl * nby - py0;
        const float *tx = tab_l + goff_l[w][1] + kGTZ * nbz + kGTY * nby + xl * nbx - px0;
        const int gb0 = goff_l[w][0];
        const float inv_count = roi_l[li + w].inv_count;
        const int qz0 = rg.pos[zl][0], qz1 = rg.pos[zl][1];
        const int qy0 = rg.pos[kGTZ + yl][0], qy1 = rg.pos[kGTZ + yl][1];
        const int qx0 = rg.pos[kGTZ + kGTY + xl][0], qx1 = rg.pos[kGTZ + kGTY + xl][1];
        for (int pz = qz0; pz <= qz1; ++pz) {
          const float wz = tz[pz] * inv_count;
          for (int py = qy0; py <= qy1; ++py) {
            const float wzy = wz * ty[py];
            const int lrow = gb0 + ((pz - pz0) * nby + (py - py0)) * nbx - px0;
            for (int px = qx0; px <= qx1; ++px) {
              const float wgt = wzy * tx[px];
#pragma unroll
              for (int k4 = 0; k4 < kGCC / 4; ++k4) {
                const float4 gv = g_l[k4][lrow + px];
                acc[4 * k4 + 0] += wgt * gv.x;
                acc[4 * k4 + 1] += wgt * gv.y;
                acc[4 * k4 + 2] += wgt * gv.z;
                acc[4 * k4 + 3] += wgt * gv.w;
              }
            }
          }
        }
      }
      li += gs;
      __syncthreads();   // the sums are done with the group's LDS state
    }
    __syncthreads();   // the batch's counts are read before the next batch writes them
  }
  const int z = t0[0] + zl, y = t0[1] + yl, x = t0[2] + xl;
  if (z < D && y < H && x < W) {
    const int64_t vol = (int64_t)D * H * W, v = ((int64_t)z * H + y) * W + x;
#pragma unroll
    for (int k = 0; k < kGCC; ++k)
      if (c0 + k < C) grad[((int64_t)n * C + c0 + k) * vol + v] = from_f<T>(acc[k]);
  }
}

// ---------------------------------------------------------------------------------------------
// Channels-last forward.  With features [N, D, H, W, C] a voxel's C channels are one contiguous
// row, so a sample's corner is one 16-byte (8-channel) load per lane and the 32 lanes of a
// 256-channel bin read whole 128-byte lines; from [N, C, D, H, W] every corner of every channel
// is a separate 2- or 4-byte access.  A block owns bpb consecutive bins of the (ph, pw) plane
// of one (roi, pd): lane group cg takes channels 8 cg .. 8 cg + 7 of one bin, the rounded
// results are staged in LDS and written out as [R, C, PD, PH, PW] runs of bpb elements per
// channel.  The blocks of a roi run on one XCD, whose L2 then serves the overlap of their taps.
// The arithmetic is the NCDHW kernel's, term by term, so both give the same bits.
constexpr int kClChannels = 8;                  // channels per lane

template <typename T>
__device__ __forceinline__ void load8(const T *p, float f[8]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const unsigned short s = (unsigned short)((k & 1) ? (w[k >> 1] >> 16) : (w[k >> 1] & 0xffffu));
      f[k] = to_f(__builtin_bit_cast(T, s));
    }
  }
}

// Bins per block: one per lane group (256 / (C / 8) groups), the (ph, pw) plane of a (roi, pd)
// cut into equal parts.  One bin per thread measured fastest (more blocks in flight; bench
// workload, rows of 7 bins: 1, 2, 7 rows per block 415, 453, 448 us).
inline void cl_split(int C, int PHW, int &bpb, int &parts) {
  const int slots = 256 / (C / kClChannels);
  parts = (PHW + slots - 1) / slots;
  bpb = (PHW + parts - 1) / parts;
}

inline bool cl_supported(int C) { return C > 0 && C % kClChannels == 0 && C / kClChannels <= 256; }

// WIDE: compiled with the separable path for grids of more than 2 samples per axis (launched
// when sampling_ratio is adaptive or above 2; without it the kernel needs fewer registers).
template <typename T, bool WIDE>
__global__ __launch_bounds__(256) void roi_align3d_forward_cl_kernel(const T *feat, const T *rois, T *out, int N, int C,
                                                                     int D, int H, int W, int PD, int PH, int PW,
                                                                     float scale, int sr, int order, int bpb, int parts,
                                                                     int nblk) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char cl_lds[];
  T *res = reinterpret_cast<T *>(cl_lds);   // [C][bpb]
  // block i runs on XCD i % 8: XCD x takes the x-th eighth of the (roi, pd, part) blocks, so a
  // roi's blocks share one L2 (gridDim.x is a multiple of 8; nblk blocks are real)
  const unsigned blk = (blockIdx.x & 7u) * (gridDim.x / 8u) + (blockIdx.x >> 3);
  if (blk >= (unsigned)nblk) return;
  const int r = (int)(blk / (unsigned)(PD * parts));
  const int rem = (int)(blk % (unsigned)(PD * parts));
  const int pd = rem / parts, b0 = (rem - pd * parts) * bpb;
  const int nbin = min(bpb, PH * PW - b0);
  const int CG = C / kClChannels, slots = 256 / CG;
  const int tid = threadIdx.x, cg = tid % CG, slot = tid / CG;
  const Roi q = roi_setup(rois, r, scale, sr, PD, PH, PW);
  const bool inb = q.b >= 0 && q.b < N;
  const int64_t vol = (int64_t)D * H * W;
  const T *base = feat + (int64_t)(inb ? q.b : 0) * vol * C + cg * kClChannels;
  const bool sep = q.gd <= 2 && q.gh <= 2 && q.gw <= 2;
  AxisTaps4 tz;
  if (inb && sep) tz = bin_taps(q.sd, pd, q.bd, q.gd, D, order);
  AxisTaps8 tz8;   // larger grids: the z taps of plane pd, if they fit
  tz8.over = true;
  if (WIDE && inb && !sep) tz8 = bin_taps_n<kSepTaps>(q.sd, pd, q.bd, q.gd, D, order);
  for (int bin = slot; slot < slots && bin < nbin; bin += slots) {
    const int ph = (b0 + bin) / PW, pw = (b0 + bin) % PW;
    float acc[kClChannels];
#pragma unroll
    for (int c = 0; c < kClChannels; ++c) acc[c] = 0.f;
    if (inb && sep) {
      const AxisTaps4 ty = bin_taps(q.sh, ph, q.bh, q.gh, H, order);
      const AxisTaps4 tx = bin_taps(q.sw, pw, q.bw, q.gw, W, order);
#pragma unroll
      for (int kz = 0; kz < 4; ++kz) {
        if (kz >= tz.n) break;
#pragma unroll
        for (int ky = 0; ky < 4; ++ky) {
          if (ky >= ty.n) break;
          const float wzy = tz.w[kz] * ty.w[ky];
          const uint32_t rowo = ((uint32_t)tz.pos[kz] * (uint32_t)H + (uint32_t)ty.pos[ky]) * (uint32_t)W;
#pragma unroll
          for (int kx = 0; kx < 4; ++kx) {
            if (kx >= tx.n) break;
            const float wgt = wzy * tx.w[kx];
            float v[kClChannels];
            load8(base + (rowo + (uint32_t)tx.pos[kx]) * (uint32_t)C, v);
#pragma unroll
            for (int c = 0; c < kClChannels; ++c) acc[c] = acc[c] + wgt * v[c];
          }
        }
      }
    }
    bool wide = inb && !sep;
    if (WIDE && wide && !tz8.over) {
      // separable too when every axis has at most kSepTaps taps (the NCDHW kernel's loop)
      AxisTaps8 ty = bin_taps_n<kSepTaps>(q.sh, ph, q.bh, q.gh, H, order);
      const AxisTaps8 tx = bin_taps_n<kSepTaps>(q.sw, pw, q.bw, q.gw, W, order);
      if (!ty.over && !tx.over) {
        wide = false;
        for (AxisTaps8 tzc = tz8; tzc.n > 0; tzc.shift()) {
          for (AxisTaps8 tyc = ty; tyc.n > 0; tyc.shift()) {
            const float wzy = tzc.w[0] * tyc.w[0];
            const uint32_t rowo = ((uint32_t)tzc.pos[0] * (uint32_t)H + (uint32_t)tyc.pos[0]) * (uint32_t)W;
#pragma unroll
            for (int kx = 0; kx < kSepTaps; ++kx) {
              if (kx >= tx.n) break;
              const float wgt = wzy * tx.w[kx];
              float v[kClChannels];
              load8(base + (rowo + (uint32_t)tx.pos[kx]) * (uint32_t)C, v);
#pragma unroll
              for (int c = 0; c < kClChannels; ++c) acc[c] = acc[c] + wgt * v[c];
            }
          }
        }
      }
    }
    for (int iz = 0; wide && iz < q.gd; ++iz) {
      const float z = sample_coord(q.sd, pd, q.bd, iz, q.gd);
      for (int iy = 0; iy < q.gh; ++iy) {
        const float y = sample_coord(q.sh, ph, q.bh, iy, q.gh);
        for (int ix = 0; ix < q.gw; ++ix) {
          const float x = sample_coord(q.sw, pw, q.bw, ix, q.gw);
          int64_t off[8];
          float w[8];
          if (!corners(z, y, x, D, H, W, order, off, w)) continue;
          float s[kClChannels];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            float v[kClChannels];
            load8(base + (uint32_t)off[k] * (uint32_t)C, v);
#pragma unroll
            for (int c = 0; c < kClChannels; ++c) s[c] = k == 0 ? w[0] * v[c] : s[c] + w[k] * v[c];
          }
#pragma unroll
          for (int c = 0; c < kClChannels; ++c) acc[c] = acc[c] + s[c];
        }
      }
    }
#pragma unroll
    for (int c = 0; c < kClChannels; ++c) res[(cg * kClChannels + c) * nbin + bin] = from_f<T>(acc[c] / q.count);
  }
  __syncthreads();
  // channel c's bins b0 .. b0 + nbin - 1 of plane pd are nbin consecutive output elements
  T *o = out + ((int64_t)r * C * PD + pd) * PH * PW + b0;
  const int64_t cs = (int64_t)PD * PH * PW;
  for (int e = tid; e < C * nbin; e += 256) {
    const int c = e / nbin, k = e - c * nbin;
    o[c * cs + k] = res[e];
  }
}

// [N, C, V] -> [N, V, C] in T, through 64 x 64 LDS tiles.  Global accesses are 16-byte pieces
// (E = 16 / sizeof(T) elements: E voxels of a channel on the way in, E channels of a voxel on
// the way out, 8 lanes per 128-byte line) when `vec` (C and V multiples of E, both buffers
// 16-byte aligned); element by element otherwise.
template <typename T>
__global__ __launch_bounds__(256) void ncdhw_to_channels_last_kernel(const T *src, T *dst, int C, int64_t V, bool vec) {
  constexpr int E = 16 / (int)sizeof(T);
  __shared__ T t[64][64 + 2];   // [voxel][channel]; rows 4 bytes apart from a multiple of 128
  const int tid = threadIdx.x;
  const int64_t v0 = (int64_t)blockIdx.x * 64;
  const int c0 = blockIdx.y * 64;
  const int64_t n = blockIdx.z;
  const T *s = src + n * C * V;
  T *d = dst + n * V * C;
  if (vec) {
    constexpr int PPL = 64 / E;   // pieces per 64-element line
#pragma unroll
    for (int i = 0; i < 64 * PPL / 256; ++i) {
      const int p = i * 256 + tid, cc = p / PPL, vv = (p % PPL) * E;
      if (c0 + cc < C && v0 + vv < V) {
        const uint4 u = *reinterpret_cast<const uint4 *>(s + (int64_t)(c0 + cc) * V + v0 + vv);
        const T *e = reinterpret_cast<const T *>(&u);
#pragma unroll
        for (int k = 0; k < E; ++k) t[vv + k][cc] = e[k];
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 64 * PPL / 256; ++i) {
      const int p = i * 256 + tid, vv = p / PPL, cc = (p % PPL) * E;
      if (v0 + vv < V && c0 + cc < C) {
        uint4 u;
        T *e = reinterpret_cast<T *>(&u);
#pragma unroll
        for (int k = 0; k < E; ++k) e[k] = t[vv][cc + k];
        *reinterpret_cast<uint4 *>(d + (v0 + vv) * C + c0 + cc) = u;
      }
    }
    return;
  }
  const int lane = tid & 63, row = tid >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int cc = i * 4 + row;
    if (c0 + cc < C && v0 + lane < V) t[lane][cc] = s[(int64_t)(c0 + cc) * V + v0 + lane];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int vv = i * 4 + row;
    if (v0 + vv < V && c0 + lane < C) d[(v0 + vv) * C + c0 + lane] = t[vv][lane];
  }
}

template <typename T>
int forward(const void *features, const void *rois, void *output, int N, int C, int D, int H, int W, int R, int PD,
            int PH, int PW, float scale, int sr, int order, hipStream_t st) {
  const T *f = static_cast<const T *>(features);
  const T *ro = static_cast<const T *>(rois);
  T *o = static_cast<T *>(output);
  // channels per thread: 4 (1 when C % 4 != 0); more channels per thread share each bin's
  // set-up but leave fewer threads to hide the gathers' latency (bench workload, separable
  // path: 1 / 2 / 4 / 8 / 16 channels 1.90 / 1.46 / 1.37 / 1.52 / 2.32 ms)
  constexpr int kC = 4;
  const int cpt = C % kC == 0 ? kC : 1;
  const int64_t total = (int64_t)R * (C / cpt) * PD * PH * PW;
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (cpt == kC)
    hipLaunchKernelGGL((roi_align3d_forward_kernel<T, kC>), dim3(grid), dim3(256), 0, st, f, ro, o, N, C, D, H, W, R, PD,
                       PH, PW, scale, sr, order);
  else
    hipLaunchKernelGGL((roi_align3d_forward_kernel<T, 1>), dim3(grid), dim3(256), 0, st, f, ro, o, N, C, D, H, W, R, PD,
                       PH, PW, scale, sr, order);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

template <typename T>
int forward_cl(const void *features_cl, const void *rois, void *output, int N, int C, int D, int H, int W, int R, int PD,
               int PH, int PW, float scale, int sr, int order, hipStream_t st) {
  int bpb = 0, parts = 0;
  cl_split(C, PH * PW, bpb, parts);
  const int64_t blocks = (int64_t)R * PD * parts;
  const int64_t grid = (blocks + 7) / 8 * 8;   // a multiple of 8: the kernel maps blocks to XCDs
  if (grid >= ((int64_t)1 << 31)) return OPS3D_FDA_EINVAL;
  const size_t lds = (size_t)C * bpb * sizeof(T);
  if (sr > 0 && sr <= 2)   // every roi's grid is separable with 4 taps per axis
    hipLaunchKernelGGL((roi_align3d_forward_cl_kernel<T, false>), dim3((unsigned)grid), dim3(256), lds, st,
                       static_cast<const T *>(features_cl), static_cast<const T *>(rois), static_cast<T *>(output), N,
                       C, D, H, W, PD, PH, PW, scale, sr, order, bpb, parts, (int)blocks);
  else
    hipLaunchKernelGGL((roi_align3d_forward_cl_kernel<T, true>), dim3((unsigned)grid), dim3(256), lds, st,
                       static_cast<const T *>(features_cl), static_cast<const T *>(rois), static_cast<T *>(output), N,
                       C, D, H, W, PD, PH, PW, scale, sr, order, bpb, parts, (int)blocks);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

template <typename T>
int to_channels_last(const void *features, void *features_cl, int N, int C, int64_t V, hipStream_t st) {
  hipLaunchKernelGGL((ncdhw_to_channels_last_kernel<T>), dim3((unsigned)((V + 63) / 64), (unsigned)((C + 63) / 64), N),
                     dim3(256), 0, st, static_cast<const T *>(features), static_cast<T *>(features_cl), C, V,
                     C % (16 / (int)sizeof(T)) == 0 && V % (16 / (int)sizeof(T)) == 0 &&
                         ((reinterpret_cast<uintptr_t>(features) | reinterpret_cast<uintptr_t>(features_cl)) & 15u) == 0);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

// Bytes of the gather backward's per-roi axis tables, rounded up to 16 (the channels-last copy of
// grad_output follows them).
inline size_t gather_tables_bytes(int R, int D, int H, int W, int PD, int PH, int PW) {
  const size_t b = (size_t)R * ((size_t)D * PD + (size_t)H * PH + (size_t)W * PW + (size_t)D + H + W) * 4;
  return (b + 15) & ~(size_t)15;
}

template <typename T>
int backward(const void *grad_output, const void *rois, void *grad_input, float *acc, int N, int C, int D, int H,
             int W, int R, int PD, int PH, int PW, float scale, int sr, int order, hipStream_t st) {
  if (gather_fits(PD, PH, PW)) {
    const int64_t blocks = (int64_t)N * ((C + kGCC - 1) / kGCC) * ((D + kGTZ - 1) / kGTZ) * ((H + kGTY - 1) / kGTY) *
                           ((W + kGTX - 1) / kGTX);
    // workspace: the per-roi axis tables, then grad_output channels-last [R, bins, C]
    float *wt = acc;
    uint32_t *ft = reinterpret_cast<uint32_t *>(acc + (size_t)R * ((size_t)D * PD + (size_t)H * PH + (size_t)W * PW));
    T *top_cl = reinterpret_cast<T *>(reinterpret_cast<char *>(acc) + gather_tables_bytes(R, D, H, W, PD, PH, PW));
    const int64_t pvol = (int64_t)PD * PH * PW;
    if (R > 0) {
      hipLaunchKernelGGL((roi_axis_table_kernel<T>), dim3((unsigned)R, 3), dim3(256), 0, st,
                         static_cast<const T *>(rois), wt, ft, D, H, W, PD, PH, PW, scale, sr, order);
      for (int r0 = 0; r0 < R; r0 += 65535) {   // grid z: at most 65535 rois per launch
        const int nr = min(65535, R - r0);
        const T *src = static_cast<const T *>(grad_output) + (int64_t)r0 * C * pvol;
        T *dst = top_cl + (int64_t)r0 * C * pvol;
        hipLaunchKernelGGL((ncdhw_to_channels_last_kernel<T>), dim3((unsigned)((pvol + 63) / 64), (unsigned)((C + 63) / 64), nr),
                           dim3(256), 0, st, src, dst, C, pvol,
                           C % (16 / (int)sizeof(T)) == 0 && pvol % (16 / (int)sizeof(T)) == 0 &&
                               ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0);
      }
    }
    hipLaunchKernelGGL((roi_align3d_backward_gather_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, st, top_cl,
                       static_cast<const T *>(rois), static_cast<T *>(grad_input), wt, ft, C % 4 == 0, N, C, D, H, W, R,
                       PD, PH, PW, scale, sr, order);
    return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
  }
  const int64_t nin = (int64_t)N * C * D * H * W;
  const int64_t vol = (int64_t)D * H * W;
  const int64_t nwaves = (int64_t)R * ((C + 63) / 64) * PD * PH;
  const int64_t fg = (nin + 255) / 256;
  const unsigned fill_grid = (unsigned)(fg < 65536 ? (fg > 0 ? fg : 1) : 65536);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(fill_grid), dim3(256), 0, st, acc, nin);
  if (nwaves > 0)
    hipLaunchKernelGGL((roi_align3d_backward_kernel<T>), dim3((unsigned)((nwaves + kBwdWaves - 1) / kBwdWaves)),
                       dim3(64 * kBwdWaves), 0, st, static_cast<const T *>(grad_output), static_cast<const T *>(rois),
                       acc, N, C, D, H, W, R, PD, PH, PW, scale, sr, order);
  hipLaunchKernelGGL((channels_last_to_ncdhw_kernel<T>), dim3((unsigned)((vol + 63) / 64), (unsigned)((C + 63) / 64), N),
                     dim3(256), 0, st, acc, static_cast<T *>(grad_input), C, vol);
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

int ops3d_roi_align3d_channels_last_supported(int dtype, int C, int D, int H, int W, int PW) {
  const int e = dtype == OPS3D_FDA_F32 ? 4 : (dtype == OPS3D_FDA_F16 || dtype == OPS3D_FDA_BF16 ? 2 : 0);
  // element offsets inside one batch item are 32-bit
  return e > 0 && PW > 0 && D > 0 && H > 0 && W > 0 && cl_supported(C) &&
                 (int64_t)D * H * W * C < ((int64_t)1 << 32)
             ? 1
             : 0;
}

int ops3d_roi_align3d_to_channels_last(const void *features, void *features_cl, int dtype, int N, int C, int D, int H,
                                       int W, void *stream) {
  if (!valid(dtype, N, C, D, H, W, 0, 1, 1, 1, 1) || N > 65535 || (C + 63) / 64 > 65535) return OPS3D_FDA_EINVAL;
  const int64_t V = (int64_t)D * H * W;
  if ((int64_t)N * C * V == 0) return OPS3D_FDA_OK;
  if (!features || !features_cl || (V + 63) / 64 >= ((int64_t)1 << 31)) return OPS3D_FDA_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case OPS3D_FDA_F32: return to_channels_last<float>(features, features_cl, N, C, V, st);
    case OPS3D_FDA_F16: return to_channels_last<__half>(features, features_cl, N, C, V, st);
    default: return to_channels_last<__hip_bfloat16>(features, features_cl, N, C, V, st);
  }
}

int ops3d_roi_align3d_forward_channels_last(const void *features_cl, const void *rois, void *output, int dtype, int N,
                                            int C, int D, int H, int W, int R, int PD, int PH, int PW,
                                            float spatial_scale, int sampling_ratio, int order, void *stream) {
  if (!valid(dtype, N, C, D, H, W, R, PD, PH, PW, order)) return OPS3D_FDA_EINVAL;
  if (!ops3d_roi_align3d_channels_last_supported(dtype, C, D, H, W, PW)) return OPS3D_FDA_EINVAL;
  if ((int64_t)R * C == 0) return OPS3D_FDA_OK;
  if (!features_cl || !rois || !output || (reinterpret_cast<uintptr_t>(features_cl) & 15u)) return OPS3D_FDA_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case OPS3D_FDA_F32:
      return forward_cl<float>(features_cl, rois, output, N, C, D, H, W, R, PD, PH, PW, spatial_scale, sampling_ratio,
                               order, st);
    case OPS3D_FDA_F16:
      return forward_cl<__half>(features_cl, rois, output, N, C, D, H, W, R, PD, PH, PW, spatial_scale, sampling_ratio,
                                order, st);
    default:
      return forward_cl<__hip_bfloat16>(features_cl, rois, output, N, C, D, H, W, R, PD, PH, PW, spatial_scale,
                                        sampling_ratio, order, st);
  }
}

size_t ops3d_roi_align3d_backward_workspace_bytes(int dtype, int N, int C, int D, int H, int W, int R, int PD,
                                                 int PH, int PW) {
  (void)dtype;
  if (N <= 0 || C <= 0 || D <= 0 || H <= 0 || W <= 0 || R < 0 || PD <= 0 || PH <= 0 || PW <= 0) return 0;
  if (gather_fits(PD, PH, PW))   // the per-roi axis tables and grad_output channels-last
    return R == 0 ? 0
                  : gather_tables_bytes(R, D, H, W, PD, PH, PW) +
                        (size_t)R * C * PD * PH * PW * (dtype == OPS3D_FDA_F32 ? 4 : 2);
  return (size_t)N * C * D * H * W * sizeof(float);
}

int ops3d_roi_align3d_backward(const void *grad_output, const void *rois, void *grad_input, void *workspace,
                               size_t workspace_bytes, int dtype, int N, int C, int D, int H, int W, int R, int PD,
                               int PH, int PW, float spatial_scale, int sampling_ratio, int order, void *stream) {
  if (!valid(dtype, N, C, D, H, W, R, PD, PH, PW, order)) return OPS3D_FDA_EINVAL;
  if ((int64_t)N * C == 0) return OPS3D_FDA_OK;
  if (!grad_input || ((int64_t)R > 0 && (!grad_output || !rois))) return OPS3D_FDA_EINVAL;
  const size_t need = ops3d_roi_align3d_backward_workspace_bytes(dtype, N, C, D, H, W, R, PD, PH, PW);
  if (need > 0 && (workspace_bytes < need || !workspace || (reinterpret_cast<uintptr_t>(workspace) & 15u)))
    return OPS3D_FDA_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case OPS3D_FDA_F32:
      return backward<float>(grad_output, rois, grad_input, static_cast<float *>(workspace), N, C, D, H, W, R, PD, PH,
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
