// libops3d_fda_bench.so: measurement baselines, gfx950 (the backward's value gradient by atomics,
// the LDS atomic rate, the random-gather ceiling).  Not part of the op (libops3d_fda.so) and not
// used by it; bench.py --atomic-baseline / --gather-ceiling and their GPU tests load it.
//
// 1. The reference's grad_value scheme, at the reference's own lane layout.  The reference's
//    backward (csrc/cuda/flash_deform_col2im_cuda.cuh:248-429, backward_kernel_warp_primitive,
//    calling ms_deform_attn_col2im_trilinear, csrc/cuda/common.h:141-262) adds
//    attn * w_corner * grad_out[c] into an fp32 grad_value with one atomic per sample, corner and
//    channel; ops3d/flash_deform_attn.py:44-62 (findspec_bwd) gives d_stride 1 at G = 8, D = 32,
//    so consecutive lanes own consecutive channels and one wave instruction adds a corner's whole
//    contiguous row of D floats for 64 / D units at once.  Same here: one lane per channel, D
//    lanes per (b, q, g) unit.
// 2. The LDS float-atomic rate (ds_add_f32, no return), the bound of any scheme that pre-combines
//    grad_value contributions with LDS atomics before writing them.
// 3. The random-gather ceiling: the rate at which waves fetch randomly placed blocks of
//    16 * G contiguous bytes (G lanes, one 16-byte load each) from a buffer of a given size, the
//    access pattern of the sampling kernels' corner rows (G = 8: one 128-byte x-pair line; G = 4:
//    a 64-byte row).  With the buffer inside L2, inside the MALL or in HBM it gives the ceiling
//    each kind of miss allows.
#include "fda_device.h"

#include "../../include/ops3d_fda_bench.h"

namespace ops3d_fda {
namespace {

constexpr int kBenchBlock = 256;

// Units of D lanes (D a power of two, 8..64), one channel per lane; 256 / D units per block in
// plain (b, q, g) order, as the reference maps its blocks.
template <typename T>
__global__ __launch_bounds__(kBenchBlock) void ref_layout_scatter_kernel(const Args a) {
  extern __shared__ float lds[];
  const int D = a.D, UPB = kBenchBlock / D;
  const int ju = threadIdx.x % D, ub = threadIdx.x / D;
  const int64_t unit = (int64_t)blockIdx.x * UPB + ub;   // ((b * Q) + q) * G + g
  const int64_t nunits = (int64_t)a.B * a.Q * a.G;
  const bool live = unit < nunits;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  float *rec = lds + ub * (P + 1);
  const T *src = static_cast<const T *>(a.loc_attn) + (live ? unit : 0) * P;
  for (int t = ju; t < P; t += D) rec[t] = live ? (float)src[t] : 0.f;
  __syncthreads();
  if (!live) return;
  // softmax over the unit's L*K logits, by every lane (fp32, max-subtracted)
  float mx = -INFINITY;
  for (int t = 0; t < LK; ++t) mx = fmaxf(mx, rec[3 * LK + t]);
  float sum = 0.f;
  for (int t = 0; t < LK; ++t) sum += expf(rec[3 * LK + t] - mx);
  const int g = (int)(unit % a.G), b = (int)(unit / ((int64_t)a.Q * a.G));
  const float tg = (float)static_cast<const T *>(a.grad_out)[unit * D + ju];
  const int GD = a.G * D;
  float *gv = a.grad_value + (int64_t)b * a.S * GD + g * D + ju;
  for (int l = 0; l < L; ++l) {
    const int Dl = (int)a.shapes[3 * l], Hl = (int)a.shapes[3 * l + 1], Wl = (int)a.shapes[3 * l + 2];
    float *gl = gv + a.lsi[l] * GD;
    for (int k = 0; k < K; ++k) {
      const int s = l * K + k;
      Sample ms;
      if (!sample_setup(rec[3 * s], rec[3 * s + 1], rec[3 * s + 2], Wl, Hl, Dl, GD, ms)) continue;
      const float at = expf(rec[3 * LK + s] - mx) / sum;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        if (ms.off[c] == OOB_ELEM) continue;
        const float w = at * ((ms.wx[c & 1] * ms.wy[(c >> 1) & 1]) * ms.wz[c >> 2]);
        atomicAdd(gl + ms.off[c], w * tg);
      }
    }
  }
}

__global__ __launch_bounds__(256) void clear_kernel(float *p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

// Every lane adds `iters` times into a 4096-float LDS array (address pattern: pattern 0
// consecutive per wave, 1 pseudo-random); the block's sum is written so nothing is dropped.
template <int PATTERN>
__global__ __launch_bounds__(256) void lds_add_kernel(float *out, int iters, float v) {
  __shared__ float acc[4096];
  for (int i = threadIdx.x; i < 4096; i += 256) acc[i] = 0.f;
  __syncthreads();
  uint32_t h = threadIdx.x * 2654435761u + blockIdx.x;
  for (int it = 0; it < iters; ++it) {
    int idx;
    if (PATTERN == 0) {
      idx = (int)((threadIdx.x + (uint32_t)it * 256u) & 4095u);
    } else {
      h = h * 1664525u + 1013904223u;
      idx = (int)((h >> 8) & 4095u);
    }
    __hip_atomic_fetch_add(&acc[idx], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int i = 0; i < 4096; ++i) s += acc[i];
    out[blockIdx.x] = s;
  }
}

// Every group of G lanes fetches `iters` random blocks (a hash of its group index and the
// iteration) and folds them into one word per thread, so nothing is optimised away.
template <int G>
__global__ __launch_bounds__(256) void gather_probe_kernel(const uint4 *src, uint32_t nblk, int iters, uint32_t *out,
                                                           uint32_t seed) {
  const int sub = (int)(threadIdx.x & 63) % G;
  uint32_t h = (blockIdx.x * 256u + threadIdx.x) / G * 2654435761u + seed;
  uint32_t acc = 0;
  for (int i = 0; i < iters; ++i) {
    h = h * 1664525u + 1013904223u;
    const uint32_t b = (h >> 7) % nblk;
    const uint4 v = src[(size_t)b * G + sub];
    acc += v.x ^ v.y ^ v.z ^ v.w;
  }
  out[blockIdx.x * 256u + threadIdx.x] = acc;
}

thread_local char g_err[256] = "";

int bench_fail(int code, const char *msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

}  // namespace
}  // namespace ops3d_fda

using namespace ops3d_fda;

extern "C" {

const char *ops3d_fda_bench_last_error(void) { return g_err; }

int ops3d_fda_bench_ref_scatter(const int64_t *spatial_shapes, const int64_t *level_start_index,
                                const void *sampling_loc_attn, const void *grad_output, float *grad_value_f32,
                                int dtype, int batch, int spatial_size, int num_heads, int channels,
                                int num_levels, int num_query, int num_point, void *stream) {
  g_err[0] = 0;
  if (dtype < 0 || dtype > 2) return bench_fail(1, "unsupported dtype");
  if (batch < 0 || spatial_size < 0 || num_heads < 1 || num_query < 0 || num_levels < 1 || num_levels > 5 ||
      num_point < 1 || num_point > 16)
    return bench_fail(1, "invalid sizes");
  if (channels != 8 && channels != 16 && channels != 32 && channels != 64)
    return bench_fail(1, "unsupported channels (one lane per channel: D in {8, 16, 32, 64})");
  const int64_t nval = (int64_t)batch * spatial_size * num_heads * channels;
  const int64_t nunits = (int64_t)batch * num_query * num_heads;
  if ((nval > 0 && !grad_value_f32) ||
      (nunits > 0 && (!spatial_shapes || !level_start_index || !sampling_loc_attn || !grad_output)))
    return bench_fail(1, "NULL pointer argument");
  if (nval >= ((int64_t)1 << 31)) return bench_fail(1, "grad_value too large for 32-bit offsets");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (nval > 0) {
    const unsigned blocks = (unsigned)((nval + 255) / 256 < 16384 ? (nval + 255) / 256 : 16384);
    hipLaunchKernelGGL(clear_kernel, dim3(blocks), dim3(256), 0, st, grad_value_f32, nval);
  }
  if (nunits == 0 || nval == 0) return hipGetLastError() == hipSuccess ? 0 : bench_fail(2, "clear failed");
  Args a{};
  a.shapes = spatial_shapes;
  a.lsi = level_start_index;
  a.loc_attn = sampling_loc_attn;
  a.grad_out = grad_output;
  a.grad_value = grad_value_f32;
  a.B = batch; a.S = spatial_size; a.G = num_heads; a.D = channels; a.L = num_levels; a.K = num_point;
  a.Q = num_query;
  a.P = 4 * num_levels * num_point;
  const int upb = kBenchBlock / channels;
  const unsigned grid = (unsigned)((nunits + upb - 1) / upb);
  const size_t lds = (size_t)upb * (a.P + 1) * sizeof(float);
  if (dtype == 0) hipLaunchKernelGGL(ref_layout_scatter_kernel<float>, dim3(grid), dim3(kBenchBlock), lds, st, a);
  else if (dtype == 1) hipLaunchKernelGGL(ref_layout_scatter_kernel<_Float16>, dim3(grid), dim3(kBenchBlock), lds, st, a);
  else hipLaunchKernelGGL(ref_layout_scatter_kernel<__bf16>, dim3(grid), dim3(kBenchBlock), lds, st, a);
  return hipGetLastError() == hipSuccess ? 0 : bench_fail(2, "launch failed");
}

int ops3d_fda_bench_gather(const void *src, size_t bytes, int group, int blocks, int iters, uint32_t *out,
                           unsigned seed, void *stream) {
  g_err[0] = 0;
  if (!src || !out || blocks < 1 || iters < 1 || (reinterpret_cast<uintptr_t>(src) & 15u))
    return bench_fail(1, "invalid arguments");
  if (group != 4 && group != 8 && group != 32 && group != 64) return bench_fail(1, "group must be 4, 8, 32 or 64");
  const size_t nblk = bytes / (16 * (size_t)group);
  if (nblk < 1 || nblk > 0xffffffffu) return bench_fail(1, "buffer size out of range");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint4 *s = static_cast<const uint4 *>(src);
  const uint32_t nb = (uint32_t)nblk;
  switch (group) {
    case 4: hipLaunchKernelGGL(gather_probe_kernel<4>, dim3(blocks), dim3(256), 0, st, s, nb, iters, out, seed); break;
    case 8: hipLaunchKernelGGL(gather_probe_kernel<8>, dim3(blocks), dim3(256), 0, st, s, nb, iters, out, seed); break;
    case 32: hipLaunchKernelGGL(gather_probe_kernel<32>, dim3(blocks), dim3(256), 0, st, s, nb, iters, out, seed); break;
    default: hipLaunchKernelGGL(gather_probe_kernel<64>, dim3(blocks), dim3(256), 0, st, s, nb, iters, out, seed); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : bench_fail(2, "launch failed");
}

int ops3d_fda_bench_lds_atomic(float *out, int blocks, int iters, int pattern, void *stream) {
  g_err[0] = 0;
  if (!out || blocks < 1 || iters < 1 || pattern < 0 || pattern > 1) return bench_fail(1, "invalid arguments");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (pattern == 0) hipLaunchKernelGGL(lds_add_kernel<0>, dim3(blocks), dim3(256), 0, st, out, iters, 1.f);
  else hipLaunchKernelGGL(lds_add_kernel<1>, dim3(blocks), dim3(256), 0, st, out, iters, 1.f);
  return hipGetLastError() == hipSuccess ? 0 : bench_fail(2, "launch failed");
}

}  // extern "C"
