// 3-D non-maximum suppression on gfx950 (replaces the reference's nms_3d_cuda,
// csrc/cuda/nms_3d_cuda.cu:49-162, bound as _C.nms_3d by csrc/nms_3d.h:27-44).
//
// Boxes are (x1, y1, z1, x2, y2, z2) fp32, already sorted by decreasing score (the caller sorts,
// as the reference's host code does with torch).  Two kernels:
//   * nms3d_mask_kernel: for every pair of 64-box blocks (row block <= column block), one wave
//     compares its 64 row boxes against the 64 column boxes staged in LDS and writes one 64-bit
//     word per row box: bit i set when the row box's IoU with column box i (a later box) exceeds
//     the threshold.  64 boxes per word is the wave width: lane r owns row box r.
//   * nms3d_reduce_kernel: the greedy pass on the GPU, one workgroup (the reference copies the
//     whole mask to the host and loops there).  Walking the sorted boxes in order, a box not yet
//     removed is kept and its mask row is OR-ed into the removed set.  It writes the kept boxes'
//     original indices (order[i]) in score order and their number; only that number has to
//     reach the host (to size the result).
// IoU (reference devIoU_3d, nms_3d_cuda.cu:36-47): intersection extents max(min - max, 0),
// volumes as products of extents, inter / (Sa + Sb - inter), each step rounded in fp32 (no
// contraction), so a CPU restatement in fp32 makes the same decisions.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ops3d_nms3d.h"

namespace ops3d_nms {

constexpr int kBoxesPerWord = 64;   // one wave64 = one 64-bit mask word
// The greedy pass keeps one removed flag per box in LDS: 2^19 boxes = 64 KB (the mask is then
// 32 GB, quadratic in the boxes).
constexpr int kMaxBoxes = 1 << 19;

__device__ __forceinline__ float iou3d(const float *a, const float *b) {
#pragma clang fp contract(off)
  const float left = fmaxf(a[0], b[0]), right = fminf(a[3], b[3]);
  const float top = fmaxf(a[1], b[1]), bottom = fminf(a[4], b[4]);
  const float front = fmaxf(a[2], b[2]), back = fminf(a[5], b[5]);
  const float w = fmaxf(right - left, 0.f), h = fmaxf(bottom - top, 0.f), d = fmaxf(back - front, 0.f);
  const float inter = w * h * d;
  const float sa = (a[3] - a[0]) * (a[4] - a[1]) * (a[5] - a[2]);
  const float sb = (b[3] - b[0]) * (b[4] - b[1]) * (b[5] - b[2]);
  return inter / (sa + sb - inter);
}

// grid: (column blocks, row blocks); block: 64 threads.  Blocks below the diagonal exit: the
// greedy pass reads only words at or after a box's own block.
__global__ __launch_bounds__(kBoxesPerWord) void nms3d_mask_kernel(const float *boxes, int n, float thresh,
                                                                   uint64_t *mask, int words) {
  const int cb = blockIdx.x, rb = blockIdx.y;
  if (cb < rb) return;
  __shared__ float cbox[kBoxesPerWord * 6];
  const int t = threadIdx.x;
  const int c0 = cb * kBoxesPerWord, r0 = rb * kBoxesPerWord;
  const int ncol = min(n - c0, kBoxesPerWord), nrow = min(n - r0, kBoxesPerWord);
  for (int i = t; i < ncol * 6; i += kBoxesPerWord) cbox[i] = boxes[(int64_t)c0 * 6 + i];
  __syncthreads();
  if (t >= nrow) return;
  float me[6];
#pragma unroll
  for (int k = 0; k < 6; ++k) me[k] = boxes[(int64_t)(r0 + t) * 6 + k];
  uint64_t bits = 0;
  const int start = cb == rb ? t + 1 : 0;   // only later boxes
  for (int i = start; i < ncol; ++i)
    if (iou3d(me, cbox + i * 6) > thresh) bits |= (uint64_t)1 << i;
  mask[(int64_t)(r0 + t) * words + cb] = bits;
}

constexpr int kReduceThreads = 256;

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// One block of kReduceThreads; the removed flags (`words` 64-bit words) live in LDS.  Per
// 64-box block: every wave holds the block's 64 diagonal mask words (lane i: box i's, loaded
// one block ahead together with the boxes' original indices), resolves which boxes survive
// serially from them (readlane, wave-uniform), wave 0 writes the survivors' indices (lane i:
// box i, at its rank among them), and all threads OR the survivors' rows into the removed words
// of later blocks: the (word, survivor) pairs are spread over the threads, consecutive threads
// reading consecutive words of a row, 8 loads in flight each, combined with LDS atomic OR.
__global__ __launch_bounds__(kReduceThreads) void nms3d_reduce_kernel(const uint64_t *mask, int n, int words,
                                                                      const int64_t *order, int64_t *keep,
                                                                      int32_t *num_keep) {
  extern __shared__ uint64_t removed_l[];
  const int t = threadIdx.x, lane = t & 63;
  for (int w = t; w < words; w += kReduceThreads) removed_l[w] = 0;
  __syncthreads();
  const auto diag_of = [&](int blk) {
    const int nb = min(n - blk * 64, 64);
    return lane < nb ? mask[(int64_t)(blk * 64 + lane) * words + blk] : (uint64_t)0;
  };
  const auto order_of = [&](int blk) {
    const int nb = min(n - blk * 64, 64);
    return lane < nb ? order[blk * 64 + lane] : (int64_t)0;
  };
  uint64_t diag_n = diag_of(0);
  int64_t ord_n = order_of(0);
  int kept = 0;
  for (int blk = 0; blk < words; ++blk) {
    const uint64_t diag = diag_n;
    const int64_t ord = ord_n;
    if (blk + 1 < words) {   // the next block's words, in flight during this block
      diag_n = diag_of(blk + 1);
      ord_n = order_of(blk + 1);
    }
    const int nb = min(n - blk * 64, 64);
    uint64_t cur = removed_l[blk];
    uint64_t km = 0;   // boxes of this block that survive
    for (int i = 0; i < nb; ++i) {
      if ((cur >> i) & 1) continue;   // wave-uniform
      km |= (uint64_t)1 << i;
      cur |= readlane64(diag, i);
    }
    __shared__ int rows_l[64];   // this block's survivors (box numbers), in order
    if (t < 64 && ((km >> lane) & 1)) {
      const int rank = __builtin_popcountll(km & (((uint64_t)1 << lane) - 1));
      keep[kept + rank] = ord;
      rows_l[rank] = blk * 64 + lane;
    }
    const int cnt = __builtin_popcountll(km);
    kept += cnt;
    __syncthreads();
    // (later word, survivor) pairs over all threads, 8 loads in flight per thread, combined by
    // LDS atomic OR
    const int later = words - blk - 1;
    const int pairs = later * cnt;
    for (int p0 = t; p0 < pairs; p0 += 8 * kReduceThreads) {
      uint64_t v[8];
      int wv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int p = p0 + u * kReduceThreads;
        const int q = p / later, w = blk + 1 + (p - q * later);   // consecutive threads: consecutive words
        wv[u] = w;
        v[u] = p < pairs ? mask[(int64_t)rows_l[q] * words + w] : (uint64_t)0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (v[u]) atomicOr(reinterpret_cast<unsigned long long *>(removed_l + wv[u]), (unsigned long long)v[u]);
    }
    __syncthreads();   // later blocks read the removed words written above
  }
  if (t == 0) *num_keep = kept;
}

}  // namespace ops3d_nms

using ops3d_nms::kMaxBoxes;

extern "C" {

size_t ops3d_nms3d_workspace_bytes(int n) {
  if (n <= 0) return 0;
  const size_t words = ((size_t)n + 63) / 64;
  return (size_t)n * words * sizeof(uint64_t);
}

int ops3d_nms3d(const float *boxes_sorted, const int64_t *order, int n, float iou_threshold, void *workspace,
                size_t workspace_bytes, int64_t *keep, int32_t *num_keep, void *stream) {
  if (n < 0) return OPS3D_FDA_EINVAL;
  if (n == 0) return OPS3D_FDA_OK;
  if (!boxes_sorted || !order || !keep || !num_keep || !workspace) return OPS3D_FDA_EINVAL;
  if (n > kMaxBoxes) return OPS3D_FDA_EINVAL;
  if (workspace_bytes < ops3d_nms3d_workspace_bytes(n) || (reinterpret_cast<uintptr_t>(workspace) & 7u))
    return OPS3D_FDA_EINVAL;
  const int words = (n + 63) / 64;
  uint64_t *mask = static_cast<uint64_t *>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ops3d_nms::nms3d_mask_kernel, dim3(words, words), dim3(64), 0, st, boxes_sorted, n,
                     iou_threshold, mask, words);
  hipLaunchKernelGGL(ops3d_nms::nms3d_reduce_kernel, dim3(1), dim3(ops3d_nms::kReduceThreads),
                     (size_t)words * sizeof(uint64_t), st, mask, n, words, order, keep, num_keep);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

}  // extern "C"
