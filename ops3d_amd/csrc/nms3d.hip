// 3-D non-maximum suppression on gfx950 (replaces the reference's nms_3d_cuda,
// csrc/cuda/nms_3d_cuda.cu:49-162, bound as _C.nms_3d by csrc/nms_3d.h:27-44).
//
// Boxes are (x1, y1, z1, x2, y2, z2) fp32, already sorted by decreasing score (the caller sorts,
// as the reference's host code does with torch).  Two kernels:
//   * nms3d_mask_kernel: for every pair of 64-box blocks (row block <= column block), one wave
//     compares its 64 row boxes against the 64 column boxes staged in LDS and writes one 64-bit
//     word per row box: bit i set when the row box's IoU with column box i (a later box) exceeds
//     the threshold.  64 boxes per word is the wave width: lane r owns row box r.  It also marks
//     which words of a row are nonzero, in a per-row bitmap (one bit per mask word, set by
//     atomic OR; cleared by a fill kernel first): boxes overlap only their neighbours, so a row
//     has few nonzero words.
//   * nms3d_reduce_kernel: the greedy pass on the GPU, one workgroup (the reference copies the
//     whole mask to the host and loops there).  Walking the sorted boxes in order, a box not yet
//     removed is kept and its mask row is OR-ed into the removed set -- only the row's nonzero
//     words, found from its bitmap.  It writes the kept boxes' original indices (order[i]) in
//     score order and their number; only that number has to reach the host (to size the
//     result).
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
                                                                   uint64_t *mask, int words, uint64_t *nzb,
                                                                   int nzw) {
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
  if (bits != 0 && cb > rb)   // off-diagonal nonzero word: mark it in the row's bitmap
    atomicOr(reinterpret_cast<unsigned long long *>(nzb + (int64_t)(r0 + t) * nzw + (cb >> 6)),
             1ull << (cb & 63));
}

__global__ __launch_bounds__(256) void fill_zero_u64_kernel(uint64_t *p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0;
}

constexpr int kReduceThreads = 256;

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// One block of kReduceThreads; the removed flags (`words` 64-bit words) live in LDS.  Per
// 64-box block: every wave holds the block's 64 diagonal mask words (lane i: box i's), resolves
// which boxes survive serially from them (in scalar registers, unrolled and branch-free: a
// branchy loop that waited on each survivor's readlane cost 8 K cycles per block), wave 0
// writes the survivors'
// indices (lane i: box i, at its rank among them), and the survivors' rows are OR-ed into the
// removed words of later blocks: thread t serves row t % 64 and every 4th of its bitmap words
// (from the one holding word blk + 1: a row's bitmap marks only words after its own block),
// loading the nonzero mask words they name, up to 8 at a time, and adding them with LDS atomic
// OR.  The next block's diagonal words, original indices and first kPrefetch bitmap words per
// thread are loaded one block ahead, issued after the serial resolution, so a block waits for
// about one round of loads (its survivors' mask words).  Loading further ahead (two blocks, or
// the mask words of every row of the next block before its survivors are known) measured no
// better: the compiler's wait counts across the loop's back edge are conservative, so later
// loads are waited for early.
constexpr int kPrefetch = 8;   // bitmap words per thread loaded ahead (rows of up to 2^17 boxes)

__global__ __launch_bounds__(kReduceThreads) void nms3d_reduce_kernel(const uint64_t *mask, const uint64_t *nzb,
                                                                      int n, int words, int nzw,
                                                                      const int64_t *order, int64_t *keep,
                                                                      int32_t *num_keep) {
  extern __shared__ uint64_t removed_l[];
  const int t = threadIdx.x, lane = t & 63, slot = t >> 6;
  constexpr int kSlots = kReduceThreads / 64;
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
  // bitmap word j of this thread for block blk: q = (blk + 1) / 64 + slot + kSlots * j
  const auto bitmap_of = [&](int blk, int j) {
    const int row = blk * 64 + lane, q = ((blk + 1) >> 6) + slot + kSlots * j;
    return row < n && q < nzw ? nzb[(int64_t)row * nzw + q] : (uint64_t)0;
  };
  uint64_t diag_n = diag_of(0);
  int64_t ord_n = order_of(0);
  uint64_t bm_n[kPrefetch];
#pragma unroll
  for (int j = 0; j < kPrefetch; ++j) bm_n[j] = bitmap_of(0, j);
  int kept = 0;
  for (int blk = 0; blk < words; ++blk) {
    const uint64_t diag = diag_n;
    const int64_t ord = ord_n;
    uint64_t bm[kPrefetch];
#pragma unroll
    for (int j = 0; j < kPrefetch; ++j) bm[j] = bm_n[j];
    const int nb = min(n - blk * 64, 64);
    // serial resolution in scalar registers, unrolled and branch-free: box i survives when no
    // kept box has removed it; a survivor removes the boxes its diagonal word marks
    const uint64_t rm = removed_l[blk];
    uint64_t cur = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(rm >> 32)) << 32) |
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)rm);
    if (nb < 64) cur |= ~(((uint64_t)1 << nb) - 1);   // boxes past n: never kept
    uint64_t km = 0;   // boxes of this block that survive
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      const uint64_t alive = ((cur >> i) & 1) ^ 1;
      km |= alive << i;
      cur |= readlane64(diag, i) & (uint64_t)0 - alive;
    }
    // the next block's words, issued only now: a wait for this block's words placed after them
    // (loads complete in order) would wait for them too
    if (blk + 1 < words) {
      diag_n = diag_of(blk + 1);
      ord_n = order_of(blk + 1);
#pragma unroll
      for (int j = 0; j < kPrefetch; ++j) bm_n[j] = bitmap_of(blk + 1, j);
    }
    if (t < 64 && ((km >> lane) & 1)) {
      const int rank = __builtin_popcountll(km & (((uint64_t)1 << lane) - 1));
      keep[kept + rank] = ord;
    }
    kept += __builtin_popcountll(km);
    if ((km >> lane) & 1) {   // this thread's row survived: OR its nonzero later words in
      const int64_t row = (int64_t)blk * 64 + lane;
      const int q0 = ((blk + 1) >> 6) + slot;
      const auto add_row_words = [&](int q, uint64_t b) {
        while (b) {
          uint64_t v[8];
          int w[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {   // up to 8 loads in flight
            w[u] = b ? (q << 6) + __builtin_ctzll(b) : -1;
            b &= b - 1;
            v[u] = w[u] >= 0 ? mask[row * words + w[u]] : (uint64_t)0;
          }
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (v[u]) atomicOr(reinterpret_cast<unsigned long long *>(removed_l + w[u]), (unsigned long long)v[u]);
        }
      };
#pragma unroll
      for (int j = 0; j < kPrefetch; ++j) add_row_words(q0 + kSlots * j, bm[j]);
      for (int q = q0 + kSlots * kPrefetch; q < nzw; q += kSlots) add_row_words(q, nzb[row * nzw + q]);
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
  const size_t words = ((size_t)n + 63) / 64, nzw = (words + 63) / 64;
  return (size_t)n * (words + nzw) * sizeof(uint64_t);
}

int ops3d_nms3d(const float *boxes_sorted, const int64_t *order, int n, float iou_threshold, void *workspace,
                size_t workspace_bytes, int64_t *keep, int32_t *num_keep, void *stream) {
  if (n < 0) return OPS3D_FDA_EINVAL;
  if (n == 0) return OPS3D_FDA_OK;
  if (!boxes_sorted || !order || !keep || !num_keep || !workspace) return OPS3D_FDA_EINVAL;
  if (n > kMaxBoxes) return OPS3D_FDA_EINVAL;
  if (workspace_bytes < ops3d_nms3d_workspace_bytes(n) || (reinterpret_cast<uintptr_t>(workspace) & 7u))
    return OPS3D_FDA_EINVAL;
  const int words = (n + 63) / 64, nzw = (words + 63) / 64;
  uint64_t *mask = static_cast<uint64_t *>(workspace);
  uint64_t *nzb = mask + (size_t)n * words;   // per-row bitmap of nonzero mask words
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nz = (int64_t)n * nzw;
  hipLaunchKernelGGL(ops3d_nms::fill_zero_u64_kernel, dim3((unsigned)((nz + 255) / 256 < 4096 ? (nz + 255) / 256 : 4096)), dim3(256),
                     0, st, nzb, nz);
  hipLaunchKernelGGL(ops3d_nms::nms3d_mask_kernel, dim3(words, words), dim3(64), 0, st, boxes_sorted, n,
                     iou_threshold, mask, words, nzb, nzw);
  hipLaunchKernelGGL(ops3d_nms::nms3d_reduce_kernel, dim3(1), dim3(ops3d_nms::kReduceThreads),
                     (size_t)words * sizeof(uint64_t), st, mask, nzb, n, words, nzw, order, keep, num_keep);
  return hipGetLastError() == hipSuccess ? OPS3D_FDA_OK : OPS3D_FDA_ERUNTIME;
}

}  // extern "C"
