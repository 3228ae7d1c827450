/*
 * C ABI of 3-D non-maximum suppression in libops3d_fda.so (gfx950).  Replaces nms_3d_cuda
 * (reference csrc/cuda/nms_3d_cuda.cu:105-162), bound as _C.nms_3d (csrc/nms_3d.h:27-44,
 * csrc/vision.cpp:15).  Plain pointers and sizes; all pointers are device memory; launches go to
 * `stream` (a hipStream_t) and are asynchronous.  Return codes as in ops3d_fda.h.
 */
#ifndef OPS3D_NMS3D_H
#define OPS3D_NMS3D_H

#include <stddef.h>
#include <stdint.h>

#include "ops3d_fda.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of device workspace ops3d_nms3d needs for n boxes: the n x ceil(n/64) 64-bit IoU mask
 * and, per row, a bitmap of its nonzero mask words (n x ceil(n/4096) 64-bit words); 0 for
 * n <= 0. */
OPS3D_FDA_API size_t ops3d_nms3d_workspace_bytes(int n);

/*
 * Greedy NMS over n boxes already sorted by decreasing score.
 *   boxes_sorted: [n, 6] fp32 (x1, y1, z1, x2, y2, z2) in score order;
 *   order:        [n] int64, original index of each sorted box;
 *   keep:         [n] int64 out: original indices of the kept boxes, in score order (the first
 *                 *num_keep entries are written);
 *   num_keep:     [1] int32 out (device memory).
 * A box is removed when its IoU with a kept, higher-scoring box exceeds iou_threshold; IoU =
 * inter / (Sa + Sb - inter) with extents max(min - max, 0), rounded in fp32 step by step (a
 * pair whose union is 0 has IoU NaN and removes nothing).  n must be <= 2^19 (the greedy pass
 * keeps a removed flag per box in 64 KB of LDS; the mask is quadratic: 128 MB at n = 2^17, 32 GB
 * at 2^19); the workspace must be 8-byte aligned.
 */
OPS3D_FDA_API int ops3d_nms3d(const float *boxes_sorted, const int64_t *order, int n, float iou_threshold,
                              void *workspace, size_t workspace_bytes, int64_t *keep, int32_t *num_keep,
                              void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OPS3D_NMS3D_H */
