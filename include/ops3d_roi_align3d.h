/*
 * C ABI of 3-D RoI Align in libops3d_fda.so (gfx950).  Replaces roi_align_3d_forward /
 * roi_align_3d_backward (reference csrc/roi_align_3d.h:97-136 -> csrc/cuda/roi_align_3d_cuda.cu:
 * 22-74 -> csrc/cuda/roi_align_3d_cuda_kernel.cuh:27-220), bound as _C.roi_align_3d_forward /
 * _C.roi_align_3d_backward (csrc/vision.cpp:17-18).  Device pointers, sizes, a hipStream_t as
 * void*; asynchronous; return codes as in ops3d_fda.h; dtype OPS3D_FDA_F32 / F16 / BF16.
 */
#ifndef OPS3D_ROI_ALIGN3D_H
#define OPS3D_ROI_ALIGN3D_H

#include <stddef.h>
#include <stdint.h>

#include "ops3d_fda.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Forward.  features [N,C,D,H,W], rois [R,7] (batch index, x1, y1, z1, x2, y2, z2) in the same
 * dtype, output [R,C,PD,PH,PW] (every element written).  Per bin: the roi scaled by
 * spatial_scale, extents clamped to >= 1, sampling_ratio samples per axis (<= 0: ceil(extent /
 * pooled)), each sample interpolated (order 1: trilinear with the reference's edge handling;
 * order 0: nearest corner) and the samples averaged, in fp32.
 */
OPS3D_FDA_API int ops3d_roi_align3d_forward(const void *features, const void *rois, void *output, int dtype, int N,
                                            int C, int D, int H, int W, int R, int PD, int PH, int PW,
                                            float spatial_scale, int sampling_ratio, int order, void *stream);

/*
 * Channels-last forward (no counterpart in the reference, whose kernel reads [N,C,D,H,W]; same
 * results as ops3d_roi_align3d_forward, bit for bit).  features_cl is [N,D,H,W,C] (PyTorch's
 * channels_last_3d layout of an [N,C,D,H,W] tensor), 16-byte aligned; output [R,C,PD,PH,PW] as
 * above.  A voxel's channels are one contiguous row there, so each corner of a sample is one
 * 16-byte load of 8 channels.  Supported when C % 8 == 0, C <= 2048 and D*H*W*C < 2^32
 * (ops3d_roi_align3d_channels_last_supported: 1 or 0); otherwise it returns OPS3D_FDA_EINVAL.
 */
OPS3D_FDA_API int ops3d_roi_align3d_channels_last_supported(int dtype, int C, int D, int H, int W, int PW);
OPS3D_FDA_API int ops3d_roi_align3d_forward_channels_last(const void *features_cl, const void *rois, void *output,
                                                          int dtype, int N, int C, int D, int H, int W, int R, int PD,
                                                          int PH, int PW, float spatial_scale, int sampling_ratio,
                                                          int order, void *stream);
/* features [N,C,D,H,W] -> features_cl [N,D,H,W,C] (N <= 65535), for the forward above. */
OPS3D_FDA_API int ops3d_roi_align3d_to_channels_last(const void *features, void *features_cl, int dtype, int N, int C,
                                                     int D, int H, int W, void *stream);

/* Bytes of workspace ops3d_roi_align3d_backward needs for R rois and output bins PD x PH x PW,
 * 16-byte aligned: when PD, PH, PW <= 64 and PD*PH*PW <= 384 (the backward is then a gather
 * straight into grad_input) the per-roi axis weight tables, R*(D*PD + H*PH + W*PW + D + H + W)*4
 * bytes rounded up to 16, plus a channels-last copy of grad_output, R*PD*PH*PW*C elements (0
 * when R = 0); else N*C*D*H*W*4 (the gradient is accumulated channels-last in fp32 by atomics,
 * then transposed into grad_input). */
OPS3D_FDA_API size_t ops3d_roi_align3d_backward_workspace_bytes(int dtype, int N, int C, int D, int H, int W, int R,
                                                                int PD, int PH, int PW);

/*
 * Backward: grad_input [N,C,D,H,W] = the adjoint of the forward applied to grad_output
 * [R,C,PD,PH,PW]; every element of grad_input is written: its old contents are overwritten
 * (the reference's kernel adds into a buffer its caller zeroed; a caller accumulating gradients
 * adds the result itself).  With the bin limits above it is a gather (after passes that write
 * each roi's per-axis bin weights and grad_output channels-last to the workspace): each voxel sums the rois that reach it in
 * roi order, the same bits on every run; else
 * the samples' corner contributions are added by fp32 atomics into the cleared workspace, whose
 * order -- and so the last bit -- can differ between runs, as with the reference's atomics.
 */
OPS3D_FDA_API int ops3d_roi_align3d_backward(const void *grad_output, const void *rois, void *grad_input,
                                             void *workspace, size_t workspace_bytes, int dtype, int N, int C, int D,
                                             int H, int W, int R, int PD, int PH, int PW, float spatial_scale,
                                             int sampling_ratio, int order, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OPS3D_ROI_ALIGN3D_H */
