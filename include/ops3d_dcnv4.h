/*
 * C ABI of DCNv4-3D (deformable 3-D convolution, version 4) in libops3d_fda.so (gfx950).
 * Replaces dcnv4_forward / dcnv4_backward (reference csrc/dcnv4.h:7-60 ->
 * csrc/cuda/dcnv4_cuda.cu:20-189 -> dcnv4_im2col_cuda.cuh / dcnv4_col2im_cuda.cuh), bound as
 * _C.dcnv4_forward / _C.dcnv4_backward (csrc/vision.cpp:20-21).  Device pointers, sizes, a
 * hipStream_t as void*; asynchronous; return codes as in ops3d_fda.h; dtype F32 / F16 / BF16.
 *
 * Layouts: value [B, Din, Hin, Win, G*D] (channels last, G groups of D channels); offset
 * [B, Dout, Hout, Wout, padded_offset_dim], per group 4*K entries -- K (x, y, z) offsets, then K
 * mask values -- with K = kd*kh*kw (minus the centre tap when remove_center) and
 * padded_offset_dim >= G*4*K; output [B, Dout, Hout, Wout, G*D].  Output size per axis:
 * (in + 2*pad - (dil*(k-1) + 1)) / stride + 1.  Tap t (order: x outermost, y, z innermost)
 * of output voxel (z, y, x) samples the input at pixel
 *     p0' + (tap*dil + offset)*offset_scale,  p0' = ((dil*(k-1))>>1) - pad + pos*stride
 *                                                  - ((dil*(k-1))>>1)*offset_scale
 * per axis (trilinear, zero outside the volume, a sample counts when every coordinate is in
 * (-1, size)), weighted by its mask value (softmax over the K values when softmax != 0), summed
 * over taps; fp32 arithmetic.
 */
#ifndef OPS3D_DCNV4_H
#define OPS3D_DCNV4_H

#include <stddef.h>
#include <stdint.h>

#include "ops3d_fda.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of device workspace (256-byte aligned) the forward (backward = 0) or backward
 * (backward = 1) needs; 0 on invalid sizes.  The first 256 bytes hold the volume's shape. */
OPS3D_FDA_API size_t ops3d_dcnv4_workspace_bytes(int dtype, int batch, int depth_in, int height_in, int width_in,
                                                 int group, int group_channels, int kernel_d, int kernel_h,
                                                 int kernel_w, int stride_d, int stride_h, int stride_w, int pad_d,
                                                 int pad_h, int pad_w, int dilation_d, int dilation_h, int dilation_w,
                                                 int remove_center, int backward);

/* Forward: writes every element of output. */
OPS3D_FDA_API int ops3d_dcnv4_forward(const void *value, const void *offset, void *output, void *workspace,
                                      size_t workspace_bytes, int dtype, int batch, int depth_in, int height_in,
                                      int width_in, int group, int group_channels, int kernel_d, int kernel_h,
                                      int kernel_w, int stride_d, int stride_h, int stride_w, int pad_d, int pad_h,
                                      int pad_w, int dilation_d, int dilation_h, int dilation_w, float offset_scale,
                                      int remove_center, int softmax, int padded_offset_dim, int im2col_step,
                                      void *stream);

/*
 * Backward: writes every element of grad_value ([B,Din,Hin,Win,G*D], a gather over tiles of
 * the volume as in ops3d_fda_backward, no atomics) and the G*4*K gradient entries of each
 * grad_offset row (offset gradients, then mask gradients -- through the softmax when softmax
 * != 0); the row's padding (from G*4*K to padded_offset_dim) is not written: pass grad_offset
 * zeroed to get the reference's zeros there.
 */
OPS3D_FDA_API int ops3d_dcnv4_backward(const void *value, const void *offset, const void *grad_output,
                                       void *grad_value, void *grad_offset, void *workspace, size_t workspace_bytes,
                                       int dtype, int batch, int depth_in, int height_in, int width_in, int group,
                                       int group_channels, int kernel_d, int kernel_h, int kernel_w, int stride_d,
                                       int stride_h, int stride_w, int pad_d, int pad_h, int pad_w, int dilation_d,
                                       int dilation_h, int dilation_w, float offset_scale, int remove_center,
                                       int softmax, int padded_offset_dim, int im2col_step, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OPS3D_DCNV4_H */
