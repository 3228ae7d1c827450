/*
 * ops3d_fda.h -- C ABI of the MI355X (gfx950) Flash Deformable 3D Attention library
 * (libops3d_fda.so).
 *
 * Plain pointers and sizes only; no torch or HIP types in the signatures.  Every device
 * pointer must point to memory on the current HIP device; `stream` is a hipStream_t (or NULL
 * for the null stream).  All entry points are asynchronous with respect to the host: they
 * enqueue kernels on `stream` and return.  Validation errors are reported synchronously.
 *
 * Tensor layouts (all C-contiguous, identical to the reference's):
 *   value                [B, S, G, D]      dtype
 *   spatial_shapes       [L, 3] int64      rows (D_l, H_l, W_l), DEVICE memory (read by kernels)
 *   level_start_index    [L]    int64      exclusive prefix sum of D_l*H_l*W_l, DEVICE memory
 *   sampling_loc_attn    [B, Q, G, P]      dtype, P = L*K*3 + L*K, per (b,q,g) planar:
 *                                          L*K (x,y,z) triples (level-major, point-minor),
 *                                          then L*K raw attention logits
 *   output / grad_output [B, Q, G*D]       dtype
 *   grad_value           [B, S, G, D]      dtype
 *   grad_sampling_loc_attn [B, Q, G, P]    dtype (logit part already through softmax backward)
 *
 * Return codes: OPS3D_FDA_OK, OPS3D_FDA_EINVAL (bad argument; a Python binding raises
 * ValueError, as the reference's std::invalid_argument does through pybind), OPS3D_FDA_ERUNTIME
 * (assertion-type error or HIP failure; RuntimeError).  ops3d_fda_last_error() returns the
 * message of the last failure on the calling thread.
 */
#ifndef OPS3D_FDA_H
#define OPS3D_FDA_H

#include <stddef.h>
#include <stdint.h>

#ifndef OPS3D_FDA_API
#define OPS3D_FDA_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum { OPS3D_FDA_F32 = 0, OPS3D_FDA_F16 = 1, OPS3D_FDA_BF16 = 2 };
enum { OPS3D_FDA_OK = 0, OPS3D_FDA_EINVAL = 1, OPS3D_FDA_ERUNTIME = 2 };

/* ABI version of this header (bumped on any change of a signature or of a workspace layout a
 * caller can hand from one call to another). */
OPS3D_FDA_API int ops3d_fda_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
OPS3D_FDA_API const char *ops3d_fda_last_error(void);

/* 1 if (dtype, channels D) has a compiled kernel configuration, else 0. */
OPS3D_FDA_API int ops3d_fda_supported(int dtype, int channels);

/*
 * Bytes of optional device workspace for ops3d_fda_forward: room for the head-major copy of value
 * that the forward makes, or 0 when it makes none -- G == 1 (value is already head-major), value
 * smaller than 8 MiB per batch item (it fits every XCD's L2), fewer corner reads than a head has
 * rows (Q*L*K*8 < S), or invalid sizes.  The copy is [B,G] slices of S rows of D elements, or,
 * with 64-byte rows (D * element size == 64), of 2*S + 10 rows, where levels larger than 8 MiB
 * per head are stored as aligned x-neighbour row pairs (each pair load then reads one 128-byte
 * line).
 */
OPS3D_FDA_API size_t ops3d_fda_forward_workspace_bytes(int dtype, int batch, int spatial_size,
                                                       int num_heads, int channels,
                                                       int num_levels, int num_query,
                                                       int num_point);

/*
 * Forward.  Replaces flash_deform_attn_forward (reference csrc/flash_deform_attn.h:7-25 ->
 * csrc/cuda/flash_deform_attn_cuda.cu:20-91).  Writes every element of `output`
 * ([B,Q,G*D], dtype), so the caller need not zero it.  The softmax over the L*K logits of each
 * (b,q,g) is computed in fp32 inside the kernel; trilinear sampling uses zero padding and
 * align_corners=False pixel coordinates (loc*size - 0.5).
 *   workspace:   optional (NULL allowed).  When ops3d_fda_forward_workspace_bytes() is not 0 and
 *                a workspace of at least that size is given, the library first copies value
 *                head-major into it, so that each head's rows are contiguous and, with heads
 *                mapped to XCDs, stay in one XCD's L2 (faster; same results).  A non-NULL
 *                workspace smaller than that is an error (OPS3D_FDA_EINVAL).
 *   im2col_step: batch chunk size of the reference; min(batch, im2col_step) must divide batch
 *                (else OPS3D_FDA_ERUNTIME, as reference flash_deform_attn_cuda.cu:56-58).  Results
 *                do not depend on it.
 *   num_levels must be 1..5 and num_point 1..16 (else OPS3D_FDA_EINVAL).
 */
OPS3D_FDA_API int ops3d_fda_forward(const void *value, const int64_t *spatial_shapes,
                                    const int64_t *level_start_index,
                                    const void *sampling_loc_attn, void *output, void *workspace,
                                    size_t workspace_bytes, int dtype, int batch,
                                    int spatial_size, int num_heads, int channels,
                                    int num_levels, int num_query, int num_point,
                                    int im2col_step, void *stream);

/*
 * Bytes of device workspace ops3d_fda_backward / ops3d_fda_backward_accumulate_f32 need (0 on
 * invalid sizes): per sample (N = B*Q*G*L*K) its home tile, tile-local corner word and a 16-byte
 * stash, up to 8 four-byte tile entries; per tile (<= B*G*S) a count, a start and a cursor; 8
 * work counters; for small volumes (B*G*ceil(S/128) < 2048) fp32 partial sums of 2048 split
 * tiles; the bucketing matrix (B*G x 64 x (S/16 + 64) words); and head-major copies of value
 * (G > 1) and of grad_output (G > 1 and grad_output larger than 64 MiB; smaller ones are read in
 * place).  The pointer passed must be 256-byte aligned.
 */
OPS3D_FDA_API size_t ops3d_fda_backward_workspace_bytes(int dtype, int batch, int spatial_size,
                                                        int num_heads, int channels,
                                                        int num_levels, int num_query,
                                                        int num_point);

/*
 * Backward.  Replaces flash_deform_attn_backward (reference csrc/flash_deform_attn.h:27-52 ->
 * csrc/cuda/flash_deform_attn_cuda.cu:93-179).  Writes every element of grad_value and
 * grad_sampling_loc_attn in `dtype` (the caller need not zero them).  grad_value is a gather:
 * the samples are grouped by spatial tile (in `workspace`, at least
 * ops3d_fda_backward_workspace_bytes() bytes) and each grad_value row is summed in fp32 by one
 * owner and written once (no atomics).  The order of that sum follows the order in which the
 * grouping fills a tile, which can differ between runs, so grad_value can differ at the fp32
 * rounding level (as with the reference's atomic scatter); grad_sampling_loc_attn is bitwise
 * repeatable.  Samples whose pixel coordinate lies outside [-1, size) on any axis contribute
 * nothing and get zero location gradients.
 */
OPS3D_FDA_API int ops3d_fda_backward(const void *value, const int64_t *spatial_shapes,
                       const int64_t *level_start_index, const void *sampling_loc_attn,
                       const void *grad_output, void *grad_value,
                       void *grad_sampling_loc_attn, void *workspace, size_t workspace_bytes,
                       int dtype, int batch, int spatial_size, int num_heads, int channels,
                       int num_levels, int num_query, int num_point, int im2col_step,
                       void *stream);

/*
 * Backward with the head-major copy of value the forward already made.  Same as
 * ops3d_fda_backward, plus value_head_major: NULL, or the head-major copy of value that
 * ops3d_fda_forward left in its workspace, for the same value, spatial_shapes and
 * level_start_index, so the backward does not make it again.  (Neither call copies value when
 * it is smaller than 8 MiB per batch item or the gathers read fewer rows than a head has,
 * Q*L*K*8 < S: the forward then leaves its workspace unused and the backward ignores
 * value_head_major.)  Ignored when G == 1.  No counterpart in the reference
 * (its backward re-reads value, flash_deform_attn_cuda.cu:93-179); for autograd functions that
 * keep the forward workspace until the backward.
 */
OPS3D_FDA_API int ops3d_fda_backward_ex(const void *value, const void *value_head_major,
                       const int64_t *spatial_shapes, const int64_t *level_start_index,
                       const void *sampling_loc_attn, const void *grad_output, void *grad_value,
                       void *grad_sampling_loc_attn, void *workspace, size_t workspace_bytes,
                       int dtype, int batch, int spatial_size, int num_heads, int channels,
                       int num_levels, int num_query, int num_point, int im2col_step,
                       void *stream);

/*
 * Backward that ADDS the value gradient into a caller-owned fp32 buffer grad_value_f32
 * ([B,S,G,D] fp32, not cleared) instead of writing it in `dtype`; grad_sampling_loc_attn is
 * written in full in `dtype`.  Same workspace as ops3d_fda_backward.  No counterpart in the
 * reference (its backward always returns freshly zeroed-and-cast gradients,
 * flash_deform_attn_cuda.cu:139-178); for callers that sum value gradients over several calls
 * (micro-batches, several query sets attending the same value) or want them in fp32.
 */
OPS3D_FDA_API int ops3d_fda_backward_accumulate_f32(
    const void *value, const int64_t *spatial_shapes, const int64_t *level_start_index,
    const void *sampling_loc_attn, const void *grad_output, float *grad_value_f32,
    void *grad_sampling_loc_attn, void *workspace, size_t workspace_bytes, int dtype, int batch,
    int spatial_size, int num_heads, int channels, int num_levels, int num_query, int num_point,
    int im2col_step, void *stream);

/*
 * Offset mode: caller-side fusion of the sampling_loc_attn producer and of the
 * grad_sampling_loc_attn consumer (no counterpart in the reference, whose callers build the packed
 * tensor with torch.cat from separately computed locations and logits,
 * tests/test_flash_deform_attn.py:30-37).  offset_attn has the packed planar layout of
 * sampling_loc_attn ([B,Q,G,P]: L*K (x,y,z) triples, then L*K logits), but its triples are
 * offsets in voxels of their level -- the output of one linear projection of the query, used as
 * is.  The kernels form each location as
 *     loc = reference_points[b,q,r] + offset / (W, H, D) of the level     (fp32, step by step),
 * r = the level when ref_levels == L, 0 when ref_levels == 1; reference_points is
 * [B,Q,ref_levels,3] fp32 whatever the value dtype (a 16-bit reference point would be off by
 * about a voxel on a 256-wide level), (x, y, z) in [0, 1].  For fp32 values the result equals
 * ops3d_fda_forward on the locations a caller computes that way in fp32; for 16-bit values it is
 * more accurate (the location is never rounded to 16 bits).  The backward writes
 * grad_offset_attn in the same layout: offset gradients (d pixel / d offset = 1, so they are the
 * location gradients divided by the level size) and logit gradients; and, when
 * grad_reference_points is not NULL, ADDS the gradient of reference_points into it ([B,Q,
 * ref_levels,3] fp32, pass it zeroed): the sum over heads and points of offset gradient * level
 * size, by fp32 atomics (the order of the heads' additions, and so the rounding, can differ
 * between runs).  Same workspaces, errors and head-major reuse as
 * ops3d_fda_forward / ops3d_fda_backward_ex; ref_levels must be 1 or num_levels.
 */
OPS3D_FDA_API int ops3d_fda_forward_offsets(const void *value, const int64_t *spatial_shapes,
                       const int64_t *level_start_index, const void *offset_attn,
                       const float *reference_points, int ref_levels, void *output, void *workspace,
                       size_t workspace_bytes, int dtype, int batch, int spatial_size, int num_heads,
                       int channels, int num_levels, int num_query, int num_point, int im2col_step,
                       void *stream);
OPS3D_FDA_API int ops3d_fda_backward_offsets(const void *value, const void *value_head_major,
                       const int64_t *spatial_shapes, const int64_t *level_start_index,
                       const void *offset_attn, const float *reference_points, int ref_levels,
                       const void *grad_output, void *grad_value, void *grad_offset_attn,
                       float *grad_reference_points, void *workspace, size_t workspace_bytes,
                       int dtype, int batch,
                       int spatial_size, int num_heads, int channels, int num_levels,
                       int num_query, int num_point, int im2col_step, void *stream);

/*
 * Allocation-free backward.  Same as ops3d_fda_backward, with no workspace argument: the
 * workspace is a static device array of OPS3D_FDA_NOALLOC_SCRATCH_BYTES (64 MiB) inside the
 * library, which every device it runs on holds until the process ends.  Problems whose
 * ops3d_fda_backward_workspace_bytes() exceed that size are refused (OPS3D_FDA_EINVAL).  The call
 * allocates nothing (no hipMalloc, hipFree or allocating library routine); its first call on a
 * device resolves that device's array address.  Every call on a device shares that device's
 * array: calls that overlap on one device (different streams or host threads) race and must be
 * serialised by the caller.  No counterpart in the reference; for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
#define OPS3D_FDA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
OPS3D_FDA_API int ops3d_fda_backward_noalloc(const void *value, const int64_t *spatial_shapes,
                       const int64_t *level_start_index, const void *sampling_loc_attn,
                       const void *grad_output, void *grad_value,
                       void *grad_sampling_loc_attn, int dtype, int batch, int spatial_size,
                       int num_heads, int channels, int num_levels, int num_query, int num_point,
                       int im2col_step, void *stream);

/*
 * Phase timing (no counterpart in the reference; for benchmarks and profilers).  After
 * ops3d_fda_profile_enable(1), every call records HIP events on its stream around its phases.
 * ops3d_fda_profile_read(which, ms, n) waits for the last call of that kind to finish and writes
 * up to n durations in ms; which = 0 (backward): [0] head-major copies, [1] query-major kernel,
 * [2] tile counting and head scan, [3] entry scatter, [4] tile kernel; which = 1 (forward):
 * [0] head-major copy, [1] forward kernel.  Returns the number written (0 if nothing recorded).
 * Process-wide state, not thread-safe; enable on the device the calls run on.
 */
OPS3D_FDA_API int ops3d_fda_profile_enable(int on);
OPS3D_FDA_API int ops3d_fda_profile_read(int which, float *ms, int n);

#ifdef __cplusplus
}
#endif

#endif /* OPS3D_FDA_H */
