/*
 * ops3d_fda_bench.h -- C ABI of libops3d_fda_bench.so: measurement baselines on gfx950 (the
 * backward's value gradient by atomics, the LDS atomic rate, the random-gather ceiling).  Not
 * part of the op: nothing in libops3d_fda.so calls these, and they replace no reference entry
 * point.  Return codes: 0 ok, 1 bad argument, 2 HIP failure
 * (message: ops3d_fda_bench_last_error()).  Pointers are device memory; `stream` a hipStream_t.
 */
#ifndef OPS3D_FDA_BENCH_H
#define OPS3D_FDA_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OPS3D_FDA_BENCH_API __attribute__((visibility("default")))

OPS3D_FDA_BENCH_API const char *ops3d_fda_bench_last_error(void);

/*
 * grad_value [B, S, G, D] in fp32 by the reference's own scheme and lane layout: one fp32 atomic
 * add per sample, corner inside the volume and channel, one lane per channel, so one wave
 * instruction adds a corner's contiguous row of D floats for 64 / D (b, q, g) units
 * (csrc/cuda/flash_deform_col2im_cuda.cuh:248-429 with csrc/cuda/common.h:141-262 at the
 * d_stride 1 of ops3d/flash_deform_attn.py:44-62).  The buffer is cleared first.  Layouts and
 * dtype codes (0 fp32, 1 fp16, 2 bf16) as in ops3d_fda.h; D in {8, 16, 32, 64}.
 */
OPS3D_FDA_BENCH_API int ops3d_fda_bench_ref_scatter(const int64_t *spatial_shapes, const int64_t *level_start_index,
                                                    const void *sampling_loc_attn, const void *grad_output,
                                                    float *grad_value_f32, int dtype, int batch, int spatial_size,
                                                    int num_heads, int channels, int num_levels, int num_query,
                                                    int num_point, void *stream);

/*
 * LDS float-atomic throughput probe: `blocks` blocks of 256 threads, each thread `iters`
 * ds_add_f32 (no return) of 1.0 into a 4096-float LDS array (pattern 0: consecutive addresses per
 * wave; 1: pseudo-random); out[block] receives the block's sum (256 * iters).  The rate bounds
 * any scheme that pre-combines value-gradient terms with LDS atomics.
 */
OPS3D_FDA_BENCH_API int ops3d_fda_bench_lds_atomic(float *out, int blocks, int iters, int pattern, void *stream);

/*
 * Random-gather ceiling probe: `blocks` blocks of 256 threads; every group of `group` lanes (4, 8,
 * 32 or 64) fetches `iters` pseudo-random blocks of 16 * group contiguous bytes (one 16-byte load
 * per lane) from src[0, bytes) (16-byte aligned); out[thread] receives a fold of what the thread
 * loaded.  Bytes fetched = blocks * 256 * iters * 16.  The rate against the buffer size (inside
 * L2, inside the MALL, in HBM) is the ceiling for the sampling kernels' random corner-row
 * gathers (group 8: 128-byte x-pair lines; group 4: 64-byte rows).
 */
OPS3D_FDA_BENCH_API int ops3d_fda_bench_gather(const void *src, size_t bytes, int group, int blocks, int iters,
                                               uint32_t *out, unsigned seed, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* OPS3D_FDA_BENCH_H */
