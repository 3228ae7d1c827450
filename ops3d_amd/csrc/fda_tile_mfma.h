// Matrix-core (gfx950 MFMA) building blocks of the tile-major backward (fda_fused.h), for 16-bit
// element types with D = 32.
//
// The value gradient of one tile is a product.  With the tile's entries e (samples with a corner
// in the tile), the 32 voxels v of one z-plane of the 8 x 4 x 4 tile and the 32 channels c:
//     grad_value[v][c] = sum_e W[v][e] * grad_out[e][c],
//     W[v][e] = attn_e * wz(e, plane) * wy(e, y_v) * wx(e, x_v)   (zero unless v is a corner of e)
// (the trilinear scatter of the reference, common.h:141-262, written as a gather).  One
// v_mfma_f32_32x32x16_{bf16,f16} adds 16 entries: the A operand (W, 32 voxels x 16 entries) is
// built by scattering the entries' 4 corner weights of the plane into a zeroed 32 x 16 LDS
// matrix, the B operand (16 grad_output rows x 32 channels) is read with ds_read_b64_tr_b16
// (transposed 16-bit reads) from the rows as loaded.  Accumulator layout (checked on gfx950):
// C[i][j] is in lane j + 32 h, register 4 m + r, for i = 8 m + 4 h + r.
#pragma once

#include "fda_device.h"

namespace ops3d_fda {

constexpr int kMfmaRowBytes = 64;                  // D = 32 16-bit channels

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma16;
template <> struct Mfma16<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ unsigned short bits(float w) {
    return __builtin_bit_cast(unsigned short, (__bf16)w);
  }
};
template <> struct Mfma16<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ unsigned short bits(float w) {
    return __builtin_bit_cast(unsigned short, (_Float16)w);
  }
};

// Four 16-bit elements through the LDS transpose unit: within each group of 16 lanes, lane
// 4a + b receives element b of the 8-byte pieces addressed by lanes a, a + 4, a + 8, a + 12.
__device__ __forceinline__ u32x2 lds_read_tr16(const unsigned char *p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4 *)(__attribute__((address_space(3))) unsigned char *)p);
  return __builtin_bit_cast(u32x2, v);
}

// Two transposed reads (8 elements, the B operand of one 32x32x16 MFMA), written as inline
// assembly: the compiler cannot tell the transpose-read builtin apart from pending LDS-DMA
// writes (buffer_load ... lds) into other LDS buffers and would wait for all of them first;
// this block waits only for its own reads (lgkmcnt).
__device__ __forceinline__ u32x4 lds_read_tr16x2(const unsigned char *p0, const unsigned char *p1) {
  u32x2 r0, r1;
  const uint32_t a0 = (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const unsigned char *)p0);
  const uint32_t a1 = (uint32_t)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const unsigned char *)p1);
  asm volatile(
      "ds_read_b64_tr_b16 %0, %2\n\t"
      "ds_read_b64_tr_b16 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1)
      : "v"(a0), "v"(a1)
      : "memory");
  return u32x4{r0.x, r0.y, r1.x, r1.y};
}

}  // namespace ops3d_fda
