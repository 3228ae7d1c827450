// Device-side building blocks of the gfx950 Flash Deformable 3D Attention kernels.
//
// Work decomposition (shared by forward and backward):
//   * a "unit" is one (b, q, g) triple: one query, one head.  LPU consecutive lanes of a wave64
//     own a unit; each lane owns CPL consecutive channels of the head (CPL*sizeof(T) bytes,
//     one 16-byte load for bf16/fp16 with CPL=8 or fp32 with CPL=4).
//   * a workgroup is 4 waves = UPB = 4*64/LPU units, all of the SAME (b, g) and consecutive q.
//     Blocks are mapped to heads XCD-first (map_tile): the hardware dispatches workgroup i to
//     XCD i % 8, so with G = 8 each XCD only ever gathers (and, in backward, scatters) the
//     channels of one head and its 4 MB L2 holds that head's slice of the value volume.
//   * the unit's packed record (L*K*3 locations + L*K logits, reference layout
//     csrc/cuda/flash_deform_im2col_cuda.cuh:151-153,217-219) is staged once into LDS as fp32
//     by the unit's own lanes; the softmax over the L*K logits runs cooperatively across the
//     LPU lanes with cross-lane reductions (no block barrier; a unit never leaves its wave).
//   * corner gathers are raw buffer loads: a corner outside the level volume gets the offset
//     OOB_ELEM, and the buffer hardware returns zeros (loads) or drops the write (atomics).
//     This is the zero padding of the reference (common.h:99-117) without branches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ops3d_fda {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;
// Corner offsets are kept in ELEMENTS.  A corner outside the volume gets OOB_ELEM; scaled to
// bytes (x2 or x4) it lands at >= 2^30, beyond every buffer we create (the host limits
// S*G*D to 2^28 elements, i.e. <= 1 GiB of fp32 per batch item), so the buffer unit returns 0
// for loads and drops atomics.
constexpr uint32_t OOB_ELEM = 0x20000000u;
constexpr int64_t kMaxLevelElems = (int64_t)1 << 28;
constexpr int kBufferFlags = 0x00020000;      // dword3 of a gfx9-family raw buffer resource

struct Args {
  const void *value;          // [B,S,G,D] T
  const int64_t *shapes;      // [L,3] (D,H,W)
  const int64_t *lsi;         // [L]
  const void *loc_attn;       // [B,Q,G,P] T
  const float *ref;           // offset mode: reference points [B,Q,ref_levels,3] fp32 (x,y,z in
                              // [0,1]); the location entries of loc_attn are then offsets in
                              // voxels of their level (NULL: normalised locations)
  int ref_levels;             // 1 (one point per query) or L (one per level)
  float *grad_ref;            // offset mode, backward: [B,Q,ref_levels,3] fp32, added into (NULL: none)
  // DCNv4-3D mode (dcn != 0): one level (the input volume), Q = Dout*Hout*Wout output voxels;
  // unit (b, q, g)'s record sits at loc_attn + (b*Q + q) * rec_stride + g * P (rows padded to
  // rec_stride); its L*K triples are offsets, turned into pixel coordinates in the kernels
  // (dcn_to_pixels); the softmax over the K mask values is optional (dcn_softmax)
  int dcn, dcn_softmax, dcn_remove_center, rec_stride;
  int kd, kh, kw, sd, sh, sw, pd, ph, pw, dld, dlh, dlw, Dout, Hout, Wout;
  float offset_scale;
  const void *grad_out;       // [B,Q,G*D] T          (backward)
  void *out;                  // [B,Q,G*D] T          (forward)
  float *grad_value;          // [B,S,G,D] fp32 acc   (backward)
  void *grad_loc_attn;        // [B,Q,G,P] T          (backward)
  // backward, tile formulation of grad_value
  uint32_t *keys;             // [N] bucketing key of each sample (tile_key; kKeyInvalid if outside)
  float4 *stash;              // [N] (x, y, z, attn) of each sample: level pixel coordinates
  uint32_t *tile_counts;      // [B*G*T_h] entries per tile
  uint32_t *tile_start;       // [B*G*T_h] first entry of each tile (head base + exclusive scan)
  uint32_t *tile_cursor;      // [B*G*T_h] fill cursor of each tile
  uint32_t *tile_queue;       // [8] tile kernel work counters (one per XCD group), zero at launch;
                              // [8] the tile kernel's split factor, for the combine kernel
  float *split_scratch;       // [split_slots][tile voxels][D] fp32 partial sums of split tiles
  uint32_t split_slots;       // scratch slots (0: tiles are never split)
  uint32_t count_clear_wcap;  // != 0: the query kernel zeroes tile_counts when a head has more
                              // tiles than this (the bucketing's atomic mode)
  uint32_t *entries;          // [<= 8N] sample indices, grouped by tile
  int TX, TY, TZ;             // nominal tile dimensions (voxels), clipped per level
  int chunk;                  // entries per LDS chunk of the tile kernel
  int tile_affinity;          // tiles of head g run on XCD g % 8 (G % 8 == 0)
  int accumulate;             // add into an fp32 grad_value instead of overwriting
  int big_tiles;              // tile kernel with tile_threads(lpu, true) threads (big_tiles())
  int vhm;                    // value is head-major [B,G,S,D] (a transposed copy)
  int pair_levels;            // head-major copy in which large levels may be paired (copy_level);
                              // 0: every level at its level_start_index, heads S rows apart
  void *gout_hm;              // head-major copy [B,G,Q,D] of grad_out (G > 1): written by the
                              // query kernel, read by the tile kernel
  double inv_lk;              // 1.0 / (L*K), for sample -> unit
  int B, S, G, D, L, K, Q, P;
  int nqb;                    // query blocks per batch = ceil(Q / UPB)
  int ncol;                   // B * nqb
  int xcd_mode;               // 0: G % 8 == 0, 1: 8 % G == 0, 2: no XCD affinity
  int hpx;                    // heads per XCD (mode 0)
  int xpg;                    // XCDs per head (mode 1)
};

// blockIdx.x -> (b, g, qb).  Returns false for padding blocks of mode 1.
__device__ __forceinline__ bool map_tile(const Args &a, int bid, int &b, int &g, int &qb) {
  int col;
  if (a.xcd_mode == 0) {
    const int xcd = bid & 7, r = bid >> 3;
    g = xcd * a.hpx + r % a.hpx;
    col = r / a.hpx;
  } else if (a.xcd_mode == 1) {
    const int xcd = bid & 7;
    g = xcd % a.G;
    col = (bid >> 3) * a.xpg + xcd / a.G;
    if (col >= a.ncol) return false;
  } else {
    g = bid % a.G;
    col = bid / a.G;
  }
  b = col / a.nqb;
  qb = col - b * a.nqb;
  return true;
}

// ---------------------------------------------------------------------------------------------
// element types: float, _Float16, __bf16.  Conversions go through 32-bit words.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kPerWord = 1;
  static __device__ __forceinline__ void unpack(uint32_t w, float *f) { f[0] = __uint_as_float(w); }
  static __device__ __forceinline__ uint32_t pack(const float *f) { return __float_as_uint(f[0]); }
  // c + sum over the word's elements of a[e] * b[e]
  static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
    return fmaf(__uint_as_float(a), __uint_as_float(b), c);
  }
};
template <> struct Elem<__bf16> {
  static constexpr int kPerWord = 2;
  static __device__ __forceinline__ void unpack(uint32_t w, float *f) {
    f[0] = __uint_as_float(w << 16);
    f[1] = __uint_as_float(w & 0xffff0000u);
  }
  static __device__ __forceinline__ uint32_t pack(const float *f) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 h;
    h.x = (__bf16)f[0];   // round to nearest even (v_cvt_pk_bf16_f32)
    h.y = (__bf16)f[1];
    return __builtin_bit_cast(uint32_t, h);
  }
  // v_dot2_f32_bf16: both bf16 products are exact in fp32, accumulated into c in fp32
  static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
  }
};
template <> struct Elem<_Float16> {
  static constexpr int kPerWord = 2;
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ void unpack(uint32_t w, float *f) {
    h2 h = __builtin_bit_cast(h2, w);
    f[0] = (float)h.x;
    f[1] = (float)h.y;
  }
  static __device__ __forceinline__ uint32_t pack(const float *f) {
    h2 h;
    h.x = (_Float16)f[0];
    h.y = (_Float16)f[1];
    return __builtin_bit_cast(uint32_t, h);
  }
  // v_dot2_f32_f16: both f16 products are exact in fp32, accumulated into c in fp32
  static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  }
};

// ---------------------------------------------------------------------------------------------
// raw buffer access
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           kBufferFlags);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Load NB bytes (NB in {4, 8, 12, 16, 24, 32, 48}) at byte offset `off` into words w[NB/4].
template <int NB>
__device__ __forceinline__ void bload(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t *w) {
  static_assert(NB % 4 == 0, "whole words only");
  if constexpr (NB == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else if constexpr (NB == 8) {
    u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (NB == 12) {
    u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z;
  } else if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (NB == 24) {
    u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    u32x2 t = __builtin_amdgcn_raw_buffer_load_b64(r, off + 16, 0, 0);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w; w[4] = t.x; w[5] = t.y;
  } else {
    static_assert(NB == 4, "unsupported vector width");
  }
}

// Load N elements of T (N*sizeof(T) bytes) at byte offset `off` and widen to fp32.
template <typename T, int N>
__device__ __forceinline__ void load_elems(__amdgpu_buffer_rsrc_t r, uint32_t off, float *f) {
  constexpr int NB = N * (int)sizeof(T);
  uint32_t w[NB / 4];
  bload<NB>(r, off, w);
#pragma unroll
  for (int i = 0; i < NB / 4; ++i) Elem<T>::unpack(w[i], f + i * Elem<T>::kPerWord);
}

// Dot product of N elements of T at byte offset `off` with N elements of T held as raw words
// `bw` (N*sizeof(T)/4 words), accumulated in fp32.
template <typename T, int N>
__device__ __forceinline__ float dot_elems(__amdgpu_buffer_rsrc_t r, uint32_t off, const uint32_t *bw) {
  constexpr int NB = N * (int)sizeof(T);
  uint32_t w[NB / 4];
  bload<NB>(r, off, w);
  float u = 0.f;
#pragma unroll
  for (int i = 0; i < NB / 4; ++i) u = Elem<T>::dot(w[i], bw[i], u);
  return u;
}

// Store N fp32 values as T to a plain global pointer (aligned to N*sizeof(T) or 16 bytes).
template <typename T, int N>
__device__ __forceinline__ void store_elems(T *p, const float *f) {
  constexpr int NB = N * (int)sizeof(T);
  constexpr int NW = NB / 4;
  uint32_t w[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) w[i] = Elem<T>::pack(f + i * Elem<T>::kPerWord);
  uint32_t *q = reinterpret_cast<uint32_t *>(p);
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i)
      *reinterpret_cast<u32x4 *>(q + 4 * i) = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
  } else if constexpr (NB % 8 == 0) {
#pragma unroll
    for (int i = 0; i < NW / 2; ++i) *reinterpret_cast<u32x2 *>(q + 2 * i) = u32x2{w[2 * i], w[2 * i + 1]};
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) q[i] = w[i];
  }
}

// ---------------------------------------------------------------------------------------------
// cross-lane sums/max inside a unit of LPU lanes (LPU a power of two, units aligned to LPU).
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
  if constexpr (M == 1) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  } else if constexpr (M == 2) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  } else if constexpr (M == 8) {
    // row_ror:8 inside a row of 16 lanes == lane ^ 8
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
  } else if constexpr (M == 4 || M == 16) {
    // ds_swizzle bit mode: and_mask = 0x1f, or_mask = 0, xor_mask = M
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (M << 10) | 0x1f));
  } else {
    return __shfl_xor(v, M, kWave);
  }
}

template <int LPU>
__device__ __forceinline__ float unit_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPU; m <<= 1) {
    if (m == 1) v += xor_lane<1>(v);
    else if (m == 2) v += xor_lane<2>(v);
    else if (m == 4) v += xor_lane<4>(v);
    else if (m == 8) v += xor_lane<8>(v);
    else if (m == 16) v += xor_lane<16>(v);
    else v += xor_lane<32>(v);
  }
  return v;
}

template <int LPU>
__device__ __forceinline__ float unit_max(float v) {
#pragma unroll
  for (int m = 1; m < LPU; m <<= 1) {
    float o;
    if (m == 1) o = xor_lane<1>(v);
    else if (m == 2) o = xor_lane<2>(v);
    else if (m == 4) o = xor_lane<4>(v);
    else if (m == 8) o = xor_lane<8>(v);
    else if (m == 16) o = xor_lane<16>(v);
    else o = xor_lane<32>(v);
    v = fmaxf(v, o);
  }
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave: a Hillis-Steele scan inside each row of 16
// lanes (DPP row shifts; lanes shifted in from outside the row read 0), then the totals of the
// rows before added from lanes 15, 31, 47.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);   // row_shr:8
  const uint32_t t0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t t1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t t2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const int row = (int)(threadIdx.x & (kWave - 1)) >> 4;
  return v + (row > 0 ? t0 : 0u) + (row > 1 ? t1 : 0u) + (row > 2 ? t2 : 0u);
}

// Make this wave's LDS writes visible to the other lanes of the same wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// ---------------------------------------------------------------------------------------------
// Stage one unit's packed record (P elements of T) into LDS as fp32; lane j of the unit loads
// words j, j+LPU, ...  Dead units (q >= Q) stage zeros.
template <typename T, int LPU>
__device__ __forceinline__ void stage_record(const T *rec_g, int P, int j, bool live, float *rec) {
  constexpr int EPW = Elem<T>::kPerWord;
  const int nw = P / EPW;
  const uint32_t *src = reinterpret_cast<const uint32_t *>(rec_g);
  for (int w = j; w < nw; w += LPU) {
    float f[EPW];
    const uint32_t word = live ? src[w] : 0u;
    Elem<T>::unpack(word, f);
#pragma unroll
    for (int e = 0; e < EPW; ++e) rec[w * EPW + e] = f[e];
  }
}

// Offset mode (Args::ref): the staged location entries are offsets in voxels of their level;
// turn them into normalised locations loc = ref + offset / size, rounded in fp32 step by step
// (division, then addition; no contraction) -- the location a caller computing it in fp32 and
// packing it would pass.  Lane j of the unit handles samples j, j+LPU, ...; bq = b*Q + q.
template <typename T, int LPU>
__device__ __forceinline__ void offsets_to_locations(const Args &a, int64_t bq, int j, bool live, float *rec) {
#pragma clang fp contract(off)
  const int LK = a.L * a.K;
  const float *ref = a.ref + bq * a.ref_levels * 3;
  for (int s = j; s < LK; s += LPU) {
    const int l = s / a.K;
    const int r = a.ref_levels > 1 ? 3 * l : 0;
    const float rx = live ? ref[r] : 0.f, ry = live ? ref[r + 1] : 0.f, rz = live ? ref[r + 2] : 0.f;
    rec[3 * s] = rx + rec[3 * s] / (float)a.shapes[3 * l + 2];
    rec[3 * s + 1] = ry + rec[3 * s + 1] / (float)a.shapes[3 * l + 1];
    rec[3 * s + 2] = rz + rec[3 * s + 2] / (float)a.shapes[3 * l];
  }
}

// Offset mode, backward: add this unit's part of the reference-point gradient,
//     grad_ref[b,q,r,c] += sum over the unit's samples of reference r of grad_offset_c * size_c
// (d loc / d ref = 1, d loc / d offset = 1 / size), from the offset gradients in rec.  Lane j
// of the unit handles (r, c) pairs j, j+LPU, ...; fp32 atomics, as the G heads of a query add
// to the same elements (their order, and so the rounding, varies between runs).
template <int LPU>
__device__ __forceinline__ void add_ref_grad(const Args &a, int64_t bq, int j, const float *rec) {
  const int R = a.ref_levels, K = a.K, L = a.L;
  for (int t = j; t < 3 * R; t += LPU) {
    const int r = t / 3, c = t - 3 * r;
    const int l0 = R > 1 ? r : 0, l1 = R > 1 ? r + 1 : L;
    float acc = 0.f;
    for (int l = l0; l < l1; ++l) {
      float sl = 0.f;
      for (int k = 0; k < K; ++k) sl += rec[3 * (l * K + k) + c];
      acc = fmaf(sl, (float)a.shapes[3 * l + 2 - c], acc);   // size of axis c: W, H, D
    }
    atomicAdd(a.grad_ref + bq * 3 * R + t, acc);
  }
}

// Modes of the query-major kernels, fixed at compile time so that the packed path carries no
// branch of the others: packed normalised locations, offsets around reference points (Args::ref)
// and DCNv4-3D (Args::dcn).
constexpr int kModePlain = 0, kModeOffsets = 1, kModeDcn = 2;

// Element offset of unit (b*Q + q)*G + g's record in loc_attn / grad_loc_attn: P per unit, or
// (DCNv4-3D) rows of rec_stride per (b, q).
template <int MODE>
__device__ __forceinline__ int64_t record_offset(const Args &a, int64_t unit) {
  if constexpr (MODE == kModeDcn) return (unit / a.G) * a.rec_stride + (unit % a.G) * a.P;
  return unit * a.P;
}

// DCNv4-3D mode: turn the staged offsets of unit (b, q) into pixel coordinates of the input
// volume (reference dcnv4_im2col_cuda.cuh:144-196):  with (z, y, x) the output voxel of q,
//     p0 = ((dil * (k - 1)) >> 1) - pad + pos * stride,  p0' = p0 - ((dil * (k - 1)) >> 1) * scale,
//     pixel = p0' + (tap * dil + offset) * scale   per axis,
// in fp32 step by step (no contraction).  Sample s is the s-th kernel tap in the order x (w)
// outermost, y, z innermost, skipping the centre tap when remove_center is set.
template <int LPU>
__device__ __forceinline__ void dcn_to_pixels(const Args &a, int q, int j, float *rec) {
#pragma clang fp contract(off)
  const int K = a.K;
  const int xo = q % a.Wout, yo = (q / a.Wout) % a.Hout, zo = q / (a.Wout * a.Hout);
  const int hw = (a.dlw * (a.kw - 1)) >> 1, hh = (a.dlh * (a.kh - 1)) >> 1, hd = (a.dld * (a.kd - 1)) >> 1;
  const float s = a.offset_scale;
  const float p0w = (float)(hw - a.pw + xo * a.sw) - (float)hw * s;
  const float p0h = (float)(hh - a.ph + yo * a.sh) - (float)hh * s;
  const float p0d = (float)(hd - a.pd + zo * a.sd) - (float)hd * s;
  const int centre = ((a.kw / 2) * a.kh + a.kh / 2) * a.kd + a.kd / 2;
  for (int t = j; t < K; t += LPU) {
    const int tap = (a.dcn_remove_center && t >= centre) ? t + 1 : t;
    const int i = tap / (a.kh * a.kd), jj = (tap / a.kd) % a.kh, k = tap % a.kd;
    rec[3 * t] = p0w + ((float)(i * a.dlw) + rec[3 * t]) * s;
    rec[3 * t + 1] = p0h + ((float)(jj * a.dlh) + rec[3 * t + 1]) * s;
    rec[3 * t + 2] = p0d + ((float)(k * a.dld) + rec[3 * t + 2]) * s;
  }
}

// Write one unit's record (P fp32 values in LDS) to global memory as T.
template <typename T, int LPU>
__device__ __forceinline__ void write_record(T *rec_g, int P, int j, const float *rec) {
  constexpr int EPW = Elem<T>::kPerWord;
  const int nw = P / EPW;
  uint32_t *dst = reinterpret_cast<uint32_t *>(rec_g);
  for (int w = j; w < nw; w += LPU) {
    float f[EPW];
#pragma unroll
    for (int e = 0; e < EPW; ++e) f[e] = rec[w * EPW + e];
    dst[w] = Elem<T>::pack(f);
  }
}

// In-place fp32 softmax over logits[0..n) of one unit (reference im2col.cuh:222-240: max,
// exp(x - max), divide by the sum; over all L*K jointly).  Lane j handles j, j+LPU, ...
template <int LPU>
__device__ __forceinline__ void unit_softmax(float *logits, int n, int j) {
  float m = -INFINITY;
  for (int s = j; s < n; s += LPU) m = fmaxf(m, logits[s]);
  m = unit_max<LPU>(m);
  float sum = 0.f;
  for (int s = j; s < n; s += LPU) {
    const float e = expf(logits[s] - m);
    logits[s] = e;
    sum += e;
  }
  sum = unit_sum<LPU>(sum);
  for (int s = j; s < n; s += LPU) logits[s] = logits[s] / sum;
}

// Pixel coordinate of a normalised location exactly as torch's grid_sample computes it for
// align_corners=False on grid = 2*loc - 1:  ((grid + 1) * size - 1) / 2, each step rounded in
// fp32, so the kernel samples at the same coordinate as the PyTorch path.  Contraction is off
// here: hipcc's default would fuse the products and subtractions into FMAs (one rounding of
// loc * size - 0.5), up to 1 ulp away from both torch and the reference CUDA's two roundings
// (float loc * size, then - 0.5 in double rounded to float, flash_deform_im2col_cuda.cuh:268-270),
// which costs the location gradients up to ~25 ulp of their terms near such a coordinate.
__device__ __forceinline__ float pixel_coord(float loc, float size) {
#pragma clang fp contract(off)
  const float grid = 2.f * loc - 1.f;
  return ((grid + 1.f) * size - 1.f) * 0.5f;
}

// Per-sample trilinear set-up shared by forward and backward.
struct Sample {
  uint32_t off[8];   // element offsets (voxel*G*D) inside the level, OOB_ELEM if outside
  float wx[2], wy[2], wz[2];
  int x0, y0, z0;    // base corner (may be -1)
};

// Whether the forward runs the x-pair kernel: 4 lanes x 16 bytes per 64-byte row, 8 lanes per
// query (host and device must agree: it sets the units per block).
__host__ __device__ constexpr bool fwd_pairs(int cpl, int lpu, int esize) {
  return lpu == 4 && cpl * esize == 16;
}

// Paired levels.  In the head-major copy of value a level whose per-head slice is larger than
// kPairedLevelBytes, with 64-byte rows (the x-pair kernels), is stored as x-pair lines: line u
// (u = -1 .. n-1 for the level's n voxels) holds rows u and u+1 in 128 aligned bytes, at rows
// 2(u+1) and 2(u+1)+1 of the level (line -1's first row and line n-1's second row are never
// read).  Each voxel is stored twice, so a corner-pair load touches exactly one 128-byte line
// instead of 1.5 on average: for slices far beyond the 4 MB L2 the gathers are bound by the
// lines fetched from HBM.  Smaller levels keep one row per voxel (doubling them would push
// them out of L2).
constexpr int64_t kPairedLevelBytes = (int64_t)8 << 20;

__host__ __device__ inline bool level_paired(int64_t voxels, int row_bytes) {
  return row_bytes == 64 && voxels * 64 > kPairedLevelBytes;
}

// Rows of a level in the head-major copy.
__host__ __device__ inline int64_t level_copy_rows(int64_t voxels, int row_bytes) {
  return level_paired(voxels, row_bytes) ? 2 * voxels + 2 : voxels;
}

// Whether any level of a volume of S voxels with rows of row_bytes can be paired (host and
// device: without it every level keeps its level_start_index and no level table is read).
__host__ __device__ inline bool pairing_possible(int64_t S, int row_bytes) {
  return level_paired(S, row_bytes);
}

// Rows of one head's slice of the head-major copy, at most: room for every level paired (the
// workspace size).
__host__ __device__ inline int64_t head_copy_rows_max(int64_t S, int row_bytes) {
  return row_bytes == 64 ? 2 * S + 2 * 5 : S;
}

// Level l in a head's slice of the head-major copy: first row and layout.  Levels are paired
// only when level_start_index is the exclusive sum of the level sizes and the levels cover the
// S rows exactly (the layout every caller builds); otherwise each level stays at its
// level_start_index, as in value.
struct CopyLevel {
  int64_t start;
  bool paired;
};

__device__ inline CopyLevel copy_level(const int64_t *shapes, const int64_t *lsi, int L, int64_t S, int l,
                                       int row_bytes) {
  if (row_bytes != 64) return {lsi[l], false};
  int64_t plain = 0, start = 0;
  bool standard = true;
  for (int i = 0; i < L; ++i) {
    const int64_t n = shapes[3 * i] * shapes[3 * i + 1] * shapes[3 * i + 2];
    standard = standard && lsi[i] == plain;
    if (i < l) start += level_copy_rows(n, row_bytes);
    plain += n;
  }
  if (!standard || plain != S) return {lsi[l], false};
  return {start, level_paired(shapes[3 * l] * shapes[3 * l + 1] * shapes[3 * l + 2], row_bytes)};
}

// A block-uniform 64-bit value read from LDS, moved to scalar registers.
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint64_t u = (uint64_t)v;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// copy_level of every level into out[0, L); returns copy_head_rows.
__device__ inline int64_t copy_levels(const int64_t *shapes, const int64_t *lsi, int L, int64_t S, int row_bytes,
                                      CopyLevel *out) {
  int64_t plain = 0;
  bool standard = row_bytes == 64;
  for (int i = 0; i < L; ++i) {
    standard = standard && lsi[i] == plain;
    plain += shapes[3 * i] * shapes[3 * i + 1] * shapes[3 * i + 2];
  }
  standard = standard && plain == S;
  int64_t start = 0;
  for (int i = 0; i < L; ++i) {
    const int64_t n = shapes[3 * i] * shapes[3 * i + 1] * shapes[3 * i + 2];
    out[i] = standard ? CopyLevel{start, level_paired(n, row_bytes)} : CopyLevel{lsi[i], false};
    start += level_copy_rows(n, row_bytes);
  }
  return standard ? start : S;
}

// Rows of one head's slice of the head-major copy (the distance between heads): S, plus the
// extra rows of the paired levels.
__device__ inline int64_t copy_head_rows(const int64_t *shapes, const int64_t *lsi, int L, int64_t S,
                                         int row_bytes) {
  if (row_bytes != 64) return S;
  int64_t extra = 0;
  for (int l = 0; l < L; ++l) {
    const CopyLevel cl = copy_level(shapes, lsi, L, S, l, row_bytes);
    if (cl.paired) extra += shapes[3 * l] * shapes[3 * l + 1] * shapes[3 * l + 2] + 2;
  }
  return S + extra;
}

// Element offset, in a paired level, of the row a pair lane loads: `o` is the corner's element
// offset in the plain layout (row * RST, or OOB_ELEM), dxl the lane's x-row of the pair.  Row r
// is read through line r - dxl: copy row 2(r - dxl + 1) + dxl.
__device__ __forceinline__ uint32_t paired_offset(uint32_t o, int dxl, int RST) {
  return o == OOB_ELEM ? OOB_ELEM : 2u * o + (uint32_t)((2 - dxl) * RST);
}

// Compile-time loop: f(IntConst<0>{}), ..., f(IntConst<N-1>{}).
template <int V> struct IntConst { static constexpr int value = V; };
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(IntConst<N - 1>{});
  }
}

// Compact per-sample set-up: base corner and the two linear weights per axis.  One lane of a
// unit computes it and broadcasts it to the unit's other lanes (unit_bcast); each lane then
// expands it into the 8 corner offsets and weights (sample_expand).
struct SampleBase {
  int x0, y0, z0;                 // base corner (-1 allowed); -2 on every axis when outside
  float wx0, wx1, wy0, wy1, wz0, wz1;
};

// A coordinate outside [-1, size) on some axis (or NaN) leaves every corner outside the volume:
// such a sample gets base corner (-2, -2, -2), so all its loads are out of range and read zero,
// and zero weights, so it contributes nothing -- as with zero padding.  Returns whether the
// sample is inside.
// pix: the coordinates are pixel coordinates already (DCNv4-3D), and the range is the
// reference DCN's open (-1, size) (at exactly -1 a sample reads 0 either way).
__device__ __forceinline__ bool sample_base(float lx, float ly, float lz, int Wl, int Hl, int Dl,
                                            SampleBase &sb, bool pix = false) {
  const float x = pix ? lx : pixel_coord(lx, (float)Wl);
  const float y = pix ? ly : pixel_coord(ly, (float)Hl);
  const float z = pix ? lz : pixel_coord(lz, (float)Dl);
  const bool in = (pix ? (x > -1.f && y > -1.f && z > -1.f) : (x >= -1.f && y >= -1.f && z >= -1.f)) &&
                  x < (float)Wl && y < (float)Hl && z < (float)Dl;
  const float x0f = floorf(x), y0f = floorf(y), z0f = floorf(z);
  sb.x0 = in ? (int)x0f : -2; sb.y0 = in ? (int)y0f : -2; sb.z0 = in ? (int)z0f : -2;
  sb.wx1 = in ? x - x0f : 0.f; sb.wx0 = in ? (x0f + 1.f) - x : 0.f;
  sb.wy1 = in ? y - y0f : 0.f; sb.wy0 = in ? (y0f + 1.f) - y : 0.f;
  sb.wz1 = in ? z - z0f : 0.f; sb.wz0 = in ? (z0f + 1.f) - z : 0.f;
  return in;
}

// Corner offsets (element offsets voxel*GD inside the level, OOB_ELEM for a corner outside the
// volume) and weights of a sample.
__device__ __forceinline__ void sample_expand(const SampleBase &sb, int Wl, int Hl, int Dl, int GD, Sample &sm) {
  const int x0 = sb.x0, y0 = sb.y0, z0 = sb.z0;
  sm.x0 = x0; sm.y0 = y0; sm.z0 = z0;
  sm.wx[0] = sb.wx0; sm.wx[1] = sb.wx1;
  sm.wy[0] = sb.wy0; sm.wy[1] = sb.wy1;
  sm.wz[0] = sb.wz0; sm.wz[1] = sb.wz1;
  const bool vx0 = x0 >= 0, vx1 = x0 + 1 < Wl;
  const bool vy0 = y0 >= 0, vy1 = y0 + 1 < Hl;
  const bool vz0 = z0 >= 0, vz1 = z0 + 1 < Dl;
  const uint32_t sx = (uint32_t)GD, sy = (uint32_t)(Wl * GD), sz = (uint32_t)(Hl * Wl) * (uint32_t)GD;
  const uint32_t ox0 = (uint32_t)x0 * sx, oy0 = (uint32_t)y0 * sy, oz0 = (uint32_t)z0 * sz;
  const uint32_t ox[2] = {ox0, ox0 + sx}, oy[2] = {oy0, oy0 + sy}, oz[2] = {oz0, oz0 + sz};
  const bool vx[2] = {vx0, vx1}, vy[2] = {vy0, vy1}, vz[2] = {vz0, vz1};
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int dz = c >> 2, dy = (c >> 1) & 1, dx = c & 1;
    const bool ok = vz[dz] && vy[dy] && vx[dx];
    sm.off[c] = ok ? oz[dz] + oy[dy] + ox[dx] : OOB_ELEM;
  }
}

// Both steps in one lane.  Always fills sm; returns whether the sample is inside the volume.
__device__ __forceinline__ bool sample_setup(float lx, float ly, float lz, int Wl, int Hl, int Dl,
                                             int GD, Sample &sm, bool pix = false) {
  SampleBase sb;
  const bool in = sample_base(lx, ly, lz, Wl, Hl, Dl, sb, pix);
  sample_expand(sb, Wl, Hl, Dl, GD, sm);
  return in;
}

// Value of lane u of this lane's unit (units are LPU consecutive lanes; u < min(LPU, 4)).
template <int LPU, int U>
__device__ __forceinline__ uint32_t unit_bcast(uint32_t v) {
  if constexpr (LPU == 1) {
    return v;
  } else if constexpr (LPU == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, U | (U << 2) | ((2 + U) << 4) | ((2 + U) << 6), 0xF, 0xF,
                                              false);
  } else if constexpr (LPU == 4) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, U * 0x55, 0xF, 0xF, false);
  } else {
    const int lane = (int)(threadIdx.x & (kWave - 1));
    return (uint32_t)__shfl((int)v, (lane & ~(LPU - 1)) | U, kWave);
  }
}

// The 8 corner offsets and 8 corner weights of lane U's sample.
struct SampleCorners {
  uint32_t off[8];
  float w[8];
};

__device__ __forceinline__ void sample_corners(const Sample &sm, SampleCorners &sc) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    sc.off[c] = sm.off[c];
    sc.w[c] = (sm.wx[c & 1] * sm.wy[(c >> 1) & 1]) * sm.wz[c >> 2];
  }
}

template <int LPU, int U>
__device__ __forceinline__ SampleCorners unit_bcast(const SampleCorners &sc) {
  SampleCorners r;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    r.off[c] = unit_bcast<LPU, U>(sc.off[c]);
    r.w[c] = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sc.w[c])));
  }
  return r;
}

template <int LPU, int U>
__device__ __forceinline__ SampleBase unit_bcast(const SampleBase &sb) {
  SampleBase r;
  r.x0 = (int)unit_bcast<LPU, U>((uint32_t)sb.x0);
  r.y0 = (int)unit_bcast<LPU, U>((uint32_t)sb.y0);
  r.z0 = (int)unit_bcast<LPU, U>((uint32_t)sb.z0);
  r.wx0 = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sb.wx0)));
  r.wx1 = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sb.wx1)));
  r.wy0 = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sb.wy0)));
  r.wy1 = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sb.wy1)));
  r.wz0 = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sb.wz0)));
  r.wz1 = __uint_as_float(unit_bcast<LPU, U>(__float_as_uint(sb.wz1)));
  return r;
}

// LDS floats per unit of the backward query kernel (record, grad_attn, 16-byte-aligned stash,
// base corner x, y, z); the block uses UPB times this.  Rounded to 4 x an odd number so that the units of
// a wave start in different LDS banks.
__host__ __device__ constexpr int bwd_query_lds_floats(int P, int LK) {
  return ((((((P + LK + 3) & ~3) + 7 * LK) + 3) / 4) | 1) * 4;
}

// Sample numbering of the backward, head-major so that one block's samples are
// contiguous: gs = ((b*G + g)*Q + q)*L*K + s.
__device__ __forceinline__ uint32_t sample_index(int b, int g, int q, int s, int G, int Q, int LK) {
  return (((uint32_t)b * G + g) * (uint32_t)Q + q) * (uint32_t)LK + s;
}

// ---------------------------------------------------------------------------------------------
// Tiles of the backward's value gradient.  Each level of each (b, g) is cut into tiles of
// TX x TY x TZ voxels (clipped to the level: a level smaller than the tile is one tile); the
// tile kernel owns one tile at a time and sums every grad_value row of it in registers.  A
// sample is listed in its HOME tile, the tile containing corner (max(x0,0), max(y0,0),
// max(z0,0)), and additionally in the next tile along each axis on which its base corner is the
// home tile's last voxel (its upper corner then lies in that tile): 1 to 8 entries per sample.
// Threads of a tile-kernel block for `lpu` lanes per x-pair: 64 * lpu, at least 256 and at
// most 1024, so tiles hold 128 voxels (512/lpu for lpu < 4, 64 for lpu = 32).  `big` (lpu 4,
// large volumes): 512 threads and 256-voxel tiles, fewer entries per sample (a sample is
// listed in a neighbour tile only when its base corner is on the tile's last plane).
__host__ __device__ constexpr int tile_threads(int lpu, bool big = false) {
  return big && lpu == 4 ? 512 : (lpu <= 4 ? 256 : (lpu >= 16 ? 1024 : 64 * lpu));
}
// Volumes of at least kBigTileVoxels voxels per batch item take the big tiles: c5 (598 016
// voxels) tile kernel 2836 -> 2728 us and scatter 544 -> 472 us with them, c4 (73 728) tile
// kernel 228 -> 249 us.
constexpr int kBigTileVoxels = 1 << 18;
__host__ __device__ constexpr bool big_tiles(int S, int lpu) { return lpu == 4 && S >= kBigTileVoxels; }
constexpr int kTileKPT = 2;   // entries per thread and chunk (chunk <= KPT * threads)
constexpr uint32_t kKeyInvalid = 0xffffffffu;

// Lanes per x-pair of voxels in the tile kernel (lane_bytes = CPL * sizeof(T) of the query
// kernels).  The same as the query kernels' LPU: fewer lanes per pair would spread each entry
// visit's fixed cost over more channels, but put more pairs -- each with its own entry count --
// into a wave, whose loops run as long as its busiest pair's (measured slower on gfx950).
__host__ __device__ constexpr int tile_lanes(int lpu, int lane_bytes) { return (void)lane_bytes, lpu; }

// Nominal tile dimensions for the tile kernel: its tile_threads(lpu) threads own x-pairs of
// voxels, lpu lanes each, so a tile has 2 * tile_threads(lpu) / lpu voxels, as cubic as powers
// of two allow (x even).
__host__ __device__ constexpr void tile_dims(int lpu, int &tx, int &ty, int &tz, bool big = false) {
  int v = 2 * tile_threads(lpu, big) / lpu, lg = 0;
  while ((1 << lg) < v) ++lg;
  // split lg bits over (x, y, z): x gets the extra bit first, then y
  const int bz = lg / 3, by = (lg - bz) / 2, bx = lg - bz - by;
  tx = 1 << bx;
  ty = 1 << by;
  tz = 1 << bz;
}

// LDS bytes of fda_bwd_tile_kernel for `chunk` entries of row_bytes each, `lpu` tile lanes
// per x-pair (host side).
inline size_t tile_kernel_lds_bytes(int chunk, int row_bytes, int lpu, bool big = false) {
  int tx, ty, tz;
  tile_dims(lpu, tx, ty, tz, big);
  const size_t nb = (size_t)(tx + 1) * (ty + 1) * (tz + 1);
  return (size_t)chunk * (16 + (size_t)row_bytes + 4) + (2 * nb + 1) * 4;
}

struct LevelTiles {
  int n[3];       // level size (D, H, W)
  int t[3];       // tile size  (tz, ty, tx), clipped to the level
  int nt[3];      // tiles per axis
  int sh[3];      // log2 of the nominal tile size: tile index of a voxel = coordinate >> sh
                  // (t is the nominal size, a power of two, or the level is one tile wide)
  uint32_t count; // tiles of the level (0 for an empty level)
};

__device__ __forceinline__ LevelTiles level_tiles(const int64_t *shapes, int l, int TX, int TY, int TZ) {
  LevelTiles lt;
  const int T[3] = {TZ, TY, TX};
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const int n = (int)shapes[3 * l + a];
    lt.n[a] = n;
    lt.t[a] = n < T[a] ? (n > 0 ? n : 1) : T[a];
    lt.nt[a] = n > 0 ? (n + lt.t[a] - 1) / lt.t[a] : 0;
    lt.sh[a] = 31 - __builtin_clz((unsigned)T[a]);
  }
  lt.count = (uint32_t)lt.nt[0] * (uint32_t)lt.nt[1] * (uint32_t)lt.nt[2];
  return lt;
}

__device__ __forceinline__ uint32_t tiles_per_head(const int64_t *shapes, int L, int TX, int TY, int TZ) {
  uint32_t t = 0;
  for (int l = 0; l < L; ++l) t += level_tiles(shapes, l, TX, TY, TZ).count;
  return t;
}

// The bucketing's atomic mode (a head has more tiles than its LDS window) adds into tile_counts,
// so they must start at zero; block 0 of the query kernel, which runs just before, clears them
// as its last work (block 0 always has queries; a whole-block call, with a barrier).
__device__ __forceinline__ void clear_tile_counts(const Args &a) {
  __shared__ uint32_t th_s;
  if (a.count_clear_wcap == 0u || blockIdx.x != 0) return;
  if (threadIdx.x == 0) th_s = tiles_per_head(a.shapes, a.L, a.TX, a.TY, a.TZ);
  __syncthreads();
  const uint32_t T_h = th_s;
  if (T_h <= a.count_clear_wcap) return;
  const uint32_t total = (uint32_t)(a.B * a.G) * T_h;
  for (uint32_t i = threadIdx.x; i < total; i += blockDim.x) a.tile_counts[i] = 0u;
}

// Bucketing key of a sample: its home tile's id within its head (bits 6 and up), the "next tile"
// flags (x bit 3, y bit 4, z bit 5: the sample is also listed in the next tile along that axis)
// and its level (bits 0-2); kKeyInvalid for a sample outside the volume.  A head has fewer than
// 2^26 - 1 tiles (the host limits a level to 2^28 elements of G*D >= 8 channels).
__device__ __forceinline__ uint32_t tile_key(uint32_t tile, uint32_t flags, uint32_t level) {
  return (tile << 6) | (flags << 3) | level;
}

}  // namespace ops3d_fda
