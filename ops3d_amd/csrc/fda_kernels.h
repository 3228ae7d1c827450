// gfx950 forward and backward kernels of Flash Deformable 3D Attention.
//
// Forward (replaces forward_kernel_reg, reference csrc/cuda/flash_deform_im2col_cuda.cuh:190-295):
//   out[b,q,g,:] = sum_{l,k} softmax(logits[b,q,g,:])[l,k] *
//                  trilinear(value_l[b,:,g,:], pixel(loc[b,q,g,l,k]))
// Backward (replaces backward_kernel_warp_primitive, flash_deform_col2im_cuda.cuh:248-429, and
// ms_deform_attn_col2im_trilinear, common.h:141-353), in two kernels around a bucketing of the
// samples by spatial tile:
//   phase 1 (query-major)  grad_loc  = attn * size * sum_c grad_out[c] * d(interp_c)/d(pixel)
//                          grad_attn = sum_c grad_out[c] * interp_c, then softmax backward
//                          grad_logit_i = a_i * (grad_attn_i - sum_j a_j grad_attn_j)
//                          + per sample: its home tile, tile-local base corner, stash
//                          (fx,fy,fz,attn)
//   phase 2 (fda_tiles.hip) entries (sample, tile-local corner) grouped by tile
//   phase 3 (tile-major)   grad_value[v] = sum over entries s of v's tile with a corner at v of
//                          attn_s * w_corner(s) * grad_out[unit(s)]   (register sums, no atomics)
// The per-sample location/attention partials are formed from U_i = sum_c grad_out[c] * V_i[c]
// (one dot product per corner) so the channel loop costs one FMA per corner and channel, and
// are summed over the unit's LPU lanes with DPP / ds_swizzle reductions.
#pragma once

#include "fda_device.h"

namespace ops3d_fda {

constexpr int kFwdWavesPerEU = 8;     // minimum waves per SIMD the x-pair forward is compiled for
// Backward query pair kernel: left to itself the compiler takes 107 VGPRs (4 waves per SIMD);
// 5 waves fit without spills.
constexpr int kQueryWavesPerEU = 5;
// Tile splitting (tile kernel): parts per tile aim at kSplitTarget jobs per block, at most
// kSplitMax parts per tile.
constexpr uint32_t kSplitTarget = 2u, kSplitMax = 8u;

// NW raw words from a plain global pointer (aligned to 16 bytes when NW % 4 == 0).
template <int NW>
__device__ __forceinline__ void load_global_words(const void *p, uint32_t *w) {
  const uint32_t *q = static_cast<const uint32_t *>(p);
  if constexpr (NW % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(q + 4 * i);
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (NW % 2 == 0) {
#pragma unroll
    for (int i = 0; i < NW / 2; ++i) {
      const u32x2 v = *reinterpret_cast<const u32x2 *>(q + 2 * i);
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = q[i];
  }
}

template <typename T, int N>
__device__ __forceinline__ void load_global_elems(const T *p, float *f) {
  constexpr int NB = N * (int)sizeof(T);
  constexpr int NW = NB / 4;
  uint32_t w[NW];
  const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(q + 4 * i);
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (NB % 8 == 0) {
#pragma unroll
    for (int i = 0; i < NW / 2; ++i) {
      const u32x2 v = *reinterpret_cast<const u32x2 *>(q + 2 * i);
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = q[i];
  }
#pragma unroll
  for (int i = 0; i < NW; ++i) Elem<T>::unpack(w[i], f + i * Elem<T>::kPerWord);
}

// ---------------------------------------------------------------------------------------------
template <typename T, int CPL, int LPU, int MODE>
__global__ __launch_bounds__(kBlock) void fda_forward_kernel(const Args a) {
  extern __shared__ float lds[];
  constexpr int UPW = kWave / LPU, UPB = kWavesPerBlock * UPW;
  int b, g, qb;
  if (!map_tile(a, blockIdx.x, b, g, qb)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int j = lane & (LPU - 1);
  const int ub = wave * UPW + lane / LPU;
  const int q = qb * UPB + ub;
  const bool live = q < a.Q;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  float *rec = lds + ub * (P + 1);
  const int64_t unit = ((int64_t)b * a.Q + (live ? q : 0)) * a.G + g;

  stage_record<T, LPU>(static_cast<const T *>(a.loc_attn) + record_offset<MODE>(a, unit), P, j, live, rec);
  wave_lds_sync();
  if constexpr (MODE == kModeOffsets) {
    offsets_to_locations<T, LPU>(a, unit / a.G, j, live, rec);
    wave_lds_sync();
  }
  if constexpr (MODE == kModeDcn) {
    dcn_to_pixels<LPU>(a, live ? q : 0, j, rec);
    wave_lds_sync();
  }
  if (MODE != kModeDcn || a.dcn_softmax) unit_softmax<LPU>(rec + 3 * LK, LK, j);
  wave_lds_sync();

  float acc[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] = 0.f;

  // value rows: [B,S,G,D] (stride G*D between voxels) or a head-major copy [B,G,S,D]
  const int RST = a.vhm ? a.D : a.G * a.D;
  const uint32_t lane_elem = (uint32_t)((a.vhm ? 0 : g * a.D) + j * CPL);
  const T *vb = static_cast<const T *>(a.value) +
                (a.vhm ? ((int64_t)b * a.G + g) * a.S * a.D : (int64_t)b * a.S * a.G * a.D);
  for (int l = 0; l < L; ++l) {
    const int Dl = (int)a.shapes[3 * l], Hl = (int)a.shapes[3 * l + 1], Wl = (int)a.shapes[3 * l + 2];
    const int64_t st = a.lsi[l];
    const uint32_t nbytes = (uint32_t)((int64_t)Dl * Hl * Wl * RST * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb + st * RST, nbytes);
    // NG samples per step: lane j < NG of each unit sets up sample k0 + j, then the unit
    // processes them one after the other from broadcast set-ups
    constexpr int NG = LPU < 4 ? LPU : 4;
    for (int k0 = 0; k0 < K; k0 += NG) {
      const int kj = k0 + (j < NG ? j : 0);
      const int sj = l * K + (kj < K ? kj : K - 1);
      Sample ms;
      sample_setup(rec[3 * sj], rec[3 * sj + 1], rec[3 * sj + 2], Wl, Hl, Dl, RST, ms, MODE == kModeDcn);
      if (!live) {   // a dead unit loads zeros
#pragma unroll
        for (int c = 0; c < 8; ++c) ms.off[c] = OOB_ELEM;
      }
      SampleCorners mine;
      sample_corners(ms, mine);
      const uint32_t at_mine = __float_as_uint(rec[3 * LK + sj]);
      static_for<NG>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if (k0 + u < K) {
          const SampleCorners sm = unit_bcast<LPU, u>(mine);
          const float at = __uint_as_float(unit_bcast<LPU, u>(at_mine));
          // raw words: widened to fp32 only where they are consumed
          constexpr int NW = CPL * (int)sizeof(T) / 4, EPW = Elem<T>::kPerWord;
          uint32_t v[8][NW];
#pragma unroll
          for (int c = 0; c < 8; ++c)
            bload<NW * 4>(rv, (sm.off[c] + lane_elem) * (uint32_t)sizeof(T), v[c]);
          const float *w = sm.w;
#pragma unroll
          for (int i = 0; i < NW; ++i) {
            float t[EPW], f[EPW];
            Elem<T>::unpack(v[0][i], f);
#pragma unroll
            for (int e = 0; e < EPW; ++e) t[e] = f[e] * w[0];
#pragma unroll
            for (int c = 1; c < 8; ++c) {
              Elem<T>::unpack(v[c][i], f);
#pragma unroll
              for (int e = 0; e < EPW; ++e) t[e] = fmaf(f[e], w[c], t[e]);
            }
#pragma unroll
            for (int e = 0; e < EPW; ++e) acc[i * EPW + e] = fmaf(at, t[e], acc[i * EPW + e]);
          }
        }
      });
    }
  }
  if (live) store_elems<T, CPL>(static_cast<T *>(a.out) + unit * a.D + j * CPL, acc);
}

// ---------------------------------------------------------------------------------------------
// Backward phase 1, query-major: gradients of the locations and logits of one unit, plus one
// (bin, sample, stash) record per sample for the value-gradient gather of phase 3.  No atomics.
// Forward for rows of 64 bytes (4 lanes x 16 bytes): the two x-neighbour rows of a corner pair
// are adjacent in memory, so a unit of 8 lanes fetches the pair as one 128-byte span (lanes 0-3
// row x0, lanes 4-7 row x0+1) -- 4 loads per sample instead of 8 and half the cache lines of
// two 64-byte loads when x0 is even.  Gathers of random rows cost per distinct 128-byte line,
// not per byte, so this halves the gather work per sample.  Each half accumulates its own x-row
// over all samples; the halves are summed once at the end.
template <typename T, int CPL, bool kPairs, int MODE>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kFwdWavesPerEU))) void fda_forward_pair_kernel(const Args a) {
  extern __shared__ float lds[];
  constexpr int LPU = 4, UL = 2 * LPU;
  constexpr int UPW = kWave / UL, UPB = kWavesPerBlock * UPW;
  static_assert(CPL * sizeof(T) == 16, "pair kernel: 16 bytes per lane, 64-byte rows");
  int b, g, qb;
  if (!map_tile(a, blockIdx.x, b, g, qb)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int ju = lane & (UL - 1);        // lane within the unit
  const int j = ju & (LPU - 1);          // channel chunk of the row
  const int dxl = ju / LPU;              // x-row of the pair this lane loads
  const int ub = wave * UPW + lane / UL;
  const int q = qb * UPB + ub;
  const bool live = q < a.Q;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  float *rec = lds + ub * (P + 1);
  const int64_t unit = ((int64_t)b * a.Q + (live ? q : 0)) * a.G + g;

  stage_record<T, UL>(static_cast<const T *>(a.loc_attn) + record_offset<MODE>(a, unit), P, ju, live, rec);
  wave_lds_sync();
  if constexpr (MODE == kModeOffsets) {
    offsets_to_locations<T, UL>(a, unit / a.G, ju, live, rec);
    wave_lds_sync();
  }
  if constexpr (MODE == kModeDcn) {
    dcn_to_pixels<UL>(a, live ? q : 0, ju, rec);
    wave_lds_sync();
  }
  if (MODE != kModeDcn || a.dcn_softmax) unit_softmax<UL>(rec + 3 * LK, LK, ju);
  wave_lds_sync();

  float acc[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] = 0.f;

  const int RST = a.vhm ? a.D : a.G * a.D;
  const uint32_t lane_elem = (uint32_t)((a.vhm ? 0 : g * a.D) + j * CPL);
  constexpr int kRowBytes = CPL * 4 * (int)sizeof(T);   // 64
  const T *vb = static_cast<const T *>(a.value) +
                (a.vhm ? ((int64_t)b * a.G + g) * (kPairs ? copy_head_rows(a.shapes, a.lsi, L, a.S, kRowBytes) : a.S) * a.D
                       : (int64_t)b * a.S * a.G * a.D);
  constexpr int NW = CPL * (int)sizeof(T) / 4, EPW = Elem<T>::kPerWord;
  for (int l = 0; l < L; ++l) {
    const int Dl = (int)a.shapes[3 * l], Hl = (int)a.shapes[3 * l + 1], Wl = (int)a.shapes[3 * l + 2];
    const CopyLevel cl = kPairs ? copy_level(a.shapes, a.lsi, L, a.S, l, kRowBytes) : CopyLevel{a.lsi[l], false};
    const int64_t rows = cl.paired ? 2 * (int64_t)Dl * Hl * Wl + 2 : (int64_t)Dl * Hl * Wl;
    const uint32_t nbytes = (uint32_t)(rows * RST * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb + cl.start * RST, nbytes);
    // 4 samples per step: lane (ju & 3) of each quad sets up sample k0 + (ju & 3) for its own
    // x-row (4 corner offsets and weights); its quad receives them by DPP broadcast
    for (int k0 = 0; k0 < K; k0 += 4) {
      const int kj = k0 + (ju & 3);
      const int sj = l * K + (kj < K ? kj : K - 1);
      Sample ms;
      sample_setup(rec[3 * sj], rec[3 * sj + 1], rec[3 * sj + 2], Wl, Hl, Dl, RST, ms, MODE == kModeDcn);
      uint32_t off4[4];
      float w4[4];
      // corner weights times the sample's attention weight (made once per set-up, not per channel)
      const float at_s = rec[3 * LK + sj];
      const float wxd = dxl ? ms.wx[1] : ms.wx[0];
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {   // c4 = (dz, dy); this lane's corner c = 2*c4 + dxl
        off4[c4] = live ? (dxl ? ms.off[2 * c4 + 1] : ms.off[2 * c4]) : OOB_ELEM;
        if (cl.paired) off4[c4] = paired_offset(off4[c4], dxl, RST);
        w4[c4] = ((wxd * ms.wy[c4 & 1]) * ms.wz[c4 >> 1]) * at_s;
      }
      static_for<4>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if (k0 + u < K) {
          uint32_t off[4];
          float w[4];
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            off[c4] = unit_bcast<4, u>(off4[c4]);
            w[c4] = __uint_as_float(unit_bcast<4, u>(__float_as_uint(w4[c4])));
          }
          uint32_t v[4][NW];
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4)
            bload<NW * 4>(rv, (off[c4] + lane_elem) * (uint32_t)sizeof(T), v[c4]);
#pragma unroll
          for (int i = 0; i < NW; ++i) {
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
              float f[EPW];
              Elem<T>::unpack(v[c4][i], f);
#pragma unroll
              for (int e = 0; e < EPW; ++e) acc[i * EPW + e] = fmaf(f[e], w[c4], acc[i * EPW + e]);
            }
          }
        }
      });
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] += xor_lane<LPU>(acc[c]);
  if (live && dxl == 0) store_elems<T, CPL>(static_cast<T *>(a.out) + unit * a.D + j * CPL, acc);
}

// Backward phase 1 for rows of 64 bytes (4 lanes x 16 bytes), the x-pair form of the forward's
// pair kernel: a unit has 8 lanes, lanes 0-3 take the x0 row and lanes 4-7 the x0+1 row of each
// corner pair (one 128-byte span per pair), so each lane loads 4 corners per sample.  Sample
// set-ups are made once per quad (lane k of a quad sets up sample k0+k) and broadcast by DPP;
// the lane that made a set-up also records that sample's stash and base corner.  The partials
// of grad_loc / grad_attn of a lane's x-row are summed over the unit's 8 lanes.
template <typename T, int CPL, bool kPairs, int MODE>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kQueryWavesPerEU))) void fda_bwd_query_pair_kernel(const Args a) {
  extern __shared__ float lds[];
  constexpr int UL = 8;
  constexpr int UPW = kWave / UL, UPB = kWavesPerBlock * UPW;
  static_assert(CPL * sizeof(T) == 16, "pair kernel: 16 bytes per lane, 64-byte rows");
  int b, g, qb;
  if (!map_tile(a, blockIdx.x, b, g, qb)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int ju = lane & (UL - 1);   // lane within the unit
  const int j = ju & 3;             // channel chunk
  const int dxl = ju >> 2;          // x-row of the corner pairs this lane loads
  const int ub = wave * UPW + lane / UL;
  const int q = qb * UPB + ub;
  const bool live = q < a.Q;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  const int RS = bwd_query_lds_floats(P, LK);
  float *rec = lds + ub * RS;
  float *gat_s = rec + P;
  float4 *st_s = reinterpret_cast<float4 *>(lds + ub * RS + ((P + LK + 3) & ~3));
  uint32_t *cx_s = reinterpret_cast<uint32_t *>(st_s + LK);
  uint32_t *cy_s = cx_s + LK, *cz_s = cy_s + LK;
  const int64_t unit = ((int64_t)b * a.Q + (live ? q : 0)) * a.G + g;
  __shared__ LevelTiles lvt[5];
  __shared__ uint32_t lvbase[5];
  __shared__ CopyLevel lvcopy[5];   // each level's place in the value rows read (copy_level)
  __shared__ int64_t head_rows;      // rows between heads of the head-major copy
  if (threadIdx.x == 0) {
    if (kPairs) head_rows = copy_levels(a.shapes, a.lsi, L, a.S, CPL * 4 * (int)sizeof(T), lvcopy);
    uint32_t t = 0;   // tile ids within the head
    for (int l = 0; l < L; ++l) {
      lvt[l] = level_tiles(a.shapes, l, a.TX, a.TY, a.TZ);
      lvbase[l] = t;
      t += lvt[l].count;
    }
  }
  __syncthreads();

  stage_record<T, UL>(static_cast<const T *>(a.loc_attn) + record_offset<MODE>(a, unit), P, ju, live, rec);
  wave_lds_sync();
  if constexpr (MODE == kModeOffsets) {
    offsets_to_locations<T, UL>(a, unit / a.G, ju, live, rec);
    wave_lds_sync();
  }
  if constexpr (MODE == kModeDcn) {
    dcn_to_pixels<UL>(a, live ? q : 0, ju, rec);
    wave_lds_sync();
  }
  if (MODE != kModeDcn || a.dcn_softmax) unit_softmax<UL>(rec + 3 * LK, LK, ju);
  wave_lds_sync();

  constexpr int NW = CPL * (int)sizeof(T) / 4;
  uint32_t tgw[NW];
  if (live) {
    load_global_words<NW>(static_cast<const T *>(a.grad_out) + unit * a.D + j * CPL, tgw);
    if (a.gout_hm && dxl == 0) {   // the row again, head-major, for the tile kernel
      uint32_t *dst = reinterpret_cast<uint32_t *>(static_cast<T *>(a.gout_hm) +
                                                   (((int64_t)b * a.G + g) * a.Q + q) * a.D + j * CPL);
#pragma unroll
      for (int c = 0; c < NW; ++c) dst[c] = tgw[c];
    }
  } else {
#pragma unroll
    for (int c = 0; c < NW; ++c) tgw[c] = 0u;
  }

  const int RST = a.vhm ? a.D : a.G * a.D;
  const uint32_t lane_elem = (uint32_t)((a.vhm ? 0 : g * a.D) + j * CPL);
  const T *vb = static_cast<const T *>(a.value) +
                (a.vhm ? ((int64_t)b * a.G + g) * (kPairs ? uniform_i64(head_rows) : (int64_t)a.S) * a.D
                       : (int64_t)b * a.S * a.G * a.D);
  for (int l = 0; l < L; ++l) {
    const int Dl = (int)a.shapes[3 * l], Hl = (int)a.shapes[3 * l + 1], Wl = (int)a.shapes[3 * l + 2];
    const CopyLevel cl = kPairs ? CopyLevel{uniform_i64(lvcopy[l].start),
                                            __builtin_amdgcn_readfirstlane((int)lvcopy[l].paired) != 0}
                                : CopyLevel{a.lsi[l], false};
    const int64_t rows = cl.paired ? 2 * (int64_t)Dl * Hl * Wl + 2 : (int64_t)Dl * Hl * Wl;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb + cl.start * RST, (uint32_t)(rows * RST * (int64_t)sizeof(T)));
    for (int k0 = 0; k0 < K; k0 += 4) {
      // lane k of each quad sets up sample k0 + k (both quads: each needs its own x-row)
      const int kq = k0 + (ju & 3);
      const bool have = kq < K;
      const int sj = l * K + (have ? kq : K - 1);
      Sample ms;
      const bool in_s = sample_setup(rec[3 * sj], rec[3 * sj + 1], rec[3 * sj + 2], Wl, Hl, Dl, RST, ms, MODE == kModeDcn) && live;
      if (dxl == 0 && have) {
        cx_s[sj] = in_s ? (uint32_t)(ms.x0 + 1) : kKeyInvalid;
        cy_s[sj] = (uint32_t)(ms.y0 + 1);
        cz_s[sj] = (uint32_t)(ms.z0 + 1);
        st_s[sj] = make_float4(ms.wx[1], ms.wy[1], ms.wz[1], rec[3 * LK + sj]);
      }
      uint32_t off4[4];
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {   // c4 = (dz, dy); a select, not an index, keeps ms in registers
        off4[c4] = live ? (dxl ? ms.off[2 * c4 + 1] : ms.off[2 * c4]) : OOB_ELEM;
        if (cl.paired) off4[c4] = paired_offset(off4[c4], dxl, RST);
      }
      const float wv[6] = {ms.wx[0], ms.wx[1], ms.wy[0], ms.wy[1], ms.wz[0], ms.wz[1]};
      // all four set-ups are computed (past K they repeat sample K-1), so U and W stay in
      // registers; only the write-back below skips them
      float U[4][4];
      static_for<4>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const uint32_t o = unit_bcast<4, u>(off4[c4]);
          U[u][c4] = dot_elems<T, CPL>(rv, (o + lane_elem) * (uint32_t)sizeof(T), tgw);
        }
      });
      static_for<4>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if (k0 + u < K) {
          float W[6];   // (wx0, wx1, wy0, wy1, wz0, wz1) of sample k0 + u
#pragma unroll
          for (int i = 0; i < 6; ++i) W[i] = __uint_as_float(unit_bcast<4, u>(__float_as_uint(wv[i])));
          const float wxd = dxl ? W[1] : W[0];
          const float sx = dxl ? 1.f : -1.f;
          float gx = 0.f, gy = 0.f, gz = 0.f, ga = 0.f;
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            const int dz = c4 >> 1, dy = c4 & 1;
            const float yz = W[2 + dy] * W[4 + dz];
            ga = fmaf(wxd * yz, U[u][c4], ga);
            gx = fmaf(sx * yz, U[u][c4], gx);
          }
          // d w / dy = (dy ? +1 : -1) * wx * wz, d w / dz = (dz ? +1 : -1) * wx * wy
#pragma unroll
          for (int dz = 0; dz < 2; ++dz) gy = fmaf(wxd * W[4 + dz], U[u][2 * dz + 1] - U[u][2 * dz], gy);
#pragma unroll
          for (int dy = 0; dy < 2; ++dy) gz = fmaf(wxd * W[2 + dy], U[u][2 + dy] - U[u][dy], gz);
          gx = unit_sum<UL>(gx);
          gy = unit_sum<UL>(gy);
          gz = unit_sum<UL>(gz);
          ga = unit_sum<UL>(ga);
          if (ju == 0) {
            const int su = l * K + k0 + u;
            const float at = rec[3 * LK + su];
            // d(pixel)/d(loc) = size (grid_sample: size/2 per unit of grid, grid = 2*loc - 1);
            // offset mode: d(pixel)/d(offset) = 1; DCNv4-3D: d(pixel)/d(offset) = offset_scale
            rec[3 * su] = gx * at * (MODE == kModeDcn ? a.offset_scale : (MODE == kModeOffsets ? 1.f : (float)Wl));
            rec[3 * su + 1] = gy * at * (MODE == kModeDcn ? a.offset_scale : (MODE == kModeOffsets ? 1.f : (float)Hl));
            rec[3 * su + 2] = gz * at * (MODE == kModeDcn ? a.offset_scale : (MODE == kModeOffsets ? 1.f : (float)Dl));
            gat_s[su] = ga;
          }
        }
      });
    }
  }
  wave_lds_sync();
  {
    // the wave's units are consecutive q of one (b, g): their samples are one contiguous range
    const int q0 = qb * UPB + wave * UPW;
    const int nlive = min(UPW, a.Q - q0);
    if (nlive > 0) {
      const uint32_t gs0 = sample_index(b, g, q0, 0, a.G, a.Q, LK);
      const int ntot = nlive * LK;
      for (int e = lane; e < ntot; e += kWave) {
        const int uu = e / LK, ss = e - uu * LK;
        const int ubx = wave * UPW + uu;
        const float4 *stx = reinterpret_cast<const float4 *>(lds + ubx * RS + ((P + LK + 3) & ~3));
        const uint32_t *kx = reinterpret_cast<const uint32_t *>(stx + LK);
        const int l = ss / K;
        const LevelTiles &lt = lvt[l];
        const uint32_t bx = kx[ss];
        const int x0 = (int)bx - 1, y0 = (int)kx[LK + ss] - 1, z0 = (int)kx[2 * LK + ss] - 1;
        const int hz = max(z0, 0) >> lt.sh[0], hy = max(y0, 0) >> lt.sh[1], hx = max(x0, 0) >> lt.sh[2];
        const int lz = z0 - hz * lt.t[0], ly = y0 - hy * lt.t[1], lx = x0 - hx * lt.t[2];
        const uint32_t ex = lx == lt.t[2] - 1 && (hx + 1) * lt.t[2] < lt.n[2];
        const uint32_t ey = ly == lt.t[1] - 1 && (hy + 1) * lt.t[1] < lt.n[1];
        const uint32_t ez = lz == lt.t[0] - 1 && (hz + 1) * lt.t[0] < lt.n[0];
        a.keys[gs0 + e] = bx == kKeyInvalid ? kKeyInvalid
                                            : tile_key(lvbase[l] + (uint32_t)((hz * lt.nt[1] + hy) * lt.nt[2] + hx),
                                                       ex | (ey << 1) | (ez << 2), (uint32_t)l);
        // pixel coordinates = base corner + fraction (exact), from which the tile kernel takes both
        const float4 fr = stx[ss];
        a.stash[gs0 + e] = make_float4((float)x0 + fr.x, (float)y0 + fr.y, (float)z0 + fr.z, fr.w);
      }
    }
  }
  // softmax backward over the unit's L*K attention weights
  float dot = 0.f;
  for (int t = ju; t < LK; t += UL) dot = fmaf(rec[3 * LK + t], gat_s[t], dot);
  dot = unit_sum<UL>(dot);
  const bool raw_mask = MODE == kModeDcn && !a.dcn_softmax;   // DCNv4-3D without softmax: d(mask) = d(attn)
  for (int t = ju; t < LK; t += UL) {
    const float at = rec[3 * LK + t];
    rec[3 * LK + t] = raw_mask ? gat_s[t] : at * (gat_s[t] - dot);
  }
  wave_lds_sync();
  if constexpr (MODE == kModeOffsets)
    if (live && a.grad_ref) add_ref_grad<UL>(a, unit / a.G, ju, rec);
  if (live) write_record<T, UL>(static_cast<T *>(a.grad_loc_attn) + record_offset<MODE>(a, unit), P, ju, rec);
  clear_tile_counts(a);
}

template <typename T, int CPL, int LPU, int MODE>
__global__ __launch_bounds__(kBlock) void fda_bwd_query_kernel(const Args a) {
  extern __shared__ float lds[];
  constexpr int UPW = kWave / LPU, UPB = kWavesPerBlock * UPW;
  int b, g, qb;
  if (!map_tile(a, blockIdx.x, b, g, qb)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int j = lane & (LPU - 1);
  const int ub = wave * UPW + lane / LPU;
  const int q = qb * UPB + ub;
  const bool live = q < a.Q;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  // per unit: [0,P) record (later its gradient), [P,P+LK) grad_attn, then LK stash float4s and
  // the LK base corners (x0+1 or kKeyInvalid, y0+1, z0+1) for the wave's coalesced write-out
  const int RS = bwd_query_lds_floats(P, LK);
  float *rec = lds + ub * RS;
  float *gat_s = rec + P;
  float4 *st_s = reinterpret_cast<float4 *>(lds + ub * RS + ((P + LK + 3) & ~3));
  uint32_t *cx_s = reinterpret_cast<uint32_t *>(st_s + LK);
  uint32_t *cy_s = cx_s + LK, *cz_s = cy_s + LK;
  const int64_t unit = ((int64_t)b * a.Q + (live ? q : 0)) * a.G + g;
  // per level: tile geometry and the id of the level's first tile of this (b, g)
  __shared__ LevelTiles lvt[5];
  __shared__ uint32_t lvbase[5];
  if (threadIdx.x == 0) {
    uint32_t t = 0;   // tile ids within the head
    for (int l = 0; l < L; ++l) {
      lvt[l] = level_tiles(a.shapes, l, a.TX, a.TY, a.TZ);
      lvbase[l] = t;
      t += lvt[l].count;
    }
  }
  __syncthreads();

  stage_record<T, LPU>(static_cast<const T *>(a.loc_attn) + record_offset<MODE>(a, unit), P, j, live, rec);
  wave_lds_sync();
  if constexpr (MODE == kModeOffsets) {
    offsets_to_locations<T, LPU>(a, unit / a.G, j, live, rec);
    wave_lds_sync();
  }
  if constexpr (MODE == kModeDcn) {
    dcn_to_pixels<LPU>(a, live ? q : 0, j, rec);
    wave_lds_sync();
  }
  if (MODE != kModeDcn || a.dcn_softmax) unit_softmax<LPU>(rec + 3 * LK, LK, j);
  wave_lds_sync();

  // the unit's grad_output channels as raw words (dot products run on the packed elements)
  constexpr int NW = CPL * (int)sizeof(T) / 4;
  uint32_t tgw[NW];
  if (live) {
    load_global_words<NW>(static_cast<const T *>(a.grad_out) + unit * a.D + j * CPL, tgw);
    if (a.gout_hm) {   // the row again, head-major, for the tile kernel
      uint32_t *dst = reinterpret_cast<uint32_t *>(static_cast<T *>(a.gout_hm) +
                                                   (((int64_t)b * a.G + g) * a.Q + q) * a.D + j * CPL);
#pragma unroll
      for (int c = 0; c < NW; ++c) dst[c] = tgw[c];
    }
  } else {
#pragma unroll
    for (int c = 0; c < NW; ++c) tgw[c] = 0u;
  }

  const int RST = a.vhm ? a.D : a.G * a.D;
  const uint32_t lane_elem = (uint32_t)((a.vhm ? 0 : g * a.D) + j * CPL);
  const T *vb = static_cast<const T *>(a.value) +
                (a.vhm ? ((int64_t)b * a.G + g) * a.S * a.D : (int64_t)b * a.S * a.G * a.D);
  int s = 0;
  for (int l = 0; l < L; ++l) {
    const int Dl = (int)a.shapes[3 * l], Hl = (int)a.shapes[3 * l + 1], Wl = (int)a.shapes[3 * l + 2];
    const int64_t st = a.lsi[l];
    const int64_t nel = (int64_t)Dl * Hl * Wl * RST;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb + st * RST, (uint32_t)(nel * (int64_t)sizeof(T)));
    // two samples per step: both records are read before either gradient is written back, so
    // the 16 corner loads of the pair are in flight together
    for (int k = 0; k < K; k += 2, s += 2) {
      const int nk = k + 1 < K ? 2 : 1;
      float at[2];
      bool in[2];
      Sample sm[2];
      float U[2][8];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int su = u < nk ? s + u : s;
        const float lx = rec[3 * su], ly = rec[3 * su + 1], lz = rec[3 * su + 2];
        at[u] = rec[3 * LK + su];
        // branch-free: a sample outside the volume (or of a dead unit) loads zeros, weighs zero
        in[u] = sample_setup(lx, ly, lz, Wl, Hl, Dl, RST, sm[u], MODE == kModeDcn) && live && u < nk;
        if (!live || u >= nk) {
#pragma unroll
          for (int c = 0; c < 8; ++c) sm[u].off[c] = OOB_ELEM;
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int c = 0; c < 8; ++c)
          U[u][c] = dot_elems<T, CPL>(rv, (sm[u].off[c] + lane_elem) * (uint32_t)sizeof(T), tgw);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const Sample &m = sm[u];
        float gx = 0.f, gy = 0.f, gz = 0.f, ga = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) ga = fmaf((m.wx[c & 1] * m.wy[(c >> 1) & 1]) * m.wz[c >> 2], U[u][c], ga);
        // d w_c / dx = (dx ? +1 : -1) * wy * wz, and likewise for y, z
#pragma unroll
        for (int zy = 0; zy < 4; ++zy) {
          const int dz = zy >> 1, dy = zy & 1;
          gx = fmaf(m.wy[dy] * m.wz[dz], U[u][4 * dz + 2 * dy + 1] - U[u][4 * dz + 2 * dy], gx);
        }
#pragma unroll
        for (int zx = 0; zx < 4; ++zx) {
          const int dz = zx >> 1, dx = zx & 1;
          gy = fmaf(m.wx[dx] * m.wz[dz], U[u][4 * dz + 2 + dx] - U[u][4 * dz + dx], gy);
        }
#pragma unroll
        for (int yx = 0; yx < 4; ++yx) {
          const int dy = yx >> 1, dx = yx & 1;
          gz = fmaf(m.wx[dx] * m.wy[dy], U[u][4 + 2 * dy + dx] - U[u][2 * dy + dx], gz);
        }
        gx = unit_sum<LPU>(gx);
        gy = unit_sum<LPU>(gy);
        gz = unit_sum<LPU>(gz);
        ga = unit_sum<LPU>(ga);
        if (j == 0 && u < nk) {
          const int su = s + u;
          // d(pixel)/d(loc) = size (grid_sample: size/2 per unit of grid, grid = 2*loc - 1);
          // offset mode: d(pixel)/d(offset) = 1; DCNv4-3D: d(pixel)/d(offset) = offset_scale
          rec[3 * su] = gx * at[u] * (MODE == kModeDcn ? a.offset_scale : (MODE == kModeOffsets ? 1.f : (float)Wl));
          rec[3 * su + 1] = gy * at[u] * (MODE == kModeDcn ? a.offset_scale : (MODE == kModeOffsets ? 1.f : (float)Hl));
          rec[3 * su + 2] = gz * at[u] * (MODE == kModeDcn ? a.offset_scale : (MODE == kModeOffsets ? 1.f : (float)Dl));
          gat_s[su] = ga;
          cx_s[su] = in[u] ? (uint32_t)(m.x0 + 1) : kKeyInvalid;
          cy_s[su] = (uint32_t)(m.y0 + 1);
          cz_s[su] = (uint32_t)(m.z0 + 1);
          st_s[su] = make_float4(m.wx[1], m.wy[1], m.wz[1], at[u]);
        }
      }
    }
    s += K - ((K + 1) & ~1);   // the steps above advanced s by K rounded up to even
  }
  wave_lds_sync();
  {
    // the wave's units are consecutive q of one (b, g): their samples are one contiguous range
    const int q0 = qb * UPB + wave * UPW;
    const int nlive = min(UPW, a.Q - q0);
    if (nlive > 0) {
      const uint32_t gs0 = sample_index(b, g, q0, 0, a.G, a.Q, LK);
      const int ntot = nlive * LK;
      for (int e = lane; e < ntot; e += kWave) {
        const int uu = e / LK, ss = e - uu * LK;
        const int ubx = wave * UPW + uu;
        const float4 *stx = reinterpret_cast<const float4 *>(lds + ubx * RS + ((P + LK + 3) & ~3));
        const uint32_t *kx = reinterpret_cast<const uint32_t *>(stx + LK);
        // home tile: the tile holding corner (max(x0,0), max(y0,0), max(z0,0)); the sample is
        // also listed in the next tile along an axis where its base corner is the tile's last
        // voxel (flags in the tile-local word)
        const int l = ss / K;
        const LevelTiles &lt = lvt[l];
        const uint32_t bx = kx[ss];
        const int x0 = (int)bx - 1, y0 = (int)kx[LK + ss] - 1, z0 = (int)kx[2 * LK + ss] - 1;
        const int hz = max(z0, 0) >> lt.sh[0], hy = max(y0, 0) >> lt.sh[1], hx = max(x0, 0) >> lt.sh[2];
        const int lz = z0 - hz * lt.t[0], ly = y0 - hy * lt.t[1], lx = x0 - hx * lt.t[2];
        const uint32_t ex = lx == lt.t[2] - 1 && (hx + 1) * lt.t[2] < lt.n[2];
        const uint32_t ey = ly == lt.t[1] - 1 && (hy + 1) * lt.t[1] < lt.n[1];
        const uint32_t ez = lz == lt.t[0] - 1 && (hz + 1) * lt.t[0] < lt.n[0];
        a.keys[gs0 + e] = bx == kKeyInvalid ? kKeyInvalid
                                            : tile_key(lvbase[l] + (uint32_t)((hz * lt.nt[1] + hy) * lt.nt[2] + hx),
                                                       ex | (ey << 1) | (ez << 2), (uint32_t)l);
        // pixel coordinates = base corner + fraction (exact), from which the tile kernel takes both
        const float4 fr = stx[ss];
        a.stash[gs0 + e] = make_float4((float)x0 + fr.x, (float)y0 + fr.y, (float)z0 + fr.z, fr.w);
      }
    }
  }
  // softmax backward over the unit's L*K attention weights
  float dot = 0.f;
  for (int t = j; t < LK; t += LPU) dot = fmaf(rec[3 * LK + t], gat_s[t], dot);
  dot = unit_sum<LPU>(dot);
  const bool raw_mask = MODE == kModeDcn && !a.dcn_softmax;   // DCNv4-3D without softmax: d(mask) = d(attn)
  for (int t = j; t < LK; t += LPU) {
    const float at = rec[3 * LK + t];
    rec[3 * LK + t] = raw_mask ? gat_s[t] : at * (gat_s[t] - dot);
  }
  wave_lds_sync();
  if constexpr (MODE == kModeOffsets)
    if (live && a.grad_ref) add_ref_grad<LPU>(a, unit / a.G, j, rec);
  if (live) write_record<T, LPU>(static_cast<T *>(a.grad_loc_attn) + record_offset<MODE>(a, unit), P, j, rec);
  clear_tile_counts(a);
}

// ---------------------------------------------------------------------------------------------
// Backward phase 3, tile-major: grad_value of one tile = for every voxel v of the tile, the sum of
// attn * w_corner * grad_out over the tile's entries (samples) with a corner at v.  A block of
// tile_threads(LPU) threads owns the tile: LPU lanes own an x-pair of voxels (x0, x0+1) and CPL channels,
// and keep their sums in registers.  The tile's entries (sample indices) are processed in chunks:
//   1. each thread takes kTileKPT entries and their stash (pixel coordinates, attention weight),
//      finds the local bin of the base corner (in [-1,tx) x [-1,ty) x [-1,tz)) and counts it
//      (LDS atomics),
//   2. exclusive scan of the bin counts,
//   3. counting sort: each entry's weights (fx, attn*fy, attn*(1-fy), fz) and grad_output row
//      index go to its sorted position in LDS, then the rows are loaded straight into LDS in
//      that order,
//   4. each owner walks the entries of the bins with a corner on its voxels -- for each (dz, dy)
//      the three contiguous bins of base x0-1, x0, x0+1 -- reading only LDS.
// The next chunk's entries and stash are loaded during the current chunk.  Every grad_value row
// of the tile is written once, in T (or added to an fp32 buffer): no zero-fill, no global
// atomics; split tiles (small volumes) write fp32 partials that a combine kernel adds.  Tiles
// are scheduled coarse levels first (their tiles hold the most entries), and with G % 8 == 0
// the tiles of head g run on XCD g % 8, whose L2 then holds that head's grad_output rows.

// Waves per SIMD the tile kernel runs at: its LDS chunk sizing puts three 256-thread blocks, two
// 512-thread blocks or one 1024-thread block on a CU (3, 4, 4 waves per SIMD); compiling for no
// more than that leaves the register allocator all the registers those waves can have.
__host__ __device__ constexpr int tile_wpe(int lpu, bool big) {
  return tile_threads(lpu, big) == 256 ? 3 : 4;
}

template <typename T, int CPL, int LPU, bool BIG>
__global__ __launch_bounds__(tile_threads(LPU, BIG)) __attribute__((amdgpu_waves_per_eu(tile_wpe(LPU, BIG))))
void fda_bwd_tile_kernel(const Args a) {
  constexpr int NT = tile_threads(LPU, BIG);
  extern __shared__ __align__(16) unsigned char tsm[];
  constexpr int EB = CPL * (int)sizeof(T);      // bytes of a lane's channels
  constexpr int NW = EB / 4;
  const int tid = threadIdx.x;
  const int D = a.D, G = a.G, L = a.L;
  constexpr int RB = CPL * LPU * (int)sizeof(T);   // bytes of a grad_output row (D = CPL*LPU)
  const int CH = a.chunk;                          // <= kTileKPT * NT
  const int NBX = (a.TX + 1) * (a.TY + 1) * (a.TZ + 1);
  // a chunk's entries in LDS in bin-sorted order: stash, grad_output row, row index
  float4 *st_l = reinterpret_cast<float4 *>(tsm);
  unsigned char *row_l = tsm + (size_t)CH * 16;
  uint32_t *start_l = reinterpret_cast<uint32_t *>(row_l + (size_t)CH * RB);   // [NBX + 1]
  uint32_t *cur_l = start_l + NBX + 1;                                        // [NBX]
  uint32_t *rowi_l = cur_l + NBX;                                             // [CH]

  // owner: x-pair p of the nominal tile, channel chunk j
  const int p = tid / LPU, j = tid & (LPU - 1);
  const int hxn = a.TX / 2;
  const int px = p % hxn, py = (p / hxn) % a.TY, pz = p / (hxn * a.TY);

  // per level: tile geometry, first tile id within a head, voxel offset (read once)
  __shared__ LevelTiles lvt[5];
  __shared__ uint32_t lvbase[6];
  __shared__ int64_t lvsi[5];
  __shared__ bool queue_l;
  if (tid == 0) {
    uint32_t t = 0;
    for (int u = 0; u < L; ++u) {
      lvt[u] = level_tiles(a.shapes, u, a.TX, a.TY, a.TZ);
      lvbase[u] = t;
      lvsi[u] = a.lsi[u];
      t += lvt[u].count;
    }
    lvbase[L] = t;
    // tile order: a per-XCD work counter after four static tiles when the tiles hold at least a
    // chunk of entries on average, else the static snake order, whose blocks pay no claim per
    // tiny tile (from the first head's entries per tile: the same in every block)
    const uint32_t last = t > 0 ? t - 1 : 0;
    const uint32_t ent = t > 0 ? a.tile_start[last] + a.tile_counts[last] - a.tile_start[0] : 0u;
    queue_l = (uint64_t)ent >= (uint64_t)a.chunk * t;
  }
  __syncthreads();
  const uint32_t T_h = lvbase[L];
  const bool use_queue = queue_l;
  int xcd = 0, bi = blockIdx.x, nbx = gridDim.x, hpx = G;   // heads served by this block's group
  if (a.tile_affinity) {
    xcd = blockIdx.x & 7;
    bi = blockIdx.x >> 3;
    nbx = ((int)gridDim.x - xcd + 7) >> 3;
    hpx = G / 8;
  }
  const uint32_t nbg = (uint32_t)a.B * (uint32_t)hpx;
  const uint32_t total = nbg * T_h;
  // Split tiles: when the group has fewer tiles than twice its blocks, each tile is cut into F
  // parts (jobs) over its entry range; a part sums into fp32 and writes its partial to a scratch
  // slot, and the tile's last part to finish adds the others' partials and writes grad_value.
  const uint32_t ngroups = a.tile_affinity ? 8u : 1u;
  uint32_t F = 1;
  if (a.split_slots > 0 && total > 0 && total < 2u * (uint32_t)nbx) {
    F = min((kSplitTarget * (uint32_t)nbx + total - 1u) / total, kSplitMax);
    F = min(F, a.split_slots / ngroups / total);
    if (F < 1) F = 1;
  }
  const uint32_t njobs = total * F;
  if (blockIdx.x == 0 && tid == 0) a.tile_queue[8] = F;   // for the combine kernel
  const uint32_t gslot = (uint32_t)xcd * (a.split_slots / ngroups);   // the group's first slot
  // part `part` of F of a tile with entries [s0, s0 + c)
  const auto part_range = [&](uint32_t s0, uint32_t c, uint32_t part, uint32_t &hs, uint32_t &hc) {
    const uint32_t lo = (uint32_t)((uint64_t)c * part / F), hi = (uint32_t)((uint64_t)c * (part + 1u) / F);
    hs = s0 + lo;
    hc = hi - lo;
  };
  // grad_output rows in sample order / (L*K): the head-major copy, or grad_out itself (G == 1)
  // grad_output rows: the head-major copy (row = sample / (L*K)), or grad_output itself
  // ([B,Q,G,D]: the row of (b, q, g) is (b*Q + q)*G + g; the same for G == 1)
  const T *go = static_cast<const T *>(a.gout_hm ? a.gout_hm : a.grad_out);
  const bool go_direct = a.gout_hm == nullptr;

  // k -> (level, head, tile), coarse (last) levels first
  const auto decode = [&](uint32_t k, int &l, uint32_t &bgi, uint32_t &t) {
    uint32_t rem = k;
    l = L - 1;
    for (; l > 0; --l) {
      const uint32_t nl = nbg * lvt[l].count;
      if (rem < nl) break;
      rem -= nl;
    }
    bgi = rem / lvt[l].count;
    t = rem - bgi * lvt[l].count;
  };
  const auto head_of = [&](uint32_t bgi, int &b, int &g) {
    b = (int)(bgi / (uint32_t)hpx);
    g = a.tile_affinity ? xcd + 8 * (int)(bgi % (uint32_t)hpx) : (int)(bgi % (uint32_t)hpx);
  };
  const auto tile_gid = [&](uint32_t k) {
    int l, b, g;
    uint32_t bgi, t;
    decode(k, l, bgi, t);
    head_of(bgi, b, g);
    return (uint32_t)(b * G + g) * T_h + lvbase[l] + t;
  };
  // Tiles: the block's first four are bi + j nbx (j < 4); after them each block takes the next
  // unclaimed tile of its XCD group from a work counter (one atomic per tile, made four tiles
  // ahead and read three ahead, so its round trip hides behind a whole tile even when tiles are
  // tiny), so blocks that drew light tiles take more of them.
  // Software pipeline: the entries of the block's next chunk are loaded when a chunk starts and
  // their stash once its rows have arrived, so the stash arrives during the owner phase; tile
  // headers (first entry, count) are loaded two tiles before they are read.
  __shared__ uint32_t grab_l[4];   // claim made at tile position p in slot p & 3 (~0u: none)
  // Tile headers (first entry, count) live in a 4-slot LDS ring indexed by the tile's position in
  // the block's sequence.  Thread 0 loads the header of the tile two ahead into registers at the
  // end of a tile and writes it to the ring only where its wave has waited for its row loads
  // anyway (end of an owner phase), so no wave waits for it; the block reads it a tile later.
  __shared__ uint32_t hdr_l[4][2];
  uint32_t k1 = (uint32_t)bi + (uint32_t)nbx, k2 = k1 + (uint32_t)nbx;   // the next two tiles
  if (!use_queue) {
    k1 = 2u * (uint32_t)nbx - 1u - (uint32_t)bi;
    k2 = 2u * (uint32_t)nbx + (uint32_t)bi;
  }
  // header of k2 (thread 0: the tile's first entry and count, and k2's part), not yet in the ring
  uint32_t hs_pend = 0, hc_pend = 0, hp_pend = 0;
  if (tid == 0) {
    const uint32_t kk[2] = {(uint32_t)bi, k1};
    for (int i = 0; i < 2; ++i) {
      uint32_t hs = 0u, hc = 0u;
      if (kk[i] < njobs) {
        const uint32_t gid = tile_gid(kk[i] / F);
        part_range(a.tile_start[gid], a.tile_counts[gid], kk[i] % F, hs, hc);
      }
      hdr_l[i][0] = hs;
      hdr_l[i][1] = hc;
    }
    if (k2 < njobs) {
      const uint32_t gid = tile_gid(k2 / F);
      hs_pend = a.tile_start[gid];
      hc_pend = a.tile_counts[gid];
      hp_pend = k2 % F;
    }
  }
  for (int i = tid; i < NBX; i += NT) cur_l[i] = 0u;   // bin counters of the first chunk
  __syncthreads();
  uint32_t pos = 0;   // position of the current tile in the block's sequence
  // the work counter's value claimed for the current tile (thread 0; declared outside the tile
  // loop so that no per-tile re-initialisation waits for the previous atomic's return)
  uint32_t taken = 0;
  bool pf = false;               // the current chunk's entries and stash are in pE / pS
  uint32_t pE[kTileKPT];
  float4 pS[kTileKPT];
#pragma unroll
  for (int e = 0; e < kTileKPT; ++e) {
    pE[e] = 0u;
    pS[e] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (uint32_t k = (uint32_t)bi; k < njobs;) {
    // claim the job of position pos + 4 (if pos + 2 exists, the queue may still hold jobs);
    // thread 0 publishes the claim in LDS only before the owner phase's closing barrier (so no
    // wave waits for the atomic), and the block reads it at the end of the next job
    const bool claimed = use_queue && k2 < njobs;
    if (claimed && tid == 0) taken = atomicAdd(a.tile_queue + xcd, 1u);
    const uint32_t ktile = k / F, part = k - ktile * F;
    int l, b, g;
    uint32_t bgi, t;
    decode(ktile, l, bgi, t);
    head_of(bgi, b, g);
    const uint32_t row0 = ((uint32_t)b * (uint32_t)G + (uint32_t)g) * (uint32_t)a.Q;   // the head's first sample row
    const LevelTiles lt = lvt[l];
    const int itx = (int)(t % (uint32_t)lt.nt[2]);
    const int ity = (int)((t / (uint32_t)lt.nt[2]) % (uint32_t)lt.nt[1]);
    const int itz = (int)(t / ((uint32_t)lt.nt[2] * (uint32_t)lt.nt[1]));
    const int tz = lt.t[0], ty = lt.t[1], tx = lt.t[2];
    const int Dl = lt.n[0], Hl = lt.n[1], Wl = lt.n[2];
    const int z = itz * tz + pz, y = ity * ty + py, x0 = itx * tx + 2 * px;
    const bool live = 2 * px < tx && py < ty && pz < tz && z < Dl && y < Hl && x0 < Wl;
    const bool two = 2 * px + 1 < tx && x0 + 1 < Wl;
    const uint32_t e0 = hdr_l[pos & 3u][0], e1 = e0 + hdr_l[pos & 3u][1];
    const uint32_t ns = hdr_l[(pos + 1u) & 3u][0], nc = hdr_l[(pos + 1u) & 3u][1];   // next tile's
    const int TXp = tx + 1, TYp = ty + 1;
    const int nb = TXp * TYp * (tz + 1);

    float acc0[CPL], acc1[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc0[c] = acc1[c] = 0.f;

    for (uint32_t c0 = e0; c0 < e1; c0 += (uint32_t)CH) {
      const int n = (int)min((uint32_t)CH, e1 - c0);
      constexpr int KPT = kTileKPT;   // entries per thread and chunk (registers)
      // this chunk's entries and stash (prefetched, or loaded now); an absent entry reads entry 0
      // (unconditional loads keep everything in registers)
      uint32_t en[KPT];
      float4 st[KPT];
      if (pf) {
#pragma unroll
        for (int e = 0; e < KPT; ++e) {
          en[e] = pE[e];
          st[e] = pS[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < KPT; ++e) en[e] = a.entries[c0 + (tid + e * NT < n ? tid + e * NT : 0)];
#pragma unroll
        for (int e = 0; e < KPT; ++e) st[e] = a.stash[en[e]];
        // wait here, so that after the two paths join nothing of this one is pending: the
        // prefetched path must not wait for the stores and claims issued since its loads
        __builtin_amdgcn_s_waitcnt(0);
      }
      // the next chunk: the rest of this tile, or the next tile's first chunk
      const bool nxt_here = c0 + (uint32_t)CH < e1;
      const uint32_t nc0 = nxt_here ? c0 + (uint32_t)CH : ns;
      const uint32_t nn = nxt_here ? min((uint32_t)CH, e1 - nc0) : min((uint32_t)CH, nc);
      const bool npf = nxt_here || (k1 < njobs && nc > 0);
      // (the bin counters are zero here: cleared at the start and after every owner phase)
      // 1a. local bin of each entry's base corner, grad_output row index, bin counts.  The stash
      // holds the pixel coordinates: base corner = floor, fraction = coordinate - floor (exact).
      const int ox = itx * tx - 1, oy = ity * ty - 1, oz = itz * tz - 1;   // bin 0 = local -1
      uint32_t lb[KPT], ri[KPT];
#pragma unroll
      for (int e = 0; e < KPT; ++e) {
        const float xf = floorf(st[e].x), yf = floorf(st[e].y), zf = floorf(st[e].z);
        lb[e] = ((uint32_t)((int)zf - oz) * (uint32_t)TYp + (uint32_t)((int)yf - oy)) * (uint32_t)TXp +
                (uint32_t)((int)xf - ox);
        // LDS record: (fx, attn*fy, attn*(1-fy), fz) -- the owner loop's y weight is static per
        // (dz, dy) row, so it picks one of the two products
        const float fx = st[e].x - xf, fy = st[e].y - yf, fz = st[e].z - zf, at = st[e].w;
        st[e] = make_float4(fx, at * fy, at * (1.f - fy), fz);
        ri[e] = (uint32_t)(((double)en[e] + 0.5) * a.inv_lk);   // sample / (L*K), exact
        if (go_direct) ri[e] = ((uint32_t)b * (uint32_t)a.Q + (ri[e] - row0)) * (uint32_t)G + (uint32_t)g;
        if (tid + e * NT < n) atomicAdd(&cur_l[lb[e]], 1u);
      }
      // the next chunk's entries, issued after this chunk's stash is used (loads complete in order,
      // so a wait for the stash would also wait for them; the scheduling barrier keeps them here)
      __builtin_amdgcn_sched_barrier(0);
      if (npf) {
#pragma unroll
        for (int e = 0; e < KPT; ++e)
          pE[e] = a.entries[nc0 + ((uint32_t)(tid + e * NT) < nn ? (uint32_t)(tid + e * NT) : 0u)];
      }
      __syncthreads();
      // 2. bin starts, by wave 0 alone (one barrier): lane k scans bins [k*per, (k+1)*per)
      if (tid < kWave) {
        const int per = (nb + kWave - 1) / kWave;
        const int b0 = tid * per;
        uint32_t sum = 0;
        for (int i = 0; i < per; ++i)
          if (b0 + i < nb) sum += cur_l[b0 + i];
        uint32_t run = wave_inclusive_scan(sum) - sum;
        for (int i = 0; i < per; ++i)
          if (b0 + i < nb) {
            const uint32_t c = cur_l[b0 + i];
            start_l[b0 + i] = run;
            cur_l[b0 + i] = run;
            run += c;
          }
        if (tid == 0) start_l[nb] = (uint32_t)n;
      }
      __syncthreads();
      // 3. counting sort by bin: each entry's stash and row index go to its sorted position
#pragma unroll
      for (int e = 0; e < KPT; ++e)
        if (tid + e * NT < n) {
          const uint32_t pos = atomicAdd(&cur_l[lb[e]], 1u);
          st_l[pos] = st[e];
          rowi_l[pos] = ri[e];
        }
      __syncthreads();
      // 3b. grad_output rows into LDS in sorted order: 16-byte pieces loaded by the memory unit
      // straight into LDS (global_load_lds_dwordx4: lane k of a wave fills base + 16*k), no
      // registers held; piece i is part i % PPR of the row of sorted entry i / PPR.  A wave's
      // last instruction may fill pieces past n*PPR with copies of the last piece: they stay
      // inside the chunk's row buffer (CH * PPR is a multiple of 64) and are never read.
      {
        constexpr int PPR = RB / 16;                 // pieces per row
        const int np = n * PPR;
        const int lane = tid & (kWave - 1);
        for (int base = tid - lane; base < np; base += NT) {
          const int i = min(base + lane, np - 1);
          const int e = i / PPR, q = i - e * PPR;
          const u32x4 *src = reinterpret_cast<const u32x4 *>(go + (size_t)rowi_l[e] * (uint32_t)D) + q;
          __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(row_l + (size_t)base * 16),
                                           16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);   // the pieces are in LDS before the barrier below
      }
      __syncthreads();
      // The next chunk's stash, issued now, after the row loads' wait: it arrives during the owner
      // phase, which no wait ends (the next wait is the next chunk's).  Issued before the row
      // loads, it was waited for with them (c4 tile kernel 250 -> 241 us, c5 2932 -> 2841 us).
      // Touching the next chunk's grad_output rows here as well, so that their sorted loads would
      // find them in L2, was slower (c4 +10 us, c5 +700 us: the touches compete with the misses).
      if (npf) {
#pragma unroll
        for (int e = 0; e < KPT; ++e) pS[e] = a.stash[pE[e]];
      }
      pf = npf;
      // 4. owners gather from LDS
      if (live) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int dz = r >> 1, dy = r & 1;
          // bins of base (x0-1, x0, x0+1) at (y-dy, z-dz): local +1-shifted x index 2*px
          const int rb = ((pz - dz + 1) * TYp + (py - dy + 1)) * TXp + 2 * px;
          const uint32_t s0 = start_l[rb], m1 = start_l[rb + 1], m2 = start_l[rb + 2];
          const uint32_t s3 = two ? start_l[rb + 3] : m2;
#pragma unroll 2
          for (uint32_t i = s0; i < s3; ++i) {
            const float4 st = st_l[i];
            uint32_t wv[NW];
            const uint32_t *rw = reinterpret_cast<const uint32_t *>(row_l + (size_t)i * RB + j * EB);
#pragma unroll
            for (int q = 0; q < NW; ++q) wv[q] = rw[q];
            float tg[CPL];
#pragma unroll
            for (int q = 0; q < NW; ++q) Elem<T>::unpack(wv[q], tg + q * Elem<T>::kPerWord);
            const float ay = dy ? st.y : st.z;          // attn * (y weight)
            const float wz = dz ? st.w : 1.f - st.w;
            const float ayz = ay * wz;
            // base x0-1: (x0, dx=1); base x0: (x0, dx=0), (x0+1, dx=1); base x0+1: (x0+1, dx=0)
            const bool lft = i < m1, ctr = i < m2;
            const float fx = st.x, gx = 1.f - st.x;
            const float aw0 = ayz * (lft ? fx : (ctr ? gx : 0.f));
            const float aw1 = ayz * (lft ? 0.f : (ctr ? fx : gx));
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
              acc0[c] = fmaf(aw0, tg[c], acc0[c]);
              acc1[c] = fmaf(aw1, tg[c], acc1[c]);
            }
          }
        }
      }
      // the owners do not read the bin counters: clear them for the next chunk before the barrier
      for (int i = tid; i < NBX; i += NT) cur_l[i] = 0u;
      if (tid == 0) {
        grab_l[pos & 3u] = claimed ? taken : ~0u;
        uint32_t hs, hc;
        part_range(hs_pend, hc_pend, hp_pend, hs, hc);
        hdr_l[(pos + 2u) & 3u][0] = hs;
        hdr_l[(pos + 2u) & 3u][1] = hc;
      }
      __syncthreads();
    }
    if (F > 1) {
      // this part's sums go to its scratch slot (voxels of the nominal tile: pair p, x-half h);
      // fda_bwd_split_combine_kernel adds a tile's parts and writes its rows
      constexpr int kTileVox = 2 * (NT / LPU);
      float *sl = a.split_scratch + ((size_t)(gslot + ktile * F + part) * kTileVox + (size_t)p * 2u) * (uint32_t)D +
                  (uint32_t)(j * CPL);
      if (live) {
        store_elems<float, CPL>(sl, acc0);
        if (two) store_elems<float, CPL>(sl + D, acc1);
      }
    }
    if (live && F == 1) {
      const int64_t vox = lvsi[l] + ((int64_t)z * Hl + y) * Wl + x0;
      const int64_t o = (((int64_t)b * a.S + vox) * G + g) * D + j * CPL;
      for (int h = 0; h < (two ? 2 : 1); ++h) {
        float res[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) res[c] = h ? acc1[c] : acc0[c];
        const int64_t oh = o + (int64_t)h * G * D;
        if (a.accumulate) {   // caller-owned fp32 buffer: add to what it holds (sole owner, no atomics)
          float *dst = static_cast<float *>(a.out) + oh;
          float old[CPL];
          load_global_elems<float, CPL>(dst, old);
#pragma unroll
          for (int c = 0; c < CPL; ++c) res[c] += old[c];
          store_elems<float, CPL>(dst, res);
        } else {
          store_elems<T, CPL>(static_cast<T *>(a.out) + oh, res);
        }
      }
    }
    if (e0 == e1) {   // no chunk: publish the claim here
      if (tid == 0) {
        grab_l[pos & 3u] = claimed ? taken : ~0u;
        uint32_t hs, hc;
        part_range(hs_pend, hc_pend, hp_pend, hs, hc);
        hdr_l[(pos + 2u) & 3u][0] = hs;
        hdr_l[(pos + 2u) & 3u][1] = hc;
      }
      __syncthreads();
    }
    uint32_t k3;   // the tile of position pos + 3
    if (use_queue) {
      if (pos == 0) {
        k3 = (uint32_t)bi + 3u * (uint32_t)nbx;
      } else {   // claimed at the previous job
        const uint32_t raw = grab_l[(pos - 1u) & 3u];
        k3 = raw == ~0u ? njobs : 4u * (uint32_t)nbx + raw;
      }
      if (k3 >= njobs) k3 = njobs;
    } else {   // static snake order: position p takes p*nbx + (p odd ? nbx-1-bi : bi)
      const uint32_t p3 = pos + 3u;
      k3 = p3 * (uint32_t)nbx + ((p3 & 1u) ? (uint32_t)(nbx - 1 - bi) : (uint32_t)bi);
      if (k3 >= njobs) k3 = njobs;
    }
    if (tid == 0 && k3 < njobs) {
      const uint32_t gid = tile_gid(k3 / F);
      hs_pend = a.tile_start[gid];
      hc_pend = a.tile_counts[gid];
      hp_pend = k3 % F;
    }
    k = k1; k1 = k2; k2 = k3;
    ++pos;
  }
}

// Split tiles (see the tile kernel): one block per tile of every group adds the F parts'
// partial sums of each of its voxels and writes the rows (in T, or added to the caller's fp32
// buffer).  Runs after the tile kernel, so plain loads see the parts; exits when F == 1.
template <typename T, int CPL, int LPU, bool BIG>
__global__ __launch_bounds__(tile_threads(LPU, BIG)) void fda_bwd_split_combine_kernel(const Args a) {
  constexpr int NT = tile_threads(LPU, BIG);
  constexpr int kTileVox = 2 * (NT / LPU);
  const uint32_t F = a.tile_queue[8];
  if (F <= 1) return;
  const int tid = threadIdx.x, D = a.D, G = a.G, L = a.L;
  const int p = tid / LPU, j = tid & (LPU - 1);
  const int hxn = a.TX / 2;
  const int px = p % hxn, py = (p / hxn) % a.TY, pz = p / (hxn * a.TY);
  const uint32_t T_h = tiles_per_head(a.shapes, L, a.TX, a.TY, a.TZ);
  const uint32_t ngroups = a.tile_affinity ? 8u : 1u;
  const int hpx = a.tile_affinity ? G / 8 : G;
  const uint32_t nbg = (uint32_t)a.B * (uint32_t)hpx, total = nbg * T_h;
  const uint32_t xcd = blockIdx.x % ngroups, k = blockIdx.x / ngroups;   // tile k of group xcd
  if (k >= total) return;
  // k -> (level, head, tile) as in the tile kernel: coarse (last) levels first
  uint32_t rem = k;
  int l = L - 1;
  for (; l > 0; --l) {
    const uint32_t nl = nbg * level_tiles(a.shapes, l, a.TX, a.TY, a.TZ).count;
    if (rem < nl) break;
    rem -= nl;
  }
  const LevelTiles lt = level_tiles(a.shapes, l, a.TX, a.TY, a.TZ);
  const uint32_t bgi = rem / lt.count, t = rem - bgi * lt.count;
  const int b = (int)(bgi / (uint32_t)hpx);
  const int g = a.tile_affinity ? (int)xcd + 8 * (int)(bgi % (uint32_t)hpx) : (int)(bgi % (uint32_t)hpx);
  const int itx = (int)(t % (uint32_t)lt.nt[2]);
  const int ity = (int)((t / (uint32_t)lt.nt[2]) % (uint32_t)lt.nt[1]);
  const int itz = (int)(t / ((uint32_t)lt.nt[2] * (uint32_t)lt.nt[1]));
  const int z = itz * lt.t[0] + pz, y = ity * lt.t[1] + py, x0 = itx * lt.t[2] + 2 * px;
  const bool live = 2 * px < lt.t[2] && py < lt.t[1] && pz < lt.t[0] && z < lt.n[0] && y < lt.n[1] && x0 < lt.n[2];
  if (!live) return;
  const bool two = 2 * px + 1 < lt.t[2] && x0 + 1 < lt.n[2];
  const uint32_t gslot = xcd * (a.split_slots / ngroups);
  const float *sl = a.split_scratch + ((size_t)(gslot + k * F) * kTileVox + (size_t)p * 2u) * (uint32_t)D +
                    (uint32_t)(j * CPL);
  float acc0[CPL], acc1[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc0[c] = acc1[c] = 0.f;
  for (uint32_t q = 0; q < F; ++q) {
    float o0[CPL], o1[CPL];
    const float *sq = sl + (size_t)q * kTileVox * D;
    load_global_elems<float, CPL>(sq, o0);
    load_global_elems<float, CPL>(two ? sq + D : sq, o1);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      acc0[c] += o0[c];
      acc1[c] += two ? o1[c] : 0.f;
    }
  }
  const int64_t vox = a.lsi[l] + ((int64_t)z * lt.n[1] + y) * lt.n[2] + x0;
  const int64_t o = (((int64_t)b * a.S + vox) * G + g) * D + j * CPL;
  for (int h = 0; h < (two ? 2 : 1); ++h) {
    float res[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) res[c] = h ? acc1[c] : acc0[c];
    const int64_t oh = o + (int64_t)h * G * D;
    if (a.accumulate) {
      float *dst = static_cast<float *>(a.out) + oh;
      float old[CPL];
      load_global_elems<float, CPL>(dst, old);
#pragma unroll
      for (int c = 0; c < CPL; ++c) res[c] += old[c];
      store_elems<float, CPL>(dst, res);
    } else {
      store_elems<T, CPL>(static_cast<T *>(a.out) + oh, res);
    }
  }
}

// which: 0 forward, 1 backward phase 1 (query-major), 2 backward phase 3 (tile-major)
template <typename T, int CPL, int LPU, int MODE>
void launch_query_major(int which, const Args &a, unsigned grid, size_t lds, hipStream_t st) {
  if (which == 0) {
    if constexpr (fwd_pairs(CPL, LPU, (int)sizeof(T))) {
      if (a.pair_levels)
        hipLaunchKernelGGL((fda_forward_pair_kernel<T, CPL, true, MODE>), dim3(grid), dim3(kBlock), lds, st, a);
      else
        hipLaunchKernelGGL((fda_forward_pair_kernel<T, CPL, false, MODE>), dim3(grid), dim3(kBlock), lds, st, a);
    } else {
      hipLaunchKernelGGL((fda_forward_kernel<T, CPL, LPU, MODE>), dim3(grid), dim3(kBlock), lds, st, a);
    }
  } else {
    if constexpr (fwd_pairs(CPL, LPU, (int)sizeof(T))) {
      if (a.pair_levels)
        hipLaunchKernelGGL((fda_bwd_query_pair_kernel<T, CPL, true, MODE>), dim3(grid), dim3(kBlock), lds, st, a);
      else
        hipLaunchKernelGGL((fda_bwd_query_pair_kernel<T, CPL, false, MODE>), dim3(grid), dim3(kBlock), lds, st, a);
    } else {
      hipLaunchKernelGGL((fda_bwd_query_kernel<T, CPL, LPU, MODE>), dim3(grid), dim3(kBlock), lds, st, a);
    }
  }
}

// which: 0 forward, 1 backward phase 1 (query-major), 2 backward phase 3 (tile-major),
// 3 split-tile combine
template <typename T, int CPL, int LPU>
hipError_t launch_one(int which, const Args &a, unsigned grid, size_t lds, hipStream_t st) {
  if (which == 0 || which == 1) {
    if (a.dcn) launch_query_major<T, CPL, LPU, kModeDcn>(which, a, grid, lds, st);
    else if (a.ref) launch_query_major<T, CPL, LPU, kModeOffsets>(which, a, grid, lds, st);
    else launch_query_major<T, CPL, LPU, kModePlain>(which, a, grid, lds, st);
  }
  else if (which == 3) {
    // one block per tile of every group (`grid` = the bound on tiles times the groups)
    constexpr int TL = tile_lanes(LPU, CPL * (int)sizeof(T)), TC = CPL * LPU / TL;
    if (a.big_tiles)
      hipLaunchKernelGGL((fda_bwd_split_combine_kernel<T, TC, TL, true>), dim3(grid), dim3(tile_threads(TL, true)), 0,
                         st, a);
    else
      hipLaunchKernelGGL((fda_bwd_split_combine_kernel<T, TC, TL, false>), dim3(grid), dim3(tile_threads(TL)), 0, st,
                         a);
  }
  else {
    // persistent: `grid` (the CU count, a multiple of 8 with XCD affinity) times the blocks that
    // fit on a CU at once
    // tile lanes per x-pair: half of LPU, twice the channels per lane
    constexpr int TL = tile_lanes(LPU, CPL * (int)sizeof(T)), TC = CPL * LPU / TL;
    const auto run = [&](auto kern, int nt) {
      int occ = 1;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, nt, lds) != hipSuccess || occ < 1) occ = 1;
      hipLaunchKernelGGL(kern, dim3(grid * (unsigned)occ), dim3(nt), lds, st, a);
    };
    if (a.big_tiles)
      run(fda_bwd_tile_kernel<T, TC, TL, true>, tile_threads(TL, true));
    else
      run(fda_bwd_tile_kernel<T, TC, TL, false>, tile_threads(TL));
  }
  return hipGetLastError();
}

template <typename T, int CPL>
hipError_t launch_cpl(int which, int lpu, const Args &a, unsigned grid, size_t lds, hipStream_t st) {
  switch (lpu) {
    case 1: return launch_one<T, CPL, 1>(which, a, grid, lds, st);
    case 2: return launch_one<T, CPL, 2>(which, a, grid, lds, st);
    case 4: return launch_one<T, CPL, 4>(which, a, grid, lds, st);
    case 8: return launch_one<T, CPL, 8>(which, a, grid, lds, st);
    case 16: return launch_one<T, CPL, 16>(which, a, grid, lds, st);
    case 32: return launch_one<T, CPL, 32>(which, a, grid, lds, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ops3d_fda
