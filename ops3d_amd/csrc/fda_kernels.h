// gfx950 forward and backward kernels of Flash Deformable 3D Attention.
//
// Forward (replaces forward_kernel_reg, reference csrc/cuda/flash_deform_im2col_cuda.cuh:190-295):
//   out[b,q,g,:] = sum_{l,k} softmax(logits[b,q,g,:])[l,k] *
//                  trilinear(value_l[b,:,g,:], pixel(loc[b,q,g,l,k]))
// Backward (replaces backward_kernel_warp_primitive, flash_deform_col2im_cuda.cuh:248-429, and
// ms_deform_attn_col2im_trilinear, common.h:141-353), in two kernels around a sort:
//   phase 1 (query-major)  grad_loc  = attn * size * sum_c grad_out[c] * d(interp_c)/d(pixel)
//                          grad_attn = sum_c grad_out[c] * interp_c, then softmax backward
//                          grad_logit_i = a_i * (grad_attn_i - sum_j a_j grad_attn_j)
//                          + per sample: key = bin of its base corner, stash (fx,fy,fz,attn)
//   phase 2                stable radix sort of (key, sample) pairs
//   phase 3 (voxel-major)  grad_value[v] = sum over samples s with a corner at v of
//                          attn_s * w_corner(s) * grad_out[unit(s)]     (register sums, no atomics)
// The per-sample location/attention partials are formed from U_i = sum_c grad_out[c] * V_i[c]
// (one dot product per corner) so the channel loop costs one FMA per corner and channel, and
// are summed over the unit's LPU lanes with DPP / ds_swizzle reductions.
#pragma once

#include "fda_device.h"

#ifndef OPS3D_FDA_VALUE_REVERSE
#define OPS3D_FDA_VALUE_REVERSE 1
#endif
#ifndef OPS3D_FDA_VALUE_BALANCED
#define OPS3D_FDA_VALUE_BALANCED 1
#endif
#ifndef OPS3D_FDA_VALUE_UNROLL
#define OPS3D_FDA_VALUE_UNROLL 2
#endif

namespace ops3d_fda {

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
template <typename T, int CPL, int LPU>
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

  stage_record<T, LPU>(static_cast<const T *>(a.loc_attn) + unit * P, P, j, live, rec);
  wave_lds_sync();
  unit_softmax<LPU>(rec + 3 * LK, LK, j);
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
      sample_setup(rec[3 * sj], rec[3 * sj + 1], rec[3 * sj + 2], Wl, Hl, Dl, RST, ms);
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
template <typename T, int CPL>
__global__ __launch_bounds__(kBlock) void fda_forward_pair_kernel(const Args a) {
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

  stage_record<T, UL>(static_cast<const T *>(a.loc_attn) + unit * P, P, ju, live, rec);
  wave_lds_sync();
  unit_softmax<UL>(rec + 3 * LK, LK, ju);
  wave_lds_sync();

  float acc[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] = 0.f;

  const int RST = a.vhm ? a.D : a.G * a.D;
  const uint32_t lane_elem = (uint32_t)((a.vhm ? 0 : g * a.D) + j * CPL);
  const T *vb = static_cast<const T *>(a.value) +
                (a.vhm ? ((int64_t)b * a.G + g) * a.S * a.D : (int64_t)b * a.S * a.G * a.D);
  constexpr int NW = CPL * (int)sizeof(T) / 4, EPW = Elem<T>::kPerWord;
  for (int l = 0; l < L; ++l) {
    const int Dl = (int)a.shapes[3 * l], Hl = (int)a.shapes[3 * l + 1], Wl = (int)a.shapes[3 * l + 2];
    const int64_t st = a.lsi[l];
    const uint32_t nbytes = (uint32_t)((int64_t)Dl * Hl * Wl * RST * (int64_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb + st * RST, nbytes);
    // 4 samples per step: lane (ju & 3) of each quad sets up sample k0 + (ju & 3) for its own
    // x-row (4 corner offsets and weights); its quad receives them by DPP broadcast
    for (int k0 = 0; k0 < K; k0 += 4) {
      const int kj = k0 + (ju & 3);
      const int sj = l * K + (kj < K ? kj : K - 1);
      Sample ms;
      sample_setup(rec[3 * sj], rec[3 * sj + 1], rec[3 * sj + 2], Wl, Hl, Dl, RST, ms);
      uint32_t off4[4];
      float w4[4];
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {   // c4 = (dz, dy); this lane's corner c = 2*c4 + dxl
        off4[c4] = live ? (dxl ? ms.off[2 * c4 + 1] : ms.off[2 * c4]) : OOB_ELEM;
        w4[c4] = (ms.wx[dxl] * ms.wy[c4 & 1]) * ms.wz[c4 >> 1];
      }
      const uint32_t at_mine = __float_as_uint(rec[3 * LK + sj]);
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
          const float at = __uint_as_float(unit_bcast<4, u>(at_mine));
          uint32_t v[4][NW];
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4)
            bload<NW * 4>(rv, (off[c4] + lane_elem) * (uint32_t)sizeof(T), v[c4]);
#pragma unroll
          for (int i = 0; i < NW; ++i) {
            float t[EPW], f[EPW];
            Elem<T>::unpack(v[0][i], f);
#pragma unroll
            for (int e = 0; e < EPW; ++e) t[e] = f[e] * w[0];
#pragma unroll
            for (int c4 = 1; c4 < 4; ++c4) {
              Elem<T>::unpack(v[c4][i], f);
#pragma unroll
              for (int e = 0; e < EPW; ++e) t[e] = fmaf(f[e], w[c4], t[e]);
            }
#pragma unroll
            for (int e = 0; e < EPW; ++e) acc[i * EPW + e] = fmaf(at, t[e], acc[i * EPW + e]);
          }
        }
      });
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] += xor_lane<LPU>(acc[c]);
  if (live && dxl == 0) store_elems<T, CPL>(static_cast<T *>(a.out) + unit * a.D + j * CPL, acc);
}

template <typename T, int CPL, int LPU>
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
  // per unit: [0,P) record (later its gradient), [P,P+LK) grad_attn, then LK stash float4s
  // and LK keys for the wave's coalesced write-out
  const int RS = bwd_query_lds_floats(P, LK);
  float *rec = lds + ub * RS;
  float *gat_s = rec + P;
  float4 *st_s = reinterpret_cast<float4 *>(lds + ub * RS + ((P + LK + 3) & ~3));
  uint32_t *key_s = reinterpret_cast<uint32_t *>(st_s + LK);
  const int64_t unit = ((int64_t)b * a.Q + (live ? q : 0)) * a.G + g;

  stage_record<T, LPU>(static_cast<const T *>(a.loc_attn) + unit * P, P, j, live, rec);
  wave_lds_sync();
  unit_softmax<LPU>(rec + 3 * LK, LK, j);
  wave_lds_sync();

  // the unit's grad_output channels as raw words (dot products run on the packed elements)
  constexpr int NW = CPL * (int)sizeof(T) / 4;
  uint32_t tgw[NW];
  if (live) {
    const int64_t grow = a.ghm ? ((int64_t)b * a.G + g) * a.Q + q : unit;
    load_global_words<NW>(static_cast<const T *>(a.grad_out) + grow * a.D + j * CPL, tgw);
  } else {
#pragma unroll
    for (int c = 0; c < NW; ++c) tgw[c] = 0u;
  }

  uint32_t bins_bg = 0;
  for (int l = 0; l < L; ++l) bins_bg += level_bins(a.shapes, l);
  uint32_t bin_base = (uint32_t)(b * a.G + g) * bins_bg;

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
        in[u] = sample_setup(lx, ly, lz, Wl, Hl, Dl, RST, sm[u]) && live && u < nk;
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
          // d(pixel)/d(loc) = size (grid_sample: size/2 per unit of grid, grid = 2*loc - 1)
          rec[3 * su] = gx * at[u] * (float)Wl;
          rec[3 * su + 1] = gy * at[u] * (float)Hl;
          rec[3 * su + 2] = gz * at[u] * (float)Dl;
          gat_s[su] = ga;
          key_s[su] = in[u] ? bin_base + (uint32_t)(((m.z0 + 1) * (Hl + 1) + (m.y0 + 1)) * (Wl + 1) + (m.x0 + 1))
                            : a.key_invalid;
          st_s[su] = make_float4(m.wx[1], m.wy[1], m.wz[1], at[u]);
        }
      }
    }
    s += K - ((K + 1) & ~1);   // the steps above advanced s by K rounded up to even
    bin_base += level_bins(a.shapes, l);
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
        a.keys[gs0 + e] = kx[ss];
        a.vals[gs0 + e] = gs0 + e;
        a.stash[gs0 + e] = stx[ss];
      }
    }
  }
  // softmax backward over the unit's L*K attention weights
  float dot = 0.f;
  for (int t = j; t < LK; t += LPU) dot = fmaf(rec[3 * LK + t], gat_s[t], dot);
  dot = unit_sum<LPU>(dot);
  for (int t = j; t < LK; t += LPU) {
    const float at = rec[3 * LK + t];
    rec[3 * LK + t] = at * (gat_s[t] - dot);
  }
  wave_lds_sync();
  if (live) write_record<T, LPU>(static_cast<T *>(a.grad_loc_attn) + unit * P, P, j, rec);
}

// ---------------------------------------------------------------------------------------------
// Backward phase 3, voxel-major: one grad_value row grad_value[b, v, g, :] of level l is the
// sum of attn * w_corner * grad_out over every sample with a corner at v, i.e. over the samples
// of the 8 bins whose base corner is v - (dz,dy,dx).  NBP lane groups (one per bin, or per
// 8/NBP bins when LPU is large) sum their bins in registers and are then reduced across the
// wave with DPP / ds_swizzle; every row is written exactly once, in T, in a deterministic order
// (stable sort of fixed-position keys): no zero-fill, no atomics.
template <int LPU, int NBP>
__device__ __forceinline__ float bin_group_sum(float v) {
#pragma unroll
  for (int m = LPU; m < LPU * NBP; m <<= 1) {
    if (m == 1) v += xor_lane<1>(v);
    else if (m == 2) v += xor_lane<2>(v);
    else if (m == 4) v += xor_lane<4>(v);
    else if (m == 8) v += xor_lane<8>(v);
    else if (m == 16) v += xor_lane<16>(v);
    else v += xor_lane<32>(v);
  }
  return v;
}

template <typename T, int CPL, int LPU>
__global__ __launch_bounds__(kBlock) void fda_bwd_value_kernel(const Args a) {
  using VG = ValueGeom<LPU>;
  constexpr int NBP = VG::NBP, VPW = VG::VPW, VPB = VG::VPB, VIT = VG::VIT;
  int b, g, vb;
  if (!map_tile(a, blockIdx.x, b, g, vb)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int j = lane & (LPU - 1);
  const int dp = (lane / LPU) % NBP;                  // which lane group of the pair
  const int vw = lane / (LPU * NBP);                  // pair within the wave
  // A "pair" is two x-neighbour voxels (x0, x0+1) of one row; pairs per level D*H*ceil(W/2).
  // Locate the level of pair block vb (block-uniform); coarse (last) levels first: their bins
  // hold the most samples, so their blocks are the longest and must not start last.
  int Dl = 0, Hl = 0, Wl = 0;
  uint32_t bin_lvl = 0, bins_bg = 0;
  uint32_t vstart = 0;
  bool found = false;
  int rem = vb;
  for (int tt = 0; tt < a.L; ++tt) {
    const int t = OPS3D_FDA_VALUE_REVERSE ? a.L - 1 - tt : tt;
    const int d = (int)a.shapes[3 * t], h = (int)a.shapes[3 * t + 1], w = (int)a.shapes[3 * t + 2];
    const uint32_t n = (uint32_t)d * (uint32_t)h * (((uint32_t)w + 1) >> 1);
    const int nvb = (int)((n + VPB * VIT - 1) / (VPB * VIT));
    if (!found) {
      if (rem < nvb) {
        found = true; Dl = d; Hl = h; Wl = w; vstart = (uint32_t)a.lsi[t];
        for (int u = 0; u < t; ++u) bin_lvl += level_bins(a.shapes, u);
      } else {
        rem -= nvb;
      }
    }
    bins_bg += level_bins(a.shapes, t);
  }
  if (!found) return;
  const uint32_t Wp = ((uint32_t)Wl + 1) >> 1;          // pairs per row
  const uint32_t npair = (uint32_t)Dl * (uint32_t)Hl * Wp;
  const uint32_t HWp = (uint32_t)Hl * Wp;
  const uint32_t bin_lb = (uint32_t)(b * a.G + g) * bins_bg + bin_lvl;
  const uint32_t W1 = (uint32_t)Wl + 1, HW1 = ((uint32_t)Hl + 1) * W1;
  const T *go = static_cast<const T *>(a.grad_out);
  const int D = a.D, GD = a.G * a.D;
  const int64_t obase = ((int64_t)b * a.S + vstart) * GD + g * D + j * CPL;

  for (int it = 0; it < VIT; ++it) {
    const uint32_t v = (uint32_t)(rem * VIT + it) * VPB + wave * VPW + vw;
    const bool live = v < npair;   // dead lanes still take part in the cross-group reduction
    float acc0[CPL], acc1[CPL];      // voxels x0 and x0 + 1
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc0[c] = acc1[c] = 0.f;
    uint32_t z = 0, y = 0, x0 = 0;
    if (live) {
      z = v / HWp;
      const uint32_t r2 = v - z * HWp;
      y = r2 / Wp;
      x0 = (r2 - y * Wp) * 2;
      // Samples with a corner on x0 or x0+1 in row (z, y): for each (dz, dy), the contiguous
      // bins of base x0-1, x0, x0+1 (shifted by +1: x0, x0+1, x0+2).  Base x0-1 feeds x0 (dx=1),
      // base x0 feeds x0 (dx=0) and x0+1 (dx=1), base x0+1 feeds x0+1 (dx=0); each grad_out
      // row is loaded and widened once for both voxels.
      const uint32_t bin_p = bin_lb + (z + 1) * HW1 + (y + 1) * W1 + x0;   // shifted base x0-1
      const bool two = x0 + 1 < (uint32_t)Wl;
      // One range per (dz, dy) (compile-time r, so wy / wz are fixed selections); the range's
      // entries are dealt round-robin to the pair's NBP lane groups.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t rb = bin_p - (uint32_t)(r >> 1) * HW1 - (uint32_t)(r & 1) * W1;   // (dz, dy) = (r>>1, r&1)
        // a pair with one voxel (x0 = W-1) has no bin of base x0+1: bin_start[rb + 3] is past
        // its row (at the end of the array: never written), so its range ends at s2
        const uint32_t s0 = a.bin_start[rb], m1 = a.bin_start[rb + 1], m2 = a.bin_start[rb + 2];
        const uint32_t s3 = two ? a.bin_start[rb + 3] : m2;
#pragma unroll OPS3D_FDA_VALUE_UNROLL
        for (uint32_t i = s0 + (uint32_t)dp; i < s3; i += NBP) {
          const float4 st = a.sorted_stash[i];
          const uint32_t row = a.sorted_row[i];
          float tg[CPL];
          load_global_elems<T, CPL>(go + (size_t)(row * (uint32_t)D) + j * CPL, tg);
          const float wy = (r & 1) ? st.y : 1.f - st.y;
          const float wz = (r >> 1) ? st.z : 1.f - st.z;
          const float ayz = st.w * (wy * wz);
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
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      acc0[c] = bin_group_sum<LPU, NBP>(acc0[c]);
      acc1[c] = bin_group_sum<LPU, NBP>(acc1[c]);
    }
    if (live && dp < 2) {   // lane group 0 stores x0, group 1 stores x0 + 1
      const uint32_t x = x0 + (uint32_t)dp;
      if (x < (uint32_t)Wl) {
        const int64_t o = obase + (int64_t)((z * (uint32_t)Hl + y) * (uint32_t)Wl + x) * GD;
        float res[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) res[c] = dp == 0 ? acc0[c] : acc1[c];
        if (a.accumulate) {   // caller-owned fp32 buffer: add to what it holds (sole owner, no atomics)
          float *dst = static_cast<float *>(a.out) + o;
          float old[CPL];
          load_global_elems<float, CPL>(dst, old);
#pragma unroll
          for (int c = 0; c < CPL; ++c) res[c] += old[c];
          store_elems<float, CPL>(dst, res);
        } else {
          store_elems<T, CPL>(static_cast<T *>(a.out) + o, res);
        }
      }
    }
  }
}

// which: 0 forward, 1 backward phase 1 (query-major), 2 backward phase 3 (voxel-major)
template <typename T, int CPL, int LPU>
hipError_t launch_one(int which, const Args &a, unsigned grid, size_t lds, hipStream_t st) {
  if (which == 0) {
    if constexpr (fwd_pairs(CPL, LPU, (int)sizeof(T)))
      hipLaunchKernelGGL((fda_forward_pair_kernel<T, CPL>), dim3(grid), dim3(kBlock), lds, st, a);
    else
      hipLaunchKernelGGL((fda_forward_kernel<T, CPL, LPU>), dim3(grid), dim3(kBlock), lds, st, a);
  }
  else if (which == 1)
    hipLaunchKernelGGL((fda_bwd_query_kernel<T, CPL, LPU>), dim3(grid), dim3(kBlock), lds, st, a);
  else
    hipLaunchKernelGGL((fda_bwd_value_kernel<T, CPL, LPU>), dim3(grid), dim3(kBlock), 0, st, a);
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
