// Tile-major backward of Flash Deformable 3D Attention for 16-bit element types with D = 32
// (gfx950 MFMA), in four kernels around the bucketing of fda_tiles.hip:
//
//   setup   (query-major, no gathers): per unit (b, q, g) the fp32 softmax of its L*K logits and,
//           per sample, the pixel coordinate; per sample a 16-byte record: home tile, tile-local
//           base corner and next-tile flags, level, fractions (16-bit fixed point), attention.
//   bucketing: the samples' entries grouped by 8 x 4 x 4 tile (sample indices, fda_tiles.hip),
//           plus a partition of every head's entries into equal ranges, one per tile-kernel block.
//   tile    (tile-major, persistent): each block streams its range of entries.  Per tile the value
//           rows of the tile and its +1 halo are loaded into LDS; per chunk of entries the records
//           and grad_output rows are loaded into LDS by the memory unit (global/buffer_load_lds),
//           one chunk ahead.  For the entries whose home tile it is, the block computes the
//           location and attention gradient partials from LDS (the trilinear chain rule of the
//           reference, common.h:279-353); every entry adds its weighted grad_output row to the
//           tile's grad_value on the matrix cores (fda_tile_mfma.h has the operand scheme).
//   finish  (query-major): softmax backward (col2im.cuh:414-427) and the packed
//           grad_sampling_loc_attn.
// Tiles cut by a block boundary are written as fp32 partial sums and added by a combine kernel.
// There are no global atomics; every output element is written once.
//
// Precision: the fractions of the pixel coordinates are carried in 16-bit fixed point (error
// <= 2^-17) and each grad_value weight is rounded once to the 16-bit type before the matrix
// product; everything else is fp32.  This path serves bf16 / fp16 only, whose outputs carry
// 2^-9 / 2^-11 relative rounding.
#pragma once

#include "fda_device.h"
#include "fda_tile_mfma.h"

namespace ops3d_fda {

// Per-sample record of the setup kernel (uint4):
//   x: home tile id (head base + level base + tile), kKeyInvalid when the sample is outside
//   y: bits 0-15 tile-local word (fused_word), bits 16-31 fz (0.16 fixed point)
//   z: attention weight (fp32 bits)
//   w: fx | fy << 16 (0.16 fixed point)
// fused_word: (lx+1) | (ly+1) << 4 | (lz+1) << 7 | next-tile flags x, y, z << 10, 11, 12 | level << 13,
// with the base corner local to the home tile (lx in [-1, 8), ly, lz in [-1, 4)).
__device__ __forceinline__ uint32_t fused_word(int lx, int ly, int lz, uint32_t ex, uint32_t ey, uint32_t ez, int l) {
  return (uint32_t)(lx + 1) | ((uint32_t)(ly + 1) << 4) | ((uint32_t)(lz + 1) << 7) | (ex << 10) | (ey << 11) |
         (ez << 12) | ((uint32_t)l << 13);
}

// The same word in the bucketing's layout (tile_word + flags + level, fda_device.h).
__device__ __forceinline__ uint32_t fused_word_expand(uint32_t w) {
  return tile_word((int)(w & 15u) - 1, (int)((w >> 4) & 7u) - 1, (int)((w >> 7) & 7u) - 1) | (((w >> 10) & 7u) << 15) |
         (((w >> 13) & 7u) << 18);
}

__device__ __forceinline__ uint32_t frac16(float f) {
  return min((uint32_t)(f * 65536.f + 0.5f), 65535u);
}

constexpr int kSetupUnitLanes = 8;
constexpr int kSetupUnits = kBlock / kSetupUnitLanes;   // units per block

// ---------------------------------------------------------------------------------------------
// Setup: one unit per 8 lanes, 32 units of one (b, g) per block (map_tile with nqb for 32 units).
template <typename T>
__global__ __launch_bounds__(kBlock) void fda_bwd_setup_kernel(const Args a) {
  extern __shared__ float lds[];
  constexpr int UL = kSetupUnitLanes, UPW = kWave / UL;
  int b, g, qb;
  if (!map_tile(a, blockIdx.x, b, g, qb)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int ju = lane & (UL - 1);
  const int ub = wave * UPW + lane / UL;
  const int q = qb * kSetupUnits + ub;
  const bool live = q < a.Q;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  float *rec = lds + ub * (P + 1);
  const int64_t unit = ((int64_t)b * a.Q + (live ? q : 0)) * a.G + g;
  __shared__ LevelTiles lvt[5];
  __shared__ uint32_t lvbase[5];
  if (threadIdx.x == 0) {
    uint32_t t = (uint32_t)(b * a.G + g) * tiles_per_head(a.shapes, L, a.TX, a.TY, a.TZ);
    for (int l = 0; l < L; ++l) {
      lvt[l] = level_tiles(a.shapes, l, a.TX, a.TY, a.TZ);
      lvbase[l] = t;
      t += lvt[l].count;
    }
  }
  __syncthreads();
  stage_record<T, UL>(static_cast<const T *>(a.loc_attn) + unit * P, P, ju, live, rec);
  wave_lds_sync();
  unit_softmax<UL>(rec + 3 * LK, LK, ju);
  wave_lds_sync();
  uint4 *srec = reinterpret_cast<uint4 *>(a.keys);
  for (int s = ju; live && s < LK; s += UL) {
    const int l = s / K;
    const LevelTiles &lt = lvt[l];
    const int Dl = lt.n[0], Hl = lt.n[1], Wl = lt.n[2];
    SampleBase sb;
    const bool in = sample_base(rec[3 * s], rec[3 * s + 1], rec[3 * s + 2], Wl, Hl, Dl, sb);
    const uint32_t gs = sample_index(b, g, q, s, a.G, a.Q, LK);
    if (!in) {
      srec[gs] = make_uint4(kKeyInvalid, 0u, 0u, 0u);
      a.ures[gs] = make_float4(0.f, 0.f, 0.f, 0.f);   // no tile computes this sample
      continue;
    }
    const int x0 = sb.x0, y0 = sb.y0, z0 = sb.z0;
    const int hz = max(z0, 0) >> lt.sh[0], hy = max(y0, 0) >> lt.sh[1], hx = max(x0, 0) >> lt.sh[2];
    const int lz = z0 - hz * lt.t[0], ly = y0 - hy * lt.t[1], lx = x0 - hx * lt.t[2];
    const uint32_t ex = lx == lt.t[2] - 1 && (hx + 1) * lt.t[2] < lt.n[2];
    const uint32_t ey = ly == lt.t[1] - 1 && (hy + 1) * lt.t[1] < lt.n[1];
    const uint32_t ez = lz == lt.t[0] - 1 && (hz + 1) * lt.t[0] < lt.n[0];
    const uint32_t key = lvbase[l] + (uint32_t)((hz * lt.nt[1] + hy) * lt.nt[2] + hx);
    srec[gs] = make_uint4(key, fused_word(lx, ly, lz, ex, ey, ez, l) | (frac16(sb.wz1) << 16),
                          __float_as_uint(rec[3 * LK + s]), frac16(sb.wx1) | (frac16(sb.wy1) << 16));
  }
  clear_tile_counts(a);   // (atomic-mode bucketing only)
}

// ---------------------------------------------------------------------------------------------
// Finish: one unit per 8 lanes, units in [B, Q, G] order.  grad_sampling_loc_attn of the unit:
// the location gradients the tile kernel left in ures (already times attn * size), and the
// softmax backward of the attention gradients.
template <typename T>
__global__ __launch_bounds__(kBlock) void fda_bwd_finish_kernel(const Args a) {
  extern __shared__ float lds[];
  constexpr int UL = kSetupUnitLanes, UPW = kWave / UL;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int ju = lane & (UL - 1);
  const int ub = wave * UPW + lane / UL;
  const int64_t unit = (int64_t)blockIdx.x * kSetupUnits + ub;
  const int64_t nunits = (int64_t)a.B * a.Q * a.G;
  const bool live = unit < nunits;
  const int L = a.L, K = a.K, LK = L * K, P = a.P;
  float *rec = lds + ub * (P + 1);
  const int64_t u = live ? unit : 0;
  const int g = (int)(u % a.G);
  const int64_t bq = u / a.G;
  const int q = (int)(bq % a.Q), b = (int)(bq / a.Q);
  stage_record<T, UL>(static_cast<const T *>(a.loc_attn) + u * P, P, ju, live, rec);
  wave_lds_sync();
  unit_softmax<UL>(rec + 3 * LK, LK, ju);
  wave_lds_sync();
  const uint32_t gs0 = sample_index(b, g, q, 0, a.G, a.Q, LK);
  float dot = 0.f;
  for (int s = ju; s < LK; s += UL) {
    const float4 r = live ? a.ures[gs0 + s] : make_float4(0.f, 0.f, 0.f, 0.f);
    rec[3 * s] = r.x;
    rec[3 * s + 1] = r.y;
    rec[3 * s + 2] = r.z;
    dot = fmaf(rec[3 * LK + s], r.w, dot);
  }
  dot = unit_sum<UL>(dot);
  for (int s = ju; s < LK; s += UL) {
    const float gw = live ? a.ures[gs0 + s].w : 0.f;   // (the line is in L1 from the loop above)
    rec[3 * LK + s] = rec[3 * LK + s] * (gw - dot);
  }
  wave_lds_sync();
  if (live) write_record<T, UL>(static_cast<T *>(a.grad_loc_attn) + u * P, P, ju, rec);
}

}  // namespace ops3d_fda

namespace ops3d_fda {

// ---------------------------------------------------------------------------------------------
// Tile kernel.  Block -> (head bg, part j of bph): with XCD affinity (G % 8 == 0) the blocks on
// XCD x serve the heads with g % 8 == x, bph blocks each; otherwise bph consecutive blocks per head.
__device__ __forceinline__ bool fused_block(const Args &a, int bid, int nblocks, int &b, int &g, int &j) {
  int hi;
  if (a.tile_affinity) {
    const int x = bid & 7, r = bid >> 3, hpx = a.G / 8;
    (void)nblocks;
    hi = r / a.bph;
    j = r - hi * a.bph;
    if (hi >= a.B * hpx) return false;
    b = hi / hpx;
    g = x + 8 * (hi - b * hpx);
  } else {
    hi = bid / a.bph;
    j = bid - hi * a.bph;
    if (hi >= a.B * a.G) return false;
    b = hi / a.G;
    g = hi - b * a.G;
  }
  return true;
}

constexpr int kFusedChunk = 256;                        // entries per chunk
constexpr int kFusedThreads = 512;                      // 8 waves: two per z-plane of the tile
constexpr int kFusedTileWin = 128;                      // tiles per LDS window of the block's list
constexpr int kValRows = 9 * 5 * 5;                     // value rows of a tile and its +1 halo

// Scratch LDS of the tile kernel (never written by the memory unit directly, so the compiler
// need not order its accesses after pending LDS DMA).  The part from 0 to kFusedXch also serves
// as the exchange area of the tile flush (the zero record and the weight matrices are restored
// afterwards).
struct FusedScr {
  static constexpr size_t lrec = 0;                                          // [CH + 1] float4 (local x, y, z, attn)
  static constexpr size_t wts = lrec + (size_t)(kFusedChunk + 1) * 16;       // [CH] 8 x 16-bit corner weights
  static constexpr size_t meta = wts + (size_t)kFusedChunk * 16;             // [CH] base corner
  static constexpr size_t home = meta + (size_t)kFusedChunk * 4;             // [CH] home entries
  static constexpr size_t hsid = home + (size_t)kFusedChunk * 4;             // [CH] their sample indices
  static constexpr size_t amat = hsid + (size_t)kFusedChunk * 4;             // [8 waves][32][16] 16-bit
  static constexpr size_t rowi = amat + (size_t)8 * 1024;                    // [CH] next chunk's row offsets
  static constexpr size_t zrow = rowi + (size_t)kFusedChunk * 4;             // 64 zero bytes
  static constexpr size_t total = zrow + 64;
  static constexpr size_t xch = 0;                                           // [4 planes][16][64] fp32
  static constexpr size_t xch_bytes = (size_t)4 * 16 * 64 * 4;
  static_assert(xch_bytes <= rowi, "flush exchange area");
};

__host__ __device__ constexpr size_t fused_tile_lds_bytes() { return 0; }   // all LDS is static

// Fill LDS from a buffer: lane k of the wave writes base + 16 k (or + 4 k); a voffset past the
// buffer reads zeros.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, void *lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_wave_base, 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, void *lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_wave_base, 4, voff, 0, 0, 0);
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint32_t sgpr(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }

// kAcc3: fp32 accumulation into the caller's buffer, each weight entered as a sum of three 16-bit
// parts (a separate instance keeps the common path's accumulator in one chain of MFMAs)
template <typename T, bool kAcc3>
__global__ __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(4))) void fda_bwd_fused_tile_kernel(const Args a) {
  constexpr int NT = kFusedThreads, CH = kFusedChunk, RB = kMfmaRowBytes, TW = kFusedTileWin;
  // memory-unit (DMA) targets: one object each, so that reads of one are not ordered after
  // pending DMA into another
  __shared__ __align__(16) unsigned char rows0_l[CH * RB], rows1_l[CH * RB];   // grad_output rows, entry order
  __shared__ __align__(16) unsigned char val_l[kValRows * RB];                 // value rows of the tile + halo
  __shared__ __align__(16) uint4 sr_l[CH];                                     // per-sample records
  __shared__ __align__(16) uint32_t idx_l[3 * CH];                             // sample indices, 3 chunks
  __shared__ __align__(16) unsigned char scr_l[FusedScr::total];
  float4 *lrec_l = reinterpret_cast<float4 *>(scr_l + FusedScr::lrec);
  unsigned short *wts_l = reinterpret_cast<unsigned short *>(scr_l + FusedScr::wts);   // [e][dz][dy][dx]
  uint32_t *meta_l = reinterpret_cast<uint32_t *>(scr_l + FusedScr::meta);
  uint32_t *home_l = reinterpret_cast<uint32_t *>(scr_l + FusedScr::home);
  uint32_t *hsid_l = reinterpret_cast<uint32_t *>(scr_l + FusedScr::hsid);
  unsigned short *amat_l = reinterpret_cast<unsigned short *>(scr_l + FusedScr::amat);
  uint32_t *rowi_l = reinterpret_cast<uint32_t *>(scr_l + FusedScr::rowi);
  const unsigned char *zrow_l = scr_l + FusedScr::zrow;
  float *xch_l = reinterpret_cast<float *>(scr_l + FusedScr::xch);
  __shared__ uint32_t wcnt[2][8];           // per chunk parity: home entries
  __shared__ uint32_t ts_l[TW], tc_l[TW];   // the window of the block's tiles: start, count
  __shared__ uint32_t tg_l[TW][2];          // and their coordinates: itx | ity << 16, itz | level << 16
  __shared__ LevelTiles lvt[5];
  __shared__ uint32_t lvbase[6];
  __shared__ uint32_t lvsi[5];              // level start index (each level's first voxel)
  __shared__ uint32_t pinfo[4];

  int b, g, j;
  if (!fused_block(a, blockIdx.x, gridDim.x, b, g, j)) return;
  const int tid0 = threadIdx.x;
#ifdef FUSED_TIMING
  unsigned long long t_acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, t_prev = clock64();
#define TM(i) do { const unsigned long long t_now = clock64(); t_acc[i] += t_now - t_prev; t_prev = t_now; } while (0)
#else
#define TM(i) ((void)0)
#endif
  const int G = a.G, L = a.L, LK = a.L * a.K;
  const uint32_t bg = (uint32_t)(b * G + g);
  const uint32_t per_head = (uint32_t)a.Q * (uint32_t)LK;
  const uint32_t hbase = bg * 8u * per_head;
  const uint32_t *part = a.part + (size_t)bg * (a.bph + 2);
  if (tid0 == 0) {
    uint32_t t = 0;
    for (int u = 0; u < L; ++u) {
      lvt[u] = level_tiles(a.shapes, u, a.TX, a.TY, a.TZ);
      lvbase[u] = t;
      lvsi[u] = (uint32_t)a.lsi[u];
      t += lvt[u].count;
    }
    lvbase[L] = t;
    pinfo[0] = part[a.bph + 1];
    pinfo[1] = part[j];
    pinfo[2] = part[j + 1];
  }
  for (int i = tid0; i < 8 * 512; i += NT) amat_l[i] = 0;
  if (tid0 < 16) reinterpret_cast<uint32_t *>(scr_l + FusedScr::zrow)[tid0] = 0u;
  if (tid0 == 0) lrec_l[CH] = make_float4(0.f, 0.f, 0.f, 0.f);   // the zero record
  if (tid0 < 16) wcnt[tid0 >> 3][tid0 & 7] = 0u;
  __syncthreads();
  const uint32_t T_h = sgpr(lvbase[L]);
  const uint32_t E = sgpr(pinfo[0]);
  const uint32_t bnd0 = hbase + (uint32_t)((uint64_t)j * E / (uint32_t)a.bph);
  const uint32_t bnd1 = hbase + (uint32_t)((uint64_t)(j + 1) * E / (uint32_t)a.bph);
  const uint32_t tbase = bg * T_h;
  uint32_t first = sgpr(pinfo[1]);
  if (first > 0 && first - 1 < T_h) {
    const uint32_t t = first - 1;
    if (a.tile_start[tbase + t] + a.tile_counts[tbase + t] > bnd0) first = t;
  }
  const uint32_t last1 = j == a.bph - 1 ? T_h : sgpr(pinfo[2]);
  if (first >= last1) return;

  // per-block buffer resources (offsets stay below 2^32 bytes: checked by the host)
  const T *go = static_cast<const T *>(a.gout_hm ? a.gout_hm : a.grad_out);
  const bool go_direct = a.gout_hm == nullptr;
  const T *go_base = go + (go_direct ? (size_t)b * a.Q * G * 32u : (size_t)bg * a.Q * 32u);
  const __amdgpu_buffer_rsrc_t r_ent = make_rsrc(a.entries + hbase, 8u * per_head * 4u);
  const __amdgpu_buffer_rsrc_t r_srec = make_rsrc(reinterpret_cast<const uint4 *>(a.keys) + (size_t)bg * per_head, per_head * 16u);
  const __amdgpu_buffer_rsrc_t r_go = make_rsrc(go_base, (uint32_t)((size_t)a.Q * (go_direct ? G : 1) * 32u * sizeof(T)));
  const T *val_base = static_cast<const T *>(a.value) + (size_t)b * a.S * G * 32u;
  const __amdgpu_buffer_rsrc_t r_val = make_rsrc(val_base, (uint32_t)((size_t)a.S * G * 32u * sizeof(T)));
  const uint32_t s0h = bg * per_head;   // the head's first sample
  // grad_output row of head sample s (relative to go_base)
  const auto row_of = [&](uint32_t s) {
    const uint32_t q = (uint32_t)(((double)s + 0.5) * a.inv_lk);   // s / (L*K), exact
    return go_direct ? q * (uint32_t)G + (uint32_t)g : q;
  };
  bool flushed = false;   // a tile flush used the exchange area (over the zero record and weight matrices)

  for (uint32_t w0 = first; w0 < last1; w0 += TW) {
    const uint32_t nwin = min((uint32_t)TW, last1 - w0);
    __syncthreads();
    for (uint32_t i = tid0; i < nwin; i += NT) {
      const uint32_t t = w0 + i;
      ts_l[i] = a.tile_start[tbase + t];
      tc_l[i] = a.tile_counts[tbase + t];
      int l = 0;
      while (l + 1 < L && t >= lvbase[l + 1]) ++l;
      const uint32_t r = t - lvbase[l];
      const LevelTiles &lt = lvt[l];
      const uint32_t itx = r % (uint32_t)lt.nt[2], ity = (r / (uint32_t)lt.nt[2]) % (uint32_t)lt.nt[1];
      const uint32_t itz = r / ((uint32_t)lt.nt[2] * (uint32_t)lt.nt[1]);
      tg_l[i][0] = itx | (ity << 16);
      tg_l[i][1] = itz | ((uint32_t)l << 16);
    }
    if (tid0 < 16) wcnt[tid0 >> 3][tid0 & 7] = 0u;   // chunk numbers restart with the window
    __syncthreads();
    struct Chunk {
      uint32_t ti, es, n;
      bool first, last, valid;
    };
    const auto chunk_at = [&](uint32_t ti, uint32_t off) {
      Chunk c;
      c.valid = ti < nwin;
      c.ti = ti;
      if (!c.valid) { c.es = 0; c.n = 0; c.first = c.last = false; return c; }
      const uint32_t ts = sgpr(ts_l[ti]), te = ts + sgpr(tc_l[ti]);
      const uint32_t s0 = max(ts, bnd0), s1 = min(te, bnd1);
      const uint32_t len = s1 > s0 ? s1 - s0 : 0u;
      c.es = s0 + off;
      c.n = min((uint32_t)CH, len - off);
      c.first = off == 0;
      c.last = off + c.n >= len;
      return c;
    };
    const auto chunk_next = [&](const Chunk &c) {
      return c.last ? chunk_at(c.ti + 1, 0) : chunk_at(c.ti, c.es + c.n - max(sgpr(ts_l[c.ti]), bnd0));
    };
    struct TileGeo {
      int l, itx, ity, itz;
    };
    const auto geo_of = [&](uint32_t ti) {
      TileGeo t;
      const uint32_t w0g = sgpr(tg_l[ti][0]), w1g = sgpr(tg_l[ti][1]);
      t.itx = (int)(w0g & 0xffffu); t.ity = (int)(w0g >> 16); t.itz = (int)(w1g & 0xffffu); t.l = (int)(w1g >> 16);
      return t;
    };
    // DMA (tid: the thread's index, recomputed where used so that no per-lane value is kept live
    // across the chunk loop)
    const auto issue_idx = [&](const Chunk &c, uint32_t slot, int tid) {
      if (!c.valid || tid >= CH) return;
      dma4(r_ent, (c.es - hbase + (uint32_t)tid) * 4u, idx_l + slot * CH + (tid & ~63));
    };
    const auto issue_sr = [&](const Chunk &c, uint32_t s, int tid) {   // thread tid < CH: entry tid's record
      if (!c.valid || tid >= CH) return;
      dma16(r_srec, (uint32_t)tid < c.n ? (s - s0h) * 16u : 0xfffffff0u, sr_l + (tid & ~63));
    };
    const auto issue_rows = [&](const Chunk &c, unsigned char *rs, int tid) {   // row offsets from rowi_l
      if (!c.valid) return;
      const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t p = (uint32_t)((2 * wave + i) * 64 + lane);   // piece: entry p / 4, quarter p % 4
        const uint32_t e = p >> 2;
        const uint32_t voff = e < c.n ? (rowi_l[e] * 32u + (p & 3u) * 8u) * (uint32_t)sizeof(T) : 0xfffffff0u;
        dma16(r_go, voff, rs + (size_t)((2 * wave + i) * 64) * 16);
      }
    };
    const auto issue_val = [&](const Chunk &c, int tid) {
      if (!c.valid) return;
      const int wave = tid >> 6, lane = tid & 63;
      const TileGeo tg = geo_of(c.ti);
      const int n0 = (int)sgpr((uint32_t)lvt[tg.l].n[0]), n1 = (int)sgpr((uint32_t)lvt[tg.l].n[1]),
                n2 = (int)sgpr((uint32_t)lvt[tg.l].n[2]);
      const int x0 = tg.itx * 8, y0 = tg.ity * 4, z0 = tg.itz * 4;   // (clipped tiles start at 0)
      const int64_t lb = sgpr(lvsi[tg.l]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int p = (2 * wave + i) * 64 + lane, r = p >> 2;   // piece: halo row r, quarter p % 4
        if (p < kValRows * 4) {
          const int x = x0 + r % 9, y = y0 + (r / 9) % 5, z = z0 + r / 45;
          const bool in = x < n2 && y < n1 && z < n0;
          const uint32_t row = (uint32_t)(lb + ((int64_t)z * n1 + y) * n2 + x) * (uint32_t)G + (uint32_t)g;
          const uint32_t voff = in ? (row * 32u + (uint32_t)(p & 3) * 8u) * (uint32_t)sizeof(T) : 0xfffffff0u;
          dma16(r_val, voff, val_l + (size_t)((2 * wave + i) * 64) * 16);
        }
      }
    };

    // prologue: chunk 0's indices and value block; then its records and rows, chunk 1's indices
    const Chunk c0 = chunk_at(0, 0);
    issue_idx(c0, 0, tid0);
    issue_val(c0, tid0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid0 < CH) {
      const uint32_t s = idx_l[tid0];
      issue_sr(c0, s, tid0);
      rowi_l[tid0] = row_of(s - s0h);
    }
    issue_idx(chunk_next(c0), 1, tid0);
    __syncthreads();
    issue_rows(c0, rows0_l, tid0);
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    uint32_t ci = 0;
    Chunk c = c0;
    // one chunk; P = ci & 1 selects the row buffer at compile time (rows of chunk ci in P, chunk
    // ci + 1's loaded into the other)
    const auto chunk_step = [&](auto P) {
      constexpr bool kOdd = decltype(P)::value != 0;
      unsigned char *rows_cur = kOdd ? rows1_l : rows0_l;
      unsigned char *rows_nxt = kOdd ? rows0_l : rows1_l;
      int tid = threadIdx.x;
      asm volatile("" : "+v"(tid));   // per-lane values are recomputed in each chunk, not kept live across it
      const int lane = tid & 63, wave = tid >> 6;
      const Chunk cn = chunk_next(c);
      TM(7);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();   // B1: records / rows of ci, indices of ci + 1 (and the value block) landed
      TM(0);
      const uint32_t islot = ci % 3u;
      const TileGeo tg = geo_of(c.ti);
      const int l = tg.l, itx = tg.itx, ity = tg.ity, itz = tg.itz;
      const int n0 = (int)sgpr((uint32_t)lvt[l].n[0]), n1 = (int)sgpr((uint32_t)lvt[l].n[1]),
                n2 = (int)sgpr((uint32_t)lvt[l].n[2]);
      const int tz = (int)sgpr((uint32_t)lvt[l].t[0]), ty = (int)sgpr((uint32_t)lvt[l].t[1]), tx = (int)sgpr((uint32_t)lvt[l].t[2]);
      const uint32_t ntx = sgpr((uint32_t)lvt[l].nt[2]), nty = sgpr((uint32_t)lvt[l].nt[1]);
      const uint32_t tgid = sgpr(lvbase[l]) + ((uint32_t)itz * nty + (uint32_t)ity) * ntx + (uint32_t)itx + tbase;
      if (flushed) {   // the flush exchange overwrote the zero record and part of the weight matrices
        for (int i = tid; i < 8 * 512; i += NT) amat_l[i] = 0;
        if (tid == 0) lrec_l[CH] = make_float4(0.f, 0.f, 0.f, 0.f);
        flushed = false;
      }
      // derive (threads < CH, one entry each): local base corner in this tile, fractions, home
      // flag, corner weights; the home entries are listed with one LDS atomic per wave
      const uint32_t par = ci & 1u;
      if (tid < CH) {
        const uint32_t e = (uint32_t)tid;
        const bool live = e < c.n;
        const uint4 r = sr_l[e];
        const uint32_t sc = idx_l[islot * CH + e];              // this entry's sample
        const uint32_t sn = idx_l[((ci + 1u) % 3u) * CH + e];   // chunk ci + 1's sample
        const uint32_t w = r.y & 0xffffu;
        int lx = (int)(w & 15u) - 1, ly = (int)((w >> 4) & 7u) - 1, lz = (int)((w >> 7) & 7u) - 1;
        const bool home = r.x == tgid;
        if (!home) {   // a next-tile entry: minus the tile size on each axis this tile is past the home tile
          uint32_t d = tgid - r.x;
          const uint32_t sz = ntx * nty;
          const uint32_t dz = d >= sz ? 1u : 0u;
          d -= dz * sz;
          const uint32_t dy = d >= ntx ? 1u : 0u;
          const uint32_t dx = d - dy * ntx;
          lx -= (int)dx * tx;
          ly -= (int)dy * ty;
          lz -= (int)dz * tz;
        }
        const float fx = (float)(r.w & 0xffffu) * (1.f / 65536.f), fy = (float)(r.w >> 16) * (1.f / 65536.f);
        const float fz = (float)(r.y >> 16) * (1.f / 65536.f);
        const float at = __uint_as_float(r.z);
        // this entry's slot of the records is refilled with chunk ci + 1's record (its read above
        // must complete first)
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
        issue_sr(cn, sn, tid);
        rowi_l[e] = row_of(sn - s0h);
        uint4 wq = make_uint4(0u, 0u, 0u, 0u);
        uint32_t meta = 0x0f000000u;   // base z 14: no plane
        if (live) {
          lrec_l[e] = make_float4((float)lx + fx, (float)ly + fy, (float)lz + fz, at);
          const float wx0 = 1.f - fx, wy0 = 1.f - fy, wz0 = 1.f - fz;
          const float a0 = at * wz0, a1 = at * fz;
          const auto pk = [&](float v0, float v1) {
            return (uint32_t)Mfma16<T>::bits(v0) | ((uint32_t)Mfma16<T>::bits(v1) << 16);
          };
          wq = make_uint4(pk(a0 * wy0 * wx0, a0 * wy0 * fx), pk(a0 * fy * wx0, a0 * fy * fx),
                          pk(a1 * wy0 * wx0, a1 * wy0 * fx), pk(a1 * fy * wx0, a1 * fy * fx));
          meta = ((uint32_t)(lx + 1) << 16) | ((uint32_t)(ly + 1) << 20) | ((uint32_t)(lz + 1) << 24);
        }
        *reinterpret_cast<uint4 *>(wts_l + (size_t)e * 8) = wq;
        meta_l[e] = meta;
        const bool ish = live && home;
        const uint64_t mh = __ballot(ish);
        uint32_t hb = 0;
        if (lane == 0 && mh) hb = atomicAdd(&wcnt[par][0], (uint32_t)__builtin_popcountll(mh));
        hb = sgpr(hb);
        if (ish) {
          home_l[hb + lanes_below(mh)] = e;
          hsid_l[hb + lanes_below(mh)] = sc;
        }
        if (tid == 0) wcnt[par ^ 1u][0] = 0u;   // the next chunk's counter
      }
      if (c.first) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
      }
      TM(1);
      __syncthreads();   // B2: records, weights, home list visible; next chunk's row offsets ready
      TM(2);
      const uint32_t nhome = sgpr(wcnt[par][0]);
      // the next chunks: rows of ci + 1, indices of ci + 2
      issue_rows(cn, rows_nxt, tid);
      issue_idx(chunk_next(cn), (ci + 2u) % 3u, tid);
      TM(3);
      const unsigned char *rows = rows_cur;
      // U: location / attention gradients of the home entries, 2 lanes (16 channels each) per
      // entry (fixed summation order: bitwise repeatable)
      for (uint32_t h0 = 0; h0 < nhome; h0 += (uint32_t)(NT / 2)) {
        const uint32_t hh = h0 + (uint32_t)(tid >> 1);
        const bool ok = hh < nhome;
        const uint32_t e = ok ? home_l[hh] : (uint32_t)CH;
        const uint32_t sidx = ok ? hsid_l[hh] : 0u;
        const float4 r = lrec_l[e];
        const float bxf = floorf(r.x), byf = floorf(r.y), bzf = floorf(r.z);
        const float fx = r.x - bxf, fy = r.y - byf, fz = r.z - bzf;
        const int bx = (int)bxf, by = (int)byf, bz = (int)bzf;
        const uint32_t h32 = (uint32_t)(tid & 1) * 32u;   // this lane's half of the row (16 channels)
        const unsigned char *grow = ok ? rows + (size_t)e * RB : zrow_l;
        const u32x4 g0 = *reinterpret_cast<const u32x4 *>(grow + (ok ? h32 : 0u));
        const u32x4 g1 = *reinterpret_cast<const u32x4 *>(grow + (ok ? h32 + 16u : 16u));
        float U[8];
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
          if ((cc & 1) == 0 && cc > 0) __builtin_amdgcn_sched_barrier(0);   // two corners' loads in flight
          const int x = bx + (cc & 1), y = by + ((cc >> 1) & 1), z = bz + (cc >> 2);
          const bool in = x >= 0 && y >= 0 && z >= 0;
          const unsigned char *vp = in ? val_l + (size_t)((z * 5 + y) * 9 + x) * RB + h32 : zrow_l;
          const u32x4 v0 = *reinterpret_cast<const u32x4 *>(vp);
          const u32x4 v1 = *reinterpret_cast<const u32x4 *>(vp + (in ? 16u : 32u));
          float u = Elem<T>::dot(v0.x, g0.x, 0.f);
          u = Elem<T>::dot(v0.y, g0.y, u);
          u = Elem<T>::dot(v0.z, g0.z, u);
          u = Elem<T>::dot(v0.w, g0.w, u);
          u = Elem<T>::dot(v1.x, g1.x, u);
          u = Elem<T>::dot(v1.y, g1.y, u);
          u = Elem<T>::dot(v1.z, g1.z, u);
          U[cc] = Elem<T>::dot(v1.w, g1.w, u);
        }
        const float wx[2] = {1.f - fx, fx}, wy[2] = {1.f - fy, fy}, wz[2] = {1.f - fz, fz};
        float ga = 0.f, gx = 0.f, gy = 0.f, gz = 0.f;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) ga = fmaf((wx[cc & 1] * wy[(cc >> 1) & 1]) * wz[cc >> 2], U[cc], ga);
#pragma unroll
        for (int zy = 0; zy < 4; ++zy)
          gx = fmaf(wy[zy & 1] * wz[zy >> 1], U[4 * (zy >> 1) + 2 * (zy & 1) + 1] - U[4 * (zy >> 1) + 2 * (zy & 1)], gx);
#pragma unroll
        for (int zx = 0; zx < 4; ++zx)
          gy = fmaf(wx[zx & 1] * wz[zx >> 1], U[4 * (zx >> 1) + 2 + (zx & 1)] - U[4 * (zx >> 1) + (zx & 1)], gy);
#pragma unroll
        for (int yx = 0; yx < 4; ++yx)
          gz = fmaf(wx[yx & 1] * wy[yx >> 1], U[4 + 2 * (yx >> 1) + (yx & 1)] - U[2 * (yx >> 1) + (yx & 1)], gz);
        gx += xor_lane<1>(gx);
        gy += xor_lane<1>(gy);
        gz += xor_lane<1>(gz);
        ga += xor_lane<1>(ga);
        if (ok && (tid & 1) == 0)   // d(pixel)/d(loc) = size (grid = 2*loc - 1, size/2 per unit of grid)
          a.ures[sidx] = make_float4(gx * r.w * (float)n2, gy * r.w * (float)n1, gz * r.w * (float)n0, ga);
      }
      TM(4);
      // the value block of the next tile, once every wave is done with this one
      if (c.last && cn.valid) {
        __syncthreads();
        issue_val(cn, tid);
      }
      // grad_value on the matrix cores: wave (plane, half) adds the entries of its half of the
      // chunk that have a corner in the plane (base z = plane - 1 or plane)
      const int plane = wave & 3, ghalf = wave >> 2;
#ifdef V_NOMFMA
      if (plane < tz && a.B < 0) {
#else
      if (plane < tz) {
#endif
        const int e_l = lane >> 2, cdx = lane & 1, cdy = (lane >> 1) & 1;
        unsigned short *Aw = amat_l + wave * 512;
        const uint32_t a_rd = (uint32_t)((lane & 31) * 32 + 16 * (lane >> 5));
        const int g4 = lane >> 4, s16 = lane & 15;
        const uint32_t b_ch = 2u * (16u * (uint32_t)(g4 & 1) + 4u * (uint32_t)(s16 & 3));
        const int b_sl = 8 * (g4 >> 1) + (s16 >> 2);
        const uint32_t kend = min(c.n, (uint32_t)(CH / 2) * (uint32_t)(ghalf + 1));
        for (uint32_t k0 = (uint32_t)(CH / 2) * (uint32_t)ghalf; k0 < kend; k0 += 16u) {
          const uint32_t e = k0 + (uint32_t)e_l;
          const uint32_t m = meta_l[e];
          const int dz = plane + 1 - (int)((m >> 24) & 15u);   // plane - base z
          const int x = (int)((m >> 16) & 15u) - 1 + cdx, y = (int)((m >> 20) & 15u) - 1 + cdy;
          const bool wv = (unsigned)dz < 2u && (unsigned)x < 8u && (unsigned)y < 4u;
          const uint32_t wa = (uint32_t)((y * 8 + x) * 16 + e_l);
          const uint32_t kb = k0 + (uint32_t)b_sl;
          const u32x4 bv = lds_read_tr16x2(rows + (size_t)kb * RB + b_ch, rows + (size_t)(kb + 4u) * RB + b_ch);
          if constexpr (!kAcc3) {
            if (wv) Aw[wa] = wts_l[(size_t)e * 8 + (uint32_t)(dz * 4 + cdy * 2 + cdx)];
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            const u32x4 av = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const unsigned char *>(Aw) + a_rd);
            acc = Mfma16<T>::mfma(av, bv, acc);
          } else {
            // fp32 accumulation: the fp32 weight as hi + mid + lo parts
            const float4 r = lrec_l[e];
            const float fx = r.x - floorf(r.x), fy = r.y - floorf(r.y), fz = r.z - floorf(r.z);
            float wrem = ((r.w * (dz ? fz : 1.f - fz)) * (cdy ? fy : 1.f - fy)) * (cdx ? fx : 1.f - fx);
            for (int pp = 0; pp < 3; ++pp) {
              const unsigned short wb = Mfma16<T>::bits(wrem);
              if (wv) Aw[wa] = wb;
              wrem -= (float)__builtin_bit_cast(T, wb);
              __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
              const u32x4 av = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const unsigned char *>(Aw) + a_rd);
              acc = Mfma16<T>::mfma(av, bv, acc);
              __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            }
          }
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          if (wv) Aw[wa] = 0;
        }
      }
      TM(5);
      // last chunk of the tile: add the two waves' sums of each plane and write the rows (fp32
      // partial sums when the tile reaches past this block's entry range)
      if (c.last) {
        __syncthreads();
        if (ghalf == 1) {
#pragma unroll
          for (int i = 0; i < 16; ++i) xch_l[(plane * 16 + i) * 64 + lane] = acc[i];
        }
        __syncthreads();
        flushed = true;
        if (ghalf == 0 && plane < tz) {
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[i] += xch_l[(plane * 16 + i) * 64 + lane];
          const uint32_t ts = sgpr(ts_l[c.ti]), te = ts + sgpr(tc_l[c.ti]);
          const bool partial = ts < bnd0 || te > bnd1;
          const int h = lane >> 5, nch = lane & 31;
          const int z = itz * tz + plane;
          if (partial) {
            const uint32_t slot = (w0 + c.ti == first) ? 0u : 1u;
            float *ps = a.pslots + ((size_t)(bg * (uint32_t)a.bph + (uint32_t)j) * 2u + slot) * 4096u;
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) ps[(plane * 32 + 8 * m + 4 * h + rr) * 32 + nch] = acc[4 * m + rr];
          } else if (z < n0) {
            // voxel 8m + 4h + rr of the plane: x = 4h + rr, y = m
            const int x0 = itx * tx, y0 = ity * ty;
            const int64_t zrow = (int64_t)sgpr(lvsi[l]) + (int64_t)z * n1 * n2;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const int y = y0 + m;
              if (m < ty && y < n1) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                  const int xl = 4 * h + rr, x = x0 + xl;
                  if (xl < tx && x < n2) {
                    const int64_t o = (((int64_t)b * a.S + zrow + (int64_t)y * n2 + x) * G + g) * 32 + nch;
                    if constexpr (kAcc3)
                      static_cast<float *>(a.out)[o] += acc[4 * m + rr];
                    else
                      static_cast<T *>(a.out)[o] = (T)acc[4 * m + rr];
                  }
                }
              }
            }
          }
        }
      }
      TM(6);
      c = cn;
      ++ci;
    };
    while (c.valid) {
      chunk_step(IntConst<0>{});
      if (!c.valid) break;
      chunk_step(IntConst<1>{});
    }
  }
#ifdef FUSED_TIMING
  if ((threadIdx.x & 63) == 0 && a.dbg)
    for (int i = 0; i < 8; ++i) atomicAdd(a.dbg + i + 8 * ((threadIdx.x >> 6) & 3), t_acc[i]);
#endif
#undef TM
}

// Tiles cut by block boundaries: the block that holds a tile's first entry adds its own partial
// sums and those of the following blocks that cover the tile, and writes the rows.  One
// 256-thread block per tile-kernel block (same mapping); exits unless its last tile is cut.
template <typename T>
__global__ __launch_bounds__(256) void fda_bwd_fused_combine_kernel(const Args a) {
  int b, g, j;
  if (!fused_block(a, blockIdx.x, gridDim.x, b, g, j)) return;
  const int G = a.G, L = a.L, LK = a.L * a.K;
  const uint32_t bg = (uint32_t)(b * G + g);
  const uint32_t T_h = tiles_per_head(a.shapes, L, a.TX, a.TY, a.TZ);
  const uint32_t hbase = bg * 8u * (uint32_t)a.Q * (uint32_t)LK;
  const uint32_t *part = a.part + (size_t)bg * (a.bph + 2);
  const uint32_t E = part[a.bph + 1];
  const auto bnd = [&](int k) { return hbase + (uint32_t)((uint64_t)k * E / (uint32_t)a.bph); };
  if (j == a.bph - 1) return;   // the last block's range ends with the head
  const uint32_t tbase = bg * T_h;
  const uint32_t f1 = part[j + 1];
  if (f1 == 0) return;
  const uint32_t t = f1 - 1;   // this block's last tile
  const uint32_t ts = a.tile_start[tbase + t], te = ts + a.tile_counts[tbase + t];
  if (te <= bnd(j + 1) || ts < bnd(j)) return;   // not cut at the end, or not its first block
  // this block's first tile (the slot rule of the tile kernel)
  uint32_t first = part[j];
  if (first > 0) {
    const uint32_t t0 = first - 1;
    if (a.tile_start[tbase + t0] + a.tile_counts[tbase + t0] > bnd(j)) first = t0;
  }
  const int tid = threadIdx.x;
  float s[16];
  {
    const float *p = a.pslots + ((size_t)(bg * (uint32_t)a.bph + (uint32_t)j) * 2u + (first == t ? 0u : 1u)) * 4096u;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = p[i * 256 + tid];
  }
  for (int k = j + 1; k < a.bph && bnd(k) < te; ++k) {
    const float *p = a.pslots + ((size_t)(bg * (uint32_t)a.bph + (uint32_t)k) * 2u) * 4096u;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] += p[i * 256 + tid];
  }
  // element i * 256 + tid of the slot: voxel (plane*32 + v), channel
  int l = 0;
  uint32_t lb = 0;
  for (int u = 0; u < L; ++u) {
    const uint32_t cnt = level_tiles(a.shapes, u, a.TX, a.TY, a.TZ).count;
    if (t >= lb + cnt) { lb += cnt; l = u + 1; } else break;
  }
  const LevelTiles lt = level_tiles(a.shapes, l, a.TX, a.TY, a.TZ);
  const uint32_t r = t - lb;
  const int itx = (int)(r % (uint32_t)lt.nt[2]);
  const int ity = (int)((r / (uint32_t)lt.nt[2]) % (uint32_t)lt.nt[1]);
  const int itz = (int)(r / ((uint32_t)lt.nt[2] * (uint32_t)lt.nt[1]));
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int el = i * 256 + tid;
    const int nch = el & 31, vv = el >> 5;
    const int zl = vv >> 5, v = vv & 31, xl = v & 7, yl = v >> 3;
    const int x = itx * lt.t[2] + xl, y = ity * lt.t[1] + yl, z = itz * lt.t[0] + zl;
    if (xl < lt.t[2] && yl < lt.t[1] && zl < lt.t[0] && x < lt.n[2] && y < lt.n[1] && z < lt.n[0]) {
      const int64_t vox = a.lsi[l] + ((int64_t)z * lt.n[1] + y) * lt.n[2] + x;
      const int64_t o = (((int64_t)b * a.S + vox) * G + g) * 32 + nch;
      if (a.accumulate)
        static_cast<float *>(a.out)[o] += s[i];
      else
        static_cast<T *>(a.out)[o] = (T)s[i];
    }
  }
}

}  // namespace ops3d_fda
