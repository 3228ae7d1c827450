// Phase 2 of the backward: group the samples' entries by spatial tile, gfx950.
//
// Every sample inside the volume has a key (fda_device.h, tile_key: its home tile within its
// head, "next tile" flags, level); it is listed in its home tile and in the next tile along each
// axis whose flag is set, 1 to 8 entries.  A block handles a contiguous range of one head's samples (about 64
// blocks per head) and keeps an LDS histogram over all of the head's tiles.
//
// Matrix mode (the head has at most wcap = min(tcap, kWin) tiles; tcap is what the workspace
// holds, and the LDS window is wcap tiles):
//   tile_count:    each block writes its histogram as a row of a [head][block][tile] matrix,
//   tile_headscan: per tile (64 tiles per block), exclusive prefix over the head's blocks (in
//                  place) and the tile's total,
//   tile_scatter:  every block scans its head's tile totals -> tile starts (block 0 of the
//                  head stores them); block c's entries of tile t go to tile_start[t] +
//                  prefix[c][t] + their rank among the block's entries of t (LDS staging).
//   No global atomics: every position is computed.
// Atomic mode (more tiles): the histograms are flushed with global atomics into zeroed
// counters, tile_headscan scans them per head (one block) into tile_start and the cursors,
// and tile_scatter reserves each block's range of a tile with one global atomic on
// the tile's cursor.  Correct for any size, slower (the atomics of all blocks contend).
// Heads of at most kFusedHeadSamples samples take one block each, and tile_scatter<.., true>
// counts, scans and places them in one launch (no count or head-scan launch; its counters are
// read past L1 in atomic mode, since other heads' blocks may have cached the same lines).
// Each head owns the entry range [bg * 8 * per_head, ...) (a sample has at most 8 entries), so
// heads are bucketed independently; a tile's entries are [tile_start, tile_start + count).
// The order of entries inside a tile (the LDS ranks, and in atomic mode the order of the
// reservations) decides the order of the tile kernel's fp32 sums, so grad_value can differ
// between runs at the rounding level.
#include "fda_device.h"

namespace ops3d_fda {

constexpr int kBucketThreads = 1024;
constexpr int kWin = 8192;                            // LDS histogram window (tiles of one head)
constexpr int kBlocksPerHead = 64;
constexpr uint32_t kFusedHeadSamples = 4096;          // heads this small take one fused block

struct BucketArgs {
  const uint32_t *keys;        // [N] tile_key of each sample or kKeyInvalid
  uint32_t n;                  // samples
  uint32_t per_head;           // samples per (b, g) = Q * L * K
  uint32_t chunk;              // samples per block (a block never spans two heads)
  uint32_t blocks_per_head;
  const int64_t *shapes;
  int L, BG, TX, TY, TZ;
  uint32_t *counts;            // [BG * T_h] entries per tile
  uint32_t *cursor;            // [BG * T_h]
  uint32_t *start;             // [BG * T_h + 1]
  uint32_t *mat;               // [BG][blocks_per_head][T_h] (matrix mode)
  uint32_t tcap;               // matrix mode when T_h <= tcap
  uint32_t wcap;               // LDS histogram window in tiles: min(tcap, kWin)
  uint32_t *entries;           // [<= 8N] sample indices
  uint32_t *queue;             // [8] the tile kernel's work counters, cleared here
  int fused;                   // one block per head: tile_scatter<.., true> counts and scans itself
};

__device__ __forceinline__ bool matrix_mode(const BucketArgs &a, uint32_t T_h) {
  return T_h <= a.wcap;
}

struct LevelGrid {
  uint32_t sy, sz;             // tile-id strides of the level's tile grid (y: ntx, z: ntx*nty)
};

__device__ __forceinline__ void level_grids(const BucketArgs &a, LevelGrid *lg) {
  for (int l = 0; l < a.L; ++l) {
    const LevelTiles lt = level_tiles(a.shapes, l, a.TX, a.TY, a.TZ);
    lg[l].sy = (uint32_t)lt.nt[2];
    lg[l].sz = (uint32_t)lt.nt[2] * (uint32_t)lt.nt[1];
  }
}

// Calls f(tile id) for each entry of a sample of the head whose first tile id is w0, from its
// key (tile_key): the home tile, then each of the 7 neighbour combinations (x, y, z bits of c)
// whose flags are all set.  Straight-line predicated calls: with 64 lanes every combination is
// taken by some lane, so a per-lane loop would run all 8 rounds anyway, with loop control on top.
template <typename F>
__device__ __forceinline__ void for_each_entry(uint32_t key, uint32_t w0, const LevelGrid *lg, F &&f) {
  const uint32_t fl = (key >> 3) & 7u;   // bit 0: next x tile, bit 1: y, bit 2: z
  const LevelGrid g = lg[key & 7u];
  const uint32_t home = w0 + (key >> 6);
  f(home);
  static_for<7>([&](auto cc) {
    constexpr uint32_t c = decltype(cc)::value + 1;
    if ((fl & c) == c) f(home + (c & 1u) + ((c & 2u) ? g.sy : 0u) + ((c & 4u) ? g.sz : 0u));
  });
}

__global__ __launch_bounds__(1024) void tile_clear_kernel(const BucketArgs a) {
  const uint32_t T_h = tiles_per_head(a.shapes, a.L, a.TX, a.TY, a.TZ);
  if (matrix_mode(a, T_h)) return;   // the column scan writes every counter
  const uint32_t total = (uint32_t)a.BG * T_h;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) a.counts[i] = 0u;
}

// Block -> its head, its index c among the head's blocks and its sample range [s0, s1).  With
// BG % 8 == 0 the blocks of head bg run on XCD bg % 8 (workgroups are dispatched to XCDs
// round-robin), so the partly written lines of one head's tile runs stay in one XCD's L2.
__device__ __forceinline__ uint32_t block_slot(const BucketArgs &a, uint32_t &bg, uint32_t &c) {
  if ((a.BG & 7) == 0) {
    const uint32_t x = blockIdx.x & 7u, r = blockIdx.x >> 3, hpx = (uint32_t)a.BG >> 3;
    bg = x + 8u * (r % hpx);
    c = r / hpx;
  } else {
    bg = blockIdx.x / a.blocks_per_head;
    c = blockIdx.x - bg * a.blocks_per_head;
  }
  return bg * a.blocks_per_head + c;   // row of the block in the count matrix
}

__device__ __forceinline__ void block_range(const BucketArgs &a, uint32_t &bg, uint32_t &s0, uint32_t &s1) {
  uint32_t c;
  block_slot(a, bg, c);
  const uint32_t h0 = bg * a.per_head;
  s0 = h0 + min(c * a.chunk, a.per_head);
  s1 = h0 + min((c + 1) * a.chunk, a.per_head);
}

__global__ __launch_bounds__(kBucketThreads) void tile_count_kernel(const BucketArgs a) {
  extern __shared__ uint32_t win[];   // [wcap]
  __shared__ LevelGrid lg[5];
  const uint32_t T_h = tiles_per_head(a.shapes, a.L, a.TX, a.TY, a.TZ);
  const uint32_t nw = min(T_h, a.wcap);
  if (threadIdx.x == 0) level_grids(a, lg);
  for (uint32_t i = threadIdx.x; i < nw; i += kBucketThreads) win[i] = 0u;
  __syncthreads();
  uint32_t bg, s0, s1;
  block_range(a, bg, s0, s1);
  const uint32_t w0 = bg * T_h;
  // batches of kCountBatch samples per thread: all their loads are issued before any is used
  constexpr int kCountBatch = 8;
  // all_in (every tile of the head in the window) drops the global-atomic path from the code
  const auto count_all = [&](auto all_in) {
    for (uint32_t sb = s0 + threadIdx.x; sb < s1; sb += kCountBatch * kBucketThreads) {
      uint32_t key[kCountBatch];
#pragma unroll
      for (int i = 0; i < kCountBatch; ++i) {
        const uint32_t s = sb + (uint32_t)i * kBucketThreads;
        key[i] = s < s1 ? a.keys[s] : kKeyInvalid;
      }
#pragma unroll
      for (int i = 0; i < kCountBatch; ++i) {
        if (key[i] == kKeyInvalid) continue;
        for_each_entry(key[i], w0, lg, [&](uint32_t id) {
          if (decltype(all_in)::value || id - w0 < nw) atomicAdd(&win[id - w0], 1u);
          else atomicAdd(&a.counts[id], 1u);
        });
      }
    }
  };
  if (nw == T_h) count_all(IntConst<1>{});
  else count_all(IntConst<0>{});
  __syncthreads();
  if (matrix_mode(a, T_h)) {
    uint32_t hb, hc;
    uint32_t *row = a.mat + (size_t)block_slot(a, hb, hc) * T_h;
    for (uint32_t i = threadIdx.x; i < T_h; i += kBucketThreads) row[i] = win[i];
  } else {
    for (uint32_t i = threadIdx.x; i < nw; i += kBucketThreads)
      if (win[i]) atomicAdd(&a.counts[w0 + i], win[i]);
  }
}

// Exclusive scan of cnt[0, n) (LDS) by the kBucketThreads threads of the block, thread i taking
// the run [i * per, (i + 1) * per): f(k, prefix of k) for each k, after cnt[k] is read (f may
// overwrite it).  Returns the total.  Starts and ends with a block barrier's worth of order:
// cnt must be complete before the call; f's LDS writes need a barrier before others read them.
template <typename F>
__device__ __forceinline__ uint32_t block_scan(const uint32_t *cnt, uint32_t n, uint32_t per, uint32_t *scan_tmp,
                                               F &&f) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
  const uint32_t b0 = (uint32_t)tid * per;
  uint32_t sum = 0;
  for (uint32_t i = 0; i < per; ++i)
    if (b0 + i < n) sum += cnt[b0 + i];
  uint32_t inc = wave_inclusive_scan(sum);
  if (lane == kWave - 1) scan_tmp[wv] = inc;
  __syncthreads();
  if (tid == 0) {
    uint32_t run = 0;
    for (int w = 0; w < kBucketThreads / kWave; ++w) {
      const uint32_t t = scan_tmp[w];
      scan_tmp[w] = run;
      run += t;
    }
    scan_tmp[kBucketThreads / kWave] = run;
  }
  __syncthreads();
  uint32_t run = scan_tmp[wv] + inc - sum;
  const uint32_t total = scan_tmp[kBucketThreads / kWave];
  for (uint32_t i = 0; i < per; ++i)
    if (b0 + i < n) {
      const uint32_t c = cnt[b0 + i];
      f(b0 + i, run);
      run += c;
    }
  return total;
}

// Entries are staged in LDS before they are written: a round of kRound samples is counted per
// tile, scanned, and placed in LDS grouped by tile; the writes then go out in that order, so
// consecutive lanes write consecutive positions of a tile's run instead of one scattered word
// each.  An entry past the staging capacity is written directly at the same position.
// Rounds of 4096 samples (8192 staged entries) keep two blocks on a CU for windows up to
// about 6000 tiles; a larger window leaves room for one block only, which then takes rounds of
// 8192 samples: half the per-round tile scans over the window.
constexpr int kRoundBitsSmall = 12, kRoundBitsLarge = 13;

size_t tile_scatter_lds_bytes(int round_bits, uint32_t wcap) {
  return (size_t)(2u << round_bits) * 4 + (size_t)2 * (wcap + 1) * 4;
}

int tile_scatter_round_bits(uint32_t wcap) {
  return tile_scatter_lds_bytes(kRoundBitsSmall, wcap) + 1024 <= 80 * 1024 ? kRoundBitsSmall : kRoundBitsLarge;
}

template <int kRoundBits, bool kFused>
__global__ __launch_bounds__(kBucketThreads) void tile_scatter_kernel(const BucketArgs a) {
  constexpr int kRound = 1 << kRoundBits;   // samples per staging round (kRound / kBucketThreads per thread)
  constexpr int kStage = 2 * kRound;        // staged entries per round (a round holds 1.5-1.8 per
                                            // sample on average, at most 8)
  extern __shared__ uint32_t lsm[];
  uint32_t *rec = lsm;                    // [kStage] (tile - w0) << kRoundBits | (sample - round start)
  uint32_t *win = rec + kStage;           // [wcap] next free position of the block in each tile
  uint32_t *cur = win + a.wcap + 1;       // [wcap] per-round counts, then placement cursors
  __shared__ LevelGrid lg[5];
  __shared__ uint32_t scan_tmp[kBucketThreads / kWave + 1];
  const uint32_t T_h = tiles_per_head(a.shapes, a.L, a.TX, a.TY, a.TZ);
  const uint32_t nw = min(T_h, a.wcap);
  const int tid = threadIdx.x;
  if (tid == 0) level_grids(a, lg);
  for (uint32_t i = tid; i < nw; i += kBucketThreads) {
    win[i] = 0u;
    cur[i] = 0u;
  }
  __syncthreads();
  uint32_t bg, s0, s1;
  block_range(a, bg, s0, s1);
  const uint32_t w0 = bg * T_h;
  const uint32_t per = (nw + kBucketThreads - 1) / kBucketThreads;   // tiles per thread in the scans
  const uint32_t hbase = bg * 8u * a.per_head;   // the head's entry range
  if (kFused) {
    // the head's only block (no count or head-scan launch): count its entries, scan the tile
    // totals, store counts and starts for the tile kernel
    if (blockIdx.x == 0 && tid < 8) a.queue[tid] = 0u;
    const bool mat = matrix_mode(a, T_h);
    for (uint32_t s = s0 + tid; s < s1; s += kBucketThreads) {
      const uint32_t key = a.keys[s];
      if (key == kKeyInvalid) continue;
      for_each_entry(key, w0, lg, [&](uint32_t id) {
        if (mat) atomicAdd(&cur[id - w0], 1u);
        else atomicAdd(&a.counts[id], 1u);   // zeroed by the query kernel
      });
    }
    if (mat) {
      __syncthreads();
      block_scan(cur, nw, per, scan_tmp, [&](uint32_t i, uint32_t ex) {
        a.counts[w0 + i] = cur[i];
        a.start[w0 + i] = hbase + ex;
        win[i] = hbase + ex;
        cur[i] = 0u;
      });
    } else {
      // the counters were added to in L2: wait for this wave's atomics, then read them past L1
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      uint32_t carry = hbase;
      for (uint32_t t0 = 0; t0 < T_h; t0 += kBucketThreads) {
        const uint32_t t = t0 + (uint32_t)tid;
        const uint32_t x = t < T_h ? __hip_atomic_load(&a.counts[w0 + t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        const uint32_t inc = wave_inclusive_scan(x);
        const int lane = tid & (kWave - 1), wv = tid / kWave;
        if (lane == kWave - 1) scan_tmp[wv] = inc;
        __syncthreads();
        uint32_t wofs = 0, all = 0;
        for (int w = 0; w < kBucketThreads / kWave; ++w) {
          if (w < wv) wofs += scan_tmp[w];
          all += scan_tmp[w];
        }
        __syncthreads();
        if (t < T_h) {
          a.start[w0 + t] = carry + wofs + inc - x;
          a.cursor[w0 + t] = carry + wofs + inc - x;
        }
        carry += all;
      }
      // the cursors are reserved below with atomics: let the stores land first
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }
  if (kFused && matrix_mode(a, T_h)) {
    // starts set above
  } else if (matrix_mode(a, T_h)) {
    // tile starts: the head's entry range base + exclusive scan of the tile totals; the block's
    // first position in each tile: its tile start + the earlier blocks' entries of the tile
    uint32_t hb, hc;
    const uint32_t *row = a.mat + (size_t)block_slot(a, hb, hc) * T_h;
    for (uint32_t i = tid; i < T_h; i += kBucketThreads) cur[i] = a.counts[w0 + i];
    __syncthreads();
    block_scan(cur, nw, per, scan_tmp, [&](uint32_t i, uint32_t ex) {
      win[i] = hbase + ex + row[i];
      if (hc == 0) a.start[w0 + i] = hbase + ex;
      cur[i] = 0u;
    });
  } else {
    // counts of the window's tiles, then one reservation per touched tile
#pragma unroll 4
    for (uint32_t s = s0 + tid; s < s1; s += kBucketThreads) {
      const uint32_t key = a.keys[s];
      if (key == kKeyInvalid) continue;
      for_each_entry(key, w0, lg, [&](uint32_t id) {
        if (id - w0 < nw) atomicAdd(&win[id - w0], 1u);
      });
    }
    __syncthreads();
    for (uint32_t i = tid; i < nw; i += kBucketThreads)
      if (win[i]) win[i] = atomicAdd(&a.cursor[w0 + i], win[i]);
  }
  __syncthreads();
  constexpr int SPT = kRound / kBucketThreads;
  const bool all_in = nw == T_h;   // no tile outside the window: no global-atomic path
  for (uint32_t r0 = s0; r0 < s1; r0 += kRound) {
    uint32_t key[SPT];
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const uint32_t s = r0 + (uint32_t)(k * kBucketThreads + tid);
      key[k] = s < s1 ? a.keys[s] : kKeyInvalid;
    }
    // (a) the round's entries per tile; tiles outside the window take a position at once
    const auto count_round = [&](auto all_in) {
#pragma unroll
      for (int k = 0; k < SPT; ++k) {
        if (key[k] == kKeyInvalid) continue;
        const uint32_t s = r0 + (uint32_t)(k * kBucketThreads + tid);
        for_each_entry(key[k], w0, lg, [&](uint32_t id) {
          if (decltype(all_in)::value || id - w0 < nw) atomicAdd(&cur[id - w0], 1u);
          else a.entries[atomicAdd(&a.cursor[id], 1u)] = s;
        });
      }
    };
    if (all_in) count_round(IntConst<1>{});
    else count_round(IntConst<0>{});
    __syncthreads();
    // (b) exclusive scan of the counts: cur = the tile's first staging slot; win -= that slot,
    // so that staging slot i of tile t goes to win[t] + i
    const uint32_t staged = min(block_scan(cur, nw, per, scan_tmp, [&](uint32_t i, uint32_t ex) {
                                  cur[i] = ex;
                                  win[i] -= ex;
                                }),
                                (uint32_t)kStage);
    __syncthreads();
    // (c) placement: staging slot by tile (LDS), or the final position past the capacity
    const auto place_round = [&](auto all_in) {
#pragma unroll
      for (int k = 0; k < SPT; ++k) {
        if (key[k] == kKeyInvalid) continue;
        const uint32_t so = (uint32_t)(k * kBucketThreads + tid);
        for_each_entry(key[k], w0, lg, [&](uint32_t id) {
          const uint32_t t = id - w0;
          if (decltype(all_in)::value || t < nw) {
            const uint32_t slot = atomicAdd(&cur[t], 1u);
            if (slot < (uint32_t)kStage) rec[slot] = (t << kRoundBits) | so;
            else a.entries[win[t] + slot] = r0 + so;
          }
        });
      }
    };
    if (all_in) place_round(IntConst<1>{});
    else place_round(IntConst<0>{});
    __syncthreads();
    // (d) the staged entries in tile order: runs of consecutive positions
    for (uint32_t i = tid; i < staged; i += kBucketThreads) {
      const uint32_t v = rec[i];
      const uint32_t t = v >> kRoundBits;
      a.entries[win[t] + i] = r0 + (v & (uint32_t)(kRound - 1));
    }
    __syncthreads();
    // (e) next free positions (cur ends at the tile's first slot + its count); counts cleared
    for (uint32_t i = tid; i < nw; i += kBucketThreads) {
      win[i] += cur[i];
      cur[i] = 0u;
    }
    __syncthreads();
  }
}

constexpr int kScanThreads = 256;
constexpr int kScanTiles = 64;        // tiles per head-scan block (matrix mode)

// Matrix mode: block (head, j) takes tiles [64 j, 64 j + 64) of the head, a wave per quarter of
// the head's block rows: per tile, the exclusive prefix of its counts over the blocks (in place)
// and its total (counts).  The tile starts are the scatter's (each of its blocks scans the
// totals of its head).
// Atomic mode: block (head, 0) alone: tile_start = head base + exclusive scan of the counts over
// the head's tiles; cursor = tile_start.
__global__ __launch_bounds__(kScanThreads) void tile_headscan_kernel(const BucketArgs a, uint32_t nblk) {
  __shared__ uint32_t part[kScanThreads / kWave][kScanTiles];
  const uint32_t T_h = tiles_per_head(a.shapes, a.L, a.TX, a.TY, a.TZ);
  const uint32_t bg = blockIdx.x / nblk, j = blockIdx.x - bg * nblk;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  if (blockIdx.x == 0 && tid < 8) a.queue[tid] = 0u;
  const uint32_t hbase = bg * 8u * a.per_head;   // the head's entry range
  if (matrix_mode(a, T_h)) {
    static_assert(kScanTiles == kWave && kScanThreads / kWave * 16 >= kBlocksPerHead, "row groups");
    if (j * kScanTiles >= T_h) return;
    const uint32_t t = j * kScanTiles + (uint32_t)lane;
    const bool ok = t < T_h;
    const uint32_t bph = a.blocks_per_head, R = (bph + 3) / 4;   // R <= 16
    const uint32_t r0 = (uint32_t)w * R, r1 = min(r0 + R, bph);
    uint32_t *col = a.mat + (size_t)bg * bph * T_h + t;
    uint32_t v[16], sum = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      v[k] = ok && r0 + k < r1 ? col[(size_t)(r0 + k) * T_h] : 0u;
      sum += v[k];
    }
    part[w][lane] = sum;
    __syncthreads();
    uint32_t x = 0;
    for (int g = 0; g < w; ++g) x += part[g][lane];
    if (!ok) return;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (r0 + k < r1) col[(size_t)(r0 + k) * T_h] = x;
      x += v[k];
    }
    if (w == kScanThreads / kWave - 1) a.counts[bg * T_h + t] = x;
    // no samples: no scatter block writes the starts
    if (bph == 0 && w == 0) a.start[bg * T_h + t] = hbase;
    return;
  }
  if (j != 0) return;
  __shared__ uint32_t tmp[kScanThreads / kWave];
  uint32_t carry = hbase;
  for (uint32_t base = 0; base < T_h; base += kScanThreads) {
    const uint32_t t = base + (uint32_t)tid;
    const uint32_t x = t < T_h ? a.counts[bg * T_h + t] : 0u;
    uint32_t inc = wave_inclusive_scan(x);
    if (lane == kWave - 1) tmp[w] = inc;
    __syncthreads();
    uint32_t wofs = 0, all = 0;
    for (int ww = 0; ww < kScanThreads / kWave; ++ww) {
      if (ww < w) wofs += tmp[ww];
      all += tmp[ww];
    }
    __syncthreads();
    if (t < T_h) {
      const uint32_t v = carry + wofs + inc - x;
      a.start[bg * T_h + t] = v;
      a.cursor[bg * T_h + t] = v;
    }
    carry += all;
  }
}

// LDS histogram window (tiles) of the bucketing kernels for a workspace matrix of tcap tiles; a
// head with more tiles is bucketed in atomic mode.
uint32_t tile_window(uint32_t tcap) { return tcap < (uint32_t)kWin ? (tcap > 0 ? tcap : 1u) : (uint32_t)kWin; }

// Workspace words of the matrix of tile_count (blocks x tiles of every head) for heads of up
// to tcap tiles.
size_t tile_matrix_words(uint32_t BG, uint32_t tcap) { return (size_t)BG * kBlocksPerHead * tcap; }

hipError_t launch_tile_bucketing(const uint32_t *keys, uint32_t n, uint32_t per_head,
                                 const int64_t *shapes, int L, int BG, int TX, int TY, int TZ, uint32_t *counts,
                                 uint32_t *start, uint32_t *cursor, uint32_t *mat, uint32_t tcap, uint32_t *entries, uint32_t *queue,
                                 bool counts_cleared, hipStream_t st, void (*mark)(int, hipStream_t)) {
  BucketArgs a{};
  a.keys = keys; a.n = n; a.per_head = per_head; a.shapes = shapes;
  a.L = L; a.BG = BG; a.TX = TX; a.TY = TY; a.TZ = TZ;
  a.counts = counts; a.cursor = cursor; a.start = start; a.mat = mat; a.tcap = tcap; a.entries = entries; a.queue = queue;
  // LDS sized to what the matrix can hold (tiles past the window take the global-atomic path),
  // so that two 1024-thread blocks fit on a CU
  a.wcap = tile_window(tcap);
  // about kBlocksPerHead blocks per head, each a whole number of kBucketThreads-sample steps
  a.chunk = (per_head + kBlocksPerHead - 1) / kBlocksPerHead;
  a.chunk = (a.chunk + kBucketThreads - 1) / kBucketThreads * kBucketThreads;
  if (a.chunk == 0) a.chunk = kBucketThreads;
  // small heads: one block per head that counts, scans and scatters in one launch
  a.fused = n > 0 && per_head <= kFusedHeadSamples;
  if (a.fused) a.chunk = (per_head + kBucketThreads - 1) / kBucketThreads * kBucketThreads;
  a.blocks_per_head = (per_head + a.chunk - 1) / a.chunk;
  if (n == 0) a.blocks_per_head = 0;   // every counter is zero: the head scan writes zeros
  const unsigned blocks = (unsigned)BG * a.blocks_per_head;
  if (!counts_cleared) hipLaunchKernelGGL(tile_clear_kernel, dim3(64), dim3(1024), 0, st, a);
  if (a.fused) {
    if (mark) mark(3, st);
    const int rb = tile_scatter_round_bits(a.wcap);
    if (rb == kRoundBitsSmall)
      hipLaunchKernelGGL((tile_scatter_kernel<kRoundBitsSmall, true>), dim3(blocks), dim3(kBucketThreads),
                         tile_scatter_lds_bytes(rb, a.wcap), st, a);
    else
      hipLaunchKernelGGL((tile_scatter_kernel<kRoundBitsLarge, true>), dim3(blocks), dim3(kBucketThreads),
                         tile_scatter_lds_bytes(rb, a.wcap), st, a);
    return hipGetLastError();
  }
  if (blocks > 0) hipLaunchKernelGGL(tile_count_kernel, dim3(blocks), dim3(kBucketThreads), a.wcap * 4, st, a);
  const uint32_t nblk = (a.wcap + kScanTiles - 1) / kScanTiles;   // matrix mode: T_h <= wcap
  if (BG > 0) hipLaunchKernelGGL(tile_headscan_kernel, dim3((unsigned)BG * nblk), dim3(kScanThreads), 0, st, a, nblk);
  if (mark) mark(3, st);
  if (blocks > 0) {
    const int rb = tile_scatter_round_bits(a.wcap);
    if (rb == kRoundBitsSmall)
      hipLaunchKernelGGL((tile_scatter_kernel<kRoundBitsSmall, false>), dim3(blocks), dim3(kBucketThreads),
                         tile_scatter_lds_bytes(rb, a.wcap), st, a);
    else
      hipLaunchKernelGGL((tile_scatter_kernel<kRoundBitsLarge, false>), dim3(blocks), dim3(kBucketThreads),
                         tile_scatter_lds_bytes(rb, a.wcap), st, a);
  }
  return hipGetLastError();
}

}  // namespace ops3d_fda
