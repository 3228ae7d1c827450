// Stable LSD bin sort of the backward's (bin key, sample) pairs, gfx950.
//
// Keys are the bins of the samples' base corners (< 2^24 for the benchmark shapes); the sort
// runs ceil(bits / 8) passes with a digit of <= 8 bits, each pass
//   1. binsort_hist:    per tile of kTile keys an LDS histogram, written digit-major to H,
//   2. exclusive scan of H (hipCUB): the output offset of every (digit, tile),
//   3. binsort_scatter: per tile, a stable rank of every key among the tile's keys of its
//                       digit (wave-local ballot matching of the digit bits + per-wave prefix
//                       counts in LDS), key and value staged in LDS in tile-sorted order and
//                       written out from there, so a wave's stores cover runs of one digit.
// Ranks follow index order, so the sort is stable and the result deterministic.  The last pass
// does not write the sample indices: it writes, in sorted order, what the value-gradient kernel
// reads -- the sample's stash (fx, fy, fz, attn) and its grad_output row -- so no separate
// permute pass is needed.
#include <hipcub/hipcub.hpp>

#include "fda_device.h"

namespace ops3d_fda {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
#ifndef OPS3D_FDA_SORT_KPL
#define OPS3D_FDA_SORT_KPL 8
#endif
constexpr int kKeysPerLane = OPS3D_FDA_SORT_KPL;
constexpr int kTile = kSortThreads * kKeysPerLane;    // 2048 keys per tile by default
// Digit width of the passes: 8 bits (3 passes for the 23-bit keys of 2^20 voxels x 8 heads).
// Wider digits give longer coalesced runs but need kSortWaves x 2^bits LDS counters, which
// caps the blocks per CU; measured on gfx950, 8 bits is the fastest width.
constexpr int kDigitBits = 8;

__global__ __launch_bounds__(kSortThreads) void binsort_hist(const uint32_t *keys, uint32_t n, int shift,
                                                             int dbits, uint32_t *H, uint32_t ntiles) {
  __shared__ uint32_t cnt[1 << kDigitBits];
  const int nd = 1 << dbits;
  const uint32_t mask = (uint32_t)nd - 1u;
  for (int d = threadIdx.x; d < nd; d += kSortThreads) cnt[d] = 0;
  __syncthreads();
  const uint32_t t0 = blockIdx.x * (uint32_t)kTile;
#pragma unroll 4
  for (int k = 0; k < kKeysPerLane; ++k) {
    const uint32_t i = t0 + (uint32_t)k * kSortThreads + threadIdx.x;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & mask], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < nd; d += kSortThreads) H[(size_t)d * ntiles + blockIdx.x] = cnt[d];
}

struct ScatterArgs {
  const uint32_t *keys_in, *vals_in;
  uint32_t *keys_out, *vals_out;
  const uint32_t *Hs;          // exclusive scan of H
  uint32_t n, ntiles;
  int shift, dbits;
  int last;                    // final pass: write stash + grad_output row instead of vals
  const float4 *stash;         // [N] per sample (final pass)
  float4 *sorted_stash;        // [N]
  uint32_t *sorted_row;        // [N]
  double inv_lk;
  uint32_t Q, G;
  int ghm;
};

// Dynamic LDS of binsort_scatter for a digit of dbits bits.
size_t scatter_lds_bytes(int dbits) {
  const size_t nd = (size_t)1 << dbits;
  return (kSortWaves * nd + 2 * nd) * 4 + (size_t)kTile * 8;
}

// Exclusive scan over the block's threads (256 = 4 waves of 64).
__device__ inline uint32_t block_exclusive_scan(uint32_t x, uint32_t *tmp) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  uint32_t inc = x;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t y = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += y;
  }
  if (lane == kWave - 1) tmp[w] = inc;
  __syncthreads();
  uint32_t wofs = 0;
  for (int ww = 0; ww < w; ++ww) wofs += tmp[ww];
  __syncthreads();
  return wofs + inc - x;
}

// One tile of kTile keys: wave w owns keys [t0 + w*kTile/4, t0 + (w+1)*kTile/4) in index order.
//  1. per-wave digit counts (LDS atomics),
//  2. tile-local start of every (wave, digit), in index order, and the digit's global base,
//  3. stable local rank (wave-local ballot matching of the digit bits), key/value staged in LDS
//     at their tile-local sorted position,
//  4. the staged tile is written out in local order: consecutive threads write consecutive
//     positions of one digit's run, so the stores of a wave touch few cache lines.
__global__ __launch_bounds__(kSortThreads) void binsort_scatter(const ScatterArgs a) {
  extern __shared__ uint32_t sm[];
  const int nd = 1 << a.dbits;
  const uint32_t mask = (uint32_t)nd - 1u;
  uint32_t *wbase = sm;                         // [kSortWaves][nd]
  uint32_t *lstart = wbase + kSortWaves * nd;   // [nd]  tile-local start of each digit
  uint32_t *gbase = lstart + nd;                // [nd]  global position of the digit's first key
  uint32_t *skey = gbase + nd;                  // [kTile]
  uint32_t *sval = skey + kTile;                // [kTile]
  __shared__ uint32_t scan_tmp[kSortWaves];
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  constexpr int kPerWave = kTile / kSortWaves;
  const uint32_t t0 = blockIdx.x * (uint32_t)kTile;
  const uint32_t w0 = t0 + (uint32_t)w * kPerWave;

  for (int d = threadIdx.x; d < kSortWaves * nd; d += kSortThreads) wbase[d] = 0;
  __syncthreads();
  for (int r = 0; r < kPerWave / kWave; ++r) {
    const uint32_t i = w0 + (uint32_t)r * kWave + lane;
    if (i < a.n) atomicAdd(&wbase[w * nd + ((a.keys_in[i] >> a.shift) & mask)], 1u);
  }
  __syncthreads();
  // thread t owns digits [t*dpt, (t+1)*dpt)
  const int dpt = nd >= kSortThreads ? nd / kSortThreads : 1;
  const int d0 = threadIdx.x * dpt;
  const bool owns = d0 < nd;
  uint32_t tot = 0;
  if (owns)
    for (int d = d0; d < d0 + dpt; ++d)
      for (int ww = 0; ww < kSortWaves; ++ww) tot += wbase[ww * nd + d];
  uint32_t run = block_exclusive_scan(tot, scan_tmp);
  if (owns) {
    for (int d = d0; d < d0 + dpt; ++d) {
      lstart[d] = run;
      gbase[d] = a.Hs[(size_t)d * a.ntiles + blockIdx.x];
      for (int ww = 0; ww < kSortWaves; ++ww) {
        const uint32_t c = wbase[ww * nd + d];
        wbase[ww * nd + d] = run;
        run += c;
      }
    }
  }
  __syncthreads();
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int r = 0; r < kPerWave / kWave; ++r) {
    const uint32_t i = w0 + (uint32_t)r * kWave + lane;
    const bool valid = i < a.n;
    const uint32_t key = valid ? a.keys_in[i] : 0u;
    const uint32_t v = valid ? a.vals_in[i] : 0u;
    const uint32_t dg = (key >> a.shift) & mask;
    uint64_t peers = __ballot(valid);
    for (int bb = 0; bb < a.dbits; ++bb) {
      const bool bit = (dg >> bb) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    uint32_t lp = 0;
    if (valid) lp = wbase[w * nd + dg] + (uint32_t)__popcll(peers & lt);
    // every lane has read the digit's offset before the group's highest lane advances it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    if (valid && (peers >> lane) == 1ull) wbase[w * nd + dg] += (uint32_t)__popcll(peers);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (valid) {
      skey[lp] = key;
      sval[lp] = v;
    }
  }
  __syncthreads();
  const uint32_t cnt = a.n - t0 < (uint32_t)kTile ? a.n - t0 : (uint32_t)kTile;
  for (uint32_t j = threadIdx.x; j < cnt; j += kSortThreads) {
    const uint32_t key = skey[j], v = sval[j];
    const uint32_t dg = (key >> a.shift) & mask;
    const uint32_t pos = gbase[dg] + (j - lstart[dg]);
    a.keys_out[pos] = key;
    if (!a.last) {
      a.vals_out[pos] = v;
    } else {
      const uint32_t t = (uint32_t)(((double)v + 0.5) * a.inv_lk);   // v / (L*K), exact
      const uint32_t bg = t / a.Q, q = t - bg * a.Q;
      const uint32_t b = bg / a.G, g = bg - b * a.G;
      a.sorted_stash[pos] = a.stash[v];
      a.sorted_row[pos] = a.ghm ? t : (b * a.Q + q) * a.G + g;
    }
  }
}

// The scan runs over ntiles * 2^dbits counters, indexed by int.
bool binsort_supported(uint32_t n, int bits) {
  const int passes = (bits + kDigitBits - 1) / kDigitBits;
  const int dbits = (bits + passes - 1) / passes;
  const uint64_t ntiles = ((uint64_t)n + kTile - 1) / kTile;
  return bits <= 32 && (ntiles << dbits) < (1ull << 31);
}

size_t binsort_temp_bytes(uint32_t n, int bits) {
  if (!binsort_supported(n, bits)) return 0;
  const int passes = (bits + kDigitBits - 1) / kDigitBits;
  const int dbits = (bits + passes - 1) / passes;
  const size_t ntiles = (n + kTile - 1) / kTile;
  const size_t m = ntiles << dbits;
  size_t scan = 0;
  if (hipcub::DeviceScan::ExclusiveSum(nullptr, scan, (uint32_t *)nullptr, (uint32_t *)nullptr, (int)m,
                                       (hipStream_t)0) != hipSuccess)
    return 0;
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  return al(m * 4) * 2 + al(scan);
}

// Sorts (keys, vals) by the low `bits` bits of the keys; keys/vals are ping-ponged between
// the given buffers.  The final pass writes sorted keys to keys_b or keys_a (returned in
// *sorted_keys) and the sorted stash / grad_output rows.
hipError_t binsort_pairs(uint32_t *keys_a, uint32_t *vals_a, uint32_t *keys_b, uint32_t *vals_b, uint32_t n,
                         int bits, void *temp, size_t temp_bytes, const float4 *stash, float4 *sorted_stash,
                         uint32_t *sorted_row, double inv_lk, uint32_t Q, uint32_t G, int ghm,
                         const uint32_t **sorted_keys, hipStream_t st) {
  const int passes = (bits + kDigitBits - 1) / kDigitBits;
  const int dbits = (bits + passes - 1) / passes;
  const uint32_t ntiles = (n + kTile - 1) / kTile;
  const size_t m = (size_t)ntiles << dbits;
  if (!binsort_supported(n, bits)) return hipErrorInvalidValue;
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  uint32_t *H = static_cast<uint32_t *>(temp);
  uint32_t *Hs = reinterpret_cast<uint32_t *>(static_cast<char *>(temp) + al(m * 4));
  void *scan_tmp = static_cast<char *>(temp) + 2 * al(m * 4);
  size_t scan_bytes = temp_bytes - 2 * al(m * 4);
  uint32_t *kin = keys_a, *vin = vals_a, *kout = keys_b, *vout = vals_b;
  for (int p = 0; p < passes; ++p) {
    const int shift = p * dbits;
    hipLaunchKernelGGL(binsort_hist, dim3(ntiles), dim3(kSortThreads), 0, st, kin, n, shift, dbits, H, ntiles);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = hipcub::DeviceScan::ExclusiveSum(scan_tmp, scan_bytes, H, Hs, (int)m, st);
    if (e != hipSuccess) return e;
    ScatterArgs a{};
    a.keys_in = kin; a.vals_in = vin; a.keys_out = kout; a.vals_out = vout;
    a.Hs = Hs; a.n = n; a.ntiles = ntiles; a.shift = shift; a.dbits = dbits;
    a.last = p == passes - 1;
    a.stash = stash; a.sorted_stash = sorted_stash; a.sorted_row = sorted_row;
    a.inv_lk = inv_lk; a.Q = Q; a.G = G; a.ghm = ghm;
    hipLaunchKernelGGL(binsort_scatter, dim3(ntiles), dim3(kSortThreads), scatter_lds_bytes(dbits), st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    *sorted_keys = kout;
    uint32_t *tk = kin; kin = kout; kout = tk;
    uint32_t *tv = vin; vin = vout; vout = tv;
  }
  return hipSuccess;
}

}  // namespace ops3d_fda
