// C ABI of libops3d_fda.so: argument validation, launch geometry and the entry points.
//
// Replaces the ATen host code of the reference (csrc/cuda/flash_deform_attn_cuda.cu:20-179)
// and its template launchers (flash_deform_im2col_cuda.cuh:298-593,
// flash_deform_col2im_cuda.cuh:432-730).  Differences by design:
//   * the launch geometry is chosen here for gfx950 (wave64 units of LPU lanes, 256-thread
//     blocks of one head, XCD-aware block order); the reference's d_stride / block_thread
//     hints are accepted by the Python layer and ignored;
//   * the whole batch is one launch: im2col_step chunking gives identical results, so it is
//     only validated (min(B, step) must divide B, as flash_deform_attn_cuda.cu:56-58);
//   * outputs are written in full by the kernels, in the value dtype: no zero-fill of output,
//     grad_offset or grad_value and no fp32 -> dtype cast passes;
//   * grad_value is a gather, not a scatter: the backward groups its samples by spatial tile and
//     every grad_value row is summed in registers by the one thread group that owns its tile
//     (fp32 global atomics on gfx950 run at ~0.5 lanes/clock per CU, LDS fp32 atomics at ~0.3,
//     far below what 8 corners x D channels per sample need).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <string>

#include "../../include/ops3d_dcnv4.h"
#include "../../include/ops3d_fda.h"
#include "fda_device.h"

namespace ops3d_fda {
hipError_t launch_f32(int, int, int, const Args &, unsigned, size_t, hipStream_t);
hipError_t launch_f16(int, int, int, const Args &, unsigned, size_t, hipStream_t);
hipError_t launch_bf16(int, int, int, const Args &, unsigned, size_t, hipStream_t);
hipError_t launch_tile_bucketing(const uint32_t *keys, uint32_t n, uint32_t per_head,
                                 const int64_t *shapes, int L, int BG, int TX, int TY, int TZ, uint32_t *counts,
                                 uint32_t *start, uint32_t *cursor, uint32_t *mat, uint32_t tcap, uint32_t *entries, uint32_t *queue,
                                 bool counts_cleared, hipStream_t st, void (*mark)(int, hipStream_t));
size_t tile_matrix_words(uint32_t BG, uint32_t tcap);
uint32_t tile_window(uint32_t tcap);
}  // namespace ops3d_fda

using namespace ops3d_fda;

namespace {

thread_local std::string g_last_error;

// backward phase timing (ops3d_fda_profile_*)
// events 0..5: backward (copies | query kernel | tile count + scan | tile scatter | tile kernel)
// events 6..8: forward (head-major copy | forward kernel)
constexpr int kProfEvents = 9;
bool g_prof_on = false;
bool g_prof_recorded[2] = {false, false};
hipEvent_t g_prof_ev[kProfEvents];
bool g_prof_created = false;

void prof_mark(int i, hipStream_t st) {
  if (g_prof_on) (void)hipEventRecord(g_prof_ev[i], st);
}

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int elem_size(int dtype) {
  switch (dtype) {
    case OPS3D_FDA_F32: return 4;
    case OPS3D_FDA_F16: return 2;
    case OPS3D_FDA_BF16: return 2;
    default: return 0;
  }
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Channels per lane (CPL) and lanes per unit (LPU) for head width D: one 16-byte vector per
// lane when possible (8 x 16-bit or 4 x fp32 channels), else 24 bytes (12 x 16-bit, 6 x fp32);
// LPU = D / CPL must be a power of two <= 32 so a unit never straddles a wave.
bool pick_config(int dtype, int D, int &cpl, int &lpu) {
  const int e = elem_size(dtype);
  if (e == 0 || D <= 0) return false;
  const int cands2[2] = {8, 12}, cands4[2] = {4, 6};
  const int *cands = (e == 2) ? cands2 : cands4;
  for (int i = 0; i < 2; ++i) {
    const int c = cands[i];
    if (D % c) continue;
    const int l = D / c;
    // (D * e) % 16: the backward stages whole grad_output rows through LDS in 16-byte pieces
    if (is_pow2(l) && l <= 32 && (D * e) % 16 == 0) {
      cpl = c;
      lpu = l;
      return true;
    }
  }
  return false;
}

struct Geometry {
  Args a;
  unsigned grid;
  size_t lds;
  int cpl, lpu;
};

// DCNv4-3D convolution geometry (reference dcnv4_cuda.cu:20-91): output size per axis
// (in + 2 pad - (dil (k - 1) + 1)) / stride + 1, K = kd kh kw taps (minus the centre).
constexpr int kDcnMaxTaps = 128;
struct DcnConv {
  int kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh, dw;
  float scale;
  int remove_center, softmax, rec_stride;
  int Din, Hin, Win, Dout, Hout, Wout, K;
  bool init(int D_, int H_, int W_) {
    Din = D_; Hin = H_; Win = W_;
    if (kd < 1 || kh < 1 || kw < 1 || sd < 1 || sh < 1 || sw < 1 || dd < 1 || dh < 1 || dw < 1 || pd < 0 ||
        ph < 0 || pw < 0)
      return false;
    Dout = (Din + 2 * pd - (dd * (kd - 1) + 1)) / sd + 1;
    Hout = (Hin + 2 * ph - (dh * (kh - 1) + 1)) / sh + 1;
    Wout = (Win + 2 * pw - (dw * (kw - 1) + 1)) / sw + 1;
    K = kd * kh * kw - (remove_center ? 1 : 0);
    return Dout > 0 && Hout > 0 && Wout > 0 && K >= 1 && K <= kDcnMaxTaps;
  }
  void apply(Args &a) const {
    a.dcn = 1;
    a.dcn_softmax = softmax ? 1 : 0;
    a.dcn_remove_center = remove_center ? 1 : 0;
    a.rec_stride = rec_stride;
    a.kd = kd; a.kh = kh; a.kw = kw; a.sd = sd; a.sh = sh; a.sw = sw; a.pd = pd; a.ph = ph; a.pw = pw;
    a.dld = dd; a.dlh = dh; a.dlw = dw;
    a.Dout = Dout; a.Hout = Hout; a.Wout = Wout;
    a.offset_scale = scale;
  }
};

int common_checks(int dtype, int B, int S, int G, int D, int L, int Q, int K, int step,
                  bool backward, Geometry &geo, int max_k = 16) {
  if (elem_size(dtype) == 0) return fail(OPS3D_FDA_EINVAL, "unsupported dtype code %d", dtype);
  if (B < 0 || S < 0 || G <= 0 || D <= 0 || Q < 0)
    return fail(OPS3D_FDA_EINVAL, "invalid sizes B=%d S=%d G=%d D=%d Q=%d", B, S, G, D, Q);
  if (L < 1 || L > 5) return fail(OPS3D_FDA_EINVAL, "invalid number of scales L=%d (supported 1..5)", L);
  if (K < 1 || K > max_k)
    return fail(OPS3D_FDA_EINVAL, "invalid number of points K=%d (supported 1..%d)", K, max_k);
  if (step <= 0) return fail(OPS3D_FDA_EINVAL, "im2col_step must be positive, got %d", step);
  const int step_ = B < step ? B : step;
  if (B > 0 && B % step_ != 0)
    return fail(OPS3D_FDA_ERUNTIME, "batch(%d) must divide im2col_step(%d)", B, step_);
  if (!pick_config(dtype, D, geo.cpl, geo.lpu))
    return fail(OPS3D_FDA_EINVAL,
                "unsupported channels per head D=%d for this dtype (need D = c * 2^k, c in %s, "
                "2^k <= 32)",
                D, elem_size(dtype) == 2 ? "{8,12}" : "{4,6}");
  if ((int64_t)S * G * D > kMaxLevelElems)
    return fail(OPS3D_FDA_EINVAL, "value too large: S*G*D = %lld exceeds %lld elements per batch item",
                (long long)S * G * D, (long long)kMaxLevelElems);
  const int LK = L * K, P = 4 * LK;
  // 64-byte rows: forward and backward query kernels give each unit 8 lanes (x-pair loads)
  const int ulanes = fwd_pairs(geo.cpl, geo.lpu, elem_size(dtype)) ? 2 * geo.lpu : geo.lpu;
  const int UPB = kWavesPerBlock * (kWave / ulanes);
  const size_t lds = (size_t)UPB * (size_t)(backward ? bwd_query_lds_floats(P, LK) : P + 1) * sizeof(float);
  if (lds > 160 * 1024)   // gfx950: 160 KB of LDS per workgroup
    return fail(OPS3D_FDA_EINVAL, "L*K=%d too large for D=%d (needs %zu bytes of LDS per block)", LK, D, lds);

  Args &a = geo.a;
  a = Args{};
  a.B = B; a.S = S; a.G = G; a.D = D; a.L = L; a.K = K; a.Q = Q; a.P = P;
  a.nqb = (Q + UPB - 1) / UPB;
  a.ncol = B * a.nqb;
  int64_t grid;
  if (G % 8 == 0) {
    a.xcd_mode = 0; a.hpx = G / 8;
    grid = (int64_t)G * a.ncol;
  } else if (8 % G == 0) {
    a.xcd_mode = 1; a.xpg = 8 / G;
    grid = 8 * (((int64_t)a.ncol + a.xpg - 1) / a.xpg);
  } else {
    a.xcd_mode = 2;
    grid = (int64_t)G * a.ncol;
  }
  if (grid > 0x7fffffff) return fail(OPS3D_FDA_EINVAL, "problem too large (%lld blocks)", (long long)grid);
  geo.grid = (unsigned)grid;
  geo.lds = lds;
  return OPS3D_FDA_OK;
}

bool misaligned(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) != 0; }

hipError_t launch(int dtype, int which, const Geometry &g, hipStream_t st) {
  switch (dtype) {
    case OPS3D_FDA_F32: return launch_f32(which, g.cpl, g.lpu, g.a, g.grid, g.lds, st);
    case OPS3D_FDA_F16: return launch_f16(which, g.cpl, g.lpu, g.a, g.grid, g.lds, st);
    default: return launch_bf16(which, g.cpl, g.lpu, g.a, g.grid, g.lds, st);
  }
}

// Workspace of the backward (all offsets 256-byte aligned):
//   keys, words    : N uint32 each, N = B*Q*G*L*K samples (home tile, tile-local word)
//   stash          : N float4 (x, y, z, attn), level pixel coordinates
//   entries        : 8N uint32 sample indices (a sample is listed in at most 8 tiles)
//   counts, start, cursor : B*G*S + 1 uint32 each (a tile holds at least one voxel, so a head
//                    has at most S tiles)
//   bucketing matrix: B*G x 64 blocks x tcap uint32, tcap = S/16 + 64 tiles per head (volumes
//                    cut into more tiles are bucketed with global atomics instead)
//   tile queues    : 8 uint32 (the tile kernel's per-XCD work counters, cleared by the bucketing)
//                    and the tile kernel's split factor
//   split scratch  : when fewer than kSplitTiles tiles can exist (at least ceil(S / tile voxels)
//                    per head), kSplitSlots fp32 partial tiles [tile voxels][D] for the tile
//                    kernel's split tiles; else nothing
//   head-major copies of value (G > 1; head slices of at most head_copy_rows_max(S) rows,
//   large levels paired) and of grad_output (grad_out_copied)
constexpr uint64_t kSplitTiles = 2048, kSplitSlots = 2048;
constexpr size_t kDirectGradOutBytes = (size_t)64 << 20;

// Whether the head-major copy of value pays.  It keeps one head's rows together so that the XCD
// serving the head caches only them; a value of less than kHeadMajorMinBytes per batch item fits
// every XCD's 4 MB L2 whole, and with fewer corner reads than a head has rows (8 per sample, Q*L*K
// samples per batch and head: cross-attention with few queries) copying the rows costs more than
// gathering them in place.  The forward and the backward decide alike, so the backward ignores a
// forward workspace the forward did not fill.
constexpr uint64_t kHeadMajorMinBytes = (uint64_t)8 << 20;
bool head_major_pays(int S, int G, int D, int e, int Q, int L, int K) {
  return (uint64_t)S * G * D * e >= kHeadMajorMinBytes && (uint64_t)Q * L * K * 8 >= (uint64_t)S;
}

// Whether the backward makes the head-major copy of grad_output for the tile kernel: for G > 1
// and more than kDirectGradOutBytes (smaller ones are read in place: the copy would cost the
// query kernel more than it saves the tile kernel).
bool grad_out_copied(int B, int Q, int G, int D, int e) {
  return G > 1 && (size_t)B * Q * G * D * e > kDirectGradOutBytes;
}

struct BwdLayout {
  uint64_t n, ntiles_bound;
  uint32_t tcap, split_slots;
  size_t off_keys, off_stash, off_entries, off_counts, off_start, off_cursor, off_queue, off_split,
      off_mat, off_vhm, off_ghm;
  size_t total;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int bwd_layout(int B, int S, int G, int D, int e, int lpu, int L, int Q, int K, BwdLayout &ly) {
  ly = BwdLayout{};
  ly.n = (uint64_t)B * Q * G * L * K;
  ly.ntiles_bound = (uint64_t)B * G * (uint64_t)S;
  if (ly.n >= 0x1fffffffull || ly.ntiles_bound >= 0xfffffff0ull)
    return fail(OPS3D_FDA_EINVAL, "backward too large for 32-bit sample/tile indices (N=%llu, tiles<=%llu)",
                (unsigned long long)ly.n, (unsigned long long)ly.ntiles_bound);
  if ((uint64_t)S >= (1ull << 26) - 1)   // tile ids within a head in 26 bits (tile_key)
    return fail(OPS3D_FDA_EINVAL, "backward too large: %d voxels per batch item (at most 2^26 - 2)", S);
  size_t o = 0;
  const size_t n4 = align256(ly.n * 4);
  const size_t t4 = align256((ly.ntiles_bound + 1) * 4);
  ly.off_keys = o; o += n4;
  ly.off_stash = o; o += align256(ly.n * 16);
  ly.off_entries = o; o += align256(ly.n * 8 * 4);
  ly.off_counts = o; o += t4;
  ly.off_start = o; o += t4;
  ly.off_cursor = o; o += t4;
  ly.off_queue = o; o += 256;
  {
    const uint64_t tvox = (uint64_t)(2 * tile_threads(lpu, big_tiles(S, lpu)) / lpu);   // voxels of a nominal tile
    const uint64_t lb = (uint64_t)B * G * ((uint64_t)S + tvox - 1) / tvox;
    ly.split_slots = (S > 0 && lb < kSplitTiles) ? (uint32_t)kSplitSlots : 0u;
    ly.off_split = o; o += align256((size_t)ly.split_slots * tvox * D * 4);
  }
  ly.tcap = (uint32_t)(S / 16 + 64);
  ly.off_mat = o; o += align256(tile_matrix_words((uint32_t)(B * G), ly.tcap) * 4);
  ly.off_vhm = o; o += G > 1 && head_major_pays(S, G, D, e, Q, L, K) ? align256((size_t)B * G * (size_t)head_copy_rows_max(S, D * e) * D * e) : 0;
  ly.off_ghm = o; o += grad_out_copied(B, Q, G, D, e) ? align256((size_t)B * Q * G * D * e) : 0;
  ly.total = o;
  return OPS3D_FDA_OK;
}

// Entries per LDS chunk of the tile kernel: as many as fit next to the bin arrays in the
// block's share of the CU's 160 KB of LDS (1024 threads: one block per CU; 512: two; 256:
// three), so that one block stages its next chunk while the others compute.
int tile_chunk(int D, int e, int lpu, bool big) {
  const int rb = D * e;
  const int nt = tile_threads(lpu, big);
  const size_t bins = tile_kernel_lds_bytes(0, rb, lpu, big);
  const size_t budget = (nt >= 1024 ? 150 : (nt >= 512 ? 76 : 50)) * (size_t)1024;
  if (budget <= bins) return 0;
  int ch = (int)((budget - bins) / (size_t)(rb + 20));
  ch = ch > kTileKPT * nt ? kTileKPT * nt : ch;
  ch &= ~63;
  return ch;
}

int device_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

// [B, N, G, R words] -> [B, G, N, R words]: the head-major copy of value, so that one head's
// rows are contiguous (one head per XCD then keeps its slice in that XCD's L2).  Head slices
// are copy_head_rows rows apart; with 64-byte rows, levels larger than
// kPairedLevelBytes per head are stored as x-pair lines (copy_level): each of their rows is
// written twice.  One 16-byte chunk per thread and step when R is a multiple of 4 words, else
// one word.
__global__ __launch_bounds__(256) void head_major_kernel(const uint32_t *src, uint32_t *dst, int64_t B,
                                                         int64_t N, int G, int R, const int64_t *shapes,
                                                         const int64_t *lsi, int L, int pair_levels) {
  __shared__ int64_t lv_src[5], lv_dst[5];
  __shared__ bool lv_pair[5];
  __shared__ CopyLevel lv[5];
  __shared__ int64_t head_rows;
  const bool vec = (R & 3) == 0;
  const int Rc = vec ? R / 4 : R;                  // chunks per row
  const int64_t total = B * N * G * Rc;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (!pair_levels && total < ((int64_t)1 << 31)) {
    // no level is paired: heads N rows apart; 32-bit index arithmetic (64-bit divisions made
    // the copy VALU-bound)
    const uint32_t rc = (uint32_t)Rc, gg = (uint32_t)G, nn = (uint32_t)N;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < (uint32_t)total; i += (uint32_t)stride) {
      const uint32_t row = i / rc, c = i - row * rc;   // (b, n, g), chunk
      const uint32_t bn = row / gg, g = row - bn * gg;
      const uint32_t b = bn / nn, n = bn - b * nn;
      const uint32_t o = ((b * gg + g) * nn + n) * rc + c;
      if (vec)
        reinterpret_cast<u32x4 *>(dst)[o] = reinterpret_cast<const u32x4 *>(src)[i];
      else
        dst[o] = src[i];
    }
    return;
  }
  if (!pair_levels) {   // no level is paired: heads N rows apart
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      const int64_t c = i % Rc;
      const int64_t row = i / Rc;                    // (b, n, g)
      const int64_t g = row % G;
      const int64_t bn = row / G;
      const int64_t n = bn % N, b = bn / N;
      const int64_t o = ((b * G + g) * N + n) * Rc + c;
      if (vec)
        reinterpret_cast<u32x4 *>(dst)[o] = reinterpret_cast<const u32x4 *>(src)[i];
      else
        dst[o] = src[i];
    }
    return;
  }
  if (threadIdx.x == 0) {
    head_rows = copy_levels(shapes, lsi, L, N, R * 4, lv);
    for (int l = 0; l < L; ++l) {
      lv_src[l] = lsi[l];
      lv_dst[l] = lv[l].start;
      lv_pair[l] = lv[l].paired;
    }
  }
  __syncthreads();
  const int64_t HS = head_rows;
  if (total < ((int64_t)1 << 31) && (B * G * HS + 2) * Rc < ((int64_t)1 << 31)) {
    // the same in 32-bit index arithmetic
    const uint32_t rc = (uint32_t)Rc, gg = (uint32_t)G, nn = (uint32_t)N, hs = (uint32_t)HS;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < (uint32_t)total; i += (uint32_t)stride) {
      const uint32_t row = i / rc, c = i - row * rc;   // (b, n, g), chunk
      const uint32_t bn = row / gg, g = row - bn * gg;
      const uint32_t b = bn / nn, n = bn - b * nn;
      const uint32_t si = i;
      const uint32_t head = (b * gg + g) * hs;
      int l = L - 1;
      while (l > 0 && (int64_t)n < lv_src[l]) --l;
      const uint32_t v = n - (uint32_t)lv_src[l];
      uint32_t r0 = (uint32_t)lv_dst[l] + v;
      const bool two = lv_pair[l];
      const uint32_t r1 = (uint32_t)lv_dst[l] + 2 * v + 1;
      if (two) r0 = (uint32_t)lv_dst[l] + 2 * v + 2;
      if (vec) {
        const u32x4 x = reinterpret_cast<const u32x4 *>(src)[si];
        reinterpret_cast<u32x4 *>(dst)[(head + r0) * rc + c] = x;
        if (two) reinterpret_cast<u32x4 *>(dst)[(head + r1) * rc + c] = x;
      } else {
        const uint32_t x = src[si];
        dst[(head + r0) * rc + c] = x;
        if (two) dst[(head + r1) * rc + c] = x;
      }
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % Rc;
    const int64_t row = i / Rc;                      // (b, n, g)
    const int64_t g = row % G;
    const int64_t bn = row / G;
    const int64_t n = bn % N, b = bn / N;
    const int64_t head = (b * G + g) * HS;
    int l = L - 1;
    while (l > 0 && n < lv_src[l]) --l;              // pairing implies the standard level layout
    const int64_t v = n - lv_src[l];
    int64_t r0 = lv_dst[l] + v, r1 = -1;             // destination rows (r1: second copy)
    if (lv_pair[l]) {
      r0 = lv_dst[l] + 2 * v + 2;                    // first row of line v
      r1 = lv_dst[l] + 2 * v + 1;                    // second row of line v - 1
    }
    if (vec) {
      const u32x4 x = reinterpret_cast<const u32x4 *>(src)[i];
      reinterpret_cast<u32x4 *>(dst)[(head + r0) * Rc + c] = x;
      if (r1 >= 0) reinterpret_cast<u32x4 *>(dst)[(head + r1) * Rc + c] = x;
    } else {
      const uint32_t x = src[i];
      dst[(head + r0) * Rc + c] = x;
      if (r1 >= 0) dst[(head + r1) * Rc + c] = x;
    }
  }
}

// Zero `n` 32-bit words (a kernel, not hipMemsetAsync, so the call is capture-safe).
hipError_t launch_head_major(const void *src, void *dst, int64_t B, int64_t N, int G, int D, int esize,
                             const int64_t *shapes, const int64_t *lsi, int L, hipStream_t st) {
  const int R = D * esize / 4;
  const int64_t chunks = B * N * G * ((R & 3) == 0 ? R / 4 : R);
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  if (blocks < 1) return hipSuccess;
  hipLaunchKernelGGL(head_major_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const uint32_t *>(src), static_cast<uint32_t *>(dst), B, N, G, R, shapes, lsi, L,
                     pairing_possible(N, R * 4) ? 1 : 0);
  return hipGetLastError();
}

}  // namespace

// Device scratch of ops3d_fda_backward_noalloc: the backward workspace for callers that cannot
// allocate.  Each device holds its own copy for the life of the process; host code uses only the
// per-device address hipGetSymbolAddress returns (the array's name is a host-side stand-in).
static __device__ __align__(256) unsigned char scratch[OPS3D_FDA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address (resolved once per device), or nullptr with the error set.
void *scratch_address() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(OPS3D_FDA_ERUNTIME, "hipGetDevice failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(OPS3D_FDA_ERUNTIME, "device %d beyond the %d devices the scratch table holds", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(OPS3D_FDA_ERUNTIME, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

int ops3d_fda_abi_version(void) { return 7; }

const char *ops3d_fda_last_error(void) { return g_last_error.c_str(); }

int ops3d_fda_supported(int dtype, int channels) {
  int cpl, lpu;
  return pick_config(dtype, channels, cpl, lpu) ? 1 : 0;
}

size_t ops3d_fda_forward_workspace_bytes(int dtype, int batch, int spatial_size, int num_heads,
                                         int channels, int num_levels, int num_query, int num_point) {
  const int e = elem_size(dtype);
  if (e == 0 || batch <= 0 || spatial_size <= 0 || num_heads <= 1 || channels <= 0 || num_levels < 1 ||
      num_query <= 0 || num_point < 1)
    return 0;
  if (!head_major_pays(spatial_size, num_heads, channels, e, num_query, num_levels, num_point)) return 0;
  return align256((size_t)batch * num_heads * (size_t)head_copy_rows_max(spatial_size, channels * e) * channels * e);
}

static int forward_impl(const void *value, const int64_t *spatial_shapes, const int64_t *level_start_index,
                        const void *sampling_loc_attn, const float *ref, int ref_levels, void *output,
                        void *workspace, size_t workspace_bytes, int dtype, int batch, int spatial_size,
                        int num_heads, int channels, int num_levels, int num_query, int num_point,
                        int im2col_step, void *stream) {
  Geometry geo;
  int rc = common_checks(dtype, batch, spatial_size, num_heads, channels, num_levels, num_query,
                         num_point, im2col_step, false, geo);
  if (rc) return rc;
  if ((int64_t)batch * num_query == 0) return OPS3D_FDA_OK;
  if (!value && spatial_size > 0) return fail(OPS3D_FDA_EINVAL, "value is NULL");
  if (!spatial_shapes || !level_start_index || !sampling_loc_attn || !output)
    return fail(OPS3D_FDA_EINVAL, "NULL pointer argument");
  if (misaligned(value) || misaligned(sampling_loc_attn) || misaligned(output) || misaligned(workspace))
    return fail(OPS3D_FDA_EINVAL, "tensor data pointers must be 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  geo.a.value = value;
  prof_mark(6, st);
  const size_t need = ops3d_fda_forward_workspace_bytes(dtype, batch, spatial_size, num_heads, channels,
                                                        num_levels, num_query, num_point);
  if (workspace && need > 0 && workspace_bytes < need)
    return fail(OPS3D_FDA_EINVAL, "forward workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
  if (workspace && need > 0) {
    hipError_t e = launch_head_major(value, workspace, batch, spatial_size, num_heads, channels,
                                     elem_size(dtype), spatial_shapes, level_start_index, num_levels, st);
    if (e != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "head-major copy failed: %s", hipGetErrorString(e));
    geo.a.value = workspace;
    geo.a.vhm = 1;
    geo.a.pair_levels = pairing_possible(spatial_size, channels * elem_size(dtype)) ? 1 : 0;
  }
  geo.a.shapes = spatial_shapes;
  geo.a.lsi = level_start_index;
  geo.a.loc_attn = sampling_loc_attn;
  geo.a.ref = ref;
  geo.a.ref_levels = ref_levels;
  geo.a.out = output;
  prof_mark(7, st);
  hipError_t e = launch(dtype, 0, geo, st);
  if (e != hipSuccess)
    return fail(OPS3D_FDA_ERUNTIME, "forward kernel launch failed: %s (grid=%u, lds=%zu)",
                hipGetErrorString(e), geo.grid, geo.lds);
  prof_mark(8, st);
  if (g_prof_on) g_prof_recorded[1] = true;
  return OPS3D_FDA_OK;
}

int ops3d_fda_forward(const void *value, const int64_t *spatial_shapes,
                      const int64_t *level_start_index, const void *sampling_loc_attn,
                      void *output, void *workspace, size_t workspace_bytes, int dtype, int batch,
                      int spatial_size, int num_heads, int channels, int num_levels,
                      int num_query, int num_point, int im2col_step, void *stream) {
  g_last_error.clear();
  return forward_impl(value, spatial_shapes, level_start_index, sampling_loc_attn, nullptr, 0, output, workspace,
                      workspace_bytes, dtype, batch, spatial_size, num_heads, channels, num_levels, num_query,
                      num_point, im2col_step, stream);
}

size_t ops3d_fda_backward_workspace_bytes(int dtype, int batch, int spatial_size, int num_heads,
                                          int channels, int num_levels, int num_query, int num_point) {
  if (elem_size(dtype) == 0 || batch < 0 || spatial_size < 0 || num_heads <= 0 || channels <= 0 ||
      num_levels < 1 || num_query < 0 || num_point < 1)
    return 0;
  BwdLayout ly;
  int cpl = 0, lpu = 0;
  if (!pick_config(dtype, channels, cpl, lpu)) return 0;
  if (bwd_layout(batch, spatial_size, num_heads, channels, elem_size(dtype), tile_lanes(lpu, cpl * elem_size(dtype)),
                 num_levels, num_query, num_point, ly))
    return 0;
  return ly.total;
}

static int backward_impl(const void *value, const void *value_head_major, const int64_t *spatial_shapes,
                         const int64_t *level_start_index, const void *sampling_loc_attn,
                         const void *grad_output, void *grad_value, bool out_f32_accumulate,
                         void *grad_sampling_loc_attn, void *workspace, size_t workspace_bytes,
                         int dtype, int batch, int spatial_size, int num_heads, int channels,
                         int num_levels, int num_query, int num_point, int im2col_step,
                         hipStream_t st, const float *ref = nullptr, int ref_levels = 0,
                         float *grad_ref = nullptr, const DcnConv *dcn = nullptr) {
  Geometry geo;
  int rc = common_checks(dtype, batch, spatial_size, num_heads, channels, num_levels, num_query,
                         num_point, im2col_step, true, geo, dcn ? kDcnMaxTaps : 16);
  if (rc) return rc;
  BwdLayout ly;
  rc = bwd_layout(batch, spatial_size, num_heads, channels, elem_size(dtype),
                  tile_lanes(geo.lpu, geo.cpl * elem_size(dtype)), num_levels, num_query, num_point, ly);
  if (rc) return rc;
  const int64_t nval = (int64_t)batch * spatial_size * num_heads * channels;
  const bool work = (int64_t)batch * num_query > 0;
  if (nval == 0 && !work) return OPS3D_FDA_OK;
  if ((int64_t)batch * num_query * num_heads * channels >= ((int64_t)1 << 32))
    return fail(OPS3D_FDA_EINVAL, "grad_output too large for 32-bit element offsets (B*Q*G*D >= 2^32)");
  if (nval > 0 && !grad_value) return fail(OPS3D_FDA_EINVAL, "grad_value is NULL");
  if (!spatial_shapes || !level_start_index) return fail(OPS3D_FDA_EINVAL, "NULL pointer argument");
  if (work && (!sampling_loc_attn || !grad_output || !grad_sampling_loc_attn || (!value && spatial_size > 0)))
    return fail(OPS3D_FDA_EINVAL, "NULL pointer argument");
  if (!workspace || workspace_bytes < ly.total)
    return fail(OPS3D_FDA_EINVAL, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, ly.total);
  if (misaligned(value) || misaligned(sampling_loc_attn) || misaligned(grad_output) ||
      misaligned(grad_sampling_loc_attn) || misaligned(grad_value))
    return fail(OPS3D_FDA_EINVAL, "tensor data pointers must be 4-byte aligned");
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(OPS3D_FDA_EINVAL, "workspace must be 256-byte aligned");

  char *ws = static_cast<char *>(workspace);
  uint32_t *keys = reinterpret_cast<uint32_t *>(ws + ly.off_keys);
  float4 *stash = reinterpret_cast<float4 *>(ws + ly.off_stash);
  uint32_t *entries = reinterpret_cast<uint32_t *>(ws + ly.off_entries);
  uint32_t *counts = reinterpret_cast<uint32_t *>(ws + ly.off_counts);
  uint32_t *tstart = reinterpret_cast<uint32_t *>(ws + ly.off_start);
  uint32_t *cursor = reinterpret_cast<uint32_t *>(ws + ly.off_cursor);

  Args &a = geo.a;
  a.value = value;
  a.shapes = spatial_shapes;
  a.lsi = level_start_index;
  a.loc_attn = sampling_loc_attn;
  a.ref = ref;
  a.ref_levels = ref_levels;
  a.grad_ref = grad_ref;
  if (dcn) dcn->apply(a);
  a.grad_out = grad_output;
  a.grad_loc_attn = grad_sampling_loc_attn;
  a.keys = keys;
  a.stash = stash;
  a.tile_counts = counts;
  a.tile_start = tstart;
  a.tile_cursor = cursor;
  a.entries = entries;
  a.tile_queue = reinterpret_cast<uint32_t *>(ws + ly.off_queue);
  a.count_clear_wcap = tile_window(ly.tcap);   // the query kernel clears the counters (atomic mode)
  a.split_scratch = reinterpret_cast<float *>(ws + ly.off_split);
  a.split_slots = ly.split_slots;
  {
    const int tl = tile_lanes(geo.lpu, geo.cpl * elem_size(dtype));
    a.big_tiles = big_tiles(spatial_size, tl) ? 1 : 0;
    tile_dims(tl, a.TX, a.TY, a.TZ, a.big_tiles != 0);
  }
  a.inv_lk = 1.0 / (double)(num_levels * num_point);
  hipError_t e;
  prof_mark(0, st);
  if (work && num_heads > 1 && head_major_pays(spatial_size, num_heads, channels, elem_size(dtype), num_query, num_levels, num_point)) {
    // head-major value (one head's rows contiguous): the caller's copy, or made here
    if (value_head_major) {
      a.value = value_head_major;
    } else {
      e = launch_head_major(value, ws + ly.off_vhm, batch, spatial_size, num_heads, channels, elem_size(dtype),
                            spatial_shapes, level_start_index, num_levels, st);
      if (e != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "head-major copy failed: %s", hipGetErrorString(e));
      a.value = ws + ly.off_vhm;
    }
    a.vhm = 1;
    a.pair_levels = pairing_possible(spatial_size, channels * elem_size(dtype)) ? 1 : 0;
  }
  // the query kernel writes the head-major copy of grad_output as it reads it
  if (work && grad_out_copied(batch, num_query, num_heads, channels, elem_size(dtype))) a.gout_hm = ws + ly.off_ghm;
  prof_mark(1, st);
  if (work) {
    // phase 1: location / logit gradients, per-sample home tile, tile-local corner and stash
    e = launch(dtype, 1, geo, st);
    if (e != hipSuccess)
      return fail(OPS3D_FDA_ERUNTIME, "backward query kernel launch failed: %s (grid=%u, lds=%zu)",
                  hipGetErrorString(e), geo.grid, geo.lds);
  }
  prof_mark(2, st);
  // phase 2: entries grouped by tile (counters are cleared even without samples: the tile
  // kernel reads the tile ranges of every tile)
  e = launch_tile_bucketing(keys, work ? (uint32_t)ly.n : 0u,
                            (uint32_t)num_query * (uint32_t)(num_levels * num_point), spatial_shapes, num_levels,
                            batch * num_heads, a.TX, a.TY, a.TZ, counts, tstart, cursor,
                            reinterpret_cast<uint32_t *>(ws + ly.off_mat), ly.tcap, entries,
                            reinterpret_cast<uint32_t *>(ws + ly.off_queue), work, st,
                            g_prof_on ? prof_mark : nullptr);
  if (e != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "tile bucketing failed: %s", hipGetErrorString(e));
  prof_mark(4, st);
  if (nval > 0) {
    // phase 3: one owner per grad_value row (per tile, in registers), written once
    Geometry g3 = geo;
    g3.a.out = grad_value;
    g3.a.accumulate = out_f32_accumulate ? 1 : 0;
    g3.a.tile_affinity = num_heads % 8 == 0;
    g3.a.chunk = tile_chunk(channels, elem_size(dtype), tile_lanes(geo.lpu, geo.cpl * elem_size(dtype)),
                            a.big_tiles != 0);
    g3.lds = tile_kernel_lds_bytes(g3.a.chunk, channels * elem_size(dtype),
                                   tile_lanes(geo.lpu, geo.cpl * elem_size(dtype)), a.big_tiles != 0);
    g3.grid = (unsigned)device_cus();   // times the resident blocks per CU (launch_one)
    if (g3.a.tile_affinity) g3.grid = (g3.grid + 7) & ~7u;
    if (g3.a.chunk < 64 || g3.lds > 160 * 1024)
      return fail(OPS3D_FDA_EINVAL, "channels per head D=%d too large for the backward tile kernel", channels);
    e = launch(dtype, 2, g3, st);
    if (e != hipSuccess)
      return fail(OPS3D_FDA_ERUNTIME, "backward tile kernel launch failed: %s (grid=%u, lds=%zu)",
                  hipGetErrorString(e), g3.grid, g3.lds);
    if (ly.split_slots > 0) {
      // split tiles: add the parts' partial sums (a split needs at least 2 parts per tile, so a
      // group has at most slots / (2 * groups) tiles; the kernel exits when nothing was split)
      Geometry g4 = g3;
      g4.grid = ly.split_slots / 2;
      g4.lds = 0;
      e = launch(dtype, 3, g4, st);
      if (e != hipSuccess)
        return fail(OPS3D_FDA_ERUNTIME, "split combine kernel launch failed: %s", hipGetErrorString(e));
    }
  }
  prof_mark(5, st);
  if (g_prof_on) g_prof_recorded[0] = true;
  return OPS3D_FDA_OK;
}

int ops3d_fda_profile_enable(int on) {
  if (on && !g_prof_created) {
    for (int i = 0; i < kProfEvents; ++i)
      if (hipEventCreate(&g_prof_ev[i]) != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "hipEventCreate failed");
    g_prof_created = true;
  }
  g_prof_on = on != 0;
  g_prof_recorded[0] = g_prof_recorded[1] = false;
  return OPS3D_FDA_OK;
}

int ops3d_fda_profile_read(int which, float *ms, int n) {
  if (which < 0 || which > 1 || !g_prof_recorded[which] || !ms) return 0;
  const int first = which == 0 ? 0 : 6, last = which == 0 ? 5 : 8;
  if (hipEventSynchronize(g_prof_ev[last]) != hipSuccess) return 0;
  int k = 0;
  for (int i = first; i < last && k < n; ++i, ++k)
    if (hipEventElapsedTime(&ms[k], g_prof_ev[i], g_prof_ev[i + 1]) != hipSuccess) ms[k] = -1.f;
  return k;
}

int ops3d_fda_backward(const void *value, const int64_t *spatial_shapes,
                       const int64_t *level_start_index, const void *sampling_loc_attn,
                       const void *grad_output, void *grad_value,
                       void *grad_sampling_loc_attn, void *workspace, size_t workspace_bytes,
                       int dtype, int batch, int spatial_size, int num_heads, int channels,
                       int num_levels, int num_query, int num_point, int im2col_step,
                       void *stream) {
  g_last_error.clear();
  return backward_impl(value, nullptr, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
                       grad_value, false, grad_sampling_loc_attn, workspace, workspace_bytes, dtype, batch, spatial_size,
                       num_heads, channels, num_levels, num_query, num_point, im2col_step,
                       static_cast<hipStream_t>(stream));
}

int ops3d_fda_backward_ex(const void *value, const void *value_head_major, const int64_t *spatial_shapes,
                          const int64_t *level_start_index, const void *sampling_loc_attn,
                          const void *grad_output, void *grad_value, void *grad_sampling_loc_attn,
                          void *workspace, size_t workspace_bytes, int dtype, int batch, int spatial_size,
                          int num_heads, int channels, int num_levels, int num_query, int num_point,
                          int im2col_step, void *stream) {
  g_last_error.clear();
  if (value_head_major && misaligned(value_head_major))
    return fail(OPS3D_FDA_EINVAL, "value_head_major must be 4-byte aligned");
  return backward_impl(value, value_head_major, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
                       grad_value, false, grad_sampling_loc_attn, workspace, workspace_bytes, dtype, batch,
                       spatial_size, num_heads, channels, num_levels, num_query, num_point, im2col_step,
                       static_cast<hipStream_t>(stream));
}

int ops3d_fda_backward_accumulate_f32(const void *value, const int64_t *spatial_shapes,
                                      const int64_t *level_start_index,
                                      const void *sampling_loc_attn, const void *grad_output,
                                      float *grad_value_f32, void *grad_sampling_loc_attn,
                                      void *workspace, size_t workspace_bytes, int dtype, int batch,
                                      int spatial_size, int num_heads, int channels, int num_levels,
                                      int num_query, int num_point, int im2col_step, void *stream) {
  g_last_error.clear();
  return backward_impl(value, nullptr, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
                       grad_value_f32, true, grad_sampling_loc_attn, workspace, workspace_bytes, dtype, batch,
                       spatial_size, num_heads, channels, num_levels, num_query, num_point, im2col_step,
                       static_cast<hipStream_t>(stream));
}

int ops3d_fda_backward_noalloc(const void *value, const int64_t *spatial_shapes,
                               const int64_t *level_start_index, const void *sampling_loc_attn,
                               const void *grad_output, void *grad_value, void *grad_sampling_loc_attn,
                               int dtype, int batch, int spatial_size, int num_heads, int channels,
                               int num_levels, int num_query, int num_point, int im2col_step, void *stream) {
  g_last_error.clear();
  Geometry geo;
  int rc = common_checks(dtype, batch, spatial_size, num_heads, channels, num_levels, num_query, num_point,
                         im2col_step, true, geo);
  if (rc) return rc;
  const size_t need = ops3d_fda_backward_workspace_bytes(dtype, batch, spatial_size, num_heads, channels,
                                                         num_levels, num_query, num_point);
  if (need > (size_t)OPS3D_FDA_NOALLOC_SCRATCH_BYTES)
    return fail(OPS3D_FDA_EINVAL,
                "problem too large for the allocation-free backward: needs %zu bytes of scratch, the "
                "library holds %zu (use ops3d_fda_backward with a caller workspace)",
                need, (size_t)OPS3D_FDA_NOALLOC_SCRATCH_BYTES);
  void *ws = scratch_address();
  if (!ws) return OPS3D_FDA_ERUNTIME;
  return backward_impl(value, nullptr, spatial_shapes, level_start_index, sampling_loc_attn, grad_output,
                       grad_value, false, grad_sampling_loc_attn, ws, (size_t)OPS3D_FDA_NOALLOC_SCRATCH_BYTES, dtype,
                       batch, spatial_size, num_heads, channels, num_levels, num_query, num_point, im2col_step,
                       static_cast<hipStream_t>(stream));
}

// Offset mode: checks of the reference points shared by both entry points.
static int offsets_checks(const float *reference_points, int ref_levels, int num_levels) {
  if (!reference_points) return fail(OPS3D_FDA_EINVAL, "reference_points is NULL");
  if (ref_levels != 1 && ref_levels != num_levels)
    return fail(OPS3D_FDA_EINVAL, "ref_levels must be 1 or num_levels (%d), got %d", num_levels, ref_levels);
  if (misaligned(reference_points)) return fail(OPS3D_FDA_EINVAL, "reference_points must be 4-byte aligned");
  return OPS3D_FDA_OK;
}

int ops3d_fda_forward_offsets(const void *value, const int64_t *spatial_shapes, const int64_t *level_start_index,
                              const void *offset_attn, const float *reference_points, int ref_levels, void *output,
                              void *workspace, size_t workspace_bytes, int dtype, int batch, int spatial_size,
                              int num_heads, int channels, int num_levels, int num_query, int num_point,
                              int im2col_step, void *stream) {
  g_last_error.clear();
  if ((int64_t)batch * num_query > 0) {
    const int rc = offsets_checks(reference_points, ref_levels, num_levels);
    if (rc) return rc;
  }
  return forward_impl(value, spatial_shapes, level_start_index, offset_attn, reference_points, ref_levels, output,
                      workspace, workspace_bytes, dtype, batch, spatial_size, num_heads, channels, num_levels,
                      num_query, num_point, im2col_step, stream);
}

int ops3d_fda_backward_offsets(const void *value, const void *value_head_major, const int64_t *spatial_shapes,
                               const int64_t *level_start_index, const void *offset_attn,
                               const float *reference_points, int ref_levels, const void *grad_output,
                               void *grad_value, void *grad_offset_attn, float *grad_reference_points,
                               void *workspace, size_t workspace_bytes,
                               int dtype, int batch, int spatial_size, int num_heads, int channels, int num_levels,
                               int num_query, int num_point, int im2col_step, void *stream) {
  g_last_error.clear();
  if ((int64_t)batch * num_query > 0) {
    const int rc = offsets_checks(reference_points, ref_levels, num_levels);
    if (rc) return rc;
  }
  if (value_head_major && misaligned(value_head_major))
    return fail(OPS3D_FDA_EINVAL, "value_head_major must be 4-byte aligned");
  return backward_impl(value, value_head_major, spatial_shapes, level_start_index, offset_attn, grad_output,
                       grad_value, false, grad_offset_attn, workspace, workspace_bytes, dtype, batch, spatial_size,
                       num_heads, channels, num_levels, num_query, num_point, im2col_step,
                       static_cast<hipStream_t>(stream), reference_points, ref_levels, grad_reference_points);
}

// ----------------------------------------------------------------------------------------------
// DCNv4-3D (reference csrc/dcnv4.h:7-60 -> csrc/cuda/dcnv4_cuda.cu:20-189): the same kernels in
// DCN mode (one level = the input volume, records of K offset triples and K mask values per
// group in rows of padded_offset_dim, pixel coordinates formed in the kernels).  The level's
// spatial_shapes / level_start_index, which the kernels read from device memory, are written
// into the first 256 bytes of the workspace by a one-thread kernel (no host copy).

__global__ void dcn_meta_kernel(int64_t *meta, int D, int H, int W) {
  meta[0] = D;
  meta[1] = H;
  meta[2] = W;
  meta[3] = 0;
}

static int dcn_setup(DcnConv &c, int dtype, int batch, int din, int hin, int win, int group, int group_channels,
                     int kd, int kh, int kw, int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                     float offset_scale, int remove_center, int softmax, int padded_offset_dim) {
  c.kd = kd; c.kh = kh; c.kw = kw; c.sd = sd; c.sh = sh; c.sw = sw; c.pd = pd; c.ph = ph; c.pw = pw;
  c.dd = dd; c.dh = dh; c.dw = dw;
  c.scale = offset_scale;
  c.remove_center = remove_center;
  c.softmax = softmax;
  c.rec_stride = padded_offset_dim;
  if (elem_size(dtype) == 0) return fail(OPS3D_FDA_EINVAL, "unsupported dtype code %d", dtype);
  if (batch < 0 || din < 1 || hin < 1 || win < 1 || group < 1 || group_channels < 1)
    return fail(OPS3D_FDA_EINVAL, "invalid sizes");
  if (!c.init(din, hin, win))
    return fail(OPS3D_FDA_EINVAL, "invalid kernel / stride / pad / dilation (or more than %d taps)", kDcnMaxTaps);
  if (padded_offset_dim < group * 4 * c.K)
    return fail(OPS3D_FDA_EINVAL, "padded_offset_dim %d smaller than group * 4 * K = %d", padded_offset_dim,
                group * 4 * c.K);
  return OPS3D_FDA_OK;
}

size_t ops3d_dcnv4_workspace_bytes(int dtype, int batch, int din, int hin, int win, int group, int group_channels,
                                   int kd, int kh, int kw, int sd, int sh, int sw, int pd, int ph, int pw, int dd,
                                   int dh, int dw, int remove_center, int backward) {
  DcnConv c;
  const std::string saved = g_last_error;
  const int rc = dcn_setup(c, dtype, batch, din, hin, win, group, group_channels, kd, kh, kw, sd, sh, sw, pd, ph, pw,
                           dd, dh, dw, 1.f, remove_center, 0, 1 << 30);
  g_last_error = saved;
  if (rc) return 0;
  if (!backward) return 256;
  int cpl = 0, lpu = 0;
  if (!pick_config(dtype, group_channels, cpl, lpu)) return 0;
  BwdLayout ly;
  if (bwd_layout(batch, din * hin * win, group, group_channels, elem_size(dtype),
                 tile_lanes(lpu, cpl * elem_size(dtype)), 1, c.Dout * c.Hout * c.Wout, c.K, ly)) {
    g_last_error = saved;
    return 0;
  }
  return 256 + ly.total;
}

int ops3d_dcnv4_forward(const void *value, const void *offset, void *output, void *workspace, size_t workspace_bytes,
                        int dtype, int batch, int din, int hin, int win, int group, int group_channels, int kd, int kh,
                        int kw, int sd, int sh, int sw, int pd, int ph, int pw, int dd, int dh, int dw,
                        float offset_scale, int remove_center, int softmax, int padded_offset_dim, int im2col_step,
                        void *stream) {
  g_last_error.clear();
  DcnConv c;
  int rc = dcn_setup(c, dtype, batch, din, hin, win, group, group_channels, kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh,
                     dw, offset_scale, remove_center, softmax, padded_offset_dim);
  if (rc) return rc;
  const int Q = c.Dout * c.Hout * c.Wout;
  Geometry geo;
  rc = common_checks(dtype, batch, din * hin * win, group, group_channels, 1, Q, c.K, im2col_step, false, geo,
                     kDcnMaxTaps);
  if (rc) return rc;
  if (batch == 0) return OPS3D_FDA_OK;
  if (!value || !offset || !output || !workspace) return fail(OPS3D_FDA_EINVAL, "NULL pointer argument");
  if (workspace_bytes < 256 || (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(OPS3D_FDA_EINVAL, "workspace must be at least 256 bytes, 256-byte aligned");
  if (misaligned(value) || misaligned(offset) || misaligned(output))
    return fail(OPS3D_FDA_EINVAL, "tensor data pointers must be 4-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t *meta = static_cast<int64_t *>(workspace);
  hipLaunchKernelGGL(dcn_meta_kernel, dim3(1), dim3(1), 0, st, meta, din, hin, win);
  geo.a.value = value;
  geo.a.shapes = meta;
  geo.a.lsi = meta + 3;
  geo.a.loc_attn = offset;
  geo.a.out = output;
  c.apply(geo.a);
  hipError_t e = launch(dtype, 0, geo, st);
  if (e != hipSuccess) return fail(OPS3D_FDA_ERUNTIME, "dcnv4 forward launch failed: %s", hipGetErrorString(e));
  return OPS3D_FDA_OK;
}

int ops3d_dcnv4_backward(const void *value, const void *offset, const void *grad_output, void *grad_value,
                         void *grad_offset, void *workspace, size_t workspace_bytes, int dtype, int batch, int din,
                         int hin, int win, int group, int group_channels, int kd, int kh, int kw, int sd, int sh,
                         int sw, int pd, int ph, int pw, int dd, int dh, int dw, float offset_scale,
                         int remove_center, int softmax, int padded_offset_dim, int im2col_step, void *stream) {
  g_last_error.clear();
  DcnConv c;
  int rc = dcn_setup(c, dtype, batch, din, hin, win, group, group_channels, kd, kh, kw, sd, sh, sw, pd, ph, pw, dd, dh,
                     dw, offset_scale, remove_center, softmax, padded_offset_dim);
  if (rc) return rc;
  if (!workspace || workspace_bytes < 256 || (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(OPS3D_FDA_EINVAL, "workspace must be at least 256 bytes, 256-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t *meta = static_cast<int64_t *>(workspace);
  hipLaunchKernelGGL(dcn_meta_kernel, dim3(1), dim3(1), 0, st, meta, din, hin, win);
  return backward_impl(value, nullptr, meta, meta + 3, offset, grad_output, grad_value, false, grad_offset,
                       static_cast<unsigned char *>(workspace) + 256, workspace_bytes - 256, dtype, batch,
                       din * hin * win, group, group_channels, 1, c.Dout * c.Hout * c.Wout, c.K, im2col_step, st,
                       nullptr, 0, nullptr, &c);
}

}  // extern "C"
