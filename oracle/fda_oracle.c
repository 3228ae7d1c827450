/*
 * fda_oracle.c -- CPU restatement of Flash Deformable 3D Attention, forward and backward.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this code, and only as the checker / CPU baseline.  The product
 * (ops3d_amd, libops3d_fda.so) never calls it.
 *
 * Plain scalar loops in float64 over the same packed layouts as the reference:
 *   value [B,S,G,D], spatial_shapes [L,3] rows (D,H,W), level_start_index [L],
 *   sampling_loc_attn [B,Q,G,P] with P = L*K*3 + L*K (planar: L*K (x,y,z) triples, then L*K
 *   logits), output [B,Q,G*D].
 * Algorithm followed (reference files, all under /root/reference):
 *   - softmax over all L*K logits of one (b,q,g), fp32-opmath in the reference:
 *       csrc/cuda/flash_deform_im2col_cuda.cuh:217-240
 *   - pixel coordinate loc*size - 0.5 and the sample-level range test:
 *       flash_deform_im2col_cuda.cuh:263-271; corner masking and weights: common.h:52-138.
 *     The reference's own PyTorch path (ops3d/flash_deform_attn.py:146-158) computes the same
 *     coordinate as grid_sample's ((2*loc - 1 + 1) * size - 1) / 2; with coord_mode = 1 the
 *     oracle rounds that expression step by step in fp32 (as torch does for fp32 inputs), with
 *     coord_mode = 0 it uses exact float64 arithmetic.  A sample contributes iff its coordinate
 *     lies in [-1, size) on every axis (outside it every corner is masked, so this equals zero
 *     padding; the reference's strict -1 < x differs only on the measure-zero set x == -1).
 *   - backward: grad_value scatter, location gradients scaled by the level size, attention
 *     gradient, softmax backward a_i * (g_i - sum_j a_j g_j):
 *       common.h:141-353, flash_deform_col2im_cuda.cuh:347-427.
 * Compiled with -ffp-contract=off so the fp32 coordinate steps are rounded one by one.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static double pixel_coord(double loc, int64_t size, int coord_mode) {
  if (coord_mode) {
    const float l = (float)loc;
    const float grid = 2.0f * l - 1.0f;
    const float t = (grid + 1.0f) * (float)size;
    return (double)((t - 1.0f) * 0.5f);
  }
  return loc * (double)size - 0.5;
}

/* Softmax over n logits (max-subtracted), into a[]. */
static void softmax(const double *logits, int n, double *a) {
  double m = -INFINITY, s = 0.0;
  for (int i = 0; i < n; ++i) m = logits[i] > m ? logits[i] : m;
  for (int i = 0; i < n; ++i) { a[i] = exp(logits[i] - m); s += a[i]; }
  for (int i = 0; i < n; ++i) a[i] /= s;
}

typedef struct {
  int valid;
  int64_t idx[8];   /* voxel index inside the level, -1 if the corner is outside */
  double w[8];      /* trilinear weight of each corner (order dz,dy,dx binary) */
  double dwx[8], dwy[8], dwz[8];  /* d w / d(pixel x, y, z) */
} corners_t;

static void setup(double x, double y, double z, int64_t Dl, int64_t Hl, int64_t Wl, corners_t *c) {
  c->valid = (x >= -1.0 && y >= -1.0 && z >= -1.0 && x < (double)Wl && y < (double)Hl && z < (double)Dl);
  if (!c->valid) return;
  const double x0 = floor(x), y0 = floor(y), z0 = floor(z);
  const double fx = x - x0, fy = y - y0, fz = z - z0;
  const double wx[2] = {1.0 - fx, fx}, wy[2] = {1.0 - fy, fy}, wz[2] = {1.0 - fz, fz};
  const double sx[2] = {-1.0, 1.0};
  for (int k = 0; k < 8; ++k) {
    const int dz = k >> 2, dy = (k >> 1) & 1, dx = k & 1;
    const int64_t xi = (int64_t)x0 + dx, yi = (int64_t)y0 + dy, zi = (int64_t)z0 + dz;
    const int in = xi >= 0 && xi < Wl && yi >= 0 && yi < Hl && zi >= 0 && zi < Dl;
    c->idx[k] = in ? (zi * Hl + yi) * Wl + xi : -1;
    c->w[k] = wx[dx] * wy[dy] * wz[dz];
    c->dwx[k] = sx[dx] * wy[dy] * wz[dz];
    c->dwy[k] = wx[dx] * sx[dy] * wz[dz];
    c->dwz[k] = wx[dx] * wy[dy] * sx[dz];
  }
}

void fda_oracle_forward(const double *value, const int64_t *shapes, const int64_t *lsi,
                        const double *loc_attn, double *out, int B, int S, int G, int D, int L,
                        int Q, int K, int coord_mode) {
  const int LK = L * K, P = 4 * LK;
  double attn[256];
  for (int64_t b = 0; b < B; ++b)
    for (int64_t q = 0; q < Q; ++q)
      for (int64_t g = 0; g < G; ++g) {
        const double *rec = loc_attn + ((b * Q + q) * G + g) * P;
        double *o = out + ((b * Q + q) * G + g) * D;
        for (int d = 0; d < D; ++d) o[d] = 0.0;
        softmax(rec + 3 * LK, LK, attn);
        for (int l = 0; l < L; ++l) {
          const int64_t Dl = shapes[3 * l], Hl = shapes[3 * l + 1], Wl = shapes[3 * l + 2];
          const double *vl = value + (b * S + lsi[l]) * G * D;
          for (int k = 0; k < K; ++k) {
            const int s = l * K + k;
            corners_t c;
            setup(pixel_coord(rec[3 * s], Wl, coord_mode), pixel_coord(rec[3 * s + 1], Hl, coord_mode),
                  pixel_coord(rec[3 * s + 2], Dl, coord_mode), Dl, Hl, Wl, &c);
            if (!c.valid) continue;
            for (int k8 = 0; k8 < 8; ++k8) {
              if (c.idx[k8] < 0) continue;
              const double *v = vl + (c.idx[k8] * G + g) * D;
              const double aw = attn[s] * c.w[k8];
              for (int d = 0; d < D; ++d) o[d] += aw * v[d];
            }
          }
        }
      }
}

/* grad_value [B,S,G,D] and grad_loc_attn [B,Q,G,P] are overwritten.
 * abs_mode = 1 computes, instead of the gradients, the sum of the absolute values of the terms
 * each gradient element is a sum of (|value|, |grad_out|, |d w / d pixel|, and for the logits
 * a_i * (|g_i| + sum_j a_j |g_j|)): the magnitude M that bounds the rounding error of any
 * fp32 evaluation order, |fl(x) - x| <= n * eps * M for an n-term sum.  abs_mode = 2 is
 * abs_mode = 1 with grad_value holding the number n of terms of each element instead. */
void fda_oracle_backward(const double *value, const int64_t *shapes, const int64_t *lsi,
                         const double *loc_attn, const double *grad_out, double *grad_value,
                         double *grad_loc_attn, int B, int S, int G, int D, int L, int Q, int K,
                         int coord_mode, int abs_mode) {
  const int LK = L * K, P = 4 * LK;
  double attn[256], gattn[256];
  memset(grad_value, 0, sizeof(double) * (size_t)B * S * G * D);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t q = 0; q < Q; ++q)
      for (int64_t g = 0; g < G; ++g) {
        const int64_t u = (b * Q + q) * G + g;
        const double *rec = loc_attn + u * P;
        const double *tg = grad_out + u * D;
        double *gr = grad_loc_attn + u * P;
        softmax(rec + 3 * LK, LK, attn);
        for (int l = 0; l < L; ++l) {
          const int64_t Dl = shapes[3 * l], Hl = shapes[3 * l + 1], Wl = shapes[3 * l + 2];
          const double *vl = value + (b * S + lsi[l]) * G * D;
          double *gvl = grad_value + (b * S + lsi[l]) * G * D;
          for (int k = 0; k < K; ++k) {
            const int s = l * K + k;
            corners_t c;
            setup(pixel_coord(rec[3 * s], Wl, coord_mode), pixel_coord(rec[3 * s + 1], Hl, coord_mode),
                  pixel_coord(rec[3 * s + 2], Dl, coord_mode), Dl, Hl, Wl, &c);
            double gx = 0.0, gy = 0.0, gz = 0.0, ga = 0.0;
            if (c.valid) {
              for (int k8 = 0; k8 < 8; ++k8) {
                if (c.idx[k8] < 0) continue;
                const double *v = vl + (c.idx[k8] * G + g) * D;
                double *gv = gvl + (c.idx[k8] * G + g) * D;
                double dot = 0.0;
                for (int d = 0; d < D; ++d) {
                  dot += abs_mode ? fabs(tg[d] * v[d]) : tg[d] * v[d];
                  if (abs_mode == 2)
                    gv[d] += 1.0;   /* term count */
                  else
                    gv[d] += attn[s] * c.w[k8] * (abs_mode ? fabs(tg[d]) : tg[d]);
                }
                ga += c.w[k8] * dot;
                gx += (abs_mode ? fabs(c.dwx[k8]) : c.dwx[k8]) * dot;
                gy += (abs_mode ? fabs(c.dwy[k8]) : c.dwy[k8]) * dot;
                gz += (abs_mode ? fabs(c.dwz[k8]) : c.dwz[k8]) * dot;
              }
            }
            /* d(pixel)/d(loc) = size */
            gr[3 * s] = attn[s] * gx * (double)Wl;
            gr[3 * s + 1] = attn[s] * gy * (double)Hl;
            gr[3 * s + 2] = attn[s] * gz * (double)Dl;
            gattn[s] = ga;
          }
        }
        double dot = 0.0;
        for (int i = 0; i < LK; ++i) dot += attn[i] * gattn[i];
        for (int i = 0; i < LK; ++i)
          gr[3 * LK + i] = abs_mode ? attn[i] * (gattn[i] + dot) : attn[i] * (gattn[i] - dot);
      }
}
