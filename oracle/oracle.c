/*
 * oracle.c — CPU restatement of TRELLIS.2's submanifold sparse conv3d path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the GPU path is compared against; nothing in
 * the product library links or calls it.  It is deliberately naive (scalar loops, fp64
 * accumulation) so that it is easy to read against the reference:
 *
 *   oracle_map_sorted  hashmap_fallback: sorted packed keys + binary search per offset
 *                      (README.md:111); offsets and bounds of conv3d_wgsl.ts:91-124
 *   oracle_map_grid    the WGSL two-pass dense-grid build, conv3d_wgsl.ts:44-128, with the batch
 *                      index added to the grid (the WGSL grid has none, conv3d_wgsl.ts:67)
 *   oracle_conv        gather-GEMM-bias, conv3d_wgsl.ts:180-229 (weight index :197), fp64
 *   oracle_layernorm   src/dense/ops/layer_norm.ts:41-64 (fp64 here)
 *   oracle_silu        src/dense/ops/silu.ts:25-29
 *
 * Conventions the reference leaves open and this restatement fixes (also used by the GPU path):
 * key = ((b*X+x)*Y+y)*Z+z in int64; neighbor values are ORIGINAL row indices; tap
 * v = kd*9+kh*3+kw with offset ((kd-1)dD, (kh-1)dH, (kw-1)dW) applied to (x, y, z).
 * Status bits: 1 = duplicate coordinate, 2 = coordinate out of range (outputs then undefined).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#define ORACLE_DUPLICATE 1u
#define ORACLE_OUT_OF_RANGE 2u

typedef struct {
  int64_t key;
  int32_t row;
} kr_t;

static int cmp_kr(const void* a, const void* b) {
  const kr_t* x = (const kr_t*)a;
  const kr_t* y = (const kr_t*)b;
  if (x->key < y->key) return -1;
  if (x->key > y->key) return 1;
  return (x->row > y->row) - (x->row < y->row);
}

static int in_grid(const int32_t* c, int32_t B, int32_t X, int32_t Y, int32_t Z) {
  return c[0] >= 0 && c[0] < B && c[1] >= 0 && c[1] < X && c[2] >= 0 && c[2] < Y && c[3] >= 0 &&
         c[3] < Z;
}

int64_t oracle_pack_key(int32_t b, int32_t x, int32_t y, int32_t z, int32_t X, int32_t Y,
                        int32_t Z) {
  return (((int64_t)b * X + x) * Y + y) * Z + z;
}

/* Sorted-key hashmap (hashmap_fallback restatement).  keys_out: N sorted unique keys; perm_out:
 * original row of each sorted key; nbr_out: (N,27).  Returns status bits. */
uint32_t oracle_map_sorted(const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                           int32_t Z, const int32_t dil[3], int64_t* keys_out, int32_t* perm_out,
                           int32_t* nbr_out) {
  uint32_t status = 0;
  kr_t* kr = (kr_t*)malloc(sizeof(kr_t) * (size_t)(N > 0 ? N : 1));
  int64_t M = 0;
  for (int64_t n = 0; n < N; ++n) {
    const int32_t* c = coords + 4 * n;
    if (!in_grid(c, B, X, Y, Z)) {
      status |= ORACLE_OUT_OF_RANGE;
      continue;
    }
    kr[M].key = oracle_pack_key(c[0], c[1], c[2], c[3], X, Y, Z);
    kr[M].row = (int32_t)n;
    ++M;
  }
  qsort(kr, (size_t)M, sizeof(kr_t), cmp_kr);
  for (int64_t i = 1; i < M; ++i)
    if (kr[i].key == kr[i - 1].key) status |= ORACLE_DUPLICATE;
  for (int64_t i = 0; i < M; ++i) {
    if (keys_out) keys_out[i] = kr[i].key;
    if (perm_out) perm_out[i] = kr[i].row;
  }
  for (int64_t n = 0; n < N; ++n) {
    const int32_t* c = coords + 4 * n;
    for (int v = 0; v < 27; ++v) {
      int32_t val = -1;
      const int kd = v / 9, kh = (v / 3) % 3, kw = v % 3;
      const int32_t nx = c[1] + (kd - 1) * dil[0];
      const int32_t ny = c[2] + (kh - 1) * dil[1];
      const int32_t nz = c[3] + (kw - 1) * dil[2];
      if (in_grid(c, B, X, Y, Z) && nx >= 0 && nx < X && ny >= 0 && ny < Y && nz >= 0 && nz < Z) {
        const int64_t nk = oracle_pack_key(c[0], nx, ny, nz, X, Y, Z);
        int64_t lo = 0, hi = M; /* first position with key >= nk (searchsorted, left) */
        while (lo < hi) {
          int64_t mid = lo + (hi - lo) / 2;
          if (kr[mid].key < nk) lo = mid + 1;
          else hi = mid;
        }
        if (lo < M && kr[lo].key == nk) val = kr[lo].row;
      }
      nbr_out[n * 27 + v] = val;
    }
  }
  free(kr);
  return status;
}

/* Dense-grid build (pass0 scatter, pass1 lookup).  Needs B*X*Y*Z int32 of memory. */
uint32_t oracle_map_grid(const int32_t* coords, int64_t N, int32_t B, int32_t X, int32_t Y,
                         int32_t Z, const int32_t dil[3], int32_t* nbr_out) {
  uint32_t status = 0;
  const int64_t cells = (int64_t)B * X * Y * Z;
  int32_t* grid = (int32_t*)malloc(sizeof(int32_t) * (size_t)cells);
  if (!grid) return 0xffffffffu;
  for (int64_t i = 0; i < cells; ++i) grid[i] = -1;
  for (int64_t n = 0; n < N; ++n) { /* pass0: sp_to_lin[lin] = i */
    const int32_t* c = coords + 4 * n;
    if (!in_grid(c, B, X, Y, Z)) {
      status |= ORACLE_OUT_OF_RANGE;
      continue;
    }
    const int64_t lin = oracle_pack_key(c[0], c[1], c[2], c[3], X, Y, Z);
    if (grid[lin] >= 0) status |= ORACLE_DUPLICATE;
    grid[lin] = (int32_t)n;
  }
  for (int64_t n = 0; n < N; ++n) { /* pass1: 27 lookups */
    const int32_t* c = coords + 4 * n;
    for (int v = 0; v < 27; ++v) {
      int32_t val = -1;
      const int kd = v / 9, kh = (v / 3) % 3, kw = v % 3;
      const int32_t nx = c[1] + (kd - 1) * dil[0];
      const int32_t ny = c[2] + (kh - 1) * dil[1];
      const int32_t nz = c[3] + (kw - 1) * dil[2];
      if (in_grid(c, B, X, Y, Z) && nx >= 0 && nx < X && ny >= 0 && ny < Y && nz >= 0 && nz < Z)
        val = grid[oracle_pack_key(c[0], nx, ny, nz, X, Y, Z)];
      nbr_out[n * 27 + v] = val;
    }
  }
  free(grid);
  return status;
}

/* out[n,co] = bias[co] + sum_v sum_ci feats[nbr[n,v],ci] * W[(co*27+v)*Ci+ci]; fp64 throughout.
 * bias may be NULL. */
void oracle_conv(const double* feats, const double* weight, const double* bias,
                 const int32_t* nbr, int64_t N, int32_t Ci, int32_t Co, double* out) {
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t n = 0; n < N; ++n) {
    for (int32_t co = 0; co < Co; ++co) {
      double acc = bias ? bias[co] : 0.0;
      for (int v = 0; v < 27; ++v) {
        const int32_t src = nbr[n * 27 + v];
        if (src < 0) continue;
        const double* f = feats + (int64_t)src * Ci;
        const double* w = weight + ((int64_t)co * 27 + v) * Ci;
        for (int32_t ci = 0; ci < Ci; ++ci) acc += f[ci] * w[ci];
      }
      out[n * Co + co] = acc;
    }
  }
}

/* Row LayerNorm: mean, biased variance, (x-mean)/sqrt(var+eps)*gamma+beta. gamma/beta NULL =
 * 1/0.  apply_silu != 0 applies x*sigmoid(x) afterwards. */
void oracle_layernorm(const double* x, int64_t N, int32_t C, const double* gamma,
                      const double* beta, double eps, int32_t apply_silu, double* y) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const double* r = x + n * C;
    double mean = 0.0;
    for (int32_t c = 0; c < C; ++c) mean += r[c];
    mean /= C;
    double var = 0.0;
    for (int32_t c = 0; c < C; ++c) var += (r[c] - mean) * (r[c] - mean);
    var /= C;
    const double inv = 1.0 / sqrt(var + eps);
    for (int32_t c = 0; c < C; ++c) {
      double t = (r[c] - mean) * inv * (gamma ? gamma[c] : 1.0) + (beta ? beta[c] : 0.0);
      if (apply_silu) t = t / (1.0 + exp(-t));
      y[n * C + c] = t;
    }
  }
}

void oracle_silu(const double* x, int64_t n, double* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = x[i] / (1.0 + exp(-x[i]));
}
