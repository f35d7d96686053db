/*
 * fh_oracle.c -- CPU restatement of flash-hyperconnections' batched
 * small-matrix exponential (forward) and its structured Frechet derivative
 * (backward), used ONLY as the checker by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg.  Nothing in the shipped package links, loads or
 * calls this file; the product path is the HIP library under
 * flash-hyperconnections_amd/csrc/.
 *
 * Every step follows the reference source (paths relative to the reference
 * repository root):
 *   padding size P            csrc/matrix_exp.cu:65
 *   FP32 conversion + zero pad csrc/matrix_exp.cu:35-44
 *   non-finite rule            csrc/MatrixExpSmall.cuh:126-140 (tiny), :318-331 (tiled)
 *   FP64 1-norm, association   csrc/MatrixExpSmall.cuh:144-153 (P<=8 butterfly),
 *                              :343-357 (P>=16 sequential)
 *   squaring count s           csrc/MatrixExpSmall.cuh:14, :154, :356
 *   scaling by 2^-s            csrc/MatrixExpSmall.cuh:157-162, :362-367
 *   product (sequential fmaf)  csrc/MatrixExpSmall.cuh:22-52, :198-256
 *   combine                    csrc/MatrixExpSmall.cuh:66-81, :268-281
 *   degree-18 polynomial t18   csrc/MatrixExpSmall.cuh:83-106, :283-299
 *   squarings                  csrc/MatrixExpSmall.cuh:168, :373
 *   output block (D or U)      csrc/MatrixExpSmall.cuh:171-172, :376-377
 *   output rounding (RNE)      csrc/MatrixExpSmall.cuh:108-112, :302-306
 *
 * Evaluation order.  Products accumulate over k = 0..P-1 with one fmaf per
 * term starting from +0.0f, as in the reference.  The reference's combine is
 * the C expression c0*I + c1*A + c2*A2 + c3*A3 + c6*A6, compiled with FMA
 * contraction; it is restated here as the left-to-right chain
 *   t = c0*I; t = fmaf(c1,A,t); t = fmaf(c2,A2,t); t = fmaf(c3,A3,t); t = fmaf(c6,A6,t)
 * (U blocks start from c1*A).  Build with -ffp-contract=off so that the
 * compiler adds no contraction of its own.
 *
 * Parity unpinned: that contraction order.  nvcc may equally contract the
 * diagonal term first (fmaf(c0, I, c1*A)), which rounds differently on the
 * diagonal of B3/B4; no fixture of the reference tells the two apart and nvcc
 * is absent here.  fho_set_combine_contraction(1) switches this restatement
 * to that order, and tests/test_oracle.py bounds the difference between the
 * two (one rounding, amplified by the squarings).  Likewise unobservable here:
 * CUDA's log2 inside the 2^-40 band above a power of two where s needs it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define FHO_THETA18 3.010066362817634 /* csrc/MatrixExpSmall.cuh:14 */
#define FHO_MAXP 32

/* Coefficient table of the degree-18 Bader-Blanes-Casas polynomial, rows
 * B1..B5, columns (c0 for I, c1 for A, c2 for A^2, c3 for A^3, c6 for A^6);
 * FP32 literals of csrc/MatrixExpSmall.cuh:89-103. */
static const float kCoef[5][5] = {
    {0.f, -0.10036558103014462f, -0.008029246482411570f, -0.000892138498045730f, 0.f},
    {0.f, 0.39784974949645076f, 1.36783778460411719f, 0.49828962252538268f, -0.00063789819459247233f},
    {-10.96763960529620626f, 1.68015813878906197f, 0.05717798464788655f, -0.00698210122488052f,
     3.349750170860705e-05f},
    {-0.09043168323908106f, -0.06764045190713819f, 0.06759613017740597f, 0.02955525704293155f,
     -1.391802575160607e-05f},
    {0.f, 0.f, -0.09233646193671186f, -0.01693649390020817f, -1.400867981820361e-05f},
};

int fho_padded_size(int n) { return n <= 4 ? 4 : n <= 8 ? 8 : n <= 16 ? 16 : 32; }

const float* fho_coefficients(void) { return &kCoef[0][0]; }

/* 1-norm (max column sum of |.|) in FP64 of the P x P FP32 tile a (and g for
 * the augmented Frechet matrix), with the reference's summation order:
 * P in {4, 8}: lane butterfly over rows, MatrixExpSmall.cuh:146-152 (each
 *   row term is |a|+|g| when g is present, :147-148);
 * P in {16, 32}: sequential over rows, |a| then |g| per row, :346-349. */
double fho_norm1(const float* a, const float* g, int P) {
  double norm = 0.;
  for (int j = 0; j < P; ++j) {
    double col;
    if (P <= 8) {
      double x[8];
      for (int r = 0; r < P; ++r) {
        x[r] = fabs((double)a[r * P + j]);
        if (g) x[r] += fabs((double)g[r * P + j]);
      }
      if (P == 4) {
        col = (x[0] + x[2]) + (x[1] + x[3]);
      } else {
        col = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
      }
    } else {
      col = 0.;
      for (int r = 0; r < P; ++r) {
        col += fabs((double)a[r * P + j]);
        if (g) col += fabs((double)g[r * P + j]);
      }
    }
    norm = fmax(norm, col);
  }
  return norm;
}

/* s = norm > theta18 ? ceil(log2(norm / theta18)) : 0, in double
 * (MatrixExpSmall.cuh:154, :356). */
int fho_squarings(double norm) {
  return norm > FHO_THETA18 ? (int)ceil(log2(norm / FHO_THETA18)) : 0;
}

/* ---- P x P row-major FP32 algebra ------------------------------------- */

typedef struct {
  float d[FHO_MAXP * FHO_MAXP];
  float u[FHO_MAXP * FHO_MAXP];
} Tile;

/* C = A.B with per-element sequential fmaf over k from +0 (MatrixExpSmall.cuh:27-40).
 * Pair: U = (D_a.U_b) + (U_a.D_b), two separate sequential sums then one add
 * (:34-49, :243-251). */
static void product(const Tile* a, const Tile* b, Tile* c, int P, int pair) {
  for (int i = 0; i < P; ++i) {
    for (int j = 0; j < P; ++j) {
      float d = 0.f, u = 0.f, v = 0.f;
      for (int k = 0; k < P; ++k) {
        d = fmaf(a->d[i * P + k], b->d[k * P + j], d);
        if (pair) u = fmaf(a->d[i * P + k], b->u[k * P + j], u);
      }
      c->d[i * P + j] = d;
      if (pair) {
        for (int k = 0; k < P; ++k) v = fmaf(a->u[i * P + k], b->d[k * P + j], v);
        c->u[i * P + j] = u + v;
      }
    }
  }
}

static void add(const Tile* a, const Tile* b, Tile* c, int P, int pair) {
  for (int e = 0; e < P * P; ++e) {
    c->d[e] = a->d[e] + b->d[e];
    if (pair) c->u[e] = a->u[e] + b->u[e];
  }
}

/* Which way the first two terms of a combine contract.  0 (the restatement):
 * fmaf(c1, A, c0*I), one rounding.  1: fmaf(c0, I, c1*A), the other form a
 * compiler may choose for the same C expression; it rounds c1*A first, which
 * changes only diagonal entries of D.  Not observable without the reference
 * build, so tests use 1 to bound how far the choice could move results.  Set
 * it before a computation, never during one. */
static int g_contract_diag_first = 0;

void fho_set_combine_contraction(int diag_first) { g_contract_diag_first = diag_first != 0; }

/* B = c0*I + c1*A + c2*A^2 + c3*A^3 + c6*A^6; the identity goes to D only
 * (MatrixExpSmall.cuh:66-81). */
static void combine(const Tile* a, const Tile* a2, const Tile* a3, const Tile* a6, const float* c,
                    Tile* b, int P, int pair) {
  for (int i = 0; i < P; ++i) {
    for (int j = 0; j < P; ++j) {
      const int e = i * P + j;
      float t = c[0] * (float)(i == j);
      if (g_contract_diag_first && c[1] != 0.f) {
        t = fmaf(c[0], (float)(i == j), c[1] * a->d[e]);
      } else {
        t = fmaf(c[1], a->d[e], t);
      }
      t = fmaf(c[2], a2->d[e], t);
      t = fmaf(c[3], a3->d[e], t);
      t = fmaf(c[4], a6->d[e], t);
      b->d[e] = t;
      if (pair) {
        float w = c[1] * a->u[e];
        w = fmaf(c[2], a2->u[e], w);
        w = fmaf(c[3], a3->u[e], w);
        w = fmaf(c[4], a6->u[e], w);
        b->u[e] = w;
      }
    }
  }
}

/* Degree-18 polynomial (MatrixExpSmall.cuh:83-106):
 * A2=A.A, A3=A2.A, A6=A3.A3, Bk=combine(ck), A9=B1.B5+B4, T=B2+(B3+A9).A9. */
static void t18(const Tile* a, Tile* out, int P, int pair, Tile* w /* scratch, 10 tiles */) {
  Tile *a2 = &w[0], *a3 = &w[1], *a6 = &w[2], *b1 = &w[3], *b2 = &w[4], *b3 = &w[5], *b4 = &w[6],
       *b5 = &w[7], *p = &w[8], *a9 = &w[9];
  product(a, a, a2, P, pair);
  product(a2, a, a3, P, pair);
  product(a3, a3, a6, P, pair);
  combine(a, a2, a3, a6, kCoef[0], b1, P, pair);
  combine(a, a2, a3, a6, kCoef[1], b2, P, pair);
  combine(a, a2, a3, a6, kCoef[2], b3, P, pair);
  combine(a, a2, a3, a6, kCoef[3], b4, P, pair);
  combine(a, a2, a3, a6, kCoef[4], b5, P, pair);
  product(b1, b5, p, P, pair);
  add(p, b4, a9, P, pair);
  add(b3, a9, b1, P, pair); /* b1 reused as (B3 + A9) */
  product(b1, a9, p, P, pair);
  add(b2, p, out, P, pair);
}

/* One matrix.  x (and g for the Frechet/pair mode) are the n x n logical
 * matrices, row-major, already converted exactly to FP32.  Writes the n x n
 * FP32 result (before output-dtype rounding) to out, and returns s, or -1
 * when the non-finite rule fired (all outputs NaN). */
static int expm_one(const float* x, const float* g, int n, float* out, double* norm_out, Tile* w) {
  const int P = fho_padded_size(n);
  const int pair = g != NULL;
  Tile* a = &w[10];
  Tile* t = &w[11];
  Tile* sq = &w[12];
  memset(a, 0, sizeof(Tile));
  int bad = 0;
  for (int r = 0; r < n; ++r) {
    for (int c = 0; c < n; ++c) {
      a->d[r * P + c] = x[r * n + c];
      bad |= !isfinite(x[r * n + c]);
      if (pair) {
        a->u[r * P + c] = g[r * n + c];
        bad |= !isfinite(g[r * n + c]);
      }
    }
  }
  if (bad) {
    for (int e = 0; e < n * n; ++e) out[e] = NAN;
    if (norm_out) *norm_out = NAN;
    return -1;
  }
  const double norm = fho_norm1(a->d, pair ? a->u : NULL, P);
  if (norm_out) *norm_out = norm;
  const int s = fho_squarings(norm);
  const float scale = ldexpf(1.f, -s);
  for (int e = 0; e < P * P; ++e) {
    a->d[e] *= scale;
    if (pair) a->u[e] *= scale;
  }
  t18(a, t, P, pair, w);
  for (int i = 0; i < s; ++i) {
    product(t, t, sq, P, pair);
    memcpy(t, sq, sizeof(Tile));
  }
  const float* src = pair ? t->u : t->d;
  for (int r = 0; r < n; ++r)
    for (int c = 0; c < n; ++c) out[r * n + c] = src[r * P + c];
  return s;
}

static Tile* scratch_tiles(void) {
  return (Tile*)malloc(13 * sizeof(Tile));
}

/* Batched entry: x, g are contiguous FP32 [batch, n, n] (g may be NULL for the
 * forward).  out is FP32 [batch, n, n]; s_out (nullable) receives s per
 * matrix (-1 for the non-finite rule); norm_out (nullable) the FP64 norm.
 * Returns 0, or -1 for an invalid n or an allocation failure. */
int fho_matrix_exp(const float* x, const float* g, int64_t batch, int n, float* out, int32_t* s_out,
                   double* norm_out) {
  if (n < 1 || n > FHO_MAXP) return -1;
  Tile* w = scratch_tiles();
  if (!w) return -1;
  const int64_t nn = (int64_t)n * n;
  for (int64_t b = 0; b < batch; ++b) {
    double norm;
    const int s = expm_one(x + b * nn, g ? g + b * nn : NULL, n, out + b * nn, &norm, w);
    if (s_out) s_out[b] = s;
    if (norm_out) norm_out[b] = norm;
  }
  free(w);
  return 0;
}

/* Per-matrix s and norm only (no polynomial), same conventions. */
int fho_expm_params(const float* x, const float* g, int64_t batch, int n, int32_t* s_out,
                    double* norm_out) {
  if (n < 1 || n > FHO_MAXP) return -1;
  const int P = fho_padded_size(n);
  const int64_t nn = (int64_t)n * n;
  float a[FHO_MAXP * FHO_MAXP], u[FHO_MAXP * FHO_MAXP];
  for (int64_t b = 0; b < batch; ++b) {
    memset(a, 0, sizeof(a));
    memset(u, 0, sizeof(u));
    int bad = 0;
    for (int r = 0; r < n; ++r) {
      for (int c = 0; c < n; ++c) {
        a[r * P + c] = x[b * nn + r * n + c];
        bad |= !isfinite(a[r * P + c]);
        if (g) {
          u[r * P + c] = g[b * nn + r * n + c];
          bad |= !isfinite(u[r * P + c]);
        }
      }
    }
    const double norm = bad ? NAN : fho_norm1(a, g ? u : NULL, P);
    if (s_out) s_out[b] = bad ? -1 : fho_squarings(norm);
    if (norm_out) norm_out[b] = norm;
  }
  return 0;
}

/* FP32 -> bfloat16 bits, round to nearest even; NaN -> 0x7FC0
 * (c10::BFloat16(float), used by MatrixExpSmall.cuh:110, :304). */
void fho_f32_to_bf16(const float* in, uint16_t* out, int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    uint32_t bits;
    memcpy(&bits, &in[i], 4);
    if (isnan(in[i])) {
      out[i] = 0x7FC0;
    } else {
      const uint32_t lsb = (bits >> 16) & 1u;
      out[i] = (uint16_t)((bits + 0x7FFFu + lsb) >> 16);
    }
  }
}
