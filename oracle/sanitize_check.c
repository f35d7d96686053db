/*
 * sanitize_check.c -- drives every entry point of fh_oracle.c over all sizes
 * n = 1..32, both directions, both combine contractions and inputs with
 * zeros, subnormals, values near FP32's maximum, infinities and NaNs, for a
 * build with AddressSanitizer and UndefinedBehaviorSanitizer
 * (tests/test_oracle_sanitized.py).  Checks on the way that the batched
 * forward and the parameters entry point report the same squaring count for
 * every matrix.  Test infrastructure only, like the oracle itself.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int fho_padded_size(int n);
const float* fho_coefficients(void);
double fho_norm1(const float* a, const float* g, int P);
int fho_squarings(double norm);
void fho_set_combine_contraction(int diag_first);
int fho_matrix_exp(const float* x, const float* g, int64_t batch, int n, float* out, int32_t* s_out,
                   double* norm_out);
int fho_expm_params(const float* x, const float* g, int64_t batch, int n, int32_t* s_out, double* norm_out);
void fho_f32_to_bf16(const float* in, uint16_t* out, int64_t count);

static uint64_t state = 0x9E3779B97F4A7C15ull;

/* xorshift64*: a uniform float in [-1, 1). */
static float uniform(void) {
  state ^= state >> 12;
  state ^= state << 25;
  state ^= state >> 27;
  const uint64_t r = state * 0x2545F4914F6CDD1Dull;
  return (float)((double)(r >> 11) / (double)(1ull << 52) - 1.0);
}

enum { kBatch = 6 };

int main(void) {
  const float specials[] = {0.f, -0.f, 1e-40f, -3e-39f, 3.0e38f, -3.0e38f, INFINITY, -INFINITY, NAN};
  const float scales[kBatch] = {1e-3f, 0.5f, 4.f, 60.f, 1e4f, 1.f};
  int failures = 0;
  for (int contraction = 0; contraction < 2; ++contraction) {
    fho_set_combine_contraction(contraction);
    for (int n = 1; n <= 32; ++n) {
      const size_t nn = (size_t)n * (size_t)n;
      float* x = malloc(kBatch * nn * sizeof(float));
      float* g = malloc(kBatch * nn * sizeof(float));
      float* out = malloc(kBatch * nn * sizeof(float));
      if (!x || !g || !out) return 2;
      for (int b = 0; b < kBatch; ++b)
        for (size_t e = 0; e < nn; ++e) {
          x[b * nn + e] = uniform() * scales[b];
          g[b * nn + e] = uniform();
        }
      /* The last matrix takes a special value at a few positions (one per call pattern). */
      for (int k = 0; k < 3; ++k) {
        const size_t at = (size_t)((uniform() + 1.f) * 0.5f * (float)(nn - 1));
        x[(kBatch - 1) * nn + at] = specials[(n + k) % (int)(sizeof(specials) / sizeof(specials[0]))];
      }
      for (int dir = 0; dir < 2; ++dir) {
        const float* gd = dir ? g : NULL;
        int32_t s[kBatch], s2[kBatch];
        double norm[kBatch], norm2[kBatch];
        if (fho_matrix_exp(x, gd, kBatch, n, out, s, norm) != 0) ++failures;
        if (fho_expm_params(x, gd, kBatch, n, s2, norm2) != 0) ++failures;
        for (int b = 0; b < kBatch; ++b) {
          if (s[b] != s2[b]) {
            fprintf(stderr, "n=%d dir=%d b=%d: s %d vs params %d\n", n, dir, b, s[b], s2[b]);
            ++failures;
          }
          if (s[b] >= 0 && memcmp(&norm[b], &norm2[b], sizeof(double)) != 0) {
            fprintf(stderr, "n=%d dir=%d b=%d: norms differ\n", n, dir, b);
            ++failures;
          }
        }
        uint16_t* bits = malloc(kBatch * nn * sizeof(uint16_t));
        if (!bits) return 2;
        fho_f32_to_bf16(out, bits, (int64_t)(kBatch * nn));
        free(bits);
      }
      const int P = fho_padded_size(n);
      float a[32 * 32] = {0};
      for (int r = 0; r < n; ++r)
        for (int c = 0; c < n; ++c) a[r * P + c] = x[r * n + c];
      (void)fho_squarings(fho_norm1(a, NULL, P));
      free(x);
      free(g);
      free(out);
    }
  }
  fho_set_combine_contraction(0);
  /* Invalid sizes are refused, not read. */
  float one = 1.f, res = 0.f;
  if (fho_matrix_exp(&one, NULL, 1, 0, &res, NULL, NULL) != -1) ++failures;
  if (fho_matrix_exp(&one, NULL, 1, 33, &res, NULL, NULL) != -1) ++failures;
  if (fho_expm_params(&one, NULL, 1, 33, NULL, NULL) != -1) ++failures;
  double sum = 0.;
  for (int i = 0; i < 25; ++i) sum += fho_coefficients()[i];
  if (!(sum == sum)) ++failures;
  printf("sanitized oracle run: %d failures\n", failures);
  return failures != 0;
}
