/*
 * msm_f64.c -- float64 brute-force restatement of MuSc's mutual scoring.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and bench.py's CPU-baseline leg as
 * the checker; the product library never links or calls it.
 *
 * Follows the definition in the reference's original backend
 * (models/modules/_MSM.py:10-30,53-59): for patch q of image i and every other
 * image j, the nearest distance min_r ||z[i,q]-z[j,r]||_2; the score is the mean
 * of ascending ranks [a, b) of those n-1 minima.  Distances are formed from
 * explicit differences in float64 (no expanded-norm cancellation), so the
 * result is the mathematical value to ~1e-15 and pins both the torch-fp32
 * restatement (oracle/msm.py) and the HIP kernels.
 *
 * NaN follows the reference's torch semantics: a NaN distance makes the minimum
 * over that reference image NaN (torch.min propagates it, _MSM.py:17), and NaN
 * minima sort after every number (torch.topk(largest=False), _MSM.py:27), so a
 * NaN inside the rank window makes the mean NaN.
 *
 * Build: see oracle/build.py (gcc -O3 -fopenmp -shared -fPIC).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* One row's minima: out[j] = min_r ||z[row]-z[j,r]||, +inf for the row's own image. */
static void nearest_row(const float* z, int n, int p, int c, long row, double* out) {
  const int i = (int)(row / p);
  const float* a = z + row * c;
  for (int j = 0; j < n; ++j) {
    double best = INFINITY;
    if (j != i) {
      for (int r = 0; r < p && !isnan(best); ++r) {
        const float* b = z + ((long)j * p + r) * c;
        double s = 0.0;
        for (int k = 0; k < c; ++k) {
          const double d = (double)a[k] - (double)b[k];
          s += d * d;
        }
        if (isnan(s) || s < best) best = s;
      }
      best = sqrt(best);
    }
    out[j] = best;
  }
}

/* nearest[(i*p+q)*n + j] = min_r ||z[i,q]-z[j,r]||, +inf for j == i. */
int msm_nearest_f64(const float* z, int n, int p, int c, double* nearest) {
  if (!z || !nearest || n < 1 || p < 1 || c < 1) return 1;
  const long rows = (long)n * p;
#pragma omp parallel for schedule(dynamic, 4)
  for (long row = 0; row < rows; ++row) nearest_row(z, n, p, c, row, nearest + row * n);
  return 0;
}

/* The same for selected global rows only: out[k*n + j] is the minimum of row rows[k]
 * (a row index i*p + q) against image j. */
int msm_nearest_rows_f64(const float* z, int n, int p, int c, const long long* rows, int nrows, double* out) {
  if (!z || !rows || !out || n < 1 || p < 1 || c < 1 || nrows < 0) return 1;
  for (int k = 0; k < nrows; ++k)
    if (rows[k] < 0 || rows[k] >= (long long)n * p) return 1;
#pragma omp parallel for schedule(dynamic, 1)
  for (int k = 0; k < nrows; ++k) nearest_row(z, n, p, c, (long)rows[k], out + (long)k * n);
  return 0;
}

/* Ascending, NaN after every number. */
static int cmp_double(const void* x, const void* y) {
  const double a = *(const double*)x, b = *(const double*)y;
  if (isnan(a)) return isnan(b) ? 0 : 1;
  if (isnan(b)) return -1;
  return (a > b) - (a < b);
}

/* scores[i*p+q] = mean of sorted(nearest row without own image)[a:b]. */
int msm_scores_from_nearest_f64(const double* nearest, int n, int p, int a, int b, double* scores) {
  if (!nearest || !scores || n < 2 || a < 0 || a >= b || b > n - 1) return 1;
  const long rows = (long)n * p;
  int failed = 0;
#pragma omp parallel
  {
    double* buf = (double*)malloc(sizeof(double) * (size_t)n);
    if (!buf) {
#pragma omp atomic write
      failed = 1;
    } else {
#pragma omp for
      for (long row = 0; row < rows; ++row) {
        const int own = (int)(row / p);
        int m = 0;
        for (int j = 0; j < n; ++j)
          if (j != own) buf[m++] = nearest[row * n + j];
        qsort(buf, (size_t)m, sizeof(double), cmp_double);
        double s = 0.0;
        for (int k = a; k < b; ++k) s += buf[k];
        scores[row] = s / (double)(b - a);
      }
      free(buf);
    }
  }
  return failed;
}

int msm_scores_f64(const float* z, int n, int p, int c, int a, int b, double* scores) {
  double* nearest = (double*)malloc(sizeof(double) * (size_t)n * p * n);
  if (!nearest) return 2;
  int rc = msm_nearest_f64(z, n, p, c, nearest);
  if (!rc) rc = msm_scores_from_nearest_f64(nearest, n, p, a, b, scores);
  free(nearest);
  return rc;
}
