/* Calls libmusc_hip's MSM entry point from plain C (no torch): HIP runtime API for the
 * buffers, musc_msm_* for the scores, a float64 brute force of models/modules/_MSM.py:10-30
 * (per-image minimum distances, ranks [a, b) averaged) for the check.
 * Prints "max_abs_err <value>" and exits 0 when it is below 2e-5. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <hip/hip_runtime_api.h>

#include "musc_hip.h"

enum { N = 5, P = 37, C = 24, A = 0, B = 2 };

static double frand(unsigned long long* s) {
  *s = *s * 6364136223846793005ULL + 1442695040888963407ULL;
  return ((double)(*s >> 11) / 9007199254740992.0) * 2.0 - 1.0;
}

static int cmp(const void* x, const void* y) {
  const double a = *(const double*)x, b = *(const double*)y;
  return (a > b) - (a < b);
}

#define CHECK(call)                                                        \
  do {                                                                     \
    int rc_ = (int)(call);                                                 \
    if (rc_) {                                                             \
      fprintf(stderr, "%s failed: %d (%s)\n", #call, rc_, musc_strerror(rc_)); \
      return 2;                                                            \
    }                                                                      \
  } while (0)

int main(void) {
  static float z[N * P * C];
  unsigned long long seed = 42;
  for (int r = 0; r < N * P; ++r) {
    double norm = 0.0;
    for (int c = 0; c < C; ++c) {
      z[r * C + c] = (float)frand(&seed);
      norm += (double)z[r * C + c] * z[r * C + c];
    }
    for (int c = 0; c < C; ++c) z[r * C + c] = (float)(z[r * C + c] / sqrt(norm));
  }
  size_t ws_bytes = 0;
  CHECK(musc_msm_workspace_bytes(N, P, C, &ws_bytes));
  void *dz, *dscores, *dws;
  CHECK(hipMalloc(&dz, sizeof(z)));
  CHECK(hipMalloc(&dscores, sizeof(double) * N * P));
  CHECK(hipMalloc(&dws, ws_bytes));
  CHECK(hipMemcpy(dz, z, sizeof(z), hipMemcpyHostToDevice));
  CHECK(musc_msm_scores_f32((const float*)dz, N, P, C, A, B, (double*)dscores, dws, ws_bytes, 0));
  CHECK(hipDeviceSynchronize());
  static double got[N * P];
  CHECK(hipMemcpy(got, dscores, sizeof(got), hipMemcpyDeviceToHost));

  double worst = 0.0;
  for (int i = 0; i < N; ++i)
    for (int p = 0; p < P; ++p) {
      double mins[N - 1];
      int m = 0;
      for (int j = 0; j < N; ++j) {
        if (j == i) continue;
        double best = INFINITY;
        for (int q = 0; q < P; ++q) {
          double d2 = 0.0;
          for (int c = 0; c < C; ++c) {
            const double t = (double)z[(i * P + p) * C + c] - (double)z[(j * P + q) * C + c];
            d2 += t * t;
          }
          if (d2 < best) best = d2;
        }
        mins[m++] = sqrt(best);
      }
      qsort(mins, N - 1, sizeof(double), cmp);
      double mean = 0.0;
      for (int k = A; k < B; ++k) mean += mins[k];
      mean /= (B - A);
      const double err = fabs(mean - got[i * P + p]);
      if (err > worst) worst = err;
    }
  printf("max_abs_err %.3e\n", worst);
  hipFree(dz);
  hipFree(dscores);
  hipFree(dws);
  return worst < 2e-5 ? 0 : 1;
}
