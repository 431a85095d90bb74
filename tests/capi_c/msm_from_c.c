/* Calls libmusc_hip from plain C (no torch): HIP runtime API for the buffers, musc_msm_*
 * for the scores, a float64 brute force of models/modules/_MSM.py:10-30 (per-image minimum
 * distances, ranks [a, b) averaged) for the check.  Also: the four MSM stages called one
 * by one (prepare, pair_minima, refine, rank) and the no-allocation entry point give the
 * one-shot call's scores bit for bit; the split engine rejects P < 256 with
 * MUSC_ERR_UNSUPPORTED; the epilogue at out_size = side returns the layer/radius mean of
 * the score grid and its maximum (models/musc.py:259-288; align_corners keeps the grid).
 * Prints "max_abs_err <value>" and exits 0 when every check holds. */
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

  /* the four stages one by one, and the entry point that allocates nothing */
  void* dscores2;
  CHECK(hipMalloc(&dscores2, sizeof(double) * N * P));
  CHECK(musc_msm_prepare_f32((const float*)dz, N, P, C, 0, dws, ws_bytes, 0));
  CHECK(musc_msm_pair_minima_f32((const float*)dz, N, P, C, dws, ws_bytes, 0));
  CHECK(musc_msm_refine_f32((const float*)dz, N, P, C, dws, ws_bytes, 0));
  CHECK(musc_msm_rank_f32(N, P, A, B, (double*)dscores2, dws, ws_bytes, 0));
  CHECK(hipDeviceSynchronize());
  static double staged[N * P], noalloc[N * P];
  CHECK(hipMemcpy(staged, dscores2, sizeof(staged), hipMemcpyDeviceToHost));
  CHECK(musc_msm_scores_f32_noalloc((const float*)dz, N, P, C, A, B, (double*)dscores2, 0));
  CHECK(hipDeviceSynchronize());
  CHECK(hipMemcpy(noalloc, dscores2, sizeof(noalloc), hipMemcpyDeviceToHost));
  for (int k = 0; k < N * P; ++k)
    if (staged[k] != got[k] || noalloc[k] != got[k]) {
      fprintf(stderr, "stage-by-stage or no-allocation scores differ at %d: %.17g %.17g %.17g\n", k, got[k],
              staged[k], noalloc[k]);
      return 3;
    }
  size_t split_bytes = 0;
  CHECK(musc_msm_split_workspace_bytes(N, P, C, &split_bytes));
  void* dsplit;
  CHECK(hipMalloc(&dsplit, split_bytes));
  if (musc_msm_split_scores_f32((const float*)dz, N, P, C, A, B, 0, (double*)dscores2, dsplit, split_bytes, 0) !=
      MUSC_ERR_UNSUPPORTED) {
    fprintf(stderr, "split engine accepted P = %d < 256\n", P);
    return 4;
  }
  /* epilogue: two radii x one layer of 6 x 6 score grids for every image, out_size = side */
  enum { S = 6, R = 2 };
  static double grid[R * N * S * S], maps[N * S * S], img[N];
  for (int k = 0; k < R * N * S * S; ++k) grid[k] = 0.5 + 0.25 * frand(&seed);
  void *dgrid, *dmaps, *dimg;
  CHECK(hipMalloc(&dgrid, sizeof(grid)));
  CHECK(hipMalloc(&dmaps, sizeof(maps)));
  CHECK(hipMalloc(&dimg, sizeof(img)));
  CHECK(hipMemcpy(dgrid, grid, sizeof(grid), hipMemcpyHostToDevice));
  CHECK(musc_maps_f64((const double*)dgrid, R, 1, N, S, S, (double*)dmaps, (double*)dimg, 0));
  CHECK(hipDeviceSynchronize());
  CHECK(hipMemcpy(maps, dmaps, sizeof(maps), hipMemcpyDeviceToHost));
  CHECK(hipMemcpy(img, dimg, sizeof(img), hipMemcpyDeviceToHost));
  for (int i = 0; i < N; ++i) {
    double mx = -INFINITY;
    for (int k = 0; k < S * S; ++k) {
      const double want = (grid[(0 * N + i) * S * S + k] + grid[(1 * N + i) * S * S + k]) / 2.0;
      if (fabs(maps[i * S * S + k] - want) > 1e-15) {
        fprintf(stderr, "epilogue map %d/%d: %.17g against %.17g\n", i, k, maps[i * S * S + k], want);
        return 5;
      }
      if (want > mx) mx = want;
    }
    if (fabs(img[i] - mx) > 1e-15) {
      fprintf(stderr, "epilogue image score %d: %.17g against %.17g\n", i, img[i], mx);
      return 5;
    }
  }
  hipFree(dscores2);
  hipFree(dsplit);
  hipFree(dgrid);
  hipFree(dmaps);
  hipFree(dimg);

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
