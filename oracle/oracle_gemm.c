/*
 * Tile GEMM for the CPU oracle: c[rows, n] = a[rows, k] @ b[k, n], f32, row-major.
 * Test infrastructure only. It stands in for the `gemm` 0.19 crate call in the reference's exact-f32
 * attention branch (kernels.rs:184 and 219); that crate is a dependency absent from the reference tree,
 * so its published algorithm (a blocked f32 GEMM with FMA microkernels) is restated here: register-
 * blocked 4 x 32 tiles, products accumulated in k order with FMA. Built with FMA contraction on.
 */
#define MR 4
#define NR 32

void oracle_gemm_rows(const float* a, const float* b, float* c, int rows, int k, int n) {
  int i0 = 0;
  for (; i0 + MR <= rows; i0 += MR) {
    int j0 = 0;
    for (; j0 + NR <= n; j0 += NR) {
      float acc[MR][NR];
      for (int r = 0; r < MR; ++r)
        for (int jj = 0; jj < NR; ++jj) acc[r][jj] = 0.0f;
      for (int kk = 0; kk < k; ++kk) {
        const float* bp = b + (long)kk * n + j0;
        for (int r = 0; r < MR; ++r) {
          const float ar = a[(long)(i0 + r) * k + kk];
          for (int jj = 0; jj < NR; ++jj) acc[r][jj] += ar * bp[jj];
        }
      }
      for (int r = 0; r < MR; ++r)
        for (int jj = 0; jj < NR; ++jj) c[(long)(i0 + r) * n + j0 + jj] = acc[r][jj];
    }
    for (; j0 < n; ++j0) { /* column tail */
      for (int r = 0; r < MR; ++r) {
        float s = 0.0f;
        for (int kk = 0; kk < k; ++kk) s += a[(long)(i0 + r) * k + kk] * b[(long)kk * n + j0];
        c[(long)(i0 + r) * n + j0] = s;
      }
    }
  }
  for (; i0 < rows; ++i0) { /* row tail */
    for (int j = 0; j < n; ++j) c[(long)i0 * n + j] = 0.0f;
    for (int kk = 0; kk < k; ++kk) {
      const float ar = a[(long)i0 * k + kk];
      const float* bp = b + (long)kk * n;
      for (int j = 0; j < n; ++j) c[(long)i0 * n + j] += ar * bp[j];
    }
  }
}
