/*
 * C restatement of the reference's hot-path arithmetic -- TEST
 * INFRASTRUCTURE ONLY (see oracle/__init__.py).  Plain loops, float64
 * accumulation (int64 for integer scans), no vectorisation tricks, so that
 * this file and the NumPy closed forms in oracle/*.py pin each other.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* cases/rbf/delivery/rbf_test.cu:24-35 and cases/rbf/reference.py:14-20:
 * K[i,j] = exp(-gamma * sum_d (X[i,d]-Y[j,d])^2), accumulated in double. */
void oracle_rbf_forward(const float* X, const float* Y, double* K, int64_t N,
                        int64_t M, int64_t D, double gamma) {
  for (int64_t i = 0; i < N; ++i)
    for (int64_t j = 0; j < M; ++j) {
      double s = 0.0;
      for (int64_t d = 0; d < D; ++d) {
        double t = (double)X[i * D + d] - (double)Y[j * D + d];
        s += t * t;
      }
      K[i * M + j] = exp(-gamma * s);
    }
}

/* cases/rbf/delivery/rbf_test.cu:37-52: coef = -2 gamma G K,
 * dX[i] += coef (x_i - y_j), dY[j] += coef (y_j - x_i). */
void oracle_rbf_backward(const float* X, const float* Y, const float* G,
                         const double* K, double* dX, double* dY, int64_t N,
                         int64_t M, int64_t D, double gamma) {
  memset(dX, 0, sizeof(double) * (size_t)(N * D));
  memset(dY, 0, sizeof(double) * (size_t)(M * D));
  for (int64_t i = 0; i < N; ++i)
    for (int64_t j = 0; j < M; ++j) {
      double coef = -2.0 * gamma * (double)G[i * M + j] * K[i * M + j];
      for (int64_t d = 0; d < D; ++d) {
        double diff = (double)X[i * D + d] - (double)Y[j * D + d];
        dX[i * D + d] += coef * diff;
        dY[j * D + d] -= coef * diff;
      }
    }
}

/* cases/scan/reference.py:8-9 (torch.cumsum along the last dim) for int32
 * input: exact int64 prefix sums (torch returns int64 for int32 input). */
void oracle_scan_i32(const int32_t* x, int64_t* y, int64_t rows, int64_t cols,
                     int reverse) {
  for (int64_t r = 0; r < rows; ++r) {
    int64_t acc = 0;
    for (int64_t c = 0; c < cols; ++c) {
      int64_t k = reverse ? cols - 1 - c : c;
      acc += x[r * cols + k];
      y[r * cols + k] = acc;
    }
  }
}

/* fp32 cumsum with a double accumulator, rounded once per output
 * (the torch CPU kernel's accumulation type for float is double). */
void oracle_scan_f32(const float* x, float* y, int64_t rows, int64_t cols,
                     int reverse) {
  for (int64_t r = 0; r < rows; ++r) {
    double acc = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      int64_t k = reverse ? cols - 1 - c : c;
      acc += (double)x[r * cols + k];
      y[r * cols + k] = (float)acc;
    }
  }
}

/* cases/spmv/reference.py:8-23 / description.md:5-7:
 * Y[m,:] = sum_{p in row m} vals[p] * X[col[p],:], double accumulation. */
void oracle_spmm_csr(const int64_t* row_ptr, const int64_t* col,
                     const float* vals, const float* X, double* Y, int64_t M,
                     int64_t D) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t d = 0; d < D; ++d) Y[m * D + d] = 0.0;
    for (int64_t p = row_ptr[m]; p < row_ptr[m + 1]; ++p)
      for (int64_t d = 0; d < D; ++d)
        Y[m * D + d] += (double)vals[p] * (double)X[col[p] * D + d];
  }
}

/* Backward of the product: dX[col[p],:] += vals[p] * dY[m,:] (A^T dY) and
 * dvals[p] = <dY[m,:], X[col[p],:]>. */
void oracle_spmm_csr_backward(const int64_t* row_ptr, const int64_t* col,
                              const float* vals, const float* X,
                              const float* dY, double* dX, double* dvals,
                              int64_t M, int64_t K, int64_t D) {
  for (int64_t k = 0; k < K * D; ++k) dX[k] = 0.0;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t p = row_ptr[m]; p < row_ptr[m + 1]; ++p) {
      double s = 0.0;
      for (int64_t d = 0; d < D; ++d) {
        dX[col[p] * D + d] += (double)vals[p] * (double)dY[m * D + d];
        s += (double)dY[m * D + d] * (double)X[col[p] * D + d];
      }
      dvals[p] = s;
    }
}

/* cases/layernorm/reference.py:14-21: two-pass mean and biased variance. */
void oracle_layernorm_forward(const float* x, const float* w, const float* b,
                              double* y, double* mean, double* rstd,
                              int64_t B, int64_t D, double eps) {
  for (int64_t r = 0; r < B; ++r) {
    double s = 0.0;
    for (int64_t d = 0; d < D; ++d) s += x[r * D + d];
    double mu = s / (double)D;
    double v = 0.0;
    for (int64_t d = 0; d < D; ++d) {
      double t = x[r * D + d] - mu;
      v += t * t;
    }
    v /= (double)D;
    double rs = 1.0 / sqrt(v + eps);
    mean[r] = mu;
    rstd[r] = rs;
    for (int64_t d = 0; d < D; ++d)
      y[r * D + d] = (x[r * D + d] - mu) * rs * w[d] + b[d];
  }
}
