// RBF (Gaussian) kernel matrix, forward and backward, fp32, for MI355X
// (gfx950).  C-ABI declared in include/rbf.h.
//
// Reference semantics (cases/rbf/reference.py:14-20, delivery/README.md:8-12):
//   K[i,j] = exp(-gamma * sum_d (X[i,d] - Y[j,d])^2)
//   backward with upstream dK: W = dK o K,
//   dX[i] = -2 gamma * sum_j W[i,j] (X[i] - Y[j])
//   dY[j] = -2 gamma * sum_i W[i,j] (Y[j] - X[i])
//
// Design (D == 64 fast path):
//  * Forward: K[i,j] = exp(-gamma * max(|x_i|^2 + |y_j|^2 - 2 x_i.y_j, 0)).
//    The cross term runs on fp32 MFMA (v_mfma_f32_16x16x4_f32).  Each wave
//    owns a 64x64 tile of K and loads its 64 X rows and 64 Y rows straight
//    into MFMA operand registers (X and Y are L2 resident).  The contraction
//    index k is permuted consistently for both operands so that every lane
//    loads 16 contiguous bytes per load; the row norms fall out of the same
//    registers.  The exp epilogue runs from the accumulators and each lane
//    writes 4 consecutive K entries of one row with a 16-byte store.
//  * Backward: one pass over dK and K.  A workgroup (8 waves) owns a region of
//    RI x RJ entries of W and walks it in 64x64 tiles that are staged through
//    LDS (double buffered: W = dK o K, and the matching 64-row slices of X and
//    Y).  Waves 0-3 run the contraction W . Y (dX side), waves 4-7 run
//    W^T . X (dY side), both on fp32 MFMA.  The dX accumulators live for one
//    64-row chunk, the dY accumulators for the whole region, so each region
//    emits one partial dX slice (over its RJ columns) and one partial dY slice
//    (over its RI rows); a small kernel sums the slices.  The row and column
//    sums of W are taken from the same MFMA operand registers.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "../../../csrc/common.h"
#include "rbf.h"

using nl2k::f32x4;
using nl2k::load4;
using nl2k::store4;
using nl2k::zero4;
using nl2k::mfma16x4;

namespace {

constexpr int kD = 64;           // feature width of the MFMA path
constexpr int kTile = 64;        // backward tile edge
constexpr int kLds = 68;         // padded LDS row stride (floats)
constexpr int kTileFloats = kTile * kLds;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTargetRegions = 256;  // one backward workgroup per CU

// ------------------------------------------------------------------ forward
__global__ __launch_bounds__(256) void rbf_fwd_d64_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    float* __restrict__ K, int N, int M, float gl2e, int vec_store) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;
  const int h = lane >> 4;
  const int i0 = blockIdx.y * 128 + (wave >> 1) * 64;
  const int j0 = blockIdx.x * 128 + (wave & 1) * 64;
  if (i0 >= N || j0 >= M) return;  // wave-uniform; no barriers below

  // Operand registers.  Lane (n, h) holds, for row block b and quarter q,
  // elements k = 16q + 4h + u (u = 0..3) of row 16b + n.  Contraction step
  // s = 4q + u uses k = 16q + 4h + u in k-slot h of the MFMA.
  f32x4 ya[4][4], xb[4][4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int jr = j0 + b * 16 + n;
    const int ir = i0 + b * 16 + n;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ya[b][q] = jr < M ? load4(Y + (size_t)jr * kD + 16 * q + 4 * h) : zero4();
      xb[b][q] = ir < N ? load4(X + (size_t)ir * kD + 16 * q + 4 * h) : zero4();
    }
  }

  // Squared row norms: partial over this lane's 16 k, then over the 4 h.
  float ny[4], nx[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float sy = 0.f, sx = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        sy = fmaf(ya[b][q][u], ya[b][q][u], sy);
        sx = fmaf(xb[b][q][u], xb[b][q][u], sx);
      }
    }
    sy += __shfl_xor(sy, 16, 64);
    sy += __shfl_xor(sy, 32, 64);
    sx += __shfl_xor(sx, 16, 64);
    sx += __shfl_xor(sx, 32, 64);
    ny[b] = sy;  // |y|^2 of row j0 + 16b + n
    nx[b] = sx;  // |x|^2 of row i0 + 16b + n
  }

  // acc[jb][ib][r] = y_j . x_i with j = j0+16jb+4h+r, i = i0+16ib+n.
  f32x4 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
          acc[jb][ib] = mfma16x4(ya[jb][q][u], xb[ib][q][u], acc[jb][ib]);

  // Epilogue: lane (n, h) writes K[i][j .. j+3].
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    float nyr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) nyr[r] = __shfl(ny[jb], 4 * h + r, 64);
    const int j = j0 + jb * 16 + 4 * h;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      const int i = i0 + ib * 16 + n;
      if (i < N && j < M) {
        f32x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float d = fmaf(-2.f, acc[jb][ib][r], nx[ib] + nyr[r]);
          d = d < 0.f ? 0.f : d;  // rounding can push d below 0; NaN passes
          o[r] = exp2f(-gl2e * d);
        }
        float* dst = K + (size_t)i * M + j;
        if (vec_store && j + 3 < M) {
          store4(dst, o);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (j + r < M) dst[r] = o[r];
        }
      }
    }
  }
}

// ----------------------------------------------------------------- backward
template <int JC>
__global__ __launch_bounds__(512) void rbf_bwd_d64_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    const float* __restrict__ dK, const float* __restrict__ Kf,
    float* __restrict__ dXo, float* __restrict__ dYo, int N, int M, int RI,
    int nRJ, float neg2g, size_t dx_slot, size_t dy_slot, int vec_nm) {
  __shared__ float P[2][kTileFloats];   // W = dK o K tile, row-major [i][j]
  __shared__ float Ys[2][kTileFloats];  // Y rows of the tile's columns [j][d]
  __shared__ float Xs[2][kTileFloats];  // X rows of the tile's rows [i][d]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int h = lane >> 4;
  const bool dx_side = wave < 4;  // waves 0-3: W . Y ; waves 4-7: W^T . X
  const int wb = wave & 3;        // 16-row (dx side) or 16-column block

  const int ri = blockIdx.x / nRJ;
  const int rj = blockIdx.x - ri * nRJ;
  const int ibase = ri * RI;
  const int jbase = rj * (JC * kTile);
  const int rows = min(RI, N - ibase);
  const int cols = min(JC * kTile, M - jbase);
  const int n_ic = (rows + kTile - 1) / kTile;
  const int n_jc = (cols + kTile - 1) / kTile;
  float* __restrict__ dXs = dXo + (size_t)rj * dx_slot;
  float* __restrict__ dYs = dYo + (size_t)ri * dy_slot;

  // Staging: thread t moves float4 #(t + 512 s) of the 64x64 tile,
  // row (t >> 4) + 32 s, columns 4 (t & 15) .. +3.
  const int srow = tid >> 4;
  const int scol = (tid & 15) * 4;
  f32x4 g_w[2], g_y[2], g_x[2];

  auto load_tile = [&](int ic, int jc) {
    const int ib = ibase + ic * kTile;
    const int jb = jbase + jc * kTile;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int r = srow + 32 * s;
      const int gi = ib + r;
      const int gj = jb + scol;
      if (gi < N && vec_nm && gj + 3 < M) {
        const size_t o = (size_t)gi * M + gj;
        g_w[s] = load4(dK + o) * load4(Kf + o);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const size_t o = (size_t)gi * M + gj + u;
          g_w[s][u] = (gi < N && gj + u < M) ? dK[o] * Kf[o] : 0.f;
        }
      }
      g_y[s] = (jb + r < M) ? load4(Y + (size_t)(jb + r) * kD + scol) : zero4();
      g_x[s] = (gi < N) ? load4(X + (size_t)gi * kD + scol) : zero4();
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int r = srow + 32 * s;
      store4(&P[buf][r * kLds + scol], g_w[s]);
      store4(&Ys[buf][r * kLds + scol], g_y[s]);
      store4(&Xs[buf][r * kLds + scol], g_x[s]);
    }
  };

  f32x4 accX[4];      // dx side: (W.Y)^T block, rows 16wb+4h+r, d = 16db+n
  float rp = 0.f;     // dx side: partial row sums of W
  f32x4 accY[JC][4];  // dy side: (W^T.X) block per column chunk
  float cp[JC];       // dy side: partial column sums of W per chunk
#pragma unroll
  for (int c = 0; c < JC; ++c) {
    cp[c] = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) accY[c][db] = zero4();
  }

  load_tile(0, 0);
  commit(0);
  __syncthreads();
  int buf = 0;

  for (int ic = 0; ic < n_ic; ++ic) {
#pragma unroll
    for (int db = 0; db < 4; ++db) accX[db] = zero4();
    rp = 0.f;
#pragma unroll
    for (int jc = 0; jc < JC; ++jc) {
      if (jc < n_jc) {
        int nic = ic, njc = jc + 1;
        if (njc >= n_jc) {
          njc = 0;
          nic = ic + 1;
        }
        const bool has_next = nic < n_ic;
        if (has_next) load_tile(nic, njc);

        const float* Pb = P[buf];
        if (dx_side) {
          const float* Yb = Ys[buf];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 a = load4(&Pb[(wb * 16 + n) * kLds + 16 * q + 4 * h]);
            rp += (a[0] + a[1]) + (a[2] + a[3]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int k = 16 * q + 4 * h + u;
#pragma unroll
              for (int db = 0; db < 4; ++db)
                accX[db] = mfma16x4(a[u], Yb[k * kLds + db * 16 + n], accX[db]);
            }
          }
        } else {
          const float* Xb = Xs[buf];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int k = 16 * q + 4 * h + u;
              const float a = Pb[k * kLds + wb * 16 + n];
              cp[jc] += a;
#pragma unroll
              for (int db = 0; db < 4; ++db)
                accY[jc][db] =
                    mfma16x4(a, Xb[k * kLds + db * 16 + n], accY[jc][db]);
            }
          }
        }
        if (has_next) commit(buf ^ 1);
        __syncthreads();
        buf ^= 1;
      }
    }

    if (dx_side) {
      // Row sums: lane (m, h) holds columns 16q+4h+u of row 16wb+m.
      float rs = rp;
      rs += __shfl_xor(rs, 16, 64);
      rs += __shfl_xor(rs, 32, 64);
      float rsr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) rsr[r] = __shfl(rs, 4 * h + r, 64);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = ibase + ic * kTile + wb * 16 + 4 * h + r;
        if (i < N) {
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const size_t o = (size_t)i * kD + db * 16 + n;
            dXs[o] = neg2g * (rsr[r] * X[o] - accX[db][r]);
          }
        }
      }
    }
  }

  if (!dx_side) {
#pragma unroll
    for (int jc = 0; jc < JC; ++jc) {
      if (jc < n_jc) {
        float cs = cp[jc];
        cs += __shfl_xor(cs, 16, 64);
        cs += __shfl_xor(cs, 32, 64);
        float csr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) csr[r] = __shfl(cs, 4 * h + r, 64);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = jbase + jc * kTile + wb * 16 + 4 * h + r;
          if (j < M) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
              const size_t o = (size_t)j * kD + db * 16 + n;
              dYs[o] = neg2g * (csr[r] * Y[o] - accY[jc][db][r]);
            }
          }
        }
      }
    }
  }
}

// out[e] = sum over `slots` slices of part (slice stride slot_floats).
__global__ __launch_bounds__(256) void rbf_sum_slots_kernel(
    const float* __restrict__ part, float* __restrict__ out, size_t n4,
    size_t slot_floats, int slots) {
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n4;
       e += (size_t)gridDim.x * blockDim.x) {
    f32x4 a = load4(part + 4 * e);
    for (int s = 1; s < slots; ++s) a += load4(part + (size_t)s * slot_floats + 4 * e);
    store4(out + 4 * e, a);
  }
}

// ------------------------------------------------------- generic (any D)
__global__ __launch_bounds__(256) void rbf_fwd_generic_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    float* __restrict__ K, int64_t N, int64_t M, int64_t D, float gamma) {
  const int64_t total = N * M;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / M, j = e - i * M;
    const float* x = X + i * D;
    const float* y = Y + j * D;
    float s = 0.f;
    for (int64_t d = 0; d < D; ++d) {
      const float t = x[d] - y[d];
      s = fmaf(t, t, s);
    }
    K[e] = expf(-gamma * s);
  }
}

// One thread per (row, d) of the output; `a` is the output's own matrix
// (X for dX, Y for dY), `b` the other one.  trans selects dY (column walk).
__global__ __launch_bounds__(256) void rbf_bwd_generic_kernel(
    const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ dK, const float* __restrict__ Kf,
    float* __restrict__ out, int64_t rows, int64_t others, int64_t M,
    int64_t D, float neg2g, int trans) {
  const int64_t total = rows * D;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / D, d = e - r * D;
    const float av = a[e];
    float acc = 0.f;
    for (int64_t o = 0; o < others; ++o) {
      const int64_t idx = trans ? o * M + r : r * M + o;
      acc = fmaf(dK[idx] * Kf[idx], av - b[o * D + d], acc);
    }
    out[e] = neg2g * acc;
  }
}

__global__ __launch_bounds__(256) void rbf_fill_zero_kernel(float* __restrict__ p,
                                                           size_t count) {
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < count;
       e += (size_t)gridDim.x * blockDim.x)
    p[e] = 0.f;
}

// ------------------------------------------------------------------ planning
struct BwdPlan {
  bool fast = false;
  int R = 64;  // region edge (rows and columns)
  int JC = 1;  // R / 64
  int nRI = 0, nRJ = 0;
  size_t dx_ws = 0, dy_ws = 0;  // floats
};

BwdPlan plan_backward(int64_t N, int64_t M, int64_t D) {
  BwdPlan p;
  if (D != kD || N <= 0 || M <= 0) return p;
  p.fast = true;
  int R = 64;
  for (int cand = 512; cand >= 64; cand >>= 1) {
    if (nl2k::ceil_div(N, cand) * nl2k::ceil_div(M, cand) >= kTargetRegions) {
      R = cand;
      break;
    }
  }
  p.R = R;
  p.JC = R / kTile;
  p.nRI = (int)nl2k::ceil_div(N, R);
  p.nRJ = (int)nl2k::ceil_div(M, R);
  p.dx_ws = p.nRJ > 1 ? (size_t)p.nRJ * N * kD : 0;
  p.dy_ws = p.nRI > 1 ? (size_t)p.nRI * M * kD : 0;
  return p;
}

int validate_sizes(int64_t N, int64_t M, int64_t D) {
  if (N < 0 || M < 0 || D < 1)
    return nl2k::fail(NL2K_ERR_SHAPE,
                      "rbf: sizes must satisfy N >= 0, M >= 0, D >= 1 (got N=%lld M=%lld D=%lld)",
                      (long long)N, (long long)M, (long long)D);
  const int64_t lim = INT32_MAX;
  if (N > lim || M > lim || D > lim || (D > 0 && (N > INT64_MAX / D || M > INT64_MAX / D)) ||
      (M > 0 && N > INT64_MAX / M))
    return nl2k::fail(NL2K_ERR_OVERFLOW, "rbf: sizes too large (N=%lld M=%lld D=%lld)",
                      (long long)N, (long long)M, (long long)D);
  return NL2K_SUCCESS;
}

int launch_fill_zero(float* p, size_t count, hipStream_t stream) {
  if (count == 0) return NL2K_SUCCESS;
  const int blocks = (int)std::min<size_t>((count + 255) / 256, 4096);
  hipLaunchKernelGGL(rbf_fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, p, count);
  return nl2k::check_launch("rbf fill");
}

template <int JC>
void launch_bwd_fast(const BwdPlan& p, const float* X, const float* Y,
                     const float* dK, const float* K, float* dXo, float* dYo,
                     int N, int M, float neg2g, size_t dx_slot, size_t dy_slot,
                     int vec_nm, hipStream_t stream) {
  hipLaunchKernelGGL(rbf_bwd_d64_kernel<JC>, dim3(p.nRI * p.nRJ), dim3(512), 0,
                     stream, X, Y, dK, K, dXo, dYo, N, M, p.R, p.nRJ, neg2g,
                     dx_slot, dy_slot, vec_nm);
}

}  // namespace

extern "C" {

const char* rbf_last_error(void) { return nl2k::error_slot().text; }

int rbf_forward_f32(const float* X, const float* Y, float* K, int64_t N,
                    int64_t M, int64_t D, float gamma, hipStream_t stream) {
  int st = validate_sizes(N, M, D);
  if (st) return st;
  if (N == 0 || M == 0) return nl2k::succeed();
  if (!X || !Y || !K)
    return nl2k::fail(NL2K_ERR_NULL, "rbf_forward_f32: X, Y and K must be non-null");

  if (D == kD && nl2k::aligned16(X) && nl2k::aligned16(Y)) {
    const int vec_store = (M % 4 == 0) && nl2k::aligned16(K);
    dim3 grid((unsigned)nl2k::ceil_div(M, 128), (unsigned)nl2k::ceil_div(N, 128));
    hipLaunchKernelGGL(rbf_fwd_d64_kernel, grid, dim3(256), 0, stream, X, Y, K,
                       (int)N, (int)M, gamma * kLog2e, vec_store);
    return nl2k::check_launch("rbf_forward_f32");
  }
  const int64_t total = N * M;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 1 << 16);
  hipLaunchKernelGGL(rbf_fwd_generic_kernel, dim3(blocks), dim3(256), 0, stream,
                     X, Y, K, N, M, D, gamma);
  return nl2k::check_launch("rbf_forward_f32 (generic)");
}

size_t rbf_backward_workspace_bytes(int64_t N, int64_t M, int64_t D) {
  if (validate_sizes(N, M, D)) return 0;
  const BwdPlan p = plan_backward(N, M, D);
  return (p.dx_ws + p.dy_ws) * sizeof(float);
}

int rbf_backward_f32(const float* X, const float* Y, const float* dK,
                     const float* K, float* dX, float* dY, int64_t N,
                     int64_t M, int64_t D, float gamma, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  int st = validate_sizes(N, M, D);
  if (st) return st;
  if (N == 0 && M == 0) return nl2k::succeed();
  if ((N > 0 && (!X || !dX)) || (M > 0 && (!Y || !dY)))
    return nl2k::fail(NL2K_ERR_NULL, "rbf_backward_f32: X, Y, dX, dY must be non-null");
  // Empty sums: dX = 0 when M == 0, dY = 0 when N == 0.
  if (M == 0) return launch_fill_zero(dX, (size_t)(N * D), stream);
  if (N == 0) return launch_fill_zero(dY, (size_t)(M * D), stream);
  if (!dK || !K)
    return nl2k::fail(NL2K_ERR_NULL, "rbf_backward_f32: dK and K must be non-null");

  const float neg2g = -2.f * gamma;
  const BwdPlan p = plan_backward(N, M, D);
  const bool aligned = nl2k::aligned16(X) && nl2k::aligned16(Y) &&
                       nl2k::aligned16(dX) && nl2k::aligned16(dY);
  if (p.fast && aligned) {
    const size_t need = (p.dx_ws + p.dy_ws) * sizeof(float);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      return nl2k::fail(NL2K_ERR_WORKSPACE,
                        "rbf_backward_f32: workspace of %zu bytes required, got %zu",
                        need, workspace ? workspace_bytes : (size_t)0);
    if (need > 0 && !nl2k::aligned16(workspace))
      return nl2k::fail(NL2K_ERR_ALIGN, "rbf_backward_f32: workspace must be 16-byte aligned");
    float* ws = static_cast<float*>(workspace);
    float* dXo = p.dx_ws ? ws : dX;
    float* dYo = p.dy_ws ? ws + p.dx_ws : dY;
    const size_t dx_slot = p.dx_ws ? (size_t)N * kD : 0;
    const size_t dy_slot = p.dy_ws ? (size_t)M * kD : 0;
    const int vec_nm = (M % 4 == 0) && nl2k::aligned16(dK) && nl2k::aligned16(K);
    switch (p.JC) {
      case 1: launch_bwd_fast<1>(p, X, Y, dK, K, dXo, dYo, (int)N, (int)M, neg2g, dx_slot, dy_slot, vec_nm, stream); break;
      case 2: launch_bwd_fast<2>(p, X, Y, dK, K, dXo, dYo, (int)N, (int)M, neg2g, dx_slot, dy_slot, vec_nm, stream); break;
      case 4: launch_bwd_fast<4>(p, X, Y, dK, K, dXo, dYo, (int)N, (int)M, neg2g, dx_slot, dy_slot, vec_nm, stream); break;
      default: launch_bwd_fast<8>(p, X, Y, dK, K, dXo, dYo, (int)N, (int)M, neg2g, dx_slot, dy_slot, vec_nm, stream); break;
    }
    st = nl2k::check_launch("rbf_backward_f32");
    if (st) return st;
    if (p.dx_ws) {
      const size_t n4 = (size_t)N * kD / 4;
      const int blocks = (int)std::min<size_t>((n4 + 255) / 256, 2048);
      hipLaunchKernelGGL(rbf_sum_slots_kernel, dim3(blocks), dim3(256), 0, stream,
                         dXo, dX, n4, dx_slot, p.nRJ);
      st = nl2k::check_launch("rbf_backward_f32 (dX reduce)");
      if (st) return st;
    }
    if (p.dy_ws) {
      const size_t n4 = (size_t)M * kD / 4;
      const int blocks = (int)std::min<size_t>((n4 + 255) / 256, 2048);
      hipLaunchKernelGGL(rbf_sum_slots_kernel, dim3(blocks), dim3(256), 0, stream,
                         dYo, dY, n4, dy_slot, p.nRI);
      st = nl2k::check_launch("rbf_backward_f32 (dY reduce)");
      if (st) return st;
    }
    return nl2k::succeed();
  }

  const int bx = (int)std::min<int64_t>((N * D + 255) / 256, 1 << 16);
  hipLaunchKernelGGL(rbf_bwd_generic_kernel, dim3(bx), dim3(256), 0, stream, X, Y,
                     dK, K, dX, N, M, M, D, neg2g, 0);
  st = nl2k::check_launch("rbf_backward_f32 (generic dX)");
  if (st) return st;
  const int by = (int)std::min<int64_t>((M * D + 255) / 256, 1 << 16);
  hipLaunchKernelGGL(rbf_bwd_generic_kernel, dim3(by), dim3(256), 0, stream, Y, X,
                     dK, K, dY, M, N, M, D, neg2g, 1);
  return nl2k::check_launch("rbf_backward_f32 (generic dY)");
}

}  // extern "C"
