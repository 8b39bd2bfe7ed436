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
//  * Forward: K[i,j] = exp2(min(2 kappa x_i.y_j - kappa (|x_i|^2 + |y_j|^2), 0))
//    with kappa = gamma log2(e).  The cross term runs on fp32 MFMA
//    (v_mfma_f32_16x16x4_f32).  Work unit = 256 rows x 64 columns of K; a
//    workgroup of four waves walks a contiguous range of units.  Each wave
//    keeps its 64 X rows in MFMA operand registers (with their norms) for as
//    long as the row block lasts, and the unit's 64 Y rows are staged once
//    per workgroup in LDS (double buffered, norms alongside) while the
//    previous unit runs on the matrix cores.  The contraction index is
//    permuted identically for both operands so every lane moves 16
//    contiguous bytes per load.  The exp epilogue runs from the accumulators
//    and each lane writes 4 consecutive K entries of a row (16-byte stores).
//  * Backward: one pass over dK and K.  A workgroup (8 waves) owns a region
//    of R x R entries of W = dK o K (R = 256 at N = M = 4096, one region per
//    CU) and walks it in 64x64 tiles.  Waves 4-7 only stage: they load dK and
//    K three tiles ahead into registers, form W into the LDS tile buffer of
//    the next tile, and stage the next 64-row X chunk (transposed).  Waves
//    0-3 only compute: per tile both contractions W . Y (rows, accumulated
//    over the region's columns and flushed per 64-row chunk) and W^T . X
//    (columns, accumulated over the whole region) on fp32 MFMA, with the row
//    and column sums of W taken from the same operand registers.  Each region
//    writes raw partial contractions and partial sums to its workspace slot;
//    rbf_bwd_reduce_kernel sums the slots and applies
//    dX = -2 gamma (rowsum(W) X - W Y), dY = -2 gamma (colsum(W) Y - W^T X).
//  * Other feature widths and misaligned pointers use the generic kernels
//    (direct sums over d, one thread per output entry / row).
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
constexpr int kFwdWorkgroups = 512;  // two forward workgroups per CU

// ------------------------------------------------------------------ forward
// Work unit = (row block of 256 rows, column tile of 64).  A workgroup of four
// waves walks a contiguous range of units; wave w owns rows 64w..64w+63 of
// the block and keeps them in MFMA operand registers, while the 64 Y rows of
// the current column tile are staged once per workgroup in LDS (double
// buffered, with their squared norms).  The next tile's Y rows are fetched
// from global memory while the current tile runs on the matrix cores.
constexpr int kFwdRows = 256;  // rows per unit (4 waves x 64)

__global__ __launch_bounds__(256, 2) void rbf_fwd_d64_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    float* __restrict__ K, int N, int M, float neg_kappa, int n_jt,
    int n_units, int units_per_wg, int vec_store) {
  __shared__ float Ys[2][kTileFloats];
  __shared__ __attribute__((aligned(16))) float nyS[2][kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int h = lane >> 4;
  const int u_begin = blockIdx.x * units_per_wg;
  const int u_end = min(u_begin + units_per_wg, n_units);
  if (u_begin >= u_end) return;  // workgroup-uniform

  // Y staging: thread t moves float4 (row (t >> 4) + 16 s, cols 4 (t & 15)..).
  const int srow = tid >> 4;
  const int scol = (tid & 15) * 4;
  f32x4 gy[4];
  auto load_y = [&](int u) {
    const int j0 = (u % n_jt) * kTile;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      gy[s] = load4(Y + (size_t)min(j0 + srow + 16 * s, M - 1) * kD + scol);
  };
  auto commit_y = [&](int buf) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int r = srow + 16 * s;
      store4(&Ys[buf][r * kLds + scol], gy[s]);
      float p = gy[s][0] * gy[s][0] + gy[s][1] * gy[s][1] + gy[s][2] * gy[s][2] +
                gy[s][3] * gy[s][3];
      p += __shfl_xor(p, 1, 64);
      p += __shfl_xor(p, 2, 64);
      p += __shfl_xor(p, 4, 64);
      p += __shfl_xor(p, 8, 64);
      if ((tid & 15) == 0) nyS[buf][r] = p;
    }
  };

  // X operand registers: lane (n, h) holds elements k = 16q + 4h + u of row
  // 16 ib + n of this wave's strip.  Contraction step (q, u) uses k-slot h.
  f32x4 xb[4][4];
  float ax[4];  // -gamma*log2(e) * |x|^2 of row 16 ib + n
  int cur_rb = -1;
  auto load_x = [&](int rb) {
    const int i0 = rb * kFwdRows + wave * 64;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      const int ir = min(i0 + ib * 16 + n, N - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) xb[ib][q] = load4(X + (size_t)ir * kD + 16 * q + 4 * h);
    }
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      float sx = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) sx = fmaf(xb[ib][q][u], xb[ib][q][u], sx);
      sx += __shfl_xor(sx, 16, 64);
      sx += __shfl_xor(sx, 32, 64);
      ax[ib] = neg_kappa * sx;
    }
    cur_rb = rb;
  };

  load_x(u_begin / n_jt);
  load_y(u_begin);
  commit_y(0);
  __syncthreads();
  int buf = 0;

  for (int u = u_begin; u < u_end; ++u) {
    const bool has_next = u + 1 < u_end;
    if (has_next) load_y(u + 1);
    __builtin_amdgcn_sched_barrier(0);

    const float* Yb = Ys[buf];
    f32x4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = zero4();
    // A operands (Y rows 16 jb + n, k = 16q + 4h .. +3), read one q ahead.
    f32x4 ya[2][4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) ya[0][jb] = load4(&Yb[(jb * 16 + n) * kLds + 4 * h]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < 3) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
          ya[(q + 1) & 1][jb] = load4(&Yb[(jb * 16 + n) * kLds + 16 * (q + 1) + 4 * h]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int uu = 0; uu < 4; ++uu)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int ib = 0; ib < 4; ++ib)
            acc[jb][ib] = mfma16x4(ya[q & 1][jb][uu], xb[ib][q][uu], acc[jb][ib]);
      __builtin_amdgcn_sched_barrier(0);
    }

    // Epilogue: K[i][j..j+3] = exp2(min(2 kappa c - kappa (|x|^2 + |y|^2), 0)),
    // i = i0 + 16 ib + n, j = j0 + 16 jb + 4h.
    const int i0 = (u / n_jt) * kFwdRows + wave * 64;
    const int j0 = (u % n_jt) * kTile;
    const bool full = vec_store && i0 + 64 <= N && j0 + 64 <= M;
    const float two_kappa = -2.f * neg_kappa;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const f32x4 ny = load4(&nyS[buf][jb * 16 + 4 * h]);
      const int j = j0 + jb * 16 + 4 * h;
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const int i = i0 + ib * 16 + n;
        f32x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float t = fmaf(two_kappa, acc[jb][ib][r], fmaf(neg_kappa, ny[r], ax[ib]));
          t = t > 0.f ? 0.f : t;  // squared distance >= 0; NaN passes through
          o[r] = __builtin_amdgcn_exp2f(t);
        }
        float* dst = K + (size_t)i * M + j;
        if (full) {
          store4(dst, o);
        } else if (i < N && j < M) {
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

    if (has_next) commit_y(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    if (has_next && (u + 1) / n_jt != cur_rb) load_x((u + 1) / n_jt);
  }
}

// ----------------------------------------------------------------- backward
// Region = RI x RJ entries of W (RJ = 64 JC), walked in 64x64 tiles, i-chunk
// outer, j-chunk inner.  The workgroup's eight waves split into two roles so
// that global-load issue stalls never hold up the matrix cores:
//  * waves 0-3 (compute) each own 16 rows and 16 columns of every tile and
//    run both contractions on fp32 MFMA:
//      (W.Y)^T   rows 16w..: A = P[i][j..j+3], B = Yt[d][j..j+3]
//      (W^T.X)^T cols 16w..: A = P[i..i+3][j] (four 4-byte reads),
//                            B = Xt[d][i..i+3]
//    accumulating the first over the region's columns (flushed per i-chunk)
//    and the second over the region's rows (flushed at the end);
//  * waves 4-7 (staging) load dK and K up to three tiles ahead into
//    registers, form W = dK o K into the LDS tile buffer of the next tile,
//    and stage the next i-chunk's X rows.
// LDS: Yt = the region's Y rows, transposed [d][j], staged once; Xt = X rows
// of an i-chunk, transposed [d][i], double buffered; P = W tile [i][j],
// double buffered.  Both roles run the same loop nest and pass exactly one
// workgroup barrier per tile.  Each region writes raw partial contractions
// and partial row / column sums of W to its workspace slot;
// rbf_bwd_reduce_kernel sums the slots and applies
// dX = -2 gamma (rowsum(W) X - W Y), dY = -2 gamma (colsum(W) Y - W^T X).
template <int JC, bool kVecNM>
__global__ __launch_bounds__(512) void rbf_bwd_d64_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    const float* dK, const float* Kf,
    float* __restrict__ Px, float* __restrict__ Rx, float* __restrict__ Py,
    float* __restrict__ Ry, int N, int M, int RI, int nRJ) {
  // dK and Kf are deliberately not __restrict__: with it the compiler treats
  // their loads as invariant and sinks the prefetch of tile t+2 past the
  // workgroup barriers to its use, which serialises the memory latency.
  constexpr int RJ = JC * kTile;
  constexpr int kYtLds = RJ + 4;
  __shared__ __attribute__((aligned(16))) float P[2][kTileFloats];
  __shared__ __attribute__((aligned(16))) float Xt[2][kTileFloats];
  __shared__ __attribute__((aligned(16))) float Yt[kD * kYtLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int h = lane >> 4;

  const int ri = blockIdx.x / nRJ;
  const int rj = blockIdx.x - ri * nRJ;
  const int ibase = ri * RI;
  const int jbase = rj * RJ;
  const int rows = min(RI, N - ibase);
  const int cols = min(RJ, M - jbase);
  const int n_ic = (rows + kTile - 1) / kTile;
  const int n_jc = (cols + kTile - 1) / kTile;
  const int n_tiles = n_ic * n_jc;

  // Staging-wave state (declared for all waves; only waves 4-7 use it).
  const int ptid = tid - 256;
  // W: float4 (row (p>>4) + 16 s, cols 4 (p & 15)..), s = 0..3.
  const int srow = (ptid >> 4) & 15;
  const int scol = (ptid & 15) * 4;
  // X chunk: row p & 63 (lanes along rows), float4 columns (p>>6) + 4 s.
  const int xrow = ptid & 63;
  const int xcol = ((ptid >> 6) & 3) * 4;
  f32x4 g_dk[3][4], g_k[3][4], g_x[3][4];
  bool g_ok[3][4];
  auto load_stage = [&](int t, f32x4 (&dk)[4], f32x4 (&kk)[4], bool (&ok)[4]) {
    const int ic = t / n_jc, jc = t - ic * n_jc;
    const int ib = ibase + ic * kTile;
    const int jb = jbase + jc * kTile;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int gi = ib + srow + 16 * s;
      const int gj = jb + scol;
      const int ci = min(gi, N - 1);
      if (kVecNM) {
        ok[s] = gi < N && gj < M;
        const size_t o = (size_t)ci * M + min(gj, M - 4);
        dk[s] = load4(dK + o);
        kk[s] = load4(Kf + o);
      } else {
        ok[s] = gi < N;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const size_t o = (size_t)ci * M + min(gj + u, M - 1);
          const bool in = gj + u < M;
          const float a = dK[o], b = Kf[o];
          dk[s][u] = in ? a : 0.f;
          kk[s][u] = in ? b : 0.f;
        }
      }
    }
  };
  auto commit_stage = [&](int t, const f32x4 (&dk)[4], const f32x4 (&kk)[4],
                          const bool (&ok)[4]) {
    float* dst = P[t & 1];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      store4(&dst[(srow + 16 * s) * kLds + scol], ok[s] ? dk[s] * kk[s] : zero4());
  };
  auto load_x = [&](int ic, f32x4 (&xs)[4]) {
    const size_t r = (size_t)min(ibase + ic * kTile + xrow, N - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) xs[s] = load4(X + r * kD + xcol + 16 * s);
  };
  auto commit_x = [&](int ic, const f32x4 (&xs)[4]) {
    float* dst = Xt[ic & 1];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) dst[(xcol + 16 * s + u) * kLds + xrow] = xs[s][u];
  };
  // X chunk published at step t: the one after the chunk of tile t (clamped;
  // at the last chunk that rewrites the chunk in use with identical bits).
  auto x_chunk = [&](int t) { return min(t / n_jc + 1, n_ic - 1); };

  // Tile 0's loads go out first, then every wave stages the region's Y rows
  // (Yt <- Y[jbase .. jbase+RJ), transposed, lanes along j so the transposed
  // LDS writes hit consecutive banks) while they are in flight.
  if (wave >= 4) {
    load_stage(0, g_dk[0], g_k[0], g_ok[0]);
    load_x(0, g_x[0]);
  }
  constexpr int kYtPerThread = RJ * 16 / 512;
  f32x4 yv[kYtPerThread];
#pragma unroll
  for (int k = 0; k < kYtPerThread; ++k) {
    const int f = tid + 512 * k;
    yv[k] = load4(Y + (size_t)min(jbase + f % RJ, M - 1) * kD + (f / RJ) * 4);
  }
#pragma unroll
  for (int k = 0; k < kYtPerThread; ++k) {
    const int f = tid + 512 * k;
    const int j = f % RJ;
    const int c = (f / RJ) * 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) Yt[(c + u) * kYtLds + j] = yv[k][u];
  }
  // Both roles pass 1 + n_steps barriers; the staging loop is unrolled by
  // three, so the compute side pads its tile barriers up to n_steps.
  const int n_steps = (n_tiles + 2) / 3 * 3;

  if (wave >= 4) {
    // ------------------------------------------------------ staging waves
    // Every step t runs the same straight-line sequence (no branches, so the
    // loads of later tiles stay in flight across steps): load tile t+3 and
    // the X chunk step t+2 publishes into the register stage published last
    // step, then publish stage (t+1) % 3, loaded two steps ago: W of tile
    // t+1 and the X chunk after tile t's.  Every wait is therefore on loads
    // two steps old (the memory counter retires in order, so one younger
    // consumer would make every step wait for the previous step's loads).
    // Indices are clamped: loads past the last tile fetch valid data nobody
    // uses; commits past it fill the idle P buffer.  A republished X chunk rewrites the buffer the compute waves
    // are reading only with identical bits.  The three register stages are
    // addressed statically (the loop is unrolled by three): a runtime stage
    // index would be if-converted into selects on the loaded data, forcing a
    // wait right after each load.
    load_stage(min(1, n_tiles - 1), g_dk[1], g_k[1], g_ok[1]);
    load_x(x_chunk(0), g_x[1]);
    load_stage(min(2, n_tiles - 1), g_dk[2], g_k[2], g_ok[2]);
    load_x(x_chunk(1), g_x[2]);
    commit_x(0, g_x[0]);
    commit_stage(0, g_dk[0], g_k[0], g_ok[0]);
    __syncthreads();
    auto step = [&](int t, f32x4 (&ldk)[4], f32x4 (&lk)[4], bool (&lok)[4], f32x4 (&lx)[4],
                    const f32x4 (&cdk)[4], const f32x4 (&ck)[4], const bool (&cok)[4],
                    const f32x4 (&cx)[4]) {
      // The scheduling fences keep each step's work between its barriers:
      // hoisting the next step's W products above the barrier would make
      // them wait on loads issued only one step earlier.
      __builtin_amdgcn_sched_barrier(0);
      load_stage(min(t + 3, n_tiles - 1), ldk, lk, lok);
      load_x(x_chunk(t + 2), lx);
      commit_x(x_chunk(t), cx);
      commit_stage(t + 1, cdk, ck, cok);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    // Tile t's data sits in stage t % 3: step t publishes stage (t+1) % 3 and
    // refills stage t % 3 (free since step t-1 published it) with tile t+3.
    for (int t = 0; t < n_steps; t += 3) {
      step(t, g_dk[0], g_k[0], g_ok[0], g_x[0], g_dk[1], g_k[1], g_ok[1], g_x[1]);
      step(t + 1, g_dk[1], g_k[1], g_ok[1], g_x[1], g_dk[2], g_k[2], g_ok[2], g_x[2]);
      step(t + 2, g_dk[2], g_k[2], g_ok[2], g_x[2], g_dk[0], g_k[0], g_ok[0], g_x[0]);
    }
    return;
  }

  // ------------------------------------------------------- compute waves
  const int wb = wave;  // 16-row block for (W.Y)^T, 16-column block for (W^T.X)^T
  f32x4 accX[4];
  float rp = 0.f;
  f32x4 accY[JC][4];
  float cp[JC];
#pragma unroll
  for (int c = 0; c < JC; ++c) {
    cp[c] = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) accY[c][db] = zero4();
  }
  __syncthreads();

  for (int ic = 0; ic < n_ic; ++ic) {
#pragma unroll
    for (int db = 0; db < 4; ++db) accX[db] = zero4();
    rp = 0.f;
    const float* Xb = Xt[ic & 1];
#pragma unroll
    for (int jc = 0; jc < JC; ++jc) {
      if (jc < n_jc) {
        const int t = ic * n_jc + jc;
        const float* Pb = P[t & 1];
        const float* Yb = Yt + jc * kTile;
        f32x4 xa[2], xbv[2][4], yb[2][4];
        float ya[2][4];
        // k-quarter 0 operands
        xa[0] = load4(&Pb[(wb * 16 + n) * kLds + 4 * h]);
#pragma unroll
        for (int db = 0; db < 4; ++db) xbv[0][db] = load4(&Yb[(db * 16 + n) * kYtLds + 4 * h]);
#pragma unroll
        for (int u = 0; u < 4; ++u) ya[0][u] = Pb[(4 * h + u) * kLds + wb * 16 + n];
#pragma unroll
        for (int db = 0; db < 4; ++db) yb[0][db] = load4(&Xb[(db * 16 + n) * kLds + 4 * h]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = q & 1;
          if (q < 3) {
            const int k1 = 16 * (q + 1) + 4 * h;
            xa[c ^ 1] = load4(&Pb[(wb * 16 + n) * kLds + k1]);
#pragma unroll
            for (int db = 0; db < 4; ++db) xbv[c ^ 1][db] = load4(&Yb[(db * 16 + n) * kYtLds + k1]);
#pragma unroll
            for (int u = 0; u < 4; ++u) ya[c ^ 1][u] = Pb[(k1 + u) * kLds + wb * 16 + n];
#pragma unroll
            for (int db = 0; db < 4; ++db) yb[c ^ 1][db] = load4(&Xb[(db * 16 + n) * kLds + k1]);
          }
          rp += (xa[c][0] + xa[c][1]) + (xa[c][2] + xa[c][3]);
          cp[jc] += (ya[c][0] + ya[c][1]) + (ya[c][2] + ya[c][3]);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int db = 0; db < 4; ++db) accX[db] = mfma16x4(xa[c][u], xbv[c][db][u], accX[db]);
#pragma unroll
            for (int db = 0; db < 4; ++db)
              accY[jc][db] = mfma16x4(ya[c][u], yb[c][db][u], accY[jc][db]);
          }
        }
        __syncthreads();
      }
    }

    // Row sums: lane (m, h) summed columns 16q+4h+u of row 16wb+m.
    float rs = rp;
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
    const size_t slot = (size_t)rj * N;
    const int i_base = ibase + ic * kTile + wb * 16;
    if (h == 0 && i_base + n < N) Rx[slot + i_base + n] = rs;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i_base + 4 * h + r;
      if (i < N) {
#pragma unroll
        for (int db = 0; db < 4; ++db) Px[(slot + i) * kD + db * 16 + n] = accX[db][r];
      }
    }
  }

  for (int t = n_tiles; t < n_steps; ++t) __syncthreads();

  const size_t slot = (size_t)ri * M;
#pragma unroll
  for (int jc = 0; jc < JC; ++jc) {
    if (jc < n_jc) {
      float cs = cp[jc];
      cs += __shfl_xor(cs, 16, 64);
      cs += __shfl_xor(cs, 32, 64);
      const int j_base = jbase + jc * kTile + wb * 16;
      if (h == 0 && j_base + n < M) Ry[slot + j_base + n] = cs;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j_base + 4 * h + r;
        if (j < M) {
#pragma unroll
          for (int db = 0; db < 4; ++db) Py[(slot + j) * kD + db * 16 + n] = accY[jc][db][r];
        }
      }
    }
  }
}

// Both outputs in one launch: block b < bx handles dX, the rest dY.
// out[r][:] = neg2g * (sum_s S[s][r] * A[r][:] - sum_s Pt[s][r][:]), D = 64,
// one thread per float4 of the output; the slot loop is unrolled by 4 so
// the loads of several slots are in flight together.
__global__ __launch_bounds__(256) void rbf_bwd_reduce_kernel(
    const float* __restrict__ Px, const float* __restrict__ Rx,
    const float* __restrict__ X, float* __restrict__ dX, int N, int sx,
    const float* __restrict__ Py, const float* __restrict__ Ry,
    const float* __restrict__ Y, float* __restrict__ dY, int M, int sy,
    int bx, float neg2g) {
  const bool is_x = (int)blockIdx.x < bx;
  const float* __restrict__ Pt = is_x ? Px : Py;
  const float* __restrict__ S = is_x ? Rx : Ry;
  const float* __restrict__ A = is_x ? X : Y;
  float* __restrict__ out = is_x ? dX : dY;
  const int rows = is_x ? N : M;
  const int slots = is_x ? sx : sy;
  const int b0 = is_x ? 0 : bx;
  const int nb = is_x ? bx : (int)gridDim.x - bx;
  const size_t n4 = (size_t)rows * (kD / 4);
  const size_t stride = (size_t)rows * kD;
  for (size_t e = (size_t)(blockIdx.x - b0) * blockDim.x + threadIdx.x; e < n4;
       e += (size_t)nb * blockDim.x) {
    const size_t r = e / (kD / 4);
    f32x4 a0 = zero4(), a1 = zero4(), a2 = zero4(), a3 = zero4();
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int s = 0;
    for (; s + 4 <= slots; s += 4) {
      a0 += load4(Pt + (size_t)s * stride + 4 * e);
      a1 += load4(Pt + (size_t)(s + 1) * stride + 4 * e);
      a2 += load4(Pt + (size_t)(s + 2) * stride + 4 * e);
      a3 += load4(Pt + (size_t)(s + 3) * stride + 4 * e);
      s0 += S[(size_t)s * rows + r];
      s1 += S[(size_t)(s + 1) * rows + r];
      s2 += S[(size_t)(s + 2) * rows + r];
      s3 += S[(size_t)(s + 3) * rows + r];
    }
    for (; s < slots; ++s) {
      a0 += load4(Pt + (size_t)s * stride + 4 * e);
      s0 += S[(size_t)s * rows + r];
    }
    const f32x4 acc = (a0 + a1) + (a2 + a3);
    const float sum = (s0 + s1) + (s2 + s3);
    store4(out + 4 * e, neg2g * (sum * load4(A + 4 * e) - acc));
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
  size_t px = 0, rx = 0, py = 0, ry = 0;  // workspace offsets (floats)
  size_t ws_floats = 0;
};

BwdPlan plan_backward(int64_t N, int64_t M, int64_t D) {
  BwdPlan p;
  if (D != kD || N <= 0 || M <= 0) return p;
  p.fast = true;
  // Region edges above 256 would need more than 256 accumulator registers
  // per lane on the dY side (two waves per SIMD), so R stays <= 256.
  int R = 64;
  for (int cand = 256; cand >= 64; cand >>= 1) {
    if (nl2k::ceil_div(N, cand) * nl2k::ceil_div(M, cand) >= kTargetRegions) {
      R = cand;
      break;
    }
  }
  p.R = R;
  p.JC = R / kTile;
  p.nRI = (int)nl2k::ceil_div(N, R);
  p.nRJ = (int)nl2k::ceil_div(M, R);
  // Workspace: partial (W.Y) [nRJ][N][64], partial row sums [nRJ][N],
  // partial (W^T.X) [nRI][M][64], partial column sums [nRI][M].
  p.px = 0;
  p.rx = p.px + (size_t)p.nRJ * N * kD;
  p.py = p.rx + (size_t)p.nRJ * N;
  p.ry = p.py + (size_t)p.nRI * M * kD;
  p.ws_floats = p.ry + (size_t)p.nRI * M;
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
                     const float* dK, const float* K, float* ws, int N, int M,
                     int vec_nm, hipStream_t stream) {
  float* Px = ws + p.px;
  float* Rx = ws + p.rx;
  float* Py = ws + p.py;
  float* Ry = ws + p.ry;
  if (vec_nm)
    hipLaunchKernelGGL((rbf_bwd_d64_kernel<JC, true>), dim3(p.nRI * p.nRJ), dim3(512), 0,
                       stream, X, Y, dK, K, Px, Rx, Py, Ry, N, M, p.R, p.nRJ);
  else
    hipLaunchKernelGGL((rbf_bwd_d64_kernel<JC, false>), dim3(p.nRI * p.nRJ), dim3(512), 0,
                       stream, X, Y, dK, K, Px, Rx, Py, Ry, N, M, p.R, p.nRJ);
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
    const int n_jt = (int)nl2k::ceil_div(M, kTile);
    const int64_t n_units64 = nl2k::ceil_div(N, kFwdRows) * n_jt;
    if (n_units64 > INT32_MAX)
      return nl2k::fail(NL2K_ERR_OVERFLOW, "rbf_forward_f32: too many tiles");
    const int n_units = (int)n_units64;
    const int upw = (int)nl2k::ceil_div(n_units, kFwdWorkgroups);
    const int n_wg = (int)nl2k::ceil_div(n_units, upw);
    hipLaunchKernelGGL(rbf_fwd_d64_kernel, dim3(n_wg), dim3(256), 0, stream, X, Y, K,
                       (int)N, (int)M, -gamma * kLog2e, n_jt, n_units, upw, vec_store);
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
  return p.ws_floats * sizeof(float);
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
    const size_t need = p.ws_floats * sizeof(float);
    if (workspace == nullptr || workspace_bytes < need)
      return nl2k::fail(NL2K_ERR_WORKSPACE,
                        "rbf_backward_f32: workspace of %zu bytes required, got %zu",
                        need, workspace ? workspace_bytes : (size_t)0);
    if (!nl2k::aligned16(workspace))
      return nl2k::fail(NL2K_ERR_ALIGN, "rbf_backward_f32: workspace must be 16-byte aligned");
    float* ws = static_cast<float*>(workspace);
    const int vec_nm = (M % 4 == 0) && nl2k::aligned16(dK) && nl2k::aligned16(K);
    switch (p.JC) {
      case 1: launch_bwd_fast<1>(p, X, Y, dK, K, ws, (int)N, (int)M, vec_nm, stream); break;
      case 2: launch_bwd_fast<2>(p, X, Y, dK, K, ws, (int)N, (int)M, vec_nm, stream); break;
      default: launch_bwd_fast<4>(p, X, Y, dK, K, ws, (int)N, (int)M, vec_nm, stream); break;
    }
    st = nl2k::check_launch("rbf_backward_f32");
    if (st) return st;
    const int bx = (int)std::min<int64_t>((N * (kD / 4) + 255) / 256, 2048);
    const int by = (int)std::min<int64_t>((M * (kD / 4) + 255) / 256, 2048);
    hipLaunchKernelGGL(rbf_bwd_reduce_kernel, dim3(bx + by), dim3(256), 0, stream,
                       ws + p.px, ws + p.rx, X, dX, (int)N, p.nRJ, ws + p.py, ws + p.ry,
                       Y, dY, (int)M, p.nRI, bx, neg2g);
    return nl2k::check_launch("rbf_backward_f32 (reduce)");
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
