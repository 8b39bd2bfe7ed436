// Pairwise row-by-row contractions at feature width 64 on fp32 MFMA
// (gfx950): the tile engines behind the RBF and cosine-similarity cases.
//
//  * pair_fwd_d64_kernel<Op>: out[i,j] = Op::out(x_i . y_j, row term i,
//    column term j) for X [N,64], Y [M,64].  Work unit = 256 (or 128) rows x
//    64 columns; a workgroup of four waves walks a contiguous range of units.
//    Each wave keeps its 64 X rows in MFMA operand registers (v_mfma_f32_
//    16x16x4_f32 layout, contraction index k = 16q + 4h + u permuted the same
//    way for both operands so every lane moves 16 contiguous bytes per load)
//    for as long as the row block lasts; the unit's 64 Y rows are staged once
//    per workgroup in LDS, double buffered, while the previous unit runs on
//    the matrix cores.  Op sees each row's squared norm when the row is
//    loaded (it may scale the row and returns the row's epilogue term) and
//    each Y row's squared norm when it is staged (likewise).
//  * pair_bwd_d64_kernel<Op, JC, kVecNM>: for an upstream [N,M] matrix W
//    (W = dK o K when Op::kProduct, else W = dK) both contractions W . Y and
//    W^T . X in one pass over the [N,M] inputs, as raw partials per region
//    (and, when Op::kSums, partial row / column sums of W); Op::kScale
//    multiplies every staged X row i by sx[i] and Y row j by sy[j] first.
//    A case-specific reduce kernel sums the partials and applies its
//    epilogue.  Layout of one region (R x R entries, R = 64 JC): waves 4-7
//    stage (load the upstream tiles three ahead into registers, form W into
//    the LDS tile buffer of the next tile, stage the next X chunk
//    transposed), waves 0-3 compute both contractions per 64x64 tile; each
//    role passes exactly one workgroup barrier per tile.
#pragma once

#include <algorithm>
#include <cstdint>

#include "common.h"

namespace nl2k {
namespace pairwise {

constexpr int kD = 64;           // feature width of the MFMA path
constexpr int kTile = 64;        // tile edge
constexpr int kLds = 68;         // padded LDS row stride (floats)
constexpr int kTileFloats = kTile * kLds;
constexpr int kTargetRegions = 256;  // one backward workgroup per CU
constexpr int kFwdWorkgroups = 512;  // two forward workgroups per CU
constexpr int kFwdRows = 256;        // rows per forward unit (4 waves x 64), or 128 (see plan_forward)
// The tile kernels index rows and columns with int, up to a tile or region
// past the last one; larger N or M take the callers' generic (int64) kernels.
constexpr int64_t kMaxTileDim = INT32_MAX - 1024;

// ------------------------------------------------------------------ forward
// Op interface:
//   static constexpr bool kSideOut      write Op::row / Op::col results to
//                                       rowv [N] / colv [M] (once each)
//   static constexpr bool kRowScales    Op::row rewrites the X row (it must
//                                       then run before the row's MFMAs)
//   float row(f32x4 (&x)[4], float sx)  row prep (x: this lane's 16 values
//                                       of the row, sx = |x|^2); returns the
//                                       row's epilogue term
//   float col(f32x4& y, float sy)       Y row prep at staging (y: 4 values)
//   float out(float dot, float rt, float ct)  the output entry
// IB: 16-row blocks per wave (4: 256-row units, 2: 128-row units).
template <class Op, int IB>
__global__ __launch_bounds__(256, 2) void pair_fwd_d64_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    float* __restrict__ K, int N, int M, Op op, int n_jt,
    int n_units, int units_per_wg, int vec_store,
    float* __restrict__ rowv, float* __restrict__ colv) {
  __shared__ float Ys[2][kTileFloats];
  __shared__ __attribute__((aligned(16))) float nyS[2][kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 15;
  const int h = lane >> 4;
  // Workgroup b takes units_per_wg units, or one more for the first
  // n_units - units_per_wg * gridDim.x workgroups (no division here: a
  // 64-bit one on every workgroup's critical path cost about 1 us).
  const int extra = n_units - units_per_wg * (int)gridDim.x;
  const int bx = (int)blockIdx.x;
  const int u_begin = bx * units_per_wg + min(bx, extra);
  const int u_end = min(u_begin + units_per_wg + (bx < extra ? 1 : 0), n_units);
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
      float p = gy[s][0] * gy[s][0] + gy[s][1] * gy[s][1] + gy[s][2] * gy[s][2] +
                gy[s][3] * gy[s][3];
      p += __shfl_xor(p, 1, 64);
      p += __shfl_xor(p, 2, 64);
      p += __shfl_xor(p, 4, 64);
      p += __shfl_xor(p, 8, 64);
      const float ct = op.col(gy[s], p);
      store4(&Ys[buf][r * kLds + scol], gy[s]);
      if ((tid & 15) == 0) nyS[buf][r] = ct;
    }
  };

  // X operand registers: lane (n, h) holds elements k = 16q + 4h + u of row
  // 16 ib + n of this wave's strip.  Contraction step (q, u) uses k-slot h.
  // The loads go out q-major, so the first contraction steps wait only for
  // their own slices.
  constexpr int kRows = 64 * IB;  // rows per unit
  f32x4 xb[IB][4];
  float ax[IB];  // Op::row term of row 16 ib + n
  int cur_rb = -1;
  auto load_x = [&](int rb) {
    const int i0 = rb * kRows + wave * 16 * IB;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int ib = 0; ib < IB; ++ib) {
        const int ir = min(i0 + ib * 16 + n, N - 1);
        xb[ib][q] = load4(X + (size_t)ir * kD + 16 * q + 4 * h);
      }
    cur_rb = rb;
  };
  auto row_terms = [&]() {
#pragma unroll
    for (int ib = 0; ib < IB; ++ib) {
      float sx = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) sx = fmaf(xb[ib][q][u], xb[ib][q][u], sx);
      sx += __shfl_xor(sx, 16, 64);
      sx += __shfl_xor(sx, 32, 64);
      ax[ib] = op.row(xb[ib], sx);
    }
  };

  // Prologue: the Y tile's loads go out first, so staging it (and the
  // barrier) waits for them alone, not for the X rows behind them; a row
  // term that leaves the row unchanged is taken after the unit's MFMAs,
  // which then wait only for the X slices they use.
  load_y(u_begin);
  load_x(u_begin / n_jt);
  commit_y(0);
  if constexpr (Op::kRowScales) row_terms();
  bool terms_due = !Op::kRowScales;
  __syncthreads();
  int buf = 0;

  for (int u = u_begin; u < u_end; ++u) {
    const bool has_next = u + 1 < u_end;
    if (has_next) load_y(u + 1);
    __builtin_amdgcn_sched_barrier(0);

    const float* Yb = Ys[buf];
    f32x4 acc[4][IB];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < IB; ++b) acc[a][b] = zero4();
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
          for (int ib = 0; ib < IB; ++ib)
            acc[jb][ib] = mfma16x4(ya[q & 1][jb][uu], xb[ib][q][uu], acc[jb][ib]);
      __builtin_amdgcn_sched_barrier(0);
    }

    if (!Op::kRowScales && terms_due) {
      row_terms();
      terms_due = false;
    }
    // Epilogue: out[i][j..j+3], i = i0 + 16 ib + n, j = j0 + 16 jb + 4h.
    const int i0 = (u / n_jt) * kRows + wave * 16 * IB;
    const int j0 = (u % n_jt) * kTile;
    if constexpr (Op::kSideOut) {
      // Row terms once per row block (its column tile 0), column terms once
      // per column tile (row block 0).
      if (u % n_jt == 0 && h == 0) {
#pragma unroll
        for (int ib = 0; ib < IB; ++ib)
          if (i0 + ib * 16 + n < N) rowv[i0 + ib * 16 + n] = ax[ib];
      }
      if (u / n_jt == 0 && tid < kTile && j0 + tid < M) colv[j0 + tid] = nyS[buf][tid];
    }
    const bool full = vec_store && i0 + 16 * IB <= N && j0 + 64 <= M;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const f32x4 ny = load4(&nyS[buf][jb * 16 + 4 * h]);
      const int j = j0 + jb * 16 + 4 * h;
#pragma unroll
      for (int ib = 0; ib < IB; ++ib) {
        const int i = i0 + ib * 16 + n;
        f32x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = op.out(acc[jb][ib][r], ax[ib], ny[r]);
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
    if (has_next && (u + 1) / n_jt != cur_rb) {
      load_x((u + 1) / n_jt);
      if constexpr (Op::kRowScales) row_terms();
      else terms_due = true;
    }
  }
}

// Launch shape of the forward: units of 256 x 64 (ib = 4 row blocks of 16
// per wave) or 128 x 64 (ib = 2), spread over at most kFwdWorkgroups
// workgroups (two per CU) as evenly as whole units allow, each workgroup
// taking a contiguous range.  128-row units when 256-row ones would give
// fewer than two per workgroup, so the grid stays full and balanced (with
// identical bits): 14.5 against 15.2 us at 2048 x 2048, 24.5 against
// 32.2 us at 3000 x 3000, 9.6 against 12.3 at 1024 x 1024; an even spread
// instead of ceil(units / 512) per workgroup: 49.1 against 54.0 us at
// 5000 x 5000, 60.3 against 65.4 at 6000 x 6000.
struct FwdPlan {
  int ib = 4, n_jt = 0, n_units = 0, upw = 0, n_wg = 0;
};

inline bool plan_forward(int64_t N, int64_t M, FwdPlan& p) {
  if (N <= 0 || M <= 0 || N > kMaxTileDim || M > kMaxTileDim) return false;  // callers skip empty
  p.n_jt = (int)ceil_div(M, kTile);
  p.ib = ceil_div(N, kFwdRows) * p.n_jt < 2 * kFwdWorkgroups ? 2 : 4;
  const int64_t n_units64 = ceil_div(N, 64 * p.ib) * p.n_jt;
  if (n_units64 > INT32_MAX) return false;
  p.n_units = (int)n_units64;
  p.n_wg = (int)std::min<int64_t>(p.n_units, kFwdWorkgroups);
  p.upw = p.n_units / p.n_wg;  // n_units % n_wg workgroups take one more
  return true;
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
//  * waves 4-7 (staging) load the upstream tiles up to three tiles ahead
//    into registers, form W into the LDS tile buffer of the next tile, and
//    stage the next i-chunk's X rows.
// LDS: Yt = the region's Y rows, transposed [d][j], staged once; Xt = X rows
// of an i-chunk, transposed [d][i], double buffered; P = W tile [i][j],
// double buffered.  Both roles run the same loop nest and pass exactly one
// workgroup barrier per tile.  Each region writes raw partial contractions
// (and partial row / column sums of W) to its workspace slot.
//
// Op interface: static constexpr bool kProduct (W = dK o K, else W = dK),
// kScale (scale X rows by sx, Y rows by sy), kSums (row / column sums).
template <class Op, int JC, bool kVecNM>
__global__ __launch_bounds__(512) void pair_bwd_d64_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    const float* dK, const float* Kf,
    float* __restrict__ Px, float* __restrict__ Rx, float* __restrict__ Py,
    float* __restrict__ Ry, int N, int M, int RI, int nRJ,
    const float* __restrict__ sx, const float* __restrict__ sy) {
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
  float g_xs[3];
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
        if constexpr (Op::kProduct) kk[s] = load4(Kf + o);
      } else {
        ok[s] = gi < N;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const size_t o = (size_t)ci * M + min(gj + u, M - 1);
          const bool in = gj + u < M;
          const float a = dK[o];
          dk[s][u] = in ? a : 0.f;
          if constexpr (Op::kProduct) {
            const float b = Kf[o];
            kk[s][u] = in ? b : 0.f;
          }
        }
      }
    }
  };
  auto commit_stage = [&](int t, const f32x4 (&dk)[4], const f32x4 (&kk)[4],
                          const bool (&ok)[4]) {
    float* dst = P[t & 1];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if constexpr (Op::kProduct)
        store4(&dst[(srow + 16 * s) * kLds + scol], ok[s] ? dk[s] * kk[s] : zero4());
      else
        store4(&dst[(srow + 16 * s) * kLds + scol], ok[s] ? dk[s] : zero4());
    }
  };
  auto load_x = [&](int ic, f32x4 (&xs)[4], float& sc) {
    const size_t r = (size_t)min(ibase + ic * kTile + xrow, N - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) xs[s] = load4(X + r * kD + xcol + 16 * s);
    if constexpr (Op::kScale) sc = sx[r];
  };
  auto commit_x = [&](int ic, const f32x4 (&xs)[4], float sc) {
    float* dst = Xt[ic & 1];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if constexpr (Op::kScale)
          dst[(xcol + 16 * s + u) * kLds + xrow] = xs[s][u] * sc;
        else
          dst[(xcol + 16 * s + u) * kLds + xrow] = xs[s][u];
      }
  };
  // X chunk published at step t: the one after the chunk of tile t (clamped;
  // at the last chunk that rewrites the chunk in use with identical bits).
  auto x_chunk = [&](int t) { return min(t / n_jc + 1, n_ic - 1); };

  // Tile 0's loads go out first, then every wave stages the region's Y rows
  // (Yt <- Y[jbase .. jbase+RJ), transposed, lanes along j so the transposed
  // LDS writes hit consecutive banks) while they are in flight.
  if (wave >= 4) {
    load_stage(0, g_dk[0], g_k[0], g_ok[0]);
    load_x(0, g_x[0], g_xs[0]);
  }
  constexpr int kYtPerThread = RJ * 16 / 512;
  f32x4 yv[kYtPerThread];
  float ys[kYtPerThread];
#pragma unroll
  for (int k = 0; k < kYtPerThread; ++k) {
    const int f = tid + 512 * k;
    const size_t yr = (size_t)min(jbase + f % RJ, M - 1);
    yv[k] = load4(Y + yr * kD + (f / RJ) * 4);
    if constexpr (Op::kScale) ys[k] = sy[yr];
  }
#pragma unroll
  for (int k = 0; k < kYtPerThread; ++k) {
    const int f = tid + 512 * k;
    const int j = f % RJ;
    const int c = (f / RJ) * 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (Op::kScale)
        Yt[(c + u) * kYtLds + j] = yv[k][u] * ys[k];
      else
        Yt[(c + u) * kYtLds + j] = yv[k][u];
    }
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
    // uses; commits past it fill the idle P buffer.  A republished X chunk
    // rewrites the buffer the compute waves are reading only with identical
    // bits.  The three register stages are addressed statically (the loop is
    // unrolled by three): a runtime stage index would be if-converted into
    // selects on the loaded data, forcing a wait right after each load.
    load_stage(min(1, n_tiles - 1), g_dk[1], g_k[1], g_ok[1]);
    load_x(x_chunk(0), g_x[1], g_xs[1]);
    load_stage(min(2, n_tiles - 1), g_dk[2], g_k[2], g_ok[2]);
    load_x(x_chunk(1), g_x[2], g_xs[2]);
    commit_x(0, g_x[0], g_xs[0]);
    commit_stage(0, g_dk[0], g_k[0], g_ok[0]);
    __syncthreads();
    auto step = [&](int t, f32x4 (&ldk)[4], f32x4 (&lk)[4], bool (&lok)[4], f32x4 (&lx)[4],
                    float& lxs, const f32x4 (&cdk)[4], const f32x4 (&ck)[4],
                    const bool (&cok)[4], const f32x4 (&cx)[4], float cxs) {
      // The scheduling fences keep each step's work between its barriers:
      // hoisting the next step's W products above the barrier would make
      // them wait on loads issued only one step earlier.
      __builtin_amdgcn_sched_barrier(0);
      load_stage(min(t + 3, n_tiles - 1), ldk, lk, lok);
      load_x(x_chunk(t + 2), lx, lxs);
      commit_x(x_chunk(t), cx, cxs);
      commit_stage(t + 1, cdk, ck, cok);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    // Tile t's data sits in stage t % 3: step t publishes stage (t+1) % 3 and
    // refills stage t % 3 (free since step t-1 published it) with tile t+3.
    for (int t = 0; t < n_steps; t += 3) {
      step(t, g_dk[0], g_k[0], g_ok[0], g_x[0], g_xs[0], g_dk[1], g_k[1], g_ok[1], g_x[1],
           g_xs[1]);
      step(t + 1, g_dk[1], g_k[1], g_ok[1], g_x[1], g_xs[1], g_dk[2], g_k[2], g_ok[2], g_x[2],
           g_xs[2]);
      step(t + 2, g_dk[2], g_k[2], g_ok[2], g_x[2], g_xs[2], g_dk[0], g_k[0], g_ok[0], g_x[0],
           g_xs[0]);
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
          if constexpr (Op::kSums) {
            rp += (xa[c][0] + xa[c][1]) + (xa[c][2] + xa[c][3]);
            cp[jc] += (ya[c][0] + ya[c][1]) + (ya[c][2] + ya[c][3]);
          }
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

    const size_t slot = (size_t)rj * N;
    const int i_base = ibase + ic * kTile + wb * 16;
    if constexpr (Op::kSums) {
      // Row sums: lane (m, h) summed columns 16q+4h+u of row 16wb+m.
      float rs = rp;
      rs += __shfl_xor(rs, 16, 64);
      rs += __shfl_xor(rs, 32, 64);
      if (h == 0 && i_base + n < N) Rx[slot + i_base + n] = rs;
    }
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
      const int j_base = jbase + jc * kTile + wb * 16;
      if constexpr (Op::kSums) {
        float cs = cp[jc];
        cs += __shfl_xor(cs, 16, 64);
        cs += __shfl_xor(cs, 32, 64);
        if (h == 0 && j_base + n < M) Ry[slot + j_base + n] = cs;
      }
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

// Region plan and workspace layout (floats): partial (W.Y) [nRJ][N][64],
// partial row sums [nRJ][N] (sums only), partial (W^T.X) [nRI][M][64],
// partial column sums [nRI][M] (sums only).
// ------------------------------------------------- backward, three roles
// The same region walk, staging pipeline, operand layouts and partial
// outputs as pair_bwd_d64_kernel, by workgroups of twelve waves in three
// roles, one wave of each per SIMD (wave w on SIMD w % 4):
//  * waves 0-3 run only the (W.Y)^T contraction (rows 16 (w & 3)..) and
//    flush its partials per i-chunk;
//  * waves 4-7 run only the (W^T.X)^T contraction (columns 16 (w & 3)..)
//    and flush at the end;
//  * waves 8-11 stage, as waves 4-7 do there, with one X register stage
//    loaded one step ahead (issued first in its step, so waiting for it
//    retires only loads at least two steps old apart from itself).
// Each SIMD thus has two waves issuing MFMAs, and one's waits on LDS,
// barriers or its partial stores are covered by the other's matrix work;
// every accumulator sees the same MFMA sequence, so the partials are
// bit-identical to pair_bwd_d64_kernel's.  The role index is read through
// readfirstlane so the compiler sees wave-uniform branches and gives each
// role its own live ranges (at most 168 VGPRs: three waves per SIMD).
// kFull (N and M multiples of 64, every byte offset of dK / K below 2^31):
// no tile is ragged, so the staging waves load through buffer resources
// with the tile's offset in a scalar register and a fixed per-lane offset,
// and form W without clamps or selects.  That takes about 50 of the ~75
// vector instructions per staging step off the SIMDs the matrix waves
// issue on (vector ALU and MFMA issue share a SIMD), with identical bits.
// Otherwise every tile is loaded with clamped addresses and masked
// (float4 loads: the launcher sends scalar-load shapes to
// pair_bwd_d64_kernel).
template <class Op, int JC, bool kFull, bool kQX>
__global__ __launch_bounds__(768) void pair_bwd_d64_3r_kernel(
    const float* X, const float* __restrict__ Y,
    const float* dK, const float* Kf,
    float* __restrict__ Px, float* __restrict__ Rx, float* __restrict__ Py,
    float* __restrict__ Ry, int N, int M, int RI, int nRJ,
    const float* sx, const float* __restrict__ sy) {
  // X, sx, dK and Kf are deliberately not __restrict__: with it the compiler
  // treats their loads as invariant and sinks a prefetch past the workgroup
  // barriers to its use (for dK / K, tile t+2's, which serialises the memory
  // latency; for X, the reload before the staging loop, which leaves the
  // loop's wait counts pessimistic).
  constexpr int RJ = JC * kTile;
  constexpr int kYtLds = RJ + 4;
  __shared__ __attribute__((aligned(16))) float P[2][kTileFloats];
  __shared__ __attribute__((aligned(16))) float Xt[2][kTileFloats];
  __shared__ __attribute__((aligned(16))) float Yt[kD * kYtLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform role
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
  // Skewed walk: region (ri, rj) visits its i-chunks starting at rj mod n_ic
  // and its j-chunks starting at ri mod n_jc.  With every region on the same
  // walk, the concurrent dK / K reads of all CUs share their address bits
  // and crowd the same memory channels; a 4096^2 read in 64 x 64 tiles took
  // 16.1 us in lockstep and 13.1 us skewed (12.2 us as whole rows).  The
  // walk position, not the chunk, selects the double buffers; the column
  // accumulators are kept per walk position and mapped back at the flush.
  const int ic0 = rj % n_ic, jc0 = ri % n_jc;
  auto chunk_at = [&](int pos) { return pos + ic0 < n_ic ? pos + ic0 : pos + ic0 - n_ic; };
  auto col_at = [&](int pos) { return pos + jc0 < n_jc ? pos + jc0 : pos + jc0 - n_jc; };

  // Staging-wave state (declared for all waves; only waves 8-11 use it).
  const int ptid = tid - 512;
  // W: float4 (row (p>>4) + 16 s, cols 4 (p & 15)..), s = 0..3.
  const int srow = (ptid >> 4) & 15;
  const int scol = (ptid & 15) * 4;
  // X chunk: row p & 63 (lanes along rows), float4 columns (p>>6) + 4 s.
  const int xrow = ptid & 63;
  const int xcol = ((ptid >> 6) & 3) * 4;
  f32x4 g_dk[3][4], g_k[3][4], g_x[4];
  float g_xs;
  bool g_ok[3][4];
  // Full-tile addressing: byte offsets of row srow, column scol of a tile
  // (and of row xrow, column xcol of an X chunk) from the tile's corner.
  const uint32_t lane_off = ((uint32_t)srow * (uint32_t)M + (uint32_t)scol) * 4u;
  const uint32_t xlane_off = (uint32_t)(xrow * kD + xcol) * 4u;
  const uint32_t nm_bytes = kFull ? (uint32_t)N * (uint32_t)M * 4u : 0u;
  const buffer_rsrc rdk = make_rsrc(dK, nm_bytes);
  const buffer_rsrc rkk = make_rsrc(Kf, Op::kProduct ? nm_bytes : 0u);
  const buffer_rsrc rxx = make_rsrc(X, kFull ? (uint32_t)N * (uint32_t)kD * 4u : 0u);
  auto load_stage = [&](int t, f32x4 (&dk)[4], f32x4 (&kk)[4], bool (&ok)[4]) {
    const int pi = t / n_jc;
    const int ic = chunk_at(pi), jc = col_at(t - pi * n_jc);
    const int ib = ibase + ic * kTile;
    const int jb = jbase + jc * kTile;
    if constexpr (kFull) {
      const int toff = (ib * M + jb) * 4;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        ok[s] = true;
        dk[s] = buffer_load4(rdk, lane_off, toff + s * 64 * M);
        if constexpr (Op::kProduct) kk[s] = buffer_load4(rkk, lane_off, toff + s * 64 * M);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int gi = ib + srow + 16 * s;
        const int gj = jb + scol;
        ok[s] = gi < N && gj < M;
        const size_t o = (size_t)min(gi, N - 1) * M + min(gj, M - 4);
        dk[s] = load4(dK + o);
        if constexpr (Op::kProduct) kk[s] = load4(Kf + o);
      }
    }
  };
  auto commit_stage = [&](int t, const f32x4 (&dk)[4], const f32x4 (&kk)[4],
                          const bool (&ok)[4]) {
    float* dst = P[t & 1];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f32x4 w = dk[s];
      if constexpr (Op::kProduct) w = w * kk[s];
      if constexpr (!kFull) w = ok[s] ? w : zero4();
      store4(&dst[(srow + 16 * s) * kLds + scol], w);
    }
  };
  auto load_x = [&](int pos, f32x4 (&xs)[4], float& sc) {
    if constexpr (kFull && !Op::kScale) {
      const int xoff = (ibase + chunk_at(pos) * kTile) * kD * 4;
#pragma unroll
      for (int s = 0; s < 4; ++s) xs[s] = buffer_load4(rxx, xlane_off + 64 * s, xoff);
      return;
    }
    const size_t r = (size_t)min(ibase + chunk_at(pos) * kTile + xrow, N - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) xs[s] = load4(X + r * kD + xcol + 16 * s);
    if constexpr (Op::kScale) sc = sx[r];
  };
  auto commit_x = [&](int pos, const f32x4 (&xs)[4], float sc) {
    float* dst = Xt[pos & 1];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if constexpr (Op::kScale)
          dst[(xcol + 16 * s + u) * kLds + xrow] = xs[s][u] * sc;
        else
          dst[(xcol + 16 * s + u) * kLds + xrow] = xs[s][u];
      }
  };
  // X chunk (walk position) published at step t: the one after tile t's
  // (clamped; at the last chunk that rewrites the chunk in use with
  // identical bits).
  auto x_chunk = [&](int t) { return min(t / n_jc + 1, n_ic - 1); };
  // kQX (every region four column tiles wide): step t publishes only part
  // t % 4 (16 of the 64 columns) of that chunk, so the next chunk is
  // complete after the four steps of the current one, with one X load and
  // four LDS writes per lane per step instead of four and sixteen.
  auto load_x_part = [&](int pos, int part, f32x4& xs) {
    xs = buffer_load4(rxx, xlane_off, (ibase + chunk_at(pos) * kTile) * kD * 4 + 64 * part);
  };
  auto commit_x_part = [&](int pos, int part, const f32x4& xs) {
    float* dst = Xt[pos & 1] + 16 * part * kLds;
#pragma unroll
    for (int u = 0; u < 4; ++u) dst[(xcol + u) * kLds + xrow] = xs[u];
  };
  f32x4 g_xq;

  // Tile 0's loads go out first.  The region's Y rows are staged by waves
  // 0-7 as four 64-column chunks, transposed into Yt[d][j]: the chunk of the
  // first walk position before the first barrier, the others (loaded now,
  // behind it) right after it, before the barrier that ends step 0 (the
  // first step that needs them).  Holding the first barrier for all 64 KB
  // of Y delayed every region's first tile by about 2 us.  Thread tid < 512
  // moves float4 f = tid + 512 k of a chunk: column f % 64 (lanes along j,
  // so the transposed LDS writes hit consecutive banks), d-group f / 64.
  if (wave >= 8) {
    load_x(0, g_x, g_xs);
    load_stage(0, g_dk[0], g_k[0], g_ok[0]);
  }
  constexpr int kYc = 2;  // float4 per thread per chunk
  f32x4 yv[JC][kYc];
  float ys[JC][kYc];
  auto commit_y = [&](int pc) {
#pragma unroll
    for (int k2 = 0; k2 < kYc; ++k2) {
      const int f = tid + 512 * k2;
      const int j = col_at(pc) * kTile + (f & 63);
      const int c = (f >> 6) * 4;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if constexpr (Op::kScale)
          Yt[(c + u) * kYtLds + j] = yv[pc][k2][u] * ys[pc][k2];
        else
          Yt[(c + u) * kYtLds + j] = yv[pc][k2][u];
      }
    }
  };
  if (tid < 512) {
#pragma unroll
    for (int pc = 0; pc < JC; ++pc) {
      if (pc < n_jc) {
#pragma unroll
        for (int k2 = 0; k2 < kYc; ++k2) {
          const int f = tid + 512 * k2;
          const size_t yr = (size_t)min(jbase + col_at(pc) * kTile + (f & 63), M - 1);
          yv[pc][k2] = load4(Y + yr * kD + (f >> 6) * 4);
          if constexpr (Op::kScale) ys[pc][k2] = sy[yr];
        }
      }
    }
    commit_y(0);
  }
  // Both roles pass 1 + n_tiles barriers.

  if (wave >= 8) {
    // ------------------------------------------------------ staging waves
    // Every step t runs the same straight-line sequence (no branches, so the
    // loads of later tiles stay in flight across steps): publish the X chunk
    // after tile t's (its registers were loaded last step), load the X chunk
    // for step t+1, load tile t+3 into the register stage published last
    // step, then publish W of tile t+1 from stage (t+1) % 3, loaded two steps
    // ago.  The memory counter retires in order, so the X wait, on the
    // step's oldest young load, retires nothing younger than two steps but
    // that load.  Indices are clamped: loads past the last tile fetch valid
    // data nobody uses; commits past it fill the idle P buffer.  A
    // republished X chunk rewrites the buffer the compute waves are reading
    // only with identical bits.  The three W register stages are addressed
    // statically (the loop is unrolled by three): a runtime stage index would
    // be if-converted into selects on the loaded data, forcing a wait right
    // after each load.
    // The X reload goes out before tiles 1 and 2 (the barrier keeps the
    // compiler from hoisting their loads above it): the loop then starts
    // with the same order of outstanding loads as every later pass, and the
    // wait counts at the loop head stay as tight as in the body.  Otherwise
    // the loop's first step of every three waited for the previous step's
    // tiles.
    commit_x(0, g_x, g_xs);
    if constexpr (kQX) load_x_part(x_chunk(0), 0, g_xq);
    else load_x(x_chunk(0), g_x, g_xs);
    __builtin_amdgcn_sched_barrier(0);
    load_stage(min(1, n_tiles - 1), g_dk[1], g_k[1], g_ok[1]);
    load_stage(min(2, n_tiles - 1), g_dk[2], g_k[2], g_ok[2]);
    __builtin_amdgcn_sched_barrier(0);
    commit_stage(0, g_dk[0], g_k[0], g_ok[0]);
    __syncthreads();
    auto step = [&](int t, f32x4 (&ldk)[4], f32x4 (&lk)[4], bool (&lok)[4],
                    const f32x4 (&cdk)[4], const f32x4 (&ck)[4], const bool (&cok)[4]) {
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kQX) {
        commit_x_part(x_chunk(t), t & 3, g_xq);
        load_x_part(x_chunk(t + 1), (t + 1) & 3, g_xq);
      } else {
        commit_x(x_chunk(t), g_x, g_xs);
        load_x(x_chunk(t + 1), g_x, g_xs);
      }
      load_stage(min(t + 3, n_tiles - 1), ldk, lk, lok);
      commit_stage(t + 1, cdk, ck, cok);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    int t = 0;
    for (; t + 3 <= n_tiles; t += 3) {
      step(t, g_dk[0], g_k[0], g_ok[0], g_dk[1], g_k[1], g_ok[1]);
      step(t + 1, g_dk[1], g_k[1], g_ok[1], g_dk[2], g_k[2], g_ok[2]);
      step(t + 2, g_dk[2], g_k[2], g_ok[2], g_dk[0], g_k[0], g_ok[0]);
    }
    // the last n_tiles % 3 steps, on the same static stages (no padding
    // steps: each would cost a barrier round and a reload of the last tile)
    if (t < n_tiles) step(t, g_dk[0], g_k[0], g_ok[0], g_dk[1], g_k[1], g_ok[1]);
    if (t + 1 < n_tiles) step(t + 1, g_dk[1], g_k[1], g_ok[1], g_dk[2], g_k[2], g_ok[2]);
    return;
  }

  // ------------------------------------------------------- compute waves
  const int wb = wave & 3;  // 16-row block of (W.Y)^T / 16-column block of (W^T.X)^T
  __syncthreads();
#pragma unroll
  for (int pc = 1; pc < JC; ++pc)
    if (pc < n_jc) commit_y(pc);
  if (wave < 4) {
    // (W.Y)^T rows 16 wb.. of every tile, accumulated over the region's
    // columns and flushed per i-chunk (dX side).
    for (int pi = 0; pi < n_ic; ++pi) {
      const int ic = chunk_at(pi);
      f32x4 accX[4];
#pragma unroll
      for (int db = 0; db < 4; ++db) accX[db] = zero4();
      float rp = 0.f;
#pragma unroll
      for (int pj = 0; pj < JC; ++pj) {
        if (pj < n_jc) {
          const int t = pi * n_jc + pj;
          const float* Pb = P[t & 1];
          const float* Yb = Yt + col_at(pj) * kTile;
          f32x4 xa[2], xbv[2][4];
          xa[0] = load4(&Pb[(wb * 16 + n) * kLds + 4 * h]);
#pragma unroll
          for (int db = 0; db < 4; ++db) xbv[0][db] = load4(&Yb[(db * 16 + n) * kYtLds + 4 * h]);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int c = q & 1;
            if (q < 3) {
              const int k1 = 16 * (q + 1) + 4 * h;
              xa[c ^ 1] = load4(&Pb[(wb * 16 + n) * kLds + k1]);
#pragma unroll
              for (int db = 0; db < 4; ++db) xbv[c ^ 1][db] = load4(&Yb[(db * 16 + n) * kYtLds + k1]);
            }
            if constexpr (Op::kSums) rp += (xa[c][0] + xa[c][1]) + (xa[c][2] + xa[c][3]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
              for (int db = 0; db < 4; ++db) accX[db] = mfma16x4(xa[c][u], xbv[c][db][u], accX[db]);
          }
          __syncthreads();
        }
      }
      const size_t slot = (size_t)rj * N;
      const int i_base = ibase + ic * kTile + wb * 16;
      if constexpr (Op::kSums) {
        float rs = rp;
        rs += __shfl_xor(rs, 16, 64);
        rs += __shfl_xor(rs, 32, 64);
        if (h == 0 && i_base + n < N) Rx[slot + i_base + n] = rs;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = i_base + 4 * h + r;
        if (i < N) {
#pragma unroll
          for (int db = 0; db < 4; ++db) Px[(slot + i) * kD + db * 16 + n] = accX[db][r];
        }
      }
    }
    return;
  }

  // (W^T.X)^T columns 16 wb.. of every tile, accumulated over the region's
  // rows (dY side), flushed at the end.
  f32x4 accY[JC][4];
  float cp[JC];
#pragma unroll
  for (int c = 0; c < JC; ++c) {
    cp[c] = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) accY[c][db] = zero4();
  }
  for (int pi = 0; pi < n_ic; ++pi) {
    const float* Xb = Xt[pi & 1];
#pragma unroll
    for (int jc = 0; jc < JC; ++jc) {  // walk position; column chunk col_at(jc)
      if (jc < n_jc) {
        const int t = pi * n_jc + jc;
        const float* Pb = P[t & 1];
        f32x4 yb[2][4];
        float ya[2][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) ya[0][u] = Pb[(4 * h + u) * kLds + wb * 16 + n];
#pragma unroll
        for (int db = 0; db < 4; ++db) yb[0][db] = load4(&Xb[(db * 16 + n) * kLds + 4 * h]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = q & 1;
          if (q < 3) {
            const int k1 = 16 * (q + 1) + 4 * h;
#pragma unroll
            for (int u = 0; u < 4; ++u) ya[c ^ 1][u] = Pb[(k1 + u) * kLds + wb * 16 + n];
#pragma unroll
            for (int db = 0; db < 4; ++db) yb[c ^ 1][db] = load4(&Xb[(db * 16 + n) * kLds + k1]);
          }
          if constexpr (Op::kSums) cp[jc] += (ya[c][0] + ya[c][1]) + (ya[c][2] + ya[c][3]);
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int db = 0; db < 4; ++db)
              accY[jc][db] = mfma16x4(ya[c][u], yb[c][db][u], accY[jc][db]);
        }
        __syncthreads();
      }
    }
  }
  const size_t slot = (size_t)ri * M;
#pragma unroll
  for (int jc = 0; jc < JC; ++jc) {
    if (jc < n_jc) {
      const int j_base = jbase + col_at(jc) * kTile + wb * 16;
      if constexpr (Op::kSums) {
        float cs = cp[jc];
        cs += __shfl_xor(cs, 16, 64);
        cs += __shfl_xor(cs, 32, 64);
        if (h == 0 && j_base + n < M) Ry[slot + j_base + n] = cs;
      }
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

struct BwdPlan {
  bool fast = false;
  int R = 64;  // region edge (rows and columns)
  int JC = 1;  // R / 64
  int nRI = 0, nRJ = 0;
  size_t px = 0, rx = 0, py = 0, ry = 0;  // workspace offsets (floats)
  size_t ws_floats = 0;
};

inline BwdPlan plan_backward(int64_t N, int64_t M, int64_t D, bool sums) {
  BwdPlan p;
  if (D != kD || N <= 0 || M <= 0 || N > kMaxTileDim || M > kMaxTileDim) return p;
  p.fast = true;
  // Region edges above 256 would need more than 256 accumulator registers
  // per lane on the dY side (two waves per SIMD), so R stays <= 256.  The
  // edge is the one with the lowest modelled time, in units of one 64 x 64
  // tile step (~2.35 us): one workgroup runs per CU at a time, so a launch
  // takes ceil(regions / 256) rounds of (R / 64)^2 steps plus about four
  // steps of fill and drain each, and the reduce moves the partial rows
  // (written once, read once) at about kStepBytes per step.  Measured
  // against the earlier rule (the largest edge giving >= 256 regions):
  // backward 44.7 against 64.3 us at 3000^2 (edge 192), 61.1 against
  // 78.6 at 3500^2 (256), 148.1 against 160.7 at 6000^2 (192), 26.1
  // against 32.7 at 1500^2 (128); 2048^2, 4096^2 and 8192^2 keep their edges.
  constexpr double kStepBytes = 11.75e6;
  int R = 64;
  double best = 0.0;
  for (int cand : {256, 192, 128, 64}) {
    const int64_t jc = cand / kTile, nri = ceil_div(N, cand), nrj = ceil_div(M, cand);
    const int64_t rounds = ceil_div(nri * nrj, kTargetRegions);
    const double partial_bytes = (double)(nrj * N + nri * M) * (kD + 1) * sizeof(float) * 2;
    const double cost = (double)(rounds * (jc * jc + 4)) + partial_bytes / kStepBytes;
    if (cand == 256 || cost < best) {
      best = cost;
      R = cand;
    }
  }
  p.R = R;
  p.JC = R / kTile;
  p.nRI = (int)ceil_div(N, R);
  p.nRJ = (int)ceil_div(M, R);
  p.px = 0;
  p.rx = p.px + (size_t)p.nRJ * N * kD;
  p.py = p.rx + (sums ? (size_t)p.nRJ * N : 0);
  p.ry = p.py + (size_t)p.nRI * M * kD;
  p.ws_floats = p.ry + (sums ? (size_t)p.nRI * M : 0);
  return p;
}

template <class Op, int JC>
void launch_bwd_tiles(const BwdPlan& p, const float* X, const float* Y, const float* dK,
                      const float* K, float* ws, int N, int M, bool vec_nm,
                      const float* sx, const float* sy, hipStream_t stream) {
  float* Px = ws + p.px;
  float* Rx = ws + p.rx;
  float* Py = ws + p.py;
  float* Ry = ws + p.ry;
  // Vector loads of the upstream tiles: the three-role kernel, with
  // full-tile buffer addressing when no tile is ragged and every byte offset
  // fits the resource's 32-bit range.  Scalar loads (M % 4 != 0 or
  // misaligned): the eight-wave kernel, which measured faster there (its
  // staging needs the registers the third role takes).
  const bool full = N % kTile == 0 && M % kTile == 0 &&
                    (int64_t)N * M * (int64_t)sizeof(float) < ((int64_t)1 << 31);
  // Quarter X publishing needs four column tiles in every region.
  const bool qx = full && JC == 4 && M % (4 * kTile) == 0 && !Op::kScale;
  if (vec_nm && qx)
    hipLaunchKernelGGL((pair_bwd_d64_3r_kernel<Op, JC, true, JC == 4 && !Op::kScale>),
                       dim3(p.nRI * p.nRJ), dim3(768), 0, stream, X, Y, dK, K, Px, Rx, Py, Ry, N, M,
                       p.R, p.nRJ, sx, sy);
  else if (vec_nm && full)
    hipLaunchKernelGGL((pair_bwd_d64_3r_kernel<Op, JC, true, false>), dim3(p.nRI * p.nRJ),
                       dim3(768), 0, stream, X, Y, dK, K, Px, Rx, Py, Ry, N, M, p.R, p.nRJ, sx, sy);
  else if (vec_nm)
    hipLaunchKernelGGL((pair_bwd_d64_3r_kernel<Op, JC, false, false>), dim3(p.nRI * p.nRJ),
                       dim3(768), 0, stream, X, Y, dK, K, Px, Rx, Py, Ry, N, M, p.R, p.nRJ, sx, sy);
  else
    hipLaunchKernelGGL((pair_bwd_d64_kernel<Op, JC, false>), dim3(p.nRI * p.nRJ), dim3(512), 0,
                       stream, X, Y, dK, K, Px, Rx, Py, Ry, N, M, p.R, p.nRJ, sx, sy);
}

template <class Op>
void launch_bwd_tiles(const BwdPlan& p, const float* X, const float* Y, const float* dK,
                      const float* K, float* ws, int N, int M, bool vec_nm,
                      const float* sx, const float* sy, hipStream_t stream) {
  switch (p.JC) {
    case 1: launch_bwd_tiles<Op, 1>(p, X, Y, dK, K, ws, N, M, vec_nm, sx, sy, stream); break;
    case 2: launch_bwd_tiles<Op, 2>(p, X, Y, dK, K, ws, N, M, vec_nm, sx, sy, stream); break;
    case 3: launch_bwd_tiles<Op, 3>(p, X, Y, dK, K, ws, N, M, vec_nm, sx, sy, stream); break;
    default: launch_bwd_tiles<Op, 4>(p, X, Y, dK, K, ws, N, M, vec_nm, sx, sy, stream); break;
  }
}

}  // namespace pairwise
}  // namespace nl2k
