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

#include "/root/repo/nl2cuda-kernel-agent_amd/csrc/common.h"
#include "rbf.h"

using nl2k::f32x4;
using nl2k::load4;
using nl2k::store4;
using nl2k::zero4;
using nl2k::mfma16x4;

__device__ unsigned long long g_tl[8 * 64 * 4];
namespace {

constexpr int kD = 64;           // feature width of the MFMA path
constexpr int kTile = 64;        // backward tile edge
constexpr int kLds = 68;         // padded LDS row stride (floats)
constexpr int kTileFloats = kTile * kLds;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTargetRegions = 256;  // one backward workgroup per CU
constexpr int kFwdWorkgroups = 512;  // two forward workgroups per CU

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

  // Region prologue (all waves): Yt <- Y[jbase .. jbase+RJ), transposed, with
  // lanes along j so the transposed LDS writes hit consecutive banks.
  for (int f = tid; f < RJ * 16; f += 512) {
    const int j = f % RJ;
    const int c = (f / RJ) * 4;
    const f32x4 v = load4(Y + (size_t)min(jbase + j, M - 1) * kD + c);
#pragma unroll
    for (int u = 0; u < 4; ++u) Yt[(c + u) * kYtLds + j] = v[u];
  }

  if (wave >= 4) {
    // ------------------------------------------------------ staging waves
    const int ptid = tid - 256;
    // W: float4 (row (p>>4) + 16 s, cols 4 (p & 15)..), s = 0..3.
    const int srow = ptid >> 4;
    const int scol = (ptid & 15) * 4;
    // X chunk: row p & 63 (lanes along rows), float4 columns (p>>6) + 4 s.
    const int xrow = ptid & 63;
    const int xcol = (ptid >> 6) * 4;
    f32x4 g_dk[2][4], g_k[2][4], g_x[4];
    bool g_ok[2][4];
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
    auto load_x = [&](int ic) {
      const size_t r = (size_t)min(ibase + ic * kTile + xrow, N - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) g_x[s] = load4(X + r * kD + xcol + 16 * s);
    };
    auto commit_x = [&](int ic) {
      float* dst = Xt[ic & 1];
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int u = 0; u < 4; ++u) dst[(xcol + 16 * s + u) * kLds + xrow] = g_x[s][u];
    };
    // One staging step per tile t (all before the tile's barrier): issue the
    // next chunk's X loads at the chunk's first tile and publish them at its
    // last, publish W of tile t+1 (loaded one step ago), issue the loads of
    // tile t+2.  The two register stages are addressed statically (the loop
    // below is unrolled by two): a runtime stage index would be if-converted
    // into selects on the loaded data, forcing a wait right after each load.
    auto step = [&](int t, f32x4 (&ldk)[4], f32x4 (&lk)[4], bool (&lok)[4],
                    const f32x4 (&cdk)[4], const f32x4 (&ck)[4], const bool (&cok)[4]) {
      const int ic = t / n_jc, jc = t - ic * n_jc;
      const bool more = ic + 1 < n_ic;
      if (jc == 0 && more) load_x(ic + 1);
      if (n_jc > 1 && jc == n_jc - 1 && more) commit_x(ic + 1);
      if (t + 1 < n_tiles) commit_stage(t + 1, cdk, ck, cok);
      if (t + 2 < n_tiles) load_stage(t + 2, ldk, lk, lok);
      if (n_jc == 1 && more) commit_x(ic + 1);
      __syncthreads();
    };

    load_x(0);
    load_stage(0, g_dk[0], g_k[0], g_ok[0]);
    if (n_tiles > 1) load_stage(1, g_dk[1], g_k[1], g_ok[1]);
    commit_x(0);
    commit_stage(0, g_dk[0], g_k[0], g_ok[0]);
    __syncthreads();
    for (int t = 0; t < n_tiles; t += 2) {
      step(t, g_dk[0], g_k[0], g_ok[0], g_dk[1], g_k[1], g_ok[1]);
      if (t + 1 < n_tiles) step(t + 1, g_dk[1], g_k[1], g_ok[1], g_dk[0], g_k[0], g_ok[0]);
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
        if (blockIdx.x == 0 && lane == 0) g_tl[(wave * 64 + t) * 4 + 0] = __builtin_amdgcn_s_memrealtime();
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


}
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s line %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)
int main() {
  int N = 4096, M = 4096, R = 256, nRI = 16, nRJ = 16;
  float *X, *Y, *dK, *Kf, *ws, *fl; size_t flb = 512u << 20;
  size_t wsf = (size_t)(nRJ * N + nRI * M) * 65;
  CK(hipMalloc(&X, N * 256)); CK(hipMalloc(&Y, M * 256)); CK(hipMalloc(&dK, (size_t)N * M * 4)); CK(hipMalloc(&Kf, (size_t)N * M * 4));
  CK(hipMalloc(&ws, wsf * 4)); CK(hipMalloc(&fl, flb));
  CK(hipMemset(X, 0, N * 256)); CK(hipMemset(Y, 0, M * 256)); CK(hipMemset(dK, 0, (size_t)N * M * 4)); CK(hipMemset(Kf, 0, (size_t)N * M * 4));
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  float* Px = ws; float* Rx = Px + (size_t)nRJ * N * 64; float* Py = Rx + (size_t)nRJ * N; float* Ry = Py + (size_t)nRI * M * 64;
  for (int rep = 0; rep < 4; ++rep) {
    CK(hipMemsetAsync(fl, rep, flb));
    CK(hipEventRecord(e0));
    hipLaunchKernelGGL((rbf_bwd_d64_kernel<4, true>), dim3(nRI * nRJ), dim3(512), 0, 0, X, Y, dK, Kf, Px, Rx, Py, Ry, N, M, R, nRJ);
    CK(hipEventRecord(e1)); CK(hipEventSynchronize(e1));
    float ms; CK(hipEventElapsedTime(&ms, e0, e1)); printf("kernel %.2f us\n", ms * 1000);
  }
  static unsigned long long t[8 * 64 * 4];
  CK(hipMemcpyFromSymbol(t, HIP_SYMBOL(g_tl), sizeof(t)));
  unsigned long long t0 = ~0ull; for (int i = 0; i < 8 * 64 * 4; ++i) if (t[i] && t[i] < t0) t0 = t[i];
  for (int w = 0; w < 8; w += 4) { printf("wave%d start/mfma/commit:\n", w); for (int k = 0; k < 16; ++k) printf("  t%2d %6.2f %6.2f %6.2f\n", k, (t[(w * 64 + k) * 4] - t0) / 100.0, (t[(w * 64 + k) * 4 + 1] - t0) / 100.0, (t[(w * 64 + k) * 4 + 2] - t0) / 100.0); }
  return 0;
}
