// Tiled SIMT kernels for pairwise row operations between X [N, D] and
// Y [M, D] at any D and alignment: the shapes the fp32 MFMA tile engine
// (pairwise_d64.h) does not take.  Shared by the RBF and cosine-similarity
// cases through small policies.
//
//  * Forward: a 64 x 64 tile of outputs per step, 256 threads, a 4 x 4
//    block per thread; features staged through LDS 16 at a time, k-major,
//    so a thread reads its 4 X and 4 Y values as two float4.  out[i][j] =
//    Op::out(sum_k Op::step(x_ik, y_jk)).
//  * Backward: for 64 output rows (X side, or the Y side with W transposed)
//    and 64 features per pass, sum over the other side of W[r][o] b[o][d]
//    (and of W[r][o] when Op::kSums), W = Op::w(dK, K) formed in LDS from
//    row-contiguous reads of dK / K in both directions.  The walk over the
//    other side is cut into S slices (about kGenericBlocks workgroups per
//    side, each slice a multiple of 64 long); each slice writes partial
//    sums [S][rows][D] (and [S][rows]) that the caller adds in slice
//    order, or, with S == 1 and no partial buffer, Op::finish writes the
//    output itself.
// Rows or columns past the end, and features past D, load as zeros; the
// grid strides over tiles, so any grid size works.
#pragma once

#include <algorithm>
#include <cstdint>

#include "common.h"

namespace nl2k {
namespace pairwise {

constexpr int kGT = 64;                 // tile edge
constexpr int kGK = 16;                 // forward: features per LDS chunk
constexpr int kGD = 64;                 // backward: output features per pass
constexpr int64_t kGenericBlocks = 1024;  // target workgroups per backward side

struct GenericSplit {
  int64_t s = 1, chunk = 0;
};

// Slices of one backward side (rows of output, `others` walked).
inline GenericSplit generic_split(int64_t rows, int64_t others, int64_t D) {
  GenericSplit g;
  const int64_t tiles = ceil_div(rows, (int64_t)kGT) * ceil_div(D, (int64_t)kGD);
  const int64_t otiles = ceil_div(others, (int64_t)kGT);
  const int64_t want = std::min(std::max<int64_t>(1, ceil_div(kGenericBlocks, tiles)), otiles);
  g.chunk = ceil_div(otiles, want) * kGT;
  g.s = ceil_div(others, g.chunk);
  return g;
}

// The unsliced walk of one side.
inline GenericSplit generic_whole(int64_t others) {
  return GenericSplit{1, ceil_div(others, (int64_t)kGT) * kGT};
}

template <class Op>
__global__ __launch_bounds__(256) void pair_fwd_generic_kernel(
    const float* __restrict__ X, const float* __restrict__ Y, float* __restrict__ out,
    int64_t N, int64_t M, int64_t D, Op op) {
  __shared__ float xs[kGK][kGT + 4];
  __shared__ float ys[kGK][kGT + 4];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int64_t ntj = (M + kGT - 1) / kGT, ntiles = (N + kGT - 1) / kGT * ntj;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t i0 = tile / ntj * kGT, j0 = tile % ntj * kGT;
    float s[4][4] = {};
    for (int64_t k0 = 0; k0 < D; k0 += kGK) {
      // 64 rows x 16 features of X and of Y: four of each per thread
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e = threadIdx.x + 256 * q;  // 0 .. 1023
        const int r = e / kGK, k = e % kGK;
        const int64_t gi = i0 + r, gj = j0 + r, gk = k0 + k;
        const bool kin = gk < D;
        const int64_t ci = min(gi, N - 1), cj = min(gj, M - 1);
        const float xv = X[ci * D + min(gk, D - 1)];
        const float yv = Y[cj * D + min(gk, D - 1)];
        xs[k][r] = (kin && gi < N) ? op.x_in(xv, ci) : 0.f;
        ys[k][r] = (kin && gj < M) ? op.y_in(yv, cj) : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int k = 0; k < kGK; ++k) {
        const f32x4 xa = *reinterpret_cast<const f32x4*>(&xs[k][4 * ty]);
        const f32x4 yb = *reinterpret_cast<const f32x4*>(&ys[k][4 * tx]);
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int b = 0; b < 4; ++b) s[a][b] = op.step(s[a][b], xa[a], yb[b]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int64_t i = i0 + 4 * ty + a;
      if (i >= N) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t j = j0 + 4 * tx + b;
        if (j < M) out[i * M + j] = op.out(s[a][b]);
      }
    }
  }
}

// TRANS = false: rows are X's (N), the walk is over Y's rows (M), W[i][j];
// TRANS = true: rows are Y's, the walk over X's, W transposed.  A: the
// output side's rows (for Op::finish), Bm: the walked side's rows.
template <class Op, bool TRANS>
__global__ __launch_bounds__(256) void pair_bwd_generic_kernel(
    const float* __restrict__ A, const float* __restrict__ Bm, const float* __restrict__ dK,
    const float* __restrict__ Kf, float* __restrict__ out, float* __restrict__ pacc,
    float* __restrict__ psum, int64_t N, int64_t M, int64_t D, int64_t S, int64_t chunk,
    Op op) {
  __shared__ float ws[kGT][kGT + 1];   // W tile, [own][other]
  __shared__ float bs[kGT][kGD + 4];   // walked side's rows, [other][feature]
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int64_t rows = TRANS ? M : N, others = TRANS ? N : M;
  const int64_t ndp = (D + kGD - 1) / kGD, ntiles = (rows + kGT - 1) / kGT * ndp * S;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r0 = tile / (ndp * S) * kGT;
    const int64_t dpass = tile % (ndp * S) / S, slice = tile % S;
    const int64_t d0 = dpass * kGD;
    const int64_t o_end = min(others, (slice + 1) * chunk);
    float acc[4][4] = {};
    float rsum[4] = {};
    for (int64_t o0 = slice * chunk; o0 < o_end; o0 += kGT) {
      // W tile: 64 x 64 entries from rows of dK / K, 16 per thread
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int e = threadIdx.x + 256 * q;  // 0 .. 4095
        const int u = e / kGT, v = e % kGT;   // u: row of dK within the tile, v: column
        const int64_t gi = (TRANS ? o0 : r0) + u, gj = (TRANS ? r0 : o0) + v;
        const bool in = gi < N && gj < M && (TRANS ? gi : gj) < o_end;
        const int64_t idx = min(gi, N - 1) * M + min(gj, M - 1);
        const float wv = op.w(dK, Kf, idx);
        if (TRANS)
          ws[v][u] = in ? wv : 0.f;
        else
          ws[u][v] = in ? wv : 0.f;
      }
      // the walked side's 64 rows x 64 features
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int e = threadIdx.x + 256 * q;
        const int u = e / kGD, v = e % kGD;
        const int64_t go = o0 + u, gd = d0 + v;
        const int64_t co = min(go, others - 1);
        const float bv = Bm[co * D + min(gd, D - 1)];
        bs[u][v] = (go < o_end && gd < D) ? op.template b_in<TRANS>(bv, co) : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int o = 0; o < kGT; ++o) {
        const f32x4 bb = *reinterpret_cast<const f32x4*>(&bs[o][4 * tx]);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float w = ws[4 * ty + a][o];
          if constexpr (Op::kSums) rsum[a] += w;
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[a][b] = fmaf(w, bb[b], acc[a][b]);
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int64_t r = r0 + 4 * ty + a;
      if (r >= rows) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t d = d0 + 4 * tx + b;
        if (d >= D) continue;
        if (pacc == nullptr)
          out[r * D + d] = op.finish(rsum[a], A[r * D + d], acc[a][b]);
        else
          pacc[(slice * rows + r) * D + d] = acc[a][b];
      }
      if (Op::kSums && pacc != nullptr && dpass == 0 && tx == 0) psum[slice * rows + r] = rsum[a];
    }
  }
}

}  // namespace pairwise
}  // namespace nl2k
