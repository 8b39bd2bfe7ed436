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
//  * Other feature widths and misaligned pointers use tiled SIMT kernels:
//    64 x 64 tiles staged through LDS, the forward summing the squared
//    differences directly, the backward forming W in LDS and walking it in
//    slices whose partial sums a reduce kernel adds in order (unsplit when
//    the caller passes no workspace for them).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>

#include "../../../csrc/common.h"
#include "../../../csrc/pairwise_d64.h"
#include "rbf.h"

using nl2k::f32x4;
using nl2k::load4;
using nl2k::store4;
using nl2k::zero4;
using nl2k::pairwise::kD;

namespace {

constexpr float kLog2e = 1.4426950408889634f;

// Forward policy: the row term is -kappa |x|^2, the column term |y|^2, and
// K = exp2(min(2 kappa x.y - kappa (|x|^2 + |y|^2), 0)); the clamp keeps
// K <= 1 when the distance cancels to a tiny negative value.
struct RbfFwdOp {
  float neg_kappa;  // -gamma log2(e)
  static constexpr bool kSideOut = false;
  static constexpr bool kRowScales = false;
  __device__ __forceinline__ float row(f32x4 (&)[4], float sx) const { return neg_kappa * sx; }
  __device__ __forceinline__ float col(f32x4&, float sy) const { return sy; }
  __device__ __forceinline__ float out(float dot, float rt, float ct) const {
    float t = fmaf(-2.f * neg_kappa, dot, fmaf(neg_kappa, ct, rt));
    t = t > 0.f ? 0.f : t;  // squared distance >= 0; NaN passes through
    return __builtin_amdgcn_exp2f(t);
  }
};

// Backward policy: W = dK o K, raw X / Y rows, row and column sums of W.
struct RbfBwdOp {
  static constexpr bool kProduct = true, kScale = false, kSums = true;
};

// ------------------------------------------------------------------ forward
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
// Tiled SIMT kernels for the shapes the MFMA engine does not take (D != 64,
// misaligned pointers, N or M past its limit).  256 threads, a 64 x 64 tile
// of entries, each thread a 4 x 4 block of them; D is staged through LDS in
// chunks, k-major, so a thread reads its 4 X and 4 Y values as two float4.
// Rows or columns past the end, and features past D, load as zeros.
constexpr int kGT = 64;   // generic tile edge
constexpr int kGK = 16;   // forward: features per LDS chunk
constexpr int kGD = 64;   // backward: output features per pass

// K[i][j] = exp(-gamma sum_d (x_id - y_jd)^2), the squared differences
// summed directly (as the reference kernel does), in feature order.
__global__ __launch_bounds__(256) void rbf_fwd_generic_kernel(
    const float* __restrict__ X, const float* __restrict__ Y,
    float* __restrict__ K, int64_t N, int64_t M, int64_t D, float gamma) {
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
      const float xv = X[min(gi, N - 1) * D + min(gk, D - 1)];
      const float yv = Y[min(gj, M - 1) * D + min(gk, D - 1)];
      xs[k][r] = (kin && gi < N) ? xv : 0.f;
      ys[k][r] = (kin && gj < M) ? yv : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < kGK; ++k) {
      const f32x4 xa = *reinterpret_cast<const f32x4*>(&xs[k][4 * ty]);
      const f32x4 yb = *reinterpret_cast<const f32x4*>(&ys[k][4 * tx]);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float t = xa[a] - yb[b];
          s[a][b] = fmaf(t, t, s[a][b]);
        }
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
      if (j < M) K[i * M + j] = expf(-gamma * s[a][b]);
    }
  }
  }
}

// TRANS = false: dX for 64 rows i0.. and 64 features d0..: out[i][d] =
// neg2g (r_i x_id - sum_j W_ij y_jd), r_i = sum_j W_ij, W = dK o K, j walked
// in 64-wide tiles in order.  TRANS = true: dY for 64 columns, the same with
// W transposed (i walked, X in place of Y).  The W tile is read from dK and
// K once per feature pass, row-contiguous in both cases.  With S > 1 slices
// the walk is cut into S ranges of `chunk` (a multiple of 64) and each
// writes its partial sums (pacc [S][rows][D], psum [S][rows]) for
// rbf_bwd_generic_reduce_kernel; with S == 1 the kernel writes out itself.
template <bool TRANS>
__global__ __launch_bounds__(256) void rbf_bwd_generic_kernel(
    const float* __restrict__ A, const float* __restrict__ Bm,
    const float* __restrict__ dK, const float* __restrict__ Kf,
    float* __restrict__ out, float* __restrict__ pacc, float* __restrict__ psum,
    int64_t N, int64_t M, int64_t D, float neg2g, int64_t S, int64_t chunk) {
  __shared__ float ws[kGT][kGT + 1];   // W tile, [own][other]
  __shared__ float bs[kGT][kGD + 4];   // other side's rows, [other][feature]
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
    // W tile: 64 x 64 entries, four float per thread, rows of dK / K
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int e = threadIdx.x + 256 * q;  // 0 .. 4095
      const int u = e / kGT, v = e % kGT;   // u: row of dK within the tile, v: column
      const int64_t gi = (TRANS ? o0 : r0) + u, gj = (TRANS ? r0 : o0) + v;
      const bool in = gi < N && gj < M && (TRANS ? gi : gj) < o_end;
      const int64_t idx = min(gi, N - 1) * M + min(gj, M - 1);
      const float wv = dK[idx] * Kf[idx];
      if (TRANS)
        ws[v][u] = in ? wv : 0.f;
      else
        ws[u][v] = in ? wv : 0.f;
    }
    // the other side's 64 rows x 64 features
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int e = threadIdx.x + 256 * q;
      const int u = e / kGD, v = e % kGD;
      const int64_t go = o0 + u, gd = d0 + v;
      const float bv = Bm[min(go, others - 1) * D + min(gd, D - 1)];
      bs[u][v] = (go < o_end && gd < D) ? bv : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int o = 0; o < kGT; ++o) {
      const f32x4 bb = *reinterpret_cast<const f32x4*>(&bs[o][4 * tx]);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const float w = ws[4 * ty + a][o];
        rsum[a] += w;
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
      if (S == 1)
        out[r * D + d] = neg2g * (rsum[a] * A[r * D + d] - acc[a][b]);
      else
        pacc[(slice * rows + r) * D + d] = acc[a][b];
    }
    if (S > 1 && dpass == 0 && tx == 0) psum[slice * rows + r] = rsum[a];
  }
  }
}

// out[r][d] = neg2g (sum_s psum[s][r] a[r][d] - sum_s pacc[s][r][d]), the
// slices added in order; block b < bx writes dX, the rest dY.
__global__ __launch_bounds__(256) void rbf_bwd_generic_reduce_kernel(
    const float* __restrict__ px, const float* __restrict__ sx, const float* __restrict__ X,
    float* __restrict__ dX, int64_t N, int64_t Sx, const float* __restrict__ py,
    const float* __restrict__ sy, const float* __restrict__ Y, float* __restrict__ dY, int64_t M,
    int64_t Sy, int64_t D, int bx, float neg2g) {
  const bool is_x = (int)blockIdx.x < bx;
  const float* __restrict__ P = is_x ? px : py;
  const float* __restrict__ Q = is_x ? sx : sy;
  const float* __restrict__ A = is_x ? X : Y;
  float* __restrict__ out = is_x ? dX : dY;
  const int64_t rows = is_x ? N : M, S = is_x ? Sx : Sy;
  const int64_t b0 = is_x ? 0 : bx, nb = is_x ? bx : (int64_t)gridDim.x - bx;
  const int64_t total = rows * D;
  for (int64_t e = ((int64_t)blockIdx.x - b0) * blockDim.x + threadIdx.x; e < total;
       e += nb * blockDim.x) {
    const int64_t r = e / D;
    float acc = 0.f, rs = 0.f;
    for (int64_t sl = 0; sl < S; ++sl) {
      acc += P[sl * total + e];
      rs += Q[sl * rows + r];
    }
    out[e] = neg2g * (rs * A[e] - acc);
  }
}

__global__ __launch_bounds__(256) void rbf_fill_zero_kernel(float* __restrict__ p,
                                                           size_t count) {
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < count;
       e += (size_t)gridDim.x * blockDim.x)
    p[e] = 0.f;
}

// ------------------------------------------------------------------ host side
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

// Slices of the generic backward's walk for one side (rows of output,
// `others` walked): enough that the side has about kGenericBlocks
// workgroups, each slice a multiple of 64 long.
constexpr int64_t kGenericBlocks = 1024;
struct GenericSplit {
  int64_t s = 1, chunk = 0;
};
inline GenericSplit generic_split(int64_t rows, int64_t others, int64_t D) {
  GenericSplit g;
  const int64_t tiles = nl2k::ceil_div(rows, (int64_t)kGT) * nl2k::ceil_div(D, (int64_t)kGD);
  const int64_t otiles = nl2k::ceil_div(others, (int64_t)kGT);
  const int64_t want = std::min(std::max<int64_t>(1, nl2k::ceil_div(kGenericBlocks, tiles)), otiles);
  g.chunk = nl2k::ceil_div(otiles, want) * kGT;
  g.s = nl2k::ceil_div(others, g.chunk);
  return g;
}
// Workspace floats of the generic backward's slices (0 when neither side splits).
inline size_t generic_ws_floats(int64_t N, int64_t M, int64_t D) {
  if (N <= 0 || M <= 0) return 0;
  const GenericSplit gx = generic_split(N, M, D), gy = generic_split(M, N, D);
  if (gx.s == 1 && gy.s == 1) return 0;
  return (size_t)(gx.s * N * (D + 1) + gy.s * M * (D + 1));
}

int launch_fill_zero(float* p, size_t count, hipStream_t stream) {
  if (count == 0) return NL2K_SUCCESS;
  const int blocks = (int)std::min<size_t>((count + 255) / 256, 4096);
  hipLaunchKernelGGL(rbf_fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, p, count);
  return nl2k::check_launch("rbf fill");
}

// The backward's tile kernels (which need the workspace) run for D == 64 and
// 16-byte aligned X, Y, dX and dY; everything else takes the generic kernels.
bool takes_tile_path(const nl2k::pairwise::BwdPlan& p, const float* X, const float* Y,
                     const float* dX, const float* dY) {
  return p.fast && nl2k::aligned16(X) && nl2k::aligned16(Y) && nl2k::aligned16(dX) &&
         nl2k::aligned16(dY);
}

// Both backward entry points: the caller's workspace, or the scratch array
// below for rbf_backward_f32_noalloc.
int backward_impl(const float* X, const float* Y, const float* dK, const float* K, float* dX,
                  float* dY, int64_t N, int64_t M, int64_t D, float gamma, void* workspace,
                  size_t workspace_bytes, hipStream_t stream, const char* who) {
  int st = validate_sizes(N, M, D);
  if (st) return st;
  if (N == 0 && M == 0) return nl2k::succeed();
  if ((N > 0 && (!X || !dX)) || (M > 0 && (!Y || !dY)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: X, Y, dX, dY must be non-null", who);
  // Empty sums: dX = 0 when M == 0, dY = 0 when N == 0.
  if (M == 0) return launch_fill_zero(dX, (size_t)(N * D), stream);
  if (N == 0) return launch_fill_zero(dY, (size_t)(M * D), stream);
  if (!dK || !K) return nl2k::fail(NL2K_ERR_NULL, "%s: dK and K must be non-null", who);

  const float neg2g = -2.f * gamma;
  const nl2k::pairwise::BwdPlan p = nl2k::pairwise::plan_backward(N, M, D, true);
  if (takes_tile_path(p, X, Y, dX, dY)) {
    const size_t need = p.ws_floats * sizeof(float);
    if (workspace == nullptr || workspace_bytes < need)
      return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                        need, workspace ? workspace_bytes : (size_t)0);
    if (!nl2k::aligned16(workspace))
      return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 16-byte aligned", who);
    float* ws = static_cast<float*>(workspace);
    const bool vec_nm = (M % 4 == 0) && nl2k::aligned16(dK) && nl2k::aligned16(K);
    nl2k::pairwise::launch_bwd_tiles<RbfBwdOp>(p, X, Y, dK, K, ws, (int)N, (int)M, vec_nm,
                                               nullptr, nullptr, stream);
    st = nl2k::check_launch(who);
    if (st) return st;
    const int bx = (int)std::min<int64_t>((N * (kD / 4) + 255) / 256, 2048);
    const int by = (int)std::min<int64_t>((M * (kD / 4) + 255) / 256, 2048);
    hipLaunchKernelGGL(rbf_bwd_reduce_kernel, dim3(bx + by), dim3(256), 0, stream,
                       ws + p.px, ws + p.rx, X, dX, (int)N, p.nRJ, ws + p.py, ws + p.ry,
                       Y, dY, (int)M, p.nRI, bx, neg2g);
    return nl2k::check_launch(who);
  }

  // Generic kernels: the walks split into slices when the workspace holds
  // their partial sums (a shorter or no workspace runs them whole).
  const int64_t dp = nl2k::ceil_div(D, (int64_t)kGD);
  GenericSplit gx = generic_split(N, M, D), gy = generic_split(M, N, D);
  const size_t gneed = generic_ws_floats(N, M, D) * sizeof(float);
  float* ws = static_cast<float*>(workspace);
  if (gneed == 0 || ws == nullptr || workspace_bytes < gneed ||
      reinterpret_cast<uintptr_t>(workspace) % 4 != 0) {
    gx = GenericSplit{1, nl2k::ceil_div(M, (int64_t)kGT) * kGT};
    gy = GenericSplit{1, nl2k::ceil_div(N, (int64_t)kGT) * kGT};
  }
  float* pxa = ws;
  float* pxs = gx.s > 1 ? pxa + gx.s * N * D : nullptr;
  float* pya = gx.s > 1 ? pxs + gx.s * N : ws;
  float* pys = gy.s > 1 ? pya + gy.s * M * D : nullptr;
  if (gx.s == 1) pxa = nullptr;
  if (gy.s == 1) pya = nullptr;
  hipLaunchKernelGGL(rbf_bwd_generic_kernel<false>,
                     dim3((unsigned)std::min<int64_t>(
                         nl2k::ceil_div(N, (int64_t)kGT) * dp * gx.s, 1 << 16)),
                     dim3(256), 0, stream, X, Y, dK, K, dX, pxa, pxs, N, M, D, neg2g, gx.s,
                     gx.chunk);
  st = nl2k::check_launch(who);
  if (st) return st;
  hipLaunchKernelGGL(rbf_bwd_generic_kernel<true>,
                     dim3((unsigned)std::min<int64_t>(
                         nl2k::ceil_div(M, (int64_t)kGT) * dp * gy.s, 1 << 16)),
                     dim3(256), 0, stream, Y, X, dK, K, dY, pya, pys, N, M, D, neg2g, gy.s,
                     gy.chunk);
  st = nl2k::check_launch(who);
  if (st || (gx.s == 1 && gy.s == 1)) return st;
  // dX and dY of the split sides in one launch (a side that did not split
  // has written its output already: zero blocks)
  const int bx = gx.s > 1 ? (int)std::min<int64_t>(nl2k::ceil_div(N * D, (int64_t)256), 2048) : 0;
  const int by = gy.s > 1 ? (int)std::min<int64_t>(nl2k::ceil_div(M * D, (int64_t)256), 2048) : 0;
  hipLaunchKernelGGL(rbf_bwd_generic_reduce_kernel, dim3((unsigned)(bx + by)), dim3(256), 0,
                     stream, pxa, pxs, X, dX, N, gx.s, pya, pys, Y, dY, M, gy.s, D, bx, neg2g);
  return nl2k::check_launch(who);
}

// ------------------------------------------------ scratch for the no-alloc entry
// rbf_backward_f32_noalloc keeps the backward's region partials here instead
// of in a caller workspace: 64 MiB per GPU, held from the first use of the
// library on that GPU until the process ends.  The name is a host-side
// stand-in; kernels get the device address that hipGetSymbolAddress returns,
// looked up once per device with that device current.
constexpr size_t kScratchBytes = size_t(64) << 20;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_ptr[kMaxDevices];

int scratch_address(void** out, const char* who) {
  int dev = -1;
  int st = nl2k::check_hip(hipGetDevice(&dev), who);
  if (st) return st;
  if (dev < 0 || dev >= kMaxDevices)
    return nl2k::fail(NL2K_ERR_HIP, "%s: device %d beyond the %d the library tracks", who, dev,
                      kMaxDevices);
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    st = nl2k::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), who);
    if (st) return st;
    if (p == nullptr)
      return nl2k::fail(NL2K_ERR_HIP, "%s: hipGetSymbolAddress returned a null scratch", who);
    scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return NL2K_SUCCESS;
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

  nl2k::pairwise::FwdPlan fp;
  if (D == kD && nl2k::aligned16(X) && nl2k::aligned16(Y) &&
      nl2k::pairwise::plan_forward(N, M, fp)) {
    const int vec_store = (M % 4 == 0) && nl2k::aligned16(K);
    auto* kernel = fp.ib == 2 ? &nl2k::pairwise::pair_fwd_d64_kernel<RbfFwdOp, 2>
                              : &nl2k::pairwise::pair_fwd_d64_kernel<RbfFwdOp, 4>;
    hipLaunchKernelGGL(kernel, dim3(fp.n_wg), dim3(256), 0, stream, X, Y, K, (int)N, (int)M,
                       RbfFwdOp{-gamma * kLog2e}, fp.n_jt, fp.n_units, fp.upw, vec_store, nullptr,
                       nullptr);
    return nl2k::check_launch("rbf_forward_f32");
  }
  const int64_t ntiles = nl2k::ceil_div(N, (int64_t)kGT) * nl2k::ceil_div(M, (int64_t)kGT);
  hipLaunchKernelGGL(rbf_fwd_generic_kernel, dim3((unsigned)std::min<int64_t>(ntiles, 1 << 16)),
                     dim3(256), 0, stream, X, Y, K, N, M, D, gamma);
  return nl2k::check_launch("rbf_forward_f32 (generic)");
}

size_t rbf_backward_workspace_bytes(int64_t N, int64_t M, int64_t D) {
  if (validate_sizes(N, M, D)) return 0;
  const nl2k::pairwise::BwdPlan p = nl2k::pairwise::plan_backward(N, M, D, true);
  // Shapes the tile path takes (when aligned) report its need; the others
  // the generic kernels' slices.  A misaligned call of a tile-path shape
  // runs the generic kernels unsplit within that workspace.
  return (p.fast ? p.ws_floats : generic_ws_floats(N, M, D)) * sizeof(float);
}

int rbf_backward_f32(const float* X, const float* Y, const float* dK,
                     const float* K, float* dX, float* dY, int64_t N,
                     int64_t M, int64_t D, float gamma, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  return backward_impl(X, Y, dK, K, dX, dY, N, M, D, gamma, workspace, workspace_bytes, stream,
                       "rbf_backward_f32");
}

size_t rbf_backward_noalloc_max_bytes(void) { return kScratchBytes; }

int rbf_backward_f32_noalloc(const float* X, const float* Y, const float* dK, const float* K,
                             float* dX, float* dY, int64_t N, int64_t M, int64_t D, float gamma,
                             hipStream_t stream) {
  const char* who = "rbf_backward_f32_noalloc";
  int st = validate_sizes(N, M, D);
  if (st) return st;
  // Only the tile path uses scratch; shapes and alignments that take the
  // generic kernels run whatever their size.
  const nl2k::pairwise::BwdPlan p = nl2k::pairwise::plan_backward(N, M, D, true);
  const size_t need = takes_tile_path(p, X, Y, dX, dY) ? p.ws_floats * sizeof(float) : 0;
  if (need > kScratchBytes)
    return nl2k::fail(NL2K_ERR_WORKSPACE,
                      "%s: N=%lld M=%lld D=%lld needs %zu bytes of scratch; the library's static "
                      "scratch holds %zu (use rbf_backward_f32 with a workspace)",
                      who, (long long)N, (long long)M, (long long)D, need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0 && N > 0 && M > 0) {
    st = scratch_address(&ws, who);
    if (st) return st;
  }
  return backward_impl(X, Y, dK, K, dX, dY, N, M, D, gamma, ws, kScratchBytes, stream, who);
}

}  // extern "C"
