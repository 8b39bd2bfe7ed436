// Pairwise cosine similarity, forward and backward, fp32, for MI355X
// (gfx950).  C-ABI declared in include/cosine_sim.h.
//
// Reference semantics (cases/cosine_sim/reference.py:13-20): with
// s_a = 1 / (|a| + eps) and ah = s_a a (the same for B),
//   S[i,j] = ah_i . bh_j
// and, by autograd of that expression, for upstream dS:
//   dah_i = sum_j dS[i,j] bh_j
//   dA_i  = s_a dah_i - (ah_i . dah_i) / |a_i| ah_i     (0 for the second
//           term when |a_i| = 0, as torch's norm backward gives)
// and symmetrically for dB with dS^T.  (The reference's CUDA kernel,
// cosine_sim.cu:63-102, uses s_a in place of 1/|a| in the second term; the
// two agree to within eps / |a|.)
//
// Design (D == 64 fast path), on the RBF tile engines of
// csrc/pairwise_d64.h:
//  * Forward: the inverse norms are folded into the MFMA operands -- each
//    wave scales its X rows in registers when it loads them, and Y rows are
//    scaled as they are staged into LDS -- so the epilogue is a plain store
//    of the accumulators (no VALU work beside the matrix cores).  The same
//    launch writes inv_a / inv_b for the backward.
//  * Backward: one pass over dS (W = dS, no product), both contractions
//    dS . bh and dS^T . ah as region partials (the staged X / Y rows scaled
//    by inv_a / inv_b); cos_bwd_reduce_kernel sums the partials and applies
//    the projection, one 16-lane group per row.
//  * Other feature widths and misaligned pointers use the tiled SIMT kernels
//    of csrc/pairwise_generic.h (rows scaled by their inverse norms as they
//    are staged), the backward's walks in slices whose partial rows the
//    projection kernel adds in order.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "../../../csrc/common.h"
#include "../../../csrc/pairwise_d64.h"
#include "../../../csrc/pairwise_generic.h"
#include "cosine_sim.h"

using nl2k::f32x4;
using nl2k::load4;
using nl2k::store4;
using nl2k::zero4;
using nl2k::pairwise::kD;

namespace {

__device__ __forceinline__ float inv_norm(float sumsq, float eps) {
  return 1.f / (sqrtf(sumsq) + eps);
}

// Forward policy: rows scaled by their inverse norms before the contraction;
// the row / column terms written out are those inverse norms.
struct CosFwdOp {
  float eps;
  static constexpr bool kSideOut = true;
  static constexpr bool kRowScales = true;
  __device__ __forceinline__ float row(f32x4 (&x)[4], float sx) const {
    const float s = inv_norm(sx, eps);
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] *= s;
    return s;
  }
  __device__ __forceinline__ float col(f32x4& y, float sy) const {
    const float s = inv_norm(sy, eps);
    y *= s;
    return s;
  }
  __device__ __forceinline__ float out(float dot, float, float) const { return dot; }
};

// Backward policy: W = dS, X / Y rows scaled by inv_a / inv_b, no sums.
struct CosBwdOp {
  static constexpr bool kProduct = false, kScale = true, kSums = false;
};

// Both outputs in one launch: block b < bx handles dA, the rest dB.  One
// thread per float4 of the output, 16 threads per row (a 16-aligned lane
// group): acc = sum of the slots, then
//   out = s acc - (ah . acc) / |a| ah,  ah = s a.
__global__ __launch_bounds__(256) void cos_bwd_reduce_kernel(
    const float* __restrict__ Px, const float* __restrict__ A,
    const float* __restrict__ inv_a, float* __restrict__ dA, int N, int sx,
    const float* __restrict__ Py, const float* __restrict__ B,
    const float* __restrict__ inv_b, float* __restrict__ dB, int M, int sy, int bx) {
  const bool is_a = (int)blockIdx.x < bx;
  const float* __restrict__ Pt = is_a ? Px : Py;
  const float* __restrict__ V = is_a ? A : B;
  const float* __restrict__ inv = is_a ? inv_a : inv_b;
  float* __restrict__ out = is_a ? dA : dB;
  const int rows = is_a ? N : M;
  const int slots = is_a ? sx : sy;
  const int b0 = is_a ? 0 : bx;
  const int nb = is_a ? bx : (int)gridDim.x - bx;
  const size_t n4 = (size_t)rows * (kD / 4);
  const size_t stride = (size_t)rows * kD;
  // The stride is a multiple of 16 and rows start at multiples of 16, so the
  // 16 threads of a row are always active together.
  for (size_t e = (size_t)(blockIdx.x - b0) * blockDim.x + threadIdx.x; e < n4;
       e += (size_t)nb * blockDim.x) {
    const size_t r = e / (kD / 4);
    f32x4 a0 = zero4(), a1 = zero4(), a2 = zero4(), a3 = zero4();
    int s = 0;
    for (; s + 4 <= slots; s += 4) {
      a0 += load4(Pt + (size_t)s * stride + 4 * e);
      a1 += load4(Pt + (size_t)(s + 1) * stride + 4 * e);
      a2 += load4(Pt + (size_t)(s + 2) * stride + 4 * e);
      a3 += load4(Pt + (size_t)(s + 3) * stride + 4 * e);
    }
    for (; s < slots; ++s) a0 += load4(Pt + (size_t)s * stride + 4 * e);
    const f32x4 acc = (a0 + a1) + (a2 + a3);
    const f32x4 a = load4(V + 4 * e);
    const float sc = inv[r];
    const f32x4 ah = a * sc;
    float dot = (ah[0] * acc[0] + ah[1] * acc[1]) + (ah[2] * acc[2] + ah[3] * acc[3]);
    float nn = (a[0] * a[0] + a[1] * a[1]) + (a[2] * a[2] + a[3] * a[3]);
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      dot += __shfl_xor(dot, off, 64);
      nn += __shfl_xor(nn, off, 64);
    }
    const float nrm = sqrtf(nn);
    const float coef = nrm > 0.f ? dot / nrm : 0.f;
    store4(out + 4 * e, sc * acc - coef * ah);
  }
}

// ------------------------------------------------------- generic (any D)
// inv[r] = 1 / (|V_r| + eps), one wave per row.
__global__ __launch_bounds__(256) void cos_norm_kernel(const float* __restrict__ V,
                                                       float* __restrict__ inv, int64_t rows,
                                                       int64_t D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t r = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); r < rows;
       r += waves) {
    float ss = 0.f;
    for (int64_t d = lane; d < D; d += 64) ss = fmaf(V[r * D + d], V[r * D + d], ss);
    ss = nl2k::wave_sum(ss);
    if (lane == 0) inv[r] = inv_norm(ss, eps);
  }
}

// Policies of the tiled SIMT kernels (csrc/pairwise_generic.h).
// Forward: S = sum_d (a_d inv_a) (b_d inv_b), rows scaled as they are staged.
struct CosGenFwd {
  const float* __restrict__ inv_a;
  const float* __restrict__ inv_b;
  __device__ __forceinline__ float x_in(float v, int64_t i) const { return v * inv_a[i]; }
  __device__ __forceinline__ float y_in(float v, int64_t j) const { return v * inv_b[j]; }
  __device__ __forceinline__ float step(float s, float x, float y) const { return fmaf(x, y, s); }
  __device__ __forceinline__ float out(float s) const { return s; }
};
// Backward: dvh[r][d] = sum_o W[r, o] inv_o[o] O[o][d], W = dS (dS^T for the
// B side); the walked rows are scaled by their inverse norms as staged.
struct CosGenBwd {
  const float* __restrict__ inv_a;
  const float* __restrict__ inv_b;
  static constexpr bool kSums = false;
  __device__ __forceinline__ float w(const float* __restrict__ dS, const float*,
                                     int64_t idx) const {
    return dS[idx];
  }
  template <bool TRANS>
  __device__ __forceinline__ float b_in(float v, int64_t o) const {
    return v * (TRANS ? inv_a[o] : inv_b[o]);
  }
  __device__ __forceinline__ float finish(float, float, float acc) const { return acc; }
};

// out_r = s dvh_r - (vh_r . dvh_r) / |v_r| vh_r, one wave per row; dvh is
// the sum, in slice order, of the S partial rows part[s][r][:].
__device__ __forceinline__ float slice_sum(const float* __restrict__ part, int64_t S,
                                           int64_t plane, int64_t e) {
  float v = 0.f;
  for (int64_t sl = 0; sl < S; ++sl) v += part[sl * plane + e];
  return v;
}
__global__ __launch_bounds__(256) void cos_project_generic_kernel(
    const float* __restrict__ V, const float* __restrict__ inv, const float* __restrict__ part,
    int64_t S, float* __restrict__ out, int64_t rows, int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / 64);
  for (int64_t r = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); r < rows;
       r += waves) {
    const float sc = inv[r];
    float dot = 0.f, nn = 0.f;
    for (int64_t d = lane; d < D; d += 64) {
      const float v = V[r * D + d];
      dot = fmaf(v * sc, slice_sum(part, S, rows * D, r * D + d), dot);
      nn = fmaf(v, v, nn);
    }
    dot = nl2k::wave_sum(dot);
    nn = nl2k::wave_sum(nn);
    const float nrm = sqrtf(nn);
    const float coef = nrm > 0.f ? dot / nrm : 0.f;
    for (int64_t d = lane; d < D; d += 64)
      out[r * D + d] = sc * slice_sum(part, S, rows * D, r * D + d) - coef * (V[r * D + d] * sc);
  }
}

// Floats of the generic backward's partial rows: S slices a side when
// `sliced`, one otherwise.
inline size_t generic_ws_floats(int64_t N, int64_t M, int64_t D, bool sliced) {
  const int64_t sx = sliced ? nl2k::pairwise::generic_split(N, M, D).s : 1;
  const int64_t sy = sliced ? nl2k::pairwise::generic_split(M, N, D).s : 1;
  return (size_t)(sx * N * D + sy * M * D);
}

__global__ __launch_bounds__(256) void cos_fill_zero_kernel(float* __restrict__ p, size_t count) {
  for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < count;
       e += (size_t)gridDim.x * blockDim.x)
    p[e] = 0.f;
}

// ----------------------------------------------------------------- host side
int validate_sizes(int64_t N, int64_t M, int64_t D, const char* who) {
  if (N < 0 || M < 0 || D < 1)
    return nl2k::fail(NL2K_ERR_SHAPE,
                      "%s: sizes must satisfy N >= 0, M >= 0, D >= 1 (got N=%lld M=%lld D=%lld)",
                      who, (long long)N, (long long)M, (long long)D);
  const int64_t lim = INT32_MAX;
  if (N > lim || M > lim || D > lim || N > INT64_MAX / D || M > INT64_MAX / D ||
      (M > 0 && N > INT64_MAX / M))
    return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: sizes too large (N=%lld M=%lld D=%lld)", who,
                      (long long)N, (long long)M, (long long)D);
  return NL2K_SUCCESS;
}

int grid_for(int64_t work, int64_t per_block, int cap) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(nl2k::ceil_div(work, per_block), cap));
}

int launch_norms(const float* V, float* inv, int64_t rows, int64_t D, float eps,
                 hipStream_t stream) {
  if (rows == 0) return NL2K_SUCCESS;
  hipLaunchKernelGGL(cos_norm_kernel, dim3(grid_for(rows, 4, 1 << 16)), dim3(256), 0, stream, V,
                     inv, rows, D, eps);
  return nl2k::check_launch("cosine_sim norms");
}

int fill_zero(float* p, size_t count, hipStream_t stream) {
  if (count == 0) return NL2K_SUCCESS;
  hipLaunchKernelGGL(cos_fill_zero_kernel, dim3(grid_for((int64_t)count, 256, 4096)), dim3(256),
                     0, stream, p, count);
  return nl2k::check_launch("cosine_sim fill");
}

bool fast_backward(int64_t D, const void* A, const void* B, const void* dA, const void* dB) {
  return D == kD && nl2k::aligned16(A) && nl2k::aligned16(B) && nl2k::aligned16(dA) &&
         nl2k::aligned16(dB);
}

}  // namespace

extern "C" {

const char* cosine_sim_last_error(void) { return nl2k::error_slot().text; }

int cosine_sim_forward_f32(const float* A, const float* B, float* S, float* inv_a,
                           float* inv_b, int64_t N, int64_t M, int64_t D, float eps,
                           hipStream_t stream) {
  const char* who = "cosine_sim_forward_f32";
  int st = validate_sizes(N, M, D, who);
  if (st) return st;
  if ((N > 0 && (!A || !inv_a)) || (M > 0 && (!B || !inv_b)) || (N > 0 && M > 0 && !S))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (!(eps >= 0.f))
    return nl2k::fail(NL2K_ERR_VALUE, "%s: eps must be >= 0 (got %g)", who, (double)eps);
  if (N == 0 || M == 0) {  // no S; the inverse norms are still defined
    st = launch_norms(A, inv_a, N, D, eps, stream);
    if (st) return st;
    return launch_norms(B, inv_b, M, D, eps, stream);
  }
  nl2k::pairwise::FwdPlan fp;
  if (D == kD && nl2k::aligned16(A) && nl2k::aligned16(B) &&
      nl2k::pairwise::plan_forward(N, M, fp)) {
    const int vec_store = (M % 4 == 0) && nl2k::aligned16(S);
    auto* kernel = fp.ib == 2 ? &nl2k::pairwise::pair_fwd_d64_kernel<CosFwdOp, 2>
                              : &nl2k::pairwise::pair_fwd_d64_kernel<CosFwdOp, 4>;
    hipLaunchKernelGGL(kernel, dim3(fp.n_wg), dim3(256), 0, stream, A, B, S, (int)N, (int)M,
                       CosFwdOp{eps}, fp.n_jt, fp.n_units, fp.upw, vec_store, inv_a, inv_b);
    return nl2k::check_launch(who);
  }
  st = launch_norms(A, inv_a, N, D, eps, stream);
  if (st) return st;
  st = launch_norms(B, inv_b, M, D, eps, stream);
  if (st) return st;
  const int64_t ntiles = nl2k::ceil_div(N, (int64_t)nl2k::pairwise::kGT) *
                         nl2k::ceil_div(M, (int64_t)nl2k::pairwise::kGT);
  hipLaunchKernelGGL(nl2k::pairwise::pair_fwd_generic_kernel<CosGenFwd>,
                     dim3((unsigned)std::min<int64_t>(ntiles, 1 << 16)), dim3(256), 0, stream, A,
                     B, S, N, M, D, CosGenFwd{inv_a, inv_b});
  return nl2k::check_launch("cosine_sim_forward_f32 (generic)");
}

size_t cosine_sim_backward_workspace_bytes(int64_t N, int64_t M, int64_t D) {
  if (validate_sizes(N, M, D, "cosine_sim_backward_workspace_bytes")) return 0;
  if (N == 0 || M == 0) return 0;
  const nl2k::pairwise::BwdPlan p = nl2k::pairwise::plan_backward(N, M, D, false);
  const size_t fast = p.fast ? p.ws_floats * sizeof(float) : 0;
  // The generic kernels' partial rows: [S][N][D] and [S][M][D] for the
  // slices of shapes the tile path never takes; one slice a side (the
  // walks whole) otherwise, which a misaligned call of a tile shape uses.
  return std::max(fast, generic_ws_floats(N, M, D, !p.fast) * sizeof(float));
}

int cosine_sim_backward_f32(const float* A, const float* B, const float* inv_a,
                            const float* inv_b, const float* dS, float* dA, float* dB,
                            int64_t N, int64_t M, int64_t D, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
  const char* who = "cosine_sim_backward_f32";
  int st = validate_sizes(N, M, D, who);
  if (st) return st;
  if (N == 0 && M == 0) return nl2k::succeed();
  if ((N > 0 && (!A || !inv_a || !dA)) || (M > 0 && (!B || !inv_b || !dB)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  // Empty sums: dA = 0 when M == 0, dB = 0 when N == 0.
  if (M == 0) return fill_zero(dA, (size_t)(N * D), stream);
  if (N == 0) return fill_zero(dB, (size_t)(M * D), stream);
  if (!dS) return nl2k::fail(NL2K_ERR_NULL, "%s: dS must be non-null", who);
  const size_t need = cosine_sim_backward_workspace_bytes(N, M, D);
  if (workspace == nullptr || workspace_bytes < need)
    return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                      need, workspace ? workspace_bytes : (size_t)0);
  if (!nl2k::aligned16(workspace))
    return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 16-byte aligned", who);
  float* ws = static_cast<float*>(workspace);

  const nl2k::pairwise::BwdPlan p = nl2k::pairwise::plan_backward(N, M, D, false);
  if (p.fast && fast_backward(D, A, B, dA, dB)) {
    const bool vec_nm = (M % 4 == 0) && nl2k::aligned16(dS);
    nl2k::pairwise::launch_bwd_tiles<CosBwdOp>(p, A, B, dS, nullptr, ws, (int)N, (int)M, vec_nm,
                                               inv_a, inv_b, stream);
    st = nl2k::check_launch(who);
    if (st) return st;
    const int bx = grid_for(N * (kD / 4), 256, 2048);
    const int by = grid_for(M * (kD / 4), 256, 2048);
    hipLaunchKernelGGL(cos_bwd_reduce_kernel, dim3(bx + by), dim3(256), 0, stream, ws + p.px, A,
                       inv_a, dA, (int)N, p.nRJ, ws + p.py, B, inv_b, dB, (int)M, p.nRI, bx);
    return nl2k::check_launch("cosine_sim_backward_f32 (reduce)");
  }

  // generic kernels: the walks in slices when the workspace holds their
  // partial rows, else whole (the entry check above guarantees that much)
  using nl2k::pairwise::kGT;
  nl2k::pairwise::GenericSplit gx = nl2k::pairwise::generic_split(N, M, D),
                               gy = nl2k::pairwise::generic_split(M, N, D);
  if (workspace_bytes < generic_ws_floats(N, M, D, true) * sizeof(float)) {
    gx = nl2k::pairwise::generic_whole(M);
    gy = nl2k::pairwise::generic_whole(N);
  }
  float* dah = ws;                               // [Sx][N][D]
  float* dbh = ws + (size_t)(gx.s * N * D);      // [Sy][M][D]
  const int64_t dp = nl2k::ceil_div(D, (int64_t)nl2k::pairwise::kGD);
  const CosGenBwd op{inv_a, inv_b};
  hipLaunchKernelGGL((nl2k::pairwise::pair_bwd_generic_kernel<CosGenBwd, false>),
                     dim3((unsigned)std::min<int64_t>(nl2k::ceil_div(N, (int64_t)kGT) * dp * gx.s,
                                                      1 << 16)),
                     dim3(256), 0, stream, A, B, dS, nullptr, nullptr, dah, nullptr, N, M, D, gx.s,
                     gx.chunk, op);
  st = nl2k::check_launch("cosine_sim_backward_f32 (generic dA)");
  if (st) return st;
  hipLaunchKernelGGL((nl2k::pairwise::pair_bwd_generic_kernel<CosGenBwd, true>),
                     dim3((unsigned)std::min<int64_t>(nl2k::ceil_div(M, (int64_t)kGT) * dp * gy.s,
                                                      1 << 16)),
                     dim3(256), 0, stream, B, A, dS, nullptr, nullptr, dbh, nullptr, N, M, D, gy.s,
                     gy.chunk, op);
  st = nl2k::check_launch("cosine_sim_backward_f32 (generic dB)");
  if (st) return st;
  hipLaunchKernelGGL(cos_project_generic_kernel, dim3(grid_for(N, 4, 1 << 16)), dim3(256), 0,
                     stream, A, inv_a, dah, gx.s, dA, N, D);
  st = nl2k::check_launch("cosine_sim_backward_f32 (generic project A)");
  if (st) return st;
  hipLaunchKernelGGL(cos_project_generic_kernel, dim3(grid_for(M, 4, 1 << 16)), dim3(256), 0,
                     stream, B, inv_b, dbh, gy.s, dB, M, D);
  return nl2k::check_launch("cosine_sim_backward_f32 (generic project B)");
}

}  // extern "C"
