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
#include "../../../csrc/pairwise_generic.h"
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
// Policies of the tiled SIMT kernels (csrc/pairwise_generic.h).
struct RbfGenFwd {
  float gamma;
  __device__ __forceinline__ float x_in(float v, int64_t) const { return v; }
  __device__ __forceinline__ float y_in(float v, int64_t) const { return v; }
  // the squared differences summed directly, as the reference kernel does
  __device__ __forceinline__ float step(float s, float x, float y) const {
    const float t = x - y;
    return fmaf(t, t, s);
  }
  __device__ __forceinline__ float out(float s) const { return expf(-gamma * s); }
};
struct RbfGenBwd {
  float neg2g;
  static constexpr bool kSums = true;
  __device__ __forceinline__ float w(const float* __restrict__ dK, const float* __restrict__ K,
                                     int64_t idx) const {
    return dK[idx] * K[idx];
  }
  template <bool TRANS>
  __device__ __forceinline__ float b_in(float v, int64_t) const {
    return v;
  }
  __device__ __forceinline__ float finish(float rs, float a, float acc) const {
    return neg2g * (rs * a - acc);
  }
};

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

// Workspace floats of the generic backward's slices (0 when neither side splits).
inline size_t generic_ws_floats(int64_t N, int64_t M, int64_t D) {
  if (N <= 0 || M <= 0) return 0;
  const nl2k::pairwise::GenericSplit gx = nl2k::pairwise::generic_split(N, M, D),
                                     gy = nl2k::pairwise::generic_split(M, N, D);
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
  using nl2k::pairwise::kGD;
  using nl2k::pairwise::kGT;
  const int64_t dp = nl2k::ceil_div(D, (int64_t)kGD);
  nl2k::pairwise::GenericSplit gx = nl2k::pairwise::generic_split(N, M, D),
                               gy = nl2k::pairwise::generic_split(M, N, D);
  const size_t gneed = generic_ws_floats(N, M, D) * sizeof(float);
  float* ws = static_cast<float*>(workspace);
  if (gneed == 0 || ws == nullptr || workspace_bytes < gneed ||
      reinterpret_cast<uintptr_t>(workspace) % 4 != 0) {
    gx = nl2k::pairwise::generic_whole(M);
    gy = nl2k::pairwise::generic_whole(N);
  }
  float* pxa = ws;
  float* pxs = gx.s > 1 ? pxa + gx.s * N * D : nullptr;
  float* pya = gx.s > 1 ? pxs + gx.s * N : ws;
  float* pys = gy.s > 1 ? pya + gy.s * M * D : nullptr;
  if (gx.s == 1) pxa = nullptr;
  if (gy.s == 1) pya = nullptr;
  hipLaunchKernelGGL((nl2k::pairwise::pair_bwd_generic_kernel<RbfGenBwd, false>),
                     dim3((unsigned)std::min<int64_t>(
                         nl2k::ceil_div(N, (int64_t)kGT) * dp * gx.s, 1 << 16)),
                     dim3(256), 0, stream, X, Y, dK, K, dX, pxa, pxs, N, M, D, gx.s, gx.chunk,
                     RbfGenBwd{neg2g});
  st = nl2k::check_launch(who);
  if (st) return st;
  hipLaunchKernelGGL((nl2k::pairwise::pair_bwd_generic_kernel<RbfGenBwd, true>),
                     dim3((unsigned)std::min<int64_t>(
                         nl2k::ceil_div(M, (int64_t)kGT) * dp * gy.s, 1 << 16)),
                     dim3(256), 0, stream, Y, X, dK, K, dY, pya, pys, N, M, D, gy.s, gy.chunk,
                     RbfGenBwd{neg2g});
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
  const int64_t ntiles = nl2k::ceil_div(N, (int64_t)nl2k::pairwise::kGT) *
                         nl2k::ceil_div(M, (int64_t)nl2k::pairwise::kGT);
  hipLaunchKernelGGL(nl2k::pairwise::pair_fwd_generic_kernel<RbfGenFwd>,
                     dim3((unsigned)std::min<int64_t>(ntiles, 1 << 16)), dim3(256), 0, stream, X,
                     Y, K, N, M, D, RbfGenFwd{gamma});
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
