// Softmax cross-entropy loss, forward and backward, fp32 logits and int64
// labels, for MI355X (gfx950).  C-ABI in include/softmax_ce.h.
//
// Reference semantics (cases/softmax_ce/reference.py:15-21):
//   lse[b]  = logsumexp_c logits[b, c]
//   loss    = mean_b (lse[b] - logits[b, labels[b]])
// and by autograd, for the upstream scalar gradient gout,
//   dlogits[b, c] = gout / B * (exp(logits[b, c] - lse[b]) - [c == labels[b]])
// (the reference kernels recompute the row max and sum in the backward and
// accumulate the loss with one atomicAdd per row,
// softmax_ce_forward.cu:14-50, softmax_ce_backward.cu:13-56).
//
// Design (HBM bound):
//  * Forward: TPR threads own a row (TPR = 16 up to C = 128, 64 up to
//    C = 1024, else 256) and
//    keep its V float4 in registers, so the row is read once; every thread
//    issues the loads of R rows before using any.  The row max, then sum
//    exp2((x - max) log2 e), reduced with DPP lane moves (plus one LDS step
//    for TPR = 256); the label's logit is loaded directly.  At most 1024
//    workgroups stride over the rows; each writes lse per row and publishes
//    one partial loss sum in a nonce-tagged slot pair (csrc/nonce_slots.h),
//    and workgroup 0 waits for all of them and adds them in a fixed order,
//    so the loss is deterministic and the forward is one launch.  Only
//    workgroup 0 waits, on workgroups that never wait.  Under graph capture
//    a fill kernel clears the slots first (replays reuse the captured
//    nonce).  (A last-arriving-
//    workgroup scheme with a shared counter measured slower: 1024 atomics on
//    one address serialise.)
//  * Backward: lse saved by the forward turns the gradient into a pure
//    streaming pass (read logits, write dlogits, no reductions).  Rows of
//    more than 1024 classes are laid out like the forward, so each row's lse
//    and label are read once; shorter rows use a flat grid-stride kernel.
//  * A label outside [0, C) makes its row's loss term and gradient NaN (the
//    reference would index out of the row; torch raises).
//  * Unaligned rows (or C % 4 != 0) of at most 32 classes take a lane each
//    in the forward.  C not a multiple of 4, misaligned rows or C > 8192 take a
//    workgroup per row in the forward (one pass with a running maximum,
//    float4 loads when aligned) and the flat backward.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "../../../csrc/common.h"
#include "../../../csrc/nonce_slots.h"
#include "softmax_ce.h"

using nl2k::f32x4;

namespace {

constexpr int kBlock = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kFwdBlocks = 1024;  // most forward workgroups (one partial loss each)
static_assert(kFwdBlocks % 256 == 0, "the loss sum reads kFwdBlocks / 256 slots per thread");
// Workspace of the forward: one nonce-tagged slot pair (16 bytes) per
// workgroup's partial loss, then an 8-byte word whose low 32 bits count
// spin-cap trips (never cleared by the library).
constexpr size_t kStatusOffset = 16 * (size_t)kFwdBlocks;
constexpr size_t kWorkspaceBytes = kStatusOffset + 8;
constexpr unsigned kSpinLimit = 1u << 24;  // hang guard for workgroup 0's wait


// Reduce N values per thread over the TPR threads that share a row (TPR = 16:
// a 16-lane row of the wave; 64: one wave; 256: the workgroup, through
// `red`, >= 4 * N floats); the results land in every thread.  MAX selects
// fmaxf, else +.
template <int TPR, int N, bool MAX>
__device__ __forceinline__ void row_reduce(float (&a)[N], float* red) {
  if constexpr (TPR == 16) {
#pragma unroll
    for (int j = 0; j < N; ++j) a[j] = MAX ? nl2k::row16_max_dpp(a[j]) : nl2k::row16_sum_dpp(a[j]);
    return;
  }
#pragma unroll
  for (int j = 0; j < N; ++j) a[j] = MAX ? nl2k::wave_max_dpp(a[j]) : nl2k::wave_sum_dpp(a[j]);
  if (TPR == 256) {
    const int wave = threadIdx.x >> 6;
    __syncthreads();  // red may still be read from the previous use
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
      for (int j = 0; j < N; ++j) red[4 * j + wave] = a[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const float* q = red + 4 * j;
      a[j] = MAX ? fmaxf(fmaxf(q[0], q[1]), fmaxf(q[2], q[3])) : (q[0] + q[1]) + (q[2] + q[3]);
    }
  }
}

// Column of the row's label, or -1 when the label is outside [0, C).
__device__ __forceinline__ int label_col(int64_t lab, int64_t C) {
  return (lab >= 0 && lab < C) ? (int)lab : -1;
}

// Rows per block step for a width class: enough rows that each thread has
// about eight float4 loads in flight before the first is used.
template <int V>
constexpr int rows_in_flight() {
  return V == 1 ? 8 : V == 2 ? 4 : 2;
}

// Workgroup 0, after its own rows: waits for the n partial losses of this
// call (slot pairs 0 .. n-1) and writes loss = (their sum, in a fixed order)
// / B.  Only this workgroup waits, and only for workgroups that never wait,
// so the wait ends whatever the residency; the spin cap (never expected)
// gives a NaN loss instead of a hang and adds 1 to the trip counter that
// follows the slots.  Thread t adds slots t + 256 j in j
// order, then the workgroup reduction: the same additions a separate
// one-workgroup kernel over the partials would make.
__device__ void sum_partials(const unsigned long long* __restrict__ slots, nl2k::slots::Key key,
                             int n, int64_t B, float* __restrict__ loss, float* red) {
  constexpr int kPer = kFwdBlocks / kBlock;
  float x[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int p = (int)threadIdx.x + j * kBlock;
    x[j] = 0.f;
    if (p < n) {
      unsigned long long w0 = nl2k::slots::load_word(slots + 2 * p);
      unsigned long long w1 = nl2k::slots::load_word(slots + 2 * p + 1);
      unsigned spins = 0;
      while (!nl2k::slots::ready(w0, w1, key)) {
        if (++spins > kSpinLimit) {
          unsigned* trips = reinterpret_cast<unsigned*>(
              const_cast<unsigned long long*>(slots) + 2 * kFwdBlocks);
          __hip_atomic_fetch_add(trips, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          w0 = key.m0 ^ (unsigned long long)__float_as_uint(NAN);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        w0 = nl2k::slots::load_word(slots + 2 * p);
        w1 = nl2k::slots::load_word(slots + 2 * p + 1);
      }
      x[j] = __uint_as_float((unsigned)nl2k::slots::decode(w0, key));
    }
  }
  float s[1] = {0.f};
#pragma unroll
  for (int j = 0; j < kPer; ++j) s[0] += (int)threadIdx.x + j * kBlock < n ? x[j] : 0.f;
  row_reduce<kBlock, 1, false>(s, red);
  if (threadIdx.x == 0) loss[0] = s[0] / (float)B;
}

// Row-cached forward.  TPR threads own a row and keep its V float4 per
// thread in registers; a block step covers R row groups of kBlock / TPR rows
// (all R rows' loads issued before any is used), block steps are strided by
// the grid.  Rows past B are clamped to B - 1 for the loads and discarded.
// Thread 0 of each row group keeps its rows' loss terms in row order; the
// workgroup's sum (groups added in a fixed order) is published in slot pair
// blockIdx.x, and workgroup 0 then adds all partials (sum_partials).
template <int TPR, int V, bool FULL>
__global__ __launch_bounds__(kBlock) void sce_fwd_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ labels,
    float* __restrict__ lse_out, unsigned long long* __restrict__ slots, nl2k::slots::Key key,
    float* __restrict__ loss, int64_t B, int C) {
  constexpr int R = rows_in_flight<V>();
  constexpr int RPB = kBlock / TPR;
  constexpr int RPI = RPB * R;
  __shared__ float red[4 * R];
  __shared__ float sacc[RPB];
  const int t = threadIdx.x % TPR;
  const int grp = threadIdx.x / TPR;
  const int C4 = C >> 2;
  float acc = 0.f;
  for (int64_t base = (int64_t)blockIdx.x * RPI; base < B; base += (int64_t)gridDim.x * RPI) {
    f32x4 v[R][V];
    int64_t lab[R];
    float xl[R];
#pragma unroll
    for (int r = 0; r < R; ++r) lab[r] = labels[min(base + r * RPB + grp, B - 1)];
    // the scheduler must not pull the label arithmetic between these loads
    // (it would wait for the labels before issuing the rows)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f32x4* xr =
          reinterpret_cast<const f32x4*>(logits + min(base + r * RPB + grp, B - 1) * C);
#pragma unroll
      for (int k = 0; k < V; ++k) v[r][k] = xr[FULL ? t + k * TPR : min(t + k * TPR, C4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    // the label's logit, addressed by the labels loaded first (column 0 for
    // an invalid label, whose term becomes NaN below)
#pragma unroll
    for (int r = 0; r < R; ++r)
      xl[r] = logits[min(base + r * RPB + grp, B - 1) * C + max(label_col(lab[r], C), 0)];
    // keep every load above any use of the row data
    __builtin_amdgcn_sched_barrier(0);
    float m[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      m[r] = -INFINITY;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const bool ok = FULL || t + k * TPR < C4;
        const f32x4 x = v[r][k];
        const float mk = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        m[r] = fmaxf(m[r], ok ? mk : -INFINITY);
      }
    }
    row_reduce<TPR, R, true>(m, red);
    float se[R];  // per row: sum of exp(x - max)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      se[r] = 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        float e4 = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) e4 += __builtin_amdgcn_exp2f((v[r][k][u] - m[r]) * kLog2e);
        se[r] += (FULL || t + k * TPR < C4) ? e4 : 0.f;
      }
    }
    row_reduce<TPR, R, false>(se, red);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = base + r * RPB + grp;
      const float lse = m[r] + __builtin_amdgcn_logf(se[r]) * kLn2;
      const float term = label_col(lab[r], C) >= 0 ? lse - xl[r] : NAN;
      const bool mine = row < B && t == 0;
      // a select, not a branch: a branch would let the compiler sink the
      // label and logit loads into it, after all the row work
      acc += mine ? term : 0.f;
      if (mine) lse_out[row] = lse;
    }
  }
  if (t == 0) sacc[grp] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float wg = 0.f;
#pragma unroll
    for (int g = 0; g < RPB; ++g) wg += sacc[g];
    nl2k::slots::publish(slots, blockIdx.x, __float_as_uint(wg), key);
  }
  if (blockIdx.x == 0) sum_partials(slots, key, (int)gridDim.x, B, loss, red);
}

// Forward for the rows the row-cached kernel does not take (C % 4 != 0,
// misaligned rows, C > 8192): a workgroup per row, one pass over it.  Each
// thread keeps a running maximum m and the sum s of exp(x - m) over its
// elements, taken in chunks of U loads issued together (float4 loads when
// VEC); a chunk that raises the maximum rescales s once.  The row maximum M
// is the workgroup's fmax of the m's and the row sum the workgroup's sum of
// s exp(m - M), both in a fixed order.  Against two passes over the row
// (the second from L2) with one float per load: 92.7 against 401 us at
// [4096, 32000], 94.0 against 478 at [1024, 128256], 77.3 against 329 at
// [2048, 50257].
template <bool VEC>
__global__ __launch_bounds__(kBlock) void sce_fwd_long_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ labels,
    float* __restrict__ lse_out, unsigned long long* __restrict__ slots, nl2k::slots::Key key,
    float* __restrict__ loss, int64_t B, int64_t C) {
  constexpr int U = VEC ? 4 : 16;  // loads per thread per chunk
  constexpr int W = VEC ? 4 : 1;   // floats per load
  __shared__ float red[4];
  float acc = 0.f;
  const int64_t n = VEC ? C / 4 : C;  // loads per row
  for (int64_t row = blockIdx.x; row < B; row += gridDim.x) {
    const float* xr = logits + row * C;
    float m = -INFINITY, s = 0.f;
    for (int64_t base = threadIdx.x; base < n; base += (int64_t)kBlock * U) {
      float v[U][W];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = min(base + (int64_t)u * kBlock, n - 1);  // clamped: no branch
        if constexpr (VEC) {
          const f32x4 q = reinterpret_cast<const f32x4*>(xr)[i];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[u][e] = q[e];
        } else {
          v[u][0] = xr[i];
        }
      }
      float cm = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = base + (int64_t)u * kBlock < n;
#pragma unroll
        for (int e = 0; e < W; ++e) cm = fmaxf(cm, ok ? v[u][e] : -INFINITY);
      }
      const float nm = fmaxf(m, cm);
      if (nm != -INFINITY) {  // nothing but -inf so far adds nothing
        float cs = 0.f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool ok = base + (int64_t)u * kBlock < n;
#pragma unroll
          for (int e = 0; e < W; ++e)
            cs += ok ? __builtin_amdgcn_exp2f((v[u][e] - nm) * kLog2e) : 0.f;
        }
        s = s * __builtin_amdgcn_exp2f((m - nm) * kLog2e) + cs;
        m = nm;
      }
    }
    float mm[1] = {m};
    row_reduce<kBlock, 1, true>(mm, red);
    const float M = mm[0];
    float ss[1] = {M == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f((m - M) * kLog2e)};
    row_reduce<kBlock, 1, false>(ss, red);
    if (threadIdx.x == 0) {
      const float lse = M + __builtin_amdgcn_logf(ss[0]) * kLn2;
      const int lab = label_col(labels[row], C);
      lse_out[row] = lse;
      acc += lab >= 0 ? lse - xr[lab] : NAN;
    }
  }
  if (threadIdx.x == 0) nl2k::slots::publish(slots, blockIdx.x, __float_as_uint(acc), key);
  if (blockIdx.x == 0) sum_partials(slots, key, (int)gridDim.x, B, loss, red);
}

// Forward for rows of at most CM <= 32 classes that are not float4 rows: a lane per
// row with its logits in registers (a wave's loads cover 64 consecutive
// rows), no cross-lane work until the workgroup's loss sum.  Each lane adds
// its rows' loss terms in row order; the workgroup sum is in a fixed order.
template <int CM>
__global__ __launch_bounds__(kBlock) void sce_fwd_lane_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ labels,
    float* __restrict__ lse_out, unsigned long long* __restrict__ slots, nl2k::slots::Key key,
    float* __restrict__ loss, int64_t B, int C) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int64_t row = (int64_t)blockIdx.x * kBlock + threadIdx.x; row < B;
       row += (int64_t)gridDim.x * kBlock) {
    const float* xr = logits + row * C;
    const int64_t lab64 = labels[row];
    float v[CM];
#pragma unroll
    for (int c = 0; c < CM; ++c) v[c] = xr[min(c, C - 1)];  // clamped: no branch
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CM; ++c) m = fmaxf(m, c < C ? v[c] : -INFINITY);
    float se = 0.f;
#pragma unroll
    for (int c = 0; c < CM; ++c) se += c < C ? __builtin_amdgcn_exp2f((v[c] - m) * kLog2e) : 0.f;
    const float lse = m + __builtin_amdgcn_logf(se) * kLn2;
    const int lab = label_col(lab64, C);
    float xl = 0.f;
#pragma unroll
    for (int c = 0; c < CM; ++c) xl = c == lab ? v[c] : xl;
    lse_out[row] = lse;
    acc += lab >= 0 ? lse - xl : NAN;
  }
  float a[1] = {acc};
  row_reduce<kBlock, 1, false>(a, red);
  if (threadIdx.x == 0) nl2k::slots::publish(slots, blockIdx.x, __float_as_uint(a[0]), key);
  if (blockIdx.x == 0) sum_partials(slots, key, (int)gridDim.x, B, loss, red);
}

// Row-cached backward, laid out like the forward: TPR threads per row, V
// float4 per thread, R rows' loads issued before any is used.  Per row,
// scale = gout / B (NaN for an invalid label); dlogits = scale * exp(x - lse)
// everywhere, then the thread holding the label's column subtracts scale
// there.
template <int TPR, int V, bool FULL>
__global__ __launch_bounds__(kBlock) void sce_bwd_rows_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ labels,
    const float* __restrict__ lse, const float* __restrict__ gout,
    float* __restrict__ dlogits, int64_t B, int C) {
  constexpr int R = rows_in_flight<V>();
  constexpr int RPB = kBlock / TPR;
  constexpr int RPI = RPB * R;
  const int t = threadIdx.x % TPR;
  const int grp = threadIdx.x / TPR;
  const int C4 = C >> 2;
  const float g = gout[0] / (float)B;
  for (int64_t base = (int64_t)blockIdx.x * RPI; base < B; base += (int64_t)gridDim.x * RPI) {
    f32x4 v[R][V];
    int64_t lab[R];
    float l[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = min(base + r * RPB + grp, B - 1);
      lab[r] = labels[row];
      l[r] = lse[row];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f32x4* xr =
          reinterpret_cast<const f32x4*>(logits + min(base + r * RPB + grp, B - 1) * C);
#pragma unroll
      for (int k = 0; k < V; ++k) v[r][k] = xr[FULL ? t + k * TPR : min(t + k * TPR, C4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    // Rows past B were loaded as row B - 1, so their results are row B - 1's,
    // bit for bit: they are stored there again (identical values from the
    // same instructions) rather than behind a branch, which would let the
    // compiler sink the loads of the last rows into it.
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t row = min(base + r * RPB + grp, B - 1);
      const int lc = label_col(lab[r], C);
      const float scale = lc >= 0 ? g : NAN;
      f32x4* dr = reinterpret_cast<f32x4*>(dlogits + row * C);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        // columns past the row were loaded as its last float4: the same
        // holds for them (their results are the last float4's, stored again)
        const int c = FULL ? t + k * TPR : min(t + k * TPR, C4 - 1);
        // scale at the label's column (never for lc = -1), else 0
        const float hit = c == (lc >> 2) ? scale : 0.f;
        f32x4 o;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          o[u] = fmaf(scale, __builtin_amdgcn_exp2f((v[r][k][u] - l[r]) * kLog2e),
                      u == (lc & 3) ? -hit : 0.f);
        dr[c] = o;
      }
    }
  }
}

// Flat backward for the shapes the row-cached kernel does not take:
// dlogits = gout / B * (exp(x - lse) - onehot); VEC: C % 4 == 0 and aligned
// rows, one float4 per thread step.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void sce_bwd_kernel(
    const float* __restrict__ logits, const int64_t* __restrict__ labels,
    const float* __restrict__ lse, const float* __restrict__ gout,
    float* __restrict__ dlogits, int64_t B, int64_t C) {
  const float scale = gout[0] / (float)B;
  const int64_t W = VEC ? C / 4 : C;
  const int64_t n = B * W;
  for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * kBlock) {
    const int64_t row = e / W;
    const int64_t c0 = (e - row * W) * (VEC ? 4 : 1);
    const float l = lse[row];
    const int lab = label_col(labels[row], C);
    const float bad = lab >= 0 ? 0.f : NAN;
    if (VEC) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(logits + row * C + c0);
      f32x4 o;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        o[u] = scale * (__builtin_amdgcn_exp2f((x[u] - l) * kLog2e) -
                        (c0 + u == lab ? 1.f : 0.f)) + bad;
      *reinterpret_cast<f32x4*>(dlogits + row * C + c0) = o;
    } else {
      const float x = logits[row * C + c0];
      dlogits[row * C + c0] =
          scale * (__builtin_amdgcn_exp2f((x - l) * kLog2e) - (c0 == lab ? 1.f : 0.f)) + bad;
    }
  }
}

// ----------------------------------------------------------------- planning
struct FwdPlan {
  bool cached = false;  // row-cached kernel
  int lane_cm = 0;      // > 0: lane-per-row kernel for rows of at most lane_cm classes
  bool vec = false;     // long-row kernel: float4 loads
  int tpr = 64, v = 4;
  unsigned blocks = 1;  // forward workgroups, one partial loss each
};

FwdPlan plan_forward(int64_t B, int64_t C, bool aligned) {
  FwdPlan p;
  int64_t rows_per_step = 1;
  if (C <= 32 && !(aligned && C % 4 == 0)) {
    p.lane_cm = C <= 8 ? 8 : C <= 16 ? 16 : 32;
    rows_per_step = kBlock;
  } else if (aligned && C % 4 == 0 && C <= 8192) {
    p.cached = true;
    const int64_t c4 = C / 4;
    if (c4 <= 32) { p.tpr = 16; p.v = c4 <= 16 ? 1 : 2; }
    else if (c4 <= 64) { p.tpr = 64; p.v = 1; }
    else if (c4 <= 256) { p.tpr = 64; p.v = 4; }
    else { p.tpr = 256; p.v = c4 <= 512 ? 2 : c4 <= 1024 ? 4 : 8; }
    const int r = p.v == 1 ? rows_in_flight<1>() : p.v == 2 ? rows_in_flight<2>()
                                                            : rows_in_flight<4>();
    rows_per_step = (kBlock / p.tpr) * r;
  } else {
    p.vec = aligned && C % 4 == 0;
  }
  // B == 0 still runs one workgroup: its partial is 0 and its loss sum
  // writes loss = 0 / 0 = NaN (the mean of no terms, as torch's mean of an
  // empty tensor)
  p.blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(kFwdBlocks,
                                                             nl2k::ceil_div(B, rows_per_step)));
  return p;
}

int validate(int64_t B, int64_t C, const char* who) {
  if (B < 0 || C < 1)
    return nl2k::fail(NL2K_ERR_SHAPE, "%s: need B >= 0 and C >= 1 (got B=%lld C=%lld)", who,
                      (long long)B, (long long)C);
  if (B > INT32_MAX || C > INT32_MAX || B > INT64_MAX / C)
    return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: sizes too large (B=%lld C=%lld)", who,
                      (long long)B, (long long)C);
  return NL2K_SUCCESS;
}

}  // namespace

extern "C" {

const char* softmax_ce_last_error(void) { return nl2k::error_slot().text; }

size_t softmax_ce_forward_workspace_bytes(int64_t B, int64_t C) {
  if (validate(B, C, "softmax_ce_forward_workspace_bytes")) return 0;
  return kWorkspaceBytes;
}

size_t softmax_ce_status_offset(void) { return kStatusOffset; }

int softmax_ce_forward_f32(const float* logits, const int64_t* labels, float* loss, float* lse,
                           int64_t B, int64_t C, void* workspace, size_t workspace_bytes,
                           hipStream_t stream) {
  const char* who = "softmax_ce_forward_f32";
  int st = validate(B, C, who);
  if (st) return st;
  if (!loss || (B > 0 && (!logits || !labels || !lse)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (!workspace || workspace_bytes < kWorkspaceBytes)
    return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                      kWorkspaceBytes, workspace ? workspace_bytes : (size_t)0);
  if (reinterpret_cast<uintptr_t>(workspace) % 8 != 0)
    return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 8-byte aligned", who);
  unsigned long long* slots = static_cast<unsigned long long*>(workspace);
  const nl2k::slots::Key key = nl2k::slots::next_key();
  const FwdPlan p = plan_forward(B, C, nl2k::aligned16(logits));
  const dim3 grid(p.blocks);
  hipError_t qe = hipSuccess;
  const bool cap = nl2k::slots::capturing(stream, &qe);
  if (qe != hipSuccess) return nl2k::check_hip(qe, "hipStreamIsCapturing");
  if (cap) nl2k::slots::clear_async(slots, 2 * (int64_t)p.blocks, stream);
  if (p.cached && B > 0) {
#define SCE_FWD(TPR, V)                                                                        \
  do {                                                                                         \
    if (C / 4 == (TPR) * (V))                                                                  \
      hipLaunchKernelGGL((sce_fwd_kernel<TPR, V, true>), grid, dim3(kBlock), 0, stream, logits, \
                         labels, lse, slots, key, loss, B, (int)C);                            \
    else                                                                                       \
      hipLaunchKernelGGL((sce_fwd_kernel<TPR, V, false>), grid, dim3(kBlock), 0, stream,       \
                         logits, labels, lse, slots, key, loss, B, (int)C);                    \
  } while (0)
    if (p.tpr == 16 && p.v == 1) SCE_FWD(16, 1);
    else if (p.tpr == 16) SCE_FWD(16, 2);
    else if (p.tpr == 64 && p.v == 1) SCE_FWD(64, 1);
    else if (p.tpr == 64) SCE_FWD(64, 4);
    else if (p.v == 2) SCE_FWD(256, 2);
    else if (p.v == 4) SCE_FWD(256, 4);
    else SCE_FWD(256, 8);
#undef SCE_FWD
  } else if (p.lane_cm == 8) {
    hipLaunchKernelGGL(sce_fwd_lane_kernel<8>, grid, dim3(kBlock), 0, stream, logits, labels, lse,
                       slots, key, loss, B, (int)C);
  } else if (p.lane_cm == 16) {
    hipLaunchKernelGGL(sce_fwd_lane_kernel<16>, grid, dim3(kBlock), 0, stream, logits, labels,
                       lse, slots, key, loss, B, (int)C);
  } else if (p.lane_cm == 32) {
    hipLaunchKernelGGL(sce_fwd_lane_kernel<32>, grid, dim3(kBlock), 0, stream, logits, labels,
                       lse, slots, key, loss, B, (int)C);
  } else if (p.vec) {
    hipLaunchKernelGGL(sce_fwd_long_kernel<true>, grid, dim3(kBlock), 0, stream, logits, labels,
                       lse, slots, key, loss, B, C);
  } else {
    hipLaunchKernelGGL(sce_fwd_long_kernel<false>, grid, dim3(kBlock), 0, stream, logits, labels,
                       lse, slots, key, loss, B, C);
  }
  return nl2k::check_launch(who);
}

int softmax_ce_backward_f32(const float* logits, const int64_t* labels, const float* lse,
                            const float* gout, float* dlogits, int64_t B, int64_t C,
                            hipStream_t stream) {
  const char* who = "softmax_ce_backward_f32";
  int st = validate(B, C, who);
  if (st) return st;
  if (B == 0) return nl2k::succeed();
  if (!logits || !labels || !lse || !gout || !dlogits)
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  const bool aligned = nl2k::aligned16(logits) && nl2k::aligned16(dlogits);
  const FwdPlan p = plan_forward(B, C, aligned);
  // Rows of more than 1024 classes use the row kernel; shorter ones, whose
  // row kernel would keep a wave per row with few float4 per lane, stream
  // faster through the flat kernel (65536 x 64: 10.7 against 13.9 us).
  if (p.cached && p.tpr == 256) {
    const dim3 grid(p.blocks);
#define SCE_BWD(TPR, V)                                                                      \
  do {                                                                                       \
    if (C / 4 == (TPR) * (V))                                                                \
      hipLaunchKernelGGL((sce_bwd_rows_kernel<TPR, V, true>), grid, dim3(kBlock), 0, stream, \
                         logits, labels, lse, gout, dlogits, B, (int)C);                     \
    else                                                                                     \
      hipLaunchKernelGGL((sce_bwd_rows_kernel<TPR, V, false>), grid, dim3(kBlock), 0, stream, \
                         logits, labels, lse, gout, dlogits, B, (int)C);                     \
  } while (0)
    if (p.v == 2) SCE_BWD(256, 2);
    else if (p.v == 4) SCE_BWD(256, 4);
    else SCE_BWD(256, 8);
#undef SCE_BWD
  } else {
    const bool vec = C % 4 == 0 && aligned;
    const int64_t work = vec ? B * C / 4 : B * C;
    const unsigned grid = (unsigned)std::min<int64_t>(nl2k::ceil_div(work, kBlock), 8192);
    if (vec)
      hipLaunchKernelGGL(sce_bwd_kernel<true>, dim3(grid), dim3(kBlock), 0, stream, logits,
                         labels, lse, gout, dlogits, B, C);
    else
      hipLaunchKernelGGL(sce_bwd_kernel<false>, dim3(grid), dim3(kBlock), 0, stream, logits,
                         labels, lse, gout, dlogits, B, C);
  }
  return nl2k::check_launch(who);
}

}  // extern "C"
