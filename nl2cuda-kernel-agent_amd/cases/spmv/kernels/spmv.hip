// CSR sparse x dense products for MI355X (gfx950).  C-ABI in include/spmv.h.
//
// Reference semantics: cases/spmv/reference.py:8-23 (Y = index_add over the
// rows of vals * X[col_idx]); backward by autograd, i.e. dvals[p] =
// dY[row(p)] . X[col(p)] and dX = A^T dY (the reference kernels,
// spmv.cu:76-166, do the same with atomicAdd into a zeroed dX).
//
// Design.  HBM bound: the structure (row_ptr, col_idx, vals) streams once,
// X is gathered (a 4 MiB vector at the acceptance shape, so the gathers hit
// L2 / MALL), Y is written once.
//  * D == 1 (SpMV), power-law rows: rows are split between waves by the
//    merge-path coordinate f(r) = row_ptr[r] + r, so every wave gets about S
//    rows-plus-nonzeros and owns its rows outright (no cross-wave carries,
//    no atomics, deterministic).  A wave finds its first row with a
//    64-way parallel search (four dependent probes at M = 2^20), then walks
//    its nonzeros in steps of 256: lane l loads positions 4l..4l+3 with one
//    16-byte load of col_idx and one of vals, gathers x, and finds each
//    position's row by binary search over the next 256 row starts staged in
//    a wave-private LDS slice.  Per step: a serial sum over each lane's four
//    products by row, a wave64 segmented inclusive scan (key = row) of the
//    lanes' trailing partial sums, and every row that ends inside the step
//    is written once; the row still open at the end of the step is carried
//    in registers.  Empty rows are written as 0 by whoever sees the gap.
//  * D == 1 backward: the same walk gives each position its row; the wave
//    writes dvals with 16-byte stores and adds vals * dy into dX with fp32
//    atomics (dX zeroed first by a fill kernel).
//  * D > 1 (SpMM): L lanes per row (L = 4, 16 or 64), float4 columns when
//    D % 4 == 0 and X / Y are 16-byte aligned; the lanes of a row share each
//    (col, val) load and read the X row coalesced.  Backward: per nonzero a
//    group reduction for dvals and per-element atomics for dX.
#include <algorithm>
#include <cstdint>

#include "../../../csrc/common.h"
#include "spmv.h"

using nl2k::f32x4;

namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef long long i64x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kPer = 4;                 // positions per lane per step
constexpr int kStep = 64 * kPer;        // positions per wave step
constexpr int kBnd = 256;               // row starts staged per step
constexpr int64_t kWaveItems = 4096;    // rows + nonzeros per wave (D == 1)

template <typename I>
__device__ __forceinline__ int64_t ld_ptr(const I* __restrict__ ptr, int64_t r, int64_t nnz) {
  const int64_t v = (int64_t)ptr[r];
  return v < 0 ? 0 : (v > nnz ? nnz : v);
}

template <typename I>
__device__ __forceinline__ int64_t ld_col(const I* __restrict__ col, int64_t p, int64_t K) {
  const int64_t c = (int64_t)col[p];
  return c < 0 ? 0 : (c >= K ? K - 1 : c);
}

__device__ __forceinline__ int lane_count(bool pred) { return __popcll(__ballot(pred)); }

// First r in [0, M] with row_ptr[r] + r >= target (wave-uniform result).
template <typename I>
__device__ int64_t rows_lower_bound(const I* __restrict__ ptr, int64_t M, int64_t nnz,
                                    int64_t target, int lane) {
  int64_t lo = 0, hi = M;
  while (hi - lo > 63) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t probe = min(hi, lo + (int64_t)lane * step);
    const int c = lane_count(ld_ptr(ptr, probe, nnz) + probe < target);
    const int64_t nlo = c > 0 ? min(hi, lo + (int64_t)(c - 1) * step) + 1 : lo;
    const int64_t nhi = c < 64 ? min(hi, lo + (int64_t)c * step) : hi;
    lo = min(nlo, nhi);
    hi = nhi;
  }
  const int64_t probe = min(hi, lo + lane);
  const int c = lane_count(lo + lane <= hi && ld_ptr(ptr, probe, nnz) + probe < target);
  return min(lo + c, M);
}

// Loads the four col / vals entries of positions p..p+3 (p % 4 == 0 when
// VEC); in[j] tells whether position p + j lies in [lo, hi) (entries outside
// read as column 0 / value 0 and must not be used).
template <typename I, bool VEC>
__device__ __forceinline__ void load_quad(const I* __restrict__ col, const float* __restrict__ vals,
                                          int64_t p, int64_t lo, int64_t hi, int64_t nnz,
                                          int64_t K, int64_t (&c)[4], float (&v)[4],
                                          bool (&in)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) in[j] = p + j >= lo && p + j < hi;
  if (VEC && p + 3 < nnz && p >= 0) {
    f32x4 vv = *reinterpret_cast<const f32x4*>(vals + p);
    int64_t cc[4];
    if constexpr (sizeof(I) == 4) {
      const i32x4_t ci = *reinterpret_cast<const i32x4_t*>(col + p);
#pragma unroll
      for (int j = 0; j < 4; ++j) cc[j] = ci[j];
    } else {
      const i64x2_t c0 = *reinterpret_cast<const i64x2_t*>(col + p);
      const i64x2_t c1 = *reinterpret_cast<const i64x2_t*>(col + p + 2);
      cc[0] = c0[0]; cc[1] = c0[1]; cc[2] = c1[0]; cc[3] = c1[1];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = in[j] ? (cc[j] < 0 ? 0 : (cc[j] >= K ? K - 1 : cc[j])) : 0;
      v[j] = in[j] ? vv[j] : 0.f;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t q = p + j;
      const int64_t qc = q < 0 ? 0 : (q >= nnz ? nnz - 1 : q);
      const int64_t cj = nnz > 0 ? ld_col(col, qc, K) : 0;
      const float vj = nnz > 0 ? vals[qc] : 0.f;
      c[j] = in[j] ? cj : 0;
      v[j] = in[j] ? vj : 0.f;
    }
  }
}

// One wave's row range and the state of its walk over the nonzeros.
struct Walk {
  int64_t r0, r1;       // owned rows [r0, r1)
  int64_t b;            // row_ptr[r1]
  int64_t pos;          // first unprocessed nonzero
  int64_t carry_row;    // row still open (its nonzeros before pos are summed)
};

template <typename I>
__device__ __forceinline__ bool walk_begin(const I* __restrict__ ptr, int64_t M, int64_t nnz,
                                           int64_t w, int64_t n_waves, int lane, Walk& s) {
  s.r0 = w == 0 ? 0 : rows_lower_bound(ptr, M, nnz, w * kWaveItems, lane);
  s.r1 = w == n_waves - 1 ? M : rows_lower_bound(ptr, M, nnz, (w + 1) * kWaveItems, lane);
  if (s.r1 <= s.r0) return false;
  s.pos = ld_ptr(ptr, s.r0, nnz);
  s.b = max(s.pos, ld_ptr(ptr, s.r1, nnz));
  s.carry_row = s.r0;
  return true;
}

// Stages the starts of rows carry_row + 1 .. carry_row + kBnd relative to
// pos (clamped to [-1, kStep + 1]; rows >= r1 start at b) into `bnd` and
// returns the absolute start of row carry_row + kBnd.
template <typename I>
__device__ __forceinline__ int64_t stage_bounds(const I* __restrict__ ptr, int64_t nnz,
                                                const Walk& s, int lane, int* bnd) {
  int64_t last = 0;
#pragma unroll
  for (int i = 0; i < kBnd / 64; ++i) {
    const int k = lane + 64 * i;
    const int64_t r = s.carry_row + 1 + k;
    const int64_t v = r < s.r1 ? ld_ptr(ptr, r, nnz) : s.b;
    const int64_t rel = v - s.pos;
    bnd[k] = (int)(rel < -1 ? -1 : (rel > kStep + 1 ? kStep + 1 : rel));
    last = v;
  }
  __builtin_amdgcn_wave_barrier();
  const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)(uint64_t)last, 63);
  const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)((uint64_t)last >> 32), 63);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Rows of this lane's four positions q0..q0+3, each clamped into
// [pos, step_end - 1]: carry_row + #{k : bnd[k] <= q - pos}.
__device__ __forceinline__ void position_rows(const int* bnd, int64_t carry_row, int off0,
                                              int off_max, int64_t (&rid)[4]) {
  int off = max(0, min(off0, off_max));
  int idx = 0;
#pragma unroll
  for (int s = kBnd / 2; s >= 1; s >>= 1)
    if (bnd[idx + s - 1] <= off) idx += s;
  rid[0] = carry_row + idx;
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    off = max(0, min(off0 + j, off_max));
    while (idx < kBnd - 1 && bnd[idx] <= off) ++idx;
    rid[j] = carry_row + idx;
  }
}

// ------------------------------------------------------------ D == 1 forward
template <typename I, bool VEC>
__global__ __launch_bounds__(kThreads) void spmv_d1_fwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ x, float* __restrict__ y, int64_t M, int64_t K, int64_t nnz,
    int64_t n_waves) {
  __shared__ int bnd_s[kThreads / 64][kBnd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t w = (int64_t)blockIdx.x * (kThreads / 64) + wave;
  if (w >= n_waves) return;  // wave-uniform; the kernel has no workgroup barrier
  int* bnd = bnd_s[wave];
  Walk s;
  if (!walk_begin(ptr, M, nnz, w, n_waves, lane, s)) return;
  float carry_val = 0.f;

  while (s.pos < s.b) {
    const int64_t last = stage_bounds(ptr, nnz, s, lane, bnd);
    if (last <= s.pos) {
      // kBnd or more rows start at or before pos: all but carry_row are empty.
      if (lane == 0) y[s.carry_row] = carry_val;
      for (int k = lane; k < kBnd - 1; k += 64) y[s.carry_row + 1 + k] = 0.f;
      s.carry_row += kBnd;
      carry_val = 0.f;
      __builtin_amdgcn_wave_barrier();
      continue;
    }
    const int64_t base = s.pos & ~(int64_t)3;
    const int64_t step_end = min(min(base + kStep, s.b), last);
    const int64_t q0 = base + kPer * lane;
    int64_t c[4];
    float v[4];
    bool in[4];
    load_quad<I, VEC>(col, vals, q0, s.pos, step_end, nnz, K, c, v, in);
    int64_t rid[4];
    position_rows(bnd, s.carry_row, (int)(q0 - s.pos), (int)(step_end - 1 - s.pos), rid);
    float pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xv = x[c[j]];
      pr[j] = in[j] ? v[j] * xv : 0.f;
    }

    // Lane-local segments: first (kf, sf), last (kl, sl); middle rows are
    // complete and written here, as are empty rows in the gaps.
    int64_t cur = rid[0];
    float acc = pr[0];
    int64_t kf = cur;
    float sf = 0.f;
    bool single = true;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      if (rid[j] == cur) {
        acc += pr[j];
      } else {
        if (single) {
          sf = acc;
          single = false;
        } else {
          y[cur] = acc;
        }
        for (int64_t r = cur + 1; r < rid[j]; ++r) y[r] = 0.f;
        cur = rid[j];
        acc = pr[j];
      }
    }
    const int64_t kl = cur;
    const float sl = acc;
    if (single) sf = acc;

    // Segmented inclusive scan of sl over lanes, key kl (keys are sorted).
    float T = sl;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float tu = __shfl_up(T, d, 64);
      const int64_t ku = __shfl_up(kl, d, 64);
      if (lane >= d && ku == kl) T += tu;
    }
    const int64_t prev_k = __shfl_up(kl, 1, 64);
    const float prev_T = __shfl_up(T, 1, 64);
    const int64_t next_kf = __shfl_down(kf, 1, 64);
    const int64_t carry_row = s.carry_row;

    if (kf != kl) {  // the lane's first row ends inside the lane
      float tot = sf;
      if (lane > 0 && prev_k == kf) tot += prev_T;
      if (kf == carry_row) tot += carry_val;
      y[kf] = tot;
    }
    const int64_t gap_lo = lane > 0 ? prev_k : carry_row;
    for (int64_t r = gap_lo + 1; r < kf; ++r) y[r] = 0.f;
    if (lane < 63 && next_kf != kl) y[kl] = kl == carry_row ? T + carry_val : T;
    if (lane == 0 && kf != carry_row) y[carry_row] = carry_val;

    const int64_t new_row = __shfl(kl, 63, 64);
    const float new_T = __shfl(T, 63, 64);
    carry_val = new_row == carry_row ? new_T + carry_val : new_T;
    s.carry_row = new_row;
    s.pos = step_end;
    __builtin_amdgcn_wave_barrier();  // bnd is restaged next step
  }
  if (lane == 0) y[s.carry_row] = carry_val;
  for (int64_t r = s.carry_row + 1 + lane; r < s.r1; r += 64) y[r] = 0.f;
}

// ----------------------------------------------------------- D == 1 backward
template <typename I, bool VEC>
__global__ __launch_bounds__(kThreads) void spmv_d1_bwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ x, const float* __restrict__ dy, float* __restrict__ dvals,
    float* __restrict__ dx, int64_t M, int64_t K, int64_t nnz, int64_t n_waves) {
  __shared__ int bnd_s[kThreads / 64][kBnd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t w = (int64_t)blockIdx.x * (kThreads / 64) + wave;
  if (w >= n_waves) return;
  int* bnd = bnd_s[wave];
  Walk s;
  if (!walk_begin(ptr, M, nnz, w, n_waves, lane, s)) return;

  while (s.pos < s.b) {
    const int64_t last = stage_bounds(ptr, nnz, s, lane, bnd);
    if (last <= s.pos) {
      s.carry_row += kBnd;
      __builtin_amdgcn_wave_barrier();
      continue;
    }
    const int64_t base = s.pos & ~(int64_t)3;
    const int64_t step_end = min(min(base + kStep, s.b), last);
    const int64_t q0 = base + kPer * lane;
    int64_t c[4];
    float v[4];
    bool in[4];
    load_quad<I, VEC>(col, vals, q0, s.pos, step_end, nnz, K, c, v, in);
    int64_t rid[4];
    position_rows(bnd, s.carry_row, (int)(q0 - s.pos), (int)(step_end - 1 - s.pos), rid);
    float g[4], dv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      g[j] = dy[rid[j]];
      dv[j] = g[j] * x[c[j]];
    }
    const bool full = in[0] && in[3];
    if (dvals) {
      if (VEC && full) {
        *reinterpret_cast<f32x4*>(dvals + q0) = f32x4{dv[0], dv[1], dv[2], dv[3]};
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (in[j]) dvals[q0 + j] = dv[j];
      }
    }
    if (dx) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (in[j])
          __hip_atomic_fetch_add(dx + c[j], v[j] * g[j], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
    s.carry_row = __shfl(rid[3], 63, 64);
    s.pos = step_end;
    __builtin_amdgcn_wave_barrier();
  }
}

// ------------------------------------------------------------------ D > 1
template <bool VEC>
struct Lanes;
template <>
struct Lanes<true> {
  using T = f32x4;
  static constexpr int W = 4;
  __device__ static T load(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
  __device__ static void store(float* p, T v) { *reinterpret_cast<f32x4*>(p) = v; }
  __device__ static T zero() { return f32x4{0.f, 0.f, 0.f, 0.f}; }
  __device__ static float dot(T a, T b) { return (a[0] * b[0] + a[1] * b[1]) + (a[2] * b[2] + a[3] * b[3]); }
};
template <>
struct Lanes<false> {
  using T = float;
  static constexpr int W = 1;
  __device__ static T load(const float* p) { return *p; }
  __device__ static void store(float* p, T v) { *p = v; }
  __device__ static T zero() { return 0.f; }
  __device__ static float dot(T a, T b) { return a * b; }
};

// L lanes per row; each lane owns W consecutive columns per pass.
template <typename I, int L, bool VEC>
__global__ __launch_bounds__(kThreads) void spmm_fwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ X, float* __restrict__ Y, int64_t M, int64_t K, int64_t D,
    int64_t nnz) {
  using V = Lanes<VEC>;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / L) + threadIdx.x / L;
  const int gl = threadIdx.x % L;
  if (row >= M) return;
  const int64_t s = ld_ptr(ptr, row, nnz), e = max(s, ld_ptr(ptr, row + 1, nnz));
  for (int64_t d0 = 0; d0 < D; d0 += (int64_t)L * V::W) {
    const int64_t d = d0 + (int64_t)gl * V::W;
    const bool active = d < D;
    const int64_t dc = active ? d : 0;
    typename V::T acc = V::zero();
    int64_t p = s;
    for (; p + 4 <= e; p += 4) {
      int64_t cc[4];
      float vv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        cc[u] = ld_col(col, p + u, K);
        vv[u] = vals[p + u];
      }
      typename V::T xs[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) xs[u] = V::load(X + cc[u] * D + dc);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc += vv[u] * xs[u];
    }
    for (; p < e; ++p) acc += vals[p] * V::load(X + ld_col(col, p, K) * D + dc);
    if (active) V::store(Y + row * D + d, acc);
  }
}

template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <typename I, int L, bool VEC>
__global__ __launch_bounds__(kThreads) void spmm_bwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ X, const float* __restrict__ dY, float* __restrict__ dvals,
    float* __restrict__ dX, int64_t M, int64_t K, int64_t D, int64_t nnz) {
  using V = Lanes<VEC>;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / L) + threadIdx.x / L;
  const int gl = threadIdx.x % L;
  if (row >= M) return;  // whole groups exit together (L divides 64)
  const int64_t s = ld_ptr(ptr, row, nnz), e = max(s, ld_ptr(ptr, row + 1, nnz));
  for (int64_t p = s; p < e; ++p) {
    const int64_t c = ld_col(col, p, K);
    const float v = vals[p];
    float dot = 0.f;
    for (int64_t d0 = 0; d0 < D; d0 += (int64_t)L * V::W) {
      const int64_t d = d0 + (int64_t)gl * V::W;
      if (d < D) {
        const typename V::T g = V::load(dY + row * D + d);
        dot += V::dot(g, V::load(X + c * D + d));
        if (dX) {
          if constexpr (VEC) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
              __hip_atomic_fetch_add(dX + c * D + d + u, v * g[u], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
          } else {
            __hip_atomic_fetch_add(dX + c * D + d, v * g, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
    dot = group_sum<L>(dot);
    if (dvals && gl == 0) dvals[p] = dot;
  }
}

__global__ __launch_bounds__(kThreads) void spmv_fill_zero_kernel(float* __restrict__ a,
                                                                   int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    a[i] = 0.f;
}

// ----------------------------------------------------------------- host side
int validate(int64_t M, int64_t K, int64_t D, int64_t nnz, int64_t index_max, const char* who) {
  if (M < 0 || K < 1 || D < 1 || nnz < 0)
    return nl2k::fail(NL2K_ERR_SHAPE,
                      "%s: need M >= 0, K >= 1, D >= 1, nnz >= 0 (got M=%lld K=%lld D=%lld "
                      "nnz=%lld)",
                      who, (long long)M, (long long)K, (long long)D, (long long)nnz);
  if (M > INT32_MAX || K > INT32_MAX || D > INT32_MAX || nnz > index_max ||
      M > INT64_MAX / D || K > INT64_MAX / D || nnz > INT64_MAX - M)
    return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: sizes too large for the index type", who);
  return NL2K_SUCCESS;
}

int lanes_for(int64_t D, bool vec) {
  const int64_t units = vec ? D / 4 : D;
  return units <= 4 ? 4 : (units <= 16 ? 16 : 64);
}

template <typename I>
int forward(const I* ptr, const I* col, const float* vals, const float* X, float* Y, int64_t M,
            int64_t K, int64_t D, int64_t nnz, hipStream_t stream, const char* who) {
  const int64_t imax = sizeof(I) == 4 ? INT32_MAX : INT64_MAX / 2;
  int st = validate(M, K, D, nnz, imax, who);
  if (st) return st;
  if (M == 0) return nl2k::succeed();
  if (!ptr || !X || !Y || (nnz > 0 && (!col || !vals)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (D == 1) {
    const int64_t n_waves = std::max<int64_t>(1, nl2k::ceil_div(nnz + M, kWaveItems));
    const int64_t blocks = nl2k::ceil_div(n_waves, kThreads / 64);
    if (blocks > INT32_MAX) return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: too many rows", who);
    const bool vec = nl2k::aligned16(col) && nl2k::aligned16(vals);
    if (vec)
      hipLaunchKernelGGL((spmv_d1_fwd_kernel<I, true>), dim3((unsigned)blocks), dim3(kThreads), 0,
                         stream, ptr, col, vals, X, Y, M, K, nnz, n_waves);
    else
      hipLaunchKernelGGL((spmv_d1_fwd_kernel<I, false>), dim3((unsigned)blocks), dim3(kThreads),
                         0, stream, ptr, col, vals, X, Y, M, K, nnz, n_waves);
    return nl2k::check_launch(who);
  }
  const bool vec = D % 4 == 0 && nl2k::aligned16(X) && nl2k::aligned16(Y);
  const int L = lanes_for(D, vec);
  const int64_t blocks = nl2k::ceil_div(M, kThreads / L);
  const dim3 grid((unsigned)blocks), block(kThreads);
#define SPMM_FWD(LL, VV) \
  hipLaunchKernelGGL((spmm_fwd_kernel<I, LL, VV>), grid, block, 0, stream, ptr, col, vals, X, Y, M, K, D, nnz)
  if (vec) {
    if (L == 4) SPMM_FWD(4, true);
    else if (L == 16) SPMM_FWD(16, true);
    else SPMM_FWD(64, true);
  } else {
    if (L == 4) SPMM_FWD(4, false);
    else if (L == 16) SPMM_FWD(16, false);
    else SPMM_FWD(64, false);
  }
#undef SPMM_FWD
  return nl2k::check_launch(who);
}

template <typename I>
int backward(const I* ptr, const I* col, const float* vals, const float* X, const float* dY,
             float* dvals, float* dX, int64_t M, int64_t K, int64_t D, int64_t nnz,
             hipStream_t stream, const char* who) {
  const int64_t imax = sizeof(I) == 4 ? INT32_MAX : INT64_MAX / 2;
  int st = validate(M, K, D, nnz, imax, who);
  if (st) return st;
  if (!ptr || !X || (M > 0 && !dY) || (nnz > 0 && (!col || !vals)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (dX) {
    const int64_t n = K * D;
    const unsigned fb = (unsigned)std::min<int64_t>(nl2k::ceil_div(n, kThreads), 4096);
    hipLaunchKernelGGL(spmv_fill_zero_kernel, dim3(fb), dim3(kThreads), 0, stream, dX, n);
    st = nl2k::check_launch(who);
    if (st) return st;
  }
  if (M == 0 || nnz == 0 || (!dX && !dvals)) return nl2k::succeed();
  if (D == 1) {
    const int64_t n_waves = std::max<int64_t>(1, nl2k::ceil_div(nnz + M, kWaveItems));
    const int64_t blocks = nl2k::ceil_div(n_waves, kThreads / 64);
    if (blocks > INT32_MAX) return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: too many rows", who);
    const bool vec = nl2k::aligned16(col) && nl2k::aligned16(vals) &&
                     (dvals == nullptr || nl2k::aligned16(dvals));
    if (vec)
      hipLaunchKernelGGL((spmv_d1_bwd_kernel<I, true>), dim3((unsigned)blocks), dim3(kThreads), 0,
                         stream, ptr, col, vals, X, dY, dvals, dX, M, K, nnz, n_waves);
    else
      hipLaunchKernelGGL((spmv_d1_bwd_kernel<I, false>), dim3((unsigned)blocks), dim3(kThreads),
                         0, stream, ptr, col, vals, X, dY, dvals, dX, M, K, nnz, n_waves);
    return nl2k::check_launch(who);
  }
  const bool vec = D % 4 == 0 && nl2k::aligned16(X) && nl2k::aligned16(dY) &&
                   (dX == nullptr || nl2k::aligned16(dX));
  const int L = lanes_for(D, vec);
  const int64_t blocks = nl2k::ceil_div(M, kThreads / L);
  const dim3 grid((unsigned)blocks), block(kThreads);
#define SPMM_BWD(LL, VV)                                                                  \
  hipLaunchKernelGGL((spmm_bwd_kernel<I, LL, VV>), grid, block, 0, stream, ptr, col, vals, X, \
                     dY, dvals, dX, M, K, D, nnz)
  if (vec) {
    if (L == 4) SPMM_BWD(4, true);
    else if (L == 16) SPMM_BWD(16, true);
    else SPMM_BWD(64, true);
  } else {
    if (L == 4) SPMM_BWD(4, false);
    else if (L == 16) SPMM_BWD(16, false);
    else SPMM_BWD(64, false);
  }
#undef SPMM_BWD
  return nl2k::check_launch(who);
}

}  // namespace

extern "C" {

const char* spmv_last_error(void) { return nl2k::error_slot().text; }

int spmv_forward_f32_i32(const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                         const float* X, float* Y, int64_t M, int64_t K, int64_t D,
                         int64_t nnz, hipStream_t stream) {
  return forward(row_ptr, col_idx, vals, X, Y, M, K, D, nnz, stream, "spmv_forward_f32_i32");
}

int spmv_forward_f32_i64(const int64_t* row_ptr, const int64_t* col_idx, const float* vals,
                         const float* X, float* Y, int64_t M, int64_t K, int64_t D,
                         int64_t nnz, hipStream_t stream) {
  return forward(row_ptr, col_idx, vals, X, Y, M, K, D, nnz, stream, "spmv_forward_f32_i64");
}

int spmv_backward_f32_i32(const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                          const float* X, const float* dY, float* dvals, float* dX,
                          int64_t M, int64_t K, int64_t D, int64_t nnz, hipStream_t stream) {
  return backward(row_ptr, col_idx, vals, X, dY, dvals, dX, M, K, D, nnz, stream,
                  "spmv_backward_f32_i32");
}

int spmv_backward_f32_i64(const int64_t* row_ptr, const int64_t* col_idx, const float* vals,
                          const float* X, const float* dY, float* dvals, float* dX,
                          int64_t M, int64_t K, int64_t D, int64_t nnz, hipStream_t stream) {
  return backward(row_ptr, col_idx, vals, X, dY, dvals, dX, M, K, D, nnz, stream,
                  "spmv_backward_f32_i64");
}

}  // extern "C"
