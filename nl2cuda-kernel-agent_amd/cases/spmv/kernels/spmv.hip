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
//    no atomics, deterministic); S is chosen so that the launch is one round
//    of the waves the device holds at once.  Rows are found with a 64-way
//    parallel search (four dependent probes at M = 2^20) of the workgroup's
//    range, then a short one per wave inside it.  A wave then walks
//    its nonzeros in steps of 256: lane l loads positions 4l..4l+3 with one
//    16-byte load of col_idx and one of vals, gathers x, and finds each
//    position's row by binary search over the next 512 row starts staged in
//    a wave-private LDS slice.  Per step: a serial sum over each lane's four
//    products by row, a wave64 segmented inclusive scan (key = row) of the
//    lanes' trailing partial sums, and every row that ends inside the step
//    is written once; the row still open at the end of the step is carried
//    in registers.  Empty rows are written as 0 by whoever sees the gap.
//  * D == 1 backward, dvals alone: the same walk gives each position its
//    row; the wave writes dvals with 16-byte stores, in position order.
//  * D == 1 backward with dX: dX = A^T dy is a sum by column, done without
//    atomics (random 4-byte atomics or stores run at the L2's request rate,
//    ~20 G/s and ~170 G/s here, far below streaming).  A sort kernel reads
//    tiles of 8192 positions (vals and columns), finds each position's row
//    in an LDS copy of the tile's row starts, forms the contribution
//    vals[p] * dy[row(p)] (and dvals), counts the tile per column bucket
//    (2^k columns, about 256 buckets) in LDS, orders it by bucket in LDS and
//    writes it out with the low column bits beside it, plus each bucket's
//    segment offsets; one workgroup per bucket then sums its segments of
//    every tile into an LDS copy of its dX slice (compare-and-swap float
//    adds) and writes the slice once.  The order of the additions within a
//    column varies between runs, as with the reference's atomics.  Column
//    counts too large for 1024 buckets of 16384 columns fall back to
//    zero-fill plus fp32 atomics from the walk.
//  * D > 1 (SpMM): groups of L lanes cover a row's columns (L = 4, 16 or
//    64), float4 columns when D % 4 == 0 and X / Y are 16-byte aligned; the
//    lanes of a group share each (col, val) load and read the X row
//    coalesced, and G groups split a long row's nonzeros (their sums added
//    by an xor butterfly).  Backward, deterministic and without atomics:
//    with D % 4 == 0, D <= 64, 128 to 256 blocks of 256 / L columns
//    (K = 4096 at the reference default) and 16-byte aligned X / dY / dX,
//    two launches: each 1024-position chunk sorts its entries by column
//    block in LDS, then each column block gathers its segment of every chunk
//    and sums dY rows per column in registers (the spmm_b_* kernels); else,
//    up to K = 16384, a stable column-major copy of A built in the workspace
//    (chunk histograms, column offsets, an in-order scatter), then the same
//    lane-group gather per column (the spmm_t_* kernels); dvals from the
//    gather pass either way.  Beyond 16384 columns: per nonzero a group
//    reduction for dvals and per-element atomics for dX.
#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "../../../csrc/common.h"
#include "../../../csrc/nonce_slots.h"
#include "spmv.h"

using nl2k::f32x4;

namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef long long i64x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kPer = 4;                 // positions per lane per step
constexpr int kStep = 64 * kPer;        // positions per wave step
constexpr int kWin = 512;               // row starts staged per LDS window (per wave)
// Rows + nonzeros per wave (D == 1).  A walk that gathers x runs as one
// round of resident waves (gather_walk_waves), with at least kWaveItemsMin
// items each.  At 2^20 rows and 16 M nonzeros (6 waves per SIMD fit) the
// forward took 151 us with 4096 items per wave (0.7 of a round), 143 with
// 2048 (1.4 rounds: a second, part-filled round), 141 with 1456 (2 rounds)
// and 134 with 2902 (one full round).  The walks that gather nothing (dX
// by atomics only, and dvals from the forward's gathered copy) keep the
// longer fixed range (143 against 147 us; 65 against 72 us).
constexpr int64_t kWaveItemsMin = 1024;
constexpr int64_t kWaveItemsLong = 4096;

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

// First r in [lo, hi] with row_ptr[r] + wr * r >= target, given that the
// answer lies in that range (wave-uniform result): wr = 1 searches the
// merge-path coordinate, wr = 0 row starts.
template <typename I>
__device__ int64_t rows_lower_bound_in(const I* __restrict__ ptr, int64_t lo, int64_t hi,
                                       int64_t nnz, int64_t target, int lane, int64_t wr = 1) {
  const int64_t top = hi;
  while (hi - lo > 63) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t probe = min(hi, lo + (int64_t)lane * step);
    const int c = lane_count(ld_ptr(ptr, probe, nnz) + wr * probe < target);
    const int64_t nlo = c > 0 ? min(hi, lo + (int64_t)(c - 1) * step) + 1 : lo;
    const int64_t nhi = c < 64 ? min(hi, lo + (int64_t)c * step) : hi;
    lo = min(nlo, nhi);
    hi = nhi;
  }
  const int64_t probe = min(hi, lo + lane);
  const int c = lane_count(lo + lane <= hi && ld_ptr(ptr, probe, nnz) + wr * probe < target);
  return min(lo + c, top);
}

// First r in [0, M] with row_ptr[r] + wr * r >= target.
template <typename I>
__device__ int64_t rows_lower_bound(const I* __restrict__ ptr, int64_t M, int64_t nnz,
                                    int64_t target, int lane, int64_t wr = 1) {
  return rows_lower_bound_in(ptr, 0, M, nnz, target, lane, wr);
}

// The raw col_idx / vals entries of positions q0..q0+3 (q0 % 4 == 0),
// loaded without branches (a load under a branch makes the compiler wait for
// it before the branch joins, which serialises the walk).  The vector form
// reads 16 bytes of each array at q0 clamped to [0, nnz_full - 4], where
// nnz_full = nnz rounded down to a multiple of 4; a wave takes it only when
// all its positions lie below nnz_full, so no entry it uses is clamped.  The
// scalar form reads each entry at its position clamped to [0, nnz - 1].
// The vector loads are nontemporal: the structure is read once, and lines
// that do not stay in the L2 leave more of it to the gathered x (forward
// 131.0 -> 127.7 us at the acceptance shape).
template <typename I, bool VEC>
struct Quad {
  I c[4];
  float v[4];
  __device__ void issue(const I* __restrict__ col, const float* __restrict__ vals, int64_t q0,
                        int64_t nnz) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t q = max((int64_t)0, min(q0 + j, nnz - 1));
      c[j] = col[q];
      v[j] = vals[q];
    }
  }
  __device__ int64_t col_at(int j) const { return (int64_t)c[j]; }
  __device__ float val_at(int j) const { return v[j]; }
};
template <>
struct Quad<int32_t, true> {
  i32x4_t c;
  f32x4 v;
  __device__ void issue(const int32_t* __restrict__ col, const float* __restrict__ vals,
                        int64_t q0, int64_t nnz) {
    const int64_t q = max((int64_t)0, min(q0, (nnz & ~(int64_t)3) - 4));
    c = __builtin_nontemporal_load(reinterpret_cast<const i32x4_t*>(col + q));
    v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(vals + q));
  }
  __device__ int64_t col_at(int j) const { return (int64_t)c[j]; }
  __device__ float val_at(int j) const { return v[j]; }
};
template <>
struct Quad<int64_t, true> {
  i64x2_t c0, c1;
  f32x4 v;
  __device__ void issue(const int64_t* __restrict__ col, const float* __restrict__ vals,
                        int64_t q0, int64_t nnz) {
    const int64_t q = max((int64_t)0, min(q0, (nnz & ~(int64_t)3) - 4));
    c0 = __builtin_nontemporal_load(reinterpret_cast<const i64x2_t*>(col + q));
    c1 = __builtin_nontemporal_load(reinterpret_cast<const i64x2_t*>(col + q + 2));
    v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(vals + q));
  }
  __device__ int64_t col_at(int j) const { return j < 2 ? c0[j] : c1[j - 2]; }
  __device__ float val_at(int j) const { return v[j]; }
};

// Values and gathered x entries (x[col[p]], written by the forward) of
// positions q0..q0+3, for the backward's dvals without gathers; the same
// clamped branch-free loads as Quad.
template <bool VEC>
struct QuadVX {
  float v[4], x[4];
  __device__ void issue(const float* __restrict__ vals, const float* __restrict__ xg, int64_t q0,
                        int64_t nnz) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t q = max((int64_t)0, min(q0 + j, nnz - 1));
      v[j] = vals[q];
      x[j] = xg[q];
    }
  }
};
template <>
struct QuadVX<true> {
  f32x4 v, x;
  __device__ void issue(const float* __restrict__ vals, const float* __restrict__ xg, int64_t q0,
                        int64_t nnz) {
    const int64_t q = max((int64_t)0, min(q0, (nnz & ~(int64_t)3) - 4));
    v = *reinterpret_cast<const f32x4*>(vals + q);
    x = *reinterpret_cast<const f32x4*>(xg + q);
  }
};

// Columns (clamped into [0, K)) and values of positions q0..q0+3; in[j]
// tells whether q0 + j lies in [lo, hi); entries outside read as column 0,
// value 0.
template <typename Q>
__device__ __forceinline__ void quad_get(const Q& qd, int64_t K, int64_t q0, int64_t lo,
                                         int64_t hi, int64_t (&c)[4], float (&v)[4],
                                         bool (&in)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    in[j] = q0 + j >= lo && q0 + j < hi;
    const int64_t cj = qd.col_at(j);
    c[j] = in[j] ? (cj < 0 ? 0 : (cj >= K ? K - 1 : cj)) : 0;
    v[j] = in[j] ? qd.val_at(j) : 0.f;
  }
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)(uint64_t)v, l);
  const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)((uint64_t)v >> 32), l);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// One wave's row range and the state of its walk over the nonzeros.
struct Walk {
  int64_t r0, r1;       // owned rows [r0, r1)
  int64_t b;            // row_ptr[r1]: end of the owned nonzeros
  int64_t pos;          // first unprocessed nonzero
  int64_t carry_row;    // row still open (its nonzeros before pos are done)
  int64_t wr;           // LDS window: bnd[k] = start of row wr + 1 + k
  int64_t wlimit;       // start of row wr + kWin: positions below it resolve
};

// Row ranges of a workgroup's four waves: wave w owns the rows from the
// first r with row_ptr[r] + r >= w * per up to the next wave's first row.
// Wave 0 finds the workgroup's first row and wave 1 the row past its last
// one, searching all M rows; waves 1-3 then find their own first rows
// inside that range (a short search), so a workgroup makes two full
// searches instead of eight.  Every wave of the workgroup calls this (it
// holds two barriers); it returns whether the wave has work.
template <typename I>
__device__ __forceinline__ bool walk_begin(const I* __restrict__ ptr, int64_t M, int64_t nnz,
                                           int64_t n_waves, int lane, int wave,
                                           int64_t* starts, Walk& s) {
  const int64_t per = (nnz + M + n_waves - 1) / n_waves;  // items per wave
  const int64_t w0 = (int64_t)blockIdx.x * (kThreads / 64);  // < n_waves
  // starts[q] = first row of wave w0 + q (M for waves past the last)
  if (wave == 0) {
    const int64_t r = w0 == 0 ? 0 : rows_lower_bound(ptr, M, nnz, w0 * per, lane);
    if (lane == 0) starts[0] = r;
  } else if (wave == 1) {
    const int64_t wn = w0 + kThreads / 64;
    const int64_t r = wn >= n_waves ? M : rows_lower_bound(ptr, M, nnz, wn * per, lane);
    if (lane == 0) starts[kThreads / 64] = r;
  }
  __syncthreads();
  const int64_t w = w0 + wave;
  if (wave > 0) {
    const int64_t r = w >= n_waves ? M
                                   : rows_lower_bound_in(ptr, starts[0], starts[kThreads / 64], nnz,
                                                         w * per, lane);
    if (lane == 0) starts[wave] = r;
  }
  __syncthreads();
  if (w >= n_waves) return false;
  s.r0 = starts[wave];
  s.r1 = starts[wave + 1];
  if (s.r1 <= s.r0) return false;
  s.pos = ld_ptr(ptr, s.r0, nnz);
  s.b = max(s.pos, ld_ptr(ptr, s.r1, nnz));
  s.carry_row = s.r0;
  return true;
}

// Stages the starts of rows carry_row + 1 .. carry_row + kWin (absolute;
// rows >= r1 read as b) into the wave's LDS window.  The row_ptr loads are
// unconditional (row index clamped to r1 <= M).
template <typename I>
__device__ __forceinline__ void stage_window(const I* __restrict__ ptr, int64_t nnz, Walk& s,
                                             int lane, int64_t* bnd) {
  int64_t v[kWin / 64];
#pragma unroll
  for (int i = 0; i < kWin / 64; ++i) {  // all loads first, then the LDS writes
    const int64_t r = s.carry_row + 1 + lane + 64 * i;
    v[i] = (int64_t)ptr[min(r, s.r1)];
  }
  __builtin_amdgcn_wave_barrier();  // every lane is done reading the old window
  int64_t last = 0;
#pragma unroll
  for (int i = 0; i < kWin / 64; ++i) {
    const int64_t r = s.carry_row + 1 + lane + 64 * i;
    last = r < s.r1 ? min(max(v[i], (int64_t)0), nnz) : s.b;
    bnd[lane + 64 * i] = last;
  }
  __builtin_amdgcn_wave_barrier();
  s.wr = s.carry_row;
  s.wlimit = readlane64(last, 63);
}

// Rows of positions q0..q0+3, each clamped into [pos, qmax]:
// wr + #{k : bnd[k] <= q}, kept inside [r0, r1 - 1].
__device__ __forceinline__ void window_rows(const int64_t* bnd, const Walk& s, int64_t q0,
                                            int64_t qmax, int64_t (&rid)[4]) {
  int64_t q = max(s.pos, min(q0, qmax));
  int idx = 0;
#pragma unroll
  for (int st = kWin / 2; st >= 1; st >>= 1)
    if (bnd[idx + st - 1] <= q) idx += st;
  rid[0] = min(s.wr + idx, s.r1 - 1);
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    q = max(s.pos, min(q0 + j, qmax));
    while (idx < kWin - 1 && bnd[idx] <= q) ++idx;
    rid[j] = min(s.wr + idx, s.r1 - 1);
  }
}

// ------------------------------------------------------------ D == 1 forward
// SAVE: also write xg[p] = x[col[p]] (column clamped) for every position.
// Steps are aligned to multiples of kStep positions (a wave's first step
// masks the positions before its first row), so position p always sits in
// lane (p mod kStep) / 4, and a step cut short by the LDS window ends at a
// row start.  With the positions past a cut keyed as a later row (below),
// every row is summed in the same order however the rows are split between
// waves: results do not depend on the wave count, which follows the
// device's CU count and each instantiation's occupancy.
template <typename I, bool VEC, bool SAVE>
__device__ __forceinline__ void fwd_walk(const I* __restrict__ ptr, const I* __restrict__ col,
                                         const float* __restrict__ vals,
                                         const float* __restrict__ x, float* __restrict__ y,
                                         float* __restrict__ xg, int64_t K, int64_t nnz, Walk& s,
                                         int lane, int64_t* bnd) {
  float carry_val = 0.f;
  stage_window(ptr, nnz, s, lane, bnd);
  Quad<I, VEC> cur;
  if (s.pos < s.b) cur.issue(col, vals, (s.pos & ~(int64_t)(kStep - 1)) + kPer * lane, nnz);

  while (s.pos < s.b) {
    const int64_t base = s.pos & ~(int64_t)(kStep - 1);
    const int64_t want = min(base + kStep, s.b);
    if (s.wlimit < want && s.wr != s.carry_row) stage_window(ptr, nnz, s, lane, bnd);
    if (s.wlimit <= s.pos) {
      // Rows carry_row .. carry_row + kWin - 1 all end at or before pos.
      if (lane == 0) y[s.carry_row] = carry_val;
      for (int k = lane; k < kWin - 1; k += 64) y[s.carry_row + 1 + k] = 0.f;
      s.carry_row += kWin;
      carry_val = 0.f;
      continue;  // restaged next iteration (wr != carry_row)
    }
    const int64_t step_end = min(want, s.wlimit);
    const int64_t q0 = base + kPer * lane;
    int64_t c[4];
    float v[4];
    bool in[4];
    quad_get(cur, K, q0, s.pos, step_end, c, v, in);
    float xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[j] = x[c[j]];
    Quad<I, VEC> nxt;  // the next step starts at step_end
    nxt.issue(col, vals, (step_end & ~(int64_t)(kStep - 1)) + kPer * lane, nnz);
    if constexpr (SAVE) {
      // Streaming stores: the copy is read once, by the backward, and must
      // not displace x from L2.
      if (VEC && in[0] && in[3]) {
        __builtin_nontemporal_store(f32x4{xv[0], xv[1], xv[2], xv[3]},
                                    reinterpret_cast<f32x4*>(xg + q0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (in[j]) __builtin_nontemporal_store(xv[j], xg + q0 + j);
      }
    }
    int64_t rid[4];
    window_rows(bnd, s, q0, step_end - 1, rid);
    // Positions at or past step_end (a step cut short by the window or by
    // the wave's end) take a row id past the last real row: the rows in
    // between are empty, and the last real row ends where it ends, as when
    // another row follows it.  (Giving them the last real row instead would
    // read that row's sum from lane 63, in another order of additions.)
    const int64_t after = min(s.r1, s.wr + kWin);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (q0 + j >= step_end) rid[j] = after;
    float pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pr[j] = in[j] ? v[j] * xv[j] : 0.f;

    // Lane-local segments: first (kf, sf), last (kl, sl); middle rows are
    // complete and written here, as are empty rows in the gaps.
    int64_t cur_row = rid[0];
    float acc = pr[0];
    int64_t kf = cur_row;
    float sf = 0.f;
    bool single = true;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      if (rid[j] == cur_row) {
        acc += pr[j];
      } else {
        if (single) {
          sf = acc;
          single = false;
        } else {
          y[cur_row] = acc;
        }
        for (int64_t r = cur_row + 1; r < rid[j]; ++r) y[r] = 0.f;
        cur_row = rid[j];
        acc = pr[j];
      }
    }
    const int64_t kl = cur_row;
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
    cur = nxt;
  }
  // carry_row is r1 when the last step ended with positions past the end
  if (lane == 0 && s.carry_row < s.r1) y[s.carry_row] = carry_val;
  for (int64_t r = s.carry_row + 1 + lane; r < s.r1; r += 64) y[r] = 0.f;
}

template <typename I, bool VEC, bool SAVE>
__global__ __launch_bounds__(kThreads) void spmv_d1_fwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ x, float* __restrict__ y, float* __restrict__ xg, int64_t M,
    int64_t K, int64_t nnz, int64_t n_waves) {
  __shared__ int64_t bnd_s[kThreads / 64][kWin];
  __shared__ int64_t starts[kThreads / 64 + 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  Walk s;
  if (!walk_begin(ptr, M, nnz, n_waves, lane, wave, starts, s)) return;  // wave-uniform
  if constexpr (VEC) {
    if (s.b <= (nnz & ~(int64_t)3)) {
      fwd_walk<I, true, SAVE>(ptr, col, vals, x, y, xg, K, nnz, s, lane, bnd_s[wave]);
      return;
    }
  }
  fwd_walk<I, false, SAVE>(ptr, col, vals, x, y, xg, K, nnz, s, lane, bnd_s[wave]);
}

// ----------------------------------------------------------- D == 1 backward
// Outputs per instantiation: dvals (DV), and for dX either nothing (kNoDx)
// or fp32 atomics into a zeroed dx (kAtomic, the fallback beyond the bucket
// sort's column limit).
constexpr int kNoDx = 0, kAtomic = 1;

// GX: x[col[p]] comes from xg (the forward's gathered copy) instead of a
// gather, and col_idx is not read at all (MODE kNoDx only).
template <typename I, bool VEC, bool DV, int MODE, bool GX>
__device__ __forceinline__ void bwd_walk(const I* __restrict__ ptr, const I* __restrict__ col,
                                         const float* __restrict__ vals,
                                         const float* __restrict__ x,
                                         const float* __restrict__ xg,
                                         const float* __restrict__ dy, float* __restrict__ dvals,
                                         float* __restrict__ out, int64_t K, int64_t nnz,
                                         Walk& s, int lane, int64_t* bnd) {
  static_assert(!GX || MODE != kAtomic, "the gathered walk does not read columns");
  using QuadT = std::conditional_t<GX, QuadVX<VEC>, Quad<I, VEC>>;
  auto issue = [&](QuadT& qd, int64_t q) {
    if constexpr (GX)
      qd.issue(vals, xg, q, nnz);
    else
      qd.issue(col, vals, q, nnz);
  };
  stage_window(ptr, nnz, s, lane, bnd);
  QuadT cur;
  if (s.pos < s.b) issue(cur, (s.pos & ~(int64_t)3) + kPer * lane);
  while (s.pos < s.b) {
    const int64_t base = s.pos & ~(int64_t)3;
    const int64_t want = min(base + kStep, s.b);
    if (s.wlimit < want && s.wr != s.carry_row) stage_window(ptr, nnz, s, lane, bnd);
    if (s.wlimit <= s.pos) {
      s.carry_row += kWin;
      continue;
    }
    const int64_t step_end = min(want, s.wlimit);
    const int64_t q0 = base + kPer * lane;
    int64_t c[4];
    float v[4], xv[4];
    bool in[4];
    if constexpr (GX) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        in[j] = q0 + j >= s.pos && q0 + j < step_end;
        v[j] = in[j] ? cur.v[j] : 0.f;
        xv[j] = cur.x[j];
        c[j] = 0;
      }
    } else {
      quad_get(cur, K, q0, s.pos, step_end, c, v, in);
    }
    int64_t rid[4];
    window_rows(bnd, s, q0, step_end - 1, rid);
    float g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) g[j] = dy[rid[j]];
    if constexpr (DV && !GX) {
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[j] = x[c[j]];
    }
    QuadT nxt;
    issue(nxt, (step_end & ~(int64_t)3) + kPer * lane);
    const bool full = in[0] && in[3];
    if constexpr (DV) {
      if (VEC && full) {
        // nontemporal, like the sort kernel's dvals stores (dvals-only
        // walk 132.3 -> 129.8 us): dvals is not read again here
        __builtin_nontemporal_store(f32x4{g[0] * xv[0], g[1] * xv[1], g[2] * xv[2], g[3] * xv[3]},
                                    reinterpret_cast<f32x4*>(dvals + q0));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (in[j]) dvals[q0 + j] = g[j] * xv[j];
      }
    }
    if constexpr (MODE == kAtomic) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (in[j])
          __hip_atomic_fetch_add(out + c[j], v[j] * g[j], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    }
    s.carry_row = __shfl(rid[3], 63, 64);
    s.pos = step_end;
    cur = nxt;
  }
}

// `out` is dx (kAtomic).
template <typename I, bool VEC, bool DV, int MODE, bool GX>
__global__ __launch_bounds__(kThreads) void spmv_d1_bwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ x, const float* __restrict__ xg, const float* __restrict__ dy,
    float* __restrict__ dvals, float* __restrict__ out, int64_t M, int64_t K, int64_t nnz,
    int64_t n_waves) {
  __shared__ int64_t bnd_s[kThreads / 64][kWin];
  __shared__ int64_t starts[kThreads / 64 + 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  Walk s;
  if (!walk_begin(ptr, M, nnz, n_waves, lane, wave, starts, s)) return;
  if (s.pos >= s.b) return;
  if constexpr (VEC) {
    if (s.b <= (nnz & ~(int64_t)3)) {
      bwd_walk<I, true, DV, MODE, GX>(ptr, col, vals, x, xg, dy, dvals, out, K, nnz, s, lane,
                                      bnd_s[wave]);
      return;
    }
  }
  bwd_walk<I, false, DV, MODE, GX>(ptr, col, vals, x, xg, dy, dvals, out, K, nnz, s, lane,
                                   bnd_s[wave]);
}

// -------------------------------------------- D == 1 dX: bucket sort + sum
constexpr int kSortThreads = 512;
constexpr int kSortTile = 8192;                     // positions per sort workgroup
constexpr int kSortPer = kSortTile / kSortThreads;  // 16 per thread, as 4 quads
constexpr int kMaxBuckets = 1024;
constexpr int kMaxBucketCols = 16384;               // LDS floats of one bucket's sums
constexpr int kSumThreads = 1024;
constexpr int kSumWaves = kSumThreads / 64;
constexpr int kSumUnroll = 8;

// Float add into LDS through a 32-bit compare-and-swap loop.  On gfx950
// ds_add_f32 retires about one lane per three clocks per CU whatever the
// addresses; a read plus ds_cmpst_rtn_b32, retried only when another lane
// changed the word in between, runs about four times faster on scattered
// addresses.  Every failed exchange means another update succeeded, so the
// loop ends.
__device__ __forceinline__ void lds_add_f32(float* p, float v) {
  unsigned* u = reinterpret_cast<unsigned*>(p);
  unsigned old = *u;
  while (true) {
    const unsigned assumed = old;
    old = atomicCAS(u, assumed, __float_as_uint(__uint_as_float(assumed) + v));
    if (old == assumed) break;
  }
}

__device__ __forceinline__ unsigned wave_incl_scan(unsigned v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const unsigned u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}

// dx[b * cols, b * cols + cols) for bucket b: the bucket's segments of
// every tile, summed in LDS.  A wave takes 64 tiles at a time and treats
// their segments as one list (an exclusive prefix of the segment lengths in
// LDS maps list entry e to its tile), so each lane loads kSumUnroll
// independent entries per round.
//
// Workgroups go to the 8 XCDs round-robin (workgroup i to XCD i % 8), and a
// segment's first and last cache lines are shared with the neighbouring
// buckets' segments.  So each XCD takes a contiguous run of buckets: within
// a tile their segments are one contiguous stretch, whose lines that XCD's
// L2 fetches once.  (Bucket b = workgroup b put neighbours on different
// XCDs, and each boundary line was fetched twice: 2.7 times the entries'
// bytes came from HBM.)
__device__ __forceinline__ int xcd_bucket(int i, int nb) {
  const int q = nb >> 3, r = nb & 7, x = i & 7;
  return x * q + min(x, r) + (i >> 3);
}

__global__ __launch_bounds__(kSumThreads) void spmv_bucket_sum_kernel(
    const float* __restrict__ val, const uint16_t* __restrict__ lowcol,
    const int64_t* __restrict__ meta, int64_t n_tiles, int nb, int cols, int64_t K,
    int64_t nnz, float* __restrict__ dx) {
  __shared__ float acc[kMaxBucketCols];
  __shared__ int64_t s_start[kSumWaves][64];
  __shared__ int s_pre[kSumWaves][65];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = xcd_bucket((int)blockIdx.x, nb);
  for (int i = tid; i < cols; i += kSumThreads) acc[i] = 0.f;
  __syncthreads();
  const int64_t n_groups = (n_tiles + 63) / 64;
  for (int64_t grp = wave; grp < n_groups; grp += kSumWaves) {
    const int64_t t = grp * 64 + lane;
    int64_t m0 = 0, m1 = 0;
    if (t < n_tiles) {
      const int64_t* m = meta + t * (nb + 1) + b;
      m0 = min(max(m[0], (int64_t)0), nnz);
      m1 = min(max(m[1], m0), min(nnz, m0 + kSortTile));
    }
    const int len = (int)(m1 - m0);
    const int incl = (int)wave_incl_scan((unsigned)len, lane);
    s_start[wave][lane] = m0;
    s_pre[wave][lane] = incl - len;
    if (lane == 63) s_pre[wave][64] = incl;
    const int E = __shfl(incl, 63, 64);
    __builtin_amdgcn_wave_barrier();
    for (int e0 = 0; e0 < E; e0 += 64 * kSumUnroll) {
      // Positions first (LDS only), then every global load without a branch
      // between them, then the LDS additions.  Entry e lies in tile j, the
      // last with s_pre[j] <= e (a fixed six-step search, independent per
      // entry, so the entries' searches overlap).
      int64_t pp[kSumUnroll];
      bool ok[kSumUnroll];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) {
        const int e = e0 + 64 * u + lane;
        ok[u] = e < E;
        const int ee = ok[u] ? e : E - 1;
        int j = 0;
#pragma unroll
        for (int step = 32; step > 0; step >>= 1) j += s_pre[wave][j + step] <= ee ? step : 0;
        pp[u] = s_start[wave][j] + (ee - s_pre[wave][j]);
      }
      __builtin_amdgcn_sched_barrier(0);
      float v[kSumUnroll];
      unsigned c[kSumUnroll];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) {
        v[u] = val[pp[u]];
        c[u] = lowcol[pp[u]];
      }
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u)
        if (ok[u]) lds_add_f32(&acc[c[u] & (unsigned)(cols - 1)], v[u]);
    }
    __builtin_amdgcn_wave_barrier();  // s_start / s_pre are rewritten next group
  }
  __syncthreads();
  const int64_t c0 = (int64_t)b * cols;
  for (int i = tid; i < cols && c0 + i < K; i += kSumThreads) dx[c0 + i] = acc[i];
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

// A row takes G groups of L lanes.  Within a group each lane owns W
// consecutive columns per pass; group g takes the row's positions s + g,
// s + g + G, ..., and the G partial sums are added across the groups by a
// butterfly (the same bits in every group), so more waves share the
// dependent col -> X load chains of a long row.  A wave holds 64 / (L * G)
// rows; lanes of rows past M run empty, since every lane takes part in the
// butterfly.
template <int L, int G, typename T>
__device__ __forceinline__ T groups_sum(T v) {
#pragma unroll
  for (int m = L; m < L * G; m <<= 1) {
    if constexpr (std::is_same<T, float>::value) {
      v += __shfl_xor(v, m, 64);
    } else {
      T o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = __shfl_xor(v[k], m, 64);
      v += o;
    }
  }
  return v;
}

// acc += vals[p + u G] * X[col[p + u G], dc..] for u < U: every load of the
// chunk is issued before the first product.
template <int U, int G, typename V, typename I>
__device__ __forceinline__ void spmm_chunk(const I* __restrict__ col,
                                           const float* __restrict__ vals,
                                           const float* __restrict__ X, int64_t p, int64_t K,
                                           int64_t D, int64_t dc, typename V::T& acc) {
  int64_t cc[U];
  float vv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    cc[u] = ld_col(col, p + u * G, K);
    vv[u] = vals[p + u * G];
  }
  typename V::T xs[U];
#pragma unroll
  for (int u = 0; u < U; ++u) xs[u] = V::load(X + cc[u] * D + dc);
#pragma unroll
  for (int u = 0; u < U; ++u) acc += vv[u] * xs[u];
}

template <typename I, int L, int G, bool VEC>
__global__ __launch_bounds__(kThreads) void spmm_fwd_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ X, float* __restrict__ Y, int64_t M, int64_t K, int64_t D,
    int64_t nnz) {
  using V = Lanes<VEC>;
  constexpr int kRowLanes = L * G;
  static_assert(kRowLanes <= 64 && (kRowLanes & (kRowLanes - 1)) == 0, "rows inside a wave");
  const int64_t row = (int64_t)blockIdx.x * (kThreads / kRowLanes) + threadIdx.x / kRowLanes;
  const int gl = threadIdx.x % L;
  const int grp = (threadIdx.x % kRowLanes) / L;
  const bool live = row < M;
  const int64_t s = live ? ld_ptr(ptr, row, nnz) : 0;
  const int64_t e = live ? max(s, ld_ptr(ptr, row + 1, nnz)) : 0;
  for (int64_t d0 = 0; d0 < D; d0 += (int64_t)L * V::W) {
    const int64_t d = d0 + (int64_t)gl * V::W;
    const bool active = d < D;
    const int64_t dc = active ? d : 0;
    typename V::T acc = V::zero();
    // chunks of 16 entries per group (the whole group's share of a
    // reference-default row: 11.6 against 12.4 us with chunks of 4), then 4
    int64_t p = s + grp;
    for (; p + 15 * G < e; p += 16 * G) spmm_chunk<16, G, V>(col, vals, X, p, K, D, dc, acc);
    for (; p + 3 * G < e; p += 4 * G) spmm_chunk<4, G, V>(col, vals, X, p, K, D, dc, acc);
    for (; p < e; p += G) acc += vals[p] * V::load(X + ld_col(col, p, K) * D + dc);
    if constexpr (G > 1) acc = groups_sum<L, G>(acc);
    if (live && active && grp == 0) V::store(Y + row * D + d, acc);
  }
}

// Sum over each aligned group of L lanes (every lane of a group active).
// L = 4 and 16 stay inside a DPP row: quad_perm [1,0,3,2] and [2,3,0,1],
// then row_half_mirror and row_mirror; L = 64 uses cross-row shuffles.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L == 4 || L == 16) {
    v += nl2k::dpp_mov<0xB1>(v);
    v += nl2k::dpp_mov<0x4E>(v);
    if constexpr (L == 16) {
      v += nl2k::dpp_mov<0x141>(v);
      v += nl2k::dpp_mov<0x140>(v);
    }
    return v;
  } else {
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
  }
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

// ------------------------------------------------ SpMM backward dX (D > 1)
// dX = A^T dY without atomics and bitwise repeatable: a stable column-major
// copy of A is built in the workspace (its entries of column c in
// increasing position order), then each column gathers dY rows in that
// order.  Positions are cut into chunks of P (P >= 1024, a multiple of 256,
// about one chunk per CU): chunk w = positions [wP, (w+1)P), one workgroup
// per chunk in S1 and S3.
//  S1 spmm_t_hist_kernel:    H[w][c] = entries of column c in chunk w, an LDS
//                            histogram (order-free integer counts), eight
//                            column loads per thread in flight.
//  S2 spmm_t_offsets_kernel: kOffCols = 16 columns per workgroup, the chunks
//                            split over 16 thread groups (each holds up to 16
//                            chunks' counts in registers); column totals,
//                            the exclusive scan over columns (this block's
//                            prefix plus the earlier blocks' totals, passed
//                            through nonce-tagged slots, 256 slots loaded
//                            per round trip), colptr, and H rewritten in
//                            place as each chunk's first slot per column.
//  S3 spmm_t_scatter_kernel: each chunk finds every position's row (an LDS
//                            copy of the chunk's row starts, else a binary
//                            search) and walks its positions in 256-position
//                            tiles, kScatterTiles tiles' loads in flight per
//                            pass; within a tile the four waves take their
//                            slots one after another, and lanes of a wave
//                            that share a column (found through LDS tags)
//                            take consecutive slots in lane order, so the
//                            entries of every column land in position order,
//                            as one 16-byte record {row, position, value}.
//  S4 spmm_t_gather_kernel:  L lanes per column (G groups of them share a
//                            long column) sum vals * dY[row] over the
//                            column's entries in that order, 16 entries per
//                            step (and, when asked and D fits one pass,
//                            dvals[p] = dY[row] . X[c]).
constexpr int kTransposeMaxCols = 16384;  // LDS of the chunk kernels (5 B per column)
constexpr int64_t kTransposeChunk = 1024;  // positions per chunk, at least

// Loads n values of src into LDS ints, eight loads per thread in flight at
// a time (a plain loop waits for each load before its LDS write).
template <typename T>
__device__ __forceinline__ void load_to_lds(const T* __restrict__ src, int* __restrict__ dst,
                                            int64_t n) {
  constexpr int B = 8;
  for (int64_t base = 0; base < n; base += (int64_t)B * kThreads) {
    T v[B];
#pragma unroll
    for (int u = 0; u < B; ++u)
      v[u] = src[min(base + (int64_t)u * kThreads + threadIdx.x, n - 1)];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int64_t i = base + (int64_t)u * kThreads + threadIdx.x;
      if (i < n) dst[i] = (int)v[u];
    }
  }
}

// Chunk w = positions [wP, (w+1)P), one workgroup each; H is int32 [w][K].
template <typename I>
__global__ __launch_bounds__(kThreads) void spmm_t_hist_kernel(const I* __restrict__ col,
                                                               int* __restrict__ H, int64_t K,
                                                               int64_t nnz, int64_t P) {
  extern __shared__ int lds_i[];
  const int64_t w = blockIdx.x;
  for (int64_t c = threadIdx.x; c < K; c += kThreads) lds_i[c] = 0;
  __syncthreads();
  const int64_t p0 = w * P, p1 = min(nnz, p0 + P);
  constexpr int B = 8;  // column loads in flight per thread
  for (int64_t base = p0; base < p1; base += (int64_t)B * kThreads) {
    I cv[B];
#pragma unroll
    for (int u = 0; u < B; ++u) cv[u] = col[min(base + (int64_t)u * kThreads + threadIdx.x, p1 - 1)];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int64_t c = (int64_t)cv[u];
      if (base + (int64_t)u * kThreads + threadIdx.x < p1)
        atomicAdd(&lds_i[c < 0 ? 0 : (c >= K ? K - 1 : c)], 1);
    }
  }
  __syncthreads();
  for (int64_t c = threadIdx.x; c < K; c += kThreads) H[w * K + c] = lds_i[c];
}

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// 16 columns per workgroup, 16 chunk groups: thread (g, j) holds the counts
// of column 16 b + j in chunks [g n/16, (g+1) n/16) in registers.  colptr[c]
// = exclusive column prefix (earlier blocks' totals, passed through
// nonce-tagged slots and added in block order, plus this block's); H[w][c]
// is rewritten as chunk w's first slot in column c.
constexpr int kOffCols = 16;
constexpr int kOffGroups = kThreads / kOffCols;  // 16
constexpr int kOffPer = 16;                      // chunks per group held in registers
template <typename I>
__global__ __launch_bounds__(kThreads) void spmm_t_offsets_kernel(
    int* __restrict__ H, I* __restrict__ colptr, int64_t K, int64_t n_chunks, int64_t nnz,
    unsigned long long* __restrict__ slots, nl2k::slots::Key key, unsigned* __restrict__ trips) {
  __shared__ long long part[kOffGroups][kOffCols];
  __shared__ long long s_prev;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = threadIdx.x % kOffCols, g = threadIdx.x / kOffCols;
  const int64_t c = (int64_t)blockIdx.x * kOffCols + j;
  const int64_t per = (n_chunks + kOffGroups - 1) / kOffGroups;
  const int64_t w0 = min(n_chunks, g * per), w1 = min(n_chunks, w0 + per);
  long long sum = 0;
  int h[kOffPer];
  const bool cached = per <= kOffPer;
  if (c < K) {
    if (cached) {
#pragma unroll
      for (int u = 0; u < kOffPer; ++u) h[u] = w0 + u < w1 ? H[(w0 + u) * K + c] : 0;
#pragma unroll
      for (int u = 0; u < kOffPer; ++u) sum += h[u];
    } else {
      for (int64_t w = w0; w < w1; ++w) sum += H[w * K + c];
    }
  }
  part[g][j] = sum;
  __syncthreads();
  long long col_total = 0, before_g = 0;
  for (int k = 0; k < kOffGroups; ++k) {
    const long long v = part[k][j];
    col_total += v;
    before_g += k < g ? v : 0;
  }
  // exclusive prefix of the 16 column totals (one 16-lane row of wave 0)
  __shared__ long long s_cpre[kOffCols];
  if (wave == 0) {
    long long ct = 0;
    if (lane < kOffCols)
      for (int k = 0; k < kOffGroups; ++k) ct += part[k][lane];
    const long long incl = wave_incl_scan(ct, lane);
    if (lane < kOffCols) s_cpre[lane] = incl - ct;
    const long long block_total = __shfl(incl, 63, 64);
    if (lane == 0) nl2k::slots::publish(slots, blockIdx.x, (unsigned long long)block_total, key);
    // The earlier blocks' totals, 256 slots per round: every slot of a round
    // is loaded before any is waited on, so a round costs one round trip.
    const int nprev = (int)blockIdx.x;
    long long v = 0;
    for (int base = 0; base < nprev; base += 4 * 64) {
      unsigned long long x0[4], x1[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int bb = min(base + 64 * k + lane, nprev - 1);
        x0[k] = nl2k::slots::load_word(slots + 2 * bb);
        x1[k] = nl2k::slots::load_word(slots + 2 * bb + 1);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int bb = base + 64 * k + lane;
        if (bb < nprev) {
          unsigned spins = 0;
          while (!nl2k::slots::ready(x0[k], x1[k], key)) {
            if (++spins > (1u << 24)) {  // never expected: report and give up
              __hip_atomic_fetch_add(trips, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              x0[k] = key.m0;
              break;
            }
            __builtin_amdgcn_s_sleep(1);
            x0[k] = nl2k::slots::load_word(slots + 2 * bb);
            x1[k] = nl2k::slots::load_word(slots + 2 * bb + 1);
          }
          v += (long long)nl2k::slots::decode(x0[k], key);
        }
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) s_prev = v;
  }
  __syncthreads();
  if (c < K) {
    const long long cbase = s_prev + s_cpre[j];
    if (g == 0) {
      colptr[c] = (I)min(cbase, (long long)nnz);
      if (c == K - 1) colptr[K] = (I)min(cbase + col_total, (long long)nnz);
    }
    long long run = cbase + before_g;
    if (cached) {
#pragma unroll
      for (int u = 0; u < kOffPer; ++u) {
        if (w0 + u < w1) H[(w0 + u) * K + c] = (int)run;
        run += h[u];
      }
    } else {
      for (int64_t w = w0; w < w1; ++w) {
        const int hv = H[w * K + c];
        H[w * K + c] = (int)run;
        run += hv;
      }
    }
  }
}

// Largest r in [lo, hi] with row_ptr[r] <= p (row_ptr[lo] <= p assumed).
template <typename I>
__device__ __forceinline__ int64_t row_of(const I* __restrict__ ptr, int64_t lo, int64_t hi,
                                          int64_t p, int64_t nnz) {
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (ld_ptr(ptr, mid, nnz) <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Chunk w: every position's row (binary search between the rows holding
// the chunk's first and last positions), then tiles of 256 positions in
// order; within a tile the four waves take their slots one after another,
// and within a wave lanes that share a column (found through LDS tags) take
// consecutive slots in lane order.  So the entries of every column land in
// position order.
constexpr int kScatterTiles = 4;      // tiles per pass whose loads are issued together
constexpr int kScatterRowWin = 2048;  // row starts of a chunk staged in LDS
template <typename I>
__global__ __launch_bounds__(kThreads) void spmm_t_scatter_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const int* __restrict__ O, i32x4_t* __restrict__ crec, int64_t M, int64_t K, int64_t nnz,
    int64_t P) {
  extern __shared__ int lds_i[];  // K cursors, then K tag bytes
  unsigned char* tag = reinterpret_cast<unsigned char*>(lds_i + K);
  __shared__ long long s_rows[2];
  __shared__ int s_win[kScatterRowWin];  // row_ptr[ra + 1 .. ra + kScatterRowWin]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t w = blockIdx.x;
  const int64_t p0 = w * P, p1 = min(nnz, p0 + P);
  // A pass's column and value loads go out first (clamped addresses, no
  // branches), so their latency overlaps the cursor load and row search.
  I craw[kScatterTiles];
  float vv[kScatterTiles];
  auto issue = [&](int64_t t0) {
#pragma unroll
    for (int k = 0; k < kScatterTiles; ++k) {
      const int64_t qc = min(t0 + (int64_t)k * kThreads + threadIdx.x, nnz - 1);
      craw[k] = col[qc];
      vv[k] = vals[qc];
    }
  };
  issue(p0);
  load_to_lds(O + w * K, lds_i, K);
  // rows holding positions p0 and p1 - 1 (the last r with row_ptr[r] <= p),
  // one search per wave
  if (wave < 2) {
    const int64_t r = rows_lower_bound(ptr, M, nnz, wave == 0 ? p0 + 1 : p1, lane, 0) - 1;
    if (lane == 0) s_rows[wave] = max((int64_t)0, min(r, M - 1));
  }
  __syncthreads();
  const int64_t ra = s_rows[0], rb = max(s_rows[0], s_rows[1]);
  // rows are found from an LDS copy of the chunk's row starts when they fit
  const bool windowed = rb - ra <= kScatterRowWin;
  if (windowed && rb > ra) load_to_lds(ptr + ra + 1, s_win, rb - ra);
  __syncthreads();
  for (int64_t t0 = p0; t0 < p1; t0 += (int64_t)kScatterTiles * kThreads) {
    if (t0 != p0) issue(t0);
    int cc[kScatterTiles];
    int64_t rr[kScatterTiles];
#pragma unroll
    for (int k = 0; k < kScatterTiles; ++k) {
      const int64_t q = t0 + (int64_t)k * kThreads + threadIdx.x;
      const int64_t c = (int64_t)craw[k];
      const int cl = (int)(c < 0 ? 0 : (c >= K ? K - 1 : c));
      cc[k] = q < p1 ? cl : -1;
      const int64_t qr = min(q, p1 - 1);
      if (windowed) {  // row ra + n with s_win[n - 1] = row_ptr[ra + n] <= qr
        int lo = 0, hi = (int)(rb - ra);
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (s_win[mid - 1] <= qr) lo = mid;
          else hi = mid - 1;
        }
        rr[k] = ra + lo;
      } else {
        rr[k] = row_of(ptr, ra, rb, qr, nnz);
      }
    }
    // Tiles in order; within a tile the four waves take their slots one
    // after another; within a wave lanes that share a column (found through
    // LDS tags) take consecutive slots in lane order.
#pragma unroll
    for (int k = 0; k < kScatterTiles; ++k) {
      const int64_t q = t0 + (int64_t)k * kThreads + threadIdx.x;
      const bool act = q < p1;
      for (int g = 0; g < kThreads / 64; ++g) {
        if (wave == g) {
          if (act) tag[cc[k]] = (unsigned char)lane;
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          const bool loser = act && tag[cc[k]] != (unsigned char)lane;
          unsigned long long pending = __ballot(loser);
          int rank = 0;
          while (pending) {
            const int leader = __builtin_ctzll(pending);
            const int c = __shfl(cc[k], leader, 64);
            const unsigned long long grp = __ballot(act && cc[k] == c);
            if (act && cc[k] == c) rank = __popcll(grp & ((1ull << lane) - 1));
            pending &= ~grp;
          }
          int base = 0;
          if (act) base = lds_i[cc[k]];
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // every read before any add
          if (act) {
            atomicAdd(&lds_i[cc[k]], 1);
            const int64_t pos = max((int64_t)0, min((int64_t)base + rank, nnz - 1));
            crec[pos] = i32x4_t{(int)rr[k], (int)q, __float_as_int(vv[k]), 0};
          }
        }
        // the next wave reads the cursors this one advanced: LDS order only
        // (a full __syncthreads would also wait for this wave's scattered
        // global stores)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
    }
  }
}

// Column c's entries, 16 per step: the group's lanes load the step's
// records (lane gl records gl, gl + L, ...; 16-byte {row, position, value})
// and shuffle each entry's fields to the whole group, which then loads the
// 16 dY rows together; the next step's records are loaded while those rows
// are in flight.  Entries past the column's end repeat its last entry (valid
// addresses) and are masked out of the sums and stores.  G groups of L lanes
// share a column: group g takes its steps g, g + G, ... (16 entries each),
// and the G partial sums are added by an xor butterfly, so more waves share
// a long column's chain of record -> row loads.  Lanes of columns past K run
// empty, since every lane takes part in the butterfly.
template <typename I, int L, int G, bool VEC, bool DV>
__global__ __launch_bounds__(kThreads) void spmm_t_gather_kernel(
    const I* __restrict__ colptr, const i32x4_t* __restrict__ crec,
    const float* __restrict__ X, const float* __restrict__ dY, float* __restrict__ dX,
    float* __restrict__ dvals, int64_t M, int64_t K, int64_t D, int64_t nnz) {
  using V = Lanes<VEC>;
  constexpr int E = 16;                   // entries per step
  constexpr int RPL = (E + L - 1) / L;    // records per lane per step
  constexpr int kColLanes = L * G;
  static_assert(kColLanes <= 64 && (kColLanes & (kColLanes - 1)) == 0, "columns inside a wave");
  const int64_t c = (int64_t)blockIdx.x * (kThreads / kColLanes) + threadIdx.x / kColLanes;
  const int gl = threadIdx.x % L;
  const int grp = (threadIdx.x % kColLanes) / L;
  const int gbase = (threadIdx.x & 63) - gl;  // first lane of the group in the wave
  const bool live = c < K;
  const int64_t cc = live ? c : 0;
  const int64_t s = live ? ld_ptr(colptr, c, nnz) : 0;
  const int64_t e = live ? max(s, ld_ptr(colptr, c + 1, nnz)) : 0;
  auto load_recs = [&](int64_t q, i32x4_t (&r)[RPL]) {
#pragma unroll
    for (int j = 0; j < RPL; ++j) r[j] = crec[max(s, min(q + gl + (int64_t)L * j, e - 1))];
  };
  for (int64_t d0 = 0; d0 < D; d0 += (int64_t)L * V::W) {
    const int64_t d = d0 + (int64_t)gl * V::W;
    const bool active = d < D;
    const int64_t dc = active ? d : 0;
    typename V::T xc = V::zero();
    if (DV) xc = V::load(X + cc * D + dc);
    typename V::T acc = V::zero();
    i32x4_t rec[RPL];
    const int64_t q0 = s + (int64_t)grp * E;
    if (q0 < e) load_recs(q0, rec);  // a column with no entries reads nothing
    for (int64_t q = q0; q < e; q += (int64_t)G * E) {
      const int my_pos = rec[0][1];  // L == 16: lane gl holds entry gl's record
      int rr[E], pp[E];
      float vv[E];  // zero past the column's end, so the sum needs no branch
#pragma unroll
      for (int u = 0; u < E; ++u) {
        const int src = gbase + (u % L);
        rr[u] = __shfl(rec[u / L][0], src, 64);
        const float v = __int_as_float(__shfl(rec[u / L][2], src, 64));
        vv[u] = q + u < e ? v : 0.f;
        if (DV) pp[u] = __shfl(rec[u / L][1], src, 64);
      }
      typename V::T gs[E];
#pragma unroll
      for (int u = 0; u < E; ++u) {
        const int64_t r = min(max((int64_t)rr[u], (int64_t)0), M - 1);
        gs[u] = V::load(dY + r * D + dc);
      }
      load_recs(q + (int64_t)G * E, rec);
      // every row load is in flight before the first use (left alone, the
      // compiler sinks each load to its add and waits for it there)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < E; ++u) acc += vv[u] * gs[u];
      if constexpr (DV && L == 16) {
        // Reduce-scatter of the 16 partial dots over the group's 16 lanes
        // (halving butterfly): afterwards lane gl holds entry gl's dot,
        // 15 exchanges for the step instead of a 4-level reduction per entry.
        float v[E];
#pragma unroll
        for (int u = 0; u < E; ++u) v[u] = active ? V::dot(gs[u], xc) : 0.f;
        auto level = [&](auto hc) {
          constexpr int h = decltype(hc)::value;
          const bool upper = (gl & h) != 0;
#pragma unroll
          for (int k = 0; k < h; ++k) {
            const float keep = upper ? v[k + h] : v[k];
            const float send = upper ? v[k] : v[k + h];
            v[k] = keep + __shfl_xor(send, h, 16);
          }
        };
        level(std::integral_constant<int, 8>{});
        level(std::integral_constant<int, 4>{});
        level(std::integral_constant<int, 2>{});
        level(std::integral_constant<int, 1>{});
        const int64_t pu = min(max((int64_t)my_pos, (int64_t)0), nnz - 1);
        if (q + gl < e) dvals[pu] = v[0];
      } else if constexpr (DV) {
        // every lane of the group stores the (identical) group sum: a
        // one-lane branch would hold the stores' addresses inside it
#pragma unroll
        for (int u = 0; u < E; ++u) {
          const float dt = group_sum<L>(active ? V::dot(gs[u], xc) : 0.f);
          const int64_t pu = min(max((int64_t)pp[u], (int64_t)0), nnz - 1);
          if (q + u < e) dvals[pu] = dt;
        }
      }
    }
    if constexpr (G > 1) acc = groups_sum<L, G>(acc);
    if (live && active && grp == 0) V::store(dX + c * D + d, acc);
  }
}

// ---------------------- SpMM backward dX by column blocks (D > 1, K small)
// dX = A^T dY in two launches, without a global column histogram, for at most
// kBktMaxKeys blocks of Kb = 256 / L columns (K <= 4096 at 16 < D <= 64,
// K <= 16384 at D <= 16; D % 4 == 0, one float4 per lane; the reference's
// default SpMM is M = K = 4096, D = 64).
//  C1 spmm_b_sort_kernel:   chunk w = positions [w kBktChunk, (w+1) kBktChunk),
//                           one workgroup each: every position's row (as in
//                           S3), then a stable LDS sort of the chunk's
//                           entries by column block (two 4-bit radix passes,
//                           ballot ranks), written back in place as 16-byte
//                           records {row, position, value, column}, with
//                           off[w][k] = the first record of block k.
//  C2 spmm_b_gather_kernel: column block b, one workgroup each: block b's
//                           segment of every chunk (in chunk order, so in
//                           position order) copied to LDS, ordered by column
//                           (a stable counting sort with ballot ranks), and
//                           lane group j (L lanes) sums vals * dY[row] over
//                           column b Kb + j's entries, 16 per step, in
//                           registers (and forms dvals[p] = dY[row] . X[c]);
//                           up to kBktCap entries per round.
// Each dX row is summed in position order, so dX is bitwise repeatable.
constexpr int kBktChunk = 1024;
constexpr int kBktThreads = 512;
constexpr int kBktWaves = kBktThreads / 64;
constexpr int kBktMaxKeys = 256;
constexpr int kBktCap = 2048;
constexpr int kBktE = 16;  // entries per lane-group step

__device__ __forceinline__ int ranks_below(unsigned long long b) {
  return __builtin_amdgcn_mbcnt_hi((unsigned)(b >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)b, 0));
}

// Stable counting sort of n <= kBktWaves * 64 * R entries by digit(e) in
// [0, S) (S <= 64): wave v takes entries [v n_v, (v+1) n_v) in rounds of 64,
// counts them per digit (16 or 64 ballots a round), and places them after the
// entries of lower digits and of earlier waves with the same digit.
// place(e, slot) moves entry e; cnt: kBktWaves * S ints of LDS; start/len
// (optional, S ints each) receive each digit's first slot and count.
template <int S, typename Digit, typename Place>
__device__ __forceinline__ void ballot_sort(int n, Digit digit, Place place, int* cnt, int* start,
                                            int* len) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per = (n + kBktWaves - 1) / kBktWaves;
  const int e0 = min(n, wave * per), e1 = min(n, e0 + per);
  int kc = 0;  // lane d: this wave's count of digit d
  for (int i0 = e0; i0 < e1; i0 += 64) {
    const int e = i0 + lane;
    const int dg = e < e1 ? digit(e) : -1;
#pragma unroll
    for (int d = 0; d < S; ++d) {
      const unsigned long long b = __ballot(dg == d);
      if (lane == d) kc += __popcll(b);
    }
  }
  if (lane < S) cnt[wave * S + lane] = kc;
  __syncthreads();
  int tot = 0, before = 0;
  if (lane < S) {
#pragma unroll
    for (int v = 0; v < kBktWaves; ++v) {
      const int x = cnt[v * S + lane];
      tot += x;
      if (v < wave) before += x;
    }
  }
  int incl = tot;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (start != nullptr && wave == 0 && lane < S) {
    start[lane] = incl - tot;
    len[lane] = tot;
  }
  int base = incl - tot + before;  // lane d: the next slot of digit d
  for (int i0 = e0; i0 < e1; i0 += 64) {
    const int e = i0 + lane;
    const bool v = e < e1;
    const int dg = v ? digit(e) : -1;
    int rank = 0, inc = 0;
#pragma unroll
    for (int d = 0; d < S; ++d) {
      const unsigned long long b = __ballot(dg == d);
      if (dg == d) rank = ranks_below(b);
      if (lane == d) inc = __popcll(b);
    }
    const int slot = __shfl(base, dg & 63, 64) + rank;
    base += inc;
    if (v) place(e, slot);
  }
  __syncthreads();
}

// Stable ranks of NT * IPT items by a 4-bit digit: thread t holds items
// t IPT .. t IPT + IPT - 1 (dg[i] < 0 marks an empty slot) and counts them in
// its own column of cnt[16][NT] (uint16, LDS); an exclusive scan of the
// counters in digit-major order (16 consecutive counters per thread, then
// across threads) turns them into starts, and rank = start + the item's
// count before it.  start16 (optional, 17 ints) receives each digit's first
// rank and the total.
template <int NT, int IPT>
__device__ __forceinline__ void rank16(const int (&dg)[IPT], int (&rank)[IPT],
                                       unsigned short* cnt, int* wtot, int* start16) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
#pragma unroll
  for (int d = 0; d < 16; ++d) cnt[d * NT + t] = 0;
  int local[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    local[i] = 0;
    if (dg[i] >= 0) {
      unsigned short* c = cnt + dg[i] * NT + t;
      local[i] = *c;
      *c = (unsigned short)(local[i] + 1);
    }
  }
  __syncthreads();
  int run = 0, ex[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    ex[j] = run;
    run += cnt[t * 16 + j];
  }
  int incl = run;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = incl - run;
#pragma unroll
  for (int v = 0; v < NT / 64; ++v) base += v < wave ? wtot[v] : 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) cnt[t * 16 + j] = (unsigned short)(base + ex[j]);
  if (start16 != nullptr && (t * 16) % NT == 0) start16[t * 16 / NT] = base;
  if (start16 != nullptr && t == NT - 1) start16[16] = base + run;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < IPT; ++i) rank[i] = dg[i] >= 0 ? cnt[dg[i] * NT + t] + local[i] : -1;
  __syncthreads();  // cnt is reused by the next call
}

template <typename I>
__global__ __launch_bounds__(kBktThreads) void spmm_b_sort_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    i32x4_t* __restrict__ crec, int* __restrict__ off, int64_t M, int64_t K, int64_t nnz,
    int n_keys, int kb_shift) {
  __shared__ i32x4_t ent[2][kBktChunk];
  __shared__ int s_win[kScatterRowWin];  // row_ptr[ra + 1 .. rb]
  __shared__ long long s_rows[2];
  __shared__ int cnt[kBktWaves * 16];
  __shared__ unsigned short rcnt[16 * kBktThreads];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t w = blockIdx.x;
  const int64_t p0 = w * kBktChunk, p1 = min(nnz, p0 + kBktChunk);
  const int n = (int)(p1 - p0);
  constexpr int kPerT = kBktChunk / kBktThreads;
  // waves 0 and 1 find the rows holding positions p0 and p1 - 1 before
  // issuing their column loads (a wave's loads complete in order, so a
  // probe issued after them would wait for them); the loads use clamped
  // addresses, no branches
  if (wave < 2) {
    const int64_t r = rows_lower_bound(ptr, M, nnz, wave == 0 ? p0 + 1 : p1, lane, 0) - 1;
    if (lane == 0) s_rows[wave] = max((int64_t)0, min(r, M - 1));
  }
  I craw[kPerT];
  float vv[kPerT];
#pragma unroll
  for (int k = 0; k < kPerT; ++k) {
    const int64_t q = min(p0 + (int64_t)k * kBktThreads + threadIdx.x, p1 - 1);
    craw[k] = col[q];
    vv[k] = vals[q];
  }
  __syncthreads();
  const int64_t ra = s_rows[0], rb = max(s_rows[0], s_rows[1]);
  const int nw = (int)min(rb - ra, (int64_t)kScatterRowWin + 1);
  const bool windowed = rb - ra <= kScatterRowWin;
  if (windowed && rb > ra && threadIdx.x < kThreads) load_to_lds(ptr + ra + 1, s_win, rb - ra);
  __syncthreads();
  int top = 1;
  while (top * 2 <= nw) top *= 2;
#pragma unroll
  for (int k = 0; k < kPerT; ++k) {
    const int e = k * kBktThreads + threadIdx.x;
    const int64_t q = p0 + e;
    const int64_t qr = min(q, p1 - 1);
    int64_t row;
    if (windowed) {  // row ra + m with s_win[m - 1] = row_ptr[ra + m] <= qr
      int m = 0;
      for (int step = top; step > 0; step >>= 1)
        if (m + step <= nw && s_win[m + step - 1] <= qr) m += step;
      row = ra + m;
    } else {
      row = row_of(ptr, ra, rb, qr, nnz);
    }
    const int64_t c = (int64_t)craw[k];
    const int cl = (int)(c < 0 ? 0 : (c >= K ? K - 1 : c));
    if (e < n) ent[0][e] = i32x4_t{(int)row, (int)q, __float_as_int(vv[k]), cl};
  }
  __syncthreads();
  // two stable radix passes over the block index c >> kb_shift (< 256);
  // thread t moves entries 2t and 2t + 1
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const i32x4_t* src = ent[pass];
    i32x4_t* dst = ent[pass ^ 1];
    int dg[2], rk[2];
    i32x4_t it[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = 2 * threadIdx.x + i;
      it[i] = src[min(e, kBktChunk - 1)];
      dg[i] = e < n ? (it[i][3] >> (kb_shift + 4 * pass)) & 15 : -1;
    }
    rank16<kBktThreads, 2>(dg, rk, rcnt, cnt, nullptr);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (rk[i] >= 0) dst[rk[i]] = it[i];
    __syncthreads();
  }
  for (int e = threadIdx.x; e < n; e += kBktThreads) crec[p0 + e] = ent[0][e];
  // off[w][k]: the first sorted entry whose block is >= k
  int* ow = off + w * (int64_t)(n_keys + 1);
  for (int k = threadIdx.x; k <= n_keys; k += kBktThreads) {
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((ent[0][mid][3] >> kb_shift) < k) lo = mid + 1;
      else hi = mid;
    }
    ow[k] = lo;
  }
}

template <int L, bool DV>
__global__ __launch_bounds__(kBktThreads) void spmm_b_gather_kernel(
    const i32x4_t* __restrict__ crec, const int* __restrict__ off, const float* __restrict__ X,
    const float* __restrict__ dY, float* __restrict__ dX, float* __restrict__ dvals, int64_t M,
    int64_t K, int64_t D, int64_t nnz, int64_t n_chunks, int n_keys) {
  constexpr int S = kThreads / L;  // columns per block
  // two lane groups per column: half h of the workgroup takes the column's
  // steps h, h + 2, ... (kBktE entries each), and the halves' sums are
  // added in that order at the end
  __shared__ i32x4_t list[kBktCap];
  __shared__ unsigned short order[kBktCap];
  __shared__ int cnt[kBktWaves * 64];
  __shared__ int gstart[S + 1], glen[S];
  __shared__ int s_wsum[kBktWaves];
  __shared__ f32x4 s_half[kThreads];  // the second half's sums
  __shared__ unsigned short rcnt[S == 16 ? 16 * kBktThreads : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = threadIdx.x / kThreads, tl = threadIdx.x % kThreads;
  const int g = tl / L, gl = tl % L;
  const int b = blockIdx.x;
  const int64_t c = (int64_t)b * S + g;
  const bool live = c < K;
  const int64_t cc = live ? c : K - 1;
  const int d = gl * 4;
  const bool active = d < D;
  const int64_t dc = active ? d : 0;
  f32x4 xc = nl2k::zero4();
  if constexpr (DV) xc = nl2k::load4(X + cc * D + dc);
  f32x4 acc = nl2k::zero4();
  const int64_t ostride = n_keys + 1;
  for (int64_t wa = 0; wa < n_chunks;) {
    // chunk wa + t's segment of this block, t = thread
    const int64_t wt = wa + threadIdx.x;
    int s = 0, len = 0;
    if (wt < n_chunks) {
      s = off[wt * ostride + b];
      len = max(off[wt * ostride + b + 1] - s, 0);
    }
    // inclusive scan of the lengths over the workgroup
    int incl = len;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
#pragma unroll
    for (int v = 0; v < kBktWaves; ++v) incl += v < wave ? s_wsum[v] : 0;
    // this round: the leading chunks whose entries fit kBktCap (the first
    // always does: a chunk has at most kBktChunk <= kBktCap entries)
    const bool take = incl <= kBktCap && wt < n_chunks;
    const int n_take = __syncthreads_count(take);
    const int excl = incl - len;
    if (take) {  // four loads in flight at a time
      const i32x4_t* src = crec + wt * kBktChunk + s;
      for (int i = 0; i < len; i += 4) {
        i32x4_t v4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v4[u] = src[min(i + u, len - 1)];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i + u < len) list[excl + i + u] = v4[u];
      }
    }
    if (take && threadIdx.x == n_take - 1) s_wsum[0] = incl;  // the round's entry count
    __syncthreads();
    const int T = s_wsum[0];
    if constexpr (S == 16) {
      // entries by column: thread t ranks entries t IPT .. t IPT + IPT - 1
      constexpr int IPT = kBktCap / kBktThreads;
      int dg[IPT], rk[IPT];
#pragma unroll
      for (int i = 0; i < IPT; ++i) {
        const int e = threadIdx.x * IPT + i;
        dg[i] = e < T ? (list[e][3] & 15) : -1;
      }
      rank16<kBktThreads, IPT>(dg, rk, rcnt, cnt, gstart);
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if (rk[i] >= 0) order[rk[i]] = (unsigned short)(threadIdx.x * IPT + i);
      __syncthreads();
    } else {
      ballot_sort<S>(
          T, [&](int e) { return list[e][3] & (S - 1); },
          [&](int e, int slot) { order[slot] = (unsigned short)e; }, cnt, gstart, glen);
    }
    // column c's entries of the round: this half's steps
    const int q0 = gstart[g], qn = S == 16 ? gstart[g + 1] - q0 : glen[g];
    for (int q = half * kBktE; q < qn; q += 2 * kBktE) {
      i32x4_t r[kBktE];
#pragma unroll
      for (int u = 0; u < kBktE; ++u) r[u] = list[order[q0 + min(q + u, qn - 1)]];
      f32x4 gy[kBktE];
#pragma unroll
      for (int u = 0; u < kBktE; ++u) {
        const int64_t row = min(max((int64_t)r[u][0], (int64_t)0), M - 1);
        gy[u] = nl2k::load4(dY + row * D + dc);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBktE; ++u)
        if (q + u < qn) acc += __int_as_float(r[u][2]) * gy[u];
      if constexpr (DV) {
        // reduce-scatter of the kBktE dots over the group's L lanes: lane gl
        // ends with the dots of entries gl * kBktE / L .. + kBktE / L - 1
        float v[kBktE];
#pragma unroll
        for (int u = 0; u < kBktE; ++u) {
          const f32x4 y = gy[u];
          v[u] = active ? (y[0] * xc[0] + y[1] * xc[1]) + (y[2] * xc[2] + y[3] * xc[3]) : 0.f;
        }
        // Each level pairs every lane with a partner whose lane bit m
        // differs, through a DPP move inside the 16-lane row: row_mirror
        // (l <-> 15 - l) for m = 8, row_half_mirror (l <-> 7 - l within each
        // half row) for m = 4, quad_perm xor 2 and xor 1; the lane with bit
        // m set keeps the upper half of its entries.  A group is a DPP row
        // (L = 16) or a quad (L = 4), so partners never leave it, and the
        // pairs of the successive levels span the group.
        auto level = [&](auto ctlc, auto mc, auto hc) {
          constexpr int ctl = decltype(ctlc)::value, m = decltype(mc)::value,
                        h = decltype(hc)::value;
          const bool upper = (gl & m) != 0;
#pragma unroll
          for (int k = 0; k < h; ++k) {
            const float keep = upper ? v[k + h] : v[k];
            const float send = upper ? v[k] : v[k + h];
            v[k] = keep + nl2k::dpp_mov<ctl>(send);
          }
        };
        using C_MIR = std::integral_constant<int, 0x140>;
        using C_HMIR = std::integral_constant<int, 0x141>;
        using C_X2 = std::integral_constant<int, 0x4E>;
        using C_X1 = std::integral_constant<int, 0xB1>;
        using IC8 = std::integral_constant<int, 8>;
        using IC4 = std::integral_constant<int, 4>;
        using IC2 = std::integral_constant<int, 2>;
        using IC1 = std::integral_constant<int, 1>;
        static_assert(kBktE == 16, "levels below are written out for 16 entries");
        if constexpr (L == 16) {
          level(C_MIR{}, IC8{}, IC8{});
          level(C_HMIR{}, IC4{}, IC4{});
          level(C_X2{}, IC2{}, IC2{});
          level(C_X1{}, IC1{}, IC1{});
        } else {
          level(C_X2{}, IC2{}, IC8{});
          level(C_X1{}, IC1{}, IC4{});
        }
        constexpr int per = kBktE / L;
#pragma unroll
        for (int j = 0; j < per; ++j) {
          const int u = gl * per + j;
          if (q + u < qn) {
            const int64_t p = min(max((int64_t)list[order[q0 + q + u]][1], (int64_t)0), nnz - 1);
            dvals[p] = v[j];
          }
        }
      }
    }
    wa += n_take;
    __syncthreads();  // the list is rewritten by the next round
  }
  if (half == 1) s_half[tl] = acc;
  __syncthreads();
  if (half == 0 && live && active) nl2k::store4(dX + c * D + d, acc + s_half[tl]);
}

// ------------------------------ D == 1 dX: contributions formed in the sort
// tile_rows[t] for t in [0, n_tiles]: the last row r with row_ptr[r] <=
// min(t * kSortTile, nnz - 1), clamped into [0, M - 1] -- the row holding
// sort tile t's first position, and (as entry t + 1) an upper bound on the
// row holding its last.  One wave per entry.
template <typename I>
__global__ __launch_bounds__(kThreads) void spmv_tile_rows_kernel(const I* __restrict__ ptr,
                                                                  int64_t* __restrict__ tile_rows,
                                                                  int64_t M, int64_t nnz,
                                                                  int64_t n_tiles) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (t > n_tiles) return;
  const int64_t p = min(t * kSortTile, nnz - 1);
  const int64_t r = rows_lower_bound(ptr, M, nnz, p + 1, lane, 0) - 1;
  if (lane == 0) tile_rows[t] = max((int64_t)0, min(r, M - 1));
}

// base + a 32-bit byte offset: the load or store takes the base from scalar
// registers and the offset from one vector register (no 64-bit address math)
template <typename T>
__device__ __forceinline__ T* at_byte(T* base, unsigned off) {
  using C = std::conditional_t<std::is_const<T>::value, const char, char>;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + off);
}

// Loads and stores with the nontemporal hint when NT (same values).
template <bool NT, typename T>
__device__ __forceinline__ T ld_hint(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename T>
__device__ __forceinline__ void st_hint(T v, T* p) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Sort tile t = positions [kSortTile t, kSortTile (t + 1)): each position's
// contribution vals[p] * dy[row(p)] -- and dvals[p] = dy[row(p)] *
// x[col(p)], from the forward's gathered copy of x (kDvKept) or by
// gathering x (kDvGather) -- ordered by bucket (column >> shift) and written
// as val_out[lo + i] with the low column bits lowcol[lo + i], plus
// meta[t * (nb + 1) + b] = absolute start of bucket b's segment (meta[.. +
// nb] = end of the tile).  A position's row comes from an LDS copy of the
// row starts inside the tile (a fixed-step search for a quad's first
// position, forward steps for the other three); a tile spanning more rows
// than the copy holds searches row_ptr in global memory.  Positions outside
// [row_ptr[0], row_ptr[M]) belong to no row: they contribute zero and get
// no dvals.
constexpr int kTileRowWin = 4096;  // row starts of a tile staged in LDS (within s_val)
static_assert(kTileRowWin <= kSortTile, "the row starts share s_val's LDS");
constexpr int kDvNone = 0, kDvKept = 1, kDvGather = 2;
template <typename I, bool VEC, int DVM>
__global__ __launch_bounds__(kSortThreads) void spmv_walk_sort_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, const float* __restrict__ vals,
    const float* __restrict__ x, const float* __restrict__ xg, const float* __restrict__ dy,
    float* __restrict__ dvals, float* __restrict__ val_out, uint16_t* __restrict__ lowcol,
    int64_t* __restrict__ meta, const int64_t* __restrict__ tile_rows, int64_t M, int64_t nnz,
    int64_t K, int shift, int nb) {
  __shared__ float s_val[kSortTile];
  __shared__ uint16_t s_low[kSortTile];
  __shared__ unsigned s_cur[kMaxBuckets];
  __shared__ unsigned s_wave[kSortThreads / 64];
  // Nontemporal hints where they measured faster at the acceptance shape
  // (Zipf 2^20, int32): structure loads when dvals are formed (gathering
  // 183.2 -> 180.8 us, kept x 126.8 -> 125.9; dX alone 103.5 -> 104.5
  // with them), output stores when x is gathered (180.8 -> 177.5 us; the
  // other variants slower by 1.5-2.5 us), where they keep the L2 for x.
  constexpr bool kNtLoads = DVM != kDvNone;
  constexpr bool kNtStores = DVM == kDvGather;
  // row_ptr[ra + 1 + k] - lo, clamped into [0, kSortTile]: read before the
  // first barrier of the counting step, s_val written after it
  int* s_win = reinterpret_cast<int*>(s_val);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t lo = (int64_t)blockIdx.x * kSortTile;
  const int n = (int)min((int64_t)kSortTile, nnz - lo);
  // Tile bases: every per-position index below is a 32-bit offset from one
  // of these (a scalar base plus a vector offset, no 64-bit address math).
  const I* __restrict__ ct = col + lo;
  const float* __restrict__ vt = vals + lo;
  const float* __restrict__ xt = xg + (DVM == kDvKept ? lo : 0);
  float* __restrict__ dvt = dvals + (DVM != kDvNone ? lo : 0);
  for (int b = tid; b < nb; b += kSortThreads) s_cur[b] = 0;
  // columns clamp into [0, K - 1]; the bucket plan keeps K at most 2^24
  const int kmax = (int)(K - 1);
  auto clamp_col = [&](auto c) -> unsigned {
    return (unsigned)(c < 0 ? 0 : (c > (decltype(c))kmax ? kmax : (int)c));
  };

  // Structure loads first, raw: one uniform branch picks whole-quad vector
  // loads (tiles of a multiple of 4 positions) or clamped scalar loads, and
  // nothing inside it reads a loaded value, so no wait separates the quads'
  // loads (the columns are clamped after the row-start loads are issued).
  I craw[kSortPer];
  float vv[kSortPer], xv[kSortPer];
  if (VEC && (n & 3) == 0) {
#pragma unroll
    for (int g = 0; g < kSortPer / 4; ++g) {
      const unsigned i = min(4u * (unsigned)(tid + kSortThreads * g), (unsigned)n - 4u);
      const f32x4 v4 = ld_hint<kNtLoads>(reinterpret_cast<const f32x4*>(at_byte(vt, 4u * i)));
      f32x4 x4 = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (DVM == kDvKept)
        x4 = ld_hint<kNtLoads>(reinterpret_cast<const f32x4*>(at_byte(xt, 4u * i)));
      if constexpr (sizeof(I) == 4) {
        const i32x4_t ci = ld_hint<kNtLoads>(reinterpret_cast<const i32x4_t*>(at_byte(ct, 4u * i)));
#pragma unroll
        for (int j = 0; j < 4; ++j) craw[4 * g + j] = ci[j];
      } else {
        const i64x2_t c0 = ld_hint<kNtLoads>(reinterpret_cast<const i64x2_t*>(at_byte(ct, 8u * i)));
        const i64x2_t c1 =
            ld_hint<kNtLoads>(reinterpret_cast<const i64x2_t*>(at_byte(ct, 8u * i + 16u)));
        craw[4 * g + 0] = c0[0];
        craw[4 * g + 1] = c0[1];
        craw[4 * g + 2] = c1[0];
        craw[4 * g + 3] = c1[1];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vv[4 * g + j] = v4[j];
        xv[4 * g + j] = x4[j];
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < kSortPer / 4; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned q = min(4u * (unsigned)(tid + kSortThreads * g) + j, (unsigned)n - 1u);
        craw[4 * g + j] = *at_byte(ct, q * (unsigned)sizeof(I));
        vv[4 * g + j] = *at_byte(vt, 4u * q);
        if constexpr (DVM == kDvKept) xv[4 * g + j] = *at_byte(xt, 4u * q);
        else xv[4 * g + j] = 0.f;
      }
  }
  // the row holding the tile's first position, and an upper bound on the
  // one holding its last (the row of the next tile's first position)
  const int64_t ra = min(max(tile_rows[blockIdx.x], (int64_t)0), M - 1);
  const int64_t rb = max(ra, min(tile_rows[blockIdx.x + 1], M - 1));
  // positions [first_rel, end_rel) of the tile belong to rows
  const int first_rel = (int)min(max(ld_ptr(ptr, 0, nnz) - lo, (int64_t)0), (int64_t)n);
  const int end_rel = (int)min(max(ld_ptr(ptr, M, nnz) - lo, (int64_t)0), (int64_t)n);
  // rows from the LDS copy when the tile's row starts fit it; entries past
  // the copied ones hold a sentinel above every tile offset
  const bool windowed = rb - ra < kTileRowWin;
  const int nwin = windowed ? (int)(rb - ra) : 0;
  // (loaded and written without branches, also when unused: indices clamp
  // in range, row_ptr[ra + 1] exists since ra <= M - 1)
  constexpr int kPerThread = kTileRowWin / kSortThreads;
  const I* __restrict__ pt = ptr + ra + 1;
  const unsigned last = (unsigned)max(nwin - 1, 0);
  I wraw[kPerThread];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u)
    wraw[u] = *at_byte(pt, min((unsigned)(tid + kSortThreads * u), last) * (unsigned)sizeof(I));
  unsigned cc[kSortPer];
#pragma unroll
  for (int k = 0; k < kSortPer; ++k) cc[k] = clamp_col(craw[k]);
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int k = tid + kSortThreads * u;
    const int v = (int)min(max((int64_t)wraw[u] - lo, (int64_t)0), (int64_t)kSortTile);
    s_win[k] = k < nwin ? v : kSortTile + 1;
  }
  __syncthreads();  // s_win; s_cur zeroed
  if constexpr (DVM == kDvGather) {
#pragma unroll
    for (int k = 0; k < kSortPer; ++k) xv[k] = *at_byte(x, 4u * cc[k]);
  }

  // Each position's row, then its contribution (and dvals).
  const float* __restrict__ dyt = dy + ra;
  float gy[kSortPer];
#pragma unroll
  for (int g = 0; g < kSortPer / 4; ++g) {
    const int i0 = 4 * (tid + kSortThreads * g);
    if (windowed) {
      // a = the number of row starts at or before i0 (at most nwin <=
      // kTileRowWin - 1): a fixed-step search, so the quads' searches
      // interleave; the quad's other positions step forward from it.  Row
      // ra + a lies in [ra, rb].
      unsigned a = 0;
#pragma unroll
      for (unsigned step = kTileRowWin / 2; step > 0; step >>= 1)
        a += s_win[a + step - 1] <= i0 ? step : 0u;
      gy[4 * g] = *at_byte(dyt, 4u * a);
#pragma unroll
      for (int j = 1; j < 4; ++j) {
        while (s_win[a] <= i0 + j) ++a;
        gy[4 * g + j] = *at_byte(dyt, 4u * a);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        gy[4 * g + j] = dy[row_of(ptr, ra, rb, lo + min(i0 + j, n - 1), nnz)];
    }
  }
#pragma unroll
  for (int g = 0; g < kSortPer / 4; ++g) {
    const int i0 = 4 * (tid + kSortThreads * g);
    bool in[4];
    f32x4 dv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      in[j] = i0 + j >= first_rel && i0 + j < end_rel;
      const int k = 4 * g + j;
      dv[j] = gy[k] * xv[k];
      vv[k] = in[j] ? vv[k] * gy[k] : 0.f;
    }
    if constexpr (DVM != kDvNone) {
      if (VEC && in[0] && in[1] && in[2] && in[3]) {
        // nontemporal: gathering 178.9 -> 174.3 us, kept x 126.2 -> 123.5
        __builtin_nontemporal_store(dv, reinterpret_cast<f32x4*>(at_byte(dvt, 4u * i0)));
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (in[j]) *at_byte(dvt, 4u * (i0 + j)) = dv[j];
      }
    }
  }

  // Count per bucket (LDS integer atomics), exclusive scan of the counts
  // (two buckets per thread), then place: a bucket's cursor hands out the
  // slots of its segment, so the tile is ordered by bucket in LDS before it
  // is written out with 16-byte stores.
#pragma unroll
  for (int g = 0; g < kSortPer / 4; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * (tid + kSortThreads * g) + j < n)
        __hip_atomic_fetch_add(&s_cur[cc[4 * g + j] >> shift], 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
  __syncthreads();
  const int b0 = 2 * tid;
  const unsigned a0 = b0 < nb ? s_cur[b0] : 0u;
  const unsigned a1 = b0 + 1 < nb ? s_cur[b0 + 1] : 0u;
  const unsigned incl = wave_incl_scan(a0 + a1, lane);
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  unsigned off = incl - (a0 + a1);
  for (int w = 0; w < wave; ++w) off += s_wave[w];
  int64_t* mrow = meta + (int64_t)blockIdx.x * (nb + 1);
  if (b0 < nb) {
    s_cur[b0] = off;
    mrow[b0] = lo + off;
  }
  if (b0 + 1 < nb) {
    s_cur[b0 + 1] = off + a0;
    mrow[b0 + 1] = lo + off + a0;
  }
  if (tid == 0) mrow[nb] = lo + n;
  __syncthreads();
  const unsigned low_mask = (1u << shift) - 1u;
#pragma unroll
  for (int g = 0; g < kSortPer / 4; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * (tid + kSortThreads * g) + j < n) {
        const unsigned c = cc[4 * g + j];
        unsigned r = __hip_atomic_fetch_add(&s_cur[c >> shift], 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_WORKGROUP);
        r = r < (unsigned)kSortTile ? r : (unsigned)kSortTile - 1u;
        s_val[r] = vv[4 * g + j];
        s_low[r] = (uint16_t)(c & low_mask);
      }
  __syncthreads();
  float* __restrict__ vo = val_out + lo;
  uint16_t* __restrict__ lw = lowcol + lo;
  for (int i = 4 * tid; i < n; i += 4 * kSortThreads) {
    if (i + 3 < n) {
      st_hint<kNtStores>(*reinterpret_cast<const f32x4*>(s_val + i),
                         reinterpret_cast<f32x4*>(at_byte(vo, 4u * i)));
      st_hint<kNtStores>(*reinterpret_cast<const uint64_t*>(s_low + i),
                         reinterpret_cast<uint64_t*>(at_byte(lw, 2u * i)));
    } else {
      for (int j = i; j < n; ++j) {
        *at_byte(vo, 4u * j) = s_val[j];
        *at_byte(lw, 2u * j) = s_low[j];
      }
    }
  }
}

__global__ __launch_bounds__(kThreads) void spmv_fill_zero_kernel(float* __restrict__ a,
                                                                   int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    a[i] = 0.f;
}

// Structure check (spmv_check_structure_*): report[0] collects the
// kStruct* bits of every violation, report[1] the smallest position whose
// column is out of [0, K), report[2] the smallest r with a bad row_ptr[r]
// (r = 0 for row_ptr[0] != 0, r = M for row_ptr[M] != nnz, else the first
// r with row_ptr[r] < row_ptr[r-1] or outside [0, nnz]).  The two kernels
// run in stream order: the first sets the report's initial values (no
// memset, so the pair can be captured into a HIP graph).
constexpr unsigned long long kStructFirst = 1, kStructOrder = 2, kStructLast = 4,
                             kStructColumn = 8;

__global__ void spmv_check_init_kernel(unsigned long long* __restrict__ report) {
  if (threadIdx.x < 4) report[threadIdx.x] = threadIdx.x == 0 || threadIdx.x == 3 ? 0ull : ~0ull;
}

template <typename I>
__global__ __launch_bounds__(kThreads) void spmv_check_kernel(
    const I* __restrict__ ptr, const I* __restrict__ col, int64_t M, int64_t K, int64_t nnz,
    unsigned long long* __restrict__ report) {
  const int64_t n = std::max<int64_t>(M + 1, nnz);
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    if (i <= M) {
      const int64_t v = (int64_t)ptr[i];
      unsigned long long bad = 0;
      if (i == 0 && v != 0) bad |= kStructFirst;
      if (i == M && v != nnz) bad |= kStructLast;
      if (v < 0 || v > nnz || (i > 0 && v < (int64_t)ptr[i - 1])) bad |= kStructOrder;
      if (bad) {
        atomicOr(&report[0], bad);
        atomicMin(&report[2], (unsigned long long)i);
      }
    }
    if (i < nnz) {
      const int64_t c = (int64_t)col[i];
      if (c < 0 || c >= K) {
        atomicOr(&report[0], kStructColumn);
        atomicMin(&report[1], (unsigned long long)i);
      }
    }
  }
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

// Groups of L lanes that share a column in the SpMM backward's gather: 2
// when L * 2 <= 64 and an average column has two 16-entry steps or more,
// else 1.  At the reference default (64 entries per column, L = 16, 159
// VGPRs: 3 waves per SIMD) the backward measured 41.9 us with G = 1, 39.5
// with G = 2 and 41.2 with G = 4, whose 4096 waves overflow one round.
int spmm_col_groups(int L, int64_t K, int64_t nnz) {
  const int64_t avg = K > 0 ? nnz / K : 0;
  return (2 * L <= 64 && avg >= 32) ? 2 : 1;
}

// Groups of L lanes that split each row's nonzeros in the SpMM forward: the
// largest power of two with L * G <= 64 that leaves each group about 8 or
// more nonzeros of an average row (G = 4 at the reference default: 64 per
// row, L = 16).
int spmm_row_groups(int L, int64_t M, int64_t nnz) {
  const int64_t avg = M > 0 ? nnz / M : 0;
  int G = 1;
  while (G * 2 * L <= 64 && G * 2 <= 16 && avg >= 8 * (G * 2)) G *= 2;
  return G;
}

// Waves of a D == 1 walk kernel that gathers x (`items` = rows +
// nonzeros): one round of the waves the device holds at once, so every wave
// starts together and no part-filled round trails, but no more than one
// wave per kWaveItemsMin items.
int gather_walk_waves(const void* kernel, int64_t items, int64_t* n_waves) {
  int resident = 1;
  const int st = nl2k::resident_blocks(kernel, kThreads, &resident);
  if (st) return st;
  const int64_t waves = (int64_t)resident * (kThreads / 64);
  *n_waves = std::max<int64_t>(1, std::min(waves, nl2k::ceil_div(items, kWaveItemsMin)));
  return NL2K_SUCCESS;
}

// Xg != nullptr (D == 1 only): also write Xg[p] = X[col[p]] for the
// backward's dvals.
template <typename I>
int forward(const I* ptr, const I* col, const float* vals, const float* X, float* Y, float* Xg,
            bool want_xg, int64_t M, int64_t K, int64_t D, int64_t nnz, hipStream_t stream,
            const char* who) {
  const int64_t imax = sizeof(I) == 4 ? INT32_MAX : INT64_MAX / 2;
  int st = validate(M, K, D, nnz, imax, who);
  if (st) return st;
  if (want_xg && D != 1)
    return nl2k::fail(NL2K_ERR_SHAPE, "%s: the gathered copy of X needs D == 1 (got D=%lld)", who,
                      (long long)D);
  if (want_xg && nnz > 0 && !Xg) return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (M == 0) return nl2k::succeed();
  if (!ptr || !X || !Y || (nnz > 0 && (!col || !vals)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (D == 1) {
    const bool save = want_xg && nnz > 0;
    const bool vec = nl2k::aligned16(col) && nl2k::aligned16(vals) && (!save || nl2k::aligned16(Xg));
    auto* kernel = vec ? (save ? &spmv_d1_fwd_kernel<I, true, true> : &spmv_d1_fwd_kernel<I, true, false>)
                       : (save ? &spmv_d1_fwd_kernel<I, false, true>
                               : &spmv_d1_fwd_kernel<I, false, false>);
    int64_t n_waves = 1;
    st = gather_walk_waves(reinterpret_cast<const void*>(kernel), nnz + M, &n_waves);
    if (st) return st;
    const int64_t blocks = nl2k::ceil_div(n_waves, kThreads / 64);
    if (blocks > INT32_MAX) return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: too many rows", who);
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, ptr, col, vals,
                       X, Y, Xg, M, K, nnz, n_waves);
    return nl2k::check_launch(who);
  }
  const bool vec = D % 4 == 0 && nl2k::aligned16(X) && nl2k::aligned16(Y);
  const int L = lanes_for(D, vec);
  const int G = spmm_row_groups(L, M, nnz);
  const int64_t blocks = nl2k::ceil_div(M, kThreads / (L * G));
  const dim3 grid((unsigned)blocks), block(kThreads);
#define SPMM_FWD(LL, GG, VV)                                                                    \
  hipLaunchKernelGGL((spmm_fwd_kernel<I, LL, GG, VV>), grid, block, 0, stream, ptr, col, vals, X, \
                     Y, M, K, D, nnz)
#define SPMM_FWD_L16(VV)              \
  if (G == 1) SPMM_FWD(16, 1, VV);    \
  else if (G == 2) SPMM_FWD(16, 2, VV); \
  else SPMM_FWD(16, 4, VV)
#define SPMM_FWD_L4(VV)               \
  if (G == 1) SPMM_FWD(4, 1, VV);     \
  else if (G == 2) SPMM_FWD(4, 2, VV);  \
  else if (G == 4) SPMM_FWD(4, 4, VV);  \
  else if (G == 8) SPMM_FWD(4, 8, VV);  \
  else SPMM_FWD(4, 16, VV)
  if (vec) {
    if (L == 4) { SPMM_FWD_L4(true); }
    else if (L == 16) { SPMM_FWD_L16(true); }
    else SPMM_FWD(64, 1, true);
  } else {
    if (L == 4) { SPMM_FWD_L4(false); }
    else if (L == 16) { SPMM_FWD_L16(false); }
    else SPMM_FWD(64, 1, false);
  }
#undef SPMM_FWD_L4
#undef SPMM_FWD_L16
#undef SPMM_FWD
  return nl2k::check_launch(who);
}

// Xg != nullptr (dvals requested, mode kNoDx): the gathered walk.  The
// walks that gather x (dvals without Xg) run as one resident round; the
// others take kWaveItemsLong items per wave.
template <typename I>
int launch_d1_bwd(bool vec, bool dv, int mode, hipStream_t stream, const I* ptr, const I* col,
                  const float* vals, const float* X, const float* Xg, const float* dY,
                  float* dvals, float* out, int64_t M, int64_t K, int64_t nnz, const char* who) {
  auto pick = [&](auto v) {
    constexpr bool V = decltype(v)::value;
    if (dv && Xg != nullptr && mode == kNoDx) return &spmv_d1_bwd_kernel<I, V, true, kNoDx, true>;
    if (dv)
      return mode == kAtomic ? &spmv_d1_bwd_kernel<I, V, true, kAtomic, false>
                             : &spmv_d1_bwd_kernel<I, V, true, kNoDx, false>;
    return mode == kAtomic ? &spmv_d1_bwd_kernel<I, V, false, kAtomic, false>
                           : &spmv_d1_bwd_kernel<I, V, false, kNoDx, false>;
  };
  auto* kernel = vec ? pick(std::true_type{}) : pick(std::false_type{});
  const bool gathers = dv && !(Xg != nullptr && mode == kNoDx);
  int64_t n_waves = std::max<int64_t>(1, nl2k::ceil_div(nnz + M, kWaveItemsLong));
  if (gathers) {
    const int st = gather_walk_waves(reinterpret_cast<const void*>(kernel), nnz + M, &n_waves);
    if (st) return st;
  }
  const int64_t blocks = nl2k::ceil_div(n_waves, kThreads / 64);
  if (blocks > INT32_MAX) return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: too many rows", who);
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, ptr, col, vals, X,
                     Xg, dY, dvals, out, M, K, nnz, n_waves);
  return nl2k::check_launch(who);
}

// dX by bucket sort (D == 1): bucket width `cols` = 2^shift, nb buckets,
// n_tiles sort tiles; workspace = contributions (sorted in place) | low
// column bits | segment offsets.
struct BucketPlan {
  bool use = false;
  int shift = 0, cols = 0, nb = 0;
  int64_t n_tiles = 0;
  size_t off_low = 0, off_meta = 0, off_rows = 0, bytes = 0;
};

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

BucketPlan bucket_plan(int64_t K, int64_t D, int64_t nnz) {
  BucketPlan p;
  if (D != 1 || nnz <= 0 || K < 1) return p;
  int shift = 8;  // about 256 buckets, 256 .. 16384 columns each
  while ((int64_t(1) << shift) < kMaxBucketCols && (int64_t(256) << shift) < K) ++shift;
  const int64_t nb = nl2k::ceil_div(K, int64_t(1) << shift);
  if (nb > kMaxBuckets) return p;
  p.use = true;
  p.shift = shift;
  p.cols = 1 << shift;
  p.nb = (int)nb;
  p.n_tiles = nl2k::ceil_div(nnz, kSortTile);
  p.off_low = align256((size_t)nnz * sizeof(float));
  p.off_meta = p.off_low + align256((size_t)nnz * sizeof(uint16_t));
  p.off_rows = p.off_meta + align256((size_t)p.n_tiles * (size_t)(p.nb + 1) * sizeof(int64_t));
  p.bytes = p.off_rows + (size_t)(p.n_tiles + 1) * sizeof(int64_t);
  return p;
}

// Stable transpose for dX at D > 1 (spmm_t_* kernels); workspace sections
// 256-byte aligned: trip counter (8 B, first, so its offset does not depend
// on the index type), look-back slots [n_blocks] (16 B), H [n_chunks][K]
// (int32 counts, then first slots), colptr [K+1] (I), records [nnz] (16 B:
// int32 row, int32 position, fp32 value, pad; nnz < 2^31 and M < 2^31).
// Chunks of P positions, about one per CU.
struct TransposePlan {
  bool use = false;
  int64_t P = 0, n_chunks = 0, n_blocks = 0;
  size_t off_status = 0, off_slots = 0, off_H = 0, off_colptr = 0, off_rec = 0, bytes = 0;
};

TransposePlan transpose_plan(int64_t M, int64_t K, int64_t D, int64_t nnz, size_t isz) {
  TransposePlan p;
  if (D <= 1 || M <= 0 || nnz <= 0 || nnz > INT32_MAX || K > kTransposeMaxCols) return p;
  p.use = true;
  p.P = std::max<int64_t>(kTransposeChunk, nl2k::ceil_div(nnz, 256));
  p.P = nl2k::ceil_div(p.P, kThreads) * kThreads;
  p.n_chunks = nl2k::ceil_div(nnz, p.P);
  while (p.n_chunks * K > (int64_t(1) << 24)) {  // keep H within 16 M entries
    p.P *= 2;
    p.n_chunks = nl2k::ceil_div(nnz, p.P);
  }
  p.n_blocks = nl2k::ceil_div(K, kOffCols);
  p.off_status = 0;
  size_t off = 256;
  p.off_slots = off;
  off += align256((size_t)p.n_blocks * 16);
  p.off_H = off;
  off += align256((size_t)(p.n_chunks * K) * sizeof(int));
  p.off_colptr = off;
  off += align256((size_t)(K + 1) * isz);
  p.off_rec = off;
  p.bytes = off + align256((size_t)nnz * 16);
  return p;
}

// dX by column blocks (spmm_b_* kernels): D > 1, D % 4 == 0, D <= 64, at
// most kBktMaxKeys blocks of 256 / L columns, nnz < 2^31.  Workspace: the
// first 256 bytes are left alone (the transposed route's trip counter lives
// there, so its offset is the same whichever route a call takes), then the
// records [nnz] (16 B) and off [n_chunks][n_keys + 1] (int32).
struct ColBlockPlan {
  bool use = false;
  int L = 0, n_keys = 0, kb_shift = 0;
  int64_t n_chunks = 0;
  size_t off_rec = 256, off_off = 0, bytes = 0;
};

constexpr int64_t kColBlockMinKeys = 128;  // column blocks the column-block route needs

ColBlockPlan col_block_plan(int64_t M, int64_t K, int64_t D, int64_t nnz) {
  ColBlockPlan p;
  if (D <= 1 || D > 64 || D % 4 != 0 || M <= 0 || M > INT32_MAX || nnz <= 0 || nnz > INT32_MAX)
    return p;
  const int L = D <= 16 ? 4 : 16;
  const int kb = kThreads / L;
  const int64_t n_keys = nl2k::ceil_div(K, (int64_t)kb);
  // Fewer column blocks than this leave most CUs idle in the gather: the
  // column-major copy is faster there (4096 columns at D = 8, 64 blocks of
  // 64 columns: 85.7 against 39.8 us; 2048 columns at D = 64, 128 blocks,
  // stay: 25.7 against 32.9).
  if (n_keys > kBktMaxKeys || n_keys < kColBlockMinKeys) return p;
  p.use = true;
  p.L = L;
  p.n_keys = (int)n_keys;
  p.kb_shift = __builtin_ctz(kb);
  p.n_chunks = nl2k::ceil_div(nnz, (int64_t)kBktChunk);
  p.off_off = p.off_rec + align256((size_t)nnz * 16);
  p.bytes = p.off_off + align256((size_t)p.n_chunks * (size_t)(n_keys + 1) * sizeof(int));
  return p;
}

template <typename I>
size_t workspace_bytes_for(int64_t M, int64_t K, int64_t D, int64_t nnz) {
  if (M <= 0) return 0;
  if (D == 1) return bucket_plan(K, D, nnz).bytes;
  // the column-block route needs 16-byte aligned X, dY and dX, known only at
  // the call: room for either route
  const ColBlockPlan cp = col_block_plan(M, K, D, nnz);
  return std::max(cp.use ? cp.bytes : (size_t)0, transpose_plan(M, K, D, nnz, sizeof(I)).bytes);
}

template <typename I>
int col_block_backward(const ColBlockPlan& cp, const I* ptr, const I* col, const float* vals,
                       const float* X, const float* dY, float* dvals, float* dX, int64_t M,
                       int64_t K, int64_t D, int64_t nnz, char* ws, hipStream_t stream,
                       const char* who) {
  i32x4_t* crec = reinterpret_cast<i32x4_t*>(ws + cp.off_rec);
  int* off = reinterpret_cast<int*>(ws + cp.off_off);
  hipLaunchKernelGGL((spmm_b_sort_kernel<I>), dim3((unsigned)cp.n_chunks), dim3(kBktThreads), 0,
                     stream, ptr, col, vals, crec, off, M, K, nnz, cp.n_keys, cp.kb_shift);
  int st = nl2k::check_launch(who);
  if (st) return st;
  const dim3 grid((unsigned)cp.n_keys), block(kBktThreads);
#define SPMM_B(LL, DVV)                                                                      \
  hipLaunchKernelGGL((spmm_b_gather_kernel<LL, DVV>), grid, block, 0, stream, crec, off, X, dY, \
                     dX, dvals, M, K, D, nnz, cp.n_chunks, cp.n_keys)
  if (cp.L == 4) {
    if (dvals) SPMM_B(4, true); else SPMM_B(4, false);
  } else {
    if (dvals) SPMM_B(16, true); else SPMM_B(16, false);
  }
#undef SPMM_B
  return nl2k::check_launch(who);
}

template <typename I>
int transpose_backward(const TransposePlan& tp, const I* ptr, const I* col, const float* vals,
                       const float* X, const float* dY, float* dvals, float* dX, int64_t M,
                       int64_t K, int64_t D, int64_t nnz, char* ws, hipStream_t stream,
                       const char* who) {
  int* H = reinterpret_cast<int*>(ws + tp.off_H);
  I* colptr = reinterpret_cast<I*>(ws + tp.off_colptr);
  unsigned long long* slots = reinterpret_cast<unsigned long long*>(ws + tp.off_slots);
  unsigned* trips = reinterpret_cast<unsigned*>(ws + tp.off_status);
  i32x4_t* crec = reinterpret_cast<i32x4_t*>(ws + tp.off_rec);
  hipError_t qe = hipSuccess;
  const bool cap = nl2k::slots::capturing(stream, &qe);
  if (qe != hipSuccess) return nl2k::check_hip(qe, "hipStreamIsCapturing");
  if (cap) nl2k::slots::clear_async(slots, 2 * tp.n_blocks, stream);
  int st = NL2K_SUCCESS;
  const size_t lds = (size_t)K * sizeof(int);               // histogram kernel
  const size_t lds_s = lds + (size_t)nl2k::ceil_div(K, 4) * 4;  // cursors + tags
  if (lds_s > (48u << 10)) {  // up to 80 KB of dynamic LDS (K <= 16384)
    st = nl2k::raise_dynamic_lds((const void*)&spmm_t_hist_kernel<I>, (int)lds);
    if (!st) st = nl2k::raise_dynamic_lds((const void*)&spmm_t_scatter_kernel<I>, (int)lds_s);
    if (st) return st;
  }
  hipLaunchKernelGGL((spmm_t_hist_kernel<I>), dim3((unsigned)tp.n_chunks), dim3(kThreads), lds,
                     stream, col, H, K, nnz, tp.P);
  st = nl2k::check_launch(who);
  if (st) return st;
  hipLaunchKernelGGL((spmm_t_offsets_kernel<I>), dim3((unsigned)tp.n_blocks), dim3(kThreads), 0,
                     stream, H, colptr, K, tp.n_chunks, nnz, slots, nl2k::slots::next_key(),
                     trips);
  st = nl2k::check_launch(who);
  if (st) return st;
  hipLaunchKernelGGL((spmm_t_scatter_kernel<I>), dim3((unsigned)tp.n_chunks), dim3(kThreads), lds_s,
                     stream, ptr, col, vals, H, crec, M, K, nnz, tp.P);
  st = nl2k::check_launch(who);
  if (st) return st;
  const bool vec = D % 4 == 0 && nl2k::aligned16(X) && nl2k::aligned16(dY) &&
                   nl2k::aligned16(dX);
  const int L = lanes_for(D, vec);
  const bool dv = dvals != nullptr && D <= (int64_t)L * (vec ? 4 : 1);
  const int G = spmm_col_groups(L, K, nnz);
  const int64_t blocks = nl2k::ceil_div(K, kThreads / (L * G));
  const dim3 grid((unsigned)blocks), block(kThreads);
#define SPMM_T(LL, GG, VV, DVV)                                                                   \
  hipLaunchKernelGGL((spmm_t_gather_kernel<I, LL, GG, VV, DVV>), grid, block, 0, stream, colptr, \
                     crec, X, dY, dX, dvals, M, K, D, nnz)
#define SPMM_T_G(LL, VV, DVV)         \
  if (G == 1) SPMM_T(LL, 1, VV, DVV); \
  else SPMM_T(LL, 2, VV, DVV)
#define SPMM_T_L(VV, DVV)                     \
  if (L == 4) { SPMM_T_G(4, VV, DVV); }       \
  else if (L == 16) { SPMM_T_G(16, VV, DVV); } \
  else SPMM_T(64, 1, VV, DVV)
  if (vec) {
    if (dv) { SPMM_T_L(true, true); } else { SPMM_T_L(true, false); }
  } else {
    if (dv) { SPMM_T_L(false, true); } else { SPMM_T_L(false, false); }
  }
#undef SPMM_T_L
#undef SPMM_T_G
#undef SPMM_T
  st = nl2k::check_launch(who);
  if (st || dvals == nullptr || dv) return st;
  // dvals for D beyond one gather pass: the row-wise kernel, without dX
  const bool vr = D % 4 == 0 && nl2k::aligned16(X) && nl2k::aligned16(dY);
  const int Lr = lanes_for(D, vr);
  const dim3 rgrid((unsigned)nl2k::ceil_div(M, kThreads / Lr));
#define SPMM_DV(LL, VV)                                                                        \
  hipLaunchKernelGGL((spmm_bwd_kernel<I, LL, VV>), rgrid, block, 0, stream, ptr, col, vals, X, \
                     dY, dvals, (float*)nullptr, M, K, D, nnz)
  if (vr) {
    if (Lr == 4) SPMM_DV(4, true);
    else if (Lr == 16) SPMM_DV(16, true);
    else SPMM_DV(64, true);
  } else {
    if (Lr == 4) SPMM_DV(4, false);
    else if (Lr == 16) SPMM_DV(16, false);
    else SPMM_DV(64, false);
  }
#undef SPMM_DV
  return nl2k::check_launch(who);
}

// Xg != nullptr (D == 1 only): dvals reads the forward's gathered copy of X
// (spmv_forward_gather_*) instead of gathering, on the routes that do not
// scatter by column (the bucket route and dvals alone).
template <typename I>
int backward(const I* ptr, const I* col, const float* vals, const float* X, const float* Xg,
             bool want_xg, const float* dY, float* dvals, float* dX, int64_t M, int64_t K,
             int64_t D, int64_t nnz, void* workspace, size_t ws_bytes, hipStream_t stream,
             const char* who) {
  const int64_t imax = sizeof(I) == 4 ? INT32_MAX : INT64_MAX / 2;
  int st = validate(M, K, D, nnz, imax, who);
  if (st) return st;
  if (want_xg && D != 1)
    return nl2k::fail(NL2K_ERR_SHAPE, "%s: the gathered copy of X needs D == 1 (got D=%lld)", who,
                      (long long)D);
  if (!ptr || !X || (M > 0 && !dY) || (nnz > 0 && (!col || !vals)) ||
      (want_xg && nnz > 0 && !Xg))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  if (!want_xg || nnz == 0) Xg = nullptr;
  const BucketPlan bp = bucket_plan(K, D, nnz);
  const bool sorted_dx = dX && bp.use && M > 0;
  if (sorted_dx) {
    if (!workspace || ws_bytes < bp.bytes)
      return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                        bp.bytes, workspace ? ws_bytes : (size_t)0);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 256-byte aligned", who);
  }
  if (sorted_dx) {
    // one kernel per sort tile forms the contributions (and dvals) and
    // sorts them by column bucket; one per bucket sums them into dx
    if (bp.n_tiles > INT32_MAX) return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: too many rows", who);
    char* ws = static_cast<char*>(workspace);
    float* contrib = reinterpret_cast<float*>(ws);
    uint16_t* low = reinterpret_cast<uint16_t*>(ws + bp.off_low);
    int64_t* meta = reinterpret_cast<int64_t*>(ws + bp.off_meta);
    int64_t* tile_rows = reinterpret_cast<int64_t*>(ws + bp.off_rows);
    hipLaunchKernelGGL((spmv_tile_rows_kernel<I>),
                       dim3((unsigned)nl2k::ceil_div(bp.n_tiles + 1, kThreads / 64)),
                       dim3(kThreads), 0, stream, ptr, tile_rows, M, nnz, bp.n_tiles);
    st = nl2k::check_launch(who);
    if (st) return st;
    const bool vec = nl2k::aligned16(col) && nl2k::aligned16(vals) &&
                     (dvals == nullptr || nl2k::aligned16(dvals)) &&
                     (Xg == nullptr || nl2k::aligned16(Xg));
    const int dvm = dvals == nullptr ? kDvNone : (Xg != nullptr ? kDvKept : kDvGather);
#define WALK_SORT(VV, DD)                                                                    \
  hipLaunchKernelGGL((spmv_walk_sort_kernel<I, VV, DD>), dim3((unsigned)bp.n_tiles),       \
                     dim3(kSortThreads), 0, stream, ptr, col, vals, X, Xg, dY, dvals, contrib, \
                     low, meta, tile_rows, M, nnz, K, bp.shift, bp.nb)
#define WALK_SORT_DV(VV)                          \
  if (dvm == kDvNone) WALK_SORT(VV, kDvNone);     \
  else if (dvm == kDvKept) WALK_SORT(VV, kDvKept); \
  else WALK_SORT(VV, kDvGather)
    if (vec) { WALK_SORT_DV(true); } else { WALK_SORT_DV(false); }
#undef WALK_SORT_DV
#undef WALK_SORT
    st = nl2k::check_launch(who);
    if (st) return st;
    hipLaunchKernelGGL(spmv_bucket_sum_kernel, dim3((unsigned)bp.nb), dim3(kSumThreads), 0,
                       stream, contrib, low, meta, bp.n_tiles, bp.nb, bp.cols, K, nnz, dX);
    return nl2k::check_launch(who);
  }
  const ColBlockPlan cp = col_block_plan(M, K, D, nnz);
  if (dX && cp.use && nl2k::aligned16(X) && nl2k::aligned16(dY) && nl2k::aligned16(dX)) {
    if (!workspace || ws_bytes < cp.bytes)
      return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                        cp.bytes, workspace ? ws_bytes : (size_t)0);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 256-byte aligned", who);
    return col_block_backward<I>(cp, ptr, col, vals, X, dY, dvals, dX, M, K, D, nnz,
                                 static_cast<char*>(workspace), stream, who);
  }
  const TransposePlan tp = transpose_plan(M, K, D, nnz, sizeof(I));
  if (dX && tp.use) {
    if (!workspace || ws_bytes < tp.bytes)
      return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                        tp.bytes, workspace ? ws_bytes : (size_t)0);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 256-byte aligned", who);
    return transpose_backward<I>(tp, ptr, col, vals, X, dY, dvals, dX, M, K, D, nnz,
                                 static_cast<char*>(workspace), stream, who);
  }
  if (dX) {
    const int64_t n = K * D;
    const unsigned fb = (unsigned)std::min<int64_t>(nl2k::ceil_div(n, kThreads), 4096);
    hipLaunchKernelGGL(spmv_fill_zero_kernel, dim3(fb), dim3(kThreads), 0, stream, dX, n);
    st = nl2k::check_launch(who);
    if (st) return st;
  }
  if (M == 0 || nnz == 0 || (!dX && !dvals)) return nl2k::succeed();
  if (D == 1) {
    const bool vec = nl2k::aligned16(col) && nl2k::aligned16(vals) &&
                     (dvals == nullptr || nl2k::aligned16(dvals)) &&
                     (Xg == nullptr || nl2k::aligned16(Xg));
    return launch_d1_bwd<I>(vec, dvals != nullptr, dX ? kAtomic : kNoDx, stream, ptr, col, vals,
                            X, Xg, dY, dvals, dX, M, K, nnz, who);
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

template <typename I>
int check_structure(const I* ptr, const I* col, int64_t M, int64_t K, int64_t nnz,
                    unsigned long long* report, hipStream_t stream, const char* who) {
  const int64_t imax = sizeof(I) == 4 ? INT32_MAX : INT64_MAX / 2;
  int st = validate(M, K, 1, nnz, imax, who);
  if (st) return st;
  if (!ptr || !report || (nnz > 0 && !col))
    return nl2k::fail(NL2K_ERR_NULL, "%s: row_ptr, col_idx and report must be non-null", who);
  if (!nl2k::aligned16(report))
    return nl2k::fail(NL2K_ERR_ALIGN, "%s: report must be 16-byte aligned", who);
  hipLaunchKernelGGL(spmv_check_init_kernel, dim3(1), dim3(64), 0, stream, report);
  st = nl2k::check_launch(who);
  if (st) return st;
  const int64_t n = std::max<int64_t>(M + 1, nnz);
  const int blocks = (int)std::min<int64_t>(nl2k::ceil_div(n, (int64_t)kThreads), 4096);
  hipLaunchKernelGGL(spmv_check_kernel<I>, dim3(blocks), dim3(kThreads), 0, stream, ptr, col, M,
                     K, nnz, report);
  return nl2k::check_launch(who);
}

}  // namespace

extern "C" {

const char* spmv_last_error(void) { return nl2k::error_slot().text; }

int spmv_check_structure_i32(const int32_t* row_ptr, const int32_t* col_idx, int64_t M,
                             int64_t K, int64_t nnz, uint64_t* report, hipStream_t stream) {
  return check_structure(row_ptr, col_idx, M, K, nnz,
                         reinterpret_cast<unsigned long long*>(report), stream,
                         "spmv_check_structure_i32");
}

int spmv_check_structure_i64(const int64_t* row_ptr, const int64_t* col_idx, int64_t M,
                             int64_t K, int64_t nnz, uint64_t* report, hipStream_t stream) {
  return check_structure(row_ptr, col_idx, M, K, nnz,
                         reinterpret_cast<unsigned long long*>(report), stream,
                         "spmv_check_structure_i64");
}

int spmv_forward_f32_i32(const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                         const float* X, float* Y, int64_t M, int64_t K, int64_t D,
                         int64_t nnz, hipStream_t stream) {
  return forward(row_ptr, col_idx, vals, X, Y, (float*)nullptr, false, M, K, D, nnz, stream,
                 "spmv_forward_f32_i32");
}

int spmv_forward_f32_i64(const int64_t* row_ptr, const int64_t* col_idx, const float* vals,
                         const float* X, float* Y, int64_t M, int64_t K, int64_t D,
                         int64_t nnz, hipStream_t stream) {
  return forward(row_ptr, col_idx, vals, X, Y, (float*)nullptr, false, M, K, D, nnz, stream,
                 "spmv_forward_f32_i64");
}

int spmv_forward_gather_f32_i32(const int32_t* row_ptr, const int32_t* col_idx,
                                const float* vals, const float* X, float* Y, float* Xg,
                                int64_t M, int64_t K, int64_t D, int64_t nnz,
                                hipStream_t stream) {
  return forward(row_ptr, col_idx, vals, X, Y, Xg, true, M, K, D, nnz, stream,
                 "spmv_forward_gather_f32_i32");
}

int spmv_forward_gather_f32_i64(const int64_t* row_ptr, const int64_t* col_idx,
                                const float* vals, const float* X, float* Y, float* Xg,
                                int64_t M, int64_t K, int64_t D, int64_t nnz,
                                hipStream_t stream) {
  return forward(row_ptr, col_idx, vals, X, Y, Xg, true, M, K, D, nnz, stream,
                 "spmv_forward_gather_f32_i64");
}

size_t spmv_backward_workspace_bytes(int64_t M, int64_t K, int64_t D, int64_t nnz) {
  if (validate(M, K, D, nnz, INT64_MAX / 2, "spmv_backward_workspace_bytes")) return 0;
  // the int64-index layout, which also serves int32 indices
  return workspace_bytes_for<int64_t>(M, K, D, nnz);
}

size_t spmv_status_offset(int64_t M, int64_t K, int64_t D, int64_t nnz) {
  if (validate(M, K, D, nnz, INT64_MAX / 2, "spmv_status_offset")) return SIZE_MAX;
  const TransposePlan tp = transpose_plan(M, K, D, nnz, sizeof(int64_t));
  return tp.use ? tp.off_status : SIZE_MAX;
}

int spmv_backward_f32_i32(const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                          const float* X, const float* dY, float* dvals, float* dX,
                          int64_t M, int64_t K, int64_t D, int64_t nnz, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
  return backward(row_ptr, col_idx, vals, X, (const float*)nullptr, false, dY, dvals, dX, M, K,
                  D, nnz, workspace, workspace_bytes, stream, "spmv_backward_f32_i32");
}

int spmv_backward_f32_i64(const int64_t* row_ptr, const int64_t* col_idx, const float* vals,
                          const float* X, const float* dY, float* dvals, float* dX,
                          int64_t M, int64_t K, int64_t D, int64_t nnz, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
  return backward(row_ptr, col_idx, vals, X, (const float*)nullptr, false, dY, dvals, dX, M, K,
                  D, nnz, workspace, workspace_bytes, stream, "spmv_backward_f32_i64");
}

int spmv_backward_gathered_f32_i32(const int32_t* row_ptr, const int32_t* col_idx,
                                   const float* vals, const float* X, const float* Xg,
                                   const float* dY, float* dvals, float* dX, int64_t M,
                                   int64_t K, int64_t D, int64_t nnz, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  return backward(row_ptr, col_idx, vals, X, Xg, true, dY, dvals, dX, M, K, D, nnz, workspace,
                  workspace_bytes, stream, "spmv_backward_gathered_f32_i32");
}

int spmv_backward_gathered_f32_i64(const int64_t* row_ptr, const int64_t* col_idx,
                                   const float* vals, const float* X, const float* Xg,
                                   const float* dY, float* dvals, float* dX, int64_t M,
                                   int64_t K, int64_t D, int64_t nnz, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  return backward(row_ptr, col_idx, vals, X, Xg, true, dY, dvals, dX, M, K, D, nnz, workspace,
                  workspace_bytes, stream, "spmv_backward_gathered_f32_i64");
}

}  // extern "C"
