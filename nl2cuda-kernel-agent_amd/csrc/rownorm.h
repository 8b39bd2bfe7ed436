// Row normalisation over the last dimension, fp32, for MI355X (gfx950): the
// kernels behind the LayerNorm and L2-norm-scale cases.
//
// A policy P selects the statistics:
//   P::kCentered  subtract the row mean and divide the sum of squares by D
//                 (LayerNorm); otherwise use the raw sum of squares (L2 norm)
//   P::kBias      an additive bias and its gradient
//   P::stat1(rs, ss)  the second per-row statistic the forward writes (rstd
//                 for LayerNorm, the norm sqrt(ss) for L2), ss = the
//                 statistic plus eps; P::rs(stat1) recovers 1 / sqrt(ss)
// and the kernels compute, per row,
//   xh = (x - mu) rs,   y = xh w (+ bias)
//   dx = rs (g - mean_g - xh c),  g = dy w,
//        mean_g = sum(g) / D, c = sum(g xh) / D          (centered)
//        mean_g = 0,          c = sum(g xh)              (L2)
//   dw = sum over rows of dy xh,  dbias = sum of dy.
//
// Design (HBM bound: read x, write y; read dy and x, write dx):
//  * Row-cached path (D % 4 == 0, 16-byte aligned, D <= 16384): TPR threads
//    own a row at a time (16 lanes for rows of at most 128 floats, a wave,
//    or a workgroup of 256 or 512 threads for long rows; the backward uses
//    1024 above 8192 floats) and walk every
//    S-th row with the next one in flight; each thread keeps V float4 of
//    the row in registers, so the row is read from HBM exactly once.
//    Statistics are exact two-pass sums over the registers; reductions are
//    wave64 DPP lane moves (quad_perm and row mirrors within each 16-lane
//    row, then v_readlane across the four rows) plus, for rows wider than a
//    wave, one LDS step across waves.
//  * Backward: each of G workgroups holds H independent row groups (16
//    rows of 16 lanes up to 128 floats, four waves up to 1024, two
//    256-thread groups up to 4096, one 512-thread group above) that walk
//    their rows G row groups apart, prefetching the next row's dy and x
//    while they finish the current one, and accumulate partial dw
//    (/ dbias) in registers; the block adds its groups' partials (in a
//    fixed order) and writes one partial row.  The per-block partials
//    ([G][D]) are summed by rn_colsum_kernel in one stream-ordered pass,
//    every sum in a fixed order, so dw and dbias are deterministic.
//  * Any other shape uses generic kernels that re-read x: one workgroup per
//    row for y / dx, and rn_bwd_generic_partial_kernel (64 columns x a group
//    of rows per block) for the partial rows, then the same column sums.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.h"

namespace nl2k {
namespace rownorm {

constexpr int kBlock = 256;
constexpr int kFwdBlocks = 512;       // row-cached forward blocks (each walks every 512 RPB-th row)
constexpr int kBwdBlocks = 512;       // row-cached backward row groups (256 threads each)
constexpr int kBwdWaveGroups1 = 4096; // row-cached backward wave row groups, rows <= 256 floats
constexpr int kBwdWaveGroups2 = 2048; // ... rows of 257 to 1024 floats
constexpr int kRow16FwdBlocks1 = 2048; // 16-lane-row forward blocks, rows <= 64 floats
constexpr int kRow16FwdBlocks2 = 512;  // ... rows of 65 to 128 floats
constexpr int kRow16BwdBlocks = 512;   // 16-lane-row backward blocks = partial rows
constexpr int kColsumWaves = 16;      // waves of a column-sum workgroup (64 columns)
constexpr int kGenericMaxSplit = 512; // partial rows of the generic path

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b) {
  return (a[0] * b[0] + a[1] * b[1]) + (a[2] * b[2] + a[3] * b[3]);
}
__device__ __forceinline__ float hsum4(f32x4 a) { return (a[0] + a[1]) + (a[2] + a[3]); }

// Sum over the TPR threads that share a row (TPR = 64, 256, 512 or 1024),
// result in all of them.  `red` is LDS scratch of at least 2 * TPR / 64
// floats per row group; with TPR > 64 every thread of the block must take
// part (it holds barriers).  The wave totals are added in a fixed order.
template <int TPR>
__device__ __forceinline__ void row_sum2(float& a, float& b, float* red) {
  static_assert(TPR == 64 || TPR == 256 || TPR == 512 || TPR == 1024, "row width");
  a = wave_sum_dpp(a);
  b = wave_sum_dpp(b);
  if constexpr (TPR > 64) {
    constexpr int W = TPR / 64;
    const int wave = (threadIdx.x >> 6) & (W - 1);  // the wave within the row's threads
    __syncthreads();  // red may still be read from the previous use
    if ((threadIdx.x & 63) == 0) {
      red[wave] = a;
      red[W + wave] = b;
    }
    __syncthreads();
    a = (red[0] + red[1]) + (red[2] + red[3]);
    b = (red[W] + red[W + 1]) + (red[W + 2] + red[W + 3]);
#pragma unroll
    for (int q = 4; q < W; q += 4) {
      a += (red[q] + red[q + 1]) + (red[q + 2] + red[q + 3]);
      b += (red[W + q] + red[W + q + 1]) + (red[W + q + 2] + red[W + q + 3]);
    }
  }
}

template <int TPR>
__device__ __forceinline__ float row_sum1(float a, float* red) {
  float b = 0.f;
  row_sum2<TPR>(a, b, red);
  return a;
}

// ------------------------------------------------------------------ forward
// FULL: D/4 == V * TPR, so every thread's V float4 are in range and the
// loads need no guard (guards become branches that defeat load batching).
// stat0 (the mean) is written only when P::kCentered, bias read only when
// P::kBias.  Row group g (TPR threads; RPB = kBlock / TPR per block) walks
// rows g, g + S, g + 2S, ... (S = the grid's row groups), with the next
// row's loads in flight while it reduces and writes the current one; w and
// bias stay in registers.  At most kFwdBlocks blocks: against one row group
// per row that streamed 47.2 against 44.0 us at [8192, 4096] and 26.6
// against 25.5 us at [16384, 1024], with identical bits.
template <class P, int TPR, int V, bool FULL>
__global__ __launch_bounds__(TPR > kBlock ? TPR : kBlock) void rn_fwd_kernel(
    const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y,
    float* __restrict__ stat0, float* __restrict__ stat1, int64_t B,
    int D, float eps) {
  constexpr int BS = TPR > kBlock ? TPR : kBlock;  // block size (TPR = 512: one row group)
  __shared__ float red[TPR >= 256 ? 2 * (TPR / 64) : 1];
  constexpr int RPB = BS / TPR;
  const int64_t S = (int64_t)gridDim.x * RPB;
  // The row group is wave uniform: from lane 0, so rows and row pointers
  // stay scalar (buffer resources need them so).
  const int64_t r0 =
      (int64_t)blockIdx.x * RPB + __builtin_amdgcn_readfirstlane((int)threadIdx.x) / TPR;
  const int t = threadIdx.x % TPR;
  const int D4 = D >> 2;
  // TPR >= 256: the grid has at most B blocks, so a whole block walks the
  // same rows and takes the reductions' barriers together.  TPR = 64: a row
  // group past the end leaves (its reductions stay inside its wave).
  if (r0 >= B) return;
  const int64_t rlast = r0 + (B - 1 - r0) / S * S;
  const f32x4* w4 = reinterpret_cast<const f32x4*>(w);
  const f32x4* b4 = reinterpret_cast<const f32x4*>(bias);
  f32x4 wv[V], bv[V], cur[V], nxt[V];
  // Ragged rows (not FULL) load and store through a buffer resource over
  // the row: lanes past its end read zeros and write nothing, with no
  // branch, so the count of memory operations in flight stays the same on
  // every path and the loop waits only for the loads it uses.
  auto load_row = [&](int64_t r, f32x4 (&v)[V]) {
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + r * D);
    const buffer_rsrc rx = make_rsrc(x + r * D, (uint32_t)D * 4u);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int c = t + k * TPR;
      v[k] = FULL ? xr[c] : buffer_load4(rx, (uint32_t)c * 16u, 0);
    }
  };
  load_row(r0, cur);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int c = FULL ? t + k * TPR : min(t + k * TPR, D4 - 1);
    wv[k] = w4[c];
    if constexpr (P::kBias) bv[k] = b4[c];
  }
  const float inv_d = 1.f / (float)D;
  for (int64_t r = r0; r < B; r += S) {
    // Unconditional prefetch (the last row re-reads itself), so the number
    // of loads in flight does not depend on the path.
    load_row(min(r + S, rlast), nxt);
    float mu = 0.f;
    if constexpr (P::kCentered) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) s += hsum4(cur[k]);
      mu = row_sum1<TPR>(s, red) * inv_d;
    }
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int c = t + k * TPR;
      if (FULL || c < D4) {
        const f32x4 dv = cur[k] - mu;
        q += dot4(dv, dv);
      }
    }
    const float ss = row_sum1<TPR>(q, red) * (P::kCentered ? inv_d : 1.f) + eps;
    const float rs = 1.f / sqrtf(ss);
    if (t == 0) {
      if constexpr (P::kCentered) stat0[r] = mu;
      stat1[r] = P::stat1(rs, ss);
    }
    f32x4* yr = reinterpret_cast<f32x4*>(y + r * D);
    const buffer_rsrc ry = make_rsrc(y + r * D, (uint32_t)D * 4u);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int c = t + k * TPR;
      f32x4 yv = (cur[k] - mu) * rs * wv[k];
      if constexpr (P::kBias) yv += bv[k];
      if (FULL)
        yr[c] = yv;
      else
        buffer_store4(ry, yv, (uint32_t)c * 16u, 0);
    }
#pragma unroll
    for (int k = 0; k < V; ++k) cur[k] = nxt[k];
  }
}

// Generic forward: one workgroup per row, any D and alignment.
template <class P>
__global__ __launch_bounds__(kBlock) void rn_fwd_generic_kernel(
    const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y,
    float* __restrict__ stat0, float* __restrict__ stat1, int64_t D, float eps) {
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * D;
  float mu = 0.f;
  if constexpr (P::kCentered) {
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < D; c += kBlock) s += xr[c];
    mu = row_sum1<kBlock>(s, red) / (float)D;
  }
  float q = 0.f;
  for (int64_t c = threadIdx.x; c < D; c += kBlock) {
    const float d = xr[c] - mu;
    q = fmaf(d, d, q);
  }
  const float ss = row_sum1<kBlock>(q, red) / (P::kCentered ? (float)D : 1.f) + eps;
  const float rs = 1.f / sqrtf(ss);
  if (threadIdx.x == 0) {
    if constexpr (P::kCentered) stat0[row] = mu;
    stat1[row] = P::stat1(rs, ss);
  }
  for (int64_t c = threadIdx.x; c < D; c += kBlock) {
    if constexpr (P::kBias)
      y[row * D + c] = (xr[c] - mu) * rs * w[c] + bias[c];
    else
      y[row * D + c] = (xr[c] - mu) * rs * w[c];
  }
}

// ----------------------------------------------------------------- backward
// Level 1: block b of G is H row groups of TPR threads (V float4 per
// thread); group h walks rows b + h G, b + h G + S, b + h G + 2S, ... (S =
// H G rows per sweep), one row at a time, and the block writes the sum of
// its groups' partial dw (/ dbias) rows (groups 0, 1, ... added in that
// order) to pw[b] (/ pb[b]).  All groups take the same number of steps,
// group 0's row count, so they pass the same barriers; a group whose row
// lies past the end runs the step on a clamped row and keeps nothing of it.
// Shapes: TPR = 64 (a wave per row, H = 4) for rows of 129 to 1024 floats,
// TPR = 256 (H = 2) up to 4096, TPR = 512 (H = 1) above; shorter rows take
// rn_bwd_row16_kernel.
//  * The strided row order keeps the concurrent reads and writes of all
//    blocks inside one window of about S consecutive rows of each array;
//    contiguous blocks of rows per block scattered them G row blocks apart
//    and streamed about 10 % slower (72.6 against 65.0 us at 8192 x 4096).
//  * Two 256-thread halves per block (V = 2 and 4) halve the partial rows for the same
//    waves per SIMD: whole backward 70.3 against 71.8 us at 8192 x 4096,
//    42.5 against 45.3 at 8192 x 2048.
//  * Rows longer than 4096 floats take 512 threads per row with V = 4
//    float4 each.  With 256 threads a thread holds eight float4 of each of
//    seven row arrays, which leaves one wave per SIMD.
//  * Rows of at most 1024 floats take a wave each (reductions inside the
//    wave, no barrier per row): with 256 threads per row, most of them
//    idle at D = 256, every row paid two workgroup barriers for 1 KB.
template <class P, int TPR, int V, bool FULL, int H>
__global__ __launch_bounds__(TPR * H) void rn_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ stat0,
    const float* __restrict__ stat1, float* __restrict__ dx,
    float* __restrict__ pw, float* __restrict__ pb, int64_t B, int D) {
  static_assert((TPR == 64 && H == 4) || (TPR == 256 && (H == 1 || H == 2)) ||
                    ((TPR == 512 || TPR == 1024) && H == 1),
                "block shape");
  constexpr int kRed = TPR > 64 ? 2 * (TPR / 64) : 1;  // LDS floats per group's row sums
  __shared__ float red[kRed * H];
  constexpr int kParts = P::kBias ? 2 : 1;
  constexpr int kPart = kParts * TPR * V;  // f32x4 of one group's partial rows
  __shared__ f32x4 s_part[H > 1 ? (H - 1) * kPart : 1];  // groups 1 .. H-1
  // The group is wave uniform: take it from lane 0 so that rows, row
  // pointers and the row predicate stay scalar.
  const int hf = H > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x) / TPR : 0;
  const int t = threadIdx.x % TPR;
  const int D4 = D >> 2;
  const int64_t G = gridDim.x;  // G <= B: every block's half 0 has a row
  const int64_t S = (int64_t)H * G;
  const int64_t r0 = (int64_t)blockIdx.x + hf * G;
  const int64_t nk = (B - 1 - (int64_t)blockIdx.x) / S + 1;  // steps: half 0's rows
  // This half's last row (B - 1 for a half with no row at all): the row the
  // prefetch is clamped to, so the last step re-reads a row it already has.
  const int64_t rlast = r0 < B ? r0 + (B - 1 - r0) / S * S : B - 1;
  const f32x4* w4 = reinterpret_cast<const f32x4*>(w);

  // TPR = 1024 (a block of 16 waves, at most 128 registers a lane) keeps w
  // in LDS, each thread its own entries, so that the prefetch fits.
  constexpr bool kWLds = TPR == 1024;
  __shared__ f32x4 s_w[kWLds ? TPR * V : 1];
  f32x4 wv[V], aw[V], ab[V], gcur[V], xcur[V], gnext[V], xnext[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int c = t + k * TPR;
    const f32x4 wk = w4[FULL ? c : min(c, D4 - 1)];
    if constexpr (kWLds)
      s_w[c] = (FULL || c < D4) ? wk : zero4();
    else
      wv[k] = (FULL || c < D4) ? wk : zero4();
    aw[k] = zero4();
    ab[k] = zero4();
  }
  auto w_at = [&](int k) { return kWLds ? s_w[t + k * TPR] : wv[k]; };
  // Ragged rows load through buffer resources (zeros past the row's end,
  // no branch; see the store below).
  auto load_row = [&](int64_t r, f32x4 (&g)[V], f32x4 (&xv)[V]) {
    const f32x4* dyr = reinterpret_cast<const f32x4*>(dy + r * D);
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + r * D);
    const buffer_rsrc rg = make_rsrc(dy + r * D, (uint32_t)D * 4u);
    const buffer_rsrc rx = make_rsrc(x + r * D, (uint32_t)D * 4u);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int c = t + k * TPR;
      g[k] = FULL ? dyr[c] : buffer_load4(rg, (uint32_t)c * 16u, 0);
      xv[k] = FULL ? xr[c] : buffer_load4(rx, (uint32_t)c * 16u, 0);
    }
  };
  load_row(min(r0, rlast), gcur, xcur);
  const float inv_d = 1.f / (float)D;
  int64_t r = r0;
  for (int64_t k = 0; k < nk; ++k, r += S) {
    const bool has = H == 1 || r < B;  // false only on half 1's extra step
    const int64_t rr = has ? r : B - 1;
    // Unconditional prefetch (the last row re-reads itself): a conditional
    // one makes the number of loads in flight path dependent and the
    // compiler then waits for all of them before using the current row.
    load_row(min(r + S, rlast), gnext, xnext);
    const float mu = P::kCentered ? stat0[rr] : 0.f;
    const float rs = P::rs(stat1[rr]);
    float sg = 0.f, sgx = 0.f;
    f32x4 xh[V];
#pragma unroll
    for (int k2 = 0; k2 < V; ++k2) {
      xh[k2] = (xcur[k2] - mu) * rs;
      const f32x4 g = gcur[k2] * w_at(k2);
      if constexpr (P::kCentered) sg += hsum4(g);
      sgx += dot4(g, xh[k2]);
    }
    if (has) {
#pragma unroll
      for (int k2 = 0; k2 < V; ++k2) {
        aw[k2] += gcur[k2] * xh[k2];
        if constexpr (P::kBias) ab[k2] += gcur[k2];
      }
    }
    float mg = 0.f, mgx;
    if constexpr (P::kCentered) {
      row_sum2<TPR>(sg, sgx, red + kRed * hf);
      mg = sg * inv_d;
      mgx = sgx * inv_d;
    } else {
      mgx = row_sum1<TPR>(sgx, red + kRed * hf);
    }
    {
      // One unconditional store per float4: the resource spans the row (none
      // of it without a row), so the column tail and a half's missing row
      // write nothing.  A store under a branch would make the count of
      // memory operations in flight path dependent, and the compiler then
      // waits for this row's stores before it uses the next row's loads.
      const buffer_rsrc rdx = make_rsrc(dx + rr * D, has ? (uint32_t)D * 4u : 0u);
#pragma unroll
      for (int k2 = 0; k2 < V; ++k2) {
        const int c = t + k2 * TPR;
        buffer_store4(rdx, rs * (gcur[k2] * w_at(k2) - mg - xh[k2] * mgx), (uint32_t)c * 16u, 0);
      }
    }
#pragma unroll
    for (int k2 = 0; k2 < V; ++k2) {
      gcur[k2] = gnext[k2];
      xcur[k2] = xnext[k2];
    }
  }
  if constexpr (H > 1) {
    if (hf > 0) {
      f32x4* sp = s_part + (hf - 1) * kPart;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        sp[t + k * TPR] = aw[k];
        if constexpr (P::kBias) sp[TPR * V + t + k * TPR] = ab[k];
      }
    }
    __syncthreads();
    if (hf > 0) return;
#pragma unroll
    for (int j = 0; j < H - 1; ++j) {
      const f32x4* sp = s_part + j * kPart;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        aw[k] += sp[t + k * TPR];
        if constexpr (P::kBias) ab[k] += sp[TPR * V + t + k * TPR];
      }
    }
  }
  f32x4* pw4 = reinterpret_cast<f32x4*>(pw + (int64_t)blockIdx.x * D);
  f32x4* pb4 = reinterpret_cast<f32x4*>(pb + (int64_t)blockIdx.x * D);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int c = t + k * TPR;
    if (FULL || c < D4) {
      pw4[c] = aw[k];
      if constexpr (P::kBias) pb4[c] = ab[k];
    }
  }
}

// ------------------------------------------- rows of at most 128 floats
__device__ __forceinline__ float row16_sum(float v) { return row16_sum_dpp(v); }

// Rows of at most 128 floats (V = 1 or 2 float4 per lane) take 16 lanes
// each: four consecutive rows per wave, 16 per block.  Block b walks row
// sets b, b + G, b + 2G, ... (16 rows each) with the next set's loads in
// flight.  Loads and stores go through buffer resources over the wave's
// rows that exist (the first min(4, B - row) of its four), and a lane past
// its row's end has an offset outside any of them: loads read zeros,
// stores write nothing, and no memory operation sits under a branch or
// depends on a per-step select (the compiler turns such a select into a
// branch).  With a wave per row, 48 of 64 lanes idled at D = 64.
constexpr uint32_t kOutside = 0x7FFFFFF0u;  // past any resource used here; no 32-bit wrap

template <class P, int V>
__global__ __launch_bounds__(kBlock) void rn_fwd_row16_kernel(
    const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ bias, float* __restrict__ y,
    float* __restrict__ stat0, float* __restrict__ stat1, int64_t B,
    int D, float eps) {
  constexpr int RPB = kBlock / 16;
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4;  // the lane's row among the wave's four
  const int t = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x) >> 6;
  const int D4 = D >> 2;
  const int64_t S = (int64_t)gridDim.x * RPB;
  const int64_t rw0 = (int64_t)blockIdx.x * RPB + 4 * wave;  // the wave's first row
  if (rw0 >= B) return;  // wave uniform; no barriers below
  const int64_t rwl = rw0 + (B - 1 - rw0) / S * S;       // its last row set
  const uint32_t rbytes = (uint32_t)D * 4u;
  auto rows = [&](int64_t rw) { return (uint32_t)min(B - rw, (int64_t)4); };
  const f32x4* w4 = reinterpret_cast<const f32x4*>(w);
  const f32x4* b4 = reinterpret_cast<const f32x4*>(bias);
  uint32_t off[V];
  f32x4 wv[V], bv[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int c = t + 16 * k;
    off[k] = c < D4 ? (uint32_t)j * rbytes + (uint32_t)c * 16u : kOutside;
    wv[k] = w4[min(c, D4 - 1)];
    if constexpr (P::kBias) bv[k] = b4[min(c, D4 - 1)];
  }
  const uint32_t soff = t == 0 ? (uint32_t)j * 4u : kOutside;
  auto load = [&](int64_t rw, f32x4 (&v)[V]) {
    const buffer_rsrc r = make_rsrc(x + rw * D, rows(rw) * rbytes);
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] = buffer_load4(r, off[k], 0);
  };
  f32x4 cur[V], nxt[V];
  load(rw0, cur);
  const float inv_d = 1.f / (float)D;
  for (int64_t rw = rw0; rw < B; rw += S) {
    load(min(rw + S, rwl), nxt);  // the last set re-reads itself
    // keep the next set's loads ahead of all work on this one
    __builtin_amdgcn_sched_barrier(0);
    float mu = 0.f;
    if constexpr (P::kCentered) {
      float sx = 0.f;
#pragma unroll
      for (int k = 0; k < V; ++k) sx += hsum4(cur[k]);  // zeros past the row
      mu = row16_sum(sx) * inv_d;
    }
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const f32x4 dv = cur[k] - mu;
      q += t + 16 * k < D4 ? dot4(dv, dv) : 0.f;
    }
    const float ss = row16_sum(q) * (P::kCentered ? inv_d : 1.f) + eps;
    const float rs = 1.f / sqrtf(ss);
    const uint32_t n = rows(rw);
    if constexpr (P::kCentered) buffer_store1(make_rsrc(stat0 + rw, 4u * n), mu, soff, 0);
    buffer_store1(make_rsrc(stat1 + rw, 4u * n), P::stat1(rs, ss), soff, 0);
    const buffer_rsrc ry = make_rsrc(y + rw * D, n * rbytes);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      f32x4 yv = (cur[k] - mu) * rs * wv[k];
      if constexpr (P::kBias) yv += bv[k];
      buffer_store4(ry, yv, off[k], 0);
    }
#pragma unroll
    for (int k = 0; k < V; ++k) cur[k] = nxt[k];
  }
}

// Backward for the same rows: the layout of rn_fwd_row16_kernel, with the
// row statistics loaded beside the row data (a row set ahead); partial dw
// (/ dbias) in registers per lane.  At the end the four row groups of a
// wave are added by two lane exchanges (16 apart, then 32 apart) and the
// four waves in LDS (0 + 1 + 2 + 3), and the block writes one partial row.
template <class P, int V>
__global__ __launch_bounds__(kBlock) void rn_bwd_row16_kernel(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ stat0,
    const float* __restrict__ stat1, float* __restrict__ dx,
    float* __restrict__ pw, float* __restrict__ pb, int64_t B, int D) {
  constexpr int RPB = kBlock / 16;
  constexpr int kParts = P::kBias ? 2 : 1;
  constexpr int kPart = kParts * 16 * V;  // f32x4 of one wave's partial rows
  __shared__ f32x4 s_part[3 * kPart];     // waves 1 .. 3
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4;
  const int t = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x) >> 6;
  const int D4 = D >> 2;
  const int64_t S = (int64_t)gridDim.x * RPB;
  const int64_t rw0 = (int64_t)blockIdx.x * RPB + 4 * wave;
  const uint32_t rbytes = (uint32_t)D * 4u;
  auto rows = [&](int64_t rw) { return (uint32_t)min(B - rw, (int64_t)4); };
  const f32x4* w4 = reinterpret_cast<const f32x4*>(w);
  uint32_t off[V];
  f32x4 wv[V], aw[V], ab[V];
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int c = t + 16 * k;
    off[k] = c < D4 ? (uint32_t)j * rbytes + (uint32_t)c * 16u : kOutside;
    const f32x4 wk = w4[min(c, D4 - 1)];
    wv[k] = c < D4 ? wk : zero4();
    aw[k] = zero4();
    ab[k] = zero4();
  }
  const uint32_t soff = (uint32_t)j * 4u;
  if (rw0 < B) {  // wave uniform: a wave past the end only adds zeros below
    const int64_t rwl = rw0 + (B - 1 - rw0) / S * S;
    struct Set {
      f32x4 g[V], xv[V];
      float s0, s1;
    };
    auto load = [&](int64_t rw, Set& q) {
      const uint32_t n = rows(rw);
      const buffer_rsrc rg = make_rsrc(dy + rw * D, n * rbytes);
      const buffer_rsrc rx = make_rsrc(x + rw * D, n * rbytes);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        q.g[k] = buffer_load4(rg, off[k], 0);
        q.xv[k] = buffer_load4(rx, off[k], 0);
      }
      q.s0 = P::kCentered ? buffer_load1(make_rsrc(stat0 + rw, 4u * n), soff, 0) : 0.f;
      q.s1 = buffer_load1(make_rsrc(stat1 + rw, 4u * n), soff, 0);
    };
    Set cur, nxt;
    load(rw0, cur);
    const float inv_d = 1.f / (float)D;
    for (int64_t rw = rw0; rw < B; rw += S) {
      load(min(rw + S, rwl), nxt);
      __builtin_amdgcn_sched_barrier(0);  // the next set's loads ahead of this set's work
      const bool ok = (uint32_t)j < rows(rw);
      const float mu = cur.s0;
      const float rs = P::rs(cur.s1);
      float sg = 0.f, sgx = 0.f;
      f32x4 xh[V];
#pragma unroll
      for (int k = 0; k < V; ++k) {
        xh[k] = (cur.xv[k] - mu) * rs;
        const f32x4 g = cur.g[k] * wv[k];
        if constexpr (P::kCentered) sg += hsum4(g);
        sgx += dot4(g, xh[k]);
      }
      const float mg = P::kCentered ? row16_sum(sg) * inv_d : 0.f;
      const float mgx = row16_sum(sgx) * (P::kCentered ? inv_d : 1.f);
      const buffer_rsrc rdx = make_rsrc(dx + rw * D, rows(rw) * rbytes);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        buffer_store4(rdx, rs * (cur.g[k] * wv[k] - mg - xh[k] * mgx), off[k], 0);
        // a row past B has no statistics (zeros, possibly an infinite rs):
        // select, so that nothing of it reaches the partial sums
        aw[k] = ok ? aw[k] + cur.g[k] * xh[k] : aw[k];
        if constexpr (P::kBias) ab[k] = ok ? ab[k] + cur.g[k] : ab[k];
      }
      cur = nxt;
    }
  }
  // The wave's four row groups hold the same columns: add them across lanes.
#pragma unroll
  for (int k = 0; k < V; ++k) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      aw[k][e] += __shfl_xor(aw[k][e], 16, 64);
      aw[k][e] += __shfl_xor(aw[k][e], 32, 64);
      if constexpr (P::kBias) {
        ab[k][e] += __shfl_xor(ab[k][e], 16, 64);
        ab[k][e] += __shfl_xor(ab[k][e], 32, 64);
      }
    }
  }
  if (wave > 0 && j == 0) {
    f32x4* sp = s_part + (wave - 1) * kPart;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      sp[t + 16 * k] = aw[k];
      if constexpr (P::kBias) sp[16 * V + t + 16 * k] = ab[k];
    }
  }
  __syncthreads();
  if (wave > 0 || j > 0) return;
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const f32x4* sp = s_part + q * kPart;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      aw[k] += sp[t + 16 * k];
      if constexpr (P::kBias) ab[k] += sp[16 * V + t + 16 * k];
    }
  }
  f32x4* pw4 = reinterpret_cast<f32x4*>(pw + (int64_t)blockIdx.x * D);
  f32x4* pb4 = reinterpret_cast<f32x4*>(pb + (int64_t)blockIdx.x * D);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int c = t + 16 * k;
    if (c < D4) {
      pw4[c] = aw[k];
      if constexpr (P::kBias) pb4[c] = ab[k];
    }
  }
}

// Generic backward (any D / alignment): one workgroup per row writes dx;
// rn_bwd_generic_partial_kernel then forms the partial parameter rows.
template <class P>
__global__ __launch_bounds__(kBlock) void rn_bwd_generic_kernel(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ stat0,
    const float* __restrict__ stat1, float* __restrict__ dx, int64_t D) {
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const float mu = P::kCentered ? stat0[row] : 0.f;
  const float rs = P::rs(stat1[row]);
  float sg = 0.f, sgx = 0.f;
  for (int64_t c = threadIdx.x; c < D; c += kBlock) {
    const float xh = (x[row * D + c] - mu) * rs;
    const float g = dy[row * D + c] * w[c];
    sg += g;
    sgx = fmaf(g, xh, sgx);
  }
  float mg = 0.f, mgx;
  if constexpr (P::kCentered) {
    row_sum2<kBlock>(sg, sgx, red);
    mg = sg / (float)D;
    mgx = sgx / (float)D;
  } else {
    mgx = row_sum1<kBlock>(sgx, red);
  }
  for (int64_t c = threadIdx.x; c < D; c += kBlock) {
    const float xh = (x[row * D + c] - mu) * rs;
    dx[row * D + c] = rs * (dy[row * D + c] * w[c] - mg - xh * mgx);
  }
}

// Partial parameter rows for the generic path.  Block (cs, g) covers the
// 64 columns [64 cs, 64 cs + 64) and rows [g per, min(B, (g + 1) per)); wave
// w takes rows a + w, a + w + 4, ... and the four waves combine in LDS, in a
// fixed order, into pw[g] (and pb[g]).
template <class P>
__global__ __launch_bounds__(kBlock) void rn_bwd_generic_partial_kernel(
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ stat0, const float* __restrict__ stat1, int64_t B,
    int64_t D, int64_t per, float* __restrict__ pw, float* __restrict__ pb) {
  __shared__ float sw[4][64], sb[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t cc = min(c, D - 1);
  const int64_t a = (int64_t)blockIdx.y * per, e = min(B, a + per);
  float aw = 0.f, ab = 0.f;
#pragma unroll 4
  for (int64_t r = a + wave; r < e; r += 4) {
    const float g = dy[r * D + cc];
    const float mu = P::kCentered ? stat0[r] : 0.f;
    aw = fmaf(g, (x[r * D + cc] - mu) * P::rs(stat1[r]), aw);
    ab += g;
  }
  sw[wave][lane] = aw;
  sb[wave][lane] = ab;
  __syncthreads();
  if (wave == 0 && c < D) {
    pw[blockIdx.y * D + c] = (sw[0][lane] + sw[1][lane]) + (sw[2][lane] + sw[3][lane]);
    if constexpr (P::kBias)
      pb[blockIdx.y * D + c] = (sb[0][lane] + sb[1][lane]) + (sb[2][lane] + sb[3][lane]);
  }
}

// dw[c] (and dbias[c]) = sum over the R partial rows of column c.  A
// workgroup of 16 waves owns 64 columns: wave w sums rows w, w + 16, ... of
// its lane's column, eight loads in flight per batch, and the 16 wave sums
// combine in LDS in a fixed order.  One pass: a second launch of a small
// kernel costs about 4 us of launch and drain on this part, more than the
// partial rows take to read.  Stream order makes the partial rows visible.
template <bool TWO>
__global__ __launch_bounds__(64 * kColsumWaves) void rn_colsum_kernel(
    const float* __restrict__ in_w, const float* __restrict__ in_b, int64_t R, int64_t D,
    float* __restrict__ out_w, float* __restrict__ out_b) {
  __shared__ float sw[kColsumWaves][64], sb[kColsumWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t cc = min(c, D - 1);
  float aw = 0.f, ab = 0.f;
  int64_t r = wave;
  for (; r + 7 * kColsumWaves < R; r += 8 * kColsumWaves) {
    float vw[8], vb[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      vw[k] = in_w[(r + k * kColsumWaves) * D + cc];
      if constexpr (TWO) vb[k] = in_b[(r + k * kColsumWaves) * D + cc];
    }
    __builtin_amdgcn_sched_barrier(0);  // the batch's loads issue before the adds
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      aw += vw[k];
      if constexpr (TWO) ab += vb[k];
    }
  }
  for (; r < R; r += kColsumWaves) {
    aw += in_w[r * D + cc];
    if constexpr (TWO) ab += in_b[r * D + cc];
  }
  sw[wave][lane] = aw;
  if constexpr (TWO) sb[wave][lane] = ab;
  __syncthreads();
  if (wave == 0 && c < D) {
    float tw = 0.f, tb = 0.f;
#pragma unroll
    for (int w = 0; w < kColsumWaves; ++w) {
      tw += sw[w][lane];
      if constexpr (TWO) tb += sb[w][lane];
    }
    out_w[c] = tw;
    if constexpr (TWO) out_b[c] = tb;
  }
}

__global__ __launch_bounds__(kBlock) void rn_fill_zero_kernel(float* __restrict__ a,
                                                             float* __restrict__ b,
                                                             int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock) {
    a[i] = 0.f;
    if (b) b[i] = 0.f;
  }
}

// ----------------------------------------------------------------- planning
struct Plan {
  bool cached = false;  // row-cached vector path
  int tpr = 256;        // forward threads per row
  int v = 4;            // float4 per thread
  int btpr = 256;       // backward (cached): threads per row
  int bv = 1;           // backward (cached): float4 per thread
  int bh = 1;           // backward (cached): row groups per block
  int64_t G = 0;        // partial rows of dw / dbias
  int64_t rpb = 0;      // generic path: rows per partial group
};

// Row groups of at most `target` with ceil(B / target) rows each.
inline int64_t row_groups(int64_t B, int64_t target) {
  return ceil_div(B, std::max<int64_t>(1, ceil_div(B, target)));
}

inline Plan plan(int64_t B, int64_t D, bool aligned) {
  Plan p;
  p.cached = aligned && D % 4 == 0 && D <= 16384;
  if (!p.cached) {
    // ~2048 blocks of 64 columns x (B / S1) rows
    const int64_t slices = ceil_div(D, 64);
    const int64_t s1 = std::min<int64_t>(
        std::min<int64_t>(std::max<int64_t>(1, ceil_div(2048, slices)), kGenericMaxSplit),
        std::max<int64_t>(B, 1));
    p.rpb = std::max<int64_t>(1, ceil_div(B, s1));
    p.G = B > 0 ? ceil_div(B, p.rpb) : 0;
    return p;
  }
  const int64_t d4 = D / 4;
  if (d4 <= 32) {  // 16 lanes per row, both directions
    p.tpr = p.btpr = 16;
    p.v = p.bv = d4 <= 16 ? 1 : 2;
    p.bh = 16;
    p.G = B > 0 ? std::min<int64_t>(ceil_div(B, 16), kRow16BwdBlocks) : 0;
    return p;
  }
  if (d4 <= 64) {
    p.tpr = 64;
    p.v = 1;
  } else if (d4 <= 256) {
    p.tpr = 64;
    p.v = (int)ceil_div(d4, 64);  // 2, 3 or 4
  } else if (d4 <= 2048) {
    p.tpr = 256;
    p.v = d4 <= 512 ? 2 : d4 <= 1024 ? 4 : 8;
  } else {  // one 512-thread row group per block
    p.tpr = 512;
    p.v = 8;
  }
  if (B == 0) return p;
  if (d4 <= 256) {  // a wave per row, four per block
    p.btpr = 64;
    p.bv = d4 <= 64 ? 1 : d4 <= 128 ? 2 : d4 <= 192 ? 3 : 4;
    p.bh = 4;
    p.G = ceil_div(row_groups(B, p.bv == 1 ? kBwdWaveGroups1 : kBwdWaveGroups2), 4);
  } else {
    // 512-thread blocks (two halves, or 512 threads per row above 4096
    // floats) fill a CU's two waves per SIMD alone, as do 1024-thread
    // blocks (above 8192 floats) its four: half as many blocks, so that all
    // of them are resident at once.
    if (d4 <= 1024) {
      p.bv = d4 <= 512 ? 2 : 4;
      p.bh = 2;
    } else {
      p.btpr = d4 <= 2048 ? 512 : 1024;
      p.bv = 4;
    }
    p.G = ceil_div(row_groups(B, kBwdBlocks), 2);
  }
  return p;
}

// Workspace: the partial rows, n G D floats (n = 2 with a bias, else 1).
template <class P>
size_t workspace_floats(int64_t D, const Plan& p) {
  const int64_t n = P::kBias ? 2 : 1;
  return (size_t)(n * p.G * D);
}

template <class P>
size_t backward_workspace_bytes(int64_t B, int64_t D) {
  // Pointer alignment picks the path at call time: cover both.
  const size_t cached = workspace_floats<P>(D, plan(B, D, true));
  const size_t generic = workspace_floats<P>(D, plan(B, D, false));
  return std::max(cached, generic) * sizeof(float);
}

// ----------------------------------------------------------------- launches
// Forward launch for B >= 1 (the caller validated sizes and pointers).
template <class P>
int run_forward(const float* x, const float* w, const float* bias, float* y, float* stat0,
                float* stat1, int64_t B, int64_t D, float eps, hipStream_t stream,
                const char* who) {
  const bool aligned = aligned16(x) && aligned16(w) && (!P::kBias || aligned16(bias)) &&
                       aligned16(y);
  const Plan p = plan(B, D, aligned);
  if (p.cached && p.tpr == 16) {
    const dim3 grid((unsigned)std::min<int64_t>(
        ceil_div(B, 16), p.v == 1 ? kRow16FwdBlocks1 : kRow16FwdBlocks2));
    if (p.v == 1)
      hipLaunchKernelGGL((rn_fwd_row16_kernel<P, 1>), grid, dim3(kBlock), 0, stream, x, w, bias,
                         y, stat0, stat1, B, (int)D, eps);
    else
      hipLaunchKernelGGL((rn_fwd_row16_kernel<P, 2>), grid, dim3(kBlock), 0, stream, x, w, bias,
                         y, stat0, stat1, B, (int)D, eps);
    return check_launch(who);
  }
  if (p.cached && p.tpr == 512) {  // one 512-thread row group per block
    const dim3 grid((unsigned)std::min<int64_t>(B, kFwdBlocks));
    if (D == 512 * 4 * 8)
      hipLaunchKernelGGL((rn_fwd_kernel<P, 512, 8, true>), grid, dim3(512), 0, stream, x, w, bias,
                         y, stat0, stat1, B, (int)D, eps);
    else
      hipLaunchKernelGGL((rn_fwd_kernel<P, 512, 8, false>), grid, dim3(512), 0, stream, x, w,
                         bias, y, stat0, stat1, B, (int)D, eps);
    return check_launch(who);
  }
  if (p.cached) {
    const int rpb = kBlock / p.tpr;
    const dim3 grid((unsigned)std::min<int64_t>(ceil_div(B, rpb), kFwdBlocks));
#define RN_FWD(TPR, V)                                                                      \
  do {                                                                                       \
    if (D / 4 == (TPR) * (V))                                                                \
      hipLaunchKernelGGL((rn_fwd_kernel<P, TPR, V, true>), grid, dim3(kBlock), 0, stream, x,  \
                         w, bias, y, stat0, stat1, B, (int)D, eps);                          \
    else                                                                                     \
      hipLaunchKernelGGL((rn_fwd_kernel<P, TPR, V, false>), grid, dim3(kBlock), 0, stream, x, \
                         w, bias, y, stat0, stat1, B, (int)D, eps);                          \
  } while (0)
    if (p.tpr == 64 && p.v == 1) RN_FWD(64, 1);
    else if (p.tpr == 64 && p.v == 2) RN_FWD(64, 2);
    else if (p.tpr == 64 && p.v == 3) RN_FWD(64, 3);
    else if (p.tpr == 64) RN_FWD(64, 4);
    else if (p.v == 2) RN_FWD(256, 2);
    else if (p.v == 4) RN_FWD(256, 4);
    else RN_FWD(256, 8);
#undef RN_FWD
    return check_launch(who);
  }
  hipLaunchKernelGGL(rn_fwd_generic_kernel<P>, dim3((unsigned)B), dim3(kBlock), 0, stream, x, w,
                     bias, y, stat0, stat1, D, eps);
  return check_launch(who);
}

// Zero parameter gradients for an empty batch.
inline int fill_zero(float* a, float* b, int64_t D, hipStream_t stream, const char* who) {
  hipLaunchKernelGGL(rn_fill_zero_kernel,
                     dim3((unsigned)std::min<int64_t>(ceil_div(D, kBlock), 1024)), dim3(kBlock),
                     0, stream, a, b, D);
  return check_launch(who);
}

// Backward launches for B >= 1 (the caller validated sizes, pointers and the
// workspace size / alignment against backward_workspace_bytes).
template <class P>
int run_backward(const float* dy, const float* x, const float* w, const float* stat0,
                 const float* stat1, float* dx, float* dw, float* dbias, int64_t B,
                 int64_t D, float* ws, hipStream_t stream, const char* who) {
  const bool aligned = aligned16(dy) && aligned16(x) && aligned16(w) && aligned16(dx);
  const Plan p = plan(B, D, aligned);
  float* pw = ws;
  float* pb = pw + p.G * D;
  int st;
  if (p.cached) {
#define RN_BWD(TPR, V, H)                                                                     \
  do {                                                                                        \
    if (D / 4 == (TPR) * (V))                                                                 \
      hipLaunchKernelGGL((rn_bwd_kernel<P, TPR, V, true, H>), dim3((unsigned)p.G),            \
                         dim3((TPR) * (H)), 0, stream, dy, x, w, stat0, stat1, dx, pw, pb, B, \
                         (int)D);                                                             \
    else                                                                                      \
      hipLaunchKernelGGL((rn_bwd_kernel<P, TPR, V, false, H>), dim3((unsigned)p.G),           \
                         dim3((TPR) * (H)), 0, stream, dy, x, w, stat0, stat1, dx, pw, pb, B, \
                         (int)D);                                                             \
  } while (0)
    if (p.btpr == 16 && p.bv == 1)
      hipLaunchKernelGGL((rn_bwd_row16_kernel<P, 1>), dim3((unsigned)p.G), dim3(kBlock), 0,
                         stream, dy, x, w, stat0, stat1, dx, pw, pb, B, (int)D);
    else if (p.btpr == 16)
      hipLaunchKernelGGL((rn_bwd_row16_kernel<P, 2>), dim3((unsigned)p.G), dim3(kBlock), 0,
                         stream, dy, x, w, stat0, stat1, dx, pw, pb, B, (int)D);
    else if (p.btpr == 64 && p.bv == 1) RN_BWD(64, 1, 4);
    else if (p.btpr == 64 && p.bv == 2) RN_BWD(64, 2, 4);
    else if (p.btpr == 64 && p.bv == 3) RN_BWD(64, 3, 4);
    else if (p.btpr == 64) RN_BWD(64, 4, 4);
    else if (p.bv == 2) RN_BWD(256, 2, 2);
    else if (p.btpr == 256) RN_BWD(256, 4, 2);
    else if (p.btpr == 512) RN_BWD(512, 4, 1);
    else RN_BWD(1024, 4, 1);
#undef RN_BWD
    st = check_launch(who);
  } else {
    hipLaunchKernelGGL(rn_bwd_generic_kernel<P>, dim3((unsigned)B), dim3(kBlock), 0, stream, dy,
                       x, w, stat0, stat1, dx, D);
    st = check_launch(who);
    if (st) return st;
    hipLaunchKernelGGL(rn_bwd_generic_partial_kernel<P>,
                       dim3((unsigned)ceil_div(D, 64), (unsigned)p.G), dim3(kBlock), 0, stream,
                       dy, x, stat0, stat1, B, D, p.rpb, pw, pb);
    st = check_launch(who);
  }
  if (st) return st;
  hipLaunchKernelGGL((rn_colsum_kernel<P::kBias>), dim3((unsigned)ceil_div(D, 64)),
                     dim3(64 * kColsumWaves), 0, stream, pw, pb, p.G, D, dw, dbias);
  return check_launch(who);
}

}  // namespace rownorm
}  // namespace nl2k
