// Peak-rate microbenchmarks for one MI355X (gfx950): the HBM stream rates
// (read, write, copy of float4) and the fp32 MFMA rate with the shader
// clock it ran at.  They confirm, on the box, the published peaks the
// roofline fractions are priced against (8 TB/s HBM, 157.3 TFLOP/s fp32
// matrix).  C-ABI; no state; launches on `stream`.
#include <algorithm>
#include <cstdint>

#include "common.h"

using nl2k::f32x4;

namespace {

constexpr int kBlock = 256;
constexpr int kChains = 8;  // independent MFMA accumulators per wave

// Grid-stride read of n4 float4, U loads in flight per thread step; each
// workgroup writes one sum to sink[blockIdx.x] so the loads stay live.
template <int U>
__global__ __launch_bounds__(kBlock) void peak_read_kernel(const f32x4* __restrict__ src,
                                                           int64_t n4, float* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  f32x4 acc = nl2k::zero4();
  for (; i + (U - 1) * stride < n4; i += U * stride) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += v[u];
  }
  for (; i < n4; i += stride) acc += src[i];
  float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  s = nl2k::wave_sum_dpp(s);
  if (threadIdx.x == 0) sink[blockIdx.x] = s;  // one wave's sum is enough to keep the loads
}

__global__ __launch_bounds__(kBlock) void peak_write_kernel(f32x4* __restrict__ dst, int64_t n4,
                                                            float v) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride)
    dst[i] = f32x4{v, v, v, v};
}

__global__ __launch_bounds__(kBlock) void peak_copy_kernel(const f32x4* __restrict__ src,
                                                           f32x4* __restrict__ dst, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  for (; i + stride < n4; i += 2 * stride) {
    const f32x4 a = src[i], b = src[i + stride];
    dst[i] = a;
    dst[i + stride] = b;
  }
  for (; i < n4; i += stride) dst[i] = src[i];
}

// iters (even) x kChains independent v_mfma_f32_16x16x4f32 per wave (2048
// flops each).  Workgroup 0's first lane records the shader-clock ticks
// (s_memtime) and the 100 MHz real-time ticks (s_memrealtime) of its loop.
__global__ __launch_bounds__(kBlock) void peak_mfma_f32_kernel(float* __restrict__ out,
                                                               unsigned long long* __restrict__ clk,
                                                               int iters) {
  f32x4 acc[kChains];
#pragma unroll
  for (int j = 0; j < kChains; ++j) acc[j] = nl2k::zero4();
  const float a = 1e-3f * (float)(threadIdx.x & 63), b = 1.0f - 1e-4f * (float)(threadIdx.x & 7);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  // unrolled by two: a single-step body gets accumulator copies (VALU work
  // between the MFMAs) from the register allocator
  for (int it = 0; it < iters; it += 2) {
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[j] = nl2k::mfma16x4(a, b, acc[j]);
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[j] = nl2k::mfma16x4(b, a, acc[j]);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kChains; ++j) s += (acc[j][0] + acc[j][1]) + (acc[j][2] + acc[j][3]);
  out[(int64_t)blockIdx.x * kBlock + threadIdx.x] = s;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clk[0] = t1 - t0;
    clk[1] = r1 - r0;
  }
}

// Co-execution of memory staging and fp32 MFMA on one CU.  One workgroup
// of 12 waves per CU (the dynamic LDS allotment keeps it alone there):
// waves 8-11 ("stagers", one per SIMD) stream `tiles` 64 x 64 fp32 tile
// pairs of two [kCoN, kCoN] arrays, the pair of region (blockIdx / 16,
// blockIdx % 16) in the backward's order, 32 KB per CU per tile, each
// through registers into LDS (direct == 0) or straight into LDS
// (global_load_lds_dwordx4, direct == 1), waiting for every tile before the
// next; waves 0-7 (two per SIMD) meanwhile run mfma_iters x 8 independent
// fp32 MFMAs (kind 1: 16x16x4, kind 2: 32x32x2 as 4 chains x 2) or nothing
// (kind 0).  ticks[4 b + w] = 100 MHz ticks of stager w of workgroup b,
// ticks[1024 + 8 b + w] those of MFMA wave w.
constexpr int kCoN = 4096;
constexpr int kCoLds = 96 * 1024;
typedef float f32x16 __attribute__((ext_vector_type(16)));
template <int NS>
__global__ __launch_bounds__(1024) void peak_coexec_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ out,
    unsigned long long* __restrict__ ticks, int tiles, int kind, int mfma_iters, int direct,
    int mfma_waves) {
  extern __shared__ float co_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ri = blockIdx.x / 16, rj = blockIdx.x % 16;
  if (wave < 8 && wave >= mfma_waves) return;  // idle MFMA slot
  if (wave < 8) {
    const unsigned long long m0 = __builtin_amdgcn_s_memrealtime();
    const float a = 1e-3f * (float)lane, b = 1.0f;
    float s = 0.f;
    if (kind == 1) {
      f32x4 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = nl2k::zero4();
      for (int i = 0; i < mfma_iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = nl2k::mfma16x4(a, b, acc[j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += acc[j][0];
    } else if (kind == 2) {
      f32x16 acc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
      for (int i = 0; i < mfma_iters; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b, a, acc[j], 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s += acc[j][0];
    }
    const unsigned long long m1 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0 && blockIdx.x < 256) ticks[2048 + 8 * blockIdx.x + wave] = m1 - m0;
    if (s == 1234.5f) out[0] = s;
    return;
  }
  // NS staging waves share each 64 x 64 tile pair: 64 / NS rows each, as
  // NL = 16 / NS loads of four rows per array
  constexpr int NL = 16 / NS;
  const int w = wave - 8;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < tiles; ++it) {
    const int t = it % 16, ic = t / 4, jc = t % 4;
    const int row0 = ri * 256 + ic * 64 + w * (64 / NS) + (lane >> 4);
    const int col = rj * 256 + jc * 64 + (lane & 15) * 4;
    float* st = co_lds + (it & 1) * 8192 + w * (8192 / NS);
    if (direct) {
#pragma unroll
      for (int s = 0; s < NL; ++s) {
        __builtin_amdgcn_global_load_lds(A + (size_t)(row0 + 4 * s) * kCoN + col, st + s * 256, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(B + (size_t)(row0 + 4 * s) * kCoN + col, st + (NL + s) * 256, 16, 0, 0);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      f32x4 v[2 * NL];
#pragma unroll
      for (int s = 0; s < NL; ++s) {
        v[s] = *reinterpret_cast<const f32x4*>(A + (size_t)(row0 + 4 * s) * kCoN + col);
        v[NL + s] = *reinterpret_cast<const f32x4*>(B + (size_t)(row0 + 4 * s) * kCoN + col);
      }
#pragma unroll
      for (int s = 0; s < 2 * NL; ++s) *reinterpret_cast<f32x4*>(st + s * 256 + lane * 4) = v[s];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (lane == 0 && blockIdx.x < 256) ticks[NS * blockIdx.x + w] = t1 - t0;
  if (co_lds[lane] == 1234.5f) out[1] = co_lds[lane + 64];
}

// Joint-time variant of the co-execution probe: per SIMD, `simd_iters`
// rounds of 8 fp32 16x16x4 MFMA chains split evenly over mfma_waves / 4
// waves (1 or 2 per SIMD), beside one staging wave that streams `tiles`
// 64 x 64 tile pairs straight into LDS with `depth` tile pairs in flight
// (its waits leave the younger tiles' loads outstanding).  ticks[4 b + w]
// gets workgroup b's span from its first wave's start to its last wave's
// end (w = 0), the staging wave's time (w = 1) and the slowest MFMA wave's
// time (w = 2), in 100 MHz ticks.
template <int DEPTH>
__global__ __launch_bounds__(768) void peak_joint_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ out,
    unsigned long long* __restrict__ ticks, int tiles, int simd_iters, int mfma_waves,
    int inline_stage) {
  extern __shared__ float co_lds[];
  __shared__ unsigned long long s_t[12][2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ri = blockIdx.x / 16, rj = blockIdx.x % 16;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  if (inline_stage) {
    // waves 0-3 run all of their SIMD's MFMA rounds and stage their quarter
    // of every tile pair themselves, one tile's loads per simd_iters / tiles
    // rounds, with DEPTH tile pairs in flight
    if (wave < 4) {
      const int w = wave;
      const int per = simd_iters / tiles;
      const float a = 1e-3f * (float)lane, b = 1.0f;
      f32x4 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = nl2k::zero4();
      auto issue = [&](int it) {
        const int t = it % 16, ic = t / 4, jc = t % 4;
        const int row0 = ri * 256 + ic * 64 + w * 16 + (lane >> 4);
        const int col = rj * 256 + jc * 64 + (lane & 15) * 4;
        float* st = co_lds + (it % DEPTH) * 8192 + w * 2048;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          __builtin_amdgcn_global_load_lds(A + (size_t)(row0 + 4 * s2) * kCoN + col, st + s2 * 256, 16, 0, 0);
          __builtin_amdgcn_global_load_lds(B + (size_t)(row0 + 4 * s2) * kCoN + col, st + (4 + s2) * 256, 16, 0, 0);
        }
      };
      for (int it = 0; it < DEPTH - 1 && it < tiles; ++it) issue(it);
      for (int it = 0; it < tiles; ++it) {
        if (it + DEPTH - 1 < tiles) issue(it + DEPTH - 1);
        for (int i = 0; i < per; ++i) {
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] = nl2k::mfma16x4(a, b, acc[j]);
        }
        if (it + DEPTH - 1 < tiles) {
          if constexpr (DEPTH == 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
          else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
      }
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += acc[j][0];
      if (sum == 1234.5f || co_lds[lane] == 1234.5f) out[0] = sum;
    }
  } else if (wave < 8) {
    if (wave < mfma_waves) {
      const int iters = simd_iters / (mfma_waves / 4);
      const float a = 1e-3f * (float)lane, b = 1.0f;
      f32x4 acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = nl2k::zero4();
      for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = nl2k::mfma16x4(a, b, acc[j]);
      }
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += acc[j][0];
      if (sum == 1234.5f) out[0] = sum;
    }
  } else if (wave < 12) {
    const int w = wave - 8;
    auto issue = [&](int it) {
      const int t = it % 16, ic = t / 4, jc = t % 4;
      const int row0 = ri * 256 + ic * 64 + w * 16 + (lane >> 4);
      const int col = rj * 256 + jc * 64 + (lane & 15) * 4;
      float* st = co_lds + (it % DEPTH) * 8192 + w * 2048;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        __builtin_amdgcn_global_load_lds(A + (size_t)(row0 + 4 * s) * kCoN + col, st + s * 256, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(B + (size_t)(row0 + 4 * s) * kCoN + col, st + (4 + s) * 256, 16, 0, 0);
      }
    };
    for (int it = 0; it < DEPTH - 1 && it < tiles; ++it) issue(it);
    for (int it = 0; it < tiles; ++it) {
      if (it + DEPTH - 1 < tiles) {
        issue(it + DEPTH - 1);
        // tile it's 8 loads are the oldest: DEPTH - 1 younger tiles stay out
        if constexpr (DEPTH == 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }
    if (co_lds[lane] == 1234.5f) out[1] = co_lds[lane + 64];
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (lane == 0) {
    s_t[wave][0] = t0;
    s_t[wave][1] = t1;
  }
  __syncthreads();
  if (threadIdx.x == 0 && blockIdx.x < 256) {
    unsigned long long lo = s_t[0][0], hi = s_t[0][1], mf = 0;
    for (int v = 0; v < 12; ++v) {
      lo = s_t[v][0] < lo ? s_t[v][0] : lo;
      hi = s_t[v][1] > hi ? s_t[v][1] : hi;
      const int mw = inline_stage ? 4 : mfma_waves;
      if (v < 8 && v < mw && s_t[v][1] - s_t[v][0] > mf) mf = s_t[v][1] - s_t[v][0];
    }
    ticks[4 * blockIdx.x] = hi - lo;
    ticks[4 * blockIdx.x + 1] = inline_stage ? mf : s_t[8][1] - s_t[8][0];
    ticks[4 * blockIdx.x + 2] = mf;
  }
}

bool bad_stream_args(int64_t n4, int blocks) { return n4 < 1 || blocks < 1 || blocks > (1 << 20); }

}  // namespace

extern "C" {

const char* peaks_last_error(void) { return nl2k::error_slot().text; }

// Stream kernels on `blocks` workgroups of 256 threads.  The read's `sink`
// holds `blocks` floats; `unroll` (4 or 8) is its loads in flight per step.
int peaks_read_f32x4(const float* src, int64_t n4, float* sink, int blocks, int unroll,
                     hipStream_t stream) {
  if (bad_stream_args(n4, blocks) || !src || !sink || (unroll != 4 && unroll != 8))
    return nl2k::fail(NL2K_ERR_SHAPE, "peaks_read_f32x4: bad arguments");
  const f32x4* p = reinterpret_cast<const f32x4*>(src);
  if (unroll == 4)
    hipLaunchKernelGGL(peak_read_kernel<4>, dim3(blocks), dim3(kBlock), 0, stream, p, n4, sink);
  else
    hipLaunchKernelGGL(peak_read_kernel<8>, dim3(blocks), dim3(kBlock), 0, stream, p, n4, sink);
  return nl2k::check_launch("peaks_read_f32x4");
}

int peaks_write_f32x4(float* dst, int64_t n4, int blocks, hipStream_t stream) {
  if (bad_stream_args(n4, blocks) || !dst)
    return nl2k::fail(NL2K_ERR_SHAPE, "peaks_write_f32x4: bad arguments");
  hipLaunchKernelGGL(peak_write_kernel, dim3(blocks), dim3(kBlock), 0, stream,
                     reinterpret_cast<f32x4*>(dst), n4, 1.0f);
  return nl2k::check_launch("peaks_write_f32x4");
}

int peaks_copy_f32x4(const float* src, float* dst, int64_t n4, int blocks, hipStream_t stream) {
  if (bad_stream_args(n4, blocks) || !src || !dst)
    return nl2k::fail(NL2K_ERR_SHAPE, "peaks_copy_f32x4: bad arguments");
  hipLaunchKernelGGL(peak_copy_kernel, dim3(blocks), dim3(kBlock), 0, stream,
                     reinterpret_cast<const f32x4*>(src), reinterpret_cast<f32x4*>(dst), n4);
  return nl2k::check_launch("peaks_copy_f32x4");
}

// Flops one peaks_mfma_f32 launch performs.
double peaks_mfma_f32_flops(int blocks, int iters) {
  return (double)blocks * (kBlock / 64) * iters * kChains * 2.0 * 16 * 16 * 4;
}

// out: blocks * 256 floats; clk: 2 values (shader-clock ticks, 100 MHz ticks).
int peaks_mfma_f32(float* out, unsigned long long* clk, int blocks, int iters,
                   hipStream_t stream) {
  if (blocks < 1 || iters < 2 || iters % 2 != 0 || !out || !clk)
    return nl2k::fail(NL2K_ERR_SHAPE, "peaks_mfma_f32: bad arguments");
  hipLaunchKernelGGL(peak_mfma_f32_kernel, dim3(blocks), dim3(kBlock), 0, stream, out, clk, iters);
  return nl2k::check_launch("peaks_mfma_f32");
}

// Co-execution probe (peak_coexec_kernel): A and B are [4096, 4096] fp32,
// out holds 2 floats, ticks 4096 values; blocks <= 256 (one per CU).
// mfma_waves (4 or 8) of the eight MFMA slots run MFMAs (4: one wave per
// SIMD); stagers (4 or 8) staging waves follow them.
int peaks_coexec(const float* A, const float* B, float* out, unsigned long long* ticks, int blocks,
                 int tiles, int kind, int mfma_iters, int direct, int mfma_waves, int stagers,
                 hipStream_t stream) {
  if (!A || !B || !out || !ticks || blocks < 1 || blocks > 256 || tiles < 1 || kind < 0 ||
      kind > 2 || mfma_iters < 0 || (direct != 0 && direct != 1) ||
      (mfma_waves != 4 && mfma_waves != 8) || (stagers != 4 && stagers != 8))
    return nl2k::fail(NL2K_ERR_SHAPE, "peaks_coexec: bad arguments");
  const void* fn = stagers == 4 ? (const void*)&peak_coexec_kernel<4> : (const void*)&peak_coexec_kernel<8>;
  int st = nl2k::raise_dynamic_lds(fn, kCoLds);
  if (st) return st;
  const dim3 block(64 * (8 + stagers));
  if (stagers == 4)
    hipLaunchKernelGGL(peak_coexec_kernel<4>, dim3(blocks), block, kCoLds, stream, A, B, out, ticks,
                       tiles, kind, mfma_iters, direct, mfma_waves);
  else
    hipLaunchKernelGGL(peak_coexec_kernel<8>, dim3(blocks), block, kCoLds, stream, A, B, out, ticks,
                       tiles, kind, mfma_iters, direct, mfma_waves);
  return nl2k::check_launch("peaks_coexec");
}

// Joint-time probe (peak_joint_kernel): A and B as for peaks_coexec, ticks
// 1024 values; depth 2 or 3 tile pairs in flight; simd_iters even.
// inline_stage: the MFMA waves (4, one per SIMD) stage the tiles themselves
// between their rounds (simd_iters a multiple of tiles) and waves 8-11 idle.
int peaks_joint(const float* A, const float* B, float* out, unsigned long long* ticks, int blocks,
                int tiles, int simd_iters, int mfma_waves, int depth, int inline_stage,
                hipStream_t stream) {
  if (!A || !B || !out || !ticks || blocks < 1 || blocks > 256 || tiles < 1 || simd_iters < 0 ||
      (simd_iters & 1) || (mfma_waves != 0 && mfma_waves != 4 && mfma_waves != 8) ||
      (depth != 2 && depth != 3) || (inline_stage != 0 && inline_stage != 1) ||
      (inline_stage && (mfma_waves != 4 || simd_iters % tiles != 0)))
    return nl2k::fail(NL2K_ERR_SHAPE, "peaks_joint: bad arguments");
  const void* fn = depth == 2 ? (const void*)&peak_joint_kernel<2> : (const void*)&peak_joint_kernel<3>;
  int st = nl2k::raise_dynamic_lds(fn, kCoLds);
  if (st) return st;
  if (depth == 2)
    hipLaunchKernelGGL(peak_joint_kernel<2>, dim3(blocks), dim3(768), kCoLds, stream, A, B, out,
                       ticks, tiles, simd_iters, mfma_waves, inline_stage);
  else
    hipLaunchKernelGGL(peak_joint_kernel<3>, dim3(blocks), dim3(768), kCoLds, stream, A, B, out,
                       ticks, tiles, simd_iters, mfma_waves, inline_stage);
  return nl2k::check_launch("peaks_joint");
}

}  // extern "C"
