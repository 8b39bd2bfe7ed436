// Shared host/device helpers for the HIP kernels of every case library.
//
// Host side: a thread-local "last error" buffer, argument-check helpers that
// run before any HIP call, and a launch check that turns a failed launch into
// NL2K_ERR_HIP with the runtime's message.
// Device side: 16-byte vector types, wave64 reductions and MFMA wrappers for
// gfx950 (CDNA4).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <utility>

#include "nl2k_status.h"

namespace nl2k {

// ---------------------------------------------------------------- host side
struct ErrorSlot {
  char text[512];
};

inline ErrorSlot& error_slot() {
  static thread_local ErrorSlot slot = {{0}};
  return slot;
}

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(error_slot().text, sizeof(error_slot().text), fmt, ap);
  va_end(ap);
  return code;
}

inline int succeed() {
  error_slot().text[0] = '\0';
  return NL2K_SUCCESS;
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(NL2K_ERR_HIP, "%s: kernel launch failed: %s", what,
                hipGetErrorString(e));
  return succeed();
}

inline int check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return fail(NL2K_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return NL2K_SUCCESS;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroups of `kernel` (launched with `threads` threads and no dynamic LDS)
// that the current device holds at once: its CU count times the occupancy
// the runtime computes from the kernel's registers, LDS and launch bounds.
// Cached per (device, kernel), so instantiations with equal signatures but
// different register counts keep their own figures.
// Raises `kernel`'s dynamic LDS limit to at least `bytes` on the current
// device.  The attribute call is made once per (device, kernel) and size
// increase; later calls, captured into a graph or not, make none.
inline int raise_dynamic_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> set;
  int dev = 0;
  int st = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (st) return st;
  std::lock_guard<std::mutex> lock(mu);
  int& have = set[{dev, kernel}];
  if (bytes <= have) return NL2K_SUCCESS;
  st = check_hip(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes),
                 "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
  if (!st) have = bytes;
  return st;
}

inline int resident_blocks(const void* kernel, int threads, int* out) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  int dev = 0;
  int st = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (st) return st;
  {
    std::lock_guard<std::mutex> lock(mu);
    const auto it = cache.find({dev, kernel});
    if (it != cache.end()) {
      *out = it->second;
      return NL2K_SUCCESS;
    }
  }
  int cus = 0, per_cu = 0;
  st = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
                 "hipDeviceGetAttribute(MultiprocessorCount)");
  if (st) return st;
  st = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0),
                 "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  if (st) return st;
  const int n = std::max(1, cus) * std::max(1, per_cu);
  std::lock_guard<std::mutex> lock(mu);
  cache[{dev, kernel}] = n;
  *out = n;
  return NL2K_SUCCESS;
}

// -------------------------------------------------------------- device side
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 load4(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}

__device__ __forceinline__ void store4(float* p, f32x4 v) {
  *reinterpret_cast<f32x4*>(p) = v;
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Raw buffer resource over `bytes` bytes at `base` (stride 0, gfx9 dword 3:
// 32-bit data format).  A load through it takes a per-lane byte offset in a
// vector register and a wave-uniform one in a scalar register, so a tile's
// address costs no vector instructions; a lane offset at or past `bytes`
// reads zeros.  The bound is checked against the lane offset: a caller that
// relies on it to drop ragged lanes passes wave_off = 0 (every such caller
// here does), and a nonzero wave_off is only for accesses known in range.
typedef __amdgpu_buffer_rsrc_t buffer_rsrc;

__device__ __forceinline__ buffer_rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ f32x4 buffer_load4(buffer_rsrc r, uint32_t lane_off, int wave_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, wave_off, 0));
}

// Store through a raw buffer resource: a lane whose offset is at or past the
// resource's `bytes` writes nothing, so a store that only some lanes (or, with
// bytes = 0, no lane) may make is still one unconditional instruction.
__device__ __forceinline__ void buffer_store4(buffer_rsrc r, f32x4 v, uint32_t lane_off,
                                              int wave_off) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, lane_off, wave_off, 0);
}

__device__ __forceinline__ float buffer_load1(buffer_rsrc r, uint32_t lane_off, int wave_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane_off, wave_off, 0));
}

__device__ __forceinline__ void buffer_store1(buffer_rsrc r, float v, uint32_t lane_off,
                                              int wave_off) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, lane_off, wave_off, 0);
}

// One 16x16x4 fp32 MFMA: acc[m][n] += sum_k A[m][k] * B[k][n].
// Lane l supplies A[l%16][l/16] in `a` and B[l/16][l%16] in `b`; the result
// element [4*(l/16)+r][l%16] lives in register r of lane l.
__device__ __forceinline__ f32x4 mfma16x4(float a, float b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
}

// Sum over all 64 lanes of a wave (result in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Wave reductions through DPP lane moves instead of LDS permutes: the row
// of 16 lanes is reduced with quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror and row_mirror (every lane then holds its row's result),
// and the four rows are combined from lanes 0, 16, 32 and 48 with
// v_readlane.  The result is wave-uniform.  Every lane of the wave must be
// active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  const int i = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(i, i, CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum / max over each 16-lane row of the wave, result in all 16 lanes (the
// first four steps of the wave reductions below).  Every lane of the row
// gets the same bits: each step combines the same two partial results, in
// one order or the other.
__device__ __forceinline__ float row16_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return v;
}

__device__ __forceinline__ float row16_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  return v;
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace nl2k
