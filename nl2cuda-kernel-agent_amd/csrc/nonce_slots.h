// Nonce-tagged 64-bit message slots in a caller's scratch workspace, for
// one launch whose workgroups hand values to each other without a cleared
// workspace, a second launch or a device-scope fence.
//
// Every call draws a fresh 64-bit nonce n on the host (next_key: a
// process-wide counter, never 0, seeded from the clock so a reloaded library
// does not repeat an earlier run's nonces) and two masks m0 and
// m1 = m0 ^ n.  A slot is two words, v ^ m0 and v ^ m1, each written with one
// relaxed agent-scope atomic store (the value is the message, so no fence or
// L2 write-back is needed).  A reader accepts the pair only when the two
// words XOR to n: a slot left complete by an earlier call XORs to that
// call's nonce and a zeroed one to 0, so neither passes; a pair read
// half-written, or never-written memory, passes only by chance (probability
// 2^-64 per read, the masks being hashes of n).
//
// Graph capture: a captured launch keeps the nonce it was captured with, so
// every replay would accept the slots the previous replay left.  Callers
// therefore check `capturing(stream)` and, while it is true, enqueue
// `clear_kernel` over the slots ahead of the launch that uses them (a fill
// kernel, not a memset node): each replay then starts from zeroed pairs,
// which never pass the check.
#pragma once

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdint>

#include <hip/hip_runtime.h>

namespace nl2k {
namespace slots {

// The call's masks (m1 = m0 ^ nonce).
struct Key {
  unsigned long long m0, m1;
};

inline unsigned long long splitmix64(unsigned long long z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// A fresh key per call (host side).
inline Key next_key() {
  static std::atomic<unsigned long long> counter{
      splitmix64((unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count())};
  unsigned long long n = counter.fetch_add(1, std::memory_order_relaxed);
  if (n == 0) n = counter.fetch_add(1, std::memory_order_relaxed);
  const unsigned long long m0 = splitmix64(n ^ 0xD1B54A32D192ED03ull);
  return Key{m0, m0 ^ n};
}

// Publishes the 64 bits b in slot pair p.
__device__ __forceinline__ void publish(unsigned long long* __restrict__ slots, int64_t p,
                                        unsigned long long b, Key key) {
  __hip_atomic_store(slots + 2 * p, b ^ key.m0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(slots + 2 * p + 1, b ^ key.m1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long load_word(const unsigned long long* __restrict__ w) {
  return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True when (w0, w1) is a pair this call published.
__device__ __forceinline__ bool ready(unsigned long long w0, unsigned long long w1, Key key) {
  return (w0 ^ w1) == (key.m0 ^ key.m1);
}

// The published bits of a ready pair.
__device__ __forceinline__ unsigned long long decode(unsigned long long w0, Key key) {
  return w0 ^ key.m0;
}

// Zeroes `nwords` 64-bit words (grid-stride, 16-byte stores; w 16-byte
// aligned).  Internal linkage: each library that includes this header gets
// its own copy.
static __global__ void clear_kernel(unsigned long long* __restrict__ w, int64_t nwords) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 2 * i + 1 < nwords;
       i += stride)
    reinterpret_cast<ulonglong2*>(w)[i] = ulonglong2{0ull, 0ull};
  if ((nwords & 1) && blockIdx.x == 0 && threadIdx.x == 0) w[nwords - 1] = 0ull;
}

// Whether `stream` is being captured into a HIP graph.  Returns a hipError_t
// through `err` when the query itself fails.
inline bool capturing(hipStream_t stream, hipError_t* err) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  *err = hipStreamIsCapturing(stream, &status);
  return *err == hipSuccess && status == hipStreamCaptureStatusActive;
}

// Enqueues clear_kernel over `nwords` words of `w` (8-byte aligned) on
// `stream`; a leading word that breaks 16-byte alignment is cleared by a
// launch of its own.
inline void clear_async(unsigned long long* w, int64_t nwords, hipStream_t stream) {
  if (nwords <= 0) return;
  if (reinterpret_cast<uintptr_t>(w) & 15u) {  // peel one word to reach 16-byte alignment
    hipLaunchKernelGGL(clear_kernel, dim3(1), dim3(64), 0, stream, w, (int64_t)1);
    ++w;
    --nwords;
    if (nwords == 0) return;
  }
  const int64_t pairs = (nwords + 1) / 2;
  const unsigned blocks = (unsigned)std::min<int64_t>((pairs + 255) / 256, 1024);
  hipLaunchKernelGGL(clear_kernel, dim3(blocks), dim3(256), 0, stream, w, nwords);
}

}  // namespace slots
}  // namespace nl2k
