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
#pragma once

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

}  // namespace slots
}  // namespace nl2k
