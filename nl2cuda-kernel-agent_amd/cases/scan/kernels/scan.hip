// Inclusive prefix sums along the last dimension for MI355X (gfx950).
// C-ABI in include/scan.h.
//
// Reference semantics: cases/scan/reference.py:8-9 (torch.cumsum over the
// last dim; autograd backward = reverse cumsum, description.md:6-15); the
// reference kernel (scan.cu:23-64) handles float32 rows of exactly 4096 with
// one CUB block scan per row.  torch's CPU cumsum of float32 accumulates in
// float64; this build does the same (fp64 VALU work is far below the memory
// time), and integer input is summed exactly in int64.
//
// Design (HBM bound: read x once, write y once):
//  * A row is cut into chunks of CE = T * 4096 elements (T = 1 unless a row
//    would need more than 256 chunks).  A workgroup of 4 waves scans a
//    4096-element tile: wave w owns elements [1024 w, 1024 w + 1024), lane l
//    holds four consecutive elements per group k at 256 k + 4 l (each load
//    instruction of a wave reads 1 KiB contiguous).  Per tile: each lane's
//    group total, a wave64 DPP scan of those totals per group (row_shr
//    1/2/4/8, row_bcast 15/31, wave_shr 1 for the exclusive prefix), wave
//    totals combined in LDS; outputs are the carry-in plus a serial sum
//    through the lane's four raw values.  Registers hold the raw inputs, so
//    four workgroups fit per CU (the residency the grid cap relies on).
//  * Rows of one chunk need nothing else.  Otherwise each chunk publishes
//    its total (one relaxed 64-bit agent-scope atomic store: the value is the
//    message, so no fence and no L2 write-back is needed) and then sums the
//    totals of the chunks before it in its row, in a fixed order, as its
//    carry-in.  A chunk waits only for totals, never for another chunk's
//    carry, so there is no serial chain; sums are deterministic.  The grid
//    is capped at the resident workgroup count of the current device (CU
//    count x the occupancy the runtime reports for this kernel), and each
//    workgroup walks its chunks in increasing order and publishes before it
//    waits, so the lowest unpublished chunk can always make progress.  A
//    spin cap ends a wait that never completes (a CU-masked queue can hold
//    fewer workgroups than the device reports): the chunk then uses a zero
//    carry and adds 1 to the workspace's trailing trip counter, which the
//    library never clears and callers may zero and read.
//  * Slots need no clearing, so a call is a single launch and the workspace
//    needs no initial contents: the slots are tagged with a fresh 64-bit
//    nonce per call (csrc/nonce_slots.h), and a reader takes only pairs this
//    call wrote.  While the stream is being captured into a graph the call
//    enqueues a fill kernel over the slots first, so that replays, which
//    reuse the captured nonce, never read an earlier replay's slots.
//  * Rows of at most 2048 elements take scan_short_kernel (16 lanes or a
//    wave per row, no messages).
//  * Reverse scans mirror the positions: logical p <-> physical D - 1 - p.
#include <algorithm>
#include <cstdint>

#include "../../../csrc/common.h"
#include "../../../csrc/nonce_slots.h"
#include "scan.h"

using nl2k::f32x4;
using nl2k::i32x4;

namespace {

typedef long long i64x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kGroups = 4;                      // 4-element groups per lane per tile
constexpr int kTile = kThreads * 4 * kGroups;   // 4096 elements
constexpr int kWaveSpan = 64 * 4 * kGroups;     // 1024 elements per wave
constexpr int64_t kMaxChunks = 256;             // chunks per row
constexpr unsigned kSpinLimit = 1u << 24;       // hang guard for the carry wait
constexpr int64_t kShortMax = 2048;             // rows up to this take scan_short_kernel
constexpr int64_t kShortBlocks = 2048;          // its most workgroups

// ------------------------------------------------ 64-bit accumulator helpers
using SlotKey = nl2k::slots::Key;

template <typename T>
__device__ __forceinline__ unsigned long long bits64(T v) {
  return __builtin_bit_cast(unsigned long long, v);
}
template <typename T>
__device__ __forceinline__ T from_bits64(unsigned long long b) {
  return __builtin_bit_cast(T, b);
}

// DPP move of a 64-bit value; lanes whose source is outside the pattern
// (or outside row_mask) read 0, the additive identity.
template <int kCtrl, int kRowMask, typename T>
__device__ __forceinline__ T dpp64(T v) {
  const unsigned long long b = bits64(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, kCtrl, kRowMask, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), kCtrl, kRowMask, 0xF,
                                             false);
  return from_bits64<T>(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Inclusive scan over the 64 lanes of a wave.
template <typename T>
__device__ __forceinline__ T wave_scan(T v) {
  v += dpp64<0x111, 0xF>(v);  // row_shr:1
  v += dpp64<0x112, 0xF>(v);  // row_shr:2
  v += dpp64<0x114, 0xF>(v);  // row_shr:4
  v += dpp64<0x118, 0xF>(v);  // row_shr:8
  v += dpp64<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp64<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

template <typename T>
__device__ __forceinline__ T lane_value(T v, int lane) {
  const unsigned long long b = bits64(v);
  const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)b, lane);
  const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
  return from_bits64<T>(((unsigned long long)hi << 32) | lo);
}

// Sum over all lanes (butterfly: every lane gets the same bits).
template <typename T>
__device__ __forceinline__ T wave_total(T v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ------------------------------------------------------- element transport
// Logical positions p..p+3 of a row as stored (zero past D), in two steps so
// that a tile's four group loads are all in flight before any is used:
// issue() only loads (clamped address, no branch), finish() masks and
// reverses.  Applying the mask right after each load made the compiler
// reuse one register quad and wait for every load in turn.  VEC: D % 4 == 0
// and 16-byte aligned rows, so a group is one 16-byte load.
template <typename In, bool REV, bool VEC>
struct RawGroup;
template <typename In, bool REV>
struct RawGroup<In, REV, true> {
  typedef In V4 __attribute__((ext_vector_type(4)));
  V4 w;
  __device__ __forceinline__ void issue(const In* __restrict__ row, int64_t D, int64_t p) {
    const int64_t q = REV ? D - 4 - min(p, D - 4) : min(p, D - 4);
    w = *reinterpret_cast<const V4*>(row + q);
  }
  __device__ __forceinline__ void finish(int64_t D, int64_t p, In (&a)[4]) const {
    const bool in = p < D;
#pragma unroll
    for (int c = 0; c < 4; ++c) a[c] = in ? w[REV ? 3 - c : c] : (In)0;
  }
};
template <typename In, bool REV>
struct RawGroup<In, REV, false> {
  In v[4];
  __device__ __forceinline__ void issue(const In* __restrict__ row, int64_t D, int64_t p) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int64_t pc = p + c;
      v[c] = row[REV ? D - 1 - min(pc, D - 1) : min(pc, D - 1)];
    }
  }
  __device__ __forceinline__ void finish(int64_t D, int64_t p, In (&a)[4]) const {
#pragma unroll
    for (int c = 0; c < 4; ++c) a[c] = p + c < D ? v[c] : (In)0;
  }
};

// The four groups of one lane in a tile: positions p0 + 256 k.
template <typename In, bool REV, bool VEC>
__device__ __forceinline__ void load_tile(const In* __restrict__ row, int64_t D, int64_t p0,
                                          In (&a)[kGroups][4]) {
  RawGroup<In, REV, VEC> g[kGroups];
#pragma unroll
  for (int k = 0; k < kGroups; ++k) g[k].issue(row, D, p0 + 256 * k);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < kGroups; ++k) g[k].finish(D, p0 + 256 * k, a[k]);
}

template <typename Out, bool REV, bool VEC, typename Acc>
__device__ __forceinline__ void store_group(Out* __restrict__ row, int64_t D, int64_t p,
                                            const Acc (&v)[4]) {
  if (p >= D) return;
  if (VEC) {
    const int64_t q = REV ? D - 4 - p : p;
    Out o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = (Out)v[REV ? 3 - c : c];
    if constexpr (__is_same(Out, float)) {
      *reinterpret_cast<f32x4*>(row + q) = f32x4{o[0], o[1], o[2], o[3]};
    } else if constexpr (__is_same(Out, int32_t)) {
      *reinterpret_cast<i32x4*>(row + q) = i32x4{o[0], o[1], o[2], o[3]};
    } else {
      *reinterpret_cast<i64x2*>(row + q) = i64x2{o[0], o[1]};
      *reinterpret_cast<i64x2*>(row + q + 2) = i64x2{o[2], o[3]};
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int64_t pc = p + c;
      if (pc < D) row[REV ? D - 1 - pc : pc] = (Out)v[c];
    }
  }
}

// --------------------------------------------------------------- the scan
// One tile's scan state: the raw values, and per group the sum of all
// elements of the wave before this lane's group (fp64 / int64).
template <typename In, typename Acc>
struct TileScan {
  In a[kGroups][4];
  Acc off[kGroups];
  Acc wave_sum;  // total of this wave's 1024 elements
};

template <typename In, typename Acc>
__device__ __forceinline__ void scan_registers(TileScan<In, Acc>& s) {
  Acc run = (Acc)0;
#pragma unroll
  for (int k = 0; k < kGroups; ++k) {
    const Acc t = (((Acc)s.a[k][0] + (Acc)s.a[k][1]) + (Acc)s.a[k][2]) + (Acc)s.a[k][3];
    const Acc incl = wave_scan(t);
    const Acc excl = dpp64<0x138, 0xF>(incl);  // wave_shr:1, lane 0 reads 0
    s.off[k] = run + excl;
    run += lane_value(incl, 63);
  }
  s.wave_sum = run;
}

// Writes one tile: element c of group k is base + off[k] + a[k][0..c].
template <typename In, typename Out, typename Acc, bool REV, bool VEC>
__device__ __forceinline__ void emit_tile(const TileScan<In, Acc>& s, Acc base, Out* __restrict__ yr,
                                          int64_t D, int64_t p0) {
#pragma unroll
  for (int k = 0; k < kGroups; ++k) {
    Acc v[4];
    Acc r = base + s.off[k];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      r += (Acc)s.a[k][c];
      v[c] = r;
    }
    store_group<Out, REV, VEC>(yr, D, p0 + 256 * k, v);
  }
}

// Publishes a chunk total in slot pair p (csrc/nonce_slots.h).
template <typename Acc>
__device__ __forceinline__ void publish(unsigned long long* __restrict__ slots, int p, Acc v,
                                        SlotKey key) {
  nl2k::slots::publish(slots, p, bits64(v), key);
}

// Sum of the totals of chunks [0, chunk) of a row, in a fixed order (wave 0).
template <typename Acc>
__device__ Acc carry_in(const unsigned long long* __restrict__ slots, int chunk, int lane,
                        SlotKey key, unsigned* __restrict__ err) {
  Acc carry = (Acc)0;
  for (int base = 0; base < chunk; base += 64) {
    const int p = base + lane;
    Acc v = (Acc)0;
    if (p < chunk) {
      unsigned long long w0 = nl2k::slots::load_word(slots + 2 * p);
      unsigned long long w1 = nl2k::slots::load_word(slots + 2 * p + 1);
      unsigned spins = 0;
      while (!nl2k::slots::ready(w0, w1, key)) {
        if (++spins > kSpinLimit) {  // never expected: report and give up
          __hip_atomic_fetch_add(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          w0 = key.m0;  // reads as 0
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        w0 = nl2k::slots::load_word(slots + 2 * p);
        w1 = nl2k::slots::load_word(slots + 2 * p + 1);
      }
      v = from_bits64<Acc>(nl2k::slots::decode(w0, key));
    }
    carry += wave_total(v);
  }
  return carry;
}

// Inclusive scan over each 16-lane row of the wave (row_shr steps only).
template <typename T>
__device__ __forceinline__ T row16_scan(T v) {
  v += dpp64<0x111, 0xF>(v);  // row_shr:1
  v += dpp64<0x112, 0xF>(v);  // row_shr:2
  v += dpp64<0x114, 0xF>(v);  // row_shr:4
  v += dpp64<0x118, 0xF>(v);  // row_shr:8
  return v;
}

// Rows of at most 2048 elements: RL lanes per row (16 up to 256 elements,
// 64 above), G 4-element groups per lane at positions 4 (t + RL k), so each
// load instruction of a row group reads RL x 16 contiguous bytes.  A row
// group walks every S-th row (S = the grid's row groups); rows need no
// messages, the carry across a row's groups being an RL-lane scan of the
// group totals, in a fixed order.  With a 4096-element tile per row, most
// of the tile was empty: 151 us for 65536 x 64.
template <typename In, typename Out, typename Acc, bool REV, bool VEC, int RL, int G>
__global__ __launch_bounds__(kThreads) void scan_short_kernel(const In* __restrict__ x,
                                                              Out* __restrict__ y, int64_t rows,
                                                              int64_t D) {
  static_assert(RL == 16 || RL == 64, "row group width");
  constexpr int RPB = kThreads / RL;
  const int lane = threadIdx.x & 63;
  const int t = threadIdx.x % RL;
  const int64_t S = (int64_t)gridDim.x * RPB;
  // A row group (16 lanes, or the wave) runs its rows together; groups of
  // one wave may take different row counts, and a DPP step only reads
  // lanes of its own group.
  for (int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / RL; r < rows; r += S) {
    const In* xr = x + r * D;
    Out* yr = y + r * D;
    RawGroup<In, REV, VEC> g[G];
#pragma unroll
    for (int k = 0; k < G; ++k) g[k].issue(xr, D, 4 * (int64_t)(t + RL * k));
    __builtin_amdgcn_sched_barrier(0);
    In a[G][4];
#pragma unroll
    for (int k = 0; k < G; ++k) g[k].finish(D, 4 * (int64_t)(t + RL * k), a[k]);
    Acc run = (Acc)0;
#pragma unroll
    for (int k = 0; k < G; ++k) {
      const Acc tot = (((Acc)a[k][0] + (Acc)a[k][1]) + (Acc)a[k][2]) + (Acc)a[k][3];
      Acc incl, excl, all;
      if constexpr (RL == 16) {
        incl = row16_scan(tot);
        excl = dpp64<0x111, 0xF>(incl);  // row_shr:1, the row's lane 0 reads 0
        all = __shfl(incl, lane | 15, 64);
      } else {
        incl = wave_scan(tot);
        excl = dpp64<0x138, 0xF>(incl);  // wave_shr:1, lane 0 reads 0
        all = lane_value(incl, 63);
      }
      Acc v[4];
      Acc q = run + excl;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        q += (Acc)a[k][c];
        v[c] = q;
      }
      store_group<Out, REV, VEC>(yr, D, 4 * (int64_t)(t + RL * k), v);
      run += all;
    }
  }
}

template <typename In, typename Out, typename Acc, bool REV, bool VEC>
__global__ __launch_bounds__(kThreads, 4) void scan_rows_kernel(
    const In* __restrict__ x, Out* __restrict__ y, int64_t D, int nchunk, int tiles,
    int64_t total_chunks, unsigned long long* __restrict__ slots, SlotKey key,
    unsigned* __restrict__ err) {
  __shared__ Acc s_wave[2][4];
  __shared__ Acc s_carry;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t chunk_elems = (int64_t)tiles * kTile;
  int phase = 0;  // alternates the s_wave buffer between uses

  for (int64_t t = blockIdx.x; t < total_chunks; t += gridDim.x) {
    const int64_t row = t / nchunk;
    const int chunk = (int)(t - row * nchunk);
    const In* xr = x + row * D;
    Out* yr = y + row * D;
    const int64_t c0 = chunk * chunk_elems;
    const int64_t lane_off = (int64_t)wave * kWaveSpan + 4 * lane;

    TileScan<In, Acc> s;
    Acc chunk_total;
    if (tiles == 1) {
      load_tile<In, REV, VEC>(xr, D, c0 + lane_off, s.a);
      scan_registers(s);
      if (lane == 0) s_wave[phase][wave] = s.wave_sum;
      __syncthreads();
      chunk_total = (s_wave[phase][0] + s_wave[phase][1]) + (s_wave[phase][2] + s_wave[phase][3]);
    } else {
      // Pass 1: the chunk total only (the chunk is re-read below, from L2).
      Acc part = (Acc)0;
      for (int tt = 0; tt < tiles; ++tt) {
        In a[kGroups][4];
        load_tile<In, REV, VEC>(xr, D, c0 + tt * kTile + lane_off, a);
#pragma unroll
        for (int k = 0; k < kGroups; ++k)
          part += (((Acc)a[k][0] + (Acc)a[k][1]) + (Acc)a[k][2]) + (Acc)a[k][3];
      }
      part = wave_total(part);
      if (lane == 0) s_wave[phase][wave] = part;
      __syncthreads();
      chunk_total = (s_wave[phase][0] + s_wave[phase][1]) + (s_wave[phase][2] + s_wave[phase][3]);
    }

    Acc carry = (Acc)0;
    if (nchunk > 1) {
      unsigned long long* row_slots = slots + 2 * row * nchunk;
      if (wave == 0) {
        if (lane == 0 && chunk + 1 < nchunk) publish<Acc>(row_slots, chunk, chunk_total, key);
        const Acc c = carry_in<Acc>(row_slots, chunk, lane, key, err);
        if (lane == 0) s_carry = c;
      }
      __syncthreads();
      carry = s_carry;
    }

    if (tiles == 1) {
      Acc wave_off = (Acc)0;
      for (int w = 0; w < wave; ++w) wave_off += s_wave[phase][w];
      emit_tile<In, Out, Acc, REV, VEC>(s, carry + wave_off, yr, D, c0 + lane_off);
    } else {
      // Pass 2: scan tile by tile with a running carry.
      Acc run = carry;
      for (int tt = 0; tt < tiles; ++tt) {
        phase ^= 1;
        load_tile<In, REV, VEC>(xr, D, c0 + tt * kTile + lane_off, s.a);
        scan_registers(s);
        if (lane == 0) s_wave[phase][wave] = s.wave_sum;
        __syncthreads();
        Acc wave_off = (Acc)0;
        for (int w = 0; w < wave; ++w) wave_off += s_wave[phase][w];
        emit_tile<In, Out, Acc, REV, VEC>(s, run + wave_off, yr, D, c0 + tt * kTile + lane_off);
        run += (s_wave[phase][0] + s_wave[phase][1]) + (s_wave[phase][2] + s_wave[phase][3]);
      }
    }
    phase ^= 1;
    // s_carry and the other s_wave buffer are rewritten only after the next
    // chunk's first barrier, which every wave reaches after finishing here.
  }
}

// ----------------------------------------------------------------- planning
struct Plan {
  int nchunk = 1;
  int tiles = 1;
  int64_t total = 0;   // chunks over all rows
  int64_t slots = 0;   // workspace slots (0: single-chunk rows)
};

Plan plan(int64_t rows, int64_t D) {
  Plan p;
  const int64_t tiles_per_row = nl2k::ceil_div(D, kTile);
  p.tiles = (int)std::max<int64_t>(1, nl2k::ceil_div(tiles_per_row, kMaxChunks));
  p.nchunk = (int)nl2k::ceil_div(tiles_per_row, p.tiles);
  p.total = rows * p.nchunk;
  p.slots = p.nchunk > 1 ? p.total : 0;
  return p;
}

size_t workspace_bytes(const Plan& p) {
  // a two-word slot per chunk, then one 8-byte word (hang-guard counter)
  return p.slots > 0 ? (size_t)p.slots * 16 + 8 : 0;
}

// Workgroups a launch uses: every chunk at once when rows are single chunks
// (nothing waits); otherwise at most `resident`, the count that can be on the
// device together.
int64_t launch_grid(const Plan& p, int64_t resident) {
  if (p.nchunk == 1) return std::min<int64_t>(p.total, INT32_MAX);
  return std::max<int64_t>(1, std::min<int64_t>(p.total, resident));
}



int validate(int64_t rows, int64_t D, const char* who) {
  if (rows < 0 || D < 1)
    return nl2k::fail(NL2K_ERR_SHAPE, "%s: need rows >= 0 and D >= 1 (got rows=%lld D=%lld)",
                      who, (long long)rows, (long long)D);
  if (D > INT32_MAX || rows > INT32_MAX || rows > INT64_MAX / D)
    return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: sizes too large (rows=%lld D=%lld)", who,
                      (long long)rows, (long long)D);
  return NL2K_SUCCESS;
}

template <typename In, typename Out, typename Acc, bool REV>
int run(const In* x, Out* y, int64_t rows, int64_t D, void* workspace, size_t ws_bytes,
        hipStream_t stream, const char* who) {
  int st = validate(rows, D, who);
  if (st) return st;
  if (rows == 0) return nl2k::succeed();
  if (!x || !y) return nl2k::fail(NL2K_ERR_NULL, "%s: null pointer argument", who);
  const Plan p = plan(rows, D);
  unsigned long long* slots = nullptr;
  unsigned* err = nullptr;
  SlotKey key{0, 0};
  if (p.slots > 0) {
    const size_t need = workspace_bytes(p);
    if (!workspace || ws_bytes < need)
      return nl2k::fail(NL2K_ERR_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", who,
                        need, workspace ? ws_bytes : (size_t)0);
    if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0)
      return nl2k::fail(NL2K_ERR_ALIGN, "%s: workspace must be 8-byte aligned", who);
    slots = static_cast<unsigned long long*>(workspace);
    err = reinterpret_cast<unsigned*>(slots + 2 * p.slots);
    key = nl2k::slots::next_key();
  }
  const bool vec = D % 4 == 0 && nl2k::aligned16(x) && nl2k::aligned16(y);
  if (D <= kShortMax) {
    const int rl = D <= 256 ? 16 : 64;
    const int64_t grid = std::min<int64_t>(nl2k::ceil_div(rows, (int64_t)(kThreads / rl)), kShortBlocks);
#define SCAN_SHORT(RL, G)                                                                    \
  do {                                                                                       \
    if (vec)                                                                                 \
      hipLaunchKernelGGL((scan_short_kernel<In, Out, Acc, REV, true, RL, G>),                \
                         dim3((unsigned)grid), dim3(kThreads), 0, stream, x, y, rows, D);    \
    else                                                                                     \
      hipLaunchKernelGGL((scan_short_kernel<In, Out, Acc, REV, false, RL, G>),               \
                         dim3((unsigned)grid), dim3(kThreads), 0, stream, x, y, rows, D);    \
  } while (0)
    if (D <= 64) SCAN_SHORT(16, 1);
    else if (D <= 128) SCAN_SHORT(16, 2);
    else if (D <= 256) SCAN_SHORT(16, 4);
    else if (D <= 512) SCAN_SHORT(64, 2);
    else if (D <= 1024) SCAN_SHORT(64, 4);
    else SCAN_SHORT(64, 8);
#undef SCAN_SHORT
    return nl2k::check_launch(who);
  }
  auto* kernel = vec ? &scan_rows_kernel<In, Out, Acc, REV, true>
                     : &scan_rows_kernel<In, Out, Acc, REV, false>;
  int resident = 1;
  if (p.nchunk > 1) {
    // the grid stays within what the device holds at once (per device and
    // instantiation), so every chunk's predecessors are running or done
    st = nl2k::resident_blocks(reinterpret_cast<const void*>(kernel), kThreads, &resident);
    if (st) return st;
    hipError_t qe = hipSuccess;
    const bool cap = nl2k::slots::capturing(stream, &qe);
    if (qe != hipSuccess) return nl2k::check_hip(qe, "hipStreamIsCapturing");
    if (cap) nl2k::slots::clear_async(slots, 2 * p.slots, stream);
  }
  const int64_t grid = launch_grid(p, resident);
  hipLaunchKernelGGL(kernel, dim3((unsigned)grid), dim3(kThreads), 0, stream, x, y, D, p.nchunk,
                     p.tiles, p.total, slots, key, err);
  return nl2k::check_launch(who);
}

}  // namespace

extern "C" {

const char* scan_last_error(void) { return nl2k::error_slot().text; }

size_t scan_workspace_bytes(int64_t rows, int64_t D) {
  if (validate(rows, D, "scan_workspace_bytes")) return 0;
  return workspace_bytes(plan(rows, D));
}

size_t scan_status_offset(int64_t rows, int64_t D) {
  if (validate(rows, D, "scan_status_offset")) return SIZE_MAX;
  const Plan p = plan(rows, D);
  return p.slots > 0 ? (size_t)p.slots * 16 : SIZE_MAX;
}

int64_t scan_launch_grid(int64_t rows, int64_t D, int64_t resident_workgroups) {
  if (validate(rows, D, "scan_launch_grid") || resident_workgroups < 1) return -1;
  if (rows == 0) return 0;
  return launch_grid(plan(rows, D), resident_workgroups);
}

int scan_forward_f32(const float* x, float* y, int64_t rows, int64_t D, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  return run<float, float, double, false>(x, y, rows, D, workspace, workspace_bytes, stream,
                                          "scan_forward_f32");
}

int scan_backward_f32(const float* dy, float* dx, int64_t rows, int64_t D, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  return run<float, float, double, true>(dy, dx, rows, D, workspace, workspace_bytes, stream,
                                         "scan_backward_f32");
}

int scan_forward_i32_i64(const int32_t* x, int64_t* y, int64_t rows, int64_t D, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  return run<int32_t, int64_t, int64_t, false>(x, y, rows, D, workspace, workspace_bytes, stream,
                                               "scan_forward_i32_i64");
}

int scan_forward_i32(const int32_t* x, int32_t* y, int64_t rows, int64_t D, void* workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  return run<int32_t, int32_t, int64_t, false>(x, y, rows, D, workspace, workspace_bytes, stream,
                                               "scan_forward_i32");
}

}  // extern "C"
