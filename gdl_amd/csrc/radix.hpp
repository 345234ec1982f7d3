// radix.hpp — stable LSD radix sort of (uint32 key, uint32 value) pairs, 8- to 11-bit digits.
//
// A sort of b-bit keys takes ceil(b / 11) passes of near-equal digit width (17-bit CSR keys: two
// passes of 9 and 8 bits instead of three of 8).  Three kernels per pass:
//   radix_hist     one 2048-key tile per block, 2^BITS-bin LDS histogram -> hist[digit][tile]
//                  (a run of equal digits in consecutive lanes adds once: sorted input does not
//                  serialise on one counter)
//   scan           device-wide exclusive scan of hist (digit-major) -> global offsets
//   radix_scatter  stable rank inside the tile: each wave walks its 512 keys in index order,
//                  peers with the same digit are found with BITS ballots, per-wave LDS counters
//                  give the running count, a cross-wave prefix finishes the tile rank.
// The first pass reads the caller's keys in one of three forms (RxSource) and writes uint32
// keys; the value of the first pass is the element index unless values are supplied.
#pragma once

#include "scan.hpp"

namespace geo {
// Internal linkage: every translation unit that includes this header gets its own copy of the
// radix sort kernels and helpers, so no two units can share a definition built differently.
namespace {

constexpr int kRxThreads = 256;
constexpr int kRxItems = 8;
constexpr int kRxTile = kRxThreads * kRxItems;
constexpr int kRxWaves = kRxThreads / kWave;
constexpr int kRxWaveSpan = kRxItems * kWave;  // keys per wave in a tile
constexpr int kRxMaxBits = 11;                  // widest digit
constexpr int kRxMaxBins = 1 << kRxMaxBits;

enum RxSource {
  kRxCol64 = 0,     // int64 keys, values outside [0, N) become N; value = index
  kRxKeysIota = 1,  // uint32 keys; value = index
  kRxPairs = 2,     // uint32 keys and uint32 values
};

template <int SRC>
__device__ __forceinline__ uint32_t rx_fetch_key(const void* keys, int64_t i, int64_t N) {
  if constexpr (SRC == kRxCol64) {
    const int64_t c = static_cast<const int64_t*>(keys)[i];
    return (c >= 0 && c < N) ? static_cast<uint32_t>(c) : static_cast<uint32_t>(N);
  } else {
    return static_cast<const uint32_t*>(keys)[i];
  }
}

// Lanes of the wave whose (valid) digit equals this lane's digit.
template <int BITS>
__device__ __forceinline__ uint64_t rx_peers(uint32_t d, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bb = __ballot(bit);
    peers &= bit ? bb : ~bb;
  }
  return peers;
}

template <int SRC, int BITS>
__global__ __launch_bounds__(kRxThreads) void radix_hist(const void* __restrict__ keys, int64_t n,
                                                         int64_t N, int shift,
                                                         uint32_t* __restrict__ hist,
                                                         int64_t ntiles,
                                                         uint32_t* __restrict__ unsorted,
                                                         const uint32_t* __restrict__ active) {
  if (active != nullptr && *active == 0u) return;
  constexpr int BINS = 1 << BITS;
  __shared__ uint32_t h[BINS];
  __shared__ uint32_t s_down;
  for (int b = threadIdx.x; b < BINS; b += kRxThreads) h[b] = 0;
  if (threadIdx.x == 0) s_down = 0u;
  // once some tile has found the input out of order, the others skip the check
  const bool check = unsorted != nullptr &&
                     __hip_atomic_load(unsorted, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kRxTile;
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < kRxItems; ++i) {
    const int64_t idx = base + static_cast<int64_t>(i) * kRxThreads + threadIdx.x;
    const bool valid = idx < n;
    // runs of equal digits in consecutive lanes add once (sorted input does not serialise on
    // one counter); invalid lanes, at the end of the range, carry a digit no key has
    const uint32_t key = valid ? rx_fetch_key<SRC>(keys, idx, N) : 0u;
    if (check) {  // first pass of a sort that may find its input already sorted
      const uint32_t up = __shfl_up(key, 1, kWave);  // lane - 1 holds key idx - 1
      const uint32_t pk = lane != 0 ? up : (valid && idx > 0 ? rx_fetch_key<SRC>(keys, idx - 1, N) : 0u);
      if (valid && pk > key) s_down = 1u;
    }
    const uint32_t d = valid ? (key >> shift) & (BINS - 1u) : BINS;
    const uint32_t prev = __shfl_up(d, 1, kWave);
    const uint64_t starts = __ballot(lane == 0 || prev != d);
    if (valid && (lane == 0 || prev != d)) {
      const uint64_t later = lane == kWave - 1 ? 0ull : (starts & (~0ull << (lane + 1)));
      const int next = later ? __builtin_ctzll(later) : kWave;
      atomicAdd(&h[d], static_cast<uint32_t>(next - lane));
    }
  }
  __syncthreads();
  // one atomic per out-of-order tile, skipped once another tile has set the flag
  if (check && threadIdx.x == 0 && s_down != 0u) atomicOr(unsorted, 1u);
  for (int b = threadIdx.x; b < BINS; b += kRxThreads)
    hist[static_cast<int64_t>(b) * ntiles + blockIdx.x] = h[b];
}

template <int SRC, int BITS>
__global__ __launch_bounds__(kRxThreads) void radix_scatter(
    const void* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n, int64_t N,
    int shift, const uint32_t* __restrict__ offsets, int64_t ntiles, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, const uint32_t* __restrict__ active,
    const uint32_t* __restrict__ unsorted, uint32_t* __restrict__ final_keys,
    uint32_t* __restrict__ final_vals) {
  if (active != nullptr && *active == 0u) return;
  constexpr int BINS = 1 << BITS;
  __shared__ uint32_t cnt[kRxWaves][BINS];
  __shared__ uint32_t goff[BINS];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  if (unsorted != nullptr && *unsorted == 0u) {  // sorted input: the sort is the identity
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = static_cast<int64_t>(blockIdx.x) * kRxTile + static_cast<int64_t>(i) * kRxThreads + t;
      if (idx < n) {
        final_keys[idx] = rx_fetch_key<SRC>(keys_in, idx, N);
        final_vals[idx] = SRC == kRxPairs ? vals_in[idx] : static_cast<uint32_t>(idx);
      }
    }
    return;
  }
  for (int b = t; b < BINS; b += kRxThreads) {
#pragma unroll
    for (int ww = 0; ww < kRxWaves; ++ww) cnt[ww][b] = 0;
    goff[b] = offsets[static_cast<int64_t>(b) * ntiles + blockIdx.x];
  }
  __syncthreads();

  const uint64_t lt = lanemask_lt();
  const int64_t wbase = static_cast<int64_t>(blockIdx.x) * kRxTile + static_cast<int64_t>(w) * kRxWaveSpan;
  uint32_t key[kRxItems], val[kRxItems], rank[kRxItems];
#pragma unroll
  for (int i = 0; i < kRxItems; ++i) {
    const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
    const bool valid = idx < n;
    key[i] = valid ? rx_fetch_key<SRC>(keys_in, idx, N) : 0u;
    if constexpr (SRC == kRxPairs) {
      val[i] = valid ? vals_in[idx] : 0u;
    } else {
      val[i] = static_cast<uint32_t>(idx);
    }
    const uint32_t d = (key[i] >> shift) & (BINS - 1u);
    const uint64_t peers = rx_peers<BITS>(d, valid);
    const uint32_t r = static_cast<uint32_t>(__popcll(peers & lt));
    const uint32_t before = cnt[w][d];
    __builtin_amdgcn_wave_barrier();
    if (valid && r == 0) cnt[w][d] = before + static_cast<uint32_t>(__popcll(peers));
    __builtin_amdgcn_wave_barrier();
    rank[i] = before + r;
  }
  __syncthreads();
  for (int b = t; b < BINS; b += kRxThreads) {
    uint32_t run = 0;
#pragma unroll
    for (int ww = 0; ww < kRxWaves; ++ww) {
      const uint32_t c = cnt[ww][b];
      cnt[ww][b] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kRxItems; ++i) {
    const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
    if (idx < n) {
      const uint32_t d = (key[i] >> shift) & (BINS - 1u);
      const uint32_t pos = goff[d] + cnt[w][d] + rank[i];
      keys_out[pos] = key[i];
      vals_out[pos] = val[i];
    }
  }
}

// Scratch of one sort of n pairs.
struct RadixBuffers {
  uint32_t *ka, *va, *kb, *vb, *hist, *hist_tiles;
  uint32_t* unsorted;  // set by the first pass's histogram when the input is out of order
};

inline RadixBuffers carve_radix(Carver& c, int64_t n) {
  RadixBuffers r;
  const int64_t ntiles = ceil_div(n > 0 ? n : 1, kRxTile);
  r.ka = c.take<uint32_t>(n);
  r.va = c.take<uint32_t>(n);
  r.kb = c.take<uint32_t>(n);
  r.vb = c.take<uint32_t>(n);
  r.hist = c.take<uint32_t>(static_cast<int64_t>(kRxMaxBins) * ntiles);
  r.hist_tiles = c.take<uint32_t>(scan_workspace_elems(static_cast<int64_t>(kRxMaxBins) * ntiles));
  r.unsorted = c.take<uint32_t>(1);
  return r;
}

// Sorted-input detection (RxSorted): the first pass's histogram sets r.unsorted when the keys are
// out of order; the first scatter then writes the identity straight to the final outputs and
// every later kernel (and the first pass's offset scan) does nothing.
struct RxSorted {
  uint32_t* detect = nullptr;        // first pass: flag to set
  const uint32_t* active = nullptr;  // kernels run only when *active != 0
  const uint32_t* check = nullptr;   // first scatter: identity when *check == 0
  uint32_t* final_keys = nullptr;
  uint32_t* final_vals = nullptr;
};

template <int SRC, int BITS>
int radix_pass(const void* kin, const uint32_t* vin, int64_t n, int64_t N, int shift,
               uint32_t* kout, uint32_t* vout, const RadixBuffers& r, hipStream_t st,
               const RxSorted& so) {
  const int64_t ntiles = ceil_div(n, kRxTile);
  hipLaunchKernelGGL((radix_hist<SRC, BITS>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, n, N,
                     shift, r.hist, ntiles, so.detect, so.active);
  GEO_LAUNCH_CHECK("radix_hist");
  // three-kernel scan: with ~10^3 tiles of offsets the look-back chain is slower (measured)
  int rc = device_exclusive_scan<uint32_t, uint32_t>(r.hist, (int64_t{1} << BITS) * ntiles, r.hist,
                                                     nullptr, false, r.hist_tiles, st,
                                                     so.detect ? so.detect : so.active);
  if (rc) return rc;
  hipLaunchKernelGGL((radix_scatter<SRC, BITS>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, vin,
                     n, N, shift, r.hist, ntiles, kout, vout, so.active, so.check, so.final_keys,
                     so.final_vals);
  GEO_LAUNCH_CHECK("radix_scatter");
  return GEO_OK;
}

template <int SRC>
int radix_pass_bits(int bits, const void* kin, const uint32_t* vin, int64_t n, int64_t N, int shift,
                    uint32_t* kout, uint32_t* vout, const RadixBuffers& r, hipStream_t st,
                    const RxSorted& so) {
  switch (bits) {
    case 8: return radix_pass<SRC, 8>(kin, vin, n, N, shift, kout, vout, r, st, so);
    case 9: return radix_pass<SRC, 9>(kin, vin, n, N, shift, kout, vout, r, st, so);
    case 10: return radix_pass<SRC, 10>(kin, vin, n, N, shift, kout, vout, r, st, so);
    default: return radix_pass<SRC, 11>(kin, vin, n, N, shift, kout, vout, r, st, so);
  }
}

// Sorts n > 0 keys below 2^key_bits (stable); the last pass writes keys_out / vals_out.  keys /
// vals are read as the first pass's source SRC.  Digit widths: ceil(key_bits / 11) passes of
// near-equal width, at least 8 bits each.
template <int SRC>
int radix_sort(const void* keys, const uint32_t* vals, int64_t n, int64_t N, int key_bits,
               uint32_t* keys_out, uint32_t* vals_out, const RadixBuffers& r, hipStream_t st,
               bool detect_sorted = false) {
  key_bits = key_bits < 1 ? 1 : (key_bits > 32 ? 32 : key_bits);
  const int passes = (key_bits + kRxMaxBits - 1) / kRxMaxBits;
  const void* kin = keys;
  const uint32_t* vin = vals;
  if (detect_sorted) {
    const int rc = device_fill<uint32_t>(r.unsorted, 1, 0u, st);
    if (rc) return rc;
  }
  int shift = 0;
  for (int p = 0; p < passes; ++p) {
    const bool first = p == 0, last = p == passes - 1;
    uint32_t* kout = last ? keys_out : ((p % 2 == 0) ? r.ka : r.kb);
    uint32_t* vout = last ? vals_out : ((p % 2 == 0) ? r.va : r.vb);
    const int left = key_bits - shift;
    int bits = (left + (passes - p) - 1) / (passes - p);
    bits = bits < 8 ? 8 : bits;
    RxSorted so;
    if (detect_sorted) {
      if (first) {
        so.detect = r.unsorted;
        so.check = r.unsorted;
        so.final_keys = keys_out;
        so.final_vals = vals_out;
      } else {
        so.active = r.unsorted;
      }
    }
    const int rc = first ? radix_pass_bits<SRC>(bits, kin, vin, n, N, shift, kout, vout, r, st, so)
                         : radix_pass_bits<kRxPairs>(bits, kin, vin, n, N, shift, kout, vout, r, st, so);
    if (rc) return rc;
    shift += bits;
    kin = kout;
    vin = vout;
  }
  return GEO_OK;
}

}  // namespace
}  // namespace geo
