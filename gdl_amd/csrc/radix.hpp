// radix.hpp — stable LSD radix sort of (uint32 key, uint32 value) pairs, 8-bit digits.
//
// Three kernels per pass:
//   radix_hist     one 2048-key tile per block, 256-bin LDS histogram -> hist[digit][tile]
//                  (lanes holding the same digit add once: sorted input does not serialise)
//   scan           device-wide exclusive scan of hist (digit-major) -> global offsets
//   radix_scatter  stable rank inside the tile: each wave walks its 512 keys in index order,
//                  peers with the same digit are found with 8 ballots, per-wave LDS counters
//                  give the running count, a cross-wave prefix finishes the tile rank.
// The first pass reads the caller's keys in one of three forms (RxSource) and writes uint32
// keys; the value of the first pass is the element index unless values are supplied.
#pragma once

#include "scan.hpp"

namespace geo {

constexpr int kRxThreads = 256;
constexpr int kRxItems = 8;
constexpr int kRxTile = kRxThreads * kRxItems;
constexpr int kRxWaves = kRxThreads / kWave;
constexpr int kRxWaveSpan = kRxItems * kWave;  // keys per wave in a tile

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
__device__ __forceinline__ uint64_t rx_peers(uint32_t d, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bb = __ballot(bit);
    peers &= bit ? bb : ~bb;
  }
  return peers;
}

template <int SRC>
__global__ __launch_bounds__(kRxThreads) void radix_hist(const void* __restrict__ keys, int64_t n,
                                                         int64_t N, int shift,
                                                         uint32_t* __restrict__ hist,
                                                         int64_t ntiles) {
  __shared__ uint32_t h[256];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kRxTile;
#pragma unroll
  for (int i = 0; i < kRxItems; ++i) {
    const int64_t idx = base + static_cast<int64_t>(i) * kRxThreads + threadIdx.x;
    const bool valid = idx < n;
    const uint32_t d = valid ? (rx_fetch_key<SRC>(keys, idx, N) >> shift) & 255u : 0u;
    const uint64_t peers = rx_peers(d, valid);
    if (valid && __popcll(peers & lanemask_lt()) == 0)
      atomicAdd(&h[d], static_cast<uint32_t>(__popcll(peers)));
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * ntiles + blockIdx.x] = h[threadIdx.x];
}

template <int SRC>
__global__ __launch_bounds__(kRxThreads) void radix_scatter(
    const void* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n, int64_t N,
    int shift, const uint32_t* __restrict__ offsets, int64_t ntiles, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t cnt[kRxWaves][256];
  __shared__ uint32_t goff[256];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
#pragma unroll
  for (int ww = 0; ww < kRxWaves; ++ww) cnt[ww][t] = 0;
  goff[t] = offsets[static_cast<int64_t>(t) * ntiles + blockIdx.x];
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
    const uint32_t d = (key[i] >> shift) & 255u;
    const uint64_t peers = rx_peers(d, valid);
    const uint32_t r = static_cast<uint32_t>(__popcll(peers & lt));
    const uint32_t before = cnt[w][d];
    __builtin_amdgcn_wave_barrier();
    if (valid && r == 0) cnt[w][d] = before + static_cast<uint32_t>(__popcll(peers));
    __builtin_amdgcn_wave_barrier();
    rank[i] = before + r;
  }
  __syncthreads();
  {
    uint32_t run = 0;
#pragma unroll
    for (int ww = 0; ww < kRxWaves; ++ww) {
      const uint32_t c = cnt[ww][t];
      cnt[ww][t] = run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kRxItems; ++i) {
    const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
    if (idx < n) {
      const uint32_t d = (key[i] >> shift) & 255u;
      const uint32_t pos = goff[d] + cnt[w][d] + rank[i];
      keys_out[pos] = key[i];
      vals_out[pos] = val[i];
    }
  }
}

// Scratch of one sort of n pairs.
struct RadixBuffers {
  uint32_t *ka, *va, *kb, *vb, *hist, *hist_tiles;
};

inline RadixBuffers carve_radix(Carver& c, int64_t n) {
  RadixBuffers r;
  const int64_t ntiles = ceil_div(n > 0 ? n : 1, kRxTile);
  r.ka = c.take<uint32_t>(n);
  r.va = c.take<uint32_t>(n);
  r.kb = c.take<uint32_t>(n);
  r.vb = c.take<uint32_t>(n);
  r.hist = c.take<uint32_t>(256 * ntiles);
  r.hist_tiles = c.take<uint32_t>(scan_workspace_elems(256 * ntiles));
  return r;
}

// Sorts n > 0 keys on digits 0 .. passes-1 (8 bits each); the last pass writes keys_out /
// vals_out.  keys / vals are read as the first pass's source SRC.
template <int SRC>
int radix_sort(const void* keys, const uint32_t* vals, int64_t n, int64_t N, int passes,
               uint32_t* keys_out, uint32_t* vals_out, const RadixBuffers& r, hipStream_t st) {
  const int64_t ntiles = ceil_div(n, kRxTile);
  const void* kin = keys;
  const uint32_t* vin = vals;
  for (int p = 0; p < passes; ++p) {
    const bool first = p == 0, last = p == passes - 1;
    uint32_t* kout = last ? keys_out : ((p % 2 == 0) ? r.ka : r.kb);
    uint32_t* vout = last ? vals_out : ((p % 2 == 0) ? r.va : r.vb);
    const int shift = 8 * p;
    if (first)
      hipLaunchKernelGGL((radix_hist<SRC>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, n, N,
                         shift, r.hist, ntiles);
    else
      hipLaunchKernelGGL((radix_hist<kRxPairs>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, n,
                         N, shift, r.hist, ntiles);
    GEO_LAUNCH_CHECK("radix_hist");
    int rc = device_exclusive_scan<uint32_t, uint32_t>(r.hist, 256 * ntiles, r.hist, nullptr,
                                                       false, r.hist_tiles, st);
    if (rc) return rc;
    if (first)
      hipLaunchKernelGGL((radix_scatter<SRC>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, vin,
                         n, N, shift, r.hist, ntiles, kout, vout);
    else
      hipLaunchKernelGGL((radix_scatter<kRxPairs>), dim3(ntiles), dim3(kRxThreads), 0, st, kin,
                         vin, n, N, shift, r.hist, ntiles, kout, vout);
    GEO_LAUNCH_CHECK("radix_scatter");
    kin = kout;
    vin = vout;
  }
  return GEO_OK;
}

}  // namespace geo
