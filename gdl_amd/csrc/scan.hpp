// scan.hpp — device-wide exclusive prefix sum, three kernels (tile reduce, tile-sum scan,
// tile apply).  Deterministic: integer sums, fixed tiling.
#pragma once

#include "common.hpp"

namespace geo {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

// Exclusive scan of one value per thread across the block.  `lds` holds kScanThreads/64
// entries.  Returns the exclusive prefix; `total` receives the block sum.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* lds, T& total) {
  const int wave = threadIdx.x / kWave;
  constexpr int kWaves = kScanThreads / kWave;
  T inc = wave_inclusive_sum(v);
  if (lane_id() == kWave - 1) lds[wave] = inc;
  __syncthreads();
  T wave_off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    T t = lds[w];
    if (w < wave) wave_off += t;
    tot += t;
  }
  __syncthreads();  // lds may be reused by the caller
  total = tot;
  return wave_off + inc - v;
}

template <typename TIn, typename TOut>
__global__ __launch_bounds__(kScanThreads) void scan_tile_reduce(const TIn* __restrict__ in,
                                                                   int64_t n,
                                                                   TOut* __restrict__ tile_sums) {
  __shared__ TOut lds[kScanThreads / kWave];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  TOut s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + static_cast<int64_t>(i) * kScanThreads + threadIdx.x;
    if (idx < n) s += static_cast<TOut>(in[idx]);
  }
  TOut total;
  block_exclusive_scan<TOut>(s, lds, total);
  if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

// Single block: exclusive scan of tile_sums[0..ntiles) in place.
template <typename TOut>
__global__ __launch_bounds__(kScanThreads) void scan_tile_sums(TOut* __restrict__ tile_sums,
                                                                 int64_t ntiles) {
  __shared__ TOut lds[kScanThreads / kWave];
  TOut carry = 0;
  for (int64_t base = 0; base < ntiles; base += kScanTile) {
    TOut v[kScanItems];
    TOut s = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
      v[i] = idx < ntiles ? tile_sums[idx] : TOut(0);
      s += v[i];
    }
    TOut total;
    TOut off = block_exclusive_scan<TOut>(s, lds, total) + carry;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
      int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
      if (idx < ntiles) tile_sums[idx] = off;
      off += v[i];
    }
    carry += total;
  }
}

// Scans each tile with its offset (tile_offsets may be NULL for a single tile).  Writes the
// exclusive scan to out_excl[0..n), the inclusive scan to out_incl (if not NULL) and, if
// write_total, the grand total to out_excl[n].
template <typename TIn, typename TOut>
__global__ __launch_bounds__(kScanThreads) void scan_tile_apply(
    const TIn* __restrict__ in, int64_t n, const TOut* __restrict__ tile_offsets,
    TOut* __restrict__ out_excl, TOut* __restrict__ out_incl, int write_total) {
  __shared__ TOut lds[kScanThreads / kWave];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
  TOut v[kScanItems];
  TOut s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
    v[i] = idx < n ? static_cast<TOut>(in[idx]) : TOut(0);
    s += v[i];
  }
  TOut total;
  TOut off = block_exclusive_scan<TOut>(s, lds, total);
  const TOut tile_off = tile_offsets ? tile_offsets[blockIdx.x] : TOut(0);
  off += tile_off;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
    if (idx < n) {
      if (out_excl) out_excl[idx] = off;
      off += v[i];
      if (out_incl) out_incl[idx] = off;
    }
  }
  if (write_total && blockIdx.x == gridDim.x - 1 && threadIdx.x == kScanThreads - 1)
    out_excl[n] = tile_off + total;
}

inline int64_t scan_workspace_elems(int64_t n) { return ceil_div(n > 0 ? n : 1, kScanTile); }

// out_excl needs n+1 entries when write_total.  tile_ws needs scan_workspace_elems(n) entries.
template <typename TIn, typename TOut>
int device_exclusive_scan(const TIn* in, int64_t n, TOut* out_excl, TOut* out_incl,
                          bool write_total, TOut* tile_ws, hipStream_t stream) {
  if (n <= 0) {
    if (write_total) {
      // total of an empty range is 0: use a one-element apply on a zero tile.
      hipLaunchKernelGGL((scan_tile_apply<TIn, TOut>), dim3(1), dim3(kScanThreads), 0, stream,
                         in, int64_t(0), static_cast<const TOut*>(nullptr), out_excl, out_incl, 1);
      GEO_LAUNCH_CHECK("scan_tile_apply(empty)");
    }
    return GEO_OK;
  }
  const int64_t ntiles = ceil_div(n, kScanTile);
  if (ntiles == 1) {
    hipLaunchKernelGGL((scan_tile_apply<TIn, TOut>), dim3(1), dim3(kScanThreads), 0, stream, in,
                       n, static_cast<const TOut*>(nullptr), out_excl, out_incl,
                       write_total ? 1 : 0);
    GEO_LAUNCH_CHECK("scan_tile_apply");
    return GEO_OK;
  }
  hipLaunchKernelGGL((scan_tile_reduce<TIn, TOut>), dim3(ntiles), dim3(kScanThreads), 0, stream,
                     in, n, tile_ws);
  GEO_LAUNCH_CHECK("scan_tile_reduce");
  hipLaunchKernelGGL((scan_tile_sums<TOut>), dim3(1), dim3(kScanThreads), 0, stream, tile_ws,
                     ntiles);
  GEO_LAUNCH_CHECK("scan_tile_sums");
  hipLaunchKernelGGL((scan_tile_apply<TIn, TOut>), dim3(ntiles), dim3(kScanThreads), 0, stream,
                     in, n, static_cast<const TOut*>(tile_ws), out_excl, out_incl,
                     write_total ? 1 : 0);
  GEO_LAUNCH_CHECK("scan_tile_apply");
  return GEO_OK;
}

// Fill kernel (used instead of hipMemsetAsync so that callers may capture graphs).
template <typename T>
__global__ void fill_kernel(T* __restrict__ p, int64_t n, T v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = v;
}

template <typename T>
int device_fill(T* p, int64_t n, T v, hipStream_t stream) {
  if (n <= 0) return GEO_OK;
  int64_t blocks = ceil_div(n, 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL((fill_kernel<T>), dim3(blocks), dim3(256), 0, stream, p, n, v);
  GEO_LAUNCH_CHECK("fill_kernel");
  return GEO_OK;
}

}  // namespace geo
