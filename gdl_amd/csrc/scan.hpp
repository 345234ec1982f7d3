// scan.hpp — device-wide exclusive prefix sum, three kernels (tile reduce, tile-sum scan,
// tile apply).  Deterministic: integer sums, fixed tiling.
#pragma once

#include "common.hpp"

namespace geo {
// Internal linkage: every translation unit that includes this header gets its own copy of the
// scan kernels and helpers, so no two units can share a definition built differently.
namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

// Exclusive scan of one value per thread across the block.  `lds` holds kScanThreads/64
// entries.  Returns the exclusive prefix; `total` receives the block sum.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* lds, T& total) {
  const int wave = threadIdx.x / kWave;
  constexpr int kWaves = kScanThreads / kWave;
  T inc = wave_inclusive_sum_int(v);
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
                                                                   TOut* __restrict__ tile_sums,
                                                                   const uint32_t* __restrict__ active) {
  if (active != nullptr && *active == 0u) return;
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
                                                                 int64_t ntiles,
                                                                 const uint32_t* __restrict__ active) {
  if (active != nullptr && *active == 0u) return;
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
    TOut* __restrict__ out_excl, TOut* __restrict__ out_incl, int write_total,
    const uint32_t* __restrict__ active = nullptr) {
  if (active != nullptr && *active == 0u) return;
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
// With `active` (device word), the kernels do nothing when it reads 0.
template <typename TIn, typename TOut>
int device_exclusive_scan(const TIn* in, int64_t n, TOut* out_excl, TOut* out_incl,
                          bool write_total, TOut* tile_ws, hipStream_t stream,
                          const uint32_t* active = nullptr) {
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
                       write_total ? 1 : 0, active);
    GEO_LAUNCH_CHECK("scan_tile_apply");
    return GEO_OK;
  }
  hipLaunchKernelGGL((scan_tile_reduce<TIn, TOut>), dim3(ntiles), dim3(kScanThreads), 0, stream,
                     in, n, tile_ws, active);
  GEO_LAUNCH_CHECK("scan_tile_reduce");
  hipLaunchKernelGGL((scan_tile_sums<TOut>), dim3(1), dim3(kScanThreads), 0, stream, tile_ws,
                     ntiles, active);
  GEO_LAUNCH_CHECK("scan_tile_sums");
  hipLaunchKernelGGL((scan_tile_apply<TIn, TOut>), dim3(ntiles), dim3(kScanThreads), 0, stream,
                     in, n, static_cast<const TOut*>(tile_ws), out_excl, out_incl,
                     write_total ? 1 : 0, active);
  GEO_LAUNCH_CHECK("scan_tile_apply");
  return GEO_OK;
}

// ---- Single-pass scan (decoupled look-back) --------------------------------------------
// One launch instead of three.  Tiles take their index from a counter in the order they start,
// publish their sum (flag A), then walk back over earlier tiles, 64 per step (one wave): the
// nearest inclusive prefix (flag P) ends the walk, aggregates before it are added.  Value and flag
// share one 64-bit word written and read with agent-scope relaxed atomics, so no fence (and no
// L2 writeback) is needed between them.  Every tile waited on started earlier and publishes its
// aggregate before it waits itself, so each wait ends; as a further guard a wait that exceeds
// kScanSpinLimit polls sums the missing tiles' inputs directly instead (same values).
// `status` needs scan_lookback_elems(n) words, zeroed on the stream before the launch.
constexpr uint64_t kScanFlagA = 1ull << 62, kScanFlagP = 2ull << 62, kScanValMask = kScanFlagA - 1;
constexpr int kScanSpinLimit = 1 << 16;

__host__ __device__ inline int64_t scan_lookback_elems(int64_t n) {
  return ceil_div(n > 0 ? n : 1, kScanTile) + 1;
}

template <typename TIn, typename TOut>
__device__ TOut scan_tile_sum_direct(const TIn* __restrict__ in, int64_t n, int64_t tile) {
  TOut s = 0;
  const int64_t a = tile * kScanTile, b = min(n, a + kScanTile);
  for (int64_t i = a; i < b; ++i) s += static_cast<TOut>(in[i]);
  return s;
}

template <typename TIn, typename TOut>
__global__ __launch_bounds__(kScanThreads) void scan_lookback(
    const TIn* __restrict__ in, int64_t n, TOut* __restrict__ out_excl, TOut* __restrict__ out_incl,
    int write_total, uint64_t* __restrict__ status, TOut* __restrict__ total_host,
    const uint32_t* __restrict__ active) {
  if (active != nullptr && *active == 0u) return;
  __shared__ TOut lds[kScanThreads / kWave];
  __shared__ int64_t s_tile;
  __shared__ TOut s_prefix;
  const int64_t ntiles = ceil_div(n, kScanTile);
  if (threadIdx.x == 0)
    s_tile = static_cast<int64_t>(__hip_atomic_fetch_add(
        reinterpret_cast<unsigned long long*>(status + ntiles), 1ull, __ATOMIC_RELAXED,
        __HIP_MEMORY_SCOPE_AGENT));
  __syncthreads();
  const int64_t tile = s_tile;
  const int64_t base = tile * kScanTile;
  TOut v[kScanItems];
  TOut s = 0;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
    v[i] = idx < n ? static_cast<TOut>(in[idx]) : TOut(0);
    s += v[i];
  }
  TOut total;
  TOut off = block_exclusive_scan<TOut>(s, lds, total);
  if (threadIdx.x < kWave) {  // wave 0 publishes and looks back over 64 earlier tiles at a time
    unsigned long long* st = reinterpret_cast<unsigned long long*>(status);
    const int lane = static_cast<int>(threadIdx.x);
    TOut prefix = 0;
    if (tile > 0) {
      if (lane == 0)
        __hip_atomic_store(st + tile, kScanFlagA | static_cast<uint64_t>(total), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      int64_t top = tile - 1;  // window: tiles top, top-1, ..., top-63 on lanes 0..63
      while (true) {
        const int64_t j = top - lane;
        uint64_t w = kScanFlagP;  // before tile 0: an inclusive prefix of 0
        int spins = 0;
        uint64_t ready, isp, need;
        while (true) {
          if (j >= 0) w = __hip_atomic_load(st + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ready = __ballot((w >> 62) != 0);
          isp = __ballot((w & kScanFlagP) != 0);
          const int firstp = isp ? __builtin_ctzll(isp) : kWave;
          need = firstp >= kWave - 1 ? ~0ull : ((2ull << firstp) - 1ull);
          if ((ready & need) == need) break;
          if (++spins > kScanSpinLimit) {  // guard: aggregates from the inputs
            if (j >= 0 && (w >> 62) == 0)
              w = kScanFlagA | static_cast<uint64_t>(scan_tile_sum_direct<TIn, TOut>(in, n, j));
            ready = __ballot((w >> 62) != 0);
            isp = __ballot((w & kScanFlagP) != 0);
            const int fp = isp ? __builtin_ctzll(isp) : kWave;
            need = fp >= kWave - 1 ? ~0ull : ((2ull << fp) - 1ull);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        const bool take = ((need >> lane) & 1ull) != 0;
        prefix += wave_sum_int<TOut>(take ? static_cast<TOut>(w & kScanValMask) : TOut(0));
        if (isp & need) break;  // reached an inclusive prefix
        top -= kWave;
      }
      if (lane == 0)
        __hip_atomic_store(st + tile, kScanFlagP | static_cast<uint64_t>(prefix + total),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (lane == 0) {
      __hip_atomic_store(st, kScanFlagP | static_cast<uint64_t>(total), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) s_prefix = prefix;
  }
  __syncthreads();
  const TOut tile_off = s_prefix;
  off += tile_off;
#pragma unroll
  for (int i = 0; i < kScanItems; ++i) {
    const int64_t idx = base + static_cast<int64_t>(threadIdx.x) * kScanItems + i;
    if (idx < n) {
      if (out_excl) out_excl[idx] = off;
      off += v[i];
      if (out_incl) out_incl[idx] = off;
    }
  }
  if (tile == ntiles - 1 && threadIdx.x == kScanThreads - 1) {
    if (write_total) out_excl[n] = tile_off + total;
    if (total_host) {  // mapped pinned host memory: the host reads it after this kernel
      *total_host = tile_off + total;
      __threadfence_system();
    }
  }
}

// Single-pass variant of device_exclusive_scan (n >= 1); status zeroed by the caller.
// total_host (optional) is a device-side address of mapped pinned host memory that receives the
// grand total as well.  With `active` (device word), the scan does nothing when it reads 0.
template <typename TIn, typename TOut>
int device_exclusive_scan_lookback(const TIn* in, int64_t n, TOut* out_excl, TOut* out_incl,
                                   bool write_total, uint64_t* status, hipStream_t stream,
                                   TOut* total_host = nullptr,
                                   const uint32_t* active = nullptr) {
  if (n <= 0) return device_exclusive_scan<TIn, TOut>(in, n, out_excl, out_incl, write_total,
                                                      nullptr, stream);
  hipLaunchKernelGGL((scan_lookback<TIn, TOut>), dim3(ceil_div(n, kScanTile)), dim3(kScanThreads),
                     0, stream, in, n, out_excl, out_incl, write_total ? 1 : 0, status,
                     total_host, active);
  GEO_LAUNCH_CHECK("scan_lookback");
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

}  // namespace
}  // namespace geo
