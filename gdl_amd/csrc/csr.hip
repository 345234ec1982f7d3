// csr.hip — stable CSR build (replaces sort_and_build_csr,
// geoembodied/csrc/segment_reduce_kernel.cu:100-169, which uses CUB radix sort + transition
// detection).
//
// Stable LSD radix sort of the int32 target ids with the edge index as value, 8-bit digits,
// three kernels per pass:
//   radix_hist     one 2048-key tile per block, 256-bin LDS histogram -> hist[digit][tile]
//   scan           device-wide exclusive scan of hist (digit-major) -> global offsets
//   radix_scatter  stable rank inside the tile: each wave walks its 512 keys in index order,
//                  peers with the same digit are found with 8 ballots, per-wave LDS counters
//                  give the running count, a cross-wave prefix finishes the tile rank.
// Targets outside [0, N) get key N and sort after all valid targets.  node_start/node_end come
// from binary searches in the sorted keys (node_start[n] = first position with key >= n), so
// empty targets get start == end and no atomics are involved.
#include "scan.hpp"

namespace geo {
namespace {

constexpr int kRxThreads = 256;
constexpr int kRxItems = 8;
constexpr int kRxTile = kRxThreads * kRxItems;
constexpr int kRxWaves = kRxThreads / kWave;
constexpr int kRxWaveSpan = kRxItems * kWave;  // keys per wave in a tile

template <bool FIRST>
__device__ __forceinline__ uint32_t fetch_key(const void* keys, int64_t i, int64_t N) {
  if constexpr (FIRST) {
    const int64_t c = static_cast<const int64_t*>(keys)[i];
    return (c >= 0 && c < N) ? static_cast<uint32_t>(c) : static_cast<uint32_t>(N);
  } else {
    return static_cast<const uint32_t*>(keys)[i];
  }
}

template <bool FIRST>
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
    const uint32_t d = valid ? (fetch_key<FIRST>(keys, idx, N) >> shift) & 255u : 0u;
    // lanes with the same digit add once (sorted input would otherwise serialise 64 atomics)
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
    if (valid && __popcll(peers & lanemask_lt()) == 0) atomicAdd(&h[d], static_cast<uint32_t>(__popcll(peers)));
  }
  __syncthreads();
  hist[static_cast<int64_t>(threadIdx.x) * ntiles + blockIdx.x] = h[threadIdx.x];
}

template <bool FIRST>
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
    key[i] = valid ? fetch_key<FIRST>(keys_in, idx, N) : 0u;
    if constexpr (FIRST) {
      val[i] = static_cast<uint32_t>(idx);
    } else {
      val[i] = valid ? vals_in[idx] : 0u;
    }
    const uint32_t d = (key[i] >> shift) & 255u;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
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

// Thread n in [0, N] computes lb(n) = first sorted position with key >= n; that is
// node_start[n] (n < N) and node_end[n - 1] (n > 0).
__global__ void csr_bounds(const uint32_t* __restrict__ sorted_keys, int64_t E, int64_t N,
                           int32_t* __restrict__ node_start, int32_t* __restrict__ node_end) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (n > N) return;
  int64_t lo = 0, hi = E;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (sorted_keys[mid] < static_cast<uint32_t>(n)) lo = mid + 1; else hi = mid;
  }
  if (n < N) node_start[n] = static_cast<int32_t>(lo);
  if (n > 0) node_end[n - 1] = static_cast<int32_t>(lo);
}

int radix_passes(int64_t N) {
  int bits = 0;
  while (bits < 32 && (static_cast<uint64_t>(N) >> bits) != 0) ++bits;  // bits to hold key N
  return bits == 0 ? 1 : (bits + 7) / 8;
}

struct CsrWs {
  uint32_t *ka, *va, *kb, *vb, *hist, *hist_tiles;
  size_t bytes;
};

CsrWs carve_csr(void* base, int64_t E, int64_t N) {
  Carver c(base);
  CsrWs w;
  const int64_t ntiles = ceil_div(E > 0 ? E : 1, kRxTile);
  w.ka = c.take<uint32_t>(E);
  w.va = c.take<uint32_t>(E);
  w.kb = c.take<uint32_t>(E);
  w.vb = c.take<uint32_t>(E);
  w.hist = c.take<uint32_t>(256 * ntiles);
  w.hist_tiles = c.take<uint32_t>(scan_workspace_elems(256 * ntiles));
  w.bytes = c.used;
  return w;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_csr_workspace_bytes(int64_t E, int64_t N) {
  if (E < 0 || N < 0) return 0;
  return carve_csr(nullptr, E, N).bytes;
}

extern "C" int geo_csr_build(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted,
                             int32_t* perm, int32_t* node_start, int32_t* node_end,
                             void* workspace, size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(E >= 0 && N >= 0, "csr_build: negative size (E=%lld N=%lld)", (long long)E,
              (long long)N);
  GEO_REQUIRE(E < 0x7fffffffLL && N < 0x7fffffffLL, "csr_build: sizes exceed int32 indexing");
  hipStream_t st = as_stream(stream);
  CsrWs w = carve_csr(workspace, E, N);
  if (workspace_bytes < w.bytes || workspace == nullptr)
    return set_error(GEO_ERR_WORKSPACE, "csr_build: workspace %zu bytes, need %zu",
                     workspace_bytes, w.bytes);
  GEO_REQUIRE(N == 0 || (node_start && node_end), "csr_build: null node_start/node_end");
  GEO_REQUIRE(E == 0 || (col && col_sorted && perm), "csr_build: null edge arrays");

  if (E == 0) {
    if (N == 0) return GEO_OK;
    int rc = device_fill<int32_t>(node_start, N, 0, st);
    if (rc) return rc;
    return device_fill<int32_t>(node_end, N, 0, st);
  }

  // Stable radix sort.
  const int passes = radix_passes(N);
  const int64_t ntiles = ceil_div(E, kRxTile);
  const void* kin = col;
  const uint32_t* vin = nullptr;
  for (int p = 0; p < passes; ++p) {
    const bool first = p == 0, last = p == passes - 1;
    uint32_t* kout = last ? reinterpret_cast<uint32_t*>(col_sorted) : ((p % 2 == 0) ? w.ka : w.kb);
    uint32_t* vout = last ? reinterpret_cast<uint32_t*>(perm) : ((p % 2 == 0) ? w.va : w.vb);
    const int shift = 8 * p;
    if (first)
      hipLaunchKernelGGL((radix_hist<true>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, E, N,
                         shift, w.hist, ntiles);
    else
      hipLaunchKernelGGL((radix_hist<false>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, E, N,
                         shift, w.hist, ntiles);
    GEO_LAUNCH_CHECK("radix_hist");
    int rc = device_exclusive_scan<uint32_t, uint32_t>(w.hist, 256 * ntiles, w.hist, nullptr,
                                                       false, w.hist_tiles, st);
    if (rc) return rc;
    if (first)
      hipLaunchKernelGGL((radix_scatter<true>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, vin,
                         E, N, shift, w.hist, ntiles, kout, vout);
    else
      hipLaunchKernelGGL((radix_scatter<false>), dim3(ntiles), dim3(kRxThreads), 0, st, kin, vin,
                         E, N, shift, w.hist, ntiles, kout, vout);
    GEO_LAUNCH_CHECK("radix_scatter");
    kin = kout;
    vin = vout;
  }
  if (N > 0) {
    hipLaunchKernelGGL(csr_bounds, dim3(ceil_div(N + 1, 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t*>(col_sorted), E, N, node_start, node_end);
    GEO_LAUNCH_CHECK("csr_bounds");
  }
  return GEO_OK;
}
