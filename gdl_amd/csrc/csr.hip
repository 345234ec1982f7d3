// csr.hip — stable CSR build (replaces sort_and_build_csr,
// geoembodied/csrc/segment_reduce_kernel.cu:100-169, which uses CUB radix sort + transition
// detection).
//
// Stable LSD radix sort (radix.hpp) of the int32 target ids with the edge index as value (small
// inputs: one workgroup sorting in LDS, csr_small).  Targets that arrive in order cost the sort's
// histogram read alone, which then also writes the identity result.
// Targets outside [0, N) get key N and sort after all valid targets.  node_start/node_end come
// from the transitions of the sorted keys (node_start[n] = first position with key >= n), so
// empty targets get start == end and no atomics are involved.
#include <mutex>

#include "radix.hpp"

namespace geo {
namespace {

// Node bounds of sorted keys (after a sort of unsorted input; sorted input gets its bounds from
// the sort's first histogram): positions 0..E (position E standing for key N) in tiles of
// kRxTile, each wave's 1024 positions staged in LDS for rx_wave_bounds.  Runs only when *active
// is set; sets *fallback when a wave's span covers too many nodes.
__global__ __launch_bounds__(kRxThreads) void csr_bounds_runs(const int32_t* __restrict__ sorted_keys,
                                                              int64_t E, int64_t N,
                                                              int32_t* __restrict__ node_start,
                                                              int32_t* __restrict__ node_end,
                                                              uint32_t* __restrict__ fallback,
                                                              const uint32_t* __restrict__ active,
                                                              int64_t ntiles) {
  if (*active == 0u) return;
  __shared__ uint32_t s_keys[kRxWaves][kRxWaveSpan];
  const int w = threadIdx.x / kWave;
  const int lane = lane_id();
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t wbase = tile * kRxTile + static_cast<int64_t>(w) * kRxWaveSpan;
    if (wbase > E) continue;  // wave-uniform
    const int64_t before = wbase > 0 ? static_cast<int64_t>(sorted_keys[wbase - 1]) : -1;
    uint32_t kv[kRxItems];  // clamped, unconditional loads, then the selects and LDS writes
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      kv[i] = static_cast<uint32_t>(sorted_keys[idx < E ? idx : E - 1]);
    }
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      if (idx <= E) s_keys[w][i * kWave + lane] = idx < E ? kv[i] : static_cast<uint32_t>(N);
    }
    wave_lds_fence();
    const int cnt = static_cast<int>(min(static_cast<int64_t>(kRxWaveSpan), E + 1 - wbase));
    const bool ok = rx_wave_bounds(s_keys[w], cnt, wbase, before, s_keys[w][cnt - 1], node_start,
                                   node_end, N);
    if (!ok && lane == 0) *fallback = 1u;  // plain store: many waves may set it
    wave_lds_fence();  // the next tile's staging follows this tile's searches
  }
}

// Thread n in [0, N] computes lb(n) by binary search over the sorted keys; runs only when
// *active is set (a wave found gaps too long to write).
constexpr int64_t kCsrBoundsGrid = 256;  // workgroups of the fallback bounds kernel

__global__ void csr_bounds(const int32_t* __restrict__ sorted_keys, int64_t E, int64_t N,
                           int32_t* __restrict__ node_start, int32_t* __restrict__ node_end,
                           const uint32_t* __restrict__ active) {
  if (*active == 0u) return;
  for (int64_t n = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; n <= N;
       n += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t lo = 0, hi = E;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (static_cast<int64_t>(sorted_keys[mid]) < n) lo = mid + 1; else hi = mid;
    }
    if (n < N) node_start[n] = static_cast<int32_t>(lo);
    if (n > 0) node_end[n - 1] = static_cast<int32_t>(lo);
  }
}

// Small inputs (E <= kCsrSmallMaxE, N <= kCsrSmallMaxN) in one launch: one workgroup holds the
// (key, index) pairs in LDS as 64-bit words key << 32 | index; input already in key order is
// written as it is, anything else is first sorted in LDS by a stable LSD radix sort of the keys
// (two 8-bit passes: keys <= N < 2^16); the bounds are binary searches in the LDS keys.  The
// radix path costs about a dozen launches, which for a few thousand edges is most of its time.
constexpr int kCsrSmallThreads = 1024;
constexpr int kCsrSmallWaves = kCsrSmallThreads / kWave;
constexpr int kCsrSmallChunks = 2;
constexpr int kCsrSmallMaxE = kCsrSmallChunks * kCsrSmallThreads;
constexpr int64_t kCsrSmallMaxN = 16384;
constexpr int kCsrSmallCounts = 256 * kCsrSmallChunks * kCsrSmallWaves;  // (digit, chunk, wave)
static_assert(kCsrSmallCounts == 8 * kCsrSmallThreads, "eight counters per thread in the scan");

__global__ __launch_bounds__(kCsrSmallThreads) void csr_small(const int64_t* __restrict__ col, int E,
                                                             int N, int32_t* __restrict__ col_sorted,
                                                             int32_t* __restrict__ perm,
                                                             int32_t* __restrict__ node_start,
                                                             int32_t* __restrict__ node_end) {
  __shared__ uint64_t s_kv[kCsrSmallMaxE];
  __shared__ uint64_t s_tmp[kCsrSmallMaxE];
  __shared__ uint32_t s_cnt[kCsrSmallCounts];
  __shared__ uint32_t s_wsum[kCsrSmallWaves];
  __shared__ int s_down;
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  if (t == 0) s_down = 0;
  for (int i = t; i < E; i += kCsrSmallThreads) {
    const int64_t c = col[i];
    const uint32_t k = (c >= 0 && c < N) ? static_cast<uint32_t>(c) : static_cast<uint32_t>(N);
    s_kv[i] = (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(i);
  }
  __syncthreads();
  bool down = false;
  for (int i = t + 1; i < E; i += kCsrSmallThreads) down |= (s_kv[i] >> 32) < (s_kv[i - 1] >> 32);
  if (down) s_down = 1;
  __syncthreads();
  if (s_down) {  // block-uniform
    // element c * kCsrSmallThreads + t of a pass's source is thread t's chunk c, so the order
    // (digit, chunk, wave, lane) is the stable order of the pass
    const uint64_t lt = lanemask_lt();
    uint64_t* src = s_kv;
    uint64_t* dst = s_tmp;
    for (int pass = 0; pass < 2; ++pass) {
      const int shift = 32 + 8 * pass;
      for (int q = t; q < kCsrSmallCounts; q += kCsrSmallThreads) s_cnt[q] = 0;
      __syncthreads();
      uint64_t v[kCsrSmallChunks];
      uint32_t d[kCsrSmallChunks], r[kCsrSmallChunks];
      bool ok[kCsrSmallChunks];
#pragma unroll
      for (int c = 0; c < kCsrSmallChunks; ++c) {
        const int i = c * kCsrSmallThreads + t;
        ok[c] = i < E;
        v[c] = ok[c] ? src[i] : 0ull;
        d[c] = static_cast<uint32_t>(v[c] >> shift) & 255u;
        const uint64_t peers = rx_peers<8>(d[c], ok[c]);  // same digit, same chunk and wave
        r[c] = static_cast<uint32_t>(__popcll(peers & lt));
        if (ok[c] && r[c] == 0)
          s_cnt[(d[c] * kCsrSmallChunks + c) * kCsrSmallWaves + w] = static_cast<uint32_t>(__popcll(peers));
      }
      __syncthreads();
      uint32_t loc[8], sum = 0;  // exclusive scan of the counters in place, eight per thread
#pragma unroll
      for (int j = 0; j < 8; ++j) { loc[j] = s_cnt[8 * t + j]; sum += loc[j]; }
      const uint32_t inc = wave_inclusive_sum_dpp(sum);
      if (lane == kWave - 1) s_wsum[w] = inc;
      __syncthreads();
      uint32_t off = inc - sum;
      for (int ww = 0; ww < w; ++ww) off += s_wsum[ww];
#pragma unroll
      for (int j = 0; j < 8; ++j) { s_cnt[8 * t + j] = off; off += loc[j]; }
      __syncthreads();
#pragma unroll
      for (int c = 0; c < kCsrSmallChunks; ++c)
        if (ok[c]) dst[s_cnt[(d[c] * kCsrSmallChunks + c) * kCsrSmallWaves + w] + r[c]] = v[c];
      __syncthreads();
      uint64_t* tmp = src;
      src = dst;
      dst = tmp;
    }
    // two passes: the result is back in s_kv
  }
  for (int i = t; i < E; i += kCsrSmallThreads) {
    const uint64_t v = s_kv[i];
    col_sorted[i] = static_cast<int32_t>(v >> 32);
    perm[i] = static_cast<int32_t>(static_cast<uint32_t>(v));
  }
  for (int n = t; n <= N; n += kCsrSmallThreads) {  // lb(n): node_start[n], node_end[n - 1]
    int lo = 0, hi = E;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (static_cast<uint32_t>(s_kv[mid] >> 32) < static_cast<uint32_t>(n)) lo = mid + 1; else hi = mid;
    }
    if (n < N) node_start[n] = lo;
    if (n > 0) node_end[n - 1] = lo;
  }
}

int radix_key_bits(int64_t N) {
  int bits = 0;
  while (bits < 32 && (static_cast<uint64_t>(N) >> bits) != 0) ++bits;  // bits to hold key N
  return bits == 0 ? 1 : bits;
}

RadixBuffers carve_csr(void* base, int64_t E, int64_t N, size_t* bytes) {
  Carver c(base);
  RadixBuffers r = carve_radix(c, E, radix_key_bits(N));
  *bytes = c.used;
  return r;
}

// The sort and the bounds, given the scratch (E > 0 or N > 0 checked by the caller).
int csr_build_into(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted, int32_t* perm,
                   int32_t* node_start, int32_t* node_end, const RadixBuffers& w, hipStream_t st) {
  if (E == 0) {
    if (N == 0) return GEO_OK;
    int rc = device_fill<int32_t>(node_start, N, 0, st);
    if (rc) return rc;
    return device_fill<int32_t>(node_end, N, 0, st);
  }
  if (E <= kCsrSmallMaxE && N <= kCsrSmallMaxN) {
    hipLaunchKernelGGL(csr_small, dim3(1), dim3(kCsrSmallThreads), 0, st, col, static_cast<int>(E),
                       static_cast<int>(N), col_sorted, perm, node_start, node_end);
    GEO_LAUNCH_CHECK("csr_small");
    return GEO_OK;
  }
  // targets that arrive sorted (a radius graph's output, CSR-ordered messages) cost one read,
  // which also writes the identity result and the node bounds
  RxDetect det;
  if (N > 0) {
    det.node_start = node_start;
    det.node_end = node_end;
    det.nodes = N;
  }
  int rc = radix_sort<kRxCol64>(col, nullptr, E, N, reinterpret_cast<uint32_t*>(col_sorted),
                                reinterpret_cast<uint32_t*>(perm), w, st, &det);
  if (rc) return rc;
  if (N > 0) {
    const int64_t ptiles = ceil_div(E + 1, kRxTile);
    hipLaunchKernelGGL(csr_bounds_runs, dim3(ptiles < kRxGrid ? ptiles : kRxGrid),
                       dim3(kRxThreads), 0, st, col_sorted, E, N, node_start, node_end, w.aux,
                       w.unsorted, ptiles);
    GEO_LAUNCH_CHECK("csr_bounds_runs");
    // the fallback runs only when a wave's keys spanned too many nodes; it strides over the
    // nodes, so a small grid does its work and costs little when it only reads its flag
    const int64_t nblocks = ceil_div(N + 1, 256);
    hipLaunchKernelGGL(csr_bounds, dim3(nblocks < kCsrBoundsGrid ? nblocks : kCsrBoundsGrid),
                       dim3(256), 0, st, col_sorted, E, N, node_start, node_end, w.aux);
    GEO_LAUNCH_CHECK("csr_bounds");
  }
  return GEO_OK;
}

int csr_check_args(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted, int32_t* perm,
                   int32_t* node_start, int32_t* node_end) {
  GEO_REQUIRE(E >= 0 && N >= 0, "csr_build: negative size (E=%lld N=%lld)", (long long)E,
              (long long)N);
  GEO_REQUIRE(E < 0x7fffffffLL && N < 0x7fffffffLL, "csr_build: sizes exceed int32 indexing");
  GEO_REQUIRE(N == 0 || (node_start && node_end), "csr_build: null node_start/node_end");
  GEO_REQUIRE(E == 0 || (col && col_sorted && perm), "csr_build: null edge arrays");
  return GEO_OK;
}

// ------------------------------------------------------- build without allocation ---
// Scratch of geo_csr_build_noalloc: one file-scope device array, so the entry point needs no
// workspace argument and performs no allocation.  Sized for kNoAllocMaxEdges edges and any N
// (the radix buffers: intermediate keys and values, the per-tile digit counts and offsets, the
// look-back words of four 8-bit passes' scans and the flags; 8.5 MiB at 2^20 edges).  The
// array is part of the library's code object, so every GPU on which the library is loaded holds
// its own copy, at its own address, from the load until the process ends, whether or not this
// entry point is called.  The host never passes `scratch` itself to a kernel (in host code it
// is a stand-in symbol, not a device address) but the address hipGetSymbolAddress returns for
// the current device.
constexpr int64_t kNoAllocMaxEdges = int64_t{1} << 20;
constexpr size_t kNoAllocScratchBytes = size_t{9} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kNoAllocMaxDevices];  // device address of `scratch` per device, set once

// Device address of `scratch` on the current device (looked up on the first call per device).
int noalloc_scratch(void** out) {
  int dev = -1;
  GEO_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(GEO_ERR_UNSUPPORTED, "csr_build_noalloc: device %d beyond the %d supported",
                     dev, kNoAllocMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    GEO_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr)
      return set_error(GEO_ERR_HIP, "csr_build_noalloc: no device address for the scratch array");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return GEO_OK;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_csr_workspace_bytes(int64_t E, int64_t N) {
  if (E < 0 || N < 0) return 0;
  size_t bytes = 0;
  carve_csr(nullptr, E, N, &bytes);
  return bytes;
}

extern "C" int geo_csr_build(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted,
                             int32_t* perm, int32_t* node_start, int32_t* node_end,
                             void* workspace, size_t workspace_bytes, void* stream) {
  int rc = csr_check_args(col, E, N, col_sorted, perm, node_start, node_end);
  if (rc) return rc;
  size_t need = 0;
  const RadixBuffers w = carve_csr(workspace, E, N, &need);
  if (workspace_bytes < need || workspace == nullptr)
    return set_error(GEO_ERR_WORKSPACE, "csr_build: workspace %zu bytes, need %zu",
                     workspace_bytes, need);
  return csr_build_into(col, E, N, col_sorted, perm, node_start, node_end, w, as_stream(stream));
}

extern "C" int geo_csr_build_noalloc(const int64_t* col, int64_t E, int64_t N,
                                     int32_t* col_sorted, int32_t* perm, int32_t* node_start,
                                     int32_t* node_end, void* stream) {
  int rc = csr_check_args(col, E, N, col_sorted, perm, node_start, node_end);
  if (rc) return rc;
  if (E > kNoAllocMaxEdges)
    return set_error(GEO_ERR_INVALID,
                     "csr_build_noalloc: %lld edges exceed the %lld its fixed scratch holds "
                     "(use geo_csr_build with a workspace)",
                     (long long)E, (long long)kNoAllocMaxEdges);
  size_t need = 0;
  carve_csr(nullptr, E, N, &need);
  if (need > kNoAllocScratchBytes)  // cannot happen for E <= kNoAllocMaxEdges
    return set_error(GEO_ERR_INVALID, "csr_build_noalloc: needs %zu scratch bytes, has %zu", need,
                     kNoAllocScratchBytes);
  hipStream_t st = as_stream(stream);
  void* base = nullptr;
  rc = noalloc_scratch(&base);
  if (rc) return rc;
  if (st != nullptr) {
    int sdev = -1, cur = -1;
    GEO_HIP_CHECK(hipStreamGetDevice(st, &sdev));
    GEO_HIP_CHECK(hipGetDevice(&cur));
    GEO_REQUIRE(sdev == cur, "csr_build_noalloc: stream of device %d, current device %d", sdev,
                cur);
  }
  const RadixBuffers w = carve_csr(base, E, N, &need);
  return csr_build_into(col, E, N, col_sorted, perm, node_start, node_end, w, st);
}
