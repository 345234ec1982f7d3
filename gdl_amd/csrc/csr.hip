// csr.hip — stable CSR build (replaces sort_and_build_csr,
// geoembodied/csrc/segment_reduce_kernel.cu:100-169, which uses CUB radix sort + transition
// detection).
//
// Stable LSD radix sort (radix.hpp) of the int32 target ids with the edge index as value.
// Targets outside [0, N) get key N and sort after all valid targets.  node_start/node_end come
// from binary searches in the sorted keys (node_start[n] = first position with key >= n), so
// empty targets get start == end and no atomics are involved.
#include "radix.hpp"

namespace geo {
namespace {

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

int radix_key_bits(int64_t N) {
  int bits = 0;
  while (bits < 32 && (static_cast<uint64_t>(N) >> bits) != 0) ++bits;  // bits to hold key N
  return bits == 0 ? 1 : bits;
}

RadixBuffers carve_csr(void* base, int64_t E, size_t* bytes) {
  Carver c(base);
  RadixBuffers r = carve_radix(c, E);
  *bytes = c.used;
  return r;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_csr_workspace_bytes(int64_t E, int64_t N) {
  if (E < 0 || N < 0) return 0;
  size_t bytes = 0;
  carve_csr(nullptr, E, &bytes);
  return bytes;
}

extern "C" int geo_csr_build(const int64_t* col, int64_t E, int64_t N, int32_t* col_sorted,
                             int32_t* perm, int32_t* node_start, int32_t* node_end,
                             void* workspace, size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(E >= 0 && N >= 0, "csr_build: negative size (E=%lld N=%lld)", (long long)E,
              (long long)N);
  GEO_REQUIRE(E < 0x7fffffffLL && N < 0x7fffffffLL, "csr_build: sizes exceed int32 indexing");
  hipStream_t st = as_stream(stream);
  size_t need = 0;
  const RadixBuffers w = carve_csr(workspace, E, &need);
  if (workspace_bytes < need || workspace == nullptr)
    return set_error(GEO_ERR_WORKSPACE, "csr_build: workspace %zu bytes, need %zu",
                     workspace_bytes, need);
  GEO_REQUIRE(N == 0 || (node_start && node_end), "csr_build: null node_start/node_end");
  GEO_REQUIRE(E == 0 || (col && col_sorted && perm), "csr_build: null edge arrays");

  if (E == 0) {
    if (N == 0) return GEO_OK;
    int rc = device_fill<int32_t>(node_start, N, 0, st);
    if (rc) return rc;
    return device_fill<int32_t>(node_end, N, 0, st);
  }

  // targets that arrive sorted (a radius graph's output, CSR-ordered messages) cost one pass
  int rc = radix_sort<kRxCol64>(col, nullptr, E, N, radix_key_bits(N),
                                reinterpret_cast<uint32_t*>(col_sorted),
                                reinterpret_cast<uint32_t*>(perm), w, st, true);
  if (rc) return rc;
  if (N > 0) {
    hipLaunchKernelGGL(csr_bounds, dim3(ceil_div(N + 1, 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t*>(col_sorted), E, N, node_start, node_end);
    GEO_LAUNCH_CHECK("csr_bounds");
  }
  return GEO_OK;
}

