// knn.hip — k nearest neighbours per query within its cloud, on gfx950.
//
// Replaces knn_kernel<MAX_K> + build_batch_map_kernel (geoembodied/csrc/knn_kernel.cu:113-193)
// with the semantics of _knn_bruteforce (geoembodied/csrc/__init__.py:435-492) made total: the
// k smallest keys (d, j), ascending, padded with -1 / 1e30f.
//
// One 256-thread workgroup serves up to 256 queries of a single cloud (a prepare kernel maps
// workgroups to (cloud, query tile) without a host round trip).  The cloud's sources stream
// through LDS in 1024-point tiles; every thread reads the same LDS entry at a time (broadcast,
// no bank conflicts) and keeps its candidates as a sorted register array.  Sources arrive in
// ascending index order, so a new candidate enters the list only on a strictly smaller
// distance and lands after every equal one — exactly the (d, j) order.
// Non-finite distances never enter the list (they report as padding).
#include "scan.hpp"

namespace geo {
namespace {

constexpr int kKnnThreads = 256;
constexpr int kKnnTile = 1024;

// tiles[b] = first workgroup of cloud b; tiles[B] = total workgroups.  Offsets are clamped to
// [0, N] so inconsistent ptr arrays stay memory-safe.
__global__ __launch_bounds__(kScanThreads) void knn_prepare_kernel(const int64_t* __restrict__ ptr_q,
                                                                   int64_t B, int64_t Nq,
                                                                   int64_t* __restrict__ tiles) {
  __shared__ int64_t lds[kScanThreads / kWave];
  int64_t carry = 0;
  for (int64_t base = 0; base < B; base += kScanThreads) {
    const int64_t b = base + threadIdx.x;
    int64_t nt = 0;
    if (b < B) {
      int64_t a = ptr_q[b], c = ptr_q[b + 1];
      a = a < 0 ? 0 : (a > Nq ? Nq : a);
      c = c < a ? a : (c > Nq ? Nq : c);
      nt = (c - a + kKnnThreads - 1) / kKnnThreads;
    }
    int64_t total;
    const int64_t off = block_exclusive_scan<int64_t>(nt, lds, total);
    if (b < B) tiles[b] = carry + off;
    carry += total;
  }
  if (threadIdx.x == 0) tiles[B] = carry;
}

template <int KMAX>
__global__ __launch_bounds__(kKnnThreads) void knn_kernel(
    const float* __restrict__ query, int64_t Nq, const float* __restrict__ source, int64_t Ns,
    const int64_t* __restrict__ ptr_q, const int64_t* __restrict__ ptr_s,
    const int64_t* __restrict__ tiles, int64_t B, int k, int64_t* __restrict__ out_idx,
    float* __restrict__ out_dist) {
  __shared__ float4 tile[kKnnTile];
  const int64_t blk = blockIdx.x;
  if (blk >= tiles[B]) return;
  // cloud of this workgroup: last b with tiles[b] <= blk
  int64_t lo = 0, hi = B - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (tiles[mid] <= blk) lo = mid; else hi = mid - 1;
  }
  const int64_t b = lo;
  int64_t qa = ptr_q[b], qc = ptr_q[b + 1];
  qa = qa < 0 ? 0 : (qa > Nq ? Nq : qa);
  qc = qc < qa ? qa : (qc > Nq ? Nq : qc);
  int64_t sa = ptr_s[b], sc = ptr_s[b + 1];
  sa = sa < 0 ? 0 : (sa > Ns ? Ns : sa);
  sc = sc < sa ? sa : (sc > Ns ? Ns : sc);
  const int64_t q = qa + (blk - tiles[b]) * kKnnThreads + threadIdx.x;
  const bool qok = q < qc;

  float qx = 0.f, qy = 0.f, qz = 0.f;
  if (qok) {
    qx = query[3 * q];
    qy = query[3 * q + 1];
    qz = query[3 * q + 2];
  }
  float D[KMAX];
  int J[KMAX];
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    D[i] = __builtin_inff();
    J[i] = -1;
  }
  for (int64_t s0 = sa; s0 < sc; s0 += kKnnTile) {
    const int n = static_cast<int>(min(static_cast<int64_t>(kKnnTile), sc - s0));
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kKnnThreads) {
      const float* p = source + 3 * (s0 + i);
      tile[i] = make_float4(p[0], p[1], p[2], 0.f);
    }
    __syncthreads();
    for (int i = 0; i < n; ++i) {
      const float4 p = tile[i];
      const float d = sqdist(qx, qy, qz, p.x, p.y, p.z);
      if (d < D[KMAX - 1]) {
        const int j = static_cast<int>(s0 + i);
#pragma unroll
        for (int m = KMAX - 1; m > 0; --m) {
          const bool shift = d < D[m - 1];
          const bool here = !shift && d < D[m];
          D[m] = shift ? D[m - 1] : (here ? d : D[m]);
          J[m] = shift ? J[m - 1] : (here ? j : J[m]);
        }
        if (d < D[0]) {
          D[0] = d;
          J[0] = j;
        }
      }
    }
  }
  if (qok) {
    int64_t* oi = out_idx + q * k;
    float* od = out_dist + q * k;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      if (i < k) {
        oi[i] = J[i] >= 0 ? static_cast<int64_t>(J[i]) : -1;
        od[i] = J[i] >= 0 ? D[i] : 1e30f;
      }
    }
  }
}

template <int KMAX>
int launch_knn(const float* query, int64_t Nq, const float* source, int64_t Ns,
               const int64_t* ptr_q, const int64_t* ptr_s, const int64_t* tiles, int64_t B, int k,
               int64_t* out_idx, float* out_dist, hipStream_t st) {
  const int64_t grid = ceil_div(Nq, kKnnThreads) + B;
  hipLaunchKernelGGL((knn_kernel<KMAX>), dim3(grid), dim3(kKnnThreads), 0, st, query, Nq, source,
                     Ns, ptr_q, ptr_s, tiles, B, k, out_idx, out_dist);
  GEO_LAUNCH_CHECK("knn_kernel");
  return GEO_OK;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_knn_workspace_bytes(int64_t Nq, int64_t Ns, int64_t B, int64_t k) {
  (void)Nq; (void)Ns; (void)k;
  return static_cast<size_t>((B > 0 ? B : 0) + 1) * sizeof(int64_t);
}

extern "C" int geo_knn(const float* query, int64_t Nq, const float* source, int64_t Ns,
                       const int64_t* ptr_q, const int64_t* ptr_s, int64_t B, int64_t k,
                       int64_t* out_idx, float* out_dist, void* workspace, size_t workspace_bytes,
                       void* stream) {
  GEO_REQUIRE(Nq >= 0 && Ns >= 0 && B >= 0, "knn: negative size");
  GEO_REQUIRE(k >= 0, "knn: k must be non-negative (got %lld)", (long long)k);
  GEO_REQUIRE(k <= 128, "knn: k=%lld above the supported maximum of 128", (long long)k);
  GEO_REQUIRE(Nq < 0x7fffffffLL && Ns < 0x7fffffffLL, "knn: sizes exceed int32 indexing");
  if (Nq == 0 || k == 0) return GEO_OK;
  GEO_REQUIRE(query && out_idx && out_dist && ptr_q && ptr_s, "knn: null pointer");
  const size_t need = geo_knn_workspace_bytes(Nq, Ns, B, k);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(GEO_ERR_WORKSPACE, "knn: workspace %zu bytes, need %zu", workspace_bytes,
                     need);
  hipStream_t st = as_stream(stream);
  int64_t* tiles = static_cast<int64_t*>(workspace);
  if (B == 0) {
    // no clouds: every query row is padding
    int rc = device_fill<int64_t>(out_idx, Nq * k, -1, st);
    if (rc) return rc;
    return device_fill<float>(out_dist, Nq * k, 1e30f, st);
  }
  // Queries outside every cloud keep padding: pre-fill only when the clouds may not cover Nq.
  int rc = device_fill<int64_t>(out_idx, Nq * k, -1, st);
  if (rc) return rc;
  rc = device_fill<float>(out_dist, Nq * k, 1e30f, st);
  if (rc) return rc;
  hipLaunchKernelGGL(knn_prepare_kernel, dim3(1), dim3(kScanThreads), 0, st, ptr_q, B, Nq, tiles);
  GEO_LAUNCH_CHECK("knn_prepare_kernel");
  GEO_REQUIRE(Ns == 0 || source != nullptr, "knn: null source");
  const int kk = static_cast<int>(k);
#define GEO_KNN_CASE(KV) \
  if (kk <= KV) return launch_knn<KV>(query, Nq, source, Ns, ptr_q, ptr_s, tiles, B, kk, out_idx, out_dist, st);
  GEO_KNN_CASE(1) GEO_KNN_CASE(2) GEO_KNN_CASE(3) GEO_KNN_CASE(4) GEO_KNN_CASE(5)
  GEO_KNN_CASE(6) GEO_KNN_CASE(7) GEO_KNN_CASE(8) GEO_KNN_CASE(10) GEO_KNN_CASE(12)
  GEO_KNN_CASE(16) GEO_KNN_CASE(24) GEO_KNN_CASE(32) GEO_KNN_CASE(48) GEO_KNN_CASE(64)
  GEO_KNN_CASE(96) GEO_KNN_CASE(128)
#undef GEO_KNN_CASE
  return set_error(GEO_ERR_UNSUPPORTED, "knn: k=%d unsupported", kk);
}
