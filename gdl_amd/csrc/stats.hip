// stats.hip — device-side neighbour-spacing statistics for adaptive radii, without a host sync.
//
// The reference estimates a graph radius from the nearest-neighbour distances of a KNN(k = 2)
// and reads it back to the host with .item() (geoembodied/nn/modules/
// multi_scale_se3_net.py:99-124: mean of sqrt(clamp(d, 1e-8, 1e20)) times a multiplier;
// equivariant_skip_fusion.py:243-248: median of sqrt(max(d, 1e-12)) times a multiplier).  Here the
// statistic is computed on the device and written as a float64 scalar that the radius graph
// reads directly (geo_radius_count_dev / geo_radius_emit_dev), so building an adaptive-radius
// graph costs no extra host round trip.
//
//   mean:   fp32 values v_i as the reference computes them, summed in fp64 in a fixed order
//           (per-block partials, then one block), divided by N and rounded to fp32 — the
//           reference's float32 mean, read back as a float64 — then times the multiplier.
//   median: the lower median (torch.median's choice for even N) of max(d_i, 1e-12), by the
//           radix sort of the non-negative float bit patterns, then sqrt and the multiplier;
//           NaN if any distance is NaN, as torch.median.
#include "radix.hpp"

namespace geo {
namespace {

constexpr int kStThreads = 256;
constexpr int kStMaxBlocks = 1024;

__global__ __launch_bounds__(kStThreads) void st_mean_partial(const float* __restrict__ dist,
                                                              int64_t N, int64_t k, int64_t col,
                                                              double* __restrict__ partial) {
  __shared__ double red[kStThreads / kWave];
  double s = 0.0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kStThreads + threadIdx.x; i < N;
       i += static_cast<int64_t>(gridDim.x) * kStThreads) {
    float d = dist[i * k + col];
    d = d > 1e20f ? 1e20f : d;  // clamp(max=1e20), then clamp(min=1e-8); NaN passes through
    d = d < 1e-8f ? 1e-8f : d;
    s += static_cast<double>(sqrtf(d));
  }
  for (int m = kWave / 2; m > 0; m >>= 1) s += __shfl_xor(s, m, kWave);
  if (lane_id() == 0) red[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < kStThreads / kWave; ++w) t += red[w];
    partial[blockIdx.x] = t;
  }
}

__global__ void st_mean_final(const double* __restrict__ partial, int nblocks, int64_t N,
                              double multiplier, double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  double t = 0.0;
  for (int b = 0; b < nblocks; ++b) t += partial[b];
  const float mean = static_cast<float>(t / static_cast<double>(N));
  *out = static_cast<double>(mean) * multiplier;
}

__global__ void st_median_keys(const float* __restrict__ dist, int64_t N, int64_t k, int64_t col,
                               uint32_t* __restrict__ keys) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  float d = dist[i * k + col];
  d = d < 1e-12f ? 1e-12f : d;  // clamp(min=1e-12); NaN passes through
  // non-negative floats (and NaN above +inf) order like their bit patterns
  keys[i] = d != d ? 0xffffffffu : __float_as_uint(d);
}

__global__ void st_median_final(const uint32_t* __restrict__ sorted, int64_t N, double multiplier,
                                double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  if (sorted[N - 1] == 0xffffffffu) {
    *out = __builtin_nan("");
    return;
  }
  const float m = __uint_as_float(sorted[(N - 1) / 2]);
  *out = static_cast<double>(sqrtf(m)) * multiplier;
}

struct StWs {
  double* partial;
  uint32_t *keys, *skeys, *order;
  RadixBuffers rx;
};

StWs carve_st(void* base, int64_t N, size_t* bytes) {
  Carver c(base);
  StWs w;
  const int64_t n = N > 0 ? N : 1;
  w.partial = c.take<double>(kStMaxBlocks);
  w.keys = c.take<uint32_t>(n);
  w.skeys = c.take<uint32_t>(n);
  w.order = c.take<uint32_t>(n);
  w.rx = carve_radix(c, n, 32);
  *bytes = c.used;
  return w;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_knn_radius_stat_workspace_bytes(int64_t N) {
  if (N < 0) return 0;
  size_t bytes = 0;
  carve_st(nullptr, N, &bytes);
  return bytes;
}

extern "C" int geo_knn_radius_stat(const float* dist, int64_t N, int64_t k, int64_t col, int mode,
                                   double multiplier, double* out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(N >= 1 && k >= 1 && col >= 0 && col < k,
              "knn_radius_stat: need N >= 1 and 0 <= col < k (N=%lld k=%lld col=%lld)",
              (long long)N, (long long)k, (long long)col);
  GEO_REQUIRE(N < 0x7fffffffLL, "knn_radius_stat: N exceeds int32 indexing");
  GEO_REQUIRE(mode == 0 || mode == 1, "knn_radius_stat: mode must be 0 (mean) or 1 (median)");
  GEO_REQUIRE(dist && out, "knn_radius_stat: null pointer");
  size_t need = 0;
  const StWs w = carve_st(workspace, N, &need);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(GEO_ERR_WORKSPACE, "knn_radius_stat: workspace %zu bytes, need %zu",
                     workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  if (mode == 0) {
    int64_t blocks = ceil_div(N, kStThreads * 8);
    if (blocks > kStMaxBlocks) blocks = kStMaxBlocks;
    hipLaunchKernelGGL(st_mean_partial, dim3(blocks), dim3(kStThreads), 0, st, dist, N, k, col,
                       w.partial);
    GEO_LAUNCH_CHECK("st_mean_partial");
    hipLaunchKernelGGL(st_mean_final, dim3(1), dim3(64), 0, st, w.partial, static_cast<int>(blocks),
                       N, multiplier, out);
    GEO_LAUNCH_CHECK("st_mean_final");
    return GEO_OK;
  }
  hipLaunchKernelGGL(st_median_keys, dim3(static_cast<unsigned>(ceil_div(N, 256))), dim3(256), 0, st,
                     dist, N, k, col, w.keys);
  GEO_LAUNCH_CHECK("st_median_keys");
  int rc = radix_sort<kRxKeysIota>(w.keys, nullptr, N, 0, w.skeys, w.order, w.rx, st);
  if (rc) return rc;
  hipLaunchKernelGGL(st_median_final, dim3(1), dim3(64), 0, st, w.skeys, N, multiplier, out);
  GEO_LAUNCH_CHECK("st_median_final");
  return GEO_OK;
}
