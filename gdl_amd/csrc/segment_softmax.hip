// segment_softmax.hip — softmax over the edges of each target segment, forward and backward.
//
// Replaces _sparse_softmax (geoembodied/nn/modules/invariant_attention.py:202-230), which runs
// scatter_reduce('amax') + gather + exp + scatter_add + gather + divide as six PyTorch kernels
// with atomics, with one kernel per direction over the CSR of the targets:
//
//   m[s,h] = max_e x[e,h],  z[s,h] = sum_e exp(x[e,h] - m[s,h]),
//   w[e,h] = exp(x[e,h] - m[s,h]) / max(z[s,h], 1e-8)            for e in segment s
//   dx[e,h] = w[e,h] * (g[e,h] - sum_{e' in s} g[e',h] w[e',h])    (backward)
//
// with x[e] = scores[perm[e]] (perm may be NULL).  One thread per (segment, head); the segment
// is walked three times (max, sum, write), so the exponentials that are summed are exactly the
// ones that are divided; the sum runs in ascending edge order.  Rows are H consecutive values,
// so the H threads of a segment read one row together.
#include "common.hpp"

namespace geo {
namespace {

constexpr int kSmThreads = 256;

template <typename T>
__device__ __forceinline__ T exp_t(T v);
template <>
__device__ __forceinline__ float exp_t<float>(float v) { return expf(v); }
template <>
__device__ __forceinline__ double exp_t<double>(double v) { return exp(v); }

__device__ __forceinline__ int clamp_idx(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

template <typename T>
__global__ __launch_bounds__(kSmThreads) void seg_softmax_fwd_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ perm, const int32_t* __restrict__ ns,
    const int32_t* __restrict__ ne, int32_t E, int64_t S, int32_t H, T* __restrict__ w) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= S * H) return;
  const int64_t s = t / H;
  const int h = static_cast<int>(t - s * H);
  const int a = clamp_idx(ns[s], 0, E);
  const int b = clamp_idx(ne[s], a, E);
  auto row = [&](int e) -> int64_t {
    const int r = perm ? perm[e] : e;
    return static_cast<unsigned>(r) < static_cast<unsigned>(E) ? r : -1;
  };
  // max (NaN propagates, as torch.amax does)
  T m = -__builtin_inf();
  bool nan = false;
  for (int e = a; e < b; ++e) {
    const int64_t r = row(e);
    if (r < 0) continue;
    const T v = x[r * H + h];
    nan |= v != v;
    m = v > m ? v : m;
  }
  if (nan) m = __builtin_nan("");
  T z = T(0);
  for (int e = a; e < b; ++e) {
    const int64_t r = row(e);
    if (r < 0) continue;
    z += exp_t<T>(x[r * H + h] - m);
  }
  const T den = z < T(1e-8) ? T(1e-8) : z;  // clamp(min=1e-8) keeps NaN, as torch's does
  for (int e = a; e < b; ++e) {
    const int64_t r = row(e);
    if (r < 0) continue;
    w[r * H + h] = exp_t<T>(x[r * H + h] - m) / den;
  }
}

template <typename T>
__global__ __launch_bounds__(kSmThreads) void seg_softmax_bwd_kernel(
    const T* __restrict__ g, const T* __restrict__ w, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ ns, const int32_t* __restrict__ ne, int32_t E, int64_t S,
    int32_t H, T* __restrict__ dx) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= S * H) return;
  const int64_t s = t / H;
  const int h = static_cast<int>(t - s * H);
  const int a = clamp_idx(ns[s], 0, E);
  const int b = clamp_idx(ne[s], a, E);
  auto row = [&](int e) -> int64_t {
    const int r = perm ? perm[e] : e;
    return static_cast<unsigned>(r) < static_cast<unsigned>(E) ? r : -1;
  };
  T dot = T(0);
  for (int e = a; e < b; ++e) {
    const int64_t r = row(e);
    if (r < 0) continue;
    dot += g[r * H + h] * w[r * H + h];
  }
  for (int e = a; e < b; ++e) {
    const int64_t r = row(e);
    if (r < 0) continue;
    const T wv = w[r * H + h];
    dx[r * H + h] = wv * (g[r * H + h] - dot);
  }
}

}  // namespace
}  // namespace geo

using namespace geo;

static int sm_check(int dtype, int64_t E, int64_t S, int64_t H) {
  GEO_REQUIRE(dtype == GEO_F32 || dtype == GEO_F64, "segment_softmax: dtype must be f32 or f64 (got %d)",
              dtype);
  GEO_REQUIRE(E >= 0 && S >= 0 && H >= 0, "segment_softmax: negative size");
  GEO_REQUIRE(E < 0x7fffffffLL && H < 0x7fffffffLL, "segment_softmax: sizes exceed int32 indexing");
  return GEO_OK;
}

extern "C" int geo_segment_softmax_fwd(int dtype, const void* scores, const int32_t* perm,
                                       const int32_t* node_start, const int32_t* node_end,
                                       int64_t E, int64_t S, int64_t H, void* out, void* stream) {
  int rc = sm_check(dtype, E, S, H);
  if (rc) return rc;
  if (S == 0 || H == 0 || E == 0) return GEO_OK;
  GEO_REQUIRE(scores && out && node_start && node_end, "segment_softmax: null pointer");
  const unsigned grid = static_cast<unsigned>(ceil_div(S * H, kSmThreads));
  hipStream_t st = as_stream(stream);
  if (dtype == GEO_F32)
    hipLaunchKernelGGL(seg_softmax_fwd_kernel<float>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(scores), perm, node_start, node_end,
                       static_cast<int32_t>(E), S, static_cast<int32_t>(H), static_cast<float*>(out));
  else
    hipLaunchKernelGGL(seg_softmax_fwd_kernel<double>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const double*>(scores), perm, node_start, node_end,
                       static_cast<int32_t>(E), S, static_cast<int32_t>(H), static_cast<double*>(out));
  GEO_LAUNCH_CHECK("seg_softmax_fwd_kernel");
  return GEO_OK;
}

extern "C" int geo_segment_softmax_bwd(int dtype, const void* grad_out, const void* out,
                                       const int32_t* perm, const int32_t* node_start,
                                       const int32_t* node_end, int64_t E, int64_t S, int64_t H,
                                       void* grad_scores, void* stream) {
  int rc = sm_check(dtype, E, S, H);
  if (rc) return rc;
  if (S == 0 || H == 0 || E == 0) return GEO_OK;
  GEO_REQUIRE(grad_out && out && grad_scores && node_start && node_end,
              "segment_softmax_bwd: null pointer");
  const unsigned grid = static_cast<unsigned>(ceil_div(S * H, kSmThreads));
  hipStream_t st = as_stream(stream);
  if (dtype == GEO_F32)
    hipLaunchKernelGGL(seg_softmax_bwd_kernel<float>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(grad_out), static_cast<const float*>(out), perm,
                       node_start, node_end, static_cast<int32_t>(E), S, static_cast<int32_t>(H),
                       static_cast<float*>(grad_scores));
  else
    hipLaunchKernelGGL(seg_softmax_bwd_kernel<double>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const double*>(grad_out), static_cast<const double*>(out), perm,
                       node_start, node_end, static_cast<int32_t>(E), S, static_cast<int32_t>(H),
                       static_cast<double*>(grad_scores));
  GEO_LAUNCH_CHECK("seg_softmax_bwd_kernel");
  return GEO_OK;
}
