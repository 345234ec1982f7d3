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

// Largest value over the wave (v >= 0; every lane active).
__device__ __forceinline__ int uniform_max(int v) {
  return static_cast<int>(wave_max_u32(static_cast<uint32_t>(v)));
}

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

// ------------------------------------------------------------------ fp32, H <= 8 ---
// Sixteen lanes (one DPP row) per segment, four segments per wave: lane li takes edges a + li,
// a + li + 16, ... with all H heads in registers, and the segment's max and sum are row
// reductions.  Segments of up to 16 edges (graph neighbourhoods) keep their scores in registers
// between the passes; longer ones re-read them.
constexpr int kSmRowHeads = 8;

template <int CTRL>
__device__ __forceinline__ float sm_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF,
                                                    0xF, false));
}
__device__ __forceinline__ float row_maxf(float v) {
  v = fmaxf(v, sm_dpp<kDppXor1>(v));
  v = fmaxf(v, sm_dpp<kDppXor2>(v));
  v = fmaxf(v, sm_dpp<kDppHalfMirror>(v));
  v = fmaxf(v, sm_dpp<kDppMirror>(v));
  return v;
}
__device__ __forceinline__ float row_sumf(float v) {
  v += sm_dpp<kDppXor1>(v);
  v += sm_dpp<kDppXor2>(v);
  v += sm_dpp<kDppHalfMirror>(v);
  v += sm_dpp<kDppMirror>(v);
  return v;
}

struct RowSeg {
  int a, b, li;
};

__device__ __forceinline__ RowSeg row_seg(const int32_t* ns, const int32_t* ne, int32_t E, int64_t S) {
  const int lane = lane_id();
  const int64_t s = (static_cast<int64_t>(blockIdx.x) * (kSmThreads / kWave) + threadIdx.x / kWave) * 4 +
                    (lane >> 4);
  RowSeg r;
  r.li = lane & 15;
  r.a = 0;
  r.b = 0;
  if (s < S) {
    r.a = clamp_idx(ns[s], 0, E);
    r.b = clamp_idx(ne[s], r.a, E);
  }
  return r;
}

__device__ __forceinline__ int sm_row(const int32_t* perm, int32_t E, int e) {
  const int r = perm ? perm[e] : e;
  return static_cast<unsigned>(r) < static_cast<unsigned>(E) ? r : -1;
}

__global__ __launch_bounds__(kSmThreads) void seg_softmax_rows_fwd(
    const float* __restrict__ x, const int32_t* __restrict__ perm, const int32_t* __restrict__ ns,
    const int32_t* __restrict__ ne, int32_t E, int64_t S, int32_t H, float* __restrict__ w) {
  const RowSeg g = row_seg(ns, ne, E, S);
  // chunks of 16 edges; every lane of the wave runs the wave's largest chunk count, so the row
  // reductions below see all sixteen lanes of every row.  The first two chunks (segments of up
  // to 32 edges) stay in registers between the passes.
  const int nch = uniform_max((g.b - g.a + 15) >> 4);
  float m[kSmRowHeads], z[kSmRowHeads], keep[2][kSmRowHeads];
  bool nan[kSmRowHeads];
  int rk[2] = {-1, -1};
#pragma unroll
  for (int h = 0; h < kSmRowHeads; ++h) {
    m[h] = -__builtin_inff(); z[h] = 0.f; nan[h] = false; keep[0][h] = 0.f; keep[1][h] = 0.f;
  }
  auto row_of = [&](int c) -> int {
    if (c < 2) return rk[c];
    const int e = g.a + 16 * c + g.li;
    return e < g.b ? sm_row(perm, E, e) : -1;
  };
  auto val = [&](int c, int r, int h) -> float {
    return c == 0 ? keep[0][h] : (c == 1 ? keep[1][h] : x[static_cast<int64_t>(r) * H + h]);
  };
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int e = g.a + 16 * c + g.li;
    rk[c] = (c < nch && e < g.b) ? sm_row(perm, E, e) : -1;
  }
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int h = 0; h < kSmRowHeads; ++h)
      if (h < H && rk[c] >= 0) keep[c][h] = x[static_cast<int64_t>(rk[c]) * H + h];
  for (int c = 0; c < nch; ++c) {
    const int r = row_of(c);
#pragma unroll
    for (int h = 0; h < kSmRowHeads; ++h) {
      if (h < H && r >= 0) {
        const float v = val(c, r, h);
        nan[h] |= v != v;
        m[h] = v > m[h] ? v : m[h];
      }
    }
  }
#pragma unroll
  for (int h = 0; h < kSmRowHeads; ++h) {
    if (h >= H) break;
    m[h] = row_maxf(m[h]);
    const bool anynan = row_maxf(nan[h] ? 1.f : 0.f) > 0.f;  // NaN propagates, as torch.amax does
    if (anynan) m[h] = __builtin_nanf("");
  }
  for (int c = 0; c < nch; ++c) {
    const int r = row_of(c);
#pragma unroll
    for (int h = 0; h < kSmRowHeads; ++h)
      if (h < H && r >= 0) z[h] += expf(val(c, r, h) - m[h]);
  }
#pragma unroll
  for (int h = 0; h < kSmRowHeads; ++h) {
    if (h >= H) break;
    const float zz = row_sumf(z[h]);
    z[h] = zz < 1e-8f ? 1e-8f : zz;  // clamp(min=1e-8) keeps NaN, as torch's does
  }
  for (int c = 0; c < nch; ++c) {
    const int r = row_of(c);
#pragma unroll
    for (int h = 0; h < kSmRowHeads; ++h)
      if (h < H && r >= 0) w[static_cast<int64_t>(r) * H + h] = expf(val(c, r, h) - m[h]) / z[h];
  }
}

__global__ __launch_bounds__(kSmThreads) void seg_softmax_rows_bwd(
    const float* __restrict__ g_, const float* __restrict__ w, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ ns, const int32_t* __restrict__ ne, int32_t E, int64_t S, int32_t H,
    float* __restrict__ dx) {
  const RowSeg g = row_seg(ns, ne, E, S);
  const int nch = uniform_max((g.b - g.a + 15) >> 4);
  float dot[kSmRowHeads], g0[kSmRowHeads], w0[kSmRowHeads];
  int r0 = -1;
#pragma unroll
  for (int h = 0; h < kSmRowHeads; ++h) { dot[h] = 0.f; g0[h] = 0.f; w0[h] = 0.f; }
  for (int c = 0; c < nch; ++c) {
    const int e = g.a + 16 * c + g.li;
    const int r = e < g.b ? sm_row(perm, E, e) : -1;
    if (c == 0) r0 = r;
#pragma unroll
    for (int h = 0; h < kSmRowHeads; ++h) {
      if (h < H && r >= 0) {
        const float gv = g_[static_cast<int64_t>(r) * H + h], wv = w[static_cast<int64_t>(r) * H + h];
        if (c == 0) { g0[h] = gv; w0[h] = wv; }
        dot[h] += gv * wv;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < kSmRowHeads; ++h) {
    if (h >= H) break;
    dot[h] = row_sumf(dot[h]);
  }
  for (int c = 0; c < nch; ++c) {
    const int e = g.a + 16 * c + g.li;
    const int r = c == 0 ? r0 : (e < g.b ? sm_row(perm, E, e) : -1);
#pragma unroll
    for (int h = 0; h < kSmRowHeads; ++h) {
      if (h < H && r >= 0) {
        const int64_t i = static_cast<int64_t>(r) * H + h;
        const float gv = c == 0 ? g0[h] : g_[i], wv = c == 0 ? w0[h] : w[i];
        dx[i] = wv * (gv - dot[h]);
      }
    }
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
  if (dtype == GEO_F32 && H <= kSmRowHeads) {
    const unsigned rgrid = static_cast<unsigned>(ceil_div(S, 4 * (kSmThreads / kWave)));
    hipLaunchKernelGGL(seg_softmax_rows_fwd, dim3(rgrid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(scores), perm, node_start, node_end,
                       static_cast<int32_t>(E), S, static_cast<int32_t>(H), static_cast<float*>(out));
  } else if (dtype == GEO_F32)
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
  if (dtype == GEO_F32 && H <= kSmRowHeads) {
    const unsigned rgrid = static_cast<unsigned>(ceil_div(S, 4 * (kSmThreads / kWave)));
    hipLaunchKernelGGL(seg_softmax_rows_bwd, dim3(rgrid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(grad_out), static_cast<const float*>(out), perm,
                       node_start, node_end, static_cast<int32_t>(E), S, static_cast<int32_t>(H),
                       static_cast<float*>(grad_scores));
  } else if (dtype == GEO_F32)
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
