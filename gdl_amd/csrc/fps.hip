// fps.hip — farthest-point sampling for packed point clouds on gfx950.
//
// Replaces fps_kernel<512> (geoembodied/csrc/fps_kernel.cu:40-153) with the semantics of the
// CPU path _fps_iterative_fallback (geoembodied/csrc/__init__.py:600-654): start at the first
// point of the cloud, each step take the LOWEST index attaining max(min squared distance).
//
// Register kernel (clouds of up to 16384 points): one 256-thread workgroup per cloud, thread t
// owns local points t, t+256, t+512, ... (PTS of them) with x, y, z and the running min
// distance in VGPRs, so an iteration touches no memory except the centroid lookup (an LDS
// table for clouds of up to 8192 points, L2 otherwise).  The per-iteration argmax is
//   thread: strict '>' over its slots in index order (lowest index on ties);
//   wave:   DPP row max of the distance bits (non-negative floats order like their bits),
//           readlane across the 4 rows, then the same for the lowest index among the lanes
//           holding that max;
//   block:  one LDS slot per wave, double-buffered by iteration parity so that a single
//           barrier per iteration suffices.
// Streaming kernel (larger clouds): same reduction, positions read from HBM/L2 each
// iteration and the running min distance kept in the workspace.
#include "scan.hpp"

namespace geo {
namespace {

constexpr int kFpsThreads = 256;
constexpr int kFpsWaves = kFpsThreads / kWave;
constexpr int kFpsLdsPoints = 8192;  // centroid table: 8192 * 16 B = 128 KB of LDS
constexpr int kFpsStreamThreads = 1024;
constexpr int kFpsStreamWaves = kFpsStreamThreads / kWave;

struct alignas(8) FpsSlot {
  uint32_t dist_bits;
  uint32_t idx;
};

// prepare: clamp k to [0, n], exclusive offsets, total, max cloud, ptr validation.
__global__ __launch_bounds__(kScanThreads) void fps_prepare_kernel(
    const int64_t* __restrict__ ptr, const int64_t* __restrict__ kpb, int64_t B, int64_t N_total,
    int64_t* __restrict__ out_ptr, int64_t* __restrict__ info) {
  __shared__ int64_t lds[kScanThreads / kWave];
  __shared__ unsigned long long s_max, s_bad;
  constexpr unsigned long long kNone = ~0ull;
  if (threadIdx.x == 0) {
    s_max = 0;
    s_bad = (ptr[0] >= 0 && ptr[0] <= N_total) ? kNone : 1ull;  // 1-based entry index
  }
  __syncthreads();
  int64_t carry = 0;
  for (int64_t base = 0; base < B; base += kScanThreads) {
    const int64_t b = base + threadIdx.x;
    int64_t k = 0;
    if (b < B) {
      const int64_t p0 = ptr[b], p1 = ptr[b + 1];
      const int64_t n = p1 - p0;
      if (n < 0 || p1 > N_total) atomicMin(&s_bad, static_cast<unsigned long long>(b + 2));
      const int64_t nn = n > 0 ? n : 0;
      k = kpb[b];
      k = k < 0 ? 0 : (k > nn ? nn : k);
      atomicMax(&s_max, static_cast<unsigned long long>(nn));
    }
    int64_t total;
    const int64_t off = block_exclusive_scan<int64_t>(k, lds, total);
    if (b < B) out_ptr[b] = carry + off;
    carry += total;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    out_ptr[B] = carry;
    info[0] = carry;
    info[1] = static_cast<int64_t>(s_max);
    info[2] = s_bad == kNone ? 0 : static_cast<int64_t>(s_bad);
  }
}

// Wave-level argmax of (dist_bits, idx): max dist, lowest idx on ties.  Uniform result.
__device__ __forceinline__ void wave_argmax(uint32_t bits, uint32_t idx, uint32_t& wbits,
                                            uint32_t& widx) {
  wbits = wave_max_u32(bits);
  widx = wave_min_u32(bits == wbits ? idx : 0xffffffffu);
}

template <int PTS, bool LDS_POS>
__global__ __launch_bounds__(kFpsThreads) void fps_register_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ ptr,
    const int64_t* __restrict__ out_ptr, int64_t* __restrict__ out_idx) {
  __shared__ FpsSlot slots[2][kFpsWaves];
  extern __shared__ float4 table[];  // LDS_POS: local positions, n entries

  const int b = blockIdx.x;
  const int64_t start = ptr[b];
  const int n = static_cast<int>(ptr[b + 1] - start);
  const int64_t o0 = out_ptr[b];
  const int k = static_cast<int>(out_ptr[b + 1] - o0);
  const int t = threadIdx.x;
  const int w = t / kWave;
  if (k <= 0 || n <= 0) return;
  if (k >= n) {  // every point, in index order
    for (int i = t; i < n; i += kFpsThreads) out_idx[o0 + i] = start + i;
    return;
  }
  const float* P = pos + start * 3;

  float px[PTS], py[PTS], pz[PTS], md[PTS];
#pragma unroll
  for (int s = 0; s < PTS; ++s) {
    const int l = t + s * kFpsThreads;
    if (l < n) {
      px[s] = P[3 * l];
      py[s] = P[3 * l + 1];
      pz[s] = P[3 * l + 2];
      md[s] = __builtin_inff();
      if constexpr (LDS_POS) table[l] = make_float4(px[s], py[s], pz[s], 0.f);
    } else {
      px[s] = py[s] = pz[s] = 0.f;
      md[s] = 0.f;  // never wins: its index is above every valid one
    }
  }
  float cx = P[0], cy = P[1], cz = P[2];
  if (t == 0) out_idx[o0] = start;
  if constexpr (LDS_POS) __syncthreads();

  for (int it = 1; it < k; ++it) {
    uint32_t bbits = 0, bidx = 0xffffffffu;
#pragma unroll
    for (int s = 0; s < PTS; ++s) {
      const int l = t + s * kFpsThreads;
      if (l < n) {
        const float d = sqdist(px[s], py[s], pz[s], cx, cy, cz);
        md[s] = fminf(md[s], d);
      }
      const uint32_t mb = __float_as_uint(md[s]);
      if (mb > bbits || bidx == 0xffffffffu) {
        bbits = mb;
        bidx = static_cast<uint32_t>(l);
      }
    }
    uint32_t wbits, widx;
    wave_argmax(bbits, bidx, wbits, widx);
    FpsSlot* sl = slots[it & 1];
    if (lane_id() == 0) sl[w] = FpsSlot{wbits, widx};
    __syncthreads();
    uint32_t gbits = sl[0].dist_bits, gidx = sl[0].idx;
#pragma unroll
    for (int ww = 1; ww < kFpsWaves; ++ww) {
      const FpsSlot o = sl[ww];
      if (o.dist_bits > gbits || (o.dist_bits == gbits && o.idx < gidx)) {
        gbits = o.dist_bits;
        gidx = o.idx;
      }
    }
    gidx = __builtin_amdgcn_readfirstlane(gidx);
    if constexpr (LDS_POS) {
      const float4 c = table[gidx];
      cx = c.x; cy = c.y; cz = c.z;
    } else {
      cx = P[3 * gidx]; cy = P[3 * gidx + 1]; cz = P[3 * gidx + 2];
    }
    if (t == 0) out_idx[o0 + it] = start + gidx;
  }
}

// Streaming kernel for clouds larger than the register kernel holds.
__global__ __launch_bounds__(kFpsStreamThreads) void fps_stream_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ ptr,
    const int64_t* __restrict__ out_ptr, int64_t* __restrict__ out_idx, float* __restrict__ mind) {
  __shared__ FpsSlot slots[2][kFpsStreamWaves];
  const int b = blockIdx.x;
  const int64_t start = ptr[b];
  const int n = static_cast<int>(ptr[b + 1] - start);
  const int64_t o0 = out_ptr[b];
  const int k = static_cast<int>(out_ptr[b + 1] - o0);
  const int t = threadIdx.x;
  const int w = t / kWave;
  if (k <= 0 || n <= 0) return;
  if (k >= n) {
    for (int i = t; i < n; i += kFpsStreamThreads) out_idx[o0 + i] = start + i;
    return;
  }
  const float* P = pos + start * 3;
  float* M = mind + start;
  for (int i = t; i < n; i += kFpsStreamThreads) M[i] = __builtin_inff();
  float cx = P[0], cy = P[1], cz = P[2];
  if (t == 0) out_idx[o0] = start;
  __syncthreads();
  for (int it = 1; it < k; ++it) {
    uint32_t bbits = 0, bidx = 0xffffffffu;
    for (int i = t; i < n; i += kFpsStreamThreads) {
      const float d = sqdist(P[3 * i], P[3 * i + 1], P[3 * i + 2], cx, cy, cz);
      const float m = fminf(M[i], d);
      M[i] = m;
      const uint32_t mb = __float_as_uint(m);
      if (mb > bbits || bidx == 0xffffffffu) {
        bbits = mb;
        bidx = static_cast<uint32_t>(i);
      }
    }
    uint32_t wbits, widx;
    wave_argmax(bbits, bidx, wbits, widx);
    FpsSlot* sl = slots[it & 1];
    if (lane_id() == 0) sl[w] = FpsSlot{wbits, widx};
    __syncthreads();
    uint32_t gbits = sl[0].dist_bits, gidx = sl[0].idx;
    for (int ww = 1; ww < kFpsStreamWaves; ++ww) {
      const FpsSlot o = sl[ww];
      if (o.dist_bits > gbits || (o.dist_bits == gbits && o.idx < gidx)) {
        gbits = o.dist_bits;
        gidx = o.idx;
      }
    }
    gidx = __builtin_amdgcn_readfirstlane(gidx);
    cx = P[3 * gidx]; cy = P[3 * gidx + 1]; cz = P[3 * gidx + 2];
    if (t == 0) out_idx[o0 + it] = start + gidx;
  }
}

template <int PTS>
int launch_register(const float* pos, const int64_t* ptr, const int64_t* out_ptr, int64_t B,
                    int64_t max_cloud, int64_t* out, hipStream_t st) {
  if (max_cloud <= kFpsLdsPoints) {
    const size_t lds = static_cast<size_t>(max_cloud > 0 ? max_cloud : 1) * sizeof(float4);
    GEO_HIP_CHECK(hipFuncSetAttribute(
        reinterpret_cast<const void*>(&fps_register_kernel<PTS, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kFpsLdsPoints * sizeof(float4))));
    hipLaunchKernelGGL((fps_register_kernel<PTS, true>), dim3(B), dim3(kFpsThreads), lds, st,
                       pos, ptr, out_ptr, out);
  } else {
    hipLaunchKernelGGL((fps_register_kernel<PTS, false>), dim3(B), dim3(kFpsThreads), 0, st, pos,
                       ptr, out_ptr, out);
  }
  GEO_LAUNCH_CHECK("fps_register_kernel");
  return GEO_OK;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" int geo_fps_prepare(const int64_t* ptr, const int64_t* k_per_batch, int64_t B,
                               int64_t N_total, int64_t* out_ptr, int64_t* info, void* stream) {
  GEO_REQUIRE(B >= 0 && N_total >= 0, "fps_prepare: negative size");
  GEO_REQUIRE(ptr && out_ptr && info && (B == 0 || k_per_batch), "fps_prepare: null pointer");
  hipLaunchKernelGGL(fps_prepare_kernel, dim3(1), dim3(kScanThreads), 0, as_stream(stream), ptr,
                     k_per_batch, B, N_total, out_ptr, info);
  GEO_LAUNCH_CHECK("fps_prepare_kernel");
  return GEO_OK;
}

extern "C" size_t geo_fps_workspace_bytes(int64_t B, int64_t N_total, int64_t max_cloud) {
  (void)B;
  if (max_cloud > 64 * kFpsThreads) return static_cast<size_t>(N_total > 0 ? N_total : 1) * 4;
  return 0;
}

extern "C" int geo_fps(const float* pos, int64_t N_total, const int64_t* ptr,
                       const int64_t* out_ptr, int64_t B, int64_t max_cloud, int64_t* out_idx,
                       void* workspace, size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(B >= 0 && N_total >= 0 && max_cloud >= 0, "fps: negative size");
  GEO_REQUIRE(max_cloud <= N_total, "fps: max_cloud %lld > N_total %lld", (long long)max_cloud,
              (long long)N_total);
  GEO_REQUIRE(N_total < 0x7fffffffLL, "fps: N_total exceeds int32 indexing");
  if (B == 0 || max_cloud == 0) return GEO_OK;
  GEO_REQUIRE(pos && ptr && out_ptr && out_idx, "fps: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t need = static_cast<int64_t>(geo_fps_workspace_bytes(B, N_total, max_cloud));
  if (need > 0 && (workspace == nullptr || workspace_bytes < static_cast<size_t>(need)))
    return set_error(GEO_ERR_WORKSPACE, "fps: workspace %zu bytes, need %lld", workspace_bytes,
                     (long long)need);
  const int64_t per = ceil_div(max_cloud, kFpsThreads);
  if (per <= 1) return launch_register<1>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 2) return launch_register<2>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 4) return launch_register<4>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 8) return launch_register<8>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 16) return launch_register<16>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 32) return launch_register<32>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 64) return launch_register<64>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  hipLaunchKernelGGL(fps_stream_kernel, dim3(B), dim3(kFpsStreamThreads), 0, st, pos, ptr,
                     out_ptr, out_idx, static_cast<float*>(workspace));
  GEO_LAUNCH_CHECK("fps_stream_kernel");
  return GEO_OK;
}
