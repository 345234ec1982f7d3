// edge_geometry.hip — the per-edge epilogue of a spatial graph and real spherical harmonics.
//
// Replaces compute_edge_vectors (geoembodied/functional/radius_graph.py:336-358: gather, sub,
// norm, clamp, divide) and the spherical harmonics kernel (geoembodied/kernels/
// triton_sph_harm.py:61-198) that SpatialGraph.build runs after the radius graph
// (geoembodied/nn/modules/spatial_graph.py:126-153), with one pass per edge:
//
//   diff = x[col] - x[row],  dist = max(|diff|, 1e-8),  dir = diff / dist,  Y = Y_lm(dir)
//
// Y holds the real spherical harmonics up to l = max_l <= 2, orthonormal on the sphere, in the
// order Y_0^0 | Y_1^{-1,0,1} | Y_2^{-2..2} with
//   Y_0^0 = 1/(2 sqrt(pi)),  Y_1 = sqrt(3/(4 pi)) (y, z, x),
//   Y_2 = sqrt(15/(4 pi)) (xy, yz) , sqrt(5/(16 pi)) (3 z^2 - 1), sqrt(15/(4 pi)) xz,
//         sqrt(15/(16 pi)) (x^2 - y^2),
// evaluated left to right as written (c * x * y = (c x) y).  The backward turns upstream
// gradients of (dir, dist, Y) into the gradient of diff (the chain rule through the
// normalisation: (g_dir - dir <dir, g_dir>) / dist + dir g_dist, or g_dir / 1e-8 where the clamp
// is active); the host scatters it to the two endpoints with segment sums.
#include <cmath>

#include "scan.hpp"

namespace geo {
namespace {

constexpr int kEgThreads = 256;

// Normalisation constants of the real spherical harmonics (from their definitions).
constexpr double kPi = 3.14159265358979323846264338327950288;

struct ShConst {
  float c0, c1, c2_0, c2_1, c2_2;
};

ShConst sh_constants() {
  ShConst c;
  c.c0 = static_cast<float>(std::sqrt(1.0 / (4.0 * kPi)));
  c.c1 = static_cast<float>(std::sqrt(3.0 / (4.0 * kPi)));
  c.c2_0 = static_cast<float>(std::sqrt(5.0 / (16.0 * kPi)));
  c.c2_1 = static_cast<float>(std::sqrt(15.0 / (4.0 * kPi)));
  c.c2_2 = static_cast<float>(std::sqrt(15.0 / (16.0 * kPi)));
  return c;
}

__device__ __forceinline__ void sh_eval(const ShConst& c, float x, float y, float z, int max_l,
                                        float* Y) {
#pragma clang fp contract(off)
  Y[0] = c.c0;
  if (max_l >= 1) {
    Y[1] = c.c1 * y;
    Y[2] = c.c1 * z;
    Y[3] = c.c1 * x;
  }
  if (max_l >= 2) {
    Y[4] = c.c2_1 * x * y;
    Y[5] = c.c2_1 * y * z;
    Y[6] = c.c2_0 * (3.0f * z * z - 1.0f);
    Y[7] = c.c2_1 * x * z;
    Y[8] = c.c2_2 * (x * x - y * y);
  }
}

// d(sum_k g_k Y_k) / d(x, y, z)
__device__ __forceinline__ void sh_grad(const ShConst& c, float x, float y, float z, int max_l,
                                        const float* g, float& gx, float& gy, float& gz) {
#pragma clang fp contract(off)
  gx = 0.f; gy = 0.f; gz = 0.f;
  if (max_l >= 1) {
    gx = c.c1 * g[3];
    gy = c.c1 * g[1];
    gz = c.c1 * g[2];
  }
  if (max_l >= 2) {
    gx = gx + c.c2_1 * y * g[4];
    gy = gy + c.c2_1 * x * g[4];
    gy = gy + c.c2_1 * z * g[5];
    gz = gz + c.c2_1 * y * g[5];
    gz = gz + c.c2_0 * 6.0f * z * g[6];
    gx = gx + c.c2_1 * z * g[7];
    gz = gz + c.c2_1 * x * g[7];
    gx = gx + c.c2_2 * 2.0f * x * g[8];
    gy = gy - c.c2_2 * 2.0f * y * g[8];
  }
}

// One thread per edge of the tile [e0, e0 + cnt); the tile's direction and Y rows are staged in
// LDS and written back as contiguous runs (a thread's own rows are 12 and 36 bytes apart from
// its neighbours').  The caller synchronises before reusing the LDS.
__device__ __forceinline__ void edge_geom_tile(const float* __restrict__ pos, int64_t N,
                                               const int64_t* __restrict__ row,
                                               const int64_t* __restrict__ col, int64_t e0,
                                               int cnt, int max_l, const ShConst& c,
                                               float* __restrict__ dir, float* __restrict__ dist,
                                               float* __restrict__ Y, float* s_dir, float* s_y) {
#pragma clang fp contract(off)
  const int t = static_cast<int>(threadIdx.x);
  const int64_t e = e0 + t;
  const int nsh = (max_l + 1) * (max_l + 1);
  if (t < cnt) {
    int64_t i = col[e], j = row[e];
    const bool ok = i >= 0 && i < N && j >= 0 && j < N;
    i = ok ? i : 0;
    j = ok ? j : 0;
    const float dx = pos[3 * i] - pos[3 * j];
    const float dy = pos[3 * i + 1] - pos[3 * j + 1];
    const float dz = pos[3 * i + 2] - pos[3 * j + 2];
    const float n = sqrtf((dx * dx + dy * dy) + dz * dz);
    const float d = n < 1e-8f ? 1e-8f : n;
    const float ux = dx / d, uy = dy / d, uz = dz / d;
    s_dir[3 * t] = ux;
    s_dir[3 * t + 1] = uy;
    s_dir[3 * t + 2] = uz;
    dist[e] = d;
    if (Y) {
      float y[9];
      sh_eval(c, ux, uy, uz, max_l, y);
      for (int k = 0; k < nsh; ++k) s_y[nsh * t + k] = y[k];
    }
  }
  __syncthreads();
  for (int q = t; q < 3 * cnt; q += kEgThreads) dir[3 * e0 + q] = s_dir[q];
  if (Y)
    for (int q = t; q < nsh * cnt; q += kEgThreads) Y[nsh * e0 + q] = s_y[q];
}

__global__ __launch_bounds__(kEgThreads) void edge_geom_kernel(
    const float* __restrict__ pos, int64_t N, const int64_t* __restrict__ row,
    const int64_t* __restrict__ col, int64_t E, int max_l, ShConst c, float* __restrict__ dir,
    float* __restrict__ dist, float* __restrict__ Y) {
  __shared__ float s_dir[3 * kEgThreads];
  __shared__ float s_y[9 * kEgThreads];
  const int64_t e0 = xcd_block() * kEgThreads;  // one contiguous edge range per XCD: shared pos rows
  const int cnt = static_cast<int>(E - e0 < kEgThreads ? E - e0 : kEgThreads);
  edge_geom_tile(pos, N, row, col, e0, cnt, max_l, c, dir, dist, Y, s_dir, s_y);
}

// The SpatialGraph epilogue of a radius graph whose edge count the host does not know yet:
// launched right behind the emit pass, it reads E = row_ptr[N] on the device (at most `cap`,
// the size of the bound-sized outputs) and walks the edges and nodes in grid-stride loops.
// Edges: the geometry of edge_geom_kernel, the int32 target and the identity permutation (the
// graph is grouped by target).  Nodes: their CSR range from row_ptr and, for contiguous clouds
// of ppc points, the cloud's average degree (its edge count, row_ptr at its last node minus at
// its first, over ppc; at least 1), the value graph_avg_degree computes.
__global__ __launch_bounds__(kEgThreads) void graph_epilogue_dev(
    const float* __restrict__ pos, int64_t N, const int64_t* __restrict__ row,
    const int64_t* __restrict__ col, const int64_t* __restrict__ row_ptr, int64_t cap, int max_l,
    ShConst c, int64_t ppc, float* __restrict__ dir, float* __restrict__ dist,
    float* __restrict__ Y, int32_t* __restrict__ col32, int32_t* __restrict__ perm,
    int32_t* __restrict__ node_start, int32_t* __restrict__ node_end, float* __restrict__ avg) {
  __shared__ float s_dir[3 * kEgThreads];
  __shared__ float s_y[9 * kEgThreads];
  int64_t E = row_ptr[N];
  E = E < 0 ? 0 : (E > cap ? cap : E);
  for (int64_t e0 = xcd_block() * kEgThreads; e0 < E;
       e0 += static_cast<int64_t>(gridDim.x) * kEgThreads) {
    const int cnt = static_cast<int>(E - e0 < kEgThreads ? E - e0 : kEgThreads);
    edge_geom_tile(pos, N, row, col, e0, cnt, max_l, c, dir, dist, Y, s_dir, s_y);
    const int64_t e = e0 + threadIdx.x;
    if (static_cast<int>(threadIdx.x) < cnt) {
      col32[e] = static_cast<int32_t>(col[e]);
      perm[e] = static_cast<int32_t>(e);
    }
    __syncthreads();  // the next tile reuses the LDS
  }
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEgThreads + threadIdx.x; i < N;
       i += static_cast<int64_t>(gridDim.x) * kEgThreads) {
    node_start[i] = static_cast<int32_t>(row_ptr[i]);
    node_end[i] = static_cast<int32_t>(row_ptr[i + 1]);
    const int64_t b0 = i / ppc * ppc;
    const float s = static_cast<float>(static_cast<unsigned long long>(row_ptr[b0 + ppc] - row_ptr[b0]));
    const float a = s / static_cast<float>(ppc);
    avg[i] = a < 1.f ? 1.f : a;
  }
}

__global__ __launch_bounds__(kEgThreads) void edge_geom_bwd_kernel(
    const float* __restrict__ dir, const float* __restrict__ dist, const float* __restrict__ g_dir,
    const float* __restrict__ g_dist, const float* __restrict__ g_Y, int64_t E, int max_l,
    ShConst c, float* __restrict__ g_diff) {
#pragma clang fp contract(off)
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const float ux = dir[3 * e], uy = dir[3 * e + 1], uz = dir[3 * e + 2];
  float gx = g_dir ? g_dir[3 * e] : 0.f;
  float gy = g_dir ? g_dir[3 * e + 1] : 0.f;
  float gz = g_dir ? g_dir[3 * e + 2] : 0.f;
  if (g_Y) {
    const int nsh = (max_l + 1) * (max_l + 1);
    float g[9];
    for (int k = 0; k < 9; ++k) g[k] = k < nsh ? g_Y[e * nsh + k] : 0.f;
    float sx, sy, sz;
    sh_grad(c, ux, uy, uz, max_l, g, sx, sy, sz);
    gx = gx + sx;
    gy = gy + sy;
    gz = gz + sz;
  }
  const float d = dist[e];
  const float gd = g_dist ? g_dist[e] : 0.f;
  // dist == 1e-8: the clamp was active, dist is a constant and dir = diff / 1e-8
  const bool clamped = d <= 1e-8f;
  float ox, oy, oz;
  if (clamped) {
    ox = gx / d; oy = gy / d; oz = gz / d;
  } else {
    const float dot = (ux * gx + uy * gy) + uz * gz;
    ox = (gx - ux * dot) / d + ux * gd;
    oy = (gy - uy * dot) / d + uy * gd;
    oz = (gz - uz * dot) / d + uz * gd;
  }
  g_diff[3 * e] = ox;
  g_diff[3 * e + 1] = oy;
  g_diff[3 * e + 2] = oz;
}

__global__ __launch_bounds__(kEgThreads) void sph_harm_kernel(const float* __restrict__ xyz,
                                                             int64_t N, int max_l, int normalize,
                                                             ShConst c, float* __restrict__ Y,
                                                             float* __restrict__ unit,
                                                             float* __restrict__ norm) {
#pragma clang fp contract(off)
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  float x = xyz[3 * i], y = xyz[3 * i + 1], z = xyz[3 * i + 2];
  if (normalize) {
    const float n = sqrtf((x * x + y * y) + z * z);
    const float d = n < 1e-8f ? 1e-8f : n;
    x = x / d; y = y / d; z = z / d;
    if (unit) { unit[3 * i] = x; unit[3 * i + 1] = y; unit[3 * i + 2] = z; }
    if (norm) norm[i] = d;
  }
  const int nsh = (max_l + 1) * (max_l + 1);
  float v[9];
  sh_eval(c, x, y, z, max_l, v);
  for (int k = 0; k < nsh; ++k) Y[i * nsh + k] = v[k];
}

__global__ __launch_bounds__(kEgThreads) void sph_harm_bwd_kernel(const float* __restrict__ xyz,
                                                                 const float* __restrict__ gY,
                                                                 int64_t N, int max_l, ShConst c,
                                                                 float* __restrict__ gxyz) {
#pragma clang fp contract(off)
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int nsh = (max_l + 1) * (max_l + 1);
  float g[9];
  for (int k = 0; k < 9; ++k) g[k] = k < nsh ? gY[i * nsh + k] : 0.f;
  float gx, gy, gz;
  sh_grad(c, xyz[3 * i], xyz[3 * i + 1], xyz[3 * i + 2], max_l, g, gx, gy, gz);
  gxyz[3 * i] = gx;
  gxyz[3 * i + 1] = gy;
  gxyz[3 * i + 2] = gz;
}

// Per-node average degree of its cloud: integer degree sums and node counts per cloud (exact,
// order-free), then avg = sum / max(count, 1) in fp32, clamped below at 1.  Each wave sums its
// lanes cloud by cloud (one pass per distinct cloud among its lanes: one or two for clouds stored
// contiguously) and issues one atomic pair per cloud, so the counters of a few clouds are not hit
// once per node.
// Degree sums and point counts per cloud.  Each thread takes kAdPer consecutive points; a wave
// whose points all lie in one cloud sums them with shuffles, and the block adds runs of waves in
// the same cloud with one atomic pair (a block of contiguous clouds: one pair per cloud it
// touches).  Points of a thread that straddles clouds, and waves mixing clouds, add per point /
// per cloud instead.
constexpr int kAdThreads = 1024;
constexpr int kAdPer = 4;

__global__ __launch_bounds__(kAdThreads) void avg_degree_sums(
    const int64_t* __restrict__ row_ptr, int64_t N, const int64_t* __restrict__ batch, int64_t B,
    int64_t ppc, unsigned long long* __restrict__ sums, unsigned long long* __restrict__ cnts) {
  constexpr int W = kAdThreads / kWave;
  __shared__ int64_t s_b[W];
  __shared__ unsigned long long s_s[W], s_c[W];
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kAdThreads + threadIdx.x) * kAdPer;
  int64_t b = -1;
  unsigned long long sv = 0, cv = 0;
  bool mixed = false;
#pragma unroll
  for (int k = 0; k < kAdPer; ++k) {
    const int64_t i = i0 + k;
    if (i < N) {
      const int64_t bk = batch ? batch[i] : (ppc > 0 ? i / ppc : 0);
      if (bk >= 0 && bk < B) {
        mixed = mixed || (b >= 0 && bk != b);
        b = bk;
        sv += static_cast<unsigned long long>(row_ptr[i + 1] - row_ptr[i]);
        cv += 1;
      }
    }
  }
  if (mixed) {  // this thread's points straddle clouds: add them one by one
#pragma unroll
    for (int k = 0; k < kAdPer; ++k) {
      const int64_t i = i0 + k;
      if (i < N) {
        const int64_t bk = batch ? batch[i] : (ppc > 0 ? i / ppc : 0);
        if (bk >= 0 && bk < B) {
          atomicAdd(&sums[bk], static_cast<unsigned long long>(row_ptr[i + 1] - row_ptr[i]));
          atomicAdd(&cnts[bk], 1ull);
        }
      }
    }
    b = -1;
    sv = cv = 0;
  }
  const int w = static_cast<int>(threadIdx.x) / kWave;
  const uint64_t has = __ballot(b >= 0);
  int64_t wb = -1;
  if (has) {
    const int64_t lb = __shfl(b, __builtin_ctzll(has), kWave);
    if (__ballot(b >= 0 && b != lb) == 0) {  // one cloud in the whole wave
      wb = lb;
      sv = wave_sum<unsigned long long>(sv);
      cv = wave_sum<unsigned long long>(cv);
    } else {
      uint64_t pending = has;
      while (pending) {  // wave-uniform loop: every lane takes part in each shuffle
        const int leader = __builtin_ctzll(pending);
        const int64_t cb = __shfl(b, leader, kWave);
        const bool mine = b >= 0 && b == cb;
        const uint64_t m = __ballot(mine);
        const unsigned long long s2 = wave_sum<unsigned long long>(mine ? sv : 0ull);
        const unsigned long long c2 = wave_sum<unsigned long long>(mine ? cv : 0ull);
        if (lane_id() == leader) {
          atomicAdd(&sums[cb], s2);
          atomicAdd(&cnts[cb], c2);
        }
        pending &= ~m;
      }
    }
  }
  if (lane_id() == 0) {
    s_b[w] = wb;
    s_s[w] = sv;
    s_c[w] = cv;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t rb = -1;
    unsigned long long rs = 0, rc = 0;
    for (int q = 0; q < W; ++q) {
      if (s_b[q] != rb) {
        if (rb >= 0) { atomicAdd(&sums[rb], rs); atomicAdd(&cnts[rb], rc); }
        rb = s_b[q];
        rs = rc = 0;
      }
      if (rb >= 0) { rs += s_s[q]; rc += s_c[q]; }
    }
    if (rb >= 0) { atomicAdd(&sums[rb], rs); atomicAdd(&cnts[rb], rc); }
  }
}

__global__ __launch_bounds__(kEgThreads) void avg_degree_write(
    const int64_t* __restrict__ batch, int64_t N, int64_t B, int64_t ppc,
    const unsigned long long* __restrict__ sums, const unsigned long long* __restrict__ cnts,
    float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int64_t b = batch ? batch[i] : (ppc > 0 ? i / ppc : 0);
  float a = 1.f;
  if (b >= 0 && b < B) {
    const float s = static_cast<float>(sums[b]);
    const float n = static_cast<float>(cnts[b] > 0 ? cnts[b] : 1);
    a = s / n;
  }
  out[i] = a < 1.f ? 1.f : a;
}

// CSR arrays of edges that are already grouped by target with offsets row_ptr (the radius
// graph's output): identity permutation, int32 targets, int32 ranges, in one pass.
__global__ void csr_from_row_ptr(const int64_t* __restrict__ row_ptr, int64_t N,
                                 const int64_t* __restrict__ col, int64_t E,
                                 int32_t* __restrict__ col32, int32_t* __restrict__ perm,
                                 int32_t* __restrict__ node_start, int32_t* __restrict__ node_end) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < E || q < N;
       q += stride) {
    if (q < E) {
      perm[q] = static_cast<int32_t>(q);
      col32[q] = static_cast<int32_t>(col[q]);
    }
    if (q < N) {
      node_start[q] = static_cast<int32_t>(row_ptr[q]);
      node_end[q] = static_cast<int32_t>(row_ptr[q + 1]);
    }
  }
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" int geo_edge_geometry(const float* pos, int64_t N, const int64_t* row,
                                 const int64_t* col, int64_t E, int max_l, float* direction,
                                 float* dist, float* Y, void* stream) {
  GEO_REQUIRE(N >= 0 && E >= 0, "edge_geometry: negative size");
  GEO_REQUIRE(max_l >= 0 && max_l <= 2, "edge_geometry: max_l must be 0, 1 or 2 (got %d)", max_l);
  if (E == 0) return GEO_OK;
  GEO_REQUIRE(N > 0 && pos && row && col && direction && dist, "edge_geometry: null pointer");
  hipLaunchKernelGGL(edge_geom_kernel, dim3(static_cast<unsigned>(ceil_div(E, kEgThreads))),
                     dim3(kEgThreads), 0, as_stream(stream), pos, N, row, col, E, max_l,
                     sh_constants(), direction, dist, Y);
  GEO_LAUNCH_CHECK("edge_geom_kernel");
  return GEO_OK;
}

extern "C" int geo_edge_geometry_bwd(const float* direction, const float* dist,
                                     const float* grad_direction, const float* grad_dist,
                                     const float* grad_Y, int64_t E, int max_l, float* grad_diff,
                                     void* stream) {
  GEO_REQUIRE(E >= 0, "edge_geometry_bwd: negative size");
  GEO_REQUIRE(max_l >= 0 && max_l <= 2, "edge_geometry_bwd: max_l must be 0, 1 or 2");
  if (E == 0) return GEO_OK;
  GEO_REQUIRE(direction && dist && grad_diff, "edge_geometry_bwd: null pointer");
  hipLaunchKernelGGL(edge_geom_bwd_kernel, dim3(static_cast<unsigned>(ceil_div(E, kEgThreads))),
                     dim3(kEgThreads), 0, as_stream(stream), direction, dist, grad_direction,
                     grad_dist, grad_Y, E, max_l, sh_constants(), grad_diff);
  GEO_LAUNCH_CHECK("edge_geom_bwd_kernel");
  return GEO_OK;
}

extern "C" int geo_spherical_harmonics(const float* xyz, int64_t N, int max_l, int normalize,
                                       float* Y, float* unit, float* norm, void* stream) {
  GEO_REQUIRE(N >= 0, "spherical_harmonics: negative size");
  GEO_REQUIRE(max_l >= 0 && max_l <= 2, "spherical_harmonics: max_l must be 0, 1 or 2");
  if (N == 0) return GEO_OK;
  GEO_REQUIRE(xyz && Y, "spherical_harmonics: null pointer");
  hipLaunchKernelGGL(sph_harm_kernel, dim3(static_cast<unsigned>(ceil_div(N, kEgThreads))),
                     dim3(kEgThreads), 0, as_stream(stream), xyz, N, max_l, normalize,
                     sh_constants(), Y, unit, norm);
  GEO_LAUNCH_CHECK("sph_harm_kernel");
  return GEO_OK;
}

extern "C" int geo_spherical_harmonics_bwd(const float* xyz, const float* grad_Y, int64_t N,
                                           int max_l, float* grad_xyz, void* stream) {
  GEO_REQUIRE(N >= 0, "spherical_harmonics_bwd: negative size");
  GEO_REQUIRE(max_l >= 0 && max_l <= 2, "spherical_harmonics_bwd: max_l must be 0, 1 or 2");
  if (N == 0) return GEO_OK;
  GEO_REQUIRE(xyz && grad_Y && grad_xyz, "spherical_harmonics_bwd: null pointer");
  hipLaunchKernelGGL(sph_harm_bwd_kernel, dim3(static_cast<unsigned>(ceil_div(N, kEgThreads))),
                     dim3(kEgThreads), 0, as_stream(stream), xyz, grad_Y, N, max_l,
                     sh_constants(), grad_xyz);
  GEO_LAUNCH_CHECK("sph_harm_bwd_kernel");
  return GEO_OK;
}

extern "C" size_t geo_graph_avg_degree_workspace_bytes(int64_t B) {
  if (B < 0) return 0;
  return static_cast<size_t>(2 * (B > 0 ? B : 1)) * sizeof(unsigned long long);
}

extern "C" int geo_graph_avg_degree(const int64_t* row_ptr, int64_t N, const int64_t* batch,
                                    int64_t B, int64_t points_per_cloud, float* out,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(N >= 0 && B >= 1, "graph_avg_degree: need N >= 0 and B >= 1");
  GEO_REQUIRE(batch != nullptr || points_per_cloud * B == N,
              "graph_avg_degree: without batch, B*points_per_cloud must equal N");
  if (N == 0) return GEO_OK;
  GEO_REQUIRE(row_ptr && out, "graph_avg_degree: null pointer");
  const size_t need = geo_graph_avg_degree_workspace_bytes(B);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(GEO_ERR_WORKSPACE, "graph_avg_degree: workspace %zu bytes, need %zu",
                     workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  auto* sums = static_cast<unsigned long long*>(workspace);
  int rc = device_fill<unsigned long long>(sums, 2 * B, 0ull, st);
  if (rc) return rc;
  const unsigned grid = static_cast<unsigned>(ceil_div(N, kEgThreads));
  hipLaunchKernelGGL(avg_degree_sums, dim3(static_cast<unsigned>(ceil_div(N, kAdThreads * kAdPer))),
                     dim3(kAdThreads), 0, st, row_ptr, N, batch, B, points_per_cloud, sums,
                     sums + B);
  GEO_LAUNCH_CHECK("avg_degree_sums");
  hipLaunchKernelGGL(avg_degree_write, dim3(grid), dim3(kEgThreads), 0, st, batch, N, B,
                     points_per_cloud, sums, sums + B, out);
  GEO_LAUNCH_CHECK("avg_degree_write");
  return GEO_OK;
}

extern "C" int geo_csr_from_row_ptr(const int64_t* row_ptr, int64_t N, const int64_t* col,
                                    int64_t E, int32_t* col32, int32_t* perm, int32_t* node_start,
                                    int32_t* node_end, void* stream) {
  GEO_REQUIRE(N >= 0 && E >= 0, "csr_from_row_ptr: negative size");
  GEO_REQUIRE(E < 0x7fffffffLL && N < 0x7fffffffLL, "csr_from_row_ptr: sizes exceed int32");
  if (N == 0 && E == 0) return GEO_OK;
  GEO_REQUIRE(row_ptr && node_start && node_end && (E == 0 || (col && col32 && perm)),
              "csr_from_row_ptr: null pointer");
  const int64_t span = E > N ? E : N;
  int64_t blocks = ceil_div(span, 256);
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(csr_from_row_ptr, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), row_ptr, N, col, E, col32, perm, node_start, node_end);
  GEO_LAUNCH_CHECK("csr_from_row_ptr");
  return GEO_OK;
}

extern "C" int geo_spatial_graph_epilogue_dev(const float* pos, int64_t N, const int64_t* row,
                                              const int64_t* col, const int64_t* row_ptr,
                                              int64_t cap, int max_l, int64_t points_per_cloud,
                                              float* direction, float* dist, float* Y,
                                              int32_t* col_sorted, int32_t* perm,
                                              int32_t* node_start, int32_t* node_end,
                                              float* avg_degree, void* stream) {
  GEO_REQUIRE(N >= 1 && cap >= 0, "spatial_graph_epilogue_dev: need N >= 1 and cap >= 0");
  GEO_REQUIRE(N < 0x7fffffffLL && cap < 0x7fffffffLL, "spatial_graph_epilogue_dev: sizes exceed int32");
  GEO_REQUIRE(max_l >= 0 && max_l <= 2, "spatial_graph_epilogue_dev: max_l must be 0, 1 or 2");
  GEO_REQUIRE(points_per_cloud >= 1 && N % points_per_cloud == 0,
              "spatial_graph_epilogue_dev: N=%lld is not a whole number of clouds of %lld points",
              (long long)N, (long long)points_per_cloud);
  GEO_REQUIRE(pos && row && col && row_ptr && direction && dist && col_sorted && perm &&
                  node_start && node_end && avg_degree,
              "spatial_graph_epilogue_dev: null pointer");
  const int64_t span = cap > N ? cap : N;
  int64_t blocks = ceil_div(span, kEgThreads);
  if (blocks > 2048) blocks = 2048;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(graph_epilogue_dev, dim3(static_cast<unsigned>(blocks)), dim3(kEgThreads), 0,
                     as_stream(stream), pos, N, row, col, row_ptr, cap, max_l, sh_constants(),
                     points_per_cloud, direction, dist, Y, col_sorted, perm, node_start, node_end,
                     avg_degree);
  GEO_LAUNCH_CHECK("graph_epilogue_dev");
  return GEO_OK;
}

extern "C" int geo_spatial_graph_epilogue(const float* pos, int64_t N, const int64_t* row,
                                          const int64_t* col, const int64_t* row_ptr, int64_t E,
                                          int max_l, const int64_t* batch, int64_t B,
                                          int64_t points_per_cloud, float* direction,
                                          float* dist, float* Y, int32_t* col_sorted,
                                          int32_t* perm, int32_t* node_start, int32_t* node_end,
                                          float* avg_degree, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  int rc = geo_csr_from_row_ptr(row_ptr, N, col, E, col_sorted, perm, node_start, node_end, stream);
  if (rc) return rc;
  rc = geo_edge_geometry(pos, N, row, col, E, max_l, direction, dist, Y, stream);
  if (rc) return rc;
  return geo_graph_avg_degree(row_ptr, N, batch, B, points_per_cloud, avg_degree, workspace,
                              workspace_bytes, stream);
}
