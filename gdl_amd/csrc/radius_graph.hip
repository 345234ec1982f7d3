// radius_graph.hip — batched fixed-radius neighbour graph on gfx950.
//
// Replaces compute_cell_indices_kernel / CUB sort / compute_cell_offsets_kernel /
// find_neighbors_kernel and the host loop over clouds (geoembodied/csrc/radius_graph_kernel.cu:
// 91-467) with one device pipeline for all clouds and exact semantics (edge j -> i iff same
// cloud, both valid, loop or i != j, d < r2; per target the K smallest (d, j)).
//
// geo_radius_count:
//   rg_front    clouds that are contiguous chunks of at most 4096 points: one workgroup per cloud
//               does all that rg_init .. rg_scatter do below, in LDS, then rg_count and the scan
//   rg_init     zero counters, reset bounding boxes
//   rg_bbox     per-cloud point count and bounding box (wave-reduced atomics; one cloud without
//               batch vector or mask: rg_bbox_one, at most 64 workgroups)
//   rg_setup    per cloud: cell edge h >= r*(1+1/32), grid dims (capped at 4*n+64 cells, 8*n+64
//               for scene-scale clouds, and 16384 per axis so that the 3x3x3 stencil stays
//               exact), cell base offsets
//   rg_cell     cell id per point, rank inside the cell (atomic counter, one per run of equal
//               cells in a wave)
//   scan        cell offsets (single pass, decoupled look-back)
//   rg_scatter  points in cell order as float4 (x, y, z, index bits)
//   rg_count    kRgGroup lanes per point in cell order (neighbouring groups share cells): count
//               of in-radius sources over the 9 z-contiguous runs of the 27-cell stencil, and
//               the first K accepted sources in a per-target list
//   scan        row_ptr = exclusive scan of min(count, K) over target index
// geo_radius_emit:
//   rg_compact  kRgGroup lanes per target: the list sorted by source index into the CSR row;
//               targets with more than K sources (or long lists) are done by the whole wave:
//               the K smallest (d, j) by a radix select on the distance bits of the in-radius
//               candidates staged in LDS (a binary search over the stencil beyond kRgSelCap)
//   rg_emit     (lists too large for the workspace) re-scans the stencil per target instead
// Traversal order inside a cell is not deterministic (atomic ranks) and does not matter: the
// accepted set is defined by a total order and the output is sorted.
#include "scan.hpp"

namespace geo {
namespace {

constexpr int kRgThreads = 256;
constexpr int kRgEmitThreads = 64;
constexpr int kRgMaxAxis = 16384;
constexpr int kRgLdsK = 256;

struct Grid {
  float ox, oy, oz, inv_h;
  int dx, dy, dz, base;
};

struct RgWs {
  int32_t* cloud_n;
  uint32_t* bbox;  // [B][6]: min x,y,z keys then max x,y,z keys
  Grid* grid;
  int32_t* pt_cell;
  int32_t* pt_rank;
  int32_t* cell_cnt;
  int32_t* cell_start;
  uint64_t* cell_scan;  // look-back status of the cell-offset scan (zeroed by rg_init)
  float4* spos;
  int32_t* cnt;
  int32_t* deg;
  uint64_t* deg_scan;   // look-back status of the row-pointer scan (zeroed by rg_init)
  int32_t* list;  // [N][K] accepted sources per target (unsorted), or null when too large
  int32_t* layout_bad;  // [B] per cloud: points of the chunk whose batch entry is another cloud
  int64_t cells_max;
  int cell_factor;  // grid cells allowed per point of a cloud (cap cell_factor * n + 64)
  size_t bytes;
  const double* r_dev = nullptr;  // radius on the device (geo_radius_*_dev), else null
};

// Threshold and cell edge: the host values, or those of the device radius r (fl32(r * r) with the
// product in float64, as the host computes it; r <= 0 or NaN gives no edges).
__device__ __forceinline__ float rg_r2(const RgWs& w, float r2) {
  if (!w.r_dev) return r2;
  const double r = *w.r_dev;
  return r > 0.0 ? static_cast<float>(r * r) : 0.0f;
}
__device__ __forceinline__ float rg_rcell(const RgWs& w, float r_cell) {
  if (!w.r_dev) return r_cell;
  const double r = *w.r_dev;
  return r > 0.0 ? static_cast<float>(r) : 1.0f;
}

// Grid cells allowed per point: 4, or 8 for clouds of 16,384 points or more on average -- a
// scene-scale cloud (the lidar frame: 0.63 m cells at 4 per point against 0.52 m at 8, 865
// against 589 stencil sources per target at r = 0.5 m) pays more in stencil scans than its
// cell scan costs.  The one-workgroup front end keeps 4 (its LDS grid).
int rg_cell_factor(int64_t N, int64_t B) { return B > 0 && N / B >= 16384 ? 8 : 4; }
int64_t cells_cap(int64_t N, int64_t B) { return rg_cell_factor(N, B) * N + 64 * B; }

// The per-target source lists are kept when they fit in 1 GiB of workspace; beyond that the
// emit pass re-scans the candidates instead.
constexpr int64_t kRgListMaxEntries = int64_t(1) << 28;

RgWs carve_rg(void* base, int64_t N, int64_t B, int64_t K) {
  Carver c(base);
  RgWs w;
  const int64_t nn = N > 0 ? N : 1, bb = B > 0 ? B : 1;
  w.cells_max = cells_cap(N, B);
  w.cell_factor = rg_cell_factor(N, B);
  w.cloud_n = c.take<int32_t>(bb);
  w.bbox = c.take<uint32_t>(6 * bb);
  w.grid = c.take<Grid>(bb);
  w.pt_cell = c.take<int32_t>(nn);
  w.pt_rank = c.take<int32_t>(nn);
  w.cell_cnt = c.take<int32_t>(w.cells_max + 1);
  w.cell_start = c.take<int32_t>(w.cells_max + 1);
  w.cell_scan = c.take<uint64_t>(scan_lookback_elems(w.cells_max));
  w.spos = c.take<float4>(nn);
  w.cnt = c.take<int32_t>(nn);
  w.deg = c.take<int32_t>(nn);
  w.deg_scan = c.take<uint64_t>(scan_lookback_elems(N));
  w.layout_bad = c.take<int32_t>(bb);
  const bool lists = K > 0 && N <= kRgListMaxEntries / K;
  w.list = lists ? c.take<int32_t>(N * K) : nullptr;
  if (lists && !base) w.list = reinterpret_cast<int32_t*>(1);  // size query: mark "present"
  w.bytes = c.used;
  return w;
}

__device__ __forceinline__ int cloud_of(int64_t i, const int64_t* __restrict__ batch, int64_t B,
                                        int64_t ppc) {
  if (batch) {
    const int64_t b = batch[i];
    return (b >= 0 && b < B) ? static_cast<int>(b) : -1;
  }
  const int64_t b = ppc > 0 ? i / ppc : 0;
  return b < B ? static_cast<int>(b) : -1;
}

__global__ void rg_init(RgWs w, int64_t N, int64_t B) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < w.cells_max + 1 || i < N || i < 6 * B; i += stride) {
    if (i < w.cells_max + 1) w.cell_cnt[i] = 0;
    if (i < N) { w.cnt[i] = 0; w.deg[i] = 0; }
    if (i < B) w.cloud_n[i] = 0;
    if (i < scan_lookback_elems(w.cells_max)) w.cell_scan[i] = 0;
    if (i < scan_lookback_elems(N)) w.deg_scan[i] = 0;
    if (i < 6 * B) w.bbox[i] = (i % 6) < 3 ? 0xffffffffu : 0u;
  }
}

// Grid of one cloud of n valid points with bounding box [mn, mx]: cell edge h >= r*(1+1/32),
// grown until the cell count is at most factor * n + 64 and no axis exceeds kRgMaxAxis cells
// (one cell for the whole cloud if that fails).  Writes the cell count; g.base is left 0.
__device__ Grid rg_grid(const float (&mn)[3], const float (&mx)[3], int64_t n, float r_cell,
                        int64_t& cells, int factor) {
  Grid g{0.f, 0.f, 0.f, 0.f, 0, 0, 0, 0};
  const double cap = static_cast<double>(factor) * n + 64.0;
  double h = static_cast<double>(r_cell) * (1.0 + 1.0 / 32.0);
  double ext[3];
  for (int a = 0; a < 3; ++a) {
    const double e = static_cast<double>(mx[a]) - static_cast<double>(mn[a]);
    ext[a] = (e >= 0.0 && e < 1e30) ? e : 0.0;  // non-finite input: one slab on that axis
  }
  int64_t d[3] = {1, 1, 1};
  bool ok = false;
  for (int iter = 0; iter < 64 && !ok; ++iter) {
    double prod = 1.0, worst_axis = 0.0;
    for (int a = 0; a < 3; ++a) {
      const double q = floor(ext[a] / h) + 1.0;
      d[a] = q < static_cast<double>(kRgMaxAxis) * 4 ? static_cast<int64_t>(q) : kRgMaxAxis * 4;
      prod *= static_cast<double>(d[a]);
      worst_axis = fmax(worst_axis, static_cast<double>(d[a]) / kRgMaxAxis);
    }
    ok = prod <= cap && worst_axis <= 1.0;
    if (!ok) h *= fmax(fmax(cbrt(prod / cap), worst_axis), 1.0) * 1.01;
  }
  g.ox = mn[0]; g.oy = mn[1]; g.oz = mn[2];
  g.inv_h = static_cast<float>(1.0 / h);
  if (!ok) {  // one cell holds the whole cloud
    d[0] = d[1] = d[2] = 1;
    g.inv_h = 0.f;
  }
  g.dx = static_cast<int>(d[0]); g.dy = static_cast<int>(d[1]); g.dz = static_cast<int>(d[2]);
  cells = d[0] * d[1] * d[2];
  return g;
}

// Single workgroup: grid parameters and cell bases for every cloud.
__global__ __launch_bounds__(kScanThreads) void rg_setup(RgWs w, int64_t B, float r_cell) {
  __shared__ int64_t lds[kScanThreads / kWave];
  r_cell = rg_rcell(w, r_cell);
  int64_t carry = 0;
  for (int64_t base = 0; base < B; base += kScanThreads) {
    const int64_t b = base + threadIdx.x;
    int64_t cells = 0;
    Grid g{0.f, 0.f, 0.f, 0.f, 0, 0, 0, 0};
    if (b < B && w.cloud_n[b] > 0) {
      const uint32_t* bb = w.bbox + 6 * b;
      const float mn[3] = {float_from_order_key(bb[0]), float_from_order_key(bb[1]),
                           float_from_order_key(bb[2])};
      const float mx[3] = {float_from_order_key(bb[3]), float_from_order_key(bb[4]),
                           float_from_order_key(bb[5])};
      g = rg_grid(mn, mx, w.cloud_n[b], r_cell, cells, w.cell_factor);
    }
    int64_t total;
    const int64_t off = block_exclusive_scan<int64_t>(cells, lds, total);
    if (b < B) {
      g.base = static_cast<int>(carry + off);
      w.grid[b] = g;
    }
    carry += total;
  }
}

__global__ __launch_bounds__(kRgThreads) void rg_bbox(RgWs w, const float* __restrict__ x, int64_t N,
                                                      const int64_t* __restrict__ batch, int64_t B,
                                                      int64_t ppc, const uint8_t* __restrict__ mask) {
  // Points of one workgroup usually belong to one cloud: reduce in the workgroup first and
  // issue 7 atomics per workgroup; mixed workgroups fall back to per-wave / per-lane atomics.
  constexpr int W = kRgThreads / kWave;
  __shared__ int s_cloud[W];
  __shared__ uint32_t s_red[7][W];
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int wv = threadIdx.x / kWave;
  int b = -1;
  float px = 0.f, py = 0.f, pz = 0.f;
  if (i < N) {
    b = cloud_of(i, batch, B, ppc);
    if (mask && !mask[i]) b = -1;
    if (b >= 0) { px = x[3 * i]; py = x[3 * i + 1]; pz = x[3 * i + 2]; }
  }
  // wave-uniform cloud (or -1 for "mixed")
  const int b0 = __builtin_amdgcn_readfirstlane(b);
  const bool uniform = __ballot(b != b0) == 0ull;
  const uint32_t kx = float_order_key(px), ky = float_order_key(py), kz = float_order_key(pz);
  const uint32_t v[7] = {wave_min_u32(kx), wave_min_u32(ky), wave_min_u32(kz), wave_max_u32(kx),
                         wave_max_u32(ky), wave_max_u32(kz), 0u};
  if (lane_id() == 0) {
    s_cloud[wv] = uniform ? b0 : -2;
#pragma unroll
    for (int q = 0; q < 6; ++q) s_red[q][wv] = v[q];
  }
  if (!uniform && b >= 0) {  // mixed wave: per-lane atomics
    atomicAdd(&w.cloud_n[b], 1);
    uint32_t* bb = w.bbox + 6 * b;
    atomicMin(&bb[0], kx); atomicMin(&bb[1], ky); atomicMin(&bb[2], kz);
    atomicMax(&bb[3], kx); atomicMax(&bb[4], ky); atomicMax(&bb[5], kz);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int c0 = s_cloud[0];
    bool same = c0 >= 0;
    for (int q = 1; q < W; ++q) same = same && s_cloud[q] == c0;
    if (same) {  // whole workgroup in one cloud
      uint32_t r[6];
      for (int q = 0; q < 6; ++q) r[q] = s_red[q][0];
      for (int ww = 1; ww < W; ++ww) {
        for (int q = 0; q < 3; ++q) r[q] = min(r[q], s_red[q][ww]);
        for (int q = 3; q < 6; ++q) r[q] = max(r[q], s_red[q][ww]);
      }
      atomicAdd(&w.cloud_n[c0], kRgThreads);
      uint32_t* bb = w.bbox + 6 * c0;
      atomicMin(&bb[0], r[0]); atomicMin(&bb[1], r[1]); atomicMin(&bb[2], r[2]);
      atomicMax(&bb[3], r[3]); atomicMax(&bb[4], r[4]); atomicMax(&bb[5], r[5]);
    } else {
      for (int ww = 0; ww < W; ++ww) {
        const int c = s_cloud[ww];
        if (c < 0) continue;  // mixed (handled per lane) or masked
        atomicAdd(&w.cloud_n[c], kWave);
        uint32_t* bb = w.bbox + 6 * c;
        atomicMin(&bb[0], s_red[0][ww]); atomicMin(&bb[1], s_red[1][ww]); atomicMin(&bb[2], s_red[2][ww]);
        atomicMax(&bb[3], s_red[3][ww]); atomicMax(&bb[4], s_red[4][ww]); atomicMax(&bb[5], s_red[5][ww]);
      }
    }
  }
}

// One cloud of all N points (no batch vector, no mask): a grid-stride loop per thread and one
// reduction per workgroup, so at most kRgBoxBlocks workgroups issue the cloud's atomics (one
// workgroup per 256 points put ~3,600 atomics on the same six words for a 131,072-point frame).
constexpr int kRgBoxBlocks = 64;
__global__ __launch_bounds__(kRgThreads) void rg_bbox_one(RgWs w, const float* __restrict__ x,
                                                          int64_t N) {
  constexpr int W = kRgThreads / kWave;
  __shared__ uint32_t s_red[6][W];
  uint32_t mn[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, mx[3] = {0u, 0u, 0u};
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < N; i += stride) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const uint32_t k = float_order_key(x[3 * i + a]);
      mn[a] = min(mn[a], k);
      mx[a] = max(mx[a], k);
    }
  }
  const int wv = threadIdx.x / kWave;
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    mn[a] = wave_min_u32(mn[a]);
    mx[a] = wave_max_u32(mx[a]);
  }
  if (lane_id() == 0) {
#pragma unroll
    for (int a = 0; a < 3; ++a) { s_red[a][wv] = mn[a]; s_red[3 + a][wv] = mx[a]; }
  }
  __syncthreads();
  if (threadIdx.x < 6) {
    const int q = threadIdx.x;
    uint32_t r = s_red[q][0];
    for (int ww = 1; ww < W; ++ww) r = q < 3 ? min(r, s_red[q][ww]) : max(r, s_red[q][ww]);
    if (q < 3) atomicMin(&w.bbox[q], r); else atomicMax(&w.bbox[q], r);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) w.cloud_n[0] = static_cast<int>(N);
}

__device__ __forceinline__ int cell_coord(float p, float o, float inv_h, int dim) {
#pragma clang fp contract(off)
  const float u = (p - o) * inv_h;
  int c = static_cast<int>(floorf(u));
  return c < 0 ? 0 : (c >= dim ? dim - 1 : c);
}

__global__ __launch_bounds__(kRgThreads) void rg_cell(RgWs w, const float* __restrict__ x, int64_t N,
                                                      const int64_t* __restrict__ batch, int64_t B,
                                                      int64_t ppc, const uint8_t* __restrict__ mask) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  int b = cloud_of(i, batch, B, ppc);
  if (mask && !mask[i]) b = -1;
  if (b < 0) {
    w.pt_cell[i] = -1;
    return;
  }
  const Grid g = w.grid[b];
  const int cx = cell_coord(x[3 * i], g.ox, g.inv_h, g.dx);
  const int cy = cell_coord(x[3 * i + 1], g.oy, g.inv_h, g.dy);
  const int cz = cell_coord(x[3 * i + 2], g.oz, g.inv_h, g.dz);
  const int c = g.base + (cx * g.dy + cy) * g.dz + cz;
  w.pt_cell[i] = c;
  w.pt_rank[i] = cell_rank(&w.cell_cnt[c], c);
}

__global__ __launch_bounds__(kRgThreads) void rg_scatter(RgWs w, const float* __restrict__ x,
                                                         int64_t N) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int c = w.pt_cell[i];
  if (c < 0) return;
  const int p = w.cell_start[c] + w.pt_rank[i];
  w.spos[p] = make_float4(x[3 * i], x[3 * i + 1], x[3 * i + 2], __int_as_float(static_cast<int>(i)));
}

// Clouds that are contiguous chunks of at most kRgFrontMax points (points_per_cloud given, or a
// batch vector verified to be that layout): one workgroup per cloud does what rg_init .. rg_scatter
// do for all clouds -- bounding box, grid, cell counts (LDS atomics, two 16-bit counts per
// word), their scan and the cell-ordered points -- with no global atomics.  Cloud b owns cells
// [b * (4 ppc + 64), ...) and spos slots [b * ppc, (b + 1) * ppc); masked points (and, with a
// batch vector, points whose entry is not b, counted in layout_bad[b]) leave holes at the end
// of the cloud's slots, marked by index -1.
constexpr int kRgFrontThreads = 1024;
constexpr int kRgFrontMax = 4096;
constexpr int kRgFrontPer = kRgFrontMax / kRgFrontThreads;
constexpr int kRgFrontCells = 4 * kRgFrontMax + 64;
constexpr int kRgFrontWords = kRgFrontCells / 2 + 1;
// beyond this many clouds (one 1024-thread workgroup each) the general path is cheaper
constexpr int64_t kRgFrontMaxClouds = 4096;

__device__ __forceinline__ uint32_t half_of(const uint32_t* s, int c) {
  return (s[c >> 1] >> ((c & 1) * 16)) & 0xffffu;
}

__global__ __launch_bounds__(kRgFrontThreads) void rg_front(RgWs w, const float* __restrict__ x,
                                                            int64_t N, const int64_t* __restrict__ batch,
                                                            int64_t B, int64_t ppc,
                                                            const uint8_t* __restrict__ mask,
                                                            float r_cell) {
  constexpr int W = kRgFrontThreads / kWave;
  __shared__ uint32_t s_cnt[kRgFrontWords];
  __shared__ uint32_t s_red[7][W];
  __shared__ Grid s_grid;
  __shared__ int s_cells, s_nv;
  const int b = blockIdx.x;
  const int64_t lo = static_cast<int64_t>(b) * ppc;
  const int tid = threadIdx.x, wv = tid / kWave, lane = lane_id();
  r_cell = rg_rcell(w, r_cell);
  float px[kRgFrontPer], py[kRgFrontPer], pz[kRgFrontPer];
  bool ok[kRgFrontPer];
  bool bad = false;
  uint32_t nv = 0;
  uint32_t kmin[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, kmax[3] = {0u, 0u, 0u};
  // every point's mask, batch entry and position requested at once, at positions clamped into
  // the cloud (ppc >= 1 here), and used for il < ppc only: loads under the per-point conditions
  // had become a chain of branches, one wait per load
  // (a missing mask or batch vector is read from x instead, whose 12 N bytes hold byte i and
  // 8-byte word i for every i < N, and the value is discarded: a load behind a pointer test
  // became a branch whose join waited for it)
  const uint8_t* mp = mask ? mask : reinterpret_cast<const uint8_t*>(x);
  const int64_t* bp = batch ? batch : reinterpret_cast<const int64_t*>(x);
  uint8_t mv[kRgFrontPer];
  int64_t bv[kRgFrontPer];
#pragma unroll
  for (int k = 0; k < kRgFrontPer; ++k) {
    const int il = tid + k * kRgFrontThreads;
    const int64_t i = lo + (il < ppc ? il : ppc - 1);
    mv[k] = mp[i];
    bv[k] = bp[i];
    px[k] = x[3 * i]; py[k] = x[3 * i + 1]; pz[k] = x[3 * i + 2];
  }
#pragma unroll
  for (int k = 0; k < kRgFrontPer; ++k) {
    mv[k] = mask ? mv[k] : static_cast<uint8_t>(1);
    bv[k] = batch ? bv[k] : static_cast<int64_t>(b);
  }
#pragma unroll
  for (int k = 0; k < kRgFrontPer; ++k) {
    const int il = tid + k * kRgFrontThreads;
    bool v = il < ppc && mv[k] != 0;
    if (il < ppc && bv[k] != b) {
      bad = true;
      v = false;
    }
    ok[k] = v;
    px[k] = v ? px[k] : 0.f;
    py[k] = v ? py[k] : 0.f;
    pz[k] = v ? pz[k] : 0.f;
    if (v) {
      const uint32_t kk[3] = {float_order_key(px[k]), float_order_key(py[k]), float_order_key(pz[k])};
#pragma unroll
      for (int a = 0; a < 3; ++a) { kmin[a] = min(kmin[a], kk[a]); kmax[a] = max(kmax[a], kk[a]); }
      ++nv;
    }
  }
  // bounding box, valid count and layout check over the workgroup
  uint32_t r7[7] = {wave_min_u32(kmin[0]), wave_min_u32(kmin[1]), wave_min_u32(kmin[2]),
                    wave_max_u32(kmax[0]), wave_max_u32(kmax[1]), wave_max_u32(kmax[2]), 0u};
  const uint32_t wnv = wave_sum_dpp(nv);
  const bool wbad = __ballot(bad) != 0ull;
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < 6; ++q) s_red[q][wv] = r7[q];
    s_red[6][wv] = wnv | (wbad ? 0x80000000u : 0u);
  }
  // This workgroup shares only LDS: its global writes are read by later kernels, so its
  // barriers need not wait for them.
  lds_barrier();
  if (wv == 0) {  // lanes 0 .. W - 1 combine the waves' partials
    static_assert(W <= 16, "one partial per lane of row 0");
    uint32_t mn_k[3], mx_k[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      mn_k[a] = row0_min_u32(lane < W ? s_red[a][lane] : 0xffffffffu);
      mx_k[a] = row0_max_u32(lane < W ? s_red[3 + a][lane] : 0u);
    }
    const uint32_t pv = lane < W ? s_red[6][lane] : 0u;
    const uint32_t n = wave_sum_dpp(pv & 0x7fffffffu);
    const bool any_bad = __ballot(pv >> 31) != 0ull;
    int64_t cells = 0;
    Grid g{0.f, 0.f, 0.f, 0.f, 0, 0, 0, 0};
    if (n > 0) {
      const float mn[3] = {float_from_order_key(mn_k[0]), float_from_order_key(mn_k[1]),
                           float_from_order_key(mn_k[2])};
      const float mx[3] = {float_from_order_key(mx_k[0]), float_from_order_key(mx_k[1]),
                           float_from_order_key(mx_k[2])};
      g = rg_grid(mn, mx, n, r_cell, cells, 4);  // the front end's LDS grid: 4n + 64 cells
    }
    g.base = static_cast<int>(static_cast<int64_t>(b) * (4 * ppc + 64));
    if (tid == 0) {
      s_grid = g;
      s_cells = static_cast<int>(cells);
      s_nv = static_cast<int>(n);
      w.grid[b] = g;
      if (batch) w.layout_bad[b] = any_bad ? 1 : 0;
    }
  }
  lds_barrier();
  const Grid g = s_grid;
  const int cells = s_cells, n_valid = s_nv;
  for (int q = tid; q < (cells >> 1) + 1; q += kRgFrontThreads) s_cnt[q] = 0u;
  lds_barrier();
  int cl[kRgFrontPer], rk[kRgFrontPer];
#pragma unroll
  for (int k = 0; k < kRgFrontPer; ++k) {
    cl[k] = 0;
    rk[k] = 0;
    if (ok[k]) {
      const int cx = cell_coord(px[k], g.ox, g.inv_h, g.dx);
      const int cy = cell_coord(py[k], g.oy, g.inv_h, g.dy);
      const int cz = cell_coord(pz[k], g.oz, g.inv_h, g.dz);
      const int c = (cx * g.dy + cy) * g.dz + cz;
      const uint32_t old = atomicAdd(&s_cnt[c >> 1], (c & 1) ? 0x10000u : 1u);
      cl[k] = c;
      rk[k] = static_cast<int>((old >> ((c & 1) * 16)) & 0xffffu);
    }
  }
  lds_barrier();
  // exclusive scan of the cell counts in place; each thread owns an even-aligned run of cells so
  // that no two threads write halves of one word
  const int per = ((cells + 2 * kRgFrontThreads - 1) / (2 * kRgFrontThreads)) * 2;
  const int c0 = tid * per, c1 = min(c0 + per, cells);
  uint32_t sum = 0;
  for (int c = c0; c < c1; ++c) sum += half_of(s_cnt, c);
  const uint32_t incl = wave_inclusive_sum_dpp(sum);
  if (lane == kWave - 1) s_red[0][wv] = incl;
  lds_barrier();
  uint32_t run = incl - sum;
  for (int q = 0; q < wv; ++q) run += s_red[0][q];
  for (int c = c0; c < c1; c += 2) {
    const uint32_t a0 = half_of(s_cnt, c);
    const uint32_t a1 = c + 1 < c1 ? half_of(s_cnt, c + 1) : 0u;
    s_cnt[c >> 1] = run | ((run + a0) << 16);
    run += a0 + a1;
  }
  lds_barrier();
  // cell starts from the scanned counts, one cell per thread per step (coalesced)
  int32_t* cs = w.cell_start + g.base;
  for (int c = tid; c < cells; c += kRgFrontThreads) cs[c] = static_cast<int32_t>(lo + half_of(s_cnt, c));
  if (tid == 0) cs[cells] = static_cast<int32_t>(lo + n_valid);
#pragma unroll
  for (int k = 0; k < kRgFrontPer; ++k) {
    if (!ok[k]) continue;
    const int64_t i = lo + tid + k * kRgFrontThreads;
    const int64_t pos = lo + half_of(s_cnt, cl[k]) + rk[k];
    if (pos < lo + ppc)  // always: the counts sum to the cloud's valid points
      w.spos[pos] = make_float4(px[k], py[k], pz[k], __int_as_float(static_cast<int>(i)));
  }
  // holes: NaN coordinates are within no radius of anything, so a stencil run that reaches one
  // (the last cloud's end sentinel is the total slot when its grid uses its whole cell cap)
  // accepts nothing from it
  const float qnan = __builtin_nanf("");
  for (int64_t h = n_valid + tid; h < ppc; h += kRgFrontThreads)
    w.spos[lo + h] = make_float4(qnan, qnan, qnan, __int_as_float(-1));
  for (int64_t il = tid; il < ppc; il += kRgFrontThreads) {
    w.cnt[lo + il] = 0;
    w.deg[lo + il] = 0;
  }
  if (b == 0)
    for (int64_t q = tid; q < scan_lookback_elems(N); q += kRgFrontThreads) w.deg_scan[q] = 0;
  if (b == B - 1 && tid == 0) w.cell_start[w.cells_max] = static_cast<int32_t>(N);
}

// Visits every source of the 27-cell stencil around the query as (d, j).
template <typename F>
__device__ __forceinline__ void for_each_candidate(const RgWs& w, const Grid& g, float qx, float qy,
                                                   float qz, int qi, bool loop, F&& f) {
  const int cx = cell_coord(qx, g.ox, g.inv_h, g.dx);
  const int cy = cell_coord(qy, g.oy, g.inv_h, g.dy);
  const int cz = cell_coord(qz, g.oz, g.inv_h, g.dz);
  const int z0 = cz > 0 ? cz - 1 : 0;
  const int z1 = cz + 1 < g.dz ? cz + 1 : g.dz - 1;
  for (int ix = cx - 1; ix <= cx + 1; ++ix) {
    if (ix < 0 || ix >= g.dx) continue;
    for (int iy = cy - 1; iy <= cy + 1; ++iy) {
      if (iy < 0 || iy >= g.dy) continue;
      const int c0 = g.base + (ix * g.dy + iy) * g.dz;
      const int a = w.cell_start[c0 + z0];
      const int e = w.cell_start[c0 + z1 + 1];
      for (int p = a; p < e; ++p) {
        const float4 s = w.spos[p];
        const int j = __float_as_int(s.w);
        if (!loop && j == qi) continue;
        f(sqdist(qx, qy, qz, s.x, s.y, s.z), j);
      }
    }
  }
}

// Accepted-source list for one query, kept sorted by index.
struct RowList {
  int32_t* lds;   // LDS column (stride kRgEmitThreads) or nullptr
  int64_t* out;   // output row
  int n = 0;
  __device__ __forceinline__ int get(int m) const {
    return lds ? lds[m * kRgEmitThreads] : static_cast<int>(out[m]);
  }
  __device__ __forceinline__ void set(int m, int v) {
    if (lds) lds[m * kRgEmitThreads] = v; else out[m] = v;
  }
  __device__ __forceinline__ void insert(int j) {
    int m = n;
    while (m > 0) {
      const int v = get(m - 1);
      if (v < j) break;
      set(m, v);
      --m;
    }
    set(m, j);
    ++n;
  }
};

// Exact K smallest (d, j) among the in-radius sources of one target (used when a target has
// more than K of them): the K-th distance bits by binary search, then the index threshold among
// the sources at that distance.  Returns (d*, j*): keep d < d*, or d == d* and j <= j*.
__device__ __forceinline__ void threshold_select(const RgWs& w, const Grid& g, float qx, float qy,
                                                 float qz, int qi, bool lp, float r2, int K,
                                                 uint32_t& dstar, int& jstar) {
  const uint32_t r2b = __float_as_uint(r2);
  uint32_t lo = 0, hi = r2b > 0 ? r2b - 1 : 0;
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    int n = 0;
    for_each_candidate(w, g, qx, qy, qz, qi, lp, [&](float d, int) {
      n += (d < r2) && (__float_as_uint(d) <= mid);
    });
    if (n >= K) hi = mid; else lo = mid + 1;
  }
  dstar = lo;
  int less = 0;
  for_each_candidate(w, g, qx, qy, qz, qi, lp, [&](float d, int) {
    less += (d < r2) && (__float_as_uint(d) < dstar);
  });
  const int need = K - less;
  int jlo = 0, jhi = 0x7ffffffe;
  while (jlo < jhi) {
    const int mid = jlo + ((jhi - jlo) >> 1);
    int n = 0;
    for_each_candidate(w, g, qx, qy, qz, qi, lp, [&](float d, int j) {
      n += (d < r2) && (__float_as_uint(d) == dstar) && (j <= mid);
    });
    if (n >= need) jhi = mid; else jlo = mid + 1;
  }
  jstar = jlo;
}

// Emit pass without the per-target lists (when they would not fit the workspace): one thread per
// target re-scans the stencil, keeping all accepted sources (count <= K) or the K smallest (d, j)
// found by the threshold search, sorted by index in an LDS column (K <= kRgLdsK) or directly in
// the output row.
__global__ void rg_emit(RgWs w, const int64_t* __restrict__ batch, int64_t B, int64_t ppc,
                        float r2, int K, int loop, const int64_t* __restrict__ row_ptr,
                        int64_t* __restrict__ row_out, int64_t* __restrict__ col_out, int use_lds) {
  extern __shared__ int32_t lbuf[];  // K entries per thread, column-major by thread
  r2 = rg_r2(w, r2);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int total = w.cell_start[w.cells_max];
  if (t >= total) return;
  const float4 q = w.spos[t];
  const int qi = __float_as_int(q.w);
  if (qi < 0) return;  // a hole of the per-cloud layout
  const int b = cloud_of(qi, batch, B, ppc);
  const Grid g = w.grid[b];
  const bool lp = loop != 0;
  const int c = w.cnt[qi];
  if (c == 0) return;
  const int64_t o = row_ptr[qi];
  RowList lst;
  lst.lds = use_lds ? lbuf + threadIdx.x : nullptr;
  lst.out = row_out + o;
  if (c <= K) {
    for_each_candidate(w, g, q.x, q.y, q.z, qi, lp, [&](float d, int j) {
      if (d < r2) lst.insert(j);
    });
  } else {
    uint32_t dstar;
    int jstar;
    threshold_select(w, g, q.x, q.y, q.z, qi, lp, r2, K, dstar, jstar);
    for_each_candidate(w, g, q.x, q.y, q.z, qi, lp, [&](float d, int j) {
      if (d < r2) {
        const uint32_t db = __float_as_uint(d);
        if (db < dstar || (db == dstar && j <= jstar)) lst.insert(j);
      }
    });
  }
  for (int m = 0; m < lst.n; ++m) {
    if (lst.lds) row_out[o + m] = lst.get(m);
    col_out[o + m] = qi;
  }
}

// Count pass with kRgGroup lanes per target (targets in cell order, so neighbouring groups
// share cells).  The 18 run bounds of the 3x3 stencil columns are loaded at once, then the first
// kRgGroup sources of all nine runs (one float4 per lane per run, all in flight together);
// longer runs continue chunk by chunk.  Accepted sources are appended to the target's list in
// ballot order (the list is unsorted; the compaction sorts it), the count is the group's total.
constexpr int kRgGroup = 8;
// workgroups per XCD run (xcd_block_runs) of the count and compaction passes: 512 targets
constexpr int64_t kRgXcdRun = 16;

__global__ __launch_bounds__(kRgThreads) void rg_count(RgWs w, const int64_t* __restrict__ batch,
                                                       int64_t B, int64_t ppc, float r2, int K,
                                                       int loop, int64_t* __restrict__ bad_out,
                                                       int check_layout) {
  if (bad_out && blockIdx.x == 0) {  // clouds failing the chunk layout, summed by workgroup 0
    __shared__ uint32_t s_bad[kRgThreads / kWave];
    uint32_t nb = 0;
    if (check_layout)
      for (int64_t b = threadIdx.x; b < B; b += kRgThreads) nb += static_cast<uint32_t>(w.layout_bad[b]);
    nb = wave_sum_dpp(nb);
    if (lane_id() == 0) s_bad[threadIdx.x / kWave] = nb;
    __syncthreads();  // workgroup-uniform: the whole of workgroup 0 takes this branch
    if (threadIdx.x == 0) {
      uint32_t t = 0;
      for (int q = 0; q < kRgThreads / kWave; ++q) t += s_bad[q];
      *bad_out = t;
    }
  }
  r2 = rg_r2(w, r2);
  // each XCD takes runs of 512 consecutive targets in cell order (neighbouring targets share
  // stencil cells in its L2; dense regions are spread over all XCDs)
  const int64_t t = (xcd_block_runs(kRgXcdRun) * kRgThreads + threadIdx.x) / kRgGroup;
  const int sub = static_cast<int>(threadIdx.x) & (kRgGroup - 1);
  const int total = w.cell_start[w.cells_max];
  if (t >= total) return;  // the whole group leaves together
  const float4 q = w.spos[t];
  const int qi = __float_as_int(q.w);
  if (qi < 0) return;  // a hole of the per-cloud layout (group-uniform)
  const int b = cloud_of(qi, batch, B, ppc);
  const Grid g = w.grid[b];
  const int cx = cell_coord(q.x, g.ox, g.inv_h, g.dx);
  const int cy = cell_coord(q.y, g.oy, g.inv_h, g.dy);
  const int cz = cell_coord(q.z, g.oz, g.inv_h, g.dz);
  const int z0 = cz > 0 ? cz - 1 : 0;
  const int z1 = cz + 1 < g.dz ? cz + 1 : g.dz - 1;
  int ra[9], rn[9];
#pragma unroll
  for (int r = 0; r < 9; ++r) {
    const int ix = cx - 1 + r / 3, iy = cy - 1 + r % 3;
    const bool in = ix >= 0 && ix < g.dx && iy >= 0 && iy < g.dy;
    const int c0 = g.base + (ix * g.dy + iy) * g.dz;
    const int a = in ? w.cell_start[c0 + z0] : 0;
    const int e = in ? w.cell_start[c0 + z1 + 1] : 0;
    ra[r] = a;
    rn[r] = e - a;
  }
  float4 sv[9];
#pragma unroll
  for (int r = 0; r < 9; ++r) sv[r] = sub < rn[r] ? w.spos[ra[r] + sub] : make_float4(0.f, 0.f, 0.f, 0.f);
  int32_t* L = w.list ? w.list + static_cast<int64_t>(qi) * K : nullptr;
  const int shift = lane_id() & ~(kRgGroup - 1);
  const uint32_t below = (1u << sub) - 1u;
  const bool lp = loop != 0;
  int c = 0;  // accepted so far (group-uniform)
  auto take = [&](const float4& s4, bool ok) {
    const int j = __float_as_int(s4.w);
    const bool acc = ok && (lp || j != qi) && sqdist(q.x, q.y, q.z, s4.x, s4.y, s4.z) < r2;
    const uint32_t m = static_cast<uint32_t>(__ballot(acc) >> shift) & ((1u << kRgGroup) - 1u);
    if (acc && L) {
      const int slot = c + __popc(m & below);
      if (slot < K) L[slot] = j;
    }
    c += __popc(m);
  };
#pragma unroll
  for (int r = 0; r < 9; ++r) take(sv[r], sub < rn[r]);
  for (int r = 0; r < 9; ++r) {
    for (int m0 = kRgGroup; m0 < rn[r]; m0 += kRgGroup) {  // group-uniform trip count
      const bool ok = m0 + sub < rn[r];
      take(ok ? w.spos[ra[r] + m0 + sub] : make_float4(0.f, 0.f, 0.f, 0.f), ok);
    }
  }
  if (sub == 0) {
    w.cnt[qi] = c;
    w.deg[qi] = c < K ? c : K;
  }
}

// After the edge count is known: kRgGroup lanes per target write its row, sources ascending.
// The collected list is unsorted (traversal order); each source goes to position
// row_ptr[i] + (number of smaller sources in the list), with the list held in the group's
// registers (kRgSlots entries per lane) and compared through lane shuffles.  Targets with more
// than K sources, or lists longer than the registers hold, are done afterwards by the whole
// wave, one at a time (rg_wave_target).
constexpr int kRgSlots = 8;
// In-radius candidates of one target whose distance bits a wave keeps in LDS for the selection.
constexpr int kRgSelCap = 1024;
// Chunks of 64 stencil sources loaded together when staging (eight measured 1.5% slower at C5).
constexpr int kRgStageLoads = 4;

// Run r (0..8) of the stencil around (qx, qy, qz): start and length.
__device__ __forceinline__ void stencil_run(const RgWs& w, const Grid& g, float qx, float qy, float qz,
                                            int r, int& a, int& n) {
  const int cx = cell_coord(qx, g.ox, g.inv_h, g.dx);
  const int cy = cell_coord(qy, g.oy, g.inv_h, g.dy);
  const int cz = cell_coord(qz, g.oz, g.inv_h, g.dz);
  const int z0 = cz > 0 ? cz - 1 : 0;
  const int z1 = cz + 1 < g.dz ? cz + 1 : g.dz - 1;
  const int ix = cx - 1 + r / 3, iy = cy - 1 + r % 3;
  const bool in = ix >= 0 && ix < g.dx && iy >= 0 && iy < g.dy;
  const int c0 = g.base + (ix * g.dy + iy) * g.dz;
  a = in ? w.cell_start[c0 + z0] : 0;
  n = in ? w.cell_start[c0 + z1 + 1] - a : 0;
}

// Calls f(d, j, ok) for every source of the stencil runs, 64 at a time across the wave (every
// lane calls f the same number of times; ok marks a real candidate).
template <typename F>
__device__ __forceinline__ void wave_scan_runs(const RgWs& w, const int (&ra)[9], const int (&rn)[9],
                                               float qx, float qy, float qz, F&& f) {
  const int lane = lane_id();
  for (int r = 0; r < 9; ++r) {
    for (int b0 = 0; b0 < rn[r]; b0 += kWave) {  // wave-uniform trip count
      const bool ok = b0 + lane < rn[r];
      const float4 s = ok ? w.spos[ra[r] + b0 + lane] : make_float4(0.f, 0.f, 0.f, 0.f);
      f(sqdist(qx, qy, qz, s.x, s.y, s.z), __float_as_int(s.w), ok);
    }
  }
}

// One target done by the whole wave: c = its count of in-radius sources (c > 0).
//  c <= K: the list L[0..c) (complete) sorted by index, 64 entries per step.
//  c > K:  the K smallest (d, j): the in-radius sources as (distance bits, index) pairs collected
//          in LDS in one stencil pass (c <= kRgSelCap; beyond that every step re-scans the
//          stencil), the K-th distance d* by radix select on the bits (binary search over the
//          stencil beyond kRgSelCap), the index threshold j*
//          among the sources at d* when they are more than needed, the accepted sources compacted
//          in place and sorted by index.
// The target's row offset o, and for c > K its position and stencil runs, come from the caller.
__device__ void rg_wave_target(const RgWs& w, float r2, int K, bool lp, int64_t i, int c, int64_t o,
                               float qx, float qy, float qz, const int (&ra)[9], const int (&rn)[9],
                               int64_t* __restrict__ row_out, int64_t* __restrict__ col_out,
                               uint32_t* __restrict__ key, int32_t* __restrict__ idx,
                               int32_t* __restrict__ hist) {
  const int lane = lane_id();
  int32_t* L = w.list + i * K;
  if (c > K) {
    const int qi = static_cast<int>(i);
    const bool inl = c <= kRgSelCap;
    int n = 0;
    if (inl) {
      // stage A: in-radius (distance bits, index) into LDS (wave compaction).  The nine runs are
      // one index space (source t of the stencil is ra[r] + t - pre[r] in the run r holding it),
      // so kRgStageLoads chunks of 64 sources are loaded together.
      int pre[9];
      pre[0] = 0;
#pragma unroll
      for (int r = 1; r < 9; ++r) pre[r] = pre[r - 1] + rn[r - 1];
      const int tot = pre[8] + rn[8];
      for (int base = 0; base < tot; base += kWave * kRgStageLoads) {  // wave-uniform
        float4 sv[kRgStageLoads];
#pragma unroll
        for (int u = 0; u < kRgStageLoads; ++u) {
          const int t = base + u * kWave + lane;
          int off = ra[0];
#pragma unroll
          for (int r = 1; r < 9; ++r) off = t >= pre[r] ? ra[r] - pre[r] : off;
          sv[u] = t < tot ? w.spos[off + t] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < kRgStageLoads; ++u) {
          const int t = base + u * kWave + lane;
          const float d = sqdist(qx, qy, qz, sv[u].x, sv[u].y, sv[u].z);
          const int j = __float_as_int(sv[u].w);
          const bool a = t < tot && (lp || j != qi) && d < r2;
          const uint64_t m = __ballot(a);
          const int slot = n + static_cast<int>(__popcll(m & lanemask_lt()));
          if (a && slot < kRgSelCap) {
            key[slot] = __float_as_uint(d);
            idx[slot] = j;
          }
          n += static_cast<int>(__popcll(m));
        }
      }
      n = n < kRgSelCap ? n : kRgSelCap;
      wave_lds_fence();
    }
    // in-radius sources with bits <= dmax (< when strict), or with bits == dmax and j <= jmax
    // (jmax >= 0)
    auto count_le = [&](uint32_t dmax, bool strict, int jmax) -> int {
      int t = 0;
      auto hit = [&](uint32_t db, int j) -> bool {
        return jmax < 0 ? (strict ? db < dmax : db <= dmax) : (db == dmax && j <= jmax);
      };
      if (inl) {
        for (int m = lane; m < n; m += kWave) t += hit(key[m], idx[m]);
      } else {
        wave_scan_runs(w, ra, rn, qx, qy, qz, [&](float d, int j, bool ok) {
          t += ok && (lp || j != qi) && d < r2 && hit(__float_as_uint(d), j);
        });
      }
      return static_cast<int>(wave_sum_dpp(static_cast<uint32_t>(t)));
    };
    // stage B: the K-th smallest distance bits (every in-radius d has bits < bits(r2)).  Staged
    // candidates: a radix select, 8 bits per pass -- a 256-bin LDS histogram of the keys that
    // match the digits chosen so far, then the bin holding the K-th by one wave scan (lane l
    // holds bins 4l .. 4l + 3).  Otherwise a binary search on the bits over the stencil.
    uint32_t dstar;
    int less = 0, at = 0;  // sources below d*, sources at d*
    if (inl) {
      uint32_t prefix = 0u, decided = 0u;
      int k = K;  // rank of the K-th among the keys that match prefix (1 <= k <= their count)
      for (int shift = 24; shift >= 0; shift -= 8) {
        for (int q = lane; q < 256; q += kWave) hist[q] = 0;
        wave_lds_fence();
        for (int m = lane; m < n; m += kWave) {
          const uint32_t v = key[m];
          if ((v & decided) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1);
        }
        wave_lds_fence();
        const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2];
        const int h3 = hist[4 * lane + 3];
        const int sum = h0 + h1 + h2 + h3;
        const int excl = static_cast<int>(wave_inclusive_sum_dpp(static_cast<uint32_t>(sum))) - sum;
        const int L = __builtin_ctzll(__ballot(excl < k && k <= excl + sum) | (1ull << 63));
        int d = 4 * lane, below = excl, hs = h0;
        if (k > below + h0) {
          d += 1; below += h0; hs = h1;
          if (k > below + h1) {
            d += 1; below += h1; hs = h2;
            if (k > below + h2) { d += 1; below += h2; hs = h3; }
          }
        }
        k -= __builtin_amdgcn_readlane(below, L);
        at = __builtin_amdgcn_readlane(hs, L);  // after the last pass: the sources at d*
        prefix |= static_cast<uint32_t>(__builtin_amdgcn_readlane(d, L)) << shift;
        decided |= 0xffu << shift;
        wave_lds_fence();  // every lane has read the histogram before the next pass clears it
      }
      dstar = prefix;
      less = K - k;
    } else {
      uint32_t lo = 0, hi = __float_as_uint(r2) - 1u;
      while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (count_le(mid, false, -1) >= K) hi = mid; else lo = mid + 1u;
      }
      dstar = lo;
      less = count_le(dstar, true, -1);
      at = count_le(dstar, false, -1) - less;
    }
    // stage C: index threshold among the sources at d* when they are more than needed
    const int need = K - less;
    int jstar = 0x7fffffff;
    if (at > need) {
      int jlo = 0, jhi = 0x7ffffffe;
      while (jlo < jhi) {
        const int mid = jlo + ((jhi - jlo) >> 1);
        if (count_le(dstar, false, mid) >= need) jhi = mid; else jlo = mid + 1;
      }
      jstar = jlo;
    }
    auto accept = [&](uint32_t db, int j) { return db < dstar || (db == dstar && j <= jstar); };
    // stage D: the K accepted sources, compacted in place over the LDS indices (a slot never
    // passes the position being read) or into the list when K exceeds the LDS; stage E: ranked
    // by index.  The two forms are separate so that the LDS one reads with LDS instructions.
    if (inl && K <= kRgSelCap) {
      int m0 = 0;
      for (int base = 0; base < n; base += kWave) {  // wave-uniform trip count
        const int m = base + lane;
        const bool a = m < n && accept(key[m], idx[m]);
        const int j = m < n ? idx[m] : 0;
        const uint64_t bm = __ballot(a);
        const int slot = m0 + static_cast<int>(__popcll(bm & lanemask_lt()));
        wave_lds_fence();  // every lane has read its entry before any slot is written
        if (a && slot < K) idx[slot] = j;
        m0 += static_cast<int>(__popcll(bm));
      }
      wave_lds_fence();
      const int K4 = K & ~3;
      for (int m = lane; m < K; m += kWave) {
        const int v = idx[m];
        int r = 0;
        for (int q = 0; q < K4; q += 4) {  // 16-byte broadcast reads
          const int4 u = *reinterpret_cast<const int4*>(idx + q);
          r += (u.x < v) + (u.y < v) + (u.z < v) + (u.w < v);
        }
        for (int q = K4; q < K; ++q) r += idx[q] < v;
        row_out[o + r] = v;
        col_out[o + m] = i;
      }
    } else {
      int m0 = 0;
      if (inl) {
        for (int base = 0; base < n; base += kWave) {  // wave-uniform trip count
          const int m = base + lane;
          const bool a = m < n && accept(key[m], idx[m]);
          const uint64_t bm = __ballot(a);
          const int slot = m0 + static_cast<int>(__popcll(bm & lanemask_lt()));
          if (a && slot < K) L[slot] = idx[m];
          m0 += static_cast<int>(__popcll(bm));
        }
      } else {
        wave_scan_runs(w, ra, rn, qx, qy, qz, [&](float d, int j, bool ok) {
          const bool a = ok && (lp || j != qi) && d < r2 && accept(__float_as_uint(d), j);
          const uint64_t bm = __ballot(a);
          const int slot = m0 + static_cast<int>(__popcll(bm & lanemask_lt()));
          if (a && slot < K) L[slot] = j;
          m0 += static_cast<int>(__popcll(bm));
        });
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      for (int m = lane; m < K; m += kWave) {
        const int v = L[m];
        int r = 0;
        for (int q = 0; q < K; ++q) r += L[q] < v;
        row_out[o + r] = v;
        col_out[o + m] = i;
      }
    }
    wave_lds_fence();  // the LDS is reused by the next target
    return;
  }
  for (int m = lane; m < c; m += kWave) {
    const int v = L[m];
    int r = 0;
    for (int q = 0; q < c; ++q) r += L[q] < v;
    row_out[o + r] = v;
    col_out[o + m] = i;
  }
}

__global__ __launch_bounds__(kRgThreads) void rg_compact(RgWs w, const float* __restrict__ x,
                                                         int64_t N, const int64_t* __restrict__ batch,
                                                         int64_t B, int64_t ppc, float r2, int K,
                                                         int loop, const int64_t* __restrict__ row_ptr,
                                                         int64_t* __restrict__ row_out,
                                                         int64_t* __restrict__ col_out) {
  __shared__ uint32_t s_key[kRgThreads / kWave][kRgSelCap];
  __shared__ __align__(16) int32_t s_idx[kRgThreads / kWave][kRgSelCap];
  __shared__ int32_t s_hist[kRgThreads / kWave][256];
  r2 = rg_r2(w, r2);
  const int64_t i = (xcd_block_runs(kRgXcdRun) * kRgThreads + threadIdx.x) / kRgGroup;
  const int sub = static_cast<int>(threadIdx.x) & (kRgGroup - 1);
  const int c = i < N ? w.cnt[i] : 0;
  const bool group = c > 0 && c <= K && c <= kRgGroup * kRgSlots;  // group-uniform
  if (group) {
    const int32_t* L = w.list + i * K;
    const int64_t o = row_ptr[i];
    int v[kRgSlots];
#pragma unroll
    for (int k = 0; k < kRgSlots; ++k) {
      const int a = k * kRgGroup + sub;
      v[k] = a < c ? L[a] : 0x7fffffff;
    }
    const int gbase = lane_id() & ~(kRgGroup - 1);
    int rank[kRgSlots];
#pragma unroll
    for (int k = 0; k < kRgSlots; ++k) rank[k] = 0;
#pragma unroll
    for (int k2 = 0; k2 < kRgSlots; ++k2) {
      if (k2 * kRgGroup >= c) break;  // group-uniform
#pragma unroll
      for (int l = 0; l < kRgGroup; ++l) {
        const int u = __shfl(v[k2], gbase + l, kWave);  // entry k2 * G + l (INT_MAX past the end)
#pragma unroll
        for (int k = 0; k < kRgSlots; ++k) rank[k] += u < v[k];
      }
    }
#pragma unroll
    for (int k = 0; k < kRgSlots; ++k) {
      const int a = k * kRgGroup + sub;
      if (a < c) {
        row_out[o + rank[k]] = v[k];
        col_out[o + a] = i;
      }
    }
  }
  // the wave's remaining targets, one at a time with all 64 lanes.  Their row offsets and, for
  // those with more than K sources, positions and stencil runs are loaded first for all of them
  // at once: run r of a group's target by the group's lane r (the ninth by its first lane).
  static_assert(kRgGroup == 8, "one lane per stencil run of the group's target");
  const bool rest_t = c > 0 && !group;  // group-uniform
  int64_t po = 0;
  float pqx = 0.f, pqy = 0.f, pqz = 0.f;
  int pa = 0, pn = 0, pa8 = 0, pn8 = 0;
  if (rest_t) {
    po = row_ptr[i];
    if (c > K) {
      const Grid g = w.grid[cloud_of(i, batch, B, ppc)];
      pqx = x[3 * i]; pqy = x[3 * i + 1]; pqz = x[3 * i + 2];
      stencil_run(w, g, pqx, pqy, pqz, sub, pa, pn);
      if (sub == 0) stencil_run(w, g, pqx, pqy, pqz, 8, pa8, pn8);
    }
  }
  uint64_t rest = __ballot(sub == 0 && rest_t);
  while (rest) {
    const int leader = __builtin_ctzll(rest);
    rest &= rest - 1;
    const int64_t ti = __builtin_amdgcn_readlane(static_cast<int>(i), leader);
    const int tc = __builtin_amdgcn_readlane(c, leader);
    const int64_t to = (static_cast<int64_t>(__builtin_amdgcn_readlane(static_cast<int>(po >> 32), leader)) << 32) |
                       static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(po), leader));
    int ra[9], rn[9];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      ra[r] = __builtin_amdgcn_readlane(pa, leader + r);
      rn[r] = __builtin_amdgcn_readlane(pn, leader + r);
    }
    ra[8] = __builtin_amdgcn_readlane(pa8, leader);
    rn[8] = __builtin_amdgcn_readlane(pn8, leader);
    const float tx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pqx), leader));
    const float ty = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pqy), leader));
    const float tz = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pqz), leader));
    rg_wave_target(w, r2, K, loop != 0, ti, tc, to, tx, ty, tz, ra, rn, row_out, col_out,
                   s_key[threadIdx.x / kWave], s_idx[threadIdx.x / kWave], s_hist[threadIdx.x / kWave]);
  }
}

int check_common(const float* x, int64_t N, int64_t B, int64_t ppc, const int64_t* batch,
                 float r2, int64_t K) {
  GEO_REQUIRE(N >= 0 && B >= 1, "radius_graph: need N >= 0 and B >= 1 (N=%lld B=%lld)",
              (long long)N, (long long)B);
  GEO_REQUIRE(N < 0x7fffffffLL / 4, "radius_graph: N=%lld too large", (long long)N);
  GEO_REQUIRE(batch != nullptr || ppc * B == N,
              "radius_graph: without batch, B*points_per_cloud must equal N");
  GEO_REQUIRE(K >= 1 && K < 0x7fffffffLL, "radius_graph: max_num_neighbors must be >= 1");
  GEO_REQUIRE(r2 == r2 && r2 >= 0.f, "radius_graph: r2 must be a non-negative number");
  GEO_REQUIRE(N == 0 || x != nullptr, "radius_graph: null x");
  return GEO_OK;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_radius_workspace_bytes(int64_t N, int64_t B, int64_t max_num_neighbors) {
  if (N < 0 || B < 0 || max_num_neighbors < 0) return 0;
  return carve_rg(nullptr, N, B, max_num_neighbors).bytes;
}

static int radius_count_impl(const float* x, int64_t N, const int64_t* batch, int64_t B,
                             int64_t points_per_cloud, const uint8_t* mask, float r2, float r_cell,
                             const double* r_dev, int64_t max_num_neighbors, int loop,
                             int64_t* row_ptr, void* workspace, size_t workspace_bytes,
                             void* stream, int64_t* edges_host = nullptr) {
  // Contiguous clouds of at most kRgFrontMax points take the per-cloud front end: given by
  // points_per_cloud alone, or by a batch vector that the front end verifies (only when the
  // caller can learn the result: edges_host[1] receives the count of clouds that fail).
  int rc = check_common(x, N, B, points_per_cloud, batch, r2, max_num_neighbors);
  if (rc) return rc;
  GEO_REQUIRE(r_cell > 0.f, "radius_graph: r_cell must be positive");
  GEO_REQUIRE(row_ptr != nullptr, "radius_graph: null row_ptr");
  RgWs w = carve_rg(workspace, N, B, max_num_neighbors);
  w.r_dev = r_dev;
  if (workspace == nullptr || workspace_bytes < w.bytes)
    return set_error(GEO_ERR_WORKSPACE, "radius_graph: workspace %zu bytes, need %zu",
                     workspace_bytes, w.bytes);
  hipStream_t st = as_stream(stream);
  const int K = static_cast<int>(max_num_neighbors);
  const bool front = N > 0 && points_per_cloud > 0 && points_per_cloud <= kRgFrontMax &&
                     B <= kRgFrontMaxClouds && points_per_cloud * B == N &&
                     (batch == nullptr || edges_host != nullptr);
  int64_t* bad_out = edges_host ? edges_host + 1 : nullptr;
  if (front) {
    hipLaunchKernelGGL(rg_front, dim3(static_cast<unsigned>(B)), dim3(kRgFrontThreads), 0, st, w, x,
                       N, batch, B, points_per_cloud, mask, r_cell);
    GEO_LAUNCH_CHECK("rg_front");
    const int64_t gblocks = ceil_div(N * kRgGroup, kRgThreads);
    hipLaunchKernelGGL(rg_count, dim3(gblocks), dim3(kRgThreads), 0, st, w, batch, B,
                       points_per_cloud, r2, K, loop, bad_out, batch ? 1 : 0);
    GEO_LAUNCH_CHECK("rg_count");
    return device_exclusive_scan_lookback<int32_t, int64_t>(w.deg, N, row_ptr, nullptr, true,
                                                            w.deg_scan, st, edges_host);
  }
  if (batch) points_per_cloud = 0;  // the general path reads cloud membership from batch
  {
    int64_t span = w.cells_max + 1;
    if (N > span) span = N;
    if (6 * B > span) span = 6 * B;
    int64_t blocks = ceil_div(span, 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(rg_init, dim3(blocks), dim3(256), 0, st, w, N, B);
    GEO_LAUNCH_CHECK("rg_init");
  }
  if (N > 0) {
    const int64_t blocks = ceil_div(N, kRgThreads);
    if (B == 1 && batch == nullptr && mask == nullptr) {
      hipLaunchKernelGGL(rg_bbox_one, dim3(static_cast<unsigned>(blocks < kRgBoxBlocks ? blocks : kRgBoxBlocks)),
                         dim3(kRgThreads), 0, st, w, x, N);
      GEO_LAUNCH_CHECK("rg_bbox_one");
    } else {
      hipLaunchKernelGGL(rg_bbox, dim3(blocks), dim3(kRgThreads), 0, st, w, x, N, batch, B,
                         points_per_cloud, mask);
      GEO_LAUNCH_CHECK("rg_bbox");
    }
    hipLaunchKernelGGL(rg_setup, dim3(1), dim3(kScanThreads), 0, st, w, B, r_cell);
    GEO_LAUNCH_CHECK("rg_setup");
    hipLaunchKernelGGL(rg_cell, dim3(blocks), dim3(kRgThreads), 0, st, w, x, N, batch, B,
                       points_per_cloud, mask);
    GEO_LAUNCH_CHECK("rg_cell");
  }
  rc = device_exclusive_scan_lookback<int32_t, int32_t>(w.cell_cnt, w.cells_max, w.cell_start,
                                                        nullptr, true, w.cell_scan, st);
  if (rc) return rc;
  if (N > 0) {
    const int64_t blocks = ceil_div(N, kRgThreads);
    hipLaunchKernelGGL(rg_scatter, dim3(blocks), dim3(kRgThreads), 0, st, w, x, N);
    GEO_LAUNCH_CHECK("rg_scatter");
    const int64_t gblocks = ceil_div(N * kRgGroup, kRgThreads);
    hipLaunchKernelGGL(rg_count, dim3(gblocks), dim3(kRgThreads), 0, st, w, batch, B,
                       points_per_cloud, r2, K, loop, bad_out, 0);
    GEO_LAUNCH_CHECK("rg_count");
  }
  if (N == 0 && edges_host) {  // no scan launch to carry the total: zero it (and the failures)
    rc = device_fill<int64_t>(edges_host, 2, int64_t{0}, st);
    if (rc) return rc;
  }
  return device_exclusive_scan_lookback<int32_t, int64_t>(w.deg, N, row_ptr, nullptr, true,
                                                          w.deg_scan, st, edges_host);
}

static int radius_emit_impl(const float* x, int64_t N, const int64_t* batch, int64_t B,
                            int64_t points_per_cloud, float r2, const double* r_dev,
                            int64_t max_num_neighbors, int loop, const int64_t* row_ptr,
                            int64_t* row_out, int64_t* col_out, void* workspace,
                            size_t workspace_bytes, void* stream) {
  int rc = check_common(x, N, B, points_per_cloud, batch, r2, max_num_neighbors);
  if (rc) return rc;
  GEO_REQUIRE(row_ptr != nullptr, "radius_graph: null row_ptr");
  RgWs w = carve_rg(workspace, N, B, max_num_neighbors);
  w.r_dev = r_dev;
  if (workspace == nullptr || workspace_bytes < w.bytes)
    return set_error(GEO_ERR_WORKSPACE, "radius_graph: workspace %zu bytes, need %zu",
                     workspace_bytes, w.bytes);
  if (N == 0) return GEO_OK;
  GEO_REQUIRE(row_out && col_out, "radius_graph: null outputs");
  hipStream_t st = as_stream(stream);
  const int K = static_cast<int>(max_num_neighbors);
  const int64_t blocks = ceil_div(N, kRgEmitThreads);
  if (w.list) {
    hipLaunchKernelGGL(rg_compact, dim3(ceil_div(N * kRgGroup, kRgThreads)), dim3(kRgThreads), 0,
                       st, w, x, N, batch, B, points_per_cloud, r2, K, loop, row_ptr, row_out,
                       col_out);
    GEO_LAUNCH_CHECK("rg_compact");
    return GEO_OK;
  }
  const int use_lds = K <= kRgLdsK ? 1 : 0;
  const size_t lds = use_lds ? static_cast<size_t>(K) * kRgEmitThreads * sizeof(int32_t) : 0;
  hipLaunchKernelGGL(rg_emit, dim3(blocks), dim3(kRgEmitThreads), lds, st, w, batch, B,
                     points_per_cloud, r2, K, loop, row_ptr, row_out, col_out, use_lds);
  GEO_LAUNCH_CHECK("rg_emit");
  return GEO_OK;
}

extern "C" int geo_radius_count(const float* x, int64_t N, const int64_t* batch, int64_t B,
                                int64_t points_per_cloud, const uint8_t* mask, float r2,
                                float r_cell, int64_t max_num_neighbors, int loop,
                                int64_t* row_ptr, void* workspace, size_t workspace_bytes,
                                void* stream) {
  return radius_count_impl(x, N, batch, B, points_per_cloud, mask, r2, r_cell, nullptr,
                           max_num_neighbors, loop, row_ptr, workspace, workspace_bytes, stream);
}

extern "C" int geo_radius_emit(const float* x, int64_t N, const int64_t* batch, int64_t B,
                               int64_t points_per_cloud, const uint8_t* mask, float r2,
                               float r_cell, int64_t max_num_neighbors, int loop,
                               const int64_t* row_ptr, int64_t* row_out, int64_t* col_out,
                               void* workspace, size_t workspace_bytes, void* stream) {
  (void)mask; (void)r_cell;
  return radius_emit_impl(x, N, batch, B, points_per_cloud, r2, nullptr, max_num_neighbors, loop,
                          row_ptr, row_out, col_out, workspace, workspace_bytes, stream);
}

extern "C" int geo_radius_count_dev(const float* x, int64_t N, const int64_t* batch, int64_t B,
                                    int64_t points_per_cloud, const uint8_t* mask,
                                    const double* radius, int64_t max_num_neighbors, int loop,
                                    int64_t* row_ptr, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  GEO_REQUIRE(radius != nullptr, "radius_graph: null device radius");
  return radius_count_impl(x, N, batch, B, points_per_cloud, mask, 0.f, 1.f, radius,
                           max_num_neighbors, loop, row_ptr, workspace, workspace_bytes, stream);
}

extern "C" int geo_radius_emit_dev(const float* x, int64_t N, const int64_t* batch, int64_t B,
                                   int64_t points_per_cloud, const uint8_t* mask,
                                   const double* radius, int64_t max_num_neighbors, int loop,
                                   const int64_t* row_ptr, int64_t* row_out, int64_t* col_out,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  (void)mask;
  GEO_REQUIRE(radius != nullptr, "radius_graph: null device radius");
  return radius_emit_impl(x, N, batch, B, points_per_cloud, 0.f, radius, max_num_neighbors, loop,
                          row_ptr, row_out, col_out, workspace, workspace_bytes, stream);
}

// Asynchronous form of the two phases: the count also writes E into mapped pinned host memory
// (edges_host: a host pointer from hipHostMalloc, e.g. a pin_memory tensor), and the emit can be
// issued at once into bound-sized buffers (N * max_num_neighbors entries) before the host has
// read E; geo_radius_copy_edges then moves the first E entries into the exact-sized outputs.
// radius_dev, when not NULL, replaces r2 / r_cell (as geo_radius_count_dev).
extern "C" int geo_radius_count_async(const float* x, int64_t N, const int64_t* batch, int64_t B,
                                      int64_t points_per_cloud, const uint8_t* mask, float r2,
                                      float r_cell, const double* radius_dev,
                                      int64_t max_num_neighbors, int loop, int64_t* row_ptr,
                                      int64_t* edges_host, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(edges_host != nullptr, "radius_graph: null edges_host");
  int64_t* host_dev = nullptr;
  GEO_HIP_CHECK(hipHostGetDevicePointer(reinterpret_cast<void**>(&host_dev), edges_host, 0));
  GEO_REQUIRE(host_dev != nullptr, "radius_graph: edges_host is not mapped pinned memory");
  if (radius_dev) { r2 = 0.f; r_cell = 1.f; }
  return radius_count_impl(x, N, batch, B, points_per_cloud, mask, r2, r_cell, radius_dev,
                           max_num_neighbors, loop, row_ptr, workspace, workspace_bytes, stream,
                           host_dev);
}

namespace geo {
namespace {
__global__ void rg_copy_edges(const int64_t* __restrict__ src_row, const int64_t* __restrict__ src_col,
                              int64_t E, int64_t* __restrict__ row, int64_t* __restrict__ col) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < E; q += stride) {
    row[q] = src_row[q];
    col[q] = src_col[q];
  }
}
}  // namespace
}  // namespace geo

extern "C" int geo_radius_copy_edges(const int64_t* src_row, const int64_t* src_col, int64_t E,
                                     int64_t* row, int64_t* col, void* stream) {
  GEO_REQUIRE(E >= 0, "radius_graph: negative edge count");
  if (E == 0) return GEO_OK;
  GEO_REQUIRE(src_row && src_col && row && col, "radius_graph: null edge arrays");
  int64_t blocks = ceil_div(E, 256);
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(rg_copy_edges, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     as_stream(stream), src_row, src_col, E, row, col);
  GEO_LAUNCH_CHECK("rg_copy_edges");
  return GEO_OK;
}
