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

// k above the largest list (kKnnMaxList) is served in passes of at most kKnnMaxList columns:
// pass p writes columns [col0, col0 + width) of each row (LB = true for p > 0) and admits only
// sources whose key (d, j) is above the key in column col0 - 1, which the previous pass wrote,
// so the passes together list the k smallest keys in order.  A row whose column col0 - 1 is
// padding has no further neighbours: the pass leaves its padding.
constexpr int kKnnMaxList = 128;

template <int KMAX, bool LB = false>
__global__ __launch_bounds__(kKnnThreads) void knn_kernel(
    const float* __restrict__ query, int64_t Nq, const float* __restrict__ source, int64_t Ns,
    const int64_t* __restrict__ ptr_q, const int64_t* __restrict__ ptr_s,
    const int64_t* __restrict__ tiles, int64_t B, int k, int64_t* __restrict__ out_idx,
    float* __restrict__ out_dist, int col0, int width) {
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
  bool qok = q < qc;
  float lbd = -__builtin_inff();  // key of column col0 - 1 (passes after the first)
  int64_t lbj = -1;
  if constexpr (LB) {
    if (qok) {
      lbj = out_idx[q * k + col0 - 1];
      lbd = out_dist[q * k + col0 - 1];
      qok = lbj >= 0;  // padding there: nothing further to list
    }
  }

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
      bool above = true;
      if constexpr (LB) above = d > lbd || (d == lbd && s0 + i > lbj);
      if (above && d < D[KMAX - 1]) {
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
    int64_t* oi = out_idx + q * k + col0;
    float* od = out_dist + q * k + col0;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      if (i < width) {
        oi[i] = J[i] >= 0 ? static_cast<int64_t>(J[i]) : -1;
        od[i] = J[i] >= 0 ? D[i] : 1e30f;
      }
    }
  }
}

template <int KMAX>
int launch_knn(const float* query, int64_t Nq, const float* source, int64_t Ns,
               const int64_t* ptr_q, const int64_t* ptr_s, const int64_t* tiles, int64_t B, int k,
               int64_t* out_idx, float* out_dist, hipStream_t st, int col0 = 0, int width = -1) {
  const int64_t grid = ceil_div(Nq, kKnnThreads) + B;
  if (width < 0) width = k;
  if (col0 == 0)
    hipLaunchKernelGGL((knn_kernel<KMAX, false>), dim3(grid), dim3(kKnnThreads), 0, st, query, Nq,
                       source, Ns, ptr_q, ptr_s, tiles, B, k, out_idx, out_dist, col0, width);
  else
    hipLaunchKernelGGL((knn_kernel<KMAX, true>), dim3(grid), dim3(kKnnThreads), 0, st, query, Nq,
                       source, Ns, ptr_q, ptr_s, tiles, B, k, out_idx, out_dist, col0, width);
  GEO_LAUNCH_CHECK("knn_kernel");
  return GEO_OK;
}

// --------------------------------------------------------------------------- grid search ---
// Clouds of many sources and k <= 32: each source cloud is binned into a uniform grid (cell
// edge chosen so a cell holds about k/4 points at the cloud's mean density, at most 1024 cells
// per axis and 2n + 64 cells), sources are counting-sorted by cell, and each query visits the
// cells in shells of growing Chebyshev radius around its own cell.  After a shell it stops when
// its k-th distance is below a bound that every unvisited source provably exceeds: the query's
// distance to the faces of the visited block, measured in cell units minus 1e-3 of a cell (the
// cell coordinates are rounded fp32 values below 1024, accurate to ~1e-4 cells), scaled by the
// cell edge and shrunk by 1e-5 relative (the fp32 distance of a farther point can round down
// by less than that).  The stop test is strict, so a source at exactly the k-th distance with a
// smaller index cannot be missed.  Candidates arrive in cell order, so the register list keeps
// the total order (d, j) explicitly, as one 64-bit key per entry (distance bits, index): one
// unsigned compare per step instead of a distance compare plus an index tie-break.
constexpr int kKnnGridThreads = 256;
constexpr int kKnnSetupThreads = 1024;
constexpr int kKnnGridMaxAxis = 1024;
constexpr int kKnnGridMaxK = 32;
constexpr double kKnnCellTarget = 0.25;  // points per cell per neighbour (measured best)
constexpr int kKnnCellCap = 2;            // cells per point
constexpr int64_t kKnnWideSources = 65536; // one cloud this large: a wave per query for k <= 8
constexpr int kKnnBoxParts = 64;           // most workgroups per cloud for the bounding box
constexpr int64_t kKnnBoxChunk = 16384;    // points per bounding-box workgroup

struct KnnGrid {
  float ox, oy, oz, inv_h, h;
  int dx, dy, dz, base, ncells;
};

struct KnnGridWs {
  KnnGrid* grid;
  int32_t* cell_cnt;
  int32_t* cell_start;
  uint64_t* cell_scan;  // look-back status of the cell scan; zeroed with cell_cnt (carved next)
  int32_t* pt_cell;
  int32_t* pt_rank;
  float4* spos;
  uint32_t* box_part;  // [B][kKnnBoxParts][6] partial bounding boxes (order keys)
  int64_t cells_max;
};

KnnGridWs carve_knn_grid(void* base, int64_t Ns, int64_t B, size_t* bytes) {
  Carver c(base);
  KnnGridWs w;
  const int64_t nn = Ns > 0 ? Ns : 1, bb = B > 0 ? B : 1;
  w.cells_max = kKnnCellCap * Ns + 64 * bb;
  w.grid = c.take<KnnGrid>(bb);
  w.cell_cnt = c.take<int32_t>(w.cells_max + 1);
  w.cell_scan = c.take<uint64_t>(scan_lookback_elems(w.cells_max + 1));
  w.cell_start = c.take<int32_t>(w.cells_max + 1);
  w.pt_cell = c.take<int32_t>(nn);
  w.pt_rank = c.take<int32_t>(nn);
  w.spos = c.take<float4>(nn);
  w.box_part = c.take<uint32_t>(bb * kKnnBoxParts * 6);
  *bytes = c.used;
  return w;
}

__device__ __forceinline__ int64_t clamp_range(int64_t v, int64_t n) { return v < 0 ? 0 : (v > n ? n : v); }

// Partial bounding boxes of large clouds: block (p, b) reduces the p-th of `parts` equal slices
// of cloud b into box_part[b][p] (order keys, so the minimum and maximum are integer ones).
__global__ __launch_bounds__(kKnnSetupThreads) void knn_grid_box_part(
    const float* __restrict__ source, int64_t Ns, const int64_t* __restrict__ ptr_s, int parts,
    uint32_t* __restrict__ box_part) {
  constexpr int W = kKnnSetupThreads / kWave;
  __shared__ uint32_t red[6][W];
  const int p = blockIdx.x, b = blockIdx.y;
  const int64_t sa = clamp_range(ptr_s[b], Ns);
  const int64_t sc = sa > clamp_range(ptr_s[b + 1], Ns) ? sa : clamp_range(ptr_s[b + 1], Ns);
  const int64_t chunk = (sc - sa + parts - 1) / parts;
  const int64_t pa = sa + p * chunk, pc = min(sc, pa + chunk);
  const int t = threadIdx.x, w = t / kWave;
  uint32_t mn[3] = {~0u, ~0u, ~0u}, mx[3] = {0u, 0u, 0u};
  for (int64_t i = pa + t; i < pc; i += kKnnSetupThreads) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const uint32_t kk = float_order_key(source[3 * i + a]);
      mn[a] = min(mn[a], kk);
      mx[a] = max(mx[a], kk);
    }
  }
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    mn[a] = wave_min_u32(mn[a]);
    mx[a] = wave_max_u32(mx[a]);
  }
  if (lane_id() == 0) {
#pragma unroll
    for (int a = 0; a < 3; ++a) { red[a][w] = mn[a]; red[3 + a][w] = mx[a]; }
  }
  __syncthreads();
  if (t < 6) {
    uint32_t v = red[t][0];
    for (int ww = 1; ww < W; ++ww) v = t < 3 ? min(v, red[t][ww]) : max(v, red[t][ww]);
    box_part[(static_cast<int64_t>(b) * kKnnBoxParts + p) * 6 + t] = v;
  }
}

// One block per source cloud: bounding box (from `parts` partial boxes when parts > 0), then
// (thread 0) the grid of that cloud.
__global__ __launch_bounds__(kKnnSetupThreads) void knn_grid_setup(
    const float* __restrict__ source, int64_t Ns, const int64_t* __restrict__ ptr_s, int k,
    KnnGrid* __restrict__ grid, const uint32_t* __restrict__ box_part, int parts) {
  constexpr int W = kKnnSetupThreads / kWave;
  __shared__ uint32_t red[6][W];
  const int b = blockIdx.x;
  const int64_t sa = clamp_range(ptr_s[b], Ns);
  const int64_t sc = sa > clamp_range(ptr_s[b + 1], Ns) ? sa : clamp_range(ptr_s[b + 1], Ns);
  const int t = threadIdx.x, w = t / kWave;
  uint32_t mn[3] = {~0u, ~0u, ~0u}, mx[3] = {0u, 0u, 0u};
  if (parts > 0) {
    if (t < parts) {
      const uint32_t* bp = box_part + (static_cast<int64_t>(b) * kKnnBoxParts + t) * 6;
#pragma unroll
      for (int a = 0; a < 3; ++a) { mn[a] = bp[a]; mx[a] = bp[3 + a]; }
    }
  } else {
#pragma unroll 4
    for (int64_t i = sa + t; i < sc; i += kKnnSetupThreads) {
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        const uint32_t kk = float_order_key(source[3 * i + a]);
        mn[a] = min(mn[a], kk);
        mx[a] = max(mx[a], kk);
      }
    }
  }
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    mn[a] = wave_min_u32(mn[a]);
    mx[a] = wave_max_u32(mx[a]);
  }
  if (lane_id() == 0) {
#pragma unroll
    for (int a = 0; a < 3; ++a) { red[a][w] = mn[a]; red[3 + a][w] = mx[a]; }
  }
  __syncthreads();
  if (t != 0) return;
  float lo[3], hi[3];
  for (int a = 0; a < 3; ++a) {
    uint32_t m0 = red[a][0], m1 = red[3 + a][0];
    for (int ww = 1; ww < W; ++ww) { m0 = min(m0, red[a][ww]); m1 = max(m1, red[3 + a][ww]); }
    lo[a] = float_from_order_key(m0);
    hi[a] = float_from_order_key(m1);
  }
  const int64_t n = sc - sa;
  KnnGrid g{0.f, 0.f, 0.f, 0.f, 0.f, 1, 1, 1, 0, 1};
  double ext[3];
  bool finite = n > 0;
  for (int a = 0; a < 3; ++a) {
    ext[a] = static_cast<double>(hi[a]) - static_cast<double>(lo[a]);
    finite = finite && ext[a] >= 0.0 && ext[a] < 1e30;
  }
  if (finite) {
    const double emax = fmax(fmax(ext[0], ext[1]), ext[2]);
    const double target = fmax(kKnnCellTarget * k, 1.0);
    double h = emax;  // fixed point of h = cbrt(prod max(ext, h) * target / n)
    for (int it = 0; it < 12 && h > 0.0; ++it)
      h = cbrt(fmax(ext[0], h) * fmax(ext[1], h) * fmax(ext[2], h) * target / static_cast<double>(n));
    if (h > 0.0) {
      const double cap = kKnnCellCap * static_cast<double>(n) + 64.0;
      int64_t d[3] = {1, 1, 1};
      bool ok = false;
      for (int it = 0; it < 64 && !ok; ++it) {
        double prod = 1.0, worst = 0.0;
        for (int a = 0; a < 3; ++a) {
          const double q = floor(ext[a] / h) + 1.0;
          d[a] = q < 4.0 * kKnnGridMaxAxis ? static_cast<int64_t>(q) : 4 * kKnnGridMaxAxis;
          prod *= static_cast<double>(d[a]);
          worst = fmax(worst, static_cast<double>(d[a]) / kKnnGridMaxAxis);
        }
        ok = prod <= cap && worst <= 1.0;
        if (!ok) h *= fmax(fmax(cbrt(prod / cap), worst), 1.0) * 1.01;
      }
      if (ok) {
        g.ox = lo[0]; g.oy = lo[1]; g.oz = lo[2];
        g.inv_h = static_cast<float>(1.0 / h);
        g.h = static_cast<float>(h * (1.0 - 1e-6));
        g.dx = static_cast<int>(d[0]); g.dy = static_cast<int>(d[1]); g.dz = static_cast<int>(d[2]);
      }
    }
  }
  g.ncells = n > 0 ? g.dx * g.dy * g.dz : 0;
  grid[b] = g;
}

// Single block: cell bases (exclusive scan of the cells per cloud).
__global__ __launch_bounds__(kScanThreads) void knn_grid_base(KnnGrid* __restrict__ grid, int64_t B) {
  __shared__ int64_t lds[kScanThreads / kWave];
  int64_t carry = 0;
  for (int64_t base = 0; base < B; base += kScanThreads) {
    const int64_t b = base + threadIdx.x;
    const int64_t cells = b < B ? grid[b].ncells : 0;
    int64_t total;
    const int64_t off = block_exclusive_scan<int64_t>(cells, lds, total);
    if (b < B) grid[b].base = static_cast<int>(carry + off);
    carry += total;
  }
}

__device__ __forceinline__ int knn_cell_coord(float p, float o, float inv_h, int dim, float* u_out) {
#pragma clang fp contract(off)
  const float u = (p - o) * inv_h;
  *u_out = u;
  const int c = static_cast<int>(floorf(u));
  return c < 0 ? 0 : (c >= dim ? dim - 1 : c);
}

// Last b in [0, B) with ptr[b] <= i (the cloud holding index i, if any).
__device__ __forceinline__ int64_t cloud_of_index(const int64_t* __restrict__ ptr, int64_t B, int64_t i) {
  int64_t lo = 0, hi = B;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ptr[mid + 1] <= i) lo = mid + 1; else hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kKnnGridThreads) void knn_grid_cell(
    const float* __restrict__ source, int64_t Ns, const int64_t* __restrict__ ptr_s, int64_t B,
    KnnGridWs w) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= Ns) return;
  const int64_t b = cloud_of_index(ptr_s, B, i);
  if (b >= B || i < ptr_s[b] || i >= ptr_s[b + 1]) {
    w.pt_cell[i] = -1;
    return;
  }
  const KnnGrid g = w.grid[b];
  float u;
  const int cx = knn_cell_coord(source[3 * i], g.ox, g.inv_h, g.dx, &u);
  const int cy = knn_cell_coord(source[3 * i + 1], g.oy, g.inv_h, g.dy, &u);
  const int cz = knn_cell_coord(source[3 * i + 2], g.oz, g.inv_h, g.dz, &u);
  const int c = g.base + (cx * g.dy + cy) * g.dz + cz;
  w.pt_cell[i] = c;
  w.pt_rank[i] = cell_rank(&w.cell_cnt[c], c);
}

__global__ __launch_bounds__(kKnnGridThreads) void knn_grid_scatter(const float* __restrict__ source,
                                                                    int64_t Ns, KnnGridWs w) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= Ns) return;
  const int c = w.pt_cell[i];
  if (c < 0) return;
  w.spos[w.cell_start[c] + w.pt_rank[i]] =
      make_float4(source[3 * i], source[3 * i + 1], source[3 * i + 2], __int_as_float(static_cast<int>(i)));
}

// Candidate key: the distance's bits above the source index.  Squared distances are
// non-negative floats, whose bits order like the values, so one unsigned compare of keys gives
// the total order used throughout: distance, then source index.  An empty slot holds ~0.
__device__ __forceinline__ uint64_t knn_key(float d, int j) {
  return (static_cast<uint64_t>(__float_as_uint(d)) << 32) | static_cast<uint32_t>(j);
}

// Sorted top-KMAX list of one lane; inserts (d, j) if it is among the KMAX smallest (infinite and
// NaN distances never enter).
template <int KMAX>
__device__ __forceinline__ void knn_insert(uint64_t (&L)[KMAX], float d, int j) {
  const uint64_t key = knn_key(d, j);
  if (__float_as_uint(d) < 0x7f800000u && key < L[KMAX - 1]) {
#pragma unroll
    for (int m = KMAX - 1; m > 0; --m) {
      const uint64_t kept = key < L[m] ? key : L[m];
      L[m] = key < L[m - 1] ? L[m - 1] : kept;
    }
    L[0] = key < L[0] ? key : L[0];
  }
}

// Merge with the list of the lane `mask` away: keep the KMAX smallest of both, sorted.  The
// element-wise minimum of one list and the other reversed is bitonic and holds exactly the KMAX
// smallest; half-cleaners sort it.  Both lanes end with the same list.
template <int KMAX>
__device__ __forceinline__ void knn_merge_xor(uint64_t (&L)[KMAX], int mask) {
  uint64_t P[KMAX];
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(static_cast<uint32_t>(L[i])), mask, kWave));
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(static_cast<uint32_t>(L[i] >> 32)), mask, kWave));
    P[i] = (static_cast<uint64_t>(hi) << 32) | lo;
  }
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    const uint64_t o = P[KMAX - 1 - i];
    L[i] = o < L[i] ? o : L[i];
  }
#pragma unroll
  for (int sd = KMAX / 2; sd > 0; sd >>= 1) {
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      if ((i & sd) == 0) {
        const uint64_t a = L[i], c = L[i + sd];
        const bool sw = c < a;
        L[i] = sw ? c : a;
        L[i + sd] = sw ? a : c;
      }
    }
  }
}

// G lanes per query: the lanes of a group split every visited cell range (consecutive sources,
// so the group's loads are contiguous), each keeps its own sorted top-KMAX, the stop test counts
// the group's candidates below the bound (exact: a lane that dropped a candidate below the bound
// already holds KMAX >= k of them), and the lists are merged pairwise at the end.
template <int KMAX, int G>
__global__ __launch_bounds__(kKnnGridThreads) void knn_grid_query(
    const float* __restrict__ query, int64_t Nq, const int64_t* __restrict__ ptr_q, int64_t B,
    KnnGridWs w, int k, int64_t* __restrict__ out_idx, float* __restrict__ out_dist) {
  const int64_t gt = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t q = gt / G;
  const int gl = static_cast<int>(gt % G);
  if (q >= Nq) return;  // whole groups leave together (G divides the block)
  const int64_t b = cloud_of_index(ptr_q, B, q);
  const bool covered = b < B && q >= ptr_q[b] && q < ptr_q[b + 1];
  if (!covered || w.grid[b].ncells == 0) {  // no cloud, or an empty source cloud: padding
    for (int i = gl; i < k; i += G) {
      out_idx[q * k + i] = -1;
      out_dist[q * k + i] = 1e30f;
    }
    return;
  }
  const KnnGrid g = w.grid[b];
  const float qx = query[3 * q], qy = query[3 * q + 1], qz = query[3 * q + 2];
  float ux, uy, uz;
  const int cx = knn_cell_coord(qx, g.ox, g.inv_h, g.dx, &ux);
  const int cy = knn_cell_coord(qy, g.oy, g.inv_h, g.dy, &uy);
  const int cz = knn_cell_coord(qz, g.oz, g.inv_h, g.dz, &uz);
  uint64_t L[KMAX];
#pragma unroll
  for (int i = 0; i < KMAX; ++i) L[i] = ~0ull;

  auto visit = [&](int a, int e) {
    for (int p = a + gl; p < e; p += G) {
      const float4 s = w.spos[p];
      knn_insert<KMAX>(L, sqdist(qx, qy, qz, s.x, s.y, s.z), __float_as_int(s.w));
    }
  };
  const int maxr = max(max(g.dx, g.dy), g.dz);
  for (int r = 0; r <= maxr; ++r) {
    const int x0 = max(cx - r, 0), x1 = min(cx + r, g.dx - 1);
    const int y0 = max(cy - r, 0), y1 = min(cy + r, g.dy - 1);
    const int z0 = max(cz - r, 0), z1 = min(cz + r, g.dz - 1);
    for (int ix = x0; ix <= x1; ++ix) {
      const bool xface = ix == cx - r || ix == cx + r;
      for (int iy = y0; iy <= y1; ++iy) {
        const int c0 = g.base + (ix * g.dy + iy) * g.dz;
        if (xface || iy == cy - r || iy == cy + r) {
          visit(w.cell_start[c0 + z0], w.cell_start[c0 + z1 + 1]);
        } else {
          if (cz - r >= 0) visit(w.cell_start[c0 + cz - r], w.cell_start[c0 + cz - r + 1]);
          if (cz + r < g.dz) visit(w.cell_start[c0 + cz + r], w.cell_start[c0 + cz + r + 1]);
        }
      }
    }
    // distance (cell units) from the query to the faces of the visited block that still have
    // cells beyond them
    float gap = __builtin_inff();
    if (cx - r > 0) gap = fminf(gap, ux - static_cast<float>(cx - r));
    if (cx + r < g.dx - 1) gap = fminf(gap, static_cast<float>(cx + r + 1) - ux);
    if (cy - r > 0) gap = fminf(gap, uy - static_cast<float>(cy - r));
    if (cy + r < g.dy - 1) gap = fminf(gap, static_cast<float>(cy + r + 1) - uy);
    if (cz - r > 0) gap = fminf(gap, uz - static_cast<float>(cz - r));
    if (cz + r < g.dz - 1) gap = fminf(gap, static_cast<float>(cz + r + 1) - uz);
    if (gap == __builtin_inff()) break;  // every cell of the cloud visited
    const float gr = (gap - 1e-3f) * g.h;
    const float bound = gap > 1e-3f ? gr * gr * (1.0f - 1e-5f) : 0.0f;
    const uint64_t bound_key = static_cast<uint64_t>(__float_as_uint(bound)) << 32;
    int below = 0;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) below += L[i] < bound_key ? 1 : 0;
#pragma unroll
    for (int m = 1; m < G; m <<= 1) below += __shfl_xor(below, m, kWave);
    if (below >= k) break;
  }
#pragma unroll
  for (int m = 1; m < G; m <<= 1) knn_merge_xor<KMAX>(L, m);
  int64_t* oi = out_idx + q * k;
  float* od = out_dist + q * k;
#pragma unroll
  for (int i = 0; i < KMAX; ++i) {
    if (i < k && i % G == gl) {
      const bool any = L[i] != ~0ull;
      oi[i] = any ? static_cast<int64_t>(static_cast<int32_t>(static_cast<uint32_t>(L[i]))) : -1;
      od[i] = any ? __uint_as_float(static_cast<uint32_t>(L[i] >> 32)) : 1e30f;
    }
  }
}

bool knn_use_grid(int64_t Ns, int64_t B, int64_t k) {
  return k >= 1 && k <= kKnnGridMaxK && B >= 1 && Ns >= 1024 * B;
}

int launch_knn_grid(const float* query, int64_t Nq, const float* source, int64_t Ns,
                    const int64_t* ptr_q, const int64_t* ptr_s, int64_t B, int k, int64_t* out_idx,
                    float* out_dist, void* workspace, hipStream_t st) {
  size_t bytes = 0;
  const KnnGridWs w = carve_knn_grid(workspace, Ns, B, &bytes);
  // Clouds of more than 2 * kKnnBoxChunk points on average: the bounding box is reduced by up to
  // kKnnBoxParts workgroups per cloud first (one workgroup reading a 131,072-point cloud took
  // 23 us), the setup then combines their partial boxes.
  const int64_t avg = ceil_div(Ns, B);
  const int64_t want = ceil_div(avg, kKnnBoxChunk);
  const int parts = avg > 2 * kKnnBoxChunk ? static_cast<int>(want < kKnnBoxParts ? want : kKnnBoxParts) : 0;
  if (parts > 0) {
    hipLaunchKernelGGL(knn_grid_box_part, dim3(parts, static_cast<unsigned>(B)),
                       dim3(kKnnSetupThreads), 0, st, source, Ns, ptr_s, parts, w.box_part);
    GEO_LAUNCH_CHECK("knn_grid_box_part");
  }
  hipLaunchKernelGGL(knn_grid_setup, dim3(B), dim3(kKnnSetupThreads), 0, st, source, Ns, ptr_s, k,
                     w.grid, w.box_part, parts);
  GEO_LAUNCH_CHECK("knn_grid_setup");
  hipLaunchKernelGGL(knn_grid_base, dim3(1), dim3(kScanThreads), 0, st, w.grid, B);
  GEO_LAUNCH_CHECK("knn_grid_base");
  // cell counts and the scan's look-back status are carved next to each other: one zero fill
  const int64_t zero_words =
      (reinterpret_cast<char*>(w.cell_scan + scan_lookback_elems(w.cells_max + 1)) -
       reinterpret_cast<char*>(w.cell_cnt)) / static_cast<int64_t>(sizeof(int32_t));
  int rc = device_fill<int32_t>(w.cell_cnt, zero_words, 0, st);
  if (rc) return rc;
  const unsigned gs = static_cast<unsigned>(ceil_div(Ns, kKnnGridThreads));
  hipLaunchKernelGGL(knn_grid_cell, dim3(gs), dim3(kKnnGridThreads), 0, st, source, Ns, ptr_s, B, w);
  GEO_LAUNCH_CHECK("knn_grid_cell");
  rc = device_exclusive_scan_lookback<int32_t, int32_t>(w.cell_cnt, w.cells_max + 1, w.cell_start,
                                                        nullptr, false, w.cell_scan, st);
  if (rc) return rc;
  hipLaunchKernelGGL(knn_grid_scatter, dim3(gs), dim3(kKnnGridThreads), 0, st, source, Ns, w);
  GEO_LAUNCH_CHECK("knn_grid_scatter");
  // Lanes per query: a wave runs as long as its slowest query.  In one scene-scale cloud (a
  // lidar frame) density varies by orders of magnitude, so the few queries in dense regions
  // scan hundreds of candidates: a whole wave per query for k <= 8 there (C5 with 8 lanes
  // 0.42 ms, 16 lanes 0.196, 32 lanes 0.152, 64 lanes 0.147 ms); batched object-scale clouds
  // are near uniform and do best with 8 (32 costs them ~10%).
  const bool wide = B == 1 && Ns >= kKnnWideSources;
#define GEO_KNN_GRID_LAUNCH(KV, GV)                                                             \
  {                                                                                             \
    const unsigned gq = static_cast<unsigned>(ceil_div(Nq * GV, kKnnGridThreads));             \
    hipLaunchKernelGGL((knn_grid_query<KV, GV>), dim3(gq), dim3(kKnnGridThreads), 0, st, query, \
                       Nq, ptr_q, B, w, k, out_idx, out_dist);                                  \
    GEO_LAUNCH_CHECK("knn_grid_query");                                                         \
    return GEO_OK;                                                                              \
  }
#define GEO_KNN_GRID_CASE(KV, GV)                                                               \
  if (k <= KV) {                                                                                \
    if (GV == 8 && wide) GEO_KNN_GRID_LAUNCH(KV, 64)                                             \
    GEO_KNN_GRID_LAUNCH(KV, GV)                                                                 \
  }
  GEO_KNN_GRID_CASE(1, 8) GEO_KNN_GRID_CASE(2, 8) GEO_KNN_GRID_CASE(4, 8)
  GEO_KNN_GRID_CASE(8, 8) GEO_KNN_GRID_CASE(16, 16) GEO_KNN_GRID_CASE(32, 16)
#undef GEO_KNN_GRID_CASE
#undef GEO_KNN_GRID_LAUNCH
  return set_error(GEO_ERR_UNSUPPORTED, "knn: k=%d unsupported by the grid search", k);
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" size_t geo_knn_workspace_bytes(int64_t Nq, int64_t Ns, int64_t B, int64_t k) {
  (void)Nq;
  if (Ns < 0 || B < 0) return 0;
  if (knn_use_grid(Ns, B, k)) {
    size_t bytes = 0;
    carve_knn_grid(nullptr, Ns, B, &bytes);
    return bytes;
  }
  return static_cast<size_t>(B + 1) * sizeof(int64_t);
}

extern "C" int geo_knn(const float* query, int64_t Nq, const float* source, int64_t Ns,
                       const int64_t* ptr_q, const int64_t* ptr_s, int64_t B, int64_t k,
                       int64_t* out_idx, float* out_dist, void* workspace, size_t workspace_bytes,
                       void* stream) {
  GEO_REQUIRE(Nq >= 0 && Ns >= 0 && B >= 0, "knn: negative size");
  GEO_REQUIRE(k >= 0, "knn: k must be non-negative (got %lld)", (long long)k);
  GEO_REQUIRE(k < 0x7fffffffLL, "knn: k=%lld exceeds int32", (long long)k);
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
  GEO_REQUIRE(Ns == 0 || source != nullptr, "knn: null source");
  const int kk = static_cast<int>(k);
  // the grid search writes every output row itself (padding for queries outside every cloud)
  if (knn_use_grid(Ns, B, k))
    return launch_knn_grid(query, Nq, source, Ns, ptr_q, ptr_s, B, kk, out_idx, out_dist,
                           workspace, st);
  // Queries outside every cloud keep padding.
  int rc = device_fill<int64_t>(out_idx, Nq * k, -1, st);
  if (rc) return rc;
  rc = device_fill<float>(out_dist, Nq * k, 1e30f, st);
  if (rc) return rc;
  hipLaunchKernelGGL(knn_prepare_kernel, dim3(1), dim3(kScanThreads), 0, st, ptr_q, B, Nq, tiles);
  GEO_LAUNCH_CHECK("knn_prepare_kernel");
  if (kk > kKnnMaxList) {  // passes of kKnnMaxList columns, the last one narrower
    for (int col0 = 0; col0 < kk; col0 += kKnnMaxList) {
      const int width = kk - col0 < kKnnMaxList ? kk - col0 : kKnnMaxList;
      rc = width <= 32 ? launch_knn<32>(query, Nq, source, Ns, ptr_q, ptr_s, tiles, B, kk, out_idx,
                                        out_dist, st, col0, width)
         : width <= 64 ? launch_knn<64>(query, Nq, source, Ns, ptr_q, ptr_s, tiles, B, kk, out_idx,
                                        out_dist, st, col0, width)
         : width <= 96 ? launch_knn<96>(query, Nq, source, Ns, ptr_q, ptr_s, tiles, B, kk, out_idx,
                                        out_dist, st, col0, width)
                       : launch_knn<128>(query, Nq, source, Ns, ptr_q, ptr_s, tiles, B, kk, out_idx,
                                         out_dist, st, col0, width);
      if (rc) return rc;
    }
    return GEO_OK;
  }
#define GEO_KNN_CASE(KV) \
  if (kk <= KV) return launch_knn<KV>(query, Nq, source, Ns, ptr_q, ptr_s, tiles, B, kk, out_idx, out_dist, st);
  GEO_KNN_CASE(1) GEO_KNN_CASE(2) GEO_KNN_CASE(3) GEO_KNN_CASE(4) GEO_KNN_CASE(5)
  GEO_KNN_CASE(6) GEO_KNN_CASE(7) GEO_KNN_CASE(8) GEO_KNN_CASE(10) GEO_KNN_CASE(12)
  GEO_KNN_CASE(16) GEO_KNN_CASE(24) GEO_KNN_CASE(32) GEO_KNN_CASE(48) GEO_KNN_CASE(64)
  GEO_KNN_CASE(96) GEO_KNN_CASE(128)
#undef GEO_KNN_CASE
  return set_error(GEO_ERR_UNSUPPORTED, "knn: k=%d unsupported", kk);
}
