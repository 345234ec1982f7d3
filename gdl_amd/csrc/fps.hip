// fps.hip — farthest-point sampling for packed point clouds on gfx950.
//
// Replaces fps_kernel<512> (geoembodied/csrc/fps_kernel.cu:40-153) with the semantics of the
// CPU path _fps_iterative_fallback (geoembodied/csrc/__init__.py:600-654): start at the first
// point of the cloud, each step take the LOWEST index attaining max(min squared distance).
//
// Four kernels, chosen by the largest cloud of the batch:
//   bucketed (clouds of up to 8192 points, the common case): one 1024-thread workgroup per
//     cloud, points ordered along a Hilbert cell grid so that each register slot of a wave holds
//     a compact bucket of 64 points; a bucket is only updated when the new centroid can lower
//     one of its distances (an exact test, see below), and the argmax is assembled from cached
//     per-bucket maxima.
//   register (8193 to 16384 points): thread t owns local points t, t+256, ... (PTS of them)
//     with x, y, z and the running min distance in VGPRs; every point is updated every
//     iteration.
//   large (16385 to 196,608 points): the bucket scheme with points sorted along the Hilbert
//     curve in the workspace and bucket records in registers (see its section below).
//   streaming (larger clouds): positions read from HBM/L2 each iteration, running min
//     distance in the workspace.
// Each reduces (distance bits, index) per iteration to one winner with one barrier: a wave max
// of the bits (DPP), the lowest index among the lanes holding it, then either one LDS record per
// wave double-buffered by iteration parity (register, streaming) or one LDS 64-bit atomic max per
// wave on a (distance, index complement) key (bucketed, large).  Squared distances are
// non-negative floats, whose bit patterns order like the values.
#include "radix.hpp"

namespace geo {
namespace {

constexpr int kFpsThreads = 256;
constexpr int kFpsWaves = kFpsThreads / kWave;
constexpr int kFpsLdsPoints = 8192;  // register kernel centroid table: 8192 * 16 B of LDS
constexpr int kFpsBucketThreads = 1024;
constexpr int kFpsStreamThreads = 1024;
constexpr int kFpsStreamWaves = kFpsStreamThreads / kWave;

struct alignas(8) FpsSlot {
  uint32_t dist_bits;
  uint32_t idx;
};

// prepare: clamp k to [0, n], exclusive offsets, total, max cloud, ptr validation.
__global__ __launch_bounds__(kScanThreads) void fps_prepare_kernel(
    const int64_t* __restrict__ ptr, const int64_t* __restrict__ kpb, int64_t k_all, int64_t B,
    int64_t N_total, int64_t* __restrict__ out_ptr, int64_t* __restrict__ info,
    int64_t* __restrict__ info_host) {
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
      k = kpb ? kpb[b] : k_all;  // one k for every cloud when no per-cloud array is given
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
    const int64_t bad = s_bad == kNone ? 0 : static_cast<int64_t>(s_bad);
    out_ptr[B] = carry;
    info[0] = carry;
    info[1] = static_cast<int64_t>(s_max);
    info[2] = bad;
    if (info_host) {  // mapped pinned host copy, read by the host once this kernel has finished
      info_host[0] = carry;
      info_host[1] = static_cast<int64_t>(s_max);
      info_host[2] = bad;
      __threadfence_system();
    }
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
    lds_barrier();  // waves share only LDS in this loop
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

// ------------------------------------------------------------------ bucketed kernel ---
//
// Clouds of up to 8192 points.  The cloud is first ordered along a 16^3 Hilbert cell grid
// (LDS counting sort), so the 64 points a wave holds in one register slot — a bucket — lie
// close together.  Each bucket keeps its bounding box in lane s of six VGPRs and its (max
// min-distance, lowest index attaining it, lane holding that point) as wave-uniform scalars, so
// a wave's best is a few scalar max / compare instructions after an update instead of another
// cross-lane reduction, and an updated bucket is re-reduced only when the point holding its
// maximum fell.  Per iteration the wave tests all its buckets at once (one lane per bucket): with
//   g_a = max(lo_a - c_a, c_a - hi_a, 0),  lb = (g_x*g_x + g_y*g_y) + g_z*g_z
// evaluated with the same fp32 operations as the distance, every rounded operation is monotone,
// so lb <= d(p, c) holds exactly for every point p of the bucket; when lb >= the bucket's max
// min-distance no point of the bucket can change and the bucket is skipped.  Skipping is
// therefore exact; only buckets near the new centroid pay for the update.
constexpr int kCellBits = 4;                  // 16 cells per axis
constexpr int kCells = 1 << (3 * kCellBits);  // 4096

__device__ __forceinline__ uint32_t spread10(uint32_t v) {  // 10 bits -> every third bit
  v &= 0x3ffu;
  v = (v | (v << 16)) & 0x030000ffu;
  v = (v | (v << 8)) & 0x0300f00fu;
  v = (v | (v << 4)) & 0x030c30c3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

// Position of cell (x, y, z) (b <= 10 bits per axis) along the 3-D Hilbert curve: the
// coordinates are brought to the curve's transposed form (J. Skilling, "Programming the Hilbert
// curve", AIP Conf. Proc. 707, 381 (2004): undo the excess work of each level from the top bit
// down, then Gray-decode), and the transposed bits interleaved x, y, z from the most significant.
// Consecutive positions are adjacent cells, so runs of points in this order have smaller boxes
// than runs in Morton order, whose curve jumps between distant cells (C5, 64-point buckets: mean
// box volume 61 against 148, buckets passing the bound test per FPS iteration 11.7 against 21.5).
__device__ __forceinline__ uint32_t hilbert3(uint32_t x, uint32_t y, uint32_t z, int b) {
  uint32_t X[3] = {x, y, z};
  const uint32_t top = 1u << (b - 1);
  for (uint32_t q = top; q > 1; q >>= 1) {
    const uint32_t p = q - 1;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (X[i] & q) {
        X[0] ^= p;
      } else {
        const uint32_t t = (X[0] ^ X[i]) & p;
        X[0] ^= t;
        X[i] ^= t;
      }
    }
  }
  X[1] ^= X[0];
  X[2] ^= X[1];
  uint32_t t = 0;
  for (uint32_t q = top; q > 1; q >>= 1)
    if (X[2] & q) t ^= q - 1;
  return (spread10(X[0] ^ t) << 2) | (spread10(X[1] ^ t) << 1) | spread10(X[2] ^ t);
}

__device__ __forceinline__ int cell16(float p, float lo, float scale) {
  int c = static_cast<int>((p - lo) * scale);
  return c < 0 ? 0 : (c > 15 ? 15 : c);
}


// order[q] = local index of the cloud's q-th point along the Hilbert curve of a 16^3 cell grid
// over the cloud's bounding box (LDS counting sort by cell; the order within a cell follows the
// atomics, which only changes which bucket a point joins, never a result).  hist holds kCells
// ints, red 6 x (THREADS / 64) words, code_rank 8 n and order 4 n bytes; ends behind a barrier.
template <int THREADS>
__device__ void fps_hilbert_order(const float* __restrict__ P, int n, int* hist,
                                  uint32_t (*red)[THREADS / kWave], int2* code_rank, int* order) {
  constexpr int WAVES = THREADS / kWave;
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  // 1. bounding box of the cloud
  {
    uint32_t mn[3] = {~0u, ~0u, ~0u}, mx[3] = {0u, 0u, 0u};
    for (int i = t; i < n; i += THREADS) {
#pragma unroll
      for (int a = 0; a < 3; ++a) {
        const uint32_t kk = float_order_key(P[3 * i + a]);
        mn[a] = min(mn[a], kk);
        mx[a] = max(mx[a], kk);
      }
    }
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      mn[a] = wave_min_u32(mn[a]);
      mx[a] = wave_max_u32(mx[a]);
    }
    if (lane == 0) {
#pragma unroll
      for (int a = 0; a < 3; ++a) { red[a][w] = mn[a]; red[3 + a][w] = mx[a]; }
    }
    for (int i = t; i < kCells; i += THREADS) hist[i] = 0;
    __syncthreads();
  }
  float lo[3], scale[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    uint32_t m0 = red[a][0], m1 = red[3 + a][0];
    for (int ww = 1; ww < WAVES; ++ww) { m0 = min(m0, red[a][ww]); m1 = max(m1, red[3 + a][ww]); }
    lo[a] = float_from_order_key(m0);
    const float ext = float_from_order_key(m1) - lo[a];
    scale[a] = ext > 0.f ? 16.f / ext : 0.f;
  }

  // 2. counting sort by Hilbert cell: int2 (code, rank) per point, then the order
  for (int i = t; i < n; i += THREADS) {
    const int cx = cell16(P[3 * i], lo[0], scale[0]);
    const int cy = cell16(P[3 * i + 1], lo[1], scale[1]);
    const int cz = cell16(P[3 * i + 2], lo[2], scale[2]);
    const int code = static_cast<int>(hilbert3(cx, cy, cz, kCellBits));
    code_rank[i] = make_int2(code, atomicAdd(&hist[code], 1));
  }
  __syncthreads();
  {  // exclusive scan of hist in place: thread t owns kCells / THREADS consecutive cells
    constexpr int PER = kCells / THREADS;
    int v[PER], s = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) { v[j] = hist[t * PER + j]; s += v[j]; }
    const int incl = wave_inclusive_sum_int(s);
    __syncthreads();
    if (lane == kWave - 1) red[0][w] = static_cast<uint32_t>(incl);
    __syncthreads();
    int off = incl - s;
    for (int ww = 0; ww < w; ++ww) off += static_cast<int>(red[0][ww]);
#pragma unroll
    for (int j = 0; j < PER; ++j) { hist[t * PER + j] = off; off += v[j]; }
  }
  __syncthreads();
  for (int i = t; i < n; i += THREADS) {
    const int2 cr = code_rank[i];
    order[hist[cr.x] + cr.y] = i;
  }
  __syncthreads();
}

template <int PTS, int THREADS>
__global__ __launch_bounds__(THREADS) void fps_bucket_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ ptr,
    const int64_t* __restrict__ out_ptr, int64_t* __restrict__ out_idx,
    const int64_t* __restrict__ guard) {
  constexpr int WAVES = THREADS / kWave;
  static_assert(PTS <= kWave, "one lane per bucket");
  // Launched before the host has seen the prepare kernel's summary: do nothing unless ptr was
  // valid and every cloud fits this variant (the host then launches the right one).
  if (guard != nullptr && (guard[2] != 0 || guard[1] > PTS * THREADS)) return;
  // Cross-wave argmax: one 64-bit LDS atomic max per wave on the key
  //   (it << 45) | (bits << 13) | (8191 - index)
  // so the largest distance wins and, among equal distances, the lowest index (clouds here have
  // at most 8192 points and iterations).  Iteration it uses slot it % 2; the iteration number in
  // the key's top bits makes every key of it larger than any left from it - 2, so no slot is
  // ever cleared; a slot is reused only after the barrier that every reader of its previous
  // round passed first.
  __shared__ unsigned long long slots[2];
  __shared__ int hist[kCells];
  __shared__ uint32_t red[6][WAVES];
  extern __shared__ float4 table[];  // sort scratch (12 B/point), then positions by index

  const int b = blockIdx.x;
  const int64_t start = ptr[b];
  const int n = static_cast<int>(ptr[b + 1] - start);
  const int64_t o0 = out_ptr[b];
  const int k = static_cast<int>(out_ptr[b + 1] - o0);
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  if (k <= 0 || n <= 0) return;
  if (k >= n) {
    for (int i = t; i < n; i += THREADS) out_idx[o0 + i] = start + i;
    return;
  }
  const float* P = pos + start * 3;

  // 1-2. the cloud ordered along the Hilbert curve of its cell grid
  int2* code_rank = reinterpret_cast<int2*>(table);
  int* order = reinterpret_cast<int*>(reinterpret_cast<char*>(table) + 8 * static_cast<size_t>(n));
  fps_hilbert_order<THREADS>(P, n, hist, red, code_rank, order);

  // 3. registers.  Bucket j = 64 consecutive sorted points; wave w owns buckets w, w+WAVES, ...
  //    (neighbouring buckets on different waves, so the buckets near a centroid spread over
  //    the SIMDs); slot s of wave w holds bucket s*WAVES + w.
  float px[PTS], py[PTS], pz[PTS], md[PTS];
  uint32_t oi[PTS];
  // loads at clamped slots, values selected after (a load under `q < n` became a branch and a
  // wait before the next slot's)
#pragma unroll
  for (int s = 0; s < PTS; ++s) {
    const int q = (s * WAVES + w) * kWave + lane;
    const bool in = q < n;
    const int i = order[in ? q : 0];
    const float x = P[3 * i], y = P[3 * i + 1], z = P[3 * i + 2];
    oi[s] = in ? static_cast<uint32_t>(i) : 0xffffffffu;
    px[s] = in ? x : 0.f;
    py[s] = in ? y : 0.f;
    pz[s] = in ? z : 0.f;
    md[s] = in ? __builtin_inff() : 0.f;  // padding: never changes, never wins
  }
  __syncthreads();  // order[] is dead: the scratch becomes the position table
  // every point sits in exactly one slot (order is a permutation of 0..n-1, PTS * THREADS >= n):
  // the table is written from the registers instead of read from memory again
#pragma unroll
  for (int s = 0; s < PTS; ++s)
    if (oi[s] != 0xffffffffu) table[oi[s]] = make_float4(px[s], py[s], pz[s], 0.f);
  if (t < 2) slots[t] = 0ull;

  // 4. bucket records: box in lane s (bucket of slot s); max min-distance bits, lowest index
  //    attaining the max and the lane holding that point as scalars bm[s], bi[s], al[s].
  float blx = __builtin_inff(), bly = __builtin_inff(), blz = __builtin_inff();
  float bhx = -__builtin_inff(), bhy = -__builtin_inff(), bhz = -__builtin_inff();
  uint32_t bmax = 0u;
  // Bucket records are wave-uniform, kept as scalars; bmax (lane s = bucket s) is the per-lane
  // copy of bm the bound test reads.
  uint32_t bm[PTS], bi[PTS], al[PTS];  // al: lane holding the max (lowest index), kWave = unknown
#pragma unroll
  for (int s = 0; s < PTS; ++s) {
    const bool valid = oi[s] != 0xffffffffu;
    const uint32_t l0 = wave_min_u32(valid ? float_order_key(px[s]) : ~0u);
    const uint32_t l1 = wave_min_u32(valid ? float_order_key(py[s]) : ~0u);
    const uint32_t l2 = wave_min_u32(valid ? float_order_key(pz[s]) : ~0u);
    const uint32_t h0 = wave_max_u32(valid ? float_order_key(px[s]) : 0u);
    const uint32_t h1 = wave_max_u32(valid ? float_order_key(py[s]) : 0u);
    const uint32_t h2 = wave_max_u32(valid ? float_order_key(pz[s]) : 0u);
    const uint32_t mi = wave_min_u32(oi[s]);
    bm[s] = mi != 0xffffffffu ? 0x7f800000u : 0u;
    bi[s] = 0xffffffffu;
    al[s] = kWave;
    if (lane == s && mi != 0xffffffffu) {
      blx = float_from_order_key(l0); bly = float_from_order_key(l1); blz = float_from_order_key(l2);
      bhx = float_from_order_key(h0); bhy = float_from_order_key(h1); bhz = float_from_order_key(h2);
      bmax = 0x7f800000u;  // +inf: every bucket takes part in the first update
    }
  }
  float cx = P[0], cy = P[1], cz = P[2];
  if (t == 0) out_idx[o0] = start;
  // The wave's best (bits, index), recomputed only after one of its buckets changed.
  uint32_t wbits = 0u, widx = 0xffffffffu;
  bool dirty = true;
  __syncthreads();

  for (int it = 1; it < k; ++it) {
    float gx, gy, gz;
    {
#pragma clang fp contract(off)
      gx = fmaxf(fmaxf(blx - cx, cx - bhx), 0.f);
      gy = fmaxf(fmaxf(bly - cy, cy - bhy), 0.f);
      gz = fmaxf(fmaxf(blz - cz, cz - bhz), 0.f);
    }
    const float lb = sqdist(gx, gy, gz, 0.f, 0.f, 0.f);
    const uint64_t act = __ballot(__float_as_uint(lb) < bmax);  // bmax = 0 on lanes >= PTS
    if (act) {
#pragma unroll
      for (int s = 0; s < PTS; ++s) {
        if (act & (1ull << s)) {
          // distances are non-negative floats, ordered like their bit patterns: the running
          // minimum is an integer min (no NaN canonicalisation step)
          const float d = sqdist(px[s], py[s], pz[s], cx, cy, cz);
          const uint32_t old = __float_as_uint(md[s]);
          const uint32_t mb = min(__float_as_uint(d), old);
          md[s] = __uint_as_float(mb);
          // Values only fall: while the point holding the bucket's max keeps its value, the
          // record (max, lowest index attaining it) stands.  Most touched buckets end here.
          if (al[s] < static_cast<uint32_t>(kWave) && !((__ballot(mb < old) >> al[s]) & 1ull))
            continue;
          const uint32_t m = wave_max_u32(mb);
          bm[s] = m;
          if (lane == s) bmax = m;
          const uint64_t hit = __ballot(mb == m);
          if ((hit & (hit - 1)) == 0) {  // one lane holds the maximum (distance ties are rare)
            al[s] = static_cast<uint32_t>(__builtin_ctzll(hit));
            bi[s] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(oi[s]), al[s]));
          } else {
            bi[s] = wave_min_u32(mb == m ? oi[s] : 0xffffffffu);
            al[s] = static_cast<uint32_t>(__builtin_ctzll(__ballot(mb == m && oi[s] == bi[s]) | (1ull << 63)));
          }
          dirty = true;
        }
      }
    }
    if (dirty) {
      // wave best: the largest bucket max, then the lowest index among the buckets holding it
      // (all scalars)
      uint32_t wb = 0u;
#pragma unroll
      for (int s = 0; s < PTS; ++s) wb = bm[s] > wb ? bm[s] : wb;
      wbits = wb;
      uint32_t best = 0xffffffffu;
#pragma unroll
      for (int s = 0; s < PTS; ++s) best = (bm[s] == wb && bi[s] < best) ? bi[s] : best;
      widx = best;
      dirty = false;
    }
    // one lane of the wave issues the atomic (the build turns the atomic optimizer off for this
    // file: its single-lane election would add three dependent VALU steps before the barrier)
    if (lane == 0)
      atomicMax(&slots[it & 1], (static_cast<unsigned long long>(it) << 45) |
                                    (static_cast<unsigned long long>(wbits) << 13) |
                                    static_cast<unsigned long long>(8191u - (widx & 8191u)));
    lds_barrier();  // waves share only LDS in this loop
    const uint32_t gidx = 8191u - (static_cast<uint32_t>(slots[it & 1]) & 8191u);
    const float4 c = table[gidx];
    cx = c.x; cy = c.y; cz = c.z;
    if (t == 0) out_idx[o0 + it] = start + gidx;
  }
}

template <int PTS, int THREADS>
int launch_bucket(const float* pos, const int64_t* ptr, const int64_t* out_ptr, int64_t B,
                  int64_t max_cloud, int64_t* out, hipStream_t st,
                  const int64_t* guard = nullptr) {
  const size_t lds = static_cast<size_t>(max_cloud > 0 ? max_cloud : 1) * sizeof(float4);
  GEO_HIP_CHECK(hipFuncSetAttribute(
      reinterpret_cast<const void*>(&fps_bucket_kernel<PTS, THREADS>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kFpsLdsPoints * sizeof(float4))));
  hipLaunchKernelGGL((fps_bucket_kernel<PTS, THREADS>), dim3(B), dim3(THREADS), lds, st, pos, ptr,
                     out_ptr, out, guard);
  GEO_LAUNCH_CHECK("fps_bucket_kernel");
  return GEO_OK;
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
    lds_barrier();  // each thread reads back only its own M entries: waves share only LDS
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

// ---------------------------------------------------------------------------- large clouds ---
// Clouds larger than the register kernel holds (up to kFpsLargeMaxPoints).  The batch is
// reordered by a device radix sort on (cloud + 1, Hilbert position of the point in its cloud's
// box), which keeps every cloud on its own index range, and each cloud is cut into buckets of 64
// consecutive sorted points.  Positions (with the original index) and running min distances
// stay in the workspace, 20 bytes per point, which for one cloud fits the L2 of the XCD that
// runs it.  One 1024-thread workgroup per cloud; lane l of wave w holds the records of buckets
// w + 16 (l + 64 r), r < kFpsLargeSlots: box, max min-distance, lowest index attaining it, the
// lane of that point and its position.  Per iteration each wave tests its buckets with the exact
// lower bound above, reloads and updates only the buckets the new centroid can change (two at a
// time, so their loads overlap), re-reduces a bucket's record only when the point holding its
// maximum fell (C5: 12% of touched buckets), rescans its best (distance, index) only when the
// bucket that best came from changed (about one wave per iteration: the winner's), and the
// workgroup agrees on the winner with one LDS 64-bit atomic max per wave on
// (bits << 32) | (index complement << 4 | wave) and one LDS-only barrier.
constexpr int kFpsLargeThreads = 1024;
constexpr int kFpsLargeWaves = kFpsLargeThreads / kWave;
constexpr int kFpsLargeSlots = 3;
constexpr int64_t kFpsLargeMaxPoints =
    static_cast<int64_t>(kFpsLargeSlots) * kFpsLargeThreads * kWave;  // 196,608
constexpr uint32_t kFpsLargeIdxMask = (1u << 18) - 1;                  // local index < 2^18
constexpr int64_t kFpsLargeMaxClouds = (1 << 11) - 2;                  // cloud id + 1 in 11 bits

// bbox[6 b .. 6 b + 5] = (lo x, lo y, lo z, hi x, hi y, hi z) of cloud b; one block per cloud.
__global__ __launch_bounds__(kFpsLargeThreads) void fps_large_bbox_kernel(
    const float* __restrict__ pos, const int64_t* __restrict__ ptr, float* __restrict__ bbox) {
  __shared__ uint32_t red[6][kFpsLargeWaves];
  const int b = blockIdx.x;
  const int64_t s = ptr[b], e = ptr[b + 1];
  const int t = threadIdx.x, w = t / kWave;
  uint32_t mn[3] = {~0u, ~0u, ~0u}, mx[3] = {0u, 0u, 0u};
  for (int64_t i = s + t; i < e; i += kFpsLargeThreads) {
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const uint32_t kk = float_order_key(pos[3 * i + a]);
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
    for (int ww = 1; ww < kFpsLargeWaves; ++ww) v = t < 3 ? min(v, red[t][ww]) : max(v, red[t][ww]);
    bbox[6 * b + t] = (e > s) ? float_from_order_key(v) : 0.f;
  }
}

// keys[i] = (cloud + 1) << 3 mbits | Hilbert position (mbits per axis) of point i in its cloud's
// box; points before the first cloud get cloud field 0, points after the last B + 1.
__global__ void fps_large_keys_kernel(const float* __restrict__ pos, const int64_t* __restrict__ ptr,
                                      int64_t B, int64_t N, const float* __restrict__ bbox,
                                      int mbits, uint32_t* __restrict__ keys) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= N) return;
  int64_t lo = 0, hi = B + 1;  // number of ptr entries <= i
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ptr[mid] <= i) lo = mid + 1; else hi = mid;
  }
  uint32_t code = 0;
  if (lo >= 1 && lo <= B) {
    const float* bb = bbox + 6 * (lo - 1);
    const float cells = static_cast<float>(1 << mbits);
    uint32_t c[3];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const float ext = bb[3 + a] - bb[a];
      const float q = ext > 0.f ? (pos[3 * i + a] - bb[a]) * (cells / ext) : 0.f;
      const int ci = static_cast<int>(q);
      c[a] = static_cast<uint32_t>(ci < 0 ? 0 : (ci >= (1 << mbits) ? (1 << mbits) - 1 : ci));
    }
    code = hilbert3(c[0], c[1], c[2], mbits);
  }
  keys[i] = (static_cast<uint32_t>(lo) << (3 * mbits)) | code;
}

// Sorted position j <- original point order[j]: (x, y, z, original index bits); md = +inf.
__global__ void fps_large_gather_kernel(const float* __restrict__ pos,
                                        const uint32_t* __restrict__ order, int64_t N,
                                        float4* __restrict__ q, float* __restrict__ md) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= N) return;
  const uint32_t i = order[j];
  q[j] = make_float4(pos[3 * static_cast<int64_t>(i)], pos[3 * static_cast<int64_t>(i) + 1],
                     pos[3 * static_cast<int64_t>(i) + 2], __uint_as_float(i));
  md[j] = __builtin_inff();
}

__global__ __launch_bounds__(kFpsLargeThreads) void fps_large_kernel(
    const float* __restrict__ pos, const float4* __restrict__ Qall, float* __restrict__ Mall,
    const int64_t* __restrict__ ptr, const int64_t* __restrict__ out_ptr,
    int64_t* __restrict__ out_idx) {
  constexpr int S = kFpsLargeSlots;
  __shared__ unsigned long long slots[3];
  __shared__ float4 cand[2][kFpsLargeWaves];
  const int b = blockIdx.x;
  const int64_t start = ptr[b];
  const int n = static_cast<int>(ptr[b + 1] - start);
  const int64_t o0 = out_ptr[b];
  const int k = static_cast<int>(out_ptr[b + 1] - o0);
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  if (k <= 0 || n <= 0) return;
  if (k >= n) {
    for (int i = t; i < n; i += kFpsLargeThreads) out_idx[o0 + i] = start + i;
    return;
  }
  const float4* Q = Qall + start;
  float* M = Mall + start;
  const int nb = (n + kWave - 1) / kWave;
  const uint32_t ustart = static_cast<uint32_t>(start);

  // Bucket records of this lane (empty buckets: +inf box, max 0, never tested or chosen).
  float blx[S], bly[S], blz[S], bhx[S], bhy[S], bhz[S], bcx[S], bcy[S], bcz[S];
  uint32_t bmax[S], bidx[S], blane[S];  // blane: lane (point) holding the max, 64 = unknown
#pragma unroll
  for (int r = 0; r < S; ++r) {
    blane[r] = kWave;
    blx[r] = bly[r] = blz[r] = __builtin_inff();
    bhx[r] = bhy[r] = bhz[r] = -__builtin_inff();
    bcx[r] = bcy[r] = bcz[r] = 0.f;
    bmax[r] = 0u;
    bidx[r] = 0xffffffffu;
    const int bk = w + kFpsLargeWaves * (lane + kWave * r);
    if (bk < nb) {
      const int q0 = bk * kWave;
      const int q1 = min(q0 + kWave, n);
#pragma unroll 8
      for (int q = q0; q < q1; ++q) {
        const float4 p = Q[q];
        blx[r] = fminf(blx[r], p.x); bly[r] = fminf(bly[r], p.y); blz[r] = fminf(blz[r], p.z);
        bhx[r] = fmaxf(bhx[r], p.x); bhy[r] = fmaxf(bhy[r], p.y); bhz[r] = fmaxf(bhz[r], p.z);
        const uint32_t li = __float_as_uint(p.w) - ustart;
        if (li < bidx[r]) { bidx[r] = li; bcx[r] = p.x; bcy[r] = p.y; bcz[r] = p.z; }
      }
      bmax[r] = 0x7f800000u;  // +inf: every bucket takes part in the first update
    }
  }
  float cx = pos[3 * start], cy = pos[3 * start + 1], cz = pos[3 * start + 2];
  if (t == 0) {
    out_idx[o0] = start;
    slots[0] = slots[1] = slots[2] = 0ull;
  }
  unsigned long long best_key = 0ull;
  float4 best_c = make_float4(0.f, 0.f, 0.f, 0.f);
  bool dirty = true;
  int best_r = -1, best_l = 0;  // the bucket the wave's best record comes from (slot, lane)
  __syncthreads();

  // slots that hold buckets at all: slot r holds buckets [1024 r, 1024 (r + 1)); the others are
  // neither tested nor searched
  const int s_used = (nb + kFpsLargeThreads - 1) / kFpsLargeThreads;

  for (int it = 1; it < k; ++it) {
    uint64_t act[S];
#pragma unroll
    for (int r = 0; r < S; ++r) {
      act[r] = 0ull;
      if (r < s_used) {  // wave-uniform
        float gx, gy, gz;
        {
#pragma clang fp contract(off)
          gx = fmaxf(fmaxf(blx[r] - cx, cx - bhx[r]), 0.f);
          gy = fmaxf(fmaxf(bly[r] - cy, cy - bhy[r]), 0.f);
          gz = fmaxf(fmaxf(blz[r] - cz, cz - bhz[r]), 0.f);
        }
        const float lb = sqdist(gx, gy, gz, 0.f, 0.f, 0.f);
        act[r] = __ballot(__float_as_uint(lb) < bmax[r]);
      }
    }
    while (act[0] | act[1] | act[2]) {
      // up to two affected buckets of this wave per round, their loads issued together (C5:
      // two per round 27.3 ms, three 27.4, four 28.8: fewer rounds for the busiest wave, but
      // every slot of a round costs its selection, address and bookkeeping)
      constexpr int G = 2;
      int rr[G], ll[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        rr[j] = act[0] ? 0 : (act[1] ? 1 : (act[2] ? 2 : -1));
        ll[j] = 0;
        if (rr[j] >= 0) {
          const uint64_t m = rr[j] == 0 ? act[0] : (rr[j] == 1 ? act[1] : act[2]);
          ll[j] = __builtin_ctzll(m);
          const uint64_t cleared = m & (m - 1);
          if (rr[j] == 0) act[0] = cleared; else if (rr[j] == 1) act[1] = cleared; else act[2] = cleared;
        }
      }
      float4 p[G];
      float mo[G];
      bool v[G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const int q = (w + kFpsLargeWaves * (ll[j] + kWave * (rr[j] < 0 ? 0 : rr[j]))) * kWave + lane;
        v[j] = rr[j] >= 0 && q < n;
        p[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        mo[j] = 0.f;
        if (rr[j] >= 0) {  // wave-uniform: no load left in flight for an unused slot
          p[j] = Q[v[j] ? q : 0];
          mo[j] = M[v[j] ? q : 0];
        }
      }
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (rr[j] < 0) continue;  // wave-uniform
        const int q = (w + kFpsLargeWaves * (ll[j] + kWave * rr[j])) * kWave + lane;
        const float d = sqdist(p[j].x, p[j].y, p[j].z, cx, cy, cz);
        const float m = __builtin_amdgcn_fmed3f(d, mo[j], -__builtin_inff());
        const bool fell = v[j] && m < mo[j];
        if (fell) M[q] = m;
        // Values only fall, so while the point holding the bucket's maximum keeps its value the
        // record (max, lowest index attaining it) stands: no other point can reach the max, and
        // points tied with it have higher indices.  Most touched buckets end here.
        const uint32_t al = static_cast<uint32_t>(__builtin_amdgcn_readlane(
            static_cast<int>(rr[j] == 0 ? blane[0] : (rr[j] == 1 ? blane[1] : blane[2])), ll[j]));
        if (al < static_cast<uint32_t>(kWave) && !((__ballot(fell) >> al) & 1ull)) continue;
        const uint32_t bits = v[j] ? __float_as_uint(m) : 0u;
        const uint32_t bm = wave_max_u32(bits);
        const uint32_t li = __float_as_uint(p[j].w) - ustart;
        const uint64_t at = __ballot(v[j] && bits == bm);
        uint32_t ii;
        int sl;
        if (__builtin_popcountll(at) == 1) {  // wave-uniform; the usual case: one lane attains it
          sl = __builtin_ctzll(at);
          ii = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(li), sl));
        } else {  // ties: the lowest index among them
          ii = wave_min_u32(v[j] && bits == bm ? li : 0xffffffffu);
          sl = __builtin_ctzll(__ballot(v[j] && bits == bm && li == ii) | (1ull << 63));
        }
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[j].x), sl));
        const float y = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[j].y), sl));
        const float z = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[j].z), sl));
        if (lane == ll[j]) {
          if (rr[j] == 0) {
            bmax[0] = bm; bidx[0] = ii; blane[0] = sl; bcx[0] = x; bcy[0] = y; bcz[0] = z;
          } else if (rr[j] == 1) {
            bmax[1] = bm; bidx[1] = ii; blane[1] = sl; bcx[1] = x; bcy[1] = y; bcz[1] = z;
          } else {
            bmax[2] = bm; bidx[2] = ii; blane[2] = sl; bcx[2] = x; bcy[2] = y; bcz[2] = z;
          }
        }
        // a record's key (max, then lower index) never rises, so only a change of the bucket the
        // wave's best came from can change the wave's best
        if (rr[j] == best_r && ll[j] == best_l) dirty = true;
      }
    }
    if (dirty) {  // the wave's best record: largest max, then lowest index
      uint32_t m3 = 0u;
#pragma unroll
      for (int r = 0; r < S; ++r) m3 = max(m3, bmax[r]);
      const uint32_t wh = wave_max_u32(m3);
      uint64_t e[S];
      int cnt = 0;
#pragma unroll
      for (int r = 0; r < S; ++r) {
        e[r] = __ballot(bmax[r] == wh && bidx[r] != 0xffffffffu);
        cnt += __builtin_popcountll(e[r]);
      }
      if (cnt != 1) {  // wave-uniform: ties (or no bucket at all): the lowest index among them
        uint32_t li = 0xffffffffu;
#pragma unroll
        for (int r = 0; r < S; ++r) li = bmax[r] == wh ? min(li, bidx[r]) : li;
        const uint32_t mi = wave_min_u32(li);
#pragma unroll
        for (int r = 0; r < S; ++r) e[r] = __ballot(bmax[r] == wh && bidx[r] == mi && mi != 0xffffffffu);
      }
      const int rs = e[0] ? 0 : (e[1] ? 1 : (e[2] ? 2 : -1));
      best_r = rs;
      if (rs < 0) {  // a wave without buckets never wins
        best_key = 0ull;
      } else {
        const int ls = __builtin_ctzll(rs == 0 ? e[0] : (rs == 1 ? e[1] : e[2]));
        best_l = ls;
        uint32_t bi;
        float ex, ey, ez;
        if (rs == 0) {
          bi = bidx[0]; ex = bcx[0]; ey = bcy[0]; ez = bcz[0];
        } else if (rs == 1) {
          bi = bidx[1]; ex = bcx[1]; ey = bcy[1]; ez = bcz[1];
        } else {
          bi = bidx[2]; ex = bcx[2]; ey = bcy[2]; ez = bcz[2];
        }
        bi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bi), ls));
        best_key = (static_cast<unsigned long long>(wh) << 32) |
                   (((kFpsLargeIdxMask - bi) << 4) | static_cast<uint32_t>(w));
        best_c = make_float4(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), ls)),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ey), ls)),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ez), ls)), 0.f);
      }
      dirty = false;
    }
    const int ps = it % 3;
    if (lane == 0) {
      cand[it & 1][w] = best_c;
      atomicMax(&slots[ps], best_key);
    }
    if (t == 0) slots[ps == 2 ? 0 : ps + 1] = 0ull;
    lds_barrier();  // each bucket's points are read and written by its own wave only
    const unsigned long long key = slots[ps];
    const uint32_t low = static_cast<uint32_t>(key);
    const float4 c = cand[it & 1][low & 15u];
    cx = c.x; cy = c.y; cz = c.z;
    if (t == 0) out_idx[o0 + it] = start + (kFpsLargeIdxMask - ((low >> 4) & kFpsLargeIdxMask));
  }
}

struct FpsLargeWs {
  float4* q;
  float* md;
  float* bbox;
  uint32_t *keys, *skeys, *order;
  RadixBuffers rx;
};

// Width of the sort keys (cloud + 1, Hilbert position): the cloud field holds 0 .. B + 1 and each
// axis of the Hilbert grid gets the same share of the rest, at most 10 bits.
int fps_large_key_bits(int64_t B, int* axis_bits) {
  int cbits = 0;
  while ((static_cast<uint64_t>(B + 1) >> cbits) != 0) ++cbits;
  int mbits = (32 - cbits) / 3;
  if (mbits > 10) mbits = 10;
  if (axis_bits) *axis_bits = mbits;
  return cbits + 3 * mbits;
}

FpsLargeWs carve_fps_large(void* base, int64_t B, int64_t N, size_t* bytes) {
  Carver c(base);
  FpsLargeWs w;
  w.q = c.take<float4>(N);
  w.md = c.take<float>(N);
  w.bbox = c.take<float>(6 * (B > 0 ? B : 1));
  w.keys = c.take<uint32_t>(N);
  w.skeys = c.take<uint32_t>(N);
  w.order = c.take<uint32_t>(N);
  w.rx = carve_radix(c, N, fps_large_key_bits(B, nullptr));
  *bytes = c.used;
  return w;
}

bool fps_use_large(int64_t B, int64_t max_cloud) {
  return max_cloud > 64 * kFpsThreads && max_cloud <= kFpsLargeMaxPoints && B <= kFpsLargeMaxClouds;
}

int launch_large(const float* pos, int64_t N, const int64_t* ptr, const int64_t* out_ptr,
                 int64_t B, int64_t* out, void* workspace, hipStream_t st) {
  size_t bytes = 0;
  const FpsLargeWs w = carve_fps_large(workspace, B, N, &bytes);
  hipLaunchKernelGGL(fps_large_bbox_kernel, dim3(B), dim3(kFpsLargeThreads), 0, st, pos, ptr, w.bbox);
  GEO_LAUNCH_CHECK("fps_large_bbox_kernel");
  int mbits = 0;
  fps_large_key_bits(B, &mbits);
  const unsigned grid = static_cast<unsigned>(ceil_div(N, 256));
  hipLaunchKernelGGL(fps_large_keys_kernel, dim3(grid), dim3(256), 0, st, pos, ptr, B, N, w.bbox,
                     mbits, w.keys);
  GEO_LAUNCH_CHECK("fps_large_keys_kernel");
  int rc = radix_sort<kRxKeysIota>(w.keys, nullptr, N, 0, w.skeys, w.order, w.rx, st);
  if (rc) return rc;
  hipLaunchKernelGGL(fps_large_gather_kernel, dim3(grid), dim3(256), 0, st, pos, w.order, N, w.q, w.md);
  GEO_LAUNCH_CHECK("fps_large_gather_kernel");
  hipLaunchKernelGGL(fps_large_kernel, dim3(B), dim3(kFpsLargeThreads), 0, st, pos, w.q, w.md, ptr,
                     out_ptr, out);
  GEO_LAUNCH_CHECK("fps_large_kernel");
  return GEO_OK;
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
                     k_per_batch, int64_t{0}, B, N_total, out_ptr, info,
                     static_cast<int64_t*>(nullptr));
  GEO_LAUNCH_CHECK("fps_prepare_kernel");
  return GEO_OK;
}

extern "C" int geo_fps_prepare_uniform(const int64_t* ptr, int64_t k, int64_t B, int64_t N_total,
                                       int64_t* out_ptr, int64_t* info, int64_t* info_host,
                                       void* stream) {
  GEO_REQUIRE(B >= 0 && N_total >= 0, "fps_prepare: negative size");
  GEO_REQUIRE(ptr && out_ptr && info, "fps_prepare: null pointer");
  int64_t* host_dev = nullptr;
  if (info_host) {
    GEO_HIP_CHECK(hipHostGetDevicePointer(reinterpret_cast<void**>(&host_dev), info_host, 0));
    GEO_REQUIRE(host_dev != nullptr, "fps_prepare: info_host is not mapped pinned memory");
  }
  hipLaunchKernelGGL(fps_prepare_kernel, dim3(1), dim3(kScanThreads), 0, as_stream(stream), ptr,
                     static_cast<const int64_t*>(nullptr), k, B, N_total, out_ptr, info, host_dev);
  GEO_LAUNCH_CHECK("fps_prepare_kernel");
  return GEO_OK;
}

extern "C" int geo_fps_guarded(const float* pos, int64_t N_total, const int64_t* ptr,
                               const int64_t* out_ptr, int64_t B, int64_t max_cloud_guess,
                               int64_t* out_idx, const int64_t* info, int64_t* capacity,
                               void* stream) {
  GEO_REQUIRE(capacity != nullptr, "fps_guarded: null capacity");
  *capacity = 0;
  GEO_REQUIRE(B >= 0 && N_total >= 0 && max_cloud_guess >= 0, "fps_guarded: negative size");
  GEO_REQUIRE(N_total < 0x7fffffffLL, "fps: N_total exceeds int32 indexing");
  if (B == 0 || max_cloud_guess == 0 || max_cloud_guess > kFpsLdsPoints) return GEO_OK;
  GEO_REQUIRE(pos && ptr && out_ptr && out_idx && info, "fps_guarded: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t p2 = ceil_div(max_cloud_guess, kFpsBucketThreads);
  const int pts = p2 <= 1 ? 1 : (p2 <= 2 ? 2 : (p2 <= 4 ? 4 : 8));
  const int64_t cap = static_cast<int64_t>(pts) * kFpsBucketThreads;
  int rc;
  switch (pts) {
    case 1: rc = launch_bucket<1, kFpsBucketThreads>(pos, ptr, out_ptr, B, cap, out_idx, st, info); break;
    case 2: rc = launch_bucket<2, kFpsBucketThreads>(pos, ptr, out_ptr, B, cap, out_idx, st, info); break;
    case 4: rc = launch_bucket<4, kFpsBucketThreads>(pos, ptr, out_ptr, B, cap, out_idx, st, info); break;
    default: rc = launch_bucket<8, kFpsBucketThreads>(pos, ptr, out_ptr, B, cap, out_idx, st, info); break;
  }
  if (rc == GEO_OK) *capacity = cap;
  return rc;
}

extern "C" size_t geo_fps_workspace_bytes(int64_t B, int64_t N_total, int64_t max_cloud) {
  if (B < 0 || N_total < 0 || max_cloud < 0) return 0;
  if (fps_use_large(B, max_cloud)) {
    size_t bytes = 0;
    carve_fps_large(nullptr, B, N_total, &bytes);
    return bytes;
  }
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
  if (max_cloud <= kFpsLdsPoints) {
    // 1024 threads: four waves per SIMD hide much of the per-iteration dependency chain.
    const int64_t p2 = ceil_div(max_cloud, kFpsBucketThreads);
    if (p2 <= 1) return launch_bucket<1, kFpsBucketThreads>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
    if (p2 <= 2) return launch_bucket<2, kFpsBucketThreads>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
    if (p2 <= 4) return launch_bucket<4, kFpsBucketThreads>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
    if (p2 <= 8) return launch_bucket<8, kFpsBucketThreads>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
    return launch_bucket<8, kFpsBucketThreads>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  }
  if (per <= 1) return launch_register<1>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 2) return launch_register<2>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 4) return launch_register<4>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 8) return launch_register<8>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 16) return launch_register<16>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 32) return launch_register<32>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (per <= 64) return launch_register<64>(pos, ptr, out_ptr, B, max_cloud, out_idx, st);
  if (fps_use_large(B, max_cloud))
    return launch_large(pos, N_total, ptr, out_ptr, B, out_idx, workspace, st);
  hipLaunchKernelGGL(fps_stream_kernel, dim3(B), dim3(kFpsStreamThreads), 0, st, pos, ptr,
                     out_ptr, out_idx, static_cast<float*>(workspace));
  GEO_LAUNCH_CHECK("fps_stream_kernel");
  return GEO_OK;
}
