// radix.hpp — stable LSD radix sort of (uint32 key, uint32 value) pairs, digits of at most 8
// bits.
//
// A sort of b-bit keys takes ceil(b / 8) passes of near-equal digit width, the wider ones first
// (19-bit CSR keys: 7, 6 and 6 bits).  Digits stay narrow because the scatter's cost grows with
// the digit count: a 4096-key tile writes one run per digit, and runs of 4 keys (10-bit digits)
// cost twice the runs of 64 (6-bit digits) per pass -- three narrow passes are faster than two
// wide ones.  Each pass is three launches over 4096-key tiles:
//   radix_hist     the tile's digit counts -> hist[digit][tile] (LDS histogram; a run of equal
//                  digits in consecutive lanes adds once, so sorted input does not serialise on
//                  one counter)
//   scan_lookback  exclusive scan of hist in digit-major order -> offs[digit][tile], the output
//                  position of the tile's first key of each digit (one launch: its look-back
//                  inspects 64 earlier scan tiles per step)
//   radix_scatter  stable rank inside the tile (per-wave digit ballots), the tile's keys grouped
//                  by digit in LDS, each digit's run written contiguously at its offset
// No kernel waits on another workgroup.  Tiles are handed to the XCDs in contiguous ranges, so
// the runs that neighbouring tiles write into one digit's region of the output meet in one L2.
// The first pass reads the caller's keys in one of three forms (RxSource) and writes uint32
// keys; the value of the first pass is the element index unless values are supplied.
//
// Sorted input (RxDetect): the first histogram also checks the key order.  Tiles in order write
// the identity result (and, for a CSR build, the node bounds of their key transitions) while no
// tile has found a descent; a tile that finds one sets a flag, and every later kernel of the
// sort runs only when that flag is set.  Flags are set with plain stores: a thousand workgroups
// setting one word by atomics serialise on it (~12 us at 4M keys), plain stores do not.
#pragma once

#include "scan.hpp"

namespace geo {
// Internal linkage: every translation unit that includes this header gets its own copy of the
// radix sort kernels and helpers, so no two units can share a definition built differently.
namespace {

constexpr int kRxThreads = 256;
constexpr int kRxItems = 16;
constexpr int kRxTile = kRxThreads * kRxItems;  // keys per tile
constexpr int kRxWaves = kRxThreads / kWave;
constexpr int kRxWaveSpan = kRxItems * kWave;  // keys per wave in a tile
constexpr int kRxMaxBits = 8;                   // widest digit
constexpr int kRxMinBits = 4;                   // narrowest kernel (fewer key bits use it)
constexpr int kRxMaxBins = 1 << kRxMaxBits;
constexpr int kRxMaxPasses = 4;                 // 32-bit keys
// control words: the sorted-input flag and one flag for the caller
constexpr int kRxCtrlUnsorted = 0;
constexpr int kRxCtrlAux = 1;
constexpr int kRxCtrlWords = 2;

enum RxSource {
  kRxCol64 = 0,     // int64 keys, values outside [0, N) become N; value = index
  kRxKeysIota = 1,  // uint32 keys; value = index
  kRxPairs = 2,     // uint32 keys and uint32 values
};

// Digit layout of a sort of key_bits-bit keys.
struct RxPlan {
  int passes;
  int bits[kRxMaxPasses];
  int shift[kRxMaxPasses];
  int max_bits;
};

__host__ __device__ inline RxPlan rx_plan(int key_bits) {
  key_bits = key_bits < 1 ? 1 : (key_bits > 32 ? 32 : key_bits);
  RxPlan p;
  p.passes = (key_bits + kRxMaxBits - 1) / kRxMaxBits;
  p.max_bits = 0;
  int shift = 0;
  for (int i = 0; i < kRxMaxPasses; ++i) {
    if (i < p.passes) {
      const int left = key_bits - shift;
      const int bits = (left + (p.passes - i) - 1) / (p.passes - i);
      p.bits[i] = bits;
      p.shift[i] = shift;
      shift += bits;
      p.max_bits = bits > p.max_bits ? bits : p.max_bits;
    } else {
      p.bits[i] = 0;
      p.shift[i] = 0;
    }
  }
  // a pass narrower than kRxMinBits runs the kRxMinBits kernel: it is the last pass (widths do
  // not grow), so the extra digit bits are key bits above the key width, all zero
  if (p.max_bits < kRxMinBits) p.max_bits = kRxMinBits;
  return p;
}

// Workgroups of a scatter or histogram launch: as many as are resident at once on 256 CUs (four
// per CU: ~120 VGPRs and up to 37 KB of LDS each).
constexpr int64_t kRxGrid = 1024;

template <int SRC>
__device__ __forceinline__ uint32_t rx_fetch_key(const void* keys, int64_t i, int64_t N) {
  if constexpr (SRC == kRxCol64) {
    const int64_t c = static_cast<const int64_t*>(keys)[i];
    return (c >= 0 && c < N) ? static_cast<uint32_t>(c) : static_cast<uint32_t>(N);
  } else {
    return static_cast<const uint32_t*>(keys)[i];
  }
}

// Lanes of the wave whose (valid) digit equals this lane's digit.
template <int BITS>
__device__ __forceinline__ uint64_t rx_peers(uint32_t d, bool valid) {
  uint64_t peers = __ballot(valid);
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bb = __ballot(bit);
    peers &= bit ? bb : ~bb;
  }
  return peers;
}

// Adds one to h[d] for every valid lane; a run of equal digits in consecutive lanes adds once.
__device__ __forceinline__ void rx_count_runs(uint32_t* h, uint32_t d, bool valid, int lane) {
  const uint32_t dd = valid ? d : 0xffffffffu;
  const uint32_t prev = __shfl_up(dd, 1, kWave);
  const bool start = lane == 0 || prev != dd;
  const uint64_t starts = __ballot(start);
  if (valid && start) {
    const uint64_t later = lane == kWave - 1 ? 0ull : (starts & (~0ull << (lane + 1)));
    const int next = later ? __builtin_ctzll(later) : kWave;
    atomicAdd(&h[d], static_cast<uint32_t>(next - lane));
  }
}

// Tiles [first, last) of this workgroup: contiguous, balanced ranges in XCD order (the
// workgroups an XCD runs get neighbouring ranges).
__device__ __forceinline__ void rx_tiles(int64_t ntiles, int64_t& first, int64_t& last) {
  const int64_t G = gridDim.x;
  const int64_t xb = xcd_block();
  const int64_t per = ntiles / G, extra = ntiles % G;
  first = xb * per + (xb < extra ? xb : extra);
  last = first + per + (xb < extra ? 1 : 0);
}

// Node bounds from sorted keys.  lb(n), the first sorted position with key >= n, is
// node_start[n] (n < nodes) and node_end[n - 1] (n >= 1); position "number of keys" counts as
// key `nodes`.  A wave handles the positions of its span p0 .. p0 + cnt - 1, whose keys it has
// staged in LDS (s_keys[0 .. cnt), ascending): lb(n) lies in the span exactly for the n in
// (before, last], `before` being the key at p0 - 1 (-1 at p0 = 0) and `last` = s_keys[cnt - 1].
// Lanes take those nodes 64 apart (consecutive nodes, so the stores are coalesced) and find
// lb(n) by binary search in LDS.  A span covering more than kRxBoundsMax nodes (nodes far
// sparser than the keys) writes nothing and returns false: the caller then has every bound
// computed by binary search over the whole key array instead, so no wave's work grows with the
// node count.
constexpr int64_t kRxBoundsMax = 64 * kWave;

__device__ bool rx_wave_bounds(const uint32_t* s_keys, int cnt, int64_t p0, int64_t before,
                               int64_t last, int32_t* __restrict__ node_start,
                               int32_t* __restrict__ node_end, int64_t nodes) {
  const int64_t span = last - before;
  if (span <= 0) return true;
  if (span > kRxBoundsMax) return false;
  for (int64_t j = lane_id(); j < span; j += kWave) {
    const int64_t n = before + 1 + j;
    int lo = 0, hi = cnt;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (static_cast<int64_t>(s_keys[mid]) < n) lo = mid + 1; else hi = mid;
    }
    const int32_t pos = static_cast<int32_t>(p0 + lo);
    if (n < nodes) node_start[n] = pos;
    if (n > 0) node_end[n - 1] = pos;
  }
  return true;
}

// lb(n) = pos for the n in (lo, hi] (the nodes after the last key, whose lower bound is the end
// position); false, writing nothing, beyond kRxBoundsMax nodes.
__device__ bool rx_fill_bounds(int64_t lo, int64_t hi, int32_t pos, int32_t* __restrict__ node_start,
                               int32_t* __restrict__ node_end, int64_t nodes) {
  const int64_t span = hi - lo;
  if (span <= 0) return true;
  if (span > kRxBoundsMax) return false;
  for (int64_t j = lane_id(); j < span; j += kWave) {
    const int64_t n = lo + 1 + j;
    if (n < nodes) node_start[n] = pos;
    if (n > 0) node_end[n - 1] = pos;
  }
  return true;
}

// Sorted-input detection of a sort's first pass.
struct RxDetect {
  uint32_t* unsorted = nullptr;   // set by a tile that finds a key below its predecessor
  uint32_t* keys_out = nullptr;   // identity result, written by in-order tiles
  uint32_t* vals_out = nullptr;
  int32_t* node_start = nullptr;  // optional: node bounds of the in-order tiles' transitions
  int32_t* node_end = nullptr;
  int64_t nodes = 0;
  uint32_t* fallback = nullptr;   // set when a wave leaves long gaps unwritten
};

// Digit counts of each tile of the pass at `shift` -> hist[d * ntiles + tile].  With `active`,
// does nothing when it reads 0.  With det.unsorted (first pass only), also the order check and
// the identity result of in-order tiles (see the header).
template <int SRC, int BITS>
__global__ __launch_bounds__(kRxThreads) void radix_hist(const void* __restrict__ keys, int64_t n,
                                                         int64_t N, int shift,
                                                         uint32_t* __restrict__ hist,
                                                         int64_t ntiles,
                                                         const uint32_t* __restrict__ active,
                                                         RxDetect det) {
  if (active != nullptr && *active == 0u) return;
  constexpr int BINS = 1 << BITS;
  __shared__ uint32_t h[BINS];
  __shared__ uint32_t s_keys[kRxWaves][kRxWaveSpan];  // a sorted tile's keys, for its node bounds
  __shared__ uint32_t s_down, s_check;
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  int64_t first, last;
  rx_tiles(ntiles, first, last);
  for (int64_t tile = first; tile < last; ++tile) {
    for (int b = t; b < BINS; b += kRxThreads) h[b] = 0;
    if (t == 0) {
      s_down = 0u;
      // once some tile has found the input out of order, the others skip the check
      s_check = det.unsorted != nullptr &&
                __hip_atomic_load(det.unsorted, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u;
    }
    const int64_t wbase = tile * kRxTile + static_cast<int64_t>(w) * kRxWaveSpan;
    uint32_t key[kRxItems];
    // loads at clamped positions, values selected after: a load under a per-lane condition
    // became a branch and a wait before the next load
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      key[i] = rx_fetch_key<SRC>(keys, idx < n ? idx : n - 1, N);
    }
#pragma unroll
    for (int i = 0; i < kRxItems; ++i)
      key[i] = wbase + static_cast<int64_t>(i) * kWave + lane < n ? key[i] : 0u;
    uint32_t before = 0u;  // key preceding the wave's range
    if (det.unsorted != nullptr && lane == 0 && wbase > 0 && wbase < n)
      before = rx_fetch_key<SRC>(keys, wbase - 1, N);
    __syncthreads();
    const bool check = s_check != 0u;  // workgroup-uniform
    bool down = false;
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      const bool valid = idx < n;
      if (check) {  // lane 0's predecessor is lane 63's key of the previous item (or `before`)
        uint32_t pk = __shfl_up(key[i], 1, kWave);
        if (i > 0) {
          const uint32_t lastk = __shfl(key[i > 0 ? i - 1 : 0], kWave - 1, kWave);
          if (lane == 0) pk = lastk;
        } else if (lane == 0) {
          pk = before;
        }
        down |= valid && idx > 0 && pk > key[i];
      }
      rx_count_runs(h, (key[i] >> shift) & (BINS - 1u), valid, lane);
    }
    if (down) s_down = 1u;
    __syncthreads();
    for (int b = t; b < BINS; b += kRxThreads) hist[static_cast<int64_t>(b) * ntiles + tile] = h[b];
    if (check) {
      if (s_down != 0u) {
        if (t == 0) *det.unsorted = 1u;
      } else {
#pragma unroll
        for (int i = 0; i < kRxItems; ++i) {
          const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
          if (idx < n) {
            det.keys_out[idx] = key[i];
            det.vals_out[idx] = static_cast<uint32_t>(idx);
          }
        }
        if (det.node_start != nullptr && wbase < n) {  // wave-uniform
#pragma unroll
          for (int i = 0; i < kRxItems; ++i) s_keys[w][i * kWave + lane] = key[i];
          wave_lds_fence();
          const int cnt = static_cast<int>(min(static_cast<int64_t>(kRxWaveSpan), n - wbase));
          const int64_t lastk = s_keys[w][cnt - 1];
          const int64_t bk = wbase > 0 ? static_cast<int64_t>(__builtin_amdgcn_readlane(before, 0)) : -1;
          bool ok = rx_wave_bounds(s_keys[w], cnt, wbase, bk, lastk, det.node_start, det.node_end,
                                   det.nodes);
          if (wbase + cnt == n)  // the nodes after the last key: lower bound n
            ok &= rx_fill_bounds(lastk, det.nodes, static_cast<int32_t>(n), det.node_start,
                                 det.node_end, det.nodes);
          if (!ok && lane == 0) *det.fallback = 1u;
        }
      }
    }
    __syncthreads();  // the next tile reuses h and s_down
  }
}

// Block-wide exclusive scan of per-thread sums (kRxThreads threads); `lds` holds kRxWaves words.
__device__ __forceinline__ uint32_t rx_block_excl(uint32_t v, uint32_t* lds, int w, int lane) {
  const uint32_t inc = wave_inclusive_sum_dpp(v);
  if (lane == kWave - 1) lds[w] = inc;
  __syncthreads();
  uint32_t off = inc - v;
#pragma unroll
  for (int ww = 0; ww < kRxWaves; ++ww)
    if (ww < w) off += lds[ww];
  __syncthreads();
  return off;
}

// One pass: keys_out / vals_out receive the pass's input stably sorted by the digit at `shift`.
// offs[d * ntiles + tile] is the output position of the tile's first key of digit d.  With
// `active`, does nothing when it reads 0.
template <int SRC, int BITS>
__global__ __launch_bounds__(kRxThreads) void radix_scatter(
    const void* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n, int64_t N,
    int shift, const uint32_t* __restrict__ offs, int64_t ntiles, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, const uint32_t* __restrict__ active) {
  if (active != nullptr && *active == 0u) return;
  constexpr int BINS = 1 << BITS;
  static_assert(BINS <= kRxThreads, "one digit per thread");
  __shared__ uint32_t cnt[kRxWaves][BINS];  // per-wave digit counts, then tile offsets
  __shared__ uint32_t s_goff[BINS];         // offs[d] minus the tile offset of digit d
  __shared__ uint32_t s_key[kRxTile];
  __shared__ uint32_t s_val[kRxTile];
  __shared__ uint32_t s_scan[kRxWaves];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = lane_id();
  const uint64_t lt = lanemask_lt();
  const bool owner = t < BINS;  // thread t owns digit t
  int64_t first, last;
  rx_tiles(ntiles, first, last);
  for (int64_t tile = first; tile < last; ++tile) {
    // requested first: the ranking below hides the latency
    const uint32_t goff = owner ? offs[static_cast<int64_t>(t) * ntiles + tile] : 0u;
    if (owner)
#pragma unroll
      for (int ww = 0; ww < kRxWaves; ++ww) cnt[ww][t] = 0;
    const int64_t wbase = tile * kRxTile + static_cast<int64_t>(w) * kRxWaveSpan;
    uint32_t key[kRxItems], val[kRxItems], rank[kRxItems];
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {  // clamped, unconditional loads (as in radix_hist)
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      const int64_t ic = idx < n ? idx : n - 1;
      key[i] = rx_fetch_key<SRC>(keys_in, ic, N);
      if constexpr (SRC == kRxPairs) {
        val[i] = vals_in[ic];
      } else {
        val[i] = static_cast<uint32_t>(idx);
      }
    }
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const bool valid = wbase + static_cast<int64_t>(i) * kWave + lane < n;
      key[i] = valid ? key[i] : 0u;
      if constexpr (SRC == kRxPairs) val[i] = valid ? val[i] : 0u;
    }
    __syncthreads();
    // stable rank among the wave's keys of the same digit, in (item, lane) = index order
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      const bool valid = idx < n;
      const uint32_t d = (key[i] >> shift) & (BINS - 1u);
      const uint64_t peers = rx_peers<BITS>(d, valid);
      const uint32_t before = cnt[w][d];
      __builtin_amdgcn_wave_barrier();
      if (valid && (peers & lt) == 0ull) cnt[w][d] = before + static_cast<uint32_t>(__popcll(peers));
      __builtin_amdgcn_wave_barrier();
      rank[i] = before + static_cast<uint32_t>(__popcll(peers & lt));
    }
    __syncthreads();
    // digit t: tile total, tile offset (exclusive scan over the digits), per-wave offsets
    uint32_t wc[kRxWaves];
    uint32_t tsum = 0;
#pragma unroll
    for (int ww = 0; ww < kRxWaves; ++ww) {
      wc[ww] = owner ? cnt[ww][t] : 0u;
      tsum += wc[ww];
    }
    uint32_t toff = rx_block_excl(tsum, s_scan, w, lane);
    if (owner) {
      s_goff[t] = goff - toff;
#pragma unroll
      for (int ww = 0; ww < kRxWaves; ++ww) {
        cnt[ww][t] = toff;
        toff += wc[ww];
      }
    }
    __syncthreads();
    // group the tile's keys by digit in LDS (stable), then write each digit's run contiguously
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int64_t idx = wbase + static_cast<int64_t>(i) * kWave + lane;
      if (idx < n) {
        const uint32_t d = (key[i] >> shift) & (BINS - 1u);
        const uint32_t lpos = cnt[w][d] + rank[i];
        s_key[lpos] = key[i];
        s_val[lpos] = val[i];
      }
    }
    __syncthreads();
    const int64_t tile_n = min(static_cast<int64_t>(kRxTile), n - tile * kRxTile);
#pragma unroll
    for (int i = 0; i < kRxItems; ++i) {
      const int j = i * kRxThreads + t;
      if (j < tile_n) {
        const uint32_t k = s_key[j];
        const uint32_t pos = s_goff[(k >> shift) & (BINS - 1u)] + static_cast<uint32_t>(j);
        keys_out[pos] = k;
        vals_out[pos] = s_val[j];
      }
    }
    __syncthreads();  // the next tile reuses the LDS arrays
  }
}

// Scratch of one sort of n keys below 2^key_bits.
struct RadixBuffers {
  uint32_t *ka, *va;      // intermediate keys and values (sorts of two or more passes)
  uint32_t *hist, *offs;  // [2^max_bits][ntiles] digit counts and output offsets of a pass
  uint64_t* scan;         // look-back words of each pass's offset scan
  uint32_t* ctrl;         // kRxCtrlWords
  uint32_t* unsorted;     // sorted-input flag (set when the input is out of order)
  uint32_t* aux;          // a flag of the caller's, zeroed with the sort's own words
  uint32_t* zero_begin;   // scan .. ctrl: cleared by one fill before each sort
  int64_t zero_words;
  int64_t ntiles;
  RxPlan plan;
};

inline RadixBuffers carve_radix(Carver& c, int64_t n, int key_bits) {
  RadixBuffers r;
  r.plan = rx_plan(key_bits);
  r.ntiles = ceil_div(n > 0 ? n : 1, kRxTile);
  const bool inter = r.plan.passes > 1;
  const int64_t cells = r.ntiles << r.plan.max_bits;
  r.ka = c.take<uint32_t>(inter ? n : 0);
  r.va = c.take<uint32_t>(inter ? n : 0);
  r.hist = c.take<uint32_t>(cells);
  r.offs = c.take<uint32_t>(cells);
  const int64_t scan_words = r.plan.passes * scan_lookback_elems(cells);
  r.scan = c.take<uint64_t>(scan_words);
  r.ctrl = c.take<uint32_t>(kRxCtrlWords);
  r.unsorted = r.ctrl ? r.ctrl + kRxCtrlUnsorted : nullptr;
  r.aux = r.ctrl ? r.ctrl + kRxCtrlAux : nullptr;
  r.zero_begin = reinterpret_cast<uint32_t*>(r.scan);
  r.zero_words = r.scan ? (r.ctrl + kRxCtrlWords) - r.zero_begin : 0;
  return r;
}

template <int SRC, int BITS>
int radix_pass(const void* kin, const uint32_t* vin, int64_t n, int64_t N, int shift,
               uint32_t* kout, uint32_t* vout, const RadixBuffers& r, uint64_t* scan,
               const uint32_t* active, const RxDetect& det, hipStream_t st) {
  const int64_t ntiles = r.ntiles;
  const int64_t grid = ntiles < kRxGrid ? ntiles : kRxGrid;
  hipLaunchKernelGGL((radix_hist<SRC, BITS>), dim3(grid), dim3(kRxThreads), 0, st, kin, n, N,
                     shift, r.hist, ntiles, det.unsorted != nullptr ? nullptr : active, det);
  GEO_LAUNCH_CHECK("radix_hist");
  const int64_t cells = ntiles << BITS;
  int rc = device_exclusive_scan_lookback<uint32_t, uint32_t>(r.hist, cells, r.offs, nullptr,
                                                              false, scan, st, nullptr, active);
  if (rc) return rc;
  hipLaunchKernelGGL((radix_scatter<SRC, BITS>), dim3(grid), dim3(kRxThreads), 0, st, kin, vin, n,
                     N, shift, r.offs, ntiles, kout, vout, active);
  GEO_LAUNCH_CHECK("radix_scatter");
  return GEO_OK;
}

template <int SRC>
int radix_pass_bits(int bits, const void* kin, const uint32_t* vin, int64_t n, int64_t N, int shift,
                    uint32_t* kout, uint32_t* vout, const RadixBuffers& r, uint64_t* scan,
                    const uint32_t* active, const RxDetect& det, hipStream_t st) {
  switch (bits) {
    case 8: return radix_pass<SRC, 8>(kin, vin, n, N, shift, kout, vout, r, scan, active, det, st);
    case 7: return radix_pass<SRC, 7>(kin, vin, n, N, shift, kout, vout, r, scan, active, det, st);
    case 6: return radix_pass<SRC, 6>(kin, vin, n, N, shift, kout, vout, r, scan, active, det, st);
    case 5: return radix_pass<SRC, 5>(kin, vin, n, N, shift, kout, vout, r, scan, active, det, st);
    default: return radix_pass<SRC, 4>(kin, vin, n, N, shift, kout, vout, r, scan, active, det, st);
  }
}

// Sorts n > 0 keys (stable); keys_out / vals_out receive the result.  keys / vals are read as
// the first pass's source SRC; r was carved for n and the same key_bits.  With `detect`
// (index values only: SRC != kRxPairs), input already in key order costs the first histogram
// alone (see the header); its unsorted / fallback / output fields are filled in here from r and
// keys_out / vals_out, the node-bound fields come from the caller.
template <int SRC>
int radix_sort(const void* keys, const uint32_t* vals, int64_t n, int64_t N, uint32_t* keys_out,
               uint32_t* vals_out, const RadixBuffers& r, hipStream_t st,
               const RxDetect* detect = nullptr) {
  if (n <= 0)  // the kernels clamp positions into [0, n)
    return set_error(GEO_ERR_INVALID, "radix_sort: needs at least one key (n=%lld)", (long long)n);
  if (SRC == kRxPairs && detect != nullptr)
    return set_error(GEO_ERR_INVALID, "radix_sort: sorted-input detection needs index values");
  const RxPlan& plan = r.plan;
  int rc = device_fill<uint32_t>(r.zero_begin, r.zero_words, 0u, st);
  if (rc) return rc;
  RxDetect det;
  if (detect != nullptr) {
    det = *detect;
    det.unsorted = r.unsorted;
    det.fallback = r.aux;
    det.keys_out = keys_out;
    det.vals_out = vals_out;
  }
  const uint32_t* active = detect != nullptr ? r.unsorted : nullptr;
  const int64_t scan_words = scan_lookback_elems(r.ntiles << plan.max_bits);
  // ping-pong so that the last pass lands in keys_out: an odd pass count starts there
  uint32_t* bk[2] = {keys_out, r.ka};
  uint32_t* bv[2] = {vals_out, r.va};
  int cur = plan.passes % 2 == 1 ? 0 : 1;
  const void* kin = keys;
  const uint32_t* vin = vals;
  for (int p = 0; p < plan.passes; ++p) {
    uint32_t* kout = bk[cur];
    uint32_t* vout = bv[cur];
    uint64_t* scan = r.scan + p * scan_words;
    rc = p == 0 ? radix_pass_bits<SRC>(plan.bits[p], kin, vin, n, N, plan.shift[p], kout, vout, r,
                                       scan, active, det, st)
                : radix_pass_bits<kRxPairs>(plan.bits[p], kin, vin, n, N, plan.shift[p], kout,
                                            vout, r, scan, active, RxDetect{}, st);
    if (rc) return rc;
    kin = kout;
    vin = vout;
    cur ^= 1;
  }
  return GEO_OK;
}

}  // namespace
}  // namespace geo
