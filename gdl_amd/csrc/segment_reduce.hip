// segment_reduce.hip — sorted-segment sum / mean / max, forward and backward, for gfx950.
//
// Forward (replaces segment_reduce_sum_kernel, geoembodied/csrc/segment_reduce_kernel.cu:66-93).
//   A row of C elements is read as 16-byte (or narrower, when C or the pointers do not allow
//   it) vectors; L lanes cover a row (L = next power of two >= vectors per row, at most 64), so
//   a wave has R = 64/L lane groups and one wave-wide load instruction moves R whole rows.
//   Two kernels:
//   * seg_fwd_merge_kernel (many short segments, the graph-aggregation case): a wave takes up
//     to L consecutive segments and splits their rows evenly over its lane groups (merge path);
//     see the comment above the kernel.
//   * seg_fwd_kernel (few long segments, the pooling case): a wave walks its segments one at a
//     time; the lane groups take rows start+g, start+g+R, ..., 8 rows per group in flight, and
//     the R partial results are combined with a xor-butterfly.
// Backward (replaces the ATen gather + un-permute of geoembodied/functional/segment_reduce.py:
//   259-270): one lane group per sorted edge row e, grad_msg[perm[e]] = f(grad_out[col_sorted[e]]).
//
// Sum / mean accumulate in fp32 (fp64 for double) in ascending row order inside a lane group;
// partial results are combined in a fixed order, so results are bitwise reproducible run to run.
// Every index read from memory is range-checked, so inconsistent CSR arrays cannot make a
// kernel access memory outside the given tensors.
#include "common.hpp"

namespace geo {
namespace {

constexpr int kSegThreads = 256;
constexpr int kSegWaves = kSegThreads / kWave;
constexpr int kUnroll = 8;

template <typename T> struct AccT { using type = float; };
template <> struct AccT<double> { using type = double; };

__device__ __forceinline__ float to_acc(float x) { return x; }
__device__ __forceinline__ float to_acc(uint16_t x) { return bf16_to_f32(x); }
__device__ __forceinline__ double to_acc(double x) { return x; }

template <typename T> __device__ __forceinline__ T from_acc(float x);
template <> __device__ __forceinline__ float from_acc<float>(float x) { return x; }
template <> __device__ __forceinline__ uint16_t from_acc<uint16_t>(float x) { return f32_to_bf16(x); }
template <typename T> __device__ __forceinline__ T from_acc(double x);
template <> __device__ __forceinline__ double from_acc<double>(double x) { return x; }

template <int VB> struct Raw;
template <> struct Raw<16> { using type = uint4; };
template <> struct Raw<8> { using type = uint2; };
template <> struct Raw<4> { using type = uint32_t; };
template <> struct Raw<2> { using type = uint16_t; };

// One lane's slice of a row: VB bytes = EPV elements.
template <typename T, int VB>
struct Vec {
  static constexpr int EPV = VB / static_cast<int>(sizeof(T));
  union {
    typename Raw<VB>::type raw;
    T e[EPV];
  };
  __device__ __forceinline__ void load(const T* p) {
    raw = *reinterpret_cast<const typename Raw<VB>::type*>(p);
  }
  // Message rows are read once per reduction: non-temporal (streaming) loads.
  __device__ __forceinline__ void load_stream(const T* p) {
    if constexpr (VB == 16) {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
      raw.x = v.x; raw.y = v.y; raw.z = v.z; raw.w = v.w;
    } else if constexpr (VB == 8) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
      raw.x = v.x; raw.y = v.y;
    } else {
      raw = __builtin_nontemporal_load(reinterpret_cast<const typename Raw<VB>::type*>(p));
    }
  }
  // Outputs are written once and not read back by this kernel: non-temporal (streaming) stores
  // keep them from displacing the message rows in the caches.
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (VB == 16) {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 v = {raw.x, raw.y, raw.z, raw.w};
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
    } else if constexpr (VB == 8) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 v = {raw.x, raw.y};
      __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
    } else {
      __builtin_nontemporal_store(raw, reinterpret_cast<typename Raw<VB>::type*>(p));
    }
  }
};

// EPV int32 argmax entries belonging to one vector slice (4..32 bytes).
template <int N>
struct IVec {
  int32_t e[N];
  __device__ __forceinline__ void load(const int32_t* p) {
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 4) {
        int4 t = *reinterpret_cast<const int4*>(p + i);
        e[i] = t.x; e[i + 1] = t.y; e[i + 2] = t.z; e[i + 3] = t.w;
      }
    } else if constexpr (N == 2) {
      int2 t = *reinterpret_cast<const int2*>(p);
      e[0] = t.x; e[1] = t.y;
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) e[i] = p[i];
    }
  }
  __device__ __forceinline__ void store(int32_t* p) const {
    typedef int i32x4 __attribute__((ext_vector_type(4)));
    typedef int i32x2 __attribute__((ext_vector_type(2)));
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int i = 0; i < N; i += 4) {
        const i32x4 v = {e[i], e[i + 1], e[i + 2], e[i + 3]};
        __builtin_nontemporal_store(v, reinterpret_cast<i32x4*>(p + i));
      }
    } else if constexpr (N == 2) {
      const i32x2 v = {e[0], e[1]};
      __builtin_nontemporal_store(v, reinterpret_cast<i32x2*>(p));
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) __builtin_nontemporal_store(e[i], p + i);
    }
  }
};

// Max ordering with NaN above every number (NaN propagates like torch.maximum).
template <typename A>
__device__ __forceinline__ bool max_gt(A a, A b) { return a != a ? (b == b) : (a > b); }
template <typename A>
__device__ __forceinline__ bool max_eq(A a, A b) { return a != a ? (b != b) : (a == b); }

template <typename A>
__device__ __forceinline__ A shfl_xor_acc(A v, int m) { return __shfl_xor(v, m, kWave); }

__device__ __forceinline__ int clamp_i(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Element offset of row r (0 <= r < 2^31) in rows of c elements (c < 2^32, checked by the host):
// one 32 x 32 -> 64-bit multiply instead of a signed 64-bit product.
__device__ __forceinline__ int64_t row_off(int r, int64_t c) {
  return static_cast<int64_t>(static_cast<uint64_t>(static_cast<uint32_t>(r)) * static_cast<uint32_t>(c));
}

template <typename T, int VB, int OP>
__global__ __launch_bounds__(kSegThreads) void seg_fwd_kernel(
    const T* __restrict__ msg, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ seg_start, const int32_t* __restrict__ seg_end, int32_t E,
    int64_t S, int64_t C, int vpr, int log_l, int segs_per_wave, T* __restrict__ out,
    int32_t* __restrict__ arg, int tie_mode) {
  using A = typename AccT<T>::type;
  using V = Vec<T, VB>;
  constexpr int EPV = V::EPV;
  const int lane = lane_id();
  const int L = 1 << log_l;
  const int R = kWave >> log_l;
  const int g = lane >> log_l;
  const int vl = lane & (L - 1);
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kSegWaves + (threadIdx.x / kWave);
  const int64_t s_begin = wave * segs_per_wave;
  const int64_t s_stop = min(S, s_begin + segs_per_wave);
  const int ncol_iter = (vpr + L - 1) >> log_l;
  // All segment offsets of this wave in one vector load (segs_per_wave <= 64).
  int my_start = 0, my_end = 0;
  if (s_begin + lane < s_stop) {
    my_start = seg_start[s_begin + lane];
    my_end = seg_end[s_begin + lane];
  }

  for (int64_t s = s_begin; s < s_stop; ++s) {
    const int j = static_cast<int>(s - s_begin);
    const int start = clamp_i(__builtin_amdgcn_readlane(my_start, j), 0, E);
    const int end = clamp_i(__builtin_amdgcn_readlane(my_end, j), start, E);
    for (int ci = 0; ci < ncol_iter; ++ci) {
      const int vb = vl + ci * L;
      const bool col_ok = vb < vpr;
      const int64_t col_off = col_ok ? static_cast<int64_t>(vb) * EPV : 0;
      A acc[EPV];
      int first[EPV];
      int cnt[EPV];
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        acc[i] = OP == GEO_REDUCE_MAX ? -__builtin_inf() : A(0);
        first[i] = 0x7fffffff;
        cnt[i] = 0;
      }
      for (int e0 = start + g; e0 < end; e0 += R * kUnroll) {
        // Row ids first (independent loads), then every row load unconditionally from a
        // valid row, so kUnroll row reads are in flight together; invalid ones are masked.
        int rows[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int ev = min(e0 + u * R, end - 1);
          rows[u] = perm ? perm[ev] : ev;
        }
        V buf[kUnroll];
        bool ok[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int e = e0 + u * R;
          const int ev = min(e, end - 1);
          ok[u] = col_ok && e < end && static_cast<unsigned>(rows[u]) < static_cast<unsigned>(E);
          const int row = static_cast<unsigned>(rows[u]) < static_cast<unsigned>(E) ? rows[u] : ev;
          buf[u].load(msg + static_cast<int64_t>(row) * C + col_off);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          if (!ok[u]) continue;
          const int e = e0 + u * R;
#pragma unroll
          for (int i = 0; i < EPV; ++i) {
            const A v = to_acc(buf[u].e[i]);
            if constexpr (OP == GEO_REDUCE_MAX) {
              if (max_gt(v, acc[i])) {
                acc[i] = v; first[i] = e; cnt[i] = 1;
              } else if (max_eq(v, acc[i])) {
                cnt[i] += 1;
                if (cnt[i] == 1) first[i] = e;
              }
            } else {
              acc[i] += v;
            }
          }
        }
      }
      // Combine the R lane groups (xor over the lane bits above log_l).
      for (int m = L; m < kWave; m <<= 1) {
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          const A o = shfl_xor_acc(acc[i], m);
          if constexpr (OP == GEO_REDUCE_MAX) {
            const int of = __shfl_xor(first[i], m, kWave);
            const int oc = __shfl_xor(cnt[i], m, kWave);
            if (max_gt(o, acc[i])) {
              acc[i] = o; first[i] = of; cnt[i] = oc;
            } else if (max_eq(o, acc[i])) {
              // equal maxima (+-0, NaN payloads): keep the value of the earlier position
              if (of < first[i]) { acc[i] = o; first[i] = of; }
              cnt[i] += oc;
            }
          } else {
            acc[i] += o;
          }
        }
      }
      if (g == 0 && col_ok) {
        V res;
        const int n = end - start;
        if constexpr (OP == GEO_REDUCE_MAX) {
          IVec<EPV> a;
#pragma unroll
          for (int i = 0; i < EPV; ++i) {
            res.e[i] = cnt[i] == 0 ? from_acc<T>(A(0)) : from_acc<T>(acc[i]);
            a.e[i] = cnt[i] == 0 ? -1 : ((cnt[i] == 1 || tie_mode == 1) ? first[i] : -cnt[i]);
          }
          a.store(arg + s * C + col_off);
        } else if constexpr (OP == GEO_REDUCE_MEAN) {
          const A denom = static_cast<A>(n > 1 ? n : 1);
#pragma unroll
          for (int i = 0; i < EPV; ++i) res.e[i] = from_acc<T>(acc[i] / denom);
        } else {
#pragma unroll
          for (int i = 0; i < EPV; ++i) res.e[i] = from_acc<T>(acc[i]);
        }
        res.store(out + s * C + col_off);
      }
    }
  }
}

// Forward for many short segments: merge-path split of a wave's rows over its lane groups.
//
// A wave owns n <= L consecutive segments (L = lanes per row); every lane group holds the whole
// segment table (lane vl <-> segment vl) and the inclusive prefix of the segment lengths, so the
// wave's rows form one "flat" range [0, T).  Group g streams the flat positions
// [g*c, min((g+1)*c, T)), c = ceil(T / R): every group has the same amount of work whatever the
// segment sizes are.  The segment of a flat position f is the number of prefixes <= f (one
// ballot) and its row is base[j] + f (one lane permute).  merge_unroll() rows per group are
// loaded per step, and the row ids of the next step are fetched while those rows are in flight.
// A segment is written by the group holding its first row; a segment that continues past the
// end of a group's range is completed with the partial results of the following groups, which
// park them in LDS (in group order, so the result does not depend on timing).
//
// Tuning (measured on MI355X, C3 shapes): one wave per workgroup schedules best; rows per group
// per step: 8 for 4/8-byte types (6: 0.406 ms, 12: 0.410 ms against 0.399 ms for the fp32 sum),
// 6 for bf16 (more accumulators per row; 4: 0.215 ms, 6: 0.211 ms, 8: 0.213 ms), 4 for max (more
// state); about 16 KB of rows per wave (kMergeWaveBytes) balances per-wave overhead against tail
// effects.
constexpr int kMergeThreads = kWave;
constexpr int64_t kMergeWaveBytes = 16384;
template <typename T, int OP>
constexpr int merge_unroll() { return OP == GEO_REDUCE_MAX ? 4 : (sizeof(T) == 2 ? 6 : 8); }

template <typename T, int VB, int OP>
struct MergeSlot {
  using A = typename AccT<T>::type;
  static constexpr int EPV = VB / static_cast<int>(sizeof(T));
  A acc[EPV];
  int first[OP == GEO_REDUCE_MAX ? EPV : 1];
  int cnt[OP == GEO_REDUCE_MAX ? EPV : 1];
};

template <typename T, int VB, int OP, bool PERM>
__global__ __launch_bounds__(kMergeThreads) void seg_fwd_merge_kernel(
    const T* __restrict__ msg, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ seg_start, const int32_t* __restrict__ seg_end, int32_t E,
    int64_t S, int64_t C, int vpr, int log_l, int segs_per_wave, T* __restrict__ out,
    int32_t* __restrict__ arg, int tie_mode) {
  using A = typename AccT<T>::type;
  using V = Vec<T, VB>;
  constexpr int EPV = V::EPV;
  constexpr bool MAX = OP == GEO_REDUCE_MAX;
  constexpr int U = merge_unroll<T, OP>();
  __shared__ MergeSlot<T, VB, OP> park[kWave];

  const int lane = lane_id();
  const int L = 1 << log_l;
  const int log_r = 6 - log_l;
  const int R = 1 << log_r;
  const int g = lane >> log_l;
  const int vl = lane & (L - 1);
  const int gbase = g << log_l;
  const uint64_t gmask = log_l == 6 ? ~0ull : ((1ull << L) - 1);
  const int64_t s_begin = static_cast<int64_t>(blockIdx.x) * segs_per_wave;
  if (s_begin >= S) return;
  const int nseg = static_cast<int>(min(S - s_begin, static_cast<int64_t>(segs_per_wave)));

  // Segment table, replicated in every group: lane vl <-> segment s_begin + vl.
  const bool has = vl < nseg;
  int st = 0, n = 0;
  if (has) {
    st = clamp_i(seg_start[s_begin + vl], 0, E);
    n = clamp_i(seg_end[s_begin + vl], st, E) - st;
  }
  int incl = n;
  for (int d = 1; d < L; d <<= 1) {
    const int o = __shfl_up(incl, d, kWave);
    if (vl >= d) incl += o;
  }
  const int excl = incl - n;
  const int T_rows = __shfl(incl, L - 1, kWave);
  const int base = st - excl;
  const int key = has ? incl : 0x7fffffff;
  const int chunk = (T_rows + R - 1) >> log_r;
  const int lo = min(g * chunk, T_rows);
  const int hi = min(lo + chunk, T_rows);
  const int ncol_iter = (vpr + L - 1) >> log_l;

  // Local segment of flat position f for this group (group-uniform result).
  auto seg_of = [&](int f) -> int {
    return static_cast<int>(__popcll((__ballot(key <= f) >> gbase) & gmask));
  };
  auto lane_of = [&](int j) { return gbase + (j < L ? j : L - 1); };

  // Empty segments: zeros (and arg -1 for max); segment j is written by group j mod R.
  {
    uint64_t mine = (__ballot(has && n == 0) >> gbase) & gmask;
    uint64_t sel = 0;
    for (int j = g; j < L; j += R) sel |= 1ull << j;
    mine &= sel;
    while (__ballot(mine != 0)) {
      if (mine != 0) {
        const int64_t s = s_begin + __builtin_ctzll(mine);
        mine &= mine - 1;
        for (int ci = 0; ci < ncol_iter; ++ci) {
          const int vb = vl + ci * L;
          if (vb >= vpr) continue;
          V z;
#pragma unroll
          for (int i = 0; i < EPV; ++i) z.e[i] = from_acc<T>(A(0));
          z.store(out + s * C + static_cast<int64_t>(vb) * EPV);
          if constexpr (MAX) {
            IVec<EPV> a;
#pragma unroll
            for (int i = 0; i < EPV; ++i) a.e[i] = -1;
            a.store(arg + s * C + static_cast<int64_t>(vb) * EPV);
          }
        }
      }
    }
  }
  if (T_rows == 0) return;
  const int steps = (chunk + U - 1) / U;

  for (int ci = 0; ci < ncol_iter; ++ci) {
    const int vb = vl + ci * L;
    const bool col_ok = vb < vpr;
    const int64_t col_off = col_ok ? static_cast<int64_t>(vb) * EPV : 0;
    A acc[EPV];
    int first[EPV];
    int cnt[EPV];
    int jcur = -1;
    // `pos0` is the position of the segment's first row in this range: with a valid
    // permutation that row is taken, so a first maximum of -inf (equal to the initial value)
    // is recorded there without a separate "nothing seen yet" test per element.
    auto reset = [&](int pos0) {
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        acc[i] = MAX ? -__builtin_inf() : A(0);
        first[i] = pos0;
        cnt[i] = 0;
      }
    };
    auto write_out = [&](int j) {
      // every lane of the group takes part in the permute, including lanes without a column
      const int nj = OP == GEO_REDUCE_MEAN ? __shfl(n, lane_of(j), kWave) : 0;
      if (!col_ok) return;
      const int64_t s = s_begin + j;
      V res;
      if constexpr (MAX) {
        IVec<EPV> a;
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          res.e[i] = cnt[i] == 0 ? from_acc<T>(A(0)) : from_acc<T>(acc[i]);
          a.e[i] = cnt[i] == 0 ? -1 : ((cnt[i] == 1 || tie_mode == 1) ? first[i] : -cnt[i]);
        }
        a.store(arg + s * C + col_off);
      } else if constexpr (OP == GEO_REDUCE_MEAN) {
        const A denom = static_cast<A>(nj > 1 ? nj : 1);
#pragma unroll
        for (int i = 0; i < EPV; ++i) res.e[i] = from_acc<T>(acc[i] / denom);
      } else {
#pragma unroll
        for (int i = 0; i < EPV; ++i) res.e[i] = from_acc<T>(acc[i]);
      }
      res.store(out + s * C + col_off);
    };
    // Park this group's partial of a segment that began in an earlier group's range.
    auto park_partial = [&]() {
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        park[lane].acc[i] = acc[i];
        if constexpr (MAX) {
          park[lane].first[i] = first[i];
          park[lane].cnt[i] = cnt[i];
        }
      }
    };
    // Segment jcur is finished inside this range: write it, or park it if it began earlier.
    auto finish = [&]() {
      const int ex = __shfl(excl, lane_of(jcur), kWave);
      if (ex >= lo) write_out(jcur);
      else park_partial();
    };

    auto locate = [&](int f0, int* e, int* rows) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int f = f0 + u;
        const int b = __shfl(base, lane_of(seg_of(f)), kWave);
        e[u] = f < hi ? b + f : 0;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) rows[u] = PERM ? perm[e[u]] : e[u];
    };

    reset(0x7fffffff);
    int e[U], rows[U];
    locate(lo, e, rows);
    for (int k = 0; k < steps; ++k) {
      const int f0 = lo + k * U;
      V buf[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = f0 + u < hi && static_cast<unsigned>(rows[u]) < static_cast<unsigned>(E);
        buf[u].load_stream(msg + row_off(ok ? rows[u] : 0, C) + col_off);
      }
      int ecur[MAX ? U : 1];
      uint32_t rok = 0;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (MAX) ecur[u] = e[u];
        rok |= static_cast<uint32_t>(static_cast<unsigned>(rows[u]) < static_cast<unsigned>(E)) << u;
      }
      locate(f0 + U, e, rows);
      // Row values are consumed through selects only, so all U loads stay ahead of first use.
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int f = f0 + u;
        const bool live = f < hi;
        const int j = seg_of(f);
        if (live && j != jcur) {
          if (jcur >= 0) finish();
          reset(MAX ? ecur[MAX ? u : 0] : 0);
          jcur = j;
        }
        const bool take = live && ((rok >> u) & 1u);
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          const A v = to_acc(buf[u].e[i]);
          if constexpr (MAX) {
            // max_gt / max_eq as mask logic (no short-circuit, so no branches): NaN above
            // every number, all NaNs equal
            const bool vn = v != v, an = acc[i] != acc[i];
            const bool gt = take & ((v > acc[i]) | (vn & !an));
            const bool eq = take & !gt & ((v == acc[i]) | (vn & an));
            const int pos = ecur[MAX ? u : 0];
            first[i] = gt ? pos : first[i];
            cnt[i] = (gt ? 0 : cnt[i]) + ((gt | eq) ? 1 : 0);
            acc[i] = gt ? v : acc[i];
          } else {
            acc[i] += take ? v : A(0);
          }
        }
      }
    }

    // Last segment of the range.  If it began earlier, park it; if it ends here, write it;
    // otherwise it continues into the following groups, whose parked partials complete it.
    bool open = false;
    if (jcur >= 0) {
      const int ex = __shfl(excl, lane_of(jcur), kWave);
      const int in = __shfl(incl, lane_of(jcur), kWave);
      if (ex < lo) park_partial();
      else if (in <= hi) write_out(jcur);
      else open = true;
    }
    if (R > 1) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (open) {
        const int in = __shfl(incl, lane_of(jcur), kWave);
        for (int k = g + 1; k < R; ++k) {
          const int lo_k = min(k * chunk, T_rows);
          if (lo_k >= in) break;                       // segment ended before group k
          const MergeSlot<T, VB, OP>& p = park[(k << log_l) + vl];
#pragma unroll
          for (int i = 0; i < EPV; ++i) {
            if constexpr (MAX) {
              const A o = p.acc[i];
              if (p.cnt[i] > 0) {
                if (cnt[i] == 0 || max_gt(o, acc[i])) {
                  acc[i] = o; first[i] = p.first[i]; cnt[i] = p.cnt[i];
                } else if (max_eq(o, acc[i])) {
                  cnt[i] += p.cnt[i];
                }
              }
            } else {
              acc[i] += p.acc[i];
            }
          }
        }
        write_out(jcur);
      }
      if (ci + 1 < ncol_iter) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
      }
    }
  }
}

template <typename T, int VB, int OP>
__global__ __launch_bounds__(kSegThreads) void seg_bwd_kernel(
    const T* __restrict__ grad_out, const T* __restrict__ msg, const T* __restrict__ fwd_out,
    const int32_t* __restrict__ arg, const int32_t* __restrict__ col_sorted,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ seg_start,
    const int32_t* __restrict__ seg_end, int32_t E, int64_t S, int64_t C, int vpr, int log_l,
    int rows_per_wave, T* __restrict__ grad_msg) {
  using A = typename AccT<T>::type;
  using V = Vec<T, VB>;
  constexpr int EPV = V::EPV;
  const int lane = lane_id();
  const int L = 1 << log_l;
  const int R = kWave >> log_l;
  const int g = lane >> log_l;
  const int vl = lane & (L - 1);
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * kSegWaves + (threadIdx.x / kWave);
  const int64_t e_begin = wave * rows_per_wave;
  const int64_t e_stop = min(static_cast<int64_t>(E), e_begin + rows_per_wave);
  const int ncol_iter = (vpr + L - 1) >> log_l;

  constexpr int U = kUnroll / 2;
  for (int64_t e0 = e_begin + g; e0 < e_stop; e0 += static_cast<int64_t>(R) * U) {
    // U rows per lane group: targets and destinations first, then the gradient rows.
    int ss[U], pp[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = min(e0 + static_cast<int64_t>(u) * R, e_stop - 1);
      ss[u] = col_sorted[e];
      pp[u] = perm ? perm[e] : static_cast<int>(e);
    }
    A scales[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      scales[u] = A(1);
      if constexpr (OP == GEO_REDUCE_MEAN) {
        if (static_cast<unsigned>(ss[u]) < static_cast<unsigned>(S)) {
          const int n = seg_end[ss[u]] - seg_start[ss[u]];
          scales[u] = static_cast<A>(n > 1 ? n : 1);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
    const int64_t e = e0 + static_cast<int64_t>(u) * R;
    if (e >= e_stop) break;
    const int s = ss[u];
    const int p = pp[u];
    if (static_cast<unsigned>(p) >= static_cast<unsigned>(E)) continue;  // not a permutation
    const bool s_ok = static_cast<unsigned>(s) < static_cast<unsigned>(S);
    const A scale = scales[u];
    for (int ci = 0; ci < ncol_iter; ++ci) {
      const int vb = vl + ci * L;
      if (vb >= vpr) continue;
      const int64_t col_off = static_cast<int64_t>(vb) * EPV;
      V gv, res;
      if (s_ok) {
        gv.load(grad_out + row_off(s, C) + col_off);
      } else {
#pragma unroll
        for (int i = 0; i < EPV; ++i) gv.e[i] = from_acc<T>(A(0));
      }
      if constexpr (OP == GEO_REDUCE_SUM) {
        res = gv;
      } else if constexpr (OP == GEO_REDUCE_MEAN) {
#pragma unroll
        for (int i = 0; i < EPV; ++i) res.e[i] = from_acc<T>(to_acc(gv.e[i]) / scale);
      } else {
        IVec<EPV> a;
        if (s_ok) {
          a.load(arg + row_off(s, C) + col_off);
        } else {
#pragma unroll
          for (int i = 0; i < EPV; ++i) a.e[i] = -1;
        }
        bool any_tie = false;
#pragma unroll
        for (int i = 0; i < EPV; ++i) any_tie |= a.e[i] <= -2;
        V mv, ov;
        if (any_tie) {
          mv.load(msg + row_off(p, C) + col_off);
          ov.load(fwd_out + row_off(s, C) + col_off);
        }
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          A r = A(0);
          if (a.e[i] == static_cast<int>(e)) {
            r = to_acc(gv.e[i]);
          } else if (a.e[i] <= -2) {
            if (max_eq(to_acc(mv.e[i]), to_acc(ov.e[i])))
              r = to_acc(gv.e[i]) / static_cast<A>(-a.e[i]);
          }
          res.e[i] = from_acc<T>(r);
        }
      }
      res.store(grad_msg + row_off(p, C) + col_off);
    }
    }
  }
}

struct Layout {
  int vb;      // bytes per lane vector
  int vpr;     // vectors per row
  int log_l;   // log2 lanes per row group
};

Layout choose_layout(int64_t C, int esize, uintptr_t align_bits) {
  const int64_t row_bytes = C * esize;
  int vb = 16;
  while (vb > esize && ((row_bytes % vb) != 0 || (align_bits % vb) != 0)) vb >>= 1;
  Layout l;
  l.vb = vb;
  l.vpr = static_cast<int>(row_bytes / vb);
  int lanes = 1, lg = 0;
  while (lanes < l.vpr && lanes < kWave) { lanes <<= 1; ++lg; }
  l.log_l = lg;
  return l;
}

template <typename T, int OP>
int launch_fwd(const Layout& lay, const T* msg, const int32_t* perm, const int32_t* ns,
               const int32_t* ne, int32_t E, int64_t S, int64_t C, T* out, int32_t* arg,
               int tie_mode, hipStream_t st) {
  // Many short segments (the common case: graph aggregation) -> merge-path waves of at most L
  // segments; few long segments (pooling) -> whole waves cooperating on one segment at a time.
  const bool merge = S >= 4096 && E <= 128 * S;
  int spw;
  int64_t blocks;
  if (merge) {
    const int L = 1 << lay.log_l;
    const double wave_bytes = (E > S ? static_cast<double>(E) / S : 1.0) * C * sizeof(T);
    spw = static_cast<int>(static_cast<double>(kMergeWaveBytes) / wave_bytes + 0.5);
    if (spw > L) spw = L;
    if (spw < 1) spw = 1;
    blocks = ceil_div(S, spw);
  } else {
    spw = static_cast<int>(ceil_div(S, 32768));
    if (spw > 64) spw = 64;
    if (spw < 1) spw = 1;
    blocks = ceil_div(ceil_div(S, spw), kSegWaves);
  }
#define GEO_FWD_CASE(VBV)                                                                   \
  case VBV:                                                                                 \
    if constexpr (VBV >= static_cast<int>(sizeof(T))) {                                     \
      if (merge && perm)                                                                    \
        hipLaunchKernelGGL((seg_fwd_merge_kernel<T, VBV, OP, true>), dim3(blocks),           \
                           dim3(kMergeThreads), 0, st, msg, perm, ns, ne, E, S, C, lay.vpr,   \
                           lay.log_l, spw, out, arg, tie_mode);                             \
      else if (merge)                                                                       \
        hipLaunchKernelGGL((seg_fwd_merge_kernel<T, VBV, OP, false>), dim3(blocks),          \
                           dim3(kMergeThreads), 0, st, msg, perm, ns, ne, E, S, C, lay.vpr,   \
                           lay.log_l, spw, out, arg, tie_mode);                             \
      else                                                                                  \
        hipLaunchKernelGGL((seg_fwd_kernel<T, VBV, OP>), dim3(blocks), dim3(kSegThreads), 0,  \
                           st, msg, perm, ns, ne, E, S, C, lay.vpr, lay.log_l, spw, out, arg, \
                           tie_mode);                                                       \
    }                                                                                       \
    break;
  switch (lay.vb) {
    GEO_FWD_CASE(16)
    GEO_FWD_CASE(8)
    GEO_FWD_CASE(4)
    GEO_FWD_CASE(2)
    default:
      return set_error(GEO_ERR_INVALID, "segment_reduce: unsupported vector width %d", lay.vb);
  }
#undef GEO_FWD_CASE
  GEO_LAUNCH_CHECK("seg_fwd_kernel");
  return GEO_OK;
}

template <typename T, int OP>
int launch_bwd(const Layout& lay, const T* grad_out, const T* msg, const T* fwd_out,
               const int32_t* arg, const int32_t* cs, const int32_t* perm, const int32_t* ns,
               const int32_t* ne, int32_t E, int64_t S, int64_t C, T* grad_msg, hipStream_t st) {
  const int R = kWave >> lay.log_l;
  int rpw = R * 16;
  const int64_t waves = ceil_div(E, rpw);
  const int64_t blocks = ceil_div(waves, kSegWaves);
#define GEO_BWD_CASE(VBV)                                                                    \
  case VBV:                                                                                  \
    if constexpr (VBV >= static_cast<int>(sizeof(T))) {                                      \
      hipLaunchKernelGGL((seg_bwd_kernel<T, VBV, OP>), dim3(blocks), dim3(kSegThreads), 0, st, \
                         grad_out, msg, fwd_out, arg, cs, perm, ns, ne, E, S, C, lay.vpr,     \
                         lay.log_l, rpw, grad_msg);                                          \
    }                                                                                        \
    break;
  switch (lay.vb) {
    GEO_BWD_CASE(16)
    GEO_BWD_CASE(8)
    GEO_BWD_CASE(4)
    GEO_BWD_CASE(2)
    default:
      return set_error(GEO_ERR_INVALID, "segment_reduce: unsupported vector width %d", lay.vb);
  }
#undef GEO_BWD_CASE
  GEO_LAUNCH_CHECK("seg_bwd_kernel");
  return GEO_OK;
}

int esize_of(int dtype) { return dtype == GEO_F32 ? 4 : dtype == GEO_BF16 ? 2 : 8; }

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" int geo_segment_reduce_fwd(int reduce, int dtype, const void* msg, const int32_t* perm,
                                      const int32_t* node_start, const int32_t* node_end,
                                      int64_t E, int64_t S, int64_t C, void* out, int32_t* arg,
                                      int tie_mode, void* stream) {
  GEO_REQUIRE(reduce >= GEO_REDUCE_SUM && reduce <= GEO_REDUCE_MAX,
              "segment_reduce: unknown reduce code %d", reduce);
  GEO_REQUIRE(dtype == GEO_F32 || dtype == GEO_BF16 || dtype == GEO_F64,
              "segment_reduce: unknown dtype code %d", dtype);
  GEO_REQUIRE(E >= 0 && S >= 0 && C >= 0, "segment_reduce: negative size (E=%lld S=%lld C=%lld)",
              (long long)E, (long long)S, (long long)C);
  GEO_REQUIRE(E < 0x7fffffffLL, "segment_reduce: E=%lld exceeds int32 indexing", (long long)E);
  GEO_REQUIRE(C <= 0xffffffffLL, "segment_reduce: C=%lld exceeds 32 bits", (long long)C);
  if (S == 0 || C == 0) return GEO_OK;
  GEO_REQUIRE(out != nullptr && node_start != nullptr && node_end != nullptr,
              "segment_reduce: null output or offsets");
  GEO_REQUIRE(E == 0 || msg != nullptr, "segment_reduce: null msg with E=%lld", (long long)E);
  GEO_REQUIRE(reduce != GEO_REDUCE_MAX || arg != nullptr, "segment_reduce: max needs arg");
  const int es = esize_of(dtype);
  uintptr_t bits = reinterpret_cast<uintptr_t>(msg) | reinterpret_cast<uintptr_t>(out);
  Layout lay = choose_layout(C, es, bits);
  if (reduce == GEO_REDUCE_MAX) {
    // Narrow the vector until the matching int32 slice of arg is naturally aligned.
    const uintptr_t abits = reinterpret_cast<uintptr_t>(arg);
    GEO_REQUIRE(abits % 4 == 0, "segment_reduce: arg must be 4-byte aligned");
    while (lay.vb > es) {
      const int ibytes = (lay.vb / es) * 4;
      const int need = ibytes >= 16 ? 16 : ibytes;
      if (abits % need == 0) break;
      lay = choose_layout(C, es, bits | uintptr_t(lay.vb / 2));
    }
  }
  hipStream_t st = as_stream(stream);
  const int32_t E32 = static_cast<int32_t>(E);
#define GEO_DISPATCH_FWD(TT)                                                                   \
  switch (reduce) {                                                                            \
    case GEO_REDUCE_SUM:                                                                       \
      return launch_fwd<TT, GEO_REDUCE_SUM>(lay, static_cast<const TT*>(msg), perm, node_start, \
                                            node_end, E32, S, C, static_cast<TT*>(out), arg,   \
                                            tie_mode, st);                                     \
    case GEO_REDUCE_MEAN:                                                                      \
      return launch_fwd<TT, GEO_REDUCE_MEAN>(lay, static_cast<const TT*>(msg), perm,           \
                                             node_start, node_end, E32, S, C,                  \
                                             static_cast<TT*>(out), arg, tie_mode, st);         \
    default:                                                                                   \
      return launch_fwd<TT, GEO_REDUCE_MAX>(lay, static_cast<const TT*>(msg), perm, node_start, \
                                            node_end, E32, S, C, static_cast<TT*>(out), arg,   \
                                            tie_mode, st);                                     \
  }
  if (dtype == GEO_F32) { GEO_DISPATCH_FWD(float) }
  if (dtype == GEO_BF16) { GEO_DISPATCH_FWD(uint16_t) }
  GEO_DISPATCH_FWD(double)
#undef GEO_DISPATCH_FWD
}

extern "C" int geo_segment_reduce_bwd(int reduce, int dtype, const void* grad_out,
                                      const void* msg, const void* out, const int32_t* arg,
                                      const int32_t* col_sorted, const int32_t* perm,
                                      const int32_t* node_start, const int32_t* node_end,
                                      int64_t E, int64_t S, int64_t C, void* grad_msg,
                                      void* stream) {
  GEO_REQUIRE(reduce >= GEO_REDUCE_SUM && reduce <= GEO_REDUCE_MAX,
              "segment_reduce_bwd: unknown reduce code %d", reduce);
  GEO_REQUIRE(dtype == GEO_F32 || dtype == GEO_BF16 || dtype == GEO_F64,
              "segment_reduce_bwd: unknown dtype code %d", dtype);
  GEO_REQUIRE(E >= 0 && S >= 0 && C >= 0, "segment_reduce_bwd: negative size");
  GEO_REQUIRE(E < 0x7fffffffLL, "segment_reduce_bwd: E=%lld exceeds int32 indexing", (long long)E);
  GEO_REQUIRE(C <= 0xffffffffLL, "segment_reduce_bwd: C=%lld exceeds 32 bits", (long long)C);
  if (E == 0 || C == 0) return GEO_OK;
  GEO_REQUIRE(grad_msg != nullptr && col_sorted != nullptr, "segment_reduce_bwd: null pointer");
  GEO_REQUIRE(S == 0 || grad_out != nullptr, "segment_reduce_bwd: null grad_out");
  GEO_REQUIRE(reduce != GEO_REDUCE_MEAN || (node_start && node_end),
              "segment_reduce_bwd: mean needs node_start/node_end");
  GEO_REQUIRE(reduce != GEO_REDUCE_MAX || (arg && msg && out),
              "segment_reduce_bwd: max needs arg, msg and out");
  const int es = esize_of(dtype);
  uintptr_t bits = reinterpret_cast<uintptr_t>(grad_out) | reinterpret_cast<uintptr_t>(grad_msg);
  if (reduce == GEO_REDUCE_MAX)
    bits |= reinterpret_cast<uintptr_t>(msg) | reinterpret_cast<uintptr_t>(out);
  Layout lay = choose_layout(C, es, bits);
  if (reduce == GEO_REDUCE_MAX) {
    // Narrow the vector until the matching int32 slice of arg is naturally aligned.
    const uintptr_t abits = reinterpret_cast<uintptr_t>(arg);
    while (lay.vb > es) {
      const int ibytes = (lay.vb / es) * 4;
      const int need = ibytes >= 16 ? 16 : ibytes;
      if (abits % need == 0) break;
      lay = choose_layout(C, es, bits | uintptr_t(lay.vb / 2));
    }
  }
  hipStream_t st = as_stream(stream);
  const int32_t E32 = static_cast<int32_t>(E);
#define GEO_DISPATCH_BWD(TT)                                                                    \
  switch (reduce) {                                                                             \
    case GEO_REDUCE_SUM:                                                                        \
      return launch_bwd<TT, GEO_REDUCE_SUM>(lay, static_cast<const TT*>(grad_out),              \
                                            static_cast<const TT*>(msg),                        \
                                            static_cast<const TT*>(out), arg, col_sorted, perm, \
                                            node_start, node_end, E32, S, C,                    \
                                            static_cast<TT*>(grad_msg), st);                    \
    case GEO_REDUCE_MEAN:                                                                       \
      return launch_bwd<TT, GEO_REDUCE_MEAN>(lay, static_cast<const TT*>(grad_out),             \
                                             static_cast<const TT*>(msg),                       \
                                             static_cast<const TT*>(out), arg, col_sorted,      \
                                             perm, node_start, node_end, E32, S, C,             \
                                             static_cast<TT*>(grad_msg), st);                   \
    default:                                                                                    \
      return launch_bwd<TT, GEO_REDUCE_MAX>(lay, static_cast<const TT*>(grad_out),              \
                                            static_cast<const TT*>(msg),                        \
                                            static_cast<const TT*>(out), arg, col_sorted, perm, \
                                            node_start, node_end, E32, S, C,                    \
                                            static_cast<TT*>(grad_msg), st);                    \
  }
  if (dtype == GEO_F32) { GEO_DISPATCH_BWD(float) }
  if (dtype == GEO_BF16) { GEO_DISPATCH_BWD(uint16_t) }
  GEO_DISPATCH_BWD(double)
#undef GEO_DISPATCH_BWD
}
