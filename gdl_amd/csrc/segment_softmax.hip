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
#include <initializer_list>

#include "scan.hpp"

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

// With zero_tail, the rows of the CSR positions [node_end[S-1], E) — the edges whose target lies
// outside [0, S) in a CSR built by geo_csr_build, whose node ranges are ascending and contiguous
// from 0 — are written as 0 by the grid's threads together, so no separate fill of the output is
// needed.  The tail is empty for a CSR that covers every edge.  The fp32 kernels load its start
// (one uniform load) together with their CSR bounds and write the zeros after their own work,
// so the load adds no step to their chain of dependent loads.
__device__ __forceinline__ int tail_start(int zero_tail, const int32_t* __restrict__ ne, int32_t E,
                                          int64_t S) {
  return zero_tail ? clamp_idx(ne[S - 1], 0, E) : E;
}

template <typename T>
__device__ __forceinline__ void zero_rows_from(T* __restrict__ out, const int32_t* __restrict__ perm,
                                               int t0, int32_t E, int64_t H) {
  const int64_t n = static_cast<int64_t>(E - t0) * H;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t q = i / H;
    const int e = t0 + static_cast<int>(q);
    const int r = perm ? perm[e] : e;
    if (static_cast<unsigned>(r) < static_cast<unsigned>(E))
      out[static_cast<int64_t>(r) * H + (i - q * H)] = T(0);
  }
}

template <typename T>
__device__ __forceinline__ void zero_tail_rows(T* __restrict__ out, const int32_t* __restrict__ perm,
                                               const int32_t* __restrict__ ne, int32_t E, int64_t S,
                                               int64_t H) {
  zero_rows_from<T>(out, perm, clamp_idx(ne[S - 1], 0, E), E, H);
}

// Largest value over the wave (v >= 0; every lane active).
__device__ __forceinline__ int uniform_max(int v) {
  return static_cast<int>(wave_max_u32(static_cast<uint32_t>(v)));
}

template <typename T>
__global__ __launch_bounds__(kSmThreads) void seg_softmax_fwd_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ perm, const int32_t* __restrict__ ns,
    const int32_t* __restrict__ ne, int32_t E, int64_t S, int32_t H, T* __restrict__ w,
    int zero_tail) {
  if (zero_tail) zero_tail_rows<T>(w, perm, ne, E, S, H);
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
    int32_t H, T* __restrict__ dx, int zero_tail) {
  if (zero_tail) zero_tail_rows<T>(dx, perm, ne, E, S, H);
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

// Rows of the CSR positions e[i] where ok[i] (-1 elsewhere, and for a permutation entry outside
// [0, E)).  Every permutation entry is loaded before any is checked: with the check right after
// its load the compiler waits for each load in turn.  Positions that are not ok read entry 0
// (E >= 1).
template <int NR>
__device__ __forceinline__ void sm_rows(const int32_t* __restrict__ perm, int32_t E,
                                        const int (&e)[NR], const bool (&ok)[NR], int (&r)[NR]) {
  if (perm) {
    int v[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) v[i] = perm[ok[i] ? e[i] : 0];
#pragma unroll
    for (int i = 0; i < NR; ++i)
      r[i] = ok[i] && static_cast<unsigned>(v[i]) < static_cast<unsigned>(E) ? v[i] : -1;
  } else {
#pragma unroll
    for (int i = 0; i < NR; ++i) r[i] = ok[i] ? e[i] : -1;
  }
}

__global__ __launch_bounds__(kSmThreads) void seg_softmax_rows_fwd(
    const float* __restrict__ x, const int32_t* __restrict__ perm, const int32_t* __restrict__ ns,
    const int32_t* __restrict__ ne, int32_t E, int64_t S, int32_t H, float* __restrict__ w,
    int zero_tail) {
  const int t0 = tail_start(zero_tail, ne, E, S);
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
  {
    int e[2];
    bool ok[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      e[c] = g.a + 16 * c + g.li;
      ok[c] = c < nch && e[c] < g.b;
    }
    sm_rows<2>(perm, E, e, ok, rk);
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
  zero_rows_from<float>(w, perm, t0, E, H);
}

__global__ __launch_bounds__(kSmThreads) void seg_softmax_rows_bwd(
    const float* __restrict__ g_, const float* __restrict__ w, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ ns, const int32_t* __restrict__ ne, int32_t E, int64_t S, int32_t H,
    float* __restrict__ dx, int zero_tail) {
  const int t0 = tail_start(zero_tail, ne, E, S);
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
  zero_rows_from<float>(dx, perm, t0, E, H);
}


// ------------------------------------------------------- fp32, H in {1, 2, 4, 8} ---
// The same row layout with H a compile-time constant: a row of H scores is one 4/8/16-byte
// vector access (two for H = 8), every exponential is computed once and kept for the division,
// and a wave takes SQ groups of segments whose CSR bounds, permutation entries and rows are all
// requested before the first is used, so the three dependent loads of one group overlap those
// of the others.  Short segments (the host picks by average degree) take 8 lanes each, so
// fewer lane slots idle; each lane sums its chunks in order, then the row is reduced.
template <int HH>
__device__ __forceinline__ void sm_load(const float* __restrict__ x, int r, float (&v)[HH]) {
  const float* p = x + static_cast<int64_t>(r) * HH;
  if constexpr (HH == 1) {
    v[0] = p[0];
  } else if constexpr (HH == 2) {
    const float2 q = *reinterpret_cast<const float2*>(p);
    v[0] = q.x; v[1] = q.y;
  } else {
#pragma unroll
    for (int j = 0; j < HH / 4; ++j) {
      const float4 q = *reinterpret_cast<const float4*>(p + 4 * j);
      v[4 * j] = q.x; v[4 * j + 1] = q.y; v[4 * j + 2] = q.z; v[4 * j + 3] = q.w;
    }
  }
}

template <int HH>
__device__ __forceinline__ void sm_store(float* __restrict__ y, int r, const float (&v)[HH]) {
  float* p = y + static_cast<int64_t>(r) * HH;
  if constexpr (HH == 1) {
    p[0] = v[0];
  } else if constexpr (HH == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  } else {
#pragma unroll
    for (int j = 0; j < HH / 4; ++j)
      *reinterpret_cast<float4*>(p + 4 * j) = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  }
}

// Segments take LW = 8 or 16 lanes (one DPP half-row or row) and a lane keeps its first KC
// chunks of LW edges (32 edges) in registers; a wave serves SQ groups of 64 / LW segments.
template <int HH, int LW>
constexpr int sm_quads() { return (LW == 8 || HH >= 8) ? 1 : 2; }

template <int LW>
__device__ __forceinline__ float grp_maxf(float v) {
  v = fmaxf(v, sm_dpp<kDppXor1>(v));
  v = fmaxf(v, sm_dpp<kDppXor2>(v));
  v = fmaxf(v, sm_dpp<kDppHalfMirror>(v));
  if constexpr (LW == 16) v = fmaxf(v, sm_dpp<kDppMirror>(v));
  return v;
}
template <int LW>
__device__ __forceinline__ float grp_sumf(float v) {
  v += sm_dpp<kDppXor1>(v);
  v += sm_dpp<kDppXor2>(v);
  v += sm_dpp<kDppHalfMirror>(v);
  if constexpr (LW == 16) v += sm_dpp<kDppMirror>(v);
  return v;
}

// Bounds of the segment of group `quad` that this lane serves.
template <int LW>
__device__ __forceinline__ void sm_bounds(const int32_t* ns, const int32_t* ne, int32_t E, int64_t S,
                                          int64_t quad, int& a, int& b) {
  const int64_t s = quad * (kWave / LW) + lane_id() / LW;
  a = 0;
  b = 0;
  if (s < S) {
    a = clamp_idx(ns[s], 0, E);
    b = clamp_idx(ne[s], a, E);
  }
}

template <int HH, int LW>
__global__ __launch_bounds__(kSmThreads) void seg_softmax_vec_fwd(
    const float* __restrict__ x, const int32_t* __restrict__ perm, const int32_t* __restrict__ ns,
    const int32_t* __restrict__ ne, int32_t E, int64_t S, float* __restrict__ w, int zero_tail) {
  const int t0 = tail_start(zero_tail, ne, E, S);
  constexpr int SQ = sm_quads<HH, LW>();
  constexpr int KC = 32 / LW;
  const int li = lane_id() & (LW - 1);
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kSmThreads / kWave) + threadIdx.x / kWave;
  int a[SQ], b[SQ], rk[SQ][KC];
  float v[SQ][KC][HH];
#pragma unroll
  for (int q = 0; q < SQ; ++q) sm_bounds<LW>(ns, ne, E, S, wave * SQ + q, a[q], b[q]);
  {
    int e[SQ * KC], r[SQ * KC];
    bool ok[SQ * KC];
#pragma unroll
    for (int q = 0; q < SQ; ++q)
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        e[q * KC + c] = a[q] + LW * c + li;
        ok[q * KC + c] = e[q * KC + c] < b[q];
      }
    sm_rows<SQ * KC>(perm, E, e, ok, r);
#pragma unroll
    for (int q = 0; q < SQ; ++q)
#pragma unroll
      for (int c = 0; c < KC; ++c) rk[q][c] = r[q * KC + c];
  }
  // unconditional loads (a lane without a row reads row 0, E >= 1) and the values selected
  // after: loads under a per-lane condition leave the compiler's wait counting unsure which
  // are still in flight, and it then waits before later stores
#pragma unroll
  for (int q = 0; q < SQ; ++q)
#pragma unroll
    for (int c = 0; c < KC; ++c) sm_load<HH>(x, rk[q][c] >= 0 ? rk[q][c] : 0, v[q][c]);
#pragma unroll
  for (int q = 0; q < SQ; ++q)
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int h = 0; h < HH; ++h) v[q][c][h] = rk[q][c] >= 0 ? v[q][c][h] : 0.f;

  // Register-held chunks (c < KC) and the tail of longer segments (c >= KC, rows loaded again
  // per pass) are walked by separate loops, in the same chunk order: the outputs of the register
  // chunks are computed first and stored back to back (interleaving each store with the next
  // chunk's divisions made the compiler wait for every store before the next chunk).
#pragma unroll
  for (int q = 0; q < SQ; ++q) {
    const int nch = uniform_max((b[q] - a[q] + LW - 1) / LW);
    auto row_of = [&](int c) -> int {
      const int e = a[q] + LW * c + li;
      return e < b[q] ? sm_row(perm, E, e) : -1;
    };
    // A NaN score is skipped by the max but makes the segment's sum, and with it every weight
    // of the segment, NaN: the result torch's amax -> exp -> sum -> divide gives.
    float m[HH], z[HH];
#pragma unroll
    for (int h = 0; h < HH; ++h) { m[h] = -__builtin_inff(); z[h] = 0.f; }
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (rk[q][c] >= 0)
#pragma unroll
        for (int h = 0; h < HH; ++h) m[h] = v[q][c][h] > m[h] ? v[q][c][h] : m[h];
    for (int c = KC; c < nch; ++c) {
      const int r = row_of(c);
      if (r >= 0) {
        float t[HH];
        sm_load<HH>(x, r, t);
#pragma unroll
        for (int h = 0; h < HH; ++h) m[h] = t[h] > m[h] ? t[h] : m[h];
      }
    }
#pragma unroll
    for (int h = 0; h < HH; ++h) m[h] = grp_maxf<LW>(m[h]);
    // exponentials of the register-held chunks are computed once, summed and divided
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (c < nch)
#pragma unroll
        for (int h = 0; h < HH; ++h) v[q][c][h] = expf(v[q][c][h] - m[h]);
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (rk[q][c] >= 0)
#pragma unroll
        for (int h = 0; h < HH; ++h) z[h] += v[q][c][h];
    for (int c = KC; c < nch; ++c) {
      const int r = row_of(c);
      if (r >= 0) {
        float t[HH];
        sm_load<HH>(x, r, t);
#pragma unroll
        for (int h = 0; h < HH; ++h) z[h] += expf(t[h] - m[h]);
      }
    }
#pragma unroll
    for (int h = 0; h < HH; ++h) {
      const float zz = grp_sumf<LW>(z[h]);
      z[h] = zz < 1e-8f ? 1e-8f : zz;  // clamp(min=1e-8) keeps NaN, as torch's does
    }
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (c < nch)  // wave-uniform: chunks past the wave's longest segment hold no row
#pragma unroll
        for (int h = 0; h < HH; ++h) v[q][c][h] = v[q][c][h] / z[h];
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (rk[q][c] >= 0) sm_store<HH>(w, rk[q][c], v[q][c]);
    for (int c = KC; c < nch; ++c) {
      const int r = row_of(c);
      if (r < 0) continue;
      float t[HH], o[HH];
      sm_load<HH>(x, r, t);
#pragma unroll
      for (int h = 0; h < HH; ++h) o[h] = expf(t[h] - m[h]) / z[h];
      sm_store<HH>(w, r, o);
    }
  }
  zero_rows_from<float>(w, perm, t0, E, HH);
}

// Backward: the first KC chunks of a segment's rows (g and w) are loaded once into registers
// with all their loads in flight, the dot product is summed in chunk order, and their outputs
// are computed before any is stored; longer segments walk the remaining chunks twice (dot, then
// outputs).  On this GPU loads and stores share one counter, so a load issued after a store
// waits for that store too: interleaving per-chunk loads and stores serialised them.
template <int HH, int LW>
__global__ __launch_bounds__(kSmThreads) void seg_softmax_vec_bwd(
    const float* __restrict__ g_, const float* __restrict__ w, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ ns, const int32_t* __restrict__ ne, int32_t E, int64_t S,
    float* __restrict__ dx, int zero_tail) {
  const int t0 = tail_start(zero_tail, ne, E, S);
  constexpr int SQ = sm_quads<HH, LW>();
  constexpr int KC = 32 / LW;
  const int li = lane_id() & (LW - 1);
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kSmThreads / kWave) + threadIdx.x / kWave;
  int a[SQ], b[SQ], rk[SQ][KC];
  float gv[SQ][KC][HH], wv[SQ][KC][HH];
#pragma unroll
  for (int q = 0; q < SQ; ++q) sm_bounds<LW>(ns, ne, E, S, wave * SQ + q, a[q], b[q]);
  {
    int e[SQ * KC], r[SQ * KC];
    bool ok[SQ * KC];
#pragma unroll
    for (int q = 0; q < SQ; ++q)
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        e[q * KC + c] = a[q] + LW * c + li;
        ok[q * KC + c] = e[q * KC + c] < b[q];
      }
    sm_rows<SQ * KC>(perm, E, e, ok, r);
#pragma unroll
    for (int q = 0; q < SQ; ++q)
#pragma unroll
      for (int c = 0; c < KC; ++c) rk[q][c] = r[q * KC + c];
  }
#pragma unroll
  for (int q = 0; q < SQ; ++q)
#pragma unroll
    for (int c = 0; c < KC; ++c) {  // unconditional, as in the forward
      const int r = rk[q][c] >= 0 ? rk[q][c] : 0;
      sm_load<HH>(g_, r, gv[q][c]);
      sm_load<HH>(w, r, wv[q][c]);
    }
#pragma unroll
  for (int q = 0; q < SQ; ++q)
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int h = 0; h < HH; ++h) {
        gv[q][c][h] = rk[q][c] >= 0 ? gv[q][c][h] : 0.f;
        wv[q][c][h] = rk[q][c] >= 0 ? wv[q][c][h] : 0.f;
      }
#pragma unroll
  for (int q = 0; q < SQ; ++q) {
    const int nch = uniform_max((b[q] - a[q] + LW - 1) / LW);
    auto row_of = [&](int c) -> int {
      const int e = a[q] + LW * c + li;
      return e < b[q] ? sm_row(perm, E, e) : -1;
    };
    float dot[HH];
#pragma unroll
    for (int h = 0; h < HH; ++h) dot[h] = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (rk[q][c] >= 0)
#pragma unroll
        for (int h = 0; h < HH; ++h) dot[h] += gv[q][c][h] * wv[q][c][h];
    for (int c = KC; c < nch; ++c) {
      const int r = row_of(c);
      if (r < 0) continue;
      float gt[HH], wt[HH];
      sm_load<HH>(g_, r, gt);
      sm_load<HH>(w, r, wt);
#pragma unroll
      for (int h = 0; h < HH; ++h) dot[h] += gt[h] * wt[h];
    }
#pragma unroll
    for (int h = 0; h < HH; ++h) dot[h] = grp_sumf<LW>(dot[h]);
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int h = 0; h < HH; ++h) gv[q][c][h] = wv[q][c][h] * (gv[q][c][h] - dot[h]);
#pragma unroll
    for (int c = 0; c < KC; ++c)
      if (rk[q][c] >= 0) sm_store<HH>(dx, rk[q][c], gv[q][c]);
    for (int c = KC; c < nch; ++c) {
      const int r = row_of(c);
      if (r < 0) continue;
      float gt[HH], wt[HH], o[HH];
      sm_load<HH>(g_, r, gt);
      sm_load<HH>(w, r, wt);
#pragma unroll
      for (int h = 0; h < HH; ++h) o[h] = wt[h] * (gt[h] - dot[h]);
      sm_store<HH>(dx, r, o);
    }
  }
  zero_rows_from<float>(dx, perm, t0, E, HH);
}

}  // namespace
}  // namespace geo

using namespace geo;

// Head counts with a vector-row kernel, when every row pointer is aligned to its vector width.
static bool sm_vec_ok(int64_t H, std::initializer_list<const void*> ps) {
  if (H != 1 && H != 2 && H != 4 && H != 8) return false;
  const uintptr_t al = H >= 4 ? 16 : static_cast<uintptr_t>(4 * H);
  for (const void* p : ps)
    if (reinterpret_cast<uintptr_t>(p) % al != 0) return false;
  return true;
}

// Lanes per segment: 8 when segments average at most 12 edges, else 16.
static int sm_lanes(int64_t E, int64_t S) { return E <= 12 * S ? 8 : 16; }

template <template <int, int> class L, int LW, typename... Args>
static void sm_launch_heads(int64_t H, int64_t S, hipStream_t st, Args... args) {
  const int64_t per_wave = (kWave / LW) * ((LW == 8 || H >= 8) ? 1 : 2);
  const dim3 grid(static_cast<unsigned>(ceil_div(S, per_wave * (kSmThreads / kWave))));
  switch (H) {
    case 1: hipLaunchKernelGGL((L<1, LW>::kernel), grid, dim3(kSmThreads), 0, st, args...); break;
    case 2: hipLaunchKernelGGL((L<2, LW>::kernel), grid, dim3(kSmThreads), 0, st, args...); break;
    case 4: hipLaunchKernelGGL((L<4, LW>::kernel), grid, dim3(kSmThreads), 0, st, args...); break;
    default: hipLaunchKernelGGL((L<8, LW>::kernel), grid, dim3(kSmThreads), 0, st, args...); break;
  }
}

template <int HH, int LW>
struct SmFwd {
  static constexpr auto kernel = seg_softmax_vec_fwd<HH, LW>;
};
template <int HH, int LW>
struct SmBwd {
  static constexpr auto kernel = seg_softmax_vec_bwd<HH, LW>;
};

template <template <int, int> class L, typename... Args>
static void sm_launch_vec(int64_t E, int64_t H, int64_t S, hipStream_t st, Args... args) {
  if (sm_lanes(E, S) == 8) sm_launch_heads<L, 8>(H, S, st, args...);
  else sm_launch_heads<L, 16>(H, S, st, args...);
}

static int sm_check(int dtype, int64_t E, int64_t S, int64_t H) {
  GEO_REQUIRE(dtype == GEO_F32 || dtype == GEO_F64, "segment_softmax: dtype must be f32 or f64 (got %d)",
              dtype);
  GEO_REQUIRE(E >= 0 && S >= 0 && H >= 0, "segment_softmax: negative size");
  GEO_REQUIRE(E < 0x7fffffffLL && H < 0x7fffffffLL, "segment_softmax: sizes exceed int32 indexing");
  return GEO_OK;
}

// S == 0 with zero_tail: every row is outside the CSR.
static int sm_zero_all(int dtype, void* out, int64_t E, int64_t H, hipStream_t st) {
  if (dtype == GEO_F32) return device_fill<float>(static_cast<float*>(out), E * H, 0.f, st);
  return device_fill<double>(static_cast<double*>(out), E * H, 0.0, st);
}

extern "C" int geo_segment_softmax_fwd(int dtype, const void* scores, const int32_t* perm,
                                       const int32_t* node_start, const int32_t* node_end,
                                       int64_t E, int64_t S, int64_t H, int zero_tail, void* out,
                                       void* stream) {
  int rc = sm_check(dtype, E, S, H);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  if (H == 0 || E == 0) return GEO_OK;
  GEO_REQUIRE(out, "segment_softmax: null output");
  if (S == 0) return zero_tail ? sm_zero_all(dtype, out, E, H, st) : GEO_OK;
  GEO_REQUIRE(scores && node_start && node_end, "segment_softmax: null pointer");
  const unsigned grid = static_cast<unsigned>(ceil_div(S * H, kSmThreads));
  const int zt = zero_tail ? 1 : 0;
  if (dtype == GEO_F32 && sm_vec_ok(H, {scores, out})) {
    sm_launch_vec<SmFwd>(E, H, S, st, static_cast<const float*>(scores), perm, node_start, node_end,
                         static_cast<int32_t>(E), S, static_cast<float*>(out), zt);
  } else if (dtype == GEO_F32 && H <= kSmRowHeads) {
    const unsigned rgrid = static_cast<unsigned>(ceil_div(S, 4 * (kSmThreads / kWave)));
    hipLaunchKernelGGL(seg_softmax_rows_fwd, dim3(rgrid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(scores), perm, node_start, node_end,
                       static_cast<int32_t>(E), S, static_cast<int32_t>(H), static_cast<float*>(out),
                       zt);
  } else if (dtype == GEO_F32)
    hipLaunchKernelGGL(seg_softmax_fwd_kernel<float>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(scores), perm, node_start, node_end,
                       static_cast<int32_t>(E), S, static_cast<int32_t>(H), static_cast<float*>(out),
                       zt);
  else
    hipLaunchKernelGGL(seg_softmax_fwd_kernel<double>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const double*>(scores), perm, node_start, node_end,
                       static_cast<int32_t>(E), S, static_cast<int32_t>(H), static_cast<double*>(out),
                       zt);
  GEO_LAUNCH_CHECK("seg_softmax_fwd_kernel");
  return GEO_OK;
}

extern "C" int geo_segment_softmax_bwd(int dtype, const void* grad_out, const void* out,
                                       const int32_t* perm, const int32_t* node_start,
                                       const int32_t* node_end, int64_t E, int64_t S, int64_t H,
                                       int zero_tail, void* grad_scores, void* stream) {
  int rc = sm_check(dtype, E, S, H);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  if (H == 0 || E == 0) return GEO_OK;
  GEO_REQUIRE(grad_scores, "segment_softmax_bwd: null output");
  if (S == 0) return zero_tail ? sm_zero_all(dtype, grad_scores, E, H, st) : GEO_OK;
  GEO_REQUIRE(grad_out && out && node_start && node_end, "segment_softmax_bwd: null pointer");
  const unsigned grid = static_cast<unsigned>(ceil_div(S * H, kSmThreads));
  const int zt = zero_tail ? 1 : 0;
  if (dtype == GEO_F32 && sm_vec_ok(H, {grad_out, out, grad_scores})) {
    sm_launch_vec<SmBwd>(E, H, S, st, static_cast<const float*>(grad_out), static_cast<const float*>(out),
                         perm, node_start, node_end, static_cast<int32_t>(E), S,
                         static_cast<float*>(grad_scores), zt);
  } else if (dtype == GEO_F32 && H <= kSmRowHeads) {
    const unsigned rgrid = static_cast<unsigned>(ceil_div(S, 4 * (kSmThreads / kWave)));
    hipLaunchKernelGGL(seg_softmax_rows_bwd, dim3(rgrid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(grad_out), static_cast<const float*>(out), perm,
                       node_start, node_end, static_cast<int32_t>(E), S, static_cast<int32_t>(H),
                       static_cast<float*>(grad_scores), zt);
  } else if (dtype == GEO_F32)
    hipLaunchKernelGGL(seg_softmax_bwd_kernel<float>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const float*>(grad_out), static_cast<const float*>(out), perm,
                       node_start, node_end, static_cast<int32_t>(E), S, static_cast<int32_t>(H),
                       static_cast<float*>(grad_scores), zt);
  else
    hipLaunchKernelGGL(seg_softmax_bwd_kernel<double>, dim3(grid), dim3(kSmThreads), 0, st,
                       static_cast<const double*>(grad_out), static_cast<const double*>(out), perm,
                       node_start, node_end, static_cast<int32_t>(E), S, static_cast<int32_t>(H),
                       static_cast<double*>(grad_scores), zt);
  GEO_LAUNCH_CHECK("seg_softmax_bwd_kernel");
  return GEO_OK;
}
