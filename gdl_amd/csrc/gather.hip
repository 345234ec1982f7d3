// gather.hip — fixed-width weighted gather-sums over KNN neighbourhoods, forward and backward.
//
// The feature pooling / interpolation layers of the reference gather the features of K
// neighbours per output point and sum them with per-neighbour weights, as separate PyTorch
// gathers, broadcasts and reductions over an [N_out, K, C] temporary
// (geoembodied/nn/modules/equivariant_interp.py:95-125, equivariant_pool.py:412-471,
// equivariant_skip_fusion.py:304-320):
//
//   out[n, :] = sum_k w[n, k] * feat[idx[n, k], :]        (idx < 0: no neighbour, skipped)
//
// Here it is one pass without the temporary.  A row of C features is read as 16-byte (or
// narrower) vectors by L lanes, a wave holds R = 64/L output rows, and the K neighbour rows of
// an output row are loaded together (all in flight at once) and summed in ascending k order.
// Workgroups take their rows through xcd_block(): each XCD serves one contiguous range of
// output rows (of source rows in the feature backward), so the feature rows gathered by the
// points of one cloud are fetched from HBM into one XCD's L2 rather than into all eight.
// geo_idw_weights computes the interpolation layer's inverse-distance weights
// (equivariant_interp.py:95-99).  The backward is two kernels: grad_w[n, k] =
// <grad_out[n], feat[idx[n, k]]> (one lane group per output row, a group-wide dot product) and
// grad_feat[j] = sum over the (n, k) with idx[n, k] = j of w[n, k] grad_out[n], walked over the
// CSR of idx (built by geo_csr_build), so every source row is written once, without atomics.
#include "scan.hpp"

namespace geo {
namespace {

constexpr int kGwThreads = 256;
constexpr int kGwWaves = kGwThreads / kWave;
constexpr int kGwMaxK = 32;

template <typename T> struct GwAcc { using type = float; };
template <> struct GwAcc<double> { using type = double; };

__device__ __forceinline__ float gw_to(float x) { return x; }
__device__ __forceinline__ float gw_to(uint16_t x) { return bf16_to_f32(x); }
__device__ __forceinline__ double gw_to(double x) { return x; }
template <typename T> __device__ __forceinline__ T gw_from(float x);
template <> __device__ __forceinline__ float gw_from<float>(float x) { return x; }
template <> __device__ __forceinline__ uint16_t gw_from<uint16_t>(float x) { return f32_to_bf16(x); }
template <typename T> __device__ __forceinline__ T gw_from(double x);
template <> __device__ __forceinline__ double gw_from<double>(double x) { return x; }

template <int VB> struct GwRaw;
template <> struct GwRaw<16> { using type = uint4; };
template <> struct GwRaw<8> { using type = uint2; };
template <> struct GwRaw<4> { using type = uint32_t; };
template <> struct GwRaw<2> { using type = uint16_t; };

template <typename T, int VB>
struct GwVec {
  static constexpr int EPV = VB / static_cast<int>(sizeof(T));
  union {
    typename GwRaw<VB>::type raw;
    T e[EPV];
  };
  __device__ __forceinline__ void load(const T* p) { raw = *reinterpret_cast<const typename GwRaw<VB>::type*>(p); }
  __device__ __forceinline__ void store(T* p) const { *reinterpret_cast<typename GwRaw<VB>::type*>(p) = raw; }
};

// Weights of (equivariant_interp.py:95-99): inverse of sqrt(max(d, 1e-4)) for valid neighbours
// (idx >= 0), normalised by the row sum clamped at 1e-8.  One thread per output row; the fused
// interpolation computes them with the same helpers in the same order.
__device__ __forceinline__ float idw_inv(int64_t j, float d) {
  return j >= 0 ? 1.0f / sqrtf(d < 1e-4f ? 1e-4f : d) : 0.0f;
}
__device__ __forceinline__ float idw_den(float sum) { return sum < 1e-8f ? 1e-8f : sum; }

// The weight as the gather uses it: rounded to the feature type first, as the two-step path
// converts the float32 weights to the features' dtype before the gather.
template <typename T> __device__ __forceinline__ typename GwAcc<T>::type idw_as(float w);
template <> __device__ __forceinline__ float idw_as<float>(float w) { return w; }
template <> __device__ __forceinline__ float idw_as<uint16_t>(float w) { return bf16_to_f32(f32_to_bf16(w)); }
template <> __device__ __forceinline__ double idw_as<double>(float w) { return static_cast<double>(w); }

__global__ void idw_weights_kernel(const int64_t* __restrict__ idx, const float* __restrict__ dist,
                                   int64_t N_out, int K, float* __restrict__ w) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (n >= N_out) return;
  const int64_t* ir = idx + n * K;
  const float* dr = dist + n * K;
  // loads in chunks of eight at clamped columns, values used for k < K only (a load under
  // `k < K` became a branch and a wait before the next one)
  float inv[kGwMaxK];
  float sum = 0.f;
#pragma unroll
  for (int k0 = 0; k0 < kGwMaxK; k0 += 8) {
    if (k0 >= K) break;  // uniform across the chunk's loads
    int64_t jv[8];
    float dv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int kc = k0 + k < K ? k0 + k : K - 1;
      jv[k] = ir[kc];
      dv[k] = dr[kc];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k0 + k < K) {
        const float v = idw_inv(jv[k], dv[k]);
        inv[k0 + k] = v;
        sum += v;
      }
    }
  }
  const float den = idw_den(sum);
#pragma unroll
  for (int k = 0; k < kGwMaxK; ++k)
    if (k < K) w[n * K + k] = inv[k] / den;
}

// A wave serves RP blocks of R consecutive output rows, (wave * RP + r) * R + g for r < RP: with
// RP > 1 (K <= 4) the neighbour rows of all RP rows of a lane group are requested together, so
// more loads are in flight per wave and fewer waves are dispatched.  With `dist` (fused IDW
// interpolation) the weights are computed from the squared distances instead of read from `w`,
// once the group's first feature loads are in flight, and written to w_out (float32) by the
// group's first lane.
template <typename T, int VB, int KK, int RP>
__global__ __launch_bounds__(kGwThreads) void gws_fwd_kernel(
    const T* __restrict__ feat, int64_t N_src, int64_t C, const int64_t* __restrict__ idx,
    const T* __restrict__ w, int64_t N_out, int K, int vpr, int log_l, T* __restrict__ out,
    const float* __restrict__ dist, float* __restrict__ w_out) {
  static_assert(RP == 1 || KK <= 4, "several rows per group only for K <= 4");
  using A = typename GwAcc<T>::type;
  using V = GwVec<T, VB>;
  constexpr int EPV = V::EPV;
  const int lane = lane_id();
  const int L = 1 << log_l;
  const int R = kWave >> log_l;
  const int g = lane >> log_l;
  const int vl = lane & (L - 1);
  const int64_t wb = (xcd_block() * kGwWaves + threadIdx.x / kWave) * RP;
  int64_t n[RP];
#pragma unroll
  for (int r = 0; r < RP; ++r) n[r] = (wb + r) * R + g;
  if (n[0] >= N_out) return;  // rows grow with r: nothing for this group
  // src: the source row, -1 for idx < 0, -2 for idx >= N_src (a neighbour for the IDW weights,
  // which count every idx >= 0, but none for the gather, which reads rows src >= 0 only)
  int32_t src[RP][KK];
  A wk[RP][KK];
  float dk[RP][KK];   // fused IDW: the squared distances
  // every load unconditional (row and column clamped into range, K >= 1, n[0] < N_out) and
  // the values selected afterwards: a load under a per-lane condition becomes a branch and a
  // wait for its data before the next load
  // (in chunks of at most 8 neighbours, which bounds the registers the 64-bit indices hold)
  auto at = [&](int r, int k) -> int64_t {
    return (n[r] < N_out ? n[r] : n[0]) * K + (k < K ? k : K - 1);
  };
  constexpr int PC = KK < 8 ? KK : 8;
#pragma unroll
  for (int k0 = 0; k0 < KK; k0 += PC) {
    int64_t jr[RP][PC];
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
      for (int k = 0; k < PC; ++k) jr[r][k] = idx[at(r, k0 + k)];
    if (dist == nullptr) {
#pragma unroll
      for (int r = 0; r < RP; ++r)
#pragma unroll
        for (int k = 0; k < PC; ++k) wk[r][k0 + k] = gw_to(w[at(r, k0 + k)]);
    } else {
#pragma unroll
      for (int r = 0; r < RP; ++r)
#pragma unroll
        for (int k = 0; k < PC; ++k) dk[r][k0 + k] = dist[at(r, k0 + k)];
    }
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
      for (int k = 0; k < PC; ++k) {
        const bool in = k0 + k < K && n[r] < N_out;
        const int64_t j = in ? jr[r][k] : -1;
        const bool ok = j >= 0 && j < N_src;
        src[r][k0 + k] = ok ? static_cast<int32_t>(j) : (j >= 0 ? -2 : -1);
        if (dist == nullptr) {
          wk[r][k0 + k] = ok ? wk[r][k0 + k] : A(0);
        } else {
          dk[r][k0 + k] = in ? dk[r][k0 + k] : 0.f;
        }
      }
  }
  // the IDW weights of the group's rows (geo_idw_weights' operations in its order); called
  // once, after the first feature loads are issued
  bool need_w = dist != nullptr;
  auto idw_fill = [&]() {
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      float inv[KK];
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < KK; ++k) {
        inv[k] = k < K ? idw_inv(src[r][k] != -1 ? 0 : -1, dk[r][k]) : 0.f;
        sum += inv[k];  // k < K only: the others add 0
      }
      const float den = idw_den(sum);
#pragma unroll
      for (int k = 0; k < KK; ++k) {
        const float wf = inv[k] / den;
        if (vl == 0 && k < K && n[r] < N_out) w_out[n[r] * K + k] = wf;
        wk[r][k] = src[r][k] >= 0 ? idw_as<T>(wf) : A(0);
      }
    }
    need_w = false;
  };
  constexpr int KC = KK < 8 ? KK : 8;  // neighbour rows in flight at once (RP == 1)
  for (int vb = vl; vb < vpr; vb += L) {
    const int64_t col = static_cast<int64_t>(vb) * EPV;
    if constexpr (RP == 1) {
      A acc[EPV];
#pragma unroll
      for (int i = 0; i < EPV; ++i) acc[i] = A(0);
#pragma unroll
      for (int k0 = 0; k0 < KK; k0 += KC) {
        V buf[KC];
#pragma unroll
        for (int k = 0; k < KC; ++k)
          buf[k].load(feat + static_cast<int64_t>(src[0][k0 + k] >= 0 ? src[0][k0 + k] : 0) * C + col);
        if (need_w) idw_fill();
#pragma unroll
        for (int k = 0; k < KC; ++k) {
#pragma unroll
          for (int i = 0; i < EPV; ++i)
            acc[i] += src[0][k0 + k] >= 0 ? wk[0][k0 + k] * gw_to(buf[k].e[i]) : A(0);
        }
      }
      V res;
#pragma unroll
      for (int i = 0; i < EPV; ++i) res.e[i] = gw_from<T>(acc[i]);
      res.store(out + n[0] * C + col);
    } else {
      V buf[RP][KK];
#pragma unroll
      for (int r = 0; r < RP; ++r)
#pragma unroll
        for (int k = 0; k < KK; ++k)
          buf[r][k].load(feat + static_cast<int64_t>(src[r][k] >= 0 ? src[r][k] : 0) * C + col);
      if (need_w) idw_fill();
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        A acc[EPV];
#pragma unroll
        for (int i = 0; i < EPV; ++i) acc[i] = A(0);
#pragma unroll
        for (int k = 0; k < KK; ++k) {
#pragma unroll
          for (int i = 0; i < EPV; ++i)
            acc[i] += src[r][k] >= 0 ? wk[r][k] * gw_to(buf[r][k].e[i]) : A(0);
        }
        V res;
#pragma unroll
        for (int i = 0; i < EPV; ++i) res.e[i] = gw_from<T>(acc[i]);
        if (n[r] < N_out) res.store(out + n[r] * C + col);
      }
    }
  }
}

// grad_w[n, k] = <grad_out[n], feat[idx[n, k]]>; the L lanes of a row's group reduce with xor
// shuffles inside the group.
template <typename T, int VB, int KK>
__global__ __launch_bounds__(kGwThreads) void gws_bwd_w_kernel(
    const T* __restrict__ grad_out, const T* __restrict__ feat, int64_t N_src, int64_t C,
    const int64_t* __restrict__ idx, int64_t N_out, int K, int vpr, int log_l, T* __restrict__ grad_w) {
  using A = typename GwAcc<T>::type;
  using V = GwVec<T, VB>;
  constexpr int EPV = V::EPV;
  const int lane = lane_id();
  const int L = 1 << log_l;
  const int R = kWave >> log_l;
  const int g = lane >> log_l;
  const int vl = lane & (L - 1);
  int64_t n = (xcd_block() * kGwWaves + threadIdx.x / kWave) * R + g;
  const bool live = n < N_out;  // dead groups still take part in the shuffles below
  if (!live) n = N_out - 1;
  int32_t src[KK];
#pragma unroll
  for (int k = 0; k < KK; ++k) {  // unconditional loads (column clamped), values selected after
    const int64_t jr = idx[n * K + (k < K ? k : K - 1)];
    const int64_t j = k < K ? jr : -1;
    src[k] = (j >= 0 && j < N_src) ? static_cast<int32_t>(j) : -1;
  }
  A dot[KK];
#pragma unroll
  for (int k = 0; k < KK; ++k) dot[k] = A(0);
  for (int vb0 = 0; vb0 < vpr; vb0 += L) {
    const int vb = vb0 + vl;
    const bool cok = vb < vpr;
    const int64_t col = cok ? static_cast<int64_t>(vb) * EPV : 0;
    V go;
    go.load(grad_out + n * C + col);
    constexpr int KC = KK < 8 ? KK : 8;
#pragma unroll
    for (int k0 = 0; k0 < KK; k0 += KC) {
      V buf[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k)
        buf[k].load(feat + static_cast<int64_t>(src[k0 + k] >= 0 ? src[k0 + k] : 0) * C + col);
#pragma unroll
      for (int k = 0; k < KC; ++k) {
#pragma unroll
        for (int i = 0; i < EPV; ++i)
          dot[k0 + k] += cok ? gw_to(go.e[i]) * gw_to(buf[k].e[i]) : A(0);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < KK; ++k) {
    for (int m = 1; m < L; m <<= 1) dot[k] += __shfl_xor(dot[k], m, kWave);
  }
  if (live && vl == 0) {
#pragma unroll
    for (int k = 0; k < KK; ++k)
      if (k < K) grad_w[n * K + k] = gw_from<T>(src[k] >= 0 ? dot[k] : A(0));
  }
}

// grad_feat[j] = sum over CSR entries e of source j (flat position p = perm[e], n = p / K) of
// w[p] * grad_out[n]; 4 entries per group in flight.
template <typename T, int VB>
__global__ __launch_bounds__(kGwThreads) void gws_bwd_feat_kernel(
    const T* __restrict__ grad_out, const T* __restrict__ w, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ ns, const int32_t* __restrict__ ne, int64_t N_src, int64_t C,
    int64_t N_out, int K, int vpr, int log_l, T* __restrict__ grad_feat) {
  using A = typename GwAcc<T>::type;
  using V = GwVec<T, VB>;
  constexpr int EPV = V::EPV;
  constexpr int U = 4;
  const int lane = lane_id();
  const int L = 1 << log_l;
  const int R = kWave >> log_l;
  const int g = lane >> log_l;
  const int vl = lane & (L - 1);
  const int64_t j = (xcd_block() * kGwWaves + threadIdx.x / kWave) * R + g;
  if (j >= N_src) return;
  const int64_t P = N_out * K;
  int64_t a = ns[j], b = ne[j];
  a = a < 0 ? 0 : (a > P ? P : a);
  b = b < a ? a : (b > P ? P : b);
  for (int vb = vl; vb < vpr; vb += L) {
    const int64_t col = static_cast<int64_t>(vb) * EPV;
    A acc[EPV];
#pragma unroll
    for (int i = 0; i < EPV; ++i) acc[i] = A(0);
    for (int64_t e0 = a; e0 < b; e0 += U) {
      int64_t p[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t e = e0 + u < b ? e0 + u : b - 1;
        const int64_t q = perm[e];
        p[u] = (q >= 0 && q < P) ? q : -1;
      }
      V buf[U];
      A wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = e0 + u < b && p[u] >= 0;
        buf[u].load(grad_out + (ok ? p[u] / K : 0) * C + col);
        wv[u] = ok ? gw_to(w[p[u]]) : A(0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = e0 + u < b && p[u] >= 0;
#pragma unroll
        for (int i = 0; i < EPV; ++i) acc[i] += ok ? wv[u] * gw_to(buf[u].e[i]) : A(0);
      }
    }
    V res;
#pragma unroll
    for (int i = 0; i < EPV; ++i) res.e[i] = gw_from<T>(acc[i]);
    res.store(grad_feat + j * C + col);
  }
}

struct GwLayout {
  int vb, vpr, log_l;
};

GwLayout gw_layout(int64_t C, int esize, uintptr_t align_bits) {
  const int64_t row_bytes = C * esize;
  int vb = 16;
  while (vb > esize && ((row_bytes % vb) != 0 || (align_bits % vb) != 0)) vb >>= 1;
  GwLayout l;
  l.vb = vb;
  l.vpr = static_cast<int>(row_bytes / vb);
  int lanes = 1, lg = 0;
  while (lanes < l.vpr && lanes < kWave) { lanes <<= 1; ++lg; }
  l.log_l = lg;
  return l;
}

int gw_esize(int dtype) { return dtype == GEO_F32 ? 4 : dtype == GEO_BF16 ? 2 : 8; }

// Zeroes n elements with a fill kernel (no memset nodes, so callers may capture it in a graph).
int gw_zero(int dtype, void* p, int64_t n, hipStream_t st) {
  if (dtype == GEO_F32) return device_fill<float>(static_cast<float*>(p), n, 0.f, st);
  if (dtype == GEO_BF16) return device_fill<uint16_t>(static_cast<uint16_t*>(p), n, 0, st);
  return device_fill<double>(static_cast<double*>(p), n, 0.0, st);
}

unsigned gw_blocks(int64_t rows, int log_l, int rp = 1) {
  const int64_t per_block = static_cast<int64_t>(kGwWaves) * (kWave >> log_l) * rp;
  return static_cast<unsigned>(ceil_div(rows, per_block));
}

// Dispatch on the vector width, then on K rounded up to 1, 2, 3, 4, 8, 16 or 32 neighbours.
#define GEO_GW_K_SWITCH(KVAR, BODY)                   \
  do {                                                \
    if (KVAR <= 1) { constexpr int KK = 1; BODY; }    \
    else if (KVAR <= 2) { constexpr int KK = 2; BODY; } \
    else if (KVAR <= 3) { constexpr int KK = 3; BODY; } \
    else if (KVAR <= 4) { constexpr int KK = 4; BODY; } \
    else if (KVAR <= 8) { constexpr int KK = 8; BODY; } \
    else if (KVAR <= 16) { constexpr int KK = 16; BODY; } \
    else { constexpr int KK = 32; BODY; }            \
  } while (0)

// Output rows per lane group of the forward kernel: two when each wave would otherwise carry
// little work (K <= 4) and enough waves remain to fill the chip (C2 interpolation, K = 3:
// 14.5 -> 13.6 us; four rows per group 14.6 us).
int gw_rows_per_group(int64_t N_out, int log_l, int K) {
  if (K > 4) return 1;
  const int64_t waves = ceil_div(N_out, static_cast<int64_t>(kWave >> log_l));  // at one row
  return waves >= 2 * 8192 ? 2 : 1;
}

template <typename T, int VBV, int KK>
void gws_fwd_launch(int rp, int log_l, hipStream_t st, const T* feat, int64_t N_src, int64_t C,
                    const int64_t* idx, const T* w, int64_t N_out, int K, int vpr, T* out,
                    const float* dist, float* w_out) {
  if constexpr (KK <= 4) {
    if (rp == 2) {
      hipLaunchKernelGGL((gws_fwd_kernel<T, VBV, KK, 2>), dim3(gw_blocks(N_out, log_l, 2)),
                         dim3(kGwThreads), 0, st, feat, N_src, C, idx, w, N_out, K, vpr, log_l, out,
                         dist, w_out);
      return;
    }
  }
  hipLaunchKernelGGL((gws_fwd_kernel<T, VBV, KK, 1>), dim3(gw_blocks(N_out, log_l)),
                     dim3(kGwThreads), 0, st, feat, N_src, C, idx, w, N_out, K, vpr, log_l, out,
                     dist, w_out);
}

// The forward gather; with `dist` the IDW weights are computed in the kernel (w unused) and
// written to w_out.
template <typename T>
int gws_fwd(const GwLayout& lay, const T* feat, int64_t N_src, int64_t C, const int64_t* idx,
            const T* w, int64_t N_out, int K, T* out, hipStream_t st,
            const float* dist = nullptr, float* w_out = nullptr) {
  const int rp = gw_rows_per_group(N_out, lay.log_l, K);
#define GEO_GW_FWD(VBV)                                                                      \
  case VBV:                                                                                  \
    if constexpr (VBV >= static_cast<int>(sizeof(T))) {                                      \
      GEO_GW_K_SWITCH(K, (gws_fwd_launch<T, VBV, KK>(rp, lay.log_l, st, feat, N_src, C, idx, \
                                                      w, N_out, K, lay.vpr, out, dist,       \
                                                      w_out)));                              \
    }                                                                                        \
    break;
  switch (lay.vb) {
    GEO_GW_FWD(16) GEO_GW_FWD(8) GEO_GW_FWD(4) GEO_GW_FWD(2)
    default: return set_error(GEO_ERR_INVALID, "gather: unsupported vector width %d", lay.vb);
  }
#undef GEO_GW_FWD
  GEO_LAUNCH_CHECK("gws_fwd_kernel");
  return GEO_OK;
}

template <typename T>
int gws_bwd(const GwLayout& lay, const T* grad_out, const T* feat, const T* w, const int64_t* idx,
            int64_t N_src, int64_t C, int64_t N_out, int K, const int32_t* perm,
            const int32_t* ns, const int32_t* ne, T* grad_feat, T* grad_w, hipStream_t st) {
#define GEO_GW_BWD(VBV)                                                                          \
  case VBV:                                                                                      \
    if constexpr (VBV >= static_cast<int>(sizeof(T))) {                                          \
      if (grad_w)                                                                                \
        GEO_GW_K_SWITCH(K, hipLaunchKernelGGL((gws_bwd_w_kernel<T, VBV, KK>),                    \
                                              dim3(gw_blocks(N_out, lay.log_l)), dim3(kGwThreads), \
                                              0, st, grad_out, feat, N_src, C, idx, N_out, K,    \
                                              lay.vpr, lay.log_l, grad_w));                      \
      if (grad_feat)                                                                             \
        hipLaunchKernelGGL((gws_bwd_feat_kernel<T, VBV>), dim3(gw_blocks(N_src, lay.log_l)),     \
                           dim3(kGwThreads), 0, st, grad_out, w, perm, ns, ne, N_src, C, N_out,  \
                           K, lay.vpr, lay.log_l, grad_feat);                                    \
    }                                                                                            \
    break;
  switch (lay.vb) {
    GEO_GW_BWD(16) GEO_GW_BWD(8) GEO_GW_BWD(4) GEO_GW_BWD(2)
    default: return set_error(GEO_ERR_INVALID, "gather: unsupported vector width %d", lay.vb);
  }
#undef GEO_GW_BWD
  GEO_LAUNCH_CHECK("gws_bwd kernels");
  return GEO_OK;
}

}  // namespace
}  // namespace geo

using namespace geo;

static int gw_check(int dtype, int64_t N_src, int64_t C, int64_t N_out, int64_t K) {
  GEO_REQUIRE(dtype == GEO_F32 || dtype == GEO_BF16 || dtype == GEO_F64,
              "gather: unknown dtype code %d", dtype);
  GEO_REQUIRE(N_src >= 0 && C >= 0 && N_out >= 0 && K >= 0, "gather: negative size");
  GEO_REQUIRE(K <= kGwMaxK, "gather: K=%lld above the supported maximum of %d", (long long)K,
              kGwMaxK);
  GEO_REQUIRE(N_out * K < 0x7fffffffLL && N_src < 0x7fffffffLL,
              "gather: N_out * K or N_src exceeds int32 indexing");
  return GEO_OK;
}

extern "C" int geo_idw_weights(const int64_t* idx, const float* dist, int64_t N_out, int64_t K,
                               float* w, void* stream) {
  GEO_REQUIRE(N_out >= 0 && K >= 0 && K <= kGwMaxK, "idw_weights: bad size (N_out=%lld K=%lld)",
              (long long)N_out, (long long)K);
  if (N_out == 0 || K == 0) return GEO_OK;
  GEO_REQUIRE(idx && dist && w, "idw_weights: null pointer");
  hipLaunchKernelGGL(idw_weights_kernel, dim3(static_cast<unsigned>(ceil_div(N_out, 256))), dim3(256),
                     0, as_stream(stream), idx, dist, N_out, static_cast<int>(K), w);
  GEO_LAUNCH_CHECK("idw_weights_kernel");
  return GEO_OK;
}

extern "C" int geo_gather_weighted_sum(int dtype, const void* feat, int64_t N_src, int64_t C,
                                       const int64_t* idx, const void* w, int64_t N_out, int64_t K,
                                       void* out, void* stream) {
  int rc = gw_check(dtype, N_src, C, N_out, K);
  if (rc) return rc;
  if (N_out == 0 || C == 0) return GEO_OK;
  GEO_REQUIRE(out != nullptr, "gather: null output");
  if (K == 0 || N_src == 0) return gw_zero(dtype, out, N_out * C, as_stream(stream));
  GEO_REQUIRE(feat && idx && w, "gather: null input");
  const uintptr_t bits = reinterpret_cast<uintptr_t>(feat) | reinterpret_cast<uintptr_t>(out);
  const GwLayout lay = gw_layout(C, gw_esize(dtype), bits);
  hipStream_t st = as_stream(stream);
  const int k = static_cast<int>(K);
  if (dtype == GEO_F32)
    return gws_fwd<float>(lay, static_cast<const float*>(feat), N_src, C, idx,
                          static_cast<const float*>(w), N_out, k, static_cast<float*>(out), st);
  if (dtype == GEO_BF16)
    return gws_fwd<uint16_t>(lay, static_cast<const uint16_t*>(feat), N_src, C, idx,
                             static_cast<const uint16_t*>(w), N_out, k, static_cast<uint16_t*>(out), st);
  return gws_fwd<double>(lay, static_cast<const double*>(feat), N_src, C, idx,
                         static_cast<const double*>(w), N_out, k, static_cast<double*>(out), st);
}

extern "C" int geo_idw_interpolate(int dtype, const void* feat, int64_t N_src, int64_t C,
                                   const int64_t* idx, const float* dist, int64_t N_out, int64_t K,
                                   void* out, float* w_out, void* stream) {
  int rc = gw_check(dtype, N_src, C, N_out, K);
  if (rc) return rc;
  if (N_out == 0) return GEO_OK;
  GEO_REQUIRE(idx && dist && w_out, "idw_interpolate: null idx, dist or w_out");
  GEO_REQUIRE(C == 0 || out != nullptr, "idw_interpolate: null output");
  hipStream_t st = as_stream(stream);
  if (K == 0 || N_src == 0 || C == 0) {  // the weights alone, as geo_idw_weights computes them
    rc = geo_idw_weights(idx, dist, N_out, K, w_out, stream);
    if (rc || C == 0) return rc;
    return gw_zero(dtype, out, N_out * C, st);
  }
  GEO_REQUIRE(feat != nullptr, "idw_interpolate: null feat");
  const uintptr_t bits = reinterpret_cast<uintptr_t>(feat) | reinterpret_cast<uintptr_t>(out);
  const GwLayout lay = gw_layout(C, gw_esize(dtype), bits);
  const int k = static_cast<int>(K);
  if (dtype == GEO_F32)
    return gws_fwd<float>(lay, static_cast<const float*>(feat), N_src, C, idx, nullptr, N_out, k,
                          static_cast<float*>(out), st, dist, w_out);
  if (dtype == GEO_BF16)
    return gws_fwd<uint16_t>(lay, static_cast<const uint16_t*>(feat), N_src, C, idx, nullptr, N_out,
                             k, static_cast<uint16_t*>(out), st, dist, w_out);
  return gws_fwd<double>(lay, static_cast<const double*>(feat), N_src, C, idx, nullptr, N_out, k,
                         static_cast<double*>(out), st, dist, w_out);
}

extern "C" int geo_gather_weighted_sum_bwd(int dtype, const void* grad_out, const void* feat,
                                           const void* w, const int64_t* idx, int64_t N_src,
                                           int64_t C, int64_t N_out, int64_t K,
                                           const int32_t* perm, const int32_t* node_start,
                                           const int32_t* node_end, void* grad_feat,
                                           void* grad_w, void* stream) {
  int rc = gw_check(dtype, N_src, C, N_out, K);
  if (rc) return rc;
  GEO_REQUIRE(grad_feat == nullptr || (w && perm && node_start && node_end),
              "gather_bwd: grad_feat needs w and the CSR of idx");
  GEO_REQUIRE(grad_w == nullptr || (feat && idx), "gather_bwd: grad_w needs feat and idx");
  if (C == 0 || (N_out == 0 && N_src == 0)) return GEO_OK;
  hipStream_t st = as_stream(stream);
  const int es = gw_esize(dtype);
  if (N_out == 0 || K == 0) {  // nothing flows: zero the gradients that were asked for
    return grad_feat ? gw_zero(dtype, grad_feat, N_src * C, st) : GEO_OK;
  }
  GEO_REQUIRE(grad_out != nullptr, "gather_bwd: null grad_out");
  if (N_src == 0) {
    return grad_w ? gw_zero(dtype, grad_w, N_out * K, st) : GEO_OK;
  }
  uintptr_t bits = reinterpret_cast<uintptr_t>(grad_out) | reinterpret_cast<uintptr_t>(feat) |
                   reinterpret_cast<uintptr_t>(grad_feat);
  const GwLayout lay = gw_layout(C, es, bits);
  const int k = static_cast<int>(K);
  if (dtype == GEO_F32)
    return gws_bwd<float>(lay, static_cast<const float*>(grad_out), static_cast<const float*>(feat),
                          static_cast<const float*>(w), idx, N_src, C, N_out, k, perm, node_start,
                          node_end, static_cast<float*>(grad_feat), static_cast<float*>(grad_w), st);
  if (dtype == GEO_BF16)
    return gws_bwd<uint16_t>(lay, static_cast<const uint16_t*>(grad_out),
                             static_cast<const uint16_t*>(feat), static_cast<const uint16_t*>(w),
                             idx, N_src, C, N_out, k, perm, node_start, node_end,
                             static_cast<uint16_t*>(grad_feat), static_cast<uint16_t*>(grad_w), st);
  return gws_bwd<double>(lay, static_cast<const double*>(grad_out), static_cast<const double*>(feat),
                         static_cast<const double*>(w), idx, N_src, C, N_out, k, perm, node_start,
                         node_end, static_cast<double*>(grad_feat), static_cast<double*>(grad_w), st);
}
