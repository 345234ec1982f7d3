// se3_message.hip — SE(3)-equivariant message passing with the aggregation folded in front of
// the channel mixing.
//
// The reference (geoembodied/nn/modules/se3_conv.py:61-235 `_compute_messages`, :516-545) builds
// one message per edge e = (m -> n) for up to nine tensor-product paths, each of the form
//     msg_e = r_e,p * W_p * x_e,p        (r_e,p: a per-edge scalar, x_e,p: a per-edge feature)
// with a weight matrix W_p shared by all edges, concatenates the messages into an [E, C] tensor
// and sums it over the edges of each target.  Because W_p is shared,
//     sum_e r_e,p W_p x_e,p = W_p (sum_e r_e,p x_e,p),
// so this library sums the r-weighted source features per target first (se3_fwd_aggregate: one
// wave per target node, lanes over input channels, no per-edge tensor) and applies the weights
// once per node with an fp32 MFMA GEMM whose epilogue divides by the node's average degree, adds
// the scalar bias and applies the mask (se3_gemm).  The per-edge GEMM work of the reference
// becomes per-node work (E/N times fewer flops) and the [E, C] message tensor never exists.
//
// Paths (source features s [N,Cs], v [N,Cv,3], t [N,Ct,5]; d = unit direction, y0 = Y_0^0,
// y2 = Y_2 of the edge; r_p = R[e, col_p]; cg = the Cartesian CG(1,1->2) table [3][3][5]):
//   0  s -> s    r0 y0 s               3  v -> s    r3 (d . v)           6  t -> t   r6 y0 t
//   1  s -> v    r1 d_k s              4  v -> v    r4 (d x v)_k         7  v -> t   r7 sum_ij d_i v_j cg_ijm
//   2  v -> v    r2 y0 v_k             5  s -> t    r5 y2_m s            8  t -> s   r8 sum_m t_m^2
//
// Per-node aggregate layout (rows zero-padded to a multiple of 16 floats):
//   Xs[n]    = [A0 (Cs) | A3 (Cv) | A8 (Ct)]                    -> s_out = Xs Ws^T, Ws = [W0|W3|W8]
//   Xv[n][k] = [A1_k (Cs) | A2_k (Cv) | A4_k (Cv)]   k = x,y,z  -> v_out = Xv Wv^T, Wv = [W1|W2|W4]
//   Xt[n][m] = [A5_m (Cs) | A6_m (Ct) | A7_m (Cv)]   m = 0..4   -> t_out = Xt Wt^T, Wt = [W5|W6|W7]
//
// The backward is the same structure transposed: se3_bwd_edge forms the per-edge gradients of
// R, the direction and Y from the per-node gradient rows gX = g W (one wave per target node) and
// se3_bwd_src sums the gradient rows of each source's targets with the per-edge weights (one wave
// per source node over the CSR of the sources), after which GEMMs with the transposed weights
// give the feature gradients.
#include <type_traits>

#include "common.hpp"

// The library is built with -ffp-contract=off because the geometry kernels must round like the
// reference's distance expressions.  These sums are compared within a tolerance instead, so here
// a multiply feeding an add may be fused (one rounding instead of two).
#pragma clang fp contract(fast)

namespace geo {
namespace {

constexpr int kSeThreads = 256;
constexpr int kSeWaves = kSeThreads / kWave;
constexpr int kSePaths = 9;

struct SeEdges {
  const int64_t* other;   // source of each edge (forward, edge grads) or target (source pass)
  const int32_t* perm;    // CSR position -> edge id
  const int32_t* ns;
  const int32_t* ne;
  int32_t E;
  int64_t N;
  const float* dir;       // [E, 3]
  const float* Y;         // [E, ysh]
  int32_t ysh;
  const float* R;         // [E, P]
  int32_t P;
  int32_t pc[kSePaths];   // column of R for each path, -1 when the path is off
  const float* cg;        // [3][3][5] device array; NULL when path 7 is off
};

struct SeFeat {
  const float* s;
  const float* v;
  const float* t;
  int32_t Cs, Cv, Ct;
};

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float rlane(float x, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), j));
}

// The scalars of one edge: the other endpoint, R of every path (0 for paths that are off), the
// direction and Y_0^0 / Y_2.
struct EdgeScalars {
  int32_t other;
  int32_t e;
  int32_t ok;
  float r[kSePaths];
  float d[3];
  float y0;
  float y2[5];
};

// Each lane loads the scalars of the edge at its CSR position `pos` (when `valid`), so the
// edges of a node are fetched in one round of parallel loads; the edge loops then read them
// from lane j with v_readlane (uniform j) or a lane shuffle (per-row j).
__device__ __forceinline__ EdgeScalars stage_edges_at(const SeEdges& g, int pos, bool valid) {
  EdgeScalars q;
  q.other = 0;
  q.e = 0;
  q.ok = 0;
#pragma unroll
  for (int i = 0; i < kSePaths; ++i) q.r[i] = 0.f;
  q.d[0] = q.d[1] = q.d[2] = 0.f;
  q.y0 = 0.f;
#pragma unroll
  for (int m = 0; m < 5; ++m) q.y2[m] = 0.f;
  if (valid) {
    const int e = g.perm ? g.perm[pos] : pos;
    if (static_cast<unsigned>(e) < static_cast<unsigned>(g.E)) {
      const int64_t o = g.other[e];
      if (o >= 0 && o < g.N) {
        q.ok = 1;
        q.other = static_cast<int32_t>(o);
        q.e = e;
        const float* rr = g.R + static_cast<int64_t>(e) * g.P;
#pragma unroll
        for (int i = 0; i < kSePaths; ++i) q.r[i] = g.pc[i] >= 0 ? rr[g.pc[i]] : 0.f;
        const float* dd = g.dir + 3 * static_cast<int64_t>(e);
        q.d[0] = dd[0];
        q.d[1] = dd[1];
        q.d[2] = dd[2];
        const float* y = g.Y + static_cast<int64_t>(e) * g.ysh;
        q.y0 = y[0];
        if (g.ysh >= 9) {
#pragma unroll
          for (int m = 0; m < 5; ++m) q.y2[m] = y[4 + m];
        }
      }
    }
  }
  return q;
}

// Lane j stages the edge at CSR position base + j (j < cnt).
__device__ __forceinline__ EdgeScalars stage_edges(const SeEdges& g, int base, int cnt, int lane) {
  return stage_edges_at(g, base + lane, lane < cnt);
}

// The staged scalars of lane j (j may differ between lanes).
__device__ __forceinline__ EdgeScalars edge_from(const EdgeScalars& st, int j) {
  EdgeScalars q;
  q.other = __shfl(st.other, j, kWave);
  q.e = __shfl(st.e, j, kWave);
  q.ok = __shfl(st.ok, j, kWave);
#pragma unroll
  for (int i = 0; i < kSePaths; ++i) q.r[i] = __shfl(st.r[i], j, kWave);
#pragma unroll
  for (int k = 0; k < 3; ++k) q.d[k] = __shfl(st.d[k], j, kWave);
  q.y0 = __shfl(st.y0, j, kWave);
#pragma unroll
  for (int m = 0; m < 5; ++m) q.y2[m] = __shfl(st.y2[m], j, kWave);
  return q;
}

// Per-edge coefficients with the edge's scalars folded in, computed once by the lane that stages
// the edge (instead of by every channel lane):
//   c0 = r0 y0, c1 = r1 d, c2 = r2 y0, c3 = r3 d, c4 = r4 d, c5 = r5 y2, c6 = r6 y0, c8 = r8,
//   d7[j][m] = r7 sum_i d_i cg[i][j][m]
// (r_p = 0 for paths that are off).  The forward accumulates c0 s, c1 s, c2 v, c3 . v, c4 x v,
// c5 s, c6 t, c8 |t|^2 and sum_j d7[j] v_j; the source-side backward the transposed products.
template <bool T2>
struct EdgeCoef {
  int32_t other;
  int32_t ok;
  float c0, c1[3], c2, c3[3], c4[3];
  float c5[5], c6, c8, d7[3][5];
};

__device__ __forceinline__ void cg_coef(const float* cg, const float d[3], float r, float D[3][5]);

template <bool T2>
__device__ __forceinline__ EdgeCoef<T2> coef_of(const SeEdges& g, const EdgeScalars& q);

template <bool T2>
__device__ __forceinline__ EdgeCoef<T2> stage_coef(const SeEdges& g, int base, int cnt, int lane) {
  return coef_of<T2>(g, stage_edges(g, base, cnt, lane));
}

template <bool T2>
__device__ __forceinline__ EdgeCoef<T2> coef_of(const SeEdges& g, const EdgeScalars& q) {
  EdgeCoef<T2> c;
  c.other = q.other;
  c.ok = q.ok;
  c.c0 = q.r[0] * q.y0;
  c.c2 = q.r[2] * q.y0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    c.c1[k] = q.r[1] * q.d[k];
    c.c3[k] = q.r[3] * q.d[k];
    c.c4[k] = q.r[4] * q.d[k];
  }
  if (T2) {
#pragma unroll
    for (int m = 0; m < 5; ++m) c.c5[m] = q.r[5] * q.y2[m];
    c.c6 = q.r[6] * q.y0;
    c.c8 = q.r[8];
    cg_coef(g.cg, q.d, q.r[7], c.d7);
  }
  return c;
}

// The staged coefficients of lane j (j wave-uniform).
template <bool T2>
__device__ __forceinline__ EdgeCoef<T2> coef_at(const EdgeCoef<T2>& st, int j) {
  EdgeCoef<T2> c;
  c.other = __builtin_amdgcn_readlane(st.other, j);
  c.ok = __builtin_amdgcn_readlane(st.ok, j);
  c.c0 = rlane(st.c0, j);
  c.c2 = rlane(st.c2, j);
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    c.c1[k] = rlane(st.c1[k], j);
    c.c3[k] = rlane(st.c3[k], j);
    c.c4[k] = rlane(st.c4[k], j);
  }
  if (T2) {
#pragma unroll
    for (int m = 0; m < 5; ++m) c.c5[m] = rlane(st.c5[m], j);
    c.c6 = rlane(st.c6, j);
    c.c8 = rlane(st.c8, j);
#pragma unroll
    for (int jj = 0; jj < 3; ++jj)
#pragma unroll
      for (int m = 0; m < 5; ++m) c.d7[jj][m] = rlane(st.d7[jj][m], j);
  }
  return c;
}

// D[j][m] = r * sum_i d_i cg[i][j][m]: path 7's per-edge coefficients, so that a lane's share
// is sum_j v_j D[j][m] (forward) or sum_m D[j][m] w_m (source-side backward).
// The table is read from device memory at a wave-uniform address (scalar loads, cached); a NULL
// table (path 7 off) gives zeros.
__device__ __forceinline__ void cg_coef(const float* cg, const float d[3], float r, float D[3][5]) {
  if (cg == nullptr) {
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int m = 0; m < 5; ++m) D[j][m] = 0.f;
    return;
  }
#pragma unroll
  for (int j = 0; j < 3; ++j)
#pragma unroll
    for (int m = 0; m < 5; ++m)
      D[j][m] = r * ((d[0] * cg[j * 5 + m] + d[1] * cg[(3 + j) * 5 + m]) + d[2] * cg[(6 + j) * 5 + m]);
}

__device__ __forceinline__ void zero_pad(float* row, int used, int K) {
  for (int q = used + lane_id(); q < K; q += kWave) row[q] = 0.f;
}

__device__ __forceinline__ void node_range(const SeEdges& g, int64_t n, int& a, int& b) {
  a = g.ns[n];
  b = g.ne[n];
  a = a < 0 ? 0 : (a > g.E ? g.E : a);
  b = b < a ? a : (b > g.E ? g.E : b);
}

constexpr int kSeUnroll = 2;  // edges whose source rows are in flight together (C2: 2, 3, 4 give
                              // the same forward aggregate; the source-side backward 112 / 125 / 123 us)

// xcd_block() (common.hpp) gives each XCD one contiguous range of the node space, so
// neighbouring nodes -- which share source rows -- are processed under the same L2.

// ------------------------------------------------------------------ forward aggregate ---
// Per-lane sums of one target node's r-weighted source features, one input channel per lane
// (the type-2 sums compile out without T2).
template <bool T2>
struct NodeAcc {
  float A0, A1[3], A2[3], A3, A4[3];
  float A5[5], A6[5], A7[5], A8;
  __device__ __forceinline__ void zero() {
    A0 = A3 = A8 = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) A1[k] = A2[k] = A4[k] = 0.f;
#pragma unroll
    for (int k = 0; k < 5; ++k) A5[k] = A6[k] = A7[k] = 0.f;
  }
};

// Adds one edge (coefficients q; the lane's source values x, v[3], t[5]) to A.  hs / hv / ht:
// the lane's channel exists in s / v / t; t_out: type-2 outputs are computed.
template <bool T2>
__device__ __forceinline__ void accumulate_edge(NodeAcc<T2>& A, const SeEdges& g,
                                                const EdgeCoef<T2>& q, bool hs, bool hv, bool ht,
                                                bool t_out, float x, const float* v,
                                                const float* t) {
  if (hs) {
    if (g.pc[0] >= 0) A.A0 += q.c0 * x;
    if (g.pc[1] >= 0) {
#pragma unroll
      for (int k = 0; k < 3; ++k) A.A1[k] += q.c1[k] * x;
    }
    if (T2 && g.pc[5] >= 0) {
#pragma unroll
      for (int k = 0; k < 5; ++k) A.A5[k] += q.c5[k] * x;
    }
  }
  if (hv) {
    if (g.pc[2] >= 0) {
#pragma unroll
      for (int k = 0; k < 3; ++k) A.A2[k] += q.c2 * v[k];
    }
    if (g.pc[3] >= 0) A.A3 += (q.c3[0] * v[0] + q.c3[1] * v[1]) + q.c3[2] * v[2];
    if (g.pc[4] >= 0) {
      A.A4[0] += q.c4[1] * v[2] - q.c4[2] * v[1];
      A.A4[1] += q.c4[2] * v[0] - q.c4[0] * v[2];
      A.A4[2] += q.c4[0] * v[1] - q.c4[1] * v[0];
    }
    if (T2 && g.pc[7] >= 0 && t_out) {
#pragma unroll
      for (int k = 0; k < 5; ++k)
        A.A7[k] += (q.d7[0][k] * v[0] + q.d7[1][k] * v[1]) + q.d7[2][k] * v[2];
    }
  }
  if (ht) {
    if (g.pc[6] >= 0) {
#pragma unroll
      for (int k = 0; k < 5; ++k) A.A6[k] += q.c6 * t[k];
    }
    if (g.pc[8] >= 0)
      A.A8 += q.c8 * ((((t[0] * t[0] + t[1] * t[1]) + t[2] * t[2]) + t[3] * t[3]) + t[4] * t[4]);
  }
}

// The lane's channel in each feature kind as a byte offset inside a source row, clamped to the
// kind's last channel: every lane loads (a lane past a kind's channels reads a channel it will
// not use), so the loads carry no per-lane condition.  A source row is read by buffer loads
// through a resource built from its wave-uniform address (scalar registers) and this 32-bit
// offset: no per-lane address arithmetic and no address registers per load, so a wave's rows are
// all in flight together.  (With per-lane conditions and 64-bit per-lane addresses the compiler
// waited for each row before issuing the next.)
struct LaneCh {
  uint32_t s, v, t;
  __device__ __forceinline__ LaneCh(const SeFeat& f, int c)
      : s(4u * min(c, max(f.Cs - 1, 0))),
        v(12u * min(c, max(f.Cv - 1, 0))),
        t(20u * min(c, max(f.Ct - 1, 0))) {}
};

// A buffer resource over `bytes` bytes at p: loads through it read zeros past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}
// The float at byte offset `byte`.
__device__ __forceinline__ float ld_row(__amdgpu_buffer_rsrc_t r, uint32_t byte) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte, 0, 0));
}

// Loads the lane's channel of source row m (wave-uniform): s, v (3) and t (5), for the kinds
// the features have.
template <bool T2>
__device__ __forceinline__ void load_source(const SeFeat& f, int m, const LaneCh& ch, float& x,
                                            float* v, float* t) {
  if (f.Cs > 0) x = ld_row(row_rsrc(f.s + static_cast<int64_t>(m) * f.Cs, 4 * f.Cs), ch.s);
  if (f.Cv > 0) {
    const auto r = row_rsrc(f.v + static_cast<int64_t>(m) * (3 * f.Cv), 12 * f.Cv);
    v[0] = ld_row(r, ch.v);
    v[1] = ld_row(r, ch.v + 4);
    v[2] = ld_row(r, ch.v + 8);
  }
  if (T2 && f.Ct > 0) {
    const auto r = row_rsrc(f.t + static_cast<int64_t>(m) * (5 * f.Ct), 20 * f.Ct);
#pragma unroll
    for (int k = 0; k < 5; ++k) t[k] = ld_row(r, ch.t + 4 * k);
  }
}

// Writes the lane's channel c of a node's aggregate rows (layout in the header comment):
// xs [Ks] = A0 | A3 | A8, xv row k (k < 3, rows sv apart) = A1_k | A2_k | A4_k, xt row m
// (m < 5, rows st apart) = A5_m | A6_m | A7_m.  A NULL row pointer skips that kind.
template <bool T2>
__device__ __forceinline__ void store_node(const NodeAcc<T2>& A, const SeFeat& f, int c, bool hs,
                                           bool hv, bool ht, float* xs, float* xv, int sv,
                                           float* xt, int st) {
  if (xs) {
    if (hs) xs[c] = A.A0;
    if (hv) xs[f.Cs + c] = A.A3;
    if (ht) xs[f.Cs + f.Cv + c] = A.A8;
  }
  if (xv) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      float* row = xv + k * sv;
      if (hs) row[c] = A.A1[k];
      if (hv) row[f.Cs + c] = A.A2[k];
      if (hv) row[f.Cs + f.Cv + c] = A.A4[k];
    }
  }
  if (T2 && xt) {
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      float* row = xt + k * st;
      if (hs) row[c] = A.A5[k];
      if (ht) row[f.Cs + c] = A.A6[k];
      if (hv) row[f.Cs + f.Ct + c] = A.A7[k];
    }
  }
}

// One wave per target node, lanes over input channels (chunks of 64).  The node's edges are
// staged in lanes, then walked kSeUnroll at a time: the source rows are loaded first, then
// accumulated in CSR order.
template <bool T2>  // T2: type-2 features or outputs present (else their paths compile out)
__global__ __launch_bounds__(kSeThreads) void se3_fwd_aggregate(SeEdges g, SeFeat f,
                                                               float* __restrict__ Xs, int Ks,
                                                               float* __restrict__ Xv, int Kv,
                                                               float* __restrict__ Xt, int Kt) {
  const int64_t n = xcd_block() * kSeWaves + uniform(threadIdx.x / kWave);
  if (n >= g.N) return;
  const int lane = lane_id();
  int a, b;
  node_range(g, n, a, b);
  const int cmax = max(f.Cs, max(f.Cv, f.Ct));
  const bool t_out = Xt != nullptr;
  for (int c0 = 0; c0 < cmax; c0 += kWave) {
    const int c = c0 + lane;
    const bool hs = c < f.Cs, hv = c < f.Cv, ht = T2 && c < f.Ct;
    const LaneCh ch(f, c);
    NodeAcc<T2> A;
    A.zero();
    for (int base = a; base < b; base += kWave) {
      const int cnt = min(kWave, b - base);
      const EdgeCoef<T2> st = stage_coef<T2>(g, base, cnt, lane);
      for (int j0 = 0; j0 < cnt; j0 += kSeUnroll) {
        float sv[kSeUnroll], vv[kSeUnroll][3], tt[kSeUnroll][5];
#pragma unroll
        for (int u = 0; u < kSeUnroll; ++u) {
          const int j = min(j0 + u, kWave - 1);
          const int m = __builtin_amdgcn_readlane(st.other, j);  // 0 past cnt: in bounds
          load_source<T2>(f, m, ch, sv[u], vv[u], tt[u]);
        }
#pragma unroll
        for (int u = 0; u < kSeUnroll; ++u) {
          if (j0 + u >= cnt) break;
          const EdgeCoef<T2> q = coef_at<T2>(st, j0 + u);
          if (!q.ok) continue;
          accumulate_edge<T2>(A, g, q, hs, hv, ht, t_out, sv[u], vv[u], tt[u]);
        }
      }
    }
    store_node<T2>(A, f, c, hs, hv, ht, Xs ? Xs + n * Ks : nullptr, Xv ? Xv + n * 3 * Kv : nullptr,
                   Kv, (T2 && Xt) ? Xt + n * 5 * Kt : nullptr, Kt);
  }
  if (Xs) zero_pad(Xs + n * Ks, f.Cs + f.Cv + f.Ct, Ks);
  if (Xv)
    for (int k = 0; k < 3; ++k) zero_pad(Xv + (n * 3 + k) * Kv, f.Cs + 2 * f.Cv, Kv);
  if (T2 && Xt)
    for (int k = 0; k < 5; ++k) zero_pad(Xt + (n * 5 + k) * Kt, f.Cs + f.Ct + f.Cv, Kt);
}

// ------------------------------------------------------------------------ MFMA GEMM ---
// out(r, o) = epilogue(sum_k A[r, k] B[o, k]) for r < M, o < O, with A [M, K] and B [>= grid
// columns, K] row-major, K a multiple of 16 and both 16-byte aligned.  Row r is node n = r / G,
// component g = r % G, stored at out[n * ostride + o * G + g] (G = 1 scalars, 3 vectors, 5
// type-2 features; a template parameter).  Epilogue: scale by 1 / avg[n] (one reciprocal per
// row), add bias[o], zero where mask[n] == 0 (each optional).
//
// v_mfma_f32_16x16x4_f32: lane l supplies A[i = l % 16][k = l / 16] and B[k = l / 16][j = l % 16]
// and holds D[i = 4 (l / 16) + q][j = l % 16] in element q.  Each lane loads four consecutive k
// of a 16-wide chunk as one float4 (k = 4 (l / 16) + q for the q-th MFMA); A and B use the same
// assignment, so the four MFMAs cover the chunk's 16 k exactly once.  A wave computes 32 rows x
// 16 NB columns; a block is four waves stacked along the rows.
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int NB, int G>
__global__ __launch_bounds__(kSeThreads) void se3_gemm(const float* __restrict__ A, int64_t M, int K,
                                                      const float* __restrict__ B, int O,
                                                      float* __restrict__ out, int64_t ostride,
                                                      const float* __restrict__ avg,
                                                      const float* __restrict__ bias,
                                                      const uint8_t* __restrict__ mask) {
  const int lane = lane_id();
  const int li = lane & 15, lk = lane >> 4;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kSeWaves + uniform(threadIdx.x / kWave)) * 32;
  if (row0 >= M) return;
  const int col0 = blockIdx.y * 16 * NB;
  const float* ap[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    int64_t r = row0 + rb * 16 + li;
    r = r < M ? r : M - 1;
    ap[rb] = A + r * K + 4 * lk;
  }
  const float* bp[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) bp[cb] = B + static_cast<int64_t>(col0 + cb * 16 + li) * K + 4 * lk;
  floatx4 acc[2][NB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) acc[rb][cb] = floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 a[2], b[NB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) a[rb] = *reinterpret_cast<const floatx4*>(ap[rb]);
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) b[cb] = *reinterpret_cast<const floatx4*>(bp[cb]);
  for (int k0 = 0; k0 < K; k0 += 16) {
    floatx4 an[2], bn[NB];
    const int kn = k0 + 16 < K ? k0 + 16 : k0;  // last chunk reloads itself (in bounds)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) an[rb] = *reinterpret_cast<const floatx4*>(ap[rb] + kn);
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) bn[cb] = *reinterpret_cast<const floatx4*>(bp[cb] + kn);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < NB; ++cb)
          acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[rb][q], b[cb][q], acc[rb][cb], 0, 0, 0);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) a[rb] = an[rb];
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) b[cb] = bn[cb];
  }
  // epilogue: per-row scale (1 / avg, 0 where masked) and per-column bias, then strided stores
  float bcol[NB];
  bool ocol[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const int o = col0 + cb * 16 + li;
    ocol[cb] = o < O;
    bcol[cb] = (bias && ocol[cb]) ? bias[o] : 0.f;
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t r = row0 + rb * 16 + 4 * lk + q;
      if (r >= M) continue;
      const int64_t n = r / G;
      const int gc = static_cast<int>(r - n * G);
      const bool keep = mask == nullptr || mask[n] != 0;
      const float scale = avg ? 1.0f / avg[n] : 1.0f;
      float* orow = out + n * ostride + gc;
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) {
        if (!ocol[cb]) continue;
        const float val = acc[rb][cb][q] * scale + bcol[cb];
        orow[static_cast<int64_t>(col0 + cb * 16 + li) * G] = keep ? val : 0.f;
      }
    }
}

// ---------------------------------------------- fused forward: aggregate + per-node GEMM ---
// One workgroup per tile of kFuTile consecutive target nodes.  Each wave sums the r-weighted
// source features of kFuNodes nodes (one input channel per lane, as se3_fwd_aggregate) into the
// tile's aggregate rows in LDS; then the waves multiply the tile by the packed weights with
// v_mfma_f32_16x16x4_f32 (the se3_gemm fragment layout, A from LDS) and apply the epilogue
// (1 / avg, bias, mask).  The aggregates reach HBM only when the caller asks for them (the
// weight gradients need them).
//
// Edges: the kFuNodes nodes' CSR ranges are concatenated into one flat list, staged 64 at a time
// (lane l takes flat edge fb + l, wherever its node's range lies), and walked U at a time with
// all U source rows loaded before any is used; the sums are flushed to LDS when the walk passes
// a node's last edge.  A node's edges are still added in CSR order.
constexpr int kFuTile = 16;                   // nodes per workgroup = MFMA rows of a scalar block
constexpr int kFuNodes = kFuTile / kSeWaves;  // nodes per wave
constexpr int kFuLdsMax = 64 * 1024;          // larger aggregate tiles take the unfused path
static_assert(kFuNodes == 4, "the flat edge walk below is written for 4 nodes per wave");

struct SeFused {
  const float* W[3];   // packed weights [rows >= 16 ceil(O / 16)][K] (kinds: s, v, t)
  float* out[3];       // s_out [N, Os], v_out [N, Ov, 3], t_out [N, Ot, 5]
  float* X[3];         // optional HBM copies of the aggregate rows ([N, K], [N, 3, K], [N, 5, K])
  int O[3];            // output channels (0: kind absent)
  int K[3];            // aggregate row length (multiple of 16)
  int ld[3];           // LDS row stride (K + 4 floats)
  int off[3];          // LDS offset of the kind's tile (floats)
  const float* avg;
  const float* bias;
  const uint8_t* mask;
};

// The k loop of the tile GEMMs (K a multiple of 16): 16-wide chunks, four per step and then
// the remaining one to three, each step's fragments all requested before its MFMAs.  la(k) /
// lw(k) return this lane's A / W fragment at column k.  (Loading four chunks and skipping the
// MFMAs of those past K let the compiler sink each chunk's loads behind its test, so every chunk
// waited for its own loads.)  The accumulation order is chunk by chunk, q = 0..3 within each.
template <int NC, class LA, class LW>
__device__ __forceinline__ floatx4 mfma_k_step(const LA& la, const LW& lw, int k0, floatx4 acc) {
  floatx4 a[NC], w[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    w[c] = lw(k0 + 16 * c);
    a[c] = la(k0 + 16 * c);
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c][q], w[c][q], acc, 0, 0, 0);
  return acc;
}

template <class LA, class LW>
__device__ __forceinline__ floatx4 mfma_k_loop(const LA& la, const LW& lw, int K) {
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  int k0 = 0;
  for (; k0 + 64 <= K; k0 += 64) acc = mfma_k_step<4>(la, lw, k0, acc);
  switch ((K - k0) >> 4) {  // wave-uniform
    case 3: acc = mfma_k_step<3>(la, lw, k0, acc); break;
    case 2: acc = mfma_k_step<2>(la, lw, k0, acc); break;
    case 1: acc = mfma_k_step<1>(la, lw, k0, acc); break;
    default: break;
  }
  return acc;
}

// The tile's MFMA blocks of one kind: block b (< G ceil(O / 16)) is row block b / ncb, column
// block b % ncb; wave w takes the blocks whose running number base + b is w mod 4.  The
// epilogue's per-row operands are requested first and the weight fragments four 16-wide k chunks
// at a time (mfma_k_loop), so a block waits for global memory about once per 64 k.
// (Holding a column block's weights for all G row blocks needs G accumulators and per-row
// operands at once: 147 VGPRs for the whole kernel, whose walk then ran at a lower occupancy.)
template <int G>
__device__ __forceinline__ void fused_gemm(const float* __restrict__ tile, int ld, int K,
                                           const float* __restrict__ W, int O,
                                           float* __restrict__ out, const SeFused& p,
                                           int64_t node0, int64_t N, int base, int wave, int lane) {
  const int ncb = (O + 15) / 16;
  const int nblk = G * ncb;
  const int li = lane & 15, lk = lane >> 4;
  for (int b = (wave - base % kSeWaves + kSeWaves) % kSeWaves; b < nblk; b += kSeWaves) {
    const int rb = b / ncb, cb = b % ncb;
    const int o = cb * 16 + li;
    // bias, degrees and mask loaded without per-lane conditions (indices clamped into range,
    // values selected after; the pointer tests are uniform): a load under a per-lane condition
    // left the compiler waiting for all memory operations, earlier stores included, before
    // each output store
    float bo = 0.f;
    if (G == 1 && p.bias) {
      const float bl = p.bias[o < O ? o : O - 1];
      bo = o < O ? bl : 0.f;
    }
    float scale[4];
    bool keep[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = node0 + (rb * 16 + 4 * lk + q) / G;
      const bool in = n < N;
      const int64_t nc = in ? n : N - 1;
      float av = 1.0f;
      if (p.avg) av = p.avg[nc];
      scale[q] = (in && p.avg) ? 1.0f / av : 1.0f;
      bool mk = true;
      if (p.mask) mk = p.mask[nc] != 0;
      keep[q] = !in || mk;
    }
    const float* ap = tile + (rb * 16 + li) * ld + 4 * lk;
    const float* bp = W + static_cast<int64_t>(cb * 16 + li) * K + 4 * lk;
    const floatx4 acc = mfma_k_loop(
        [&](int k) { return *reinterpret_cast<const floatx4*>(ap + k); },
        [&](int k) { return *reinterpret_cast<const floatx4*>(bp + k); }, K);
    // every load of the block has completed here (the k loop waited for its later ones); the
    // explicit wait, free at this point, tells the compiler so, which otherwise waited for all
    // memory operations, the previous store included, before each store below
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = rb * 16 + 4 * lk + q;  // tile row: node r / G, component r % G
      const int64_t n = node0 + r / G;
      if (n >= N || o >= O) continue;
      const float val = acc[q] * scale[q] + bo;
      out[(n * O + o) * G + r % G] = keep[q] ? val : 0.f;
    }
  }
}

// Zeroes the padding columns [used, K) of every row of the tile; the walks write every used column.
__device__ __forceinline__ void zero_tile_pads(const SeFeat& f, const SeFused& p, float* lds) {
  const int used[3] = {f.Cs + f.Cv + f.Ct, f.Cs + 2 * f.Cv, f.Cs + f.Ct + f.Cv};
  const int rows[3] = {kFuTile, 3 * kFuTile, 5 * kFuTile};
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int pad = p.K[k] - used[k];
    if (p.O[k] <= 0 || pad <= 0) continue;
    for (int i = threadIdx.x; i < rows[k] * pad; i += kSeThreads)
      lds[p.off[k] + (i / pad) * p.ld[k] + used[k] + i % pad] = 0.f;
  }
}

// After the tile's aggregate rows are complete in LDS (behind a barrier): copies them to HBM
// when the caller keeps them (a tile's rows are contiguous there), then computes the outputs,
// the kinds' MFMA blocks spread over the four waves.
template <bool T2>
__device__ __forceinline__ void fused_tile_out(const SeFused& p, const float* lds, int64_t node0,
                                               int64_t N, int wave, int lane) {
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int G = k == 0 ? 1 : (k == 1 ? 3 : 5);
    if (p.O[k] <= 0 || p.X[k] == nullptr || (k == 2 && !T2)) continue;
    const int rows = static_cast<int>(min(static_cast<int64_t>(kFuTile), N - node0)) * G;
    const int K4 = p.K[k] / 4;  // 16-byte pieces per row (K is a multiple of 16)
    floatx4* dst = reinterpret_cast<floatx4*>(p.X[k] + node0 * G * p.K[k]);
    for (int r = wave; r < rows; r += kSeWaves)
      for (int c = lane; c < K4; c += kWave)
        dst[r * K4 + c] = *reinterpret_cast<const floatx4*>(lds + p.off[k] + r * p.ld[k] + 4 * c);
  }
  const int nb0 = p.O[0] > 0 ? (p.O[0] + 15) / 16 : 0;
  const int nb1 = p.O[1] > 0 ? 3 * ((p.O[1] + 15) / 16) : 0;
  if (p.O[0] > 0)
    fused_gemm<1>(lds + p.off[0], p.ld[0], p.K[0], p.W[0], p.O[0], p.out[0], p, node0, N, 0, wave,
                  lane);
  if (p.O[1] > 0)
    fused_gemm<3>(lds + p.off[1], p.ld[1], p.K[1], p.W[1], p.O[1], p.out[1], p, node0, N, nb0,
                  wave, lane);
  if (T2 && p.O[2] > 0)
    fused_gemm<5>(lds + p.off[2], p.ld[2], p.K[2], p.W[2], p.O[2], p.out[2], p, node0, N,
                  nb0 + nb1, wave, lane);
}

template <bool T2, int U>  // U: source rows in flight per lane
__global__ __launch_bounds__(kSeThreads) void se3_fwd_fused(SeEdges g, SeFeat f, SeFused p) {
  extern __shared__ floatx4 fu_lds[];
  float* lds = reinterpret_cast<float*>(fu_lds);
  const int64_t node0 = xcd_block() * kFuTile;  // grid = ceil(N / kFuTile): node0 < N
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  float* ts = p.O[0] > 0 ? lds + p.off[0] : nullptr;
  float* tv = p.O[1] > 0 ? lds + p.off[1] : nullptr;
  float* tt = (T2 && p.O[2] > 0) ? lds + p.off[2] : nullptr;

  zero_tile_pads(f, p, lds);

  // the wave's nodes: CSR ranges loaded by lanes 0..3, concatenated into one flat edge list
  const int64_t nw = node0 + wave * kFuNodes;
  int la = 0, lb = 0;
  if (lane < kFuNodes && nw + lane < g.N) node_range(g, nw + lane, la, lb);
  const int a0 = __builtin_amdgcn_readlane(la, 0), a1 = __builtin_amdgcn_readlane(la, 1);
  const int a2 = __builtin_amdgcn_readlane(la, 2), a3 = __builtin_amdgcn_readlane(la, 3);
  const int cnt_l = lb - la;
  const int e1 = __builtin_amdgcn_readlane(cnt_l, 0);           // flat end of node 0
  const int e2 = e1 + __builtin_amdgcn_readlane(cnt_l, 1);      // of node 1
  const int e3 = e2 + __builtin_amdgcn_readlane(cnt_l, 2);      // of node 2
  const int total = e3 + __builtin_amdgcn_readlane(cnt_l, 3);  // of node 3
  const bool t_out = tt != nullptr;
  const int cmax = max(f.Cs, max(f.Cv, f.Ct));
  for (int c0 = 0; c0 < cmax; c0 += kWave) {
    const int c = c0 + lane;
    const bool hs = c < f.Cs, hv = c < f.Cv, ht = T2 && c < f.Ct;
    const LaneCh ch(f, c);
    NodeAcc<T2> A;
    A.zero();
    int cur = 0, cur_end = e1;  // node being summed and its flat end
    auto flush = [&](int i) {
      const int nt = wave * kFuNodes + i;
      store_node<T2>(A, f, c, hs, hv, ht, ts ? ts + nt * p.ld[0] : nullptr,
                     tv ? tv + nt * 3 * p.ld[1] : nullptr, p.ld[1],
                     tt ? tt + nt * 5 * p.ld[2] : nullptr, p.ld[2]);
      A.zero();
    };
    for (int fb = 0; fb < total; fb += kWave) {
      const int fl = fb + lane;
      const int i = (fl >= e1) + (fl >= e2) + (fl >= e3);
      const int start = i == 0 ? a0 : (i == 1 ? a1 : (i == 2 ? a2 : a3));
      const int first = i == 0 ? 0 : (i == 1 ? e1 : (i == 2 ? e2 : e3));
      const EdgeCoef<T2> st = coef_of<T2>(g, stage_edges_at(g, start + fl - first, fl < total));
      const int cnt = min(kWave, total - fb);
      for (int j0 = 0; j0 < cnt; j0 += U) {
        float sv[U], vv[U][3], tw[U][5];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = min(j0 + u, kWave - 1);
          const int m = __builtin_amdgcn_readlane(st.other, j);  // 0 past the list: in bounds
          load_source<T2>(f, m, ch, sv[u], vv[u], tw[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (j0 + u >= cnt) break;
          while (fb + j0 + u >= cur_end) {  // past the current node's last edge
            flush(cur);
            ++cur;
            cur_end = cur == 1 ? e2 : (cur == 2 ? e3 : total);
          }
          const EdgeCoef<T2> q = coef_at<T2>(st, j0 + u);
          if (!q.ok) continue;
          accumulate_edge<T2>(A, g, q, hs, hv, ht, t_out, sv[u], vv[u], tw[u]);
        }
      }
    }
    for (; cur < kFuNodes; ++cur) flush(cur);
  }
  __syncthreads();
  fused_tile_out<T2>(p, lds, node0, g.N, wave, lane);
}

// ------------------------------ fused forward, one node per 16-lane row (no type-2 paths) ---
// Layers without type-2 features or outputs whose Cs <= 64 and Cv <= 16 (Cs a multiple of 4;
// e.g. 64 scalar + 16 vector channels): a wave sums four nodes at once, one per 16-lane row.
// Lane j of a row holds scalar channels 4j..4j+3 and vector channel j, so one 16-byte load (s)
// and one 12-byte load (v) per lane fetch a source row for each of the four nodes -- two
// vector-memory instructions per four edges where the channel-per-lane walk above issues four
// per edge.  That walk keeps the texture address unit busy ~70% of its time (counters at C2);
// this one needs an eighth of its instructions.  A row's edges are staged one per lane, 16 per
// round, and edge u's source and coefficients reach the row's lanes by DPP row_newbcast:u.
constexpr int kRowNodes = kFuTile / kSeWaves;  // nodes per wave = 16-lane rows
constexpr int kRowStage = 16;                  // edges staged per row per round
constexpr uint32_t kPastRows = 0x80000000u;    // a byte offset past every array (each < 2 GiB)
static_assert(kRowNodes * 16 == kWave, "one node per 16-lane row");

// Lane u of the lane's 16-lane row (u a compile-time constant).
template <int u>
__device__ __forceinline__ int row_bcast(int x) {
  return __builtin_amdgcn_update_dpp(0, x, 0x150 + u, 0xf, 0xf, false);  // row_newbcast:u
}
template <int u>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, row_bcast<u>(__builtin_bit_cast(int, x)));
}

// Calls f(std::integral_constant<int, I>) for I = B, B + 1, ..., E - 1.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Per-lane sums of the row's node: scalar channels 4j..4j+3 (A0, A1_k) and vector channel j
// (A2_k, A3, A4_k).
struct RowAcc {
  float A0[4], A1[3][4];
  float A2[3], A3, A4[3];
};

// Staging of the row kernel: the lane's edge at CSR position pos (when valid) -- its source, the
// radial weights of paths 0-4, the direction (one 12-byte load) and Y_0^0 -- as coefficients
// (coef_of's c0..c4).  The loads go through buffer resources and a lane without an edge reads
// past the arrays (zeros), so none of them waits on a branch or on the source load; only the
// permutation, when there is one, comes first.  Every array here is below 2 GiB (the host checks).
__device__ __forceinline__ EdgeCoef<false> stage_rows(const SeEdges& g, int pos, bool valid) {
  constexpr uint32_t kPast = kPastRows;
  int e = valid ? pos : -1;
  if (g.perm) {
    const auto rp = row_rsrc(g.perm, g.E * 4);
    e = valid ? static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rp, 4u * pos, 0, 0)) : -1;
  }
  const bool ein = static_cast<unsigned>(e) < static_cast<unsigned>(g.E);
  const uint32_t ue = ein ? static_cast<uint32_t>(e) : 0u;
  const auto ro = row_rsrc(g.other, g.E * 8);
  const auto w = __builtin_amdgcn_raw_buffer_load_b64(ro, ein ? 8u * ue : kPast, 0, 0);
  const uint32_t lo = w[0], hi = w[1];
  const int64_t o = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  const auto rr = row_rsrc(g.R, g.E * g.P * 4);
  float r[5];
#pragma unroll
  for (int i = 0; i < 5; ++i)
    r[i] = g.pc[i] >= 0 ? ld_row(rr, ein ? 4u * (ue * g.P + g.pc[i]) : kPast) : 0.f;
  const auto rd = row_rsrc(g.dir, g.E * 12);
  const auto dv = __builtin_amdgcn_raw_buffer_load_b96(rd, ein ? 12u * ue : kPast, 0, 0);
  const float d[3] = {__uint_as_float(dv[0]), __uint_as_float(dv[1]), __uint_as_float(dv[2])};
  const auto ry = row_rsrc(g.Y, g.E * g.ysh * 4);
  const float y0 = ld_row(ry, ein ? 4u * ue * g.ysh : kPast);
  const bool ok = ein && o >= 0 && o < g.N;
  EdgeCoef<false> c;
  c.other = ok ? static_cast<int32_t>(o) : 0;
  c.ok = ok ? 1 : 0;
#pragma unroll
  for (int i = 0; i < 5; ++i) r[i] = ok ? r[i] : 0.f;
  c.c0 = r[0] * y0;
  c.c2 = r[2] * y0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    c.c1[k] = r[1] * d[k];
    c.c3[k] = r[3] * d[k];
    c.c4[k] = r[4] * d[k];
  }
  return c;
}

template <int U>
__global__ __launch_bounds__(kSeThreads) void se3_fwd_fused_rows(SeEdges g, SeFeat f, SeFused p) {
  extern __shared__ floatx4 fu_lds[];
  float* lds = reinterpret_cast<float*>(fu_lds);
  const int64_t node0 = xcd_block() * kFuTile;  // grid = ceil(N / kFuTile): node0 < N
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x / kWave);
  const int j = lane & 15;
  const int nt = wave * kRowNodes + (lane >> 4);  // the row's node in the tile
  zero_tile_pads(f, p, lds);

  int a = 0, b = 0;
  if (node0 + nt < g.N) node_range(g, node0 + nt, a, b);
  const int deg = b - a;
  const int maxdeg = max(max(__builtin_amdgcn_readlane(deg, 0), __builtin_amdgcn_readlane(deg, 16)),
                         max(__builtin_amdgcn_readlane(deg, 32), __builtin_amdgcn_readlane(deg, 48)));
  // whole-array resources (the host keeps both arrays below 4 GiB): a lane past the row's
  // channels reads the next row (unused) or, past the array, zeros
  const auto rs = row_rsrc(f.s, static_cast<int>(g.N * f.Cs * 4));
  const auto rv = row_rsrc(f.v, static_cast<int>(g.N * f.Cv * 12));
  const uint32_t rowb_s = 4u * f.Cs, rowb_v = 12u * f.Cv;
  const uint32_t js = 16u * j, jv = 12u * j;

  RowAcc A;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    A.A0[i] = 0.f;
    A.A1[0][i] = A.A1[1][i] = A.A1[2][i] = 0.f;
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) A.A2[k] = A.A4[k] = 0.f;
  A.A3 = 0.f;

  for (int base = 0; base < maxdeg; base += kRowStage) {
    const EdgeCoef<false> st = stage_rows(g, a + base + j, base + j < deg);
    const int cnt = min(kRowStage, maxdeg - base);
    static_for<0, kRowStage / U>([&](auto ci) {
      constexpr int c0 = decltype(ci)::value * U;
      if (c0 >= cnt) return;
      floatx4 sx[U];
      float vx[U][3];
      static_for<0, U>([&](auto ui) {  // the U source rows of every row in flight together
        constexpr int u = c0 + decltype(ui)::value;
        // a row without edge u (its node has fewer edges) reads past the arrays: zeros, no traffic
        const bool have = row_bcast<u>(st.ok) != 0;
        const uint32_t m = static_cast<uint32_t>(row_bcast<u>(st.other));
        const auto ls = __builtin_amdgcn_raw_buffer_load_b128(rs, have ? m * rowb_s + js : kPastRows,
                                                              0, 0);
        const auto lv = __builtin_amdgcn_raw_buffer_load_b96(rv, have ? m * rowb_v + jv : kPastRows,
                                                             0, 0);
        // element by value: __builtin_bit_cast of a vector element reads the vector's first
        // element whatever the index
#pragma unroll
        for (int i = 0; i < 4; ++i) sx[decltype(ui)::value][i] = __uint_as_float(ls[i]);
#pragma unroll
        for (int k = 0; k < 3; ++k) vx[decltype(ui)::value][k] = __uint_as_float(lv[k]);
      });
      static_for<0, U>([&](auto ui) {
        constexpr int uu = decltype(ui)::value;
        constexpr int u = c0 + uu;
        // an edge that is not there (past the row's degree, or a source out of range) adds
        // nothing: its values are replaced by zeros, so a non-finite row 0 cannot leak in
        const bool ok = row_bcast<u>(st.ok) != 0;
        float x[4], v[3];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = ok ? sx[uu][i] : 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) v[k] = ok ? vx[uu][k] : 0.f;
        if (g.pc[0] >= 0) {
          const float c = row_bcast<u>(st.c0);
#pragma unroll
          for (int i = 0; i < 4; ++i) A.A0[i] += c * x[i];
        }
        if (g.pc[1] >= 0) {
#pragma unroll
          for (int k = 0; k < 3; ++k) {
            const float c = row_bcast<u>(st.c1[k]);
#pragma unroll
            for (int i = 0; i < 4; ++i) A.A1[k][i] += c * x[i];
          }
        }
        if (g.pc[2] >= 0) {
          const float c = row_bcast<u>(st.c2);
#pragma unroll
          for (int k = 0; k < 3; ++k) A.A2[k] += c * v[k];
        }
        if (g.pc[3] >= 0) {
          const float d0 = row_bcast<u>(st.c3[0]), d1 = row_bcast<u>(st.c3[1]);
          const float d2 = row_bcast<u>(st.c3[2]);
          A.A3 += (d0 * v[0] + d1 * v[1]) + d2 * v[2];
        }
        if (g.pc[4] >= 0) {
          const float e0 = row_bcast<u>(st.c4[0]), e1 = row_bcast<u>(st.c4[1]);
          const float e2 = row_bcast<u>(st.c4[2]);
          A.A4[0] += e1 * v[2] - e2 * v[1];
          A.A4[1] += e2 * v[0] - e0 * v[2];
          A.A4[2] += e0 * v[1] - e1 * v[0];
        }
      });
    });
  }

  // the node's aggregate rows into the tile (layout as se3_fwd_aggregate's rows)
  float* ts = p.O[0] > 0 ? lds + p.off[0] + nt * p.ld[0] : nullptr;
  float* tv = p.O[1] > 0 ? lds + p.off[1] + nt * 3 * p.ld[1] : nullptr;
  if (4 * j < f.Cs) {
    if (ts) *reinterpret_cast<floatx4*>(ts + 4 * j) = floatx4{A.A0[0], A.A0[1], A.A0[2], A.A0[3]};
    if (tv)
#pragma unroll
      for (int k = 0; k < 3; ++k)
        *reinterpret_cast<floatx4*>(tv + k * p.ld[1] + 4 * j) =
            floatx4{A.A1[k][0], A.A1[k][1], A.A1[k][2], A.A1[k][3]};
  }
  if (j < f.Cv) {
    if (ts) ts[f.Cs + j] = A.A3;
    if (tv)
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        tv[k * p.ld[1] + f.Cs + j] = A.A2[k];
        tv[k * p.ld[1] + f.Cs + f.Cv + j] = A.A4[k];
      }
  }
  __syncthreads();
  fused_tile_out<false>(p, lds, node0, g.N, wave, lane);
}

// Whether se3_fwd_fused_rows covers the layer (see its comment), with every array it reads
// through a buffer resource below 2 GiB.
bool fused_rows_ok(int64_t N, int Cs, int Cv, bool t2, int64_t E, int P, int ysh) {
  const int64_t lim = int64_t{1} << 31;
  return !t2 && Cs <= 64 && Cv <= 16 && Cs % 4 == 0 && N * Cs * 4 < lim && N * Cv * 12 < lim &&
         E * 12 < lim && E * P * 4 < lim && E * ysh * 4 < lim;
}

// LDS layout of the fused kernel's tile: per present kind, kFuTile * G rows of K + 4 floats.
// Returns the bytes, or 0 when they exceed kFuLdsMax.
size_t fused_layout(int Os, int Ov, int Ot, int Ks, int Kv, int Kt, SeFused* p) {
  const int O[3] = {Os, Ov, Ot}, K[3] = {Ks, Kv, Kt}, G[3] = {1, 3, 5};
  size_t floats = 0;
  for (int k = 0; k < 3; ++k) {
    const int ld = K[k] + 4;
    if (p) {
      p->O[k] = O[k] > 0 ? O[k] : 0;
      p->K[k] = O[k] > 0 ? K[k] : 0;
      p->ld[k] = ld;
      p->off[k] = static_cast<int>(floats);
    }
    if (O[k] > 0) floats += static_cast<size_t>(kFuTile) * G[k] * ld;
  }
  const size_t bytes = floats * sizeof(float);
  return bytes <= static_cast<size_t>(kFuLdsMax) ? bytes : 0;
}

// ------------------------------------------------------------ split-K transposed GEMM ---
// out[o][k] = sum_r A[r * lda + o] * B[r * ldb + k] over r < M (o < O, k < K): the weight
// gradients (output gradients x per-node aggregates, summed over nodes).  The reduction
// dimension M is long and O, K are small, so the rows are split over the waves of the grid;
// each wave accumulates its OB x KB tiles of 16 x 16 in MFMA accumulators (A^T as the MFMA A
// operand, B as the B operand, k = rows), the block's waves are added in LDS and the block
// writes one partial; se3_gemm_tn_final adds the partials in a fixed order.
template <int OB, int KB>
__global__ __launch_bounds__(kSeThreads) void se3_gemm_tn(const float* __restrict__ A, int64_t M,
                                                         int lda, int O,
                                                         const float* __restrict__ B, int ldb,
                                                         int K, int64_t rows_per_wave, int kb_groups,
                                                         float* __restrict__ part, int Opad,
                                                         int Kpad) {
  const int lane = lane_id();
  const int g = lane >> 4, li = lane & 15;
  const int w = uniform(threadIdx.x / kWave);
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * kSeWaves + w;
  const int ob0 = (blockIdx.y / kb_groups) * OB, kb0 = (blockIdx.y % kb_groups) * KB;
  const int64_t r_begin = wid * rows_per_wave;
  const int64_t r_end = min(M, r_begin + rows_per_wave);
  floatx4 acc[OB][KB];
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc[ob][kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int64_t r0 = r_begin; r0 < r_end; r0 += 16) {
    float a[OB][4], b[KB][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t r = r0 + 4 * g + q;
      const bool ok = r < r_end;
#pragma unroll
      for (int ob = 0; ob < OB; ++ob) {
        const int o = 16 * (ob0 + ob) + li;
        a[ob][q] = ok && o < O ? A[r * lda + o] : 0.f;
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int k = 16 * (kb0 + kb) + li;
        b[kb][q] = ok && k < K ? B[r * ldb + k] : 0.f;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
          acc[ob][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ob][q], b[kb][q], acc[ob][kb], 0, 0, 0);
  }
  // The block's four waves add their tiles in LDS, (w0 + w2) + (w1 + w3), so one partial per
  // block reaches memory and the grid can hold many more waves for the same partial traffic.
  static_assert(kSeWaves == 4, "two reduction rounds");
  __shared__ floatx4 red[2][OB * KB][kWave];
  if (w >= 2)
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) red[w - 2][ob * KB + kb][lane] = acc[ob][kb];
  __syncthreads();
  if (w < 2)
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) acc[ob][kb] += red[w][ob * KB + kb][lane];
  __syncthreads();
  if (w == 1)
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) red[0][ob * KB + kb][lane] = acc[ob][kb];
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc[ob][kb] += red[0][ob * KB + kb][lane];
  float* my = part + static_cast<int64_t>(blockIdx.x) * Opad * Kpad;
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int o = 16 * (ob0 + ob) + 4 * g + q, k = 16 * (kb0 + kb) + li;
        if (o < Opad && k < Kpad) my[static_cast<int64_t>(o) * Kpad + k] = acc[ob][kb][q];
      }
}

// Destinations of the product's columns: part j (j < n <= 3) covers columns [c[j], c[j+1]) and
// is written row-major with row stride ld[j] at p[j] (skipped when p[j] is null).
struct TnOut {
  int n;
  int c[4];
  float* p[3];
  int ld[3];
};

__global__ __launch_bounds__(kSeThreads) void se3_gemm_tn_final(const float* __restrict__ part,
                                                               int nparts, int Opad, int Kpad,
                                                               int O, int K, TnOut out) {
  __shared__ float red[4][64];
  const int kl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 64 + kl;
  const int64_t n = static_cast<int64_t>(Opad) * Kpad;
  float s = 0.f;
  if (idx < n) {
#pragma unroll 8
    for (int b = grp; b < nparts; b += 4) s += part[b * n + idx];
  }
  red[grp][kl] = s;
  __syncthreads();
  if (grp != 0 || idx >= n) return;
  const int o = static_cast<int>(idx / Kpad), k = static_cast<int>(idx % Kpad);
  if (o >= O || k >= K) return;
  int j = 0;
  while (j + 1 < out.n && k >= out.c[j + 1]) ++j;
  if (out.p[j] != nullptr)
    out.p[j][static_cast<int64_t>(o) * out.ld[j] + (k - out.c[j])] =
        ((red[0][kl] + red[1][kl]) + red[2][kl]) + red[3][kl];
}

// Column sums of a row-major [N][O] matrix over the rows whose mask byte is non-zero (all rows
// without a mask), in two launches with a fixed summation order (results reproducible bit for
// bit).  se3_colsum_part: block b sums rows [b R, (b + 1) R) into part[b][o].  When O is a
// multiple of 4 and the matrix 16-byte aligned, a lane holds four columns (16-byte loads), the
// lanes of a 64-column chunk form 16-lane rows, and a wave issues its rows sixteen loads at a time
// before adding them (16 KB in flight per wave: about one memory round trip for the whole
// matrix); the four 16-lane rows of a wave and then the four waves are added in order.  Otherwise
// a thread per column walks every fourth row, eight in flight.  se3_colsum_final adds the block
// partials, sixteen groups over the blocks, in group order.
constexpr int kColsumBlocks = 256;
constexpr int kColsumFinalThreads = 1024;  // 16 groups of 64 columns

template <bool VEC4>
__global__ __launch_bounds__(kSeThreads) void se3_colsum_part(const float* __restrict__ g,
                                                             int64_t N, int O,
                                                             const uint8_t* __restrict__ mask,
                                                             int64_t R, float* __restrict__ part) {
  __shared__ float red[kSeWaves][64];
  const int lane = lane_id(), w = threadIdx.x / kWave;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * R;
  const int64_t r1 = r0 + R < N ? r0 + R : N;
  if constexpr (VEC4) {
    // wave w takes rows r0 + 4 w + rr (rr = lane / 16), then every 16th row; lane % 16 = column quad
    const int cq = lane & 15, rr = lane >> 4;
    for (int c0 = 0; c0 < O; c0 += 64) {
      const int o = c0 + 4 * cq;  // first of the lane's four columns
      float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
      if (o < O) {
        int64_t r = r0 + 4 * w + rr;
        for (; r + 15 * 16 < r1; r += 16 * 16) {
          float4 v[16];
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const int64_t q = r + 16 * k;
            const float4 x = *reinterpret_cast<const float4*>(g + q * O + o);
            const bool on = mask == nullptr || mask[q] != 0;
            v[k] = on ? x : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int k = 0; k < 16; ++k) { s.x += v[k].x; s.y += v[k].y; s.z += v[k].z; s.w += v[k].w; }
        }
        for (; r < r1; r += 16) {
          const float4 x = *reinterpret_cast<const float4*>(g + r * O + o);
          if (mask == nullptr || mask[r] != 0) { s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w; }
        }
      }
      // the wave's four 16-lane rows, in order: lanes cq, cq + 16, cq + 32, cq + 48
      float t[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a1 = __shfl(t[k], cq + 16, kWave), a2 = __shfl(t[k], cq + 32, kWave),
                    a3 = __shfl(t[k], cq + 48, kWave), a0 = __shfl(t[k], cq, kWave);
        t[k] = ((a0 + a1) + a2) + a3;
      }
      if (rr == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) red[w][4 * cq + k] = t[k];
      }
      __syncthreads();
      if (w == 0 && c0 + lane < O) {
        float u = red[0][lane];
#pragma unroll
        for (int ww = 1; ww < kSeWaves; ++ww) u += red[ww][lane];
        part[static_cast<int64_t>(blockIdx.x) * O + c0 + lane] = u;
      }
      __syncthreads();
    }
  } else {
    // a thread per column: wave w takes rows r0 + w, r0 + w + 4, ...
    for (int c0 = 0; c0 < O; c0 += 64) {
      const int o = c0 + lane;
      float s = 0.f;
      if (o < O) {
        int64_t r = r0 + w;
        for (; r + 28 < r1; r += 32) {
          float v[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int64_t q = r + 4 * k;
            const float x = g[q * O + o];
            v[k] = (mask == nullptr || mask[q] != 0) ? x : 0.f;
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) s += v[k];
        }
        for (; r < r1; r += 4) {
          const float x = g[r * O + o];
          s += (mask == nullptr || mask[r] != 0) ? x : 0.f;
        }
      }
      red[w][lane] = s;
      __syncthreads();
      if (w == 0 && o < O) {
        float u = red[0][lane];
#pragma unroll
        for (int ww = 1; ww < kSeWaves; ++ww) u += red[ww][lane];
        part[static_cast<int64_t>(blockIdx.x) * O + o] = u;
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(kColsumFinalThreads) void se3_colsum_final(const float* __restrict__ part,
                                                                        int nb, int O,
                                                                        float* __restrict__ out) {
  constexpr int kGroups = kColsumFinalThreads / 64;
  __shared__ float red[kGroups][64];
  const int cl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int o = blockIdx.x * 64 + cl;
  float s = 0.f;
  if (o < O) {
    int b = grp;
    for (; b + 7 * kGroups < nb; b += 8 * kGroups) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = part[static_cast<int64_t>(b + k * kGroups) * O + o];
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[k];
    }
    for (; b < nb; b += kGroups) s += part[static_cast<int64_t>(b) * O + o];
  }
  red[grp][cl] = s;
  __syncthreads();
  if (grp == 0 && o < O) {
    float t = red[0][cl];
#pragma unroll
    for (int gg = 1; gg < kGroups; ++gg) t += red[gg][cl];
    out[o] = t;
  }
}

struct TnPlan {
  int ob, kb, kb_groups, groups, nparts_x;
  int64_t rows_per_wave;
};

TnPlan tn_plan(int64_t M, int O, int K) {
  TnPlan t;
  const int nob = (O + 15) / 16, nkb = (K + 15) / 16;
  t.ob = nob <= 1 ? 1 : 2;  // wider O tiles spill accumulators in the LDS reduction
  const int kb = nkb < 8 ? nkb : 8;
  t.kb = kb <= 2 ? 2 : (kb <= 4 ? 4 : (kb <= 6 ? 6 : 8));
  t.kb_groups = (nkb + t.kb - 1) / t.kb;
  t.groups = ((nob + t.ob - 1) / t.ob) * t.kb_groups;
  // about 64 rows per wave (four 16-row steps), at most 512 blocks (2048 waves)
  int64_t blocks = ceil_div(M, 256);
  blocks = blocks < 1 ? 1 : (blocks > 512 ? 512 : blocks);
  t.nparts_x = static_cast<int>(blocks);
  t.rows_per_wave = ceil_div(ceil_div(M, blocks * kSeWaves), 16) * 16;
  return t;
}

// ------------------------------------------------------------------- weight packing ---
// The GEMMs read the nine path weights W_p [out][in] as zero-padded blocks (one launch builds
// them all instead of a zeroing pass and a copy per block).  Block kinds (rows x cols):
//   0 Ws  [Os][Cs|Cv|Ct]      = [W0 | W3 | W8]         forward, scalar outputs
//   1 Wv  [Ov][Cs|Cv|Cv]      = [W1 | W2 | W4]         forward, vector outputs
//   2 Wt  [Ot][Cs|Ct|Cv]      = [W5 | W6 | W7]         forward, type-2 outputs
//   3-5   the transposes of 0-2 (rows = input slots, cols = outputs)     backward, gX = g W
//   6 Bs  [Cs][Os|Ov|Ot]      = [W0^T | W1^T | W5^T]   backward, d scalars
//   7 Bv  [Cv][Ov|Os|Ov|Ot]   = [W2^T | W3^T | W4^T | W7^T]
//   8 Bt  [Ct][Ot]            = W6^T
//   9 B8  [Ct][Os]            = W8^T
struct SePackOut {
  float* p;
  int rows, cols, kind;  // rows / cols of the padded block; entries outside the real block are 0
};
struct SePack {
  const float* W[kSePaths];
  int Cs, Cv, Ct, Os, Ov, Ot;
  int nout;
  SePackOut out[10];
  int64_t start[11];  // element offsets of the outputs in the flattened launch
};

__device__ __forceinline__ float w_at(const SePack& k, int path, int o, int i, int O, int I) {
  return (k.W[path] && o < O && i < I) ? k.W[path][o * I + i] : 0.f;
}

__device__ float pack_elem(const SePack& k, int kind, int r, int c) {
  const int Cs = k.Cs, Cv = k.Cv, Ct = k.Ct, Os = k.Os, Ov = k.Ov, Ot = k.Ot;
  if (kind >= 3 && kind <= 5) {  // transpose of the forward block
    const int t = r;
    r = c;
    c = t;
    kind -= 3;
  }
  switch (kind) {
    case 0:
      if (r >= Os) return 0.f;
      if (c < Cs) return w_at(k, 0, r, c, Os, Cs);
      if (c < Cs + Cv) return w_at(k, 3, r, c - Cs, Os, Cv);
      return w_at(k, 8, r, c - Cs - Cv, Os, Ct);
    case 1:
      if (r >= Ov) return 0.f;
      if (c < Cs) return w_at(k, 1, r, c, Ov, Cs);
      if (c < Cs + Cv) return w_at(k, 2, r, c - Cs, Ov, Cv);
      return w_at(k, 4, r, c - Cs - Cv, Ov, Cv);
    case 2:
      if (r >= Ot) return 0.f;
      if (c < Cs) return w_at(k, 5, r, c, Ot, Cs);
      if (c < Cs + Ct) return w_at(k, 6, r, c - Cs, Ot, Ct);
      return w_at(k, 7, r, c - Cs - Ct, Ot, Cv);
    case 6:
      if (r >= Cs) return 0.f;
      if (c < Os) return w_at(k, 0, c, r, Os, Cs);
      if (c < Os + Ov) return w_at(k, 1, c - Os, r, Ov, Cs);
      return w_at(k, 5, c - Os - Ov, r, Ot, Cs);
    case 7:
      if (r >= Cv) return 0.f;
      if (c < Ov) return w_at(k, 2, c, r, Ov, Cv);
      if (c < Ov + Os) return w_at(k, 3, c - Ov, r, Os, Cv);
      if (c < 2 * Ov + Os) return w_at(k, 4, c - Ov - Os, r, Ov, Cv);
      return w_at(k, 7, c - 2 * Ov - Os, r, Ot, Cv);
    case 8:
      return r < Ct ? w_at(k, 6, c, r, Ot, Ct) : 0.f;
    default:
      return r < Ct ? w_at(k, 8, c, r, Os, Ct) : 0.f;
  }
}

__global__ __launch_bounds__(kSeThreads) void se3_pack_kernel(SePack k) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= k.start[k.nout]) return;
  int j = 0;
  while (j + 1 < k.nout && t >= k.start[j + 1]) ++j;
  const SePackOut& o = k.out[j];
  const int64_t local = t - k.start[j];
  const int r = static_cast<int>(local / o.cols), c = static_cast<int>(local % o.cols);
  o.p[local] = pack_elem(k, o.kind, r, c);
}

// ------------------------------------------------------------------ backward helpers ---
// out[n][g][o] (row length Opad, zero padded) = in[n][o][g] / avg[n], zero where mask[n] == 0.
__global__ __launch_bounds__(kSeThreads) void se3_grad_prep(const float* __restrict__ gin, int64_t N,
                                                           int O, int G, int Opad,
                                                           const float* __restrict__ avg,
                                                           const uint8_t* __restrict__ mask,
                                                           float* __restrict__ out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N * G * Opad) return;
  const int o = static_cast<int>(t % Opad);
  const int64_t ng = t / Opad;
  const int64_t n = ng / G;
  const int gc = static_cast<int>(ng - n * G);
  float val = 0.f;
  if (o < O && (mask == nullptr || mask[n] != 0)) {
    val = gin[(n * O + o) * G + gc];
    if (avg) val = val / avg[n];
  }
  out[t] = val;
}

// v + (v of the DPP source lane); lanes without a source, or outside ROWS, add 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_add(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, true);
  return v + __int_as_float(s);
}

// Lane 0 of a row turns the 21 per-edge sums into the edge's gradients of R, the direction and Y
// (without T2 only S[0..15] are read).
template <bool T2>
__device__ __forceinline__ void write_edge_grads(const SeEdges& g, const EdgeScalars& q,
                                                 const float* S, float* dR, float* ddir,
                                                 float* dY) {
  const int64_t e = q.e;
  const float* d = q.d;
  if (dR) {
    float* o = dR + e * g.P;
    float val[kSePaths];
    val[0] = q.y0 * S[0];
    val[1] = (d[0] * S[1] + d[1] * S[2]) + d[2] * S[3];
    val[2] = q.y0 * S[9];
    val[3] = (d[0] * S[10] + d[1] * S[11]) + d[2] * S[12];
    val[4] = (d[0] * S[13] + d[1] * S[14]) + d[2] * S[15];
    if (T2) {
      val[5] = (((q.y2[0] * S[4] + q.y2[1] * S[5]) + q.y2[2] * S[6]) + q.y2[3] * S[7]) + q.y2[4] * S[8];
      val[6] = q.y0 * S[19];
      val[7] = (d[0] * S[16] + d[1] * S[17]) + d[2] * S[18];
      val[8] = S[20];
    }
#pragma unroll
    for (int i = 0; i < (T2 ? kSePaths : 5); ++i)
      if (g.pc[i] >= 0) o[g.pc[i]] = val[i];
  }
  if (ddir) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      float v = q.r[1] * S[1 + k] + q.r[3] * S[10 + k] + q.r[4] * S[13 + k];
      if (T2) v += q.r[7] * S[16 + k];
      ddir[3 * e + k] = v;
    }
  }
  if (dY) {
    float* o = dY + e * g.ysh;
    float v0 = q.r[0] * S[0] + q.r[2] * S[9];
    if (T2) v0 += q.r[6] * S[19];
    o[0] = v0;
    if (T2 && g.ysh >= 9) {
#pragma unroll
      for (int k = 0; k < 5; ++k) o[4 + k] = q.r[5] * S[4 + k];
    }
  }
}

// Sum over the 16 lanes of each row; every lane of the row receives its row's total.
__device__ __forceinline__ float row_total(float v) {
  v = dpp_add<kDppXor1, 0xF>(v);
  v = dpp_add<kDppXor2, 0xF>(v);
  v = dpp_add<kDppHalfMirror, 0xF>(v);
  v = dpp_add<kDppMirror, 0xF>(v);
  return v;
}

// The target's gradient row for one channel chunk, as held by one lane: scalar-input channels
// c = cs0 + 4 li + u (u < 4), vector and type-2 input channels c = cv0 + li.
struct GRow {
  float s0[4], s1[3][4], s5[5][4];
  float v2[3], v3, v4[3], v7c[3][3];  // v7c[i][j] = sum_m cg[i][j][m] G7_m
  float t6[5], t8;
};

template <bool T2>
__device__ __forceinline__ void load_grow(GRow& G, const SeFeat& f, const float* cg, int64_t n,
                                          int h, int li, const float* Gs, int Ks, const float* Gv,
                                          int Kv, const float* Gt, int Kt) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = 64 * h + 4 * li + u;
    const bool ok = c < f.Cs;
    G.s0[u] = ok && Gs ? Gs[n * Ks + c] : 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) G.s1[k][u] = ok && Gv ? Gv[(n * 3 + k) * Kv + c] : 0.f;
#pragma unroll
    for (int k = 0; k < 5; ++k) G.s5[k][u] = T2 && ok && Gt ? Gt[(n * 5 + k) * Kt + c] : 0.f;
  }
  const int c = 16 * h + li;
  const bool okv = c < f.Cv, okt = T2 && c < f.Ct;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    G.v2[k] = okv && Gv ? Gv[(n * 3 + k) * Kv + f.Cs + c] : 0.f;
    G.v4[k] = okv && Gv ? Gv[(n * 3 + k) * Kv + f.Cs + f.Cv + c] : 0.f;
  }
  G.v3 = okv && Gs ? Gs[n * Ks + f.Cs + c] : 0.f;
  float v7[5];
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    v7[k] = T2 && okv && Gt ? Gt[(n * 5 + k) * Kt + f.Cs + f.Ct + c] : 0.f;
    G.t6[k] = okt && Gt ? Gt[(n * 5 + k) * Kt + f.Cs + c] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      if (cg == nullptr) {
        G.v7c[i][j] = 0.f;
        continue;
      }
      const float* cc = cg + (i * 3 + j) * 5;
      G.v7c[i][j] = (((cc[0] * v7[0] + cc[1] * v7[1]) + cc[2] * v7[2]) + cc[3] * v7[3]) + cc[4] * v7[4];
    }
  G.t8 = okt && Gs ? Gs[n * Ks + f.Cs + f.Cv + c] : 0.f;
}

// Per-edge gradients of R, the direction and Y.  One wave per target node n; its four 16-lane
// rows take four edges at a time (row r: edge j0 + r), the lanes of a row split the channels
// (64 scalar channels as 4 per lane, 16 vector / type-2 channels as 1 per lane, per chunk), and
// the 21 per-edge sums are reduced within the row.  With one chunk (ONE) the target's gradient
// row stays in registers for all of its edges.
// Without the type-2 paths the kernel fits 75 registers: six waves per SIMD instead of four
// (measured 207 -> 165 us at C2); with them the register file sets the occupancy.
template <bool ONE, bool T2>
__global__ __launch_bounds__(kSeThreads, T2 ? 1 : 6) void se3_bwd_edge(SeEdges g, SeFeat f,
                                                          const float* __restrict__ Gs, int Ks,
                                                          const float* __restrict__ Gv, int Kv,
                                                          const float* __restrict__ Gt, int Kt,
                                                          float* __restrict__ dR,
                                                          float* __restrict__ ddir,
                                                          float* __restrict__ dY) {
  const int64_t n = xcd_block() * kSeWaves + uniform(threadIdx.x / kWave);
  if (n >= g.N) return;
  const int lane = lane_id();
  const int row = lane >> 4, li = lane & 15;
  int a, b;
  node_range(g, n, a, b);
  const int nch = ONE ? 1 : max((f.Cs + 63) / 64, max((f.Cv + 15) / 16, (f.Ct + 15) / 16));
  GRow G;
  if (ONE) load_grow<T2>(G, f, g.cg, n, 0, li, Gs, Ks, Gv, Kv, Gt, Kt);
  for (int base = a; base < b; base += kWave) {
    const int cnt = min(kWave, b - base);
    const EdgeScalars st = stage_edges(g, base, cnt, lane);
    for (int j0 = 0; j0 < cnt; j0 += 4) {
      const int j = j0 + row;
      const EdgeScalars q = edge_from(st, min(j, kWave - 1));
      const bool ok = j < cnt && q.ok;
      const int64_t m = ok ? q.other : 0;
      float S[21];
#pragma unroll
      for (int i = 0; i < 21; ++i) S[i] = 0.f;
      for (int h = 0; h < nch; ++h) {
        if (!ONE) load_grow<T2>(G, f, g.cg, n, h, li, Gs, Ks, Gv, Kv, Gt, Kt);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = 64 * h + 4 * li + u;
          if (c < f.Cs) {
            const float x = f.s[m * f.Cs + c];
            S[0] += G.s0[u] * x;
#pragma unroll
            for (int k = 0; k < 3; ++k) S[1 + k] += G.s1[k][u] * x;
#pragma unroll
            for (int k = 0; k < 5; ++k)
              if (T2) S[4 + k] += G.s5[k][u] * x;
          }
        }
        const int c = 16 * h + li;
        if (c < f.Cv) {
          const float* vp = f.v + (m * f.Cv + c) * 3;
          const float v[3] = {vp[0], vp[1], vp[2]};
          S[9] += (G.v2[0] * v[0] + G.v2[1] * v[1]) + G.v2[2] * v[2];
#pragma unroll
          for (int k = 0; k < 3; ++k) S[10 + k] += G.v3 * v[k];
          S[13] += v[1] * G.v4[2] - v[2] * G.v4[1];  // v x G4
          S[14] += v[2] * G.v4[0] - v[0] * G.v4[2];
          S[15] += v[0] * G.v4[1] - v[1] * G.v4[0];
          if (T2) {
#pragma unroll
            for (int i = 0; i < 3; ++i)
              S[16 + i] += (v[0] * G.v7c[i][0] + v[1] * G.v7c[i][1]) + v[2] * G.v7c[i][2];
          }
        }
        if (T2 && c < f.Ct) {
          const float* tp = f.t + (m * f.Ct + c) * 5;
          const float t[5] = {tp[0], tp[1], tp[2], tp[3], tp[4]};
          S[19] += (((G.t6[0] * t[0] + G.t6[1] * t[1]) + G.t6[2] * t[2]) + G.t6[3] * t[3]) + G.t6[4] * t[4];
          S[20] += G.t8 * ((((t[0] * t[0] + t[1] * t[1]) + t[2] * t[2]) + t[3] * t[3]) + t[4] * t[4]);
        }
      }
#pragma unroll
      for (int i = 0; i < 21; ++i)
        if (T2 || i < 4 || (i >= 9 && i < 16)) S[i] = row_total(S[i]);
      if (li == 0 && ok) write_edge_grads<T2>(g, q, S, dR, ddir, dY);
    }
  }
}

// Per-edge gradients for layers without type-2 paths, Cs <= 64 (a multiple of 4), Cv <= 16 (the target's
// gradient row in registers, as se3_bwd_edge<true, false>): the same sums in the same order, with
// the source rows read by buffer loads whose offsets point past the arrays for channels a lane
// does not hold (zeros), so no load carries a per-lane condition, and U steps of four edges
// (row r: edge j0 + 4 u + r) in flight.
template <int U>
__device__ __forceinline__ void edge_rows_walk(const SeEdges& g, const SeFeat& f, int64_t n,
                                               const GRow& G, int lane, float* __restrict__ dR,
                                               float* __restrict__ ddir, float* __restrict__ dY) {
  const int row = lane >> 4, li = lane & 15;
  int a, b;
  node_range(g, n, a, b);
  const auto rs = row_rsrc(f.s, static_cast<int>(g.N * f.Cs * 4));
  const auto rv = row_rsrc(f.v, static_cast<int>(g.N * f.Cv * 12));
  // byte offset of the lane's scalar channels 4 li .. 4 li + 3 inside a row (Cs is a multiple of
  // 4), or past the arrays
  const uint32_t cs = 4 * li < f.Cs ? 16u * li : kPastRows;
  const uint32_t cv = li < f.Cv ? 12u * li : kPastRows;
  for (int base = a; base < b; base += kWave) {
    const int cnt = min(kWave, b - base);
    const EdgeScalars st = stage_edges(g, base, cnt, lane);
    for (int j0 = 0; j0 < cnt; j0 += 4 * U) {
      float x[U][4], v[U][3];
#pragma unroll
      for (int u = 0; u < U; ++u) {  // every step's source rows first
        const int jj = j0 + 4 * u + row;
        // the shuffles run on every lane: a lane shuffle under a condition reads zeros from
        // source lanes the condition switched off (the staging lane of an edge sits in another row)
        const int src = __shfl(st.other, min(jj, kWave - 1), kWave);
        const int okl = __shfl(st.ok, min(jj, kWave - 1), kWave);
        const bool ok = jj < cnt && okl != 0;
        const uint32_t ms = ok ? static_cast<uint32_t>(src) * (4u * f.Cs) : kPastRows;
        const uint32_t mv = ok ? static_cast<uint32_t>(src) * (12u * f.Cv) : kPastRows;
        const auto xs = __builtin_amdgcn_raw_buffer_load_b128(rs, cs == kPastRows ? kPastRows : ms + cs,
                                                              0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) x[u][q] = __uint_as_float(xs[q]);  // element by value
        const uint32_t vo = cv == kPastRows ? kPastRows : mv + cv;
#pragma unroll
        for (int k = 0; k < 3; ++k) v[u][k] = ld_row(rv, vo + 4u * k);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int jj = j0 + 4 * u + row;
        if (j0 + 4 * u >= cnt) break;  // wave-uniform
        float S[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (4 * li + q < f.Cs) {
            S[0] += G.s0[q] * x[u][q];
#pragma unroll
            for (int k = 0; k < 3; ++k) S[1 + k] += G.s1[k][q] * x[u][q];
          }
        }
        if (li < f.Cv) {
          const float* w = v[u];
          S[9] += (G.v2[0] * w[0] + G.v2[1] * w[1]) + G.v2[2] * w[2];
#pragma unroll
          for (int k = 0; k < 3; ++k) S[10 + k] += G.v3 * w[k];
          S[13] += w[1] * G.v4[2] - w[2] * G.v4[1];  // v x G4
          S[14] += w[2] * G.v4[0] - w[0] * G.v4[2];
          S[15] += w[0] * G.v4[1] - w[1] * G.v4[0];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (i < 4 || i >= 9) S[i] = row_total(S[i]);
        const EdgeScalars q = edge_from(st, min(jj, kWave - 1));
        // without the type-2 paths write_edge_grads reads S[0..15] only
        if (li == 0 && jj < cnt && q.ok) write_edge_grads<false>(g, q, S, dR, ddir, dY);
      }
    }
  }
}

template <int U>
__global__ __launch_bounds__(kSeThreads, 6) void se3_bwd_edge_rows(SeEdges g, SeFeat f,
                                                                  const float* __restrict__ Gs,
                                                                  int Ks,
                                                                  const float* __restrict__ Gv,
                                                                  int Kv, float* __restrict__ dR,
                                                                  float* __restrict__ ddir,
                                                                  float* __restrict__ dY) {
  const int64_t n = xcd_block() * kSeWaves + uniform(threadIdx.x / kWave);
  if (n >= g.N) return;
  const int lane = lane_id();
  GRow G;
  load_grow<false>(G, f, nullptr, n, 0, lane & 15, Gs, Ks, Gv, Kv, nullptr, 0);
  edge_rows_walk<U>(g, f, n, G, lane, dR, ddir, dY);
}

// The tile's rows times the packed weights, into LDS: out[r][o] = sum_k A[r][k] W[o][k] for the
// 16 G rows r of A (LDS, row stride lda) and the columns o < 16 ceil(O / 16) (W has that many
// rows, zero past O), written with row stride ldo.  The MFMA fragments and the k order are
// fused_gemm's (and se3_gemm's), so the result equals theirs bit for bit.  Wave w takes the
// blocks whose running number base + b is w mod 4.
template <int G>
__device__ __forceinline__ void lds_gemm(const float* A, int lda, int K, const float* __restrict__ W,
                                         int O, float* out, int ldo, int base, int wave, int lane) {
  const int ncb = (O + 15) / 16;
  const int nblk = G * ncb;
  const int li = lane & 15, lk = lane >> 4;
  for (int b = (wave - base % kSeWaves + kSeWaves) % kSeWaves; b < nblk; b += kSeWaves) {
    const int rb = b / ncb, cb = b % ncb;
    const float* ap = A + (rb * 16 + li) * lda + 4 * lk;
    const float* bp = W + static_cast<int64_t>(cb * 16 + li) * K + 4 * lk;
    const floatx4 acc = mfma_k_loop(
        [&](int k) { return *reinterpret_cast<const floatx4*>(ap + k); },
        [&](int k) { return *reinterpret_cast<const floatx4*>(bp + k); }, K);
#pragma unroll
    for (int q = 0; q < 4; ++q) out[(rb * 16 + 4 * lk + q) * ldo + cb * 16 + li] = acc[q];
  }
}

// lds_gemm with A read from global memory: rows row0 .. row0 + 16 G - 1 of a row-major [rows][K]
// matrix behind the buffer resource ra (rows past its end read zeros).
template <int G>
__device__ __forceinline__ void lds_gemm_ga(__amdgpu_buffer_rsrc_t ra, int64_t row0, int K,
                                            const float* __restrict__ W, int O, float* out, int ldo,
                                            int base, int wave, int lane) {
  const int ncb = (O + 15) / 16;
  const int nblk = G * ncb;
  const int li = lane & 15, lk = lane >> 4;
  for (int b = (wave - base % kSeWaves + kSeWaves) % kSeWaves; b < nblk; b += kSeWaves) {
    const int rb = b / ncb, cb = b % ncb;
    const uint32_t arow = static_cast<uint32_t>((row0 + rb * 16 + li) * K * 4 + 16 * lk);
    const float* bp = W + static_cast<int64_t>(cb * 16 + li) * K + 4 * lk;
    const floatx4 acc = mfma_k_loop(
        [&](int k) {
          const auto v = __builtin_amdgcn_raw_buffer_load_b128(ra, arow + 4u * k, 0, 0);
          floatx4 a;
#pragma unroll
          for (int q = 0; q < 4; ++q) a[q] = __uint_as_float(v[q]);  // element by value
          return a;
        },
        [&](int k) { return *reinterpret_cast<const floatx4*>(bp + k); }, K);
#pragma unroll
    for (int q = 0; q < 4; ++q) out[(rb * 16 + 4 * lk + q) * ldo + cb * 16 + li] = acc[q];
  }
}

// se3_bwd_edge_rows with gX formed in LDS: a workgroup takes 16 consecutive targets, multiplies
// their prepared output-gradient rows (Gs [16][OsP], Gv [48][OvP], read as MFMA fragments straight
// from memory; zeros past N) by the packed transposed weights into the tile's gX rows in LDS
// (gXs = Gs WsT^T, gXv = Gv WvT^T, as the GEMMs of the unfused path compute them, bit for bit),
// and each wave then walks the edges of four of the targets in turn, its gradient row read from
// the tile; gX never reaches HBM.  (Staging the gradient rows in LDS as well took 32 KB per
// workgroup: five waves per SIMD instead of six.)
struct SeEdgeTile {
  const float* Gs;   // [N][OsP] or NULL
  const float* Gv;   // [N][3][OvP] or NULL
  const float* WsT;  // [>= 16 ceil(Ks / 16)][OsP]
  const float* WvT;  // [>= 16 ceil(Kv / 16)][OvP]
  int OsP, OvP, Ks, Kv;
};

__host__ __device__ inline size_t edge_tile_floats(int Ks, int Kv) {
  return static_cast<size_t>(kFuTile) * (Ks + 4) + 3 * kFuTile * (Kv + 4);
}

template <int U>
__global__ __launch_bounds__(kSeThreads, 5) void se3_bwd_edge_tile(SeEdges g, SeFeat f, SeEdgeTile q,
                                                                  float* __restrict__ dR,
                                                                  float* __restrict__ ddir,
                                                                  float* __restrict__ dY) {
  extern __shared__ floatx4 et_lds[];
  const int ldxs = q.Ks + 4, ldxv = q.Kv + 4;
  float* xS = reinterpret_cast<float*>(et_lds);
  float* xV = xS + kFuTile * ldxs;
  const int64_t node0 = xcd_block() * kFuTile;
  const int wave = uniform(threadIdx.x / kWave), lane = lane_id();
  // the A fragments straight from the gradient rows (rows past N read zeros)
  const int nb0 = q.Gs ? (q.Ks + 15) / 16 : 0;
  if (q.Gs)
    lds_gemm_ga<1>(row_rsrc(q.Gs, static_cast<int>(g.N * q.OsP * 4)), node0, q.OsP, q.WsT, q.Ks, xS,
                   ldxs, 0, wave, lane);
  if (q.Gv)
    lds_gemm_ga<3>(row_rsrc(q.Gv, static_cast<int>(g.N * 3 * q.OvP * 4)), node0 * 3, q.OvP, q.WvT,
                   q.Kv, xV, ldxv, nb0, wave, lane);
  __syncthreads();
  for (int tt = 0; tt < kFuTile / kSeWaves; ++tt) {
    const int r = (kFuTile / kSeWaves) * wave + tt;
    const int64_t n = node0 + r;
    if (n >= g.N) break;  // wave-uniform
    GRow G;
    load_grow<false>(G, f, nullptr, r, 0, lane & 15, q.Gs ? xS : nullptr, ldxs,
                     q.Gv ? xV : nullptr, ldxv, nullptr, 0);
    edge_rows_walk<U>(g, f, n, G, lane, dR, ddir, dY);
  }
}

// Whether se3_bwd_edge_rows covers the call, with both feature arrays below 2 GiB.
bool bwd_edge_rows_ok(int64_t N, int Cs, int Cv, bool t2) {
  const int64_t lim = int64_t{1} << 31;
  return !t2 && Cs <= 64 && Cs % 4 == 0 && Cv <= 16 && N * Cs * 4 < lim && N * Cv * 12 < lim;
}

// Source-side sums of the output-gradient rows (edges grouped by source m; the wave's lanes
// run over output channels, the target's rows are gathered per edge, four edges in flight):
//   Zs[m]    = [Z0 (Os) | Z1 (Ov) | Z5 (Ot)]                 -> ds = Zs [W0|W1|W5]
//   Zv[m][k] = [Z2_k (Ov) | Z3_k (Os) | Z4_k (Ov) | Z7_k (Ot)] -> dv = Zv [W2|W3|W4|W7]
//   Zt[m][j] = [Z6_j (Ot)]                                   -> dt = Zt W6 + 2 t (Z8 W8)
//   Z8[m]    = [Z8 (Os)]
// with gs [N, Os], gv [N][3][Ov], gt [N][5][Ot] the prepared output gradients.
template <bool T2>
__global__ __launch_bounds__(kSeThreads) void se3_bwd_src(SeEdges g, const float* __restrict__ gs,
                                                         int Os, int OsP,
                                                         const float* __restrict__ gv, int Ov,
                                                         int OvP, const float* __restrict__ gt,
                                                         int Ot, int OtP, float* __restrict__ Zs,
                                                         int KZs, float* __restrict__ Zv, int KZv,
                                                         float* __restrict__ Zt, int KZt,
                                                         float* __restrict__ Z8, int KZ8) {
  const int64_t m = xcd_block() * kSeWaves + uniform(threadIdx.x / kWave);
  if (m >= g.N) return;
  const int lane = lane_id();
  int a, b;
  node_range(g, m, a, b);
  const int omax = max(Os, max(Ov, Ot));
  for (int o0 = 0; o0 < omax; o0 += kWave) {
    const int o = o0 + lane;
    const bool hs = o < Os && gs, hv = o < Ov && gv, ht = T2 && o < Ot && gt;
    float z0 = 0.f, z1 = 0.f, z5 = 0.f, z8 = 0.f;
    float z2[3] = {0.f, 0.f, 0.f}, z3[3] = {0.f, 0.f, 0.f}, z4[3] = {0.f, 0.f, 0.f};
    float z7[3] = {0.f, 0.f, 0.f}, z6[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
    for (int base = a; base < b; base += kWave) {
      const int cnt = min(kWave, b - base);
      const EdgeCoef<T2> st = stage_coef<T2>(g, base, cnt, lane);
      for (int j0 = 0; j0 < cnt; j0 += kSeUnroll) {
        float ws[kSeUnroll], wv[kSeUnroll][3], wt[kSeUnroll][5];
#pragma unroll
        for (int u = 0; u < kSeUnroll; ++u) {
          const int j = min(j0 + u, kWave - 1);
          const int64_t n = __builtin_amdgcn_readlane(st.other, j);  // 0 past cnt: in bounds
          if (hs) ws[u] = gs[n * OsP + o];
          if (hv) {
#pragma unroll
            for (int k = 0; k < 3; ++k) wv[u][k] = gv[(n * 3 + k) * OvP + o];
          }
          if (ht) {
#pragma unroll
            for (int k = 0; k < 5; ++k) wt[u][k] = gt[(n * 5 + k) * OtP + o];
          }
        }
#pragma unroll
        for (int u = 0; u < kSeUnroll; ++u) {
          if (j0 + u >= cnt) break;
          const EdgeCoef<T2> q = coef_at<T2>(st, j0 + u);
          if (!q.ok) continue;
          if (hs) {
            const float gsv = ws[u];
            z0 += q.c0 * gsv;
#pragma unroll
            for (int k = 0; k < 3; ++k) z3[k] += q.c3[k] * gsv;
            if (T2) z8 += q.c8 * gsv;
          }
          if (hv) {
            const float* w = wv[u];
            z1 += (q.c1[0] * w[0] + q.c1[1] * w[1]) + q.c1[2] * w[2];
#pragma unroll
            for (int k = 0; k < 3; ++k) z2[k] += q.c2 * w[k];
            z4[0] += w[1] * q.c4[2] - w[2] * q.c4[1];  // w x (r4 d)
            z4[1] += w[2] * q.c4[0] - w[0] * q.c4[2];
            z4[2] += w[0] * q.c4[1] - w[1] * q.c4[0];
          }
          if (ht) {
            const float* w = wt[u];
            z5 += (((q.c5[0] * w[0] + q.c5[1] * w[1]) + q.c5[2] * w[2]) + q.c5[3] * w[3]) + q.c5[4] * w[4];
#pragma unroll
            for (int k = 0; k < 5; ++k) z6[k] += q.c6 * w[k];
#pragma unroll
            for (int jj = 0; jj < 3; ++jj)
              z7[jj] += (((q.d7[jj][0] * w[0] + q.d7[jj][1] * w[1]) + q.d7[jj][2] * w[2]) + q.d7[jj][3] * w[3]) +
                        q.d7[jj][4] * w[4];
          }
        }
      }
    }
    if (Zs) {
      float* row = Zs + m * KZs;
      if (hs) row[o] = z0;
      if (hv) row[Os + o] = z1;
      if (ht) row[Os + Ov + o] = z5;
    }
    if (Zv) {
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        float* row = Zv + (m * 3 + k) * KZv;
        if (hv) row[o] = z2[k];
        if (hs) row[Ov + o] = z3[k];
        if (hv) row[Ov + Os + o] = z4[k];
        if (ht) row[2 * Ov + Os + o] = z7[k];
      }
    }
    if (Zt) {
#pragma unroll
      for (int k = 0; k < 5; ++k)
        if (ht) Zt[(m * 5 + k) * KZt + o] = z6[k];
    }
    if (Z8 && hs) Z8[m * KZ8 + o] = z8;
  }
  // lanes whose group is absent wrote nothing: clear those slots and the padding
  if (Zs) {
    float* row = Zs + m * KZs;
    for (int q = lane; q < KZs; q += kWave) {
      const bool written = (q < Os && gs) || (q >= Os && q < Os + Ov && gv) ||
                           (q >= Os + Ov && q < Os + Ov + Ot && gt);
      if (!written) row[q] = 0.f;
    }
  }
  if (Zv) {
    for (int k = 0; k < 3; ++k) {
      float* row = Zv + (m * 3 + k) * KZv;
      for (int q = lane; q < KZv; q += kWave) {
        const bool written = (q < Ov && gv) || (q >= Ov && q < Ov + Os && gs) ||
                             (q >= Ov + Os && q < 2 * Ov + Os && gv) ||
                             (q >= 2 * Ov + Os && q < 2 * Ov + Os + Ot && gt);
        if (!written) row[q] = 0.f;
      }
    }
  }
  if (Zt)
    for (int k = 0; k < 5; ++k) {
      float* row = Zt + (m * 5 + k) * KZt;
      for (int q = lane; q < KZt; q += kWave)
        if (!(q < Ot && gt)) row[q] = 0.f;
    }
  if (Z8)
    for (int q = lane; q < KZ8; q += kWave)
      if (!(q < Os && gs)) Z8[m * KZ8 + q] = 0.f;
}


// Source-side sums in the row layout of se3_fwd_fused_rows (layers without type-2 paths,
// Os <= 64, Ov <= 16): a wave takes four sources, one per 16-lane row, over the CSR of the
// sources; lane j holds scalar-gradient channels 4j..4j+3 (one 16-byte load of the target's
// prepared row) and vector channel j (one dword per component row), so the gradient rows of four
// edges cost four vector-memory instructions where the channel-per-lane walk above issues four
// per edge.  Same products, in the same order, as se3_bwd_src.
//
// FUSED: the block's 16 sources (four waves x four rows: consecutive nodes) write their Z rows
// into an LDS tile laid out as the fused forward's aggregate tile (q.off / q.ld), and after a
// barrier the block multiplies the tile by the packed transposed weights there (fused_tile_out:
// ds = Zs Bs^T, dv = Zv Bv^T), so Z never reaches HBM.  q's epilogue operands (avg, bias, mask)
// and aggregate copies are NULL.
template <int U, bool FUSED>
__global__ __launch_bounds__(kSeThreads) void se3_bwd_src_rows(SeEdges g, const float* __restrict__ gs,
                                                              int Os, int OsP,
                                                              const float* __restrict__ gv, int Ov,
                                                              int OvP, float* __restrict__ Zs,
                                                              int KZs, float* __restrict__ Zv,
                                                              int KZv, SeFused q) {
  const int lane = lane_id();
  const int j = lane & 15;
  const int64_t m = (xcd_block() * kSeWaves + uniform(threadIdx.x / kWave)) * kRowNodes + (lane >> 4);
  int a = 0, b = 0;
  if (m < g.N) node_range(g, m, a, b);
  const int deg = b - a;
  const int maxdeg = max(max(__builtin_amdgcn_readlane(deg, 0), __builtin_amdgcn_readlane(deg, 16)),
                         max(__builtin_amdgcn_readlane(deg, 32), __builtin_amdgcn_readlane(deg, 48)));
  // whole-array resources (each below 2 GiB, checked by the host); an absent kind reads zeros
  const auto rs = row_rsrc(gs, gs ? static_cast<int>(g.N * OsP * 4) : 0);
  const auto rv = row_rsrc(gv, gv ? static_cast<int>(g.N * 3 * OvP * 4) : 0);
  const uint32_t rowb_s = 4u * OsP, rowb_v = 12u * OvP, kb = 4u * OvP;
  const uint32_t js = 16u * j, jv = 4u * j;
  float z0[4] = {0.f, 0.f, 0.f, 0.f}, z3[3][4] = {};
  float z1 = 0.f, z2[3] = {0.f, 0.f, 0.f}, z4[3] = {0.f, 0.f, 0.f};
  for (int base = 0; base < maxdeg; base += kRowStage) {
    const EdgeCoef<false> st = stage_rows(g, a + base + j, base + j < deg);
    const int cnt = min(kRowStage, maxdeg - base);
    static_for<0, kRowStage / U>([&](auto ci) {
      constexpr int c0 = decltype(ci)::value * U;
      if (c0 >= cnt) return;
      float sx[U][4], vx[U][3];
      static_for<0, U>([&](auto ui) {  // the U gradient rows of every row in flight together
        constexpr int uu = decltype(ui)::value;
        constexpr int u = c0 + uu;
        const bool have = row_bcast<u>(st.ok) != 0;
        const uint32_t n = static_cast<uint32_t>(row_bcast<u>(st.other));
        const auto ls = __builtin_amdgcn_raw_buffer_load_b128(rs, have ? n * rowb_s + js : kPastRows,
                                                              0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sx[uu][i] = __uint_as_float(ls[i]);  // element by value
        const uint32_t vo = have ? n * rowb_v + jv : kPastRows;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          vx[uu][k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, vo + k * kb, 0, 0));
      });
      static_for<0, U>([&](auto ui) {
        constexpr int uu = decltype(ui)::value;
        constexpr int u = c0 + uu;
        const bool ok = row_bcast<u>(st.ok) != 0;  // an absent edge adds nothing
        float x[4], w[3];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = ok ? sx[uu][i] : 0.f;
#pragma unroll
        for (int k = 0; k < 3; ++k) w[k] = ok ? vx[uu][k] : 0.f;
        const float c0v = row_bcast<u>(st.c0), c2v = row_bcast<u>(st.c2);
        float c1[3], c3[3], c4[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          c1[k] = row_bcast<u>(st.c1[k]);
          c3[k] = row_bcast<u>(st.c3[k]);
          c4[k] = row_bcast<u>(st.c4[k]);
        }
        if (gs) {  // an absent kind leaves its sums at zero, as se3_bwd_src does
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            z0[i] += c0v * x[i];
#pragma unroll
            for (int k = 0; k < 3; ++k) z3[k][i] += c3[k] * x[i];
          }
        }
        if (gv) {
          z1 += (c1[0] * w[0] + c1[1] * w[1]) + c1[2] * w[2];
#pragma unroll
          for (int k = 0; k < 3; ++k) z2[k] += c2v * w[k];
          z4[0] += w[1] * c4[2] - w[2] * c4[1];  // w x (r4 d)
          z4[1] += w[2] * c4[0] - w[0] * c4[2];
          z4[2] += w[0] * c4[1] - w[1] * c4[0];
        }
      });
    });
  }
  if constexpr (FUSED) {
    extern __shared__ floatx4 src_lds[];
    float* lds = reinterpret_cast<float*>(src_lds);
    const int64_t node0 = xcd_block() * kFuTile;  // m = node0 + 4 wave + lane / 16
    const int r = static_cast<int>(m - node0);
    if (m < g.N) {  // rows of nodes past N are never multiplied into an output
      // the tile rows as se3_bwd_src writes Zs / Zv, padding zeroed (the packed weights are
      // zero there, so a stale value could only turn into NaN)
      if (q.O[0] > 0) {
        float* row = lds + q.off[0] + r * q.ld[0];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * j + i < Os) row[4 * j + i] = z0[i];
        if (j < Ov) row[Os + j] = z1;
        for (int c = Os + Ov + j; c < KZs; c += 16) row[c] = 0.f;
      }
      if (q.O[1] > 0) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          float* row = lds + q.off[1] + (3 * r + k) * q.ld[1];
          if (j < Ov) {
            row[j] = z2[k];
            row[Ov + Os + j] = z4[k];
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (4 * j + i < Os) row[Ov + 4 * j + i] = z3[k][i];
          for (int c = 2 * Ov + Os + j; c < KZv; c += 16) row[c] = 0.f;
        }
      }
    }
    __syncthreads();
    fused_tile_out<false>(q, lds, node0, g.N, uniform(threadIdx.x / kWave), lane);
    return;
  }
  if (m >= g.N) return;
  // rows as se3_bwd_src writes them; columns of absent kinds and the padding are zeros
  if (Zs) {
    float* row = Zs + m * KZs;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * j + i < Os) row[4 * j + i] = z0[i];
    if (j < Ov) row[Os + j] = z1;
    for (int q = Os + Ov + j; q < KZs; q += 16) row[q] = 0.f;
  }
  if (Zv) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      float* row = Zv + (m * 3 + k) * KZv;
      if (j < Ov) {
        row[j] = z2[k];
        row[Ov + Os + j] = z4[k];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * j + i < Os) row[Ov + 4 * j + i] = z3[k][i];
      for (int q = 2 * Ov + Os + j; q < KZv; q += 16) row[q] = 0.f;
    }
  }
}

// Whether se3_bwd_src_rows covers the call, with every array it reads through a buffer
// resource below 2 GiB.
bool bwd_src_rows_ok(int64_t N, int Os, int OsP, int Ov, int OvP, bool t2, int64_t E, int P,
                     int ysh) {
  const int64_t lim = int64_t{1} << 31;
  return !t2 && Os <= 64 && Ov <= 16 && OsP % 4 == 0 && N * OsP * 4 < lim &&
         N * 3 * OvP * 4 < lim && E * 12 < lim && E * P * 4 < lim && E * ysh * 4 < lim;
}

SeEdges make_edges(const int64_t* other, const int32_t* perm, const int32_t* ns, const int32_t* ne,
                   int64_t N, int64_t E, const float* dir, const float* Y, int ysh, const float* R,
                   int P, const int32_t* path_cols, const float* cg) {
  SeEdges g;
  g.other = other;
  g.perm = perm;
  g.ns = ns;
  g.ne = ne;
  g.E = static_cast<int32_t>(E);
  g.N = N;
  g.dir = dir;
  g.Y = Y;
  g.ysh = ysh;
  g.R = R;
  g.P = P;
  for (int i = 0; i < kSePaths; ++i) g.pc[i] = path_cols[i];
  g.cg = path_cols[7] >= 0 ? cg : nullptr;
  return g;
}

int check_edges(const char* who, int64_t N, int64_t E, int ysh, int P, const int32_t* path_cols,
                const float* cg) {
  GEO_REQUIRE(N >= 0 && E >= 0, "%s: negative size", who);
  GEO_REQUIRE(N < 0x7fffffffLL && E < 0x7fffffffLL, "%s: sizes exceed int32 indexing", who);
  GEO_REQUIRE(path_cols, "%s: null path table", who);
  GEO_REQUIRE(path_cols[7] < 0 || cg, "%s: path 7 needs the CG table", who);
  GEO_REQUIRE(ysh >= 1, "%s: Y needs at least one channel", who);
  for (int i = 0; i < kSePaths; ++i)
    GEO_REQUIRE(path_cols[i] >= -1 && path_cols[i] < P, "%s: path %d uses column %d of R (P=%d)",
                who, i, path_cols[i], P);
  GEO_REQUIRE(path_cols[5] < 0 || ysh >= 9, "%s: path 5 needs Y with 9 channels", who);
  return GEO_OK;
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" int geo_se3_aggregate_fwd(const float* s, const float* v, const float* t, int64_t N,
                                     int32_t Cs, int32_t Cv, int32_t Ct, const int64_t* row,
                                     const int32_t* perm, const int32_t* node_start,
                                     const int32_t* node_end, int64_t E, const float* dir,
                                     const float* Y, int32_t ysh, const float* R, int32_t P,
                                     const int32_t* path_cols, const float* cg, float* Xs,
                                     int32_t Ks, float* Xv, int32_t Kv, float* Xt, int32_t Kt,
                                     void* stream) {
  int rc = check_edges("se3_aggregate_fwd", N, E, ysh, P, path_cols, cg);
  if (rc) return rc;
  GEO_REQUIRE(Cs >= 0 && Cv >= 0 && Ct >= 0, "se3_aggregate_fwd: negative channel count");
  GEO_REQUIRE(!Xs || Ks >= Cs + Cv + Ct, "se3_aggregate_fwd: Ks=%d < Cs+Cv+Ct", Ks);
  GEO_REQUIRE(!Xv || Kv >= Cs + 2 * Cv, "se3_aggregate_fwd: Kv=%d < Cs+2Cv", Kv);
  GEO_REQUIRE(!Xt || Kt >= Cs + Ct + Cv, "se3_aggregate_fwd: Kt=%d < Cs+Ct+Cv", Kt);
  GEO_REQUIRE((Cs == 0 || s) && (Cv == 0 || v) && (Ct == 0 || t), "se3_aggregate_fwd: null features");
  GEO_REQUIRE(path_cols[6] < 0 || Ct > 0, "se3_aggregate_fwd: path 6 without type-2 input");
  GEO_REQUIRE(path_cols[8] < 0 || Ct > 0, "se3_aggregate_fwd: path 8 without type-2 input");
  if (N == 0 || (!Xs && !Xv && !Xt)) return GEO_OK;
  GEO_REQUIRE(node_start && node_end && (E == 0 || (row && dir && Y && R)),
              "se3_aggregate_fwd: null graph array");
  SeEdges g = make_edges(row, perm, node_start, node_end, N, E, dir, Y, ysh, R, P, path_cols, cg);
  SeFeat f{s, v, t, Cs, Cv, Ct};
  const bool t2 = Ct > 0 || Xt != nullptr || path_cols[5] >= 0 || path_cols[6] >= 0 ||
                  path_cols[7] >= 0 || path_cols[8] >= 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kSeWaves)));
  if (t2)
    hipLaunchKernelGGL(se3_fwd_aggregate<true>, grid, dim3(kSeThreads), 0, as_stream(stream), g, f,
                       Xs, Ks, Xv, Kv, Xt, Kt);
  else
    hipLaunchKernelGGL(se3_fwd_aggregate<false>, grid, dim3(kSeThreads), 0, as_stream(stream), g, f,
                       Xs, Ks, Xv, Kv, Xt, Kt);
  GEO_LAUNCH_CHECK("se3_fwd_aggregate");
  return GEO_OK;
}

extern "C" int geo_se3_gemm(const float* A, int64_t M, int32_t K, const float* B, int32_t B_rows,
                            int32_t O, int32_t G, float* out, int64_t out_stride, const float* avg,
                            const float* bias, const uint8_t* mask, void* stream) {
  GEO_REQUIRE(M >= 0 && K > 0 && O >= 0 && G >= 1, "se3_gemm: bad sizes");
  GEO_REQUIRE(K % 16 == 0, "se3_gemm: K=%d must be a multiple of 16", K);
  if (M == 0 || O == 0) return GEO_OK;
  GEO_REQUIRE(M % G == 0, "se3_gemm: M=%lld is not a multiple of G=%d", (long long)M, G);
  GEO_REQUIRE(A && B && out, "se3_gemm: null pointer");
  GEO_REQUIRE((reinterpret_cast<uintptr_t>(A) & 15) == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0,
              "se3_gemm: A and B must be 16-byte aligned");
  GEO_REQUIRE(out_stride >= static_cast<int64_t>(O) * G, "se3_gemm: out_stride too small");
  const int nb = O > 32 ? 4 : (O > 16 ? 2 : 1);
  const int cols = 16 * nb;
  const int64_t gy = ceil_div(O, cols);
  GEO_REQUIRE(B_rows >= gy * cols, "se3_gemm: B has %d rows, the launch reads %lld", B_rows,
              (long long)(gy * cols));
  GEO_REQUIRE(G == 1 || G == 3 || G == 5, "se3_gemm: G=%d must be 1, 3 or 5", G);
  const dim3 grid(static_cast<unsigned>(ceil_div(M, 32 * kSeWaves)), static_cast<unsigned>(gy));
  hipStream_t st = as_stream(stream);
#define GEO_GEMM(NB_, G_)                                                                         \
  if (nb == NB_ && G == G_)                                                                       \
    hipLaunchKernelGGL((se3_gemm<NB_, G_>), grid, dim3(kSeThreads), 0, st, A, M, K, B, O, out,     \
                       out_stride, avg, bias, mask);
  GEO_GEMM(1, 1) GEO_GEMM(2, 1) GEO_GEMM(4, 1)
  GEO_GEMM(1, 3) GEO_GEMM(2, 3) GEO_GEMM(4, 3)
  GEO_GEMM(1, 5) GEO_GEMM(2, 5) GEO_GEMM(4, 5)
#undef GEO_GEMM
  GEO_LAUNCH_CHECK("se3_gemm");
  return GEO_OK;
}

extern "C" size_t geo_se3_fwd_fused_lds_bytes(int32_t Os, int32_t Ov, int32_t Ot, int32_t Ks,
                                              int32_t Kv, int32_t Kt) {
  if (Os < 0 || Ov < 0 || Ot < 0 || Ks < 0 || Kv < 0 || Kt < 0) return 0;
  return fused_layout(Os, Ov, Ot, Ks, Kv, Kt, nullptr);
}

extern "C" int geo_se3_fwd_fused(const float* s, const float* v, const float* t, int64_t N,
                                 int32_t Cs, int32_t Cv, int32_t Ct, const int64_t* row,
                                 const int32_t* perm, const int32_t* node_start,
                                 const int32_t* node_end, int64_t E, const float* dir,
                                 const float* Y, int32_t ysh, const float* R, int32_t P,
                                 const int32_t* path_cols, const float* cg, const float* Ws,
                                 int32_t Ws_rows, const float* Wv, int32_t Wv_rows, const float* Wt,
                                 int32_t Wt_rows, int32_t Os, int32_t Ov, int32_t Ot, int32_t Ks,
                                 int32_t Kv, int32_t Kt, const float* avg, const float* bias,
                                 const uint8_t* mask, float* s_out, float* v_out, float* t_out,
                                 float* Xs, float* Xv, float* Xt, void* stream) {
  int rc = check_edges("se3_fwd_fused", N, E, ysh, P, path_cols, cg);
  if (rc) return rc;
  GEO_REQUIRE(Cs >= 0 && Cv >= 0 && Ct >= 0 && Os >= 0 && Ov >= 0 && Ot >= 0,
              "se3_fwd_fused: negative channel count");
  GEO_REQUIRE((Cs == 0 || s) && (Cv == 0 || v) && (Ct == 0 || t), "se3_fwd_fused: null features");
  GEO_REQUIRE(path_cols[6] < 0 || Ct > 0, "se3_fwd_fused: path 6 without type-2 input");
  GEO_REQUIRE(path_cols[8] < 0 || Ct > 0, "se3_fwd_fused: path 8 without type-2 input");
  const int used[3] = {Cs + Cv + Ct, Cs + 2 * Cv, Cs + Ct + Cv};
  const int32_t O[3] = {Os, Ov, Ot}, K[3] = {Ks, Kv, Kt}, rows[3] = {Ws_rows, Wv_rows, Wt_rows};
  const float* W[3] = {Ws, Wv, Wt};
  float* out[3] = {s_out, v_out, t_out};
  const char* kind[3] = {"scalar", "vector", "type-2"};
  for (int k = 0; k < 3; ++k) {
    if (O[k] == 0) continue;
    GEO_REQUIRE(K[k] >= used[k] && K[k] % 16 == 0,
                "se3_fwd_fused: %s row length %d must be a multiple of 16 and >= %d", kind[k], K[k],
                used[k]);
    GEO_REQUIRE(W[k] && out[k], "se3_fwd_fused: null %s weights or output", kind[k]);
    GEO_REQUIRE((reinterpret_cast<uintptr_t>(W[k]) & 15) == 0,
                "se3_fwd_fused: %s weights must be 16-byte aligned", kind[k]);
    GEO_REQUIRE(rows[k] >= (O[k] + 15) / 16 * 16, "se3_fwd_fused: %s weights have %d rows, need %d",
                kind[k], rows[k], (O[k] + 15) / 16 * 16);
  }
  SeFused p{};
  const size_t lds = fused_layout(Os, Ov, Ot, Ks, Kv, Kt, &p);
  GEO_REQUIRE(lds > 0 || (Os == 0 && Ov == 0 && Ot == 0),
              "se3_fwd_fused: aggregate tile exceeds %d bytes of LDS (use the unfused path)",
              kFuLdsMax);
  if (N == 0 || lds == 0) return GEO_OK;
  GEO_REQUIRE(node_start && node_end && (E == 0 || (row && dir && Y && R)),
              "se3_fwd_fused: null graph array");
  for (int k = 0; k < 3; ++k) {
    p.W[k] = W[k];
    p.out[k] = out[k];
  }
  p.X[0] = Xs;
  p.X[1] = Xv;
  p.X[2] = Xt;
  for (int k = 0; k < 3; ++k)
    GEO_REQUIRE((reinterpret_cast<uintptr_t>(p.X[k]) & 15) == 0,
                "se3_fwd_fused: kept %s aggregates must be 16-byte aligned", kind[k]);
  p.avg = avg;
  p.bias = bias;
  p.mask = mask;
  SeEdges g = make_edges(row, perm, node_start, node_end, N, E, dir, Y, ysh, R, P, path_cols, cg);
  SeFeat f{s, v, t, Cs, Cv, Ct};
  const bool t2 = Ct > 0 || Ot > 0 || path_cols[5] >= 0 || path_cols[6] >= 0 ||
                  path_cols[7] >= 0 || path_cols[8] >= 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kFuTile)));
  hipStream_t st = as_stream(stream);
  if (fused_rows_ok(N, Cs, Cv, t2, E, P, ysh))
    hipLaunchKernelGGL((se3_fwd_fused_rows<4>), grid, dim3(kSeThreads), lds, st, g, f, p);
  else if (t2)
    hipLaunchKernelGGL((se3_fwd_fused<true, 4>), grid, dim3(kSeThreads), lds, st, g, f, p);
  else
    hipLaunchKernelGGL((se3_fwd_fused<false, 8>), grid, dim3(kSeThreads), lds, st, g, f, p);
  GEO_LAUNCH_CHECK("se3_fwd_fused");
  return GEO_OK;
}

extern "C" int geo_se3_grad_prep(const float* grad, int64_t N, int32_t O, int32_t G, int32_t Opad,
                                 const float* avg, const uint8_t* mask, float* out, void* stream) {
  GEO_REQUIRE(N >= 0 && O >= 0 && G >= 1 && Opad >= O, "se3_grad_prep: bad sizes");
  const int64_t total = N * G * Opad;
  if (total == 0) return GEO_OK;
  GEO_REQUIRE(out && (O == 0 || grad), "se3_grad_prep: null pointer");
  hipLaunchKernelGGL(se3_grad_prep, dim3(static_cast<unsigned>(ceil_div(total, kSeThreads))),
                     dim3(kSeThreads), 0, as_stream(stream), grad, N, O, G, Opad, avg, mask, out);
  GEO_LAUNCH_CHECK("se3_grad_prep");
  return GEO_OK;
}

extern "C" int geo_se3_bwd_edge(const float* s, const float* v, const float* t, int64_t N,
                                int32_t Cs, int32_t Cv, int32_t Ct, const int64_t* row,
                                const int32_t* perm, const int32_t* node_start,
                                const int32_t* node_end, int64_t E, const float* dir, const float* Y,
                                int32_t ysh, const float* R, int32_t P, const int32_t* path_cols,
                                const float* cg, const float* gXs, int32_t Ks, const float* gXv,
                                int32_t Kv, const float* gXt, int32_t Kt, float* dR, float* ddir,
                                float* dY, void* stream) {
  int rc = check_edges("se3_bwd_edge", N, E, ysh, P, path_cols, cg);
  if (rc) return rc;
  GEO_REQUIRE(!gXs || Ks >= Cs + Cv + Ct, "se3_bwd_edge: Ks too small");
  GEO_REQUIRE(!gXv || Kv >= Cs + 2 * Cv, "se3_bwd_edge: Kv too small");
  GEO_REQUIRE(!gXt || Kt >= Cs + Ct + Cv, "se3_bwd_edge: Kt too small");
  GEO_REQUIRE((Cs == 0 || s) && (Cv == 0 || v) && (Ct == 0 || t), "se3_bwd_edge: null features");
  if (N == 0 || E == 0 || (!dR && !ddir && !dY)) return GEO_OK;
  GEO_REQUIRE(row && node_start && node_end && dir && Y && R, "se3_bwd_edge: null graph array");
  SeEdges g = make_edges(row, perm, node_start, node_end, N, E, dir, Y, ysh, R, P, path_cols, cg);
  SeFeat f{s, v, t, Cs, Cv, Ct};
  const bool one = Cs <= 64 && Cv <= 16 && Ct <= 16;
  const bool t2 = Ct > 0 || gXt != nullptr || path_cols[5] >= 0 || path_cols[6] >= 0 ||
                  path_cols[7] >= 0 || path_cols[8] >= 0;
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kSeWaves)));
  hipStream_t st = as_stream(stream);
#define GEO_BWD_EDGE(ONE_, T2_)                                                                    \
  hipLaunchKernelGGL((se3_bwd_edge<ONE_, T2_>), grid, dim3(kSeThreads), 0, st, g, f, gXs, Ks, gXv, Kv, \
                     gXt, Kt, dR, ddir, dY)
  if (bwd_edge_rows_ok(N, Cs, Cv, t2)) {
    hipLaunchKernelGGL((se3_bwd_edge_rows<1>), grid, dim3(kSeThreads), 0, st, g, f, gXs, Ks, gXv, Kv,
                       dR, ddir, dY);
    GEO_LAUNCH_CHECK("se3_bwd_edge_rows");
    return GEO_OK;
  }
  if (one && t2) GEO_BWD_EDGE(true, true);
  else if (one) GEO_BWD_EDGE(true, false);
  else if (t2) GEO_BWD_EDGE(false, true);
  else GEO_BWD_EDGE(false, false);
#undef GEO_BWD_EDGE
  GEO_LAUNCH_CHECK("se3_bwd_edge");
  return GEO_OK;
}

extern "C" int geo_se3_bwd_edge_fused(const float* s, const float* v, int64_t N, int32_t Cs,
                                      int32_t Cv, const int64_t* row, const int32_t* perm,
                                      const int32_t* node_start, const int32_t* node_end, int64_t E,
                                      const float* dir, const float* Y, int32_t ysh, const float* R,
                                      int32_t P, const int32_t* path_cols, const float* cg,
                                      const float* Gs, int32_t OsP, const float* Gv, int32_t OvP,
                                      const float* WsT, int32_t WsT_rows, const float* WvT,
                                      int32_t WvT_rows, int32_t Ks, int32_t Kv, float* dR,
                                      float* ddir, float* dY, void* stream) {
  int rc = check_edges("se3_bwd_edge_fused", N, E, ysh, P, path_cols, cg);
  if (rc) return rc;
  GEO_REQUIRE(Cs >= 0 && Cv >= 0, "se3_bwd_edge_fused: negative channel count");
  GEO_REQUIRE(Ks >= Cs + Cv && Ks % 16 == 0 && Kv >= Cs + 2 * Cv && Kv % 16 == 0,
              "se3_bwd_edge_fused: Ks / Kv too small or not multiples of 16");
  GEO_REQUIRE((!Gs || (OsP > 0 && OsP % 16 == 0)) && (!Gv || (OvP > 0 && OvP % 16 == 0)),
              "se3_bwd_edge_fused: OsP / OvP must be positive multiples of 16");
  GEO_REQUIRE(!Gs || (WsT && WsT_rows >= Ks), "se3_bwd_edge_fused: WsT too short");
  GEO_REQUIRE(!Gv || (WvT && WvT_rows >= Kv), "se3_bwd_edge_fused: WvT too short");
  GEO_REQUIRE((!Gs || (reinterpret_cast<uintptr_t>(WsT) & 15) == 0) &&
              (!Gv || (reinterpret_cast<uintptr_t>(WvT) & 15) == 0),
              "se3_bwd_edge_fused: packed weights must be 16-byte aligned");
  GEO_REQUIRE((Cs == 0 || s) && (Cv == 0 || v), "se3_bwd_edge_fused: null features");
  const bool t2 = path_cols[5] >= 0 || path_cols[6] >= 0 || path_cols[7] >= 0 || path_cols[8] >= 0;
  const size_t lds = edge_tile_floats(Ks, Kv) * sizeof(float);
  const int64_t lim = int64_t{1} << 31;  // the gradient rows are read through buffer resources
  if (!bwd_edge_rows_ok(N, Cs, Cv, t2) || lds > static_cast<size_t>(kFuLdsMax) ||
      N * OsP * 4 >= lim || N * 3 * OvP * 4 >= lim)
    return set_error(GEO_ERR_UNSUPPORTED, "se3_bwd_edge_fused: layer not covered by the tile kernel "
                                          "(type-2 paths, Cs > 64 or not a multiple of 4, Cv > 16, "
                                          "arrays of 2 GiB, tiles beyond 64 KB of LDS)");
  if (N == 0 || E == 0 || (!dR && !ddir && !dY)) return GEO_OK;
  GEO_REQUIRE(row && node_start && node_end && dir && Y && R, "se3_bwd_edge_fused: null graph array");
  SeEdges g = make_edges(row, perm, node_start, node_end, N, E, dir, Y, ysh, R, P, path_cols, cg);
  SeFeat f{s, v, nullptr, Cs, Cv, 0};
  SeEdgeTile q{Gs, Gv, WsT, WvT, Gs ? OsP : 0, Gv ? OvP : 0, Ks, Kv};
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kFuTile)));
  hipLaunchKernelGGL((se3_bwd_edge_tile<1>), grid, dim3(kSeThreads), lds, as_stream(stream), g, f, q,
                     dR, ddir, dY);
  GEO_LAUNCH_CHECK("se3_bwd_edge_tile");
  return GEO_OK;
}

extern "C" int geo_se3_bwd_src(const float* gs, int32_t Os, int32_t OsP, const float* gv, int32_t Ov,
                               int32_t OvP, const float* gt, int32_t Ot, int32_t OtP, int64_t N,
                               const int64_t* col, const int32_t* perm, const int32_t* node_start,
                               const int32_t* node_end, int64_t E, const float* dir, const float* Y,
                               int32_t ysh, const float* R, int32_t P, const int32_t* path_cols,
                               const float* cg, float* Zs, int32_t KZs, float* Zv, int32_t KZv,
                               float* Zt, int32_t KZt, float* Z8, int32_t KZ8, void* stream) {
  int rc = check_edges("se3_bwd_src", N, E, ysh, P, path_cols, cg);
  if (rc) return rc;
  GEO_REQUIRE(Os >= 0 && Ov >= 0 && Ot >= 0, "se3_bwd_src: negative channel count");
  GEO_REQUIRE((!gs || OsP >= Os) && (!gv || OvP >= Ov) && (!gt || OtP >= Ot),
              "se3_bwd_src: padded widths too small");
  GEO_REQUIRE(!Zs || KZs >= Os + Ov + Ot, "se3_bwd_src: KZs too small");
  GEO_REQUIRE(!Zv || KZv >= 2 * Ov + Os + Ot, "se3_bwd_src: KZv too small");
  GEO_REQUIRE(!Zt || KZt >= Ot, "se3_bwd_src: KZt too small");
  GEO_REQUIRE(!Z8 || KZ8 >= Os, "se3_bwd_src: KZ8 too small");
  if (N == 0 || (!Zs && !Zv && !Zt && !Z8)) return GEO_OK;
  GEO_REQUIRE(node_start && node_end && (E == 0 || (col && dir && Y && R)),
              "se3_bwd_src: null graph array");
  SeEdges g = make_edges(col, perm, node_start, node_end, N, E, dir, Y, ysh, R, P, path_cols, cg);
  const bool t2 = (gt != nullptr && Ot > 0) || Zt != nullptr || Z8 != nullptr || path_cols[5] >= 0 ||
                  path_cols[6] >= 0 || path_cols[7] >= 0 || path_cols[8] >= 0;
  if (bwd_src_rows_ok(N, Os, OsP, Ov, OvP, t2, E, P, ysh)) {
    const dim3 grid4(static_cast<unsigned>(ceil_div(N, kSeWaves * kRowNodes)));
    hipLaunchKernelGGL((se3_bwd_src_rows<4, false>), grid4, dim3(kSeThreads), 0, as_stream(stream),
                       g, gs, Os, OsP, gv, Ov, OvP, Zs, KZs, Zv, KZv, SeFused{});
    GEO_LAUNCH_CHECK("se3_bwd_src_rows");
    return GEO_OK;
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kSeWaves)));
  if (gt != nullptr && Ot > 0)
    hipLaunchKernelGGL(se3_bwd_src<true>, grid, dim3(kSeThreads), 0, as_stream(stream), g, gs, Os,
                       OsP, gv, Ov, OvP, gt, Ot, OtP, Zs, KZs, Zv, KZv, Zt, KZt, Z8, KZ8);
  else
    hipLaunchKernelGGL(se3_bwd_src<false>, grid, dim3(kSeThreads), 0, as_stream(stream), g, gs, Os,
                       OsP, gv, Ov, OvP, gt, Ot, OtP, Zs, KZs, Zv, KZv, Zt, KZt, Z8, KZ8);
  GEO_LAUNCH_CHECK("se3_bwd_src");
  return GEO_OK;
}

extern "C" int geo_se3_bwd_src_fused(const float* gs, int32_t Os, int32_t OsP, const float* gv,
                                     int32_t Ov, int32_t OvP, int64_t N, const int64_t* col,
                                     const int32_t* perm, const int32_t* node_start,
                                     const int32_t* node_end, int64_t E, const float* dir,
                                     const float* Y, int32_t ysh, const float* R, int32_t P,
                                     const int32_t* path_cols, const float* cg, int32_t KZs,
                                     int32_t KZv, const float* Bs, int32_t Bs_rows, int32_t Cs,
                                     float* ds, const float* Bv, int32_t Bv_rows, int32_t Cv,
                                     float* dv, void* stream) {
  int rc = check_edges("se3_bwd_src_fused", N, E, ysh, P, path_cols, cg);
  if (rc) return rc;
  GEO_REQUIRE(Os >= 0 && Ov >= 0 && Cs >= 0 && Cv >= 0, "se3_bwd_src_fused: negative channel count");
  GEO_REQUIRE((!gs || OsP >= Os) && (!gv || OvP >= Ov), "se3_bwd_src_fused: padded widths too small");
  GEO_REQUIRE(KZs >= Os + Ov && KZs % 16 == 0 && KZv >= 2 * Ov + Os && KZv % 16 == 0,
              "se3_bwd_src_fused: KZs / KZv too small or not multiples of 16");
  const bool want_s = ds != nullptr && Cs > 0, want_v = dv != nullptr && Cv > 0;
  GEO_REQUIRE(!want_s || (Bs && Bs_rows >= 16 * ((Cs + 15) / 16)), "se3_bwd_src_fused: Bs too short");
  GEO_REQUIRE(!want_v || (Bv && Bv_rows >= 16 * ((Cv + 15) / 16)), "se3_bwd_src_fused: Bv too short");
  GEO_REQUIRE((!want_s || (reinterpret_cast<uintptr_t>(Bs) & 15) == 0) &&
              (!want_v || (reinterpret_cast<uintptr_t>(Bv) & 15) == 0),
              "se3_bwd_src_fused: packed weights must be 16-byte aligned");
  const bool t2 = path_cols[5] >= 0 || path_cols[6] >= 0 || path_cols[7] >= 0 || path_cols[8] >= 0;
  if (!bwd_src_rows_ok(N, Os, OsP, Ov, OvP, t2, E, P, ysh))
    return set_error(GEO_ERR_UNSUPPORTED, "se3_bwd_src_fused: layer not covered by the row kernel "
                                          "(type-2 paths, Os > 64, Ov > 16 or arrays of 2 GiB)");
  SeFused q{};
  q.W[0] = Bs;
  q.W[1] = Bv;
  q.out[0] = ds;
  q.out[1] = dv;
  q.O[0] = want_s ? Cs : 0;
  q.O[1] = want_v ? Cv : 0;
  q.K[0] = KZs;
  q.K[1] = KZv;
  q.ld[0] = KZs + 4;
  q.ld[1] = KZv + 4;
  q.off[0] = 0;
  q.off[1] = kFuTile * q.ld[0];
  const size_t lds = static_cast<size_t>(q.off[1] + 3 * kFuTile * q.ld[1]) * sizeof(float);
  if (lds > static_cast<size_t>(kFuLdsMax))
    return set_error(GEO_ERR_UNSUPPORTED, "se3_bwd_src_fused: tile of %zu bytes exceeds LDS", lds);
  if (N == 0 || (!want_s && !want_v)) return GEO_OK;
  GEO_REQUIRE(node_start && node_end && (E == 0 || (col && dir && Y && R)),
              "se3_bwd_src_fused: null graph array");
  SeEdges g = make_edges(col, perm, node_start, node_end, N, E, dir, Y, ysh, R, P, path_cols, cg);
  const dim3 grid(static_cast<unsigned>(ceil_div(N, kFuTile)));  // tile <= 64 KB: default LDS limit
  hipLaunchKernelGGL((se3_bwd_src_rows<4, true>), grid, dim3(kSeThreads), lds, as_stream(stream), g,
                     gs, Os, OsP, gv, Ov, OvP, nullptr, KZs, nullptr, KZv, q);
  GEO_LAUNCH_CHECK("se3_bwd_src_rows");
  return GEO_OK;
}

extern "C" size_t geo_se3_gemm_tn_workspace_bytes(int64_t M, int32_t O, int32_t K) {
  if (M < 0 || O < 0 || K < 0) return 0;
  const TnPlan t = tn_plan(M, O, K);
  const int64_t Opad = ((O + 15) / 16) * 16, Kpad = ((K + 15) / 16) * 16;
  return static_cast<size_t>(t.nparts_x) * Opad * Kpad * sizeof(float);
}

namespace geo {
namespace {

int gemm_tn_into(const float* A, int64_t M, int32_t lda, int32_t O, const float* B, int32_t ldb,
                 int32_t K, const TnOut& dst, void* workspace, size_t workspace_bytes,
                 void* stream) {
  GEO_REQUIRE(M >= 0 && O >= 0 && K >= 0 && lda >= O && ldb >= K,
              "se3_gemm_tn: bad sizes (M=%lld O=%d K=%d lda=%d ldb=%d)", (long long)M, O, K, lda,
              ldb);
  if (O == 0 || K == 0) return GEO_OK;
  GEO_REQUIRE(M == 0 || (A && B), "se3_gemm_tn: null pointer");
  const size_t need = geo_se3_gemm_tn_workspace_bytes(M, O, K);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(GEO_ERR_WORKSPACE, "se3_gemm_tn: workspace %zu bytes, need %zu",
                     workspace_bytes, need);
  const TnPlan t = tn_plan(M, O, K);
  const int Opad = ((O + 15) / 16) * 16, Kpad = ((K + 15) / 16) * 16;
  float* part = static_cast<float*>(workspace);
  hipStream_t st = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(t.nparts_x), static_cast<unsigned>(t.groups));
#define GEO_TN(OB_, KB_)                                                                         \
  if (t.ob == OB_ && t.kb == KB_)                                                                \
    hipLaunchKernelGGL((se3_gemm_tn<OB_, KB_>), grid, dim3(kSeThreads), 0, st, A, M, lda, O, B, ldb, \
                       K, t.rows_per_wave, t.kb_groups, part, Opad, Kpad);
  GEO_TN(1, 2) GEO_TN(1, 4) GEO_TN(1, 6) GEO_TN(1, 8)
  GEO_TN(2, 2) GEO_TN(2, 4) GEO_TN(2, 6) GEO_TN(2, 8)
  GEO_TN(4, 2) GEO_TN(4, 4) GEO_TN(4, 6) GEO_TN(4, 8)
#undef GEO_TN
  GEO_LAUNCH_CHECK("se3_gemm_tn");
  const int nparts = t.nparts_x;
  hipLaunchKernelGGL(se3_gemm_tn_final,
                     dim3(static_cast<unsigned>(ceil_div(static_cast<int64_t>(Opad) * Kpad, 64))),
                     dim3(kSeThreads), 0, st, part, nparts, Opad, Kpad, O, K, dst);
  GEO_LAUNCH_CHECK("se3_gemm_tn_final");
  return GEO_OK;
}

}  // namespace
}  // namespace geo

extern "C" int geo_se3_gemm_tn(const float* A, int64_t M, int32_t lda, int32_t O, const float* B,
                               int32_t ldb, int32_t K, float* out, int32_t ldo, void* workspace,
                               size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(ldo >= K, "se3_gemm_tn: ldo %d < K %d", ldo, K);
  GEO_REQUIRE(out || O == 0 || K == 0, "se3_gemm_tn: null pointer");
  TnOut dst{};
  dst.n = 1;
  dst.c[0] = 0;
  dst.c[1] = K;
  dst.p[0] = out;
  dst.ld[0] = ldo;
  return gemm_tn_into(A, M, lda, O, B, ldb, K, dst, workspace, workspace_bytes, stream);
}

extern "C" int geo_se3_gemm_tn_split(const float* A, int64_t M, int32_t lda, int32_t O,
                                     const float* B, int32_t ldb, int32_t K, int32_t nsplit,
                                     const int32_t* cols, float* const* outs, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(nsplit >= 1 && nsplit <= 3 && cols && outs, "se3_gemm_tn_split: 1 to 3 parts");
  GEO_REQUIRE(cols[0] == 0 && cols[nsplit] == K, "se3_gemm_tn_split: parts must cover 0..K");
  TnOut dst{};
  dst.n = nsplit;
  for (int j = 0; j <= nsplit; ++j) dst.c[j] = cols[j];
  for (int j = 0; j < nsplit; ++j) {
    GEO_REQUIRE(cols[j + 1] >= cols[j], "se3_gemm_tn_split: part bounds must ascend");
    dst.p[j] = outs[j];
    dst.ld[j] = cols[j + 1] - cols[j];
  }
  return gemm_tn_into(A, M, lda, O, B, ldb, K, dst, workspace, workspace_bytes, stream);
}

extern "C" size_t geo_se3_colsum_workspace_bytes(int64_t N, int32_t O) {
  if (N < 0 || O < 0) return 0;
  return static_cast<size_t>(kColsumBlocks) * static_cast<size_t>(O) * sizeof(float);
}

extern "C" int geo_se3_colsum(const float* g, int64_t N, int32_t O, const uint8_t* mask, float* out,
                              void* workspace, size_t workspace_bytes, void* stream) {
  GEO_REQUIRE(N >= 0 && O >= 0, "se3_colsum: bad sizes (N=%lld O=%d)", (long long)N, O);
  if (O == 0) return GEO_OK;
  GEO_REQUIRE(out && (N == 0 || g), "se3_colsum: null pointer");
  hipStream_t st = as_stream(stream);
  float* part = static_cast<float*>(workspace);
  int nb = 0;  // N == 0: the final kernel adds no partials and writes zeros
  if (N > 0) {
    const size_t need = geo_se3_colsum_workspace_bytes(N, O);
    if (workspace == nullptr || workspace_bytes < need)
      return set_error(GEO_ERR_WORKSPACE, "se3_colsum: workspace %zu bytes, need %zu",
                       workspace_bytes, need);
    const int64_t R = ceil_div(N, static_cast<int64_t>(kColsumBlocks));
    if (O % 4 == 0 && (reinterpret_cast<uintptr_t>(g) & 15) == 0)
      hipLaunchKernelGGL(se3_colsum_part<true>, dim3(kColsumBlocks), dim3(kSeThreads), 0, st, g,
                         N, O, mask, R, part);
    else
      hipLaunchKernelGGL(se3_colsum_part<false>, dim3(kColsumBlocks), dim3(kSeThreads), 0, st, g,
                         N, O, mask, R, part);
    GEO_LAUNCH_CHECK("se3_colsum_part");
    nb = kColsumBlocks;
  }
  hipLaunchKernelGGL(se3_colsum_final, dim3(static_cast<unsigned>(ceil_div(static_cast<int64_t>(O), 64))),
                     dim3(kColsumFinalThreads), 0, st, part, nb, O, out);
  GEO_LAUNCH_CHECK("se3_colsum_final");
  return GEO_OK;
}

extern "C" int geo_se3_pack_weights(const float* const* W, int32_t Cs, int32_t Cv, int32_t Ct,
                                    int32_t Os, int32_t Ov, int32_t Ot, int32_t nout,
                                    float* const* out, const int32_t* rows, const int32_t* cols,
                                    const int32_t* kinds, void* stream) {
  GEO_REQUIRE(W && out && rows && cols && kinds, "se3_pack_weights: null table");
  GEO_REQUIRE(nout >= 1 && nout <= 10, "se3_pack_weights: nout=%d outside [1, 10]", nout);
  GEO_REQUIRE(Cs >= 0 && Cv >= 0 && Ct >= 0 && Os >= 0 && Ov >= 0 && Ot >= 0,
              "se3_pack_weights: negative channel count");
  SePack k;
  for (int i = 0; i < kSePaths; ++i) k.W[i] = W[i];
  k.Cs = Cs; k.Cv = Cv; k.Ct = Ct; k.Os = Os; k.Ov = Ov; k.Ot = Ot;
  k.nout = nout;
  k.start[0] = 0;
  for (int j = 0; j < nout; ++j) {
    GEO_REQUIRE(kinds[j] >= 0 && kinds[j] <= 9 && rows[j] >= 0 && cols[j] >= 0 && out[j],
                "se3_pack_weights: bad output %d", j);
    k.out[j] = SePackOut{out[j], rows[j], cols[j], kinds[j]};
    k.start[j + 1] = k.start[j] + static_cast<int64_t>(rows[j]) * cols[j];
  }
  if (k.start[nout] == 0) return GEO_OK;
  hipLaunchKernelGGL(se3_pack_kernel, dim3(static_cast<unsigned>(ceil_div(k.start[nout], kSeThreads))),
                     dim3(kSeThreads), 0, as_stream(stream), k);
  GEO_LAUNCH_CHECK("se3_pack_kernel");
  return GEO_OK;
}
