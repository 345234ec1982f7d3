// radial.hip — the radial basis MLP of SE3Conv, forward and backward, on the matrix cores.
//
// Reference: RadialBasis.forward (geoembodied/nn/modules/se3_conv.py:238-282), per edge e with
// length d:
//   x_i = sin(f_i d) / max(d, 1e-8) * env(d),  env(d) = max(0.5 (1 + cos((pi d) / cutoff)), 0)
//   z_j = b1_j + sum_i W1[j][i] x_i,  h_j = silu(z_j) = z_j / (1 + exp(-z_j))
//   R_p = b2_p + sum_j W2[p][j] h_j
// with i < NB basis functions, j < H hidden units and p < P outputs (the matrix-core kernels below
// take NB <= 16, H <= 64, P <= 16; larger layers take the general kernels further down).  PyTorch
// runs this as a dozen kernels with [E, 64] intermediates, and its weight gradients as GEMMs
// whose reduction dimension is E.  Here one wave takes 16 edges at a time through fp32 MFMA
// (v_mfma_f32_16x16x4_f32) tiles, nothing per edge but d, R and dR touches memory, and the weight
// gradients accumulate in MFMA accumulators across all of a wave's edges.
//
// MFMA operand convention (as in se3_message.hip): in MFMA number q (q < 4) of a 16-wide k chunk,
// lane l supplies A[row = l % 16][k = 4 (l / 16) + q] and B[k = 4 (l / 16) + q][col = l % 16];
// the result D[row = 4 (l / 16) + q][col = l % 16] sits in element q of lane l.  So the result of
// one GEMM is directly the B operand of the next along the same k chunk.
//
// Forward:  Z^T = W1 X^T (A = W1, B = X^T), H^T = silu(Z^T + b1), R^T = W2 H^T (B = H^T as is).
// Backward (per 16 edges):  Z = X W1^T and dH = dR W2 in the edge-major layout, dZ = dH silu'(Z);
//   dW2 += dR^T H,  dW1^T += X^T dZ,  db1 += colsum dZ,  db2 += colsum dR  (accumulators);
//   dX^T = W1^T dZ^T (dZ transposed through LDS), d(dist) = sum_i dX_i dx_i/dd.
// Per-block partial sums of the weight gradients are combined by one more kernel in block order,
// so results are deterministic.
#include "scan.hpp"

namespace geo {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kRbThreads = 256;
constexpr int kRbWaves = kRbThreads / kWave;
constexpr int kRbMaxBasis = 16;
constexpr int kRbMaxHidden = 64;
constexpr int kRbMaxOut = 16;
constexpr int kRbPart = 16 * 64 + 16 * 64 + 64 + 16;  // dW1^T | dW2 | db1 | db2 per block
constexpr int kRbMaxBlocks = 1024;

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct RbParams {
  const float* dist;
  int64_t E;
  const float* freqs;
  int NB;
  float cutoff;
  const float* W1;  // [H][NB]
  const float* b1;  // [H]
  int H;
  const float* W2;  // [P][H]
  const float* b2;  // [P]
  int P;
};

// Sine and cosine from the hardware (v_sin_f32 / v_cos_f32 take the argument in revolutions).
// Measured on gfx950 against float64 over [0, 50) rad: absolute error <= 3.5e-6, which is the
// rounding of the fp32 argument scaled to revolutions and no larger than the rounding of the
// product f * d itself at those magnitudes; relative error <= 1e-6 below 0.5 rad, so sin(x) / d
// keeps its accuracy as d -> 0.  Arguments beyond +-1000 rad (outside the unit's range) take the
// library functions.
constexpr float kInv2Pi = 0.15915494309189535f;
__device__ __forceinline__ float rb_sin(float x) {
  return fabsf(x) < 1000.f ? __builtin_amdgcn_sinf(x * kInv2Pi) : sinf(x);
}
__device__ __forceinline__ float rb_cos(float x) {
  return fabsf(x) < 1000.f ? __builtin_amdgcn_cosf(x * kInv2Pi) : cosf(x);
}

// Envelope and its derivative with respect to d (the clamp at 0 never bites: 0.5 (1 + cos) >= 0).
// pic = pi / cutoff.
__device__ __forceinline__ void envelope(float d, float pic, float& env, float& denv) {
#pragma clang fp contract(off)
  const float t = pic * d;
  const float c = rb_cos(t);
  const float e = 0.5f * (1.0f + c);
  env = e < 0.f ? 0.f : e;
  denv = -0.5f * rb_sin(t) * pic;
}

// x_i(d) and, when asked, dx_i/dd; rdc = 1 / max(d, 1e-8).
__device__ __forceinline__ float basis(float f, float d, float rdc, float env, float denv,
                                       float* dx) {
#pragma clang fp contract(off)
  const float s = rb_sin(f * d);
  const float b = s * rdc;
  if (dx) {
    // d/dd [sin(f d) / dc] = f cos(f d) / dc - [d >= 1e-8] sin(f d) / dc^2
    const float db = f * rb_cos(f * d) * rdc - (d >= 1e-8f ? b * rdc : 0.f);
    *dx = db * env + b * denv;
  }
  return b * env;
}
__device__ __forceinline__ float rb_rdc(float d) { return 1.0f / (d < 1e-8f ? 1e-8f : d); }

// Logistic sigmoid 1 / (1 + e^-z) from the hardware exp2 and reciprocal (each within 1 ulp):
// saturates to 0 / 1 for large |z| like the exact function.
__device__ __forceinline__ float sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}
__device__ __forceinline__ float silu(float z) { return z * sigmoid(z); }

// A buffer resource over the `count` floats at p (none when count <= 0): loads past the end read
// 0 and stores past the end are dropped, so a tile's edge and output bounds need no branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rb_rsrc(const float* p, int64_t count) {
  const int bytes = count <= 0 ? 0 : static_cast<int>(4 * count);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, bytes, 0x00020000);
}

// Distance of edge e0 + li (e0 wave-uniform); 0 for edges at or past E (their basis values are
// 0 and their outputs are not stored).  The loaded value is returned as it is, so the wait for it
// falls where the next tile first uses it, not in the tile that issued the load.
__device__ __forceinline__ float rb_dist(const RbParams& p, int64_t e0, int li) {
  const int64_t left = p.E - e0;
  const auto rs = rb_rsrc(left > 0 ? p.dist + e0 : p.dist, left > 16 ? 16 : left);
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, 4u * li, 0, 0));
}

// Tiles whose sine and cosine arguments (f d and pi d / cutoff) are all below kRbFastArg in
// magnitude -- every edge of a radius graph -- evaluate the basis without per-call range checks.
constexpr float kRbFastArg = 1000.f;

// x[q] = x_{4g+q}(d), the lane's four basis values.  When every lane of the wave passes the
// argument test (a wave-uniform branch), the hardware sine and cosine are called directly and
// 1 / max(d, 1e-8) comes from the hardware reciprocal (within 1 ulp); a column past NB has
// f = 0 and so the value 0.  Other tiles take the range-checked functions.
__device__ __forceinline__ void rb_basis_fwd(const float* fr, int NB, int g, float pic, float d,
                                             float* x) {
  const float t = pic * d;
  float a[4];
  bool fast = fabsf(t) < kRbFastArg;  // false for NaN
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = fr[q] * d;
    fast &= fabsf(a[q]) < kRbFastArg;
  }
  if (__ballot(!fast) == 0ull) {
    const float e = 0.5f * (1.0f + __builtin_amdgcn_cosf(t * kInv2Pi));
    const float env = e < 0.f ? 0.f : e;
    const float rdc = __builtin_amdgcn_rcpf(d < 1e-8f ? 1e-8f : d);
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = (__builtin_amdgcn_sinf(a[q] * kInv2Pi) * rdc) * env;
  } else {
    float env, denv;
    envelope(d, pic, env, denv);
    const float rdc = rb_rdc(d);
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = 4 * g + q < NB ? basis(fr[q], d, rdc, env, denv, nullptr) : 0.f;
  }
}

// Weights of the forward in MFMA operand layout (see the header), per lane.
struct RbFwdWeights {
  float w1[4][4], b1r[4][4], w2[4][4], fr[4], b2r[4];
};

// One 16-edge tile of the forward: R[e0 + li][4g + q] from the lane's distance d.  (Measured
// with the counters: the matrix core and the vector ALU do not run at the same time in this
// kernel -- no co-executed cycles -- so its time is close to the sum of the two; this is why the
// tile keeps the VALU work per edge small rather than interleaving it with the MFMAs.)
__device__ __forceinline__ void rb_fwd_tile(const RbParams& p, const RbFwdWeights& w, float pic,
                                            int g, int li, int64_t e0, float d,
                                            float* __restrict__ R) {
  float x[4];
  rb_basis_fwd(w.fr, p.NB, g, pic, d, x);
  // the biases start the accumulators: Z^T = b1 + W1 X^T, R^T = b2 + W2 H^T
  floatx4 h[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    floatx4 z = {w.b1r[jb][0], w.b1r[jb][1], w.b1r[jb][2], w.b1r[jb][3]};
#pragma unroll
    for (int q = 0; q < 4; ++q) z = mfma4(w.w1[jb][q], x[q], z);
#pragma unroll
    for (int q = 0; q < 4; ++q) h[jb][q] = silu(z[q]);
  }
  floatx4 r = {w.b2r[0], w.b2r[1], w.b2r[2], w.b2r[3]};
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) r = mfma4(w.w2[c][q], h[c][q], r);
  // lanes past E and outputs >= P store nothing (out of the resource)
  const int64_t left = p.E - e0;
  const auto rs = rb_rsrc(R + e0 * p.P, (left > 16 ? 16 : left) * p.P);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int pp = 4 * g + q;
    const uint32_t off = pp < p.P ? 4u * static_cast<uint32_t>(li * p.P + pp) : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(r[q]), rs, off, 0, 0);
  }
}

__global__ __launch_bounds__(kRbThreads) void radial_fwd_kernel(RbParams p, float* __restrict__ R) {
  const float pic = 3.14159265358979323846f / p.cutoff;
  const int lane = lane_id();
  const int g = lane >> 4, li = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  RbFwdWeights w;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * g + q;
    w.fr[q] = i < p.NB ? p.freqs[i] : 0.f;
    w.b2r[q] = i < p.P ? p.b2[i] : 0.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int j = 16 * jb + li;
      w.w1[jb][q] = (j < p.H && i < p.NB) ? p.W1[j * p.NB + i] : 0.f;      // A of Z^T: W1[j][i]
      const int jj = 16 * jb + 4 * g + q;
      w.b1r[jb][q] = jj < p.H ? p.b1[jj] : 0.f;                              // rows of Z^T
      w.w2[jb][q] = (li < p.P && jj < p.H) ? p.W2[li * p.H + jj] : 0.f;      // A of R^T: W2[p][j]
    }
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRbWaves * 16;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kRbWaves + wave) * 16;
  // Two tiles per trip, each tile's distances requested one tile ahead into its own register:
  // the wait for a load falls at the tile that uses it, a whole tile after the request.
  float da = rb_dist(p, first, li);
  for (int64_t e0 = first; e0 < p.E; e0 += 2 * stride) {
    const float db = rb_dist(p, e0 + stride, li);
    rb_fwd_tile(p, w, pic, g, li, e0, da, R);
    if (e0 + stride >= p.E) break;  // wave-uniform
    da = rb_dist(p, e0 + 2 * stride, li);
    rb_fwd_tile(p, w, pic, g, li, e0 + stride, db, R);
  }
}

// x_i(d) and dx_i/dd through the range-checked functions, returned by value.
__device__ __forceinline__ float2 basis_checked(float f, float d, float rdc, float env, float denv) {
#pragma clang fp contract(off)
  const float s = rb_sin(f * d);
  const float b = s * rdc;
  // d/dd [sin(f d) / dc] = f cos(f d) / dc - [d >= 1e-8] sin(f d) / dc^2
  const float db = f * rb_cos(f * d) * rdc - (d >= 1e-8f ? b * rdc : 0.f);
  return make_float2(b * env, db * env + b * denv);
}

// The lane's four basis values x_{4g+q}(d) and their derivatives in d.
struct RbBasis {
  float x[4], dx[4];
};

// Basis values and derivatives: the fast path as in rb_basis_fwd (wave-uniform), otherwise the
// range-checked functions.  Returned by value: output pointers into the caller's arrays kept
// those arrays in scratch memory.
__device__ __forceinline__ RbBasis rb_basis_bwd(const float* fr, int NB, int g, float pic, float d) {
  RbBasis r;
  const float t = pic * d;
  float a[4];
  bool fast = fabsf(t) < kRbFastArg;  // false for NaN
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = fr[q] * d;
    fast &= fabsf(a[q]) < kRbFastArg;
  }
  if (__ballot(!fast) == 0ull) {
    const float tr = t * kInv2Pi;
    const float e = 0.5f * (1.0f + __builtin_amdgcn_cosf(tr));
    const float env = e < 0.f ? 0.f : e;
    const float denv = -0.5f * __builtin_amdgcn_sinf(tr) * pic;
    const bool big = d >= 1e-8f;
    const float rdc = __builtin_amdgcn_rcpf(big ? d : 1e-8f);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float ar = a[q] * kInv2Pi;
      const float b = __builtin_amdgcn_sinf(ar) * rdc;
      const float db = fr[q] * __builtin_amdgcn_cosf(ar) * rdc - (big ? b * rdc : 0.f);
      r.dx[q] = db * env + b * denv;
      r.x[q] = b * env;
    }
  } else {
    float env, denv;
    envelope(d, pic, env, denv);
    const float rdc = rb_rdc(d);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float2 v = 4 * g + q < NB ? basis_checked(fr[q], d, rdc, env, denv) : make_float2(0.f, 0.f);
      r.x[q] = v.x;
      r.dx[q] = v.y;
    }
  }
  return r;
}

// Backward.  NQP = ceil(P / 4): in the products over the outputs (dH = dR W2) lane group g of MFMA
// q holds output 4q + g, so only the first NQP of the four k chunks are non-zero and issued
// (P = 5: 8 of the 16 MFMAs).  Distances and dR rows come through per-tile buffer resources:
// edges past E read 0 (basis values 0, dR 0), so they add nothing and need no branches.
// Waves per SIMD of the backward: three fit its registers for P <= 8; more outputs need two.
template <int NQP>
constexpr int rb_bwd_waves() { return NQP <= 2 ? 3 : 2; }

template <int NQP>
__global__ __launch_bounds__(kRbThreads, rb_bwd_waves<NQP>()) void radial_bwd_kernel(RbParams p, const float* __restrict__ dR,
                                                               float* __restrict__ ddist,
                                                               float* __restrict__ part) {
  // The edge-loop transposes (tz, tx) and the final per-wave partials (red) share one LDS buffer
  // (a barrier separates them): 34 KB per block instead of 55 KB, so LDS no longer caps the
  // occupancy below what the registers allow.
  constexpr int kTz = kRbWaves * 16 * (kRbMaxHidden + 1), kTx = kRbWaves * 16 * 17;
  constexpr int kRed = kRbWaves * kRbPart;
  __shared__ float smem[kTz + kTx > kRed ? kTz + kTx : kRed];
  auto tz = reinterpret_cast<float (*)[16][kRbMaxHidden + 1]>(smem);  // dZ of 16 edges, per wave
  auto tx = reinterpret_cast<float (*)[16][17]>(smem + kTz);          // X of 16 edges x 16 basis
  auto red = reinterpret_cast<float (*)[kRbPart]>(smem);
  const float pic = 3.14159265358979323846f / p.cutoff;
  const int lane = lane_id();
  const int g = lane >> 4, li = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  float fr[4];
  float w1[4][4], w2b[4][NQP], w1t[4][4], b1z[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * g + q;
    fr[q] = i < p.NB ? p.freqs[i] : 0.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int j = 16 * jb + li;
      w1[jb][q] = (j < p.H && i < p.NB) ? p.W1[j * p.NB + i] : 0.f;   // B of Z = X W1^T
      const int po = 4 * q + g;
      if (q < NQP) w2b[jb][q] = (po < p.P && j < p.H) ? p.W2[po * p.H + j] : 0.f;  // B of dH = dR W2
      const int jj = 16 * jb + 4 * g + q;
      w1t[jb][q] = (jj < p.H && li < p.NB) ? p.W1[jj * p.NB + li] : 0.f;  // A of dX^T = W1^T dZ^T
    }
  }
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) b1z[jb] = 16 * jb + li < p.H ? p.b1[16 * jb + li] : 0.f;
  floatx4 aw1[4], aw2[4];
  float db1p[4] = {0.f, 0.f, 0.f, 0.f}, db2p = 0.f;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    aw1[jb] = floatx4{0.f, 0.f, 0.f, 0.f};
    aw2[jb] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRbWaves * 16;
  for (int64_t e0 = (static_cast<int64_t>(blockIdx.x) * kRbWaves + wave) * 16; e0 < p.E; e0 += stride) {
    const int64_t left = p.E - e0;
    const int64_t nr = left > 16 ? 16 : left;
    const auto rsd = rb_rsrc(p.dist + e0, nr);
    const auto rsg = rb_rsrc(dR + e0 * p.P, nr * p.P);
    // edge li: x_i, i = 4g + q (A of Z; also the layout of dX^T) and dR[e][4q + g] (A of dH)
    const float da = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsd, 4u * li, 0, 0));
    float dra[NQP], drb[4];
#pragma unroll
    for (int q = 0; q < NQP; ++q) {
      const int po = 4 * q + g;
      const uint32_t off = po < p.P ? 4u * static_cast<uint32_t>(li * p.P + po) : 0x80000000u;
      dra[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsg, off, 0, 0));
    }
    // edges 4g + q: dR[e][li] (A of dW2)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t off = li < p.P ? 4u * static_cast<uint32_t>((4 * g + q) * p.P + li) : 0x80000000u;
      drb[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsg, off, 0, 0));
    }
    const RbBasis bs = rb_basis_bwd(fr, p.NB, g, pic, da);
    const float* xa = bs.x;
    const float* dxa = bs.dx;
    // edges 4g + q: x_li (A of dW1^T, the transpose of xa through LDS)
#pragma unroll
    for (int q = 0; q < 4; ++q) tx[wave][li][4 * g + q] = xa[q];
    float xb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) db2p += drb[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < 4; ++q) xb[q] = tx[wave][4 * g + q][li];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      // the bias starts the accumulator: Z = b1 + X W1^T
      floatx4 z = {b1z[jb], b1z[jb], b1z[jb], b1z[jb]}, dh = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) z = mfma4(xa[q], w1[jb][q], z);     // Z[e = 4g + q'][j = 16 jb + li]
#pragma unroll
      for (int q = 0; q < NQP; ++q) dh = mfma4(dra[q], w2b[jb][q], dh);  // dH, same layout
      floatx4 h, dz;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float zz = z[q];
        const float sg = sigmoid(zz);
        h[q] = zz * sg;
        dz[q] = dh[q] * (sg * (1.0f + zz * (1.0f - sg)));  // silu'(z) = s (1 + z (1 - s))
        db1p[jb] += dz[q];
        tz[wave][4 * g + q][16 * jb + li] = dz[q];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        aw2[jb] = mfma4(drb[q], h[q], aw2[jb]);   // dW2[p = 4g + q'][j]   (k = edges)
        aw1[jb] = mfma4(xb[q], dz[q], aw1[jb]);   // dW1^T[i = 4g + q'][j]
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (ddist) {
      floatx4 dx = {0.f, 0.f, 0.f, 0.f};  // dX^T[i = 4g + q][e = li]
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) dx = mfma4(w1t[c][q], tz[wave][li][16 * c + 4 * g + q], dx);
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) s += dx[q] * dxa[q];
      s += __shfl_xor(s, 16, kWave);
      s += __shfl_xor(s, 32, kWave);
      if (g == 0 && li < nr) ddist[e0 + li] = s;
    }
    __builtin_amdgcn_wave_barrier();
  }
  // db1 / db2: sum over the four lane groups
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    db1p[jb] += __shfl_xor(db1p[jb], 16, kWave);
    db1p[jb] += __shfl_xor(db1p[jb], 32, kWave);
  }
  db2p += __shfl_xor(db2p, 16, kWave);
  db2p += __shfl_xor(db2p, 32, kWave);
  __syncthreads();  // every wave is past its edge loop: tz / tx are dead, red may overwrite them
  float* my = red[wave];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      my[(4 * g + q) * 64 + 16 * jb + li] = aw1[jb][q];
      my[1024 + (4 * g + q) * 64 + 16 * jb + li] = aw2[jb][q];
    }
  if (g == 0) {
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) my[2048 + 16 * jb + li] = db1p[jb];
    my[2112 + li] = db2p;
  }
  __syncthreads();
  for (int k = threadIdx.x; k < kRbPart; k += kRbThreads) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kRbWaves; ++w) s += red[w][k];
    part[static_cast<int64_t>(blockIdx.x) * kRbPart + k] = s;
  }
}

// Sum of the per-block partials, then scattered into the gradient tensors.  Each block sums 64
// entries over all partial blocks with kRbFinalGroups thread groups (group g takes blocks
// b = g mod kRbFinalGroups in order), then adds the group sums in order: a fixed order, so results
// are deterministic.  Sixteen groups keep about 50 independent loads per thread in flight for
// 768 partial blocks (four groups left the kernel waiting on 192 loads per thread).
constexpr int kRbFinalGroups = 16;
constexpr int kRbFinalThreads = 64 * kRbFinalGroups;

__global__ __launch_bounds__(kRbFinalThreads) void radial_bwd_final(const float* __restrict__ part, int nblk,
                                                              int NB, int H, int P,
                                                              float* __restrict__ dW1,
                                                              float* __restrict__ db1,
                                                              float* __restrict__ dW2,
                                                              float* __restrict__ db2) {
  __shared__ float red[kRbFinalGroups][64];
  const int kl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + kl;
  float s = 0.f;
  if (k < kRbPart) {
#pragma unroll 8
    for (int b = grp; b < nblk; b += kRbFinalGroups) s += part[static_cast<int64_t>(b) * kRbPart + k];
  }
  red[grp][kl] = s;
  __syncthreads();
  if (grp != 0 || k >= kRbPart) return;
  s = red[0][kl];
#pragma unroll
  for (int gg = 1; gg < kRbFinalGroups; ++gg) s += red[gg][kl];
  if (k < 1024) {
    const int i = k / 64, j = k % 64;
    if (i < NB && j < H && dW1) dW1[j * NB + i] = s;
  } else if (k < 2048) {
    const int pp = (k - 1024) / 64, j = (k - 1024) % 64;
    if (pp < P && j < H && dW2) dW2[pp * H + j] = s;
  } else if (k < 2112) {
    const int j = k - 2048;
    if (j < H && db1) db1[j] = s;
  } else {
    const int pp = k - 2112;
    if (pp < P && db2) db2[pp] = s;
  }
}

// --------------------------------------------------------------- any layer sizes ---
// Layers beyond the MFMA kernels' 16 basis functions, 64 hidden units or 16 outputs.  A
// workgroup takes TE edges at a time (TE from the layer sizes, so the tile's values fit 48 KB of
// LDS): the basis values x[i][e], the hidden pre-activations z[j][e] and, in the backward, their
// gradients are staged in LDS with the edge index fastest (consecutive threads, consecutive
// edges: no bank conflicts), and every sum runs over its index in ascending order.  The weight
// rows are read from global memory (the same row by all threads of a step: cached).  The
// backward keeps per-workgroup weight-gradient partials in the workspace (each element owned by
// one thread) and sums them over the workgroups in order, as the MFMA path does, so the results
// are deterministic.
constexpr int kRgLdsFloats = 12288;  // 48 KB
constexpr int kRgMaxBlocks = 512;

__host__ __device__ inline int rg_tile_fwd(int NB, int H) {
  const int t = kRgLdsFloats / (NB + H);
  return t < 1 ? 1 : (t > 64 ? 64 : t);
}
__host__ __device__ inline int rg_tile_bwd(int NB, int H, int P) {
  const int t = kRgLdsFloats / (2 * NB + 2 * H + P);
  return t < 1 ? 1 : (t > 64 ? 64 : t);
}
__host__ __device__ inline int64_t rg_part_elems(int NB, int H, int P) {
  return static_cast<int64_t>(H) * NB + static_cast<int64_t>(P) * H + H + P;
}

// x[i][e] (and dx/dd) of the tile's edges; env/rdc per edge first.
__device__ __forceinline__ void rg_basis_tile(const RbParams& p, int64_t e0, int te, float pic,
                                              float* x, float* dxdd) {
  for (int q = threadIdx.x; q < te * p.NB; q += kRbThreads) {
    const int i = q / te, e = q % te;
    const int64_t ge = e0 + e;
    const float d = ge < p.E ? p.dist[ge] : 1.f;
    float env, denv;
    envelope(d, pic, env, denv);
    float dx = 0.f;
    x[i * te + e] = basis(p.freqs[i], d, rb_rdc(d), env, denv, dxdd ? &dx : nullptr);
    if (dxdd) dxdd[i * te + e] = dx;
  }
}

__global__ __launch_bounds__(kRbThreads) void radial_fwd_general(RbParams p, float* __restrict__ R) {
  extern __shared__ float smem[];
  const int te = rg_tile_fwd(p.NB, p.H);
  float* x = smem;                // [NB][te]
  float* h = smem + p.NB * te;    // [H][te]
  const float pic = 3.14159265358979323846f / p.cutoff;
  for (int64_t e0 = static_cast<int64_t>(blockIdx.x) * te; e0 < p.E;
       e0 += static_cast<int64_t>(gridDim.x) * te) {
    rg_basis_tile(p, e0, te, pic, x, nullptr);
    __syncthreads();
    for (int q = threadIdx.x; q < te * p.H; q += kRbThreads) {
      const int j = q / te, e = q % te;
      const float* w = p.W1 + static_cast<int64_t>(j) * p.NB;
      float z = 0.f;
      for (int i = 0; i < p.NB; ++i) z += w[i] * x[i * te + e];
      h[j * te + e] = silu(z + p.b1[j]);
    }
    __syncthreads();
    for (int q = threadIdx.x; q < te * p.P; q += kRbThreads) {
      const int e = q / p.P, pp = q % p.P;  // output-major: consecutive threads, consecutive R
      const int64_t ge = e0 + e;
      const float* w = p.W2 + static_cast<int64_t>(pp) * p.H;
      float r = 0.f;
      for (int j = 0; j < p.H; ++j) r += w[j] * h[j * te + e];
      if (ge < p.E) R[ge * p.P + pp] = r + p.b2[pp];
    }
    __syncthreads();
  }
}

// Backward of one tile per step; part (rg_part_elems floats per workgroup) accumulates
// dW1 [H][NB] | dW2 [P][H] | db1 [H] | db2 [P] over the workgroup's tiles.
__global__ __launch_bounds__(kRbThreads) void radial_bwd_general(RbParams p, const float* __restrict__ dR,
                                                                 float* __restrict__ ddist,
                                                                 float* __restrict__ part) {
  extern __shared__ float smem[];
  const int NB = p.NB, H = p.H, P = p.P;
  const int te = rg_tile_bwd(NB, H, P);
  float* x = smem;             // [NB][te]
  float* dxdd = x + NB * te;   // [NB][te]
  float* h = dxdd + NB * te;   // [H][te]
  float* dz = h + H * te;      // [H][te]: z, then its gradient
  float* dr = dz + H * te;     // [P][te]
  const float pic = 3.14159265358979323846f / p.cutoff;
  const int64_t np = rg_part_elems(NB, H, P);
  float* mine = part + static_cast<int64_t>(blockIdx.x) * np;
  for (int64_t q = threadIdx.x; q < np; q += kRbThreads) mine[q] = 0.f;
  for (int64_t e0 = static_cast<int64_t>(blockIdx.x) * te; e0 < p.E;
       e0 += static_cast<int64_t>(gridDim.x) * te) {
    rg_basis_tile(p, e0, te, pic, x, dxdd);
    for (int q = threadIdx.x; q < te * P; q += kRbThreads) {
      const int e = q / P, pp = q % P;
      const int64_t ge = e0 + e;
      dr[pp * te + e] = ge < p.E ? dR[ge * P + pp] : 0.f;  // edges past E add nothing
    }
    __syncthreads();
    for (int q = threadIdx.x; q < te * H; q += kRbThreads) {
      const int j = q / te, e = q % te;
      const float* w = p.W1 + static_cast<int64_t>(j) * NB;
      float z = 0.f;
      for (int i = 0; i < NB; ++i) z += w[i] * x[i * te + e];
      z += p.b1[j];
      const float sg = sigmoid(z);
      h[j * te + e] = z * sg;
      float g = 0.f;  // dH = dR W2
      for (int pp = 0; pp < P; ++pp) g += dr[pp * te + e] * p.W2[static_cast<int64_t>(pp) * H + j];
      dz[j * te + e] = g * (sg * (1.f + z * (1.f - sg)));  // silu'(z)
    }
    __syncthreads();
    // d dist: dX = dZ W1, then sum_i dX_i dx_i/dd
    if (ddist)
      for (int e = threadIdx.x; e < te; e += kRbThreads) {
        const int64_t ge = e0 + e;
        float dd = 0.f;
        for (int i = 0; i < NB; ++i) {
          float gx = 0.f;
          for (int j = 0; j < H; ++j) gx += dz[j * te + e] * p.W1[static_cast<int64_t>(j) * NB + i];
          dd += gx * dxdd[i * te + e];
        }
        if (ge < p.E) ddist[ge] = dd;
      }
    // weight gradients of the tile, added to this workgroup's partials
    for (int64_t q = threadIdx.x; q < np; q += kRbThreads) {
      float s = 0.f;
      if (q < static_cast<int64_t>(H) * NB) {
        const int j = static_cast<int>(q / NB), i = static_cast<int>(q % NB);
        for (int e = 0; e < te; ++e) s += dz[j * te + e] * x[i * te + e];
      } else if (q < static_cast<int64_t>(H) * NB + static_cast<int64_t>(P) * H) {
        const int64_t r = q - static_cast<int64_t>(H) * NB;
        const int pp = static_cast<int>(r / H), j = static_cast<int>(r % H);
        for (int e = 0; e < te; ++e) s += dr[pp * te + e] * h[j * te + e];
      } else if (q < static_cast<int64_t>(H) * NB + static_cast<int64_t>(P) * H + H) {
        const int j = static_cast<int>(q - static_cast<int64_t>(H) * NB - static_cast<int64_t>(P) * H);
        for (int e = 0; e < te; ++e) s += dz[j * te + e];
      } else {
        const int pp = static_cast<int>(q - static_cast<int64_t>(H) * NB - static_cast<int64_t>(P) * H - H);
        for (int e = 0; e < te; ++e) s += dr[pp * te + e];
      }
      mine[q] += s;
    }
    __syncthreads();
  }
}

// Sums the workgroups' partials in workgroup order into the requested gradients.
__global__ __launch_bounds__(kRbThreads) void radial_bwd_general_final(
    const float* __restrict__ part, int nblk, int NB, int H, int P, float* __restrict__ dW1,
    float* __restrict__ db1, float* __restrict__ dW2, float* __restrict__ db2) {
  const int64_t np = rg_part_elems(NB, H, P);
  const int64_t q = static_cast<int64_t>(blockIdx.x) * kRbThreads + threadIdx.x;
  if (q >= np) return;
  float s = 0.f;
  for (int b = 0; b < nblk; ++b) s += part[static_cast<int64_t>(b) * np + q];
  const int64_t a = static_cast<int64_t>(H) * NB, b2 = a + static_cast<int64_t>(P) * H;
  if (q < a) {
    if (dW1) dW1[q] = s;  // [H][NB], the same layout
  } else if (q < b2) {
    if (dW2) dW2[q - a] = s;  // [P][H]
  } else if (q < b2 + H) {
    if (db1) db1[q - b2] = s;
  } else if (db2) {
    db2[q - b2 - H] = s;
  }
}

bool rb_fits_mfma(int NB, int H, int P) {
  return NB <= kRbMaxBasis && H <= kRbMaxHidden && P <= kRbMaxOut;
}

unsigned rg_blocks(int64_t E, int te) {
  const int64_t b = ceil_div(E, te);
  return static_cast<unsigned>(b < 1 ? 1 : (b > kRgMaxBlocks ? kRgMaxBlocks : b));
}

int rb_check(const char* who, int64_t E, int NB, int H, int P, float cutoff) {
  GEO_REQUIRE(E >= 0, "%s: negative E", who);
  GEO_REQUIRE(NB >= 1 && H >= 1 && P >= 1, "%s: layer sizes must be positive (num_basis=%d, "
              "hidden=%d, outputs=%d)", who, NB, H, P);
  GEO_REQUIRE(static_cast<int64_t>(NB) + H <= kRgLdsFloats && 2LL * NB + 2LL * H + P <= kRgLdsFloats,
              "%s: layer sizes too large (num_basis=%d, hidden=%d, outputs=%d)", who, NB, H, P);
  GEO_REQUIRE(cutoff > 0.f, "%s: cutoff must be positive", who);
  return GEO_OK;
}

unsigned rb_blocks(int64_t E) {
  const int64_t b = ceil_div(E, 16 * kRbWaves * 4);  // about four 16-edge tiles per wave
  return static_cast<unsigned>(b < 1 ? 1 : (b > kRbMaxBlocks ? kRbMaxBlocks : b));
}

}  // namespace
}  // namespace geo

using namespace geo;

extern "C" int geo_radial_mlp_fwd(const float* dist, int64_t E, const float* freqs, int32_t NB,
                                  float cutoff, const float* W1, const float* b1, int32_t H,
                                  const float* W2, const float* b2, int32_t P, float* R,
                                  void* stream) {
  int rc = rb_check("radial_mlp_fwd", E, NB, H, P, cutoff);
  if (rc) return rc;
  if (E == 0) return GEO_OK;
  GEO_REQUIRE(dist && freqs && W1 && b1 && W2 && b2 && R, "radial_mlp_fwd: null pointer");
  RbParams p{dist, E, freqs, NB, cutoff, W1, b1, H, W2, b2, P};
  if (!rb_fits_mfma(NB, H, P)) {
    const int te = rg_tile_fwd(NB, H);
    hipLaunchKernelGGL(radial_fwd_general, dim3(rg_blocks(E, te)), dim3(kRbThreads),
                       static_cast<size_t>(te) * (NB + H) * sizeof(float), as_stream(stream), p, R);
    GEO_LAUNCH_CHECK("radial_fwd_general");
    return GEO_OK;
  }
  hipLaunchKernelGGL(radial_fwd_kernel, dim3(rb_blocks(E)), dim3(kRbThreads), 0, as_stream(stream), p, R);
  GEO_LAUNCH_CHECK("radial_fwd_kernel");
  return GEO_OK;
}

extern "C" size_t geo_radial_mlp_bwd_workspace_bytes(int64_t E, int32_t NB, int32_t H, int32_t P) {
  if (E < 0 || NB < 1 || H < 1 || P < 1) return 0;
  if (!rb_fits_mfma(NB, H, P))
    return static_cast<size_t>(rg_blocks(E, rg_tile_bwd(NB, H, P))) * rg_part_elems(NB, H, P) *
           sizeof(float);
  return static_cast<size_t>(rb_blocks(E)) * kRbPart * sizeof(float);
}

extern "C" int geo_radial_mlp_bwd(const float* dist, int64_t E, const float* freqs, int32_t NB,
                                  float cutoff, const float* W1, const float* b1, int32_t H,
                                  const float* W2, const float* b2, int32_t P, const float* dR,
                                  float* d_dist, float* dW1, float* db1, float* dW2, float* db2,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = rb_check("radial_mlp_bwd", E, NB, H, P, cutoff);
  if (rc) return rc;
  GEO_REQUIRE(freqs && W1 && b1 && W2 && b2, "radial_mlp_bwd: null weight pointer");
  hipStream_t st = as_stream(stream);
  if (E == 0) {  // weight gradients of an empty batch are zero
    if (dW1) { rc = device_fill<float>(dW1, static_cast<int64_t>(H) * NB, 0.f, st); if (rc) return rc; }
    if (db1) { rc = device_fill<float>(db1, H, 0.f, st); if (rc) return rc; }
    if (dW2) { rc = device_fill<float>(dW2, static_cast<int64_t>(P) * H, 0.f, st); if (rc) return rc; }
    if (db2) { rc = device_fill<float>(db2, P, 0.f, st); if (rc) return rc; }
    return GEO_OK;
  }
  GEO_REQUIRE(dist && dR, "radial_mlp_bwd: null pointer");
  const size_t need = geo_radial_mlp_bwd_workspace_bytes(E, NB, H, P);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(GEO_ERR_WORKSPACE, "radial_mlp_bwd: workspace %zu bytes, need %zu",
                     workspace_bytes, need);
  RbParams p{dist, E, freqs, NB, cutoff, W1, b1, H, W2, b2, P};
  if (!rb_fits_mfma(NB, H, P)) {
    const int te = rg_tile_bwd(NB, H, P);
    const unsigned nb = rg_blocks(E, te);
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(radial_bwd_general, dim3(nb), dim3(kRbThreads),
                       static_cast<size_t>(te) * (2 * NB + 2 * H + P) * sizeof(float), st, p, dR,
                       d_dist, part);
    GEO_LAUNCH_CHECK("radial_bwd_general");
    hipLaunchKernelGGL(radial_bwd_general_final,
                       dim3(static_cast<unsigned>(ceil_div(rg_part_elems(NB, H, P), kRbThreads))),
                       dim3(kRbThreads), 0, st, part, static_cast<int>(nb), NB, H, P, dW1, db1, dW2,
                       db2);
    GEO_LAUNCH_CHECK("radial_bwd_general_final");
    return GEO_OK;
  }
  // one resident round: three (P <= 8) or two waves per SIMD, 768 or 512 blocks on 256 CUs
  const unsigned cap = P <= 8 ? 768u : 512u;
  const unsigned nblk = rb_blocks(E) < cap ? rb_blocks(E) : cap;
  float* part = static_cast<float*>(workspace);
  switch ((P + 3) / 4) {
    case 1: hipLaunchKernelGGL(radial_bwd_kernel<1>, dim3(nblk), dim3(kRbThreads), 0, st, p, dR, d_dist, part); break;
    case 2: hipLaunchKernelGGL(radial_bwd_kernel<2>, dim3(nblk), dim3(kRbThreads), 0, st, p, dR, d_dist, part); break;
    case 3: hipLaunchKernelGGL(radial_bwd_kernel<3>, dim3(nblk), dim3(kRbThreads), 0, st, p, dR, d_dist, part); break;
    default: hipLaunchKernelGGL(radial_bwd_kernel<4>, dim3(nblk), dim3(kRbThreads), 0, st, p, dR, d_dist, part); break;
  }
  GEO_LAUNCH_CHECK("radial_bwd_kernel");
  hipLaunchKernelGGL(radial_bwd_final, dim3(static_cast<unsigned>(ceil_div(kRbPart, 64))),
                     dim3(kRbFinalThreads), 0, st, part, static_cast<int>(nblk), NB, H, P, dW1, db1,
                     dW2, db2);
  GEO_LAUNCH_CHECK("radial_bwd_final");
  return GEO_OK;
}
