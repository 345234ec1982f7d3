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

__global__ __launch_bounds__(kRbThreads) void radial_fwd_kernel(RbParams p, float* __restrict__ R) {
  const float pic = 3.14159265358979323846f / p.cutoff;
  const int lane = lane_id();
  const int g = lane >> 4, li = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  float w1[4][4], b1r[4][4], w2[4][4], fr[4], b2r[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * g + q;
    fr[q] = i < p.NB ? p.freqs[i] : 0.f;
    b2r[q] = i < p.P ? p.b2[i] : 0.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int j = 16 * jb + li;
      w1[jb][q] = (j < p.H && i < p.NB) ? p.W1[j * p.NB + i] : 0.f;      // A of Z^T: W1[j][i]
      const int jj = 16 * jb + 4 * g + q;
      b1r[jb][q] = jj < p.H ? p.b1[jj] : 0.f;                              // rows of Z^T
      w2[jb][q] = (li < p.P && jj < p.H) ? p.W2[li * p.H + jj] : 0.f;      // A of R^T: W2[p][j]
    }
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRbWaves * 16;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kRbWaves + wave) * 16;
  float d_next = first + li < p.E ? p.dist[first + li] : 1.f;  // distances one tile ahead
  for (int64_t e0 = first; e0 < p.E; e0 += stride) {
    const int64_t e = e0 + li;
    const bool ok = e < p.E;
    const float d = d_next;
    d_next = e + stride < p.E ? p.dist[e + stride] : 1.f;
    float env, denv;
    envelope(d, pic, env, denv);
    const float rdc = rb_rdc(d);
    float x[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) x[q] = 4 * g + q < p.NB ? basis(fr[q], d, rdc, env, denv, nullptr) : 0.f;
    floatx4 h[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      floatx4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) z = mfma4(w1[jb][q], x[q], z);
#pragma unroll
      for (int q = 0; q < 4; ++q) h[jb][q] = silu(z[q] + b1r[jb][q]);
    }
    // four independent accumulation chains (one per 16-wide hidden chunk), summed at the end
    floatx4 rc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) rc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int c = 0; c < 4; ++c) rc[c] = mfma4(w2[c][q], h[c][q], rc[c]);
    const floatx4 r = (rc[0] + rc[1]) + (rc[2] + rc[3]);
    if (ok) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * g + q < p.P) R[e * p.P + 4 * g + q] = r[q] + b2r[q];
    }
  }
}

__global__ __launch_bounds__(kRbThreads, 3) void radial_bwd_kernel(RbParams p, const float* __restrict__ dR,
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
  float w1[4][4], w2b[4][4], w1t[4][4], b1z[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 4 * g + q;
    fr[q] = i < p.NB ? p.freqs[i] : 0.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int j = 16 * jb + li;
      w1[jb][q] = (j < p.H && i < p.NB) ? p.W1[j * p.NB + i] : 0.f;   // B of Z = X W1^T
      w2b[jb][q] = (i < p.P && j < p.H) ? p.W2[i * p.H + j] : 0.f;    // B of dH = dR W2
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
    // edge li: x_i, i = 4g + q (A of Z; also the layout of dX^T) and dR[e][4g + q] (A of dH)
    const int64_t ea = e0 + li;
    const bool oka = ea < p.E;
    const float da = oka ? p.dist[ea] : 1.f;
    float enva, denva;
    envelope(da, pic, enva, denva);
    const float rdca = rb_rdc(da);
    float xa[4], dxa[4], dra[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = 4 * g + q;
      xa[q] = i < p.NB ? basis(fr[q], da, rdca, enva, denva, &dxa[q]) : 0.f;
      if (i >= p.NB) dxa[q] = 0.f;
      dra[q] = (oka && i < p.P) ? dR[ea * p.P + i] : 0.f;
    }
    // edges 4g + q: x_li (A of dW1^T, the transpose of xa through LDS) and dR[e][li] (A of dW2)
#pragma unroll
    for (int q = 0; q < 4; ++q) tx[wave][li][4 * g + q] = oka ? xa[q] : 0.f;
    float xb[4], drb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t eb = e0 + 4 * g + q;
      const bool okb = eb < p.E;
      drb[q] = (okb && li < p.P) ? dR[eb * p.P + li] : 0.f;
      db2p += drb[q];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int q = 0; q < 4; ++q) xb[q] = tx[wave][4 * g + q][li];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      floatx4 z = {0.f, 0.f, 0.f, 0.f}, dh = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        z = mfma4(xa[q], w1[jb][q], z);     // Z[e = 4g + q'][j = 16 jb + li]
        dh = mfma4(dra[q], w2b[jb][q], dh);  // dH, same layout
      }
      floatx4 h, dz;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float zz = z[q] + b1z[jb];
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
      floatx4 dxc[4];  // four independent accumulation chains, summed at the end
#pragma unroll
      for (int c = 0; c < 4; ++c) dxc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int c = 0; c < 4; ++c) dxc[c] = mfma4(w1t[c][q], tz[wave][li][16 * c + 4 * g + q], dxc[c]);
      const floatx4 dx = (dxc[0] + dxc[1]) + (dxc[2] + dxc[3]);
      // dX^T[i = 4g + q][e = li]
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) s += dx[q] * dxa[q];
      s += __shfl_xor(s, 16, kWave);
      s += __shfl_xor(s, 32, kWave);
      if (g == 0 && oka) ddist[ea] = s;
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
// entries over all partial blocks with four thread groups (group g takes blocks b = g mod 4 in
// order), then adds the four group sums in order: a fixed order, so results are deterministic.
__global__ __launch_bounds__(kRbThreads) void radial_bwd_final(const float* __restrict__ part, int nblk,
                                                              int NB, int H, int P,
                                                              float* __restrict__ dW1,
                                                              float* __restrict__ db1,
                                                              float* __restrict__ dW2,
                                                              float* __restrict__ db2) {
  __shared__ float red[4][64];
  const int kl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + kl;
  float s = 0.f;
  if (k < kRbPart) {
#pragma unroll 8
    for (int b = grp; b < nblk; b += 4) s += part[static_cast<int64_t>(b) * kRbPart + k];
  }
  red[grp][kl] = s;
  __syncthreads();
  if (grp != 0 || k >= kRbPart) return;
  s = ((red[0][kl] + red[1][kl]) + red[2][kl]) + red[3][kl];
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
  // three waves per SIMD fit the backward: one resident round of 768 blocks on 256 CUs
  const unsigned nblk = rb_blocks(E) < 768u ? rb_blocks(E) : 768u;
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(radial_bwd_kernel, dim3(nblk), dim3(kRbThreads), 0, st, p, dR, d_dist, part);
  GEO_LAUNCH_CHECK("radial_bwd_kernel");
  hipLaunchKernelGGL(radial_bwd_final, dim3(static_cast<unsigned>(ceil_div(kRbPart, 64))),
                     dim3(kRbThreads), 0, st, part, static_cast<int>(nblk), NB, H, P, dW1, db1, dW2, db2);
  GEO_LAUNCH_CHECK("radial_bwd_final");
  return GEO_OK;
}
