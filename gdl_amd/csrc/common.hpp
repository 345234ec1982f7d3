// common.hpp — shared host/device helpers for the gfx950 geometry kernels.
//
// gfx950 (CDNA4) runs 64-lane wavefronts only; every cross-lane helper below assumes that.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/geo_api.h"

namespace geo {

constexpr int kWave = 64;

// ---------------------------------------------------------------- host errors ---

// Records a message for geo_last_error() on the calling thread; returns `code`.
int set_error(int code, const char* fmt, ...);

#define GEO_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::geo::set_error(GEO_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define GEO_HIP_CHECK(expr)                                                        \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess)                                                          \
      return ::geo::set_error(GEO_ERR_HIP, "%s failed: %s (%s:%d)", #expr,         \
                              hipGetErrorString(_e), __FILE__, __LINE__);          \
  } while (0)

// Checks the launch status of the kernels enqueued just before.
#define GEO_LAUNCH_CHECK(what)                                                     \
  do {                                                                             \
    hipError_t _e = hipGetLastError();                                             \
    if (_e != hipSuccess)                                                          \
      return ::geo::set_error(GEO_ERR_HIP, "launch of %s failed: %s", what,        \
                              hipGetErrorString(_e));                              \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves aligned sub-buffers out of one caller-provided workspace.
struct Carver {
  char* base;
  size_t used = 0;
  explicit Carver(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t count) {
    used = align_up(used, 256);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
};

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------- lane primitives ---

__device__ __forceinline__ int lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// DPP control codes (GFX9 encoding).
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;       // lane i <-> 15-i within 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Sum over all 64 lanes (every lane must be active), wave-uniform: DPP sums within each 16-lane
// row, then the four row totals read from lanes 0, 16, 32, 48 (no LDS round trips, unlike a
// shuffle tree).
__device__ __forceinline__ uint32_t wave_sum_dpp(uint32_t v) {
  v += dpp_u32<kDppXor1>(v);
  v += dpp_u32<kDppXor2>(v);
  v += dpp_u32<kDppHalfMirror>(v);
  v += dpp_u32<kDppMirror>(v);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return (static_cast<uint64_t>(dpp_u32<CTRL>(static_cast<uint32_t>(v >> 32))) << 32) |
         dpp_u32<CTRL>(static_cast<uint32_t>(v));
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l))) << 32) |
         static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}
__device__ __forceinline__ uint64_t wave_sum_dpp(uint64_t v) {
  v += dpp_u64<kDppXor1>(v);
  v += dpp_u64<kDppXor2>(v);
  v += dpp_u64<kDppHalfMirror>(v);
  v += dpp_u64<kDppMirror>(v);
  return readlane_u64(v, 0) + readlane_u64(v, 16) + readlane_u64(v, 32) + readlane_u64(v, 48);
}

// DPP move with bound_ctrl: lanes without a source read 0, which lets the compiler fuse the
// move into the consuming v_max_u32 (one v_max_u32_dpp per step).  0 is the identity of an
// unsigned max.
constexpr int kDppBcast15 = 0x142;      // lane 15 of each row -> the next row
constexpr int kDppBcast31 = 0x143;      // lane 31 -> rows 2 and 3

template <int CTRL>
__device__ __forceinline__ uint32_t dpp0_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also orders global memory,
// which on gfx950 means waiting for every outstanding vector memory operation of the wave,
// stores included, before the barrier; loops whose waves exchange data only through LDS use this
// one, so their global stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS writes of some lanes become visible to later reads of other lanes of the same wave.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// Wave-uniform max over all 64 lanes (every lane must be active): four in-row steps, two row
// broadcasts, lane 63 holds the result.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp0_u32<kDppXor1>(v));
  v = max(v, dpp0_u32<kDppXor2>(v));
  v = max(v, dpp0_u32<kDppHalfMirror>(v));
  v = max(v, dpp0_u32<kDppMirror>(v));
  v = max(v, dpp0_u32<kDppBcast15>(v));
  v = max(v, dpp0_u32<kDppBcast31>(v));
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return ~wave_max_u32(~v); }

// DPP move into the rows of ROWS (bit r = row r) with bound_ctrl: sources outside the row, and
// rows outside ROWS, read 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp0_rows_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROWS, 0xF, true));
}

// Wave-wide inclusive prefix sum of 32-bit values (every lane must be active), all in DPP:
// Hillis-Steele steps within each 16-lane row (row_shr 1, 2, 4, 8), then each row's total
// carried up (lane 15 of the row below into rows 1 and 3, lane 31 into rows 2 and 3).
__device__ __forceinline__ uint32_t wave_inclusive_sum_dpp(uint32_t v) {
  v += dpp0_rows_u32<0x111, 0xF>(v);  // row_shr:1
  v += dpp0_rows_u32<0x112, 0xF>(v);  // row_shr:2
  v += dpp0_rows_u32<0x114, 0xF>(v);  // row_shr:4
  v += dpp0_rows_u32<0x118, 0xF>(v);  // row_shr:8
  v += dpp0_rows_u32<kDppBcast15, 0xA>(v);
  v += dpp0_rows_u32<kDppBcast31, 0xC>(v);
  return v;
}

// The same two DPP patterns on 64-bit values, both halves moved by the same control.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t dpp0_rows_u64(uint64_t v) {
  return (static_cast<uint64_t>(dpp0_rows_u32<CTRL, ROWS>(static_cast<uint32_t>(v >> 32))) << 32) |
         dpp0_rows_u32<CTRL, ROWS>(static_cast<uint32_t>(v));
}
__device__ __forceinline__ uint64_t wave_inclusive_sum_dpp(uint64_t v) {
  v += dpp0_rows_u64<0x111, 0xF>(v);
  v += dpp0_rows_u64<0x112, 0xF>(v);
  v += dpp0_rows_u64<0x114, 0xF>(v);
  v += dpp0_rows_u64<0x118, 0xF>(v);
  v += dpp0_rows_u64<kDppBcast15, 0xA>(v);
  v += dpp0_rows_u64<kDppBcast31, 0xC>(v);
  return v;
}

// Max / min over lanes 0..15 only (row 0); other lanes' values are ignored.
__device__ __forceinline__ uint32_t row0_max_u32(uint32_t v) {
  v = max(v, dpp0_u32<kDppXor1>(v));
  v = max(v, dpp0_u32<kDppXor2>(v));
  v = max(v, dpp0_u32<kDppHalfMirror>(v));
  v = max(v, dpp0_u32<kDppMirror>(v));
  return __builtin_amdgcn_readlane(v, 0);
}
__device__ __forceinline__ uint32_t row0_min_u32(uint32_t v) { return ~row0_max_u32(~v); }

// Slot of this lane among the increments of counter[key] made by the active lanes: lanes with
// the same key share one atomic add (issued by the lowest of them), so a counter that many
// lanes hit at once is not serialised.  The adds are issued back to back and their results
// gathered once at the end.  `counter` must be the same address for equal keys.
__device__ __forceinline__ int wave_aggregated_rank(int* counter, int key) {
  const int lane = lane_id();
  uint64_t todo = __ballot(true);
  int base = 0, my_leader = lane, my_rank = 0;
  while (todo) {
    const int leader = __builtin_ctzll(todo);
    const int lk = __builtin_amdgcn_readlane(key, leader);
    const uint64_t peers = __ballot(key == lk) & todo;
    if (lane == leader) base = atomicAdd(counter, static_cast<int>(__popcll(peers)));
    if ((peers >> lane) & 1ull) {
      my_leader = leader;
      my_rank = static_cast<int>(__popcll(peers & lanemask_lt()));
    }
    todo &= ~peers;
  }
  return __shfl(base, my_leader, kWave) + my_rank;
}

// Rank of this point in its cell's counter (counter = its cell's count, key = its cell).  Points
// in scan order (lidar) put long runs of a wave into one cell: there one atomic per distinct cell
// (wave-aggregated) avoids serialising 64 atomics on one address; scattered points take plain
// per-lane atomics, since aggregation would loop over up to 64 distinct cells.  The run count
// comes from neighbouring-lane equality.
__device__ __forceinline__ int cell_rank(int* counter, int key) {
  const int lane = lane_id();
  const int prev = __shfl_up(key, 1, kWave);
  const int runs = __popcll(__ballot(lane == 0 || prev != key));
  if (runs <= 16) return wave_aggregated_rank(counter, key);
  return atomicAdd(counter, 1);
}

// Inclusive prefix sum and sum of 4- or 8-byte integers over the wave, all in DPP (every lane
// must be active).
template <typename T>
__device__ __forceinline__ T wave_inclusive_sum_int(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit integers");
  if constexpr (sizeof(T) == 4) return static_cast<T>(wave_inclusive_sum_dpp(static_cast<uint32_t>(v)));
  else return static_cast<T>(wave_inclusive_sum_dpp(static_cast<uint64_t>(v)));
}
template <typename T>
__device__ __forceinline__ T wave_sum_int(T v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit integers");
  if constexpr (sizeof(T) == 4) return static_cast<T>(wave_sum_dpp(static_cast<uint32_t>(v)));
  else return static_cast<T>(wave_sum_dpp(static_cast<uint64_t>(v)));
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// The dispatcher hands workgroups to the 8 XCDs in turn (workgroup b to XCD b mod 8).  This
// renumbering gives each XCD one contiguous range of workgroup indices, so neighbouring work
// items -- which share input rows -- are processed under the same L2.
__device__ __forceinline__ int64_t xcd_block() {
  const int64_t G = gridDim.x, b = blockIdx.x;
  const int64_t q = G / 8, r = G % 8, x = b % 8, k = b / 8;
  return x * q + (x < r ? x : r) + k;
}

// The same idea with the workgroup space cut into runs of `run` consecutive workgroups handed
// to the XCDs in turn: neighbouring work items still share an L2, and work whose cost varies
// over the index space (dense regions of a scene) is spread over all XCDs.  Workgroups past the
// last whole round of 8 runs keep their index.
__device__ __forceinline__ int64_t xcd_block_runs(int64_t run) {
  const int64_t G = gridDim.x, b = blockIdx.x;
  const int64_t whole = G / (8 * run) * (8 * run);
  if (b >= whole) return b;
  const int64_t x = b % 8, k = b / 8;
  return ((k / run) * 8 + x) * run + k % run;
}

// ---------------------------------------------------------- exact distance ---
// Squared distance with the reference's operation order, (dx*dx + dy*dy) + dz*dz, each
// operation rounded to fp32.  The library is compiled with -ffp-contract=off; the pragma keeps
// the multiply-adds unfused here even if that flag is dropped.
__device__ __forceinline__ float sqdist(float ax, float ay, float az, float bx, float by,
                                        float bz) {
#pragma clang fp contract(off)
  const float dx = ax - bx, dy = ay - by, dz = az - bz;
  return (dx * dx + dy * dy) + dz * dz;
}

// ---------------------------------------------------------------- bfloat16 ---
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round to nearest even; NaN -> canonical quiet NaN (matches PyTorch's conversion).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Float -> uint32 key that orders like the float (for atomic min / max on floats).
__device__ __forceinline__ uint32_t float_order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float float_from_order_key(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

}  // namespace geo
