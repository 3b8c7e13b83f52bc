// common.hpp -- shared helpers for the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>
#include <cstdint>
#include <string>

#include "fusiongpu.h"

namespace fgpu {

constexpr int kWave = 64;   // CDNA wavefront width
constexpr int kPQK = 256;   // PQ_K (defs.h:11): 8-bit codes
constexpr uint32_t kPruned = 0xFFFFFFFFu;  // pruned probe sentinel (gpu_global.cu:49)
constexpr int kPadId = INT_MAX;  // internal padding id; reported as -1

// ---- status plumbing (host) ----------------------------------------------
fgpu_status set_error(fgpu_status st, const std::string& msg);
inline fgpu_status ok() { return FGPU_OK; }

#define FGPU_HIP(call)                                                                   \
  do {                                                                                   \
    hipError_t e_ = (call);                                                              \
    if (e_ != hipSuccess)                                                                \
      return ::fgpu::set_error(FGPU_ERR_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define FGPU_CHECK(cond, st, msg)                        \
  do {                                                   \
    if (!(cond)) return ::fgpu::set_error((st), (msg));  \
  } while (0)

#define FGPU_TRY(expr)                   \
  do {                                   \
    fgpu_status s_ = (expr);             \
    if (s_ != FGPU_OK) return s_;        \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Bump allocator over a caller-owned device workspace.
struct Carve {
  char* base;
  size_t cap;
  size_t used = 0;
  Carve(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
  template <class T>
  T* take(size_t count) {
    size_t off = align_up(used, 256);
    used = off + align_up(count * sizeof(T), 256);
    return used <= cap ? reinterpret_cast<T*>(base + off) : nullptr;
  }
  bool ok() const { return used <= cap; }
};
template <class T>
inline size_t carve_bytes(size_t count) { return align_up(count * sizeof(T), 256); }

// ---- device helpers --------------------------------------------------------

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, kWave); }

// Order-preserving map float -> uint32 (ascending).
__device__ __forceinline__ uint32_t float_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

// ---- cross-lane exchange on the VALU ----------------------------------------
// x(lane ^ S) for one wave, without the LDS crossbar: DPP quad permutes for
// S = 1, 2, row rotates for S = 4, 8 (rotating a 16-lane row by 8 is xor 8;
// xor 4 picks the rotate by 4 or by 12 from bit 2 of the lane), and the gfx950
// permlane16/32 swaps for S = 16, 32.  Every lane must be active.
// A lane whose DPP source lies outside the wave (wave_shr:1 at lane 0) reads 0.
template <int C>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_mov_dpp(v, C, 0xF, 0xF, true);
}
template <int S>
__device__ __forceinline__ int xchg(int v) {
  if constexpr (S == 1) {
    return dpp_mov<0xB1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (S == 2) {
    return dpp_mov<0x4E>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (S == 4) {
    const int a = dpp_mov<0x124>(v), b = dpp_mov<0x12C>(v);  // row_ror:4, row_ror:12
    return (lane_id() & 4) ? a : b;
  } else if constexpr (S == 8) {
    return dpp_mov<0x128>(v);  // row_ror:8
  } else if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (lane_id() & 16) ? (int)r[0] : (int)r[1];
  } else {
    static_assert(S == 32, "xor exchange distance");
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (lane_id() & 32) ? (int)r[0] : (int)r[1];
  }
}

// x(63 - lane): mirror inside each 16-lane row, then swap rows 0<->3, 1<->2.
__device__ __forceinline__ int wave_reverse(int v) { return xchg<32>(xchg<16>(dpp_mov<0x140>(v))); }

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// ---- the same networks on packed 64-bit keys ---------------------------------
// A key is (float bits << 32) | id.  For distances >= 0 (sums of squares) and
// ids >= 0, ascending key order is exactly the tie rule (distance, then id),
// so a compare-exchange is one 64-bit compare and two selects, without the
// branchy two-field compare of the (d, id) pair form.
__device__ __forceinline__ uint64_t key_of(float d, int id) {
  return ((uint64_t)__float_as_uint(d) << 32) | (uint32_t)id;
}
__device__ __forceinline__ float key_dist(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }
__device__ __forceinline__ int key_id(uint64_t k) { return (int)(uint32_t)k; }
constexpr uint64_t kPadKey = ((uint64_t)0x7F7FFFFFu << 32) | (uint32_t)kPadId;  // (FLT_MAX, kPadId)

template <int S>
__device__ __forceinline__ uint64_t xchg64(uint64_t v) {
  const uint32_t lo = (uint32_t)xchg<S>((int)(uint32_t)v), hi = (uint32_t)xchg<S>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <int C>
__device__ __forceinline__ uint64_t dpp_mov64(uint64_t v) {
  const uint32_t lo = (uint32_t)dpp_mov<C>((int)(uint32_t)v), hi = (uint32_t)dpp_mov<C>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

// Compare-exchange at distance S: the lower lane of each pair keeps the
// smaller key when `up`, the larger otherwise (equal keys are interchangeable).
template <int S>
__device__ __forceinline__ void bitonic_stage_k(uint64_t& k, bool up) {
  const uint64_t o = xchg64<S>(k);
  const bool lower = (lane_id() & S) == 0;
  k = ((k < o) == (lower == up)) ? k : o;
}
template <int SIZE>
__device__ __forceinline__ void bitonic_pass_k(uint64_t& k, bool up) {
  if constexpr (SIZE > 32) bitonic_stage_k<32>(k, up);
  if constexpr (SIZE > 16) bitonic_stage_k<16>(k, up);
  if constexpr (SIZE > 8) bitonic_stage_k<8>(k, up);
  if constexpr (SIZE > 4) bitonic_stage_k<4>(k, up);
  if constexpr (SIZE > 2) bitonic_stage_k<2>(k, up);
  bitonic_stage_k<1>(k, up);
}
// Ascending bitonic sort of one key per lane across the wave.
__device__ __forceinline__ void wave_sort64_k(uint64_t& k) {
  const int lane = lane_id();
  bitonic_pass_k<2>(k, (lane & 2) == 0);
  bitonic_pass_k<4>(k, (lane & 4) == 0);
  bitonic_pass_k<8>(k, (lane & 8) == 0);
  bitonic_pass_k<16>(k, (lane & 16) == 0);
  bitonic_pass_k<32>(k, (lane & 32) == 0);
  bitonic_pass_k<64>(k, true);
}
// Ascending bitonic sort of one 32-bit key per lane across the wave.
template <int S>
__device__ __forceinline__ void bitonic_stage_u32(uint32_t& k, bool up) {
  const uint32_t o = (uint32_t)xchg<S>((int)k);
  const bool lower = (lane_id() & S) == 0;
  k = ((k < o) == (lower == up)) ? k : o;
}
template <int SIZE>
__device__ __forceinline__ void bitonic_pass_u32(uint32_t& k, bool up) {
  if constexpr (SIZE > 32) bitonic_stage_u32<32>(k, up);
  if constexpr (SIZE > 16) bitonic_stage_u32<16>(k, up);
  if constexpr (SIZE > 8) bitonic_stage_u32<8>(k, up);
  if constexpr (SIZE > 4) bitonic_stage_u32<4>(k, up);
  if constexpr (SIZE > 2) bitonic_stage_u32<2>(k, up);
  bitonic_stage_u32<1>(k, up);
}
__device__ __forceinline__ void wave_sort_u32(uint32_t& k) {
  const int lane = lane_id();
  bitonic_pass_u32<2>(k, (lane & 2) == 0);
  bitonic_pass_u32<4>(k, (lane & 4) == 0);
  bitonic_pass_u32<8>(k, (lane & 8) == 0);
  bitonic_pass_u32<16>(k, (lane & 16) == 0);
  bitonic_pass_u32<32>(k, (lane & 32) == 0);
  bitonic_pass_u32<64>(k, true);
}

__device__ __forceinline__ uint64_t wave_reverse64(uint64_t v) {
  const uint32_t lo = (uint32_t)wave_reverse((int)(uint32_t)v), hi = (uint32_t)wave_reverse((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
// list (ascending) := the 64 smallest of list U cand (cand ascending too).
__device__ __forceinline__ void wave_merge_sorted64_k(uint64_t& k, uint64_t cand) {
  const uint64_t r = wave_reverse64(cand);
  k = r < k ? r : k;
  bitonic_pass_k<64>(k, true);
}
// The same with an int payload travelling with each key.  A pair of equal
// keys is left in place, so payloads are never duplicated.
template <int S>
__device__ __forceinline__ void bitonic_stage_kp(uint64_t& k, int& p, bool up) {
  const uint64_t o = xchg64<S>(k);
  const int op = xchg<S>(p);
  const bool lower = (lane_id() & S) == 0;
  const bool take = (lower == up) ? (o < k) : (k < o);
  k = take ? o : k;
  p = take ? op : p;
}
// list (ascending, with payload) := the 64 smallest of list U cand (cand
// ascending, entering with payload cp).
__device__ __forceinline__ void wave_merge_sorted64_kp(uint64_t& k, int& p, uint64_t cand, int cp) {
  const uint64_t r = wave_reverse64(cand);
  const int rp = wave_reverse(cp);
  if (r < k) {
    k = r;
    p = rp;
  }
  bitonic_stage_kp<32>(k, p, true);
  bitonic_stage_kp<16>(k, p, true);
  bitonic_stage_kp<8>(k, p, true);
  bitonic_stage_kp<4>(k, p, true);
  bitonic_stage_kp<2>(k, p, true);
  bitonic_stage_kp<1>(k, p, true);
}

// Insert nk into the ascending list; the last entry drops off.
__device__ __forceinline__ void wave_insert64_k(uint64_t& k, uint64_t nk) {
  const uint64_t p = dpp_mov64<0x138>(k);  // wave_shr:1: lane i gets lane i-1
  if (!(k < nk)) k = (lane_id() == 0 || p < nk) ? nk : p;
}

__device__ __forceinline__ float wave_min_f(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = fminf(v, shfl_xor_f(v, m));
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, shfl_xor_f(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += shfl_xor_f(v, m);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += shfl_xor_i(v, m);
  return v;
}

// Exact squared L2 in the reference's device form: sequential fused
// multiply-add over dimensions (tune_parameters.cu:39-46 built by nvcc).
__device__ __forceinline__ float l2_fma(const float* __restrict__ a, const float* __restrict__ b, int d) {
  float acc = 0.0f;
  for (int i = 0; i < d; ++i) {
    float diff = a[i] - b[i];
    acc = __builtin_fmaf(diff, diff, acc);
  }
  return acc;
}

}  // namespace fgpu
