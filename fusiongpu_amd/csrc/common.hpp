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

// Tie rule: ascending distance, then ascending id.
__device__ __forceinline__ bool lt_pair(float da, int ia, float db, int ib) {
  return da < db || (da == db && ia < ib);
}

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

// Bitonic sort of one (d, id) pair per lane across the wave, ascending by the tie rule.
__device__ __forceinline__ void wave_sort64(float& d, int& id) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      float od = shfl_xor_f(d, stride);
      int oi = shfl_xor_i(id, stride);
      const bool up = (lane & size) == 0 || size == kWave;
      const bool lower = (lane & stride) == 0;
      const bool other_less = lt_pair(od, oi, d, id);
      const bool take = (lower == up) ? other_less : (!other_less && !(od == d && oi == id));
      if (take) { d = od; id = oi; }
    }
  }
}

// Bitonic merge (ascending) of a bitonic sequence held one pair per lane.
__device__ __forceinline__ void wave_bitonic_merge64(float& d, int& id) {
  const int lane = lane_id();
#pragma unroll
  for (int stride = kWave >> 1; stride > 0; stride >>= 1) {
    float od = shfl_xor_f(d, stride);
    int oi = shfl_xor_i(id, stride);
    const bool lower = (lane & stride) == 0;
    const bool other_less = lt_pair(od, oi, d, id);
    const bool take = lower ? other_less : (!other_less && !(od == d && oi == id));
    if (take) { d = od; id = oi; }
  }
}

// list (ascending) := the 64 smallest of list U cand, where cand is ascending too.
__device__ __forceinline__ void wave_merge_sorted64(float& d, int& id, float cd, int ci) {
  const int lane = lane_id();
  const float rd = __shfl(cd, kWave - 1 - lane, kWave);
  const int ri = __shfl(ci, kWave - 1 - lane, kWave);
  if (lt_pair(rd, ri, d, id)) { d = rd; id = ri; }
  wave_bitonic_merge64(d, id);
}

// Insert one (nd, nid) into the ascending list (one pair per lane); the last entry drops off.
__device__ __forceinline__ void wave_insert64(float& d, int& id, float nd, int nid) {
  const int lane = lane_id();
  float pd = __shfl_up(d, 1, kWave);
  int pi = __shfl_up(id, 1, kWave);
  if (!lt_pair(d, id, nd, nid)) {
    if (lane == 0 || lt_pair(pd, pi, nd, nid)) { d = nd; id = nid; }
    else { d = pd; id = pi; }
  }
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

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
