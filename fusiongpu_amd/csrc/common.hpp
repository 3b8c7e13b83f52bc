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

// Orders one wave's LDS writes before its later LDS reads (and the reads
// before later writes) when lanes exchange data through LDS.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- exact L2 of random rows, one row per lane, loaded eight lanes a row ------
// A load instruction in which every lane reads its own row touches 64 rows in
// 64 places; over a 3.8 GB array (10 M rows of 384 bytes) such loads read
// 1.66 TB/s, against 6.1 TB/s when eight lanes share a row (each lane 16 bytes
// of one 128-byte line, 8 rows an instruction).  So the wave loads its 64 rows
// the second way and hands each 128-byte line through its LDS buffer `tr` to
// the lane that owns the row, which then runs the sequential chain
// acc = fma(q[d] - x[d], q[d] - x[d], acc) over d = 0, 1, ..., D-1, the same
// operations in the same order as a lane reading its row itself.
// Keeps the compiler from moving the wave's LDS accesses across this point.
// The LDS carries out one wave's accesses in issue order, so a read after it
// sees what every lane wrote before it.  (A wavefront-scope fence would do the
// same but also pins the caller's private arrays in scratch memory.)
__device__ __forceinline__ void wave_lds_order() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

constexpr int kRowTrStride = 36;  // floats a row in `tr`: 32 + 4 pad, so b128 reads down the rows spread over the banks
// Floats of a wave's `tr` buffer when RX rows (64 or 32) change hands a round.
template <int RX = kWave>
constexpr int row_tr_floats() { return RX * kRowTrStride; }

// Called by the whole wave.  `row` is the lane's row index into base[][D];
// every lane must pass one inside the array.  `qs` is the query (D floats) in
// LDS; `tr` is the wave's buffer of row_tr_floats<RX>() floats, 16-byte
// aligned.  RX = 32 halves the buffer: each line then changes hands in two
// rounds, rows 0-31 and rows 32-63.  The loads go in batches of up to LB
// lines (LB = D / 32: all of them in one memory round trip, 8 LB float4
// registers a lane).
template <int D, int RX = kWave, int LBATCH = D / 32>
__device__ __forceinline__ float wave_rows_l2(const float* __restrict__ base, int row, const float* qs, float* tr) {
  static_assert(D % 32 == 0, "rows must be whole 128-byte lines");
  static_assert(RX == 64 || RX == 32, "64 or 32 rows a round");
  static_assert(LBATCH >= 1, "at least a line a batch");
  constexpr int L = D / 32;       // 128-byte lines a row
  constexpr int LB = LBATCH < L ? LBATCH : L;
  constexpr int NR = kWave / RX;  // rounds a line
  constexpr int IR = 8 / NR;      // load registers a round (each 8 rows)
  const int lane = lane_id(), sub = lane & 7, r8 = lane >> 3;
  float acc = 0.0f;
#pragma unroll
  for (int b = 0; b < (L + LB - 1) / LB; ++b) {
    // The row index passes through an empty asm so that these loads stay
    // after the earlier LDS hand-overs (loads hoisted above them would hold
    // twice the registers).
    asm volatile("" : "+v"(row));
    // v[8 p + i]: 16 bytes (sub) of line LB b + p of row 8 i + r8.
    float4 v[LB * 8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rv = __shfl(row, 8 * i + r8, kWave);
      const float4* rp = reinterpret_cast<const float4*>(base + (size_t)rv * D) + 8 * LB * b + sub;
#pragma unroll
      for (int p = 0; p < LB; ++p)
        if (LB * b + p < L) v[8 * p + i] = rp[8 * p];
    }
    // Every load of the batch issued before its first exchange: without these
    // empty uses the compiler places each line's loads just before its
    // exchange, one memory round trip a line.
#pragma unroll
    for (int k = 0; k < LB * 8; ++k)
      if (LB * b + k / 8 < L) asm volatile("" ::"v"(v[k].x), "v"(v[k].y), "v"(v[k].z), "v"(v[k].w));
#pragma unroll
    for (int p = 0; p < LB; ++p) {
      if (LB * b + p >= L) break;
      float4 w[8];  // this line of the lane's row
#pragma unroll
      for (int h = 0; h < NR; ++h) {
#pragma unroll
        for (int i = 0; i < IR; ++i)
          *reinterpret_cast<float4*>(tr + (8 * i + r8) * kRowTrStride + 4 * sub) = v[8 * p + IR * h + i];
        wave_lds_order();
        if (NR == 1 || (lane >> 5) == h) {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            w[j] = *reinterpret_cast<const float4*>(tr + (lane % RX) * kRowTrStride + 4 * j);
        }
        wave_lds_order();
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float* qd = qs + 32 * (LB * b + p) + 4 * j;
        float df = qd[0] - w[j].x;
        acc = __builtin_fmaf(df, df, acc);
        df = qd[1] - w[j].y;
        acc = __builtin_fmaf(df, df, acc);
        df = qd[2] - w[j].z;
        acc = __builtin_fmaf(df, df, acc);
        df = qd[3] - w[j].w;
        acc = __builtin_fmaf(df, df, acc);
      }
      // The line's chain done here: left to the scheduler, the chains sink
      // below the later lines' hand-overs and every line stays live.
      asm volatile("" : "+v"(acc));
    }
  }
  return acc;
}

}  // namespace fgpu
