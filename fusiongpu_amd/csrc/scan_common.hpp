// scan_common.hpp -- device building blocks shared by the ADC scan kernels
// (adc.hip, twophase.hip): per-(query, list) LUT entries in the reference's
// exact op order, 128-bit code loads, the sequential ADC chain with exact
// early abandon, and the wave-level top-k offer.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {

constexpr int kSerialMax = 12;  // passers up to this count are inserted one by one

template <int D, int M>
struct Cfg {
  static constexpr int S = D / M;
  static constexpr int LUT = M * kPQK;  // floats per LUT
  static constexpr bool DBUF = 2 * LUT * 4 <= 65536;  // both LUTs within the DS immediate-offset reach
  static constexpr int NBUF = DBUF ? 2 : 1;
  static constexpr int R_OFF = NBUF * LUT;      // residual double buffer [2][D]
  static constexpr int Q_OFF = R_OFF + 2 * D;   // query [D]
  static constexpr int SMEM = Q_OFF + D;
  static constexpr int NV4 = M / 16;            // 128-bit code loads per vector
  static_assert(D % M == 0, "dim must be a multiple of pq_m");
  static_assert(M % 16 == 0, "pq_m must be a multiple of 16");
  static_assert(LUT >= 2 * 8 * kWave, "merge area must fit in the LUT area");
};

template <int S>
__device__ __forceinline__ float lut_entry(const float* r, const float* p) {
  if constexpr (S == 4) {
    const float dx = r[0] - p[0], dy = r[1] - p[1], dz = r[2] - p[2], dw = r[3] - p[3];
    return __builtin_fmaf(dx, dx, __builtin_fmaf(dy, dy, __builtin_fmaf(dz, dz, dw * dw)));
  } else if constexpr (S == 8) {
    const float x1 = r[0] - p[0], y1 = r[1] - p[1], z1 = r[2] - p[2], w1 = r[3] - p[3];
    const float x2 = r[4] - p[4], y2 = r[5] - p[5], z2 = r[6] - p[6], w2 = r[7] - p[7];
    const float d = __builtin_fmaf(x1, x1, __builtin_fmaf(y1, y1, __builtin_fmaf(z1, z1, w1 * w1)));
    return __builtin_fmaf(x2, x2, __builtin_fmaf(y2, y2, __builtin_fmaf(z2, z2, __builtin_fmaf(w2, w2, d))));
  } else {
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const float df = r[j] - p[j];
      d = __builtin_fmaf(df, df, d);
    }
    return d;
  }
}

template <int M>
__device__ __forceinline__ void load_codes(const uint8_t* __restrict__ codes, int64_t vec, uint4 (&w)[M / 16]) {
  const uint4* p = reinterpret_cast<const uint4*>(codes + vec * M);
#pragma unroll
  for (int i = 0; i < M / 16; ++i) w[i] = p[i];
}

template <int M>
__device__ __forceinline__ float adc_sum(const float* __restrict__ lut, const uint4 (&w)[M / 16]) {
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < M / 16; ++i) {
    const uint32_t ws[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t code = (ws[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      d += lut[(i * 16 + j) * kPQK + code];
    }
  }
  return d;
}

// Two ADC chains at once, interleaved so each wave keeps twice as many LDS
// gathers in flight.  Each chain is still the sequential sum over ascending m.
// Lanes past the end of a list run on stale codes: every byte value indexes
// inside the LUT, and the caller masks those results.
//
// Early abandon: every term is a sum of squares (>= +0), and adding a
// non-negative float never lowers a rounded sum, so a partial sum already above
// thr_d bounds the final distance from below.  After each group of 8
// subspaces, if no valid lane of either chain is still <= thr_d, the wave
// stops: none of its vectors can enter the top-k (a vector equal to thr_d
// could still win on its id, so equality keeps a lane alive).  Returns false
// in that case; otherwise d0/d1 are the complete, exact distances.
template <int M>
__device__ __forceinline__ bool adc_sum2(const float* __restrict__ lut, const uint4 (&w0)[M / 16],
                                         const uint4 (&w1)[M / 16], bool ok0, bool ok1, float thr_d, float& d0,
                                         float& d1) {
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < M / 16; ++i) {
    const uint32_t x[4] = {w0[i].x, w0[i].y, w0[i].z, w0[i].w};
    const uint32_t y[4] = {w1[i].x, w1[i].y, w1[i].z, w1[i].w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t cx = (x[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      const uint32_t cy = (y[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      a += lut[(i * 16 + j) * kPQK + cx];
      b += lut[(i * 16 + j) * kPQK + cy];
      if ((j & 7) == 7 && i * 16 + j + 1 < M) {
        if (!__ballot((ok0 && a <= thr_d) || (ok1 && b <= thr_d))) return false;
      }
    }
  }
  d0 = a;
  d1 = b;
  return true;
}

// The ADC distances of the two vectors of a scanner round, every term.  A
// wave-wide early abandon of a 128-vector round almost never fires against a
// top-k threshold (C2 plain search: none of 325 k rounds stopped at any
// checkpoint; C3 phase 1: 0.02% of 2.1 M), so such rounds pay no per-lane
// bound tests.  Each group of 8 subspaces still ends in
// a branch, on a uniform test that never holds (thr is a distance, >= 0): the
// branches keep the code in the regions the register allocator fits into the
// 128-VGPR budget of a 16-wave workgroup.  The first term starts each sum
// (0 + t == t for the non-negative LUT entries).
template <int M>
__device__ __forceinline__ bool adc_sum2_full(const float* __restrict__ lut, const uint4 (&w0)[M / 16],
                                              const uint4 (&w1)[M / 16], float thr, float& d0, float& d1) {
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < M / 16; ++i) {
    const uint32_t x[4] = {w0[i].x, w0[i].y, w0[i].z, w0[i].w};
    const uint32_t y[4] = {w1[i].x, w1[i].y, w1[i].z, w1[i].w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t cx = (x[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      const uint32_t cy = (y[j >> 2] >> (8 * (j & 3))) & 0xFFu;
      const float ta = lut[(i * 16 + j) * kPQK + cx], tb = lut[(i * 16 + j) * kPQK + cy];
      if (i == 0 && j == 0) {
        a = ta;
        b = tb;
      } else {
        a += ta;
        b += tb;
      }
      if ((j & 7) == 7 && i * 16 + j + 1 < M && thr < 0.0f) return false;
    }
  }
  d0 = a;
  d1 = b;
  return true;
}

// The same sums for a list's partial last chunk: each chain's gathers run
// only in the lanes that hold a vector (ok0 / ok1), so the empty lanes send
// no LDS requests; their results are FLT_MAX and the caller masks them.
// Same order of terms as adc_sum2_full.
template <int M>
__device__ __forceinline__ void adc_sum2_part(const float* __restrict__ lut, const uint4 (&w0)[M / 16],
                                              const uint4 (&w1)[M / 16], bool ok0, bool ok1, float& d0,
                                              float& d1) {
  float a = FLT_MAX, b = FLT_MAX;
  if (ok0) {
#pragma unroll
    for (int i = 0; i < M / 16; ++i) {
      const uint32_t x[4] = {w0[i].x, w0[i].y, w0[i].z, w0[i].w};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float t = lut[(i * 16 + j) * kPQK + ((x[j >> 2] >> (8 * (j & 3))) & 0xFFu)];
        a = (i == 0 && j == 0) ? t : a + t;
      }
    }
  }
  if (ok1) {
#pragma unroll
    for (int i = 0; i < M / 16; ++i) {
      const uint32_t y[4] = {w1[i].x, w1[i].y, w1[i].z, w1[i].w};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float t = lut[(i * 16 + j) * kPQK + ((y[j >> 2] >> (8 * (j & 3))) & 0xFFu)];
        b = (i == 0 && j == 0) ? t : b + t;
      }
    }
  }
  d0 = a;
  d1 = b;
}

// "No threshold yet": the padding key (FLT_MAX, kPadId); every real
// candidate key (key_of: distances are sums of squares, never negative) is
// below it.
constexpr uint64_t kNoThr = kPadKey;

// Offer one packed (distance, id) key per lane to the wave's running top-64
// list lk (ascending keys); only keys strictly below `thr` (the k-th best
// known to the workgroup) enter.  Returns true if the list changed.
__device__ __forceinline__ bool offer_k(uint64_t key, bool valid, uint64_t thr, uint64_t& lk) {
  const bool pass = valid && key < thr;
  uint64_t bm = __ballot(pass);
  if (!bm) return false;
  if (__popcll(bm) > kSerialMax) {
    uint64_t c = pass ? key : kPadKey;
    wave_sort64_k(c);
    wave_merge_sorted64_k(lk, c);
  } else {
    while (bm) {
      const int src = __ffsll((unsigned long long)bm) - 1;
      bm &= bm - 1;
      wave_insert64_k(lk, readlane64(key, src));
    }
  }
  return true;
}

// Offer a round's two keys per lane (kPadKey for an invalid vector) to the
// running list lk; `kk` is the rank whose key bounds later candidates.  Few
// passers are inserted one by one.  Many passers (the first round of a list
// or query) are split per lane into the smaller and the larger key: the 64
// smaller ones are sorted and merged in (taken as they are when lk is still
// empty), and only the larger keys below the updated kk-th key follow.  For
// kk much below 64 almost none do, so a first round costs one 64-lane sort.
// Returns true if lk changed.
__device__ __forceinline__ bool offer2_k(uint64_t k0, uint64_t k1, uint64_t thr, int kk, uint64_t& lk) {
  const bool p0 = k0 < thr, p1 = k1 < thr;
  uint64_t b0 = __ballot(p0), b1 = __ballot(p1);
  const int c = __popcll(b0) + __popcll(b1);
  if (c == 0) return false;
  if (c <= kSerialMax) {
    while (b0) {
      const int src = __ffsll((unsigned long long)b0) - 1;
      b0 &= b0 - 1;
      wave_insert64_k(lk, readlane64(k0, src));
    }
    while (b1) {
      const int src = __ffsll((unsigned long long)b1) - 1;
      b1 &= b1 - 1;
      wave_insert64_k(lk, readlane64(k1, src));
    }
    return true;
  }
  const uint64_t a = p0 ? k0 : kPadKey, b = p1 ? k1 : kPadKey;
  uint64_t lo = a < b ? a : b;
  const uint64_t hi = a < b ? b : a;
  wave_sort64_k(lo);
  if (readlane64(lk, 0) == kPadKey)
    lk = lo;  // an empty list: the sorted keys are the list
  else
    wave_merge_sorted64_k(lk, lo);
  const uint64_t kth = readlane64(lk, kk - 1);
  offer_k(hi, true, kth < thr ? kth : thr, lk);
  return true;
}

// Each scanning wave takes 128 consecutive vectors per round (two per lane).
constexpr int kVecPerWaveRound = 2 * kWave;

// Codes and vector ids of this lane's two vectors of a round (ids come along
// so the top-k filter never waits on a dependent load).
template <int M>
__device__ __forceinline__ void load_pair(const uint8_t* __restrict__ codes, const int32_t* __restrict__ ids, int start,
                                          int n, int v0, uint4 (&w0)[M / 16], uint4 (&w1)[M / 16], int& i0, int& i1) {
  if (v0 < n) { load_codes<M>(codes, (int64_t)start + v0, w0); i0 = ids[start + v0]; }
  if (v0 + kWave < n) { load_codes<M>(codes, (int64_t)start + v0 + kWave, w1); i1 = ids[start + v0 + kWave]; }
}


// Inclusive prefix sum across the wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int t = __shfl_up(v, o, kWave);
    if (lane >= o) v += t;
  }
  return v;
}

// Lower bound on every ADC distance of a list, from s2 = a float sum of the
// squared residual coordinates r = fl(q - c) (the residual the LUT is built
// from) and rl >= the norm of any decoded residual of the list.
//   * The LUT entries and their ascending sum are chains of at most
//     D/M + 2 + M <= 68 correctly rounded steps on non-negative terms (M <= 64),
//     so the computed ADC distance is at least (1 - 2^-17) ||r - p||^2 for the
//     decoded residual p; and ||r - p|| >= ||r|| - ||p|| >= ||r|| - rl.
//   * s2 is within 129 u of ||r||^2 (D <= 128), so
//     fl(sqrt(fl(s2 (1 - 2^-14)))) <= ||r||.
//   * The returned value carries one more factor (1 - 2^-14); with the four
//     roundings of the subtraction, the square and that product it stays
//     below (1 - 2^-14 + 4u) (||r|| - rl)^2 < (1 - 2^-17) (||r|| - rl)^2, so it
//     is strictly below the computed distance of every vector in the list
//     whenever it is > 0.
__device__ __forceinline__ float list_lower_bound(float s2, float rl) {
  const float nr = sqrtf(s2 * (1.0f - 0x1p-14f));
  const float gap = nr - rl;
  return gap > 0.0f ? gap * gap * (1.0f - 0x1p-14f) : 0.0f;
}

}  // namespace fgpu
