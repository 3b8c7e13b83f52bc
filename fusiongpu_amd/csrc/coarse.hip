// coarse.hip -- exact nearest-centroid selection for the coarse quantizer
// (A2), the k-means assignment (A13) and exact kNN (A18).
//
// The reference ranks centroids with cuVS CAGRA (search_pipeline.cu:341) and
// assigns k-means points with a cuBLAS -2*X*C^T GEMM plus norms
// (kmeans_gpu.cuh:197-229).  Here the dense contraction runs on the MFMA
// units (v_mfma_f32_32x32x2f32), producing an estimate
//     est = ||x||^2 + ||c||^2 - 2<x,c>
// whose error against the exact device-form distance (a sequential fused
// multiply-add over dimensions, tune_parameters.cu:39-46) is bounded by
//     |est - exact| <= E = kappa * (||x||^2 + max_c ||c||^2),
//     kappa = 8 * gamma(2*dim + 8),  gamma(n) = n*u / (1 - n*u),  u = 2^-24
// (standard forward error bounds for dot products in any summation order,
// with a factor 2 of slack).  For dim % 32 == 0 the contraction runs on the
// bf16 MFMA units instead, with each operand split as v = hi + lo + e, hi and
// lo bf16 and |e| <= 2^-14 |v| (two faithful bf16 roundings), and
// <x,c> ~ hi_x.hi_c + hi_x.lo_c + lo_x.hi_c: the three products of bf16
// values are exact in fp32, and the dropped terms add at most
// 3.1 * 2^-14 * sum|x_k c_k| <= 1.55 * 2^-14 (||x||^2 + ||c||^2) to the dot
// product, so that kappa gains 4 * 2^-14 and the fp32 sum runs over 3*dim
// products (kappa = 8 gamma(3 dim + 8) + 4 * 2^-14).  With T the p-th smallest estimate, every column
// of the exact top-p has est <= T + 2E, so re-scoring exactly that superset
// and sorting by (exact distance, index) yields the exact answer with the tie
// rule, independent of the GEMM's summation order.
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>

namespace fgpu {

typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace {

constexpr int kTM = 64, kTN = 64, kTK = 32, kLdsStride = 96;

__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__global__ __launch_bounds__(256) void row_norms_kernel(const float* __restrict__ x, int64_t n, int dim,
                                                        float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const float* r = x + row * dim;
  float s = 0.0f;
  for (int d = lane; d < dim; d += kWave) s = __builtin_fmaf(r[d], r[d], s);
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) s += __shfl_xor(s, m, kWave);
  if (lane == 0) out[row] = s;
}

__global__ __launch_bounds__(1024) void max_reduce_kernel(const float* __restrict__ v, int64_t n,
                                                          float* __restrict__ out) {
  __shared__ float part[16];
  float m = -FLT_MAX;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, v[i]);
  m = wave_max_f(m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x < 64) {
    float t = threadIdx.x < (blockDim.x >> 6) ? part[threadIdx.x] : -FLT_MAX;
    t = wave_max_f(t);
    if (threadIdx.x == 0) *out = t;
  }
}

// fp16 lower bounds of the estimates (the select's input): the largest fp16
// value <= v (round to nearest, then one step toward -inf when that rounded
// up; above the fp16 range this is 65504, below it -inf).
__device__ __forceinline__ uint16_t half_at_or_below(float v) {
  const _Float16 h = (_Float16)v;
  uint16_t u = __builtin_bit_cast(uint16_t, h);
  if ((float)h > v) u = (u & 0x8000u) ? (uint16_t)(u + 1u) : (uint16_t)(u - 1u);
  return u;
}
__device__ __forceinline__ float half_bits_float(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
// The smallest fp16 value above the fp16 value f (+inf and NaN stay).
__device__ __forceinline__ float half_next_up(float f) {
  uint16_t u = __builtin_bit_cast(uint16_t, (_Float16)f);
  if ((u & 0x7C00u) == 0x7C00u && !(u & 0x8000u)) return f;  // +inf, NaN
  if ((u & 0x7FFFu) == 0) u = 1u;                            // +-0 -> smallest subnormal
  else u = (u & 0x8000u) ? (uint16_t)(u - 1u) : (uint16_t)(u + 1u);
  return half_bits_float(u);
}

// The fp16 estimates of a row are scaled by 2^-s so that they stay inside the
// fp16 range: |cn_j - 2 <x, c_j>| <= ||x||^2 + 2 max ||c||^2 = t/2 with
// t = 2 (xn + cn_max) < 2^e, so 2^-s with s = max(0, e - 15) keeps every
// shifted estimate (plus its small error) below 2^15.  A power-of-two scale is
// exact in fp32 (a product that falls below the fp32 normal range rounds by
// less than 2^-126, far inside the select's margin at any s > 0), so the
// scaled fp16 values stay lower bounds of the scaled estimates; the select
// scales its margin the same way.  xn is the row's fp32 sum of squares as
// the GEMM forms it; every workgroup of a row forms it alike, so they agree on
// s, and the select reads the s the row's first column tile stores.
__device__ __forceinline__ int est_shift(float xn, float cn_max) {
  const float t = 2.0f * (xn + cn_max);
  if (!(t < 0x1p120f)) return 110;  // inf or NaN inputs: any scale
  int e = 0;
  (void)frexpf(t, &e);  // t = m 2^e, m in [0.5, 1) (e = 0 for t = 0)
  return e > 15 ? e - 15 : 0;
}
__device__ __forceinline__ float pow2_neg(int s) { return __int_as_float((127 - s) << 23); }  // 2^-s, 0 <= s <= 126

// The row shifts (one byte a row) of an fp16 estimate block of nrows rows:
// stored after the estimates, inside the block's float-sized allocation.
__host__ __device__ __forceinline__ uint8_t* est_row_shift(void* est, int64_t nrows, int64_t ld) {
  return reinterpret_cast<uint8_t*>(static_cast<uint16_t*>(est) + nrows * ld);
}

// Where an estimate tile goes (output mode OM).  kOutFull: fp32
// xn[i] + cn[j] - 2 <x_i, c_j>.  kOutShift: fp32 cn[j] - 2 <x_i, c_j>, the row
// shifted by its norm (xn unused).  kOutHalf: the fp16 lower bound (bit
// pattern) of the shifted value times the row's 2^-s (sc).
constexpr int kOutFull = 0, kOutShift = 1, kOutHalf = 2;
template <int OM>
__device__ __forceinline__ void put_est(void* est, int64_t off, const float* xn, int64_t i, float cj, float acc,
                                        float sc = 1.0f) {
  if constexpr (OM == kOutHalf)
    static_cast<uint16_t*>(est)[off] = half_at_or_below((cj - 2.0f * acc) * sc);
  else if constexpr (OM == kOutShift)
    static_cast<float*>(est)[off] = cj - 2.0f * acc;
  else
    static_cast<float*>(est)[off] = (xn[i] + cj) - 2.0f * acc;
}

// 64x64 output tile per workgroup, 4 waves each owning a 32x32 quadrant.
// Operand tiles are staged k-major in LDS with a 96-float row stride, so the
// MFMA operand reads (lanes 0-31: k, lanes 32-63: k+1) and the staging writes
// (one row per lane) both hit distinct banks.
template <int OM>
__global__ __launch_bounds__(256) void gemm_est_kernel(const float* __restrict__ x, int64_t nrows,
                                                       const float* __restrict__ c, int ncols, int dim,
                                                       const float* __restrict__ xn,
                                                       const float* __restrict__ cn,
                                                       void* __restrict__ est, int64_t ld,
                                                       const float* __restrict__ cn_max,
                                                       uint8_t* __restrict__ rsh) {
  __shared__ float As[kTK][kLdsStride];
  __shared__ float Bs[kTK][kLdsStride];
  __shared__ float sq_s[4][64];  // kOutHalf: each wave's part of each tile row's sum of squares
  __shared__ float sc_s[64];     // kOutHalf: each tile row's 2^-s
  float sq = 0.0f;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kTM;
  const int col0 = blockIdx.y * kTN;
  const int wr = wave >> 1, wc = wave & 1;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

  const int64_t ar = row0 + lane;
  const int bc = col0 + lane;
  for (int k0 = 0; k0 < dim; k0 += kTK) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kk = wave * 8 + j * 4;
      float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
      if (k0 + kk < dim) {
        if (ar < nrows) va = *reinterpret_cast<const float4*>(x + ar * dim + k0 + kk);
        if (bc < ncols) vb = *reinterpret_cast<const float4*>(c + (int64_t)bc * dim + k0 + kk);
      }
      if constexpr (OM == kOutHalf) sq += va.x * va.x + va.y * va.y + va.z * va.z + va.w * va.w;
      As[kk + 0][lane] = va.x; As[kk + 1][lane] = va.y; As[kk + 2][lane] = va.z; As[kk + 3][lane] = va.w;
      Bs[kk + 0][lane] = vb.x; Bs[kk + 1][lane] = vb.y; Bs[kk + 2][lane] = vb.z; Bs[kk + 3][lane] = vb.w;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kTK; kk += 2) {
      const float a = As[kk + (lane >> 5)][wr * 32 + (lane & 31)];
      const float b = Bs[kk + (lane >> 5)][wc * 32 + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
    __syncthreads();
  }
  if constexpr (OM == kOutHalf) {
    sq_s[wave][lane] = sq;
    __syncthreads();
    if (wave == 0) {
      const int sh = est_shift(sq_s[0][lane] + sq_s[1][lane] + sq_s[2][lane] + sq_s[3][lane], *cn_max);
      sc_s[lane] = pow2_neg(sh);
      if (blockIdx.y == 0 && ar < nrows) rsh[ar] = (uint8_t)sh;
    }
    __syncthreads();
  }
  // D layout of v_mfma_f32_32x32x2f32: lane l, accumulator r holds
  // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  const int j = col0 + wc * 32 + (lane & 31);
  if (j >= ncols) return;
  const float cj = cn[j];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int rr = wr * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    const int64_t i = row0 + rr;
    if (i < nrows) put_est<OM>(est, i * ld + j, xn, i, cj, acc[r], OM == kOutHalf ? sc_s[rr] : 1.0f);
  }
}

// The estimate for dim % 32 == 0 on v_mfma_f32_32x32x16_bf16 with the
// hi/lo split above (three MFMAs a k-step: hi.hi, hi.lo, lo.hi).  Same grid
// and 64x64 tile as gemm_est_kernel.  Each K stage of 32 is staged with
// coalesced 16-byte loads (a thread loads rows t / 8 and t / 8 + 32 at float4
// t % 8: eight rows of 128 bytes an instruction), the next stage's loads are
// in flight while the current stage's MFMAs run, and the two LDS buffers take
// turns, so one barrier a stage.  A stage is split into bf16 hi/lo while it
// is written to LDS, one staged row = 32 hi, 32 lo and 8 pad bf16 (144 bytes,
// an odd multiple of 16: the 16-byte operand reads of 16 consecutive rows hit
// distinct banks).  MFMA s of a stage contracts k = 16 s + 8 h + e (lane half
// h, element e) for A and B alike.  Rows and columns past the end are loaded
// clamped to the last one and never written.  The tile leaves through LDS
// (stride 72 floats: a store's two row segments hit distinct banks) so that
// each thread writes four float4 rows of it instead of sixteen scattered
// floats.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
constexpr int kB3Row = 72;
constexpr int kCStride = 72;
// The select reads fp16 lower bounds of the shifted estimates (true) or the
// fp32 values themselves (false).  Measured on C2: the same select time,
// and the fp16 form's GEMM writes half the bytes (20.1 against 21.8 us).
constexpr bool kEstHalf = true;  // 64 x 72 floats = 18 KB, inside the 36 KB of operand buffers

__device__ __forceinline__ void split_put(__bf16* row, int sf, const float4 v) {
  bf16x4 h, l;
  h[0] = (__bf16)v.x; h[1] = (__bf16)v.y; h[2] = (__bf16)v.z; h[3] = (__bf16)v.w;
  l[0] = (__bf16)(v.x - (float)h[0]);
  l[1] = (__bf16)(v.y - (float)h[1]);
  l[2] = (__bf16)(v.z - (float)h[2]);
  l[3] = (__bf16)(v.w - (float)h[3]);
  *reinterpret_cast<bf16x4*>(row + 4 * sf) = h;
  *reinterpret_cast<bf16x4*>(row + 32 + 4 * sf) = l;
}

template <int OM>
__global__ __launch_bounds__(256) void gemm_est_split_kernel(const float* __restrict__ x, int64_t nrows,
                                                             const float* __restrict__ c, int ncols, int dim,
                                                             const float* __restrict__ xn,
                                                             const float* __restrict__ cn,
                                                             void* __restrict__ est, int64_t ld,
                                                             const float* __restrict__ cn_max,
                                                             uint8_t* __restrict__ rsh) {
  __shared__ __align__(16) __bf16 As[2][kTM * kB3Row];
  __shared__ __align__(16) __bf16 Bs[2][kTN * kB3Row];
  __shared__ float sc_s[kTM];  // kOutHalf: each tile row's 2^-s
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kTM;
  const int col0 = blockIdx.y * kTN;
  const int wr = wave >> 1, wc = wave & 1;
  const int li = lane & 31, lh = lane >> 5;
  const int sr = tid >> 3, sf = tid & 7;
  const float* ap0 = x + min(row0 + sr, nrows - 1) * dim + 4 * sf;
  const float* ap1 = x + min(row0 + sr + 32, nrows - 1) * dim + 4 * sf;
  const float* bp0 = c + (int64_t)min(col0 + sr, ncols - 1) * dim + 4 * sf;
  const float* bp1 = c + (int64_t)min(col0 + sr + 32, ncols - 1) * dim + 4 * sf;
  float4 ra0 = *reinterpret_cast<const float4*>(ap0), ra1 = *reinterpret_cast<const float4*>(ap1);
  float4 rb0 = *reinterpret_cast<const float4*>(bp0), rb1 = *reinterpret_cast<const float4*>(bp1);
  // kOutHalf: this thread's part of the sums of squares of rows sr and sr + 32
  float sq0 = 0.0f, sq1 = 0.0f;
  auto add_sq = [&]() {
    if constexpr (OM == kOutHalf) {
      sq0 += ra0.x * ra0.x + ra0.y * ra0.y + ra0.z * ra0.z + ra0.w * ra0.w;
      sq1 += ra1.x * ra1.x + ra1.y * ra1.y + ra1.z * ra1.z + ra1.w * ra1.w;
    }
  };
  add_sq();
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  const int nst = dim / 32;
  split_put(&As[0][sr * kB3Row], sf, ra0);
  split_put(&As[0][(sr + 32) * kB3Row], sf, ra1);
  split_put(&Bs[0][sr * kB3Row], sf, rb0);
  split_put(&Bs[0][(sr + 32) * kB3Row], sf, rb1);
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) {
      const int ko = 32 * (st + 1);
      ra0 = *reinterpret_cast<const float4*>(ap0 + ko);
      ra1 = *reinterpret_cast<const float4*>(ap1 + ko);
      rb0 = *reinterpret_cast<const float4*>(bp0 + ko);
      rb1 = *reinterpret_cast<const float4*>(bp1 + ko);
      add_sq();
    }
    const __bf16* Ar = &As[buf][(wr * 32 + li) * kB3Row + 8 * lh];
    const __bf16* Br = &Bs[buf][(wc * 32 + li) * kB3Row + 8 * lh];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(Ar + 16 * s2);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(Ar + 32 + 16 * s2);
      const bf16x8 bh = *reinterpret_cast<const bf16x8*>(Br + 16 * s2);
      const bf16x8 bl = *reinterpret_cast<const bf16x8*>(Br + 32 + 16 * s2);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
    }
    if (st + 1 < nst) {
      const int nb = buf ^ 1;
      split_put(&As[nb][sr * kB3Row], sf, ra0);
      split_put(&As[nb][(sr + 32) * kB3Row], sf, ra1);
      split_put(&Bs[nb][sr * kB3Row], sf, rb0);
      split_put(&Bs[nb][(sr + 32) * kB3Row], sf, rb1);
    }
    __syncthreads();
  }
  if constexpr (OM == kOutHalf) {
    // the eight threads of a row are consecutive lanes
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
      sq0 += __shfl_xor(sq0, m, kWave);
      sq1 += __shfl_xor(sq1, m, kWave);
    }
    if (sf == 0) {
      const float cm = *cn_max;
      const int s0 = est_shift(sq0, cm), s1 = est_shift(sq1, cm);
      sc_s[sr] = pow2_neg(s0);
      sc_s[sr + 32] = pow2_neg(s1);
      if (blockIdx.y == 0) {
        if (row0 + sr < nrows) rsh[row0 + sr] = (uint8_t)s0;
        if (row0 + sr + 32 < nrows) rsh[row0 + sr + 32] = (uint8_t)s1;
      }
    }
  }
  // acc layout as in gemm_est_kernel; the operand buffers are free after the
  // last barrier.
  float* Cs = reinterpret_cast<float*>(&As[0][0]);
#pragma unroll
  for (int r = 0; r < 16; ++r) Cs[(wr * 32 + 8 * (r >> 2) + 4 * lh + (r & 3)) * kCStride + wc * 32 + li] = acc[r];
  __syncthreads();
  const int c4 = 4 * (tid & 15);
  const int j = col0 + c4;
  if (j >= ncols) return;
  const bool full = j + 3 < ncols;
  float4 cj;
  if (full) {
    cj = *reinterpret_cast<const float4*>(cn + j);
  } else {
    cj.x = cn[j];
    cj.y = j + 1 < ncols ? cn[j + 1] : 0.0f;
    cj.z = j + 2 < ncols ? cn[j + 2] : 0.0f;
    cj.w = 0.0f;
  }
  const bool vec = full && (ld & 3) == 0;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int rr = 16 * it + (tid >> 4);
    const int64_t i = row0 + rr;
    if (i >= nrows) break;
    const float4 a = *reinterpret_cast<const float4*>(&Cs[rr * kCStride + c4]);
    const int64_t off = i * ld + j;
    const float sc = OM == kOutHalf ? sc_s[rr] : 1.0f;
    if (vec) {
      if constexpr (OM == kOutHalf) {
        const uint32_t lo = (uint32_t)half_at_or_below((cj.x - 2.0f * a.x) * sc) |
                            ((uint32_t)half_at_or_below((cj.y - 2.0f * a.y) * sc) << 16);
        const uint32_t hi = (uint32_t)half_at_or_below((cj.z - 2.0f * a.z) * sc) |
                            ((uint32_t)half_at_or_below((cj.w - 2.0f * a.w) * sc) << 16);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(est) + off) = make_uint2(lo, hi);
      } else if constexpr (OM == kOutShift) {
        *reinterpret_cast<float4*>(static_cast<float*>(est) + off) =
            make_float4(cj.x - 2.0f * a.x, cj.y - 2.0f * a.y, cj.z - 2.0f * a.z, cj.w - 2.0f * a.w);
      } else {
        const float xi = xn[i];
        *reinterpret_cast<float4*>(static_cast<float*>(est) + off) =
            make_float4((xi + cj.x) - 2.0f * a.x, (xi + cj.y) - 2.0f * a.y, (xi + cj.z) - 2.0f * a.z,
                        (xi + cj.w) - 2.0f * a.w);
      }
    } else {
      put_est<OM>(est, off, xn, i, cj.x, a.x, sc);
      if (j + 1 < ncols) put_est<OM>(est, off + 1, xn, i, cj.y, a.y, sc);
      if (j + 2 < ncols) put_est<OM>(est, off + 2, xn, i, cj.z, a.z, sc);
      if (j + 3 < ncols) put_est<OM>(est, off + 3, xn, i, cj.w, a.w, sc);
    }
  }
}

// E for one row.  The absolute term covers products and operands below the
// fp32 normal range, which the MFMA units may flush to zero: each such term
// is under 2^-126 times an operand, so all of them together stay far below
// 2^-100 (1 + ||x||^2 + ||c||^2) for any dim up to 2^20.
__device__ __forceinline__ double est_margin(float kappa, float xn, float cn_max) {
  const double nn = (double)xn + (double)cn_max;
  return (double)kappa * nn + 0x1p-100 * (1.0 + nn);
}

constexpr int kCandCap = 512;
constexpr int kSelectMax = 4 * kWave;  // p limit of the coarse select: four sorted 64-key lists

// Which column a lane's value j holds: V = 1, column j*64 + lane; V = 4 or 8
// (a row read as 16-byte vectors), runs of V consecutive columns a lane,
// column (j / V) * 64 V + V lane + j % V.
template <int V>
__device__ __forceinline__ int col_of(int j, int lane) {
  if constexpr (V == 1) return j * kWave + lane;
  else return (j / V) * (kWave * V) + V * lane + (j % V);
}

// The p-th smallest of the wave's estimates val[j] (column col_of<V>(j, lane),
// only columns < ncols count): LDS radix select, 8 bits a pass, over the
// order-preserving integer map of the floats.  p == 1 is a plain minimum.
// For p <= 64 the p-th smallest of the 64 per-lane minima bounds the answer
// from above (those minima are p of the keys), and only keys at or below it
// enter the histograms: the first passes otherwise pile most of the keys into
// one or two bins, whose LDS atomics serialise.
template <int VPL, int V = 1>
__device__ float wave_kth_estimate(const float (&val)[VPL], int ncols, int p, uint32_t* hist) {
  const int lane = threadIdx.x & 63;
  if (p == 1) {
    float m = val[0];
#pragma unroll
    for (int j = 1; j < VPL; ++j) m = fminf(m, val[j]);
    return wave_min_f(m);
  }
  uint32_t key[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) key[j] = (col_of<V>(j, lane) < ncols) ? float_key(val[j]) : 0xFFFFFFFFu;
  uint32_t cap = 0xFFFFFFFFu;
  if (p <= kWave) {
    uint32_t mn = key[0];
#pragma unroll
    for (int j = 1; j < VPL; ++j) mn = key[j] < mn ? key[j] : mn;
    wave_sort_u32(mn);
    cap = (uint32_t)readlane_i((int)mn, p - 1);
    // The keys at or below cap (at least p of them) usually number at most
    // 64: gather them in column order and take the p-th of one sorted wave.
    int n = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const bool f = key[j] <= cap;
      const uint64_t bm = __ballot(f);
      const int pos = n + lanes_below(bm);
      if (f && pos < kWave) hist[pos] = key[j];
      n += __popcll(bm);
    }
    if (n <= kWave) {
      wave_lds_sync();
      uint32_t k = lane < n ? hist[lane] : 0xFFFFFFFFu;
      wave_sort_u32(k);
      const uint32_t t = (uint32_t)readlane_i((int)k, p - 1);
      wave_lds_sync();
      return key_float(t);
    }
    wave_lds_sync();
  }
  uint32_t prefix = 0, mask = 0;
  uint32_t rem = (uint32_t)p;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = lane; b < 256; b += kWave) hist[b] = 0u;
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < VPL; ++j)
      if ((key[j] & mask) == prefix && key[j] <= cap) atomicAdd(&hist[(key[j] >> shift) & 255u], 1u);
    wave_lds_sync();
    const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2],
                   h3 = hist[4 * lane + 3];
    const uint32_t s = h0 + h1 + h2 + h3;
    uint32_t inc = s;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      uint32_t t = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += t;
    }
    const uint32_t exc = inc - s;
    const uint64_t bm = __ballot(exc < rem && rem <= inc);
    const int L = __ffsll((unsigned long long)bm) - 1;
    int bin = 3;
    uint32_t below = exc + h0 + h1 + h2;
    if (rem <= exc + h0) { bin = 0; below = exc; }
    else if (rem <= exc + h0 + h1) { bin = 1; below = exc + h0; }
    else if (rem <= exc + h0 + h1 + h2) { bin = 2; below = exc + h0 + h1; }
    bin = readlane_i(bin, L) + 4 * L;
    below = (uint32_t)readlane_i((int)below, L);
    rem -= below;
    prefix |= (uint32_t)bin << shift;
    mask |= 0xFFu << shift;
    wave_lds_sync();
  }
  return key_float(prefix);
}

// Exact squared L2 of the wave's staged row xs against row cr of c, in the
// reference's device form (sequential fused multiply-add over dimensions).
// The row is read 32 floats at a time, all eight loads issued before the
// first multiply-add (the scheduling barrier keeps them together): one
// memory round trip per 32 dimensions instead of one per few float4.
__device__ __forceinline__ float exact_l2(const float* __restrict__ xs, const float* __restrict__ cr, int dim) {
  float acc = 0.0f;
  if ((dim & 3) == 0) {
    int t = 0;
    for (; t + 32 <= dim; t += 32) {
      float4 cv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) cv[u] = *reinterpret_cast<const float4*>(cr + t + 4 * u);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float4 xv = *reinterpret_cast<const float4*>(xs + t + 4 * u);
        float df = xv.x - cv[u].x; acc = __builtin_fmaf(df, df, acc);
        df = xv.y - cv[u].y; acc = __builtin_fmaf(df, df, acc);
        df = xv.z - cv[u].z; acc = __builtin_fmaf(df, df, acc);
        df = xv.w - cv[u].w; acc = __builtin_fmaf(df, df, acc);
      }
    }
    for (; t < dim; t += 4) {
      const float4 cv = *reinterpret_cast<const float4*>(cr + t);
      const float4 xv = *reinterpret_cast<const float4*>(xs + t);
      float df = xv.x - cv.x; acc = __builtin_fmaf(df, df, acc);
      df = xv.y - cv.y; acc = __builtin_fmaf(df, df, acc);
      df = xv.z - cv.z; acc = __builtin_fmaf(df, df, acc);
      df = xv.w - cv.w; acc = __builtin_fmaf(df, df, acc);
    }
  } else {
    for (int t = 0; t < dim; ++t) {
      const float df = xs[t] - cr[t];
      acc = __builtin_fmaf(df, df, acc);
    }
  }
  return acc;
}

// Merge a sorted batch (ascending, one key a lane) into the running top-4*64
// held as four sorted 64-lists a <= b <= c <= d (ranks 1-64, 65-128, ...):
// each level keeps the 64 smallest of its list and what arrives, and passes
// the 64 largest down; nl lists are live (nl = ceil(p / 64)).
__device__ __forceinline__ void split_merge64(uint64_t& lo, uint64_t& inc) {
  const uint64_t r = wave_reverse64(inc);
  const bool take = r < lo;
  const uint64_t hi = take ? lo : r;
  lo = take ? r : lo;
  inc = hi;
  bitonic_pass_k<64>(lo, true);
  bitonic_pass_k<64>(inc, true);
}
__device__ __forceinline__ void merge_top256(uint64_t (&l)[4], int nl, uint64_t key) {
  if (nl == 1) {
    wave_merge_sorted64_k(l[0], key);
    return;
  }
  split_merge64(l[0], key);
  if (nl == 2) {
    wave_merge_sorted64_k(l[1], key);
    return;
  }
  split_merge64(l[1], key);
  if (nl == 3) {
    wave_merge_sorted64_k(l[2], key);
    return;
  }
  split_merge64(l[2], key);
  wave_merge_sorted64_k(l[3], key);
}

// The largest float <= t: for a float v, v <= t exactly when v <= this.
__device__ __forceinline__ float float_at_or_below(double t) {
  float f = (float)t;
  if ((double)f > t) {
    const uint32_t u = __float_as_uint(f);
    f = __uint_as_float(f > 0.0f ? u - 1u : (f == 0.0f ? 0x80000001u : u + 1u));
  }
  return f;
}

// The select for one row, given its estimates (val[j]: column
// col_of<V>(j, lane), FLT_MAX past ncols; fp16 lower bounds when HALF) and
// its query row xs in LDS: p-th smallest estimate, margin superset, exact
// re-score, bitonic sort by (distance, index); p <= 256.  One wave; hist
// (256 words) and cand (kCandCap ints) are the wave's own LDS.
template <int VPL, int V, bool HALF>
__device__ __forceinline__ void select_row(const float (&val)[VPL], int64_t row, int ncols, const float* xs,
                                           uint32_t* hist, int* cand, const float* __restrict__ c, int dim,
                                           float xnr, const float* __restrict__ cn_max,
                                           float kappa, int p, int prune, float prune_ratio,
                                           int32_t* __restrict__ out_ids, float* __restrict__ out_d, int shift,
                                           unsigned long long* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  // With fp16 lower bounds and T' their p-th smallest, the p smallest
  // estimates lie below the next fp16 value above T' (each is below the next
  // fp16 value above its own bound), so T = that value bounds the p-th
  // smallest estimate from above, and every column whose estimate is
  // <= (p-th smallest estimate) + 2E has val <= T + 2E.
  // The values are the row's estimates times 2^-shift, so is the margin.
  const float Tv = wave_kth_estimate<VPL, V>(val, ncols, p, hist);
  const float T = HALF ? half_next_up(Tv) : Tv;
  const double E = std::ldexp(est_margin(kappa, xnr, *cn_max), -shift);
  const float thr = float_at_or_below((double)T + 2.0 * E);

  // Compaction of the candidate columns.
  int C = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int col = col_of<V>(j, lane);
    const bool f = col < ncols && val[j] <= thr;
    const uint64_t bm = __ballot(f);
    const int pos = C + lanes_below(bm);
    if (f && pos < kCandCap) cand[pos] = col;
    C += __popcll(bm);
  }
  wave_lds_sync();
  const bool all_cols = C > kCandCap;  // pathological ties: re-score everything
  const int ncand = all_cols ? ncols : C;
  if (stats && lane == 0) {  // instrumentation: columns re-scored, rows re-scoring every column
    atomicAdd(&stats[0], (unsigned long long)ncand);
    if (all_cols) atomicAdd(&stats[1], 1ull);
  }

  // Running top-p of packed (distance, id) keys: squared L2 distances are
  // >= 0, so key order is the tie rule.
  const int nl = (p + kWave - 1) / kWave;
  uint64_t lk[4] = {kPadKey, kPadKey, kPadKey, kPadKey};
  bool first = true;
  for (int base = 0; base < ncand; base += kWave) {
    uint64_t key = kPadKey;
    if (base + lane < ncand) {
      const int id = all_cols ? base + lane : cand[base + lane];
      key = key_of(exact_l2(xs, c + (int64_t)id * dim, dim), id);
    }
    wave_sort64_k(key);
    if (first) { lk[0] = key; first = false; }
    else merge_top256(lk, nl, key);
  }

  const float best = key_dist(readlane64(lk[0], 0));
  const float pthr = best * prune_ratio;
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const int r = l * kWave + lane;
    if (r < p) {
      const float ld_ = key_dist(lk[l]);
      int32_t oid = key_id(lk[l]);
      if (prune && ld_ > pthr) oid = (int32_t)kPruned;
      out_ids[row * p + r] = oid;
      out_d[row * p + r] = ld_;
    }
  }
}

// One wave per row over the estimate matrix est (row stride ld).  The
// estimates may leave out the row's own norm (a shift of the whole row: the
// p-th estimate and the candidate set move with it); the margin takes the
// norm computed here, the same lane-strided chain and reduction as
// row_norms_kernel.
template <int VPL, typename E>
__global__ __launch_bounds__(256) void select_exact_kernel(
    const E* __restrict__ est, int64_t ld, int64_t nrows, int ncols,
    const float* __restrict__ x, const float* __restrict__ c, int dim,
    const float* __restrict__ cn_max, float kappa, int p, int prune,
    float prune_ratio, int32_t* __restrict__ out_ids, float* __restrict__ out_d, int* side, int side_val,
    const uint8_t* __restrict__ rsh, unsigned long long* __restrict__ stats) {
  __shared__ uint32_t hist_s[4][256];
  __shared__ int cand_s[4][kCandCap];
  __shared__ __align__(16) float x_s[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (side && blockIdx.x == 0 && threadIdx.x == 0) *side = side_val;  // the caller's one-word side write
  if (row >= nrows) return;  // whole wave leaves; no workgroup barrier follows
  float* xs = x_s[wave];
  float xnr = 0.0f;
  for (int d = lane; d < dim; d += kWave) {
    const float v = x[row * dim + d];
    xs[d] = v;
    xnr = __builtin_fmaf(v, v, xnr);
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) xnr += __shfl_xor(xnr, m, kWave);

  // The row as 16-byte vectors (ld % 8 == 0): runs of V columns a lane.
  constexpr bool HALF = sizeof(E) == 2;
  constexpr int VEC = HALF ? 8 : 4;
  constexpr int V = VPL >= VEC ? VEC : 1;
  auto cvt = [](E e) -> float {
    if constexpr (HALF) return half_bits_float(e);
    else return e;
  };
  float val[VPL];
  const E* er = est + row * ld;
  if constexpr (V > 1) {
#pragma unroll
    for (int jj = 0; jj < VPL / V; ++jj) {
      const int c0 = col_of<V>(jj * V, lane);
      if (c0 + V <= ncols) {
        const uint4 w = *reinterpret_cast<const uint4*>(er + c0);
        const E* e = reinterpret_cast<const E*>(&w);
#pragma unroll
        for (int t = 0; t < V; ++t) val[jj * V + t] = cvt(e[t]);
      } else {
#pragma unroll
        for (int t = 0; t < V; ++t) val[jj * V + t] = c0 + t < ncols ? cvt(er[c0 + t]) : FLT_MAX;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int col = j * kWave + lane;
      val[j] = col < ncols ? cvt(er[col]) : FLT_MAX;
    }
  }
  select_row<VPL, V, HALF>(val, row, ncols, xs, hist_s[wave], cand_s[wave], c, dim, xnr, cn_max, kappa, p, prune,
                           prune_ratio, out_ids, out_d, HALF ? (int)rsh[row] : 0, stats);
}

// p == 1 over many columns (the k-means assignment at k > 1024): the row is
// read twice in pieces of 64 16-byte vectors (its minimum, then the
// compaction) instead of being held whole in registers, so a wave stays
// small and a CU holds many of them (the whole-row form needs 218 VGPRs at
// 4096 columns).  Same margin, candidates and exact re-score as select_row;
// the answer is the smallest (distance, id) key.
__device__ __forceinline__ uint64_t wave_min64(uint64_t k) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(k >> 32), m, kWave) << 32) |
                       (uint32_t)__shfl_xor((int)(uint32_t)k, m, kWave);
    k = o < k ? o : k;
  }
  return k;
}

template <typename E>
__global__ __launch_bounds__(256) void select_min_kernel(
    const E* __restrict__ est, int64_t ld, int64_t nrows, int ncols,
    const float* __restrict__ x, const float* __restrict__ c, int dim,
    const float* __restrict__ cn_max, float kappa, int prune, float prune_ratio,
    int32_t* __restrict__ out_ids, float* __restrict__ out_d, int* side, int side_val,
    const uint8_t* __restrict__ rsh, unsigned long long* __restrict__ stats) {
  __shared__ int cand_s[4][kCandCap];
  __shared__ __align__(16) float x_s[4][256];
  constexpr bool HALF = sizeof(E) == 2;
  constexpr int V = HALF ? 8 : 4;      // elements a 16-byte vector
  constexpr int PIECE = V * kWave;     // columns a piece
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (side && blockIdx.x == 0 && threadIdx.x == 0) *side = side_val;  // the caller's one-word side write
  if (row >= nrows) return;  // whole wave leaves; no workgroup barrier follows
  float* xs = x_s[wave];
  int* cand = cand_s[wave];
  float xnr = 0.0f;
  for (int d = lane; d < dim; d += kWave) {
    const float v = x[row * dim + d];
    xs[d] = v;
    xnr = __builtin_fmaf(v, v, xnr);
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) xnr += __shfl_xor(xnr, m, kWave);
  auto cvt = [](E e) -> float {
    if constexpr (HALF) return half_bits_float(e);
    else return e;
  };
  const E* er = est + row * ld;
  auto load = [&](int c0, float (&v)[V]) {  // columns c0 .. c0 + V - 1 (ld % 8 == 0)
    if (c0 + V <= ncols) {
      const uint4 w = *reinterpret_cast<const uint4*>(er + c0);
      const E* e = reinterpret_cast<const E*>(&w);
#pragma unroll
      for (int t = 0; t < V; ++t) v[t] = cvt(e[t]);
    } else {
#pragma unroll
      for (int t = 0; t < V; ++t) v[t] = c0 + t < ncols ? cvt(er[c0 + t]) : FLT_MAX;
    }
  };
  float mn = FLT_MAX;
  for (int base = 0; base < ncols; base += PIECE) {
    float v[V];
    load(base + V * lane, v);
#pragma unroll
    for (int t = 0; t < V; ++t) mn = fminf(mn, v[t]);
  }
  const float Tv = wave_min_f(mn);
  const float T = HALF ? half_next_up(Tv) : Tv;
  // the values are the row's estimates times 2^-shift, so is the margin
  const int shift = HALF ? (int)rsh[row] : 0;
  const float thr = float_at_or_below((double)T + 2.0 * std::ldexp(est_margin(kappa, xnr, *cn_max), -shift));
  int C = 0;
  for (int base = 0; base < ncols; base += PIECE) {
    float v[V];
    load(base + V * lane, v);
#pragma unroll
    for (int t = 0; t < V; ++t) {
      const int col = base + V * lane + t;
      const bool f = col < ncols && v[t] <= thr;
      const uint64_t bm = __ballot(f);
      const int pos = C + lanes_below(bm);
      if (f && pos < kCandCap) cand[pos] = col;
      C += __popcll(bm);
    }
  }
  wave_lds_sync();
  const bool all_cols = C > kCandCap;  // pathological ties: re-score everything
  const int ncand = all_cols ? ncols : C;
  if (stats && lane == 0) {  // instrumentation: columns re-scored, rows re-scoring every column
    atomicAdd(&stats[0], (unsigned long long)ncand);
    if (all_cols) atomicAdd(&stats[1], 1ull);
  }
  uint64_t best = kPadKey;
  for (int b = 0; b < ncand; b += kWave) {
    if (b + lane < ncand) {
      const int id = all_cols ? b + lane : cand[b + lane];
      const uint64_t key = key_of(exact_l2(xs, c + (int64_t)id * dim, dim), id);
      best = key < best ? key : best;
    }
  }
  best = wave_min64(best);
  if (lane == 0) {
    const float bd = key_dist(best);
    int32_t oid = key_id(best);
    if (prune && bd > bd * prune_ratio) oid = (int32_t)kPruned;
    out_ids[row] = oid;
    out_d[row] = bd;
  }
}

// Exact kNN (brute_force_search_kernel, tune_parameters.cu:49-96) over one
// chunk of base rows, merged into each query's running top-k (k <= 128):
// the running list sits in two sorted 64-lists per wave, A (ranks 1-64) and
// B (ranks 65-128).  Chunk columns carry ids id_base + col, above every id
// of earlier chunks, so the tie rule (distance, id) needs no extra care.
// Candidate superset: est <= min(T + 2E, kth + E), T the min(k, ncols)-th
// estimate of the chunk and kth the running k-th exact distance; the second
// bound alone is tried first once the running list is full, which spares the
// radix select in every chunk after the first.
constexpr int kKnnCap = 512;

template <int VPL>
__global__ __launch_bounds__(256) void knn_chunk_kernel(
    const float* __restrict__ est, int64_t ld, int64_t nrows, int ncols, const float* __restrict__ x,
    const float* __restrict__ c, int dim, const float* __restrict__ xn, const float* __restrict__ cn_max,
    float kappa, int k, int id_base, int accum, int32_t* __restrict__ out_ids, float* __restrict__ out_d) {
  __shared__ uint32_t hist_s[4][256];
  __shared__ int cand_s[4][kKnnCap];
  __shared__ __align__(16) float x_s[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= nrows) return;  // whole wave leaves; no workgroup barrier follows
  uint32_t* hist = hist_s[wave];
  int* cand = cand_s[wave];
  float* xs = x_s[wave];
  for (int d = lane; d < dim; d += kWave) xs[d] = x[row * dim + d];

  // running top-k as packed (distance, id) keys (squared L2 >= 0, so key
  // order is the tie rule)
  uint64_t ak = kPadKey, bk = kPadKey;
  if (accum) {
    if (lane < k) {
      const int id = out_ids[row * k + lane];
      if (id >= 0) ak = key_of(out_d[row * k + lane], id);
    }
    if (lane + kWave < k) {
      const int id = out_ids[row * k + lane + kWave];
      if (id >= 0) bk = key_of(out_d[row * k + lane + kWave], id);
    }
  }
  const uint64_t kk = k <= kWave ? readlane64(ak, k - 1) : readlane64(bk, k - kWave - 1);
  const float kth = key_dist(kk);
  const bool full = key_id(kk) != kPadId;

  float val[VPL];
  const float* er = est + row * ld;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int col = j * kWave + lane;
    val[j] = col < ncols ? er[col] : FLT_MAX;
  }
  const double E = est_margin(kappa, xn[row], *cn_max);
  const int p = k < ncols ? k : ncols;

  // Ordered compaction of the columns with estimate <= thr; the count may exceed the cap.
  auto gather = [&](double thr) {
    int C = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int col = j * kWave + lane;
      const bool f = col < ncols && (double)val[j] <= thr;
      const uint64_t bm = __ballot(f);
      const int pos = C + lanes_below(bm);
      if (f && pos < kKnnCap) cand[pos] = col;
      C += __popcll(bm);
    }
    wave_lds_sync();
    return C;
  };
  double thr = full ? (double)kth + E : 0.0;
  int C = full ? gather(thr) : kKnnCap + 1;
  if (C > kKnnCap) {
    const float T = wave_kth_estimate<VPL>(val, ncols, p, hist);
    const double t2 = (double)T + 2.0 * E;
    thr = full && thr < t2 ? thr : t2;
    C = gather(thr);
  }
  const bool all_cols = C > kKnnCap;  // pathological ties: re-score everything
  const int ncand = all_cols ? ncols : C;

  for (int base = 0; base < ncand; base += kWave) {
    uint64_t key = kPadKey;
    if (base + lane < ncand) {
      const int col = all_cols ? base + lane : cand[base + lane];
      key = key_of(exact_l2(xs, c + (int64_t)col * dim, dim), id_base + col);
    }
    wave_sort64_k(key);
    if (k <= kWave) {
      wave_merge_sorted64_k(ak, key);
    } else {
      // A U C splits into its 64 smallest (new A) and 64 largest (H); B := best 64 of B U H.
      const uint64_t r = wave_reverse64(key);
      const bool c_lo = r < ak;
      const uint64_t hk = c_lo ? ak : r;
      ak = c_lo ? r : ak;
      uint64_t h = hk;
      bitonic_pass_k<64>(ak, true);
      bitonic_pass_k<64>(h, true);
      wave_merge_sorted64_k(bk, h);
    }
  }
  if (lane < k) {
    const int ai = key_id(ak);
    out_ids[row * k + lane] = ai == kPadId ? -1 : ai;
    out_d[row * k + lane] = ai == kPadId ? FLT_MAX : key_dist(ak);
  }
  if (lane + kWave < k) {
    const int bi = key_id(bk);
    out_ids[row * k + lane + kWave] = bi == kPadId ? -1 : bi;
    out_d[row * k + lane + kWave] = bi == kPadId ? FLT_MAX : key_dist(bk);
  }
}

template <int VPL>
fgpu_status launch_knn_t(const float* est, int64_t ld, int64_t nrows, int ncols, const float* x, const float* c,
                         int dim, const float* xn, const float* cn_max, float kappa, int k, int id_base, int accum,
                         int32_t* ids, float* d, hipStream_t s) {
  const int64_t blocks = (nrows + 3) / 4;
  hipLaunchKernelGGL(knn_chunk_kernel<VPL>, dim3((unsigned)blocks), dim3(256), 0, s, est, ld, nrows, ncols, x, c,
                     dim, xn, cn_max, kappa, k, id_base, accum, ids, d);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

template <int VPL>
fgpu_status launch_select_t(const void* est, int64_t ld, int64_t nrows, int ncols, const float* x,
                            const float* c, int dim, const float* cn_max, float kappa,
                            int p, int prune, float prune_ratio, int32_t* ids, float* d, int* side, int side_val,
                            hipStream_t s, unsigned long long* stats) {
  const int64_t blocks = (nrows + 3) / 4;
  if constexpr (kEstHalf)
    hipLaunchKernelGGL((select_exact_kernel<VPL, uint16_t>), dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const uint16_t*>(est), ld, nrows, ncols, x, c, dim, cn_max, kappa, p, prune,
                       prune_ratio, ids, d, side, side_val, est_row_shift(const_cast<void*>(est), nrows, ld), stats);
  else
    hipLaunchKernelGGL((select_exact_kernel<VPL, float>), dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const float*>(est), ld, nrows, ncols, x, c, dim, cn_max, kappa, p, prune,
                       prune_ratio, ids, d, side, side_val, nullptr, stats);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace

fgpu_status launch_row_norms(const float* rows, int64_t n, int dim, float* norms, hipStream_t s) {
  if (n <= 0) return FGPU_OK;
  hipLaunchKernelGGL(row_norms_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, rows, n, dim, norms);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_max_reduce(const float* v, int64_t n, float* out, hipStream_t s) {
  hipLaunchKernelGGL(max_reduce_kernel, dim3(1), dim3(1024), 0, s, v, n, out);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

template <int OM>
fgpu_status launch_gemm_t(const float* x, int64_t nrows, const float* c, int ncols, int dim, const float* xn,
                          const float* cn, void* est, int64_t ld, hipStream_t s, const float* cn_max = nullptr) {
  FGPU_CHECK(dim % 4 == 0, FGPU_ERR_UNSUPPORTED, "gemm_est: dim must be a multiple of 4");
  FGPU_CHECK(OM != kOutHalf || cn_max, FGPU_ERR_ARG, "gemm_est: the fp16 form needs max ||c||^2");
  if (nrows <= 0 || ncols <= 0) return FGPU_OK;
  dim3 grid((unsigned)((nrows + kTM - 1) / kTM), (unsigned)((ncols + kTN - 1) / kTN));
  FGPU_CHECK(grid.y <= 65535u, FGPU_ERR_UNSUPPORTED, "gemm_est: too many columns");
  uint8_t* rsh = OM == kOutHalf ? est_row_shift(est, nrows, ld) : nullptr;
  if (dim % 32 == 0)
    hipLaunchKernelGGL(gemm_est_split_kernel<OM>, grid, dim3(256), 0, s, x, nrows, c, ncols, dim, xn, cn, est, ld,
                       cn_max, rsh);
  else
    hipLaunchKernelGGL(gemm_est_kernel<OM>, grid, dim3(256), 0, s, x, nrows, c, ncols, dim, xn, cn, est, ld, cn_max,
                       rsh);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_gemm_est(const float* x, int64_t nrows, const float* c, int ncols, int dim,
                            const float* xn, const float* cn, float* est, int64_t ld, hipStream_t s) {
  return launch_gemm_t<kOutFull>(x, nrows, c, ncols, dim, xn, cn, est, ld, s);
}

fgpu_status launch_gemm_est_sel(const float* x, int64_t nrows, const float* c, int ncols, int dim, const float* cn,
                                const float* cn_max, void* est, int64_t ld, hipStream_t s) {
  FGPU_CHECK(ld % 8 == 0, FGPU_ERR_ARG, "gemm_est_sel: row stride must be a multiple of 8");
  if constexpr (kEstHalf)
    return launch_gemm_t<kOutHalf>(x, nrows, c, ncols, dim, nullptr, cn, est, ld, s, cn_max);
  else
    return launch_gemm_t<kOutShift>(x, nrows, c, ncols, dim, nullptr, cn, est, ld, s);
}

int64_t est_sel_ld(int ncols) { return ((int64_t)ncols + 7) / 8 * 8; }

// The margin factor of the estimate launch_gemm_est computes for this dim.
static float coarse_kappa(int dim) {
  const double u = std::ldexp(1.0, -24);
  if (dim % 32 == 0) {  // gemm_est_split_kernel
    const double n = 3.0 * dim + 8.0;
    const double gamma = n * u / (1.0 - n * u);
    return (float)(8.0 * gamma * 1.001 + 4.0 * std::ldexp(1.0, -14));
  }
  const double n = 2.0 * dim + 8.0;
  const double gamma = n * u / (1.0 - n * u);
  return (float)(8.0 * gamma * 1.001);
}

fgpu_status launch_select_exact(const void* est, int64_t ld, int64_t nrows, int ncols, const float* x,
                                const float* c, int dim, const float* cn_max, int p,
                                int prune, float prune_ratio, int32_t* ids, float* d, hipStream_t s, int* side,
                                int side_val, unsigned long long* stats) {
  FGPU_CHECK(ld % 8 == 0, FGPU_ERR_ARG, "select: row stride must be a multiple of 8");
  FGPU_CHECK(p >= 1 && p <= kSelectMax && p <= ncols, FGPU_ERR_UNSUPPORTED, "select: need 1 <= p <= min(256, ncols)");
  FGPU_CHECK(dim <= 256, FGPU_ERR_UNSUPPORTED, "select: dim must be <= 256");
  if (nrows <= 0) return FGPU_OK;
  const float kappa = coarse_kappa(dim);
  if (p == 1 && ncols > 16 * kWave) {
    const dim3 grid((unsigned)((nrows + 3) / 4));
    if constexpr (kEstHalf)
      hipLaunchKernelGGL(select_min_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(est), ld,
                         nrows, ncols, x, c, dim, cn_max, kappa, prune, prune_ratio, ids, d, side, side_val,
                         est_row_shift(const_cast<void*>(est), nrows, ld), stats);
    else
      hipLaunchKernelGGL(select_min_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(est), ld, nrows,
                         ncols, x, c, dim, cn_max, kappa, prune, prune_ratio, ids, d, side, side_val, nullptr,
                         stats);
    FGPU_HIP(hipGetLastError());
    return FGPU_OK;
  }
#define FGPU_SEL(V) \
  if (ncols <= (V) * kWave) \
    return launch_select_t<V>(est, ld, nrows, ncols, x, c, dim, cn_max, kappa, p, prune, prune_ratio, ids, d, side, \
                              side_val, s, stats)
  FGPU_SEL(1);
  FGPU_SEL(2);
  FGPU_SEL(4);
  FGPU_SEL(8);
  FGPU_SEL(16);
  FGPU_SEL(32);
  FGPU_SEL(64);
#undef FGPU_SEL
  return set_error(FGPU_ERR_UNSUPPORTED, "select: more than 4096 columns");
}

fgpu_status launch_knn_chunk(const float* est, int64_t ld, int64_t nrows, int ncols, const float* x, const float* c,
                             int dim, const float* xn, const float* cn_max, int k, int id_base, int accum,
                             int32_t* ids, float* d, hipStream_t s) {
  FGPU_CHECK(k >= 1 && k <= 2 * kWave, FGPU_ERR_UNSUPPORTED, "knn: k must be in [1, 128]");
  FGPU_CHECK(dim <= 256, FGPU_ERR_UNSUPPORTED, "knn: dim must be <= 256");
  FGPU_CHECK(ncols >= 1 && ncols <= 64 * kWave, FGPU_ERR_UNSUPPORTED, "knn: chunk must hold 1..4096 rows");
  if (nrows <= 0) return FGPU_OK;
  const float kappa = coarse_kappa(dim);
  if (ncols <= 16 * kWave)
    return launch_knn_t<16>(est, ld, nrows, ncols, x, c, dim, xn, cn_max, kappa, k, id_base, accum, ids, d, s);
  return launch_knn_t<64>(est, ld, nrows, ncols, x, c, dim, xn, cn_max, kappa, k, id_base, accum, ids, d, s);
}

int64_t est_rows_per_batch(size_t bytes, int ncols) {
  int64_t r = (int64_t)(bytes / ((size_t)ncols * sizeof(float)));
  return r - r % 64;
}

}  // namespace fgpu
