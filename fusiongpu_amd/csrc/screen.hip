// screen.hip -- the plain IVF-PQ search (A4, A5, A6 and A10 with p1 = nprobe,
// limit_k = rerank_m = k) as an MFMA screen followed by an exact rescore.
//
// What is computed is unchanged.  The answer is the k smallest (ADC distance,
// vector id) keys over the probed lists, where each ADC distance is the
// sequential fp32 sum over ascending m of LUT[m][code_m] (gpu_global.cu:196-253)
// and each LUT entry is the reference's fused chain over the residual
// r = fl(q - c) minus the codeword (gpu_global.cu:79-166).  The reference
// builds that LUT for every (query, probed list), scans every probed vector
// with it (gpu_global.cu:321-390) and sorts (gpu_global.cu:852-867).
//
// Here no LUT is built.  Instead:
//   1. Threshold.  For every query, its first usable probed list is screened
//      with upper bounds U(v) >= d(q, v) of the exact distances.  The list's
//      vectors fall into 32 groups by position; the k-th smallest of the 32
//      group minima of U is T(q): k distinct vectors have d <= T(q), so the
//      final k-th distance is <= T(q).
//   2. Screen.  Every probed list whose lower bound (list_lower_bound, the
//      flow kernel's rule) is <= T(q) is screened with lower bounds
//      L(v) <= d(q, v) in the form V(v) = L(v) - T(q) <= 0: a vector with
//      d <= T(q) always passes, so every member of the top-k is a candidate.
//   3. Rescore.  The candidates' exact distances are recomputed with the
//      reference's direct form (gpu_global.cu:259-319: the same fused chain per
//      subspace and the same sequential sum, so each equals the LUT value bit
//      for bit) and the k smallest keys are kept.  Queries without a threshold
//      (a first list shorter than k, out-of-range values) or with more
//      candidates than the buffer holds go to the LUT kernel instead; a query
//      without a usable probe, or whose only probe's list is shorter than k,
//      has every vector there (none, or that list) as its candidates.
//
// The bounds.  With p the decoded residual of v (codebook rows, fp32) and
// D* = ||r - p||^2 exactly, d = D* (1 +- gamma_c), gamma_c = gamma(s + M + 1)
// < 2^-16 (non-negative terms, s + M + 1 roundings; gamma(n) = n u/(1 - n u),
// u = 2^-24).  The screen works on the data times 2^S (S per index: every
// decoded norm at most 64 after scaling), so it bounds D*' = 2^(2S) D*, and
// each row (pair) runs at its own scale 2^-t (all its values times 2^-t,
// which keeps every fp16 value below 2^15; see the pair record).  Powers of
// two change neither the signs of the tests nor the order of one row's
// values.  At the data's scale, with r' = 2^S r, p'' = 2^S p, the screen forms
//     <a', p'>  +  per-query and per-vector constants,   a = -2 r' (exact),
// on v_mfma_f32_32x32x16_f16, a' = fp16(a) and p' = fp16(p'') (nearest, zero
// below 2^-14): the main K range holds a' against p'; one extra K block of 16
// carries the constants, each split into three fp16 values with directed
// rounding, so the MFMA sum is the whole test value.  With the rounding
// errors' norms E_a = ||a' - a|| (per query and list) and E_p = ||p' - p''||
// (per vector),
//     |<a', p'> - <a, p''>| <= E_a X + 2 R E_p + E_a E_p  (Cauchy-Schwarz)
// for R >= ||r'||, X >= ||p''||: the norms are measured, about 2^-12.4
// relative per element (fp16 has 11 significant bits; bf16 would leave 8).
// The fp16 values are normal or zero (the helpers below flush in the stated
// direction), their products exact in fp32.  The MFMA adds at most 144 fp32
// roundings over terms whose magnitudes sum to <= 1.03 (T + (R + X)^2), and
// may flush partial sums below 2^-126 (< 2^-118 in all, at the row scale).
// With B = (E_a + k R) X' + 2 R E_p, X' >= X + E_p, k = 2^-14, g = 2^-15 and
// t = 1 + 2^-14 the two tests are (at the data's scale; each row's record
// holds them times 2^-t)
//     V = ||p''||^2 - gX'^2 + <a',p'> - B
//         - (t T - nr2' + g R^2) - 2^-110 (1 + R)          <= 0,
//     U = ||p''||^2 + gX'^2 + <a',p'> + B
//         + (t nr2' + g R^2) + 2^-110 (1 + R)              >= D*',
// nr2' = 2^(2S) times the fp32 sum of squares of r (within gamma(129) of
// ||r'||^2).  Collecting terms, every coefficient of V - (d' - T)-style slack
// is negative (1.8e-5 is twice the MFMA's 144 u 1.03): T (1/(1-gamma_c) - t
// + 1.8e-5) < 0, R X (3.6e-5 - k) < 0, R^2 (gamma(129) + 1.8e-5 - g) < 0,
// X^2 (1.8e-5 - g) < 0 (g = 3.05e-5, t - 1 = k = 6.1e-5) and the absolute
// terms; so d' <= T implies V <= 0, and U >= D*' for the threshold, which is
// then inflated by t.  The per-vector constants (X' rounded up to fp16,
// ||p''||^2 -+ gX'^2 in double, split; E_p rounded up) are built once per
// index; the per-query ones per (query, list), E_a from the fp32 sum of the
// squared errors (relative error below 2^-16, plus 2^-100 absolute for
// underflow).  Indexes whose decoded norms exceed 2^40 take the LUT kernels;
// a pair whose residual norm leaves the row scales (t > 14) or exceeds 2^40
// sends its query to the LUT kernel.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"
#include "scan_common.hpp"

namespace fgpu {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

namespace {

constexpr double kRX = 0x1p-14;          // coefficient of R X (the MFMA's roundings)
constexpr double kG = 0x1p-15;           // coefficient of R^2 and X^2
constexpr double kTInfl = 1.0 + 0x1p-14;
constexpr double kAbs = 0x1p-110;
constexpr double kDbl = 0x1p-40;         // slack for the double-precision constant arithmetic
constexpr float kMaxNorm2 = 0x1p80f;     // squared residual norms above this take the LUT kernel
constexpr int kQB = 32;                  // queries per work item (MFMA rows)
constexpr int kTV = 32;                  // vectors per tile (MFMA columns)
constexpr int kSW = 16;                  // waves per screen workgroup
constexpr int kCandBuf = 256;            // per-wave candidate staging entries (LDS)
constexpr int kChunk = 256;              // list vectors per round-1 work item (at most kMaxChunks items a group)
constexpr int kMaxChunks = 8;
constexpr int kMaxGroups = 64;           // round-1 groups a query's first list splits into, at most
constexpr int kPairBatch = 8;            // round-2 pairs whose centroid rows a wave loads together
// Groups of round 1: the k-th smallest group minimum bounds the k-th smallest
// U from above only when k <= groups.
__host__ __device__ constexpr int screen_groups(int k) { return k > 32 ? 64 : 32; }

constexpr int kRecHalf = 9;              // uint4 per lane half of a pair record: 8 A fragments, the extra block
constexpr int kRec = 2 * kRecHalf;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int lanes_below64(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// ---- fp16 with stated rounding, normal values and zero only ----------------------
// Every operand and constant the screen gives the MFMA is 0 or a normal fp16:
// magnitudes below 2^-14 are flushed by these helpers (in the stated
// direction), and the error norms are measured against the stored values, so
// nothing depends on how the MFMA treats subnormal inputs.
constexpr float kHMin = 0x1p-14f;            // smallest normal fp16
constexpr uint16_t kHOne = 0x3C00u;          // 1.0
constexpr uint16_t kHBig = 0x7BFFu;          // 65504, the largest finite fp16
constexpr uint32_t kOneOne = 0x3C003C00u;    // two fp16 1.0
__device__ __forceinline__ double h_val(uint16_t b) { return (double)(float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ float h_float(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// Nearest (f finite, |f| < 65504), magnitudes below 2^-14 to zero.
__device__ __forceinline__ uint16_t h_rn(float f) {
  return fabsf(f) < kHMin ? (uint16_t)0 : __builtin_bit_cast(uint16_t, (_Float16)f);
}
// The neighbours of b among {0, normal fp16}.
__device__ __forceinline__ uint16_t h_next_down(uint16_t b) {
  const uint16_t mag = b & 0x7FFFu;
  if (mag == 0) return 0x8400u;                                     // 0 -> -2^-14
  if (b & 0x8000u) return (uint16_t)(b + 1u);                       // larger magnitude
  return mag == 0x0400u ? (uint16_t)0 : (uint16_t)(b - 1u);         // 2^-14 -> 0
}
__device__ __forceinline__ uint16_t h_next_up(uint16_t b) {
  const uint16_t mag = b & 0x7FFFu;
  if (mag == 0) return 0x0400u;                                     // 0 -> 2^-14
  if (b & 0x8000u) return mag == 0x0400u ? (uint16_t)0 : (uint16_t)(b - 1u);
  return (uint16_t)(b + 1u);
}
// A value of {0, normal fp16} <= v, and one >= v (|v| < 65504): the nearest,
// moved one step when it lies on the wrong side.
__device__ __forceinline__ uint16_t h_down(double v) {
  uint16_t b = h_rn((float)v);
  while (h_val(b) > v) b = h_next_down(b);
  return b;
}
__device__ __forceinline__ uint16_t h_up(double v) {
  uint16_t b = h_rn((float)v);
  while (h_val(b) < v) b = h_next_up(b);
  return b;
}
// The largest float <= v and the smallest float >= v (v finite).
__device__ __forceinline__ float f_step_down(float f) {
  if (f == 0.0f) return -0x1p-149f;
  const uint32_t u = __float_as_uint(f);
  return __uint_as_float(f > 0.0f ? u - 1u : u + 1u);
}
__device__ __forceinline__ float f_step_up(float f) {
  if (f == 0.0f) return 0x1p-149f;
  const uint32_t u = __float_as_uint(f);
  return __uint_as_float(f > 0.0f ? u + 1u : u - 1u);
}
__device__ __forceinline__ float f_below(double v) {
  const float f = (float)v;
  return (double)f > v ? f_step_down(f) : f;
}
__device__ __forceinline__ float f_above(double v) {
  const float f = (float)v;
  return (double)f < v ? f_step_up(f) : f;
}
// Three fp16 whose sum is <= v (UP false) or >= v (UP true), within about
// 2^-34 |v| + 2^-13 (|v| < 65504).  The first two parts are nearest roundings,
// so each remainder is exact in double; the last is rounded in the stated
// direction.
template <bool UP>
__device__ __forceinline__ void split3(double v, uint16_t& b1, uint16_t& b2, uint16_t& b3) {
  b1 = h_rn((float)v);
  const double r1 = v - h_val(b1);
  b2 = h_rn((float)r1);
  const double r2 = r1 - h_val(b2);
  b3 = UP ? h_up(r2) : h_down(r2);
}
__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return (uint32_t)lo | ((uint32_t)hi << 16); }

// ---- index-time arrays -----------------------------------------------------------
// The screen works on the data times 2^S (S per index, scale_exp: every
// decoded residual norm at most 64 after scaling), so the squared distances
// it bounds are 2^(2S) times the exact ones; the sign of every test, and the
// order of values within one row, are unchanged.
// vext[v]: the per-vector block of the extra K range, 8 fp16 (scaled data):
//   [X', y'_1, y'_2, y'_3, y''_1, y''_2, y''_3, E_p]
// with p' = fp16(2^S p) (each element nearest, flushed below 2^-14, as
// cb16 holds it), E_p >= ||p' - 2^S p|| and X' >= ||2^S p|| + E_p (rounded
// up), y' <= P - g X'^2 - 2^-110 X', y'' >= P + g X'^2 + 2^-110 X',
// P = ||2^S p||^2 (each a three-part split).  P and the squared errors are
// summed in double (each square exact; 128 roundings of 2^-53 are covered by
// the 2^-40 slack).  xmax_bits: the largest X' as float bits (atomic max).
__global__ __launch_bounds__(256) void screen_prep_kernel(const float* __restrict__ cb, int m, int s, int scale_exp,
                                                          const uint8_t* __restrict__ codes, int64_t total,
                                                          uint4* __restrict__ vext,
                                                          unsigned int* __restrict__ xmax_bits) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const double sc = ldexp(1.0, scale_exp);
  float xm = 0.0f;
  if (v < total) {
    const uint8_t* c = codes + v * m;
    double p2 = 0.0, e2 = 0.0;
    for (int j = 0; j < m; ++j) {
      const float* p = cb + ((size_t)j * kPQK + c[j]) * s;
      for (int d = 0; d < s; ++d) {
        const double x = (double)p[d] * sc;
        const double e = x - h_val(h_rn((float)x));
        p2 += x * x;
        e2 += e * e;
      }
    }
    const uint16_t eb = h_up(sqrt(e2) * (1.0 + kDbl));
    const uint16_t xb = h_up((sqrt(p2) + h_val(eb)) * (1.0 + kDbl));
    const double xu = h_val(xb);
    const double lo = p2 - kG * xu * xu - kAbs * xu - kDbl * p2;
    const double hi = p2 + kG * xu * xu + kAbs * xu + kDbl * p2;
    uint16_t l1, l2, l3, h1, h2, h3;
    split3<false>(lo, l1, l2, l3);
    split3<true>(hi, h1, h2, h3);
    vext[v] = make_uint4(pack2(xb, l1), pack2(l2, l3), pack2(h1, h2), pack2(h3, eb));
    xm = (float)xu;
  }
  xm = wave_max_f(xm);
  if ((threadIdx.x & 63) == 0 && xm > 0.0f) atomicMax(xmax_bits, __float_as_uint(xm));
}

// The codebook times 2^S in fp16 (nearest, flushed below 2^-14), as the
// screen's B operand.  The scaling is exact in double.
__global__ __launch_bounds__(256) void cb_f16_kernel(const float* __restrict__ cb, int64_t n, int scale_exp,
                                                     uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = h_rn((float)((double)cb[i] * ldexp(1.0, scale_exp)));
}

// ---- work lists ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void screen_zero_kernel(int* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

// Pair entry `ent` (= q nprobe + p) of query q goes to slot `pos` of list
// l's bucket, taken earlier with an atomic on the list's count (the screen
// kernels derive their work items from the final counts).
__device__ __forceinline__ size_t bucket_base(const ScreenArgs& a, int l) {
  return a.boff ? (size_t)a.boff[l] : (size_t)l * a.nq;
}
// Entries list l's bucket can hold.
__device__ __forceinline__ int bucket_len(const ScreenArgs& a, int l) {
  return a.boff ? a.boff[l + 1] - a.boff[l] : a.nq;
}
__device__ __forceinline__ int bucket_put(const ScreenArgs& a, int l, int q, int ent, int pos) {
  // A probe list repeating a list id (or more pairs than a compact bucket
  // holds): the query takes the LUT kernel.
  if (pos >= bucket_len(a, l)) {
    a.thr[q] = __builtin_nanf("");
    return -1;
  }
  a.bucket[bucket_base(a, l) + pos] = ent;
  return pos;
}

// Work items of list l: groups of kQB queries times chunks of the list of
// kChunk vectors (longer chunks, multiples of kTV, past kMaxChunks of them).
// Round 2 takes its chunk length and count from the launch (ScreenArgs).
template <int ROUND = 1>
__device__ __forceinline__ int chunk_len(const ScreenArgs& a, int n) {
  const int kc = ROUND == 1 ? kChunk : a.r2_chunk, km = ROUND == 1 ? kMaxChunks : a.r2_max_chunks;
  return max(kc, (n + km * kTV - 1) / (km * kTV) * kTV);
}
template <int ROUND = 1>
__device__ __forceinline__ int list_items(const ScreenArgs& a, int cnt, int nq, int n) {
  if (cnt <= 0 || n <= 0) return 0;
  const int ng = (min(cnt, nq) + kQB - 1) / kQB;
  const int per = chunk_len<ROUND>(a, n);
  return ng * ((n + per - 1) / per);
}

// The pair record of entry ent = (query q, probe p of list l), at the pair's
// row scale 2^-t (t >= 0 the smallest with max(R'^2, t T') 2^-t <= 2^14, R'
// and T' the scaled residual norm and threshold; t <= 14, else the pair is
// unusable): for each lane half h (dims [h D/2, (h+1) D/2)) the A fragments
// a' = fp16(-2 r 2^(S-t)), r = fl(q - c), in MFMA operand order (fragment c
// holds dims h D/2 + 8c .. + 7), then the extra K block of the round's test:
//   round 1 (U):  h0 [ e, 0, 0, 0, u, u, u,  w]   h1 [c1, c2, c3, 1, 0 ...]
//   round 2 (V):  h0 [-e, u, u, u, 0, 0, 0, -w]   h1 [v1, v2, v3, 1, 0 ...]
// against the vector's block [X', y'1..3, y''1..3, E_p] (h0) and
// [1, 1, 1, 0 ...] (h1; [1, 1, 1, 65504, 0 ...] for a column past the range,
// which so exceeds every real value): u = 2^-t, e >= (E_a + k R') 2^-t with
// E_a = ||a' - (-2 r 2^(S-t))|| 2^t, w >= 2 R' 2^-t (so e X' + w E_p >= B 2^-t),
// c1 + c2 + c3 >= (t nr2' + g R'^2) 2^-t + 2^-110 (1 + R' 2^-t),
// v1 + v2 + v3 <= -(t T' - nr2' + g R'^2) 2^-t - 2^-110 (1 + R' 2^-t), each
// with the 2^-40 slack of the double arithmetic (nr2' = 2^(2S) nr2).  Every value
// of a row is 2^-t times its value at the data's scale 2^S, so the row's
// tests keep their signs and its U values their order, and every fp16 value
// stays below 2^15.  The record is unusable when nr2 is not <= kMaxNorm2
// (NaN included) or t > 14: then its A fragments are zero and its block the
// round's inactive one (round 2: V = 65504 through h1's first slot), so its
// row passes nothing and bounds nothing, and the caller adds no pair or
// drops the query.
//
// pair_a: the A fragments, by a whole wave (qv, cv: this lane's two dims of
// the query and of the list's centroid; tt: t T' for round 2, else 0);
// returns nr2, the fp32 sum of the squared errors of a' (at the row scale)
// and t on every lane.
struct PairA {
  float nr2, ea2;
  int t;  // > 14: unusable
};
template <int D>
__device__ __forceinline__ float2 centroid_dims(const ScreenArgs& a, int l) {
  const int lane = threadIdx.x & 63;
  return 2 * lane < D ? reinterpret_cast<const float2*>(a.centroids + (size_t)l * D)[lane] : make_float2(0.0f, 0.0f);
}
// The row scale exponent of a pair: nr2 unscaled, tt scaled; with `room`,
// also room for any threshold the pair's own list can give, (R' + 64)^2.
__device__ __forceinline__ int row_scale_exp(float nr2, double tt, int scale_exp, bool room = false) {
  const double n2 = ldexp((double)nr2, 2 * scale_exp);
  const double rt = sqrt(n2) + 64.0;
  const double m = fmax(fmax(n2, room ? rt * rt * (1.0 + 0x1p-10) : tt), fmax(tt, 1.0)) * (1.0 + 0x1p-10);
  if (!(m <= 0x1p60)) return 99;  // NaN or far out of range
  int t = 0;
  while (ldexp(m, -t) > 0x1p14) ++t;
  return t;
}
template <int D>
__device__ PairA pair_a(const ScreenArgs& a, int64_t ent, float2 qv, float2 cv, double tt, bool room = false) {
  const int lane = threadIdx.x & 63;
  const bool has = 2 * lane < D;
  const float r0 = has ? qv.x - cv.x : 0.0f, r1 = has ? qv.y - cv.y : 0.0f;
  const float nr2 = wave_sum_f(__builtin_fmaf(r1, r1, r0 * r0));
  const int t = row_scale_exp(nr2, tt, a.scale_exp, room);
  const bool ok = nr2 <= kMaxNorm2 && t <= 14;  // false for NaN
  // -2 r 2^(S-t): a power-of-two scaling, exact in fp32 (up to underflow below
  // 2^-126, covered by the absolute slack); its difference from the stored
  // fp16 value is exact in fp32
  const float f = ok ? ldexpf(-2.0f, a.scale_exp - t) : 0.0f;
  const float x0 = r0 * f, x1 = r1 * f;
  const uint16_t b0 = h_rn(x0), b1 = h_rn(x1);
  const float e0 = x0 - h_float(b0), e1 = x1 - h_float(b1);
  const float ea2 = wave_sum_f(ok ? __builtin_fmaf(e1, e1, e0 * e0) : 0.0f);
  uint32_t* rec = reinterpret_cast<uint32_t*>(a.arec + ent * kRec);
  if (has) {
    const int d = 2 * lane, h = d / (D / 2), w = d % (D / 2);
    rec[(h * kRecHalf + w / 8) * 4 + (w % 8) / 2] = ok ? pack2(b0, b1) : 0u;
  }
  return PairA{nr2, ea2, ok ? t : 99};
}
// pair_ex: both lane halves' extra blocks of entry ent, by one lane (pa: what
// pair_a returned; T: the scaled threshold, round 2).
template <int ROUND>
__device__ void pair_ex(const ScreenArgs& a, int64_t ent, PairA pa, float T) {
  uint4* rec = a.arec + ent * kRec;
  if (pa.t > 14) {
    rec[kRecHalf - 1] = make_uint4(0u, 0u, 0u, 0u);
    rec[2 * kRecHalf - 1] = make_uint4(ROUND == 2 ? pack2(kHBig, 0u) : 0u, 0u, 0u, 0u);
    return;
  }
  const double n2 = ldexp((double)pa.nr2, 2 * a.scale_exp);
  const double R = sqrt(n2 * (1.0 + 0x1p-16)) * (1.0 + kDbl);
  const double u = ldexp(1.0, -pa.t);
  const double Ea = sqrt((double)pa.ea2 * (1.0 + 0x1p-16) + 0x1p-100) * (1.0 + kDbl);
  const uint16_t e = h_up(Ea + kRX * R * u), w = h_up(2.0 * R * u);
  const uint16_t ub = (uint16_t)((15 - pa.t) << 10);  // 2^-t
  const uint32_t uu = pack2(ub, ub);
  uint16_t p1, p2, p3;
  if (ROUND == 2) {
    const double t = (double)fmaxf(T, 0.0f);
    const double rhs = (t * kTInfl - n2 + kG * R * R) * u + kAbs * (1.0 + R * u);
    split3<false>(-rhs - kDbl * (t + n2 + kG * R * R) * u, p1, p2, p3);
    rec[kRecHalf - 1] = make_uint4(pack2(e ^ 0x8000u, ub), uu, 0u, pack2(0u, w ^ 0x8000u));
  } else {
    const double c = (n2 * kTInfl + kG * R * R) * u + kAbs * (1.0 + R * u);
    split3<true>(c * (1.0 + kDbl), p1, p2, p3);
    rec[kRecHalf - 1] = make_uint4(pack2(e, 0u), 0u, uu, pack2(ub, w));
  }
  rec[2 * kRecHalf - 1] = make_uint4(pack2(p1, p2), pack2(p3, kHOne), 0u, 0u);
}

__device__ __forceinline__ float2 query_dims(const ScreenArgs& a, int q, int dim) {
  const int lane = threadIdx.x & 63;
  return 2 * lane < dim ? reinterpret_cast<const float2*>(a.queries + (size_t)(q / a.qdiv) * dim)[lane]
                        : make_float2(0.0f, 0.0f);
}

// Round 1 pairs, one wave a query: the query with its first usable probe (in
// range, non-empty) when that list holds at least k vectors and the residual
// norm is in range; its pair record carries the U test.  A query without a
// usable probe, or with a single probe whose list is shorter than k, takes
// that list's vectors as its candidates at once.
template <int D>
__global__ __launch_bounds__(256) void screen_pairs1_kernel(ScreenArgs a) {
  const int lane = threadIdx.x & 63;
  const int q = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (q >= a.nq) return;
  int pf = -1, lf = 0;
  for (int p0 = 0; p0 < a.nprobe; p0 += kWave) {
    const int p = p0 + lane;
    uint32_t l = 0xFFFFFFFFu;
    bool use = false;
    if (p < a.nprobe) {
      l = a.probes[(size_t)q * a.nprobe + p];
      use = l < (uint32_t)a.nlist && a.offsets[l + 1] - a.offsets[l] > 0;
    }
    const uint64_t m = __ballot(use);
    if (m) {
      const int b = __builtin_ctzll(m);
      pf = p0 + b;
      lf = __builtin_amdgcn_readlane((int)l, b);
      break;
    }
  }
  int2 f = make_int2(-1, -1);
  const int n = pf >= 0 ? a.offsets[lf + 1] - a.offsets[lf] : 0;
  if (pf < 0 || (a.nprobe == 1 && n < a.k)) {
    // No usable probe, or a single probe whose list holds fewer than k
    // vectors: the answer is every vector there (then padding), so those are
    // the candidates, with no screen (first = -2; the rescore sorts them).
    const int start = pf >= 0 ? a.offsets[lf] : 0;
    for (int i = lane; i < n; i += kWave)
      a.cand[(size_t)q * a.cand_cap + i] = make_uint2((uint32_t)(start + i), (uint32_t)lf);
    if (lane == 0) a.cand_cnt[q] = n;
    f = make_int2(-2, 0);
  } else if (n >= a.k) {
    const int64_t ent = (int64_t)q * a.nprobe + pf;
    // first.y: the row scale exponent t and the list's round-1 chunk count
    const int per = chunk_len<1>(a, n), fy = (((n + per - 1) / per) << 8);
    // single-probe mode: the row scale leaves room for round 2's threshold
    // (at most (R' + 64)^2 (1 + 2^-10) with 2^S-scaled decoded norms <= 64),
    // so round 2 reuses this record's A fragments
    const PairA pa = pair_a<D>(a, ent, query_dims(a, q, D), centroid_dims<D>(a, lf), 0.0, a.sp_cnt != nullptr);
    if (lane == 0) pair_ex<1>(a, ent, pa, 0.0f);
    if (a.sp_cnt) {
      // the caller placed the query in its list's bucket
      if (lane == 0) {
        a.pnorm[q] = make_float2(pa.nr2, pa.ea2);
        if (pa.t <= 14) f = make_int2(lf, fy | pa.t);
      }
    } else if (pa.t <= 14 && lane == 0) {
      const int pos = bucket_put(a, lf, q, (int)ent, atomicAdd(&a.cnt1[lf], 1));
      if (pos >= 0) f = make_int2(lf, fy | pa.t);
    }
  }
  if (lane == 0) a.first[q] = f;
}

// Round 2 pairs, one wave a query.  First T(q): the k-th smallest of the 32
// group minima of U over the query's first list (the minimum, over the list's
// chunks, of each chunk's per-group minimum), taken back from the round-1
// row's scale 2^-t to the data's scale 2^S and inflated by 1 + 2^-14; +inf
// without a round-1 pair or with fewer than k groups holding a value
// (FLT_MAX, and nothing more, for the queries whose candidates are set).  Then
// every usable probe whose list bound does not exceed T(q) 2^-2S (the
// bounds are in the data's units), with its pair record carrying the V test.
// A probe whose pair is out of range sends the query to the LUT kernel
// (T = +inf).
template <int D>
__global__ __launch_bounds__(256) void screen_pairs2_kernel(ScreenArgs a) {
  const int lane = threadIdx.x & 63;
  const int q = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (q >= a.nq) return;
  const bool sp = a.sp_cnt != nullptr;
  // The first 64 probes' lists, sizes, bounds and the query's dims do not
  // depend on T: their loads go out before the threshold's (not needed in
  // single-probe mode).
  uint32_t l0 = 0xFFFFFFFFu;
  float lb0 = INFINITY;
  if (!sp && lane < a.nprobe) {
    const size_t t = (size_t)q * a.nprobe + lane;
    l0 = a.probes[t];
    if (l0 < (uint32_t)a.nlist && a.offsets[l0 + 1] - a.offsets[l0] > 0)
      lb0 = list_lower_bound(a.probe_dists[t], a.rmax[l0]);
  }
  const float2 qv = sp ? make_float2(0.0f, 0.0f) : query_dims(a, q, D);
  // Every chunk's group minima load goes out with the first pair's record
  // (a chain of the two is the kernel's longest latency); the query's block
  // holds kMaxChunks x kMaxGroups words, those past its chunks are unused.
  uint32_t gc[kMaxChunks];
  {
    const uint32_t* g = a.gminbuf + (size_t)q * kMaxChunks * kMaxGroups + lane;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) gc[c] = g[c * kMaxGroups];
  }
  const int2 f = a.first[q];
  const int ft = f.y & 0xFF;  // the round-1 row scale exponent
  if (f.x == -2) {
    // candidates set by the first pair kernel: the largest finite threshold
    // sends them to the rescore
    if (lane == 0) a.thr[q] = FLT_MAX;
    return;
  }
  uint32_t gm = 0x7F800000u;
  if (f.x >= 0 && lane < screen_groups(a.k)) {
    const int nch = f.y >> 8;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) gm = min(gm, c < nch ? gc[c] : 0x7F800000u);
  }
  // U >= 0, so float order is unsigned order of the bits
  wave_sort_u32(gm);
  const float kth = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)gm, a.k - 1));
  // the group minima are at the round-1 row's scale 2^-t
  const float T = kth < INFINITY ? f_above(ldexp((double)kth, ft) * kTInfl) : INFINITY;
  if (sp) {
    // Single-probe mode: the round-2 pair is the round-1 pair (the only
    // probe, whose list holds the threshold's own k vectors, so its bound
    // never exceeds T), and only its constant block changes; its A fragments
    // stay valid because round 1 chose the row scale with room for any
    // threshold its list can give.  A row in a bucket without a threshold
    // (an unusable round-1 pair) gets the unusable block, and its query the
    // LUT kernel.
    if (lane == 0) {
      PairA pa{0.0f, 0.0f, 99};
      if (f.x >= 0 && T < INFINITY) {
        const float2 pn = a.pnorm[q];
        pa = PairA{pn.x, pn.y, ft};
      }
      pair_ex<2>(a, (int64_t)q * a.nprobe, pa, T);
      a.thr[q] = pa.t <= 14 ? T : INFINITY;
    }
    return;
  }
  if (lane == 0) a.thr[q] = T;
  if (!(T < INFINITY)) return;
  const double tt = (double)T * kTInfl;            // the V constants' largest term
  const float Tu = ldexpf(T, -2 * a.scale_exp);    // in the data's units, for the list bounds
  bool bad = false;
  for (int p0 = 0; p0 < a.nprobe; p0 += kWave) {
    const int p = p0 + lane;
    uint32_t l = l0;
    bool pass = p0 == 0 && lb0 <= Tu;
    if (p0 > 0 && p < a.nprobe) {
      const size_t t = (size_t)q * a.nprobe + p;
      l = a.probes[t];
      pass = l < (uint32_t)a.nlist && a.offsets[l + 1] - a.offsets[l] > 0 &&
             list_lower_bound(a.probe_dists[t], a.rmax[l]) <= Tu;
    }
    // Every passing probe takes its slot of its list's bucket at once (one
    // atomic a lane) and writes it after the pair records, so the atomic's
    // round trip overlaps the centroid loads; a pair whose record turns out
    // unusable sends the whole query to the LUT kernel, whose rescore then
    // ignores its candidates.
    const int pos = pass ? atomicAdd(&a.cnt2[l], 1) : 0;
    // The A fragments, one pair at a time, eight pairs' centroid rows loaded
    // together ahead of them (a chain of single row loads is this loop's
    // longest latency); the lane of each probe keeps its pair's (nr2, error
    // sum), and the extra blocks follow lane-parallel (one lane a pair).
    uint64_t m = __ballot(pass);
    if (!m) continue;
    PairA my_pa{0.0f, 0.0f, 99};
    while (m) {
      int b[kPairBatch];
      float2 cv[kPairBatch];
#pragma unroll
      for (int j = 0; j < kPairBatch; ++j) {
        b[j] = m ? __builtin_ctzll(m) : -1;
        if (m) m &= m - 1;
        // list 0 stands in past the last pair (a row that exists; unused)
        cv[j] = centroid_dims<D>(a, b[j] >= 0 ? __builtin_amdgcn_readlane((int)l, b[j]) : 0);
      }
#pragma unroll
      for (int j = 0; j < kPairBatch; ++j) {
        if (b[j] < 0) break;
        const PairA pa = pair_a<D>(a, (int64_t)q * a.nprobe + p0 + b[j], qv, cv[j], tt);
        if (lane == b[j]) my_pa = pa;
      }
    }
    if (pass) {
      pair_ex<2>(a, (int64_t)q * a.nprobe + p, my_pa, T);
      bad = bad || my_pa.t > 14;
      bucket_put(a, (int)l, q, (int)((int64_t)q * a.nprobe + p), pos);
    }
  }
  if (__ballot(bad) && lane == 0) a.thr[q] = INFINITY;
}

// ---- the screen ---------------------------------------------------------------------------
// The 16 code bytes a lane half needs per 16-dim chunk group come from its
// half of the code row.  Lane half h covers dims [h D/2, (h+1) D/2): chunk c
// holds dims h D/2 + 8c + e (e < 8) for A and B alike.
template <int M>
__device__ __forceinline__ void load_half(const uint8_t* p, uint32_t (&w)[M / 8]) {
  if constexpr (M % 32 == 0) {
#pragma unroll
    for (int i = 0; i < M / 32; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < M / 16; ++i) {
      const uint2 v = reinterpret_cast<const uint2*>(p)[i];
      w[2 * i] = v.x; w[2 * i + 1] = v.y;
    }
  }
}

// 16-bit words code | (h M/2) << 8 for code bytes b and b + 1 of w: times the
// entry size this is the code's row in the lane half's part of the fp16
// codebook, so every gather below takes one shift and an immediate offset.
__device__ __forceinline__ uint32_t words2(uint32_t w, uint32_t hsel, int b) {
  const uint32_t sel = (uint32_t)b | (4u << 8) | ((uint32_t)(b + 1) << 16) | (4u << 24);
  return __builtin_amdgcn_perm(hsel, w, sel);
}

// The B fragment of chunk c: dims 8c .. 8c + 7 of the lane half's decoded row.
template <int D, int M>
__device__ __forceinline__ f16x8 decode_chunk(const uint16_t* cbs, const uint32_t (&cw)[M / 8], uint32_t hsel,
                                               int c) {
  constexpr int S = D / M;
  constexpr int SUB = 512 * S;  // bytes per subspace of the fp16 codebook
  const char* base = reinterpret_cast<const char*>(cbs);
  uint32_t f[4];
  if constexpr (S == 4) {
    const uint32_t wd = words2(cw[c >> 1], hsel, 2 * (c & 1));
    const uint32_t a0 = (wd & 0xFFFFu) << 3, a1 = (wd >> 16) << 3;
    const uint2 e0 = *reinterpret_cast<const uint2*>(base + a0 + (2 * c) * SUB);
    const uint2 e1 = *reinterpret_cast<const uint2*>(base + a1 + (2 * c + 1) * SUB);
    f[0] = e0.x; f[1] = e0.y; f[2] = e1.x; f[3] = e1.y;
  } else if constexpr (S == 8) {
    const uint32_t wd = words2(cw[c >> 2], hsel, c & 3);  // byte c & 3 (the second word is unused)
    const uint32_t a0 = (wd & 0xFFFFu) << 4;
    const uint4 e = *reinterpret_cast<const uint4*>(base + a0 + c * SUB);
    f[0] = e.x; f[1] = e.y; f[2] = e.z; f[3] = e.w;
  } else {
    static_assert(S == 2, "screen: sub-dimension 2, 4 or 8");
    const uint32_t w01 = words2(cw[c], hsel, 0), w23 = words2(cw[c], hsel, 2);
    f[0] = *reinterpret_cast<const uint32_t*>(base + ((w01 & 0xFFFFu) << 2) + (4 * c) * SUB);
    f[1] = *reinterpret_cast<const uint32_t*>(base + ((w01 >> 16) << 2) + (4 * c + 1) * SUB);
    f[2] = *reinterpret_cast<const uint32_t*>(base + ((w23 & 0xFFFFu) << 2) + (4 * c + 2) * SUB);
    f[3] = *reinterpret_cast<const uint32_t*>(base + ((w23 >> 16) << 2) + (4 * c + 3) * SUB);
  }
  return __builtin_bit_cast(f16x8, f);
}

__device__ __forceinline__ f16x8 frag_of(uint32_t x, uint32_t y, uint32_t z, uint32_t w) {
  const uint32_t f[4] = {x, y, z, w};
  return __builtin_bit_cast(f16x8, f);
}

// k-th smallest (1 <= k <= 32) of 32 values: bitonic sort in registers.
__device__ __forceinline__ uint32_t kth_of_32(uint32_t (&v)[32], int k) {
#pragma unroll
  for (int size = 2; size <= 32; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const bool up = (i & size) == 0;
          const uint32_t lo = min(v[i], v[j]), hi = max(v[i], v[j]);
          v[i] = up ? lo : hi;
          v[j] = up ? hi : lo;
        }
      }
    }
  }
  uint32_t r = v[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) r = (i == k - 1) ? v[i] : r;
  return r;
}

// One persistent workgroup per CU; each wave takes work items (list, group of
// up to kQB pairs of the list's bucket, range of the list's vectors) in turn:
// items w, w + waves, ... where w is its global index.  Each item's rows come
// from the pair records; the range is screened in tiles of kTV vectors.
// ROUND 1 stores each row's per-group minima of U; ROUND 2 appends the
// candidates (V <= 0) to their queries' arrays.
// LDS: the fp16 codebook first (offset 0, so every gather's subspace offset is
// the instruction's immediate), then per-wave staging.
template <int D, int M, int ROUND, int G = 32>
__global__ __launch_bounds__(kSW * kWave) void screen_kernel(ScreenArgs a) {
  static_assert(G == 32 || G == 64, "round-1 groups: 32 or 64");
  constexpr int NC = D / 16;  // main K chunks
  constexpr int HB = M / 2;   // code bytes per lane half
  static_assert(D % 32 == 0 && D <= 128, "screen: dim a multiple of 32, at most 128");
  constexpr int kCbBytes = D * kPQK * 2;
  constexpr int kWaveWords = ROUND == 1 ? 0 : 2 * kCandBuf;  // staged (row, vector position) pairs
  constexpr int kRowWords = ROUND == 1 ? kQB : 3 * kQB;        // each row's query (+ round 2: count, first slot)
  constexpr int kPreOff = kCbBytes + kSW * (kWaveWords + kRowWords) * 4;
  __shared__ __align__(16) unsigned char lds[kPreOff + (kScreenMaxLists + 1 + kSW) * 4];
  uint16_t* cbs = reinterpret_cast<uint16_t*>(lds);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint2* wbuf = reinterpret_cast<uint2*>(lds + kCbBytes + wave * kWaveWords * 4);
  int* rowq = reinterpret_cast<int*>(lds + kCbBytes + kSW * kWaveWords * 4) + wave * kRowWords;
  int* rcnt = rowq + kQB;  // round 2: each row's candidates in the staging buffer, then its first slot
  int* pre = reinterpret_cast<int*>(lds + kPreOff);  // [nlist + 1] first item of each list
  int* wsum = pre + kScreenMaxLists + 1;             // [kSW]
  const int li = lane & 31, h = lane >> 5;
  const long long t_begin = a.stats ? clock64() : 0;
  const int* cnt = a.sp_cnt ? a.sp_cnt : ROUND == 1 ? a.cnt1 : a.cnt2;
  for (int i = tid; i < kCbBytes / 16; i += kSW * kWave)
    reinterpret_cast<uint4*>(lds)[i] = reinterpret_cast<const uint4*>(a.cb16)[i];
  // The work items: for each list, its groups of queries times its chunks,
  // numbered by an exclusive scan over the lists (each thread 8 lists).
  {
    constexpr int kPer = kScreenMaxLists / (kSW * kWave);
    int v[kPer], s = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int l = tid * kPer + i;
      v[i] = l < a.nlist ? list_items<ROUND>(a, cnt[l], bucket_len(a, l), a.offsets[l + 1] - a.offsets[l]) : 0;
      s += v[i];
    }
    const int incl = wave_incl_scan(s);
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    if (wave == 0) {
      int x = lane < kSW ? wsum[lane] : 0;
      x = wave_incl_scan(x);
      if (lane < kSW) wsum[lane] = x;
    }
    __syncthreads();
    int base = (wave > 0 ? wsum[wave - 1] : 0) + incl - s;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int l = tid * kPer + i;
      if (l <= a.nlist) pre[l] = base;
      base += v[i];
    }
    __syncthreads();
  }
  const int nitems = __builtin_amdgcn_readfirstlane(wsum[kSW - 1]);
  long long ck = a.stats ? clock64() : 0;
  long long ck_pre = ck - t_begin, ck_setup = 0, ck_tiles = 0, ck_post = 0, ntiles = 0, nit = 0;
  const int nwaves = (int)gridDim.x * kSW;
  const uint32_t hsel = h ? (uint32_t)HB * 0x01010101u : 0u;
  // The extra block of a column: lane half 0 its vector's block (zeros past
  // the end of the range), lane half 1 the [1, 1, 1, 0 ...] multipliers, with
  // 65504 in slot 3 past the end: every row's record has 1 there, so such a
  // column's value (>= 65504 - 2^14 at every row scale) is never a candidate
  // and never a group minimum over real vectors (their values stay below 2^15).
  const uint4 h1_real = make_uint4(kOneOne, (uint32_t)kHOne, 0u, 0u);
  const uint4 h1_pad = make_uint4(kOneOne, pack2(kHOne, kHBig), 0u, 0u);

  for (int w = (int)blockIdx.x * kSW + wave; w < nitems; w += nwaves) {
    // Item w: the last list whose first item is <= w, then its group and chunk.
    int lo = 0, hi = a.nlist - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= w) lo = mid; else hi = mid - 1;
    }
    const int l = __builtin_amdgcn_readfirstlane(lo);
    const int start = a.offsets[l], n = a.offsets[l + 1] - start;
    const int per = chunk_len<ROUND>(a, n), nch = (n + per - 1) / per;
    const int local = w - __builtin_amdgcn_readfirstlane(pre[l]);
    const int grp = local / nch, jb = (local % nch) * per, je = min(n, jb + per);
    const int nrow = min(kQB, min(cnt[l], bucket_len(a, l)) - grp * kQB);
    const int ent = li < nrow ? a.bucket[bucket_base(a, l) + grp * kQB + li] : -1;

    // A tile's codes and extra blocks.  Every lane loads on every call (a
    // column past the range reloads the range's last vector; lane half 1
    // loads a block it does not use), so each tile issues the same loads and
    // the wait for a buffer never has to cover the loads issued after it;
    // the padding block replaces the loaded one where the tile uses it.
    auto load_tile = [&](int j0, uint32_t (&cw)[M / 8], uint4& bx) {
      const int j = min(j0 + li, je - 1);
      const int64_t v = (int64_t)start + j;
      load_half<M>(a.codes + v * M + h * HB, cw);
      bx = a.vext[v];
    };
    uint32_t cwA[M / 8], cwB[M / 8];
    uint4 bxA, bxB;
    load_tile(jb, cwA, bxA);
    load_tile(jb + kTV, cwB, bxB);

    // A rows and the extra block from the row's pair record.  A row without a
    // pair: zeros, and in round 2 V = 65504, so it never passes (in round 1
    // its minima are not stored).
    f16x8 A[NC];
    f16x8 Aex;
    {
      const uint4* rec = a.arec + (int64_t)(ent >= 0 ? ent : 0) * kRec + h * kRecHalf;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 v = ent >= 0 ? rec[c] : make_uint4(0u, 0u, 0u, 0u);
        A[c] = frag_of(v.x, v.y, v.z, v.w);
      }
      const uint4 e = ent >= 0 ? rec[kRecHalf - 1]
                               : make_uint4(ROUND == 2 && h == 1 ? pack2(kHBig, 0u) : 0u, 0u, 0u, 0u);
      Aex = frag_of(e.x, e.y, e.z, e.w);
    }
    // The query of each row, for the candidate flush and the round-1 store.
    if (h == 0) rowq[li] = ent >= 0 ? ent / a.nprobe : -1;

    // Per row and lane column, the smallest U bits seen (ROUND 1; every U is
    // >= 0, where float order is unsigned order).
    uint32_t mins[G / 32][16];
#pragma unroll
    for (int gp = 0; gp < G / 32; ++gp)
#pragma unroll
      for (int r = 0; r < 16; ++r) mins[gp][r] = 0x7F800000u;
    // ROUND 2 candidates: staged in wbuf as (row, vector position).  A
    // flush ranks each entry within its row (LDS atomics), reserves each
    // row's slots of its query's candidate array with one global atomic a
    // row, then writes the entries: one global round trip a flush instead of
    // one atomic a candidate.  The order of a query's candidates is free (the
    // rescore sorts them).
    int nb = 0;  // staged entries (wave-uniform)
    // A full buffer inside a tile (rare): one atomic a candidate, which keeps
    // the tile loop's registers down.
    auto flush_full = [&]() {
      wave_sync();
      for (int i0 = 0; i0 < nb; i0 += kWave) {
        const int i = i0 + lane;
        if (i < nb) {
          const uint2 e = wbuf[i];
          const int q = rowq[e.x];
          const int slot = atomicAdd(&a.cand_cnt[q], 1);
          if (slot < a.cand_cap) a.cand[(size_t)q * a.cand_cap + slot] = make_uint2((uint32_t)start + e.y, (uint32_t)l);
        }
      }
      nb = 0;
      wave_sync();
    };
    auto flush = [&]() {
      wave_sync();
      if (lane < kQB) rcnt[lane] = 0;
      wave_sync();
      for (int i0 = 0; i0 < nb; i0 += kWave) {
        const int i = i0 + lane;
        if (i < nb) {
          const uint32_t row = wbuf[i].x;
          const int rank = atomicAdd(&rcnt[row], 1);
          wbuf[i].x = row | ((uint32_t)rank << 8);  // row < 32, rank < kCandBuf
        }
      }
      wave_sync();
      if (lane < kQB) {
        const int c = rcnt[lane];
        rcnt[lane] = c > 0 ? atomicAdd(&a.cand_cnt[rowq[lane]], c) : 0;
      }
      wave_sync();
      for (int i0 = 0; i0 < nb; i0 += kWave) {
        const int i = i0 + lane;
        if (i < nb) {
          const uint2 e = wbuf[i];
          const int row = (int)(e.x & 255u), q = rowq[row];
          const int slot = rcnt[row] + (int)(e.x >> 8);
          if (slot < a.cand_cap) a.cand[(size_t)q * a.cand_cap + slot] = make_uint2((uint32_t)start + e.y, (uint32_t)l);
        }
      }
      nb = 0;
      wave_sync();
    };
    if (a.stats) {
      const long long t = clock64();
      ck_setup += t - ck;
      ck = t;
    }

    // One tile: the MFMA chain, each chunk's gathers just before its MFMA,
    // then the reload of the same buffer two tiles ahead (two buffers
    // alternate, so a tile never waits for the loads of the next one), then
    // the tile's results.
    // par: the tile's position within the chunk, mod 2 (its column group
    // half when G = 64)
    auto tile = [&](int j0, uint32_t (&cw)[M / 8], uint4& bx, int par) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[c], decode_chunk<D, M>(cbs, cw, hsel, c), acc, 0, 0, 0);
      const bool col = j0 + li < je;
      const uint4 bh = h == 0 ? (col ? bx : make_uint4(0u, 0u, 0u, 0u)) : (col ? h1_real : h1_pad);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aex, frag_of(bh.x, bh.y, bh.z, bh.w), acc, 0, 0, 0);
      load_tile(j0 + 2 * kTV, cw, bx);
      // acc[r]: row 8 (r / 4) + 4 h + r % 4 of the work item, column li (vector j0 + li).
      if constexpr (ROUND == 1) {
        if (G == 64 && par) {
#pragma unroll
          for (int r = 0; r < 16; ++r) mins[G / 32 - 1][r] = min(mins[G / 32 - 1][r], __float_as_uint(acc[r]));
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) mins[0][r] = min(mins[0][r], __float_as_uint(acc[r]));
        }
      } else {
        // V <= 0: the bits as a signed int are <= 0 (+0, or the sign set).
        int mn = __float_as_int(acc[0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mn = min(mn, __float_as_int(acc[r]));
        if (__ballot(mn <= 0)) {
          const int j = j0 + li;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const bool pass = __float_as_int(acc[r]) <= 0;
            const uint64_t bm = __ballot(pass);
            if (bm) {
              const int c = __popcll(bm);
              if (nb + c > kCandBuf) flush_full();
              const int row = 8 * (r >> 2) + 4 * h + (r & 3);
              if (pass) wbuf[nb + lanes_below64(bm)] = make_uint2((uint32_t)row, (uint32_t)j);
              nb += c;
            }
          }
        }
      }
    };
    for (int j0 = jb; j0 < je; j0 += 2 * kTV) {
      tile(j0, cwA, bxA, 0);
      if (j0 + kTV < je) tile(j0 + kTV, cwB, bxB, 1);
    }

    if (a.stats) {
      const long long t = clock64();
      ck_tiles += t - ck;
      ck = t;
    }
    if constexpr (ROUND == 2) {
      if (nb > 0) flush();
    } else {
      // Groups are vector positions within the chunk mod G (the lane column,
      // plus 32 for odd tiles when G = 64): this item's per-row, per-group
      // minima go to the row's query, at the item's chunk (each (query,
      // chunk) slot has exactly one writer); the pair kernel of round 2
      // combines the chunks of a query's list, group by group, which is again
      // a partition of the list.
      wave_sync();
      const int cidx = local % nch;
#pragma unroll
      for (int gp = 0; gp < G / 32; ++gp)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 8 * (r >> 2) + 4 * h + (r & 3);
          const int q = rowq[row];
          if (q >= 0) a.gminbuf[((size_t)q * kMaxChunks + cidx) * kMaxGroups + 32 * gp + li] = mins[gp][r];
        }
    }
    wave_sync();
    if (a.stats) {
      const long long t = clock64();
      ck_post += t - ck;
      ck = t;
    }
  }
  if (a.stats && lane == 0) {
    const int o = ROUND == 1 ? 0 : 4;
    atomicAdd(&a.stats[o], (unsigned long long)ck_pre);
    atomicAdd(&a.stats[o + 1], (unsigned long long)ck_setup);
    atomicAdd(&a.stats[o + 2], (unsigned long long)ck_tiles);
    atomicAdd(&a.stats[o + 3], (unsigned long long)ck_post);
    (void)ntiles;
    (void)nit;
  }
}

// ---- exact rescore ------------------------------------------------------------------------
template <int S>
__device__ __forceinline__ void load_row(const float* p, float (&v)[S]) {
  if constexpr (S % 4 == 0) {
#pragma unroll
    for (int i = 0; i < S / 4; ++i) {
      const float4 t = reinterpret_cast<const float4*>(p)[i];
      v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
  } else if constexpr (S % 2 == 0) {
#pragma unroll
    for (int i = 0; i < S / 2; ++i) {
      const float2 t = reinterpret_cast<const float2*>(p)[i];
      v[2 * i] = t.x; v[2 * i + 1] = t.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < S; ++i) v[i] = p[i];
  }
}

// One wave a query: the exact ADC distance of every candidate in the
// reference's direct form (the LUT entry's chain per subspace, summed in
// ascending m), then the k smallest (distance, id) keys.  A persistent grid
// of one workgroup per CU holding the fp32 codebook in LDS; wave g takes
// queries g, g + G, ... (of a.order when set), where workgroup b counts as
// b / 8 + (b % 8) G / (8 kRW) when the grid is a multiple of 8: workgroups go
// round-robin over the 8 XCDs, so neighbouring positions of the order (one
// list's queries, whose code rows they gather) share an XCD's L2.
// ONE (single-probe queries): every candidate lies in
// the query's one list, so the residual r = fl(q - c) is formed once in LDS
// (the same fp32 subtraction) instead of loading the centroid per candidate.
constexpr int kRW = 16;  // waves per rescore workgroup
template <int D, int M, bool ONE>
__global__ __launch_bounds__(kRW * kWave) void rescore_kernel(ScreenArgs a) {
  constexpr int S = D / M;
  __shared__ __align__(16) float cbf[D * kPQK];
  __shared__ float qs[kRW][D];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  for (int i = threadIdx.x; i < D * kPQK / 4; i += kRW * kWave)
    reinterpret_cast<float4*>(cbf)[i] = reinterpret_cast<const float4*>(a.codebook)[i];
  __syncthreads();
  const int stride = (int)gridDim.x * kRW;
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int lb = nb % 8 == 0 ? (b % 8) * (nb / 8) + b / 8 : b;
  int i = lb * kRW + wave;
  int qn = i < a.nq ? (a.order ? a.order[i] : i) : 0;
  for (; i < a.nq; i += stride) {
    const int q = __builtin_amdgcn_readfirstlane(qn);
    if (i + stride < a.nq) qn = a.order ? a.order[i + stride] : i + stride;  // the next query's index, early
    const float T = a.thr[q];
    const int cnt = __builtin_amdgcn_readfirstlane(a.cand_cnt[q]);
    if (!(T < INFINITY) || cnt > a.cand_cap) {
      if (lane == 0) {
        const int f = atomicAdd(&a.ctr[kCtrFlag], 1);
        a.flist[f] = q;
      }
      continue;
    }
    if constexpr (ONE) {
      const uint32_t l1 = a.probes[q];  // cnt > 0 only when it is a usable list
      for (int d = lane; d < D; d += kWave)
        qs[wave][d] = cnt > 0 ? a.queries[(size_t)(q / a.qdiv) * D + d] - a.centroids[(size_t)l1 * D + d] : 0.0f;
    } else {
      for (int d = lane; d < D; d += kWave) qs[wave][d] = a.queries[(size_t)(q / a.qdiv) * D + d];
    }
    wave_sync();
    const float* qv = qs[wave];
    uint64_t lk = kPadKey;
    for (int i0 = 0; i0 < cnt; i0 += kWave) {
      const int i = i0 + lane;
      uint64_t key = kPadKey;
      if (i < cnt) {
        const uint2 e = a.cand[(size_t)q * a.cand_cap + i];
        const int64_t pos = e.x;
        const float* cen = a.centroids + (size_t)(ONE ? 0 : e.y) * D;
        uint4 w[M / 16];
        load_codes<M>(a.codes, pos, w);
        const int id = a.vec_ids[pos];
        float dist = 0.0f;
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
          const uint32_t ww = mm % 16 < 4 ? w[mm / 16].x : mm % 16 < 8 ? w[mm / 16].y
                                                       : mm % 16 < 12 ? w[mm / 16].z : w[mm / 16].w;
          const uint32_t code = (ww >> (8 * (mm & 3))) & 0xFFu;
          float pr[S], r[S];
#pragma unroll
          for (int e2 = 0; e2 < S; ++e2) pr[e2] = cbf[(mm * kPQK + code) * S + e2];
          if constexpr (ONE) {
#pragma unroll
            for (int e2 = 0; e2 < S; ++e2) r[e2] = qv[mm * S + e2];
          } else {
            float cr[S];
            load_row<S>(cen + mm * S, cr);
#pragma unroll
            for (int e2 = 0; e2 < S; ++e2) r[e2] = qv[mm * S + e2] - cr[e2];
          }
          const float t = lut_entry<S>(r, pr);
          dist = mm == 0 ? t : dist + t;
        }
        key = key_of(dist, id);
      }
      wave_sort64_k(key);
      if (i0 == 0)
        lk = key;
      else
        wave_merge_sorted64_k(lk, key);
    }
    if (lane < a.k) {
      const int id = key_id(lk);
      const bool pad = id == kPadId;
      a.out_ids[(size_t)q * a.k + lane] = pad ? -1 : id;
      a.out_d[(size_t)q * a.k + lane] = pad ? FLT_MAX : key_dist(lk);
    }
    wave_sync();
  }
}

int cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

template <int D, int M>
fgpu_status launch_screen_dm(const ScreenArgs& a, hipStream_t s) {
  const int cus = cu_count();
  const int64_t nz = kCtrCount + 2 * (int64_t)a.nlist + (int64_t)a.nq;
  hipLaunchKernelGGL(screen_zero_kernel, dim3((unsigned)std::min<int64_t>((nz + 255) / 256, 2048)), dim3(256), 0, s,
                     a.ctr, nz);
  auto mark = [&](int i) { return a.events ? hipEventRecord(a.events[i], s) : hipSuccess; };
  hipLaunchKernelGGL(screen_pairs1_kernel<D>, dim3((unsigned)((a.nq + 3) / 4)), dim3(256), 0, s, a);
  FGPU_HIP(mark(0));
  if (screen_groups(a.k) == 64)
    hipLaunchKernelGGL((screen_kernel<D, M, 1, 64>), dim3((unsigned)cus), dim3(kSW * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((screen_kernel<D, M, 1>), dim3((unsigned)cus), dim3(kSW * kWave), 0, s, a);
  FGPU_HIP(mark(1));
  hipLaunchKernelGGL(screen_pairs2_kernel<D>, dim3((unsigned)((a.nq + 3) / 4)), dim3(256), 0, s, a);
  FGPU_HIP(mark(2));
  hipLaunchKernelGGL((screen_kernel<D, M, 2>), dim3((unsigned)cus), dim3(kSW * kWave), 0, s, a);
  FGPU_HIP(mark(3));
  if (a.nprobe == 1)
    hipLaunchKernelGGL((rescore_kernel<D, M, true>), dim3((unsigned)cus), dim3(kRW * kWave), 0, s, a);
  else
    hipLaunchKernelGGL((rescore_kernel<D, M, false>), dim3((unsigned)cus), dim3(kRW * kWave), 0, s, a);
  FGPU_HIP(mark(4));
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace

int64_t screen_gmin_words(int nq) {
  // Round 1: per query, per chunk of its first list, up to 64 group minima.
  return (int64_t)nq * kMaxChunks * kMaxGroups;
}

bool screen_supported(int dim, int m) {
  return (dim == 128 && (m == 16 || m == 32 || m == 64)) || (dim == 96 && m == 48);
}


fgpu_status launch_screen_prep(const float* codebook, int m, int sub, int scale_exp, const uint8_t* codes,
                               int64_t total, uint16_t* cb16, uint4* vext, unsigned int* xmax_bits, hipStream_t s) {
  const int64_t ncb = (int64_t)m * kPQK * sub;
  hipLaunchKernelGGL(cb_f16_kernel, dim3((unsigned)((ncb + 255) / 256)), dim3(256), 0, s, codebook, ncb, scale_exp,
                     cb16);
  FGPU_HIP(hipMemsetAsync(xmax_bits, 0, sizeof(unsigned int), s));
  if (total > 0)
    hipLaunchKernelGGL(screen_prep_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, codebook, m, sub,
                       scale_exp, codes, total, vext, xmax_bits);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_screen(int dim, int m, const ScreenArgs& a, hipStream_t s) {
  FGPU_CHECK(a.k >= 1 && a.k <= 64, FGPU_ERR_UNSUPPORTED, "screen: k must be in [1, 64]");
  FGPU_CHECK(a.r2_chunk >= kTV && a.r2_chunk % kTV == 0 && a.r2_max_chunks >= 1, FGPU_ERR_ARG,
             "screen: bad round-2 chunking");
  if (a.nq <= 0) return FGPU_OK;
  if (dim == 128 && m == 32) return launch_screen_dm<128, 32>(a, s);
  if (dim == 128 && m == 16) return launch_screen_dm<128, 16>(a, s);
  if (dim == 128 && m == 64) return launch_screen_dm<128, 64>(a, s);
  if (dim == 96 && m == 48) return launch_screen_dm<96, 48>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "screen: unsupported (dim, pq_m)");
}

}  // namespace fgpu
