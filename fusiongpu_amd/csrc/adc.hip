// adc.hip -- per-query LUT build in LDS, ADC scan over the probed inverted
// lists and top-k selection (A4, A5, A6, A10 in plain IVF-PQ form).
//
// Reference: batch_residual_precompute_kernel (gpu_global.cu:79-166) writes
// every (query, probe) LUT to global memory; ivf_scan_phase1_kernel
// (gpu_global.cu:321-390) scans at most 1024 items of a list per block and
// sorts them with a CUB block radix sort; a segmented radix sort then orders
// the union (gpu_global.cu:852-861).
//
// Here one workgroup (8 waves) owns one query and walks its probed lists in
// coarse order:
//   * LUT[m][k] lives in LDS ([m][256] floats).  Thread t builds the entries
//     of codeword k = t % 256 for its half of the subspaces; that codeword's
//     sub-vectors stay in registers for the whole query, so the codebook is
//     read from HBM once per workgroup.  Entries use the reference's exact
//     fused chains (gpu_global.cu:115-158), so they are bit-identical.
//   * When two LUTs fit under the 64 KiB reach of the DS immediate offset
//     (pq_m <= 32 at dim 128) they are double-buffered: one barrier per probe.
//   * The scan streams each vector's pq_m code bytes with 128-bit loads
//     (prefetching the next round), and sums LUT[m][code_m] in ascending m as
//     the reference does (gpu_global.cu:196-253): one SDWA byte-to-address
//     shift and one ds_read_b32 with an immediate row offset per term.
//   * Each wave keeps its own running top-64 (one (distance, id) per lane,
//     sorted by the tie rule).  A vector is a candidate only if it beats the
//     wave's k-th entry; after the first list almost nothing passes, so the
//     selection costs one compare per vector.  Few passers are inserted one
//     by one; many are bitonic-sorted and merged.  At the end the 8 wave lists
//     are merged in LDS.
#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {
namespace {

constexpr int kNW = 8;  // waves per workgroup
constexpr int kNT = kNW * kWave;
constexpr int kSerialMax = 12;  // passers up to this count are inserted one by one

template <int D, int M>
struct Cfg {
  static constexpr int S = D / M;
  static constexpr int G = kNT / kPQK;  // threads sharing one codeword
  static constexpr int MG = M / G;      // subspaces per thread in the LUT build
  static constexpr int LUT = M * kPQK;  // floats per LUT
  static constexpr bool DBUF = 2 * LUT * 4 <= 65536;
  static constexpr int NBUF = DBUF ? 2 : 1;
  static constexpr int R_OFF = NBUF * LUT;      // residual double buffer [2][D]
  static constexpr int Q_OFF = R_OFF + 2 * D;   // query [D]
  static constexpr int SMEM = Q_OFF + D;
  static constexpr int NV4 = M / 16;            // 128-bit code loads per vector
  static_assert(D % M == 0, "dim must be a multiple of pq_m");
  static_assert(M % 16 == 0, "pq_m must be a multiple of 16");
  static_assert(M % G == 0, "pq_m must split across the codeword threads");
  static_assert(LUT >= 2 * kNW * kWave, "merge area must fit in the LUT area");
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

// Scan one list with the LUT at a compile-time LDS position.
template <int D, int M, int BUF>
__device__ __forceinline__ void scan_list(const float* smem, const uint8_t* __restrict__ codes,
                                          const int32_t* __restrict__ ids, int start, int n, int k,
                                          float& ld, int& li, float& thr_d, int& thr_i) {
  using C = Cfg<D, M>;
  const float* lut = smem + BUF * C::LUT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int v = wave * kWave + lane;
  uint4 w[C::NV4], wn[C::NV4];
  if (v < n) load_codes<M>(codes, (int64_t)start + v, w);
  for (int base = wave * kWave; base < n; base += kNT) {
    const int vn = v + kNT;
    if (vn < n) load_codes<M>(codes, (int64_t)start + vn, wn);
    float d = FLT_MAX;
    if (v < n) d = adc_sum<M>(lut, w);
    const bool cand = v < n && d <= thr_d;
    if (__ballot(cand)) {
      const int id = cand ? ids[start + v] : kPadId;
      const bool pass = cand && lt_pair(d, id, thr_d, thr_i);
      uint64_t bm = __ballot(pass);
      if (bm) {
        if (__popcll(bm) > kSerialMax) {
          float cd = pass ? d : FLT_MAX;
          int ci = pass ? id : kPadId;
          wave_sort64(cd, ci);
          wave_merge_sorted64(ld, li, cd, ci);
        } else {
          while (bm) {
            const int src = __ffsll((unsigned long long)bm) - 1;
            bm &= bm - 1;
            wave_insert64(ld, li, readlane_f(d, src), readlane_i(id, src));
          }
        }
        thr_d = readlane_f(ld, k - 1);
        thr_i = readlane_i(li, k - 1);
      }
    }
#pragma unroll
    for (int i = 0; i < C::NV4; ++i) w[i] = wn[i];
    v = vn;
  }
}

template <int D, int M>
__global__ __launch_bounds__(kNT) void adc_plain_kernel(AdcArgs a) {
  using C = Cfg<D, M>;
  __shared__ __align__(16) float smem[C::SMEM];
  float* rbuf = smem + C::R_OFF;
  float* qs = smem + C::Q_OFF;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = tid & (kPQK - 1), g = tid / kPQK;
  const int q = blockIdx.x;
  const int P = a.nprobe, k = a.k;
  const uint32_t NL = (uint32_t)a.nlist;

  // This thread's codeword sub-vectors for its subspaces, resident for the query.
  float cb[C::MG * C::S];
#pragma unroll
  for (int mm = 0; mm < C::MG; ++mm) {
    const float* src = a.codebook + ((size_t)(g * C::MG + mm) * kPQK + kc) * C::S;
#pragma unroll
    for (int j = 0; j < C::S; ++j) cb[mm * C::S + j] = src[j];
  }
  for (int i = tid; i < D; i += kNT) qs[i] = a.queries[(size_t)q * D + i];
  const uint32_t* probes = a.probes + (size_t)q * P;
  __syncthreads();

  int p = 0;
  while (p < P && probes[p] >= NL) ++p;  // pruned (0xFFFFFFFF) or out of range
  if (p < P && tid < D) rbuf[tid] = qs[tid] - a.centroids[(size_t)probes[p] * D + tid];
  __syncthreads();

  float ld = FLT_MAX, thr_d = FLT_MAX;
  int li = kPadId, thr_i = kPadId;
  int it = 0;
  while (p < P) {
    const uint32_t l = probes[p];
    int pn = p + 1;
    while (pn < P && probes[pn] >= NL) ++pn;
    const int buf = C::DBUF ? (it & 1) : 0;
    float* lut = smem + buf * C::LUT;
    const float* r = rbuf + (it & 1) * D;
#pragma unroll
    for (int mm = 0; mm < C::MG; ++mm) {
      const int m = g * C::MG + mm;
      float rr[C::S];
#pragma unroll
      for (int j = 0; j < C::S; ++j) rr[j] = r[m * C::S + j];
      lut[m * kPQK + kc] = lut_entry<C::S>(rr, cb + mm * C::S);
    }
    if (pn < P && tid < D) rbuf[((it + 1) & 1) * D + tid] = qs[tid] - a.centroids[(size_t)probes[pn] * D + tid];
    __syncthreads();
    const int start = a.offsets[l];
    const int n = a.offsets[l + 1] - start;
    if (buf == 0) scan_list<D, M, 0>(smem, a.codes, a.vec_ids, start, n, k, ld, li, thr_d, thr_i);
    else scan_list<D, M, (C::DBUF ? 1 : 0)>(smem, a.codes, a.vec_ids, start, n, k, ld, li, thr_d, thr_i);
    if (!C::DBUF) __syncthreads();
    p = pn;
    ++it;
  }

  // Merge the per-wave lists.
  __syncthreads();
  float* md = smem;
  int* mi = reinterpret_cast<int*>(smem + kNW * kWave);
  md[wave * kWave + lane] = ld;
  mi[wave * kWave + lane] = li;
  __syncthreads();
  if (wave == 0) {
#pragma unroll 1
    for (int w = 1; w < kNW; ++w) wave_merge_sorted64(ld, li, md[w * kWave + lane], mi[w * kWave + lane]);
    if (lane < k) {
      const bool pad = li == kPadId;
      a.out_ids[(size_t)q * k + lane] = pad ? -1 : li;
      a.out_d[(size_t)q * k + lane] = pad ? FLT_MAX : ld;
    }
  }
}

template <int D, int M>
fgpu_status launch_t(const AdcArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((adc_plain_kernel<D, M>), dim3((unsigned)a.nq), dim3(kNT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace

bool adc_supported(int dim, int m) {
  return (dim == 128 && (m == 16 || m == 32 || m == 64)) || (dim == 96 && (m == 16 || m == 32 || m == 48));
}

fgpu_status launch_adc_plain(int dim, int m, const AdcArgs& a, hipStream_t s) {
  FGPU_CHECK(a.k >= 1 && a.k <= 64, FGPU_ERR_UNSUPPORTED, "adc: k must be in [1, 64]");
  if (a.nq <= 0) return FGPU_OK;
  if (dim == 128 && m == 32) return launch_t<128, 32>(a, s);
  if (dim == 128 && m == 16) return launch_t<128, 16>(a, s);
  if (dim == 128 && m == 64) return launch_t<128, 64>(a, s);
  if (dim == 96 && m == 48) return launch_t<96, 48>(a, s);
  if (dim == 96 && m == 32) return launch_t<96, 32>(a, s);
  if (dim == 96 && m == 16) return launch_t<96, 16>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "adc: unsupported (dim, pq_m)");
}

}  // namespace fgpu
