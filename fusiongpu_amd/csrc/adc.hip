// adc.hip -- per-query LUT build in LDS, ADC scan over the probed inverted
// lists and top-k selection (A4, A5, A6, A10 in plain IVF-PQ form).
//
// Reference: batch_residual_precompute_kernel (gpu_global.cu:79-166) writes
// every (query, probe) LUT to global memory; ivf_scan_phase1_kernel
// (gpu_global.cu:321-390) scans at most 1024 items of a list per block and
// sorts them with a CUB block radix sort; a segmented radix sort then orders
// the union (gpu_global.cu:852-861).
//
// Here one workgroup owns one query and walks its probed lists in coarse
// order:
//   * LUT[m][k] lives in LDS ([m][256] floats).  The threads that build it
//     keep the codebook sub-vectors of their codeword in registers for the
//     whole query, so the codebook is read from HBM once per workgroup.
//     Entries use the reference's exact fused chains (gpu_global.cu:115-158),
//     so they are bit-identical.
//   * The scan streams each vector's pq_m code bytes with 128-bit loads, two
//     vectors per lane per round (two independent ADC chains in flight).  Each
//     distance sums LUT[m][code_m] in ascending m as the reference does
//     (gpu_global.cu:196-253): one SDWA byte-to-address shift and one
//     ds_read_b32 with an immediate row offset per term.
//   * Each scanning wave keeps its own running top-64 (one (distance, id) per
//     lane, sorted by the tie rule).  A vector is a candidate only if it beats
//     the wave's k-th entry; after the first list almost nothing passes, so
//     the selection costs one compare per vector.  Few passers are inserted
//     one by one; many are bitonic-sorted and merged.  At the end the wave
//     lists are merged in LDS.
//   * adc_spec_kernel (pq_m <= 32): 16 waves, 8 build LUT(p+1) into one LDS
//     buffer while 8 scan list p out of the other; one barrier per list.
//     adc_plain_kernel (pq_m 48, 64): 8 waves alternate build and scan.
#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {
namespace {

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

// Offer one distance per lane to the wave's running top-k.
__device__ __forceinline__ void offer(float d, bool valid, int vid_index, const int32_t* __restrict__ ids, int k,
                                      float& ld, int& li, float& thr_d, int& thr_i) {
  const bool cand = valid && d <= thr_d;
  if (__ballot(cand)) {
    const int id = cand ? ids[vid_index] : kPadId;
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
}

// Each scanning wave takes 128 consecutive vectors per round (two per lane).
constexpr int kVecPerWaveRound = 2 * kWave;

template <int M>
__device__ __forceinline__ void load_pair(const uint8_t* __restrict__ codes, int start, int n, int v0,
                                          uint4 (&w0)[M / 16], uint4 (&w1)[M / 16]) {
  if (v0 < n) load_codes<M>(codes, (int64_t)start + v0, w0);
  if (v0 + kWave < n) load_codes<M>(codes, (int64_t)start + v0 + kWave, w1);
}

// Scan one list with the LUT at a compile-time LDS position.  w0/w1 hold the
// codes of this wave's first round (loaded by the caller ahead of time); with
// PREFETCH later rounds are loaded one round ahead, otherwise at round start.
template <int D, int M, int BUF, int SCAN_WAVES, bool PREFETCH>
__device__ __forceinline__ void scan_list(const float* smem, const uint8_t* __restrict__ codes,
                                          const int32_t* __restrict__ ids, int start, int n, int k, int swave,
                                          uint4 (&w0)[M / 16], uint4 (&w1)[M / 16], float& ld, int& li,
                                          float& thr_d, int& thr_i) {
  using C = Cfg<D, M>;
  constexpr int kRound = SCAN_WAVES * kVecPerWaveRound;
  const float* lut = smem + BUF * C::LUT;
  const int lane = threadIdx.x & 63;
  for (int base = swave * kVecPerWaveRound; base < n; base += kRound) {
    const int v0 = base + lane, v1 = v0 + kWave;
    uint4 n0[C::NV4], n1[C::NV4];
    const bool more = base + kRound < n;
    if (PREFETCH) {
      if (more) load_pair<M>(codes, start, n, v0 + kRound, n0, n1);
    } else if (base != swave * kVecPerWaveRound) {
      load_pair<M>(codes, start, n, v0, w0, w1);
    }
    const float d0 = v0 < n ? adc_sum<M>(lut, w0) : FLT_MAX;
    const float d1 = v1 < n ? adc_sum<M>(lut, w1) : FLT_MAX;
    offer(d0, v0 < n, start + v0, ids, k, ld, li, thr_d, thr_i);
    offer(d1, v1 < n, start + v1, ids, k, ld, li, thr_d, thr_i);
    if (PREFETCH && more) {
#pragma unroll
      for (int i = 0; i < C::NV4; ++i) { w0[i] = n0[i]; w1[i] = n1[i]; }
    }
  }
}

// Merge `nw` sorted wave lists held in LDS (md/mi, 64 entries each) into this
// wave's registers and write the k best.
__device__ __forceinline__ void merge_and_write(float ld, int li, const float* md, const int* mi, int nw, int q, int k,
                                                const AdcArgs& a) {
  const int lane = threadIdx.x & 63;
#pragma unroll 1
  for (int w = 1; w < nw; ++w) wave_merge_sorted64(ld, li, md[w * kWave + lane], mi[w * kWave + lane]);
  if (lane < k) {
    const bool pad = li == kPadId;
    a.out_ids[(size_t)q * k + lane] = pad ? -1 : li;
    a.out_d[(size_t)q * k + lane] = pad ? FLT_MAX : ld;
  }
}

// ---------------------------------------------------------------------------
// Generic kernel: 8 waves build the LUT together (thread t owns codeword t%256
// for half of the subspaces), then all 8 scan.
constexpr int kNW = 8;
constexpr int kNT = kNW * kWave;

template <int D, int M>
__global__ __launch_bounds__(kNT) void adc_plain_kernel(AdcArgs a) {
  using C = Cfg<D, M>;
  constexpr int G = kNT / kPQK;  // threads sharing one codeword
  constexpr int MG = M / G;      // subspaces per thread
  static_assert(M % G == 0, "pq_m must split across the codeword threads");
  __shared__ __align__(16) float smem[C::SMEM];
  float* rbuf = smem + C::R_OFF;
  float* qs = smem + C::Q_OFF;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = tid & (kPQK - 1), g = tid / kPQK;
  const int q = blockIdx.x;
  const int P = a.nprobe, k = a.k;
  const uint32_t NL = (uint32_t)a.nlist;

  float cb[MG * C::S];
#pragma unroll
  for (int mm = 0; mm < MG; ++mm) {
    const float* src = a.codebook + ((size_t)(g * MG + mm) * kPQK + kc) * C::S;
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
  uint4 w0[C::NV4], w1[C::NV4];
  while (p < P) {
    const uint32_t l = probes[p];
    int pn = p + 1;
    while (pn < P && probes[pn] >= NL) ++pn;
    const int start = a.offsets[l];
    const int n = a.offsets[l + 1] - start;
    // First-round code loads go out before the LUT build, which hides their latency.
    load_pair<M>(a.codes, start, n, wave * kVecPerWaveRound + lane, w0, w1);
    const int buf = C::DBUF ? (it & 1) : 0;
    float* lut = smem + buf * C::LUT;
    const float* r = rbuf + (it & 1) * D;
#pragma unroll
    for (int mm = 0; mm < MG; ++mm) {
      const int m = g * MG + mm;
      float rr[C::S];
#pragma unroll
      for (int j = 0; j < C::S; ++j) rr[j] = r[m * C::S + j];
      lut[m * kPQK + kc] = lut_entry<C::S>(rr, cb + mm * C::S);
    }
    if (pn < P && tid < D) rbuf[((it + 1) & 1) * D + tid] = qs[tid] - a.centroids[(size_t)probes[pn] * D + tid];
    __syncthreads();
    if (buf == 0)
      scan_list<D, M, 0, kNW, false>(smem, a.codes, a.vec_ids, start, n, k, wave, w0, w1, ld, li, thr_d, thr_i);
    else
      scan_list<D, M, (C::DBUF ? 1 : 0), kNW, false>(smem, a.codes, a.vec_ids, start, n, k, wave, w0, w1, ld, li,
                                                    thr_d, thr_i);
    if (!C::DBUF) __syncthreads();
    p = pn;
    ++it;
  }

  __syncthreads();
  float* md = smem;
  int* mi = reinterpret_cast<int*>(smem + kNW * kWave);
  md[wave * kWave + lane] = ld;
  mi[wave * kWave + lane] = li;
  __syncthreads();
  if (wave == 0) merge_and_write(ld, li, md, mi, kNW, q, k, a);
}

// ---------------------------------------------------------------------------
// Wave-specialised kernel (two LUTs within the 64 KiB DS-offset reach).
// 16 waves: waves 0-7 build LUTs (the codebook lives in their registers),
// waves 8-15 scan.  Phase f: builders write LUT(f) into buffer f&1 while
// scanners scan list f-1 out of buffer (f-1)&1; one barrier ends the phase.
constexpr int kSpecWaves = 16;
constexpr int kBuilderWaves = 8;
constexpr int kScanWaves = kSpecWaves - kBuilderWaves;

template <int D, int M>
__global__ __launch_bounds__(kSpecWaves * kWave, 4) void adc_spec_kernel(AdcArgs a) {
  using C = Cfg<D, M>;
  static_assert(C::DBUF, "wave-specialised kernel needs two LUTs within the DS offset reach");
  constexpr int MB = M / 2;  // subspaces per builder thread (512 builder threads, 2 per codeword)
  __shared__ __align__(16) float smem[C::SMEM];
  __shared__ int plist[64];
  __shared__ int pcount;
  float* rbuf = smem + C::R_OFF;
  float* qs = smem + C::Q_OFF;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool builder = wave < kBuilderWaves;
  const int kc = tid & (kPQK - 1), g = (tid >> 8) & 1;
  const int swave = wave - kBuilderWaves;
  const int q = blockIdx.x;
  const int P = a.nprobe, k = a.k;
  const uint32_t NL = (uint32_t)a.nlist;

  for (int i = tid; i < D; i += kSpecWaves * kWave) qs[i] = a.queries[(size_t)q * D + i];
  if (tid == 0) {
    int c = 0;
    for (int p = 0; p < P; ++p) {
      const uint32_t l = a.probes[(size_t)q * P + p];
      if (l < NL) plist[c++] = (int)l;  // pruned (0xFFFFFFFF) or out-of-range probes are skipped
    }
    pcount = c;
  }
  __syncthreads();
  const int nv = pcount;
  if (nv > 0 && tid < D) rbuf[tid] = qs[tid] - a.centroids[(size_t)plist[0] * D + tid];
  __syncthreads();

  float ld = FLT_MAX;
  int li = kPadId;
  // The two roles run separate loops with the same barrier count (nv + 1), so
  // the register allocator can give the codebook and the scan state the same
  // physical registers.
  if (builder) {
    float cb[MB * C::S];
#pragma unroll
    for (int mm = 0; mm < MB; ++mm) {
      const float* src = a.codebook + ((size_t)(g * MB + mm) * kPQK + kc) * C::S;
#pragma unroll
      for (int j = 0; j < C::S; ++j) cb[mm * C::S + j] = src[j];
    }
    for (int f = 0; f <= nv; ++f) {
      if (f < nv) {
        float* lut = smem + (f & 1) * C::LUT;
        const float* r = rbuf + (f & 1) * D;
#pragma unroll
        for (int mm = 0; mm < MB; ++mm) {
          const int m = g * MB + mm;
          float rr[C::S];
#pragma unroll
          for (int j = 0; j < C::S; ++j) rr[j] = r[m * C::S + j];
          lut[m * kPQK + kc] = lut_entry<C::S>(rr, cb + mm * C::S);
        }
        if (f + 1 < nv && tid < D)
          rbuf[((f + 1) & 1) * D + tid] = qs[tid] - a.centroids[(size_t)plist[f + 1] * D + tid];
      }
      __syncthreads();
    }
  } else {
    float thr_d = FLT_MAX;
    int thr_i = kPadId;
    uint4 w0[C::NV4], w1[C::NV4];
    if (nv > 0) {
      const int l0 = plist[0];
      load_pair<M>(a.codes, a.offsets[l0], a.offsets[l0 + 1] - a.offsets[l0], swave * kVecPerWaveRound + lane, w0, w1);
    }
    for (int f = 0; f <= nv; ++f) {
      if (f >= 1) {
        const int l = plist[f - 1];
        const int start = a.offsets[l], n = a.offsets[l + 1] - start;
        if ((f - 1) & 1)
          scan_list<D, M, 1, kScanWaves, true>(smem, a.codes, a.vec_ids, start, n, k, swave, w0, w1, ld, li, thr_d,
                                               thr_i);
        else
          scan_list<D, M, 0, kScanWaves, true>(smem, a.codes, a.vec_ids, start, n, k, swave, w0, w1, ld, li, thr_d,
                                               thr_i);
        if (f < nv) {  // first-round codes of the next list land while this phase's barrier waits
          const int l2 = plist[f];
          load_pair<M>(a.codes, a.offsets[l2], a.offsets[l2 + 1] - a.offsets[l2], swave * kVecPerWaveRound + lane,
                       w0, w1);
        }
      }
      __syncthreads();
    }
  }

  // Merge the scanner waves' lists.
  float* md = smem;
  int* mi = reinterpret_cast<int*>(smem + kScanWaves * kWave);
  if (!builder) {
    md[swave * kWave + lane] = ld;
    mi[swave * kWave + lane] = li;
  }
  __syncthreads();
  if (wave == kBuilderWaves) merge_and_write(ld, li, md, mi, kScanWaves, q, k, a);
}

template <int D, int M>
fgpu_status launch_plain(const AdcArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((adc_plain_kernel<D, M>), dim3((unsigned)a.nq), dim3(kNT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

template <int D, int M>
fgpu_status launch_spec(const AdcArgs& a, hipStream_t s) {
  FGPU_CHECK(a.nprobe <= 64, FGPU_ERR_UNSUPPORTED, "adc: nprobe must be <= 64");
  hipLaunchKernelGGL((adc_spec_kernel<D, M>), dim3((unsigned)a.nq), dim3(kSpecWaves * kWave), 0, s, a);
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
  if (dim == 128 && m == 32) return launch_spec<128, 32>(a, s);
  if (dim == 128 && m == 16) return launch_spec<128, 16>(a, s);
  if (dim == 128 && m == 64) return launch_plain<128, 64>(a, s);
  if (dim == 96 && m == 48) return launch_plain<96, 48>(a, s);
  if (dim == 96 && m == 32) return launch_spec<96, 32>(a, s);
  if (dim == 96 && m == 16) return launch_spec<96, 16>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "adc: unsupported (dim, pq_m)");
}

}  // namespace fgpu
