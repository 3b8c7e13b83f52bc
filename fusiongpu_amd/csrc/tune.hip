// tune.hip -- statistics for the offline parameter tuner (tune_parameters).
//
// Reference: tune_search_parameters (tune_parameters.cu:459-1012).  For each
// ground-truth neighbour the reference copies its list to the GPU with a
// cudaMalloc per item, builds a LUT with precompute_lut_kernel (:101-123),
// sums it with compute_pq_dist_with_lut_kernel (:127-145), computes exact
// distances with compute_exact_distances_kernel (:148-166), copies everything
// back and ranks on the host (:755-784); the threshold step does the same per
// phase-1 list and sorts the PQ distances on the host for the limit_k-th one
// (:855-903).  Here one workgroup handles one (query, list) pair entirely on
// the device: LUT in LDS, the target's distances, both ranks and the k-th
// smallest PQ distance (an exact radix select), with no host round trip.
//
// Floating-point forms (the reference's kernels built by nvcc, which fuses
// `dist += diff * diff`):
//   * tuner LUT entry: r = q - c per coordinate, diff = r - codeword, then a
//     sequential fused chain dist = fma(diff, diff, dist) from 0 over the
//     sub-vector (precompute_lut_kernel; this is not the search LUT's chain);
//   * PQ distance: ascending sum over subspaces of LUT[m][code_m];
//   * exact distance: sequential fused chain over all dimensions of q - x.
#include <algorithm>
#include <cmath>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {
namespace {

constexpr int kTuneThreads = 256;
constexpr int kTuneMaxDim = 128;

__device__ __forceinline__ void block_sync() { __syncthreads(); }

// Sum of a per-thread int over the workgroup (all threads get the result).
__device__ int block_sum(int v, int* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_i(v);
  if (lane == 0) red[wave] = v;
  block_sync();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kTuneThreads / kWave; ++w) t += red[w];
  block_sync();
  return t;
}

__global__ __launch_bounds__(kTuneThreads) void tune_list_stats_kernel(TuneStatsArgs a) {
  __shared__ float lut[kMaxTuneLut];
  __shared__ float qs[kTuneMaxDim], rs[kTuneMaxDim];
  __shared__ uint32_t hist[256];
  __shared__ int red[kTuneThreads / kWave];
  __shared__ int s_pos;
  __shared__ uint32_t s_prefix;
  __shared__ int s_rem;
  const int p = blockIdx.x, tid = threadIdx.x;
  const int D = a.dim, M = a.pq_m, S = D / M;
  const int qi = a.pair_query[p], l = a.pair_list[p], target = a.pair_target ? a.pair_target[p] : -1;
  const int kth = a.pair_kth ? a.pair_kth[p] : 0;
  if (qi < 0 || qi >= a.nq || l < 0 || l >= a.nlist) {  // a pair outside the inputs: nothing to measure
    if (tid == 0) {
      if (a.pair_target) {
        a.target_pq[p] = -1.0f;
        a.target_exact[p] = -1.0f;
        a.pq_rank[p] = 0;
        a.exact_rank[p] = 0;
      }
      if (a.pair_kth) a.kth_pq[p] = 0.0f;
    }
    return;  // uniform over the workgroup: no barrier is skipped by part of it
  }
  const int start = a.offsets[l], n = a.offsets[l + 1] - start;
  for (int d = tid; d < D; d += kTuneThreads) {
    const float qv = a.queries[(size_t)qi * D + d];
    qs[d] = qv;
    rs[d] = qv - a.centroids[(size_t)l * D + d];
  }
  if (tid == 0) s_pos = INT_MAX;
  block_sync();
  // Tuner LUT: thread t owns codeword t of every subspace.
  for (int m = 0; m < M; ++m) {
    const float* cw = a.codebook + ((size_t)m * kPQK + tid) * S;
    float dist = 0.0f;
    for (int d = 0; d < S; ++d) {
      const float diff = rs[m * S + d] - cw[d];
      dist = __builtin_fmaf(diff, diff, dist);
    }
    lut[m * kPQK + tid] = dist;
  }
  // First position of the target id in the list.
  if (target >= 0)
    for (int j = tid; j < n; j += kTuneThreads)
      if (a.ids[start + j] == target) atomicMin(&s_pos, j);
  block_sync();
  const uint8_t* codes = a.codes + (size_t)start * M;
  auto pq_dist = [&](int j) {
    const uint8_t* c = codes + (size_t)j * M;
    float s = 0.0f;
    for (int m = 0; m < M; ++m) s += lut[m * kPQK + c[m]];
    return s;
  };
  auto exact_dist = [&](int j) {
    const int id = a.ids[start + j];
    if (id < 0 || (long long)id >= a.n_base) return __builtin_inff();  // no raw vector: never below
    const float* x = a.base + (size_t)id * D;
    float s = 0.0f;
    for (int d = 0; d < D; ++d) {
      const float diff = qs[d] - x[d];
      s = __builtin_fmaf(diff, diff, s);
    }
    return s;
  };

  const int pos = s_pos;
  if (a.pair_target) {
    // Ranks: 1 + the list's vectors strictly below the target (tune_parameters.cu:766-778).
    const bool found = target >= 0 && pos != INT_MAX;
    const float tp = found ? pq_dist(pos) : 0.0f;
    const bool use_exact = a.base != nullptr && found;
    const float te = use_exact ? exact_dist(pos) : 0.0f;
    int below_pq = 0, below_ex = 0;
    if (found)
      for (int j = tid; j < n; j += kTuneThreads) {
        below_pq += pq_dist(j) < tp;
        if (use_exact) below_ex += exact_dist(j) < te;
      }
    below_pq = block_sum(below_pq, red);
    below_ex = block_sum(below_ex, red);
    if (tid == 0) {
      a.target_pq[p] = found ? tp : -1.0f;
      a.target_exact[p] = use_exact ? te : -1.0f;
      a.pq_rank[p] = found ? below_pq + 1 : 0;
      a.exact_rank[p] = use_exact ? below_ex + 1 : 0;
    }
  }

  if (kth > 0) {
    // The min(kth, n)-th smallest PQ distance of the list (:893-899), by an
    // MSB-first radix select over the bit patterns (distances are >= 0, so
    // their bits order like the floats).
    float out = 0.0f;
    if (n > 0) {
      if (tid == 0) {
        s_prefix = 0u;
        s_rem = (kth < n ? kth : n);
      }
      for (int shift = 24; shift >= 0; shift -= 8) {
        hist[tid] = 0u;
        block_sync();
        const uint32_t prefix = s_prefix;
        for (int j = tid; j < n; j += kTuneThreads) {
          const uint32_t key = __float_as_uint(pq_dist(j));
          const bool match = shift == 24 || ((key ^ prefix) >> (shift + 8)) == 0u;
          if (match) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        block_sync();
        if (tid == 0) {
          int rem = s_rem;
          uint32_t b = 0;
          for (; b < 255u; ++b) {
            if ((int)hist[b] >= rem) break;
            rem -= (int)hist[b];
          }
          s_prefix = prefix | (b << shift);
          s_rem = rem;
        }
        block_sync();
      }
      out = __uint_as_float(s_prefix);
    }
    if (tid == 0) a.kth_pq[p] = out;
  }
}

}  // namespace

fgpu_status launch_tune_list_stats(const TuneStatsArgs& a, int npairs, hipStream_t s) {
  FGPU_CHECK(a.dim >= 1 && a.dim <= kTuneMaxDim && a.pq_m >= 1 && a.dim % a.pq_m == 0 &&
                 a.pq_m * kPQK <= kMaxTuneLut,
             FGPU_ERR_UNSUPPORTED, "tune_list_stats: need dim <= 128, pq_m | dim, pq_m <= 64");
  if (npairs <= 0) return FGPU_OK;
  hipLaunchKernelGGL(tune_list_stats_kernel, dim3((unsigned)npairs), dim3(kTuneThreads), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace fgpu

namespace fgpu {
namespace {
// compute_percentile / compute_percentile_int (tune_parameters.cu:170-183):
// the sorted sample's element at floor(size * pct) with the product taken in
// single precision, clamped to the last element; 0 for an empty sample.
template <class T>
T percentile_of(const T* v, int64_t n, float pct) {
  if (n <= 0) return T(0);
  std::vector<T> d(v, v + n);
  std::sort(d.begin(), d.end());
  long long idx = (long long)((float)(size_t)n * pct);
  if (idx >= (long long)n) idx = n - 1;
  if (idx < 0) idx = 0;
  return d[(size_t)idx];
}
}  // namespace
}  // namespace fgpu

extern "C" {

int fgpu_tune_percentile_int(const int32_t* values, int64_t n, float pct) {
  return fgpu::percentile_of<int32_t>(values, n, pct);
}

float fgpu_tune_percentile(const float* values, int64_t n, float pct) {
  return fgpu::percentile_of<float>(values, n, pct);
}

// find_elbow_point (tune_parameters.cu:199-456) without its printed tables.
// Scores each list count i + 1 (i = 2 .. min(n - 2, 29)) whose cumulative
// coverage of the hits is >= 0.6:
//   |curvature of the 3-point-smoothed log(hits + 1)| * 10
//   + 8 * (relative drop before - relative drop after) when the drop slows
//   + 4 * (1 - (i / 32)^2)
//   - 5 where the raw hits change direction at i;
// the best score among coverage >= 0.8 wins (first on ties), else the first
// count with coverage >= 0.6.  Single-precision arithmetic throughout, as the
// reference's host code.
int fgpu_tune_elbow(const int32_t* hits, int n, int64_t total_hits, float* coverage_out) {
  if (coverage_out) *coverage_out = 0.0f;
  if (n <= 0 || total_hits == 0 || !hits) return 1;
  std::vector<float> cov(n), lg(n), sm(n), curv(n, 0.0f), vol(n, 0.0f);
  long long cum = 0;
  for (int i = 0; i < n; ++i) {
    cum += hits[i];
    cov[i] = static_cast<float>(cum) / (float)total_hits;
    lg[i] = std::log(hits[i] + 1.0f);
  }
  for (int i = 0; i < n; ++i)
    sm[i] = (i == 0 || i == n - 1) ? lg[i] : 0.25f * lg[i - 1] + 0.50f * lg[i] + 0.25f * lg[i + 1];
  for (int i = 1; i + 1 < n; ++i) curv[i] = sm[i + 1] - 2.0f * sm[i] + sm[i - 1];
  for (int i = 1; i < n - 1; ++i) {
    const float d1 = (float)(hits[i - 1] - hits[i]), d2 = (float)(hits[i] - hits[i + 1]);
    if (d1 * d2 < 0) vol[i] = 1.0f;
  }
  int best = -1;
  float best_score = -1e9f;
  for (int i = 2; i + 1 < n && i < 30; ++i) {
    if (cov[i] < 0.60f) continue;
    const float curvature_score = std::fabs(curv[i]) * 10.0f;
    const float drop_before = (float)(hits[i - 1] - hits[i]) / (hits[i - 1] + 1.0f);
    const float drop_after = (float)(hits[i] - hits[i + 1]) / (hits[i] + 1.0f);
    const float drop_score = drop_after < drop_before ? (drop_before - drop_after) * 8.0f : 0.0f;
    const float penalty = vol[i] * 5.0f;
    const float ratio = (float)i / 32.0f;
    const float bonus = 4.0f * (1.0f - ratio * ratio);
    const float score = curvature_score + drop_score + bonus - penalty;
    if (cov[i] >= 0.80f && score > best_score) {
      best_score = score;
      best = i;
    }
  }
  if (best >= 0) {
    if (coverage_out) *coverage_out = cov[best];
    return best + 1;
  }
  for (int i = 0; i < n; ++i)
    if (cov[i] >= 0.60f) {
      if (coverage_out) *coverage_out = cov[i];
      return i + 1;
    }
  return 1;
}

}  // extern "C"
