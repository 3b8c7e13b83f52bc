// graph.hip -- graph (CAGRA-style) search over a fixed-degree adjacency array
// (A19).
//
// Reference: search_cagra_index (cagra_adapter.cuh:38-68) calls cuVS CAGRA
// with an internal top-k list of itopk entries, a search width and a maximum
// iteration count.  cuVS is not in the repository, so the algorithm here is
// stated on its own (the oracle restates the same definition):
//   * 64 seed nodes, node_j = mix64(seed ^ mix64((q << 20) | j)) % n;
//   * each step expands the `width` best not-yet-expanded entries of the
//     itopk list and offers their `degree` neighbours;
//   * a candidate is dropped if its id is outside [0, n) or its bit in the
//     query's visited bitmap was set before the step (2^16 bits, bit =
//     (uint32)(id * 2654435761) >> 16; a hash collision drops a node);
//     duplicates within the step are kept once; then the kept candidates'
//     bits are set;
//   * kept candidates get the exact device-form L2 and merge into the list by
//     (distance, id); the search stops when nothing is left to expand or after
//     max_iter steps.
// Reading the bitmap as it was before the step makes the result independent
// of the order in which lanes set bits.
//
// One wave per query, 4 queries per workgroup: the itopk list is one entry per
// lane (with its expanded flag), the bitmap (8 KB) sits in the wave's LDS, and
// a step's <= 128 candidates are two per lane.  Every sort and merge is a
// DPP/permlane bitonic network; there is no workgroup barrier.  The kept
// candidates' rows are read eight lanes a row and handed to their lanes
// through LDS (wave_rows_l2), so each distance is still one lane's sequential
// chain.
#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {
namespace {

constexpr int kGW = 4;                  // queries (waves) per workgroup
constexpr int kBitmapWords = 1 << 11;   // 2^16 bits per query
constexpr int kMaxWidth = 8;
// Candidate rows change hands 32 rows a round (a 4.6 KB buffer a wave, so 3
// workgroups fit a CU beside the bitmaps) and load 2 lines a batch: C5
// measured 2.40 ms against 2.52-2.78 ms for the other choices of 64 / 32 rows
// and 1, 2 or 4 lines, and 3.61 ms with one lane reading each row.
constexpr int kGRX = 32, kGLB = 2;

__device__ __forceinline__ uint64_t gmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint32_t graph_bit(int id) { return ((uint32_t)id * 2654435761u) >> 16; }

template <int D>
__global__ __launch_bounds__(kGW * kWave) void graph_search_kernel(GraphArgs a) {
  __shared__ uint32_t bm_s[kGW][kBitmapWords];
  __shared__ __align__(16) float qs_s[kGW][D];
  __shared__ int par_s[kGW][kMaxWidth];
  __shared__ __align__(16) float tr_s[kGW][row_tr_floats<kGRX>()];  // each wave's row hand-over buffer
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qi = blockIdx.x * kGW + wave;
  if (qi >= a.nq) return;  // the whole wave leaves; the kernel has no workgroup barrier
  uint32_t* bm = bm_s[wave];
  float* qs = qs_s[wave];
  int* par = par_s[wave];
  float* tr = tr_s[wave];
  for (int i = lane; i < kBitmapWords; i += kWave) bm[i] = 0u;
  for (int i = lane; i < D; i += kWave) qs[i] = a.queries[(size_t)qi * D + i];
  wave_lds_sync();
  const long long n = a.n;
  const int deg = a.degree, itopk = a.itopk;

  // the itopk list: one packed (distance, id) key per lane, ascending; ex =
  // expanded flag
  uint64_t lk = kPadKey;
  int ex = 0;
  int nev = 0;  // exact distances computed by this lane

  // One step: candidates c0, c1 (-1 = none) -> visited filter, dedup, exact
  // distances, merge into the list.
  auto step = [&](int c0, int c1) {
    const uint32_t b0 = graph_bit(c0), b1 = graph_bit(c1);
    const bool v0 = c0 >= 0 && (long long)c0 < n && !((bm[b0 >> 5] >> (b0 & 31)) & 1u);
    const bool v1 = c1 >= 0 && (long long)c1 < n && !((bm[b1 >> 5] >> (b1 & 31)) & 1u);
    // sort the 128 candidates by id: keys (0, id), dropped ones the padding key
    uint64_t k0 = v0 ? (uint64_t)(uint32_t)c0 : kPadKey, k1 = v1 ? (uint64_t)(uint32_t)c1 : kPadKey;
    wave_sort64_k(k0);
    wave_sort64_k(k1);
    {  // split into the 64 smallest (k0) and 64 largest (k1), both ascending
      const uint64_t r = wave_reverse64(k1);
      const bool c_lo = r < k0;
      k1 = c_lo ? k0 : r;
      k0 = c_lo ? r : k0;
      bitonic_pass_k<64>(k0, true);
      bitonic_pass_k<64>(k1, true);
    }
    int i0 = key_id(k0), i1 = key_id(k1);
    // keep each id once: drop an entry equal to its predecessor in the 128-sequence
    const int p0 = dpp_mov<0x138>(i0);  // wave_shr:1
    int p1 = dpp_mov<0x138>(i1);
    const int last0 = readlane_i(i0, kWave - 1);
    if (lane == 0) p1 = last0;
    if (i0 != kPadId && lane > 0 && i0 == p0) i0 = kPadId;
    if (i1 != kPadId && i1 == p1) i1 = kPadId;
    // mark the kept candidates visited (every bitmap read of this step is done)
    if (i0 != kPadId) { const uint32_t b = graph_bit(i0); atomicOr(&bm[b >> 5], 1u << (b & 31)); }
    if (i1 != kPadId) { const uint32_t b = graph_bit(i1); atomicOr(&bm[b >> 5], 1u << (b & 31)); }
    // exact distances: the kept rows, eight lanes a row, one lane's chain each
    float d0 = FLT_MAX, d1 = FLT_MAX;
#pragma unroll 1
    for (int h = 0; h < 2; ++h) {
      const int ih = h ? i1 : i0;
      const uint64_t mh = __ballot(ih != kPadId);
      if (!mh) break;  // the kept ids are sorted: an empty first half means an empty second
      const int fill = readlane_i(ih, __ffsll((unsigned long long)mh) - 1);  // a kept row for the empty lanes
      const float t = wave_rows_l2<D, kGRX, kGLB>(a.base, ih != kPadId ? ih : fill, qs, tr);
      if (ih != kPadId) {
        ++nev;
        if (h) d1 = t; else d0 = t;
      }
    }
    uint64_t e0 = key_of(d0, i0), e1 = key_of(d1, i1);  // padding ids give the padding key
    wave_sort64_k(e0);
    wave_sort64_k(e1);
    wave_merge_sorted64_kp(lk, ex, e0, 0);
    wave_merge_sorted64_kp(lk, ex, e1, 0);
    if (lane >= itopk) {
      lk = kPadKey;
      ex = 0;
    }
    wave_lds_sync();
  };

  const uint64_t qg = (uint64_t)a.q0 + (uint64_t)qi;
  step((int)(gmix64(a.seed ^ gmix64((qg << 20) | (uint64_t)lane)) % (uint64_t)n), -1);
  int it = 0;
  for (; it < a.max_iter; ++it) {
    uint64_t open = __ballot(key_id(lk) != kPadId && !ex);
    if (!open) break;
    int np = 0;
    for (; np < a.width && open; ++np) {
      const int L = __ffsll((unsigned long long)open) - 1;
      open &= open - 1;
      if (lane == L) ex = 1;
      const int pid = readlane_i(key_id(lk), L);
      if (lane == 0) par[np] = pid;
    }
    wave_lds_sync();
    int c0 = -1, c1 = -1;
    const int s0 = lane / deg, s1 = (lane + kWave) / deg;
    if (s0 < np) c0 = a.graph[(size_t)par[s0] * deg + (lane - s0 * deg)];
    if (s1 < np) c1 = a.graph[(size_t)par[s1] * deg + (lane + kWave - s1 * deg)];
    wave_lds_sync();
    step(c0, c1);
  }
  if (lane < a.k) {
    const int li = key_id(lk);
    a.out_ids[(size_t)qi * a.k + lane] = li == kPadId ? -1 : li;
    a.out_d[(size_t)qi * a.k + lane] = li == kPadId ? FLT_MAX : key_dist(lk);
  }
  if (a.iters && lane == 0) a.iters[qi] = it;
  if (a.evals) {
    const int tot = wave_sum_i(nev);
    if (lane == 0) a.evals[qi] = tot;
  }
}

template <int D>
fgpu_status launch_graph_t(const GraphArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(graph_search_kernel<D>, dim3((unsigned)((a.nq + kGW - 1) / kGW)), dim3(kGW * kWave), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

// Row i of an exact kNN list of the points themselves ([n][degree + 1],
// ascending) without i: the first `degree` other ids.
__global__ __launch_bounds__(256) void drop_self_kernel(const int32_t* __restrict__ knn, int n, int degree,
                                                        int32_t* __restrict__ out) {
  const int row = blockIdx.x * 256 + threadIdx.x;
  if (row >= n) return;
  const int32_t* r = knn + (size_t)row * (degree + 1);
  int32_t* o = out + (size_t)row * degree;
  int j = 0;
  for (int t = 0; t <= degree && j < degree; ++t) {
    const int v = r[t];
    if (v != row) o[j++] = v;
  }
}

// The coarse prune rule (prune_and_count_fused_kernel, gpu_global.cu:43-50)
// on graph-walk results: a probe whose distance exceeds best * prune_ratio,
// or a slot the walk left empty (id -1), becomes 0xFFFFFFFF.
__global__ __launch_bounds__(256) void coarse_prune_kernel(int32_t* __restrict__ ids, const float* __restrict__ d,
                                                           int nq, int p, float prune_ratio) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)nq * p) return;
  const float pthr = d[i - i % p] * prune_ratio;
  if (ids[i] < 0 || d[i] > pthr) ids[i] = (int32_t)kPruned;
}

}  // namespace

fgpu_status launch_drop_self(const int32_t* knn, int n, int degree, int32_t* out, hipStream_t s) {
  if (n <= 0) return FGPU_OK;
  hipLaunchKernelGGL(drop_self_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, knn, n, degree, out);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_coarse_prune(int32_t* ids, const float* d, int nq, int p, float prune_ratio, hipStream_t s) {
  const int64_t total = (int64_t)nq * p;
  if (total <= 0) return FGPU_OK;
  hipLaunchKernelGGL(coarse_prune_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, ids, d, nq, p,
                     prune_ratio);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_graph_search(int dim, const GraphArgs& a, hipStream_t s) {
  FGPU_CHECK(a.n >= 1 && a.n < INT32_MAX, FGPU_ERR_ARG, "graph_search: need 1 <= n < 2^31");
  FGPU_CHECK(a.degree >= 1 && a.width >= 1 && a.width <= kMaxWidth && a.width * a.degree <= 2 * kWave,
             FGPU_ERR_UNSUPPORTED, "graph_search: need width <= 8 and width * degree <= 128");
  FGPU_CHECK(a.itopk >= 1 && a.itopk <= kWave && a.k >= 1 && a.k <= a.itopk && a.max_iter >= 0, FGPU_ERR_UNSUPPORTED,
             "graph_search: need 1 <= k <= itopk <= 64 and max_iter >= 0");
  if (a.nq <= 0) return FGPU_OK;
  if (dim == 128) return launch_graph_t<128>(a, s);
  if (dim == 96) return launch_graph_t<96>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "graph_search: dim must be 96 or 128");
}

}  // namespace fgpu
