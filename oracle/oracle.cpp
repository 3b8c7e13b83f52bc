// oracle.cpp -- CPU restatement of the reference's IVF-PQ search and index-build path.
//
// TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
// product in fusiongpu_amd/.  Only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py may load it, and only to check or to time the
// CPU baseline.  Nothing in the product links, loads or calls it.
//
// Every function restates one piece of Hello-day/FusionGPU's algorithm and
// cites the reference file:line it follows.  Floating-point semantics are
// spelled out per function, because bit-exact parity depends on them:
//   * reference device kernels are built by nvcc with its default --fmad=true,
//     so `acc += a*b` there is one fused multiply-add per term;
//   * reference host code (pq_utils.h) is built by g++ -O3 for plain x86-64
//     (Makefile:35), which has no FMA instructions, so `acc += a*b` rounds the
//     product and the sum separately.
// This file is compiled with -ffp-contract=off, so every fused multiply-add
// below is an explicit std::fma/fmaf call and nothing else is contracted.
//
// Tie rule used wherever an order is needed: ascending fp32 distance, then
// ascending id (list id / codeword index / vector id).
//
// Parity pinning (what checks each function; see tests/test_oracle.py):
//   orc_l2_fma            closed form vs float64 (tolerance) and tiny brute force
//   orc_lut               fp64 closed form; special cases s=2,4,8 chains
//   orc_adc               brute force decode-and-sum identity
//   orc_coarse            brute force over all lists + tie rule
//   orc_search_plain      brute force over all candidates of the probed lists
//   orc_search_two_phase  reductions to orc_search_plain (p1 = nprobe with
//                         limit_k >= list length; p1 = 0; one list at a time
//                         for the cutoffs) and the threshold identities
//   orc_rerank            known answers: eps < 0 (never stable) is the exact
//                         top-k of all candidates (brute force); eps >= 1,
//                         beta = 1 stops after one batch; a hand-built stop
//                         sequence
//   orc_kmeans_*          Lloyd invariants, brute-force argmin, fixed-point sum
//   orc_pq_kmeans_fast,
//   orc_pq_train,
//   orc_pq_encode(host)   bit-exact against the reference's own pq_utils.h
//                         compiled from /root/reference (oracle/_ref) and the
//                         golden fixtures it wrote (tests/golden/)
//   orc_pq_encode(device) brute-force argmin of the fused chain
//   orc_build_lists       round trip with the ivf_data.bin writer layout
//   orc_knn_exact         brute force, tie rule
//   orc_graph_search      own definition (cuVS absent): complete graphs reduce
//                         it to exact kNN; a hand-built path graph fixes the
//                         step count; a planted bitmap collision drops a node
//   orc_gen_gmm           no reference counterpart: the synthetic workload
//                         generator; pinned by moments and determinism
//   orc_tune_list_stats   LUT entries against the fused chain evaluated in
//                         exact rational arithmetic with one correct rounding
//                         per step; on dyadic data (every operation exact)
//                         distances and ranks against numpy brute force; the
//                         k-th value and the ranks against sorted numpy arrays
//   orc_tune_coarse_order brute force numpy sort with the tie rule, distances
//                         as separately rounded float32 products and sums
#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <random>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

constexpr int kPQK = 256;  // PQ_K, defs.h:11

inline bool lt_pair(float da, int ia, float db, int ib) {
  return da < db || (da == db && ia < ib);
}

// Squared L2 in the form the reference's device kernels compute it: a
// sequential sum over dimensions where each term is fused into the running sum
// (tune_parameters.cu:39-46 and :76 as nvcc compiles them for the device;
// gpu_global.cu:636; kmeans_gpu.cuh:432-436).
inline float l2_fma(const float* a, const float* b, int d) {
  float acc = 0.0f;
  for (int i = 0; i < d; ++i) {
    float diff = a[i] - b[i];
    acc = std::fmaf(diff, diff, acc);
  }
  return acc;
}

// One LUT entry, exact per-subdimension op order of
// batch_residual_precompute_kernel (gpu_global.cu:115-158) and of
// compute_pq_dist_direct (gpu_global.cu:274-312).
inline float lut_entry(const float* r, const float* p, int s) {
  if (s == 4) {
    float dx = r[0] - p[0], dy = r[1] - p[1], dz = r[2] - p[2], dw = r[3] - p[3];
    return std::fmaf(dx, dx, std::fmaf(dy, dy, std::fmaf(dz, dz, dw * dw)));
  }
  if (s == 8) {
    float x1 = r[0] - p[0], y1 = r[1] - p[1], z1 = r[2] - p[2], w1 = r[3] - p[3];
    float x2 = r[4] - p[4], y2 = r[5] - p[5], z2 = r[6] - p[6], w2 = r[7] - p[7];
    float dist = std::fmaf(x1, x1, std::fmaf(y1, y1, std::fmaf(z1, z1, w1 * w1)));
    return std::fmaf(x2, x2, std::fmaf(y2, y2, std::fmaf(z2, z2, std::fmaf(w2, w2, dist))));
  }
  float dist = 0.0f;
  for (int d = 0; d < s; ++d) {
    float diff = r[d] - p[d];
    dist = std::fmaf(diff, diff, dist);
  }
  return dist;
}

// Sorted (ascending by tie rule) bounded list of the k best (dist, id) pairs.
struct TopK {
  int k;
  std::vector<float> d;
  std::vector<int> id;
  int n = 0;
  explicit TopK(int kk) : k(kk), d(kk), id(kk) {}
  bool full() const { return n == k; }
  void push(float dist, int vid) {
    if (k <= 0) return;
    if (n == k && !lt_pair(dist, vid, d[k - 1], id[k - 1])) return;
    int pos = (n < k) ? n++ : k - 1;
    while (pos > 0 && lt_pair(dist, vid, d[pos - 1], id[pos - 1])) {
      d[pos] = d[pos - 1];
      id[pos] = id[pos - 1];
      --pos;
    }
    d[pos] = dist;
    id[pos] = vid;
  }
};

inline int set_threads(int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
  return omp_get_max_threads();
#else
  (void)nthreads;
  return 1;
#endif
}

// splitmix64 finaliser: the counter-based generator behind orc_gen_gmm.
inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
inline double u01(uint64_t seed, uint64_t stream, uint64_t idx) {
  uint64_t h = mix64(seed ^ mix64(stream * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull) ^ mix64(idx));
  return (double)(h >> 11) * (1.0 / 9007199254740992.0);
}

}  // namespace

extern "C" {

int orc_version(void) { return 1; }

int orc_max_threads(void) { return set_threads(0); }

// ---------------------------------------------------------------------------
// Synthetic Gaussian-mixture generator (no reference counterpart).  The
// product library carries its own implementation of the same definition
// (fusiongpu_amd/csrc/gen.cpp); tests check the two agree bit for bit.
//   centre[j][d]  = lo + (hi-lo) * U(seed, stream 1, j*dim+d)
//   sigma[j]      = sig_lo + (sig_hi-sig_lo) * U(seed, stream 2, j)
//   label[i]      = floor(U(seed, stream 3+2*set, i) * ncomp)
//   x[i][d]       = centre[label][d] + sigma[label] * N(i*dim+d)
//   N(e)          = Box-Muller on the pair (U(seed, 4+2*set, 2*(e/2)),
//                   U(seed, 4+2*set, 2*(e/2)+1)); cos for even e, sin for odd
// `set` separates base vectors (0) from queries (1).  All in double, cast to
// float once.
void orc_gen_gmm(long long n, int dim, int ncomp, double lo, double hi, double sig_lo,
                 double sig_hi, unsigned long long seed, int set, float* out, int nthreads) {
  set_threads(nthreads);
  std::vector<double> centre((size_t)ncomp * dim), sigma(ncomp);
  for (long long j = 0; j < (long long)ncomp * dim; ++j) centre[j] = lo + (hi - lo) * u01(seed, 1, j);
  for (int j = 0; j < ncomp; ++j) sigma[j] = sig_lo + (sig_hi - sig_lo) * u01(seed, 2, j);
  const uint64_t s_lab = 3 + 2 * (uint64_t)set, s_noise = 4 + 2 * (uint64_t)set;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    int lab = (int)(u01(seed, s_lab, i) * ncomp);
    if (lab >= ncomp) lab = ncomp - 1;
    for (int d = 0; d < dim; ++d) {
      uint64_t e = (uint64_t)i * dim + d;
      uint64_t pr = e >> 1;
      double a = u01(seed, s_noise, 2 * pr), b = u01(seed, s_noise, 2 * pr + 1);
      double rad = std::sqrt(-2.0 * std::log(1.0 - a));
      double ang = 6.283185307179586476925286766559 * b;
      double z = (e & 1) ? rad * std::sin(ang) : rad * std::cos(ang);
      out[(size_t)e] = (float)(centre[(size_t)lab * dim + d] + sigma[lab] * z);
    }
  }
}

// ---------------------------------------------------------------------------
// A4/A5 building blocks.
float orc_l2_fma(const float* a, const float* b, int d) { return l2_fma(a, b, d); }

// LUT[m][k] = || (q - c)_m - P[m][k] ||^2 (gpu_global.cu:79-166).  The
// residual is formed first as q - c (gpu_global.cu:98-100).
void orc_lut(const float* q, const float* c, const float* codebook, int dim, int m, float* lut) {
  const int s = dim / m;
  std::vector<float> r(dim);
  for (int i = 0; i < dim; ++i) r[i] = q[i] - c[i];
  for (int sub = 0; sub < m; ++sub)
    for (int k = 0; k < kPQK; ++k)
      lut[sub * kPQK + k] = lut_entry(&r[sub * s], codebook + ((size_t)sub * kPQK + k) * s, s);
}

// ADC distance: sequential fp32 sum over subspaces in ascending m
// (compute_pq_dist_vectorized, gpu_global.cu:196-253).
float orc_adc(const uint8_t* code, const float* lut, int m) {
  float dist = 0.0f;
  for (int sub = 0; sub < m; ++sub) dist += lut[sub * kPQK + code[sub]];
  return dist;
}

// ---------------------------------------------------------------------------
// A2 + A3: coarse quantizer.  The reference asks cuVS CAGRA for the top_m
// nearest centroids (search_pipeline.cu:341); its exact analogue is the
// tuner's full ranking (tune_parameters.cu:538-546: distance to every
// centroid, std::sort of (dist, id) pairs).  This restates the exact ranking
// with the device distance form, then applies prune_and_count_fused_kernel's
// prune rule (gpu_global.cu:43-50): a probe whose distance exceeds
// best * prune_ratio becomes 0xFFFFFFFF.  Returns 0, or -1 on bad arguments.
int orc_coarse(const float* q, int nq, const float* cent, int nlist, int dim, int nprobe,
               float prune_ratio, uint32_t* ids, float* dists, int nthreads) {
  if (nprobe <= 0 || nprobe > nlist) return -1;
  set_threads(nthreads);
#pragma omp parallel
  {
    std::vector<std::pair<float, int>> all(nlist);
#pragma omp for schedule(dynamic, 16)
    for (int i = 0; i < nq; ++i) {
      const float* qi = q + (size_t)i * dim;
      for (int l = 0; l < nlist; ++l) all[l] = {l2_fma(qi, cent + (size_t)l * dim, dim), l};
      std::partial_sort(all.begin(), all.begin() + nprobe, all.end());
      float thr = all[0].first * prune_ratio;
      for (int p = 0; p < nprobe; ++p) {
        dists[(size_t)i * nprobe + p] = all[p].first;
        ids[(size_t)i * nprobe + p] = (all[p].first > thr) ? 0xFFFFFFFFu : (uint32_t)all[p].second;
      }
    }
  }
  return 0;
}

// counts[q] = sum of list sizes over surviving probes (gpu_global.cu:54-76).
void orc_probe_counts(const uint32_t* probe_ids, int nq, int nprobe, const int* offsets, int* counts) {
  for (int i = 0; i < nq; ++i) {
    int c = 0;
    for (int p = 0; p < nprobe; ++p) {
      uint32_t l = probe_ids[(size_t)i * nprobe + p];
      if (l != 0xFFFFFFFFu) c += offsets[l + 1] - offsets[l];
    }
    counts[i] = c;
  }
}

// ---------------------------------------------------------------------------
// A4-A6, A10 in plain IVF-PQ form (p1_lists = nprobe, limit_k = k, no
// rerank): the k best (ADC distance, vector id) pairs over every vector of
// every surviving probed list.  The reference computes per-list top-limit_k
// (gpu_global.cu:321-390), unions them and sorts (gpu_global.cu:852-861), then
// keeps the first rerank_m = k (gpu_global.cu:556-576); with limit_k = k the
// union of per-list top-k contains the global top-k, so this is the same set.
// Deviations kept on purpose: whole lists are scanned (the reference stops at
// 1024 items per list, gpu_global.cu:346), and ties across lists follow the
// tie rule (the reference's order there depends on atomic slot races).
// Missing results are padded with id -1 and distance FLT_MAX
// (gpu_global.cu:573-574).
void orc_search_plain(const float* q, int nq, int dim, int m, const float* cent,
                      const float* codebook, const int* offsets, const int* vec_ids,
                      const uint8_t* codes, const uint32_t* probe_ids, int nprobe, int k,
                      int* out_ids, float* out_dists, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel
  {
    std::vector<float> lut((size_t)m * kPQK);
#pragma omp for schedule(dynamic, 4)
    for (int i = 0; i < nq; ++i) {
      TopK top(k);
      const float* qi = q + (size_t)i * dim;
      for (int p = 0; p < nprobe; ++p) {
        uint32_t l = probe_ids[(size_t)i * nprobe + p];
        if (l == 0xFFFFFFFFu) continue;
        orc_lut(qi, cent + (size_t)l * dim, codebook, dim, m, lut.data());
        for (int v = offsets[l]; v < offsets[l + 1]; ++v)
          top.push(orc_adc(codes + (size_t)v * m, lut.data(), m), vec_ids[v]);
      }
      for (int j = 0; j < k; ++j) {
        out_ids[(size_t)i * k + j] = j < top.n ? top.id[j] : -1;
        out_dists[(size_t)i * k + j] = j < top.n ? top.d[j] : FLT_MAX;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// A6-A10 in their general form: the two-phase pruned scan of
// run_gpu_batch_logic (gpu_global.cu:679-874).
//   * phase 1 (ivf_scan_phase1_kernel, gpu_global.cu:321-390): for each of the
//     first p1 = min(nprobe, p1_lists) probes, ADC over the whole list, the
//     w = min(n_l, limit_k) best (dist, id) become candidates and the w-th
//     distance is the list's cutoff; a pruned or empty probe leaves cutoff 0;
//   * threshold (compute_threshold_kernel, gpu_global.cu:394-426):
//     thr = coeff * min(cutoff > 0), or FLT_MAX if no cutoff is > 0;
//   * phase 2 (ivf_scan_phase2_kernel, gpu_global.cu:428-527): for the other
//     probes every vector with dist <= thr is a candidate (the reference's
//     direct-codebook distance is bit-identical to the LUT distance);
//   * compaction + segmented sort + gather (gpu_global.cu:533-576, 852-867):
//     the candidates sorted ascending, the first rerank_m kept, padded with
//     id -1 / FLT_MAX, counts[q] = min(#candidates, rerank_m).
// Deviations kept on purpose: whole lists are scanned in phase 1 (the
// reference stops at 1024 items, gpu_global.cu:346), phase 2 emits each
// passing vector exactly once (the reference's overflow path re-writes some,
// gpu_global.cu:508-526), all rerank_m entries are gathered (the reference's
// gather writes at most 128, gpu_global.cu:867), and order is the tie rule
// (dist, then id) where the reference's depends on atomic slot races.
// Probe ids >= nlist count as pruned.  cutoffs ([nq][p1]), thr ([nq]) and
// pre_cut ([nq]) are optional outputs; pre_cut[q] is the number of candidates
// before the rerank_m cut, the count the reference accumulates in
// query_atomic_counters (gpu_global.cu:349, 493-526): sum over phase-1 lists
// of min(n_l, limit_k) plus every phase-2 vector with dist <= thr.
void orc_search_two_phase(const float* q, int nq, int dim, int m, const float* cent,
                          const float* codebook, const int* offsets, const int* vec_ids,
                          const uint8_t* codes, int nlist, const uint32_t* probe_ids, int nprobe,
                          int p1_lists, int limit_k, float threshold_coeff, int rerank_m,
                          int* out_ids, float* out_dists, int* out_counts, float* cutoffs,
                          float* thr_out, int* pre_cut, int nthreads) {
  set_threads(nthreads);
  const int p1 = std::max(0, std::min(nprobe, p1_lists));
#pragma omp parallel
  {
    std::vector<float> lut((size_t)m * kPQK);
    std::vector<std::pair<float, int>> cand, list;
#pragma omp for schedule(dynamic, 2)
    for (int i = 0; i < nq; ++i) {
      const float* qi = q + (size_t)i * dim;
      cand.clear();
      float min_cut = FLT_MAX;
      for (int p = 0; p < p1; ++p) {
        const uint32_t l = probe_ids[(size_t)i * nprobe + p];
        float cut = 0.0f;
        if (l < (uint32_t)nlist && offsets[l + 1] > offsets[l]) {
          orc_lut(qi, cent + (size_t)l * dim, codebook, dim, m, lut.data());
          list.clear();
          for (int v = offsets[l]; v < offsets[l + 1]; ++v)
            list.push_back({orc_adc(codes + (size_t)v * m, lut.data(), m), vec_ids[v]});
          const int w = std::min((int)list.size(), limit_k);
          std::partial_sort(list.begin(), list.begin() + w, list.end());
          cand.insert(cand.end(), list.begin(), list.begin() + w);
          cut = list[w - 1].first;
        }
        if (cutoffs) cutoffs[(size_t)i * p1 + p] = cut;
        if (cut > 0.0f && cut < min_cut) min_cut = cut;
      }
      const float thr = min_cut < FLT_MAX ? min_cut * threshold_coeff : FLT_MAX;
      if (thr_out) thr_out[i] = thr;
      for (int p = p1; p < nprobe; ++p) {
        const uint32_t l = probe_ids[(size_t)i * nprobe + p];
        if (l >= (uint32_t)nlist) continue;
        orc_lut(qi, cent + (size_t)l * dim, codebook, dim, m, lut.data());
        for (int v = offsets[l]; v < offsets[l + 1]; ++v) {
          const float d = orc_adc(codes + (size_t)v * m, lut.data(), m);
          if (d <= thr) cand.push_back({d, vec_ids[v]});
        }
      }
      if (pre_cut) pre_cut[i] = (int)cand.size();
      const int cnt = std::min((int)cand.size(), rerank_m);
      std::partial_sort(cand.begin(), cand.begin() + cnt, cand.end());
      for (int j = 0; j < rerank_m; ++j) {
        out_ids[(size_t)i * rerank_m + j] = j < cnt ? cand[j].second : -1;
        out_dists[(size_t)i * rerank_m + j] = j < cnt ? cand[j].first : FLT_MAX;
      }
      out_counts[i] = cnt;
    }
  }
}

// A11: heuristic early-stopping exact rerank (run_gpu_rerank +
// heuristic_rerank_kernel, gpu_global.cu:603-673).  Per query, walk the first
// counts[q] candidates (of a row of rm) in mini-batches of mb: exact
// device-form L2 (`local_d += diff*diff` contracted, gpu_global.cu:636), merge
// with the running top-k, chg = number of real ids in the new top-k that were
// not in the old one; stable += 1 if (float)chg/k <= eps else stable = 0; stop
// after beta stable batches or when the candidates run out (gpu_global.cu:
// 615, 653-662).  Order: ascending (distance, id) with the padding entry
// (FLT_MAX, -1) after every real entry; the reference sorts only 128 of the
// k+mb entries (gpu_global.cu:644-647) -- all are sorted here.  A candidate id
// outside [0, n) is skipped (treated as padding).  visited ([nq], optional) =
// candidates evaluated; stable_out / finished_out ([nq], optional) = the
// state the reference leaves in stab[] and fin[] (gpu_global.cu:603-609,
// 615, 653-662): the stable count after the last batch evaluated, and
// finished when the walk stopped on stability or reached an offset past the
// candidates before rm.
void orc_rerank(const float* q, int nq, int dim, const float* base, long long n,
                const int* cand_ids, const int* counts, int rm, int k, int mb, float eps, int beta,
                int* out_ids, float* out_dists, int* visited, int* stable_out, uint8_t* finished_out,
                int nthreads) {
  set_threads(nthreads);
#pragma omp parallel
  {
    std::vector<std::pair<float, uint32_t>> top, merged;
#pragma omp for schedule(dynamic, 4)
    for (int i = 0; i < nq; ++i) {
      const float* qi = q + (size_t)i * dim;
      top.assign(k, {FLT_MAX, 0xFFFFFFFFu});
      int stable = 0, seen = 0;
      bool fin = false;
      const int total = std::min(counts[i], rm);
      for (int off = 0; off < rm; off += mb) {
        if (off >= total) {
          fin = true;
          break;
        }
        const int eff = std::min(mb, total - off);
        merged = top;
        for (int j = 0; j < eff; ++j) {
          const int vid = cand_ids[(size_t)i * rm + off + j];
          if (vid >= 0 && (long long)vid < n)
            merged.push_back({l2_fma(qi, base + (size_t)vid * dim, dim), (uint32_t)vid});
          else
            merged.push_back({FLT_MAX, 0xFFFFFFFFu});
        }
        seen += eff;
        std::stable_sort(merged.begin(), merged.end());
        int chg = 0;
        for (int j = 0; j < k; ++j) {
          const uint32_t nid = merged[j].second;
          if (nid == 0xFFFFFFFFu) continue;
          bool found = false;
          for (int t = 0; t < k; ++t)
            if (top[t].second == nid) { found = true; break; }
          if (!found) ++chg;
        }
        std::copy(merged.begin(), merged.begin() + k, top.begin());
        if ((float)chg / (float)k <= eps) ++stable; else stable = 0;
        if (stable >= beta) {
          fin = true;
          break;
        }
      }
      if (stable_out) stable_out[i] = stable;
      if (finished_out) finished_out[i] = fin ? 1 : 0;
      for (int j = 0; j < k; ++j) {
        const bool pad = top[j].second == 0xFFFFFFFFu;
        out_ids[(size_t)i * k + j] = pad ? -1 : (int)top[j].second;
        out_dists[(size_t)i * k + j] = pad ? FLT_MAX : top[j].first;
      }
      if (visited) visited[i] = seen;
    }
  }
}

// ---------------------------------------------------------------------------
// A19: graph (CAGRA-style) search.  The reference calls cuVS CAGRA
// (cagra_adapter.cuh:38-68: itopk, search width, max iterations), whose
// algorithm is not in the repository, so this is a stated definition, not a
// restatement:
//   * 64 seed nodes, node_j = mix64(seed ^ mix64((q << 20) | j)) % n, with q
//     the query's index;
//   * each step takes the `width` best entries of the itopk list not yet
//     expanded (in list order), marks them expanded, and offers their
//     `degree` neighbours graph[p][0..degree) as candidates;
//   * a candidate is dropped if its id is outside [0, n) or if its bit in the
//     query's visited bitmap (2^16 bits, bit = (uint32)(id * 2654435761) >> 16)
//     was set before the step (hash collisions drop a node: the bitmap is
//     approximate by design); duplicates within the step are kept once; then
//     the bits of the kept candidates are set;
//   * kept candidates get the exact device-form L2 and are merged into the
//     itopk list by (distance, id), which keeps its itopk best;
//   * the search stops when no entry is left to expand or after max_iter
//     steps; the first k entries are the answer (pad -1 / FLT_MAX).
// iters ([nq], optional) = steps taken.
static inline uint32_t graph_bit(int id) { return (uint32_t)((uint32_t)id * 2654435761u) >> 16; }

void orc_graph_search(const float* q, int nq, const float* base, long long n, int dim, const int* graph,
                      int degree, int itopk, int width, int max_iter, int k, unsigned long long seed,
                      int* out_ids, float* out_dists, int* iters, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel
  {
    std::vector<uint8_t> bits(1 << 16);
    struct E { float d; int id; bool ex; };
    std::vector<E> list, add;
    std::vector<int> cand, keep;
#pragma omp for schedule(dynamic, 4)
    for (int i = 0; i < nq; ++i) {
      const float* qi = q + (size_t)i * dim;
      std::fill(bits.begin(), bits.end(), 0);
      list.clear();
      auto step = [&]() {
        keep.clear();
        for (int c : cand)
          if (c >= 0 && (long long)c < n && !bits[graph_bit(c)]) keep.push_back(c);
        std::sort(keep.begin(), keep.end());
        keep.erase(std::unique(keep.begin(), keep.end()), keep.end());
        for (int c : keep) bits[graph_bit(c)] = 1;
        for (int c : keep) list.push_back({l2_fma(qi, base + (size_t)c * dim, dim), c, false});
        std::sort(list.begin(), list.end(), [](const E& x, const E& y) { return lt_pair(x.d, x.id, y.d, y.id); });
        if ((int)list.size() > itopk) list.resize(itopk);
      };
      cand.clear();
      for (int j = 0; j < 64; ++j)
        cand.push_back((int)(mix64(seed ^ mix64(((uint64_t)i << 20) | (uint64_t)j)) % (uint64_t)n));
      step();
      int it = 0;
      for (; it < max_iter; ++it) {
        cand.clear();
        int taken = 0;
        for (auto& e : list) {
          if (taken == width) break;
          if (e.ex) continue;
          e.ex = true;
          ++taken;
          for (int j = 0; j < degree; ++j) cand.push_back(graph[(size_t)e.id * degree + j]);
        }
        if (taken == 0) break;
        step();
      }
      for (int j = 0; j < k; ++j) {
        const bool real = j < (int)list.size();
        out_ids[(size_t)i * k + j] = real ? list[j].id : -1;
        out_dists[(size_t)i * k + j] = real ? list[j].d : FLT_MAX;
      }
      if (iters) iters[i] = it;
    }
  }
}

// ---------------------------------------------------------------------------
// A18: exact kNN ground truth (brute_force_search_kernel,
// tune_parameters.cu:49-96): device distance form, insertion top-k with
// strict < so the earlier id wins a tie.
void orc_knn_exact(const float* q, int nq, const float* base, long long n, int dim, int k,
                   int* out_ids, float* out_dists, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
  for (int i = 0; i < nq; ++i) {
    TopK top(k);
    const float* qi = q + (size_t)i * dim;
    for (long long v = 0; v < n; ++v) top.push(l2_fma(qi, base + (size_t)v * dim, dim), (int)v);
    for (int j = 0; j < k; ++j) {
      out_ids[(size_t)i * k + j] = j < top.n ? top.id[j] : -1;
      out_dists[(size_t)i * k + j] = j < top.n ? top.d[j] : FLT_MAX;
    }
  }
}

// ---------------------------------------------------------------------------
// A13: k-means assignment.  The reference ranks with a cuBLAS -2*X*C^T GEMM
// plus norms (kmeans_gpu.cuh:197-229), whose summation order is not
// reproducible; its argmin keeps the lowest index on ties (strict <,
// kmeans_gpu.cuh:67-76).  Restated as the argmin of the exact device-form
// distance with the same tie rule.
void orc_kmeans_assign(const float* x, long long n, const float* cent, int k, int dim, int* out,
                       int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    float best = FLT_MAX;
    int bi = 0;
    for (int c = 0; c < k; ++c) {
      float d = l2_fma(x + (size_t)i * dim, cent + (size_t)c * dim, dim);
      if (d < best) { best = d; bi = c; }
    }
    out[i] = bi;
  }
}

// Fixed-point scale for the deterministic centroid sum: the largest S such
// that n * max|x| * 2^S stays below 2^61, capped to [0, 60].
int orc_fixed_shift(float maxabs, long long n) {
  int e = 0;
  if (maxabs > 0.0f) std::frexp((double)maxabs, &e);  // maxabs < 2^e
  int lg = 0;
  while ((1LL << lg) < (n > 0 ? n : 1)) ++lg;
  int s = 61 - lg - e;
  return s < 0 ? 0 : (s > 60 ? 60 : s);
}

// A14: one Lloyd update (accumulate_centroids_kernel + compute_centroids_kernel,
// kmeans_gpu.cuh:81-116).  The reference adds coordinates with float
// atomicAdd, so its sum order is a race; the restatement sums fixed-point
// integers  round(x * 2^S)  (associative, hence order free), converts once and
// then scales as the reference does:  c = (float)(sum * 2^-S) * (1.0f/count).
// empty_rule 0: an empty cluster becomes the zero vector (the reference
// memsets the sums, kmeans_gpu.cuh:293, and skips the scale, :110);
// empty_rule 1: it keeps its old centroid (pq_utils.h:65-70).
void orc_kmeans_update(const float* x, long long n, const int* assign, int k, int dim, int shift,
                       int empty_rule, float* cent, int* counts) {
  std::vector<long long> sum((size_t)k * dim, 0);
  std::vector<int> cnt(k, 0);
  for (long long i = 0; i < n; ++i) {
    int c = assign[i];
    cnt[c]++;
    for (int d = 0; d < dim; ++d)
      sum[(size_t)c * dim + d] += std::llrint(std::ldexp(x[(size_t)i * dim + d], shift));
  }
  for (int c = 0; c < k; ++c) {
    if (counts) counts[c] = cnt[c];
    if (cnt[c] == 0) {
      if (empty_rule == 0)
        for (int d = 0; d < dim; ++d) cent[(size_t)c * dim + d] = 0.0f;
      continue;
    }
    float inv = 1.0f / (float)cnt[c];
    for (int d = 0; d < dim; ++d) {
      float s = (float)std::ldexp((double)sum[(size_t)c * dim + d], -shift);
      cent[(size_t)c * dim + d] = s * inv;
    }
  }
}

// Reference initialisation of run_kmeans_gpu (kmeans_gpu.cuh:259-267):
// mt19937(seed), stride = max(1, n/k), row i*stride + rng()%stride (mod n).
void orc_kmeans_init_strided(const float* x, long long n, int dim, int k, unsigned seed,
                             float* out, int* rows) {
  std::mt19937 rng(seed);
  long long stride = std::max<long long>(1, n / k);
  for (int i = 0; i < k; ++i) {
    long long idx = ((long long)i * stride + (long long)(rng() % (unsigned long long)stride)) % n;
    if (rows) rows[i] = (int)idx;
    std::memcpy(out + (size_t)i * dim, x + (size_t)idx * dim, sizeof(float) * dim);
  }
}

// k-means++ style seeding (no reference counterpart).
// Deterministic definition: rng = splitmix64 counter stream (seed, 7);
// first centre = row (r0 % n); weight w_i = round(D2_i * 2^S) as uint64 with
// S fixed from the first round's max D2 so that n * max w < 2^62; next centre =
// smallest i whose inclusive prefix sum of w exceeds (r_j % total); D2 is the
// device-form exact distance to the nearest chosen centre.  If every weight is
// zero the next centre is the lowest row not yet chosen.
void orc_kmeans_init_pp(const float* x, long long n, int dim, int k, unsigned long long seed,
                        float* out, int* rows, int nthreads) {
  set_threads(nthreads);
  std::vector<float> d2(n);
  std::vector<char> chosen(n, 0);
  long long r0 = (long long)(mix64(seed ^ mix64(7)) % (uint64_t)n);
  rows[0] = (int)r0;
  chosen[r0] = 1;
  std::memcpy(out, x + (size_t)r0 * dim, sizeof(float) * dim);
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) d2[i] = l2_fma(x + (size_t)i * dim, out, dim);
  float mx = 0.0f;
  for (long long i = 0; i < n; ++i) mx = std::max(mx, d2[i]);
  int e = 0;
  if (mx > 0.0f) std::frexp((double)mx, &e);
  int lg = 0;
  while ((1LL << lg) < n) ++lg;
  int S = 62 - lg - e;
  if (S > 60) S = 60;
  if (S < 0) S = 0;
  std::vector<uint64_t> w(n);
  for (int j = 1; j < k; ++j) {
    uint64_t total = 0;
    for (long long i = 0; i < n; ++i) {
      w[i] = (uint64_t)std::llrint(std::ldexp((double)d2[i], S));
      total += w[i];
    }
    long long pick = -1;
    if (total == 0) {
      for (long long i = 0; i < n; ++i)
        if (!chosen[i]) { pick = i; break; }
      if (pick < 0) pick = 0;
    } else {
      uint64_t u = mix64(seed ^ mix64(7) ^ mix64(0x100000000ull + (uint64_t)j)) % total;
      uint64_t acc = 0;
      for (long long i = 0; i < n; ++i) {
        acc += w[i];
        if (acc > u) { pick = i; break; }
      }
    }
    rows[j] = (int)pick;
    chosen[pick] = 1;
    float* cj = out + (size_t)j * dim;
    std::memcpy(cj, x + (size_t)pick * dim, sizeof(float) * dim);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < n; ++i) {
      float d = l2_fma(x + (size_t)i * dim, cj, dim);
      if (d < d2[i]) d2[i] = d;
    }
  }
}

// ---------------------------------------------------------------------------
// A15: PQ codebook training (pq_utils.h:17-138), host floating point.
// run_kmeans_pq_fast (pq_utils.h:17-72): mt19937(seed) + std::shuffle of
// 0..n-1, first k rows as centres; E-step sequential `d += diff*diff` (product
// and sum rounded separately), strict <; M-step double sums in row order,
// (float)(sum / count); an empty cluster keeps its centre.  Returns -1 if n < k
// (the reference would read past its index vector).
int orc_pq_kmeans_fast(const float* data, int n, int dim, int k, int seed, int max_iter,
                       float* centroids) {
  if (n < k) return -1;
  std::mt19937 rng(seed);
  std::vector<int> indices(n);
  std::iota(indices.begin(), indices.end(), 0);
  std::shuffle(indices.begin(), indices.end(), rng);
  for (int c = 0; c < k; ++c)
    std::memcpy(centroids + (size_t)c * dim, data + (size_t)indices[c] * dim, dim * sizeof(float));
  std::vector<int> assign(n);
  std::vector<double> acc((size_t)k * dim);
  std::vector<int> counts(k);
  for (int it = 0; it < max_iter; ++it) {
    for (int i = 0; i < n; ++i) {
      float min_d = FLT_MAX;
      int best = 0;
      for (int c = 0; c < k; ++c) {
        float d = 0.0f;
        for (int j = 0; j < dim; ++j) {
          float diff = data[(size_t)i * dim + j] - centroids[(size_t)c * dim + j];
          float sq = diff * diff;
          d = d + sq;
        }
        if (d < min_d) { min_d = d; best = c; }
      }
      assign[i] = best;
    }
    std::fill(acc.begin(), acc.end(), 0.0);
    std::fill(counts.begin(), counts.end(), 0);
    for (int i = 0; i < n; ++i) {
      int c = assign[i];
      counts[c]++;
      for (int j = 0; j < dim; ++j) acc[(size_t)c * dim + j] += data[(size_t)i * dim + j];
    }
    for (int c = 0; c < k; ++c)
      if (counts[c] > 0)
        for (int j = 0; j < dim; ++j)
          centroids[(size_t)c * dim + j] = (float)(acc[(size_t)c * dim + j] / counts[c]);
  }
  return 0;
}

// Sample rows for PQ training (pq_utils.h:91-97): mt19937(12345) shuffle of
// 0..n-1, keep the first min(sample, n).  Returns the sample size.
int orc_pq_sample(long long n, int sample_size, int* out_rows) {
  int actual = (int)std::min<long long>(sample_size, n);
  std::vector<int> idx(n);
  std::iota(idx.begin(), idx.end(), 0);
  std::mt19937 rng(12345);
  std::shuffle(idx.begin(), idx.end(), rng);
  std::memcpy(out_rows, idx.data(), sizeof(int) * actual);
  return actual;
}

// train_residual_pq_codebooks (pq_utils.h:77-138): residuals of the sampled
// rows against their list centroid, one run_kmeans_pq_fast per subspace with
// seed 1234+m.  codebook is [m][256][dim/m].
int orc_pq_train(const float* x, long long n, int dim, int m, const int* assign, const float* cent,
                 int sample_size, int max_iter, float* codebook, int nthreads) {
  set_threads(nthreads);
  const int s = dim / m;
  std::vector<int> rows(std::min<long long>(sample_size, n));
  int actual = orc_pq_sample(n, sample_size, rows.data());
  if (actual < kPQK) return -1;
  std::vector<float> res((size_t)actual * dim);
  for (int i = 0; i < actual; ++i) {
    int o = rows[i], c = assign[o];
    for (int j = 0; j < dim; ++j) res[(size_t)i * dim + j] = x[(size_t)o * dim + j] - cent[(size_t)c * dim + j];
  }
  int bad = 0;
#pragma omp parallel for schedule(dynamic) reduction(+ : bad)
  for (int sub = 0; sub < m; ++sub) {
    std::vector<float> sv((size_t)actual * s);
    for (int i = 0; i < actual; ++i)
      for (int d = 0; d < s; ++d) sv[(size_t)i * s + d] = res[(size_t)i * dim + sub * s + d];
    bad += orc_pq_kmeans_fast(sv.data(), actual, s, kPQK, 1234 + sub, max_iter,
                              codebook + (size_t)sub * kPQK * s) != 0;
  }
  return bad ? -1 : 0;
}

// A16: residual PQ encoding.  fma_mode 1 follows the GPU encoder the
// reference's build uses (encode_residuals_kernel, kmeans_gpu.cuh:403-445, with
// nvcc's contraction: dist = fma(diff, diff, dist)); fma_mode 0 follows its
// CPU twin (encode_residuals_to_pq, pq_utils.h:141-175: product and sum
// rounded separately).  Residual first, then the codeword difference; strict <
// keeps the lowest codeword on ties.
void orc_pq_encode(const float* x, long long n, int dim, int m, const int* assign, const float* cent,
                   const float* codebook, int fma_mode, uint8_t* codes, int nthreads) {
  set_threads(nthreads);
  const int s = dim / m;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    const float* xi = x + (size_t)i * dim;
    const float* ci = cent + (size_t)assign[i] * dim;
    for (int sub = 0; sub < m; ++sub) {
      float min_d = FLT_MAX;
      int best = 0;
      for (int k = 0; k < kPQK; ++k) {
        const float* p = codebook + ((size_t)sub * kPQK + k) * s;
        float d = 0.0f;
        for (int j = 0; j < s; ++j) {
          float residual = xi[sub * s + j] - ci[sub * s + j];
          float diff = residual - p[j];
          if (fma_mode) {
            d = std::fmaf(diff, diff, d);
          } else {
            float sq = diff * diff;
            d = d + sq;
          }
        }
        if (d < min_d) { min_d = d; best = k; }
      }
      codes[(size_t)i * m + sub] = (uint8_t)best;
    }
  }
}

// A17: inverted-list assembly (build_global.cu:225-240): lists in cluster
// order, vector ids ascending inside a list, codes copied in the same order.
void orc_build_lists(const int* assign, long long n, int nlist, const uint8_t* codes, int m,
                     int* offsets, int* ids, uint8_t* list_codes) {
  std::vector<int> cnt(nlist + 1, 0);
  for (long long i = 0; i < n; ++i) cnt[assign[i] + 1]++;
  for (int l = 0; l < nlist; ++l) cnt[l + 1] += cnt[l];
  std::memcpy(offsets, cnt.data(), sizeof(int) * (nlist + 1));
  std::vector<int> pos(cnt.begin(), cnt.end() - 1);
  for (long long i = 0; i < n; ++i) {
    int p = pos[assign[i]]++;
    ids[p] = (int)i;
    std::memcpy(list_codes + (size_t)p * m, codes + (size_t)i * m, m);
  }
}


// ---------------------------------------------------------------------------
// Offline tuner (tune_parameters.cu:459-1012), the per-(query, list) part.
// For each pair: the tuner's own LUT (precompute_lut_kernel, :101-123; built
// by nvcc, so `dist += diff*diff` is fused: dist = fmaf(diff, diff, dist) from
// 0 over the sub-vector, with diff = (q - c) - codeword), the PQ distance as an
// ascending sum of LUT entries (:127-145), the exact distance as the fused
// chain over all dimensions (:148-166).  At the first list position holding
// the target id: its distances and 1 + the count strictly below each
// (:755-784); the min(kth, n)-th smallest PQ distance (:893-899).  Absent
// target: ranks 0, distances -1.  base == nullptr: no exact part.
void orc_tune_list_stats(const float* q, int nq, int dim, const float* cent, int nlist, const float* codebook,
                         int m, const int* offsets, const int* ids, const uint8_t* codes, const float* base,
                         long long n_base, const int* pair_q, const int* pair_l, const int* pair_t,
                         const int* pair_k, int npairs, float* t_pq, float* t_ex, int* pq_rank, int* ex_rank,
                         float* kth_pq, int nthreads) {
  set_threads(nthreads);
  const int S = dim / m;
#pragma omp parallel for schedule(dynamic, 1)
  for (int p = 0; p < npairs; ++p) {
    const int qi = pair_q[p], l = pair_l[p];
    const int target = pair_t ? pair_t[p] : -1, kk = pair_k ? pair_k[p] : 0;
    if (qi < 0 || qi >= nq || l < 0 || l >= nlist) {
      if (pair_t) { t_pq[p] = -1.0f; t_ex[p] = -1.0f; pq_rank[p] = 0; ex_rank[p] = 0; }
      if (pair_k) kth_pq[p] = 0.0f;
      continue;
    }
    const float* qv = q + (size_t)qi * dim;
    const float* cv = cent + (size_t)l * dim;
    std::vector<float> lut((size_t)m * kPQK);
    for (int mm = 0; mm < m; ++mm)
      for (int k = 0; k < kPQK; ++k) {
        const float* cw = codebook + ((size_t)mm * kPQK + k) * S;
        float dist = 0.0f;
        for (int d = 0; d < S; ++d) {
          const float r = qv[mm * S + d] - cv[mm * S + d];
          const float diff = r - cw[d];
          dist = std::fmaf(diff, diff, dist);
        }
        lut[(size_t)mm * kPQK + k] = dist;
      }
    const int st = offsets[l], n = offsets[l + 1] - st;
    std::vector<float> pq(n), ex(n);
    for (int j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (int mm = 0; mm < m; ++mm) sum += lut[(size_t)mm * kPQK + codes[(size_t)(st + j) * m + mm]];
      pq[j] = sum;
      const int id = ids[st + j];
      ex[j] = (base && id >= 0 && id < n_base) ? l2_fma(qv, base + (size_t)id * dim, dim) : INFINITY;
    }
    if (pair_t) {
      int pos = -1;
      for (int j = 0; j < n && pos < 0 && target >= 0; ++j)
        if (ids[st + j] == target) pos = j;
      if (pos < 0) {
        t_pq[p] = -1.0f; t_ex[p] = -1.0f; pq_rank[p] = 0; ex_rank[p] = 0;
      } else {
        int bp = 0, be = 0;
        for (int j = 0; j < n; ++j) {
          bp += pq[j] < pq[pos];
          be += ex[j] < ex[pos];
        }
        t_pq[p] = pq[pos];
        pq_rank[p] = bp + 1;
        t_ex[p] = base ? ex[pos] : -1.0f;
        ex_rank[p] = base ? be + 1 : 0;
      }
    }
    if (pair_k && kk > 0) {
      if (n == 0) {
        kth_pq[p] = 0.0f;
      } else {
        std::vector<float> srt(pq);
        std::sort(srt.begin(), srt.end());
        kth_pq[p] = srt[(size_t)std::min(kk, n) - 1];
      }
    }
  }
}

// The tuner's coarse order (tune_parameters.cu:533-546): host-form squared
// distances (g++ for x86-64 without FMA: `dist += diff*diff` rounds the
// product and the sum separately) and std::sort over (distance, list id).
// order[i][r] = list at 0-based position r; rank_of[i][c] = 1-based position.
void orc_tune_coarse_order(const float* q, int nq, const float* cent, int nlist, int dim, int* order,
                           int* rank_of, int nthreads) {
  set_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int i = 0; i < nq; ++i) {
    std::vector<std::pair<float, int>> v(nlist);
    for (int c = 0; c < nlist; ++c) {
      float dist = 0.0f;
      for (int d = 0; d < dim; ++d) {
        const float diff = q[(size_t)i * dim + d] - cent[(size_t)c * dim + d];
        const float sq = diff * diff;
        dist = dist + sq;
      }
      v[c] = {dist, c};
    }
    std::sort(v.begin(), v.end());
    for (int r = 0; r < nlist; ++r) {
      order[(size_t)i * nlist + r] = v[r].second;
      rank_of[(size_t)i * nlist + v[r].second] = r + 1;
    }
  }
}

}  // extern "C"
