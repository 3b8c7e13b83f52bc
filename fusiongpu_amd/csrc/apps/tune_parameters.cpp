// tune_parameters -- offline parameter tuner, drop-in for the reference's
// tune_parameters (tune_parameters.cu:1122-1224):
//   tune_parameters <base.fvecs> [-n samples] [-k topk] [-o search_config.txt]
//     [--seed S] [--pq_m M] [--res DIR] [--samples_out ids.ivecs]
// It loads <res>/ivf_data.bin + global_pq_codebook.bin (default ../res, as the
// reference), samples -n base vectors as queries, and recommends:
//   RECOMMENDED_TOP_M    the P99.5 of the coarse ranks of the queries' exact
//                        k nearest neighbours' lists (:586-591);
//   RECOMMENDED_P1_LISTS the elbow of the hits per coarse rank (:593-610);
//   RECOMMENDED_LIMIT_K  the largest PQ rank, inside its own list, of a
//                        neighbour whose list is among the first P1_LISTS
//                        (:798-803; P98 of all PQ ranks when there is none);
//   THRESHOLD_COEFF      the largest ratio, over queries, of the farthest
//                        neighbour's PQ distance to the smallest LIMIT_K-th PQ
//                        distance of the first P1_LISTS lists (:827-988).
// and writes them as KEY=VALUE lines (save_tune_results, :1015-1053).
//
// Differences from the reference, each for a stated reason:
//   * sampling is seeded (--seed, default 42); the reference seeds from
//     std::random_device (:479-480), so its runs cannot be repeated;
//     --samples_out records the sampled base rows (one-column ivecs);
//   * a vector id's list comes from an inverse map built once (the reference
//     searches every list linearly per neighbour, :553-564); with a valid
//     index both name the same, first, list;
//   * the ground truth is this library's exact kNN (fgpu_knn_exact), equal to
//     brute_force_search_kernel (:49-96) under the same tie rule, and the
//     per-item PQ/exact statistics run as one batched device call
//     (fgpu_tune_list_stats) instead of a cudaMalloc and three kernels per
//     item (:690-749);
//   * the coarse ranking stays on the host with the reference's host form of
//     the squared distance (:39-46, a plain multiply-add loop, no fusion) and
//     std::sort over (distance, list id) pairs (:538-546).
#include <algorithm>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <random>

#include "app_common.hpp"

using app::Dev;
using app::hip_ok;
using app::ok;

namespace {

// euclidean_distance_sq as the reference's host code computes it (:39-46).
float host_l2(const float* a, const float* b, int dim) {
  float dist = 0.0f;
  for (int i = 0; i < dim; ++i) {
    const float diff = a[i] - b[i];
    dist += diff * diff;
  }
  return dist;
}

// Coarse order of every list for one query: rank_of[c] = 1-based position.
void coarse_order(const float* q, const std::vector<float>& cent, int nlist, int dim,
                  std::vector<std::pair<float, int>>& order, std::vector<int>& rank_of) {
  order.resize(nlist);
  for (int c = 0; c < nlist; ++c) order[c] = {host_l2(q, cent.data() + (size_t)c * dim, dim), c};
  std::sort(order.begin(), order.end());
  rank_of.assign(nlist, 0);
  for (int r = 0; r < nlist; ++r) rank_of[order[r].second] = r + 1;
}

void print_deciles(const char* title, std::vector<double> v, int prec) {
  std::cout << "\n" << title << ":" << std::endl;
  if (v.empty()) {
    std::cout << "  (none)" << std::endl;
    return;
  }
  std::sort(v.begin(), v.end());
  for (int p = 10; p <= 100; p += 10) {
    long long idx = (long long)(v.size() * p / 100.0) - 1;
    if (idx < 0) idx = 0;
    if (idx >= (long long)v.size()) idx = (long long)v.size() - 1;
    std::cout << "  P" << p << ": " << std::fixed << std::setprecision(prec) << v[(size_t)idx] << std::endl;
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::cerr << "Usage: ./tune_parameters <base.fvecs> [options]\n"
                 "  -n <num>     sampled queries (default 1000)\n"
                 "  -k <num>     target top-k (default 10)\n"
                 "  -o <file>    output config file (default search_config.txt)\n"
                 "  --seed <s>   sampling seed (default 42)\n"
                 "  --pq_m <m>   PQ subspaces of the index (default 32)\n"
                 "  --res <dir>  index directory (default ../res)\n"
                 "  --samples_out <file>  write the sampled base rows as ivecs\n";
    return 1;
  }
  std::string base_path = argv[1], out_path = "search_config.txt", res = "../res", samples_out;
  int n_samples = 1000, final_k = 10, pq_m = 32;
  unsigned long long seed = 42;
  for (int i = 2; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) {
        std::cerr << "missing value for " << a << "\n";
        std::exit(1);
      }
      return argv[++i];
    };
    if (a == "-n") n_samples = std::atoi(next());
    else if (a == "-k") final_k = std::atoi(next());
    else if (a == "-o") out_path = next();
    else if (a == "--seed") seed = std::strtoull(next(), nullptr, 10);
    else if (a == "--pq_m") pq_m = std::atoi(next());
    else if (a == "--res") res = next();
    else if (a == "--samples_out") samples_out = next();
    else {
      std::cerr << "unknown argument " << a << "\n";
      return 1;
    }
  }
  if (n_samples < 1 || final_k < 1 || final_k > 128) {
    std::cerr << "need -n >= 1 and 1 <= -k <= 128\n";
    return 1;
  }

  std::cout << "========== Parameter tuning ==========" << std::endl;
  std::cout << "dataset: " << base_path << "\nsamples: " << n_samples << "\ntarget top-k: " << final_k
            << "\noutput: " << out_path << "\nseed: " << seed << std::endl;
  const int dim = app::fvecs_dim(base_path);
  int64_t n_base = 0;
  const std::vector<float> base = app::read_fvecs(base_path, dim, n_base);
  std::cout << "dataset size: " << n_base << " vectors of dim " << dim << std::endl;
  if (n_base < 1) {
    std::cerr << "empty dataset\n";
    return 1;
  }

  if (pq_m < 1 || dim % pq_m != 0) {
    std::cerr << "dimension " << dim << " is not a multiple of pq_m " << pq_m << "\n";
    return 1;
  }
  // Index, on the host (coarse ranking, inverse map) and in HBM.
  int64_t total = 0;
  int nlist = 0;
  const std::string ivf = res + "/ivf_data.bin", cbf = res + "/global_pq_codebook.bin";
  ok(fgpu_read_ivf_header(ivf.c_str(), &total, &nlist), ("reading " + ivf).c_str());
  std::vector<int32_t> offsets(nlist + 1), ids(total);
  std::vector<uint8_t> codes((size_t)total * pq_m);
  std::vector<float> cent((size_t)nlist * dim);
  ok(fgpu_read_ivf_data(ivf.c_str(), pq_m, dim, offsets.data(), ids.data(), codes.data(), cent.data()),
     ("reading " + ivf).c_str());
  std::vector<float> cb((size_t)pq_m * 256 * (dim / pq_m));
  {
    std::ifstream f(cbf, std::ios::binary);
    f.read(reinterpret_cast<char*>(cb.data()), sizeof(float) * cb.size());
    if (!f.good()) {
      std::cerr << "cannot read " << cbf << " (" << cb.size() << " floats expected)\n";
      return 1;
    }
  }
  fgpu_index* idx = nullptr;
  ok(fgpu_index_create(dim, pq_m, nlist, total, offsets.data(), ids.data(), codes.data(), cent.data(), cb.data(),
                       &idx),
     "index");
  std::cout << "lists: " << nlist << "\nindexed vectors: " << total << std::endl;
  // A vector id's list: the first list, in list order, that holds it.
  std::vector<int32_t> list_of;
  for (int c = 0; c < nlist; ++c)
    for (int j = offsets[c]; j < offsets[c + 1]; ++j) {
      const int32_t v = ids[j];
      if (v < 0) continue;
      if ((size_t)v >= list_of.size()) list_of.resize((size_t)v + 1, -1);
      if (list_of[v] < 0) list_of[v] = c;
    }
  auto list_of_id = [&](int32_t v) { return (v >= 0 && (size_t)v < list_of.size()) ? list_of[v] : -1; };

  // [1/4] sampled queries (tune_parameters.cu:478-492, seeded).
  std::cout << "\n[1/4] sampling queries..." << std::endl;
  std::mt19937 gen((std::mt19937::result_type)seed);
  std::uniform_int_distribution<> dis(0, (int)(n_base - 1));
  std::vector<float> q((size_t)n_samples * dim);
  std::vector<int32_t> sampled(n_samples);
  for (int i = 0; i < n_samples; ++i) {
    const int s = dis(gen);
    sampled[i] = s;
    std::copy(base.begin() + (size_t)s * dim, base.begin() + (size_t)(s + 1) * dim, q.begin() + (size_t)i * dim);
  }
  if (!samples_out.empty()) {
    std::ofstream f(samples_out, std::ios::binary);
    const int32_t one = 1;
    for (int32_t v : sampled) {
      f.write(reinterpret_cast<const char*>(&one), 4);
      f.write(reinterpret_cast<const char*>(&v), 4);
    }
    if (!f.good()) {
      std::cerr << "cannot write " << samples_out << "\n";
      return 1;
    }
  }

  // [2/4] exact ground truth on the GPU.
  std::cout << "[2/4] exact ground truth (GPU)..." << std::endl;
  Dev<float> d_base((size_t)n_base * dim), d_q((size_t)n_samples * dim), d_gd((size_t)n_samples * final_k);
  Dev<int32_t> d_gi((size_t)n_samples * final_k);
  hip_ok(hipMemcpy(d_base.p, base.data(), sizeof(float) * base.size(), hipMemcpyHostToDevice), "copy base");
  hip_ok(hipMemcpy(d_q.p, q.data(), sizeof(float) * q.size(), hipMemcpyHostToDevice), "copy queries");
  const size_t ws = fgpu_knn_exact_workspace_bytes(n_samples, n_base);
  Dev<char> d_ws(ws);
  ok(fgpu_knn_exact(d_q.p, n_samples, d_base.p, n_base, dim, final_k, d_gi.p, d_gd.p, d_ws.p, ws, nullptr),
     "exact kNN");
  std::vector<int32_t> gt((size_t)n_samples * final_k);
  hip_ok(hipMemcpy(gt.data(), d_gi.p, sizeof(int32_t) * gt.size(), hipMemcpyDeviceToHost), "copy ground truth");

  // [3/4] coarse ranks of the neighbours' lists (:529-591) and the elbow (:593-610).
  std::cout << "\n[3/4] coarse ranks..." << std::endl;
  std::vector<std::vector<std::pair<float, int>>> order(n_samples);
  std::vector<std::vector<int>> rank_of(n_samples);
  std::vector<int32_t> cluster_ranks;
  int missing = 0;
  for (int i = 0; i < n_samples; ++i) {
    coarse_order(q.data() + (size_t)i * dim, cent, nlist, dim, order[i], rank_of[i]);
    for (int kk = 0; kk < final_k; ++kk) {
      const int c = list_of_id(gt[(size_t)i * final_k + kk]);
      if (c < 0) {
        ++missing;
        continue;
      }
      cluster_ranks.push_back(rank_of[i][c]);
    }
  }
  if (missing) std::cerr << "warning: " << missing << " ground-truth ids are in no list\n";
  if (cluster_ranks.empty()) {
    std::cerr << "no ground-truth id is indexed\n";
    return 1;
  }
  const int top_m = fgpu_tune_percentile_int(cluster_ranks.data(), (int64_t)cluster_ranks.size(), 0.995f);
  const int max_rank = *std::max_element(cluster_ranks.begin(), cluster_ranks.end());
  std::vector<int32_t> hits(max_rank, 0);
  for (int r : cluster_ranks) ++hits[r - 1];
  float elbow_cov = 0.0f;
  const int p1 = fgpu_tune_elbow(hits.data(), max_rank, (int64_t)cluster_ranks.size(), &elbow_cov);
  const double mean_rank =
      std::accumulate(cluster_ranks.begin(), cluster_ranks.end(), 0.0) / (double)cluster_ranks.size();
  std::cout << "  samples (queries x k): " << cluster_ranks.size() << "\n  mean rank: " << mean_rank
            << "\n  max rank: " << max_rank << "\n  hits per coarse rank (first 30):";
  for (int r = 0; r < std::min(30, max_rank); ++r) std::cout << (r % 10 ? " " : "\n    ") << hits[r];
  std::cout << "\n  [P99.5] RECOMMENDED_TOP_M: " << top_m << "\n  [elbow] RECOMMENDED_P1_LISTS: " << p1
            << " (coverage " << std::fixed << std::setprecision(2) << elbow_cov * 100.0f << "%)" << std::endl;

  // [4/4] PQ ranks inside the neighbours' own lists (:614-812).
  std::cout << "\n[4/4] PQ rank analysis (first " << p1 << " lists)..." << std::endl;
  std::vector<int32_t> pq_q, pq_l, pq_t, pq_in_p1;
  for (int i = 0; i < n_samples; ++i)
    for (int kk = 0; kk < final_k; ++kk) {
      const int32_t t = gt[(size_t)i * final_k + kk];
      const int c = list_of_id(t);
      if (c < 0 || offsets[c + 1] == offsets[c]) continue;
      pq_q.push_back(i);
      pq_l.push_back(c);
      pq_t.push_back(t);
      pq_in_p1.push_back(rank_of[i][c] <= std::min(p1, nlist));
    }
  const int np = (int)pq_q.size();
  std::vector<int32_t> pq_rank(np), ex_rank(np);
  if (np > 0) {
    Dev<int32_t> dq_(np), dl(np), dt(np), dpr(np), der(np);
    Dev<float> dtp(np), dte(np);
    hip_ok(hipMemcpy(dq_.p, pq_q.data(), 4 * (size_t)np, hipMemcpyHostToDevice), "copy pairs");
    hip_ok(hipMemcpy(dl.p, pq_l.data(), 4 * (size_t)np, hipMemcpyHostToDevice), "copy pairs");
    hip_ok(hipMemcpy(dt.p, pq_t.data(), 4 * (size_t)np, hipMemcpyHostToDevice), "copy pairs");
    ok(fgpu_tune_list_stats(idx, d_q.p, n_samples, d_base.p, n_base, dq_.p, dl.p, dt.p, nullptr, np, dtp.p, dte.p,
                            dpr.p, der.p, nullptr, nullptr),
       "list statistics");
    hip_ok(hipMemcpy(pq_rank.data(), dpr.p, 4 * (size_t)np, hipMemcpyDeviceToHost), "copy ranks");
    hip_ok(hipMemcpy(ex_rank.data(), der.p, 4 * (size_t)np, hipMemcpyDeviceToHost), "copy ranks");
  }
  std::vector<int32_t> all_pq, p1_pq;
  std::vector<double> all_ex_d, diffs_d, all_pq_d;
  for (int j = 0; j < np; ++j) {
    if (pq_rank[j] <= 0) continue;
    all_pq.push_back(pq_rank[j]);
    all_pq_d.push_back(pq_rank[j]);
    all_ex_d.push_back(ex_rank[j]);
    diffs_d.push_back((double)pq_rank[j] - ex_rank[j]);
    if (pq_in_p1[j]) p1_pq.push_back(pq_rank[j]);
  }
  const int limit_k = !p1_pq.empty() ? *std::max_element(p1_pq.begin(), p1_pq.end())
                                     : fgpu_tune_percentile_int(all_pq.data(), (int64_t)all_pq.size(), 0.98f);
  auto mean = [](const std::vector<double>& v) {
    return v.empty() ? 0.0 : std::accumulate(v.begin(), v.end(), 0.0) / (double)v.size();
  };
  std::cout << "  samples: " << all_pq.size() << " (inside the first P1_LISTS lists: " << p1_pq.size() << ")"
            << "\n  mean PQ rank: " << mean(all_pq_d) << "\n  mean exact rank: " << mean(all_ex_d)
            << "\n  mean rank difference (PQ - exact): " << mean(diffs_d)
            << "\n  RECOMMENDED_LIMIT_K: " << limit_k << std::endl;

  // Threshold coefficient (:815-988): per query, the smallest LIMIT_K-th PQ
  // distance over its first P1_LISTS non-empty lists and the farthest
  // neighbour's PQ distance in its own list.
  std::cout << "\nthreshold coefficient (P1_LISTS=" << p1 << ", LIMIT_K=" << limit_k << ")..." << std::endl;
  std::vector<int32_t> th_q, th_l, th_k, far_q, far_l, far_t;
  std::vector<int> first_pair(n_samples + 1, 0);
  for (int i = 0; i < n_samples; ++i) {
    first_pair[i] = (int)th_q.size();
    for (int r = 0; r < std::min(p1, nlist); ++r) {
      const int c = order[i][r].second;
      if (offsets[c + 1] == offsets[c]) continue;
      th_q.push_back(i);
      th_l.push_back(c);
      th_k.push_back(std::max(limit_k, 1));
    }
    const int32_t t = gt[(size_t)i * final_k + final_k - 1];
    far_q.push_back(i);
    far_l.push_back(std::max(list_of_id(t), 0));
    far_t.push_back(list_of_id(t) < 0 ? -1 : t);
  }
  first_pair[n_samples] = (int)th_q.size();
  const int nt = (int)th_q.size();
  std::vector<float> cut(nt), far_pq(n_samples);
  {
    Dev<int32_t> a1(std::max(nt, 1)), a2(std::max(nt, 1)), a3(std::max(nt, 1));
    Dev<float> kth(std::max(nt, 1));
    if (nt > 0) {
      hip_ok(hipMemcpy(a1.p, th_q.data(), 4 * (size_t)nt, hipMemcpyHostToDevice), "copy pairs");
      hip_ok(hipMemcpy(a2.p, th_l.data(), 4 * (size_t)nt, hipMemcpyHostToDevice), "copy pairs");
      hip_ok(hipMemcpy(a3.p, th_k.data(), 4 * (size_t)nt, hipMemcpyHostToDevice), "copy pairs");
      ok(fgpu_tune_list_stats(idx, d_q.p, n_samples, nullptr, 0, a1.p, a2.p, nullptr, a3.p, nt, nullptr, nullptr,
                              nullptr, nullptr, kth.p, nullptr),
         "list cutoffs");
      hip_ok(hipMemcpy(cut.data(), kth.p, 4 * (size_t)nt, hipMemcpyDeviceToHost), "copy cutoffs");
    }
    Dev<int32_t> b1(n_samples), b2(n_samples), b3(n_samples), r1(n_samples), r2(n_samples);
    Dev<float> tp(n_samples), te(n_samples);
    hip_ok(hipMemcpy(b1.p, far_q.data(), 4 * (size_t)n_samples, hipMemcpyHostToDevice), "copy pairs");
    hip_ok(hipMemcpy(b2.p, far_l.data(), 4 * (size_t)n_samples, hipMemcpyHostToDevice), "copy pairs");
    hip_ok(hipMemcpy(b3.p, far_t.data(), 4 * (size_t)n_samples, hipMemcpyHostToDevice), "copy pairs");
    ok(fgpu_tune_list_stats(idx, d_q.p, n_samples, nullptr, 0, b1.p, b2.p, b3.p, nullptr, n_samples, tp.p, te.p,
                            r1.p, r2.p, nullptr, nullptr),
       "farthest neighbours");
    hip_ok(hipMemcpy(far_pq.data(), tp.p, 4 * (size_t)n_samples, hipMemcpyDeviceToHost), "copy distances");
  }
  std::vector<float> ratios;
  for (int i = 0; i < n_samples; ++i) {
    if (first_pair[i] == first_pair[i + 1]) continue;  // no non-empty phase-1 list
    const float min_cut = *std::min_element(cut.begin() + first_pair[i], cut.begin() + first_pair[i + 1]);
    if (far_pq[i] < 0.0f) continue;  // farthest neighbour not indexed
    if (min_cut > 0.0f) ratios.push_back(far_pq[i] / min_cut);
  }
  const float coeff = ratios.empty() ? 2.0f : *std::max_element(ratios.begin(), ratios.end());
  std::vector<double> ratios_d(ratios.begin(), ratios.end());
  std::cout << "  valid samples: " << ratios.size();
  if (!ratios.empty())
    std::cout << "\n  mean ratio (farthest kNN PQ / min cutoff): "
              << std::accumulate(ratios.begin(), ratios.end(), 0.0f) / (float)ratios.size()
              << "\n  max ratio: " << coeff
              << "\n  P99 ratio: " << fgpu_tune_percentile(ratios.data(), (int64_t)ratios.size(), 0.99f);
  std::cout << "\n  THRESHOLD_COEFF (100% coverage): " << coeff << std::endl;

  std::cout << "\n========== Recommended parameters ==========\n"
            << "RECOMMENDED_TOP_M     = " << top_m << " (P99.5)\n"
            << "RECOMMENDED_P1_LISTS  = " << p1 << " (elbow)\n"
            << "RECOMMENDED_LIMIT_K   = " << limit_k << "\n"
            << "THRESHOLD_COEFF       = " << std::fixed << std::setprecision(3) << coeff << "\n"
            << "============================================" << std::endl;
  std::vector<double> cr(cluster_ranks.begin(), cluster_ranks.end());
  print_deciles("coarse rank distribution", cr, 0);
  print_deciles("PQ rank distribution (inside the list)", all_pq_d, 0);
  print_deciles("exact rank distribution (inside the list)", all_ex_d, 0);
  print_deciles("rank difference distribution (PQ - exact)", diffs_d, 0);
  print_deciles("ratio distribution", ratios_d, 3);

  std::ofstream ofs(out_path);
  if (!ofs) {
    std::cerr << "cannot create " << out_path << "\n";
    return 1;
  }
  ofs << "# Search parameter tuning results\n"
         "# written by tune_parameters\n\n"
         "# ===== coarse search range =====\n\n"
         "# TOP_M: lists probed per query (P99.5 of the neighbours' coarse ranks)\n"
      << "RECOMMENDED_TOP_M=" << top_m << "\n\n"
      << "# P1_LISTS: lists scanned densely in phase 1 (elbow of the hits per coarse rank)\n"
      << "RECOMMENDED_P1_LISTS=" << p1 << "\n\n"
      << "# ===== PQ distance parameters =====\n\n"
      << "# LIMIT_K: candidates kept per phase-1 list\n"
      << "RECOMMENDED_LIMIT_K=" << limit_k << "\n\n"
      << "# THRESHOLD_COEFF: phase-2 threshold = coeff * min(phase-1 cutoffs)\n"
      << "THRESHOLD_COEFF=" << std::fixed << std::setprecision(3) << coeff << "\n";
  ofs.close();
  std::cout << "\nconfig written to: " << out_path << std::endl;
  fgpu_index_destroy(idx);
  return 0;
}
