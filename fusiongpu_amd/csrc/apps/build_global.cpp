// build_global -- index build command, drop-in for the reference's
// build_global (build_global.cu:21-258): `build_global <base.fvecs> [options]`
// writes <res>/ivf_data.bin, <res>/global_pq_codebook.bin and
// cluster_distribution.csv in the reference's formats.
//
// Flow (build_global.cu): k-means over all rows (run_kmeans_gpu, 20
// iterations, the reference's strided init by default), assignment, the
// queue-based recursive split of every list above 2x the average size
// (local k-means of ceil(size/avg) centres, 15 iterations; :62-169), PQ
// training on a 50k sample, encoding and list assembly in bucket order.  The
// CAGRA index over the centroids is not built: the search ranks centroids
// exactly (fgpu_coarse_search).
//
// Options (defaults are the reference's compile-time values, defs.h:9-23):
//   --nlist N (2048)  --pq_m M (32)  --iters I (20)  --pq_iters I (8)
//   --sample S (50000)  --init strided|pp (strided)  --seed S (42)
//   --no-rebalance  --res DIR (../res)
//   --train_rows T: train the k-means on the rows floor(j*n/T), j < T (all rows
//     by default, as the reference does); every row is then assigned
//   --elbow L1,L2,...: before the build, run the k-means for each list count,
//     print its SSE (sum of exact squared distances of the training rows to
//     their nearest centroid) and build with the knee: the list count whose
//     normalised (log2 L, SSE) point lies farthest below the chord from the
//     first to the last point (the Kneedle rule)
#include <cmath>
#include <cstring>
#include <deque>
#include <fstream>
#include <iostream>
#include <numeric>

#include <sstream>

#include "app_common.hpp"

using app::Dev;
using app::hip_ok;
using app::ok;

namespace {

struct Bucket {
  std::vector<int32_t> rows;  // base rows, in the order they joined
  std::vector<float> centroid;
};

// Rows of x assigned to their nearest of k centroids (device arrays in, host out).
std::vector<int32_t> assign(const float* d_x, int64_t n, const float* d_c, int k, int dim) {
  Dev<int32_t> a(n);
  Dev<float> d(n);
  const size_t wb = fgpu_l2_topk_workspace_bytes(n, k);
  Dev<char> ws(wb);
  ok(fgpu_l2_topk(d_x, n, d_c, k, dim, 1, a.p, d.p, ws.p, wb, nullptr), "assignment");
  std::vector<int32_t> h(n);
  hip_ok(hipMemcpy(h.data(), a.p, sizeof(int32_t) * n, hipMemcpyDeviceToHost), "copy assignment");
  return h;
}

// Sum over rows of the exact squared distance to the nearest centroid.
double kmeans_sse(const float* d_x, int64_t n, const float* d_c, int k, int dim) {
  Dev<int32_t> a(n);
  Dev<float> d(n);
  const size_t wb = fgpu_l2_topk_workspace_bytes(n, k);
  Dev<char> ws(wb);
  ok(fgpu_l2_topk(d_x, n, d_c, k, dim, 1, a.p, d.p, ws.p, wb, nullptr), "SSE assignment");
  std::vector<float> h(n);
  hip_ok(hipMemcpy(h.data(), d.p, sizeof(float) * n, hipMemcpyDeviceToHost), "copy distances");
  double s = 0.0;
  for (float v : h) s += v;
  return s;
}

// Kneedle on a decreasing curve: normalise x = log2 L and y = SSE to [0, 1] and
// pick the point with the largest (chord - y); the first point on ties.
int knee(const std::vector<int>& L, const std::vector<double>& sse) {
  const size_t m = L.size();
  if (m < 3) return L[0];
  const double x0 = std::log2((double)L.front()), x1 = std::log2((double)L.back());
  const double y0 = sse.front(), y1 = sse.back();
  int best = L[0];
  double best_gap = -1.0;
  for (size_t i = 0; i < m; ++i) {
    const double xn = (std::log2((double)L[i]) - x0) / (x1 - x0);
    const double yn = (y0 == y1) ? 0.0 : (sse[i] - y1) / (y0 - y1);
    const double gap = (1.0 - xn) - yn;  // the chord from (0, 1) to (1, 0)
    if (gap > best_gap) {
      best_gap = gap;
      best = L[i];
    }
  }
  return best;
}

}  // namespace

int main(int argc, char** argv) {
  std::string base, res = "../res", init = "strided";
  int nlist = 2048, pq_m = 32, iters = 20, pq_iters = 8, sample = 50000;
  uint64_t seed = 42;
  bool rebalance = true;
  int64_t train_rows = 0;
  std::vector<int> elbow;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) { std::cerr << "missing value for " << a << "\n"; std::exit(1); }
      return argv[++i];
    };
    if (a == "--nlist") nlist = std::atoi(next());
    else if (a == "--pq_m") pq_m = std::atoi(next());
    else if (a == "--iters") iters = std::atoi(next());
    else if (a == "--pq_iters") pq_iters = std::atoi(next());
    else if (a == "--sample") sample = std::atoi(next());
    else if (a == "--init") init = next();
    else if (a == "--seed") seed = std::strtoull(next(), nullptr, 10);
    else if (a == "--res") res = next();
    else if (a == "--no-rebalance") rebalance = false;
    else if (a == "--train_rows") train_rows = std::atoll(next());
    else if (a == "--elbow") {
      std::stringstream ss(next());
      std::string tok;
      while (std::getline(ss, tok, ',')) elbow.push_back(std::atoi(tok.c_str()));
    }
    else if (!a.empty() && a[0] != '-' && base.empty()) base = a;
    else { std::cerr << "unknown argument " << a << "\n"; return 1; }
  }
  if (base.empty()) {
    std::cerr << "Usage: ./build_global <base.fvecs> [--nlist N] [--pq_m M] [--iters I] [--pq_iters I] "
                 "[--sample S] [--init strided|pp] [--seed S] [--no-rebalance] [--res DIR] [--train_rows T] "
                 "[--elbow L1,L2,...]\n";
    return 1;
  }
  const int dim = app::fvecs_dim(base);
  if (dim % pq_m != 0) { std::cerr << "dim " << dim << " is not a multiple of pq_m " << pq_m << "\n"; return 1; }
  int64_t n = 0;
  std::vector<float> h_x = app::read_fvecs(base, dim, n);
  std::cout << "Loaded " << n << " vectors." << std::endl;
  if (n < nlist) { std::cerr << "need at least nlist vectors\n"; return 1; }

  Dev<float> d_x((size_t)n * dim);
  hip_ok(hipMemcpy(d_x.p, h_x.data(), sizeof(float) * h_x.size(), hipMemcpyHostToDevice), "copy base");

  // training rows: all (the reference) or the systematic sample
  const float* d_train = d_x.p;
  int64_t nt = n;
  Dev<float> d_sample(train_rows > 0 && train_rows < n ? (size_t)train_rows * dim : 1);
  if (train_rows > 0 && train_rows < n) {
    std::vector<float> hs((size_t)train_rows * dim);
    for (int64_t j = 0; j < train_rows; ++j)
      std::memcpy(hs.data() + (size_t)j * dim, h_x.data() + (size_t)(j * n / train_rows) * dim, sizeof(float) * dim);
    hip_ok(hipMemcpy(d_sample.p, hs.data(), sizeof(float) * hs.size(), hipMemcpyHostToDevice), "copy sample");
    d_train = d_sample.p;
    nt = train_rows;
    std::cout << "Training on " << nt << " sampled rows." << std::endl;
  }
  const int initm = init == "pp" ? 1 : 0;
  if (!elbow.empty()) {
    std::vector<double> sse;
    for (int L : elbow) {
      if (L < 1 || L > nt) { std::cerr << "elbow list count " << L << " out of range\n"; return 1; }
      Dev<float> d_e((size_t)L * dim);
      ok(fgpu_kmeans_fit(d_train, nt, dim, L, iters, initm, seed, d_e.p, nullptr, nullptr), "elbow k-means");
      sse.push_back(kmeans_sse(d_train, nt, d_e.p, L, dim));
      std::cout << "Elbow: nlist " << L << " SSE " << sse.back() << std::endl;
    }
    nlist = knee(elbow, sse);
    std::cout << "Elbow: chosen nlist " << nlist << std::endl;
  }

  // k-means (run_kmeans_gpu, kmeans_gpu.cuh:234-324)
  std::cout << "Training " << nlist << " initial centroids (GPU)..." << std::endl;
  Dev<float> d_c((size_t)nlist * dim);
  ok(fgpu_kmeans_fit(d_train, nt, dim, nlist, iters, initm, seed, d_c.p, nullptr, nullptr), "k-means");
  std::cout << "Assigning vectors to initial clusters (GPU)..." << std::endl;
  std::vector<int32_t> a0 = assign(d_x.p, n, d_c.p, nlist, dim);
  std::vector<float> h_c((size_t)nlist * dim);
  hip_ok(hipMemcpy(h_c.data(), d_c.p, sizeof(float) * h_c.size(), hipMemcpyDeviceToHost), "copy centroids");

  std::vector<Bucket> buckets(nlist);
  for (int c = 0; c < nlist; ++c) buckets[c].centroid.assign(h_c.begin() + (size_t)c * dim, h_c.begin() + (size_t)(c + 1) * dim);
  for (int64_t i = 0; i < n; ++i) buckets[a0[i]].rows.push_back((int32_t)i);

  std::vector<Bucket> final_b;
  if (rebalance) {
    // Queue-based recursive split (build_global.cu:62-169).
    std::cout << "--- Advanced Recursive Rebalancing (Queue-based) ---" << std::endl;
    const double avg = (double)n / nlist;
    const size_t split_threshold = (size_t)(avg * 2), min_splittable = 32;
    std::cout << "Target Avg Size: " << avg << ", Split Threshold: " << split_threshold << std::endl;
    std::deque<Bucket> queue;
    for (auto& b : buckets)
      if (!b.rows.empty()) queue.push_back(std::move(b));
    int split_ops = 0;
    while (!queue.empty()) {
      Bucket t = std::move(queue.front());
      queue.pop_front();
      const size_t sz = t.rows.size();
      if (sz <= split_threshold || sz < min_splittable) {
        final_b.push_back(std::move(t));
        continue;
      }
      ++split_ops;
      int sub_k = (int)std::ceil((double)sz / avg);
      if (sub_k < 2) sub_k = 2;
      if (sub_k > (int)sz / 2) sub_k = (int)sz / 2;
      std::vector<float> sub((size_t)sz * dim);
      for (size_t i = 0; i < sz; ++i)
        std::memcpy(sub.data() + i * dim, h_x.data() + (size_t)t.rows[i] * dim, sizeof(float) * dim);
      Dev<float> d_sub(sub.size()), d_sc((size_t)sub_k * dim);
      hip_ok(hipMemcpy(d_sub.p, sub.data(), sizeof(float) * sub.size(), hipMemcpyHostToDevice), "copy subset");
      ok(fgpu_kmeans_fit(d_sub.p, (int64_t)sz, dim, sub_k, 15, initm, seed, d_sc.p, nullptr, nullptr),
         "local k-means");
      std::vector<int32_t> la = assign(d_sub.p, (int64_t)sz, d_sc.p, sub_k, dim);
      std::vector<float> sc((size_t)sub_k * dim);
      hip_ok(hipMemcpy(sc.data(), d_sc.p, sizeof(float) * sc.size(), hipMemcpyDeviceToHost), "copy sub-centroids");
      std::vector<Bucket> child(sub_k);
      for (size_t i = 0; i < sz; ++i) child[la[i]].rows.push_back(t.rows[i]);
      for (int k = 0; k < sub_k; ++k) {
        if (child[k].rows.empty()) continue;
        child[k].centroid.assign(sc.begin() + (size_t)k * dim, sc.begin() + (size_t)(k + 1) * dim);
        queue.push_back(std::move(child[k]));
      }
    }
    std::cout << "Rebalancing Complete." << std::endl;
    std::cout << "Split Ops: " << split_ops << std::endl;
    std::cout << "Cluster Count: " << nlist << " -> " << final_b.size() << std::endl;
  } else {
    for (auto& b : buckets) final_b.push_back(std::move(b));  // empty lists stay, as listed
  }
  const int L = (int)final_b.size();

  std::cout << "Exporting distribution stats..." << std::endl;
  {
    std::ofstream csv("cluster_distribution.csv");
    csv << "cluster_id,count\n";
    for (int c = 0; c < L; ++c) csv << c << "," << final_b[c].rows.size() << "\n";
  }

  std::vector<int32_t> vec_list(n, -1);
  std::vector<float> cent((size_t)L * dim);
  for (int c = 0; c < L; ++c) {
    for (int32_t r : final_b[c].rows) vec_list[r] = c;
    std::memcpy(cent.data() + (size_t)c * dim, final_b[c].centroid.data(), sizeof(float) * dim);
  }
  Dev<int32_t> d_a(n);
  Dev<float> d_cent(cent.size()), d_cb((size_t)pq_m * 256 * (dim / pq_m));
  Dev<uint8_t> d_codes((size_t)n * pq_m);
  hip_ok(hipMemcpy(d_a.p, vec_list.data(), sizeof(int32_t) * n, hipMemcpyHostToDevice), "copy assignment");
  hip_ok(hipMemcpy(d_cent.p, cent.data(), sizeof(float) * cent.size(), hipMemcpyHostToDevice), "copy centroids");

  std::cout << "Training Residual Global PQ..." << std::endl;
  ok(fgpu_pq_train(d_x.p, n, dim, pq_m, d_a.p, d_cent.p, sample, pq_iters, d_cb.p, nullptr), "PQ training");
  std::vector<float> cb((size_t)pq_m * 256 * (dim / pq_m));
  hip_ok(hipMemcpy(cb.data(), d_cb.p, sizeof(float) * cb.size(), hipMemcpyDeviceToHost), "copy codebook");
  {
    std::ofstream out(res + "/global_pq_codebook.bin", std::ios::binary);
    out.write(reinterpret_cast<const char*>(cb.data()), sizeof(float) * cb.size());
    if (!out.good()) { std::cerr << "cannot write " << res << "/global_pq_codebook.bin\n"; return 1; }
  }
  std::cout << "Encoding residuals (GPU)..." << std::endl;
  ok(fgpu_pq_encode(d_x.p, n, dim, pq_m, d_a.p, d_cent.p, d_cb.p, d_codes.p, nullptr), "PQ encoding");
  std::vector<uint8_t> codes((size_t)n * pq_m);
  hip_ok(hipMemcpy(codes.data(), d_codes.p, codes.size(), hipMemcpyDeviceToHost), "copy codes");

  std::cout << "Building Inverted Lists..." << std::endl;
  std::vector<int32_t> offsets(L + 1, 0), ids;
  std::vector<uint8_t> list_codes;
  ids.reserve(n);
  list_codes.reserve((size_t)n * pq_m);
  for (int c = 0; c < L; ++c) {
    offsets[c] = (int32_t)ids.size();
    for (int32_t r : final_b[c].rows) {
      ids.push_back(r);
      list_codes.insert(list_codes.end(), codes.begin() + (size_t)r * pq_m, codes.begin() + (size_t)(r + 1) * pq_m);
    }
  }
  offsets[L] = (int32_t)ids.size();
  ok(fgpu_write_ivf_data((res + "/ivf_data.bin").c_str(), (int64_t)ids.size(), L, pq_m, dim, offsets.data(), ids.data(),
                         list_codes.data(), cent.data()),
     "writing ivf_data.bin");
  std::cout << "Build complete." << std::endl;
  return 0;
}
