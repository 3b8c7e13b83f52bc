// compat_driver.cpp -- test driver for include/fusiongpu_compat.hpp: calls the
// reference-signature entry points the way the reference's callers do and
// writes their outputs as raw little-endian arrays for the GPU tests to
// compare with the oracle.
//
//   compat_driver search <res_dir> <queries.fvecs> <base.fvecs> <probes.u32> <probe_dists.f32> <out_dir>
//                 <top_m> <p1_lists> <limit_k> <threshold_coeff> <rerank_m> <final_k> <mini_batch> <eps>
//                 <beta> <prune_ratio> <batch>
//     load_ivf_index_to_gpu, then per batch of queries (search_pipeline.cu:311-372):
//     run_gpu_batch_logic on the given probes (the coarse step's output) and
//     run_gpu_rerank.  The pool starts with room for 16 ints, so the first
//     batch takes the reallocation path.
//   compat_driver build <base.fvecs> <k> <kmeans_iters> <sample_size> <pq_iters> <out_dir>
//     build_global's calls (build_global.cu:41-57, 202-220): run_kmeans_gpu,
//     gpu_assign_to_centroids, gpu_assign_initial_clusters,
//     train_residual_pq_codebooks, encode_residuals_to_pq_gpu and the host
//     twin encode_residuals_to_pq.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "fusiongpu_compat.hpp"

namespace {

std::vector<float> read_fvecs(const std::string& path, int dim, int64_t& n) {
  if (fgpu_read_fvecs(path.c_str(), dim, &n, nullptr) != FGPU_OK) throw std::runtime_error(fgpu_last_error());
  std::vector<float> v((size_t)n * dim);
  if (fgpu_read_fvecs(path.c_str(), dim, &n, v.data()) != FGPU_OK) throw std::runtime_error(fgpu_last_error());
  return v;
}

template <class T>
std::vector<T> read_raw(const std::string& path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::vector<T> v((size_t)f.tellg() / sizeof(T));
  f.seekg(0);
  f.read(reinterpret_cast<char*>(v.data()), v.size() * sizeof(T));
  return v;
}

template <class T>
void write_raw(const std::string& path, const T* p, size_t count) {
  std::ofstream f(path, std::ios::binary);
  f.write(reinterpret_cast<const char*>(p), count * sizeof(T));
  if (!f) throw std::runtime_error("cannot write " + path);
}

void hip(hipError_t e) {
  if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
}

int search(char** a) {
  const std::string res = a[2], qpath = a[3], bpath = a[4], ppath = a[5], pdpath = a[6], out = a[7];
  const int top_m = std::atoi(a[8]), p1 = std::atoi(a[9]), limit_k = std::atoi(a[10]);
  const float coeff = (float)std::atof(a[11]);
  const int rerank_m = std::atoi(a[12]), final_k = std::atoi(a[13]), mb = std::atoi(a[14]);
  const float eps = (float)std::atof(a[15]);
  const int beta = std::atoi(a[16]);
  const float prune = (float)std::atof(a[17]);
  const int batch = std::atoi(a[18]);
  hipStream_t s;
  hip(hipStreamCreate(&s));
  IVFIndexGPU idx{};
  load_ivf_index_to_gpu(res, idx, s);
  int64_t nq = 0, nb = 0;
  std::vector<float> q = read_fvecs(qpath, DIM, nq), base = read_fvecs(bpath, DIM, nb);
  std::vector<uint32_t> probes = read_raw<uint32_t>(ppath);
  std::vector<float> pdist = read_raw<float>(pdpath);
  if ((int64_t)probes.size() != nq * top_m || pdist.size() != probes.size()) throw std::runtime_error("probe shape");
  float *d_q, *d_base, *d_pd, *d_td, *d_fd, *d_cut, *d_thr;
  uint32_t* d_p;
  int *d_counts, *d_offsets, *d_atomic, *d_tid, *d_tcnt, *d_fid, *d_st, *d_comp;
  bool* d_fin;
  const int p1e = top_m < p1 ? top_m : p1;
  hip(hipMalloc(&d_q, sizeof(float) * batch * DIM));
  hip(hipMalloc(&d_base, sizeof(float) * base.size()));
  hip(hipMalloc(&d_p, sizeof(uint32_t) * batch * top_m));
  hip(hipMalloc(&d_pd, sizeof(float) * batch * top_m));
  hip(hipMalloc(&d_counts, sizeof(int) * batch));
  hip(hipMalloc(&d_offsets, sizeof(int) * (batch + 1)));
  hip(hipMalloc(&d_atomic, sizeof(int) * batch));
  hip(hipMalloc(&d_comp, sizeof(int) * (batch + 1)));
  hip(hipMalloc(&d_tid, sizeof(int) * batch * rerank_m));
  hip(hipMalloc(&d_td, sizeof(float) * batch * rerank_m));
  hip(hipMalloc(&d_tcnt, sizeof(int) * batch));
  hip(hipMalloc(&d_cut, sizeof(float) * batch * (p1e > 0 ? p1e : 1)));
  hip(hipMalloc(&d_thr, sizeof(float) * batch));
  hip(hipMalloc(&d_fid, sizeof(int) * batch * final_k));
  hip(hipMalloc(&d_fd, sizeof(float) * batch * final_k));
  hip(hipMalloc(&d_st, sizeof(int) * batch));
  hip(hipMalloc(&d_fin, sizeof(bool) * batch));
  hip(hipMemcpy(d_base, base.data(), sizeof(float) * base.size(), hipMemcpyHostToDevice));
  size_t cap = 16;
  int *d_flat_ids, *d_flat_ids_alt;
  float *d_flat_dists, *d_flat_dists_alt;
  hip(hipMalloc(&d_flat_ids, cap * sizeof(int)));
  hip(hipMalloc(&d_flat_dists, cap * sizeof(float)));
  hip(hipMalloc(&d_flat_ids_alt, cap * sizeof(int)));
  hip(hipMalloc(&d_flat_dists_alt, cap * sizeof(float)));
  BatchLogicEvents ev{};
  for (hipEvent_t* e : {&ev.evt_start, &ev.evt_prune_count, &ev.evt_precompute, &ev.evt_scan_offset,
                        &ev.evt_resize_sync, &ev.evt_scan_phase1_end, &ev.evt_scan_cand, &ev.evt_compact, &ev.evt_sort,
                        &ev.evt_gather})
    hip(hipEventCreate(e));
  std::vector<uint32_t> pruned(probes.size());
  std::vector<int> tid((size_t)nq * rerank_m), tcnt(nq), counts(nq), atomic(nq), fid((size_t)nq * final_k), stab(nq);
  std::vector<uint8_t> fin(nq);
  std::vector<float> td((size_t)nq * rerank_m), cut((size_t)nq * (p1e > 0 ? p1e : 1)), thr(nq),
      fd((size_t)nq * final_k);
  std::vector<int> offs_last;
  int grows = 0;
  for (int64_t b0 = 0; b0 < nq; b0 += batch) {
    const int bs = (int)std::min<int64_t>(batch, nq - b0);
    hip(hipMemcpyAsync(d_q, q.data() + b0 * DIM, sizeof(float) * bs * DIM, hipMemcpyHostToDevice, s));
    hip(hipMemcpyAsync(d_p, probes.data() + b0 * top_m, sizeof(uint32_t) * bs * top_m, hipMemcpyHostToDevice, s));
    hip(hipMemcpyAsync(d_pd, pdist.data() + b0 * top_m, sizeof(float) * bs * top_m, hipMemcpyHostToDevice, s));
    const size_t cap0 = cap;
    run_gpu_batch_logic(idx, d_q, d_p, d_pd, nullptr, d_flat_ids, d_flat_dists, d_flat_ids_alt, d_flat_dists_alt, cap,
                        d_counts, d_offsets, d_atomic, d_tid, d_td, d_tcnt, bs, top_m, rerank_m, final_k, prune, d_cut,
                        d_thr, d_comp, s, &ev, p1, limit_k, coeff);
    grows += cap != cap0;
    run_gpu_rerank(d_q, d_tid, d_tcnt, d_base, d_fid, d_fd, d_st, d_fin, bs, rerank_m, final_k, (int)nb, mb, eps, beta,
                   s);
    hip(hipMemcpyAsync(pruned.data() + b0 * top_m, d_p, sizeof(uint32_t) * bs * top_m, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(tid.data() + b0 * rerank_m, d_tid, sizeof(int) * bs * rerank_m, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(td.data() + b0 * rerank_m, d_td, sizeof(float) * bs * rerank_m, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(tcnt.data() + b0, d_tcnt, sizeof(int) * bs, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(counts.data() + b0, d_counts, sizeof(int) * bs, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(atomic.data() + b0, d_atomic, sizeof(int) * bs, hipMemcpyDeviceToHost, s));
    if (p1e > 0)
      hip(hipMemcpyAsync(cut.data() + b0 * p1e, d_cut, sizeof(float) * bs * p1e, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(thr.data() + b0, d_thr, sizeof(float) * bs, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(fid.data() + b0 * final_k, d_fid, sizeof(int) * bs * final_k, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(fd.data() + b0 * final_k, d_fd, sizeof(float) * bs * final_k, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(stab.data() + b0, d_st, sizeof(int) * bs, hipMemcpyDeviceToHost, s));
    hip(hipMemcpyAsync(fin.data() + b0, d_fin, sizeof(bool) * bs, hipMemcpyDeviceToHost, s));
    offs_last.assign(bs + 1, 0);
    hip(hipMemcpyAsync(offs_last.data(), d_offsets, sizeof(int) * (bs + 1), hipMemcpyDeviceToHost, s));
    hip(hipStreamSynchronize(s));
    float t = 0.0f;
    hip(hipEventElapsedTime(&t, ev.evt_start, ev.evt_gather));
    if (!(t >= 0.0f)) throw std::runtime_error("stage events not recorded");
    int acc = 0;
    for (int i = 0; i < bs; ++i) {
      if (offs_last[i] != acc) throw std::runtime_error("d_offsets is not the exclusive scan of d_counts");
      acc += counts[b0 + i];
    }
    if (offs_last[bs] != acc) throw std::runtime_error("d_offsets[batch] is not the total");
  }
  write_raw(out + "/pruned.u32", pruned.data(), pruned.size());
  write_raw(out + "/top_ids.i32", tid.data(), tid.size());
  write_raw(out + "/top_dists.f32", td.data(), td.size());
  write_raw(out + "/top_counts.i32", tcnt.data(), tcnt.size());
  write_raw(out + "/counts.i32", counts.data(), counts.size());
  write_raw(out + "/atomic.i32", atomic.data(), atomic.size());
  write_raw(out + "/cutoffs.f32", cut.data(), cut.size());
  write_raw(out + "/thresholds.f32", thr.data(), thr.size());
  write_raw(out + "/final_ids.i32", fid.data(), fid.size());
  write_raw(out + "/final_dists.f32", fd.data(), fd.size());
  write_raw(out + "/stable.i32", stab.data(), stab.size());
  write_raw(out + "/finished.u8", fin.data(), fin.size());
  std::printf("search ok: %lld queries, %d batches, pool grew %d time(s) to %zu ints, num_clusters %d\n",
              (long long)nq, (int)((nq + batch - 1) / batch), grows, cap, idx.num_clusters);
  fgpu_compat_release_index(idx);
  return 0;
}

int build(char** a) {
  const std::string bpath = a[2], out = a[7];
  const int k = std::atoi(a[3]), iters = std::atoi(a[4]), sample = std::atoi(a[5]), pq_iters = std::atoi(a[6]);
  int64_t n64 = 0;
  std::vector<float> x = read_fvecs(bpath, DIM, n64);
  const int n = (int)n64;
  std::vector<float> cent;
  run_kmeans_gpu(x.data(), n, DIM, k, cent, iters);
  std::vector<int> assign;
  gpu_assign_to_centroids(x.data(), cent.data(), n, DIM, k, assign);
  std::vector<std::vector<int>> buckets;
  gpu_assign_initial_clusters(x.data(), cent.data(), n, DIM, k, buckets);
  size_t seen = 0;
  for (int c = 0; c < k; ++c)
    for (size_t j = 0; j < buckets[c].size(); ++j) {
      const int i = buckets[c][j];
      if (assign[i] != c || (j > 0 && buckets[c][j - 1] >= i)) throw std::runtime_error("buckets disagree");
      ++seen;
    }
  if (seen != (size_t)n) throw std::runtime_error("buckets do not cover every row");
  const auto* pts = reinterpret_cast<const point_t<float>*>(x.data());
  std::vector<float> codebook;
  train_residual_pq_codebooks(pts, n, assign, cent, codebook, sample, pq_iters);
  std::vector<uint8_t> codes_dev((size_t)n * PQ_M), codes_host((size_t)n * PQ_M);
  encode_residuals_to_pq_gpu(x.data(), n, DIM, assign, cent, codebook, codes_dev.data(), PQ_M, PQ_K, PQ_SUB_DIM);
  encode_residuals_to_pq(pts, n, assign, cent, codebook, codes_host.data());
  cleanup_kmeans_gpu();
  write_raw(out + "/centroids.f32", cent.data(), cent.size());
  write_raw(out + "/assign.i32", assign.data(), assign.size());
  write_raw(out + "/codebook.f32", codebook.data(), codebook.size());
  write_raw(out + "/codes_dev.u8", codes_dev.data(), codes_dev.size());
  write_raw(out + "/codes_host.u8", codes_host.data(), codes_host.size());
  std::printf("build ok: %d rows, %d centroids\n", n, k);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc == 19 && std::string(argv[1]) == "search") return search(argv);
    if (argc == 8 && std::string(argv[1]) == "build") return build(argv);
  } catch (const fgpu_compat_error& e) {
    std::fprintf(stderr, "fgpu_compat_error (status %d): %s\n", (int)e.status, e.what());
    return 3;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 2;
  }
  std::fprintf(stderr, "usage: compat_driver search ... | build ...\n");
  return 1;
}
