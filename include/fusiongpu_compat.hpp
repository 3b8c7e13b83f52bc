/* fusiongpu_compat.hpp -- the reference's C++ entry points, with the
 * reference's signatures, over the C ABI of libfusiongpu.so (fusiongpu.h).
 *
 * For the reference's own callers (Hello-day/FusionGPU search_pipeline.cu,
 * build_global.cu): include this header where they include defs.h,
 * kmeans_gpu.cuh and pq_utils.h, spell cudaStream_t / cudaEvent_t as
 * hipStream_t / hipEvent_t, and link libfusiongpu.so.  Header-only: the
 * reference fixes the geometry at compile time (DIM, PQ_M; defs.h:9-12), and
 * so does the caller here, by defining them before the include (defaults
 * below are the reference's).
 *
 * Kept from the reference: names, argument order and meaning, default
 * arguments, the IVFIndexGPU / BatchLogicEvents / point_t layouts, host
 * pointers in and out of the build functions, the pool buffers that
 * run_gpu_batch_logic may reallocate, the in-place prune of the probe ids.
 * Changed on purpose:
 *   * errors throw fgpu_compat_error (a std::runtime_error carrying the
 *     fgpu_status) where the reference calls exit(1) or ignores CUDA errors;
 *   * no hidden host synchronisation in run_gpu_batch_logic except when its
 *     pool must grow (the reference syncs twice per batch);
 *   * the reference's bugs are not reproduced (whole lists are scanned, no
 *     duplicate candidates, every rerank_m entry gathered, all k + mini_batch
 *     rerank entries sorted); ties follow (distance, id);
 *   * the coarse step's results arrive in d_cagra_top_m / d_cagra_dists as
 *     before; fgpu_coarse_search (exact) or fgpu_coarse_graph_search fill them.
 */
#ifndef FUSIONGPU_COMPAT_HPP_
#define FUSIONGPU_COMPAT_HPP_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <fstream>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "fusiongpu.h"

/* ---- geometry and defaults (defs.h:9-41) -------------------------------- */
#ifndef DIM
#define DIM 128
#endif
#ifndef PQ_M
#define PQ_M 32
#endif
#ifndef PQ_K
#define PQ_K 256
#endif
#ifndef PQ_SUB_DIM
#define PQ_SUB_DIM (DIM / PQ_M)
#endif
#ifndef K_CLUSTERS
#define K_CLUSTERS 2048
#endif
#ifndef DEFAULT_BATCH_SIZE
#define DEFAULT_BATCH_SIZE 128
#endif
#ifndef DEFAULT_TOP_M
#define DEFAULT_TOP_M 20
#endif
#ifndef DEFAULT_RERANK_M
#define DEFAULT_RERANK_M 10000
#endif
#ifndef DEFAULT_P1_LISTS
#define DEFAULT_P1_LISTS 12
#endif
#ifndef DEFAULT_LIMIT_K
#define DEFAULT_LIMIT_K 50
#endif
#ifndef DEFAULT_THRESHOLD_COEFF
#define DEFAULT_THRESHOLD_COEFF 1.0f
#endif
#ifndef DEFAULT_RERANK_MINI_BATCH
#define DEFAULT_RERANK_MINI_BATCH 128
#endif
#ifndef DEFAULT_RERANK_EPSILON
#define DEFAULT_RERANK_EPSILON 0.1f
#endif
#ifndef DEFAULT_RERANK_BETA
#define DEFAULT_RERANK_BETA 2
#endif

static_assert(PQ_K == 256, "libfusiongpu's codes are 8-bit (256 codewords per subspace)");
static_assert(DIM % PQ_M == 0, "DIM must be a multiple of PQ_M");

/* ---- types (defs.h:43-103) ---------------------------------------------- */
using pq_code_t = uint8_t;

template <typename T>
struct point_t {
  T coordinates[DIM];
};

/* The device index as the reference's callers hold it (defs.h:51-58).  The
 * reference's loader leaves num_clusters unset (search_pipeline.cu:481-529);
 * load_ivf_index_to_gpu below sets it, and run_gpu_batch_logic needs it. */
struct IVFIndexGPU {
  float* d_pq_codebook;    // [PQ_M][PQ_K][PQ_SUB_DIM]
  int* d_cluster_offsets;  // [num_clusters + 1]
  uint8_t* d_all_pq_codes; // [total][PQ_M], list-major
  int* d_all_vector_ids;   // [total]
  float* d_centroids;      // [num_clusters][DIM]
  int num_clusters;
};

/* Stage events of run_gpu_batch_logic (defs.h:61-80).  Here one fused kernel
 * does every stage after the prune and counts, so the scan-to-gather events
 * are recorded around it; the caller creates the ten events the reference
 * records (search_pipeline.cu:94-103). */
struct BatchLogicEvents {
  hipEvent_t evt_start;
  hipEvent_t evt_prune_count;
  hipEvent_t evt_precompute_p1;
  hipEvent_t evt_precompute;
  hipEvent_t evt_scan_offset;
  hipEvent_t evt_resize_sync;
  hipEvent_t evt_scan_phase1_end;
  hipEvent_t evt_d2h_p1_start;
  hipEvent_t evt_d2h_p1_end;
  hipEvent_t evt_precompute_p2;
  hipEvent_t evt_h2d_threshold;
  hipEvent_t evt_scan_cand;
  hipEvent_t evt_compact;
  hipEvent_t evt_sort;
  hipEvent_t evt_gather;
};

/* Per-stage timings the reference's pipeline fills (defs.h:83-103). */
struct GPUStageTimings {
  float prune_count_ms = 0;
  float precompute_p1_ms = 0;
  float precompute_ms = 0;
  float scan_offset_ms = 0;
  float resize_sync_ms = 0;
  float scan_phase1_ms = 0;
  float d2h_p1_ms = 0;
  float cpu_sort_ms = 0;
  float precompute_p2_ms = 0;
  float h2d_threshold_ms = 0;
  float scan_phase2_ms = 0;
  float compact_ms = 0;
  float sort_ms = 0;
  float gather_ms = 0;
  float total_ms = 0;
  long long total_candidates = 0;
  long long total_max_candidates = 0;
};

/* A failed call: the fgpu_status and the library's message. */
struct fgpu_compat_error : std::runtime_error {
  fgpu_status status;
  fgpu_compat_error(fgpu_status st, const std::string& msg) : std::runtime_error(msg), status(st) {}
};

namespace fgpu_compat_detail {

inline void check(fgpu_status st, const char* what) {
  if (st != FGPU_OK) throw fgpu_compat_error(st, std::string(what) + ": " + fgpu_last_error());
}

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw fgpu_compat_error(FGPU_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

/* Device buffer owned for the length of one host-pointer build call (the
 * reference's build functions allocate and free the same way). */
template <class T>
struct dev_buf {
  T* p = nullptr;
  explicit dev_buf(size_t count) { hip_check(hipMalloc(&p, (count ? count : 1) * sizeof(T)), "hipMalloc"); }
  ~dev_buf() { if (p) (void)hipFree(p); }
  dev_buf(const dev_buf&) = delete;
  dev_buf& operator=(const dev_buf&) = delete;
  void upload(const T* h, size_t count) {
    if (count) hip_check(hipMemcpy(p, h, count * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  void download(T* h, size_t count) const {
    if (count) hip_check(hipMemcpy(h, p, count * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
  }
};

using view_key = std::tuple<const void*, const void*, const void*, const void*, const void*, int>;

inline std::mutex& view_mutex() {
  static std::mutex mu;
  return mu;
}
inline std::map<view_key, fgpu_index*>& view_map() {
  static std::map<view_key, fgpu_index*> views;
  return views;
}

/* The library's handle over the caller's IVFIndexGPU arrays (fgpu_index_wrap),
 * made on first use and kept until fgpu_compat_release_index.  Its derived
 * arrays (list radii, centroid norms) describe the arrays' contents at that
 * time: release it before changing or freeing them. */
inline fgpu_index* view(const IVFIndexGPU& idx, hipStream_t s) {
  if (idx.num_clusters <= 0)
    throw fgpu_compat_error(FGPU_ERR_ARG, "IVFIndexGPU.num_clusters must be set (load_ivf_index_to_gpu sets it)");
  const view_key key{idx.d_pq_codebook, idx.d_cluster_offsets, idx.d_all_pq_codes, idx.d_all_vector_ids,
                     idx.d_centroids, idx.num_clusters};
  std::lock_guard<std::mutex> lock(view_mutex());
  auto it = view_map().find(key);
  if (it != view_map().end()) return it->second;
  fgpu_index* ix = nullptr;
  check(fgpu_index_wrap(DIM, PQ_M, idx.num_clusters, idx.d_cluster_offsets, idx.d_all_vector_ids,
                        idx.d_all_pq_codes, idx.d_centroids, idx.d_pq_codebook, s, &ix),
        "IVFIndexGPU");
  view_map()[key] = ix;
  return ix;
}

inline void record(hipEvent_t e, hipStream_t s) { hip_check(hipEventRecord(e, s), "hipEventRecord"); }

}  // namespace fgpu_compat_detail

/* The library's handle over these arrays (no reference counterpart), for the
 * C-ABI calls a port adds, such as the coarse step that replaces CAGRA:
 * fgpu_coarse_search(fgpu_compat_handle(idx, s), ...). */
inline fgpu_index* fgpu_compat_handle(const IVFIndexGPU& idx, hipStream_t stream = nullptr) {
  return fgpu_compat_detail::view(idx, stream);
}

/* Drops the library's handle over these arrays (no reference counterpart;
 * the reference never frees its index). */
inline void fgpu_compat_release_index(const IVFIndexGPU& idx) {
  namespace d = fgpu_compat_detail;
  std::lock_guard<std::mutex> lock(d::view_mutex());
  auto& m = d::view_map();
  for (auto it = m.begin(); it != m.end();) {
    if (std::get<0>(it->first) == idx.d_pq_codebook && std::get<1>(it->first) == idx.d_cluster_offsets) {
      fgpu_index_destroy(it->second);
      it = m.erase(it);
    } else {
      ++it;
    }
  }
}

/* ---- search ---------------------------------------------------------------- */

/* load_ivf_index_to_gpu (search_pipeline.cu:481-529): res_dir/global_pq_codebook.bin
 * and res_dir/ivf_data.bin into newly allocated device arrays, copies on
 * `stream` when given.  Sets num_clusters; waits for the copies. */
inline void load_ivf_index_to_gpu(const std::string& res_dir, IVFIndexGPU& idx, hipStream_t stream = nullptr) {
  namespace d = fgpu_compat_detail;
  const std::string ivf = res_dir + "/ivf_data.bin", cbp = res_dir + "/global_pq_codebook.bin";
  std::vector<float> codebook((size_t)PQ_M * PQ_K * PQ_SUB_DIM);
  {
    std::ifstream f(cbp, std::ios::binary | std::ios::ate);
    if (!f) throw fgpu_compat_error(FGPU_ERR_IO, "cannot open " + cbp);
    if ((size_t)f.tellg() != codebook.size() * sizeof(float))
      throw fgpu_compat_error(FGPU_ERR_IO, cbp + ": size does not match PQ_M * PQ_K * PQ_SUB_DIM floats");
    f.seekg(0);
    f.read(reinterpret_cast<char*>(codebook.data()), codebook.size() * sizeof(float));
  }
  int64_t total = 0;
  int nlist = 0;
  d::check(fgpu_read_ivf_header(ivf.c_str(), &total, &nlist), "load_ivf_index_to_gpu");
  std::vector<int32_t> offsets(nlist + 1), ids(total);
  std::vector<uint8_t> codes((size_t)total * PQ_M);
  std::vector<float> centroids((size_t)nlist * DIM);
  d::check(fgpu_read_ivf_data(ivf.c_str(), PQ_M, DIM, offsets.data(), ids.data(), codes.data(), centroids.data()),
           "load_ivf_index_to_gpu");
  auto put = [&](void** dst, const void* src, size_t bytes, size_t pad) {
    d::hip_check(hipMalloc(dst, bytes + pad), "hipMalloc");
    if (bytes) d::hip_check(hipMemcpyAsync(*dst, src, bytes, hipMemcpyHostToDevice, stream), "hipMemcpyAsync");
  };
  put((void**)&idx.d_pq_codebook, codebook.data(), codebook.size() * sizeof(float), 0);
  put((void**)&idx.d_cluster_offsets, offsets.data(), offsets.size() * sizeof(int32_t), 0);
  put((void**)&idx.d_all_vector_ids, ids.data(), ids.size() * sizeof(int32_t), 0);
  put((void**)&idx.d_all_pq_codes, codes.data(), codes.size(), 256);
  put((void**)&idx.d_centroids, centroids.data(), centroids.size() * sizeof(float), 0);
  idx.num_clusters = nlist;
  d::hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

/* run_gpu_batch_logic (gpu_global.cu:679-874), the per-batch search after the
 * coarse step: prune d_cagra_top_m in place (prune_ratio against each
 * query's first distance), counts and offsets of the surviving probes into
 * d_counts / d_offsets (d_offsets[batch_size] = total), then the two-phase
 * scan (p1_lists, limit_k, threshold_coeff) and the top rerank_m into
 * d_top_ids / d_top_dists [batch_size][rerank_m] (pad -1 / FLT_MAX) and
 * d_top_counts; d_list_cutoffs [batch_size][min(top_m, p1_lists)] and
 * d_thresholds [batch_size] as the reference writes them; d_atomic gets each
 * query's candidate count before the rerank_m cut (the reference's
 * query_atomic_counters, gpu_global.cu:349, 493-526, which
 * search_pipeline.cu:455-457 sums).  The candidate pool lives in d_flat_ids
 * (current_pool_cap ints); when that is too small for the batch the four pool
 * buffers are reallocated (the reference's growth rule: 1.5x what is needed)
 * after the stream is synchronised.  d_global_tables, d_compact_offsets and
 * final_k are not used (the LUTs live in on-chip memory).  events may be
 * NULL. */
inline void run_gpu_batch_logic(const IVFIndexGPU& idx, float* d_queries, uint32_t* d_cagra_top_m,
                                float* d_cagra_dists, float* d_global_tables, int*& d_flat_ids, float*& d_flat_dists,
                                int*& d_flat_ids_alt, float*& d_flat_dists_alt, size_t& current_pool_cap,
                                int* d_counts, int* d_offsets, int* d_atomic, int* d_top_ids, float* d_top_dists,
                                int* d_top_counts, int batch_size, int top_m, int rerank_m, int final_k,
                                float prune_ratio, float* d_list_cutoffs, float* d_thresholds, int* d_compact_offsets,
                                hipStream_t stream_main, BatchLogicEvents* events, int p1_lists = DEFAULT_P1_LISTS,
                                int limit_k = DEFAULT_LIMIT_K, float threshold_coeff = DEFAULT_THRESHOLD_COEFF) {
  namespace d = fgpu_compat_detail;
  (void)d_global_tables;
  (void)final_k;
  (void)d_compact_offsets;
  hipStream_t s = stream_main;
  fgpu_index* ix = d::view(idx, s);
  if (events) d::record(events->evt_start, s);
  d::check(fgpu_prune_probes(d_cagra_top_m, d_cagra_dists, batch_size, top_m, prune_ratio, s), "run_gpu_batch_logic");
  d::check(fgpu_probe_counts(ix, d_cagra_top_m, batch_size, top_m, d_counts, d_offsets, s), "run_gpu_batch_logic");
  if (events) {
    d::record(events->evt_prune_count, s);
    d::record(events->evt_scan_offset, s);
    d::record(events->evt_precompute, s);
  }
  const size_t need = fgpu_two_phase_workspace_bytes(batch_size, top_m, p1_lists, limit_k, rerank_m);
  if (current_pool_cap * sizeof(int) < need) {
    d::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    for (void* p : {(void*)d_flat_ids, (void*)d_flat_dists, (void*)d_flat_ids_alt, (void*)d_flat_dists_alt})
      if (p) d::hip_check(hipFree(p), "hipFree");
    current_pool_cap = (need / sizeof(int) + 1) * 3 / 2;
    d::hip_check(hipMalloc(&d_flat_ids, current_pool_cap * sizeof(int)), "hipMalloc");
    d::hip_check(hipMalloc(&d_flat_dists, current_pool_cap * sizeof(float)), "hipMalloc");
    d::hip_check(hipMalloc(&d_flat_ids_alt, current_pool_cap * sizeof(int)), "hipMalloc");
    d::hip_check(hipMalloc(&d_flat_dists_alt, current_pool_cap * sizeof(float)), "hipMalloc");
  }
  if (events) d::record(events->evt_resize_sync, s);
  if (d_atomic)
    d::check(fgpu_two_phase_search_precut(ix, d_queries, batch_size, d_cagra_top_m, top_m, p1_lists, limit_k,
                                          threshold_coeff, rerank_m, d_top_ids, d_top_dists, d_top_counts,
                                          d_list_cutoffs, d_thresholds, d_atomic, d_flat_ids,
                                          current_pool_cap * sizeof(int), s),
             "run_gpu_batch_logic");
  else
    d::check(fgpu_two_phase_search(ix, d_queries, batch_size, d_cagra_top_m, top_m, p1_lists, limit_k,
                                   threshold_coeff, rerank_m, d_top_ids, d_top_dists, d_top_counts, d_list_cutoffs,
                                   d_thresholds, d_flat_ids, current_pool_cap * sizeof(int), s),
             "run_gpu_batch_logic");
  if (events) {
    d::record(events->evt_scan_phase1_end, s);
    d::record(events->evt_scan_cand, s);
  }
  if (events) {
    d::record(events->evt_compact, s);
    d::record(events->evt_sort, s);
    d::record(events->evt_gather, s);
  }
}

/* run_gpu_rerank (gpu_global.cu:667-673): exact L2 over the first
 * d_top_counts[q] ids of d_top_ids [bs][rm] in mini-batches of mb, early stop
 * after b batches that change at most eps * k of the top k.  d_base_vecs
 * [tv][DIM].  d_stable_cnt and d_finished [batch_size] are left as the
 * reference leaves them (gpu_global.cu:603-609, 653-662): the stable count
 * after the last batch evaluated, and whether the walk stopped on stability
 * or ran past its candidates before rerank_m. */
inline void run_gpu_rerank(float* d_queries, int* d_top_ids, int* d_top_counts, float* d_base_vecs, int* d_final_ids,
                           float* d_final_dists, int* d_stable_cnt, bool* d_finished, int batch_size, int rerank_m,
                           int final_k, int total_vecs, int mini_batch_size, float epsilon, int beta,
                           hipStream_t stream) {
  static_assert(sizeof(bool) == 1, "d_finished is read as one byte a query");
  fgpu_compat_detail::check(fgpu_rerank_state(d_queries, batch_size, DIM, d_base_vecs, total_vecs, d_top_ids,
                                              d_top_counts, rerank_m, final_k, mini_batch_size, epsilon, beta,
                                              d_final_ids, d_final_dists, nullptr, d_stable_cnt,
                                              reinterpret_cast<uint8_t*>(d_finished), 0, stream),
                            "run_gpu_rerank");
}

/* ---- build (host pointers in and out, as kmeans_gpu.cuh / pq_utils.h) ---- */

/* run_kmeans_gpu (kmeans_gpu.cuh:234-324): the reference's strided mt19937(42)
 * initialisation, then max_iter Lloyd iterations (exact assignment, fixed-point
 * deterministic update, an empty cluster becomes zero).  h_centroids is
 * resized to k * dim. */
inline void run_kmeans_gpu(const float* h_data, int n, int dim, int k, std::vector<float>& h_centroids,
                           int max_iter = 20) {
  namespace d = fgpu_compat_detail;
  d::dev_buf<float> x((size_t)n * dim), c((size_t)k * dim);
  x.upload(h_data, (size_t)n * dim);
  d::check(fgpu_kmeans_fit(x.p, n, dim, k, max_iter, 0, 42, c.p, nullptr, nullptr), "run_kmeans_gpu");
  h_centroids.resize((size_t)k * dim);
  c.download(h_centroids.data(), h_centroids.size());
}

inline void fgpu_compat_assign(const float* h_data, const float* h_centroids, int n, int dim, int k,
                               std::vector<int>& out) {
  namespace d = fgpu_compat_detail;
  d::dev_buf<float> x((size_t)n * dim), c((size_t)k * dim), dist(n);
  d::dev_buf<int32_t> a(n);
  x.upload(h_data, (size_t)n * dim);
  c.upload(h_centroids, (size_t)k * dim);
  const size_t wb = fgpu_l2_topk_workspace_bytes(n, k);
  d::dev_buf<char> ws(wb);
  d::check(fgpu_l2_topk(x.p, n, c.p, k, dim, 1, a.p, dist.p, ws.p, wb, nullptr), "k-means assignment");
  out.resize(n);
  a.download(out.data(), n);
}

/* gpu_assign_initial_clusters (kmeans_gpu.cuh:329-362): nearest centroid of
 * every row (lowest index on ties), as buckets of row indices in row order. */
inline void gpu_assign_initial_clusters(const float* h_data, const float* h_centroids, int n, int dim, int k,
                                        std::vector<std::vector<int>>& buckets) {
  std::vector<int> a;
  fgpu_compat_assign(h_data, h_centroids, n, dim, k, a);
  buckets.clear();
  buckets.resize(k);
  for (int i = 0; i < n; ++i) buckets[a[i]].push_back(i);
}

/* gpu_assign_to_centroids (kmeans_gpu.cuh:367-394). */
inline void gpu_assign_to_centroids(const float* h_data, const float* h_centroids, int n, int dim, int k,
                                    std::vector<int>& assignments) {
  fgpu_compat_assign(h_data, h_centroids, n, dim, k, assignments);
}

/* cleanup_kmeans_gpu (kmeans_gpu.cuh:396-398): nothing is kept between calls. */
inline void cleanup_kmeans_gpu() {}

/* encode_residuals_to_pq_gpu (kmeans_gpu.cuh:450-508): the device form
 * (fused chain) of the residual encoding; pq_k must be 256. */
inline void encode_residuals_to_pq_gpu(const float* h_data, int n, int dim, const std::vector<int>& h_cluster_ids,
                                       const std::vector<float>& h_centroids, const std::vector<float>& h_codebook,
                                       uint8_t* h_codes, int pq_m, int pq_k, int sub_dim) {
  namespace d = fgpu_compat_detail;
  if (pq_k != 256 || pq_m * sub_dim != dim)
    throw fgpu_compat_error(FGPU_ERR_UNSUPPORTED, "encode_residuals_to_pq_gpu: need pq_k 256 and pq_m * sub_dim == dim");
  d::dev_buf<float> x((size_t)n * dim), c(h_centroids.size()), cb(h_codebook.size());
  d::dev_buf<int32_t> a(n);
  d::dev_buf<uint8_t> codes((size_t)n * pq_m);
  x.upload(h_data, (size_t)n * dim);
  c.upload(h_centroids.data(), h_centroids.size());
  cb.upload(h_codebook.data(), h_codebook.size());
  a.upload(h_cluster_ids.data(), n);
  d::check(fgpu_pq_encode_form(x.p, n, dim, pq_m, a.p, c.p, cb.p, 1, codes.p, nullptr), "encode_residuals_to_pq_gpu");
  codes.download(h_codes, (size_t)n * pq_m);
}

/* train_residual_pq_codebooks (pq_utils.h:77-138): the same sample
 * (mt19937(12345) shuffle of min(sample_size, n) rows), per-subspace
 * initialisation (mt19937(1234 + m)), E and M steps in the host's arithmetic,
 * run on the device.  codebook is resized to PQ_M * PQ_K * PQ_SUB_DIM. */
inline void train_residual_pq_codebooks(const point_t<float>* points, int n, const std::vector<int>& vec_cluster_ids,
                                        const std::vector<float>& clusters, std::vector<float>& codebook,
                                        int sample_size = 50000, int max_iter = 8) {
  namespace d = fgpu_compat_detail;
  d::dev_buf<float> x((size_t)n * DIM), c(clusters.size()), cb((size_t)PQ_M * PQ_K * PQ_SUB_DIM);
  d::dev_buf<int32_t> a(n);
  x.upload(reinterpret_cast<const float*>(points), (size_t)n * DIM);
  c.upload(clusters.data(), clusters.size());
  a.upload(vec_cluster_ids.data(), n);
  d::check(fgpu_pq_train(x.p, n, DIM, PQ_M, a.p, c.p, sample_size, max_iter, cb.p, nullptr),
           "train_residual_pq_codebooks");
  codebook.resize((size_t)PQ_M * PQ_K * PQ_SUB_DIM);
  cb.download(codebook.data(), codebook.size());
}

/* encode_residuals_to_pq (pq_utils.h:141-175): the host form of the encoding
 * (every product and sum rounded separately), run on the device. */
inline void encode_residuals_to_pq(const point_t<float>* points, int n, const std::vector<int>& vec_cluster_ids,
                                   const std::vector<float>& clusters, const std::vector<float>& codebook,
                                   uint8_t* codes) {
  namespace d = fgpu_compat_detail;
  d::dev_buf<float> x((size_t)n * DIM), c(clusters.size()), cb(codebook.size());
  d::dev_buf<int32_t> a(n);
  d::dev_buf<uint8_t> out((size_t)n * PQ_M);
  x.upload(reinterpret_cast<const float*>(points), (size_t)n * DIM);
  c.upload(clusters.data(), clusters.size());
  cb.upload(codebook.data(), codebook.size());
  a.upload(vec_cluster_ids.data(), n);
  d::check(fgpu_pq_encode_form(x.p, n, DIM, PQ_M, a.p, c.p, cb.p, 0, out.p, nullptr), "encode_residuals_to_pq");
  out.download(codes, (size_t)n * PQ_M);
}

/* train_pq_codebooks_gpu (kmeans_gpu.cuh:514-542): per subspace, run_kmeans_gpu
 * (15 iterations) on that subspace's coordinates of every row. */
template <int PQ_M_T, int PQ_K_T, int PQ_SUB_DIM_T>
inline void train_pq_codebooks_gpu(const float* flat_data, int n, int full_dim, std::vector<float>& codebook) {
  codebook.resize((size_t)PQ_M_T * PQ_K_T * PQ_SUB_DIM_T);
  std::vector<float> sub((size_t)n * PQ_SUB_DIM_T), cent;
  for (int m = 0; m < PQ_M_T; ++m) {
    for (int i = 0; i < n; ++i)
      for (int j = 0; j < PQ_SUB_DIM_T; ++j)
        sub[(size_t)i * PQ_SUB_DIM_T + j] = flat_data[(size_t)i * full_dim + m * PQ_SUB_DIM_T + j];
    run_kmeans_gpu(sub.data(), n, PQ_SUB_DIM_T, PQ_K_T, cent, 15);
    std::copy(cent.begin(), cent.end(), codebook.begin() + (size_t)m * PQ_K_T * PQ_SUB_DIM_T);
  }
}

#endif /* FUSIONGPU_COMPAT_HPP_ */
