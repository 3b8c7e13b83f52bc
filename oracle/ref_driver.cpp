// ref_driver.cpp -- exposes the reference's own CPU code (pq_utils.h, utils.h
// from /root/reference, compiled as-is) through a C ABI so the tests can pin
// the oracle against it.  TEST INFRASTRUCTURE ONLY; built into oracle/_ref/
// by oracle/Makefile when /root/reference is present.  defs.h fixes DIM=128
// and PQ_M=32 (defs.h:9-12), so these wrappers take no geometry arguments.
#include "pq_utils.h"
#include "utils.h"
#include <cstring>

extern "C" {

int ref_dim(void) { return DIM; }
int ref_pq_m(void) { return PQ_M; }

// pq_utils.h:17 run_kmeans_pq_fast
void ref_run_kmeans_pq_fast(const float* data, int n, int dim, int k, int seed, int max_iter,
                            float* out) {
  std::vector<float> c;
  run_kmeans_pq_fast(data, n, dim, k, c, seed, max_iter);
  std::memcpy(out, c.data(), sizeof(float) * c.size());
}

// pq_utils.h:77 train_residual_pq_codebooks
void ref_train_residual_pq_codebooks(const float* points, int n, const int* ids,
                                     const float* clusters, int nclusters, int sample_size,
                                     int max_iter, float* out_codebook) {
  std::vector<int> vid(ids, ids + n);
  std::vector<float> cl(clusters, clusters + (size_t)nclusters * DIM);
  std::vector<float> cb;
  train_residual_pq_codebooks(reinterpret_cast<const point_t<float>*>(points), n, vid, cl, cb,
                              sample_size, max_iter);
  std::memcpy(out_codebook, cb.data(), sizeof(float) * cb.size());
}

// pq_utils.h:141 encode_residuals_to_pq
void ref_encode_residuals_to_pq(const float* points, int n, const int* ids, const float* clusters,
                                int nclusters, const float* codebook, uint8_t* codes) {
  std::vector<int> vid(ids, ids + n);
  std::vector<float> cl(clusters, clusters + (size_t)nclusters * DIM);
  std::vector<float> cb(codebook, codebook + (size_t)PQ_M * PQ_K * PQ_SUB_DIM);
  encode_residuals_to_pq(reinterpret_cast<const point_t<float>*>(points), n, vid, cl, cb, codes);
}

// utils.h:22 read_vecs<float>; returns the row count, fills *out (caller frees with ref_free)
int ref_read_fvecs(const char* path, int d, float** out) {
  float* v = nullptr;
  int n = read_vecs<float>(path, v, d);
  *out = v;
  return n;
}

// utils.h:75 read_ivecs
int ref_read_ivecs(const char* path, int* d, int** out) {
  int* v = nullptr;
  int n = read_ivecs(path, v, *d);
  *out = v;
  return n;
}

void ref_free_f(float* p) { delete[] p; }
void ref_free_i(int* p) { delete[] p; }
}
