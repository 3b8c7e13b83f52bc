// app_common.hpp -- shared helpers of the command-line tools (build_global,
// search_pipeline): argument parsing, status checks and fvecs/ivecs loading
// through the library's readers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "fusiongpu.h"

namespace app {

// The reference's tools print and exit(1) on any failure (kmeans_gpu.cuh:18-34,
// utils.h:27-79); the tools keep that behaviour at their own top level.
inline void ok(fgpu_status st, const char* what) {
  if (st != FGPU_OK) {
    std::fprintf(stderr, "%s failed: %s\n", what, fgpu_last_error());
    std::exit(1);
  }
}
inline void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

// fvecs with a known dimension (read_vecs, utils.h:22-48): exits on a missing
// file or a dimension mismatch, as the reference does.
inline std::vector<float> read_fvecs(const std::string& path, int dim, int64_t& n) {
  ok(fgpu_read_fvecs(path.c_str(), dim, &n, nullptr), ("reading " + path).c_str());
  std::vector<float> v((size_t)n * dim);
  ok(fgpu_read_fvecs(path.c_str(), dim, &n, v.data()), ("reading " + path).c_str());
  return v;
}

// The dimension stored in an fvecs file's first record.
inline int fvecs_dim(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    std::fprintf(stderr, "cannot open %s\n", path.c_str());
    std::exit(1);
  }
  int d = 0;
  const size_t got = std::fread(&d, 4, 1, f);
  std::fclose(f);
  if (got != 1 || d <= 0) {
    std::fprintf(stderr, "%s: bad fvecs header\n", path.c_str());
    std::exit(1);
  }
  return d;
}

template <class T>
struct Dev {
  T* p = nullptr;
  explicit Dev(size_t count) { hip_ok(hipMalloc(&p, (count ? count : 1) * sizeof(T)), "hipMalloc"); }
  ~Dev() { if (p) (void)hipFree(p); }
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
};

}  // namespace app
