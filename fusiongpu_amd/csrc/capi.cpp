// capi.cpp -- the extern "C" boundary (include/fusiongpu.h): index handle,
// search and build orchestration, file formats and the synthetic generator.
#include <algorithm>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <numeric>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

// Events fgpu_search records with FGPU_OPT_STAGE_EVENTS: before the coarse
// step, after it, after each of the screen's five stages, after the scan.
constexpr int kStageEvents = 8;

struct fgpu_index {
  int dim = 0, m = 0, nlist = 0, max_list_len = 0;
  int64_t total = 0;
  float* d_codebook = nullptr;
  int32_t* d_offsets = nullptr;
  uint8_t* d_codes = nullptr;
  int32_t* d_ids = nullptr;
  float* d_centroids = nullptr;
  float* d_cnorm = nullptr;      // [nlist] ||c||^2
  float* d_cnorm_max = nullptr;  // [1]
  float* d_rmax = nullptr;       // [nlist] decoded-residual radius per list
  unsigned long long* d_faults = nullptr;  // [1] bounded-wait give-ups of the flow scan
  bool borrowed = false;  // the A1 arrays belong to the caller (fgpu_index_wrap)
  // The MFMA screen of the plain search (screen.hip): bf16 codebook and the
  // per-vector extra blocks, built at creation when the geometry allows it.
  uint16_t* d_cb16 = nullptr;
  int screen_scale_exp = 0;  // S: the screen works on the data times 2^S
  uint4* d_vext = nullptr;
  bool screen_ok = false;
  // Per-index options (fgpu_index_set_option).
  int opt_list_skip = 1;
  int opt_spin_limit = 0;
  int opt_screen = 1;
  int opt_screen_clocks = 0;
  int opt_two_phase_split = 0;
  int opt_two_phase_screen = 0;  // FGPU_OPT_TWO_PHASE_SCREEN
  // FGPU_OPT_STAGE_EVENTS: events fgpu_search records between its stages.
  int opt_stage_events = 0;
  hipEvent_t stage_ev[kStageEvents] = {};
};

namespace fgpu {

thread_local std::string g_err;
fgpu_status set_error(fgpu_status st, const std::string& msg) {
  g_err = msg;
  return st;
}

namespace {

// RAII device buffer for the build path (search entry points never allocate).
template <class T>
struct DevBuf {
  T* p = nullptr;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { if (p) (void)hipFree(p); }
  fgpu_status alloc(size_t count) {
    if (count == 0) count = 1;
    if (hipMalloc(&p, count * sizeof(T)) != hipSuccess) {
      p = nullptr;
      (void)hipGetLastError();
      return set_error(FGPU_ERR_NOMEM, "hipMalloc failed (" + std::to_string(count * sizeof(T)) + " bytes)");
    }
    return FGPU_OK;
  }
};

void free_index(fgpu_index* ix) {
  if (!ix) return;
  if (!ix->borrowed)
    for (void* p : {(void*)ix->d_codebook, (void*)ix->d_offsets, (void*)ix->d_codes, (void*)ix->d_ids,
                    (void*)ix->d_centroids})
      if (p) (void)hipFree(p);
  for (void* p : {(void*)ix->d_cnorm, (void*)ix->d_cnorm_max, (void*)ix->d_rmax, (void*)ix->d_faults,
                  (void*)ix->d_cb16, (void*)ix->d_vext})
    if (p) (void)hipFree(p);
  for (hipEvent_t e : ix->stage_ev)
    if (e) (void)hipEventDestroy(e);
  delete ix;
}

// The derived arrays of an index whose A1 arrays are on the device: centroid
// norms, their maximum, the per-list decoded-residual radius and the give-up
// counter.
fgpu_status finish_index(fgpu_index* ix, hipStream_t s) {
  auto alloc = [&](void** p, size_t b) { return hipMalloc(p, b == 0 ? 256 : b) == hipSuccess; };
  if (!alloc((void**)&ix->d_cnorm, sizeof(float) * ix->nlist) || !alloc((void**)&ix->d_cnorm_max, 256) ||
      !alloc((void**)&ix->d_rmax, sizeof(float) * ix->nlist) || !alloc((void**)&ix->d_faults, 256)) {
    (void)hipGetLastError();
    return set_error(FGPU_ERR_NOMEM, "index: device allocation failed");
  }
  FGPU_HIP(hipMemsetAsync(ix->d_faults, 0, 256, s));
  // Per-device lookups that searches would otherwise make on their first
  // call (which may be under graph capture): the no-allocation scratch
  // address and the flow kernel's resident grid, both cached per device.
  FGPU_TRY(noalloc_prepare());
  (void)flow_grid(ix->dim, ix->m, 1, 1);
  FGPU_TRY(launch_row_norms(ix->d_centroids, ix->nlist, ix->dim, ix->d_cnorm, s));
  FGPU_TRY(launch_max_reduce(ix->d_cnorm, ix->nlist, ix->d_cnorm_max, s));
  FGPU_TRY(launch_list_radius(ix->d_codebook, ix->m, ix->dim / ix->m, ix->d_codes, ix->d_offsets, ix->nlist, ix->d_rmax,
                              s));
  // The screen's arrays: only for its geometries, 16-byte aligned arrays,
  // lists below 2^24 vectors, and decoded norms below 2^40.  The screen works
  // on the data times 2^S, S the largest with every decoded norm at most 64
  // after scaling; the bound sqrt(sum_j max_c ||codeword||^2) comes from the
  // codebook alone.
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  unsigned int* xmax = nullptr;
  double xcb = -1.0;
  if (screen_supported(ix->dim, ix->m) && ix->max_list_len < (1 << 24) && al16(ix->d_codebook) &&
      al16(ix->d_centroids) && al16(ix->d_codes)) {
    const int sub = ix->dim / ix->m;
    std::vector<float> hcb((size_t)ix->dim * kPQK);
    FGPU_HIP(hipStreamSynchronize(s));
    FGPU_HIP(hipMemcpy(hcb.data(), ix->d_codebook, hcb.size() * sizeof(float), hipMemcpyDeviceToHost));
    double sum = 0.0;
    for (int j = 0; j < ix->m; ++j) {
      double mx = 0.0;
      for (int c = 0; c < kPQK; ++c) {
        double n2 = 0.0;
        for (int d = 0; d < sub; ++d) {
          const double v = hcb[((size_t)j * kPQK + c) * sub + d];
          n2 += v * v;
        }
        mx = std::max(mx, n2);
      }
      sum += mx;
    }
    xcb = std::sqrt(sum);
  }
  if (xcb >= 0.0 && xcb <= 0x1p40) {
    int se = 0;
    if (xcb > 0.0) {
      se = (int)std::floor(std::log2(64.0 / xcb));
      while (std::ldexp(xcb, se) > 64.0) --se;
      se = std::max(-60, std::min(60, se));
    }
    ix->screen_scale_exp = se;
    if (alloc((void**)&ix->d_cb16, (size_t)ix->dim * kPQK * sizeof(uint16_t)) &&
        alloc((void**)&ix->d_vext, sizeof(uint4) * (size_t)std::max<int64_t>(ix->total, 1)) &&
        alloc((void**)&xmax, 256)) {
      FGPU_TRY(launch_screen_prep(ix->d_codebook, ix->m, ix->dim / ix->m, se, ix->d_codes, ix->total, ix->d_cb16,
                                  ix->d_vext, xmax, s));
    } else {
      (void)hipGetLastError();  // no room for the screen: the plain search keeps the LUT kernels
    }
  }
  FGPU_HIP(hipStreamSynchronize(s));
  if (xmax) {
    unsigned int bits = 0;
    const bool got = hipMemcpy(&bits, xmax, sizeof(bits), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(xmax);
    float xm = 0.0f;
    std::memcpy(&xm, &bits, sizeof(xm));
    ix->screen_ok = got && xm <= 65.0f;  // every scaled norm bound X' (at most 64 plus its fp16 rounding)
  }
  if (!ix->screen_ok) {
    for (void* p : {(void*)ix->d_cb16, (void*)ix->d_vext})
      if (p) (void)hipFree(p);
    ix->d_cb16 = nullptr;
    ix->d_vext = nullptr;
  }
  return FGPU_OK;
}

AdcArgs adc_args(const fgpu_index* ix, const float* dq, int nq, const uint32_t* probes, const float* probe_dists,
                 int nprobe, int k, int32_t* out_ids, float* out_d) {
  AdcArgs a{dq, ix->d_centroids, ix->d_codebook, ix->d_offsets, ix->d_codes, ix->d_ids, probes, ix->d_rmax,
            nq, nprobe, k, ix->nlist, out_ids, out_d};
  a.probe_dists = probe_dists;
  a.total = ix->total;
  a.faults = ix->d_faults;
  a.max_list_len = ix->max_list_len;
  a.spin_limit = ix->opt_spin_limit;
  a.list_skip = ix->opt_list_skip;
  return a;
}

// The screen's workspace, carved from `base` (fgpu_search, after the probe
// arrays).  The counters, per-list counts and per-query candidate counts are
// one contiguous block that the first screen kernel zeroes.
constexpr int kScreenCandCap = 512;  // candidates kept per query before it takes the LUT kernel
struct ScreenWs {
  int* zero = nullptr;  // [zero_words(nq, nlist)]
  int* bucket = nullptr;
  uint4* arec = nullptr;
  float* thr = nullptr;
  uint2* cand = nullptr;
  int* flist = nullptr;
  int2* first = nullptr;
  uint32_t* gminbuf = nullptr;
  static size_t zero_words(int nq, int nlist) { return (size_t)kCtrCount + 2 * (size_t)nlist + (size_t)nq; }
  static size_t gmin_words(int nq) { return (size_t)screen_gmin_words(nq); }
  static size_t rec_count(int nq, int nprobe) { return (size_t)nq * nprobe * 18; }
  // Bucket entries: [nlist][nq], or with compact buckets (one probe a query,
  // ScreenArgs::boff) one a query.
  static size_t bucket_words(int nq, int nlist, bool compact) { return compact ? (size_t)nq : (size_t)nlist * nq; }
  bool carve(void* base, size_t bytes, int nq, int nlist, int nprobe, bool compact = false) {
    Carve cv(base, bytes);
    zero = cv.take<int>(zero_words(nq, nlist));
    bucket = cv.take<int>(bucket_words(nq, nlist, compact));
    arec = cv.take<uint4>(rec_count(nq, nprobe));
    thr = cv.take<float>((size_t)nq);
    cand = cv.take<uint2>((size_t)nq * kScreenCandCap);
    flist = cv.take<int>((size_t)nq);
    first = cv.take<int2>((size_t)nq);
    gminbuf = cv.take<uint32_t>(gmin_words(nq));
    return cv.ok();
  }
  static size_t bytes(int nq, int nlist, int nprobe, bool compact = false) {
    return carve_bytes<int>(zero_words(nq, nlist)) + carve_bytes<int>(bucket_words(nq, nlist, compact)) +
           carve_bytes<uint4>(rec_count(nq, nprobe)) +
           carve_bytes<float>((size_t)nq) + carve_bytes<uint2>((size_t)nq * kScreenCandCap) +
           carve_bytes<int>((size_t)nq) + carve_bytes<int2>((size_t)nq) +
           carve_bytes<uint32_t>(gmin_words(nq));
  }
};

// Phase 1 of fgpu_two_phase_search through the screen: the buffers of one
// chunk of nvq virtual queries (one per (query, phase-1 probe); virtual query
// v reads query row v / p1 of the chunk): their probes and (zero) probe distances, their top-limit_k results, the
// per-list counts and compact bucket offsets, and the screen's workspace.
// Batches below this many queries keep phase 1 in the two-phase kernel (the
// screen's fixed launches cost more than they save there).
constexpr int kTpScreenMinQueries = 1024;
constexpr int kTpVqMax = 131072;  // virtual queries a chunk (fuller 32-row MFMA groups per list)
struct TpScreenWs {
  uint32_t* vprobe = nullptr;
  float* vpd = nullptr;
  int32_t* vids = nullptr;
  float* vd = nullptr;
  int* hist = nullptr;  // [2 nlist + 1]: list counts, nlist unused, the count of those without a list
  int32_t* rank = nullptr;  // [nvq] each virtual query's rank in its list
  int32_t* boff = nullptr;
  int32_t* order = nullptr;   // the virtual queries by list: the rescore's order and the screen's buckets
  int32_t* sp_cnt = nullptr;  // [nlist] the screen's single-probe counts
  float2* pnorm = nullptr;    // [nvq]
  ScreenWs sw;
  bool carve(void* base, size_t bytes, int nvq, int nlist, int dim, int k) {
    Carve cv(base, bytes);
    (void)dim;
    vprobe = cv.take<uint32_t>((size_t)nvq);
    vpd = cv.take<float>((size_t)nvq);
    vids = cv.take<int32_t>((size_t)nvq * k);
    vd = cv.take<float>((size_t)nvq * k);
    hist = cv.take<int>(2 * (size_t)nlist + 1);
    rank = cv.take<int32_t>((size_t)nvq);
    boff = cv.take<int32_t>((size_t)nlist + 1);
    order = cv.take<int32_t>((size_t)nvq);
    sp_cnt = cv.take<int32_t>((size_t)nlist);
    pnorm = cv.take<float2>((size_t)nvq);
    return cv.ok() && sw.carve(cv.base + cv.used, bytes - cv.used, nvq, nlist, 1, true);
  }
  static size_t bytes(int nvq, int nlist, int dim, int k) {
    (void)dim;
    return carve_bytes<uint32_t>((size_t)nvq) +
           carve_bytes<float>((size_t)nvq) + carve_bytes<int32_t>((size_t)nvq * k) +
           carve_bytes<float>((size_t)nvq * k) + carve_bytes<int>(2 * (size_t)nlist + 1) + carve_bytes<int32_t>((size_t)nvq) +
           carve_bytes<int32_t>((size_t)nlist + 1) + carve_bytes<int32_t>((size_t)nvq) +
           carve_bytes<int32_t>((size_t)nlist) + carve_bytes<float2>((size_t)nvq) + ScreenWs::bytes(nvq, nlist, 1, true);
  }
};

// The first k entries of what std::shuffle(iota(n), rng) leaves, drawing
// exactly as std::shuffle does.  When rng's range is below n^2, libstdc++'s
// std::shuffle swaps position i with position d(rng, [0, i]) for i = 1, 2, ...,
// n - 1, one draw of a stateless uniform_int_distribution<size_t-like> each
// (bits/stl_algo.h).  Position i still holds i when its turn comes, so the
// prefix needs only the draws: a prefix slot j < k drawn at step i >= k takes
// the value i.  Otherwise (small n: the paired-draw path) std::shuffle itself.
// The oracle's full shuffle is the check (tests/test_capi.py).
std::vector<int32_t> shuffled_prefix(int64_t n, int64_t k, std::mt19937& rng) {
  using UD = std::make_unsigned<std::vector<int32_t>::difference_type>::type;
  using UC = std::common_type<std::mt19937::result_type, UD>::type;
  k = std::min(k, n);
  const UC urng_range = rng.max() - rng.min();
  if (n <= 1 || urng_range / (UC)n >= (UC)n) {
    std::vector<int32_t> idx(n);
    std::iota(idx.begin(), idx.end(), 0);
    std::shuffle(idx.begin(), idx.end(), rng);
    idx.resize(k);
    return idx;
  }
  std::vector<int32_t> a(k);
  std::iota(a.begin(), a.end(), 0);
  std::uniform_int_distribution<UD> d;
  using P = std::uniform_int_distribution<UD>::param_type;
  for (int64_t i = 1; i < n; ++i) {
    const UD j = d(rng, P(0, (UD)i));
    if (i < k)
      std::swap(a[i], a[j]);
    else if ((int64_t)j < k)
      a[j] = (int32_t)i;
  }
  return a;
}

int64_t topk_batch_rows(int64_t n, int nc) {
  const size_t budget = 256ull << 20;  // estimate tile budget per batch
  int64_t b = est_rows_per_batch(budget, nc);
  if (b < 64) b = 64;
  return std::min<int64_t>(b, ((n + 63) / 64) * 64);
}

// splitmix64 finaliser (same definition as the oracle's generator).
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
}  // namespace fgpu

using namespace fgpu;

extern "C" {

const char* fgpu_last_error(void) { return g_err.c_str(); }
int fgpu_abi_version(void) { return 1; }

// ---------------------------------------------------------------------------
fgpu_status fgpu_index_create(int dim, int pq_m, int nlist, int64_t total, const int32_t* h_offsets,
                              const int32_t* h_ids, const uint8_t* h_codes, const float* h_centroids,
                              const float* h_codebook, fgpu_index** out) {
  FGPU_CHECK(out && h_offsets && h_centroids && h_codebook, FGPU_ERR_ARG, "index_create: null argument");
  FGPU_CHECK(total == 0 || (h_ids && h_codes), FGPU_ERR_ARG, "index_create: null ids/codes");
  FGPU_CHECK(dim > 0 && pq_m > 0 && dim % pq_m == 0 && nlist > 0 && total >= 0 && total < INT32_MAX,
             FGPU_ERR_ARG, "index_create: bad geometry");
  FGPU_CHECK(h_offsets[0] == 0 && h_offsets[nlist] == total, FGPU_ERR_ARG,
             "index_create: offsets must start at 0 and end at total");
  int maxlen = 0;
  for (int l = 0; l < nlist; ++l) {
    const int len = h_offsets[l + 1] - h_offsets[l];
    FGPU_CHECK(len >= 0, FGPU_ERR_ARG, "index_create: offsets not monotone");
    maxlen = std::max(maxlen, len);
  }
  fgpu_index* ix = new fgpu_index();
  ix->dim = dim; ix->m = pq_m; ix->nlist = nlist; ix->total = total; ix->max_list_len = maxlen;
  auto fail = [&](fgpu_status st) { free_index(ix); return st; };
  auto alloc = [&](void** p, size_t b) { return hipMalloc(p, b == 0 ? 256 : b) == hipSuccess; };
  const size_t cb_bytes = (size_t)pq_m * kPQK * (dim / pq_m) * sizeof(float);
  if (!alloc((void**)&ix->d_codebook, cb_bytes) || !alloc((void**)&ix->d_offsets, sizeof(int32_t) * (nlist + 1)) ||
      !alloc((void**)&ix->d_codes, (size_t)total * pq_m + 256) || !alloc((void**)&ix->d_ids, sizeof(int32_t) * total) ||
      !alloc((void**)&ix->d_centroids, sizeof(float) * (size_t)nlist * dim)) {
    (void)hipGetLastError();
    return fail(set_error(FGPU_ERR_NOMEM, "index_create: device allocation failed"));
  }
  if (hipMemcpy(ix->d_codebook, h_codebook, cb_bytes, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(ix->d_offsets, h_offsets, sizeof(int32_t) * (nlist + 1), hipMemcpyHostToDevice) != hipSuccess ||
      (total && hipMemcpy(ix->d_codes, h_codes, (size_t)total * pq_m, hipMemcpyHostToDevice) != hipSuccess) ||
      (total && hipMemcpy(ix->d_ids, h_ids, sizeof(int32_t) * total, hipMemcpyHostToDevice) != hipSuccess) ||
      hipMemcpy(ix->d_centroids, h_centroids, sizeof(float) * (size_t)nlist * dim, hipMemcpyHostToDevice) != hipSuccess)
    return fail(set_error(FGPU_ERR_HIP, "index_create: copy to device failed"));
  const fgpu_status st = finish_index(ix, nullptr);
  if (st != FGPU_OK) return fail(st);
  *out = ix;
  return FGPU_OK;
}

fgpu_status fgpu_index_wrap(int dim, int pq_m, int nlist, const int32_t* d_offsets, const int32_t* d_ids,
                            const uint8_t* d_codes, const float* d_centroids, const float* d_codebook, void* stream,
                            fgpu_index** out) {
  FGPU_CHECK(out && d_offsets && d_centroids && d_codebook, FGPU_ERR_ARG, "index_wrap: null argument");
  FGPU_CHECK(dim > 0 && pq_m > 0 && dim % pq_m == 0 && pq_m % 16 == 0 && nlist > 0, FGPU_ERR_ARG,
             "index_wrap: bad geometry (pq_m must be a multiple of 16)");
  FGPU_CHECK(((uintptr_t)d_codes & 15) == 0, FGPU_ERR_ARG, "index_wrap: codes must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  std::vector<int32_t> offs(nlist + 1);
  FGPU_HIP(hipMemcpyAsync(offs.data(), d_offsets, sizeof(int32_t) * (nlist + 1), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipStreamSynchronize(s));
  FGPU_CHECK(offs[0] == 0 && offs[nlist] >= 0 && offs[nlist] < INT32_MAX, FGPU_ERR_ARG,
             "index_wrap: offsets must start at 0 and end below 2^31");
  FGPU_CHECK(offs[nlist] == 0 || (d_ids && d_codes), FGPU_ERR_ARG, "index_wrap: null ids/codes");
  int maxlen = 0;
  for (int l = 0; l < nlist; ++l) {
    const int len = offs[l + 1] - offs[l];
    FGPU_CHECK(len >= 0, FGPU_ERR_ARG, "index_wrap: offsets not monotone");
    maxlen = std::max(maxlen, len);
  }
  fgpu_index* ix = new fgpu_index();
  ix->dim = dim; ix->m = pq_m; ix->nlist = nlist; ix->total = offs[nlist]; ix->max_list_len = maxlen;
  ix->borrowed = true;
  ix->d_codebook = const_cast<float*>(d_codebook);
  ix->d_offsets = const_cast<int32_t*>(d_offsets);
  ix->d_codes = const_cast<uint8_t*>(d_codes);
  ix->d_ids = const_cast<int32_t*>(d_ids);
  ix->d_centroids = const_cast<float*>(d_centroids);
  const fgpu_status st = finish_index(ix, s);
  if (st != FGPU_OK) {
    free_index(ix);
    return st;
  }
  *out = ix;
  return FGPU_OK;
}

void fgpu_index_destroy(fgpu_index* idx) { free_index(idx); }

fgpu_status fgpu_index_get_info(const fgpu_index* ix, fgpu_index_info* o) {
  FGPU_CHECK(ix && o, FGPU_ERR_ARG, "index_get_info: null argument");
  o->dim = ix->dim; o->pq_m = ix->m; o->pq_k = kPQK; o->nlist = ix->nlist; o->total = ix->total;
  o->d_pq_codebook = ix->d_codebook; o->d_cluster_offsets = ix->d_offsets; o->d_all_pq_codes = ix->d_codes;
  o->d_all_vector_ids = ix->d_ids; o->d_centroids = ix->d_centroids; o->max_list_len = ix->max_list_len;
  return FGPU_OK;
}

fgpu_status fgpu_index_load(const char* ivf_path, const char* cb_path, int dim, int pq_m, fgpu_index** out) {
  int64_t total = 0;
  int nlist = 0;
  FGPU_TRY(fgpu_read_ivf_header(ivf_path, &total, &nlist));
  FGPU_CHECK(dim > 0 && pq_m > 0 && dim % pq_m == 0, FGPU_ERR_ARG, "index_load: bad geometry");
  std::vector<int32_t> offs(nlist + 1), ids(total);
  std::vector<uint8_t> codes((size_t)total * pq_m);
  std::vector<float> cent((size_t)nlist * dim);
  FGPU_TRY(fgpu_read_ivf_data(ivf_path, pq_m, dim, offs.data(), ids.data(), codes.data(), cent.data()));
  std::ifstream f(cb_path, std::ios::binary | std::ios::ate);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, std::string("cannot open codebook: ") + cb_path);
  const size_t want = (size_t)pq_m * kPQK * (dim / pq_m) * sizeof(float);
  FGPU_CHECK((size_t)f.tellg() == want, FGPU_ERR_IO, "codebook file size does not match dim/pq_m");
  std::vector<float> cb(want / sizeof(float));
  f.seekg(0);
  f.read(reinterpret_cast<char*>(cb.data()), want);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, "short read of codebook");
  return fgpu_index_create(dim, pq_m, nlist, total, offs.data(), ids.data(), codes.data(), cent.data(), cb.data(), out);
}

// ---------------------------------------------------------------------------
size_t fgpu_coarse_workspace_bytes(int nq, int nlist) {
  // The estimate block holds whole 64-row GEMM tiles: with room for every
  // query row rounded up to 64, the coarse step is one GEMM + one select.
  const size_t rows = ((size_t)std::max(nq, 64) + 63) / 64 * 64;
  return carve_bytes<float>(rows * (size_t)est_sel_ld(nlist)) + 256;
}

}  // extern "C"

namespace {
// fgpu_coarse_search; with side != nullptr its first select launch also
// stores side_val at *side (the scan's query counter, so the scan needs no
// reset kernel of its own).
fgpu_status coarse_search(const fgpu_index* ix, const float* dq, int nq, int nprobe, float prune_ratio,
                          uint32_t* d_ids, float* d_dists, void* ws, size_t ws_bytes, void* stream, int* side,
                          int side_val, unsigned long long* stats = nullptr) {
  // An empty batch may come with empty (null) arrays.
  FGPU_CHECK(ix && ws && (nq == 0 || (dq && d_ids && d_dists)), FGPU_ERR_ARG, "coarse_search: null argument");
  FGPU_CHECK(((uintptr_t)ws & 15) == 0, FGPU_ERR_ARG, "coarse_search: workspace must be 16-byte aligned");
  FGPU_CHECK(nq >= 0 && nprobe >= 1 && nprobe <= ix->nlist && nprobe <= 256, FGPU_ERR_ARG,
             "coarse_search: need 1 <= nprobe <= min(nlist, 256)");
  if (nq == 0) return FGPU_OK;
  hipStream_t s = as_stream(stream);
  Carve cv(ws, ws_bytes);
  const int64_t ld = est_sel_ld(ix->nlist);
  int64_t rows = std::min<int64_t>(est_rows_per_batch(ws_bytes > 256 ? ws_bytes - 256 : 0, (int)ld), ((nq + 63) / 64) * 64);
  FGPU_CHECK(rows >= 64, FGPU_ERR_WORKSPACE, "coarse_search: workspace too small");
  void* est = cv.take<float>((size_t)rows * ld);
  FGPU_CHECK(est, FGPU_ERR_WORKSPACE, "coarse_search: workspace too small");
  // The estimates leave out each query's norm; the select computes it for
  // its margin.
  for (int64_t b0 = 0; b0 < nq; b0 += rows) {
    const int64_t nb = std::min<int64_t>(rows, nq - b0);
    FGPU_TRY(launch_gemm_est_sel(dq + b0 * ix->dim, nb, ix->d_centroids, ix->nlist, ix->dim, ix->d_cnorm,
                                 ix->d_cnorm_max, est, ld, s));
    FGPU_TRY(launch_select_exact(est, ld, nb, ix->nlist, dq + b0 * ix->dim, ix->d_centroids, ix->dim,
                                 ix->d_cnorm_max, nprobe, 1, prune_ratio,
                                 reinterpret_cast<int32_t*>(d_ids) + b0 * nprobe, d_dists + b0 * nprobe, s,
                                 b0 == 0 ? side : nullptr, side_val, stats));
  }
  return FGPU_OK;
}
}  // namespace

extern "C" {

fgpu_status fgpu_coarse_search(const fgpu_index* ix, const float* dq, int nq, int nprobe, float prune_ratio,
                               uint32_t* d_ids, float* d_dists, void* ws, size_t ws_bytes, void* stream) {
  return coarse_search(ix, dq, nq, nprobe, prune_ratio, d_ids, d_dists, ws, ws_bytes, stream, nullptr, 0);
}

fgpu_status fgpu_coarse_search_stats(const fgpu_index* ix, const float* dq, int nq, int nprobe, float prune_ratio,
                                     uint32_t* d_ids, float* d_dists, unsigned long long* d_stats, void* ws,
                                     size_t ws_bytes, void* stream) {
  FGPU_CHECK(d_stats, FGPU_ERR_ARG, "coarse_search_stats: null stats");
  return coarse_search(ix, dq, nq, nprobe, prune_ratio, d_ids, d_dists, ws, ws_bytes, stream, nullptr, 0, d_stats);
}

fgpu_status fgpu_prune_probes(uint32_t* d_probe_ids, const float* d_probe_dists, int nq, int nprobe, float prune_ratio,
                              void* stream) {
  FGPU_CHECK(d_probe_ids && d_probe_dists && nq >= 0 && nprobe >= 1, FGPU_ERR_ARG, "prune_probes: bad argument");
  if (nq == 0) return FGPU_OK;
  return launch_coarse_prune(reinterpret_cast<int32_t*>(d_probe_ids), d_probe_dists, nq, nprobe, prune_ratio,
                             as_stream(stream));
}

fgpu_status fgpu_probe_counts(const fgpu_index* ix, const uint32_t* d_probe_ids, int nq, int nprobe, int32_t* d_counts,
                              int32_t* d_offsets, void* stream) {
  FGPU_CHECK(ix && d_probe_ids && d_counts && d_offsets && nq >= 0 && nprobe >= 1, FGPU_ERR_ARG,
             "probe_counts: bad argument");
  return launch_probe_counts(d_probe_ids, nq, nprobe, ix->nlist, ix->d_offsets, d_counts, d_offsets, as_stream(stream));
}

fgpu_status fgpu_adc_search(const fgpu_index* ix, const float* dq, int nq, const uint32_t* d_probe_ids,
                            const float* d_probe_dists, int nprobe, int k, int32_t* d_out_ids, float* d_out_dists,
                            void* stream) {
  FGPU_CHECK(ix && (nq == 0 || (dq && d_probe_ids && d_out_ids && d_out_dists)), FGPU_ERR_ARG,
             "adc_search: null argument");
  FGPU_CHECK(nq >= 0 && nprobe >= 1 && k >= 1, FGPU_ERR_ARG, "adc_search: bad sizes");
  FGPU_CHECK(adc_supported(ix->dim, ix->m), FGPU_ERR_UNSUPPORTED, "adc_search: no kernel for this (dim, pq_m)");
  AdcArgs a = adc_args(ix, dq, nq, d_probe_ids, d_probe_dists, nprobe, k, d_out_ids, d_out_dists);
  return launch_adc_plain(ix->dim, ix->m, a, as_stream(stream));
}

fgpu_status fgpu_adc_search_stats(const fgpu_index* ix, const float* dq, int nq, const uint32_t* d_probe_ids,
                                  const float* d_probe_dists, int nprobe, int k, int32_t* d_out_ids,
                                  float* d_out_dists, unsigned long long* d_stats, void* stream) {
  FGPU_CHECK(ix && d_stats && (nq == 0 || (dq && d_probe_ids && d_out_ids && d_out_dists)), FGPU_ERR_ARG,
             "adc_search_stats: null argument");
  FGPU_CHECK(nq >= 0 && nprobe >= 1 && k >= 1, FGPU_ERR_ARG, "adc_search_stats: bad sizes");
  FGPU_CHECK(adc_supported(ix->dim, ix->m), FGPU_ERR_UNSUPPORTED, "adc_search_stats: no kernel for this (dim, pq_m)");
  AdcArgs a = adc_args(ix, dq, nq, d_probe_ids, d_probe_dists, nprobe, k, d_out_ids, d_out_dists);
  a.stats = d_stats;
  return launch_adc_plain(ix->dim, ix->m, a, as_stream(stream));
}

fgpu_status fgpu_index_faults(const fgpu_index* ix, void* stream, unsigned long long* count, int reset) {
  FGPU_CHECK(ix && count, FGPU_ERR_ARG, "index_faults: null argument");
  hipStream_t s = as_stream(stream);
  unsigned long long v = 0;
  FGPU_HIP(hipMemcpyAsync(&v, ix->d_faults, sizeof(v), hipMemcpyDeviceToHost, s));
  if (reset) FGPU_HIP(hipMemsetAsync(ix->d_faults, 0, sizeof(v), s));
  FGPU_HIP(hipStreamSynchronize(s));
  *count = v;
  return FGPU_OK;
}

fgpu_status fgpu_index_check(const fgpu_index* ix, void* stream) {
  unsigned long long v = 0;
  FGPU_TRY(fgpu_index_faults(ix, stream, &v, 0));
  FGPU_CHECK(v == 0, FGPU_ERR_WAIT,
             std::to_string(v) + " bounded wait(s) of the scan kernel gave up; the affected queries carry id -2");
  return FGPU_OK;
}


int fgpu_debug_pq_sample(int64_t n, int sample_size, int32_t* h_rows) {
  if (n < 1 || sample_size < 0 || !h_rows) return -1;
  std::mt19937 rng(12345);
  const std::vector<int32_t> r = shuffled_prefix(n, sample_size, rng);
  std::memcpy(h_rows, r.data(), sizeof(int32_t) * r.size());
  return (int)r.size();
}

int fgpu_stream_read_grid(void) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus * 8;
}

fgpu_status fgpu_stream_read(const void* d, size_t bytes, unsigned long long* d_sink, void* stream) {
  FGPU_CHECK(d && d_sink && bytes % 16 == 0 && ((uintptr_t)d & 15) == 0, FGPU_ERR_ARG,
             "stream_read: need 16-byte aligned data, a size multiple of 16 and a sink");
  return launch_stream_read(d, bytes, d_sink, fgpu_stream_read_grid(), as_stream(stream));
}

fgpu_status fgpu_row_gather_lanes(const void* d_rows, int64_t nrows, int row_bytes, const int32_t* d_idx, int64_t n,
                                  int lanes_per_row, unsigned long long* d_sink, void* stream) {
  FGPU_CHECK(d_rows && d_idx && d_sink && n >= 0 && nrows >= 1 && ((uintptr_t)d_rows & 15) == 0, FGPU_ERR_ARG,
             "row_gather: need 16-byte aligned rows, indices and a sink");
  return launch_row_gather(d_rows, nrows, row_bytes, d_idx, n, lanes_per_row, d_sink, fgpu_stream_read_grid(),
                           as_stream(stream));
}

fgpu_status fgpu_row_gather(const void* d_rows, int64_t nrows, int row_bytes, const int32_t* d_idx, int64_t n,
                            unsigned long long* d_sink, void* stream) {
  return fgpu_row_gather_lanes(d_rows, nrows, row_bytes, d_idx, n, 8, d_sink, stream);
}

}  // extern "C"

namespace fgpu {
size_t search_lut_workspace_bytes(int nq, int nlist, int nprobe) {
  return carve_bytes<uint32_t>((size_t)nq * nprobe) + carve_bytes<float>((size_t)nq * nprobe) +
         carve_bytes<int>(1) + fgpu_coarse_workspace_bytes(nq, nlist);
}
}  // namespace fgpu

extern "C" {

size_t fgpu_search_workspace_bytes(int nq, int nlist, int nprobe) {
  // The coarse step's estimate tile and the screen's buffers are never live
  // at once, so they share one region (no screen beyond kScreenMaxLists lists).
  const size_t screen = nlist <= kScreenMaxLists ? ScreenWs::bytes(nq, nlist, nprobe) : 0;
  return carve_bytes<uint32_t>((size_t)nq * nprobe) + carve_bytes<float>((size_t)nq * nprobe) +
         carve_bytes<int>(1) + std::max(fgpu_coarse_workspace_bytes(nq, nlist), screen);
}

fgpu_status fgpu_search(const fgpu_index* ix, const float* dq, int nq, int nprobe, int k, float prune_ratio,
                        int32_t* d_out_ids, float* d_out_dists, void* ws, size_t ws_bytes, void* stream) {
  FGPU_CHECK(ix && ws, FGPU_ERR_ARG, "search: null argument");
  Carve cv(ws, ws_bytes);
  uint32_t* pid = cv.take<uint32_t>((size_t)nq * nprobe);
  float* pd = cv.take<float>((size_t)nq * nprobe);
  int* qctr = cv.take<int>(1);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "search: workspace too small");
  FGPU_CHECK(nq >= 0 && k >= 1, FGPU_ERR_ARG, "search: bad sizes");
  FGPU_CHECK(adc_supported(ix->dim, ix->m), FGPU_ERR_UNSUPPORTED, "search: no kernel for this (dim, pq_m)");
  void* rest = cv.base + cv.used;
  const size_t rest_bytes = ws_bytes - cv.used;
  // The MFMA screen + exact rescore (screen.hip), when the index has its
  // arrays, k <= 64 and the workspace holds its buffers; the queries it hands
  // back go through the generic LUT kernel.  Otherwise the LUT flow kernel.
  // With FGPU_OPT_STAGE_EVENTS, events between the stages (fgpu_search_stage_times).
  hipStream_t s = as_stream(stream);
  const hipEvent_t* ev = ix->opt_stage_events ? ix->stage_ev : nullptr;
  auto mark = [&](int i) { return ev ? hipEventRecord(ev[i], s) : hipSuccess; };
  FGPU_HIP(mark(0));
  ScreenWs sw;
  if (ix->screen_ok && ix->opt_screen && k <= 64 && nq > 0 && ((uintptr_t)dq & 15) == 0 &&
      ix->nlist <= kScreenMaxLists && (int64_t)nq * nprobe < INT32_MAX &&
      sw.carve(rest, rest_bytes, nq, ix->nlist, nprobe)) {
    FGPU_TRY(coarse_search(ix, dq, nq, nprobe, prune_ratio, pid, pd, rest, rest_bytes, stream, nullptr, 0));
    FGPU_HIP(mark(1));
    ScreenArgs sa{dq, ix->d_centroids, ix->d_offsets, ix->d_codes, ix->d_ids, ix->d_codebook, ix->d_cb16,
                  ix->d_vext, ix->d_rmax, pid, pd, nq, nprobe, k, ix->nlist};
    sa.scale_exp = ix->screen_scale_exp;
    sa.ctr = sw.zero;
    sa.cnt1 = sw.zero + kCtrCount;
    sa.cnt2 = sa.cnt1 + ix->nlist;
    sa.cand_cnt = sa.cnt2 + ix->nlist;
    sa.first = sw.first;
    sa.gminbuf = sw.gminbuf;
    sa.bucket = sw.bucket;
    sa.arec = sw.arec;
    sa.thr = sw.thr;
    sa.cand = sw.cand;
    sa.cand_cap = kScreenCandCap;
    sa.flist = sw.flist;
    sa.out_ids = d_out_ids;
    sa.out_d = d_out_dists;
    if (ix->opt_screen_clocks) sa.stats = reinterpret_cast<unsigned long long*>(sw.zero + 16);
    sa.events = ev ? ev + 2 : nullptr;
    FGPU_TRY(launch_screen(ix->dim, ix->m, sa, s));
    AdcArgs a = adc_args(ix, dq, nq, pid, pd, nprobe, k, d_out_ids, d_out_dists);
    a.qlist = sw.flist;
    a.qcount = sw.zero + kCtrFlag;
    FGPU_TRY(launch_adc_plain_list(ix->dim, ix->m, a, s));
    FGPU_HIP(mark(kStageEvents - 1));
    return FGPU_OK;
  }
  // The scan claims queries from a counter that starts at its grid size; the
  // coarse step's select stores that value on the way.
  const int grid = flow_grid(ix->dim, ix->m, nq, nprobe);
  FGPU_TRY(coarse_search(ix, dq, nq, nprobe, prune_ratio, pid, pd, rest, rest_bytes, stream,
                         grid > 0 ? qctr : nullptr, grid));
  for (int i = 1; i < kStageEvents - 1; ++i) FGPU_HIP(mark(i));  // no screen stages
  AdcArgs a = adc_args(ix, dq, nq, pid, pd, nprobe, k, d_out_ids, d_out_dists);
  a.qctr = qctr;
  a.qctr_preset = grid;
  FGPU_TRY(launch_adc_plain(ix->dim, ix->m, a, s));
  FGPU_HIP(mark(kStageEvents - 1));
  return FGPU_OK;
}

fgpu_status fgpu_search_stage_times(const fgpu_index* ix, float* h_ms, int n) {
  FGPU_CHECK(ix && h_ms, FGPU_ERR_ARG, "search_stage_times: null argument");
  FGPU_CHECK(ix->opt_stage_events && ix->stage_ev[0], FGPU_ERR_ARG,
             "search_stage_times: FGPU_OPT_STAGE_EVENTS is off for this index");
  FGPU_HIP(hipEventSynchronize(ix->stage_ev[kStageEvents - 1]));
  for (int i = 0; i + 1 < kStageEvents && i < n; ++i)
    FGPU_HIP(hipEventElapsedTime(&h_ms[i], ix->stage_ev[i], ix->stage_ev[i + 1]));
  return FGPU_OK;
}

fgpu_status fgpu_search_screen_stats(const fgpu_index* ix, int nq, int nprobe, const void* ws, size_t ws_bytes,
                                     void* stream, long long* h_stats, int n_stats) {
  FGPU_CHECK(ix && ws && h_stats && n_stats >= 0 && nq >= 0 && nprobe >= 1, FGPU_ERR_ARG,
             "search_screen_stats: bad argument");
  Carve cv(const_cast<void*>(ws), ws_bytes);
  cv.take<uint32_t>((size_t)nq * nprobe);
  cv.take<float>((size_t)nq * nprobe);
  cv.take<int>(1);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "search_screen_stats: workspace too small");
  ScreenWs sw;
  FGPU_CHECK(sw.carve(cv.base + cv.used, ws_bytes - cv.used, nq, ix->nlist, nprobe), FGPU_ERR_WORKSPACE,
             "search_screen_stats: workspace too small for the screen");
  hipStream_t s = as_stream(stream);
  std::vector<int> z(ScreenWs::zero_words(nq, ix->nlist));
  std::vector<float> thr((size_t)nq);
  FGPU_HIP(hipMemcpyAsync(z.data(), sw.zero, sizeof(int) * z.size(), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipMemcpyAsync(thr.data(), sw.thr, sizeof(float) * thr.size(), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipStreamSynchronize(s));
  long long st[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int l = 0; l < ix->nlist; ++l) {
    st[0] += z[kCtrCount + l];
    st[2] += z[kCtrCount + ix->nlist + l];
    st[1] += z[kCtrCount + ix->nlist + l] > 0 ? 1 : 0;
  }
  for (int q = 0; q < nq; ++q) {
    const int c = z[kCtrCount + 2 * ix->nlist + q];
    st[3] += std::min(c, kScreenCandCap);
    st[4] = std::max<long long>(st[4], c);
    st[6] += thr[q] < FLT_MAX ? 1 : 0;  // FLT_MAX: candidates set without a screen
  }
  st[5] = z[kCtrFlag];
  for (int i = 0; i < n_stats && i < 8; ++i) h_stats[i] = st[i];
  // With FGPU_OPT_SCREEN_CLOCKS: the screen kernels' clock and tile counts.
  unsigned long long ck[8];
  std::memcpy(ck, z.data() + 16, sizeof(ck));
  for (int i = 0; i < 8 && 8 + i < n_stats; ++i) h_stats[8 + i] = (long long)ck[i];
  if (n_stats > 16) {
    // The work of each round: (query, vector) pairs screened, and the MFMA
    // tiles run (32-query groups of a list times its 32-vector tiles).
    std::vector<int32_t> off((size_t)ix->nlist + 1);
    FGPU_HIP(hipMemcpy(off.data(), ix->d_offsets, sizeof(int32_t) * off.size(), hipMemcpyDeviceToHost));
    long long w[4] = {0, 0, 0, 0};
    for (int l = 0; l < ix->nlist; ++l) {
      const long long n = off[l + 1] - off[l];
      for (int r = 0; r < 2; ++r) {
        const long long c = std::min(z[kCtrCount + r * ix->nlist + l], nq);
        w[r] += c * n;
        w[2 + r] += (c + 31) / 32 * ((n + 31) / 32);
      }
    }
    for (int i = 0; i < 4 && 16 + i < n_stats; ++i) h_stats[16 + i] = w[i];
  }
  return FGPU_OK;
}

fgpu_status fgpu_index_set_option(fgpu_index* ix, int option, int value) {
  FGPU_CHECK(ix, FGPU_ERR_ARG, "index_set_option: null index");
  switch (option) {
    case FGPU_OPT_LIST_SKIP: ix->opt_list_skip = value ? 1 : 0; return FGPU_OK;
    case FGPU_OPT_SPIN_LIMIT: ix->opt_spin_limit = value > 0 ? value : 0; return FGPU_OK;
    case FGPU_OPT_SCREEN: ix->opt_screen = value ? 1 : 0; return FGPU_OK;
    case FGPU_OPT_SCREEN_CLOCKS: ix->opt_screen_clocks = value ? 1 : 0; return FGPU_OK;
    case FGPU_OPT_TWO_PHASE_SPLIT: ix->opt_two_phase_split = value > 0 ? value : 0; return FGPU_OK;
    case FGPU_OPT_TWO_PHASE_SCREEN: ix->opt_two_phase_screen = value >= 0 && value <= 2 ? value : 0; return FGPU_OK;
    case FGPU_OPT_STAGE_EVENTS:
      if (value && !ix->stage_ev[0])
        for (hipEvent_t& e : ix->stage_ev) FGPU_HIP(hipEventCreate(&e));
      ix->opt_stage_events = value ? 1 : 0;
      return FGPU_OK;
    default: return set_error(FGPU_ERR_ARG, "index_set_option: unknown option " + std::to_string(option));
  }
}

int fgpu_index_screen_ready(const fgpu_index* ix) { return ix && ix->screen_ok ? 1 : 0; }

// ---------------------------------------------------------------------------
size_t fgpu_two_phase_workspace_bytes(int nq, int nprobe, int p1_lists, int limit_k, int rerank_m) {
  const int p1 = std::max(0, std::min(nprobe, p1_lists));
  const size_t rows = (size_t)std::max(nq, 1);
  // Each query's candidate pool, then its phase-1 cutoffs (split phase 1),
  // then (limit_k <= 64) the buffers of phase 1 through the screen for up to
  // kTpVqMax virtual queries, sized for the largest lists count and dim, and
  // the list of queries that take the general second half.
  size_t b = carve_bytes<uint64_t>(rows * two_phase_pool_cap(p1, limit_k, rerank_m)) +
             carve_bytes<float>(rows * (size_t)std::max(nprobe, 1));
  if (limit_k >= 1 && limit_k <= 64 && p1 >= 1)
    b += TpScreenWs::bytes((int)std::min<int64_t>((int64_t)rows * p1, kTpVqMax), kScreenMaxLists, 128, limit_k) +
         carve_bytes<int32_t>(rows + 1) + 1024;
  return b;
}

}  // extern "C"

namespace {
fgpu_status two_phase(const fgpu_index* ix, const float* dq, int nq, const uint32_t* d_probe_ids, int nprobe,
                      int p1_lists, int limit_k, float threshold_coeff, int rerank_m, int32_t* d_top_ids,
                      float* d_top_dists, int32_t* d_top_counts, float* d_list_cutoffs, float* d_thresholds,
                      unsigned long long* d_stats, void* ws, size_t ws_bytes, void* stream,
                      int32_t* d_pre_cut = nullptr, const float* d_probe_dists = nullptr) {
  FGPU_CHECK(ix && ws && (nq == 0 || (dq && d_probe_ids && d_top_ids && d_top_dists && d_top_counts)), FGPU_ERR_ARG,
             "two_phase_search: null argument");
  FGPU_CHECK(nq >= 0 && nprobe >= 1 && nprobe <= 256, FGPU_ERR_ARG, "two_phase_search: need 1 <= nprobe <= 256");
  FGPU_CHECK(limit_k >= 1 && rerank_m >= 1, FGPU_ERR_ARG, "two_phase_search: limit_k and rerank_m must be >= 1");
  FGPU_CHECK(adc_supported(ix->dim, ix->m), FGPU_ERR_UNSUPPORTED, "two_phase_search: no kernel for this (dim, pq_m)");
  if (nq == 0) return FGPU_OK;
  const int p1 = std::max(0, std::min(nprobe, p1_lists));
  const int cap = two_phase_pool_cap(p1, limit_k, rerank_m);
  hipStream_t s = as_stream(stream);
  // Phase 1 through the MFMA screen (limit_k <= 64, an index with the
  // screen's arrays, queries 16-byte aligned): every (query, phase-1 probe)
  // is a virtual query of one probe whose exact top-limit_k the screen
  // returns (its LUT kernel takes the virtual queries it cannot settle); they
  // fill the pool slots and cutoffs a split phase 1 leaves, and the
  // two-phase kernel's second half runs the threshold, phase 2 and the final
  // select.  The virtual queries' buffers take the end of the workspace; the
  // pools and cutoff rows the rest.
  const bool tp_screen = ix->opt_two_phase_screen == 2 ||
                         (ix->opt_two_phase_screen == 0 && (int64_t)nq >= kTpScreenMinQueries);
  if (tp_screen && ix->screen_ok && ix->opt_screen && limit_k <= 64 && p1 >= 1 && screen_supported(ix->dim, ix->m) &&
      ix->nlist <= kScreenMaxLists && ((uintptr_t)dq & 15) == 0) {
    // With FGPU_OPT_STAGE_EVENTS, the stage events of fgpu_search_stage_times
    // around the last virtual-query chunk's set-up and screen stages; the
    // last stage runs from its rescore to the end of the call.
    const hipEvent_t* ev = ix->opt_stage_events ? ix->stage_ev : nullptr;
    auto mark = [&](int i) { return ev ? hipEventRecord(ev[i], s) : hipSuccess; };
    const int qv = std::max(1, kTpVqMax / p1);  // queries a virtual-query chunk
    const int nvq_max = (int)std::min<int64_t>((int64_t)nq, qv) * p1;
    const size_t tbytes = TpScreenWs::bytes(nvq_max, ix->nlist, ix->dim, limit_k);
    const size_t per_q = (size_t)cap * sizeof(uint64_t) + nprobe * sizeof(float) + sizeof(int32_t);
    if (ws_bytes > tbytes + 3 * 256 + per_q) {
      const size_t tofs = align_up(ws_bytes - tbytes, 256) - 256;  // 256-aligned, inside the workspace
      char* tbase = static_cast<char*>(ws) + tofs;
      // per query chunk: pools, cutoff rows, and the list of queries that
      // take the general second half (its count first)
      auto need = [&](int64_t c) {
        return carve_bytes<uint64_t>((size_t)c * cap) + carve_bytes<float>((size_t)c * nprobe) +
               carve_bytes<int32_t>((size_t)c + 1);
      };
      int64_t chunk = std::min<int64_t>(nq, (int64_t)(tofs / per_q));
      while (chunk > 0 && need(chunk) > tofs) --chunk;
      if (chunk >= 1) {
        Carve pc(ws, tofs);
        uint64_t* pool = pc.take<uint64_t>((size_t)chunk * cap);
        float* cut_ws = pc.take<float>((size_t)chunk * nprobe);
        int32_t* slow = pc.take<int32_t>((size_t)chunk + 1);  // [0]: count, then the queries
        for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
          const int nb = (int)std::min<int64_t>(chunk, nq - q0);
          const float* qq = dq + q0 * ix->dim;
          const uint32_t* pp = d_probe_ids + q0 * nprobe;
          TwoPhaseArgs a{qq, ix->d_centroids, ix->d_codebook, ix->d_offsets, ix->d_codes, ix->d_ids, pp, ix->d_rmax,
                         nb, nprobe, ix->nlist, p1, limit_k, threshold_coeff, rerank_m, pool, cap,
                         d_top_ids + q0 * rerank_m, d_top_dists + q0 * rerank_m, d_top_counts + q0,
                         d_list_cutoffs ? d_list_cutoffs + q0 * p1 : nullptr,
                         d_thresholds ? d_thresholds + q0 : nullptr, d_stats};
          a.cut_ws = cut_ws;
          a.pre_cut = d_pre_cut ? d_pre_cut + q0 : nullptr;
          FGPU_TRY(launch_tp_zero(slow, 1, s));
          for (int s0 = 0; s0 < nb; s0 += qv) {
            const int ns = std::min(qv, nb - s0), nvq = ns * p1;
            TpScreenWs tw;
            FGPU_CHECK(tw.carve(tbase, ws_bytes - tofs, nvq, ix->nlist, ix->dim, limit_k), FGPU_ERR_WORKSPACE,
                       "two_phase_search: screen buffers do not fit");
            FGPU_HIP(mark(0));
            const float* cq = qq + (int64_t)s0 * ix->dim;  // the chunk's query rows
            FGPU_TRY(launch_tp_virtual(pp + (int64_t)s0 * nprobe, nprobe, p1, ns, ix->d_offsets, ix->nlist, tw.vprobe,
                                       tw.vpd, tw.hist, tw.rank, s));
            FGPU_TRY(launch_tp_offsets(tw.hist, ix->nlist, tw.boff, ix->d_offsets, limit_k, tw.sp_cnt, s));
            FGPU_TRY(launch_tp_order(tw.vprobe, tw.rank, nvq, ix->nlist, tw.boff, tw.order, s));
            FGPU_HIP(mark(1));
            ScreenArgs sa{cq, ix->d_centroids, ix->d_offsets, ix->d_codes, ix->d_ids, ix->d_codebook, ix->d_cb16,
                          ix->d_vext, ix->d_rmax, tw.vprobe, tw.vpd, nvq, 1, limit_k, ix->nlist};
            sa.scale_exp = ix->screen_scale_exp;
            sa.qdiv = p1;
            sa.ctr = tw.sw.zero;
            sa.cnt1 = tw.sw.zero + kCtrCount;
            sa.cnt2 = sa.cnt1 + ix->nlist;
            sa.cand_cnt = sa.cnt2 + ix->nlist;
            sa.first = tw.sw.first;
            sa.gminbuf = tw.sw.gminbuf;
            sa.bucket = tw.order;  // single-probe mode: each list's queries, as ordered
            sa.boff = tw.boff;
            sa.order = tw.order;
            sa.sp_cnt = tw.sp_cnt;
            sa.pnorm = tw.pnorm;
            sa.r2_chunk = 128;  // one 32-query group a list: shorter chunks balance round 2
            sa.r2_max_chunks = 16;
            sa.arec = tw.sw.arec;
            sa.thr = tw.sw.thr;
            sa.cand = tw.sw.cand;
            sa.cand_cap = kScreenCandCap;
            sa.flist = tw.sw.flist;
            sa.out_ids = tw.vids;
            sa.out_d = tw.vd;
            sa.events = ev ? ev + 2 : nullptr;
            FGPU_TRY(launch_screen(ix->dim, ix->m, sa, s));
            AdcArgs la = adc_args(ix, cq, nvq, tw.vprobe, tw.vpd, 1, limit_k, tw.vids, tw.vd);
            la.qdiv = p1;
            la.qlist = tw.sw.flist;
            la.qcount = tw.sw.zero + kCtrFlag;
            FGPU_TRY(launch_adc_plain_list(ix->dim, ix->m, la, s));
            // single-probe mode: both rounds screen the sp_cnt pairs
            FGPU_TRY(launch_tp_stats(sa.cand_cnt, sa.thr, nvq, kScreenCandCap, tw.sw.zero + kCtrFlag, tw.sp_cnt,
                                     tw.sp_cnt, tw.boff, ix->d_offsets, ix->nlist, d_stats, s));
            FGPU_TRY(launch_tp_finish(a, ix->dim, s0, ns, tw.vids, tw.vd,
                                      d_probe_dists ? d_probe_dists + q0 * nprobe : nullptr, slow + 1, slow, s));
          }
          // the queries whose phase 2 may append, or whose keys need a select
          a.qlist = slow + 1;
          a.qcount = slow;
          FGPU_TRY(launch_two_phase_after_phase1(ix->dim, ix->m, a, s));
        }
        FGPU_HIP(mark(kStageEvents - 1));
        return FGPU_OK;
      }
    }
  }
  // Queries a launch: their pools and cutoff rows fit the workspace.
  auto need = [&](int64_t c) {
    return carve_bytes<uint64_t>((size_t)c * cap) + carve_bytes<float>((size_t)c * nprobe);
  };
  int64_t chunk = std::min<int64_t>(nq, (int64_t)(ws_bytes / ((size_t)cap * sizeof(uint64_t) + nprobe * sizeof(float))));
  while (chunk > 0 && need(chunk) > ws_bytes) --chunk;
  FGPU_CHECK(chunk >= 1, FGPU_ERR_WORKSPACE, "two_phase_search: workspace smaller than one query's pool");
  float* cut_ws = reinterpret_cast<float*>(static_cast<char*>(ws) + carve_bytes<uint64_t>((size_t)chunk * cap));
  for (int64_t q0 = 0; q0 < nq; q0 += chunk) {
    const int nb = (int)std::min<int64_t>(chunk, nq - q0);
    TwoPhaseArgs a{dq + q0 * ix->dim, ix->d_centroids, ix->d_codebook, ix->d_offsets, ix->d_codes, ix->d_ids,
                   d_probe_ids + q0 * nprobe, ix->d_rmax, nb, nprobe, ix->nlist, p1, limit_k, threshold_coeff,
                   rerank_m, reinterpret_cast<uint64_t*>(ws), cap, d_top_ids + q0 * rerank_m,
                   d_top_dists + q0 * rerank_m, d_top_counts + q0,
                   d_list_cutoffs ? d_list_cutoffs + q0 * p1 : nullptr, d_thresholds ? d_thresholds + q0 : nullptr,
                   d_stats};
    // A batch too small to fill the GPU (two workgroups a CU) spreads each
    // query's phase-1 lists over several workgroups.
    a.split = two_phase_split(nb, p1, limit_k, ix->opt_two_phase_split);
    a.cut_ws = cut_ws;
    a.pre_cut = d_pre_cut ? d_pre_cut + q0 : nullptr;
    FGPU_TRY(launch_two_phase(ix->dim, ix->m, a, as_stream(stream)));
  }
  return FGPU_OK;
}
}  // namespace

extern "C" {

fgpu_status fgpu_two_phase_search(const fgpu_index* ix, const float* dq, int nq, const uint32_t* d_probe_ids,
                                  int nprobe, int p1_lists, int limit_k, float threshold_coeff, int rerank_m,
                                  int32_t* d_top_ids, float* d_top_dists, int32_t* d_top_counts,
                                  float* d_list_cutoffs, float* d_thresholds, void* ws, size_t ws_bytes,
                                  void* stream) {
  return two_phase(ix, dq, nq, d_probe_ids, nprobe, p1_lists, limit_k, threshold_coeff, rerank_m, d_top_ids,
                   d_top_dists, d_top_counts, d_list_cutoffs, d_thresholds, nullptr, ws, ws_bytes, stream);
}

fgpu_status fgpu_two_phase_search_precut(const fgpu_index* ix, const float* dq, int nq,
                                         const uint32_t* d_probe_ids, int nprobe, int p1_lists, int limit_k,
                                         float threshold_coeff, int rerank_m, int32_t* d_top_ids, float* d_top_dists,
                                         int32_t* d_top_counts, float* d_list_cutoffs, float* d_thresholds,
                                         int32_t* d_pre_cut, void* ws, size_t ws_bytes, void* stream) {
  FGPU_CHECK(d_pre_cut || nq == 0, FGPU_ERR_ARG, "two_phase_search_precut: null d_pre_cut");
  return two_phase(ix, dq, nq, d_probe_ids, nprobe, p1_lists, limit_k, threshold_coeff, rerank_m, d_top_ids,
                   d_top_dists, d_top_counts, d_list_cutoffs, d_thresholds, nullptr, ws, ws_bytes, stream, d_pre_cut);
}

fgpu_status fgpu_two_phase_search_stats(const fgpu_index* ix, const float* dq, int nq, const uint32_t* d_probe_ids,
                                        int nprobe, int p1_lists, int limit_k, float threshold_coeff, int rerank_m,
                                        int32_t* d_top_ids, float* d_top_dists, int32_t* d_top_counts,
                                        unsigned long long* d_stats, void* ws, size_t ws_bytes, void* stream) {
  FGPU_CHECK(d_stats, FGPU_ERR_ARG, "two_phase_search_stats: null stats");
  return two_phase(ix, dq, nq, d_probe_ids, nprobe, p1_lists, limit_k, threshold_coeff, rerank_m, d_top_ids,
                   d_top_dists, d_top_counts, nullptr, nullptr, d_stats, ws, ws_bytes, stream);
}

fgpu_status fgpu_rerank(const float* dq, int nq, int dim, const float* d_base, int64_t n, const int32_t* d_top_ids,
                        const int32_t* d_top_counts, int rerank_m, int k, int mini_batch, float eps, int beta,
                        int32_t* d_final_ids, float* d_final_dists, int32_t* d_visited, void* stream) {
  return fgpu_rerank_spec(dq, nq, dim, d_base, n, d_top_ids, d_top_counts, rerank_m, k, mini_batch, eps, beta,
                          d_final_ids, d_final_dists, d_visited, 0, stream);
}

fgpu_status fgpu_rerank_spec(const float* dq, int nq, int dim, const float* d_base, int64_t n,
                             const int32_t* d_top_ids, const int32_t* d_top_counts, int rerank_m, int k,
                             int mini_batch, float eps, int beta, int32_t* d_final_ids, float* d_final_dists,
                             int32_t* d_visited, int spec, void* stream) {
  return fgpu_rerank_state(dq, nq, dim, d_base, n, d_top_ids, d_top_counts, rerank_m, k, mini_batch, eps, beta,
                           d_final_ids, d_final_dists, d_visited, nullptr, nullptr, spec, stream);
}

fgpu_status fgpu_rerank_state(const float* dq, int nq, int dim, const float* d_base, int64_t n,
                              const int32_t* d_top_ids, const int32_t* d_top_counts, int rerank_m, int k,
                              int mini_batch, float eps, int beta, int32_t* d_final_ids, float* d_final_dists,
                              int32_t* d_visited, int32_t* d_stable_cnt, uint8_t* d_finished, int spec,
                              void* stream) {
  FGPU_CHECK(d_base && (nq == 0 || (dq && d_top_ids && d_top_counts && d_final_ids && d_final_dists)), FGPU_ERR_ARG,
             "rerank: null argument");
  FGPU_CHECK(nq >= 0 && n >= 0 && rerank_m >= 1 && k >= 1 && mini_batch >= 1, FGPU_ERR_ARG, "rerank: bad sizes");
  FGPU_CHECK(((uintptr_t)d_base & 15) == 0 && ((uintptr_t)dq & 15) == 0, FGPU_ERR_ARG,
             "rerank: base vectors and queries must be 16-byte aligned");
  RerankArgs a{dq, d_base, (long long)n, d_top_ids, d_top_counts, nq, rerank_m, k, mini_batch, eps, beta,
               d_final_ids, d_final_dists, d_visited};
  a.spec = spec < 0 ? 0 : spec;
  a.stable = d_stable_cnt;
  a.finished = d_finished;
  return launch_rerank(dim, a, as_stream(stream));
}

size_t fgpu_search_rerank_workspace_bytes(int nq, int nlist, int nprobe, int p1_lists, int limit_k, int rerank_m) {
  return carve_bytes<uint32_t>((size_t)nq * nprobe) + carve_bytes<float>((size_t)nq * nprobe) +
         carve_bytes<int32_t>((size_t)nq * rerank_m) + carve_bytes<float>((size_t)nq * rerank_m) +
         carve_bytes<int32_t>((size_t)nq) +
         std::max(fgpu_coarse_workspace_bytes(nq, nlist),
                  fgpu_two_phase_workspace_bytes(nq, nprobe, p1_lists, limit_k, rerank_m));
}

fgpu_status fgpu_search_rerank(const fgpu_index* ix, const float* dq, int nq, int nprobe, float prune_ratio,
                               int p1_lists, int limit_k, float threshold_coeff, int rerank_m, const float* d_base,
                               int64_t n, int k, int mini_batch, float eps, int beta, int32_t* d_out_ids,
                               float* d_out_dists, void* ws, size_t ws_bytes, void* stream) {
  FGPU_CHECK(ix && ws, FGPU_ERR_ARG, "search_rerank: null argument");
  if (nq == 0) return FGPU_OK;
  Carve cv(ws, ws_bytes);
  uint32_t* pid = cv.take<uint32_t>((size_t)nq * nprobe);
  float* pd = cv.take<float>((size_t)nq * nprobe);
  int32_t* tid = cv.take<int32_t>((size_t)nq * rerank_m);
  float* tdist = cv.take<float>((size_t)nq * rerank_m);
  int32_t* tcnt = cv.take<int32_t>((size_t)nq);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "search_rerank: workspace too small");
  void* rest = cv.base + cv.used;
  const size_t rest_bytes = ws_bytes - cv.used;
  FGPU_TRY(fgpu_coarse_search(ix, dq, nq, nprobe, prune_ratio, pid, pd, rest, rest_bytes, stream));
  // the coarse step's probe distances give the phase-2 list bounds
  FGPU_TRY(two_phase(ix, dq, nq, pid, nprobe, p1_lists, limit_k, threshold_coeff, rerank_m, tid, tdist, tcnt, nullptr,
                     nullptr, nullptr, rest, rest_bytes, stream, nullptr, pd));
  return fgpu_rerank(dq, nq, ix->dim, d_base, n, tid, tcnt, rerank_m, k, mini_batch, eps, beta, d_out_ids,
                     d_out_dists, nullptr, stream);
}

// ---------------------------------------------------------------------------
size_t fgpu_l2_topk_workspace_bytes(int64_t n, int nc) {
  return carve_bytes<float>(nc) + 256 + carve_bytes<float>((size_t)topk_batch_rows(n, nc) * (size_t)est_sel_ld(nc));
}

fgpu_status fgpu_l2_topk(const float* dx, int64_t n, const float* dc, int nc, int dim, int p, int32_t* d_ids,
                         float* d_dists, void* ws, size_t ws_bytes, void* stream) {
  FGPU_CHECK(dc && ws && (n == 0 || (dx && d_ids && d_dists)), FGPU_ERR_ARG, "l2_topk: null argument");
  FGPU_CHECK(((uintptr_t)ws & 15) == 0, FGPU_ERR_ARG, "l2_topk: workspace must be 16-byte aligned");
  FGPU_CHECK(n >= 0 && nc >= 1 && dim >= 1 && p >= 1 && p <= nc && p <= 256, FGPU_ERR_ARG, "l2_topk: bad sizes");
  if (n == 0) return FGPU_OK;
  hipStream_t s = as_stream(stream);
  Carve cv(ws, ws_bytes);
  float* cn = cv.take<float>(nc);
  float* cmax = cv.take<float>(64);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "l2_topk: workspace too small");
  const size_t rest = ws_bytes - cv.used;
  const int64_t ld = est_sel_ld(nc);
  const int64_t rows = std::min<int64_t>(est_rows_per_batch(rest, (int)ld), ((n + 63) / 64) * 64);
  FGPU_CHECK(rows >= 64, FGPU_ERR_WORKSPACE, "l2_topk: workspace too small");
  void* est = cv.take<float>((size_t)rows * ld);
  FGPU_TRY(launch_row_norms(dc, nc, dim, cn, s));
  FGPU_TRY(launch_max_reduce(cn, nc, cmax, s));
  for (int64_t b0 = 0; b0 < n; b0 += rows) {
    const int64_t nb = std::min<int64_t>(rows, n - b0);
    FGPU_TRY(launch_gemm_est_sel(dx + b0 * dim, nb, dc, nc, dim, cn, cmax, est, ld, s));
    FGPU_TRY(launch_select_exact(est, ld, nb, nc, dx + b0 * dim, dc, dim, cmax, p, 0, 0.0f, d_ids + b0 * p,
                                 d_dists + b0 * p, s));
  }
  return FGPU_OK;
}

// ---------------------------------------------------------------------------
}  // extern "C"

namespace {
constexpr int kKnnChunk = 4096;
int64_t knn_rows(int nq) {
  const int64_t budget = 256ll << 20;
  const int64_t r = budget / ((int64_t)kKnnChunk * sizeof(float));
  return std::min<int64_t>(r - r % 64, ((int64_t)nq + 63) / 64 * 64);
}
}  // namespace

extern "C" {

size_t fgpu_knn_exact_workspace_bytes(int nq, int64_t n) {
  return carve_bytes<float>((size_t)std::max(nq, 1)) + carve_bytes<float>((size_t)std::max<int64_t>(n, 1)) +
         carve_bytes<float>(64) + carve_bytes<float>((size_t)knn_rows(std::max(nq, 1)) * kKnnChunk);
}

fgpu_status fgpu_knn_exact(const float* dq, int nq, const float* d_base, int64_t n, int dim, int k, int32_t* d_ids,
                           float* d_dists, void* ws, size_t ws_bytes, void* stream) {
  FGPU_CHECK(d_base && ws && (nq == 0 || (dq && d_ids && d_dists)), FGPU_ERR_ARG, "knn_exact: null argument");
  FGPU_CHECK(nq >= 0 && n >= 1 && n < INT32_MAX && k >= 1 && k <= 128, FGPU_ERR_ARG,
             "knn_exact: need 1 <= k <= 128 and 1 <= n < 2^31");
  FGPU_CHECK(dim >= 4 && dim <= 256 && dim % 4 == 0, FGPU_ERR_UNSUPPORTED,
             "knn_exact: dim must be a multiple of 4 in [4, 256]");
  if (nq == 0) return FGPU_OK;
  hipStream_t s = as_stream(stream);
  Carve cv(ws, ws_bytes);
  float* qn = cv.take<float>(nq);
  float* bn = cv.take<float>(n);
  float* bmax = cv.take<float>(64);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "knn_exact: workspace too small");
  const size_t rest = ws_bytes - cv.used;
  const int64_t rows = std::min<int64_t>(est_rows_per_batch(rest, kKnnChunk), ((int64_t)nq + 63) / 64 * 64);
  FGPU_CHECK(rows >= 64, FGPU_ERR_WORKSPACE, "knn_exact: workspace too small");
  float* est = cv.take<float>((size_t)rows * kKnnChunk);
  FGPU_TRY(launch_row_norms(dq, nq, dim, qn, s));
  FGPU_TRY(launch_row_norms(d_base, n, dim, bn, s));
  FGPU_TRY(launch_max_reduce(bn, n, bmax, s));
  for (int64_t b0 = 0; b0 < nq; b0 += rows) {
    const int64_t nb = std::min<int64_t>(rows, nq - b0);
    for (int64_t c0 = 0; c0 < n; c0 += kKnnChunk) {
      const int ncols = (int)std::min<int64_t>(kKnnChunk, n - c0);
      FGPU_TRY(launch_gemm_est(dq + b0 * dim, nb, d_base + c0 * dim, ncols, dim, qn + b0, bn + c0, est, kKnnChunk, s));
      FGPU_TRY(launch_knn_chunk(est, kKnnChunk, nb, ncols, dq + b0 * dim, d_base + c0 * dim, dim, qn + b0, bmax, k,
                                (int)c0, c0 > 0, d_ids + b0 * k, d_dists + b0 * k, s));
    }
  }
  return FGPU_OK;
}

fgpu_status fgpu_graph_search(const float* dq, int nq, const float* d_base, int64_t n, int dim, const int32_t* d_graph,
                              int degree, int itopk, int width, int max_iter, int k, uint64_t seed, int32_t* d_out_ids,
                              float* d_out_dists, int32_t* d_iters, int32_t* d_evals, void* stream) {
  FGPU_CHECK(d_base && d_graph && (nq == 0 || (dq && d_out_ids && d_out_dists)), FGPU_ERR_ARG,
             "graph_search: null argument");
  FGPU_CHECK(nq >= 0, FGPU_ERR_ARG, "graph_search: nq must be >= 0");
  FGPU_CHECK(((uintptr_t)d_base & 15) == 0, FGPU_ERR_ARG, "graph_search: base vectors must be 16-byte aligned");
  GraphArgs a{dq, d_base, (long long)n, d_graph, degree, itopk, width, max_iter, k, seed, 0, nq,
              d_out_ids, d_out_dists, d_iters, d_evals};
  return launch_graph_search(dim, a, as_stream(stream));
}

size_t fgpu_coarse_graph_workspace_bytes(int nlist, int degree) {
  const size_t cells = (size_t)std::max(nlist, 1) * (size_t)(2 * std::max(degree, 1) + 1);
  return 2 * carve_bytes<int32_t>(cells) + carve_bytes<float>(cells) + fgpu_knn_exact_workspace_bytes(nlist, nlist) +
         256;
}

fgpu_status fgpu_coarse_graph_build(const fgpu_index* ix, int degree, int32_t* d_graph, void* ws, size_t ws_bytes,
                                    void* stream) {
  FGPU_CHECK(ix && d_graph && ws, FGPU_ERR_ARG, "coarse_graph_build: null argument");
  FGPU_CHECK(degree >= 1 && degree <= 64 && 2 * degree < ix->nlist, FGPU_ERR_ARG,
             "coarse_graph_build: need 1 <= degree <= 64 and 2 * degree < nlist");
  hipStream_t s = as_stream(stream);
  const int nl = ix->nlist, d2 = 2 * degree;
  Carve cv(ws, ws_bytes);
  int32_t* kid = cv.take<int32_t>((size_t)nl * (d2 + 1));
  float* kd = cv.take<float>((size_t)nl * (d2 + 1));
  int32_t* fwd = cv.take<int32_t>((size_t)nl * d2);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "coarse_graph_build: workspace too small");
  // The 2 * degree nearest other centroids of each centroid (tie rule).
  FGPU_TRY(fgpu_knn_exact(ix->d_centroids, nl, ix->d_centroids, nl, ix->dim, d2 + 1, kid, kd, cv.base + cv.used,
                          ws_bytes - cv.used, stream));
  FGPU_TRY(launch_drop_self(kid, nl, d2, fwd, s));
  std::vector<int32_t> f((size_t)nl * d2), g((size_t)nl * degree);
  FGPU_HIP(hipMemcpyAsync(f.data(), fwd, sizeof(int32_t) * f.size(), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipStreamSynchronize(s));
  FGPU_TRY(fgpu_graph_add_reverse(f.data(), nl, d2, degree, g.data(), 1));
  FGPU_HIP(hipMemcpyAsync(d_graph, g.data(), sizeof(int32_t) * g.size(), hipMemcpyHostToDevice, s));
  FGPU_HIP(hipStreamSynchronize(s));
  return FGPU_OK;
}

fgpu_status fgpu_graph_add_reverse(const int32_t* h_fwd, int64_t n, int width, int degree, int32_t* h_out,
                                   int nthreads) {
  FGPU_CHECK(h_fwd && h_out && n >= 0 && degree >= 1 && width >= degree && n < INT32_MAX, FGPU_ERR_ARG,
             "graph_add_reverse: need n < 2^31 and 1 <= degree <= width");
  // Reverse edges, as CAGRA adds them (Ootomo et al., 2023): each edge u -> v
  // of the degree-nearest lists is listed at v, ordered by (rank of v in u's
  // list, u).  Counting sort: in-degrees, offsets, then a fill by rank, then
  // source, which leaves every node's list in that order.
  std::vector<int64_t> off((size_t)n + 1, 0);
  auto fwd = [&](int64_t u, int r) { return h_fwd[u * width + r]; };
  for (int64_t u = 0; u < n; ++u)
    for (int r = 0; r < degree; ++r) {
      const int32_t v = fwd(u, r);
      if (v >= 0 && v < n && v != u) ++off[(size_t)v + 1];
    }
  for (int64_t v = 0; v < n; ++v) off[(size_t)v + 1] += off[(size_t)v];
  std::vector<int32_t> rev((size_t)off[(size_t)n]);
  std::vector<int64_t> fill(off.begin(), off.end() - 1);
  for (int r = 0; r < degree; ++r)
    for (int64_t u = 0; u < n; ++u) {
      const int32_t v = fwd(u, r);
      if (v >= 0 && v < n && v != u) rev[(size_t)fill[(size_t)v]++] = (int32_t)u;
    }
  // Row v: its nearest degree - degree / 2 forward edges, then its reverse
  // edges, then the rest of its forward list, without repeats; -1 pads.
  const int nf = degree - degree / 2;
  auto rows = [&](int64_t v0, int64_t v1) {
    for (int64_t v = v0; v < v1; ++v) {
      int32_t* o = h_out + v * degree;
      int cnt = 0;
      auto add = [&](int32_t id) {
        if (id >= 0 && id < n && id != v && cnt < degree && std::find(o, o + cnt, id) == o + cnt) o[cnt++] = id;
      };
      for (int r = 0; r < nf; ++r) add(fwd(v, r));
      for (int64_t j = off[(size_t)v]; j < off[(size_t)v + 1] && cnt < degree; ++j) add(rev[(size_t)j]);
      for (int r = nf; r < width && cnt < degree; ++r) add(fwd(v, r));
      for (; cnt < degree; ++cnt) o[cnt] = -1;
    }
  };
  const int nt = (int)std::max<int64_t>(1, std::min<int64_t>(nthreads > 0 ? nthreads : 16, (n + 4095) / 4096));
  std::vector<std::thread> th;
  for (int t = 0; t < nt; ++t) th.emplace_back(rows, n * t / nt, n * (t + 1) / nt);
  for (auto& t : th) t.join();
  return FGPU_OK;
}

fgpu_status fgpu_coarse_graph_search(const fgpu_index* ix, const float* dq, int nq, int first_query, int nprobe,
                                     const int32_t* d_graph, int degree, int itopk, int width, int max_iter,
                                     uint64_t seed, float prune_ratio, uint32_t* d_probe_ids, float* d_probe_dists,
                                     void* stream) {
  FGPU_CHECK(ix && d_graph && (nq == 0 || (dq && d_probe_ids && d_probe_dists)), FGPU_ERR_ARG,
             "coarse_graph_search: null argument");
  FGPU_CHECK(nq >= 0 && first_query >= 0 && nprobe >= 1 && nprobe <= ix->nlist && nprobe <= itopk, FGPU_ERR_ARG,
             "coarse_graph_search: need first_query >= 0 and 1 <= nprobe <= min(nlist, itopk)");
  if (nq == 0) return FGPU_OK;
  hipStream_t s = as_stream(stream);
  int32_t* ids = reinterpret_cast<int32_t*>(d_probe_ids);
  GraphArgs a{dq, ix->d_centroids, (long long)ix->nlist, d_graph, degree, itopk, width, max_iter, nprobe, seed,
              first_query, nq, ids, d_probe_dists, nullptr, nullptr};
  FGPU_TRY(launch_graph_search(ix->dim, a, s));
  return launch_coarse_prune(ids, d_probe_dists, nq, nprobe, prune_ratio, s);
}

fgpu_status fgpu_tune_list_stats(const fgpu_index* idx, const float* d_queries, int nq, const float* d_base,
                                 int64_t n_base, const int32_t* d_pair_query, const int32_t* d_pair_list,
                                 const int32_t* d_pair_target, const int32_t* d_pair_kth, int npairs,
                                 float* d_target_pq, float* d_target_exact, int32_t* d_pq_rank,
                                 int32_t* d_exact_rank, float* d_kth_pq, void* stream) {
  FGPU_CHECK(idx && d_queries && d_pair_query && d_pair_list && npairs >= 0 && nq >= 0, FGPU_ERR_ARG,
             "tune_list_stats: bad argument");
  FGPU_CHECK(!d_pair_target || (d_target_pq && d_target_exact && d_pq_rank && d_exact_rank), FGPU_ERR_ARG,
             "tune_list_stats: target outputs missing");
  FGPU_CHECK(!d_pair_kth || d_kth_pq, FGPU_ERR_ARG, "tune_list_stats: k-th output missing");
  FGPU_CHECK(!d_base || n_base >= 0, FGPU_ERR_ARG, "tune_list_stats: bad n_base");
  TuneStatsArgs a{d_queries, nq, idx->dim, idx->m, idx->nlist, idx->d_offsets, idx->d_ids, idx->d_codes,
                  idx->d_centroids, idx->d_codebook, d_base, (long long)(d_base ? n_base : 0),
                  d_pair_query, d_pair_list, d_pair_target, d_pair_kth,
                  d_target_pq, d_target_exact, d_pq_rank, d_exact_rank, d_kth_pq};
  return launch_tune_list_stats(a, npairs, as_stream(stream));
}

// ---------------------------------------------------------------------------
int fgpu_fixed_shift(float maxabs, int64_t n) {
  int e = 0;
  if (maxabs > 0.0f) std::frexp((double)maxabs, &e);
  int lg = 0;
  while ((1LL << lg) < (n > 0 ? n : 1)) ++lg;
  int s = 61 - lg - e;
  return s < 0 ? 0 : (s > 60 ? 60 : s);
}

size_t fgpu_kmeans_workspace_bytes(int k, int dim) {
  return carve_bytes<unsigned long long>((size_t)k * dim) + carve_bytes<int32_t>(k);
}

fgpu_status fgpu_kmeans_update(const float* dx, int64_t n, const int32_t* d_assign, int k, int dim, int shift,
                               int empty_rule, float* d_cent, int32_t* d_counts, void* ws, size_t ws_bytes,
                               void* stream) {
  FGPU_CHECK(dx && d_assign && d_cent && ws && k >= 1 && dim >= 1 && n >= 0, FGPU_ERR_ARG, "kmeans_update: bad argument");
  hipStream_t s = as_stream(stream);
  Carve cv(ws, ws_bytes);
  auto* sums = cv.take<unsigned long long>((size_t)k * dim);
  int32_t* cnt = cv.take<int32_t>(k);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "kmeans_update: workspace too small");
  if (d_counts) cnt = d_counts;
  FGPU_TRY(launch_kmeans_accumulate(dx, n, d_assign, k, dim, shift, sums, cnt, s));
  return launch_kmeans_finalize(sums, cnt, k, dim, shift, empty_rule, d_cent, s);
}

fgpu_status fgpu_kmeans_fit(const float* dx, int64_t n, int dim, int k, int iters, int init_mode, uint64_t seed,
                            float* d_cent, int32_t* d_assign_out, void* stream) {
  FGPU_CHECK(dx && d_cent && n >= 1 && dim >= 1 && k >= 1 && k <= n && iters >= 0, FGPU_ERR_ARG,
             "kmeans_fit: bad argument");
  FGPU_CHECK(init_mode == 0 || init_mode == 1, FGPU_ERR_ARG, "kmeans_fit: init_mode must be 0 or 1");
  hipStream_t s = as_stream(stream);
  // fixed-point shift from max |x|
  DevBuf<float> scratch;
  FGPU_TRY(scratch.alloc(1024));
  FGPU_TRY(launch_maxabs(dx, n * dim, scratch.p, s));
  float maxabs = 0.0f;
  FGPU_HIP(hipMemcpyAsync(&maxabs, scratch.p + 1023, sizeof(float), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipStreamSynchronize(s));
  const int shift = fgpu_fixed_shift(maxabs, n);

  DevBuf<int32_t> rows;
  FGPU_TRY(rows.alloc(k));
  if (init_mode == 0) {
    // run_kmeans_gpu's initialisation (kmeans_gpu.cuh:259-267)
    std::vector<int32_t> h(k);
    std::mt19937 rng((unsigned)seed);
    const int64_t stride = std::max<int64_t>(1, n / k);
    for (int i = 0; i < k; ++i)
      h[i] = (int32_t)(((int64_t)i * stride + (int64_t)(rng() % (unsigned long long)stride)) % n);
    FGPU_HIP(hipMemcpyAsync(rows.p, h.data(), sizeof(int32_t) * k, hipMemcpyHostToDevice, s));
    FGPU_TRY(launch_gather_rows(dx, dim, rows.p, k, d_cent, s));
    FGPU_HIP(hipStreamSynchronize(s));
  } else {
    DevBuf<char> pws;
    const size_t b = kmeans_pp_ws_bytes(n, k);
    FGPU_TRY(pws.alloc(b));
    FGPU_TRY(launch_kmeans_pp(dx, n, dim, k, seed, d_cent, rows.p, pws.p, b, s));
    FGPU_HIP(hipStreamSynchronize(s));
  }
  DevBuf<int32_t> assign;
  DevBuf<float> dist;
  DevBuf<char> tws, kws;
  const size_t tb = fgpu_l2_topk_workspace_bytes(n, k), kb = fgpu_kmeans_workspace_bytes(k, dim);
  FGPU_TRY(assign.alloc(n));
  FGPU_TRY(dist.alloc(n));
  FGPU_TRY(tws.alloc(tb));
  FGPU_TRY(kws.alloc(kb));
  for (int it = 0; it < iters; ++it) {
    FGPU_TRY(fgpu_l2_topk(dx, n, d_cent, k, dim, 1, assign.p, dist.p, tws.p, tb, stream));
    FGPU_TRY(fgpu_kmeans_update(dx, n, assign.p, k, dim, shift, 0, d_cent, nullptr, kws.p, kb, stream));
  }
  if (d_assign_out) FGPU_TRY(fgpu_l2_topk(dx, n, d_cent, k, dim, 1, d_assign_out, dist.p, tws.p, tb, stream));
  FGPU_HIP(hipStreamSynchronize(s));
  return FGPU_OK;
}

fgpu_status fgpu_pq_train(const float* dx, int64_t n, int dim, int pq_m, const int32_t* d_assign, const float* d_cent,
                          int sample_size, int iters, float* d_codebook, void* stream) {
  FGPU_CHECK(dx && d_assign && d_cent && d_codebook && n >= 1 && pq_m >= 1 && dim % pq_m == 0 && iters >= 0,
             FGPU_ERR_ARG, "pq_train: bad argument");
  hipStream_t s = as_stream(stream);
  // sample rows (pq_utils.h:91-97)
  const int actual = (int)std::min<int64_t>(sample_size, n);
  FGPU_CHECK(actual >= kPQK, FGPU_ERR_ARG, "pq_train: need at least 256 sample rows");
  std::vector<int32_t> idx;
  {
    std::mt19937 rng(12345);
    idx = shuffled_prefix(n, actual, rng);
  }
  // per-subspace initial rows (pq_utils.h:20-31, seed 1234+m)
  // Each subspace's shuffle has its own generator: a few host threads.
  std::vector<int32_t> init((size_t)pq_m * kPQK);
  {
    const int nt = std::max(1, std::min(pq_m, 8));
    std::vector<std::thread> th;
    for (int t0 = 0; t0 < nt; ++t0)
      th.emplace_back([&, t0] {
        std::vector<int> ind(actual);
        for (int sub = t0; sub < pq_m; sub += nt) {
          std::iota(ind.begin(), ind.end(), 0);
          std::mt19937 rng(1234 + sub);
          std::shuffle(ind.begin(), ind.end(), rng);
          std::copy(ind.begin(), ind.begin() + kPQK, init.begin() + (size_t)sub * kPQK);
        }
      });
    for (auto& t : th) t.join();
  }
  DevBuf<int32_t> drows, dinit, dassign;
  DevBuf<float> res;
  FGPU_TRY(drows.alloc(actual));
  FGPU_TRY(dinit.alloc(init.size()));
  FGPU_TRY(dassign.alloc((size_t)actual * pq_m));
  FGPU_TRY(res.alloc((size_t)actual * dim));
  FGPU_HIP(hipMemcpyAsync(drows.p, idx.data(), sizeof(int32_t) * actual, hipMemcpyHostToDevice, s));
  FGPU_HIP(hipMemcpyAsync(dinit.p, init.data(), sizeof(int32_t) * init.size(), hipMemcpyHostToDevice, s));
  FGPU_TRY(launch_pq_residuals(dx, dim, drows.p, actual, d_assign, d_cent, res.p, s));
  FGPU_TRY(launch_pq_init(res.p, actual, dim, pq_m, dinit.p, d_codebook, s));
  for (int it = 0; it < iters; ++it) {
    FGPU_TRY(launch_pq_estep(res.p, actual, dim, pq_m, d_codebook, dassign.p, s));
    FGPU_TRY(launch_pq_mstep(res.p, actual, dim, pq_m, dassign.p, d_codebook, s));
  }
  FGPU_HIP(hipStreamSynchronize(s));
  return FGPU_OK;
}

fgpu_status fgpu_pq_encode(const float* dx, int64_t n, int dim, int pq_m, const int32_t* d_assign,
                           const float* d_cent, const float* d_codebook, uint8_t* d_codes, void* stream) {
  return fgpu_pq_encode_form(dx, n, dim, pq_m, d_assign, d_cent, d_codebook, 1, d_codes, stream);
}

fgpu_status fgpu_pq_encode_form(const float* dx, int64_t n, int dim, int pq_m, const int32_t* d_assign,
                                const float* d_cent, const float* d_codebook, int fma_mode, uint8_t* d_codes,
                                void* stream) {
  FGPU_CHECK(dx && d_assign && d_cent && d_codebook && d_codes && n >= 0 && pq_m >= 1 && dim % pq_m == 0,
             FGPU_ERR_ARG, "pq_encode: bad argument");
  return launch_pq_encode(dx, n, dim, pq_m, d_assign, d_cent, d_codebook, d_codes, as_stream(stream), fma_mode);
}

fgpu_status fgpu_build_ivfpq(const float* dx, int64_t n, int dim, int nlist, int pq_m, int kmeans_iters, int init_mode,
                             uint64_t seed, int pq_iters, int sample_size, int32_t* h_offsets, int32_t* h_ids,
                             uint8_t* h_codes, float* h_centroids, float* h_codebook, void* stream) {
  return fgpu_build_ivfpq_sampled(dx, n, dim, nlist, pq_m, 0, kmeans_iters, init_mode, seed, pq_iters, sample_size,
                                  h_offsets, h_ids, h_codes, h_centroids, h_codebook, stream);
}

fgpu_status fgpu_build_ivfpq_sampled(const float* dx, int64_t n, int dim, int nlist, int pq_m, int64_t train_rows,
                                     int kmeans_iters, int init_mode, uint64_t seed, int pq_iters, int sample_size,
                                     int32_t* h_offsets, int32_t* h_ids, uint8_t* h_codes, float* h_centroids,
                                     float* h_codebook, void* stream) {
  FGPU_CHECK(dx && h_offsets && h_ids && h_codes && h_centroids && h_codebook, FGPU_ERR_ARG, "build: null argument");
  FGPU_CHECK(n < INT32_MAX, FGPU_ERR_ARG, "build: more than 2^31-1 vectors");
  hipStream_t s = as_stream(stream);
  DevBuf<float> cent, cb;
  DevBuf<int32_t> assign;
  DevBuf<uint8_t> codes;
  FGPU_TRY(cent.alloc((size_t)nlist * dim));
  FGPU_TRY(cb.alloc((size_t)pq_m * kPQK * (dim / pq_m)));
  FGPU_TRY(assign.alloc(n));
  FGPU_TRY(codes.alloc((size_t)n * pq_m));
  if (train_rows <= 0 || train_rows >= n) {
    FGPU_TRY(fgpu_kmeans_fit(dx, n, dim, nlist, kmeans_iters, init_mode, seed, cent.p, assign.p, stream));
  } else {
    FGPU_CHECK(train_rows >= nlist, FGPU_ERR_ARG, "build: train_rows must be >= nlist");
    std::vector<int32_t> rows(train_rows);
    for (int64_t j = 0; j < train_rows; ++j) rows[j] = (int32_t)(j * n / train_rows);
    DevBuf<int32_t> drows;
    DevBuf<float> train, dist;
    DevBuf<char> tws;
    FGPU_TRY(drows.alloc(train_rows));
    FGPU_TRY(train.alloc((size_t)train_rows * dim));
    FGPU_HIP(hipMemcpyAsync(drows.p, rows.data(), sizeof(int32_t) * train_rows, hipMemcpyHostToDevice, s));
    FGPU_TRY(launch_gather_rows(dx, dim, drows.p, (int)train_rows, train.p, s));
    FGPU_TRY(fgpu_kmeans_fit(train.p, train_rows, dim, nlist, kmeans_iters, init_mode, seed, cent.p, nullptr, stream));
    const size_t tb = fgpu_l2_topk_workspace_bytes(n, nlist);
    FGPU_TRY(dist.alloc(n));
    FGPU_TRY(tws.alloc(tb));
    FGPU_TRY(fgpu_l2_topk(dx, n, cent.p, nlist, dim, 1, assign.p, dist.p, tws.p, tb, stream));
    FGPU_HIP(hipStreamSynchronize(s));
  }
  FGPU_TRY(fgpu_pq_train(dx, n, dim, pq_m, assign.p, cent.p, sample_size, pq_iters, cb.p, stream));
  FGPU_TRY(fgpu_pq_encode(dx, n, dim, pq_m, assign.p, cent.p, cb.p, codes.p, stream));
  std::vector<int32_t> ha(n);
  std::vector<uint8_t> hc((size_t)n * pq_m);
  FGPU_HIP(hipMemcpyAsync(ha.data(), assign.p, sizeof(int32_t) * n, hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipMemcpyAsync(hc.data(), codes.p, hc.size(), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipMemcpyAsync(h_centroids, cent.p, sizeof(float) * (size_t)nlist * dim, hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipMemcpyAsync(h_codebook, cb.p, sizeof(float) * (size_t)pq_m * kPQK * (dim / pq_m), hipMemcpyDeviceToHost, s));
  FGPU_HIP(hipStreamSynchronize(s));
  // inverted lists in cluster order, ids ascending inside a list (build_global.cu:225-240)
  std::vector<int64_t> cnt(nlist + 1, 0);
  for (int64_t i = 0; i < n; ++i) cnt[ha[i] + 1]++;
  for (int l = 0; l < nlist; ++l) cnt[l + 1] += cnt[l];
  for (int l = 0; l <= nlist; ++l) h_offsets[l] = (int32_t)cnt[l];
  std::vector<int64_t> pos(cnt.begin(), cnt.end() - 1);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t pp = pos[ha[i]]++;
    h_ids[pp] = (int32_t)i;
    std::memcpy(h_codes + pp * pq_m, hc.data() + i * pq_m, pq_m);
  }
  return FGPU_OK;
}

// ---------------------------------------------------------------------------
fgpu_status fgpu_write_ivf_data(const char* path, int64_t total, int nlist, int pq_m, int dim, const int32_t* offsets,
                                const int32_t* ids, const uint8_t* codes, const float* centroids) {
  FGPU_CHECK(path && offsets && centroids && total >= 0 && total < INT32_MAX, FGPU_ERR_ARG, "write_ivf_data: bad argument");
  std::ofstream f(path, std::ios::binary);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, std::string("cannot create ") + path);
  const int32_t t32 = (int32_t)total, nl = nlist;
  f.write(reinterpret_cast<const char*>(&t32), 4);
  f.write(reinterpret_cast<const char*>(&nl), 4);
  f.write(reinterpret_cast<const char*>(offsets), sizeof(int32_t) * (nlist + 1));
  f.write(reinterpret_cast<const char*>(ids), sizeof(int32_t) * total);
  f.write(reinterpret_cast<const char*>(codes), (size_t)total * pq_m);
  f.write(reinterpret_cast<const char*>(centroids), sizeof(float) * (size_t)nlist * dim);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, "write_ivf_data: write failed");
  return FGPU_OK;
}

fgpu_status fgpu_read_ivf_header(const char* path, int64_t* total, int* nlist) {
  std::ifstream f(path, std::ios::binary);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, std::string("cannot open ") + (path ? path : "(null)"));
  int32_t t = 0, nl = 0;
  f.read(reinterpret_cast<char*>(&t), 4);
  f.read(reinterpret_cast<char*>(&nl), 4);
  FGPU_CHECK(f.good() && t >= 0 && nl > 0, FGPU_ERR_IO, "ivf_data.bin: bad header");
  *total = t;
  *nlist = nl;
  return FGPU_OK;
}

fgpu_status fgpu_read_ivf_data(const char* path, int pq_m, int dim, int32_t* offsets, int32_t* ids, uint8_t* codes,
                               float* centroids) {
  int64_t total = 0;
  int nlist = 0;
  FGPU_TRY(fgpu_read_ivf_header(path, &total, &nlist));
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  const int64_t size = (int64_t)f.tellg();
  const int64_t want = 8 + 4 * (int64_t)(nlist + 1) + 4 * total + total * pq_m + 4 * (int64_t)nlist * dim;
  FGPU_CHECK(size == want, FGPU_ERR_IO,
             "ivf_data.bin: size " + std::to_string(size) + " != expected " + std::to_string(want) +
                 " for the stated dim/pq_m");
  f.seekg(8);
  f.read(reinterpret_cast<char*>(offsets), sizeof(int32_t) * (nlist + 1));
  f.read(reinterpret_cast<char*>(ids), sizeof(int32_t) * total);
  f.read(reinterpret_cast<char*>(codes), (size_t)total * pq_m);
  f.read(reinterpret_cast<char*>(centroids), sizeof(float) * (size_t)nlist * dim);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, "ivf_data.bin: short read");
  return FGPU_OK;
}

fgpu_status fgpu_write_fvecs(const char* path, const float* v, int64_t n, int dim) {
  std::ofstream f(path, std::ios::binary);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, std::string("cannot create ") + path);
  for (int64_t i = 0; i < n; ++i) {
    f.write(reinterpret_cast<const char*>(&dim), 4);
    f.write(reinterpret_cast<const char*>(v + i * dim), sizeof(float) * dim);
  }
  FGPU_CHECK(f.good(), FGPU_ERR_IO, "write_fvecs: write failed");
  return FGPU_OK;
}

fgpu_status fgpu_read_fvecs(const char* path, int dim, int64_t* n, float* out) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, std::string("cannot open ") + (path ? path : "(null)"));
  const int64_t size = (int64_t)f.tellg();
  f.seekg(0);
  int32_t d = 0;
  f.read(reinterpret_cast<char*>(&d), 4);
  FGPU_CHECK(f.good() && d == dim, FGPU_ERR_IO,
             "fvecs dimension mismatch: expected " + std::to_string(dim) + ", got " + std::to_string(d));
  const int64_t rec = 4 + 4 * (int64_t)dim;
  *n = size / rec;
  if (!out) return FGPU_OK;
  f.seekg(0);
  for (int64_t i = 0; i < *n; ++i) {
    f.seekg(4, std::ios::cur);
    f.read(reinterpret_cast<char*>(out + i * dim), sizeof(float) * dim);
  }
  FGPU_CHECK(f.good(), FGPU_ERR_IO, "fvecs: short read");
  return FGPU_OK;
}

fgpu_status fgpu_read_ivecs(const char* path, int* dim, int64_t* n, int32_t* out) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  FGPU_CHECK(f.good(), FGPU_ERR_IO, std::string("cannot open ") + (path ? path : "(null)"));
  const int64_t size = (int64_t)f.tellg();
  f.seekg(0);
  int32_t d = 0;
  f.read(reinterpret_cast<char*>(&d), 4);
  FGPU_CHECK(f.good() && d > 0, FGPU_ERR_IO, "ivecs: bad header");
  *dim = d;
  *n = size / (4 + 4 * (int64_t)d);
  if (!out) return FGPU_OK;
  f.seekg(0);
  for (int64_t i = 0; i < *n; ++i) {
    f.seekg(4, std::ios::cur);
    f.read(reinterpret_cast<char*>(out + i * d), sizeof(int32_t) * d);
  }
  FGPU_CHECK(f.good(), FGPU_ERR_IO, "ivecs: short read");
  return FGPU_OK;
}

// ---------------------------------------------------------------------------
void fgpu_gen_gmm(int64_t n, int dim, int ncomp, double lo, double hi, double sig_lo, double sig_hi, uint64_t seed,
                  int set, float* out, int nthreads) {
  std::vector<double> centre((size_t)ncomp * dim), sigma(ncomp);
  for (int64_t j = 0; j < (int64_t)ncomp * dim; ++j) centre[j] = lo + (hi - lo) * u01(seed, 1, j);
  for (int j = 0; j < ncomp; ++j) sigma[j] = sig_lo + (sig_hi - sig_lo) * u01(seed, 2, j);
  const uint64_t s_lab = 3 + 2 * (uint64_t)set, s_noise = 4 + 2 * (uint64_t)set;
  auto rows = [&](int64_t r0, int64_t r1) {
    for (int64_t i = r0; i < r1; ++i) {
      int lab = (int)(u01(seed, s_lab, i) * ncomp);
      if (lab >= ncomp) lab = ncomp - 1;
      for (int d = 0; d < dim; ++d) {
        const uint64_t e = (uint64_t)i * dim + d;
        const uint64_t pr = e >> 1;
        const double a = u01(seed, s_noise, 2 * pr), b = u01(seed, s_noise, 2 * pr + 1);
        const double rad = std::sqrt(-2.0 * std::log(1.0 - a));
        const double ang = 6.283185307179586476925286766559 * b;
        const double z = (e & 1) ? rad * std::sin(ang) : rad * std::cos(ang);
        out[e] = (float)(centre[(size_t)lab * dim + d] + sigma[lab] * z);
      }
    }
  };
  int nt = nthreads > 0 ? nthreads : (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (n < 4096) nt = 1;
  std::vector<std::thread> th;
  for (int t = 0; t < nt; ++t) th.emplace_back(rows, n * t / nt, n * (t + 1) / nt);
  for (auto& x : th) x.join();
}

}  // extern "C"
