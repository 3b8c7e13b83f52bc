// noalloc.hip -- fgpu_search_noalloc: the plain search (fgpu_search) for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).  Its scratch -- the
// probe ids and distances, the query norms and the coarse step's estimate
// tile -- lives in one file-scope device array instead of a caller workspace.
//
// Each GPU holds its own copy of the array from module load until the process
// ends.  Host code never passes the array's name to a kernel or a copy: the
// host-side symbol is only a stand-in.  Index creation (with the device
// current) asks the runtime for the array's device address once per device
// and keeps it; every use goes through that address, so a call made under
// graph capture does no lookup of its own.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one
// GPU (different streams, or host threads) race on it.  Nothing in the array
// needs clearing between calls: each stage writes all of its part before the
// next reads it.
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {
namespace {

constexpr size_t kScratchBytes = FGPU_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of this device's scratch array (looked up once per device).
fgpu_status scratch_address(void** out) {
  int dev = -1;
  FGPU_HIP(hipGetDevice(&dev));
  FGPU_CHECK(dev >= 0 && dev < kMaxDevices, FGPU_ERR_UNSUPPORTED, "search_noalloc: device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    FGPU_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    FGPU_CHECK(p != nullptr, FGPU_ERR_HIP, "search_noalloc: no device address for the scratch array");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return FGPU_OK;
}

}  // namespace

fgpu_status noalloc_prepare() {
  void* p = nullptr;
  return scratch_address(&p);
}

}  // namespace fgpu

using namespace fgpu;

extern "C" {

size_t fgpu_search_noalloc_max_bytes(void) { return kScratchBytes; }

int fgpu_search_noalloc_max_rows(int nlist, int nprobe) {
  if (nlist < 1 || nprobe < 1) return 0;
  // Largest multiple of 64 query rows whose whole fgpu_search workspace fits
  // (the screen path included); when not even 64 rows of that fit, the
  // largest whose LUT-path workspace fits (fgpu_search then takes the LUT
  // flow kernel, whose results are the same).
  auto max_rows = [&](size_t (*need)(int, int, int)) {
    int lo = 0, hi = 1 << 20;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (need(mid * 64, nlist, nprobe) <= kScratchBytes)
        lo = mid;
      else
        hi = mid - 1;
    }
    return lo * 64;
  };
  const int full = max_rows(fgpu_search_workspace_bytes);
  return full >= 64 ? full : max_rows(search_lut_workspace_bytes);
}

fgpu_status fgpu_search_noalloc(const fgpu_index* ix, const float* dq, int nq, int nprobe, int k, float prune_ratio,
                                int32_t* d_out_ids, float* d_out_dists, void* stream) {
  FGPU_CHECK(ix && dq && d_out_ids && d_out_dists, FGPU_ERR_ARG, "search_noalloc: null argument");
  FGPU_CHECK(nq >= 0 && nprobe >= 1 && k >= 1, FGPU_ERR_ARG, "search_noalloc: bad sizes");
  fgpu_index_info info;
  FGPU_TRY(fgpu_index_get_info(ix, &info));
  const int rows = fgpu_search_noalloc_max_rows(info.nlist, nprobe);
  FGPU_CHECK(rows >= 64, FGPU_ERR_WORKSPACE,
             "search_noalloc: 64 query rows of scratch for nlist " + std::to_string(info.nlist) + ", nprobe " +
                 std::to_string(nprobe) + " need " + std::to_string(search_lut_workspace_bytes(64, info.nlist, nprobe)) +
                 " bytes, more than the " + std::to_string(kScratchBytes) + "-byte scratch array");
  if (nq == 0) return FGPU_OK;
  void* ws = nullptr;
  FGPU_TRY(scratch_address(&ws));
  // Query chunks that fit the array; each chunk is an ordinary fgpu_search
  // (coarse + scan) on the scratch array, so results equal fgpu_search's.
  for (int q0 = 0; q0 < nq; q0 += rows) {
    const int nb = std::min(rows, nq - q0);
    FGPU_TRY(fgpu_search(ix, dq + (size_t)q0 * info.dim, nb, nprobe, k, prune_ratio, d_out_ids + (size_t)q0 * k,
                         d_out_dists + (size_t)q0 * k, ws, kScratchBytes, stream));
  }
  return FGPU_OK;
}

}  // extern "C"
