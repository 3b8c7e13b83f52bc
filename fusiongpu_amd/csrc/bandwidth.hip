// bandwidth.hip -- a streaming read and a random-row gather of device memory,
// to measure the HBM read rates the roofline figures are set against (no
// reference counterpart).
#include "common.hpp"
#include "kernels.hpp"

namespace fgpu {
namespace {

// Grid-stride 16-byte loads, four independent ones in flight per lane; the
// XOR of everything read goes to one sink slot per workgroup.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ d, size_t n16,
                                                          unsigned long long* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = d[i], b = d[i + stride], c = d[i + 2 * stride], e = d[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ e.x ^ e.y ^ e.z ^ e.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = d[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] ^= red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0];
}

// Random rows: n whole rows idx[i], LPR lanes a row.  With LPR = 1 each lane
// reads its own row (RB 16-byte loads, all issued before any is used), so a
// load instruction touches 64 rows; with LPR = 8 eight lanes share a row, each
// 16 bytes of every 128-byte line, so an instruction touches 8 rows.  The
// exact rerank and the graph search load their candidate rows the second way
// (wave_rows_l2).
template <int RB, int LPR>
__global__ __launch_bounds__(256) void row_gather_kernel(const uint4* __restrict__ d, int64_t nrows,
                                                         const int32_t* __restrict__ idx, int64_t n,
                                                         unsigned long long* __restrict__ sink) {
  static_assert(RB % LPR == 0, "a row splits evenly over its lanes");
  constexpr int kRowsPerGroup = 256 / LPR;
  const int sub = (int)threadIdx.x % LPR;
  uint32_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * kRowsPerGroup + threadIdx.x / LPR; i < n;
       i += (int64_t)gridDim.x * kRowsPerGroup) {
    const int64_t r = min(max((int64_t)idx[i], (int64_t)0), nrows - 1);  // out-of-range ids read a valid row
    const uint4* row = d + r * RB + sub;
    uint4 v[RB / LPR];
#pragma unroll
    for (int j = 0; j < RB / LPR; ++j) v[j] = row[LPR * j];
#pragma unroll
    for (int j = 0; j < RB / LPR; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] ^= red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0];
}

template <int RB>
void launch_gather_rb(int lanes, const uint4* p, int64_t nrows, const int32_t* idx, int64_t n,
                      unsigned long long* sink, int grid, hipStream_t s) {
  if (lanes == 1)
    hipLaunchKernelGGL((row_gather_kernel<RB, 1>), dim3((unsigned)grid), dim3(256), 0, s, p, nrows, idx, n, sink);
  else
    hipLaunchKernelGGL((row_gather_kernel<RB, 8>), dim3((unsigned)grid), dim3(256), 0, s, p, nrows, idx, n, sink);
}

}  // namespace

fgpu_status launch_row_gather(const void* d, int64_t nrows, int row_bytes, const int32_t* idx, int64_t n,
                              int lanes_per_row, unsigned long long* sink, int grid, hipStream_t s) {
  FGPU_CHECK(lanes_per_row == 1 || lanes_per_row == 8, FGPU_ERR_UNSUPPORTED, "row_gather: lanes_per_row must be 1 or 8");
  FGPU_CHECK(row_bytes == 384 || row_bytes == 512, FGPU_ERR_UNSUPPORTED, "row_gather: row_bytes must be 384 or 512");
  if (n <= 0 || nrows <= 0 || grid <= 0) return FGPU_OK;
  const uint4* p = reinterpret_cast<const uint4*>(d);
  if (row_bytes == 384)
    launch_gather_rb<24>(lanes_per_row, p, nrows, idx, n, sink, grid, s);
  else
    launch_gather_rb<32>(lanes_per_row, p, nrows, idx, n, sink, grid, s);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_stream_read(const void* d, size_t bytes, unsigned long long* sink, int grid, hipStream_t s) {
  if (bytes == 0 || grid <= 0) return FGPU_OK;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(256), 0, s, reinterpret_cast<const uint4*>(d),
                     bytes / 16, sink);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace fgpu
