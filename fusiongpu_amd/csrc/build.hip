// build.hip -- index-build kernels: probe counts (A3), k-means update (A14),
// PQ encoding (A16), PQ codebook training (A15), k-means++ seeding.
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>

namespace fgpu {
namespace {

// ---- A3: probe counts + exclusive scan (gpu_global.cu:31-77, 704-723) -----
__global__ void probe_counts_kernel(const uint32_t* __restrict__ probes, int nq, int nprobe, int nlist,
                                    const int32_t* __restrict__ offsets, int32_t* __restrict__ counts) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= nq) return;
  int c = 0;
  for (int p = 0; p < nprobe; ++p) {
    const uint32_t l = probes[(size_t)q * nprobe + p];
    if (l < (uint32_t)nlist) c += offsets[l + 1] - offsets[l];  // pruned ids are >= nlist
  }
  counts[q] = c;
}

// Single-workgroup exclusive scan; out[n] = total.
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(const int32_t* __restrict__ in, int n,
                                                               int32_t* __restrict__ out) {
  __shared__ int32_t part[16];
  __shared__ int32_t carry;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < n; base += 1024) {
    const int i = base + threadIdx.x;
    const int32_t v = i < n ? in[i] : 0;
    int32_t inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      int32_t t = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += t;
    }
    if (lane == 63) part[wave] = inc;
    __syncthreads();
    int32_t wbase = 0;
    for (int w = 0; w < wave; ++w) wbase += part[w];
    const int32_t c0 = carry;
    if (i < n) out[i] = c0 + wbase + inc - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry = c0 + wbase + inc;
    __syncthreads();
  }
  if (threadIdx.x == 0) out[n] = carry;
}

// ---- helpers ------------------------------------------------------------------
__global__ void maxabs_partial_kernel(const float* __restrict__ x, int64_t count, float* __restrict__ part) {
  float m = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    m = fmaxf(m, fabsf(x[i]));
  __shared__ float s[4];
  m = wave_max_f(m);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
}

__global__ void fill_u64_kernel(unsigned long long* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0ull;
}
__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ void gather_rows_kernel(const float* __restrict__ x, int dim, const int32_t* __restrict__ rows,
                                   int nrows, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)nrows * dim) return;
  const int r = (int)(t / dim), d = (int)(t % dim);
  out[t] = x[(int64_t)rows[r] * dim + d];
}

// ---- A14: deterministic Lloyd update ------------------------------------------
// Sums of round(x * 2^shift) in int64 (two's complement through unsigned
// atomics): integer addition is associative, so the result does not depend on
// the order the atomics land, unlike the reference's float atomicAdd
// (kmeans_gpu.cuh:94-97).
__global__ __launch_bounds__(256) void kmeans_accumulate_kernel(
    const float* __restrict__ x, int64_t n, const int32_t* __restrict__ assign, int dim, int shift,
    unsigned long long* __restrict__ sums, int32_t* __restrict__ counts) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * dim) return;
  const int64_t i = t / dim;
  const int d = (int)(t % dim);
  const int c = assign[i];
  const long long q = __float2ll_rn(ldexpf(x[t], shift));
  atomicAdd(&sums[(int64_t)c * dim + d], (unsigned long long)q);
  if (d == 0) atomicAdd(&counts[c], 1);
}

__global__ void kmeans_finalize_kernel(const unsigned long long* __restrict__ sums,
                                       const int32_t* __restrict__ counts, int k, int dim, int shift,
                                       int empty_rule, float* __restrict__ cent) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)k * dim) return;
  const int c = (int)(t / dim);
  const int cnt = counts[c];
  if (cnt == 0) {
    if (empty_rule == 0) cent[t] = 0.0f;
    return;
  }
  const float inv = __fdiv_rn(1.0f, (float)cnt);
  const float s = (float)ldexp((double)(long long)sums[t], -shift);
  cent[t] = __fmul_rn(s, inv);
}

// ---- A16: residual PQ encoding (kmeans_gpu.cuh:403-445) ---------------------------
// Codebook staged in LDS as [k][m][S] so lanes of one wave (consecutive
// subspaces, same codeword) read consecutive 16-byte chunks.  FMA: the device
// form, dist = fmaf(diff, diff, dist) as nvcc contracts encode_residuals_kernel
// (kmeans_gpu.cuh:428-433); otherwise the host form of encode_residuals_to_pq
// (pq_utils.h:160-166, built without FMA): the product and the sum each rounded.
template <int S, bool FMA>
__global__ __launch_bounds__(1024) void pq_encode_kernel(const float* __restrict__ x, int64_t n, int dim, int m,
                                                         const int32_t* __restrict__ assign,
                                                         const float* __restrict__ cent,
                                                         const float* __restrict__ codebook,
                                                         uint8_t* __restrict__ codes) {
  extern __shared__ __align__(16) float cbs[];  // [256][m][S]
  for (int t = threadIdx.x; t < kPQK * m * S; t += blockDim.x) {
    const int j = t % S, sub = (t / S) % m, kk = t / (S * m);
    cbs[t] = codebook[((size_t)sub * kPQK + kk) * S + j];
  }
  __syncthreads();
  const int64_t total = n * m;
  for (int64_t pr = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; pr < total; pr += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = pr / m;
    const int sub = (int)(pr % m);
    const float* xi = x + i * dim + sub * S;
    const float* ci = cent + (int64_t)assign[i] * dim + sub * S;
    float r[S];
#pragma unroll
    for (int j = 0; j < S; ++j) r[j] = xi[j] - ci[j];
    float best = FLT_MAX;
    int bk = 0;
    for (int kk = 0; kk < kPQK; ++kk) {
      const float* p = cbs + ((size_t)kk * m + sub) * S;
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const float df = r[j] - p[j];
        d = FMA ? __builtin_fmaf(df, df, d) : __fadd_rn(d, __fmul_rn(df, df));
      }
      if (d < best) { best = d; bk = kk; }
    }
    codes[pr] = (uint8_t)bk;
  }
}

// ---- A15: PQ codebook training (pq_utils.h:17-138) ------------------------------
__global__ void pq_residuals_kernel(const float* __restrict__ x, int dim, const int32_t* __restrict__ rows,
                                    int nrows, const int32_t* __restrict__ assign,
                                    const float* __restrict__ cent, float* __restrict__ res) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)nrows * dim) return;
  const int r = (int)(t / dim), d = (int)(t % dim);
  const int64_t o = rows[r];
  res[t] = x[o * dim + d] - cent[(int64_t)assign[o] * dim + d];
}

// codebook[m][c][j] = res[init_rows[m][c]][m*S + j]
__global__ void pq_init_kernel(const float* __restrict__ res, int dim, int m, int S,
                               const int32_t* __restrict__ init_rows, float* __restrict__ codebook) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= m * kPQK * S) return;
  const int j = t % S, c = (t / S) % kPQK, sub = t / (S * kPQK);
  codebook[t] = res[(int64_t)init_rows[sub * kPQK + c] * dim + sub * S + j];
}

// E-step of run_kmeans_pq_fast (pq_utils.h:39-52), host floating point: the
// square and the running sum are rounded separately (no fused multiply-add).
template <int S>
__global__ __launch_bounds__(256) void pq_estep_kernel(const float* __restrict__ res, int ns, int dim, int m,
                                                       const float* __restrict__ codebook,
                                                       int32_t* __restrict__ assign_pq) {
  __shared__ float cbs[kPQK * S];
  const int sub = blockIdx.y;
  for (int t = threadIdx.x; t < kPQK * S; t += blockDim.x) cbs[t] = codebook[(size_t)sub * kPQK * S + t];
  __syncthreads();
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ns) return;
  float xv[S];
#pragma unroll
  for (int j = 0; j < S; ++j) xv[j] = res[(int64_t)i * dim + sub * S + j];
  float best = FLT_MAX;
  int bc = 0;
  for (int c = 0; c < kPQK; ++c) {
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const float df = xv[j] - cbs[c * S + j];
      d = __fadd_rn(d, __fmul_rn(df, df));
    }
    if (d < best) { best = d; bc = c; }
  }
  assign_pq[(int64_t)sub * ns + i] = bc;
}

// M-step (pq_utils.h:54-71): members of cluster c summed in double in
// ascending row order, (float)(sum / count); an empty cluster keeps its
// centre.  One wave per (cluster, subspace); lanes j < S own dimension j.
__global__ __launch_bounds__(64) void pq_mstep_kernel(const float* __restrict__ res, int ns, int dim, int m, int S,
                                                      const int32_t* __restrict__ assign_pq,
                                                      float* __restrict__ codebook) {
  const int c = blockIdx.x, sub = blockIdx.y, lane = threadIdx.x;
  const int32_t* as = assign_pq + (int64_t)sub * ns;
  double acc = 0.0;
  int cnt = 0;
  for (int base = 0; base < ns; base += kWave) {
    const int i = base + lane;
    const bool hit = i < ns && as[i] == c;
    uint64_t bm = __ballot(hit);
    while (bm) {
      const int b = __ffsll((unsigned long long)bm) - 1;
      bm &= bm - 1;
      if (lane < S) acc += (double)res[(int64_t)(base + b) * dim + sub * S + lane];
      ++cnt;
    }
  }
  if (lane < S && cnt > 0) codebook[((size_t)sub * kPQK + c) * S + lane] = (float)(acc / (double)cnt);
}

// ---- k-means++ seeding (definition: oracle.cpp orc_kmeans_init_pp) ---------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

constexpr int kPPBlock = 1024;

// The exact skip of the d2 update.  asg[i] is the centre whose distance d2[i]
// holds, cc[a] = ||c_new - c_a||^2 for every earlier centre a.  By the
// triangle inequality ||x - c_new|| >= ||c_new - c_a|| - ||x - c_a||, so with
// cc >= 4 (1 + 1%) d2 the new distance exceeds d2 by about 2% even after the
// roundings of the three fused chains (each within 1e-4 relative of its exact
// value, D <= 256): the row cannot move, and its d2, weight and asg stay as
// they are without reading the row.  d2 = 0 rows never move either.  The
// 1e-4 bound is relative and needs values far above the fp32 subnormal range
// (where a rounding step is absolute), so rows with 0 < d2 < 2^-100 always
// compute; from d2 >= 2^-100 on, cc >= 4 d2 is as far above it.
constexpr float kPPSkip = 4.04f;
constexpr float kPPSkipMin = 0x1p-100f;

// Whether row i must compute its distance to the new centre (always, when
// asg is null: the first passes).
__device__ __forceinline__ bool pp_needs(const int32_t* asg, const float* cc, int64_t i, float old) {
  if (asg == nullptr) return true;
  if (old == 0.0f) return false;
  return !(old >= kPPSkipMin && cc[asg[i]] >= kPPSkip * old);
}

// d2[i] = min(d2[i], ||x_i - c||^2) (init: d2 = dist); w[i] = round(d2 * 2^S);
// part[b] = sum of w over block b.  With asg: rows the triangle bound clears
// are skipped, and a row that moves records centre j.
__global__ __launch_bounds__(kPPBlock) void pp_update_kernel(const float* __restrict__ x, int64_t n, int dim,
                                                             const float* __restrict__ c, int init,
                                                             float* __restrict__ d2, const int* __restrict__ shift,
                                                             uint64_t* __restrict__ w, uint64_t* __restrict__ part,
                                                             int32_t* __restrict__ asg, const float* __restrict__ cc,
                                                             int j) {
  const int64_t i = (int64_t)blockIdx.x * kPPBlock + threadIdx.x;
  uint64_t wi = 0;
  if (i < n) {
    const float old = init ? 0.0f : d2[i];
    float v = old;
    bool moved = false;
    if (init || pp_needs(init ? nullptr : asg, cc, i, old)) {
      const float* xi = x + i * dim;
      float acc = 0.0f;
      for (int d = 0; d < dim; ++d) {
        const float df = xi[d] - c[d];
        acc = __builtin_fmaf(df, df, acc);
      }
      moved = init || acc < old;
      v = moved ? acc : old;
    }
    if (moved) {
      d2[i] = v;
      if (asg) asg[i] = j;
    }
    if (shift) {
      wi = (uint64_t)__double2ll_rn(ldexp((double)v, *shift));
      if (moved || !asg) w[i] = wi;
    }
  }
  if (shift) {
    __shared__ uint64_t s[kPPBlock / kWave];
    uint64_t t = wi;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) t += __shfl_xor(t, m, kWave);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t tot = 0;
      for (int j = 0; j < kPPBlock / kWave; ++j) tot += s[j];
      part[blockIdx.x] = tot;
    }
  }
}

// The same update for a compile-time dim: each lane still owns one row and
// keeps the sequential fused chain, but the row arrives as D/4 16-byte loads
// that are all issued before the chain starts, instead of D dependent scalar
// loads.
template <int D>
__global__ __launch_bounds__(kPPBlock) void pp_update_vec_kernel(const float* __restrict__ x, int64_t n,
                                                                 const float* __restrict__ c, int init,
                                                                 float* __restrict__ d2, const int* __restrict__ shift,
                                                                 uint64_t* __restrict__ w, uint64_t* __restrict__ part,
                                                                 int32_t* __restrict__ asg,
                                                                 const float* __restrict__ cc, int jc) {
  static_assert(D % 4 == 0, "16-byte row loads");
  __shared__ float cs[D];
  for (int d = threadIdx.x; d < D; d += kPPBlock) cs[d] = c[d];
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * kPPBlock + threadIdx.x;
  uint64_t wi = 0;
  if (i < n) {
    const float old = init ? 0.0f : d2[i];
    float v2 = old;
    bool moved = false;
    if (init || pp_needs(init ? nullptr : asg, cc, i, old)) {
      const float4* xi = reinterpret_cast<const float4*>(x + i * D);
      float4 v[D / 4];
#pragma unroll
      for (int j = 0; j < D / 4; ++j) v[j] = xi[j];
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < D / 4; ++j) {
        float df = v[j].x - cs[4 * j];
        acc = __builtin_fmaf(df, df, acc);
        df = v[j].y - cs[4 * j + 1];
        acc = __builtin_fmaf(df, df, acc);
        df = v[j].z - cs[4 * j + 2];
        acc = __builtin_fmaf(df, df, acc);
        df = v[j].w - cs[4 * j + 3];
        acc = __builtin_fmaf(df, df, acc);
      }
      moved = init || acc < old;
      v2 = moved ? acc : old;
    }
    if (moved) {
      d2[i] = v2;
      if (asg) asg[i] = jc;
    }
    if (shift) {
      wi = (uint64_t)__double2ll_rn(ldexp((double)v2, *shift));
      if (moved || !asg) w[i] = wi;
    }
  }
  if (shift) {
    __shared__ uint64_t s[kPPBlock / kWave];
    uint64_t t = wi;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) t += __shfl_xor(t, m, kWave);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t tot = 0;
      for (int j = 0; j < kPPBlock / kWave; ++j) tot += s[j];
      part[blockIdx.x] = tot;
    }
  }
}

// One pass of the d2 update: the vectorised kernel for the common dims (rows
// 16-byte aligned), the generic one otherwise.
// asg == nullptr: every row computes (the first passes); otherwise the skip
// above applies (cc filled for centre j).
fgpu_status pp_update(const float* x, int64_t n, int dim, const float* c, int init, float* d2, const int* shift,
                      uint64_t* w, uint64_t* part, int nb, int32_t* asg, const float* cc, int j, hipStream_t s) {
  const bool vec = ((uintptr_t)x & 15) == 0;
  if (vec && dim == 128)
    hipLaunchKernelGGL(pp_update_vec_kernel<128>, dim3(nb), dim3(kPPBlock), 0, s, x, n, c, init, d2, shift, w, part,
                       asg, cc, j);
  else if (vec && dim == 96)
    hipLaunchKernelGGL(pp_update_vec_kernel<96>, dim3(nb), dim3(kPPBlock), 0, s, x, n, c, init, d2, shift, w, part,
                       asg, cc, j);
  else if (vec && dim == 64)
    hipLaunchKernelGGL(pp_update_vec_kernel<64>, dim3(nb), dim3(kPPBlock), 0, s, x, n, c, init, d2, shift, w, part,
                       asg, cc, j);
  else
    hipLaunchKernelGGL(pp_update_kernel, dim3(nb), dim3(kPPBlock), 0, s, x, n, dim, c, init, d2, shift, w, part, asg,
                       cc, j);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

// shift from the first round's max d2 (so n * max w < 2^62).
__global__ __launch_bounds__(1024) void pp_shift_kernel(const float* __restrict__ d2, int64_t n, int* __restrict__ shift) {
  __shared__ float part[16];
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, d2[i]);
  m = wave_max_f(m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float mx = 0.0f;
    for (int j = 0; j < 16; ++j) mx = fmaxf(mx, part[j]);
    int e = 0;
    if (mx > 0.0f) frexp((double)mx, &e);
    int lg = 0;
    while ((1LL << lg) < n) ++lg;
    int s = 62 - lg - e;
    *shift = s > 60 ? 60 : (s < 0 ? 0 : s);
  }
}

// Pick the next centre: smallest i with inclusive prefix(w) > u, u = r_j % total.
// One workgroup; state[0] = chosen row.  chosen[] marks picked rows for the
// all-zero fallback.
// Then (cent != nullptr) take the picked row as centre j.
__global__ __launch_bounds__(1024) void pp_pick_kernel(const uint64_t* __restrict__ w, const uint64_t* __restrict__ part,
                                                       int nblocks, int64_t n, uint64_t seed, int j,
                                                       uint8_t* __restrict__ chosen, int32_t* __restrict__ rows,
                                                       const float* __restrict__ x, int dim, float* __restrict__ cent) {
  __shared__ uint64_t s_tot;
  __shared__ uint64_t s_u;
  __shared__ int64_t s_pick;
  __shared__ uint64_t s_before;
  __shared__ int s_blk;
  const int tid = threadIdx.x;
  // Total and the block holding u: chunked parallel scan over the block sums.
  __shared__ uint64_t sc[kPPBlock];
  if (tid == 0) { s_tot = 0; s_blk = -1; s_pick = -1; s_before = 0; }
  __syncthreads();
  for (int base = 0; base < nblocks; base += kPPBlock) {
    const uint64_t v = base + tid < nblocks ? part[base + tid] : 0;
    sc[tid] = v;
    __syncthreads();
    for (int o = 1; o < kPPBlock; o <<= 1) {
      const uint64_t t = tid >= o ? sc[tid - o] : 0;
      __syncthreads();
      sc[tid] += t;
      __syncthreads();
    }
    if (tid == kPPBlock - 1) s_before = s_tot;  // running total before this chunk
    __syncthreads();
    const uint64_t chunk_before = s_before;
    __syncthreads();
    if (tid == kPPBlock - 1) s_tot = chunk_before + sc[tid];
    __syncthreads();
  }
  if (tid == 0 && s_tot != 0) s_u = mix64(seed ^ mix64(7) ^ mix64(0x100000000ull + (uint64_t)j)) % s_tot;
  __syncthreads();
  if (s_tot != 0) {
    uint64_t acc = 0;
    for (int base = 0; base < nblocks; base += kPPBlock) {
      const uint64_t v = base + tid < nblocks ? part[base + tid] : 0;
      sc[tid] = v;
      __syncthreads();
      for (int o = 1; o < kPPBlock; o <<= 1) {
        const uint64_t t = tid >= o ? sc[tid - o] : 0;
        __syncthreads();
        sc[tid] += t;
        __syncthreads();
      }
      const uint64_t incl = acc + sc[tid], excl = incl - v;
      if (base + tid < nblocks && excl <= s_u && s_u < incl) { s_blk = base + tid; s_before = excl; }
      acc += sc[kPPBlock - 1];
      __syncthreads();
    }
  }
  __syncthreads();
  if (tid == 0 && s_blk < 0) { s_blk = 0; s_before = 0; }  // unreachable when u < total; keeps indices in range
  __syncthreads();
  if (s_tot == 0) {
    if (tid == 0) {
      int64_t pick = 0;
      for (int64_t i = 0; i < n; ++i)
        if (!chosen[i]) { pick = i; break; }
      s_pick = pick;
    }
  } else {
    // Inside the block: inclusive scan of its 1024 weights.
    const int64_t i = (int64_t)s_blk * kPPBlock + tid;
    const uint64_t wi = i < n ? w[i] : 0;
    sc[tid] = wi;
    __syncthreads();
    for (int o = 1; o < kPPBlock; o <<= 1) {
      uint64_t t = tid >= o ? sc[tid - o] : 0;
      __syncthreads();
      sc[tid] += t;
      __syncthreads();
    }
    const uint64_t incl = s_before + sc[tid];
    const uint64_t excl = incl - wi;
    if (i < n && excl <= s_u && s_u < incl) s_pick = i;
    __syncthreads();
    // s_u lies inside block s_blk by construction; the fallback only keeps the row in range.
    if (tid == 0 && s_pick < 0) s_pick = (int64_t)s_blk * kPPBlock;
  }
  __syncthreads();
  const int64_t r = s_pick;
  if (tid == 0) rows[j] = (int32_t)r;
  if (!cent) return;
  for (int d = tid; d < dim; d += kPPBlock) cent[(int64_t)j * dim + d] = x[r * dim + d];
  if (tid == 0) chosen[r] = 1;
}

// cc[a] = ||c_j - c_a||^2 for every earlier centre a < j: one wave per centre,
// lanes over dimensions.  Only the skip bound reads cc, and that bound holds
// for any summation order.
__global__ __launch_bounds__(256) void pp_cc_kernel(const float* __restrict__ cent, int dim, int j,
                                                    float* __restrict__ cc) {
  const int a = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (a >= j) return;
  const float* cj = cent + (size_t)j * dim;
  const float* ca = cent + (size_t)a * dim;
  float acc = 0.0f;
  for (int d = lane; d < dim; d += 64) {
    const float df = cj[d] - ca[d];
    acc = __builtin_fmaf(df, df, acc);
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) acc += shfl_xor_f(acc, m);
  if (lane == 0) cc[a] = acc;
}

__global__ void pp_take_kernel(const float* __restrict__ x, int dim, const int32_t* __restrict__ rows, int j,
                               float* __restrict__ cent, uint8_t* __restrict__ chosen) {
  const int r = rows[j];
  for (int d = threadIdx.x; d < dim; d += blockDim.x) cent[(int64_t)j * dim + d] = x[(int64_t)r * dim + d];
  if (threadIdx.x == 0) chosen[r] = 1;
}

__global__ void pp_first_kernel(int64_t n, uint64_t seed, int32_t* __restrict__ rows, uint8_t* __restrict__ chosen) {
  const int64_t r0 = (int64_t)(mix64(seed ^ mix64(7)) % (uint64_t)n);
  rows[0] = (int32_t)r0;
  (void)chosen;
}

template <class K, class... A>
fgpu_status launch1d(K kern, int64_t n, int block, hipStream_t s, A... args) {
  if (n <= 0) return FGPU_OK;
  hipLaunchKernelGGL(kern, dim3((unsigned)((n + block - 1) / block)), dim3(block), 0, s, args...);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

// ---------------------------------------------------------------------------
// Per-list radius of the decoded residuals: rmax[l] >= ||decode(x)|| for every
// vector x of list l, where decode(x)_m = codebook[m][code_m].  Squared
// codeword norms and their sums are formed in double (each product of two
// floats is exact in double; the few roundings of the sums are far below the
// final margin), and the float result is rounded up.  One block per list.
__global__ __launch_bounds__(256) void list_radius_kernel(const float* __restrict__ cb, int m, int sub,
                                                          const uint8_t* __restrict__ codes,
                                                          const int32_t* __restrict__ offsets,
                                                          float* __restrict__ rmax) {
  extern __shared__ double cbn2[];  // [m][256]
  for (int i = threadIdx.x; i < m * kPQK; i += blockDim.x) {
    double t = 0.0;
    for (int d = 0; d < sub; ++d) {
      const double v = cb[(size_t)i * sub + d];
      t += v * v;
    }
    cbn2[i] = t;
  }
  __syncthreads();
  const int l = blockIdx.x;
  const int start = offsets[l], end = offsets[l + 1];
  double mx = 0.0;
  for (int v = start + threadIdx.x; v < end; v += blockDim.x) {
    const uint8_t* c = codes + (size_t)v * m;
    double t = 0.0;
    for (int j = 0; j < m; ++j) t += cbn2[j * kPQK + c[j]];
    mx = fmax(mx, t);
  }
  __shared__ double red[256];
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  if (threadIdx.x == 0) rmax[l] = __double2float_ru(sqrt(red[0]) * (1.0 + 0x1p-30));
}

}  // namespace

fgpu_status launch_probe_counts(const uint32_t* probes, int nq, int nprobe, int nlist, const int32_t* offsets,
                                int32_t* counts, int32_t* offs, hipStream_t s) {
  FGPU_TRY(launch1d(probe_counts_kernel, nq, 256, s, probes, nq, nprobe, nlist, offsets, counts));
  hipLaunchKernelGGL(exclusive_scan_kernel, dim3(1), dim3(1024), 0, s, counts, nq, offs);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_maxabs(const float* x, int64_t count, float* out, hipStream_t s) {
  // out must hold 1024 floats of scratch; the result lands in out[1023].
  hipLaunchKernelGGL(maxabs_partial_kernel, dim3(1023), dim3(256), 0, s, x, count, out);
  FGPU_HIP(hipGetLastError());
  return launch_max_reduce(out, 1023, out + 1023, s);
}

fgpu_status launch_kmeans_accumulate(const float* x, int64_t n, const int32_t* assign, int k, int dim, int shift,
                                     unsigned long long* sums, int32_t* counts, hipStream_t s) {
  FGPU_TRY(launch1d(fill_u64_kernel, (int64_t)k * dim, 256, s, sums, (int64_t)k * dim));
  FGPU_TRY(launch1d(fill_i32_kernel, (int64_t)k, 256, s, counts, (int64_t)k));
  return launch1d(kmeans_accumulate_kernel, n * dim, 256, s, x, n, assign, dim, shift, sums, counts);
}

fgpu_status launch_kmeans_finalize(const unsigned long long* sums, const int32_t* counts, int k, int dim, int shift,
                                   int empty_rule, float* cent, hipStream_t s) {
  return launch1d(kmeans_finalize_kernel, (int64_t)k * dim, 256, s, sums, counts, k, dim, shift, empty_rule, cent);
}

fgpu_status launch_gather_rows(const float* x, int dim, const int32_t* rows, int nrows, float* out, hipStream_t s) {
  return launch1d(gather_rows_kernel, (int64_t)nrows * dim, 256, s, x, dim, rows, nrows, out);
}

fgpu_status launch_pq_encode(const float* x, int64_t n, int dim, int m, const int32_t* assign, const float* cent,
                             const float* codebook, uint8_t* codes, hipStream_t s, int fma_mode) {
  const int S = dim / m;
  const size_t lds = (size_t)kPQK * dim * sizeof(float);
  FGPU_CHECK(lds <= 160 * 1024, FGPU_ERR_UNSUPPORTED, "pq_encode: codebook exceeds LDS");
  if (n <= 0) return FGPU_OK;
  const int64_t pairs = n * m;
  const unsigned grid = (unsigned)std::min<int64_t>((pairs + 1023) / 1024, 256 * 8);
#define FGPU_ENC(SS, F)                                                                                       \
  if (S == SS && (fma_mode != 0) == F) {                                                                      \
    FGPU_HIP(hipFuncSetAttribute((const void*)pq_encode_kernel<SS, F>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                 (int)lds));                                                                  \
    hipLaunchKernelGGL((pq_encode_kernel<SS, F>), dim3(grid), dim3(1024), lds, s, x, n, dim, m, assign, cent, codebook, \
                       codes);                                                                                \
    FGPU_HIP(hipGetLastError());                                                                              \
    return FGPU_OK;                                                                                           \
  }
  FGPU_ENC(1, true) FGPU_ENC(2, true) FGPU_ENC(3, true) FGPU_ENC(4, true) FGPU_ENC(6, true) FGPU_ENC(8, true)
  FGPU_ENC(16, true)
  FGPU_ENC(1, false) FGPU_ENC(2, false) FGPU_ENC(3, false) FGPU_ENC(4, false) FGPU_ENC(6, false) FGPU_ENC(8, false)
  FGPU_ENC(16, false)
#undef FGPU_ENC
  return set_error(FGPU_ERR_UNSUPPORTED, "pq_encode: unsupported sub-dimension");
}

fgpu_status launch_pq_residuals(const float* x, int dim, const int32_t* rows, int nrows, const int32_t* assign,
                                const float* cent, float* res, hipStream_t s) {
  return launch1d(pq_residuals_kernel, (int64_t)nrows * dim, 256, s, x, dim, rows, nrows, assign, cent, res);
}

fgpu_status launch_pq_init(const float* res, int nsample, int dim, int m, const int32_t* init_rows, float* codebook,
                           hipStream_t s) {
  (void)nsample;
  const int S = dim / m;
  return launch1d(pq_init_kernel, (int64_t)m * kPQK * S, 256, s, res, dim, m, S, init_rows, codebook);
}

fgpu_status launch_pq_estep(const float* res, int ns, int dim, int m, const float* codebook, int32_t* assign_pq,
                            hipStream_t s) {
  const int S = dim / m;
  dim3 grid((unsigned)((ns + 255) / 256), (unsigned)m);
#define FGPU_EST(SS)                                                                                   \
  if (S == SS) {                                                                                       \
    hipLaunchKernelGGL(pq_estep_kernel<SS>, grid, dim3(256), 0, s, res, ns, dim, m, codebook, assign_pq); \
    FGPU_HIP(hipGetLastError());                                                                       \
    return FGPU_OK;                                                                                    \
  }
  FGPU_EST(1) FGPU_EST(2) FGPU_EST(3) FGPU_EST(4) FGPU_EST(6) FGPU_EST(8) FGPU_EST(16)
#undef FGPU_EST
  return set_error(FGPU_ERR_UNSUPPORTED, "pq_estep: unsupported sub-dimension");
}

fgpu_status launch_pq_mstep(const float* res, int ns, int dim, int m, const int32_t* assign_pq, float* codebook,
                            hipStream_t s) {
  const int S = dim / m;
  FGPU_CHECK(S <= kWave, FGPU_ERR_UNSUPPORTED, "pq_mstep: sub-dimension above 64");
  hipLaunchKernelGGL(pq_mstep_kernel, dim3(kPQK, (unsigned)m), dim3(64), 0, s, res, ns, dim, m, S, assign_pq, codebook);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

size_t kmeans_pp_ws_bytes(int64_t n, int k) {
  const int64_t nb = (n + kPPBlock - 1) / kPPBlock;
  return carve_bytes<float>(n) + carve_bytes<uint64_t>(n) + carve_bytes<uint64_t>(nb) + carve_bytes<uint8_t>(n) +
         carve_bytes<int>(1) + carve_bytes<int32_t>(n) + carve_bytes<float>(k > 0 ? k : 1);
}

fgpu_status launch_kmeans_pp(const float* x, int64_t n, int dim, int k, uint64_t seed, float* cent, int32_t* rows,
                             void* ws, size_t ws_bytes, hipStream_t s) {
  Carve cv(ws, ws_bytes);
  float* d2 = cv.take<float>(n);
  uint64_t* w = cv.take<uint64_t>(n);
  const int nb = (int)((n + kPPBlock - 1) / kPPBlock);
  uint64_t* part = cv.take<uint64_t>(nb);
  uint8_t* chosen = cv.take<uint8_t>(n);
  int* shift = cv.take<int>(1);
  int32_t* asg = cv.take<int32_t>(n);
  float* cc = cv.take<float>(k > 0 ? k : 1);
  FGPU_CHECK(cv.ok(), FGPU_ERR_WORKSPACE, "kmeans++: workspace too small");
  FGPU_HIP(hipMemsetAsync(chosen, 0, n, s));
  hipLaunchKernelGGL(pp_first_kernel, dim3(1), dim3(1), 0, s, n, seed, rows, chosen);
  hipLaunchKernelGGL(pp_take_kernel, dim3(1), dim3(256), 0, s, x, dim, rows, 0, cent, chosen);
  FGPU_TRY(pp_update(x, n, dim, cent, 1, d2, nullptr, w, part, nb, asg, cc, 0, s));  // asg := 0
  hipLaunchKernelGGL(pp_shift_kernel, dim3(1), dim3(1024), 0, s, d2, n, shift);
  FGPU_HIP(hipGetLastError());
  // weights for round 1 from the initial d2 (every row: no skip yet)
  FGPU_TRY(pp_update(x, n, dim, cent, 0, d2, shift, w, part, nb, nullptr, cc, 0, s));
  for (int j = 1; j < k; ++j) {
    // pick and take the row as centre j in one workgroup
    hipLaunchKernelGGL(pp_pick_kernel, dim3(1), dim3(kPPBlock), 0, s, w, part, nb, n, seed, j, chosen, rows, x, dim,
                       cent);
    if (j + 1 < k) {
      hipLaunchKernelGGL(pp_cc_kernel, dim3((unsigned)((j + 3) / 4)), dim3(256), 0, s, cent, dim, j, cc);
      FGPU_TRY(pp_update(x, n, dim, cent + (size_t)j * dim, 0, d2, shift, w, part, nb, asg, cc, j, s));
    }
  }
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}


fgpu_status launch_list_radius(const float* codebook, int m, int sub, const uint8_t* codes, const int32_t* offsets,
                               int nlist, float* rmax, hipStream_t s) {
  if (nlist <= 0) return FGPU_OK;
  const size_t lds = (size_t)m * kPQK * sizeof(double);
  FGPU_CHECK(lds <= 128 * 1024, FGPU_ERR_UNSUPPORTED, "list_radius: pq_m too large");
  FGPU_HIP(hipFuncSetAttribute((const void*)list_radius_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL(list_radius_kernel, dim3((unsigned)nlist), dim3(256), lds, s, codebook, m, sub, codes, offsets,
                     rmax);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace fgpu
