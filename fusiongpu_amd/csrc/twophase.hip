// twophase.hip -- the general form of the reference's per-batch search and its
// exact rerank.
//
// Reference: run_gpu_batch_logic (gpu_global.cu:679-874) runs phase 1
// (ivf_scan_phase1_kernel, :321-390: per-list top-limit_k + cutoff), the
// threshold (compute_threshold_kernel, :394-426), phase 2
// (ivf_scan_phase2_kernel, :428-527: every vector with dist <= thr), then
// compaction, a segmented radix sort of every candidate and a gather of the
// first rerank_m (:533-576, :798-867), with two blocking host round trips to
// size the candidate pool (:739-763, :813-849).  run_gpu_rerank
// (:603-673) then walks the top rerank_m in mini-batches of exact L2.
//
// Here one workgroup owns one query for the whole search:
//   * phase-1 lists: LUT in LDS, all 8 waves scan with a per-list shared
//     threshold, the wave lists are merged and the list's w best plus its
//     cutoff are appended to the query's candidate pool;
//   * phase-2 lists: a list whose lower bound (residual norm minus the list's
//     decoded-residual radius) exceeds the threshold is skipped whole;
//     otherwise passers are appended with wave ballot + mbcnt compaction;
//   * the pool lives in the workspace.  When it would overflow, the workgroup
//     radix-selects the rerank_m best, keeps only those and admits later
//     candidates only below the rerank_m-th key: exact, bounded memory, no
//     host round trip;
//   * at the end a select and LDS bitonic sorts give the top rerank_m: one
//     sort up to 4096 keys, otherwise sorted runs of 4096 placed by
//     binary-search ranks against the other runs (rerank_m up to 2^17).
// The rerank kernel gives each query one 128-thread workgroup: exact
// distances one candidate per lane, wave bitonic sorts and a merge-path merge
// with the running top-k in LDS.
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"
#include "scan_common.hpp"

namespace fgpu {
namespace {

constexpr int kTW = 8;                               // waves per workgroup
constexpr int kTT = kTW * kWave;                     // 512 threads
constexpr int kTRound = kTW * kVecPerWaveRound;      // vectors per workgroup round
constexpr int kSortMax = 4096;                       // keys of one final LDS sort (a run)
constexpr int kRerankMax = 1 << 17;                  // rerank_m limit: at most 32 runs
constexpr uint64_t kNoKey = ~0ull;                   // "no admission bound yet"
constexpr int kMaxProbes = 4 * kWave;                // nprobe limit: four 64-probe chunks at set-up
constexpr int kMaxLimitK = 4096;                     // limit_k limit (above 64: the pool-select phase 1)
// Phase 1 stages the eight sorted wave lists of up to kStage lists; the waves
// merge the staged lists in parallel when the stage is full and at the end of
// phase 1, so no merge sits between two lists.  Four lists (16 KB) keep the
// workgroup's LDS within half a CU for pq_m <= 48.
constexpr int kStage = 4;
constexpr int kStageFloats = kStage * kTW * kWave * 2;

template <int D, int M>
struct TCfg {
  static constexpr int S = D / M;
  static constexpr int LUT = M * kPQK;
  static constexpr int SMEM = LUT > 2 * kSortMax ? LUT : 2 * kSortMax;  // floats: LUT, later the sort area
  static constexpr int NV4 = M / 16;
  // Two workgroups (queries) per CU where the LDS allows: 4 waves a SIMD,
  // hence at most 128 VGPRs.
  static constexpr int WPE = (SMEM + kStageFloats) * 4 <= 72 * 1024 ? 4 : 2;
};

__device__ __forceinline__ float key_dist(uint64_t key) {
  return key == kNoKey ? FLT_MAX : __uint_as_float((uint32_t)(key >> 32));
}

// Keeps the R smallest keys of pool[0..cnt) (cnt > R) in pool[0..R), in no
// particular order, and returns the R-th smallest key K: every kept key is
// <= K, so a later candidate can still enter the R best only if its key is
// < K.  MSB-first radix select, 8 bits a pass, over the full 64-bit key, then
// an in-place stream compaction: round r reads pool[r*512 + tid] before it
// writes, and its writes land below (r+1)*512, where later rounds no longer
// read.  Every thread of the workgroup calls it.
__device__ uint64_t pool_select(uint64_t* pool, int cnt, int R, int* hist, int* misc) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t prefix = 0, mask = 0;
  int need = R;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kTT) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < cnt; i += kTT) {
      const uint64_t key = pool[i];
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
    }
    __syncthreads();
    if (wave == 0) {
      const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
      const int tot = h0 + h1 + h2 + h3;
      const int incl = wave_incl_scan(tot), excl = incl - tot;
      if (excl < need && need <= incl) {
        int r = need - excl, b = 4 * lane;
        if (r > h0) {
          r -= h0; ++b;
          if (r > h1) {
            r -= h1; ++b;
            if (r > h2) { r -= h2; ++b; }
          }
        }
        misc[0] = b;
        misc[1] = r;
      }
    }
    __syncthreads();
    prefix |= (uint64_t)misc[0] << shift;
    mask |= (uint64_t)0xFF << shift;
    need = misc[1];
  }
  const uint64_t K = prefix;  // exactly the R-th smallest; `need` copies of K complete the R
  if (tid == 0) misc[2] = 0;
  __syncthreads();
  int out = 0;
  for (int r0 = 0; r0 < cnt; r0 += kTT) {
    const int i = r0 + tid;
    const uint64_t key = i < cnt ? pool[i] : kNoKey;
    const bool keep = i < cnt && (key < K || (key == K && atomicAdd(&misc[2], 1) < need));
    const uint64_t bm = __ballot(keep);
    if (lane == 0) hist[wave] = __popcll(bm);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kTW; ++w) {
      const int c = hist[w];
      before += w < wave ? c : 0;
      total += c;
    }
    if (keep) pool[out + before + __popcll(bm & ((1ull << lane) - 1ull))] = key;
    out += total;
    __syncthreads();
  }
  return K;
}

// Ascending bitonic sort of sk[0..np2) (np2 a power of two) by all threads.
__device__ void lds_bitonic_sort(uint64_t* sk, int np2) {
  for (int size = 2; size <= np2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (np2 >> 1); i += kTT) {
        const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
        const bool up = (lo & size) == 0;
        const uint64_t x = sk[lo], y = sk[hi];
        if ((x > y) == up) {
          sk[lo] = y;
          sk[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

template <int D, int M, int MODE>
__global__ __launch_bounds__(kTT) __attribute__((amdgpu_waves_per_eu(TCfg<D, M>::WPE, TCfg<D, M>::WPE)))
void two_phase_kernel(TwoPhaseArgs a) {
  using C = TCfg<D, M>;
  constexpr int G = kTT / kPQK;  // threads sharing one codeword
  constexpr int MG = M / G;      // subspaces per thread in the LUT build
  static_assert(M % G == 0 && M % 16 == 0 && D % M == 0, "geometry");
  static_assert(D <= 2 * kWave, "the list bound takes two residual coordinates per lane");
  // The LUT (later the sort area) opens the array so that every LUT row is
  // within the 16-bit immediate offset of a DS instruction; the phase-1 stage
  // follows it.
  __shared__ __align__(16) float smem[C::SMEM + kStageFloats];
  __shared__ float rbuf[2][D];
  __shared__ float qs[D];
  __shared__ int st_f[kStage], st_base[kStage];
  __shared__ int hist[256];
  __shared__ int misc[4];
  __shared__ float s_cut[kMaxProbes];
  __shared__ int f_list[kMaxProbes], f_start[kMaxProbes], f_n[kMaxProbes], f_p[kMaxProbes];  // usable probes, in order
  __shared__ float f_lb[kMaxProbes];                                                          // phase-2 list bounds
  __shared__ int f_base[kMaxProbes + 1];  // phase-1 list f's pool slots start at f_base[f] (limit_k <= 64)
  __shared__ int s_nv, s_nv1;
  __shared__ int s_cnt;
  __shared__ int s_pre;  // phase-2 vectors with dist <= thr (TwoPhaseArgs::pre_cut)
  __shared__ unsigned long long s_lthr;
  __shared__ unsigned long long s_pub[kTW];  // phase 1: each wave's Q-th best key of the current list

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = tid & (kPQK - 1), g = __builtin_amdgcn_readfirstlane(tid / kPQK);
  // Split phase 1 (small batches, limit_k <= 64): a launch with MODE 1 runs
  // a.split workgroups a query, workgroup g scanning phase-1 lists g,
  // g + split, ...; each list's pool slots and cutoff depend only on the list,
  // so the workgroups write them independently (cutoffs to a.cut_ws).  A
  // second launch with MODE 2 (one workgroup a query) reads the cutoffs back
  // and runs the threshold, phase 2 and the final select.  MODE 0 does it
  // all in one workgroup (separate instantiations keep its code as it is).
  constexpr int mode = MODE;
  int q = mode == 1 ? (int)blockIdx.x / a.split : (int)blockIdx.x;
  if (mode == 2 && a.qlist) {  // uniform over the workgroup, before any barrier
    if ((int)blockIdx.x >= *a.qcount) return;
    q = a.qlist[blockIdx.x];
  }
  const int gsub = mode == 1 ? (int)blockIdx.x % a.split : 0;
  const int gstep = mode == 1 ? a.split : 1;
  const int P = a.nprobe, p1 = a.p1, R = a.rerank_m, cap = a.pool_cap, K1 = a.limit_k;
  // If every wave holds Q = ceil(K1 / 8) vectors at or below its published
  // key, the list has >= 8 Q >= K1 vectors at or below the largest published
  // key, so nothing above it can be among the list's K1 best.
  const int Q = (K1 + kTW - 1) / kTW;
  const uint32_t NL = (uint32_t)a.nlist;
  uint64_t* pool = a.pool + (size_t)q * cap;
  const long long t_start = a.stats ? clock64() : 0;

  for (int i = tid; i < D; i += kTT) qs[i] = a.queries[(size_t)q * D + i];
  if (tid < kMaxProbes) s_cut[tid] = 0.0f;
  if (tid < kTW) s_pub[tid] = kNoThr;
  if (wave == 0) {
    // Usable probes (in range, non-empty) in probe order, 64 probes a step;
    // the first s_nv1 are phase 1 (probe index < p1).
    int nv_run = 0, nv1_run = 0, base_run = 0;
    for (int c0 = 0; c0 < P; c0 += kWave) {
      const int pi = c0 + lane;
      int l = 0, st = 0, n = 0;
      if (pi < P) {
        const uint32_t pl = a.probes[(size_t)q * P + pi];
        if (pl < NL) {
          l = (int)pl;
          st = a.offsets[pl];
          n = a.offsets[pl + 1] - st;
        }
      }
      const uint64_t bm = __ballot(n > 0);
      const int pos = nv_run + __popcll(bm & ((1ull << lane) - 1ull));
      // Pool slots of a phase-1 list: min(n, limit_k) (used with limit_k <= 64).
      const int w1 = n > 0 && pi < p1 ? (n < K1 ? n : K1) : 0;
      const int incl = wave_incl_scan(w1);
      if (n > 0) {
        f_list[pos] = l;
        f_start[pos] = st;
        f_n[pos] = n;
        f_p[pos] = pi;
        if (pi < p1) f_base[pos] = base_run + incl - w1;
      }
      nv_run += __popcll(bm);
      nv1_run += __popcll(__ballot(n > 0 && pi < p1));
      base_run += __shfl(incl, kWave - 1, kWave);
    }
    if (lane == 0) {
      f_base[nv1_run] = base_run;
      s_nv = nv_run;
      s_nv1 = nv1_run;
      s_cnt = 0;
      s_pre = 0;
      s_lthr = kNoThr;
    }
  }
  __syncthreads();
  const int nv = s_nv, nv1 = s_nv1;

  auto residual = [&](int f, float* r) {
    if (tid < D) r[tid] = qs[tid] - a.centroids[(size_t)f_list[f] * D + tid];
  };
  // Lower bound of every phase-2 list, one wave per list: every later skip
  // decision is an LDS read.
  for (int f = nv1 + wave; mode != 1 && f < nv; f += kTW) {
    const float* cr = a.centroids + (size_t)f_list[f] * D;
    const float ra = lane < D ? qs[lane] - cr[lane] : 0.0f;
    const float rb = lane + kWave < D ? qs[lane + kWave] - cr[lane + kWave] : 0.0f;
    float s2 = ra * ra + rb * rb;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s2 += shfl_xor_f(s2, o);
    if (lane == 0) f_lb[f] = list_lower_bound(s2, a.rmax[f_list[f]]);
  }
  // The first list this workgroup scans: gsub in phase 1, none ahead of
  // phase 2 in mode 2 (phase 2 computes its residuals itself).
  if (mode != 2 && gsub < nv) residual(gsub, rbuf[0]);
  __syncthreads();
  const long long t_setup = a.stats ? clock64() : 0;

  float* lut = smem;
  auto build_lut = [&](const float* r) {
    int kcv = kc;
    asm volatile("" : "+v"(kcv));
    float* dst = lut + g * MG * kPQK + kcv;
    // The codebook rows come from L2 at each build (the codebook is shared
    // by every workgroup); holding them in registers would halve occupancy.
    const float* cbp = a.codebook + ((size_t)g * MG * kPQK + kcv) * C::S;
    const float* rg = r + g * MG * C::S;
    // Groups of about 16 codebook floats: a group's loads are all issued
    // before its entries are computed (the scheduling barrier keeps them
    // together), one L2 round trip a group instead of one a subspace.
    constexpr int GR = 16 / C::S > 0 ? 16 / C::S : 1;
#pragma unroll
    for (int m0 = 0; m0 < MG; m0 += GR) {
      float cv[GR * C::S];
#pragma unroll
      for (int mm = 0; mm < GR; ++mm) {
#pragma unroll
        for (int j = 0; j < C::S; ++j)
          cv[mm * C::S + j] = m0 + mm < MG ? cbp[(m0 + mm) * kPQK * C::S + j] : 0.0f;
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mm = 0; mm < GR; ++mm) {
        if (m0 + mm < MG) {
          float rr[C::S];
#pragma unroll
          for (int j = 0; j < C::S; ++j) rr[j] = rg[(m0 + mm) * C::S + j];
          dst[(m0 + mm) * kPQK] = lut_entry<C::S>(rr, cv + mm * C::S);
        }
      }
    }
  };

  uint4 w0[C::NV4], w1[C::NV4], n0[C::NV4], n1[C::NV4];
  int i0 = kPadId, i1 = kPadId, j0 = kPadId, j1 = kPadId;
  int it = 0;       // lists processed: rbuf[it & 1] holds the residual of list pre_f
  int pre_f = mode != 2 && gsub < nv ? gsub : -1;
  // instrumentation (per wave; summed at the end when a.stats is set)
  unsigned st_load = 0, st_lut = 0, st_skip = 0, st_pass = 0;
  auto count_load = [&](int base, int end) { st_load += (unsigned)max(0, min(kVecPerWaveRound, end - base)); };

  // ---------------- phase 1: per-list top-limit_k and cutoffs
  int cnt_p1 = 0;  // pool entries of the phase-1 lists so far (the same in every wave)
  int nst = 0;     // lists staged
  uint64_t(*stage)[kTW * kWave] = reinterpret_cast<uint64_t(*)[kTW * kWave]>(smem + C::SMEM);
  // Merge round: wave w merges staged lists w, w + 8, ...; the list's w best
  // keys go to its pool slots and the w-th distance is its cutoff.
  auto flush = [&]() {
    for (int t = wave; t < nst; t += kTW) {
      uint64_t k = stage[t][lane];
#pragma unroll 1
      for (int v = 1; v < kTW; ++v) wave_merge_sorted64_k(k, stage[t][v * kWave + lane]);
      const int lf = st_f[t], n = f_n[lf];
      const int w = n < K1 ? n : K1;
      if (lane < w) pool[st_base[t] + lane] = k;
      const float cut = key_dist(readlane64(k, w - 1));
      if (lane == 0) {
        s_cut[f_p[lf]] = cut;
        if (mode == 1) a.cut_ws[(size_t)q * P + f_p[lf]] = cut;
      }
    }
    nst = 0;
    __syncthreads();  // the stage is free again
  };
  long long c_build = 0, c_scan = 0, c_merge = 0;
  // limit_k > 64: every vector of a phase-1 list is a candidate.  The list's
  // keys go to the pool above the earlier lists' entries; whenever the next
  // segment could overflow the pool, pool_select cuts them to the limit_k
  // best, and later keys enter only below the limit_k-th.  The pool leaves at
  // least 2048 slots above limit_k for every list (two_phase_pool_cap).  The
  // list's cutoff is then the largest of the w = min(n, limit_k) keys kept,
  // its w-th smallest distance.
  for (int f = 0; K1 > kWave && mode == 0 && f < nv1; ++f) {
    const int start = f_start[f], n = f_n[f];
    const int first = wave * kVecPerWaveRound;
    load_pair<M>(a.codes, a.vec_ids, start, n, first + lane, w0, w1, i0, i1);
    count_load(first, n);
    ++st_lut;
    build_lut(rbuf[it & 1]);
    const int nf = f + 1 < nv ? f + 1 : -1;
    if (nf >= 0) residual(nf, rbuf[(it + 1) & 1]);
    if (tid == 0) s_cnt = 0;
    __syncthreads();  // LUT and next residual ready; the list's count is 0
    uint64_t* lp = pool + cnt_p1;
    const int room = cap - cnt_p1;
    const int segl = room - K1;
    uint64_t ladm = kNoKey;
    int held = 0;
    int s0 = 0;
    bool loaded = true;
    while (true) {
      const int s1 = n - s0 > segl ? s0 + segl : n;
      if (held + (s1 - s0) > room) {
        ladm = pool_select(lp, held, K1, hist, misc);
        held = K1;
        if (tid == 0) s_cnt = K1;
        __syncthreads();
      }
      for (int base = s0 + first; base < s1; base += kTRound) {
        if (!loaded) {
          load_pair<M>(a.codes, a.vec_ids, start, n, base + lane, w0, w1, i0, i1);
          count_load(base, n);
        }
        loaded = false;
        const int v0 = base + lane, v1 = v0 + kWave;
        float d0, d1;
        adc_sum2_full<M>(lut, w0, w1, 0.0f, d0, d1);
        const uint64_t k0 = key_of(d0, i0), k1 = key_of(d1, i1);
        const bool pass0 = v0 < s1 && k0 < ladm, pass1 = v1 < s1 && k1 < ladm;
        const uint64_t b0 = __ballot(pass0), b1 = __ballot(pass1);
        const int c0 = __popcll(b0), c = c0 + __popcll(b1);
        if (c) {
          int at = 0;
          if (lane == 0) at = atomicAdd(&s_cnt, c);
          at = __shfl(at, 0, kWave);
          const uint64_t below = (1ull << lane) - 1ull;
          if (pass0) lp[at + __popcll(b0 & below)] = k0;
          if (pass1) lp[at + c0 + __popcll(b1 & below)] = k1;
        }
      }
      loaded = false;
      __syncthreads();  // the segment's appends are done
      held = s_cnt;
      __syncthreads();  // every thread has read the count
      if (s1 >= n) break;
      s0 = s1;
    }
    if (held > K1) {
      pool_select(lp, held, K1, hist, misc);
      held = K1;
    }
    // cutoff: the largest kept key (the w-th smallest of the list)
    uint64_t mx = 0;
    for (int i = tid; i < held; i += kTT) mx = lp[i] > mx ? lp[i] : mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t t = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(mx >> 32), o, kWave) << 32) |
                         (uint32_t)__shfl_xor((int)(uint32_t)mx, o, kWave);
      mx = t > mx ? t : mx;
    }
    if (lane == 0) s_pub[wave] = mx;
    __syncthreads();
    if (tid == 0) {
      uint64_t m = s_pub[0];
      for (int w = 1; w < kTW; ++w) m = s_pub[w] > m ? s_pub[w] : m;
      s_cut[f_p[f]] = held > 0 ? key_dist(m) : 0.0f;
    }
    cnt_p1 += held;
    ++it;
    pre_f = nf;
    __syncthreads();  // every wave is through list f: the LUT and s_pub are free
  }
  for (int f = gsub; K1 <= kWave && mode != 2 && f < nv1; f += gstep) {
    const long long c0 = a.stats ? clock64() : 0;
    const int start = f_start[f], n = f_n[f];
    const int first = wave * kVecPerWaveRound;
    load_pair<M>(a.codes, a.vec_ids, start, n, first + lane, w0, w1, i0, i1);
    count_load(first, n);
    ++st_lut;
    // All waves have finished scanning list f-1 (they passed the barrier
    // after it), so the single LUT buffer is free.
    build_lut(rbuf[it & 1]);
    // The next list's residual: the next phase-1 list of this workgroup, or in
    // mode 0 whatever list follows (the first phase-2 list after phase 1).
    const int nf = mode == 1 ? (f + gstep < nv1 ? f + gstep : -1) : (f + 1 < nv ? f + 1 : -1);
    if (nf >= 0) residual(nf, rbuf[(it + 1) & 1]);
    __syncthreads();  // LUT f and the next residual ready; s_lthr reset
    const long long c1 = a.stats ? clock64() : 0;
    uint64_t lk = kPadKey;
    uint64_t own = kNoThr;
    for (int base = first; base < n; base += kTRound) {
      const int nb = base + kTRound;
      if (nb < n) {
        load_pair<M>(a.codes, a.vec_ids, start, n, nb + lane, n0, n1, j0, j1);
        count_load(nb, n);
      }
      const int v0 = base + lane, v1 = v0 + kWave;
      uint64_t thr = s_lthr;
      thr = own < thr ? own : thr;
      {
        uint64_t pub = s_pub[0];
#pragma unroll
        for (int w = 1; w < kTW; ++w) {
          const uint64_t pw = s_pub[w];
          pub = pw > pub ? pw : pub;
        }
        thr = pub < thr ? pub : thr;
      }
      float d0, d1;
      if (adc_sum2_full<M>(lut, w0, w1, __uint_as_float((uint32_t)(thr >> 32)), d0, d1)) {
        if (offer2_k(v0 < n ? key_of(d0, i0) : kPadKey, v1 < n ? key_of(d1, i1) : kPadKey, thr, K1, lk)) {
          own = readlane64(lk, K1 - 1);
          const uint64_t qth = readlane64(lk, Q - 1);
          if (lane == 0) {
            atomicMin(&s_lthr, (unsigned long long)own);
            s_pub[wave] = qth;
          }
        }
      }
      if (nb < n) {
#pragma unroll
        for (int i = 0; i < C::NV4; ++i) {
          w0[i] = n0[i];
          w1[i] = n1[i];
        }
        i0 = j0;
        i1 = j1;
      }
    }
    const long long c2 = a.stats ? clock64() : 0;
    stage[nst][wave * kWave + lane] = lk;
    if (tid == 0) {
      st_f[nst] = f;
      st_base[nst] = mode == 0 ? cnt_p1 : f_base[f];
    }
    cnt_p1 += n < K1 ? n : K1;
    ++nst;
    __syncthreads();  // every wave is through list f: its list is staged, the LUT is free
    if (wave == 0) {
      if (lane == 0) s_lthr = kNoThr;
      if (lane < kTW) s_pub[lane] = kNoThr;
    }
    if (nst == kStage || f + gstep >= nv1) flush();
    if (a.stats) {
      const long long c3 = clock64();
      c_build += c1 - c0;
      c_scan += c2 - c1;
      c_merge += c3 - c2;
    }
    ++it;
    pre_f = nf;
  }
  if constexpr (mode == 1) {  // this workgroup's phase-1 lists are in the pool, their cutoffs in a.cut_ws
    if (a.stats) {
      if (lane == 0) {
        atomicAdd(&a.stats[0], (unsigned long long)st_load);
        if (wave == 0) atomicAdd(&a.stats[1], (unsigned long long)st_lut);
      }
      if (tid == 0) {
        atomicAdd(&a.stats[4], (unsigned long long)(t_setup - t_start));
        atomicAdd(&a.stats[5], (unsigned long long)(clock64() - t_setup));
        atomicAdd(&a.stats[8], (unsigned long long)c_build);
        atomicAdd(&a.stats[9], (unsigned long long)c_scan);
        atomicAdd(&a.stats[10], (unsigned long long)c_merge);
      }
    }
    return;
  }
  if constexpr (mode == 2) {  // phase 1 ran in the mode-1 launch: its pool slots and cutoffs
    if (K1 <= kWave) cnt_p1 = f_base[nv1];
    for (int f = tid; f < nv1; f += kTT) s_cut[f_p[f]] = a.cut_ws[(size_t)q * P + f_p[f]];
  }
  if (tid == 0) s_cnt = cnt_p1;
  __syncthreads();
  const long long t_phase1 = a.stats ? clock64() : 0;

  // ---------------- threshold (compute_threshold_kernel): coeff * min(cutoff > 0)
  float min_cut = FLT_MAX;
  for (int p = 0; p < p1; ++p) {
    const float c = s_cut[p];
    if (c > 0.0f && c < min_cut) min_cut = c;
  }
  const float thr = min_cut < FLT_MAX ? min_cut * a.coeff : FLT_MAX;
  if (a.cutoffs && tid < p1) a.cutoffs[(size_t)q * p1 + tid] = s_cut[tid];
  if (a.thr && tid == 0) a.thr[q] = thr;

  // ---------------- phase 2: every vector with dist <= thr, bounded pool
  const int seg = cap - R;  // vectors per segment: their passers always fit after a select
  uint64_t adm = kNoKey;
  float thr_d = thr;
  // Counting the candidates before the cut: every vector with dist <= thr is
  // counted, so skips and early ends use thr, never the admission bound.
  const bool count_all = a.pre_cut != nullptr;
  int n_thr = 0;  // this wave's phase-2 vectors with dist <= thr (count_all)
  for (int f = nv1; f < nv; ++f) {
    // thr_d only shrinks (selects lower adm), so a list skipped now stays skippable.
    const float thr_hi = (count_all ? thr : thr_d) * (1.0f + 0x1p-16f);
    if (f_lb[f] > thr_hi) {
      ++st_skip;
      continue;
    }
    const int start = f_start[f], n = f_n[f];
    float* r = rbuf[it & 1];
    if (pre_f != f) residual(f, r);
    __syncthreads();  // residual ready; the previous list is scanned and its appends are done
    int cnt0 = s_cnt;
    const int first = wave * kVecPerWaveRound;
    load_pair<M>(a.codes, a.vec_ids, start, n, first + lane, w0, w1, i0, i1);
    count_load(first, n);
    ++st_lut;
    build_lut(r);
    int nf = f + 1;
    while (nf < nv && f_lb[nf] > thr_hi) ++nf;
    if (nf < nv) residual(nf, rbuf[(it + 1) & 1]);
    __syncthreads();  // LUT ready; every thread has read cnt0
    int s0 = 0;
    while (true) {
      const int s1 = n - s0 > seg ? s0 + seg : n;
      if (cnt0 + (s1 - s0) > cap) {
        adm = pool_select(pool, cnt0, R, hist, misc);
        cnt0 = R;
        if (tid == 0) s_cnt = R;
        __syncthreads();
        thr_d = fminf(thr, key_dist(adm));
      }
      int base = s0 + first;
      bool loaded = s0 == 0;  // segment 0's first round was loaded before the LUT build
      // Phase 2 loads each round when it starts: most of its lists are
      // skipped whole, and prefetch registers here would spill at the
      // two-workgroup register budget.
      while (base < s1) {
        const int nb = base + kTRound;
        if (!loaded) {
          load_pair<M>(a.codes, a.vec_ids, start, n, base + lane, w0, w1, i0, i1);
          count_load(base, n);
        }
        loaded = false;
        const int v0 = base + lane, v1 = v0 + kWave;
        float d0, d1;
        if (adc_sum2<M>(lut, w0, w1, v0 < s1, v1 < s1, count_all ? thr : thr_d, d0, d1)) {
          if (count_all)
            n_thr += __popcll(__ballot(v0 < s1 && d0 <= thr)) + __popcll(__ballot(v1 < s1 && d1 <= thr));
          const uint64_t k0 = key_of(d0, i0), k1 = key_of(d1, i1);
          const bool pass0 = v0 < s1 && d0 <= thr && k0 < adm;
          const bool pass1 = v1 < s1 && d1 <= thr && k1 < adm;
          const uint64_t b0 = __ballot(pass0), b1 = __ballot(pass1);
          const int c0 = __popcll(b0), c = c0 + __popcll(b1);
          if (c) {
            st_pass += c;
            int at = 0;
            if (lane == 0) at = atomicAdd(&s_cnt, c);
            at = __shfl(at, 0, kWave);
            const uint64_t below = (1ull << lane) - 1ull;
            if (pass0) pool[at + __popcll(b0 & below)] = k0;
            if (pass1) pool[at + c0 + __popcll(b1 & below)] = k1;
          }
        }
        base = nb;
      }
      if (s1 >= n) break;
      s0 = s1;
      __syncthreads();  // the segment's appends are done
      cnt0 = s_cnt;
      __syncthreads();  // everyone has read the count before new appends
    }
    ++it;
    pre_f = nf < nv ? nf : -1;
  }
  const long long t_phase2 = a.stats ? clock64() : 0;
  if (a.stats && lane == 0) {
    atomicAdd(&a.stats[0], (unsigned long long)st_load);
    if (wave == 0) {
      atomicAdd(&a.stats[1], (unsigned long long)st_lut);
      atomicAdd(&a.stats[2], (unsigned long long)st_skip);
    }
    atomicAdd(&a.stats[3], (unsigned long long)st_pass);
  }

  // ---------------- top rerank_m: select, LDS bitonic sort, gather
  if (count_all && lane == 0 && n_thr) atomicAdd(&s_pre, n_thr);
  __syncthreads();
  int cnt = s_cnt;
  if (count_all && tid == 0) a.pre_cut[q] = f_base[nv1] + s_pre;
  if (cnt > R) {
    pool_select(pool, cnt, R, hist, misc);
    cnt = R;
  }
  uint64_t* sk = reinterpret_cast<uint64_t*>(smem);
  int32_t* out_id = a.top_ids + (size_t)q * R;
  float* out_d = a.top_d + (size_t)q * R;
  if (cnt <= kSortMax / 2) {
    // Runs of 64 keys sorted in registers (one wave a run, no barriers),
    // then merged pairwise by ranks between two LDS buffers: a key's place
    // in the merged pair is its index in its run plus the keys of the other
    // run before it (on equal keys the left run goes first).  The last merge
    // writes the output.  Padding keys (kNoKey) sort after every real key.
    const int nk = (cnt + kWave - 1) / kWave * kWave;
    uint64_t* src = sk;
    uint64_t* dst = sk + kSortMax / 2;
    for (int r = wave; r * kWave < nk; r += kTW) {
      const int i = r * kWave + lane;
      uint64_t key = i < cnt ? pool[i] : kNoKey;
      wave_sort64_k(key);
      src[i] = key;
    }
    __syncthreads();
    for (int width = kWave;; width *= 2) {
      const bool last = 2 * width >= nk;
      for (int i = tid; i < nk; i += kTT) {
        const int run = i / width, other = (run ^ 1) * width;
        const uint64_t key = src[i];
        int lo = 0, hi = other < nk ? min(width, nk - other) : 0;
        if (run & 1) {  // right run: the left run's keys <= key come first
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (src[other + mid] <= key) lo = mid + 1; else hi = mid;
          }
        } else {  // left run: the right run's keys < key come first
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (src[other + mid] < key) lo = mid + 1; else hi = mid;
          }
        }
        const int pos = (run & ~1) * width + (i - run * width) + lo;
        if (!last) {
          dst[pos] = key;
        } else if (pos < cnt) {
          out_id[pos] = (int32_t)(uint32_t)key;
          out_d[pos] = __uint_as_float((uint32_t)(key >> 32));
        }
      }
      if (last) break;
      __syncthreads();
      uint64_t* t = src;
      src = dst;
      dst = t;
    }
  } else if (cnt <= kSortMax) {
    int np2 = 1;
    while (np2 < cnt) np2 <<= 1;
    for (int i = tid; i < np2; i += kTT) sk[i] = i < cnt ? pool[i] : kNoKey;
    __syncthreads();
    lds_bitonic_sort(sk, np2);
    for (int j = tid; j < cnt; j += kTT) {
      const uint64_t key = sk[j];
      out_id[j] = (int32_t)(uint32_t)key;
      out_d[j] = __uint_as_float((uint32_t)(key >> 32));
    }
  } else {
    // More keys than one LDS sort holds: sort runs of kSortMax keys in LDS and
    // write each back in place, then put every key at its final position,
    // its index in its run plus, for every other run, the keys there that
    // precede it (binary search; on equal keys the earlier run goes first).
    const int nruns = (cnt + kSortMax - 1) / kSortMax;
    for (int r = 0; r < nruns; ++r) {
      const int r0 = r * kSortMax, len = min(kSortMax, cnt - r0);
      int np2 = 1;
      while (np2 < len) np2 <<= 1;
      for (int i = tid; i < np2; i += kTT) sk[i] = i < len ? pool[r0 + i] : kNoKey;
      __syncthreads();
      lds_bitonic_sort(sk, np2);
      for (int i = tid; i < len; i += kTT) pool[r0 + i] = sk[i];
      __syncthreads();  // the run is back in the pool before the sort area is reused / ranks are read
    }
    for (int j = tid; j < cnt; j += kTT) {
      const int r = j / kSortMax;
      const uint64_t key = pool[j];
      int pos = j - r * kSortMax;
      for (int o = 0; o < nruns; ++o) {
        if (o == r) continue;
        const uint64_t* run = pool + o * kSortMax;
        int lo = 0, hi = min(kSortMax, cnt - o * kSortMax);  // count of run keys < key (o > r) or <= key (o < r)
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          const uint64_t v = run[mid];
          if (o < r ? v <= key : v < key)
            lo = mid + 1;
          else
            hi = mid;
        }
        pos += lo;
      }
      out_id[pos] = (int32_t)(uint32_t)key;
      out_d[pos] = __uint_as_float((uint32_t)(key >> 32));
    }
  }
  for (int j = cnt + tid; j < R; j += kTT) {
    out_id[j] = -1;
    out_d[j] = FLT_MAX;
  }
  if (tid == 0) a.top_counts[q] = cnt;
  if (a.stats && tid == 0) {
    const long long t_end = clock64();
    atomicAdd(&a.stats[4], (unsigned long long)(t_setup - t_start));
    atomicAdd(&a.stats[5], (unsigned long long)(t_phase1 - t_setup));
    atomicAdd(&a.stats[6], (unsigned long long)(t_phase2 - t_phase1));
    atomicAdd(&a.stats[7], (unsigned long long)(t_end - t_phase2));
    atomicAdd(&a.stats[8], (unsigned long long)c_build);
    atomicAdd(&a.stats[9], (unsigned long long)c_scan);
    atomicAdd(&a.stats[10], (unsigned long long)c_merge);
  }
}

template <int D, int M>
fgpu_status launch_tp(const TwoPhaseArgs& a, int nq, hipStream_t s) {
  if (a.split > 1 && a.limit_k <= kWave && a.cut_ws) {
    hipLaunchKernelGGL((two_phase_kernel<D, M, 1>), dim3((unsigned)(nq * a.split)), dim3(kTT), 0, s, a);
    FGPU_HIP(hipGetLastError());
    hipLaunchKernelGGL((two_phase_kernel<D, M, 2>), dim3((unsigned)nq), dim3(kTT), 0, s, a);
    FGPU_HIP(hipGetLastError());
    return FGPU_OK;
  }
  hipLaunchKernelGGL((two_phase_kernel<D, M, 0>), dim3((unsigned)nq), dim3(kTT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

// ---------------------------------------------------------------------------
// Exact rerank.  128 threads per query; thread t evaluates candidate t of a
// mini-batch (mb <= 128) with the reference's exact distance (sequential
// fused chain over the dimensions, gpu_global.cu:636).  The rows are loaded
// eight lanes a row and handed to their lanes through LDS (wave_rows_l2).
constexpr int kRT = 2 * kWave;

// SPEC mini-batches a step: the workgroup's SPEC groups of 128 threads
// compute the exact distances of the next SPEC mini-batches at once (the row
// loads of a small batch are latency-bound), then apply them one after
// another in candidate order, each with the merge and the stop test of the
// one-batch form; a stop discards the mini-batches after it, which count as
// never visited.  SPEC = 1 is the one-batch form.
template <int D, int SPEC>
__global__ __launch_bounds__(kRT * SPEC) void rerank_kernel(RerankArgs a) {
  constexpr int kT = kRT * SPEC;
  __shared__ float qs[D];
  __shared__ __align__(16) float trb[2 * SPEC][row_tr_floats()];  // each wave's row hand-over buffer
  __shared__ uint64_t tk[2][256];     // running top-k keys (double-buffered), ascending
  __shared__ uint64_t nk[SPEC][kRT];  // each group's mini-batch, sorted
  __shared__ int s_chg, s_stable, s_fin;
  const int tid = threadIdx.x, lane = tid & 63;
  const int grp = tid / kRT, gt = tid % kRT, wave = gt >> 6;  // group, thread and wave within the group
  const int q = blockIdx.x, k = a.k, mb = a.mb, rm = a.rm;
  for (int i = tid; i < D; i += kT) qs[i] = a.queries[(size_t)q * D + i];
  for (int i = tid; i < k; i += kT) tk[0][i] = kPadKey;
  if (tid == 0) {
    s_stable = 0;
    s_fin = 0;
  }
  const int total = min(a.counts[q], rm);
  const int32_t* cand = a.cand + (size_t)q * rm;
  __syncthreads();
  int cur = 0, seen = 0;
  for (int off0 = 0; off0 < rm && off0 < total; off0 += SPEC * mb) {
    // exact distances of this group's mini-batch, one candidate per thread
    const int off = off0 + grp * mb;
    const int eff = off < rm && off < total ? min(mb, total - off) : 0;
    float d = FLT_MAX;
    int id = kPadId;
    {
      const int vid = gt < eff ? cand[off + gt] : -1;
      const bool ok = vid >= 0 && (long long)vid < a.n;
      const uint64_t okm = __ballot(ok);
      if (okm) {  // the wave's rows, all requested before the first multiply-add, eight lanes a row
        const int fill = readlane_i(vid, __ffsll((unsigned long long)okm) - 1);  // a valid row for the other lanes
        const float dd = wave_rows_l2<D>(a.base, ok ? vid : fill, qs, trb[tid >> 6]);
        if (ok) {
          d = dd;
          id = vid;
        }
      }
    }
    // sort each mini-batch: each wave its 64 keys, then a merge by ranks
    uint64_t key = key_of(d, id);
    wave_sort64_k(key);
    nk[grp][gt] = key;
    if (tid == 0) s_chg = 0;
    __syncthreads();
    {
      const uint64_t* ok = nk[grp] + (wave ^ 1) * kWave;
      // rank in the other wave's sorted list: wave 0 counts strictly smaller
      // keys, wave 1 counts smaller-or-equal ones, so equal keys keep a fixed
      // order and every position is taken once.
      int lo = 0, hi = kWave;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const bool before = wave == 0 ? ok[mid] < key : ok[mid] <= key;
        if (before) lo = mid + 1; else hi = mid;
      }
      __syncthreads();
      nk[grp][lane + lo] = key;
    }
    __syncthreads();
    // apply the mini-batches in order
    for (int g = 0; g < SPEC; ++g) {
      const int offg = off0 + g * mb;
      if (offg >= rm || offg >= total) break;
      seen += min(mb, total - offg);
      // merge the sorted batch (nk[g], kRT keys) with the top-k (tk[cur])
      const uint64_t* ck = tk[cur];
      uint64_t* xk = tk[cur ^ 1];
      if (tid < kRT) {
        const uint64_t bk = nk[g][tid];
        // old entries precede equal batch entries
        int lo = 0, hi = k;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (ck[mid] <= bk) lo = mid + 1; else hi = mid;
        }
        const int pos = tid + lo;
        bool fresh = false;
        if (pos < k) {
          xk[pos] = bk;
          const int bi = key_id(bk);
          if (bi != kPadId) {
            fresh = true;
            for (int j = 0; j < k; ++j)
              if (key_id(ck[j]) == bi) { fresh = false; break; }
          }
        }
        const uint64_t bm = __ballot(fresh);
        if (lane == 0 && bm) atomicAdd(&s_chg, (int)__popcll(bm));
      }
      for (int j = tid; j < k; j += kT) {
        const uint64_t okey = ck[j];
        int lo = 0, hi = kRT;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (nk[g][mid] < okey) lo = mid + 1; else hi = mid;
        }
        const int pos = j + lo;
        if (pos < k) xk[pos] = okey;
      }
      __syncthreads();
      if (tid == 0) {
        const int st = ((float)s_chg / (float)k <= a.eps) ? s_stable + 1 : 0;
        s_stable = st;
        s_fin = st >= a.beta;
        s_chg = 0;  // for the next mini-batch
      }
      cur ^= 1;
      __syncthreads();
      if (s_fin) break;
    }
    if (s_fin) break;
  }
  for (int j = tid; j < k; j += kT) {
    const uint64_t kk = tk[cur][j];
    const bool pad = key_id(kk) == kPadId;
    a.out_ids[(size_t)q * k + j] = pad ? -1 : key_id(kk);
    a.out_d[(size_t)q * k + j] = pad ? FLT_MAX : key_dist(kk);
  }
  if (a.visited && tid == 0) a.visited[q] = seen;
  if (tid == 0) {
    if (a.stable) a.stable[q] = s_stable;
    // finished: stopped on stability, or an offset below rm reached the end of the candidates
    if (a.finished) a.finished[q] = (s_fin || (total + mb - 1) / mb * mb < rm) ? 1 : 0;
  }
}

// ---------------------------------------------------------------------------
// Phase 1 through the MFMA screen (fgpu_two_phase_search with limit_k <= 64):
// every (query, phase-1 probe) becomes a virtual query of one probe, whose
// exact top-limit_k over its list the screen (screen.hip) returns; these
// kernels set the virtual queries up and put their results where phase 2
// reads phase 1's (the pool slots and cutoffs of a split phase 1).

__global__ __launch_bounds__(256) void tp_zero_kernel(int* __restrict__ p, int n) {
  const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (i < n) p[i] = 0;
}

// Virtual query v = q p1 + p (q of the chunk; it reads query row q, as
// v / p1, from the chunk's rows): its probe p (0xFFFFFFFF when out of range or
// empty), a zero
// probe distance (the lower bound of its only list is then 0, so the list is
// always screened), its list's count in hist and its rank among the list's
// virtual queries (the order of the list's atomics; those without a list
// ranked by hist[2 nlist]).
__global__ __launch_bounds__(256) void tp_virtual_kernel(const uint32_t* __restrict__ probes, int P, int p1, int nvq,
                                                         const int32_t* __restrict__ offsets, int nlist,
                                                         uint32_t* __restrict__ vprobe, float* __restrict__ vpd,
                                                         int* __restrict__ hist, int32_t* __restrict__ rank) {
  const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (i >= nvq) return;
  const int qq = i / p1, p = i - qq * p1;
  const uint32_t l = probes[(size_t)qq * P + p];
  const bool use = l < (uint32_t)nlist && offsets[l + 1] > offsets[l];
  vprobe[i] = use ? l : 0xFFFFFFFFu;
  vpd[i] = 0.0f;
  // the queries without a list share one count (hist[2 nlist]): one atomic a wave
  const uint64_t bm = __ballot(!use);
  int base = 0;
  if (bm) {
    const int lead = __builtin_ctzll(bm);
    if ((int)(threadIdx.x & 63) == lead) base = atomicAdd(&hist[2 * nlist], __popcll(bm));
    base = __shfl(base, lead, kWave);
  }
  rank[i] = use ? atomicAdd(&hist[l], 1) : base + __popcll(bm & ((1ull << (threadIdx.x & 63)) - 1ull));
}

// The virtual queries grouped by list: list l's take order[boff[l] ..
// boff[l + 1]) by their rank in it, those without a usable list the slots
// from boff[nlist] on.
__global__ __launch_bounds__(256) void tp_order_kernel(const uint32_t* __restrict__ vprobe,
                                                       const int32_t* __restrict__ rank, int nvq, int nlist,
                                                       const int32_t* __restrict__ boff, int32_t* __restrict__ order) {
  const int v = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (v >= nvq) return;
  const uint32_t l = vprobe[v];
  order[boff[l < (uint32_t)nlist ? l : (uint32_t)nlist] + rank[v]] = v;
}

// boff[l] = hist[0] + ... + hist[l - 1] for l = 0 .. nlist (one workgroup,
// nlist <= 8192: each thread sums 8 consecutive counts), and the screen's
// single-probe counts sp_cnt[l] = hist[l] for lists of at least k vectors, 0
// for the shorter ones (their queries take the list's vectors directly).
__global__ __launch_bounds__(1024) void tp_offsets_kernel(const int* __restrict__ hist, int nlist,
                                                          int32_t* __restrict__ boff,
                                                          const int32_t* __restrict__ offsets, int k,
                                                          int32_t* __restrict__ sp_cnt) {
  __shared__ int wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int v[8], sum = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int l = tid * 8 + i;
    v[i] = l < nlist ? hist[l] : 0;
    sum += v[i];
    if (l < nlist) sp_cnt[l] = offsets[l + 1] - offsets[l] >= k ? v[i] : 0;
  }
  const int incl = wave_incl_scan(sum);
  if (lane == kWave - 1) wsum[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int x = lane < 16 ? wsum[lane] : 0;
    x = wave_incl_scan(x);
    if (lane < 16) wsum[lane] = x;
  }
  __syncthreads();
  int base = (wave > 0 ? wsum[wave - 1] : 0) + incl - sum;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int l = tid * 8 + i;
    if (l <= nlist) boff[l] = base;
    base += v[i];
  }
}

// The second half of the two-phase scan when phase 1 ran through the screen,
// one wave a query (queries q_base + ql, ql < nqc; probe p's phase-1 result
// is virtual query ql p1 + p's ascending top-limit_k in vids/vd).  As the
// two-phase kernel's mode 2 does: each phase-1 cutoff is the w-th distance of
// a usable phase-1 probe (w = min(n, limit_k); 0 for the others) and the
// threshold is coeff times the smallest positive cutoff.  Then every usable
// phase-2 list's lower bound (list_lower_bound of the coarse step's probe
// distance, or of a wave-wide fp32 sum of the squared residual; any valid
// bound skips the same lists' appends, since none of their vectors reaches
// the threshold): when
// none is <= thr (1 + 2^-16) -- the mode-2 skip test -- phase 2 appends
// nothing, and when the phase-1 keys also fit rerank_m they are the answer,
// sorted: each usable phase-1 probe's keys are one 64-lane vector (padded
// with kNoKey, odd vectors reversed), and a bitonic network over the vectors
// (across vectors elementwise, within one by lane exchanges) sorts them, as
// the mode-2 final sort does (equal keys are equal outputs); then padding to
// rerank_m.  Other queries (a list that can reach the threshold, more keys
// than rerank_m, more than kFinRuns phase-1 lists) get their pool slots and
// cutoffs as the split phase 1 leaves them and go to slow_list.
constexpr int kFinWaves = 4;
constexpr int kFinRuns = 16;  // usable phase-1 probes the wave sorts (64-key vectors)

// Ascending sort of the NV x 64 keys x[v] (lane j: flat position 64 v + j),
// each vector already sorted, ascending for even v and descending for odd v.
template <int NV>
__device__ __forceinline__ void wave_sort_vectors(uint64_t (&x)[NV]) {
#pragma unroll
  for (int size = 128; size <= 64 * NV; size <<= 1) {
#pragma unroll
    for (int sv = size / 128; sv >= 1; sv >>= 1) {
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        if ((v & sv) == 0) {
          const bool up = size == 64 * NV || ((64 * v) & size) == 0;
          const uint64_t p = x[v], q = x[v + sv];
          const bool sw = (p > q) == up;
          x[v] = sw ? q : p;
          x[v + sv] = sw ? p : q;
        }
      }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) bitonic_pass_k<64>(x[v], size == 64 * NV || ((64 * v) & size) == 0);
  }
}

template <int NV>
__device__ __forceinline__ void fin_sort_write(const TwoPhaseArgs& a, int q, int ql, int nrun, int total,
                                               const int* rp, const int* rw, const int32_t* __restrict__ vids,
                                               const float* __restrict__ vd) {
  const int lane = threadIdx.x & 63;
  const int p1 = a.p1, K1 = a.limit_k;
  uint64_t x[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    x[v] = kNoKey;
    if (v < nrun) {
      const int w = rw[v];
      // even vectors ascending (keys, then padding), odd ones descending
      const int j = (v & 1) ? kWave - 1 - lane : lane;
      if (j < w) {
        const size_t e = ((size_t)ql * p1 + rp[v]) * K1 + j;
        x[v] = key_of(vd[e], vids[e]);
      }
    }
  }
  wave_sort_vectors<NV>(x);
  int32_t* out_id = a.top_ids + (size_t)q * a.rerank_m;
  float* out_d = a.top_d + (size_t)q * a.rerank_m;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = v * kWave + lane;
    if (i < total) {
      out_id[i] = (int32_t)(uint32_t)x[v];
      out_d[i] = __uint_as_float((uint32_t)(x[v] >> 32));
    }
  }
}

__global__ __launch_bounds__(kFinWaves * kWave) void tp_finish_kernel(TwoPhaseArgs a, int dim, int q_base, int nqc,
                                                                      const int32_t* __restrict__ vids,
                                                                      const float* __restrict__ vd,
                                                                      const float* __restrict__ pd,
                                                                      int32_t* __restrict__ slow_list,
                                                                      int* __restrict__ slow_cnt) {
  __shared__ int rp[kFinWaves][kFinRuns];  // vector (run) -> phase-1 probe index
  __shared__ int rw[kFinWaves][kFinRuns];  // its key count
  const int lane = threadIdx.x & 63, wv = (int)(threadIdx.x >> 6);
  const int ql = (int)blockIdx.x * kFinWaves + wv;
  if (ql >= nqc) return;  // no workgroup barrier below
  const int q = q_base + ql;
  const int P = a.nprobe, p1 = a.p1, K1 = a.limit_k, R = a.rerank_m;
  const uint32_t NL = (uint32_t)a.nlist;
  const uint32_t* pr = a.probes + (size_t)q * P;
  float mcut = FLT_MAX;
  int nrun = 0, total = 0;
  for (int c0 = 0; c0 < p1; c0 += kWave) {
    const int p = c0 + lane;
    int w = 0;
    float cut = 0.0f;
    if (p < p1) {
      const uint32_t l = pr[p];
      if (l < NL) {
        const int n = a.offsets[l + 1] - a.offsets[l];
        w = n < K1 ? n : K1;
      }
      if (w > 0) cut = vd[((size_t)ql * p1 + p) * K1 + w - 1];
      if (a.cutoffs) a.cutoffs[(size_t)q * p1 + p] = cut;
    }
    if (cut > 0.0f && cut < mcut) mcut = cut;
    const uint64_t bm = __ballot(w > 0);
    const int idx = nrun + __popcll(bm & ((1ull << lane) - 1ull));
    if (w > 0 && idx < kFinRuns) {
      rp[wv][idx] = p;
      rw[wv][idx] = w;
    }
    nrun += __popcll(bm);
    total += wave_sum_i(w);
  }
  mcut = wave_min_f(mcut);
  const float thr = mcut < FLT_MAX ? mcut * a.coeff : FLT_MAX;
  const float thr_hi = thr * (1.0f + 0x1p-16f);
  bool slow = nrun > kFinRuns || total > R;
  int skipped = 0;
  // this lane's two query dims (without probe distances, each list's residual
  // norm is one wave-wide sum over a coalesced read of its centroid row)
  const bool dl = 2 * lane < dim;
  const float2 qd = !pd && dl ? reinterpret_cast<const float2*>(a.queries + (size_t)q * dim)[lane]
                              : make_float2(0.0f, 0.0f);
  for (int c0 = p1; !slow && c0 < P; c0 += kWave) {
    const int p = c0 + lane;
    uint32_t l = NL;
    bool use = false;
    if (p < P) {
      l = pr[p];
      use = l < NL && a.offsets[l + 1] > a.offsets[l];
    }
    float s2 = 0.0f;
    if (pd) {
      if (use) s2 = pd[(size_t)q * P + p];
    } else {
      uint64_t m = __ballot(use);
      while (m) {  // four lists at a time: their row loads in flight together
        int b[4];
        float2 cv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          b[k] = m ? __builtin_ctzll(m) : -1;
          if (m) m &= m - 1;
          const uint32_t lk = b[k] >= 0 ? (uint32_t)__builtin_amdgcn_readlane((int)l, b[k]) : 0u;
          cv[k] = b[k] >= 0 && dl ? reinterpret_cast<const float2*>(a.centroids + (size_t)lk * dim)[lane]
                                  : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float r0 = dl ? qd.x - cv[k].x : 0.0f, r1 = dl ? qd.y - cv[k].y : 0.0f;
          const float v = wave_sum_f(__builtin_fmaf(r1, r1, r0 * r0));
          if (lane == b[k]) s2 = v;
        }
      }
    }
    const bool reach = use && list_lower_bound(s2, a.rmax[use ? l : 0]) <= thr_hi;
    slow = __ballot(reach) != 0;
    skipped += __popcll(__ballot(use));
  }
  if (slow) {
    int base = 0;
    for (int c0 = 0; c0 < p1; c0 += kWave) {
      const int p = c0 + lane;
      int w = 0;
      if (p < p1) {
        const uint32_t l = pr[p];
        if (l < NL) {
          const int n = a.offsets[l + 1] - a.offsets[l];
          w = n < K1 ? n : K1;
        }
      }
      const int incl = wave_incl_scan(w);
      const int mine = base + incl - w;
      uint64_t m = __ballot(w > 0);
      while (m) {
        const int b = __ffsll((unsigned long long)m) - 1;
        m &= m - 1;
        const int wb = readlane_i(w, b), bb = readlane_i(mine, b);
        const size_t v = ((size_t)ql * p1 + c0 + b) * K1;
        if (lane < wb) a.pool[(size_t)q * a.pool_cap + bb + lane] = key_of(vd[v + lane], vids[v + lane]);
        if (lane == 0) a.cut_ws[(size_t)q * P + c0 + b] = vd[v + wb - 1];
      }
      base += readlane_i(incl, kWave - 1);
    }
    if (lane == 0) slow_list[atomicAdd(slow_cnt, 1)] = q;
    return;
  }
  if (lane == 0) {
    if (a.thr) a.thr[q] = thr;
    if (a.pre_cut) a.pre_cut[q] = total;
    a.top_counts[q] = total;
    if (a.stats && skipped) atomicAdd(&a.stats[2], (unsigned long long)skipped);
  }
  wave_lds_sync();  // rp, rw
  if (nrun <= 1)
    fin_sort_write<1>(a, q, ql, nrun, total, rp[wv], rw[wv], vids, vd);
  else if (nrun <= 2)
    fin_sort_write<2>(a, q, ql, nrun, total, rp[wv], rw[wv], vids, vd);
  else if (nrun <= 4)
    fin_sort_write<4>(a, q, ql, nrun, total, rp[wv], rw[wv], vids, vd);
  else if (nrun <= 8)
    fin_sort_write<8>(a, q, ql, nrun, total, rp[wv], rw[wv], vids, vd);
  else
    fin_sort_write<16>(a, q, ql, nrun, total, rp[wv], rw[wv], vids, vd);
  int32_t* out_id = a.top_ids + (size_t)q * R;
  float* out_d = a.top_d + (size_t)q * R;
  for (int j = total + lane; j < R; j += kWave) {
    out_id[j] = -1;
    out_d[j] = FLT_MAX;
  }
}

// Instrumentation of phase 1 through the screen: stats[11] += virtual
// queries, [12] += their candidates (every count, also past the cap), [13] +=
// those handed to the LUT kernel, [14] += those without a threshold, [15] +=
// those with more candidates than cap; per list l (cnt1/cnt2: its virtual
// queries in rounds 1 and 2, at most its bucket's length), [16]/[17] +=
// (query, vector) pairs screened in round 1/2 and [18]/[19] += 32 x 32 MFMA
// tiles run.
__global__ __launch_bounds__(256) void tp_stats_kernel(const int* __restrict__ cand_cnt, const float* __restrict__ thr,
                                                       int nvq, int cap, const int* __restrict__ flag_cnt,
                                                       const int* __restrict__ cnt1, const int* __restrict__ cnt2,
                                                       const int32_t* __restrict__ boff,
                                                       const int32_t* __restrict__ offsets, int nlist,
                                                       unsigned long long* __restrict__ stats) {
  const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
  const int c = i < nvq ? cand_cnt[i] : 0;
  const bool no_t = i < nvq && !(thr[i] < INFINITY);
  const int sc = wave_sum_i(c), sn = wave_sum_i(no_t ? 1 : 0), so = wave_sum_i(!no_t && c > cap ? 1 : 0);
  if ((threadIdx.x & 63) == 0) {
    if (sc) atomicAdd(&stats[12], (unsigned long long)sc);
    if (sn) atomicAdd(&stats[14], (unsigned long long)sn);
    if (so) atomicAdd(&stats[15], (unsigned long long)so);
  }
  if (i < nlist) {
    const long long n = offsets[i + 1] - offsets[i], len = boff[i + 1] - boff[i];
    const long long c1 = min((long long)cnt1[i], len), c2 = min((long long)cnt2[i], len);
    if (c1 > 0) {
      atomicAdd(&stats[16], (unsigned long long)(c1 * n));
      atomicAdd(&stats[18], (unsigned long long)((c1 + 31) / 32 * ((n + 31) / 32)));
    }
    if (c2 > 0) {
      atomicAdd(&stats[17], (unsigned long long)(c2 * n));
      atomicAdd(&stats[19], (unsigned long long)((c2 + 31) / 32 * ((n + 31) / 32)));
    }
  }
  if (i == 0) {
    atomicAdd(&stats[11], (unsigned long long)nvq);
    atomicAdd(&stats[13], (unsigned long long)*flag_cnt);
  }
}

template <int D, int M>
fgpu_status launch_tp_after(const TwoPhaseArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((two_phase_kernel<D, M, 2>), dim3((unsigned)a.nq), dim3(kTT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

template <int D>
fgpu_status launch_rr(const RerankArgs& a, hipStream_t s) {
  if (rerank_spec(a.nq, a.spec) > 1) {
    hipLaunchKernelGGL((rerank_kernel<D, 4>), dim3((unsigned)a.nq), dim3(kRT * 4), 0, s, a);
    FGPU_HIP(hipGetLastError());
    return FGPU_OK;
  }
  hipLaunchKernelGGL((rerank_kernel<D, 1>), dim3((unsigned)a.nq), dim3(kRT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace

int two_phase_pool_cap(int p1, int limit_k, int rerank_m) {
  // limit_k > 64 keeps each phase-1 list's keys in the pool while it is cut
  // to its limit_k best, so every list needs 2048 free slots above them.
  const int extra = limit_k > kWave ? p1 * limit_k + 2048 : (p1 * limit_k > 2048 ? p1 * limit_k : 2048);
  return (rerank_m + extra + 63) / 64 * 64;
}

// CUs of the current device (cached per device).
static int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

// Mini-batches the rerank computes a step: four while the batch leaves CUs
// free (one 512-thread workgroup a query, latency-bound row loads), else one
// (a large batch is bound by the row reads, and work past a stop is wasted).
// force: 0 automatic, 1 one, anything else four.
int rerank_spec(int nq, int force) {
  if (force == 1) return 1;
  if (force > 1) return 4;
  return nq <= cu_count() ? 4 : 1;
}

// force: 0 automatic, 1 never split, s >= 2 split phase 1 s ways (at most p1).
int two_phase_split(int nq, int p1, int limit_k, int force) {
  if (limit_k > kWave || p1 < 2 || nq <= 0 || force == 1) return 1;
  if (force > 1) return std::min(p1, force);
  const int slots = 2 * cu_count();  // two_phase_kernel workgroups resident at once
  return nq >= slots ? 1 : std::min(p1, std::max(1, slots / nq));
}

fgpu_status launch_two_phase(int dim, int m, const TwoPhaseArgs& a, hipStream_t s) {
  FGPU_CHECK(a.limit_k >= 1 && a.limit_k <= kMaxLimitK, FGPU_ERR_UNSUPPORTED, "two_phase: limit_k must be in [1, 4096]");
  FGPU_CHECK(a.rerank_m >= 1 && a.rerank_m <= kRerankMax, FGPU_ERR_UNSUPPORTED,
             "two_phase: rerank_m must be in [1, 131072]");
  FGPU_CHECK(a.nprobe >= 1 && a.nprobe <= kMaxProbes && a.p1 >= 0 && a.p1 <= a.nprobe, FGPU_ERR_ARG,
             "two_phase: need 1 <= nprobe <= 256 and 0 <= p1 <= nprobe");
  FGPU_CHECK(a.pool_cap >= two_phase_pool_cap(a.p1, a.limit_k, a.rerank_m), FGPU_ERR_ARG, "two_phase: pool too small");
  if (a.nq <= 0) return FGPU_OK;
  const int nq = a.nq;
  if (dim == 128 && m == 32) return launch_tp<128, 32>(a, nq, s);
  if (dim == 128 && m == 16) return launch_tp<128, 16>(a, nq, s);
  if (dim == 128 && m == 64) return launch_tp<128, 64>(a, nq, s);
  if (dim == 96 && m == 48) return launch_tp<96, 48>(a, nq, s);
  if (dim == 96 && m == 32) return launch_tp<96, 32>(a, nq, s);
  if (dim == 96 && m == 16) return launch_tp<96, 16>(a, nq, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "two_phase: unsupported (dim, pq_m)");
}

fgpu_status launch_tp_virtual(const uint32_t* probes, int nprobe, int p1, int nqc, const int32_t* offsets, int nlist,
                              uint32_t* vprobe, float* vpd, int* hist, int32_t* rank, hipStream_t s) {
  FGPU_CHECK(p1 >= 1 && nlist >= 1 && nlist <= 8192 && (int64_t)nqc * p1 < INT32_MAX, FGPU_ERR_ARG,
             "two_phase: bad virtual queries");
  if (nqc <= 0) return FGPU_OK;
  // hist: the list counts, nlist unused ints, the count of those without a list
  hipLaunchKernelGGL(tp_zero_kernel, dim3((unsigned)((2 * nlist + 1 + 255) / 256)), dim3(256), 0, s, hist,
                     2 * nlist + 1);
  const int nvq = nqc * p1;
  hipLaunchKernelGGL(tp_virtual_kernel, dim3((unsigned)((nvq + 255) / 256)), dim3(256), 0, s, probes, nprobe, p1, nvq,
                     offsets, nlist, vprobe, vpd, hist, rank);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_tp_offsets(const int* hist, int nlist, int32_t* boff, const int32_t* offsets, int k,
                              int32_t* sp_cnt, hipStream_t s) {
  FGPU_CHECK(nlist >= 1 && nlist <= 8192, FGPU_ERR_ARG, "two_phase: bad list count");
  hipLaunchKernelGGL(tp_offsets_kernel, dim3(1), dim3(1024), 0, s, hist, nlist, boff, offsets, k, sp_cnt);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_tp_finish(const TwoPhaseArgs& a, int dim, int q_base, int nqc, const int32_t* vids, const float* vd,
                             const float* probe_dists, int32_t* slow_list, int* slow_cnt, hipStream_t s) {
  FGPU_CHECK(dim % 4 == 0 && dim <= 2 * kWave && a.limit_k >= 1 && a.limit_k <= kWave && a.cut_ws && a.pool,
             FGPU_ERR_ARG, "two_phase: bad finish arguments");
  if (nqc <= 0) return FGPU_OK;
  hipLaunchKernelGGL(tp_finish_kernel, dim3((unsigned)((nqc + kFinWaves - 1) / kFinWaves)), dim3(kFinWaves * kWave), 0,
                     s, a, dim, q_base, nqc, vids, vd, probe_dists, slow_list, slow_cnt);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_tp_zero(int* p, int n, hipStream_t s) {
  if (n <= 0) return FGPU_OK;
  hipLaunchKernelGGL(tp_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_tp_order(const uint32_t* vprobe, const int32_t* rank, int nvq, int nlist, const int32_t* boff,
                            int32_t* order, hipStream_t s) {
  if (nvq <= 0) return FGPU_OK;
  hipLaunchKernelGGL(tp_order_kernel, dim3((unsigned)((nvq + 255) / 256)), dim3(256), 0, s, vprobe, rank, nvq, nlist,
                     boff, order);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_tp_stats(const int* cand_cnt, const float* thr, int nvq, int cap, const int* flag_cnt,
                            const int* cnt1, const int* cnt2, const int32_t* boff, const int32_t* offsets, int nlist,
                            unsigned long long* stats, hipStream_t s) {
  if (nvq <= 0 || !stats) return FGPU_OK;
  const int nt = std::max(nvq, nlist);
  hipLaunchKernelGGL(tp_stats_kernel, dim3((unsigned)((nt + 255) / 256)), dim3(256), 0, s, cand_cnt, thr, nvq, cap,
                     flag_cnt, cnt1, cnt2, boff, offsets, nlist, stats);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

fgpu_status launch_two_phase_after_phase1(int dim, int m, const TwoPhaseArgs& a, hipStream_t s) {
  FGPU_CHECK(a.limit_k >= 1 && a.limit_k <= kWave && a.cut_ws, FGPU_ERR_ARG,
             "two_phase: phase 2 after a separate phase 1 needs limit_k <= 64 and the cutoff rows");
  FGPU_CHECK(a.rerank_m >= 1 && a.rerank_m <= kRerankMax, FGPU_ERR_UNSUPPORTED,
             "two_phase: rerank_m must be in [1, 131072]");
  FGPU_CHECK(a.nprobe >= 1 && a.nprobe <= kMaxProbes && a.p1 >= 0 && a.p1 <= a.nprobe, FGPU_ERR_ARG,
             "two_phase: need 1 <= nprobe <= 256 and 0 <= p1 <= nprobe");
  FGPU_CHECK(a.pool_cap >= two_phase_pool_cap(a.p1, a.limit_k, a.rerank_m), FGPU_ERR_ARG, "two_phase: pool too small");
  if (a.nq <= 0) return FGPU_OK;
  if (dim == 128 && m == 32) return launch_tp_after<128, 32>(a, s);
  if (dim == 128 && m == 16) return launch_tp_after<128, 16>(a, s);
  if (dim == 128 && m == 64) return launch_tp_after<128, 64>(a, s);
  if (dim == 96 && m == 48) return launch_tp_after<96, 48>(a, s);
  if (dim == 96 && m == 32) return launch_tp_after<96, 32>(a, s);
  if (dim == 96 && m == 16) return launch_tp_after<96, 16>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "two_phase: unsupported (dim, pq_m)");
}

fgpu_status launch_rerank(int dim, const RerankArgs& a, hipStream_t s) {
  FGPU_CHECK(a.k >= 1 && a.k <= 256, FGPU_ERR_UNSUPPORTED, "rerank: k must be in [1, 256]");
  FGPU_CHECK(a.mb >= 1 && a.mb <= kRT, FGPU_ERR_UNSUPPORTED, "rerank: mini_batch must be in [1, 128]");
  if (a.nq <= 0) return FGPU_OK;
  if (dim == 128) return launch_rr<128>(a, s);
  if (dim == 96) return launch_rr<96>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "rerank: dim must be 96 or 128");
}

}  // namespace fgpu
