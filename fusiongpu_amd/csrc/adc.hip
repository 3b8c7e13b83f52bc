// adc.hip -- per-query LUT build in LDS, ADC scan over the probed inverted
// lists and top-k selection (A4, A5, A6, A10 in plain IVF-PQ form).
//
// Reference: batch_residual_precompute_kernel (gpu_global.cu:79-166) writes
// every (query, probe) LUT to global memory; ivf_scan_phase1_kernel
// (gpu_global.cu:321-390) scans at most 1024 items of a list per block and
// sorts them with a CUB block radix sort; a segmented radix sort then orders
// the union (gpu_global.cu:852-861).
//
// Here one workgroup owns one query and walks its probed lists in coarse
// order:
//   * LUT[m][k] lives in LDS ([m][256] floats).  The threads that build it
//     keep the codebook sub-vectors of their codeword in registers for the
//     whole query, so the codebook is read from HBM once per workgroup.
//     Entries use the reference's exact fused chains (gpu_global.cu:115-158),
//     so they are bit-identical.
//   * The scan streams each vector's pq_m code bytes with 128-bit loads, two
//     vectors per lane per round (two independent ADC chains in flight).  Each
//     distance sums LUT[m][code_m] in ascending m as the reference does
//     (gpu_global.cu:196-253): one SDWA byte-to-address shift and one
//     ds_read_b32 with an immediate row offset per term.
//   * Each scanning wave keeps its own running top-64 (one (distance, id) per
//     lane, sorted by the tie rule).  A vector is a candidate only if its
//     (distance, id) beats the smallest k-th entry over all scanning waves,
//     kept in LDS with a 64-bit atomic min; ids are loaded with the codes, so
//     the test is one 64-bit compare with no dependent load.  After the first
//     list almost nothing passes.  Few passers are inserted one by one; many
//     are bitonic-sorted and merged.  At the end the wave lists are merged.
//   * adc_flow_kernel (pq_m <= 32): 16 waves; 8 build the LUTs of the coming
//     lists into two LDS buffers while 8 scan, handing buffers over through
//     LDS counters instead of workgroup barriers.
//     adc_plain_kernel (pq_m 48, 64): 8 waves alternate build and scan.
#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "kernels.hpp"
#include "scan_common.hpp"

namespace fgpu {
namespace {

// Scan one list with the LUT at a compile-time LDS position.  w0/w1 (i0/i1)
// hold the codes (ids) of this wave's first round, loaded by the caller ahead
// of time; with PREFETCH later rounds are loaded one round ahead, otherwise at
// round start.  `own` is this wave's k-th best as a packed key; `s_thr` is the
// workgroup-wide minimum of those keys, shared through LDS: a vector that does
// not beat it cannot enter the query's top-k, because k vectors seen by some
// wave already do.
template <int D, int M, int BUF, int SCAN_WAVES, bool PREFETCH>
__device__ __forceinline__ void scan_list(const float* smem, const uint8_t* __restrict__ codes,
                                          const int32_t* __restrict__ ids, int start, int n, int k, int swave,
                                          uint4 (&w0)[M / 16], uint4 (&w1)[M / 16], int& i0, int& i1, uint64_t& lk,
                                          uint64_t& own, unsigned long long* s_thr) {
  using C = Cfg<D, M>;
  constexpr int kRound = SCAN_WAVES * kVecPerWaveRound;
  const float* lut = smem + BUF * C::LUT;
  const int lane = threadIdx.x & 63;
  for (int base = swave * kVecPerWaveRound; base < n; base += kRound) {
    const int v0 = base + lane, v1 = v0 + kWave;
    uint4 n0[C::NV4], n1[C::NV4];
    int j0 = kPadId, j1 = kPadId;
    const bool more = base + kRound < n;
    if (PREFETCH) {
      if (more) load_pair<M>(codes, ids, start, n, v0 + kRound, n0, n1, j0, j1);
    } else if (base != swave * kVecPerWaveRound) {
      load_pair<M>(codes, ids, start, n, v0, w0, w1, i0, i1);
    }
    const uint64_t shared_thr = *s_thr;
    uint64_t thr = own < shared_thr ? own : shared_thr;
    float d0, d1;
    if (adc_sum2<M>(lut, w0, w1, v0 < n, v1 < n, __uint_as_float((uint32_t)(thr >> 32)), d0, d1)) {
      if (offer2_k(v0 < n ? key_of(d0, i0) : kPadKey, v1 < n ? key_of(d1, i1) : kPadKey, thr, k, lk)) {
        own = readlane64(lk, k - 1);
        if (lane == 0) atomicMin(s_thr, (unsigned long long)own);
      }
    }
    if (PREFETCH && more) {
#pragma unroll
      for (int i = 0; i < C::NV4; ++i) { w0[i] = n0[i]; w1[i] = n1[i]; }
      i0 = j0;
      i1 = j1;
    }
  }
}

// One full scanner round: thr is the packed k-th key this wave filters
// against (own or shared, whichever is smaller).
template <int D, int M, int BUF>
__device__ __forceinline__ void scan_round_full(const float* smem, int v0, int n, int k, const uint4 (&w0)[M / 16],
                                                const uint4 (&w1)[M / 16], int i0, int i1, uint64_t thr,
                                                uint64_t& lk, uint64_t& own, unsigned long long* s_thr) {
  using C = Cfg<D, M>;
  const float* lut = smem + BUF * C::LUT;
  const int v1 = v0 + kWave;
  float d0, d1;
  bool go = true;
  if (v0 - (int)(threadIdx.x & 63) + 2 * kWave <= n)  // a full chunk (uniform)
    go = adc_sum2_full<M>(lut, w0, w1, __uint_as_float((uint32_t)(thr >> 32)), d0, d1);
  else  // the list's partial last chunk: empty lanes send no gathers (C2: 0.444 -> 0.440 ms)
    adc_sum2_part<M>(lut, w0, w1, v0 < n, v1 < n, d0, d1);
  if (go) {
    if (offer2_k(v0 < n ? key_of(d0, i0) : kPadKey, v1 < n ? key_of(d1, i1) : kPadKey, thr, k, lk)) {
      own = readlane64(lk, k - 1);
      if ((threadIdx.x & 63) == 0) atomicMin(s_thr, (unsigned long long)own);
    }
  }
}

// Workgroup-local hand-off through LDS counters.  The waits are bounded: a
// wave that has polled `limit` times gives up and carries on, so every wave
// reaches the end of the kernel whatever the counters say.  The limit
// (flow_spin_limit) is far above the longest legitimate wait, the scan of
// every probed list of a query.  A give-up is never silent: the wave adds 1 to
// the device counter a.faults and sets the workgroup's LDS flag, and every
// query whose top-k the workgroup writes after that gets kFaultId / NaN in all
// its slots.  Queries written before the flag was set were complete, so no
// later give-up can have touched them.
// Each poll is an LDS read and a few VALU instructions taken from the waves
// that do the work, so waits off the critical path (builders waiting for
// scanners) poll kLazySleep times less often: s_sleep N idles about 64 N
// clocks.
constexpr int kLazySleep = 8;

struct WaitCtl {
  int limit;                   // polls of s_sleep 1 before a give-up
  int* flag;                   // the workgroup's LDS give-up flag
  unsigned long long* faults;  // device give-up counter
};

__device__ __forceinline__ void note_give_up(const WaitCtl& w) {
  if ((threadIdx.x & 63) == 0) {
    __hip_atomic_store(w.flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    atomicAdd(w.faults, 1ull);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
}

template <int SLEEP = 1>
__device__ __forceinline__ void lds_wait_at_least(const int* p, int target, const WaitCtl& w) {
  int spins = 0;
  while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    if (++spins >= w.limit / SLEEP) {
      note_give_up(w);
      break;
    }
    __builtin_amdgcn_s_sleep(SLEEP);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Publish this wave's earlier LDS reads and writes, then add `v` to *p.
__device__ __forceinline__ void lds_signal_add(int* p, int v) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Write the k best of a sorted wave list (padding as id -1, distance FLT_MAX;
// with `fault`, every slot kFaultId / NaN).
__device__ __forceinline__ void write_topk(uint64_t lk, int q, int k, const AdcArgs& a, bool fault = false) {
  const int lane = threadIdx.x & 63;
  if (lane < k) {
    const int id = key_id(lk);
    const bool pad = id == kPadId;
    a.out_ids[(size_t)q * k + lane] = fault ? kFaultId : pad ? -1 : id;
    a.out_d[(size_t)q * k + lane] = fault ? __builtin_nanf("") : pad ? FLT_MAX : key_dist(lk);
  }
}

// Merge `nw` sorted wave lists held in LDS (64 keys each) into this wave's
// registers and write the k best.
__device__ __forceinline__ void merge_and_write(uint64_t lk, const uint64_t* mk, int nw, int q, int k,
                                                const AdcArgs& a) {
  const int lane = threadIdx.x & 63;
#pragma unroll 1
  for (int w = 1; w < nw; ++w) wave_merge_sorted64_k(lk, mk[w * kWave + lane]);
  write_topk(lk, q, k, a);
}

// ---------------------------------------------------------------------------
// Generic kernel: 8 waves build the LUT together (thread t owns codeword t%256
// for half of the subspaces), then all 8 scan.
constexpr int kNW = 8;
constexpr int kNT = kNW * kWave;

// One query of the generic kernel (the whole workgroup).
template <int D, int M>
__device__ __forceinline__ void plain_query(const AdcArgs& a, int q, float* smem, unsigned long long& s_thr) {
  using C = Cfg<D, M>;
  constexpr int G = kNT / kPQK;  // threads sharing one codeword
  constexpr int MG = M / G;      // subspaces per thread
  static_assert(M % G == 0, "pq_m must split across the codeword threads");
  float* rbuf = smem + C::R_OFF;
  float* qs = smem + C::Q_OFF;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kc = tid & (kPQK - 1), g = tid / kPQK;
  if (tid == 0) s_thr = kNoThr;
  const int P = a.nprobe, k = a.k;
  const uint32_t NL = (uint32_t)a.nlist;

  float cb[MG * C::S];
#pragma unroll
  for (int mm = 0; mm < MG; ++mm) {
    const float* src = a.codebook + ((size_t)(g * MG + mm) * kPQK + kc) * C::S;
#pragma unroll
    for (int j = 0; j < C::S; ++j) cb[mm * C::S + j] = src[j];
  }
  for (int i = tid; i < D; i += kNT) qs[i] = a.queries[(size_t)(q / a.qdiv) * D + i];
  const uint32_t* probes = a.probes + (size_t)q * P;
  __syncthreads();

  int p = 0;
  while (p < P && probes[p] >= NL) ++p;  // pruned (0xFFFFFFFF) or out of range
  if (p < P && tid < D) rbuf[tid] = qs[tid] - a.centroids[(size_t)probes[p] * D + tid];
  __syncthreads();

  uint64_t lk = kPadKey;
  uint64_t own = kNoThr;
  int it = 0;
  uint4 w0[C::NV4], w1[C::NV4];
  int i0 = kPadId, i1 = kPadId;
  while (p < P) {
    const uint32_t l = probes[p];
    int pn = p + 1;
    while (pn < P && probes[pn] >= NL) ++pn;
    const int start = a.offsets[l];
    const int n = a.offsets[l + 1] - start;
    // First-round code loads go out before the LUT build, which hides their latency.
    load_pair<M>(a.codes, a.vec_ids, start, n, wave * kVecPerWaveRound + lane, w0, w1, i0, i1);
    const int buf = C::DBUF ? (it & 1) : 0;
    float* lut = smem + buf * C::LUT;
    const float* r = rbuf + (it & 1) * D;
#pragma unroll
    for (int mm = 0; mm < MG; ++mm) {
      const int m = g * MG + mm;
      float rr[C::S];
#pragma unroll
      for (int j = 0; j < C::S; ++j) rr[j] = r[m * C::S + j];
      lut[m * kPQK + kc] = lut_entry<C::S>(rr, cb + mm * C::S);
    }
    if (pn < P && tid < D) rbuf[((it + 1) & 1) * D + tid] = qs[tid] - a.centroids[(size_t)probes[pn] * D + tid];
    __syncthreads();
    if (buf == 0)
      scan_list<D, M, 0, kNW, false>(smem, a.codes, a.vec_ids, start, n, k, wave, w0, w1, i0, i1, lk, own, &s_thr);
    else
      scan_list<D, M, (C::DBUF ? 1 : 0), kNW, false>(smem, a.codes, a.vec_ids, start, n, k, wave, w0, w1, i0, i1, lk,
                                                    own, &s_thr);
    if (!C::DBUF) __syncthreads();
    p = pn;
    ++it;
    if (a.stats && tid == 0) atomicAdd(&a.stats[0], (unsigned long long)n);
  }
  if (a.stats && tid == 0) atomicAdd(&a.stats[1], (unsigned long long)it);

  __syncthreads();
  uint64_t* mk = reinterpret_cast<uint64_t*>(smem);
  mk[wave * kWave + lane] = lk;
  __syncthreads();
  if (wave == 0) merge_and_write(lk, mk, kNW, q, k, a);
}

template <int D, int M>
__global__ __launch_bounds__(kNT) void adc_plain_kernel(AdcArgs a) {
  __shared__ __align__(16) float smem[Cfg<D, M>::SMEM];
  __shared__ unsigned long long s_thr;
  plain_query<D, M>(a, (int)blockIdx.x, smem, s_thr);
}

// The generic kernel over the queries a.qlist[0 .. *a.qcount): the exact LUT
// path for the queries the MFMA screen hands back.  A persistent grid; with
// an empty list every workgroup ends at once.
template <int D, int M>
__global__ __launch_bounds__(kNT) void adc_plain_list_kernel(AdcArgs a) {
  __shared__ __align__(16) float smem[Cfg<D, M>::SMEM];
  __shared__ unsigned long long s_thr;
  const int count = min(*a.qcount, a.nq);
  for (int i = (int)blockIdx.x; i < count; i += (int)gridDim.x) {
    const int q = a.qlist[i];
    if (q >= 0 && q < a.nq) plain_query<D, M>(a, q, smem, s_thr);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Wave-specialised kernels: 16 waves; waves 0-7 build LUTs (the codebook lives
// in their registers), waves 8-15 scan.
constexpr int kSpecWaves = 16;
constexpr int kBuilderWaves = 8;
constexpr int kScanWaves = kSpecWaves - kBuilderWaves;

// ---------------------------------------------------------------------------
// Decoupled wave-specialised kernel, persistent over queries: no workgroup
// barrier after the start.  Workgroup g takes queries g, g + G, g + 2G, ...
// (G = grid size, at most one workgroup per CU); the per-query state lives in
// two LDS slots used by alternate queries, so builder waves set up query i + 1
// while scanner waves are still in query i.
//   * The probed, non-empty lists are cut into chunks of 128 vectors (one
//     scanner round) and numbered in coarse order; scanner wave w takes chunks
//     w, w + 8, w + 16, ..., so a wave that finishes its part of a list moves
//     on while slower waves are still in it.
//   * Before building list f's LUT, builder wave 0 tests a lower bound on
//     every ADC distance the list can produce against the current k-th
//     distance (list_lower_bound).  A list that cannot contribute is skipped:
//     no LUT, no LDS buffer, and the scanners pass over its chunks without
//     loading codes.  Wave 0 records each decision in dec[f], and every wave
//     follows it.  Built lists are numbered j = 0, 1, ... over the workgroup's
//     whole run and use LUT buffer b = j % 3, so the builders can be two
//     lists ahead of the scanners.  Buffer 2 lies beyond the 64 KB reach of
//     the DS immediate offset, so its gathers take a base register (one more
//     VALU instruction each); the gathers are bound by LDS bank conflicts,
//     not VALU issue, and three buffers beat two (C2 ADC 0.467 -> 0.447 ms)
//     and four (0.462 ms, with staler list decisions).
//   * Builder waves write LUT j once every chunk of built list j - 3 (the
//     buffer's previous user) has been scanned, then add 1 to built[b]; a
//     scanner entering built list j waits for built[b] >= 8 (j / 3 + 1).
//   * Scanners add the chunks of a built list they finish to done[b] when they
//     leave it; the builder of list j waits for done[b] to reach the chunk
//     count of the earlier built lists of buffer b.
//   * A scanner that is through query i climbs a binary merge tree over the 8
//     scanner lists: at each node the second of the two children to arrive
//     merges both and climbs on, the first is done; nobody waits.  The
//     second arrival at the root writes the query's top-k and frees the slot.
//   * Set-up of query i (builders, once the slot's previous query is freed):
//     the list bounds come from the coarse step's probe distances when the
//     caller passes them (wave 0: probe ids and distances, then radii and
//     offsets), otherwise every builder wave computes those of its share of
//     the probes from the centroid rows; wave 0 adds offsets, compacts the
//     usable lists and marks the slot ready.
//   * A scanner round computes both of its vectors' full ADC sums and offers
//     them to the wave's top-k; on C2 a per-lane early abandon would almost
//     never stop a 128-vector round, so the list bound above is the only
//     pruning.
// All counters are cumulative.  A count cannot run ahead of the list it
// stands for: a builder wave contributes to built list j + 3 only after all of
// list j is scanned, and a scanner scans list j + 3 only after it is built, so
// the first time a threshold is met every contribution comes from earlier
// lists of that buffer.  Deadlock-free: builders decide lists in order and
// wait only on chunks of lists already built, or on the end of query i - 1
// when they set up query i + 1, whose lists were all built before query i's;
// scanners take chunks in increasing order and report a list before waiting
// on the next.  Each builder wave computes its own part of the residual, so
// builders never wait on each other outside the set-up.
constexpr int kLutBufs = 3;  // LUT buffers of the flow kernel
constexpr int kUndecided = -1;
constexpr int kSkipped = -2;

template <int SLEEP = 1>
__device__ __forceinline__ int lds_wait_decided(const int* p, const WaitCtl& w) {
  int spins = 0, v;
  while ((v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == kUndecided) {
    if (++spins >= w.limit / SLEEP) {
      note_give_up(w);
      break;
    }
    __builtin_amdgcn_s_sleep(SLEEP);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return v;
}

// list := the 64 smallest of list U the sorted list of keys held in LDS at pk.
__device__ __forceinline__ void wave_merge_lds64(uint64_t& k, const uint64_t* pk) {
  const uint64_t r = pk[kWave - 1 - (threadIdx.x & 63)];
  k = r < k ? r : k;
  bitonic_pass_k<64>(k, true);
}

template <int D, int M>
__global__ __launch_bounds__(kSpecWaves * kWave, 4) void adc_flow_kernel(AdcArgs a) {
  using C = Cfg<D, M>;
  static_assert(C::DBUF, "decoupled kernel needs two LUTs within the DS offset reach");
  static_assert(D <= 2 * kWave, "the list bound takes two residual coordinates per lane");
  constexpr int kChunk = kVecPerWaveRound;
  // Builder layout: builder wave w owns subspaces w*SPW .. w*SPW + SPW-1
  // whole: TPM lanes per subspace, each with E codewords k = 4t + 4 TPM u + j
  // (u < E/4, j < 4), so every 4 entries are one 16-byte LDS write and
  // consecutive lanes write consecutive 16 bytes.  The codebook rows of those
  // codewords stay in registers for the whole run.
  constexpr int SPW = M / kBuilderWaves;
  constexpr int TPM = kWave / SPW;
  constexpr int E = kPQK / TPM;
  constexpr int RW = SPW * C::S;  // residual floats per builder wave
  constexpr int kMaxPerWave = 64 / kBuilderWaves;  // set-up: probes per builder wave (nprobe <= 64)
  static_assert(M % kBuilderWaves == 0 && (TPM == 16 || TPM == 32) && E % 4 == 0, "builder layout");
  __shared__ __align__(16) float smem[kLutBufs * C::LUT];
  __shared__ float rws[kBuilderWaves][16];
  // Per query slot.  p_*: by probe index (set-up); f_*: compacted usable lists.
  __shared__ float p_lb[2][64];
  __shared__ int f_list[2][64], f_start[2][64], f_n[2][64], f_cst[2][65], s_dec[2][64];
  __shared__ float f_lb[2][64];  // list_lower_bound of each usable list
  __shared__ int s_nv[2];
  __shared__ unsigned long long s_thr[2];
  // Merge tree of the scanner lists: node n has two child lists; level 0 is
  // nodes 0-3 (waves 2j, 2j+1), level 1 nodes 4-5, the root node 6.
  __shared__ uint64_t s_tree[2][kScanWaves - 1][2][kWave];
  __shared__ int s_arr[2][kScanWaves - 1];  // arrivals per tree node
  __shared__ int s_ready[2], s_free[2], s_lbdone[2];
  __shared__ int s_q[2];  // query of each slot; -1 once the workgroup's queries are done
  __shared__ unsigned long long s_tend;  // instrumentation: the workgroup's end
  __shared__ int s_built[kLutBufs], s_done[kLutBufs];  // per LUT buffer
  __shared__ int s_fault;                               // a wave of this workgroup gave up a wait
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool builder = wave < kBuilderWaves;
  const long long t_start = a.stats ? clock64() : 0;
  const int P = a.nprobe, k = a.k;
  const uint32_t NL = (uint32_t)a.nlist;
  const int G = (int)gridDim.x;
  const int nqw = a.nq > (int)blockIdx.x ? (a.nq - (int)blockIdx.x + G - 1) / G : 0;  // this workgroup's queries
  // Dynamic claims: after its first query (blockIdx.x) a workgroup takes the
  // next unclaimed query from the counter a.qctr (reset to the grid size
  // before the launch), so workgroups finish within about one query of each
  // other.  Otherwise (no counter) workgroup g takes g, g + G, g + 2G, ...
  const bool dyn = a.qctr != nullptr && a.probe_dists != nullptr;

  if (tid < 2) {
    s_nv[tid] = 0;
    s_q[tid] = -1;
    s_ready[tid] = 0;
    s_free[tid] = 0;
    s_lbdone[tid] = 0;
  }
  if (tid < kLutBufs) {
    s_built[tid] = 0;
    s_done[tid] = 0;
  }
  if (tid == 0) {
    s_fault = 0;
    s_tend = 0;
  }
  const WaitCtl wc{a.spin_limit, &s_fault, a.faults};
  const int total = (int)a.total;
  __syncthreads();

  // Builder codebook registers: loaded first, so the loads overlap the set-up.
  const int ms = wave * SPW + lane / TPM, t = lane % TPM;
  float cb[E * C::S];
  if (builder) {
#pragma unroll
    for (int u = 0; u < E / 4; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float* src = a.codebook + ((size_t)ms * kPQK + 4 * t + 4 * TPM * u + j) * C::S;
#pragma unroll
        for (int d = 0; d < C::S; ++d) cb[(4 * u + j) * C::S + d] = src[d];
      }
    }
  }

  // First usable list >= from (below nv) of slot s whose decision is not
  // "skipped" and for which `want` holds; nv if none.  One LDS round trip for
  // up to 64 lists.
  auto next_list = [&](int s, int nv, int from, auto want) {
    const int g = from + lane;
    const bool cand = g < nv && want(g) && __hip_atomic_load(&s_dec[s][g], __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_WORKGROUP) != kSkipped;
    const uint64_t bm = __ballot(cand);
    return bm ? from + __ffsll((unsigned long long)bm) - 1 : nv;
  };

  if (builder) {
    float* rw = rws[wave];
    auto any_list = [](int) { return true; };
    // Set-up of this workgroup's query i into slot i & 1 (all builder waves).
    auto setup = [&](int i) {
      const int s = i & 1;
      lds_wait_at_least<kLazySleep>(&s_free[s], i / 2, wc);  // the slot's previous query is written out
      // The query of this slot: -1 past the workgroup's last one, which then
      // sets up an empty slot that tells every wave to stop.  With dynamic
      // claims only wave 0 knows it (the other builder waves have no set-up
      // work when the coarse distances are given).
      int q = (int)blockIdx.x + i * G;
      if (dyn) {
        int c = 0;
        if (wave == 0 && lane == 0) c = i == 0 ? (int)blockIdx.x : atomicAdd(a.qctr, 1);
        q = wave == 0 ? __builtin_amdgcn_readfirstlane(c) : -1;
      }
      if (q >= a.nq) q = -1;
      const uint32_t* pr = a.probes + (size_t)(q >= 0 ? q : 0) * P;
      const uint32_t pl_lane = q >= 0 && lane < P ? pr[lane] : kPruned;
      // With the coarse distances at hand, wave 0 bounds every list from them
      // (one lane a probe) and the other builder waves have nothing to do.
      float lb_lane = 0.0f;
      if (a.probe_dists) {
        if (wave == 0 && pl_lane < NL) lb_lane = list_lower_bound(a.probe_dists[(size_t)q * P + lane], a.rmax[pl_lane]);
      }
      const float qa = !a.probe_dists && q >= 0 && lane < D ? a.queries[(size_t)(q / a.qdiv) * D + lane] : 0.0f;
      const float qb =
          !a.probe_dists && q >= 0 && lane + kWave < D ? a.queries[(size_t)(q / a.qdiv) * D + lane + kWave] : 0.0f;
      // Otherwise each builder wave computes the bounds of its probes
      // p = wave + 8 j from the centroid rows, four lists at a time.
      constexpr int kBatch = 4;
#pragma unroll 1
      for (int j0 = 0; !a.probe_dists && j0 < kMaxPerWave && wave + kBuilderWaves * j0 < P; j0 += kBatch) {
        float ca[kBatch], cc[kBatch], rl[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = wave + kBuilderWaves * (j0 + j);
          const uint32_t pl = (uint32_t)__builtin_amdgcn_readlane((int)pl_lane, p);
          ca[j] = cc[j] = rl[j] = 0.0f;
          if (p < P && pl < NL) {
            const float* cr = a.centroids + (size_t)pl * D;
            ca[j] = lane < D ? cr[lane] : 0.0f;
            cc[j] = lane + kWave < D ? cr[lane + kWave] : 0.0f;
            rl[j] = a.rmax[pl];
          }
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = wave + kBuilderWaves * (j0 + j);
          if (p < P) {
            const float ra = lane < D ? qa - ca[j] : 0.0f;
            const float rb = lane + kWave < D ? qb - cc[j] : 0.0f;
            float s2 = ra * ra + rb * rb;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) s2 += shfl_xor_f(s2, o);  // same value in every lane
            if (lane == 0) p_lb[s][p] = list_lower_bound(s2, rl[j]);
          }
        }
      }
      lds_signal_add(&s_lbdone[s], 1);
      if (wave == 0) {
        // The query's result row starts as the fault marker; its root write
        // replaces it.  A row whose query a give-up kept from completing thus
        // never holds silently wrong or stale values.
        if (q >= 0 && lane < k) {
          a.out_ids[(size_t)q * k + lane] = kFaultId;
          a.out_d[(size_t)q * k + lane] = __builtin_nanf("");
        }
        // Compact the usable probes (in range, non-empty) in coarse order and
        // number their chunks: f_cst[f] = first chunk of list f.
        int st = 0, n = 0;
        if (pl_lane < NL) {
          st = a.offsets[pl_lane];
          n = a.offsets[pl_lane + 1] - st;
        }
        const bool valid = n > 0;
        const uint64_t bm = __ballot(valid);
        const int pos = __popcll(bm & ((1ull << lane) - 1ull));
        const int nch = valid ? (n + kChunk - 1) / kChunk : 0;
        const int incl = wave_incl_scan(nch);
        // Every builder wave has signalled this set-up, so each has left the
        // loop of query i - 1 and of query i - 2, the slot's previous user:
        // no wave reads its decisions any more.
        lds_wait_at_least<kLazySleep>(&s_lbdone[s], kBuilderWaves * (i / 2 + 1), wc);
        s_dec[s][lane] = kUndecided;
        if (valid) {
          f_list[s][pos] = (int)pl_lane;
          f_start[s][pos] = st;
          f_n[s][pos] = n;
          f_cst[s][pos] = incl - nch;
          f_lb[s][pos] = a.probe_dists ? lb_lane : p_lb[s][lane];
        }
        const int nv = __popcll(bm);
        const int total = __shfl(incl, kWave - 1, kWave);
        if (lane < kScanWaves - 1) s_arr[s][lane] = 0;
        if (lane == 0) {
          f_cst[s][nv] = total;
          s_nv[s] = nv;
          s_q[s] = q;
          s_thr[s] = kNoThr;

        }
        lds_signal_add(&s_ready[s], 1);
      }
    };

    int nbuilt = 0, need0 = 0, need1 = 0, need2 = 0, nskip = 0;
    long long t_su = 0;
    if (nqw > 0) setup(0);
    for (int i = 0; dyn || i < nqw; ++i) {
      const int s = i & 1;
      lds_wait_at_least(&s_ready[s], i / 2 + 1, wc);
      const int q = dyn ? s_q[s] : (int)blockIdx.x + i * G;
      if (q < 0 || q >= a.nq) break;
      const int nv = s_nv[s];
      const float qv = lane < RW ? a.queries[(size_t)(q / a.qdiv) * D + wave * RW + lane] : 0.0f;
      // This wave's centroid coordinates of the next list that may be built,
      // loaded ahead (cnext belongs to list cnext_f).
      int cnext_f = nv > 0 ? 0 : nv;
      float cnext = 0.0f;
      if (nv > 0 && lane < RW) cnext = a.centroids[(size_t)f_list[s][0] * D + wave * RW + lane];
      int f = 0;
      while (f < nv) {
        int dec;
        if (wave == 0) {
          // Builder wave 0 decides, a run at a time: the lists from f on whose
          // bound exceeds the current threshold are skipped, and the first one
          // that does not is built as list number nbuilt.  Later lists wait for
          // a later (tighter) threshold.
          dec = s_dec[s][f];
          if (dec == kUndecided) {
            const uint64_t thr = s_thr[s];
            const float thr_hi = __uint_as_float((uint32_t)(thr >> 32)) * (1.0f + 0x1p-16f);
            const int g = f + lane;
            const bool cand = a.list_skip && g < nv && f_lb[s][g] > thr_hi;
            const uint64_t run = ~__ballot(cand);  // bit i clear: list f + i is skippable
            const int p = run ? __ffsll((unsigned long long)run) - 1 : kWave;
            if (lane < p && g < nv) s_dec[s][g] = kSkipped;
            if (lane == p && g < nv) s_dec[s][g] = nbuilt;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            dec = p > 0 ? kSkipped : nbuilt;
            nskip += min(p, nv - f);
          }
        } else {
          dec = lds_wait_decided<kLazySleep>(&s_dec[s][f], wc);
        }
        if (dec < 0) {
          f = next_list(s, nv, f + 1, any_list);
          continue;
        }
        const int b = dec % kLutBufs;
        ++nbuilt;
        float cs = cnext;
        if (cnext_f != f && lane < RW) cs = a.centroids[(size_t)f_list[s][f] * D + wave * RW + lane];
        cnext_f = next_list(s, nv, f + 1, any_list);
        if (cnext_f < nv && lane < RW) cnext = a.centroids[(size_t)f_list[s][cnext_f] * D + wave * RW + lane];
        // Residual q - c of this wave's subspaces, shared through the wave's own
        // LDS slot (a wave's LDS accesses complete in order).
        if (lane < RW) rw[lane] = qv - cs;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float r[C::S];
#pragma unroll
        for (int d = 0; d < C::S; ++d) r[d] = rw[(lane / TPM) * C::S + d];
        lds_wait_at_least<kLazySleep>(&s_done[b], b == 0 ? need0 : b == 1 ? need1 : need2, wc);
        float* lut = smem + b * C::LUT + ms * kPQK + 4 * t;
#pragma unroll
        for (int u = 0; u < E / 4; ++u) {
          float4 v;
          v.x = lut_entry<C::S>(r, cb + (4 * u + 0) * C::S);
          v.y = lut_entry<C::S>(r, cb + (4 * u + 1) * C::S);
          v.z = lut_entry<C::S>(r, cb + (4 * u + 2) * C::S);
          v.w = lut_entry<C::S>(r, cb + (4 * u + 3) * C::S);
          *reinterpret_cast<float4*>(lut + 4 * TPM * u) = v;
        }
        lds_signal_add(&s_built[b], 1);
        const int nch = f_cst[s][f + 1] - f_cst[s][f];
        if (b == 0)
          need0 += nch;
        else if (b == 1)
          need1 += nch;
        else
          need2 += nch;
        f = cnext_f;
      }
      if (dyn || i + 1 < nqw) {
        const long long t0 = a.stats ? clock64() : 0;
        setup(i + 1);
        if (a.stats) t_su += clock64() - t0;
      }
    }
    if (a.stats && wave == 0 && lane == 0) {
      atomicAdd(&a.stats[1], (unsigned long long)nbuilt);
      atomicAdd(&a.stats[2], (unsigned long long)nskip);
      atomicAdd(&a.stats[3], (unsigned long long)t_su);
      atomicAdd(&a.stats[4], (unsigned long long)(clock64() - t_start));
    }
  } else {
    const int swave = wave - kBuilderWaves;
    // Scanner instructions issue ahead of the builders' on a shared SIMD: the
    // builders run ahead of the scanners and have slack, the scanners set the
    // pace (3% on C2).
    __builtin_amdgcn_s_setprio(2);
    // This wave's first chunk at or after chunk cc.
    auto first_own = [&](int cc) { return cc + (((swave - cc) % kScanWaves) + kScanWaves) % kScanWaves; };
    unsigned nload = 0;  // vectors whose codes this wave loaded
    long long t_end = 0;
    // This wave's chunks of built list number dec (buffer dec % 3, vectors
    // start .. start + n - 1, chunks c0 .. c_end - 1 of slot s's query):
    // wait for its LUT, scan them into lk / own, and count them done.
    auto scan_chunks = [&](int s, int dec, int start, int n, int c0, int c_end, uint64_t& lk, uint64_t& own) {
      int c = first_own(c0);
      uint4 w0[C::NV4], w1[C::NV4];
      int i0 = kPadId, i1 = kPadId;
      load_pair<M>(a.codes, a.vec_ids, start, n, (c - c0) * kChunk + lane, w0, w1, i0, i1);
      nload += (unsigned)min(kChunk, n - (c - c0) * kChunk);
      const int b = dec % kLutBufs;
      lds_wait_at_least(&s_built[b], kBuilderWaves * (dec / kLutBufs + 1), wc);
      int mine = 0;
      while (true) {
        const uint64_t shared_thr = s_thr[s];
        const uint64_t thr = own < shared_thr ? own : shared_thr;
        const int v0 = (c - c0) * kChunk + lane;
        if (b == 0)
          scan_round_full<D, M, 0>(smem, v0, n, k, w0, w1, i0, i1, thr, lk, own, &s_thr[s]);
        else if (b == 1)
          scan_round_full<D, M, 1>(smem, v0, n, k, w0, w1, i0, i1, thr, lk, own, &s_thr[s]);
        else  // beyond the 64 KB DS offset reach: addresses take a base register
          scan_round_full<D, M, 2>(smem, v0, n, k, w0, w1, i0, i1, thr, lk, own, &s_thr[s]);
        ++mine;
        c += kScanWaves;
        if (c >= c_end) break;
        load_pair<M>(a.codes, a.vec_ids, start, n, (c - c0) * kChunk + lane, w0, w1, i0, i1);
        nload += (unsigned)min(kChunk, n - (c - c0) * kChunk);
      }
      // List done by this wave: its LUT buffer may be reused once all its
      // chunks are in.
      lds_signal_add(&s_done[b], mine);
    };
    // Through query q (slot s): climb the merge tree without waiting.  At each
    // node the wave deposits its list, then counts itself in; the first of the
    // two children to arrive is done with the query, the second merges its
    // sibling's list and climbs on.  The second arrival at the root holds all
    // eight lists merged: it writes the top-k and frees the slot.  Returns
    // whether this wave was that root.
    auto climb = [&](uint64_t lk, int s, int q) {
      int base = 0;
#pragma unroll
      for (int lvl = 0, width = kScanWaves / 2; width >= 1; ++lvl, base += width, width >>= 1) {
        const int nd = base + (swave >> (lvl + 1)), ch = (swave >> lvl) & 1;
        s_tree[s][nd][ch][lane] = lk;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        int old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&s_arr[s][nd], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        old = __builtin_amdgcn_readfirstlane(old);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (old == 0) return false;
        wave_merge_lds64(lk, s_tree[s][nd][ch ^ 1]);
      }
      write_topk(lk, q, k, a, __hip_atomic_load(&s_fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0);
      lds_signal_add(&s_free[s], 1);
      return true;
    };
    for (int i = 0; dyn || i < nqw; ++i) {
      const int s = i & 1;
      lds_wait_at_least(&s_ready[s], i / 2 + 1, wc);
      const int q = dyn ? s_q[s] : (int)blockIdx.x + i * G;
      if (q < 0 || q >= a.nq) break;
      const int nv = s_nv[s];
      const int* cst = f_cst[s];
      uint64_t lk = kPadKey, own = kNoThr;
      // List steps.  Each step reads every usable list's table entry and
      // decision in one batch of LDS reads (one lane a list, nv <= 64), so a
      // step costs one LDS round trip, not a chain of them: under the scan's
      // gather load each LDS round trip waits hundreds of clocks.  A wave
      // visits the lists holding one of its chunks in coarse order; the step
      // index f only grows, so the loop ends.
      int f = -1;
      while (true) {
        const int dec_l = lane < nv ? __hip_atomic_load(&s_dec[s][lane], __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_WORKGROUP)
                                    : kSkipped;
        const int cst_l = cst[lane], cst_n = cst[lane + 1];
        const int st_l = f_start[s][lane], n_l = f_n[s][lane];
        const uint64_t bm = __ballot(lane > f && dec_l != kSkipped && first_own(cst_l) < cst_n);
        if (!bm) break;
        f = __ffsll((unsigned long long)bm) - 1;
        int dec = __builtin_amdgcn_readlane(dec_l, f);
        if (dec == kUndecided) dec = lds_wait_decided(&s_dec[s][f], wc);
        if (dec < 0) continue;
        // A list range as the set-up wrote it lies inside the index; the clamp
        // keeps the loads inside it even after a give-up.
        const int start = __builtin_amdgcn_readlane(st_l, f);
        const int n = min(__builtin_amdgcn_readlane(n_l, f), total - start);
        scan_chunks(s, dec, start, n, __builtin_amdgcn_readlane(cst_l, f), __builtin_amdgcn_readlane(cst_n, f), lk, own);
      }
      if (climb(lk, s, q) && a.stats) t_end = clock64() - t_start;
    }
    // The workgroup's end: the latest of the scanner waves' last root writes.
    if (a.stats && lane == 0 && t_end > 0) atomicMax(&s_tend, (unsigned long long)t_end);
    if (a.stats && lane == 0) {
      atomicAdd(&a.stats[0], (unsigned long long)nload);
      if (wave == kBuilderWaves) atomicAdd(&a.stats[5], (unsigned long long)(clock64() - t_start));
    }
  }
  if (a.stats) {  // every wave of the workgroup gets here (a.stats is uniform)
    __syncthreads();
    if (tid == 0) atomicAdd(&a.stats[6], s_tend);
  }
}

// Workgroups resident at once for a kernel (one query each at a time): the
// persistent flow kernel launches no more than that.
template <class K>
int resident_groups(K kernel, int threads, std::atomic<int> (&cached)[64]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || per <= 0) per = 1;
  v = cus * per;
  cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

// The claim counter of a launch starts at the grid size: the first G queries
// are the workgroups' static first ones.  A kernel, not a memset, so that a
// captured graph replays it correctly.
__global__ void qctr_reset_kernel(int* qctr, int grid) {
  if (threadIdx.x == 0) *qctr = grid;
}

// Flow-kernel workgroups resident at once on the current device.
template <int D, int M>
int flow_resident() {
  static std::atomic<int> cached[64];
  return resident_groups(adc_flow_kernel<D, M>, kSpecWaves * kWave, cached);
}

template <int D, int M>
fgpu_status launch_flow(const AdcArgs& args, hipStream_t s) {
  FGPU_CHECK(args.nprobe <= 64, FGPU_ERR_UNSUPPORTED, "adc: nprobe must be <= 64");
  FGPU_CHECK(args.faults, FGPU_ERR_ARG, "adc: the flow kernel needs a device give-up counter");
  AdcArgs a = args;
  if (a.spin_limit <= 0) a.spin_limit = (int)flow_spin_limit(a.nprobe, a.max_list_len);
  const int grid = std::min(a.nq, flow_resident<D, M>());
  if (a.qctr && a.qctr_preset != grid) hipLaunchKernelGGL(qctr_reset_kernel, dim3(1), dim3(64), 0, s, a.qctr, grid);
  hipLaunchKernelGGL((adc_flow_kernel<D, M>), dim3((unsigned)grid), dim3(kSpecWaves * kWave), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

template <int D, int M>
fgpu_status launch_plain(const AdcArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((adc_plain_kernel<D, M>), dim3((unsigned)a.nq), dim3(kNT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

template <int D, int M>
fgpu_status launch_plain_list(const AdcArgs& a, hipStream_t s) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  // Few workgroups: the list is usually empty, and then each ends at once.
  const int grid = std::max(1, std::min(a.nq, cus / 4));
  hipLaunchKernelGGL((adc_plain_list_kernel<D, M>), dim3((unsigned)grid), dim3(kNT), 0, s, a);
  FGPU_HIP(hipGetLastError());
  return FGPU_OK;
}

}  // namespace

long long flow_spin_limit(int nprobe, int max_list_len) {
  // Longest legitimate wait: a builder setting up query i + 1 waits for query
  // i - 1 to be written, i.e. for up to nprobe lists of max_list_len vectors
  // to be scanned.  At 32 clocks a vector and >= 64 clocks a poll that is
  // nprobe * max_list_len / 2 polls; the limit allows 4x that, plus 2^16.
  const long long v = (1ll << 16) + 2ll * (long long)std::max(nprobe, 1) * (long long)std::max(max_list_len, 0);
  return std::min<long long>(v, 1ll << 30);
}

bool adc_supported(int dim, int m) {
  return (dim == 128 && (m == 16 || m == 32 || m == 64)) || (dim == 96 && (m == 16 || m == 32 || m == 48));
}

fgpu_status launch_adc_plain(int dim, int m, const AdcArgs& a, hipStream_t s) {
  FGPU_CHECK(a.k >= 1 && a.k <= 64, FGPU_ERR_UNSUPPORTED, "adc: k must be in [1, 64]");
  if (a.nq <= 0) return FGPU_OK;
  // The flow kernel's per-query tables hold 64 lists; more probes go to the
  // barrier-per-list kernel, which walks any number of them (every probed
  // list scanned, no list bound).
  if (a.nprobe > 64) {
    if (dim == 128 && m == 32) return launch_plain<128, 32>(a, s);
    if (dim == 128 && m == 16) return launch_plain<128, 16>(a, s);
    if (dim == 96 && m == 32) return launch_plain<96, 32>(a, s);
    if (dim == 96 && m == 16) return launch_plain<96, 16>(a, s);
  }
  if (dim == 128 && m == 32) return launch_flow<128, 32>(a, s);
  if (dim == 128 && m == 16) return launch_flow<128, 16>(a, s);
  if (dim == 128 && m == 64) return launch_plain<128, 64>(a, s);
  if (dim == 96 && m == 48) return launch_plain<96, 48>(a, s);
  if (dim == 96 && m == 32) return launch_flow<96, 32>(a, s);
  if (dim == 96 && m == 16) return launch_flow<96, 16>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "adc: unsupported (dim, pq_m)");
}

fgpu_status launch_adc_plain_list(int dim, int m, const AdcArgs& a, hipStream_t s) {
  FGPU_CHECK(a.k >= 1 && a.k <= 64 && a.qlist && a.qcount, FGPU_ERR_ARG, "adc: bad query list launch");
  if (a.nq <= 0) return FGPU_OK;
  if (dim == 128 && m == 32) return launch_plain_list<128, 32>(a, s);
  if (dim == 128 && m == 16) return launch_plain_list<128, 16>(a, s);
  if (dim == 128 && m == 64) return launch_plain_list<128, 64>(a, s);
  if (dim == 96 && m == 48) return launch_plain_list<96, 48>(a, s);
  if (dim == 96 && m == 32) return launch_plain_list<96, 32>(a, s);
  if (dim == 96 && m == 16) return launch_plain_list<96, 16>(a, s);
  return set_error(FGPU_ERR_UNSUPPORTED, "adc: unsupported (dim, pq_m)");
}

int flow_grid(int dim, int m, int nq, int nprobe) {
  if (nq <= 0 || nprobe > 64) return 0;
  int r = 0;
  if (dim == 128 && m == 32) r = flow_resident<128, 32>();
  else if (dim == 128 && m == 16) r = flow_resident<128, 16>();
  else if (dim == 96 && m == 32) r = flow_resident<96, 32>();
  else if (dim == 96 && m == 16) r = flow_resident<96, 16>();
  return r > 0 ? std::min(nq, r) : 0;
}

}  // namespace fgpu
