// kernels.hpp -- host-side launchers for the HIP kernels (C++ linkage).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fusiongpu.h"

namespace fgpu {

// ---- coarse.hip -------------------------------------------------------------
// norms[i] = ||rows[i]||^2 (fp32, any order: it only feeds the GEMM estimate).
fgpu_status launch_row_norms(const float* rows, int64_t n, int dim, float* norms, hipStream_t s);
// *out = max(norms[0..n)).
fgpu_status launch_max_reduce(const float* v, int64_t n, float* out, hipStream_t s);
// est[i][j] = xn[i] + cn[j] - 2 <x_i, c_j> for i in [0,nrows), j in [0,ncols);
// est row stride is ld floats.  dim % 32 == 0: bf16 MFMA on a hi/lo split of
// both operands; otherwise MFMA f32 32x32x2.
fgpu_status launch_gemm_est(const float* x, int64_t nrows, const float* c, int ncols, int dim,
                            const float* xn, const float* cn, float* est, int64_t ld, hipStream_t s);
// The same contraction for launch_select_exact: cn[j] - 2 <x_i, c_j>, each
// row shifted by its norm, in the select's element form (fp32, or the fp16
// lower bound of the row scaled by a power of two that keeps it inside the
// fp16 range, the row's exponent stored after the block); ld % 8 == 0, at
// least est_sel_ld(ncols); est holds nrows * ld floats; cn_max = max cn.
fgpu_status launch_gemm_est_sel(const float* x, int64_t nrows, const float* c, int ncols, int dim, const float* cn,
                                const float* cn_max, void* est, int64_t ld, hipStream_t s);
int64_t est_sel_ld(int ncols);
// Per row: the p nearest columns by exact device-form L2, chosen from the
// estimates of launch_gemm_est_sel with a rigorous error margin.  ids
// are int32 bit patterns; with prune != 0 a column farther than
// best*prune_ratio gets 0xFFFFFFFF.  With side != nullptr the launch also
// stores side_val at *side (one word, for the next kernel on the stream).
// stats (nullptr = off): adds the columns re-scored exactly to stats[0] and
// the rows that re-scored every column to stats[1].
fgpu_status launch_select_exact(const void* est, int64_t ld, int64_t nrows, int ncols,
                                const float* x, const float* c, int dim,
                                const float* cn_max, int p, int prune, float prune_ratio,
                                int32_t* out_ids, float* out_d, hipStream_t s, int* side = nullptr,
                                int side_val = 0, unsigned long long* stats = nullptr);
// Exact kNN over one chunk of <= 4096 base rows c (ids id_base + col), merged
// into the running top-k in ids/d (k <= 128) when accum != 0.
fgpu_status launch_knn_chunk(const float* est, int64_t ld, int64_t nrows, int ncols, const float* x, const float* c,
                             int dim, const float* xn, const float* cn_max, int k, int id_base, int accum,
                             int32_t* ids, float* d, hipStream_t s);
// Rows per batch of the estimate matrix that fit in `bytes`.
int64_t est_rows_per_batch(size_t bytes, int ncols);

// ---- adc.hip ------------------------------------------------------------------
struct AdcArgs {
  const float* queries;     // [nq][dim]
  const float* centroids;   // [nlist][dim]
  const float* codebook;    // [m][256][dim/m]
  const int32_t* offsets;   // [nlist+1]
  const uint8_t* codes;     // [total][m]
  const int32_t* vec_ids;   // [total]
  const uint32_t* probes;   // [nq][nprobe]
  const float* rmax;        // [nlist] upper bound on the norm of any decoded residual of the list
  int nq, nprobe, k, nlist;  // probe ids >= nlist are skipped like pruned ones
  int32_t* out_ids;         // [nq][k]
  float* out_d;             // [nq][k]
  // Optional: [nq][nprobe] squared L2 of query and probed centroid in the
  // coarse step's form (sequential fused chain over fl(q - c)), which the
  // list lower bound accepts in place of its own sum (nullptr = compute).
  const float* probe_dists = nullptr;
  // Queries per row of `queries`: query q reads row q / qdiv (several
  // virtual queries of one query share its row).
  int qdiv = 1;
  // Optional instrumentation (nullptr = off), summed over the launch:
  // [0] vectors whose codes were loaded, [1] LUTs built, [2] probed lists
  // skipped by the list lower bound; shader clocks per workgroup: [3] set-up,
  // [4] builder wave 0 after set-up, [5] scanner wave 8 after set-up, [6] the
  // whole workgroup (thread 0, start to end).
  unsigned long long* stats = nullptr;
  // Vectors in the index: list ranges read from LDS are clamped to it, so a
  // scan stays inside the code and id arrays whatever the hand-off counters say.
  long long total = 0;
  // Bounded waits of the flow kernel: polls (of s_sleep 1) before a wave gives
  // up; 0 = derive from nprobe and the longest list (flow_spin_limit).
  int spin_limit = 0;
  // Device counter (required by the flow kernel): every wait that gives up
  // adds 1, and each query whose top-k is written after a give-up in its
  // workgroup gets id kFaultId / distance NaN in every slot.
  unsigned long long* faults = nullptr;
  int max_list_len = 0;
  // 0: never skip a list on its lower bound (timing of the scan reading every
  // probed list; results are the same).
  int list_skip = 1;
  // Optional device int (workspace) for dynamic query claims of the flow
  // kernel, which resets it on the launch stream; needs probe_dists.
  int* qctr = nullptr;
  // A positive value: an earlier kernel on the stream has already stored it
  // in *qctr (the select's side write).  The launch skips its own reset when
  // it equals the grid it launches (flow_grid).
  int qctr_preset = 0;
  // launch_adc_plain_list only: the queries to search, qlist[0 .. *qcount)
  // (device memory; the count is read on the device).
  const int* qlist = nullptr;
  const int* qcount = nullptr;
};
// Id written to every slot of a query whose result a bounded-wait give-up may
// have touched (the reference's padding id is -1; it never writes -2).
constexpr int kFaultId = -2;
// Polls a flow-kernel wave makes before it gives up: far above the longest
// legitimate wait, the scan of every probed list of one query (a scanner CU
// handles a vector in well under 32 clocks; a poll takes >= 64).
long long flow_spin_limit(int nprobe, int max_list_len);
bool adc_supported(int dim, int m);
// rmax[l] >= max over vectors x of list l of ||decode(x)|| (exact, rounded up).
fgpu_status launch_list_radius(const float* codebook, int m, int sub, const uint8_t* codes, const int32_t* offsets,
                               int nlist, float* rmax, hipStream_t s);
fgpu_status launch_adc_plain(int dim, int m, const AdcArgs& a, hipStream_t s);
// The generic (one workgroup a query, every probed list) kernel over the
// queries a.qlist[0 .. *a.qcount), on a persistent grid.
fgpu_status launch_adc_plain_list(int dim, int m, const AdcArgs& a, hipStream_t s);
// The grid of the flow-kernel launch launch_adc_plain makes for these sizes
// (the start value of its query counter), or 0 if that call takes another
// kernel.
int flow_grid(int dim, int m, int nq, int nprobe);
// noalloc.hip: resolve this device's scratch array address (index creation
// calls it, so that fgpu_search_noalloc needs no first-call lookup).
fgpu_status noalloc_prepare();

// ---- capi.cpp -----------------------------------------------------------------------
// Workspace of fgpu_search on the LUT kernels alone (probe arrays + the coarse
// step); fgpu_search_workspace_bytes adds room for the MFMA screen.
size_t search_lut_workspace_bytes(int nq, int nlist, int nprobe);

// ---- screen.hip -----------------------------------------------------------------
// Counters at the head of the screen's zeroed region.
constexpr int kCtrFlag = 0, kCtrCount = 32;
// Lists an index may have for the screen (its work-item scan lives in LDS).
constexpr int kScreenMaxLists = 8192;
struct ScreenArgs {
  const float* queries;     // [nq][dim]
  const float* centroids;   // [nlist][dim]
  const int32_t* offsets;   // [nlist+1]
  const uint8_t* codes;     // [total][m]
  const int32_t* vec_ids;   // [total]
  const float* codebook;    // [m][256][dim/m] fp32
  const uint16_t* cb16;     // [m][256][dim/m] fp16 of the codebook times 2^scale_exp (nearest, flushed below 2^-14)
  const uint4* vext;        // [total] per-vector extra block (screen_prep)
  const float* rmax;        // [nlist]
  const uint32_t* probes;   // [nq][nprobe]; ids >= nlist are skipped
  const float* probe_dists; // [nq][nprobe] the coarse step's squared distances
  int nq, nprobe, k, nlist;
  int scale_exp;            // S: the screen's operands are the data times 2^S (the index's choice)
  // One region, zeroed at the start of a launch: ctr[kCtrCount], cnt1[nlist],
  // cnt2[nlist], cand_cnt[nq] (in this order, contiguous).
  int* ctr;
  int* cnt1;
  int* cnt2;
  int* cand_cnt;
  int* bucket;              // [nlist][nq] pair entries (q nprobe + p) of each list, or compact (boff)
  // [nlist + 1] or nullptr: compact buckets for one probe a query, list l's
  // entries at bucket[boff[l] .. boff[l + 1]) (boff[l + 1] - boff[l] = the
  // queries whose probe is l); nullptr = bucket[l nq + pos].
  const int32_t* boff = nullptr;
  // The rescore's order of the queries (a permutation of 0 .. nq-1, e.g.
  // single-probe queries grouped by list so a list's codes stay in L2);
  // nullptr = ascending.
  const int32_t* order = nullptr;
  // Single-probe mode (nprobe 1, compact buckets): sp_cnt[l] = the queries
  // screened against list l in both rounds, whose entries are
  // bucket[boff[l] .. boff[l] + sp_cnt[l]) (filled by the caller); round 2
  // keeps round 1's pairs and records, and pnorm[q] holds the round-1 pair's
  // (nr2, squared error sum).  nullptr = the general buckets.
  const int32_t* sp_cnt = nullptr;
  float2* pnorm = nullptr;
  // Round 2's work items: list chunks of at least r2_chunk vectors (a
  // multiple of 32), at most r2_max_chunks of them.
  int r2_chunk = 256, r2_max_chunks = 8;
  // Queries per row of `queries`: query q reads row q / qdiv.
  int qdiv = 1;
  uint4* arec;              // [nq nprobe][2][9] pair records: per lane half 8 A fragments and the extra block
  int2* first;              // [nq] round 1: (list, t | chunks << 8) of the query's pair (t its row scale
                            // exponent, chunks its list's round-1 work items), (-1, -1), or (-2, 0)
  uint32_t* gminbuf;        // [nq][kMaxChunks][64] round 1: per query, first-list chunk and group, min U bits
  float* thr;               // [nq] T(q)
  uint2* cand;              // [nq][cand_cap] (vector position, list)
  int cand_cap;
  int* flist;               // [nq] queries handed to the LUT kernel
  int32_t* out_ids;         // [nq][k]
  float* out_d;             // [nq][k]
  // Optional instrumentation (nullptr = off), summed over the waves: shader
  // clocks [0] before the first item, [1] in item set-up, [2] in the tile
  // loops, [3] after the tiles; [0..3] round 1, [4..7] round 2.
  unsigned long long* stats = nullptr;
  // Optional (nullptr = off): events recorded on the launch stream after the
  // pair kernel of round 1 (with the zeroing), round 1, the pair kernel of
  // round 2, round 2 and the rescore, in that order.
  const hipEvent_t* events = nullptr;
};
bool screen_supported(int dim, int m);
// Words of ScreenArgs::gminbuf for nq queries.
int64_t screen_gmin_words(int nq);
// The fp16 codebook (times 2^scale_exp) and the per-vector extra blocks of an
// index; *xmax_bits = the largest scaled decoded norm bound X' (float bits).
fgpu_status launch_screen_prep(const float* codebook, int m, int sub, int scale_exp, const uint8_t* codes,
                               int64_t total, uint16_t* cb16, uint4* vext, unsigned int* xmax_bits, hipStream_t s);
// Threshold, screen and rescore; the queries it cannot answer are listed in
// flist[0 .. ctr[kCtrFlag]) for launch_adc_plain_list.
fgpu_status launch_screen(int dim, int m, const ScreenArgs& a, hipStream_t s);

// ---- twophase.hip --------------------------------------------------------------
struct TwoPhaseArgs {
  const float* queries;     // [nq][dim]
  const float* centroids;   // [nlist][dim]
  const float* codebook;    // [m][256][dim/m]
  const int32_t* offsets;   // [nlist+1]
  const uint8_t* codes;     // [total][m]
  const int32_t* vec_ids;   // [total]
  const uint32_t* probes;   // [nq][nprobe]; ids >= nlist are skipped
  const float* rmax;        // [nlist] decoded-residual radius per list
  int nq, nprobe, nlist;
  int p1;                   // phase-1 probes = min(nprobe, p1_lists)
  int limit_k;              // per-list candidates in phase 1 (<= 64)
  float coeff;              // threshold coefficient
  int rerank_m;             // candidates kept (<= 2^17)
  uint64_t* pool;           // [nq][pool_cap] candidate keys (workspace)
  int pool_cap;             // >= two_phase_pool_cap(p1, limit_k, rerank_m)
  int32_t* top_ids;         // [nq][rerank_m]
  float* top_d;             // [nq][rerank_m]
  int32_t* top_counts;      // [nq]
  float* cutoffs;           // [nq][p1] or nullptr
  float* thr;               // [nq] or nullptr
  // Optional instrumentation (nullptr = off), summed over the launch:
  // [0] vectors whose codes were loaded, [1] LUTs built, [2] phase-2 lists
  // skipped by the list lower bound, [3] phase-2 candidates appended,
  // [4..7] shader clocks of workgroup thread 0 in set-up, phase 1, phase 2
  // and the final select + sort; [8..10] of its phase-1 clocks, those spent
  // up to the LUT barrier, in the scan loop, and in the merge barrier + merge.
  unsigned long long* stats = nullptr;
  // Phase 1 over `split` workgroups a query (limit_k <= 64; small batches):
  // cut_ws holds [nq][nprobe] phase-1 cutoffs between the two launches.
  int split = 1;
  float* cut_ws = nullptr;
  // [nq] or nullptr: candidates before the rerank_m cut (phase-1 slots plus
  // every phase-2 vector with dist <= thr).  When set, phase 2 skips lists
  // and ends sums against thr itself rather than the pool's admission bound,
  // so that every such vector is seen.
  int32_t* pre_cut = nullptr;
  // Mode 2 (after a separate phase 1) over the queries qlist[0 .. *qcount)
  // only (workgroup i takes qlist[i]; nullptr = every query).
  const int32_t* qlist = nullptr;
  const int* qcount = nullptr;
};
int two_phase_pool_cap(int p1, int limit_k, int rerank_m);
// Phase 1 through the screen: virtual query v = q p1 + p for the nqc queries
// of a chunk (the query row copied to vq, probe p in vprobe, 0xFFFFFFFF when
// unusable, a zero probe distance in vpd) and each usable list's count in
// hist (zeroed first); boff = the exclusive scan of hist (nlist + 1 entries)
// and sp_cnt the screen's single-probe counts (ScreenArgs::sp_cnt).
// After the screen, launch_tp_finish completes most queries and leaves the
// others' pool slots and cutoffs to launch_two_phase_after_phase1, which
// runs the threshold, phase 2 and the final select (limit_k <= 64).
fgpu_status launch_tp_virtual(const uint32_t* probes, int nprobe, int p1, int nqc, const int32_t* offsets, int nlist,
                              uint32_t* vprobe, float* vpd, int* hist, int32_t* rank, hipStream_t s);
fgpu_status launch_tp_offsets(const int* hist, int nlist, int32_t* boff, const int32_t* offsets, int k,
                              int32_t* sp_cnt, hipStream_t s);
fgpu_status launch_two_phase_after_phase1(int dim, int m, const TwoPhaseArgs& a, hipStream_t s);
// order[0 .. nvq): the virtual queries grouped by list (list l's at
// boff[l] .. boff[l + 1), in no fixed order within it), those without a
// usable list last, each at its rank from launch_tp_virtual.
fgpu_status launch_tp_order(const uint32_t* vprobe, const int32_t* rank, int nvq, int nlist, const int32_t* boff,
                            int32_t* order, hipStream_t s);
// The second half of the two-phase scan for queries q_base .. q_base + nqc - 1
// of a (phase 1 done by the screen: virtual query (q - q_base) p1 + p holds
// probe p's top-limit_k in vids/vd): threshold, phase-2 list bounds (from
// probe_dists[q][p] when given, else from the centroids) and, when no
// phase-2 list can reach the threshold and the phase-1 keys fit rerank_m,
// the final ranking; any other query gets its pool slots and cutoffs and
// joins slow_list (slow_cnt counts them) for launch_two_phase_after_phase1.
fgpu_status launch_tp_finish(const TwoPhaseArgs& a, int dim, int q_base, int nqc, const int32_t* vids, const float* vd,
                             const float* probe_dists, int32_t* slow_list, int* slow_cnt, hipStream_t s);
fgpu_status launch_tp_zero(int* p, int n, hipStream_t s);
// stats[11] += nvq, [12] += the sum of cand_cnt[0..nvq), [13] += *flag_cnt,
// [14] += entries of thr[0..nvq) that are not below +inf, [15] += the others
// whose cand_cnt exceeds cap; [16]/[17] += (query, vector) pairs screened in
// round 1/2 and [18]/[19] += their 32 x 32 MFMA tiles (per list: the counts
// cnt1/cnt2, capped at the compact bucket's length, against the list size).
fgpu_status launch_tp_stats(const int* cand_cnt, const float* thr, int nvq, int cap, const int* flag_cnt,
                            const int* cnt1, const int* cnt2, const int32_t* boff, const int32_t* offsets, int nlist,
                            unsigned long long* stats, hipStream_t s);
// Workgroups a query for phase 1 (TwoPhaseArgs::split) for a launch of nq
// queries: 1 once nq fills every CU twice; a test override can force it.
// (force: 0 automatic, 1 never, s >= 2 s ways, at most p1.)
int two_phase_split(int nq, int p1, int limit_k, int force = 0);
fgpu_status launch_two_phase(int dim, int m, const TwoPhaseArgs& a, hipStream_t s);

struct RerankArgs {
  const float* queries;     // [nq][dim]
  const float* base;        // [n][dim] raw vectors
  long long n;
  const int32_t* cand;      // [nq][rm] candidate ids in ADC order
  const int32_t* counts;    // [nq] valid candidates per row
  int nq, rm, k, mb;
  float eps;
  int beta;
  int32_t* out_ids;         // [nq][k]
  float* out_d;             // [nq][k]
  int32_t* visited;         // [nq] or nullptr
  int spec = 0;             // mini-batches computed a step: 0 automatic, 1, or 4 (any other value)
  // [nq] or nullptr: the stable count after the last batch evaluated, and 1
  // when the walk stopped on stability or reached an offset at or past the
  // candidates before rm (the reference's stab[] and fin[]).
  int32_t* stable = nullptr;
  uint8_t* finished = nullptr;
};
fgpu_status launch_rerank(int dim, const RerankArgs& a, hipStream_t s);
// Mini-batches the rerank kernel computes at once for nq queries (1 or 4);
// a test override can force either.
// (force: 0 automatic, 1 one, anything else four.)
int rerank_spec(int nq, int force = 0);

// ---- graph.hip -----------------------------------------------------------------
struct GraphArgs {
  const float* queries;     // [nq][dim]
  const float* base;        // [n][dim], 16-byte aligned
  long long n;
  const int32_t* graph;     // [n][degree] neighbour ids (ids outside [0, n) are skipped)
  int degree, itopk, width, max_iter, k;
  uint64_t seed;
  int q0;                   // index of the first query (seeds depend on it)
  int nq;
  int32_t* out_ids;         // [nq][k]
  float* out_d;             // [nq][k]
  int32_t* iters;           // [nq] or nullptr: steps taken
  int32_t* evals;           // [nq] or nullptr: exact distances computed
};
fgpu_status launch_graph_search(int dim, const GraphArgs& a, hipStream_t s);
fgpu_status launch_drop_self(const int32_t* knn, int n, int degree, int32_t* out, hipStream_t s);
fgpu_status launch_coarse_prune(int32_t* ids, const float* d, int nq, int p, float prune_ratio, hipStream_t s);

// ---- tune.hip -------------------------------------------------------------------
constexpr int kMaxTuneLut = 64 * 256;  // pq_m <= 64
struct TuneStatsArgs {
  const float* queries;     // [nq][dim]
  int nq, dim, pq_m, nlist;
  const int32_t* offsets;   // [nlist+1]
  const int32_t* ids;       // [total]
  const uint8_t* codes;     // [total][pq_m]
  const float* centroids;   // [nlist][dim]
  const float* codebook;    // [pq_m][256][dim/pq_m]
  const float* base;        // [n_base][dim] or nullptr (no exact distances)
  long long n_base;
  const int32_t* pair_query;   // [npairs] row of queries
  const int32_t* pair_list;    // [npairs] list id
  const int32_t* pair_target;  // [npairs] vector id, or -1; nullptr: none
  const int32_t* pair_kth;     // [npairs] k for the k-th PQ distance, <= 0 none; nullptr: none
  float* target_pq;         // [npairs]
  float* target_exact;      // [npairs]
  int32_t* pq_rank;         // [npairs]
  int32_t* exact_rank;      // [npairs]
  float* kth_pq;            // [npairs]
};
fgpu_status launch_tune_list_stats(const TuneStatsArgs& a, int npairs, hipStream_t s);

// ---- bandwidth.hip --------------------------------------------------------------
// Reads `bytes` (a multiple of 16) from d with 16-byte loads; one XOR per
// workgroup goes to sink[blockIdx.x] so the loads cannot be dropped.
fgpu_status launch_stream_read(const void* d, size_t bytes, unsigned long long* sink, int grid, hipStream_t s);
fgpu_status launch_row_gather(const void* d, int64_t nrows, int row_bytes, const int32_t* idx, int64_t n,
                              int lanes_per_row, unsigned long long* sink, int grid, hipStream_t s);

// ---- build.hip ----------------------------------------------------------------
fgpu_status launch_probe_counts(const uint32_t* probes, int nq, int nprobe, int nlist, const int32_t* offsets,
                                int32_t* counts, int32_t* offs, hipStream_t s);
fgpu_status launch_maxabs(const float* x, int64_t count, float* out, hipStream_t s);
fgpu_status launch_kmeans_accumulate(const float* x, int64_t n, const int32_t* assign, int k,
                                     int dim, int shift, unsigned long long* sums, int32_t* counts,
                                     hipStream_t s);
fgpu_status launch_kmeans_finalize(const unsigned long long* sums, const int32_t* counts, int k,
                                   int dim, int shift, int empty_rule, float* cent, hipStream_t s);
fgpu_status launch_gather_rows(const float* x, int dim, const int32_t* rows, int nrows, float* out,
                               hipStream_t s);
// fma_mode 1: the device form (fused chain); 0: the host form (separate roundings).
fgpu_status launch_pq_encode(const float* x, int64_t n, int dim, int m, const int32_t* assign,
                             const float* cent, const float* codebook, uint8_t* codes, hipStream_t s,
                             int fma_mode = 1);
fgpu_status launch_pq_residuals(const float* x, int dim, const int32_t* rows, int nrows,
                                const int32_t* assign, const float* cent, float* res, hipStream_t s);
fgpu_status launch_pq_init(const float* res, int nsample, int dim, int m, const int32_t* init_rows,
                           float* codebook, hipStream_t s);
fgpu_status launch_pq_estep(const float* res, int nsample, int dim, int m, const float* codebook,
                            int32_t* assign_pq, hipStream_t s);
fgpu_status launch_pq_mstep(const float* res, int nsample, int dim, int m, const int32_t* assign_pq,
                            float* codebook, hipStream_t s);
// k-means++ seeding on the device (definition in oracle.cpp orc_kmeans_init_pp).
fgpu_status launch_kmeans_pp(const float* x, int64_t n, int dim, int k, uint64_t seed, float* cent,
                             int32_t* rows, void* ws, size_t ws_bytes, hipStream_t s);
size_t kmeans_pp_ws_bytes(int64_t n, int k);

}  // namespace fgpu
