/* fusiongpu.h -- C ABI of the MI355X-native IVF-PQ engine (libfusiongpu.so).
 *
 * Plain C types only: device pointers are `void*`/typed pointers into HBM,
 * streams are passed as `void*` (a hipStream_t; NULL = the null stream).
 * Every call returns an fgpu_status (0 = ok) and never exits the process;
 * fgpu_last_error() returns a thread-local message for the last failure.
 * Calls that take a stream only enqueue work on it: no hidden host
 * synchronisation, no static scratch.  Scratch comes from a caller-owned
 * device workspace whose size the matching *_workspace_bytes() call returns,
 * 16-byte aligned (hipMalloc and torch allocations are 256-byte aligned).
 *
 * Each entry point names the reference interface it replaces
 * (Hello-day/FusionGPU, file:line).
 */
#ifndef FUSIONGPU_H_
#define FUSIONGPU_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  FGPU_OK = 0,
  FGPU_ERR_ARG = 1,         /* invalid argument (shape, null pointer, range) */
  FGPU_ERR_UNSUPPORTED = 2, /* geometry (dim, pq_m, k, nprobe) with no kernel instance */
  FGPU_ERR_HIP = 3,         /* a HIP runtime call failed */
  FGPU_ERR_IO = 4,          /* missing, short or inconsistent file */
  FGPU_ERR_NOMEM = 5,       /* device or host allocation failed */
  FGPU_ERR_WORKSPACE = 6,   /* workspace smaller than *_workspace_bytes() */
  FGPU_ERR_WAIT = 7         /* a bounded device-side wait gave up (fgpu_index_check) */
} fgpu_status;

/* Id written in every result slot of a query that a bounded-wait give-up of
 * the scan kernel may have touched (its distances are NaN).  The reference
 * pads with -1 and never returns -2. */
#define FGPU_FAULT_ID (-2)

typedef struct fgpu_index fgpu_index; /* opaque device-resident IVF-PQ index */

/* Device view of an index: the reference's IVFIndexGPU (defs.h:51-58) plus
 * the geometry that defs.h fixes at compile time (defs.h:9-12). */
typedef struct {
  int dim, pq_m, pq_k, nlist;
  int64_t total;
  const float* d_pq_codebook;      /* [pq_m][256][dim/pq_m] */
  const int32_t* d_cluster_offsets; /* [nlist+1] */
  const uint8_t* d_all_pq_codes;   /* [total][pq_m], list-major */
  const int32_t* d_all_vector_ids; /* [total] */
  const float* d_centroids;        /* [nlist][dim] */
  int max_list_len;
} fgpu_index_info;

const char* fgpu_last_error(void);
int fgpu_abi_version(void);

/* ---- index (A1) ------------------------------------------------------- */

/* Copies host arrays laid out as ivf_data.bin holds them (build_global.cu:242-252)
 * plus the codebook (global_pq_codebook.bin, build_global.cu:204-206) to HBM.
 * Replaces load_ivf_index_to_gpu (search_pipeline.cu:481-529). */
fgpu_status fgpu_index_create(int dim, int pq_m, int nlist, int64_t total, const int32_t* h_offsets,
                              const int32_t* h_ids, const uint8_t* h_codes, const float* h_centroids,
                              const float* h_codebook, fgpu_index** out);
/* Reads ivf_data.bin + global_pq_codebook.bin (search_pipeline.cu:481-503); dim and
 * pq_m are not stored in the files (defs.h fixes them), so the caller states them. */
fgpu_status fgpu_index_load(const char* ivf_data_path, const char* codebook_path, int dim, int pq_m,
                            fgpu_index** out);
void fgpu_index_destroy(fgpu_index* idx);
fgpu_status fgpu_index_get_info(const fgpu_index* idx, fgpu_index_info* out);

/* An index over A1 arrays the caller already holds in HBM, laid out as the
 * reference's IVFIndexGPU holds them (defs.h:51-58; filled by
 * load_ivf_index_to_gpu, search_pipeline.cu:481-529): no copy.  The handle
 * computes its own derived arrays (centroid norms, list radii) and reads the
 * offsets once (it synchronises `stream`).  fgpu_index_destroy frees only what
 * the handle allocated; the caller's arrays must outlive it.  d_codes must be
 * 16-byte aligned and pq_m a multiple of 16. */
fgpu_status fgpu_index_wrap(int dim, int pq_m, int nlist, const int32_t* d_offsets, const int32_t* d_ids,
                            const uint8_t* d_codes, const float* d_centroids, const float* d_codebook,
                            void* stream, fgpu_index** out);

/* The plain scan (fgpu_adc_search, fgpu_search) hands LUT buffers and query
 * slots between the waves of a workgroup through LDS counters.  Every wait on
 * them is bounded, far above the longest legitimate wait (the scan of all
 * probed lists of one query), so a counting error ends in a give-up rather
 * than a hang.  A give-up is recorded: the index's device counter grows by 1,
 * and every query whose results the workgroup writes afterwards gets
 * FGPU_FAULT_ID / NaN in all k slots.  No reference counterpart: the
 * reference's batch logic (gpu_global.cu:679-874) uses no such hand-offs.
 * fgpu_index_faults waits for `stream`, then returns the count (and zeroes it
 * when reset != 0); fgpu_index_check returns FGPU_ERR_WAIT when it is not 0.
 * A correct run always reads 0. */
fgpu_status fgpu_index_faults(const fgpu_index* idx, void* stream, unsigned long long* count, int reset);
fgpu_status fgpu_index_check(const fgpu_index* idx, void* stream);
/* Test hook (host only): the PQ training sample rows of fgpu_pq_train, the
 * first min(sample_size, n) entries of std::shuffle(0 .. n-1, mt19937(12345))
 * (pq_utils.h:91-97), into h_rows.  Returns their count, or -1 on a bad
 * argument. */
int fgpu_debug_pq_sample(int64_t n, int sample_size, int32_t* h_rows);

/* ---- measurement (no reference counterpart) ---------------------------- */

/* Streams `bytes` (a multiple of 16, 16-byte aligned) of device memory
 * through 16-byte loads, to measure the achievable HBM read rate next to the
 * 8 TB/s figure.  d_sink: fgpu_stream_read_grid() uint64 values, overwritten. */
int fgpu_stream_read_grid(void);
fgpu_status fgpu_stream_read(const void* d_data, size_t bytes, unsigned long long* d_sink, void* stream);
/* Reads n whole rows d_rows[d_idx[i]] of row_bytes (384 or 512) each, eight
 * lanes a row (each lane 16 bytes of every 128-byte line), with all of a
 * lane's loads in flight: the access pattern of the exact rerank and the graph
 * search, to measure the random-row read rate their rooflines are set against.
 * Ids outside [0, nrows) are clamped.  d_sink as for fgpu_stream_read. */
fgpu_status fgpu_row_gather(const void* d_rows, int64_t nrows, int row_bytes, const int32_t* d_idx, int64_t n,
                            unsigned long long* d_sink, void* stream);
/* The same with lanes_per_row 1 (each lane reads its own whole row, so one
 * load instruction touches 64 rows) or 8 (fgpu_row_gather).  Over arrays of
 * a few GB the first form reads far slower; it is kept to measure that. */
fgpu_status fgpu_row_gather_lanes(const void* d_rows, int64_t nrows, int row_bytes, const int32_t* d_idx, int64_t n,
                                  int lanes_per_row, unsigned long long* d_sink, void* stream);

/* ---- search: coarse quantizer (A2 + A3) -------------------------------- */

/* Exact top-nprobe lists per query, ascending (distance, list id), with the
 * prune rule of prune_and_count_fused_kernel (gpu_global.cu:43-50): a probe
 * whose distance exceeds best*prune_ratio becomes 0xFFFFFFFF.  Replaces the
 * cuVS CAGRA call (search_pipeline.cu:341; cagra_adapter.cuh:38-68) with an
 * MFMA GEMM plus an exact re-score.  nprobe <= 256. */
size_t fgpu_coarse_workspace_bytes(int nq, int nlist);
fgpu_status fgpu_coarse_search(const fgpu_index* idx, const float* d_queries, int nq, int nprobe,
                               float prune_ratio, uint32_t* d_probe_ids, float* d_probe_dists,
                               void* d_workspace, size_t workspace_bytes, void* stream);
/* fgpu_coarse_search plus instrumentation (no reference counterpart): adds to
 * d_stats[0..1] (device, caller-zeroed, uint64) the centroids re-scored
 * exactly over all queries and the queries whose margin admitted more than
 * 512 centroids (those re-score every centroid).  Results are unchanged. */
fgpu_status fgpu_coarse_search_stats(const fgpu_index* idx, const float* d_queries, int nq, int nprobe,
                                     float prune_ratio, uint32_t* d_probe_ids, float* d_probe_dists,
                                     unsigned long long* d_stats, void* d_workspace, size_t workspace_bytes,
                                     void* stream);

/* The prune step of prune_and_count_fused_kernel (gpu_global.cu:43-50), in
 * place: a probe whose distance exceeds (its query's first distance) *
 * prune_ratio becomes 0xFFFFFFFF. */
fgpu_status fgpu_prune_probes(uint32_t* d_probe_ids, const float* d_probe_dists, int nq, int nprobe,
                              float prune_ratio, void* stream);

/* counts[q] = sum of list sizes over surviving probes; offsets = exclusive
 * scan with offsets[nq] = total (gpu_global.cu:31-77, 704-723). */
fgpu_status fgpu_probe_counts(const fgpu_index* idx, const uint32_t* d_probe_ids, int nq, int nprobe,
                              int32_t* d_counts, int32_t* d_offsets, void* stream);

/* ---- search: LUT + ADC scan + top-k (A4-A6, A10, plain IVF-PQ) ---------- */

/* The k best (ADC distance, vector id) over every vector of every surviving
 * probed list; padding id -1 / distance FLT_MAX.  Equals run_gpu_batch_logic
 * (gpu_global.cu:679-874) with p1_lists = nprobe, limit_k = k, rerank_m = k.
 * k <= 64; nprobe above 64 runs a kernel that scans every probed list (no
 * list bound; same results).  d_probe_dists (may be NULL) takes the place of the reference's
 * d_cagra_dists: fgpu_coarse_search's distances for these probes, which the
 * scan then uses for its exact list bounds instead of recomputing them from
 * the centroids.  Non-NULL, they must be exactly the distances
 * fgpu_coarse_search or fgpu_coarse_graph_search returned for these probes:
 * the bounds allow only the rounding of that form, so other distances (a
 * GEMM's expanded ||q||^2 + ||c||^2 - 2 q.c, an approximation) can make the
 * scan skip lists that hold top-k vectors; pass NULL for them.  With valid
 * distances or NULL the results are the same. */
fgpu_status fgpu_adc_search(const fgpu_index* idx, const float* d_queries, int nq,
                            const uint32_t* d_probe_ids, const float* d_probe_dists, int nprobe, int k,
                            int32_t* d_out_ids, float* d_out_dists, void* stream);

/* fgpu_adc_search plus instrumentation (no reference counterpart): adds to
 * d_stats[0..6] (device, caller-zeroed, uint64) the number of vectors whose
 * codes the scan loaded, the number of LUTs built, the number of probed
 * lists the scan skipped because a lower bound on every distance in the list
 * exceeded the running k-th distance, and per-workgroup shader clocks (set-up,
 * a builder wave, a scanner wave, the whole workgroup).  Results equal
 * fgpu_adc_search's. */
fgpu_status fgpu_adc_search_stats(const fgpu_index* idx, const float* d_queries, int nq,
                                  const uint32_t* d_probe_ids, const float* d_probe_dists, int nprobe, int k,
                                  int32_t* d_out_ids, float* d_out_dists, unsigned long long* d_stats,
                                  void* stream);

/* coarse + ADC in one call: the same results as fgpu_coarse_search followed
 * by fgpu_adc_search.  For k <= 64 on the geometries (dim, pq_m) = (128, 16),
 * (128, 32), (128, 64), (96, 48) the scan part runs as an MFMA screen with an
 * exact rescore (no per-(query, list) LUT): every query's first list gives an
 * upper bound T on its k-th distance, every probed vector whose rigorous lower
 * bound does not exceed T is rescored with the reference's direct ADC form
 * (gpu_global.cu:259-319, bit-identical to the LUT sum), and the few queries
 * it cannot settle (a first list shorter than k, more than 512 candidates)
 * are scanned by the LUT kernel.  That needs fgpu_search_workspace_bytes; a
 * smaller workspace that still holds the coarse step runs the LUT kernels. */
size_t fgpu_search_workspace_bytes(int nq, int nlist, int nprobe);
fgpu_status fgpu_search(const fgpu_index* idx, const float* d_queries, int nq, int nprobe, int k,
                        float prune_ratio, int32_t* d_out_ids, float* d_out_dists,
                        void* d_workspace, size_t workspace_bytes, void* stream);
/* Instrumentation of the last fgpu_search on this workspace (waits for
 * `stream`; no reference counterpart): h_stats[0..7] = (query, list) pairs
 * screened for the thresholds, lists screened in the second round, (query,
 * list) pairs screened there, candidates rescored, the largest candidate count
 * of a query, queries handed to the LUT kernel, queries with a threshold
 * from the screen (not those whose candidates are every vector of their
 * probes: no usable probe, or one probe holding fewer than k vectors), 0;
 * h_stats[8..15] the clocks of FGPU_OPT_SCREEN_CLOCKS;
 * h_stats[16..19] = (query, vector) pairs screened in round 1 and round 2,
 * MFMA tiles (32 queries x 32 vectors) run in round 1 and round 2.  Only
 * meaningful after a call that took the screen. */
fgpu_status fgpu_search_screen_stats(const fgpu_index* idx, int nq, int nprobe, const void* d_workspace,
                                     size_t workspace_bytes, void* stream, long long* h_stats, int n_stats);
/* 1 when the index carries the screen's arrays (built at creation for the
 * geometries above when decoded norms stay below 2^40). */
int fgpu_index_screen_ready(const fgpu_index* idx);

/* Per-index options (no reference counterpart).  They affect only later
 * calls on this index, never another index:
 *   FGPU_OPT_LIST_SKIP  0: the LUT scan reads every probed list (timing of the
 *                       scan without its list bound; same results), 1 default;
 *   FGPU_OPT_SPIN_LIMIT polls before a flow-kernel wait gives up (0 = automatic;
 *                       a tiny limit makes give-ups certain while every wave
 *                       still runs to the end of the kernel);
 *   FGPU_OPT_TWO_PHASE_SPLIT phase 1 of fgpu_two_phase_search on `split`
 *                       workgroups a query (0 = automatic: split only batches
 *                       too small to fill the GPU; 1 = never; s >= 2 = s, at
 *                       most p1; limit_k <= 64 only; same results);
 *   FGPU_OPT_SCREEN     0: fgpu_search runs the LUT kernels, and
 *                       fgpu_two_phase_search phase 1 in its own kernel; 1
 *                       default;
 *   FGPU_OPT_TWO_PHASE_SCREEN phase 1 of fgpu_two_phase_search (limit_k <=
 *                       64) through the MFMA screen: 0 automatic (batches of
 *                       1024 queries or more), 1 never, 2 always; same
 *                       results;
 *   FGPU_OPT_SCREEN_CLOCKS 1: the screen kernels add their waves' shader
 *                       clocks (before the first item, item set-up, tile
 *                       loops, after the tiles; round 1 then round 2) to the
 *                       counters fgpu_search_screen_stats returns in
 *                       h_stats[8..15]; 0 default;
 *   FGPU_OPT_STAGE_EVENTS 1: fgpu_search records HIP events on its stream
 *                       between its stages (fgpu_search_stage_times), and so
 *                       does fgpu_two_phase_search when its phase 1 runs
 *                       through the screen; 0 default.  The events belong to
 *                       the index, so calls that overlap on one index
 *                       overwrite each other's. */
#define FGPU_OPT_LIST_SKIP 1
#define FGPU_OPT_SPIN_LIMIT 2
#define FGPU_OPT_SCREEN 3
#define FGPU_OPT_SCREEN_CLOCKS 4
#define FGPU_OPT_TWO_PHASE_SPLIT 5
#define FGPU_OPT_STAGE_EVENTS 6
#define FGPU_OPT_TWO_PHASE_SCREEN 7
fgpu_status fgpu_index_set_option(fgpu_index* idx, int option, int value);
/* With FGPU_OPT_STAGE_EVENTS on: the milliseconds of the last fgpu_search's
 * stages (waits for it), h_ms[0..6] = coarse step, the screen's zeroing and
 * round-1 pairs, round 1, round-2 pairs, round 2, rescore, and the LUT kernel
 * (the whole scan when the call did not take the screen; the screen stages
 * are then 0).  After an fgpu_two_phase_search whose phase 1 took the screen
 * (the last call of the two on the index): h_ms[0] = the virtual queries'
 * set-up, h_ms[1..5] the same screen stages, h_ms[6] the LUT hand-off, the
 * pool fill and the second half of the two-phase kernel (threshold, phase 2,
 * final select), for the last chunk of virtual queries.  No reference
 * counterpart. */
fgpu_status fgpu_search_stage_times(const fgpu_index* idx, float* h_ms, int n);

/* ---- search without allocation ----------------------------------------- */

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): fgpu_search with its scratch (probe ids and distances,
 * query norms, the coarse estimate tile, the screen's buckets and candidates)
 * in a file-scope device array of FGPU_NOALLOC_SCRATCH_BYTES that each GPU the
 * library runs on holds until the process ends, instead of a caller workspace.
 * Queries run in chunks of fgpu_search_noalloc_max_rows(nlist, nprobe) rows
 * (sized so the screen path fits when 64 rows of it do, else for the LUT
 * kernel); results equal fgpu_search's.  FGPU_ERR_WORKSPACE when not even 64 rows fit (nlist above
 * about 120k at nprobe 32).  No hipMalloc, hipFree or allocating library call.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other host threads) race and must be serialised by the
 * caller.  Index creation resolves the array's address on the current device,
 * so the first call may itself be under graph capture. */
#define FGPU_NOALLOC_SCRATCH_BYTES (32u << 20)
size_t fgpu_search_noalloc_max_bytes(void);
int fgpu_search_noalloc_max_rows(int nlist, int nprobe);
fgpu_status fgpu_search_noalloc(const fgpu_index* idx, const float* d_queries, int nq, int nprobe, int k,
                                float prune_ratio, int32_t* d_out_ids, float* d_out_dists, void* stream);

/* ---- search: two-phase pruned scan + top-rerank_m (A6-A10) ------------- */

/* The general form of run_gpu_batch_logic (gpu_global.cu:679-874) after the
 * coarse step.  Phase 1 (ivf_scan_phase1_kernel, :321-390): for the first
 * p1 = min(nprobe, p1_lists) probes, the w = min(n_l, limit_k) best vectors of
 * each list are candidates and the w-th distance is the list's cutoff (0 for a
 * pruned or empty probe).  Threshold (compute_threshold_kernel, :394-426):
 * thr = threshold_coeff * min(cutoff > 0), FLT_MAX if none.  Phase 2
 * (ivf_scan_phase2_kernel, :428-527): every vector of the other probed lists
 * with distance <= thr is a candidate.  Outputs (compaction + sort + gather,
 * :533-576, 798-867): the rerank_m best candidates ascending by (distance, id)
 * in d_top_ids/d_top_dists [nq][rerank_m] (pad -1 / FLT_MAX) and
 * d_top_counts[nq] = min(#candidates, rerank_m).  d_list_cutoffs [nq][p1] and
 * d_thresholds [nq] are optional (NULL).  Whole lists are scanned (the
 * reference stops at 1024 items), every passing vector is emitted once and
 * all rerank_m entries are gathered.  No host synchronisation and no pool
 * reallocation: the candidate pool is a bounded workspace, kept exact by
 * selecting the rerank_m best whenever it would overflow.  limit_k <= 4096 (above 64 a
 * slower phase 1 that cuts each list's keys to its limit_k best in the pool),
 * rerank_m <= 131072 (the reference's default is 10000), nprobe <= 256.  A workspace smaller than the returned size
 * is used in query chunks (it must hold at least one query's pool). */
size_t fgpu_two_phase_workspace_bytes(int nq, int nprobe, int p1_lists, int limit_k, int rerank_m);
fgpu_status fgpu_two_phase_search(const fgpu_index* idx, const float* d_queries, int nq,
                                  const uint32_t* d_probe_ids, int nprobe, int p1_lists, int limit_k,
                                  float threshold_coeff, int rerank_m, int32_t* d_top_ids,
                                  float* d_top_dists, int32_t* d_top_counts, float* d_list_cutoffs,
                                  float* d_thresholds, void* d_workspace, size_t workspace_bytes,
                                  void* stream);

/* fgpu_two_phase_search that also writes d_pre_cut [nq]: each query's
 * candidates before the rerank_m cut, the count the reference accumulates in
 * d_atomic (query_atomic_counters, gpu_global.cu:349, 493-526; summed by
 * search_pipeline.cu:455-457 for its pruning figures): the sum over the
 * phase-1 lists of min(n_l, limit_k) plus every phase-2 vector with dist <=
 * thr.  Results are those of fgpu_two_phase_search; phase 2 then skips lists
 * against thr itself, not against the pool's admission bound, so a batch
 * whose pools overflow may take longer. */
fgpu_status fgpu_two_phase_search_precut(const fgpu_index* idx, const float* d_queries, int nq,
                                         const uint32_t* d_probe_ids, int nprobe, int p1_lists, int limit_k,
                                         float threshold_coeff, int rerank_m, int32_t* d_top_ids, float* d_top_dists,
                                         int32_t* d_top_counts, float* d_list_cutoffs, float* d_thresholds,
                                         int32_t* d_pre_cut, void* d_workspace, size_t workspace_bytes,
                                         void* stream);

/* fgpu_two_phase_search plus instrumentation (no reference counterpart): adds
 * to d_stats[0..19] (device, caller-zeroed, uint64) the vectors whose codes
 * were loaded, the LUTs built, the phase-2 lists skipped by the list lower
 * bound, the phase-2 candidates appended, the shader clocks each workgroup
 * spent in set-up, phase 1, phase 2 and the final select + sort, and the
 * phase-1 clocks up to the LUT barrier, in the scan and in the merge; and
 * when phase 1 runs through the MFMA screen (limit_k <= 64, see
 * fgpu_two_phase_search), d_stats[11..19]: the virtual queries screened (one
 * per query and phase-1 probe), their candidates, those handed to the LUT
 * kernel, and of these the ones without a threshold and the ones with more
 * candidates than the screen keeps; the (query, vector) pairs screened in
 * rounds 1 and 2, and the 32 x 32 MFMA tiles run in rounds 1 and 2.  Results
 * are unchanged. */
fgpu_status fgpu_two_phase_search_stats(const fgpu_index* idx, const float* d_queries, int nq,
                                        const uint32_t* d_probe_ids, int nprobe, int p1_lists, int limit_k,
                                        float threshold_coeff, int rerank_m, int32_t* d_top_ids,
                                        float* d_top_dists, int32_t* d_top_counts,
                                        unsigned long long* d_stats, void* d_workspace,
                                        size_t workspace_bytes, void* stream);

/* ---- search: exact rerank (A11) ---------------------------------------- */

/* run_gpu_rerank (gpu_global.cu:603-673): per query, walk the first
 * d_top_counts[q] ids of d_top_ids [nq][rerank_m] in mini-batches of
 * mini_batch; exact squared L2 against d_base [n][dim] (sequential fused
 * chain, gpu_global.cu:636); merge into the running top-k ascending by
 * (distance, id); chg = ids new to the top-k; stable += 1 if chg/k <= eps else
 * 0; stop after beta stable batches or when candidates run out.  Ids outside
 * [0, n) are skipped.  All k + mini_batch entries are sorted (the reference
 * sorts only 128 of them).  d_visited [nq] (optional) = candidates evaluated.
 * dim 96 or 128, d_base 16-byte aligned, k <= 256, mini_batch <= 128. */
fgpu_status fgpu_rerank(const float* d_queries, int nq, int dim, const float* d_base, int64_t n,
                        const int32_t* d_top_ids, const int32_t* d_top_counts, int rerank_m, int k,
                        int mini_batch, float eps, int beta, int32_t* d_final_ids, float* d_final_dists,
                        int32_t* d_visited, void* stream);
/* fgpu_rerank with the number of mini-batches computed at once stated per
 * call (no reference counterpart): spec 0 automatic (four while the batch
 * leaves CUs free, else one), 1 one, any other value four.  Results and
 * visit counts are the same whatever spec. */
fgpu_status fgpu_rerank_spec(const float* d_queries, int nq, int dim, const float* d_base, int64_t n,
                             const int32_t* d_top_ids, const int32_t* d_top_counts, int rerank_m, int k,
                             int mini_batch, float eps, int beta, int32_t* d_final_ids, float* d_final_dists,
                             int32_t* d_visited, int spec, void* stream);
/* fgpu_rerank_spec that also writes the state the reference's rerank leaves
 * in stab[] and fin[] (gpu_global.cu:603-609, 615, 653-662; run_gpu_rerank's
 * d_stable_cnt and d_finished): d_stable_cnt [nq] (optional) = the stable
 * count after the last batch evaluated; d_finished [nq] (optional, one byte a
 * query, 0 or 1) = 1 when the walk stopped on stability or reached an offset
 * below rerank_m at or past the query's candidates. */
fgpu_status fgpu_rerank_state(const float* d_queries, int nq, int dim, const float* d_base, int64_t n,
                              const int32_t* d_top_ids, const int32_t* d_top_counts, int rerank_m, int k,
                              int mini_batch, float eps, int beta, int32_t* d_final_ids, float* d_final_dists,
                              int32_t* d_visited, int32_t* d_stable_cnt, uint8_t* d_finished, int spec,
                              void* stream);

/* coarse + two-phase + rerank in one call: the SearchPipeline per-batch path
 * (search_pipeline.cu:341-361) with final_k = k. */
size_t fgpu_search_rerank_workspace_bytes(int nq, int nlist, int nprobe, int p1_lists, int limit_k,
                                          int rerank_m);
fgpu_status fgpu_search_rerank(const fgpu_index* idx, const float* d_queries, int nq, int nprobe,
                               float prune_ratio, int p1_lists, int limit_k, float threshold_coeff,
                               int rerank_m, const float* d_base, int64_t n, int k, int mini_batch,
                               float eps, int beta, int32_t* d_out_ids, float* d_out_dists,
                               void* d_workspace, size_t workspace_bytes, void* stream);

/* ---- exact nearest centroids (A13 / A2 core) -------------------------- */

/* For each row x of d_x [n][dim]: the p nearest rows of d_c [nc][dim] by
 * exact squared L2 in the reference's device form (sequential fused
 * multiply-add, tune_parameters.cu:39-46), ascending (distance, index).
 * p = 1 is the k-means assignment (kmeans_gpu.cuh:197-229, lowest index wins
 * ties).  MFMA GEMM + rigorous-margin re-score.  p <= 256. */
size_t fgpu_l2_topk_workspace_bytes(int64_t n, int nc);
fgpu_status fgpu_l2_topk(const float* d_x, int64_t n, const float* d_c, int nc, int dim, int p,
                         int32_t* d_ids, float* d_dists, void* d_workspace, size_t workspace_bytes,
                         void* stream);

/* ---- exact kNN ground truth (A18) -------------------------------------- */

/* brute_force_search_kernel (tune_parameters.cu:49-96): for each query row of
 * d_queries [nq][dim], the k nearest rows of d_base [n][dim] by exact squared
 * L2 in the reference's device form, ascending (distance, row index) -- the
 * reference's strict-< insertion keeps the earlier row on ties; padding -1 /
 * FLT_MAX when n < k.  The base streams through in chunks of 4096 rows: an
 * MFMA GEMM estimate per chunk, then an exact re-score of every row that the
 * rigorous error margin cannot rule out, merged into each query's running
 * top-k.  k <= 128, dim <= 256 and a multiple of 4, n < 2^31. */
size_t fgpu_knn_exact_workspace_bytes(int nq, int64_t n);
fgpu_status fgpu_knn_exact(const float* d_queries, int nq, const float* d_base, int64_t n, int dim, int k,
                           int32_t* d_ids, float* d_dists, void* d_workspace, size_t workspace_bytes,
                           void* stream);

/* ---- graph search (A19) ------------------------------------------------- */

/* The role of cuVS CAGRA search (cagra_adapter.cuh:38-68: itopk list,
 * search width, maximum iterations) over a caller-supplied fixed-degree
 * adjacency d_graph [n][degree] (ids outside [0, n) are skipped) of the base
 * vectors d_base [n][dim].  cuVS is not in the reference, so the algorithm is
 * this library's own, deterministic one: 64 seeded start nodes; each step
 * expands the `width` best unexpanded entries of the itopk list; candidates
 * whose bit in a per-query 2^16-bit visited bitmap (in LDS) was already set
 * are dropped; exact squared L2 (sequential fused chain); merge by
 * (distance, id); stop when nothing is left to expand or after max_iter steps.
 * Outputs the k best ids/dists [nq][k] and, optionally, d_iters [nq] (steps)
 * and d_evals [nq] (exact distances computed, i.e. base rows read).
 * dim 96 or 128, d_base 16-byte aligned, k <= itopk <= 64, width <= 8,
 * width * degree <= 128. */
fgpu_status fgpu_graph_search(const float* d_queries, int nq, const float* d_base, int64_t n, int dim,
                              const int32_t* d_graph, int degree, int itopk, int width, int max_iter, int k,
                              uint64_t seed, int32_t* d_out_ids, float* d_out_dists, int32_t* d_iters,
                              int32_t* d_evals, void* stream);

/* ---- graph coarse quantizer (the reference's CAGRA-over-centroids mode) -- */

/* The reference builds a cuVS CAGRA graph over the coarse centroids
 * (build_cagra_index, cagra_adapter.cuh:10-27: graph_degree 8, intermediate
 * degree 16, called from build_global) and walks it for every query batch
 * (search_cagra_index, cagra_adapter.cuh:38-68, from search_pipeline.cu:341).
 * Here, with F(v) the 2*degree nearest other centroids of v in tie-rule order
 * (fgpu_knn_exact), row v of d_graph [nlist][degree] holds the first
 * degree - degree/2 entries of F(v), then the reverse edges: every u whose
 * first `degree` entries of F(u) include v, by (rank of v in F(u), u), then
 * the rest of F(v), skipping ids already present, up to degree ids.  Reverse
 * edges as in CAGRA (Ootomo et al., 2023) keep the graph navigable; CAGRA's
 * NN-descent and rank-based pruning and its file (cagra_centroids.index) are
 * not reproduced.  1 <= degree <= 64, 2 * degree < nlist.  The reverse-edge
 * step runs on the host: the call synchronises `stream`.
 * Workspace: fgpu_coarse_graph_workspace_bytes(nlist, degree). */
size_t fgpu_coarse_graph_workspace_bytes(int nlist, int degree);
fgpu_status fgpu_coarse_graph_build(const fgpu_index* idx, int degree, int32_t* d_graph, void* d_workspace,
                                    size_t workspace_bytes, void* stream);
/* CAGRA's reverse-edge step on host arrays (no reference counterpart: the
 * reference gets its graphs from cuVS, cagra_adapter.cuh:10-26): h_fwd
 * [n][width] holds each node's forward candidates nearest first (-1 and out-
 * of-range ids are skipped); row v of h_out [n][degree] gets its nearest
 * degree - degree / 2 forward edges, then the nodes u whose first `degree`
 * forward edges include v, ordered by (rank of v there, u), then the rest of
 * its forward list, without repeats or self edges, -1 padded.  nthreads <= 0:
 * 16 host threads.  fgpu_coarse_graph_build uses it over the centroids. */
fgpu_status fgpu_graph_add_reverse(const int32_t* h_fwd, int64_t n, int width, int degree, int32_t* h_out,
                                   int nthreads);

/* Approximate top-nprobe lists per query by that walk (itopk, width,
 * max_iter, seed as in fgpu_graph_search; nprobe <= itopk <= 64; the
 * reference uses itopk = max(32, nprobe), width 4, max_iter 200).  A query's
 * seed nodes depend on seed and on its index first_query + i, so a query set
 * split into batches gets the same results as one call.  Ascending
 * (distance, list id) with exact distances (the same chain as
 * fgpu_coarse_search), then the same prune rule; slots the walk leaves empty
 * are 0xFFFFFFFF.  When the walk evaluates every centroid (the visited bitmap
 * holds every id below 16384 without a collision) the result equals
 * fgpu_coarse_search's bit for bit. */
fgpu_status fgpu_coarse_graph_search(const fgpu_index* idx, const float* d_queries, int nq, int first_query,
                                     int nprobe, const int32_t* d_graph, int degree, int itopk, int width,
                                     int max_iter, uint64_t seed, float prune_ratio, uint32_t* d_probe_ids,
                                     float* d_probe_dists, void* stream);

/* ---- index build (A13-A17) -------------------------------------------- */

/* One Lloyd update (kmeans_gpu.cuh:81-116) with deterministic fixed-point
 * sums: c = (float)(sum(round(x*2^shift)) * 2^-shift) * (1.0f/count).
 * empty_rule 0 = empty cluster becomes zero (kmeans_gpu.cuh:293,110), 1 = keeps
 * its centroid.  Workspace: fgpu_kmeans_workspace_bytes(k, dim). */
size_t fgpu_kmeans_workspace_bytes(int k, int dim);
fgpu_status fgpu_kmeans_update(const float* d_x, int64_t n, const int32_t* d_assign, int k, int dim,
                               int shift, int empty_rule, float* d_centroids, int32_t* d_counts,
                               void* d_workspace, size_t workspace_bytes, void* stream);
/* Fixed-point shift for data with max |x| = maxabs and n rows. */
int fgpu_fixed_shift(float maxabs, int64_t n);

/* Full k-means (run_kmeans_gpu, kmeans_gpu.cuh:234-324): init_mode 0 = the
 * reference's strided mt19937 init (kmeans_gpu.cuh:259-267), 1 = k-means++
 * seeding; then iters x (assign, update).  d_centroids [k][dim] out. */
fgpu_status fgpu_kmeans_fit(const float* d_x, int64_t n, int dim, int k, int iters, int init_mode,
                            uint64_t seed, float* d_centroids, int32_t* d_assign_out, void* stream);

/* Residual PQ codebook training (train_residual_pq_codebooks, pq_utils.h:77-138):
 * d_codebook [pq_m][256][dim/pq_m] out. */
fgpu_status fgpu_pq_train(const float* d_x, int64_t n, int dim, int pq_m, const int32_t* d_assign,
                          const float* d_centroids, int sample_size, int iters, float* d_codebook,
                          void* stream);
/* Residual PQ encoding (encode_residuals_kernel, kmeans_gpu.cuh:403-445). */
fgpu_status fgpu_pq_encode(const float* d_x, int64_t n, int dim, int pq_m, const int32_t* d_assign,
                           const float* d_centroids, const float* d_codebook, uint8_t* d_codes,
                           void* stream);
/* The same with the distance form chosen: fma_mode 1 = the device kernel's
 * fused chain (kmeans_gpu.cuh:428-433, as fgpu_pq_encode), 0 = the host twin
 * encode_residuals_to_pq (pq_utils.h:141-175, built without FMA): every
 * product and sum rounded separately.  The two can pick different codewords
 * on near ties. */
fgpu_status fgpu_pq_encode_form(const float* d_x, int64_t n, int dim, int pq_m, const int32_t* d_assign,
                                const float* d_centroids, const float* d_codebook, int fma_mode,
                                uint8_t* d_codes, void* stream);

/* build_global (build_global.cu:21-258) without rebalancing and CAGRA: k-means
 * (nlist, kmeans_iters), assignment, PQ training (pq_iters, sample_size),
 * encoding and list assembly.  Outputs are host arrays in ivf_data.bin layout:
 * h_offsets [nlist+1], h_ids [n], h_codes [n][pq_m], h_centroids [nlist][dim],
 * h_codebook [pq_m][256][dim/pq_m]. */
fgpu_status fgpu_build_ivfpq(const float* d_x, int64_t n, int dim, int nlist, int pq_m,
                             int kmeans_iters, int init_mode, uint64_t seed, int pq_iters,
                             int sample_size, int32_t* h_offsets, int32_t* h_ids, uint8_t* h_codes,
                             float* h_centroids, float* h_codebook, void* stream);

/* fgpu_build_ivfpq with the k-means trained on a sample: rows
 * floor(j * n / train_rows), j < train_rows (a systematic sample; BASELINE
 * config 4 trains on 1M of 10M rows), then every row is assigned to its
 * nearest centroid and the PQ training, encoding and lists follow as in
 * fgpu_build_ivfpq.  train_rows <= 0 or >= n trains on every row, as
 * build_global does (build_global.cu:41). */
fgpu_status fgpu_build_ivfpq_sampled(const float* d_x, int64_t n, int dim, int nlist, int pq_m,
                                     int64_t train_rows, int kmeans_iters, int init_mode, uint64_t seed,
                                     int pq_iters, int sample_size, int32_t* h_offsets, int32_t* h_ids,
                                     uint8_t* h_codes, float* h_centroids, float* h_codebook, void* stream);

/* ---- offline parameter tuner (tune_parameters.cu:459-1053) ------------- */

/* Per (query, list) statistics of the tuner, one pair per entry.  Replaces the
 * per-item cudaMalloc + precompute_lut_kernel + compute_pq_dist_with_lut_kernel
 * + compute_exact_distances_kernel + host ranking of tune_parameters.cu:690-784
 * and the per-list cutoff of :843-900.  PQ distances use the tuner's own LUT
 * (tune_parameters.cu:101-123: per entry, a sequential fused chain over the
 * sub-vector of (q - c) - codeword; not the search LUT) summed in ascending
 * subspace order (:127-145); exact distances are sequential fused chains over
 * the dimensions (:148-166) against d_base rows (vector ids index d_base).
 * For pair p (query row d_pair_query[p] of d_queries, list d_pair_list[p]):
 *   with d_pair_target (vector id t, or -1): at the first list position
 *     holding t, d_target_pq / d_target_exact get its distances and d_pq_rank /
 *     d_exact_rank 1 + the list's vectors strictly below them (:766-778);
 *     0 ranks and -1 distances when t is absent (d_base NULL: no exact part);
 *   with d_pair_kth (k, or <= 0): d_kth_pq gets the min(k, n_l)-th smallest PQ
 *     distance of the list (:893-899), 0 for an empty list.
 * Pairs naming a query row outside [0, nq) or a list outside [0, nlist) get
 * the "absent" values.  dim <= 128, pq_m <= 64. */
fgpu_status fgpu_tune_list_stats(const fgpu_index* idx, const float* d_queries, int nq, const float* d_base,
                                 int64_t n_base, const int32_t* d_pair_query, const int32_t* d_pair_list,
                                 const int32_t* d_pair_target, const int32_t* d_pair_kth, int npairs,
                                 float* d_target_pq, float* d_target_exact, int32_t* d_pq_rank,
                                 int32_t* d_exact_rank, float* d_kth_pq, void* stream);
/* compute_percentile_int / compute_percentile (tune_parameters.cu:170-183):
 * the sorted sample's element at floor(n * pct) (product in single precision),
 * clamped to the last element; 0 for an empty sample.  Host only. */
int fgpu_tune_percentile_int(const int32_t* values, int64_t n, float pct);
float fgpu_tune_percentile(const float* values, int64_t n, float pct);
/* find_elbow_point (tune_parameters.cu:199-456) without its printed tables:
 * the recommended phase-1 list count (1-based) from the ground-truth hits per
 * coarse rank; *coverage gets the cumulative coverage there.  Host only. */
int fgpu_tune_elbow(const int32_t* hits_per_rank, int n, int64_t total_hits, float* coverage);

/* ---- files (utils.h, build_global.cu:242-252) -------------------------- */

fgpu_status fgpu_write_ivf_data(const char* path, int64_t total, int nlist, int pq_m, int dim,
                                const int32_t* offsets, const int32_t* ids, const uint8_t* codes,
                                const float* centroids);
/* Reads the header: *total, *nlist. */
fgpu_status fgpu_read_ivf_header(const char* path, int64_t* total, int* nlist);
fgpu_status fgpu_read_ivf_data(const char* path, int pq_m, int dim, int32_t* offsets, int32_t* ids,
                               uint8_t* codes, float* centroids);
fgpu_status fgpu_write_fvecs(const char* path, const float* v, int64_t n, int dim);
/* fvecs/ivecs readers (utils.h:22-48, 75-95): *n rows of dim; pass out=NULL to query. */
fgpu_status fgpu_read_fvecs(const char* path, int dim, int64_t* n, float* out);
fgpu_status fgpu_read_ivecs(const char* path, int* dim, int64_t* n, int32_t* out);

/* ---- synthetic data (no reference counterpart) ------------------------- */

/* Seeded Gaussian mixture, identical on every host (counter-based splitmix64 +
 * Box-Muller in double).  set 0 = base vectors, 1 = queries. */
void fgpu_gen_gmm(int64_t n, int dim, int ncomp, double lo, double hi, double sig_lo, double sig_hi,
                  uint64_t seed, int set, float* out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif /* FUSIONGPU_H_ */
