/*
 * flashgann.h -- C ABI of the MI355X (gfx950) adaptive graph beam search.
 *
 * Drop-in boundary for the reference's search path.  The reference exposes it
 * as a C++ member function, not a plugin:
 *   QuantizationGraph::QuantizationGraph(num_node, dim, degree, codebook_path)
 *       include/qg.hpp:17-42
 *   void QuantizationGraph::gpu_search_adaptive(int nq, const float *queries,
 *       int K, vidType *result_idx, int beam_sz, double &elapsed)
 *       include/qg.hpp:62-63, gpu_search_adaptive.cu:12-114
 *   __global__ QuantizedPrunedBeamSearch(...)   src/adaptive_search.cuh:5-11
 * The entry points below carry the same arguments with the same meaning, as
 * plain pointers and sizes.  Buffers are caller-owned; the index owns its
 * device copy of the codebook (uploaded once, instead of once per call as
 * gpu_search_adaptive.cu:65-71 does).
 *
 * Every function returns 0 on success and a negative FG_E* code on failure;
 * fg_last_error() then describes the failure (thread-local string).
 *
 * An index lives on the device that was current when it was created, and its
 * searches must be called with that device current (FG_EINVAL otherwise).
 * fg_search keeps its staging buffers in the index: calls on one index come
 * from one host thread at a time; different indices are independent.  One
 * search covers at most 2^31 - 1 queries (one workgroup each).
 */
#ifndef FLASHGANN_H
#define FLASHGANN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FG_OK 0
#define FG_EINVAL -1     /* argument outside the supported range */
#define FG_ENOMEM -2     /* device allocation failed / not enough free memory */
#define FG_EDEVICE -3    /* HIP runtime error */
#define FG_EIO -4        /* file missing or truncated */

#define FG_METRIC_L2 0   /* include/metric.hpp:9 METRIC_L2 */
#define FG_METRIC_IP 1   /* include/metric.hpp:9 METRIC_IP */

#define FG_ENTRY_AUTO 0xFFFFFFFFu  /* qg.hpp entry field == UINT32_MAX */

typedef struct fg_index fg_index;

/* Codebook geometry in float units (include/qg.hpp:66-73). */
typedef struct {
    uint32_t dim;
    uint32_t padded_dim;
    uint32_t degree;
    uint32_t entry;
    uint64_t npoints;
    uint64_t code_offset;
    uint64_t factor_offset;
    uint64_t neighbor_offset;
    uint64_t row_offset;
    int metric;
} fg_index_info;

/* Per-call statistics. */
typedef struct {
    double elapsed_s;        /* host wall clock around launch + sync
                                (gpu_search_adaptive.cu:98-107) */
    float kernel_ms;         /* HIP-event time of the search kernel */
    uint32_t lds_bytes;      /* dynamic LDS per workgroup (one query) */
    uint32_t visited_slots;  /* visited-table slots used by the kernel */
} fg_stats;

/* Per-query work counters (6 x uint32 per query when requested):
 * iterations, expansions, ids_read, estimates, exact, stage2_iter. */
#define FG_COUNTERS_PER_QUERY 6

/* Replaces the QuantizationGraph constructor's upload half
 * (include/qg.hpp:17-42 + gpu_search_adaptive.cu:65-71): copies npoints rows
 * of the codebook (row layout of fg_index_info) and padded_dim signs to the
 * current device.  entry == FG_ENTRY_AUTO picks the node nearest the float
 * centroid with the reference's host routine semantics
 * (include/common.hpp:26-47, gpu_search_adaptive.cu:74-77). */
int fg_index_create(const float *rows, uint64_t npoints, uint32_t dim, uint32_t degree,
                    const float *signs, uint32_t entry, int metric, fg_index **out);
/* (The search has kernels specialised for d = 128 / degree 32 and d = 96 /
 * degree 32 or 16 while the codebook is under 4 GiB; an index created with
 * the environment variable FG_FORCE_RUNTIME_GEOMETRY=1 uses the general
 * kernels instead.  Same results; a test knob.) */

/* Same as fg_index_create but reads the reference's codebook file
 * (include/qg.hpp:17-42); a truncated file is FG_EIO instead of being read
 * short. */
int fg_index_load(const char *codebook_path, uint64_t npoints, uint32_t dim, uint32_t degree,
                  int metric, fg_index **out);

/* Releases the index (the destructor, include/qg.hpp:44-47).  The searches
 * the index keeps track of (fg_search_stream's batches on its internal
 * streams, the last two-launch search) are waited for first; any other search
 * the caller queued with fg_search_device must have ended. */
void fg_index_destroy(fg_index *index);

int fg_index_get_info(const fg_index *index, fg_index_info *info);

/* Replaces QuantizationGraph::gpu_search_adaptive (gpu_search_adaptive.cu:12-114):
 * host queries (nq x dim float32, row-major) in, host result ids
 * (nq x K uint32) out.  stats->elapsed_s is the kernel-only time the reference
 * reports as `elapsed`.  counters may be NULL, else nq*6 uint32 (host). */
int fg_search(fg_index *index, const float *queries, uint32_t nq, uint32_t K, uint32_t beam,
              uint32_t *result_ids, uint32_t *counters, fg_stats *stats);

/* Allocation-free variant of fg_search.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory while they search (tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, results,
 * counters and statistics as fg_search, but the device copies of the queries,
 * result ids and counters are staged in a fixed area of
 * FG_NOALLOC_STAGING_BYTES that the library holds on each device until the
 * process ends (set up by fg_index_create), instead of buffers it allocates;
 * the call itself allocates nothing.  A call needs
 * align256(nq*dim*4) + align256(nq*K*4) [+ align256(nq*24) with counters]
 * bytes of it and is rejected with FG_EINVAL above the maximum (about 17,900
 * queries at dim 128, K 100, with counters).  Every call on one device
 * shares that area: calls on one device from several host threads take a
 * per-device host lock for their whole duration and run one after another
 * (the lock is host memory; nothing is allocated on the device).  Calls on
 * one index still come from one host thread at a time, as for fg_search. */
#define FG_NOALLOC_STAGING_BYTES (16u << 20)
int fg_search_noalloc(fg_index *index, const float *queries, uint32_t nq, uint32_t K, uint32_t beam,
                      uint32_t *result_ids, uint32_t *counters, fg_stats *stats);

/* Device-resident variant: d_queries, d_results (and d_counters, may be NULL)
 * are device pointers; the kernel is enqueued on `stream` (a hipStream_t, NULL
 * = default stream) and the call returns without synchronising.  This is the
 * kernel launch of gpu_search_adaptive.cu:99-103 on its own. */
int fg_search_device(fg_index *index, const float *d_queries, uint32_t nq, uint32_t K,
                     uint32_t beam, uint32_t *d_results, uint32_t *d_counters, void *stream);

/* Serving form of fg_search_device for a stream of query batches (the
 * reference has no counterpart: its gpu_search_adaptive.cu:99-103 launches
 * one kernel per call and synchronises).  The nq device-resident queries are
 * searched as consecutive batches of `batch` queries, batch b on internal
 * stream b % nstreams (1 <= nstreams <= 8, created on first use and owned by
 * the index), so one batch's last, partly filled wave slots overlap the next
 * batch's start.  Results land in query order in d_results (nq x K); each
 * query's ids are those fg_search_device returns.  All batches run after the
 * work already queued on `stream` and that stream's later work waits for
 * all of them; the call returns without synchronising.  Calls on one index
 * share its internal streams: issue them from one host thread. */
int fg_search_stream(fg_index *index, const float *d_queries, uint32_t nq, uint32_t K, uint32_t beam,
                     uint32_t *d_results, uint32_t batch, uint32_t nstreams, void *stream);

/* Diagnostics: the same search as fg_search_device, built with phase timers.
 * d_phase receives FG_PROFILE_SLOTS uint64 per query: shader-clock cycles
 * spent in query preparation + set-up, visited-table restore, beam merge,
 * controller + pick, single-expander scoring, single-expander exact
 * distances, speculative id loads + visited tests, speculative estimates +
 * selection + inserts, speculative exact distances, and the result write;
 * then the query's start and end on the device's constant 100 MHz clock.
 * No counterpart in the reference (its only diagnostics are printfs). */
#define FG_PROFILE_SLOTS 12
int fg_search_profile(fg_index *index, const float *d_queries, uint32_t nq, uint32_t K, uint32_t beam,
                      uint32_t *d_results, unsigned long long *d_phase, void *stream);

/* Dynamic LDS bytes one query's workgroup needs (the analogue of
 * calculate_shared_mem_size, src/adaptive_search_utils.cuh:152-176). */
uint32_t fg_lds_bytes(uint32_t dim, uint32_t beam, uint32_t degree);

/* Waves per query (1 or 2) that a search of nq queries at this K and beam
 * launches on the current device: two, the kernel's team form, when the batch
 * is too small to fill the device with one wave per query; FLASHGANN_TEAM=0/1
 * in the environment forces one form.  Results are identical either way.
 * Negative FG_E* on invalid arguments.  No counterpart in the reference (one
 * warp-per-parent block shape). */
int fg_search_waves(fg_index *index, uint32_t nq, uint32_t K, uint32_t beam);

/* Kernel launches (1 or 2) that fg_search / fg_search_device make for a
 * search of nq queries at this K and beam.  Two when the batch, in the
 * one-wave form, holds more queries than the device runs at once (6,144 at
 * d 128, degree 32, beam 256), for either metric, while the suspended state
 * stays within 1 GiB (about 400,000 queries at d 128, beam 256): every query
 * first runs to iteration 15 and an unfinished one keeps its state (beam,
 * candidates, controller, counters and prepared query) in memory the index
 * holds, then the unfinished queries resume in a second launch, those with
 * the largest best distance so far first, so the longest searches start
 * early.  The first such search of a larger batch allocates that memory,
 * which synchronises the device; if it cannot be allocated the search makes
 * one launch.
 * Results are identical either way; FLASHGANN_SLICE=0/1 in the environment
 * forces one launch / two wherever the form allows.  Device searches on one index that
 * overlap on different streams run one after another when they take two
 * launches.  fg_search_stream, fg_search_noalloc and a device search on a
 * stream that is being captured into a graph always make one.
 * Negative FG_E* on invalid arguments.  No counterpart in the reference (one
 * launch per call, gpu_search_adaptive.cu:99-103). */
int fg_search_launches(fg_index *index, uint32_t nq, uint32_t K, uint32_t beam);

/* Which kernels serve searches on this index: FG_GEOMETRY_FIXED, the
 * kernels specialised for d 128 / degree 32 and d 96 / degree 32 or 16,
 * whose row offsets are compile-time constants and whose row addresses are
 * 32-bit byte offsets (codebooks under 4 GiB), or FG_GEOMETRY_GENERAL, the
 * kernels with runtime offsets and 64-bit row addresses (other shapes,
 * codebooks of 4 GiB or more, FG_FORCE_RUNTIME_GEOMETRY=1).  Results are
 * identical either way; negative FG_E* for a NULL index.  Diagnostic, no
 * counterpart in the reference (which addresses rows as
 * size_t(node) * row_offset, src/adaptive_search.cuh:225, 366, 438). */
#define FG_GEOMETRY_FIXED 0
#define FG_GEOMETRY_GENERAL 1
int fg_search_geometry(const fg_index *index);

/* Query preparation only (utils.cuh:840-939): rotated query (padded_dim
 * float32), quantized levels (padded_dim uint8), and {low, high, width} plus
 * sum_q, for nq host queries.  Test hook for the preparation stage. */
int fg_query_prepare(fg_index *index, const float *queries, uint32_t nq, float *rotated,
                     uint8_t *quantized, float *low_high_width, int32_t *sum_q);

/* Estimates and exact distances for explicit (query, parent, neighbour slot)
 * triples, with both estimator variants (utils.cuh:941-1027) and the exact
 * distance (utils.cuh:269-305).  Test hook for the scoring stages.
 * est_lanes/est_seq/exact are n floats each; any may be NULL. */
int fg_score_edges(fg_index *index, const float *queries, uint32_t nq, const uint32_t *query_ix,
                   const uint32_t *parents, const uint32_t *slots, uint32_t n, float *est_lanes,
                   float *est_seq, float *exact);

const char *fg_last_error(void);
const char *fg_version(void);

#ifdef __cplusplus
}
#endif
#endif /* FLASHGANN_H */
