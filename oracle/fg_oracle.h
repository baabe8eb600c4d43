/*
 * fg_oracle.h -- CPU restatement of FlashGANN's adaptive graph beam search.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP search
 * path.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product path (flashgann_amd) never links, loads or calls
 * anything under oracle/.
 *
 * Every function restates one piece of the reference and cites the file:line
 * it follows (paths relative to the reference repository root).  Where the
 * reference is nondeterministic or relies on compiler choices, the oracle fixes
 * one legal behaviour and says so in the comment:
 *   - fp contraction (nvcc --fmad=true) is written as explicit fmaf() at the
 *     sites a contracting compiler fuses;
 *   - speculative (theta > 1) expansion: every task of one 8-task round tests
 *     the visited set as it stood when the round began, then inserts in
 *     (task, lane) order, so the lowest (task, lane) wins a duplicate child;
 *   - theta == 1 expansion: duplicate ids inside one neighbour list are
 *     inserted in index order (lowest index wins).
 *
 * Parity status of each piece is listed in the header comment of fg_oracle.c.
 */
#ifndef FG_ORACLE_H
#define FG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FGO_MAX_INDEX 0xFFFFFFFFu
#define FGO_MSB 0x80000000u
#define FGO_SEARCH_WIDTH 8        /* utils.cuh:26, adaptive_search_config.cuh:8 */
#define FGO_BUFFER_BOUND 32       /* adaptive_search_config.cuh:54 */
#define FGO_MAX_ITERATIONS 1024   /* adaptive_search_config.cuh:12 */
#define FGO_HASH_RESET 16         /* utils.cuh:683 */
#define FGO_BQUERY 6              /* common.hpp:17 */
#define FGO_MAX_BEAM 1024
#define FGO_MAX_DEGREE 1024
#define FGO_MAX_PADDED_DIM 2048

/* Codebook geometry (qg.hpp:66-73), all offsets in floats. */
typedef struct {
    uint32_t dim;
    uint32_t padded_dim;
    uint32_t degree;
    uint64_t code_offset;
    uint64_t factor_offset;
    uint64_t neighbor_offset;
    uint64_t row_offset;
} fgo_layout;

typedef struct {
    const float *data;   /* npoints * row_offset floats */
    const float *signs;  /* padded_dim floats */
    uint64_t npoints;
    fgo_layout lay;
    uint32_t entry;
    int use_ip;
} fgo_index;

/* Rotated / quantized query (utils.cuh:57-65, 840-939). */
typedef struct {
    float rotated[FGO_MAX_PADDED_DIM];
    uint8_t q[FGO_MAX_PADDED_DIM];
    uint8_t lut[4 * FGO_MAX_PADDED_DIM];
    float low, high, width;
    int32_t sum_q;
} fgo_query_factors;

/* Per-query work counters; the HIP kernel reports the same fields. */
typedef struct {
    uint32_t iterations;   /* main-loop iterations that reached expander picking */
    uint32_t expansions;   /* parents expanded */
    uint32_t ids_read;     /* neighbour ids read from parent rows */
    uint32_t estimates;    /* RaBitQ estimates evaluated */
    uint32_t exact;        /* exact distances evaluated (entry point included) */
    uint32_t stage2_iter;  /* first iteration run with theta > 1, or 0xFFFFFFFF */
} fgo_counters;

/* Optional per-iteration trace, for locating the first divergence. */
typedef struct {
    uint32_t iter;
    uint32_t theta;
    float rho;
    uint32_t n_parents;
    uint32_t parents[FGO_SEARCH_WIDTH];
    uint32_t top1;
    float top1_dist;
    float kth_cutoff;
    uint32_t n_cand;
    uint32_t cand_idx[FGO_BUFFER_BOUND];
    float cand_dist[FGO_BUFFER_BOUND];
    /* controller state after this iteration's update and expander record */
    int32_t stall;               /* top1_stall_iters */
    float last_expander_distance;
    float current_expander_distance;
    uint32_t restored;           /* 1 if the visited set was rebuilt this iteration */
} fgo_trace_rec;

/* Adaptive controller state (adaptive_search_utils.cuh:8-18). */
typedef struct {
    int spec_degree;
    float rho;
    int policy_iters;
    uint32_t top1_node;
    int top1_stall_iters;
    int warmup_done;
    float entry_distance;
    float last_expander_distance;
    float current_expander_distance;
} fgo_ctl_state;

/* ---- sizing helpers ---- */
int fgo_compute_layout(uint32_t dim, uint32_t degree, fgo_layout *out);
uint32_t fgo_round_up_pow2(uint32_t x);
uint32_t fgo_effective_sort_beam_size(uint32_t beam);
uint32_t fgo_hash_bitlen(uint32_t pbeam, uint32_t cbs, uint32_t reset_interval);
uint32_t fgo_candidate_buffer_capacity(uint32_t degree);
float fgo_max_rho_bound(uint32_t degree);
uint32_t fgo_keep_count_per_parent(uint32_t max_degree, float rho);
int fgo_keep_count_for_expander(uint32_t active, int theta, float rho, int kth_valid, uint32_t near);

/* ---- query preparation and estimators ---- */
void fgo_rotate(const float *src, const float *signs, int dim, int padded_dim, float *dst);
void fgo_query_prepare(const float *query, const float *signs, int dim, int padded_dim,
                       fgo_query_factors *qf);
uint32_t fgo_raw_lut(const fgo_query_factors *qf, const uint8_t *code, int padded_dim);
float fgo_estimate_lanes(const fgo_query_factors *qf, const uint8_t *code, float triple_x,
                         float factor_dq, float factor_vq, float parent_dist, int padded_dim);
float fgo_estimate_seq(const fgo_query_factors *qf, const uint8_t *code, float triple_x,
                       float factor_dq, float factor_vq, float parent_dist, int padded_dim);

/* ---- distances ---- */
float fgo_warp_l2(int dim, const float *a, const float *b);
float fgo_warp_ip(int dim, const float *a, const float *b);
float fgo_scalar_l2(int dim, const float *a, const float *b);
float fgo_scalar_ip(int dim, const float *a, const float *b);

/* ---- networks, merges, hash ---- */
void fgo_bitonic_sort(float *keys, uint32_t *vals, uint32_t n);
void fgo_bitonic_stage(float *keys, uint32_t *vals, uint32_t n, uint32_t kk);
void fgo_merge_candidates(float *beam_d, uint32_t *beam_i, float *cand_d, uint32_t *cand_i,
                          uint32_t cbs, uint32_t pbeam, int first, float *scratch_d,
                          uint32_t *scratch_i);
int fgo_merge_path_partition(const float *a, int na, const float *b, int nb, int diag);
uint32_t fgo_hash_insert(uint32_t *table, unsigned bitlen, uint32_t key);
uint32_t fgo_hash_contains(const uint32_t *table, unsigned bitlen, uint32_t key);
uint32_t fgo_pick_expanders(int n, uint32_t *out, int m, uint32_t *beam_idx);
int fgo_warp_keep_topk(const float *values, const int *valid, int keep_k, int *keep_out);

/* ---- controller ---- */
void fgo_ctl_init(fgo_ctl_state *st, float entry_distance);
void fgo_controller_step(fgo_ctl_state *st, uint32_t beam0, float phase2_rho);
void fgo_record_expander(fgo_ctl_state *st, const float *parent_dist, uint32_t n_parents);
float fgo_kth_cutoff(int K, int beam, const uint32_t *beam_idx, const float *beam_dist);

/* ---- search ---- */
int fgo_search_one(const fgo_index *ix, const float *query, int K, int beam, uint32_t *out,
                   fgo_counters *cnt, fgo_trace_rec *trace, uint32_t trace_cap,
                   uint32_t *trace_len);
int fgo_search_batch(const fgo_index *ix, const float *queries, uint64_t nq, int K, int beam,
                     uint32_t *out, fgo_counters *cnt, int nthreads);

/* ---- host helpers on the path ---- */
uint32_t fgo_entry_point(const float *data, uint64_t npoints, uint32_t dim, uint64_t row_offset,
                         int use_ip);
float fgo_recall(const uint32_t *pred, const int32_t *gt, uint64_t nq, int topk, int gt_k);

#ifdef __cplusplus
}
#endif
#endif
