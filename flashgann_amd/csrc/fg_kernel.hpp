// fg_kernel.hpp -- the search kernel of fg_search.hip and its launch
// templates, shared by the translation units that instantiate it: each
// shape class (fg_shapes.hip, compiled once per class) instantiates its
// kernels and launch function in its own object, so the classes compile in
// parallel; fg_search.hip holds the host side and calls them.
#pragma once
// sees the visited set as of the round's start; the lowest (task, lane) wins".
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/flashgann.h"

namespace fgk {

constexpr uint32_t kMaxIndex = 0xFFFFFFFFu;
constexpr uint32_t kMsb = 0x80000000u;
constexpr int kSearchWidth = 8;       // THETA_MAX = WARPS_PER_BLOCK (adaptive_search_config.cuh:32)
constexpr int kBufferBound = 32;      // BUFFER_BOUND (adaptive_search_config.cuh:54)
constexpr int kMaxIterations = 1024;  // MAX_ITERATIONS (adaptive_search_config.cuh:12)
constexpr int kHashReset = 16;        // SMALL_HASH_RESET_INTERVAL (utils.cuh:683)
constexpr int kRefBlock = 256;        // reference block size: fixes merge-path segmentation
constexpr int kMaxBeam = 1024;
constexpr int kMaxDegree = 1024;
constexpr int kMaxPaddedDim = 2048;
constexpr float kPhase1Rho = 0.25f;   // PHASE1_RHO
constexpr float kRhoMax = 0.99f;      // RHO_MAX
constexpr int kStallIters = 4;        // TOP1_WARMUP_STALL_ITERS
constexpr int kPlanes = 6;            // q in [1, 64]: q - 1 needs 6 bit-planes
constexpr int kWrapPlane = 6;         // chunks whose four levels are all 64
constexpr int kZeroPlane = 7;         // levels that are 0 (a degenerate query only)

// ------------------------------------------------------------ host+device

__host__ __device__ inline uint32_t round_up_pow2(uint32_t x) {
    if (x <= 1) return 1;
    --x;
    x |= x >> 1; x |= x >> 2; x |= x >> 4; x |= x >> 8; x |= x >> 16;
    return x + 1;
}

// utils.cuh:119-127
__host__ __device__ inline uint32_t effective_sort_beam(uint32_t beam) {
    uint32_t r = round_up_pow2(beam);
    if (r <= 128) return r < 32 ? 32 : r;
    return beam;
}

__host__ __device__ inline int clamp_i(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
__host__ __device__ inline float clamp_f(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

// utils.cuh:104-117
__host__ __device__ inline int keep_count_per_parent(uint32_t max_degree, float rho) {
    float kf = 1.0f - rho;
    if (kf < 0.0f) kf = 0.0f;
    if (kf > 1.0f) kf = 1.0f;
    uint32_t k = static_cast<uint32_t>(ceilf(static_cast<float>(max_degree) * kf));
    if (k < 1) k = 1;
    if (k > max_degree) k = max_degree;
    return static_cast<int>(k);
}

// keep_count_for_expander below, split: keep_limit is the part that does not
// depend on the K-th cutoff, min(rho_keep, budget), always in [1, active];
// with a valid cutoff the count is then min(max(near, 1), limit), otherwise
// the limit itself.
__host__ __device__ inline int keep_limit(uint32_t active, int theta, float rho) {
    const int rho_keep = keep_count_per_parent(active, rho);
    const int budget = clamp_i(static_cast<int>(static_cast<uint32_t>(kBufferBound) / static_cast<uint32_t>(theta)), 1,
                               static_cast<int>(active));
    return rho_keep < budget ? rho_keep : budget;
}

__host__ __device__ inline int keep_with_cutoff(int limit, bool kth_valid, uint32_t near) {
    if (!kth_valid) return limit;
    const int n = near < 1u ? 1 : static_cast<int>(near);
    return n < limit ? n : limit;
}

// adaptive_search_utils.cuh:121-135
__host__ __device__ inline int keep_count_for_expander(uint32_t active, int theta, float rho,
                                                       bool kth_valid, uint32_t near) {
    const int active_count = static_cast<int>(active);
    const int rho_keep = keep_count_per_parent(active, rho);
    const int budget = clamp_i(static_cast<int>(static_cast<uint32_t>(kBufferBound) / static_cast<uint32_t>(theta)), 1,
                               active_count);
    int max_keep = rho_keep < budget ? rho_keep : budget;
    if (kth_valid) max_keep = clamp_i(static_cast<int>(near), 1, max_keep);
    return clamp_i(max_keep, 1, active_count);
}

// Visited-table size bounds, in 4-slot buckets.  Between two resets the
// table receives at most beam + 16 * 32 * tiles + 1 distinct keys (restore +
// one reset interval of inserts, <= 32 per 8-task round, + the entry point).
// A table with more slots than that never fills, so it answers every
// membership query exactly like the reference's 2^11-entry table
// (utils.cuh:137-151), which never fills either.  The smallest table keeps
// that worst case at <= 99% load with at least one slot to spare (an insert
// always finds a free slot, a lookup's walk always meets one); the roomiest
// at <= 90% (fewer lookups that walk on).  visited_buckets() picks between
// them.
__host__ __device__ inline uint32_t visited_keys_max(uint32_t beam, uint32_t degree) {
    return beam + 16u * 32u * ((degree + 31) / 32) + 1u;
}
__host__ __device__ inline uint32_t visited_buckets_min(uint32_t beam, uint32_t degree) {
    const uint32_t slots = (visited_keys_max(beam, degree) * 100u + 98u) / 99u + 1u;
    return (slots + 3u) / 4u;
}
__host__ __device__ inline uint32_t visited_buckets_roomy(uint32_t beam, uint32_t degree) {
    const uint32_t slots = (visited_keys_max(beam, degree) * 10u + 8u) / 9u;
    return (slots + 3u) / 4u;
}

struct LdsLayout {
    uint32_t hash_off, beam_off, msort_off, plane_off, scratch_off, prof_off, total, total_prof, team_off,
        total_team;
};

// Candidate buffer and sorted-candidate staging of the beam merge, one array
// of (distance, id) pairs at indices -1 .. kMsortHi: the 32 candidates at
// 0..31 between a -FLT_MAX sentinel (index -1) and FLT_MAX sentinels (32 and
// up).  The stages fill slots 0..31 in any order; the merge reads them into
// registers, sorts them and writes them back sorted before it merges.
constexpr int kMsortHi = 35;
constexpr uint32_t kMsortPairs = 38;
// Beam: (distance, id) pairs at indices -1 .. pbeam + kBeamPad - 1: a
// -FLT_MAX sentinel, the pbeam entries, a FLT_MAX sentinel at pbeam, then pad
// entries (segment reads may run up to 3 past pbeam; the merge's unused
// slots are written to pbeam + 2).
constexpr uint32_t kBeamPad = 4;

// A team launch runs each query on two waves: the lead wave runs the search,
// the helper takes half of every stage-II round (visited tests, estimates
// and keep decisions of its tasks) and half of every exact-distance batch.
// They meet at workgroup barriers and exchange through this LDS block.
struct TeamBlock {
    // per iteration, from the lead wave: stop flag, theta, rho, K-th cutoff,
    // number of expanders; then the exact batch's size and list kind
    uint32_t stop, theta, nexp, kth_bits, rho_bits, ex_n, ex_alist, pad0;
    // per query (written once): the quantised query's constants
    uint32_t sum_q, qwidth_bits, qlow_bits, any_wrap, any_zero;
    // the helper's work counters (counting build)
    uint32_t c_ids, c_est, pad1;
    // the helper's stage-II results: kept-lane masks and child ids of its
    // sub-rounds
    uint64_t klm[2];
    uint32_t cid[2][64];
};
constexpr uint32_t kTeamBytes = 640;
static_assert(sizeof(TeamBlock) <= kTeamBytes, "team block");

// The lead wave's way out of the search loop in the team form: it tells the
// helper to stop at their meeting point (the helper then leaves too).
template <int NW>
__device__ __forceinline__ void team_stop(TeamBlock *tb, int lane) {
    if constexpr (NW > 1) {
        if (lane == 0) tb->stop = 1u;
        __syncthreads();
    }
}


// Per-query LDS: visited table and beam (aliased by the rotated query during
// preparation), the candidate pairs, 8 x B/32 plane words and a small
// scratch area (32-entry child list + parent ids and distances).  The raw
// query is read from global memory, where it stays cached (the fixed
// geometries keep it in registers through the loop).
__host__ __device__ constexpr LdsLayout lds_layout(uint32_t dim, uint32_t padded_dim, uint32_t pbeam,
                                                   uint32_t buckets) {
    // fixed-size regions first (compile-time offsets for a fixed geometry),
    // then the beam-dependent visited table and beam
    LdsLayout L{};
    uint32_t off = 0;
    L.msort_off = off;
    off += kMsortPairs * 8u;
    (void)dim;
    L.plane_off = off;
    off += 8u * (padded_dim / 32u) * 4u;
    L.scratch_off = off;
    off += (32u + 2u * 8u) * 4u;
    off = (off + 15u) & ~15u;
    L.hash_off = off;
    // during query preparation the rotated query (padded_dim floats) spans the
    // visited table and the beam, which are initialised after it
    uint32_t hash_bytes = buckets * 16u;
    const uint32_t beam_bytes = (pbeam + 1u + kBeamPad) * 8u;
    if (hash_bytes + beam_bytes < padded_dim * 4u) hash_bytes = (padded_dim * 4u - beam_bytes + 15u) & ~15u;
    off += hash_bytes;
    L.beam_off = off;
    off += (pbeam + 1u + kBeamPad) * 8u;
    L.total = (off + 15u) & ~15u;
    // phase timers of the profiling build only, past the end of the rest
    L.prof_off = L.total;
    L.total_prof = L.total + 16u * 8u;
    // a team launch's exchange block, past the phase timers
    L.team_off = L.total_prof;
    L.total_team = L.total_prof + kTeamBytes;
    return L;
}

// LDS is allocated to a workgroup in units of 1,280 bytes on gfx950
// (measured: 7,632-byte workgroups fit 21 to a CU, 7,760-byte ones 18).
constexpr uint32_t kLdsGranule = 1280;

// The visited table a search uses: the roomiest table (at most 90% worst-case
// load) that fits in as many LDS granules as the smallest one needs, so the
// table never costs a workgroup per CU (beam 384: 21 instead of 18 per CU,
// beam 512: 18 instead of 16, beam 1024: 10 instead of 9) and keeps its
// slack where that is free (beam 256).
__host__ __device__ inline uint32_t visited_buckets(uint32_t dim, uint32_t padded_dim, uint32_t pbeam, uint32_t beam,
                                                    uint32_t degree) {
    const uint32_t lo = visited_buckets_min(beam, degree);
    const uint32_t total = lds_layout(dim, padded_dim, pbeam, lo).total;
    const uint32_t cap = (total + kLdsGranule - 1u) / kLdsGranule * kLdsGranule;
    uint32_t b = visited_buckets_roomy(beam, degree);
    while (b > lo && lds_layout(dim, padded_dim, pbeam, b).total > cap) --b;
    return b;
}

struct SearchParams {
    const float *data;
    const float *signs;
    const float *queries;
    uint32_t *results;
    uint32_t *counters;
    unsigned long long *phase;  // per-query phase cycles + start/end time (profiling build only)
    uint64_t npoints;
    uint64_t row_offset, code_offset, factor_offset, neighbor_offset;
    int dim, padded_dim, degree;
    int K, beam, pbeam, cbs, collect_cap;
    int buckets, max_iter;  // visited-table buckets (4 slots each), iteration limit
    int seg_active;      // merge-path segments (pbeam > 128)
    uint32_t seg_magic;  // floor(2^32 / seg_active) + 1: t * pbeam / seg_active by one mulhi
    float phase2_rho;
    int use_ip;
    int dup_free;
    int vec_ok;
    int runtime_geo;  // host only: run the runtime-geometry kernels
    int team;         // host only: the team form (two waves per query) may run
    uint32_t entry;
    int nq;
    // Sliced search (one-wave form): a slice that suspends
    // runs its queries to the top of iteration slice_suspend and keeps an
    // unfinished query's state in slice_state; a slice that resumes runs the
    // queries slice_order lists (longest expected first), the first
    // slice_state[0] of them, from iteration slice_resume.
    int slice_suspend = 0;  // > 0: an unfinished query stops at the top of this iteration and keeps its state
    int slice_resume = 0;   // > 0: resume the ordered queries at this iteration
    uint32_t *slice_state = nullptr;        // kSliceHeader words, then slice_words(pbeam) per query
    uint32_t *slice_keys = nullptr;         // per query: ordering key, or kSliceDone
    const uint32_t *slice_order = nullptr;  // second slice: query of each workgroup
    LdsLayout lds;
};

// Per-query state of a suspended search, in 32-bit words after a header of
// kSliceHeader words (word 0: the number of suspended queries, set by the
// order step).  Per query: a mark (1), the ordering key, the controller (9
// words), the work counters (6), the candidate span, the split flag and the
// pick's start (beams over 256), then the pbeam beam pairs and the 32
// candidate pairs, then the prepared query: low, width, sum_q, a pad word and
// the 8 planes of W = padded_dim / 32 words (so the second slice does not
// rotate and quantise the query again, nor read the entry point's row).
// slice_keys holds the key (bits of a finite float: the best distance so far)
// of each suspended query and kSliceDone (a NaN pattern, never a key) for a
// query the first slice finished.
constexpr uint32_t kSliceHeader = 64;
constexpr uint32_t kSliceFixed = 20;  // 2 + 9 + 6 + 2 + 1 (the pick's start, beams over 256)
__host__ __device__ inline uint32_t slice_prep_offset(uint32_t pbeam) { return kSliceFixed + 2u * (pbeam + 32u); }
__host__ __device__ inline uint32_t slice_words(uint32_t pbeam, uint32_t padded_dim) {
    return slice_prep_offset(pbeam) + 4u + 8u * (padded_dim / 32u);
}
constexpr uint32_t kSliceDone = 0xFFFFFFFFu;
constexpr int kSliceMaxQueries = 16384;  // the one-workgroup order kernel holds every query's bin in LDS
constexpr int kSliceBins = 4096;

// The ordering key of a suspended query: the best distance so far, made
// finite (+inf -> FLT_MAX, -inf and NaN -> -FLT_MAX) so that it orders as a
// float for either metric (inner-product distances are negative).
__device__ __forceinline__ uint32_t slice_key(float d) {
    const float k = isnan(d) ? -FLT_MAX : fminf(fmaxf(d, -FLT_MAX), FLT_MAX);
    return __float_as_uint(k);
}
// Order-preserving unsigned image of a finite float key (larger key, larger image).
__host__ __device__ inline uint32_t key_order_bits(uint32_t bits) {
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}
__host__ __device__ inline uint32_t key_from_order_bits(uint32_t o) {
    return (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
}


// Row geometry (include/qg.hpp:66-73), compile-time for the specialised
// shapes (DIM_T, DEG_T > 0) so every field offset is an immediate, runtime
// otherwise.
__host__ __device__ constexpr int pow2_at_least(int d) { return d <= 1 ? 1 : 2 * pow2_at_least((d + 1) / 2); }

template <int DIM_T, int DEG_T>
struct Geo {
    static constexpr bool kFixed = DIM_T > 0 && DEG_T > 0;
    static constexpr int kB = kFixed ? pow2_at_least(DIM_T) : 0;
    static constexpr int kFactor = DIM_T + kB / 64 * 2 * DEG_T;
    static constexpr int kNbr = kFactor + 3 * DEG_T;
    static constexpr int kRow = kNbr + DEG_T;
    // byte offsets of the fixed geometry: the host runs it only when every
    // row starts below 4 GiB, so a row's byte offset is node * kRowB in 32
    // bits (node < 2^24) and loads take a uniform base plus a 32-bit offset
    static constexpr uint32_t kRowB = 4u * kRow, kCodeB = 4u * DIM_T, kFactorB = 4u * kFactor, kNbrB = 4u * kNbr;
    int dim, deg, B;
    uint64_t row, code, factor, nbr;
    __device__ __forceinline__ explicit Geo(const SearchParams &P)
        : dim(kFixed ? DIM_T : P.dim),
          deg(kFixed ? DEG_T : P.degree),
          B(kFixed ? kB : P.padded_dim),
          row(kFixed ? static_cast<uint64_t>(kRow) : P.row_offset),
          code(kFixed ? static_cast<uint64_t>(DIM_T) : P.code_offset),
          factor(kFixed ? static_cast<uint64_t>(kFactor) : P.factor_offset),
          nbr(kFixed ? static_cast<uint64_t>(kNbr) : P.neighbor_offset) {}
};

// ------------------------------------------------------------ device helpers

// A T at byte offset `off` of `base` (a kernel argument, so uniform): the
// address is a scalar base plus a 32-bit vector offset, with no 64-bit
// per-lane address arithmetic.
template <class T>
__device__ __forceinline__ T ld_at(const float *base, uint32_t off) {
    return *reinterpret_cast<const T *>(reinterpret_cast<const char *>(base) + off);
}

// The lane id, through an empty asm: values derived from it (lane masks,
// addresses) are computed where they are used instead of being hoisted out of
// the search loop, where they would hold registers -- lane masks hold scalar
// register pairs -- through every phase of every iteration.
__device__ __forceinline__ int lane_id() {
    int l = static_cast<int>(threadIdx.x) & 63;
    asm volatile("" : "+v"(l));
    return l;
}

__device__ __forceinline__ int lane_id_opaque() { return lane_id(); }

// Lane masks straight from a bool (HIP's __ballot / __any take an int, which
// costs a mask -> 0/1 -> mask round trip per use).
__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
__device__ __forceinline__ bool any_lane(bool p) { return ballot(p) != 0ull; }

__device__ __forceinline__ uint32_t half_bits(uint64_t m, int h) {
    return static_cast<uint32_t>(m >> (32 * h));
}

// Lanes whose index has bit v set (v a power of two <= 32).
__host__ __device__ constexpr uint64_t lane_bit_mask(int v) {
    return v == 1    ? 0xAAAAAAAAAAAAAAAAull
           : v == 2  ? 0xCCCCCCCCCCCCCCCCull
           : v == 4  ? 0xF0F0F0F0F0F0F0F0ull
           : v == 8  ? 0xFF00FF00FF00FF00ull
           : v == 16 ? 0xFFFF0000FFFF0000ull
           : v == 32 ? 0xFFFFFFFF00000000ull
                     : 0ull;
}

// A uniform lane mask as this lane's bool (no instructions: the mask is the
// condition register).
__device__ __forceinline__ bool lane_in(uint64_t mask) { return __builtin_amdgcn_inverse_ballot_w64(mask); }

// Set bits in this lane's 32-lane half of a ballot: two scalar counts and
// one select, instead of a per-lane 64-bit shift and count.
__device__ __forceinline__ uint32_t half_popc(uint64_t m) {
    const uint32_t lo = static_cast<uint32_t>(__popc(static_cast<uint32_t>(m)));
    const uint32_t hi = static_cast<uint32_t>(__popc(static_cast<uint32_t>(m >> 32)));
    return lane_in(0xFFFFFFFF00000000ull) ? hi : lo;
}

// Set bits in this lane's G-lane group of a ballot (G = 32: its half; G = 16:
// its row), from scalar counts and selects.
template <int G>
__device__ __forceinline__ uint32_t group_popc(uint64_t m) {
    if constexpr (G == 32) {
        return half_popc(m);
    } else {
        const uint32_t r0 = static_cast<uint32_t>(__popc(static_cast<uint32_t>(m) & 0xFFFFu));
        const uint32_t r1 = static_cast<uint32_t>(__popc(static_cast<uint32_t>(m) >> 16));
        const uint32_t r2 = static_cast<uint32_t>(__popc(static_cast<uint32_t>(m >> 32) & 0xFFFFu));
        const uint32_t r3 = static_cast<uint32_t>(__popc(static_cast<uint32_t>(m >> 48)));
        const bool odd = lane_in(0xFFFF0000FFFF0000ull), high = lane_in(0xFFFFFFFF00000000ull);
        return high ? (odd ? r3 : r2) : (odd ? r1 : r0);
    }
}

// Lane i reads lane i ^ m, all lanes active.  m < 16 stays inside a 16-lane
// row: DPP quad_perm (1, 2), half-row mirror then quad reverse
// ((i^7)^3 = i^4), row rotate by 8 (i + 8 mod 16 = i^8).  16 and
// 32 use gfx950's permlane16/32 swaps (row pairs / wave halves exchanged
// between two copies of the value) and keep the half this lane needs.  Every
// DPP source lane lies inside the row, so bound_ctrl changes no value; set,
// it lets the compiler fold the move into the ALU op that consumes it.
__device__ __forceinline__ int xshfl(int v, int m) {
    switch (m) {
    case 1:
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
    case 2:
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
    case 4:
        return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true);
    case 8:
        return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true);  // row rotate by 8 = xor 8 in a 16-lane row
    case 16: {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return lane_in(lane_bit_mask(16)) ? static_cast<int>(r[0]) : static_cast<int>(r[1]);
    }
    case 32: {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return lane_in(lane_bit_mask(32)) ? static_cast<int>(r[0]) : static_cast<int>(r[1]);
    }
    default:
        return __shfl_xor(v, m);
    }
}
__device__ __forceinline__ float xshfl(float v, int m) { return __int_as_float(xshfl(__float_as_int(v), m)); }
__device__ __forceinline__ uint32_t xshfl(uint32_t v, int m) {
    return static_cast<uint32_t>(xshfl(static_cast<int>(v), m));
}

// The two values a lane pairs with across 16-lane rows or 32-lane halves.
// One permlane swap of (a, b) leaves in the first result a's even row and
// b's even row interleaved as (a.R0, b.R0, a.R2, b.R2), in the second
// (a.R1, b.R1, a.R3, b.R3) (rows of 16 lanes); the 32-lane form does the same
// with halves.  Adding the two results is a reduce-scatter step: rows with
// bit 16 clear get a's pair sum, the others b's.  With a == b it is the
// xor-16 (xor-32) combine of a symmetric op, with no select: every lane sees
// (even, odd) in the same order, which for a commutative op equals
// (own, partner).
struct Pair {
    float lo, hi;
};
__device__ __forceinline__ Pair swap16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ Pair swap32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ uint32_t min16(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return min(static_cast<uint32_t>(r[0]), static_cast<uint32_t>(r[1]));
}
__device__ __forceinline__ int add32i(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
    return static_cast<int>(r[0]) + static_cast<int>(r[1]);
}
__device__ __forceinline__ int add16i(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
    return static_cast<int>(r[0]) + static_cast<int>(r[1]);
}

// Reductions over all 64 lanes (xor distances 32 .. 1, written out).
__device__ __forceinline__ float wave_min(float v) {
    Pair p = swap32(v, v);
    v = fminf(p.lo, p.hi);
    p = swap16(v, v);
    v = fminf(p.lo, p.hi);
    v = fminf(v, xshfl(v, 8));
    v = fminf(v, xshfl(v, 4));
    v = fminf(v, xshfl(v, 2));
    return fminf(v, xshfl(v, 1));
}
__device__ __forceinline__ float wave_max(float v) {
    Pair p = swap32(v, v);
    v = fmaxf(p.lo, p.hi);
    p = swap16(v, v);
    v = fmaxf(p.lo, p.hi);
    v = fmaxf(v, xshfl(v, 8));
    v = fmaxf(v, xshfl(v, 4));
    v = fmaxf(v, xshfl(v, 2));
    return fmaxf(v, xshfl(v, 1));
}
__device__ __forceinline__ int wave_sum(int v) {
    v = add32i(v);
    v = add16i(v);
    v += xshfl(v, 8);
    v += xshfl(v, 4);
    v += xshfl(v, 2);
    return v + xshfl(v, 1);
}

// uniform value -> scalar register
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// A flag that stays the same through the search loop, kept as a 32-bit
// scalar and tested where it is used (one scalar compare).  Held as a bool it
// becomes a 64-bit lane mask live across the whole loop, and the loop is
// short of scalar registers (such masks are spilled to vector-register lanes
// and reloaded with v_readlane, a vector instruction).
__device__ __forceinline__ bool sflag(uint32_t v) {
    uint32_t u = __builtin_amdgcn_readfirstlane(v);
    asm volatile("" : "+s"(u));
    return u != 0u;
}
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uni(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

__device__ __forceinline__ bool finite_below_max(float x) { return isfinite(x) && x < FLT_MAX; }

// An exact distance as a beam key: NaN and values beyond +-FLT_MAX (from an
// overflowing or NaN vector) become +-FLT_MAX (NaN: FLT_MAX).  The merge-path
// partition stands -FLT_MAX / FLT_MAX in for positions before / past the
// arrays (utils.cuh:600-603); a key outside that range, or unordered, sends
// the partition past the arrays, so keys are kept within it.
__device__ __forceinline__ float beam_key(float d) {
    return d != d ? FLT_MAX : (d > FLT_MAX ? FLT_MAX : (d < -FLT_MAX ? -FLT_MAX : d));
}

// ------------------------------------------------------------ query preparation

// Orders the LDS accesses of code that the search's lead wave runs alone.
// NW = 1 (one wave per workgroup): the workgroup barrier, which the compiler
// reduces to a wave barrier.  NW > 1 (a team of waves per query, the others
// waiting at a workgroup barrier meanwhile): a wavefront-scope fence, since
// one wave's LDS operations complete in issue order.
template <int NW>
__device__ __forceinline__ void lead_sync() {
    if constexpr (NW == 1) {
        __syncthreads();
    } else {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// utils.cuh:790-939 for one wave: rotate (x*signs, pad, FWHT len = 1..B/2 with
// butterflies (u+v, u-v)), min/max, width = (hi-lo)*fl(1/63), q = round(fma(
// y-lo, 1/width, 0.5)) (NaN -> 0), then the 6 popcount planes of q - 1, the
// level-0 mask and the chunks whose uint8 LUT entry would wrap.  Writes
// planes (8 x W words) and returns low, width, sum_q.  `rot` is LDS scratch
// of B floats.
template <int NW = 1>
__device__ __forceinline__ void prepare_query(const float *__restrict__ query, const float *__restrict__ signs, int dim,
                              int B, float *rot, float *qv, uint32_t *planes, float &low_out,
                              float &high_out, float &width_out, int &sumq_out, uint8_t *qdump) {
    const int lane = lane_id();
    for (int i = lane; i < B; i += 64) {
        float x = 0.0f;
        if (i < dim) {
            const float v = query[i];
            if (qv) qv[i] = v;
            x = v * signs[i];
        }
        rot[i] = x;
    }
    lead_sync<NW>();
    for (int len = 1; len < B; len <<= 1) {
        for (int p = lane; p < (B >> 1); p += 64) {
            const int blk = p / len, j = p - blk * len;
            const int i1 = blk * (len << 1) + j, i2 = i1 + len;
            const float u = rot[i1], v = rot[i2];
            rot[i1] = u + v;
            rot[i2] = u - v;
        }
        lead_sync<NW>();
    }
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (int i = lane; i < B; i += 64) {
        lo = fminf(lo, rot[i]);
        hi = fmaxf(hi, rot[i]);
    }
    lo = uni(wave_min(lo));
    hi = uni(wave_max(hi));
    const float levels_inv = 1.0f / 63.0f;
    const float width = (hi - lo) * levels_inv;
    const float inv_width = 1.0f / width;
    const int W = B >> 5;
    const int h = lane >> 5, nl = lane & 31;
    int sum = 0;
    for (int w0 = 0; w0 < W; w0 += 2) {
        const int w = w0 + h;  // W is even (B >= 64)
        const int g = 32 * w + nl;
        const int i = 4 * (g >> 2) + 3 - (g & 3);
        const float scaled = fmaf(rot[i] - lo, inv_width, 0.5f);
        const uint32_t q = isnan(scaled) ? 0u : static_cast<uint32_t>(roundf(scaled));
        if (qdump) qdump[i] = static_cast<uint8_t>(q);
        sum += static_cast<int>(q);
        // planes of q - 1: a code's sum over its set bits is then
        // popcount(code) + sum_p 2^p popcount(code & plane_p), minus the set
        // bits at level 0 (plane kZeroPlane; only a query whose rotation is
        // constant or not finite has such levels, and then all of them)
        const uint32_t r = q != 0u ? q - 1u : 0u;
        for (int p = 0; p < kPlanes; ++p) {
            const uint64_t m = ballot(((r >> p) & 1u) != 0u);
            if (nl == 0) planes[p * W + w] = half_bits(m, h);
        }
        const uint64_t zm = ballot(q == 0u);
        if (nl == 0) planes[kZeroPlane * W + w] = half_bits(zm, h);
        // a chunk's full-nibble LUT entry is (q0+q1+q2+q3) mod 256 (utils.cuh:913-917)
        uint32_t s = q + xshfl(q, 1);
        s += xshfl(s, 2);
        const uint64_t wm = ballot(s >= 256u);
        if (nl == 0) planes[kWrapPlane * W + w] = half_bits(wm, h);
    }
    sumq_out = uni(wave_sum(sum));
    low_out = lo;
    high_out = hi;
    width_out = width;
    lead_sync<NW>();
}

// popcount(x) + acc as one v_bcnt_u32_b32.  Written as an instruction so a
// chain of them stays a chain: as plain additions the compiler splits it into
// popcounts from zero joined by three-input adds, two more instructions per
// plane and code block.
__device__ __forceinline__ uint32_t bcnt_acc(uint32_t x, uint32_t acc) {
    uint32_t r;
    asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(acc));
    return r;
}

// raw = sum_cb LUT[cb][nibble] (utils.cuh:976-980) over code words [w0, w1):
// popcount(code) + sum_p 2^p popcount(code & plane_p) (the planes hold
// q - 1), less the set bits at level 0 and 256 per wrapped chunk.
__device__ __forceinline__ int32_t raw_partial(const uint32_t *__restrict__ code, int w0, int w1,
                                               const uint32_t *planes, int W) {
    uint32_t acc[kPlanes];
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) acc[p] = 0;
    uint32_t ones = 0, zeros = 0, wraps = 0;
    for (int w = w0; w < w1; ++w) {
        const uint32_t c = code[w];
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) acc[p] += __popc(c & planes[p * W + w]);
        ones += __popc(c);
        zeros += __popc(c & planes[kZeroPlane * W + w]);
        const uint32_t x = c & planes[kWrapPlane * W + w];
        wraps += __popc(x & (x >> 1) & (x >> 2) & (x >> 3) & 0x11111111u);
    }
    uint32_t raw = ones - zeros;
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) raw += acc[p] << p;
    return static_cast<int32_t>(raw - 256u * wraps);
}

// popcount(c) + sum_p 2^p popcount(c & plane_p) - popcount(c & zero plane)
// over NB code words starting at word w0 (added to raw), and the count of
// wrapped chunks among them (added to wraps).  NB is a compile-time width,
// so the plane reads carry no per-step condition and can be issued ahead of
// the popcounts that consume them.
template <int NB>
__device__ __forceinline__ void raw_span(const uint32_t *__restrict__ code, const uint32_t *planes, int W, int w0,
                                         bool vec_ok, bool any_wrap, bool any_zero, uint32_t &raw, uint32_t &wraps) {
    uint32_t c[NB];
    if (vec_ok) {
#pragma unroll
        for (int j = 0; j < NB / 4; ++j) {
            const uint4 v = reinterpret_cast<const uint4 *>(code + w0)[j];
            c[4 * j] = v.x; c[4 * j + 1] = v.y; c[4 * j + 2] = v.z; c[4 * j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < NB; ++j) c[j] = code[w0 + j];
    }
    // one accumulator per plane (six independent chains), four words at a
    // time: the six plane reads of a group are in flight together, and the
    // next group's reads are issued before this group's popcounts; the
    // code's own popcount (the level offset 1) joins plane 0's chain
    uint32_t acc[kPlanes];
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) acc[p] = 0;
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[0] = bcnt_acc(c[j], acc[0]);
    uint4 cur[kPlanes], nxt[kPlanes];
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) cur[p] = reinterpret_cast<const uint4 *>(planes + p * W + w0)[0];
#pragma unroll
    for (int j = 0; j < NB / 4; ++j) {
        if (j + 1 < NB / 4) {
#pragma unroll
            for (int p = 0; p < kPlanes; ++p) nxt[p] = reinterpret_cast<const uint4 *>(planes + p * W + w0)[j + 1];
        }
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) {
            acc[p] = bcnt_acc(c[4 * j] & cur[p].x, acc[p]);
            acc[p] = bcnt_acc(c[4 * j + 1] & cur[p].y, acc[p]);
            acc[p] = bcnt_acc(c[4 * j + 2] & cur[p].z, acc[p]);
            acc[p] = bcnt_acc(c[4 * j + 3] & cur[p].w, acc[p]);
        }
        if (j + 1 < NB / 4) {
#pragma unroll
            for (int p = 0; p < kPlanes; ++p) cur[p] = nxt[p];
        }
    }
    // sum_p 2^p acc[p], top plane first
    uint32_t hb = acc[kPlanes - 1];
#pragma unroll
    for (int p = kPlanes - 2; p >= 0; --p) hb = (hb << 1) + acc[p];
    raw += hb;
    if (any_zero) {
        const uint32_t *zp = planes + kZeroPlane * W + w0;
#pragma unroll
        for (int j = 0; j < NB; ++j) raw -= static_cast<uint32_t>(__popc(c[j] & zp[j]));
    }
    if (any_wrap) {
        const uint32_t *wp = planes + kWrapPlane * W + w0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t x = c[j] & wp[j];
            wraps += __popc(x & (x >> 1) & (x >> 2) & (x >> 3) & 0x11111111u);
        }
    }
}

// raw for one neighbour code of W words (W a power of two >= 8: padded
// dimension >= 256), the same sum as raw_partial over [0, W): the code words
// are loaded 32 at a time (eight 16-byte loads when the row layout keeps
// codes 16-byte aligned), and each plane's matching words come from LDS as
// 16-byte reads.
__device__ __forceinline__ int32_t raw_words(const uint32_t *__restrict__ code, const uint32_t *planes, int W,
                                             bool vec_ok, bool any_wrap, bool any_zero) {
    uint32_t raw = 0, wraps = 0;
    if (W >= 32) {
        for (int w0 = 0; w0 < W; w0 += 32) raw_span<32>(code, planes, W, w0, vec_ok, any_wrap, any_zero, raw, wraps);
    } else if (W == 16) {
        raw_span<16>(code, planes, W, 0, vec_ok, any_wrap, any_zero, raw, wraps);
    } else {
        raw_span<8>(code, planes, W, 0, vec_ok, any_wrap, any_zero, raw, wraps);
    }
    return static_cast<int32_t>(raw - 256u * wraps);
}

// utils.cuh:989-993 with nvcc's contraction of the two multiply-adds.
__device__ __forceinline__ float estimate_formula(int32_t raw, int32_t sum_q, float width, float low,
                                                  float tx, float fdq, float fvq, float pdist) {
    const float rf = static_cast<float>((raw << 1) - sum_q);
    float est = tx + pdist;
    est = fmaf(fdq * width, rf, est);
    est = fmaf(fvq, low, est);
    return est;
}

// utils.cuh:269-305 for one 32-lane half: lane nl accumulates dims nl, nl+32,
// ... with a contracted multiply-add, then the xor butterfly 16..1 (lane 0 of
// the half holds exactly the shfl_down tree's sum; every lane gets the same).
__device__ __forceinline__ float half_distance(const float *__restrict__ row, const float *qv, int dim,
                                               int nl, bool use_ip, bool active) {
    float val = 0.0f;
    if (active) {
        if (use_ip) {
            for (int i = nl; i < dim; i += 32) val = fmaf(qv[i], row[i], val);
        } else {
            for (int i = nl; i < dim; i += 32) {
                const float d = qv[i] - row[i];
                val = fmaf(d, d, val);
            }
        }
    }
    const Pair p16 = swap16(val, val);
    val = p16.lo + p16.hi;
    val += xshfl(val, 8);
    val += xshfl(val, 4);
    val += xshfl(val, 2);
    val += xshfl(val, 1);
    return use_ip ? -val : val;
}

// The reduction of half_distance on its own: every lane of the half gets
// the shfl_down tree's sum of the half's 32 partial sums.
__device__ __forceinline__ float half_reduce(float val) {
    const Pair p16 = swap16(val, val);
    val = p16.lo + p16.hi;
    val += xshfl(val, 8);
    val += xshfl(val, 4);
    val += xshfl(val, 2);
    val += xshfl(val, 1);
    return val;
}

// Exact distances of the generic geometry, PB children per 32-lane half
// (child e0 + 2 j + h): lane nl accumulates dimensions nl, nl + 32, ... of
// each child in that order (the reference's per-lane order, as
// half_distance), with the loads of KB consecutive steps of every child
// issued together.  Indices past the row's dimension are clamped to its last
// dimension and their terms skipped.
// KB dimension steps of PB rows per half (lane nl: dimensions nl + 32 k in
// turn).  CHECK: some step may lie past dim; such a step reads a valid
// element and leaves the sum as it is.
template <int PB, int KB, bool IP, bool CHECK>
__device__ __forceinline__ void exact_generic_batch(const float *const (&rows)[PB], const float *qv, int dim, int nl,
                                                    int k0, float (&acc)[PB]) {
    float q[KB], v[PB][KB];
    bool ok[KB];
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
        const int i = nl + 32 * (k0 + kk);
        ok[kk] = !CHECK || i < dim;
        const int is = ok[kk] ? i : dim - 1;
        q[kk] = qv[is];
#pragma unroll
        for (int j = 0; j < PB; ++j) v[j][kk] = rows[j][is];
    }
#pragma unroll
    for (int kk = 0; kk < KB; ++kk)
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            float t;
            if constexpr (IP) {
                t = fmaf(q[kk], v[j][kk], acc[j]);
            } else {
                const float d = q[kk] - v[j][kk];
                t = fmaf(d, d, acc[j]);
            }
            acc[j] = ok[kk] ? t : acc[j];
        }
}

template <int PB, int KB>
__device__ __forceinline__ void exact_generic_pass(const SearchParams &P, uint64_t row_floats, int dim, int e0, int n,
                                                   const uint32_t *slot_list, float *cd, const uint32_t *ci,
                                                   const float *qv, bool ip) {
    const int lane = lane_id();
    const int h = lane >> 5, nl = lane & 31;
    const float *rows[PB];
#pragma unroll
    for (int j = 0; j < PB; ++j) {
        const int e = e0 + 2 * j + h;
        const int slot = e < n ? static_cast<int>(slot_list ? slot_list[e] : static_cast<uint32_t>(e)) : 0;
        const uint32_t child = e < n ? ci[2 * slot] : 0u;
        rows[j] = P.data + static_cast<uint64_t>(child) * row_floats;
    }
    float acc[PB];
#pragma unroll
    for (int j = 0; j < PB; ++j) acc[j] = 0.0f;
    // the metric and the test for a step past the last dimension are taken
    // outside the loops (inside, each dimension became both updates and two
    // selects); only a batch that reaches past dim tests its steps
    const int steps = (dim + 31) >> 5;
    for (int k0 = 0; k0 < steps; k0 += KB) {
        const bool full = (k0 + KB) * 32 <= dim;
        if (ip) {
            if (full) exact_generic_batch<PB, KB, true, false>(rows, qv, dim, nl, k0, acc);
            else exact_generic_batch<PB, KB, true, true>(rows, qv, dim, nl, k0, acc);
        } else {
            if (full) exact_generic_batch<PB, KB, false, false>(rows, qv, dim, nl, k0, acc);
            else exact_generic_batch<PB, KB, false, true>(rows, qv, dim, nl, k0, acc);
        }
    }
#pragma unroll
    for (int j = 0; j < PB; ++j) {
        const float r = half_reduce(acc[j]);
        const int e = e0 + 2 * j + h;
        if (e < n && nl == 0) {
            const int slot = static_cast<int>(slot_list ? slot_list[e] : static_cast<uint32_t>(e));
            cd[2 * slot] = beam_key(ip ? -r : r);
        }
    }
}

// ------------------------------------------------------------ sorting networks

// Positions of a register layout: item e of lane l sits at position
// E*l + e, or at l & 31 when HALF (both 32-lane halves hold the same 32
// positions).  pos_bit(v, e) is the lane mask of items e whose position has
// bit v set.
template <int E, bool HALF>
__device__ __forceinline__ uint64_t pos_bit(int v, int e) {
    if (HALF) return v >= 32 ? 0ull : lane_bit_mask(v);
    if (v < E) return (e & v) ? ~0ull : 0ull;
    return lane_bit_mask(v / E);
}

// One compare-exchange step of a bitonic network, block size KK and compare
// distance J, on the layout (E, HALF).  Cross-lane steps use the reference's
// per-lane rule (utils.cuh:309-316, 340-341): a lane takes its partner's pair
// iff the keys differ and (k < pk) != p with p = (pos & KK != 0) ==
// (pos & J != 0).  In-lane steps are utils.cuh:319-328 with ascending =
// (pos_lo & KK) == 0.  KK and J are template arguments so that every step is
// straight-line code with immediate lane masks and shuffle patterns.
template <int E, bool HALF, int KK, int J>
__device__ __forceinline__ void bitonic_step(float (&k)[E], uint32_t (&v)[E]) {
    if constexpr (J >= E) {
        constexpr int M = J / E;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float pk = xshfl(k[e], M);
            const uint32_t pv = xshfl(v[e], M);
            const bool p = lane_in(~(pos_bit<E, HALF>(KK, e) ^ pos_bit<E, HALF>(J, e)));
            if (k[e] != pk && ((k[e] < pk) != p)) {
                k[e] = pk;
                v[e] = pv;
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            if (e & J) continue;
            const int hi = e | J;
            const bool asc = lane_in(~pos_bit<E, HALF>(KK, e));
            if (k[e] != k[hi] && ((k[e] < k[hi]) != asc)) {
                const float tk = k[e]; k[e] = k[hi]; k[hi] = tk;
                const uint32_t tv = v[e]; v[e] = v[hi]; v[hi] = tv;
            }
        }
    }
}

// The steps J, J/2, .. 1 of block size KK.
template <int E, bool HALF, int KK, int J>
__device__ __forceinline__ void bitonic_stage(float (&k)[E], uint32_t (&v)[E]) {
    bitonic_step<E, HALF, KK, J>(k, v);
    if constexpr (J > 1) bitonic_stage<E, HALF, KK, J / 2>(k, v);
}

// Block sizes KK, 2 KK, .. TOP on the HALF layout.
template <int KK, int TOP = 32>
__device__ __forceinline__ void sort32_from(float (&k)[1], uint32_t (&v)[1]) {
    bitonic_stage<1, true, KK, KK / 2>(k, v);
    if constexpr (KK < TOP) sort32_from<KK * 2, TOP>(k, v);
}

// warp_sort<1> on 32 positions (utils.cuh:409-414): position = lane & 31, both
// halves sort the same data.  With TOP < 32 only the stages of block sizes up
// to TOP run.  That equals the full network when positions TOP..31 all hold
// the same (FLT_MAX, MAX_INDEX) pair and no key below them exceeds FLT_MAX:
// block 0 then ends sorted ascending, every later compare-exchange meets
// either that pair or equal or ordered keys, and none of them swaps.
template <int TOP = 32>
__device__ __forceinline__ void sort32(float &key, uint32_t &val) {
    float k[1] = {key};
    uint32_t v[1] = {val};
    sort32_from<2, TOP>(k, v);
    key = k[0];
    val = v[0];
}

__device__ __forceinline__ float pair_key(uint2 e) { return __uint_as_float(e.x); }

// Small merge, pbeam <= 128: topk_small_by_bitonic_sort<1, pbeam/32>
// (utils.cuh:490-586).  Beam position p takes sorted candidate pbeam-1-p when
// that one is smaller (the reversed candidates turn beam + candidates into a
// bitonic sequence), then the merge stages of block size pbeam.  The sorted
// candidates come from the staging array: index min(pbeam-1-p, 32) is a
// FLT_MAX entry whenever pbeam-1-p >= cbs, which never replaces anything.
// The reference's `first` strided load + sort is skipped: it runs only at
// iteration 0, when every beam entry is the identical (FLT_MAX, MAX_INDEX)
// pair, where it is the identity.
template <int E, bool HALF>
__device__ __forceinline__ void small_merge(int pbeam, uint2 *bp, const uint2 *ms, int base, bool writer) {
    float k[E];
    uint32_t v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const uint2 b = bp[base + e];
        const int kc = pbeam - 1 - (base + e);
        const uint2 c = ms[kc < 32 ? kc : 32];
        const bool take = pair_key(c) < pair_key(b);
        k[e] = take ? pair_key(c) : pair_key(b);
        v[e] = take ? c.y : b.y;
    }
    bitonic_stage<E, HALF, (HALF ? 32 : 64 * E), (HALF ? 16 : 32 * E)>(k, v);
    if (writer) {
#pragma unroll
        for (int e = 0; e < E; ++e) bp[base + e] = make_uint2(__float_as_uint(k[e]), v[e]);
    }
}

// Merge-path, pbeam > 128: topk_candidate_sort_and_merge (utils.cuh:618-680)
// with the reference block's segmentation: `active` segments, segment t
// writes outputs [d(t), d(t+1)) with d(t) = t * pbeam / active (at most 4,
// since active >= pbeam / 4), its split point found by the reference's
// binary search (utils.cuh:588-616); inside a segment beam entries go first
// on ties (utils.cuh:652-671).  Each lane searches the right boundaries of
// its segments; a left one is the previous segment's right one.  The
// searches read the sentinel-padded arrays, so no bound needs a branch:
// bp[-1], ms[-1] = -FLT_MAX and bp[pbeam], ms[32] = FLT_MAX stand for the
// reference's out-of-range values.  Segments before `tbase` are not touched
// (the caller has shown that they output the beam unchanged); lane l owns
// segments tbase + l, tbase + 64 + l, ... (SPL of them).
//
// The splits valid at a diagonal d (i beam entries and d - i candidates,
// with beam[i-1] <= cand[d-i] and cand[d-i-1] <= beam[i]) form an interval
// [L, R], and R - 1 is valid only if beam[R-1] and cand[d-R] have equal keys.
// When no boundary has such a pair the split is unique, and the reference's
// bisection, which returns some valid split, returns R: then R is found by a
// plain binary search for the last i with beam[i-1] <= cand[d-i] (steps of
// 32 .. 1 over at most 33 values).  An equal pair at the key FLT_MAX is two
// empty (FLT_MAX, MAX_INDEX) entries when `fast_ok` (no other pair with a key
// outside (-FLT_MAX, FLT_MAX) has been merged into this beam), and every
// split of such a tie gives the same output.  Any other equal pair sends the
// whole wave through the reference's bisection, replayed step by step.
template <int SPL, int NW = 1>
__device__ __forceinline__ void merge_path(const SearchParams &P, uint2 *bp, const uint2 *ms, bool fast_ok,
                                           int tbase) {
    const int lane = lane_id_opaque();
    const int cbs = P.cbs, pbeam = P.pbeam, active = P.seg_active;
    // step k of lane l: segment tbase + 64 k + l (consecutive lanes, and so
    // nearby LDS addresses, in every step)
    int tk[SPL], dl[SPL], dr[SPL], rl[SPL], rr[SPL];
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
        tk[k] = tbase + 64 * k + lane;
        const int a = min(tk[k], active), b = min(tk[k] + 1, active);
        dl[k] = static_cast<int>(__umulhi(static_cast<uint32_t>(a * pbeam), P.seg_magic));
        dr[k] = static_cast<int>(__umulhi(static_cast<uint32_t>(b * pbeam), P.seg_magic));
    }
    const float *bk = reinterpret_cast<const float *>(bp);  // key of entry i at bk[2 i]
    const float *mk = reinterpret_cast<const float *>(ms);
    bool replay = !fast_ok;
    if (fast_ok) {
        // pos holds a split with beam[pos-1] <= cand[d-pos] (true at lo0);
        // steps of 32, 16, .. 1 move it to the last such split up to hi,
        // testing min(pos + s, hi) so that every read stays in range
        int pos[SPL], hi[SPL], lo0[SPL], dd[SPL];
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
            const bool act = tk[k] + 1 <= active;
            dd[k] = act ? dr[k] : 0;
            lo0[k] = max(dd[k] - cbs, 0);
            hi[k] = min(dd[k], pbeam);
            pos[k] = lo0[k];
        }
#pragma unroll
        for (int st = 32; st >= 1; st >>= 1) {
#pragma unroll
            for (int k = 0; k < SPL; ++k) {
                const int c = min(pos[k] + st, hi[k]);
                pos[k] = bk[2 * c - 2] <= mk[2 * (dd[k] - c)] ? c : pos[k];
            }
        }
        bool tie = false;
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
            const int r = pos[k];
            const bool below = r > lo0[k];  // then beam[r-1] and cand[d-r] both exist
            const float a = bk[2 * (below ? r : 1) - 2], b = mk[2 * (below ? dd[k] - r : 0)];
            tie |= below && a == b && a != FLT_MAX;
            rr[k] = r;
        }
        replay = any_lane(tie);
    }
    if (replay) {
        int lo[SPL], hi[SPL];
        bool done[SPL];
#pragma unroll
        for (int k = 0; k < SPL; ++k) {
            lo[k] = max(dr[k] - cbs, 0);
            hi[k] = min(dr[k], pbeam);
            done[k] = tk[k] + 1 > active;
            rr[k] = 0;
        }
        for (;;) {
            bool live = false;
#pragma unroll
            for (int k = 0; k < SPL; ++k) {
                // branch-free round: all four values are read (one LDS round
                // trip, two ds_read2), then the reference's if / else-if / else
                // picks the update
                const bool exit_low = !done[k] && lo[k] > hi[k];  // loop exit: return low
                rr[k] = exit_low ? lo[k] : rr[k];
                done[k] = done[k] || exit_low;
                const int ai = done[k] ? 0 : (lo[k] + hi[k]) >> 1;
                const int bj = done[k] ? 0 : dr[k] - ai;
                const float al = bk[2 * ai - 2], ar = bk[2 * ai];
                const float bl = mk[2 * bj - 2], br = mk[2 * bj];
                const bool go_left = al > br, go_right = !go_left && bl > ar;
                const bool found = !done[k] && !go_left && !go_right;
                hi[k] = (!done[k] && go_left) ? ai - 1 : hi[k];
                lo[k] = (!done[k] && go_right) ? ai + 1 : lo[k];
                rr[k] = found ? ai : rr[k];
                done[k] = done[k] || found;
                live |= !done[k];
            }
            if (!any_lane(live)) break;
        }
    }
    // left boundaries: the right boundary of the previous segment, on the
    // lane below (DPP wave_shr:1), or for lane 0 on lane 63 of the previous
    // step; segment tbase starts with beam entries only (d(0) = 0)
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
        rl[k] = __builtin_amdgcn_update_dpp(0, rr[k], 0x138, 0xF, 0xF, false);
        if (lane == 0) rl[k] = k == 0 ? dl[0] : __builtin_amdgcn_readlane(rr[k > 0 ? k - 1 : 0], 63);
    }
    // Each segment's na beam entries and nb candidates (na + nb <= 4) are
    // read into 4 slots: slot s is beam entry tb + s for s < na, candidate
    // cb + s - na after.  Output position of a slot = d(t) + the number of
    // slots ordered before it: within one list by index, across lists beam
    // first unless the candidate is strictly smaller.
    uint2 slot[SPL][4];
    int pos[SPL][4];
    int nsl[SPL];
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
        const bool act = tk[k] < active;
        const int tb = act ? rl[k] : 0;
        const int cb = act ? dl[k] - rl[k] : 0;
        nsl[k] = act ? dr[k] - dl[k] : 0;
        // The bisection resolves equal keys at each boundary on its own, so
        // two boundaries can disagree (seen at the first merge, where every
        // entry is the empty pair): more than nsl beam entries, or fewer
        // than none.  The reference's output loop then takes only beam
        // entries, or only candidates from cb on (utils.cuh:660-671), which is
        // what the count clamped to [0, nsl] gives.
        const int na = act ? min(max(rr[k] - rl[k], 0), nsl[k]) : 0;
        bool ina[4];
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
            ina[s2] = s2 < na;
            slot[k][s2] = ina[s2] ? bp[tb + s2] : ms[cb + s2 - na];
            pos[k][s2] = dl[k];
        }
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
            for (int u = s2 + 1; u < 4; ++u) {
                // slots at or past nsl are unused: they never count
                const bool cross = ina[s2] && !ina[u];
                const bool first = !cross || !(pair_key(slot[k][u]) < pair_key(slot[k][s2]));
                pos[k][u] += first ? 1 : 0;
                pos[k][s2] += (!first && u < nsl[k]) ? 1 : 0;
            }
    }
    // every lane has read its inputs before any output overwrites them
    lead_sync<NW>();
#pragma unroll
    for (int k = 0; k < SPL; ++k)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) bp[s2 < nsl[k] ? pos[k][s2] : pbeam + 2] = slot[k][s2];
}

// Beam merge (utils.cuh:1369-1399 dispatch for a <= 32-entry buffer): the
// candidates (slot s: distance cd[2 s], id ci[2 s], the pairs of `ms`) are
// read into registers, sorted (warp_sort<1>), written back to `ms` in sorted
// order, and merged into the beam in place.  `span`: slots at or past it hold (FLT_MAX, MAX_INDEX), so a
// candidate buffer filled only in its first 8 or 16 slots is sorted with the
// stages that reach that block size (sort32<TOP>).  `fast_ok` stays true while
// every pair merged into this beam has a key in (-FLT_MAX, FLT_MAX) or is the
// empty (FLT_MAX, MAX_INDEX) pair (merge_path's condition for its split
// search).
// BIG: pbeam > 256 (the merge-path with two or more segments per lane).
template <bool BIG, int NW = 1>
__device__ __forceinline__ void merge_beam(const SearchParams &P, uint2 *bp, uint2 *ms, const float *cd,
                                           const uint32_t *ci, int span, bool &fast_ok, int &lb_out) {
    const int lane = lane_id_opaque();
    lb_out = 0;
    const int nl = lane & 31, h = lane >> 5;
    const int cbs = P.cbs, pbeam = P.pbeam;
    float ck = nl < cbs ? cd[2 * nl] : FLT_MAX;
    uint32_t cv = nl < cbs ? ci[2 * nl] : kMaxIndex;
    fast_ok = fast_ok && !any_lane(!((ck > -FLT_MAX && ck < FLT_MAX) || (ck == FLT_MAX && cv == kMaxIndex)));
    // every key of the span at most FLT_MAX (never inf or NaN)
    const bool short_ok = !any_lane(nl < span && !(ck <= FLT_MAX));
    if (short_ok && span <= 8) sort32<8>(ck, cv);
    else if (short_ok && span <= 16) sort32<16>(ck, cv);
    else sort32(ck, cv);
    if (h == 0) ms[nl] = make_uint2(__float_as_uint(ck), cv);
    lead_sync<NW>();
    if constexpr (!BIG) {
        if (pbeam == 128) {
            small_merge<2, false>(pbeam, bp, ms, 2 * lane, true);
        } else if (pbeam == 64) {
            small_merge<1, false>(pbeam, bp, ms, lane, true);
        } else if (pbeam == 32) {
            small_merge<1, true>(pbeam, bp, ms, nl, h == 0);
        } else {
            merge_path<1, NW>(P, bp, ms, fast_ok, 0);  // one segment per lane: nothing to save
        }
    } else {
        // Segments whose outputs lie wholly at or before position lb, the
        // number of beam entries with a key below the smallest candidate's,
        // output the beam unchanged: at a diagonal d <= lb the only valid split
        // takes d beam entries (beam[d-1] < cand[0], and any split with fewer
        // would need cand[j] <= beam[i] for some i < d), so the reference's
        // bisection returns it.  lb in two steps of 64 probes; then the first
        // segment t with d(t+1) > lb.
        const int active = P.seg_active;
        const float c0 = pair_key(ms[0]);
        const float *bk = reinterpret_cast<const float *>(bp);
        const int st = (pbeam + 63) / 64;  // <= 16
        const int p1 = min((lane + 1) * st, pbeam) - 1;
        const int c1 = __popcll(ballot(bk[2 * p1] < c0));
        const int q2 = c1 * st + lane;
        const int c2 = __popcll(ballot(lane < st && q2 < pbeam && bk[2 * min(q2, pbeam)] < c0));
        const int lb = uni(min(c1 * st + c2, pbeam));
        lb_out = lb;
        int tf = static_cast<int>(static_cast<uint32_t>(lb) * static_cast<uint32_t>(active) / static_cast<uint32_t>(pbeam));
        const auto seg_end = [&](int t) {
            return static_cast<int>(__umulhi(static_cast<uint32_t>(t * pbeam), P.seg_magic));
        };
        if (tf < active && seg_end(tf + 1) <= lb) ++tf;
        const int spl = (active - tf + 63) / 64;
        if (spl == 1) merge_path<1, NW>(P, bp, ms, fast_ok, tf);
        else if (spl == 2) merge_path<2, NW>(P, bp, ms, fast_ok, tf);
        else if (spl > 2) merge_path<4, NW>(P, bp, ms, fast_ok, tf);
    }
    lead_sync<NW>();
}

// ------------------------------------------------------------ visited table

// Visited set (the reference's utils.cuh:682-750 table, same membership
// semantics): an exact set of node ids in LDS in 4-slot buckets, one 16-byte
// read per bucket.  Each key has two buckets, its home and its alternate; it
// is added to whichever of the two has more empty slots (the home on a tie),
// and only when both are full to the first bucket with an empty slot after
// the alternate (wrapping).  Slots of a bucket fill in order and stay filled
// until the reset, so a bucket is full iff its last slot is taken and a full
// bucket stays full: a lookup reads both buckets and walks on only when both
// are full, stopping at the first bucket that holds the key or has room.
// Empty slots are 0xFFFFFFFF; keys (node ids, and 0x7FFFFFFF for the restore
// of an empty beam slot, utils.cuh:747-748) have the top bit clear.
__device__ __forceinline__ uint32_t hash_home(uint32_t key, uint32_t nb) {
    const uint32_t h16 = (key ^ (key >> 13)) & 0xFFFFu;
    return __umul24(h16, nb) >> 16;
}

// bits 8..23 of a 24-bit product of the key: mixed independently of the home
__device__ __forceinline__ uint32_t hash_alt(uint32_t key, uint32_t nb) {
    const uint32_t h16 = (__umul24(key, 0x9E3779u) >> 8) & 0xFFFFu;
    return __umul24(h16, nb) >> 16;
}

__device__ __forceinline__ uint32_t hash_next(uint32_t b, uint32_t nb) { return b + 1u == nb ? 0u : b + 1u; }

// (min of the four XORs is zero iff one slot equals the key: integer ops the
// compiler keeps as such, where four compares became packed 16-bit flags)
__device__ __forceinline__ bool bucket_has(uint4 s, uint32_t key) {
    return min(min(s.x ^ key, s.y ^ key), min(s.z ^ key, s.w ^ key)) == 0u;
}

__device__ __forceinline__ bool bucket_open(uint4 s) { return static_cast<int32_t>(s.w) < 0; }

__device__ __forceinline__ bool both_full(uint4 a, uint4 b) { return static_cast<int32_t>(a.w | b.w) >= 0; }

// number of empty slots (the empty ones are the last)
__device__ __forceinline__ uint32_t bucket_free(uint4 s) { return (s.x >> 31) + (s.y >> 31) + (s.z >> 31) + (s.w >> 31); }

// 1 if the key was added, 0 if it was present (utils.cuh:697-716).
__device__ __forceinline__ uint32_t hash_insert(uint32_t *t, uint32_t nb, uint32_t key) {
    const uint4 *t4 = reinterpret_cast<const uint4 *>(t);
    const uint32_t ba = hash_home(key, nb), bb = hash_alt(key, nb);
    // a failed CAS means another lane filled a slot of one of the two
    // buckets: at most 8 passes before both are full
    for (int pass = 0; pass < 9; ++pass) {
        const uint4 sa = t4[ba], sb = t4[bb];
        if (bucket_has(sa, key) || bucket_has(sb, key)) return 0;
        const uint32_t fa = bucket_free(sa), fb = bucket_free(sb);
        if (fa == 0u && fb == 0u) break;
        const bool alt = fb > fa;
        const uint32_t slot = 4u * (alt ? bb : ba) + 4u - (alt ? fb : fa);
        const uint32_t old = atomicCAS(&t[slot], kMaxIndex, key);
        if (old == kMaxIndex) return 1;
        if (old == key) return 0;
    }
    uint32_t b = hash_next(bb, nb);
    // each pass either moves to the next bucket or retries after another
    // lane filled a slot of this one: at most 5 passes per bucket
    for (uint32_t i = 0; i < 5u * nb; ++i) {
        const uint4 sl = t4[b];
        if (bucket_has(sl, key)) return 0;
        const uint32_t f = bucket_free(sl);
        if (f == 0u) {
            b = hash_next(b, nb);
            continue;
        }
        const uint32_t old = atomicCAS(&t[4u * b + 4u - f], kMaxIndex, key);
        if (old == kMaxIndex) return 1;
        if (old == key) return 0;
    }
    return 0;
}

__device__ __forceinline__ void hash_reset(uint32_t *t, uint32_t nb) {
    uint4 *t4 = reinterpret_cast<uint4 *>(t);
    const uint4 e = make_uint4(kMaxIndex, kMaxIndex, kMaxIndex, kMaxIndex);
    for (uint32_t i = static_cast<uint32_t>(lane_id()); i < nb; i += 64) t4[i] = e;
}

// true iff an earlier (lower-lane) member of `members` in this half carries
// the same key.  Scans lanes of half h in order via readlane.
__device__ __forceinline__ bool dup_of_earlier(uint32_t key, uint32_t members, int nl, int h) {
    bool dup = false;
    uint32_t m = members;
    while (m) {
        const int s = __builtin_ctz(m);
        m &= m - 1;
        if (s >= 31) break;
        const uint32_t k0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), s));
        const uint32_t k1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), s + 32));
        const uint32_t other = h ? k1 : k0;
        dup |= (s < nl) && (other == key);
    }
    return dup;
}

// ------------------------------------------------------------ the search kernel

struct Controller {
    int spec;
    float rho;
    int policy_iters;
    uint32_t top1;
    int stall;
    bool warm;
    float entry_d, last_e, cur_e;
    uint32_t entry_ok;  // 1 while entry_d is finite and |entry_d| > 1e-20 (set with entry_d)
};

__device__ __forceinline__ uint32_t entry_guard(float e) {
    return (isfinite(e) && fabsf(e) > 1.0e-20f) ? 1u : 0u;
}

// src/adaptive_search.cuh:166-190 + adaptive_search_utils.cuh:32-39, 51-119
// (CHECK_INTERVAL = 1): every lane computes the same values.
__device__ __forceinline__ void controller_step(Controller &c, uint32_t beam0, float phase2_rho) {
    const uint32_t top = beam0 & 0x7fffffffu;
    const int stall = (c.policy_iters > 0 && top == c.top1) ? c.stall + 1 : 0;
    const bool phase_changed = c.warm || stall >= kStallIters;
    const float entry = c.entry_d;
    const float last = finite_below_max(c.last_e) ? c.last_e : entry;
    const float cur = finite_below_max(c.cur_e) ? c.cur_e : last;
    float rate = 0.0f;  // only read while the search stays in stage I
    const float denom = fabsf(entry);
    if (!phase_changed && isfinite(last) && isfinite(cur) && sflag(c.entry_ok)) {
        const float pr = (last - cur) / denom;
        if (isfinite(pr) && pr > 0.0f) rate = pr < 1.0f ? pr : 1.0f;
    }
    c.top1 = top;
    c.stall = stall;
    c.last_e = last;
    c.cur_e = cur;
    if (phase_changed) {
        c.warm = true;
        c.spec = kSearchWidth;
        c.rho = phase2_rho;
    } else {
        const float span = phase2_rho > kPhase1Rho ? phase2_rho - kPhase1Rho : kRhoMax - 0.0f;
        const float base = c.policy_iters == 0 ? kPhase1Rho : c.rho;
        const float cap = phase2_rho > kPhase1Rho ? phase2_rho : kRhoMax;
        c.warm = false;
        c.spec = 1;
        c.rho = clamp_f(fmaf(span, rate, base), 0.0f, cap);
    }
    c.policy_iters += 1;
}

// Loads one neighbour's B/8-byte code as WT words (16-byte vector load when
// the row layout keeps the code block 16-byte aligned).
template <int WT>
__device__ __forceinline__ void load_code(const uint32_t *__restrict__ code, bool vec_ok, uint32_t (&c)[WT]) {
    if constexpr (WT == 4) {
        if (vec_ok) {
            const uint4 v = *reinterpret_cast<const uint4 *>(code);
            c[0] = v.x; c[1] = v.y; c[2] = v.z; c[3] = v.w;
            return;
        }
    }
#pragma unroll
    for (int w = 0; w < WT; ++w) c[w] = code[w];
}

// Horner step over the planes of WT words: 2 acc + sum_w popcount(c_w & pw_w)
// (the top plane starts from zero).
template <int WT>
__device__ __forceinline__ uint32_t plane_step(const uint32_t *c, const uint32_t *pw, uint32_t acc, bool top) {
    uint32_t a = top ? static_cast<uint32_t>(__popc(c[0] & pw[0])) : bcnt_acc(c[0] & pw[0], acc << 1);
#pragma unroll
    for (int w = 1; w < WT; ++w) a = bcnt_acc(c[w] & pw[w], a);
    return a;
}

// raw for NB code blocks at once, walking the planes one at a time from LDS
// (one plane's WT words live at a time), top plane first: raw_b =
// popcount(code_b) + sum_p 2^p popcount(code_b & plane_p) (the planes hold
// q - 1) - popcount(code_b & zero plane) - 256 * wraps_b, the powers of two
// by Horner's rule (one shift per plane and block).
template <int NB, int WT>
__device__ __forceinline__ void raw_batch(const uint32_t (&c)[NB][WT], const uint32_t *planes, bool any_wrap,
                                          bool any_zero, int32_t (&raw)[NB]) {
    uint32_t acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0;
#pragma unroll
    for (int p = kPlanes - 1; p >= 0; --p) {
        uint32_t pw[WT];
#pragma unroll
        for (int w = 0; w < WT; ++w) pw[w] = planes[p * WT + w];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = plane_step<WT>(c[b], pw, acc[b], p == kPlanes - 1);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int w = 0; w < WT; ++w) acc[b] = bcnt_acc(c[b][w], acc[b]);
    if (any_zero) {
        uint32_t pw[WT];
#pragma unroll
        for (int w = 0; w < WT; ++w) pw[w] = planes[kZeroPlane * WT + w];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int w = 0; w < WT; ++w) acc[b] -= static_cast<uint32_t>(__popc(c[b][w] & pw[w]));
    }
    if (any_wrap) {
        uint32_t pw[WT];
#pragma unroll
        for (int w = 0; w < WT; ++w) pw[w] = planes[kWrapPlane * WT + w];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            uint32_t wr = 0;
#pragma unroll
            for (int w = 0; w < WT; ++w) {
                const uint32_t x = c[b][w] & pw[w];
                wr += __popc(x & (x >> 1) & (x >> 2) & (x >> 3) & 0x11111111u);
            }
            acc[b] -= 256u * wr;
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) raw[b] = static_cast<int32_t>(acc[b]);
}

// One pass of exact distances over children e0 .. e0 + 2 PB - 1 (child
// e0 + 2 j + h on half h): PB row loads per lane issued together, then a
// reduce-scatter over the half.  At distance 16 lanes keep children
// j < PB/2 (lower) / j + PB/2 (upper), at 8 the same on what is left, and so
// on until one child per lane group remains; the remaining distances are
// butterflies.  Every step adds lane l and lane l ^ m of the same child, in
// the order 16, 8, 4, 2, 1, so each child's sum is the shfl_down tree of
// utils.cuh:277-281 up to operand order.
template <int PB, int DPL, class G>
__device__ __forceinline__ void exact_pass(const SearchParams &P, const G &g, int e0, int n, const uint32_t *slot_list,
                                           float *cd, const uint32_t *ci, const float (&qr)[DPL], bool ip) {
    const int lane = lane_id();
    const int h = lane >> 5, nl = lane & 31;
    // loads are unconditional: an inactive lane reads a valid list entry
    // and candidate slot and then row 0; its sum is never written.  Slots,
    // then ids, then rows, each group issued together.
    int sl[PB];
    if (slot_list) {
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            const int e = e0 + 2 * j + h;
            sl[j] = static_cast<int>(slot_list[e < 32 ? e : 31] & 31u);  // entries past n may be stale
        }
    } else {
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            const int e = e0 + 2 * j + h;
            sl[j] = e < 32 ? e : 31;
        }
    }
    uint32_t cid[PB];
#pragma unroll
    for (int j = 0; j < PB; ++j) cid[j] = ci[2 * sl[j]];
    float v[PB][DPL];
    if constexpr (G::kFixed) {
        const uint32_t lo = static_cast<uint32_t>(nl) * 4u;  // this lane's first dimension
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            const uint32_t child = e0 + 2 * j + h < n ? cid[j] : 0u;
            const uint32_t off = __umul24(child, G::kRowB) + lo;
#pragma unroll
            for (int k = 0; k < DPL; ++k) v[j][k] = nl + 32 * k < g.dim ? ld_at<float>(P.data, off + 128u * k) : 0.0f;
        }
    } else {
        const float *dl = P.data + nl;  // this lane's first dimension of row 0
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            const uint32_t child = e0 + 2 * j + h < n ? cid[j] : 0u;
            const float *row = dl + static_cast<uint64_t>(child) * g.row;
#pragma unroll
            for (int k = 0; k < DPL; ++k) v[j][k] = nl + 32 * k < g.dim ? row[32 * k] : 0.0f;
        }
    }
    // the metric test sits outside the loops: inside, each dimension became
    // both updates and a select
    float acc[PB];
    if (ip) {
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            acc[j] = 0.0f;
#pragma unroll
            for (int k = 0; k < DPL; ++k)
                if (nl + 32 * k < g.dim) acc[j] = fmaf(qr[k], v[j][k], acc[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            acc[j] = 0.0f;
#pragma unroll
            for (int k = 0; k < DPL; ++k) {
                if (nl + 32 * k < g.dim) {
                    const float d = qr[k] - v[j][k];
                    acc[j] = fmaf(d, d, acc[j]);
                }
            }
        }
    }
    // reduce-scatter while more than one child is left per lane
    int c = 0;  // index of the child this lane's value belongs to
    constexpr int L16 = PB >= 2 ? PB / 2 : 1;
    float r16[L16];
    if constexpr (PB >= 2) {
        // rows with bit 16 clear keep child j, the others child j + L16
#pragma unroll
        for (int j = 0; j < L16; ++j) {
            const Pair q = swap16(acc[j], acc[j + L16]);
            r16[j] = q.lo + q.hi;
        }
        c += (nl & 16) ? L16 : 0;
    } else {
        const Pair q = swap16(acc[0], acc[0]);
        r16[0] = q.lo + q.hi;
    }
    constexpr int L8 = L16 >= 2 ? L16 / 2 : 1;
    float r8[L8];
    if constexpr (L16 >= 2) {
        const bool b = (nl & 8) != 0;
#pragma unroll
        for (int j = 0; j < L8; ++j) {
            const float send = b ? r16[j] : r16[j + L8];
            const float own = b ? r16[j + L8] : r16[j];
            r8[j] = own + xshfl(send, 8);
        }
        c += b ? L8 : 0;
    } else {
        r8[0] = r16[0] + xshfl(r16[0], 8);
    }
    float r4;
    if constexpr (L8 >= 2) {
        const bool b = (nl & 4) != 0;
        const float send = b ? r8[0] : r8[1];
        const float own = b ? r8[1] : r8[0];
        r4 = own + xshfl(send, 4);
        c += b ? 1 : 0;
    } else {
        r4 = r8[0] + xshfl(r8[0], 4);
    }
    r4 += xshfl(r4, 2);
    r4 += xshfl(r4, 1);
    // lanes holding child c: one writer per child (the lowest lane of its group)
    constexpr int kGroup = PB >= 8 ? 4 : PB >= 4 ? 8 : PB >= 2 ? 16 : 32;
    const int e = e0 + 2 * c + h;
    if (e < n && (nl & (kGroup - 1)) == 0) {
        const int sl = slot_list ? static_cast<int>(slot_list[e] & 31u) : e;
        cd[2 * sl] = beam_key(ip ? -r4 : r4);
    }
}

// Exact distances for children lo .. n-1 held in the candidate pairs (id at
// ci[2 s], distance written to cd[2 s]) at slots
// slot_list[lo..n) (or lo..n when slot_list is null): passes of 16
// children, the last one sized to what is left (DPL > 0: dims per lane known
// at compile time; DPL == 0: generic geometry, exact_generic_pass).
// exact_batch: all n (lo = 0).
template <int DPL, class G>
__device__ __forceinline__ void exact_batch_range(const SearchParams &P, const G &g, int lo, int n,
                                                  const uint32_t *slot_list, float *cd, const uint32_t *ci,
                                                  const float (&qr)[DPL > 0 ? DPL : 1], const float *qv) {
    const int lane = lane_id();
    const int h = lane >> 5, nl = lane & 31;
    const bool ip = sflag(static_cast<uint32_t>(P.use_ip));
    if constexpr (DPL > 0) {
        int e0 = lo;
        for (; n - e0 > 8; e0 += 16) exact_pass<8, DPL>(P, g, e0, n, slot_list, cd, ci, qr, ip);
        const int rem = n - e0;
        if (rem > 4) exact_pass<4, DPL>(P, g, e0, n, slot_list, cd, ci, qr, ip);
        else if (rem > 2) exact_pass<2, DPL>(P, g, e0, n, slot_list, cd, ci, qr, ip);
        else if (rem > 0) exact_pass<1, DPL>(P, g, e0, n, slot_list, cd, ci, qr, ip);
    } else {
        // six children per pass (three per half), 16 dimension steps per
        // load batch; the last pass sized to what is left
        int e0 = lo;
        for (; n - e0 > 4; e0 += 6) exact_generic_pass<3, 16>(P, g.row, g.dim, e0, n, slot_list, cd, ci, qv, ip);
        if (n - e0 > 2) exact_generic_pass<2, 16>(P, g.row, g.dim, e0, n, slot_list, cd, ci, qv, ip);
        else if (e0 < n) exact_generic_pass<1, 16>(P, g.row, g.dim, e0, n, slot_list, cd, ci, qv, ip);
    }
}

template <int DPL, class G>
__device__ __forceinline__ void exact_batch(const SearchParams &P, const G &g, int n, const uint32_t *slot_list, float *cd,
                                            const uint32_t *ci, const float (&qr)[DPL > 0 ? DPL : 1], const float *qv) {
    exact_batch_range<DPL>(P, g, 0, n, slot_list, cd, ci, qr, qv);
}

// The keep_k smallest valid (value, lane) pairs of each 32-lane half, as
// warp_keep_topk_smallest_f32 (utils.cuh:251-267) selects them, found by
// keep_k rounds of group argmin (G = 32: half-wave; 16: 16-lane row) instead
// of a 32-step rank count.  keep_k is uniform within each group; valid lanes
// and the result are lane masks.
template <int G>
__device__ __forceinline__ uint64_t select_smallest(float value, uint64_t valid, int keep_k, int max_k) {
    // order-preserving unsigned image of the float; -0 joins +0 so equal
    // values tie exactly as in the float comparison
    const uint32_t bits = __float_as_uint(value == 0.0f ? 0.0f : value);
    const uint32_t key = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    uint64_t remaining = valid, kept = 0ull;
    for (int r = 0; r < max_k; ++r) {
        uint32_t m = lane_in(remaining) ? key : 0xFFFFFFFFu;
        // minimum over the 32-lane half: quad (xor 1, xor 2), then the
        // half-row and row mirrors bring in the other quad and the other
        // half-row, then the neighbouring row
        m = min(m, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(m), 0xB1, 0xF, 0xF, true)));
        m = min(m, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(m), 0x4E, 0xF, 0xF, true)));
        m = min(m, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(m), 0x141, 0xF, 0xF, true)));
        m = min(m, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(m), 0x140, 0xF, 0xF, true)));
        if constexpr (G == 32) m = min16(m);  // (G = 16: the row's minimum is the group's)
        // the lowest lane of each group holding its group's minimum (x & -x on
        // each G-bit part of the mask), taken while the group keeps more
        const uint64_t cand = ballot(key == m) & remaining;
        uint64_t first;
        if constexpr (G == 32) {
            const uint32_t c0 = static_cast<uint32_t>(cand), c1 = static_cast<uint32_t>(cand >> 32);
            first = (static_cast<uint64_t>(c1 & (0u - c1)) << 32) | (c0 & (0u - c0));
        } else {
            first = 0ull;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t c = static_cast<uint32_t>(cand >> (16 * g)) & 0xFFFFu;
                first |= static_cast<uint64_t>(c & (0u - c)) << (16 * g);
            }
        }
        const uint64_t take = first & ballot(r < keep_k);
        kept |= take;
        remaining &= ~take;
    }
    return kept;
}

// Visited test for up to four keys per lane: both buckets of every key are
// read at once; the rare keys whose two buckets are full walk on together.
template <int NK>
__device__ __forceinline__ void hash_contains_n(const uint32_t *t, uint32_t nb, const uint32_t (&key)[NK],
                                                bool (&test)[NK]) {
    const uint4 *t4 = reinterpret_cast<const uint4 *>(t);
    uint32_t b[NK];
    bool pend[NK];
    bool anyp = false;
#pragma unroll
    for (int s = 0; s < NK; ++s) {
        // branch-free: every lane reads both buckets (indices always in range)
        b[s] = hash_alt(key[s], nb);
        const uint4 sa = t4[hash_home(key[s], nb)], sb = t4[b[s]];
        const bool has = bucket_has(sa, key[s]) || bucket_has(sb, key[s]);
        pend[s] = test[s] && !has && both_full(sa, sb);
        test[s] = test[s] && !has;  // contained: not a fresh child
        anyp |= pend[s];
    }
    if (!any_lane(anyp)) return;
    for (uint32_t step = 0; step < nb; ++step) {
        anyp = false;
#pragma unroll
        for (int s = 0; s < NK; ++s) {
            b[s] = pend[s] ? hash_next(b[s], nb) : b[s];
            const uint4 sl = t4[b[s]];
            const bool has = bucket_has(sl, key[s]);
            test[s] = (pend[s] && has) ? false : test[s];
            pend[s] = pend[s] && !has && !bucket_open(sl);
            anyp |= pend[s];
        }
        if (!any_lane(anyp)) break;
    }
}

// Phase timer for the profiling instantiation: cycles since the previous
// mark are added to LDS counter `i` (s_memtime, per wave).
#define FG_PHASE(i)                                                  \
    do {                                                             \
        if constexpr (PROF) {                                        \
            const unsigned long long t_ = __builtin_amdgcn_s_memtime(); \
            if (lead && lane == 0) prof[i] += t_ - t_last;           \
            t_last = t_;                                             \
        }                                                            \
    } while (0)

#define FG_COUNT(stmt)            \
    do {                          \
        if constexpr (COUNT) stmt; \
    } while (0)

// One wave per workgroup; the register budget targets 5 waves per SIMD
// (<= 96 VGPRs; the fixed-geometry kernels use 77-79, which leaves room for
// a sixth), which LDS also allows for beams up to 256 (6,144 bytes a
// workgroup at beam 256).  The generic-geometry instantiation (padded dimension
// >= 256) gets 3 (<= 168 VGPRs) for its wide code batches and the plane reads
// it keeps in flight: at padded dimension 2048 its LDS (raw query, planes,
// rotation scratch) holds it to 3 waves per SIMD anyway, and at 1024 a
// 1,000-query launch fills one wave per SIMD.
// NW = 2: the team form (two waves per query; see TeamBlock).  Wave 0 leads:
// it runs every phase, the helper wave joins it in stage II's rounds and the
// exact distances; `lead_sync` orders the lead wave's own LDS accesses and
// the workgroup barriers mark the meeting points.
template <int WT, int DPL, int DIM_T, int DEG_T, bool COUNT, bool PROF, bool BIG, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WT == 0 ? 3 : 5))) void fg_search_kernel(SearchParams P) {
    static_assert(NW == 1 || NW == 2, "team form: two waves");
    extern __shared__ __align__(16) unsigned char smem[];
    int qid = blockIdx.x;
    if (qid >= P.nq) return;
    // the two-launch search runs in the one-wave form
    constexpr bool kSliceable = NW == 1 && !PROF;
    if constexpr (kSliceable) {
        if (P.slice_resume > 0) {
            // workgroup w resumes the w-th query of the order, if there is one
            const uint32_t n = __builtin_amdgcn_readfirstlane(P.slice_state[0]);
            if (static_cast<uint32_t>(qid) >= n) return;
            const uint32_t o = __builtin_amdgcn_readfirstlane(P.slice_order[qid]);
            if (o >= static_cast<uint32_t>(P.nq)) return;
            qid = static_cast<int>(o);
        }
    }
    const int lane = lane_id();
    // wave index within the team (0 for the one-wave form)
    const int wv = NW > 1 ? (__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x)) >> 6) : 0;
    const bool lead = NW == 1 || wv == 0;
    TeamBlock *tb = reinterpret_cast<TeamBlock *>(smem + P.lds.team_off);
    (void)tb;
    const int h = lane >> 5, nl = lane & 31;
    const Geo<DIM_T, DEG_T> g(P);
    const int B = g.B, W = B >> 5;
    const int deg = g.deg;
    const uint32_t nbk = static_cast<uint32_t>(P.buckets);
    const bool vec_ok = P.vec_ok != 0;

    // fixed-size regions at compile-time offsets for the specialised shapes
    // (the same layout function the host sizes the launch with)
    constexpr bool kFixedGeo = Geo<DIM_T, DEG_T>::kFixed;
    constexpr LdsLayout kL = lds_layout(DIM_T, Geo<DIM_T, DEG_T>::kB, 0, 0);
    const uint32_t plane_off = kFixedGeo ? kL.plane_off : P.lds.plane_off;
    const uint32_t scratch_off = kFixedGeo ? kL.scratch_off : P.lds.scratch_off;
    const uint32_t prof_off = P.lds.prof_off;
    static_assert(kL.msort_off == 0u, "fixed LDS regions");
    uint32_t *H = reinterpret_cast<uint32_t *>(smem + P.lds.hash_off);
    // beam pairs: bp[-1] and bp[pbeam] are sentinels
    uint2 *bp = reinterpret_cast<uint2 *>(smem + P.lds.beam_off) + 1;
    uint2 *ms = reinterpret_cast<uint2 *>(smem + kL.msort_off) + 1;
    // candidate slot s: distance at cd[2 s], id at ci[2 s] (the pair ms[s])
    float *cd = reinterpret_cast<float *>(ms);
    uint32_t *ci = reinterpret_cast<uint32_t *>(ms) + 1;
    uint32_t *planes = reinterpret_cast<uint32_t *>(smem + plane_off);
    uint32_t *alist = reinterpret_cast<uint32_t *>(smem + scratch_off);
    uint32_t *pnode = alist + 32;
    float *pdist = reinterpret_cast<float *>(pnode + 8);
    unsigned long long *prof = reinterpret_cast<unsigned long long *>(smem + prof_off);
    unsigned long long t_last = 0, t_begin = 0;
    if constexpr (PROF) {
        if (lane < 16) prof[lane] = 0;
        t_begin = __builtin_amdgcn_s_memrealtime();
        t_last = __builtin_amdgcn_s_memtime();
    }

    // ---- query preparation (the visited table's LDS holds the rotation); a
    // query resumed by the second slice reads back the planes and constants
    // the first slice kept instead
    float qlow = 0.0f, qhigh = 0.0f, qwidth = 0.0f;
    int sum_q = 0;
    const bool resuming = kSliceable && P.slice_resume > 0;
    if (lead) {
        if (resuming) {
            const uint32_t *sp = P.slice_state + kSliceHeader +
                                 static_cast<uint64_t>(qid) * slice_words(static_cast<uint32_t>(P.pbeam), B) +
                                 slice_prep_offset(static_cast<uint32_t>(P.pbeam));
            for (int i = lane; i < 8 * W; i += 64) planes[i] = sp[4 + i];
            qlow = __uint_as_float(uni(sp[0]));
            qwidth = __uint_as_float(uni(sp[1]));
            sum_q = static_cast<int>(uni(sp[2]));
            lead_sync<NW>();
        } else {
            prepare_query<NW>(P.queries + static_cast<uint64_t>(qid) * g.dim, P.signs, g.dim, B,
                              reinterpret_cast<float *>(H), nullptr, planes, qlow, qhigh, qwidth, sum_q, nullptr);
        }
    }
    // the query is read from global memory, where it stays cached (the
    // generic geometry's exact distances read it there; the others keep it in
    // registers, qr below)
    const float *qsrc = P.queries + static_cast<uint64_t>(qid) * g.dim;
    constexpr int WTR = WT > 0 ? WT : 1;
    // whether any chunk of the quantized query wraps the reference's uint8
    // LUT entry (then the estimates subtract the wrapped chunks)
    uint32_t any_wrap = 0u, any_zero = 0u;  // 0 / 1 (sflag at each use)
    if (lead) {
        if constexpr (WT > 0) {
            uint32_t wor = 0, zor = 0;
#pragma unroll
            for (int w = 0; w < WT; ++w) {
                wor |= planes[kWrapPlane * WT + w];
                zor |= planes[kZeroPlane * WT + w];
            }
            any_wrap = uni(wor) != 0u ? 1u : 0u;
            any_zero = uni(zor) != 0u ? 1u : 0u;
        } else {
            uint32_t wor = 0, zor = 0;
            for (int w = lane; w < W; w += 64) {
                wor |= planes[kWrapPlane * W + w];
                zor |= planes[kZeroPlane * W + w];
            }
            any_wrap = any_lane(wor != 0u) ? 1u : 0u;
            any_zero = any_lane(zor != 0u) ? 1u : 0u;
        }
    }
    constexpr int DPLR = DPL > 0 ? DPL : 1;
    float qr[DPLR];
#pragma unroll
    for (int k = 0; k < DPLR; ++k) {
        const int i = nl + 32 * k;
        qr[k] = (DPL > 0 && i < g.dim) ? qsrc[i] : 0.0f;
    }

    const uint2 kEmpty = make_uint2(__float_as_uint(FLT_MAX), kMaxIndex);
    const uint2 kLowSentinel = make_uint2(__float_as_uint(-FLT_MAX), kMaxIndex);
    float entry_d = 0.0f;
    if (lead) {
        // (a resumed query's entry distance comes back with its controller)
        if (!resuming)
            entry_d = uni(beam_key(half_distance(P.data + static_cast<uint64_t>(P.entry) * g.row, qsrc, g.dim, nl,
                                                 P.use_ip != 0, true)));

        // ---- state (adaptive_search.cuh:67-107)
        hash_reset(H, nbk);
        for (int i = lane - 1; i < P.pbeam + static_cast<int>(kBeamPad); i += 64) bp[i] = i < 0 ? kLowSentinel : kEmpty;
        if (lane <= kMsortHi + 1) ms[lane - 1] = lane == 0 ? kLowSentinel : kEmpty;  // candidates empty
        lead_sync<NW>();
        if (lane == 0) {
            ms[0] = make_uint2(__float_as_uint(entry_d), P.entry);
            hash_insert(H, nbk, P.entry);
        }
        lead_sync<NW>();
    }
    if constexpr (NW > 1) {
        // the quantised query's constants, for the helper
        if (lead && lane == 0) {
            tb->sum_q = static_cast<uint32_t>(sum_q);
            tb->qwidth_bits = __float_as_uint(qwidth);
            tb->qlow_bits = __float_as_uint(qlow);
            tb->any_wrap = any_wrap;
            tb->any_zero = any_zero;
        }
        __syncthreads();
        if (!lead) {
            sum_q = static_cast<int>(uni(tb->sum_q));
            qwidth = __uint_as_float(uni(tb->qwidth_bits));
            qlow = __uint_as_float(uni(tb->qlow_bits));
            any_wrap = uni(tb->any_wrap) != 0u ? 1u : 0u;
            any_zero = uni(tb->any_zero) != 0u ? 1u : 0u;
        }
    }

    Controller ctl{1, kPhase1Rho, 0, kMaxIndex, 0, false, entry_d, FLT_MAX, FLT_MAX, uni(entry_guard(entry_d))};
    uint32_t c_iters = 0, c_exp = 0, c_ids = 0, c_est = 0, c_exact = 1, c_st2 = kMaxIndex;
    const int beam_sz = P.beam, pbeam = P.pbeam;
    const int cbs = P.cbs;
    // ranges the host guarantees (make_params), stated so that the compiler
    // keeps no guard on them live across the search loop: each such guard is
    // a 64-bit lane mask, and the loop is short of scalar registers
    __builtin_assume(beam_sz >= 1 && beam_sz <= kMaxBeam && pbeam >= beam_sz && pbeam <= kMaxBeam);
    __builtin_assume(cbs >= 1 && cbs <= kBufferBound && nbk >= 1u && P.K >= 1);
    // the node count as a 32-bit bound: ids are 32-bit and MAX_INDEX is tested
    // apart wherever an id is checked, so min(npoints, MAX_INDEX) decides
    // the same and is one scalar register and a 32-bit compare
    const uint32_t np32 = uni(P.npoints > 0xFFFFFFFFull ? 0xFFFFFFFFu : static_cast<uint32_t>(P.npoints));
    // candidate slots the next merge may find filled (the rest hold the
    // reset pair): the entry point's slot 0 first, then what each stage fills
    int cand_span = 1;
    bool split_fast = true;  // merge_path may search its splits directly
    // beams over 256: every beam entry before scan_from is expanded (the pick
    // starts there); a merge leaves entries before its lb in place
    int scan_from = 0, lb_merge = 0;
    const float *data = P.data;

    int iter = 0;
    bool suspended = false;
    // the iteration at whose top an unfinished query suspends (-1: never)
    const int suspend_at = (kSliceable && P.slice_suspend > 0) ? P.slice_suspend : -1;
    if constexpr (kSliceable) {
        if (P.slice_resume > 0) {
            // resume at the top of iteration slice_resume (before its visited-table
            // rebuild, which derives the table from the beam): the beam, the
            // unmerged candidates, the controller and the counters as the first
            // slice left them.  Ids are checked so that no later row read can
            // leave the codebook, whatever the buffer holds.
            const uint32_t *st = P.slice_state + kSliceHeader + static_cast<uint64_t>(qid) * slice_words(pbeam, B);
            const uint2 *sb = reinterpret_cast<const uint2 *>(st + kSliceFixed);
            const uint2 kEmptyPair = make_uint2(__float_as_uint(FLT_MAX), kMaxIndex);
            for (int i = lane; i < pbeam + 32; i += 64) {
                const uint2 e = sb[i];
                const bool ok = e.y == kMaxIndex || static_cast<uint64_t>(e.y & 0x7FFFFFFFu) < P.npoints;
                if (i < pbeam) bp[i] = ok ? e : kEmptyPair;
                else ms[i - pbeam] = ok ? e : kEmptyPair;
            }
            ctl.spec = clamp_i(static_cast<int>(uni(st[2])), 1, kSearchWidth);
            ctl.rho = __uint_as_float(uni(st[3]));
            ctl.policy_iters = static_cast<int>(uni(st[4]));
            ctl.top1 = uni(st[5]);
            ctl.stall = static_cast<int>(uni(st[6]));
            ctl.warm = uni(st[7]) != 0u;
            ctl.entry_d = __uint_as_float(uni(st[8]));
            ctl.entry_ok = uni(entry_guard(ctl.entry_d));
            ctl.last_e = __uint_as_float(uni(st[9]));
            ctl.cur_e = __uint_as_float(uni(st[10]));
            c_iters = uni(st[11]);
            c_exp = uni(st[12]);
            c_ids = uni(st[13]);
            c_est = uni(st[14]);
            c_exact = uni(st[15]);
            c_st2 = uni(st[16]);
            cand_span = clamp_i(static_cast<int>(uni(st[17])), 0, kBufferBound);
            split_fast = uni(st[18]) != 0u;
            scan_from = clamp_i(static_cast<int>(uni(st[19])), 0, beam_sz);
            iter = P.slice_resume;
            lead_sync<NW>();
        }
    }

    FG_PHASE(0);
    for (; iter < kMaxIterations; ++iter) {
        if constexpr (kSliceable) {
            if (iter == suspend_at) {
                suspended = true;
                break;
            }
        }
        // lane-derived values are recomputed in each iteration, not held
        const int lane = lane_id_opaque();
        const int h = lane >> 5, nl = lane & 31;
        // the iteration's uniform state; the lead wave computes it, a helper
        // wave receives it at the meeting point below
        float kth = FLT_MAX, rho = 0.0f;
        int theta = 1;
        uint32_t nexp = 0;
        if (lead) {
            if (((iter + 1) % kHashReset) == 0) {  // adaptive_search.cuh:128-134
                hash_reset(H, nbk);
                lead_sync<NW>();
                for (int i = lane; i < beam_sz; i += 64) hash_insert(H, nbk, bp[i].y & ~kMsb);
                lead_sync<NW>();
            }
            FG_PHASE(1);
            // The merge runs before the iteration-limit test, so a search stopped
            // by max_iter merges its last candidates here (the reference's final
            // merge, adaptive_search.cuh:447-451).  A search that stops because no
            // beam entry is left to expand has merged them already: its final
            // merge sees an empty candidate buffer and leaves the beam as it is.
            // A search that runs all kMaxIterations iterations (max_iter > 1024,
            // i.e. beam >= 931) leaves the loop without passing here again and
            // merges after it.
            merge_beam<BIG, NW>(P, bp, ms, cd, ci, cand_span, split_fast, lb_merge);
            if constexpr (BIG) scan_from = min(scan_from, lb_merge);
            FG_PHASE(2);
            if (iter >= P.max_iter) {
                team_stop<NW>(tb, lane);
                break;
            }
            for (int i = beam_sz + lane; i < pbeam; i += 64) bp[i] = kEmpty;
            ms[nl] = kEmpty;  // both halves store the same pair: no branch
            lead_sync<NW>();
            kth = FLT_MAX;  // adaptive_search_utils.cuh:25-30
            if (bp[beam_sz - 1].y != kMaxIndex) kth = __uint_as_float(bp[(P.K < beam_sz ? P.K : beam_sz) - 1].x);
            kth = uni(kth);
            controller_step(ctl, uni(bp[0].y), P.phase2_rho);
            theta = ctl.spec;
            rho = ctl.rho;

            // pick_expanders (utils.cuh:752-787): first theta unexpanded entries
            // the picked entries' ids and distances go straight to the parent
            // lists (an unexpanded entry's id has the top bit clear)
            // Beams up to 256: lane l reads entry base + l (64 per step).  Larger
            // beams, where the first unexpanded entry sits about halfway down: 256
            // entries per step, from the first entry that can be unexpanded.
            nexp = 0;
            if constexpr (!BIG) {
                for (int base = 0; base < beam_sz; base += 64) {
                    const int j = base + lane;
                    const uint2 e = bp[j < pbeam ? j : pbeam];  // unconditional read; bp[pbeam] is a sentinel
                    const bool fresh = j < beam_sz && (e.y & kMsb) == 0;
                    const uint64_t m = ballot(fresh);
                    if (fresh) {
                        const uint32_t r = static_cast<uint32_t>(__popcll(m & ((1ull << lane) - 1ull))) + nexp;
                        if (r < static_cast<uint32_t>(theta)) {
                            pnode[r] = e.y;
                            pdist[r] = __uint_as_float(e.x);
                            bp[j].y = e.y | kMsb;
                        }
                    }
                    nexp += static_cast<uint32_t>(__popcll(m));
                    if (nexp >= static_cast<uint32_t>(theta)) {
                        nexp = static_cast<uint32_t>(theta);
                        break;
                    }
                }
            } else {
              int lastj = -1;  // the entry that took rank theta - 1
              for (int base = scan_from; base < beam_sz; base += 256) {
                // entry base + 64 k + l on lane l (each read covers 64
                // consecutive entries); index order is k, then lane
                uint2 e[4];
                uint64_t m[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int j = base + 64 * k + lane;
                    e[k] = bp[j < pbeam ? j : pbeam];  // unconditional read; bp[pbeam] is a sentinel
                    m[k] = ballot(j < beam_sz && (e[k].y & kMsb) == 0);
                }
                const uint64_t lt = (1ull << lane) - 1ull;
                uint32_t before = nexp;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (lane_in(m[k])) {
                        const uint32_t r = before + static_cast<uint32_t>(__popcll(m[k] & lt));
                        if (r < static_cast<uint32_t>(theta)) {
                            const int j = base + 64 * k + lane;
                            pnode[r] = e[k].y;
                            pdist[r] = __uint_as_float(e[k].x);
                            bp[j].y = e[k].y | kMsb;
                            if (r + 1 == static_cast<uint32_t>(theta)) lastj = j;
                        }
                    }
                    before += static_cast<uint32_t>(__popcll(m[k]));
                }
                nexp = before;
                if (nexp >= static_cast<uint32_t>(theta)) {
                    nexp = static_cast<uint32_t>(theta);
                    break;
                }
              }
              // entries up to the last one picked are now all expanded
              const uint64_t bl = ballot(lastj >= 0);
              scan_from = bl ? __builtin_amdgcn_readlane(lastj, __builtin_ctzll(bl)) + 1 : beam_sz;
            }
            lead_sync<NW>();
            if (nexp == 0) {
                team_stop<NW>(tb, lane);
                break;
            }
            FG_COUNT(c_iters++);
            FG_COUNT(c_exp += nexp);
            // adaptive_search_utils.cuh:41-49
            ctl.last_e = finite_below_max(ctl.cur_e) ? ctl.cur_e : ctl.entry_d;
            ctl.cur_e = uni(pdist[nexp - 1]);
        }
        if constexpr (NW > 1) {
            if (lead && lane == 0) {
                tb->stop = 0u;
                tb->theta = static_cast<uint32_t>(theta);
                tb->nexp = nexp;
                tb->kth_bits = __float_as_uint(kth);
                tb->rho_bits = __float_as_uint(rho);
            }
            __syncthreads();
            if (!lead) {
                if (uni(tb->stop) != 0u) break;
                theta = static_cast<int>(uni(tb->theta));
                nexp = uni(tb->nexp);
                kth = __uint_as_float(uni(tb->kth_bits));
                rho = __uint_as_float(uni(tb->rho_bits));
            }
        }
        const bool kth_valid = finite_below_max(kth);
        FG_PHASE(3);

        // children to score exactly, set by either stage (one call site below)
        int ex_n = 0;
        const uint32_t *ex_list = nullptr;
        if (theta <= 1) {
            // (the lead wave's alone; a helper waits for the exact batch)
            if (lead) {
                // ---------------- single expander (adaptive_search.cuh:221-343)
                const int cwc = deg < cbs ? deg : cbs;
                const uint32_t parent = uni(pnode[0]);
                const float pd0 = uni(pdist[0]);
                const float *prow = data + static_cast<uint64_t>(parent) * g.row;
                const uint32_t *nbrs = reinterpret_cast<const uint32_t *>(prow + g.nbr);
                FG_COUNT(c_ids += static_cast<uint32_t>(cwc));
                // id, factors and code issued together (one HBM round trip);
                // unconditional loads, lanes past cwc read the last slot
                const int nsafe = nl < cwc ? nl : cwc - 1;
                const float *factors = prow + g.factor;
                uint32_t ck[1] = {nbrs[nsafe]};
                const float tx = factors[nsafe];
                const float fdq = factors[deg + nsafe];
                const float fvq = factors[2 * deg + nsafe];
                uint32_t c1[1][WTR];
                if constexpr (WT > 0)
                    load_code<WT>(reinterpret_cast<const uint32_t *>(prow + g.code) + static_cast<uint64_t>(nsafe) * WT,
                                  vec_ok, c1[0]);
                bool fresh[1] = {nl < cwc && ck[0] < np32};
                hash_contains_n<1>(H, nbk, ck, fresh);
                uint32_t child = fresh[0] ? ck[0] : kMaxIndex;
                const uint32_t vmask = half_bits(ballot(child != kMaxIndex), 0);
                const int valid_count = __popc(vmask);
                const int keep = keep_count_for_expander(static_cast<uint32_t>(cwc), 1, ctl.rho, false, 0);
                const bool keep_all = keep >= valid_count;
                float dist = child == kMaxIndex ? FLT_MAX : 0.0f;
                uint32_t admit_mask;
                if (!keep_all) {
                    FG_COUNT(c_est += static_cast<uint32_t>(valid_count));
                    const uint32_t *codes = reinterpret_cast<const uint32_t *>(prow + g.code);
                    const bool valid = child != kMaxIndex;
                    float est = FLT_MAX;
                    int32_t r1[1] = {0};
                    if constexpr (WT > 0) {
                        // computed on every lane, selected for the valid ones
                        raw_batch<1, WT>(c1, planes, sflag(any_wrap), sflag(any_zero), r1);
                        est = tx == FLT_MAX ? 0.0f : estimate_formula(r1[0], sum_q, qwidth, qlow, tx, fdq, fvq, pd0);
                    } else if (valid) {
                        const int32_t raw = raw_words(codes + static_cast<uint64_t>(nsafe) * W, planes, W, vec_ok,
                                                      sflag(any_wrap), sflag(any_zero));
                        est = tx == FLT_MAX ? 0.0f : estimate_formula(raw, sum_q, qwidth, qlow, tx, fdq, fvq, pd0);
                    }
                    const bool fin = isfinite(est);
                    child = (valid && !fin) ? kMaxIndex : child;
                    dist = valid ? (fin ? est : FLT_MAX) : dist;
                    uint32_t near = 0;
                    if (kth_valid)
                        near = __popc(half_bits(ballot(child != kMaxIndex && isfinite(dist) && dist <= kth), 0));
                    const int eff = keep_count_for_expander(static_cast<uint32_t>(cwc), 1, ctl.rho, kth_valid, near);
                    // dispatch_candidate_bitonic_sort over the cbs-entry buffer (padding beyond it)
                    float sk = nl < cbs ? dist : FLT_MAX;
                    uint32_t sv = nl < cbs ? child : kMaxIndex;
                    sort32(sk, sv);
                    dist = sk;
                    child = sv;
                    if (nl >= eff) {
                        child = kMaxIndex;
                        dist = FLT_MAX;
                    }
                    admit_mask = eff >= 32 ? 0xFFFFFFFFu : ((1u << eff) - 1u);
                } else {
                    admit_mask = cwc >= 32 ? 0xFFFFFFFFu : ((1u << cwc) - 1u);
                }
                // admit in slot order: insert, drop repeats (lowest slot wins)
                const bool want = ((admit_mask >> nl) & 1u) && child != kMaxIndex && dist < FLT_MAX;
                const uint32_t want_mask = half_bits(ballot(want), 0);
                bool ins = want;
                if (!sflag(static_cast<uint32_t>(P.dup_free))) ins = want && !dup_of_earlier(child, want_mask, nl, 0);
                if (h == 0 && ins) hash_insert(H, nbk, child);
                if (!ins) {
                    if ((admit_mask >> nl) & 1u) {
                        child = kMaxIndex;
                        dist = FLT_MAX;
                    }
                }
                const uint32_t ins_mask = half_bits(ballot(ins), 0);
                if (h == 0) {
                    ms[nl] = make_uint2(__float_as_uint(dist), child);
                    if (ins) alist[__popc(ins_mask & ((1u << nl) - 1u))] = static_cast<uint32_t>(nl);
                }
                lead_sync<NW>();
                const int nins = __popc(ins_mask);
                FG_COUNT(c_exact += static_cast<uint32_t>(nins));
                ex_n = nins;
                ex_list = alist;
                cand_span = 32;  // single-expander children sit at their lane's slot
                FG_PHASE(4);
            }
        } else {
            // ---------------- speculative expansion (adaptive_search.cuh:344-444)
            FG_COUNT(if (c_st2 == kMaxIndex) c_st2 = static_cast<uint32_t>(iter));
            const int tiles = (deg + 31) / 32;
            const int tasks = static_cast<int>(nexp) * tiles;
            // keep limits of a full 32-neighbour tile and of the last,
            // partial one (utils uniform over the iteration)
            const int an_full = deg < 32 ? deg : 32;
            const int an_last = deg - (tiles - 1) * 32;
            const int lim_full = uni(keep_limit(static_cast<uint32_t>(an_full), theta, rho));
            const int lim_last = an_last == an_full ? lim_full : uni(keep_limit(static_cast<uint32_t>(an_last), theta, rho));
            uint32_t compact = 0;
            // A task (one 32-neighbour tile of one parent: one reference warp)
            // takes G lanes: a 32-lane half, or for degree 16 a 16-lane row, so
            // a wave runs TPW tasks at once; lane order is task order.
            constexpr int G = DEG_T == 16 ? 16 : 32;
            constexpr int TPW = 64 / G;
            const int grp = lane / G, nlg = lane % G;
            for (int rbase = 0; rbase < tasks; rbase += kSearchWidth) {
                constexpr int SR = kSearchWidth / TPW;  // sub-rounds of TPW tasks
                // this wave's sub-rounds: all of them, or in the team form
                // the first half (lead) or the second (helper)
                constexpr int SRN = SR / NW;
                const int sr0 = wv * SRN;
                uint32_t cid[SRN];
                bool val[SRN];
                int an[SRN], tsk[SRN], pix[SRN];
                const float *prw[SRN];
                uint32_t rof[SRN];  // fixed geometry: the parents' row byte offsets
                float tx[SRN], fdq[SRN], fvq[SRN];
                uint32_t code[SRN][WTR];
                // (a) neighbour ids of the round's 8 tasks, then their factors and
                // codes: all loads issued together (one HBM round trip), ids first
                // so the visited test can start when they arrive.  Loads are
                // unconditional (an inactive lane reads a valid slot of parent 0
                // or of its own parent's last neighbour); inactive lanes' ids are
                // replaced after.
                bool lact[SRN];
                int nsafe[SRN];
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr) {
                    const int task = rbase + TPW * (sr0 + sr) + grp;
                    const bool tact = task < tasks;
                    const int pidx = tact ? task / tiles : 0;
                    const int tile = tact ? task - pidx * tiles : 0;
                    const int nidx = tile * 32 + nlg;
                    lact[sr] = tact && nidx < deg;
                    nsafe[sr] = nidx < deg ? nidx : deg - 1;
                    tsk[sr] = tact ? tile * 32 : -1;
                    pix[sr] = pidx;
                    if constexpr (kFixedGeo) {
                        rof[sr] = __umul24(pnode[pidx], Geo<DIM_T, DEG_T>::kRowB);
                        cid[sr] = ld_at<uint32_t>(data, rof[sr] + Geo<DIM_T, DEG_T>::kNbrB + 4u * nsafe[sr]);
                    } else {
                        prw[sr] = data + static_cast<uint64_t>(pnode[pidx]) * g.row;
                        cid[sr] = reinterpret_cast<const uint32_t *>(prw[sr] + g.nbr)[nsafe[sr]];
                    }
                    int a = tact ? deg - tile * 32 : 0;
                    an[sr] = a > 32 ? 32 : a;
                    FG_COUNT(c_ids += static_cast<uint32_t>(__popcll(ballot(lact[sr]))));
                }
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr) {
                    if constexpr (kFixedGeo) {
                        using GF = Geo<DIM_T, DEG_T>;
                        const uint32_t fo = rof[sr] + GF::kFactorB + 4u * nsafe[sr];
                        tx[sr] = ld_at<float>(data, fo);
                        fdq[sr] = ld_at<float>(data, fo + 4u * DEG_T);
                        fvq[sr] = ld_at<float>(data, fo + 8u * DEG_T);
                        const uint32_t co = rof[sr] + GF::kCodeB + 4u * WT * nsafe[sr];
                        if constexpr (WT == 4) {
                            // 16-byte aligned: the fixed rows and code blocks are multiples of 16 bytes
                            const uint4 c4 = ld_at<uint4>(data, co);
                            code[sr][0] = c4.x;
                            code[sr][1] = c4.y;
                            code[sr][2] = c4.z;
                            code[sr][3] = c4.w;
                        } else {
#pragma unroll
                            for (int w = 0; w < WTR; ++w) code[sr][w] = ld_at<uint32_t>(data, co + 4u * w);
                        }
                    } else {
                        const float *factors = prw[sr] + g.factor;
                        tx[sr] = factors[nsafe[sr]];
                        fdq[sr] = factors[deg + nsafe[sr]];
                        fvq[sr] = factors[2 * deg + nsafe[sr]];
                        if constexpr (WT > 0)
                            load_code<WT>(reinterpret_cast<const uint32_t *>(prw[sr] + g.code) +
                                              static_cast<uint64_t>(nsafe[sr]) * WT,
                                          vec_ok, code[sr]);
                    }
                }
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr)
                    if (!lact[sr]) cid[sr] = kMaxIndex;
                // (b) visited test against the table as it stood at the round's start
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr) val[sr] = cid[sr] != kMaxIndex && cid[sr] < np32;
                hash_contains_n<SRN>(H, nbk, cid, val);
                // (c) which tasks need estimates.  Lane predicates from here on
                // are masks taken straight from compares.  A task without
                // children has no valid lane, so it never needs estimates and
                // its keep limit is never read.
                uint64_t valm[SRN], needm[SRN];
                int keep[SRN];
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr) {
                    valm[sr] = ballot(val[sr]);
                    const int rvc = static_cast<int>(group_popc<G>(valm[sr]));
                    keep[sr] = an[sr] == an_full ? lim_full : lim_last;
                    needm[sr] = ballot(keep[sr] < rvc);
                    FG_COUNT(c_est += static_cast<uint32_t>(__popcll(needm[sr] & valm[sr])));
                }
                FG_PHASE(6);
                // (d) estimates, kth-near counts, keep decisions
                uint64_t klm[SRN];
                int32_t rawb[SRN];
                if constexpr (WT > 0) raw_batch<SRN, WT>(code, planes, sflag(any_wrap), sflag(any_zero), rawb);
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr) {
                    float est = FLT_MAX;
                    const uint64_t scored = needm[sr] & valm[sr];
                    if constexpr (WT > 0) {
                        // computed on every lane and selected (most lanes need it;
                        // a branch would cost more than the few wasted lanes)
                        const float e = estimate_formula(rawb[sr], sum_q, qwidth, qlow, tx[sr], fdq[sr], fvq[sr],
                                                         pdist[pix[sr]]);
                        est = (lane_in(scored) && tx[sr] != FLT_MAX) ? e : FLT_MAX;
                    } else if (lane_in(scored) && tx[sr] != FLT_MAX) {
                        const int nidx = tsk[sr] + nlg;
                        const int32_t raw = raw_words(reinterpret_cast<const uint32_t *>(prw[sr] + g.code) +
                                                          static_cast<uint64_t>(nidx) * W,
                                                      planes, W, vec_ok, sflag(any_wrap), sflag(any_zero));
                        est = estimate_formula(raw, sum_q, qwidth, qlow, tx[sr], fdq[sr], fvq[sr], pdist[pix[sr]]);
                    }
                    // a scored child with a non-finite estimate is dropped
                    // (finiteness as an integer compare on opaque bits, which
                    // the ballot takes as it is; a float class test would pass
                    // through a vector register on its way to the mask)
                    uint32_t eb = __float_as_uint(est);
                    asm volatile("" : "+v"(eb));
                    const uint64_t finm = ballot((eb & 0x7F800000u) != 0x7F800000u);
                    valm[sr] = (valm[sr] & ~scored) | (scored & finm);
                    uint64_t kl = valm[sr];
                    if (needm[sr] != 0ull) {
                        const uint64_t belowm = kth_valid ? (valm[sr] & ballot(est <= kth)) : 0ull;
                        const uint32_t near = group_popc<G>(belowm);
                        const int kp = keep[sr];
                        const bool nd = lane_in(needm[sr]);
                        const int eff = nd ? keep_with_cutoff(kp, kth_valid, near) : kp;
                        // With a valid cutoff and 1 <= near <= keep the count is
                        // near, and the near smallest (value, lane) pairs are the
                        // ones at or below the cutoff: every such lane ranks
                        // ahead of every lane above it.  No selection rounds.
                        const uint64_t cutm =
                            kth_valid ? (needm[sr] & ballot(near >= 1u) & ballot(static_cast<int>(near) <= kp)) : 0ull;
                        const int rounds = (nd && !lane_in(cutm)) ? eff : 0;
                        // uniform within each group: the largest over the groups' first lanes
                        int maxk = max(__builtin_amdgcn_readlane(rounds, 0), __builtin_amdgcn_readlane(rounds, 32));
                        if constexpr (G == 16)
                            maxk = max(maxk, max(__builtin_amdgcn_readlane(rounds, 16), __builtin_amdgcn_readlane(rounds, 48)));
                        const uint64_t selm = select_smallest<G>(est, valm[sr], eff, maxk);
                        const uint64_t effm = ballot(eff > 0);
                        kl = (valm[sr] & ~needm[sr]) | (needm[sr] & valm[sr] & effm & ((cutm & belowm) | (selm & ~cutm)));
                    }
                    klm[sr] = kl;
                }
                // the kept lanes of all sub-rounds; in the team form the
                // helper's half reaches the lead wave through LDS
                uint64_t klmA[SR];
                uint32_t cidA[SR];
#pragma unroll
                for (int sr = 0; sr < SRN; ++sr) {
                    klmA[sr] = klm[sr];
                    cidA[sr] = cid[sr];
                }
                if constexpr (NW > 1) {
                    if (!lead) {
#pragma unroll
                        for (int sr = 0; sr < SRN; ++sr) {
                            if (lane == 0) tb->klm[sr] = klm[sr];
                            tb->cid[sr][lane] = cid[sr];
                        }
                    }
                    __syncthreads();
                    if (lead) {
#pragma unroll
                        for (int sr = 0; sr < SRN; ++sr) {
                            const uint64_t m = tb->klm[sr];
                            klmA[SRN + sr] = (static_cast<uint64_t>(uni(static_cast<uint32_t>(m >> 32))) << 32) |
                                             uni(static_cast<uint32_t>(m));
                            cidA[SRN + sr] = tb->cid[sr][lane];
                        }
                    }
                }
                if (lead) {
                    // (e) kept children listed in (task, lane) order
                    uint32_t total = 0;
#pragma unroll
                    for (int sr = 0; sr < SR; ++sr) {
                        // the sub-round's TPW tasks sit in lane order and follow
                        // each other in the list: a kept lane's place is the running
                        // total plus its rank among the kept lanes of the wave
                        if (lane_in(klmA[sr])) {
                            const uint32_t e = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(klmA[sr] >> 32),
                                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(klmA[sr]), total));
                            if (e < 32) alist[e] = cidA[sr];
                        }
                        total += static_cast<uint32_t>(__popcll(klmA[sr]));
                    }
                    lead_sync<NW>();
                    if (total > 32) total = 32;  // <= 4 kept per task at theta = 8
                    // (f) insert in list order; a repeat of an earlier entry is dropped
                    const bool mine = lane < static_cast<int>(total);
                    const uint32_t key = mine ? alist[lane] : kMaxIndex;
                    const uint32_t got = mine ? hash_insert(H, nbk, key) : 0u;
                    // Every listed child was absent from the table when this
                    // round's visited tests ran, so an insert that finds its key
                    // present met a repeat within the list, added by another lane
                    // of this batch: of each such group the earliest lane is kept.
                    bool acc = got != 0u;
                    uint64_t lost = ballot(mine && !got);
                    while (lost != 0ull) {
                        const uint32_t kr = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), __builtin_ctzll(lost)));
                        const uint64_t same = ballot(mine && key == kr);
                        acc = lane_in(same) ? (lane == __builtin_ctzll(same)) : acc;
                        lost &= ~same;
                    }
                    const uint32_t accm = half_bits(ballot(acc), 0);
                    if (acc) {
                        // (the distance was reset at the iteration's start; the exact pass fills it)
                        const uint32_t slot = __builtin_amdgcn_mbcnt_lo(accm, compact);
                        if (slot < static_cast<uint32_t>(P.collect_cap)) ci[2 * slot] = key;
                    }
                    compact += static_cast<uint32_t>(__popc(accm));
                    lead_sync<NW>();
                }
                // in the team form the round's inserts are in the table before
                // the helper's visited tests of the next round
                if constexpr (NW > 1) {
                    if (rbase + kSearchWidth < tasks) __syncthreads();
                }
            }
            if (lead) {
                if (compact > static_cast<uint32_t>(P.collect_cap)) compact = static_cast<uint32_t>(P.collect_cap);
                FG_COUNT(c_exact += compact);
                ex_n = static_cast<int>(compact);
                cand_span = ex_n;  // compacted into slots 0 .. compact - 1
            }
            FG_PHASE(7);
        }
        if constexpr (NW == 1) {
            exact_batch<DPL>(P, g, ex_n, ex_list, cd, ci, qr, qsrc);
        } else {
            // the exact batch in two halves, one per wave
            if (lead && lane == 0) {
                tb->ex_n = static_cast<uint32_t>(ex_n);
                tb->ex_alist = ex_list != nullptr ? 1u : 0u;
            }
            __syncthreads();
            const int n_all = static_cast<int>(uni(tb->ex_n));
            const uint32_t *lst = uni(tb->ex_alist) != 0u ? alist : nullptr;
            const int mid = (n_all + 1) >> 1;
            exact_batch_range<DPL>(P, g, lead ? 0 : mid, lead ? mid : n_all, lst, cd, ci, qr, qsrc);
            __syncthreads();
        }
        if (theta <= 1) FG_PHASE(5);
        else FG_PHASE(8);
        lead_sync<NW>();
    }
    if constexpr (NW > 1) {
        // the helper's work counters; from here on the lead wave is alone
        if (!lead && lane == 0) {
            tb->c_ids = c_ids;
            tb->c_est = c_est;
        }
        __syncthreads();
        if (!lead) return;
        if constexpr (COUNT) {
            c_ids += uni(tb->c_ids);
            c_est += uni(tb->c_est);
        }
    }
    if constexpr (kSliceable) {
        if (P.slice_suspend > 0) {
            uint32_t *st = P.slice_state + kSliceHeader + static_cast<uint64_t>(qid) * slice_words(pbeam, B);
            if (suspended) {
                // the state the next slice resumes from; the ordering key is the
                // best distance found so far (the larger, the longer the rest of
                // the search tends to run)
                uint2 *sb = reinterpret_cast<uint2 *>(st + kSliceFixed);
                const float kd = pair_key(bp[0]);
                for (int i = lane; i < pbeam + 32; i += 64) sb[i] = i < pbeam ? bp[i] : ms[i - pbeam];
                uint32_t *sp = st + slice_prep_offset(pbeam);
                for (int i = lane; i < 8 * W; i += 64) sp[4 + i] = planes[i];
                if (lane == 0) {
                    sp[0] = __float_as_uint(qlow);
                    sp[1] = __float_as_uint(qwidth);
                    sp[2] = static_cast<uint32_t>(sum_q);
                    sp[3] = 0u;
                    const uint32_t key = slice_key(kd);
                    P.slice_keys[qid] = key;
                    st[0] = 1u;
                    st[1] = key;
                    st[2] = static_cast<uint32_t>(ctl.spec);
                    st[3] = __float_as_uint(ctl.rho);
                    st[4] = static_cast<uint32_t>(ctl.policy_iters);
                    st[5] = ctl.top1;
                    st[6] = static_cast<uint32_t>(ctl.stall);
                    st[7] = ctl.warm ? 1u : 0u;
                    st[8] = __float_as_uint(ctl.entry_d);
                    st[9] = __float_as_uint(ctl.last_e);
                    st[10] = __float_as_uint(ctl.cur_e);
                    st[11] = c_iters;
                    st[12] = c_exp;
                    st[13] = c_ids;
                    st[14] = c_est;
                    st[15] = c_exact;
                    st[16] = c_st2;
                    st[17] = static_cast<uint32_t>(cand_span);
                    st[18] = split_fast ? 1u : 0u;
                    st[19] = static_cast<uint32_t>(scan_from);
                }
                return;
            }
            if (lane == 0) P.slice_keys[qid] = kSliceDone;  // finished within this slice
        }
    }
    // the loop ran out at kMaxIterations: the last iteration's exact-scored
    // candidates are still in the buffer (adaptive_search.cuh:449-451)
    if (iter == kMaxIterations) merge_beam<BIG, NW>(P, bp, ms, cd, ci, cand_span, split_fast, lb_merge);

    FG_PHASE(3);
    // result writer (adaptive_search.cuh:455-464)
    for (int i = lane; i < P.K; i += 64) {
        const uint32_t r = i < beam_sz ? (bp[i].y & 0x7fffffffu) : (bp[beam_sz - 1].y & 0x7fffffffu);
        P.results[static_cast<uint64_t>(qid) * P.K + i] = r;
    }
    FG_PHASE(9);
    if constexpr (PROF) {
        const unsigned long long t_end = __builtin_amdgcn_s_memrealtime();
        unsigned long long *out = P.phase + static_cast<uint64_t>(qid) * FG_PROFILE_SLOTS;
        if (lane < 10) out[lane] = prof[lane];
        if (lane == 10) out[lane] = t_begin;
        if (lane == 11) out[lane] = t_end;
    }
    if (COUNT && P.counters && lane == 0) {
        uint32_t *c = P.counters + static_cast<uint64_t>(qid) * FG_COUNTERS_PER_QUERY;
        c[0] = c_iters;
        c[1] = c_exp;
        c[2] = c_ids;
        c[3] = c_est;
        c[4] = c_exact;
        c[5] = c_st2;
    }
}

// Whether a launch runs the team form: when the batch is too small to fill
// the device with one wave per query (twice the queries fit in the
// one-wave form's resident workgroups), a second wave per query costs no
// query a slot and shortens every search.  FLASHGANN_TEAM=0 / 1 forces the
// one-wave / team form (tests run both).
// Workgroups of the one-wave kernel the device holds at once (0 if unknown).
inline long long resident_one_wave(const SearchParams &P, const void *one_wave_kernel) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, one_wave_kernel, 64, P.lds.total) != hipSuccess) return 0;
    return static_cast<long long>(per_cu) * cus;
}

inline bool use_team(const SearchParams &P, const void *one_wave_kernel) {
    if (!P.team) return false;
    if (const char *e = std::getenv("FLASHGANN_TEAM")) {
        if (e[0] == '0') return false;
        if (e[0] == '1') return true;
    }
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, one_wave_kernel, 64, P.lds.total) != hipSuccess)
        return false;
    return 2ll * P.nq <= static_cast<long long>(per_cu) * cus;
}

template <int WT, int DPL, int DIM_T, int DEG_T, bool BIG>
void launch_geo_b(const SearchParams &P, hipStream_t stream, bool count, bool prof, int *waves_only, bool one_wave,
                  long long *resident) {
    const dim3 grid(P.nq), block(64);
    const void *one = reinterpret_cast<const void *>(&fg_search_kernel<WT, DPL, DIM_T, DEG_T, false, false, BIG, 1>);
    const bool team = !one_wave && use_team(P, one);
    if (waves_only) {  // the form only, no launch
        *waves_only = team ? 2 : 1;
        if (resident) *resident = resident_one_wave(P, one);
        return;
    }
    if (team) {
        const dim3 team_block(128);
        if (prof)
            hipLaunchKernelGGL((fg_search_kernel<WT, DPL, DIM_T, DEG_T, false, true, BIG, 2>), grid, team_block,
                               P.lds.total_team, stream, P);
        else if (count)
            hipLaunchKernelGGL((fg_search_kernel<WT, DPL, DIM_T, DEG_T, true, false, BIG, 2>), grid, team_block,
                               P.lds.total_team, stream, P);
        else
            hipLaunchKernelGGL((fg_search_kernel<WT, DPL, DIM_T, DEG_T, false, false, BIG, 2>), grid, team_block,
                               P.lds.total_team, stream, P);
        return;
    }
    if (prof)
        hipLaunchKernelGGL((fg_search_kernel<WT, DPL, DIM_T, DEG_T, false, true, BIG, 1>), grid, block,
                           P.lds.total_prof, stream, P);
    else if (count)
        hipLaunchKernelGGL((fg_search_kernel<WT, DPL, DIM_T, DEG_T, true, false, BIG, 1>), grid, block, P.lds.total,
                           stream, P);
    else
        hipLaunchKernelGGL((fg_search_kernel<WT, DPL, DIM_T, DEG_T, false, false, BIG, 1>), grid, block, P.lds.total,
                           stream, P);
}

// Beams over 256 (two or more merge-path segments per lane, the pick's wide
// scan) and smaller ones run separately compiled kernels.
template <int WT, int DPL, int DIM_T, int DEG_T>
void launch_geo(const SearchParams &P, hipStream_t stream, bool count, bool prof, int *waves_only, bool one_wave,
                long long *resident) {
    if (P.pbeam > 256) launch_geo_b<WT, DPL, DIM_T, DEG_T, true>(P, stream, count, prof, waves_only, one_wave, resident);
    else launch_geo_b<WT, DPL, DIM_T, DEG_T, false>(P, stream, count, prof, waves_only, one_wave, resident);
}

// Launch functions of the shape classes, one translation unit each
// (fg_shapes.hip with FG_SHAPE = 0 .. 6): d 128 / degree 32, d 96 / degree
// 32, d 96 / degree 16 (compile-time geometry), then the runtime-geometry
// kernels for padded dimension 64, 128 with d <= 96, 128, and >= 256.
using LaunchShape = void (*)(const SearchParams &, hipStream_t, bool count, bool prof, int *waves_only,
                             bool one_wave, long long *resident);
void launch_shape0(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);
void launch_shape1(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);
void launch_shape2(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);
void launch_shape3(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);
void launch_shape4(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);
void launch_shape5(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);
void launch_shape6(const SearchParams &, hipStream_t, bool, bool, int *, bool, long long *);

}  // namespace fgk
