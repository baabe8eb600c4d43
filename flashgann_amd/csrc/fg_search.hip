// fg_search.hip -- adaptive graph beam search for MI355X (gfx950, wave64).
//
// The search path of the reference (src/adaptive_search.cuh:5-466 with the
// primitives of include/utils.cuh and src/adaptive_search_utils.cuh) rebuilt
// around one 64-lane wavefront per query:
//   * one workgroup = one wave = one query; the reference's 256-thread block
//     barriers become wave-ordered LDS traffic, so the beam, candidate buffer,
//     visited table and controller state never leave the CU's LDS/registers
//     (a launch too small to fill the device runs the team form instead: a
//     second wave per query takes half of the expansion rounds and of the
//     exact distances);
//   * the reference's 32-lane sorting networks are data-oblivious, so the
//     same compare-exchange sequence is replayed on the wave (two 32-lane
//     halves, or 1-2 positions per lane) and ties resolve identically;
//   * RaBitQ scores come from 6 popcount bit-planes of the quantized query
//     minus one, held in LDS (raw = popcount(code) + sum_p 2^p
//     popcount(code & plane_p)), corrected for the reference's uint8 LUT wrap,
//     instead of per-nibble LUT gathers;
//   * exact distances keep the reference's per-lane accumulation order and
//     reduction tree, so results are bitwise equal to the 32-lane original.
// Determinism: where the reference races (concurrent inserts of one child by
// two warps in the speculative path), this kernel fixes "every task of a round
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

#include "fg_kernel.hpp"

using namespace fgk;

namespace {

// Order of the second slice: the suspended queries sorted by key, largest
// first: a counting sort over kSliceBins bins spread linearly over [smallest
// key, largest key] (keys are finite floats of either sign; within a bin the
// order is arbitrary).  Writes the count of suspended queries to
// slice_state[0] and the queries to order[0 .. count).
//
// Up to kSliceMaxQueries queries: one workgroup does it all.
__device__ __forceinline__ uint32_t slice_bin(uint32_t key_bits, float kmin, double scale) {
    const double x = (static_cast<double>(__uint_as_float(key_bits)) - static_cast<double>(kmin)) * scale;
    const int b = x >= static_cast<double>(kSliceBins - 1) ? kSliceBins - 1 : (x > 0.0 ? static_cast<int>(x) : 0);
    return static_cast<uint32_t>(kSliceBins - 1 - b);  // largest key first
}

__device__ __forceinline__ double slice_scale(uint32_t omin, uint32_t omax) {
    const float kmin = __uint_as_float(key_from_order_bits(omin)), kmax = __uint_as_float(key_from_order_bits(omax));
    const double range = static_cast<double>(kmax) - static_cast<double>(kmin);
    return range > 0.0 ? static_cast<double>(kSliceBins - 1) / range : 0.0;
}

// (xor distances 32 .. 1 written out: each is a different cross-lane move)
__device__ __forceinline__ uint32_t wave_umin(uint32_t v) {
    v = min(v, xshfl(v, 32));
    v = min(v, xshfl(v, 16));
    v = min(v, xshfl(v, 8));
    v = min(v, xshfl(v, 4));
    v = min(v, xshfl(v, 2));
    return min(v, xshfl(v, 1));
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
    v = max(v, xshfl(v, 32));
    v = max(v, xshfl(v, 16));
    v = max(v, xshfl(v, 8));
    v = max(v, xshfl(v, 4));
    v = max(v, xshfl(v, 2));
    return max(v, xshfl(v, 1));
}

// Exclusive scan of the kSliceBins counts in[] into out[] (in == out allowed)
// by a workgroup of 1024 threads, four consecutive bins per thread: a scan
// within each wave by shuffles, then each wave adds the totals of the waves
// before it (wsum: 16 words of LDS).  Returns the sum of all bins.
__device__ __forceinline__ uint32_t block_scan_bins(const uint32_t *in, uint32_t *out, uint32_t *wsum) {
    constexpr int kPer = kSliceBins / 1024;
    const int t = static_cast<int>(threadIdx.x), lane = t & 63, w = t >> 6;
    uint32_t loc[kPer], sum = 0u;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        loc[j] = sum;
        sum += in[t * kPer + j];
    }
    uint32_t inc = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t x = __shfl_up(inc, d);
        if (lane >= d) inc += x;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    uint32_t base = inc - sum, total = 0u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t x = wsum[i];
        base += i < w ? x : 0u;
        total += x;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) out[t * kPer + j] = base + loc[j];
    return total;
}

__global__ __launch_bounds__(1024) void fg_slice_order_kernel(uint32_t *state, const uint32_t *keys, int nq,
                                                             uint32_t *order) {
    constexpr int kPerThread = kSliceMaxQueries / 1024;
    __shared__ uint32_t hist[kSliceBins];
    __shared__ uint32_t wlo[16], whi[16], wsum[16];
    const int t = static_cast<int>(threadIdx.x), lane = t & 63, w = t >> 6;
    for (int b = t; b < kSliceBins; b += 1024) hist[b] = 0u;
    // every key this thread handles, loaded at once (query t + 1024 j)
    uint32_t v[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int q = t + 1024 * j;
        v[j] = q < nq ? keys[q] : kSliceDone;
    }
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j)
        if (v[j] != kSliceDone) {
            const uint32_t o = key_order_bits(v[j]);
            lo = min(lo, o);
            hi = max(hi, o);
        }
    lo = wave_umin(lo);
    hi = wave_umax(hi);
    if (lane == 0) {
        wlo[w] = lo;
        whi[w] = hi;
    }
    __syncthreads();
    uint32_t omin = wlo[0], omax = whi[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        omin = min(omin, wlo[i]);
        omax = max(omax, whi[i]);
    }
    const float kmin = __uint_as_float(key_from_order_bits(omin));
    const double scale = slice_scale(omin, omax);
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        if (v[j] != kSliceDone) {
            v[j] = slice_bin(v[j], kmin, scale);
            atomicAdd(&hist[v[j]], 1u);
        }
    }
    __syncthreads();
    const uint32_t total = block_scan_bins(hist, hist, wsum);
    if (t == 0) state[0] = total;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPerThread; ++j)
        if (v[j] != kSliceDone) order[atomicAdd(&hist[v[j]], 1u)] = static_cast<uint32_t>(t + 1024 * j);
}

// More queries: four steps over chunks of kSliceChunk queries, one workgroup
// of 256 threads per chunk, through a work area of (2 + kSliceBins) words plus
// two words per chunk and one per query:
//   minmax  each chunk's smallest and largest key (order-preserving bits);
//           the workgroups also clear the global histogram
//   hist    every workgroup reduces the chunks' extremes, bins its keys
//           (kept per query) and adds its chunk's histogram to the global one
//   scan    one workgroup: exclusive scan of the global histogram, the count
//   scatter each suspended query takes the next place of its bin
constexpr int kSliceChunk = 4096;

__global__ __launch_bounds__(256) void fg_slice_minmax_kernel(const uint32_t *keys, int nq, uint32_t *ext,
                                                              uint32_t *ghist, int nchunks) {
    __shared__ uint32_t lo_s, hi_s;
    const int t = static_cast<int>(threadIdx.x), c = static_cast<int>(blockIdx.x);
    for (int b = c * 256 + t; b < kSliceBins; b += nchunks * 256) ghist[b] = 0u;
    if (t == 0) {
        lo_s = 0xFFFFFFFFu;
        hi_s = 0u;
    }
    __syncthreads();
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    const int q1 = min(nq, (c + 1) * kSliceChunk);
    for (int q = c * kSliceChunk + t; q < q1; q += 256) {
        const uint32_t k = keys[q];
        if (k != kSliceDone) {
            const uint32_t o = key_order_bits(k);
            lo = min(lo, o);
            hi = max(hi, o);
        }
    }
    lo = wave_umin(lo);
    hi = wave_umax(hi);
    if ((t & 63) == 0 && hi >= lo) {
        atomicMin(&lo_s, lo);
        atomicMax(&hi_s, hi);
    }
    __syncthreads();
    if (t == 0) {
        ext[2 * c] = lo_s;
        ext[2 * c + 1] = hi_s;
    }
}

__global__ __launch_bounds__(256) void fg_slice_hist_kernel(const uint32_t *keys, int nq, const uint32_t *ext,
                                                            int nchunks, uint32_t *ghist, uint32_t *qbin) {
    __shared__ uint32_t hist[kSliceBins];
    __shared__ uint32_t lo_s, hi_s;
    const int t = static_cast<int>(threadIdx.x), c = static_cast<int>(blockIdx.x);
    for (int b = t; b < kSliceBins; b += 256) hist[b] = 0u;
    if (t == 0) {
        lo_s = 0xFFFFFFFFu;
        hi_s = 0u;
    }
    __syncthreads();
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    for (int j = t; j < nchunks; j += 256) {
        lo = min(lo, ext[2 * j]);
        hi = max(hi, ext[2 * j + 1]);
    }
    lo = wave_umin(lo);
    hi = wave_umax(hi);
    if ((t & 63) == 0) {
        atomicMin(&lo_s, lo);
        atomicMax(&hi_s, hi);
    }
    __syncthreads();
    const float kmin = __uint_as_float(key_from_order_bits(lo_s));
    const double scale = hi_s >= lo_s ? slice_scale(lo_s, hi_s) : 0.0;
    const int q1 = min(nq, (c + 1) * kSliceChunk);
    for (int q = c * kSliceChunk + t; q < q1; q += 256) {
        const uint32_t k = keys[q];
        uint32_t b = kSliceDone;
        if (k != kSliceDone) {
            b = slice_bin(k, kmin, scale);
            atomicAdd(&hist[b], 1u);
        }
        qbin[q] = b;
    }
    __syncthreads();
    for (int b = t; b < kSliceBins; b += 256)
        if (hist[b]) atomicAdd(&ghist[b], hist[b]);
}

__global__ __launch_bounds__(1024) void fg_slice_scan_kernel(uint32_t *ghist, uint32_t *state) {
    __shared__ uint32_t wsum[16];
    const uint32_t total = block_scan_bins(ghist, ghist, wsum);
    if (threadIdx.x == 0) state[0] = total;
}

__global__ __launch_bounds__(256) void fg_slice_scatter_kernel(const uint32_t *qbin, int nq, uint32_t *goff,
                                                               uint32_t *order) {
    const int q = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (q >= nq) return;
    const uint32_t b = qbin[q];
    if (b != kSliceDone) order[atomicAdd(&goff[b], 1u)] = static_cast<uint32_t>(q);
}

// ------------------------------------------------------------ test-hook kernels

__global__ __launch_bounds__(64) void fg_prepare_kernel(const float *queries, const float *signs, int dim, int B,
                                                        int nq, float *rotated, uint8_t *quant, float *lhw,
                                                        int32_t *sumq, uint32_t scratch_off) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int qid = blockIdx.x;
    if (qid >= nq) return;
    float *rot = reinterpret_cast<float *>(smem);
    uint32_t *planes = reinterpret_cast<uint32_t *>(smem + scratch_off);
    float lo, hi, w;
    int s;
    prepare_query(queries + static_cast<uint64_t>(qid) * dim, signs, dim, B, rot, nullptr, planes, lo, hi, w, s,
                  quant + static_cast<uint64_t>(qid) * B);
    for (int i = lane_id(); i < B; i += 64) rotated[static_cast<uint64_t>(qid) * B + i] = rot[i];
    if (lane_id() == 0) {
        lhw[3 * qid] = lo;
        lhw[3 * qid + 1] = hi;
        lhw[3 * qid + 2] = w;
        sumq[qid] = s;
    }
}

struct ScoreParams {
    const float *data, *signs, *queries;
    const uint32_t *qix, *parents, *slots;
    float *est_lanes, *est_seq, *exact;
    uint64_t row_offset, code_offset, factor_offset, npoints;
    int dim, B, deg, use_ip;
    uint32_t n;
    uint32_t plane_off, query_off;
};

// One workgroup per scored edge: prepares the query, then evaluates both
// estimator variants and the exact distance of the neighbour in `slot`.
__global__ __launch_bounds__(64) void fg_score_kernel(ScoreParams S) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t e = blockIdx.x;
    if (e >= S.n) return;
    const int lane = lane_id();
    const int nl = lane & 31, h = lane >> 5;
    float *rot = reinterpret_cast<float *>(smem);
    float *qv = reinterpret_cast<float *>(smem + S.query_off);
    uint32_t *planes = reinterpret_cast<uint32_t *>(smem + S.plane_off);
    float lo, hi, w;
    int sq;
    prepare_query(S.queries + static_cast<uint64_t>(S.qix[e]) * S.dim, S.signs, S.dim, S.B, rot, qv, planes, lo, hi,
                  w, sq, nullptr);
    const uint32_t parent = S.parents[e];
    const int slot = static_cast<int>(S.slots[e]);
    const float *prow = S.data + static_cast<uint64_t>(parent) * S.row_offset;
    const float pd = uni(half_distance(prow, qv, S.dim, nl, S.use_ip != 0, true));
    const int W = S.B >> 5;
    const uint32_t *code = reinterpret_cast<const uint32_t *>(prow + S.code_offset) + static_cast<uint64_t>(slot) * W;
    const float *f = prow + S.factor_offset;
    const float tx = f[slot], fdq = f[S.deg + slot], fvq = f[2 * S.deg + slot];
    // both halves split the words (theta == 1 layout) and one lane does all
    // words (theta > 1 layout): the integer sums must agree.
    const int hw = W >> 1;
    const int32_t part = raw_partial(code, h * hw, (h + 1) * hw, planes, W);
    const int32_t raw_split = add32i(part);
    // the search kernel's own routines: raw_batch for padded dimensions 64 and
    // 128 (W = 2, 4; the fixed geometries), raw_words for W >= 8
    const bool vec_ok = S.row_offset % 4 == 0 && S.code_offset % 4 == 0;
    uint32_t wor = 0, zor = 0;
    for (int w = 0; w < W; ++w) {
        wor |= planes[kWrapPlane * W + w];
        zor |= planes[kZeroPlane * W + w];
    }
    const bool any_wrap = uni(wor) != 0u, any_zero = uni(zor) != 0u;
    int32_t raw_full;
    if (W == 4 || W == 2) {
        int32_t r[1];
        if (W == 4) {
            uint32_t c[1][4];
            load_code<4>(code, vec_ok, c[0]);
            raw_batch<1, 4>(c, planes, any_wrap, any_zero, r);
        } else {
            uint32_t c[1][2];
            load_code<2>(code, vec_ok, c[0]);
            raw_batch<1, 2>(c, planes, any_wrap, any_zero, r);
        }
        raw_full = r[0];
    } else {
        raw_full = raw_words(code, planes, W, vec_ok, any_wrap, any_zero);
    }
    const float el = tx == FLT_MAX ? 0.0f : estimate_formula(raw_split, sq, w, lo, tx, fdq, fvq, pd);
    const float es = tx == FLT_MAX ? FLT_MAX : estimate_formula(raw_full, sq, w, lo, tx, fdq, fvq, pd);
    const uint32_t child = reinterpret_cast<const uint32_t *>(prow + (S.factor_offset + 3 * S.deg))[slot];
    const bool child_ok = child < S.npoints;
    const float ex = uni(half_distance(S.data + static_cast<uint64_t>(child_ok ? child : 0u) * S.row_offset, qv,
                                       S.dim, nl, S.use_ip != 0, child_ok));
    if (lane == 0) {
        if (S.est_lanes) S.est_lanes[e] = el;
        if (S.est_seq) S.est_seq[e] = es;
        if (S.exact) S.exact[e] = ex;
    }
}

}  // namespace

// ================================================================== host side

// Staging area of fg_search_noalloc: the device copies of one call's queries,
// result ids and counters, at 256-byte aligned offsets.  Each device holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: its device address comes from
// hipGetSymbolAddress (noalloc_staging), and only that address is passed to
// kernels and copies.
static __device__ __align__(256) unsigned char scratch[FG_NOALLOC_STAGING_BYTES];

struct fg_index {
    int device = 0;
    float *d_rows = nullptr;
    float *d_signs = nullptr;
    uint64_t npoints = 0;
    uint32_t dim = 0, padded_dim = 0, degree = 0, entry = 0;
    uint64_t code_offset = 0, factor_offset = 0, neighbor_offset = 0, row_offset = 0;
    int metric = FG_METRIC_L2;
    int dup_free = 0;
    int runtime_geo = 0;  // FG_FORCE_RUNTIME_GEOMETRY at creation (a test knob)
    float *d_q = nullptr;
    size_t q_cap = 0;
    uint32_t *d_res = nullptr;
    size_t res_cap = 0;
    uint32_t *d_cnt = nullptr;
    size_t cnt_cap = 0;
    // two-launch search: suspended queries' state, keys and order; the event
    // after the last sliced search, which the next one waits for
    uint32_t *d_slice = nullptr;
    size_t slice_cap = 0;
    hipEvent_t slice_done = nullptr;
    bool slice_pending = false;
    hipStream_t slice_stream = nullptr;  // the stream of the last sliced search
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    // this device's staging area of fg_search_noalloc (device address)
    unsigned char *noalloc = nullptr;
    // serving streams of fg_search_stream (created on first use, default priority)
    static constexpr int kMaxServeStreams = 8;
    hipStream_t serve[kMaxServeStreams] = {};
    hipEvent_t serve_done[kMaxServeStreams] = {};
    hipEvent_t serve_start = nullptr;
    int serve_count = 0;
};

namespace {

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

#define FG_HIP(call, what)                                                                          \
    do {                                                                                            \
        hipError_t _e = (call);                                                                     \
        if (_e != hipSuccess) return fail(FG_EDEVICE, std::string(what) + ": " + hipGetErrorString(_e)); \
    } while (0)

void compute_offsets(fg_index *ix) {
    uint32_t b = 1;
    while (b < ix->dim) b <<= 1;
    ix->padded_dim = b;
    ix->code_offset = ix->dim;
    ix->factor_offset = ix->code_offset + static_cast<uint64_t>(b / 64) * 2u * ix->degree;
    ix->neighbor_offset = ix->factor_offset + 3ull * ix->degree;
    ix->row_offset = ix->neighbor_offset + ix->degree;
}

int check_shape(uint32_t dim, uint32_t degree) {
    if (dim < 33 || dim > static_cast<uint32_t>(kMaxPaddedDim))
        return fail(FG_EINVAL, "dim must be in [33, 2048] (the code layout needs padded_dim >= 64)");
    if (degree < 1 || degree > static_cast<uint32_t>(kMaxDegree)) return fail(FG_EINVAL, "degree must be in [1, 1024]");
    return FG_OK;
}

// include/common.hpp:26-47 + distance.hpp:14-29 (scalar loops, no contraction)
uint32_t host_entry_point(const float *rows, uint64_t n, uint32_t dim, uint64_t row_offset, int metric) {
    std::vector<float> c(dim, 0.0f);
    const float inv = 1.0f / static_cast<float>(n);
    for (uint64_t i = 0; i < n; ++i) {
        const float *r = rows + i * row_offset;
        for (uint32_t d = 0; d < dim; ++d) {
            volatile float t = r[d] * inv;
            c[d] += t;
        }
    }
    uint32_t best = 0;
    float best_d = FLT_MAX;
    for (uint64_t i = 0; i < n; ++i) {
        const float *r = rows + i * row_offset;
        float s = 0.0f;
        for (uint32_t d = 0; d < dim; ++d) {
            if (metric == FG_METRIC_IP) {
                volatile float p = r[d] * c[d];
                s += p;
            } else {
                const float df = r[d] - c[d];
                volatile float p = df * df;
                s += p;
            }
        }
        if (metric == FG_METRIC_IP) s = -s;
        if (s < best_d) {
            best_d = s;
            best = static_cast<uint32_t>(i);
        }
    }
    return best;
}

// Device address of `scratch` on `device` (which must be current), resolved
// once per device and kept for the life of the process.
constexpr int kMaxDevices = 64;
std::mutex g_staging_mu;
unsigned char *g_staging[kMaxDevices] = {};
// held by fg_search_noalloc for the whole of its use of a device's staging
// area (upload, launch, synchronisation, download): calls on one device from
// several host threads run one after another instead of overwriting each
// other's queries and ids
std::mutex g_staging_use[kMaxDevices];

int noalloc_staging(int device, unsigned char **out) {
    std::lock_guard<std::mutex> lock(g_staging_mu);
    if (device < 0 || device >= kMaxDevices) return fail(FG_EDEVICE, "device ordinal out of range");
    if (!g_staging[device]) {
        void *p = nullptr;
        FG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "address of the fg_search_noalloc staging area");
        if (!p) return fail(FG_EDEVICE, "address of the fg_search_noalloc staging area is NULL");
        g_staging[device] = static_cast<unsigned char *>(p);
    }
    *out = g_staging[device];
    return FG_OK;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int ensure(void **p, size_t *cap, size_t need) {
    if (*cap >= need) return FG_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    if (hipMalloc(p, need) != hipSuccess) return fail(FG_ENOMEM, "hipMalloc of search buffers failed");
    *cap = need;
    return FG_OK;
}

// Whether an index must use the general kernels: the fixed-geometry kernels
// address rows with 32-bit byte offsets, so a codebook of 4 GiB or more (or
// an index created with FG_FORCE_RUNTIME_GEOMETRY=1) takes runtime offsets
// and 64-bit row addresses.
inline bool index_runtime_geo(const fg_index *ix) {
    return ix->runtime_geo || ix->npoints * ix->row_offset * 4ull > 0xFFFFFFFFull;
}

// The benchmark shapes that get compile-time geometry (d 128 / degree 32;
// d 96 / degree 32 and 16) while 32-bit row offsets reach every row.
inline bool fixed_geometry(int runtime_geo, int dim, int degree) {
    return !runtime_geo && ((dim == 128 && degree == 32) || (dim == 96 && (degree == 32 || degree == 16)));
}

int make_params(fg_index *ix, uint32_t nq, uint32_t K, uint32_t beam, SearchParams &P) {
    if (K < 1) return fail(FG_EINVAL, "K must be >= 1");
    if (beam < 1 || beam > static_cast<uint32_t>(kMaxBeam))
        return fail(FG_EINVAL, "beam must be in [1, 1024]");
    if (nq > static_cast<uint32_t>(INT32_MAX)) return fail(FG_EINVAL, "nq must be at most 2^31 - 1 (one workgroup per query)");
    int cur = -1;
    FG_HIP(hipGetDevice(&cur), "current device");
    if (cur != ix->device)
        return fail(FG_EINVAL, "the index lives on device " + std::to_string(ix->device) + " but device " +
                                   std::to_string(cur) + " is current");
    P.data = ix->d_rows;
    P.signs = ix->d_signs;
    P.npoints = ix->npoints;
    P.row_offset = ix->row_offset;
    P.code_offset = ix->code_offset;
    P.factor_offset = ix->factor_offset;
    P.neighbor_offset = ix->neighbor_offset;
    P.dim = static_cast<int>(ix->dim);
    P.padded_dim = static_cast<int>(ix->padded_dim);
    P.degree = static_cast<int>(ix->degree);
    P.K = static_cast<int>(K);
    P.beam = static_cast<int>(beam);
    P.pbeam = static_cast<int>(effective_sort_beam(beam));
    uint32_t cap = static_cast<uint32_t>(kSearchWidth) * ix->degree;
    if (cap > static_cast<uint32_t>(kBufferBound)) cap = kBufferBound;
    P.cbs = static_cast<int>(round_up_pow2(cap));
    P.collect_cap = P.cbs < kBufferBound ? P.cbs : kBufferBound;
    P.buckets = static_cast<int>(
        visited_buckets(ix->dim, ix->padded_dim, static_cast<uint32_t>(P.pbeam), beam, ix->degree));
    // The reference's visited table has 2^bitlen slots with bitlen sized for
    // 32 inserts per iteration (utils.cuh:137-151): 2048 at every beam up to
    // 1024.  Between two resets it receives at most beam + 16 * 32 * tiles
    // distinct keys; above 64 neighbours that can exceed its slots, and a full
    // table reports new keys as visited, which no exact set reproduces.  Such
    // (beam, degree) pairs are refused; every degree up to 64 fits.
    {
        const uint32_t tiles = (ix->degree + 31u) / 32u;
        const uint32_t need = beam + 16u * 32u * tiles;
        uint32_t target = ((static_cast<uint32_t>(P.pbeam) + 32u * 16u) * 4u + 2u) / 3u, cap = 1u << 11;
        while (cap < target) cap <<= 1;
        if (need > cap)
            return fail(FG_EINVAL, "degree " + std::to_string(ix->degree) + " at beam " + std::to_string(beam) +
                                       ": up to " + std::to_string(need) + " visited keys between resets exceed the " +
                                       std::to_string(cap) + "-slot table whose overflow the search reproduces "
                                       "(use a smaller beam or degree)");
    }
    P.max_iter = static_cast<int>((beam * 11 + 9) / 10);  // gpu_search_adaptive.cu:96
    // merge-path segmentation of the reference's 256-thread block
    // (utils.cuh:633-641): ceil(pbeam / 4) rounded up to a multiple of 32
    P.seg_active = 0;
    P.seg_magic = 0;
    if (P.pbeam > 128) {
        int active = ((P.pbeam + 3) / 4 + 31) / 32 * 32;
        if (active > kRefBlock) active = kRefBlock;
        P.seg_active = active;
        // exact for t * pbeam < 2^18: the reciprocal's error adds < 2^-14
        // while t * pbeam / active sits >= 1 / active below the next integer
        P.seg_magic = static_cast<uint32_t>((1ull << 32) / static_cast<uint64_t>(active) + 1ull);
    }
    P.phase2_rho = ix->degree <= 4u ? 0.0f : 1.0f - 4.0f / static_cast<float>(ix->degree);  // utils 20-23
    P.use_ip = ix->metric == FG_METRIC_IP ? 1 : 0;
    P.dup_free = ix->dup_free;
    P.vec_ok = (ix->row_offset % 4 == 0 && ix->code_offset % 4 == 0) ? 1 : 0;
    P.runtime_geo = index_runtime_geo(ix) ? 1 : 0;
    P.entry = ix->entry;
    P.nq = static_cast<int>(nq);
    P.slice_suspend = 0;
    P.slice_resume = 0;
    P.slice_state = nullptr;
    P.slice_keys = nullptr;
    P.slice_order = nullptr;
    P.lds = lds_layout(ix->dim, ix->padded_dim, static_cast<uint32_t>(P.pbeam), static_cast<uint32_t>(P.buckets));
    P.team = P.lds.total_team <= 65536u ? 1 : 0;
    return FG_OK;
}

// Shape classes: the benchmark shapes (d 128 / deg 32; d 96 / deg 32 and 16)
// get fully compile-time geometry while the codebook is under 4 GiB; other
// shapes and larger codebooks use runtime offsets.
// one_wave: the one-wave form without asking the occupancy rule again (the
// slices of a search whose form is already known)
// resident (with waves_only): the one-wave kernel's workgroups the device holds at once
template <bool PROF>
int launch_t(const SearchParams &P, hipStream_t stream, int *waves_only = nullptr, bool one_wave = false,
             long long *resident = nullptr) {
    if (P.nq == 0 && !waves_only) return FG_OK;
    const bool count = P.counters != nullptr;
    const int W = P.padded_dim / 32;
    const bool fixed = fixed_geometry(P.runtime_geo, P.dim, P.degree);
    if (fixed && P.dim == 128) {
        launch_shape0(P, stream, count, PROF, waves_only, one_wave, resident);
    } else if (fixed && P.degree == 32) {
        launch_shape1(P, stream, count, PROF, waves_only, one_wave, resident);
    } else if (fixed) {
        launch_shape2(P, stream, count, PROF, waves_only, one_wave, resident);
    } else if (W == 2 && P.dim <= 64) {
        launch_shape3(P, stream, count, PROF, waves_only, one_wave, resident);
    } else if (W == 4 && P.dim <= 96) {
        launch_shape4(P, stream, count, PROF, waves_only, one_wave, resident);
    } else if (W == 4) {
        launch_shape5(P, stream, count, PROF, waves_only, one_wave, resident);
    } else {
        launch_shape6(P, stream, count, PROF, waves_only, one_wave, resident);
    }
    if (waves_only) return FG_OK;
    FG_HIP(hipGetLastError(), "search kernel launch");
    return FG_OK;
}

// Whether a search may run as two launches (first slice, order, second
// slice): searches that reach the suspension point, with suspended state of
// at most kSliceMaxBytes (about 400,000 queries at d 128, beam 256).
// slice_fits then asks for the one-wave form and a batch larger than the
// device holds at once (the last queries to start are the ones that make a
// launch's tail).  FLASHGANN_SLICE=0 / 1 forces one launch / two launches
// wherever the form allows them (tests run both).
constexpr int kSliceStop = 15;  // the top of the first iteration that rebuilds the visited table
constexpr uint64_t kSliceMaxBytes = 1ull << 30;

// Words of the two-launch search's buffer: the header, the per-query states,
// the keys and the order, and above kSliceMaxQueries queries the order
// step's work area (per-query bins, the histogram, two words per chunk).
uint64_t slice_buffer_words(const SearchParams &P, uint64_t *states_out, uint64_t *pad_out) {
    const uint64_t nq = static_cast<uint64_t>(P.nq), pad = (nq + 63u) & ~63ull;
    const uint64_t states = nq * slice_words(static_cast<uint32_t>(P.pbeam), static_cast<uint32_t>(P.padded_dim));
    uint64_t words = kSliceHeader + states + 2u * pad;
    if (nq > static_cast<uint64_t>(kSliceMaxQueries)) {
        const uint64_t chunks = (nq + kSliceChunk - 1) / kSliceChunk;
        words += pad + kSliceBins + 2u * chunks;
    }
    if (states_out) *states_out = states;
    if (pad_out) *pad_out = pad;
    return words;
}

bool slice_wanted(const SearchParams &P) {
    if (P.nq < 1 || P.max_iter <= kSliceStop) return false;
    return slice_buffer_words(P, nullptr, nullptr) * 4u <= kSliceMaxBytes;
}

// slice_wanted's answer for a batch whose form is known: the one-wave form,
// and more queries than the device holds at once (when every query starts
// at once, there is no order to improve), or FLASHGANN_SLICE's answer.
bool slice_fits(const SearchParams &P, int waves, long long resident) {
    if (waves != 1) return false;
    if (const char *e = std::getenv("FLASHGANN_SLICE")) {
        if (e[0] == '0') return false;
        if (e[0] == '1') return true;
    }
    return resident > 0 && static_cast<long long>(P.nq) > resident;
}

int launch(fg_index *ix, const SearchParams &P0, hipStream_t stream, bool may_slice) {
    // a stream being captured into a graph gets one launch: the two-launch
    // search may allocate its state buffer and orders itself with an event
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (may_slice && hipStreamIsCapturing(stream, &capture) == hipSuccess && capture != hipStreamCaptureStatusNone)
        may_slice = false;
    if (may_slice && slice_wanted(P0)) {
        int waves = 0;
        long long resident = 0;
        if (int rc = launch_t<false>(P0, stream, &waves, false, &resident)) return rc;
        if (slice_fits(P0, waves, resident)) {
            // one buffer: header (word 0: the count of suspended queries), the
            // per-query states, the keys, the order (and the order step's work
            // area).  If it cannot be allocated, the search makes one launch.
            uint64_t states = 0, pad = 0;
            const uint64_t words = slice_buffer_words(P0, &states, &pad);
            if (ensure(reinterpret_cast<void **>(&ix->d_slice), &ix->slice_cap, words * 4u) != FG_OK) {
                (void)hipGetLastError();
                return launch_t<false>(P0, stream, nullptr, true);
            }
            if (!ix->slice_done) FG_HIP(hipEventCreateWithFlags(&ix->slice_done, hipEventDisableTiming), "event");
            // a sliced search on another stream may still use the buffer
            if (ix->slice_pending && ix->slice_stream != stream)
                FG_HIP(hipStreamWaitEvent(stream, ix->slice_done, 0), "stream wait");
            uint32_t *state = ix->d_slice, *keys = state + kSliceHeader + states, *order = keys + pad;
            SearchParams P = P0;
            P.slice_state = state;
            P.slice_keys = keys;
            P.slice_order = order;
            // (a third slice, suspending again at iteration 31 and reordering by
            // the K-th cutoff, measured 4-10% slower than two)
            P.slice_suspend = kSliceStop;
            P.slice_resume = 0;
            if (int rc = launch_t<false>(P, stream, nullptr, true)) return rc;
            if (P0.nq <= kSliceMaxQueries) {
                hipLaunchKernelGGL(fg_slice_order_kernel, dim3(1), dim3(1024), 0, stream, state, keys, P0.nq, order);
            } else {
                const int chunks = (P0.nq + kSliceChunk - 1) / kSliceChunk;
                uint32_t *qbin = order + pad, *ghist = qbin + pad, *ext = ghist + kSliceBins;
                hipLaunchKernelGGL(fg_slice_minmax_kernel, dim3(chunks), dim3(256), 0, stream, keys, P0.nq, ext, ghist,
                                   chunks);
                hipLaunchKernelGGL(fg_slice_hist_kernel, dim3(chunks), dim3(256), 0, stream, keys, P0.nq, ext, chunks,
                                   ghist, qbin);
                hipLaunchKernelGGL(fg_slice_scan_kernel, dim3(1), dim3(1024), 0, stream, ghist, state);
                hipLaunchKernelGGL(fg_slice_scatter_kernel, dim3((P0.nq + 255) / 256), dim3(256), 0, stream, qbin,
                                   P0.nq, ghist, order);
            }
            FG_HIP(hipGetLastError(), "order kernel launch");
            P.slice_resume = kSliceStop;
            P.slice_suspend = 0;
            if (int rc = launch_t<false>(P, stream, nullptr, true)) return rc;
            FG_HIP(hipEventRecord(ix->slice_done, stream), "event record");
            ix->slice_pending = true;
            ix->slice_stream = stream;
            return FG_OK;
        }
    }
    return launch_t<false>(P0, stream);
}

bool rows_dup_free(const float *rows, uint64_t n, uint32_t degree, uint64_t nbr_off, uint64_t row_off) {
    std::vector<uint32_t> tmp(degree);
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t *nb = reinterpret_cast<const uint32_t *>(rows + i * row_off + nbr_off);
        std::copy(nb, nb + degree, tmp.begin());
        std::sort(tmp.begin(), tmp.end());
        for (uint32_t j = 1; j < degree; ++j)
            if (tmp[j] == tmp[j - 1] && tmp[j] != kMaxIndex) return false;
    }
    return true;
}

}  // namespace

extern "C" {

const char *fg_last_error(void) { return g_err.c_str(); }
const char *fg_version(void) { return "flashgann-amd 0.1 (gfx950, wave64)"; }

uint32_t fg_lds_bytes(uint32_t dim, uint32_t beam, uint32_t degree) {
    uint32_t b = 1;
    while (b < dim) b <<= 1;
    const uint32_t pb = effective_sort_beam(beam);
    return lds_layout(dim, b, pb, visited_buckets(dim, b, pb, beam, degree)).total;
}

int fg_search_waves(fg_index *ix, uint32_t nq, uint32_t K, uint32_t beam) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    SearchParams P;
    if (int rc = make_params(ix, nq, K, beam, P)) return rc;
    int waves = 1;
    if (int rc = launch_t<false>(P, nullptr, &waves)) return rc;
    return waves;
}

int fg_search_launches(fg_index *ix, uint32_t nq, uint32_t K, uint32_t beam) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    SearchParams P;
    if (int rc = make_params(ix, nq, K, beam, P)) return rc;
    if (!slice_wanted(P)) return 1;
    int waves = 1;
    long long resident = 0;
    if (int rc = launch_t<false>(P, nullptr, &waves, false, &resident)) return rc;
    return slice_fits(P, waves, resident) ? 2 : 1;
}

int fg_search_geometry(const fg_index *ix) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    const bool rt = index_runtime_geo(ix);
    return fixed_geometry(rt ? 1 : 0, static_cast<int>(ix->dim), static_cast<int>(ix->degree)) ? FG_GEOMETRY_FIXED
                                                                                                : FG_GEOMETRY_GENERAL;
}

int fg_index_create(const float *rows, uint64_t npoints, uint32_t dim, uint32_t degree, const float *signs,
                    uint32_t entry, int metric, fg_index **out) {
    if (!out) return fail(FG_EINVAL, "out is NULL");
    *out = nullptr;
    if (!rows || !signs || npoints == 0) return fail(FG_EINVAL, "rows/signs must be non-NULL and npoints > 0");
    if (int rc = check_shape(dim, degree)) return rc;
    if (metric != FG_METRIC_L2 && metric != FG_METRIC_IP) return fail(FG_EINVAL, "unknown metric");
    fg_index *ix = new (std::nothrow) fg_index();
    if (!ix) return fail(FG_ENOMEM, "host allocation failed");
    ix->npoints = npoints;
    ix->dim = dim;
    ix->degree = degree;
    ix->metric = metric;
    compute_offsets(ix);
    if (entry == FG_ENTRY_AUTO) entry = host_entry_point(rows, npoints, dim, ix->row_offset, metric);
    if (entry >= npoints) {
        delete ix;
        return fail(FG_EINVAL, "entry point out of range");
    }
    ix->entry = entry;
    ix->dup_free = rows_dup_free(rows, npoints, degree, ix->neighbor_offset, ix->row_offset) ? 1 : 0;
    {
        const char *env = std::getenv("FG_FORCE_RUNTIME_GEOMETRY");
        ix->runtime_geo = env && env[0] == '1' ? 1 : 0;
    }
    const size_t bytes = static_cast<size_t>(npoints) * ix->row_offset * sizeof(float);
    size_t free_b = 0, total_b = 0;
    if (hipGetDevice(&ix->device) != hipSuccess || hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        delete ix;
        return fail(FG_EDEVICE, "no HIP device available");
    }
    if (bytes + ix->padded_dim * sizeof(float) > free_b) {  // gpu_search_adaptive.cu:61-63
        delete ix;
        return fail(FG_ENOMEM, "QG upload exceeds currently available GPU memory");
    }
    // set-up of fg_search_noalloc on this device (current here)
    if (int rc = noalloc_staging(ix->device, &ix->noalloc)) {
        delete ix;
        return rc;
    }
    if (hipMalloc(&ix->d_rows, bytes) != hipSuccess || hipMalloc(&ix->d_signs, ix->padded_dim * sizeof(float)) != hipSuccess) {
        fg_index_destroy(ix);
        return fail(FG_ENOMEM, "hipMalloc of the codebook failed");
    }
    if (hipMemcpy(ix->d_rows, rows, bytes, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ix->d_signs, signs, ix->padded_dim * sizeof(float), hipMemcpyHostToDevice) != hipSuccess ||
        hipEventCreate(&ix->ev0) != hipSuccess || hipEventCreate(&ix->ev1) != hipSuccess) {
        fg_index_destroy(ix);
        return fail(FG_EDEVICE, "codebook upload failed");
    }
    *out = ix;
    return FG_OK;
}

int fg_index_load(const char *path, uint64_t npoints, uint32_t dim, uint32_t degree, int metric, fg_index **out) {
    if (!out || !path) return fail(FG_EINVAL, "NULL argument");
    *out = nullptr;
    if (int rc = check_shape(dim, degree)) return rc;
    fg_index tmp;
    tmp.dim = dim;
    tmp.degree = degree;
    compute_offsets(&tmp);
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(FG_EIO, std::string("Cannot open codebook file: ") + path);
    uint32_t entry = 0;
    const size_t nfl = static_cast<size_t>(npoints) * tmp.row_offset;
    std::vector<float> rows;
    std::vector<float> signs(tmp.padded_dim);
    try {
        rows.resize(nfl);
    } catch (...) {
        return fail(FG_ENOMEM, "host allocation for the codebook failed");
    }
    f.read(reinterpret_cast<char *>(&entry), sizeof(entry));
    f.read(reinterpret_cast<char *>(rows.data()), static_cast<std::streamsize>(nfl * sizeof(float)));
    f.read(reinterpret_cast<char *>(signs.data()), static_cast<std::streamsize>(signs.size() * sizeof(float)));
    if (!f) return fail(FG_EIO, std::string("codebook file is truncated: ") + path);
    return fg_index_create(rows.data(), npoints, dim, degree, signs.data(), entry, metric, out);
}

void fg_index_destroy(fg_index *ix) {
    if (!ix) return;
    // searches still running on the index's own streams (serving batches, a
    // two-launch search) end before any of its memory is released
    if (ix->slice_done) (void)hipEventSynchronize(ix->slice_done);
    for (int i = 0; i < ix->serve_count; ++i) (void)hipStreamSynchronize(ix->serve[i]);
    if (ix->d_rows) (void)hipFree(ix->d_rows);
    if (ix->d_signs) (void)hipFree(ix->d_signs);
    if (ix->d_q) (void)hipFree(ix->d_q);
    if (ix->d_res) (void)hipFree(ix->d_res);
    if (ix->d_cnt) (void)hipFree(ix->d_cnt);
    if (ix->slice_done) (void)hipEventDestroy(ix->slice_done);
    if (ix->d_slice) (void)hipFree(ix->d_slice);
    if (ix->ev0) (void)hipEventDestroy(ix->ev0);
    if (ix->ev1) (void)hipEventDestroy(ix->ev1);
    for (int i = 0; i < ix->serve_count; ++i) {
        (void)hipStreamDestroy(ix->serve[i]);
        (void)hipEventDestroy(ix->serve_done[i]);
    }
    if (ix->serve_start) (void)hipEventDestroy(ix->serve_start);
    delete ix;
}

int fg_index_get_info(const fg_index *ix, fg_index_info *info) {
    if (!ix || !info) return fail(FG_EINVAL, "NULL argument");
    info->dim = ix->dim;
    info->padded_dim = ix->padded_dim;
    info->degree = ix->degree;
    info->entry = ix->entry;
    info->npoints = ix->npoints;
    info->code_offset = ix->code_offset;
    info->factor_offset = ix->factor_offset;
    info->neighbor_offset = ix->neighbor_offset;
    info->row_offset = ix->row_offset;
    info->metric = ix->metric;
    return FG_OK;
}

int fg_search_device(fg_index *ix, const float *d_queries, uint32_t nq, uint32_t K, uint32_t beam,
                     uint32_t *d_results, uint32_t *d_counters, void *stream) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    if (nq && (!d_queries || !d_results)) return fail(FG_EINVAL, "NULL device buffer");
    SearchParams P;
    if (int rc = make_params(ix, nq, K, beam, P)) return rc;
    P.queries = d_queries;
    P.results = d_results;
    P.counters = d_counters;
    P.phase = nullptr;
    return launch(ix, P, reinterpret_cast<hipStream_t>(stream), true);
}

int fg_search_stream(fg_index *ix, const float *d_queries, uint32_t nq, uint32_t K, uint32_t beam,
                     uint32_t *d_results, uint32_t batch, uint32_t nstreams, void *stream) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    if (batch == 0) return fail(FG_EINVAL, "batch must be >= 1");
    if (nstreams < 1 || nstreams > static_cast<uint32_t>(fg_index::kMaxServeStreams))
        return fail(FG_EINVAL, "nstreams must be in [1, 8]");
    if (nq && (!d_queries || !d_results)) return fail(FG_EINVAL, "NULL device buffer");
    SearchParams P;
    if (int rc = make_params(ix, batch < nq ? batch : nq, K, beam, P)) return rc;
    if (nq == 0) return FG_OK;
    hipStream_t caller = reinterpret_cast<hipStream_t>(stream);
    while (ix->serve_count < static_cast<int>(nstreams)) {
        const int i = ix->serve_count;
        FG_HIP(hipStreamCreateWithFlags(&ix->serve[i], hipStreamNonBlocking), "serving stream");
        if (hipEventCreateWithFlags(&ix->serve_done[i], hipEventDisableTiming) != hipSuccess) {
            (void)hipStreamDestroy(ix->serve[i]);
            return fail(FG_EDEVICE, "serving event");
        }
        ix->serve_count = i + 1;
    }
    if (!ix->serve_start) FG_HIP(hipEventCreateWithFlags(&ix->serve_start, hipEventDisableTiming), "serving event");
    // every batch runs after the work already queued on the caller's stream
    FG_HIP(hipEventRecord(ix->serve_start, caller), "event record");
    const uint32_t nbatch = (nq + batch - 1) / batch;
    const uint32_t used = nbatch < nstreams ? nbatch : nstreams;
    for (uint32_t i = 0; i < used; ++i) FG_HIP(hipStreamWaitEvent(ix->serve[i], ix->serve_start, 0), "stream wait");
    for (uint32_t b = 0; b < nbatch; ++b) {
        const uint64_t q0 = static_cast<uint64_t>(b) * batch;
        const uint32_t n = static_cast<uint32_t>(nq - q0 < batch ? nq - q0 : batch);
        SearchParams Pb = P;
        Pb.nq = static_cast<int>(n);
        Pb.queries = d_queries + q0 * ix->dim;
        Pb.results = d_results + q0 * K;
        Pb.counters = nullptr;
        Pb.phase = nullptr;
        if (int rc = launch(ix, Pb, ix->serve[b % nstreams], false)) return rc;
    }
    // and the caller's later work runs after every batch
    for (uint32_t i = 0; i < used; ++i) {
        FG_HIP(hipEventRecord(ix->serve_done[i], ix->serve[i]), "event record");
        FG_HIP(hipStreamWaitEvent(caller, ix->serve_done[i], 0), "stream wait");
    }
    return FG_OK;
}

int fg_search_profile(fg_index *ix, const float *d_queries, uint32_t nq, uint32_t K, uint32_t beam,
                      uint32_t *d_results, unsigned long long *d_phase, void *stream) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    if (nq && (!d_queries || !d_results || !d_phase)) return fail(FG_EINVAL, "NULL device buffer");
    SearchParams P;
    if (int rc = make_params(ix, nq, K, beam, P)) return rc;
    P.queries = d_queries;
    P.results = d_results;
    P.counters = nullptr;
    P.phase = d_phase;
    return launch_t<true>(P, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Host-buffer search of fg_search / fg_search_noalloc: the queries are copied
// into `dq`, the kernel runs on the null stream, and the ids (and counters)
// are copied back from `dres` (`dcnt`).
int search_host(fg_index *ix, SearchParams &P, const float *queries, uint32_t nq, uint32_t K, uint32_t *result_ids,
                uint32_t *counters, fg_stats *stats, float *dq, uint32_t *dres, uint32_t *dcnt, bool may_slice) {
    const size_t qb = static_cast<size_t>(nq) * ix->dim * sizeof(float);
    const size_t rb = static_cast<size_t>(nq) * K * sizeof(uint32_t);
    const size_t cb = static_cast<size_t>(nq) * FG_COUNTERS_PER_QUERY * sizeof(uint32_t);
    FG_HIP(hipMemcpy(dq, queries, qb, hipMemcpyHostToDevice), "query upload");
    FG_HIP(hipDeviceSynchronize(), "sync before search");
    P.queries = dq;
    P.results = dres;
    P.counters = counters ? dcnt : nullptr;
    P.phase = nullptr;
    const auto t0 = std::chrono::high_resolution_clock::now();
    FG_HIP(hipEventRecord(ix->ev0, nullptr), "event record");
    if (int rc = launch(ix, P, nullptr, may_slice)) return rc;
    FG_HIP(hipEventRecord(ix->ev1, nullptr), "event record");
    FG_HIP(hipDeviceSynchronize(), "search kernel");
    const auto t1 = std::chrono::high_resolution_clock::now();
    if (stats) {
        stats->elapsed_s = std::chrono::duration<double>(t1 - t0).count();
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, ix->ev0, ix->ev1) == hipSuccess) stats->kernel_ms = ms;
    }
    FG_HIP(hipMemcpy(result_ids, dres, rb, hipMemcpyDeviceToHost), "result download");
    if (counters) FG_HIP(hipMemcpy(counters, dcnt, cb, hipMemcpyDeviceToHost), "counter download");
    return FG_OK;
}

int search_prologue(fg_index *ix, const float *queries, uint32_t nq, uint32_t K, uint32_t beam, uint32_t *result_ids,
                    fg_stats *stats, SearchParams &P) {
    if (!ix) return fail(FG_EINVAL, "index is NULL");
    if (nq && (!queries || !result_ids)) return fail(FG_EINVAL, "NULL host buffer");
    if (int rc = make_params(ix, nq, K, beam, P)) return rc;
    if (stats) {
        stats->elapsed_s = 0.0;
        stats->kernel_ms = 0.0f;
        stats->lds_bytes = P.lds.total;
        stats->visited_slots = 4u * static_cast<uint32_t>(P.buckets);
    }
    return FG_OK;
}

}  // namespace

extern "C" {

int fg_search(fg_index *ix, const float *queries, uint32_t nq, uint32_t K, uint32_t beam, uint32_t *result_ids,
              uint32_t *counters, fg_stats *stats) {
    SearchParams P;
    if (int rc = search_prologue(ix, queries, nq, K, beam, result_ids, stats, P)) return rc;
    if (nq == 0) return FG_OK;
    const size_t qb = static_cast<size_t>(nq) * ix->dim * sizeof(float);
    const size_t rb = static_cast<size_t>(nq) * K * sizeof(uint32_t);
    const size_t cb = static_cast<size_t>(nq) * FG_COUNTERS_PER_QUERY * sizeof(uint32_t);
    if (int rc = ensure(reinterpret_cast<void **>(&ix->d_q), &ix->q_cap, qb)) return rc;
    if (int rc = ensure(reinterpret_cast<void **>(&ix->d_res), &ix->res_cap, rb)) return rc;
    if (counters)
        if (int rc = ensure(reinterpret_cast<void **>(&ix->d_cnt), &ix->cnt_cap, cb)) return rc;
    return search_host(ix, P, queries, nq, K, result_ids, counters, stats, ix->d_q, ix->d_res, ix->d_cnt, true);
}

int fg_search_noalloc(fg_index *ix, const float *queries, uint32_t nq, uint32_t K, uint32_t beam,
                      uint32_t *result_ids, uint32_t *counters, fg_stats *stats) {
    SearchParams P;
    if (int rc = search_prologue(ix, queries, nq, K, beam, result_ids, stats, P)) return rc;
    if (nq == 0) return FG_OK;
    // staging: queries, then result ids, then counters, each 256-byte aligned
    const size_t qb = align256(static_cast<size_t>(nq) * ix->dim * sizeof(float));
    const size_t rb = align256(static_cast<size_t>(nq) * K * sizeof(uint32_t));
    const size_t cb = counters ? align256(static_cast<size_t>(nq) * FG_COUNTERS_PER_QUERY * sizeof(uint32_t)) : 0;
    if (qb + rb + cb > FG_NOALLOC_STAGING_BYTES)
        return fail(FG_EINVAL, "fg_search_noalloc: " + std::to_string(nq) + " queries need " +
                                   std::to_string(qb + rb + cb) + " bytes of staging, above its maximum of " +
                                   std::to_string(FG_NOALLOC_STAGING_BYTES) + " (use fewer queries per call)");
    if (!ix->noalloc) return fail(FG_EDEVICE, "fg_search_noalloc: staging area not set up");
    unsigned char *base = ix->noalloc;
    std::lock_guard<std::mutex> use(g_staging_use[ix->device]);
    // (one launch: the two-launch search keeps its state in memory the index allocates)
    return search_host(ix, P, queries, nq, K, result_ids, counters, stats, reinterpret_cast<float *>(base),
                       reinterpret_cast<uint32_t *>(base + qb), reinterpret_cast<uint32_t *>(base + qb + rb), false);
}

int fg_query_prepare(fg_index *ix, const float *queries, uint32_t nq, float *rotated, uint8_t *quantized,
                     float *lhw, int32_t *sum_q) {
    if (!ix || !queries || !rotated || !quantized || !lhw || !sum_q) return fail(FG_EINVAL, "NULL argument");
    if (nq == 0) return FG_OK;
    const uint32_t B = ix->padded_dim;
    float *dq = nullptr, *drot = nullptr, *dl = nullptr;
    uint8_t *dqt = nullptr;
    int32_t *ds = nullptr;
    int rc = FG_OK;
    const size_t qb = static_cast<size_t>(nq) * ix->dim * 4;
    if (hipMalloc(&dq, qb) != hipSuccess || hipMalloc(&drot, static_cast<size_t>(nq) * B * 4) != hipSuccess ||
        hipMalloc(&dqt, static_cast<size_t>(nq) * B) != hipSuccess || hipMalloc(&dl, nq * 12ull) != hipSuccess ||
        hipMalloc(&ds, nq * 4ull) != hipSuccess) {
        rc = fail(FG_ENOMEM, "hipMalloc failed");
    }
    if (rc == FG_OK && hipMemcpy(dq, queries, qb, hipMemcpyHostToDevice) != hipSuccess) rc = fail(FG_EDEVICE, "upload");
    if (rc == FG_OK) {
        const uint32_t scratch = B * 4;
        const uint32_t lds = scratch + 8 * (B / 32) * 4;
        hipLaunchKernelGGL(fg_prepare_kernel, dim3(nq), dim3(64), lds, nullptr, dq, ix->d_signs,
                           static_cast<int>(ix->dim), static_cast<int>(B), static_cast<int>(nq), drot, dqt, dl, ds,
                           scratch);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = fail(FG_EDEVICE, "prepare kernel");
    }
    if (rc == FG_OK && (hipMemcpy(rotated, drot, static_cast<size_t>(nq) * B * 4, hipMemcpyDeviceToHost) != hipSuccess ||
                        hipMemcpy(quantized, dqt, static_cast<size_t>(nq) * B, hipMemcpyDeviceToHost) != hipSuccess ||
                        hipMemcpy(lhw, dl, nq * 12ull, hipMemcpyDeviceToHost) != hipSuccess ||
                        hipMemcpy(sum_q, ds, nq * 4ull, hipMemcpyDeviceToHost) != hipSuccess))
        rc = fail(FG_EDEVICE, "download");
    (void)hipFree(dq);
    (void)hipFree(drot);
    (void)hipFree(dqt);
    (void)hipFree(dl);
    (void)hipFree(ds);
    return rc;
}

int fg_score_edges(fg_index *ix, const float *queries, uint32_t nq, const uint32_t *query_ix, const uint32_t *parents,
                   const uint32_t *slots, uint32_t n, float *est_lanes, float *est_seq, float *exact) {
    if (!ix || !queries || !query_ix || !parents || !slots) return fail(FG_EINVAL, "NULL argument");
    if (n == 0) return FG_OK;
    for (uint32_t i = 0; i < n; ++i) {
        if (query_ix[i] >= nq || parents[i] >= ix->npoints || slots[i] >= ix->degree)
            return fail(FG_EINVAL, "score triple out of range");
    }
    const uint32_t B = ix->padded_dim;
    ScoreParams S{};
    S.data = ix->d_rows;
    S.signs = ix->d_signs;
    S.row_offset = ix->row_offset;
    S.code_offset = ix->code_offset;
    S.factor_offset = ix->factor_offset;
    S.npoints = ix->npoints;
    S.dim = static_cast<int>(ix->dim);
    S.B = static_cast<int>(B);
    S.deg = static_cast<int>(ix->degree);
    S.use_ip = ix->metric == FG_METRIC_IP;
    S.n = n;
    S.query_off = B * 4;
    S.plane_off = S.query_off + ((ix->dim + 3) & ~3u) * 4;
    const uint32_t lds = S.plane_off + 8 * (B / 32) * 4;
    float *dq = nullptr, *o1 = nullptr, *o2 = nullptr, *o3 = nullptr;
    uint32_t *t1 = nullptr, *t2 = nullptr, *t3 = nullptr;
    int rc = FG_OK;
    const size_t qb = static_cast<size_t>(nq) * ix->dim * 4;
    if (hipMalloc(&dq, qb) != hipSuccess || hipMalloc(&o1, n * 4ull) != hipSuccess || hipMalloc(&o2, n * 4ull) != hipSuccess ||
        hipMalloc(&o3, n * 4ull) != hipSuccess || hipMalloc(&t1, n * 4ull) != hipSuccess ||
        hipMalloc(&t2, n * 4ull) != hipSuccess || hipMalloc(&t3, n * 4ull) != hipSuccess)
        rc = fail(FG_ENOMEM, "hipMalloc failed");
    if (rc == FG_OK && (hipMemcpy(dq, queries, qb, hipMemcpyHostToDevice) != hipSuccess ||
                        hipMemcpy(t1, query_ix, n * 4ull, hipMemcpyHostToDevice) != hipSuccess ||
                        hipMemcpy(t2, parents, n * 4ull, hipMemcpyHostToDevice) != hipSuccess ||
                        hipMemcpy(t3, slots, n * 4ull, hipMemcpyHostToDevice) != hipSuccess))
        rc = fail(FG_EDEVICE, "upload");
    if (rc == FG_OK) {
        S.queries = dq;
        S.qix = t1;
        S.parents = t2;
        S.slots = t3;
        S.est_lanes = o1;
        S.est_seq = o2;
        S.exact = o3;
        hipLaunchKernelGGL(fg_score_kernel, dim3(n), dim3(64), lds, nullptr, S);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = fail(FG_EDEVICE, "score kernel");
    }
    if (rc == FG_OK) {
        if ((est_lanes && hipMemcpy(est_lanes, o1, n * 4ull, hipMemcpyDeviceToHost) != hipSuccess) ||
            (est_seq && hipMemcpy(est_seq, o2, n * 4ull, hipMemcpyDeviceToHost) != hipSuccess) ||
            (exact && hipMemcpy(exact, o3, n * 4ull, hipMemcpyDeviceToHost) != hipSuccess))
            rc = fail(FG_EDEVICE, "download");
    }
    (void)hipFree(dq);
    (void)hipFree(o1);
    (void)hipFree(o2);
    (void)hipFree(o3);
    (void)hipFree(t1);
    (void)hipFree(t2);
    (void)hipFree(t3);
    return rc;
}

}  // extern "C"
