// Test driver: exposes the reference's own host-side helpers (compiled from
// the reference tree, include path -I<reference root>) through a C ABI so the
// tests can pin the oracle and the product's host code against them.
// Nothing here re-implements reference logic; each function only forwards.
#include <cstdint>
#include <cstring>
#include <string>

#include "include/common.hpp"
#include "include/data_io.hpp"
#include "include/metric.hpp"
#include "include/qg.hpp"

extern "C" {

// include/common.hpp:49-66
float ref_compute_recall(const uint32_t *pred, const int *gt, uint64_t nq, int topk, int gt_k) {
    return compute_recall<uint32_t>(pred, gt, static_cast<size_t>(nq), topk, gt_k);
}

// include/common.hpp:26-47 (distance via the global metric, metric.hpp:11)
uint32_t ref_compute_entry_point(const float *data, uint64_t n, uint64_t dim, uint64_t row_offset,
                                 int use_ip) {
    g_metric_type = use_ip ? METRIC_IP : METRIC_L2;
    uint32_t e = compute_rabitq_entry_point(data, n, dim, row_offset);
    g_metric_type = METRIC_L2;
    return e;
}

// include/metric.hpp:13-28
int ref_infer_metric_is_ip(const char *path) {
    return infer_metric_from_dataset_path(path) == METRIC_IP ? 1 : 0;
}

// include/data_io.hpp:18-47; returns count, writes dim; copies up to cap floats.
uint64_t ref_load_fvecs(const char *path, int *dim_out, float *dst, uint64_t cap) {
    LoadedVectors<float> v = load_fvecs<float>(path, "ref");
    *dim_out = v.dim;
    uint64_t n = v.values.size() < cap ? v.values.size() : cap;
    if (dst && n) std::memcpy(dst, v.values.data(), n * sizeof(float));
    return v.count;
}

// include/data_io.hpp:49-77
uint64_t ref_load_ivecs(const char *path, int *dim_out, int *dst, uint64_t cap) {
    LoadedVectors<int> v = load_ivecs(path, "ref");
    *dim_out = v.dim;
    uint64_t n = v.values.size() < cap ? v.values.size() : cap;
    if (dst && n) std::memcpy(dst, v.values.data(), n * sizeof(int));
    return v.count;
}

// include/qg.hpp:17-42, 49-60, 66-73: loads a codebook file and reports the
// layout offsets (floats), the entry point, and copies row data / signs.
int ref_qg_load(const char *path, uint64_t n, uint64_t dim, int degree, uint64_t *offsets5,
                uint32_t *entry, float *rows, uint64_t rows_cap, float *signs, uint64_t signs_cap) {
    QuantizationGraph qg(n, dim, degree, std::string(path));
    offsets5[0] = qg.get_code_offset();
    offsets5[1] = qg.get_factor_offset();
    offsets5[2] = qg.get_neighbor_offset();
    offsets5[3] = qg.get_row_offset();
    offsets5[4] = qg.get_signs_bytes() / sizeof(float);
    *entry = qg.get_entry_point();
    uint64_t nf = qg.get_data_bytes() / sizeof(float);
    if (rows && rows_cap) std::memcpy(rows, qg.get_data_ptr(), (nf < rows_cap ? nf : rows_cap) * sizeof(float));
    uint64_t ns = offsets5[4];
    if (signs && signs_cap) std::memcpy(signs, qg.get_signs_ptr(), (ns < signs_cap ? ns : signs_cap) * sizeof(float));
    return 0;
}

}  // extern "C"
