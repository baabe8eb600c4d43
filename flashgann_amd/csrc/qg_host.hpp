// qg_host.hpp -- host-side QuantizationGraph over the flashgann C ABI.
//
// Same constructor and search signature as the reference's class
// (include/qg.hpp:14-89, gpu_search_adaptive.cu:12-114) so a caller written
// against it (main.cu) compiles unchanged.  Differences, all at the boundary:
//   * a truncated codebook file throws instead of being read short
//     (qg.hpp:33-36 leaves fin.read unchecked);
//   * the device copy of the codebook is created on the first search and kept
//     for later calls (the reference re-uploads per call);
//   * HIP failures print the runtime's message and exit(EXIT_FAILURE) like
//     CUDA_SAFE_CALL (utils.cuh:42-50); a device-memory shortfall throws
//     std::runtime_error like gpu_search_adaptive.cu:61-63.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/flashgann.h"
#include "host_io.hpp"

typedef uint32_t vidType;

class QuantizationGraph {
public:
    QuantizationGraph(size_t num_node, size_t dim, int degree, const std::string &codebook_path)
        : num_nodes_(num_node), dim_(dim), degree_(degree) {
        init_layout();
        std::ifstream fin(codebook_path, std::ios::binary);
        if (!fin) throw std::runtime_error("Cannot open codebook file: " + codebook_path);
        fin.read(reinterpret_cast<char *>(&entry_point_), sizeof(uint32_t));
        data_.resize(num_nodes_ * row_offset_);
        fin.read(reinterpret_cast<char *>(data_.data()), static_cast<std::streamsize>(data_.size() * sizeof(float)));
        signs_.resize(padded_dim_);
        fin.read(reinterpret_cast<char *>(signs_.data()), static_cast<std::streamsize>(signs_.size() * sizeof(float)));
        if (!fin) throw std::runtime_error("Codebook file is truncated: " + codebook_path);
        printf("Loaded codebook: %zu nodes, dim=%zu, degree=%d, padded_dim=%zu, row_offset=%zu floats (entry_point=%u)\n",
               num_nodes_, dim_, degree_, padded_dim_, row_offset_, entry_point_);
    }

    ~QuantizationGraph() { fg_index_destroy(index_); }
    QuantizationGraph(const QuantizationGraph &) = delete;
    QuantizationGraph &operator=(const QuantizationGraph &) = delete;

    const float *get_data_ptr() const { return data_.data(); }
    const float *get_signs_ptr() const { return signs_.data(); }
    size_t get_data_bytes() const { return num_nodes_ * row_offset_ * sizeof(float); }
    size_t get_signs_bytes() const { return padded_dim_ * sizeof(float); }
    int get_metric() const { return metric_; }
    void set_metric(int metric) { metric_ = metric; }
    size_t get_code_offset() const { return code_offset_; }
    size_t get_factor_offset() const { return factor_offset_; }
    size_t get_neighbor_offset() const { return neighbor_offset_; }
    size_t get_row_offset() const { return row_offset_; }
    vidType get_entry_point() const { return entry_point_; }

    void gpu_search_adaptive(int nq, const float *queries, int K, vidType *result_idx, int beam_sz, double &elapsed) {
        ensure_index();
        printf("\nGPU adaptive search: K=%d, nq=%d, dim=%zu, npoints=%zu, beam_size=%d, lds_bytes=%u\n", K, nq, dim_,
               num_nodes_, beam_sz, fg_lds_bytes(static_cast<uint32_t>(dim_), static_cast<uint32_t>(beam_sz),
                                                  static_cast<uint32_t>(degree_)));
        fg_stats st;
        const int rc = fg_search(index_, queries, static_cast<uint32_t>(nq), static_cast<uint32_t>(K),
                                 static_cast<uint32_t>(beam_sz), result_idx, nullptr, &st);
        if (rc == FG_ENOMEM) throw std::runtime_error(fg_last_error());
        if (rc != FG_OK) {
            fprintf(stderr, "error %d: %s\n", rc, fg_last_error());
            exit(EXIT_FAILURE);
        }
        printf("GPU adaptive search entry point: %u, visited table %u slots, kernel %.3f ms (event)\n", active_entry_,
               st.visited_slots, st.kernel_ms);
        elapsed = st.elapsed_s;
    }

private:
    void init_layout() {  // qg.hpp:66-73 with an integer power-of-two round-up
        padded_dim_ = 1;
        while (padded_dim_ < dim_) padded_dim_ <<= 1;
        code_offset_ = dim_;
        factor_offset_ = code_offset_ + (padded_dim_ / 64) * 2 * static_cast<size_t>(degree_);
        neighbor_offset_ = factor_offset_ + 3 * static_cast<size_t>(degree_);
        row_offset_ = neighbor_offset_ + static_cast<size_t>(degree_);
    }

    void ensure_index() {
        if (index_ && index_metric_ == metric_) return;
        fg_index_destroy(index_);
        index_ = nullptr;
        const int rc = fg_index_create(data_.data(), num_nodes_, static_cast<uint32_t>(dim_),
                                       static_cast<uint32_t>(degree_), signs_.data(), entry_point_, metric_, &index_);
        if (rc == FG_ENOMEM) throw std::runtime_error(fg_last_error());
        if (rc != FG_OK) {
            fprintf(stderr, "error %d: %s\n", rc, fg_last_error());
            exit(EXIT_FAILURE);
        }
        fg_index_info info;
        fg_index_get_info(index_, &info);
        active_entry_ = info.entry;
        index_metric_ = metric_;
    }

    size_t num_nodes_, dim_, padded_dim_ = 0;
    int degree_;
    vidType entry_point_ = 0, active_entry_ = 0;
    size_t code_offset_ = 0, factor_offset_ = 0, neighbor_offset_ = 0, row_offset_ = 0;
    std::vector<float> data_;
    std::vector<float> signs_;
    int metric_ = FG_METRIC_L2;
    int index_metric_ = -1;
    fg_index *index_ = nullptr;
};
