// host_io.hpp -- the CLI's file formats, recall and CSV row.
//
// fvecs/ivecs: each row is an int32 dimension followed by that many 4-byte
// values; the row count is file_size / (4 + 4*dim) (include/data_io.hpp:18-77).
// Recall counts, over every predicted id, whether it occurs in the first
// min(K, gt_k) ground-truth ids; repeated predictions count each time
// (include/common.hpp:49-66).  The CSV row is TopK,Beam_size,Runtime,Latency,
// Throughput,Recall with the header written when the file is new
// (include/common.hpp:68-94).
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

template <typename T>
struct VecFile {
    size_t count = 0;
    int dim = 0;
    std::vector<T> values;
};

template <typename T>
inline VecFile<T> read_vecs(const std::string &path, const char *label) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) {
        fprintf(stderr, "Error: cannot open %s\n", path.c_str());
        exit(1);
    }
    const size_t size = static_cast<size_t>(f.tellg());
    f.seekg(0);
    VecFile<T> v;
    if (size >= sizeof(int32_t)) f.read(reinterpret_cast<char *>(&v.dim), sizeof(int32_t));
    const size_t stride = sizeof(int32_t) + static_cast<size_t>(v.dim) * sizeof(T);
    v.count = stride ? size / stride : 0;
    v.values.resize(v.count * static_cast<size_t>(v.dim));
    f.seekg(0);
    for (size_t i = 0; i < v.count; ++i) {
        int32_t d = 0;
        f.read(reinterpret_cast<char *>(&d), sizeof(d));
        if (d != v.dim) {
            fprintf(stderr, "Error: %s row %zu has dimension %d, expected %d\n", path.c_str(), i, d, v.dim);
            exit(1);
        }
        f.read(reinterpret_cast<char *>(v.values.data() + i * v.dim), static_cast<std::streamsize>(v.dim * sizeof(T)));
    }
    printf("Loading %s: n=%zu, dim=%d\n", label, v.count, v.dim);
    return v;
}

inline float recall_at_k(const uint32_t *pred, const int32_t *gt, size_t nq, int k, int gt_k) {
    const int eval = k < gt_k ? k : gt_k;
    size_t hit = 0;
    for (size_t q = 0; q < nq; ++q) {
        const int32_t *g = gt + q * static_cast<size_t>(gt_k);
        for (int j = 0; j < k; ++j) {
            const int p = static_cast<int>(pred[q * static_cast<size_t>(k) + j]);
            for (int t = 0; t < eval; ++t)
                if (g[t] == p) {
                    ++hit;
                    break;
                }
        }
    }
    return static_cast<float>(hit) / static_cast<float>(nq * static_cast<size_t>(k));
}

inline void append_csv_row(const std::string &path, int k, int beam, double runtime, double latency, double qps,
                           double recall) {
    std::ifstream probe(path);
    const bool exists = probe.good();
    probe.close();
    std::ofstream out(path, std::ios::app);
    if (!out) {
        fprintf(stderr, "Error: cannot open CSV file %s\n", path.c_str());
        return;
    }
    if (!exists) out << "TopK,Beam_size,Runtime,Latency,Throughput,Recall\n";
    out << k << "," << beam << "," << runtime << "," << latency << "," << qps << "," << recall << "\n";
}
