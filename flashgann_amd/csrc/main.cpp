// gpu_flashgann -- command-line front end with the reference's interface
// (main.cu:11-109):
//   gpu_flashgann <data.fvecs> <query.fvecs> <gt.ivecs> <qg_codebook>
//                 [K=100] [beam_size=128] [degree=32] [-csv output.csv]
// Same argument handling, validation exits, printed results and CSV row.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "host_io.hpp"
#include "qg_host.hpp"

static int metric_from_path(const std::string &path) {  // include/metric.hpp:13-28
    std::string lower = path;
    for (char &c : lower) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
    return lower.find("text2image1m") != std::string::npos ? FG_METRIC_IP : FG_METRIC_L2;
}

int main(int argc, char **argv) {
    if (argc < 5) {
        fprintf(stderr,
                "Usage: %s <data.fvecs> <query.fvecs> <gt.ivecs> <qg_codebook> [K=100] [beam_size=128] [degree=32] "
                "[-csv output.csv]\n",
                argv[0]);
        return 1;
    }
    const char *data_file = argv[1];
    const char *query_file = argv[2];
    const char *gt_file = argv[3];
    const char *codebook = argv[4];
    int K = 100, beam = 128, degree = 32;
    std::string csv;
    int a = 5;
    if (a < argc && argv[a][0] != '-') K = atoi(argv[a++]);
    if (a < argc && argv[a][0] != '-') beam = atoi(argv[a++]);
    if (a < argc && argv[a][0] != '-') degree = atoi(argv[a++]);
    for (; a < argc; ++a) {
        const std::string arg = argv[a];
        if (arg == "-csv" && a + 1 < argc) {
            csv = argv[++a];
        } else {
            fprintf(stderr, "Unknown argument: %s\n", arg.c_str());
            return 1;
        }
    }
    printf("========================================\n");
    printf("FlashGANN AP Loading from:\n");
    printf("========================================\n");
    printf("Data file: %s\n", data_file);
    printf("Query file: %s\n", query_file);
    printf("Ground truth: %s\n", gt_file);
    printf("QG codebook: %s\n", codebook);
    printf("K: %d\n", K);
    printf("Beam size: %d\n", beam);
    printf("Degree: %d\n", degree);
    if (!csv.empty()) printf("CSV output: %s\n", csv.c_str());
    const int metric = metric_from_path(data_file);
    printf("Metric: %s\n", metric == FG_METRIC_IP ? "ip" : "l2");
    printf("========================================\n\n");

    VecFile<float> base = read_vecs<float>(data_file, "data");
    VecFile<float> queries = read_vecs<float>(query_file, "queries");
    VecFile<int32_t> gt = read_vecs<int32_t>(gt_file, "ground truth");
    const size_t nq = queries.count;
    if (queries.dim != base.dim) {
        fprintf(stderr, "Query dimension %d does not match data dimension %d\n", queries.dim, base.dim);
        return 1;
    }
    if (gt.count != nq) {
        fprintf(stderr, "Ground-truth query count %zu does not match query count %zu\n", gt.count, nq);
        return 1;
    }

    std::vector<vidType> results(nq * static_cast<size_t>(K));
    double elapsed = 0.0;
    QuantizationGraph qg(base.count, static_cast<size_t>(base.dim), degree, codebook);
    qg.set_metric(metric);
    qg.gpu_search_adaptive(static_cast<int>(nq), queries.values.data(), K, results.data(), beam, elapsed);

    const float recall = recall_at_k(results.data(), gt.values.data(), nq, K, gt.dim) * 100.0f;
    const double latency_ms = nq > 0 ? elapsed * 1000.0 / static_cast<double>(nq) : 0.0;
    const double qps = elapsed > 0.0 ? static_cast<double>(nq) / elapsed : 0.0;
    printf("\n========================================\n");
    printf("Results\n");
    printf("========================================\n");
    printf("Total time: %.6f ms\n", elapsed * 1000.0);
    printf("Throughput: %.6f queries/sec\n", qps);
    printf("Avg latency: %.6f ms/query\n", latency_ms);
    printf("Recall@%d: %.6f\n", K, recall);
    printf("========================================\n");
    if (!csv.empty()) {
        append_csv_row(csv, K, beam, elapsed, latency_ms, qps, recall);
        printf("Saved GPU stats CSV row to: %s\n", csv.c_str());
    }
    return 0;
}
