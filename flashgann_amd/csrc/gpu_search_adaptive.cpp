// Drop-in replacement for the reference's gpu_search_adaptive.cu: the
// definition of QuantizationGraph::gpu_search_adaptive (include/qg.hpp:62-63)
// on the C ABI of libflashgann.so.  Compiled against the reference's own
// include/qg.hpp and linked with its unchanged main.cu, it moves that program
// to the MI355X search without touching any other file:
//
//   g++ -std=c++20 -O2 -I<reference> -I<this repo> -x c++ <reference>/main.cu \
//       -x none flashgann_amd/csrc/gpu_search_adaptive.cpp \
//       -Lflashgann_amd -lflashgann -L/opt/rocm/lib -lamdhip64
//
// Like gpu_search_adaptive.cu:65-71, 110-113 it uploads the codebook on every
// call and frees it afterwards, so it keeps no state between calls or
// instances (qg_host.hpp's class keeps the index resident instead).  The
// entry-point fallback (:74-77) runs inside fg_index_create; the error
// behaviour follows the reference: a device-memory shortfall throws
// std::runtime_error (:61-63), any other failure prints and exits
// (CUDA_SAFE_CALL, utils.cuh:42-50); `elapsed` is the wall clock around
// launch + synchronise (:98-107).
#include <cstdio>
#include <cstdlib>
#include <stdexcept>

#include "include/flashgann.h"
#include "include/qg.hpp"

namespace {

void fg_check(int rc, const char *what) {
    if (rc == FG_OK) return;
    if (rc == FG_ENOMEM) throw std::runtime_error(fg_last_error());
    fprintf(stderr, "%s failed (%d): %s\n", what, rc, fg_last_error());
    exit(EXIT_FAILURE);
}

}  // namespace

void QuantizationGraph::gpu_search_adaptive(int nq, const float *queries, int K, vidType *result_idx, int beam_sz,
                                            double &elapsed) {
    printf("\nGPU adaptive search (flashgann-amd, %s): K=%d, nq=%d, dim=%zu, npoints=%zu, beam_size=%d\n",
           fg_version(), K, nq, dim_, num_nodes_, beam_sz);
    printf("Metric: %s\n", metric_name(get_metric()));
    if (nq < 0 || K < 1 || beam_sz < 1) fg_check(FG_EINVAL, "argument check");
    fg_index *ix = nullptr;
    fg_check(fg_index_create(get_data_ptr(), num_nodes_, static_cast<uint32_t>(dim_), static_cast<uint32_t>(degree_),
                             get_signs_ptr(), get_entry_point(),
                             get_metric() == METRIC_IP ? FG_METRIC_IP : FG_METRIC_L2, &ix),
             "codebook upload");
    fg_index_info info;
    fg_check(fg_index_get_info(ix, &info), "index info");
    printf("GPU adaptive search entry point: %u\n", info.entry);
    fg_stats st;
    const int rc = fg_search(ix, queries, static_cast<uint32_t>(nq), static_cast<uint32_t>(K),
                             static_cast<uint32_t>(beam_sz), result_idx, nullptr, &st);
    fg_index_destroy(ix);
    fg_check(rc, "search");
    printf("Dynamic shared memory size = %u bytes\n", st.lds_bytes);
    elapsed = st.elapsed_s;
}
