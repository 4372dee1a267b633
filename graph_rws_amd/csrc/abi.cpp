// Host-side C ABI pieces: error reporting, version, and the host-core
// CSR->BCSR converter that replaces core_lib.csr_to_bcsr_cpu
// (core/wrapper/convert_wrapper.cpp:27-180).
#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "grws_host.h"

namespace grws {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

namespace {

// Dynamic parallel-for over [0, n) in chunks, on plain threads (the library
// must not bring its own OpenMP runtime into a torch process).
template <typename F>
void parallel_for(int64_t n, int64_t chunk, int nthreads, F&& f) {
    if (nthreads <= 0) {
        unsigned hc = std::thread::hardware_concurrency();
        nthreads = hc ? (int)hc : 1;
    }
    int64_t nchunks = (n + chunk - 1) / chunk;
    if (nthreads > nchunks) nthreads = (int)std::max<int64_t>(1, nchunks);
    std::atomic<int64_t> next{0};
    auto worker = [&]() {
        std::vector<int32_t> scratch;
        for (;;) {
            int64_t c = next.fetch_add(1);
            if (c >= nchunks) break;
            int64_t b = c * chunk, e = std::min(n, b + chunk);
            for (int64_t i = b; i < e; ++i) f(i, scratch);
        }
    };
    if (nthreads == 1) {
        worker();
        return;
    }
    std::vector<std::thread> th;
    th.reserve(nthreads - 1);
    for (int t = 0; t < nthreads - 1; ++t) th.emplace_back(worker);
    worker();
    for (auto& t : th) t.join();
}

// Sorted unique columns of rows [r0, r1) into `u`.
void window_unique(const int64_t* row_ptr, const int32_t* col_idx, int64_t r0, int64_t r1,
                   std::vector<int32_t>& u) {
    u.assign(col_idx + row_ptr[r0], col_idx + row_ptr[r1]);
    std::sort(u.begin(), u.end());
    u.erase(std::unique(u.begin(), u.end()), u.end());
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" const char* grws_last_error(void) { return g_last_error.c_str(); }

extern "C" int grws_abi_version(void) { return GRWS_ABI_VERSION; }

extern "C" int grws_csr_to_bcsr_host_count(int64_t num_rows, const int64_t* row_ptr, const int32_t* col_idx,
                                           int32_t tile_rows, int32_t tile_cols, int64_t* window_offset,
                                           int64_t* num_tiles_out, int32_t num_threads) {
    clear_error();
    GRWS_CHECK_ARG(num_rows >= 0, "csr_to_bcsr: negative num_rows");
    GRWS_CHECK_ARG(tile_rows > 0 && tile_cols > 0, "csr_to_bcsr: tile sizes must be positive");
    GRWS_CHECK_ARG(row_ptr && window_offset && num_tiles_out, "csr_to_bcsr: null pointer");
    const int64_t W = (num_rows + tile_rows - 1) / tile_rows;
    if (row_ptr[num_rows] > 0) GRWS_CHECK_ARG(col_idx != nullptr, "csr_to_bcsr: null col_idx");
    for (int64_t r = 0; r < num_rows; ++r)
        if (row_ptr[r + 1] < row_ptr[r]) return set_error(GRWS_E_RANGE, "csr_to_bcsr: row_ptr decreases at row %lld", (long long)r);
    window_offset[0] = 0;
    parallel_for(W, 64, num_threads, [&](int64_t w, std::vector<int32_t>& u) {
        int64_t r0 = w * tile_rows, r1 = std::min(r0 + tile_rows, num_rows);
        window_unique(row_ptr, col_idx, r0, r1, u);
        window_offset[w + 1] = ((int64_t)u.size() + tile_cols - 1) / tile_cols;
    });
    for (int64_t w = 0; w < W; ++w) window_offset[w + 1] += window_offset[w];
    *num_tiles_out = window_offset[W];
    return GRWS_OK;
}

extern "C" int grws_csr_to_bcsr_host_fill(int64_t num_rows, const int64_t* row_ptr, const int32_t* col_idx,
                                          const float* values, int32_t tile_rows, int32_t tile_cols,
                                          const int64_t* window_offset, int32_t* col_indices, float* out_values,
                                          int32_t num_threads) {
    clear_error();
    GRWS_CHECK_ARG(num_rows >= 0, "csr_to_bcsr: negative num_rows");
    GRWS_CHECK_ARG(tile_rows > 0 && tile_cols > 0, "csr_to_bcsr: tile sizes must be positive");
    GRWS_CHECK_ARG(row_ptr && window_offset, "csr_to_bcsr: null pointer");
    const int64_t W = (num_rows + tile_rows - 1) / tile_rows;
    const int64_t T = window_offset[W];
    if (T > 0) GRWS_CHECK_ARG(col_indices && out_values, "csr_to_bcsr: null output");
    if (row_ptr[num_rows] > 0) GRWS_CHECK_ARG(col_idx && values, "csr_to_bcsr: null input");
    std::fill(col_indices, col_indices + T * tile_cols, -1);
    std::fill(out_values, out_values + T * tile_rows * tile_cols, 0.0f);
    const int64_t tile_elems = (int64_t)tile_rows * tile_cols;
    parallel_for(W, 64, num_threads, [&](int64_t w, std::vector<int32_t>& u) {
        int64_t t0 = window_offset[w];
        if (window_offset[w + 1] == t0) return;
        int64_t r0 = w * tile_rows, r1 = std::min(r0 + tile_rows, num_rows);
        window_unique(row_ptr, col_idx, r0, r1, u);
        std::copy(u.begin(), u.end(), col_indices + t0 * tile_cols);
        for (int64_t r = r0; r < r1; ++r) {
            for (int64_t e = row_ptr[r]; e < row_ptr[r + 1]; ++e) {
                int64_t pos = std::lower_bound(u.begin(), u.end(), col_idx[e]) - u.begin();
                out_values[(t0 + pos / tile_cols) * tile_elems + (r - r0) * tile_cols + pos % tile_cols] = values[e];
            }
        }
    });
    return GRWS_OK;
}
