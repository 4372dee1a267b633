// Sanitizer check of the host-side code (built by tests/sanitize/Makefile with
// -fsanitize=address,undefined): the product's CSR -> BCSR converter
// (graph_rws_amd/csrc/abi.cpp, the replacement of convert_wrapper.cpp:27-180)
// against the C oracle's restatement on random CSR graphs (empty rows,
// duplicate edges, rectangular, 1-2 tile widths, 1 or 3 threads), plus its
// error paths.  Exit status 0 and "host_check: ... ok" when every case matches.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "grws.h"

extern "C" {
int64_t orc_csr_to_bcsr_count(int64_t num_rows, const int64_t* row_ptr, const int32_t* col_idx, int64_t tile_rows,
                              int64_t tile_cols, int64_t* win_off);
void orc_csr_to_bcsr_fill(int64_t num_rows, const int64_t* row_ptr, const int32_t* col_idx, const double* values,
                          int64_t tile_rows, int64_t tile_cols, const int64_t* win_off, int32_t* out_cols,
                          double* out_vals);
}

static int fail(const char* what, int c) {
    std::fprintf(stderr, "host_check: case %d: %s\n", c, what);
    return 1;
}

int main() {
    std::mt19937_64 rng(12345);
    int cases = 0;
    for (int c = 0; c < 400; ++c) {
        const int64_t rows = (int64_t)(rng() % 300);
        const int64_t cols = 1 + (int64_t)(rng() % 500);
        const int64_t per = (int64_t)(rng() % 40);
        std::vector<int64_t> rp(rows + 1, 0);
        std::vector<int32_t> ci;
        std::vector<float> va;
        for (int64_t r = 0; r < rows; ++r) {
            const int64_t d = (rng() % 7 == 0) ? 0 : (int64_t)(rng() % (per + 1));
            for (int64_t e = 0; e < d; ++e) {
                ci.push_back((int32_t)(rng() % cols));
                va.push_back((float)((int64_t)(rng() % 2001) - 1000) / 64.0f);
            }
            rp[r + 1] = (int64_t)ci.size();
        }
        std::vector<double> vd(va.begin(), va.end());
        for (int tc : {8, 16}) {
            for (int threads : {1, 3}) {
                const int64_t W = (rows + 15) / 16;
                std::vector<int64_t> win(W + 1), owin(W + 1);
                int64_t T = -1;
                if (grws_csr_to_bcsr_host_count(rows, rp.data(), ci.empty() ? nullptr : ci.data(), 16, tc,
                                                win.data(), &T, threads) != GRWS_OK)
                    return fail(grws_last_error(), c);
                const int64_t oT = orc_csr_to_bcsr_count(rows, rp.data(), ci.data(), 16, tc, owin.data());
                if (T != oT || win != owin) return fail("tile counts differ", c);
                std::vector<int32_t> oc(T * tc + 1), hc(T * tc + 1);
                std::vector<double> ov(T * 16 * tc + 1);
                std::vector<float> hv(T * 16 * tc + 1);
                orc_csr_to_bcsr_fill(rows, rp.data(), ci.data(), vd.data(), 16, tc, owin.data(), oc.data(), ov.data());
                if (grws_csr_to_bcsr_host_fill(rows, rp.data(), ci.empty() ? nullptr : ci.data(),
                                               va.empty() ? nullptr : va.data(), 16, tc, win.data(), hc.data(),
                                               hv.data(), threads) != GRWS_OK)
                    return fail(grws_last_error(), c);
                for (int64_t i = 0; i < T * tc; ++i)
                    if (hc[i] != oc[i]) return fail("columns differ", c);
                for (int64_t i = 0; i < T * 16 * tc; ++i)
                    if ((double)hv[i] != ov[i]) return fail("values differ", c);
                ++cases;
            }
        }
    }
    // error paths
    int64_t win[4], T;
    int64_t bad_rp[3] = {0, 3, 2};
    int32_t ci[3] = {0, 1, 2};
    if (grws_csr_to_bcsr_host_count(2, bad_rp, ci, 16, 8, win, &T, 1) != GRWS_E_RANGE) return fail("decreasing row_ptr", -1);
    if (grws_csr_to_bcsr_host_count(-1, bad_rp, ci, 16, 8, win, &T, 1) != GRWS_E_INVALID) return fail("negative rows", -1);
    if (grws_csr_to_bcsr_host_count(2, nullptr, ci, 16, 8, win, &T, 1) != GRWS_E_INVALID) return fail("null row_ptr", -1);
    if (std::strlen(grws_last_error()) == 0) return fail("no message", -1);
    std::printf("host_check: %d converter cases and 3 error paths ok\n", cases);
    return 0;
}
