/*
 * grws_oracle.c -- CPU restatement of the Graph_RWS hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in graph_rws_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or as the
 * timed CPU baseline.  The product path never links or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Plain C11 (+ optional OpenMP), no dependencies.  Built by oracle/Makefile
 * into oracle/liboracle.so and loaded through oracle/__init__.py (ctypes).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* small helpers                                                             */
/* ------------------------------------------------------------------------ */
static int cmp_i32(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

/* sort + unique of a window's columns; returns the unique count.
 * Restates convert_wrapper.cpp:67-83 (gather, std::sort, std::unique). */
static int64_t window_unique_cols(const int64_t* row_ptr, const int32_t* col_idx,
                                  int64_t r_start, int64_t r_end, int32_t** out) {
    int64_t e0 = row_ptr[r_start], e1 = row_ptr[r_end];
    int64_t n = e1 - e0;
    *out = NULL;
    if (n <= 0) return 0;
    int32_t* buf = (int32_t*)malloc((size_t)n * sizeof(int32_t));
    memcpy(buf, col_idx + e0, (size_t)n * sizeof(int32_t));
    qsort(buf, (size_t)n, sizeof(int32_t), cmp_i32);
    int64_t u = 0;
    for (int64_t i = 0; i < n; ++i)
        if (i == 0 || buf[i] != buf[u - 1]) buf[u++] = buf[i];
    *out = buf;
    return u;
}

static int64_t lower_bound_i32(const int32_t* a, int64_t n, int32_t v) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        int64_t mid = lo + (hi - lo) / 2;
        if (a[mid] < v) lo = mid + 1; else hi = mid;
    }
    return lo;
}

/* ------------------------------------------------------------------------ */
/* CSR -> BCSR  (convert_wrapper.cpp:27-180)                                 */
/* ------------------------------------------------------------------------ */

/* Phase 1 + 1.5 (convert_wrapper.cpp:58-100): tiles per window, prefix sum.
 * win_off has num_windows+1 entries.  Returns total tiles. */
ORC_API int64_t orc_csr_to_bcsr_count(int64_t num_rows, const int64_t* row_ptr,
                                      const int32_t* col_idx, int64_t tile_rows,
                                      int64_t tile_cols, int64_t* win_off) {
    int64_t W = (num_rows + tile_rows - 1) / tile_rows;
    win_off[0] = 0;
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t w = 0; w < W; ++w) {
        int64_t r0 = w * tile_rows;
        int64_t r1 = r0 + tile_rows < num_rows ? r0 + tile_rows : num_rows;
        int32_t* u = NULL;
        int64_t nu = window_unique_cols(row_ptr, col_idx, r0, r1, &u);
        free(u);
        win_off[w + 1] = (nu + tile_cols - 1) / tile_cols;
    }
    for (int64_t w = 0; w < W; ++w) win_off[w + 1] += win_off[w];
    return win_off[W];
}

/* Phase 2 (convert_wrapper.cpp:102-177): cols filled with -1 and values with
 * 0, then each window's sorted unique columns are written and every CSR edge
 * is scattered to [tile][row][col] via lower_bound.  Duplicate (r,c) edges:
 * the last one in CSR order wins (plain store, :174).  vals is float64 so the
 * oracle can carry any input precision exactly. */
ORC_API void orc_csr_to_bcsr_fill(int64_t num_rows, const int64_t* row_ptr,
                                  const int32_t* col_idx, const double* values,
                                  int64_t tile_rows, int64_t tile_cols,
                                  const int64_t* win_off, int32_t* out_cols,
                                  double* out_vals) {
    int64_t W = (num_rows + tile_rows - 1) / tile_rows;
    int64_t T = win_off[W];
    for (int64_t i = 0; i < T * tile_cols; ++i) out_cols[i] = -1;
    for (int64_t i = 0; i < T * tile_rows * tile_cols; ++i) out_vals[i] = 0.0;
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t w = 0; w < W; ++w) {
        int64_t t0 = win_off[w];
        if (win_off[w + 1] == t0) continue;
        int64_t r0 = w * tile_rows;
        int64_t r1 = r0 + tile_rows < num_rows ? r0 + tile_rows : num_rows;
        int32_t* u = NULL;
        int64_t nu = window_unique_cols(row_ptr, col_idx, r0, r1, &u);
        for (int64_t i = 0; i < nu; ++i) out_cols[t0 * tile_cols + i] = u[i];
        for (int64_t r = r0; r < r1; ++r) {
            for (int64_t e = row_ptr[r]; e < row_ptr[r + 1]; ++e) {
                int64_t pos = lower_bound_i32(u, nu, col_idx[e]);
                int64_t tile = t0 + pos / tile_cols;
                int64_t c = pos % tile_cols;
                out_vals[tile * tile_rows * tile_cols + (r - r0) * tile_cols + c] = values[e];
            }
        }
        free(u);
    }
}

/* ------------------------------------------------------------------------ */
/* BCSR SpMM forward  (spmm_tc.cuh:113-193 semantics, every output column)   */
/* ------------------------------------------------------------------------ */

/* Y[16W x N] = A * X in float64.  Also returns AX_abs = |A|*|X| (the
 * elementwise error scale used by the parity tolerance).  Column slots equal
 * to -1 contribute nothing (spmm_tc.cuh:130-141).  A column outside
 * [0, x_rows) also contributes nothing: the reference kernel would read out
 * of bounds there, and its model layer masks such columns to zero before the
 * call (model.py:118-125).  Output rows are zero-initialised
 * (spmm_wrapper.cu:63). */
ORC_API void orc_bcsr_spmm_f64(int64_t W, const int64_t* win_off, const int32_t* cols,
                               const double* vals, int64_t tile_rows, int64_t tile_cols,
                               const double* X, int64_t x_rows, int64_t ldx, int64_t N,
                               double* Y, double* AX_abs) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t w = 0; w < W; ++w) {
        for (int64_t r = 0; r < tile_rows; ++r) {
            double* y = Y + (w * tile_rows + r) * N;
            double* ya = AX_abs ? AX_abs + (w * tile_rows + r) * N : NULL;
            for (int64_t n = 0; n < N; ++n) { y[n] = 0.0; if (ya) ya[n] = 0.0; }
            for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
                for (int64_t c = 0; c < tile_cols; ++c) {
                    int32_t col = cols[t * tile_cols + c];
                    if (col < 0 || col >= x_rows) continue;
                    double a = vals[(t * tile_rows + r) * tile_cols + c];
                    const double* x = X + (int64_t)col * ldx;
                    for (int64_t n = 0; n < N; ++n) {
                        y[n] += a * x[n];
                        if (ya) ya[n] += fabs(a) * fabs(x[n]);
                    }
                }
            }
        }
    }
}

/* The same product in float32 with fp32 accumulation: the timed CPU baseline
 * (the reference has no CPU SpMM; this is its kernel's arithmetic restated on
 * host cores).  Processes windows [w_begin, w_end) only, so a bounded sample
 * of a large workload can be timed. */
ORC_API void orc_bcsr_spmm_f32(int64_t w_begin, int64_t w_end, const int64_t* win_off,
                               const int32_t* cols, const float* vals, int64_t tile_rows,
                               int64_t tile_cols, const float* X, int64_t x_rows, int64_t ldx,
                               int64_t N, float* Y) {
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t w = w_begin; w < w_end; ++w) {
        float* yw = Y + (w - w_begin) * tile_rows * N;
        for (int64_t i = 0; i < tile_rows * N; ++i) yw[i] = 0.0f;
        for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
            for (int64_t c = 0; c < tile_cols; ++c) {
                int32_t col = cols[t * tile_cols + c];
                if (col < 0 || col >= x_rows) continue;
                const float* x = X + (int64_t)col * ldx;
                for (int64_t r = 0; r < tile_rows; ++r) {
                    float a = vals[(t * tile_rows + r) * tile_cols + c];
                    if (a == 0.0f) continue;
                    float* y = yw + r * N;
                    for (int64_t n = 0; n < N; ++n) y[n] += a * x[n];
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Full-size checks: the same products on the stored element types, over a  */
/* subset of windows or projected onto one vector, so graphs whose values    */
/* would not fit in memory as float64 (c3: 1.2G slots) can be checked.       */
/* Element types: 0 = float32, 1 = float16, 2 = bfloat16 (raw bits).         */
/* ------------------------------------------------------------------------ */

/* IEEE binary16 bits -> double, exactly (normals, subnormals, inf, NaN). */
static double half_bits_to_double(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 1024), e - 25);
    return s ? -v : v;
}

/* bfloat16 bits -> double, exactly (the high half of a float32). */
static double bf16_bits_to_double(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

/* Table of the 65536 values of a 16-bit type (dt 1 or 2), or NULL for f32. */
static double* elem_table(int32_t dt) {
    if (dt != 1 && dt != 2) return NULL;
    double* t = (double*)malloc(65536 * sizeof(double));
    for (uint32_t i = 0; i < 65536; ++i)
        t[i] = dt == 1 ? half_bits_to_double((uint16_t)i) : bf16_bits_to_double((uint16_t)i);
    return t;
}

static inline double elem_at(const void* p, const double* tab, int64_t i) {
    if (tab) return tab[((const uint16_t*)p)[i]];
    return (double)((const float*)p)[i];
}

/* Rows of Y = A X (and |A||X|) for the windows sel[0..nsel), in float64 on
 * the stored values and features: output row 16k + r is row r of window
 * sel[k] (spmm_tc.cuh:113-193 semantics as orc_bcsr_spmm_f64: -1 and
 * columns outside [0, x_rows) contribute nothing). */
ORC_API void orc_bcsr_spmm_windows_f64(int64_t nsel, const int64_t* sel, const int64_t* win_off,
                                       const int32_t* cols, const void* vals, int32_t vdt,
                                       int64_t tile_rows, int64_t tile_cols, const void* X,
                                       int32_t xdt, int64_t x_rows, int64_t ldx, int64_t N,
                                       double* Y, double* AX_abs) {
    double* vt = elem_table(vdt);
    double* xt = elem_table(xdt);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t k = 0; k < nsel; ++k) {
        const int64_t w = sel[k];
        double* yw = Y + k * tile_rows * N;
        double* aw = AX_abs + k * tile_rows * N;
        for (int64_t i = 0; i < tile_rows * N; ++i) { yw[i] = 0.0; aw[i] = 0.0; }
        for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
            for (int64_t c = 0; c < tile_cols; ++c) {
                const int32_t col = cols[t * tile_cols + c];
                if (col < 0 || col >= x_rows) continue;
                for (int64_t r = 0; r < tile_rows; ++r) {
                    const double a = elem_at(vals, vt, (t * tile_rows + r) * tile_cols + c);
                    if (a == 0.0) continue;
                    double* y = yw + r * N;
                    double* ya = aw + r * N;
                    const int64_t xo = (int64_t)col * ldx;
                    for (int64_t n = 0; n < N; ++n) {
                        const double x = elem_at(X, xt, xo + n);
                        y[n] += a * x;
                        ya[n] += fabs(a) * fabs(x);
                    }
                }
            }
        }
    }
    free(vt);
    free(xt);
}

/* z = A v and z_abs = |A| v_abs over all 16W rows, in float64 on the stored
 * values (v = X r projects the product onto r: (A X) r = A (X r)). */
ORC_API void orc_bcsr_spmv_f64(int64_t W, const int64_t* win_off, const int32_t* cols,
                               const void* vals, int32_t vdt, int64_t tile_rows, int64_t tile_cols,
                               const double* v, const double* v_abs, int64_t x_rows, double* z,
                               double* z_abs) {
    double* vt = elem_table(vdt);
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t w = 0; w < W; ++w) {
        double acc[64], acca[64];
        for (int64_t r = 0; r < tile_rows; ++r) { acc[r] = 0.0; acca[r] = 0.0; }
        for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
            for (int64_t c = 0; c < tile_cols; ++c) {
                const int32_t col = cols[t * tile_cols + c];
                if (col < 0 || col >= x_rows) continue;
                for (int64_t r = 0; r < tile_rows; ++r) {
                    const double a = elem_at(vals, vt, (t * tile_rows + r) * tile_cols + c);
                    acc[r] += a * v[col];
                    acca[r] += fabs(a) * v_abs[col];
                }
            }
        }
        for (int64_t r = 0; r < tile_rows; ++r) {
            z[w * tile_rows + r] = acc[r];
            z_abs[w * tile_rows + r] = acca[r];
        }
    }
    free(vt);
}

/* z = A^T u and z_abs = |A|^T u_abs over num_cols outputs (u has 16W rows):
 * the projection of A^T G onto r when u = G r (spmm_tc.cuh:238-269
 * semantics).  Per-thread partial vectors, added afterwards. */
ORC_API void orc_bcsr_spmv_t_f64(int64_t W, const int64_t* win_off, const int32_t* cols,
                                 const void* vals, int32_t vdt, int64_t tile_rows,
                                 int64_t tile_cols, const double* u, const double* u_abs,
                                 int64_t num_cols, double* z, double* z_abs) {
    double* vt = elem_table(vdt);
    for (int64_t i = 0; i < num_cols; ++i) { z[i] = 0.0; z_abs[i] = 0.0; }
#pragma omp parallel
    {
        double* pz = (double*)calloc((size_t)num_cols, sizeof(double));
        double* pa = (double*)calloc((size_t)num_cols, sizeof(double));
#pragma omp for schedule(dynamic, 64)
        for (int64_t w = 0; w < W; ++w) {
            for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
                for (int64_t c = 0; c < tile_cols; ++c) {
                    const int32_t col = cols[t * tile_cols + c];
                    if (col < 0 || col >= num_cols) continue;
                    double s = 0.0, sa = 0.0;
                    for (int64_t r = 0; r < tile_rows; ++r) {
                        const double a = elem_at(vals, vt, (t * tile_rows + r) * tile_cols + c);
                        s += a * u[w * tile_rows + r];
                        sa += fabs(a) * u_abs[w * tile_rows + r];
                    }
                    pz[col] += s;
                    pa[col] += sa;
                }
            }
        }
#pragma omp critical
        {
            for (int64_t i = 0; i < num_cols; ++i) { z[i] += pz[i]; z_abs[i] += pa[i]; }
        }
        free(pz);
        free(pa);
    }
    free(vt);
}

/* Selected rows of A^T G: out row map[col] (>= 0) receives sum_r A[r][col]
 * G[r] over every stored slot of that column, out_abs the same with
 * absolute values; columns with map[col] < 0 are skipped.  G is [16W, ldg]
 * of type gdt.  Per-thread partial outputs, added afterwards. */
ORC_API void orc_bcsr_spmm_t_rows_f64(int64_t W, const int64_t* win_off, const int32_t* cols,
                                      const void* vals, int32_t vdt, int64_t tile_rows,
                                      int64_t tile_cols, const void* G, int32_t gdt, int64_t ldg,
                                      int64_t D, int64_t num_cols, const int32_t* map,
                                      int64_t nout, double* out, double* out_abs) {
    double* vt = elem_table(vdt);
    double* gt = elem_table(gdt);
    for (int64_t i = 0; i < nout * D; ++i) { out[i] = 0.0; out_abs[i] = 0.0; }
#pragma omp parallel
    {
        double* po = (double*)calloc((size_t)(nout * D), sizeof(double));
        double* pa = (double*)calloc((size_t)(nout * D), sizeof(double));
#pragma omp for schedule(dynamic, 64)
        for (int64_t w = 0; w < W; ++w) {
            for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
                for (int64_t c = 0; c < tile_cols; ++c) {
                    const int32_t col = cols[t * tile_cols + c];
                    if (col < 0 || col >= num_cols || map[col] < 0) continue;
                    double* o = po + (int64_t)map[col] * D;
                    double* oa = pa + (int64_t)map[col] * D;
                    for (int64_t r = 0; r < tile_rows; ++r) {
                        const double a = elem_at(vals, vt, (t * tile_rows + r) * tile_cols + c);
                        if (a == 0.0) continue;
                        const int64_t go = (w * tile_rows + r) * ldg;
                        for (int64_t f = 0; f < D; ++f) {
                            const double g = elem_at(G, gt, go + f);
                            o[f] += a * g;
                            oa[f] += fabs(a) * fabs(g);
                        }
                    }
                }
            }
        }
#pragma omp critical
        {
            for (int64_t i = 0; i < nout * D; ++i) { out[i] += po[i]; out_abs[i] += pa[i]; }
        }
        free(po);
        free(pa);
    }
    free(vt);
    free(gt);
}

/* ------------------------------------------------------------------------ */
/* BCSR SpMM transpose  (spmm_tc.cuh:211-270 semantics)                      */
/* ------------------------------------------------------------------------ */

/* G_in[num_cols x D] = A^T * G_out, G_out is [16W x D].  Restates the atomic
 * scatter grad_in[col][f] += w * g[row][f] over all tiles/rows/cols with
 * col != -1 and w != 0 (spmm_tc.cuh:238-266), in exact float64 and without
 * the reference's |g| < 1e-9 skip (:250), its int32 index math (:247,265) and
 * its D > 1024 truncation (spmm_wrapper.cu:131-132).  Columns outside
 * [0, num_cols) are ignored.  Serial so the summation order is fixed. */
ORC_API void orc_bcsr_spmm_t_f64(int64_t W, const int64_t* win_off, const int32_t* cols,
                                 const double* vals, int64_t tile_rows, int64_t tile_cols,
                                 const double* G, int64_t ldg, int64_t D, int64_t num_cols,
                                 double* Gin, double* Gin_abs) {
    for (int64_t i = 0; i < num_cols * D; ++i) { Gin[i] = 0.0; if (Gin_abs) Gin_abs[i] = 0.0; }
    for (int64_t w = 0; w < W; ++w) {
        for (int64_t t = win_off[w]; t < win_off[w + 1]; ++t) {
            for (int64_t r = 0; r < tile_rows; ++r) {
                const double* g = G + (w * tile_rows + r) * ldg;
                for (int64_t c = 0; c < tile_cols; ++c) {
                    int32_t col = cols[t * tile_cols + c];
                    if (col < 0 || col >= num_cols) continue;
                    double a = vals[(t * tile_rows + r) * tile_cols + c];
                    if (a == 0.0) continue;
                    double* o = Gin + (int64_t)col * D;
                    double* oa = Gin_abs ? Gin_abs + (int64_t)col * D : NULL;
                    for (int64_t f = 0; f < D; ++f) {
                        o[f] += a * g[f];
                        if (oa) oa[f] += fabs(a) * fabs(g[f]);
                    }
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Reindex + prune  (reindex.cuh:33-102, reindex_wrapper.cu:27-68)           */
/* ------------------------------------------------------------------------ */

/* For every column slot: target window = col / tile_rows with C truncation
 * (so -1 maps to window 0 with in-window offset -1, reindex.cuh:49,89),
 * binary search in the sorted active_windows (:53-68).  Hit: idx*tile_rows +
 * col % tile_rows (:89).  Miss: column 0 and the tile_rows values of that
 * tile column set to 0 in place (:93-100). */
ORC_API void orc_reindex_prune(const int32_t* in_cols, int64_t num_indices, float* values,
                               const int32_t* active_windows, int64_t num_active,
                               int32_t tile_rows, int32_t tile_cols, int32_t* out_cols) {
    for (int64_t idx = 0; idx < num_indices; ++idx) {
        int32_t g = in_cols[idx];
        int32_t target = g / tile_rows;
        int64_t lo = 0, hi = num_active - 1, found = -1;
        while (lo <= hi) {
            int64_t mid = (lo + hi) / 2;
            int32_t win = active_windows[mid];
            if (win == target) { found = mid; break; }
            if (win < target) lo = mid + 1; else hi = mid - 1;
        }
        if (found != -1) {
            out_cols[idx] = (int32_t)(found * tile_rows + g % tile_rows);
        } else {
            out_cols[idx] = 0;
            int64_t blk = idx / tile_cols, cit = idx % tile_cols;
            for (int32_t r = 0; r < tile_rows; ++r)
                values[blk * tile_rows * tile_cols + (int64_t)r * tile_cols + cit] = 0.0f;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Philox4x32-10  (Salmon, Moraes, Dror, Shaw, SC'11 "Parallel random       */
/* numbers: as easy as 1, 2, 3").  No reference counterpart: the reference  */
/* has no RNG in core/ (grep), the node-wise sampler is new per north_star. */
/* ------------------------------------------------------------------------ */
ORC_API void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int round = 0; round < 10; ++round) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* The draw used by the node-wise sampler: word 0 of
 * Philox4x32-10(counter = (node_lo, node_hi, draw, 0), key = (seed_lo, seed_hi)). */
static inline uint32_t draw_word(uint64_t seed, uint64_t node, uint32_t draw) {
    uint32_t ctr[4] = {(uint32_t)node, (uint32_t)(node >> 32), draw, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    orc_philox4x32_10(ctr, key, out);
    return out[0];
}

ORC_API void orc_philox_draws(uint64_t seed, const int64_t* nodes, const uint32_t* draws,
                              int64_t n, uint32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = draw_word(seed, (uint64_t)nodes[i], draws[i]);
}

/* ------------------------------------------------------------------------ */
/* Node-wise fanout sampling without replacement (Floyd) + relabel.          */
/* New semantics per north_star (no reference function); the frontier /     */
/* source layout follows from_dgl_block (bcsr.py:266-306) and the target-top */
/* convention of layer.py:159-161.                                           */
/* ------------------------------------------------------------------------ */

/* Chooses min(deg, k) distinct CSR positions of `node` by Floyd's algorithm:
 * for j = deg-k .. deg-1 (draw index d = j-(deg-k)):
 *   t = (u64(philox(seed,node,d)) * (j+1)) >> 32
 *   S += (t in S) ? j : t
 * deg <= k takes every neighbour.  Output positions sorted ascending.
 * Returns the number chosen. */
static int floyd_positions(uint64_t seed, int64_t node, int64_t deg, int k, int64_t* pos) {
    if (deg <= k) {
        for (int64_t i = 0; i < deg; ++i) pos[i] = i;
        return (int)deg;
    }
    int cnt = 0;
    for (int64_t j = deg - k; j < deg; ++j) {
        uint32_t d = (uint32_t)(j - (deg - k));
        uint32_t u = draw_word(seed, (uint64_t)node, d);
        int64_t t = (int64_t)(((uint64_t)u * (uint64_t)(j + 1)) >> 32);
        int seen = 0;
        for (int i = 0; i < cnt; ++i) if (pos[i] == t) { seen = 1; break; }
        pos[cnt++] = seen ? j : t;
    }
    /* insertion sort, k <= 64 */
    for (int i = 1; i < cnt; ++i) {
        int64_t v = pos[i]; int j = i - 1;
        while (j >= 0 && pos[j] > v) { pos[j + 1] = pos[j]; --j; }
        pos[j + 1] = v;
    }
    return cnt;
}

/* One hop.  frontier[F] are global ids (local ids 0..F-1 in frontier order).
 * Output edges (dst_local, src_global) in frontier order then CSR-position
 * order; edge_count_out gets the total.  Caller sizes the edge buffers to
 * F*k.  Returns 0. */
ORC_API int64_t orc_sample_hop(const int64_t* indptr, const int32_t* indices, uint64_t seed,
                               const int64_t* frontier, int64_t F, int k,
                               int32_t* edge_dst, int64_t* edge_src) {
    int64_t e = 0;
    int64_t pos[64];
    for (int64_t i = 0; i < F; ++i) {
        int64_t v = frontier[i];
        int64_t deg = indptr[v + 1] - indptr[v];
        int cnt = floyd_positions(seed, v, deg, k, pos);
        for (int c = 0; c < cnt; ++c) {
            edge_dst[e] = (int32_t)i;
            edge_src[e] = (int64_t)indices[indptr[v] + pos[c]];
            ++e;
        }
    }
    return e;
}

static int cmp_i64(const void* a, const void* b) {
    int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
    return (x > y) - (x < y);
}

/* Relabel: frontier nodes keep local ids [0,F) in frontier order; source ids
 * not in the frontier are appended in ascending global id.  Writes
 * src_local[E] and the new source list (global ids, frontier first) to
 * next_frontier (capacity F+E).  Returns the number of source nodes. */
ORC_API int64_t orc_relabel(const int64_t* frontier, int64_t F, const int64_t* edge_src,
                            int64_t E, int32_t* src_local, int64_t* next_frontier) {
    /* sorted frontier copy with positions */
    int64_t* fs = (int64_t*)malloc((size_t)(F > 0 ? F : 1) * 2 * sizeof(int64_t));
    for (int64_t i = 0; i < F; ++i) { fs[2 * i] = frontier[i]; fs[2 * i + 1] = i; }
    /* sort pairs by id (ids in a frontier are distinct) */
    qsort(fs, (size_t)F, 2 * sizeof(int64_t), cmp_i64);
    int64_t* es = (int64_t*)malloc((size_t)(E > 0 ? E : 1) * sizeof(int64_t));
    memcpy(es, edge_src, (size_t)E * sizeof(int64_t));
    qsort(es, (size_t)E, sizeof(int64_t), cmp_i64);
    for (int64_t i = 0; i < F; ++i) next_frontier[i] = frontier[i];
    int64_t n = F;
    /* unique new ids ascending */
    int64_t* newids = (int64_t*)malloc((size_t)(E > 0 ? E : 1) * sizeof(int64_t));
    int64_t nn = 0;
    for (int64_t i = 0; i < E; ++i) {
        if (i > 0 && es[i] == es[i - 1]) continue;
        /* in frontier? */
        int64_t lo = 0, hi = F;
        while (lo < hi) { int64_t m = (lo + hi) / 2; if (fs[2 * m] < es[i]) lo = m + 1; else hi = m; }
        if (lo < F && fs[2 * lo] == es[i]) continue;
        newids[nn++] = es[i];
    }
    for (int64_t i = 0; i < nn; ++i) next_frontier[n++] = newids[i];
    for (int64_t i = 0; i < E; ++i) {
        int64_t v = edge_src[i];
        int64_t lo = 0, hi = F;
        while (lo < hi) { int64_t m = (lo + hi) / 2; if (fs[2 * m] < v) lo = m + 1; else hi = m; }
        if (lo < F && fs[2 * lo] == v) { src_local[i] = (int32_t)fs[2 * lo + 1]; continue; }
        lo = 0; hi = nn;
        while (lo < hi) { int64_t m = (lo + hi) / 2; if (newids[m] < v) lo = m + 1; else hi = m; }
        src_local[i] = (int32_t)(F + lo);
    }
    free(fs); free(es); free(newids);
    return n;
}

/* ------------------------------------------------------------------------ */
/* Window top-K sampling  (sampling.cuh:65-579, 707-773;                    */
/* sampling_wrapper.cu:58-347), restated step by step as the reference      */
/* executes it: per batch of warps_per_block tiles, per-tile candidate lists */
/* in element order, a single-threaded merge into the window list, a sort   */
/* by (total desc, column asc) with (INT_MAX, 0) padding, truncation to     */
/* CAP; finally an ascending sort by column and the first min(cnt, S).      */
/* ------------------------------------------------------------------------ */

/* C's (int) of a float as a GPU converts it (cvt.rzi.s32.f32 /             */
/* v_cvt_i32_f32): toward zero, saturating, NaN -> 0.                        */
static int32_t f2i_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

typedef struct { int32_t col; int32_t freq; } orc_cand;

/* ColumnCandidateComparator (sampling_helper.h:28-34) */
static int cmp_cand(const void* a, const void* b) {
    const orc_cand* x = (const orc_cand*)a;
    const orc_cand* y = (const orc_cand*)b;
    if (x->freq != y->freq) return x->freq > y->freq ? -1 : 1;
    return (x->col > y->col) - (x->col < y->col);
}

static int32_t wrap_add(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }

typedef struct {
    const float* static_scores;
    const int32_t* window_part_ids;
    const int32_t* part_starts;
    const int32_t* part_ends;
    float alpha, beta, delta, gamma_bonus, score_scale;
    int32_t use_hacs, locality_enabled;
} orc_hacs;

/* Score of one element (sampling.cuh:251-275). */
static int32_t elem_score(const orc_hacs* h, int32_t window, int32_t col, float v) {
    if (h && h->use_hacs) {
        float q = h->static_scores ? h->static_scores[col] : 1.0f;
        float f = fmaf(h->beta, fabsf(v), h->alpha) * q;
        if (h->locality_enabled && h->window_part_ids && h->part_starts && h->part_ends) {
            int32_t pid = h->window_part_ids[window];
            if (pid >= 0 && col >= h->part_starts[pid] && col < h->part_ends[pid]) f += h->delta;
        }
        return f2i_sat(f * h->score_scale);
    }
    return f2i_sat(fmaf(10.0f, fabsf(v), 1.0f) * 1000.0f);
}

ORC_API int32_t orc_window_cap(int32_t S) { return S <= 32 ? 32 : (S <= 128 ? 128 : 256); }

/* Candidate buffer size of the reference kernel (sampling.cuh:128-139). */
static int32_t global_buffer(int32_t cap, int32_t warps, int32_t tile_cols) {
    int32_t block = warps * 32;
    int32_t max_items = cap + warps * 16 * tile_cols;
    int32_t raw = (max_items + block - 1) / block;
    int32_t ipt = raw <= 1 ? 1 : raw <= 2 ? 2 : raw <= 4 ? 4 : raw <= 8 ? 8 : 16;
    return ipt * block;
}

/* Phase 1 for every active window.  sampled [A*S] (-1 padded), tiles [A]. */
ORC_API void orc_window_topk(const int64_t* win_off, const int32_t* cols, const float* vals,
                             int32_t tile_cols, const int32_t* active, int64_t A, int32_t fanout,
                             int32_t warps, const orc_hacs* h, int32_t* sampled, int32_t* tiles) {
    const int32_t S = ((fanout + 31) / 32) * 32;
    const int32_t cap = orc_window_cap(S);
    const int32_t G = global_buffer(cap, warps, tile_cols);
    const int32_t per_tile = 16 * tile_cols;
    const int32_t gamma_int = (h && h->use_hacs && h->gamma_bonus > 0.0f)
                                  ? (int32_t)(h->gamma_bonus * h->score_scale) : 0;
    orc_cand* glob = (orc_cand*)malloc(sizeof(orc_cand) * (size_t)G);
    orc_cand* wl = (orc_cand*)malloc(sizeof(orc_cand) * (size_t)warps * per_tile);
    int32_t* wcnt = (int32_t*)malloc(sizeof(int32_t) * (size_t)warps);
    int32_t* keys = (int32_t*)malloc(sizeof(int32_t) * (size_t)G);
    for (int64_t b = 0; b < A; ++b) {
        const int32_t w = active[b];
        const int64_t t0 = win_off[w], total = win_off[w + 1] - t0;
        int32_t* out = sampled + b * S;
        if (total == 0) {
            for (int32_t i = 0; i < S; ++i) out[i] = -1;
            tiles[b] = 0;
            continue;
        }
        int32_t gcnt = 0;
        for (int64_t bs = 0; bs < total; bs += warps) {
            int32_t bt = (int32_t)(total - bs < warps ? total - bs : warps);
            for (int32_t j = 0; j < bt; ++j) {
                const int64_t tile = t0 + bs + j;
                orc_cand* L = wl + (size_t)j * per_tile;
                wcnt[j] = 0;
                for (int32_t off = 0; off < per_tile; ++off) { /* lanes in order, elements in order */
                    const int32_t r = off / tile_cols, c = off % tile_cols;
                    const int32_t col = cols[tile * tile_cols + c];
                    if (col == -1) continue;
                    const int32_t sc = elem_score(h, w, col, vals[tile * per_tile + r * tile_cols + c]);
                    if (sc <= 0) continue;
                    int32_t i = 0;
                    for (; i < wcnt[j]; ++i) if (L[i].col == col) { L[i].freq = wrap_add(L[i].freq, sc); break; }
                    if (i == wcnt[j] && wcnt[j] < per_tile) { L[wcnt[j]].col = col; L[wcnt[j]].freq = sc; wcnt[j]++; }
                }
            }
            /* single-threaded merge (sampling.cuh:306-344) */
            for (int32_t j = 0; j < bt && gcnt < G; ++j) {
                const orc_cand* L = wl + (size_t)j * per_tile;
                for (int32_t i = 0; i < wcnt[j]; ++i) {
                    if (gcnt >= G) break;
                    int32_t k = 0;
                    for (; k < gcnt; ++k) if (glob[k].col == L[i].col) { glob[k].freq = wrap_add(glob[k].freq, L[i].freq); break; }
                    if (k == gcnt && gcnt < G) {
                        glob[gcnt].col = L[i].col;
                        glob[gcnt].freq = wrap_add(L[i].freq, gamma_int);
                        gcnt++;
                    }
                }
            }
            if (gcnt > 1) { /* sort with (INT_MAX, 0) padding over the block's G slots */
                for (int32_t k = gcnt; k < G; ++k) { glob[k].col = INT32_MAX; glob[k].freq = 0; }
                qsort(glob, (size_t)G, sizeof(orc_cand), cmp_cand);
            }
            if (gcnt > cap) gcnt = cap;
        }
        if (gcnt > 1) {
            for (int32_t k = 0; k < gcnt; ++k) keys[k] = glob[k].col;
            qsort(keys, (size_t)gcnt, sizeof(int32_t), cmp_i32);
            for (int32_t k = 0; k < gcnt; ++k) glob[k].col = keys[k];
        }
        const int32_t valid = gcnt < S ? gcnt : S;
        tiles[b] = (valid + tile_cols - 1) / tile_cols;
        for (int32_t i = 0; i < S; ++i) out[i] = i < valid ? glob[i].col : -1;
    }
    free(glob); free(wl); free(wcnt); free(keys);
}

/* Phases 2-3: values of the sampled columns (build_col_to_val_map_kernel's */
/* linear search, sampling.cuh:707-773; recompress_sampled_bcsr_kernel,    */
/* :471-579).  out_off [A+1] is the prefix sum of tiles; out_cols / out_vals */
/* are written for every output tile. */
ORC_API void orc_window_recompress(const int64_t* win_off, const int32_t* cols, const float* vals,
                                   int64_t num_entries, int32_t tile_cols, const int32_t* active,
                                   int64_t A, int32_t fanout, const int32_t* sampled,
                                   const int64_t* out_off, int32_t* out_cols, float* out_vals) {
    const int32_t S = ((fanout + 31) / 32) * 32;
    const int32_t per_tile = 16 * tile_cols;
    for (int64_t b = 0; b < A; ++b) {
        const int32_t w = active[b];
        const int64_t t0 = win_off[w], t1 = win_off[w + 1];
        for (int64_t t = 0; t < out_off[b + 1] - out_off[b]; ++t) {
            const int64_t ot = out_off[b] + t;
            for (int32_t c = 0; c < tile_cols; ++c) {
                const int64_t j = t * tile_cols + c;
                const int32_t col = j < S ? sampled[b * S + j] : -1;
                out_cols[ot * tile_cols + c] = col;
                int64_t map_tile = -1; int32_t map_c = -1;
                if (col != -1) {
                    for (int64_t it = t0; it < t1 && map_tile < 0; ++it)
                        for (int32_t cc = 0; cc < tile_cols; ++cc)
                            if (cols[it * tile_cols + cc] == col) { map_tile = it - t0; map_c = cc; break; }
                }
                for (int32_t r = 0; r < 16; ++r) {
                    float v = 0.0f;
                    if (map_tile >= 0) {
                        int64_t idx = (t0 + map_tile) * per_tile + (int64_t)r * tile_cols + map_c;
                        if (idx < num_entries) v = vals[idx];
                    }
                    out_vals[ot * per_tile + (int64_t)r * tile_cols + c] = v;
                }
            }
        }
    }
}

/* prepare_windows_and_masks (sampling_wrapper.cu:283-347): seeds -> sorted */
/* unique windows with OR-ed masks; -1 dropped.  Returns the window count.   */
typedef struct { int32_t w; uint32_t m; } orc_wm;
static int cmp_wm(const void* a, const void* b) {
    int32_t x = ((const orc_wm*)a)->w, y = ((const orc_wm*)b)->w;
    return (x > y) - (x < y);
}
ORC_API int64_t orc_prepare_windows(const int32_t* seeds, int64_t n, int32_t tile_rows,
                                    int32_t* windows, int32_t* masks) {
    orc_wm* t = (orc_wm*)malloc(sizeof(orc_wm) * (size_t)(n > 0 ? n : 1));
    for (int64_t i = 0; i < n; ++i) {
        if (seeds[i] == -1) { t[i].w = INT32_MAX; t[i].m = 0; }
        else { t[i].w = seeds[i] / tile_rows; t[i].m = 1u << (seeds[i] % tile_rows); }
    }
    qsort(t, (size_t)n, sizeof(orc_wm), cmp_wm);
    int64_t na = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (na > 0 && windows[na - 1] == t[i].w) { masks[na - 1] = (int32_t)((uint32_t)masks[na - 1] | t[i].m); continue; }
        windows[na] = t[i].w; masks[na] = (int32_t)t[i].m; na++;
    }
    if (na > 0 && windows[na - 1] == INT32_MAX) na--;
    free(t);
    return na;
}

ORC_API int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

ORC_API void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
