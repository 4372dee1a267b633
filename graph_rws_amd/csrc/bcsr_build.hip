// On-device COO / CSR -> BCSR construction, BCSR -> COO, COO -> CSR (gfx950).
//
// Replaces the host-core converter the reference runs on every graph
// (core/wrapper/convert_wrapper.cpp:27-180, reached from data/bcsr.py:190-234)
// and the torch COO -> CSR of data/bcsr.py:162-187, and adds the transposed
// build that the backward pass uses in place of the reference's atomic
// scatter (core/include/spmm_tc.cuh:211-270).
//
// BCSR build, one sort for the whole graph:
//   key = (window << (cbits + 4)) | (column << 4) | row-in-window, with the
//   edge value as payload, sorted by the stable LSD radix sort (sort.hip) over
//   exactly the bits the graph needs.  After the sort every window's edges
//   are contiguous and column-ascending, so
//     unique-column flag  = key>>4 differs from the previous key's,
//     column position     = exclusive scan of those flags,
//     tiles per window    = ceil(unique columns / tile_cols) -> scan,
//   and one scatter writes every column slot and value.  Duplicate (row,
//   column) edges keep input order through the stable sort; the last one
//   wins, as in the reference's plain store (convert_wrapper.cpp:174).
// The transposed build swaps the roles of rows and columns in the key.
#include <mutex>

#include "grws_internal.h"

namespace grws {
namespace {

constexpr int kBlk = 256;

enum : int32_t { kErrRow = 1, kErrCol = 2, kErrRowPtr = 4 };

// Bits needed to hold every value in [0, x).
inline int bits_for(int64_t x) {
    int b = 0;
    while (b < 63 && ((int64_t)1 << b) < x) ++b;
    return b;
}

inline unsigned grid_for(int64_t n, int64_t per_block = kBlk) {
    int64_t g = (n + per_block - 1) / per_block;
    return (unsigned)(g < 1 ? 1 : g);
}

// Shape of one build, derived identically by the count and fill phases.
struct BuildShape {
    int64_t n, R, C, W;  // edges; rows / columns of the built matrix; windows
    int cbits, wbits, bits;
};

BuildShape build_shape(int64_t nnz, int64_t num_rows, int64_t num_cols, int32_t transpose) {
    BuildShape s;
    s.n = nnz;
    s.R = transpose ? num_cols : num_rows;
    s.C = transpose ? num_rows : num_cols;
    s.W = (s.R + 15) / 16;
    s.cbits = bits_for(s.C);
    s.wbits = bits_for(s.W);
    s.bits = s.wbits + s.cbits + 4;
    return s;
}

// Workspace of a build (the fill phase re-derives the same pointers).
struct BuildWs {
    uint64_t *ka, *kb;
    uint32_t *va, *vb;
    int32_t* uflag;
    int64_t* uidx;
    int64_t *wstart, *wend;
    int32_t* wtiles;
    int32_t* blist;  // windows of more than kWinCap edges (per-window path)
    int32_t* err;
    char* sort_ws;
    size_t sort_bytes;
    char* scan_ws;
    size_t scan_bytes;
};

template <typename C>
void carve_build(C& cv, const BuildShape& s, BuildWs* w) {
    const int64_t n = s.n > 0 ? s.n : 1;
    w->ka = cv.template take<uint64_t>(n);
    w->kb = cv.template take<uint64_t>(n);
    w->va = cv.template take<uint32_t>(n);
    w->vb = cv.template take<uint32_t>(n);
    w->uflag = cv.template take<int32_t>(n);
    w->uidx = cv.template take<int64_t>(n + 1);
    w->wstart = cv.template take<int64_t>(s.W + 1);
    w->wend = cv.template take<int64_t>(s.W + 1);
    w->wtiles = cv.template take<int32_t>(s.W + 1);
    w->blist = cv.template take<int32_t>(s.W + 1);
    w->err = cv.template take<int32_t>(64);
    w->sort_bytes = radix_sort_workspace_bytes(n);
    w->sort_ws = cv.template take<char>(w->sort_bytes);
    int64_t m = n > s.W ? n : s.W;
    w->scan_bytes = scan_workspace_bytes(m);
    w->scan_ws = cv.template take<char>(w->scan_bytes);
}

struct NullCarver {
    Sizer s;
    template <typename T>
    T* take(size_t k) {
        s.take<T>(k);
        return nullptr;
    }
};

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
__global__ void check_row_ptr_kernel(const int64_t* __restrict__ row_ptr, int64_t num_rows, int64_t nnz,
                                     int32_t* __restrict__ err) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > num_rows) return;
    bool bad = false;
    if (r == 0) bad = row_ptr[0] != 0;
    if (r == num_rows) bad = bad || row_ptr[num_rows] != nnz;
    if (r < num_rows) bad = bad || row_ptr[r + 1] < row_ptr[r];
    if (bad) atomicOr(err, kErrRowPtr);
}

// Row of edge e in a CSR: the largest r with row_ptr[r] <= e.
__device__ __forceinline__ int64_t csr_row_of(const int64_t* __restrict__ row_ptr, int64_t num_rows, int64_t e) {
    int64_t lo = 0, hi = num_rows - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (row_ptr[mid] <= e) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// An edge's sort key from its window-row wr (the BCSR row) and column cc.
// wbits == 0: (window, column, row-in-window), the global sort's key.
// wbits > 0 (a multiple of 8): window | row-in-window << wbits | column <<
// (wbits + 4), for the window-major sort (only the low wbits bits sorted);
// equal edges have equal keys, so a stable sort keeps duplicates in input
// order.
__device__ __forceinline__ uint64_t edge_key(int64_t wr, int64_t cc, int cbits, int wbits) {
    if (wbits) return (uint64_t)(wr >> 4) | ((uint64_t)(wr & 15) << wbits) | ((uint64_t)cc << (wbits + 4));
    return ((uint64_t)(wr >> 4) << (cbits + 4)) | ((uint64_t)cc << 4) | (uint64_t)(wr & 15);
}

__global__ void build_keys_kernel(const int64_t* __restrict__ row_ptr, const int32_t* __restrict__ rows,
                                  const int32_t* __restrict__ cols, const float* __restrict__ vals, int64_t n,
                                  int64_t num_rows, int64_t num_cols, int transpose, int cbits, int wbits,
                                  uint64_t* __restrict__ keys, uint32_t* __restrict__ pay, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t r = rows ? (int64_t)rows[i] : csr_row_of(row_ptr, num_rows, i);
    int64_t c = cols[i];
    int32_t e = 0;
    if (r < 0 || r >= num_rows) { e |= kErrRow; r = 0; }
    if (c < 0 || c >= num_cols) { e |= kErrCol; c = 0; }
    if (e) atomicOr(err, e);
    keys[i] = transpose ? edge_key(c, r, cbits, wbits) : edge_key(r, c, cbits, wbits);
    pay[i] = vals ? __float_as_uint(vals[i]) : 0x3f800000u;  // 1.0f when no values are given
}

// The same keys from a CSR, one wave per row: the row is known, its edges
// [row_ptr[r], row_ptr[r+1]) are read in order (a per-edge binary search for
// the row took 2.3 ms on 115M edges).  A valid row pointer covers [0, nnz)
// exactly, so every edge gets its key.  check_row_ptr_kernel runs first: when
// it flagged the row pointer, every key is written as 0 instead (in range for
// the kernels after the sort; the call then reports the error).
__global__ __launch_bounds__(256) void build_keys_rows_kernel(const int64_t* __restrict__ row_ptr,
                                                              const int32_t* __restrict__ cols,
                                                              const float* __restrict__ vals, int64_t n,
                                                              int64_t num_rows, int64_t num_cols, int transpose,
                                                              int cbits, int wbits, uint64_t* __restrict__ keys,
                                                              uint32_t* __restrict__ pay, int32_t* __restrict__ err) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / kWave);
    if (*err & kErrRowPtr) {  // uniform: set by the check before this launch
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
            keys[i] = 0;
            pay[i] = 0;
        }
        return;
    }
    for (int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave; r < num_rows; r += nwaves) {
        int64_t lo = row_ptr[r], hi = row_ptr[r + 1];
        lo = lo < 0 ? 0 : (lo > n ? n : lo);
        hi = hi < lo ? lo : (hi > n ? n : hi);
        bool bad = false;
        for (int64_t i = lo + lane; i < hi; i += kWave) {
            int64_t c = cols[i];
            if (c < 0 || c >= num_cols) {
                bad = true;
                c = 0;
            }
            keys[i] = transpose ? edge_key(c, r, cbits, wbits) : edge_key(r, c, cbits, wbits);
            pay[i] = vals ? __float_as_uint(vals[i]) : 0x3f800000u;  // 1.0f when no values are given
        }
        if (bad) atomicOr(err, kErrCol);
    }
}

__global__ void unique_flag_kernel(const uint64_t* __restrict__ keys, int64_t n, int32_t* __restrict__ uflag) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uflag[i] = (i == 0 || (keys[i] >> 4) != (keys[i - 1] >> 4)) ? 1 : 0;
}

__global__ void window_bounds_kernel(const uint64_t* __restrict__ keys, int64_t n, int wshift,
                                     const int32_t* __restrict__ uflag, const int64_t* __restrict__ uidx,
                                     int64_t* __restrict__ wstart, int64_t* __restrict__ wend) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t w = keys[i] >> wshift;
    if (i == 0 || (keys[i - 1] >> wshift) != w) wstart[w] = uidx[i];
    if (i == n - 1 || (keys[i + 1] >> wshift) != w) wend[w] = uidx[i] + uflag[i];
}

__global__ void window_tiles_kernel(const int64_t* __restrict__ wstart, const int64_t* __restrict__ wend, int64_t W,
                                    int tc, int32_t* __restrict__ wtiles) {
    const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= W) return;
    const int64_t u = wend[w] - wstart[w];
    wtiles[w] = (int32_t)((u + tc - 1) / tc);
}

// Window bounds of window-major sorted keys (edge_key with wbits > 0).
__global__ void keyed_bounds_kernel(const uint64_t* __restrict__ keys, int64_t n, uint64_t wmask,
                                    int64_t* __restrict__ wstart, int64_t* __restrict__ wend) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t w = keys[i] & wmask;
    if (i == 0 || (keys[i - 1] & wmask) != w) wstart[w] = i;
    if (i == n - 1 || (keys[i + 1] & wmask) != w) wend[w] = i + 1;
}

template <typename VT>
__device__ __forceinline__ void store_value(void* vals, int64_t idx, float v);
template <>
__device__ __forceinline__ void store_value<float>(void* vals, int64_t idx, float v) {
    static_cast<float*>(vals)[idx] = v;
}
template <>
__device__ __forceinline__ void store_value<_Float16>(void* vals, int64_t idx, float v) {
    static_cast<_Float16*>(vals)[idx] = (_Float16)v;
}
template <>
__device__ __forceinline__ void store_value<__hip_bfloat16>(void* vals, int64_t idx, float v) {
    static_cast<__hip_bfloat16*>(vals)[idx] = __float2bfloat16(v);
}

template <typename VT>
__global__ void build_scatter_kernel(const uint64_t* __restrict__ keys, const uint32_t* __restrict__ pay, int64_t n,
                                     int cbits, const int32_t* __restrict__ uflag, const int64_t* __restrict__ uidx,
                                     const int64_t* __restrict__ wstart, const int64_t* __restrict__ win_off,
                                     int tc, int32_t* __restrict__ out_cols, void* __restrict__ out_vals,
                                     const int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || err[2] != 0) return;  // err[2] != 0: the per-window build ran
    const uint64_t k = keys[i];
    const int wshift = cbits + 4;
    const int64_t w = (int64_t)(k >> wshift);
    const int64_t col = (int64_t)((k >> 4) & ((1ull << cbits) - 1ull));
    const int r = (int)(k & 15u);
    const int32_t f = uflag[i];
    const int64_t p = uidx[i] + f - 1 - wstart[w];
    const int64_t tile = win_off[w] + p / tc;
    const int c = (int)(p % tc);
    if (f) out_cols[tile * tc + c] = (int32_t)col;
    if (i == n - 1 || keys[i + 1] != k) store_value<VT>(out_vals, (tile * 16 + r) * tc + c, __uint_as_float(pay[i]));
}

// --- window-by-window build ---------------------------------------------------
// A CSR's edges come grouped by window already (16 consecutive rows); COO
// input and transposed builds are grouped by a sort over the window bits of
// their keys.  Each window of at most kWinCap edges is then built by one
// work-group from LDS (win_sort_kernel: each distinct column's place among the
// window's distinct columns, from a column bitmap or an LDS radix sort, and one
// record per edge; win_fill_kernel: the tiles assembled in LDS), larger ones
// by one work-group each from global scratch (win_sort_big_kernel,
// win_fill_big_kernel).
//
// record of a window of more than kWinCap edges (in (column, row, offset)
// order): value bits (f32) | place << 32 (27 bits) | row << 59 (4 bits) |
// last of its (column, row) run << 63; the window's last record holds its
// last place, so the fill knows the count of distinct columns.
constexpr int64_t kWinHuge = (int64_t)1 << 27;  // windows of more edges take the global sort
__device__ __forceinline__ uint64_t win_record(uint32_t vbits, int place, int row, bool last) {
    return (uint64_t)vbits | ((uint64_t)place << 32) | ((uint64_t)row << 59) | ((uint64_t)last << 63);
}
__device__ __forceinline__ int rec_place(uint64_t r) { return (int)((r >> 32) & (uint64_t)(kWinHuge - 1)); }
__device__ __forceinline__ int rec_row(uint64_t r) { return (int)((r >> 59) & 15u); }
__device__ __forceinline__ bool rec_last(uint64_t r) { return (r >> 63) & 1u; }

// record of a window of at most kWinCap edges (in any order): value bits |
// place << 32 (14 bits) | row << 46 (4 bits) | edge offset in the window <<
// 50 (14 bits); of duplicate (row, column) edges the fill keeps the largest
// offset, the last in input order.
__device__ __forceinline__ uint64_t srec(uint32_t vbits, int place, int row, int j) {
    return (uint64_t)vbits | ((uint64_t)place << 32) | ((uint64_t)row << 46) | ((uint64_t)j << 50);
}
__device__ __forceinline__ int srec_place(uint64_t r) { return (int)((r >> 32) & 16383u); }
__device__ __forceinline__ int srec_row(uint64_t r) { return (int)((r >> 46) & 15u); }
__device__ __forceinline__ int srec_j(uint64_t r) { return (int)(r >> 50); }

constexpr int kWinCap = 16384;  // windows of up to 8,192 edges use a half-size LDS twin
constexpr int kWinBlk = 512;
constexpr int kWinDig = 9;                 // radix digit bits
constexpr int kWinBkt = 1 << kWinDig;      // digit values: one per thread in the offset scan
static_assert(kWinBkt == kWinBlk, "the offset scan gives each thread one digit");

// Windows of more than kWinCap edges: counted in err[1] and listed in blist
// (in no particular order; each is built by itself); windows of more than
// kWinHuge edges counted in err[3].  From a valid row pointer.
__device__ __forceinline__ void note_window_size(int64_t w, int64_t m, int32_t* __restrict__ blist,
                                                 int32_t* __restrict__ err) {
    if (m > kWinCap) blist[atomicAdd(&err[1], 1)] = (int32_t)w;
    if (m > kWinHuge) atomicAdd(&err[3], 1);
}

__global__ void win_big_kernel(const int64_t* __restrict__ row_ptr, int64_t R, int64_t W, int64_t n,
                               int32_t* __restrict__ blist, int32_t* __restrict__ err) {
    const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= W) return;
    const int64_t r1 = 16 * w + 16 < R ? 16 * w + 16 : R;
    note_window_size(w, row_ptr[r1] - row_ptr[16 * w], blist, err);
}

// The same from window bounds (the window-major sorted keys').
__global__ void keyed_big_kernel(const int64_t* __restrict__ wstart, const int64_t* __restrict__ wend, int64_t W,
                                 int32_t* __restrict__ blist, int32_t* __restrict__ err) {
    const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= W) return;
    note_window_size(w, wend[w] - wstart[w], blist, err);
}

// KEYED false: the window's edges straight from a CSR (row_ptr, cols, vals).
// KEYED true: from window-major sorted keys (edge_key with wbits > 0) and
// their value bits (tkeys, tvals, bounds in wstart / wend); the LDS key is
// (column - min) << 4 | row, which needs column spans under 2^27 (the host
// checks).  The records (skeys) and distinct columns (ucol) never share
// memory with the input.
//
// Places: a bitmap of the window's columns over its span when the span fits
// the offsets' LDS (2 bits an edge slot; c3: every window), its popcounts
// giving each column's place, the records in input order; else a stable LSD
// radix sort of the edge offsets by the LDS key (9-bit digits, 8 with 256
// threads) and first-of-column flags counted per wave, the records in sorted
// order.  Either way the fill keeps, of duplicate (row, column) edges, the
// largest offset, i.e. the last in input order.
template <int CAP, int BLK, bool KEYED>
__global__ __launch_bounds__(BLK) __attribute__((amdgpu_waves_per_eu(CAP == 8192 ? 4 : (CAP == 16384 ? 2 : 1)))) void win_sort_kernel(
    const int64_t* __restrict__ row_ptr, const int32_t* __restrict__ cols, const float* __restrict__ vals,
    const uint64_t* __restrict__ tkeys, const uint32_t* __restrict__ tvals, int wbits, int64_t n, int64_t R, int64_t W,
    int64_t num_cols, int tc, uint64_t* __restrict__ skeys, int32_t* __restrict__ ucol, int64_t* __restrict__ wstart,
    int64_t* __restrict__ wend, int32_t* __restrict__ wtiles, int32_t* __restrict__ err) {
    // CAP 2048 (256 threads, 8-bit digits, 18 KB of LDS): the windows of at
    // most 2,048 edges; CAP 8192 (512 threads, 9-bit digits, 73 KB: two
    // work-groups per CU): up to 8,192; CAP 16384: the larger ones (at most
    // kWinCap edges: checked before the launch)
    static_assert((CAP == 2048 && BLK == 256) || (CAP != 2048 && BLK == BLK), "launch shapes");
    constexpr int NW = BLK / kWave;
    constexpr int PER = CAP / BLK;            // edges per thread
    constexpr int DIG = BLK == 256 ? 8 : 9;   // digit bits: one digit per thread in the offset scan
    constexpr int MLO = CAP == 2048 ? -1 : (CAP == 8192 ? 2048 : 8192);  // this launch: MLO < edges <= CAP
    __shared__ int32_t colv[CAP];             // the window's sort keys, by edge offset
    // edge offsets: sort source and destination (radix); or the column bitmap
    __shared__ __align__(16) uint16_t iab[2 * CAP];
    uint16_t* const ia = iab;
    uint16_t* const ib = iab + CAP;
    // [wave][digit] counts, then scatter positions, 16 bits each (at most
    // CAP), two digits a word; or the bitmap's popcount bases
    __shared__ uint32_t cnt[NW * BLK / 2];
    __shared__ int64_t rp[17];
    __shared__ int64_t tmp[NW + 1];
    __shared__ int32_t mm[2 * NW];            // per-wave column range
    __shared__ int32_t wcnt[NW];              // per-wave distinct columns
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {  // uniform over the work-group
        int nr = 16;
        int64_t e0;
        int m;
        if (KEYED) {
            e0 = wstart[w];
            const int64_t mm64 = wend[w] - e0;
            m = (int)(mm64 < 0 ? 0 : (mm64 > CAP ? CAP : mm64));
            // another launch's window (uniform; no LDS yet)
            if (mm64 <= MLO || mm64 > CAP) continue;
        } else {
            const int64_t r0 = 16 * w;
            nr = (int)(R - r0 < 16 ? R - r0 : 16);
            if (tid <= nr) {
                int64_t v = row_ptr[r0 + tid];
                rp[tid] = v < 0 ? 0 : (v > n ? n : v);
            }
            __syncthreads();
            e0 = rp[0];
            const int64_t mm64 = rp[nr] - e0;
            m = (int)(mm64 > CAP ? CAP : mm64);
            if (mm64 <= MLO || mm64 > CAP) {  // another launch's window (uniform)
                __syncthreads();
                continue;
            }
        }
        // columns into LDS (checked), offsets in input order, the column
        // span; every load issued before the first is used
        int cmin = 0x7fffffff, cmax = 0;
        int cbase;  // subtracted from colv[] for the digits
        if (KEYED) {
            uint64_t kk[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                kk[k] = j < m ? tkeys[e0 + j] : 0;
            }
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                if (tid + k * BLK < m) {
                    const int c = (int)(kk[k] >> (wbits + 4));
                    cmin = min(cmin, c);
                    cmax = max(cmax, c);
                }
            }
            for (int d = kWave / 2; d >= 1; d >>= 1) {
                cmin = min(cmin, __shfl_xor(cmin, d, kWave));
                cmax = max(cmax, __shfl_xor(cmax, d, kWave));
            }
            if (lane == 0) {
                mm[wv] = cmin;
                mm[NW + wv] = cmax;
            }
            __syncthreads();
            for (int v = 0; v < NW; ++v) {
                cmin = min(cmin, mm[v]);
                cmax = max(cmax, mm[NW + v]);
            }
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                if (j < m) {
                    const int c = (int)(kk[k] >> (wbits + 4)), q = (int)((kk[k] >> wbits) & 15u);
                    colv[j] = ((c - cmin) << 4) | q;
                    ia[j] = (uint16_t)j;
                }
            }
            __syncthreads();
            cbase = 0;
        } else {
            int32_t cv[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                cv[k] = j < m ? cols[e0 + j] : 0;
            }
            bool bad = false;
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                if (j < m) {
                    int32_t c = cv[k];
                    if (c < 0 || (int64_t)c >= num_cols) {
                        bad = true;
                        c = 0;
                    }
                    colv[j] = c;
                    ia[j] = (uint16_t)j;
                    cmin = min(cmin, c);
                    cmax = max(cmax, c);
                }
            }
            if (bad) atomicOr(err, kErrCol);
            for (int d = kWave / 2; d >= 1; d >>= 1) {
                cmin = min(cmin, __shfl_xor(cmin, d, kWave));
                cmax = max(cmax, __shfl_xor(cmax, d, kWave));
            }
            if (lane == 0) {
                mm[wv] = cmin;
                mm[NW + wv] = cmax;
            }
            __syncthreads();
            for (int v = 0; v < NW; ++v) {
                cmin = min(cmin, mm[v]);
                cmax = max(cmax, mm[NW + v]);
            }
            cbase = cmin;
        }
        auto row_of = [&](int j) {  // CSR: the edge's row in the window, the last q with rp[q] <= e0 + j
            const int64_t e = e0 + j;
            int q = 0;
#pragma unroll
            for (int st = 8; st >= 1; st >>= 1)
                if (q + st < nr && rp[q + st] <= e) q += st;
            return q;
        };
        // the edge's column relative to cmin (KEYED: colv >> 4; the row colv & 15)
        auto rel_col = [&](int j) { return KEYED ? colv[j] >> 4 : colv[j] - cmin; };
        int u;  // distinct columns
        // a column bitmap over the span when it fits the offsets' LDS (2 bits
        // an edge slot): places straight from popcounts, no sort
        constexpr int kBmWords = CAP;                 // 32-bit words in iab
        constexpr int G = CAP / (NW * BLK);           // words per popcount base (16-bit bases in cnt)
        const bool bm = m > 0 && (int64_t)cmax - cmin < (int64_t)kBmWords * 32;  // uniform
        if (bm) {
            // value bits of edge offsets tid + k BLK, every load issued first
            uint32_t vv[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                if (KEYED) vv[k] = j < m ? tvals[e0 + j] : 0u;
                else vv[k] = (vals && j < m) ? __float_as_uint(vals[e0 + j]) : 0x3f800000u;
            }
            uint32_t* bmp = reinterpret_cast<uint32_t*>(iab);
            uint16_t* wb = reinterpret_cast<uint16_t*>(cnt);
            const int nwords = (cmax - cmin) / 32 + 1;
            const int nent = (nwords + G - 1) / G;
            for (int x = tid; x < nwords; x += BLK) bmp[x] = 0;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                if (j < m) {
                    const int rc = rel_col(j);
                    atomicOr(&bmp[rc >> 5], 1u << (rc & 31));
                }
            }
            __syncthreads();
            {  // bases: each thread a contiguous run of entries, one block scan
                const int E = (nent + BLK - 1) / BLK;
                const int a0 = min(tid * E, nent), a1 = min(a0 + E, nent);
                int sum = 0;
                for (int e = a0; e < a1; ++e)
#pragma unroll
                    for (int g = 0; g < G; ++g)
                        if (e * G + g < nwords) sum += __popc(bmp[e * G + g]);
                int64_t tot;
                int run = (int)(block_incl_scan<BLK>(sum, tmp, &tot) - sum);
                for (int e = a0; e < a1; ++e) {
                    wb[e] = (uint16_t)run;
#pragma unroll
                    for (int g = 0; g < G; ++g)
                        if (e * G + g < nwords) run += __popc(bmp[e * G + g]);
                }
                u = (int)tot;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int j = tid + k * BLK;
                if (j < m) {
                    const int rc = rel_col(j), wd = rc >> 5;
                    int pl = wb[wd / G] + __popc(bmp[wd] & ((1u << (rc & 31)) - 1u));
#pragma unroll
                    for (int g = 1; g < G; ++g)
                        if (g <= wd % G) pl += __popc(bmp[wd - g]);
                    const int q = KEYED ? (colv[j] & 15) : row_of(j);
                    ucol[e0 + pl] = rc + cmin;  // every edge of the column writes the same id
                    skeys[e0 + j] = srec(vv[k], pl, q, j);
                }
            }
        } else {
            const uint32_t span = m > 0 ? (KEYED ? ((uint32_t)(cmax - cmin) << 4) | 15u : (uint32_t)(cmax - cmin)) : 0u;
            const int bits = span ? 32 - __clz(span) : 0;
            // wave v sorts positions [lo, hi): whole rounds of 64, in wave order
            const int chunk = ((m + NW * kWave - 1) / (NW * kWave)) * kWave;
            const int lo = min(wv * chunk, m), hi = min(lo + chunk, m);
            uint16_t* src = ia;
            uint16_t* dst = ib;
            for (int sh = 0; sh < bits; sh += DIG) {  // uniform
                for (int i = tid; i < NW * BLK / 2; i += BLK) cnt[i] = 0;
                __syncthreads();
                for (int i = lo + lane; i < hi; i += kWave) {
                    const uint32_t d = ((uint32_t)(colv[src[i]] - cbase) >> sh) & (BLK - 1);
                    atomicAdd(&cnt[wv * (BLK / 2) + (d >> 1)], 1u << (16 * (d & 1)));
                }
                __syncthreads();
                {  // exclusive offsets in (digit, wave) order; this thread's digit is tid
                    const int hw = 16 * (tid & 1);
                    int pos[NW];
                    int t = 0;
#pragma unroll
                    for (int v = 0; v < NW; ++v) {
                        pos[v] = (int)((cnt[v * (BLK / 2) + (tid >> 1)] >> hw) & 0xffffu);
                        t += pos[v];
                    }
                    int64_t tot;
                    int run = (int)(block_incl_scan<BLK>(t, tmp, &tot) - t);  // every count read first
#pragma unroll
                    for (int v = 0; v < NW; ++v) {
                        const int c = pos[v];
                        pos[v] = run;
                        run += c;
                    }
                    // the even digit's thread writes the pair's word
#pragma unroll
                    for (int v = 0; v < NW; ++v) {
                        const int odd = __shfl_down(pos[v], 1, kWave);
                        if (!(tid & 1)) cnt[v * (BLK / 2) + (tid >> 1)] = (uint32_t)pos[v] | ((uint32_t)odd << 16);
                    }
                }
                __syncthreads();
                // scatter: each wave walks its positions in order, 64 at a
                // time; lanes with equal digits take consecutive places in
                // lane order, and the group's highest lane advances the count
                for (int b = lo; b < hi; b += kWave) {  // uniform over the wave
                    const int i = b + lane;
                    const bool v = i < hi;
                    uint16_t x = 0;
                    int d = 0;
                    if (v) {
                        x = src[i];
                        d = (int)(((uint32_t)(colv[x] - cbase) >> sh) & (BLK - 1));
                    }
                    uint64_t peers = __ballot(v);
#pragma unroll
                    for (int k = 0; k < DIG; ++k) {
                        const bool bit = (d >> k) & 1;
                        const uint64_t bb = __ballot(bit);
                        peers &= bit ? bb : ~bb;
                    }
                    if (v) {
                        const int word = wv * (BLK / 2) + (d >> 1), hw = 16 * (d & 1);
                        const int base = (int)((cnt[word] >> hw) & 0xffffu);
                        dst[base + __popcll(peers & ((1ull << lane) - 1))] = x;
                        if ((peers >> lane) == 1ull) atomicAdd(&cnt[word], (uint32_t)__popcll(peers) << hw);
                    }
                }
                __syncthreads();
                uint16_t* t = src;
                src = dst;
                dst = t;
            }
            auto first_of_col = [&](int i) { return i == 0 || rel_col(src[i - 1]) != rel_col(src[i]); };
            // places: every wave walks its sorted positions in rounds of 64
            // consecutive ones, counts first-of-column flags by ballot, and
            // one barrier gives the waves' offsets
            int wbase = 0;
            {
                int wcount = 0;
                for (int b = lo; b < hi; b += kWave) {  // uniform over the wave
                    const int i = b + lane;
                    wcount += __popcll(__ballot(i < hi && first_of_col(i)));
                }
                if (lane == 0) wcnt[wv] = wcount;
                __syncthreads();
                u = 0;
                for (int v = 0; v < NW; ++v) {
                    const int c = wcnt[v];
                    wbase += v < wv ? c : 0;
                    u += c;
                }
            }
            for (int b = lo; b < hi; b += kWave) {  // uniform over the wave
                const int i = b + lane;
                const bool in = i < hi;
                const bool f = in && first_of_col(i);
                const uint64_t fm = __ballot(f);
                const int pl = wbase + __popcll(fm & ((2ull << lane) - 1)) - 1;  // flags up to this lane
                wbase += __popcll(fm);
                if (in) {
                    const int j = src[i];
                    const int q = KEYED ? (colv[j] & 15) : row_of(j);
                    if (f) ucol[e0 + pl] = rel_col(j) + cmin;
                    // the value of offset j sits in another thread's vv[]: read
                    // it from the input again (cache-resident)
                    const uint32_t vb = KEYED ? tvals[e0 + j] : (vals ? __float_as_uint(vals[e0 + j]) : 0x3f800000u);
                    skeys[e0 + i] = srec(vb, pl, q, j);
                }
            }
        }
        // -1 after the distinct columns, up to the tile boundary (within the
        // window's slots; the fill writes -1 beyond them itself)
        {
            const int upad = min((u + tc - 1) / tc * tc, m);
            for (int x = u + tid; x < upad; x += BLK) ucol[e0 + x] = -1;
        }
        if (tid == 0) {
            wtiles[w] = (u + tc - 1) / tc;
            if (!KEYED) {
                wstart[w] = e0;
                wend[w] = e0 + m;
            }
        }
        __syncthreads();  // LDS is rewritten for the next window
    }
}

// Windows of more than kWinCap edges (listed in blist; at most kWinHuge
// edges, checked before the launch), one work-group each: the same stable
// radix sort and records, with the edge offsets double-buffered in global
// scratch (jbuf, 2 m entries at 2 e0), the places in pbuf, and every sort key
// read from the input where it is used.
constexpr int kBig = 8;  // rounds of 64 edges whose loads are issued together
template <bool KEYED>
__global__ __launch_bounds__(kWinBlk) void win_sort_big_kernel(
    const int64_t* __restrict__ row_ptr, const int32_t* __restrict__ cols, const float* __restrict__ vals,
    const uint64_t* __restrict__ tkeys, const uint32_t* __restrict__ tvals, int wbits, int64_t n, int64_t R,
    const int32_t* __restrict__ blist, int nbig, int64_t num_cols, int tc, uint32_t* __restrict__ jbuf,
    uint32_t* __restrict__ pbuf, uint64_t* __restrict__ skeys, int32_t* __restrict__ ucol, int64_t* __restrict__ wstart,
    int64_t* __restrict__ wend, int32_t* __restrict__ wtiles, int32_t* __restrict__ err) {
    constexpr int NW = kWinBlk / kWave;
    __shared__ uint32_t cnt[NW * kWinBkt];  // [wave][digit] counts, then scatter positions
    __shared__ int64_t rp[17];
    __shared__ int64_t tmp[NW + 1];
    __shared__ int32_t mm[2 * NW];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    for (int bi = blockIdx.x; bi < nbig; bi += gridDim.x) {  // uniform over the work-group
        const int64_t w = blist[bi];
        int nr = 16;
        int64_t e0;
        int m;
        if (KEYED) {
            e0 = wstart[w];
            m = (int)(wend[w] - e0);
        } else {
            const int64_t r0 = 16 * w;
            nr = (int)(R - r0 < 16 ? R - r0 : 16);
            if (tid <= nr) {
                int64_t v = row_ptr[r0 + tid];
                rp[tid] = v < 0 ? 0 : (v > n ? n : v);
            }
            __syncthreads();
            e0 = rp[0];
            m = (int)(rp[nr] - e0);
        }
        const uint64_t* tk = tkeys;
        const uint32_t* tv = tvals;
        int cmin = 0x7fffffff, cmax = 0;
        bool bad = false;
        for (int j = tid; j < m; j += kWinBlk) {
            int c;
            if (KEYED) {
                c = (int)(tk[e0 + j] >> (wbits + 4));
            } else {
                int64_t cc = cols[e0 + j];
                if (cc < 0 || cc >= num_cols) {
                    bad = true;
                    cc = 0;
                }
                c = (int)cc;
            }
            cmin = min(cmin, c);
            cmax = max(cmax, c);
        }
        if (bad) atomicOr(err, kErrCol);
        for (int d = kWave / 2; d >= 1; d >>= 1) {
            cmin = min(cmin, __shfl_xor(cmin, d, kWave));
            cmax = max(cmax, __shfl_xor(cmax, d, kWave));
        }
        if (lane == 0) {
            mm[wv] = cmin;
            mm[NW + wv] = cmax;
        }
        __syncthreads();
        for (int v = 0; v < NW; ++v) {
            cmin = min(cmin, mm[v]);
            cmax = max(cmax, mm[NW + v]);
        }
        // the sort key of edge offset j: (column - min) << 4 | row (KEYED),
        // column - min (CSR; the rows are in input order already)
        auto skey = [&](uint32_t j) -> uint32_t {
            if (KEYED) {
                const uint64_t k = tk[e0 + j];
                return ((uint32_t)((int)(k >> (wbits + 4)) - cmin) << 4) | (uint32_t)((k >> wbits) & 15u);
            }
            int64_t cc = cols[e0 + j];
            if (cc < 0 || cc >= num_cols) cc = 0;
            return (uint32_t)((int)cc - cmin);
        };
        auto colkey = [&](uint32_t j) -> uint32_t { return KEYED ? skey(j) >> 4 : skey(j); };
        auto row_of = [&](uint32_t j) {  // CSR: the last q with rp[q] <= e0 + j
            const int64_t e = e0 + j;
            int q = 0;
#pragma unroll
            for (int st = 8; st >= 1; st >>= 1)
                if (q + st < nr && rp[q + st] <= e) q += st;
            return q;
        };
        const uint32_t span = m > 0 ? (KEYED ? ((uint32_t)(cmax - cmin) << 4) | 15u : (uint32_t)(cmax - cmin)) : 0u;
        const int bits = span ? 32 - __clz(span) : 0;
        uint32_t* src = jbuf + 2 * e0;
        uint32_t* dst = src + m;
        for (int j = tid; j < m; j += kWinBlk) src[j] = (uint32_t)j;
        __syncthreads();
        const int chunk = ((m + NW * kWave - 1) / (NW * kWave)) * kWave;
        const int lo = min(wv * chunk, m), hi = min(lo + chunk, m);
        for (int sh = 0; sh < bits; sh += kWinDig) {  // uniform
            for (int i = tid; i < NW * kWinBkt; i += kWinBlk) cnt[i] = 0;
            __syncthreads();
            // kBig rounds of 64 at a time: their loads in flight together
            for (int b = lo; b < hi; b += kBig * kWave) {  // uniform over the wave
                uint32_t x[kBig];
#pragma unroll
                for (int r = 0; r < kBig; ++r) {
                    const int i = b + r * kWave + lane;
                    x[r] = i < hi ? src[i] : 0u;
                }
#pragma unroll
                for (int r = 0; r < kBig; ++r) {
                    const int i = b + r * kWave + lane;
                    if (i < hi) atomicAdd(&cnt[wv * kWinBkt + ((skey(x[r]) >> sh) & (kWinBkt - 1))], 1u);
                }
            }
            __syncthreads();
            {  // exclusive offsets in (digit, wave) order; this thread's digit is tid
                int pos[NW];
                int t = 0;
#pragma unroll
                for (int v = 0; v < NW; ++v) {
                    pos[v] = (int)cnt[v * kWinBkt + tid];
                    t += pos[v];
                }
                int64_t tot;
                int run = (int)(block_incl_scan<kWinBlk>(t, tmp, &tot) - t);  // every count read first
#pragma unroll
                for (int v = 0; v < NW; ++v) {
                    cnt[v * kWinBkt + tid] = (uint32_t)run;
                    run += pos[v];
                }
            }
            __syncthreads();
            for (int b0 = lo; b0 < hi; b0 += kBig * kWave) {  // uniform over the wave
                uint32_t x[kBig];
                int d[kBig];
#pragma unroll
                for (int r = 0; r < kBig; ++r) {
                    const int i = b0 + r * kWave + lane;
                    x[r] = i < hi ? src[i] : 0u;
                }
#pragma unroll
                for (int r = 0; r < kBig; ++r) {
                    const int i = b0 + r * kWave + lane;
                    d[r] = i < hi ? (int)((skey(x[r]) >> sh) & (kWinBkt - 1)) : 0;
                }
#pragma unroll
                for (int r = 0; r < kBig; ++r) {  // the rounds in order
                    const int i = b0 + r * kWave + lane;
                    const bool v = i < hi;
                    uint64_t peers = __ballot(v);
#pragma unroll
                    for (int k = 0; k < kWinDig; ++k) {
                        const bool bit = (d[r] >> k) & 1;
                        const uint64_t bb = __ballot(bit);
                        peers &= bit ? bb : ~bb;
                    }
                    if (v) {
                        const uint32_t base = cnt[wv * kWinBkt + d[r]];
                        dst[base + __popcll(peers & ((1ull << lane) - 1))] = x[r];
                        if ((peers >> lane) == 1ull) cnt[wv * kWinBkt + d[r]] = base + (uint32_t)__popcll(peers);
                    }
                }
            }
            __syncthreads();
            uint32_t* t = src;
            src = dst;
            dst = t;
        }
        {  // places: contiguous runs of sorted positions, one block scan
            const int run = (m + kWinBlk - 1) / kWinBlk;
            const int a0 = min(tid * run, m), a1 = min(a0 + run, m);
            int f = 0;
            uint32_t prev = a0 > 0 ? colkey(src[a0 - 1]) : 0u;
#pragma unroll 8
            for (int i = a0; i < a1; ++i) {
                const uint32_t ck = colkey(src[i]);
                f += (i == 0 || ck != prev) ? 1 : 0;
                prev = ck;
            }
            int64_t tot;
            int pl = (int)block_incl_scan<kWinBlk>(f, tmp, &tot) - f;
            prev = a0 > 0 ? colkey(src[a0 - 1]) : 0u;
#pragma unroll 8
            for (int i = a0; i < a1; ++i) {
                const uint32_t ck = colkey(src[i]);
                pl += (i == 0 || ck != prev) ? 1 : 0;
                prev = ck;
                pbuf[e0 + i] = (uint32_t)(pl - 1);
            }
            if (tid == 0) {
                wtiles[w] = (int32_t)((tot + tc - 1) / tc);
                if (!KEYED) {
                    wstart[w] = e0;
                    wend[w] = e0 + m;
                }
            }
        }
        __syncthreads();
#pragma unroll 4
        for (int i = tid; i < m; i += kWinBlk) {
            const uint32_t j = src[i];
            const uint32_t kj = skey(j);
            int c, q;
            bool last = true;
            if (KEYED) {
                c = (int)(kj >> 4) + cmin;
                q = (int)(kj & 15u);
                if (i + 1 < m) last = skey(src[i + 1]) != kj;
            } else {
                c = (int)kj + cmin;
                q = row_of(j);
                if (i + 1 < m) {  // as in win_sort_kernel
                    const uint32_t jn = src[i + 1];
                    last = skey(jn) != kj || e0 + jn >= rp[q + 1];
                }
            }
            const int pl = (int)pbuf[e0 + i];
            if (i == 0 || (int)pbuf[e0 + i - 1] != pl) ucol[e0 + pl] = c;
            const uint32_t vb = KEYED ? tv[e0 + j] : (vals ? __float_as_uint(vals[e0 + j]) : 0x3f800000u);
            skeys[e0 + i] = win_record(vb, pl, q, last);
        }
        __syncthreads();  // LDS and scratch are rewritten for the next window
    }
}

template <typename VT>
__device__ __forceinline__ VT to_value(float v);
template <>
__device__ __forceinline__ float to_value<float>(float v) {
    return v;
}
template <>
__device__ __forceinline__ _Float16 to_value<_Float16>(float v) {
    return (_Float16)v;
}
template <>
__device__ __forceinline__ __hip_bfloat16 to_value<__hip_bfloat16>(float v) {
    return __float2bfloat16(v);
}

// The fill of the per-window build (err[2] = 1 or 2; the global path's
// scatter exits then, and this kernel exits otherwise).  One work-group per
// window writes the window's whole tile range, padding included, so the
// outputs need no clearing first: the columns straight from the
// distinct-column list (which holds -1 after its last column), the values
// kFillVals at a time (32 tiles of 16 x 16, 64 of 16 x 8) assembled in LDS
// from the records, which every thread loads once, and written out with
// 16-byte stores.  Of records with the same (tile, row, column) slot --
// duplicate edges -- the one with the largest offset, the last in input
// order, is stored.
constexpr int kFillVals = 8192;
template <typename VT>
__device__ __forceinline__ uint32_t value_bits(VT v) {
    static_assert(sizeof(VT) == 2 || sizeof(VT) == 4, "16- or 32-bit values");
    if constexpr (sizeof(VT) == 2) {
        uint16_t b;
        __builtin_memcpy(&b, &v, 2);
        return b;
    } else {
        uint32_t b;
        __builtin_memcpy(&b, &v, 4);
        return b;
    }
}
template <int CAP, int BLK, typename VT>
__global__ __launch_bounds__(BLK) __attribute__((amdgpu_waves_per_eu(CAP == 8192 ? 4 : (CAP == 16384 ? 2 : 1)))) void win_fill_kernel(
    const uint64_t* __restrict__ rec, const int32_t* __restrict__ ucol, const int64_t* __restrict__ wstart,
    const int64_t* __restrict__ wend, const int64_t* __restrict__ win_off, int64_t W, int tc,
    int32_t* __restrict__ out_cols, void* __restrict__ out_vals, int aligned, const int32_t* __restrict__ err) {
    // CAP 2048 (256 threads): the windows of at most 2,048 edges; CAP 8192:
    // up to 8,192; CAP 16384: the larger ones (at most kWinCap)
    constexpr int PER = CAP / BLK;  // records per thread
    constexpr int MLO = CAP == 2048 ? -1 : (CAP == 8192 ? 2048 : 8192);  // this launch: MLO < edges <= CAP
    constexpr int VPU = 16 / (int)sizeof(VT);  // values per 16 bytes
    // a slot holds (1 + offset) << value bits | the value's bits: one atomicMax
    // keeps the last duplicate with its value; 0 is an empty slot (value 0)
    using PT = std::conditional_t<sizeof(VT) == 4, unsigned long long, uint32_t>;
    constexpr int VB = 8 * (int)sizeof(VT);
    constexpr int SPU = 16 / (int)sizeof(PT);  // slots per 16 bytes
    __shared__ __align__(16) PT stage[kFillVals];
    if (err[2] == 0) return;  // uniform
    const int tid = threadIdx.x;
    const int ltc = tc == 16 ? 4 : 3;
    const int gt = kFillVals / (16 * tc);  // tiles per step
    for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {  // uniform over the work-group
        const int64_t e0 = wstart[w], wo = win_off[w];
        const int64_t mm64 = wend[w] - e0;
        if (mm64 <= MLO || mm64 > CAP) continue;  // another launch's window (uniform)
        const int m = (int)mm64;
        const int64_t nt64 = win_off[w + 1] - wo;
        const int nt = (int)(nt64 < 0 ? 0 : nt64);
        uint64_t r[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = tid + k * BLK;
            r[k] = i < m ? rec[e0 + i] : 0;
        }
        int32_t* oc = out_cols + wo * tc;
        for (int x = tid; x < nt * tc; x += BLK) oc[x] = x < m ? ucol[e0 + x] : -1;
        for (int g0 = 0; g0 < nt; g0 += gt) {  // uniform over the work-group
            const int g1 = g0 + gt < nt ? g0 + gt : nt;
            const int nv = (g1 - g0) * 16 * tc;
            for (int x = tid; x < nv / SPU; x += BLK) reinterpret_cast<uint4*>(stage)[x] = make_uint4(0, 0, 0, 0);
            __syncthreads();
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                if (tid + k * BLK < m) {
                    const int pl = srec_place(r[k]);
                    const int t = (pl >> ltc) - g0;
                    if (t >= 0 && t < g1 - g0) {
                        const PT pk = ((PT)(srec_j(r[k]) + 1) << VB) |
                                      (PT)value_bits(to_value<VT>(__uint_as_float((uint32_t)r[k])));
                        atomicMax(&stage[((t * 16 + srec_row(r[k])) << ltc) + (pl & (tc - 1))], pk);
                    }
                }
            }
            __syncthreads();
            VT* ov = static_cast<VT*>(out_vals) + (wo + g0) * 16 * tc;
            if (aligned) {  // the values 16-byte aligned (uniform)
                for (int x = tid; x < nv / VPU; x += BLK) {
                    uint32_t o[4];
                    if constexpr (sizeof(VT) == 2) {
#pragma unroll
                        for (int h = 0; h < 4; ++h)
                            o[h] = ((uint32_t)stage[x * 8 + 2 * h] & 0xffffu) |
                                   (((uint32_t)stage[x * 8 + 2 * h + 1] & 0xffffu) << 16);
                    } else {
#pragma unroll
                        for (int h = 0; h < 4; ++h) o[h] = (uint32_t)stage[x * 4 + h];
                    }
                    reinterpret_cast<uint4*>(ov)[x] = make_uint4(o[0], o[1], o[2], o[3]);
                }
            } else {
                for (int x = tid; x < nv; x += BLK) {
                    const uint32_t bits = (uint32_t)stage[x] & (VB == 16 ? 0xffffu : 0xffffffffu);
                    if constexpr (sizeof(VT) == 2) {
                        const uint16_t h = (uint16_t)bits;
                        __builtin_memcpy(&ov[x], &h, 2);
                    } else {
                        __builtin_memcpy(&ov[x], &bits, 4);
                    }
                }
            }
            __syncthreads();
        }
    }
}

// The fill of the windows of more than kWinCap edges (listed in blist), one
// work-group each: the columns as in win_fill_kernel; the records are read
// in order, 512 at a time, and their places only grow, so the values are
// assembled kFillVals at a time in LDS and each step written out once no
// later record can fall in it.
template <typename VT>
__global__ __launch_bounds__(kWinBlk) void win_fill_big_kernel(const uint64_t* __restrict__ rec,
                                                               const int32_t* __restrict__ ucol,
                                                               const int64_t* __restrict__ wstart,
                                                               const int64_t* __restrict__ wend,
                                                               const int64_t* __restrict__ win_off,
                                                               const int32_t* __restrict__ blist, int nbig, int tc,
                                                               int32_t* __restrict__ out_cols, void* __restrict__ out_vals,
                                                               int aligned, const int32_t* __restrict__ err) {
    constexpr int VPU = 16 / (int)sizeof(VT);  // values per 16 bytes
    __shared__ __align__(16) VT sval[kFillVals];
    if (err[2] == 0) return;  // uniform
    const int tid = threadIdx.x;
    const int ltc = tc == 16 ? 4 : 3;
    const int gt = kFillVals / (16 * tc);  // tiles per step
    for (int bi = blockIdx.x; bi < nbig; bi += gridDim.x) {  // uniform over the work-group
        const int64_t w = blist[bi];
        const int64_t e0 = wstart[w], wo = win_off[w];
        const int m = (int)(wend[w] - e0);
        const int64_t nt64 = win_off[w + 1] - wo;
        const int nt = (int)(nt64 < 0 ? 0 : nt64);
        const int u = m > 0 ? rec_place(rec[e0 + m - 1]) + 1 : 0;
        int32_t* oc = out_cols + wo * tc;
        for (int64_t x = tid; x < (int64_t)nt * tc; x += kWinBlk) oc[x] = x < u ? ucol[e0 + x] : -1;
        // write out the step at tile g0 (its first min(gt, nt - g0) tiles)
        auto flush = [&](int g0) {
            const int g1 = g0 + gt < nt ? g0 + gt : nt;
            if (g1 <= g0) return;
            const int nv = (g1 - g0) * 16 * tc;
            VT* ov = static_cast<VT*>(out_vals) + (wo + g0) * 16 * tc;
            if (aligned) {
                for (int x = tid; x < nv / VPU; x += kWinBlk)
                    reinterpret_cast<uint4*>(ov)[x] = reinterpret_cast<const uint4*>(sval)[x];
            } else {
                for (int x = tid; x < nv; x += kWinBlk) ov[x] = sval[x];
            }
        };
        auto clear = [&]() {
            for (int x = tid; x < kFillVals / VPU; x += kWinBlk) reinterpret_cast<uint4*>(sval)[x] = make_uint4(0, 0, 0, 0);
        };
        int g0 = 0;
        clear();
        __syncthreads();
        for (int b = 0; b < m; b += kWinBlk) {  // uniform over the work-group
            const int i = b + tid;
            const uint64_t r = i < m ? rec[e0 + i] : 0;
            // the chunk's last place (places do not decrease): one address for all
            const int last_tile = rec_place(rec[e0 + (b + kWinBlk < m ? b + kWinBlk : m) - 1]) >> ltc;
            for (;;) {  // uniform
                if (i < m && rec_last(r)) {
                    const int pl = rec_place(r);
                    const int t = (pl >> ltc) - g0;
                    if (t >= 0 && t < gt)
                        sval[((t * 16 + rec_row(r)) << ltc) + (pl & (tc - 1))] = to_value<VT>(__uint_as_float((uint32_t)r));
                }
                if (last_tile < g0 + gt) break;  // every record of the chunk placed
                __syncthreads();
                flush(g0);
                __syncthreads();
                clear();
                __syncthreads();
                g0 += gt;
            }
        }
        __syncthreads();
        for (; g0 < nt; g0 += gt) {  // the last step, and any steps after it (zeros)
            flush(g0);
            __syncthreads();
            clear();
            __syncthreads();
        }
    }
}

// --- BCSR -> COO ---------------------------------------------------------
template <typename VT>
__device__ __forceinline__ float load_value(const void* v, int64_t idx);
template <>
__device__ __forceinline__ float load_value<float>(const void* v, int64_t idx) {
    return static_cast<const float*>(v)[idx];
}
template <>
__device__ __forceinline__ float load_value<_Float16>(const void* v, int64_t idx) {
    return (float)static_cast<const _Float16*>(v)[idx];
}
template <>
__device__ __forceinline__ float load_value<__hip_bfloat16>(const void* v, int64_t idx) {
    return __bfloat162float(static_cast<const __hip_bfloat16*>(v)[idx]);
}

// Tiles' values read 16 bytes a lane: chunk x holds values [x V, x V + V) (V
// = 16 / sizeof(VT)), i.e. slots s0 .. s0 + V - 1 of tile x / tpb (tpb =
// chunks per tile, 16 to 64: a tile's chunks sit on consecutive lanes of one
// wave); slot s is (row s / tc, column s % tc).  A slot counts when its
// column is in [0, num_cols) and its value is nonzero.  ALIGNED: the values
// 16-byte aligned (else read value by value).
template <typename VT, bool ALIGNED>
__device__ __forceinline__ void load_chunk(const void* __restrict__ vals, int64_t chunk, float* out) {
    constexpr int V = 16 / (int)sizeof(VT);
    if (ALIGNED) {
        const uint4 raw = static_cast<const uint4*>(vals)[chunk];
        const VT* v = reinterpret_cast<const VT*>(&raw);
#pragma unroll
        for (int k = 0; k < V; ++k) out[k] = (float)v[k];
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) out[k] = load_value<VT>(vals, chunk * V + k);
    }
}

template <typename VT, bool ALIGNED>
__global__ __launch_bounds__(256) void tile_nnz_kernel(const int32_t* __restrict__ cols, const void* __restrict__ vals,
                                                       int64_t T, int tc, int64_t num_cols, int32_t* __restrict__ cnt) {
    constexpr int V = 16 / (int)sizeof(VT);
    const int tpb = 16 * tc / V;
    const int64_t nch = T * tpb;
    for (int64_t xb = (int64_t)blockIdx.x * 256; xb < nch; xb += (int64_t)gridDim.x * 256) {  // uniform
        const int64_t x = xb + threadIdx.x;
        int c = 0;
        if (x < nch) {
            const int64_t t = x / tpb;
            const int s0 = (int)(x % tpb) * V;
            float v[V];
            load_chunk<VT, ALIGNED>(vals, x, v);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const int64_t col = cols[t * tc + (s0 + k) % tc];
                c += (col >= 0 && col < num_cols && v[k] != 0.0f) ? 1 : 0;
            }
        }
        for (int d = tpb / 2; d >= 1; d >>= 1) c += __shfl_xor(c, d, tpb);
        if (x < nch && x % tpb == 0) cnt[x / tpb] = c;
    }
}

// The window of every tile (twin), one work-group per window; tiles outside
// every window (only from a malformed window_offset) keep window 0.
__global__ __launch_bounds__(256) void tile_window_kernel(const int64_t* __restrict__ win_off, int64_t W, int64_t T,
                                                          int32_t* __restrict__ twin) {
    for (int64_t w = blockIdx.x; w < W; w += gridDim.x) {
        const int64_t a = win_off[w], e = win_off[w + 1];
        const int64_t t0 = a < 0 ? 0 : (a > T ? T : a);
        const int64_t t1 = e < t0 ? t0 : (e > T ? T : e);
        for (int64_t t = t0 + threadIdx.x; t < t1; t += 256) twin[t] = (int32_t)w;
    }
}

template <typename VT, bool ALIGNED>
__global__ __launch_bounds__(256) void tile_to_coo_kernel(const int32_t* __restrict__ twin,
                                                          const int32_t* __restrict__ cols,
                                                          const void* __restrict__ vals, int64_t T, int tc,
                                                          int64_t num_cols, const int64_t* __restrict__ toff,
                                                          int32_t* __restrict__ out_rows,
                                                          int32_t* __restrict__ out_cols,
                                                          float* __restrict__ out_vals) {
    constexpr int V = 16 / (int)sizeof(VT);
    const int tpb = 16 * tc / V;
    const int64_t nch = T * tpb;
    for (int64_t xb = (int64_t)blockIdx.x * 256; xb < nch; xb += (int64_t)gridDim.x * 256) {  // uniform
        const int64_t x = xb + threadIdx.x;
        const bool in = x < nch;
        const int64_t t = in ? x / tpb : 0;
        const int s0 = in ? (int)(x % tpb) * V : 0;
        float v[V];
        int32_t cc[V];
        int c = 0;
        if (in) {
            load_chunk<VT, ALIGNED>(vals, x, v);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                cc[k] = cols[t * tc + (s0 + k) % tc];
                c += (cc[k] >= 0 && cc[k] < num_cols && v[k] != 0.0f) ? 1 : 0;
            }
        }
        // exclusive prefix over the tile's chunks (consecutive lanes)
        int inc = c;
        const int gl = (int)(threadIdx.x % tpb);
        for (int d = 1; d < tpb; d <<= 1) {
            const int y = __shfl_up(inc, d, tpb);
            if (gl >= d) inc += y;
        }
        if (in && c) {
            int64_t pos = toff[t] + inc - c;
            const int64_t row0 = 16 * (int64_t)twin[t];
#pragma unroll
            for (int k = 0; k < V; ++k) {
                if (cc[k] >= 0 && cc[k] < num_cols && v[k] != 0.0f) {
                    out_rows[pos] = (int32_t)(row0 + (s0 + k) / tc);
                    out_cols[pos] = cc[k];
                    out_vals[pos] = v[k];
                    ++pos;
                }
            }
        }
    }
}

// --- COO -> CSR ------------------------------------------------------------
__global__ void coo_keys_kernel(const int32_t* __restrict__ src, const int32_t* __restrict__ dst, int64_t n,
                                int64_t num_rows, int64_t num_cols, int cbits, uint64_t* __restrict__ keys,
                                uint32_t* __restrict__ pay, int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t r = src[i], c = dst[i];
    int32_t e = 0;
    if (r < 0 || r >= num_rows) { e |= kErrRow; r = 0; }
    if (c < 0 || c >= num_cols) { e |= kErrCol; c = 0; }
    if (e) atomicOr(err, e);
    keys[i] = ((uint64_t)r << cbits) | (uint64_t)c;
    pay[i] = (uint32_t)i;
}

__global__ void coo_emit_kernel(const uint64_t* __restrict__ keys, const uint32_t* __restrict__ perm, int64_t n,
                                int cbits, const float* __restrict__ w, int32_t* __restrict__ col_idx,
                                float* __restrict__ values) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    col_idx[i] = (int32_t)(keys[i] & ((1ull << cbits) - 1ull));
    values[i] = w ? w[perm[i]] : 1.0f;
}

// row_ptr[r] = first sorted position whose row is >= r.
__global__ void coo_row_ptr_kernel(const uint64_t* __restrict__ keys, int64_t n, int cbits, int64_t num_rows,
                                   int64_t* __restrict__ row_ptr) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > num_rows) return;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)(keys[mid] >> cbits) < r) lo = mid + 1;
        else hi = mid;
    }
    row_ptr[r] = lo;
}

int read_error_flag(const int32_t* err_dev, hipStream_t stream, int32_t* out) {
    GRWS_HIP(hipMemcpyAsync(out, err_dev, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    return GRWS_OK;
}

int report_input_error(int32_t e, const char* who) {
    if (e & kErrRowPtr) return set_error(GRWS_E_RANGE, "%s: row_ptr is not a valid CSR row pointer", who);
    if (e & kErrRow) return set_error(GRWS_E_RANGE, "%s: a row index is out of range", who);
    if (e & kErrCol) return set_error(GRWS_E_RANGE, "%s: a column index is out of range", who);
    return GRWS_OK;
}

// Windows over kWinCap edges take one work-group each, a long serial chain
// that leaves most of the GPU idle; on a second stream (SideStream,
// grws_internal.h) they run beside the size classes' kernels instead of
// after them.

// The build synchronises on data-dependent sizes, which a stream under
// capture does not allow.  Refused before the stream is touched, so the
// caller's capture stays valid.
int refuse_capture(hipStream_t stream, const char* who) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_error(GRWS_E_INVALID, "%s: cannot read the stream's capture state (%s)", who,
                         hipGetErrorString(e));
    }
    if (cs != hipStreamCaptureStatusNone)
        return set_error(GRWS_E_INVALID,
                         "%s: the stream is being captured; the build waits for its data-dependent sizes, "
                         "so build before the capture", who);
    return GRWS_OK;
}

}  // namespace
}  // namespace grws

using namespace grws;

// ---------------------------------------------------------------------------
// COO / CSR -> BCSR
// ---------------------------------------------------------------------------
extern "C" size_t grws_bcsr_build_workspace_bytes(int64_t nnz, int64_t num_rows, int64_t num_cols,
                                                  int32_t transpose) {
    if (nnz < 0 || num_rows < 0 || num_cols < 0) return 0;
    BuildShape s = build_shape(nnz, num_rows, num_cols, transpose);
    NullCarver nc;
    BuildWs w;
    carve_build(nc, s, &w);
    return nc.s.used + 256;
}

extern "C" int grws_bcsr_build_count(const int64_t* row_ptr, const int32_t* rows, const int32_t* cols,
                                     const float* values, int64_t nnz, int64_t num_rows, int64_t num_cols,
                                     int32_t tile_cols, int32_t transpose, int64_t* window_offset, void* workspace,
                                     size_t workspace_bytes, int64_t* num_tiles_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(refuse_capture(stream, "bcsr_build_count"));
    GRWS_CHECK_ARG(nnz >= 0 && num_rows >= 0 && num_cols >= 0, "bcsr_build: negative size");
    GRWS_CHECK_ARG(num_rows <= INT32_MAX && num_cols <= INT32_MAX, "bcsr_build: dimensions exceed int32 ids");
    GRWS_CHECK_ARG(nnz <= (int64_t)UINT32_MAX, "bcsr_build: more than 2^32-1 edges");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "bcsr_build: tile_cols must be 8 or 16 (got %d)", tile_cols);
    GRWS_CHECK_ARG(window_offset && num_tiles_out, "bcsr_build: null output");
    GRWS_CHECK_ARG(row_ptr == nullptr || rows == nullptr, "bcsr_build: pass only one of row_ptr and rows");
    if (nnz > 0) GRWS_CHECK_ARG(row_ptr != nullptr || rows != nullptr, "bcsr_build: pass row_ptr or rows");
    if (nnz > 0) GRWS_CHECK_ARG(cols != nullptr, "bcsr_build: null cols");
    if (row_ptr) GRWS_CHECK_ARG(num_rows > 0 || nnz == 0, "bcsr_build: edges without rows");
    BuildShape s = build_shape(nnz, num_rows, num_cols, transpose);
    Carver cv(workspace, workspace_bytes);
    BuildWs w;
    carve_build(cv, s, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "bcsr_build: workspace too small (%zu < %zu)", workspace_bytes, cv.used);

    GRWS_TRY(fill_i32(w.err, 4, 0, stream));  // error flags, big windows, path of the fill, huge windows
    if (s.W == 0) {
        GRWS_TRY(fill_i64(window_offset, 1, 0, stream));
        GRWS_HIP(hipStreamSynchronize(stream));
        *num_tiles_out = 0;
        return nnz == 0 ? GRWS_OK : set_error(GRWS_E_RANGE, "bcsr_build: edges in an empty matrix");
    }
    GRWS_TRY(fill_i64(w.wstart, s.W, 0, stream));
    GRWS_TRY(fill_i64(w.wend, s.W, 0, stream));
    if (row_ptr) {
        hipLaunchKernelGGL(check_row_ptr_kernel, dim3(grid_for(num_rows + 1)), dim3(kBlk), 0, stream, row_ptr,
                           num_rows, nnz, w.err);
        GRWS_LAUNCH_CHECK();
    }
    // A build goes window by window from LDS when every window holds at most
    // kWinCap edges (one sync decides); anything else by the global sort.  A
    // CSR is already grouped by window; a transposed build or COO input is
    // grouped first by a stable sort over the window bits of its keys
    // (keyed), given BCSR column spans under 2^27.
    bool per_window = false, keyed = false, kalt = false;
    int nbig = 0;
    // the window field of the keyed layout: whole bytes, since the radix
    // passes sort bytes and the field must hold the window and nothing else
    const int kwbits = 8 * (((s.wbits > 0 ? s.wbits : 1) + 7) / 8);
    if (row_ptr && !transpose && nnz > 0) {
        hipLaunchKernelGGL(win_big_kernel, dim3(grid_for(s.W)), dim3(kBlk), 0, stream, row_ptr, s.R, s.W, nnz,
                           w.blist, w.err);
        GRWS_LAUNCH_CHECK();
        int32_t h[4] = {0, 0, 0, 0};
        GRWS_HIP(hipMemcpyAsync(h, w.err, 4 * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
        GRWS_HIP(hipStreamSynchronize(stream));
        per_window = (h[0] & kErrRowPtr) == 0 && h[3] == 0;
        nbig = h[1];
    } else if (nnz > 0 && s.C <= ((int64_t)1 << 27)) {
        if (rows) {
            hipLaunchKernelGGL(build_keys_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, row_ptr, rows, cols,
                               values, nnz, num_rows, num_cols, (int)transpose, s.cbits, kwbits, w.ka, w.va, w.err);
        } else {
            const int64_t wg = std::min<int64_t>((num_rows + 3) / 4, 65536);
            hipLaunchKernelGGL(build_keys_rows_kernel, dim3((unsigned)std::max<int64_t>(wg, 1)), dim3(256), 0, stream,
                               row_ptr, cols, values, nnz, num_rows, num_cols, (int)transpose, s.cbits, kwbits, w.ka,
                               w.va, w.err);
        }
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(radix_sort_pairs(w.ka, w.va, w.kb, w.vb, nnz, kwbits, w.sort_ws, w.sort_bytes, stream, &kalt));
        hipLaunchKernelGGL(keyed_bounds_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, kalt ? w.kb : w.ka, nnz,
                           ((uint64_t)1 << kwbits) - 1, w.wstart, w.wend);
        GRWS_LAUNCH_CHECK();
        hipLaunchKernelGGL(keyed_big_kernel, dim3(grid_for(s.W)), dim3(kBlk), 0, stream, w.wstart, w.wend, s.W,
                           w.blist, w.err);
        GRWS_LAUNCH_CHECK();
        int32_t h[4] = {0, 0, 0, 0};
        GRWS_HIP(hipMemcpyAsync(h, w.err, 4 * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
        GRWS_HIP(hipStreamSynchronize(stream));
        GRWS_TRY(report_input_error(h[0], "bcsr_build"));
        if (h[3] == 0) {
            per_window = keyed = true;
            nbig = h[1];
        } else {  // the global sort rebuilds its keys and bounds
            GRWS_TRY(fill_i64(w.wstart, s.W, 0, stream));
            GRWS_TRY(fill_i64(w.wend, s.W, 0, stream));
        }
    }
    if (per_window) {
        GRWS_TRY(fill_i32(w.err + 2, 1, 1, stream));
        const unsigned wg = (unsigned)std::min<int64_t>(s.W, 4096);
        const unsigned wgs = (unsigned)std::min<int64_t>(s.W, 16384);  // the 2,048-edge class, 256 threads
        int32_t* ucol = reinterpret_cast<int32_t*>(w.va);
        if (keyed) {
            // sorted keys and values in ka / va or kb / vb; the records and
            // distinct columns go to the other pair (path 2: kb / vb)
            const uint64_t* tk = kalt ? w.kb : w.ka;
            const uint32_t* tv = kalt ? w.vb : w.va;
            uint64_t* rk = kalt ? w.ka : w.kb;
            ucol = reinterpret_cast<int32_t*>(kalt ? w.va : w.vb);
            if (!kalt) GRWS_TRY(fill_i32(w.err + 2, 1, 2, stream));
            SideStream ss(stream);
            if (nbig > 0) {
                GRWS_TRY(ss.fork());
                const hipStream_t side = ss.side;
                hipLaunchKernelGGL((win_sort_big_kernel<true>), dim3(std::min(nbig, 1024)), dim3(kWinBlk), 0, side,
                                   nullptr, nullptr, nullptr, tk, tv, kwbits, nnz, s.R, w.blist, nbig,
                                   s.C, (int)tile_cols, reinterpret_cast<uint32_t*>(w.uidx),
                                   reinterpret_cast<uint32_t*>(w.uflag), rk, ucol, w.wstart, w.wend, w.wtiles, w.err);
                GRWS_LAUNCH_CHECK();
            }
            hipLaunchKernelGGL((win_sort_kernel<2048, 256, true>), dim3(wgs), dim3(256), 0, stream, nullptr, nullptr,
                               nullptr, tk, tv, kwbits, nnz, s.R, s.W, s.C, (int)tile_cols, rk, ucol, w.wstart, w.wend,
                               w.wtiles, w.err);
            GRWS_LAUNCH_CHECK();
            hipLaunchKernelGGL((win_sort_kernel<8192, kWinBlk, true>), dim3(wg), dim3(kWinBlk), 0, stream, nullptr,
                               nullptr, nullptr, tk, tv, kwbits, nnz, s.R, s.W, s.C, (int)tile_cols, rk, ucol, w.wstart,
                               w.wend, w.wtiles, w.err);
            GRWS_LAUNCH_CHECK();
            hipLaunchKernelGGL((win_sort_kernel<16384, kWinBlk, true>), dim3(std::min<unsigned>(wg, 512)), dim3(kWinBlk), 0,
                               stream, nullptr, nullptr, nullptr, tk, tv, kwbits, nnz, s.R, s.W, s.C, (int)tile_cols,
                               rk, ucol, w.wstart, w.wend, w.wtiles, w.err);
            GRWS_LAUNCH_CHECK();
            GRWS_TRY(ss.join());
        } else {
            SideStream ss(stream);
            if (nbig > 0) {
                GRWS_TRY(ss.fork());
                const hipStream_t side = ss.side;
                hipLaunchKernelGGL((win_sort_big_kernel<false>), dim3(std::min(nbig, 1024)), dim3(kWinBlk), 0, side,
                                   row_ptr, cols, values, nullptr, nullptr, 0, nnz, s.R, w.blist,
                                   nbig, num_cols, (int)tile_cols, reinterpret_cast<uint32_t*>(w.uidx),
                                   reinterpret_cast<uint32_t*>(w.uflag), w.ka, ucol, w.wstart, w.wend, w.wtiles,
                                   w.err);
                GRWS_LAUNCH_CHECK();
            }
            hipLaunchKernelGGL((win_sort_kernel<2048, 256, false>), dim3(wgs), dim3(256), 0, stream, row_ptr, cols,
                               values, nullptr, nullptr, 0, nnz, s.R, s.W, num_cols, (int)tile_cols, w.ka, ucol,
                               w.wstart, w.wend, w.wtiles, w.err);
            GRWS_LAUNCH_CHECK();
            hipLaunchKernelGGL((win_sort_kernel<8192, kWinBlk, false>), dim3(wg), dim3(kWinBlk), 0, stream, row_ptr,
                               cols, values, nullptr, nullptr, 0, nnz, s.R, s.W, num_cols, (int)tile_cols, w.ka, ucol,
                               w.wstart, w.wend, w.wtiles, w.err);
            GRWS_LAUNCH_CHECK();
            hipLaunchKernelGGL((win_sort_kernel<16384, kWinBlk, false>), dim3(std::min<unsigned>(wg, 512)), dim3(kWinBlk), 0,
                               stream, row_ptr, cols, values, nullptr, nullptr, 0, nnz, s.R, s.W, num_cols,
                               (int)tile_cols, w.ka, ucol, w.wstart, w.wend, w.wtiles, w.err);
            GRWS_LAUNCH_CHECK();
            GRWS_TRY(ss.join());
        }
    }
    bool alt = false;
    if (nnz > 0 && !per_window) {
        if (rows) {
            hipLaunchKernelGGL(build_keys_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, row_ptr, rows, cols,
                               values, nnz, num_rows, num_cols, (int)transpose, s.cbits, 0, w.ka, w.va, w.err);
        } else {
            // every edge lies in some row's range (check_row_ptr_kernel flags
            // a row pointer that does not cover [0, nnz) exactly)
            const int64_t wg = std::min<int64_t>((num_rows + 3) / 4, 65536);
            hipLaunchKernelGGL(build_keys_rows_kernel, dim3((unsigned)std::max<int64_t>(wg, 1)), dim3(256), 0, stream,
                               row_ptr, cols, values, nnz, num_rows, num_cols, (int)transpose, s.cbits, 0, w.ka,
                               w.va, w.err);
        }
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(radix_sort_pairs(w.ka, w.va, w.kb, w.vb, nnz, s.bits, w.sort_ws, w.sort_bytes, stream, &alt));
        const uint64_t* k = alt ? w.kb : w.ka;
        hipLaunchKernelGGL(unique_flag_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, k, nnz, w.uflag);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(scan_i32_to_i64(w.uflag, w.uidx, nnz, false, w.scan_ws, w.scan_bytes, stream));
        hipLaunchKernelGGL(window_bounds_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, k, nnz, s.cbits + 4,
                           w.uflag, w.uidx, w.wstart, w.wend);
        GRWS_LAUNCH_CHECK();
    }
    if (!per_window) {
        hipLaunchKernelGGL(window_tiles_kernel, dim3(grid_for(s.W)), dim3(kBlk), 0, stream, w.wstart, w.wend, s.W,
                           (int)tile_cols, w.wtiles);
        GRWS_LAUNCH_CHECK();
    }
    GRWS_TRY(scan_i32_to_i64(w.wtiles, window_offset, s.W, false, w.scan_ws, w.scan_bytes, stream));
    int64_t T = 0;
    int32_t e = 0;
    GRWS_HIP(hipMemcpyAsync(&T, window_offset + s.W, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_TRY(read_error_flag(w.err, stream, &e));
    GRWS_HIP(hipStreamSynchronize(stream));
    GRWS_TRY(report_input_error(e, "bcsr_build"));
    *num_tiles_out = T;
    return GRWS_OK;
}

extern "C" int grws_bcsr_build_fill(int64_t nnz, int64_t num_rows, int64_t num_cols, int32_t tile_cols,
                                    int32_t transpose, const int64_t* window_offset, int64_t num_tiles,
                                    int32_t* col_indices, void* values, int32_t values_dtype, void* workspace,
                                    size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(refuse_capture(stream, "bcsr_build_fill"));
    GRWS_CHECK_ARG(nnz >= 0 && num_rows >= 0 && num_cols >= 0 && num_tiles >= 0, "bcsr_build: negative size");
    GRWS_CHECK_ARG(tile_cols == 8 || tile_cols == 16, "bcsr_build: tile_cols must be 8 or 16 (got %d)", tile_cols);
    if (values_dtype != GRWS_F32 && values_dtype != GRWS_F16 && values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "bcsr_build: unsupported values dtype %d", values_dtype);
    if (num_tiles == 0) return GRWS_OK;
    GRWS_CHECK_ARG(window_offset && col_indices && values, "bcsr_build: null output");
    BuildShape s = build_shape(nnz, num_rows, num_cols, transpose);
    Carver cv(workspace, workspace_bytes);
    BuildWs w;
    carve_build(cv, s, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "bcsr_build: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int passes = (s.bits + 7) / 8;
    const bool alt = nnz > 1 && (passes & 1);
    const uint64_t* k = alt ? w.kb : w.ka;
    const uint32_t* v = alt ? w.vb : w.va;
    // the path the count phase took: err[2] = 0 the global sort; 1 window by
    // window with the records and distinct columns in ka / va, 2 in kb / vb
    // (its fill writes every tile, padding included)
    int32_t hf[3] = {0, 0, 0};  // err[0..2]: flags, windows over kWinCap edges, path
    if (nnz > 0) {
        GRWS_HIP(hipMemcpyAsync(hf, w.err, 3 * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
        GRWS_HIP(hipStreamSynchronize(stream));
    }
    const int32_t path = hf[2];
    const int nbig = path != 0 ? hf[1] : 0;
    if (path == 0) {
        GRWS_TRY(fill_i32(col_indices, num_tiles * tile_cols, -1, stream));
        GRWS_TRY(fill_bytes_zero(values, (size_t)num_tiles * 16 * tile_cols * dtype_size(values_dtype), stream));
    }
    if (nnz == 0) return GRWS_OK;
    const unsigned wg = (unsigned)std::min<int64_t>(s.W, 4096);
    const int aligned = (reinterpret_cast<uintptr_t>(values) & 15) == 0;
    const uint64_t* wrec = path == 2 ? w.kb : w.ka;
    const int32_t* wcol = reinterpret_cast<const int32_t*>(path == 2 ? w.vb : w.va);
    SideStream ss(stream);
    if (nbig > 0) GRWS_TRY(ss.fork());
    const hipStream_t side = ss.side;
#define GRWS_BUILD_FILL(VT)                                                                                        \
    if (path != 0)                                                                                                 \
    {                                                                                                              \
        if (nbig > 0)                                                                                              \
            hipLaunchKernelGGL(win_fill_big_kernel<VT>, dim3(std::min(nbig, 1024)), dim3(kWinBlk), 0, side,        \
                               wrec, wcol, w.wstart, w.wend, window_offset, w.blist, nbig, (int)tile_cols,        \
                               col_indices, values, aligned, w.err);                                               \
        hipLaunchKernelGGL((win_fill_kernel<2048, 256, VT>), dim3((unsigned)std::min<int64_t>(s.W, 16384)),     \
                           dim3(256), 0, stream, wrec, wcol, w.wstart, w.wend, window_offset, s.W, (int)tile_cols, \
                           col_indices, values, aligned, w.err);                                                   \
        hipLaunchKernelGGL((win_fill_kernel<8192, kWinBlk, VT>), dim3(wg), dim3(kWinBlk), 0, stream, wrec, wcol,   \
                           w.wstart, w.wend, window_offset, s.W, (int)tile_cols, col_indices, values, aligned,     \
                           w.err);                                                                                 \
        hipLaunchKernelGGL((win_fill_kernel<16384, kWinBlk, VT>), dim3(std::min<unsigned>(wg, 512)), dim3(kWinBlk), \
                           0, stream, wrec, wcol, w.wstart, w.wend, window_offset, s.W, (int)tile_cols,            \
                           col_indices, values, aligned, w.err);                                                   \
    } else                                                                                                         \
        hipLaunchKernelGGL(build_scatter_kernel<VT>, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, k, v, nnz, s.cbits, \
                           w.uflag, w.uidx, w.wstart, window_offset, (int)tile_cols, col_indices, values, w.err)
    switch (values_dtype) {
        case GRWS_F32: GRWS_BUILD_FILL(float); break;
        case GRWS_F16: GRWS_BUILD_FILL(_Float16); break;
        default: GRWS_BUILD_FILL(__hip_bfloat16); break;
    }
#undef GRWS_BUILD_FILL
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(ss.join());
    return GRWS_OK;
}

// ---------------------------------------------------------------------------
// BCSR -> COO
// ---------------------------------------------------------------------------
extern "C" size_t grws_bcsr_to_coo_workspace_bytes(int64_t num_tiles) {
    if (num_tiles < 0) return 0;
    Sizer s;
    s.take<int32_t>((size_t)num_tiles + 1);
    s.take<int64_t>((size_t)num_tiles + 2);
    s.used += scan_workspace_bytes(num_tiles) + 256;
    return s.used;
}

static int coo_ws(void* workspace, size_t workspace_bytes, int64_t T, int32_t** cnt, int64_t** toff, char** scan_ws,
                  size_t* scan_bytes) {
    Carver cv(workspace, workspace_bytes);
    *cnt = cv.take<int32_t>(T + 1);
    *toff = cv.take<int64_t>(T + 2);
    *scan_bytes = scan_workspace_bytes(T);
    *scan_ws = cv.take<char>(*scan_bytes);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "bcsr_to_coo: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    return GRWS_OK;
}

static int check_bcsr(const grws_bcsr* A, const char* who) {
    GRWS_CHECK_ARG(A != nullptr, "%s: null graph", who);
    GRWS_CHECK_ARG(A->tile_rows == 16, "%s: tile_rows must be 16", who);
    GRWS_CHECK_ARG(A->tile_cols == 8 || A->tile_cols == 16, "%s: tile_cols must be 8 or 16", who);
    GRWS_CHECK_ARG(A->num_windows >= 0 && A->num_tiles >= 0, "%s: negative size", who);
    if (A->values_dtype != GRWS_F32 && A->values_dtype != GRWS_F16 && A->values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "%s: unsupported values dtype %d", who, A->values_dtype);
    if (A->num_tiles > 0) GRWS_CHECK_ARG(A->window_offset && A->col_indices && A->values, "%s: null arrays", who);
    GRWS_CHECK_ARG(A->num_windows * 16 <= INT32_MAX, "%s: rows exceed int32 ids", who);
    return GRWS_OK;
}

extern "C" int grws_bcsr_to_coo_count(const grws_bcsr* A, int64_t num_cols, void* workspace, size_t workspace_bytes,
                                      int64_t* nnz_out, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_bcsr(A, "bcsr_to_coo"));
    GRWS_CHECK_ARG(nnz_out != nullptr && num_cols >= 0, "bcsr_to_coo: bad argument");
    const int64_t T = A->num_tiles;
    if (T == 0) {
        *nnz_out = 0;
        return GRWS_OK;
    }
    int32_t* cnt;
    int64_t* toff;
    char* sws;
    size_t sb;
    GRWS_TRY(coo_ws(workspace, workspace_bytes, T, &cnt, &toff, &sws, &sb));
    const int64_t nch = T * 16 * A->tile_cols / (16 / dtype_size(A->values_dtype));
    const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((nch + 255) / 256, 65536));
    const bool al = (reinterpret_cast<uintptr_t>(A->values) & 15) == 0;
#define GRWS_TILE_NNZ(VT)                                                                                          \
    if (al)                                                                                                        \
        hipLaunchKernelGGL((tile_nnz_kernel<VT, true>), dim3(grid), dim3(256), 0, stream, A->col_indices,          \
                           A->values, T, A->tile_cols, num_cols, cnt);                                             \
    else                                                                                                           \
        hipLaunchKernelGGL((tile_nnz_kernel<VT, false>), dim3(grid), dim3(256), 0, stream, A->col_indices,         \
                           A->values, T, A->tile_cols, num_cols, cnt)
    switch (A->values_dtype) {
        case GRWS_F32: GRWS_TILE_NNZ(float); break;
        case GRWS_F16: GRWS_TILE_NNZ(_Float16); break;
        default: GRWS_TILE_NNZ(__hip_bfloat16); break;
    }
#undef GRWS_TILE_NNZ
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(cnt, toff, T, false, sws, sb, stream));
    int64_t nnz = 0;
    GRWS_HIP(hipMemcpyAsync(&nnz, toff + T, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    *nnz_out = nnz;
    return GRWS_OK;
}

extern "C" int grws_bcsr_to_coo_fill(const grws_bcsr* A, int64_t num_cols, int32_t* rows, int32_t* cols,
                                     float* values, void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_bcsr(A, "bcsr_to_coo"));
    GRWS_CHECK_ARG(num_cols >= 0, "bcsr_to_coo: negative num_cols");
    const int64_t T = A->num_tiles;
    if (T == 0) return GRWS_OK;
    GRWS_CHECK_ARG(rows && cols && values, "bcsr_to_coo: null output");
    int32_t* cnt;
    int64_t* toff;
    char* sws;
    size_t sb;
    GRWS_TRY(coo_ws(workspace, workspace_bytes, T, &cnt, &toff, &sws, &sb));
    // the count's per-tile counts are spent (toff holds their scan): the
    // array takes each tile's window
    GRWS_TRY(fill_i32(cnt, T, 0, stream));
    hipLaunchKernelGGL(tile_window_kernel, dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>(A->num_windows, 8192))),
                       dim3(256), 0, stream, A->window_offset, A->num_windows, T, cnt);
    GRWS_LAUNCH_CHECK();
    const int64_t nch = T * 16 * A->tile_cols / (16 / dtype_size(A->values_dtype));
    const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((nch + 255) / 256, 65536));
    const bool al = (reinterpret_cast<uintptr_t>(A->values) & 15) == 0;
#define GRWS_TILE_COO(VT)                                                                                          \
    if (al)                                                                                                        \
        hipLaunchKernelGGL((tile_to_coo_kernel<VT, true>), dim3(grid), dim3(256), 0, stream, cnt, A->col_indices,  \
                           A->values, T, A->tile_cols, num_cols, toff, rows, cols, values);                        \
    else                                                                                                           \
        hipLaunchKernelGGL((tile_to_coo_kernel<VT, false>), dim3(grid), dim3(256), 0, stream, cnt, A->col_indices, \
                           A->values, T, A->tile_cols, num_cols, toff, rows, cols, values)
    switch (A->values_dtype) {
        case GRWS_F32: GRWS_TILE_COO(float); break;
        case GRWS_F16: GRWS_TILE_COO(_Float16); break;
        default: GRWS_TILE_COO(__hip_bfloat16); break;
    }
#undef GRWS_TILE_COO
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

// ---------------------------------------------------------------------------
// COO -> CSR  (data/bcsr.py:162-187)
// ---------------------------------------------------------------------------
extern "C" size_t grws_coo_to_csr_workspace_bytes(int64_t nnz, int64_t num_rows, int64_t num_cols) {
    if (nnz < 0 || num_rows < 0 || num_cols < 0) return 0;
    const int64_t n = nnz > 0 ? nnz : 1;
    Sizer s;
    s.take<uint64_t>(n);
    s.take<uint64_t>(n);
    s.take<uint32_t>(n);
    s.take<uint32_t>(n);
    s.take<int32_t>(64);
    s.used += radix_sort_workspace_bytes(n) + 256;
    return s.used;
}

extern "C" int grws_coo_to_csr(const int32_t* src, const int32_t* dst, const float* weights, int64_t nnz,
                               int64_t num_rows, int64_t num_cols, int64_t* row_ptr, int32_t* col_idx, float* values,
                               void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(nnz >= 0 && num_rows >= 0 && num_cols >= 0, "coo_to_csr: negative size");
    GRWS_CHECK_ARG(num_rows <= INT32_MAX && num_cols <= INT32_MAX, "coo_to_csr: dimensions exceed int32 ids");
    GRWS_CHECK_ARG(nnz <= (int64_t)UINT32_MAX, "coo_to_csr: more than 2^32-1 edges");
    GRWS_CHECK_ARG(row_ptr != nullptr, "coo_to_csr: null row_ptr");
    if (nnz > 0) GRWS_CHECK_ARG(src && dst && col_idx && values, "coo_to_csr: null array");
    const int64_t n = nnz > 0 ? nnz : 1;
    Carver cv(workspace, workspace_bytes);
    uint64_t* ka = cv.take<uint64_t>(n);
    uint64_t* kb = cv.take<uint64_t>(n);
    uint32_t* va = cv.take<uint32_t>(n);
    uint32_t* vb = cv.take<uint32_t>(n);
    int32_t* err = cv.take<int32_t>(64);
    const size_t sort_bytes = radix_sort_workspace_bytes(n);
    char* sort_ws = cv.take<char>(sort_bytes);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "coo_to_csr: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    const int cbits = bits_for(num_cols);
    const int bits = bits_for(num_rows) + cbits;
    GRWS_TRY(fill_i32(err, 1, 0, stream));
    const uint64_t* k = ka;
    const uint32_t* p = va;
    if (nnz > 0) {
        hipLaunchKernelGGL(coo_keys_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, src, dst, nnz, num_rows,
                           num_cols, cbits, ka, va, err);
        GRWS_LAUNCH_CHECK();
        bool alt = false;
        GRWS_TRY(radix_sort_pairs(ka, va, kb, vb, nnz, bits, sort_ws, sort_bytes, stream, &alt));
        k = alt ? kb : ka;
        p = alt ? vb : va;
        hipLaunchKernelGGL(coo_emit_kernel, dim3(grid_for(nnz)), dim3(kBlk), 0, stream, k, p, nnz, cbits, weights,
                           col_idx, values);
        GRWS_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(coo_row_ptr_kernel, dim3(grid_for(num_rows + 1)), dim3(kBlk), 0, stream, k, nnz, cbits,
                       num_rows, row_ptr);
    GRWS_LAUNCH_CHECK();
    int32_t e = 0;
    GRWS_TRY(read_error_flag(err, stream, &e));
    GRWS_HIP(hipStreamSynchronize(stream));
    return report_input_error(e, "coo_to_csr");
}
