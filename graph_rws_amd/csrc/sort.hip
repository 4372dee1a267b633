// Stable LSD radix sort of 64-bit keys with a 32-bit payload (gfx950).
//
// Used by the device BCSR builder (key = window, column, row-in-window) and
// by the sampler's unique-and-relabel (key = global node id).  Each pass over
// one 8-bit digit is three launches:
//   1. digit histogram per tile of 256 x iters keys (wave64 match by ballot,
//      one LDS atomic per distinct digit per wave); iters is 16 for large
//      inputs and as small as 1 below 16k keys, so that a small sort still
//      spreads over up to 64 work-groups instead of a few long ones,
//   2. exclusive scan of the digit-major [256][tiles] histogram, which gives
//      every (digit, tile) its output base in stable order,
//   3. stable scatter: each tile re-reads its keys in index order and ranks
//      them by (wave prefix across waves, ballot rank within the wave).
// Only ceil(bits / 8) passes run, so keys that use few bits sort fast.
#include "grws_internal.h"

namespace grws {

namespace {

constexpr int kRsBlock = 256;
constexpr int kRsWaves = kRsBlock / kWave;
constexpr int kRsMaxIters = 16;

// Keys per tile: 256 x iters, iters = ceil(n / 16k) clamped to [1, 16]: up
// to 256k keys a sort has at most 64 tiles, so its 256 x tiles digit counts
// take the one-launch scan (16k elements).
inline int radix_iters(int64_t n) {
    const int64_t it = (n + 16383) / 16384;
    return (int)(it < 1 ? 1 : (it > kRsMaxIters ? kRsMaxIters : it));
}

// Lanes of the wave whose 8-bit digit equals this lane's (valid lanes only).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid) {
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bb = __ballot(bit);
        m &= bit ? bb : ~bb;
    }
    return m;
}

__global__ __launch_bounds__(kRsBlock) void radix_hist_kernel(const uint64_t* __restrict__ keys, int64_t n, int shift,
                                                              int64_t ntiles, int iters, int32_t* __restrict__ counts) {
    __shared__ int32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kRsBlock * iters;
    for (int it = 0; it < iters; ++it) {
        const int64_t i = base + (int64_t)it * kRsBlock + threadIdx.x;
        const bool valid = i < n;
        const uint32_t d = valid ? (uint32_t)(keys[i] >> shift) & 255u : 0u;
        const uint64_t m = match_digit(d, valid);
        if (valid && (m & lanemask_lt()) == 0) atomicAdd(&h[d], (int32_t)__popcll(m));
    }
    __syncthreads();
    counts[(int64_t)threadIdx.x * ntiles + blockIdx.x] = h[threadIdx.x];
}

__global__ __launch_bounds__(kRsBlock) void radix_scatter_kernel(const uint64_t* __restrict__ kin,
                                                                 const uint32_t* __restrict__ vin, int64_t n,
                                                                 int shift, int64_t ntiles, int iters,
                                                                 const int64_t* __restrict__ offsets,
                                                                 uint64_t* __restrict__ kout,
                                                                 uint32_t* __restrict__ vout) {
    __shared__ int64_t base_off[256];
    __shared__ int32_t wcnt[kRsWaves][256];
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    base_off[tid] = offsets[(int64_t)tid * ntiles + blockIdx.x];
    const int64_t tile0 = (int64_t)blockIdx.x * kRsBlock * iters;
    for (int it = 0; it < iters; ++it) {
        const int64_t i = tile0 + (int64_t)it * kRsBlock + tid;
        const bool valid = i < n;
        uint64_t k = 0;
        uint32_t v = 0;
        if (valid) {
            k = kin[i];
            if (vin) v = vin[i];
        }
        const uint32_t d = (uint32_t)(k >> shift) & 255u;
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) wcnt[w][tid] = 0;
        __syncthreads();
        const uint64_t m = match_digit(d, valid);
        const int rank = __popcll(m & lanemask_lt());
        if (valid && rank == 0) wcnt[wave][d] = __popcll(m);
        __syncthreads();
        int32_t tot = 0;
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) {
            const int32_t t = wcnt[w][tid];
            wcnt[w][tid] = tot;
            tot += t;
        }
        __syncthreads();
        if (valid) {
            const int64_t pos = base_off[d] + wcnt[wave][d] + rank;
            kout[pos] = k;
            if (vin) vout[pos] = v;
        }
        __syncthreads();
        base_off[tid] += tot;
    }
}

}  // namespace

// Sized for any sort of at most n keys (callers size by a capacity and sort
// what a batch holds): up to 256k keys a sort uses at most 64 tiles (at most
// ceil(n / 256) of them), above it ceil(n / 4096).
size_t radix_sort_workspace_bytes(int64_t n) {
    const int64_t small = (n + kRsBlock - 1) / kRsBlock;
    const int64_t big = (n + (int64_t)kRsBlock * kRsMaxIters - 1) / ((int64_t)kRsBlock * kRsMaxIters);
    const int64_t ntiles = std::max(std::min<int64_t>(small, 64), big);
    Sizer s;
    s.take<int32_t>((size_t)(256 * ntiles + 1));
    s.take<int64_t>((size_t)(256 * ntiles + 2));
    s.used += scan_workspace_bytes(256 * ntiles) + 256;
    return s.used;
}

int radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt, int64_t n, int bits,
                     void* ws, size_t ws_bytes, hipStream_t stream, bool* result_in_alt) {
    *result_in_alt = false;
    if (n <= 1 || bits <= 0) return GRWS_OK;
    if (bits > 64) bits = 64;
    const int iters = radix_iters(n);
    const int64_t tile = (int64_t)kRsBlock * iters;
    const int64_t ntiles = (n + tile - 1) / tile;
    if (ntiles > INT32_MAX / 2) return set_error(GRWS_E_INVALID, "radix sort: %lld keys is too many", (long long)n);
    Carver cv(ws, ws_bytes);
    int32_t* counts = cv.take<int32_t>(256 * ntiles + 1);
    int64_t* offsets = cv.take<int64_t>(256 * ntiles + 2);
    const size_t scan_bytes = scan_workspace_bytes(256 * ntiles);
    char* scan_ws = cv.take<char>(scan_bytes);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "radix sort: workspace too small (%zu < %zu)", ws_bytes, cv.used);
    uint64_t* ka = keys;
    uint32_t* va = vals;
    uint64_t* kb = keys_alt;
    uint32_t* vb = vals_alt;
    bool alt = false;
    for (int shift = 0; shift < bits; shift += 8) {
        hipLaunchKernelGGL(radix_hist_kernel, dim3((unsigned)ntiles), dim3(kRsBlock), 0, stream, ka, n, shift, ntiles,
                           iters, counts);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(scan_i32_to_i64(counts, offsets, 256 * ntiles, false, scan_ws, scan_bytes, stream));
        hipLaunchKernelGGL(radix_scatter_kernel, dim3((unsigned)ntiles), dim3(kRsBlock), 0, stream, ka, va, n, shift,
                           ntiles, iters, offsets, kb, vb);
        GRWS_LAUNCH_CHECK();
        std::swap(ka, kb);
        std::swap(va, vb);
        alt = !alt;
    }
    *result_in_alt = alt;
    return GRWS_OK;
}

}  // namespace grws
