// Device-wide prefix sums and fills.  A scan is one launch up to 16,384
// elements, reduce + scan (the scan adds the preceding tiles' sums itself)
// up to 1,024 tiles of 4,096, and reduce + scan of the tile sums + scan
// beyond that.  Within a tile each thread scans 16 consecutive elements in
// registers; one wave scan and one barrier join the threads.
#include "grws_internal.h"

namespace grws {

namespace {

constexpr int kScanBlock = 256;
constexpr int kScanIters = 16;
constexpr int64_t kScanTile = (int64_t)kScanBlock * kScanIters;

template <typename TIn>
__global__ __launch_bounds__(kScanBlock) void scan_reduce_kernel(const TIn* __restrict__ in, int64_t n,
                                                                 int64_t* __restrict__ partial) {
    __shared__ int64_t smem[kScanBlock / kWave + 1];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int64_t s = 0;
    for (int it = 0; it < kScanIters; ++it) {
        int64_t i = base + (int64_t)it * kScanBlock + threadIdx.x;
        if (i < n) s += (int64_t)in[i];
    }
    int64_t total;
    block_incl_scan<kScanBlock>(s, smem, &total);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// Single-block exclusive scan of the per-block partials, in place.
__global__ __launch_bounds__(1024) void scan_partials_kernel(int64_t* __restrict__ partial, int64_t nb) {
    __shared__ int64_t smem[1024 / kWave + 1];
    int64_t carry = 0;
    for (int64_t base = 0; base < nb; base += 1024) {
        int64_t i = base + threadIdx.x;
        int64_t v = i < nb ? partial[i] : 0;
        int64_t total;
        int64_t inc = block_incl_scan<1024>(v, smem, &total);
        if (i < nb) partial[i] = carry + inc - v;
        carry += total;
    }
}

// Scans one tile of BLOCK * kScanIters elements starting at `base`: thread
// t owns the kScanIters consecutive elements at base + t * kScanIters and
// scans them serially in registers; one wave scan of the thread totals and
// one barrier for the wave totals give each thread its prefix.  dst[i] =
// carry + inclusive prefix for i < n.
template <typename TIn, int BLOCK>
__device__ __forceinline__ void scan_tile(const TIn* __restrict__ in, int64_t n, int64_t base, int64_t carry,
                                          int64_t* __restrict__ dst, int64_t* smem) {
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t t0 = base + (int64_t)threadIdx.x * kScanIters;
    int64_t v[kScanIters];
    if (t0 + kScanIters <= n) {
#pragma unroll
        for (int j = 0; j < kScanIters; ++j) v[j] = (int64_t)in[t0 + j];
    } else {
#pragma unroll
        for (int j = 0; j < kScanIters; ++j) v[j] = t0 + j < n ? (int64_t)in[t0 + j] : 0;
    }
    int64_t run = 0;
#pragma unroll
    for (int j = 0; j < kScanIters; ++j) {
        run += v[j];
        v[j] = run;
    }
    const int64_t inc = wave_incl_scan(run);
    if (lane == kWave - 1) smem[wave] = inc;
    __syncthreads();
    carry += inc - run;
    for (int k = 0; k < wave; ++k) carry += smem[k];
    if (t0 + kScanIters <= n) {
#pragma unroll
        for (int j = 0; j < kScanIters; ++j) dst[t0 + j] = carry + v[j];
    } else {
#pragma unroll
        for (int j = 0; j < kScanIters; ++j)
            if (t0 + j < n) dst[t0 + j] = carry + v[j];
    }
}

// CARRY 0: a single tile (carry 0); 1: the carry is the sum of the
// preceding tiles' partials, added up here (few tiles); 2: partial[] already
// holds each tile's exclusive prefix.
template <typename TIn, int BLOCK, int CARRY>
__global__ __launch_bounds__(BLOCK) void scan_down_kernel(const TIn* __restrict__ in, int64_t n,
                                                          const int64_t* __restrict__ partial,
                                                          int64_t* __restrict__ out, int inclusive) {
    __shared__ int64_t smem[BLOCK / kWave];
    const int64_t base = (int64_t)blockIdx.x * BLOCK * kScanIters;
    int64_t carry = 0;
    if constexpr (CARRY == 2) {
        carry = partial[blockIdx.x];
    } else if constexpr (CARRY == 1) {
        int64_t s = 0;
        for (int64_t k = threadIdx.x; k < (int64_t)blockIdx.x; k += BLOCK) s += partial[k];
#pragma unroll
        for (int d = kWave / 2; d > 0; d >>= 1) s += __shfl_xor(s, d, kWave);
        if (threadIdx.x % kWave == 0) smem[threadIdx.x / kWave] = s;
        __syncthreads();
        for (int k = 0; k < BLOCK / kWave; ++k) carry += smem[k];
        __syncthreads();
    }
    // exclusive results are written shifted by one: out[i+1] = inclusive[i]
    scan_tile<TIn, BLOCK>(in, n, base, carry, inclusive ? out : out + 1, smem);
    if (!inclusive && blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0;
}

constexpr int kSingleBlock = 1024;                                 // one-launch scans
constexpr int64_t kSingleTile = (int64_t)kSingleBlock * kScanIters;  // up to 16,384 elements
constexpr int64_t kMaxSummedTiles = 1024;                          // two-launch scans

template <typename TIn>
int scan_impl(const TIn* in, int64_t* out, int64_t n, bool inclusive, void* ws, size_t ws_bytes,
              hipStream_t stream) {
    GRWS_CHECK_ARG(n >= 0, "scan: negative length");
    if (n == 0) {
        if (!inclusive) return fill_i64(out, 1, 0, stream);
        return GRWS_OK;
    }
    const int inc = inclusive ? 1 : 0;
    if (n <= kSingleTile) {
        hipLaunchKernelGGL((scan_down_kernel<TIn, kSingleBlock, 0>), dim3(1), dim3(kSingleBlock), 0, stream, in, n,
                           (const int64_t*)nullptr, out, inc);
        GRWS_LAUNCH_CHECK();
        return GRWS_OK;
    }
    int64_t nb = (n + kScanTile - 1) / kScanTile;
    Carver cv(ws, ws_bytes);
    int64_t* partial = cv.take<int64_t>(nb);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "scan: workspace too small (%zu < %zu)", ws_bytes, cv.used);
    hipLaunchKernelGGL(scan_reduce_kernel<TIn>, dim3((unsigned)nb), dim3(kScanBlock), 0, stream, in, n, partial);
    GRWS_LAUNCH_CHECK();
    if (nb <= kMaxSummedTiles) {
        hipLaunchKernelGGL((scan_down_kernel<TIn, kScanBlock, 1>), dim3((unsigned)nb), dim3(kScanBlock), 0, stream,
                           in, n, partial, out, inc);
        GRWS_LAUNCH_CHECK();
        return GRWS_OK;
    }
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(1024), 0, stream, partial, nb);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL((scan_down_kernel<TIn, kScanBlock, 2>), dim3((unsigned)nb), dim3(kScanBlock), 0, stream, in,
                       n, partial, out, inc);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

template <typename T>
__global__ void fill_kernel(T* __restrict__ p, int64_t n, T v) {
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

template <typename T>
int fill_impl(T* p, int64_t n, T v, hipStream_t stream) {
    if (n <= 0) return GRWS_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, p, n, v);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

}  // namespace

size_t scan_workspace_bytes(int64_t n) {
    Sizer s;
    s.take<int64_t>((size_t)((n + kScanTile - 1) / kScanTile + 1));
    return s.used;
}

int scan_i32_to_i64(const int32_t* in, int64_t* out, int64_t n, bool inclusive, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
    return scan_impl<int32_t>(in, out, n, inclusive, ws, ws_bytes, stream);
}

int scan_i64_to_i64(const int64_t* in, int64_t* out, int64_t n, bool inclusive, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
    return scan_impl<int64_t>(in, out, n, inclusive, ws, ws_bytes, stream);
}

int fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream) { return fill_impl<int32_t>(p, n, v, stream); }
int fill_i64(int64_t* p, int64_t n, int64_t v, hipStream_t stream) { return fill_impl<int64_t>(p, n, v, stream); }

int fill_bytes_zero(void* p, size_t bytes, hipStream_t stream) {
    // callers pass 4-byte multiples; tail bytes handled through an int8 view
    int64_t words = (int64_t)(bytes / 4);
    GRWS_TRY(fill_impl<int32_t>(static_cast<int32_t*>(p), words, 0, stream));
    int64_t tail = (int64_t)(bytes % 4);
    if (tail) GRWS_TRY(fill_impl<int8_t>(static_cast<int8_t*>(p) + words * 4, tail, (int8_t)0, stream));
    return GRWS_OK;
}

}  // namespace grws
