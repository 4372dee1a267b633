// Device-wide prefix sums and fills (reduce-then-scan, three launches).
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

template <typename TIn>
__global__ __launch_bounds__(kScanBlock) void scan_down_kernel(const TIn* __restrict__ in, int64_t n,
                                                               const int64_t* __restrict__ partial,
                                                               int64_t* __restrict__ out, int inclusive) {
    __shared__ int64_t smem[kScanBlock / kWave + 1];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int64_t carry = partial[blockIdx.x];
    // exclusive results are written shifted by one: out[i+1] = inclusive[i]
    int64_t* dst = inclusive ? out : out + 1;
    for (int it = 0; it < kScanIters; ++it) {
        int64_t i = base + (int64_t)it * kScanBlock + threadIdx.x;
        int64_t v = i < n ? (int64_t)in[i] : 0;
        int64_t total;
        int64_t inc = block_incl_scan<kScanBlock>(v, smem, &total);
        if (i < n) dst[i] = carry + inc;
        carry += total;
    }
    if (!inclusive && blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0;
}

template <typename TIn>
int scan_impl(const TIn* in, int64_t* out, int64_t n, bool inclusive, void* ws, size_t ws_bytes,
              hipStream_t stream) {
    GRWS_CHECK_ARG(n >= 0, "scan: negative length");
    if (n == 0) {
        if (!inclusive) return fill_i64(out, 1, 0, stream);
        return GRWS_OK;
    }
    int64_t nb = (n + kScanTile - 1) / kScanTile;
    Carver cv(ws, ws_bytes);
    int64_t* partial = cv.take<int64_t>(nb);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "scan: workspace too small (%zu < %zu)", ws_bytes, cv.used);
    hipLaunchKernelGGL(scan_reduce_kernel<TIn>, dim3((unsigned)nb), dim3(kScanBlock), 0, stream, in, n, partial);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(1024), 0, stream, partial, nb);
    GRWS_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_down_kernel<TIn>, dim3((unsigned)nb), dim3(kScanBlock), 0, stream, in, n, partial,
                       out, inclusive ? 1 : 0);
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
