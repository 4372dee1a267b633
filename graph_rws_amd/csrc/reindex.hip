// Global -> local column reindex with pruning (gfx950).
//
// Replaces reindex_and_prune_kernel (core/include/reindex.cuh:33-102,
// launched by core/wrapper/reindex_wrapper.cu:27-68).  For every column slot
// g: target window = g / tile_rows with C truncation, binary search in the
// sorted active windows; a hit maps to idx * tile_rows + g % tile_rows (C
// remainder, so -1 stays -1 when window 0 is active), a miss maps to column
// 0 and zeroes that tile column's tile_rows values in place.  Index math is
// 64-bit (the reference counts slots in int, reindex_wrapper.cu:45).
#include "grws_internal.h"

namespace grws {
namespace {

template <typename VT>
__global__ void reindex_prune_kernel(const int32_t* __restrict__ in_cols, int64_t n, VT* __restrict__ values,
                                     const int32_t* __restrict__ active, int64_t num_active, int tile_rows,
                                     int tile_cols, int32_t* __restrict__ out_cols) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int32_t g = in_cols[idx];
    const int32_t target = g / tile_rows;
    int64_t lo = 0, hi = num_active - 1, found = -1;
    while (lo <= hi) {
        const int64_t mid = (lo + hi) >> 1;
        const int32_t w = active[mid];
        if (w == target) {
            found = mid;
            break;
        }
        if (w < target) lo = mid + 1;
        else hi = mid - 1;
    }
    if (found >= 0) {
        out_cols[idx] = (int32_t)(found * tile_rows + g % tile_rows);
    } else {
        out_cols[idx] = 0;
        const int64_t blk = idx / tile_cols;
        const int64_t c = idx % tile_cols;
        VT* v = values + blk * tile_rows * tile_cols + c;
        for (int r = 0; r < tile_rows; ++r) v[(int64_t)r * tile_cols] = VT(0);
    }
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" int grws_reindex_prune(const int32_t* in_cols, int64_t num_indices, void* values, int32_t values_dtype,
                                  const int32_t* active_windows, int64_t num_active, int32_t tile_rows,
                                  int32_t tile_cols, int32_t* out_cols, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(num_indices >= 0 && num_active >= 0, "reindex: negative size");
    GRWS_CHECK_ARG(tile_rows > 0 && tile_cols > 0, "reindex: tile sizes must be positive");
    GRWS_CHECK_ARG(num_indices % tile_cols == 0, "reindex: num_indices is not a multiple of tile_cols");
    if (values_dtype != GRWS_F32 && values_dtype != GRWS_F16 && values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "reindex: unsupported values dtype %d", values_dtype);
    if (num_indices == 0) return GRWS_OK;
    GRWS_CHECK_ARG(in_cols && out_cols && values, "reindex: null pointer");
    if (num_active > 0) GRWS_CHECK_ARG(active_windows != nullptr, "reindex: null active_windows");
    const unsigned grid = (unsigned)((num_indices + 255) / 256);
    switch (values_dtype) {
        case GRWS_F32:
            hipLaunchKernelGGL(reindex_prune_kernel<float>, dim3(grid), dim3(256), 0, stream, in_cols, num_indices,
                               static_cast<float*>(values), active_windows, num_active, (int)tile_rows,
                               (int)tile_cols, out_cols);
            break;
        case GRWS_F16:
            hipLaunchKernelGGL(reindex_prune_kernel<_Float16>, dim3(grid), dim3(256), 0, stream, in_cols, num_indices,
                               static_cast<_Float16*>(values), active_windows, num_active, (int)tile_rows,
                               (int)tile_cols, out_cols);
            break;
        default:
            hipLaunchKernelGGL(reindex_prune_kernel<uint16_t>, dim3(grid), dim3(256), 0, stream, in_cols, num_indices,
                               static_cast<uint16_t*>(values), active_windows, num_active, (int)tile_rows,
                               (int)tile_cols, out_cols);
            break;
    }
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}
