// Row-gather ceiling probe (gfx950): measurement only, no counterpart in
// the reference.
//
// The SpMM's X reads are gathers of whole row segments at random row
// indices.  This kernel does those gathers and nothing else: every wave
// walks a list of row indices eight at a time and loads, per instruction,
// one 128-byte segment of each of the eight rows (lanes 8r .. 8r + 7 take
// row r's 16-byte pieces), two groups of eight rows in flight, and folds
// what it read into one word per wave.  Timed over a table that does not
// fit the L2s it gives the rate at which the chip serves random segments
// from beyond the L2 (the Infinity Cache and HBM); over a table that fits
// one XCD's L2, the L2's own rate.  bench.py reports both beside the
// SpMM's measured L2-miss traffic.
#include "grws_internal.h"

namespace grws {
namespace {

typedef uint32_t pu32x4_t __attribute__((ext_vector_type(4)));

template <int SEGS>
__global__ __launch_bounds__(256) void row_gather_probe_kernel(const void* table, uint32_t table_bytes, uint32_t pitch,
                                                               const int32_t* __restrict__ idx, int64_t groups,
                                                               uint32_t* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
    // offsets past table_bytes return zeros without a memory access
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(table), (short)0, (int)table_bytes, 0x00020000);
    pu32x4_t acc = {0u, 0u, 0u, 0u};
    for (int64_t q = 2 * wave; q < groups; q += 2 * nw) {
        pu32x4_t v[2][SEGS];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t gq = q + u;
            const uint32_t row = gq < groups ? (uint32_t)idx[gq * 8 + (lane >> 3)] : 0xffffffffu;
            const uint32_t base = row < table_bytes / pitch ? row * pitch + (uint32_t)(lane & 7) * 16u : table_bytes;
#pragma unroll
            for (int k = 0; k < SEGS; ++k)
                v[u][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(base + (uint32_t)k * 128u), 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int k = 0; k < SEGS; ++k) acc ^= v[u][k];
    }
    const uint32_t w = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    uint32_t folded = w;
    for (int m = 32; m >= 1; m >>= 1) folded ^= (uint32_t)__shfl_xor((int)folded, m, 64);
    if (lane == 0) out[wave] = folded;
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" int grws_probe_row_gather(const void* table, int64_t rows, int64_t pitch_bytes, int32_t segments,
                                     const int32_t* idx, int64_t n_idx, uint32_t* out, int32_t blocks,
                                     void* stream_) {
    clear_error();
    GRWS_CHECK_ARG(rows > 0 && pitch_bytes > 0 && pitch_bytes % 16 == 0, "probe_row_gather: bad table shape");
    GRWS_CHECK_ARG(segments == 1 || segments == 5 || segments == 10, "probe_row_gather: segments must be 1, 5 or 10");
    GRWS_CHECK_ARG((int64_t)segments * 128 <= pitch_bytes, "probe_row_gather: segments exceed the row pitch");
    GRWS_CHECK_ARG(rows * pitch_bytes <= (int64_t)INT32_MAX, "probe_row_gather: table exceeds 2^31 bytes");
    GRWS_CHECK_ARG(n_idx >= 0 && n_idx % 8 == 0, "probe_row_gather: n_idx must be a multiple of 8");
    GRWS_CHECK_ARG(blocks >= 1 && blocks <= 65536, "probe_row_gather: blocks must be 1..65536");
    GRWS_CHECK_ARG(table && idx && out, "probe_row_gather: null pointer");
    GRWS_CHECK_ARG(reinterpret_cast<uintptr_t>(table) % 16 == 0, "probe_row_gather: table not 16-byte aligned");
    const hipStream_t stream = as_stream(stream_);
    const uint32_t tb = (uint32_t)(rows * pitch_bytes), pitch = (uint32_t)pitch_bytes;
    const int64_t groups = n_idx / 8;
#define GRWS_PROBE(S)                                                                                      \
    if (segments == S)                                                                                     \
        hipLaunchKernelGGL(row_gather_probe_kernel<S>, dim3((unsigned)blocks), dim3(256), 0, stream, table, tb, \
                           pitch, idx, groups, out)
    GRWS_PROBE(1);
    GRWS_PROBE(5);
    GRWS_PROBE(10);
#undef GRWS_PROBE
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}
