// Halo-aware subgraph repack (gfx950): the device part of the reference's
// BCSRSampler.repack_subgraph (sampler/sampler.py:420-690).
//
// Given a BCSR graph and an ascending list of window ids, the repack
//   * gathers the selected windows' tiles (columns and values) into a new
//     BCSR whose window i is selected window i;
//   * takes the internal nodes (the selected windows' rows below num_nodes,
//     window order then row order) and the external candidates (valid
//     neighbour columns that are not internal), the latter ascending;
//   * keeps every candidate, or -- when there are more than a budget -- a
//     caller-chosen ascending subset;
//   * relabels columns to positions in [internal..., kept external...]
//     (dropped or invalid columns -1, their 16 values zeroed), and derives
//     the "inner" copy in which every column >= num_internal is masked too.
// The reference builds this from torch.unique, a dense boolean mask, a
// dense global -> local map and masked fills; here a dense bitmap marks the
// candidates (ascending order falls out of a popcount prefix, no sort) and a
// dense int32 node map relabels, both caller-owned state that every call
// leaves as it found it (all 0 / all -1).  Three calls:
//   grws_repack_prepare    offsets, candidate bitmap, counts (one sync)
//   grws_repack_externals  the candidates ascending (only when over budget)
//   grws_repack_finish     relabel, gather values, restore state (one sync)
#include "grws_internal.h"

namespace grws {
namespace {

constexpr int kBlk = 256;

inline unsigned grid_for(int64_t n, int64_t per = kBlk) {
    int64_t g = (n + per - 1) / per;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (unsigned)g;
}

enum : int32_t { kErrOrder = 1, kErrRange = 2 };

// Index i of the selected window holding output tile t: new_off[i] <= t < new_off[i+1].
__device__ __forceinline__ int64_t window_of_tile(const int64_t* __restrict__ new_off, int64_t n_sel, int64_t t) {
    int64_t lo = 0, hi = n_sel;  // invariant: new_off[lo] <= t < new_off[hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (new_off[mid] <= t) lo = mid;
        else hi = mid;
    }
    return lo;
}

__global__ void window_lengths_kernel(const int64_t* __restrict__ win_off, int64_t g_windows, int64_t g_tiles,
                                      const int64_t* __restrict__ ids, int64_t n_sel, int64_t* __restrict__ len,
                                      int32_t* __restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_sel) return;
    const int64_t w = ids[i];
    if (w < 0 || w >= g_windows) {
        atomicOr(err, kErrRange);
        len[i] = 0;
        return;
    }
    if (i > 0 && ids[i - 1] >= w) atomicOr(err, kErrOrder);
    int64_t t0 = win_off[w], t1 = win_off[w + 1];
    t1 = t1 < 0 ? 0 : (t1 > g_tiles ? g_tiles : t1);
    t0 = t0 < 0 ? 0 : (t0 > t1 ? t1 : t0);
    len[i] = t1 - t0;
}

// Marks every valid neighbour column of the gathered tiles in the bitmap.
__global__ void mark_neighbours_kernel(const int64_t* __restrict__ win_off, const int32_t* __restrict__ cols,
                                       int tc, const int64_t* __restrict__ ids, const int64_t* __restrict__ new_off,
                                       int64_t n_sel, int64_t num_nodes, uint32_t* __restrict__ bitmap) {
    const int64_t nslots = new_off[n_sel] * tc;
    for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < nslots;
         s += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = s / tc;
        const int64_t i = window_of_tile(new_off, n_sel, t);
        const int64_t src = (win_off[ids[i]] + (t - new_off[i])) * tc + s % tc;
        const int64_t c = cols[src];
        if (c >= 0 && c < num_nodes) atomicOr(&bitmap[c >> 5], 1u << (c & 31));
    }
}

// Clears the internal nodes' bits (16 consecutive nodes = half a word) and
// counts the internal nodes (rows below num_nodes).
__global__ void clear_internal_kernel(const int64_t* __restrict__ ids, int64_t n_sel, int64_t num_nodes,
                                      uint32_t* __restrict__ bitmap, unsigned long long* __restrict__ n_internal) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_sel) return;
    const int64_t w = ids[i];
    if (w < 0) return;  // reported by window_lengths_kernel
    const int64_t first = w * 16;
    int64_t rows = num_nodes - first;
    rows = rows < 0 ? 0 : (rows > 16 ? 16 : rows);
    if (rows == 0) return;
    const uint32_t mask = (rows == 16 ? 0xFFFFu : ((1u << rows) - 1u)) << (16 * (w & 1));
    atomicAnd(&bitmap[w >> 1], ~mask);
    atomicAdd(n_internal, (unsigned long long)rows);
}

__global__ void word_popcount_kernel(const uint32_t* __restrict__ bitmap, int64_t nwords, int32_t* __restrict__ cnt) {
    for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < nwords; w += (int64_t)gridDim.x * blockDim.x)
        cnt[w] = __popc(bitmap[w]);
}

// Candidates in ascending order: word w's set bits go to wprefix[w] + rank.
__global__ void compact_bits_kernel(const uint32_t* __restrict__ bitmap, int64_t nwords,
                                    const int64_t* __restrict__ wprefix, int64_t* __restrict__ out) {
    for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < nwords;
         w += (int64_t)gridDim.x * blockDim.x) {
        uint32_t b = bitmap[w];
        int64_t o = wprefix[w];
        while (b) {
            const int k = __ffs(b) - 1;
            out[o++] = (w << 5) + k;
            b &= b - 1;
        }
    }
}

// Internal node (i, r) -> local id 16 i + r (every selected window but a
// final partial one has 16 rows below num_nodes, so positions are dense).
__global__ void map_internal_kernel(const int64_t* __restrict__ ids, int64_t n_sel, int64_t num_nodes,
                                    int32_t* __restrict__ node_map, int64_t* __restrict__ input_nodes) {
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= n_sel * 16) return;
    const int64_t node = ids[k >> 4] * 16 + (k & 15);
    if (node < 0 || node >= num_nodes) return;
    node_map[node] = (int32_t)k;
    input_nodes[k] = node;
}

// Every candidate kept: local id num_internal + ascending rank.
__global__ void map_all_external_kernel(const uint32_t* __restrict__ bitmap, int64_t nwords,
                                        const int64_t* __restrict__ wprefix, int64_t num_internal, int64_t limit,
                                        int32_t* __restrict__ node_map, int64_t* __restrict__ input_nodes) {
    for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < nwords;
         w += (int64_t)gridDim.x * blockDim.x) {
        uint32_t b = bitmap[w];
        int64_t o = num_internal + wprefix[w];
        while (b) {
            const int k = __ffs(b) - 1;
            const int64_t node = (w << 5) + k;
            if (o < limit) {  // limit = num_internal + num_kept, the caller's output size
                node_map[node] = (int32_t)o;
                input_nodes[o] = node;
            }
            ++o;
            b &= b - 1;
        }
    }
}

__global__ void map_kept_external_kernel(const int64_t* __restrict__ kept, int64_t n_kept, int64_t num_internal,
                                         int64_t num_nodes, int32_t* __restrict__ node_map,
                                         int64_t* __restrict__ input_nodes, int32_t* __restrict__ err) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n_kept) return;
    const int64_t v = kept[j];
    if (v < 0 || v >= num_nodes) {
        atomicOr(err, kErrRange);
        return;
    }
    node_map[v] = (int32_t)(num_internal + j);
    input_nodes[num_internal + j] = v;
}

// One wave per output tile: relabel its tc columns (halo and inner) and
// copy its 16 x tc values twice, zeroing masked columns.  Sets *any_nan if a
// halo value is NaN.
template <typename VT>
__global__ __launch_bounds__(kBlk) void repack_tiles_kernel(
    const int64_t* __restrict__ win_off, const int32_t* __restrict__ cols, const VT* __restrict__ vals, int tc,
    const int64_t* __restrict__ ids, const int64_t* __restrict__ new_off, int64_t n_sel, int64_t num_nodes,
    int64_t num_internal, const int32_t* __restrict__ node_map, int32_t* __restrict__ halo_cols,
    VT* __restrict__ halo_vals, int32_t* __restrict__ inner_cols, VT* __restrict__ inner_vals,
    int32_t* __restrict__ any_nan) {
    const int lane = threadIdx.x & 63;
    const int64_t T = new_off[n_sel];
    const int64_t waves = (int64_t)gridDim.x * (kBlk / 64);
    for (int64_t t = (int64_t)blockIdx.x * (kBlk / 64) + (threadIdx.x >> 6); t < T; t += waves) {
        const int64_t i = window_of_tile(new_off, n_sel, t);
        const int64_t st = win_off[ids[i]] + (t - new_off[i]);  // source tile
        int32_t hc = -1;
        if (lane < tc) {
            const int64_t c = cols[st * tc + lane];
            hc = (c >= 0 && c < num_nodes) ? node_map[c] : -1;
            halo_cols[t * tc + lane] = hc;
            inner_cols[t * tc + lane] = hc >= num_internal ? -1 : hc;
        }
        bool nan_seen = false;
        for (int e = lane; e < 16 * tc; e += 64) {
            const int col = e % tc;
            const int32_t h = __shfl(hc, col, 64);
            const VT v = vals[st * 16 * tc + e];
            const VT z = from_float<VT>(0.0f);
            const VT hv = h < 0 ? z : v;
            halo_vals[t * 16 * tc + e] = hv;
            inner_vals[t * 16 * tc + e] = (h < 0 || h >= num_internal) ? z : hv;
            const float f = to_float(hv);
            nan_seen |= (f != f);
        }
        if (__any(nan_seen) && lane == 0) atomicOr(any_nan, 1);
    }
}

// node_map entries of the input nodes back to -1.
__global__ void unmap_kernel(const int64_t* __restrict__ input_nodes, int64_t n, int64_t num_nodes,
                             int32_t* __restrict__ node_map) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j < n) {
        const int64_t v = input_nodes[j];
        if (v >= 0 && v < num_nodes) node_map[v] = -1;
    }
}

struct RepackWs {
    int64_t* len;
    int32_t* err;
    unsigned long long* n_internal;
    int32_t* wcnt;
    int64_t* wprefix;
    char* scan_ws;
    size_t scan_bytes;
};

template <typename C>
void carve_repack(C& c, int64_t n_sel, int64_t nwords, RepackWs* w) {
    const int64_t nscan = (n_sel > nwords ? n_sel : nwords) + 1;
    w->len = c.template take<int64_t>((size_t)n_sel + 1);
    w->err = c.template take<int32_t>(4);
    w->n_internal = c.template take<unsigned long long>(1);
    w->wcnt = c.template take<int32_t>((size_t)nwords + 1);
    w->wprefix = c.template take<int64_t>((size_t)nwords + 1);
    w->scan_bytes = scan_workspace_bytes(nscan);
    w->scan_ws = c.template take<char>(w->scan_bytes);
}

int check_graph(const grws_bcsr* g) {
    GRWS_CHECK_ARG(g != nullptr, "repack: null graph");
    GRWS_CHECK_ARG(g->tile_rows == 16, "repack: tile_rows must be 16");
    GRWS_CHECK_ARG(g->tile_cols == 8 || g->tile_cols == 16, "repack: tile_cols must be 8 or 16");
    GRWS_CHECK_ARG(g->num_windows >= 0 && g->num_tiles >= 0, "repack: negative graph size");
    GRWS_CHECK_ARG(g->window_offset != nullptr, "repack: null window_offset");
    if (g->num_tiles > 0) GRWS_CHECK_ARG(g->col_indices && g->values, "repack: null tile arrays");
    if (g->values_dtype != GRWS_F32 && g->values_dtype != GRWS_F16 && g->values_dtype != GRWS_BF16)
        return set_error(GRWS_E_DTYPE, "repack: unsupported values dtype %d", g->values_dtype);
    return GRWS_OK;
}

}  // namespace
}  // namespace grws

using namespace grws;

extern "C" size_t grws_repack_workspace_bytes(int64_t num_selected, int64_t num_nodes) {
    if (num_selected < 0 || num_nodes < 0) return 0;
    Sizer s;
    const int64_t nwords = (num_nodes + 31) / 32;
    const int64_t nscan = (num_selected > nwords ? num_selected : nwords) + 1;
    s.take<int64_t>((size_t)num_selected + 1);
    s.take<int32_t>(4);
    s.take<unsigned long long>(1);
    s.take<int32_t>((size_t)nwords + 1);
    s.take<int64_t>((size_t)nwords + 1);
    s.take<char>(scan_workspace_bytes(nscan));
    return s.used;
}

extern "C" int grws_repack_prepare(const grws_bcsr* g, int64_t num_nodes, const int64_t* window_ids,
                                   int64_t num_selected, uint32_t* bitmap, int64_t* new_offsets,
                                   int64_t* counts_out, void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_graph(g));
    GRWS_CHECK_ARG(num_nodes >= 0 && num_nodes <= INT32_MAX, "repack: num_nodes out of range");
    GRWS_CHECK_ARG(num_selected >= 0, "repack: negative window count");
    GRWS_CHECK_ARG(num_selected * 16 <= INT32_MAX, "repack: too many windows for int32 local ids");
    GRWS_CHECK_ARG(bitmap && new_offsets && counts_out, "repack: null pointer");
    if (num_selected > 0) GRWS_CHECK_ARG(window_ids != nullptr, "repack: null window ids");
    const int64_t nwords = (num_nodes + 31) / 32;
    Carver cv(workspace, workspace_bytes);
    RepackWs w;
    carve_repack(cv, num_selected, nwords, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "repack: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    GRWS_TRY(fill_i32(w.err, 4, 0, stream));
    GRWS_TRY(fill_i64(reinterpret_cast<int64_t*>(w.n_internal), 1, 0, stream));
    if (num_selected > 0) {
        hipLaunchKernelGGL(window_lengths_kernel, dim3(grid_for(num_selected)), dim3(kBlk), 0, stream,
                           g->window_offset, g->num_windows, g->num_tiles, window_ids, num_selected, w.len, w.err);
        GRWS_LAUNCH_CHECK();
    }
    GRWS_TRY(scan_i64_to_i64(w.len, new_offsets, num_selected, false, w.scan_ws, w.scan_bytes, stream));
    if (num_selected > 0) {
        hipLaunchKernelGGL(mark_neighbours_kernel, dim3(grid_for(g->num_tiles * g->tile_cols)), dim3(kBlk), 0, stream,
                           g->window_offset, g->col_indices, (int)g->tile_cols, window_ids, new_offsets,
                           num_selected, num_nodes, bitmap);
        GRWS_LAUNCH_CHECK();
        hipLaunchKernelGGL(clear_internal_kernel, dim3(grid_for(num_selected)), dim3(kBlk), 0, stream, window_ids,
                           num_selected, num_nodes, bitmap, w.n_internal);
        GRWS_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(word_popcount_kernel, dim3(grid_for(nwords)), dim3(kBlk), 0, stream, bitmap, nwords, w.wcnt);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.wcnt, w.wprefix, nwords, false, w.scan_ws, w.scan_bytes, stream));
    int64_t h[4] = {0, 0, 0, 0};
    int32_t err = 0;
    GRWS_HIP(hipMemcpyAsync(&h[0], new_offsets + num_selected, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[1], w.n_internal, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&h[2], w.wprefix + nwords, sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipMemcpyAsync(&err, w.err, sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    if (err) {
        // leave the state as found: the bitmap may hold marks
        GRWS_TRY(fill_bytes_zero(bitmap, (size_t)nwords * 4, stream));
        if (err & kErrRange) return set_error(GRWS_E_INVALID, "repack: window id outside [0, num_windows)");
        return set_error(GRWS_E_INVALID, "repack: window ids must be strictly ascending");
    }
    counts_out[0] = h[0];  // tiles of the new graph
    counts_out[1] = h[1];  // internal nodes
    counts_out[2] = h[2];  // external candidates
    return GRWS_OK;
}

extern "C" int grws_repack_externals(const uint32_t* bitmap, int64_t num_nodes, int64_t* external_out,
                                     void* workspace, size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_CHECK_ARG(bitmap && external_out, "repack_externals: null pointer");
    GRWS_CHECK_ARG(num_nodes >= 0, "repack_externals: negative size");
    const int64_t nwords = (num_nodes + 31) / 32;
    Carver cv(workspace, workspace_bytes);
    RepackWs w;
    carve_repack(cv, 0, nwords, &w);
    if (!cv.ok)
        return set_error(GRWS_E_CAPACITY, "repack_externals: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    hipLaunchKernelGGL(word_popcount_kernel, dim3(grid_for(nwords)), dim3(kBlk), 0, stream, bitmap, nwords, w.wcnt);
    GRWS_LAUNCH_CHECK();
    GRWS_TRY(scan_i32_to_i64(w.wcnt, w.wprefix, nwords, false, w.scan_ws, w.scan_bytes, stream));
    hipLaunchKernelGGL(compact_bits_kernel, dim3(grid_for(nwords)), dim3(kBlk), 0, stream, bitmap, nwords, w.wprefix,
                       external_out);
    GRWS_LAUNCH_CHECK();
    return GRWS_OK;
}

extern "C" int grws_repack_finish(const grws_bcsr* g, int64_t num_nodes, const int64_t* window_ids,
                                  int64_t num_selected, const int64_t* new_offsets, int64_t num_internal,
                                  const int64_t* kept_external, int64_t num_kept, int32_t* node_map,
                                  uint32_t* bitmap, int64_t* input_nodes, int32_t* halo_cols, void* halo_values,
                                  int32_t* inner_cols, void* inner_values, int32_t* flags_out, void* workspace,
                                  size_t workspace_bytes, void* stream_) {
    clear_error();
    hipStream_t stream = as_stream(stream_);
    GRWS_TRY(check_graph(g));
    GRWS_CHECK_ARG(num_nodes >= 0 && num_nodes <= INT32_MAX, "repack: num_nodes out of range");
    GRWS_CHECK_ARG(num_selected >= 0 && num_internal >= 0 && num_kept >= 0, "repack: negative size");
    GRWS_CHECK_ARG(num_internal <= num_selected * 16, "repack: num_internal exceeds 16 rows per window");
    GRWS_CHECK_ARG(num_internal + num_kept <= INT32_MAX, "repack: too many input nodes for int32 local ids");
    GRWS_CHECK_ARG(node_map && bitmap && new_offsets && flags_out, "repack: null pointer");
    const int64_t nwords = (num_nodes + 31) / 32;
    Carver cv(workspace, workspace_bytes);
    RepackWs w;
    carve_repack(cv, num_selected, nwords, &w);
    if (!cv.ok) return set_error(GRWS_E_CAPACITY, "repack: workspace too small (%zu < %zu)", workspace_bytes, cv.used);
    GRWS_TRY(fill_i32(w.err, 4, 0, stream));
    const int64_t n_in = num_internal + num_kept;
    if (n_in > 0) {
        GRWS_CHECK_ARG(input_nodes != nullptr, "repack: null input_nodes");
        GRWS_TRY(fill_i64(input_nodes, n_in, -1, stream));
    }
    if (num_selected > 0) {
        GRWS_CHECK_ARG(window_ids != nullptr, "repack: null window ids");
        hipLaunchKernelGGL(map_internal_kernel, dim3(grid_for(num_selected * 16)), dim3(kBlk), 0, stream, window_ids,
                           num_selected, num_nodes, node_map, input_nodes);
        GRWS_LAUNCH_CHECK();
    }
    if (kept_external == nullptr) {
        // every candidate is kept: ranks from the bitmap
        hipLaunchKernelGGL(word_popcount_kernel, dim3(grid_for(nwords)), dim3(kBlk), 0, stream, bitmap, nwords, w.wcnt);
        GRWS_LAUNCH_CHECK();
        GRWS_TRY(scan_i32_to_i64(w.wcnt, w.wprefix, nwords, false, w.scan_ws, w.scan_bytes, stream));
        if (num_kept > 0) {
            hipLaunchKernelGGL(map_all_external_kernel, dim3(grid_for(nwords)), dim3(kBlk), 0, stream, bitmap, nwords,
                               w.wprefix, num_internal, n_in, node_map, input_nodes);
            GRWS_LAUNCH_CHECK();
        }
    } else if (num_kept > 0) {
        hipLaunchKernelGGL(map_kept_external_kernel, dim3(grid_for(num_kept)), dim3(kBlk), 0, stream, kept_external,
                           num_kept, num_internal, num_nodes, node_map, input_nodes, w.err);
        GRWS_LAUNCH_CHECK();
    }
    if (num_selected > 0 && g->num_tiles > 0) {
        GRWS_CHECK_ARG(halo_cols && halo_values && inner_cols && inner_values, "repack: null output");
        const unsigned grid = grid_for(g->num_tiles, kBlk / 64);
#define GRWS_REPACK_TILES(VT)                                                                                     \
    hipLaunchKernelGGL(repack_tiles_kernel<VT>, dim3(grid), dim3(kBlk), 0, stream, g->window_offset,              \
                       g->col_indices, static_cast<const VT*>(g->values), (int)g->tile_cols, window_ids,         \
                       new_offsets, num_selected, num_nodes, num_internal, node_map, halo_cols,                  \
                       static_cast<VT*>(halo_values), inner_cols, static_cast<VT*>(inner_values), w.err + 1)
        if (g->values_dtype == GRWS_F32) GRWS_REPACK_TILES(float);
        else if (g->values_dtype == GRWS_F16) GRWS_REPACK_TILES(_Float16);
        else GRWS_REPACK_TILES(__hip_bfloat16);
#undef GRWS_REPACK_TILES
        GRWS_LAUNCH_CHECK();
    }
    // state back to all -1 / all 0
    if (n_in > 0) {
        hipLaunchKernelGGL(unmap_kernel, dim3(grid_for(n_in)), dim3(kBlk), 0, stream, input_nodes, n_in, num_nodes,
                           node_map);
        GRWS_LAUNCH_CHECK();
    }
    GRWS_TRY(fill_bytes_zero(bitmap, (size_t)nwords * 4, stream));
    int32_t h[2] = {0, 0};
    GRWS_HIP(hipMemcpyAsync(h, w.err, 2 * sizeof(int32_t), hipMemcpyDeviceToHost, stream));
    GRWS_HIP(hipStreamSynchronize(stream));
    if (h[0] & kErrRange) return set_error(GRWS_E_INVALID, "repack: kept external id outside [0, num_nodes)");
    flags_out[0] = h[1];  // a halo value is NaN
    return GRWS_OK;
}
